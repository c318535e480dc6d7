/* qmsg_gguf.h - the parsed form of a GGUF file, shared by the header reader (qmsg_gguf.cpp)
 * and the staged upload into HBM (qmsg_api.cpp). Host code only. */
#ifndef QMSG_GGUF_INTERNAL_H
#define QMSG_GGUF_INTERNAL_H

#include <cstdint>
#include <string>
#include <vector>

#include "../../include/qmsg.h"

struct qmsg_gguf {
    /* one scalar of the first shard's metadata; every numeric view filled as it is read */
    struct KV {
        std::string key;   /* at most 95 bytes, like QmsKV.key */
        int vtype = 0;
        uint64_t u = 0;
        int64_t i = 0;
        double f = 0.0;
        std::string str;   /* string values, at most 255 bytes */
    };
    std::vector<std::string> paths;
    std::vector<int> fds;
    std::vector<uint64_t> sizes;
    std::vector<qmsg_tensor> tensors;
    std::vector<KV> kv;
};

namespace qmsg {

/* Read exactly n bytes at byte offset off of shard `shard`; 0 on success. Thread-safe. */
int gguf_pread(const qmsg_gguf *g, int shard, uint64_t off, uint64_t n, void *dst);

/* Index of the first tensor called `name`, or -1. */
int gguf_find(const qmsg_gguf *g, const char *name);

/* Set the message qmsg_last_error(NULL) returns (calls that have no context). */
void set_global_error(const char *msg);

}  // namespace qmsg

#endif
