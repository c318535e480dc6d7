/* qmsg_gguf.h - the parsed form of a GGUF file, shared by the header reader (qmsg_gguf.cpp)
 * and the staged upload into HBM (qmsg_api.cpp). Host code only. */
#ifndef QMSG_GGUF_INTERNAL_H
#define QMSG_GGUF_INTERNAL_H

#include <cstdint>
#include <string>
#include <vector>

#include "../../include/qmsg.h"

struct qmsg_gguf {
    /* one open file of the set */
    struct Shard {
        std::string path;
        int fd = -1;
        uint64_t size = 0;
    };
    /* one scalar of the first shard's metadata: its GGUF value type and payload */
    struct Scalar {
        std::string key;       /* cut to 95 bytes */
        uint32_t type = 0;
        uint64_t bits = 0;     /* integers and bool; signed types sign-extended */
        double real = 0.0;     /* f32 / f64 */
        std::string text;      /* strings, cut to 255 bytes */
    };
    std::vector<Shard> shards;
    std::vector<qmsg_tensor> tensors;
    std::vector<Scalar> meta;

    const Scalar *scalar(const char *key) const;
    /* integer and real views of a numeric scalar; false for strings */
    bool numeric(const Scalar &s, int64_t *i, double *f) const;
    /* the unsigned view (general.alignment): integer bits, 0 for reals and strings */
    uint64_t unsigned_view(const Scalar &s) const;
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
