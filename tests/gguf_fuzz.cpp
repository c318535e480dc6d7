// Mutation fuzz of the GGUF reader (host code, built with AddressSanitizer and UBSan by
// tests/test_gguf.py): random byte flips, overwrites with boundary integers and truncations of
// a valid file; every table entry and key of a file that opens is queried.
// Usage: gguf_fuzz <seed file> <iterations> <rng seed>
#include "qmsg.h"
#include <cstdio>
#include <cstdint>
#include <cstring>
#include <random>
#include <string>
#include <vector>
#include <unistd.h>
namespace qmsg { void set_global_error(const char *) {} }
int main(int argc, char **argv)
{
    if (argc < 4) return 2;
    FILE *f = fopen(argv[1], "rb");
    if (!f) return 2;
    std::vector<unsigned char> seed;
    int ch;
    while ((ch = fgetc(f)) != EOF) seed.push_back((unsigned char)ch);
    fclose(f);
    const long iters = atol(argv[2]);
    std::mt19937_64 rng(strtoull(argv[3], nullptr, 10));
    const std::string path = "/tmp/fz_" + std::to_string(getpid()) + ".gguf";
    const uint64_t specials[] = { 0, 1, 2, 3, 0x7f, 0x80, 0xff, 0x7fffffff, 0x80000000u, 0xffffffffu,
                                  0x100000000ull, 0x7fffffffffffffffull, 0x8000000000000000ull, ~0ull, 96, 97, 4096 };
    long opened = 0;
    for (long it = 0; it < iters; it++) {
        std::vector<unsigned char> d = seed;
        const int nops = 1 + (int)(rng() % 4);
        for (int k = 0; k < nops; k++) {
            const int op = (int)(rng() % 4);
            // bias positions toward the header and tables (the first 2 KB)
            const size_t lim = (rng() % 4) ? std::min<size_t>(d.size(), 2048) : d.size();
            if (d.empty() || lim == 0) break;
            const size_t pos = rng() % lim;
            if (op == 0) d[pos] ^= (unsigned char)(1u << (rng() % 8));
            else if (op == 1) d[pos] = (unsigned char)rng();
            else if (op == 2) {
                const uint64_t v = specials[rng() % (sizeof specials / sizeof specials[0])];
                const int w = (rng() % 2) ? 8 : 4;
                for (int b = 0; b < w && pos + b < d.size(); b++) d[pos + b] = (unsigned char)(v >> (8 * b));
            } else d.resize(rng() % (d.size() + 1));
        }
        FILE *o = fopen(path.c_str(), "wb");
        if (!o) return 3;
        if (!d.empty()) fwrite(d.data(), 1, d.size(), o);
        fclose(o);
        qmsg_gguf *g = nullptr;
        if (qmsg_gguf_open(&g, path.c_str()) == 0 && g) {
            opened++;
            const int n = qmsg_gguf_n_tensors(g);
            for (int i = 0; i < n; i++) {
                qmsg_tensor t;
                if (qmsg_gguf_tensor(g, i, &t) == 0) (void)qmsg_gguf_find(g, t.name);
            }
            int64_t iv; double fv; char buf[64];
            const char *keys[] = { "general.architecture", "qwen3moe.block_count", "qwen3moe.embedding_length",
                                   "qwen3moe.expert_count", "qwen3moe.expert_used_count",
                                   "qwen3moe.expert_feed_forward_length", "qwen3moe.attention.layer_norm_rms_epsilon" };
            for (const char *k : keys) {
                (void)qmsg_gguf_get_int(g, k, &iv);
                (void)qmsg_gguf_get_float(g, k, &fv);
                (void)qmsg_gguf_get_str(g, k, buf, sizeof buf);
            }
            qmsg_cfg cfg; int nl; float eps;
            (void)qmsg_gguf_moe_cfg(g, &cfg, &nl, &eps);
            qmsg_gguf_close(g);
        }
    }
    unlink(path.c_str());
    printf("iterations %ld, opened %ld\n", iters, opened);
    return 0;
}
