/* qmsg_gguf.cpp - GGUF v3 header reader: scalar metadata of the first shard and the tensor
 * table of every shard (the reference's qms_gguf_open, src/gguf.c:112-241). Only headers are
 * read here; tensor bytes are fetched by the upload with gguf_pread. No GPU calls. */
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "qmsg_gguf.h"

namespace {

/* GGUF metadata value types (GGUF v3 specification). */
enum { V_U8, V_I8, V_U16, V_I16, V_U32, V_I32, V_F32, V_BOOL, V_STR, V_ARR, V_U64, V_I64, V_F64 };
constexpr int kValueBytes[] = { 1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8 };

constexpr size_t kKeyCap = 96, kStrCap = 256, kNameCap = sizeof(((qmsg_tensor *)nullptr)->name);
constexpr int kMaxShards = 256;

int fail_open(const char *fmt, ...)
{
    char buf[640];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    qmsg::set_global_error(buf);
    return QMSG_E_INVALID;
}

int pread_all(int fd, void *dst, uint64_t n, uint64_t off)
{
    uint8_t *d = (uint8_t *)dst;
    while (n > 0) {
        const size_t want = n > (1ull << 30) ? (size_t)(1ull << 30) : (size_t)n;
        const ssize_t got = ::pread(fd, d, want, (off_t)off);
        if (got < 0 && errno == EINTR) continue;
        if (got <= 0) return -1;
        d += got;
        off += (uint64_t)got;
        n -= (uint64_t)got;
    }
    return 0;
}

/* Sequential reader over a file with a 1 MiB window; any short read latches `bad`. */
class Cursor {
public:
    Cursor(int fd, uint64_t size) : fd_(fd), size_(size), win_(1u << 20) {}

    bool bad() const { return bad_; }
    uint64_t tell() const { return base_ + at_; }

    void bytes(void *dst, uint64_t n)
    {
        uint8_t *d = (uint8_t *)dst;
        while (n > 0 && !bad_) {
            if (at_ == len_ && !refill()) return;
            const uint64_t k = len_ - at_ < n ? len_ - at_ : n;
            if (d) {
                memcpy(d, win_.data() + at_, (size_t)k);
                d += k;
            }
            at_ += (size_t)k;
            n -= k;
        }
    }
    void skip(uint64_t n) { bytes(nullptr, n); }
    uint32_t u32() { uint32_t v = 0; bytes(&v, 4); return v; }
    uint64_t u64() { uint64_t v = 0; bytes(&v, 8); return v; }

    /* A GGUF string (u64 length + bytes); keeps at most cap-1 bytes, consumes all of it. */
    std::string str(size_t cap)
    {
        const uint64_t n = u64();
        if (bad_ || n > (1ull << 32)) { bad_ = true; return std::string(); }
        const uint64_t keep = n < cap - 1 ? n : cap - 1;
        std::string s((size_t)keep, '\0');
        bytes(&s[0], keep);
        skip(n - keep);
        return s;
    }

    /* Skip one value of type t (nested arrays included). */
    void skip_value(uint32_t t)
    {
        if (t == V_STR) { (void)str(1); return; }
        if (t == V_ARR) {
            const uint32_t et = u32();
            const uint64_t n = u64();
            if (et > V_F64) { bad_ = true; return; }
            if (et == V_STR || et == V_ARR) {
                for (uint64_t k = 0; k < n && !bad_; k++) skip_value(et);
                return;
            }
            skip(n * (uint64_t)kValueBytes[et]);
            return;
        }
        if (t > V_F64) { bad_ = true; return; }
        skip((uint64_t)kValueBytes[t]);
    }

private:
    bool refill()
    {
        base_ += at_;
        at_ = 0;
        const uint64_t left = size_ > base_ ? size_ - base_ : 0;
        len_ = left < win_.size() ? (size_t)left : win_.size();
        if (len_ == 0 || pread_all(fd_, win_.data(), len_, base_) != 0) {
            bad_ = true;
            len_ = 0;
            return false;
        }
        return true;
    }

    int fd_;
    uint64_t size_, base_ = 0;
    std::vector<uint8_t> win_;
    size_t len_ = 0, at_ = 0;
    bool bad_ = false;
};

uint64_t row_bytes_of(int type, int64_t ne0)
{
    switch (type) {
    case QMSG_T_F32: return (uint64_t)ne0 * 4;
    case QMSG_T_F16: return (uint64_t)ne0 * 2;
    case QMSG_T_Q4_0: return ne0 % 32 ? 0 : (uint64_t)ne0 / 32 * 18;
    case QMSG_T_Q4_1: return ne0 % 32 ? 0 : (uint64_t)ne0 / 32 * 20;
    case QMSG_T_Q8_0: return ne0 % 32 ? 0 : (uint64_t)ne0 / 32 * 34;
    case QMSG_T_Q6_K: return ne0 % 256 ? 0 : (uint64_t)ne0 / 256 * 210;
    default: return 0;
    }
}

/* One shard: header, metadata (kept for the first shard only), tensor table; offsets made
 * absolute against the aligned start of the data section. */
int parse_shard(qmsg_gguf *g, int si)
{
    const char *path = g->paths[(size_t)si].c_str();
    Cursor r(g->fds[(size_t)si], g->sizes[(size_t)si]);
    char magic[4] = { 0 };
    r.bytes(magic, 4);
    if (r.bad() || memcmp(magic, "GGUF", 4) != 0) return fail_open("gguf: %s is not a GGUF file", path);
    const uint32_t version = r.u32();
    if (r.bad() || version != 3) return fail_open("gguf: %s version %u unsupported", path, version);
    const uint64_t n_tensors = r.u64(), n_kv = r.u64();
    uint64_t alignment = 32;
    for (uint64_t k = 0; k < n_kv && !r.bad(); k++) {
        qmsg_gguf::KV kv;
        kv.key = r.str(kKeyCap);
        const uint32_t t = r.u32();
        kv.vtype = (int)t;
        bool keep = si == 0;
        switch (t) {
        case V_U8: { uint8_t v = 0; r.bytes(&v, 1); kv.u = v; kv.i = v; kv.f = v; break; }
        case V_I8: { int8_t v = 0; r.bytes(&v, 1); kv.i = v; kv.u = (uint64_t)v; kv.f = v; break; }
        case V_U16: { uint16_t v = 0; r.bytes(&v, 2); kv.u = v; kv.i = v; kv.f = v; break; }
        case V_I16: { int16_t v = 0; r.bytes(&v, 2); kv.i = v; kv.u = (uint64_t)v; kv.f = v; break; }
        case V_U32: { uint32_t v = 0; r.bytes(&v, 4); kv.u = v; kv.i = v; kv.f = v; break; }
        case V_I32: { int32_t v = 0; r.bytes(&v, 4); kv.i = v; kv.u = (uint64_t)v; kv.f = v; break; }
        case V_F32: { float v = 0; r.bytes(&v, 4); kv.f = v; kv.i = (int64_t)v; break; }
        case V_BOOL: { uint8_t v = 0; r.bytes(&v, 1); kv.u = v; kv.i = v; kv.f = v; break; }
        case V_U64: { uint64_t v = 0; r.bytes(&v, 8); kv.u = v; kv.i = (int64_t)v; kv.f = (double)v; break; }
        case V_I64: { int64_t v = 0; r.bytes(&v, 8); kv.i = v; kv.u = (uint64_t)v; kv.f = (double)v; break; }
        case V_F64: { double v = 0; r.bytes(&v, 8); kv.f = v; kv.i = (int64_t)v; break; }
        case V_STR: kv.str = r.str(kStrCap); break;
        default: r.skip_value(t); keep = false; break;      /* arrays (tokenizer tables) */
        }
        if (kv.key == "general.alignment") alignment = kv.u;
        if (keep && !r.bad()) g->kv.push_back(std::move(kv));
    }
    if (r.bad()) return fail_open("gguf: truncated metadata in %s", path);
    if (alignment == 0) return fail_open("gguf: %s has general.alignment 0", path);

    const size_t first = g->tensors.size();
    for (uint64_t k = 0; k < n_tensors && !r.bad(); k++) {
        qmsg_tensor t;
        memset(&t, 0, sizeof t);
        const std::string name = r.str(kNameCap);
        memcpy(t.name, name.data(), name.size());
        t.n_dims = (int)r.u32();
        if (r.bad() || t.n_dims < 1 || t.n_dims > 4)
            return fail_open("gguf: truncated tensor table in %s", path);
        for (int d = 0; d < 4; d++) t.ne[d] = 1;
        for (int d = 0; d < t.n_dims; d++) t.ne[d] = (int64_t)r.u64();
        t.type = (int)r.u32();
        t.off = r.u64();                                   /* relative to the data section */
        t.shard = si;
        g->tensors.push_back(t);
    }
    if (r.bad()) return fail_open("gguf: truncated tensor table in %s", path);

    const uint64_t data_start = (r.tell() + alignment - 1) / alignment * alignment;
    for (size_t k = first; k < g->tensors.size(); k++) {
        qmsg_tensor &t = g->tensors[k];
        const uint64_t rb = row_bytes_of(t.type, t.ne[0]);
        t.nbytes = rb * (uint64_t)(t.ne[1] * t.ne[2] * t.ne[3]);
        t.off += data_start;
        if (rb && t.off + t.nbytes > g->sizes[(size_t)si])
            return fail_open("gguf: tensor %s runs past end of %s", t.name, path);
    }
    return QMSG_OK;
}

/* "<stem>-00001-of-0000N.gguf" names every shard of the set; any other path is one file. */
int shard_paths(const char *path, std::vector<std::string> &out)
{
    const size_t n = strlen(path), tl = strlen("-00001-of-00000.gguf");
    if (n > tl && strncmp(path + n - tl, "-00001-of-", 10) == 0) {
        const int count = atoi(path + n - tl + 10);
        if (count < 1 || count > kMaxShards) return -1;
        for (int i = 0; i < count; i++) {
            char buf[32];
            snprintf(buf, sizeof buf, "-%05d-of-%05d.gguf", i + 1, count);
            out.push_back(std::string(path, n - tl) + buf);
        }
    } else {
        out.push_back(path);
    }
    return 0;
}

const qmsg_gguf::KV *find_kv(const qmsg_gguf *g, const char *key)
{
    for (const auto &kv : g->kv)
        if (kv.key == key) return &kv;
    return nullptr;
}

}  // namespace

namespace qmsg {

int gguf_pread(const qmsg_gguf *g, int shard, uint64_t off, uint64_t n, void *dst)
{
    if (shard < 0 || shard >= (int)g->fds.size()) return -1;
    return pread_all(g->fds[(size_t)shard], dst, n, off);
}

int gguf_find(const qmsg_gguf *g, const char *name)
{
    for (size_t i = 0; i < g->tensors.size(); i++)
        if (strcmp(g->tensors[i].name, name) == 0) return (int)i;
    return -1;
}

}  // namespace qmsg

extern "C" {

void qmsg_gguf_close(qmsg_gguf *g)
{
    if (!g) return;
    for (int fd : g->fds)
        if (fd >= 0) ::close(fd);
    delete g;
}

int qmsg_gguf_open(qmsg_gguf **out, const char *path)
{
    if (!out || !path) return fail_open("qmsg_gguf_open: null argument");
    *out = nullptr;
    qmsg_gguf *g = new qmsg_gguf;
    if (shard_paths(path, g->paths) != 0) {
        delete g;
        return fail_open("gguf: bad shard name %s", path);
    }
    for (size_t i = 0; i < g->paths.size(); i++) {
        const int fd = ::open(g->paths[i].c_str(), O_RDONLY | O_CLOEXEC);
        struct stat st;
        if (fd < 0 || fstat(fd, &st) != 0 || st.st_size <= 0) {
            if (fd >= 0) ::close(fd);
            const int rc = fail_open("gguf: cannot open %s", g->paths[i].c_str());
            qmsg_gguf_close(g);
            return rc;
        }
        g->fds.push_back(fd);
        g->sizes.push_back((uint64_t)st.st_size);
        const int rc = parse_shard(g, (int)i);
        if (rc != QMSG_OK) {
            qmsg_gguf_close(g);
            return rc;
        }
    }
    *out = g;
    return QMSG_OK;
}

int qmsg_gguf_n_tensors(const qmsg_gguf *g) { return g ? (int)g->tensors.size() : QMSG_E_INVALID; }

int qmsg_gguf_tensor(const qmsg_gguf *g, int i, qmsg_tensor *out)
{
    if (!g || !out || i < 0 || i >= (int)g->tensors.size()) return QMSG_E_INVALID;
    *out = g->tensors[(size_t)i];
    return QMSG_OK;
}

int qmsg_gguf_find(const qmsg_gguf *g, const char *name)
{
    if (!g || !name) return -1;
    return qmsg::gguf_find(g, name);
}

int qmsg_gguf_get_int(const qmsg_gguf *g, const char *key, int64_t *out)
{
    if (!g || !key || !out) return QMSG_E_INVALID;
    const qmsg_gguf::KV *kv = find_kv(g, key);
    if (!kv || kv->vtype == V_STR) return fail_open("gguf: missing required key %s", key);
    *out = kv->i;
    return QMSG_OK;
}

int qmsg_gguf_get_float(const qmsg_gguf *g, const char *key, double *out)
{
    if (!g || !key || !out) return QMSG_E_INVALID;
    const qmsg_gguf::KV *kv = find_kv(g, key);
    if (!kv || kv->vtype == V_STR) return fail_open("gguf: missing required key %s", key);
    *out = kv->f;
    return QMSG_OK;
}

int qmsg_gguf_get_str(const qmsg_gguf *g, const char *key, char *buf, size_t n)
{
    if (!g || !key || !buf || n == 0) return QMSG_E_INVALID;
    const qmsg_gguf::KV *kv = find_kv(g, key);
    if (!kv || kv->vtype != V_STR) return fail_open("gguf: missing string key %s", key);
    const size_t k = kv->str.size() < n - 1 ? kv->str.size() : n - 1;
    memcpy(buf, kv->str.data(), k);
    buf[k] = '\0';
    return QMSG_OK;
}

int qmsg_gguf_moe_cfg(const qmsg_gguf *g, qmsg_cfg *cfg, int *n_layer, float *eps)
{
    if (!g) return QMSG_E_INVALID;
    const qmsg_gguf::KV *arch = find_kv(g, "general.architecture");
    if (!arch || arch->vtype != V_STR || arch->str != "qwen3moe")
        return fail_open("model: architecture %s is not qwen3moe",
                         arch && arch->vtype == V_STR ? arch->str.c_str() : "(missing)");
    struct { const char *key; int64_t v; } k[5] = {
        { "qwen3moe.block_count", 0 }, { "qwen3moe.embedding_length", 0 }, { "qwen3moe.expert_count", 0 },
        { "qwen3moe.expert_used_count", 0 }, { "qwen3moe.expert_feed_forward_length", 0 },
    };
    for (auto &e : k) {
        const int rc = qmsg_gguf_get_int(g, e.key, &e.v);
        if (rc) return rc;
        if (e.v <= 0 || e.v > (1 << 30)) return fail_open("model: %s = %lld is out of range", e.key, (long long)e.v);
    }
    double f = 0.0;
    const int rc = qmsg_gguf_get_float(g, "qwen3moe.attention.layer_norm_rms_epsilon", &f);
    if (rc) return rc;
    if (k[3].v > k[2].v) return fail_open("model: inconsistent config (expert_used_count > expert_count)");
    if (cfg) {
        cfg->n_embd = (int)k[1].v;
        cfg->n_expert = (int)k[2].v;
        cfg->n_used = (int)k[3].v;
        cfg->n_ff_exp = (int)k[4].v;
    }
    if (n_layer) *n_layer = (int)k[0].v;
    if (eps) *eps = (float)f;
    return QMSG_OK;
}

}  // extern "C"
