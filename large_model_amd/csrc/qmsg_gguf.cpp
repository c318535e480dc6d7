/* qmsg_gguf.cpp - GGUF v3 header reader for the upload into HBM. Behaviour follows the reference's
 * qms_gguf_open / qms_gguf_get_* (src/gguf.c:112-283): the scalar metadata of the first shard, the
 * tensor table of every shard with absolute offsets, the same refusals. The layout is read from the
 * GGUF v3 format itself:
 *
 *   "GGUF" u32:version u64:n_tensors u64:n_kv
 *   n_kv    x { string key, u32 value_type, value }
 *   n_tensors x { string name, u32 n_dims, u64 ne[n_dims], u32 ggml_type, u64 offset }
 *   padding to general.alignment (default 32), then the tensor data; offsets are relative to it.
 *   string = u64 length + bytes; array value = u32 element_type + u64 count + elements.
 *
 * Each shard's header is parsed from a read-only mapping of the file with bounds-checked field
 * reads; the mapping is dropped once the table is built and tensor bytes are fetched later with
 * pread (gguf_pread). Sizes taken from the file are combined with overflow-checked arithmetic.
 * No GPU calls. */
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string_view>

#include "qmsg_gguf.h"

namespace {

/* How each GGUF value type is stored: payload bytes and how its scalar views derive. */
enum class Kind : uint8_t { Unsigned, Signed, Real, Text, List, None };
struct TypeInfo {
    uint8_t bytes;
    Kind kind;
};
constexpr uint32_t kTypeStr = 8, kTypeArr = 9, kNumTypes = 13;
constexpr TypeInfo kTypeInfo[kNumTypes] = {
    { 1, Kind::Unsigned }, { 1, Kind::Signed }, { 2, Kind::Unsigned }, { 2, Kind::Signed },  /* u8 i8 u16 i16 */
    { 4, Kind::Unsigned }, { 4, Kind::Signed }, { 4, Kind::Real },                         /* u32 i32 f32    */
    { 1, Kind::Unsigned },                                                                   /* bool           */
    { 0, Kind::Text },     { 0, Kind::List },                                                /* string array   */
    { 8, Kind::Unsigned }, { 8, Kind::Signed }, { 8, Kind::Real },                         /* u64 i64 f64    */
};
inline TypeInfo type_info(uint32_t t) { return t < kNumTypes ? kTypeInfo[t] : TypeInfo{ 0, Kind::None }; }

/* Kept lengths of the reference's fixed-size fields (QmsKV.key[96], QmsKV.str[256],
 * QmsTensor.name[96]): longer keys, strings and names are cut, the rest of the bytes skipped. */
constexpr size_t kKeyKeep = 95, kTextKeep = 255, kNameKeep = sizeof(((qmsg_tensor *)nullptr)->name) - 1;
constexpr int kMaxShards = 256;
constexpr int kMaxNesting = 16;          /* arrays of arrays deeper than this are refused */

int refuse(const char *fmt, ...)
{
    char msg[640];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(msg, sizeof msg, fmt, ap);
    va_end(ap);
    qmsg::set_global_error(msg);
    return QMSG_E_INVALID;
}

/* Bounds-checked little-endian fields of a mapped header. Any read past the end clears ok()
 * and yields zeros; callers check ok() at the points where a refusal is reported. */
class FieldReader {
public:
    FieldReader(const uint8_t *base, uint64_t size) : base_(base), size_(size) {}

    bool ok() const { return ok_; }
    uint64_t offset() const { return at_; }

    /* Advance over n bytes; returns where they start, or nullptr past the end. */
    const uint8_t *advance(uint64_t n)
    {
        if (!ok_ || n > size_ - at_) {
            ok_ = false;
            return nullptr;
        }
        const uint8_t *p = base_ + at_;
        at_ += n;
        return p;
    }
    template <class T>
    T field()
    {
        T v{};
        if (const uint8_t *p = advance(sizeof(T))) memcpy(&v, p, sizeof(T));
        return v;
    }
    /* A GGUF string; the view spans all of its bytes. */
    std::string_view text()
    {
        const uint64_t n = field<uint64_t>();
        const uint8_t *p = advance(n);
        return p ? std::string_view((const char *)p, (size_t)n) : std::string_view();
    }
    void fail() { ok_ = false; }

private:
    const uint8_t *base_;
    uint64_t size_, at_ = 0;
    bool ok_ = true;
};

std::string cut(std::string_view s, size_t keep) { return std::string(s.substr(0, keep)); }

/* Step over one value of type t (arrays: every element, nested arrays included). */
void pass_value(FieldReader &rd, uint32_t t, int depth)
{
    const TypeInfo ti = type_info(t);
    switch (ti.kind) {
    case Kind::Text: (void)rd.text(); return;
    case Kind::List: {
        const uint32_t et = rd.field<uint32_t>();
        const uint64_t count = rd.field<uint64_t>();
        const TypeInfo ei = type_info(et);
        if (ei.kind == Kind::None || depth >= kMaxNesting) return rd.fail();
        if (ei.bytes) {
            uint64_t span = 0;
            if (__builtin_mul_overflow(count, (uint64_t)ei.bytes, &span)) return rd.fail();
            (void)rd.advance(span);
            return;
        }
        for (uint64_t k = 0; k < count && rd.ok(); k++) pass_value(rd, et, depth + 1);
        return;
    }
    case Kind::None: return rd.fail();
    default: (void)rd.advance(ti.bytes); return;
    }
}

/* A scalar's payload: raw little-endian bits (integers, sign-extended for signed types) or the
 * value as a double (f32 / f64). */
void read_scalar(FieldReader &rd, const TypeInfo &ti, qmsg_gguf::Scalar &s)
{
    const uint8_t *p = rd.advance(ti.bytes);
    if (!p) return;
    uint64_t raw = 0;
    memcpy(&raw, p, ti.bytes);
    if (ti.kind == Kind::Signed && ti.bytes < 8) {
        const int sh = 64 - 8 * ti.bytes;
        raw = (uint64_t)((int64_t)(raw << sh) >> sh);
    }
    if (ti.kind == Kind::Real) {
        if (ti.bytes == 4) {
            float f;
            memcpy(&f, p, 4);
            s.real = f;
        } else {
            memcpy(&s.real, p, 8);
        }
    } else {
        s.bits = raw;
    }
}

/* Bytes of one row of ne0 elements, 0 where the type is not one the upload knows or ne0 is not a
 * whole number of its blocks (src/gguf.c:85-96: those tensors keep nbytes 0). */
uint64_t bytes_per_row(int type, int64_t ne0)
{
    if (ne0 < 0) return 0;
    struct Blk { int type, elems, bytes; };
    static constexpr Blk kBlk[] = { { QMSG_T_F32, 1, 4 },    { QMSG_T_F16, 1, 2 },   { QMSG_T_Q4_0, 32, 18 },
                                    { QMSG_T_Q4_1, 32, 20 }, { QMSG_T_Q8_0, 32, 34 }, { QMSG_T_Q6_K, 256, 210 } };
    for (const Blk &b : kBlk)
        if (b.type == type) return ne0 % b.elems ? 0 : (uint64_t)(ne0 / b.elems) * (uint64_t)b.bytes;
    return 0;
}

/* A file mapped read-only for the duration of its header parse. */
struct HeaderMap {
    const uint8_t *p = nullptr;
    uint64_t n = 0;
    HeaderMap(int fd, uint64_t size)
    {
        void *m = mmap(nullptr, (size_t)size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m != MAP_FAILED) {
            p = (const uint8_t *)m;
            n = size;
        }
    }
    ~HeaderMap()
    {
        if (p) munmap((void *)p, (size_t)n);
    }
    HeaderMap(const HeaderMap &) = delete;
    HeaderMap &operator=(const HeaderMap &) = delete;
};

/* Metadata section of one shard. Scalars go to g->meta when keep is set (first shard); the
 * shard's own general.alignment is returned through align. */
int read_metadata(FieldReader &rd, uint64_t n_kv, bool keep, qmsg_gguf *g, uint64_t *align, const char *path)
{
    for (uint64_t k = 0; k < n_kv && rd.ok(); k++) {
        qmsg_gguf::Scalar s;
        s.key = cut(rd.text(), kKeyKeep);
        s.type = rd.field<uint32_t>();
        const TypeInfo ti = type_info(s.type);
        if (!rd.ok()) break;
        switch (ti.kind) {
        case Kind::Unsigned:
        case Kind::Signed:
        case Kind::Real: read_scalar(rd, ti, s); break;
        case Kind::Text: s.text = cut(rd.text(), kTextKeep); break;
        default: pass_value(rd, s.type, 0); break;       /* arrays (tokenizer tables) are not kept */
        }
        if (!rd.ok()) break;
        if (s.key == "general.alignment") *align = g->unsigned_view(s);
        if (keep && ti.kind != Kind::List) g->meta.push_back(std::move(s));
    }
    if (!rd.ok()) return refuse("gguf %s: metadata is cut short or holds a value of unknown type", path);
    return QMSG_OK;
}

/* Tensor table of one shard, appended to g->tensors with offsets made absolute. */
int read_tensors(FieldReader &rd, uint64_t n_tensors, int shard, uint64_t align, qmsg_gguf *g, const char *path)
{
    const size_t first = g->tensors.size();
    for (uint64_t k = 0; k < n_tensors; k++) {
        qmsg_tensor t;
        memset(&t, 0, sizeof t);
        const std::string name = cut(rd.text(), kNameKeep);
        memcpy(t.name, name.data(), name.size());
        const uint32_t dims = rd.field<uint32_t>();
        if (!rd.ok() || dims < 1 || dims > 4)
            return refuse("gguf %s: tensor table cut short or a tensor with %u dimensions (1 to 4 allowed)", path,
                          dims);
        t.n_dims = (int)dims;
        for (int d = 0; d < 4; d++) t.ne[d] = d < t.n_dims ? (int64_t)rd.field<uint64_t>() : 1;
        t.type = (int)rd.field<uint32_t>();
        t.off = rd.field<uint64_t>();
        t.shard = shard;
        if (!rd.ok()) return refuse("gguf %s: tensor table cut short at entry %llu", path, (unsigned long long)k);
        g->tensors.push_back(t);
    }
    if (align == 0) return refuse("gguf %s: general.alignment is 0", path);
    uint64_t data = 0;
    if (__builtin_add_overflow(rd.offset(), align - 1, &data))
        return refuse("gguf %s: general.alignment %llu is too large", path, (unsigned long long)align);
    data -= data % align;
    const uint64_t fsize = g->shards[(size_t)shard].size;
    for (size_t k = first; k < g->tensors.size(); k++) {
        qmsg_tensor &t = g->tensors[k];
        const uint64_t rb = bytes_per_row(t.type, t.ne[0]);
        uint64_t rows = 1, nb = 0, end = 0;
        bool bad = __builtin_add_overflow(t.off, data, &t.off);
        if (rb) {
            for (int d = 1; d < 4; d++)
                bad = bad || t.ne[d] < 0 || __builtin_mul_overflow(rows, (uint64_t)t.ne[d], &rows);
            bad = bad || __builtin_mul_overflow(rb, rows, &nb) || __builtin_add_overflow(t.off, nb, &end);
            if (bad || end > fsize)
                return refuse("gguf %s: tensor %s (%lld x %lld x %lld x %lld, type %d) does not fit in the file's "
                              "%llu bytes", path, t.name, (long long)t.ne[0], (long long)t.ne[1], (long long)t.ne[2],
                              (long long)t.ne[3], t.type, (unsigned long long)fsize);
        } else if (bad) {
            return refuse("gguf %s: tensor %s has an offset past 2^64", path, t.name);
        }
        t.nbytes = nb;
    }
    return QMSG_OK;
}

int read_shard(qmsg_gguf *g, int shard)
{
    const qmsg_gguf::Shard &sh = g->shards[(size_t)shard];
    const char *path = sh.path.c_str();
    HeaderMap map(sh.fd, sh.size);
    if (!map.p) return refuse("gguf %s: cannot map the header (%s)", path, strerror(errno));
    FieldReader rd(map.p, map.n);
    const uint8_t *magic = rd.advance(4);
    if (!magic || memcmp(magic, "GGUF", 4) != 0) return refuse("gguf %s: no GGUF magic at offset 0", path);
    const uint32_t version = rd.field<uint32_t>();
    if (!rd.ok() || version != 3) return refuse("gguf %s: format version %u, this reader takes version 3", path, version);
    const uint64_t n_tensors = rd.field<uint64_t>(), n_kv = rd.field<uint64_t>();
    uint64_t align = 32;
    int rc = read_metadata(rd, n_kv, shard == 0, g, &align, path);
    if (rc == QMSG_OK) rc = read_tensors(rd, n_tensors, shard, align, g, path);
    return rc;
}

/* Files of a set: a path ending "-00001-of-NNNNN.gguf" (first shard of N) names N files with
 * the index field counted up; any other path is a single file. */
int expand_set(const std::string &path, std::vector<std::string> &files)
{
    constexpr size_t kTail = sizeof("-00001-of-00000.gguf") - 1;
    auto digits = [](const char *s, int *v) {
        *v = 0;
        for (int i = 0; i < 5; i++) {
            if (s[i] < '0' || s[i] > '9') return false;
            *v = 10 * *v + (s[i] - '0');
        }
        return true;
    };
    const size_t n = path.size();
    int first = 0, count = 0;
    const char *tail = path.c_str() + (n > kTail ? n - kTail : 0);
    const bool is_set = n > kTail && tail[0] == '-' && digits(tail + 1, &first) && first == 1 &&
                        memcmp(tail + 6, "-of-", 4) == 0;
    if (!is_set) {
        files.push_back(path);
        return QMSG_OK;
    }
    if (!digits(tail + 10, &count) || memcmp(tail + 15, ".gguf", 5) != 0 || count < 1 || count > kMaxShards)
        return refuse("gguf %s: a shard set needs 1 to %d files", path.c_str(), kMaxShards);
    const std::string stem = path.substr(0, n - kTail);
    for (int i = 1; i <= count; i++) {
        char idx[kTail + 1];
        snprintf(idx, sizeof idx, "-%05d-of-%05d.gguf", i, count);
        files.push_back(stem + idx);
    }
    return QMSG_OK;
}

int read_fully(int fd, void *dst, uint64_t n, uint64_t off)
{
    uint8_t *d = (uint8_t *)dst;
    for (uint64_t done = 0; done < n;) {
        const uint64_t ask = n - done < (1ull << 30) ? n - done : (1ull << 30);
        const ssize_t got = ::pread(fd, d + done, (size_t)ask, (off_t)(off + done));
        if (got > 0) done += (uint64_t)got;
        else if (!(got < 0 && errno == EINTR)) return -1;
    }
    return 0;
}

}  // namespace

uint64_t qmsg_gguf::unsigned_view(const Scalar &s) const
{
    const Kind k = type_info(s.type).kind;
    return k == Kind::Unsigned || k == Kind::Signed ? s.bits : 0;
}

bool qmsg_gguf::numeric(const Scalar &s, int64_t *i, double *f) const
{
    /* the reference's three views (src/gguf.c:143-153): integers as themselves, reals truncated
     * toward zero for the integer view (x86 conversion: INT64_MIN where the value has no int64) */
    switch (type_info(s.type).kind) {
    case Kind::Unsigned:
        *i = (int64_t)s.bits;
        *f = (double)s.bits;
        return true;
    case Kind::Signed:
        *i = (int64_t)s.bits;
        *f = (double)(int64_t)s.bits;
        return true;
    case Kind::Real:
        *i = s.real >= -0x1p63 && s.real < 0x1p63 ? (int64_t)s.real : INT64_MIN;
        *f = s.real;
        return true;
    default: return false;
    }
}

const qmsg_gguf::Scalar *qmsg_gguf::scalar(const char *key) const
{
    for (const Scalar &s : meta)
        if (s.key == key) return &s;
    return nullptr;
}

namespace qmsg {

int gguf_pread(const qmsg_gguf *g, int shard, uint64_t off, uint64_t n, void *dst)
{
    if (shard < 0 || shard >= (int)g->shards.size()) return -1;
    return read_fully(g->shards[(size_t)shard].fd, dst, n, off);
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
    for (const qmsg_gguf::Shard &s : g->shards)
        if (s.fd >= 0) ::close(s.fd);
    delete g;
}

int qmsg_gguf_open(qmsg_gguf **out, const char *path)
{
    if (!out || !path) return refuse("qmsg_gguf_open: out and path must not be NULL");
    *out = nullptr;
    std::vector<std::string> files;
    int rc = expand_set(path, files);
    if (rc) return rc;
    qmsg_gguf *g = new qmsg_gguf;
    for (size_t i = 0; i < files.size() && rc == QMSG_OK; i++) {
        qmsg_gguf::Shard s;
        s.path = files[i];
        s.fd = ::open(s.path.c_str(), O_RDONLY | O_CLOEXEC);
        struct stat st;
        const bool usable = s.fd >= 0 && fstat(s.fd, &st) == 0 && S_ISREG(st.st_mode) && st.st_size > 0;
        if (usable) s.size = (uint64_t)st.st_size;
        g->shards.push_back(s);
        rc = usable ? read_shard(g, (int)i)
                    : refuse("gguf %s: not a readable, non-empty regular file (%s)", s.path.c_str(),
                             s.fd < 0 ? strerror(errno) : "empty or special");
    }
    if (rc != QMSG_OK) {
        qmsg_gguf_close(g);
        return rc;
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
    const qmsg_gguf::Scalar *s = g->scalar(key);
    double f;
    if (!s || !g->numeric(*s, out, &f)) return refuse("gguf: no numeric scalar %s in the metadata", key);
    return QMSG_OK;
}

int qmsg_gguf_get_float(const qmsg_gguf *g, const char *key, double *out)
{
    if (!g || !key || !out) return QMSG_E_INVALID;
    const qmsg_gguf::Scalar *s = g->scalar(key);
    int64_t i;
    if (!s || !g->numeric(*s, &i, out)) return refuse("gguf: no numeric scalar %s in the metadata", key);
    return QMSG_OK;
}

int qmsg_gguf_get_str(const qmsg_gguf *g, const char *key, char *buf, size_t n)
{
    if (!g || !key || !buf || n == 0) return QMSG_E_INVALID;
    const qmsg_gguf::Scalar *s = g->scalar(key);
    if (!s || s->type != kTypeStr) return refuse("gguf: no string scalar %s in the metadata", key);
    const size_t k = s->text.size() < n - 1 ? s->text.size() : n - 1;
    memcpy(buf, s->text.data(), k);
    buf[k] = '\0';
    return QMSG_OK;
}

int qmsg_gguf_moe_cfg(const qmsg_gguf *g, qmsg_cfg *cfg, int *n_layer, float *eps)
{
    /* the keys the reference's read_cfg takes for the expert layers (src/model.c:275-300) */
    if (!g) return QMSG_E_INVALID;
    const qmsg_gguf::Scalar *arch = g->scalar("general.architecture");
    if (!arch || arch->type != kTypeStr || arch->text != "qwen3moe")
        return refuse("qmsg_gguf_moe_cfg: general.architecture is %s%s%s, not qwen3moe", arch ? "\"" : "",
                      arch ? arch->text.c_str() : "absent", arch ? "\"" : "");
    const char *names[5] = { "qwen3moe.block_count", "qwen3moe.embedding_length", "qwen3moe.expert_count",
                             "qwen3moe.expert_used_count", "qwen3moe.expert_feed_forward_length" };
    int64_t v[5];
    for (int k = 0; k < 5; k++) {
        const int rc = qmsg_gguf_get_int(g, names[k], &v[k]);
        if (rc) return rc;
        if (v[k] <= 0 || v[k] > (1 << 30))
            return refuse("qmsg_gguf_moe_cfg: %s = %lld is outside 1 .. 2^30", names[k], (long long)v[k]);
    }
    double f = 0.0;
    const int rc = qmsg_gguf_get_float(g, "qwen3moe.attention.layer_norm_rms_epsilon", &f);
    if (rc) return rc;
    if (v[3] > v[2])
        return refuse("qmsg_gguf_moe_cfg: expert_used_count %lld exceeds expert_count %lld", (long long)v[3],
                      (long long)v[2]);
    if (cfg) {
        cfg->n_embd = (int)v[1];
        cfg->n_expert = (int)v[2];
        cfg->n_used = (int)v[3];
        cfg->n_ff_exp = (int)v[4];
    }
    if (n_layer) *n_layer = (int)v[0];
    if (eps) *eps = (float)f;
    return QMSG_OK;
}

}  // extern "C"
