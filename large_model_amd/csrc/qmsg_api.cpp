/* qmsg_api.cpp - the C ABI of libqmsg: contexts, resident weights, the layer entry points. */
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <atomic>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/qmsg.h"
#include "qmsg_gguf.h"
#include "qmsg_internal.h"
#include "qmsg_synth.h"

using namespace qmsg;

namespace {

struct LayerStore {
    float *router = nullptr;
    float *norm = nullptr;        /* ffn_norm [E], nullptr: unit weights */
    uint8_t *gate = nullptr, *up = nullptr, *down = nullptr;
    int gate_type = -1, up_type = -1, down_type = -1;
    bool ready = false;
};

/* A dense (trunk) matrix resident in HBM, QmsMat (src/quant.h:11-16) with device data. */
struct DenseStore {
    uint8_t *w = nullptr;
    int type = -1;
    int64_t rows = 0, cols = 0;
    uint64_t rb = 0;
};

struct ProfRec {
    std::string name;
    hipEvent_t a, b;
};

/* qms_row_bytes (src/gguf.c:85-96). */
uint64_t row_bytes(int type, int64_t ne0)
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

thread_local std::string g_create_error;

/* The device scratch arrays of one layer call for T tokens: where each pointer of S goes and
 * how many bytes it needs. */
struct ScratchItem {
    void **p;
    size_t bytes;
};

std::vector<ScratchItem> scratch_items(const qmsg_cfg &cfg, size_t T, Scratch *S)
{
    const size_t E = (size_t)cfg.n_embd, X = (size_t)cfg.n_expert, F = (size_t)cfg.n_ff_exp;
    const size_t NS = T * (size_t)cfg.n_used, nbE = E / 32, nbF = F / 32;
    return {
        { (void **)&S->logits, T * X * 4 },     { (void **)&S->sel, NS * 4 },
        { (void **)&S->wt, NS * 4 },            { (void **)&S->slot_t, NS * 4 },
        { (void **)&S->slot_of, NS * 4 },       { (void **)&S->start, (X + 1) * 4 },
        { (void **)&S->active, X * 4 },         { (void **)&S->meta, 64 },
        { (void **)&S->work, X * 16 },          { (void **)&S->tiles, (X + NS / kTileN + 1) * 16 },
        { (void **)&S->xq, T * nbE * sizeof(Q8) }, { (void **)&S->xqk, T * (nbE / 2) * kPairBytes },
        { (void **)&S->gu, NS * 2 * F * 4 },    { (void **)&S->act, NS * F * 4 },
        { (void **)&S->aq, NS * nbF * sizeof(Q8) }, { (void **)&S->aqk, NS * (nbF / 2) * kPairBytes },
        { (void **)&S->dn, NS * E * 4 },
        { (void **)&S->mxx, T * nbE * kMxRec },  { (void **)&S->mxa, NS * nbF * kMxRec },
        { (void **)&S->mxflag, 16 },
    };
}

/* ---- the allocation-free layer call (qmsg_moe_device_noalloc) ----
 * Its scratch arrays live in this file-scope device array, one copy per GPU, held until the
 * process ends. Host code never passes `scratch` itself (in host code the name is only a
 * stand-in): each device's address comes from hipGetSymbolAddress, taken once per device
 * with that device current (in qmsg_create), and only that address is used. */
constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
constexpr int kMaxDevices = 64;
__device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

std::mutex g_noalloc_mu;
void *g_noalloc_ptr[kMaxDevices];

/* The device's address of `scratch`; the calling thread has `device` current. */
hipError_t noalloc_scratch_setup(int device)
{
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (g_noalloc_ptr[device]) return hipSuccess;
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e == hipSuccess) g_noalloc_ptr[device] = ptr;
    return e;
}

/* Carve the scratch of a T-token call out of [base, base + cap): every array 256-byte aligned
 * and followed by 256 bytes, as dev_alloc pads (kernels may read one aligned word past an
 * array's end). Returns the bytes needed; S is filled only when they fit. */
size_t scratch_carve(const qmsg_cfg &cfg, size_t T, uint8_t *base, size_t cap, Scratch *S)
{
    Scratch tmp{};
    size_t off = 0;
    std::vector<ScratchItem> items = scratch_items(cfg, T, &tmp);
    for (auto &it : items) {
        *it.p = base + off;
        off += ((it.bytes + 255) & ~(size_t)255) + 256;
    }
    if (off <= cap) *S = tmp;
    return off;
}

}  // namespace

struct qmsg_ctx {
    int device = 0;
    qmsg_cfg cfg{};
    int n_layer = 0, max_tokens = 0, path = QMSG_PATH_AUTO;
    int norm_walk = 0;                      /* rmsnorm: form every row's sum in order */
    unsigned long long *d_walked = nullptr; /* rmsnorm: rows that formed it in order */
    float *d_hb = nullptr;                  /* the one-token chain's second row of h */
    int n_cu = 256;
    hipStream_t stream = nullptr;
    std::vector<LayerStore> layers;
    Scratch S{};
    std::vector<void *> scratch_allocs, user_allocs;
    float *d_x = nullptr, *d_out = nullptr;
    std::vector<DenseStore> mats;
    /* grow-on-demand buffers of the dense products: input records, host-call staging */
    void *dense_xqk = nullptr;
    size_t dense_xqk_bytes = 0;
    void *dense_io = nullptr;
    size_t dense_io_bytes = 0;
    std::string err;
    bool prof = false;
    std::vector<ProfRec> prof_recs, prof_free;
    struct Tot { std::string name; int64_t n; double ms; };
    std::vector<Tot> prof_tot;
};

static int fail(qmsg_ctx *c, int code, const char *fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (c) c->err = buf;
    else g_create_error = buf;
    return code;
}

#define HIP_TRY(c, call)                                                                               \
    do {                                                                                               \
        hipError_t e_ = (call);                                                                        \
        if (e_ != hipSuccess) return fail((c), QMSG_E_DEVICE, "%s: %s", #call, hipGetErrorString(e_)); \
    } while (0)

static int dev_alloc(qmsg_ctx *c, void **p, size_t bytes, std::vector<void *> &list)
{
    /* 256 bytes of tail padding: kernels may read one aligned word past a tensor's end. */
    hipError_t e = hipMalloc(p, bytes + 256);
    if (e != hipSuccess) return fail(c, QMSG_E_NOMEM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    list.push_back(*p);
    return QMSG_OK;
}

/* Timing hook: hands out an event pair per kernel dispatch while profiling is on. */
static void prof_events(void *vc, const char *kernel, hipEvent_t *start, hipEvent_t *stop)
{
    qmsg_ctx *c = (qmsg_ctx *)vc;
    ProfRec r;
    if (!c->prof_free.empty()) {
        r = c->prof_free.back();
        c->prof_free.pop_back();
    } else if (hipEventCreate(&r.a) != hipSuccess || hipEventCreate(&r.b) != hipSuccess) {
        return;  /* no events: the launch goes untimed */
    }
    r.name = kernel;
    c->prof_recs.push_back(r);
    *start = r.a;
    *stop = r.b;
}

#define LAUNCH(c, name, expr)                                                                             \
    do {                                                                                                  \
        const LaunchTimer timer_{ (c), prof_events };                                                     \
        g_launch_timer = (c)->prof ? &timer_ : nullptr;                                                   \
        hipError_t e_ = (expr);                                                                           \
        g_launch_timer = nullptr;                                                                         \
        if (e_ != hipSuccess) return fail((c), QMSG_E_DEVICE, "%s launch: %s", (name), hipGetErrorString(e_)); \
    } while (0)

extern "C" {

int qmsg_create(qmsg_ctx **out, int device, const qmsg_cfg *cfg, int n_layer, int max_tokens)
{
    if (!out || !cfg) return fail(nullptr, QMSG_E_INVALID, "qmsg_create: null argument");
    *out = nullptr;
    const int E = cfg->n_embd, X = cfg->n_expert, K = cfg->n_used, F = cfg->n_ff_exp;
    if (E <= 0 || X <= 0 || K <= 0 || F <= 0 || K > X || n_layer <= 0 || max_tokens <= 0)
        return fail(nullptr, QMSG_E_INVALID, "qmsg_create: bad shape E=%d X=%d K=%d F=%d layers=%d T=%d", E, X, K, F,
                    n_layer, max_tokens);
    /* Rows of whole 32-blocks (E % 32 == 0, F % 32 == 0): what the reference's qms_matmul needs
     * for its int8 path (src/quant.c:134-136) on every row the layer has. Shapes off the integer
     * kernels' grid (integer_grid_shape: E % 256, F % 64) run slot by slot, as the reference's
     * moe_group_exact does past its fast gate (src/model.c:1090-1093). The routing keeps
     * per-expert state in 256-entry LDS arrays (X <= 256, K <= 64). */
    if (E % 32 || F % 32 || X > kMaxExperts || K > 64)
        return fail(nullptr, QMSG_E_UNSUPPORTED, "qmsg_create: unsupported shape E=%d X=%d K=%d F=%d", E, X, K, F);
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev)
        return fail(nullptr, QMSG_E_DEVICE, "qmsg_create: HIP device %d not available (%d devices)", device, ndev);
    qmsg_ctx *c = new qmsg_ctx;
    c->device = device;
    c->cfg = *cfg;
    c->n_layer = n_layer;
    c->max_tokens = max_tokens;
    c->layers.resize((size_t)n_layer);
    hipError_t e = hipSetDevice(device);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&c->n_cu, hipDeviceAttributeMultiprocessorCount, device);
    if (e != hipSuccess) {
        fail(nullptr, QMSG_E_DEVICE, "qmsg_create: %s", hipGetErrorString(e));
        delete c;
        return QMSG_E_DEVICE;
    }
    e = noalloc_scratch_setup(device);
    if (e != hipSuccess) {
        fail(nullptr, QMSG_E_DEVICE, "qmsg_create: static scratch of device %d: %s", device, hipGetErrorString(e));
        qmsg_destroy(c);    /* releases the stream */
        return QMSG_E_DEVICE;
    }
    std::vector<ScratchItem> items = scratch_items(*cfg, (size_t)max_tokens, &c->S);
    items.push_back({ (void **)&c->d_x, (size_t)max_tokens * E * 4 });
    items.push_back({ (void **)&c->d_out, (size_t)max_tokens * E * 4 });
    items.push_back({ (void **)&c->d_walked, 8 });
    items.push_back({ (void **)&c->d_hb, (size_t)E * 4 });
    for (auto &it : items) {
        if (dev_alloc(c, it.p, it.bytes, c->scratch_allocs) != QMSG_OK) {
            g_create_error = c->err;
            qmsg_destroy(c);
            return QMSG_E_NOMEM;
        }
    }
    e = hipMemset(c->S.meta, 0, 64);
    if (e == hipSuccess) e = hipMemset(c->d_walked, 0, 8);
    if (e != hipSuccess) {
        fail(nullptr, QMSG_E_DEVICE, "qmsg_create: %s", hipGetErrorString(e));
        qmsg_destroy(c);
        return QMSG_E_DEVICE;
    }
    *out = c;
    return QMSG_OK;
}

void qmsg_destroy(qmsg_ctx *c)
{
    if (!c) return;
    hipSetDevice(c->device);
    if (c->stream) hipStreamSynchronize(c->stream);
    for (auto &L : c->layers) {
        hipFree(L.router);
        hipFree(L.norm);
        hipFree(L.gate);
        hipFree(L.up);
        hipFree(L.down);
    }
    for (auto &m : c->mats) hipFree(m.w);
    hipFree(c->dense_xqk);
    hipFree(c->dense_io);
    for (void *p : c->scratch_allocs) hipFree(p);
    for (void *p : c->user_allocs) hipFree(p);
    for (auto &r : c->prof_recs) { hipEventDestroy(r.a); hipEventDestroy(r.b); }
    for (auto &r : c->prof_free) { hipEventDestroy(r.a); hipEventDestroy(r.b); }
    if (c->stream) hipStreamDestroy(c->stream);
    delete c;
}

const char *qmsg_last_error(const qmsg_ctx *c) { return c ? c->err.c_str() : g_create_error.c_str(); }

void *qmsg_stream(qmsg_ctx *c) { return c ? (void *)c->stream : nullptr; }

int qmsg_set_path(qmsg_ctx *c, int path)
{
    if (!c) return QMSG_E_INVALID;
    if (path != QMSG_PATH_AUTO && path != QMSG_PATH_EXACT && path != QMSG_PATH_MFMA && path != QMSG_PATH_FP32)
        return fail(c, QMSG_E_INVALID, "qmsg_set_path: unknown path %d", path);
    c->path = path;
    return QMSG_OK;
}

static int check_layer_index(qmsg_ctx *c, int layer)
{
    if (layer < 0 || layer >= c->n_layer) return fail(c, QMSG_E_RANGE, "layer %d out of range [0, %d)", layer, c->n_layer);
    return QMSG_OK;
}

/* Allocate a layer's four tensors (freeing an earlier set) for the given types. */
static int layer_alloc(qmsg_ctx *c, LayerStore &L, int gt, int ut, int dt)
{
    const int64_t E = c->cfg.n_embd, X = c->cfg.n_expert, F = c->cfg.n_ff_exp;
    auto known = [](int t) {
        return t == QMSG_T_Q4_0 || t == QMSG_T_Q4_1 || t == QMSG_T_Q6_K || t == QMSG_T_Q8_0 || t == QMSG_T_F16 ||
               t == QMSG_T_F32;
    };
    if (!known(gt) || !known(ut) || !known(dt))
        return fail(c, QMSG_E_UNSUPPORTED,
                    "expert types gate=%d up=%d down=%d: kernels take Q4_0, Q4_1, Q6_K, Q8_0, F16 and F32", gt, ut, dt);
    /* The reference's fast gate (src/model.c:1090-1093) checks gate and down for F32 but not up,
     * and its qms_vec_dot_q8 has no F32 case (src/kernels.c:223-231): such a layer's up rows
     * come out NaN there, its quantiser makes the activation blocks zero, and the layer's
     * output is zero. Refused rather than reproduced. */
    auto fast = [](int t) { return t == QMSG_T_Q4_0 || t == QMSG_T_Q4_1 || t == QMSG_T_Q6_K || t == QMSG_T_F32; };
    if (ut == QMSG_T_F32 && fast(gt) && fast(dt) && gt != QMSG_T_F32 && dt != QMSG_T_F32 && E % 256 == 0)
        return fail(c, QMSG_E_UNSUPPORTED,
                    "F32 up experts with quantised gate and down: the reference's fast path has no F32 dot for them");
    if (dt == QMSG_T_Q6_K && F % 256)
        return fail(c, QMSG_E_UNSUPPORTED, "Q6_K down needs n_ff_exp %% 256 == 0 (got %lld)", (long long)F);
    if ((gt == QMSG_T_Q6_K || ut == QMSG_T_Q6_K) && E % 256)
        return fail(c, QMSG_E_UNSUPPORTED, "Q6_K gate/up needs n_embd %% 256 == 0 (got %lld)", (long long)E);
    hipFree(L.router); hipFree(L.gate); hipFree(L.up); hipFree(L.down);
    float *norm = L.norm;                     /* the ffn_norm weights stay with the layer */
    L = LayerStore{};
    L.norm = norm;
    std::vector<void *> dummy;
    const size_t gb = (size_t)row_bytes(gt, E) * F * X, ub = (size_t)row_bytes(ut, E) * F * X,
                 db = (size_t)row_bytes(dt, F) * E * X;
    int rc;
    if ((rc = dev_alloc(c, (void **)&L.router, (size_t)X * E * 4, dummy)) ||
        (rc = dev_alloc(c, (void **)&L.gate, gb, dummy)) || (rc = dev_alloc(c, (void **)&L.up, ub, dummy)) ||
        (rc = dev_alloc(c, (void **)&L.down, db, dummy))) {
        hipFree(L.router); hipFree(L.gate); hipFree(L.up); hipFree(L.down);
        L = LayerStore{};
        L.norm = norm;
        return rc;
    }
    L.gate_type = gt;
    L.up_type = ut;
    L.down_type = dt;
    return QMSG_OK;
}

static LayerDev layer_dev(const qmsg_ctx *c, const LayerStore &L)
{
    const int64_t E = c->cfg.n_embd, F = c->cfg.n_ff_exp;
    LayerDev d;
    d.router = L.router;
    d.gate = L.gate;
    d.up = L.up;
    d.down = L.down;
    d.gate_type = L.gate_type;
    d.up_type = L.up_type;
    d.down_type = L.down_type;
    d.gate_rb = row_bytes(L.gate_type, E);
    d.up_rb = row_bytes(L.up_type, E);
    d.down_rb = row_bytes(L.down_type, F);
    d.gate_eb = d.gate_rb * F;
    d.up_eb = d.up_rb * F;
    d.down_eb = d.down_rb * E;
    return d;
}

int qmsg_layer_upload(qmsg_ctx *c, int layer, const qmsg_layer *h)
{
    if (!c || !h) return QMSG_E_INVALID;
    int rc = check_layer_index(c, layer);
    if (rc) return rc;
    const int64_t E = c->cfg.n_embd, X = c->cfg.n_expert, F = c->cfg.n_ff_exp;
    if (h->router.type != QMSG_T_F32 || h->router.rows != X || h->router.cols != E ||
        h->router.row_bytes != (uint64_t)E * 4 || !h->router.data)
        return fail(c, QMSG_E_INVALID, "router must be F32 [%lld][%lld]", (long long)X, (long long)E);
    const struct { const qmsg_experts *x; int64_t rows, cols; const char *name; } t[3] = {
        { &h->gate, F, E, "gate" }, { &h->up, F, E, "up" }, { &h->down, E, F, "down" }
    };
    for (auto &k : t) {
        const uint64_t rb = row_bytes(k.x->m.type, k.cols);
        if (!rb || k.x->m.rows != k.rows || k.x->m.cols != k.cols || k.x->m.row_bytes != rb ||
            k.x->expert_bytes != rb * (uint64_t)k.rows || !k.x->m.data)
            return fail(c, QMSG_E_INVALID, "%s experts: expected [%lld x %lld] of type %d with row_bytes %llu", k.name,
                        (long long)k.rows, (long long)k.cols, k.x->m.type, (unsigned long long)rb);
    }
    HIP_TRY(c, hipSetDevice(c->device));
    LayerStore &L = c->layers[(size_t)layer];
    if ((rc = layer_alloc(c, L, h->gate.m.type, h->up.m.type, h->down.m.type))) return rc;
    HIP_TRY(c, hipMemcpy(L.router, h->router.data, (size_t)X * E * 4, hipMemcpyHostToDevice));
    HIP_TRY(c, hipMemcpy(L.gate, h->gate.m.data, h->gate.expert_bytes * X, hipMemcpyHostToDevice));
    HIP_TRY(c, hipMemcpy(L.up, h->up.m.data, h->up.expert_bytes * X, hipMemcpyHostToDevice));
    HIP_TRY(c, hipMemcpy(L.down, h->down.m.data, h->down.expert_bytes * X, hipMemcpyHostToDevice));
    L.ready = true;
    return QMSG_OK;
}

int qmsg_layer_synth(qmsg_ctx *c, int layer, uint64_t seed, int gt, int ut, int dt, float sigma,
                     const float *router_col0)
{
    if (!c) return QMSG_E_INVALID;
    int rc = check_layer_index(c, layer);
    if (rc) return rc;
    const int64_t E = c->cfg.n_embd, X = c->cfg.n_expert, F = c->cfg.n_ff_exp;
    if (!integer_expert_types(gt, ut, dt))
        return fail(c, QMSG_E_UNSUPPORTED, "qmsg_layer_synth: the generator writes Q4_0, Q4_1 and Q6_K experts");
    HIP_TRY(c, hipSetDevice(c->device));
    LayerStore &L = c->layers[(size_t)layer];
    if ((rc = layer_alloc(c, L, gt, ut, dt))) return rc;
    const uint64_t rkey = qmsg_tensor_key(seed, (uint32_t)layer, QMSG_KIND_ROUTER, 0);
    HIP_TRY(c, launch_synth_f32(rkey, (uint64_t)X * E, sigma, L.router, c->stream));
    if (router_col0) {
        float *tmp = nullptr;
        HIP_TRY(c, hipMalloc((void **)&tmp, (size_t)X * 4));
        hipError_t e = hipMemcpyAsync(tmp, router_col0, (size_t)X * 4, hipMemcpyHostToDevice, c->stream);
        if (e == hipSuccess) e = launch_set_col0(L.router, (int)X, (int)E, tmp, 0.0f, c->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
        hipFree(tmp);
        if (e != hipSuccess) return fail(c, QMSG_E_DEVICE, "router bias: %s", hipGetErrorString(e));
    }
    HIP_TRY(c, launch_synth_experts(seed, (uint32_t)layer, QMSG_KIND_GATE, gt, F, E, (int)X, sigma, L.gate, c->stream));
    HIP_TRY(c, launch_synth_experts(seed, (uint32_t)layer, QMSG_KIND_UP, ut, F, E, (int)X, sigma, L.up, c->stream));
    HIP_TRY(c, launch_synth_experts(seed, (uint32_t)layer, QMSG_KIND_DOWN, dt, E, F, (int)X, sigma, L.down, c->stream));
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    L.ready = true;
    return QMSG_OK;
}

int qmsg_layer_download(qmsg_ctx *c, int layer, float *router, void *gate, void *up, void *down)
{
    if (!c) return QMSG_E_INVALID;
    int rc = check_layer_index(c, layer);
    if (rc) return rc;
    const LayerStore &L = c->layers[(size_t)layer];
    if (!L.ready) return fail(c, QMSG_E_INVALID, "layer %d has no weights", layer);
    const LayerDev d = layer_dev(c, L);
    const size_t X = (size_t)c->cfg.n_expert;
    HIP_TRY(c, hipSetDevice(c->device));
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    if (router) HIP_TRY(c, hipMemcpy(router, L.router, X * c->cfg.n_embd * 4, hipMemcpyDeviceToHost));
    if (gate) HIP_TRY(c, hipMemcpy(gate, L.gate, X * d.gate_eb, hipMemcpyDeviceToHost));
    if (up) HIP_TRY(c, hipMemcpy(up, L.up, X * d.up_eb, hipMemcpyDeviceToHost));
    if (down) HIP_TRY(c, hipMemcpy(down, L.down, X * d.down_eb, hipMemcpyDeviceToHost));
    return QMSG_OK;
}

}  // extern "C"

namespace {

/* File -> HBM copies through two pinned staging buffers: while one buffer's bytes travel
 * over PCIe (hipMemcpyAsync on the context's stream), reader threads fill the other with
 * pread. A buffer is refilled only after the event recorded behind its last copy. */
class Stager {
public:
    static constexpr size_t kCap = 64u << 20;        /* bytes per staging buffer            */
    static constexpr size_t kPiece = 8u << 20;       /* bytes per reader thread and fill    */

    explicit Stager(qmsg_ctx *c) : c_(c) {}
    ~Stager()
    {
        for (int k = 0; k < 2; k++) {
            if (ev_[k]) {
                hipEventSynchronize(ev_[k]);
                hipEventDestroy(ev_[k]);
            }
            if (buf_[k]) hipHostFree(buf_[k]);
        }
    }

    int init()
    {
        for (int k = 0; k < 2; k++) {
            if (hipHostMalloc(&buf_[k], kCap, hipHostMallocDefault) != hipSuccess) {
                buf_[k] = nullptr;
                return fail(c_, QMSG_E_NOMEM, "gguf upload: pinned staging buffer of %zu bytes", kCap);
            }
            HIP_TRY(c_, hipEventCreateWithFlags(&ev_[k], hipEventDisableTiming));
        }
        return QMSG_OK;
    }

    /* Tensor t of g (all its bytes) to device address dst. */
    int copy(const qmsg_gguf *g, const qmsg_tensor &t, void *dst)
    {
        for (uint64_t done = 0; done < t.nbytes;) {
            const size_t n = (size_t)(t.nbytes - done < kCap ? t.nbytes - done : kCap);
            const int k = next_;
            next_ ^= 1;
            if (used_[k]) HIP_TRY(c_, hipEventSynchronize(ev_[k]));
            if (read(g, t.shard, t.off + done, n, (uint8_t *)buf_[k]))
                return fail(c_, QMSG_E_INVALID, "gguf upload: read failed for %s", t.name);
            HIP_TRY(c_, hipMemcpyAsync((uint8_t *)dst + done, buf_[k], n, hipMemcpyHostToDevice, c_->stream));
            HIP_TRY(c_, hipEventRecord(ev_[k], c_->stream));
            used_[k] = true;
            done += n;
            bytes_ += n;
        }
        return QMSG_OK;
    }

    int finish()
    {
        HIP_TRY(c_, hipStreamSynchronize(c_->stream));
        return QMSG_OK;
    }

private:
    static int read(const qmsg_gguf *g, int shard, uint64_t off, size_t n, uint8_t *dst)
    {
        const size_t np = (n + kPiece - 1) / kPiece;
        if (np <= 1) return gguf_pread(g, shard, off, n, dst);
        std::vector<std::thread> th;
        std::vector<int> rc(np, 0);
        for (size_t p = 1; p < np; p++)
            th.emplace_back([&, p] {
                const size_t a = p * kPiece, m = n - a < kPiece ? n - a : kPiece;
                rc[p] = gguf_pread(g, shard, off + a, m, dst + a);
            });
        rc[0] = gguf_pread(g, shard, off, kPiece, dst);
        for (auto &x : th) x.join();
        for (int v : rc)
            if (v) return v;
        return 0;
    }

    qmsg_ctx *c_;
    void *buf_[2] = { nullptr, nullptr };
    hipEvent_t ev_[2] = { nullptr, nullptr };
    bool used_[2] = { false, false };
    int next_ = 0;
    uint64_t bytes_ = 0;
};

/* One layer's MoE tensors in the table, checked like load_mat / load_experts / load_f32_vec
 * (src/model.c:52-85, 133-157). */
struct LayerTensors {
    const qmsg_tensor *router, *gate, *up, *down, *norm;
};

int find_layer(qmsg_ctx *c, const qmsg_gguf *g, int l, LayerTensors &out)
{
    const int64_t E = c->cfg.n_embd, X = c->cfg.n_expert, F = c->cfg.n_ff_exp;
    auto need = [&](const char *what, const qmsg_tensor *&t) -> int {
        char name[96];
        snprintf(name, sizeof name, "blk.%d.%s.weight", l, what);
        const int i = gguf_find(g, name);
        if (i < 0) return fail(c, QMSG_E_INVALID, "model: missing tensor %s", name);
        t = &g->tensors[(size_t)i];
        return QMSG_OK;
    };
    int rc;
    if ((rc = need("ffn_gate_inp", out.router)) || (rc = need("ffn_gate_exps", out.gate)) ||
        (rc = need("ffn_up_exps", out.up)) || (rc = need("ffn_down_exps", out.down)) ||
        (rc = need("ffn_norm", out.norm)))
        return rc;
    const qmsg_tensor *r = out.router;
    if (r->ne[0] != E || r->ne[1] != X || r->ne[2] != 1 || !row_bytes(r->type, E))
        return fail(c, QMSG_E_INVALID, "model: %s expected [%lld x %lld], got ne=[%lld,%lld,%lld]", r->name,
                    (long long)X, (long long)E, (long long)r->ne[0], (long long)r->ne[1], (long long)r->ne[2]);
    if (r->type != QMSG_T_F32)
        return fail(c, QMSG_E_UNSUPPORTED, "%s: the router kernels take F32 (got type %d)", r->name, r->type);
    const struct { const qmsg_tensor *t; int64_t rows, cols; } ex[3] = {
        { out.gate, F, E }, { out.up, F, E }, { out.down, E, F }
    };
    for (const auto &k : ex)
        if (k.t->ne[0] != k.cols || k.t->ne[1] != k.rows || k.t->ne[2] != X || !row_bytes(k.t->type, k.cols))
            return fail(c, QMSG_E_INVALID, "model: %s expected [%lld x %lld x %lld], got ne=[%lld,%lld,%lld]", k.t->name,
                        (long long)X, (long long)k.rows, (long long)k.cols, (long long)k.t->ne[0],
                        (long long)k.t->ne[1], (long long)k.t->ne[2]);
    if (out.norm->type != QMSG_T_F32 || out.norm->ne[0] != E)
        return fail(c, QMSG_E_INVALID, "model: %s expected F32[%lld], got type %d [%lld]", out.norm->name,
                    (long long)E, out.norm->type, (long long)out.norm->ne[0]);
    return QMSG_OK;
}

}  // namespace

namespace qmsg {
void set_global_error(const char *msg) { g_create_error = msg; }
}  // namespace qmsg

extern "C" {

int qmsg_gguf_upload(qmsg_ctx *c, const qmsg_gguf *g, int first, int n)
{
    if (!c || !g || n < 0) return QMSG_E_INVALID;
    if (first < 0 || first + n > c->n_layer)
        return fail(c, QMSG_E_RANGE, "layers %d .. %d outside [0, %d)", first, first + n - 1, c->n_layer);
    /* every layer's tensors are checked before any device memory changes */
    std::vector<LayerTensors> lt((size_t)n);
    int rc;
    for (int i = 0; i < n; i++)
        if ((rc = find_layer(c, g, first + i, lt[(size_t)i]))) return rc;
    HIP_TRY(c, hipSetDevice(c->device));
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    Stager st(c);
    if ((rc = st.init())) return rc;
    for (int i = 0; i < n; i++) {
        const LayerTensors &t = lt[(size_t)i];
        LayerStore &L = c->layers[(size_t)(first + i)];
        if ((rc = layer_alloc(c, L, t.gate->type, t.up->type, t.down->type))) return rc;
        if (!L.norm) {
            std::vector<void *> tmp;
            if ((rc = dev_alloc(c, (void **)&L.norm, (size_t)c->cfg.n_embd * 4, tmp))) return rc;
        }
        if ((rc = st.copy(g, *t.router, L.router)) || (rc = st.copy(g, *t.gate, L.gate)) ||
            (rc = st.copy(g, *t.up, L.up)) || (rc = st.copy(g, *t.down, L.down)) || (rc = st.copy(g, *t.norm, L.norm)))
            return rc;
    }
    if ((rc = st.finish())) return rc;
    for (int i = 0; i < n; i++) c->layers[(size_t)(first + i)].ready = true;
    return QMSG_OK;
}

/* ------------------------------------------------------------------ dense (trunk) products ---- */

static int dense_check(qmsg_ctx *c, int type, int64_t rows, int64_t cols, const char *what)
{
    /* the types of qms_matmul_n's fast path (src/quant.c:128-170, qms_fast_supported), and F16
     * and Q8_0, which it (and so every matrix of a call holding one) sends to matmul_exact */
    if (type != QMSG_T_F32 && type != QMSG_T_Q4_0 && type != QMSG_T_Q4_1 && type != QMSG_T_Q6_K &&
        type != QMSG_T_F16 && type != QMSG_T_Q8_0)
        return fail(c, QMSG_E_UNSUPPORTED,
                    "%s: the dense kernels take F32, F16, Q4_0, Q4_1, Q8_0 and Q6_K (got type %d)", what, type);
    const int64_t step = type == QMSG_T_Q6_K ? 256 : 32;     /* src/quant.c:135-136 */
    /* both bounded by 2^30: rows x row bytes stays far inside 64 bits and cols fits an int */
    if (rows <= 0 || rows > (1 << 30) || cols <= 0 || cols > (1 << 30) || cols % step)
        return fail(c, QMSG_E_UNSUPPORTED, "%s: needs 0 < rows, cols <= 2^30 and cols %% %lld == 0 (got %lld x %lld)",
                    what, (long long)step, (long long)rows, (long long)cols);
    /* widths off the chunked kernels' grid (cols % 256, Q6_K cols % 2048) take the direct-read
     * kernel, whose quantised input row must fit in LDS: 48 bytes per 32-block, 160 KiB */
    const bool direct = cols % (type == QMSG_T_Q6_K ? 2048 : 256) != 0;
    const bool exact_only = type == QMSG_T_F16 || type == QMSG_T_Q8_0;
    if (direct && !exact_only && type != QMSG_T_F32 && cols / 32 * 48 > 160 * 1024)
        return fail(c, QMSG_E_UNSUPPORTED, "%s: cols %lld is not a multiple of %d and above %d", what, (long long)cols,
                    type == QMSG_T_Q6_K ? 2048 : 256, 160 * 1024 / 48 * 32);
    /* the fp32-chain kernel stages one input row of cols floats in LDS */
    if (exact_only && cols * 4 > 160 * 1024)
        return fail(c, QMSG_E_UNSUPPORTED, "%s: F16 / Q8_0 rows above %d columns", what, 160 * 1024 / 4);
    return QMSG_OK;
}

/* A new resident matrix of the given shape; its bytes are written by the caller. */
static int dense_new(qmsg_ctx *c, int type, int64_t rows, int64_t cols, int *id)
{
    DenseStore m;
    m.type = type;
    m.rows = rows;
    m.cols = cols;
    m.rb = row_bytes(type, cols);
    std::vector<void *> tmp;
    const int rc = dev_alloc(c, (void **)&m.w, m.rb * (uint64_t)rows, tmp);
    if (rc) return rc;
    c->mats.push_back(m);
    *id = (int)c->mats.size() - 1;
    return QMSG_OK;
}

int qmsg_mat_upload(qmsg_ctx *c, const qmsg_mat *h, int *id)
{
    if (!c || !h || !id || !h->data) return QMSG_E_INVALID;
    int rc = dense_check(c, h->type, h->rows, h->cols, "qmsg_mat_upload");
    if (rc) return rc;
    if (h->row_bytes != row_bytes(h->type, h->cols))
        return fail(c, QMSG_E_INVALID, "qmsg_mat_upload: row_bytes %llu, expected %llu",
                    (unsigned long long)h->row_bytes, (unsigned long long)row_bytes(h->type, h->cols));
    HIP_TRY(c, hipSetDevice(c->device));
    if ((rc = dense_new(c, h->type, h->rows, h->cols, id))) return rc;
    const DenseStore &m = c->mats[(size_t)*id];
    HIP_TRY(c, hipMemcpy(m.w, h->data, m.rb * (uint64_t)m.rows, hipMemcpyHostToDevice));
    return QMSG_OK;
}

int qmsg_mat_synth(qmsg_ctx *c, int type, int64_t rows, int64_t cols, uint64_t seed, float sigma, int *id)
{
    if (!c || !id) return QMSG_E_INVALID;
    int rc = dense_check(c, type, rows, cols, "qmsg_mat_synth");
    if (rc) return rc;
    if (type == QMSG_T_F16 || type == QMSG_T_Q8_0)
        return fail(c, QMSG_E_UNSUPPORTED, "qmsg_mat_synth: the generator writes F32, Q4_0, Q4_1 and Q6_K");
    HIP_TRY(c, hipSetDevice(c->device));
    if ((rc = dense_new(c, type, rows, cols, id))) return rc;
    /* the generator of the expert tensors with one "expert" of kind gate, layer 0 (F32: the
     * generator's normal values) */
    if (type == QMSG_T_F32)
        HIP_TRY(c, launch_synth_f32(qmsg_tensor_key(seed, 0, QMSG_KIND_GATE, 0), (uint64_t)rows * (uint64_t)cols, sigma,
                                    (float *)c->mats[(size_t)*id].w, c->stream));
    else
        HIP_TRY(c, launch_synth_experts(seed, 0, QMSG_KIND_GATE, type, rows, cols, 1, sigma, c->mats[(size_t)*id].w,
                                        c->stream));
    return QMSG_OK;
}

int qmsg_gguf_upload_mat(qmsg_ctx *c, const qmsg_gguf *g, const char *name, int *id)
{
    if (!c || !g || !name || !id) return QMSG_E_INVALID;
    const int i = gguf_find(g, name);
    if (i < 0) return fail(c, QMSG_E_INVALID, "model: missing tensor %s", name);
    const qmsg_tensor &t = g->tensors[(size_t)i];
    if (t.n_dims != 2 || t.ne[2] != 1 || t.ne[3] != 1)
        return fail(c, QMSG_E_INVALID, "model: %s is not a 2-D matrix (ne=[%lld,%lld,%lld])", name, (long long)t.ne[0],
                    (long long)t.ne[1], (long long)t.ne[2]);
    int rc = dense_check(c, t.type, t.ne[1], t.ne[0], name);
    if (rc) return rc;
    HIP_TRY(c, hipSetDevice(c->device));
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    int nid = -1;
    if ((rc = dense_new(c, t.type, t.ne[1], t.ne[0], &nid))) return rc;
    Stager st(c);
    if ((rc = st.init()) || (rc = st.copy(g, t, c->mats[(size_t)nid].w)) || (rc = st.finish())) return rc;
    *id = nid;
    return QMSG_OK;
}

/* Device buffer *p of at least `bytes`, reallocated (after the stream drains) when smaller. */
static int grow(qmsg_ctx *c, void **p, size_t *cap, size_t bytes)
{
    if (*cap >= bytes) return QMSG_OK;
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    hipFree(*p);
    *p = nullptr;
    *cap = 0;
    std::vector<void *> tmp;
    const int rc = dev_alloc(c, p, bytes, tmp);
    if (rc == QMSG_OK) *cap = bytes;
    return rc;
}

int qmsg_matmul_n_device(qmsg_ctx *c, const int *ids, int nW, const float *d_x, int T, float *const *d_ys)
{
    if (!c || !ids || !d_ys || nW <= 0 || T < 0) return QMSG_E_INVALID;
    int64_t C = -1;
    for (int i = 0; i < nW; i++) {
        if (ids[i] < 0 || ids[i] >= (int)c->mats.size())
            return fail(c, QMSG_E_INVALID, "qmsg_matmul_n: matrix id %d unknown", ids[i]);
        const DenseStore &m = c->mats[(size_t)ids[i]];
        if (C >= 0 && m.cols != C) return fail(c, QMSG_E_INVALID, "qmsg_matmul_n: matrices differ in cols");
        C = m.cols;
        if (!d_ys[i] || ((uintptr_t)d_ys[i] & 3)) return fail(c, QMSG_E_INVALID, "qmsg_matmul_n: output %d", i);
    }
    if (T == 0) return QMSG_OK;
    if (!d_x || ((uintptr_t)d_x & 15)) return fail(c, QMSG_E_INVALID, "qmsg_matmul_n: x must be 16-byte aligned");
    HIP_TRY(c, hipSetDevice(c->device));
    if (T >= kDenseQuantT) {
        const int rc = grow(c, &c->dense_xqk, &c->dense_xqk_bytes, (size_t)T * (size_t)(C / 64) * kPairBytes);
        if (rc) return rc;
    }
    /* qms_matmul_n's choice for the whole call (src/quant.c:131-141): the fast loop, or
     * matmul_exact for every matrix when --exact is set or one of them is F16 / Q8_0 */
    bool exact = c->path == QMSG_PATH_FP32;
    for (int i = 0; i < nW; i++) {
        const int t = c->mats[(size_t)ids[i]].type;
        exact = exact || t == QMSG_T_F16 || t == QMSG_T_Q8_0;
    }
    if (exact && C * 4 > 160 * 1024)
        return fail(c, QMSG_E_UNSUPPORTED, "qmsg_matmul_n: fp32-chain rows above %d columns", 160 * 1024 / 4);
    /* launches of up to kDenseMats matrices of one type, in argument order */
    std::vector<bool> done((size_t)nW, false);
    for (int i = 0; i < nW; i++) {
        if (done[(size_t)i]) continue;
        const int type = c->mats[(size_t)ids[i]].type;
        DenseArgs a{};
        a.rb = c->mats[(size_t)ids[i]].rb;
        a.C = (int)C;
        a.T = T;
        a.x = d_x;
        for (int j = i; j < nW && a.nm < kDenseMats; j++) {
            const DenseStore &m = c->mats[(size_t)ids[j]];
            if (done[(size_t)j] || m.type != type) continue;
            a.m[a.nm].w = m.w;
            a.m[a.nm].y = d_ys[j];
            a.m[a.nm].rows = (int)m.rows;
            a.nm++;
            done[(size_t)j] = true;
        }
        if (exact) LAUNCH(c, "dense", launch_dense_exact(a, type, c->stream));
        else LAUNCH(c, "dense", launch_dense(a, type, (uint8_t *)c->dense_xqk, c->stream));
    }
    return QMSG_OK;
}

int qmsg_matmul_n(qmsg_ctx *c, const int *ids, int nW, const float *x, int T, float *const *ys)
{
    if (!c || !ids || !ys || nW <= 0 || T < 0) return QMSG_E_INVALID;
    for (int i = 0; i < nW; i++)
        if (ids[i] < 0 || ids[i] >= (int)c->mats.size())
            return fail(c, QMSG_E_INVALID, "qmsg_matmul_n: matrix id %d unknown", ids[i]);
    if (T == 0) return QMSG_OK;
    if (!x) return QMSG_E_INVALID;
    const int64_t C = c->mats[(size_t)ids[0]].cols;
    size_t bytes = (size_t)T * (size_t)C * 4;
    std::vector<size_t> off((size_t)nW);
    for (int i = 0; i < nW; i++) {
        off[(size_t)i] = bytes;
        bytes += ((size_t)T * (size_t)c->mats[(size_t)ids[i]].rows * 4 + 255) & ~(size_t)255;
    }
    HIP_TRY(c, hipSetDevice(c->device));
    int rc = grow(c, &c->dense_io, &c->dense_io_bytes, bytes);
    if (rc) return rc;
    uint8_t *io = (uint8_t *)c->dense_io;
    std::vector<float *> dy((size_t)nW);
    for (int i = 0; i < nW; i++) dy[(size_t)i] = (float *)(io + off[(size_t)i]);
    HIP_TRY(c, hipMemcpyAsync(io, x, (size_t)T * (size_t)C * 4, hipMemcpyHostToDevice, c->stream));
    if ((rc = qmsg_matmul_n_device(c, ids, nW, (const float *)io, T, dy.data()))) return rc;
    for (int i = 0; i < nW; i++)
        HIP_TRY(c, hipMemcpyAsync(ys[i], dy[(size_t)i], (size_t)T * (size_t)c->mats[(size_t)ids[i]].rows * 4,
                                  hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    return QMSG_OK;
}

/* One layer on device buffers with the scratch arrays S (the context's, or carved from the
 * library's static array by qmsg_moe_device_noalloc). With ni (one token, rows route_norm_fits
 * takes, not the fp32 path) the router launch forms xn = ni's rmsnorm itself and stores it to
 * d_xn (= ni->xn_out) for the launches after it. */
static int run_layer_s(qmsg_ctx *c, const Scratch &S0, int layer, const float *d_xn, int T, float *d_out, int debug,
                       const NormIn *ni = nullptr)
{
    /* every layer call gets an epoch of its own: record producers store it in S.mxflag when a
     * record falls outside the MFMA kernels' scaled range, and the consumers compare */
    static std::atomic<uint64_t> epochs{ 0 };
    Scratch S = S0;
    S.epoch = ++epochs;
    int rc = check_layer_index(c, layer);
    if (rc) return rc;
    const LayerStore &L = c->layers[(size_t)layer];
    if (!L.ready) return fail(c, QMSG_E_INVALID, "layer %d has no weights", layer);
    if (T == 0) return QMSG_OK;
    if (((uintptr_t)d_xn & 15) || ((uintptr_t)d_out & 3))
        return fail(c, QMSG_E_INVALID, "device buffers must be 16-byte aligned (xn) and 4-byte aligned (out)");
    const Shape s{ c->cfg.n_embd, c->cfg.n_expert, c->cfg.n_used, c->cfg.n_ff_exp };
    const LayerDev d = layer_dev(c, L);
    const bool types = integer_expert_types(d.gate_type, d.up_type, d.down_type);
    const bool integer = integer_grid_shape(s.E, s.F) && types;
    /* n_ff_exp an odd multiple of 32 at an n_embd on the grid: the streaming gate/up kernel
     * (rows n_embd wide) and the slot kernels for the down rows */
    const bool odd_f = !integer && types && s.E % 256 == 0 && s.F % 64 == 32 && gateup_streams(d) &&
                       c->path != QMSG_PATH_FP32;
    if (ni && (T != 1 || c->path == QMSG_PATH_FP32 || !route_norm_fits(s.E) || !integer || ni->xn_out != d_xn))
        return fail(c, QMSG_E_INVALID, "run_layer_s: the fused rmsnorm takes one token on the integer paths");
    if (odd_f) {
        LAUNCH(c, "route", launch_route(s, d, S, d_xn, T, c->stream));
        LAUNCH(c, "select", launch_select(s, S, T, 1, c->stream));
        LAUNCH(c, "gateup", launch_gateup_exact(s, d, S, T, debug, c->n_cu, 0, c->stream));
        LAUNCH(c, "down", launch_layer_slots(s, d, S, d_xn, d_out, T, 0, debug, c->stream, 1));
        return QMSG_OK;
    }
    if (c->path == QMSG_PATH_FP32 || !integer) {
        LAUNCH(c, "layer", launch_layer_slots(s, d, S, d_xn, d_out, T, c->path == QMSG_PATH_FP32 ? 1 : 0, debug,
                                              c->stream));
        return QMSG_OK;
    }
    /* gate and up of one type take the streaming gate/up kernel (which also routes one-token
     * batches), mixed types the slot-tile row kernel; batches with several slots per expert
     * take the MFMA kernels when gate and up share a type */
    const bool q4 = gateup_streams(d);      /* the streaming gate/up kernel takes gate and up */
    int dn_ok = 0;
    const bool many = !use_small_route(T, s.K);
    const bool gu_ok = mx_supported(s, d, &dn_ok) && many;   /* gate and up of one type */
    const bool forced = c->path == QMSG_PATH_MFMA, autop = c->path == QMSG_PATH_AUTO;
    /* against the streaming kernel the MFMA kernels win from 1.25 slots per expert (Q4_1:
     * 139.7 / 128.2 us at 16 tokens, 173.8 / 174.0 at 24, 196.3 / 216.6 at 32), or 2.5 for Q6_K */
    const bool gu_mx = gu_ok && (forced || (autop && mx_auto(T, s.K, s.X, d.gate_type)));
    /* rows too long for every exact down kernel's LDS (n_ff_exp 14336: 8 KB per Q4_0 row) take
     * the MFMA down kernel on any path that allows it */
    const bool dn_long = dn_ok && T >= 2 && c->path != QMSG_PATH_EXACT && !down_exact_fits(s, d, T);
    const bool dn_mx = dn_ok && (dn_long || (many && (forced || (autop && mx_auto_down(T, s.K, d.down_type)))));
    if (ni) LAUNCH(c, "route", launch_route_norm(s, d, S, *ni, c->stream));
    else LAUNCH(c, "route", launch_route(s, d, S, d_xn, T, c->stream));
    LAUNCH(c, "select", launch_select(s, S, T, q4 ? 1 : 0, c->stream));
    if (gu_mx) {
        LAUNCH(c, "experts", launch_experts_mx(s, d, S, d_out, T, debug, c->stream));
        return QMSG_OK;
    }
    /* two to four tokens: the streaming gate/up stores the activations' int8 blocks once,
     * instead of every block of the small-batch down kernel forming them (235B shape, 4
     * tokens: down 34.4 -> 29.9 us, gate/up in 32-row blocks 45.3 -> 48.5, 1-2 us per layer) */
    const bool qa = q4 && !dn_mx && down_small_fits(s, d, T) && s.F % 32 == 0;
    if (!q4) LAUNCH(c, "gateup", launch_gateup_tiles(s, d, S, T, c->stream));
    else LAUNCH(c, "gateup", launch_gateup_exact(s, d, S, T, debug, c->n_cu, qa ? 1 : 0, c->stream));
    if (dn_mx) LAUNCH(c, "down", launch_down_mx(s, d, S, d_out, T, c->stream));
    else LAUNCH(c, "down", launch_down_exact(s, d, S, d_out, T, qa ? 0 : 1, c->stream));
    return QMSG_OK;
}

static int run_layer(qmsg_ctx *c, int layer, const float *d_xn, int T, float *d_out, int debug)
{
    if (T < 0 || T > c->max_tokens)
        return fail(c, QMSG_E_RANGE, "T=%d outside [0, max_tokens=%d]", T, c->max_tokens);
    return run_layer_s(c, c->S, layer, d_xn, T, d_out, debug);
}

int qmsg_moe_device(qmsg_ctx *c, int layer, const float *d_xn, int T, float *d_out)
{
    if (!c) return QMSG_E_INVALID;
    return run_layer(c, layer, d_xn, T, d_out, 0);
}

int qmsg_moe_device_noalloc(qmsg_ctx *c, int layer, const float *d_xn, int T, float *d_out)
{
    if (!c) return QMSG_E_INVALID;
    if (T < 0) return fail(c, QMSG_E_RANGE, "T=%d is negative", T);
    if (c->device < 0 || c->device >= kMaxDevices || !g_noalloc_ptr[c->device])
        return fail(c, QMSG_E_DEVICE, "qmsg_moe_device_noalloc: no static scratch on device %d", c->device);
    Scratch S{};
    const size_t need = scratch_carve(c->cfg, (size_t)T, (uint8_t *)g_noalloc_ptr[c->device], kNoAllocScratchBytes, &S);
    if (need > kNoAllocScratchBytes)
        return fail(c, QMSG_E_RANGE,
                    "qmsg_moe_device_noalloc: T=%d needs %zu bytes of scratch, above the static maximum of %zu", T,
                    need, kNoAllocScratchBytes);
    if (T == 0) return run_layer_s(c, S, layer, d_xn, T, d_out, 0);
    HIP_TRY(c, hipSetDevice(c->device));
    /* the select kernel's ticket counter (meta[4]) must start at zero, and the record-range
     * flags are cleared so a replay of a captured call does not inherit an earlier replay's */
    LAUNCH(c, "fill", launch_call_reset(S, c->stream));
    return run_layer_s(c, S, layer, d_xn, T, d_out, 0);
}

int qmsg_layer_norm(qmsg_ctx *c, int layer, const float *w)
{
    if (!c) return QMSG_E_INVALID;
    int rc = check_layer_index(c, layer);
    if (rc) return rc;
    HIP_TRY(c, hipSetDevice(c->device));
    LayerStore &L = c->layers[(size_t)layer];
    if (!w) {
        hipFree(L.norm);
        L.norm = nullptr;
        return QMSG_OK;
    }
    const size_t bytes = (size_t)c->cfg.n_embd * 4;
    if (!L.norm) {
        std::vector<void *> tmp;
        if ((rc = dev_alloc(c, (void **)&L.norm, bytes, tmp))) return rc;
    }
    HIP_TRY(c, hipMemcpy(L.norm, w, bytes, hipMemcpyHostToDevice));
    return QMSG_OK;
}

int qmsg_moe_chain(qmsg_ctx *c, int first, int n, float *d_h, int T, float eps)
{
    if (!c || !d_h || n < 0) return QMSG_E_INVALID;
    if (first < 0 || first + n > c->n_layer)
        return fail(c, QMSG_E_RANGE, "layers %d .. %d outside [0, %d)", first, first + n - 1, c->n_layer);
    if (T < 0 || T > c->max_tokens) return fail(c, QMSG_E_RANGE, "T=%d outside [0, max_tokens=%d]", T, c->max_tokens);
    if (T == 0 || n == 0) return QMSG_OK;
    if ((uintptr_t)d_h & 15) return fail(c, QMSG_E_INVALID, "qmsg_moe_chain: d_h must be 16-byte aligned");
    HIP_TRY(c, hipSetDevice(c->device));
    const int E = c->cfg.n_embd;
    bool integer = integer_grid_shape(E, c->cfg.n_ff_exp);
    for (int l = first; l < first + n; l++) {
        const LayerStore &L = c->layers[(size_t)l];
        if (!L.ready) return fail(c, QMSG_E_INVALID, "layer %d has no weights", l);
        integer = integer && integer_expert_types(L.gate_type, L.up_type, L.down_type);
    }
    if (T == 1 && c->path != QMSG_PATH_FP32 && route_norm_fits(E) && integer) {
        /* One token: each layer's router launch forms the rmsnorm itself, every block from h
         * and the previous layer's output, so h + out goes to the other of two rows (d_h and
         * d_hb, in turn) while the blocks still read the first. */
        float *cur = d_h;
        for (int l = first; l < first + n; l++) {
            const float *pending = l > first ? c->d_out : nullptr;
            float *next = pending ? (cur == d_h ? c->d_hb : d_h) : cur;
            const NormIn ni{ cur, pending, c->layers[(size_t)l].norm, pending ? next : nullptr, c->d_x, eps,
                             c->norm_walk, c->d_walked };
            const int rc = run_layer_s(c, c->S, l, c->d_x, T, c->d_out, 0, &ni);
            if (rc) return rc;
            cur = next;
        }
        LAUNCH(c, "add", launch_add_rows_to(d_h, cur, c->d_out, (size_t)E, c->stream));
        return QMSG_OK;
    }
    /* each layer's residual add h += out rides in the next layer's rmsnorm launch */
    for (int l = first; l < first + n; l++) {
        const float *pending = l > first ? c->d_out : nullptr;
        LAUNCH(c, "rmsnorm", launch_rmsnorm(d_h, pending, c->layers[(size_t)l].norm, c->d_x, T, E, eps, c->norm_walk,
                                             c->d_walked, c->stream));
        const int rc = run_layer(c, l, c->d_x, T, c->d_out, 0);
        if (rc) return rc;
    }
    LAUNCH(c, "add", launch_add_rows(d_h, c->d_out, (size_t)T * E, c->stream));
    return QMSG_OK;
}

int qmsg_rmsnorm_device(qmsg_ctx *c, float *d_y, const float *d_x, const float *d_w, int rows, int n, float eps)
{
    if (!c) return QMSG_E_INVALID;
    if (rows < 0 || n <= 0 || n % 4) return fail(c, QMSG_E_INVALID, "qmsg_rmsnorm_device: rows=%d n=%d (n a positive multiple of 4)", rows, n);
    if (rmsnorm_lds_bytes(n) > 160 * 1024)
        return fail(c, QMSG_E_UNSUPPORTED, "qmsg_rmsnorm_device: rows of %d floats exceed the kernel's LDS", n);
    if (rows == 0) return QMSG_OK;
    if (!d_x || !d_y) return fail(c, QMSG_E_INVALID, "qmsg_rmsnorm_device: null buffer");
    if (((uintptr_t)d_x | (uintptr_t)d_y | (uintptr_t)d_w) & 15)
        return fail(c, QMSG_E_INVALID, "qmsg_rmsnorm_device: d_x, d_y and d_w must be 16-byte aligned");
    HIP_TRY(c, hipSetDevice(c->device));
    LAUNCH(c, "rmsnorm", launch_rmsnorm(const_cast<float *>(d_x), nullptr, d_w, d_y, rows, n, eps, c->norm_walk,
                                         c->d_walked, c->stream));
    return QMSG_OK;
}

int qmsg_rmsnorm_mode(qmsg_ctx *c, int always_walk, int64_t *walked)
{
    if (!c) return QMSG_E_INVALID;
    if (always_walk != 0 && always_walk != 1) return fail(c, QMSG_E_INVALID, "qmsg_rmsnorm_mode: always_walk=%d", always_walk);
    HIP_TRY(c, hipSetDevice(c->device));
    if (walked) {
        unsigned long long n = 0;
        const unsigned long long zero = 0;
        HIP_TRY(c, hipStreamSynchronize(c->stream));
        HIP_TRY(c, hipMemcpy(&n, c->d_walked, 8, hipMemcpyDeviceToHost));
        HIP_TRY(c, hipMemcpy(c->d_walked, &zero, 8, hipMemcpyHostToDevice));
        *walked = (int64_t)n;
    }
    c->norm_walk = always_walk;
    return QMSG_OK;
}

int qmsg_moe(qmsg_ctx *c, int layer, const float *xn, const float *h, int T, float *out)
{
    (void)h;
    if (!c) return QMSG_E_INVALID;
    if (T < 0 || T > c->max_tokens) return fail(c, QMSG_E_RANGE, "T=%d outside [0, max_tokens=%d]", T, c->max_tokens);
    if (T == 0) return QMSG_OK;
    if (!xn || !out) return fail(c, QMSG_E_INVALID, "qmsg_moe: null buffer");
    const size_t bytes = (size_t)T * c->cfg.n_embd * 4;
    HIP_TRY(c, hipSetDevice(c->device));
    HIP_TRY(c, hipMemcpyAsync(c->d_x, xn, bytes, hipMemcpyHostToDevice, c->stream));
    int rc = run_layer(c, layer, c->d_x, T, c->d_out, 0);
    if (rc) return rc;
    HIP_TRY(c, hipMemcpyAsync(out, c->d_out, bytes, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    return QMSG_OK;
}

int qmsg_sync(qmsg_ctx *c)
{
    if (!c) return QMSG_E_INVALID;
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    return QMSG_OK;
}

void *qmsg_device_alloc(qmsg_ctx *c, size_t bytes)
{
    if (!c) return nullptr;
    void *p = nullptr;
    if (hipSetDevice(c->device) != hipSuccess) return nullptr;
    if (dev_alloc(c, &p, bytes, c->user_allocs) != QMSG_OK) return nullptr;
    return p;
}

int qmsg_memcpy_h2d(qmsg_ctx *c, void *dst, const void *src, size_t bytes)
{
    if (!c) return QMSG_E_INVALID;
    HIP_TRY(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    return QMSG_OK;
}

int qmsg_memcpy_d2h(qmsg_ctx *c, void *dst, const void *src, size_t bytes)
{
    if (!c) return QMSG_E_INVALID;
    HIP_TRY(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    return QMSG_OK;
}

int qmsg_synth_input(qmsg_ctx *c, uint64_t seed, int layer, int T, float sigma, int rmsnorm, int bias_col0, float *d_x)
{
    if (!c || !d_x || T < 0) return QMSG_E_INVALID;
    const int E = c->cfg.n_embd;
    const uint64_t key = qmsg_tensor_key(seed, (uint32_t)layer, QMSG_KIND_X, 0);
    HIP_TRY(c, hipSetDevice(c->device));
    HIP_TRY(c, launch_synth_f32(key, (uint64_t)T * E, sigma, d_x, c->stream));
    if (rmsnorm) HIP_TRY(c, launch_rmsnorm_rows(d_x, T, E, 1e-6f, c->stream));
    if (bias_col0) HIP_TRY(c, launch_set_col0(d_x, T, E, nullptr, 1.0f, c->stream));
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    return QMSG_OK;
}

int qmsg_moe_debug(qmsg_ctx *c, int layer, const float *xn, int T, float *out, qmsg_debug *g)
{
    if (!c || !xn || !out) return QMSG_E_INVALID;
    if (T <= 0 || T > c->max_tokens) return fail(c, QMSG_E_RANGE, "T=%d outside [1, max_tokens=%d]", T, c->max_tokens);
    const size_t E = c->cfg.n_embd, X = c->cfg.n_expert, K = c->cfg.n_used, F = c->cfg.n_ff_exp, NS = (size_t)T * K;
    HIP_TRY(c, hipSetDevice(c->device));
    HIP_TRY(c, hipMemcpyAsync(c->d_x, xn, (size_t)T * E * 4, hipMemcpyHostToDevice, c->stream));
    int rc = run_layer(c, layer, c->d_x, T, c->d_out, 1);
    if (rc) return rc;
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    HIP_TRY(c, hipMemcpy(out, c->d_out, (size_t)T * E * 4, hipMemcpyDeviceToHost));
    if (!g) return QMSG_OK;
    struct { void *dst; const void *src; size_t bytes; } cp[] = {
        { g->logits, c->S.logits, (size_t)T * X * 4 }, { g->sel, c->S.sel, NS * 4 },
        { g->wt, c->S.wt, NS * 4 },                    { g->start, c->S.start, (X + 1) * 4 },
        { g->slot_t, c->S.slot_t, NS * 4 },            { g->slot_of, c->S.slot_of, NS * 4 },
        { g->active, c->S.active, X * 4 },             { g->n_active, c->S.meta, 4 },
        { g->xq, c->S.xq, (size_t)T * (E / 32) * sizeof(Q8) }, { g->gu, c->S.gu, NS * 2 * F * 4 },
        { g->act, c->S.act, NS * F * 4 },              { g->aq, c->S.aq, NS * (F / 32) * sizeof(Q8) },
        { g->dn, c->S.dn, NS * E * 4 },
    };
    for (auto &x : cp)
        if (x.dst) HIP_TRY(c, hipMemcpy(x.dst, x.src, x.bytes, hipMemcpyDeviceToHost));
    return QMSG_OK;
}

int qmsg_block_dots(qmsg_ctx *c, int layer, int which, int n, const int32_t *expert, const int32_t *row,
                    const int32_t *block, const void *xq_blocks, int32_t *out)
{
    if (!c || n < 0 || which < 0 || which > 2) return QMSG_E_INVALID;
    int rc = check_layer_index(c, layer);
    if (rc) return rc;
    if (n == 0) return QMSG_OK;
    const LayerStore &L = c->layers[(size_t)layer];
    if (!L.ready) return fail(c, QMSG_E_INVALID, "layer %d has no weights", layer);
    const LayerDev d = layer_dev(c, L);
    const uint8_t *base = which == 0 ? d.gate : (which == 1 ? d.up : d.down);
    const int type = which == 0 ? d.gate_type : (which == 1 ? d.up_type : d.down_type);
    if (type != QMSG_T_Q4_0 && type != QMSG_T_Q4_1 && type != QMSG_T_Q6_K)
        return fail(c, QMSG_E_UNSUPPORTED, "qmsg_block_dots: int8 block dots take Q4_0, Q4_1 and Q6_K rows (type %d)",
                    type);
    const uint64_t rb = which == 0 ? d.gate_rb : (which == 1 ? d.up_rb : d.down_rb);
    const uint64_t eb = which == 0 ? d.gate_eb : (which == 1 ? d.up_eb : d.down_eb);
    const int64_t rows = which == 2 ? c->cfg.n_embd : c->cfg.n_ff_exp;
    const int64_t nblk = (which == 2 ? c->cfg.n_ff_exp : c->cfg.n_embd) / 32;
    for (int i = 0; i < n; i++)
        if (expert[i] < 0 || expert[i] >= c->cfg.n_expert || row[i] < 0 || row[i] >= rows || block[i] < 0 ||
            block[i] >= nblk)
            return fail(c, QMSG_E_INVALID, "qmsg_block_dots: entry %d out of range", i);
    HIP_TRY(c, hipSetDevice(c->device));
    std::vector<void *> tmp;
    int32_t *dbuf = nullptr;
    Q8 *dx = nullptr;
    const size_t ib = (size_t)n * 4;
    if ((rc = dev_alloc(c, (void **)&dbuf, ib * 4, tmp))) return rc;
    if ((rc = dev_alloc(c, (void **)&dx, (size_t)n * sizeof(Q8), tmp))) { hipFree(dbuf); return rc; }
    hipError_t e = hipMemcpy(dbuf, expert, ib, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(dbuf + n, row, ib, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(dbuf + 2 * n, block, ib, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(dx, xq_blocks, (size_t)n * sizeof(Q8), hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = launch_block_dots(base, type, rb, eb, n, dbuf, dbuf + n, dbuf + 2 * n, dx, dbuf + 3 * n, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e == hipSuccess) e = hipMemcpy(out, dbuf + 3 * n, ib, hipMemcpyDeviceToHost);
    hipFree(dbuf);
    hipFree(dx);
    if (e != hipSuccess) return fail(c, QMSG_E_DEVICE, "qmsg_block_dots: %s", hipGetErrorString(e));
    return QMSG_OK;
}

int qmsg_profile(qmsg_ctx *c, int enable)
{
    if (!c) return QMSG_E_INVALID;
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    for (auto &r : c->prof_recs) c->prof_free.push_back(r);
    c->prof_recs.clear();
    c->prof_tot.clear();
    c->prof = enable != 0;
    return QMSG_OK;
}

int qmsg_profile_read(qmsg_ctx *c, const char *name, int64_t *launches, double *total_ms)
{
    if (!c || !name) return QMSG_E_INVALID;
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    for (auto &r : c->prof_recs) {
        float ms = 0.0f;
        HIP_TRY(c, hipEventElapsedTime(&ms, r.a, r.b));
        bool found = false;
        for (auto &t : c->prof_tot)
            if (t.name == r.name) { t.n++; t.ms += ms; found = true; break; }
        if (!found) c->prof_tot.push_back({ r.name, 1, (double)ms });
        c->prof_free.push_back(r);
    }
    c->prof_recs.clear();
    int64_t n = 0;
    double ms = 0.0;
    for (auto &t : c->prof_tot)
        if (t.name == name) { n = t.n; ms = t.ms; }
    if (launches) *launches = n;
    if (total_ms) *total_ms = ms;
    return QMSG_OK;
}

}  /* extern "C" */

/* Run one of the element-wise check kernels on n host values of `esz` bytes each. */
template <class F>
static int eval_elementwise(qmsg_ctx *c, const char *what, const void *x, int n, void *out, size_t esz, F launch)
{
    if (!c || n < 0 || (n && (!x || !out))) return QMSG_E_INVALID;
    if (n == 0) return QMSG_OK;
    HIP_TRY(c, hipSetDevice(c->device));
    std::vector<void *> tmp;
    uint8_t *d = nullptr;
    int rc = dev_alloc(c, (void **)&d, (size_t)n * esz * 2, tmp);
    if (rc) return rc;
    hipError_t e = hipMemcpy(d, x, (size_t)n * esz, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = launch(d, d + (size_t)n * esz);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e == hipSuccess) e = hipMemcpy(out, d + (size_t)n * esz, (size_t)n * esz, hipMemcpyDeviceToHost);
    hipFree(d);
    if (e != hipSuccess) return fail(c, QMSG_E_DEVICE, "%s: %s", what, hipGetErrorString(e));
    return QMSG_OK;
}

extern "C" {

int qmsg_eval_silu(qmsg_ctx *c, const float *x, int n, float *out)
{
    return eval_elementwise(c, "qmsg_eval_silu", x, n, out, 4, [&](uint8_t *in, uint8_t *o) {
        return launch_silu((const float *)in, n, (float *)o, c->stream);
    });
}

int qmsg_eval_exp(qmsg_ctx *c, const double *x, int n, double *out)
{
    return eval_elementwise(c, "qmsg_eval_exp", x, n, out, 8, [&](uint8_t *in, uint8_t *o) {
        return launch_exp((const double *)in, n, (double *)o, c->stream);
    });
}

int qmsg_calibrate_copy(qmsg_ctx *c, void *d_dst, const void *d_src, size_t bytes)
{
    if (!c || !d_dst || !d_src || bytes % 16) return QMSG_E_INVALID;
    HIP_TRY(c, hipSetDevice(c->device));
    LAUNCH(c, "copy", launch_copy(d_dst, d_src, bytes, c->stream));
    return QMSG_OK;
}

int qmsg_device_info(qmsg_ctx *c, int *n_cu, int *clock_khz, uint64_t *hbm_bytes, char *arch, int arch_len)
{
    if (!c) return QMSG_E_INVALID;
    hipDeviceProp_t p;
    HIP_TRY(c, hipGetDeviceProperties(&p, c->device));
    if (n_cu) *n_cu = p.multiProcessorCount;
    if (clock_khz) *clock_khz = p.clockRate;
    if (hbm_bytes) *hbm_bytes = (uint64_t)p.totalGlobalMem;
    if (arch && arch_len > 0) {
        strncpy(arch, p.gcnArchName, (size_t)arch_len - 1);
        arch[arch_len - 1] = 0;
    }
    return QMSG_OK;
}

}  // extern "C"
