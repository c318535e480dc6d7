/* qmsg_internal.h - shapes and device pointers shared by the host API and the kernels. */
#ifndef QMSG_INTERNAL_H
#define QMSG_INTERNAL_H

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qmsg {

/* QmsQ8 (src/kernels.h:7-12): the reference's 44-byte int8 activation block. */
struct Q8 {
    float d;
    float ds;
    int16_t s16[2];
    int8_t q[32];
};
static_assert(sizeof(Q8) == 44, "QmsQ8 is 44 bytes");

/* Kernel-side copy of the same blocks, grouped by pairs of 32-blocks (b even, b+1) so one
 * 16-byte LDS read gives a lane both of its code dwords for two blocks. 96 bytes per pair:
 *   [16p .. 16p+15]  for lane p = 0..3: q[4p..4p+3] of b, q[16+4p..] of b,
 *                                        q[4p..4p+3] of b+1, q[16+4p..] of b+1
 *   [64 .. 79]       d(b), ds(b), d(b+1), ds(b+1)
 *   [80 .. 87]       s16 pair of b, s16 pair of b+1 (low half = s16[0])
 *   [88 .. 95]       zero */
constexpr int kPairBytes = 96;

/* Optional per-dispatch timing. While a hook is installed on the calling thread, every kernel
 * launch of the library asks it for an event pair and launches through hipExtLaunchKernel,
 * which stamps the dispatch's own start and end into the events (no marker packets between
 * kernels). `kernel` is the launch's short name: route, select, dispatch, gateup, down,
 * combine, copy. */
struct LaunchTimer {
    void *ctx;
    void (*events)(void *ctx, const char *kernel, hipEvent_t *start, hipEvent_t *stop);
};
extern thread_local const LaunchTimer *g_launch_timer;

/* Static shape limits of the kernels. */
constexpr int kMaxExperts = 256;

/* Slots (tokens of one expert) per slot tile of the batch kernels (dispatch's tile list). */
constexpr int kTileN = 32;
/* Bytes of one activation record of the MFMA kernels (one int8 block as f16 codes, its scales
 * and the MFMA accumulator inputs). */
constexpr int kMxRec = 128;

/* The default path takes the MFMA kernels for gate/up once a batch averages kMxAutoQuarters / 4
 * slots per active expert, and for down from kMxDownMinSlotsQ4 slots (Q4_0 / Q4_1 rows) or
 * kMxDownMinSlotsQ6 (Q6_K rows). Measured per layer at the 235B shape, MFMA against the row
 * kernels (us; Q4 MFMA kernels on the 16x16x16 instructions): gate/up with the records each
 * needs 132.2 / 130.1 at 16 tokens, 114.2 / 107.1 at 12, and from 20 tokens (1.25 slots per
 * expert) 149.6 / 154.8; Q4_0 down after row-kernel gate/up, with the activation records it
 * needs: 41.3 / 41.5 at 6 tokens, 49.6 / 51.6 at 8, 55.8 / 62.1 at 12; Q6_K 41.6 / 32.9 at 2,
 * 49.4 / 46.2 at 3, 58.2 / 58.2 at 4, 105 / 118 at 8. */
constexpr int kMxAutoQuarters = 5;
/* Q6_K gate/up (its MFMA kernel unpacks 6-bit codes): from 2.5 slots per expert (streaming /
 * MFMA us: 442 / 487 at 32 tokens, 618 / 435 at 48) */
constexpr int kMxAutoQuartersQ6 = 10;
constexpr int kMxDownMinSlotsQ4 = 64;
constexpr int kMxDownMinSlotsQ6 = 32;
inline bool mx_auto(int T, int K, int X, int gate_type)
{
    const long NS = (long)T * K, act = X < NS ? X : NS;
    return 4 * NS >= (long)(gate_type == 14 ? kMxAutoQuartersQ6 : kMxAutoQuarters) * act;
}
inline bool mx_auto_down(int T, int K, int down_type)
{
    return (long)T * K >= (down_type == 14 ? kMxDownMinSlotsQ6 : kMxDownMinSlotsQ4);
}

/* One-token batches (n_used <= 8) are routed inside the gate/up kernel instead of by a
 * separate select launch. */
inline int use_small_route(int T, int K) { return T == 1 && K <= 8; }

/* Per-layer device weights: the GGUF bytes, unchanged, in one allocation per tensor. */
struct LayerDev {
    const float *router;    /* [X][E] */
    const uint8_t *gate;    /* [X][F] rows of gate_rb bytes */
    const uint8_t *up;      /* [X][F] rows of up_rb bytes   */
    const uint8_t *down;    /* [X][E] rows of down_rb bytes */
    int gate_type, up_type, down_type;
    uint64_t gate_rb, up_rb, down_rb;
    uint64_t gate_eb, up_eb, down_eb;
};

/* Device scratch of a context, sized for max_tokens. */
struct Scratch {
    float *logits;      /* [Tm][X]             */
    int32_t *sel;       /* [Tm*K]              */
    float *wt;          /* [Tm*K]              */
    int32_t *slot_t;    /* [Tm*K]              */
    int32_t *slot_of;   /* [Tm*K]              */
    int32_t *start;     /* [X+1]               */
    int32_t *active;    /* [X]                 */
    int4 *work;         /* [X] per active expert: {expert, first slot, end slot, 0}; expert -1 after */
    int4 *tiles;        /* [X + Tm*K/kTileN + 1] slot tiles of the MFMA kernels: {expert, first, end, 0} */
    int32_t *meta;      /* [0] n_active, [1] number of slot tiles */
    Q8 *xq;             /* [Tm][E/32]          */
    uint8_t *xqk;       /* [Tm][E/64][96]      */
    float *gu;          /* [Tm*K][2F]          */
    float *act;         /* [Tm*K][F]           */
    Q8 *aq;             /* [Tm*K][F/32]        */
    uint8_t *aqk;       /* [Tm*K][F/64][96]    */
    float *dn;          /* [Tm*K][E]           */
    uint8_t *mxx;       /* [Tm][E/32][kMxRec] MFMA records of the layer input */
    uint8_t *mxa;       /* [Tm*K][F/32][kMxRec] MFMA records of the activations */
    uint64_t *mxflag;   /* [2] the epoch of the last call whose input (0) / activation (1) records
                         * hold a d_x outside the MFMA kernels' scaled range */
    uint64_t epoch;     /* this call's epoch (unique per layer call in the process) */
};

struct Shape {
    int E, X, K, F;
};

/* Dense (trunk) matrices of one qms_matmul_n call: same type and cols, at most kDenseMats. */
constexpr int kDenseMats = 4;
struct DenseMat {
    const uint8_t *w;       /* rows of rb bytes (GGUF layout) */
    float *y;               /* [T][rows]                      */
    int rows;
    int first_block;        /* set by the launcher            */
};
struct DenseArgs {
    DenseMat m[kDenseMats];
    int nm;
    uint64_t rb;
    int C, T;
    const float *x;         /* [T][C] input rows (16-byte aligned) */
    const uint8_t *xqk;     /* [T][C/64] pair records, or NULL: the kernel quantises x */
};

/* Batches of at least this many rows are quantised once by a separate launch; smaller ones
 * inside every dense block. */
constexpr int kDenseQuantT = 8;

/* Launchers (qmsg_kernels.hip). Each returns hipSuccess or the launch error. */
hipError_t launch_route(const Shape &s, const LayerDev &L, const Scratch &S, const float *xn, int T,
                        hipStream_t st);
/* Top-K and dispatch; a one-token batch is left to the Q4_0 gate/up kernel when gateup_routes. */
hipError_t launch_select(const Shape &s, const Scratch &S, int T, int gateup_routes, hipStream_t st);
/* Whether gate and up take the streaming gate/up kernel (launch_gateup_exact): one type, Q4_0,
 * Q4_1, or Q6_K with rows a multiple of 4 bytes long. */
bool gateup_streams(const LayerDev &L);
/* quant_act: batches (not the one-token routing kernel) in blocks of 32 rows that also store
 * the activations' int8 blocks (aq, aqk) for the down kernel. */
hipError_t launch_gateup_exact(const Shape &s, const LayerDev &L, const Scratch &S, int T, int debug, int n_cu,
                               int quant_act, hipStream_t st);
/* The expert products on the matrix cores (order-exact): gate/up, then down and the combine.
 * mx_supported: whether the layer's types and shape fit the MFMA kernels (gate and up of one
 * type: Q4_0, Q4_1 or Q6_K;
 * *down_mx: whether down runs on them too, else on the exact down kernel). */
bool mx_supported(const Shape &s, const LayerDev &L, int *down_mx);
hipError_t launch_experts_mx(const Shape &s, const LayerDev &L, const Scratch &S, float *out, int T, int debug,
                             hipStream_t st);
/* Down alone on the MFMA kernels after a row-kernel gate/up: activation blocks and records from
 * act, the down tiles, the combine (needs *down_mx of mx_supported). */
hipError_t launch_down_mx(const Shape &s, const LayerDev &L, const Scratch &S, float *out, int T, hipStream_t st);
/* Gate/up rows of Q4_1 / Q6_K (or mixed) layers by slot tiles, then the SwiGLU. */
hipError_t launch_gateup_tiles(const Shape &s, const LayerDev &L, const Scratch &S, int T, hipStream_t st);
/* Whether two to four tokens take the small-batch down kernel. */
bool down_small_fits(const Shape &s, const LayerDev &L, int T);
/* Whether one of the exact down kernels (one-token, small-batch, slot tiles) holds this shape
 * in LDS; rows too long for all of them take the MFMA down kernel, which stages them in chunks. */
bool down_exact_fits(const Shape &s, const LayerDev &L, int T);
/* quant: the activations' int8 blocks are formed here (else read from aqk, where gate/up or the
 * MFMA gate/up stored them). */
hipError_t launch_down_exact(const Shape &s, const LayerDev &L, const Scratch &S, float *out, int T, int quant,
                             hipStream_t st);
/* The whole layer slot by slot, as the reference's moe_group_exact (src/model.c:1009-1030): with
 * exact its --exact mode (fp32 dequantised rows, fp32 activations), else each qms_matmul on its
 * int8 path, for shapes off the integer kernels' grid (integer_grid_shape). debug also stores
 * the int8 blocks of the inputs and activations (xq, aq) that the slot kernels keep in LDS. */
hipError_t launch_layer_slots(const Shape &s, const LayerDev &L, const Scratch &S, const float *xn, float *out, int T,
                              int exact, int debug, hipStream_t st, int down_only = 0);
/* The shapes the integer kernels take: n_embd % 256 == 0 (the reference's fast gate,
 * src/model.c:1090-1093) and n_ff_exp % 64 == 0 (they pair 32-blocks). */
inline bool integer_grid_shape(int E, int F) { return E % 256 == 0 && F % 64 == 0; }
/* down_only: the down rows, the debug copies and the combine alone, after the integer kernels'
 * routing and gate/up (with SwiGLU) have run: n_ff_exp an odd multiple of 32, whose down rows
 * the integer kernels do not pair. */
/* Expert types the integer kernels take (the quantised types of qms_fast_supported); layers
 * with F32, F16 or Q8_0 expert tensors run slot by slot. */
inline bool integer_expert_types(int gt, int ut, int dt)
{
    auto q = [](int t) { return t == 2 || t == 3 || t == 14; };
    return q(gt) && q(ut) && q(dt);
}
hipError_t launch_synth_f32(uint64_t key, uint64_t n, float sigma, float *out, hipStream_t st);
hipError_t launch_synth_experts(uint64_t seed, uint32_t layer, uint32_t kind, int type, int64_t rows,
                                int64_t cols, int X, float sigma, uint8_t *base, hipStream_t st);
hipError_t launch_rmsnorm_rows(float *x, int T, int E, float eps, hipStream_t st);
/* LDS bytes of the rmsnorm kernel for rows of E floats (at most 160 KiB is launchable). */
inline size_t rmsnorm_lds_bytes(int E)
{
    const size_t sq = E % 512 == 0 ? (size_t)(E / 64) * 65 : (size_t)E;      /* squares, in doubles */
    return sq * 8;
}
/* y = rmsnorm(x) * w per row of E floats; with add (not NULL) x += add first, stored back.
 * walk: form every row's sum in order (else only rows the bracket leaves open); rows that do
 * are counted into *walked when it is not NULL. */
hipError_t launch_rmsnorm(float *x, const float *add, const float *w, float *y, int T, int E, float eps,
                          int walk, unsigned long long *walked, hipStream_t st);
hipError_t launch_add_rows(float *h, const float *d, size_t n, hipStream_t st);
/* dst = h + d over n floats (dst may be h). */
hipError_t launch_add_rows_to(float *dst, const float *h, const float *d, size_t n, hipStream_t st);

/* The rmsnorm of the one-token router launch (launch_route_norm): xn = rmsnorm(h + add) * w
 * (add and w may be null), stored to xn_out; h + add stored to h_out when add is not null
 * (h_out must then differ from h). */
struct NormIn {
    const float *h, *add, *w;
    float *h_out, *xn_out;
    float eps;
    int walk;
    unsigned long long *walked;
};
/* Row widths the fused launch takes. */
inline bool route_norm_fits(int E) { return E % 512 == 0 && E <= 4096; }
/* launch_route for one token with the rmsnorm in front (route_norm_kernel). */
hipError_t launch_route_norm(const Shape &s, const LayerDev &L, const Scratch &S, const NormIn &n, hipStream_t st);
hipError_t launch_set_col0(float *m, int rows, int stride, const float *vals, float fill, hipStream_t st);
hipError_t launch_silu(const float *x, int n, float *out, hipStream_t st);
hipError_t launch_exp(const double *x, int n, double *out, hipStream_t st);
hipError_t launch_copy(void *dst, const void *src, size_t bytes, hipStream_t st);
/* p[0 .. n-1] = v (a kernel, not a memset node: safe inside a captured graph). */
hipError_t launch_call_reset(const Scratch &S, hipStream_t st);
/* The dense rows kernel; for T >= kDenseQuantT the input records are formed first into xqk
 * (T*C/64 records of 96 bytes). */
hipError_t launch_dense(const DenseArgs &a, int type, uint8_t *xqk, hipStream_t st);
/* matmul_exact for every matrix of a call (--exact, or an F16 / Q8_0 matrix in the call). */
hipError_t launch_dense_exact(const DenseArgs &args, int type, hipStream_t st);
hipError_t launch_block_dots(const uint8_t *base, int type, uint64_t rb, uint64_t eb, int n, const int32_t *expert,
                             const int32_t *row, const int32_t *block, const Q8 *xq, int32_t *out,
                             hipStream_t st);

}  // namespace qmsg

#endif /* QMSG_INTERNAL_H */
