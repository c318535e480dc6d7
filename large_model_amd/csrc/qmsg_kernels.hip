/* qmsg_kernels.hip - gfx950 kernels for the Qwen3-MoE expert-FFN layer.
 *
 * Layer = route (router dots + int8 input blocks; one-token batches also take their softmax and
 *         top-K inside the gate/up kernel, larger ones a select launch with the counting sort)
 *       -> gateup (gate/up row dots over Q4_0, SwiGLU)
 *       -> down   (int8 activation blocks, down row dots over Q4_0/Q4_1/Q6_K, weighted combine).
 * Prefill-sized batches run gate/up and down on the MFMA kernels instead (section "MFMA expert
 * products"), which fuse SwiGLU and the activation blocks into gate/up.
 *
 * Every fp32 operation reproduces the reference's AVX2 order (src/kernels.c, src/model.c):
 * each row's dot is eight 4-element int32 lanes per 32-block, a per-lane fp32 FMA chain
 * over blocks, an FMA chain for the offset term, the hsum256 tree and an unfused final
 * subtraction. Build with -ffp-contract=off: every fused multiply-add here is explicit.
 *
 * Work mapping of the row kernels (64-wide waves): one quad of lanes per weight row; lane p of
 * the quad owns the reference lanes k = p (low nibbles) and k = p + 4 (high nibbles), which
 * read the same code dword. Weight tiles stream from HBM with 16-byte coalesced loads into LDS;
 * the int8 activations sit in LDS in a pair-of-blocks layout so a lane gets its two code
 * partners with one 16-byte read. */
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>

#include <type_traits>

#include "qmsg_internal.h"
#include "qmsg_libm.h"
#include "qmsg_synth.h"

namespace qmsg {
thread_local const LaunchTimer *g_launch_timer = nullptr;
}

/* Phase stamps for development builds (-DQMSG_PHASE_TRACE): thread 0 of a block records the
 * 100 MHz real-time counter at numbered points of a kernel into a device table of 8 stamps
 * per block (route blocks from row 0, gate/up from 1024, down from 2048), read back with
 * qmsg_phase_read. Compiled out otherwise. */
#ifdef QMSG_PHASE_TRACE
namespace qmsg {
__device__ unsigned long long g_phase[4096 * 8];
}
#define PHASE(region, k)                                                                        \
    do {                                                                                        \
        if (threadIdx.x == 0) {                                                                 \
            const unsigned b_ = (region) + blockIdx.y * gridDim.x + blockIdx.x;                 \
            if (b_ < 4096) qmsg::g_phase[b_ * 8 + (k)] = __builtin_amdgcn_s_memrealtime();      \
        }                                                                                       \
    } while (0)
extern "C" int qmsg_phase_read(void *dst, size_t bytes)
{
    return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(qmsg::g_phase), bytes);
}
#else
#define PHASE(region, k) ((void)0)
#endif

/* Launch `kern` on `st`; with a timing hook installed the dispatch stamps its own events. */
#define QLAUNCH(name, kern, grid, block, lds, st, ...)                                          \
    do {                                                                                       \
        hipEvent_t qa_ = nullptr, qb_ = nullptr;                                               \
        if (qmsg::g_launch_timer)                                                              \
            qmsg::g_launch_timer->events(qmsg::g_launch_timer->ctx, (name), &qa_, &qb_);       \
        if (qa_)                                                                               \
            hipExtLaunchKernelGGL(kern, (grid), (block), (lds), (st), qa_, qb_, 0u, __VA_ARGS__); \
        else                                                                                   \
            hipLaunchKernelGGL(kern, (grid), (block), (lds), (st), __VA_ARGS__);              \
    } while (0)

namespace qmsg {

/* ------------------------------------------------------------------ scalar helpers ---- */

__device__ __forceinline__ float h2f(uint32_t bits16)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

__device__ __forceinline__ int sdot4(int a, int b) { return __builtin_amdgcn_sdot4(a, b, 0, false); }

/* fp16 (low or high half of h) times an fp32, rounded once: the product of the exact fp32
 * value of the half and f (the added zero cannot change a non-zero product). */
template <int HI>
__device__ __forceinline__ float mul_f16_f32(uint32_t h, float f)
{
    float r;
    if (HI) asm volatile("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(f));
    else asm volatile("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(f));
    return r;
}

/* src/model.c:424 */
__device__ __forceinline__ float silu_ref(float a) { return a / (1.0f + qmsg_expf(-a)); }

/* An unaligned 32-bit read from LDS at an even byte address (two aligned reads). */
__device__ __forceinline__ uint32_t lds_u32(const uint8_t *base, uint32_t a)
{
    const uint32_t *w = (const uint32_t *)(base + (a & ~3u));
    return __builtin_amdgcn_alignbyte(w[1], w[0], a & 3u);
}

__device__ __forceinline__ uint32_t pack4(const int8_t *q)
{
    return (uint32_t)(uint8_t)q[0] | ((uint32_t)(uint8_t)q[1] << 8) | ((uint32_t)(uint8_t)q[2] << 16) |
           ((uint32_t)(uint8_t)q[3] << 24);
}

/* Quantise 32 floats the way qms_quantize_q8 does (src/kernels.c:34-53) and store the block
 * in both layouts: the reference's 44-byte Q8 and half of a 96-byte pair record. */
/* One 32-block of the int8 quantiser (src/kernels.c:34-53): d = amax/127, q = rint(x/d) with
 * the reference's reciprocal, per-half code sums and ds = d*sum. */
struct Q8Vals {
    float d, ds;
    uint32_t s16;
    uint32_t qw[8];          /* q[4w .. 4w+3] packed little-endian */
};

__device__ Q8Vals quantize_block(const float *v)
{
    /* the maximum and the integer sums as trees: both are exact in any order, and a tree has a
     * dependency depth of 5 instead of 32 (the quantiser often runs one wave per SIMD, where
     * every dependent step costs its full latency). fmaxf ignores NaN like the reference's
     * running fmaxf from 0; the final fmaxf with 0 covers an all-NaN block. */
    float m[16];
#pragma unroll
    for (int j = 0; j < 16; j++) m[j] = fmaxf(fabsf(v[j]), fabsf(v[j + 16]));
#pragma unroll
    for (int w = 8; w > 0; w >>= 1)
#pragma unroll
        for (int j = 0; j < w; j++) m[j] = fmaxf(m[j], m[j + w]);
    const float amax = fmaxf(0.0f, m[0]);
    Q8Vals r;
    r.d = amax / 127.0f;
    const float id = r.d > 0.0f ? 1.0f / r.d : 0.0f;
    int8_t q[32];
    int qs[32];
#pragma unroll
    for (int j = 0; j < 32; j++) {
        /* the reference's (int)nearbyintf compiles to x86's conversion, which gives INT_MIN
         * for a NaN or a value outside int's range (id = +inf when d is below 2^-128, or an
         * infinite input); v_cvt_i32_f32 would clamp, so that case is chosen here */
        const float r = rintf(v[j] * id);
        qs[j] = fabsf(r) < 0x1p31f ? (int)r : (int)0x80000000u;
        q[j] = (int8_t)qs[j];
    }
#pragma unroll
    for (int w = 8; w > 0; w >>= 1)
#pragma unroll
        for (int j = 0; j < w; j++) {
            qs[j] = (int)((uint32_t)qs[j] + (uint32_t)qs[j + w]);      /* wrapping, as the reference's */
            qs[16 + j] = (int)((uint32_t)qs[16 + j] + (uint32_t)qs[16 + j + w]);
        }
    const int s0 = qs[0], s1 = qs[16];
    r.ds = r.d * (float)(int)((uint32_t)s0 + (uint32_t)s1);
    r.s16 = (uint32_t)(uint16_t)(int16_t)s0 | ((uint32_t)(uint16_t)(int16_t)s1 << 16);
    for (int w = 0; w < 8; w++) r.qw[w] = pack4(q + 4 * w);
    return r;
}

/* The 44-byte QmsQ8 record. */
__device__ void store_q8(const Q8Vals &q, Q8 *dst)
{
    uint32_t *o = (uint32_t *)dst;
    o[0] = __float_as_uint(q.d);
    o[1] = __float_as_uint(q.ds);
    o[2] = q.s16;
    for (int w = 0; w < 8; w++) o[3 + w] = q.qw[w];
}

/* Block `half` (0: even, 1: odd) of a 96-byte pair record. */
__device__ void store_pair_half(const Q8Vals &q, uint32_t *pair, int half)
{
    for (int p = 0; p < 4; p++) {
        pair[4 * p + 2 * half] = q.qw[p];
        pair[4 * p + 2 * half + 1] = q.qw[4 + p];
    }
    pair[16 + 2 * half] = __float_as_uint(q.d);
    pair[17 + 2 * half] = __float_as_uint(q.ds);
    pair[20 + half] = q.s16;
    if (half == 0) { pair[22] = 0; pair[23] = 0; }
}

__device__ void quantize_block_store(const float *v, Q8 *dst, uint32_t *pair, int half)
{
    const Q8Vals q = quantize_block(v);
    store_q8(q, dst);
    store_pair_half(q, pair, half);
}

/* ------------------------------------------------------------------ wave primitives ---- */

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

/* LDS ordering between the lanes of one wave (its LDS operations complete in order). */
__device__ __forceinline__ void wave_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

/* DPP lane moves (GFX9 encodings): row_shr:n = 0x110+n, row_bcast:15 = 0x142, row_bcast:31 = 0x143.
 * Lanes without a valid source, or in rows outside ROWM, return `old`. */
template <int CTRL, int ROWM = 0xf>
__device__ __forceinline__ uint32_t dpp32(uint32_t old, uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROWM, 0xf, false);
}

/* Inclusive prefix sum over the 64 lanes. */
__device__ __forceinline__ int wave_scan_add(int v)
{
    v += (int)dpp32<0x111>(0u, (uint32_t)v);
    v += (int)dpp32<0x112>(0u, (uint32_t)v);
    v += (int)dpp32<0x114>(0u, (uint32_t)v);
    v += (int)dpp32<0x118>(0u, (uint32_t)v);
    v += (int)dpp32<0x142, 0xa>(0u, (uint32_t)v);
    v += (int)dpp32<0x143, 0xc>(0u, (uint32_t)v);
    return v;
}

/* A 64-bit value of lane l (l wave-uniform), as a wave-uniform value. */
__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int l)
{
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), l);
    return ((uint64_t)hi << 32) | lo;
}

/* ------------------------------------------------------------------ route ---- */

struct RouteArgs {
    const float *router, *xn;
    int E, X, K, T;
    int n_route_wg;    /* blocks doing router dots; the blocks after them quantise the input */
    float *y;          /* logits: y[t * ystride + e] (the router: S.logits, stride X)        */
    int ystride;
    Scratch S;
};

/* Blocks past the router blocks: one input 32-block per thread (src/kernels.c:34-53). */
__device__ void route_quantize(const RouteArgs &a)
{
    const int nbE = a.E >> 5;
    const int b = ((int)blockIdx.x - a.n_route_wg) * (int)blockDim.x + (int)threadIdx.x;
    if (b >= a.T * nbE) return;
    const int t = b / nbE, blk = b - t * nbE;
    float v[32];
    const float4 *src = (const float4 *)(a.xn + (size_t)t * a.E + (size_t)blk * 32);
    for (int j = 0; j < 8; j++) {
        const float4 f = src[j];
        v[4 * j] = f.x; v[4 * j + 1] = f.y; v[4 * j + 2] = f.z; v[4 * j + 3] = f.w;
    }
    uint32_t *pair = (uint32_t *)(a.S.xqk + ((size_t)t * (nbE >> 1) + (blk >> 1)) * kPairBytes);
    quantize_block_store(v, a.S.xq + (size_t)t * nbE + blk, pair, blk & 1);
}

/* hsum of dot_f32 (src/kernels.c:211, 66-72) over the 16 chain lanes of a 16-lane group:
 * v_j = a0_j + a1_j (chains j and j+8), s_j = v_j + v_{j+4}, (s0+s2)+(s1+s3). Lane 0 holds it. */
__device__ __forceinline__ float chain16_sum(float acc)
{
    acc += __shfl_down(acc, 8, 16);
    acc += __shfl_down(acc, 4, 16);
    acc += __shfl_down(acc, 2, 16);
    acc += __shfl_down(acc, 1, 16);
    return acc;
}

/* Steps q0 .. q1-1 (16-byte groups of four) of one FMA chain over chain-major rows in LDS,
 * B groups per batch: the batch's reads are all issued before its FMAs. */
template <int B>
__device__ __forceinline__ float chain_steps(const float4 *wr, const float4 *xr, int q0, int q1, float acc)
{
    for (int q = q0; q < q1; q += B) {
        float4 w[B], x[B];
#pragma unroll
        for (int u = 0; u < B; u++) {
            w[u] = wr[q + u];
            x[u] = xr[q + u];
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < B; u++) {
            acc = __builtin_fmaf(w[u].x, x[u].x, acc);
            acc = __builtin_fmaf(w[u].y, x[u].y, acc);
            acc = __builtin_fmaf(w[u].z, x[u].z, acc);
            acc = __builtin_fmaf(w[u].w, x[u].w, acc);
        }
    }
    return acc;
}

/* Router for T <= 4: one block per expert, 256 threads. The expert's router row and the T
 * input rows are requested all at once, staged into LDS chain-major (chain c of a row holds
 * elements c, c+16, ... contiguously, so one 16-byte read gives a lane four steps of its
 * chain), and lane (t, c) of wave 0 then runs the reference's FMA chain c of token t
 * (src/kernels.c:202-213) with its reads batched ahead of the FMAs: 256 dependent FMAs per
 * chain for n_embd 4096. Chains advanced chunk by chunk as the data landed were slower (a
 * block barrier per chunk). */
template <int T>
__global__ __launch_bounds__(256) void route_small_kernel(RouteArgs a)
{
    extern __shared__ __align__(16) uint8_t smem[];
    if ((int)blockIdx.x >= a.n_route_wg) { route_quantize(a); return; }
    PHASE(0, 0);
    constexpr int NCH = 4, MPC = 1 + T;          /* chunks; loads per thread per chunk (E <= 4096) */
    const int tid = threadIdx.x, E = a.E, e = blockIdx.x;
    const int CS = E / 16 + 4;                   /* floats per chain: E/16 steps, padded (16-byte rows) */
    float *buf = (float *)smem;                  /* [1 + T rows][16 chains][CS]: row 0 router, 1.. inputs */
    const int cw = E / (4 * NCH);                /* 16-byte slots of one row per chunk */
    const int sc = cw * (1 + T);                 /* slots of one chunk */
    const u32x4 *wsrc = (const u32x4 *)(a.router + (size_t)e * E);
    const u32x4 *xsrc = (const u32x4 *)a.xn;
    u32x4 v[NCH][MPC];
#pragma unroll
    for (int c = 0; c < NCH; c++)
#pragma unroll
        for (int m = 0; m < MPC; m++) {
            const int i = min(tid + 256 * m, sc - 1), r = i / cw, j = c * cw + (i - r * cw);
            v[c][m] = r == 0 ? wsrc[j] : xsrc[(size_t)(r - 1) * (E / 4) + j];
        }
    const int t = tid >> 4, cc = tid & 15;
    const float4 *wr = (const float4 *)(buf + cc * CS);
    const float4 *xr = (const float4 *)(buf + ((1 + t) * 16 + cc) * CS);
    const int q4 = E / (16 * NCH * 4);           /* float4 steps of one chain per chunk */
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; c++) {
#pragma unroll
        for (int m = 0; m < MPC; m++) {
            const int i = tid + 256 * m;
            if (i < sc) {
                /* slot j holds elements 4j .. 4j+3: chains 4(j%4) .. 4(j%4)+3, step j/4 */
                const int r = i / cw, j = c * cw + (i - r * cw);
                float *dst = buf + (r * 16 + 4 * (j & 3)) * CS + (j >> 2);
                dst[0] = __uint_as_float(v[c][m].x);
                dst[CS] = __uint_as_float(v[c][m].y);
                dst[2 * CS] = __uint_as_float(v[c][m].z);
                dst[3 * CS] = __uint_as_float(v[c][m].w);
            }
        }
    }
    __syncthreads();
    PHASE(0, 1);
    if (tid < 16 * T) {
        const int q1 = NCH * q4;
        if ((q1 & 7) == 0) acc = chain_steps<8>(wr, xr, 0, q1, acc);
        else if ((q1 & 3) == 0) acc = chain_steps<4>(wr, xr, 0, q1, acc);
        else acc = chain_steps<1>(wr, xr, 0, q1, acc);
    }
    PHASE(0, 2);
    if (tid < 16 * T) {
        acc = chain16_sum(acc);
        if (cc == 0) a.y[(size_t)t * a.ystride + e] = acc;
    }
}

/* Router for T > 4: one block per 4KT tokens x 4J experts, 256 threads. Thread (c, ea, tb)
 * runs chain c of J experts x KT tokens over 256-element chunks staged in LDS chain-major (as
 * route_small_kernel does: chain c of a row holds its 16 elements c, c+16, ... of the chunk
 * contiguously, padded to CSC floats, so one 16-byte read gives a lane four steps of its
 * chain), so each chain still walks its elements c, c+16, ... in order. The next P chunks are
 * in flight in registers while one is consumed. Small blocks (J = KT = 1: 4 experts x 4
 * tokens) spread batches of up to 64 tokens over many CUs; larger batches take J = KT = 4
 * (16 x 16), which reads each router and input row fewer times. TAIL takes rows of any
 * multiple of 32 floats: a last partial chunk of E % 256 elements gives every chain
 * (E % 256) / 16 more steps, in order (dot_f32 has no scalar tail at these widths). */
constexpr int kRouteBigCSC = 20;                  /* floats per chain and chunk in LDS (16 + pad) */
/* LDS bytes of route_big_kernel<J, J, P>: 4J expert rows and 4J token rows of 16 chains. */
constexpr size_t route_big_lds(int J) { return (size_t)(8 * J) * 16 * kRouteBigCSC * 4; }
template <int J, int KT, int P, bool TAIL = false>
__global__ __launch_bounds__(256) void route_big_kernel(RouteArgs a)
{
    extern __shared__ __align__(16) uint8_t smem[];
    if ((int)blockIdx.x >= a.n_route_wg) { route_quantize(a); return; }
    constexpr int CH = 256, CSC = kRouteBigCSC, RSC = 16 * CSC;   /* chunk elements, chain and row strides */
    constexpr int EB = 4 * J;                     /* experts per block              */
    const int tid = threadIdx.x, E = a.E, T = a.T, X = a.X;
    constexpr int TB = 4 * KT;                    /* tokens per block               */
    const int egs = (X + EB - 1) / EB, tg = (int)blockIdx.x / egs, eg = (int)blockIdx.x - tg * egs;
    const int t0 = tg * TB, e0 = eg * EB;
    const int c = tid & 15, ea = (tid >> 4) & 3, tb = tid >> 6;
    float *W = (float *)smem, *Xt = W + EB * RSC;
    float acc[J][KT];
    for (int j = 0; j < J; j++) for (int k = 0; k < KT; k++) acc[j][k] = 0.0f;
    u32x4 pw[P][J], px[P][KT];
    /* TAIL: rows of any multiple of 32 floats; the last chunk holds E % 256 of them (pieces
     * past the row are not loaded, and the chains take only its steps) */
    const int nch = TAIL ? (E + CH - 1) / CH : E / CH;
    auto load = [&](int ch, u32x4 *w, u32x4 *x) {
#pragma unroll
        for (int m = 0; m < J; m++) {
            const int q = tid + 256 * m, col = ch * CH + (q & 63) * 4;
            if (TAIL && col >= E) w[m] = u32x4{ 0u, 0u, 0u, 0u };
            else w[m] = *(const u32x4 *)(a.router + (size_t)min(e0 + (q >> 6), X - 1) * E + col);
        }
#pragma unroll
        for (int m = 0; m < KT; m++) {
            const int q = tid + 256 * m, col = ch * CH + (q & 63) * 4;
            if (TAIL && col >= E) x[m] = u32x4{ 0u, 0u, 0u, 0u };
            else x[m] = *(const u32x4 *)(a.xn + (size_t)min(t0 + (q >> 6), T - 1) * E + col);
        }
    };
    /* the 16-byte slot q4 of a row's chunk holds elements 4 q4 .. 4 q4 + 3: step q4 / 4 of chains
     * 4 (q4 % 4) .. 4 (q4 % 4) + 3 */
    auto stage = [&](float *rowbase, int q4, const u32x4 &v) {
        float *dst = rowbase + (4 * (q4 & 3)) * CSC + (q4 >> 2);
        dst[0] = __uint_as_float(v.x);
        dst[CSC] = __uint_as_float(v.y);
        dst[2 * CSC] = __uint_as_float(v.z);
        dst[3 * CSC] = __uint_as_float(v.w);
    };
#pragma unroll
    for (int d = 0; d < P; d++)
        if (d < nch) load(d, pw[d], px[d]);
    for (int ch0 = 0; ch0 < nch; ch0 += P) {
#pragma unroll
        for (int d = 0; d < P; d++) {
            const int ch = ch0 + d;
            if (ch < nch) {
                __syncthreads();
#pragma unroll
                for (int m = 0; m < J; m++) {
                    const int q = tid + 256 * m;
                    stage(W + (q >> 6) * RSC, q & 63, pw[d][m]);
                }
#pragma unroll
                for (int m = 0; m < KT; m++) {
                    const int q = tid + 256 * m;
                    stage(Xt + (q >> 6) * RSC, q & 63, px[d][m]);
                }
                __syncthreads();
                if (ch + P < nch) load(ch + P, pw[d], px[d]);
                /* steps of each chain in this chunk: 16, or (E % 256) / 16 (even) in a last
                 * partial one */
                const int steps = TAIL ? min(16, (E - ch * CH) / 16) : 16;
#pragma unroll
                for (int s0 = 0; s0 < 16; s0 += 4) {
                    if (TAIL && s0 >= steps) break;
                    float4 wv[J], xv[KT];
                    for (int j = 0; j < J; j++) wv[j] = *(const float4 *)(W + (J * ea + j) * RSC + c * CSC + s0);
                    for (int k = 0; k < KT; k++) xv[k] = *(const float4 *)(Xt + (KT * tb + k) * RSC + c * CSC + s0);
                    const bool four = !TAIL || s0 + 4 <= steps;
                    for (int j = 0; j < J; j++)
                        for (int k = 0; k < KT; k++) {
                            acc[j][k] = __builtin_fmaf(wv[j].x, xv[k].x, acc[j][k]);
                            acc[j][k] = __builtin_fmaf(wv[j].y, xv[k].y, acc[j][k]);
                            if (four) {
                                acc[j][k] = __builtin_fmaf(wv[j].z, xv[k].z, acc[j][k]);
                                acc[j][k] = __builtin_fmaf(wv[j].w, xv[k].w, acc[j][k]);
                            }
                        }
                }
            }
        }
    }
    for (int j = 0; j < J; j++)
        for (int k = 0; k < KT; k++) {
            const float v = chain16_sum(acc[j][k]);
            const int t = t0 + KT * tb + k, e = e0 + J * ea + j;
            if (c == 0 && t < T && e < X) a.y[(size_t)t * a.ystride + e] = v;
        }
}

/* Chunks in flight per thread of the T > 4 router. */
constexpr int kRouteBigP = 4;

hipError_t launch_route(const Shape &s, const LayerDev &L, const Scratch &S, const float *xn, int T, hipStream_t st)
{
    RouteArgs a;
    a.router = L.router;
    a.xn = xn;
    a.E = s.E;
    a.X = s.X;
    a.K = s.K;
    a.T = T;
    a.y = S.logits;
    a.ystride = s.X;
    a.S = S;
    const int nq = (T * (s.E / 32) + 255) / 256;
    if (T <= 4 && s.E <= 4096) {
        a.n_route_wg = s.X;
        const size_t lds = (size_t)(1 + T) * 16 * (s.E / 16 + 4) * 4;
        const dim3 grid(a.n_route_wg + nq);
        if (T == 1) QLAUNCH("route", route_small_kernel<1>, grid, dim3(256), lds, st, a);
        else if (T == 2) QLAUNCH("route", route_small_kernel<2>, grid, dim3(256), lds, st, a);
        else if (T == 3) QLAUNCH("route", route_small_kernel<3>, grid, dim3(256), lds, st, a);
        else QLAUNCH("route", route_small_kernel<4>, grid, dim3(256), lds, st, a);
    } else {
        const int J = T <= 64 ? 1 : 4;               /* experts and tokens per thread group */
        a.n_route_wg = ((T + 4 * J - 1) / (4 * J)) * ((s.X + 4 * J - 1) / (4 * J));
        const size_t lds = route_big_lds(J);
        if (J == 1) QLAUNCH("route", (route_big_kernel<1, 1, kRouteBigP>), dim3(a.n_route_wg + nq), dim3(256), lds, st, a);
        else QLAUNCH("route", (route_big_kernel<4, 4, kRouteBigP>), dim3(a.n_route_wg + nq), dim3(256), lds, st, a);
    }
    return hipGetLastError();
}

/* ------------------------------------------------------------------ select + dispatch ---- */

struct SelectArgs {
    int X, K, T;
    Scratch S;
};

__device__ void route_one_rank(const float *logits, int X, float *L, double *P, int *rank, int *selidx);
__device__ void topk_from_ranks(int K, int X, const float *L, const double *P, const int *rank, int *cand, int *sel);

/* Softmax over one token's logits in double, the top K by (probability descending, index
 * ascending) - the order K rounds of argmax with ties to the lower index produce - and the
 * weights renormalised over the selection (src/model.c:1045-1064). One block of 256 threads
 * per token, as the one-token routing does it: wave 0 runs the softmax while waves 1-3 rank
 * the float logits (p is non-decreasing in the logit), then wave 0 takes the first K of that
 * order after checking it for rounding ties (else it ranks the p exactly) and forms the
 * weights, wsum summed in selection order. LDS: P[X] doubles, part[] the float logits and
 * their ranks, selb[0 .. 63] the selection and selb[64 ..] K + 1 candidates. */
__device__ void topk_token(const SelectArgs &a, int t, int tid, double *P, int *part, int *selb)
{
    const int X = a.X, K = a.K;
    float *L = (float *)part;
    int *rank = part + kMaxExperts;
    route_one_rank(a.S.logits + (size_t)t * X, X, L, P, rank, nullptr);
    PHASE(0, 1);
    if (tid < 64) {
        topk_from_ranks(K, X, L, P, rank, selb + 64, selb);
        const int sj = tid < K ? selb[tid] : 0;
        const double pj = tid < K ? P[sj] : 0.0;
        double wsum = 0.0;
        for (int j = 0; j < K; j++) wsum += __shfl(pj, j);
        if (tid < K) {
            a.S.sel[(size_t)t * K + tid] = sj;
            a.S.wt[(size_t)t * K + tid] = (float)(pj / wsum);
        }
    }
    PHASE(0, 4);
    __syncthreads();
}

/* Counting sort of the T*K (token, selection) slots by expert, src/model.c:1066-1088:
 * slots of one expert are contiguous, experts ascend, and inside an expert slots follow
 * token order then selection order. Also writes one work record per active expert
 * (expert, first slot, end slot) for the expert kernels, and -1 records after them. One wave. */
__device__ void dispatch_slots(const SelectArgs &a, const int *sel, int *cnt, int *cur, int *tok)
{
    constexpr int NPL = kMaxExperts / 64;
    const int X = a.X, NS = a.T * a.K, lane = threadIdx.x & 63;
    for (int e = lane; e < X; e += 64) { cnt[e] = 0; cur[e] = 0; tok[e] = 0; }
    wave_sync();
    for (int i = lane; i < NS; i += 64) atomicAdd(&cnt[sel[i]], 1);
    wave_sync();
    /* lane l owns experts l*NPL .. l*NPL+NPL-1 (contiguous, so a lane scan orders them) */
    int c[NPL], tot = 0, act = 0;
#pragma unroll
    for (int i = 0; i < NPL; i++) {
        const int e = lane * NPL + i;
        c[i] = e < X ? cnt[e] : 0;
        tot += c[i];
        act += c[i] > 0;
    }
    const int incl = wave_scan_add(tot), incl_a = wave_scan_add(act);
    int st = incl - tot, pos = incl_a - act;
    const int na = __builtin_amdgcn_readlane(incl_a, 63);
    wave_sync();
#pragma unroll
    for (int i = 0; i < NPL; i++) {
        const int e = lane * NPL + i;
        if (e < X) {
            cnt[e] = st;                         /* cnt now holds start[e] */
            a.S.start[e] = st;
            if (c[i]) a.S.active[pos++] = e;
            st += c[i];
        }
    }
    if (lane == 63) a.S.start[X] = incl;
    for (int i = na + lane; i < X; i += 64) a.S.work[i] = make_int4(-1, 0, 0, 0);
    if (lane == 0) a.S.meta[0] = na;
    wave_sync();
    const unsigned long long below = (1ULL << lane) - 1ULL;
    for (int base = 0; base < NS; base += 64) {
        const int i = base + lane;
        const int e = i < NS ? sel[i] : -1;
        unsigned long long same = __ballot(i < NS);
        for (int bit = 0; bit < 9; bit++) {
            const unsigned long long b = __ballot(i < NS && ((e >> bit) & 1));
            same &= ((e >> bit) & 1) ? b : ~b;
        }
        int s = 0;
        if (i < NS) s = cnt[e] + cur[e] + __popcll(same & below);
        wave_sync();
        if (i < NS) {
            const int t = i / a.K, k = s - cnt[e];
            a.S.slot_t[s] = t;
            a.S.slot_of[i] = s;
            if (k < 4) atomicOr(&tok[e], (t & 0xff) << (8 * k));
            if ((same >> lane) == 1ULL) cur[e] += __popcll(same);   /* highest lane of the group */
        }
        wave_sync();
    }
    /* one work record per active expert: {expert, first slot, end slot, tokens of its first
     * four slots (one byte each)} */
    int wpos = incl_a - act;
#pragma unroll
    for (int i = 0; i < NPL; i++) {
        const int e = lane * NPL + i;
        if (e < X && c[i]) {
            a.S.work[wpos] = make_int4(e, cnt[e], cnt[e] + cur[e], tok[e]);
            wpos++;
        }
    }
    /* slot tiles of at most kTileN slots of one expert, experts ascending (MFMA kernels) */
    int nt = 0;
#pragma unroll
    for (int i = 0; i < NPL; i++) nt += (c[i] + kTileN - 1) / kTileN;
    const int incl_t = wave_scan_add(nt);
    int tpos = incl_t - nt;
#pragma unroll
    for (int i = 0; i < NPL; i++) {
        const int e = lane * NPL + i;
        if (e < X)
            for (int b = 0; b < c[i]; b += kTileN)
                a.S.tiles[tpos++] = make_int4(e, cnt[e] + b, cnt[e] + min(c[i], b + kTileN), 0);
    }
    if (lane == 63) a.S.meta[1] = incl_t;
}

/* Top-K of one token per block. The block that finishes last sorts the slots: each block
 * releases its selection (device-scope fence by the wave that wrote it) and takes a ticket
 * from meta[4]; the last ticket acquires the others' selections, dispatches and resets the
 * counter for the next launch. A one-block launch (T == 1) dispatches directly. */
__global__ __launch_bounds__(256) void select_kernel(SelectArgs a, int do_dispatch)
{
    __shared__ double P[kMaxExperts];
    __shared__ __align__(16) int part[2 * kMaxExperts];   /* float logits (16-byte reads), then ranks */
    __shared__ int selb[64 + 65];                /* the selection, then K + 1 candidates */
    __shared__ int tok[kMaxExperts];
    __shared__ int last;
    const int t = blockIdx.x;
    PHASE(0, 0);
    if (t < a.T) topk_token(a, t, threadIdx.x, P, part, selb);
    PHASE(0, 5);
    if (!do_dispatch) return;
    if (gridDim.x > 1) {
        if (threadIdx.x < 64) __threadfence();          /* sel/wt were written by wave 0 */
        __syncthreads();
        if (threadIdx.x == 0) last = atomicAdd(a.S.meta + 4, 1) == (int)gridDim.x - 1;
        __syncthreads();
        if (!last) return;
        __threadfence();
    }
    PHASE(0, 6);
    if (threadIdx.x < 64) dispatch_slots(a, a.S.sel, part, part + kMaxExperts, tok);
    if (gridDim.x > 1 && threadIdx.x == 0) __hip_atomic_store(a.S.meta + 4, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    PHASE(0, 7);
}

__global__ __launch_bounds__(64) void dispatch_kernel(SelectArgs a)
{
    __shared__ int cnt[kMaxExperts], cur[kMaxExperts], tok[kMaxExperts];
    dispatch_slots(a, a.S.sel, cnt, cur, tok);
}

/* Inclusive sum over the block's first kMaxExperts threads (4 waves); others return 0. */
__device__ __forceinline__ int experts_scan(int v, int *wsum)
{
    const int tid = threadIdx.x, lane = tid & 63;
    int incl = 0;
    if (tid < kMaxExperts) {
        incl = wave_scan_add(v);
        if (lane == 63) wsum[tid >> 6] = incl;
    }
    __syncthreads();
    if (tid < kMaxExperts)
        for (int j = 0; j < (tid >> 6); j++) incl += wsum[j];
    __syncthreads();
    return incl;
}

/* The same counting sort as dispatch_slots for large batches, on 16 waves: wave w owns a
 * contiguous run of the (token, selection) entries; the per-wave expert counts and their
 * prefix (experts ascending, then waves in entry order) give every slot its position, so the
 * order inside an expert is still token order then selection order (src/model.c:1066-1088). */
constexpr int kDispWaves = 16;
__global__ __launch_bounds__(64 * kDispWaves) void dispatch_wide_kernel(SelectArgs a)
{
    __shared__ int cw[kDispWaves][kMaxExperts];       /* per-wave counts, then next positions */
    __shared__ int start[kMaxExperts], tok[kMaxExperts], wsum[4], n_active;
    const int X = a.X, K = a.K, NS = a.T * K, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int per = (NS + kDispWaves - 1) / kDispWaves, lo = min(w * per, NS), hi = min(lo + per, NS);
    for (int i = tid; i < kDispWaves * kMaxExperts; i += 64 * kDispWaves) (&cw[0][0])[i] = 0;
    for (int e = tid; e < kMaxExperts; e += 64 * kDispWaves) tok[e] = 0;
    __syncthreads();
    const unsigned long long below = (1ULL << lane) - 1ULL;
    /* lanes of this 64-entry chunk with the same expert as this lane's entry */
    auto group = [&](int i, int e) {
        unsigned long long same = __ballot(i < hi);
        for (int bit = 0; bit < 9; bit++) {
            const unsigned long long b = __ballot(i < hi && ((e >> bit) & 1));
            same &= ((e >> bit) & 1) ? b : ~b;
        }
        return same;
    };
    for (int base = lo; base < hi; base += 64) {
        const int i = base + lane, e = i < hi ? a.S.sel[i] : -1;
        const unsigned long long same = group(i, e);
        if (i < hi && (same >> lane) == 1ULL) cw[w][e] += __popcll(same);   /* highest lane of the group */
        wave_sync();
    }
    __syncthreads();
    /* thread e: the expert's total, start, active index and tile count; per-wave first slots */
    int tot = 0;
    if (tid < kMaxExperts && tid < X)
        for (int v = 0; v < kDispWaves; v++) tot += cw[v][tid];
    const int incl = experts_scan(tot, wsum);
    const int act = tot > 0 ? 1 : 0, incl_a = experts_scan(act, wsum);
    const int nt = (tot + kTileN - 1) / kTileN, incl_t = experts_scan(nt, wsum);
    if (tid < X) {
        int run = incl - tot;
        start[tid] = run;
        a.S.start[tid] = run;
        if (act) a.S.active[incl_a - 1] = tid;
        for (int v = 0; v < kDispWaves; v++) {
            const int c = cw[v][tid];
            cw[v][tid] = run;
            run += c;
        }
        if (tid == X - 1) {
            a.S.start[X] = incl;
            a.S.meta[0] = incl_a;
            a.S.meta[1] = incl_t;
            n_active = incl_a;
        }
    }
    __syncthreads();
    for (int base = lo; base < hi; base += 64) {
        const int i = base + lane, e = i < hi ? a.S.sel[i] : -1;
        const unsigned long long same = group(i, e);
        int s = 0;
        if (i < hi) s = cw[w][e] + __popcll(same & below);
        wave_sync();
        if (i < hi) {
            const int t = i / K, k = s - start[e];
            a.S.slot_t[s] = t;
            a.S.slot_of[i] = s;
            if (k < 4) atomicOr(&tok[e], (t & 0xff) << (8 * k));
            if ((same >> lane) == 1ULL) cw[w][e] += __popcll(same);
        }
        wave_sync();
    }
    __syncthreads();
    /* work records per active expert {expert, first slot, end slot, tokens of its first four
     * slots}, -1 records after them; slot tiles of at most kTileN slots, experts ascending */
    const int na = n_active;
    if (tid < X) {
        if (act) a.S.work[incl_a - 1] = make_int4(tid, start[tid], start[tid] + tot, tok[tid]);
        if (tid >= na) a.S.work[tid] = make_int4(-1, 0, 0, 0);
        int tpos = incl_t - nt;
        for (int b = 0; b < tot; b += kTileN)
            a.S.tiles[tpos++] = make_int4(tid, start[tid] + b, start[tid] + min(tot, b + kTileN), 0);
    }
}

hipError_t launch_select(const Shape &s, const Scratch &S, int T, int gateup_routes, hipStream_t st)
{
    SelectArgs a;
    a.X = s.X;
    a.K = s.K;
    a.T = T;
    a.S = S;
    if (gateup_routes && use_small_route(T, s.K)) return hipSuccess;   /* the gate/up kernel routes the batch */
    /* up to 16 tokens the last select block also dispatches (one wave); larger batches take the
     * 16-wave dispatch launch (measured 5 us less per layer at 48 and 64 tokens) */
    QLAUNCH("select", select_kernel, dim3(T), dim3(256), 0, st, a, T <= 16 ? 1 : 0);
    if (T > 16) QLAUNCH("dispatch", dispatch_wide_kernel, dim3(1), dim3(64 * kDispWaves), 0, st, a);
    return hipGetLastError();
}

/* ------------------------------------------------------------------ expert row dots ---- */

/* Running state of one quad's row dot for one token: the two reference lanes this lane
 * owns and the offset chain (identical on the four lanes of the quad). */
struct RowAcc {
    float lo, hi, corr;
};

typedef float f32x4 __attribute__((ext_vector_type(4)));

/* The words one lane needs from a pair of Q4_0 blocks (36 bytes at W, 4-byte aligned): its
 * code dword of each block (bytes 4p..4p+3 of qs) and both scales. */
struct Q4Pair {
    uint32_t c0, c1;
    uint32_t w0, w4;      /* d of block b in the low half of w0, d of b+1 in the high half of w4 */
};

__device__ __forceinline__ Q4Pair q4_0_load(const uint32_t *W, int p)
{
    const uint32_t wa = W[p], wb = W[p + 1];
    Q4Pair r;
    r.w0 = W[0];
    r.w4 = W[4];
    r.c0 = __builtin_amdgcn_alignbyte(wb, wa, 2);
    r.c1 = W[5 + p];
    return r;
}

/* One token's part of a pair record for lane p: its q dwords of both blocks and d/ds. */
struct XPair {
    u32x4 q;
    f32x4 d;
};

__device__ __forceinline__ XPair x_load(const uint8_t *xp, int p)
{
    XPair r;
    r.q = *(const u32x4 *)(xp + 16 * p);
    r.d = *(const f32x4 *)(xp + 64);
    return r;
}

/* src/kernels.c:87-93 for blocks b and b+1, reference lanes k = p (low nibbles) and p + 4. */
__device__ __forceinline__ void q4_0_math(const Q4Pair &w, const XPair &x, RowAcc &r)
{
    const int s0 = sdot4((int)(w.c0 & 0x0f0f0f0fu), (int)x.q.x);
    const int s1 = sdot4((int)((w.c0 >> 4) & 0x0f0f0f0fu), (int)x.q.y);
    const int s2 = sdot4((int)(w.c1 & 0x0f0f0f0fu), (int)x.q.z);
    const int s3 = sdot4((int)((w.c1 >> 4) & 0x0f0f0f0fu), (int)x.q.w);
    const float d0 = h2f(w.w0 & 0xffffu), d1 = h2f(w.w4 >> 16);
    const float m0 = mul_f16_f32<0>(w.w0, x.d.x), m1 = mul_f16_f32<1>(w.w4, x.d.z);
    r.lo = __builtin_fmaf((float)s0, m0, r.lo);
    r.hi = __builtin_fmaf((float)s1, m0, r.hi);
    r.corr = __builtin_fmaf(d0, x.d.y, r.corr);
    r.lo = __builtin_fmaf((float)s2, m1, r.lo);
    r.hi = __builtin_fmaf((float)s3, m1, r.hi);
    r.corr = __builtin_fmaf(d1, x.d.w, r.corr);
}

/* The words one lane needs from a pair of Q4_1 blocks {f16 d; f16 m; u8 qs[16]} (40 bytes at
 * W, 4-byte aligned): its code dword of each block and the d|m word of each. */
struct Q41Pair {
    uint32_t c0, c1;
    uint32_t w0, w5;      /* d of block b in the low half of w0, m in its high half; w5 for b+1 */
};

__device__ __forceinline__ Q41Pair q4_1_load(const uint32_t *W, int p)
{
    Q41Pair r;
    r.w0 = W[0];
    r.c0 = W[1 + p];
    r.w5 = W[5];
    r.c1 = W[6 + p];
    return r;
}

/* src/kernels.c:113-119 for blocks b and b+1: unsigned codes (no -8), lane sums scaled by
 * fl(d*xd), and the offset chain off = fma(m, ds, off) kept in corr. */
__device__ __forceinline__ void q4_1_math(const Q41Pair &w, const XPair &x, RowAcc &r)
{
    const int s0 = sdot4((int)(w.c0 & 0x0f0f0f0fu), (int)x.q.x);
    const int s1 = sdot4((int)((w.c0 >> 4) & 0x0f0f0f0fu), (int)x.q.y);
    const int s2 = sdot4((int)(w.c1 & 0x0f0f0f0fu), (int)x.q.z);
    const int s3 = sdot4((int)((w.c1 >> 4) & 0x0f0f0f0fu), (int)x.q.w);
    const float o0 = h2f(w.w0 >> 16), o1 = h2f(w.w5 >> 16);
    const float m0 = mul_f16_f32<0>(w.w0, x.d.x), m1 = mul_f16_f32<0>(w.w5, x.d.z);
    r.lo = __builtin_fmaf((float)s0, m0, r.lo);
    r.hi = __builtin_fmaf((float)s1, m0, r.hi);
    r.corr = __builtin_fmaf(o0, x.d.y, r.corr);
    r.lo = __builtin_fmaf((float)s2, m1, r.lo);
    r.hi = __builtin_fmaf((float)s3, m1, r.hi);
    r.corr = __builtin_fmaf(o1, x.d.w, r.corr);
}

/* The weight side of one Q6_K 32-block for lane p (src/kernels.c:148-160): its two 6-bit code
 * dwords (elements 4p.. of the low 16 and of the high 16), the two sub-scales and d. Read once
 * and used for every token of a pass. */
struct Q6W {
    uint32_t q6lo, q6hi;
    int sa, sb;
    float d;
};

template <bool AL>
__device__ __forceinline__ uint32_t lds_word(const uint8_t *base, uint32_t a)
{
    if (AL) return *(const uint32_t *)(base + a);      /* a is a multiple of 4 */
    return lds_u32(base, a);
}

/* AL: the super-block starts at a multiple of 4 bytes, so its code dwords are single reads. */
template <bool AL>
__device__ __forceinline__ Q6W q6_k_weights(const uint8_t *tile, uint32_t sb, int h, int g, int p)
{
    const uint32_t qlo = lds_word<AL>(tile, sb + 64 * h + 32 * (g & 1) + 4 * p);
    const uint32_t qhi = lds_word<AL>(tile, sb + 64 * h + 32 * (g & 1) + 16 + 4 * p);
    const uint32_t hlo = lds_word<AL>(tile, sb + 128 + 32 * h + 4 * p);
    const uint32_t hhi = lds_word<AL>(tile, sb + 128 + 32 * h + 16 + 4 * p);
    const uint32_t scw = AL ? (lds_word<true>(tile, sb + 192 + 8 * h + 4 * (g >> 1)) >> (16 * (g & 1)))
                            : lds_u32(tile, sb + 192 + 8 * h + 2 * g);
    const int sh = 2 * g;
    const uint32_t nlo = g < 2 ? (qlo & 0x0f0f0f0fu) : ((qlo >> 4) & 0x0f0f0f0fu);
    const uint32_t nhi = g < 2 ? (qhi & 0x0f0f0f0fu) : ((qhi >> 4) & 0x0f0f0f0fu);
    Q6W w;
    w.q6lo = nlo | (((hlo >> sh) & 0x03030303u) << 4);
    w.q6hi = nhi | (((hhi >> sh) & 0x03030303u) << 4);
    w.sa = (int)(int8_t)(scw & 0xff);
    w.sb = (int)(int8_t)((scw >> 8) & 0xff);
    w.d = h2f(lds_word<AL>(tile, sb + 208) & 0xffffu);
    return w;
}

/* The token side of the same block against one token's pair record (lanes k < 4 use sc[2g],
 * k >= 4 sc[2g+1]; src/kernels.c:161-167), on weights already read. */
__device__ __forceinline__ void q6_k_token(const Q6W &w, const uint8_t *xp, int p, int xhalf, RowAcc &r)
{
    const uint32_t xlo = *(const uint32_t *)(xp + 16 * p + 8 * xhalf);
    const uint32_t xhi = *(const uint32_t *)(xp + 16 * p + 8 * xhalf + 4);
    const float xd = *(const float *)(xp + 64 + 8 * xhalf);
    const uint32_t s16 = *(const uint32_t *)(xp + 80 + 4 * xhalf);
    const int s16a = (int)(int16_t)(s16 & 0xffffu), s16b = (int)(int16_t)(s16 >> 16);
    const float dd = w.d * xd;
    r.lo = __builtin_fmaf((float)(sdot4((int)w.q6lo, (int)xlo) * w.sa), dd, r.lo);
    r.hi = __builtin_fmaf((float)(sdot4((int)w.q6hi, (int)xhi) * w.sb), dd, r.hi);
    r.corr = __builtin_fmaf(dd, (float)(w.sa * s16a + w.sb * s16b), r.corr);
}

/* hsum256 over the quad, then the unfused offset term h - scale*corr: scale 8 (Q4_0), 32
 * (Q6_K), or -1 for Q4_1's h + off (src/kernels.c:120; -1*off is exact, so h - (-off) is the
 * reference's sum). Valid on lane p == 0. */
__device__ __forceinline__ float quad_finish(const RowAcc &r, float scale)
{
    const float s = r.lo + r.hi;                      /* s_p = acc_p + acc_{p+4}   */
    const float t = s + __shfl_down(s, 2, 4);         /* (s0+s2) on p0, (s1+s3) on p1 */
    const float h = t + __shfl_down(t, 1, 4);
    return h - scale * r.corr;
}

/* ------------------------------------------------------------------ small-batch routing ---- */

/* A one-token batch is routed inside the expert kernel: every block recomputes the softmax,
 * top-K and slot order from the logits, which removes a launch and a round trip through
 * memory between the router and the experts. */
constexpr int kSelNS = 8;              /* slots of such a batch (n_used <= 8) */

struct alignas(16) SmallRoute {
    int4 work[kSelNS];                 /* per active expert, as Scratch::work */
    int sel[kSelNS];
    float wt[kSelNS];
    int slot_t[kSelNS];
    int slot_of[kSelNS];
    int cand[kSelNS + 1];              /* the first K+1 experts of the logit order */
    int na;
    int pad[2];
};

/* Routing of a one-token batch inside each gate/up block (src/model.c:1045-1088).
 *
 * The softmax runs on wave 0: P_e = exp(l_e - max) in double, z summed in expert order, p_e =
 * P_e / z. Meanwhile the other waves rank the float logits (descending, ties to the lower
 * index). Since p is non-decreasing in l, the reference's top K (p descending, ties to the
 * lower index) is the first K of that order whenever p strictly decreases along its first
 * K+1 entries, except between equal logits, whose p are equal and whose order is by index in
 * both rankings; this is checked, and if a rounding tie shows up (logits of different value
 * with equal p), wave 0 ranks the p exactly instead. Weights are renormalised with wsum in
 * selection order; the slots of the token are its experts in ascending order.
 * Shared scratch (LDS): L[X rounded up to 4] floats (16-byte aligned), P[X] doubles,
 * rank[X], selidx[X] (may be null), start[X+1]. This first half (softmax and logit ranks)
 * ends with a block barrier. */
__device__ void route_one_rank(const float *logits, int X, float *L, double *P, int *rank, int *selidx)
{
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    for (int e = tid; e < ((X + 3) & ~3); e += blockDim.x) {
        L[e] = e < X ? logits[e] : -__builtin_inff();
        if (e < X) {
            rank[e] = 0;
            if (selidx) selidx[e] = -1;
        }
    }
    __syncthreads();
    if (wave == 0) {
        constexpr int NPL = kMaxExperts / 64;
        double v[NPL];
        float mf = -__builtin_inff();
#pragma unroll
        for (int i = 0; i < NPL; i++) {
            const int e = lane + 64 * i;
            const float l = e < X ? L[e] : -__builtin_inff();
            mf = l > mf ? l : mf;
        }
        for (int o = 32; o > 0; o >>= 1) {
            const float w = __shfl_xor(mf, o);
            mf = w > mf ? w : mf;
        }
        const double mx = (double)mf;
#pragma unroll
        for (int i = 0; i < NPL; i++) {
            const int e = lane + 64 * i;
            v[i] = e < X ? qmsg_exp((double)L[e] - mx) : 0.0;
            if (e < X) P[e] = v[i];
        }
        wave_sync();
        double z = 0.0;
        const double2 *P2 = (const double2 *)P;
#pragma unroll 16
        for (int e2 = 0; e2 < (X >> 1); e2++) {
            const double2 q = P2[e2];
            z += q.x;
            z += q.y;
        }
        if (X & 1) z += P[X - 1];
        wave_sync();
#pragma unroll
        for (int i = 0; i < NPL; i++) {
            const int e = lane + 64 * i;
            if (e < X) P[e] = v[i] / z;
        }
    } else {
        /* float ranks, item (e, part) over waves 1 .. nw-1, four logits per LDS read (the
         * entries past X hold -inf and never count) */
        const int nth = blockDim.x - 64, t = tid - 64, X4 = (X + 3) & ~3;
        const int np = max(1, nth / X), len = ((X4 + np - 1) / np + 3) & ~3;
        for (int it = t; it < X * np; it += nth) {
            const int part = it % np, e = it / np;
            const float le = L[e];
            const int f0 = part * len, f1 = min(X4, f0 + len);
            int r = 0;
#pragma unroll 4
            for (int f = f0; f < f1; f += 4) {
                const float4 lf = *(const float4 *)(L + f);
                r += (lf.x > le) | ((lf.x == le) & (f < e));
                r += (lf.y > le) | ((lf.y == le) & (f + 1 < e));
                r += (lf.z > le) | ((lf.z == le) & (f + 2 < e));
                r += (lf.w > le) | ((lf.w == le) & (f + 3 < e));
            }
            if (r) atomicAdd(&rank[e], r);
        }
    }
    __syncthreads();
}

/* The y-th smallest expert id among the K first of the logit order (every wave forms it):
 * the expert a gate/up block of a one-token batch almost always gets, known before the
 * exact selection is. */
__device__ int spec_expert(const int *rank, int X, int K, int y)
{
    const int lane = threadIdx.x & 63;
    int below = 0, found = 0;
    for (int e0 = 0; e0 < X; e0 += 64) {
        const int e = e0 + lane;
        const unsigned long long m = __ballot(e < X && rank[e] < K);
        const int c = __popcll(m);
        if (y >= below && y < below + c) {
            /* the (y - below)-th set bit of m */
            const int pos = below + __popcll(m & ((1ULL << lane) - 1ULL));
            const unsigned long long hit = __ballot(e < X && rank[e] < K && pos == y);
            found = e0 + (int)__builtin_ctzll(hit);
        }
        below += c;
    }
    return found;
}

/* The reference's top K (src/model.c:1053-1062) from route_one_rank's softmax and logit
 * ranks, on one wave: sel[0 .. K-1] in selection order. cand holds K + 1 ints. */
__device__ void topk_from_ranks(int K, int X, const float *L, const double *P, const int *rank, int *cand, int *sel)
{
    const int lane = threadIdx.x & 63;
    /* A NaN or infinite logit makes z and every p NaN (p is finite otherwise): no p then
     * compares greater, so the reference's argmax rounds take experts 0 .. K-1 in order. The
     * logit ranks are no permutation then and stay unused. */
    const bool nan_p = P[0] != P[0];
    if (!nan_p)
        for (int e = lane; e < X; e += 64)
            if (rank[e] <= K) cand[rank[e]] = e;
    wave_sync();
    /* Equal logits have equal p and sort by index in both orders. A p tie between logits of
     * different value sorts by logit here but by index in the reference, so every adjacent
     * pair must have strictly decreasing p or equal logits; across the boundary (K-1, K) the p
     * must decrease strictly, since an equal-p run may continue past K with a lower logit and
     * a lower index. With K == X there is no expert past the boundary. */
    bool ok = true;
    if (lane < K && lane + 1 < X && !nan_p) {
        const int a = cand[lane], b = cand[lane + 1];
        ok = P[a] > P[b] || (lane < K - 1 && L[a] == L[b]);
    }
    if (nan_p) {
        if (lane < K) sel[lane] = lane;
    } else if (__ballot(!ok) == 0ULL) {
        if (lane < K) sel[lane] = cand[lane];
    } else {
        /* a rounding tie among the candidates: rank the p exactly */
        for (int e = lane; e < X; e += 64) {
            const double pe = P[e];
            int r = 0;
            for (int f = 0; f < X; f++) {
                const double pf = P[f];
                r += (pf > pe) | ((pf == pe) & (f < e));
            }
            if (r < K) sel[r] = e;
        }
    }
    wave_sync();
}

/* Second half of the one-token routing: the exact top K (with the rounding-tie check),
 * weights, slots and the published scratch arrays; ends with a block barrier. */
__device__ void route_one_select(const Scratch &S, int K, int X, SmallRoute *R, float *L, double *P, int *rank,
                                 int *selidx, int *start)
{
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    if (wave == 0) {
        topk_from_ranks(K, X, L, P, rank, R->cand, R->sel);
        const int sj = lane < K ? R->sel[lane] : 0;
        const double pj = lane < K ? P[sj] : 0.0;
        double wsum = 0.0;
        for (int j = 0; j < K; j++) wsum += __shfl(pj, j);
        if (lane < K) {
            R->wt[lane] = (float)(pj / wsum);
            selidx[sj] = lane;
        }
        wave_sync();
        /* the token's slots are its experts in ascending order */
        int below = 0;
        for (int e0 = 0; e0 <= X; e0 += 64) {
            const int e = e0 + lane;
            const int j = e < X ? selidx[e] : -1;
            const unsigned long long m = __ballot(j >= 0);
            const int pos = below + __popcll(m & ((1ULL << lane) - 1ULL));
            if (e <= X) start[e] = pos;
            if (j >= 0) {
                R->work[pos] = make_int4(e, pos, pos + 1, 0);
                R->slot_of[j] = pos;
            }
            below += __popcll(m);
        }
        wave_sync();
        if (lane < K) R->slot_t[lane] = 0;
        if (lane == 0) R->na = K;
    }
    __syncthreads();
    if (blockIdx.x == 0 && blockIdx.y == 0) {
        for (int i = tid; i < K; i += blockDim.x) {
            S.sel[i] = R->sel[i];
            S.wt[i] = R->wt[i];
            S.slot_t[i] = 0;
            S.slot_of[i] = R->slot_of[i];
        }
        for (int e = tid; e <= X; e += blockDim.x) S.start[e] = start[e];
        for (int i = tid; i < X; i += blockDim.x) {
            S.work[i] = i < K ? R->work[i] : make_int4(-1, 0, 0, 0);
            if (i < K) {
                S.active[i] = R->work[i].x;
                S.tiles[i] = make_int4(R->work[i].x, i, i + 1, 0);   /* one slot per expert */
            }
        }
        if (tid == 0) {
            S.meta[0] = K;
            S.meta[1] = K;
        }
    }
}

/* ------------------------------------------------------------------ gate / up ---- */

struct GateUpArgs {
    const uint8_t *gate, *up;
    uint64_t rb, eb;
    int E, F, K, X, T, debug;
    int quant_act;     /* blocks of 32 rows also store the int8 activation blocks (aq, aqk) */
    Scratch S;
};

/* Pairs of one row for NT tokens, loads batched B pairs at a time so their latencies overlap. */
template <int NT, int B>
__device__ __forceinline__ void q4_0_rows(const uint32_t *Wrow, int p, const uint8_t *x0, size_t xrec, int q0, int nq,
                                          int nt, RowAcc *acc)
{
    int q = 0;
    for (; q + B <= nq; q += B) {
        Q4Pair w[B];
        XPair x[B][NT];
#pragma unroll
        for (int u = 0; u < B; u++) {
            w[u] = q4_0_load(Wrow + (q + u) * 9, p);
#pragma unroll
            for (int n = 0; n < NT; n++)
                if (n < nt) x[u][n] = x_load(x0 + n * xrec + (size_t)(q0 + q + u) * kPairBytes, p);
        }
#pragma unroll
        for (int u = 0; u < B; u++)
#pragma unroll
            for (int n = 0; n < NT; n++)
                if (n < nt) q4_0_math(w[u], x[u][n], acc[n]);
    }
    for (; q < nq; q++) {
        const Q4Pair w = q4_0_load(Wrow + q * 9, p);
#pragma unroll
        for (int n = 0; n < NT; n++)
            if (n < nt) q4_0_math(w, x_load(x0 + n * xrec + (size_t)(q0 + q) * kPairBytes, p), acc[n]);
    }
}

/* The same for Q4_1 rows (40-byte block pairs). */
template <int NT, int B>
__device__ __forceinline__ void q4_1_rows(const uint32_t *Wrow, int p, const uint8_t *x0, size_t xrec, int q0, int nq,
                                          int nt, RowAcc *acc)
{
    int q = 0;
    for (; q + B <= nq; q += B) {
        Q41Pair w[B];
        XPair x[B][NT];
#pragma unroll
        for (int u = 0; u < B; u++) {
            w[u] = q4_1_load(Wrow + (q + u) * 10, p);
#pragma unroll
            for (int n = 0; n < NT; n++)
                if (n < nt) x[u][n] = x_load(x0 + n * xrec + (size_t)(q0 + q + u) * kPairBytes, p);
        }
#pragma unroll
        for (int u = 0; u < B; u++)
#pragma unroll
            for (int n = 0; n < NT; n++)
                if (n < nt) q4_1_math(w[u], x[u][n], acc[n]);
    }
    for (; q < nq; q++) {
        const Q41Pair w = q4_1_load(Wrow + q * 10, p);
#pragma unroll
        for (int n = 0; n < NT; n++)
            if (n < nt) q4_1_math(w, x_load(x0 + n * xrec + (size_t)(q0 + q) * kPairBytes, p), acc[n]);
    }
}

/* Row dots of one Q4_0 (TYPE 2) or Q4_1 (TYPE 3) row for nt <= NT tokens, batching as many
 * pairs as nt allows: a kernel built for NT tokens per pass mostly serves one-token slot
 * tiles at small batches, where NT-wide batching would leave each pair's LDS reads unhidden. */
template <int TYPE, int NT>
__device__ __forceinline__ void q4_rows_nt(const uint32_t *Wrow, int p, const uint8_t *x0, size_t xrec, int q0,
                                           int nq, int nt, RowAcc *acc)
{
    constexpr int B = NT >= 4 ? 1 : (NT == 2 ? 2 : 4);
    if (NT >= 2 && nt == 1) {
        if (TYPE == 3) q4_1_rows<1, 4>(Wrow, p, x0, xrec, q0, nq, 1, acc);
        else q4_0_rows<1, 4>(Wrow, p, x0, xrec, q0, nq, 1, acc);
    } else if (NT >= 4 && nt == 2) {
        if (TYPE == 3) q4_1_rows<2, 2>(Wrow, p, x0, xrec, q0, nq, 2, acc);
        else q4_0_rows<2, 2>(Wrow, p, x0, xrec, q0, nq, 2, acc);
    } else {
        if (TYPE == 3) q4_1_rows<NT, B>(Wrow, p, x0, xrec, q0, nq, nt, acc);
        else q4_0_rows<NT, B>(Wrow, p, x0, xrec, q0, nq, nt, acc);
    }
}

/* Offset scale of quad_finish for a row type (Q4_0 8, Q4_1 -1, Q6_K 32). */
__host__ __device__ constexpr float finish_scale(int type) { return type == 2 ? 8.0f : (type == 3 ? -1.0f : 32.0f); }

/* LDS bytes of a gateup block (shared by the kernel's carve-up and the launcher). */
/* LDS row stride of the gate/up kernel's staged rows (bytes; odd in 16-byte units, Q6_K in
 * 4-byte units: a super-block from the 4-byte boundary below it, 216 bytes). */
__host__ __device__ constexpr int gateup_ws(int type, int CB)
{
    return type == 14 ? 220 : CB * (type == 3 ? 20 : 18) + (((CB * (type == 3 ? 20 : 18) / 16) & 1) ? 0 : 16);
}

__host__ __device__ constexpr size_t gateup_lds(int W, int NT, int CB, int nP, int sel, int type = 2)
{
    return (size_t)W * 16 * gateup_ws(type, CB) + (size_t)NT * nP * kPairBytes +
           (size_t)NT * 2 * 8 * W * 4 +
           (sel ? sizeof(SmallRoute) + (size_t)kMaxExperts * (8 + 4 + 4 + 4) + (kMaxExperts + 1) * 4 : 0);
}

/* One block of W waves: expert work[blockIdx.y].x, gate rows and up rows r0 .. r0+8W-1
 * (r0 = 8W*blockIdx.x), for every slot of the expert, NT slots per pass. W is chosen so the
 * grid spreads evenly over the CUs (48 row pairs of the 235B shape: 256 blocks, one per CU).
 * Wave w owns gate rows r0+8w .. r0+8w+7 (quads 0-7) and the same up rows (quads 8-15) and
 * streams exactly those rows in chunks of CB blocks, D chunks in flight: a chunk is copied
 * into the wave's own LDS buffer, its registers are refilled with chunk c+D, then its dots
 * run, so each wave computes while its later bytes are still on the way and waves never wait
 * for each other. With SEL the block first routes the batch itself; a one-token batch
 * requests its input records before that, so they arrive during the routing. Epilogue:
 * a = silu(g)*u (src/model.c:989-997); the int8 requantisation of a happens where all 32 rows
 * of a block are known (the down kernel). */
template <int TYPE, int W, int NT, int CB, int D, int SEL>
__global__ __launch_bounds__(64 * W) void gateup_kernel(GateUpArgs a)
{
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr bool Q6 = TYPE == 14;
    static_assert(TYPE == 2 || TYPE == 3 || (Q6 && CB == 8), "Q4_0 / Q4_1 rows, or Q6_K super-blocks");
    constexpr int NTH = 64 * W, R = 8 * W;
    constexpr int BB = TYPE == 3 ? 20 : 18;           /* bytes per 32-block (Q4 types)        */
    constexpr int UNIT = Q6 ? 4 : 16;                 /* bytes per load                       */
    constexpr int SPR = Q6 ? 54 : CB * BB / 16;       /* loads per row per chunk              */
    constexpr int NSL = 16 * SPR;                     /* loads of one wave's chunk            */
    constexpr int SPT = (NSL + 63) / 64;              /* loads per lane per chunk             */
    constexpr int WS = gateup_ws(TYPE, CB);           /* LDS row stride                       */
    typedef typename std::conditional<Q6, uint32_t, u32x4>::type Unit;
    const int nbE = a.E >> 5, nP = nbE >> 1, nchunk = nbE / CB;
    const int xsl = nP * 6;                           /* 16-byte slots of one token's records */
    constexpr int XS = (NT * (4096 / 64) * 6 + NTH - 1) / NTH;  /* x slots per thread in registers */
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, qd = lane >> 2, p = lane & 3;
    uint8_t *wbuf = smem + wave * 16 * WS;
    uint8_t *xbuf = smem + W * 16 * WS;
    float *res = (float *)(xbuf + NT * nP * kPairBytes);               /* [NT][2R] */
    PHASE(1024, 0);

    /* a one-token batch: its only token's records can be requested before the routing */
    u32x4 xv[XS];
    if constexpr (NT == 1) {
#pragma unroll
        for (int m = 0; m < XS; m++) xv[m] = ((const u32x4 *)a.S.xqk)[min(tid + NTH * m, xsl - 1)];
    }
    const int r0 = (int)blockIdx.x * R, rw = r0 + 8 * wave;     /* this wave's first row */
    const uint8_t *gbase, *ubase;
    Unit wv[D][SPT];
    auto load_chunk = [&](int c, Unit *dst) {
#pragma unroll
        for (int m = 0; m < SPT; m++) {
            const int i = min(lane + 64 * m, NSL - 1), row = i / SPR, j = i - row * SPR;
            const uint8_t *rp = row < 8 ? gbase + (size_t)row * a.rb : ubase + (size_t)(row - 8) * a.rb;
            if constexpr (Q6)     /* the super-block starts 2 bytes past a 4-byte boundary on odd chunks */
                dst[m] = *(const uint32_t *)(rp + (size_t)(c * 210 - 2 * (c & 1)) + 4 * j);
            else
                dst[m] = *(const u32x4 *)(rp + (size_t)c * CB * BB + 16 * j);
        }
    };
    auto set_expert = [&](int ex) {
        gbase = a.gate + (size_t)ex * a.eb + (size_t)rw * a.rb;
        ubase = a.up + (size_t)ex * a.eb + (size_t)rw * a.rb;
    };
    int4 wk;
    const int *slot_t = a.S.slot_t;
    bool prefetched = false;
    if constexpr (SEL) {
        SmallRoute *sr = (SmallRoute *)(res + NT * 2 * R);
        double *P = (double *)(sr + 1);
        float *L = (float *)(P + kMaxExperts);
        int *rank = (int *)(L + kMaxExperts);
        route_one_rank(a.S.logits, a.X, L, P, rank, rank + kMaxExperts);
        PHASE(1024, 1);
        /* start streaming the expert the logit order points at while the exact selection
         * finishes; the rare block whose expert changes reloads below */
        const int e_spec = spec_expert(rank, a.X, a.K, (int)blockIdx.y);
        set_expert(e_spec);
        if (wave > 0) {                    /* wave 0 finishes the selection first */
#pragma unroll
            for (int d = 0; d < D; d++)
                if (d < nchunk) load_chunk(d, wv[d]);
        }
        route_one_select(a.S, a.K, a.X, sr, L, P, rank, rank + kMaxExperts, rank + 2 * kMaxExperts);
        PHASE(1024, 2);
        if ((int)blockIdx.y >= sr->na) return;
        wk = sr->work[blockIdx.y];
        slot_t = sr->slot_t;
        prefetched = wk.x == e_spec && wave > 0;
    } else {
        if ((int)blockIdx.y >= a.S.meta[1]) return;
        wk = a.S.tiles[blockIdx.y];                  /* at most kTileN slots of one expert */
    }
    const int e = wk.x, s_begin = wk.y, s_end = wk.z;
    if (!prefetched) {
        /* the first pass's weight chunks go out before the token records are fetched */
        set_expert(e);
#pragma unroll
        for (int d = 0; d < D; d++)
            if (d < nchunk) load_chunk(d, wv[d]);
    }
    const int F = a.F;
    const int rho = qd < 8 ? 8 * wave + qd : R + 8 * wave + (qd - 8);   /* tile row of this quad */
    const bool tok_bytes = SEL && a.T <= 256;       /* work.w holds the first four tokens */

    for (int g0 = s_begin; g0 < s_end; g0 += NT) {
        const int nt = min(NT, s_end - g0);
        if constexpr (NT > 1) {
#pragma unroll
            for (int m = 0; m < XS; m++) {
                const int i = min(tid + NTH * m, nt * xsl - 1), n = i / xsl, off = i - n * xsl;
                const int k = g0 - s_begin + n;
                const int tok = (k < 4 && tok_bytes) ? (wk.w >> (8 * k)) & 0xff : slot_t[g0 + n];
                xv[m] = ((const u32x4 *)(a.S.xqk + (size_t)tok * nP * kPairBytes))[off];
            }
        }
        if (NT > 1 || g0 == s_begin) {
#pragma unroll
            for (int m = 0; m < XS; m++) ((u32x4 *)xbuf)[min(tid + NTH * m, nt * xsl - 1)] = xv[m];
            /* rows wider than 4096: the records past the register share */
            for (int i = tid + NTH * XS; i < nt * xsl; i += NTH) {
                const int n = i / xsl, off = i - n * xsl, k = g0 - s_begin + n;
                const int tok = NT == 1 ? 0 : ((k < 4 && tok_bytes) ? (wk.w >> (8 * k)) & 0xff : slot_t[g0 + n]);
                ((u32x4 *)xbuf)[i] = ((const u32x4 *)(a.S.xqk + (size_t)tok * nP * kPairBytes))[off];
            }
        }
        __syncthreads();
        RowAcc acc[NT];
        for (int n = 0; n < NT; n++) acc[n] = RowAcc{ 0.0f, 0.0f, 0.0f };
        if (g0 != s_begin) {
#pragma unroll
            for (int d = 0; d < D; d++)
                if (d < nchunk) load_chunk(d, wv[d]);
        }
        for (int c0 = 0; c0 < nchunk; c0 += D) {
#pragma unroll
            for (int d = 0; d < D; d++) {
                const int c = c0 + d;
                if (c < nchunk) {
                    wave_sync();
#pragma unroll
                    for (int m = 0; m < SPT; m++) {
                        const int i = min(lane + 64 * m, NSL - 1), row = i / SPR, j = i - row * SPR;
                        *(Unit *)(wbuf + row * WS + UNIT * j) = wv[d][m];
                    }
                    wave_sync();
                    if (c + D < nchunk) load_chunk(c + D, wv[d]);
                    if constexpr (Q6) {
                        /* the 8 blocks of super-block c (src/kernels.c:142-170) for every slot */
                        auto superblock = [&](auto al) {
#pragma unroll
                            for (int h = 0; h < 2; h++)
#pragma unroll
                                for (int g = 0; g < 4; g++) {
                                    const int blk = c * 8 + h * 4 + g;
                                    const Q6W w = q6_k_weights<decltype(al)::value>(wbuf + qd * WS, al ? 0 : 2, h, g, p);
#pragma unroll
                                    for (int n = 0; n < NT; n++)
                                        if (n < nt)
                                            q6_k_token(w, xbuf + (size_t)n * nP * kPairBytes + (size_t)(blk >> 1) * kPairBytes,
                                                       p, blk & 1, acc[n]);
                                }
                        };
                        if (c & 1) superblock(std::integral_constant<bool, false>());
                        else superblock(std::integral_constant<bool, true>());
                    } else {
                        q4_rows_nt<TYPE, NT>((const uint32_t *)(wbuf + qd * WS), p, xbuf, (size_t)nP * kPairBytes,
                                             c * (CB / 2), CB / 2, nt, acc);
                    }
                    if (c == 0 && g0 == s_begin) PHASE(1024, 3);
                }
            }
        }
        if (g0 == s_begin) PHASE(1024, 4);
#pragma unroll
        for (int n = 0; n < NT; n++) {
            const float v = quad_finish(acc[n], finish_scale(TYPE));
            if (p == 0 && n < nt) res[n * 2 * R + rho] = v;
        }
        __syncthreads();
        for (int i = tid; i < nt * R; i += NTH) {
            const int n = i / R, l = i - n * R, s = g0 + n;
            const float g = res[n * 2 * R + l], u = res[n * 2 * R + R + l];
            const float av = silu_ref(g) * u;
            a.S.act[(size_t)s * F + r0 + l] = av;
            if (a.debug) {
                a.S.gu[(size_t)s * 2 * F + r0 + l] = g;
                a.S.gu[(size_t)s * 2 * F + F + r0 + l] = u;
            }
            if (R % 32 == 0 && a.quant_act) res[n * 2 * R + l] = av;
        }
        __syncthreads();
        if constexpr (R % 32 == 0 && !SEL) {
            /* the int8 blocks of the block's whole 32-row groups (src/model.c:996-997), as
             * act_quant_kernel forms them */
            if (a.quant_act) {
                const int nbF = F >> 5;
                for (int i = tid; i < nt * (R / 32); i += NTH) {
                    const int n = i / (R / 32), g = i - n * (R / 32), s = g0 + n, blk = (r0 >> 5) + g;
                    float v[32];
#pragma unroll
                    for (int j = 0; j < 32; j++) v[j] = res[n * 2 * R + 32 * g + j];
                    const Q8Vals q = quantize_block(v);
                    store_q8(q, a.S.aq + (size_t)s * nbF + blk);
                    store_pair_half(q, (uint32_t *)(a.S.aqk + ((size_t)s * (nbF >> 1) + (blk >> 1)) * kPairBytes),
                                    blk & 1);
                }
                __syncthreads();
            }
        }
    }
    PHASE(1024, 5);
}

template <int TYPE, int W, int NT, int SEL>
static void launch_gateup_w(const GateUpArgs &a, int CB, dim3 grid, size_t lds, hipStream_t st)
{
    if constexpr (TYPE == 14)      /* a super-block per chunk, three in flight */
        QLAUNCH("gateup", (gateup_kernel<TYPE, W, NT, 8, 3, SEL>), grid, dim3(64 * W), lds, st, a);
    else if (CB == 16) QLAUNCH("gateup", (gateup_kernel<TYPE, W, NT, 16, 2, SEL>), grid, dim3(64 * W), lds, st, a);
    else QLAUNCH("gateup", (gateup_kernel<TYPE, W, NT, 8, 1, SEL>), grid, dim3(64 * W), lds, st, a);
}

template <int TYPE, int NT, int SEL>
static void launch_gateup_nt(const GateUpArgs &a, int W, int CB, dim3 grid, size_t lds, hipStream_t st)
{
    if (W == 6) launch_gateup_w<TYPE, 6, NT, SEL>(a, CB, grid, lds, st);
    else if (W == 4) launch_gateup_w<TYPE, 4, NT, SEL>(a, CB, grid, lds, st);
    else if (W == 3) launch_gateup_w<TYPE, 3, NT, SEL>(a, CB, grid, lds, st);
    else launch_gateup_w<TYPE, 2, NT, SEL>(a, CB, grid, lds, st);
}

template <int TYPE>
static void launch_gateup_type(const GateUpArgs &a, int sel, int NT, int W, int CB, dim3 grid, size_t lds,
                               hipStream_t st)
{
    if (sel) launch_gateup_nt<TYPE, 1, 1>(a, W, CB, grid, lds, st);     /* one token: NT == 1 */
    else if (NT == 2) launch_gateup_nt<TYPE, 2, 0>(a, W, CB, grid, lds, st);
    else launch_gateup_nt<TYPE, 1, 0>(a, W, CB, grid, lds, st);
}

/* Waves per gateup block: the W (rows 8W per block) whose grid, at the largest possible
 * number of active experts, puts the least work on the busiest CU (one block per CU per
 * pass); ties go to the larger block. Slot-tile grids (batch) leave out W = 6, measured
 * 20-60 % slower there at the 235B shape (W = 2, 3, 4 within 2 % of each other). */
int gateup_waves(int F, int max_active, int n_cu, int batch, int rows32)
{
    int best = 0, best_cost = 0;
    for (int W : { 6, 4, 3, 2 }) {
        if (F % (8 * W) || (batch && W == 6) || (rows32 && (8 * W) % 32)) continue;
        const long nblk = (long)(F / (8 * W)) * max_active;
        const long cost = ((nblk + n_cu - 1) / n_cu) * W;
        if (!best || cost < best_cost) { best = W; best_cost = (int)cost; }
    }
    return best;
}

bool gateup_streams(const LayerDev &L)
{
    return L.gate_type == L.up_type &&
           (L.gate_type == 2 || L.gate_type == 3 || (L.gate_type == 14 && L.gate_rb % 4 == 0));
}

hipError_t launch_gateup_exact(const Shape &s, const LayerDev &L, const Scratch &S, int T, int debug, int n_cu,
                               int quant_act, hipStream_t st)
{
    GateUpArgs a;
    a.quant_act = quant_act;
    a.gate = L.gate;
    a.up = L.up;
    a.rb = L.gate_rb;
    a.eb = L.gate_eb;
    a.E = s.E;
    a.F = s.F;
    a.K = s.K;
    a.X = s.X;
    a.T = T;
    a.debug = debug;
    a.S = S;
    const int nbE = s.E / 32, nP = nbE / 2;
    /* chunks of CB blocks, two in flight per wave (16-block chunks measured fastest for the
     * 4096-wide rows: less in flight per wave lets the first chunks land sooner) */
    const int CB = nbE % 32 == 0 ? 16 : 8;
    /* two slots per pass for every batch: measured faster than four at T = 4, 16, 64 and 512
     * (fewer registers and a smaller record buffer let more blocks share a CU; most
     * decode tiles hold one or two slots) and than one */
    const int NT = T >= 2 ? 2 : 1;
    const int maxact = s.X < T * s.K ? s.X : T * s.K;
    const int sel = use_small_route(T, s.K);
    const int rows_y = sel ? maxact : maxact + T * s.K / kTileN + 1;   /* active experts, or slot tiles */
    const int W = gateup_waves(s.F, rows_y, n_cu, !sel, quant_act);
    if (!W) return hipErrorInvalidValue;
    dim3 grid(s.F / (8 * W), rows_y);
    if (!gateup_streams(L)) return hipErrorInvalidValue;
    const int cb = L.gate_type == 14 ? 8 : CB;
    const size_t lds = gateup_lds(W, NT, cb, nP, sel, L.gate_type);
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    if (L.gate_type == 14) launch_gateup_type<14>(a, sel, NT, W, cb, grid, lds, st);
    else if (L.gate_type == 3) launch_gateup_type<3>(a, sel, NT, W, cb, grid, lds, st);
    else launch_gateup_type<2>(a, sel, NT, W, cb, grid, lds, st);
    return hipGetLastError();
}

/* ------------------------------------------------------------------ down + combine ---- */

struct DownArgs {
    const uint8_t *down;
    uint64_t rb, eb;
    int E, F, K, T, X;
    int quant;         /* the kernel forms the activations' int8 blocks (else they are in aqk) */
    float *out;
    Scratch S;
};

/* Rows of one expert's matrix against the int8 input records of one slot tile (at most kTileN
 * slots of one expert, from the dispatch's tile list): RT rows R0 .. R0+RT-1 (one per lane
 * quad), staged once in LDS, NT slots per pass. The records are the slot's own (down: the
 * activations) or, with BT, those of the slot's token (gate / up: the layer input). Writes
 * y[slot * y_stride + y_off + row]; for down the combine runs afterwards in selection order. */
struct TileArgs {
    const uint8_t *w;       /* expert 0's rows of rb bytes; expert e at w + e*eb */
    uint64_t rb, eb;
    int cols;               /* elements per row (a multiple of 64; 256 for Q6_K) */
    const uint8_t *rec;     /* pair records, cols/64 per slot (or per token with BT) */
    float *y;
    int y_stride, y_off;
    Scratch S;
};

template <int TYPE, int NT, int RT, int BT, int QA = 0>
__global__ __launch_bounds__(4 * RT) void tile_rows_kernel(TileArgs a)
{
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int NTH = 4 * RT;
    if ((int)blockIdx.y >= a.S.meta[1]) return;
    const int4 tl = a.S.tiles[blockIdx.y];
    const int e = tl.x, s0 = tl.y, ns = tl.z - tl.y;
    const int tid = threadIdx.x, quad = tid >> 2, p = tid & 3;
    const int R0 = (int)blockIdx.x * RT, nPF = a.cols >> 6, xrec = nPF * kPairBytes, x16 = xrec >> 4;
    const int rb = (int)a.rb, n16 = RT * rb / 16;
    uint8_t *tile = smem;
    uint8_t *xbuf = smem + ((RT * rb + 15) & ~15);            /* [NT][xrec] */
    const u32x4 *wsrc = (const u32x4 *)(a.w + (size_t)e * a.eb + (size_t)R0 * a.rb);
    /* 16-byte slot i of pass g0's input records */
    auto rec_slot = [&](int g0, int i) -> const u32x4 * {
        const int n = i / x16;
        const size_t src = BT ? (size_t)a.S.slot_t[s0 + g0 + n] : (size_t)(s0 + g0 + n);
        return (const u32x4 *)(a.rec + src * xrec) + (i - n * x16);
    };
    /* the weight tile (up to WPT loads per thread) and the first pass's records (XPT per
     * thread; with QA the first activation block of this thread instead) are all requested
     * before any of them is waited for */
    constexpr int WPT = 16, XPT = QA ? 1 : 4;
    const int nt0 = min(NT, ns), nx0 = nt0 * x16;
    const int nbF = a.cols >> 5, nq0 = nt0 * nbF;
    u32x4 xr[XPT];
    float4 av[QA ? 8 : 1];
    /* QA: activation block i of pass g0 (slot s0+g0+i/nbF, block i%nbF), 32 floats */
    auto act_block = [&](int g0, int i) -> const float4 * {
        const int n = i / nbF;
        return (const float4 *)(a.S.act + (size_t)(s0 + g0 + n) * a.cols + (size_t)(i - n * nbF) * 32);
    };
    for (int i0 = 0; i0 < n16; i0 += NTH * WPT) {
        u32x4 v[WPT];
#pragma unroll
        for (int m = 0; m < WPT; m++) v[m] = wsrc[min(i0 + tid + NTH * m, n16 - 1)];
        if (i0 == 0) {
            if (QA) {
                const float4 *src = act_block(0, min(tid, nq0 - 1));
#pragma unroll
                for (int j = 0; j < (QA ? 8 : 1); j++) av[j] = src[j];
            } else {
#pragma unroll
                for (int m = 0; m < XPT; m++) xr[m] = *rec_slot(0, min(tid + NTH * m, nx0 - 1));
            }
        }
#pragma unroll
        for (int m = 0; m < WPT; m++)
            if (i0 + tid + NTH * m < n16) ((u32x4 *)tile)[i0 + tid + NTH * m] = v[m];
    }
    const uint8_t *row = tile + quad * rb;
    for (int g0 = 0; g0 < ns; g0 += NT) {
        const int nt = min(NT, ns - g0);
        __syncthreads();                                  /* the weights landed; xbuf is free */
        if (QA) {
            /* the int8 records of this pass's slots, formed here (src/model.c:996-997); the
             * first column of blocks also writes them out for the debug copy */
            auto quant = [&](int i, const float4 *f) {
                float v[32];
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    v[4 * j] = f[j].x; v[4 * j + 1] = f[j].y; v[4 * j + 2] = f[j].z; v[4 * j + 3] = f[j].w;
                }
                const int n = i / nbF, blk = i - n * nbF, slot = s0 + g0 + n;
                const Q8Vals q = quantize_block(v);
                store_pair_half(q, (uint32_t *)(xbuf + (size_t)n * xrec + (size_t)(blk >> 1) * kPairBytes), blk & 1);
                if (blockIdx.x == 0) {
                    store_q8(q, a.S.aq + (size_t)slot * nbF + blk);
                    store_pair_half(q, (uint32_t *)(a.S.aqk + ((size_t)slot * nPF + (blk >> 1)) * kPairBytes), blk & 1);
                }
            };
            int i = tid;
            if (g0 == 0) {
                if (tid < nq0) quant(tid, av);
                i = tid + NTH;
            }
            for (; i < nt * nbF; i += NTH) {
                float4 f[8];
                const float4 *src = act_block(g0, i);
#pragma unroll
                for (int j = 0; j < 8; j++) f[j] = src[j];
                quant(i, f);
            }
        } else {
            int i = tid;
            if (g0 == 0) {
#pragma unroll
                for (int m = 0; m < XPT; m++)
                    if (tid + NTH * m < nx0) ((u32x4 *)xbuf)[tid + NTH * m] = xr[m];
                i = tid + NTH * XPT;
            }
            for (; i < nt * x16; i += NTH) ((u32x4 *)xbuf)[i] = *rec_slot(g0, i);
        }
        __syncthreads();
        RowAcc acc[NT];
        for (int n = 0; n < NT; n++) acc[n] = RowAcc{ 0.0f, 0.0f, 0.0f };
        if (TYPE == 2 || TYPE == 3) {
            q4_rows_nt<TYPE, NT>((const uint32_t *)row, p, xbuf, (size_t)xrec, 0, nPF, nt, acc);
        } else {
            const int nsb = a.cols >> 8;
            const uint32_t rowoff = (uint32_t)(row - tile);
            /* rows of a multiple of 4 bytes: even super-blocks start 4-aligned on every row */
            const bool even_al = (rb & 3) == 0;
            auto superblock = [&](auto al, int sbi) {
                const uint32_t sb = rowoff + (uint32_t)(sbi * 210);
#pragma unroll
                for (int h = 0; h < 2; h++)
#pragma unroll
                    for (int g = 0; g < 4; g++) {
                        const int blk = sbi * 8 + h * 4 + g;
                        const Q6W w = q6_k_weights<decltype(al)::value>(tile, sb, h, g, p);
#pragma unroll
                        for (int n = 0; n < NT; n++)
                            if (n < nt)
                                q6_k_token(w, xbuf + (size_t)n * xrec + (size_t)(blk >> 1) * kPairBytes, p, blk & 1,
                                           acc[n]);
                    }
            };
            for (int sbi = 0; sbi < nsb; sbi++) {
                if (even_al && !(sbi & 1)) superblock(std::integral_constant<bool, true>(), sbi);
                else superblock(std::integral_constant<bool, false>(), sbi);
            }
        }
#pragma unroll
        for (int n = 0; n < NT; n++) {
            const float d = quad_finish(acc[n], finish_scale(TYPE));
            if (p == 0 && n < nt) a.y[(size_t)(s0 + g0 + n) * a.y_stride + a.y_off + R0 + quad] = d;
        }
    }
}

/* One-token batch, Q4_0, Q4_1 or Q6_K down weights (K <= 8 experts, one slot each, slot j = j-th
 * active expert): one block per RD output rows r0 .. r0+RD-1 and RD/2 waves. Wave w owns the
 * 16/RD active experts 16w/RD .. (16 rows, one per lane quad) and streams exactly those rows in
 * chunks of CB blocks, D chunks in flight, through its own LDS buffer, so its dots start as
 * soon as its first bytes land. Q6_K rows go a super-block per chunk (CB = 8), 216 bytes from
 * the 4-byte boundary below it in 4-byte units (row bytes a multiple of 4; tensors carry 256
 * bytes of tail padding). The prologue requests the first chunks, then quantises the K
 * activation rows into int8 pair records in LDS (block 0 also writes them out for the debug
 * copy-back). The block ends with the weighted combine of its RD rows in selection order
 * (src/model.c:1152-1162). */
template <int TYPE, int CB, int D, int RD>
__global__ __launch_bounds__(32 * RD) void down_t1_kernel(DownArgs a)
{
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr bool Q6 = TYPE == 14;
    static_assert(!Q6 || CB == 8, "a Q6_K chunk is one super-block");
    constexpr int NW = RD / 2, NTH = 64 * NW;         /* waves: 8 experts x RD rows / 16      */
    constexpr int EPW = 16 / RD;                      /* experts per wave                     */
    constexpr int QPT = (512 + NTH - 1) / NTH;        /* int8 blocks per thread in registers  */
    constexpr int BB = TYPE == 3 ? 20 : 18;           /* bytes per 32-block (Q4 types)        */
    constexpr int UNIT = 16;                          /* bytes per load                       */
    /* loads per row per chunk; a Q6_K super-block (210 bytes, 2-byte aligned) is read as the
     * 14 16-byte units from the 16-byte boundary below it, and found at that row's offset */
    constexpr int SPR = Q6 ? 14 : CB * BB / 16;
    constexpr int NSL = 16 * SPR;                     /* loads of one wave's chunk            */
    constexpr int SPT = (NSL + 63) / 64;              /* loads per lane per chunk             */
    /* LDS row stride, odd in 16-byte units */
    constexpr int WS = Q6 ? 240 : CB * BB + ((SPR & 1) ? 0 : 16);
    typedef u32x4 Unit;
    const int tid = threadIdx.x, lane = tid & 63, qd = lane >> 2, p = lane & 3;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r0 = (int)blockIdx.x * RD, E = a.E, K = a.K, nbF = a.F >> 5, nPF = a.F >> 6;
    const int nchunk = nbF / CB, xrec = nPF * kPairBytes;
    uint8_t *wbuf = smem + wave * 16 * WS;
    uint8_t *xbuf = smem + NW * 16 * WS;              /* [K][xrec]                            */
    float *dnl = (float *)(xbuf + (size_t)K * xrec);  /* [K][RD]                              */

    /* this wave's experts, j0 = EPW*w and j0 + 1 when a wave holds two, and the combine's
     * weights and slots: wave-uniform scalar loads, requested first, so that the weight rows
     * are not requested behind the activation loads (vector loads complete in order) */
    const int j0 = EPW * wave, j1 = j0 + EPW - 1;
    const int e0 = j0 < K ? a.S.work[j0].x : -1, e1 = j1 < K ? a.S.work[j1].x : -1;
    float wtk[kSelNS];
    int sok[kSelNS];
#pragma unroll
    for (int j = 0; j < kSelNS; j++) {
        wtk[j] = a.S.wt[min(j, K - 1)];
        sok[j] = a.S.slot_of[min(j, K - 1)];
    }

    /* the activations to quantise: 32 floats per int8 block, the first QPT*NTH in registers */
    const int nqb = K * nbF;
    float4 av[QPT][8];
#pragma unroll
    for (int u = 0; u < QPT; u++) {
        const float4 *src = (const float4 *)(a.S.act + (size_t)min(tid + NTH * u, nqb - 1) * 32);
#pragma unroll
        for (int j = 0; j < 8; j++) av[u][j] = src[j];
    }
    const uint8_t *b0 = a.down + (size_t)max(e0, 0) * a.eb + (size_t)r0 * a.rb;
    const uint8_t *b1 = a.down + (size_t)max(e1, 0) * a.eb + (size_t)r0 * a.rb;
    __builtin_amdgcn_sched_barrier(0);
    Unit wv[D][SPT];
    auto load_chunk = [&](int c, Unit *dst) {
#pragma unroll
        for (int m = 0; m < SPT; m++) {
            const int i = min(lane + 64 * m, NSL - 1), row = i / SPR, j = i - row * SPR;
            const uint8_t *rp = (EPW == 1 || row < RD) ? b0 + (size_t)row * a.rb : b1 + (size_t)(row - RD) * a.rb;
            if constexpr (Q6)     /* up to 14 bytes past the super-block: within the tensor's tail padding */
                dst[m] = *(const u32x4 *)(((uintptr_t)(rp + (size_t)c * 210) & ~(uintptr_t)15) + 16 * j);
            else
                dst[m] = *(const u32x4 *)(rp + (size_t)c * CB * BB + 16 * j);
        }
    };
    PHASE(2048, 0);
    const bool active = e0 >= 0;
    if (active) {
#pragma unroll
        for (int d = 0; d < D; d++)
            if (d < nchunk) load_chunk(d, wv[d]);
    }
    PHASE(2048, 1);
    auto quant = [&](int b, const float *v) {
        const int s = b / nbF, blk = b - s * nbF;
        const Q8Vals q = quantize_block(v);
        store_pair_half(q, (uint32_t *)(xbuf + (size_t)s * xrec + (size_t)(blk >> 1) * kPairBytes), blk & 1);
        if (blockIdx.x == 0) {
            store_q8(q, a.S.aq + b);
            store_pair_half(q, (uint32_t *)(a.S.aqk + ((size_t)s * (nbF >> 1) + (blk >> 1)) * kPairBytes), blk & 1);
        }
    };
#pragma unroll
    for (int u = 0; u < QPT; u++) {
        const int b = tid + NTH * u;
        if (b < nqb) {
            float v[32];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                v[4 * j] = av[u][j].x; v[4 * j + 1] = av[u][j].y; v[4 * j + 2] = av[u][j].z; v[4 * j + 3] = av[u][j].w;
            }
            quant(b, v);
        }
    }
    for (int b = tid + NTH * QPT; b < nqb; b += NTH) {  /* rows longer than the register share */
        float v[32];
        const float4 *src = (const float4 *)(a.S.act + (size_t)b * 32);
        for (int j = 0; j < 8; j++) {
            const float4 f = src[j];
            v[4 * j] = f.x; v[4 * j + 1] = f.y; v[4 * j + 2] = f.z; v[4 * j + 3] = f.w;
        }
        quant(b, v);
    }
    __syncthreads();
    PHASE(2048, 2);
    if (active) {
        /* quad qd: expert j0 + qd/RD, row r0 + qd%RD; its slot is its active index */
        const int jq = j0 + qd / RD, rr = qd % RD;
        const uint8_t *xq = xbuf + (size_t)min(jq, K - 1) * xrec;
        const uint8_t *rq = (EPW == 1 || qd < RD ? b0 : b1) + (size_t)rr * a.rb;   /* this quad's row */
        RowAcc acc[1] = { RowAcc{ 0.0f, 0.0f, 0.0f } };
        for (int c0 = 0; c0 < nchunk; c0 += D) {
#pragma unroll
            for (int d = 0; d < D; d++) {
                const int c = c0 + d;
                if (c < nchunk) {
                    wave_sync();
#pragma unroll
                    for (int m = 0; m < SPT; m++) {
                        const int i = min(lane + 64 * m, NSL - 1), row = i / SPR, j = i - row * SPR;
                        *(Unit *)(wbuf + row * WS + UNIT * j) = wv[d][m];
                    }
                    wave_sync();
                    if (c + D < nchunk) load_chunk(c + D, wv[d]);
                    if constexpr (Q6) {
                        /* the super-block's offset in the row's staged units; a multiple of 4
                         * on even chunks (rows are 4-byte aligned), 2 past one on odd ones */
                        const uint32_t sbo = (uint32_t)((uintptr_t)(rq + (size_t)c * 210) & 15);
                        /* the 8 blocks of super-block c (src/kernels.c:142-170) */
                        auto superblock = [&](auto al) {
#pragma unroll
                            for (int h = 0; h < 2; h++)
#pragma unroll
                                for (int g = 0; g < 4; g++) {
                                    const int blk = c * 8 + h * 4 + g;
                                    const Q6W w = q6_k_weights<decltype(al)::value>(wbuf + qd * WS, sbo, h, g, p);
                                    q6_k_token(w, xq + (size_t)(blk >> 1) * kPairBytes, p, blk & 1, acc[0]);
                                }
                        };
                        if (c & 1) superblock(std::integral_constant<bool, false>());
                        else superblock(std::integral_constant<bool, true>());
                    } else if (TYPE == 3) {
                        q4_1_rows<1, 4>((const uint32_t *)(wbuf + qd * WS), p, xq, (size_t)xrec, c * (CB / 2), CB / 2,
                                        1, acc);
                    } else {
                        q4_0_rows<1, 4>((const uint32_t *)(wbuf + qd * WS), p, xq, (size_t)xrec, c * (CB / 2), CB / 2,
                                        1, acc);
                    }
                    if (c == 0) PHASE(2048, 3);
                }
            }
        }
        PHASE(2048, 4);
        const float v = quad_finish(acc[0], finish_scale(TYPE));
        if (p == 0 && jq < K) {
            a.S.dn[(size_t)jq * E + r0 + rr] = v;
            dnl[jq * RD + rr] = v;
        }
    }
    __syncthreads();
    if (tid < RD) {
        float o = 0.0f;
#pragma unroll
        for (int j = 0; j < kSelNS; j++)
            if (j < K) o = __builtin_fmaf(wtk[j], dnl[sok[j] * RD + tid], o);
        a.out[r0 + tid] = o;
    }
    PHASE(2048, 5);
}

/* Slots of the batches the small-batch down kernel takes (two to four tokens). */
constexpr int kSmallDownNS = 32;

/* Two to four tokens, Q4_0, Q4_1 or Q6_K down weights (at most kSmallDownNS slots; Q6_K a
 * super-block per chunk, as in down_t1_kernel): the layout of down_t1_kernel, one block per RD
 * output rows and RD/2 waves, but wave w streams the active
 * experts w, w + RD/2, ... one after another, each against its one to four slots, and
 * requests the next expert's first chunks while it consumes the current one's last. The block
 * first quantises every slot's activations into LDS pair records and ends with the weighted
 * combine of its rows for every token, in selection order (src/model.c:998-1005, 1152-1162). */
template <int TYPE, int CB, int D, int RD>
__global__ __launch_bounds__(32 * RD) void down_small_kernel(DownArgs a)
{
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr bool Q6 = TYPE == 14;
    static_assert(!Q6 || CB == 8, "a Q6_K chunk is one super-block");
    constexpr int NW = RD / 2, NTH = 64 * NW, NT = 4;
    constexpr int QPT = 2;                            /* int8 blocks per thread in registers  */
    constexpr int BB = TYPE == 3 ? 20 : 18;           /* bytes per 32-block (Q4 types)        */
    constexpr int UNIT = 16;                          /* bytes per load                       */
    /* loads per row per chunk (a Q6_K super-block: the 14 16-byte units from the 16-byte
     * boundary below it, as in down_t1_kernel) */
    constexpr int SPR = Q6 ? 14 : CB * BB / 16;
    constexpr int NSL = RD * SPR;                     /* loads of one wave's chunk            */
    constexpr int SPT = (NSL + 63) / 64;              /* loads per lane per chunk             */
    constexpr int WS = Q6 ? 240 : CB * BB + ((SPR & 1) ? 0 : 16);   /* LDS row stride        */
    typedef u32x4 Unit;
    static_assert(RD == 16, "a lane quad per row of the wave's 16");
    const int tid = threadIdx.x, lane = tid & 63, qd = lane >> 2, p = lane & 3;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r0 = (int)blockIdx.x * RD, E = a.E, K = a.K, T = a.T, NS = T * K;
    const int nbF = a.F >> 5, nPF = a.F >> 6, nchunk = nbF / CB, xrec = nPF * kPairBytes;
    uint8_t *wbuf = smem + wave * 16 * WS;
    uint8_t *xbuf = smem + NW * 16 * WS;              /* [NS][xrec]                           */
    float *dnl = (float *)(xbuf + (size_t)NS * xrec); /* [NS][RD]                             */
    PHASE(2048, 0);

    /* the wave's first expert (wave-uniform scalar loads first, as in the one-token kernel) */
    const int na = a.S.meta[0];
    int j = wave;
    int4 wk = j < na ? a.S.work[j] : make_int4(-1, 0, 0, 0);
    const int nqb = NS * nbF;
    const bool quant = a.quant != 0;
    float4 av[QPT][8];
    if (quant) {
#pragma unroll
        for (int u = 0; u < QPT; u++) {
            const float4 *src = (const float4 *)(a.S.act + (size_t)min(tid + NTH * u, nqb - 1) * 32);
#pragma unroll
            for (int q = 0; q < 8; q++) av[u][q] = src[q];
        }
    }
    const uint8_t *b = a.down + (size_t)max(wk.x, 0) * a.eb + (size_t)r0 * a.rb;
    __builtin_amdgcn_sched_barrier(0);
    Unit wv[D][SPT];
    auto load_chunk = [&](int c, Unit *dst) {
#pragma unroll
        for (int m = 0; m < SPT; m++) {
            const int i = min(lane + 64 * m, NSL - 1), row = i / SPR, q = i - row * SPR;
            if constexpr (Q6)     /* up to 14 bytes past the super-block: within the tensor's tail padding */
                dst[m] = *(const u32x4 *)(((uintptr_t)(b + (size_t)row * a.rb + (size_t)c * 210) & ~(uintptr_t)15) +
                                          16 * q);
            else
                dst[m] = *(const u32x4 *)(b + (size_t)row * a.rb + (size_t)c * CB * BB + 16 * q);
        }
    };
    if (wk.x >= 0) {
#pragma unroll
        for (int d = 0; d < D; d++)
            if (d < nchunk) load_chunk(d, wv[d]);
    }
    auto quant_blk = [&](int qb, const float *v) {
        const int sl = qb / nbF, blk = qb - sl * nbF;
        const Q8Vals q = quantize_block(v);
        store_pair_half(q, (uint32_t *)(xbuf + (size_t)sl * xrec + (size_t)(blk >> 1) * kPairBytes), blk & 1);
        if (blockIdx.x == 0) {
            store_q8(q, a.S.aq + qb);
            store_pair_half(q, (uint32_t *)(a.S.aqk + ((size_t)sl * (nbF >> 1) + (blk >> 1)) * kPairBytes), blk & 1);
        }
    };
    if (quant) {
#pragma unroll
        for (int u = 0; u < QPT; u++) {
            const int qb = tid + NTH * u;
            if (qb < nqb) {
                float v[32];
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    v[4 * q] = av[u][q].x; v[4 * q + 1] = av[u][q].y; v[4 * q + 2] = av[u][q].z; v[4 * q + 3] = av[u][q].w;
                }
                quant_blk(qb, v);
            }
        }
        for (int qb = tid + NTH * QPT; qb < nqb; qb += NTH) {   /* past the register share */
            float v[32];
            const float4 *src = (const float4 *)(a.S.act + (size_t)qb * 32);
            for (int q = 0; q < 8; q++) {
                const float4 f = src[q];
                v[4 * q] = f.x; v[4 * q + 1] = f.y; v[4 * q + 2] = f.z; v[4 * q + 3] = f.w;
            }
            quant_blk(qb, v);
        }
    } else {
        /* the pair records gate/up stored: [slot][F/64] in both places */
        const int n16 = (int)((size_t)NS * xrec / 16);
        for (int i = tid; i < n16; i += NTH) ((u32x4 *)xbuf)[i] = ((const u32x4 *)a.S.aqk)[i];
    }
    __syncthreads();
    PHASE(2048, 1);
    const bool can_pre = nchunk % D == 0;             /* chunk c + D - nchunk lands in c's registers */
    while (wk.x >= 0) {
        const int jn = j + NW;
        const int4 wn = jn < na ? a.S.work[jn] : make_int4(-1, 0, 0, 0);
        const bool pre = can_pre && wn.x >= 0;
        bool switched = false;
        const int s0 = wk.y, nt = wk.z - wk.y;        /* one slot per token of the expert: nt <= T */
        const uint8_t *cb = a.down + (size_t)wk.x * a.eb + (size_t)r0 * a.rb;    /* its rows (b may move on) */
        const uint8_t *xq = xbuf + (size_t)s0 * xrec;
        RowAcc acc[NT];
        for (int n = 0; n < NT; n++) acc[n] = RowAcc{ 0.0f, 0.0f, 0.0f };
        for (int c0 = 0; c0 < nchunk; c0 += D) {
#pragma unroll
            for (int d = 0; d < D; d++) {
                const int c = c0 + d;
                if (c < nchunk) {
                    wave_sync();
#pragma unroll
                    for (int m = 0; m < SPT; m++) {
                        const int i = min(lane + 64 * m, NSL - 1), row = i / SPR, q = i - row * SPR;
                        *(Unit *)(wbuf + row * WS + UNIT * q) = wv[d][m];
                    }
                    wave_sync();
                    if (c + D < nchunk) {
                        load_chunk(c + D, wv[d]);
                    } else if (pre && c + D - nchunk < nchunk) {
                        if (!switched) {                 /* every chunk of this expert is requested */
                            b = a.down + (size_t)wn.x * a.eb + (size_t)r0 * a.rb;
                            switched = true;
                        }
                        load_chunk(c + D - nchunk, wv[d]);
                    }
                    if constexpr (Q6) {
                        /* the super-block's offset in this quad's staged row (b: the expert
                         * whose rows this chunk holds) */
                        const uint32_t sbo = (uint32_t)((uintptr_t)(cb + (size_t)qd * a.rb + (size_t)c * 210) & 15);
                        /* the 8 blocks of super-block c (src/kernels.c:142-170) for every slot */
                        auto superblock = [&](auto al) {
#pragma unroll
                            for (int h = 0; h < 2; h++)
#pragma unroll
                                for (int g = 0; g < 4; g++) {
                                    const int blk = c * 8 + h * 4 + g;
                                    const Q6W w = q6_k_weights<decltype(al)::value>(wbuf + qd * WS, sbo, h, g, p);
#pragma unroll
                                    for (int n = 0; n < NT; n++)
                                        if (n < nt)
                                            q6_k_token(w, xq + (size_t)n * xrec + (size_t)(blk >> 1) * kPairBytes, p,
                                                       blk & 1, acc[n]);
                                }
                        };
                        if (c & 1) superblock(std::integral_constant<bool, false>());
                        else superblock(std::integral_constant<bool, true>());
                    } else {
                        q4_rows_nt<TYPE, NT>((const uint32_t *)(wbuf + qd * WS), p, xq, (size_t)xrec, c * (CB / 2),
                                             CB / 2, nt, acc);
                    }
                }
            }
        }
#pragma unroll
        for (int n = 0; n < NT; n++) {
            const float v = quad_finish(acc[n], finish_scale(TYPE));
            if (p == 0 && n < nt) {
                a.S.dn[(size_t)(s0 + n) * E + r0 + qd] = v;
                dnl[(s0 + n) * RD + qd] = v;
            }
        }
        j = jn;
        wk = wn;
        if (wk.x >= 0 && !pre) {
            b = a.down + (size_t)wk.x * a.eb + (size_t)r0 * a.rb;
#pragma unroll
            for (int d = 0; d < D; d++)
                if (d < nchunk) load_chunk(d, wv[d]);
        }
    }
    PHASE(2048, 2);
    __syncthreads();
    PHASE(2048, 3);
    for (int i = tid; i < T * RD; i += NTH) {
        const int t = i / RD, r = i - t * RD;
        float o = 0.0f;
        for (int jj = 0; jj < K; jj++)
            o = __builtin_fmaf(a.S.wt[t * K + jj], dnl[a.S.slot_of[t * K + jj] * RD + r], o);
        a.out[(size_t)t * E + r0 + r] = o;
    }
}

/* The int8 blocks of every slot's activations (src/model.c:996-997) for batches whose
 * records do not fit the down kernel's LDS: one thread per 32-block. */
__device__ bool mx_store_record(const Q8Vals &q, uint8_t *rec, bool hi16);

/* The int8 activation blocks of every slot (src/model.c:996-997) from act: QmsQ8 blocks, pair
 * records, and, when mxrec is set, the MFMA kernels' records too. */
__global__ void act_quant_kernel(Scratch S, int F, int NS, uint8_t *mxrec, int hi16)
{
    const int nbF = F >> 5;
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= NS * nbF) return;
    const int s = b / nbF, blk = b - s * nbF;
    float v[32];
    const float4 *src = (const float4 *)(S.act + (size_t)s * F + (size_t)blk * 32);
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const float4 f = src[j];
        v[4 * j] = f.x; v[4 * j + 1] = f.y; v[4 * j + 2] = f.z; v[4 * j + 3] = f.w;
    }
    const Q8Vals q = quantize_block(v);
    store_q8(q, S.aq + b);
    store_pair_half(q, (uint32_t *)(S.aqk + ((size_t)s * (nbF >> 1) + (blk >> 1)) * kPairBytes), blk & 1);
    if (mxrec && !mx_store_record(q, mxrec + (size_t)b * kMxRec, hi16)) S.mxflag[1] = S.epoch;
}

/* Weighted sum per token in selection order (src/model.c:1152-1162) when dn did not fit. */
/* Threads per combine block: 4 x threads divides n_embd (a multiple of 256), so a block never
 * straddles two tokens. */
static inline int combine_threads(int E) { return (E / 4) % 256 == 0 ? 256 : ((E / 4) % 128 == 0 ? 128 : 64); }

__global__ void combine_kernel(const Scratch S, int E, int K, int T, float *out)
{
    /* four output elements per thread, 16-byte reads of the dn rows; n_embd is a multiple of
     * 4 x the block size (combine_threads), so the token is block-uniform and its weights and
     * slots are scalar loads. Each element's sum runs over j in order (src/model.c:1152-1162). */
    const int i4 = blockIdx.x * blockDim.x + threadIdx.x;
    if (i4 * 4 >= T * E) return;
    const int t = (int)(blockIdx.x * blockDim.x * 4) / E, r = 4 * i4 - t * E;
    float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int j = 0; j < K; j++) {
        const float w = S.wt[(size_t)t * K + j];
        const float4 d = *(const float4 *)(S.dn + (size_t)S.slot_of[(size_t)t * K + j] * E + r);
        o.x = __builtin_fmaf(w, d.x, o.x);
        o.y = __builtin_fmaf(w, d.y, o.y);
        o.z = __builtin_fmaf(w, d.z, o.z);
        o.w = __builtin_fmaf(w, d.w, o.w);
    }
    /* out need only be 4-byte aligned */
    float *dst = out + 4 * (size_t)i4;
    dst[0] = o.x;
    dst[1] = o.y;
    dst[2] = o.z;
    dst[3] = o.w;
}

template <int TYPE, int RT, int QA>
static void launch_down_tile(const TileArgs &a, int NT, dim3 grid, size_t lds, hipStream_t st)
{
    if (NT == 4) QLAUNCH("down", (tile_rows_kernel<TYPE, 4, RT, 0, QA>), grid, dim3(4 * RT), lds, st, a);
    else if (NT == 2) QLAUNCH("down", (tile_rows_kernel<TYPE, 2, RT, 0, QA>), grid, dim3(4 * RT), lds, st, a);
    else QLAUNCH("down", (tile_rows_kernel<TYPE, 1, RT, 0, QA>), grid, dim3(4 * RT), lds, st, a);
}

/* Batches up to this many tokens form the activation records inside the down tiles (each of
 * a tile's row blocks quantises the tile's slots again) instead of in a separate launch. */
constexpr int kTileQuantT = 8;

/* Rows per block of the Q6_K slot-tile kernel (its 210-byte super-blocks make a 64-row tile
 * 81 KB of LDS for n_ff_exp 1536, one block per CU). */
constexpr int kDownTileRowsQ6K = 32;

/* Output rows per block of the one-token down kernel (8: 512 blocks of 4 waves for E = 4096;
 * 16: 256 blocks of 8 waves, half the activation reads). */
constexpr int kDownT1Rows = 16;

#ifndef QMSG_DOWN_SMALL_D
#define QMSG_DOWN_SMALL_D 3
#endif
bool down_small_fits(const Shape &s, const LayerDev &L, int T)
{
    constexpr int RD = kDownT1Rows, CB = 8;
    const int bb = L.down_type == 3 ? 20 : 18;
    const size_t xrec = (size_t)(s.F / 64) * kPairBytes;
    const size_t ws = L.down_type == 14 ? 240 : (size_t)CB * bb + (((CB * bb / 16) & 1) ? 0 : 16);
    const size_t lds_s = (size_t)(RD / 2) * 16 * ws + (size_t)T * s.K * (xrec + RD * 4);
    const bool t1_type = L.down_type == 2 || L.down_type == 3 || (L.down_type == 14 && L.down_rb % 4 == 0);
    return T >= 2 && T <= 4 && T * s.K <= kSmallDownNS && t1_type && s.F % 256 == 0 && s.E % RD == 0 &&
           lds_s <= 160 * 1024;
}

/* LDS bytes of the one-token down kernel, and of the slot-tile down kernel at NT slots per pass. */
static size_t down_t1_lds(const Shape &s, const LayerDev &L)
{
    constexpr int RD = kDownT1Rows, CB = 8;
    const int bb = L.down_type == 3 ? 20 : 18;
    const size_t xrec = (size_t)(s.F / 64) * kPairBytes;
    const size_t ws = L.down_type == 14 ? 240 : (size_t)CB * bb + (((CB * bb / 16) & 1) ? 0 : 16);
    return (size_t)(RD / 2) * 16 * ws + (size_t)s.K * xrec + (size_t)s.K * RD * 4;
}

static size_t down_tile_lds(const Shape &s, const LayerDev &L, int T)
{
    const size_t xrec = (size_t)(s.F / 64) * kPairBytes;
    const int NT = T >= 4 ? 4 : (T >= 2 ? 2 : 1);
    const int RT = L.down_type == 14 ? kDownTileRowsQ6K : 64;
    return ((RT * L.down_rb + 15) & ~(size_t)15) + (size_t)NT * xrec;
}

bool down_exact_fits(const Shape &s, const LayerDev &L, int T)
{
    const bool t1_type = L.down_type == 2 || L.down_type == 3 || (L.down_type == 14 && L.down_rb % 4 == 0);
    if (T == 1 && s.K <= 8 && t1_type && s.F % 256 == 0 && s.E % kDownT1Rows == 0 && down_t1_lds(s, L) <= 160 * 1024)
        return true;
    if (down_small_fits(s, L, T)) return true;
    const int RT = L.down_type == 14 ? kDownTileRowsQ6K : 64;
    return down_tile_lds(s, L, T) <= 160 * 1024 && s.E % RT == 0;
}

hipError_t launch_down_exact(const Shape &s, const LayerDev &L, const Scratch &S, float *out, int T, int quant,
                             hipStream_t st)
{
    DownArgs a;
    a.down = L.down;
    a.rb = L.down_rb;
    a.eb = L.down_eb;
    a.E = s.E;
    a.F = s.F;
    a.K = s.K;
    a.T = T;
    a.X = s.X;
    a.out = out;
    a.quant = quant;
    a.S = S;
    /* one token: each wave streams its own experts' rows (Q4_0 / Q4_1); RD output rows per
     * block, RD/2 waves */
    /* chunks of 8 blocks, three in flight per wave: measured faster than 16-block chunks two
     * in flight (10.7 vs 11.4 us for the 235B shape) and than deeper pipelines */
    constexpr int RD = kDownT1Rows, CB = 8;
    const int bb = L.down_type == 3 ? 20 : 18;
    const size_t xrec = (size_t)(s.F / 64) * kPairBytes;
    const size_t ws = L.down_type == 14 ? 240 : (size_t)CB * bb + (((CB * bb / 16) & 1) ? 0 : 16);
    const size_t lds_t1 = down_t1_lds(s, L);
    const bool t1_type = L.down_type == 2 || L.down_type == 3 || (L.down_type == 14 && L.down_rb % 4 == 0);
    if (T == 1 && s.K <= 8 && t1_type && s.F % 256 == 0 && s.E % RD == 0 && lds_t1 <= 160 * 1024) {
        const dim3 grid(s.E / RD), block(32 * RD);
        if (L.down_type == 14) QLAUNCH("down", (down_t1_kernel<14, CB, 3, RD>), grid, block, lds_t1, st, a);
        else if (L.down_type == 3) QLAUNCH("down", (down_t1_kernel<3, CB, 3, RD>), grid, block, lds_t1, st, a);
        else QLAUNCH("down", (down_t1_kernel<2, CB, 3, RD>), grid, block, lds_t1, st, a);
        return hipGetLastError();
    }
    /* two to four tokens: the same layout, each wave streaming several experts (the
     * activations' records formed in the kernel, or read from aqk) */
    if (down_small_fits(s, L, T)) {
        const size_t lds_s = (size_t)(RD / 2) * 16 * ws + (size_t)T * s.K * (xrec + RD * 4);
        const dim3 grid(s.E / RD), block(32 * RD);
        if (L.down_type == 14) QLAUNCH("down", (down_small_kernel<14, CB, 3, RD>), grid, block, lds_s, st, a);
        else if (L.down_type == 3) QLAUNCH("down", (down_small_kernel<3, CB, QMSG_DOWN_SMALL_D, RD>), grid, block, lds_s, st, a);
        else QLAUNCH("down", (down_small_kernel<2, CB, QMSG_DOWN_SMALL_D, RD>), grid, block, lds_s, st, a);
        return hipGetLastError();
    }
    /* slot tiles: the activations' int8 records first (unless the MFMA gate/up wrote them) */
    const int NS = T * s.K, maxt = (s.X < NS ? s.X : NS) + NS / kTileN + 1;
    const bool qa = quant && T <= kTileQuantT;
    if (quant && !qa) {
        const int nq = NS * (s.F / 32);
        QLAUNCH("actq", act_quant_kernel, dim3((nq + 255) / 256), dim3(256), 0, st, S, s.F, NS, (uint8_t *)nullptr, 0);
    }
    const int NT = T >= 4 ? 4 : (T >= 2 ? 2 : 1);
    const int RT = L.down_type == 14 ? kDownTileRowsQ6K : 64;
    const size_t lds = down_tile_lds(s, L, T);
    if (lds > 160 * 1024 || s.E % RT) return hipErrorInvalidValue;
    const dim3 grid(s.E / RT, maxt);
    TileArgs ta;
    ta.w = L.down;
    ta.rb = L.down_rb;
    ta.eb = L.down_eb;
    ta.cols = s.F;
    ta.rec = S.aqk;
    ta.y = S.dn;
    ta.y_stride = s.E;
    ta.y_off = 0;
    ta.S = S;
    if (qa) {
        if (L.down_type == 2) launch_down_tile<2, 64, 1>(ta, NT, grid, lds, st);
        else if (L.down_type == 3) launch_down_tile<3, 64, 1>(ta, NT, grid, lds, st);
        else launch_down_tile<14, kDownTileRowsQ6K, 1>(ta, NT, grid, lds, st);
    } else {
        if (L.down_type == 2) launch_down_tile<2, 64, 0>(ta, NT, grid, lds, st);
        else if (L.down_type == 3) launch_down_tile<3, 64, 0>(ta, NT, grid, lds, st);
        else launch_down_tile<14, kDownTileRowsQ6K, 0>(ta, NT, grid, lds, st);
    }
    const int n = T * s.E;
    QLAUNCH("combine", combine_kernel, dim3(n / (4 * combine_threads(s.E))), dim3(combine_threads(s.E)), 0, st, S, s.E, s.K, T, out);
    return hipGetLastError();
}

/* a = silu(g) * u per slot (src/model.c:994; in --exact mode 1024), fp32. */
__global__ void swiglu_kernel(Scratch S, int F, int NS)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= NS * F) return;
    const int s = i / F, j = i - s * F;
    S.act[i] = silu_ref(S.gu[(size_t)s * 2 * F + j]) * S.gu[(size_t)s * 2 * F + F + j];
}

/* Gate and up rows of any of Q4_0 / Q4_1 / Q6_K (the reference's fast path takes each,
 * src/kernels.c:197-200; src/model.c:979-988) by slot tiles against the tokens' int8 input
 * records, then a = silu(g) * u. Layers whose gate and up are both Q4_0 take gateup_kernel. */
template <int TYPE, int RT>
static void launch_gu_tile(const TileArgs &a, dim3 grid, size_t lds, hipStream_t st)
{
    QLAUNCH("gateup", (tile_rows_kernel<TYPE, 4, RT, 1>), grid, dim3(4 * RT), lds, st, a);
}

hipError_t launch_gateup_tiles(const Shape &s, const LayerDev &L, const Scratch &S, int T, hipStream_t st)
{
    const int NS = T * s.K, maxt = (s.X < NS ? s.X : NS) + NS / kTileN + 1;
    const size_t xrec = (size_t)(s.E / 64) * kPairBytes;
    for (int i = 0; i < 2; i++) {
        TileArgs a;
        a.w = i ? L.up : L.gate;
        a.rb = i ? L.up_rb : L.gate_rb;
        a.eb = i ? L.up_eb : L.gate_eb;
        a.cols = s.E;
        a.rec = S.xqk;
        a.y = S.gu;
        a.y_stride = 2 * s.F;
        a.y_off = i ? s.F : 0;
        a.S = S;
        const int type = i ? L.up_type : L.gate_type;
        /* 32 rows per block where they fit in LDS with four slots' records, else 16 */
        int RT = 32;
        if (((RT * a.rb + 15) & ~(uint64_t)15) + 4 * xrec > 160 * 1024) RT = 16;
        const size_t lds = ((RT * a.rb + 15) & ~(size_t)15) + 4 * xrec;
        if (lds > 160 * 1024 || s.F % RT) return hipErrorInvalidValue;
        const dim3 grid(s.F / RT, maxt);
        if (type == 2) RT == 32 ? launch_gu_tile<2, 32>(a, grid, lds, st) : launch_gu_tile<2, 16>(a, grid, lds, st);
        else if (type == 3) RT == 32 ? launch_gu_tile<3, 32>(a, grid, lds, st) : launch_gu_tile<3, 16>(a, grid, lds, st);
        else RT == 32 ? launch_gu_tile<14, 32>(a, grid, lds, st) : launch_gu_tile<14, 16>(a, grid, lds, st);
    }
    const int n = NS * s.F;
    QLAUNCH("swiglu", swiglu_kernel, dim3((n + 255) / 256), dim3(256), 0, st, S, s.F, NS);
    return hipGetLastError();
}

/* ------------------------------------------------------------------ MFMA expert products ---- */

/* Batches with several slots per expert: the expert products on the matrix cores, order-exact.
 *
 * For a weight row, a slot's int8 block x and a 32-block b, the reference's AVX2 dot forms
 * eight int32 lane sums S_k = sum_{i in 4k..4k+3} u_i x_i (u the unsigned weight code, lanes
 * 0-3 over the low nibbles) and folds each into its own fp32 chain
 * acc_k = fma((float)S_k, fl(d_w d_x), acc_k) (src/kernels.c:85-94, 113-119, 145-166). One
 * v_mfma_f32_16x16x32_f16 returns those eight S_k, scaled by 2^-24, for 16 weight rows and 2
 * slots:
 *   - B holds the codes of 16 rows as f16 subnormals: the bits of code u are the f16 u 2^-24,
 *     so a mask unpacks them (the matrix cores keep subnormal inputs; checked on the device);
 *   - A is block-diagonal over the lane groups: its row (slot j, lane k) holds x_j only at the
 *     four K positions of group k, so D-row (j, k) of column r sums group k only.
 * Every product and partial sum is an integer multiple of 2^-24 below 1, so the f32
 * accumulation inside the MFMA is exact in any order and D equals S_k 2^-24. The VALU then runs
 * the reference's chains, acc_k = fma(S_k, fl(d_w d_x), acc_k) per block, as
 * fma(D, fl(d_w d_x 2^24), acc_k): the record carries d_x 2^24, and for d_x in [2^-102, 2^88]
 * (or 0) fl(d_w d_x 2^24) = fl(d_w d_x) 2^24 for every f16 d_w (no subnormal or overflowing
 * product), so the FMA sees the reference's exact product. A chunk with a d_x outside that
 * range (the record's scaled word is then a NaN) runs fma(D 2^24, fl(d_w d_x), acc_k) instead.
 * Then the offset chain, and at the end the hsum256 tree and the unfused final term. Q6_K
 * multiplies D by its int8 sub-scale times 2^24 first (exact), which needs no range.
 *
 * Operand layout of the 16x16x32 f16 MFMA (checked on the device): lane l supplies
 * A[l%16][8(l/16) + e] and B[8(l/16) + e][l%16] for e = 0..7 and receives D[4(l/16) + v][l%16].
 * K position 8g + e of lane group g is block element pi(8g + e) =
 * 4g, 4g+2, 4g+1, 4g+3, 16+4g, 16+4g+2, 16+4g+1, 16+4g+3: the first four are reference lane
 * k = g, the last four lane k = g + 4, and both come from one code dword (Q4) of the block
 * with one shift and four masks: the high nibbles stay in place as 16 x code, against x / 16
 * in the records' lanes 4-7 (the product is the same). D-row 4(l/16) + v is slot j = l/32 of the pair and lane
 * k = 4((l/16)&1) + v, so a lane holds four chains of one (row, slot): one fl(d_w d_x) product
 * serves its four FMAs.
 *
 * Activation records (kMxRec bytes per slot, or per token, and 32-block) carry x in that
 * order as f16 (64 bytes; for Q4 rows lanes 4-7 hold x / 16), then d 2^24 (or the NaN that sends the chunk to the unscaled
 * chains), ds, the half sums and d (16 bytes), then 16 zero bytes, which the lanes of A
 * outside their group read; the kernels stage those first 96 bytes of each record. Gate/up
 * writes the records of the activations it quantises, so the down products read them
 * directly.
 *
 * A block of 8 waves computes 512/WSG weight rows x 8*WSG slots of one expert's slot tile:
 * wave (wr, ws) owns 64 rows (four 16-row MFMA tiles) and 8 slots (four pairs). For gate/up the
 * 64 rows are 32 gate rows and the same 32 up rows, so SwiGLU and the int8 requantisation of
 * whole 32-blocks happen in the block. K is staged through LDS in chunks of kMxC blocks,
 * double-buffered: the next chunk's loads are in flight while the current one computes. */
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short short2_t __attribute__((ext_vector_type(2)));

constexpr int kMxC = 8;          /* 32-blocks per staged chunk (one Q6_K super-block) */
constexpr int kMxNA = 8;         /* accumulator tiles per 16-row tile: 4 pairs, or 4 quads x 2 halves */
constexpr int kMxDx = 64;        /* offset of the record's d 2^24, ds, half sums, d */
constexpr int kMxZero = 80;      /* offset of the record's zero words */
static_assert(kMxRec == 128, "record layout: 64 bytes of codes, 16 of scales, 16 of zeros (32 unused)");
/* bytes of one record in LDS */
__host__ __device__ constexpr int mx_recl(int) { return 96; }

/* d 2^24 where fl(d_w d 2^24) = fl(d_w d) 2^24 for every f16 d_w, else a NaN. */
__device__ __forceinline__ float mx_scaled_d(float d)
{
    const bool ok = d == 0.0f || (d >= 0x1p-102f && d <= 0x1p88f);
    return ok ? d * 0x1p24f : __builtin_nanf("");
}

/* One int8 block as an activation record (layout above); false when its d_x 2^24 word is the
 * NaN (d_x outside the scaled range). hi16: for Q4_0 / Q4_1 rows, whose B operand takes the
 * high nibbles in place (code 16 2^-24), lanes 4-7 carry x / 16 (exact in f16). */
__device__ bool mx_store_record(const Q8Vals &q, uint8_t *rec, bool hi16)
{
    u32x4 w[6];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t c = q.qw[k];
        const int x0 = (int)(int8_t)(c & 0xffu), x1 = (int)(int8_t)((c >> 8) & 0xffu);
        const int x2 = (int)(int8_t)((c >> 16) & 0xffu), x3 = (int)(int8_t)(c >> 24);
        const float sc = (hi16 && k >= 4) ? 0.0625f : 1.0f;
        auto h = [sc](int x) { return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)((float)x * sc)); };
        w[k >> 1][2 * (k & 1)] = h(x0) | (h(x2) << 16);
        w[k >> 1][2 * (k & 1) + 1] = h(x1) | (h(x3) << 16);
    }
    const float dsc = mx_scaled_d(q.d);
    w[4] = u32x4{ __float_as_uint(dsc), __float_as_uint(q.ds), q.s16, __float_as_uint(q.d) };
    w[5] = u32x4{ 0u, 0u, 0u, 0u };
#pragma unroll
    for (int i = 0; i < 6; i++) ((u32x4 *)rec)[i] = w[i];
    return dsc == dsc;
}

/* The layer input's records from its int8 blocks (one thread per block). */
__global__ void mx_input_kernel(const Q8 *xq, int n, uint8_t *rec, uint64_t *flag, uint64_t epoch, int hi16)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint32_t *s = (const uint32_t *)(xq + i);
    Q8Vals q;
    q.d = __uint_as_float(s[0]);
    q.ds = __uint_as_float(s[1]);
    q.s16 = s[2];
#pragma unroll
    for (int w = 0; w < 8; w++) q.qw[w] = s[3 + w];
    if (!mx_store_record(q, rec + (size_t)i * kMxRec, hi16)) *flag = epoch;
}

struct MxArgs {
    const uint8_t *w0, *w1;      /* gate and up (gate/up kernel); down (down kernel) */
    uint64_t rb, eb;
    int E, F, debug;
    const uint8_t *rec;          /* input records: [token][E/32] (gate/up) or [slot][F/32] (down) */
    uint8_t *rec_out;            /* gate/up: the activation records [slot][F/32] */
    int rec_out_hi16;            /* gate/up: the down rows are Q4_0 / Q4_1 (records' lanes 4-7 x / 16) */
    Scratch S;
};

/* LDS bytes of one staged weight row (kMxC blocks): Q4_0 144, Q4_1 160, Q6_K one super-block
 * copied from the 4-byte boundary below it (216 bytes, 54 words). */
__host__ __device__ constexpr int mx_wstride(int type) { return type == 14 ? 216 : (type == 3 ? 160 : 144); }

/* Staged chunk layout of a block of 8 waves: (8/WSG) row groups of 32 weight rows, WSG slot
 * groups of 8 slots; the weight rows, then each slot's kMxC records at a stride of
 * mx_rstride bytes: 64 bytes past the records for Q6_K (two 80 KB blocks fill a CU's LDS), 320
 * for the Q4 types, so that two pairs' records lie more than 2040 bytes apart and every A read
 * stays a single read straight into the MFMA operand (closer records get merged into paired
 * reads plus register moves); either way the two slots of a pair sit 16 LDS banks apart. Every
 * piece is copied by the LDS DMA (global_load_lds): a wave instruction moves 64 lanes x 16 bytes
 * (Q6_K weights: x 4 bytes) to consecutive LDS bytes. Two buffers: the next chunk's copy is in
 * flight while the current one computes. */
#ifndef QMSG_MX_RPAD
#define QMSG_MX_RPAD 32
#endif
__host__ __device__ constexpr int mx_rstride(int type) { return kMxC * mx_recl(type) + QMSG_MX_RPAD; }

template <int TYPE, int WSG, int PPW = 4, int NW = 8, int NT = 2>
struct MxLayout {
    static constexpr int RWG = 16 * NT * NW / WSG, SWG = 2 * PPW * WSG, WS = mx_wstride(TYPE);
    static constexpr int RS = mx_rstride(TYPE);
    static constexpr int WBYTES = RWG * WS, BUF = WBYTES + SWG * RS;
    static constexpr int WUNIT = TYPE == 14 ? 4 : 16;                 /* bytes per lane per DMA   */
    static constexpr int WUR = WS / WUNIT;                             /* DMA units per row        */
    static constexpr int WINSTR = (RWG * WUR + 63) / 64;               /* weight DMA instructions  */
};

/* nb: staging buffers, 1 or 2 of weights and records; 3: two of weights, one of records. */
__host__ __device__ constexpr int mx_lds_bytes(int type, int wsg, int ppw = 4, int nw = 8, int nb = 2, int nt = 2)
{
    return nb == 3 ? 2 * ((16 * nt * nw / wsg) * mx_wstride(type)) + 2 * ppw * wsg * mx_rstride(type)
                   : nb * ((16 * nt * nw / wsg) * mx_wstride(type) + 2 * ppw * wsg * mx_rstride(type));
}

/* (x & m) | c in one instruction; m and c in registers (no literal operands in VOP3 here). */
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m, uint32_t c)
{
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(m), "v"(c));
    return r;
}

/* The B operand of one 16-row tile for 32-block b of the staged chunk (row = this lane's row in
 * LDS) and the scale words the chains need. */
struct MxB {
    f16x8 op;
    uint32_t dw;      /* Q4_0: d (low half); Q4_1: d | m << 16; Q6_K: d (low half) */
    float sc;         /* Q6_K: the lane's sub-scale times 2^24 (k < 4: sc[2g], k >= 4: sc[2g+1]) */
    uint32_t sab;     /* Q6_K: both sub-scales as int16 pair (sc[2g] low) */
    float sc1;        /* Q6_K: sc[2g+1] times 2^24 */
};

/* a.lo*b.lo + a.hi*b.hi over int16 halves (v_dot2_i32_i16 with a zero addend: no register to
 * clear first, as the accumulating form needs). */
__device__ __forceinline__ int sdot2_i16(uint32_t a, uint32_t b)
{
    int r;
    asm("v_dot2_i32_i16 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

typedef __attribute__((address_space(3))) const uint8_t *LdsPtr;
typedef __attribute__((address_space(3))) const u32x2 LdsU32x2;
typedef __attribute__((address_space(3))) const u32x4 LdsU32x4;

/* The B operand of one 16-row tile for a Q4_0 / Q4_1 block of the staged chunk, and its scale
 * word, from two LDS pointers: pq at the lane's code word of the block in tile row lr (Q4_0
 * even blocks: 2 bytes past a word boundary), pd at the block's scale word; tile t is an
 * immediate offset. */
template <int TYPE, int PAR, bool SC, int TS = 16>
__device__ __forceinline__ MxB mx_weights_q4(LdsPtr pq, LdsPtr pd, int t)
{
    constexpr int WS = mx_wstride(TYPE);
    const uint32_t m4 = 0x000f000fu;
    MxB w;
    uint32_t v;
    if constexpr (TYPE == 3 || PAR) {
        v = *(const __attribute__((address_space(3))) uint32_t *)(pq + TS * t * WS);
    } else {
        const uint32_t a0 = *(const __attribute__((address_space(3))) uint32_t *)(pq + TS * t * WS - 2);
        const uint32_t a1 = *(const __attribute__((address_space(3))) uint32_t *)(pq + TS * t * WS + 2);
        v = __builtin_amdgcn_alignbyte(a1, a0, 2);
    }
    /* the high nibbles stay in place, as 16 x code (the records' lanes 4-7 carry x / 16) */
    const uint32_t mh = 0x00f000f0u, v8 = v >> 8;
    if constexpr (SC) {
        /* the f16 subnormals code 2^-24 (high nibbles 16 code 2^-24) */
        w.op = __builtin_bit_cast(f16x8, u32x4{ v & m4, v8 & m4, v & mh, v8 & mh });
    } else {
        /* the codes themselves: f16 1024 + c (0x6400 | c) minus 1024, exact */
        const uint32_t bias = 0x64006400u;
        typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
        const f16x2 k = { (_Float16)1024.0f, (_Float16)1024.0f };
        const f16x2 c0 = __builtin_bit_cast(f16x2, and_or(v, m4, bias)) - k;
        const f16x2 c1 = __builtin_bit_cast(f16x2, and_or(v8, m4, bias)) - k;
        const f16x2 c2 = __builtin_bit_cast(f16x2, and_or(v, mh, bias)) - k;
        const f16x2 c3 = __builtin_bit_cast(f16x2, and_or(v8, mh, bias)) - k;
        w.op = f16x8{ c0.x, c0.y, c1.x, c1.y, c2.x, c2.y, c3.x, c3.y };
    }
    if constexpr (TYPE == 3) w.dw = *(const __attribute__((address_space(3))) uint32_t *)(pd + TS * t * WS);
    else w.dw = *(const __attribute__((address_space(3))) uint16_t *)(pd + TS * t * WS);
    w.sc = 0.0f;
    w.sab = 0u;
    w.sc1 = 0.0f;
    return w;
}

/* fl(h * f) for the f16 in the low half of h (v_fma_mix, one rounding; the added zero cannot
 * change a non-zero product). */
__device__ __forceinline__ float mix_mul(uint32_t h, float f)
{
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(f));
    return r;
}

/* fma(f16 low half of h, f, c) in one rounding. */
__device__ __forceinline__ float mix_fma_lo(uint32_t h, float f, float c)
{
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(f), "v"(c));
    return r;
}

/* fma(f16 high half of h, f, c) in one rounding. */
__device__ __forceinline__ float mix_fma_hi(uint32_t h, float f, float c)
{
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(f), "v"(c));
    return r;
}

/* One block b (parity PAR) of the staged chunk: NP slot pairs of this wave against its two
 * 16-row tiles. */
/* A lane's LDS read streams over a staged chunk, each one register: A low and high words and
 * the slot's d/ds words (at the trip's first block; the pair p adds 2p record strides), and for
 * Q4_0 / Q4_1 the code word and the scale word of tile row lr (the tile t adds 16t rows). One
 * trip covers two blocks; the second block and the pairs and tiles are immediate offsets. */
struct MxStreams {
    LdsPtr alo, ahi, d, q, dw;
};

/* The empty asm keeps each stream a single register: otherwise every (pair, stream) address
 * becomes a loop variable of its own and the registers run out. */
__device__ __forceinline__ void mx_opaque(MxStreams &st)
{
    asm("" : "+v"(st.alo), "+v"(st.ahi), "+v"(st.d), "+v"(st.q), "+v"(st.dw));
}

/* One block b (parity PAR within the trip) of the staged chunk: NP slot pairs of this wave
 * against its two 16-row tiles. SC: the chunk's records all carry d_x 2^24 and B holds the
 * codes 2^-24; else B holds the codes themselves and the chains take d_x unscaled. */
template <int TYPE, int NP, int PAR, bool SC, int TS>
__device__ __forceinline__ void mx_block(const MxStreams &st, bool kh, f32x4 (&acc)[2][kMxNA], float (&cr)[2][4])
{
    static_assert(TYPE == 2 || TYPE == 3, "Q6_K chunks take mx_chunk_q6");
    constexpr int BB = TYPE == 3 ? 20 : 18, RB = PAR * mx_recl(TYPE), RS = mx_rstride(TYPE);
    MxB w[2];
#pragma unroll
    for (int t = 0; t < 2; t++) w[t] = mx_weights_q4<TYPE, PAR, SC, TS>(st.q + PAR * BB, st.dw + PAR * BB, t);
    /* the two lanes of a (row, slot) share its offset chain: the k-half-0 lane runs tile 0's,
     * the other tile 1's (cr[0][p]; the epilogue fetches the partner's) */
    const uint32_t dwc = kh ? w[1].dw : w[0].dw;
    /* pair p's two MFMAs are issued before pair p-1's results are used, so the chains of one
     * pair run while the matrix core works on the next */
    f32x4 S[2][2];
    float xd[2], xds[2];
    auto issue = [&](int p, int k) {
        const u32x2 lo = *(const LdsU32x2 *)(st.alo + RB + 2 * p * RS);
        const u32x2 hi = *(const LdsU32x2 *)(st.ahi + RB + 2 * p * RS);
        if constexpr (SC) {
            const u32x2 d2 = *(const LdsU32x2 *)(st.d + RB + 2 * p * RS);      /* d 2^24, ds */
            xd[k] = __uint_as_float(d2.x);
            xds[k] = __uint_as_float(d2.y);
        } else {
            typedef __attribute__((address_space(3))) const float LdsF32;
            xd[k] = *(LdsF32 *)(st.d + RB + 2 * p * RS + 12);                     /* d */
            xds[k] = *(LdsF32 *)(st.d + RB + 2 * p * RS + 4);                     /* ds */
        }
        const f16x8 aop = __builtin_bit_cast(f16x8, u32x4{ lo.x, lo.y, hi.x, hi.y });
#pragma unroll
        for (int t = 0; t < 2; t++)
            S[k][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, w[t].op, f32x4{ 0.0f, 0.0f, 0.0f, 0.0f }, 0, 0, 0);
    };
    issue(0, 0);
#pragma unroll
    for (int p = 0; p < NP; p++) {
        const int k = p & 1;
        if (p + 1 < NP) issue(p + 1, k ^ 1);
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const float dd = mix_mul(w[t].dw, xd[k]);
#pragma unroll
            for (int v = 0; v < 4; v++)
                acc[t][p][v] = __builtin_fmaf(S[k][t][v], dd, acc[t][p][v]);
        }
        if constexpr (TYPE == 3) cr[0][p] = mix_fma_hi(dwc, xds[k], cr[0][p]);   /* off += m*ds */
        else cr[0][p] = mix_fma_lo(dwc, xds[k], cr[0][p]);                     /* corr += d*ds */
    }
}

/* One staged chunk (kMxC blocks), two blocks per loop trip. A lane's A words are its x words
 * where it holds x, else the record's zero words. */
template <int TYPE, int NP, bool SC, int TS>
__device__ __forceinline__ void mx_chunk(const uint8_t *W, const uint8_t *R, int lr, int lg, int jd, bool kh,
                                         int offa_lo, int offa_hi, f32x4 (&acc)[2][kMxNA], float (&cr)[2][4])
{
    constexpr int WS = mx_wstride(TYPE), BB = TYPE == 3 ? 20 : 18, QO = TYPE == 3 ? 4 : 2;
    MxStreams st;
    st.alo = (LdsPtr)(R + offa_lo);
    st.ahi = (LdsPtr)(R + offa_hi);
    st.d = (LdsPtr)(R + jd * mx_rstride(TYPE) + kMxDx);
    st.q = (LdsPtr)(W + lr * WS + QO + 4 * lg);
    st.dw = (LdsPtr)(W + lr * WS);
#pragma unroll 1
    for (int b = 0; b < kMxC; b += 2) {
        mx_opaque(st);
        mx_block<TYPE, NP, 0, SC, TS>(st, kh, acc, cr);
        __builtin_amdgcn_sched_barrier(0);      /* one block's operands in registers at a time */
        mx_block<TYPE, NP, 1, SC, TS>(st, kh, acc, cr);
        st.alo += 2 * mx_recl(TYPE);
        st.ahi += 2 * mx_recl(TYPE);
        st.d += 2 * mx_recl(TYPE);
        st.q += 2 * BB;
        st.dw += 2 * BB;
    }
}

/* Q4_0 / Q4_1 lane sums on v_mfma_f32_16x16x16_f16, four slots per instruction. A row i of an
 * instruction is (slot i / 4 of the quad, reference lane ka = i % 4 + 4h) for half h of the
 * 32-block (h = 0: the low nibbles, reference lanes 0-3; h = 1: the high nibbles, lanes 4-7);
 * K group lg of a lane holds reference lane lg + 4h, so A row i is non-zero only in the lane
 * with lg == i % 4, and every other lane reads the records' zero words at one shared address.
 * The lane (row lr, K group lg) of the result holds all eight chains of (tile row lr, slot
 * 4q + lg): the two halves' four values each. One d_w d_x product and one offset-chain step per
 * (tile, quad, block) serve both halves. */
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

template <int TYPE, int NQ, int BI, bool SC, int NT, int TS>
__device__ __forceinline__ void mx_block16(const MxStreams &st, f32x4 (&acc)[2][kMxNA], float (&cr)[2][4])
{
    static_assert(TYPE == 2 || TYPE == 3, "Q4_0 / Q4_1 rows");
    /* block BI of the staged chunk: every stream offset an immediate */
    constexpr int BB = TYPE == 3 ? 20 : 18, RB = BI * mx_recl(TYPE), RS = mx_rstride(TYPE), PAR = BI & 1;
    MxB w[2];
    f16x4 b[2][2];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        w[t] = mx_weights_q4<TYPE, PAR, SC, TS>(st.q + BI * BB, st.dw + BI * BB, t);
        b[t][0] = __builtin_shufflevector(w[t].op, w[t].op, 0, 1, 2, 3);
        b[t][1] = __builtin_shufflevector(w[t].op, w[t].op, 4, 5, 6, 7);
    }
    /* unit u = (quad u / 2, half u % 2); unit u + 1's two MFMAs are issued before unit u's
     * results are used */
    f32x4 S[2][2];
    float xd[NQ], xds[NQ], dd[2];
    auto issue = [&](int u, int k) {
        const int q = u >> 1, h = u & 1;
        const u32x2 av = *(const LdsU32x2 *)((h ? st.ahi : st.alo) + RB + 4 * q * RS);
        if (h == 0) {
            if constexpr (SC) {
                const u32x2 d2 = *(const LdsU32x2 *)(st.d + RB + 4 * q * RS);      /* d 2^24, ds */
                xd[q] = __uint_as_float(d2.x);
                xds[q] = __uint_as_float(d2.y);
            } else {
                typedef __attribute__((address_space(3))) const float LdsF32;
                xd[q] = *(LdsF32 *)(st.d + RB + 4 * q * RS + 12);                   /* d */
                xds[q] = *(LdsF32 *)(st.d + RB + 4 * q * RS + 4);                   /* ds */
            }
        }
        const f16x4 aop = __builtin_bit_cast(f16x4, av);
#pragma unroll
        for (int t = 0; t < NT; t++)
            S[k][t] = __builtin_amdgcn_mfma_f32_16x16x16f16(aop, b[t][h], f32x4{ 0.0f, 0.0f, 0.0f, 0.0f }, 0, 0, 0);
    };
    issue(0, 0);
#pragma unroll
    for (int u = 0; u < 2 * NQ; u++) {
        const int k = u & 1, q = u >> 1, h = u & 1;
        if (u + 1 < 2 * NQ) issue(u + 1, k ^ 1);
        if (h == 0) {
#pragma unroll
            for (int t = 0; t < NT; t++) dd[t] = mix_mul(w[t].dw, xd[q]);
        }
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int v = 0; v < 4; v++)
                acc[t][2 * q + h][v] = __builtin_fmaf(S[k][t][v], dd[t], acc[t][2 * q + h][v]);
        if (h == 1) {
#pragma unroll
            for (int t = 0; t < NT; t++) {
                if constexpr (TYPE == 3) cr[t][q] = mix_fma_hi(w[t].dw, xds[q], cr[t][q]);   /* off += m*ds */
                else cr[t][q] = mix_fma_lo(w[t].dw, xds[q], cr[t][q]);                     /* corr += d*ds */
            }
        }
    }
}

/* One staged chunk on the 16x16x16 instructions, its 8 blocks unrolled; offa_lo / offa_hi are
 * the lane's A words of the low and high halves (or the shared zero words). */
template <int TYPE, int NQ, bool SC, int NT, int TS>
__device__ __forceinline__ void mx_chunk16(const uint8_t *W, const uint8_t *R, int lr, int lg, int offa_lo,
                                           int offa_hi, f32x4 (&acc)[2][kMxNA], float (&cr)[2][4])
{
    static_assert(kMxC == 8, "eight blocks per staged chunk");
    constexpr int WS = mx_wstride(TYPE), QO = TYPE == 3 ? 4 : 2;
    MxStreams st;
    st.alo = (LdsPtr)(R + offa_lo);
    st.ahi = (LdsPtr)(R + offa_hi);
    st.d = (LdsPtr)(R + lg * mx_rstride(TYPE) + kMxDx);
    st.q = (LdsPtr)(W + lr * WS + QO + 4 * lg);
    st.dw = (LdsPtr)(W + lr * WS);
    mx_opaque(st);
    /* one block's operands in registers at a time */
    mx_block16<TYPE, NQ, 0, SC, NT, TS>(st, acc, cr);
    __builtin_amdgcn_sched_barrier(0);
    mx_block16<TYPE, NQ, 1, SC, NT, TS>(st, acc, cr);
    __builtin_amdgcn_sched_barrier(0);
    mx_block16<TYPE, NQ, 2, SC, NT, TS>(st, acc, cr);
    __builtin_amdgcn_sched_barrier(0);
    mx_block16<TYPE, NQ, 3, SC, NT, TS>(st, acc, cr);
    __builtin_amdgcn_sched_barrier(0);
    mx_block16<TYPE, NQ, 4, SC, NT, TS>(st, acc, cr);
    __builtin_amdgcn_sched_barrier(0);
    mx_block16<TYPE, NQ, 5, SC, NT, TS>(st, acc, cr);
    __builtin_amdgcn_sched_barrier(0);
    mx_block16<TYPE, NQ, 6, SC, NT, TS>(st, acc, cr);
    __builtin_amdgcn_sched_barrier(0);
    mx_block16<TYPE, NQ, 7, SC, NT, TS>(st, acc, cr);
}

/* A word of a staged Q6_K row at byte off past the row's 4-byte-aligned LDS base (O = 2: the
 * super-block sits 2 bytes in, so the word straddles two aligned words). */
template <int O>
__device__ __forceinline__ uint32_t q6_word(LdsPtr base, int off)
{
    typedef __attribute__((address_space(3))) const uint32_t LdsU32;
    if constexpr (O == 0) return *(LdsU32 *)(base + off);
    else return __builtin_amdgcn_alignbyte(*(LdsU32 *)(base + off + 2), *(LdsU32 *)(base + off - 2), 2);
}

/* The B operand and scales of 32-block B (0..7) of the staged Q6_K super-block for tile t:
 * q points at the lane's code words (row base + 4*lg), rb at the row base. Every offset and
 * shift is a constant. The 6-bit code dword is the low nibbles (shifted down for the upper
 * two blocks of a half) with the two high bits of qh moved to bits 4-5 (src/kernels.c:148-160). */
template <int O, int B, int TS>
__device__ __forceinline__ MxB mx_weights_q6(LdsPtr q, LdsPtr rb, int t, int kh)
{
    constexpr int WS = mx_wstride(14), h = B >> 2, g = B & 3, ns = 4 * (g >> 1), hs = 2 * g;
    constexpr int oql = O + 64 * h + 32 * (g & 1), oqh = O + 128 + 32 * h;
    const uint32_t lo4 = 0x0f0f0f0fu;
    auto code = [&](int dq) {
        const uint32_t ql = q6_word<O>(q, TS * t * WS + oql + dq), qh = q6_word<O>(q, TS * t * WS + oqh + dq);
        uint32_t hi;
        if constexpr (hs < 4) hi = (qh << (4 - hs)) & 0x30303030u;
        else if constexpr (hs == 4) hi = qh & 0x30303030u;
        else hi = (qh >> (hs - 4)) & 0x30303030u;
        return and_or(ns ? (ql >> ns) : ql, lo4, hi);
    };
    const uint32_t cA = code(0), cB = code(16);
    MxB w;
    /* the f16 subnormals code 2^-24: bytes 0 and 2, then 1 and 3, of each code dword into the
     * low bytes of its halves (one byte permute each) */
    w.op = __builtin_bit_cast(f16x8, u32x4{ __builtin_amdgcn_perm(cA, cA, 0x0c020c00u), __builtin_amdgcn_perm(cA, cA, 0x0c030c01u),
                                            __builtin_amdgcn_perm(cB, cB, 0x0c020c00u), __builtin_amdgcn_perm(cB, cB, 0x0c030c01u) });
    const uint32_t scw = *(const __attribute__((address_space(3))) uint16_t *)(rb + TS * t * WS + O + 192 + 8 * h + 2 * g);
    /* the int16 pair {sc[2g], sc[2g+1]}: byte permute with sign fills (selector 10: the sign of
     * byte 1 of the first source, scw << 8, i.e. of sc[2g]; selector 8: of byte 1 of scw) */
    w.sab = __builtin_amdgcn_perm(scw << 8, scw, 0x08010a00u);
    /* sc * 2^24 = (u - 128) * 2^24 for the byte u = sc ^ 0x80, exact in one fma */
    const uint32_t sx = scw ^ 0x8080u;
    const float s0 = __builtin_fmaf((float)(sx & 0xffu), 16777216.0f, -2147483648.0f);
    const float s1 = __builtin_fmaf((float)((sx >> 8) & 0xffu), 16777216.0f, -2147483648.0f);
    w.sc = kh ? s1 : s0;
    w.sc1 = s1;
    w.dw = *(const __attribute__((address_space(3))) uint16_t *)(rb + TS * t * WS + O + 208);
    return w;
}

/* One Q6_K block B of the staged chunk: NP slot pairs against the wave's two 16-row tiles. */
template <int NP, int O, int B, int TS>
__device__ __forceinline__ void mx_block_q6(const MxStreams &st, int kh, f32x4 (&acc)[2][kMxNA], float (&cr)[2][4])
{
    constexpr int RS = mx_rstride(14), RB = B * mx_recl(14);
    MxB w[2];
#pragma unroll
    for (int t = 0; t < 2; t++) w[t] = mx_weights_q6<O, B, TS>(st.q, st.dw, t, kh);
#pragma unroll
    for (int p = 0; p < NP; p++) {
        /* volatile: keeps each A read a single read into the MFMA operand (records 832 bytes
         * apart would otherwise be merged into paired reads plus register moves) */
        const u32x2 lo = *(const volatile LdsU32x2 *)(st.alo + RB + 2 * p * RS);
        const u32x2 hi = *(const volatile LdsU32x2 *)(st.ahi + RB + 2 * p * RS);
        const f16x8 aop = __builtin_bit_cast(f16x8, u32x4{ lo.x, lo.y, hi.x, hi.y });
        const u32x4 dx = *(const LdsU32x4 *)(st.d + RB + 2 * p * RS);          /* -, ds, s16 pair, d */
        const float xd = __uint_as_float(dx.w);
        const uint32_t s16p = dx.z;           /* (bit_cast of a vector element itself reads .x) */
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const f32x4 S =
                __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, w[t].op, f32x4{ 0.0f, 0.0f, 0.0f, 0.0f }, 0, 0, 0);
            const float dd = mix_mul(w[t].dw, xd);
#pragma unroll
            for (int v = 0; v < 4; v++) acc[t][p][v] = __builtin_fmaf(S[v] * w[t].sc, dd, acc[t][p][v]);
            /* sc[2g]*s16[0] + sc[2g+1]*s16[1] in one packed int16 dot */
            const int ssum = sdot2_i16(w[t].sab, s16p);
            cr[t][p] = __builtin_fmaf(dd, (float)ssum, cr[t][p]);
        }
    }
}

/* A staged Q6_K super-block, its 8 blocks unrolled (offsets and shifts depend on the block);
 * the wave's two tiles TS staged rows apart. */
template <int NP, int O, int TS>
__device__ __forceinline__ void mx_chunk_q6(const uint8_t *W, const uint8_t *R, int lr, int lg, int kh, int jd,
                                            int offa_lo, int offa_hi, f32x4 (&acc)[2][kMxNA], float (&cr)[2][4])
{
    constexpr int WS = mx_wstride(14);
    MxStreams st;
    st.alo = (LdsPtr)(R + offa_lo);
    st.ahi = (LdsPtr)(R + offa_hi);
    st.d = (LdsPtr)(R + jd * mx_rstride(14) + kMxDx);
    st.q = (LdsPtr)(W + lr * WS + 4 * lg);
    st.dw = (LdsPtr)(W + lr * WS);
    mx_opaque(st);
    mx_block_q6<NP, O, 0, TS>(st, kh, acc, cr);
    __builtin_amdgcn_sched_barrier(0);
    mx_block_q6<NP, O, 1, TS>(st, kh, acc, cr);
    __builtin_amdgcn_sched_barrier(0);
    mx_block_q6<NP, O, 2, TS>(st, kh, acc, cr);
    __builtin_amdgcn_sched_barrier(0);
    mx_block_q6<NP, O, 3, TS>(st, kh, acc, cr);
    __builtin_amdgcn_sched_barrier(0);
    mx_block_q6<NP, O, 4, TS>(st, kh, acc, cr);
    __builtin_amdgcn_sched_barrier(0);
    mx_block_q6<NP, O, 5, TS>(st, kh, acc, cr);
    __builtin_amdgcn_sched_barrier(0);
    mx_block_q6<NP, O, 6, TS>(st, kh, acc, cr);
    __builtin_amdgcn_sched_barrier(0);
    mx_block_q6<NP, O, 7, TS>(st, kh, acc, cr);
}

/* One Q6_K block B of the staged chunk on the 16x16x16 instructions (the layout of mx_block16):
 * half h of the 32-block is sub-block 2g + h, so each instruction's lane sums share one
 * sub-scale per row; one d_w d_x product and one half-sum offset step per (tile, quad, block). */
template <int NQ, int O, int B, int TS>
__device__ __forceinline__ void mx_block16_q6(const MxStreams &st, f32x4 (&acc)[2][kMxNA], float (&cr)[2][4])
{
    constexpr int RS = mx_rstride(14), RB = B * mx_recl(14);
    MxB w[2];
    f16x4 b[2][2];
    float sc[2][2];
#pragma unroll
    for (int t = 0; t < 2; t++) {
        w[t] = mx_weights_q6<O, B, TS>(st.q, st.dw, t, 0);
        b[t][0] = __builtin_shufflevector(w[t].op, w[t].op, 0, 1, 2, 3);
        b[t][1] = __builtin_shufflevector(w[t].op, w[t].op, 4, 5, 6, 7);
        sc[t][0] = w[t].sc;                                              /* sc[2g] 2^24 */
        sc[t][1] = w[t].sc1;                                             /* sc[2g+1] 2^24 */
    }
    f32x4 S[2][2];
    float xd[NQ], dd[2];
    uint32_t s16p[NQ];
    auto issue = [&](int u, int k) {
        const int q = u >> 1, h = u & 1;
        const u32x2 av = *(const LdsU32x2 *)((h ? st.ahi : st.alo) + RB + 4 * q * RS);
        if (h == 0) {
            const u32x4 dx = *(const LdsU32x4 *)(st.d + RB + 4 * q * RS);    /* -, ds, s16 pair, d */
            xd[q] = __uint_as_float(dx.w);
            s16p[q] = dx.z;
        }
        const f16x4 aop = __builtin_bit_cast(f16x4, av);
#pragma unroll
        for (int t = 0; t < 2; t++)
            S[k][t] = __builtin_amdgcn_mfma_f32_16x16x16f16(aop, b[t][h], f32x4{ 0.0f, 0.0f, 0.0f, 0.0f }, 0, 0, 0);
    };
    issue(0, 0);
#pragma unroll
    for (int u = 0; u < 2 * NQ; u++) {
        const int k = u & 1, q = u >> 1, h = u & 1;
        if (u + 1 < 2 * NQ) issue(u + 1, k ^ 1);
        if (h == 0) {
#pragma unroll
            for (int t = 0; t < 2; t++) dd[t] = mix_mul(w[t].dw, xd[q]);
        }
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int v = 0; v < 4; v++)
                acc[t][2 * q + h][v] = __builtin_fmaf(S[k][t][v] * sc[t][h], dd[t], acc[t][2 * q + h][v]);
        if (h == 1) {
#pragma unroll
            for (int t = 0; t < 2; t++) {
                /* sc[2g]*s16[0] + sc[2g+1]*s16[1] in one packed int16 dot */
                const int ssum = sdot2_i16(w[t].sab, s16p[q]);
                cr[t][q] = __builtin_fmaf(dd[t], (float)ssum, cr[t][q]);
            }
        }
    }
}

/* A staged Q6_K super-block on the 16x16x16 instructions, its 8 blocks unrolled. */
template <int NQ, int O, int TS>
__device__ __forceinline__ void mx_chunk16_q6(const uint8_t *W, const uint8_t *R, int lr, int lg, int offa_lo,
                                              int offa_hi, f32x4 (&acc)[2][kMxNA], float (&cr)[2][4])
{
    constexpr int WS = mx_wstride(14);
    MxStreams st;
    st.alo = (LdsPtr)(R + offa_lo);
    st.ahi = (LdsPtr)(R + offa_hi);
    st.d = (LdsPtr)(R + lg * mx_rstride(14) + kMxDx);
    st.q = (LdsPtr)(W + lr * WS + 4 * lg);
    st.dw = (LdsPtr)(W + lr * WS);
    mx_opaque(st);
    mx_block16_q6<NQ, O, 0, TS>(st, acc, cr);
    __builtin_amdgcn_sched_barrier(0);
    mx_block16_q6<NQ, O, 1, TS>(st, acc, cr);
    __builtin_amdgcn_sched_barrier(0);
    mx_block16_q6<NQ, O, 2, TS>(st, acc, cr);
    __builtin_amdgcn_sched_barrier(0);
    mx_block16_q6<NQ, O, 3, TS>(st, acc, cr);
    __builtin_amdgcn_sched_barrier(0);
    mx_block16_q6<NQ, O, 4, TS>(st, acc, cr);
    __builtin_amdgcn_sched_barrier(0);
    mx_block16_q6<NQ, O, 5, TS>(st, acc, cr);
    __builtin_amdgcn_sched_barrier(0);
    mx_block16_q6<NQ, O, 6, TS>(st, acc, cr);
    __builtin_amdgcn_sched_barrier(0);
    mx_block16_q6<NQ, O, 7, TS>(st, acc, cr);
}

/* The LDS DMA: `bytes` (4 or 16) from src of every active lane to dst + lane * bytes. */
template <int BYTES>
__device__ __forceinline__ void dma_to_lds(const void *src, uint8_t *dst)
{
    if constexpr (BYTES == 4) __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)dst, 4, 0, 0);
    else __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)dst, 16, 0, 0);
}

/* Wait for all of this wave's vector memory instructions (its LDS DMA included) and LDS
 * accesses, then the block barrier. The memory clobber keeps the compiler from moving LDS
 * accesses across it. */
__device__ __forceinline__ void mx_wait_barrier()
{
    asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

/* Wait for this wave's LDS accesses only (DMA still in flight), then the block barrier. */
__device__ __forceinline__ void mx_lds_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

#ifndef QMSG_MX_WIDE16_SLOTS
#define QMSG_MX_WIDE16_SLOTS 8
#endif
#ifndef QMSG_MX_NARROW_GU
#define QMSG_MX_NARROW_GU 8
#endif
#ifndef QMSG_MX_NARROW_DN
#define QMSG_MX_NARROW_DN 8
#endif
#ifndef QMSG_MX_MID_NB
#define QMSG_MX_MID_NB 2
#endif
#ifndef QMSG_MX_MID_NB_Q6
#define QMSG_MX_MID_NB_Q6 1
#endif
/* staging of the 16-slot blocks: the weights in two buffers, the records in one
 * (mx_lds_bytes nb 3) */
#ifndef QMSG_MX_WIDE16_NB_GU
#define QMSG_MX_WIDE16_NB_GU 3
#endif
#ifndef QMSG_MX_WIDE16_NB_DN
#define QMSG_MX_WIDE16_NB_DN 3
#endif
#ifndef QMSG_MX_WIDE16_NT
#define QMSG_MX_WIDE16_NT 2
#endif
#ifndef QMSG_MX_WIDE16_NW
#define QMSG_MX_WIDE16_NW 8
#endif
/* Waves per SIMD the MFMA kernel is built for: six where three double-buffered blocks' LDS
 * fits a CU, else four (the register budget follows: 80 or 128 VGPRs). */
template <int TYPE, int WSG, int PPW, int NW, int NB, int NT>
constexpr int mx_waves()
{
    if (PPW == 8 && NT == 2) return NB == 2 ? 2 : 3;    /* two tiles x 16 slots per wave: 168 VGPRs */
    return NB == 1 ? 4 : (160 * 1024 / mx_lds_bytes(TYPE, WSG, PPW, NW, NB, NT)) * NW / 4 >= 6 ? 6 : 4;
}

/* Gate/up (GU = 1: gate rows against the token's input records, the same up rows, SwiGLU, the
 * int8 activation blocks and their records) or down (GU = 0: dn rows) of one slot tile, with NB
 * staging buffers: 2 (the next chunk's copy in flight while this one computes) or 1 (copy, wait,
 * compute; the other blocks on the CU hide the copy). Several blocks share a CU, which hides the
 * LDS and memory latency. */
template <int TYPE, int WSG, int GU, int PPW, int NW, int NB, int NT>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(mx_waves<TYPE, WSG, PPW, NW, NB, NT>(),
                                                                         mx_waves<TYPE, WSG, PPW, NW, NB, NT>())))
void mx_kernel(MxArgs a)
{
    extern __shared__ __align__(16) uint8_t smem[];
    using Lay = MxLayout<TYPE, WSG, PPW, NW, NT>;
    static_assert(NT == 2 || (NT == 1 && TYPE != 14), "one-tile waves take Q4_0 / Q4_1 rows");
    /* Q6_K gate/up (4-byte DMA units) steps through its gate rows, then its up rows */
    constexpr bool QS6 = GU && TYPE == 14;
    /* gate/up on two-tile waves: the RWG/2 gate rows staged first, then the same up rows, so
     * each DMA instruction reads one matrix (a wave-uniform base) and a wave's two tiles (its
     * gate and up rows) lie RWG/2 rows apart */
    constexpr bool GSEP = GU && NT == 2;
#ifdef QMSG_MX_X32
    constexpr bool X16Q = false;
#elif defined(QMSG_MX_Q6_PAIRS)
    constexpr bool X16Q = TYPE != 14;
#else
    constexpr bool X16Q = true;                /* lane sums on the 16x16x16 instructions (waves of 3+ slots) */
#endif
    constexpr int RWG = Lay::RWG, SWG = Lay::SWG, WS = Lay::WS, BUF = Lay::BUF;
    static_assert(PPW <= 4 || X16Q, "waves of more than 8 slots take the 16x16x16 quads");
    if ((int)blockIdx.y >= a.S.meta[1]) return;
    const int4 tl = a.S.tiles[blockIdx.y];
    const int e = tl.x, s0 = tl.y + (int)blockIdx.z * SWG, ns = min(SWG, tl.z - s0);
    if (ns <= 0) return;
    const int tid = threadIdx.x, lane = tid & 63, lr = lane & 15, lg = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);          /* wave-uniform */
    const int wr = wave / WSG, ws = wave % WSG, kh = lg & 1, jd = lg >> 1;
    const int nb = (GU ? a.E : a.F) >> 5, nch = nb / kMxC;
    const int R0 = (int)blockIdx.x * (GU ? RWG / 2 : RWG);

    /* row i of the staged tile: for gate/up on two-tile waves gate row R0 + i below RWG/2 and
     * up row R0 + i - RWG/2 above; on one-tile waves row group g = i / 32 holds gate rows
     * R0 + 16g .. R0 + 16g + 15 and then the same up rows. Byte offsets inside one expert's
     * matrix fit 31 bits (mx_supported); the expert bases are wave-uniform. */
    const uint8_t *wb0 = a.w0 + (size_t)e * a.eb, *wb1 = GU ? a.w1 + (size_t)e * a.eb : wb0;
    const uint32_t rb = (uint32_t)a.rb;
    /* slot i's records (slots past the tile repeat its last slot) */
    auto rec_ptr = [&](int i) -> const uint8_t * {
        const int s = s0 + min(i, ns - 1);
        return a.rec + (size_t)(GU ? a.S.slot_t[s] : s) * nb * kMxRec;
    };
    /* the DMA of chunk c into buffer k: weight instruction q goes to wave q % 8, the records of
     * slot i (one instruction) to wave i % 8, their source fixed per block */
    constexpr int RPW = SWG / NW;                     /* slots whose records one wave copies */
    static_assert(RPW >= 1 && SWG % NW == 0, "every slot's records copied by one wave");
    const uint8_t *rsrc[RPW];
#pragma unroll
    for (int j = 0; j < RPW; j++) rsrc[j] = rec_ptr(wave + NW * j);
    /* Each lane's weight DMA sources, computed once: unit n = 64q + lane of the staged tile
     * (row n / WUR, unit n % WUR) for this wave's instructions q = wave, wave + 8, ... Q4 types:
     * the offset inside the expert's matrix per instruction (bit 31: an up row); Q6_K (down
     * rows, whose 108 instructions per chunk would take too many registers): the first one,
     * stepped by 512 units per instruction. */
    static_assert(RWG * Lay::WUR % 64 == 0, "whole DMA instructions per chunk");
    static_assert(!GSEP || (RWG / 2) * Lay::WUR % 64 == 0, "gate rows in whole DMA instructions");
    constexpr int NQ = (Lay::WINSTR + NW - 1) / NW;
    uint32_t qoff[TYPE == 14 ? 1 : NQ];
    int qu = 0;
    auto unit_off = [&](int n, int *u_out) -> uint32_t {
        const int i = n / Lay::WUR, u = n - i * Lay::WUR;
        *u_out = u;
        /* two-tile gate/up: gate rows first, up rows from staged row RWG/2 on (GSEP); one-tile
         * gate/up: 16 gate rows, then the same up rows (bit 31 of the offset: an up row) */
        const int row = GSEP ? R0 + (i % (RWG / 2)) : (GU ? R0 + 16 * (i >> 5) + (i & 15) : R0 + i);
        const uint32_t up = GU && !GSEP && (i & 31) >= 16 ? 0x80000000u : 0u;
        return ((uint32_t)row * rb + (uint32_t)(Lay::WUNIT * u)) | up;
    };
    /* Q6_K gate/up: the first instruction of this wave in the up half, and its source */
    constexpr int HALF = Lay::WINSTR / 2;
    const int q_up = wave + NW * ((HALF - wave + NW - 1) / NW);
    uint32_t qoff_up = 0;
    int qu_up = 0;
    if constexpr (TYPE == 14) {
        qoff[0] = unit_off(64 * wave + lane, &qu);
        if constexpr (QS6) qoff_up = unit_off(64 * (q_up - HALF) + lane, &qu_up);
    } else {
#pragma unroll
        for (int j = 0; j < NQ; j++) {
            int u;
            qoff[j] = unit_off(min(64 * (wave + NW * j) + lane, RWG * Lay::WUR - 1), &u);
        }
    }
    /* chunk c's weight rows into the weight area at base, its records into the record area
     * at rbase */
    auto issue_w = [&](int c, uint8_t *base) {
        if constexpr (TYPE == 14) {
            /* the super-block starts 2 bytes past a 4-byte boundary on odd chunks */
            const uint32_t cb = (uint32_t)(c * 210 - 2 * (c & 1));
            uint32_t o = qoff[0];
            int u = qu;
            const uint8_t *wq = wb0;
            /* 64 NW units on: STEP / WUR rows and STEP % WUR units, one row more where the
             * units wrap */
            constexpr int STEP = 64 * NW, SR = STEP / Lay::WUR, SU = STEP % Lay::WUR;
            for (int q = wave; q < Lay::WINSTR; q += NW) {
                if (QS6 && q == q_up) {        /* into the up half: the up matrix from its row R0 */
                    o = qoff_up;
                    u = qu_up;
                    wq = wb1;
                }
                dma_to_lds<4>(wq + (o + cb), base + 256 * q);
                u += SU;
                o += SR * rb + 4 * SU;
                if (u >= Lay::WUR) {
                    u -= Lay::WUR;
                    o += rb - 4 * Lay::WUR;
                }
            }
        } else {
            const uint32_t cb = (uint32_t)(c * (kMxC * (TYPE == 3 ? 20 : 18)));
#pragma unroll
            for (int j = 0; j < NQ; j++) {
                const int q = wave + NW * j;
                if (q < Lay::WINSTR) {
                    const uint32_t o = qoff[j];
                    if constexpr (GSEP)   /* instructions 0 .. HALF-1 read gate rows, the rest up rows */
                        dma_to_lds<16>((q >= HALF ? wb1 : wb0) + (o + cb), base + 1024 * q);
                    else
                        dma_to_lds<16>(((o >> 31) ? wb1 : wb0) + ((o & 0x7fffffffu) + cb), base + 1024 * q);
                }
            }
        }
    };
    auto issue_r = [&](int c, uint8_t *rbase) {
        /* a slot's kMxC records, the first 96 bytes of each: 48 lanes x 16 bytes */
        if (lane < kMxC * mx_recl(TYPE) / 16) {
            const uint32_t src = (uint32_t)((lane / 6) * kMxRec + 16 * (lane % 6));
#pragma unroll
            for (int j = 0; j < RPW; j++)
                dma_to_lds<16>(rsrc[j] + (size_t)c * kMxC * kMxRec + src, rbase + (wave + NW * j) * Lay::RS);
        }
    };
    auto issue = [&](int c, int k) {
        issue_w(c, smem + k * BUF);
        issue_r(c, smem + k * BUF + Lay::WBYTES);
    };
    /* NB == 3: weights in two buffers (W0, W1), records in one after them */
    uint8_t *const rarea = smem + 2 * Lay::WBYTES;

    /* A reads: lane row lr is slot ja = lr/8 of the pair, reference lane ka = lr%8; it holds x
     * only if ka%4 == lg, in the low half of its 8 K positions for ka < 4 */
    const int ja = lr >> 3, ka = lr & 7;
    const bool nz = (ka & 3) == lg;
    const int offa_lo = ja * Lay::RS + ((nz && ka < 4) ? 8 * ka : kMxZero);
    const int offa_hi = ja * Lay::RS + ((nz && ka >= 4) ? 8 * ka : kMxZero);
    /* 16x16x16 instructions: lane row lr is slot lr / 4 of the quad, reference lane lr % 4 (+4 in
     * the high half); it holds x only if lr % 4 == lg. The other lanes read the zero words of
     * the quad's slot 3 (one address: a broadcast), whose LDS banks (word mod 64) the lanes
     * holding x leave free at the 200-word record stride: their words sit at s * RS + 2 lg
     * (+ 8 in the high half), the zero words at 3 RS + 20. */
    const bool nz4 = (lr & 3) == lg;
    const int offq_lo = nz4 ? (lr >> 2) * Lay::RS + 8 * lg : 3 * Lay::RS + kMxZero;
    const int offq_hi = nz4 ? (lr >> 2) * Lay::RS + 8 * (lg + 4) : 3 * Lay::RS + kMxZero;
    const int nw = min(max(ns - 2 * PPW * ws, 0), 2 * PPW), np = (nw + 1) >> 1;   /* this wave's slot pairs */

    /* The whole chunk loop and the row sums for one slot-pair count NP, chosen once per wave,
     * so the accumulators keep their registers from the first chunk to the last. Every wave
     * issues its share of the DMA and meets every barrier, whatever its NP (0 included). */
    constexpr float scale = finish_scale(TYPE);
    float *res = (float *)smem;                                   /* [RWG][SWG + 1], after the loop */
    auto run = [&](auto npc, auto scc, auto x16c) {
        constexpr int NP = decltype(npc)::value;
        constexpr bool SC = decltype(scc)::value;
        constexpr bool X16 = decltype(x16c)::value;     /* NP / 2 quads on 16x16x16, else NP pairs */
        f32x4 acc[2][kMxNA];
        float cr[2][4];
#pragma unroll
        for (int t = 0; t < 2; t++) {
#pragma unroll
            for (int p = 0; p < kMxNA; p++) acc[t][p] = f32x4{ 0.0f, 0.0f, 0.0f, 0.0f };
#pragma unroll
            for (int p = 0; p < 4; p++) cr[t][p] = 0.0f;
        }
        if (NB == 2) {
            issue(0, 0);
            mx_wait_barrier();
        } else if (NB == 3) {
            issue_w(0, smem);
            issue_r(0, rarea);
            mx_wait_barrier();
        }
        for (int c = 0; c < nch; c++) {
            const int buf = NB >= 2 ? c & 1 : 0;
            if (NB == 1) {
                issue(c, 0);
                mx_wait_barrier();
            } else if (NB == 2) {
                if (c + 1 < nch) issue(c + 1, buf ^ 1);
            } else {
                if (c > 0) {
                    /* this chunk's records (every wave is past its reads of the last ones),
                     * then its weights, requested a chunk ago, and they */
                    issue_r(c, rarea);
                    mx_wait_barrier();
                }
                /* the next chunk's weights stream in while this one computes */
                if (c + 1 < nch) issue_w(c + 1, smem + (buf ^ 1) * Lay::WBYTES);
            }
            if constexpr (NP > 0) {
                const uint8_t *Wl = (NB == 3 ? smem + buf * Lay::WBYTES : smem + buf * BUF) +
                                    ((GSEP ? 16 : 16 * NT) * wr) * WS;
                const uint8_t *Rl = (NB == 3 ? rarea : smem + buf * BUF + Lay::WBYTES) + (2 * PPW * ws) * Lay::RS;
                if constexpr (TYPE == 14 && X16) {
                    constexpr int TS6 = QS6 ? RWG / 2 : 16;
                    if (c & 1) mx_chunk16_q6<NP / 2, 2, TS6>(Wl, Rl, lr, lg, offq_lo, offq_hi, acc, cr);
                    else mx_chunk16_q6<NP / 2, 0, TS6>(Wl, Rl, lr, lg, offq_lo, offq_hi, acc, cr);
                } else if constexpr (TYPE == 14) {
                    constexpr int TS6 = QS6 ? RWG / 2 : 16;
                    if (c & 1) mx_chunk_q6<NP, 2, TS6>(Wl, Rl, lr, lg, kh, jd, offa_lo, offa_hi, acc, cr);
                    else mx_chunk_q6<NP, 0, TS6>(Wl, Rl, lr, lg, kh, jd, offa_lo, offa_hi, acc, cr);
                } else if constexpr (X16) {
                    mx_chunk16<TYPE, NP / 2, SC, NT, GSEP ? RWG / 2 : 16>(Wl, Rl, lr, lg, offq_lo, offq_hi, acc, cr);
                } else {
                    mx_chunk<TYPE, NP, SC, GSEP ? RWG / 2 : 16>(Wl, Rl, lr, lg, jd, kh != 0, offa_lo, offa_hi, acc, cr);
                }
            }
            if (NB == 3) {
                /* every wave's record and weight reads of chunk c are done */
                mx_lds_barrier();
            } else {
                /* chunk c+1 has landed; buffer c is free for chunk c+2 (one buffer: it is free) */
                mx_wait_barrier();
            }
        }
        if (NB == 3) mx_wait_barrier();
        if constexpr (X16) {
            /* hsum256 per (row, slot), all eight chains in the lane: acc[t][2q] lanes 0-3,
             * acc[t][2q + 1] lanes 4-7 */
#pragma unroll
            for (int t = 0; t < NT; t++)
#pragma unroll
                for (int q = 0; q < NP / 2; q++) {
                    const f32x4 &lo = acc[t][2 * q], &hi = acc[t][2 * q + 1];
                    const float h = ((lo[0] + hi[0]) + (lo[2] + hi[2])) + ((lo[1] + hi[1]) + (lo[3] + hi[3]));
                    const float val = h - scale * cr[t][q];
                    const int row = 16 * NT * wr + 16 * t + lr, sl = 2 * PPW * ws + 4 * q + lg;
                    if (GU) res[row * (SWG + 1) + sl] = val;
                    else if (sl < ns) a.S.dn[(size_t)(s0 + sl) * a.E + R0 + row] = val;
                }
            return;
        }
        /* hsum256 per (row, slot): lanes of k-half 0 take the partner lane's k + 4 chains (Q4
         * types: and, for tile 1, the partner's offset chain); two-tile waves only */
        static_assert(NT == 2 || X16 || NP == 0, "one-tile waves run quads only");
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int p = 0; p < NP; p++) {
                f32x4 o;
#pragma unroll
                for (int v = 0; v < 4; v++) o[v] = __shfl_xor(acc[t][p][v], 16);
                float crv = cr[t][p];
                if constexpr (TYPE != 14) {
                    const float other = __shfl_xor(cr[0][p], 16);
                    crv = t == 0 ? cr[0][p] : other;
                }
                if (kh == 0) {
                    const f32x4 &q = acc[t][p];
                    const float h = ((q[0] + o[0]) + (q[2] + o[2])) + ((q[1] + o[1]) + (q[3] + o[3]));
                    const float val = h - scale * crv;
                    const int row = 32 * wr + 16 * t + lr, sl = 2 * PPW * ws + 2 * p + jd;
                    if (GU) res[row * (SWG + 1) + sl] = val;
                    else if (sl < ns) a.S.dn[(size_t)(s0 + sl) * a.E + R0 + row] = val;
                }
            }
    };
    auto by_pairs = [&](auto scc) {
        using Q = std::integral_constant<bool, X16Q>;
        using P = std::false_type;
        if constexpr (X16Q) {
            /* quads of slots (NP = 2 x quads); a wave of one or two slots keeps the pair
             * instructions, on which a quad's padding would double its work */
            const int nq = (nw + 3) >> 2;
            if (PPW == 8 && nq == 4) run(std::integral_constant<int, PPW == 8 ? 8 : 0>{}, scc, Q{});
            else if (PPW == 8 && nq == 3) run(std::integral_constant<int, PPW == 8 ? 6 : 0>{}, scc, Q{});
            else if (PPW >= 4 && nq == 2) run(std::integral_constant<int, PPW >= 4 ? 4 : 0>{}, scc, Q{});
            else if (nw > 2 || (NT == 1 && nw > 0)) run(std::integral_constant<int, 2>{}, scc, Q{});
            else if (nw > 0) run(std::integral_constant<int, NT == 2 ? 1 : 0>{}, scc, P{});
            else run(std::integral_constant<int, 0>{}, scc, P{});
        } else {
            if (PPW == 4 && np == 4) run(std::integral_constant<int, PPW == 4 ? 4 : 0>{}, scc, P{});
            else if (PPW == 4 && np == 3) run(std::integral_constant<int, PPW == 4 ? 3 : 0>{}, scc, P{});
            else if (np == 2) run(std::integral_constant<int, 2>{}, scc, P{});
            else if (np == 1) run(std::integral_constant<int, 1>{}, scc, P{});
            else run(std::integral_constant<int, 0>{}, scc, P{});
        }
    };
    /* Q4 types: whether every record this launch reads carries d_x 2^24 (their producers
     * stored this call's epoch in the flag otherwise); both loops are whole, so neither's
     * registers depend on the other */
    if constexpr (TYPE == 14) by_pairs(std::true_type{});
    else if (a.S.mxflag[GU ? 0 : 1] != a.S.epoch) by_pairs(std::true_type{});
    else by_pairs(std::false_type{});
    if (!GU) return;
    __syncthreads();
    /* a = silu(g) * u (src/model.c:989-994) into the gate rows of res, then the int8 blocks of
     * whole 32-row blocks (src/model.c:996-997) and their records. F-row fr sits in row group
     * fr / 16: gate at res row 32 (fr / 16) + fr % 16, up 16 rows further. */
    const int F = a.F, nbF = F >> 5;
    auto gate_row = [](int fr) { return 32 * (fr >> 4) + (fr & 15); };
    for (int i = tid; i < (RWG / 2) * SWG; i += 64 * NW) {
        const int fr = i / SWG, sl = i - fr * SWG;
        if (sl >= ns) continue;
        const float gv = res[gate_row(fr) * (SWG + 1) + sl], uv = res[(gate_row(fr) + 16) * (SWG + 1) + sl];
        const float av = silu_ref(gv) * uv;
        res[gate_row(fr) * (SWG + 1) + sl] = av;
        if (a.debug) {
            const size_t s = (size_t)(s0 + sl);
            a.S.gu[s * 2 * F + R0 + fr] = gv;
            a.S.gu[s * 2 * F + F + R0 + fr] = uv;
            a.S.act[s * F + R0 + fr] = av;
        }
    }
    __syncthreads();
    constexpr int NFB = RWG / 64;                                  /* activation blocks per slot */
    for (int i = tid; i < SWG * NFB; i += 64 * NW) {
        const int sl = i / NFB, g = i - sl * NFB;
        if (sl >= ns) continue;
        float v[32];
#pragma unroll
        for (int j = 0; j < 32; j++) v[j] = res[gate_row(32 * g + j) * (SWG + 1) + sl];
        const Q8Vals q = quantize_block(v);
        const int s = s0 + sl, blk = (R0 >> 5) + g;
        store_q8(q, a.S.aq + (size_t)s * nbF + blk);
        store_pair_half(q, (uint32_t *)(a.S.aqk + ((size_t)s * (nbF >> 1) + (blk >> 1)) * kPairBytes), blk & 1);
        if (!mx_store_record(q, a.rec_out + ((size_t)s * nbF + blk) * kMxRec, a.rec_out_hi16))
            a.S.mxflag[1] = a.S.epoch;
    }
}

/* Two 80 KB Q6_K blocks (16-slot, 128 rows) share a CU. */
static_assert(2 * mx_lds_bytes(14, 2) <= 160 * 1024, "two Q6_K blocks per CU");

/* Block shapes, chosen per kernel by the batch's slots per active expert r (the more slots a
 * block takes, the more of them are padding on sparse tiles; the fewer, the fewer MFMAs each
 * staged weight row feeds). A block's waves form row groups of 32 rows x slot groups:
 *   wide16 (Q4_0 / Q4_1, r >= 8): 4 waves, 4 row groups of 8 pairs: 128 rows x 16 slots, each
 *          wave's unpacked weight tiles feeding four quads, three waves per SIMD. The weights
 *          sit in two buffers and the records in one (49 KB, still three blocks per CU), the
 *          next chunk's weights streaming in while one computes: at the 512-token prefill
 *          gate/up 794-820 against 850 us with one buffer, down 384 against 407; gate/up at
 *          128 / 192 / 256 tokens 295 / 363 / 483 against 324 / 391 / 525. Gate/up stages
 *          its gate rows, then its up rows, so each DMA instruction reads one matrix from a
 *          wave-uniform base (with 16-row groups interleaved it spilled 20 registers this
 *          way and ran 970 us). Against the shapes below at the 235B shape (us, gate/up / down): 321 / 155
 *          against 350 / 158 at r = 8, 353 / 171 against 422 / 196 at 10, 384 / 186 against
 *          403 / 213 at 12, 719 / 348 against 734 / 364 at 24; 286 / 138 against 275 / 128 at
 *          6 and 262 / 125 against 239 / 114 at 4, where it is not taken;
 *   wide   (other types: gate/up r >= 12, down r >= 16): 8 waves, 4 row groups x 2 slot groups of 4 pairs:
 *          128 rows x 16 slots, two staging buffers;
 *   mid:   4 waves, 4 row groups x 1 slot group of 4 pairs: 128 rows x 8 slots; Q4_0 / Q4_1
 *          two staging buffers (three blocks per CU: the 64-token stack's gate/up 231-233 us
 *          against 235-242 with one), Q6_K one (four blocks per CU);
 *   narrow (Q4_0 / Q4_1 gate/up and down r < 2, Q6_K gate/up r < 3, Q6_K down r < 2.5): 4 waves,
 *          4 row groups x 1 slot group of 2 pairs (128 rows x 4 slots), two buffers (Q6_K down:
 *          one). With the double-buffered mid blocks, Q4_0 narrow / mid (us, gate/up, down):
 *          126-131 / 133, 64-66 / 67 at r = 1; 165 / 165-166, 82 / 82 at 1.5; 188 / 186-187,
 *          92 / 91 at 2; 207-208 / 201-202, 100.5 / 97 at 2.5.
 * Measured per layer at the 235B shape with one-buffer mid blocks (us): gate/up narrow / mid 166 / 178 at r = 1.5, 187 /
 * 199 at 2, 236 / 237 at 3, 287 / 269 at 4; mid / 8-slot blocks of 8 waves 317-325 / 364-378 at
 * 6; mid / wide 407-416 / 460-467 at 8, 571-620 / 581-593 at 12 (run to run), 765-786 / 723-751
 * at 16. Down narrow / mid: Q4_0 89 / 100 at 1.5, 124 / 133 at 3, 154 / 150 at 4; Q6_K 198 /
 * 200 at 1.5, 223 / 223 at 2, 288 / 271 at 3. Down mid / wide: Q4_0 193 / 229 at 8, 271 / 288 at
 * 12, 373 / 375 at 16; Q6_K 362 / 460 at 8, 496 / 549 at 12, 701 / 719 at 16. */
constexpr int kMxWideSlots = 16;
constexpr int kMxWideSlotsGateUp = 12;
enum MxShape { kMxNarrow, kMxMid, kMxWide, kMxWide16 };

static MxShape mx_shape(const Shape &s, int T, int gu, int type)
{
    const long NS = (long)T * s.K, act = s.X < NS ? s.X : NS;
    const long wide_slots = gu ? kMxWideSlotsGateUp : kMxWideSlots;
    if (type != 14 && QMSG_MX_WIDE16_SLOTS > 0 && NS >= QMSG_MX_WIDE16_SLOTS * act) return kMxWide16;
    if (NS >= wide_slots * act) return kMxWide;
    const long narrow_quarters = type == 14 ? (gu ? 12 : 10) : (gu ? QMSG_MX_NARROW_GU : QMSG_MX_NARROW_DN);
    return 4 * NS < narrow_quarters * act ? kMxNarrow : kMxMid;
}

template <int TYPE, int GU, int WSG, int PPW, int NW, int NB = 2, int NT = 2>
static void launch_mx_shape(const MxArgs &a, int rows, int maxt, hipStream_t st)
{
    using Lay = MxLayout<TYPE, WSG, PPW, NW, NT>;
    const size_t lds = (size_t)mx_lds_bytes(TYPE, WSG, PPW, NW, NB, NT);
    QLAUNCH(GU ? "gateup" : "down", (mx_kernel<TYPE, WSG, GU, PPW, NW, NB, NT>),
            dim3(rows / (GU ? Lay::RWG / 2 : Lay::RWG), maxt, kTileN / Lay::SWG), dim3(64 * NW), lds, st, a);
}

/* Other shapes of the same kernel measured at the 512-token prefill: 32-slot blocks of 16
 * waves (one per CU) 1.76 ms for gate/up, 64-row blocks of 4 waves (three per CU) 1.25,
 * against 1.24 for the wide blocks.
 * Staging buffers: the 8-slot blocks of 4 waves, and the 4-slot Q6_K down blocks, stage one
 * chunk at a time (half the LDS, so four blocks share a CU instead of two or three: the waves of
 * other blocks cover each block's copy); the others double-buffer. Measured at the 235B shape,
 * one buffer against two: Q6_K down 236 / 303 us at 4 slots per expert, 124 / 154 at 1 slot;
 * Q4_0 down 129 / 148 at 4 slots, 72.5 / 70.6 at 1 slot; the 4-slot gate/up blocks 297 / 287 at
 * 4 slots; the wide blocks 481 / 463 (Q6_K down) and 510 / 455 (gate/up) at 8 slots. */
template <int TYPE, int GU>
static void launch_mx(const MxArgs &a, int rows, int maxt, MxShape shape, hipStream_t st)
{
    if (shape == kMxWide) launch_mx_shape<TYPE, GU, 2, 4, 8>(a, rows, maxt, st);
    else if (shape == kMxWide16) {
        /* Q4_0 / Q4_1 only (mx_shape) */
        if constexpr (TYPE != 14 && QMSG_MX_WIDE16_NT == 1)
            launch_mx_shape<TYPE, GU, 1, 8, QMSG_MX_WIDE16_NW, GU ? QMSG_MX_WIDE16_NB_GU : QMSG_MX_WIDE16_NB_DN, 1>(
                a, rows, maxt, st);
        else if constexpr (TYPE != 14)
            launch_mx_shape<TYPE, GU, 1, 8, 4, GU ? QMSG_MX_WIDE16_NB_GU : QMSG_MX_WIDE16_NB_DN>(a, rows, maxt, st);
    }
    else if (shape == kMxNarrow) launch_mx_shape<TYPE, GU, 1, 2, 4, (!GU && TYPE == 14) ? 1 : 2>(a, rows, maxt, st);
    else launch_mx_shape<TYPE, GU, 1, 4, 4, TYPE == 14 ? QMSG_MX_MID_NB_Q6 : QMSG_MX_MID_NB>(a, rows, maxt, st);
}

/* Whether the MFMA kernels take this layer: gate and up of one type (Q4_0, Q4_1, or Q6_K with
 * rows a multiple of 4 bytes long); Q4_0, Q4_1 or Q6_K down (Q6_K
 * rows a multiple of 4 bytes long); 32-blocks in whole chunks; rows in whole blocks' tiles. */
bool mx_supported(const Shape &s, const LayerDev &L, int *down_mx)
{
    const int nbE = s.E / 32, nbF = s.F / 32;
    const bool gu = L.gate_type == L.up_type &&
                    (L.gate_type == 2 || L.gate_type == 3 || (L.gate_type == 14 && L.gate_rb % 4 == 0)) &&
                    nbE % kMxC == 0 && s.F % 128 == 0 && (uint64_t)s.F * L.gate_rb < (1ull << 31);
    const bool dn = (L.down_type == 2 || L.down_type == 3 || (L.down_type == 14 && L.down_rb % 4 == 0)) &&
                    nbF % kMxC == 0 && s.E % 256 == 0 && (uint64_t)s.E * L.down_rb < (1ull << 31);
    if (down_mx) *down_mx = dn;
    return gu;
}

hipError_t launch_experts_mx(const Shape &s, const LayerDev &L, const Scratch &S, float *out, int T, int debug,
                             hipStream_t st)
{
    int down_mx = 0;
    if (!mx_supported(s, L, &down_mx)) return hipErrorInvalidValue;
    const int NS = T * s.K, maxt = (s.X < NS ? s.X : NS) + NS / kTileN + 1;
    const int nx = T * (s.E / 32);
    QLAUNCH("mxin", mx_input_kernel, dim3((nx + 255) / 256), dim3(256), 0, st, S.xq, nx, S.mxx, S.mxflag, S.epoch,
            L.gate_type != 14 ? 1 : 0);
    MxArgs a;
    a.w0 = L.gate;
    a.w1 = L.up;
    a.rb = L.gate_rb;
    a.eb = L.gate_eb;
    a.E = s.E;
    a.F = s.F;
    a.debug = debug;
    a.rec = S.mxx;
    a.rec_out = S.mxa;
    a.rec_out_hi16 = L.down_type != 14 ? 1 : 0;
    a.S = S;
    if (L.gate_type == 14) launch_mx<14, 1>(a, s.F, maxt, mx_shape(s, T, 1, 14), st);
    else if (L.gate_type == 3) launch_mx<3, 1>(a, s.F, maxt, mx_shape(s, T, 1, 3), st);
    else launch_mx<2, 1>(a, s.F, maxt, mx_shape(s, T, 1, 2), st);
    if (!down_mx) {
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        return launch_down_exact(s, L, S, out, T, 0, st);    /* on the aqk records written above */
    }
    a.w0 = L.down;
    a.w1 = nullptr;
    a.rb = L.down_rb;
    a.eb = L.down_eb;
    a.rec = S.mxa;
    a.rec_out = nullptr;
    a.rec_out_hi16 = 0;
    if (L.down_type == 14) launch_mx<14, 0>(a, s.E, maxt, mx_shape(s, T, 0, 14), st);
    else if (L.down_type == 3) launch_mx<3, 0>(a, s.E, maxt, mx_shape(s, T, 0, 3), st);
    else launch_mx<2, 0>(a, s.E, maxt, mx_shape(s, T, 0, 2), st);
    const int n = T * s.E;
    QLAUNCH("combine", combine_kernel, dim3(n / (4 * combine_threads(s.E))), dim3(combine_threads(s.E)), 0, st, S, s.E, s.K, T, out);
    return hipGetLastError();
}

/* Down on the MFMA kernels after the row kernels' gate/up (which leave act in scratch): the
 * activation blocks and their MFMA records in one pass, the down tiles, the combine. */
hipError_t launch_down_mx(const Shape &s, const LayerDev &L, const Scratch &S, float *out, int T, hipStream_t st)
{
    int down_mx = 0;
    (void)mx_supported(s, L, &down_mx);
    if (!down_mx) return hipErrorInvalidValue;
    const int NS = T * s.K, maxt = (s.X < NS ? s.X : NS) + NS / kTileN + 1;
    const int nq = NS * (s.F / 32);
    QLAUNCH("actq", act_quant_kernel, dim3((nq + 255) / 256), dim3(256), 0, st, S, s.F, NS, S.mxa,
            L.down_type != 14 ? 1 : 0);
    MxArgs a;
    a.w0 = L.down;
    a.w1 = nullptr;
    a.rb = L.down_rb;
    a.eb = L.down_eb;
    a.E = s.E;
    a.F = s.F;
    a.debug = 0;
    a.rec = S.mxa;
    a.rec_out = nullptr;
    a.rec_out_hi16 = 0;
    a.S = S;
    if (L.down_type == 14) launch_mx<14, 0>(a, s.E, maxt, mx_shape(s, T, 0, 14), st);
    else if (L.down_type == 3) launch_mx<3, 0>(a, s.E, maxt, mx_shape(s, T, 0, 3), st);
    else launch_mx<2, 0>(a, s.E, maxt, mx_shape(s, T, 0, 2), st);
    const int n = T * s.E;
    QLAUNCH("combine", combine_kernel, dim3(n / (4 * combine_threads(s.E))), dim3(combine_threads(s.E)), 0, st, S, s.E, s.K, T, out);
    return hipGetLastError();
}

/* ------------------------------------------------------------------ dense rows (trunk) ---- */

/* The int8 pair records of T input rows of C floats (src/quant.c:151-154: qms_quantize_q8 of
 * every row), once, for batches where every dense block forming them itself costs more than
 * a launch: one thread per 32-block. */
__global__ void dense_quant_kernel(const float *x, int C, int T, uint8_t *xqk)
{
    const int nb = C >> 5;
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= T * nb) return;
    const int t = b / nb, blk = b - t * nb;
    float v[32];
    const float4 *src = (const float4 *)(x + (size_t)t * C + (size_t)blk * 32);
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const float4 f = src[j];
        v[4 * j] = f.x; v[4 * j + 1] = f.y; v[4 * j + 2] = f.z; v[4 * j + 3] = f.w;
    }
    store_pair_half(quantize_block(v), (uint32_t *)(xqk + ((size_t)t * (nb >> 1) + (blk >> 1)) * kPairBytes), blk & 1);
}

/* qms_matmul_n's fast loop (src/quant.c:151-169) over up to kDenseMats matrices of one type
 * sharing cols: every input row quantised to int8 blocks (qms_quantize_q8), then y_i[t][r] =
 * qms_vec_dot_q8(row r of W_i, xq_t). Block b covers rows 16W*(b - first_i) .. +16W-1 of the
 * matrix i whose block range holds b; wave w owns 16 of them (one per lane quad) and streams
 * exactly those rows in chunks of CB blocks, D chunks in flight, through its own LDS buffer,
 * as the expert kernels do. With a.xqk NULL the block quantises the input rows itself, NT
 * tokens per pass, straight into LDS pair records while its first chunks are on the way (no
 * separate launch: the choice below kDenseQuantT tokens); otherwise it copies the records
 * dense_quant_kernel formed.
 * Rows past the matrix's end load its last row and store nothing. */
template <int TYPE, int W, int NT, int CB, int D>
__global__ __launch_bounds__(64 * W) void dense_kernel(DenseArgs a)
{
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int BB = TYPE == 3 ? 20 : 18;           /* bytes per 32-block                   */
    constexpr int NTH = 64 * W;
    constexpr int SPR = CB * BB / 16;                 /* 16-byte slots per row per chunk      */
    constexpr int NSL = 16 * SPR;                     /* slots of one wave's chunk            */
    constexpr int SPT = (NSL + 63) / 64;              /* slots per lane per chunk             */
    constexpr int WS = CB * BB + ((SPR & 1) ? 0 : 16);/* LDS row stride, odd in 16-byte units */
    const int nb = a.C >> 5, nP = nb >> 1, nchunk = nb / CB;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, qd = lane >> 2, p = lane & 3;
    uint8_t *wbuf = smem + wave * 16 * WS;
    uint8_t *xbuf = smem + W * 16 * WS;

    int mi = 0;
#pragma unroll
    for (int i = 1; i < kDenseMats; i++)
        if (i < a.nm && (int)blockIdx.x >= a.m[i].first_block) mi = i;
    const DenseMat M = a.m[mi];
    const int rw = ((int)blockIdx.x - M.first_block) * 16 * W + 16 * wave;   /* this wave's first row */
    const uint8_t *wbase = M.w + (size_t)min(rw, M.rows - 1) * a.rb;
    const int last = M.rows - 1 - min(rw, M.rows - 1);                      /* rows of this wave - 1 */
    u32x4 wv[D][SPT];
    auto load_chunk = [&](int c, u32x4 *dst) {
#pragma unroll
        for (int m = 0; m < SPT; m++) {
            const int i = min(lane + 64 * m, NSL - 1), row = i / SPR, j = i - row * SPR;
            dst[m] = *(const u32x4 *)(wbase + (size_t)min(row, last) * a.rb + (size_t)c * CB * BB + 16 * j);
        }
    };
    const int row = rw + qd;
    for (int t0 = 0; t0 < a.T; t0 += NT) {
        const int nt = min(NT, a.T - t0);
#pragma unroll
        for (int d = 0; d < D; d++)
            if (d < nchunk) load_chunk(d, wv[d]);
        if (t0 > 0) __syncthreads();                  /* the previous pass is done with xbuf  */
        if (a.xqk) {                                  /* records formed by dense_quant_kernel */
            for (int i = tid; i < nt * nP * 6; i += NTH)
                ((u32x4 *)xbuf)[i] = ((const u32x4 *)(a.xqk + (size_t)t0 * nP * kPairBytes))[i];
        }
        for (int i = a.xqk ? nt * nb : tid; i < nt * nb; i += NTH) {
            const int n = i / nb, blk = i - n * nb;
            float v[32];
            const float4 *src = (const float4 *)(a.x + (size_t)(t0 + n) * a.C + (size_t)blk * 32);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float4 f = src[j];
                v[4 * j] = f.x; v[4 * j + 1] = f.y; v[4 * j + 2] = f.z; v[4 * j + 3] = f.w;
            }
            store_pair_half(quantize_block(v), (uint32_t *)(xbuf + ((size_t)n * nP + (blk >> 1)) * kPairBytes), blk & 1);
        }
        __syncthreads();
        RowAcc acc[NT];
        for (int n = 0; n < NT; n++) acc[n] = RowAcc{ 0.0f, 0.0f, 0.0f };
        for (int c0 = 0; c0 < nchunk; c0 += D) {
#pragma unroll
            for (int d = 0; d < D; d++) {
                const int c = c0 + d;
                if (c < nchunk) {
                    wave_sync();
#pragma unroll
                    for (int m = 0; m < SPT; m++) {
                        const int i = min(lane + 64 * m, NSL - 1), r = i / SPR, j = i - r * SPR;
                        *(u32x4 *)(wbuf + r * WS + 16 * j) = wv[d][m];
                    }
                    wave_sync();
                    if (c + D < nchunk) load_chunk(c + D, wv[d]);
                    if (TYPE == 3)
                        q4_1_rows<NT, (NT >= 4 ? 1 : (NT == 2 ? 2 : 4))>((const uint32_t *)(wbuf + qd * WS), p, xbuf,
                                                                          (size_t)nP * kPairBytes, c * (CB / 2),
                                                                          CB / 2, nt, acc);
                    else
                        q4_0_rows<NT, (NT >= 4 ? 1 : (NT == 2 ? 2 : 4))>((const uint32_t *)(wbuf + qd * WS), p, xbuf,
                                                                          (size_t)nP * kPairBytes, c * (CB / 2),
                                                                          CB / 2, nt, acc);
                }
            }
        }
#pragma unroll
        for (int n = 0; n < NT; n++) {
            const float v = quad_finish(acc[n], finish_scale(TYPE));
            if (p == 0 && n < nt && row < M.rows) M.y[(size_t)(t0 + n) * M.rows + row] = v;
        }
    }
}

/* One block pair of a Q4_0 (TYPE 2) or Q4_1 (TYPE 3) row for lane k of an octet: the lane keeps
 * the reference's FMA chain k (elements 4k..4k+3 of each block, src/kernels.c:82-94, 109-121)
 * and the offset chain. */
/* The LDS words one lane of an octet needs for a pair of 32-blocks, then its arithmetic:
 * split so that a loop can request the next pairs before summing the current one. */
struct OctIn {
    XPair x;
    uint32_t c0, c1, wa, wb;
};

template <int TYPE>
__device__ __forceinline__ OctIn oct_load(const uint32_t *W, int k, const uint8_t *xp)
{
    const int p = k & 3;
    OctIn r;
    r.x = x_load(xp, p);
    if (TYPE == 3) {
        const Q41Pair w = q4_1_load(W, p);
        r.c0 = w.c0; r.c1 = w.c1; r.wa = w.w0; r.wb = w.w5;
    } else {
        const Q4Pair w = q4_0_load(W, p);
        r.c0 = w.c0; r.c1 = w.c1; r.wa = w.w0; r.wb = w.w4;
    }
    return r;
}

template <int TYPE>
__device__ __forceinline__ void oct_math(const OctIn &in, int k, float &acc, float &corr)
{
    const int hi = k >> 2;
    const XPair &x = in.x;
    const uint32_t xb = hi ? x.q.y : x.q.x, xb1 = hi ? x.q.w : x.q.z;
    const uint32_t c0 = in.c0, c1 = in.c1, wa = in.wa, wb = in.wb;
    const uint32_t n0 = (hi ? c0 >> 4 : c0) & 0x0f0f0f0fu, n1 = (hi ? c1 >> 4 : c1) & 0x0f0f0f0fu;
    const int s0 = sdot4((int)n0, (int)xb), s1 = sdot4((int)n1, (int)xb1);
    float m0, m1, o0, o1;
    if (TYPE == 3) {
        m0 = mul_f16_f32<0>(wa, x.d.x);
        m1 = mul_f16_f32<0>(wb, x.d.z);
        o0 = h2f(wa >> 16);
        o1 = h2f(wb >> 16);
    } else {
        m0 = mul_f16_f32<0>(wa, x.d.x);
        m1 = mul_f16_f32<1>(wb, x.d.z);
        o0 = h2f(wa & 0xffffu);
        o1 = h2f(wb >> 16);
    }
    acc = __builtin_fmaf((float)s0, m0, acc);
    corr = __builtin_fmaf(o0, x.d.y, corr);
    acc = __builtin_fmaf((float)s1, m1, acc);
    corr = __builtin_fmaf(o1, x.d.w, corr);
}

template <int TYPE>
__device__ __forceinline__ void oct_pair(const uint32_t *W, int k, const uint8_t *xp, float &acc, float &corr)
{
    oct_math<TYPE>(oct_load<TYPE>(W, k, xp), k, acc, corr);
}

/* hsum256 over the octet (s_j = a_j + a_{j+4}, then (s0+s2)+(s1+s3)) and the unfused offset
 * term, as quad_finish. Valid on lane k == 0. */
__device__ __forceinline__ float oct_finish(float acc, float corr, float scale)
{
    const float s = acc + __shfl_down(acc, 4, 8);
    const float t = s + __shfl_down(s, 2, 8);
    const float h = t + __shfl_down(t, 1, 8);
    return h - scale * corr;
}

/* One-token dense products: as dense_kernel, but eight lanes per row (one per reference lane
 * chain), so a wave streams 8 rows and a launch has twice the waves, each with half the bytes.
 * The trunk's one-token launches have few rows (attn_k/v: 512), and each wave's stream is a
 * serial chain of chunk waits, so more and shorter streams finish sooner. */

/* Q6_K super-block s of a row's chunk in LDS for octet lane k, against the chunk's pair
 * records xc: the lane's chain of dot_q6_k (src/kernels.c:148-167) takes bytes 4k..4k+3 of
 * each 32-block's codes with sub-scale sc[2g] (k < 4) or sc[2g+1] (k >= 4); the offset chain
 * (corr) runs on every lane alike. For each of the nt <= NT tokens (records xs bytes apart)
 * a half's words are all requested before its arithmetic; the weight words are read once.
 * AL: the super-block starts at a multiple of 4 bytes. */
template <bool AL, int NT>
__device__ __forceinline__ void q6_k_oct(const uint8_t *Wr, int s, int k, const uint8_t *xc, size_t xs, int nt,
                                         float *acc, float *corr)
{
    const int p = k & 3, hi = k >> 2;
    const uint32_t sb = (uint32_t)(s * 210);
    const float d = h2f(*(const uint16_t *)(Wr + sb + 208));
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const uint32_t ql0 = lds_word<AL>(Wr, sb + 64 * h + 4 * k), ql1 = lds_word<AL>(Wr, sb + 64 * h + 32 + 4 * k);
        const uint32_t qh = lds_word<AL>(Wr, sb + 128 + 32 * h + 4 * k);
        const uint32_t sc0 = lds_word<AL>(Wr, sb + 192 + 8 * h), sc1 = lds_word<AL>(Wr, sb + 196 + 8 * h);
#pragma unroll
        for (int n = 0; n < NT; n++) {
            if (n >= nt) break;
            const uint8_t *xp = xc + n * xs + (size_t)(4 * s + 2 * h) * kPairBytes;   /* blocks 8s+4h .. +3 */
            uint32_t xq[4];
            float4 xd[2];
            uint2 x16[2];
#pragma unroll
            for (int g = 0; g < 4; g++)
                xq[g] = *(const uint32_t *)(xp + (g >> 1) * kPairBytes + 16 * p + 8 * (g & 1) + 4 * hi);
#pragma unroll
            for (int j = 0; j < 2; j++) {
                xd[j] = *(const float4 *)(xp + j * kPairBytes + 64);
                x16[j] = *(const uint2 *)(xp + j * kPairBytes + 80);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const uint32_t ql = (g & 1) ? ql1 : ql0;
                const uint32_t nib = g < 2 ? (ql & 0x0f0f0f0fu) : ((ql >> 4) & 0x0f0f0f0fu);
                const uint32_t q6 = nib | (((qh >> (2 * g)) & 0x03030303u) << 4);
                const uint32_t scw = (g < 2 ? sc0 : sc1) >> (16 * (g & 1));
                const int sa = (int)(int8_t)(scw & 0xff), sbv = (int)(int8_t)((scw >> 8) & 0xff);
                const float xdv = (g & 1) ? xd[g >> 1].z : xd[g >> 1].x;
                const uint32_t s16 = (g & 1) ? x16[g >> 1].y : x16[g >> 1].x;
                const int s16a = (int)(int16_t)(s16 & 0xffffu), s16b = (int)(int16_t)(s16 >> 16);
                const float dd = d * xdv;
                acc[n] = __builtin_fmaf((float)(sdot4((int)q6, (int)xq[g]) * (hi ? sbv : sa)), dd, acc[n]);
                corr[n] = __builtin_fmaf(dd, (float)(sa * s16a + sbv * s16b), corr[n]);
            }
        }
    }
}

template <int TYPE, int CB, int D, int W, int NT = 1>
__global__ __launch_bounds__(64 * W) void dense_oct_kernel(DenseArgs a)
{
    static_assert(NT == 1 || TYPE == 14, "several tokens only for Q6_K rows");
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int BB = TYPE == 3 ? 20 : 18;           /* bytes per 32-block (Q4_0, Q4_1)      */
    /* one row's chunk: CB 32-blocks (Q6_K: CB/8 super-blocks, CB = 64 keeps 16-byte slots) */
    constexpr int RCB = TYPE == 14 ? CB / 8 * 210 : CB * BB;
    constexpr int SPR = RCB / 16;                     /* 16-byte slots per row per chunk      */
    static_assert(RCB % 16 == 0, "chunk rows are whole 16-byte slots");
    constexpr int NSL = 8 * SPR;                      /* slots of the wave's chunk            */
    constexpr int SPT = (NSL + 63) / 64;              /* slots per lane per chunk             */
    constexpr int WS = RCB + ((SPR & 1) ? 0 : 16);    /* LDS row stride, odd in 16-byte units */
    constexpr int NTH = 64 * W;
    const int nb = a.C >> 5, nP = nb >> 1, nchunk = nb / CB;
    const int tid = threadIdx.x, lane = tid & 63, rr = lane >> 3, k = lane & 7;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    uint8_t *wbuf = smem + wave * 8 * WS;
    uint8_t *xbuf = smem + W * 8 * WS;                /* [a.T][nP][96]                        */
    const int nqb = a.T * nb;                         /* input 32-blocks of every token       */

    int mi = 0;
#pragma unroll
    for (int i = 1; i < kDenseMats; i++)
        if (i < a.nm && (int)blockIdx.x >= a.m[i].first_block) mi = i;
    const DenseMat M = a.m[mi];
    const int rw = ((int)blockIdx.x - M.first_block) * 8 * W + 8 * wave;   /* the wave's first row */
    const uint8_t *wbase = M.w + (size_t)min(rw, M.rows - 1) * a.rb;
    const int last = M.rows - 1 - min(rw, M.rows - 1);
    u32x4 wv[D][SPT];
    auto load_chunk = [&](int c, u32x4 *dst) {
#pragma unroll
        for (int m = 0; m < SPT; m++) {
            const int i = min(lane + 64 * m, NSL - 1), row = i / SPR, j = i - row * SPR;
            dst[m] = *(const u32x4 *)(wbase + (size_t)min(row, last) * a.rb + (size_t)c * RCB + 16 * j);
        }
    };
    /* the input row first, then the weights: loads complete in order, so quantising the row
     * waits only for its own bytes while the first chunks are still on the way. The block's
     * W waves share one quantisation of the row (one 32-block per thread, then any rest). */
    float4 xr[8];
    {
        const float4 *src = (const float4 *)(a.x + (size_t)min(tid, nqb - 1) * 32);
#pragma unroll
        for (int j = 0; j < 8; j++) xr[j] = src[j];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int d = 0; d < D; d++)
        if (d < nchunk) load_chunk(d, wv[d]);
    __builtin_amdgcn_sched_barrier(0);
    if (tid < nqb) {
        float v[32];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            v[4 * j] = xr[j].x; v[4 * j + 1] = xr[j].y; v[4 * j + 2] = xr[j].z; v[4 * j + 3] = xr[j].w;
        }
        const int n = tid / nb, blk = tid - n * nb;
        store_pair_half(quantize_block(v), (uint32_t *)(xbuf + ((size_t)n * nP + (blk >> 1)) * kPairBytes), blk & 1);
    }
    for (int b = tid + NTH; b < nqb; b += NTH) {      /* rows longer than one block per thread */
        float v[32];
        const float4 *src = (const float4 *)(a.x + (size_t)b * 32);
        for (int j = 0; j < 8; j++) {
            const float4 f = src[j];
            v[4 * j] = f.x; v[4 * j + 1] = f.y; v[4 * j + 2] = f.z; v[4 * j + 3] = f.w;
        }
        const int n = b / nb, blk = b - n * nb;
        store_pair_half(quantize_block(v), (uint32_t *)(xbuf + ((size_t)n * nP + (blk >> 1)) * kPairBytes), blk & 1);
    }
    if (W > 1) __syncthreads();
    else wave_sync();
    float acc[NT], corr[NT];
#pragma unroll
    for (int n = 0; n < NT; n++) acc[n] = corr[n] = 0.0f;
    for (int c0 = 0; c0 < nchunk; c0 += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            const int c = c0 + d;
            if (c < nchunk) {
                wave_sync();
#pragma unroll
                for (int m = 0; m < SPT; m++) {
                    const int i = min(lane + 64 * m, NSL - 1), r = i / SPR, j = i - r * SPR;
                    *(u32x4 *)(wbuf + r * WS + 16 * j) = wv[d][m];
                }
                wave_sync();
                if (c + D < nchunk) load_chunk(c + D, wv[d]);
                if constexpr (TYPE == 14) {
                    const uint8_t *xc = xbuf + (size_t)c * (CB / 2) * kPairBytes;
#pragma unroll 1
                    for (int sbi = 0; sbi < CB / 8; sbi += 2) {   /* even super-blocks 4-aligned */
                        q6_k_oct<true, NT>(wbuf + rr * WS, sbi, k, xc, (size_t)nP * kPairBytes, a.T, acc, corr);
                        q6_k_oct<false, NT>(wbuf + rr * WS, sbi + 1, k, xc, (size_t)nP * kPairBytes, a.T, acc,
                                            corr);
                    }
                } else {
                    const uint32_t *Wrow = (const uint32_t *)(wbuf + rr * WS);
                    /* four pairs' LDS words requested before their arithmetic (one wave per
                     * SIMD leaves each read's latency otherwise exposed) */
                    constexpr int PB = CB / 2 >= 4 ? 4 : CB / 2;
#pragma unroll
                    for (int q0 = 0; q0 < CB / 2; q0 += PB) {
                        OctIn in[PB];
#pragma unroll
                        for (int u = 0; u < PB; u++)
                            in[u] = oct_load<TYPE>(Wrow + (q0 + u) * (BB * 2 / 4), k,
                                                   xbuf + (size_t)(c * (CB / 2) + q0 + u) * kPairBytes);
                        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                        for (int u = 0; u < PB; u++) oct_math<TYPE>(in[u], k, acc[0], corr[0]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int n = 0; n < NT; n++) {
        const float v = oct_finish(acc[n], corr[n], finish_scale(TYPE));
        if (k == 0 && n < a.T && rw + rr < M.rows) M.y[(size_t)n * M.rows + rw + rr] = v;
    }
}

/* Two chunks in flight per wave (2, 4 and 8 were measured at the trunk's shapes: 2 fastest). */
/* Batches of two or more tokens: a block owns 16 rows (one per lane quad) and stages each
 * chunk of them once into LDS for its W waves; wave w computes tokens w*NT .. w*NT+NT-1 of the
 * pass (W*NT tokens per pass, the rows streamed once per pass). A block's waves thus share the
 * weight bytes, and a launch has W times the waves of one wave doing every token, which keeps
 * the per-lane reference chains (src/quant.c:151-169, qms_vec_dot_q8) spread over every SIMD.
 * Chunk c sits in buffer c % D; one block barrier per chunk both publishes it and, with
 * D >= 2, guarantees every wave is done with the chunk that last used that buffer. */
template <int TYPE, int CB, int D, int W, int NT>
__global__ __launch_bounds__(64 * W) void dense_tok_kernel(DenseArgs a)
{
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int BB = TYPE == 3 ? 20 : 18;           /* bytes per 32-block (Q4_0, Q4_1)      */
    /* one row's chunk: CB 32-blocks (Q6_K: CB/8 super-blocks of 210 bytes, CB = 64 keeps it a
     * whole number of 16-byte slots) */
    constexpr int RCB = TYPE == 14 ? CB / 8 * 210 : CB * BB;
    constexpr int NTH = 64 * W, TP = W * NT;
    constexpr int SPR = RCB / 16;                     /* 16-byte slots per row per chunk      */
    static_assert(RCB % 16 == 0, "chunk rows are whole 16-byte slots");
    constexpr int NSL = 16 * SPR;                     /* slots of one chunk (16 rows)         */
    constexpr int SPT = (NSL + NTH - 1) / NTH;        /* slots per thread per chunk           */
    constexpr int WS = RCB + ((SPR & 1) ? 0 : 16);    /* LDS row stride, odd in 16-byte units */
    const int nb = a.C >> 5, nP = nb >> 1, nchunk = nb / CB;
    const int tid = threadIdx.x, lane = tid & 63, qd = lane >> 2, p = lane & 3;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    uint8_t *wbuf = smem;                             /* [D][16][WS]                          */
    uint8_t *xbuf = smem + D * 16 * WS;               /* [TP][nP][96]                         */

    int mi = 0;
#pragma unroll
    for (int i = 1; i < kDenseMats; i++)
        if (i < a.nm && (int)blockIdx.x >= a.m[i].first_block) mi = i;
    const DenseMat M = a.m[mi];
    const int r0 = ((int)blockIdx.x - M.first_block) * 16;
    const uint8_t *wbase = M.w + (size_t)min(r0, M.rows - 1) * a.rb;
    const int last = M.rows - 1 - min(r0, M.rows - 1);
    u32x4 wv[D][SPT];
    auto load_chunk = [&](int c, u32x4 *dst) {
#pragma unroll
        for (int m = 0; m < SPT; m++) {
            const int i = min(tid + NTH * m, NSL - 1), row = i / SPR, j = i - row * SPR;
            dst[m] = *(const u32x4 *)(wbase + (size_t)min(row, last) * a.rb + (size_t)c * RCB + 16 * j);
        }
    };
    const int row = r0 + qd, tw0 = wave * NT;
    for (int t0 = 0; t0 < a.T; t0 += TP) {
        const int ntp = min(TP, a.T - t0), ntw = max(0, min(NT, ntp - tw0));
#pragma unroll
        for (int d = 0; d < D; d++)
            if (d < nchunk) load_chunk(d, wv[d]);
        if (t0 > 0) __syncthreads();                  /* the previous pass is done with LDS   */
        if (a.xqk) {                                  /* records formed by dense_quant_kernel */
            for (int i = tid; i < ntp * nP * 6; i += NTH)
                ((u32x4 *)xbuf)[i] = ((const u32x4 *)(a.xqk + (size_t)t0 * nP * kPairBytes))[i];
        } else {
            for (int i = tid; i < ntp * nb; i += NTH) {
                const int n = i / nb, blk = i - n * nb;
                float v[32];
                const float4 *src = (const float4 *)(a.x + (size_t)(t0 + n) * a.C + (size_t)blk * 32);
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float4 f = src[j];
                    v[4 * j] = f.x; v[4 * j + 1] = f.y; v[4 * j + 2] = f.z; v[4 * j + 3] = f.w;
                }
                store_pair_half(quantize_block(v), (uint32_t *)(xbuf + ((size_t)n * nP + (blk >> 1)) * kPairBytes),
                                blk & 1);
            }
        }
        RowAcc acc[NT];
        for (int n = 0; n < NT; n++) acc[n] = RowAcc{ 0.0f, 0.0f, 0.0f };
        for (int c0 = 0; c0 < nchunk; c0 += D) {
#pragma unroll
            for (int d = 0; d < D; d++) {
                const int c = c0 + d;
                if (c < nchunk) {
                    uint8_t *cb = wbuf + d * 16 * WS;
#pragma unroll
                    for (int m = 0; m < SPT; m++) {
                        const int i = tid + NTH * m;
                        if (i < NSL) {
                            const int r = i / SPR, j = i - r * SPR;
                            *(u32x4 *)(cb + r * WS + 16 * j) = wv[d][m];
                        }
                    }
                    __syncthreads();
                    if (c + D < nchunk) load_chunk(c + D, wv[d]);
                    if (ntw > 0 && TYPE == 14) {
                        /* super-block k of the chunk: Q6_K rows as the expert tile kernel
                         * reads them (an even super-block starts 4-byte aligned: WS and 420
                         * are multiples of 4) */
                        const uint8_t *xw = xbuf + (size_t)tw0 * nP * kPairBytes;
                        auto superblock = [&](auto al, int k) {
                            const uint32_t sb = (uint32_t)(qd * WS + k * 210);
#pragma unroll
                            for (int h = 0; h < 2; h++)
#pragma unroll
                                for (int g = 0; g < 4; g++) {
                                    const int blk = (c * (CB / 8) + k) * 8 + h * 4 + g;
                                    const Q6W w6 = q6_k_weights<decltype(al)::value>(cb, sb, h, g, p);
#pragma unroll
                                    for (int n = 0; n < NT; n++)
                                        if (n < ntw)
                                            q6_k_token(w6, xw + (size_t)n * nP * kPairBytes +
                                                               (size_t)(blk >> 1) * kPairBytes, p, blk & 1, acc[n]);
                                }
                        };
                        /* two super-blocks per iteration: unrolling the chunk's eight
                         * spilled the NT = 2, 4 variants */
#pragma unroll 1
                        for (int k = 0; k < CB / 8; k += 2) {
                            superblock(std::integral_constant<bool, true>(), k);
                            superblock(std::integral_constant<bool, false>(), k + 1);
                        }
                    } else if (ntw > 0) {
                        if (TYPE == 3)
                            q4_1_rows<NT, (NT >= 4 ? 1 : (NT == 2 ? 2 : 4))>((const uint32_t *)(cb + qd * WS), p,
                                                                              xbuf + (size_t)tw0 * nP * kPairBytes,
                                                                              (size_t)nP * kPairBytes, c * (CB / 2),
                                                                              CB / 2, ntw, acc);
                        else
                            q4_0_rows<NT, (NT >= 4 ? 1 : (NT == 2 ? 2 : 4))>((const uint32_t *)(cb + qd * WS), p,
                                                                              xbuf + (size_t)tw0 * nP * kPairBytes,
                                                                              (size_t)nP * kPairBytes, c * (CB / 2),
                                                                              CB / 2, ntw, acc);
                    }
                }
            }
        }
#pragma unroll
        for (int n = 0; n < NT; n++) {
            const float v = quad_finish(acc[n], finish_scale(TYPE));
            if (p == 0 && n < ntw && row < M.rows) M.y[(size_t)(t0 + tw0 + n) * M.rows + row] = v;
        }
    }
}

/* qms_matmul_n's fast loop (src/quant.c:134-169) for the row widths the chunked kernels above
 * do not take: Q4_0 and Q4_1 rows with cols % 256 != 0 and Q6_K rows with cols % 2048 != 0,
 * which the reference's fast path still admits (cols % 32; Q6_K cols % 256); F32 rows of such
 * widths take the router kernels' tail form (launch_f32_rows). A lane group per row reads the
 * row's words straight from memory: eight lanes per quantised row, lane k keeping the
 * reference's FMA chain k (elements 4k..4k+3 of every 32-block) and the offset chain; the
 * per-slot expert form (slot_any_kernel) also takes F32 expert rows, sixteen lanes each, lane
 * c keeping chain c of dot_f32 (elements c, c+16, ...; src/kernels.c:202-213). Up to NT
 * tokens share a pass: their int8 blocks (qms_quantize_q8) sit in LDS as 48-byte records
 * {q[32], d, ds, s16[2], pad}; F32 passes read the inputs from memory. Rows past a matrix's
 * end read its last row and store nothing. No Qwen3-MoE trunk matrix has such a width; this
 * path is for completeness, not speed. */
constexpr int kDenseAnyRec = 48;

__device__ __forceinline__ uint32_t ld_u32_a2(const uint8_t *p)   /* p a multiple of 2 */
{
    const uint16_t *h = (const uint16_t *)p;
    return (uint32_t)h[0] | ((uint32_t)h[1] << 16);
}

/* One pass of a lane group's row (bytes wr, C columns) against nt <= NT input rows, xrow(n)
 * giving row n's C floats (16-byte aligned); res[n] holds the product on lane k == 0 of the
 * group. Every thread of the block calls it (the quantised records are formed block-wide). */
template <int TYPE, int NT, typename XRow>
__device__ __forceinline__ void any_rows_pass(const uint8_t *wr, int C, int nt, int k, XRow xrow, uint8_t *smem,
                                              float *res)
{
    const int tid = threadIdx.x, nb = C >> 5;
    float acc[NT], corr[NT];
#pragma unroll
    for (int n = 0; n < NT; n++) { acc[n] = 0.0f; corr[n] = 0.0f; }
    if constexpr (TYPE == 0) {
        const float *w = (const float *)wr;
        for (int i = k; i < C; i += 16) {
            const float wv = w[i];
#pragma unroll
            for (int n = 0; n < NT; n++)
                if (n < nt) acc[n] = __builtin_fmaf(wv, xrow(n)[i], acc[n]);
        }
    } else {
        __syncthreads();                              /* an earlier pass is done with the records */
        for (int i = tid; i < nt * nb; i += blockDim.x) {
            const int n = i / nb, blk = i - n * nb;
            float v[32];
            const float4 *src = (const float4 *)(xrow(n) + (size_t)blk * 32);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float4 f = src[j];
                v[4 * j] = f.x; v[4 * j + 1] = f.y; v[4 * j + 2] = f.z; v[4 * j + 3] = f.w;
            }
            const Q8Vals q = quantize_block(v);
            uint32_t *o = (uint32_t *)(smem + (size_t)i * kDenseAnyRec);
#pragma unroll
            for (int j = 0; j < 8; j++) o[j] = q.qw[j];
            o[8] = __float_as_uint(q.d);
            o[9] = __float_as_uint(q.ds);
            o[10] = q.s16;
            o[11] = 0;
        }
        __syncthreads();
        auto rec = [&](int n, int blk) { return smem + ((size_t)n * nb + blk) * kDenseAnyRec; };
        if constexpr (TYPE == 14) {
            const int hi = k >> 2;
            for (int s = 0; s < nb / 8; s++) {
                const uint8_t *sp = wr + (size_t)s * 210;
                const float d = h2f(*(const uint16_t *)(sp + 208));
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const uint32_t ql0 = ld_u32_a2(sp + 64 * h + 4 * k), ql1 = ld_u32_a2(sp + 64 * h + 32 + 4 * k);
                    const uint32_t qh = ld_u32_a2(sp + 128 + 32 * h + 4 * k);
                    const uint32_t sc0 = ld_u32_a2(sp + 192 + 8 * h), sc1 = ld_u32_a2(sp + 196 + 8 * h);
#pragma unroll
                    for (int g = 0; g < 4; g++) {
                        const uint32_t ql = (g & 1) ? ql1 : ql0;
                        const uint32_t nib = g < 2 ? (ql & 0x0f0f0f0fu) : ((ql >> 4) & 0x0f0f0f0fu);
                        const uint32_t q6 = nib | (((qh >> (2 * g)) & 0x03030303u) << 4);
                        const uint32_t scw = (g < 2 ? sc0 : sc1) >> (16 * (g & 1));
                        const int sa = (int)(int8_t)(scw & 0xff), sbv = (int)(int8_t)((scw >> 8) & 0xff);
#pragma unroll
                        for (int n = 0; n < NT; n++) {
                            if (n >= nt) break;
                            const uint32_t *xr = (const uint32_t *)rec(n, 8 * s + 4 * h + g);
                            const float dd = d * __uint_as_float(xr[8]);
                            const int s16a = (int)(int16_t)(xr[10] & 0xffffu), s16b = (int)(int16_t)(xr[10] >> 16);
                            acc[n] = __builtin_fmaf((float)(sdot4((int)q6, (int)xr[k]) * (hi ? sbv : sa)), dd, acc[n]);
                            corr[n] = __builtin_fmaf(dd, (float)(sa * s16a + sbv * s16b), corr[n]);
                        }
                    }
                }
            }
        } else {
            constexpr int BB = TYPE == 3 ? 20 : 18;
            for (int b = 0; b < nb; b++) {
                const uint8_t *bp = wr + (size_t)b * BB;
                float d, o;
                uint32_t c;
                if (TYPE == 3) {
                    const uint32_t dm = *(const uint32_t *)bp;      /* 20-byte blocks: 4-byte aligned */
                    d = h2f(dm & 0xffffu);
                    o = h2f(dm >> 16);
                    c = *(const uint32_t *)(bp + 4 + 4 * (k & 3));
                } else {
                    d = h2f(*(const uint16_t *)bp);
                    o = d;
                    c = ld_u32_a2(bp + 2 + 4 * (k & 3));
                }
                const uint32_t nib = (k < 4 ? c : c >> 4) & 0x0f0f0f0fu;
#pragma unroll
                for (int n = 0; n < NT; n++) {
                    if (n >= nt) break;
                    const uint32_t *xr = (const uint32_t *)rec(n, b);
                    acc[n] = __builtin_fmaf((float)sdot4((int)nib, (int)xr[k]), d * __uint_as_float(xr[8]), acc[n]);
                    corr[n] = __builtin_fmaf(o, __uint_as_float(xr[9]), corr[n]);
                }
            }
        }
    }
#pragma unroll
    for (int n = 0; n < NT; n++)
        res[n] = TYPE == 0 ? chain16_sum(acc[n]) : oct_finish(acc[n], corr[n], finish_scale(TYPE));
}

template <int TYPE, int NT>
__global__ __launch_bounds__(256) void dense_any_kernel(DenseArgs a)
{
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int RPW = TYPE == 0 ? 4 : 8;            /* rows per wave  */
    constexpr int LPR = 64 / RPW;                     /* lanes per row  */
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, k = lane % LPR;
    int mi = 0;
#pragma unroll
    for (int i = 1; i < kDenseMats; i++)
        if (i < a.nm && (int)blockIdx.x >= a.m[i].first_block) mi = i;
    const DenseMat M = a.m[mi];
    const int row = ((int)blockIdx.x - M.first_block) * 4 * RPW + wave * RPW + lane / LPR;
    const uint8_t *wr = M.w + (size_t)min(row, M.rows - 1) * a.rb;
    const int C = a.C;
    for (int t0 = 0; t0 < a.T; t0 += NT) {
        const int nt = min(NT, a.T - t0);
        float res[NT];
        any_rows_pass<TYPE, NT>(wr, C, nt, k, [&](int n) { return a.x + (size_t)(t0 + n) * C; }, smem, res);
#pragma unroll
        for (int n = 0; n < NT; n++)
            if (k == 0 && n < nt && row < M.rows) M.y[(size_t)(t0 + n) * M.rows + row] = res[n];
    }
}

/* The same products per slot for MoE layers the integer kernels do not take: shapes off their
 * grid (n_embd % 256 != 0 or n_ff_exp % 64 != 0) and expert tensors of other types. The
 * reference then runs moe_group_exact, whose qms_matmul of each slot's gate, up and down rows
 * takes this int8 path for Q4_0 / Q4_1 / Q6_K rows and dot_f32 for F32 rows (src/model.c:
 * 1009-1030, src/quant.c:134-169; with n_embd % 256 == 0 its moe_group_fast gives the same
 * numbers, src/model.c:969-1006). Block (32 rows, or 16 F32 rows; active expert blockIdx.y) as
 * exact_rows_kernel; the input of slot s is row slot_t[s] of x (by_token) or row s. */
struct SlotAnyArgs {
    const uint8_t *w;
    uint64_t rb, eb;
    int rows, cols, by_token;
    const float *x;
    float *y;
    int y_stride, y_off;
    /* blockIdx.z == 1: a second matrix of the same type, shape and inputs (up beside gate) */
    const uint8_t *w2;
    uint64_t rb2, eb2;
    int y_off2;
    Scratch S;
};

template <int TYPE, int NT>
__global__ __launch_bounds__(256) void slot_any_kernel(SlotAnyArgs a)
{
    extern __shared__ __align__(16) uint8_t smem[];
    if ((int)blockIdx.y >= a.S.meta[0]) return;       /* block-uniform */
    constexpr int RPW = TYPE == 0 ? 4 : 8;            /* rows per wave  */
    constexpr int LPR = 64 / RPW;                     /* lanes per row  */
    const int4 wk = a.S.work[blockIdx.y];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, k = lane % LPR;
    const int row = (int)blockIdx.x * 4 * RPW + wave * RPW + lane / LPR, C = a.cols;
    const bool second = blockIdx.z == 1;
    const int y_off = second ? a.y_off2 : a.y_off;
    const uint8_t *wr = second ? a.w2 + (size_t)wk.x * a.eb2 + (size_t)min(row, a.rows - 1) * a.rb2
                               : a.w + (size_t)wk.x * a.eb + (size_t)min(row, a.rows - 1) * a.rb;
    for (int s0 = wk.y; s0 < wk.z; s0 += NT) {
        const int nt = min(NT, wk.z - s0);
        float res[NT];
        any_rows_pass<TYPE, NT>(wr, C, nt, k, [&](int n) {
            const size_t src = a.by_token ? (size_t)a.S.slot_t[s0 + n] : (size_t)(s0 + n);
            return a.x + src * C;
        }, smem, res);
#pragma unroll
        for (int n = 0; n < NT; n++)
            if (k == 0 && n < nt && row < a.rows) a.y[(size_t)(s0 + n) * a.y_stride + y_off + row] = res[n];
    }
}

/* The weighted sum of combine_kernel for any n_embd: one thread per output element. */
__global__ void combine_any_kernel(const Scratch S, int E, int K, int T, float *out)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)T * E) return;
    const int t = (int)(i / E), r = (int)(i - (size_t)t * E);
    float o = 0.0f;
    for (int j = 0; j < K; j++)
        o = __builtin_fmaf(S.wt[(size_t)t * K + j], S.dn[(size_t)S.slot_of[(size_t)t * K + j] * E + r], o);
    out[i] = o;
}

/* The 44-byte Q8 records of rows of C floats (qms_quantize_q8): the debug copies of the
 * inputs' and activations' int8 blocks where the slot kernels keep theirs in LDS only. */
__global__ void quant_rows_kernel(const float *x, int C, int rows, Q8 *dst)
{
    const int nb = C >> 5;
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= rows * nb) return;
    float v[32];
    const float4 *src = (const float4 *)(x + (size_t)b * 32);
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const float4 f = src[j];
        v[4 * j] = f.x; v[4 * j + 1] = f.y; v[4 * j + 2] = f.z; v[4 * j + 3] = f.w;
    }
    store_q8(quantize_block(v), dst + b);
}

/* Tokens per pass of dense_any_kernel for a batch of T and nb 32-blocks per row: the fewest
 * passes whose records fit 64 KiB of LDS (0: one token's do not fit at all). */
static int dense_any_nt(int type, int T, int nb)
{
    int nt = T <= 1 ? 1 : (T <= 2 ? 2 : (T <= 4 ? 4 : 8));
    if (type == 0) return nt;
    while (nt > 1 && (size_t)nt * nb * kDenseAnyRec > 64 * 1024) nt >>= 1;
    return (size_t)nb * kDenseAnyRec <= 160 * 1024 ? nt : 0;
}

/* Tokens per wave of dense_tok_kernel's passes for a batch of T (four waves per block), and
 * its LDS bytes. */
constexpr int kDenseTokW = 4;
static size_t dense_tok_lds(int NT, int CB, int type, int nb)
{
    const int rcb = type == 14 ? CB / 8 * 210 : CB * (type == 3 ? 20 : 18);
    const size_t ws = (size_t)rcb + (((rcb / 16) & 1) ? 0 : 16);
    return 2 * 16 * ws + (size_t)kDenseTokW * NT * (nb / 2) * kPairBytes;
}

template <int TYPE, int NT>
static void launch_dense_t(const DenseArgs &a, int CB, dim3 grid, size_t lds, hipStream_t st)
{
    if (CB == 16) QLAUNCH("dense", (dense_kernel<TYPE, 1, NT, 16, 2>), grid, dim3(64), lds, st, a);
    else QLAUNCH("dense", (dense_kernel<TYPE, 1, NT, 8, 2>), grid, dim3(64), lds, st, a);
}

/* y[t][r] (row stride ystride) = dot_f32 of F32 row r of w [rows][C] with x[t] for T tokens
 * (src/kernels.c:202-221, sixteen chains), for rows of any multiple of 32 floats: one token
 * takes a block per row (rows of a multiple of 256 floats up to 4096) or 4 rows per block;
 * more tokens 16 rows x 16 tokens per block, so each row is read once per 16 tokens (a block
 * per row and token group re-read the rows, measured 5x slower at 4). Rows off the 256-float
 * grid take the chunked kernel's tail form. */
hipError_t launch_f32_rows(const float *w, int rows, int C, const float *x, int T, float *y, int ystride,
                           const char *name, hipStream_t st)
{
    RouteArgs r;
    r.router = w;
    r.xn = x;
    r.E = C;
    r.X = rows;
    r.K = 0;
    r.T = T;
    r.y = y;
    r.ystride = ystride;
    r.S = Scratch{};
    const bool tail = C % 256 != 0;
    if (T == 1 && C <= 4096 && !tail) {
        r.n_route_wg = rows;
        const size_t lds = (size_t)2 * 16 * (C / 16 + 4) * 4;
        QLAUNCH(name, route_small_kernel<1>, dim3(rows), dim3(256), lds, st, r);
    } else if (T == 1) {
        r.n_route_wg = (rows + 3) / 4;
        if (tail) QLAUNCH(name, (route_big_kernel<1, 1, kRouteBigP, true>), dim3(r.n_route_wg), dim3(256), route_big_lds(1), st, r);
        else QLAUNCH(name, (route_big_kernel<1, 1, kRouteBigP>), dim3(r.n_route_wg), dim3(256), route_big_lds(1), st, r);
    } else {
        r.n_route_wg = ((T + 15) / 16) * ((rows + 15) / 16);
        if (tail) QLAUNCH(name, (route_big_kernel<4, 4, kRouteBigP, true>), dim3(r.n_route_wg), dim3(256), route_big_lds(4), st, r);
        else QLAUNCH(name, (route_big_kernel<4, 4, kRouteBigP>), dim3(r.n_route_wg), dim3(256), route_big_lds(4), st, r);
    }
    return hipGetLastError();
}

hipError_t launch_dense(const DenseArgs &args, int type, uint8_t *xqk, hipStream_t st)
{
    DenseArgs a = args;
    const int nb = a.C / 32;
    if (type != 0 && (type == 14 ? nb % 64 != 0 : nb % 8 != 0)) {
        /* widths the chunked kernels do not take: one direct-read pass per NT tokens */
        const int NT = dense_any_nt(type, a.T, nb);
        if (!NT) return hipErrorInvalidValue;
        const int rpb = 32;
        int nblk = 0;
        for (int i = 0; i < a.nm; i++) {
            a.m[i].first_block = nblk;
            nblk += (a.m[i].rows + rpb - 1) / rpb;
        }
        const size_t lds = (size_t)NT * nb * kDenseAnyRec;
        auto go = [&](auto ty) {
            constexpr int TY = decltype(ty)::value;
            if (NT == 8) QLAUNCH("dense", (dense_any_kernel<TY, 8>), dim3(nblk), dim3(256), lds, st, a);
            else if (NT == 4) QLAUNCH("dense", (dense_any_kernel<TY, 4>), dim3(nblk), dim3(256), lds, st, a);
            else if (NT == 2) QLAUNCH("dense", (dense_any_kernel<TY, 2>), dim3(nblk), dim3(256), lds, st, a);
            else QLAUNCH("dense", (dense_any_kernel<TY, 1>), dim3(nblk), dim3(256), lds, st, a);
        };
        if (type == 14) go(std::integral_constant<int, 14>());
        else if (type == 3) go(std::integral_constant<int, 3>());
        else go(std::integral_constant<int, 2>());
        return hipGetLastError();
    }
    if (type == 0) {
        /* F32 rows: qms_vec_dot_f32 (src/quant.c:161-163, src/kernels.c:202-221), the router's
         * arithmetic; one launch per matrix */
        for (int i = 0; i < a.nm; i++) {
            const hipError_t e = launch_f32_rows((const float *)a.m[i].w, a.m[i].rows, a.C, a.x, a.T, a.m[i].y,
                                                 a.m[i].rows, "dense", st);
            if (e != hipSuccess) return e;
        }
        return hipGetLastError();
    }
    a.xqk = nullptr;
    if (a.T >= kDenseQuantT && xqk) {
        QLAUNCH("dquant", dense_quant_kernel, dim3((a.T * nb + 255) / 256), dim3(256), 0, st, a.x, a.C, a.T, xqk);
        a.xqk = xqk;
    }
    /* one wave per block, 16 rows each: the trunk's small matrices (attn_k/v: 512 rows) still
     * spread over 32 CUs, the large ones over every CU */
    /* eight lanes per row, 8 rows per wave: one token, or Q6_K rows for two or three (each
     * super-block's weight words read once for all of them: trunk layer 81.9 -> 56.3 us at
     * T = 2, 85.4 -> 74.6 at T = 3; at T = 4 the token-parallel kernel is faster, 85.6
     * against 90.6) */
    if ((a.T == 1 && (type != 14 || nb % 64 == 0)) || (type == 14 && a.T <= 3 && nb % 64 == 0)) {
        /* W waves per block share the input row's quantisation: the most that still gives
         * every CU a block */
        int rows = 0;
        for (int i = 0; i < a.nm; i++) rows += a.m[i].rows;
        const int W = rows >= 256 * 32 ? 4 : (rows >= 256 * 16 ? 2 : 1);
        int nbw = 0;
        for (int i = 0; i < a.nm; i++) {
            a.m[i].first_block = nbw;
            nbw += (a.m[i].rows + 8 * W - 1) / (8 * W);
        }
        const int CB = type == 14 ? 64 : (nb % 16 == 0 ? 16 : 8);
        const int rcb = type == 14 ? CB / 8 * 210 : CB * (type == 3 ? 20 : 18);
        const size_t ws = (size_t)rcb + (((rcb / 16) & 1) ? 0 : 16);
        const size_t lds8 = (size_t)W * 8 * ws + (size_t)a.T * (nb / 2) * kPairBytes;
        if (lds8 > 160 * 1024) return hipErrorInvalidValue;
        auto go = [&](auto tw) {
            constexpr int WW = decltype(tw)::value;
            if (type == 14) {
                if (a.T == 1) QLAUNCH("dense", (dense_oct_kernel<14, 64, 2, WW>), dim3(nbw), dim3(64 * WW), lds8, st, a);
                else if (a.T == 2)
                    QLAUNCH("dense", (dense_oct_kernel<14, 64, 2, WW, 2>), dim3(nbw), dim3(64 * WW), lds8, st, a);
                else QLAUNCH("dense", (dense_oct_kernel<14, 64, 2, WW, 4>), dim3(nbw), dim3(64 * WW), lds8, st, a);
            } else if (type == 3) {
                if (CB == 16) QLAUNCH("dense", (dense_oct_kernel<3, 16, 2, WW>), dim3(nbw), dim3(64 * WW), lds8, st, a);
                else QLAUNCH("dense", (dense_oct_kernel<3, 8, 2, WW>), dim3(nbw), dim3(64 * WW), lds8, st, a);
            } else {
                if (CB == 16) QLAUNCH("dense", (dense_oct_kernel<2, 16, 2, WW>), dim3(nbw), dim3(64 * WW), lds8, st, a);
                else QLAUNCH("dense", (dense_oct_kernel<2, 8, 2, WW>), dim3(nbw), dim3(64 * WW), lds8, st, a);
            }
        };
        if (W == 4) go(std::integral_constant<int, 4>());
        else if (W == 2) go(std::integral_constant<int, 2>());
        else go(std::integral_constant<int, 1>());
        return hipGetLastError();
    }
    int nblk = 0;
    for (int i = 0; i < a.nm; i++) {
        a.m[i].first_block = nblk;
        nblk += (a.m[i].rows + 15) / 16;
    }
    {
        /* four waves sharing each block's 16 rows, NT tokens each: the smallest NT whose pass
         * covers the batch, as long as the records fit in LDS */
        const int CB = type == 14 ? 64 : (nb % 16 == 0 ? 16 : 8);
        if (type == 14 && nb % 64) return hipErrorInvalidValue;     /* Q6_K: cols % 2048 */
        /* Q4_0 / Q4_1: at most two tokens per wave and pass, although the rows are then
         * streamed once per 8 tokens instead of 16 (T = 16 154.7 -> 128.3 us per trunk layer,
         * T = 32 294 -> 242: half the record buffer lets two blocks share a CU); Q6_K, whose
         * per-token work is heavier, measured 1-2 % slower that way and keeps four */
        int NT = a.T <= kDenseTokW ? 1 : ((type == 14 && a.T > 2 * kDenseTokW) ? 4 : 2);
        while (NT > 1 && dense_tok_lds(NT, CB, type, nb) > 160 * 1024) NT >>= 1;
        const size_t lds = dense_tok_lds(NT, CB, type, nb);
        if (lds <= 160 * 1024) {
            const dim3 grid(nblk), block(64 * kDenseTokW);
            auto go = [&](auto ty, auto nt) {
                constexpr int TY = decltype(ty)::value, N = decltype(nt)::value;
                if constexpr (TY == 14) {
                    QLAUNCH("dense", (dense_tok_kernel<14, 64, 2, kDenseTokW, N>), grid, block, lds, st, a);
                } else {
                    if (CB == 16) QLAUNCH("dense", (dense_tok_kernel<TY, 16, 2, kDenseTokW, N>), grid, block, lds, st, a);
                    else QLAUNCH("dense", (dense_tok_kernel<TY, 8, 2, kDenseTokW, N>), grid, block, lds, st, a);
                }
            };
            auto by_nt = [&](auto ty) {
                if (NT == 4) go(ty, std::integral_constant<int, 4>());
                else if (NT == 2) go(ty, std::integral_constant<int, 2>());
                else go(ty, std::integral_constant<int, 1>());
            };
            if (type == 14) by_nt(std::integral_constant<int, 14>());
            else if (type == 3) by_nt(std::integral_constant<int, 3>());
            else by_nt(std::integral_constant<int, 2>());
            return hipGetLastError();
        }
    }
    if (type == 14) return hipErrorInvalidValue;
    const int NT = a.T >= 4 ? 4 : (a.T >= 2 ? 2 : 1);
    const int CB = nb % 16 == 0 ? 16 : 8;
    const int bb = type == 3 ? 20 : 18;
    const size_t ws = (size_t)CB * bb + (((CB * bb / 16) & 1) ? 0 : 16);
    const size_t lds = 16 * ws + (size_t)NT * (nb / 2) * kPairBytes;
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    const dim3 grid(nblk);
    if (type == 3) {
        if (NT == 4) launch_dense_t<3, 4>(a, CB, grid, lds, st);
        else if (NT == 2) launch_dense_t<3, 2>(a, CB, grid, lds, st);
        else launch_dense_t<3, 1>(a, CB, grid, lds, st);
    } else {
        if (NT == 4) launch_dense_t<2, 4>(a, CB, grid, lds, st);
        else if (NT == 2) launch_dense_t<2, 2>(a, CB, grid, lds, st);
        else launch_dense_t<2, 1>(a, CB, grid, lds, st);
    }
    return hipGetLastError();
}

/* ------------------------------------------------------------------ fp32 mode (--exact) ---- */

/* The reference's --exact mode (qms_exact_math = 1): every product is matmul_exact
 * (src/quant.c:97-115), a row dequantised to fp32 (qms_dequant_row, src/quant.c:17-93) against
 * fp32 inputs in one FMA chain in element order; the activations stay fp32. */

/* Router logits of the --exact mode (matmul_exact, src/quant.c:97-115): one fp32 chain per
 * (expert, token), acc = fma(w_c, x_c, acc) in element order. A block takes 8 experts of
 * token blockIdx.y, so the router rows stream through many CUs: its 256 threads copy each
 * chunk of kRouteExactCW columns of the 8 rows into LDS with 16-byte loads along the rows
 * (the next chunk in registers while lanes 0-7 run the chains on this one, reading four
 * steps per 16-byte LDS read), rows padded so the 8 chain lanes read distinct banks. n_embd
 * a multiple of 32. */
constexpr int kRouteExactCW = 1024;
constexpr int kRouteExactRS = kRouteExactCW + 4;   /* 16-byte rows 4 banks apart: 8 lanes, 32 banks */
constexpr size_t route_exact_lds(int E) { return ((size_t)E + 2 * 8 * kRouteExactRS) * 4; }

__global__ __launch_bounds__(256) void route_exact_kernel(const float *router, const float *xn, int E, int X,
                                                          float *logits)
{
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int PT = 8 * kRouteExactCW / 4 / 256;   /* 16-byte loads per thread per chunk */
    float *xr = (float *)smem;                        /* [E]                                 */
    float *wl = xr + E;                               /* [2][8][kRouteExactRS]               */
    const int t = blockIdx.y, e0 = blockIdx.x * 8, tid = threadIdx.x;
    for (int i = tid; i < E / 4; i += 256) ((float4 *)xr)[i] = ((const float4 *)(xn + (size_t)t * E))[i];
    float4 v[PT];
    auto load = [&](int c0) {
        const int cw = min(kRouteExactCW, E - c0);
#pragma unroll
        for (int m = 0; m < PT; m++) {
            const int i = tid + 256 * m, r = i / (kRouteExactCW / 4), q = i - r * (kRouteExactCW / 4);
            if (4 * q < cw) v[m] = *(const float4 *)(router + (size_t)min(e0 + r, X - 1) * E + c0 + 4 * q);
        }
    };
    auto stage = [&](int c0, float *buf) {
        const int cw = min(kRouteExactCW, E - c0);
#pragma unroll
        for (int m = 0; m < PT; m++) {
            const int i = tid + 256 * m, r = i / (kRouteExactCW / 4), q = i - r * (kRouteExactCW / 4);
            if (4 * q < cw) {
                float *d = buf + r * kRouteExactRS + 4 * q;
                d[0] = v[m].x;
                d[1] = v[m].y;
                d[2] = v[m].z;
                d[3] = v[m].w;
            }
        }
    };
    load(0);
    stage(0, wl);
    float acc = 0.0f;
    int buf = 0;
    for (int c0 = 0; c0 < E; c0 += kRouteExactCW) {
        __syncthreads();                              /* chunk c0 staged (and x, the first time) */
        if (c0 + kRouteExactCW < E) load(c0 + kRouteExactCW);
        if (tid < 8) {
            const float4 *wr = (const float4 *)(wl + buf * 8 * kRouteExactRS + tid * kRouteExactRS);
            const float4 *x4 = (const float4 *)(xr + c0);
            const int cw4 = min(kRouteExactCW, E - c0) / 4;
#pragma unroll 8
            for (int j = 0; j < cw4; j++) {
                const float4 w = wr[j], x = x4[j];
                acc = __builtin_fmaf(w.x, x.x, acc);
                acc = __builtin_fmaf(w.y, x.y, acc);
                acc = __builtin_fmaf(w.z, x.z, acc);
                acc = __builtin_fmaf(w.w, x.w, acc);
            }
        }
        if (c0 + kRouteExactCW < E) stage(c0 + kRouteExactCW, wl + (buf ^ 1) * 8 * kRouteExactRS);
        buf ^= 1;
    }
    if (tid < 8 && e0 + tid < X) logits[(size_t)t * X + e0 + tid] = acc;
}

/* Dequantised 32-block b of a row (src/quant.c:17-93): Q4_0 (q-8)*d, Q4_1 q*d+m (fused like
 * the reference build), Q8_0 q*d, Q6_K (d*sc)*q, F16 and F32 as they are. */
__device__ __forceinline__ void dequant_block(int type, const uint8_t *row, int b, float *w)
{
    /* each lane reads its own row, so every load touches another cache line per lane: words
     * as wide as the row's alignment allows (F32 / F16 rows of 32-multiples are 16-byte
     * aligned, Q4_1 blocks 4-byte, the others 2-byte) */
    if (type == 0) {
        const float4 *p = (const float4 *)(row + (size_t)b * 128);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float4 f = p[j];
            w[4 * j] = f.x; w[4 * j + 1] = f.y; w[4 * j + 2] = f.z; w[4 * j + 3] = f.w;
        }
    } else if (type == 1) {
        const u32x4 *p = (const u32x4 *)(row + (size_t)b * 64);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const u32x4 v = p[j];
            const uint32_t u[4] = { v.x, v.y, v.z, v.w };
#pragma unroll
            for (int k = 0; k < 4; k++) {
                w[8 * j + 2 * k] = h2f(u[k] & 0xffffu);
                w[8 * j + 2 * k + 1] = h2f(u[k] >> 16);
            }
        }
    } else if (type == 8) {
        const uint16_t *p = (const uint16_t *)(row + (size_t)b * 34);
        const float d = h2f(p[0]);
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const uint32_t h = p[1 + j];
            w[2 * j] = (float)(int8_t)(h & 0xff) * d;
            w[2 * j + 1] = (float)(int8_t)(h >> 8) * d;
        }
    } else if (type == 14) {
        const uint8_t *sb = row + (size_t)(b >> 3) * 210;
        const int h = (b & 7) >> 2, g = b & 3;
        const uint16_t *ql = (const uint16_t *)(sb + 64 * h + 32 * (g & 1)), *qh = (const uint16_t *)(sb + 128 + 32 * h);
        const uint32_t sc = *(const uint16_t *)(sb + 192 + 8 * h + 2 * g);
        const float d = h2f(*(const uint16_t *)(sb + 208));
        const float d0 = d * (float)(int8_t)(sc & 0xff);
        const float d1 = d * (float)(int8_t)(sc >> 8);
#pragma unroll
        for (int l2 = 0; l2 < 16; l2++) {
            const uint32_t lo2 = ql[l2], hi2 = qh[l2];
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const int l = 2 * l2 + k;
                const int lo = (lo2 >> (8 * k)) & 0xff, hb = (hi2 >> (8 * k)) & 0xff;
                const int q = ((g < 2 ? lo & 15 : lo >> 4) | (((hb >> (2 * g)) & 3) << 4)) - 32;
                w[l] = (l < 16 ? d0 : d1) * (float)q;
            }
        }
    } else if (type == 3) {
        const uint32_t *p = (const uint32_t *)(row + (size_t)b * 20);
        const uint32_t dm = p[0];
        const float d = h2f(dm & 0xffffu), m = h2f(dm >> 16);
#pragma unroll
        for (int j4 = 0; j4 < 4; j4++) {
            const uint32_t c = p[1 + j4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t q = (c >> (8 * k)) & 0xff;
                w[4 * j4 + k] = __builtin_fmaf((float)(q & 15), d, m);
                w[4 * j4 + k + 16] = __builtin_fmaf((float)(q >> 4), d, m);
            }
        }
    } else {
        const uint16_t *p = (const uint16_t *)(row + (size_t)b * 18);
        const float d = h2f(p[0]);
#pragma unroll
        for (int j2 = 0; j2 < 8; j2++) {
            const uint32_t c = p[1 + j2];
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const int q = (int)((c >> (8 * k)) & 0xff);
                w[2 * j2 + k] = (float)((q & 15) - 8) * d;
                w[2 * j2 + k + 16] = (float)((q >> 4) - 8) * d;
            }
        }
    }
}

/* y = matmul_exact rows of each active expert's matrix for its slots: one lane per row
 * (64 rows per block, blockIdx.y = active expert), up to 4 slots per pass with their input
 * rows staged in LDS. Inputs: the slot's token row of xn (by_token) or its own row of x. */
struct ExactArgs {
    const uint8_t *w;
    uint64_t rb, eb;
    int type, rows, cols, by_token;
    const float *x;
    float *y;
    int y_stride, y_off;
    /* blockIdx.z == 1: a second matrix of the same shape and inputs (up beside gate) */
    const uint8_t *w2;
    uint64_t rb2, eb2;
    int type2, y_off2;
    Scratch S;
};

__global__ __launch_bounds__(64) void exact_rows_kernel(ExactArgs a)
{
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int NT = 4;
    if ((int)blockIdx.y >= a.S.meta[0]) return;
    const int4 wk = a.S.work[blockIdx.y];
    const int e = wk.x, lane = threadIdx.x, r = blockIdx.x * 64 + lane, C = a.cols;
    float *xr = (float *)smem;                                      /* [NT][C] */
    const bool second = blockIdx.z == 1;
    const int type = second ? a.type2 : a.type, y_off = second ? a.y_off2 : a.y_off;
    const uint8_t *row = (second ? a.w2 + (size_t)e * a.eb2 + (size_t)min(r, a.rows - 1) * a.rb2
                                 : a.w + (size_t)e * a.eb + (size_t)min(r, a.rows - 1) * a.rb);
    for (int s0 = wk.y; s0 < wk.z; s0 += NT) {
        const int nt = min(NT, wk.z - s0);
        __syncthreads();
        for (int i = lane; i < nt * (C / 4); i += 64) {
            const int n = i / (C / 4), j = i - n * (C / 4);
            const size_t src = a.by_token ? (size_t)a.S.slot_t[s0 + n] : (size_t)(s0 + n);
            ((float4 *)xr)[i] = ((const float4 *)(a.x + src * C))[j];
        }
        __syncthreads();
        float acc[NT] = { 0.0f, 0.0f, 0.0f, 0.0f };
        for (int b = 0; b < C / 32; b++) {
            float w[32];
            dequant_block(type, row, b, w);
#pragma unroll
            for (int n = 0; n < NT; n++)
                if (n < nt)
#pragma unroll
                    for (int j = 0; j < 32; j++) acc[n] = __builtin_fmaf(w[j], xr[n * C + 32 * b + j], acc[n]);
        }
        if (r < a.rows)
            for (int n = 0; n < nt; n++) a.y[(size_t)(s0 + n) * a.y_stride + y_off + r] = acc[n];
    }
}

hipError_t launch_layer_slots(const Shape &s, const LayerDev &L, const Scratch &S, const float *xn, float *out, int T,
                              int exact, int debug, hipStream_t st, int down_only)
{
    SelectArgs sa;
    sa.X = s.X;
    sa.K = s.K;
    sa.T = T;
    sa.S = S;
    if (down_only) {
        /* routing, gate/up and SwiGLU done by the integer kernels */
    } else if (exact) {
        if (route_exact_lds(s.E) > 160 * 1024) return hipErrorInvalidValue;
        QLAUNCH("route", route_exact_kernel, dim3((s.X + 7) / 8, T), dim3(256), route_exact_lds(s.E), st, L.router, xn,
                s.E, s.X, S.logits);
    } else {
        /* qms_matmul of the F32 router (src/model.c:1043): dot_f32's sixteen chains */
        const hipError_t e = launch_f32_rows(L.router, s.X, s.E, xn, T, S.logits, s.X, "route", st);
        if (e != hipSuccess) return e;
    }
    if (!down_only) {
        QLAUNCH("select", select_kernel, dim3(T), dim3(256), 0, st, sa, 0);
        QLAUNCH("dispatch", dispatch_kernel, dim3(1), dim3(64), 0, st, sa);
    }
    const int maxact = s.X < T * s.K ? s.X : T * s.K;
    const struct { const uint8_t *w; uint64_t rb, eb; int type, rows, cols, by_token; const float *x; float *y;
                   int stride, off; } m[3] = {
        { L.gate, L.gate_rb, L.gate_eb, L.gate_type, s.F, s.E, 1, xn, S.gu, 2 * s.F, 0 },
        { L.up, L.up_rb, L.up_eb, L.up_type, s.F, s.E, 1, xn, S.gu, 2 * s.F, s.F },
        { L.down, L.down_rb, L.down_eb, L.down_type, s.E, s.F, 0, S.act, S.dn, s.E, 0 },
    };
    for (int i = down_only ? 2 : 0; i < 3; i++) {
        if (i == 2 && !down_only) {
            const int n = T * s.K * s.F;
            QLAUNCH("swiglu", swiglu_kernel, dim3((n + 255) / 256), dim3(256), 0, st, S, s.F, T * s.K);
        }
        const char *name = i == 2 ? "down" : "gateup";
        /* --exact, and F16 / Q8_0 rows at any setting (outside qms_fast_supported, so the
         * reference's qms_matmul takes matmul_exact for them): the fp32 chain */
        auto chain_rows = [&](int t) { return exact || t == 1 || t == 8; };
        /* gate and up in one launch (grid z = 2) when they take the same kernel */
        const bool pair = i == 0 && (chain_rows(m[0].type) ? chain_rows(m[1].type)
                                                           : !chain_rows(m[1].type) && m[1].type == m[0].type);
        if (chain_rows(m[i].type)) {
            ExactArgs a;
            a.S = S;
            a.w = m[i].w;
            a.rb = m[i].rb;
            a.eb = m[i].eb;
            a.type = m[i].type;
            a.rows = m[i].rows;
            a.cols = m[i].cols;
            a.by_token = m[i].by_token;
            a.x = m[i].x;
            a.y = m[i].y;
            a.y_stride = m[i].stride;
            a.y_off = m[i].off;
            a.w2 = m[1].w;
            a.rb2 = m[1].rb;
            a.eb2 = m[1].eb;
            a.type2 = m[1].type;
            a.y_off2 = m[1].off;
            /* input rows for the slots of one pass: at most min(4, T), an expert's slots
             * being distinct tokens */
            const size_t lds = (size_t)min(4, T) * m[i].cols * 4;
            if (lds > 160 * 1024) return hipErrorInvalidValue;
            QLAUNCH(name, exact_rows_kernel, dim3((m[i].rows + 63) / 64, maxact, pair ? 2 : 1), dim3(64), lds, st, a);
            if (pair) i++;
            continue;
        }
        SlotAnyArgs a;
        a.S = S;
        a.w = m[i].w;
        a.rb = m[i].rb;
        a.eb = m[i].eb;
        a.rows = m[i].rows;
        a.cols = m[i].cols;
        a.by_token = m[i].by_token;
        a.x = m[i].x;
        a.y = m[i].y;
        a.y_stride = m[i].stride;
        a.y_off = m[i].off;
        a.w2 = m[1].w;
        a.rb2 = m[1].rb;
        a.eb2 = m[1].eb;
        a.y_off2 = m[1].off;
        const int nb = m[i].cols / 32, NT = dense_any_nt(m[i].type, T, nb);
        if (!NT) return hipErrorInvalidValue;
        const size_t lds = m[i].type == 0 ? 0 : (size_t)NT * nb * kDenseAnyRec;
        const int rpb = m[i].type == 0 ? 16 : 32;
        const dim3 grid((m[i].rows + rpb - 1) / rpb, maxact, pair ? 2 : 1);
        auto go = [&](auto ty) {
            constexpr int TY = decltype(ty)::value;
            if (NT == 8) QLAUNCH(name, (slot_any_kernel<TY, 8>), grid, dim3(256), lds, st, a);
            else if (NT == 4) QLAUNCH(name, (slot_any_kernel<TY, 4>), grid, dim3(256), lds, st, a);
            else if (NT == 2) QLAUNCH(name, (slot_any_kernel<TY, 2>), grid, dim3(256), lds, st, a);
            else QLAUNCH(name, (slot_any_kernel<TY, 1>), grid, dim3(256), lds, st, a);
        };
        if (m[i].type == 14) go(std::integral_constant<int, 14>());
        else if (m[i].type == 3) go(std::integral_constant<int, 3>());
        else if (m[i].type == 0) go(std::integral_constant<int, 0>());
        else go(std::integral_constant<int, 2>());
        if (pair) i++;
    }
    if (debug && !exact) {
        /* the int8 blocks the slot kernels formed in LDS, for the debug copies */
        const int nx = T * (s.E / 32), na = T * s.K * (s.F / 32);
        if (!down_only)
            QLAUNCH("debug", quant_rows_kernel, dim3((nx + 255) / 256), dim3(256), 0, st, xn, s.E, T, S.xq);
        QLAUNCH("debug", quant_rows_kernel, dim3((na + 255) / 256), dim3(256), 0, st, S.act, s.F, T * s.K, S.aq);
    }
    const int n = T * s.E;
    if (s.E % 256 == 0)
        QLAUNCH("combine", combine_kernel, dim3(n / (4 * combine_threads(s.E))), dim3(combine_threads(s.E)), 0, st, S,
                s.E, s.K, T, out);
    else QLAUNCH("combine", combine_any_kernel, dim3((n + 255) / 256), dim3(256), 0, st, S, s.E, s.K, T, out);
    return hipGetLastError();
}

/* ------------------------------------------------------------------ dense rows, fp32 chains ---- */

/* qms_matmul_n's matmul_exact (src/quant.c:97-115) for calls the fast loop does not take: the
 * --exact mode, or any matrix of a type outside qms_fast_supported (F16, Q8_0) in the call,
 * which sends every matrix of it there (src/quant.c:131-141). One lane per row of the call's
 * matrices (one type per launch), its dequantised 32-blocks against up to NT tokens staged in
 * LDS, acc = fma(w, x, acc) in element order. Rows past a matrix's end read its last row and
 * store nothing. */
template <int NT>
__global__ __launch_bounds__(64) void dense_exact_kernel(DenseArgs a, int type)
{
    extern __shared__ __align__(16) uint8_t smem[];
    float *xr = (float *)smem;                        /* [NT][C] */
    int mi = 0;
#pragma unroll
    for (int i = 1; i < kDenseMats; i++)
        if (i < a.nm && (int)blockIdx.x >= a.m[i].first_block) mi = i;
    const DenseMat M = a.m[mi];
    const int lane = threadIdx.x, C = a.C;
    const int row = ((int)blockIdx.x - M.first_block) * 64 + lane;
    const uint8_t *wr = M.w + (size_t)min(row, M.rows - 1) * a.rb;
    for (int t0 = 0; t0 < a.T; t0 += NT) {
        const int nt = min(NT, a.T - t0);
        __syncthreads();
        for (int i = lane; i < nt * (C / 4); i += 64)
            ((float4 *)xr)[i] = ((const float4 *)(a.x + (size_t)t0 * C))[i];
        __syncthreads();
        float acc[NT];
#pragma unroll
        for (int n = 0; n < NT; n++) acc[n] = 0.0f;
        for (int b = 0; b < C / 32; b++) {
            float w[32];
            dequant_block(type, wr, b, w);
#pragma unroll
            for (int n = 0; n < NT; n++)
                if (n < nt)
#pragma unroll
                    for (int j = 0; j < 32; j++) acc[n] = __builtin_fmaf(w[j], xr[n * C + 32 * b + j], acc[n]);
        }
        if (row < M.rows)
            for (int n = 0; n < nt; n++) M.y[(size_t)(t0 + n) * M.rows + row] = acc[n];
    }
}

hipError_t launch_dense_exact(const DenseArgs &args, int type, hipStream_t st)
{
    DenseArgs a = args;
    const size_t row_lds = (size_t)a.C * 4;
    const int NT = 4 * row_lds <= 160 * 1024 ? 4 : (2 * row_lds <= 160 * 1024 ? 2 : 1);
    if (row_lds > 160 * 1024) return hipErrorInvalidValue;
    int nblk = 0;
    for (int i = 0; i < a.nm; i++) {
        a.m[i].first_block = nblk;
        nblk += (a.m[i].rows + 63) / 64;
    }
    const size_t lds = NT * row_lds;
    if (NT == 4) QLAUNCH("dense", dense_exact_kernel<4>, dim3(nblk), dim3(64), lds, st, a, type);
    else if (NT == 2) QLAUNCH("dense", dense_exact_kernel<2>, dim3(nblk), dim3(64), lds, st, a, type);
    else QLAUNCH("dense", dense_exact_kernel<1>, dim3(nblk), dim3(64), lds, st, a, type);
    return hipGetLastError();
}

/* ------------------------------------------------------------------ block dots (checks) ---- */

/* Exact signed int32 dot of one 32-block of a weight row with one Q8 block, formed with the
 * same unpacking and sdot4 steps the row kernels use. */
__global__ void block_dots_kernel(const uint8_t *base, int type, uint64_t rb, uint64_t eb, int n, const int32_t *ex,
                                  const int32_t *row, const int32_t *blk, const Q8 *xq, int32_t *out)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint8_t *r = base + (size_t)ex[i] * eb + (size_t)row[i] * rb;
    const Q8 &x = xq[i];
    const uint32_t *xw = (const uint32_t *)x.q;
    int s = 0;
    if (type == 2) {
        const uint8_t *b = r + (size_t)blk[i] * 18 + 2;
        for (int p = 0; p < 4; p++) {
            const uint32_t c = (uint32_t)b[4 * p] | ((uint32_t)b[4 * p + 1] << 8) | ((uint32_t)b[4 * p + 2] << 16) |
                               ((uint32_t)b[4 * p + 3] << 24);
            s += sdot4((int)(c & 0x0f0f0f0fu), (int)xw[p]) + sdot4((int)((c >> 4) & 0x0f0f0f0fu), (int)xw[4 + p]);
        }
        s -= 8 * ((int)x.s16[0] + (int)x.s16[1]);
    } else if (type == 3) {
        const uint8_t *b = r + (size_t)blk[i] * 20 + 4;
        for (int p = 0; p < 4; p++) {
            const uint32_t c = (uint32_t)b[4 * p] | ((uint32_t)b[4 * p + 1] << 8) | ((uint32_t)b[4 * p + 2] << 16) |
                               ((uint32_t)b[4 * p + 3] << 24);
            s += sdot4((int)(c & 0x0f0f0f0fu), (int)xw[p]) + sdot4((int)((c >> 4) & 0x0f0f0f0fu), (int)xw[4 + p]);
        }
    } else {
        const int b = blk[i], sbi = b >> 3, h = (b & 7) >> 2, g = b & 3;
        const uint8_t *sb = r + (size_t)sbi * 210;
        const uint8_t *ql = sb + 64 * h + 32 * (g & 1), *qh = sb + 128 + 32 * h;
        const int sa = (int)(int8_t)sb[192 + 8 * h + 2 * g], sbb = (int)(int8_t)sb[193 + 8 * h + 2 * g];
        int lo = 0, hi = 0;
        for (int p = 0; p < 8; p++) {
            uint32_t q6 = 0;
            for (int k = 0; k < 4; k++) {
                const int l = 4 * p + k;
                const int nb = g < 2 ? (ql[l] & 15) : (ql[l] >> 4);
                q6 |= (uint32_t)(nb | (((qh[l] >> (2 * g)) & 3) << 4)) << (8 * k);
            }
            const int v = sdot4((int)q6, (int)xw[p]);
            if (p < 4) lo += v; else hi += v;
        }
        s = sa * (lo - 32 * (int)x.s16[0]) + sbb * (hi - 32 * (int)x.s16[1]);
    }
    out[i] = s;
}

hipError_t launch_block_dots(const uint8_t *base, int type, uint64_t rb, uint64_t eb, int n, const int32_t *expert,
                             const int32_t *row, const int32_t *block, const Q8 *xq, int32_t *out, hipStream_t st)
{
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(block_dots_kernel, dim3((n + 255) / 256), dim3(256), 0, st, base, type, rb, eb, n, expert, row,
                       block, xq, out);
    return hipGetLastError();
}

/* ------------------------------------------------------------------ SiLU check ---- */

__global__ void silu_kernel(const float *x, int n, float *out)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = silu_ref(x[i]);
}

__global__ void exp_kernel(const double *x, int n, double *out)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = qmsg_exp(x[i]);
}

hipError_t launch_exp(const double *x, int n, double *out, hipStream_t st)
{
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(exp_kernel, dim3((n + 255) / 256), dim3(256), 0, st, x, n, out);
    return hipGetLastError();
}

hipError_t launch_silu(const float *x, int n, float *out, hipStream_t st)
{
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(silu_kernel, dim3((n + 255) / 256), dim3(256), 0, st, x, n, out);
    return hipGetLastError();
}

/* ------------------------------------------------------------------ calibration copy ---- */

__global__ void copy_kernel(uint4 *dst, const uint4 *src, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        dst[i] = src[i];
}

hipError_t launch_copy(void *dst, const void *src, size_t bytes, hipStream_t st)
{
    const size_t n = bytes / 16;
    QLAUNCH("copy", copy_kernel, dim3(4096), dim3(256), 0, st, (uint4 *)dst, (const uint4 *)src, n);
    return hipGetLastError();
}

/* Clears the per-call state of a scratch set: the 16 meta words (the select kernel's ticket
 * counter among them) and the two record-range flags, whose epoch would otherwise stay set
 * across replays of a captured call. A kernel rather than a memset node, so the call can be
 * captured into a graph. */
__global__ void call_reset_kernel(uint32_t *meta, uint64_t *mxflag)
{
    if (threadIdx.x < 16) meta[threadIdx.x] = 0u;
    if (threadIdx.x < 2) mxflag[threadIdx.x] = 0ull;
}

hipError_t launch_call_reset(const Scratch &S, hipStream_t st)
{
    QLAUNCH("fill", call_reset_kernel, dim3(1), dim3(64), 0, st, (uint32_t *)S.meta, S.mxflag);
    return hipGetLastError();
}

/* ------------------------------------------------------------------ synthetic data ---- */

__global__ void synth_f32_kernel(uint64_t key, uint64_t n, float sigma, float *out)
{
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = qmsg_normal(key, i) * sigma;
}

hipError_t launch_synth_f32(uint64_t key, uint64_t n, float sigma, float *out, hipStream_t st)
{
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(synth_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, key, n, sigma, out);
    return hipGetLastError();
}

/* One thread per Q4_0 / Q4_1 block (or Q6_K super-block) of all X experts. */
__global__ void synth_experts_kernel(uint64_t seed, uint32_t layer, uint32_t kind, int type, int64_t rows,
                                     int64_t cols, int X, float sigma, uint8_t *base)
{
    const int64_t per_row = type == 14 ? cols / 256 : cols / 32;
    const uint64_t rb = (uint64_t)per_row * (type == 14 ? 210 : (type == 3 ? 20 : 18));
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t per_e = rows * per_row;
    if (i >= per_e * X) return;
    const int e = (int)(i / per_e);
    const int64_t rem = i - (int64_t)e * per_e, r = rem / per_row, b = rem - r * per_row;
    const uint64_t key = qmsg_tensor_key(seed, layer, kind, (uint32_t)e);
    uint8_t *dst = base + (uint64_t)e * rb * (uint64_t)rows + (uint64_t)r * rb;
    if (type == 14) {
        uint8_t blk[210];
        qmsg_synth_q6_k_block(key, (uint64_t)r * (uint64_t)cols + (uint64_t)b * 256, sigma, blk);
        for (int k = 0; k < 210; k++) dst[(uint64_t)b * 210 + k] = blk[k];
    } else if (type == 3) {
        uint8_t blk[20];
        qmsg_synth_q4_1_block(key, (uint64_t)cols, (uint64_t)r, (uint64_t)b, sigma, blk);
        for (int k = 0; k < 20; k++) dst[(uint64_t)b * 20 + k] = blk[k];
    } else {
        uint8_t blk[18];
        qmsg_synth_q4_0_block(key, (uint64_t)cols, (uint64_t)r, (uint64_t)b, sigma, blk);
        for (int k = 0; k < 18; k++) dst[(uint64_t)b * 18 + k] = blk[k];
    }
}

hipError_t launch_synth_experts(uint64_t seed, uint32_t layer, uint32_t kind, int type, int64_t rows, int64_t cols,
                                int X, float sigma, uint8_t *base, hipStream_t st)
{
    const int64_t per_row = type == 14 ? cols / 256 : cols / 32;
    const int64_t n = rows * per_row * X;
    hipLaunchKernelGGL(synth_experts_kernel, dim3((unsigned)((n + 127) / 128)), dim3(128), 0, st, seed, layer, kind,
                       type, rows, cols, X, sigma, base);
    return hipGetLastError();
}

/* src/model.c:403-409 with a unit weight, one row per block: the sum of squares is the
 * reference's sequential double FMA chain (lane 0), so rows match it bit for bit. */
__global__ void rmsnorm_rows_kernel(float *x, int E, float eps)
{
    __shared__ double inv;
    float *row = x + (size_t)blockIdx.x * E;
    if (threadIdx.x == 0) {
        double ss = 0.0;
        for (int i = 0; i < E; i++) ss = __builtin_fma((double)row[i], (double)row[i], ss);
        inv = 1.0 / sqrt(ss / E + (double)eps);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < E; i += blockDim.x) row[i] = (float)((double)row[i] * inv) * 1.0f;
}

hipError_t launch_rmsnorm_rows(float *x, int T, int E, float eps, hipStream_t st)
{
    if (T <= 0) return hipSuccess;
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(T), dim3(256), 0, st, x, E, eps);
    return hipGetLastError();
}

/* Biased exponent field of a double. */
__device__ __forceinline__ int dexp(double v) { return (int)((__double_as_longlong(v) >> 52) & 0x7ff); }

/* Pitch (in doubles) of a term row of the chunked layout: term i of lane j's chunk at
 * qt[i * kSumPitch + j], so the 64 lanes read 64 consecutive doubles per step. */
constexpr int kSumPitch = 65;

/* NR sequential sums over the column col of qt (C terms, C % 8 == 0), chain r starting from
 * s[r]: every term is added to every chain in order; the next 8 terms are read while the
 * current 8 are added, so only the adds' latency is on the chains. */
template <int NR>
__device__ __forceinline__ void column_run(const double *qt, int col, int C, double (&s)[NR])
{
    double a[8], b[8];
#pragma unroll
    for (int k = 0; k < 8; k++) a[k] = qt[k * kSumPitch + col];
    for (int i = 0; i < C; i += 16) {
        if (i + 8 < C) {
#pragma unroll
            for (int k = 0; k < 8; k++) b[k] = qt[(i + 8 + k) * kSumPitch + col];
        }
#pragma unroll
        for (int k = 0; k < 8; k++)
#pragma unroll
            for (int r = 0; r < NR; r++) s[r] += a[k];
        if (i + 8 >= C) break;
        if (i + 16 < C) {
#pragma unroll
            for (int k = 0; k < 8; k++) a[k] = qt[(i + 16 + k) * kSumPitch + col];
        }
#pragma unroll
        for (int k = 0; k < 8; k++)
#pragma unroll
            for (int r = 0; r < NR; r++) s[r] += b[k];
    }
}


__device__ __forceinline__ uint64_t dbits(double v) { return (uint64_t)__double_as_longlong(v); }

/* The sequential sum s_{i+1} = fl(s_i + q_i), s_0 = 0, of n = 64 C terms q_i >= 0 (C % 8 == 0),
 * bit for bit, by one wave (all 64 lanes, the result in every lane); lane j's chunk is terms
 * jC .. jC + C - 1, stored at qt[i * kSumPitch + j].
 *  1. Approximate chunk starts P_j: every chunk summed in any order, an exclusive lane scan.
 *  2. Every lane runs its chunk term by term from P_j and from P_j + u, u = 2^(e - 52) for
 *     P_j in the binade [2^e, 2^(e+1)): ends G0_j and G1_j.
 *  3. A walk over the chunks with the true sum s, the same on every lane: if s == P_j the chunk
 *     ends at G0_j; else if s, P_j, P_j + u, G0_j and G1_j all lie in P_j's binade, r is the
 *     parity of (s - P_j) / u and s + (G_r - P_r) (P_1 = P_j + u) lies in it too, the chunk ends
 *     there; otherwise the chunk is added to s term by term.
 * Why the second case is exact: inside one binade the doubles are the multiples of u, and for
 * such an a, fl(a + q) = a + (q rounded to a multiple of u); the increment depends on a only in
 * a tie (q/u with fraction 1/2 exactly), through the parity of a/u, which picks the even
 * multiple. Runs from starts equal modulo 2u take the same increments while both stay in the
 * binade; the run from s does, since it ends below 2^(e+1) and never decreases (q_i >= 0); and
 * the differences and the final sum are multiples of u below 2^(e+1), so exact. A chunk whose
 * sum crosses a power of two takes the term-by-term case. Non-finite sums take it everywhere.
 * Inside one binade the bit pattern of a non-negative double is its value in units of u plus a
 * constant, so the walk runs on bit patterns in integer (scalar) arithmetic: (s - P_j) / u is
 * bits(s) - bits(P_j), and adding G_r - P_r adds bits(G_r) - bits(P_r). */
__device__ __forceinline__ double ordered_sum_chunked(const double *qt, int C)
{
    const int j = threadIdx.x & 63;
    /* 1 */
    double c0 = 0.0, c1 = 0.0, c2 = 0.0, c3 = 0.0;
    for (int i = 0; i < C; i += 4) {
        c0 += qt[i * kSumPitch + j];
        c1 += qt[(i + 1) * kSumPitch + j];
        c2 += qt[(i + 2) * kSumPitch + j];
        c3 += qt[(i + 3) * kSumPitch + j];
    }
    double inc = (c0 + c1) + (c2 + c3);
    PHASE(3072, 3);
    if (!__all(__builtin_isfinite(inc))) {
        /* an infinite or NaN term: term by term throughout */
        double s[1] = { 0.0 };
        for (int k = 0; k < 64; k++) column_run<1>(qt, k, C, s);
        return s[0];
    }
    for (int d = 1; d < 64; d <<= 1) {
        const double t = __shfl_up(inc, d);
        if (j >= d) inc += t;
    }
    double P = __shfl_up(inc, 1);
    if (j == 0) P = 0.0;
    /* 2 */
    const int e = dexp(P);
    const bool normal = e > 52;                        /* u = 2^(e - 52) a normal double too */
    const double P1 = P + __longlong_as_double((long long)(normal ? e - 52 : 1) << 52);
    double g[2] = { P, P1 };
    column_run<2>(qt, j, C, g);
    PHASE(3072, 4);
    const uint64_t pb = dbits(P);
    const uint64_t d0 = dbits(g[0]) - pb, d1 = dbits(g[1]) - (pb + 1);
    const int ex = normal && dexp(P1) == e && dexp(g[0]) == e && dexp(g[1]) == e ? e : -1;
    /* 3. In bit patterns, an in-binade chunk maps s to s + a[s & 1] (a: the deltas by the parity
     * of s itself, a[r ^ (P & 1)] = D_r). Such maps compose (f then g: s + f[p] + g[(p + f[p]) & 1]
     * for p = s & 1), so a run of in-binade chunks is walked at once: a prefix over its lanes
     * gives every chunk's start from the run's, each lane checks that its start and end stay in
     * its binade (or that its start is its P), and the run ends at its last chunk's end; a
     * chunk that fails the check, or one outside the rule, is added term by term. */
    const uint64_t a0 = (pb & 1) ? d1 : d0, a1 = (pb & 1) ? d0 : d1;
    const uint64_t outside = __ballot(ex < 0);
    auto shfl_up_u64 = [](uint64_t v, int d) {
        const uint32_t lo = (uint32_t)__shfl_up((int)(uint32_t)v, d), hi = (uint32_t)__shfl_up((int)(uint32_t)(v >> 32), d);
        return ((uint64_t)hi << 32) | lo;
    };
    uint64_t sb = 0;                                   /* bits of s = +0.0 */
#ifdef QMSG_PHASE_TRACE
    int nslow = 0;
    unsigned long long tslow = 0;
#endif
    auto term_by_term = [&](int k, uint64_t from) {
#ifdef QMSG_PHASE_TRACE
        const unsigned long long ts0 = __builtin_amdgcn_s_memrealtime();
#endif
        double t[1] = { __longlong_as_double((long long)from) };
        column_run<1>(qt, k, C, t);
#ifdef QMSG_PHASE_TRACE
        nslow++;
        tslow += __builtin_amdgcn_s_memrealtime() - ts0;
#endif
        return readlane_u64(dbits(t[0]), 0);
    };
    int k = 0;
    while (k < 64) {
        if ((outside >> k) & 1) {
            const uint64_t pk = readlane_u64(pb, k);
            sb = sb == pk ? pk + readlane_u64(d0, k) : term_by_term(k, sb);
            k++;
            continue;
        }
        const uint64_t later = outside >> k;
        const int r = later ? k + __builtin_ctzll(later) : 64;     /* the run is chunks k .. r-1 */
        const bool in = j >= k && j < r;
        uint64_t i0 = a0, i1 = a1;                     /* the maps of chunks k .. j composed */
        for (int d = 1; d < 64; d <<= 1) {
            const uint64_t p0 = shfl_up_u64(i0, d), p1 = shfl_up_u64(i1, d);
            if (in && j - d >= k) {
                const uint64_t n0 = p0 + ((p0 & 1) ? i1 : i0), n1 = p1 + ((p1 & 1) ? i0 : i1);
                i0 = n0;
                i1 = n1;
            }
        }
        uint64_t e0 = shfl_up_u64(i0, 1), e1 = shfl_up_u64(i1, 1);
        if (j == k) e0 = e1 = 0;
        const uint64_t sj = sb + ((sb & 1) ? e1 : e0);  /* chunk j's start */
        const uint64_t nj = sj + ((sj & 1) ? a1 : a0);
        const bool ok = sj == pb || ((int)(sj >> 52) == ex && (int)(nj >> 52) == ex);
        const uint64_t bad = __ballot(in && !ok);
        if (!bad) {
            sb = readlane_u64(nj, r - 1);
            k = r;
        } else {
            const int b = __builtin_ctzll(bad);
            sb = term_by_term(b, readlane_u64(sj, b));
            k = b + 1;
        }
    }
#ifdef QMSG_PHASE_TRACE
    if (threadIdx.x == 0 && blockIdx.x < 1024) qmsg::g_phase[(3072 + blockIdx.x) * 8 + 7] = (unsigned long long)nslow | (tslow << 8);
#endif
    return __longlong_as_double((long long)sb);
}

/* rmsnorm of one row per block into another buffer, with a weight vector (nullptr: unit)
 * (src/model.c:403-409): y = (float)(x * inv) * w, inv = 1 / sqrt(ss / E + eps). ss accumulates
 * (double)x*(double)x in index order; each square is exact in double (48 significant bits), so
 * the reference's fma(x, x, ss) equals ss + x*x with the square formed first.
 * The output needs ss only through the floats (float)(x * inv), so the kernel first brackets
 * ss: S = the squares summed in any order, and the sequential sum's distance from the exact one
 * is at most u * sum_k s_{k+1} (u = 2^-53, s the running sums, each step's rounding at most u
 * times its result), with s_{k+1} <= (1 + u)^k times the exact partial sum, so at most
 * u (1 + 2^-20) W, W = sum_j q_j (E - j) (q_j the square of element j); S's own distance from
 * the exact sum is at most (E / 256 + 16) 2^-52 S (the depth of the parallel sum, with room
 * for the rounding of the bracket's own operations). inv is monotone in ss (every rounded
 * operation is), and so is (float)(x * inv) in inv: when every element gives the same float
 * at both ends of the bracket, every ss inside gives it too, and the row is written from one
 * end. Otherwise (about one 4096-wide row in 200 on normal data: an element within 1e-13 of a
 * float rounding boundary), or for a non-finite sum, or with walk set, the sum is formed in
 * order: every thread has put its squares into LDS, and wave 0 forms their sequential sum
 * (ordered_sum_chunked for E a multiple of 512, else one lane term by term); a row that does
 * so is counted into *walked (if not null). Rows of up to kNormVec * 1024 floats stay in
 * registers, with their weights, loaded before the sum; longer rows are read again for the
 * check and the output. With add, the row is first x + add in float (the residual add
 * h += out of the previous layer, src/model.c:1285), stored back to x, and normalised. */
constexpr int kNormVec = 8;

template <int CTRL>
__device__ __forceinline__ double dpp_f64(double x)
{
    const uint64_t b = dbits(x);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, 0xF, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, 0xF, 0xF, false);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

/* A sum of a double over the 64 lanes of a wave, in some fixed order, in every lane: the
 * quads, halves of rows and rows by lane permutations, then the four rows' sums read out. */
__device__ __forceinline__ double wave_sum_any(double v)
{
    v += dpp_f64<0xB1>(v);      /* quad_perm 1, 0, 3, 2 */
    v += dpp_f64<0x4E>(v);      /* quad_perm 2, 3, 0, 1 */
    v += dpp_f64<0x141>(v);     /* row_half_mirror      */
    v += dpp_f64<0x140>(v);     /* row_mirror           */
    const double r0 = __longlong_as_double((long long)readlane_u64(dbits(v), 0));
    const double r1 = __longlong_as_double((long long)readlane_u64(dbits(v), 16));
    const double r2 = __longlong_as_double((long long)readlane_u64(dbits(v), 32));
    const double r3 = __longlong_as_double((long long)readlane_u64(dbits(v), 48));
    return (r0 + r1) + (r2 + r3);
}

/* The inverse norm inv = 1 / sqrt(ss / E + eps) of one row (rmsnorm_kernel describes the
 * bracket) from this thread's partial sums of the squares (sum_s) and of the squares weighted
 * by E - j (sum_w); same(lo, hi) tells whether every element this thread holds gives one
 * float (float)(x * inv) at inv = lo and at inv = hi, and fill() stores this thread's squares
 * into LDS at q in the layout the ordered sum reads (norm_store), called only when the sum is
 * formed in order. stage(v) runs with the bracket's end before the block's vote on it (its
 * LDS writes are visible to the block after the call when *open_out is false); when the vote
 * opens the row, the caller stages again with the returned inv. All 256 threads of the block
 * call it, with the same E, eps and walk; part is 8 doubles of LDS and inv_sh one. A row that
 * forms its sum in order is counted into *walked when walked is not null. */
template <class Same, class Fill, class Stage>
__device__ double norm_inv(double sum_s, double sum_w, const double *q, int E, float eps, int walk,
                           unsigned long long *walked, Same same, Fill fill, double *part, double *inv_sh,
                           Stage stage, bool &open_out)
{
    const int tid = threadIdx.x;
    sum_s = wave_sum_any(sum_s);
    sum_w = wave_sum_any(sum_w);
    if ((tid & 63) == 0) {
        part[tid >> 6] = sum_s;
        part[4 + (tid >> 6)] = sum_w;
    }
    PHASE(3072, 1);
    __syncthreads();
    PHASE(3072, 2);
    /* the same operations in the same order on every thread: S, W and the verdict are uniform */
    const double S = (part[0] + part[1]) + (part[2] + part[3]);
    const double W = (part[4] + part[5]) + (part[6] + part[7]);
    bool open = walk || !__builtin_isfinite(S) || !__builtin_isfinite(W);
    double inv_lo = 0.0;
    if (!open) {
        const double err = W * 0x1.00001p-53 + S * ((double)(E / 256 + 16) * 0x1p-52);
        inv_lo = 1.0 / sqrt((S + err) / E + (double)eps);
        const double inv_hi = 1.0 / sqrt((S - err) / E + (double)eps);
        const bool differ = !same(inv_lo, inv_hi);
        stage(inv_lo);                 /* the caller's use of the bracket's answer, before the vote */
        open = __syncthreads_or(differ);
    }
    open_out = open;
    if (!open) return inv_lo;
    fill();
    __syncthreads();
    if (tid < 64) {
        double ss;
        if (E % 512 == 0) {
            ss = ordered_sum_chunked(q, E >> 6);
            PHASE(3072, 5);
        } else {
            ss = 0.0;
            if (tid == 0)
                for (int i = 0; i < E; i++) ss += q[i];
        }
        if (tid == 0) {
            *inv_sh = 1.0 / sqrt(ss / E + (double)eps);
            if (walked) atomicAdd(walked, 1ull);
        }
    }
    __syncthreads();
    return *inv_sh;
}

/* Whether a float4 of x gives the same (float)(x * inv) at inv = lo and inv = hi. */
__device__ __forceinline__ bool same_at_both(float4 a, double lo, double hi)
{
    return (float)((double)a.x * lo) == (float)((double)a.x * hi) &&
           (float)((double)a.y * lo) == (float)((double)a.y * hi) &&
           (float)((double)a.z * lo) == (float)((double)a.z * hi) &&
           (float)((double)a.w * lo) == (float)((double)a.w * hi);
}

/* y = (float)(x * inv) * w for a float4. */
__device__ __forceinline__ float4 norm_apply(float4 a, float4 b, double v)
{
    return make_float4((float)((double)a.x * v) * b.x, (float)((double)a.y * v) * b.y,
                       (float)((double)a.z * v) * b.z, (float)((double)a.w * v) * b.w);
}

/* The squares of a float4 of x at float4 index i of the row into the partial sums: sum_s of
 * the squares, sum_w of the squares weighted by E - j (j the element's index). */
__device__ __forceinline__ void norm_partials(float4 v, int i, int E, double &sum_s, double &sum_w)
{
    const double sq[4] = { (double)v.x * (double)v.x, (double)v.y * (double)v.y,
                           (double)v.z * (double)v.z, (double)v.w * (double)v.w };
#pragma unroll
    for (int k = 0; k < 4; k++) {
        sum_s += sq[k];
        sum_w += sq[k] * (double)(E - (4 * i + k));
    }
}

/* The squares of a float4 of x at float4 index i of the row into q in the ordered sum's layout:
 * for chunked rows element 4i + k at lane (4i + k) / C, term (4i + k) % C of its chunk. */
__device__ __forceinline__ void norm_store(float4 v, int i, int E, double *q)
{
    const bool chunked = E % 512 == 0;
    const int C = E >> 6;
    const double sq[4] = { (double)v.x * (double)v.x, (double)v.y * (double)v.y,
                           (double)v.z * (double)v.z, (double)v.w * (double)v.w };
    const int lj = chunked ? (4 * i) / C : 0, ti = 4 * i - lj * C;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        if (chunked) q[(ti + k) * kSumPitch + lj] = sq[k];
        else q[4 * i + k] = sq[k];
    }
}

__global__ __launch_bounds__(256) void rmsnorm_kernel(float *x, const float *add, const float *w, float *y, int E,
                                                      float eps, int walk, unsigned long long *walked)
{
    extern __shared__ __align__(16) double q[];      /* the squares */
    __shared__ double inv_sh, part[8];
    PHASE(3072, 0);
    float4 *xrow = (float4 *)(x + (size_t)blockIdx.x * E);
    const float4 *arow = add ? (const float4 *)(add + (size_t)blockIdx.x * E) : nullptr;
    const float4 *row = xrow;
    const float4 *w4 = (const float4 *)w;
    float4 *out = (float4 *)(y + (size_t)blockIdx.x * E);
    const int n4 = E >> 2, tid = threadIdx.x;
    const bool held = n4 <= 256 * kNormVec;
    const float4 one = make_float4(1.0f, 1.0f, 1.0f, 1.0f);
    float4 xv[kNormVec], wv[kNormVec];
    double sum_s = 0.0, sum_w = 0.0;
    for (int base = 0; base < n4; base += 256 * kNormVec) {
#pragma unroll
        for (int m = 0; m < kNormVec; m++) {
            const int i = base + tid + 256 * m;
            if (i < n4) {
                xv[m] = row[i];
                wv[m] = w ? w4[i] : one;
            }
        }
        if (arow) {
#pragma unroll
            for (int m = 0; m < kNormVec; m++) {
                const int i = base + tid + 256 * m;
                if (i < n4) {
                    const float4 d = arow[i];
                    xv[m] = make_float4(xv[m].x + d.x, xv[m].y + d.y, xv[m].z + d.z, xv[m].w + d.w);
                    xrow[i] = xv[m];
                }
            }
        }
#pragma unroll
        for (int m = 0; m < kNormVec; m++) {
            const int i = base + tid + 256 * m;
            if (i < n4) norm_partials(xv[m], i, E, sum_s, sum_w);
        }
    }
    auto same = [&](double lo, double hi) {
        bool ok = true;
        if (held) {
#pragma unroll
            for (int m = 0; m < kNormVec; m++) {
                const int i = tid + 256 * m;
                if (i < n4 && !same_at_both(xv[m], lo, hi)) ok = false;
            }
        } else {
            for (int i = tid; i < n4; i += 256)
                if (!same_at_both(row[i], lo, hi)) ok = false;
        }
        return ok;
    };
    auto fill = [&]() {
        if (held) {
#pragma unroll
            for (int m = 0; m < kNormVec; m++) {
                const int i = tid + 256 * m;
                if (i < n4) norm_store(xv[m], i, E, q);
            }
        } else {
            for (int i = tid; i < n4; i += 256) norm_store(row[i], i, E, q);
        }
    };
    bool open;
    const double v = norm_inv(sum_s, sum_w, q, E, eps, walk, walked, same, fill, part, &inv_sh, [](double) {},
                              open);
    PHASE(3072, 6);
    if (held) {
#pragma unroll
        for (int m = 0; m < kNormVec; m++) {
            const int i = tid + 256 * m;
            if (i < n4) out[i] = norm_apply(xv[m], wv[m], v);
        }
    } else {
        for (int i = tid; i < n4; i += 256) out[i] = norm_apply(row[i], w ? w4[i] : one, v);
    }
    PHASE(3072, 3);
}

/* rmsnorm fused ahead of the one-token router, for the layer chain (src/model.c:1283-1284, then
 * the router of src/model.c:1032-1167 as route_small_kernel<1> runs it): every block forms
 * x = h + add (float) and xn = rmsnorm(x) * w itself, bit for bit as rmsnorm_kernel does (the
 * bracket, and the ordered sum where it is open); router blocks, one per expert, then run the
 * expert's 16 FMA chains over xn staged chain-major in LDS, and the last block stores x to
 * h_out (when add is not null), xn to xn_out and the int8 input blocks of xn. h_out is not h,
 * which every block reads. E a multiple of 512, at most 4096. */
__global__ __launch_bounds__(256) void route_norm_kernel(RouteArgs a, NormIn n)
{
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ double inv_sh, part[8];
    constexpr int NV = 4;                            /* float4s i = tid + 256 m, E <= 4096 */
    const int tid = threadIdx.x, E = a.E, n4 = E >> 2, e = blockIdx.x;
    const bool router = e < a.n_route_wg;
    const int C = E >> 6, CS = E / 16 + 4;
    double *q = (double *)smem;                      /* the squares: C * kSumPitch doubles */
    float *buf = (float *)(smem + (size_t)C * kSumPitch * 8);   /* [2 rows][16 chains][CS] */
    const float4 *h4 = (const float4 *)n.h, *a4 = (const float4 *)n.add, *w4 = (const float4 *)n.w;
    const float4 *r4 = (const float4 *)(a.router + (size_t)(router ? e : 0) * E);
    const float4 one = make_float4(1.0f, 1.0f, 1.0f, 1.0f);
    float4 xv[NV], wv[NV], rv[NV];
#pragma unroll
    for (int m = 0; m < NV; m++) {
        const int i = tid + 256 * m;
        if (i < n4) {
            if (router) rv[m] = r4[i];
            xv[m] = h4[i];
            wv[m] = w4 ? w4[i] : one;
            if (a4) {
                const float4 d = a4[i];
                xv[m] = make_float4(xv[m].x + d.x, xv[m].y + d.y, xv[m].z + d.z, xv[m].w + d.w);
            }
        }
    }
    double sum_s = 0.0, sum_w = 0.0;
#pragma unroll
    for (int m = 0; m < NV; m++) {
        const int i = tid + 256 * m;
        if (i < n4) norm_partials(xv[m], i, E, sum_s, sum_w);
    }
    auto same = [&](double lo, double hi) {
        bool ok = true;
#pragma unroll
        for (int m = 0; m < NV; m++) {
            const int i = tid + 256 * m;
            if (i < n4 && !same_at_both(xv[m], lo, hi)) ok = false;
        }
        return ok;
    };
    auto fill = [&]() {
#pragma unroll
        for (int m = 0; m < NV; m++) {
            const int i = tid + 256 * m;
            if (i < n4) norm_store(xv[m], i, E, q);
        }
    };
    float4 xn[NV];
    float4 *lin = (float4 *)buf;
    /* router blocks: the router row and xn chain-major (float4 j holds elements 4j .. 4j+3:
     * chains 4(j%4) .. 4(j%4)+3, step j/4); the quantiser block: xn in order */
    auto stage = [&](double v) {
#pragma unroll
        for (int m = 0; m < NV; m++) {
            const int j = tid + 256 * m;
            if (j >= n4) continue;
            xn[m] = norm_apply(xv[m], wv[m], v);
            if (router) {
                float *dw = buf + (4 * (j & 3)) * CS + (j >> 2), *dx = dw + 16 * CS;
                dw[0] = rv[m].x; dw[CS] = rv[m].y; dw[2 * CS] = rv[m].z; dw[3 * CS] = rv[m].w;
                dx[0] = xn[m].x; dx[CS] = xn[m].y; dx[2 * CS] = xn[m].z; dx[3 * CS] = xn[m].w;
            } else {
                lin[j] = xn[m];
            }
        }
    };
    bool open;
    const double v = norm_inv(sum_s, sum_w, q, E, n.eps, n.walk, router ? nullptr : n.walked, same, fill, part,
                              &inv_sh, stage, open);
    if (open) {
        stage(v);
        __syncthreads();
    }
    if (router) {
        if (tid < 16) {
            const float4 *wr = (const float4 *)(buf + tid * CS), *xr = (const float4 *)(buf + (16 + tid) * CS);
            const int q1 = E / 64;                   /* float4 steps of one chain */
            float acc = 0.0f;
            if ((q1 & 7) == 0) acc = chain_steps<8>(wr, xr, 0, q1, acc);
            else acc = chain_steps<1>(wr, xr, 0, q1, acc);
            acc = chain16_sum(acc);
            if (tid == 0) a.y[e] = acc;
        }
        return;
    }
#pragma unroll
    for (int m = 0; m < NV; m++) {
        const int i = tid + 256 * m;
        if (i < n4) {
            if (a4) ((float4 *)n.h_out)[i] = xv[m];
            ((float4 *)n.xn_out)[i] = xn[m];
        }
    }
    const int nbE = E >> 5;
    if (tid < nbE) {
        float vb[32];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float4 f = lin[8 * tid + j];
            vb[4 * j] = f.x; vb[4 * j + 1] = f.y; vb[4 * j + 2] = f.z; vb[4 * j + 3] = f.w;
        }
        uint32_t *pair = (uint32_t *)(a.S.xqk + (size_t)(tid >> 1) * kPairBytes);
        quantize_block_store(vb, a.S.xq + tid, pair, tid & 1);
    }
}

hipError_t launch_route_norm(const Shape &s, const LayerDev &L, const Scratch &S, const NormIn &n, hipStream_t st)
{
    if (!route_norm_fits(s.E) || !n.h || !n.xn_out || (n.add && (!n.h_out || n.h_out == n.h)))
        return hipErrorInvalidValue;
    RouteArgs a;
    a.router = L.router;
    a.xn = n.xn_out;
    a.E = s.E;
    a.X = s.X;
    a.K = s.K;
    a.T = 1;
    a.y = S.logits;
    a.ystride = s.X;
    a.S = S;
    a.n_route_wg = s.X;
    const size_t lds = (size_t)(s.E / 64) * kSumPitch * 8 + (size_t)2 * 16 * (s.E / 16 + 4) * 4;
    QLAUNCH("route", route_norm_kernel, dim3(s.X + 1), dim3(256), lds, st, a, n);
    return hipGetLastError();
}

hipError_t launch_rmsnorm(float *x, const float *add, const float *w, float *y, int T, int E, float eps,
                          int walk, unsigned long long *walked, hipStream_t st)
{
    if (T <= 0) return hipSuccess;
    if (E % 4) return hipErrorInvalidValue;
    static_assert(kSumPitch == 65, "rmsnorm_lds_bytes assumes the pitch");
    if (rmsnorm_lds_bytes(E) > 160 * 1024) return hipErrorInvalidValue;
    QLAUNCH("rmsnorm", rmsnorm_kernel, dim3(T), dim3(256), rmsnorm_lds_bytes(E), st, x, add, w, y, E, eps, walk,
            walked);
    return hipGetLastError();
}

/* dst = h + d (src/model.c:1285), float adds; dst may be h. */
__global__ void add_rows_kernel(float4 *dst, const float4 *h, const float4 *d, size_t n4)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n4) {
        float4 a = h[i];
        const float4 b = d[i];
        a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
        dst[i] = a;
    }
}

hipError_t launch_add_rows_to(float *dst, const float *h, const float *d, size_t n, hipStream_t st)
{
    if (n % 4) return hipErrorInvalidValue;
    const size_t n4 = n / 4;
    if (n4) QLAUNCH("add", add_rows_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st, (float4 *)dst,
                    (const float4 *)h, (const float4 *)d, n4);
    return hipGetLastError();
}

hipError_t launch_add_rows(float *h, const float *d, size_t n, hipStream_t st)
{
    return launch_add_rows_to(h, h, d, n, st);
}

__global__ void set_col0_kernel(float *m, int rows, int stride, const float *vals, float fill)
{
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r < rows) m[(size_t)r * stride] = vals ? vals[r] : fill;
}

hipError_t launch_set_col0(float *m, int rows, int stride, const float *vals, float fill, hipStream_t st)
{
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(set_col0_kernel, dim3((rows + 255) / 256), dim3(256), 0, st, m, rows, stride, vals, fill);
    return hipGetLastError();
}

}  // namespace qmsg
