/* qmsg_kernels.hip - gfx950 kernels for the Qwen3-MoE expert-FFN layer (exact path).
 *
 * Layer = route (router dots + int8 input blocks + softmax/top-K + counting sort, one launch)
 *       -> gateup (gate/up row dots over Q4_0, SwiGLU, int8 activation blocks, one launch)
 *       -> down   (down row dots over Q4_0/Q6_K, weighted combine, one launch).
 *
 * Every fp32 operation reproduces the reference's AVX2 order (src/kernels.c, src/model.c):
 * each row's dot is eight 4-element int32 lanes per 32-block, a per-lane fp32 FMA chain
 * over blocks, an FMA chain for the offset term, the hsum256 tree and an unfused final
 * subtraction. Build with -ffp-contract=off: every fused multiply-add here is explicit.
 *
 * Work mapping (64-wide waves): one quad of lanes per weight row; lane p of the quad owns
 * the reference lanes k = p (low nibbles) and k = p + 4 (high nibbles), which read the same
 * code dword. Weight tiles stream from HBM with 16-byte coalesced loads into LDS; the int8
 * activations sit in LDS in a pair-of-blocks layout so a lane gets its two code partners
 * with one 16-byte read. */
#include <hip/hip_runtime.h>

#include "qmsg_internal.h"
#include "qmsg_synth.h"

namespace qmsg {

/* ------------------------------------------------------------------ scalar helpers ---- */

__device__ __forceinline__ float h2f(uint32_t bits16)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

__device__ __forceinline__ int sdot4(int a, int b) { return __builtin_amdgcn_sdot4(a, b, 0, false); }

/* 2^(i/32) rounded to double, minus i << 47 (the exponent part added back at use). */
__device__ const uint64_t kExp2fTab[32] = {
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
    0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
    0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
    0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
    0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
    0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL
};

/* expf with the same result bits as the host C library the reference links (glibc 2.35's
 * FMA variant on x86-64, which implements the ARM optimized-routines method: x*32/ln2 =
 * k + r with round-to-nearest via a 1.5*2^52 shift, 2^(k/32) from the table above, a cubic
 * in r, everything in double, one final rounding to float). Checked on all 2^32 inputs. */
__device__ __forceinline__ float expf_ref(float x)
{
    const uint32_t ux = __float_as_uint(x);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {                     /* |x| >= 88, inf or nan */
        if (ux == 0xff800000u) return 0.0f;
        if (abstop >= 0x7f8u) return x + x;
        if (x > 0x1.62e42ep6f) return __builtin_inff();
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double InvLn2N = 0x1.71547652b82fep+0 * 32.0, Shift = 0x1.8p+52;
    const double C0 = 0x1.c6af84b912394p-5 / 32768.0, C1 = 0x1.ebfce50fac4f3p-3 / 1024.0,
                 C2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    double kd = __builtin_fma(InvLn2N, xd, Shift);
    const uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd -= Shift;
    const double r = __builtin_fma(InvLn2N, xd, -kd);
    const uint64_t t = kExp2fTab[ki & 31u] + (ki << 47);
    const double s = __longlong_as_double((long long)t);
    const double z = __builtin_fma(C0, r, C1);
    const double r2 = r * r;
    double y = __builtin_fma(C2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}

/* src/model.c:424 */
__device__ __forceinline__ float silu_ref(float a) { return a / (1.0f + expf_ref(-a)); }

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
__device__ void quantize_block_store(const float *v, Q8 *dst, uint32_t *pair, int half)
{
    float amax = 0.0f;
    for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(v[j]));
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    int8_t q[32];
    int s0 = 0, s1 = 0;
    for (int j = 0; j < 32; j++) {
        const int qi = (int)rintf(v[j] * id);
        q[j] = (int8_t)qi;
        if (j < 16) s0 += qi; else s1 += qi;
    }
    const float ds = d * (float)(s0 + s1);
    const uint32_t s16 = (uint32_t)(uint16_t)(int16_t)s0 | ((uint32_t)(uint16_t)(int16_t)s1 << 16);
    uint32_t *o = (uint32_t *)dst;
    o[0] = __float_as_uint(d);
    o[1] = __float_as_uint(ds);
    o[2] = s16;
    for (int w = 0; w < 8; w++) o[3 + w] = pack4(q + 4 * w);
    for (int p = 0; p < 4; p++) {
        pair[4 * p + 2 * half] = pack4(q + 4 * p);
        pair[4 * p + 2 * half + 1] = pack4(q + 16 + 4 * p);
    }
    pair[16 + 2 * half] = __float_as_uint(d);
    pair[17 + 2 * half] = __float_as_uint(ds);
    pair[20 + half] = s16;
    if (half == 0) { pair[22] = 0; pair[23] = 0; }
}

/* ------------------------------------------------------------------ route ---- */

struct RouteArgs {
    const float *router, *xn;
    int E, X, K, T, n_dot_wg;
    Scratch S;
};

/* Softmax over one token's logits in double, K rounds of argmax with ties to the lower
 * index, weights renormalised over the selection (src/model.c:1045-1064). One wave. */
__device__ void topk_token(const RouteArgs &a, int t, double *P, int *taken)
{
    const int X = a.X, K = a.K, lane = threadIdx.x;
    const float *lt = a.S.logits + (size_t)t * a.X;
    double mx = -__builtin_inf();
    for (int e = lane; e < X; e += 64) {
        const double v = (double)lt[e];
        if (v > mx) mx = v;
    }
    for (int o = 32; o > 0; o >>= 1) {
        const double v = __shfl_xor(mx, o);
        if (v > mx) mx = v;
    }
    for (int e = lane; e < X; e += 64) {
        P[e] = exp((double)lt[e] - mx);
        taken[e] = 0;
    }
    __syncthreads();
    double z = 0.0;
    if (lane == 0)
        for (int e = 0; e < X; e++) z += P[e];           /* sequential, as the reference */
    z = __shfl(z, 0);
    for (int e = lane; e < X; e += 64) P[e] /= z;
    __syncthreads();
    double wsum = 0.0;
    int *sel = a.S.sel + (size_t)t * K;
    for (int j = 0; j < K; j++) {
        double bp = 0.0;
        int be = -1;
        for (int e = lane; e < X; e += 64)
            if (!taken[e] && (be < 0 || P[e] > bp)) { bp = P[e]; be = e; }
        for (int o = 32; o > 0; o >>= 1) {
            const double op = __shfl_xor(bp, o);
            const int oe = __shfl_xor(be, o);
            if (oe >= 0 && (be < 0 || op > bp || (op == bp && oe < be))) { bp = op; be = oe; }
        }
        if (lane == 0) {
            sel[j] = be;
            taken[be] = 1;
            wsum += P[be];
        }
        __syncthreads();
    }
    if (lane == 0)
        for (int j = 0; j < K; j++) a.S.wt[(size_t)t * K + j] = (float)(P[sel[j]] / wsum);
}

/* Counting sort of the T*K (token, selection) slots by expert, src/model.c:1066-1088:
 * slots of one expert are contiguous, experts ascend, and inside an expert slots follow
 * token order then selection order. One wave. */
__device__ void dispatch_slots(const RouteArgs &a, int *cnt, int *cur)
{
    const int X = a.X, NS = a.T * a.K, lane = threadIdx.x;
    for (int e = lane; e < X; e += 64) { cnt[e] = 0; cur[e] = 0; }
    __syncthreads();
    for (int i = lane; i < NS; i += 64) atomicAdd(&cnt[a.S.sel[i]], 1);
    __syncthreads();
    if (lane == 0) {
        int acc = 0, na = 0;
        a.S.start[0] = 0;
        for (int e = 0; e < X; e++) {
            const int c = cnt[e];
            cnt[e] = acc;                    /* cnt now holds start[e] */
            acc += c;
            a.S.start[e + 1] = acc;
            if (c) a.S.active[na++] = e;
        }
        a.S.meta[0] = na;
    }
    __syncthreads();
    const unsigned long long below = (1ULL << lane) - 1ULL;
    for (int base = 0; base < NS; base += 64) {
        const int i = base + lane;
        const int e = i < NS ? a.S.sel[i] : -1;
        unsigned long long same = __ballot(i < NS);
        for (int bit = 0; bit < 9; bit++) {
            const unsigned long long b = __ballot(i < NS && ((e >> bit) & 1));
            same &= ((e >> bit) & 1) ? b : ~b;
        }
        int s = 0;
        if (i < NS) s = cnt[e] + cur[e] + __popcll(same & below);
        __syncthreads();
        if (i < NS) {
            a.S.slot_t[s] = i / a.K;
            a.S.slot_of[i] = s;
            if ((same >> lane) == 1ULL) cur[e] += __popcll(same);   /* highest lane of the group */
        }
        __syncthreads();
    }
}

/* Router dots + input quantisation. Blocks [0, n_dot_wg): one wave, four (token, expert)
 * dots of 16 lanes each; lane c runs the reference's FMA chain over elements c, c+16, ...
 * (two 8-lane AVX registers = 16 chains), then the hsum256 tree over the 16 chain sums.
 * The last block to finish a token runs its top-K; the last token to finish runs the
 * counting sort. Remaining blocks quantise the input rows, one 32-block per thread. */
__global__ __launch_bounds__(64) void route_kernel(RouteArgs a)
{
    __shared__ double P[256];
    __shared__ int taken[256];
    __shared__ int cnt[256], cur[256];
    __shared__ int flag;
    const int lane = threadIdx.x;
    if ((int)blockIdx.x >= a.n_dot_wg) {
        const int nbE = a.E >> 5;
        const int b = ((int)blockIdx.x - a.n_dot_wg) * 64 + lane;
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
        return;
    }
    const int dot = (int)blockIdx.x * 4 + (lane >> 4), c = lane & 15;
    const int t = dot / a.X, e = dot - t * a.X;
    const float *w = a.router + (size_t)e * a.E, *x = a.xn + (size_t)t * a.E;
    const int E16 = a.E & ~15;
    float acc = 0.0f;
#pragma unroll 16
    for (int i = c; i < E16; i += 16) acc = __builtin_fmaf(w[i], x[i], acc);
    acc += __shfl_down(acc, 8, 16);      /* v_j = a0_j + a1_j            */
    acc += __shfl_down(acc, 4, 16);      /* s_j = v_j + v_{j+4}          */
    acc += __shfl_down(acc, 2, 16);      /* (s0 + s2), (s1 + s3)         */
    acc += __shfl_down(acc, 1, 16);      /* (s0 + s2) + (s1 + s3)        */
    if (c == 0) {
        for (int i = E16; i < a.E; i++) acc = __builtin_fmaf(w[i], x[i], acc);
        a.S.logits[(size_t)t * a.X + e] = acc;
    }
    __threadfence();
    if (lane == 0) flag = atomicAdd(&a.S.tok_cnt[t], 1) == a.X / 4 - 1;
    __syncthreads();
    if (!flag) return;
    __threadfence();
    topk_token(a, t, P, taken);
    if (lane == 0) a.S.tok_cnt[t] = 0;
    __threadfence();
    if (lane == 0) flag = atomicAdd(&a.S.meta[1], 1) == a.T - 1;
    __syncthreads();
    if (!flag) return;
    __threadfence();
    dispatch_slots(a, cnt, cur);
    if (lane == 0) a.S.meta[1] = 0;
}

hipError_t launch_route(const Shape &s, const LayerDev &L, const Scratch &S, const float *xn, int T, hipStream_t st)
{
    RouteArgs a;
    a.router = L.router;
    a.xn = xn;
    a.E = s.E;
    a.X = s.X;
    a.K = s.K;
    a.T = T;
    a.n_dot_wg = T * s.X / 4;
    a.S = S;
    const int nq = (T * (s.E / 32) + 63) / 64;
    hipLaunchKernelGGL(route_kernel, dim3(a.n_dot_wg + nq), dim3(64), 0, st, a);
    return hipGetLastError();
}

/* ------------------------------------------------------------------ expert row dots ---- */

/* Running state of one quad's row dot for one token: the two reference lanes this lane
 * owns and the offset chain (identical on the four lanes of the quad). */
struct RowAcc {
    float lo, hi, corr;
};

/* One pair of Q4_0 blocks (36 bytes at W, 4-byte aligned) against one token's pair record.
 * src/kernels.c:87-93 for blocks b and b+1, lanes k = p and p + 4. */
__device__ __forceinline__ void q4_0_pair(const uint32_t *W, int p, const uint8_t *xp, RowAcc &r)
{
    const uint32_t w0 = W[0], w4 = W[4], wa = W[p], wb = W[p + 1], wc = W[5 + p];
    const uint32_t c0 = __builtin_amdgcn_alignbyte(wb, wa, 2);
    const float d0 = h2f(w0 & 0xffffu), d1 = h2f(w4 >> 16);
    const uint4 xv = *(const uint4 *)(xp + 16 * p);
    const float4 dv = *(const float4 *)(xp + 64);
    const float m0 = d0 * dv.x;
    r.lo = __builtin_fmaf((float)sdot4((int)(c0 & 0x0f0f0f0fu), (int)xv.x), m0, r.lo);
    r.hi = __builtin_fmaf((float)sdot4((int)((c0 >> 4) & 0x0f0f0f0fu), (int)xv.y), m0, r.hi);
    r.corr = __builtin_fmaf(d0, dv.y, r.corr);
    const float m1 = d1 * dv.z;
    r.lo = __builtin_fmaf((float)sdot4((int)(wc & 0x0f0f0f0fu), (int)xv.z), m1, r.lo);
    r.hi = __builtin_fmaf((float)sdot4((int)((wc >> 4) & 0x0f0f0f0fu), (int)xv.w), m1, r.hi);
    r.corr = __builtin_fmaf(d1, dv.w, r.corr);
}

/* One Q6_K 32-block (index g of half h of the super-block at byte sb of the LDS tile)
 * against one token's block, src/kernels.c:148-167: lanes k < 4 use sc[2g], k >= 4 sc[2g+1]. */
__device__ __forceinline__ void q6_k_block(const uint8_t *tile, uint32_t sb, int h, int g, int p, const uint8_t *xp,
                                           int xhalf, RowAcc &r)
{
    const uint32_t qlo = lds_u32(tile, sb + 64 * h + 32 * (g & 1) + 4 * p);
    const uint32_t qhi = lds_u32(tile, sb + 64 * h + 32 * (g & 1) + 16 + 4 * p);
    const uint32_t hlo = lds_u32(tile, sb + 128 + 32 * h + 4 * p);
    const uint32_t hhi = lds_u32(tile, sb + 128 + 32 * h + 16 + 4 * p);
    const uint32_t scw = lds_u32(tile, sb + 192 + 8 * h + 2 * g);
    const float d = h2f(lds_u32(tile, sb + 208) & 0xffffu);
    const int sa = (int)(int8_t)(scw & 0xff), sbb = (int)(int8_t)((scw >> 8) & 0xff);
    const int sh = 2 * g;
    const uint32_t nlo = g < 2 ? (qlo & 0x0f0f0f0fu) : ((qlo >> 4) & 0x0f0f0f0fu);
    const uint32_t nhi = g < 2 ? (qhi & 0x0f0f0f0fu) : ((qhi >> 4) & 0x0f0f0f0fu);
    const uint32_t q6lo = nlo | (((hlo >> sh) & 0x03030303u) << 4);
    const uint32_t q6hi = nhi | (((hhi >> sh) & 0x03030303u) << 4);
    const uint32_t xlo = *(const uint32_t *)(xp + 16 * p + 8 * xhalf);
    const uint32_t xhi = *(const uint32_t *)(xp + 16 * p + 8 * xhalf + 4);
    const float xd = *(const float *)(xp + 64 + 8 * xhalf);
    const uint32_t s16 = *(const uint32_t *)(xp + 80 + 4 * xhalf);
    const int s16a = (int)(int16_t)(s16 & 0xffffu), s16b = (int)(int16_t)(s16 >> 16);
    const float dd = d * xd;
    r.lo = __builtin_fmaf((float)(sdot4((int)q6lo, (int)xlo) * sa), dd, r.lo);
    r.hi = __builtin_fmaf((float)(sdot4((int)q6hi, (int)xhi) * sbb), dd, r.hi);
    r.corr = __builtin_fmaf(dd, (float)(sa * s16a + sbb * s16b), r.corr);
}

/* hsum256 over the quad, then the unfused offset subtraction. Valid on lane p == 0. */
__device__ __forceinline__ float quad_finish(const RowAcc &r, float scale)
{
    const float s = r.lo + r.hi;                      /* s_p = acc_p + acc_{p+4}   */
    const float t = s + __shfl_down(s, 2, 4);         /* (s0+s2) on p0, (s1+s3) on p1 */
    const float h = t + __shfl_down(t, 1, 4);
    return h - scale * r.corr;
}

/* ------------------------------------------------------------------ gate / up ---- */

struct GateUpArgs {
    const uint8_t *gate, *up;
    uint64_t rb, eb;
    int E, F, CB, wstride, debug;
    Scratch S;
};

/* One block: expert active[blockIdx.y], gate rows and up rows r0 .. r0+31 (r0 = 32*blockIdx.x),
 * for every slot of that expert, NT slots per pass. Rows 0-31 of the tile are gate, 32-63 up.
 * Epilogue: a = silu(g)*u (src/model.c:989-997), then one 32-block of int8 activations. */
template <int NT>
__global__ __launch_bounds__(256) void gateup_exact_kernel(GateUpArgs a)
{
    extern __shared__ __align__(16) uint8_t smem[];
    const int nbE = a.E >> 5, nP = nbE >> 1, CB = a.CB, WS = a.wstride;
    const int nchunk = nbE / CB, spr = CB * 18 / 16, nslot = 64 * spr;
    uint8_t *wbuf = smem;
    uint8_t *xbuf = smem + 64 * WS;
    float *res = (float *)(xbuf + NT * nP * kPairBytes);
    int8_t *qb = (int8_t *)(res + NT * 64);

    const int ai = blockIdx.y;
    if (ai >= a.S.meta[0]) return;
    const int e = a.S.active[ai];
    const int s_begin = a.S.start[e], s_end = a.S.start[e + 1];
    const int r0 = (int)blockIdx.x * 32;
    const int tid = threadIdx.x, rho = tid >> 2, p = tid & 3;
    const uint8_t *gbase = a.gate + (size_t)e * a.eb, *ubase = a.up + (size_t)e * a.eb;
    const int F = a.F, nbF = F >> 5;

    for (int g0 = s_begin; g0 < s_end; g0 += NT) {
        const int nt = min(NT, s_end - g0);
        for (int i = tid; i < nt * nP * 6; i += 256) {
            const int n = i / (nP * 6), off = i - n * nP * 6;
            const int tok = a.S.slot_t[g0 + n];
            ((uint4 *)xbuf)[n * nP * 6 + off] = ((const uint4 *)(a.S.xqk + (size_t)tok * nP * kPairBytes))[off];
        }
        RowAcc acc[NT];
        for (int n = 0; n < NT; n++) acc[n] = RowAcc{ 0.0f, 0.0f, 0.0f };
        /* register double buffer: nine 16-byte slots per thread cover a 64 x 576-byte chunk */
        uint4 p0, p1, p2, p3, p4, p5, p6, p7, p8;
#define QMSG_SLOT_SRC(m, c)                                                                         \
    ({                                                                                              \
        const int i_ = min(tid + 256 * (m), nslot - 1);                                             \
        const int row_ = i_ / spr, j_ = i_ - row_ * spr;                                            \
        (const uint4 *)((row_ < 32 ? gbase + (size_t)(r0 + row_) * a.rb                              \
                                   : ubase + (size_t)(r0 + row_ - 32) * a.rb) +                      \
                        (size_t)(c) * CB * 18 + 16 * j_);                                           \
    })
#define QMSG_SLOT_DST(m)                                                                            \
    ({                                                                                              \
        const int i_ = min(tid + 256 * (m), nslot - 1);                                             \
        const int row_ = i_ / spr, j_ = i_ - row_ * spr;                                            \
        (uint4 *)(wbuf + row_ * WS + 16 * j_);                                                      \
    })
#define QMSG_LOAD_ALL(c)                                                                            \
    p0 = *QMSG_SLOT_SRC(0, c); p1 = *QMSG_SLOT_SRC(1, c); p2 = *QMSG_SLOT_SRC(2, c);                \
    p3 = *QMSG_SLOT_SRC(3, c); p4 = *QMSG_SLOT_SRC(4, c); p5 = *QMSG_SLOT_SRC(5, c);                \
    p6 = *QMSG_SLOT_SRC(6, c); p7 = *QMSG_SLOT_SRC(7, c); p8 = *QMSG_SLOT_SRC(8, c);
        QMSG_LOAD_ALL(0)
        for (int c = 0; c < nchunk; c++) {
            __syncthreads();
            *QMSG_SLOT_DST(0) = p0; *QMSG_SLOT_DST(1) = p1; *QMSG_SLOT_DST(2) = p2;
            *QMSG_SLOT_DST(3) = p3; *QMSG_SLOT_DST(4) = p4; *QMSG_SLOT_DST(5) = p5;
            *QMSG_SLOT_DST(6) = p6; *QMSG_SLOT_DST(7) = p7; *QMSG_SLOT_DST(8) = p8;
            __syncthreads();
            if (c + 1 < nchunk) { QMSG_LOAD_ALL(c + 1) }
#undef QMSG_LOAD_ALL
#undef QMSG_SLOT_DST
#undef QMSG_SLOT_SRC
            const uint32_t *Wrow = (const uint32_t *)(wbuf + rho * WS);
            for (int q = 0; q < CB / 2; q++) {
                const int gp = c * (CB / 2) + q;
#pragma unroll
                for (int n = 0; n < NT; n++)
                    if (n < nt) q4_0_pair(Wrow + q * 9, p, xbuf + (size_t)(n * nP + gp) * kPairBytes, acc[n]);
            }
        }
#pragma unroll
        for (int n = 0; n < NT; n++) {
            const float v = quad_finish(acc[n], 8.0f);
            if (p == 0 && n < nt) res[n * 64 + rho] = v;
        }
        __syncthreads();
        const int wave = tid >> 6, l = tid & 63;
        for (int n = wave; n < nt; n += 4) {
            const int s = g0 + n;
            float av = 0.0f;
            if (l < 32) {
                const float g = res[n * 64 + l], u = res[n * 64 + 32 + l];
                av = silu_ref(g) * u;
                a.S.act[(size_t)s * F + r0 + l] = av;
                if (a.debug) {
                    a.S.gu[(size_t)s * 2 * F + r0 + l] = g;
                    a.S.gu[(size_t)s * 2 * F + F + r0 + l] = u;
                }
            }
            float amax = l < 32 ? fabsf(av) : 0.0f;
            for (int o = 16; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 32));
            const float d = amax / 127.0f;
            const float id = d > 0.0f ? 1.0f / d : 0.0f;
            const int qi = (int)rintf(av * id);
            int sum = qi;
            for (int o = 8; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 16);   /* lanes 0-15, 16-31 */
            const int s0 = __shfl(sum, 0), s1 = __shfl(sum, 16);
            if (l < 32) qb[n * 32 + l] = (int8_t)qi;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
            const float ds = d * (float)(s0 + s1);
            const uint32_t s16 = (uint32_t)(uint16_t)(int16_t)s0 | ((uint32_t)(uint16_t)(int16_t)s1 << 16);
            const uint32_t *qw = (const uint32_t *)(qb + n * 32);
            uint32_t *o = (uint32_t *)(a.S.aq + (size_t)s * nbF + (r0 >> 5));
            if (l == 0) o[0] = __float_as_uint(d);
            if (l == 1) o[1] = __float_as_uint(ds);
            if (l == 2) o[2] = s16;
            if (l >= 3 && l < 11) o[l] = qw[l - 3];
            const int tile = r0 >> 5, half = tile & 1;
            uint32_t *pr = (uint32_t *)(a.S.aqk + ((size_t)s * (nbF >> 1) + (tile >> 1)) * kPairBytes);
            if (l >= 16 && l < 20) {
                const int pp = l - 16;
                pr[4 * pp + 2 * half] = qw[pp];
                pr[4 * pp + 2 * half + 1] = qw[4 + pp];
            }
            if (l == 20) pr[16 + 2 * half] = __float_as_uint(d);
            if (l == 21) pr[17 + 2 * half] = __float_as_uint(ds);
            if (l == 22) pr[20 + half] = s16;
            if (l == 23 && half == 0) { pr[22] = 0; pr[23] = 0; }
        }
        __syncthreads();
    }
}

hipError_t launch_gateup_exact(const Shape &s, const LayerDev &L, const Scratch &S, int T, int debug, hipStream_t st)
{
    GateUpArgs a;
    a.gate = L.gate;
    a.up = L.up;
    a.rb = L.gate_rb;
    a.eb = L.gate_eb;
    a.E = s.E;
    a.F = s.F;
    const int nbE = s.E / 32;
    a.CB = nbE % 32 == 0 ? 32 : (nbE % 16 == 0 ? 16 : 8);
    const int spr = a.CB * 18 / 16;
    a.wstride = a.CB * 18 + ((spr & 1) ? 0 : 16);
    a.debug = debug;
    a.S = S;
    const int nP = nbE / 2;
    const int maxact = s.X < T * s.K ? s.X : T * s.K;
    dim3 grid(s.F / 32, maxact);
    const int NT = T >= 4 ? 4 : (T >= 2 ? 2 : 1);
    const size_t lds = (size_t)64 * a.wstride + (size_t)NT * nP * kPairBytes + (size_t)NT * 64 * 4 + NT * 32;
    if (NT == 4) hipLaunchKernelGGL(gateup_exact_kernel<4>, grid, dim3(256), lds, st, a);
    else if (NT == 2) hipLaunchKernelGGL(gateup_exact_kernel<2>, grid, dim3(256), lds, st, a);
    else hipLaunchKernelGGL(gateup_exact_kernel<1>, grid, dim3(256), lds, st, a);
    return hipGetLastError();
}

/* ------------------------------------------------------------------ down + combine ---- */

struct DownArgs {
    const uint8_t *down;
    uint64_t rb, eb;
    int E, F, K, T, type;
    float *out;
    Scratch S;
};

/* One block: expert active[blockIdx.y], down rows r0 .. r0+ROWS-1 (one contiguous byte range,
 * staged whole into LDS), for every slot of that expert; dn[s][r] to HBM. The last block to
 * finish a row tile forms out[t][r] = sum_j wt[t][j] * dn[slot_of[t][j]][r] in selection
 * order (src/model.c:1152-1162). */
template <int TYPE, int ROWS, int NT>
__global__ __launch_bounds__(4 * ROWS) void down_exact_kernel(DownArgs a)
{
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int NTH = 4 * ROWS;
    const int nbF = a.F >> 5, nPF = nbF >> 1, E = a.E;
    const int tile_bytes = (int)(ROWS * a.rb);
    uint8_t *tile = smem;
    uint8_t *xbuf = smem + ((tile_bytes + 16 + 15) & ~15);
    __shared__ int flag;
    const int tid = threadIdx.x, rho = tid >> 2, p = tid & 3;
    const int ai = blockIdx.y, r0 = (int)blockIdx.x * ROWS;
    const int n_active = a.S.meta[0];
    if (ai >= n_active) return;
    const int e = a.S.active[ai];
    const int s_begin = a.S.start[e], s_end = a.S.start[e + 1];

    const uint4 *src = (const uint4 *)(a.down + (size_t)e * a.eb + (size_t)r0 * a.rb);
    for (int i = tid; i < tile_bytes / 16; i += NTH) ((uint4 *)tile)[i] = src[i];

    for (int g0 = s_begin; g0 < s_end; g0 += NT) {
        const int nt = min(NT, s_end - g0);
        __syncthreads();
        for (int i = tid; i < nt * nPF * 6; i += NTH) {
            const int n = i / (nPF * 6), off = i - n * nPF * 6;
            ((uint4 *)xbuf)[n * nPF * 6 + off] = ((const uint4 *)(a.S.aqk + (size_t)(g0 + n) * nPF * kPairBytes))[off];
        }
        __syncthreads();
        RowAcc acc[NT];
        for (int n = 0; n < NT; n++) acc[n] = RowAcc{ 0.0f, 0.0f, 0.0f };
        if (TYPE == 2) {    /* Q4_0: pairs of 18-byte blocks, 36-byte aligned within the row */
            const uint32_t *Wrow = (const uint32_t *)(tile + (size_t)rho * a.rb);
            for (int q = 0; q < nPF; q++) {
#pragma unroll
                for (int n = 0; n < NT; n++)
                    if (n < nt) q4_0_pair(Wrow + q * 9, p, xbuf + (size_t)(n * nPF + q) * kPairBytes, acc[n]);
            }
        } else {            /* Q6_K: 210-byte super-blocks of 8 blocks */
            const int nsb = a.F >> 8;
            for (int sbi = 0; sbi < nsb; sbi++) {
                const uint32_t sb = (uint32_t)(rho * a.rb + sbi * 210);
                for (int h = 0; h < 2; h++)
                    for (int g = 0; g < 4; g++) {
                        const int blk = sbi * 8 + h * 4 + g;
#pragma unroll
                        for (int n = 0; n < NT; n++)
                            if (n < nt)
                                q6_k_block(tile, sb, h, g, p, xbuf + (size_t)(n * nPF + (blk >> 1)) * kPairBytes,
                                           blk & 1, acc[n]);
                    }
            }
        }
#pragma unroll
        for (int n = 0; n < NT; n++) {
            const float v = quad_finish(acc[n], TYPE == 2 ? 8.0f : 32.0f);
            if (p == 0 && n < nt) a.S.dn[(size_t)(g0 + n) * E + r0 + rho] = v;
        }
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) flag = atomicAdd(&a.S.tile_cnt[blockIdx.x], 1) == n_active - 1;
    __syncthreads();
    if (!flag) return;
    __threadfence();
    const int K = a.K;
    for (int i = tid; i < a.T * ROWS; i += NTH) {
        const int t = i / ROWS, r = r0 + (i - t * ROWS);
        float o = 0.0f;
        for (int j = 0; j < K; j++)
            o = __builtin_fmaf(a.S.wt[(size_t)t * K + j], a.S.dn[(size_t)a.S.slot_of[(size_t)t * K + j] * E + r], o);
        a.out[(size_t)t * E + r] = o;
    }
    if (tid == 0) a.S.tile_cnt[blockIdx.x] = 0;
}

template <int TYPE, int ROWS>
static hipError_t launch_down_t(const DownArgs &a, dim3 grid, int T, hipStream_t st)
{
    const int nPF = a.F / 64;
    const int tile_bytes = (int)(ROWS * a.rb);
    const int NT = T >= 4 ? 4 : (T >= 2 ? 2 : 1);
    const size_t lds = (size_t)((tile_bytes + 16 + 15) & ~15) + (size_t)NT * nPF * kPairBytes;
    if (NT == 4) hipLaunchKernelGGL((down_exact_kernel<TYPE, ROWS, 4>), grid, dim3(4 * ROWS), lds, st, a);
    else if (NT == 2) hipLaunchKernelGGL((down_exact_kernel<TYPE, ROWS, 2>), grid, dim3(4 * ROWS), lds, st, a);
    else hipLaunchKernelGGL((down_exact_kernel<TYPE, ROWS, 1>), grid, dim3(4 * ROWS), lds, st, a);
    return hipGetLastError();
}

hipError_t launch_down_exact(const Shape &s, const LayerDev &L, const Scratch &S, float *out, int T, hipStream_t st)
{
    DownArgs a;
    a.down = L.down;
    a.rb = L.down_rb;
    a.eb = L.down_eb;
    a.E = s.E;
    a.F = s.F;
    a.K = s.K;
    a.T = T;
    a.type = L.down_type;
    a.out = out;
    a.S = S;
    const int maxact = s.X < T * s.K ? s.X : T * s.K;
    if (L.down_type == 2) return launch_down_t<2, 64>(a, dim3(s.E / 64, maxact), T, st);
    return launch_down_t<14, 32>(a, dim3(s.E / 32, maxact), T, st);
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

/* One thread per Q4_0 block (or Q6_K super-block) of all X experts. */
__global__ void synth_experts_kernel(uint64_t seed, uint32_t layer, uint32_t kind, int type, int64_t rows,
                                     int64_t cols, int X, float sigma, uint8_t *base)
{
    const int64_t per_row = type == 14 ? cols / 256 : cols / 32;
    const uint64_t rb = type == 14 ? (uint64_t)per_row * 210 : (uint64_t)per_row * 18;
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
