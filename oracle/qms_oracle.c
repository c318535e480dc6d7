/* qms_oracle.c - CPU oracle (test infrastructure) for the qms expert-FFN layer.
 *
 * A plain-C restatement of the reference's integer fast path as its AVX2/VNNI build computes
 * it (gcc -O2 -march=native, -ffp-contract=fast by default in GNU C). The scalar code below
 * spells out the vector lanes so that every fp32 rounding happens in the same order. Build it
 * with -ffp-contract=off: every fused multiply-add of the reference is an explicit fmaf here.
 *
 * Used only by tests/, __graft_entry__.smoke() and the CPU-baseline leg of bench.py, as the
 * checker. Nothing in the product links or loads it. */
#include "qms_oracle.h"
#include "qmsg_synth.h"

#include <limits.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* Planted-mistake switch for the tests' sensitivity checks: 0 (the default) is the faithful
 * restatement; each other value changes one detail the golden vectors must catch. */
int orc_mutation = 0;

/* ---------------------------------------------------------------- formats ---- */

/* src/qms.h:11-33 (exact for every finite half; F16C's vcvtph2ps gives the same values). */
float orc_f16_to_f32(uint16_t h) { return qmsg_f16_to_f32(h); }

static inline float f16_at(const uint8_t *p) { return qmsg_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* src/gguf.c:85-96 */
uint64_t orc_row_bytes(int type, int64_t ne0)
{
    switch (type) {
    case ORC_T_F32: return (uint64_t)ne0 * 4;
    case ORC_T_F16: return (uint64_t)ne0 * 2;
    case ORC_T_Q4_0: return ne0 % 32 ? 0 : (uint64_t)ne0 / 32 * 18;
    case ORC_T_Q4_1: return ne0 % 32 ? 0 : (uint64_t)ne0 / 32 * 20;
    case ORC_T_Q8_0: return ne0 % 32 ? 0 : (uint64_t)ne0 / 32 * 34;
    case ORC_T_Q6_K: return ne0 % 256 ? 0 : (uint64_t)ne0 / 256 * 210;
    default: return 0;
    }
}

/* src/quant.c:17-93: dequantised weights, used by the tests' dequant-then-dot invariant. */
int orc_dequant_row(int type, const void *src, float *y, int64_t n)
{
    const uint8_t *b = (const uint8_t *)src;
    switch (type) {
    case ORC_T_F32: memcpy(y, b, (size_t)n * 4); return 0;
    case ORC_T_F16:
        for (int64_t i = 0; i < n; i++) y[i] = f16_at(b + 2 * i);
        return 0;
    case ORC_T_Q4_0:
        if (n % 32) return -1;
        for (int64_t i = 0; i < n; i += 32, b += 18) {
            const float d = f16_at(b);
            for (int j = 0; j < 16; j++) {
                y[i + j] = (float)((b[2 + j] & 15) - 8) * d;
                y[i + j + 16] = (float)((b[2 + j] >> 4) - 8) * d;
            }
        }
        return 0;
    case ORC_T_Q4_1:
        if (n % 32) return -1;
        for (int64_t i = 0; i < n; i += 32, b += 20) {
            const float d = f16_at(b), m = f16_at(b + 2);
            for (int j = 0; j < 16; j++) {
                y[i + j] = fmaf((float)(b[4 + j] & 15), d, m);      /* q*d + m, contracted */
                y[i + j + 16] = fmaf((float)(b[4 + j] >> 4), d, m);
            }
        }
        return 0;
    case ORC_T_Q8_0:
        if (n % 32) return -1;
        for (int64_t i = 0; i < n; i += 32, b += 34) {
            const float d = f16_at(b);
            for (int j = 0; j < 32; j++) y[i + j] = (float)(int8_t)b[2 + j] * d;
        }
        return 0;
    case ORC_T_Q6_K:
        if (n % 256) return -1;
        for (int64_t i = 0; i < n; i += 256, b += 210) {
            const float d = f16_at(b + 208);
            const int8_t *sc = (const int8_t *)(b + 192);
            for (int e = 0; e < 256; e++) {
                const int h = e / 128, m = e % 128, g = m / 32, l = m % 32;
                const int lo = b[64 * h + 32 * (g & 1) + l];
                const int q = ((g < 2 ? lo & 15 : lo >> 4) | (((b[128 + 32 * h + l] >> (2 * g)) & 3) << 4)) - 32;
                y[i + e] = d * (float)sc[8 * h + m / 16] * (float)q;
            }
        }
        return 0;
    default: return -1;
    }
}

/* ---------------------------------------------------------------- int8 activations ---- */

/* src/kernels.c:34-53 */
void orc_quantize_q8(const float *x, int64_t n, orc_q8 *out)
{
    for (int64_t b = 0; b < n / 32; b++) {
        const float *xb = x + b * 32;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(xb[j]));
        const float d = amax / 127.0f;
        const float id = d > 0.0f ? 1.0f / d : 0.0f;
        int s0 = 0, s1 = 0;
        for (int j = 0; j < 32; j++) {
            /* (int) of a value outside int's range, or of a NaN, is undefined in C; the x86
             * conversion the reference compiles to gives INT_MIN (the "integer indefinite").
             * That happens when id is +inf (d below 2^-128) or xb[j] is NaN or infinite. */
            const float r = orc_mutation == ORC_MUT_ROUND_AWAY ? roundf(xb[j] * id) : nearbyintf(xb[j] * id);
            const int q = fabsf(r) < 2147483648.0f ? (int)r : INT_MIN;
            out[b].q[j] = (int8_t)q;
            /* wrapping sums (several INT_MIN codes overflow int; the reference's adds wrap) */
            if (j < 16) s0 = (int)((unsigned)s0 + (unsigned)q);
            else s1 = (int)((unsigned)s1 + (unsigned)q);
        }
        out[b].d = d;
        out[b].s16[0] = (int16_t)s0;
        out[b].s16[1] = (int16_t)s1;
        out[b].ds = d * (float)(int)((unsigned)s0 + (unsigned)s1);
    }
}

/* ---------------------------------------------------------------- row dots ---- */

/* hsum256 (src/kernels.c:66-72): lanes j and j+4 first, then (s0+s2)+(s1+s3). */
static inline float hsum8(const float a[8])
{
    if (orc_mutation == ORC_MUT_HSUM_LINEAR) {
        float s = 0.0f;
        for (int k = 0; k < 8; k++) s += a[k];
        return s;
    }
    const float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
    return (s0 + s2) + (s1 + s3);
}

/* Unsigned code of element j (0..31) of a Q4_0/Q4_1 block: low nibbles are elements 0..15. */
static inline int nib(const uint8_t *qs, int j)
{
    if (orc_mutation == ORC_MUT_NIBBLE_ORDER) return (j & 1) ? qs[j >> 1] >> 4 : qs[j >> 1] & 15;
    return j < 16 ? qs[j] & 15 : qs[j - 16] >> 4;
}

/* dot_u8s8 lane k of one 32-block (src/kernels.c:56-64): elements 4k..4k+3. */
static inline int lane_q4(const uint8_t *qs, const int8_t *q, int k)
{
    int s = 0;
    for (int i = 0; i < 4; i++) s += nib(qs, 4 * k + i) * q[4 * k + i];
    return s;
}

/* src/kernels.c:82-94 (AVX2 branch). */
static float dot_q4_0(const uint8_t *w, const orc_q8 *x, int64_t nb)
{
    float acc[8] = { 0 }, corr = 0.0f;
    for (int64_t b = 0; b < nb; b++, w += 18) {
        const float d = f16_at(w);
        const float dd = d * x[b].d;
        for (int k = 0; k < 8; k++) acc[k] = fmaf((float)lane_q4(w + 2, x[b].q, k), dd, acc[k]);
        corr = orc_mutation == ORC_MUT_CORR_UNFUSED ? corr + d * x[b].ds : fmaf(d, x[b].ds, corr);
    }
    /* 8*corr is exact, so fusing this subtraction (as -ffp-contract=fast may) changes nothing */
    return hsum8(acc) - 8.0f * corr;
}

/* src/kernels.c:109-121 (AVX2 branch). */
static float dot_q4_1(const uint8_t *w, const orc_q8 *x, int64_t nb)
{
    float acc[8] = { 0 }, off = 0.0f;
    for (int64_t b = 0; b < nb; b++, w += 20) {
        const float d = f16_at(w), m = f16_at(w + 2);
        const float dd = d * x[b].d;
        for (int k = 0; k < 8; k++) acc[k] = fmaf((float)lane_q4(w + 4, x[b].q, k), dd, acc[k]);
        off = fmaf(m, x[b].ds, off);
    }
    return hsum8(acc) + off;
}

/* Unsigned 6-bit code of element l (0..31) of 32-block g (0..3) in one 128-half
 * (src/kernels.c:136-138, 155-160). */
static inline int q6code(const uint8_t *ql, const uint8_t *qh, int g, int l)
{
    const int lo = ql[(g & 1) * 32 + l];
    return (g < 2 ? lo & 15 : lo >> 4) | (((qh[l] >> (2 * g)) & 3) << 4);
}

/* src/kernels.c:139-170 (AVX2 branch): lanes 0-3 scaled by sc[2g], lanes 4-7 by sc[2g+1]. */
static float dot_q6_k(const uint8_t *w, const orc_q8 *x, int64_t nsb)
{
    float acc[8] = { 0 }, corr = 0.0f;
    for (int64_t sb = 0; sb < nsb; sb++, w += 210) {
        const float d = f16_at(w + 208);
        const int8_t *scs = (const int8_t *)(w + 192);
        for (int half = 0; half < 2; half++) {
            const uint8_t *ql = w + half * 64, *qh = w + 128 + half * 32;
            const int8_t *sc = scs + half * 8;
            for (int g = 0; g < 4; g++) {
                const orc_q8 *xb = &x[sb * 8 + half * 4 + g];
                const int sa = sc[2 * g], sbb = sc[2 * g + 1];
                const float dd = d * xb->d;
                for (int k = 0; k < 8; k++) {
                    int s = 0;
                    for (int i = 0; i < 4; i++) s += q6code(ql, qh, g, 4 * k + i) * xb->q[4 * k + i];
                    s *= k < 4 ? sa : sbb;
                    acc[k] = fmaf((float)s, dd, acc[k]);
                }
                corr = fmaf(dd, (float)(sa * xb->s16[0] + sbb * xb->s16[1]), corr);
            }
        }
    }
    return hsum8(acc) - 32.0f * corr;
}

/* src/kernels.c:202-213 (AVX2 branch): 16 FMA chains (two 8-lane registers), a0+a1, hsum256. */
float orc_vec_dot_f32(const float *w, const float *x, int64_t n)
{
    float a0[8] = { 0 }, a1[8] = { 0 };
    int64_t i = 0;
    for (; i + 16 <= n; i += 16)
        for (int k = 0; k < 8; k++) {
            a0[k] = fmaf(w[i + k], x[i + k], a0[k]);
            a1[k] = fmaf(w[i + 8 + k], x[i + 8 + k], a1[k]);
        }
    float v[8];
    for (int k = 0; k < 8; k++) v[k] = a0[k] + a1[k];
    float s = hsum8(v);
    if (orc_mutation == ORC_MUT_ROUTER_TREE) {
        s = 0.0f;
        for (int k = 0; k < 8; k++) s += v[k];
    }
    for (; i < n; i++) s = fmaf(w[i], x[i], s);   /* tail: never taken when n % 16 == 0 */
    return s;
}

/* src/kernels.c:223-231 */
float orc_vec_dot_q8(int type, const uint8_t *w, const orc_q8 *x, int64_t n)
{
    switch (type) {
    case ORC_T_Q4_0: return dot_q4_0(w, x, n / 32);
    case ORC_T_Q4_1: return dot_q4_1(w, x, n / 32);
    case ORC_T_Q6_K: return dot_q6_k(w, x, n / 256);
    default: return NAN;
    }
}

/* src/kernels.c:197-200 */
int orc_fast_supported(int type)
{
    return type == ORC_T_Q4_0 || type == ORC_T_Q4_1 || type == ORC_T_Q6_K || type == ORC_T_F32;
}

/* The exact signed int32 dot of 32-block `blk` of a weight row with x[blk]: what the
 * reference's integer lanes sum to before any float scaling. Q4_0: sum (q-8)*x. Q6_K:
 * sc[lo]*sum_{l<16} (q6-32)*x + sc[hi]*sum_{l>=16} (q6-32)*x. Q4_1: sum q*x (offset is fp). */
int32_t orc_block_dot(int type, const uint8_t *w, const orc_q8 *x, int64_t blk)
{
    const int8_t *q = x[blk].q;
    int32_t s = 0;
    if (type == ORC_T_Q4_0 || type == ORC_T_Q4_1) {
        const uint8_t *qs = w + blk * (type == ORC_T_Q4_0 ? 18 : 20) + (type == ORC_T_Q4_0 ? 2 : 4);
        for (int j = 0; j < 32; j++) s += (nib(qs, j) - (type == ORC_T_Q4_0 ? 8 : 0)) * q[j];
        return s;
    }
    if (type == ORC_T_Q6_K) {
        const uint8_t *sb = w + (blk / 8) * 210;
        const int half = (int)(blk % 8) / 4, g = (int)(blk % 4);
        const uint8_t *ql = sb + half * 64, *qh = sb + 128 + half * 32;
        const int8_t *sc = (const int8_t *)(sb + 192) + half * 8;
        int32_t lo = 0, hi = 0;
        for (int l = 0; l < 32; l++) {
            const int v = (q6code(ql, qh, g, l) - 32) * q[l];
            if (l < 16) lo += v; else hi += v;
        }
        return sc[2 * g] * lo + sc[2 * g + 1] * hi;
    }
    return 0;
}

/* orc_block_dot over n (expert, row, block) triples of one stacked expert tensor, each against
 * the Q8 row starting at block xrow[i] of x (test driver of the row above, no reference code). */
void orc_block_dots_at(int type, const uint8_t *w, uint64_t row_bytes, uint64_t expert_bytes, int64_t n,
                       const int32_t *ex, const int32_t *row, const int32_t *blk, const orc_q8 *x,
                       const int64_t *xrow, int32_t *out)
{
    for (int64_t i = 0; i < n; i++)
        out[i] = orc_block_dot(type, w + (uint64_t)ex[i] * expert_bytes + (uint64_t)row[i] * row_bytes,
                               x + xrow[i], blk[i]);
}

/* src/model.c:424 (glibc expf). */
float orc_silu(float a) { return a / (1.0f + expf(-a)); }

/* ---------------------------------------------------------------- the layer ---- */

static inline const uint8_t *expert_row(const orc_mat *m, int e, int64_t r)
{
    return m->data + (uint64_t)e * m->expert_bytes + (uint64_t)r * m->row_bytes;
}

/* Router of one layer: logits = W xn (qms_matmul on the F32 router, src/model.c:1043 ->
 * src/quant.c:128-170 -> dot_f32), then per token a double softmax, top-K by repeated argmax
 * with ties to the lower index, and weights renormalised over the selection
 * (src/model.c:1045-1064). */
/* src/model.c:1045-1064 on given logits: softmax in double, top K (ties to the lower index),
 * weights renormalised in selection order. */
static void topk_all(int X, int K, const float *logits, int T, int *selv, float *wtv)
{
    double *prob = (double *)malloc((size_t)X * sizeof(double));
    for (int t = 0; t < T; t++) {
        const float *lt = logits + (size_t)t * X;
        double mx = -INFINITY, z = 0.0;
        for (int e = 0; e < X; e++) if (lt[e] > mx) mx = lt[e];
        for (int e = 0; e < X; e++) { prob[e] = exp((double)lt[e] - mx); z += prob[e]; }
        for (int e = 0; e < X; e++) prob[e] /= z;
        int *sel = selv + (size_t)t * K;
        double wsum = 0.0;
        for (int j = 0; j < K; j++) {
            int best = -1;
            for (int e = 0; e < X; e++) {
                int taken = 0;
                for (int i = 0; i < j; i++) if (sel[i] == e) { taken = 1; break; }
                if (!taken && (best < 0 || prob[e] > prob[best] ||
                               (orc_mutation == ORC_MUT_TIE_HIGH && prob[e] == prob[best])))
                    best = e;
            }
            sel[j] = best;
            wsum += prob[best];
        }
        for (int j = 0; j < K; j++) wtv[(size_t)t * K + j] = (float)(prob[sel[j]] / wsum);
    }
    free(prob);
}

void orc_route(int E, int X, int K, const float *router, const float *xn, int T, float *logits, int *selv,
               float *wtv)
{
#pragma omp parallel for schedule(static) if ((int64_t)X * E * T >= (1 << 21))
    for (int r = 0; r < X; r++)
        for (int t = 0; t < T; t++)
            logits[(size_t)t * X + r] = orc_vec_dot_f32(router + (size_t)r * E, xn + (size_t)t * E, E);
    topk_all(X, K, logits, T, selv, wtv);
}

static float dot_exact(const float *row, const float *x, int64_t n);

/* Routing of the reference's --exact mode: logits by matmul_exact on the F32 router. */
void orc_route_exact(int E, int X, int K, const float *router, const float *xn, int T, float *logits, int *selv,
                     float *wtv)
{
#pragma omp parallel for schedule(static) if ((int64_t)X * E * T >= (1 << 21))
    for (int r = 0; r < X; r++)
        for (int t = 0; t < T; t++)
            logits[(size_t)t * X + r] = dot_exact(router + (size_t)r * E, xn + (size_t)t * E, E);
    topk_all(X, K, logits, T, selv, wtv);
}

/* matmul_exact's dot (src/quant.c:97-115): a dequantised row against fp32 x, one FMA chain
 * in element order (the reference build contracts acc += row*x). */
static float dot_exact(const float *row, const float *x, int64_t n)
{
    float acc = 0.0f;
    for (int64_t c = 0; c < n; c++) acc = fmaf(row[c], x[c], acc);
    return acc;
}

/* One product of moe_group_exact's per-slot qms_matmul with qms_exact_math = 0 (src/quant.c:
 * 128-170, model.c:1024-1027): int8 blocks (xq, the row x quantised) for the quantised types of
 * the fast path, dot_f32 on x for F32 rows of whole 32-blocks, and otherwise (F16, Q8_0) the
 * fp32 chain of matmul_exact on the dequantised row (tmp: n floats). */
static float slot_dot(int type, const uint8_t *w, const orc_q8 *xq, const float *x, int64_t n, float *tmp)
{
    if (type == ORC_T_Q4_0 || type == ORC_T_Q4_1 || type == ORC_T_Q6_K) return orc_vec_dot_q8(type, w, xq, n);
    if (type == ORC_T_F32 && n % 32 == 0) return orc_vec_dot_f32((const float *)w, x, n);
    orc_dequant_row(type, w, tmp, n);
    return dot_exact(tmp, x, n);
}

/* qms_matmul with qms_exact_math set (src/quant.c:97-115, 128-139): every row dequantised to
 * fp32 (qms_dequant_row), y[t][r] = dot_exact(row r, x_t). */
int orc_matmul_exact(int type, const uint8_t *w, int64_t rows, int64_t cols, uint64_t row_bytes, const float *x,
                     int T, float *y)
{
    if (!orc_row_bytes(type, cols)) return -1;
    int bad = 0;
#pragma omp parallel
    {
        float *row = (float *)malloc((size_t)cols * sizeof(float));
#pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; r++) {
            if (orc_dequant_row(type, w + (uint64_t)r * row_bytes, row, cols) != 0) { bad = 1; continue; }
            for (int t = 0; t < T; t++) y[(size_t)t * rows + r] = dot_exact(row, x + (size_t)t * cols, cols);
        }
        free(row);
    }
    return bad ? -1 : 0;
}

/* src/model.c:1032-1167 for resident experts (one group): with exact = 0 the integer path,
 * moe_group_fast (969-1007); with exact = 1 the reference's --exact mode (qms_exact_math),
 * where the router and moe_group_exact (1010-1030) use matmul_exact and the activations stay
 * fp32. Past moe()'s fast gate (n_embd % 256 != 0 or n_ff_exp % 32 != 0; 1090-1093) without
 * --exact, the reference runs moe_group_exact, whose per-slot qms_matmul calls take the int8
 * path of src/quant.c:134-169 for quantised rows of whole blocks: the input row quantised, the
 * gate and up dots, silu(g)*u, the activation row quantised, the down dots. Those are the
 * integer branch's steps, so it serves that case too (rows of whole 32-blocks, any n_embd). */
static int moe_common(int exact, int E, int X, int K, int F, const orc_mat *router, const orc_mat *gate,
                      const orc_mat *up, const orc_mat *down, const float *xn, int T, float *out, orc_moe_dbg *dbg)
{
    if (T < 0 || K <= 0 || K > X) return -1;
    if (router->type != ORC_T_F32 || router->cols != E || router->rows != X) return -1;
    if (exact) {
        if (!orc_row_bytes(gate->type, E) || !orc_row_bytes(up->type, E) || !orc_row_bytes(down->type, F)) return -1;
    } else {
        /* model.c:1090-1093: moe_group_fast, or moe_group_exact whose per-slot qms_matmul picks
         * each matrix's dot by its type (slot_dot). Rows of whole 32-blocks here. Not modelled:
         * the fast gate with F32 up rows, which it sends to qms_vec_dot_q8 (no F32 case there:
         * NaN, src/kernels.c:223-231). */
        const int fast = orc_fast_supported(gate->type) && orc_fast_supported(up->type) &&
                         orc_fast_supported(down->type) && gate->type != ORC_T_F32 &&
                         down->type != ORC_T_F32 && E % 256 == 0 && F % 32 == 0;
        if (E % 32 || F % 32 || !orc_row_bytes(gate->type, E) || !orc_row_bytes(up->type, E) ||
            !orc_row_bytes(down->type, F) || (fast && up->type == ORC_T_F32))
            return -1;
    }
    if (T == 0) return 0;
    const int NS = T * K, nbE = E / 32, nbF = F / 32;
    float *logits = (float *)malloc((size_t)T * X * sizeof(float));
    int *selv = (int *)malloc((size_t)NS * sizeof(int));
    float *wtv = (float *)malloc((size_t)NS * sizeof(float));
    if (exact) {
        orc_route_exact(E, X, K, (const float *)router->data, xn, T, logits, selv, wtv);
    } else {
        orc_route(E, X, K, (const float *)router->data, xn, T, logits, selv, wtv);
    }

    /* counting sort of slots by expert: model.c:1066-1088 */
    int *start = (int *)calloc((size_t)X + 1, sizeof(int));
    int *slot_t = (int *)malloc((size_t)NS * sizeof(int));
    int *slot_of = (int *)malloc((size_t)NS * sizeof(int));
    int *active = (int *)malloc((size_t)X * sizeof(int));
    int *cnt = (int *)calloc((size_t)X, sizeof(int));
    int na = 0;
    for (int i = 0; i < NS; i++) cnt[selv[i]]++;
    for (int e = 0; e < X; e++) {
        start[e + 1] = start[e] + cnt[e];
        if (cnt[e]) active[na++] = e;
    }
    memset(cnt, 0, (size_t)X * sizeof(int));
    for (int t = 0; t < T; t++)
        for (int j = 0; j < K; j++) {
            const int e = selv[t * K + j], s = start[e] + cnt[e]++;
            slot_t[s] = t;
            slot_of[t * K + j] = s;
        }
    free(cnt);

    /* model.c:1096-1097 */
    orc_q8 *xq = (orc_q8 *)calloc((size_t)T * nbE, sizeof(orc_q8));
    if (!exact)
        for (int t = 0; t < T; t++) orc_quantize_q8(xn + (size_t)t * E, E, xq + (size_t)t * nbE);
    float *gu = (float *)malloc((size_t)NS * 2 * F * sizeof(float));
    float *act = (float *)malloc((size_t)NS * F * sizeof(float));
    orc_q8 *aq = (orc_q8 *)calloc((size_t)NS * nbF, sizeof(orc_q8));
    float *dn = (float *)malloc((size_t)NS * E * sizeof(float));

    if (exact) {
        /* moe_group_exact, model.c:1010-1030: per slot g, u by matmul_exact, a = silu(g)*u,
         * dn = matmul_exact(down, a) */
#pragma omp parallel
        {
            float *row = (float *)malloc((size_t)(E > F ? E : F) * sizeof(float));
#pragma omp for schedule(static)
            for (int64_t it = 0; it < (int64_t)na * 2 * F; it++) {
                const int e = active[it / (2 * F)];
                const int r = (int)(it % (2 * F));
                const orc_mat *W = r < F ? gate : up;
                orc_dequant_row(W->type, expert_row(W, e, r < F ? r : r - F), row, E);
                for (int s = start[e]; s < start[e + 1]; s++)
                    gu[(size_t)s * 2 * F + r] = dot_exact(row, xn + (size_t)slot_t[s] * E, E);
            }
#pragma omp for schedule(static)
            for (int s = 0; s < NS; s++) {
                const float *g = gu + (size_t)s * 2 * F;
                float *a = act + (size_t)s * F;
                for (int j = 0; j < F; j++) a[j] = orc_silu(g[j]) * g[F + j];
            }
#pragma omp for schedule(static)
            for (int64_t it = 0; it < (int64_t)na * E; it++) {
                const int e = active[it / E];
                const int r = (int)(it % E);
                orc_dequant_row(down->type, expert_row(down, e, r), row, F);
                for (int s = start[e]; s < start[e + 1]; s++)
                    dn[(size_t)s * E + r] = dot_exact(row, act + (size_t)s * F, F);
            }
            free(row);
        }
    } else {
    /* moe_group_fast, model.c:979-1005; with every matrix quantised moe_group_exact's steps are
     * the same, and slot_dot picks the dot of its other types */
#pragma omp parallel
    {
        float *tmp = (float *)malloc((size_t)(E > F ? E : F) * sizeof(float));
#pragma omp for schedule(static)
        for (int64_t it = 0; it < (int64_t)na * 2 * F; it++) {
            const int e = active[it / (2 * F)];
            const int r = (int)(it % (2 * F));
            const orc_mat *W = r < F ? gate : up;
            const uint8_t *row = expert_row(W, e, r < F ? r : r - F);
            for (int s = start[e]; s < start[e + 1]; s++)
                gu[(size_t)s * 2 * F + r] = slot_dot(W->type, row, xq + (size_t)slot_t[s] * nbE,
                                                     xn + (size_t)slot_t[s] * E, E, tmp);
        }
#pragma omp for schedule(static)
        for (int s = 0; s < NS; s++) {
            const float *g = gu + (size_t)s * 2 * F;
            float *a = act + (size_t)s * F;
            for (int j = 0; j < F; j++) a[j] = orc_silu(g[j]) * g[F + j];
            orc_quantize_q8(a, F, aq + (size_t)s * nbF);
        }
#pragma omp for schedule(static)
        for (int64_t it = 0; it < (int64_t)na * E; it++) {
            const int e = active[it / E];
            const int r = (int)(it % E);
            const uint8_t *row = expert_row(down, e, r);
            for (int s = start[e]; s < start[e + 1]; s++)
                dn[(size_t)s * E + r] = slot_dot(down->type, row, aq + (size_t)s * nbF, act + (size_t)s * F, F, tmp);
        }
        free(tmp);
    }
    }

    /* weighted sum per token in selection order: model.c:1152-1162 */
    memset(out, 0, (size_t)T * E * sizeof(float));
    for (int t = 0; t < T; t++) {
        float *ot = out + (size_t)t * E;
        for (int jj = 0; jj < K; jj++) {
            const int j = orc_mutation == ORC_MUT_COMBINE_ORDER ? K - 1 - jj : jj;
            const float wj = wtv[t * K + j];
            const float *d = dn + (size_t)slot_of[t * K + j] * E;
            for (int i = 0; i < E; i++) ot[i] = fmaf(wj, d[i], ot[i]);
        }
    }

    if (dbg) {
        if (dbg->logits) memcpy(dbg->logits, logits, (size_t)T * X * sizeof(float));
        if (dbg->sel) memcpy(dbg->sel, selv, (size_t)NS * sizeof(int));
        if (dbg->wt) memcpy(dbg->wt, wtv, (size_t)NS * sizeof(float));
        if (dbg->start) memcpy(dbg->start, start, (size_t)(X + 1) * sizeof(int));
        if (dbg->slot_t) memcpy(dbg->slot_t, slot_t, (size_t)NS * sizeof(int));
        if (dbg->slot_of) memcpy(dbg->slot_of, slot_of, (size_t)NS * sizeof(int));
        if (dbg->active) memcpy(dbg->active, active, (size_t)na * sizeof(int));
        if (dbg->n_active) *dbg->n_active = na;
        if (dbg->xq) memcpy(dbg->xq, xq, (size_t)T * nbE * sizeof(orc_q8));
        if (dbg->gu) memcpy(dbg->gu, gu, (size_t)NS * 2 * F * sizeof(float));
        if (dbg->act) memcpy(dbg->act, act, (size_t)NS * F * sizeof(float));
        if (dbg->aq) memcpy(dbg->aq, aq, (size_t)NS * nbF * sizeof(orc_q8));
        if (dbg->dn) memcpy(dbg->dn, dn, (size_t)NS * E * sizeof(float));
    }
    free(start); free(slot_t); free(slot_of); free(active);
    free(xq); free(gu); free(act); free(aq); free(dn);
    free(logits); free(selv); free(wtv);
    return 0;
}

int orc_moe(int E, int X, int K, int F, const orc_mat *router, const orc_mat *gate, const orc_mat *up,
            const orc_mat *down, const float *xn, int T, float *out, orc_moe_dbg *dbg)
{
    return moe_common(0, E, X, K, F, router, gate, up, down, xn, T, out, dbg);
}

int orc_moe_exact(int E, int X, int K, int F, const orc_mat *router, const orc_mat *gate, const orc_mat *up,
                  const orc_mat *down, const float *xn, int T, float *out, orc_moe_dbg *dbg)
{
    return moe_common(1, E, X, K, F, router, gate, up, down, xn, T, out, dbg);
}

/* The fast path of qms_matmul_n for one matrix (src/quant.c:128-170): for a quantised type
 * each row of x [T][cols] is quantised to int8 blocks and y[t][r] = vec_dot_q8(row r, xq_t);
 * F32 rows take qms_vec_dot_f32 against x itself (src/quant.c:161-163). */
int orc_matmul_q8(int type, const uint8_t *w, int64_t rows, int64_t cols, uint64_t row_bytes, const float *x, int T,
                  float *y)
{
    if (cols % 32 || !orc_row_bytes(type, cols) || type == ORC_T_F16 || type == ORC_T_Q8_0) return -1;
    if (type == ORC_T_F32) {
#pragma omp parallel for schedule(static)
        for (int64_t r = 0; r < rows; r++)
            for (int t = 0; t < T; t++)
                y[(size_t)t * rows + r] =
                    orc_vec_dot_f32((const float *)(w + (uint64_t)r * row_bytes), x + (size_t)t * cols, cols);
        return 0;
    }
    const int64_t nb = cols / 32;
    orc_q8 *xq = (orc_q8 *)malloc((size_t)T * (size_t)nb * sizeof(orc_q8));
    if (!xq) return -1;
    for (int t = 0; t < T; t++) orc_quantize_q8(x + (size_t)t * cols, cols, xq + (size_t)t * nb);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++)
        for (int t = 0; t < T; t++)
            y[(size_t)t * rows + r] = orc_vec_dot_q8(type, w + (uint64_t)r * row_bytes, xq + (size_t)t * nb, cols);
    free(xq);
    return 0;
}

/* ---------------------------------------------------------------- synthetic inputs ---- */

void orc_synth_f32(uint64_t seed, uint32_t layer, uint32_t kind, uint32_t expert, uint64_t n, float sigma,
                   float *out)
{
    const uint64_t key = qmsg_tensor_key(seed, layer, kind, expert);
#pragma omp parallel for schedule(static) if (n >= 65536)
    for (int64_t i = 0; i < (int64_t)n; i++) out[i] = qmsg_normal(key, (uint64_t)i) * sigma;
}

/* Experts e0..e1-1 of a stacked [X][rows][cols] tensor, written at base + e*expert_bytes. */
void orc_synth_experts(uint64_t seed, uint32_t layer, uint32_t kind, int type, int64_t rows, int64_t cols,
                       int e0, int e1, float sigma, uint8_t *base)
{
    const uint64_t rb = orc_row_bytes(type, cols), eb = rb * (uint64_t)rows;
    const int64_t per_row = type == ORC_T_Q6_K ? cols / 256 : cols / 32;
    for (int e = e0; e < e1; e++) {
        const uint64_t key = qmsg_tensor_key(seed, layer, kind, (uint32_t)e);
        uint8_t *m = base + (uint64_t)e * eb;
#pragma omp parallel for schedule(static)
        for (int64_t r = 0; r < rows; r++)
            for (int64_t b = 0; b < per_row; b++) {
                if (type == ORC_T_Q6_K)
                    qmsg_synth_q6_k_block(key, (uint64_t)r * cols + (uint64_t)b * 256, sigma,
                                          m + (uint64_t)r * rb + (uint64_t)b * 210);
                else if (type == ORC_T_Q4_1)
                    qmsg_synth_q4_1_block(key, (uint64_t)cols, (uint64_t)r, (uint64_t)b, sigma,
                                          m + (uint64_t)r * rb + (uint64_t)b * 20);
                else
                    qmsg_synth_q4_0_block(key, (uint64_t)cols, (uint64_t)r, (uint64_t)b, sigma,
                                          m + (uint64_t)r * rb + (uint64_t)b * 18);
            }
    }
}

/* src/model.c:403-409: sum of squares as a double FMA chain (contracted by the reference
 * build), 1/sqrt in double, then (float)(x*inv) * w in float; w = NULL is a unit weight. */
void orc_rmsnorm(float *y, const float *x, const float *w, int n, float eps)
{
    double ss = 0.0;
    for (int i = 0; i < n; i++) ss = fma((double)x[i], (double)x[i], ss);
    const double inv = 1.0 / sqrt(ss / n + (double)eps);
    for (int i = 0; i < n; i++) y[i] = (float)((double)x[i] * inv) * (w ? w[i] : 1.0f);
}

void orc_rmsnorm_unit(float *y, const float *x, int n, float eps) { orc_rmsnorm(y, x, NULL, n, eps); }
