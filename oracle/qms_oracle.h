/* qms_oracle.h - CPU oracle for the qms Qwen3-MoE expert-FFN layer.
 *
 * TEST INFRASTRUCTURE. This is a plain-C restatement of the reference's AVX path
 * (src/kernels.c, src/quant.c, src/model.c of ZeningXiong/large_model), used only by the tests,
 * by the smoke check and by the CPU-baseline leg of the benchmark, and only as the checker.
 * The product (libqmsg) never links, loads or calls it.
 *
 * Every float operation follows the reference's x86 AVX2/VNNI build (gcc -O2, GNU C's default
 * -ffp-contract=fast): eight 4-element int32 lanes per 32-block, a per-lane fp32 FMA chain
 * over blocks, an fp32 FMA chain for the offset term, the hsum256 tree, and the final
 * unfused subtraction. See each function for the reference lines it follows. */
#ifndef QMS_ORACLE_H
#define QMS_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_T_F32 = 0, ORC_T_F16 = 1, ORC_T_Q4_0 = 2, ORC_T_Q4_1 = 3, ORC_T_Q8_0 = 8, ORC_T_Q6_K = 14 };

/* int8 activation block, byte-compatible with QmsQ8 (src/kernels.h:7-12), 44 bytes. */
typedef struct {
    float d;
    float ds;
    int16_t s16[2];
    int8_t q[32];
} orc_q8;

/* Stacked expert matrix in GGUF layout (QmsMat src/quant.h:11-16 + expert_bytes of
 * QmsExperts src/model.h:31-35): expert e's row r starts at data + e*expert_bytes + r*row_bytes. */
typedef struct {
    int type;
    int64_t rows, cols;
    uint64_t row_bytes;
    uint64_t expert_bytes;
    const uint8_t *data;
} orc_mat;

/* Intermediates of one layer call; every pointer may be NULL. Sizes: NS = T*K slots. */
typedef struct {
    float *logits;    /* [T][X]            router logits                         */
    int *sel;         /* [T][K]            selected experts in selection order   */
    float *wt;        /* [T][K]            renormalised routing weights          */
    int *start;       /* [X+1]             slots of expert e: start[e]..start[e+1]-1 */
    int *slot_t;      /* [NS]              token of each slot                    */
    int *slot_of;     /* [T][K]            slot of (token, selection)            */
    int *active;      /* [X]               active experts, ascending; count in n_active */
    int *n_active;
    orc_q8 *xq;       /* [T][E/32]         quantised layer input                 */
    float *gu;        /* [NS][2F]          gate rows 0..F-1, up rows F..2F-1     */
    float *act;       /* [NS][F]           silu(g)*u                             */
    orc_q8 *aq;       /* [NS][F/32]        quantised activation                  */
    float *dn;        /* [NS][E]           per-slot expert output                */
} orc_moe_dbg;

/* Planted mistakes (orc_mutation): each one is a plausible slip the golden vectors must catch. */
enum {
    ORC_MUT_NONE = 0,
    ORC_MUT_HSUM_LINEAR = 1,    /* the eight dot lanes summed left to right         */
    ORC_MUT_CORR_UNFUSED = 2,   /* offset chain as mul + add                        */
    ORC_MUT_NIBBLE_ORDER = 3,   /* interleaved instead of low-then-high nibbles     */
    ORC_MUT_ROUTER_TREE = 4,    /* router dot reduced left to right                 */
    ORC_MUT_ROUND_AWAY = 5,     /* quantiser rounds halves away from zero           */
    ORC_MUT_TIE_HIGH = 6,       /* top-k ties go to the higher expert index         */
    ORC_MUT_COMBINE_ORDER = 7   /* weighted sum in reverse selection order          */
};
extern int orc_mutation;

float orc_f16_to_f32(uint16_t h);
uint64_t orc_row_bytes(int type, int64_t ne0);
int orc_dequant_row(int type, const void *src, float *dst, int64_t n);
void orc_quantize_q8(const float *x, int64_t n, orc_q8 *out);
float orc_vec_dot_q8(int type, const uint8_t *w, const orc_q8 *x, int64_t n);
int orc_matmul_q8(int type, const uint8_t *w, int64_t rows, int64_t cols, uint64_t row_bytes, const float *x, int T,
                  float *y);
float orc_vec_dot_f32(const float *w, const float *x, int64_t n);
int32_t orc_block_dot(int type, const uint8_t *w_row, const orc_q8 *x, int64_t blk);
void orc_block_dots_at(int type, const uint8_t *w, uint64_t row_bytes, uint64_t expert_bytes, int64_t n,
                       const int32_t *ex, const int32_t *row, const int32_t *blk, const orc_q8 *x,
                       const int64_t *xrow, int32_t *out);
float orc_silu(float a);
int orc_fast_supported(int type);

void orc_route(int E, int X, int K, const float *router, const float *xn, int T, float *logits, int *sel,
               float *wt);

/* The MoE layer, out[T][E] = sum_j wt[t][j] * expert_sel(xn[t]). Returns 0, or -1 when the
 * shapes or types are outside the reference's integer fast path. */
int orc_moe(int E, int X, int K, int F, const orc_mat *router, const orc_mat *gate, const orc_mat *up,
            const orc_mat *down, const float *xn, int T, float *out, orc_moe_dbg *dbg);
/* The reference's --exact mode (qms_exact_math): matmul_exact everywhere, fp32 activations. */
void orc_route_exact(int E, int X, int K, const float *router, const float *xn, int T, float *logits, int *selv,
                     float *wtv);
int orc_moe_exact(int E, int X, int K, int F, const orc_mat *router, const orc_mat *gate, const orc_mat *up,
                  const orc_mat *down, const float *xn, int T, float *out, orc_moe_dbg *dbg);
int orc_matmul_exact(int type, const uint8_t *w, int64_t rows, int64_t cols, uint64_t row_bytes, const float *x,
                     int T, float *y);

/* Host copies of the synthetic generator (same source as the device kernels). */
void orc_synth_f32(uint64_t seed, uint32_t layer, uint32_t kind, uint32_t expert, uint64_t n, float sigma,
                   float *out);
void orc_synth_experts(uint64_t seed, uint32_t layer, uint32_t kind, int type, int64_t rows, int64_t cols,
                       int e0, int e1, float sigma, uint8_t *base);
void orc_rmsnorm(float *y, const float *x, const float *w, int n, float eps);
void orc_rmsnorm_unit(float *y, const float *x, int n, float eps);

#ifdef __cplusplus
}
#endif
#endif /* QMS_ORACLE_H */
