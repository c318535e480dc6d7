/* qmsg.h - MI355X (gfx950) Qwen3-MoE expert-FFN layer behind a plain C ABI.
 *
 * Drop-in for the reference engine's MoE layer with resident experts:
 *   static int moe(QmsModel *m, int l, const float *xn, const float *h, int T, float *out)
 *   (src/model.c:1032-1167), called once per layer by qms_forward (src/model.c:1284).
 * The weights are the GGUF tensor bytes exactly as the reference holds them (stacked
 * ffn_{gate,up,down}_exps [X][rows][cols] and the F32 ffn_gate_inp router,
 * src/model.c:133-157, 359-362), copied once to HBM and never repacked.
 *
 * Conventions follow the reference: int status (0 ok, negative error, reason available from
 * qmsg_last_error), no exceptions, no abort. A context is thread-compatible, not thread-safe:
 * one host thread drives it, like the reference's moe() (src/model.c:329 shares m->eptr).
 * Everything is enqueued on the context's own HIP stream. */
#ifndef QMSG_H
#define QMSG_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ status codes ---- */
#define QMSG_OK 0
#define QMSG_E_INVALID (-1)      /* bad argument or shape                                   */
#define QMSG_E_UNSUPPORTED (-2)  /* outside the integer fast path (src/model.c:1090-1093)    */
#define QMSG_E_NOMEM (-3)        /* device or host allocation failed                         */
#define QMSG_E_DEVICE (-4)       /* HIP runtime error                                        */
#define QMSG_E_RANGE (-5)        /* T above the context's max_tokens, or layer out of range  */

/* GGUF tensor type ids (src/gguf.h:8-10). */
enum {
    QMSG_T_F32 = 0,
    QMSG_T_F16 = 1,
    QMSG_T_Q4_0 = 2,
    QMSG_T_Q4_1 = 3,
    QMSG_T_Q8_0 = 8,
    QMSG_T_Q6_K = 14
};

/* A 2-D weight view, QmsMat (src/quant.h:11-16): row r starts at data + r*row_bytes. */
typedef struct {
    int type;
    int64_t rows, cols;
    uint64_t row_bytes;
    const void *data;
} qmsg_mat;

/* n_expert stacked matrices, QmsExperts (src/model.h:31-35) for resident weights:
 * m.data points at expert 0, expert e at m.data + e*expert_bytes. */
typedef struct {
    qmsg_mat m;
    uint64_t expert_bytes;
} qmsg_experts;

/* The MoE part of QmsLayer (src/model.h:37-45): F32 router [n_expert][n_embd] and the
 * stacked gate/up [n_expert][n_ff_exp][n_embd] and down [n_expert][n_embd][n_ff_exp]. */
typedef struct {
    qmsg_mat router;
    qmsg_experts gate, up, down;
} qmsg_layer;

/* The hyper-parameters moe() reads from QmsCfg (src/model.h:24-29). */
typedef struct {
    int n_embd;    /* E */
    int n_expert;  /* X */
    int n_used;    /* K, top-k */
    int n_ff_exp;  /* F */
} qmsg_cfg;

typedef struct qmsg_ctx qmsg_ctx;

/* Which kernels run the expert products. Every integer path gives the same bits: the int8
 * blocks, the per-block int32 dots and the fp32 rows follow the reference's AVX path exactly.
 *   EXACT: per-row VALU kernels (integer dot4 lane sums, the reference's fp32 lane chains).
 *   MFMA:  the lane sums on f16 MFMAs (exact small integers: 16 rows x 4 slots x half a
 *          block per instruction, 16 rows x 2 slots x a block for waves of one or two
 *          slots), the same fp32 chains on the VALU; for batches of two or
 *          more tokens with gate and up of one type (down Q4_0, Q4_1 or Q6_K; other down rows
 *          on the EXACT kernel).
 *   AUTO:  per stage: Q4_0 / Q4_1 gate/up on MFMA for batches averaging at least 1.25 slots
 *          per active expert, Q6_K gate/up from 2.5, down on MFMA for
 *          batches of at least 64 slots (tokens x n_used; Q6_K down rows: 32), EXACT
 *          otherwise.
 *   FP32:  the reference's --exact mode (qms_exact_math = 1, src/quant.c:95-115,
 *          model.c:1009-1030): router, gate/up and down rows dequantised to fp32 and dotted in
 *          one FMA chain per row (matmul_exact), fp32 activations, no int8 blocks; bit-identical
 *          to the reference run with --exact. Takes Q4_0, Q4_1 or Q6_K for every expert tensor.
 * Every path takes Q4_0, Q4_1 or Q6_K in each expert tensor (src/kernels.c:197-200). On the
 * integer paths a layer whose gate or up is not Q4_0 runs its gate/up rows on the exact
 * slot-tile kernel. */
enum { QMSG_PATH_AUTO = 0, QMSG_PATH_EXACT = 1, QMSG_PATH_MFMA = 2, QMSG_PATH_FP32 = 3 };

/* ------------------------------------------------------------------ lifecycle ---- */

/* No reference counterpart (the reference keeps this state in QmsModel, src/model.h:106-139):
 * create a context on HIP device `device` for `n_layer` resident layers of shape `cfg`,
 * with device scratch for up to `max_tokens` tokens per call. Shapes: n_embd % 32 == 0 and
 * n_ff_exp % 32 == 0 (rows of whole 32-blocks, which the reference's qms_matmul needs for its
 * int8 path, src/quant.c:134-136), n_expert <= 256 (any count), n_used <= min(n_expert, 64);
 * QMSG_E_UNSUPPORTED otherwise. Layers with n_embd % 256 != 0 (past the reference's fast gate,
 * src/model.c:1090-1093, where it runs moe_group_exact) or n_ff_exp % 64 != 0 run slot by slot
 * with the same int8 arithmetic. */
int qmsg_create(qmsg_ctx **out, int device, const qmsg_cfg *cfg, int n_layer, int max_tokens);
void qmsg_destroy(qmsg_ctx *ctx);

/* Text of the last error on this context (or of the last qmsg_create failure when ctx is NULL). */
const char *qmsg_last_error(const qmsg_ctx *ctx);

/* The HIP stream (hipStream_t) all work of this context is enqueued on. */
void *qmsg_stream(qmsg_ctx *ctx);

/* Choose the expert-product kernels (QMSG_PATH_*); AUTO by default. */
int qmsg_set_path(qmsg_ctx *ctx, int path);

/* ------------------------------------------------------------------ weights ---- */

/* Replaces load_experts/load_mat's resident read (src/model.c:133-157, 67-85): copy one
 * layer's router and expert tensors (host memory, GGUF bytes) into HBM unchanged. Shapes
 * and row_bytes are checked against cfg and qms_row_bytes (src/gguf.c:85-96). Expert types:
 * Q4_0, Q4_1, Q6_K (the integer kernels), and Q8_0, F16, F32, whose layers run slot by slot
 * as the reference's moe_group_exact does (src/model.c:1009-1030); F32 up rows with
 * quantised gate and down at n_embd % 256 == 0 are QMSG_E_UNSUPPORTED (the reference's fast
 * path has no F32 dot for them, src/kernels.c:223-231). */
int qmsg_layer_upload(qmsg_ctx *ctx, int layer, const qmsg_layer *host);

/* No reference counterpart: fill a layer with the seeded synthetic weights described in
 * large_model_amd/csrc/qmsg_synth.h, generated on the device (router F32 N(0, sigma), experts
 * N(0, sigma) quantised to gate_type/up_type/down_type: Q4_0, Q4_1 or Q6_K). If router_col0 is not NULL its
 * n_expert floats replace column 0 of the router (a routing bias for skewed expert load). */
int qmsg_layer_synth(qmsg_ctx *ctx, int layer, uint64_t seed, int gate_type, int up_type, int down_type,
                     float sigma, const float *router_col0);

/* No reference counterpart: copy a resident layer back to host memory (for checks). Any
 * pointer may be NULL; sizes are X*E*4 for the router and X*expert_bytes for each tensor. */
int qmsg_layer_download(qmsg_ctx *ctx, int layer, float *router, void *gate, void *up, void *down);

/* ------------------------------------------------------------------ GGUF files ---- */

/* A parsed GGUF v3 model: the tensor table and the first shard's scalar metadata, QmsGguf
 * (src/gguf.h:33-44). Parsing reads headers only and needs no GPU. */
typedef struct qmsg_gguf qmsg_gguf;

/* One tensor-table entry, QmsTensor (src/gguf.h:15-23): ne[0] is the contiguous dimension,
 * unused ne are 1; off is the absolute byte offset in its shard file; nbytes is 0 for a type
 * qms_row_bytes does not know. */
typedef struct {
    char name[96];
    int type;
    int n_dims;
    int64_t ne[4];
    int shard;
    uint64_t off;
    uint64_t nbytes;
} qmsg_tensor;

/* qms_gguf_open (src/gguf.c:222-241, 112-194): parse `path`, or every shard of a
 * "<stem>-00001-of-0000N.gguf" set (src/gguf.c:198-219). Version 3 only; a tensor that runs
 * past the end of its file (its extent computed without wrapping), a truncated header or an
 * unknown value type is an error. On failure *out is NULL and
 * qmsg_last_error(NULL) has the reason. */
int qmsg_gguf_open(qmsg_gguf **out, const char *path);
/* qms_gguf_close (src/gguf.c:243-253). */
void qmsg_gguf_close(qmsg_gguf *g);

/* Number of tensors, and entry i of the table (shard order, then file order). */
int qmsg_gguf_n_tensors(const qmsg_gguf *g);
int qmsg_gguf_tensor(const qmsg_gguf *g, int i, qmsg_tensor *out);
/* qms_gguf_find (src/gguf.c:255-260): index of the tensor called `name`, or -1. */
int qmsg_gguf_find(const qmsg_gguf *g, const char *name);
/* qms_gguf_get_int / qms_gguf_get_float (src/gguf.c:269-283): a required numeric scalar of
 * the first shard's metadata (any integer, float or bool type, converted as the reference
 * does); QMSG_E_INVALID when the key is missing or holds a string. Arrays are not kept. */
int qmsg_gguf_get_int(const qmsg_gguf *g, const char *key, int64_t *out);
int qmsg_gguf_get_float(const qmsg_gguf *g, const char *key, double *out);
/* A string scalar (such as general.architecture) into buf (truncated to n-1 bytes). */
int qmsg_gguf_get_str(const qmsg_gguf *g, const char *key, char *buf, size_t n);

/* The MoE half of read_cfg (src/model.c:278-310): general.architecture must be qwen3moe;
 * qwen3moe.{embedding_length, expert_count, expert_used_count, expert_feed_forward_length}
 * fill cfg, qwen3moe.block_count n_layer and qwen3moe.attention.layer_norm_rms_epsilon eps
 * (either pointer may be NULL). */
int qmsg_gguf_moe_cfg(const qmsg_gguf *g, qmsg_cfg *cfg, int *n_layer, float *eps);

/* The MoE lines of qms_model_load (src/model.c:349, 359-362) for file layers first ..
 * first+n-1 into the context's layers of the same index: blk.L.ffn_gate_inp.weight (F32
 * [n_expert][n_embd]), blk.L.ffn_{gate,up}_exps.weight ([n_expert][n_ff_exp][n_embd]),
 * blk.L.ffn_down_exps.weight ([n_expert][n_embd][n_ff_exp]) and blk.L.ffn_norm.weight (F32
 * [n_embd]), shapes checked like load_mat / load_experts / load_f32_vec (src/model.c:52-85,
 * 133-157). The bytes go from the file to HBM unchanged, through pinned staging buffers
 * that several reader threads fill while the previous buffer is copied. */
int qmsg_gguf_upload(qmsg_ctx *ctx, const qmsg_gguf *g, int first, int n);

/* ------------------------------------------------------------------ dense (trunk) products ---- */

/* A dense weight matrix resident in HBM, a QmsMat (src/quant.h:11-16) loaded by load_mat
 * (src/model.c:67-85): rows of row_bytes GGUF bytes, copied unchanged; *id names it in
 * qmsg_matmul_n. The types of the reference's fast path (qms_fast_supported,
 * src/kernels.c:197-200) at the widths it admits (src/quant.c:134-136): F32, Q4_0 and Q4_1
 * rows with cols % 32 == 0, Q6_K rows with cols % 256 == 0. Widths off the chunked kernels'
 * grid (cols % 256, Q6_K cols % 2048; no Qwen3-MoE trunk matrix has one) take a direct-read
 * kernel, which bounds quantised rows to cols <= 109,216 there. F16 and Q8_0 rows (cols % 32,
 * cols <= 40,960) are taken too: as in the reference, a call holding one of them, and every
 * call on a QMSG_PATH_FP32 context, runs matmul_exact's fp32 chains for all its matrices
 * (src/quant.c:97-115, 131-141). Other types: QMSG_E_UNSUPPORTED. */
int qmsg_mat_upload(qmsg_ctx *ctx, const qmsg_mat *host, int *id);
/* The same from a parsed GGUF file, by tensor name (e.g. "blk.0.attn_q.weight"). */
int qmsg_gguf_upload_mat(qmsg_ctx *ctx, const qmsg_gguf *g, const char *name, int *id);
/* No reference counterpart: a resident matrix of seeded synthetic rows generated on the device
 * (the generator of qmsg_layer_synth, one expert of kind gate, layer 0), for benchmarks. */
int qmsg_mat_synth(qmsg_ctx *ctx, int type, int64_t rows, int64_t cols, uint64_t seed, float sigma, int *id);

/* qms_matmul_n (src/quant.c:128-170) on resident matrices ids[0..nW-1] of equal cols C
 * (types may differ): for a quantised W_i every row of x [T][C] is quantised to int8 blocks
 * (qms_quantize_q8) and ys[i][t][r] = qms_vec_dot_q8(row r of W_i, xq_t); for F32 rows
 * ys[i][t][r] = qms_vec_dot_f32(row r, x_t). Bit-identical to the reference's fast path. Host
 * buffers; blocks until done. The first call with a larger T*C allocates device buffers. */
int qmsg_matmul_n(qmsg_ctx *ctx, const int *ids, int nW, const float *x, int T, float *const *ys);
/* The same on device buffers (x 16-byte aligned), enqueued on the context's stream. */
int qmsg_matmul_n_device(qmsg_ctx *ctx, const int *ids, int nW, const float *d_x, int T, float *const *d_ys);

/* ------------------------------------------------------------------ the layer ---- */

/* moe(m, l, xn, h, T, out) (src/model.c:1032): out[T][E] = sum over the top-K experts of
 * each token of wt * down(silu(gate xq) * up xq), with host buffers; blocks until done.
 * h is accepted for signature parity and ignored (the reference only uses it to prefetch
 * streamed experts, src/model.c:1118). T may be 0. */
int qmsg_moe(qmsg_ctx *ctx, int layer, const float *xn, const float *h, int T, float *out);

/* The same layer on device buffers (d_xn [T][E], d_out [T][E] fp32), enqueued on the
 * context's stream without waiting. */
int qmsg_moe_device(qmsg_ctx *ctx, int layer, const float *d_xn, int T, float *d_out);

/* No counterpart in the reference: for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). The same layer as
 * qmsg_moe_device, with the same results, but its scratch arrays come from a static 32 MiB
 * device array of the library (one per GPU, held until the process ends) instead of the
 * context's, and it calls no hipMalloc, hipFree or other allocating routine. T is not bound
 * by max_tokens; a T whose scratch exceeds 32 MiB (above about 80 tokens at the 235B shape)
 * returns QMSG_E_RANGE. Every call on one GPU shares that array: calls that overlap on one
 * GPU (two streams, or two contexts on one device) race and must be serialised. */
int qmsg_moe_device_noalloc(qmsg_ctx *ctx, int layer, const float *d_xn, int T, float *d_out);

/* The MoE half of qms_forward's layer loop (src/model.c:1283-1285) over the resident layers
 * first .. first+n-1, on device rows d_h [T][E] updated in place: for each layer,
 * xn = rmsnorm(h, ffn_norm) (src/model.c:403-409, eps as the model's rms_norm_eps) and
 * h += moe(l, xn). The attention half of each layer is not part of this library. Enqueued
 * without waiting. */
int qmsg_moe_chain(qmsg_ctx *ctx, int first, int n, float *d_h, int T, float eps);

/* rmsnorm (src/model.c:403-409) of rows device rows of n floats (n % 4 == 0; d_x, d_y and d_w
 * 16-byte aligned): d_y[r] = (float)(x * inv) * w with inv = 1 / sqrt(ss / n + eps) in double
 * and ss the sequential double sum of the squares, bit for bit; d_w is n device floats or NULL
 * (unit weights). d_y may equal d_x. Enqueued without waiting. */
int qmsg_rmsnorm_device(qmsg_ctx *ctx, float *d_y, const float *d_x, const float *d_w, int rows, int n, float eps);

/* How this context's rmsnorm launches (qmsg_moe_chain, qmsg_rmsnorm_device) form ss; the result
 * is the same bits either way. always_walk 0 (the default): a parallel sum brackets ss, and the
 * sum is formed in the reference's order only for rows where some output float differs between
 * the bracket's ends; 1: every row forms it in order. *walked (if not NULL) receives the number
 * of rows that formed it in order since the previous such read, after the stream has drained;
 * the count restarts at 0. No counterpart in the reference (its rmsnorm, src/model.c:403-409,
 * has one order only): for tests and measurement. */
int qmsg_rmsnorm_mode(qmsg_ctx *ctx, int always_walk, int64_t *walked);

/* A layer's ffn_norm weight vector (QmsLayer.ffn_norm, src/model.h:37-45), n_embd floats on
 * the host, copied to HBM; NULL restores the default unit weights. */
int qmsg_layer_norm(qmsg_ctx *ctx, int layer, const float *w);

/* Wait for everything enqueued on the context's stream. */
int qmsg_sync(qmsg_ctx *ctx);

/* ------------------------------------------------------------------ device buffers ---- */

/* No reference counterpart: device memory owned by the context (freed by qmsg_destroy). */
void *qmsg_device_alloc(qmsg_ctx *ctx, size_t bytes);
int qmsg_memcpy_h2d(qmsg_ctx *ctx, void *dst, const void *src, size_t bytes);
int qmsg_memcpy_d2h(qmsg_ctx *ctx, void *dst, const void *src, size_t bytes);

/* No reference counterpart: seeded synthetic layer inputs written to d_x [T][E] on the device
 * (N(0, sigma), optionally RMS-normalised per row like src/model.c:403-409 with a unit weight,
 * optionally with column 0 set to 1.0 to carry a router bias). */
int qmsg_synth_input(qmsg_ctx *ctx, uint64_t seed, int layer, int T, float sigma, int rmsnorm, int bias_col0,
                     float *d_x);

/* ------------------------------------------------------------------ checks and timing ---- */

/* Intermediates of one layer call for parity checks (no counterpart: the reference frees
 * them inside moe()). Host buffers, each optional (NULL = skip). NS = T*K slots. */
typedef struct {
    float *logits;   /* [T][X]                                                    */
    int32_t *sel;    /* [T][K] experts in selection order                         */
    float *wt;       /* [T][K] renormalised routing weights                       */
    int32_t *start;  /* [X+1]  slots of expert e are start[e] .. start[e+1]-1     */
    int32_t *slot_t; /* [NS]   token of each slot                                 */
    int32_t *slot_of;/* [T][K] slot of (token, selection)                         */
    int32_t *active; /* [X]    active experts ascending; count in *n_active       */
    int32_t *n_active;
    void *xq;        /* [T][E/32]  QmsQ8 blocks, 44 bytes each (src/kernels.h:7-12) */
    float *gu;       /* [NS][2F]   gate rows then up rows (EXACT path only)       */
    float *act;      /* [NS][F]    silu(g)*u                                      */
    void *aq;        /* [NS][F/32] QmsQ8 blocks                                   */
    float *dn;       /* [NS][E]    per-slot expert outputs                        */
} qmsg_debug;

/* Run one layer like qmsg_moe and copy the requested intermediates back. */
int qmsg_moe_debug(qmsg_ctx *ctx, int layer, const float *xn, int T, float *out, qmsg_debug *dbg);

/* Exact signed int32 dot of one 32-element block of an expert row with a QmsQ8 block, as the
 * device kernels form it: which = 0 gate, 1 up, 2 down; x is one 44-byte QmsQ8 block.
 * Q4_0: sum (q-8)*x; Q4_1: sum q*x (its m*ds offset is fp32, outside the block dot);
 * Q6_K: sc_lo*sum_{l<16}(q-32)*x + sc_hi*sum_{l>=16}(q-32)*x. */
int qmsg_block_dots(qmsg_ctx *ctx, int layer, int which, int n, const int32_t *expert, const int32_t *row,
                    const int32_t *block, const void *xq_blocks, int32_t *out);

/* No reference counterpart: SiLU as the device kernels evaluate it, a/(1+expf(-a)) with the
 * kernels' expf (src/model.c:424), on n host floats; for checking against the C library. */
int qmsg_eval_silu(qmsg_ctx *ctx, const float *x, int n, float *out);
/* No reference counterpart: exp in double as the routing softmax evaluates it on the device
 * (src/model.c:1049), on n host doubles; for checking against the C library. */
int qmsg_eval_exp(qmsg_ctx *ctx, const double *x, int n, double *out);

/* Per-kernel timing with HIP events on the context's stream (off by default). While on,
 * every kernel launch of the context is bracketed by an event pair. */
int qmsg_profile(qmsg_ctx *ctx, int enable);
/* Launch count and summed milliseconds of kernel `name` since profiling was enabled
 * (synchronises the stream). Names: "route", "gateup", "down", and the MFMA-path kernels. */
int qmsg_profile_read(qmsg_ctx *ctx, const char *name, int64_t *launches, double *total_ms);

/* No reference counterpart: a plain device copy of `bytes` (multiple of 16) with a simple
 * coalesced kernel, used to calibrate HBM byte counters against a known transfer. */
int qmsg_calibrate_copy(qmsg_ctx *ctx, void *d_dst, const void *d_src, size_t bytes);

/* Device facts used by the roofline report: CU count, peak engine clock (kHz), HBM bytes. */
int qmsg_device_info(qmsg_ctx *ctx, int *n_cu, int *clock_khz, uint64_t *hbm_bytes, char *arch, int arch_len);

#ifdef __cplusplus
}
#endif
#endif /* QMSG_H */
