/* ref_harness.c - C entry points into the reference build (oracle/_ref only, test infrastructure).
 *
 * Compiled together with the reference's own src/kernels.c, src/quant.c and src/gguf.c, where
 * they lie, by oracle/Makefile. The reference's MoE layer `moe()` (src/model.c:1032) is file
 * static, so this translation unit includes src/model.c to reach it, builds a one-layer
 * resident QmsModel around caller-owned weight bytes, and calls it unchanged. Nothing here
 * is shipped in the product; the built library is only used to pin the oracle and to time the
 * reference beside the GPU. */
#include "model.c"

#include <omp.h>

/* One MoE layer through the reference's moe(). Types are GGUF ids; each expert tensor is the
 * stacked [X][rows][cols] GGUF layout. Returns moe()'s status. */
int qref_moe(int E, int X, int K, int F, const float *router, int gate_type, const void *gate,
             int up_type, const void *up, int down_type, const void *down, const float *xn, int T,
             float *out)
{
    QmsModel m;
    QmsLayer L;
    memset(&m, 0, sizeof m);
    memset(&L, 0, sizeof L);
    m.c.n_embd = E;
    m.c.n_expert = X;
    m.c.n_used = K;
    m.c.n_ff_exp = F;
    m.c.n_layer = 1;
    L.router.type = QMS_T_F32;
    L.router.rows = X;
    L.router.cols = E;
    L.router.row_bytes = (uint64_t)E * 4;
    L.router.data = (const unsigned char *)router;
    const struct { QmsExperts *x; int type; const void *p; int64_t rows, cols; } t[3] = {
        { &L.gate, gate_type, gate, F, E }, { &L.up, up_type, up, F, E }, { &L.down, down_type, down, E, F }
    };
    for (int i = 0; i < 3; i++) {
        t[i].x->m.type = t[i].type;
        t[i].x->m.rows = t[i].rows;
        t[i].x->m.cols = t[i].cols;
        t[i].x->m.row_bytes = qms_row_bytes(t[i].type, t[i].cols);
        t[i].x->m.data = (const unsigned char *)t[i].p;
        t[i].x->expert_bytes = t[i].x->m.row_bytes * (uint64_t)t[i].rows;
    }
    m.L = &L;
    m.eptr = (const unsigned char **)calloc((size_t)3 * X, sizeof(void *));
    m.overlap = 0;
    const int rc = moe(&m, 0, xn, xn, T, out);
    free(m.eptr);
    return rc;
}

/* The reference's own rmsnorm (src/model.c:403-409) with a unit weight vector. */
void qref_rmsnorm_unit(float *y, const float *x, int n, float eps)
{
    float *w = (float *)malloc((size_t)n * sizeof(float));
    for (int i = 0; i < n; i++) w[i] = 1.0f;
    rmsnorm(y, x, w, n, eps);
    free(w);
}

/* The reference's rmsnorm (src/model.c:403-409) with a caller's weight vector. */
void qref_rmsnorm(float *y, const float *x, const float *w, int n, float eps) { rmsnorm(y, x, w, n, eps); }

/* silu as the reference defines it (src/model.c:424), for element-wise checks. */
float qref_silu(float a) { return silu(a); }

int qref_max_threads(void) { return omp_get_max_threads(); }

/* Which SIMD path this build took (kernels.c selects at compile time). */
const char *qref_isa(void)
{
#if defined(__AVX512VNNI__) && defined(__AVX512VL__)
    return "avx2+avx512vnni";
#elif defined(__AVX2__)
    return "avx2";
#else
    return "scalar";
#endif
}

/* The reference's GGUF reader (qms_gguf_open, src/gguf.c:222-241) on a file: the tensor
 * table flattened into caller arrays (up to cap entries; names 96 bytes apart). Returns the
 * number of tensors, or -1 where qms_gguf_open fails. */
int qref_gguf_table(const char *path, int cap, char *names, int *type, int *n_dims, int64_t *ne, int *shard,
                    uint64_t *off, uint64_t *nbytes)
{
    QmsGguf g;
    if (qms_gguf_open(&g, path) != 0) return -1;
    const int n = g.n_tensors;
    for (int i = 0; i < n && i < cap; i++) {
        const QmsTensor *t = &g.tensors[i];
        memcpy(names + (size_t)i * QMS_MAX_NAME, t->name, QMS_MAX_NAME);
        type[i] = t->type;
        n_dims[i] = t->n_dims;
        for (int d = 0; d < 4; d++) ne[4 * i + d] = t->ne[d];
        shard[i] = t->shard;
        off[i] = t->off;
        nbytes[i] = t->nbytes;
    }
    qms_gguf_close(&g);
    return n;
}

/* qms_gguf_get_int and qms_gguf_get_float of one key: bit 0 set when get_int failed, bit 1
 * when get_float failed; -1 where the file does not open. */
int qref_gguf_value(const char *path, const char *key, int64_t *i, double *f)
{
    QmsGguf g;
    if (qms_gguf_open(&g, path) != 0) return -1;
    int rc = 0;
    if (qms_gguf_get_int(&g, key, i) != 0) rc |= 1;
    if (qms_gguf_get_float(&g, key, f) != 0) rc |= 2;
    qms_gguf_close(&g);
    return rc;
}

/* A whole model file loaded by the reference (qms_model_load: resident weights, KV cache for
 * 8 positions), then its moe() on layer l for caller rows xn [T][n_embd]. Returns -1 when the
 * load fails, else moe()'s status. */
int qref_gguf_moe(const char *path, int l, const float *xn, int T, float *out)
{
    QmsModel m;
    QmsLoadOpts o;
    memset(&o, 0, sizeof o);
    o.ctx = 8;
    o.force = 1;
    o.pin_layers = -1;
    if (qms_model_load(&m, path, &o) != 0) return -1;
    const int rc = l >= 0 && l < m.c.n_layer ? moe(&m, l, xn, xn, T, out) : -1;
    qms_model_free(&m);
    return rc;
}
