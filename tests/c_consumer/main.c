/* A C11 consumer of include/qmsg.h: the integration guide's C blocks (snippets.inc, cut out of
 * the guide by tests/test_c_consumer.py) compiled as a qms maintainer would paste them into
 * src/model.c, driven by a small main.
 *
 *   consumer probe                                 qmsg_create on device 0: prints the status
 *   consumer run MODEL.gguf LAYER T IN.f32 OUT.f32 attach the file (qmsg_attach_file), run the
 *                                                  call site (qms_forward's locals) on IN, write
 *                                                  the layer output to OUT
 *
 * Exit status: 0 done, 2 bad arguments or files, 3 the attach failed, 4 the call site failed. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "qmsg.h"
#ifdef QMSG_WITH_QMS
#include "model.h"        /* the reference's QmsModel / QmsCfg / QmsLayer, for the in-RAM attach */
#endif

#include "snippets.inc"

static float *read_floats(const char *path, long *count)
{
    FILE *f = fopen(path, "rb");
    if (!f) return NULL;
    fseek(f, 0, SEEK_END);
    const long bytes = ftell(f);
    fseek(f, 0, SEEK_SET);
    float *v = bytes > 0 ? (float *)malloc((size_t)bytes) : NULL;
    if (v && fread(v, 1, (size_t)bytes, f) != (size_t)bytes) {
        free(v);
        v = NULL;
    }
    fclose(f);
    *count = bytes / (long)sizeof(float);
    return v;
}

int main(int argc, char **argv)
{
    snippets_mark_used();
    if (argc == 2 && strcmp(argv[1], "probe") == 0) {
        qmsg_cfg cfg = { 256, 16, 4, 256 };
        qmsg_ctx *ctx = NULL;
        const int rc = qmsg_create(&ctx, 0, &cfg, 1, 4);
        printf("status %d %s\n", rc, rc == QMSG_OK ? "ok" : qmsg_last_error(NULL));
        qmsg_destroy(ctx);
        return 0;
    }
    if (argc != 7 || strcmp(argv[1], "run") != 0) {
        fprintf(stderr, "usage: %s probe | run MODEL.gguf LAYER T IN.f32 OUT.f32\n", argv[0]);
        return 2;
    }
    const int layer = atoi(argv[3]), T = atoi(argv[4]);
    long n = 0;
    float *xn = read_floats(argv[5], &n);
    if (!xn || T < 1 || n % T) {
        fprintf(stderr, "consumer: cannot read %d rows from %s\n", T, argv[5]);
        free(xn);
        return 2;
    }
    if (qmsg_attach_file(argv[2], T) != 0) {
        free(xn);
        return 3;
    }
    /* qms_forward's buffers: the residual stream h, the normed input xn, the layer output tmp */
    float *h = (float *)calloc((size_t)n, sizeof(float));
    float *tmp = (float *)malloc((size_t)n * sizeof(float));
    if (qmsg_call_site(layer, xn, h, T, tmp) != 0) {    /* frees all three on failure */
        qmsg_destroy(g_qmsg);
        return 4;
    }
    FILE *f = fopen(argv[6], "wb");
    const int ok = f && fwrite(tmp, sizeof(float), (size_t)n, f) == (size_t)n;
    if (f) fclose(f);
    free(h);
    free(xn);
    free(tmp);
    qmsg_destroy(g_qmsg);
    return ok ? 0 : 2;
}
