/*
 * A C99 program that drives the library through include/chat_wgpu.h alone,
 * the way a cgo or Rust FFI binding would (no C++, no Python): one Q4_0 GEMV
 * through cw_q4_gemv, then a synthetic Qwen3-shaped model's greedy generate
 * (src/model/mod.rs:57-125), then two calls that must fail with CW_ERR_ARG.
 *
 * usage: generate_demo SEED MODE N_NEW TOKEN...
 *   MODE is CW_STEP_EAGER (0) or CW_STEP_GRAPH (1).
 * Output, one item per line:
 *   gemv <checksum of y as %.9g>
 *   ids <N_NEW produced ids>
 *   refused <cw_last_error() of each refused call>
 * Exit status 0 on success, 2 when a call fails (its message on stderr).
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "chat_wgpu.h"

#define TRY(call)                                                              \
    do {                                                                       \
        int rc_ = (call);                                                      \
        if (rc_ != CW_OK) {                                                    \
            fprintf(stderr, "error: %s -> %d: %s\n", #call, rc_, cw_last_error()); \
            return 2;                                                          \
        }                                                                      \
    } while (0)

/* a fixed, seeded GEMV: y[64] = W[64][256] x[256], Q4_0 scales d = 1/64 */
static int run_gemv(cw_ctx *ctx) {
    enum { IN = 256, OUT = 64, NB = OUT * IN / 32 };
    static float x[IN], y[OUT];
    static uint16_t sc[NB];
    static uint8_t q[NB * 16];
    uint32_t s = 12345u;
    for (int i = 0; i < IN; ++i) {
        s = s * 1664525u + 1013904223u;
        x[i] = (float)((int)(s >> 24) - 128) / 128.0f;
    }
    for (int b = 0; b < NB; ++b) sc[b] = 0x2400; /* f16 1/64 */
    for (int i = 0; i < NB * 16; ++i) {
        s = s * 1664525u + 1013904223u;
        q[i] = (uint8_t)(s >> 24);
    }
    void *dx, *ds, *dq, *dy;
    TRY(cw_alloc(ctx, sizeof x, &dx));
    TRY(cw_alloc(ctx, sizeof sc, &ds));
    TRY(cw_alloc(ctx, sizeof q, &dq));
    TRY(cw_alloc(ctx, sizeof y, &dy));
    TRY(cw_upload(ctx, dx, x, sizeof x));
    TRY(cw_upload(ctx, ds, sc, sizeof sc));
    TRY(cw_upload(ctx, dq, q, sizeof q));
    TRY(cw_q4_gemv(ctx, (const float *)dx, (const uint16_t *)ds, (const uint8_t *)dq, IN, OUT,
                   (float *)dy));
    TRY(cw_download(ctx, y, dy, sizeof y));
    double sum = 0.0;
    for (int i = 0; i < OUT; ++i) sum += (double)y[i] * (double)(i + 1);
    printf("gemv %.9g\n", sum);
    TRY(cw_free(ctx, dx));
    TRY(cw_free(ctx, ds));
    TRY(cw_free(ctx, dq));
    TRY(cw_free(ctx, dy));
    return 0;
}

int main(int argc, char **argv) {
    if (argc < 5) {
        fprintf(stderr, "usage: %s SEED MODE N_NEW TOKEN...\n", argv[0]);
        return 2;
    }
    const unsigned long long seed = strtoull(argv[1], NULL, 10);
    const int mode = atoi(argv[2]);
    const int n_new = atoi(argv[3]);
    const int n_prompt = argc - 4;
    uint32_t prompt[64];
    uint32_t out[64];
    if (n_prompt > 64 || n_new < 1 || n_new > 64) {
        fprintf(stderr, "at most 64 prompt and 64 new tokens\n");
        return 2;
    }
    for (int i = 0; i < n_prompt; ++i) prompt[i] = (uint32_t)strtoul(argv[4 + i], NULL, 10);

    cw_ctx *ctx = NULL;
    TRY(cw_ctx_create(0, &ctx));
    if (run_gemv(ctx) != 0) return 2;

    /* 2 layers, dim 256, 4 query heads over 2 kv heads of 64, hidden 512,
     * vocab 1000, f32 cache of 64 positions */
    cw_model_config cfg;
    memset(&cfg, 0, sizeof cfg);
    cfg.family.qk_norm = 1;
    cfg.n_layers = 2;
    cfg.dim = 256;
    cfg.n_heads = 4;
    cfg.n_kv_heads = 2;
    cfg.head_dim = 64;
    cfg.hidden = 512;
    cfg.vocab = 1000;
    cfg.eps = 1e-6f;
    cfg.rope_theta = 1e6f;
    cfg.max_seq = 64;
    cfg.kv_dtype = CW_F32;
    cw_model *m = NULL;
    TRY(cw_model_create(ctx, &cfg, &m));
    TRY(cw_model_load_synthetic(m, (uint64_t)seed));
    TRY(cw_model_finalize(m));
    TRY(cw_generate(m, prompt, n_prompt, n_new, 0, mode, out));
    printf("ids");
    for (int i = 0; i < n_new; ++i) printf(" %u", out[i]);
    printf("\n");

    /* errors come back as codes with a message, nothing is launched */
    if (cw_generate(m, prompt, n_prompt, 64, 0, mode, out) != CW_ERR_ARG) return 2;
    printf("refused %s\n", cw_last_error());
    if (cw_q4_gemv(ctx, NULL, NULL, NULL, 33, 8, NULL) != CW_ERR_ARG) return 2;
    printf("refused %s\n", cw_last_error());

    TRY(cw_model_destroy(m));
    TRY(cw_ctx_destroy(ctx));
    return 0;
}
