/* abi_smoke.c - a plain C caller of include/fastgguf_hip.h (test infrastructure): proves the header
 * compiles as C and the library links and runs from C, as fastgguf.c would call it.
 *
 *   gcc -std=c99 -Wall -Werror -I include tests/c_abi/abi_smoke.c -L fastgguf_amd -lfastgguf_hip
 *
 * argv[1]: a GGUF file (tests/golden/tiny.gguf). Without a usable device fgh_open fails and the
 * program, like fastgguf.c's fg_gpu_init, stays on its CPU path; with one, it runs a closed-form
 * Q8_0 matvec (every weight 3, scale 1, x = 127 -> q = 127, d = 1: y = 3 * 127 * 256 = 97536),
 * the same product through the prompt GEMM for 16 tokens (token b's x = 127 - b, so its outputs are
 * 3 * 256 * (127 - b): q = 127 - b with d = 1), and checks the upload counters. */
#include <stdio.h>
#include <string.h>

#include "fastgguf_hip.h"

int main(int argc, char **argv) {
    if (argc < 2) return 2;
    char err[256] = {0};
    fgh_gguf *g = NULL;
    if (fgh_gguf_open(argv[1], &g, err, sizeof(err)) != FGH_OK) {
        fprintf(stderr, "gguf_open: %s\n", err);
        return 1;
    }
    int64_t n_tensors = 0;
    uint64_t alignment = 0;
    fgh_gguf_summary(g, NULL, &alignment, NULL, &n_tensors);
    const int64_t i = fgh_gguf_find(g, "output.weight");
    fgh_gguf_tensor_info ti;
    if (i < 0 || fgh_gguf_tensor(g, i, &ti) != FGH_OK || ti.type != FGH_T_Q8_0) return 1;
    printf("gguf: %lld tensors, alignment %llu, output.weight %llu x %llu Q8_0\n", (long long)n_tensors,
           (unsigned long long)alignment, (unsigned long long)ti.ne[1], (unsigned long long)ti.ne[0]);

    fgh_ctx *ctx = NULL;
    const int rc = fgh_open(-1, 0, &ctx);
    if (rc != FGH_OK) {
        printf("open: status %d, staying on the CPU path\n", rc);  /* the reference's g_gpu.state = -1 */
        fgh_gguf_close(g);
        return rc == FGH_ERR_DEVICE && ctx == NULL ? 0 : 1;
    }
    enum { COLS = 256, ROWS = 16 };
    static unsigned char w[ROWS * (COLS / 32) * 34];
    for (int b = 0; b < ROWS * COLS / 32; b++) {
        unsigned char *p = w + 34 * b;
        p[0] = 0x00;
        p[1] = 0x3C; /* fp16 1.0 */
        memset(p + 2, 3, 32);
    }
    fgh_tensor *t = NULL;
    float x[COLS], y[ROWS];
    for (int k = 0; k < COLS; k++) x[k] = 127.0f;
    int ok = fgh_upload(ctx, FGH_T_Q8_0, COLS, ROWS, 1, FGH_ORDER_AUTO, w, sizeof(w), &t) == FGH_OK &&
             fgh_matvec(ctx, t, x, y) == FGH_OK;
    for (int r = 0; ok && r < ROWS; r++) ok = y[r] == 97536.0f;
    printf("matvec: %s\n", ok ? "ok" : fgh_last_error(ctx));
    enum { NB = 16 };
    static float X[NB * COLS], Y[NB * ROWS];
    for (int b = 0; b < NB; b++)
        for (int k = 0; k < COLS; k++) X[b * COLS + k] = (float)(127 - b);
    int okm = ok && fgh_matmul(ctx, t, X, COLS, Y, ROWS, NB) == FGH_OK;
    for (int b = 0; okm && b < NB; b++)
        for (int r = 0; okm && r < ROWS; r++) okm = Y[b * ROWS + r] == 3.0f * 256.0f * (float)(127 - b);
    printf("matmul: %s\n", okm ? "ok" : fgh_last_error(ctx));
    fgh_info_t in;
    int oki = fgh_info(ctx, &in) == FGH_OK && in.n_offloaded == 1 && in.used > 0;
    printf("info: %s (%s, %llu MB)\n", oki ? "ok" : "wrong counters", in.name, (unsigned long long)(in.vram >> 20));
    ok = ok && okm && oki;
    fgh_tensor_free(t);
    fgh_close(ctx);
    fgh_gguf_close(g);
    return ok ? 0 : 1;
}
