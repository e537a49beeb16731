/*
 * ref_harness.c - exports the reference's own CPU kernels (lawnak/FastGGUF fastgguf.c, compiled
 * from where it lies under /root/reference) as plain C entry points, so the test suite can write
 * golden vectors with them and bench.py can time them as the CPU baseline.
 *
 * TEST INFRASTRUCTURE ONLY. Built by oracle/Makefile into oracle/_ref/ (git-ignored); never
 * linked into the product library. The reference source is #included, not copied: compiling it
 * with FG_VARIANT set renames its main() functions (fastgguf.c:51-59) so this file can add its own
 * exported wrappers around the `static` kernels.
 *
 * Built with FG_HIP on a copy of fastgguf.c that include/fastgguf_c_hip.patch has patched, the same
 * wrappers run the reference's own call sites (matvec 2575, matvec_multi 2552, matmul 3004,
 * moe_ffn 4588) with their tensors uploaded by the patched gpu_upload_tensor (2060): the drop-in
 * test calls them on the GPU box and compares with the unpatched build's CPU results.
 */
#define FG_VARIANT ref
#include FG_REF_SOURCE

#define FGR_EXPORT __attribute__((visibility("default")))

FGR_EXPORT const char *fgr_build(void) { return FG_CPU_BUILD; }

FGR_EXPORT void fgr_init(int max_cols) {
    static int fp16_ready;
    if (!fp16_ready) { fp16_init(); fp16_ready = 1; }
    matvec_init_scratch(max_cols);
}

FGR_EXPORT int fgr_threads(void) { return omp_get_max_threads(); }

#ifdef FG_HIP
/* the patched fg_gpu_init_ex (1968; mode 0 honours FASTGGUF_GPU, 1 probes) and what it left in
 * g_gpu: state 1 ready, -1 on the CPU; counts[3] = n_offloaded, n_skip_type, n_skip_mem */
FGR_EXPORT int fgr_hip_init(int mode) {
    fg_gpu_init_ex(mode);
    return g_gpu.state;
}
FGR_EXPORT int fgr_hip_state(int *counts) {
    if (counts) {
        counts[0] = g_gpu.n_offloaded;
        counts[1] = g_gpu.n_skip_type;
        counts[2] = g_gpu.n_skip_mem;
    }
    return g_gpu.state;
}
#endif

FGR_EXPORT void fgr_quantize_q8(const float *x, void *out, int n) { quantize_q8(x, (q8_blk_t *)out, n); }
FGR_EXPORT void fgr_quantize_q8k(const float *x, void *out, int n) { quantize_q8k(x, (q8k_blk_t *)out, n); }

FGR_EXPORT float fgr_dot_q8_0(const uint8_t *row, const void *xq, int nb) { return dot_q8_0_q8(row, (const q8_blk_t *)xq, nb); }
FGR_EXPORT float fgr_dot_q4_K(const uint8_t *row, const void *y, int nb) { return dot_q4_K_q8k(row, (const q8k_blk_t *)y, nb); }
FGR_EXPORT float fgr_dot_q6_K(const uint8_t *row, const void *y, int nb) { return dot_q6_K_q8k(row, (const q8k_blk_t *)y, nb); }
FGR_EXPORT float fgr_dot_q5_0(const uint8_t *row, const void *xq, int nb) { return dot_q5_0_q8(row, (const q8_blk_t *)xq, nb); }
FGR_EXPORT float fgr_dot_q5_K(const uint8_t *row, const void *y, int nb) { return dot_q5_K_q8k(row, (const q8k_blk_t *)y, nb); }
/* dot_row (2183-2201) for a 32-value type on Q8 activations */
FGR_EXPORT float fgr_dot_q32(uint32_t type, const uint8_t *row, const void *xq, int nb) {
    int fail = 0;
    return dot_row(type, ACT_Q8, row, (const q8_blk_t *)xq, NULL, NULL, 32 * nb, &fail);
}

/* a tensor view over caller memory; `repack` asks for the 8-row layout the reference builds at
 * load time (repack_tensor, 2486). repack_tensor drops the source pages with MADV_DONTNEED, so
 * it is given a private copy of the weights. */
static int make_tensor(tensor_t *t, uint32_t type, int repack, const uint8_t *w, int64_t rows, int cols,
                       uint8_t **copy) {
    memset(t, 0, sizeof(*t));
    snprintf(t->name, sizeof(t->name), "harness");
    t->type = type;
    t->n_dims = 2;
    t->ne[0] = (uint64_t)cols;
    t->ne[1] = (uint64_t)rows;
    t->data = w;
    t->nbytes = row_stride(type, (uint64_t)cols) * (uint64_t)rows;
    *copy = NULL;
#ifdef FG_HIP
    gpu_upload_tensor(t);     /* before the repack, as in model_load (4509-4557) */
    if (t->gpu) return 0;
#endif
    if (repack) {
        *copy = (uint8_t *)malloc(t->nbytes);
        if (!*copy) return -1;
        memcpy(*copy, w, t->nbytes);
        t->data = *copy;
        if (repack_tensor(t) == 0) return -1;
    }
    return 0;
}

static void drop_tensor(tensor_t *t, uint8_t *copy) {
#ifdef FG_HIP
    if (t->gpu) {
        fgh_tensor_free((fgh_tensor *)t->gpu);
        g_gpu.used -= t->nbytes;
        t->gpu = NULL;
    }
#endif
    free((void *)t->rp);
    free(copy);
}

FGR_EXPORT int fgr_matvec(uint32_t type, int repack, const uint8_t *w, int64_t rows, int cols,
                          const float *x, float *y) {
    tensor_t t;
    uint8_t *copy;
    fgr_init(cols);
    if (make_tensor(&t, type, repack, w, rows, cols, &copy) != 0) return -1;
    int rc = matvec(&t, x, y);
    drop_tensor(&t, copy);
    return rc;
}

/* matvec_multi over n <= 4 tensors with the same x (2552) */
FGR_EXPORT int fgr_matvec_multi(int n, const uint32_t *types, const int *repack, const uint8_t *const *w,
                                const int64_t *rows, int cols, const float *x, float *const *y) {
    tensor_t t[4], *tp[4];
    uint8_t *copy[4] = {0};
    if (n < 1 || n > 4) return -1;
    fgr_init(cols);
    for (int i = 0; i < n; i++) {
        if (make_tensor(&t[i], types[i], repack[i], w[i], rows[i], cols, &copy[i]) != 0) return -1;
        tp[i] = &t[i];
    }
    int rc = matvec_multi(n, tp, x, y);
    for (int i = 0; i < n; i++) drop_tensor(&t[i], copy[i]);
    return rc;
}

FGR_EXPORT int fgr_matmul(uint32_t type, int repack, const uint8_t *w, int64_t rows, int cols,
                          const float *X, int ldx, float *Y, int ldy, int nb) {
    tensor_t t;
    uint8_t *copy;
    if (nb < 1 || nb > FG_BATCH) return -1;
    fgr_init(cols);
    if (make_tensor(&t, type, repack, w, rows, cols, &copy) != 0) return -1;
    int rc = matmul(&t, X, ldx, Y, ldy, nb);
    drop_tensor(&t, copy);
    return rc;
}

/* moe_ffn (4588) for n_tok tokens, one call per token as forward_chunk does (5089-5091).
 * The router is an F32 tensor whose row e is (logit_e, 0, ..., 0); with X[t][0] == 1 the
 * reference's own router matvec then reproduces the given logits exactly. */
FGR_EXPORT int fgr_moe_ffn(uint32_t tg_type, uint32_t tu_type, uint32_t td_type,
                           const uint8_t *gate, const uint8_t *up, const uint8_t *down,
                           int n_expert, int k, int n_embd, int ff, const float *logits,
                           const float *X, float *Y, int n_tok, int32_t *sel_out, float *w_out) {
    fgr_init(n_embd > ff ? n_embd : ff);
    model_t *mm = (model_t *)calloc(1, sizeof(model_t));
    float *router = (float *)calloc((size_t)n_expert * n_embd, sizeof(float));
    if (!mm || !router) { free(mm); free(router); return -1; }
    mm->n_embd = n_embd; mm->ff_exp = ff; mm->n_expert = n_expert; mm->n_expert_used = k;
    mm->moe_probs = (float *)malloc((size_t)n_expert * sizeof(float));
    mm->moe_w = (float *)malloc((size_t)k * sizeof(float));
    mm->moe_sel = (int *)malloc((size_t)k * sizeof(int));
    mm->moe_h = (float *)malloc((size_t)k * ff * sizeof(float));
    mm->moe_xq = (q8_blk_t *)malloc(((size_t)k * ff / 32 + 1) * sizeof(q8_blk_t));
    mm->moe_xk = (q8k_blk_t *)malloc(((size_t)k * ff / 256 + 1) * sizeof(q8k_blk_t));
    tensor_t ti, tg, tu, td;
    memset(&ti, 0, sizeof(ti));
    ti.type = T_F32; ti.n_dims = 2; ti.ne[0] = (uint64_t)n_embd; ti.ne[1] = (uint64_t)n_expert;
    ti.data = (const uint8_t *)router;
    tg = tu = td = ti;
    tg.type = tg_type; tu.type = tu_type; td.type = td_type;
    tg.n_dims = tu.n_dims = td.n_dims = 3;
    tg.ne[0] = tu.ne[0] = (uint64_t)n_embd; tg.ne[1] = tu.ne[1] = (uint64_t)ff;
    tg.ne[2] = tu.ne[2] = (uint64_t)n_expert;
    td.ne[0] = (uint64_t)ff; td.ne[1] = (uint64_t)n_embd; td.ne[2] = (uint64_t)n_expert;
    tg.data = gate; tu.data = up; td.data = down;
    layer_t LL;
    memset(&LL, 0, sizeof(LL));
    LL.ffn_gate_inp = &ti; LL.ffn_gate_exps = &tg; LL.ffn_up_exps = &tu; LL.ffn_down_exps = &td;
    int rc = 0;
#ifdef FG_HIP
    tg.nbytes = row_stride(tg_type, (uint64_t)n_embd) * ff * n_expert;
    tu.nbytes = row_stride(tu_type, (uint64_t)n_embd) * ff * n_expert;
    td.nbytes = row_stride(td_type, (uint64_t)ff) * n_embd * n_expert;
    gpu_upload_tensor(&tg);
    gpu_upload_tensor(&tu);
    gpu_upload_tensor(&td);
#endif
    for (int t = 0; t < n_tok && rc == 0; t++) {
        const float *x = X + (size_t)t * n_embd;
        if (x[0] != 1.0f) { rc = -2; break; }
        for (int e = 0; e < n_expert; e++) router[(size_t)e * n_embd] = logits[(size_t)t * n_expert + e];
        rc = moe_ffn(mm, &LL, x, Y + (size_t)t * n_embd);
        for (int j = 0; j < k; j++) {
            if (sel_out) sel_out[(size_t)t * k + j] = mm->moe_sel[j];
            if (w_out) w_out[(size_t)t * k + j] = mm->moe_w[j];
        }
    }
#ifdef FG_HIP
    drop_tensor(&tg, NULL);
    drop_tensor(&tu, NULL);
    drop_tensor(&td, NULL);
#endif
    free(mm->moe_probs); free(mm->moe_w); free(mm->moe_sel); free(mm->moe_h);
    free(mm->moe_xq); free(mm->moe_xk); free(mm); free(router);
    return rc;
}

/* persistent tensors for timing the reference's CPU path (bench.py cpu_baseline): the 8-row
 * repack happens once, as at model load (4542-4557), and each call is one matvec / matvec_multi */
typedef struct { tensor_t t; uint8_t *copy; } fgr_tensor;

FGR_EXPORT void *fgr_tensor_new(uint32_t type, int repack, const uint8_t *w, int64_t rows, int cols) {
    fgr_tensor *h = (fgr_tensor *)calloc(1, sizeof(fgr_tensor));
    if (!h) return NULL;
    fgr_init(cols);
    if (make_tensor(&h->t, type, repack, w, rows, cols, &h->copy) != 0) { free(h); return NULL; }
    return h;
}

FGR_EXPORT void fgr_tensor_free(void *p) {
    fgr_tensor *h = (fgr_tensor *)p;
    if (!h) return;
    drop_tensor(&h->t, h->copy);
    free(h);
}

FGR_EXPORT int fgr_tensor_matvec_multi(int n, void *const *hs, const float *x, float *const *y) {
    tensor_t *tp[4];
    if (n < 1 || n > 4) return -1;
    for (int i = 0; i < n; i++) tp[i] = &((fgr_tensor *)hs[i])->t;
    return n == 1 ? matvec(tp[0], x, y[0]) : matvec_multi(n, tp, x, y);
}

/* gguf_open (342-440) on a file: 0 and its summary and tensor table (up to cap tensors: names
 * [cap][128], dims [cap][4], offsets from the start of the file), kv_num (441-448) of n_keys
 * NUL-separated keys with default -1; or gguf_open's -1 */
FGR_EXPORT int fgr_gguf_table(const char *path, uint32_t *version, uint64_t *alignment, int64_t *n_kvs,
                              int64_t *n_tensors, char *names, uint32_t *types, int32_t *n_dims, uint64_t *ne,
                              uint64_t *offsets, uint64_t *nbytes, int64_t cap, const char *keys, int n_keys,
                              double *kv_vals) {
    gguf_t g;
    if (gguf_open(&g, path) != 0) return -1;
    *version = g.version;
    *alignment = g.alignment;
    *n_kvs = (int64_t)g.n_kvs;
    *n_tensors = (int64_t)g.n_tensors;
    for (size_t i = 0; i < g.n_tensors && (int64_t)i < cap; i++) {
        tensor_t *t = &g.tensors[i];
        memcpy(names + 128 * i, t->name, 128);
        types[i] = t->type;
        n_dims[i] = t->n_dims;
        for (int j = 0; j < 4; j++) ne[4 * i + j] = t->ne[j];
        offsets[i] = (uint64_t)(t->data - g.map.data);
        nbytes[i] = t->nbytes;
    }
    for (int k = 0; k < n_keys; k++) {
        kv_vals[k] = kv_num(&g, keys, -1.0);
        keys += strlen(keys) + 1;
    }
    mmap_close(&g.map);
    return 0;
}

/* attn_rows (3273-3326) for nr <= 4 query rows sharing one KV head: q [nr][hd], o [nr][hd] */
FGR_EXPORT int fgr_attn_rows(int nr, const float *q, float *o, const int *st, const int *en, const float *ck,
                             const float *cv, int kv_dim, int kvo, int cap, int hd, float scale) {
    if (nr < 1 || nr > 4) return -1;
    int lo = st[0], hi = en[0];
    for (int r = 1; r < nr; r++) { if (st[r] < lo) lo = st[r]; if (en[r] > hi) hi = en[r]; }
    int sld = hi - lo + 1 + 8;
    float *sb = (float *)calloc((size_t)4 * sld, sizeof(float));
    if (!sb) return -1;
    const float *qr[4];
    float *orow[4];
    for (int r = 0; r < nr; r++) { qr[r] = q + (size_t)r * hd; orow[r] = o + (size_t)r * hd; }
    attn_rows(nr, qr, orow, st, en, ck, cv, kv_dim, kvo, cap, hd, scale, sb, sld);
    free(sb);
    return 0;
}

/* TurboQuant KV cache (fastgguf.c:3341-3513): the reference's own rotation, slice quantizer and
 * the per-head attention step of forward (4760-4846) over a quantized ring cache, one row at a
 * time. kq / vq: [cap] slots of kqs / vqs bytes; row r reads head kvh[r]'s record. q is the
 * unrotated query; o receives the unrotated output. */
FGR_EXPORT void fgr_kvq_signs(float *out, int n) {
    kvq_init();
    for (int i = 0; i < n && i < KVQ_MAX_HD; i++) out[i] = g_kvq_sign[i];
}
FGR_EXPORT void fgr_kvq_rotate(float *x, int n, int inverse) {
    kvq_init();
    if (inverse) kvq_unrotate(x, n);
    else kvq_rotate(x, n);
}
FGR_EXPORT void fgr_kvq_quant(const float *x, int hd, uint8_t *rec, int bits) { kvq_quant_slice(x, hd, rec, bits); }
FGR_EXPORT void fgr_kvq_dequant(const uint8_t *rec, float *out, int hd, int bits) { kvq_dequant_slice(rec, out, hd, bits); }
FGR_EXPORT int fgr_kvq_attn_rows(int nr, const float *q, float *o, const int *st, const int *en, const uint8_t *kq,
                                 const uint8_t *vq, int kqs, int vqs, const int *kvh, int cap, int hd, int kbits,
                                 int vbits, float scale) {
    kvq_init();
    for (int r = 0; r < nr; r++) {
        int n = en[r] - st[r] + 1;
        if (n < 1 || n > cap) return -1;
        float *qh = (float *)malloc((size_t)hd * sizeof(float));
        float *scores = (float *)malloc((size_t)n * sizeof(float));
        if (!qh || !scores) { free(qh); free(scores); return -1; }
        memcpy(qh, q + (size_t)r * hd, (size_t)hd * sizeof(float));
        kvq_rotate(qh, hd);
        for (int p = st[r]; p <= en[r]; p++)
            scores[p - st[r]] = kvq_dot_k(qh, kq + (size_t)(p % cap) * kqs + (size_t)kvh[r] * KVQ_REC(hd, kbits), hd,
                                          kbits) * scale;
        softmax_inplace(scores, n);
        float *oh = o + (size_t)r * hd;
        memset(oh, 0, (size_t)hd * sizeof(float));
        for (int p = st[r]; p <= en[r]; p++) {
            float w = scores[p - st[r]];
            if (w == 0.0f) continue;
            kvq_axpy_v(oh, w, vq + (size_t)(p % cap) * vqs + (size_t)kvh[r] * KVQ_REC(hd, vbits), hd, vbits);
        }
        kvq_unrotate(oh, hd);
        free(qh);
        free(scores);
    }
    return 0;
}
