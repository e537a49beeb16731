/*
 * fastgguf_hip.h - C ABI of the MI355X (gfx950) backend for fastgguf's quantized
 * weight x Q8-activation hot path: GGUF Q4_K / Q6_K / Q8_0 weights, and Q5_K, Q5_0, Q4_0, Q4_1,
 * Q5_1, IQ4_NL, Q2_K, Q3_K and IQ4_XS (the other block types of the reference's integer kernels;
 * its own OpenCL offload leaves the last three on the CPU), multiplied by
 * activations quantized to the reference's Q8 / Q8_K blocks, as a decode matvec, a <=64-token prompt matmul and a
 * mixture-of-experts FFN over the router-selected experts; and the float weight types F32, F16
 * and BF16, whose row kernels take x in fp32 (dot_row, fastgguf.c:2207-2214).
 *
 * The ABI is plain C: fixed-width integers, plain pointers and sizes, opaque handles, no
 * callbacks, no varargs, no C++ or torch types. A Rust `extern "C"` block or a C caller binds it
 * directly. Every entry point returns FGH_OK (0) or a negative FGH_* status and never aborts; a
 * caller treats any non-zero status the way fastgguf.c treats a failed fg_gpu_matvec
 * (fastgguf.c:2577-2581): report it and recompute on its own CPU kernels.
 *
 * Results are those of the reference's CPU kernels (the ones `fastgguf selftest` checks), not of
 * its OpenCL kernels: activations are quantized exactly as quantize_q8 / quantize_q8k
 * (fastgguf.c:746-793) do, per-block integer dot products are exact, and the fp32 outputs follow
 * the reference's accumulation order for matvec and MoE (bit-identical) and agree to within
 * 1e-5 relative per output vector for the MFMA prompt GEMM (and for the per-token kernels that
 * stand in for the reference's CPU prompt GEMM of Q6_K tensors and the 32-value types).
 *
 * Threading: a context is used by one host thread at a time, like the reference's g_gpu state
 * (fastgguf.c:1845-1857). Host-pointer calls are synchronous: outputs are valid on return, as
 * with fg_gpu_matvec_raw's blocking read (fastgguf.c:2110). *_dev calls take device pointers and
 * are asynchronous on the context's stream.
 */
#ifndef FASTGGUF_HIP_H
#define FASTGGUF_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FGH_ABI_VERSION 1

/* exported from the shared library (built with -fvisibility=hidden) */
#if defined(__GNUC__) || defined(__clang__)
#define FGH_API __attribute__((visibility("default")))
#else
#define FGH_API
#endif

/* GGML tensor types handled here (the reference's enum, fastgguf.c:215-221) */
#define FGH_T_F32 0u
#define FGH_T_F16 1u
#define FGH_T_Q4_0 2u
#define FGH_T_Q4_1 3u
#define FGH_T_Q5_0 6u
#define FGH_T_Q5_1 7u
#define FGH_T_Q8_0 8u
#define FGH_T_Q2_K 10u
#define FGH_T_Q3_K 11u
#define FGH_T_Q4_K 12u
#define FGH_T_Q5_K 13u
#define FGH_T_Q6_K 14u
#define FGH_T_IQ4_NL 20u
#define FGH_T_IQ4_XS 23u
#define FGH_T_BF16 30u

/* status codes */
#define FGH_OK 0
#define FGH_ERR (-1)           /* operation failed (the reference's -1 from fg_gpu_matvec) */
#define FGH_ERR_ARG (-2)       /* bad argument or shape mismatch */
#define FGH_SKIP_TYPE (-3)     /* upload: unsupported type, cols not a block multiple, or too many
                                  cols for the kernel's LDS copy of x */
#define FGH_SKIP_MEM (-4)      /* upload: over the memory budget, or device allocation failed */
#define FGH_ERR_DEVICE (-5)    /* no usable device, or a HIP runtime error */

/* fp32 accumulation order of a Q4_K / Q4_0 tensor's matvec: which reference kernel it reproduces
 * (the other types have one order) */
#define FGH_ORDER_AUTO (-1)    /* what the reference CPU path would pick (repack_tensor, 2486) */
#define FGH_ORDER_ROW 0        /* dot_q4_K_q8k / dot_q4_0_q8 (fastgguf.c:1118, 833), file-layout rows */
#define FGH_ORDER_REPACKED 1   /* dot_q4Kx8 / dot_q40x8 (fastgguf.c:2322, 2424), the 8-row repacked layout */

/* activation block kinds for the quantizer test hook (type_uses_q8, fastgguf.c:2167) */
#define FGH_ACT_Q8 1           /* q8_blk_t  {f32 d; i8 qs[32];  i16 s16[2];}    40 bytes */
#define FGH_ACT_Q8K 2          /* q8k_blk_t {f32 d; i8 qs[256]; i16 bsums[16];} 292 bytes */

typedef struct fgh_ctx fgh_ctx;
typedef struct fgh_tensor fgh_tensor;

/* counters mirroring g_gpu (fastgguf.c:1845-1857) */
typedef struct {
    uint64_t vram;          /* device memory in bytes */
    uint64_t budget;        /* weight memory budget in bytes */
    uint64_t used;          /* bytes held by uploaded tensors */
    int32_t n_offloaded;    /* tensors uploaded */
    int32_t n_skip_type;    /* uploads refused: unsupported type / shape */
    int32_t n_skip_mem;     /* uploads refused: over budget / allocation failed */
    int32_t device;         /* HIP device index */
    char name[96];          /* device name */
} fgh_info_t;

/* ---- context: replaces fg_gpu_init / fg_gpu_init_ex (fastgguf.c:1968-2057) ----
 * device < 0 picks device 0 (the reference's FASTGGUF_GPU_DEVICE default is the largest discrete
 * GPU; on a one-GPU MI355X box that is device 0). budget_bytes == 0 means 87.5 % of device memory
 * (fastgguf.c:2045). Runs a self-check (the role of gpu_selfcheck, 1898-1965): a weight type of
 * every kernel family through upload and matvec (Q4_K in both orders and through the prompt
 * GEMM) on small cases
 * whose outputs are exact integers in closed form; on any failure it prints the case to stderr,
 * returns < 0 with *out = NULL, and the caller stays on the CPU. */
FGH_API int fgh_open(int device, uint64_t budget_bytes, fgh_ctx **out);
FGH_API void fgh_close(fgh_ctx *ctx);
FGH_API int fgh_info(const fgh_ctx *ctx, fgh_info_t *out);
/* message for the last failing call on this context (never NULL) */
FGH_API const char *fgh_last_error(const fgh_ctx *ctx);

/* ---- upload: replaces gpu_upload_tensor (fastgguf.c:2060-2081) ----
 * host_data holds n_mats x rows x row_bytes(type, cols) bytes in the GGUF file layout (a 2-D
 * tensor has n_mats = 1; a 3-D MoE expert tensor [n_mats][rows][cols] has n_mats = n_expert).
 * The copy is synchronous; the device copy is re-laid out for the kernels (rows interleaved in
 * groups of 8, as the reference's CPU repack does, fastgguf.c:2237-2282). Returns FGH_SKIP_TYPE /
 * FGH_SKIP_MEM like the reference's n_skip_type / n_skip_mem paths, with *out = NULL. */
FGH_API int fgh_upload(fgh_ctx *ctx, uint32_t ggml_type, int64_t cols, int64_t rows, int64_t n_mats,
               int order, const void *host_data, uint64_t nbytes, fgh_tensor **out);
FGH_API void fgh_tensor_free(fgh_tensor *t);

/* ---- GGUF files: replaces gguf_open (fastgguf.c:342-440), kv_num (441-448) and tensor_find
 * (450-454); fgh_upload_gguf is gpu_upload_tensor (2060-2081) on a tensor of the mapped file ----
 * fgh_gguf_open maps the file read-only and parses its header, metadata and tensor table with the
 * reference's rules (magic, general.alignment, block sizes, bounds); it needs no device. On
 * failure it returns a negative status, *out = NULL, and a message in err (err_len bytes; err may
 * be NULL). A tensor info holds the reference's tensor_t fields: name, type, dims (ne[0] = cols,
 * the reduction; ne[1] = rows; ne[2] = experts of a 3-D MoE tensor), the byte offset of its data
 * from the start of the file, and its byte count. fgh_gguf_find returns a tensor's index or -1;
 * fgh_gguf_kv_num gives a numeric entry (or the first element of an integer array), else def;
 * fgh_gguf_kv_str a string entry or NULL; fgh_gguf_data a tensor's bytes in the mapping (valid
 * until fgh_gguf_close). fgh_upload_gguf uploads tensor `index` as fgh_upload would its bytes,
 * with cols = ne[0], rows = ne[1] and n_mats = the product of the higher dims. */
typedef struct fgh_gguf fgh_gguf;
typedef struct {
    char name[128];
    uint32_t type;
    int32_t n_dims;
    uint64_t ne[4];
    uint64_t offset;
    uint64_t nbytes;
} fgh_gguf_tensor_info;
FGH_API int fgh_gguf_open(const char *path, fgh_gguf **out, char *err, size_t err_len);
FGH_API void fgh_gguf_close(fgh_gguf *g);
FGH_API int fgh_gguf_summary(const fgh_gguf *g, uint32_t *version, uint64_t *alignment, int64_t *n_kvs,
                             int64_t *n_tensors);
FGH_API int fgh_gguf_tensor(const fgh_gguf *g, int64_t index, fgh_gguf_tensor_info *out);
FGH_API int64_t fgh_gguf_find(const fgh_gguf *g, const char *name);
FGH_API int fgh_gguf_kv_num(const fgh_gguf *g, const char *key, double def, double *out);
FGH_API const char *fgh_gguf_kv_str(const fgh_gguf *g, const char *key);
FGH_API const void *fgh_gguf_data(const fgh_gguf *g, int64_t index);
FGH_API int fgh_upload_gguf(fgh_ctx *ctx, const fgh_gguf *g, int64_t index, int order, fgh_tensor **out);

/* ---- matvec: replaces fg_gpu_matvec (fastgguf.c:2114) and the CPU matvec (2575) ----
 * y[r] = dot(W[r], Q8(x)) for all rows of all matrices (rows * n_mats outputs); x has cols
 * floats. Host pointers, synchronous. */
FGH_API int fgh_matvec(fgh_ctx *ctx, const fgh_tensor *t, const float *x, float *y);

/* ---- matvec_multi: replaces matvec_multi (fastgguf.c:2552) ----
 * n <= 4 tensors with the same cols read the same x, which is quantized once. */
FGH_API int fgh_matvec_multi(fgh_ctx *ctx, int n, const fgh_tensor *const *t, const float *x, float *const *y);

/* ---- matmul: replaces matmul (fastgguf.c:3004) for nb <= 64 tokens ----
 * Y[tok * ldy + r] = dot(W[r], Q8(X[tok * ldx ...])). nb >= 8 runs the int8 MFMA prompt GEMM
 * (the role of gemm_kquant 2818 / gemm_q32 2981); nb < 8 runs the decode kernel per token, as the
 * reference does for repacked tensors (3006-3009). */
FGH_API int fgh_matmul(fgh_ctx *ctx, const fgh_tensor *t, const float *X, int ldx, float *Y, int ldy, int nb);

/* ---- MoE FFN: replaces moe_ffn (fastgguf.c:4588) for n_tok tokens ----
 * gate, up: 3-D tensors [n_expert][ff][n_embd]; down: [n_expert][n_embd][ff].
 * logits: [n_tok][n_expert] router outputs (the reference's matvec(ffn_gate_inp), 4593).
 * X, Y: [n_tok][n_embd]. Each token is routed independently (softmax, top-k, renormalise,
 * 4594-4604); tokens are grouped by expert on the device. sel_out / w_out ([n_tok][k], optional,
 * may be NULL) receive the selected experts and their weights. */
FGH_API int fgh_moe_ffn(fgh_ctx *ctx, const fgh_tensor *gate, const fgh_tensor *up, const fgh_tensor *down,
                int k, const float *logits, const float *X, float *Y, int n_tok,
                int32_t *sel_out, float *w_out);

/* ---- attention: replaces attn_rows (fastgguf.c:3273-3326), both of its paths ----
 * Rows are (token, head) pairs, row t * n_head + h: q and o are [n_tok][n_head][hd]; the K and V
 * caches are rings of cap rows of kv_dim floats (position p in row p % cap), head h reading the
 * cache columns (h / (n_head / n_head_kv)) * hd .. + hd (the GQA grouping of forward, 4770-4790).
 * Token t attends to positions st[t]..en[t] (1 <= en - st + 1 <= cap). Every output equals the
 * reference's bit for bit: scores as att_qk_kern's lane chains and hsum4_ps (3227-3246), softmax
 * as softmax_vec (3194-3219, exp_neg_ps 3168-3184 on whole groups of 8, libm expf on the tail),
 * value sums as att_v_kern's chain over the positions in order (3249-3270). Head sizes that are
 * not a multiple of 32 take the reference's per-row path (3313-3325): scores as dot_f32v
 * (1618-1632), then the same softmax and value sums. scale is the reference's 1/sqrt(hd).
 * Requires 1 <= hd <= 256, n_head % n_head_kv == 0, n_head_kv * hd <= kv_dim; for hd % 32 == 0
 * also kv_dim % 4 == 0 and 16-byte aligned device pointers (4-byte aligned otherwise). */
FGH_API int fgh_attention(fgh_ctx *ctx, int n_tok, int n_head, int n_head_kv, int hd, const float *q, float *o,
                  const float *k_cache, const float *v_cache, int kv_dim, int cap, const int32_t *st,
                  const int32_t *en, float scale);

/* ---- device-resident variants: device pointers, asynchronous on the context stream ----
 * These skip the host<->device copies of the synchronous calls above (the copies fastgguf.c
 * makes at 2102 and 2110), for callers that keep activations in device memory. */
FGH_API int fgh_matvec_dev(fgh_ctx *ctx, const fgh_tensor *t, const float *x_dev, float *y_dev);
FGH_API int fgh_matvec_multi_dev(fgh_ctx *ctx, int n, const fgh_tensor *const *t, const float *x_dev,
                         float *const *y_dev);
/* The dense SiLU FFN's down projection, y = t * Q8(h) with h[i] = silu(g[i]) * u[i] (g, u: the
 * gate and up outputs, t->cols values each): replaces forward's loop
 * `gate[i] = silu_f(gate[i]) * up[i]` followed by matvec(ffn_down, gate) (4874-4877, silu_f
 * 3118): one short launch forms h in the context's scratch (t->cols floats; like all scratch, it
 * must have its size from an eager call before a graph capture uses it), then the matvec. Same
 * results bit for bit as that loop followed by fgh_matvec_dev. */
FGH_API int fgh_matvec_silu_dev(fgh_ctx *ctx, const fgh_tensor *t, const float *g_dev, const float *u_dev,
                        float *y_dev);
/* The dense SiLU FFN's gate and up projections and the loop between them and the down
 * projection: h[i] = silu_f(gate[i] . Q(x)) * (up[i] . Q(x)) (forward 4870-4876: matvec_multi of
 * ffn_gate and ffn_up, then `gate[i] = silu_f(gate[i]) * up[i]`), gate->rows values to h_dev;
 * gate and up: single matrices of one shape. Q4_K / Q5_K tensors of one type and order take one
 * launch (a workgroup holds gate and up tiles of the same rows, so g and u are never stored);
 * other types run the matvecs, then a short silu launch (with the context's scratch, which must
 * have its size from an eager call before a graph capture uses it). Same results bit for bit as
 * fgh_matvec_multi_dev followed by that loop; h_dev then feeds fgh_matvec_dev(ffn_down). */
FGH_API int fgh_matvec_gate_up_silu_dev(fgh_ctx *ctx, const fgh_tensor *gate, const fgh_tensor *up,
                                const float *x_dev, float *h_dev);
/* The dense SiLU FFN of one token: replaces forward's matvec_multi(ffn_gate, ffn_up), the loop
 * `gate[i] = silu_f(gate[i]) * up[i]` and matvec(ffn_down, gate) (4870-4877): h_dev receives
 * gate->rows values of h, y_dev down->rows outputs, bit for bit fgh_matvec_gate_up_silu_dev
 * followed by fgh_matvec_dev(down, h_dev, y_dev), which is what it runs (two launches for Q4_K /
 * Q5_K gate and up of one type and order). down: one matrix with gate->rows columns. */
FGH_API int fgh_ffn_dev(fgh_ctx *ctx, const fgh_tensor *gate, const fgh_tensor *up, const fgh_tensor *down,
                        const float *x_dev, float *h_dev, float *y_dev);
FGH_API int fgh_matmul_dev(fgh_ctx *ctx, const fgh_tensor *t, const float *X_dev, int ldx, float *Y_dev,
                   int ldy, int nb);
/* fgh_matmul_dev without any device allocation. No counterpart in the reference: it is for
 * callers that cannot allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). From nb >= 8 tokens the prompt GEMM's scratch goes to a static device
 * array of FGH_NOALLOC_SCRATCH_BYTES per device, held until the process ends (under 8 tokens the
 * decode kernels run and need none). Its size per type, Tp = nb rounded up to 16 (Q8_0: 32 or 64):
 *   Q4_K, Q6_K  (256-blocks + 1) * 292 * Tp bytes of activation records;
 *   Q8_0        (steps + KH) * 144 * Tp bytes of records, steps = ceil(32-blocks / 4), KH = 4
 *               from 4 steps (2 for 2-3 steps, 1 for one);
 *   Q4_0, Q4_1, Q5_0, Q5_1  (Tp / 16) * ceil(32-blocks / 4) * 2560 bytes of records;
 * and for Q4_K, Q6_K and Q8_0 tensors with few 64-row groups (ks >= 2 K splits fit beside them on
 * the compute units, as for a 14336 -> 4096 down projection) the split's counters, 4 bytes per
 * group rounded to 256, and partials of ks * groups * 64 * Tp * 4 bytes, at most 4 MiB on 256
 * compute units. At 64 tokens that holds every K the upload accepts when the GEMM does not split,
 * and, with a split, Q4_K and Q6_K K <= 57088 (223 blocks) and Q8_0 K <= 57728 (1804 blocks). A
 * call that would need more fails with FGH_ERR_ARG before it launches anything. Every call on a
 * device shares that device's array: calls that overlap on one device (several streams or
 * contexts) race. Nothing in the array needs to start at zero; each call writes what it reads
 * (the split's counters are zeroed by the call's own first launch). Same results bit for bit as
 * fgh_matmul_dev. */
#define FGH_NOALLOC_SCRATCH_BYTES (8u << 20)
FGH_API int fgh_matmul_dev_noalloc(fgh_ctx *ctx, const fgh_tensor *t, const float *X_dev, int ldx,
                           float *Y_dev, int ldy, int nb);
FGH_API int fgh_moe_ffn_dev(fgh_ctx *ctx, const fgh_tensor *gate, const fgh_tensor *up,
                    const fgh_tensor *down, int k, const float *logits_dev, const float *X_dev,
                    float *Y_dev, int n_tok);
/* fgh_attention on device pointers (st_dev, en_dev: int32 [n_tok] in device memory). max_len
 * bounds every row's length en - st + 1 (it sizes the score buffer): a row whose range is empty,
 * longer than cap or than max_len gets NaN outputs, not an error, since the ranges stay on the
 * device. */
FGH_API int fgh_attention_dev(fgh_ctx *ctx, int n_tok, int n_head, int n_head_kv, int hd, const float *q_dev,
                      float *o_dev, const float *k_cache_dev, const float *v_cache_dev, int kv_dim, int cap,
                      const int32_t *st_dev, const int32_t *en_dev, int max_len, float scale);

/* ---- TurboQuant KV cache: replaces kvq_rotate / kvq_quant_slice (fastgguf.c:3341-3444) at the
 * cache write (forward 4726-4735) and the attention step over the quantized cache (4760-4846:
 * q rotated, kvq_dot_k 3447-3462, softmax_inplace 3147-3156, kvq_axpy_v 3465-3489, the output
 * rotated back). A cache is cap slots; slot p % cap holds n_head_kv records of
 * 4 + hd * bits / 8 bytes (float scale, then the codes) back to back, the reference's layout
 * (KVQ_REC, 3361). hd a power of 2 from 32 to 256; K bits 4 or 8, V bits 2, 4 or 8. Outputs equal
 * the reference's bit for bit. */
/* k_dev, v_dev: [n_tok][stride] new K / V rows; pos_dev: int32 [n_tok] their positions. */
FGH_API int fgh_kvq_store_dev(fgh_ctx *ctx, int n_tok, int n_head_kv, int hd, int kbits, int vbits,
                      const float *k_dev, const float *v_dev, int stride, uint8_t *kq_dev, uint8_t *vq_dev,
                      int cap, const int32_t *pos_dev);
/* q_dev, o_dev: [n_tok][n_head][hd], unrotated; ranges and NaN rows as fgh_attention_dev. */
FGH_API int fgh_kvq_attention_dev(fgh_ctx *ctx, int n_tok, int n_head, int n_head_kv, int hd, int kbits, int vbits,
                          const float *q_dev, float *o_dev, const uint8_t *kq_dev, const uint8_t *vq_dev,
                          int cap, const int32_t *st_dev, const int32_t *en_dev, int max_len, float scale);

/* ---- HIP graphs of device-resident calls (launch-bound decode loops) ----
 * fgh_graph_begin starts capturing the context stream; the *_dev calls that follow are recorded,
 * not run; fgh_graph_end instantiates them as one executable graph that fgh_graph_launch replays
 * on the context stream. While capturing, calls that would allocate or synchronize fail with
 * FGH_ERR. No entry point records a memset, so replays are safe to repeat. */
FGH_API int fgh_graph_begin(fgh_ctx *ctx);
FGH_API int fgh_graph_end(fgh_ctx *ctx, void **graph);
FGH_API int fgh_graph_launch(fgh_ctx *ctx, void *graph);
FGH_API int fgh_graph_destroy(fgh_ctx *ctx, void *graph);

/* ---- device memory, stream and timing helpers (for device-resident callers and benchmarks) */
FGH_API int fgh_dev_alloc(fgh_ctx *ctx, uint64_t bytes, void **ptr);
FGH_API int fgh_dev_free(fgh_ctx *ctx, void *ptr);
FGH_API int fgh_copy_h2d(fgh_ctx *ctx, void *dst_dev, const void *src_host, uint64_t bytes);
FGH_API int fgh_copy_d2h(fgh_ctx *ctx, void *dst_host, const void *src_dev, uint64_t bytes);
/* device-to-device copy by a plain streaming kernel (16-byte loads and stores), asynchronous on
 * the context stream; bytes % 16 == 0. Also the known-size kernel that calibrates HBM counters. */
FGH_API int fgh_copy_d2d(fgh_ctx *ctx, void *dst_dev, const void *src_dev, uint64_t bytes);
/* wrapping 32-bit sum of the little-endian 32-bit words of a device buffer (bytes % 16 == 0),
 * written to *out_dev (device memory), asynchronous on the context stream: an integrity check of
 * uploaded or copied data, and the plain streaming-read kernel that gives the read rate a
 * matvec's weight stream is compared against: each workgroup streams one contiguous share with
 * nontemporal 16-byte loads, the fastest read form measured on MI355X (out_dev == NULL: only the
 * streaming pass runs, its per-workgroup parts stay in the context). No counterpart in the
 * reference (device-side helper).
 * The first call allocates a small part buffer: make it once before graph capture. */
FGH_API int fgh_checksum_dev(fgh_ctx *ctx, const void *src_dev, uint64_t bytes, uint32_t *out_dev);
/* device-to-device copy by the HIP runtime (hipMemcpyAsync on the context stream): the runtime's
 * own copy rate, an independent figure beside fgh_checksum_dev's read rate. No counterpart in the
 * reference. */
FGH_API int fgh_memcpy_dev(fgh_ctx *ctx, void *dst_dev, const void *src_dev, uint64_t bytes);
/* The int8 MFMA rate this device delivers to a kernel that runs nothing but MFMA: one launch, on
 * the context stream, of 8 independent v_mfma_i32_16x16x64_i8 chains per wavefront for `iters`
 * rounds over two 4-wavefront workgroups per compute unit (no memory traffic); *ops receives the
 * int8 operations (2 per multiply-add) the launch performs, to divide by its timed duration. The
 * attainable peak the prompt GEMM is compared against, beside the published one. No counterpart
 * in the reference. Shares the small part buffer of fgh_checksum_dev (make one call before a
 * graph capture). */
FGH_API int fgh_mfma_peak_dev(fgh_ctx *ctx, int iters, uint64_t *ops);
FGH_API int fgh_sync(fgh_ctx *ctx);
/* HIP events recorded on the context stream */
FGH_API int fgh_event_create(fgh_ctx *ctx, void **ev);
FGH_API int fgh_event_record(fgh_ctx *ctx, void *ev);
FGH_API int fgh_event_elapsed_ms(fgh_ctx *ctx, void *ev_start, void *ev_stop, float *ms);
FGH_API int fgh_event_destroy(fgh_ctx *ctx, void *ev);

/* ---- test hooks (bit-exactness checks; not needed by a production caller) ----
 * fgh_quantize: the device quantizer's output in the reference struct layout (kind FGH_ACT_Q8:
 * n/32 blocks of 40 bytes; FGH_ACT_Q8K: n/256 blocks of 292 bytes), from host x.
 * fgh_block_ints: per (row, block) integer parts of dot(W[r], Q8(x)) as the device kernels
 * compute them: sumi / msum [rows * n_mats][blocks per row] (see the oracle's fgo_block_ints);
 * FGH_ERR_ARG for the float types, which have none.
 * fgh_gemm_block_ints: the same integers as the prompt GEMMs (Q4_K, Q6_K, Q8_0, Q4_0, Q4_1, Q5_0
 * or Q5_1, nb tokens, 8..64) compute them: sumi / msum [nb][rows * n_mats][blocks per row], token t
 * from row t of X (stride ldx). The 32-value types have msum zeros; for Q4_0 / Q4_1 / Q5_0 / Q5_1
 * sumi is gemm_q32's integer over the unsigned weights (nibble or 5-bit value) times the quants
 * (fastgguf.c:2876-2894, 2919-2931), i.e. fgh_block_ints' sumi plus 8 (Q4_0) or 16 (Q5_0) times
 * the block's quant sum.
 * fgh_fp16_to_f32: the device's fp16 -> fp32 decode of n codes.
 * fgh_expf: the device's expf (the MoE softmax and silu) of n values.
 * fgh_matvec_shape: the launch shape a decode launch of `type` (order as fgh_upload resolved it)
 * over row_tiles row tiles of all its tensors (16 rows per tile for Q4_K / Q5_K / Q2_K / Q3_K /
 * IQ4_XS, 4 for F32, 8 for F16, 64 for BF16, 8 otherwise) and ntok tokens picks: shape[0]
 * wavefronts per tile, [1] ring depth, [2]
 * tiles per workgroup, [3]
 * LDS bytes. Lets the tests run every kernel instantiation the launchers can choose. */
FGH_API int fgh_quantize(fgh_ctx *ctx, int kind, const float *x, int n, void *out_blocks);
FGH_API int fgh_block_ints(fgh_ctx *ctx, const fgh_tensor *t, const float *x, int32_t *sumi, int32_t *msum);
FGH_API int fgh_gemm_block_ints(fgh_ctx *ctx, const fgh_tensor *t, const float *X, int ldx, int nb,
                                int32_t *sumi, int32_t *msum);
/* fgh_moe_block_ints: fgh_moe_ffn of n_tok >= 2 tokens over Q4_K row-order experts (the grouped
 * int8 MFMA path), returning the per (slot, row, block) integers its expert kernels formed: slot
 * t * k + j is token t's j-th selected expert; gate_* [n_tok * k][ff][gate blocks] are gate's
 * sumi / msum of Q8_K(x_t), down_* [n_tok * k][n_embd][down blocks] down's of Q8_K(h_tj)
 * (the oracle's fgo_block_ints of those rows and activations). */
FGH_API int fgh_moe_block_ints(fgh_ctx *ctx, const fgh_tensor *gate, const fgh_tensor *up, const fgh_tensor *down,
                               int k, const float *logits, const float *X, int n_tok, int32_t *gate_sumi,
                               int32_t *gate_msum, int32_t *down_sumi, int32_t *down_msum);
FGH_API int fgh_expf(fgh_ctx *ctx, const float *x, int n, float *out);
FGH_API int fgh_fp16_to_f32(fgh_ctx *ctx, const uint16_t *h, int n, float *out);
FGH_API int fgh_matvec_shape(fgh_ctx *ctx, uint32_t type, int order, int64_t cols, int64_t row_tiles, int ntok,
                             int32_t *shape);

#ifdef __cplusplus
}
#endif
#endif
