/*
 * fg_oracle.h - CPU restatement of fastgguf's quantized weight x Q8-activation kernels.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP backend in
 * fastgguf_amd/: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it. Nothing in the product path calls it, and the HIP backend never falls back to it.
 *
 * Every function restates one reference function (file:line into lawnak/FastGGUF fastgguf.c) and
 * reproduces the fp32 evaluation order of the reference's AVX2 / AVX-VNNI / AVX-512-VNNI builds,
 * lane by lane, so that results are bit-identical to the compiled reference.
 *
 * Activation block layouts are the reference's C structs (little-endian, no padding):
 *   q8_blk  (fastgguf.c:743) = { float d; int8 qs[32]; int16 s16[2]; }        40 bytes
 *   q8k_blk (fastgguf.c:771) = { float d; int8 qs[256]; int16 bsums[16]; }   292 bytes
 */
#ifndef FG_ORACLE_H
#define FG_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    FGO_T_F32 = 0, FGO_T_F16 = 1, FGO_T_BF16 = 30, FGO_T_Q4_0 = 2, FGO_T_Q4_1 = 3, FGO_T_Q5_0 = 6, FGO_T_Q5_1 = 7, FGO_T_Q8_0 = 8,
    FGO_T_Q2_K = 10, FGO_T_Q3_K = 11, FGO_T_Q4_K = 12, FGO_T_Q5_K = 13, FGO_T_Q6_K = 14, FGO_T_IQ4_NL = 20,
    FGO_T_IQ4_XS = 23
};

/* fp32 evaluation order a kernel follows (which reference kernel the call restates) */
enum {
    FGO_ORDER_ROW = 0,      /* dot_q4_K_q8k / dot_q6_K_q8k / dot_q8_0_q8 (file layout) */
    FGO_ORDER_REPACKED = 1, /* dot_q4Kx8 / dot_q40x8 (8-row repacked Q4_K / Q4_0, fastgguf.c:2322, 2424) */
};

typedef struct { float d; int8_t qs[32]; int16_t s16[2]; } fgo_q8_blk;
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } fgo_q8k_blk;

float fgo_fp16(uint16_t h);
void fgo_quantize_q8(const float *x, fgo_q8_blk *out, int n);
void fgo_quantize_q8k(const float *x, fgo_q8k_blk *out, int n);

float fgo_dot_q8_0(const uint8_t *row, const fgo_q8_blk *xq, int nb);
float fgo_dot_q4_K(const uint8_t *row, const fgo_q8k_blk *y, int nb);
float fgo_dot_q4_K_rp(const uint8_t *row, const fgo_q8k_blk *y, int nb);
float fgo_dot_q6_K(const uint8_t *row, const fgo_q8k_blk *y, int nb);
float fgo_dot_q5_0(const uint8_t *row, const fgo_q8_blk *xq, int nb);
float fgo_dot_q5_K(const uint8_t *row, const fgo_q8k_blk *y, int nb);
/* any 32-value type (Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, IQ4_NL) in its row kernel's order */
float fgo_dot_q32(uint32_t type, const uint8_t *row, const fgo_q8_blk *xq, int nb);
/* the 256-value types on Q8 activations (Q2_K, Q3_K, IQ4_XS); nb256 blocks of the row */
float fgo_dot_k256q8(uint32_t type, const uint8_t *row, const fgo_q8_blk *xq, int nb256);
float fgo_dot_q4_0_rp(const uint8_t *row, const fgo_q8_blk *xq, int nb);
/* the float types (F32, F16, BF16) on fp32 activations, n values of the row (dot_row 2207-2214) */
float fgo_dot_float(uint32_t type, const uint8_t *row, const float *x, int n);

/* per-block integer parts (the bit-exact targets):
 *   Q4_K, Q5_K: sumi[b] = sum_s sc_s * sum_32 q*y,   msum[b] = sum_s m_s * (bs_2s + bs_2s+1)
 *   Q6_K:       sumi[b] = sum_g sc_g * sum_16 q*y,   msum[b] = sum_g sc_g * bs_g  (q in 0..63)
 *   32-value types: sumi[b] = sum_32 w*x, msum[b] = 0, with w the int8 value the row kernel
 *   multiplies (Q5_0: q5 - 16, Q4_0: nib - 8, Q4_1: nib, Q5_1: q5, IQ4_NL: kvalues[nib]) */
void fgo_block_ints(uint32_t type, const uint8_t *row, const void *act, int nb,
                    int32_t *sumi, int32_t *msum);

/* y[r] = dot(W[r], Q8(x)) for r < rows: quantize once, then the row kernel (matvec 2575) */
int fgo_matvec(uint32_t type, int order, const uint8_t *w, int64_t rows, int cols,
               const float *x, float *y);

/* Y[t*ldy + r] for t < nb tokens, with the kernel choice of matmul (fastgguf.c:3004) */
int fgo_matmul(uint32_t type, int order, const uint8_t *w, int64_t rows, int cols,
               const float *X, int ldx, float *Y, int ldy, int nb);

/* the prompt GEMM on pre-quantized activations (gemm_kquant 2818 / gemm_q32 2981) */
int fgo_gemm(uint32_t type, const uint8_t *w, int64_t rows, int cols, const void *act,
             int act_stride_blocks, float *Y, int ldy, int nb);

/* moe_ffn (fastgguf.c:4588) for n_tok independent tokens, router logits given:
 *   logits [n_tok][n_expert], X [n_tok][n_embd], Y [n_tok][n_embd]
 *   gate/up: [n_expert][ff][n_embd] expert rows, down: [n_expert][n_embd][ff]
 *   sel_out [n_tok][k] and w_out [n_tok][k] (optional, may be NULL) receive the routing.
 *   h_out [n_tok][k][ff] (optional) receives silu(gate)*up before its quantization. */
int fgo_moe_ffn(uint32_t type_gate, uint32_t type_up, uint32_t type_down,
                const uint8_t *gate, const uint8_t *up, const uint8_t *down,
                int n_expert, int k, int n_embd, int ff, const float *logits,
                const float *X, float *Y, int n_tok, int32_t *sel_out, float *w_out,
                float *h_out);

/* the MoE down-projection stage alone, with h given: out = sum_j w_j * dot(down_j, Q8K(h_j)) */
int fgo_moe_down(uint32_t type_down, const uint8_t *down, int n_embd, int ff, int k,
                 const int32_t *sel, const float *w, const float *h, float *out);

/* attention over an fp32 ring cache, attn_rows (fastgguf.c:3273-3326) restated row by row: row r
 * (q + r*hd -> o + r*hd) over positions st[r]..en[r] (slot p % cap) of the cache rows of kv_dim
 * floats at offset kvo[r]; hd % 32 == 0 (the reference's vector path). fgo_exp_neg is its
 * exp_neg_ps (3168-3184) on one value. */
int fgo_attn_rows(int nr, const float *q, float *o, const int *st, const int *en, const float *ck, const float *cv,
                  int kv_dim, const int *kvo, int cap, int hd, float scale);
float fgo_exp_neg(float x);

/* TurboQuant KV cache (fastgguf.c:3341-3513, forward 4760-4846): the rotation's signs, the
 * rotation (inverse = 1: its inverse), slice records of fgo_kvq_rec_bytes(hd, bits) bytes, and
 * attention rows over quantized ring caches (kq / vq: cap slots of kqs / vqs bytes; row r reads
 * K / V head kvh[r]; q unrotated, o unrotated). hd a power of 2 up to 1024. */
void fgo_kvq_signs(float *out, int n);
int fgo_kvq_rotate(float *x, int n, int inverse);
int fgo_kvq_rec_bytes(int hd, int bits);
int fgo_kvq_quant(const float *x, int hd, uint8_t *rec, int bits);
int fgo_kvq_attn_rows(int nr, const float *q, float *o, const int *st, const int *en, const uint8_t *kq,
                      const uint8_t *vq, int kqs, int vqs, const int *kvh, int cap, int hd, int kbits, int vbits,
                      float scale);

/* reference order for the router: softmax (3147), top-k by argmax (3328), renormalise (4603) */
void fgo_moe_route(const float *logits, int n_expert, int k, int32_t *sel, float *w);

/* silu_f (fastgguf.c:3118) with the C library's expf */
float fgo_silu(float x);

/* expf restated from its published method (ARM optimized-routines, glibc >= 2.27), as the GPU
 * backend computes it. fgo_expf_compare counts the float inputs x (every stride-th bit pattern of
 * [lo, hi]) where it differs from this libm's expf, and the largest difference in ulps; the
 * reference's softmax and silu call expf (fastgguf.c:3118, 3151). */
float fgo_expf_restated(float x);
void fgo_expf_n(const float *x, int n, float *out); /* this libm's expf of n values */
uint64_t fgo_expf_compare(float lo, float hi, uint32_t stride, uint64_t *n_checked, int *max_ulp);

/* dequantize_row (fastgguf.c:475-727) for every type here: textbook value decode */
int fgo_dequantize_row(uint32_t type, const uint8_t *raw, float *out, int n);

/* block geometry: elements and bytes per block (block_size_of, fastgguf.c:235) */
int fgo_block_size(uint32_t type, int *elems, int *bytes);

#ifdef __cplusplus
}
#endif
#endif
