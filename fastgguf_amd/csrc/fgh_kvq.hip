// fgh_kvq.hip - the TurboQuant KV cache on gfx950 (fastgguf.c:3341-3513 and forward's attention
// step over it, 4726-4735 and 4760-4846), bit-exact with the compiled reference.
//
// Records: one per (slot, K / V head), KVQ_REC = 4 + hd * bits / 8 bytes: the float scale, then
// the codes (8 bits: int8; 4 bits: low nibble first; 2 bits: low bits first). A slot holds the
// n_head_kv records of one position back to back. The rotation R x = H(D x) / sqrt(hd) (signs D
// of xorshift64*, kvq_init 3363-3372; butterflies kvq_fwht 3375-3386) is done in LDS, one
// butterfly per thread per stage, so every value sees the reference's additions.
//
// Attention (hd a power of 2, 32..256):
//   q rows rotated (4763)                                    kvq_rotate_kernel
//   scores: kvq_dot_k (3447-3462) times scale, per key       kvq_scores_kernel
//   softmax_inplace (3147-3156), then w' = w * s_V(p)         kvq_softmax_kernel
//   o = fma(w', centroid, o) over the positions in order     attn_values (fgh_attn.hip), which
//                                                            decodes the V codes as it stages them
//   output rows rotated back (4846)                           kvq_rotate_kernel
// kvq_axpy_v (3465-3489) adds fma(w * s, value, o) for each position with w != 0; w' = w * s is
// that product, and a position with w = 0 gets w' = 0 (not 0 * s, which an inf or NaN scale would
// turn into NaN) and adds fma(0, centroid, o) = o, so the value chains of the fp32 attention give
// its sums. No fp32 copy of the cache is made.
#include <hip/hip_runtime.h>

#include "fgh_internal.h"

namespace fgh {

namespace {

struct SignTable {
    float v[1024];
    constexpr SignTable() : v() {
        uint64_t s = 0x243F6A8885A308D3ULL;
        for (int i = 0; i < 1024; ++i) {
            uint64_t x = s;
            x ^= x >> 12;
            x ^= x << 25;
            x ^= x >> 27;
            s = x;
            v[i] = ((x * 0x2545F4914F6CDD1DULL) >> 63) ? 1.0f : -1.0f;
        }
    }
};
__constant__ SignTable kvq_sign = SignTable();

// Lloyd-Max centroids of N(0, 1) (kvq_c4 / kvq_c2, 3356-3359) and the midpoints between
// neighbours, in float as kvq_enc4 / kvq_enc2 form them
__constant__ float kvq_c4[16] = {-2.7326f, -2.0690f, -1.6181f, -1.2562f, -0.9424f, -0.6568f, -0.3881f, -0.1284f,
                                 0.1284f,  0.3881f,  0.6568f,  0.9424f,  1.2562f,  1.6181f,  2.0690f,  2.7326f};
__constant__ float kvq_c2[4] = {-1.5104f, -0.4528f, 0.4528f, 1.5104f};

__device__ __forceinline__ int64_t slot_of(int p, int cap) { return (int64_t)(((p % cap) + cap) % cap); }

// the rotation (or its inverse) of x[0..hd) in LDS; 256 threads, all of them call it
__device__ void rotate_lds(float *x, int hd, bool inverse) {
    const int tid = threadIdx.x;
    if (!inverse)
        for (int i = tid; i < hd; i += 256) x[i] = x[i] * kvq_sign.v[i];
    __syncthreads();
    for (int len = 1; len < hd; len <<= 1) {
        for (int t = tid; t < hd / 2; t += 256) {
            const int i = (t / len) * 2 * len + (t % len);
            const float a = x[i], b = x[i + len];
            x[i] = a + b;
            x[i + len] = a - b;
        }
        __syncthreads();
    }
    const float inv = 1.0f / sqrtf((float)hd);
    for (int i = tid; i < hd; i += 256) x[i] = inverse ? x[i] * inv * kvq_sign.v[i] : x[i] * inv;
    __syncthreads();
}

__device__ __forceinline__ uint32_t code4(float u) {
    uint32_t c = 0;
    while (c < 15 && u > (kvq_c4[c] + kvq_c4[c + 1]) * 0.5f) ++c;
    return c;
}
__device__ __forceinline__ uint32_t code2(float u) {
    uint32_t c = 0;
    while (c < 3 && u > (kvq_c2[c] + kvq_c2[c + 1]) * 0.5f) ++c;
    return c;
}

// store: grid (tokens, K / V heads, 2: K then V), 256 threads. Rotates the head slice of the
// token's new K or V row and writes its record into slot pos % cap (kvq_quant_slice 3415-3444).
// The reference writes token after token: where two tokens of a call share a slot, only the
// later one writes.
__global__ __launch_bounds__(256) void kvq_store_kernel(KvqStoreArgs a, int n_tok) {
    __shared__ float x[256];
    __shared__ float sc[2];
    const int tok = blockIdx.x, kh = blockIdx.y, isv = blockIdx.z, tid = threadIdx.x, hd = a.hd;
    const int64_t my_slot = slot_of(a.pos[tok], a.cap);
    bool later = false;
    for (int t = tok + 1 + tid; t < n_tok; t += 256) later |= slot_of(a.pos[t], a.cap) == my_slot;
    if (__syncthreads_or(later)) return;  // the whole workgroup
    const int bits = isv ? a.vbits : a.kbits;
    const float *src = (isv ? a.v : a.k) + (size_t)tok * a.stride + (size_t)kh * hd;
    for (int i = tid; i < hd; i += 256) x[i] = src[i];
    __syncthreads();
    rotate_lds(x, hd, false);
    if (tid == 0) {
        float s;
        if (bits == 8) {
            float amax = 0.0f;
            for (int i = 0; i < hd; ++i) amax = fmaxf(amax, fabsf(x[i]));
            s = amax / 127.0f;
        } else {
            float ss = 0.0f;
            for (int i = 0; i < hd; ++i) ss = ss + x[i] * x[i];
            s = sqrtf(ss / (float)hd);
        }
        sc[0] = s;
        sc[1] = s > 0.0f ? 1.0f / s : 0.0f;
    }
    __syncthreads();
    const float inv = sc[1];
    const int rec = 4 + hd * bits / 8;
    uint8_t *dst = (isv ? a.vq : a.kq) + my_slot * (int64_t)(a.n_head_kv * rec) + (int64_t)kh * rec;
    if (tid == 0) *(float *)dst = sc[0];
    uint32_t *words = (uint32_t *)(dst + 4);
    const int per = 32 / bits;  // codes per 32-bit word
    for (int w = tid; w < hd / per; w += 256) {
        uint32_t v = 0;
        for (int j = 0; j < per; ++j) {
            const float u = x[w * per + j] * inv;
            const uint32_t c = bits == 8 ? (uint32_t)(uint8_t)(int8_t)(int)rintf(u) : bits == 4 ? code4(u) : code2(u);
            v |= c << (bits * j);
        }
        words[w] = v;
    }
}

// rows of hd values rotated (inverse = false) or rotated back: one workgroup per row
__global__ __launch_bounds__(256) void kvq_rotate_kernel(const float *in, float *out, int hd, bool inverse) {
    __shared__ float x[256];
    const size_t base = (size_t)blockIdx.x * hd;
    for (int i = threadIdx.x; i < hd; i += 256) x[i] = in[base + i];
    __syncthreads();
    rotate_lds(x, hd, inverse);
    for (int i = threadIdx.x; i < hd; i += 256) out[base + i] = x[i];
}

__device__ __forceinline__ int kvq_row_len(const KvqAttnArgs &a, int tok) {
    const int n = a.en[tok] - a.st[tok] + 1;
    return n >= 1 && n <= a.cap && n <= a.max_len ? n : 0;
}

// Groups of R rows that read one K / V head kh: j = R q .. R q + R - 1 of the head's n_tok * G
// rows, j = t * G + g (token t, query head kh * G + g); the scores of a group run over the union
// of its rows' ranges and are stored for each row's own range.
struct KvqRow {
    int row, st, en;  // row = -1: no such row; en < st: no valid range
};
__device__ __forceinline__ KvqRow kvq_group_row(const KvqAttnArgs &a, int n_tok, int R, int grp, int kh, int r) {
    const int G = a.n_head / a.n_head_kv, j = grp * R + r;
    KvqRow g{-1, 0, -1};
    if (j < n_tok * G) {
        const int t = j / G;
        g.row = t * a.n_head + kh * G + (j - t * G);
        if (kvq_row_len(a, t) > 0) {
            g.st = a.st[t];
            g.en = a.en[t];
        }
    }
    return g;
}

// scores: grid (key blocks, groups of R rows, K / V heads), 256 threads; thread = one key of the
// group's union for its R rows: each record's codes are loaded and looked up once for R chains
// in kvq_dot_k's order, then times s, times scale. R = 16 for prompt batches.
template <int R>
__global__ __launch_bounds__(256) void kvq_scores_kernel(KvqAttnArgs a, int n_tok) {
    __shared__ float q[R][256];
    __shared__ float c4[16];
    const int grp = blockIdx.y, kh = blockIdx.z, tid = threadIdx.x, hd = a.hd;
    int lo = 0x7fffffff, hi = -0x7fffffff;
    for (int r = 0; r < R; ++r) {
        const KvqRow g = kvq_group_row(a, n_tok, R, grp, kh, r);
        if (g.en >= g.st) {
            lo = min(lo, g.st);
            hi = max(hi, g.en);
        }
    }
    if (hi < lo) return;
    for (int i = tid; i < R * hd; i += 256) {
        const int r = i / hd, x = i - r * hd;
        const KvqRow g = kvq_group_row(a, n_tok, R, grp, kh, r);
        q[r][x] = g.en >= g.st ? a.qr[(size_t)g.row * hd + x] : 0.0f;
    }
    if (tid < 16) c4[tid] = kvq_c4[tid];
    __syncthreads();
    const int rec = 4 + hd * a.kbits / 8;
    for (int p = lo + (int)blockIdx.x * 256 + tid; p <= hi; p += (int)gridDim.x * 256) {
        const uint8_t *rp = a.kq + slot_of(p, a.cap) * (int64_t)(a.n_head_kv * rec) + (int64_t)kh * rec;
        const float s = *(const float *)rp;
        const uint32_t *w = (const uint32_t *)(rp + 4);
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.0f;
        if (a.kbits == 8) {
            for (int i = 0; i < hd; i += 4) {
                const uint32_t v = w[i / 4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float c = (float)(int8_t)(v >> (8 * j));
#pragma unroll
                    for (int r = 0; r < R; ++r) acc[r] = __builtin_fmaf(q[r][i + j], c, acc[r]);
                }
            }
        } else {
            for (int i = 0; i < hd; i += 8) {
                const uint32_t v = w[i / 8];
#pragma unroll
                for (int j = 0; j < 8; j += 2) {
                    const float clo = c4[(v >> (4 * j)) & 15], chi = c4[(v >> (4 * j + 4)) & 15];
#pragma unroll
                    for (int r = 0; r < R; ++r)
                        acc[r] = acc[r] + __builtin_fmaf(q[r][i + j], clo, q[r][i + j + 1] * chi);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const KvqRow g = kvq_group_row(a, n_tok, R, grp, kh, r);
            if (p >= g.st && p <= g.en) a.s[(size_t)g.row * a.max_len + (p - g.st)] = acc[r] * s * a.scale;
        }
    }
}

// softmax_inplace over each row's scores, then each weight times its position's V scale
constexpr int KVQ_RES = 12288;
__global__ __launch_bounds__(256) void kvq_softmax_kernel(KvqAttnArgs a) {
    extern __shared__ float e[];  // min(max_len, KVQ_RES) values: rows up to that length stay in LDS
    __shared__ float red[4];
    __shared__ float total;
    const int row = blockIdx.x, tok = row / a.n_head, h = row - tok * a.n_head, tid = threadIdx.x;
    const int n = kvq_row_len(a, tok);
    if (n == 0) return;
    float *s = a.s + (size_t)row * a.max_len;
    float mx = -__builtin_inff();
    for (int i = tid; i < n; i += 256) mx = fmaxf(mx, s[i]);
    for (int o = 1; o < 64; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const bool resident = n <= KVQ_RES;
    for (int i = tid; i < n; i += 256) {
        const float ev = expf_ref(s[i] - mx);
        if (resident) e[i] = ev;
        else s[i] = ev;
    }
    __syncthreads();
    if (tid == 0) {  // the sum in order: 32 values loaded ahead of their adds
        float sum = 0.0f;
        const float *src = resident ? e : s;
        int i = 0;
        for (; i + 32 <= n; i += 32) {
            float t[32];
#pragma unroll
            for (int u = 0; u < 32; ++u) t[u] = src[i + u];
#pragma unroll
            for (int u = 0; u < 32; ++u) sum += t[u];
        }
        for (; i < n; ++i) sum += src[i];
        total = sum;
    }
    __syncthreads();
    const float sum = total, inv = 1.0f / sum;
    const int kvh = h / (a.n_head / a.n_head_kv), rec = 4 + a.hd * a.vbits / 8;
    for (int i = tid; i < n; i += 256) {
        const float ev = resident ? e[i] : s[i];
        const float w = sum > 0.0f ? ev * inv : ev;
        const float sv =
            *(const float *)(a.vq + slot_of(a.st[tok] + i, a.cap) * (int64_t)(a.n_head_kv * rec) + (int64_t)kvh * rec);
        // kvq_axpy_v skips a zero weight (fastgguf.c:4829-4831): stored as 0, never 0 * s_V, so a V
        // record whose scale is inf or NaN adds nothing where the reference adds nothing
        s[i] = w == 0.0f ? 0.0f : w * sv;
    }
}

}  // namespace

hipError_t launch_kvq_store(const KvqStoreArgs &a, int n_tok, hipStream_t s) {
    if (n_tok < 1 || a.hd < 32 || a.hd > 256 || (a.hd & (a.hd - 1)) || (a.kbits != 4 && a.kbits != 8) ||
        (a.vbits != 2 && a.vbits != 4 && a.vbits != 8) || a.n_head_kv < 1 || a.n_head_kv > 65535)
        return hipErrorInvalidValue;
    kvq_store_kernel<<<dim3((unsigned)n_tok, (unsigned)a.n_head_kv, 2), 256, 0, s>>>(a, n_tok);
    return hipGetLastError();
}

hipError_t launch_kvq_attention(const KvqAttnArgs &a, int n_tok, hipStream_t s) {
    const int rows = n_tok * a.n_head;
    if (n_tok < 1 || a.hd < 32 || a.hd > 256 || (a.hd & (a.hd - 1)) || (a.kbits != 4 && a.kbits != 8) ||
        (a.vbits != 2 && a.vbits != 4 && a.vbits != 8) || a.n_head_kv < 1 || a.n_head % a.n_head_kv != 0 ||
        a.max_len < 1 || rows > 65535)
        return hipErrorInvalidValue;
    kvq_rotate_kernel<<<rows, 256, 0, s>>>(a.q, a.qr, a.hd, false);
    const int rows_kv = n_tok * (a.n_head / a.n_head_kv);
    const unsigned kb = (unsigned)std::min((a.max_len + 255) / 256, 1024);
    if (rows_kv >= 16)
        kvq_scores_kernel<16><<<dim3(kb, (unsigned)((rows_kv + 15) / 16), (unsigned)a.n_head_kv), 256, 0, s>>>(a, n_tok);
    else
        kvq_scores_kernel<4><<<dim3(kb, (unsigned)((rows_kv + 3) / 4), (unsigned)a.n_head_kv), 256, 0, s>>>(a, n_tok);
    kvq_softmax_kernel<<<rows, 256, (size_t)std::min(a.max_len, KVQ_RES) * 4, s>>>(a);
    AttnArgs v{nullptr, a.orot, nullptr, nullptr, a.s, a.st, a.en, a.n_head, a.n_head_kv, a.hd,
               a.n_head_kv * a.hd, a.cap, a.max_len, 1.0f};
    v.vq = a.vq;  // the value chains decode the V records' codes themselves
    v.vbits = a.vbits;
    hipError_t e = launch_attention_values(v, n_tok, s);
    if (e != hipSuccess) return e;
    kvq_rotate_kernel<<<rows, 256, 0, s>>>(a.orot, a.o, a.hd, true);
    return hipGetLastError();
}

}  // namespace fgh
