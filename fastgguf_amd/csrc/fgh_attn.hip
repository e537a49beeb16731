// fgh_attn.hip - attention over an fp32 KV ring cache on gfx950, bit-exact with the vector path of
// the reference's attn_rows (fastgguf.c:3273-3326; hd % 32 == 0).
//
// Rows are (token, head) pairs: row i = t * n_head + h reads q / writes o at i * hd and the K / V
// head (h / G) * hd of each cache row (G = n_head / n_head_kv, the GQA grouping of the reference's
// forward, 4770-4790), over the positions st[t]..en[t] (slot p % cap). Three launches:
//   scores   8 chains per key: chain l runs fma over q[8m + l] k[8m + l] (att_qk_kern,
//            3227-3246), then hsum4_ps's tree ((a0+a1)+(a2+a3))+((a4+a5)+(a6+a7)) (3187-3190),
//            times scale
//   softmax  one workgroup per row (softmax_vec, 3194-3219): the maximum, exp_neg_ps (3168-3184)
//            over whole groups of 8 and libm's expf over the tail, the sum as 8 ordered lane sums
//            (lane l over e[8g + l]) added in hsum_ps's tree then the tail in order, and every
//            value times 1 / sum
//   values   one lane per output element (att_v_kern, 3249-3270): acc = fma(w_p, v_p[c], acc)
//            over the positions in order
// The value sums are one dependent chain per (row, element) over every position: the
// reference's order, which no split over positions keeps. What bounds them is the latency of
// their operands, so the kernel keeps many tiles of V in flight per workgroup and runs the
// chains out of LDS. Head sizes up to 256; kv_dim and the cache pointers 16-byte aligned.
#include <hip/hip_runtime.h>

#include "fgh_internal.h"

namespace fgh {

// exp_neg_ps (fastgguf.c:3168-3184) on one value: Cephes polynomial after x = max(x, -87),
// fx = floor(x log2(e) + 0.5), and 0 for x <= -87
__device__ __forceinline__ float exp_neg_ref(float x) {
    const bool keep = x > -87.0f;
    x = x > -87.0f ? x : -87.0f;
    const float fx = floorf(__builtin_fmaf(x, 1.44269504088896341f, 0.5f));
    x = __builtin_fmaf(-fx, 0.693359375f, x);
    x = __builtin_fmaf(-fx, -2.12194440e-4f, x);
    float y = 1.9875691500E-4f;
    y = __builtin_fmaf(y, x, 1.3981999507E-3f);
    y = __builtin_fmaf(y, x, 8.3334519073E-3f);
    y = __builtin_fmaf(y, x, 4.1665795894E-2f);
    y = __builtin_fmaf(y, x, 1.6666665459E-1f);
    y = __builtin_fmaf(y, x, 5.0000001201E-1f);
    const float xx = x * x, x1 = x + 1.0f;
    y = __builtin_fmaf(y, xx, x1);
    const float e = __builtin_bit_cast(float, (uint32_t)((int)fx + 127) << 23);
    return keep ? y * e : 0.0f;
}

__device__ __forceinline__ float f_xor1(float v) { return __builtin_bit_cast(float, dpp_xor1(__builtin_bit_cast(int, v))); }
__device__ __forceinline__ float f_xor2(float v) { return __builtin_bit_cast(float, dpp_xor2(__builtin_bit_cast(int, v))); }

// the rows' ranges: n = en - st + 1, or 0 when the range is empty, longer than the cache or than
// the score buffer (such a row gets NaN outputs)
__device__ __forceinline__ int row_len(const AttnArgs &a, int tok) {
    const int n = a.en[tok] - a.st[tok] + 1;
    return n >= 1 && n <= a.cap && n <= a.max_len ? n : 0;
}
__device__ __forceinline__ int64_t kv_slot(int p, int cap) { return (int64_t)(((p % cap) + cap) % cap); }

// A group is 4 rows that read the same K / V head kh: group q of head kh holds j = 4q .. 4q + 3 of
// the head's n_tok * G rows, j = t * G + g (token t, query head kh * G + g). The scores and the
// value sums of a group run over the union lo..hi of its rows' ranges, as attn_rows runs its 4-row
// calls; a position outside a row's own range has weight 0, and fma(0, v, acc) = acc, so every
// row's sums are those of its own range.
struct GroupRow {
    int row, st, en;  // row = -1: no such row; en < st: no valid range
};
__device__ __forceinline__ GroupRow group_row(const AttnArgs &a, int n_tok, int grp, int kh, int r) {
    const int G = a.n_head / a.n_head_kv, j = grp * 4 + r;
    GroupRow g{-1, 0, -1};
    if (j < n_tok * G) {
        const int t = j / G;
        g.row = t * a.n_head + kh * G + (j - t * G);
        if (row_len(a, t) > 0) {
            g.st = a.st[t];
            g.en = a.en[t];
        }
    }
    return g;
}
__device__ __forceinline__ bool group_span(const AttnArgs &a, int n_tok, int grp, int kh, int &lo, int &hi) {
    lo = 0x7fffffff;
    hi = -0x7fffffff;
    for (int r = 0; r < 4; ++r) {
        const GroupRow g = group_row(a, n_tok, grp, kh, r);
        if (g.en >= g.st) {
            lo = min(lo, g.st);
            hi = max(hi, g.en);
        }
    }
    return hi >= lo;
}

// scores: grid (key blocks, groups, K heads), 256 threads; thread = one key of the union for the
// group's 4 rows, 8 lane chains per row over the head's values (2 x float4 of K per step), the q
// rows from LDS (one address for the whole wavefront: a broadcast read)
__global__ __launch_bounds__(256) void attn_scores_kernel(AttnArgs a, int n_tok) {
    __shared__ float4 qs[4][64];
    const int grp = blockIdx.y, kh = blockIdx.z, tid = threadIdx.x;
    int lo, hi;
    if (!group_span(a, n_tok, grp, kh, lo, hi)) return;
    GroupRow gr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) gr[r] = group_row(a, n_tok, grp, kh, r);
    const int h4 = a.hd / 4;
    for (int i = tid; i < 4 * h4; i += 256) {
        const int r = i / h4, x = i - r * h4;
        const GroupRow g = group_row(a, n_tok, grp, kh, r);
        qs[r][x] = g.en >= g.st ? ((const float4 *)(a.q + (size_t)g.row * a.hd))[x] : make_float4(0, 0, 0, 0);
    }
    __syncthreads();
    const int64_t kvo = (int64_t)kh * a.hd;
    for (int p = lo + (int)blockIdx.x * 256 + tid; p <= hi; p += (int)gridDim.x * 256) {
        const float4 *kp = (const float4 *)(a.k + kv_slot(p, a.cap) * a.kv_dim + kvo);
        float acc[4][8];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int l = 0; l < 8; ++l) acc[r][l] = 0.0f;
#pragma unroll 4
        for (int m = 0; m < a.hd / 8; ++m) {
            const float4 k0 = kp[2 * m], k1 = kp[2 * m + 1];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float4 q0 = qs[r][2 * m], q1 = qs[r][2 * m + 1];
                acc[r][0] = __builtin_fmaf(q0.x, k0.x, acc[r][0]);
                acc[r][1] = __builtin_fmaf(q0.y, k0.y, acc[r][1]);
                acc[r][2] = __builtin_fmaf(q0.z, k0.z, acc[r][2]);
                acc[r][3] = __builtin_fmaf(q0.w, k0.w, acc[r][3]);
                acc[r][4] = __builtin_fmaf(q1.x, k1.x, acc[r][4]);
                acc[r][5] = __builtin_fmaf(q1.y, k1.y, acc[r][5]);
                acc[r][6] = __builtin_fmaf(q1.z, k1.z, acc[r][6]);
                acc[r][7] = __builtin_fmaf(q1.w, k1.w, acc[r][7]);
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if (p >= gr[r].st && p <= gr[r].en) {
                const float t = ((acc[r][0] + acc[r][1]) + (acc[r][2] + acc[r][3])) +
                                ((acc[r][4] + acc[r][5]) + (acc[r][6] + acc[r][7]));
                a.s[(size_t)gr[r].row * a.max_len + (p - gr[r].st)] = t * a.scale;
            }
        }
    }
}

// softmax: one workgroup per row, in place over the row's scores, the exponentials staged in LDS
// 4096 at a time; lanes 0..7 of wavefront 0 carry the 8 ordered sums across the chunks
constexpr int SM_CHUNK = 4096;
__global__ __launch_bounds__(256) void attn_softmax_kernel(AttnArgs a) {
    __shared__ float e[SM_CHUNK];
    __shared__ float red[4];
    __shared__ float total;
    const int row = blockIdx.x, tok = row / a.n_head, tid = threadIdx.x;
    const int n = row_len(a, tok);
    if (n == 0) return;
    float *s = a.s + (size_t)row * a.max_len;
    float mx = -__builtin_inff();
    for (int i = tid; i < n; i += 256) mx = fmaxf(mx, s[i]);
    for (int o = 1; o < 64; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const int nv = n & ~7;  // whole groups of 8
    float v = 0.0f;
    for (int c0 = 0; c0 < n; c0 += SM_CHUNK) {
        const int cn = min(SM_CHUNK, n - c0);
        for (int i = tid; i < cn; i += 256) {
            const float x = s[c0 + i] - mx;
            const float ev = c0 + i < nv ? exp_neg_ref(x) : expf_ref(x);
            e[i] = ev;
            s[c0 + i] = ev;
        }
        __syncthreads();
        if (tid < 8) {
            const int ng = (min(c0 + cn, nv) - c0) / 8;
            int g = 0;
            for (; g + 8 <= ng; g += 8) {
                float t[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) t[u] = e[8 * (g + u) + tid];
#pragma unroll
                for (int u = 0; u < 8; ++u) v += t[u];
            }
            for (; g < ng; ++g) v += e[8 * g + tid];
            if (c0 + cn == n) {  // the last chunk holds the tail
                v = v + __shfl_xor(v, 4, 8);  // (v0 + v4), (v1 + v5), ...
                v = v + __shfl_xor(v, 1, 8);
                v = v + __shfl_xor(v, 2, 8);  // ((v0 + v4) + (v1 + v5)) + ((v2 + v6) + (v3 + v7))
                if (tid == 0) {
                    for (int i = nv; i < n; ++i) v += e[i - c0];
                    total = v;
                }
            }
        }
        __syncthreads();
    }
    const float sum = total;
    if (sum > 0.0f) {
        const float inv = 1.0f / sum;
        for (int i = tid; i < n; i += 256) s[i] = s[i] * inv;
    }
}

// values: grid (64-column chunks, groups, K heads), 256 threads. Lane (r, c) of wavefront w runs
// row r's chain for column 16 w + c of the chunk: acc = fma(w_p, v_p, acc) over the union in
// order. Tiles of 64 positions (V: 64 x 64 floats, weights: 4 x 64) are loaded by all 256
// threads S tiles ahead into registers, then stored to a double-buffered LDS tile (one barrier
// per tile): each chain takes its operands from LDS while S tiles of loads are in flight.
constexpr int AV_S = 6;
__global__ __launch_bounds__(256) void attn_values_kernel(AttnArgs a, int n_tok) {
    __shared__ float4 vt[2][64][16];
    __shared__ float4 wt[2][4][16];
    const int grp = blockIdx.y, kh = blockIdx.z, cc = (int)blockIdx.x * 64, tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int r = lane >> 4, c = wave * 16 + (lane & 15);
    const GroupRow me = group_row(a, n_tok, grp, kh, r);
    int lo, hi;
    if (!group_span(a, n_tok, grp, kh, lo, hi)) {
        if (me.row >= 0 && cc + c < a.hd) a.o[(size_t)me.row * a.hd + cc + c] = __builtin_nanf("");
        return;
    }
    const int span = hi - lo + 1, ns = (span + 63) / 64;
    // loader: V rows lp + 16 m, columns lc .. lc + 3 of the chunk; weight of row wr at position wj
    const int lp = tid >> 4, lc = (tid & 15) * 4, wr = tid >> 6, wj = tid & 63;
    const bool lcol = cc + lc < a.hd;
    const float *vb = a.v + (int64_t)kh * a.hd + cc + lc;
    const GroupRow wg = group_row(a, n_tok, grp, kh, wr);
    const float *wrow = a.s + (size_t)(wg.row < 0 ? 0 : wg.row) * a.max_len;
    auto load = [&](int k, float4(&v)[4], float &w) {
        const int p0 = lo + k * 64;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int p = min(p0 + lp + 16 * m, hi);
            v[m] = lcol ? *(const float4 *)(vb + kv_slot(p, a.cap) * a.kv_dim) : make_float4(0, 0, 0, 0);
        }
        const int p = p0 + wj;
        w = p >= wg.st && p <= wg.en ? wrow[p - wg.st] : 0.0f;
    };
    float4 rv[AV_S][4];
    float rw[AV_S];
#pragma unroll
    for (int u = 0; u < AV_S; ++u)
        if (u < ns) load(u, rv[u], rw[u]);
    float acc = 0.0f;
    for (int k0 = 0; k0 < ns; k0 += AV_S) {
#pragma unroll
        for (int u = 0; u < AV_S; ++u) {
            const int k = k0 + u;
            if (k < ns) {
                const int b = k & 1;
#pragma unroll
                for (int m = 0; m < 4; ++m) vt[b][lp + 16 * m][tid & 15] = rv[u][m];
                ((float *)wt[b])[wr * 64 + wj] = rw[u];
                __syncthreads();
                if (k + AV_S < ns) load(k + AV_S, rv[u], rw[u]);
                const float *vs = (const float *)vt[b] + c;
                const float4 *ws = wt[b][r];
                const int cnt = min(64, span - k * 64);
                if (cnt == 64) {
#pragma unroll
                    for (int j4 = 0; j4 < 16; ++j4) {
                        const float4 w4 = ws[j4];
                        acc = __builtin_fmaf(w4.x, vs[(4 * j4 + 0) * 64], acc);
                        acc = __builtin_fmaf(w4.y, vs[(4 * j4 + 1) * 64], acc);
                        acc = __builtin_fmaf(w4.z, vs[(4 * j4 + 2) * 64], acc);
                        acc = __builtin_fmaf(w4.w, vs[(4 * j4 + 3) * 64], acc);
                    }
                } else {
                    const float *wf = (const float *)ws;
                    for (int j = 0; j < cnt; ++j) acc = __builtin_fmaf(wf[j], vs[j * 64], acc);
                }
            }
        }
    }
    if (me.row >= 0 && cc + c < a.hd)
        a.o[(size_t)me.row * a.hd + cc + c] = me.en >= me.st ? acc : __builtin_nanf("");
}

hipError_t launch_attention(const AttnArgs &a, int n_tok, hipStream_t s) {
    if (n_tok < 1 || a.hd < 32 || a.hd > 256 || a.hd % 32 != 0 || a.n_head_kv < 1 || a.n_head % a.n_head_kv != 0 ||
        a.max_len < 1 || a.kv_dim % 4 != 0)
        return hipErrorInvalidValue;
    const int groups = (n_tok * (a.n_head / a.n_head_kv) + 3) / 4;
    if (groups > 65535 || a.n_head_kv > 65535) return hipErrorInvalidValue;
    const unsigned kb = (unsigned)std::min((a.max_len + 255) / 256, 1024);
    attn_scores_kernel<<<dim3(kb, (unsigned)groups, (unsigned)a.n_head_kv), 256, 0, s>>>(a, n_tok);
    attn_softmax_kernel<<<n_tok * a.n_head, 256, 0, s>>>(a);
    attn_values_kernel<<<dim3((unsigned)((a.hd + 63) / 64), (unsigned)groups, (unsigned)a.n_head_kv), 256, 0, s>>>(
        a, n_tok);
    return hipGetLastError();
}

}  // namespace fgh
