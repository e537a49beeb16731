// fgh_attn.hip - attention over an fp32 KV ring cache on gfx950, bit-exact with the reference's
// attn_rows (fastgguf.c:3273-3326): its vector path (hd % 32 == 0) and its per-row path (any
// other head size up to 256).
//
// Rows are (token, head) pairs: row i = t * n_head + h reads q / writes o at i * hd and the K / V
// head (h / G) * hd of each cache row (G = n_head / n_head_kv, the GQA grouping of the reference's
// forward, 4770-4790), over the positions st[t]..en[t] (slot p % cap). Three launches:
//   scores   8 chains per key: chain l runs fma over q[8m + l] k[8m + l] (att_qk_kern,
//            3227-3246), then hsum4_ps's tree ((a0+a1)+(a2+a3))+((a4+a5)+(a6+a7)) (3187-3190),
//            times scale; other head sizes dot_f32v's order (1618-1632): 8-lane chains s0 over
//            values 16 i + l and s1 over 16 i + 8 + l, one more group of 8 into s0, hsum_ps of
//            s0 + s1, then the last hd % 8 values one fma each, times scale (3313-3315)
//   softmax  one workgroup per row (softmax_vec, 3194-3219): the maximum, exp_neg_ps (3168-3184)
//            over whole groups of 8 and libm's expf over the tail, the sum as 8 ordered lane sums
//            (lane l over e[8g + l]) added in hsum_ps's tree then the tail in order, and every
//            value times 1 / sum
//   values   one lane per output element (att_v_kern, 3249-3270): acc = fma(w_p, v_p[c], acc)
//            over the positions in order
// The value sums are one dependent chain per (row, element) over every position: the
// reference's order, which no split over positions keeps. What bounds them is the latency of
// their operands, so the kernel keeps many tiles of V in flight per workgroup and runs the
// chains out of LDS. Head sizes up to 256; for hd % 32 == 0, kv_dim % 4 == 0 and 16-byte aligned
// pointers; other head sizes read K and (when a 16-byte read would not be aligned) V value by value.
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

// A group is R rows that read the same K / V head kh: group q of head kh holds j = R q .. R q + R - 1
// of the head's n_tok * G rows, j = t * G + g (token t, query head kh * G + g). The scores and the
// value sums of a group run over the union lo..hi of its rows' ranges, as attn_rows runs its 4-row
// calls; a position outside a row's own range has weight 0, and fma(0, v, acc) = acc, so every
// row's sums are those of its own range.
struct GroupRow {
    int row, st, en;  // row = -1: no such row; en < st: no valid range
};
__device__ __forceinline__ GroupRow group_row(const AttnArgs &a, int n_tok, int R, int grp, int kh, int r) {
    const int G = a.n_head / a.n_head_kv, j = grp * R + r;
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
__device__ __forceinline__ bool group_span(const AttnArgs &a, int n_tok, int R, int grp, int kh, int &lo, int &hi) {
    lo = 0x7fffffff;
    hi = -0x7fffffff;
    for (int r = 0; r < R; ++r) {
        const GroupRow g = group_row(a, n_tok, R, grp, kh, r);
        if (g.en >= g.st) {
            lo = min(lo, g.st);
            hi = max(hi, g.en);
        }
    }
    return hi >= lo;
}

// scores: grid (key blocks, groups of R rows, K heads), 256 threads; thread = one key of the union
// for the group's R rows, 8 lane chains per row over the head's values (2 x float4 of K per step),
// the q rows from LDS (one address for the whole wavefront: a broadcast read). R = 16 for prompt
// batches: each K row loaded serves 16 rows.
template <int R>
__global__ __launch_bounds__(256) void attn_scores_kernel(AttnArgs a, int n_tok) {
    __shared__ float4 qs[R][64];
    const int grp = blockIdx.y, kh = blockIdx.z, tid = threadIdx.x;
    int lo, hi;
    if (!group_span(a, n_tok, R, grp, kh, lo, hi)) return;
    const int h4 = a.hd / 4;
    for (int i = tid; i < R * h4; i += 256) {
        const int r = i / h4, x = i - r * h4;
        const GroupRow g = group_row(a, n_tok, R, grp, kh, r);
        qs[r][x] = g.en >= g.st ? ((const float4 *)(a.q + (size_t)g.row * a.hd))[x] : make_float4(0, 0, 0, 0);
    }
    __syncthreads();
    const int64_t kvo = (int64_t)kh * a.hd;
    for (int p = lo + (int)blockIdx.x * 256 + tid; p <= hi; p += (int)gridDim.x * 256) {
        const float4 *kp = (const float4 *)(a.k + kv_slot(p, a.cap) * a.kv_dim + kvo);
        float acc[R][8];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int l = 0; l < 8; ++l) acc[r][l] = 0.0f;
#pragma unroll(R == 4 ? 4 : 1)
        for (int m = 0; m < a.hd / 8; ++m) {
            const float4 k0 = kp[2 * m], k1 = kp[2 * m + 1];
#pragma unroll
            for (int r = 0; r < R; ++r) {
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
        for (int r = 0; r < R; ++r) {
            const GroupRow g = group_row(a, n_tok, R, grp, kh, r);
            if (p >= g.st && p <= g.en) {
                const float t = ((acc[r][0] + acc[r][1]) + (acc[r][2] + acc[r][3])) +
                                ((acc[r][4] + acc[r][5]) + (acc[r][6] + acc[r][7]));
                a.s[(size_t)g.row * a.max_len + (p - g.st)] = t * a.scale;
            }
        }
    }
}

// scores of the per-row path (hd % 32 != 0): as attn_scores_kernel, thread = one key of the group's
// union, the q rows from LDS, K read value by value (any head size and offset), dot_f32v's order
template <int R>
__global__ __launch_bounds__(256) void attn_scores_row_kernel(AttnArgs a, int n_tok) {
    __shared__ float qs[R][256];
    const int grp = blockIdx.y, kh = blockIdx.z, tid = threadIdx.x;
    int lo, hi;
    if (!group_span(a, n_tok, R, grp, kh, lo, hi)) return;
    const int hd = a.hd;
    for (int i = tid; i < R * hd; i += 256) {
        const int r = i / hd, x = i - r * hd;
        const GroupRow g = group_row(a, n_tok, R, grp, kh, r);
        qs[r][x] = g.en >= g.st ? a.q[(size_t)g.row * hd + x] : 0.0f;
    }
    __syncthreads();
    const int64_t kvo = (int64_t)kh * hd;
    for (int p = lo + (int)blockIdx.x * 256 + tid; p <= hi; p += (int)gridDim.x * 256) {
        const float *kp = a.k + kv_slot(p, a.cap) * a.kv_dim + kvo;
        float s0[R][8], s1[R][8];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int l = 0; l < 8; ++l) s0[r][l] = s1[r][l] = 0.0f;
        int i = 0;
        for (; i + 16 <= hd; i += 16) {
            float k0[8], k1[8];
#pragma unroll
            for (int l = 0; l < 8; ++l) {
                k0[l] = kp[i + l];
                k1[l] = kp[i + 8 + l];
            }
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int l = 0; l < 8; ++l) {
                    s0[r][l] = __builtin_fmaf(qs[r][i + l], k0[l], s0[r][l]);
                    s1[r][l] = __builtin_fmaf(qs[r][i + 8 + l], k1[l], s1[r][l]);
                }
        }
        if (i + 8 <= hd) {
#pragma unroll
            for (int l = 0; l < 8; ++l) {
                const float k0 = kp[i + l];
#pragma unroll
                for (int r = 0; r < R; ++r) s0[r][l] = __builtin_fmaf(qs[r][i + l], k0, s0[r][l]);
            }
            i += 8;
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const GroupRow g = group_row(a, n_tok, R, grp, kh, r);
            if (p >= g.st && p <= g.en) {
                float v[8];
#pragma unroll
                for (int l = 0; l < 8; ++l) v[l] = s0[r][l] + s1[r][l];
                float t = ((v[0] + v[4]) + (v[1] + v[5])) + ((v[2] + v[6]) + (v[3] + v[7]));  // hsum_ps
                for (int j = i; j < hd; ++j) t = __builtin_fmaf(qs[r][j], kp[j], t);
                a.s[(size_t)g.row * a.max_len + (p - g.st)] = t * a.scale;
            }
        }
    }
}

// softmax: one workgroup per row, in place over the row's scores. A row of up to SM_RES positions
// stays in LDS (sized min(max_len, SM_RES) at launch, so short rows leave room for more
// workgroups per CU) from its one load to its one store: maximum, exponentials, lanes 0..7 of
// wavefront 0 running the 8 ordered sums, then every value times 1 / sum. Longer rows go
// through LDS SM_RES positions at a time, the 8 sums carried across the chunks.
constexpr int SM_RES = 12288;
__device__ __forceinline__ float sum8_tree(float v) {  // lanes 0..7: hsum_ps's tree
    v = v + __shfl_xor(v, 4, 8);                       // (v0 + v4), (v1 + v5), ...
    v = v + __shfl_xor(v, 1, 8);
    return v + __shfl_xor(v, 2, 8);  // ((v0 + v4) + (v1 + v5)) + ((v2 + v6) + (v3 + v7))
}
__device__ __forceinline__ float lane_sum(const float *e, int ng, int l, float v) {  // v += e[8g + l], g < ng
    int g = 0;
    for (; g + 8 <= ng; g += 8) {
        float t[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) t[u] = e[8 * (g + u) + l];
#pragma unroll
        for (int u = 0; u < 8; ++u) v += t[u];
    }
    for (; g < ng; ++g) v += e[8 * g + l];
    return v;
}
__global__ __launch_bounds__(256) void attn_softmax_kernel(AttnArgs a) {
    extern __shared__ float e[];  // min(max_len, SM_RES) values
    __shared__ float red[4];
    __shared__ float total;
    const int row = blockIdx.x, tok = row / a.n_head, tid = threadIdx.x;
    const int n = row_len(a, tok);
    if (n == 0) return;
    float *s = a.s + (size_t)row * a.max_len;
    const int nv = n & ~7;  // whole groups of 8
    const bool resident = n <= SM_RES;
    float mx = -__builtin_inff();
    if (resident) {
#pragma unroll 8
        for (int i = tid; i < n; i += 256) {
            const float x = s[i];
            e[i] = x;
            mx = fmaxf(mx, x);
        }
    } else {
        for (int i = tid; i < n; i += 256) mx = fmaxf(mx, s[i]);
    }
    for (int o = 1; o < 64; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    if (resident) {
        for (int i = tid; i < n; i += 256) e[i] = i < nv ? exp_neg_ref(e[i] - mx) : expf_ref(e[i] - mx);
        __syncthreads();
        if (tid < 8) {
            float v = sum8_tree(lane_sum(e, nv / 8, tid, 0.0f));
            if (tid == 0) {
                for (int i = nv; i < n; ++i) v += e[i];  // the tail, in order
                total = v;
            }
        }
        __syncthreads();
        const float sum = total;
        const float inv = 1.0f / sum;
        for (int i = tid; i < n; i += 256) s[i] = sum > 0.0f ? e[i] * inv : e[i];
        return;
    }
    float v = 0.0f;
    for (int c0 = 0; c0 < n; c0 += SM_RES) {
        const int cn = min(SM_RES, n - c0);
        for (int i = tid; i < cn; i += 256) {
            const float x = s[c0 + i] - mx;
            const float ev = c0 + i < nv ? exp_neg_ref(x) : expf_ref(x);
            e[i] = ev;
            s[c0 + i] = ev;
        }
        __syncthreads();
        if (tid < 8) {
            v = lane_sum(e, (min(c0 + cn, nv) - c0) / 8, tid, v);
            if (c0 + cn == n) {  // the last chunk holds the tail
                v = sum8_tree(v);
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

// values: grid (64-column chunks, groups of 4 CH rows, K heads), 256 threads. Lane c of wavefront w
// runs the chains of rows CH w .. CH w + CH - 1 for column c of the chunk: acc_r = fma(w_rp, v_p,
// acc_r) over the union in order, one LDS read of v_p serving the CH chains. CH = 1 for decode
// (few rows: every wavefront gets a row of its own), CH = 4 for prompt batches (fewer LDS reads
// per fma). Tiles of 64 positions (V: 64 x 64 floats; weights: CH = 1 row-major 4 x 64, so one
// 16-byte read gives 4 positions, CH = 4 position-major 64 x 16, so one 16-byte read gives a
// wavefront's 4 rows) are loaded by all 256 threads AV_S tiles ahead into registers, then stored
// to a double-buffered LDS tile (one barrier per tile). Every load is unconditional (clamped
// addresses, the range mask applied at the store, the loop padded to whole rounds of AV_S
// tiles) and the stages' loads keep their order, so the wait before a tile's store covers that
// tile's loads only while AV_S - 1 tiles stay in flight.
typedef float av4 __attribute__((ext_vector_type(4)));  // a native vector: kept in registers when staged
template <int CH>
struct AvStage {
    av4 v0, v1, v2, v3;  // fp32 V: 4 columns at each of the thread's 4 positions
    uint32_t k0, k1, k2, k3;  // TurboQuant V: the same values' raw codes
    av4 w;  // CH = 4: 4 positions of one row; CH = 1: .x only
};
// VB = 0: V in fp32 (a.v); VB = 2, 4, 8: V as TurboQuant records (a.vq), decoded to centroids
// (int8 codes for VB = 8) through an LDS table when a tile is stored
// SC: V read value by value (hd or kv_dim not a multiple of 4: a 16-byte read would not be aligned),
// columns past hd reading column 0
// PR: the reference's per-row path (hd % 32 != 0, fastgguf.c:3318-3323): each row's chain walks
// only its own positions st..en, so a position of another row of the group adds nothing to it (not
// even fma(0, v, acc), which is NaN for a non-finite v and turns -0 into +0); the vector path's
// att_v_kern walks the group's whole span with zero weights, as the chains do without PR
template <int CH, int AV_S, int VB, bool SC = false, bool PR = false>  // AV_S: tiles in flight, 4 or 8 (the named stages below)
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void attn_values_kernel(AttnArgs a,
                                                                                                     int n_tok) {
    constexpr int GR = 4 * CH;  // rows per group
    // CH = 1: two tiles per barrier over a ring of 4 LDS tiles (a wavefront overwrites a pair's
    // tiles only after the next pair's barrier, which every wavefront reaches after consuming it)
    constexpr bool PAIR = CH == 1;
    constexpr int NB = PAIR ? 4 : 2;
    __shared__ av4 vt[NB][64][16];
    __shared__ __attribute__((aligned(16))) float wt[NB][64 * GR];
    __shared__ float ctab[16];
    const int grp = blockIdx.y, kh = blockIdx.z, cc = (int)blockIdx.x * 64, tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    int lo, hi;
    if (!group_span(a, n_tok, GR, grp, kh, lo, hi)) {
        for (int r = 0; r < CH; ++r) {
            const GroupRow g = group_row(a, n_tok, GR, grp, kh, CH * wave + r);
            if (g.row >= 0 && cc + lane < a.hd) a.o[(size_t)g.row * a.hd + cc + lane] = __builtin_nanf("");
        }
        return;
    }
    const int span = hi - lo + 1, ns = (span + 63) / 64;
    // loader: V positions lp + 16 m, columns lc .. lc + 3 of the chunk (columns past hd read
    // column 0 instead: always a valid address; those outputs are not stored); weights: CH = 4,
    // row wr at positions wp .. wp + 3; CH = 1, row wr1 at position wp1
    const int lp = tid >> 4, lc = (tid & 15) * 4;
    const int wr = CH == 4 ? tid >> 4 : tid >> 6, wp = CH == 4 ? (tid & 15) * 4 : tid & 63;
    const int lcol = cc + lc < a.hd ? cc + lc : 0;
    const float *vb = VB ? nullptr : a.v + (int64_t)kh * a.hd + lcol;
    // SC: the offsets of columns lcol + 1 .. + 3 from lcol (0 where a column is past hd: column lcol)
    const int sc1 = cc + lc + 1 < a.hd ? 1 : 0, sc2 = cc + lc + 2 < a.hd ? 2 : 0, sc3 = cc + lc + 3 < a.hd ? 3 : 0;
    const int vrec = 4 + a.hd * VB / 8;  // TurboQuant: record bytes, the slot's records back to back
    const uint8_t *qb = VB ? a.vq + (int64_t)kh * vrec + 4 + (int64_t)lcol * VB / 8 : nullptr;
    const int64_t qstride = (int64_t)a.n_head_kv * vrec;
    if (VB == 4 && tid < 16) ctab[tid] = kvq_centroid4(tid);
    if (VB == 2 && tid < 4) ctab[tid] = kvq_centroid2(tid);
    if constexpr (VB == 2 || VB == 4) __syncthreads();  // the table is read by the first tile's store
    const GroupRow wg = group_row(a, n_tok, GR, grp, kh, wr);
    const float *wrow = a.s + (size_t)(wg.row < 0 ? 0 : wg.row) * a.max_len;
    // the loads walk the tiles in order, so the positions and ring slots advance by 64 per load
    // (slot + 64 % cap, one conditional subtract) with no division in the loop; a position past
    // hi reads hi's slot (a valid address; its weight is masked)
    const int step64 = 64 % a.cap, slot_hi = (int)kv_slot(hi, a.cap);
    int vpos[4], vslot[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        vpos[m] = lo + lp + 16 * m;
        vslot[m] = (int)kv_slot(vpos[m], a.cap);
    }
    int wx = lo + wp - wg.st;  // score index of the next weight load
    auto load = [&](AvStage<CH> &t) {
        av4 *dst[4] = {&t.v0, &t.v1, &t.v2, &t.v3};
        uint32_t *kdst[4] = {&t.k0, &t.k1, &t.k2, &t.k3};
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int sl = vpos[m] <= hi ? vslot[m] : slot_hi;
            if constexpr (VB == 0 && SC) {
                const float *vp = vb + (int64_t)sl * a.kv_dim;
                *dst[m] = (av4){vp[0], vp[sc1], vp[sc2], vp[sc3]};
            } else if constexpr (VB == 0)
                *dst[m] = *(const av4 *)(vb + (int64_t)sl * a.kv_dim);
            else if constexpr (VB == 8)
                *kdst[m] = *(const uint32_t *)(qb + sl * qstride);
            else if constexpr (VB == 4)
                *kdst[m] = *(const uint16_t *)(qb + sl * qstride);
            else
                *kdst[m] = *(qb + sl * qstride);
            vpos[m] += 64;
            vslot[m] += step64;
            if (vslot[m] >= a.cap) vslot[m] -= a.cap;
        }
        // raw loads only: the range mask is applied at the store
        if constexpr (CH == 4)
            t.w = (av4){wrow[min(max(wx, 0), a.max_len - 1)], wrow[min(max(wx + 1, 0), a.max_len - 1)],
                        wrow[min(max(wx + 2, 0), a.max_len - 1)], wrow[min(max(wx + 3, 0), a.max_len - 1)]};
        else
            t.w.x = wrow[min(max(wx, 0), a.max_len - 1)];
        wx += 64;
    };
    auto in_range = [&](int p) { return p >= wg.st && p <= wg.en; };
    float acc[CH];
    int rst[CH], ren[CH];  // PR: the ranges of this wavefront's rows (uniform over its lanes)
#pragma unroll
    for (int r = 0; r < CH; ++r) {
        acc[r] = 0.0f;
        if constexpr (PR) {
            const GroupRow g = group_row(a, n_tok, GR, grp, kh, CH * wave + r);
            rst[r] = g.st;
            ren[r] = g.en;
        }
    }
    // acc = fma(w, v, acc) for a position p of row r's chain (PR: only inside its own range)
    auto fma_at = [&](int r, int p, float w, float v) {
        if constexpr (PR)
            acc[r] = p >= rst[r] && p <= ren[r] ? __builtin_fmaf(w, v, acc[r]) : acc[r];
        else
            acc[r] = __builtin_fmaf(w, v, acc[r]);
    };
    const float *vcol = (const float *)vt + lane;
    auto decode = [&](uint32_t c) -> av4 {  // 4 values of TurboQuant codes
        if constexpr (VB == 8)
            return (av4){(float)(int8_t)c, (float)(int8_t)(c >> 8), (float)(int8_t)(c >> 16), (float)(int8_t)(c >> 24)};
        else if constexpr (VB == 4)
            return (av4){ctab[c & 15], ctab[(c >> 4) & 15], ctab[(c >> 8) & 15], ctab[(c >> 12) & 15]};
        else
            return (av4){ctab[c & 3], ctab[(c >> 2) & 3], ctab[(c >> 4) & 3], ctab[(c >> 6) & 3]};
    };
    auto store = [&](int k, AvStage<CH> &t) {
        const int b = k & (NB - 1);
        if constexpr (VB == 0) {
            vt[b][lp][tid & 15] = t.v0;
            vt[b][lp + 16][tid & 15] = t.v1;
            vt[b][lp + 32][tid & 15] = t.v2;
            vt[b][lp + 48][tid & 15] = t.v3;
        } else {
            vt[b][lp][tid & 15] = decode(t.k0);
            vt[b][lp + 16][tid & 15] = decode(t.k1);
            vt[b][lp + 32][tid & 15] = decode(t.k2);
            vt[b][lp + 48][tid & 15] = decode(t.k3);
        }
        const int p = lo + k * 64 + wp;
        if constexpr (CH == 4) {
            float *wf = wt[b];
            wf[(wp + 0) * GR + wr] = in_range(p) ? t.w.x : 0.0f;
            wf[(wp + 1) * GR + wr] = in_range(p + 1) ? t.w.y : 0.0f;
            wf[(wp + 2) * GR + wr] = in_range(p + 2) ? t.w.z : 0.0f;
            wf[(wp + 3) * GR + wr] = in_range(p + 3) ? t.w.w : 0.0f;
        } else {
            wt[b][wr * 64 + wp] = in_range(p) ? t.w.x : 0.0f;
        }
    };
    auto consume = [&](int k) {
        const int b = k & (NB - 1);
        const float *vs = vcol + b * 64 * 64;
        const int cnt = min(64, span - k * 64);  // <= 0 past the end
        const int p0 = lo + k * 64;              // the tile's first position
        if constexpr (CH == 4) {
            const av4 *ws = (const av4 *)wt[b] + wave;  // [pos][16 rows]: this wavefront's 4
            auto chain = [&](int j) {
                const float x = vs[j * 64];
                const av4 w4 = ws[j * 4];
                fma_at(0, p0 + j, w4.x, x);
                fma_at(1, p0 + j, w4.y, x);
                fma_at(2, p0 + j, w4.z, x);
                fma_at(3, p0 + j, w4.w, x);
            };
            if (cnt == 64) {
#pragma unroll 8
                for (int j = 0; j < 64; ++j) chain(j);
            } else {
                for (int j = 0; j < cnt; ++j) chain(j);
            }
        } else {
            const float *wf = wt[b] + wave * 64;  // [4 rows][pos]: this wavefront's row
            if (cnt == 64) {
#pragma unroll
                for (int j4 = 0; j4 < 16; ++j4) {
                    const av4 w4 = *(const av4 *)(wf + 4 * j4);
                    fma_at(0, p0 + 4 * j4 + 0, w4.x, vs[(4 * j4 + 0) * 64]);
                    fma_at(0, p0 + 4 * j4 + 1, w4.y, vs[(4 * j4 + 1) * 64]);
                    fma_at(0, p0 + 4 * j4 + 2, w4.z, vs[(4 * j4 + 2) * 64]);
                    fma_at(0, p0 + 4 * j4 + 3, w4.w, vs[(4 * j4 + 3) * 64]);
                }
            } else {
                for (int j = 0; j < cnt; ++j) fma_at(0, p0 + j, wf[j], vs[j * 64]);
            }
        }
    };
    // one tile: store the staged registers, barrier, reload them AV_S tiles ahead, run the chains
    auto step = [&](int k, AvStage<CH> &t) {
        store(k, t);
        __syncthreads();
        load(t);  // tile k + AV_S
        consume(k);
    };
    auto step2 = [&](int k, AvStage<CH> &ta, AvStage<CH> &tb) {  // tiles k and k + 1, one barrier
        store(k, ta);
        store(k + 1, tb);
        __syncthreads();
        load(ta);  // tile k + AV_S
        load(tb);  // tile k + 1 + AV_S
        consume(k);
        consume(k + 1);
    };
    // the stages' loads are issued strictly in order (scheduling barriers), so the loop head
    // waits for the oldest stage only
    AvStage<CH> t0, t1, t2, t3, t4, t5, t6, t7;
#define AV_LOAD(i) \
    load(t##i); \
    __builtin_amdgcn_sched_barrier(0);
#define AV_STEP(i) \
    step(k0 + i, t##i); \
    __builtin_amdgcn_sched_barrier(0);
    AV_LOAD(0) AV_LOAD(1) AV_LOAD(2) AV_LOAD(3)
    if constexpr (AV_S == 8) {
        AV_LOAD(4) AV_LOAD(5) AV_LOAD(6) AV_LOAD(7)
    }
#define AV_STEP2(i, j) \
    step2(k0 + i, t##i, t##j); \
    __builtin_amdgcn_sched_barrier(0);
    for (int k0 = 0; k0 < ns; k0 += AV_S) {
        if constexpr (PAIR) {
            AV_STEP2(0, 1) AV_STEP2(2, 3)
            if constexpr (AV_S == 8) {
                AV_STEP2(4, 5) AV_STEP2(6, 7)
            }
        } else {
            AV_STEP(0) AV_STEP(1) AV_STEP(2) AV_STEP(3)
            if constexpr (AV_S == 8) {
                AV_STEP(4) AV_STEP(5) AV_STEP(6) AV_STEP(7)
            }
        }
    }
#undef AV_STEP2
#undef AV_LOAD
#undef AV_STEP
#pragma unroll
    for (int r = 0; r < CH; ++r) {
        const GroupRow g = group_row(a, n_tok, GR, grp, kh, CH * wave + r);
        if (g.row >= 0 && cc + lane < a.hd)
            a.o[(size_t)g.row * a.hd + cc + lane] = g.en >= g.st ? acc[r] : __builtin_nanf("");
    }
}

hipError_t launch_attention_values(const AttnArgs &a, int n_tok, hipStream_t s) {
    if (n_tok < 1 || a.hd < 1 || a.hd > 256 || a.n_head_kv < 1 || a.n_head % a.n_head_kv != 0 || a.max_len < 1)
        return hipErrorInvalidValue;
    // 16-byte V reads need 4-value columns and rows; TurboQuant records need a multiple of 32
    const bool sc = a.hd % 4 != 0 || a.kv_dim % 4 != 0 || (uintptr_t)a.v % 16 != 0;
    if (a.vq && (a.hd % 32 != 0 || sc)) return hipErrorInvalidValue;
    const int rows_kv = n_tok * (a.n_head / a.n_head_kv);
    if ((rows_kv + 3) / 4 > 65535 || a.n_head_kv > 65535) return hipErrorInvalidValue;
    if (a.vq ? (a.vbits != 2 && a.vbits != 4 && a.vbits != 8) : !a.v) return hipErrorInvalidValue;
    const unsigned cch = (unsigned)((a.hd + 63) / 64), kvh = (unsigned)a.n_head_kv;
    const dim3 g16(cch, (unsigned)((rows_kv + 15) / 16), kvh), g4(cch, (unsigned)((rows_kv + 3) / 4), kvh);
    const int vb = a.vq ? a.vbits : 0;
    if (a.hd % 32 != 0) {  // the per-row path (TurboQuant V needs hd % 32 == 0)
        if (sc) {
            if (rows_kv >= 64) attn_values_kernel<4, 4, 0, true, true><<<g16, 256, 0, s>>>(a, n_tok);
            else attn_values_kernel<1, 8, 0, true, true><<<g4, 256, 0, s>>>(a, n_tok);
        } else {
            if (rows_kv >= 64) attn_values_kernel<4, 4, 0, false, true><<<g16, 256, 0, s>>>(a, n_tok);
            else attn_values_kernel<1, 8, 0, false, true><<<g4, 256, 0, s>>>(a, n_tok);
        }
    } else if (sc) {
        if (rows_kv >= 64) attn_values_kernel<4, 4, 0, true><<<g16, 256, 0, s>>>(a, n_tok);
        else attn_values_kernel<1, 8, 0, true><<<g4, 256, 0, s>>>(a, n_tok);
    } else if (rows_kv >= 64) {
        if (vb == 0) attn_values_kernel<4, 4, 0><<<g16, 256, 0, s>>>(a, n_tok);
        else if (vb == 8) attn_values_kernel<4, 4, 8><<<g16, 256, 0, s>>>(a, n_tok);
        else if (vb == 4) attn_values_kernel<4, 4, 4><<<g16, 256, 0, s>>>(a, n_tok);
        else attn_values_kernel<4, 4, 2><<<g16, 256, 0, s>>>(a, n_tok);
    } else {
        if (vb == 0) attn_values_kernel<1, 8, 0><<<g4, 256, 0, s>>>(a, n_tok);
        else if (vb == 8) attn_values_kernel<1, 8, 8><<<g4, 256, 0, s>>>(a, n_tok);
        else if (vb == 4) attn_values_kernel<1, 8, 4><<<g4, 256, 0, s>>>(a, n_tok);
        else attn_values_kernel<1, 8, 2><<<g4, 256, 0, s>>>(a, n_tok);
    }
    return hipGetLastError();
}

hipError_t launch_attention(const AttnArgs &a, int n_tok, hipStream_t s) {
    if (n_tok < 1 || a.hd < 1 || a.hd > 256 || a.n_head_kv < 1 || a.n_head % a.n_head_kv != 0 || a.max_len < 1)
        return hipErrorInvalidValue;
    const bool vec = a.hd % 32 == 0;  // the reference's vector path: 16-byte reads of q and K
    if (vec && (a.kv_dim % 4 != 0 || ((uintptr_t)a.q | (uintptr_t)a.k) % 16 != 0)) return hipErrorInvalidValue;
    const int rows_kv = n_tok * (a.n_head / a.n_head_kv);  // rows per K / V head
    if ((rows_kv + 3) / 4 > 65535 || a.n_head_kv > 65535) return hipErrorInvalidValue;
    const unsigned kb = (unsigned)std::min((a.max_len + 255) / 256, 1024);
    const dim3 kvh(1, 1, (unsigned)a.n_head_kv);
    if (!vec)
        attn_scores_row_kernel<4><<<dim3(kb, (unsigned)((rows_kv + 3) / 4), kvh.z), 256, 0, s>>>(a, n_tok);
    else if (rows_kv >= 16)
        attn_scores_kernel<16><<<dim3(kb, (unsigned)((rows_kv + 15) / 16), kvh.z), 256, 0, s>>>(a, n_tok);
    else
        attn_scores_kernel<4><<<dim3(kb, (unsigned)((rows_kv + 3) / 4), kvh.z), 256, 0, s>>>(a, n_tok);
    attn_softmax_kernel<<<n_tok * a.n_head, 256, (size_t)std::min(a.max_len, SM_RES) * 4, s>>>(a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_attention_values(a, n_tok, s);  // 4 chains per lane from 64 rows per K / V head
}

}  // namespace fgh
