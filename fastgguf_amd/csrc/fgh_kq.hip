// fgh_kq.hip - the decode matvec for the 256-value types on Q8 activations: Q2_K, Q3_K and IQ4_XS
// (dot_q2_K_q8 fastgguf.c:1426-1479, dot_q3_K_q8 1481-1545, dot_iq4_xs_q8 1580-1614; the
// reference's own GPU path leaves these types on the CPU, gpu_kernel_for 1744-1751).
//
// Each of these row kernels runs ONE fp32 chain per row over the row's 32-value blocks in order;
// the integers of a 32-block are exact. So a wavefront takes 8 rows of one 256-value block per
// step and lane L = 8 r + c takes 32-block c of row r: it forms the block's integers alone, from
// its own bytes and 32 LDS activations, and reduces them to the chain's two factors (a_c, b_c);
// lane 8 r then gathers the row's 8 pairs by DPP and runs the chain over them, block after block:
//   Q2_K:   S = sum q sc x (sc per 16), M = m_0 s16_0 + m_1 s16_1 (the 4-bit mins);
//           a = xd, b = fma(d, S, -(dmin M))
//   Q3_K:   q = lo | 4 hbit (0..7), sc' = 6-bit scale - 32, S = sum q sc' x,
//           M = sc'_0 s16_0 + sc'_1 s16_1; a = d xd, b = S - 4 M
//   IQ4_XS: si = sum kvalues[nib] x; a = d (ls - 32) xd, b = si
//   sum = fma(a_c, b_c, sum)
// (these are the contractions gcc makes of the reference's `sum += xk->d * (d * S - dmin * M)`
// and its like, which the results are bit-identical to). Short matrices split the steps of a
// tile over S wavefronts; wavefronts ks >= 1 park their pairs in LDS and wavefront 0 continues
// the chains over them. Up to 4 tensors of one type and width share one launch, and an expert
// index per token slot (the MoE's sel) picks the matrix, as in the other decode kernels.
//
// Tiles: 8 rows of one block, step-major like the other types (step s of row tile t of matrix m
// at ((m * steps + s) * tpm + t) * tile bytes). Value l of 32-block c = 4 n + j is, in the file,
// bit pair j of qs[32 n + l] (Q2_K, Q3_K); in a tile, lane L's two quant dwords hold it as bit
// pair t of byte b of dword u, l = 16 u + 4 t + b, so (dword u >> 2 t) & 0x03030303 is the four
// values that meet activation dword 4 u + t:
//   Q2_K tile 672 B:   [0, 512) quants, lane L at 8 L; [512, 640) the row's scale bytes 2c, 2c+1
//                      (file bytes 2c, 2c+1) at 512 + 2 L; [640, 672) fp16 d, dmin of row r at 640 + 4 r
//   Q3_K tile 880 B:   [0, 512) low bit pairs as Q2_K; [512, 768) high bits, lane L's dword at
//                      512 + 4 L with bit 8 b + 4 u + t = hmask bit c of value 16 u + 4 t + b;
//                      [768, 864) the row's 12 packed scale bytes at 768 + 12 r; [864, 880) fp16 d
//   IQ4_XS tile 1088 B: [0, 1024) nibbles, lane L at 16 L (file qs[16 c .. 16 c + 15]);
//                      [1024, 1088) file bytes 0..7 of row r (d, scales_h, scales_l) at 1024 + 8 r
// The activations of a workgroup live in LDS as Q8 blocks (quantize_q8, fastgguf.c:746-768):
// qs [nb32][32] at 0, d [nb32] fp32 at 32 nb32, the half sums s16 [nb32][2] int16 at 36 nb32.
#include "fgh_internal.h"

namespace fgh {

template <int AUX = 0>
__device__ __forceinline__ uint32_t bld4(BufRes r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, AUX);
}
// DPP row_shl:k: lane + k within its 16-lane row (lanes without a source read 0: bound_ctrl, which
// also spares the zeroed old value per move)
__device__ __forceinline__ float shl_f32(float v, int k) {
    const int iv = __builtin_bit_cast(int, v);
    int o;
    switch (k) {
    case 1: o = __builtin_amdgcn_update_dpp(0, iv, 0x101, 0xF, 0xF, true); break;
    case 2: o = __builtin_amdgcn_update_dpp(0, iv, 0x102, 0xF, 0xF, true); break;
    case 3: o = __builtin_amdgcn_update_dpp(0, iv, 0x103, 0xF, 0xF, true); break;
    case 4: o = __builtin_amdgcn_update_dpp(0, iv, 0x104, 0xF, 0xF, true); break;
    case 5: o = __builtin_amdgcn_update_dpp(0, iv, 0x105, 0xF, 0xF, true); break;
    case 6: o = __builtin_amdgcn_update_dpp(0, iv, 0x106, 0xF, 0xF, true); break;
    default: o = __builtin_amdgcn_update_dpp(0, iv, 0x107, 0xF, 0xF, true); break;
    }
    return __builtin_bit_cast(float, o);
}

__host__ __device__ constexpr size_t kq_off_d(int nb) { return (size_t)256 * nb; }  // 32 * nb32
__host__ __device__ constexpr size_t kq_off_s(int nb) { return (size_t)288 * nb; }  // 36 * nb32
__host__ __device__ constexpr size_t kq_act_bytes(int nb) { return (size_t)320 * nb; }
constexpr int KQ_REC = 512;  // a parked step: 64 lanes x {a, b}

// ---- quantization of x into LDS: 2 threads per 32-value block, 16 values each ----
struct KqX {
    float4 v[4];
};
template <int WPG>
__device__ __forceinline__ void kq_xload(const float *__restrict__ x, int nb32, int rb, KqX &xv) {
    const int b = rb + (int)threadIdx.x / 2, tl = (int)threadIdx.x & 1;
    const float *p = x + (size_t)(b < nb32 ? b : 0) * 32 + 16 * tl;  // past the end: block 0, unused
#pragma unroll
    for (int u = 0; u < 4; ++u) xv.v[u] = *(const float4 *)(p + 4 * u);
}
template <int WPG>
__device__ __forceinline__ void kq_xstore(int nb, int rb, const KqX &xv, uint8_t *act) {
    const int nb32 = 8 * nb;
    const int b = rb + (int)threadIdx.x / 2, tl = (int)threadIdx.x & 1;
    float v[16];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        v[4 * u] = xv.v[u].x; v[4 * u + 1] = xv.v[u].y; v[4 * u + 2] = xv.v[u].z; v[4 * u + 3] = xv.v[u].w;
    }
    float amax = 0.0f;
#pragma unroll
    for (int u = 0; u < 16; ++u) amax = fmaxf(amax, fabsf(v[u]));
    amax = fmaxf(amax, __builtin_bit_cast(float, dpp_xor1(__builtin_bit_cast(int, amax))));
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    uint32_t w[4];
    int s = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int q0 = q8_round(v[4 * u] * id), q1 = q8_round(v[4 * u + 1] * id);
        const int q2 = q8_round(v[4 * u + 2] * id), q3 = q8_round(v[4 * u + 3] * id);
        s += q0 + q1 + q2 + q3;
        w[u] = pack_q(q0, q1, q2, q3);
    }
    if (b >= nb32) return;
    *(uint4 *)(act + (size_t)32 * b + 16 * tl) = make_uint4(w[0], w[1], w[2], w[3]);
    ((int16_t *)(act + kq_off_s(nb)))[2 * b + tl] = (int16_t)s;  // s16[tl]: the sum of its 16 quants
    if (tl == 0) ((float *)(act + kq_off_d(nb)))[b] = d;
}
template <int WPG>
__device__ __forceinline__ void kq_xfinish(const float *__restrict__ x, int nb, KqX &xv, uint8_t *act) {
    constexpr int BPR = 32 * WPG;  // blocks per round
    kq_xstore<WPG>(nb, 0, xv, act);
    for (int rb = BPR; rb < 8 * nb; rb += BPR) {
        kq_xload<WPG>(x, 8 * nb, rb, xv);
        kq_xstore<WPG>(nb, rb, xv, act);
    }
}

// ---- one lane's bytes of one step ----
template <int TYPE>
struct KqW;
template <>
struct KqW<T_Q2_K> {
    uint2 q;
    uint32_t sc, dd;  // scale bytes 2c, 2c+1; fp16 d | dmin << 16
};
template <>
struct KqW<T_Q3_K> {
    uint2 q;
    uint32_t h, slo, shi, d;  // high bits; scale bytes (2c) % 8, +1 and 8 + (2c) % 4, +1; fp16 d
};
template <>
struct KqW<T_IQ4_XS> {
    uint4 q;
    uint2 rec;  // fp16 d | scales_h << 16, scales_l
};
// T: the tile (wavefront-uniform); live = false: zeros without a memory access
__device__ __forceinline__ void kq_load(const uint8_t *T, uint32_t lane, KqW<T_Q2_K> &w, bool live) {
    const BufRes r = buf_res(T, live ? kq_tile(T_Q2_K) : 0);
    w.q = bld8<WNT>(r, 8 * lane);
    w.sc = bld2<WNT>(r, 512 + 2 * lane);
    w.dd = bld4<WNT>(r, 640 + 4 * (lane >> 3));
}
__device__ __forceinline__ void kq_load(const uint8_t *T, uint32_t lane, KqW<T_Q3_K> &w, bool live) {
    const BufRes r = buf_res(T, live ? kq_tile(T_Q3_K) : 0);
    const uint32_t rr = lane >> 3, c = lane & 7;
    w.q = bld8<WNT>(r, 8 * lane);
    w.h = bld4<WNT>(r, 512 + 4 * lane);
    w.slo = bld2<WNT>(r, 768 + 12 * rr + 2 * (c & 3));
    w.shi = bld2<WNT>(r, 768 + 12 * rr + 8 + 2 * (c & 1));
    w.d = bld2<WNT>(r, 864 + 2 * rr);
}
__device__ __forceinline__ void kq_load(const uint8_t *T, uint32_t lane, KqW<T_IQ4_XS> &w, bool live) {
    const BufRes r = buf_res(T, live ? kq_tile(T_IQ4_XS) : 0);
    w.q = bld16<WNT>(r, 16 * lane);
    w.rec = bld8<WNT>(r, 1024 + 8 * (lane >> 3));
}

// the chain factors (a, b) of 32-block c of the lane's row, and its integers (for the dump):
// y = the block's 8 activation dwords, xd its scale, s16 its two half sums (int16 pair)
__device__ __forceinline__ void kq_pair(const KqW<T_Q2_K> &w, int, const uint32_t y[8], float xd, uint32_t s16,
                                        float &a, float &b, int &S, int &M) {
    const uint32_t D[2] = {w.q.x, w.q.y};
    int s[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        int acc = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t) acc = dot4((int)((D[u] >> (2 * t)) & 0x03030303u), (int)y[4 * u + t], acc);
        s[u] = acc;  // |s| <= 16 * 3 * 127: an int16
    }
    const uint32_t sc = w.sc & 0x0F0Fu, mn = (w.sc >> 4) & 0x0F0Fu;  // bytes -> (lo, hi) int16 pairs
    S = dot2_i16((sc & 0xFu) | ((sc >> 8) << 16), pack_i16(s[0], s[1]), 0);
    M = dot2_i16((mn & 0xFu) | ((mn >> 8) << 16), s16, 0);
    const float d = fp16_bits_to_f32(w.dd & 0xFFFFu), dmin = fp16_bits_to_f32(w.dd >> 16);
    a = xd;
    b = __builtin_fmaf(d, (float)S, -(dmin * (float)M));
}
__device__ __forceinline__ void kq_pair(const KqW<T_Q3_K> &w, int c, const uint32_t y[8], float xd, uint32_t s16,
                                        float &a, float &b, int &S, int &M) {
    const uint32_t D[2] = {w.q.x, w.q.y};
    int s[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        int acc = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t q = ((D[u] >> (2 * t)) & 0x03030303u) | (((w.h >> (4 * u + t)) & 0x01010101u) << 2);
            acc = dot4((int)q, (int)y[4 * u + t], acc);
        }
        s[u] = acc;  // |s| <= 16 * 7 * 127: an int16
    }
    // scales 2c, 2c+1: low nibbles (c / 4) of bytes (2c) % 8, +1; high bit pairs 2 (c / 2) of 8 + (2c) % 4, +1
    const int ln = 4 * (c >> 2), hs = 2 * (c >> 1);
    const int sa = (int)(((w.slo >> ln) & 0xFu) | (((w.shi >> hs) & 3u) << 4)) - 32;
    const int sb = (int)(((w.slo >> (8 + ln)) & 0xFu) | (((w.shi >> (8 + hs)) & 3u) << 4)) - 32;
    const uint32_t scp = pack_i16(sa, sb);
    S = dot2_i16(scp, pack_i16(s[0], s[1]), 0);
    M = dot2_i16(scp, s16, 0);
    a = fp16_bits_to_f32(w.d) * xd;
    b = (float)(S - 4 * M);
}
__device__ __forceinline__ void kq_pair(const KqW<T_IQ4_XS> &w, int c, const uint32_t y[8], float xd, uint32_t,
                                        float &a, float &b, int &S, int &M) {
    const uint32_t Q[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
    int si = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        si = dot4((int)iq4nl_values(Q[k] & 0x0F0F0F0Fu), (int)y[k], si);
        si = dot4((int)iq4nl_values((Q[k] >> 4) & 0x0F0F0F0Fu), (int)y[4 + k], si);
    }
    const uint32_t sh = w.rec.x >> 16;
    const int ls = (int)(((w.rec.y >> (4 * c)) & 0xFu) | (((sh >> (2 * c)) & 3u) << 4));
    a = fp16_bits_to_f32(w.rec.x & 0xFFFFu) * (float)(ls - 32) * xd;
    b = (float)si;
    S = si;
    M = 0;
}

// the tensor of global tile g in a multi-tensor launch
__device__ __forceinline__ int kq_tensor_of(const MvArgs &a, int64_t g) {
    int ti = 0;
#pragma unroll
    for (int k = 1; k < 4; ++k)
        if (k < a.nt && g >= a.t[k].gfirst) ti = k;
    return ti;
}

// Workgroup = TPW tiles x S wavefronts per tile (wavefront ks of a tile takes its ks-th run of
// ceil(steps / S) steps); grid = (tiles over all tensors / TPW, token slots).
template <int TYPE, int R, int TPW, int S, bool DUMP>
__global__ __launch_bounds__(64 * TPW * S) void kq_mv_kernel(MvArgs a) {
    constexpr int WPG = TPW * S;
    constexpr int TB = kq_tile(TYPE);
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ts = wave / S, ks = wave - ts * S;
    const int r = lane >> 3, c = lane & 7;
    const int nb = a.nb, nst = a.nb, nb32 = 8 * a.nb;
    const int tok = blockIdx.y;
    const int64_t tile = (int64_t)blockIdx.x * TPW + ts;
    const bool live = tile < a.groups;
    const int64_t tc = live ? tile : a.groups - 1;
    const int ti = kq_tensor_of(a, tc);
    const uint32_t lt = (uint32_t)(tc - a.t[ti].gfirst), tpm = (uint32_t)a.t[ti].gpm;
    const uint32_t mi = (a.sel ? (uint32_t)a.sel[tok] : 0u) + lt / tpm, tt = lt % tpm;
    const int nsw = (nst + S - 1) / S, s0 = ks * nsw;
    const int nsl = max(0, min(nst, s0 + nsw) - s0), sl = max(nsl - 1, 0);
    const size_t sstride = (size_t)tpm * TB;
    const uint8_t *T0 = a.t[ti].W + (((size_t)mi * nst + min(s0, nst - 1)) * tpm + tt) * TB;

    const float *x = a.x + (size_t)(tok / a.xdiv) * a.ldx;
    KqX xv;
    kq_xload<WPG>(x, nb32, 0, xv);
    KqW<TYPE> ring[R];
#pragma unroll
    for (int k = 0; k < R; ++k) kq_load(T0 + (size_t)min(k, sl) * sstride, (uint32_t)lane, ring[k], k < nsl);
    uint8_t *act = smem;
    kq_xfinish<WPG>(x, nb, xv, act);
    __syncthreads();

    const float *ad = (const float *)(act + kq_off_d(nb));
    const uint32_t *as = (const uint32_t *)(act + kq_off_s(nb));
    const int64_t rows = a.t[ti].rows, mrow = (int64_t)tt * 8;
    const int64_t obase = (int64_t)(lt / tpm) * rows;
    const bool row_ok = live && mrow + r < rows;
    uint8_t *rec = smem + kq_act_bytes(nb) + (size_t)ts * (nst - nsw) * KQ_REC;
    float acc = 0.0f;

    auto step = [&](const KqW<TYPE> &w, int st) {
        const int blk = 8 * st + c;
        const uint4 y0 = *(const uint4 *)(act + (size_t)32 * blk), y1 = *(const uint4 *)(act + (size_t)32 * blk + 16);
        const uint32_t y[8] = {y0.x, y0.y, y0.z, y0.w, y1.x, y1.y, y1.z, y1.w};
        float fa, fb;
        int Si, Mi;
        kq_pair(w, c, y, ad[blk], as[blk], fa, fb, Si, Mi);
        if (S == 1 || ks == 0) {  // lane 8r: the row's chain over its 8 blocks, in order
            acc = __builtin_fmaf(fa, fb, acc);
#pragma unroll
            for (int k = 1; k < 8; ++k) acc = __builtin_fmaf(shl_f32(fa, k), shl_f32(fb, k), acc);
        } else {
            ((float2 *)(rec + (size_t)(st - nsw) * KQ_REC))[lane] = make_float2(fa, fb);
        }
        if (DUMP && row_ok) {
            const size_t di = (size_t)(obase + mrow + r) * nb32 + blk;
            a.dump_s[di] = Si;
            a.dump_m[di] = Mi;
        }
    };
    // whole rounds of R steps, refilling the ring; the last round's refills past the wavefront's
    // last step load nothing; then the last nsl % R steps
    int b0 = 0;
    for (; b0 + R <= nsl; b0 += R) {
#pragma unroll
        for (int k = 0; k < R; ++k) {
            step(ring[k], s0 + b0 + k);
            kq_load(T0 + (size_t)min(b0 + k + R, sl) * sstride, (uint32_t)lane, ring[k], b0 + k + R <= sl);
        }
    }
#pragma unroll
    for (int k = 0; k < R - 1; ++k)
        if (b0 + k < nsl) step(ring[k], s0 + b0 + k);  // uniform

    if (S > 1) {
        __syncthreads();
        if (ks != 0) return;
        // the chains over the other wavefronts' steps (the row's 8 pairs of a step: 64 B)
        for (int st = nsw; st < nst; ++st) {
            const float4 *p = (const float4 *)(rec + (size_t)(st - nsw) * KQ_REC + 64 * r);
            const float4 v0 = p[0], v1 = p[1], v2 = p[2], v3 = p[3];
            acc = __builtin_fmaf(v0.x, v0.y, acc);
            acc = __builtin_fmaf(v0.z, v0.w, acc);
            acc = __builtin_fmaf(v1.x, v1.y, acc);
            acc = __builtin_fmaf(v1.z, v1.w, acc);
            acc = __builtin_fmaf(v2.x, v2.y, acc);
            acc = __builtin_fmaf(v2.z, v2.w, acc);
            acc = __builtin_fmaf(v3.x, v3.y, acc);
            acc = __builtin_fmaf(v3.z, v3.w, acc);
        }
    }
    if (row_ok && c == 0) a.t[ti].y[(size_t)tok * a.ldy + obase + mrow + r] = acc;
}

// ---- upload: file rows -> tiles, one thread per destination byte ----
// value l of 32-block c of a file block (Q2_K / Q3_K low bit pairs, qs at qoff)
__device__ __forceinline__ int kq_lo(const uint8_t *p, int qoff, int c, int l) {
    return (p[qoff + 32 * (c >> 2) + l] >> (2 * (c & 3))) & 3;
}
__global__ void kq_relayout_kernel(int type, const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, int64_t rows,
                                   int nb, int64_t gpm, int64_t total, int64_t row_bytes) {
    const int TB = kq_tile(type), BB = kq_block_bytes(type);
    for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < total; o += (int64_t)gridDim.x * blockDim.x) {
        const int64_t t = o / TB;  // = (m * nb + blk) * gpm + gl
        const int ob = (int)(o - t * TB);
        const int64_t mt = t / gpm, gl = t - mt * gpm;
        const int64_t m = mt / nb;
        const int blk = (int)(mt - m * nb);
        int r, v = 0;
        const uint8_t *p = nullptr;
        auto row_block = [&](int rr) {
            const int64_t row = gl * 8 + rr;
            return row < rows ? src + (m * rows + row) * row_bytes + (int64_t)blk * BB : nullptr;
        };
        if (type != T_IQ4_XS && ob < 512) {  // quant dwords: byte b of dword u, bit pair t = value 16u + 4t + b
            const int L = ob >> 3, u = (ob >> 2) & 1, bb = ob & 3, cc = L & 7;
            if ((p = row_block(L >> 3)))
                for (int t2 = 0; t2 < 4; ++t2) v |= kq_lo(p, type == T_Q2_K ? 16 : 32, cc, 16 * u + 4 * t2 + bb) << (2 * t2);
        } else if (type == T_Q2_K) {
            if (ob < 640) {  // scale bytes 2c, 2c+1
                const int L = (ob - 512) >> 1;
                if ((p = row_block(L >> 3))) v = p[2 * (L & 7) + (ob & 1)];
            } else {         // d, dmin
                r = (ob - 640) >> 2;
                if ((p = row_block(r))) v = p[80 + ((ob - 640) & 3)];
            }
        } else if (type == T_Q3_K) {
            if (ob < 768) {  // high bits: bit 8b + 4u + t of lane L's dword = hmask bit c of value 16u + 4t + b
                const int L = (ob - 512) >> 2, bb = (ob - 512) & 3, cc = L & 7;
                if ((p = row_block(L >> 3)))
                    for (int sb = 0; sb < 8; ++sb) v |= ((p[16 * (sb >> 2) + 4 * (sb & 3) + bb] >> cc) & 1) << sb;
            } else if (ob < 864) {  // the 12 packed scale bytes
                r = (ob - 768) / 12;
                if ((p = row_block(r))) v = p[96 + (ob - 768) % 12];
            } else {  // d
                r = (ob - 864) >> 1;
                if ((p = row_block(r))) v = p[108 + ((ob - 864) & 1)];
            }
        } else {  // IQ4_XS
            if (ob < 1024) {
                const int L = ob >> 4;
                if ((p = row_block(L >> 3))) v = p[8 + 16 * (L & 7) + (ob & 15)];
            } else {
                r = (ob - 1024) >> 3;
                if ((p = row_block(r))) v = p[(ob - 1024) & 7];
            }
        }
        dst[o] = (uint8_t)v;
    }
}

// ---- host side ----
size_t kq_lds_bytes(int nb) { return kq_act_bytes(nb); }
static int kq_tpw(int s) { return s == 1 ? 4 : s <= 4 ? 2 : 1; }
static size_t kq_lds(int nb, int tpw, int s) {
    const int nsw = (nb + s - 1) / s;
    return kq_act_bytes(nb) + (s > 1 ? (size_t)tpw * (nb - nsw) * KQ_REC : 0);
}
// launches of fewer than 768 tiles (tiles x tokens) split the steps of a tile over up to 8
// wavefronts while the launch stays within 2048 wavefronts, each wavefront keeps 4 steps or more,
// the records fit the LDS and every workgroup is resident at once; ring depth 4 (measured at
// 4096 -> 14336: 8.6 us for Q2_K against 9.7 with 2 and 8.6 with 8; 2 wins nowhere: a step here
// is 672 - 1088 bytes of a tile, a third to a half of a Q4_K step's)
MvShape kq_matvec_shape(int, int64_t tiles, int nb, int num_cu) {
    int S = 1;
    if (tiles < 768)
        while (S < 8 && tiles * 2 * S <= 2048 && nb >= 8 * S && kq_lds(nb, kq_tpw(2 * S), 2 * S) <= GEMM_LDS_MAX &&
               all_resident((tiles + kq_tpw(2 * S) - 1) / kq_tpw(2 * S), 2 * S * kq_tpw(2 * S),
                            kq_lds(nb, kq_tpw(2 * S), 2 * S), num_cu))
            S *= 2;
    return MvShape{S, 4, kq_tpw(S), kq_lds(nb, kq_tpw(S), S)};
}

template <int TYPE, int R, int TPW, int S>
static hipError_t kq_launch(const MvArgs &a, int ntok, size_t lds, hipStream_t s) {
    const unsigned wg = (unsigned)((a.groups + TPW - 1) / TPW);
    if (a.dump_s) kq_mv_kernel<TYPE, R, TPW, S, true><<<dim3(wg, ntok), 64 * TPW * S, lds, s>>>(a);
    else kq_mv_kernel<TYPE, R, TPW, S, false><<<dim3(wg, ntok), 64 * TPW * S, lds, s>>>(a);
    return hipGetLastError();
}
template <int TYPE>
static hipError_t kq_launch_type(const MvArgs &a, int ntok, int num_cu, hipStream_t s) {
    const MvShape sh = kq_matvec_shape(TYPE, a.groups * ntok, a.nb, num_cu);
    if (sh.lds > (sh.S == 1 ? (size_t)65536 : GEMM_LDS_MAX)) return hipErrorInvalidValue;
    switch (sh.S) {
    case 1: return kq_launch<TYPE, 4, 4, 1>(a, ntok, sh.lds, s);
    case 2: return kq_launch<TYPE, 4, 2, 2>(a, ntok, sh.lds, s);
    case 4: return kq_launch<TYPE, 4, 2, 4>(a, ntok, sh.lds, s);
    default: return kq_launch<TYPE, 4, 1, 8>(a, ntok, sh.lds, s);
    }
}
hipError_t launch_kq_matvec(int type, const MvArgs &a, int ntok, int num_cu, hipStream_t s) {
    if (a.nb < 1 || a.ntile != a.nb) return hipErrorInvalidValue;
    switch (type) {
    case T_Q2_K: return kq_launch_type<T_Q2_K>(a, ntok, num_cu, s);
    case T_Q3_K: return kq_launch_type<T_Q3_K>(a, ntok, num_cu, s);
    case T_IQ4_XS: return kq_launch_type<T_IQ4_XS>(a, ntok, num_cu, s);
    default: return hipErrorInvalidValue;
    }
}
hipError_t launch_kq_relayout(int type, const uint8_t *src, uint8_t *dst, int64_t rows, int nb, int64_t gpm,
                              int64_t total, int64_t row_bytes, hipStream_t s) {
    if (!kq_kind(type)) return hipErrorInvalidValue;
    const int64_t want = (total + 255) / 256;
    const unsigned grid = (unsigned)(want < 65536 ? want : 65536);
    kq_relayout_kernel<<<grid, 256, 0, s>>>(type, src, dst, rows, nb, gpm, total, row_bytes);
    return hipGetLastError();
}

}  // namespace fgh
