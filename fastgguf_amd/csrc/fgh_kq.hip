// fgh_kq.hip - the decode matvec for the 256-value types on Q8 activations: Q2_K, Q3_K and IQ4_XS
// (dot_q2_K_q8 fastgguf.c:1426-1479, dot_q3_K_q8 1481-1545, dot_iq4_xs_q8 1580-1614; the
// reference's own GPU path leaves these types on the CPU, gpu_kernel_for 1744-1751).
//
// Each of these row kernels runs ONE fp32 chain per row over the row's 32-value blocks in order;
// the integers of a 32-block are exact. So a wavefront takes 16 rows of one 256-value block per
// step and lane L = 4 r + j takes 32-blocks c = 2j and 2j + 1 of row r: it forms each block's
// integers alone, from its own bytes and the block's 32 LDS activations, and reduces them to the
// chain's two factors (a_c, b_c); lane 4 r then gathers the row's other 6 pairs from its quad
// by DPP and runs the chain over the 8, block after block:
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
// Tiles: 16 rows of one block, step-major like the other types (step s of row tile t of matrix m
// at ((m * steps + s) * tpm + t) * tile bytes). Value l of 32-block c = 4 n + j' is, in the
// file, bit pair j' of qs[32 n + l] (Q2_K, Q3_K); in a tile, a block's two quant dwords hold it
// as bit pair t of byte b of dword u, l = 16 u + 4 t + b, so (dword u >> 2 t) & 0x03030303 is the
// four values that meet activation dword 4 u + t. Lane L's 16 bytes are block 2j's two dwords,
// then block 2j + 1's:
//   Q2_K tile 1344 B:   [0, 1024) quants, lane L at 16 L; [1024, 1280) the row's scale bytes
//                       4j .. 4j + 3 (the same file bytes) at 1024 + 4 L; [1280, 1344) fp16 d,
//                       dmin of row r at 1280 + 4 r
//   Q3_K tile 1760 B:   [0, 1024) low bit pairs as Q2_K; [1024, 1536) high bits, lane L's two
//                       dwords at 1024 + 8 L (block 2j, then 2j + 1; bit 8 b + 4 u + t = hmask bit
//                       c of value 16 u + 4 t + b); [1536, 1728) the row's 12 packed scale bytes
//                       at 1536 + 12 r; [1728, 1760) fp16 d of row r at 1728 + 2 r
//   IQ4_XS tile 2176 B: [0, 2048) nibbles, lane L at 32 L (file qs[32 j .. 32 j + 31]);
//                       [2048, 2176) file bytes 0..7 of row r (d, scales_h, scales_l) at 2048 + 8 r
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
constexpr int KQ_REC = 1024;  // a parked step: 64 lanes x {a, b} of their two blocks

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

// ---- one lane's bytes of one step (its two 32-blocks c = 2j, 2j + 1 of one row) ----
template <int TYPE>
struct KqW;
template <>
struct KqW<T_Q2_K> {
    uint4 q;          // quant dwords: .xy block 2j, .zw block 2j + 1
    uint32_t sc, dd;  // scale bytes 4j .. 4j + 3; fp16 d | dmin << 16
};
template <>
struct KqW<T_Q3_K> {
    uint4 q;                // low bit pairs as Q2_K's
    uint2 h;                // high bits of blocks 2j, 2j + 1
    uint32_t slo, shi, d;   // scale bytes 4 (j & 1) .. + 3 and 8 .. 11 of the 12; fp16 d
};
template <>
struct KqW<T_IQ4_XS> {
    uint4 q0, q1;  // nibbles of blocks 2j, 2j + 1
    uint2 rec;     // fp16 d | scales_h << 16, scales_l
};
// T: the tile (wavefront-uniform); live = false: zeros without a memory access
__device__ __forceinline__ void kq_load(const uint8_t *T, uint32_t lane, KqW<T_Q2_K> &w, bool live) {
    const BufRes r = buf_res(T, live ? kq_tile(T_Q2_K) : 0);
    w.q = bld16<WNT>(r, 16 * lane);
    w.sc = bld4<WNT>(r, 1024 + 4 * lane);
    w.dd = bld4<WNT>(r, 1280 + 4 * (lane >> 2));
}
__device__ __forceinline__ void kq_load(const uint8_t *T, uint32_t lane, KqW<T_Q3_K> &w, bool live) {
    const BufRes r = buf_res(T, live ? kq_tile(T_Q3_K) : 0);
    const uint32_t rr = lane >> 2, j = lane & 3;
    w.q = bld16<WNT>(r, 16 * lane);
    w.h = bld8<WNT>(r, 1024 + 8 * lane);
    w.slo = bld4<WNT>(r, 1536 + 12 * rr + 4 * (j & 1));
    w.shi = bld4<WNT>(r, 1536 + 12 * rr + 8);
    w.d = bld2<WNT>(r, 1728 + 2 * rr);
}
__device__ __forceinline__ void kq_load(const uint8_t *T, uint32_t lane, KqW<T_IQ4_XS> &w, bool live) {
    const BufRes r = buf_res(T, live ? kq_tile(T_IQ4_XS) : 0);
    w.q0 = bld16<WNT>(r, 32 * lane);
    w.q1 = bld16<WNT>(r, 32 * lane + 16);
    w.rec = bld8<WNT>(r, 2048 + 8 * (lane >> 2));
}

// the sums of q * y over values 0..15 and 16..31 of a block whose quant dwords are D0, D1 (bit
// pair t of byte b of dword u: value 16 u + 4 t + b) and whose high-bit dword is H (Q3_K: bit
// 8 b + 4 u + t; H = 0: none); y = the block's 8 activation dwords
__device__ __forceinline__ void kq_halves(uint32_t D0, uint32_t D1, uint32_t H, const uint32_t y[8], int s[2]) {
    const uint32_t D[2] = {D0, D1};
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        int acc = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t q = ((D[u] >> (2 * t)) & 0x03030303u) | (((H >> (4 * u + t)) & 0x01010101u) << 2);
            acc = dot4((int)q, (int)y[4 * u + t], acc);
        }
        s[u] = acc;  // |s| <= 16 * 7 * 127: an int16
    }
}
// the chain factors (a, b) of block h (c = 2j + h) of the lane's pair, and its integers (for the
// dump): y = the block's 8 activation dwords, xd its scale, s16 its two half sums (int16 pair)
__device__ __forceinline__ void kq_pair(const KqW<T_Q2_K> &w, int, int h, const uint32_t y[8], float xd, uint32_t s16,
                                        float &a, float &b, int &S, int &M) {
    int s[2];
    kq_halves(h ? w.q.z : w.q.x, h ? w.q.w : w.q.y, 0u, y, s);
    const uint32_t b2 = w.sc >> (16 * h);  // scale bytes 2c, 2c + 1
    const uint32_t sc = b2 & 0x0F0Fu, mn = (b2 >> 4) & 0x0F0Fu;  // bytes -> (lo, hi) int16 pairs
    S = dot2_i16((sc & 0xFu) | ((sc >> 8) << 16), pack_i16(s[0], s[1]), 0);
    M = dot2_i16((mn & 0xFu) | ((mn >> 8) << 16), s16, 0);
    const float d = fp16_bits_to_f32(w.dd & 0xFFFFu), dmin = fp16_bits_to_f32(w.dd >> 16);
    a = xd;
    b = __builtin_fmaf(d, (float)S, -(dmin * (float)M));
}
__device__ __forceinline__ void kq_pair(const KqW<T_Q3_K> &w, int j, int h, const uint32_t y[8], float xd, uint32_t s16,
                                        float &a, float &b, int &S, int &M) {
    int s[2];
    kq_halves(h ? w.q.z : w.q.x, h ? w.q.w : w.q.y, h ? w.h.y : w.h.x, y, s);
    // scales 2c, 2c + 1 (c = 2j + h): low nibbles j / 2 of bytes (2c) % 8, + 1 (bytes 2h, 2h + 1 of
    // slo); high bit pairs 2j of bytes 8 + (2c) % 4, + 1 (bytes 2h, 2h + 1 of shi)
    const uint32_t lo = w.slo >> (16 * h), hi = w.shi >> (16 * h);
    const int ln = 4 * (j >> 1), hs = 2 * j;
    const int sa = (int)(((lo >> ln) & 0xFu) | (((hi >> hs) & 3u) << 4)) - 32;
    const int sb = (int)(((lo >> (8 + ln)) & 0xFu) | (((hi >> (8 + hs)) & 3u) << 4)) - 32;
    const uint32_t scp = pack_i16(sa, sb);
    S = dot2_i16(scp, pack_i16(s[0], s[1]), 0);
    M = dot2_i16(scp, s16, 0);
    a = fp16_bits_to_f32(w.d) * xd;
    b = (float)(S - 4 * M);
}
__device__ __forceinline__ void kq_pair(const KqW<T_IQ4_XS> &w, int j, int h, const uint32_t y[8], float xd, uint32_t,
                                        float &a, float &b, int &S, int &M) {
    const uint4 q = h ? w.q1 : w.q0;
    const uint32_t Q[4] = {q.x, q.y, q.z, q.w};
    int si = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        si = dot4((int)iq4nl_values(Q[k] & 0x0F0F0F0Fu), (int)y[k], si);
        si = dot4((int)iq4nl_values((Q[k] >> 4) & 0x0F0F0F0Fu), (int)y[4 + k], si);
    }
    const int c = 2 * j + h;
    const uint32_t sh = w.rec.x >> 16;
    const int ls = (int)(((w.rec.y >> (4 * c)) & 0xFu) | (((sh >> (2 * c)) & 3u) << 4));
    a = fp16_bits_to_f32(w.rec.x & 0xFFFFu) * (float)(ls - 32) * xd;
    b = (float)si;
    S = si;
    M = 0;
}
// lane k of the lane's quad (DPP quad_perm [k, k, k, k])
__device__ __forceinline__ float quad_f32(float v, int k) {
    const int iv = __builtin_bit_cast(int, v);
    int o;
    switch (k) {
    case 1: o = __builtin_amdgcn_update_dpp(0, iv, 0x55, 0xF, 0xF, false); break;
    case 2: o = __builtin_amdgcn_update_dpp(0, iv, 0xAA, 0xF, 0xF, false); break;
    default: o = __builtin_amdgcn_update_dpp(0, iv, 0xFF, 0xF, 0xF, false); break;
    }
    return __builtin_bit_cast(float, o);
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
    const int r = lane >> 2, j = lane & 3;
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

    const int64_t rows = a.t[ti].rows, mrow = (int64_t)tt * KQ_TILE_ROWS;
    const int64_t obase = (int64_t)(lt / tpm) * rows;
    const bool row_ok = live && mrow + r < rows;
    uint8_t *rec = smem + kq_act_bytes(nb) + (size_t)ts * (nst - nsw) * KQ_REC;
    float acc = 0.0f;

    auto step = [&](const KqW<TYPE> &w, int st) {
        const int blk = 8 * st + 2 * j;  // the lane's first block: blk, blk + 1 are contiguous in LDS
        const uint4 *yp = (const uint4 *)(act + (size_t)32 * blk);
        const uint4 y0 = yp[0], y1 = yp[1], y2 = yp[2], y3 = yp[3];
        const uint32_t ya[8] = {y0.x, y0.y, y0.z, y0.w, y1.x, y1.y, y1.z, y1.w};
        const uint32_t yb[8] = {y2.x, y2.y, y2.z, y2.w, y3.x, y3.y, y3.z, y3.w};
        const float2 xd = *(const float2 *)(act + kq_off_d(nb) + 4 * (size_t)blk);
        const uint2 s16 = *(const uint2 *)(act + kq_off_s(nb) + 4 * (size_t)blk);
        float a0, b0, a1, b1;
        int S0, M0, S1, M1;
        kq_pair(w, j, 0, ya, xd.x, s16.x, a0, b0, S0, M0);
        kq_pair(w, j, 1, yb, xd.y, s16.y, a1, b1, S1, M1);
        if (S == 1 || ks == 0) {  // lane 4r: the row's chain over its 8 blocks, in order
            acc = __builtin_fmaf(a0, b0, acc);
            acc = __builtin_fmaf(a1, b1, acc);
#pragma unroll
            for (int k = 1; k < 4; ++k) {
                acc = __builtin_fmaf(quad_f32(a0, k), quad_f32(b0, k), acc);
                acc = __builtin_fmaf(quad_f32(a1, k), quad_f32(b1, k), acc);
            }
        } else {
            ((float4 *)(rec + (size_t)(st - nsw) * KQ_REC))[lane] = make_float4(a0, b0, a1, b1);
        }
        if (DUMP && row_ok) {
            const size_t di = (size_t)(obase + mrow + r) * nb32 + blk;
            a.dump_s[di] = S0;
            a.dump_m[di] = M0;
            a.dump_s[di + 1] = S1;
            a.dump_m[di + 1] = M1;
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
        // the chains over the other wavefronts' steps (the row's 8 pairs of a step: 64 B), the
        // records of 4 steps read before their 32 fmas (one LDS round trip per 4 steps), then
        // the last steps one at a time
        auto chain8 = [&](const float4 (&v)[4]) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                acc = __builtin_fmaf(v[q].x, v[q].y, acc);
                acc = __builtin_fmaf(v[q].z, v[q].w, acc);
            }
        };
        int st = nsw;
        for (; st + 4 <= nst; st += 4) {
            float4 v[4][4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float4 *p = (const float4 *)(rec + (size_t)(st + u - nsw) * KQ_REC + 64 * r);
#pragma unroll
                for (int q = 0; q < 4; ++q) v[u][q] = p[q];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) chain8(v[u]);
        }
        for (; st < nst; ++st) {
            const float4 *p = (const float4 *)(rec + (size_t)(st - nsw) * KQ_REC + 64 * r);
            const float4 v[4] = {p[0], p[1], p[2], p[3]};
            chain8(v);
        }
    }
    if (row_ok && j == 0) a.t[ti].y[(size_t)tok * a.ldy + obase + mrow + r] = acc;
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
        int v = 0;
        const uint8_t *p = nullptr;
        auto row_block = [&](int rr) {
            const int64_t row = gl * KQ_TILE_ROWS + rr;
            return row < rows ? src + (m * rows + row) * row_bytes + (int64_t)blk * BB : nullptr;
        };
        if (type != T_IQ4_XS && ob < 1024) {
            // lane L = 4 r + j, byte bo of its 16: block 2j + (bo >> 3), dword u, byte b; bit pair t
            // = value 16 u + 4 t + b
            const int L = ob >> 4, bo = ob & 15, u = (bo >> 2) & 1, bb = bo & 3, cc = 2 * (L & 3) + (bo >> 3);
            if ((p = row_block(L >> 2)))
                for (int t2 = 0; t2 < 4; ++t2) v |= kq_lo(p, type == T_Q2_K ? 16 : 32, cc, 16 * u + 4 * t2 + bb) << (2 * t2);
        } else if (type == T_Q2_K) {
            if (ob < 1280) {  // scale bytes 4j .. 4j + 3
                const int L = (ob - 1024) >> 2;
                if ((p = row_block(L >> 2))) v = p[4 * (L & 3) + (ob & 3)];
            } else {          // d, dmin
                if ((p = row_block((ob - 1280) >> 2))) v = p[80 + (ob & 3)];
            }
        } else if (type == T_Q3_K) {
            if (ob < 1536) {  // high bits: byte bo of lane L's 8, block 2j + (bo >> 2), byte b; bit
                              // 8 b + 4 u + t = hmask bit c of value 16 u + 4 t + b
                const int L = (ob - 1024) >> 3, bo = (ob - 1024) & 7, bb = bo & 3, cc = 2 * (L & 3) + (bo >> 2);
                if ((p = row_block(L >> 2)))
                    for (int sb = 0; sb < 8; ++sb) v |= ((p[16 * (sb >> 2) + 4 * (sb & 3) + bb] >> cc) & 1) << sb;
            } else if (ob < 1728) {  // the 12 packed scale bytes
                if ((p = row_block((ob - 1536) / 12))) v = p[96 + (ob - 1536) % 12];
            } else {  // d
                if ((p = row_block((ob - 1728) >> 1))) v = p[108 + (ob & 1)];
            }
        } else {  // IQ4_XS
            if (ob < 2048) {  // lane L's 32 bytes: file qs[32 j .. 32 j + 31]
                const int L = ob >> 5;
                if ((p = row_block(L >> 2))) v = p[8 + 32 * (L & 3) + (ob & 31)];
            } else {
                if ((p = row_block((ob - 2048) >> 3))) v = p[(ob - 2048) & 7];
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
// the split: while the launch stays within 4096 wavefronts whose steps are 6.5 MB in all, each
// wavefront keeps 2 steps or more, the records fit the LDS and every workgroup is resident at
// once, the steps of a tile split over twice the wavefronts (up to 8); ring depth 2 for split
// launches, 4 for whole rows. Measured (graph of back-to-back launches over >= 512 MB of copies,
// every S in {1, 2, 4, 8} x R in {2, 4, 8}): at 14336 x 4096 the fastest were (S 4, R 2) for
// Q2_K and Q3_K (8.6 -> 7.6 us, 9.9 -> 9.0 us against whole rows at R 4) and (S 2, R 2) for
// IQ4_XS's larger steps (11.4 -> 10.0 us); at 4096 x 14336 and 4096 x 4096 (S 8, R 2) for all three.
MvShape kq_matvec_shape(int type, int64_t tiles, int nb, int num_cu) {
    int S = 1;
    while (S < 8 && tiles * 2 * S <= 4096 && tiles * 2 * S * kq_tile(type) <= 6500000 && nb >= 4 * S &&
           kq_lds(nb, kq_tpw(2 * S), 2 * S) <= GEMM_LDS_MAX &&
           all_resident((tiles + kq_tpw(2 * S) - 1) / kq_tpw(2 * S), 2 * S * kq_tpw(2 * S),
                        kq_lds(nb, kq_tpw(2 * S), 2 * S), num_cu))
        S *= 2;
    return MvShape{S, S > 1 ? 2 : 4, kq_tpw(S), kq_lds(nb, kq_tpw(S), S)};
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
    case 2: return kq_launch<TYPE, 2, 2, 2>(a, ntok, sh.lds, s);
    case 4: return kq_launch<TYPE, 2, 2, 4>(a, ntok, sh.lds, s);
    default: return kq_launch<TYPE, 2, 1, 8>(a, ntok, sh.lds, s);
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
