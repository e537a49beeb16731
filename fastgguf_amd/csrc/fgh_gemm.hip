// fgh_gemm.hip - the prompt-batch (8..64 tokens) Q4_K x Q8_K matmul on gfx950 int8 MFMA
// (the reference's matmul -> gemm_kquant path, fastgguf.c:2818-2854 and 3004-3031).
//
// Y[tok * ldy + row] = sum_b yd[tok][b] * (d[row][b] * isum - dmin[row][b] * msum), with the exact
// per-block integers of the reference (dot_q4_K_q8k, fastgguf.c:1118-1176):
//   isum = sum_g sc_g * sum_{32 values of g} q * y        msum = sum_g m_g * (bs_2g + bs_2g+1)
//
// The 6-bit sub-block scale does not fit an int8 operand together with the 4-bit quant
// (q * sc <= 945), so it is split, sc = 8 sh + sl with sh, sl <= 7, and two v_mfma_i32_32x32x32_i8
// passes run per 32-value group on pre-scaled weights q*sh and q*sl (both <= 105): every group of
// a block accumulates into the same two accumulators, and isum = 8 Chi + Clo exactly, with no
// per-group vector work. msum comes from two v_mfma_i32_32x32x16_i8 on the block's eight 32-value
// activation sums split into bytes (bs = bl + 128 bh, bl in [0,127], bh in [-32,31]) against the
// row's eight 6-bit mins: msum = C1 + 128 C2.
//
// MFMA roles: A = activations (M = 32 tokens), B = weights (N = 32 rows). Lane l holds row
// l % 32 of the output tile and 16 tokens 8 (v / 4) + 4 (l / 32) + v % 4, v = 0..15, so a row's
// d, dmin, scales and mins are per-lane constants. Both operands give lane l the 16 consecutive
// values 32 g + 16 (l / 32) + i of a group, so the products pair up whatever order the hardware
// uses inside one K step.
//
// Weights are read in the decode layout (fgh_q4k.hip): the GEMM needs no second copy. A
// workgroup owns 64 rows (4 tiles) and all tokens: 4 * NTW wavefronts = 2 slices of 32 rows x 2
// halves of the blocks (even / odd) x NTW tiles of 32 tokens. It walks the blocks in steps of two:
// the step's weights for all 64 rows (18 KB) are staged in LDS by the whole workgroup with
// coalesced loads (1 KB contiguous per wavefront load) and read back as MFMA fragments; activations are read
// straight from global memory in a fragment-ordered layout (1 KB contiguous per load). Both are
// double-buffered one step ahead. The two halves of the blocks are added at the end through LDS.
//
// fp32 order: per (row, token) and block t = d * float(isum) - dmin * float(msum) (one fma),
// acc = fma(yd, t, acc) over the wavefront's blocks, out = acc_even + acc_odd. The integers are
// exact; the fp32 result differs from gemmk_kern's order (fastgguf.c:2765-2797) only by rounding.
#include "fgh_internal.h"

namespace fgh {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------------------------
// Activation quantizer for the GEMM (quantize_q8k, fastgguf.c:773-793, bit-exact): one wavefront
// per (token, 256-block); lane l holds values 4l..4l+3 (group g = l / 8, half h = (l / 4) % 2).
// Writes, with NTT = Tp / 32 token tiles and token t = 32 tt + n:
//   qs  [nb][NTT][8][2][32][16] int8: values 32 g + 16 h .. + 15 of token t at
//                    ((((b NTT + tt) 8 + g) 2 + h) 32 + n) 16, so the MFMA fragment of (tt, g) is
//                    1 KB contiguous in lane order (lane = 32 h + n)
//   ydT [nb][Tp]     fp32 block scales, token-minor (one float4 = 4 consecutive tokens)
//   bsp [nb][2][32][NTT][8] int8: the 32-value sums bs_g = bsums[2g] + bsums[2g+1] of token t as
//                    bl_g = bs & 127 at [0][n][tt][g] and bh_g = bs >> 7 at [1][n][tt][g]: MFMA
//                    lane (n, h) reads its 8 bytes of every token tile at once, lanes contiguous
// Tokens T..Tp-1 are written as zeros. The block maximum is a DPP reduction within each row of
// 16 lanes and then across the four rows; the group sums a DPP reduction over 8 lanes.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void gemm_quant_kernel(const float *__restrict__ x, int64_t ldx, int nb, int T,
                                                         int Tp, int8_t *__restrict__ qs, float *__restrict__ ydT,
                                                         int8_t *__restrict__ bsp) {
    const int lane = threadIdx.x & 63;
    const int b = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int tok = blockIdx.y;
    if (b >= nb) return;  // whole wavefront leaves together
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (tok < T) v = *(const float4 *)(x + (size_t)tok * ldx + (size_t)b * 256 + 4 * lane);
    // the block maximum as the reference forms it (a NaN never replaces the running maximum:
    // fmaxf keeps the other operand)
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
#define FGH_ROR(f, ctrl) __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, f), ctrl, 0xF, 0xF, false))
    amax = fmaxf(amax, FGH_ROR(amax, 0x128));  // row_ror 8, 4, 2, 1: every lane of a row of 16
    amax = fmaxf(amax, FGH_ROR(amax, 0x124));
    amax = fmaxf(amax, FGH_ROR(amax, 0x122));
    amax = fmaxf(amax, FGH_ROR(amax, 0x121));
#undef FGH_ROR
    auto lane_f = [&](int l) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, amax), l)); };
    amax = fmaxf(fmaxf(lane_f(0), lane_f(16)), fmaxf(lane_f(32), lane_f(48)));
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    const int q0 = q8_round(v.x * id), q1 = q8_round(v.y * id);
    const int q2 = q8_round(v.z * id), q3 = q8_round(v.w * id);
    const int ntt = Tp >> 5, n = tok & 31, tt = tok >> 5, g = lane >> 3, h = (lane >> 2) & 1;
    *(uint32_t *)(qs + (((((size_t)b * ntt + tt) * 8 + g) * 2 + h) * 32 + n) * 16 + 4 * (lane & 3)) =
        pack_q(q0, q1, q2, q3);
    const int s = sum8_i32(q0 + q1 + q2 + q3);  // 32-value group g = lanes 8g..8g+7
    if ((lane & 7) == 0) {
        int8_t *p = bsp + (size_t)b * Tp * 16 + (n * ntt + tt) * 8 + g;
        p[0] = (int8_t)(s & 127);
        p[32 * ntt * 8] = (int8_t)(s >> 7);
    }
    if (lane == 0) ydT[(size_t)b * Tp + tok] = d;
}

// ---------------------------------------------------------------------------------------------
// The GEMM kernel
// ---------------------------------------------------------------------------------------------
// LDS stage of one step (blocks KQ s .. KQ s + KQ - 1), copied from the quantizer's output, where
// those blocks are adjacent: the quants qs [KQ][NTT][8][32][32], and apart from them bsp [KQ][Tp][16]
// followed by ydT [KQ][Tp] (each stage part its own LDS array, so the compiler can tell the stage
// being read from the one being filled)
__host__ __device__ constexpr int gs_q(int Tp, int KQ) { return KQ * Tp * 256; }
__host__ __device__ constexpr int gs_e(int Tp, int KQ) { return KQ * Tp * 20; }
__host__ __device__ constexpr int gs_yd(int Tp, int KQ) { return KQ * Tp * 16; }  // in the e part

// the tile-layout address of (row R over all matrices, block 0): its tile and its row in the tile
// (block b is b * gpm * 2304 further)
__device__ __forceinline__ const uint8_t *gemm_tile(const GemmArgs &a, int64_t R, int &rr) {
    R = R < a.nrows ? R : a.nrows - 1;
    const int64_t mat = R / a.rows, r = R - mat * a.rows;
    rr = (int)(r & 15);
    return a.W + ((size_t)mat * a.nb * a.gpm + (size_t)(r >> 4)) * 2304;
}

// one lane's weights of one block: pieces h (= lane / 32) of the four chunks of its row, and the
// row's meta
struct WOps {
    uint4 q[4], m;
};
__device__ __forceinline__ void w_load(WOps &w, const uint8_t *T, size_t boff, int rr, int h) {
    const uint8_t *p = T + boff;
#pragma unroll
    for (int j = 0; j < 4; ++j) w.q[j] = ld16(p + 256 + 1024 * (h ^ (j >> 1)) + 16 * (4 * rr + j));
    w.m = ld16(p + 16 * rr);
}

// The workgroup's copy of step s into an LDS stage: three contiguous runs of the quantizer's
// output, moved by direct-to-LDS loads (global_load_lds_dwordx4: each lane's 16 bytes land at the
// wavefront's LDS base + 16 * lane, so the stage takes no registers). Completion: vmcnt, then a
// workgroup barrier. Tp tokens, KQ blocks, NT threads.
typedef __attribute__((address_space(3))) uint8_t lds_u8;
// One direct-to-LDS load of 16 bytes per lane (global_load_lds_dwordx4): lane i's bytes land at
// dst + 16 i; dst must be the same in every lane. The compiler builtin sets M0 itself (M0 is a
// register the compiler reserves, so inline assembly that writes it is not safe); completion is
// awaited explicitly (s_dma_wait) before the workgroup barrier that publishes the stage.
__device__ __forceinline__ void dma16(const void *src, uint8_t *dst) {
    __builtin_amdgcn_global_load_lds(src, (lds_u8 *)dst, 16, 0, 0);
}
template <int NT, int Tp, int KQ>
__device__ __forceinline__ void s_dma(const GemmArgs &a, uint8_t *sq, uint8_t *se, int s, int tid, int wave) {
    constexpr int QB = Tp * 16;               // 16-byte units of qs per block
    constexpr int NQ = KQ * QB / NT;          // rounds for the step's blocks
    constexpr int NE = KQ * Tp + KQ * Tp / 4;  // units of bsp (Tp per block) then ydT (Tp / 4)
    static_assert(KQ * QB % NT == 0 && NE <= NT, "stage copy shape");
    const int nb = a.nb;
#pragma unroll
    for (int k = 0; k < NQ; ++k) {
        const int u = tid + k * NT, blk = u / QB;
        const int b = min(KQ * s + blk, nb - 1);  // blocks past the end: the last again (padding)
        const int8_t *src = a.qs + (size_t)b * Tp * 256 + 16 * (u - blk * QB);
        dma16(src, sq + 16 * (k * NT + 64 * wave));
    }
    if (64 * wave < NE) {  // uniform: wavefronts holding bsp / ydT units
        const int e = tid;
        if (e < NE) {
            const void *src;
            if (e < KQ * Tp) {
                const int blk = e / Tp, b = min(KQ * s + blk, nb - 1);
                src = a.bsp + ((size_t)b * Tp + (e - blk * Tp)) * 16;
            } else {
                const int e2 = e - KQ * Tp, blk = e2 / (Tp / 4), b = min(KQ * s + blk, nb - 1);
                src = a.ydT + (size_t)b * Tp + 4 * (e2 - blk * (Tp / 4));
            }
            dma16(src, se + 1024 * wave);
        }
    }
}
// every direct-to-LDS load of this wavefront has landed (s_waitcnt vmcnt(0))
__device__ __forceinline__ void s_dma_wait() { __builtin_amdgcn_s_waitcnt(0x0F70); }

__device__ __forceinline__ v4i u4v(uint4 u) { return v4i{(int)u.x, (int)u.y, (int)u.z, (int)u.w}; }

// bytes of q (each <= 15) times a small factor (<= 7): no carry between bytes, two 16-bit lanes
__device__ __forceinline__ uint32_t bmul(uint32_t q, uint32_t f2) {
    const u16x2 r = __builtin_bit_cast(u16x2, q) * __builtin_bit_cast(u16x2, f2);
    return __builtin_bit_cast(uint32_t, r);
}

// One 256-block of one wavefront for all its NTT token tiles: weights from registers (prepared
// once per group for every tile), activations from the LDS stage (slice blk). live == false: a
// padding block (odd block counts): computed, weighted by zero, not dumped.
template <int NTT, int KQ, bool DUMP>
__device__ __forceinline__ void gemm_block(const WOps &w, const uint8_t *sq, const uint8_t *se, int blk, int n, int h,
                                           float (&acc)[NTT][16], int b, bool live, int64_t row, const GemmArgs &a) {
    const int Tp = NTT * 32;
    const Q4KScales sc = q4k_scales(w.m.y, w.m.z, w.m.w);
    // a padding block contributes zero: its scales are zeroed once here
    const float d = live ? fp16_bits_to_f32(w.m.x & 0xFFFF) : 0.0f;
    const float dmin = live ? fp16_bits_to_f32(w.m.x >> 16) : 0.0f;
    // the split scale factors of the 8 groups as bytes: sh = sc >> 3, sl = sc & 7
    const uint32_t shb[2] = {(sc.sc_lo >> 3) & 0x07070707u, (sc.sc_hi >> 3) & 0x07070707u};
    const uint32_t slb[2] = {sc.sc_lo & 0x07070707u, sc.sc_hi & 0x07070707u};
    // per group g (32 values, sub-block g): the lane's 16 nibbles (chunk g / 2, low or high) times
    // sh (into Ch) and times sl (into Cl) against the activation fragment of every token tile
    // (group g of tile tt: 1 KB contiguous per wavefront in the stage); isum = 8 Ch + Cl
    const uint8_t *qs = sq + (size_t)blk * Tp * 256;
    v16i ch[NTT], cl[NTT];
#pragma unroll
    for (int g = 0; g < 8; ++g) {
        const uint4 pc = w.q[g >> 1];
        const uint32_t P[4] = {pc.x, pc.y, pc.z, pc.w};
        // byte g of the factors into both 16-bit lanes (v_perm_b32; selector 0x0C = zero)
        const uint32_t sel = 0x0C000C00u | (uint32_t)((g & 3) * 0x00010001);
        const uint32_t fh = __builtin_amdgcn_perm(0u, shb[g >> 2], sel), fl = __builtin_amdgcn_perm(0u, slb[g >> 2], sel);
        v4i bh, bl;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t q = (g & 1) ? ((P[k] >> 4) & 0x0F0F0F0Fu) : (P[k] & 0x0F0F0F0Fu);
            bh[k] = (int)bmul(q, fh);
            bl[k] = (int)bmul(q, fl);
        }
#pragma unroll
        for (int tt = 0; tt < NTT; ++tt) {
            const v4i av = u4v(*(const uint4 *)(qs + (((tt * 8 + g) * 2 + h) * 32 + n) * 16));
            if (g == 0) {
                const v16i z = {};
                ch[tt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bh, z, 0, 0, 0);
                cl[tt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bl, z, 0, 0, 0);
            } else {
                ch[tt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bh, ch[tt], 0, 0, 0);
                cl[tt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bl, cl[tt], 0, 0, 0);
            }
        }
    }
    // the row's eight mins as bytes; lanes 0-31 feed K slots 0..7 (bl), lanes 32-63 slots 8..15 (bh)
    const long mp = (long)(((uint64_t)sc.mn_hi << 32) | sc.mn_lo);
    const long b1 = h == 0 ? mp : 0L, b2 = h == 0 ? 0L : mp;
    // the lane's activation-sum bytes of every token tile in one read (8 bytes per tile)
    const uint8_t *bsp = se + (size_t)blk * Tp * 16 + (h * 32 + n) * NTT * 8;
    uint32_t amw[2 * NTT];
    if (NTT == 2) {
        const uint4 t = *(const uint4 *)bsp;
        amw[0] = t.x; amw[1] = t.y; amw[2 % (2 * NTT)] = t.z; amw[3 % (2 * NTT)] = t.w;
    } else {
        const uint2 t = *(const uint2 *)bsp;
        amw[0] = t.x; amw[1] = t.y;
    }
    const float *yds = (const float *)(se + gs_yd(Tp, KQ)) + blk * Tp;
#pragma unroll
    for (int tt = 0; tt < NTT; ++tt) {
        const v16i z = {};
        const long ab = (long)(((uint64_t)amw[2 * tt + 1] << 32) | amw[2 * tt]);
        v16i ms = __builtin_amdgcn_mfma_i32_32x32x16_i8(ab, b2, z, 0, 0, 0);
#pragma unroll
        for (int v = 0; v < 16; ++v) ms[v] <<= 7;
        ms = __builtin_amdgcn_mfma_i32_32x32x16_i8(ab, b1, ms, 0, 0, 0);
        float4 yd[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) yd[k] = *(const float4 *)(yds + 32 * tt + 8 * k + 4 * h);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int isum = (ch[tt][v] << 3) + cl[tt][v], msum = ms[v];
            const float4 q4 = yd[v >> 2];
            const float ydv = (v & 3) == 0 ? q4.x : (v & 3) == 1 ? q4.y : (v & 3) == 2 ? q4.z : q4.w;
            const float t = __builtin_fmaf(-dmin, (float)msum, d * (float)isum);
            acc[tt][v] = __builtin_fmaf(ydv, t, acc[tt][v]);
            if (DUMP) {
                const int tok = 32 * tt + 8 * (v >> 2) + 4 * h + (v & 3);
                if (live && tok < a.T && row < a.nrows) {
                    const size_t i = ((size_t)tok * a.nrows + row) * a.nb + b;
                    a.dump_s[i] = isum;
                    a.dump_m[i] = msum;
                }
            }
        }
    }
}

// NTT = token tiles (1 or 2), KQ = parts of the blocks (2 or 4). Wavefront w: rs = w & 1 (32-row
// slice), kq = w >> 1 (blocks b = kq mod KQ); it computes its 32 rows for every token. Step s
// covers blocks KQ s .. KQ s + KQ - 1: the weights go straight to registers (each wavefront its
// own rows, one step ahead), the activations of the step's blocks by direct-to-LDS loads to an LDS
// stage shared by the two row slices (double-buffered, one step ahead). The KQ partial sums are added at the end through LDS, in order.
template <int NTT, int KQ, bool DUMP>
__global__ __launch_bounds__(128 * KQ) void q4k_gemm_kernel(GemmArgs a) {
    constexpr int NT = 128 * KQ, Tp = 32 * NTT;
    __shared__ __align__(16) uint8_t q0[gs_q(Tp, KQ)], q1[gs_q(Tp, KQ)];
    __shared__ __align__(16) uint8_t e0[gs_e(Tp, KQ)], e1[gs_e(Tp, KQ)];
    const int tid = threadIdx.x, l = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rs = wave & 1, kq = wave >> 1;
    const int n = l & 31, h = l >> 5;
    const int nb = a.nb, nsteps = (nb + KQ - 1) / KQ;
    const int64_t row0 = (int64_t)blockIdx.x * 64;
    const int64_t row = row0 + 32 * rs + n;
    const size_t bstride = (size_t)a.gpm * 2304;  // one block further in the tile layout
    int rr;
    const uint8_t *T = gemm_tile(a, row, rr);

    WOps wa, wb;
    w_load(wa, T, (size_t)min(kq, nb - 1) * bstride, rr, h);
    s_dma<NT, Tp, KQ>(a, q0, e0, 0, tid, wave);
    s_dma_wait();
    __syncthreads();

    float acc[NTT][16];
#pragma unroll
    for (int tt = 0; tt < NTT; ++tt)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[tt][v] = 0.0f;
    for (int s = 0; s < nsteps; s += 2) {
        // step s: stage0, weights wa; step s + 1 loads (stage1, wb) in flight
        w_load(wb, T, (size_t)min(KQ * (s + 1) + kq, nb - 1) * bstride, rr, h);
        s_dma<NT, Tp, KQ>(a, q1, e1, min(s + 1, nsteps - 1), tid, wave);
        __builtin_amdgcn_sched_barrier(0);
        gemm_block<NTT, KQ, DUMP>(wa, q0, e0, kq, n, h, acc, min(KQ * s + kq, nb - 1), KQ * s + kq < nb, row, a);
        __builtin_amdgcn_sched_barrier(0);
        s_dma_wait();
        __syncthreads();
        if (s + 1 < nsteps) {  // uniform
            // step s + 1: stage1, weights wb; step s + 2 loads (stage0, wa) in flight
            w_load(wa, T, (size_t)min(KQ * (s + 2) + kq, nb - 1) * bstride, rr, h);
            s_dma<NT, Tp, KQ>(a, q0, e0, min(s + 2, nsteps - 1), tid, wave);
            __builtin_amdgcn_sched_barrier(0);
            gemm_block<NTT, KQ, DUMP>(wb, q1, e1, kq, n, h, acc, min(KQ * (s + 1) + kq, nb - 1),
                                      KQ * (s + 1) + kq < nb, row, a);
            __builtin_amdgcn_sched_barrier(0);
            s_dma_wait();
            __syncthreads();
        }
    }
    // parts kq > 0 -> LDS (over the first stage: every wavefront is past its last read of it);
    // part 0 adds them in order and stores
    float(*red)[2][NTT][16][64] = (float(*)[2][NTT][16][64])q0;
    if (kq > 0) {
#pragma unroll
        for (int tt = 0; tt < NTT; ++tt)
#pragma unroll
            for (int v = 0; v < 16; ++v) red[kq - 1][rs][tt][v][l] = acc[tt][v];
    }
    __syncthreads();
    if (kq == 0 && row < a.nrows) {
#pragma unroll
        for (int tt = 0; tt < NTT; ++tt)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int tk = 32 * tt + 8 * (v >> 2) + 4 * h + (v & 3);
                float y = acc[tt][v];
#pragma unroll
                for (int k = 1; k < KQ; ++k) y += red[k - 1][rs][tt][v][l];
                if (tk < a.T) a.Y[(size_t)tk * a.ldy + row] = y;
            }
    }
}

hipError_t launch_gemm_quant(const float *x, int64_t ldx, int nb, int T, int Tp, int8_t *qs, float *ydT, int8_t *bsp,
                             hipStream_t s) {
    dim3 grid((nb + 3) / 4, Tp);
    gemm_quant_kernel<<<grid, 256, 0, s>>>(x, ldx, nb, T, Tp, qs, ydT, bsp);
    return hipGetLastError();
}

static int gemm_kq(int nb) { return nb >= 8 ? 4 : 2; }  // parts of the blocks per workgroup

// the kernel's (static) LDS: two stages
size_t q4k_gemm_lds_bytes(int nb, int Tp) { return 2 * (size_t)(gs_q(Tp, gemm_kq(nb)) + gs_e(Tp, gemm_kq(nb))); }

template <int NTT, int KQ>
static void gemm_launch(const GemmArgs &a, hipStream_t s) {
    const dim3 grid((unsigned)((a.nrows + 63) / 64));
    if (a.dump_s) q4k_gemm_kernel<NTT, KQ, true><<<grid, 128 * KQ, 0, s>>>(a);
    else q4k_gemm_kernel<NTT, KQ, false><<<grid, 128 * KQ, 0, s>>>(a);
}

hipError_t launch_q4k_gemm(const GemmArgs &a, hipStream_t s) {
    if (a.T < 1 || a.T > 64 || a.Tp != (a.T > 32 ? 64 : 32) || a.nb < 1 || a.nrows < 1) return hipErrorInvalidValue;
    if (q4k_gemm_lds_bytes(a.nb, a.Tp) > GEMM_LDS_MAX) return hipErrorInvalidValue;
    const int kq = gemm_kq(a.nb);
    if (a.Tp == 64) kq == 4 ? gemm_launch<2, 4>(a, s) : gemm_launch<2, 2>(a, s);
    else kq == 4 ? gemm_launch<1, 4>(a, s) : gemm_launch<1, 2>(a, s);
    return hipGetLastError();
}

}  // namespace fgh
