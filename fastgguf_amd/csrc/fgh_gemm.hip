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

// ---------------------------------------------------------------------------------------------
// Activation quantizer for the GEMM (quantize_q8k, fastgguf.c:773-793, bit-exact): one wavefront
// per (token, 256-block); lane l holds values 4l..4l+3. Writes
//   qs  [nb][Tp/32][8][32][32] int8: group g of block b of token t = 32 tt + n at
//                    (((b Tp/32 + tt) 8 + g) 32 + n) 32, so one MFMA fragment (32 tokens x 32
//                    values) is 1 KB contiguous and a block's 8 fragments of one token tile 8 KB
//   ydT [nb][Tp]     fp32 block scales, token-minor (one float4 = 4 consecutive tokens)
//   bsp [nb][Tp][16] int8: the 32-value sums bs_g = bsums[2g] + bsums[2g+1] as bl_g (bytes 0..7,
//                    bs & 127) and bh_g (bytes 8..15, bs >> 7)
// Tokens T..Tp-1 are written as zeros.
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
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    const int q0 = q8_round(v.x * id), q1 = q8_round(v.y * id);
    const int q2 = q8_round(v.z * id), q3 = q8_round(v.w * id);
    *(uint32_t *)(qs + ((((size_t)b * (Tp >> 5) + (tok >> 5)) * 8 + (lane >> 3)) * 32 + (tok & 31)) * 32 +
                  4 * (lane & 7)) = pack_q(q0, q1, q2, q3);
    int s = q0 + q1 + q2 + q3;  // 32-value group g = lanes 8g..8g+7
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    s += __shfl_xor(s, 4, 64);
    if ((lane & 7) == 0) {
        int8_t *p = bsp + ((size_t)b * Tp + tok) * 16;
        p[lane >> 3] = (int8_t)(s & 127);
        p[8 + (lane >> 3)] = (int8_t)(s >> 7);
    }
    if (lane == 0) ydT[(size_t)b * Tp + tok] = d;
}

// ---------------------------------------------------------------------------------------------
// The GEMM kernel
// ---------------------------------------------------------------------------------------------
constexpr int GW_STAGE = 18432;  // LDS bytes of one weight stage: quants 16 KB + meta 2 KB

// One workgroup's share of a weight stage (blocks 2s and 2s+1 of its 64 rows = 4 tiles), held by
// thread tid: quant units u = tid + k * NT, u = ((blk * 4 + tile) * 2 + hh) * 64 + L, i.e. slot
// (hh, L) of the tile layout (64 consecutive units read 1 KB contiguous), and for tid < 128 the
// meta of (row tid % 64, blk tid / 64).
template <int NT>
struct WStage {
    static constexpr int NU = 1024 / NT;
    const uint8_t *src[NU];  // per unit: its address in block 0 of its tile
    int slot[NU];            // per unit: its LDS slot
    const uint8_t *msrc;     // the meta row's address in block 0 of its tile
    uint4 q[NU], m;
};

// LDS stage layout: quants [blk][j][h][row 0..63] x 16 B (a fragment = 512 B contiguous per h),
// meta at 16 KB: [blk][row] x 16 B. Row slots are XOR-swizzled with 2j (quants) and 4 blk (meta):
// the eight threads of one 128-byte write phase hold rows 2m, 2m+1 x chunks j = 0..3 of one tile,
// and the swizzle sends them to eight different bank quads; a fragment read stays a permutation
// of 32 consecutive slots.
__device__ __forceinline__ int gq_slot(int blk, int j, int h, int row) {
    return ((blk * 4 + j) * 2 + h) * 64 + (row ^ (2 * j));
}
__device__ __forceinline__ int gm_slot(int blk, int row) { return 1024 + blk * 64 + (row ^ (blk << 2)); }

// the tile-layout address of (row R over all matrices, block 0): its tile and its row in the tile
// (block b is b * gpm * 2304 further)
__device__ __forceinline__ const uint8_t *gemm_tile(const GemmArgs &a, int64_t R, int &rr) {
    R = R < a.nrows ? R : a.nrows - 1;
    const int64_t mat = R / a.rows, r = R - mat * a.rows;
    rr = (int)(r & 15);
    return a.W + ((size_t)mat * a.nb * a.gpm + (size_t)(r >> 4)) * 2304;
}

template <int NT>
__device__ __forceinline__ void wstage_init(WStage<NT> &w, const GemmArgs &a, int64_t row0, int tid) {
#pragma unroll
    for (int k = 0; k < WStage<NT>::NU; ++k) {
        const int u = tid + k * NT;
        const int L = u & 63, hh = (u >> 6) & 1, tl = (u >> 7) & 3, blk = u >> 9, j = L & 3;
        const int row = 16 * tl + (L >> 2);
        int rr;
        const uint8_t *T = gemm_tile(a, row0 + row, rr);
        w.src[k] = T + 256 + 1024 * hh + 16 * (4 * rr + j);
        w.slot[k] = gq_slot(blk, j, hh ^ (j >> 1), row);  // slot hh holds piece hh ^ (j >> 1)
    }
    int rr;
    const uint8_t *T = gemm_tile(a, row0 + (tid & 63), rr);
    w.msrc = T + 16 * rr;
}

template <int NT>
__device__ __forceinline__ void wstage_load(WStage<NT> &w, int nb, size_t bstride, int s, int tid) {
#pragma unroll
    for (int k = 0; k < WStage<NT>::NU; ++k) {
        const int blk = (tid + k * NT) >> 9;
        w.q[k] = ld16(w.src[k] + (size_t)min(2 * s + blk, nb - 1) * bstride);
    }
    if (tid < 128) w.m = ld16(w.msrc + (size_t)min(2 * s + (tid >> 6), nb - 1) * bstride);
}

template <int NT>
__device__ __forceinline__ void wstage_store(const WStage<NT> &w, uint8_t *buf, int tid) {
#pragma unroll
    for (int k = 0; k < WStage<NT>::NU; ++k) *(uint4 *)(buf + 16 * w.slot[k]) = w.q[k];
    if (tid < 128) *(uint4 *)(buf + 16 * gm_slot(tid >> 6, tid & 63)) = w.m;
}

// one lane's activation operands of one block: group g (16 values of token 32 tt + l % 32) and
// the token's 32-value sums as bytes (bl_0..7 or bh_0..7)
struct ActOps {
    uint4 av[8];
    uint2 am;
};

__device__ __forceinline__ void act_load(ActOps &o, const GemmArgs &a, int b, int tok, int h) {
    // the block's 8 fragments of this token tile are 8 KB contiguous: two bases, immediate offsets
    const int8_t *p = a.qs + (((size_t)b * (a.Tp >> 5) + (tok >> 5)) * 8 * 32 + (tok & 31)) * 32 + 16 * h;
#pragma unroll
    for (int g = 0; g < 8; ++g) o.av[g] = *(const uint4 *)(p + 1024 * g);
    o.am = *(const uint2 *)(a.bsp + ((size_t)b * a.Tp + tok) * 16 + 8 * h);
}

__device__ __forceinline__ v4i u4v(uint4 u) { return v4i{(int)u.x, (int)u.y, (int)u.z, (int)u.w}; }

// bytes of q (each <= 15) times a small factor (<= 7): no carry between bytes, two 16-bit lanes
__device__ __forceinline__ uint32_t bmul(uint32_t q, uint32_t f2) {
    const u16x2 r = __builtin_bit_cast(u16x2, q) * __builtin_bit_cast(u16x2, f2);
    return __builtin_bit_cast(uint32_t, r);
}

// One 256-block of one wavefront: weights from the LDS stage (slice blk of the step), activations
// from registers. live == false: a padding block (odd block counts): computed, weighted by zero,
// not dumped.
template <bool DUMP>
__device__ __forceinline__ void gemm_block(const ActOps &o, const uint8_t *stage, int blk, int rs, int n, int h,
                                           int tt, float (&acc)[16], const float *__restrict__ yds, int b, bool live,
                                           int64_t row, const GemmArgs &a) {
    const int row32 = rs * 32 + n;
    const uint4 meta = *(const uint4 *)(stage + 16 * gm_slot(blk, row32));
    uint4 pc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) pc[j] = *(const uint4 *)(stage + 16 * gq_slot(blk, j, h, row32));
    const Q4KScales sc = q4k_scales(meta.y, meta.z, meta.w);
    // a padding block contributes zero: its scales are zeroed once here
    const float d = live ? fp16_bits_to_f32(meta.x & 0xFFFF) : 0.0f;
    const float dmin = live ? fp16_bits_to_f32(meta.x >> 16) : 0.0f;
    // the split scale factors of the 8 groups as bytes: sh = sc >> 3, sl = sc & 7
    const uint32_t shb[2] = {(sc.sc_lo >> 3) & 0x07070707u, (sc.sc_hi >> 3) & 0x07070707u};
    const uint32_t slb[2] = {sc.sc_lo & 0x07070707u, sc.sc_hi & 0x07070707u};
    // pass 0: q * sh over the block's 8 groups; pass 1 continues from 8 * Chi with q * sl
    v16i ai;
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t P[4] = {pc[j].x, pc[j].y, pc[j].z, pc[j].w};
#pragma unroll
            for (int hn = 0; hn < 2; ++hn) {
                const int g = 2 * j + hn;
                // byte g of the factors into both 16-bit lanes (v_perm_b32; selector 0x0C = zero)
                const uint32_t f = __builtin_amdgcn_perm(0u, pass == 0 ? shb[g >> 2] : slb[g >> 2],
                                                         0x0C000C00u | (uint32_t)((g & 3) * 0x00010001));
                v4i bw;
#pragma unroll
                for (int k = 0; k < 4; ++k) bw[k] = (int)bmul(hn ? ((P[k] >> 4) & 0x0F0F0F0Fu) : (P[k] & 0x0F0F0F0Fu), f);
                if (pass == 0 && g == 0) {
                    const v16i z = {};
                    ai = __builtin_amdgcn_mfma_i32_32x32x32_i8(u4v(o.av[g]), bw, z, 0, 0, 0);
                } else {
                    ai = __builtin_amdgcn_mfma_i32_32x32x32_i8(u4v(o.av[g]), bw, ai, 0, 0, 0);
                }
            }
        }
        if (pass == 0) {
#pragma unroll
            for (int v = 0; v < 16; ++v) ai[v] <<= 3;
        }
    }
    // the row's eight mins as bytes; lanes 0-31 feed K slots 0..7 (bl), lanes 32-63 slots 8..15 (bh)
    const long mp = (long)(((uint64_t)sc.mn_hi << 32) | sc.mn_lo);
    const long b1 = h == 0 ? mp : 0L, b2 = h == 0 ? 0L : mp;
    const v16i z = {};
    const long ab = (long)(((uint64_t)o.am.y << 32) | o.am.x);
    v16i ms = __builtin_amdgcn_mfma_i32_32x32x16_i8(ab, b2, z, 0, 0, 0);
#pragma unroll
    for (int v = 0; v < 16; ++v) ms[v] <<= 7;
    ms = __builtin_amdgcn_mfma_i32_32x32x16_i8(ab, b1, ms, 0, 0, 0);
    float4 yd[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) yd[k] = *(const float4 *)(yds + b * a.Tp + 32 * tt + 8 * k + 4 * h);
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int isum = ai[v], msum = ms[v];
        const float4 q4 = yd[v >> 2];
        const float ydv = (v & 3) == 0 ? q4.x : (v & 3) == 1 ? q4.y : (v & 3) == 2 ? q4.z : q4.w;
        const float t = __builtin_fmaf(-dmin, (float)msum, d * (float)isum);
        acc[v] = __builtin_fmaf(ydv, t, acc[v]);
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

// NTW = token tiles (1 or 2). Wavefront w: rs = w & 1 (32-row slice), kh = (w >> 1) & 1 (even /
// odd blocks), tt = w >> 2 (32-token tile). Step s covers blocks 2s (kh 0) and 2s + 1 (kh 1).
template <int NTW, bool DUMP>
__global__ __launch_bounds__(256 * NTW) void q4k_gemm_kernel(GemmArgs a) {
    constexpr int NT = 256 * NTW;
    // LDS: the block scales of every token (ydT, nb x Tp floats), then two weight stages (the
    // reduction area reuses the first after the loop)
    extern __shared__ __align__(16) float lds_g[];
    float *yds = lds_g;
    uint8_t *stage0 = (uint8_t *)(lds_g + (size_t)a.nb * a.Tp);
    uint8_t *stage1 = stage0 + GW_STAGE;
    const int tid = threadIdx.x, l = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rs = wave & 1, kh = (wave >> 1) & 1, tt = wave >> 2;
    const int n = l & 31, h = l >> 5;
    const int nb = a.nb, nsteps = (nb + 1) >> 1;
    const int64_t row0 = (int64_t)blockIdx.x * 64;
    const int64_t row = row0 + 32 * rs + n;
    const int tok = 32 * tt + n;

    const size_t bstride = (size_t)a.gpm * 2304;  // one block further in the tile layout
    WStage<NT> ws;
    wstage_init(ws, a, row0, tid);
    wstage_load(ws, nb, bstride, 0, tid);
    ActOps A, B;
    act_load(A, a, min(kh, nb - 1), tok, h);
    for (int i = tid; i < nb * a.Tp / 4; i += NT) ((float4 *)yds)[i] = ((const float4 *)a.ydT)[i];
    wstage_store(ws, stage0, tid);
    __syncthreads();

    float acc[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
    for (int s = 0; s < nsteps; s += 2) {
        // step s: stage0, set A; loads of step s + 1 (stage1, set B) in flight
        wstage_load(ws, nb, bstride, min(s + 1, nsteps - 1), tid);
        act_load(B, a, min(2 * (s + 1) + kh, nb - 1), tok, h);
        __builtin_amdgcn_sched_barrier(0);
        gemm_block<DUMP>(A, stage0, kh, rs, n, h, tt, acc, yds, min(2 * s + kh, nb - 1), 2 * s + kh < nb, row, a);
        __builtin_amdgcn_sched_barrier(0);
        wstage_store(ws, stage1, tid);
        __syncthreads();
        if (s + 1 < nsteps) {  // uniform
            // step s + 1: stage1, set B; loads of step s + 2 (stage0, set A) in flight
            wstage_load(ws, nb, bstride, min(s + 2, nsteps - 1), tid);
            act_load(A, a, min(2 * (s + 2) + kh, nb - 1), tok, h);
            __builtin_amdgcn_sched_barrier(0);
            gemm_block<DUMP>(B, stage1, kh, rs, n, h, tt, acc, yds, min(2 * (s + 1) + kh, nb - 1),
                             2 * (s + 1) + kh < nb, row, a);
            __builtin_amdgcn_sched_barrier(0);
            wstage_store(ws, stage0, tid);
            __syncthreads();
        }
    }
    // odd-block half -> LDS (over the first stage: every wavefront is past its last read of it);
    // the even half adds it (fixed order) and stores
    float(*red)[2][16][64] = (float(*)[2][16][64])stage0;
    if (kh == 1) {
#pragma unroll
        for (int v = 0; v < 16; ++v) red[tt][rs][v][l] = acc[v];
    }
    __syncthreads();
    if (kh == 0 && row < a.nrows) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int tk = 32 * tt + 8 * (v >> 2) + 4 * h + (v & 3);
            if (tk < a.T) a.Y[(size_t)tk * a.ldy + row] = acc[v] + red[tt][rs][v][l];
        }
    }
}

hipError_t launch_gemm_quant(const float *x, int64_t ldx, int nb, int T, int Tp, int8_t *qs, float *ydT, int8_t *bsp,
                             hipStream_t s) {
    dim3 grid((nb + 3) / 4, Tp);
    gemm_quant_kernel<<<grid, 256, 0, s>>>(x, ldx, nb, T, Tp, qs, ydT, bsp);
    return hipGetLastError();
}

size_t q4k_gemm_lds_bytes(int nb, int Tp) { return (size_t)nb * Tp * 4 + 2 * (size_t)GW_STAGE; }

hipError_t launch_q4k_gemm(const GemmArgs &a, hipStream_t s) {
    if (a.T < 1 || a.T > 64 || a.Tp != (a.T > 32 ? 64 : 32) || a.nb < 1 || a.nrows < 1) return hipErrorInvalidValue;
    const size_t lds = q4k_gemm_lds_bytes(a.nb, a.Tp);
    if (lds > GEMM_LDS_MAX) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((a.nrows + 63) / 64));
    if (a.Tp == 64) {
        if (a.dump_s) q4k_gemm_kernel<2, true><<<grid, 512, lds, s>>>(a);
        else q4k_gemm_kernel<2, false><<<grid, 512, lds, s>>>(a);
    } else {
        if (a.dump_s) q4k_gemm_kernel<1, true><<<grid, 256, lds, s>>>(a);
        else q4k_gemm_kernel<1, false><<<grid, 256, lds, s>>>(a);
    }
    return hipGetLastError();
}

}  // namespace fgh
