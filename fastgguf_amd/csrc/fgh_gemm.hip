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
// Weights are read in the decode layout (fgh_q4k.hip): the GEMM needs no second copy.
// Workgroup: 4 wavefronts = 2 slices of 32 rows x 2 halves of the blocks (b even / b odd); each
// wavefront covers all tokens (one or two 32-token tiles) and keeps the next block's operands in
// flight while it computes the current one. The two halves are added at the end through LDS.
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
//   qs  [Tp][K]      int8, natural order
//   ydT [nb][Tp]     fp32 block scales, token-minor (one float4 = 4 consecutive tokens)
//   bsp [Tp][nb][16] int8: the 32-value sums bs_g = bsums[2g] + bsums[2g+1] as bl_g (bytes 0..7,
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
    const size_t K = (size_t)nb * 256;
    *(uint32_t *)(qs + (size_t)tok * K + (size_t)b * 256 + 4 * lane) = pack_q(q0, q1, q2, q3);
    int s = q0 + q1 + q2 + q3;  // 32-value group g = lanes 8g..8g+7
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    s += __shfl_xor(s, 4, 64);
    if ((lane & 7) == 0) {
        int8_t *p = bsp + ((size_t)tok * nb + b) * 16;
        p[lane >> 3] = (int8_t)(s & 127);
        p[8 + (lane >> 3)] = (int8_t)(s >> 7);
    }
    if (lane == 0) ydT[(size_t)b * Tp + tok] = d;
}

// ---------------------------------------------------------------------------------------------
// The GEMM kernel
// ---------------------------------------------------------------------------------------------
struct BlockOps {
    uint4 meta;      // fp16 d, fp16 dmin, 12 bytes of packed scales / mins
    uint4 pc[4];     // chunk j (sub-blocks 2j, 2j+1): 16 bytes, piece l / 32
    uint4 a[2][8];   // activations: token tile t, group g
    uint2 am[2];     // activation group sums as bytes, token tile t
    float4 yd[2][4]; // block scales of tokens 8k + 4 (l / 32) + 0..3 of tile t
};

template <int NTT>
__device__ __forceinline__ void gemm_load(BlockOps &o, const uint8_t *G, int nb, int rr, int b, int h, int n,
                                          const GemmArgs &a) {
    const int q = (rr & 1) * nb + b;
    const int w = rr >> 1;
    o.meta = ld16(G + 16 * ((size_t)2 * nb * w + q));
    const int s = q >> 4, p = q & 15, np = min(16, 2 * nb - 16 * s);
    const uint8_t *qb = G + (size_t)128 * nb + (size_t)256 * nb * w + 2048 * s + h * 64 * np + 64 * p;
#pragma unroll
    for (int j = 0; j < 4; ++j) o.pc[j] = ld16(qb + 16 * j);
    const size_t K = (size_t)nb * 256;
#pragma unroll
    for (int t = 0; t < NTT; ++t) {
        const int8_t *yq = a.qs + (size_t)(32 * t + n) * K + (size_t)b * 256 + 16 * h;
#pragma unroll
        for (int g = 0; g < 8; ++g) o.a[t][g] = *(const uint4 *)(yq + 32 * g);
        o.am[t] = *(const uint2 *)(a.bsp + ((size_t)(32 * t + n) * nb + b) * 16 + 8 * h);
#pragma unroll
        for (int k = 0; k < 4; ++k) o.yd[t][k] = *(const float4 *)(a.ydT + (size_t)b * a.Tp + 32 * t + 8 * k + 4 * h);
    }
}

__device__ __forceinline__ v4i u4v(uint4 u) { return v4i{(int)u.x, (int)u.y, (int)u.z, (int)u.w}; }

// bytes of q (each <= 15) times a small factor (<= 7): no carry between bytes, two 16-bit lanes
__device__ __forceinline__ uint32_t bmul(uint32_t q, uint32_t f2) {
    const u16x2 r = __builtin_bit_cast(u16x2, q) * __builtin_bit_cast(u16x2, f2);
    return __builtin_bit_cast(uint32_t, r);
}

template <int NTT, bool DUMP>
__device__ __forceinline__ void gemm_block(const BlockOps &o, float (&acc)[NTT][16], int h, int b, int64_t R,
                                           const GemmArgs &a) {
    const float d = fp16_bits_to_f32(o.meta.x & 0xFFFF);
    const float dmin = fp16_bits_to_f32(o.meta.x >> 16);
    const Q4KScales sc = q4k_scales(o.meta.y, o.meta.z, o.meta.w);
    v16i chi[NTT], clo[NTT];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t P[4] = {o.pc[j].x, o.pc[j].y, o.pc[j].z, o.pc[j].w};
#pragma unroll
        for (int hn = 0; hn < 2; ++hn) {
            const int g = 2 * j + hn;
            const uint32_t s6 = (uint32_t)q4k_sc(sc, g);
            const uint32_t fh = (s6 >> 3) * 0x00010001u, fl = (s6 & 7) * 0x00010001u;
            v4i bh, bl;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t qn = hn ? ((P[k] >> 4) & 0x0F0F0F0Fu) : (P[k] & 0x0F0F0F0Fu);
                bh[k] = (int)bmul(qn, fh);
                bl[k] = (int)bmul(qn, fl);
            }
#pragma unroll
            for (int t = 0; t < NTT; ++t) {
                const v4i av = u4v(o.a[t][g]);
                if (g == 0) {
                    const v16i z = {};
                    chi[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bh, z, 0, 0, 0);
                    clo[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bl, z, 0, 0, 0);
                } else {
                    chi[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bh, chi[t], 0, 0, 0);
                    clo[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bl, clo[t], 0, 0, 0);
                }
            }
        }
    }
    // the row's eight mins as bytes; lanes 0-31 feed K slots 0..7 (bl), lanes 32-63 slots 8..15 (bh)
    uint32_t m0 = 0, m1 = 0;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        m0 |= (uint32_t)q4k_mn(sc, g) << (8 * g);
        m1 |= (uint32_t)q4k_mn(sc, g + 4) << (8 * g);
    }
    const long mp = (long)(((uint64_t)m1 << 32) | m0);
    const long b1 = h == 0 ? mp : 0L, b2 = h == 0 ? 0L : mp;
#pragma unroll
    for (int t = 0; t < NTT; ++t) {
        const v16i z = {};
        const long av = (long)(((uint64_t)o.am[t].y << 32) | o.am[t].x);
        const v16i c1 = __builtin_amdgcn_mfma_i32_32x32x16_i8(av, b1, z, 0, 0, 0);
        const v16i c2 = __builtin_amdgcn_mfma_i32_32x32x16_i8(av, b2, z, 0, 0, 0);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int isum = (chi[t][v] << 3) + clo[t][v];
            const int msum = c1[v] + (c2[v] << 7);
            const float4 y4 = o.yd[t][v >> 2];
            const float yd = (v & 3) == 0 ? y4.x : (v & 3) == 1 ? y4.y : (v & 3) == 2 ? y4.z : y4.w;
            const float tt = __builtin_fmaf(-dmin, (float)msum, d * (float)isum);
            acc[t][v] = __builtin_fmaf(yd, tt, acc[t][v]);
            if (DUMP) {
                const int tok = 32 * t + 8 * (v >> 2) + 4 * h + (v & 3);
                if (tok < a.T && R < a.nrows) {
                    const size_t i = ((size_t)tok * a.nrows + R) * a.nb + b;
                    a.dump_s[i] = isum;
                    a.dump_m[i] = msum;
                }
            }
        }
    }
}

template <int NTT, bool DUMP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void q4k_gemm_kernel(GemmArgs a) {
    __shared__ float red[2][NTT][16][64];
    const int tid = threadIdx.x, l = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rs = wave & 1, kh = wave >> 1;
    const int n = l & 31, h = l >> 5;
    const int nb = a.nb;
    const int64_t row = (int64_t)blockIdx.x * 64 + 32 * rs + n;
    const int64_t R = row < a.nrows ? row : a.nrows - 1;  // rows past the end re-read the last one
    const int64_t mat = R / a.rows, r = R - mat * a.rows;
    const int rr = (int)(r & 7);
    const uint8_t *G = a.W + (size_t)(mat * a.gpm + (r >> 3)) * 1152 * nb;

    float acc[NTT][16];
#pragma unroll
    for (int t = 0; t < NTT; ++t)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[t][v] = 0.0f;

    // blocks kh, kh + 2, ...: two operand sets alternate, the next block's loads in flight while
    // the current one computes (loads past the end repeat the wavefront's last block)
    const int cnt = (nb - kh + 1) >> 1;
    const int last = kh + 2 * (cnt - 1);
    BlockOps o0, o1;
    if (cnt > 0) {
        gemm_load<NTT>(o0, G, nb, rr, kh, h, n, a);
        for (int i = 0; i < cnt; i += 2) {
            const int b0 = kh + 2 * i, b1 = min(b0 + 2, last), b2 = min(b0 + 4, last);
            gemm_load<NTT>(o1, G, nb, rr, b1, h, n, a);
            gemm_block<NTT, DUMP>(o0, acc, h, b0, row, a);
            if (i + 1 < cnt) {
                gemm_load<NTT>(o0, G, nb, rr, b2, h, n, a);
                gemm_block<NTT, DUMP>(o1, acc, h, b1, row, a);
            }
        }
    }
    // odd-block half -> LDS; the even half adds it (fixed order) and stores
    if (kh == 1) {
#pragma unroll
        for (int t = 0; t < NTT; ++t)
#pragma unroll
            for (int v = 0; v < 16; ++v) red[rs][t][v][l] = acc[t][v];
    }
    __syncthreads();
    if (kh == 0 && row < a.nrows) {
#pragma unroll
        for (int t = 0; t < NTT; ++t)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int tok = 32 * t + 8 * (v >> 2) + 4 * h + (v & 3);
                if (tok < a.T) a.Y[(size_t)tok * a.ldy + row] = acc[t][v] + red[rs][t][v][l];
            }
    }
}

hipError_t launch_gemm_quant(const float *x, int64_t ldx, int nb, int T, int Tp, int8_t *qs, float *ydT, int8_t *bsp,
                             hipStream_t s) {
    dim3 grid((nb + 3) / 4, Tp);
    gemm_quant_kernel<<<grid, 256, 0, s>>>(x, ldx, nb, T, Tp, qs, ydT, bsp);
    return hipGetLastError();
}

hipError_t launch_q4k_gemm(const GemmArgs &a, hipStream_t s) {
    if (a.T < 1 || a.T > 64 || a.Tp != (a.T > 32 ? 64 : 32) || a.nb < 1 || a.nrows < 1) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((a.nrows + 63) / 64));
    if (a.Tp == 64) {
        if (a.dump_s) q4k_gemm_kernel<2, true><<<grid, 256, 0, s>>>(a);
        else q4k_gemm_kernel<2, false><<<grid, 256, 0, s>>>(a);
    } else {
        if (a.dump_s) q4k_gemm_kernel<1, true><<<grid, 256, 0, s>>>(a);
        else q4k_gemm_kernel<1, false><<<grid, 256, 0, s>>>(a);
    }
    return hipGetLastError();
}

}  // namespace fgh
