// fgh_gemm32n.hip - the prompt-batch (8..64 tokens) matmul of the 32-value nibble types Q4_0,
// Q4_1, Q5_0 and Q5_1 with Q8 activations on gfx950 MFMA, in gemm_q32's own fp32 order
// (fastgguf.c:2856-2999; the matmul dispatch at 3027-3030).
//
// gemm_q32 multiplies UNSIGNED weights u (the nibble, or the 5-bit value) with the int8 activations
// and takes the offset out with the activation sums. Per row, token and 32-block g, in block order
// (unpack_row_q32 2876-2894, gemm_pack_q8 2897-2913, gemm32_kern 2919-2948):
//     acc = fma(d_g * xd_g, float(sum_32 u * xq), acc)
//     acc = fma(-m_g, ys_g, acc)            ys_g = xd_g * float(s16_0 + s16_1)
// with m = 8 d (Q4_0), 16 d (Q5_0), -FP16(min) (Q4_1, Q5_1). Each output is one chain over its
// row's blocks in order, so there is no K split here: the result is the reference's, bit for bit.
//
// One block is one K = 32 step of v_mfma_i32_16x16x32_i8 (A = 16 tokens, B = 16 rows), so the
// block's integer comes out of the matrix unit whole (it is exact in any order of K). A wavefront
// owns 16 rows (two 8-row decode tiles) and NT tiles of 16 tokens:
//   - lane (g, n) supplies row n's elements 8 g .. 8 g + 7 of each block: slices 2 g and 2 g + 1
//     of its row in the decode layout (fgh_internal.h), 16 contiguous nibble bytes per 4-block
//     step (and 4 bytes of fifth bits), and its row's fp16 d (and min) of the step's 4 blocks;
//   - its activation record gives lane (g, m) token m's elements 8 g .. 8 g + 7;
//   - it ends with the integers of tokens 4 g + e (e = 0..3) of row n.
// The per-token scales reach the lanes without LDS: a record register holds, in lane 16 g + e,
// token 4 g + e's xd of the step's 4 blocks and, in lane 16 g + 4 + e, its ys, and a DPP row
// broadcast (row_newbcast) hands lane 16 g + e's value to the 16 lanes of row g, as an operand of
// the multiply or fma itself. So each (row, token, block) costs one MFMA share and four VALU
// instructions: convert, d * xd, and the two fma.
//
// Wavefronts are independent (no LDS, no barrier): each streams its weights and its token tiles'
// records D tile steps ahead in a ring of registers. Blocks past a row's end are zeros in both the
// tiles and the records; they add +0 products to chains that start at +0 and so are never -0,
// which leaves every chain bit-identical.
#include "fgh_internal.h"

namespace fgh {

typedef int v4i __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------------------------
// Activation records, GEMMN_REC bytes per (16-token tile tt, tile step s) at (tt * nsteps + s):
//   [0, 2048)     int8 fragments, half hf (blocks 2 hf, 2 hf + 1) at 1024 hf: lane l = 16 g + m
//                 holds at 16 l the 8 quants 8 g .. 8 g + 7 of block 4 s + 2 hf of token
//                 16 tt + m, then the same of block 4 s + 2 hf + 1
//   [2048, 2304)  fp32 xd [16 tokens][4 blocks]
//   [2304, 2560)  fp32 ys [16 tokens][4 blocks], ys = xd * float(s16_0 + s16_1)
// Tokens T.. and blocks past the row's last are zeros.
// ---------------------------------------------------------------------------------------------
constexpr int GEMMN_REC = 2560;

// quantize_q8 (fastgguf.c:746-770, bit-exact) into the records: one wavefront per (block b, 16
// tokens); lane l = 16 g + m takes token 16 blockIdx.y + m and values 8 g .. 8 g + 7 of the block.
// The block maximum and the quant sum combine the four lanes of a token; fmaxf ignores NaN, as
// the reference's comparison does, and the integer sum is exact in any order.
__global__ __launch_bounds__(64) void gemmn_quant_kernel(const float *__restrict__ x, int64_t ldx, int nb, int ns,
                                                         int T, uint8_t *__restrict__ rec) {
    const int l = threadIdx.x, g = l >> 4, m = l & 15;
    const int b = blockIdx.x, tt = blockIdx.y, tok = 16 * tt + m;
    float v[8];
    if (tok < T && b < nb) {
        const float *src = x + (size_t)tok * ldx + (size_t)b * 32 + 8 * g;
        const float4 f0 = *(const float4 *)src, f1 = *(const float4 *)(src + 4);
        v[0] = f0.x; v[1] = f0.y; v[2] = f0.z; v[3] = f0.w;
        v[4] = f1.x; v[5] = f1.y; v[6] = f1.z; v[7] = f1.w;
    } else {
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = 0.0f;
    }
    float amax = 0.0f;
#pragma unroll
    for (int u = 0; u < 8; ++u) amax = fmaxf(amax, fabsf(v[u]));
    amax = fmaxf(amax, __shfl_xor(amax, 16, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    int q[8], s = 0;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        q[u] = (int)(int8_t)q8_round(v[u] * id);
        s += q[u];
    }
    s += __shfl_xor(s, 16, 64);
    s += __shfl_xor(s, 32, 64);
    uint8_t *r = rec + ((size_t)tt * ns + (b >> 2)) * GEMMN_REC;
    const int bb = b & 3;
    *(uint2 *)(r + (bb >> 1) * 1024 + 16 * l + 8 * (bb & 1)) =
        make_uint2(pack_q(q[0], q[1], q[2], q[3]), pack_q(q[4], q[5], q[6], q[7]));
    if (g == 0) {
        ((float *)(r + 2048))[4 * m + bb] = d;
        ((float *)(r + 2304))[4 * m + bb] = d * (float)s;
    }
}

size_t gemmn_act_bytes(int nb, int Tp) { return (size_t)(Tp / 16) * ((nb + 3) / 4) * GEMMN_REC; }

hipError_t launch_gemmn_quant(const float *x, int64_t ldx, int nb, int T, int Tp, uint8_t *rec, hipStream_t s) {
    if (T < 1 || T > Tp || Tp % 16 || Tp > 64 || nb < 1) return hipErrorInvalidValue;
    const int ns = (nb + 3) / 4;
    // every block of every tile step, the ones past the row's end as zeros
    gemmn_quant_kernel<<<dim3((unsigned)(4 * ns), (unsigned)(Tp / 16)), 64, 0, s>>>(x, ldx, nb, ns, T, rec);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// The GEMM kernel
// ---------------------------------------------------------------------------------------------
// value of lane 16 (l / 16) + K, as the first operand of the instruction that consumes it
template <int K>
__device__ __forceinline__ float row_bcast(uint32_t v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, (int)v, 0x150 + K, 0xF, 0xF, false));
}

// acc[e] = fma(v of lane 16 (l / 16) + 4 + e, m, acc[e]) for e = 0..3: v_fmac_f32 with a DPP row
// broadcast of its first operand (the compiler folds DPP into a multiply, not into a
// multiply-accumulate). The s_nop gives the two wait states a DPP read needs after a VALU write
// of its source.
__device__ __forceinline__ void fmac_ys4(float (&acc)[4], uint32_t v, float m) {
    asm("s_nop 1\n\t"
        "v_fmac_f32_dpp %0, %4, %5 row_newbcast:4 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %1, %4, %5 row_newbcast:5 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %2, %4, %5 row_newbcast:6 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %3, %4, %5 row_newbcast:7 row_mask:0xf bank_mask:0xf"
        : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3])
        : "v"(v), "v"(m));
}

// one lane's weights of one tile step
struct WStepN {
    uint4 n;     // slices 2 g (x, y) and 2 g + 1 (z, w): dword w of a slice = blocks 2 w, 2 w + 1
    uint2 d, m;  // fp16 d (and min) of the row's 4 blocks
    uint32_t h;  // fifth bits of slices 2 g (low 16) and 2 g + 1 (high 16)
};
// one lane's records of one tile step for one token tile
struct AStepN {
    uint4 f0, f1;  // fragments of blocks 0, 1 and 2, 3
    uint4 sc;      // xd (lanes 16 g + 0..3) or ys (16 g + 4..7) of the 4 blocks
};

// the B operand of block bb: elements 8 g .. 8 g + 7 as unsigned bytes (the nibble, with the
// fifth bit as bit 4)
template <int TYPE>
__device__ __forceinline__ long wq_block(const WStepN &w, int bb) {
    constexpr bool Q5 = TYPE == T_Q5_0 || TYPE == T_Q5_1;
    const uint32_t s0 = (bb >> 1) ? w.n.y : w.n.x, s1 = (bb >> 1) ? w.n.w : w.n.z;
    uint32_t b0 = ((bb & 1) ? s0 >> 4 : s0) & 0x0F0F0F0Fu, b1 = ((bb & 1) ? s1 >> 4 : s1) & 0x0F0F0F0Fu;
    if (Q5) {
        // slice bits n0 | n2 << 4 | n1 << 8 | n3 << 12 -> byte t = n_t (bit k = block k)
        const uint32_t e0 = (w.h & 0x0F0Fu) | ((w.h << 12) & 0x0F0F0000u);
        const uint32_t e1 = ((w.h >> 16) & 0x0F0Fu) | ((w.h >> 4) & 0x0F0F0000u);
        b0 |= (e0 << (4 - bb)) & 0x10101010u;
        b1 |= (e1 << (4 - bb)) & 0x10101010u;
    }
    return (long)(((uint64_t)b1 << 32) | b0);
}

template <int TYPE, int NT, int D, bool DUMP>
__global__ __launch_bounds__(256) void q32n_gemm_kernel(GemmNArgs a) {
    constexpr bool Q5 = TYPE == T_Q5_0 || TYPE == T_Q5_1, MIN = q32_min(TYPE);
    constexpr Q32Layout L = q32_layout(TYPE);
    const int l = threadIdx.x & 63;
    const int64_t wid = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nch = a.Tp / (16 * NT);  // token chunks of NT tiles
    const int64_t grp = wid / nch;
    const int ch = (int)(wid - grp * nch);
    if (grp >= a.groups) return;  // wavefronts are independent
    const int64_t mi = grp / a.ppm, p = grp - mi * a.ppm;
    const int g = l >> 4, n = l & 15, r8 = n & 7;
    const int64_t row = 16 * p + n;
    const bool store = row < a.rows;
    const int64_t orow = mi * a.rows + row;
    const int ns = a.nsteps;
    const uint32_t wbytes = (uint32_t)min<int64_t>(2, a.tpm - 2 * p) * L.tile;  // valid tiles of the pair
    const uint8_t *wbase = a.W + ((size_t)mi * ns * a.tpm + 2 * p) * L.tile;
    const size_t wstride = (size_t)a.tpm * L.tile;
    const uint32_t toff = (uint32_t)(n >> 3) * L.tile;
    const uint32_t noff = toff + L.n + 8 * (8 * r8 + 2 * g), doff = toff + L.ds * r8;
    const uint32_t hoff = toff + (Q5 ? L.h : 0) + 2 * (8 * r8 + 2 * g);
    const uint32_t soff = 2048 + ((l & 4) ? 256 : 0) + 16 * (4 * g + (l & 3));  // xd or ys of token 4 g + l % 4
    const uint32_t abytes = (uint32_t)ns * GEMMN_REC;
    BufRes ar[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) ar[t] = buf_res(a.act + (size_t)(ch * NT + t) * ns * GEMMN_REC, abytes);

    // step s < ns (the callers clamp where a step could pass the end)
    auto load = [&](int s, WStepN &w, AStepN (&x)[NT]) __attribute__((always_inline)) {
        const BufRes rw = buf_res(wbase + (size_t)s * wstride, wbytes);
        w.n = bld16(rw, noff);
        if (MIN) {  // the row's d and m in one record
            const uint4 dm = bld16(rw, doff);
            w.d = make_uint2(dm.x, dm.y);
            w.m = make_uint2(dm.z, dm.w);
        } else {
            w.d = bld8(rw, doff);
        }
        if (Q5) w.h = __builtin_amdgcn_raw_buffer_load_b32(rw, (int)hoff, 0, 0);
        const int so = s * GEMMN_REC;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const auto f0 = __builtin_amdgcn_raw_buffer_load_b128(ar[t], (int)(16 * l), so, 0);
            const auto f1 = __builtin_amdgcn_raw_buffer_load_b128(ar[t], (int)(1024 + 16 * l), so, 0);
            const auto sc = __builtin_amdgcn_raw_buffer_load_b128(ar[t], (int)soff, so, 0);
            x[t].f0 = make_uint4(f0[0], f0[1], f0[2], f0[3]);
            x[t].f1 = make_uint4(f1[0], f1[1], f1[2], f1[3]);
            x[t].sc = make_uint4(sc[0], sc[1], sc[2], sc[3]);
        }
    };

    float acc[NT][4];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[t][e] = 0.0f;

    auto compute = [&](int s, const WStepN &w, const AStepN (&x)[NT]) __attribute__((always_inline)) {
        // the step's integers first (the MFMA latency hides behind the other blocks' epilogues)
        v4i isums[4][NT];
#pragma unroll
        for (int bb = 0; bb < 4; ++bb) {
            const long bq = wq_block<TYPE>(w, bb);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const uint4 f = (bb >> 1) ? x[t].f1 : x[t].f0;
                const long aq = (long)((bb & 1) ? (((uint64_t)f.w << 32) | f.z) : (((uint64_t)f.y << 32) | f.x));
                isums[bb][t] = __builtin_amdgcn_mfma_i32_16x16x32_i8(aq, bq, v4i{0, 0, 0, 0}, 0, 0, 0);
            }
        }
#pragma unroll
        for (int bb = 0; bb < 4; ++bb) {
            const uint32_t dd = (bb >> 1) ? w.d.y : w.d.x;
            const float dw = fp16_bits_to_f32((bb & 1) ? dd >> 16 : dd);
            float negm;
            if (MIN) {
                const uint32_t mm = (bb >> 1) ? w.m.y : w.m.x;
                negm = fp16_bits_to_f32((bb & 1) ? mm >> 16 : mm);  // m = -FP16(min)
            } else {
                negm = (TYPE == T_Q5_0 ? -16.0f : -8.0f) * dw;
            }
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const v4i isum = isums[bb][t];
                const uint32_t sv = bb == 0 ? x[t].sc.x : bb == 1 ? x[t].sc.y : bb == 2 ? x[t].sc.z : x[t].sc.w;
                const float xd[4] = {row_bcast<0>(sv), row_bcast<1>(sv), row_bcast<2>(sv), row_bcast<3>(sv)};
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[t][e] = __builtin_fmaf(xd[e] * dw, (float)isum[e], acc[t][e]);
                fmac_ys4(acc[t], sv, negm);
                if (DUMP) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int tok = 16 * (ch * NT + t) + 4 * g + e, blk = 4 * s + bb;
                        if (store && tok < a.T && blk < a.nb) a.dump_s[((size_t)tok * a.nrows + orow) * a.nb + blk] = isum[e];
                    }
                }
            }
        }
    };

    // ring of D steps: step j + u computes from slot u, which then loads step j + u + D. Every
    // load of the main loop is in range (no clamp on its addresses); the one round that can reach
    // past the last step clamps (its extra loads re-read the last step), then the rest drains.
    WStepN w[D];
    AStepN x[D][NT];
#pragma unroll
    for (int u = 0; u < D; ++u) load(min(u, ns - 1), w[u], x[u]);
    int j = 0;
    for (; j + 2 * D <= ns; j += D) {
#pragma unroll
        for (int u = 0; u < D; ++u) {
            compute(j + u, w[u], x[u]);
            load(j + u + D, w[u], x[u]);
        }
    }
    if (j + D <= ns) {
#pragma unroll
        for (int u = 0; u < D; ++u) {
            compute(j + u, w[u], x[u]);
            load(min(j + u + D, ns - 1), w[u], x[u]);
        }
        j += D;
    }
#pragma unroll
    for (int u = 0; u < D; ++u)
        if (j + u < ns) compute(j + u, w[u], x[u]);

    if (store) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int tok = 16 * (ch * NT + t) + 4 * g + e;
                if (tok < a.T) a.Y[(size_t)tok * a.ldy + orow] = acc[t][e];
            }
    }
}

// token tiles per wavefront: two when that still leaves about 1.5 wavefronts per SIMD of a
// 256-CU part, else one (a long row with few row groups keeps its wavefronts short)
static int gemmn_nt(const GemmNArgs &a) { return a.Tp >= 32 && a.groups * (a.Tp / 32) >= 1536 ? 2 : 1; }

template <int TYPE, int NT>
static void gemmn_launch(const GemmNArgs &a, hipStream_t s) {
    constexpr int D = NT == 1 ? 6 : 4;  // ring depth (within 256 VGPRs: two wavefronts per SIMD)
    const int64_t waves = a.groups * (a.Tp / (16 * NT));
    const dim3 grid((unsigned)((waves + 3) / 4));
    if (a.dump_s) q32n_gemm_kernel<TYPE, NT, 2, true><<<grid, 256, 0, s>>>(a);  // test hook: short ring
    else q32n_gemm_kernel<TYPE, NT, D, false><<<grid, 256, 0, s>>>(a);
}
template <int TYPE>
static void gemmn_launch_nt(const GemmNArgs &a, hipStream_t s) {
    if (gemmn_nt(a) == 2) gemmn_launch<TYPE, 2>(a, s);
    else gemmn_launch<TYPE, 1>(a, s);
}

hipError_t launch_q32n_gemm(const GemmNArgs &a, hipStream_t s) {
    if (a.T < 1 || a.T > a.Tp || a.Tp % 16 || a.Tp > 64 || a.Tp - a.T >= 16 || a.nb < 1 ||
        a.nsteps != (a.nb + 3) / 4 || a.groups < 1 || a.ppm != (a.tpm + 1) / 2 || a.rows > 8 * a.tpm)
        return hipErrorInvalidValue;
    switch (a.type) {
    case T_Q4_0: gemmn_launch_nt<T_Q4_0>(a, s); break;
    case T_Q4_1: gemmn_launch_nt<T_Q4_1>(a, s); break;
    case T_Q5_0: gemmn_launch_nt<T_Q5_0>(a, s); break;
    case T_Q5_1: gemmn_launch_nt<T_Q5_1>(a, s); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace fgh
