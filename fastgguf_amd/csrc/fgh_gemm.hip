// fgh_gemm.hip - the prompt-batch (8..64 tokens) Q4_K x Q8_K matmul on gfx950 MFMA (the role of
// the reference's matmul -> gemm_kquant path, fastgguf.c:2756-2854 and 3004-3031).
//
// Y[tok * ldy + row] = sum_b yd[tok][b] * (d[row][b] * isum - dmin[row][b] * msum), with the exact
// per-block integers of dot_q4_K_q8k (fastgguf.c:1118-1176):
//   isum = sum_g sc_g * sum_{32 values of g} q * y        msum = sum_g m_g * bs_g
// (bs_g = bsums[2g] + bsums[2g+1], the sum of sub-block g's 32 quantized activations).
//
// isum on int8 MFMA (v_mfma_i32_16x16x64_i8). The 6-bit sub-block scale times a 4-bit quant does
// not fit an int8 operand (q * sc <= 945), so sc = 8 sh + sl (sh, sl <= 7) and two chains run on
// pre-scaled weights q * sh and q * sl (both <= 105; one packed 16-bit multiply per 4 values):
// isum = 8 Ch + Cl exactly.
// msum on f16 MFMA (v_mfma_f32_16x16x16_f16), exact: bs in [-4064, 4064] is split bs = 64 bh + bl
// (bl in [0, 63], bh in [-64, 63]); the 16 K-slots hold bl_g against m_g and bh_g against 64 m_g,
// all exact in f16, every product and partial sum an integer below 2^24 in magnitude, so the
// fp32 result is msum exactly, already a float.
//
// MFMA roles: A = activations (M = 16 tokens), B = weights (N = 16 rows of one Q4_K tile). A lane
// l = 16 kg + n holds output row n and tokens 4 kg .. 4 kg + 3 of its token tile, so a row's d,
// dmin, scales and mins are per-lane constants. The weights come straight from the decode layout
// (fgh_q4k.hip): lane (kg, n) loads chunk kg of row n as the decode kernel's lane 4 n + kg does
// (two 16-byte slots and the row's 16-byte meta; each load instruction reads 1 KB contiguous),
// so the GEMM needs no second copy of the weights. In K-step i (0..3) of a block the lane feeds
// the low (i < 2) or high (i >= 2) nibbles of its slot i & 1: 16 values of sub-block 2 kg or
// 2 kg + 1. The activation record feeds lane (kg, m) the same 16 K positions of token m, so the
// products pair up whatever order the hardware uses inside one K step.
//
// Workgroup: 4 tiles (64 rows) x KH K-halves, one wavefront each (KH = 2: two per SIMD). Block b
// is walked by K-half b % KH. Each step the workgroup loads the activation records of the step
// three ahead (launch_gemm_quant's layout, 1 KB contiguous per wavefront load) straight into one
// of four LDS stages (buffer loads to LDS) while it computes, and each wavefront keeps a ring of
// 4 blocks of its weights in registers (three steps ahead). A step's barrier waits only for the
// records of the next step, not for the weights loaded after them.
//
// Short output (fewer row groups than compute units): grid.y = ks K splits of consecutive blocks
// (gemm_splits); each split's workgroup writes its partial and the last of a row group's splits to
// arrive adds them in split order.
//
// fp32 order: per (row, token) and block t = fma(-dmin, msum, d * float(isum)),
// acc = fma(yd, t, acc) over the wavefront's blocks; out = acc_half0 + acc_half1 (then, with a K
// split, ((part_0 + part_1) + part_2) + part_3). The integers are exact; the fp32 result differs
// from gemmk_kern's order (fastgguf.c:2765-2797) only by rounding.
#include <type_traits>

#include "fgh_internal.h"

namespace fgh {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------------------------
// Activation records. Per 256-block b, at b * gemm_rec_bytes(Tp), for Tp = 16 NT tokens (token
// tiles tt of 16, token t = 16 tt + m):
//   [0, 256 Tp)        int8 fragments (tt, i), i = 0..3, 1 KB each at (4 tt + i) KB: lane
//                      l = 16 kg + m holds the 16 quants of token t at K positions
//                      32 (2 kg + (i >> 1)) + 16 ((i & 1) ^ (kg >> 1)) + 0..15 of the block
//   [256 Tp, 288 Tp)   f16 min fragments tt, 512 B each: lane (kg, m) holds bl of sub-blocks
//                      4 kg .. 4 kg + 3 (kg < 2) or bh of sub-blocks 4 (kg - 2) .. + 3 (kg >= 2)
//   [288 Tp, 292 Tp)   fp32 yd [Tp]
// Tokens T..Tp-1 are zeros.
// ---------------------------------------------------------------------------------------------
__host__ __device__ constexpr int gemm_rec_bytes(int Tp) { return Tp * 292; }

// quantize_q8k (fastgguf.c:773-793, bit-exact) into the records: one wavefront per (block b,
// 4 tokens); lane l = 16 u + p takes token 4 blockIdx.y + u and the 16 values 16 p .. 16 p + 15 of
// the block (piece p of sub-block g = p / 2). The block maximum and the 32-value sums combine
// lanes of one token by lane exchanges (no LDS, no barrier); fmaxf ignores NaN, so any order
// gives the reference's maximum.
__global__ __launch_bounds__(64) void gemm_quant_kernel(const float *__restrict__ x, int64_t ldx, int T, int Tp,
                                                        uint8_t *__restrict__ rec, int32_t *__restrict__ cnt, int ncnt) {
    const int l = threadIdx.x, p = l & 15;
    if (blockIdx.x == 0 && blockIdx.y == 0)
        for (int i = l; i < ncnt; i += 64) cnt[i] = 0;  // the K split's arrival counters
    const int b = blockIdx.x, tok = 4 * blockIdx.y + (l >> 4);
    float v[16];
    if (tok < T) {
        const float *src = x + (size_t)tok * ldx + (size_t)b * 256 + 16 * p;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const float4 f = *(const float4 *)(src + 4 * u);
            v[4 * u] = f.x; v[4 * u + 1] = f.y; v[4 * u + 2] = f.z; v[4 * u + 3] = f.w;
        }
    } else {
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] = 0.0f;
    }
    float amax = 0.0f;
#pragma unroll
    for (int u = 0; u < 16; ++u) amax = fmaxf(amax, fabsf(v[u]));
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    uint32_t pk[4];
    int s = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int q0 = q8_round(v[4 * u] * id), q1 = q8_round(v[4 * u + 1] * id);
        const int q2 = q8_round(v[4 * u + 2] * id), q3 = q8_round(v[4 * u + 3] * id);
        s += q0 + q1 + q2 + q3;
        pk[u] = pack_q(q0, q1, q2, q3);
    }
    uint8_t *r = rec + (size_t)b * gemm_rec_bytes(Tp);
    const int tt = tok >> 4, m = tok & 15, g = p >> 1, kg = g >> 1;
    // piece p = 2 g + h lands in fragment i = 2 (g & 1) + (h ^ (kg >> 1)) of lane 16 kg + m
    const int i = 2 * (g & 1) + ((p & 1) ^ (kg >> 1));
    *(uint4 *)(r + ((size_t)(4 * tt + i) * 64 + 16 * kg + m) * 16) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    s += __shfl_xor(s, 1, 64);  // the sub-block's two pieces
    if ((p & 1) == 0) {
        const int bl = s & 63, bh = s >> 6;  // s = 64 bh + bl
        _Float16 *mn = (_Float16 *)(r + 256 * Tp + (size_t)tt * 512);
        mn[(16 * (g >> 2) + m) * 4 + (g & 3)] = (_Float16)bl;
        mn[(16 * (2 + (g >> 2)) + m) * 4 + (g & 3)] = (_Float16)bh;
    }
    if (p == 0) ((float *)(r + 288 * Tp))[tok] = d;
}

hipError_t launch_gemm_quant(const float *x, int64_t ldx, int nb, int T, int Tp, uint8_t *rec, int32_t *cnt, int ncnt,
                             hipStream_t s) {
    if (T < 1 || T > Tp || Tp % 16 || Tp > 64 || nb < 1 || ncnt < 0) return hipErrorInvalidValue;
    gemm_quant_kernel<<<dim3((unsigned)nb, (unsigned)(Tp / 4)), 64, 0, s>>>(x, ldx, T, Tp, rec, cnt, ncnt);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// The GEMM kernel
// ---------------------------------------------------------------------------------------------


// one lane's weights of one block: slots 0 and 1 of its chunk and its row's meta (rb_load's loads)
struct GW {
    uint4 p0, p1, m;
};
__device__ __forceinline__ void gw_load(const uint8_t *blk, int L, int n, GW &w) {
    const BufRes r = buf_res(blk, 2304);
    w.p0 = bld16(r, 256 + 16 * L);
    w.p1 = bld16(r, 1280 + 16 * L);
    w.m = bld16(r, 16 * n);
}


// the integer results of one block of a wavefront
template <int NT>
struct GAcc {
    v4i ch[NT], cl[NT];
    v4f ms[NT];
    float d, dmin;
};

// bytes of q (each <= 15) times a small factor (<= 7) in both 16-bit lanes: no carry between bytes
__device__ __forceinline__ uint32_t bmul(uint32_t q, uint32_t f2) {
    const u16x2 r = __builtin_bit_cast(u16x2, q) * __builtin_bit_cast(u16x2, f2);
    return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ v4i u4v(uint4 u) { return v4i{(int)u.x, (int)u.y, (int)u.z, (int)u.w}; }

// TPW tiles x KH K-halves per workgroup, one wavefront each; with at most 2 wavefronts per SIMD
// the compiler may use up to 256 VGPRs per wavefront (all of them VGPRs, so the epilogue reads
// the MFMA results without moves).
template <int NT, int KH, int TPW, bool DUMP>
__global__ __launch_bounds__(64 * TPW * KH) __attribute__((amdgpu_waves_per_eu(2, 2))) void q4k_gemm_kernel(GemmArgs a) {
    constexpr int Tp = 16 * NT, REC = gemm_rec_bytes(Tp), NTH = 64 * TPW * KH;
    constexpr int R = (KH * REC + 16 * NTH - 1) / (16 * NTH), SB = R * 16 * NTH;
    static_assert(GEMM_NST * SB <= 163840, "the record stages fit the workgroup's 160 KiB of LDS");
    // four separate arrays, so that the compiler sees a stage's LDS reads never meet the loads
    // landing in the other stages (one array would make it wait for them before every read)
    __shared__ __align__(16) uint8_t sa0[SB];
    __shared__ __align__(16) uint8_t sa1[SB];
    __shared__ __align__(16) uint8_t sa2[SB];
    __shared__ __align__(16) uint8_t sa3[SB];
    const int tid = threadIdx.x, l = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tw = wave % TPW, kh = wave / TPW;
    const int n = l & 15, kg = l >> 4, L = 4 * n + kg;
    // K split ksi of a.ks: blocks [b_lo, b_lo + nbk)
    const int nb = a.nb, ksi = blockIdx.y, nbs = (nb + a.ks - 1) / a.ks;
    const int b_lo = ksi * nbs, nbk = min(nb - b_lo, nbs);
    const int nsteps = (nbk + KH - 1) / KH;
    const int64_t tile = (int64_t)blockIdx.x * TPW + tw;
    const bool live = tile < a.groups;
    const int64_t tc = live ? tile : a.groups - 1;
    const int64_t mi = tc / a.gpm, ti = tc - mi * a.gpm;
    const size_t bstride = (size_t)a.gpm * 2304;
    const uint8_t *W0 = a.W + ((size_t)mi * nb * a.gpm + (size_t)ti) * 2304;

    // the step's records: a linear copy of KH records from block b_lo + KH s (the quantizer's
    // buffer holds a record of slack past the last block) into a stage (gemm_dma)
    static_assert(R >= 1 && R <= 10, "one step's records take 1..10 rounds per thread");
    auto adma = [&](int s, uint8_t *st) {
        const int s2 = b_lo + KH * min(s, nsteps - 1), avail = min(KH, nb + 1 - s2);  // >= 2 records
        gemm_dma<R, NTH>(buf_res(a.act + (size_t)s2 * REC, avail * REC), st, wave, tid);
    };
    // a step ends once step s + 1's records have landed: the loads issued after them are the
    // weights of s + 1, the records and weights of s + 2 and of s + 3 (3 + R + 3 + R + 3). The
    // dump form's stores are memory operations of the same counter, issued among them: it waits
    // for everything.
    auto stage_barrier = [&]() { gemm_stage_barrier<DUMP ? 0 : 9 + 2 * R>(); };
    auto wload = [&](int s, GW &w) {
gw_load(W0 + (size_t)(b_lo + min(KH * s + kh, nbk - 1)) * bstride, L, n, w); };

    v4f acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
    const int64_t rows = a.rows, row = ti * 16 + n;
    const bool store = live && row < rows;
    const int64_t orow = mi * rows + row;

    // one block of this wavefront from stage st with weights w
    auto block = [&](const GW &w, const uint8_t *st, GAcc<NT> &g, auto &&issue) {
        const uint8_t *rec = st + kh * REC;
        // sub-block scales 2 kg and 2 kg + 1 as bytes 0 and 1 of scp (scale_min_k4, fastgguf.c:466-472)
        const int sh = 16 * (kg & 1);
        const uint32_t A = w.m.y >> sh, C = w.m.w >> sh;
        const uint32_t sc_lo = A & 0x3f3fu, sc_hi = (C & 0x0f0fu) | ((A >> 2) & 0x3030u);
        const uint32_t scp = kg >= 2 ? sc_hi : sc_lo;
        // split factors of the two sub-blocks in both 16-bit lanes
        const uint32_t fh0 = ((scp >> 3) & 7u) * 0x10001u, fl0 = (scp & 7u) * 0x10001u;
        const uint32_t fh1 = ((scp >> 11) & 7u) * 0x10001u, fl1 = ((scp >> 8) & 7u) * 0x10001u;
        // the eight 6-bit mins: m0..m3 in the bytes of u1 & 0x3f3f3f3f, m4..m7 of the nibbles of u2
        // with u1's top bits; lanes kg & 1 take the second four, as f16 (1024 + m) - 1024, times 64
        // for kg >= 2
        const uint32_t mlo = w.m.z & 0x3f3f3f3fu;
        const uint32_t mhi = ((w.m.w >> 4) & 0x0f0f0f0fu) | (((w.m.z >> 6) & 0x03030303u) << 4);
        const uint32_t mw = (kg & 1) ? mhi : mlo;
        const h2v k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
        const h2v msc = kg >= 2 ? h2v{(_Float16)64.0f, (_Float16)64.0f} : h2v{(_Float16)1.0f, (_Float16)1.0f};
        const h2v m01 = (__builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, mw, 0x04010400u)) - k1024) * msc;
        const h2v m23 = (__builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, mw, 0x04030402u)) - k1024) * msc;
        const v4h bmin = {m01[0], m01[1], m23[0], m23[1]};
        g.d = fp16_bits_to_f32(w.m.x & 0xFFFF);
        g.dmin = fp16_bits_to_f32(w.m.x >> 16);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const uint2 am = *(const uint2 *)(rec + 256 * Tp + (size_t)t * 512 + 8 * l);
            g.ms[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(v4h, am), bmin, v4f{0.f, 0.f, 0.f, 0.f},
                                                          0, 0, 0);
        }
        const uint32_t P0[4] = {w.p0.x, w.p0.y, w.p0.z, w.p0.w}, P1[4] = {w.p1.x, w.p1.y, w.p1.z, w.p1.w};
        // the A fragments of K-step i are read from LDS during K-step i - 1
        auto afrag = [&](int t, int i) { return u4v(*(const uint4 *)(rec + ((size_t)(4 * t + i) * 64 + l) * 16)); };
        v4i av[NT], an[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) av[t] = afrag(t, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (i < 3) {
#pragma unroll
                for (int t = 0; t < NT; ++t) an[t] = afrag(t, i + 1);
            }
            const uint32_t fh = i < 2 ? fh0 : fh1, fl = i < 2 ? fl0 : fl1;
            v4i bh, bl;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t p = (i & 1) ? P1[k] : P0[k];
                const uint32_t v = i < 2 ? (p & 0x0F0F0F0Fu) : ((p >> 4) & 0x0F0F0F0Fu);
                bh[k] = (int)bmul(v, fh);
                bl[k] = (int)bmul(v, fl);
            }
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                if (i == 0) {
                    g.ch[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[t], bh, v4i{0, 0, 0, 0}, 0, 0, 0);
                    g.cl[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[t], bl, v4i{0, 0, 0, 0}, 0, 0, 0);
                } else {
                    g.ch[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[t], bh, g.ch[t], 0, 0, 0);
                    g.cl[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[t], bl, g.cl[t], 0, 0, 0);
                }
            }
            if (i < 3) {
#pragma unroll
                for (int t = 0; t < NT; ++t) av[t] = an[t];
            }
            issue(i);
        }
    };
    // block b's fp32 epilogue from its integers and its stage's yd
    auto epilogue = [&](const GAcc<NT> &g, const uint8_t *st, int b) {
        const float *yds = (const float *)(st + kh * REC + 288 * Tp);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float4 yd = *(const float4 *)(yds + 16 * t + 4 * kg);
            const float ydv[4] = {yd.x, yd.y, yd.z, yd.w};
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int isum = (g.ch[t][r] << 3) + g.cl[t][r];
                const float tt = __builtin_fmaf(-g.dmin, g.ms[t][r], g.d * (float)isum);
                acc[t][r] = __builtin_fmaf(ydv[r], tt, acc[t][r]);
                if (DUMP) {
                    const int tok = 16 * t + 4 * kg + r;
                    if (store && tok < a.T) {
                        const size_t di = ((size_t)tok * a.nrows + orow) * nb + b;
                        a.dump_s[di] = isum;
                        a.dump_m[di] = (int)g.ms[t][r];
                    }
                }
            }
        }
    };

    // prologue: the records of steps 0..2 into stages 0..2 and the weights of steps 0..2, each
    // step's records then weights (the order the steps keep); step 0's records landed
    GW w0, w1, w2, w3;
    GAcc<NT> g;
    uint8_t *const st0 = sa0, *const st1 = sa1, *const st2 = sa2, *const st3 = sa3;
    // (the scheduling barriers keep the loads in this order: the barrier's count relies on it)
    __builtin_amdgcn_sched_barrier(0);
    adma(0, st0);
    __builtin_amdgcn_sched_barrier(0);
    wload(0, w0);
    __builtin_amdgcn_sched_barrier(0);
    adma(1, st1);
    __builtin_amdgcn_sched_barrier(0);
    wload(1, w1);
    __builtin_amdgcn_sched_barrier(0);
    adma(2, st2);
    __builtin_amdgcn_sched_barrier(0);
    wload(2, w2);
    stage_barrier();
    // step s: compute step s from its stage and weights; between its K-steps load step s + 3's
    // records (after K-step 0, into the stage step s - 1 used, free since the last barrier) and
    // step s + 3's weights (after K-step 2, into the ring slot step s - 1 used); then the
    // epilogue and the barrier, once step s + 1's records have landed. Every step issues the
    // same loads (the last ones re-read the last step's), so the count the barrier waits for is
    // the same at every step. Issued at the top of the step instead, the workgroup's loads fill
    // the address queue and every wavefront waits to issue them before computing. The main
    // loop's steps have a block for every K-half and no branch, so the compiler's load counters
    // stay exact across them (a branch makes it wait for every outstanding load, the prefetches
    // included, at the next block); the last steps test.
    auto step = [&](auto full, int s, GW &wc, GW &wn3, const uint8_t *stc, uint8_t *st3n) {
        const int b = b_lo + KH * s + kh;
        auto issue = [&](int i) {
            __builtin_amdgcn_sched_barrier(0);
            if (i == 0) adma(s + 3, st3n);
            if (i == 2) wload(s + 3, wn3);
            __builtin_amdgcn_sched_barrier(0);
        };
        if (decltype(full)::value || b < b_lo + nbk) {  // uniform per wavefront
            block(wc, stc, g, issue);
            epilogue(g, stc, b);
        } else {
            issue(0);
            issue(2);
        }
        stage_barrier();
    };
    using Full = std::true_type;
    using Edge = std::false_type;
    const int nfull = nbk / KH;  // steps with a block for every K-half
    int s = 0;
    for (; s + 4 <= nfull; s += 4) {
        step(Full(), s, w0, w3, st0, st3);
        step(Full(), s + 1, w1, w0, st1, st0);
        step(Full(), s + 2, w2, w1, st2, st1);
        step(Full(), s + 3, w3, w2, st3, st2);
    }
    // the remaining steps (at most 4), with the same rings and stages
    if (s < nsteps) step(Edge(), s, w0, w3, st0, st3);
    if (s + 1 < nsteps) step(Edge(), s + 1, w1, w0, st1, st0);
    if (s + 2 < nsteps) step(Edge(), s + 2, w2, w1, st2, st1);
    if (s + 3 < nsteps) step(Edge(), s + 3, w3, w2, st3, st2);
    // every load has landed (the last steps' loads into stages past the last step included) and
    // every wavefront is past its reads of the stages: the reduction reuses them
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (KH == 2) {  // half 1 -> LDS, half 0 adds it in order
        // tiles 0, 1 in stage 0, tiles 2, 3 in stage 1: 2 x 4 KB x NT <= one stage
        static_assert(KH == 1 || (TPW <= 4 && 2 * 4096 * NT <= SB), "the reduction fits two stages");
        float *red = (float *)(tw < 2 ? st0 : st1) + (size_t)(tw & 1) * 64 * 4 * NT;
        if (kh == 1) {
#pragma unroll
            for (int t = 0; t < NT; ++t) *(v4f *)(red + (size_t)(t * 64 + l) * 4) = acc[t];
        }
        __syncthreads();
        if (kh == 0) {
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[t] += *(const v4f *)(red + (size_t)(t * 64 + l) * 4);
        }
    }
    // a K split (at least 8 blocks, so KH = 2) puts its flag in stage 2 (the reduction used 0, 1)
    if (a.ks > 1) {  // the K split's partials (the reduction's LDS area is done with)
        gemm_split_finish<4 * NT>([&](int e) { return 16 * (e >> 2) + 4 * kg + (e & 3); },
                                  [&](int e) { return acc[e >> 2][e & 3]; }, kh == 0, store, tid, tw, TPW, orow, a.ks,
                                  ksi, a.T, a.ldy, a.part, a.cnt, a.Y, (int *)st2);
        return;
    }
    if (kh == 0 && store) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int tok = 16 * t + 4 * kg + r;
                if (tok < a.T) a.Y[(size_t)tok * a.ldy + orow] = acc[t][r];
            }
    }
}

static int gemm_kh(int nb) { return nb >= 2 ? 2 : 1; }  // wavefronts per tile (K-halves)
constexpr int GEMM_TPW = 4;                              // tiles per workgroup
size_t gemm_act_bytes(int nb, int Tp) { return (size_t)(nb + 1) * gemm_rec_bytes(Tp); }

template <int NT, int KH>
static void gemm_launch(const GemmArgs &a, hipStream_t s) {
    constexpr int TPW = GEMM_TPW;
    const dim3 grid((unsigned)((a.groups + TPW - 1) / TPW), (unsigned)a.ks);
    // the record stages are the kernel's static LDS
    if (a.dump_s) q4k_gemm_kernel<NT, KH, TPW, true><<<grid, 64 * TPW * KH, 0, s>>>(a);
    else q4k_gemm_kernel<NT, KH, TPW, false><<<grid, 64 * TPW * KH, 0, s>>>(a);
}
template <int NT>
static void gemm_launch_kh(const GemmArgs &a, hipStream_t s) {
    if (gemm_kh(a.nb) == 2) gemm_launch<NT, 2>(a, s);
    else gemm_launch<NT, 1>(a, s);
}

static size_t up256(size_t n) { return (n + 255) / 256 * 256; }
GemmScratch gemm_split_scratch(size_t rec_bytes, int64_t wg, int units, int min_units, int Tp, int num_cu) {
    GemmScratch g;
    g.ks = 1;
    while (g.ks < 4 && wg * (g.ks + 1) <= num_cu && units / (g.ks + 1) >= min_units) ++g.ks;
    g.ncnt = g.ks > 1 ? (int)wg : 0;
    g.cnt_off = up256(rec_bytes);
    g.part_off = g.cnt_off + up256((size_t)g.ncnt * 4);
    g.bytes = g.ks > 1 ? g.part_off + (size_t)g.ks * wg * 64 * Tp * 4 : rec_bytes;
    return g;
}
// the Q4_K GEMM: workgroups of 4 tiles, splits of at least 4 blocks
GemmScratch gemm_scratch(int64_t groups, int nb, int T, int num_cu) {
    const int Tp = (T + 15) / 16 * 16;
    return gemm_split_scratch(gemm_act_bytes(nb, Tp), (groups + GEMM_TPW - 1) / GEMM_TPW, nb, 4, Tp, num_cu);
}
hipError_t launch_q4k_gemm(const GemmArgs &a, hipStream_t s) {
    if (a.T < 1 || a.T > a.Tp || a.Tp % 16 || a.Tp > 64 || a.Tp - a.T >= 16 || a.nb < 1 || a.groups < 1)
        return hipErrorInvalidValue;
    if (a.ks < 1 || a.ks > 4 || (a.ks > 1 && (!a.part || !a.cnt || gemm_kh(a.nb) == 1))) return hipErrorInvalidValue;
    switch (a.Tp / 16) {
    case 1: gemm_launch_kh<1>(a, s); break;
    case 2: gemm_launch_kh<2>(a, s); break;
    case 3: gemm_launch_kh<3>(a, s); break;
    default: gemm_launch_kh<4>(a, s); break;
    }
    return hipGetLastError();
}

}  // namespace fgh
