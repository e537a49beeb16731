// fgh_gemm6.hip - the prompt-batch (8..64 tokens) Q6_K x Q8_K matmul on gfx950 MFMA (the role of
// the reference's matmul -> gemm_kquant path for Q6_K, fastgguf.c:2704-2725, 2818-2854, 3023-3026).
//
// Y[tok * ldy + row] = sum_b d[row][b] * yd[tok][b] * isum, with the exact per-block integer of
// dot_q6_K_q8k (fastgguf.c:1232-1264) taken with its -32 offset inside:
//   isum = sum_g sc_g * sum_{16 values of g} (q - 32) * y = sumi - 32 msum
// (sumi = sum_g sc_g sum q y and msum = sum_g sc_g bs_g are the reference's two integers; the
// fp32 path needs only their combination).
//
// isum on int8 MFMA (v_mfma_i32_16x16x64_i8). A signed 8-bit scale times a 6-bit quant does not fit
// an int8 operand, so each scale is written in balanced base 8, sc = 64 d2 + 8 d1 + d0 with every
// digit in [-3, 4], and three chains run on pre-scaled weights w * dk (w = q - 32 in [-32, 31]:
// every product in [-128, 124]): isum = 64 C2 + 8 C1 + C0 exactly. A lane forms w * dk for 2
// values at a time in 16-bit lanes (one packed multiply-add, (q dk - 32 dk) mod 2^16, whose low byte
// is the signed product) and packs the low bytes back, so the -32 offset costs nothing.
//
// MFMA roles: A = activations (M = 16 tokens), B = weights (N = 16 rows: two 8-row decode tiles of
// one block). Lane l = 16 kg + n holds row n (tile n / 8, row n % 8) and takes slices 2 kg and
// 2 kg + 1 of the row from the decode layout (fgh_internal.h, Q6_K tile): the values with in-chunk
// index j in 8 kg .. 8 kg + 7 of every (half h, chunk c). In K-step t (0..3) it feeds the 16 values
// of (h, c) = (t / 2, 2 (t % 2) + c'), c' = 0, 1: byte 8 c' + j % 8, two scale groups (one per c').
// The activation record feeds lane (kg, m) the same 16 values of token m.
//
// Workgroup and pipeline as the Q4_K GEMM (fgh_gemm.hip): 4 tiles x KH K-halves, one wavefront
// each; the next step's records staged through registers into the other of two LDS stages; a ring
// of 4 blocks of weights per wavefront, three steps ahead; branch-free main steps.
//
// fp32 order: per (row, token) and block acc = fma(d * yd, float(isum), acc) over the wavefront's
// blocks, out = acc_half0 + acc_half1. The integers are exact; the fp32 result differs from
// gemmk_kern's order (fastgguf.c:2765-2797) only by rounding.
#include <type_traits>

#include "fgh_internal.h"

namespace fgh {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------------------------
// Activation records. Per 256-block b, at b * gemm6_rec_bytes(Tp), for Tp = 16 NT tokens (token
// tiles tt of 16, token tok = 16 tt + m):
//   [0, 256 Tp)        int8 fragments (tt, t), t = 0..3, 1 KB each at (4 tt + t) KB: lane
//                      l = 16 kg + m holds, at byte 8 c' + u, the quant of element
//                      128 h + 32 (2 (t % 2) + c') + 8 kg + u of token tok (h = t / 2)
//   [256 Tp, 260 Tp)   fp32 yd [Tp]
//   [260 Tp, 292 Tp)   int16 bsums [Tp][16] (the sums of each 16 quants; the integer dump's msum)
// Tokens T..Tp-1 are zeros.
// ---------------------------------------------------------------------------------------------
__host__ __device__ constexpr int gemm6_rec_bytes(int Tp) { return Tp * 292; }

// quantize_q8k (fastgguf.c:773-793, bit-exact) into the records: one wavefront per (block b, 4
// tokens); lane l = 16 u + p takes token 4 blockIdx.y + u and the 16 values 16 p .. 16 p + 15 of the
// block (scale group p). The block maximum combines the token's 16 lanes by lane exchanges; fmaxf
// ignores NaN, so any order gives the reference's maximum.
__global__ __launch_bounds__(64) void gemm6_quant_kernel(const float *__restrict__ x, int64_t ldx, int T, int Tp,
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
    uint8_t *r = rec + (size_t)b * gemm6_rec_bytes(Tp);
    // element 16 p + u: h = p / 8, c = (p / 2) % 4, j = 16 (p % 2) + u -> K-step t = 2 h + c / 2,
    // lane kg = j / 8, byte 8 (c % 2) + u % 8: values 0..7 and 8..15 go to consecutive lanes
    const int tt = tok >> 4, m = tok & 15, h = p >> 3, c = (p >> 1) & 3, t = 2 * h + (c >> 1);
    const int kg0 = 2 * (p & 1);
    uint8_t *f = r + (size_t)(4 * tt + t) * 1024 + 8 * (c & 1);
    *(uint2 *)(f + (16 * kg0 + m) * 16) = make_uint2(pk[0], pk[1]);
    *(uint2 *)(f + (16 * (kg0 + 1) + m) * 16) = make_uint2(pk[2], pk[3]);
    ((int16_t *)(r + 260 * Tp))[16 * tok + p] = (int16_t)s;
    if (p == 0) ((float *)(r + 256 * Tp))[tok] = d;
}

hipError_t launch_gemm6_quant(const float *x, int64_t ldx, int nb, int T, int Tp, uint8_t *rec, int32_t *cnt, int ncnt,
                              hipStream_t s) {
    if (ncnt < 0) return hipErrorInvalidValue;
    if (T < 1 || T > Tp || Tp % 16 || Tp > 64 || nb < 1) return hipErrorInvalidValue;
    gemm6_quant_kernel<<<dim3((unsigned)nb, (unsigned)(Tp / 4)), 64, 0, s>>>(x, ldx, T, Tp, rec, cnt, ncnt);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// The GEMM kernel
// ---------------------------------------------------------------------------------------------
// one lane's weights of one block: ql of slices 2 kg and 2 kg + 1 (dword 2 h + s: file bytes
// 64 h + 32 s + 4 i .. + 3), their qh (dwords (i - 2 kg) * 2 + h), its row's 16 scales and fp16 d
struct GW6 {
    v4i ql0, ql1, qh, sc;
    uint32_t d;
};
__device__ __forceinline__ v4i bld16v(BufRes r, uint32_t off) {
    return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));  // weights
}

// one step's activation records held by a thread between their load and their LDS write
struct ARec6 {
    uint4 v0, v1, v2, v3, v4, v5, v6, v7, v8, v9;
};

// the integer chains of one block of a wavefront
template <int NT>
struct GAcc6 {
    v4i c0[NT], c1[NT], c2[NT];
    float d;
};

// 4 six-bit quants from a ql dword (nibble at nsh) and a qh dword (2 bits at hsh), as bytes
__device__ __forceinline__ uint32_t six(uint32_t ql, uint32_t qh, int nsh, int hsh) {
    return ((ql >> nsh) & 0x0F0F0F0Fu) | (((qh >> hsh) & 0x03030303u) << 4);
}
// balanced base-8 digits of a scale (sc = 64 d2 + 8 d1 + d0, each in [-3, 4]) in both 16-bit
// lanes, with -32 times each (the offset of w = q - 32)
struct Dig6 {
    u16x2 m0, m1, m2, o0, o1, o2;
};
__device__ __forceinline__ Dig6 digits6(int sc) {
    const int d0 = ((sc + 3) & 7) - 3, t1 = (sc - d0) >> 3;
    const int d1 = ((t1 + 3) & 7) - 3, d2 = (t1 - d1) >> 3;
    const u16x2 m32 = {(unsigned short)0xFFE0, (unsigned short)0xFFE0};
    Dig6 g;
    g.m0 = u16x2{(unsigned short)d0, (unsigned short)d0};
    g.m1 = u16x2{(unsigned short)d1, (unsigned short)d1};
    g.m2 = u16x2{(unsigned short)d2, (unsigned short)d2};
    g.o0 = g.m0 * m32;
    g.o1 = g.m1 * m32;
    g.o2 = g.m2 * m32;
    return g;
}
// the 4 bytes (q - 32) * digit of 4 quant bytes: bytes 0, 2 and 1, 3 in 16-bit lanes, one packed
// multiply-add each, low bytes packed back in order
__device__ __forceinline__ uint32_t wmul(uint32_t lo, uint32_t hi, u16x2 m, u16x2 o) {
    const u16x2 pl = __builtin_bit_cast(u16x2, lo) * m + o, ph = __builtin_bit_cast(u16x2, hi) * m + o;
    return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, ph), __builtin_bit_cast(uint32_t, pl), 0x06020400u);
}

template <int NT, int KH, int TPW, bool DUMP>
__global__ __launch_bounds__(64 * TPW * KH) __attribute__((amdgpu_waves_per_eu(2, 2))) void q6k_gemm_kernel(Gemm6Args a) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int Tp = 16 * NT, REC = gemm6_rec_bytes(Tp), NTH = 64 * TPW * KH;
    constexpr int R = (KH * REC + 16 * NTH - 1) / (16 * NTH), SB = R * 16 * NTH;
    static_assert(R >= 1 && R <= 10, "one step's records take 1..10 rounds per thread");
    const int tid = threadIdx.x, l = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tw = wave % TPW, kh = wave / TPW;
    const int n = l & 15, kg = l >> 4, r8 = n & 7, dt = n >> 3;
    // K split ksi of a.ks (grid.y): blocks [b_lo, b_lo + nbk)
    const int nb = a.nb, ksi = blockIdx.y, nbs = (nb + a.ks - 1) / a.ks;
    const int b_lo = ksi * nbs, nbk = min(nb - b_lo, nbs);
    const int nsteps = (nbk + KH - 1) / KH;
    const int64_t tile = (int64_t)blockIdx.x * TPW + tw;
    const bool live = tile < a.groups;
    const int64_t tc = live ? tile : a.groups - 1;
    const int64_t mi = tc / a.gpm16, ti = tc - mi * a.gpm16;
    const int nvalid = (int)min<int64_t>(2, a.tpm - 2 * ti);  // decode tiles of the pair inside the matrix
    const int64_t rows = a.rows, row = ti * 16 + n;
    const bool store = live && row < rows;
    const int64_t orow = mi * rows + row;
    const uint32_t toff = (uint32_t)(dt * Q6K_TILE);
    const uint32_t qloff = toff + 144 + 16 * (8 * r8 + 2 * kg), qhoff = toff + 1168 + 8 * (8 * r8 + 2 * kg);
    const uint32_t scoff = toff + 16 * r8, doff = toff + 128 + 2 * r8;

    auto aload = [&](int s, ARec6 &ar) __attribute__((always_inline)) {
        // KH records from block b_lo + KH s (the buffer holds a record of slack past the last block)
        const int s2 = b_lo + KH * min(s, nsteps - 1), avail = min(KH, nb + 1 - s2);  // >= 2 records
        const BufRes src = buf_res(a.act + (size_t)s2 * REC, avail * REC);
        auto ld = [&](int k) __attribute__((always_inline)) { return bld16(src, 16 * (k * NTH + tid)); };
        ar.v0 = ld(0);
        if (R > 1) ar.v1 = ld(1);
        if (R > 2) ar.v2 = ld(2);
        if (R > 3) ar.v3 = ld(3);
        if (R > 4) ar.v4 = ld(4);
        if (R > 5) ar.v5 = ld(5);
        if (R > 6) ar.v6 = ld(6);
        if (R > 7) ar.v7 = ld(7);
        if (R > 8) ar.v8 = ld(8);
        if (R > 9) ar.v9 = ld(9);
    };
    auto astore = [&](uint8_t *st, const ARec6 &ar) __attribute__((always_inline)) {
        uint4 *dst = (uint4 *)st + tid;
        dst[0] = ar.v0;
        if (R > 1) dst[NTH] = ar.v1;
        if (R > 2) dst[2 * NTH] = ar.v2;
        if (R > 3) dst[3 * NTH] = ar.v3;
        if (R > 4) dst[4 * NTH] = ar.v4;
        if (R > 5) dst[5 * NTH] = ar.v5;
        if (R > 6) dst[6 * NTH] = ar.v6;
        if (R > 7) dst[7 * NTH] = ar.v7;
        if (R > 8) dst[8 * NTH] = ar.v8;
        if (R > 9) dst[9 * NTH] = ar.v9;
    };
    // block b_lo + KH s + kh of the tile pair; reads past the valid tiles (a matrix's last pair)
    // return 0
    auto wload = [&](int s, GW6 &w) __attribute__((always_inline)) {
        const int b = b_lo + min(KH * s + kh, nbk - 1);
        const BufRes r = buf_res(a.W + ((size_t)(mi * nb + b) * a.tpm + 2 * ti) * Q6K_TILE, nvalid * Q6K_TILE);
        w.ql0 = bld16v(r, qloff);
        w.ql1 = bld16v(r, qloff + 16);
        w.qh = bld16v(r, qhoff);
        w.sc = bld16v(r, scoff);
        w.d = bld2(r, doff);
    };

    v4f acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};

    // one block of this wavefront from stage st with weights w
    auto block = [&](const GW6 &w, const uint8_t *st, GAcc6<NT> &g, auto &&issue) __attribute__((always_inline)) {
        const uint8_t *rec = st + kh * REC;
        g.d = fp16_bits_to_f32(w.d & 0xFFFF);
        const int gsh = 8 * (kg >> 1);  // byte of the lane's scale groups within a scale word
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int h = t >> 1, nsh = 4 * (t & 1), cb = 2 * (t & 1);
            // scale groups 8 h + 2 cb + kg / 2 (c' = 0) and that + 2 (c' = 1), one word
            const uint32_t sw = (uint32_t)w.sc[2 * h + (t & 1)];
            const Dig6 g0 = digits6((int)(int8_t)(sw >> gsh)), g1 = digits6((int)(int8_t)(sw >> (gsh + 16)));
            uint32_t q[4];
            q[0] = six((uint32_t)w.ql0[2 * h], (uint32_t)w.qh[h], nsh, 2 * cb);
            q[1] = six((uint32_t)w.ql1[2 * h], (uint32_t)w.qh[2 + h], nsh, 2 * cb);
            q[2] = six((uint32_t)w.ql0[2 * h + 1], (uint32_t)w.qh[h], nsh, 2 * cb + 2);
            q[3] = six((uint32_t)w.ql1[2 * h + 1], (uint32_t)w.qh[2 + h], nsh, 2 * cb + 2);
            v4i b0, b1, b2;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const Dig6 &gg = k < 2 ? g0 : g1;
                const uint32_t lo = __builtin_amdgcn_perm(0u, q[k], 0x0C020C00u), hi = __builtin_amdgcn_perm(0u, q[k], 0x0C030C01u);
                b0[k] = (int)wmul(lo, hi, gg.m0, gg.o0);
                b1[k] = (int)wmul(lo, hi, gg.m1, gg.o1);
                b2[k] = (int)wmul(lo, hi, gg.m2, gg.o2);
            }
#pragma unroll
            for (int tt = 0; tt < NT; ++tt) {
                const uint4 au = *(const uint4 *)(rec + ((size_t)(4 * tt + t) * 64 + l) * 16);
                const v4i av = {(int)au.x, (int)au.y, (int)au.z, (int)au.w};
                const v4i z = {0, 0, 0, 0};
                g.c0[tt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b0, t == 0 ? z : g.c0[tt], 0, 0, 0);
                g.c1[tt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b1, t == 0 ? z : g.c1[tt], 0, 0, 0);
                g.c2[tt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b2, t == 0 ? z : g.c2[tt], 0, 0, 0);
            }
            issue(t);
        }
    };
    // block b's fp32 epilogue from its integers and its stage's yd (and, for the dump, msum from
    // the stage's bsums and the row's scales)
    auto epilogue = [&](const GAcc6<NT> &g, const GW6 &w, const uint8_t *st, int b) __attribute__((always_inline)) {
        const uint8_t *rec = st + kh * REC;
        const float *yds = (const float *)(rec + 256 * Tp);
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) {
            const v4f yd = *(const v4f *)(yds + 16 * tt + 4 * kg);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int isum = (((g.c2[tt][r] << 3) + g.c1[tt][r]) << 3) + g.c0[tt][r];
                acc[tt][r] = __builtin_fmaf(g.d * yd[r], (float)isum, acc[tt][r]);
                if (DUMP) {
                    const int tok = 16 * tt + 4 * kg + r;
                    if (store && tok < a.T) {
                        const int16_t *bs = (const int16_t *)(rec + 260 * Tp) + 16 * tok;
                        int msum = 0;
#pragma unroll
                        for (int gi = 0; gi < 16; ++gi)
                            msum += (int)(int8_t)((uint32_t)w.sc[gi >> 2] >> (8 * (gi & 3))) * (int)bs[gi];
                        const size_t di = ((size_t)tok * a.nrows + orow) * nb + b;
                        a.dump_s[di] = isum + 32 * msum;  // sumi, over the unsigned quants
                        a.dump_m[di] = msum;
                    }
                }
            }
        }
    };

    // prologue: step 0's records in LDS, the weights of steps 0..2 in flight
    GW6 w0, w1, w2, w3;
    ARec6 rr;
    GAcc6<NT> g;
    uint8_t *st0 = smem, *st1 = smem + SB;
    aload(0, rr);
    __builtin_amdgcn_sched_barrier(0);
    wload(0, w0);
    wload(1, w1);
    wload(2, w2);
    __builtin_amdgcn_sched_barrier(0);
    astore(st0, rr);
    __syncthreads();
    // step s: block KH s + kh from its stage and weights; the next step's records load after
    // K-step 0 and the weights of step s + 3 after K-step 2 (into the ring slot step s - 1 used);
    // then the epilogue, the records to the other stage, the barrier. Steps with a block for every
    // K-half run without branches (exact load counters); the last may test.
    auto step = [&](auto full, int s, GW6 &wc, GW6 &wn3, const uint8_t *stc, uint8_t *stn) __attribute__((always_inline)) {
        const int b = b_lo + KH * s + kh;
        auto issue = [&](int i) __attribute__((always_inline)) {
            __builtin_amdgcn_sched_barrier(0);
            if (i == 0) aload(s + 1, rr);
            if (i == 2) wload(s + 3, wn3);
            __builtin_amdgcn_sched_barrier(0);
        };
        if (decltype(full)::value || b < b_lo + nbk) {  // uniform per wavefront
            block(wc, stc, g, issue);
            epilogue(g, wc, stc, b);
        } else {
            issue(0);
            issue(2);
        }
        __builtin_amdgcn_sched_barrier(0);
        astore(stn, rr);
        __syncthreads();
    };
    using Full = std::true_type;
    using Edge = std::false_type;
    const int nfull = nbk / KH;
    int s = 0;
    for (; s + 4 <= nfull; s += 4) {
        step(Full(), s, w0, w3, st0, st1);
        step(Full(), s + 1, w1, w0, st1, st0);
        step(Full(), s + 2, w2, w1, st0, st1);
        step(Full(), s + 3, w3, w2, st1, st0);
    }
    if (s < nsteps) step(Edge(), s, w0, w3, st0, st1);
    if (s + 1 < nsteps) step(Edge(), s + 1, w1, w0, st1, st0);
    if (s + 2 < nsteps) step(Edge(), s + 2, w2, w1, st0, st1);
    if (s + 3 < nsteps) step(Edge(), s + 3, w3, w2, st1, st0);
    __syncthreads();  // every wavefront is past its reads of the stages (the reduction reuses them)
    if (KH == 2) {  // half 1 -> LDS, half 0 adds it in order
        float *red = (float *)smem + (size_t)tw * 64 * 4 * NT;  // TPW * 4 KB * NT <= one stage
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
    // a K split (at least 8 blocks, so KH = 2) puts its flag at LDS int 4096, inside the stages
    static_assert(KH == 1 || 2 * SB >= 4 * 4096 + 4, "the K split's flag lies inside the stages");
    if (a.ks > 1) {  // the K split's partials (the reduction's LDS area is done with)
        gemm_split_finish<4 * NT>([&](int e) { return 16 * (e >> 2) + 4 * kg + (e & 3); },
                                  [&](int e) { return acc[e >> 2][e & 3]; }, kh == 0, store, tid, tw, TPW, orow, a.ks,
                                  ksi, a.T, a.ldy, a.part, a.cnt, a.Y, (int *)smem + 4096);
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

constexpr int GEMM6_TPW = 4;  // 16-row tiles per workgroup
static int gemm6_kh(int nb) { return nb >= 2 ? 2 : 1; }
template <int NT, int KH>
static size_t gemm6_lds() {
    const int nth = 64 * GEMM6_TPW * KH, r = (KH * gemm6_rec_bytes(16 * NT) + 16 * nth - 1) / (16 * nth);
    return (size_t)2 * r * 16 * nth;
}

size_t gemm6_act_bytes(int nb, int Tp) { return (size_t)(nb + 1) * gemm6_rec_bytes(Tp); }

template <int NT, int KH>
static void gemm6_launch(const Gemm6Args &a, hipStream_t s) {
    const dim3 grid((unsigned)((a.groups + GEMM6_TPW - 1) / GEMM6_TPW), (unsigned)a.ks);
    const size_t lds = gemm6_lds<NT, KH>();
    if (a.dump_s) q6k_gemm_kernel<NT, KH, GEMM6_TPW, true><<<grid, 64 * GEMM6_TPW * KH, lds, s>>>(a);
    else q6k_gemm_kernel<NT, KH, GEMM6_TPW, false><<<grid, 64 * GEMM6_TPW * KH, lds, s>>>(a);
}
template <int NT>
static void gemm6_launch_kh(const Gemm6Args &a, hipStream_t s) {
    if (gemm6_kh(a.nb) == 2) gemm6_launch<NT, 2>(a, s);
    else gemm6_launch<NT, 1>(a, s);
}

hipError_t launch_q6k_gemm(const Gemm6Args &a, hipStream_t s) {
    if (a.T < 1 || a.T > a.Tp || a.Tp % 16 || a.Tp > 64 || a.Tp - a.T >= 16 || a.nb < 1 || a.groups < 1 ||
        a.gpm16 != (a.tpm + 1) / 2)
        return hipErrorInvalidValue;
    if (a.ks < 1 || a.ks > 4 || (a.ks > 1 && (!a.part || !a.cnt || gemm6_kh(a.nb) == 1))) return hipErrorInvalidValue;
    switch (a.Tp / 16) {
    case 1: gemm6_launch_kh<1>(a, s); break;
    case 2: gemm6_launch_kh<2>(a, s); break;
    case 3: gemm6_launch_kh<3>(a, s); break;
    default: gemm6_launch_kh<4>(a, s); break;
    }
    return hipGetLastError();
}

}  // namespace fgh
