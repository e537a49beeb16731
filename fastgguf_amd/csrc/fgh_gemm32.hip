// fgh_gemm32.hip - the prompt-batch (8..64 tokens) Q8_0 x Q8 matmul on gfx950 MFMA (the role of the
// reference's matmul -> gemm_q32 path, fastgguf.c:2856-2999 and 3027-3030).
//
// Y[tok * ldy + row] = sum_b d[row][b] * xd[tok][b] * isum, with the exact per-block integers of
// dot_q8_0_q8 (fastgguf.c:891-902): isum = sum_{32 values of block b} q * xq.
//
// One Q8_0 block is one K = 32 step of v_mfma_i32_32x32x32_i8 (A = 32 tokens, B = 32 rows), so the
// block's integer comes out of the matrix unit whole: the quants are the B operand as they are,
// with no unpacking and no scale splitting, and each (token, row, block) costs one MFMA share and
// three VALU instructions (convert, d * xd, fma). The weights come straight from the decode
// layout (fgh_internal.h, Q8_0 tile: 8 rows x 4 blocks): lane (h, n) of a 32-row group takes row
// n and the 16 values 16 h .. 16 h + 15 of each block from slices 4 h .. 4 h + 3 of its row (64
// contiguous bytes per step) and its row's four fp16 d; the activation record gives lane (h, m)
// the same 16 values of token m.
//
// Workgroup: TPW groups of 32 rows x KH K-parts, one wavefront each (two per SIMD). A step is one
// tile step (4 blocks); step s is walked by K-part s % KH. Each workgroup step loads the next
// step's activation records (KH tile steps, 1 KB contiguous per wavefront load) into registers
// while it computes and writes them to the other of two LDS stages before its barrier; each
// wavefront keeps a ring of 4 steps of its weights in registers (three steps ahead).
//
// fp32 order: per (row, token) acc = fma(d * xd, float(isum), acc) over the K-part's blocks in
// order, out = ((acc_0 + acc_1) + acc_2) + acc_3. The integers are exact; the fp32 result
// differs from gemm32_kern's order (fastgguf.c:2919-2948) only by rounding.
#include <type_traits>

#include "fgh_internal.h"

namespace fgh {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------------------------------------
// Activation records. Per tile step s (4 blocks of 32 values), at s * gemm32_rec_bytes(Tp), for
// Tp = 32 NT tokens (token tiles tt of 32, token t = 32 tt + m):
//   [0, 128 Tp)        int8 fragments (bb, tt), 1 KB each at (bb NT + tt) KB: lane l = 32 h + m
//                      holds the 16 quants 16 h .. 16 h + 15 of block 4 s + bb of token t
//   [128 Tp, 144 Tp)   fp32 xd [4][Tp]
// Tokens T..Tp-1 and blocks past the row's last are zeros.
// ---------------------------------------------------------------------------------------------
__host__ __device__ constexpr int gemm32_rec_bytes(int Tp) { return Tp * 144; }

// quantize_q8 (fastgguf.c:746-770, bit-exact) into the records: one wavefront per (block b, 32
// tokens); lane l = 32 h + m takes token 32 blockIdx.y + m and values 16 h .. 16 h + 15 of the
// block. The block maximum combines the lane pair (m, m + 32); fmaxf ignores NaN, as the
// reference's comparison does.
__global__ __launch_bounds__(64) void gemm32_quant_kernel(const float *__restrict__ x, int64_t ldx, int nb, int T,
                                                          int Tp, uint8_t *__restrict__ rec, int32_t *__restrict__ cnt,
                                                          int ncnt) {
    const int l = threadIdx.x, h = l >> 5, m = l & 31;
    if (blockIdx.x == 0 && blockIdx.y == 0)
        for (int i = l; i < ncnt; i += 64) cnt[i] = 0;  // the K split's arrival counters
    const int b = blockIdx.x, tt = blockIdx.y, tok = 32 * tt + m;
    float v[16];
    if (tok < T && b < nb) {
        const float *src = x + (size_t)tok * ldx + (size_t)b * 32 + 16 * h;
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
    amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    uint32_t pk[4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
        pk[u] = pack_q(q8_round(v[4 * u] * id), q8_round(v[4 * u + 1] * id), q8_round(v[4 * u + 2] * id),
                       q8_round(v[4 * u + 3] * id));
    const int NT = Tp / 32, bb = b & 3;
    uint8_t *r = rec + (size_t)(b >> 2) * gemm32_rec_bytes(Tp);
    *(uint4 *)(r + ((size_t)(bb * NT + tt) * 64 + l) * 16) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    if (h == 0) ((float *)(r + 128 * Tp))[bb * Tp + tok] = d;
}

hipError_t launch_gemm32_quant(const float *x, int64_t ldx, int nb, int T, int Tp, uint8_t *rec, int32_t *cnt, int ncnt,
                               hipStream_t s) {
    if (ncnt < 0) return hipErrorInvalidValue;
    if (T < 1 || T > Tp || Tp % 32 || Tp > 64 || nb < 1) return hipErrorInvalidValue;
    // every block of every tile step, the ones past the row's end as zeros
    gemm32_quant_kernel<<<dim3((unsigned)((nb + 3) / 4 * 4), (unsigned)(Tp / 32)), 64, 0, s>>>(x, ldx, nb, T, Tp, rec,
                                                                                              cnt, ncnt);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// The GEMM kernel
// ---------------------------------------------------------------------------------------------
// one lane's weights of one tile step: slices 4 h .. 4 h + 3 of its row (dword bb = block bb's 4
// values) and its row's four fp16 d
typedef int v2i __attribute__((ext_vector_type(2)));
struct GW32 {
    v4i s0, s1, s2, s3;  // native vectors: gathering dword bb of each stays in registers
    v2i d;
};
__device__ __forceinline__ v4i bld16v(BufRes r, uint32_t off) {
    return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));  // weights
}
__device__ __forceinline__ v2i bld8v(BufRes r, uint32_t off) {
    return __builtin_bit_cast(v2i, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0));  // weights
}

// one step's activation records held by a thread between their load and their LDS write
struct ARec32 {
    uint4 v0, v1, v2, v3, v4, v5;
};

template <int NT, int KH, int TPW, bool DUMP>
__global__ __launch_bounds__(64 * TPW * KH) __attribute__((amdgpu_waves_per_eu(2, 2))) void q80_gemm_kernel(Gemm32Args a) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int Tp = 32 * NT, REC = gemm32_rec_bytes(Tp), NTH = 64 * TPW * KH;
    constexpr int R = (KH * REC + 16 * NTH - 1) / (16 * NTH), SB = R * 16 * NTH;
    static_assert(R >= 1 && R <= 6, "one step's records take 1..6 rounds per thread");
    const int tid = threadIdx.x, l = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tw = wave % TPW, kh = wave / TPW;
    const int n = l & 31, h = l >> 5, r8 = n & 7;
    // K split ksi of a.ks (grid.y): tile steps [s_lo, s_lo + nsk) of the row's ns
    const int ns = a.nsteps, ksi = blockIdx.y, nss = (ns + a.ks - 1) / a.ks;
    const int s_lo = ksi * nss, nsk = min(ns - s_lo, nss);
    const int nws = (nsk + KH - 1) / KH;  // workgroup steps
    const int64_t grp = (int64_t)blockIdx.x * TPW + tw;
    const bool live = grp < a.groups;
    const int64_t gc = live ? grp : a.groups - 1;
    const int64_t mi = gc / a.gpm32, gi = gc - mi * a.gpm32;
    const int64_t t8 = 4 * gi + (n >> 3);                      // the lane's 8-row tile in its matrix
    const int nvalid = (int)min<int64_t>(4, a.tpm - 4 * gi);  // tiles of the group inside the matrix
    const int64_t rows = a.rows, row = t8 * 8 + r8;
    const bool store = live && t8 < a.tpm && row < rows;
    const int64_t orow = mi * rows + row;
    const uint32_t woff = (uint32_t)((n >> 3) * Q80_TILE), qoff = woff + 64 + 16 * (8 * r8 + 4 * h), doff = woff + 8 * r8;

    // the step's records: a linear copy of KH tile-step records from tile step s_lo + KH j (the
    // quantizer's buffer holds KH records of slack past the last)
    auto aload = [&](int j, ARec32 &ar) __attribute__((always_inline)) {
        const BufRes src = buf_res(a.act + (size_t)(s_lo + KH * min(j, nws - 1)) * REC, KH * REC);
        auto ld = [&](int k) __attribute__((always_inline)) { return bld16(src, 16 * (k * NTH + tid)); };
        ar.v0 = ld(0);
        if (R > 1) ar.v1 = ld(1);
        if (R > 2) ar.v2 = ld(2);
        if (R > 3) ar.v3 = ld(3);
        if (R > 4) ar.v4 = ld(4);
        if (R > 5) ar.v5 = ld(5);
    };
    auto astore = [&](uint8_t *st, const ARec32 &ar) __attribute__((always_inline)) {
        uint4 *dst = (uint4 *)st + tid;
        dst[0] = ar.v0;
        if (R > 1) dst[NTH] = ar.v1;
        if (R > 2) dst[2 * NTH] = ar.v2;
        if (R > 3) dst[3 * NTH] = ar.v3;
        if (R > 4) dst[4 * NTH] = ar.v4;
        if (R > 5) dst[5 * NTH] = ar.v5;
    };
    // the group's weights of tile step KH j + kh: its (up to) 4 tiles are contiguous; reads past
    // the valid tiles (a matrix's last group) return zeros
    auto wload = [&](int j, GW32 &w) __attribute__((always_inline)) {
        const int s = s_lo + min(KH * j + kh, nsk - 1);
        const BufRes r = buf_res(a.W + ((size_t)(mi * ns + s) * a.tpm + 4 * gi) * Q80_TILE, nvalid * Q80_TILE);
        w.s0 = bld16v(r, qoff);
        w.s1 = bld16v(r, qoff + 16);
        w.s2 = bld16v(r, qoff + 32);
        w.s3 = bld16v(r, qoff + 48);
        w.d = bld8v(r, doff);
    };

    v16f acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = v16f{};

    // tile step s of this K-part from stage st with weights w
    auto block = [&](const GW32 &w, const uint8_t *st, int s, auto &&issue) __attribute__((always_inline)) {
        const uint8_t *rec = st + kh * REC;
        const float *xds = (const float *)(rec + 128 * Tp);
#pragma unroll
        for (int bb = 0; bb < 4; ++bb) {
            const v4i bv = {w.s0[bb], w.s1[bb], w.s2[bb], w.s3[bb]};
            const float dw = fp16_bits_to_f32(((uint32_t)w.d[bb >> 1] >> (16 * (bb & 1))) & 0xFFFF);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const uint4 au = *(const uint4 *)(rec + ((size_t)(bb * NT + t) * 64 + l) * 16);
                const v4i av = {(int)au.x, (int)au.y, (int)au.z, (int)au.w};
                const v16i isum = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, v16i{}, 0, 0, 0);
                // output i: token 32 t + 8 (i / 4) + 4 h + i % 4 of row n
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const v4f xd = *(const v4f *)(xds + bb * Tp + 32 * t + 8 * q + 4 * h);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int i = 4 * q + e;
                        acc[t][i] = __builtin_fmaf(dw * xd[e], (float)isum[i], acc[t][i]);
                        if (DUMP) {
                            const int tok = 32 * t + 8 * q + 4 * h + e, blk = 4 * s + bb;
                            if (store && tok < a.T && blk < a.nb) a.dump_s[((size_t)tok * a.nrows + orow) * a.nb + blk] = isum[i];
                        }
                    }
                }
            }
            issue(bb);
        }
    };

    // prologue: step 0's records in LDS, the weights of steps 0..2 in flight
    GW32 w0, w1, w2, w3;
    ARec32 rr;
    uint8_t *st0 = smem, *st1 = smem + SB;
    aload(0, rr);
    __builtin_amdgcn_sched_barrier(0);
    wload(0, w0);
    wload(1, w1);
    wload(2, w2);
    __builtin_amdgcn_sched_barrier(0);
    astore(st0, rr);
    __syncthreads();
    // workgroup step j: this K-part's tile step KH j + kh from stage j % 2; the next step's
    // records load after its first block and the weights of step j + 3 after its third (into the
    // ring slot step j - 1 used); then the records go to the other stage and the barrier. Steps in
    // which every K-part has a tile step run without branches (exact load counters); the last
    // may test.
    auto step = [&](auto full, int j, GW32 &wc, GW32 &wn3, const uint8_t *stc, uint8_t *stn) __attribute__((always_inline)) {
        const int s = s_lo + KH * j + kh;
        auto issue = [&](int bb) __attribute__((always_inline)) {
            __builtin_amdgcn_sched_barrier(0);
            if (bb == 0) aload(j + 1, rr);
            if (bb == 2) wload(j + 3, wn3);
            __builtin_amdgcn_sched_barrier(0);
        };
        if (decltype(full)::value || s < s_lo + nsk) {  // uniform per wavefront
            block(wc, stc, s, issue);
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
    const int nfull = nsk / KH;  // workgroup steps in which every K-part has a tile step
    int j = 0;
    for (; j + 4 <= nfull; j += 4) {
        step(Full(), j, w0, w3, st0, st1);
        step(Full(), j + 1, w1, w0, st1, st0);
        step(Full(), j + 2, w2, w1, st0, st1);
        step(Full(), j + 3, w3, w2, st1, st0);
    }
    if (j < nws) step(Edge(), j, w0, w3, st0, st1);
    if (j + 1 < nws) step(Edge(), j + 1, w1, w0, st1, st0);
    if (j + 2 < nws) step(Edge(), j + 2, w2, w1, st0, st1);
    if (j + 3 < nws) step(Edge(), j + 3, w3, w2, st1, st0);
    __syncthreads();  // every wavefront is past its reads of the stages (the reduction reuses them)
    if (KH > 1) {  // K-parts 1.. -> LDS; K-part 0 adds them in order and stores
        float *red = (float *)smem + (size_t)tw * (KH - 1) * 64 * 16 * NT;
        if (kh > 0) {
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    *(v4f *)(red + ((size_t)((kh - 1) * NT + t) * 4 * 64 + q * 64 + l) * 4) =
                        v4f{acc[t][4 * q], acc[t][4 * q + 1], acc[t][4 * q + 2], acc[t][4 * q + 3]};
        }
        __syncthreads();
        if (kh == 0) {
#pragma unroll
            for (int k = 1; k < KH; ++k)
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const v4f o = *(const v4f *)(red + ((size_t)((k - 1) * NT + t) * 4 * 64 + q * 64 + l) * 4);
#pragma unroll
                        for (int e = 0; e < 4; ++e) acc[t][4 * q + e] += o[e];
                    }
        }
    }
    if (a.ks > 1) {  // the K split's partials; the flag sits past the reduction area
        gemm_split_finish<16 * NT>([&](int e) { return 32 * (e >> 4) + 8 * ((e & 15) >> 2) + 4 * h + (e & 3); },
                                   [&](int e) { return acc[e >> 4][e & 15]; }, kh == 0, store, tid, tw, TPW, orow, a.ks,
                                   ksi, a.T, a.ldy, a.part, a.cnt, a.Y, (int *)smem + TPW * (KH - 1) * 64 * 16 * NT);
        return;
    }
    if (kh == 0 && store) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int tok = 32 * t + 8 * (i >> 2) + 4 * h + (i & 3);
                if (tok < a.T) a.Y[(size_t)tok * a.ldy + orow] = acc[t][i];
            }
    }
}

constexpr int GEMM32_TPW = 2;  // 32-row groups per workgroup
static int gemm32_kh(int nsteps) { return nsteps >= 4 ? 4 : nsteps >= 2 ? 2 : 1; }  // K-parts
template <int NT, int KH>
static size_t gemm32_lds() {
    const int nth = 64 * GEMM32_TPW * KH, r = (KH * gemm32_rec_bytes(32 * NT) + 16 * nth - 1) / (16 * nth);
    const size_t stages = (size_t)2 * r * 16 * nth, red = (size_t)GEMM32_TPW * (KH - 1) * 64 * 16 * NT * 4;
    return std::max(stages, red + 4);  // + the K split's flag past the reduction area
}
int gemm32_workgroups(int64_t groups) { return (int)((groups + GEMM32_TPW - 1) / GEMM32_TPW); }

size_t gemm32_act_bytes(int nb, int Tp) {
    const int ns = (nb + 3) / 4;
    return (size_t)(ns + gemm32_kh(ns)) * gemm32_rec_bytes(Tp);  // KH records of slack
}

template <int NT, int KH>
static void gemm32_launch(const Gemm32Args &a, hipStream_t s) {
    const dim3 grid((unsigned)((a.groups + GEMM32_TPW - 1) / GEMM32_TPW), (unsigned)a.ks);
    const size_t lds = gemm32_lds<NT, KH>();
    if (a.dump_s) q80_gemm_kernel<NT, KH, GEMM32_TPW, true><<<grid, 64 * GEMM32_TPW * KH, lds, s>>>(a);
    else q80_gemm_kernel<NT, KH, GEMM32_TPW, false><<<grid, 64 * GEMM32_TPW * KH, lds, s>>>(a);
}
template <int NT>
static void gemm32_launch_kh(const Gemm32Args &a, hipStream_t s) {
    switch (gemm32_kh(a.nsteps)) {
    case 4: gemm32_launch<NT, 4>(a, s); break;
    case 2: gemm32_launch<NT, 2>(a, s); break;
    default: gemm32_launch<NT, 1>(a, s); break;
    }
}

hipError_t launch_q80_gemm(const Gemm32Args &a, hipStream_t s) {
    if (a.T < 1 || a.T > a.Tp || (a.Tp != 32 && a.Tp != 64) || a.Tp - a.T >= 32 || a.nb < 1 ||
        a.nsteps != (a.nb + 3) / 4 || a.groups < 1 || a.gpm32 != (a.tpm + 3) / 4)
        return hipErrorInvalidValue;
    if (a.ks < 1 || a.ks > 4 || (a.ks > 1 && (!a.part || !a.cnt)) || (a.nsteps + a.ks - 1) / a.ks * (a.ks - 1) >= a.nsteps)
        return hipErrorInvalidValue;  // every split has a tile step
    if (a.Tp == 32) gemm32_launch_kh<1>(a, s);
    else gemm32_launch_kh<2>(a, s);
    return hipGetLastError();
}

}  // namespace fgh
