// fgh_matvec.hip - the decode matvec for Q6_K and the 32-value types (Q8_0, Q5_0, Q4_0, Q4_1, Q5_1,
// IQ4_NL) on gfx950 (Q4_K and Q5_K have their own kernel in fgh_q4k.hip, on the same plan, and so
// do Q2_K, Q3_K and IQ4_XS in fgh_kq.hip, and F32, F16 and BF16 in fgh_float.hip).
//
// Tiles (fgh_internal.h) are 8 rows of one step: one block (Q6_K, 1680 B) or four blocks (Q8_0,
// 1088 B; Q5_0 704 B, Q4_0 / IQ4_NL 576 B, Q4_1 640 B, Q5_1 768 B). They lie step-major: step s of row tile t of matrix m at
// ((m * steps + s) * tpm + t) * tile bytes (tpm = row tiles per matrix), so the wavefronts of a
// launch, all at about the same step, read one contiguous stretch of HBM at a time.
//
// A wavefront owns one row tile; lane L = 8 r + i holds slice i of row r, which is exactly what
// the reference's AVX2 fp32 accumulator lane i of that row sums. Every workgroup quantizes x into
// LDS (bit-exact with quantize_q8k / quantize_q8, fastgguf.c:746-793) while the first steps of its
// wavefronts' rings of R steps are in flight; activations are LDS broadcasts. Per step a lane
// forms its exact integer lane partial (v_dot4_i32_i8, 16-bit scale products by v_dot2_i32_i16)
// and advances its fp32 chain in registers in block order:
//   Q8_0, dot_q8_0_q8 (fastgguf.c:891-902):   acc_i = fma(d * xd, s_i, acc_i), out = hsum8(acc)
//   Q5_0, Q4_0, IQ4_NL (944-959, 833-857, 1547-1562): the same, s_i over q5 - 16, q - 8, kvalues[q]
//   Q4_1, Q5_1 (1020-1031, 973-989): the same over q, plus one min chain per row,
//        macc = fma(m * xd, s16_0 + s16_1, macc), out = hsum8(acc) + macc
//   Q4_0 repacked, dot_q40x8 (2424-2467): acc = fma(d * xd, isum, acc) per row over whole blocks
//   Q6_K, dot_q6_K_q8k (fastgguf.c:1232-1264): acc_i = fma(d * yd, lane_i, acc_i),
//        cacc_p = fma(32 d yd, corr_p, cacc_p) in lanes i = p < 4, out = hsum8(acc) - hsum4(cacc)
// so the outputs are bit-identical to the reference's row kernels. Short matrices split the steps
// of a tile over S wavefronts: wavefront 0 runs its chains as it streams, the others park their
// fp32 step records {d * yd, lane partials} in LDS, and wavefront 0 continues the chains over them.
// Up to 4 tensors of one type and width share one launch (matvec_multi, fastgguf.c:2552).
#include <type_traits>

#include "fgh_internal.h"

namespace fgh {

// ---- LDS activations --------------------------------------------------------------------------
// Q8_K (Q6_K): qs [nb][256] lane-permuted (position 32 i + 4 c holds element 32 c + 4 i, so lane
//   i's 32 bytes are contiguous), d [nb] fp32, bs [nb][16] int16.
// Q8 (Q8_0 / Q5_0): per group of 4 blocks g, qs at 128 g: dword i of block 4 g + k at 128 g + 16 i + 4 k
//   (a lane's 4 blocks in one 16-byte read); d [4 * groups] fp32.
__host__ __device__ constexpr size_t align16(size_t v) { return (v + 15) & ~(size_t)15; }
__host__ __device__ constexpr int mv_steps(int type, int nb) { return q8_kind(type) ? (nb + 3) / 4 : nb; }
__host__ __device__ constexpr size_t act_off_d(int type, int nb) {
    return q8_kind(type) ? (size_t)128 * mv_steps(type, nb) : (size_t)256 * nb;
}
__host__ __device__ constexpr size_t act_off_s(int type, int nb) {
    return align16(act_off_d(type, nb) + 4 * (size_t)(q8_kind(type) ? 4 * mv_steps(type, nb) : nb));
}
// Q8: after d, for Q4_1 / Q5_1 only, the sum of each block's 32 quants (s16[0] + s16[1], the min
// term) as fp32, exact [4 * steps]; Q8_K: bs [nb][16] int16
__host__ __device__ constexpr size_t act_lds_bytes(int type, int nb) {
    return q8_kind(type) ? act_off_s(type, nb) + (q32_min(type) ? (size_t)16 * mv_steps(type, nb) : 0)
                         : align16(act_off_s(type, nb) + (size_t)nb * 32);
}
// records of one step of one tile (block split): lane partials, then fp32 d * yd per row (and
// m * yd per row for Q4_1 / Q5_1)
// Q4_0 / Q4_1 / Q5_0 / Q5_1 keep the lane partials as int16 (exact: a lane's 4 products are at most
// 4 * 31 * 127, repacked Q4_0's whole-block sum at most 32 * 8 * 127 = 32512), half the bytes, so
// a long row splits further within the LDS; Q8_0 and IQ4_NL need 17 bits and keep fp32
__host__ __device__ constexpr bool rec_i16(int type) { return q8_kind(type) && type != T_Q8_0 && type != T_IQ4_NL; }
__host__ __device__ constexpr size_t rec_fd_off(int type) { return q8_kind(type) ? (rec_i16(type) ? 512 : 1024) : 512; }
__host__ __device__ constexpr size_t rec_bytes(int type) {
    return q8_kind(type) ? rec_fd_off(type) + 8 * 16 + (q32_min(type) ? 8 * 16 : 0) : 64 * 8 + 8 * 4;
}
__host__ __device__ constexpr int mv_tile_bytes(int type) {
    return type == T_Q6_K ? Q6K_TILE : type == T_Q8_0 ? Q80_TILE : q32_layout(type).tile;
}

__device__ __forceinline__ float ror_f32(float v, int n) {  // DPP row_ror:n within 16 lanes
    const int iv = __builtin_bit_cast(int, v);
    int r;
    switch (n) {
    case 8: r = __builtin_amdgcn_update_dpp(0, iv, 0x128, 0xF, 0xF, false); break;
    case 4: r = __builtin_amdgcn_update_dpp(0, iv, 0x124, 0xF, 0xF, false); break;
    case 2: r = __builtin_amdgcn_update_dpp(0, iv, 0x122, 0xF, 0xF, false); break;
    default: r = __builtin_amdgcn_update_dpp(0, iv, 0x121, 0xF, 0xF, false); break;
    }
    return __builtin_bit_cast(float, r);
}
__device__ __forceinline__ float xor1_f32(float v) { return __builtin_bit_cast(float, dpp_xor1(__builtin_bit_cast(int, v))); }
__device__ __forceinline__ float xor2_f32(float v) { return __builtin_bit_cast(float, dpp_xor2(__builtin_bit_cast(int, v))); }

// Quantization in rounds over all 64 * WPG threads, 16 values per thread: Q8_K 16 threads per
// 256-value block (4 WPG blocks a round), Q8 2 threads per 32-value block (32 WPG a round).
// xq_load issues a round's loads (the first one before the weight loads, so that waiting for x
// never waits for weights); xq_finish quantizes and stores the first round, then the rest.
struct XVals {
    float4 v[4];
};
template <int TYPE, int WPG>
struct XQ {
    static constexpr int TPB = q8_kind(TYPE) ? 2 : 16;            // threads per block
    static constexpr int BPR = 64 * WPG / TPB;                     // blocks per round
    static constexpr int BV = q8_kind(TYPE) ? 32 : 256;            // values per block
};
template <int TYPE, int WPG>
__device__ __forceinline__ void xq_load(const float *__restrict__ x, int nb, int rb, XVals &xv) {
    using Q = XQ<TYPE, WPG>;
    const int b = rb + (int)threadIdx.x / Q::TPB, tl = (int)threadIdx.x % Q::TPB;
    const float *p = x + (size_t)(b < nb ? b : 0) * Q::BV + 16 * tl;  // past the end: block 0, unused
#pragma unroll
    for (int u = 0; u < 4; ++u) xv.v[u] = *(const float4 *)(p + 4 * u);
}
template <int TYPE, int WPG>
__device__ __forceinline__ void xq_store(int nb, int rb, const XVals &xv, uint8_t *act) {
    using Q = XQ<TYPE, WPG>;
    const int b = rb + (int)threadIdx.x / Q::TPB, tl = (int)threadIdx.x % Q::TPB;
    float v[16];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        v[4 * u] = xv.v[u].x; v[4 * u + 1] = xv.v[u].y; v[4 * u + 2] = xv.v[u].z; v[4 * u + 3] = xv.v[u].w;
    }
    float amax = 0.0f;
#pragma unroll
    for (int u = 0; u < 16; ++u) amax = fmaxf(amax, fabsf(v[u]));
    if (q8_kind(TYPE)) {
        amax = fmaxf(amax, xor1_f32(amax));
    } else {  // the block's 16 threads are one DPP row
        amax = fmaxf(amax, ror_f32(amax, 8));
        amax = fmaxf(amax, ror_f32(amax, 4));
        amax = fmaxf(amax, ror_f32(amax, 2));
        amax = fmaxf(amax, ror_f32(amax, 1));
    }
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
    if (q32_min(TYPE)) s += dpp_xor1(s);  // the block's two threads: its 32 quants
    if (b >= nb) return;
    if (q8_kind(TYPE)) {  // dwords 4 tl .. 4 tl + 3 of block b
        uint8_t *g = act + (size_t)128 * (b >> 2) + 4 * (b & 3);
#pragma unroll
        for (int u = 0; u < 4; ++u) *(uint32_t *)(g + 16 * (4 * tl + u)) = w[u];
        if (tl == 0) {
            ((float *)(act + act_off_d(TYPE, nb)))[b] = d;
            if (q32_min(TYPE)) ((float *)(act + act_off_s(TYPE, nb)))[b] = (float)s;  // exact: |s| < 2^13
        }
    } else {  // value 16 tl + 4 u = 32 c + 4 i (c = tl / 2, i = 4 (tl % 2) + u) -> position 32 i + 4 c
        const int c = tl >> 1;
#pragma unroll
        for (int u = 0; u < 4; ++u) *(uint32_t *)(act + (size_t)b * 256 + 32 * (4 * (tl & 1) + u) + 4 * c) = w[u];
        ((int16_t *)(act + act_off_s(TYPE, nb)))[16 * b + tl] = (int16_t)s;
        if (tl == 0) ((float *)(act + act_off_d(TYPE, nb)))[b] = d;
    }
}
// the rounds after the first (xv: the first round, loaded before the weights)
template <int TYPE, int WPG>
__device__ __forceinline__ void xq_finish(const float *__restrict__ x, int nb, XVals &xv, uint8_t *act) {
    using Q = XQ<TYPE, WPG>;
    xq_store<TYPE, WPG>(nb, 0, xv, act);
    for (int rb = Q::BPR; rb < nb; rb += Q::BPR) {
        xq_load<TYPE, WPG>(x, nb, rb, xv);
        xq_store<TYPE, WPG>(nb, rb, xv, act);
    }
}

// ---- one step of one lane -----------------------------------------------------------------------
// Q8_0: q = the lane's dword of each of the 4 blocks, d = its row's 4 fp16 scales.
// Q5_0: n = the lane's nibble bytes of the 4 blocks, h = its 16 fifth bits, d as Q8_0.
// Q6_K: q = 4 ql dwords (2 h + s), h = 2 qh dwords, sc = its row's 16 int8 scales, d = fp16 d.
// nibble types (Q4_0, Q4_1, Q5_0, Q5_1, IQ4_NL): n = the lane's nibble bytes of the 4 blocks,
// d (and m) = its row's 4 fp16 scales (and mins), h = its 16 fifth bits
template <int TYPE>
struct StepW {
    uint2 n, d, m;
    uint32_t h;
};
template <>
struct StepW<T_Q8_0> {
    uint4 q;
    uint2 d;
};
template <>
struct StepW<T_Q6_K> {
    uint4 q, sc;
    uint2 h;
    uint32_t d;
};
// T: the tile (wavefront-uniform); live = false: zeros without a memory access (a refill past the
// wavefront's last step: re-reading the last step's bytes missed the caches under nontemporal
// loads, 2 % more HBM traffic)
__device__ __forceinline__ void step_load(const uint8_t *T, uint32_t lane, StepW<T_Q8_0> &w, bool live = true) {
    const BufRes r = buf_res(T, live ? Q80_TILE : 0);
    w.q = bld16<WNT>(r, 64 + 16 * lane);
    w.d = bld8<WNT>(r, 8 * (lane >> 3));
}
template <int TYPE>
__device__ __forceinline__ void step_load(const uint8_t *T, uint32_t lane, StepW<TYPE> &w, bool live = true) {
    constexpr Q32Layout L = q32_layout(TYPE);
    const BufRes r = buf_res(T, live ? L.tile : 0);
    w.n = bld8<WNT>(r, L.n + 8 * lane);
    if (L.m >= 0) {  // the row's d and m in one record
        const uint4 dm = bld16<WNT>(r, L.ds * (lane >> 3));
        w.d = make_uint2(dm.x, dm.y);
        w.m = make_uint2(dm.z, dm.w);
    } else {
        w.d = bld8<WNT>(r, L.ds * (lane >> 3));
    }
    if (L.h >= 0) w.h = bld2<WNT>(r, L.h + 2 * lane);
}
__device__ __forceinline__ void step_load(const uint8_t *T, uint32_t lane, StepW<T_Q6_K> &w, bool live = true) {
    const BufRes r = buf_res(T, live ? Q6K_TILE : 0);
    w.q = bld16<WNT>(r, 144 + 16 * lane);
    w.h = bld8<WNT>(r, 1168 + 8 * lane);
    w.sc = bld16<WNT>(r, 16 * (lane >> 3));
    w.d = bld2<WNT>(r, 128 + 2 * (lane >> 3));
}

// the lane's partial s_i of each of the step's 4 blocks (y: the lane's activation dword of each)
__device__ __forceinline__ void q32_sums(const StepW<T_Q8_0> &w, uint4 y, int sd[4]) {
    sd[0] = dot4((int)w.q.x, (int)y.x, 0);
    sd[1] = dot4((int)w.q.y, (int)y.y, 0);
    sd[2] = dot4((int)w.q.z, (int)y.z, 0);
    sd[3] = dot4((int)w.q.w, (int)y.w, 0);
}
// Nibble types: the value of element 4i + t of block k is nibble byte t of n (blocks 2w / 2w + 1
// in the low / high nibbles of dword w), with (Q5_0 / Q5_1) bit 4 from the fifth bits spread to
// one nibble per byte. The offsets of Q4_0 (-8) and Q5_0 (-16), the reference's bx = q - 8 and
// q5 - 16, enter as a second dot with the offset in every byte.
template <int TYPE>
__device__ __forceinline__ void q32_sums(const StepW<TYPE> &w, uint4 y, int sd[4]) {
    constexpr bool Q5 = TYPE == T_Q5_0 || TYPE == T_Q5_1;
    const uint32_t e = Q5 ? (w.h & 0x0F0Fu) | ((w.h << 12) & 0x0F0F0000u) : 0u;  // byte t: bit k = block k
    const uint32_t Y[4] = {y.x, y.y, y.z, y.w};
    const uint32_t N[2] = {w.n.x, w.n.y};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        uint32_t q = ((k & 1) ? N[k >> 1] >> 4 : N[k >> 1]) & 0x0F0F0F0Fu;
        if (Q5) q |= (e << (4 - k)) & 0x10101010u;
        if (TYPE == T_IQ4_NL) q = iq4nl_values(q);
        const int off = TYPE == T_Q5_0 ? dot4((int)0xF0F0F0F0u, (int)Y[k], 0)
                      : TYPE == T_Q4_0 ? dot4((int)0xF8F8F8F8u, (int)Y[k], 0)
                                       : 0;
        sd[k] = dot4((int)q, (int)Y[k], off);
    }
}

// int16 pair (sext byte 1, sext byte 3) of x (v_perm_b32 selectors 8, 9: sign of bytes 1, 3)
__device__ __forceinline__ uint32_t sx_b13(uint32_t x) { return __builtin_amdgcn_perm(x, x, 0x09030801u); }
// int16 pair (sext byte 0, sext byte 1) of x (selector 10: the sign of byte 1 of x << 8)
__device__ __forceinline__ uint32_t sx_b01(uint32_t x) { return __builtin_amdgcn_perm(x << 8, x, 0x08010A00u); }

// Q6_K lane partial of one block (lane i): sum over (h, k) of sc[8h + 2k + (i >= 4)] times the dot
// of its 4 values (0..63, offset not removed) of chunk (h, k) with the activations; and the
// correction partial of p = i & 3, (sc_2p bs_2p + sc_2p+1 bs_2p+1) + (sc_2p+8 bs_2p+8 +
// sc_2p+9 bs_2p+9) (q6_corr_vec, fastgguf.c:1085-1088). Each 4-value dot is at most
// 4 * 63 * 127 < 2^15 in magnitude: int16 pairs for v_dot2_i32_i16.
__device__ __forceinline__ void q6_ints(const StepW<T_Q6_K> &w, const uint8_t *act, int nb, int b, int i, int &sum,
                                        int &corr) {
    const uint8_t *yb = act + (size_t)b * 256 + 32 * i;
    const uint4 y0 = *(const uint4 *)yb, y1 = *(const uint4 *)(yb + 16);
    const uint32_t yv[8] = {y0.x, y0.y, y0.z, y0.w, y1.x, y1.y, y1.z, y1.w};
    const uint32_t A[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
    const uint32_t H[2] = {w.h.x, w.h.y};
    const uint32_t S[4] = {w.sc.x, w.sc.y, w.sc.z, w.sc.w};
    const uint32_t M4 = 0x0F0F0F0Fu, M2 = 0x30303030u;
    const int shl = i >= 4 ? 0 : 8;  // the lane's scales: bytes 1, 3 of (S_k << shl)
    int s = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t A0 = A[2 * h], A1 = A[2 * h + 1], Hh = H[h];
        const uint32_t q0 = (A0 & M4) | ((Hh << 4) & M2), q1 = (A1 & M4) | ((Hh << 2) & M2);
        const uint32_t q2 = ((A0 >> 4) & M4) | (Hh & M2), q3 = ((A1 >> 4) & M4) | ((Hh >> 2) & M2);
        const int d0 = dot4((int)q0, (int)yv[4 * h], 0), d1 = dot4((int)q1, (int)yv[4 * h + 1], 0);
        const int d2 = dot4((int)q2, (int)yv[4 * h + 2], 0), d3 = dot4((int)q3, (int)yv[4 * h + 3], 0);
        s = dot2_i16(sx_b13(S[2 * h] << shl), pack_i16(d0, d1), s);
        s = dot2_i16(sx_b13(S[2 * h + 1] << shl), pack_i16(d2, d3), s);
    }
    sum = s;
    const int p = i & 3;
    const int cs = 16 * (p & 1);
    const uint32_t lo = ((p >> 1) ? S[1] : S[0]) >> cs, hi = ((p >> 1) ? S[3] : S[2]) >> cs;
    const uint32_t *bq = (const uint32_t *)((const int16_t *)(act + act_off_s(T_Q6_K, nb)) + 16 * b + 2 * p);
    corr = dot2_i16(sx_b01(lo), bq[0], 0) + dot2_i16(sx_b01(hi), bq[4], 0);
}

// the tensor of global tile g in a multi-tensor launch
__device__ __forceinline__ int mv_tensor_of(const MvArgs &a, int64_t g) {
    int ti = 0;
#pragma unroll
    for (int k = 1; k < 4; ++k)
        if (k < a.nt && g >= a.t[k].gfirst) ti = k;
    return ti;
}

// Workgroup = TPW tiles x S wavefronts per tile (wavefront ks of a tile takes its ks-th run of
// ceil(steps / S) steps); grid = (tiles over all tensors / TPW, tokens).
// ORDER 1 (Q4_0 only): the repacked order of dot_q40x8 (fastgguf.c:2424-2467), one chain per row
// over whole-block integers, acc = fma(d * yd, isum, acc), out = acc.
template <int TYPE, int R, int TPW, int S, bool DUMP, int ORDER = 0>
__global__ __launch_bounds__(64 * TPW * S) void mv_kernel(MvArgs a) {
    static_assert(ORDER == 0 || TYPE == T_Q4_0, "only Q4_0 has a repacked order here");
    constexpr int WPG = TPW * S;
    constexpr int TB = mv_tile_bytes(TYPE);
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ts = wave / S, ks = wave - ts * S;
    const int r = lane >> 3, i = lane & 7;
    const int nb = a.nb, nst = a.ntile;
    const int tok = blockIdx.y;
    const int64_t tile = (int64_t)blockIdx.x * TPW + ts;
    const bool live = tile < a.groups;
    const int64_t tc = live ? tile : a.groups - 1;
    const int ti = mv_tensor_of(a, tc);
    const uint32_t lt = (uint32_t)(tc - a.t[ti].gfirst), tpm = (uint32_t)a.t[ti].gpm;
    const uint32_t mi = (a.sel ? (uint32_t)a.sel[tok] : 0u) + lt / tpm, tt = lt % tpm;
    const int nsw = (nst + S - 1) / S, s0 = ks * nsw;
    const int nsl = max(0, min(nst, s0 + nsw) - s0), sl = max(nsl - 1, 0);
    const size_t sstride = (size_t)tpm * TB;
    const uint8_t *T0 = a.t[ti].W + (((size_t)mi * nst + min(s0, nst - 1)) * tpm + tt) * TB;

    const float *x = a.x + (size_t)(tok / a.xdiv) * a.ldx;
    XVals xv;
    xq_load<TYPE, WPG>(x, nb, 0, xv);
    StepW<TYPE> ring[R];
#pragma unroll
    for (int k = 0; k < R; ++k) step_load(T0 + (size_t)min(k, sl) * sstride, (uint32_t)lane, ring[k]);
    uint8_t *act = smem;
    xq_finish<TYPE, WPG>(x, nb, xv, act);
    __syncthreads();

    const float *ad = (const float *)(act + act_off_d(TYPE, nb));
    const int64_t rows = a.t[ti].rows, mrow = (int64_t)tt * 8;
    const int64_t obase = (int64_t)(lt / tpm) * rows;
    const bool row_ok = live && mrow + r < rows;
    // records of the wavefronts ks >= 1 (step s of the tile at s - nsw): lane partials, then fd
    uint8_t *rec = smem + act_lds_bytes(TYPE, nb) + (size_t)ts * (nst - nsw) * rec_bytes(TYPE);
    const float *abs = (const float *)(act + act_off_s(TYPE, nb));  // Q4_1 / Q5_1: block sums, as fp32
    float acc = 0.0f, cacc = 0.0f;  // cacc: Q6_K's correction chain, or Q4_1 / Q5_1's min chain

    // CHECK: the step may be the tile's last, with fewer than 4 blocks (the checks are uniform)
    auto step = [&](const StepW<TYPE> &w, int st, auto check) {
        constexpr bool CHECK = decltype(check)::value;
        const bool chain = S == 1 || ks == 0;
        uint8_t *rs = rec + (size_t)(st - nsw) * rec_bytes(TYPE);
        if constexpr (q8_kind(TYPE)) {
            const uint4 y = *(const uint4 *)(act + (size_t)128 * st + 16 * i);
            const float4 yd = *(const float4 *)(ad + 4 * st);
            int sd[4];
            q32_sums(w, y, sd);
            const float fd[4] = {fp16_bits_to_f32(w.d.x & 0xFFFF) * yd.x, fp16_bits_to_f32(w.d.x >> 16) * yd.y,
                                 fp16_bits_to_f32(w.d.y & 0xFFFF) * yd.z, fp16_bits_to_f32(w.d.y >> 16) * yd.w};
            float fm[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // Q4_1 / Q5_1: FP16(m) * xd of the min chain
            if constexpr (q32_min(TYPE)) {
                fm[0] = fp16_bits_to_f32(w.m.x & 0xFFFF) * yd.x;
                fm[1] = fp16_bits_to_f32(w.m.x >> 16) * yd.y;
                fm[2] = fp16_bits_to_f32(w.m.y & 0xFFFF) * yd.z;
                fm[3] = fp16_bits_to_f32(w.m.y >> 16) * yd.w;
            }
            if (ORDER == 1) {  // whole-block integers in every lane of the row
#pragma unroll
                for (int k = 0; k < 4; ++k) sd[k] = sum8_i32(sd[k]);
            }
            const int nbs = nb - 4 * st;  // blocks of this step (the last one may have fewer)
            if (chain) {
                float bsv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                if constexpr (q32_min(TYPE)) {
                    const float4 bs = *(const float4 *)(abs + 4 * st);
                    bsv[0] = bs.x; bsv[1] = bs.y; bsv[2] = bs.z; bsv[3] = bs.w;
                }
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if (!CHECK || nbs >= 4 || k < nbs) {  // uniform
                        acc = __builtin_fmaf(fd[k], (float)sd[k], acc);
                        if (q32_min(TYPE)) cacc = __builtin_fmaf(fm[k], bsv[k], cacc);
                    }
            } else {
                if (rec_i16(TYPE))
                    ((uint2 *)rs)[lane] = make_uint2(pack_i16(sd[0], sd[1]), pack_i16(sd[2], sd[3]));
                else
                    ((float4 *)rs)[lane] = make_float4((float)sd[0], (float)sd[1], (float)sd[2], (float)sd[3]);
                constexpr size_t FD = rec_fd_off(TYPE);
                if (i == 0) ((float4 *)(rs + FD))[r] = make_float4(fd[0], fd[1], fd[2], fd[3]);
                if (q32_min(TYPE) && i == 0) ((float4 *)(rs + FD + 128))[r] = make_float4(fm[0], fm[1], fm[2], fm[3]);
            }
            if (DUMP) {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int tsum = ORDER == 1 ? sd[k] : sum8_i32(sd[k]);
                    if (row_ok && i == 0 && k < nbs) {
                        const size_t di = (size_t)(obase + mrow + r) * nb + 4 * st + k;
                        a.dump_s[di] = tsum;
                        a.dump_m[di] = 0;
                    }
                }
            }
        } else {
            int sum, corr;
            q6_ints(w, act, nb, st, i, sum, corr);
            const float fd = fp16_bits_to_f32(w.d) * ad[st];
            if (chain) {
                acc = __builtin_fmaf(fd, (float)sum, acc);
                cacc = __builtin_fmaf(fd * 32.0f, (float)corr, cacc);
            } else {
                ((float2 *)rs)[lane] = make_float2((float)sum, (float)corr);
                if (i == 0) ((float *)(rs + 512))[r] = fd;
            }
            if (DUMP) {
                const int tsum = sum8_i32(sum), tcorr = sum4_i32(corr);
                if (row_ok && i == 0) {
                    const size_t di = (size_t)(obase + mrow + r) * nb + st;
                    a.dump_s[di] = tsum;
                    a.dump_m[di] = tcorr;
                }
            }
        }
    };
    // whole rounds of R steps as straight-line code, refilling the ring. The rounds that end at
    // least R steps before the wavefront's last step neither reach a partial step nor refill past
    // the last (no checks, no clamp on the refill address); the next round may do both; then the
    // last nsl % R steps.
    using Check = std::true_type;
    using NoCheck = std::false_type;
    int b0 = 0;
    for (; b0 + 2 * R <= nsl; b0 += R) {
#pragma unroll
        for (int k = 0; k < R; ++k) {
            step(ring[k], s0 + b0 + k, NoCheck());
            step_load(T0 + (size_t)(b0 + k + R) * sstride, (uint32_t)lane, ring[k]);
        }
    }
    if (b0 + R <= nsl) {
#pragma unroll
        for (int k = 0; k < R; ++k) {
            step(ring[k], s0 + b0 + k, Check());
            step_load(T0 + (size_t)min(b0 + k + R, sl) * sstride, (uint32_t)lane, ring[k], b0 + k + R <= sl);
        }
        b0 += R;
    }
#pragma unroll
    for (int k = 0; k < R - 1; ++k)
        if (b0 + k < nsl) step(ring[k], s0 + b0 + k, Check());  // uniform

    if (S > 1) {
        __syncthreads();
        if (ks != 0) return;
        // the chains over the other wavefronts' steps, CH steps at a time (all reads first).
        // CHECK: the batch may reach the tile's partial last step or past the tile's end (the
        // tests are uniform; without them the chain is one fma per block, no select)
        constexpr int CH = q8_kind(TYPE) ? 4 : 8;
        auto batch = [&](int st0, auto check) {
            constexpr bool CHECK = decltype(check)::value;
            const uint8_t *rs = rec + (size_t)(st0 - nsw) * rec_bytes(TYPE);
            if constexpr (q8_kind(TYPE)) {
                float4 sv[CH], fv[CH], mv[CH];
                float4 bv[CH];
                constexpr size_t FD = rec_fd_off(TYPE);
#pragma unroll
                for (int c = 0; c < CH; ++c) {  // records past the end are read but not used
                    if (rec_i16(TYPE)) {
                        const uint2 p = ((const uint2 *)(rs + c * rec_bytes(TYPE)))[lane];
                        sv[c] = make_float4((float)(int16_t)(p.x & 0xFFFF), (float)((int)p.x >> 16),
                                            (float)(int16_t)(p.y & 0xFFFF), (float)((int)p.y >> 16));
                    } else {
                        sv[c] = ((const float4 *)(rs + c * rec_bytes(TYPE)))[lane];
                    }
                    fv[c] = ((const float4 *)(rs + c * rec_bytes(TYPE) + FD))[r];
                    if (q32_min(TYPE)) {
                        mv[c] = ((const float4 *)(rs + c * rec_bytes(TYPE) + FD + 128))[r];
                        bv[c] = *(const float4 *)(abs + 4 * (st0 + c));
                    }
                }
#pragma unroll
                for (int c = 0; c < CH; ++c) {
                    const int nbs = nb - 4 * (st0 + c);  // uniform
                    const float sk[4] = {sv[c].x, sv[c].y, sv[c].z, sv[c].w}, fk[4] = {fv[c].x, fv[c].y, fv[c].z, fv[c].w};
                    const float mk[4] = {mv[c].x, mv[c].y, mv[c].z, mv[c].w};
                    const float bk[4] = {bv[c].x, bv[c].y, bv[c].z, bv[c].w};
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        if (!CHECK || nbs >= 4 || k < nbs) {
                            acc = __builtin_fmaf(fk[k], sk[k], acc);
                            if (q32_min(TYPE)) cacc = __builtin_fmaf(mk[k], bk[k], cacc);
                        }
                }
            } else {
                float2 sv[CH];
                float fd[CH];
#pragma unroll
                for (int c = 0; c < CH; ++c) {
                    sv[c] = ((const float2 *)(rs + c * rec_bytes(TYPE)))[lane];
                    fd[c] = ((const float *)(rs + c * rec_bytes(TYPE) + 512))[r];
                }
#pragma unroll
                for (int c = 0; c < CH; ++c)
                    if (!CHECK || st0 + c < nst) {  // uniform
                        acc = __builtin_fmaf(fd[c], sv[c].x, acc);
                        cacc = __builtin_fmaf(fd[c] * 32.0f, sv[c].y, cacc);
                    }
            }
        };
        // batches of whole steps (4 blocks each for the 32-value types), then the rest
        const int nwhole = q8_kind(TYPE) ? nb / 4 : nst;
        int st0 = nsw;
        for (; st0 + CH <= nwhole; st0 += CH) batch(st0, NoCheck());
        for (; st0 < nst; st0 += CH) batch(st0, Check());
    }
    // hsum8(acc) - hsum4(cacc) over the row's 8 lanes (fastgguf.c:797-806, 1089-1095), in lane i = 0;
    // Q4_1 / Q5_1: hsum8(acc) + macc (973-989, 1020-1031); repacked Q4_0: the row chain itself
    const float e = acc + __shfl_xor(acc, 4);  // v_i + v_i+4
    const float f = e + xor1_f32(e);
    const float h8 = f + xor2_f32(f);
    float out = ORDER == 1 ? acc : h8;
    if (TYPE == T_Q6_K) {
        const float g = cacc + xor1_f32(cacc);
        out = h8 - (g + xor2_f32(g));
    }
    if (q32_min(TYPE)) out = h8 + cacc;
    if (row_ok && i == 0) a.t[ti].y[(size_t)tok * a.ldy + obase + mrow + r] = out;
}

// LDS of a launch: the activations and, with a block split, the records of TPW tiles (plus the
// steps that the last batch of the chain loop reads past the end)
static size_t mv_lds(int type, int nb, int tpw, int s) {
    const int nst = mv_steps(type, nb), nsw = (nst + s - 1) / s;
    const int pad = q8_kind(type) ? 3 : 7;
    return act_lds_bytes(type, nb) + (s > 1 ? ((size_t)tpw * (nst - nsw) + pad) * rec_bytes(type) : 0);
}
static int mv_tpw(int s) { return s == 1 ? 4 : s <= 4 ? 2 : 1; }

size_t matvec_lds_bytes(int type, int order, int nb) {
    if (type == T_Q4_K || type == T_Q5_K) return q4k_lds_bytes(order, nb);
    if (kq_kind(type)) return kq_lds_bytes(nb);
    if (fl_kind(type)) return fl_lds_bytes(type, nb);  // nb: the row's values
    return mv_lds(type, nb, 4, 1);
}

template <int TYPE, int ORDER, int R, int TPW, int S>
static hipError_t mv_launch(const MvArgs &a, int ntok, size_t lds, hipStream_t s) {
    const unsigned wg = (unsigned)((a.groups + TPW - 1) / TPW);
    if (a.dump_s) mv_kernel<TYPE, R, TPW, S, true, ORDER><<<dim3(wg, ntok), 64 * TPW * S, lds, s>>>(a);
    else mv_kernel<TYPE, R, TPW, S, false, ORDER><<<dim3(wg, ntok), 64 * TPW * S, lds, s>>>(a);
    return hipGetLastError();
}
template <int TYPE, int ORDER, int TPW, int S>
static hipError_t mv_launch_r(int R, const MvArgs &a, int ntok, size_t lds, hipStream_t s) {
    if constexpr (S == 1 && TPW == 4 && (TYPE == T_Q4_0 || TYPE == T_IQ4_NL))
        if (R == 16) return mv_launch<TYPE, ORDER, 16, TPW, S>(a, ntok, lds, s);
    if constexpr ((S == 2 && (TYPE == T_Q8_0 || TYPE == T_IQ4_NL)) || (S == 1 && TYPE != T_Q6_K))
        if (R == 8) return mv_launch<TYPE, ORDER, 8, TPW, S>(a, ntok, lds, s);
    return R == 2 ? mv_launch<TYPE, ORDER, 2, TPW, S>(a, ntok, lds, s) : mv_launch<TYPE, ORDER, 4, TPW, S>(a, ntok, lds, s);
}

// Launch shape: launches of fewer than 768 tiles (tiles x tokens) split the steps of a tile over up
// to 8 wavefronts, as many as keep the launch within 2048 wavefronts, each wavefront at 2 steps or
// more, the records within the 160 KiB of LDS of a workgroup and every workgroup of the launch
// resident at once; tiles per workgroup 4 for S = 1, 2 for S = 2 and 4 (halving the workgroups
// that each quantize x), 1 for S = 8. (With 4 steps or more per wavefront, as before for the
// 32-value types, 2048 x 2048, 1024 x 2048 and 512 x 2048 ran 9-15 % slower, 4096 x 1024 3-8 %;
// 1024 x 1024 and 2048 x 1024 of Q4_1 / Q5_0 gain 1-3 % with it; larger shapes do not split
// differently.) Q4_0, Q5_0 and IQ4_NL also split 2 ways from 768 to 1536 tiles within 3072
// wavefronts (11008 x 4096, 8192 x 4096, 6400 x 4096: IQ4_NL 13-15 %, Q4_0 / Q5_0 2-4 % faster;
// Q8_0 and Q6_K gain at some of these shapes and lose at others, 3-7 %, and Q4_1 / Q5_1 lose up
// to 5 %: they keep the 768-tile limit). Q6_K splits only up to 512 tiles: from 576 to 768
// (4608 .. 6144 rows) every split leaves some compute units two workgroups (288 .. 384 of them for
// 256 units) and waits for them, 18.0 - 19.4 us at 14336 columns against 16.7 - 16.9 unsplit, while
// 512 tiles split 4 ways fill the 256 units once (12.9 us against 16.5). Ring depth:
// 2 steps for launches of 1024 wavefronts or more over rows shorter than 32 steps and for
// wavefronts of 2 steps, 4 otherwise;
// Q6_K (steps of 1680 B, 1.5x the others'): 2 for split launches and for the LM-head size (8192
// tiles or more over rows shorter than 32 steps), 4 otherwise (measured, graph of back-to-back
// launches: 14336 x 4096 11.9 -> 11.0 us, 8192 x 2048 6.4 -> 5.8, 4096 x 14336 13.4 -> 13.1;
// the LM head, QKV and the split shapes unchanged). Q8_0 and IQ4_NL 2-way splits of rows of 64
// steps or more take ring depth 8 (4096 x 14336: 16.1 -> 15.6 us and 17.0 -> 16.2 us; the 4-way
// splits of the other types measured no faster with it). Unsplit launches of at most 1024 tiles
// over rows of 32 steps or more (rows whose split would not stay resident, or launches past the
// split limit), every type but Q6_K: ring depth 8 (8192 x 4096 / 6144 x 5120 / 7168 x 7168:
// Q8_0 9.4 / 10.7 / 14.0 -> 8.8 / 9.1 / 11.9 us, Q4_1 9.5 / 11.2 / 14.3 -> 8.1 / 9.8 / 11.8,
// Q5_1 10.7 / 12.6 / 16.2 -> 9.1 / 10.5 / 12.9; at 14336 x 4096, 1792 tiles, within 7 % either
// way, so that keeps depth 4; graph of back-to-back launches, 5120 x 13824 / 6144 x 16384 / 8192 x 8192:
// Q8_0 22.6 / 26.3 / 15.6 -> 17.8 / 20.6 / 14.9 us, Q5_0 24.8 / 28.5 -> 18.0 / 20.1, Q5_1
// 27.4 / 31.6 / 18.1 -> 21.3 / 24.0 / 14.5, Q4_1 23.7 / 27.6 / 15.8 -> 19.2 / 21.5 / 13.2,
// IQ4_NL 26.9 / 31.1 / 17.4 -> 23.1 / 26.2 / 15.5, Q4_0 22.2 / 25.5 -> 21.6 / 24.6; Q6_K no
// change); Q4_0 and IQ4_NL (the smallest steps, 576 B) ring depth 16 (IQ4_NL 23.1 / 26.1 / 15.6
// -> 21.3 / 23.0 / 14.5 us, Q4_0 21.7 / 24.6 -> 20.5 / 22.0; 16 was slower for the others).
template <int TYPE>
static MvShape mv_shape(int64_t tiles, int nb, int num_cu) {
    const int nst = mv_steps(TYPE, nb);
    int S = 1;
    // Q4_0, Q5_0 and IQ4_NL split 2 ways up to 1536 tiles and 3072 wavefronts too; Q6_K splits
    // only up to 512 tiles
    constexpr bool NIB = TYPE == T_Q4_0 || TYPE == T_Q5_0 || TYPE == T_IQ4_NL;
    if (tiles < (NIB ? 1536 : TYPE == T_Q6_K ? 513 : 768))
        while (S < 8 && (tiles * 2 * S <= 2048 || (NIB && S == 1 && tiles * 2 <= 3072)) && nst >= 4 * S &&
               mv_lds(TYPE, nb, mv_tpw(2 * S), 2 * S) <= GEMM_LDS_MAX &&
               all_resident((tiles + mv_tpw(2 * S) - 1) / mv_tpw(2 * S), 2 * S * mv_tpw(2 * S),
                            mv_lds(TYPE, nb, mv_tpw(2 * S), 2 * S), num_cu))
            S *= 2;
    int R = TYPE == T_Q6_K ? (S > 1 || (tiles >= 8192 && nst < 32) ? 2 : 4)
                           : (nst < 32 && tiles * S >= 1024) || (nst + S - 1) / S <= 2 ? 2 : 4;
    if ((TYPE == T_Q8_0 || TYPE == T_IQ4_NL) && S == 2 && (nst + 1) / 2 >= 32) R = 8;
    if (TYPE != T_Q6_K && S == 1 && tiles <= 1024 && nst >= 32)
        R = (TYPE == T_Q4_0 || TYPE == T_IQ4_NL) && nst >= 64 ? 16 : 8;
    return MvShape{S, R, mv_tpw(S), mv_lds(TYPE, nb, mv_tpw(S), S)};
}
template <int TYPE, int ORDER = 0>
static hipError_t mv_launch_type(const MvArgs &a, int ntok, int num_cu, hipStream_t s) {
    const MvShape sh = mv_shape<TYPE>(a.groups * ntok, a.nb, num_cu);
    if (sh.lds > (sh.S == 1 ? (size_t)65536 : GEMM_LDS_MAX)) return hipErrorInvalidValue;
    switch (sh.S) {
    case 1: return mv_launch_r<TYPE, ORDER, 4, 1>(sh.R, a, ntok, sh.lds, s);
    case 2: return mv_launch_r<TYPE, ORDER, 2, 2>(sh.R, a, ntok, sh.lds, s);
    case 4: return mv_launch_r<TYPE, ORDER, 2, 4>(sh.R, a, ntok, sh.lds, s);
    default: return mv_launch_r<TYPE, ORDER, 1, 8>(sh.R, a, ntok, sh.lds, s);
    }
}

MvShape matvec_shape(int type, int order, int64_t tiles, int nb, int num_cu) {
    switch (type) {
    case T_Q4_K: case T_Q5_K: return q4k_matvec_shape(type, order, tiles, nb, num_cu);
    case T_Q2_K: case T_Q3_K: case T_IQ4_XS: return kq_matvec_shape(type, tiles, nb, num_cu);
    case T_F32: case T_F16: case T_BF16: return fl_matvec_shape(type, tiles, nb, num_cu);
    case T_Q6_K: return mv_shape<T_Q6_K>(tiles, nb, num_cu);
    case T_Q8_0: return mv_shape<T_Q8_0>(tiles, nb, num_cu);
    case T_Q5_0: return mv_shape<T_Q5_0>(tiles, nb, num_cu);
    case T_Q5_1: return mv_shape<T_Q5_1>(tiles, nb, num_cu);
    case T_Q4_1: return mv_shape<T_Q4_1>(tiles, nb, num_cu);
    case T_IQ4_NL: return mv_shape<T_IQ4_NL>(tiles, nb, num_cu);
    case T_Q4_0: return mv_shape<T_Q4_0>(tiles, nb, num_cu);
    default: return MvShape{0, 0, 0, 0};
    }
}

hipError_t launch_matvec2(int type, int order, const MvArgs &a, int ntok, int num_cu, hipStream_t s) {
    if (type == T_Q4_K || type == T_Q5_K) return launch_q4k_matvec(type, order, a, ntok, num_cu, s);
    if (kq_kind(type)) return launch_kq_matvec(type, a, ntok, num_cu, s);
    if (fl_kind(type)) return launch_fl_matvec(type, a, ntok, num_cu, s);
    if (type == T_Q6_K) return mv_launch_type<T_Q6_K>(a, ntok, num_cu, s);
    if (type == T_Q8_0) return mv_launch_type<T_Q8_0>(a, ntok, num_cu, s);
    if (type == T_Q5_0) return mv_launch_type<T_Q5_0>(a, ntok, num_cu, s);
    if (type == T_Q5_1) return mv_launch_type<T_Q5_1>(a, ntok, num_cu, s);
    if (type == T_Q4_1) return mv_launch_type<T_Q4_1>(a, ntok, num_cu, s);
    if (type == T_IQ4_NL) return mv_launch_type<T_IQ4_NL>(a, ntok, num_cu, s);
    if (type == T_Q4_0)
        return order == 1 ? mv_launch_type<T_Q4_0, 1>(a, ntok, num_cu, s) : mv_launch_type<T_Q4_0, 0>(a, ntok, num_cu, s);
    return hipErrorInvalidValue;
}

}  // namespace fgh
