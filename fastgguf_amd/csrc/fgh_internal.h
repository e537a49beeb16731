// fgh_internal.h - device layouts and helpers shared by the gfx950 kernels of the fastgguf
// backend. Internal: the public surface is include/fastgguf_hip.h.
#pragma once

#include <hip/hip_runtime.h>
#include <limits.h>
#include <stdint.h>

namespace fgh {

// ---------------------------------------------------------------------------------------------
// Device weight layouts ("tiles"). Rows are interleaved in groups of 8, as the reference's CPU
// repack does for Q4_K (q4kx8_t, fastgguf.c:2260-2266), so one wavefront of 64 lanes = 8 rows x 8
// slices reads one contiguous tile per block with 16-byte loads. Lane (r, i) holds slice i of row
// r; slice i of a 256-weight block is exactly the part of the block the reference's AVX2 fp32
// accumulator lane i sums (its bytes 4i..4i+3 of every 32-byte chunk), so the per-lane integer
// partials are the reference's lane partials, and the fp32 chains can follow its order.
// Rows past the end of a matrix are zero-filled (d = 0) and never stored. Tiles lie step-major:
// step s (a block, or 4 blocks for Q8_0 / Q5_0) of row tile t of matrix m is tile
// (m * steps + s) * tpm + t, tpm = row tiles per matrix.
//
//   (Q4_K and Q5_K use their own layout of 16-row tiles, described in fgh_q4k.hip)
//   Q6_K tile, one block of 8 rows, 1680 B (= 8 x 210):
//     [0, 128)     int8 scales, row r at 16r (file bytes 192..207)
//     [128, 144)   fp16 d, row r at 128 + 2r (file bytes 208..209)
//     [144, 1168)  ql words, slice (r,i) at 144 + 16(8r+i): dword 2h+s = file bytes 64h+32s+4i..+3
//     [1168, 1680) qh words, slice (r,i) at 1168 + 8(8r+i): dword h = file bytes 128+32h+4i..+3
//   Q8_0 tile, 4 blocks of 8 rows, 1088 B (= 8 x 4 x 34):
//     [0, 64)      fp16 d of row r, block bb at 8r + 2bb
//     [64, 1088)   quants: slice (r, i) at 64 + 16(8r + i); dword bb = block bb's bytes 2+4i..+3
//   Q5_0 tile, 4 blocks of 8 rows, 704 B (= 8 x 4 x 22); slice (r, i) = elements 4i..4i+3 of each
//   block (element e: nibble e of the block's qs, low nibbles first, with bit e of qh as bit 4):
//     [0, 64)      fp16 d of row r, block bb at 8r + 2bb
//     [64, 576)    nibbles: slice (r, i) at 64 + 8(8r + i): byte 4w + t holds element 4i + t of
//                  block 2w in its low nibble and of block 2w + 1 in its high nibble
//     [576, 704)   fifth bits: slice (r, i) at 576 + 2(8r + i), 16 bits n0 | n2 << 4 | n1 << 8 |
//                  n3 << 12, where bit bb of the nibble n_t is the fifth bit of element 4i + t
//                  of block bb
//   Q4_0 / IQ4_NL tile (4 blocks of 8 rows, 576 B), Q4_1 (640 B), Q5_1 (768 B): Q5_0's regions
//     in the order scales, nibbles [512 B], fifth bits [128 B, Q5_1]; the scales of Q4_1 / Q5_1
//     are 16-byte row records [128 B]: fp16 d of row r, block bb at 16r + 2bb, then its fp16 m at
//     16r + 8 + 2bb (one 16-byte load per row and step); q32_layout gives the offsets
//   (Q5_K shares the Q4_K layout with 512 B of fifth bits per (tile, block), fgh_q4k.hip)
// ---------------------------------------------------------------------------------------------
constexpr int T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q4_1 = 3, T_Q5_0 = 6, T_Q5_1 = 7, T_Q8_0 = 8, T_Q2_K = 10,
              T_Q3_K = 11, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_IQ4_NL = 20, T_IQ4_XS = 23, T_BF16 = 30;
constexpr int Q4K_TILE = 2304, Q5K_TILE = 2816, Q6K_TILE = 1680, Q80_TILE = 1088, Q50_TILE = 704;
constexpr int Q4K_TILE_ROWS = 16;  // rows per Q4_K / Q5_K tile (8 for the other types)
// the activation kind of a weight type (type_uses_q8, fastgguf.c:2167-2173): Q8 blocks of 32 for
// the 32-value types, Q8_K blocks of 256 for the K-quants
__host__ __device__ constexpr bool q8_kind(int type) {
    return type == T_Q8_0 || type == T_Q5_0 || type == T_Q4_0 || type == T_Q4_1 || type == T_Q5_1 ||
           type == T_IQ4_NL;
}
// 32-value nibble types: tile bytes, region offsets (-1: absent) of a 4-block step, and the
// scale records: row r's at ds r, its fp16 d first, its fp16 m (Q4_1 / Q5_1) at + m
struct Q32Layout {
    int tile, m, n, h, ds;
};
__host__ __device__ constexpr Q32Layout q32_layout(int type) {
    return type == T_Q5_0 ? Q32Layout{704, -1, 64, 576, 8}
         : type == T_Q4_1 ? Q32Layout{640, 8, 128, -1, 16}
         : type == T_Q5_1 ? Q32Layout{768, 8, 128, 640, 16}
                          : Q32Layout{576, -1, 64, -1, 8};  // Q4_0, IQ4_NL
}
__host__ __device__ constexpr bool q32_min(int type) { return type == T_Q4_1 || type == T_Q5_1; }
// the 256-value types on Q8 activations (Q2_K, Q3_K, IQ4_XS; their own kernel, fgh_kq.hip):
// file block bytes and device tile bytes (16 rows of one block)
__host__ __device__ constexpr bool kq_kind(int type) { return type == T_Q2_K || type == T_Q3_K || type == T_IQ4_XS; }
__host__ __device__ constexpr int kq_block_bytes(int type) { return type == T_Q2_K ? 84 : type == T_Q3_K ? 110 : 136; }
constexpr int KQ_TILE_ROWS = 16;
__host__ __device__ constexpr int kq_tile(int type) { return KQ_TILE_ROWS * kq_block_bytes(type); }
// the float types F32, F16, BF16 (fp32 activations, their own kernel, fgh_float.hip): a step of a
// row tile is 1 KB, 16 bytes per lane: F32 tiles of 4 rows x 64 values, F16 8 x 64, BF16 64 x 8
__host__ __device__ constexpr bool fl_kind(int type) { return type == T_F32 || type == T_F16 || type == T_BF16; }
constexpr int FL_TILE = 1024;
__host__ __device__ constexpr int fl_tile_rows(int type) { return type == T_F32 ? 4 : type == T_F16 ? 8 : 64; }
__host__ __device__ constexpr int fl_step_elems(int type) { return type == T_BF16 ? 8 : 64; }
__host__ __device__ constexpr int fl_value_bytes(int type) { return type == T_F32 ? 4 : 2; }

// Device activation layouts. Q8_K (for the K-quants): per token, nb blocks of
//   qs [nb][256] int8, permuted so lane i's 32 bytes are contiguous: position 32i + 4c + k holds
//                 element 32c + 4i + k (an 8x8 transpose of the block's dwords)
//   d  [nb] fp32, bs [nb][16] int16 (the reference's bsums)
// Q8 (for Q8_0 / Q5_0): per token, nb32 blocks of qs [nb32][32] int8 (natural order), d [nb32] fp32,
//   s16 [nb32][2] int16.
// The Q4_K / Q5_K kernels' activation image (their LDS, and the MoE path's per-row images in
// HBM): natural-order Q8_K blocks: qs [nb][256] at 0, d [nb] fp32 at 256 nb, and the sums of each
// 32 values, bs32 [nb][8] int16 at align16(260 nb) (bs32[g] = bsums[2g] + bsums[2g+1] of the
// reference's q8k_blk_t: the min terms only ever use these pairs)
__host__ __device__ constexpr size_t q4_off_d(int nb) { return (size_t)nb * 256; }
__host__ __device__ constexpr size_t q4_off_s(int nb) { return ((size_t)nb * 260 + 15) & ~(size_t)15; }
__host__ __device__ constexpr size_t q4_act_bytes(int nb) { return (q4_off_s(nb) + (size_t)nb * 16 + 15) & ~(size_t)15; }
struct ActQ8K {
    int8_t *qs;
    float *d;
    int16_t *bs;
};
struct ActQ8 {
    int8_t *qs;
    float *d;
    int16_t *s16;
};

// (int)lrintf(v) as the reference computes it on x86 (fastgguf.c:762, 786): round half to even;
// a NaN or infinite v (id = 1/d overflows when amax is subnormal) gives the "integer indefinite"
// value, whose low byte is 0. A finite id keeps |v| <= 127, so no other case arises.
__device__ __forceinline__ int q8_round(float v) {
    return fabsf(v) < 2147483648.0f ? (int)rintf(v) : 0;
}
__device__ __forceinline__ uint32_t pack_q(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xFF) | ((uint32_t)(b & 0xFF) << 8) | ((uint32_t)(c & 0xFF) << 16) | ((uint32_t)(d & 0xFF) << 24);
}

// ---- cross-lane helpers (DPP: no LDS traffic) ----
__device__ __forceinline__ int dpp_xor1(int v) {  // quad_perm [1,0,3,2]
    return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
}
__device__ __forceinline__ int dpp_xor2(int v) {  // quad_perm [2,3,0,1]
    return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
}
__device__ __forceinline__ int dpp_half_mirror(int v) {  // lane j <-> 7-j within 8 lanes
    return __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, true);  // every lane has a source
}
// exact integer sum over the 8 lanes of a row group; every lane of the group gets the total
__device__ __forceinline__ int sum8_i32(int v) {
    v += dpp_xor1(v);
    v += dpp_xor2(v);
    v += dpp_half_mirror(v);
    return v;
}
__device__ __forceinline__ int sum4_i32(int v) {
    v += dpp_xor1(v);
    v += dpp_xor2(v);
    return v;
}

// ---- Q8_K quantization of one 256-value block by 16 threads (the Q4_K / Q5_K kernels' images) ----
// 16 threads per 256-value block; thread tl holds values 16tl..16tl+15 (4 float4 loads)
struct XRound {
    float4 v[4];
};
// block b of x (thread's 16 values: tl = threadIdx.x % 16); blocks past the end read block 0
__device__ __forceinline__ void q8k_load_b(const float *__restrict__ x, int b, bool live, XRound &xr) {
    const float *p = x + (size_t)(live ? b : 0) * 256 + 16 * (threadIdx.x & 15);
#pragma unroll
    for (int u = 0; u < 4; ++u) xr.v[u] = *(const float4 *)(p + 4 * u);
}
__device__ __forceinline__ float dpp_ror_f32(float v, int ctrl_n) {
    const int iv = __builtin_bit_cast(int, v);
    int r;
    switch (ctrl_n) {
    case 8: r = __builtin_amdgcn_update_dpp(0, iv, 0x128, 0xF, 0xF, false); break;
    case 4: r = __builtin_amdgcn_update_dpp(0, iv, 0x124, 0xF, 0xF, false); break;
    case 2: r = __builtin_amdgcn_update_dpp(0, iv, 0x122, 0xF, 0xF, false); break;
    default: r = __builtin_amdgcn_update_dpp(0, iv, 0x121, 0xF, 0xF, false); break;
    }
    return __builtin_bit_cast(float, r);
}
// quantizes the 16 threads' block b into act (stored only if live); the 16 threads of a block
// are one DPP row, so a row is either wholly live or wholly not
__device__ __forceinline__ void q8k_store_b(int nb, int b, bool live, const XRound &xr, uint8_t *act) {
    const int tl = threadIdx.x & 15;
    float v[16];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        v[4 * u] = xr.v[u].x; v[4 * u + 1] = xr.v[u].y; v[4 * u + 2] = xr.v[u].z; v[4 * u + 3] = xr.v[u].w;
    }
    float amax = 0.0f;
#pragma unroll
    for (int u = 0; u < 16; ++u) amax = fmaxf(amax, fabsf(v[u]));
    amax = fmaxf(amax, dpp_ror_f32(amax, 8));
    amax = fmaxf(amax, dpp_ror_f32(amax, 4));
    amax = fmaxf(amax, dpp_ror_f32(amax, 2));
    amax = fmaxf(amax, dpp_ror_f32(amax, 1));
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
    s += dpp_xor1(s);  // threads 2g, 2g+1: the 32 values of sub-block g
    if (live) {
        *(uint4 *)(act + (size_t)b * 256 + 16 * tl) = make_uint4(w[0], w[1], w[2], w[3]);
        if ((tl & 1) == 0) ((int16_t *)(act + q4_off_s(nb)))[8 * b + (tl >> 1)] = (int16_t)s;
        if (tl == 0) ((float *)(act + q4_off_d(nb)))[b] = d;
    }
}
__device__ __forceinline__ float fp16_bits_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// sum of four int8 x int8 products plus c (v_dot4_i32_i8)
__device__ __forceinline__ int dot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

// (lo & 0xFFFF) | (hi << 16): two int16 values packed for dot2_i16 (v_perm_b32)
__device__ __forceinline__ uint32_t pack_i16(int lo, int hi) {
    return __builtin_amdgcn_perm((uint32_t)hi, (uint32_t)lo, 0x05040100u);
}
// dot product of two packed int16 pairs plus c (v_dot2_i32_i16)
typedef short fgh_short2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ int dot2_i16(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(fgh_short2, a), __builtin_bit_cast(fgh_short2, b), c, false);
}

// IQ4_NL / IQ4_XS: the value kvalues_iq4nl[q] (fastgguf.c:475-477) of each nibble byte, by two
// byte permutes over the table's halves and a third that picks, per byte, the half by bit 3
__device__ __forceinline__ uint32_t iq4nl_values(uint32_t nib) {
    constexpr uint32_t T0 = 0xBFAD9881u, T1 = 0xF6EADDCFu, T2 = 0x26190D01u, T3 = 0x71594535u;  // -127 .. 113
    const uint32_t sel = nib & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(T1, T0, sel), hi = __builtin_amdgcn_perm(T3, T2, sel);
    return __builtin_amdgcn_perm(hi, lo, ((nib >> 1) & 0x04040404u) | 0x03020100u);
}

__device__ __forceinline__ int sbyte(uint32_t w, int k) {  // signed byte k of a dword
    return (int)(int8_t)(w >> (8 * k));
}
__device__ __forceinline__ int ubyte(uint32_t w, int k) { return (int)((w >> (8 * k)) & 0xFF); }

__device__ __forceinline__ uint4 ld16(const uint8_t *p) { return *(const uint4 *)p; }
__device__ __forceinline__ uint2 ld8(const uint8_t *p) { return *(const uint2 *)p; }

// Loads from a wavefront-uniform base through a buffer resource: the base lives in scalar
// registers and each lane adds its own 32-bit offset, so a walk that moves the base costs no
// vector instructions per load; reads at or past nbytes return 0 (0x00020000: the gfx9 resource
// word 3, 32-bit data format).
typedef __amdgpu_buffer_rsrc_t BufRes;
typedef unsigned fgh_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ BufRes buf_res(const uint8_t *base, uint32_t nbytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)base, 0, (int)nbytes, 0x00020000);
}
// AUX: the load's cache policy; WNT (the nt bit) for the decode and MoE weight streams, which every
// launch reads once: a streaming read of 0.2-1 GB with nt loads runs 9-12 % faster than with
// default loads (measured). The prompt GEMMs keep default loads: with nt their weight loads took
// Q8_0 23.7 -> 31.1 us and Q4_0 27.8 -> 29.7 us at 64 x 4096 -> 14336 (Q4_K and Q6_K unchanged).
#ifndef FGH_WEIGHT_AUX
#define FGH_WEIGHT_AUX 2
#endif
constexpr int WNT = FGH_WEIGHT_AUX;
template <int AUX = 0>
__device__ __forceinline__ uint4 bld16(BufRes r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, AUX);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
template <int AUX = 0>
__device__ __forceinline__ uint2 bld8(BufRes r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, AUX);
    return make_uint2(v[0], v[1]);
}
template <int AUX = 0>
__device__ __forceinline__ uint32_t bld2(BufRes r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, AUX); }

// Q4_K 12-byte scales -> sc (4 bytes each in lo/hi words) and mins, the word form of
// scale_min_k4 (fastgguf.c:466-472) that unpack_scales_k4 (1057-1067) also uses
struct Q4KScales {
    uint32_t sc_lo, sc_hi, mn_lo, mn_hi;  // bytes: sc0..3, sc4..7, m0..3, m4..7
};
__device__ __forceinline__ Q4KScales q4k_scales(uint32_t u0, uint32_t u1, uint32_t u2) {
    const uint32_t k1 = 0x3f3f3f3fu, k2 = 0x0f0f0f0fu, k3 = 0x03030303u;
    Q4KScales s;
    s.sc_lo = u0 & k1;
    s.sc_hi = (u2 & k2) | (((u0 >> 6) & k3) << 4);
    s.mn_lo = u1 & k1;
    s.mn_hi = ((u2 >> 4) & k2) | (((u1 >> 6) & k3) << 4);
    return s;
}
__device__ __forceinline__ int q4k_sc(const Q4KScales &s, int j) {
    return ubyte(j < 4 ? s.sc_lo : s.sc_hi, j & 3);
}
__device__ __forceinline__ int q4k_mn(const Q4KScales &s, int j) {
    return ubyte(j < 4 ? s.mn_lo : s.mn_hi, j & 3);
}


// host-side launchers (fgh_kernels.hip)
hipError_t launch_quant_q8k(const float *x, int64_t ldx, int nb, int ntok, ActQ8K act, hipStream_t s);
hipError_t launch_quant_q8(const float *x, int64_t ldx, int nb, int ntok, ActQ8 act, hipStream_t s);
hipError_t launch_relayout(const uint8_t *src, uint8_t *dst, int type, int64_t rows, int nb, int ntile,
                           int64_t gpm, int64_t total, int64_t row_bytes, hipStream_t s);
hipError_t launch_fp16(const uint16_t *h, float *out, int n, hipStream_t s);
hipError_t launch_copy16(const void *src, void *dst, int64_t n16, hipStream_t s);
int checksum_parts(int num_cu);  // the most workgroups of launch_checksum (words of its part buffer)
hipError_t launch_checksum(const void *src, int64_t n16, uint32_t *part, int num_cu, uint32_t *out, hipStream_t s);

// decode matvec (fgh_matvec.hip): up to 4 tensors of one type, order and width in one launch
struct MvT {
    const uint8_t *W;
    float *y;
    int64_t rows;    // rows per matrix
    int64_t gpm;     // row tiles per matrix (16 rows for Q4_K / Q5_K / Q2_K / Q3_K / IQ4_XS, 8 otherwise)
    int64_t gfirst;  // first global tile index of this tensor
};
struct MvArgs {
    MvT t[4];
    int nt;
    int64_t groups;    // row tiles over all the tensors
    const float *x;    // fp32 activations, quantized inside the kernel
    int64_t ldx, ldy;  // token strides of x and of every y
    int nb, ntile;     // blocks and tiles per row
    int32_t *dump_s, *dump_m;  // test hook: per (row, block) integers of tensor 0, or null
    // expert indirection (MoE): when sel is set, token slot y (blockIdx.y) uses matrix sel[y] of
    // every tensor (launched with the tiles of one matrix) and activation row y / xdiv
    const int32_t *sel;
    int xdiv;
    // MoE routing inside the launch (Q4_K / Q5_K kernels, instead of sel): token slot y routes
    // token y / xdiv itself (logits [tokens][n_expert]) and takes its selected expert y % xdiv; the
    // slot-0 workgroup 0 of each token writes its k = xdiv experts and weights to sel_out / w_out.
    // Such a launch takes t[0] = gate, t[1] = up of the same shape and writes h = silu(g) * u to
    // t[0].y (g and u themselves are not stored). route_off: the LDS byte offset of the
    // wavefronts' routing buffers (set by the launcher)
    const float *logits;
    int n_expert;
    int32_t *sel_out;
    float *w_out;
    uint32_t route_off;
    // the same pairing of gate (t[0]) and up (t[1]) without routing: h = silu(g) * u to t[0].y
    int pair;
};
enum { MV_PLAIN = 0, MV_PAIR = 1, MV_ROUTE = 2 };  // decode kernel forms (Q4_K / Q5_K)
size_t matvec_lds_bytes(int type, int order, int nb);  // every type (fgh_matvec.hip)
// the launch shape a decode launch of `tiles` row tiles (over all tokens) picks: S wavefronts per
// tile, ring depth R, TPW tiles per workgroup, its dynamic LDS bytes (S == 0: no kernel)
struct MvShape {
    int S, R, TPW;
    size_t lds;
};
MvShape matvec_shape(int type, int order, int64_t tiles, int nb, int num_cu);
MvShape q4k_matvec_shape(int type, int order, int64_t tiles, int nb, int num_cu);
// Q4_K / Q5_K (fgh_q4k.hip): their own tile layout and kernel
size_t q4k_lds_bytes(int order, int nb);
hipError_t launch_q4k_matvec(int type, int order, const MvArgs &a, int ntok, int num_cu, hipStream_t s);
// F32 / F16 / BF16 (fgh_float.hip): a.nb = the row's values, a.ntile = its steps
size_t fl_lds_bytes(int type, int64_t cols);
MvShape fl_matvec_shape(int type, int64_t tiles, int64_t cols, int num_cu);
hipError_t launch_fl_matvec(int type, const MvArgs &a, int ntok, int num_cu, hipStream_t s);
hipError_t launch_fl_relayout(int type, const uint8_t *src, uint8_t *dst, int64_t rows, int64_t cols, int steps,
                              int64_t gpm, int64_t total, hipStream_t s);
// the MoE down projection and ordered combine of each token in one launch (Q4_K / Q5_K row order):
// a.t[0] = {down, y}, a.x = the h = silu(g) * u rows of the token slots (stride a.ldx), a.sel the
// slots' experts, wts their weights, k <= 8 experts per token
size_t q4k_moe_down_lds(int nb, int k);
// whether a Q4_K / Q5_K decode launch over `tiles` tiles x tokens has room to route its tokens
bool q4k_route_fits(int type, int order, int64_t tiles, int nb, int num_cu);
hipError_t launch_q4k_moe_down(int type, const MvArgs &a, const float *wts, int k, int ntok, hipStream_t s);
hipError_t launch_q4k_relayout(int type, const uint8_t *src, uint8_t *dst, int64_t rows, int nb, int64_t tpm,
                               int64_t total, int64_t row_bytes, hipStream_t s);
hipError_t launch_matvec2(int type, int order, const MvArgs &a, int ntok, int num_cu, hipStream_t s);
// Q2_K / Q3_K / IQ4_XS (fgh_kq.hip): tiles, decode kernel, launch shape
size_t kq_lds_bytes(int nb);
MvShape kq_matvec_shape(int type, int64_t tiles, int nb, int num_cu);
hipError_t launch_kq_matvec(int type, const MvArgs &a, int ntok, int num_cu, hipStream_t s);
hipError_t launch_kq_relayout(int type, const uint8_t *src, uint8_t *dst, int64_t rows, int nb, int64_t gpm,
                              int64_t total, int64_t row_bytes, hipStream_t s);

// MoE around the expert matvecs (fgh_moe.hip)
// expf as glibc >= 2.27 computes it (the method of ARM's optimized-routines expf), in double:
// with N = 32, z = x N / ln 2, k = round(z), r = fma(N / ln 2, x, -k) (glibc's x86-64 FMA build
// fuses it), exp(x) = 2^(k / N) * 2^(r / N), where
// 2^(k / N) = table[k mod N] (the correctly rounded 2^(i / N), i < N, stored with i << 47
// subtracted) with k << 47 added to its bits, and 2^(r / N) ~ (c0 r + c1) r^2 + (c2 r + 1)
// (fused multiply-adds);
// one rounding to float at the end. Matches the host libm bit for bit (the oracle tests sweep the
// floats); the reference calls expf in softmax and silu (fastgguf.c:3118, 3151).
__host__ __device__ inline float expf_ref(float x) {
    constexpr uint64_t tab[32] = {
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
    0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
    0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
    0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
    0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
    0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL,
    };
    const double invln2n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32;
    // No branch and no select on the result (the compiler would turn either into a branch around
    // the table read, whose wait then serializes unrolled calls): x is clamped to [-128, 128], where
    // the method itself gives 0 and +inf (as glibc's early returns do), and a NaN x is added back.
    const float xc = fminf(fmaxf(x, -128.0f), 128.0f);  // a NaN x becomes -128 (result 0)
    const float nan_x = x != x ? x : 0.0f;
    const double xd = xc;
    const double z = invln2n * xd;
    double kd = z + shift;
    uint64_t ki;
    __builtin_memcpy(&ki, &kd, 8);
    kd -= shift;
    const double r = __builtin_fma(invln2n, xd, -kd);  // fused, as glibc's FMA build (x86-64)
    const uint64_t t = tab[ki % 32] + (ki << 47);
    double s;
    __builtin_memcpy(&s, &t, 8);
    const double p = __builtin_fma(c0, r, c1), r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(p, r2, y);
    return (float)(y * s) + nan_x;
}

// ---- MoE routing (fgh_moe.hip's route launch, and the decode kernel when it routes itself) ----
constexpr int MOE_EPL = 8;

// an int whose signed order is the float order (for non-NaN floats)
__device__ __forceinline__ int f32_ord(float f) {
    const int b = __builtin_bit_cast(int, f);
    return b < 0 ? b ^ 0x7FFFFFFF : b;
}
// maximum over the 64 lanes, in every lane: within rows of 16 by DPP, then the four row results
__device__ __forceinline__ int wave_max_i32(int v) {
    v = max(v, __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xF, 0xF, false));   // quad_perm [1,0,3,2]
    v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xF, 0xF, false));   // quad_perm [2,3,0,1]
    v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x141, 0xF, 0xF, false));  // row_half_mirror
    v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x140, 0xF, 0xF, false));  // row_mirror
    return max(max(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
               max(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}
__device__ __forceinline__ float wave_fmax(float v) {  // fmaxf over the lanes (a NaN lane loses)
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false)));
    auto rl = [&](int l) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l)); };
    return fmaxf(fmaxf(rl(0), rl(16)), fmaxf(rl(32), rl(48)));
}

// The routing of one token by one wavefront (the reference's moe_ffn routing, fastgguf.c:4594-4604,
// over softmax_inplace 3147-3156 and argmax_f 3328-3332): lg its n_expert logits (NS = the 64-expert
// slots a lane holds, n_expert <= 64 NS), ps 64 * MOE_EPL floats of LDS for this wavefront. Writes
// the k selected experts to sel and their weights to w (either may be null) and returns selected
// expert number `want` (uniform). Lane l holds experts 64 s + l (slot s) in registers; the maxima
// are DPP / lane-read reductions (no barrier) and only the reference's sequential softmax sum goes
// through LDS. Straight-line code over the slots: no branch waits on a memory read.
template <int NS>
__device__ __forceinline__ int moe_route_ns(const float *__restrict__ lg, int n_expert, int k, float *ps,
                                            int32_t *sel, float *w, int want) {
    const int lane = threadIdx.x & 63;
    const BufRes lr = buf_res((const uint8_t *)lg, (uint32_t)n_expert * 4);
    float pv[NS];
    // max: the reference keeps the larger of each value and the running max (starting at -inf),
    // which fmaxf does, NaN never winning; the same value in every lane
    float mx = -INFINITY;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        const float v = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(lr, 4 * (64 * s + lane), 0, 0));
        pv[s] = 64 * s + lane < n_expert ? v : -INFINITY;
        mx = fmaxf(mx, pv[s]);
    }
    mx = wave_fmax(mx);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        pv[s] = expf_ref(pv[s] - mx);
        ps[64 * s + lane] = pv[s];
    }
    // one wavefront: its LDS writes above precede lane 0's reads below.
    // The reference's sequential sum: lane 0 adds 16 values at a time while the next 16 are read.
    float sum = 0.0f;
    if (lane == 0) {
        const float4 *p4 = (const float4 *)ps;
        const int nf = n_expert >> 4;
        float4 c0 = p4[0], c1 = p4[1], c2 = p4[2], c3 = p4[3];
        for (int c = 0; c < nf; ++c) {
            const int nx = 4 * min(c + 1, nf - 1);
            const float4 d0 = p4[nx], d1 = p4[nx + 1], d2 = p4[nx + 2], d3 = p4[nx + 3];
            sum += c0.x; sum += c0.y; sum += c0.z; sum += c0.w;
            sum += c1.x; sum += c1.y; sum += c1.z; sum += c1.w;
            sum += c2.x; sum += c2.y; sum += c2.z; sum += c2.w;
            sum += c3.x; sum += c3.y; sum += c3.z; sum += c3.w;
            c0 = d0; c1 = d1; c2 = d2; c3 = d3;
        }
        for (int i = 16 * nf; i < n_expert; ++i) sum += ps[i];
    }
    sum = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sum), 0));
    const float inv = 1.0f / sum;
#pragma unroll
    for (int s = 0; s < NS; ++s) pv[s] = sum > 0.0f ? pv[s] * inv : pv[s];  // skipped unless sum > 0
    // top-k by repeated argmax: candidates are values > -inf (a NaN never is), the first index of
    // the largest wins, and with no candidate index 0 is taken; the chosen value becomes -1
    const int ord_m1 = f32_ord(-1.0f);
    int key[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) key[s] = 64 * s + lane < n_expert && pv[s] > -INFINITY ? f32_ord(pv[s]) : INT_MIN;
    float wsum = 0.0f, wl = 0.0f;
    int sl = 0, pick_want = 0;
    for (int j = 0; j < k; ++j) {
        int m = key[0];
#pragma unroll
        for (int s = 1; s < NS; ++s) m = max(m, key[s]);
        m = wave_max_i32(m);
        int bi = 0;  // the lowest expert holding the maximum (uniform)
#pragma unroll
        for (int s = NS - 1; s >= 0; --s) {
            const uint64_t hit = __ballot(key[s] == m);
            bi = hit ? 64 * s + (int)__builtin_ctzll(hit) : bi;
        }
        bi = m == INT_MIN ? 0 : bi;
        const int bl = bi & 63, bs = bi >> 6;
        float pick = pv[0];
#pragma unroll
        for (int s = 1; s < NS; ++s) pick = s == bs ? pv[s] : pick;
        const float pvj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pick), bl));
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const bool hitme = lane == bl && s == bs;
            pv[s] = hitme ? -1.0f : pv[s];
            key[s] = hitme ? ord_m1 : key[s];
        }
        wl = lane == j ? pvj : wl;
        sl = lane == j ? bi : sl;
        pick_want = j == want ? bi : pick_want;
        wsum += pvj;  // every lane keeps the same sequential sum
    }
    if (wsum < 6.103515625e-5f) wsum = 6.103515625e-5f;
    if (sel && lane < k) sel[lane] = sl;
    if (w && lane < k) w[lane] = wl / wsum;
    return pick_want;
}
// n_expert <= 64 * MOE_EPL, k <= min(n_expert, 64)
__device__ __forceinline__ int moe_route_wave(const float *__restrict__ lg, int n_expert, int k, float *ps,
                                              int32_t *sel, float *w, int want) {
    if (n_expert <= 64) return moe_route_ns<1>(lg, n_expert, k, ps, sel, w, want);
    if (n_expert <= 128) return moe_route_ns<2>(lg, n_expert, k, ps, sel, w, want);
    if (n_expert <= 256) return moe_route_ns<4>(lg, n_expert, k, ps, sel, w, want);
    return moe_route_ns<MOE_EPL>(lg, n_expert, k, ps, sel, w, want);
}

hipError_t launch_expf(const float *x, float *y, int n, hipStream_t s);  // test hook
// the MFMA-only rate probe (fgh_kernels.hip): launch, its workgroups, int8 ops per launch
int mfma_peak_blocks(int num_cu);
uint64_t mfma_peak_ops(int num_cu, int iters);
hipError_t launch_mfma_peak(int iters, uint32_t *sink, int num_cu, hipStream_t s);
// h = silu(g) * u over n values (silu_f, fastgguf.c:3118); h may be g
hipError_t launch_silu_mul(const float *g, const float *u, float *h, int64_t n, hipStream_t s);
hipError_t launch_moe_route(const float *logits, int n_expert, int k, int n_tok, int32_t *sel, float *w, hipStream_t s);
// the grouped path's first launch (fgh_q4k.hip): x images, routing, and the slots filed in
// per-expert buckets of n_tok * k entries (a token may pick one expert more than once when its
// probabilities are not finite); cnt[n_expert] zero on entry; moe_combine clears it
hipError_t launch_moe_prep(const float *x, int64_t ldx, int nb, uint8_t *img, const float *logits, int n_expert,
                           int k, int n_tok, int32_t *sel, float *w, int32_t *cnt, int32_t *bucket, hipStream_t s);
// grouped Q4_K row-order expert matvecs on the VALU (fgh_q4k.hip): a.groups = tiles of one matrix
// over a.t; rows of at most q4k_moe_max_blocks() blocks; expert e's slots in buckets[e * cap ..),
// cnt[e] of them
size_t q4k_moe_lds_bytes(int nb);
int q4k_moe_max_blocks();
hipError_t launch_q4k_moe(const MvArgs &a, const int32_t *cnt, const int32_t *buckets, int cap, int n_expert,
                          const uint8_t *img, hipStream_t s);
// the same on int8 MFMA (fgh_moemm.hip), bit-identical: one launch over w0 (and w1 of the same
// shape, its tiles after w0's) [E][rows][cols], y0 / y1 [slot * ldy + row], activation image row
// slot / xdiv; chunks of 4 * nsg slots (1, 2 or 4) side by side, q4k_moe_mfma_lds(nsg, nb) bytes of
// LDS; r: ring depth (2, 3 or 4 blocks); tt: tiles per wavefront (0: about three wavefronts per
// SIMD over all experts). dump_s / dump_m (or null): w0's integers [slot][rows][nb].
struct MoeMmShape {
    int nsg = 2, r = 3, tt = 0;
};
size_t q4k_moe_mfma_lds(int nsg, int nb);
hipError_t launch_q4k_moe_mfma(const MoeMmShape &sh, const uint8_t *w0, const uint8_t *w1, int64_t rows, int64_t gpm,
                               int nb, const int32_t *cnt, const int32_t *buckets, int cap, int n_expert, int n_tok,
                               const uint8_t *img, int xdiv, float *y0, float *y1, int64_t ldy, int32_t *dump_s,
                               int32_t *dump_m, int num_cu, hipStream_t s);
// zeroes n ints (a small fill kernel: the grouped path's counts after a failed launch)
hipError_t launch_zero_i32(int32_t *p, int n, hipStream_t s);
// Q8_K images of rows in the decode kernels' LDS layout; u != null: the rows are silu(x) * u
size_t q4_image_bytes(int nb);
hipError_t launch_q4_image(const float *x, const float *u, int64_t ldx, int nb, int64_t rows, uint8_t *img,
                           hipStream_t s);
// y = the ordered combine of the k experts' rows; cnt != null: also clears cnt[n_expert] (the
// grouped path's bucket counts, for its next call)
hipError_t launch_moe_combine(const float *d, const float *w, float *y, int n_embd, int k, int n_tok, int64_t ldy,
                              int32_t *cnt, int n_expert, hipStream_t s);

// attention over an fp32 KV ring cache (fgh_attn.hip): rows (token, head), row t * n_head + h
struct AttnArgs {
    const float *q;           // [rows][hd]
    float *o;                 // [rows][hd]
    const float *k, *v;       // [cap][kv_dim] ring caches (slot = position % cap)
    float *s;                 // [rows][max_len] scores, then weights
    const int32_t *st, *en;   // [tokens] position ranges
    int n_head, n_head_kv, hd, kv_dim, cap, max_len;
    float scale;
    // the value chains only: V as TurboQuant records instead of v (vbits 2, 4 or 8; the records'
    // scales already folded into the weights), each value its centroid or int8 code
    const uint8_t *vq = nullptr;
    int vbits = 0;
};
hipError_t launch_attention(const AttnArgs &a, int n_tok, hipStream_t s);

// the Lloyd-Max centroids of N(0, 1) of the TurboQuant cache (fastgguf.c:3356-3359)
__host__ __device__ inline float kvq_centroid4(int i) {
    switch (i & 15) {
    case 0: return -2.7326f;  case 1: return -2.0690f;  case 2: return -1.6181f;  case 3: return -1.2562f;
    case 4: return -0.9424f;  case 5: return -0.6568f;  case 6: return -0.3881f;  case 7: return -0.1284f;
    case 8: return 0.1284f;   case 9: return 0.3881f;   case 10: return 0.6568f;  case 11: return 0.9424f;
    case 12: return 1.2562f;  case 13: return 1.6181f;  case 14: return 2.0690f;  default: return 2.7326f;
    }
}
__host__ __device__ inline float kvq_centroid2(int i) {
    switch (i & 3) {
    case 0: return -1.5104f;  case 1: return -0.4528f;  case 2: return 0.4528f;  default: return 1.5104f;
    }
}
hipError_t launch_attention_values(const AttnArgs &a, int n_tok, hipStream_t s);  // the value chains only

// TurboQuant KV cache (fgh_kvq.hip): records of 4 + hd * bits / 8 bytes per (slot, K / V head)
struct KvqStoreArgs {
    const float *k, *v;  // [tokens][stride] new K / V rows (n_head_kv * hd values each)
    uint8_t *kq, *vq;    // [cap][n_head_kv records]
    const int32_t *pos;  // [tokens] positions (slot = pos % cap)
    int stride, n_head_kv, hd, kbits, vbits, cap;
};
hipError_t launch_kvq_store(const KvqStoreArgs &a, int n_tok, hipStream_t s);
struct KvqAttnArgs {
    const float *q;           // [rows][hd] unrotated queries
    float *o;                 // [rows][hd] outputs, rotated back
    float *qr, *orot;         // [rows][hd] scratch: rotated queries, rotated outputs
    float *s;                 // [rows][max_len] scores, then weights
    const uint8_t *kq, *vq;   // quantized caches
    const int32_t *st, *en;   // [tokens] position ranges
    int n_head, n_head_kv, hd, kbits, vbits, cap, max_len;
    float scale;
};
hipError_t launch_kvq_attention(const KvqAttnArgs &a, int n_tok, hipStream_t s);

// prompt-batch Q4_K GEMM (fgh_gemm.hip): 1..64 tokens, weights in the Q4_K decode layout
struct GemmArgs {
    const uint8_t *W;      // Q4_K tensor (tile layout)
    float *Y;              // Y[tok * ldy + row]
    int64_t rows, gpm;     // rows and 16-row tiles per matrix
    int64_t groups;        // tiles over all matrices
    int64_t nrows;         // rows over all matrices (outputs per token)
    int nb;                // 256-blocks per row
    const uint8_t *act;    // activation records from launch_gemm_quant
    int Tp, T;             // padded token count (a multiple of 16, Tp - T < 16), tokens
    int64_t ldy;
    int32_t *dump_s, *dump_m;  // test hook: [T][nrows][nb] integers, or null
    int ks;                    // K splits (grid.y); ks > 1: partials [ks][T][nrows] and counters
    float *part;
    int32_t *cnt;
};
// the Q8_0 prompt GEMM (fgh_gemm32.hip) on the decode tiles (8-row tiles, 4 blocks per tile step)
struct Gemm32Args {
    const uint8_t *W;      // Q8_0 tensor (tile layout)
    float *Y;              // Y[tok * ldy + row]
    int64_t rows;          // rows per matrix
    int64_t tpm;           // 8-row tiles per matrix
    int64_t gpm32;         // 32-row groups per matrix, (tpm + 3) / 4
    int64_t groups;        // 32-row groups over all matrices
    int64_t nrows;         // rows over all matrices (outputs per token)
    int nb, nsteps;        // 32-blocks per row, tile steps per row ((nb + 3) / 4)
    const uint8_t *act;    // activation records from launch_gemm32_quant
    int Tp, T;             // padded token count (32 or 64, Tp - T < 32), tokens
    int64_t ldy;
    int32_t *dump_s;       // test hook: [T][nrows][nb] integers, or null
    int ks;                // K splits of the tile steps (grid.y); ks > 1: partials and counters
    float *part;
    int32_t *cnt;
};
// the Q8_0 GEMM's records; zeroes the K split's ncnt counters
hipError_t launch_gemm32_quant(const float *x, int64_t ldx, int nb, int T, int Tp, uint8_t *rec, int32_t *cnt, int ncnt,
                               hipStream_t s);
int gemm32_workgroups(int64_t groups);  // workgroups (row groups of the Q8_0 GEMM) over groups
size_t gemm32_act_bytes(int nb, int Tp);
hipError_t launch_q80_gemm(const Gemm32Args &a, hipStream_t s);

// the prompt GEMM of the nibble types Q4_0 / Q4_1 / Q5_0 / Q5_1 (fgh_gemm32n.hip) on the decode
// tiles (8-row tiles, 4 blocks per tile step)
struct GemmNArgs {
    const uint8_t *W;      // tensor (tile layout)
    float *Y;              // Y[tok * ldy + row]
    int64_t rows;          // rows per matrix
    int64_t tpm;           // 8-row tiles per matrix
    int64_t ppm;           // 16-row pairs of tiles per matrix, (tpm + 1) / 2
    int64_t groups;        // pairs over all matrices
    int64_t nrows;         // rows over all matrices (outputs per token)
    int nb, nsteps;        // 32-blocks per row, tile steps per row ((nb + 3) / 4)
    const uint8_t *act;    // activation records from launch_gemmn_quant
    int Tp, T;             // padded token count (a multiple of 16, Tp - T < 16), tokens
    int64_t ldy;
    int32_t *dump_s;       // test hook: [T][nrows][nb] integers sum u * xq, or null
    int type;
};
hipError_t launch_gemmn_quant(const float *x, int64_t ldx, int nb, int T, int Tp, uint8_t *rec, hipStream_t s);
size_t gemmn_act_bytes(int nb, int Tp);
hipError_t launch_q32n_gemm(const GemmNArgs &a, hipStream_t s);

// the Q6_K prompt GEMM (fgh_gemm6.hip) on the decode tiles (8-row tiles, one block per tile step)
struct Gemm6Args {
    const uint8_t *W;      // Q6_K tensor (tile layout)
    float *Y;              // Y[tok * ldy + row]
    int64_t rows;          // rows per matrix
    int64_t tpm;           // 8-row tiles per matrix
    int64_t gpm16;         // 16-row tiles (pairs of decode tiles) per matrix, (tpm + 1) / 2
    int64_t groups;        // 16-row tiles over all matrices
    int64_t nrows;         // rows over all matrices (outputs per token)
    int nb;                // 256-blocks per row
    const uint8_t *act;    // activation records from launch_gemm6_quant
    int Tp, T;             // padded token count (a multiple of 16, Tp - T < 16), tokens
    int64_t ldy;
    int32_t *dump_s, *dump_m;  // test hook: [T][nrows][nb] sumi / msum, or null
    int ks;                    // K splits (grid.y); ks > 1: partials [ks][T][nrows] and counters
    float *part;
    int32_t *cnt;
};
// the Q6_K GEMM's records (gemm6_act_bytes(nb, Tp)); zeroes the K split's ncnt counters
hipError_t launch_gemm6_quant(const float *x, int64_t ldx, int nb, int T, int Tp, uint8_t *rec, int32_t *cnt, int ncnt,
                              hipStream_t s);
size_t gemm6_act_bytes(int nb, int Tp);
hipError_t launch_q6k_gemm(const Gemm6Args &a, hipStream_t s);

// quantizes T rows of x (stride ldx) into the GEMM's activation records (gemm_act_bytes(nb, Tp))
// and zeroes the K split's ncnt arrival counters (cnt may be null when ncnt is 0)
hipError_t launch_gemm_quant(const float *x, int64_t ldx, int nb, int T, int Tp, uint8_t *rec, int32_t *cnt, int ncnt,
                             hipStream_t s);
size_t gemm_act_bytes(int nb, int Tp);
// The scratch of a prompt GEMM (Q4_K, Q6_K, Q8_0): its activation records (rec_bytes), then, when
// it splits K (ks > 1), one arrival counter per workgroup of a split (ncnt) and the partials: per
// split and workgroup 64 rows x Tp tokens of fp32. ks: as many splits (up to 4) of the units
// along K (blocks or tile steps) as still give each workgroup its own compute unit, each split at
// least min_units; short outputs (the down projection 14336 -> 4096: 64 workgroups) otherwise
// leave most units idle.
struct GemmScratch {
    int ks, ncnt;
    size_t cnt_off, part_off, bytes;
};
GemmScratch gemm_split_scratch(size_t rec_bytes, int64_t wg, int units, int min_units, int Tp, int num_cu);
GemmScratch gemm_scratch(int64_t groups, int nb, int T, int num_cu);  // Q4_K's

// The end of a K-split prompt GEMM workgroup (grid.y = ks splits of consecutive K units;
// blockIdx.x = the row group; nslot storing wavefronts, this one slot). A storing wavefront
// (mine: uniform) holds NE outputs per lane: element e is token tok(e) of row orow, value val(e).
// Its partial goes to its own NE x 64 floats of part, quad q of lane l at 16 (64 q + l) bytes
// (each store instruction writes 1 KB contiguous), as write-through stores (sc1, agent scope);
// every wavefront waits until its stores have completed, then thread 0 bumps the row group's
// counter. The last split to arrive loads the other partials (sc1 loads, which read past the L2 of
// the reading XCD; all in flight at once) and writes Y = ((p_0 + p_1) + p_2) + p_3 for its lanes
// with store set, in split order whichever arrives last. Every wavefront of the workgroup calls
// it (two barriers); flag is one int of LDS. An agent-scope release instead of the write-through
// stores writes back the whole L2 of the workgroup's XCD; 4-byte stores and loads scattered by
// token took 10 us more at 64 x 14336 -> 4096.
template <int NE, class Tok, class Val>
__device__ __forceinline__ void gemm_split_finish(Tok tok, Val val, bool mine, bool store, int tid, int slot, int nslot,
                                                  int64_t orow, int ks, int ksi, int T, int64_t ldy, float *part,
                                                  int32_t *cnt, float *Y, int *flag) {
    static_assert(NE % 4 == 0, "whole quads");
    constexpr int NQ = NE / 4, WF = NE * 64;  // quads per lane, floats per wavefront
    constexpr int SC1 = 16;                    // cache policy: agent-scope coherent (write-through / no L2 hit)
    const int lane = tid & 63;
    auto res = [&](int k) {
        return buf_res((const uint8_t *)(part + (((size_t)k * gridDim.x + blockIdx.x) * nslot + slot) * WF), WF * 4);
    };
    if (mine) {
        const BufRes r = res(ksi);
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const uint4 v = make_uint4(__float_as_uint(val(4 * q)), __float_as_uint(val(4 * q + 1)),
                                       __float_as_uint(val(4 * q + 2)), __float_as_uint(val(4 * q + 3)));
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(fgh_u32x4, v), r, 16 * (64 * q + lane), 0, SC1);
        }
    }
    __builtin_amdgcn_s_waitcnt(0xF70);  // vmcnt 0: this wavefront's partial stores have completed
    __syncthreads();
    if (tid == 0)
        *flag = __hip_atomic_fetch_add(&cnt[blockIdx.x], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == ks - 1;
    __syncthreads();
    if (!*flag || !mine) return;
    float pv[4][NE];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        if (k < ks && k != ksi) {  // uniform
            const BufRes r = res(k);
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
                const fgh_u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(r, 16 * (64 * q + lane), 0, SC1);
#pragma unroll
                for (int c = 0; c < 4; ++c) pv[k][4 * q + c] = __uint_as_float(w[c]);
            }
        } else {
#pragma unroll
            for (int e = 0; e < NE; ++e) pv[k][e] = 0.0f;
        }
    }
    if (!store) return;
#pragma unroll
    for (int e = 0; e < NE; ++e) {
        if (tok(e) < T) {
            float v = ksi == 0 ? val(e) : pv[0][e];
#pragma unroll
            for (int k = 1; k < 4; ++k)
                if (k < ks) v += ksi == k ? val(e) : pv[k][e];
            Y[(size_t)tok(e) * ldy + orow] = v;
        }
    }
}
constexpr size_t GEMM_LDS_MAX = 163840;  // gfx950: 160 KiB of LDS per workgroup
// The prompt GEMMs' activation records go straight from memory into one of GEMM_NST LDS stages
// (buffer loads to LDS: no registers, no LDS writes of their own), three steps ahead: round k of
// thread t copies 16-byte unit k * NTH + t of the step's records (each wavefront load reads and
// writes 1 KB contiguous, 16 bytes per lane); reads past src's range return 0.
constexpr int GEMM_NST = 4;
typedef __attribute__((address_space(3))) void *LdsPtr;
template <int R, int NTH>
__device__ __forceinline__ void gemm_dma(BufRes src, uint8_t *st, int wave, int tid) {
#pragma unroll
    for (int k = 0; k < R; ++k)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(src, (LdsPtr)(st + (size_t)(k * NTH + 64 * wave) * 16), 16,
                                                 16 * (k * NTH + tid), 0, 0, 0);
}
// The end of a GEMM step: this wavefront's loads into the next step's stage have landed (the N
// loads issued after them may still be in flight) and its LDS reads are done; then the
// workgroup's barrier. No fence: a workgroup fence would wait for every load in flight, the
// ring's weights and the later stages' records included.
template <int N>
__device__ __forceinline__ void gemm_stage_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));  // vmcnt(N) expcnt(7) lgkmcnt(0)
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}
// true when all wg workgroups of a launch (waves wavefronts and lds bytes each) can be resident
// on num_cu CUs at once: a split launch whose workgroups need a second round is slower than a
// smaller split (measured: Q8_0 4096 x 14336 with 4-way splits in two rounds 26 us, 2-way 18 us)
inline bool all_resident(int64_t wg, int waves, size_t lds, int num_cu) {
    const int64_t by_lds = lds ? (int64_t)(GEMM_LDS_MAX / lds) : 64, by_waves = 32 / waves;
    return wg <= (int64_t)num_cu * (by_lds < by_waves ? by_lds : by_waves);
}
hipError_t launch_q4k_gemm(const GemmArgs &a, hipStream_t s);

}  // namespace fgh
