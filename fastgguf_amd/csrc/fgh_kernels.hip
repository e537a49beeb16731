// fgh_kernels.hip - gfx950 kernels around the hot path: stand-alone activation quantizers
// (bit-exact with the reference's quantize_q8 / quantize_q8k; used by the prompt GEMM and the
// quantizer test hook), the upload-time weight re-layout, and the fp16 decode test hook.
#include "fgh_internal.h"

namespace fgh {

// =============================================================================================
// Activation quantizers
// =============================================================================================

// wave-wide max of a non-negative float (exact: max is order-independent)
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// (int)lrintf(v) as the reference computes it on x86 (fastgguf.c:762, 786): round half to even;
// a NaN or infinite v (id = 1/d overflows when amax is subnormal) gives the "integer indefinite"
// value, whose low bits are 0. A finite id keeps |v| <= 127, so no other case arises.
__device__ __forceinline__ int q_round(float v) {
    return fabsf(v) < 2147483648.0f ? (int)rintf(v) : 0;
}

__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xFF) | ((uint32_t)(b & 0xFF) << 8) | ((uint32_t)(c & 0xFF) << 16) |
           ((uint32_t)(d & 0xFF) << 24);
}

// quantize_q8k (fastgguf.c:773-793): one wavefront per 256-value block; lane l holds values
// 4l..4l+3. d = amax/127 and id = 1/d are IEEE divisions, q = round-half-even(x*id).
__global__ __launch_bounds__(256) void quant_q8k_kernel(const float *__restrict__ x, int64_t ldx, int nb,
                                                        ActQ8K act) {
    const int lane = threadIdx.x & 63;
    const int b = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int tok = blockIdx.y;
    if (b >= nb) return;  // whole wavefront leaves together
    const float4 v = *(const float4 *)(x + (size_t)tok * ldx + (size_t)b * 256 + 4 * lane);
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = wave_max(amax);
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    const int q0 = q_round(v.x * id), q1 = q_round(v.y * id);
    const int q2 = q_round(v.z * id), q3 = q_round(v.w * id);
    const size_t blk = (size_t)tok * nb + b;
    // element 4l = 32c + 4i (c = l/8, i = l%8) goes to position 32i + 4c
    *(uint32_t *)(act.qs + blk * 256 + 32 * (lane & 7) + 4 * (lane >> 3)) = pack4(q0, q1, q2, q3);
    const int s = sum4_i32(q0 + q1 + q2 + q3);  // 16 values = 4 lanes
    if ((lane & 3) == 0) act.bs[blk * 16 + (lane >> 2)] = (int16_t)s;
    if (lane == 0) act.d[blk] = d;
}

// quantize_q8 (fastgguf.c:746-768): 8 lanes per 32-value block, 8 blocks per wavefront
__global__ __launch_bounds__(256) void quant_q8_kernel(const float *__restrict__ x, int64_t ldx, int nb,
                                                       ActQ8 act) {
    const int lane = threadIdx.x & 63, sub = lane & 7;
    const int b = blockIdx.x * 32 + (threadIdx.x >> 3);
    const int tok = blockIdx.y;
    const bool live = b < nb;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (live) v = *(const float4 *)(x + (size_t)tok * ldx + (size_t)b * 32 + 4 * sub);
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    const int q0 = q_round(v.x * id), q1 = q_round(v.y * id);
    const int q2 = q_round(v.z * id), q3 = q_round(v.w * id);
    const int s = sum4_i32(q0 + q1 + q2 + q3);  // lanes 0-3: values 0..15, lanes 4-7: 16..31
    if (live) {
        const size_t blk = (size_t)tok * nb + b;
        *(uint32_t *)(act.qs + blk * 32 + 4 * sub) = pack4(q0, q1, q2, q3);
        if ((sub & 3) == 0) act.s16[blk * 2 + (sub >> 2)] = (int16_t)s;
        if (sub == 0) act.d[blk] = d;
    }
}

// =============================================================================================
// Upload-time re-layout of Q6_K / Q8_0 / the nibble types: file-layout rows (n_mats x rows x row_bytes) -> tiles in
// step-major order, step tb of row tile gl of matrix m at (m * ntile + tb) * gpm + gl (Q4_K has its
// own, fgh_q4k.hip). One thread per destination byte; padding rows and padding blocks are zero.
// =============================================================================================
__global__ void relayout_kernel(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, int type,
                                int64_t rows, int nb, int ntile, int64_t gpm, int64_t total, int64_t row_bytes) {
    const int tile_bytes = type == T_Q6_K ? Q6K_TILE : Q80_TILE;
    for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < total;
         o += (int64_t)gridDim.x * blockDim.x) {
        const int64_t t = o / tile_bytes;  // = (m * ntile + tb) * gpm + gl
        const int ob = (int)(o - t * tile_bytes);
        const int64_t mt = t / gpm, gl = t - mt * gpm;
        const int64_t m = mt / ntile;
        const int tb = (int)(mt - m * ntile);
        int r, blk, byte;  // source row in group, block in row, byte in block
        if (type == T_Q6_K) {
            blk = tb;
            if (ob < 128) {
                r = ob >> 4;
                byte = 192 + (ob & 15);
            } else if (ob < 144) {
                r = (ob - 128) >> 1;
                byte = 208 + ((ob - 128) & 1);
            } else if (ob < 1168) {
                const int q = ob - 144, lane = q >> 4, w = (q & 15) >> 2, k = q & 3, i = lane & 7;
                r = lane >> 3;
                byte = 64 * (w >> 1) + 32 * (w & 1) + 4 * i + k;
            } else {
                const int q = ob - 1168, lane = q >> 3, h = (q & 7) >> 2, k = q & 3, i = lane & 7;
                r = lane >> 3;
                byte = 128 + 32 * h + 4 * i + k;
            }
        } else {  // Q8_0: tile of 4 blocks
            if (ob < 64) {
                r = ob >> 3;
                blk = 4 * tb + ((ob & 7) >> 1);
                byte = ob & 1;
            } else {
                const int q = ob - 64, lane = q >> 4, bb = (q & 15) >> 2, k = q & 3, i = lane & 7;
                r = lane >> 3;
                blk = 4 * tb + bb;
                byte = 2 + 4 * i + k;
            }
        }
        const int64_t row = gl * 8 + r;
        const int bb = type == T_Q8_0 ? 34 : 210;
        uint8_t v = 0;
        if (row < rows && blk < nb) v = src[(m * rows + row) * row_bytes + (int64_t)blk * bb + byte];
        dst[o] = v;
    }
}

// The nibble types (tile of 4 blocks: Q5_0 704 B, Q4_0 / IQ4_NL 576 B, Q4_1 640 B, Q5_1 768 B,
// regions at q32_layout's offsets, fgh_internal.h): one thread per destination byte, gathering the
// nibbles and fifth bits it packs from the file's blocks (Q4_0 / IQ4_NL {d, qs[16]}, Q4_1 {d, m,
// qs}, Q5_0 {d, qh, qs}, Q5_1 {d, m, qh, qs}; fastgguf.c:485-550, 694-706); element e of a block
// is nibble e of qs (low nibbles of qs[0..15], then their high nibbles) with bit e of qh above it
// (nibbles32 809-814, q5_elem 939-942)
struct Q32Src {
    int bytes, qs, qh;  // block bytes, offsets of qs and qh (-1: none)
};
__device__ __forceinline__ Q32Src q32_src(int type) {
    switch (type) {
    case T_Q5_0: return {22, 6, 2};
    case T_Q4_1: return {20, 4, -1};
    case T_Q5_1: return {24, 8, 4};
    default: return {18, 2, -1};  // Q4_0, IQ4_NL
    }
}
__global__ void relayout_q32_kernel(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, int type, int64_t rows,
                                    int nb, int ntile, int64_t gpm, int64_t total, int64_t row_bytes) {
    const Q32Layout L = q32_layout(type);
    const Q32Src B = q32_src(type);
    for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < total;
         o += (int64_t)gridDim.x * blockDim.x) {
        const int64_t t = o / L.tile;  // = (m * ntile + tb) * gpm + gl
        const int ob = (int)(o - t * L.tile);
        const int64_t mt = t / gpm, gl = t - mt * gpm;
        const int64_t m = mt / ntile;
        const int tb = (int)(mt - m * ntile);
        const bool in_sc = ob < 8 * L.ds;  // the scale records, L.ds bytes per row
        const int sj = ob % L.ds;          // byte of the row's record: d, then m from L.m
        const bool in_m = in_sc && L.m >= 0 && sj >= L.m;
        const bool in_h = L.h >= 0 && ob >= L.h;
        const int r = in_sc ? ob / L.ds : in_h ? (ob - L.h) >> 4 : (ob - L.n) >> 6;
        const int64_t row = gl * 8 + r;
        // block bb of the step in this row, or null past the row's end
        auto blk = [&](int bb) -> const uint8_t * {
            const int b = 4 * tb + bb;
            return row < rows && b < nb ? src + (m * rows + row) * row_bytes + (int64_t)b * B.bytes : nullptr;
        };
        auto nib = [&](const uint8_t *p, int e) { return e < 16 ? (p[B.qs + e] & 15) : (p[B.qs + e - 16] >> 4); };
        auto bit = [&](const uint8_t *p, int e) { return (p[B.qh + (e >> 3)] >> (e & 7)) & 1; };
        int v = 0;
        if (in_sc) {  // fp16 d (or m) of block (sj & 7) >> 1
            const uint8_t *p = blk((sj & 7) >> 1);
            v = p ? p[(in_m ? 2 : 0) + (sj & 1)] : 0;
        } else if (!in_h) {  // byte 4w + t of slice i: element 4i + t of blocks 2w (low), 2w + 1 (high)
            const int q = ob - L.n, i = (q >> 3) & 7, w = (q >> 2) & 1, e = 4 * i + (q & 3);
            const uint8_t *p0 = blk(2 * w), *p1 = blk(2 * w + 1);
            v = (p0 ? nib(p0, e) : 0) | (p1 ? nib(p1, e) << 4 : 0);
        } else {  // byte hb of slice i's fifth bits: nibbles n_hb (low) and n_hb+2 (high)
            const int q = ob - L.h, i = (q >> 1) & 7, hb = q & 1;
#pragma unroll
            for (int bb = 0; bb < 4; ++bb) {
                const uint8_t *p = blk(bb);
                if (p) v |= (bit(p, 4 * i + hb) << bb) | (bit(p, 4 * i + hb + 2) << (4 + bb));
            }
        }
        dst[o] = (uint8_t)v;
    }
}

__global__ void fp16_kernel(const uint16_t *__restrict__ h, float *__restrict__ out, int n) {
    const int k = blockIdx.x * blockDim.x + threadIdx.x;
    if (k < n) out[k] = fp16_bits_to_f32(h[k]);
}

// ---------------------------------------------------------------------------------------------
// host-side launchers (called from fgh_api.hip)
// ---------------------------------------------------------------------------------------------
hipError_t launch_quant_q8k(const float *x, int64_t ldx, int nb, int ntok, ActQ8K act, hipStream_t s) {
    dim3 grid((nb + 3) / 4, ntok);
    quant_q8k_kernel<<<grid, 256, 0, s>>>(x, ldx, nb, act);
    return hipGetLastError();
}

hipError_t launch_quant_q8(const float *x, int64_t ldx, int nb, int ntok, ActQ8 act, hipStream_t s) {
    dim3 grid((nb + 31) / 32, ntok);
    quant_q8_kernel<<<grid, 256, 0, s>>>(x, ldx, nb, act);
    return hipGetLastError();
}

hipError_t launch_relayout(const uint8_t *src, uint8_t *dst, int type, int64_t rows, int nb, int ntile,
                           int64_t gpm, int64_t total, int64_t row_bytes, hipStream_t s) {
    const int64_t want = (total + 255) / 256;
    const int grid = (int)(want < 65536 ? want : 65536);
    if (q8_kind(type) && type != T_Q8_0)
        relayout_q32_kernel<<<grid, 256, 0, s>>>(src, dst, type, rows, nb, ntile, gpm, total, row_bytes);
    else relayout_kernel<<<grid, 256, 0, s>>>(src, dst, type, rows, nb, ntile, gpm, total, row_bytes);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void copy16_kernel(const uint4 *__restrict__ src, uint4 *__restrict__ dst, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        dst[i] = src[i];
}

hipError_t launch_copy16(const void *src, void *dst, int64_t n16, hipStream_t s) {
    const int64_t want = (n16 + 255) / 256;
    copy16_kernel<<<(unsigned)(want < 8192 ? want : 8192), 256, 0, s>>>((const uint4 *)src, (uint4 *)dst, n16);
    return hipGetLastError();
}

// Wrapping 32-bit sum of the little-endian words of n16 16-byte units in two launches: the first
// gives each workgroup one contiguous share of the buffer, which its threads stream with U
// nontemporal 16-byte loads in flight each, and writes the share's sum; the second adds the parts
// (integer wrapping addition is associative: the result does not depend on the launch shape). The
// kernel boundary makes the parts visible across the XCDs. The shape is the fastest of a sweep on
// MI355X (workgroups per CU 8 / 16 / 32, loads in flight 4 / 8 / 16, grid-stride or contiguous
// shares, default or nontemporal loads, 66 MB to 1 GB rotating over 3 GB): contiguous shares with
// nontemporal loads, 32 workgroups per CU of 4 loads each below 128 MB (66 MB: 5.85 TB/s against
// 5.10 for the grid-stride form), 16 of 8 loads above (1 GB: 6.98 TB/s against 5.13); hipMemcpyAsync
// moves 4.9-5.4 TB/s (read plus write) in the same sweep.
__device__ __forceinline__ uint32_t wg_sum256(uint32_t v, uint32_t *red) {
    v += __shfl_xor(v, 32);
    v += __shfl_xor(v, 16);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xF, 0xF, false);  // row_ror 8, 4, 2, 1
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x124, 0xF, 0xF, false);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x122, 0xF, 0xF, false);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x121, 0xF, 0xF, false);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}
typedef unsigned ck_u32x4 __attribute__((ext_vector_type(4)));
template <int U>
__global__ __launch_bounds__(256) void checksum_part_kernel(const uint4 *__restrict__ src, int64_t n16,
                                                            uint32_t *__restrict__ part) {
    __shared__ uint32_t red[4];
    const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const int64_t lo = min((int64_t)blockIdx.x * per, n16), hi = min(lo + per, n16);
    const ck_u32x4 *p = (const ck_u32x4 *)src;
    int64_t i = lo + threadIdx.x;
    uint32_t sum = 0;
    for (; i + (U - 1) * 256 < hi; i += U * 256) {
        ck_u32x4 a[U];
#pragma unroll
        for (int u = 0; u < U; ++u) a[u] = __builtin_nontemporal_load(p + i + u * 256);
#pragma unroll
        for (int u = 0; u < U; ++u) sum += (a[u][0] + a[u][1]) + (a[u][2] + a[u][3]);
    }
    for (; i < hi; i += 256) {
        const ck_u32x4 a = __builtin_nontemporal_load(p + i);
        sum += (a[0] + a[1]) + (a[2] + a[3]);
    }
    const uint32_t ws = wg_sum256(sum, red);
    if (threadIdx.x == 0) part[blockIdx.x] = ws;
}
__global__ __launch_bounds__(256) void checksum_final_kernel(const uint32_t *__restrict__ part, int n,
                                                             uint32_t *__restrict__ out) {
    __shared__ uint32_t red[4];
    uint32_t v = 0;
    for (int k = threadIdx.x; k < n; k += blockDim.x) v += part[k];
    const uint32_t total = wg_sum256(v, red);
    if (threadIdx.x == 0) *out = total;
}
int checksum_parts(int num_cu) { return 32 * num_cu; }  // the most workgroups a launch uses
// out == nullptr: the streaming part only
hipError_t launch_checksum(const void *src, int64_t n16, uint32_t *part, int num_cu, uint32_t *out, hipStream_t s) {
    const bool small = n16 * 16 < ((int64_t)128 << 20);
    const int np = small ? 32 * num_cu : 16 * num_cu;
    if (small) checksum_part_kernel<4><<<np, 256, 0, s>>>((const uint4 *)src, n16, part);
    else checksum_part_kernel<8><<<np, 256, 0, s>>>((const uint4 *)src, n16, part);
    if (out) checksum_final_kernel<<<1, 256, 0, s>>>(part, np, out);
    return hipGetLastError();
}

// The int8 MFMA rate the box delivers to a kernel that does nothing else: every wavefront runs
// `iters` rounds of 8 independent v_mfma_i32_16x16x64_i8 chains (operands in registers, no memory
// traffic); a result reaches memory only if its sum equals `magic`, so none of the work can be
// dropped. Two workgroups of 4 wavefronts per compute unit.
typedef int v4i_t __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void mfma_peak_kernel(int iters, uint32_t magic, uint32_t *__restrict__ sink) {
    const int t = threadIdx.x;
    v4i_t a = {t, t + 1, t + 2, (int)magic}, b = {3 * t, 1, 2, 3};
    v4i_t c[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j] = v4i_t{0, 0, 0, 0};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; ++j) c[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c[j], 0, 0, 0);
        a.x += it;
    }
    uint32_t sum = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) sum += (uint32_t)(c[j][0] + c[j][1] + c[j][2] + c[j][3]);
    if (sum == magic) sink[blockIdx.x] = sum;
}
int mfma_peak_blocks(int num_cu) { return 2 * num_cu; }
uint64_t mfma_peak_ops(int num_cu, int iters) {
    return (uint64_t)mfma_peak_blocks(num_cu) * 4 * (uint64_t)iters * 8 * (2 * 16 * 16 * 64);
}
hipError_t launch_mfma_peak(int iters, uint32_t *sink, int num_cu, hipStream_t s) {
    mfma_peak_kernel<<<mfma_peak_blocks(num_cu), 256, 0, s>>>(iters, 0x9E3779B9u, sink);
    return hipGetLastError();
}

hipError_t launch_fp16(const uint16_t *h, float *out, int n, hipStream_t s) {
    fp16_kernel<<<(n + 255) / 256, 256, 0, s>>>(h, out, n);
    return hipGetLastError();
}

}  // namespace fgh
