// fgh_kernels.hip - gfx950 kernels of the decode path: activation quantizers (bit-exact with the
// reference's quantize_q8 / quantize_q8k), the upload-time weight re-layout, and the Q4_K / Q6_K /
// Q8_0 decode matvecs.
//
// Matvec structure (all three types): a workgroup of 4 wavefronts owns one group of 8 rows.
// Blocks are processed in chunks; in the integer phase each wavefront takes some blocks of the
// chunk and its 64 lanes (8 rows x 8 slices) compute the exact integer partials of the
// reference's fp32 accumulator lanes with v_dot4_i32_i8, from 16-byte coalesced weight loads;
// the partials (converted to fp32, which is exact) go to LDS. In the chain phase a few lanes walk
// the chunk's blocks in ascending order applying exactly the fused multiply-adds of the reference
// kernel, so the fp32 output is bit-identical to it. Weight bytes stream from HBM once; the
// chain costs a few fma per block per row.
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
    const int q0 = (int)rintf(v.x * id), q1 = (int)rintf(v.y * id);
    const int q2 = (int)rintf(v.z * id), q3 = (int)rintf(v.w * id);
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
    const int q0 = (int)rintf(v.x * id), q1 = (int)rintf(v.y * id);
    const int q2 = (int)rintf(v.z * id), q3 = (int)rintf(v.w * id);
    const int s = sum4_i32(q0 + q1 + q2 + q3);  // lanes 0-3: values 0..15, lanes 4-7: 16..31
    if (live) {
        const size_t blk = (size_t)tok * nb + b;
        *(uint32_t *)(act.qs + blk * 32 + 4 * sub) = pack4(q0, q1, q2, q3);
        if ((sub & 3) == 0) act.s16[blk * 2 + (sub >> 2)] = (int16_t)s;
        if (sub == 0) act.d[blk] = d;
    }
}

// =============================================================================================
// Upload-time re-layout: file-layout rows (n_mats x rows x row_bytes) -> tiles. One thread per
// destination byte; padding rows and padding blocks are zero.
// =============================================================================================
__global__ void relayout_kernel(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, int type,
                                int64_t rows, int nb, int ntile, int64_t gpm, int64_t total, int64_t row_bytes) {
    const int tile_bytes = type == T_Q4_K ? Q4K_TILE : type == T_Q6_K ? Q6K_TILE : Q80_TILE;
    for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < total;
         o += (int64_t)gridDim.x * blockDim.x) {
        const int64_t t = o / tile_bytes;
        const int ob = (int)(o - t * tile_bytes);
        const int64_t g = t / ntile;
        const int tb = (int)(t - g * ntile);
        const int64_t m = g / gpm, gl = g - m * gpm;
        int r, blk, byte;  // source row in group, block in row, byte in block
        if (type == T_Q4_K) {
            blk = tb;
            if (ob < 128) {
                r = ob >> 4;
                byte = ob & 15;
            } else {
                const int q = ob - 128, i = (q & 127) >> 4, j = (q & 15) >> 2, k = q & 3;
                r = q >> 7;
                byte = 16 + 32 * j + 4 * i + k;
            }
        } else if (type == T_Q6_K) {
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
        const int bb = type == T_Q8_0 ? 34 : type == T_Q4_K ? 144 : 210;
        uint8_t v = 0;
        if (row < rows && blk < nb) v = src[(m * rows + row) * row_bytes + (int64_t)blk * bb + byte];
        dst[o] = v;
    }
}

// =============================================================================================
// Decode matvecs. Grid: x = row group (n_mats * groups per matrix), y = token. 256 threads.
// Output row of group g, row r: m * rows + gl * 8 + r with g = m * gpm + gl.
// dump_s / dump_m (DUMP variants only) receive the per (row, block) integer parts.
// =============================================================================================


// ---- Q4_K, repacked order: dot_q4Kx8 (fastgguf.c:2322-2358) --------------------------------
// per block: sumi = sum_s sc_s * sum_32 q*y, msum = sum_s m_s * (bs_2s + bs_2s+1) (exact ints);
// acc = fma(FP16(d)*yd, sumi, acc), macc = fma(FP16(dmin)*yd, msum, macc) over blocks in order;
// out = acc - macc.
template <int BPW, bool DUMP>
__global__ __launch_bounds__(256) void mv_q4k_rp_kernel(const uint8_t *__restrict__ W, int nb, ActQ8K act,
                                                        MvOut out) {
    constexpr int CB = 4 * BPW;
    __shared__ float4 part[CB][8];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, r = lane >> 3, i = lane & 7;
    const int64_t g = blockIdx.x;
    const int tok = blockIdx.y;
    const uint8_t *Wg = W + (size_t)g * nb * Q4K_TILE;
    const size_t a0 = (size_t)tok * nb;
    float acc = 0.0f, macc = 0.0f;
    bool ok;
    const int64_t orow = out.row_of(g, r, ok);
    for (int c0 = 0; c0 < nb; c0 += CB) {
        uint4 q[BPW], m[BPW], ya[BPW], yb[BPW];
        uint32_t bsp[BPW];
#pragma unroll
        for (int k = 0; k < BPW; ++k) {
            const int b = c0 + wave * BPW + k;
            if (b < nb) {
                const uint8_t *t = Wg + (size_t)b * Q4K_TILE;
                q[k] = ld16(t + 128 + 16 * lane);
                m[k] = ld16(t + 16 * r);
                const uint8_t *ap = (const uint8_t *)act.qs + (a0 + b) * 256 + 32 * i;
                ya[k] = ld16(ap);
                yb[k] = ld16(ap + 16);
                bsp[k] = *(const uint32_t *)(act.bs + (a0 + b) * 16 + 2 * i);
            }
        }
#pragma unroll
        for (int k = 0; k < BPW; ++k) {
            const int b = c0 + wave * BPW + k;
            if (b < nb) {
                const Q4KScales s = q4k_scales(m[k].y, m[k].z, m[k].w);
                const uint32_t qw[4] = {q[k].x, q[k].y, q[k].z, q[k].w};
                const int yv[8] = {(int)ya[k].x, (int)ya[k].y, (int)ya[k].z, (int)ya[k].w,
                                   (int)yb[k].x, (int)yb[k].y, (int)yb[k].z, (int)yb[k].w};
                int sum = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int lo = (int)(qw[j] & 0x0F0F0F0Fu), hi = (int)((qw[j] >> 4) & 0x0F0F0F0Fu);
                    sum += q4k_sc(s, 2 * j) * dot4(lo, yv[2 * j], 0) + q4k_sc(s, 2 * j + 1) * dot4(hi, yv[2 * j + 1], 0);
                }
                const int bs2 = (int)(int16_t)(bsp[k] & 0xFFFF) + (int)(int16_t)(bsp[k] >> 16);
                const int mterm = ubyte(i < 4 ? s.mn_lo : s.mn_hi, i & 3) * bs2;
                const int sumi = sum8_i32(sum), msum = sum8_i32(mterm);
                if (i == 0) {
                    const float yd = act.d[a0 + b];
                    const float d = fp16_bits_to_f32(m[k].x & 0xFFFF), dm = fp16_bits_to_f32(m[k].x >> 16);
                    part[b - c0][r] = make_float4(d * yd, (float)sumi, dm * yd, (float)msum);
                    if (DUMP && ok) {
                        out.dump_s[orow * nb + b] = sumi;
                        out.dump_m[orow * nb + b] = msum;
                    }
                }
            }
        }
        __syncthreads();
        if (tid < 8) {
            const int nc = min(CB, nb - c0);
            for (int bb = 0; bb < nc; ++bb) {
                const float4 p = part[bb][tid];
                acc = __builtin_fmaf(p.x, p.y, acc);
                macc = __builtin_fmaf(p.z, p.w, macc);
            }
        }
        __syncthreads();
    }
    if (tid < 8) {
        const int64_t row = out.row_of(g, tid, ok);
        if (ok) out.y[(size_t)tok * out.ldy + row] = acc - macc;
    }
}

// ---- Q4_K, file-layout order: dot_q4_K_q8k (fastgguf.c:1118-1153) --------------------------
// lane i: sum_j sc_2j * dot(lo bytes 4i.., y) + sc_2j+1 * dot(hi bytes 4i.., y); acc_i =
// fma(FP16(d)*yd, lane_i, acc_i); min lane p: m_2p (bs_4p+bs_4p+1) + m_2p+1 (bs_4p+2+bs_4p+3),
// macc_p = fma(FP16(dmin)*yd, ., macc_p); out = hsum8(acc) - hsum4(macc).
// ---- Q6_K: dot_q6_K_q8k (fastgguf.c:1232-1264) -------------------------------------------
// lane i: sum_{h,k} sc[8h+2k+(i>=4)] * dot(q(128h+32k+4i..), y); acc_i = fma(dd, lane_i, acc_i);
// correction lane p: (sc_2p bs_2p + sc_2p+1 bs_2p+1) + (sc_2p+8 bs_2p+8 + sc_2p+9 bs_2p+9),
// cacc_p = fma(32 dd, ., cacc_p); out = hsum8(acc) - hsum4(cacc).
// Both are "8 lane chains + 4 min chains"; one kernel body, the integer phase per type.
template <int TYPE, int BPW, bool DUMP>
__global__ __launch_bounds__(256) void mv_lanes_kernel(const uint8_t *__restrict__ W, int nb, ActQ8K act,
                                                       MvOut out) {
    constexpr int CB = 4 * BPW;
    constexpr int TILE = TYPE == T_Q4_K ? Q4K_TILE : Q6K_TILE;
    __shared__ float lanev[CB][8][8];
    __shared__ float minv[CB][8][4];
    __shared__ float2 dyv[CB][8];
    __shared__ float fin[8][12];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, r = lane >> 3, i = lane & 7;
    const int64_t g = blockIdx.x;
    const int tok = blockIdx.y;
    const uint8_t *Wg = W + (size_t)g * nb * TILE;
    const size_t a0 = (size_t)tok * nb;
    float acc = 0.0f, macc = 0.0f;  // chain lanes: tid < 64 -> (row tid/8, lane tid%8)
    bool ok;
    const int64_t orow = out.row_of(g, r, ok);
    for (int c0 = 0; c0 < nb; c0 += CB) {
        uint4 q[BPW], m[BPW], ya[BPW], yb[BPW];
        uint2 qh[BPW], bsv[BPW];
        uint32_t dbits[BPW];
#pragma unroll
        for (int k = 0; k < BPW; ++k) {
            const int b = c0 + wave * BPW + k;
            if (b < nb) {
                const uint8_t *t = Wg + (size_t)b * TILE;
                if (TYPE == T_Q4_K) {
                    q[k] = ld16(t + 128 + 16 * lane);
                    m[k] = ld16(t + 16 * r);
                    bsv[k] = ld8((const uint8_t *)(act.bs + (a0 + b) * 16 + 4 * (i & 3)));
                } else {
                    q[k] = ld16(t + 144 + 16 * lane);
                    qh[k] = ld8(t + 1168 + 8 * lane);
                    m[k] = ld16(t + 16 * r);
                    dbits[k] = *(const uint16_t *)(t + 128 + 2 * r);
                    // correction lane p = i & 3 needs bs[2p], bs[2p+1], bs[2p+8], bs[2p+9]
                    const uint32_t *bp = (const uint32_t *)(act.bs + (a0 + b) * 16);
                    bsv[k] = make_uint2(bp[i & 3], bp[(i & 3) + 4]);
                }
                const uint8_t *ap = (const uint8_t *)act.qs + (a0 + b) * 256 + 32 * i;
                ya[k] = ld16(ap);
                yb[k] = ld16(ap + 16);
            }
        }
#pragma unroll
        for (int k = 0; k < BPW; ++k) {
            const int b = c0 + wave * BPW + k;
            if (b < nb) {
                const int yv[8] = {(int)ya[k].x, (int)ya[k].y, (int)ya[k].z, (int)ya[k].w,
                                   (int)yb[k].x, (int)yb[k].y, (int)yb[k].z, (int)yb[k].w};
                int sum = 0, mterm = 0;
                float fd, fdm;
                if (TYPE == T_Q4_K) {
                    const Q4KScales s = q4k_scales(m[k].y, m[k].z, m[k].w);
                    const uint32_t qw[4] = {q[k].x, q[k].y, q[k].z, q[k].w};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int lo = (int)(qw[j] & 0x0F0F0F0Fu), hi = (int)((qw[j] >> 4) & 0x0F0F0F0Fu);
                        sum += q4k_sc(s, 2 * j) * dot4(lo, yv[2 * j], 0) +
                               q4k_sc(s, 2 * j + 1) * dot4(hi, yv[2 * j + 1], 0);
                    }
                    const int p = i & 3;
                    const int bs_lo = (int)(int16_t)(bsv[k].x & 0xFFFF) + (int)(int16_t)(bsv[k].x >> 16);
                    const int bs_hi = (int)(int16_t)(bsv[k].y & 0xFFFF) + (int)(int16_t)(bsv[k].y >> 16);
                    const uint32_t mw = p < 2 ? s.mn_lo : s.mn_hi;
                    mterm = ubyte(mw, 2 * (p & 1)) * bs_lo + ubyte(mw, 2 * (p & 1) + 1) * bs_hi;
                    const float yd = act.d[a0 + b];
                    fd = fp16_bits_to_f32(m[k].x & 0xFFFF) * yd;
                    fdm = fp16_bits_to_f32(m[k].x >> 16) * yd;
                } else {
                    const uint32_t sw[4] = {m[k].x, m[k].y, m[k].z, m[k].w};  // int8 scales 0..15
                    const uint32_t A[4] = {q[k].x, q[k].y, q[k].z, q[k].w};
                    const uint32_t H[2] = {qh[k].x, qh[k].y};
                    const int hi4 = i >= 4;
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const uint32_t A0 = A[2 * h], A1 = A[2 * h + 1], Hh = H[h];
                        const uint32_t M4 = 0x0F0F0F0Fu, M2 = 0x03030303u;
                        const uint32_t qv[4] = {(A0 & M4) | ((Hh & M2) << 4),
                                                (A1 & M4) | (((Hh >> 2) & M2) << 4),
                                                ((A0 >> 4) & M4) | (((Hh >> 4) & M2) << 4),
                                                ((A1 >> 4) & M4) | (((Hh >> 6) & M2) << 4)};
#pragma unroll
                        for (int kk = 0; kk < 4; ++kk) {
                            const int si = 8 * h + 2 * kk + hi4;  // scale index, 0..15
                            sum += sbyte(sw[si >> 2], si & 3) * dot4((int)qv[kk], yv[4 * h + kk], 0);
                        }
                    }
                    const int p = i & 3;
                    const int s0 = sbyte(sw[(2 * p) >> 2], (2 * p) & 3), s1 = sbyte(sw[(2 * p + 1) >> 2], (2 * p + 1) & 3);
                    const int s8 = sbyte(sw[(2 * p + 8) >> 2], (2 * p + 8) & 3), s9 = sbyte(sw[(2 * p + 9) >> 2], (2 * p + 9) & 3);
                    const int b0 = (int)(int16_t)(bsv[k].x & 0xFFFF), b1 = (int)(int16_t)(bsv[k].x >> 16);
                    const int b8 = (int)(int16_t)(bsv[k].y & 0xFFFF), b9 = (int)(int16_t)(bsv[k].y >> 16);
                    mterm = (s0 * b0 + s1 * b1) + (s8 * b8 + s9 * b9);
                    fd = fp16_bits_to_f32(dbits[k]) * act.d[a0 + b];
                    fdm = fd * 32.0f;
                }
                lanev[b - c0][r][i] = (float)sum;
                if (i < 4) minv[b - c0][r][i] = (float)mterm;
                if (i == 0) dyv[b - c0][r] = make_float2(fd, fdm);
                if (DUMP) {
                    const int ts = sum8_i32(sum), tm = sum4_i32(mterm);  // lanes 0-3 hold the 4 min lanes
                    if (i == 0 && ok) {
                        out.dump_s[orow * nb + b] = ts;
                        out.dump_m[orow * nb + b] = tm;
                    }
                }
            }
        }
        __syncthreads();
        if (tid < 64) {
            const int cr = tid >> 3, ci = tid & 7;
            const int nc = min(CB, nb - c0);
            for (int bb = 0; bb < nc; ++bb) {
                const float2 dv = dyv[bb][cr];
                acc = __builtin_fmaf(dv.x, lanev[bb][cr][ci], acc);
                if (ci < 4) macc = __builtin_fmaf(dv.y, minv[bb][cr][ci], macc);
            }
        }
        __syncthreads();
    }
    if (tid < 64) {
        fin[tid >> 3][tid & 7] = acc;
        if ((tid & 7) < 4) fin[tid >> 3][8 + (tid & 7)] = macc;
    }
    __syncthreads();
    if (tid < 8) {
        const float *v = fin[tid];
        const float h8 = ((v[0] + v[4]) + (v[1] + v[5])) + ((v[2] + v[6]) + (v[3] + v[7]));
        const float h4 = (v[8] + v[9]) + (v[10] + v[11]);
        const int64_t row = out.row_of(g, tid, ok);
        if (ok) out.y[(size_t)tok * out.ldy + row] = h8 - h4;
    }
}

// ---- Q8_0: dot_q8_0_q8 (fastgguf.c:891-902) ------------------------------------------------
// lane i of block b: s_i = sum_{t=4i}^{4i+3} w_t x_t; acc_i = fma(FP16(d)*xd, s_i, acc_i);
// out = hsum8(acc). Tiles hold 4 blocks; a chunk is 4 wavefronts x BPW tiles.
template <int BPW, bool DUMP>
__global__ __launch_bounds__(256) void mv_q80_kernel(const uint8_t *__restrict__ W, int nb, int ntile, ActQ8 act,
                                                     MvOut out) {
    constexpr int CT = 4 * BPW;  // tiles per chunk
    constexpr int CBK = 4 * CT;  // blocks per chunk
    __shared__ float lanev[CBK][8][8];
    __shared__ float dyv[CBK][8];
    __shared__ float fin[8][8];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, r = lane >> 3, i = lane & 7;
    const int64_t g = blockIdx.x;
    const int tok = blockIdx.y;
    const uint8_t *Wg = W + (size_t)g * ntile * Q80_TILE;
    const size_t a0 = (size_t)tok * nb;
    float acc = 0.0f;
    bool ok;
    const int64_t orow = out.row_of(g, r, ok);
    for (int t0 = 0; t0 < ntile; t0 += CT) {
        uint4 q[BPW];
        uint2 dw[BPW];
        uint32_t yv[BPW][4];
        float xd[BPW][4];
#pragma unroll
        for (int k = 0; k < BPW; ++k) {
            const int tb = t0 + wave * BPW + k;
            if (tb < ntile) {
                const uint8_t *t = Wg + (size_t)tb * Q80_TILE;
                q[k] = ld16(t + 64 + 16 * lane);
                dw[k] = ld8(t + 8 * r);
#pragma unroll
                for (int bb = 0; bb < 4; ++bb) {
                    const int b = 4 * tb + bb;
                    yv[k][bb] = b < nb ? *(const uint32_t *)(act.qs + (a0 + b) * 32 + 4 * i) : 0u;
                    xd[k][bb] = b < nb ? act.d[a0 + b] : 0.0f;
                }
            }
        }
#pragma unroll
        for (int k = 0; k < BPW; ++k) {
            const int tb = t0 + wave * BPW + k;
            if (tb < ntile) {
                const uint32_t qw[4] = {q[k].x, q[k].y, q[k].z, q[k].w};
                const uint32_t dd[4] = {dw[k].x & 0xFFFF, dw[k].x >> 16, dw[k].y & 0xFFFF, dw[k].y >> 16};
#pragma unroll
                for (int bb = 0; bb < 4; ++bb) {
                    const int b = 4 * tb + bb;
                    if (b < nb) {
                        const int s = dot4((int)qw[bb], (int)yv[k][bb], 0);
                        const int lb = b - 4 * t0;
                        lanev[lb][r][i] = (float)s;
                        if (i == 0) dyv[lb][r] = fp16_bits_to_f32(dd[bb]) * xd[k][bb];
                        if (DUMP) {
                            const int ts = sum8_i32(s);
                            if (i == 0 && ok) {
                                out.dump_s[orow * nb + b] = ts;
                                out.dump_m[orow * nb + b] = 0;
                            }
                        }
                    }
                }
            }
        }
        __syncthreads();
        if (tid < 64) {
            const int cr = tid >> 3, ci = tid & 7;
            const int nc = min(CBK, nb - 4 * t0);
            for (int bb = 0; bb < nc; ++bb) acc = __builtin_fmaf(dyv[bb][cr], lanev[bb][cr][ci], acc);
        }
        __syncthreads();
    }
    if (tid < 64) fin[tid >> 3][tid & 7] = acc;
    __syncthreads();
    if (tid < 8) {
        const float *v = fin[tid];
        const int64_t row = out.row_of(g, tid, ok);
        if (ok) out.y[(size_t)tok * out.ldy + row] = ((v[0] + v[4]) + (v[1] + v[5])) + ((v[2] + v[6]) + (v[3] + v[7]));
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
    relayout_kernel<<<grid, 256, 0, s>>>(src, dst, type, rows, nb, ntile, gpm, total, row_bytes);
    return hipGetLastError();
}

hipError_t launch_fp16(const uint16_t *h, float *out, int n, hipStream_t s) {
    fp16_kernel<<<(n + 255) / 256, 256, 0, s>>>(h, out, n);
    return hipGetLastError();
}

// groups: row groups over all matrices; ntok: tokens (grid.y); order only for Q4_K
hipError_t launch_matvec(int type, int order, const uint8_t *W, int nb, int64_t groups, int ntok,
                         const void *act, MvOut out, bool dump, hipStream_t s) {
    dim3 grid((unsigned)groups, ntok);
    if (type == T_Q4_K) {
        const ActQ8K a = *(const ActQ8K *)act;
        if (order == 1) {
            if (dump) mv_q4k_rp_kernel<4, true><<<grid, 256, 0, s>>>(W, nb, a, out);
            else mv_q4k_rp_kernel<4, false><<<grid, 256, 0, s>>>(W, nb, a, out);
        } else {
            if (dump) mv_lanes_kernel<T_Q4_K, 2, true><<<grid, 256, 0, s>>>(W, nb, a, out);
            else mv_lanes_kernel<T_Q4_K, 2, false><<<grid, 256, 0, s>>>(W, nb, a, out);
        }
    } else if (type == T_Q6_K) {
        const ActQ8K a = *(const ActQ8K *)act;
        if (dump) mv_lanes_kernel<T_Q6_K, 4, true><<<grid, 256, 0, s>>>(W, nb, a, out);
        else mv_lanes_kernel<T_Q6_K, 4, false><<<grid, 256, 0, s>>>(W, nb, a, out);
    } else if (type == T_Q8_0) {
        const ActQ8 a = *(const ActQ8 *)act;
        const int ntile = (nb + 3) / 4;
        if (dump) mv_q80_kernel<8, true><<<grid, 256, 0, s>>>(W, nb, ntile, a, out);
        else mv_q80_kernel<8, false><<<grid, 256, 0, s>>>(W, nb, ntile, a, out);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace fgh
