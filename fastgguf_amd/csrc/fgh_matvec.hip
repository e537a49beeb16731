// fgh_matvec.hip - the decode matvec for Q6_K / Q8_0 on gfx950 (Q4_K has its own kernel in
// fgh_q4k.hip): one persistent kernel per call that quantizes x itself and streams the weights.
//
//  * Quantization (once per workgroup and token): x (fp32, device) -> Q8_K or Q8 blocks in LDS,
//    bit-exact with the reference's quantize_q8k / quantize_q8 (fastgguf.c:746-793). 16 lanes
//    share one 256-value block (Q8_K) or 2 lanes one 32-value block (Q8); the block maximum is a
//    DPP reduction, d = amax/127 and id = 1/d are IEEE divisions, q = round-half-even(x * id).
//  * Matvec: workgroups loop over 8-row groups (the tile layout of fgh_internal.h); wavefront w
//    owns rows 2w and 2w+1 of a group. A "step" is one 16-byte load per lane covering 4 tiles x
//    2 rows x 8 slices (lane = slot*16 + row*8 + slice). Weight loads for the next chunk of steps
//    are issued before the current chunk is computed, so each wavefront keeps several KB in
//    flight. Lanes compute the exact integer partials of the reference's fp32 accumulator lanes
//    (v_dot4_i32_i8) and park them, converted to fp32 (exact), in wavefront-private LDS; then 2
//    or 16 lanes walk the tiles in ascending order applying the reference kernel's fused
//    multiply-adds, so outputs are bit-identical to it. No workgroup barrier after quantization.
//  * Up to 4 tensors of one type and width share one launch (matvec_multi, fastgguf.c:2552).
#include "fgh_internal.h"

namespace fgh {

constexpr int WAVES = 4;         // wavefronts per workgroup (256 threads)
constexpr int CS = 4;            // steps per pipelined chunk
constexpr int CT = 4 * CS;       // tiles per chunk

// per (row, tile) record in wavefront LDS, in floats
template <int TYPE, int ORDER>
struct Rec {
    // Q6_K: 8 lane partials, 4 correction lanes, d*yd (16 with padding); Q8_0: 4 blocks x 8 lane
    // partials + 4 d*xd
    static constexpr int N = TYPE == T_Q8_0 ? 36 : 16;
};

// LDS activation region, each array 16-byte aligned: qs at 0, d at act_off_d, sums at act_off_s
__host__ __device__ constexpr size_t align16(size_t v) { return (v + 15) & ~(size_t)15; }
__host__ __device__ constexpr size_t act_off_d(int type, int nb) { return (size_t)nb * (type == T_Q8_0 ? 32 : 256); }
__host__ __device__ constexpr size_t act_off_s(int type, int nb) { return align16(act_off_d(type, nb) + 4 * (size_t)nb); }
__host__ __device__ constexpr size_t act_lds_bytes(int type, int nb) {
    return align16(act_off_s(type, nb) + (size_t)nb * (type == T_Q8_0 ? 4 : 32));
}

template <int TYPE, int ORDER>
__host__ __device__ constexpr int wave_lds_bytes() {
    return 2 * CT * Rec<TYPE, ORDER>::N * 4 + 2 * 12 * 4;  // records + final-combine scratch
}

__device__ __forceinline__ float dpp_ror_f(float v, int n) {
    const int iv = __builtin_bit_cast(int, v);
    int r;
    switch (n) {  // row_ror:n (rotate within a row of 16 lanes)
    case 8: r = __builtin_amdgcn_update_dpp(0, iv, 0x128, 0xF, 0xF, false); break;
    case 4: r = __builtin_amdgcn_update_dpp(0, iv, 0x124, 0xF, 0xF, false); break;
    case 2: r = __builtin_amdgcn_update_dpp(0, iv, 0x122, 0xF, 0xF, false); break;
    default: r = __builtin_amdgcn_update_dpp(0, iv, 0x121, 0xF, 0xF, false); break;
    }
    return __builtin_bit_cast(float, r);
}

__device__ __forceinline__ int q_round(float v) {  // (int)lrintf(v) on x86 (see fgh_kernels.hip)
    return fabsf(v) < 2147483648.0f ? (int)rintf(v) : 0;
}
__device__ __forceinline__ uint32_t pack4q(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xFF) | ((uint32_t)(b & 0xFF) << 8) | ((uint32_t)(c & 0xFF) << 16) | ((uint32_t)(d & 0xFF) << 24);
}

// LDS activation region (offsets above). Q8_K: qs [nb][256] (lane-permuted as in
// fgh_internal.h), d [nb], bs [nb][16] int16. Q8: qs [nb][32], d [nb], s16 [nb][2].
template <int TYPE>
__device__ void quantize_to_lds(const float *__restrict__ x, int nb, uint8_t *smem) {
    const int tid = threadIdx.x;
    if (TYPE == T_Q8_0) {
        int8_t *qs = (int8_t *)smem;
        float *dd = (float *)(smem + act_off_d(T_Q8_0, nb));
        int16_t *s16 = (int16_t *)(smem + act_off_s(T_Q8_0, nb));
        // 2 threads per 32-value block, 128 blocks per round
        for (int rb = 0; rb < nb; rb += 128) {
            const int b = rb + (tid >> 1), h = tid & 1;
            const bool live = b < nb;
            float v[16];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                float4 f = live ? *(const float4 *)(x + (size_t)b * 32 + 16 * h + 4 * u) : make_float4(0.f, 0.f, 0.f, 0.f);
                v[4 * u] = f.x; v[4 * u + 1] = f.y; v[4 * u + 2] = f.z; v[4 * u + 3] = f.w;
            }
            float amax = 0.0f;
#pragma unroll
            for (int u = 0; u < 16; ++u) amax = fmaxf(amax, fabsf(v[u]));
            amax = fmaxf(amax, __builtin_bit_cast(float, dpp_xor1(__builtin_bit_cast(int, amax))));
            const float d = amax / 127.0f;
            const float id = d > 0.0f ? 1.0f / d : 0.0f;
            int s = 0;
            uint32_t w[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int q0 = q_round(v[4 * u] * id), q1 = q_round(v[4 * u + 1] * id);
                const int q2 = q_round(v[4 * u + 2] * id), q3 = q_round(v[4 * u + 3] * id);
                s += q0 + q1 + q2 + q3;
                w[u] = pack4q(q0, q1, q2, q3);
            }
            if (live) {
                *(uint4 *)(qs + (size_t)b * 32 + 16 * h) = make_uint4(w[0], w[1], w[2], w[3]);
                s16[2 * b + h] = (int16_t)s;
                if (h == 0) dd[b] = d;
            }
        }
    } else {
        int8_t *qs = (int8_t *)smem;
        float *dd = (float *)(smem + act_off_d(TYPE, nb));
        int16_t *bs = (int16_t *)(smem + act_off_s(TYPE, nb));
        // 16 threads per 256-value block, 16 blocks per round; thread tl holds values 16tl..16tl+15
        for (int rb = 0; rb < nb; rb += 16) {
            const int b = rb + (tid >> 4), tl = tid & 15;
            const bool live = b < nb;
            float v[16];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                float4 f = live ? *(const float4 *)(x + (size_t)b * 256 + 16 * tl + 4 * u) : make_float4(0.f, 0.f, 0.f, 0.f);
                v[4 * u] = f.x; v[4 * u + 1] = f.y; v[4 * u + 2] = f.z; v[4 * u + 3] = f.w;
            }
            float amax = 0.0f;
#pragma unroll
            for (int u = 0; u < 16; ++u) amax = fmaxf(amax, fabsf(v[u]));
            amax = fmaxf(amax, dpp_ror_f(amax, 8));
            amax = fmaxf(amax, dpp_ror_f(amax, 4));
            amax = fmaxf(amax, dpp_ror_f(amax, 2));
            amax = fmaxf(amax, dpp_ror_f(amax, 1));
            const float d = amax / 127.0f;
            const float id = d > 0.0f ? 1.0f / d : 0.0f;
            int s = 0;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int q0 = q_round(v[4 * u] * id), q1 = q_round(v[4 * u + 1] * id);
                const int q2 = q_round(v[4 * u + 2] * id), q3 = q_round(v[4 * u + 3] * id);
                s += q0 + q1 + q2 + q3;
                // value 16tl + 4u = 32c + 4i (c = tl/2, i = 4(tl%2) + u) goes to position 32i + 4c
                const int c = tl >> 1, i = 4 * (tl & 1) + u;
                if (live) *(uint32_t *)(qs + (size_t)b * 256 + 32 * i + 4 * c) = pack4q(q0, q1, q2, q3);
            }
            if (live) {
                bs[16 * b + tl] = (int16_t)s;
                if (tl == 0) dd[b] = d;
            }
        }
    }
}

// weights of one step for one lane: q = 16 quant bytes of its slice; m = the row's 16 meta bytes
// (Q6_K: int8 scales); h = Q6_K qh words, or the row's 4 fp16 d (Q8_0);
// e = Q6_K fp16 d of the row
struct StepW {
    uint4 q, m;
    uint2 h;
    uint32_t e;
};

template <int TYPE>
__device__ __forceinline__ void load_step(const uint8_t *__restrict__ Wg, int tile, int slice, int r, StepW &s) {
    constexpr int TILE = TYPE == T_Q6_K ? Q6K_TILE : Q80_TILE;
    const uint8_t *t = Wg + (size_t)tile * TILE;
    if (TYPE == T_Q6_K) {
        s.q = ld16(t + 144 + 16 * slice);
        s.h = ld8(t + 1168 + 8 * slice);
        s.m = ld16(t + 16 * r);
        s.e = *(const uint16_t *)(t + 128 + 2 * r);
    } else {
        s.q = ld16(t + 64 + 16 * slice);
        s.h = ld8(t + 8 * r);
    }
}

template <int TYPE, int ORDER, bool DUMP>
__global__ __launch_bounds__(256) void mv_kernel(MvArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int RN = Rec<TYPE, ORDER>::N;
    constexpr int TILE = TYPE == T_Q6_K ? Q6K_TILE : Q80_TILE;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int slot = lane >> 4, r2 = (lane >> 3) & 1, i = lane & 7;
    const int r = 2 * wave + r2;  // row within the 8-row group
    const int tok = blockIdx.y;
    const int nb = a.nb, ntile = a.ntile;
    uint8_t *act = smem;
    float *wrec = (float *)(smem + act_lds_bytes(TYPE, nb) + (size_t)wave * wave_lds_bytes<TYPE, ORDER>());
    float *wfin = wrec + 2 * CT * RN;

    // groups of this workgroup: g = blockIdx.x + n * gridDim.x
    const int64_t ng = a.groups > blockIdx.x ? (a.groups - 1 - blockIdx.x) / gridDim.x + 1 : 0;
    const int nchunk = (ntile + CT - 1) / CT;
    const int64_t nitems = ng * nchunk;

    auto tensor_of = [&](int64_t g, int &ti) {
        ti = 0;
        while (ti + 1 < a.nt && g >= a.t[ti + 1].gfirst) ++ti;
        return g - a.t[ti].gfirst;
    };
    auto load_item = [&](int64_t it, StepW (&sw)[CS]) {
        const int64_t g = blockIdx.x + (it / nchunk) * gridDim.x;
        const int c = (int)(it % nchunk);
        int ti;
        const int64_t lg = tensor_of(g, ti);
        const int64_t mg = a.sel ? (int64_t)a.sel[tok] * a.t[ti].gpm : 0;  // selected matrix (MoE)
        const uint8_t *Wg = a.t[ti].W + (size_t)(mg + lg) * ntile * TILE;
        // unconditional loads (slots past the end re-read the last tile and are not used), so
        // the compiler can count outstanding loads and wait only for the chunk it computes
#pragma unroll
        for (int k = 0; k < CS; ++k) {
            const int tile = min(c * CT + 4 * k + slot, ntile - 1);
            load_step<TYPE>(Wg, tile, 8 * r + i, r, sw[k]);
        }
    };

    StepW bufA[CS], bufB[CS];
    if (nitems > 0) load_item(0, bufA);  // first weights in flight during quantization

    quantize_to_lds<TYPE>(a.x + (size_t)(tok / a.xdiv) * a.ldx, nb, act);
    __syncthreads();

    const int8_t *aqs = (const int8_t *)act;
    const float *ad = (const float *)(act + act_off_d(TYPE, nb));
    const int16_t *abs16 = (const int16_t *)(act + act_off_s(TYPE, nb));

    // chain state: lanes 0..15 (r2, i)
    float acc = 0.0f, macc = 0.0f;

    auto process = [&](int64_t it, const StepW (&cur)[CS]) {
        const int c = (int)(it % nchunk);
        const int64_t g = blockIdx.x + (it / nchunk) * gridDim.x;
        int ti;
        const int64_t lg = tensor_of(g, ti);
        const int64_t lrow = (lg % a.t[ti].gpm) * 8 + r;
        const int64_t orow = (lg / a.t[ti].gpm) * a.t[ti].rows + lrow;
        const bool row_ok = lrow < a.t[ti].rows;

        // ---- integer phase: CS steps ----
#pragma unroll
        for (int k = 0; k < CS; ++k) {
            const int tile = c * CT + 4 * k + slot;
            const int tl = 4 * k + slot;  // tile within the chunk
            float *rec = wrec + ((size_t)r2 * CT + tl) * RN;
            if (TYPE == T_Q6_K) {
                if (c * CT + 4 * k < ntile) {
                    const bool live = tile < ntile;
                    const int b = live ? tile : 0;
                    const uint4 yv0 = *(const uint4 *)(aqs + (size_t)b * 256 + 32 * i);
                    const uint4 yv1 = *(const uint4 *)(aqs + (size_t)b * 256 + 32 * i + 16);
                    const int yv[8] = {(int)yv0.x, (int)yv0.y, (int)yv0.z, (int)yv0.w,
                                       (int)yv1.x, (int)yv1.y, (int)yv1.z, (int)yv1.w};
                    const StepW &s = cur[k];
                    const uint32_t sw[4] = {s.m.x, s.m.y, s.m.z, s.m.w};
                    const uint32_t A[4] = {s.q.x, s.q.y, s.q.z, s.q.w};
                    const uint32_t H[2] = {s.h.x, s.h.y};
                    const int hi4 = i >= 4;
                    int sum = 0;
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const uint32_t A0 = A[2 * h], A1 = A[2 * h + 1], Hh = H[h];
                        const uint32_t M4 = 0x0F0F0F0Fu, M2 = 0x03030303u;
                        const uint32_t qv[4] = {(A0 & M4) | ((Hh & M2) << 4), (A1 & M4) | (((Hh >> 2) & M2) << 4),
                                                ((A0 >> 4) & M4) | (((Hh >> 4) & M2) << 4),
                                                ((A1 >> 4) & M4) | (((Hh >> 6) & M2) << 4)};
#pragma unroll
                        for (int kk = 0; kk < 4; ++kk) {
                            const int si = 8 * h + 2 * kk + hi4;
                            sum += sbyte(sw[si >> 2], si & 3) * dot4((int)qv[kk], yv[4 * h + kk], 0);
                        }
                    }
                    const int p = i & 3;
                    const uint32_t *bp = (const uint32_t *)(abs16 + 16 * b);
                    const uint32_t b01 = bp[p], b89 = bp[p + 4];
                    const int s0 = sbyte(sw[(2 * p) >> 2], (2 * p) & 3), s1 = sbyte(sw[(2 * p + 1) >> 2], (2 * p + 1) & 3);
                    const int s8 = sbyte(sw[(2 * p + 8) >> 2], (2 * p + 8) & 3), s9 = sbyte(sw[(2 * p + 9) >> 2], (2 * p + 9) & 3);
                    const int mterm = (s0 * (int)(int16_t)(b01 & 0xFFFF) + s1 * (int)(int16_t)(b01 >> 16)) +
                                      (s8 * (int)(int16_t)(b89 & 0xFFFF) + s9 * (int)(int16_t)(b89 >> 16));
                    const float fd = fp16_bits_to_f32(s.e) * ad[b];
                    if (live) {
                        rec[i] = (float)sum;
                        if (i < 4) rec[8 + i] = (float)mterm;
                        if (i == 0) { rec[12] = fd; rec[13] = fd * 32.0f; }
                    }
                    if (DUMP) {
                        const int ts = sum8_i32(sum), tm = sum4_i32(mterm);
                        if (live && i == 0 && row_ok) {
                            a.dump_s[orow * nb + b] = ts;
                            a.dump_m[orow * nb + b] = tm;
                        }
                    }
                }
            } else {  // Q8_0: a tile is 4 blocks
                if (c * CT + 4 * k < ntile) {
                    const bool live = tile < ntile;
                    const StepW &s = cur[k];
                    const uint32_t qw[4] = {s.q.x, s.q.y, s.q.z, s.q.w};
                    const uint32_t dw[4] = {s.h.x & 0xFFFF, s.h.x >> 16, s.h.y & 0xFFFF, s.h.y >> 16};
#pragma unroll
                    for (int bb = 0; bb < 4; ++bb) {
                        const int b = 4 * tile + bb;
                        const bool bl = live && b < nb;
                        const int bsafe = bl ? b : 0;
                        const int yw = *(const int *)(aqs + (size_t)bsafe * 32 + 4 * i);
                        const int sdot = dot4((int)qw[bb], yw, 0);
                        if (bl) {
                            rec[8 * bb + i] = (float)sdot;
                            if (i == 0) rec[32 + bb] = fp16_bits_to_f32(dw[bb]) * ad[bsafe];
                        }
                        if (DUMP) {
                            const int ts = sum8_i32(sdot);
                            if (bl && i == 0 && row_ok) {
                                a.dump_s[orow * nb + b] = ts;
                                a.dump_m[orow * nb + b] = 0;
                            }
                        }
                    }
                }
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        // ---- chain phase: ascending tiles of this chunk ----
        const int nct = min(CT, ntile - c * CT);
        // (all reads first, then the ordered fused multiply-adds; records past nct are skipped)
        if (TYPE == T_Q8_0) {
            if (slot == 0) {
                const float *rec = wrec + (size_t)r2 * CT * RN;
                const int nblk = min(4 * nct, nb - 4 * c * CT);
#pragma unroll
                for (int tl = 0; tl < CT; ++tl) {
                    float lv[4], dv[4];
#pragma unroll
                    for (int bb = 0; bb < 4; ++bb) {
                        lv[bb] = rec[tl * RN + 8 * bb + i];
                        dv[bb] = rec[tl * RN + 32 + bb];
                    }
#pragma unroll
                    for (int bb = 0; bb < 4; ++bb)
                        if (4 * tl + bb < nblk) acc = __builtin_fmaf(dv[bb], lv[bb], acc);
                }
            }
        } else {
            if (slot == 0) {
                const float *rec = wrec + (size_t)r2 * CT * RN;
#pragma unroll
                for (int t0 = 0; t0 < CT; t0 += 4) {
                    float lv[4], mv[4], dv[4], mdv[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        lv[u] = rec[(t0 + u) * RN + i];
                        mv[u] = rec[(t0 + u) * RN + 8 + (i & 3)];
                        dv[u] = rec[(t0 + u) * RN + 12];
                        mdv[u] = rec[(t0 + u) * RN + 13];
                    }
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        if (t0 + u < nct) {
                            acc = __builtin_fmaf(dv[u], lv[u], acc);
                            macc = __builtin_fmaf(mdv[u], mv[u], macc);
                        }
                }
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        // ---- end of a group: combine the lanes in the reference's order and store ----
        if (c == nchunk - 1) {
            float *y = a.t[ti].y + (size_t)tok * a.ldy;
            if (slot == 0) {
                wfin[12 * r2 + i] = acc;
                if (i < 4) wfin[12 * r2 + 8 + i] = macc;
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            if (slot == 0 && i == 0 && row_ok) {
                const float *v = wfin + 12 * r2;
                const float h8 = ((v[0] + v[4]) + (v[1] + v[5])) + ((v[2] + v[6]) + (v[3] + v[7]));
                y[orow] = TYPE == T_Q8_0 ? h8 : h8 - ((v[8] + v[9]) + (v[10] + v[11]));
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            acc = 0.0f;
            macc = 0.0f;
        }
    };

    // two register buffers, swapped by unrolling: the next item's loads are in flight while the
    // current one is computed
    for (int64_t it = 0; it < nitems; it += 2) {
        if (it + 1 < nitems) load_item(it + 1, bufB);
        process(it, bufA);
        if (it + 1 >= nitems) break;
        if (it + 2 < nitems) load_item(it + 2, bufA);
        process(it + 1, bufB);
    }
}

template <int TYPE, int ORDER>
static size_t mv_lds_bytes(int nb) {
    return act_lds_bytes(TYPE, nb) + (size_t)WAVES * wave_lds_bytes<TYPE, ORDER>();
}

size_t matvec_lds_bytes(int type, int order, int nb) {
    if (type == T_Q4_K) return q4k_lds_bytes(order, nb);
    if (type == T_Q6_K) return mv_lds_bytes<T_Q6_K, 0>(nb);
    return mv_lds_bytes<T_Q8_0, 0>(nb);
}

// persistent grid: as many workgroups as fit on the device at once (occupancy of this variant at
// this LDS size), balanced so that every workgroup gets the same number of row groups (+-1)
template <int TYPE, int ORDER, bool DUMP>
static hipError_t launch_t(const MvArgs &a, int ntok, int num_cu, hipStream_t s) {
    const size_t lds = matvec_lds_bytes(TYPE, ORDER, a.nb);
    if (lds > 65536) return hipErrorInvalidValue;
    int per_cu = 0;
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, mv_kernel<TYPE, ORDER, DUMP>, 256, lds);
    if (e != hipSuccess) return e;
    const int64_t max_wg = (int64_t)num_cu * (per_cu > 0 ? per_cu : 1);
    int64_t wg = a.groups;
    if (wg > max_wg) {
        const int64_t per = (a.groups + max_wg - 1) / max_wg;
        wg = (a.groups + per - 1) / per;
    }
    mv_kernel<TYPE, ORDER, DUMP><<<dim3((unsigned)wg, ntok), 256, lds, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_matvec2(int type, int order, const MvArgs &a, int ntok, int num_cu, hipStream_t s) {
    const bool dump = a.dump_s != nullptr;
    if (type == T_Q4_K) return launch_q4k_matvec(order, a, ntok, num_cu, s);
    if (type == T_Q6_K)
        return dump ? launch_t<T_Q6_K, 0, true>(a, ntok, num_cu, s) : launch_t<T_Q6_K, 0, false>(a, ntok, num_cu, s);
    if (type == T_Q8_0)
        return dump ? launch_t<T_Q8_0, 0, true>(a, ntok, num_cu, s) : launch_t<T_Q8_0, 0, false>(a, ntok, num_cu, s);
    return hipErrorInvalidValue;
}

}  // namespace fgh
