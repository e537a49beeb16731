// fgh_q4k.hip - Q4_K decode matvec for gfx950 (the dominant kernel of a Q4_K_M decode layer).
//
// Device layout of a Q4_K tensor (written at upload by q4k_relayout_kernel): rows in groups of
// 8, each group 1152 * nb bytes (the same bytes as the file: 8 rows x nb blocks x 144 B).
// Wavefront w of a group's workgroup owns rows 2w and 2w+1; its P = 2 * nb (row, block) "pairs"
// are numbered q = r2 * nb + b. Inside the group:
//   meta   [0, 128 nb):        pair q of wavefront w at 16 * (P * w + q): the block's first 16
//                              bytes (fp16 d, fp16 dmin, 12 bytes of 6-bit scales and mins)
//   quants [128 nb, 1152 nb):  wavefront w at + 256 nb * w, in steps of 16 pairs (2 KB each);
//                              lane L = 4 * (q % 16) + j holds chunk j (32 bytes = sub-blocks 2j
//                              and 2j+1) of pair q as two 16-byte pieces: piece h at
//                              + 2048 * step + h * 64 * np + 16 * L (np = pairs in the step)
// so every load instruction of a wavefront reads one contiguous span and the layout is dense
// for any nb.
//
// One workgroup per 8-row group (grid.y = token). It issues the loads of x (to quantize it) and
// then every weight load of its group, quantizes x into LDS (Q8_K, bit-exact with quantize_q8k,
// fastgguf.c:773-793) while the weights are in flight, and then computes: each lane the exact
// integer dot products of its chunk (v_dot4_i32_i8), a quad reduction per (row, block), fp32
// records in wavefront LDS, and the reference's fused multiply-add chain in block order by one
// lane per row:
//   repacked order, dot_q4Kx8 (fastgguf.c:2322-2358): acc = fma(d*yd, sumi, acc),
//                   macc = fma(dmin*yd, msum, macc), out = acc - macc
//   row order, dot_q4_K_q8k (fastgguf.c:1118-1153): 8 lane chains and 4 min chains, out =
//                   hsum8(acc) - hsum4(macc)
#include "fgh_internal.h"

namespace fgh {

constexpr int Q4_MAXS = 8;  // steps (16 pairs each) of one wavefront held in registers at once

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

// LDS: natural-order Q8_K blocks: qs [nb][256] at 0, d [nb] at 256 nb, bsums [nb][16] at
// align16(260 nb); then 4 wavefront record areas
__host__ __device__ constexpr size_t q4_off_d(int nb) { return (size_t)nb * 256; }
__host__ __device__ constexpr size_t q4_off_s(int nb) { return ((size_t)nb * 260 + 15) & ~(size_t)15; }
__host__ __device__ constexpr size_t q4_act_bytes(int nb) { return (q4_off_s(nb) + (size_t)nb * 32 + 15) & ~(size_t)15; }
template <int ORDER>
__host__ __device__ constexpr size_t q4_rec_floats() { return ORDER == 1 ? 4 : 16; }
__host__ __device__ inline size_t q4_wave_bytes(int order, int nb) {
    return (size_t)2 * nb * (order == 1 ? 4 : 16) * 4 + 2 * 12 * 4;
}
size_t q4k_lds_bytes(int order, int nb, int gpw) { return q4_act_bytes(nb) + 4 * (size_t)gpw * q4_wave_bytes(order, nb); }

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
__device__ __forceinline__ void q8k_load(const float *__restrict__ x, int nb, int rb, XRound &xr) {
    const int b = rb + (threadIdx.x >> 4);
    q8k_load_b(x, b, b < nb, xr);
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
    if (live) {
        *(uint4 *)(act + (size_t)b * 256 + 16 * tl) = make_uint4(w[0], w[1], w[2], w[3]);
        ((int16_t *)(act + q4_off_s(nb)))[16 * b + tl] = (int16_t)s;
        if (tl == 0) ((float *)(act + q4_off_d(nb)))[b] = d;
    }
}
__device__ __forceinline__ void q8k_store(int nb, int rb, const XRound &xr, uint8_t *act) {
    const int b = rb + (threadIdx.x >> 4);
    q8k_store_b(nb, b, b < nb, xr, act);
}

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// one step's registers: two 16-byte pieces of the lane's chunk and the pair's 16 meta bytes
struct Q4Step {
    uint4 p0, p1, m;
};

// what one wavefront needs to compute its steps: the quantized x and its record area (LDS)
struct Q4Ctx {
    const uint8_t *act;
    const float *ad;
    const int16_t *abs16;
    float *rec;
    int nb, P, j, pl;
};

// where the per-(row, block) integers of the test hook go: rows dbase + r2 if r2 < dleft
struct Q4Dump {
    int32_t *s, *m;
    int64_t base;
    int64_t left;
};

// One step (16 (row, block) pairs) of one wavefront from its registers: the exact integers of the
// lane's chunk (v_dot4_i32_i8), reduced over the pair's 4 lanes, and the pair's fp32 record in LDS
//   repacked: float4 {d*yd, sumi, dmin*yd, msum} at pair q
//   row:      16 floats at pair q: the 8 lane partials (dword i = the reference's lane i), the 4
//             min partials at 8 + j, d*yd at 12, dmin*yd at 13
template <int ORDER, bool DUMP>
__device__ __forceinline__ void q4_step(const Q4Step &st, int s, const Q4Ctx &c, const Q4Dump &dump) {
    const int nb = c.nb, j = c.j, pl = c.pl;
    const int np = min(16, c.P - 16 * s);
    const bool live = pl < np;
    const int q = 16 * s + min(pl, np - 1);
    const int r2 = q >= nb, b = q - r2 * nb;
    const uint8_t *yb = c.act + (size_t)b * 256 + 64 * j;
    const uint4 ylo0 = *(const uint4 *)yb, ylo1 = *(const uint4 *)(yb + 16);
    const uint4 yhi0 = *(const uint4 *)(yb + 32), yhi1 = *(const uint4 *)(yb + 48);
    const uint32_t qd[8] = {st.p0.x, st.p0.y, st.p0.z, st.p0.w, st.p1.x, st.p1.y, st.p1.z, st.p1.w};
    const uint32_t ylo[8] = {ylo0.x, ylo0.y, ylo0.z, ylo0.w, ylo1.x, ylo1.y, ylo1.z, ylo1.w};
    const uint32_t yhi[8] = {yhi0.x, yhi0.y, yhi0.z, yhi0.w, yhi1.x, yhi1.y, yhi1.z, yhi1.w};
    // scales and mins of sub-blocks 2j (low nibbles) and 2j+1 (high nibbles) of this chunk,
    // straight from the packed words u0..u2 (scale_min_k4, fastgguf.c:466-472): for j < 2 the low
    // 6 bits of bytes 2j, 2j+1 of u0 (scales) and u1 (mins); for j >= 2 the nibbles of bytes
    // 2j-4, 2j-3 of u2 with the top 2 bits of the same bytes of u0 / u1
    const int sh = 16 * (j & 1);
    const uint32_t A = st.m.y >> sh, B = st.m.z >> sh, C = st.m.w >> sh;
    const uint32_t scp = j < 2 ? (A & 0x3f3fu) : ((C & 0x0f0fu) | ((A & 0xc0c0u) >> 2));
    const uint32_t mnp = j < 2 ? (B & 0x3f3fu) : (((C >> 4) & 0x0f0fu) | ((B & 0xc0c0u) >> 2));
    // (s_lo, s_hi) as an int16 pair for the packed dots below; m_lo, m_hi as bytes
    const uint32_t sc2 = __builtin_amdgcn_perm(0u, scp, 0x0C010C00u);
    const int m_lo = (int)(mnp & 0x3F), m_hi = (int)((mnp >> 8) & 0x3F);
    // min term m_2j (bs[4j] + bs[4j+1]) + m_2j+1 (bs[4j+2] + bs[4j+3]): two packed int16 dots on
    // the activation sums as stored (all values fit int16)
    const uint2 bq = *(const uint2 *)(c.abs16 + 16 * b + 4 * j);
    const int mterm = dot2_i16((uint32_t)m_lo | ((uint32_t)m_lo << 16), bq.x,
                               dot2_i16((uint32_t)m_hi | ((uint32_t)m_hi << 16), bq.y, 0));
    const float yd = c.ad[b];
    const float fd = fp16_bits_to_f32(st.m.x & 0xFFFF) * yd;
    const float fdm = fp16_bits_to_f32(st.m.x >> 16) * yd;
    if (ORDER == 1) {
        // integer dots of the low / high nibbles in two halves of 16 values each: every partial is
        // at most 16 * 15 * 127 = 30480 in magnitude, so fits int16, and the scale products are
        // two packed int16 dots
        int il0 = 0, il1 = 0, ih0 = 0, ih1 = 0;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            il0 = dot4((int)(qd[d] & 0x0F0F0F0Fu), (int)ylo[d], il0);
            ih0 = dot4((int)((qd[d] >> 4) & 0x0F0F0F0Fu), (int)yhi[d], ih0);
            il1 = dot4((int)(qd[d + 4] & 0x0F0F0F0Fu), (int)ylo[d + 4], il1);
            ih1 = dot4((int)((qd[d + 4] >> 4) & 0x0F0F0F0Fu), (int)yhi[d + 4], ih1);
        }
        const int sumi = sum4_i32(dot2_i16(sc2, pack_i16(il0, ih0), dot2_i16(sc2, pack_i16(il1, ih1), 0)));
        const int msum = sum4_i32(mterm);
        if (live && j == 0) {
            *(float4 *)(c.rec + 4 * q) = make_float4(fd, (float)sumi, fdm, (float)msum);
            if (DUMP && r2 < dump.left) {
                dump.s[(dump.base + r2) * nb + b] = sumi;
                dump.m[(dump.base + r2) * nb + b] = msum;
            }
        }
    } else {
        // the reference's lane i sums bytes 4i..4i+3 of every chunk: dword i here
        int lv[8];
#pragma unroll
        for (int d = 0; d < 8; ++d) {
            // each dot4 is at most 4 * 15 * 127 = 7620 in magnitude: an int16 pair
            lv[d] = dot2_i16(sc2, pack_i16(dot4((int)(qd[d] & 0x0F0F0F0Fu), (int)ylo[d], 0),
                                           dot4((int)((qd[d] >> 4) & 0x0F0F0F0Fu), (int)yhi[d], 0)), 0);
            lv[d] = sum4_i32(lv[d]);
        }
        float *rq = c.rec + 16 * q;
        if (live) {
            rq[8 + j] = (float)mterm;  // min lane p = j
            if (j == 0) {
#pragma unroll
                for (int d = 0; d < 8; ++d) rq[d] = (float)lv[d];
                rq[12] = fd;
                rq[13] = fdm;
            }
        }
        if (DUMP) {
            int ts = 0;
#pragma unroll
            for (int d = 0; d < 8; ++d) ts += lv[d];
            const int tm = sum4_i32(mterm);
            if (live && j == 0 && r2 < dump.left) {
                dump.s[(dump.base + r2) * nb + b] = ts;
                dump.m[(dump.base + r2) * nb + b] = tm;
            }
        }
    }
}

// The reference's fp32 chain over the wavefront's records, in ascending block order, and its
// final combination; rows ybase[0], ybase[1] (if r2 < left). Call after a wave_sync.
template <int ORDER>
__device__ __forceinline__ void q4_chain(const Q4Ctx &c, int lane, float *__restrict__ ybase, int64_t left) {
    const int nb = c.nb;
    if (ORDER == 1) {
        if (lane < 2) {
            const float *rr = c.rec + 4 * (size_t)lane * nb;
            float acc = 0.0f, macc = 0.0f;
            int b = 0;
            for (; b + 4 <= nb; b += 4) {
                float4 p[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) p[u] = *(const float4 *)(rr + 4 * (b + u));
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    acc = __builtin_fmaf(p[u].x, p[u].y, acc);
                    macc = __builtin_fmaf(p[u].z, p[u].w, macc);
                }
            }
            for (; b < nb; ++b) {
                const float4 p = *(const float4 *)(rr + 4 * b);
                acc = __builtin_fmaf(p.x, p.y, acc);
                macc = __builtin_fmaf(p.z, p.w, macc);
            }
            if (lane < left) ybase[lane] = acc - macc;
        }
    } else {
        float *fin = c.rec + (size_t)2 * nb * 16;
        if (lane < 16) {
            const int r2 = lane >> 3, i = lane & 7;
            const float *rr = c.rec + 16 * (size_t)r2 * nb;
            float acc = 0.0f, macc = 0.0f;
            for (int b = 0; b < nb; ++b) {
                const float *p = rr + 16 * b;
                acc = __builtin_fmaf(p[12], p[i], acc);
                macc = __builtin_fmaf(p[13], p[8 + (i & 3)], macc);
            }
            fin[12 * r2 + i] = acc;
            if (i < 4) fin[12 * r2 + 8 + i] = macc;
        }
        wave_sync();
        if (lane < 2 && lane < left) {
            const float *v = fin + 12 * lane;
            const float h8 = ((v[0] + v[4]) + (v[1] + v[5])) + ((v[2] + v[6]) + (v[3] + v[7]));
            ybase[lane] = h8 - ((v[8] + v[9]) + (v[10] + v[11]));
        }
    }
}

// the tensor of global group g in a multi-tensor launch
__device__ __forceinline__ int q4_tensor_of(const MvArgs &a, int64_t g) {
    int ti = 0;
#pragma unroll
    for (int k = 1; k < 4; ++k)
        if (k < a.nt && g >= a.t[k].gfirst) ti = k;
    return ti;
}

template <int ORDER, int MAXS, int GPW, bool DUMP>
__global__ __launch_bounds__(256 * GPW) void q4k_mv_kernel(MvArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    // wave-uniform indices in scalar registers: the tensor selection below then reads the kernel
    // arguments with scalar loads instead of per-lane memory loads ahead of the weight stream
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane((tid >> 6) & 3);
    const int gsub = __builtin_amdgcn_readfirstlane(tid >> 8);
    const int j = lane & 3, pl = lane >> 2;  // chunk, pair within the step
    const int nb = a.nb, P = 2 * nb;
    const int nsteps = (P + 15) >> 4;
    const int tok = blockIdx.y;
    const int64_t g = (int64_t)blockIdx.x * GPW + gsub;
    if (g >= a.groups) {  // a trailing workgroup's spare group: only help quantize
        const float *xs = a.x + (size_t)(blockIdx.y / a.xdiv) * a.ldx;
        for (int rb = 0; rb < nb; rb += 16 * GPW) {
            XRound xr;
            q8k_load(xs, nb, rb, xr);
            q8k_store(nb, rb, xr, smem);
        }
        __syncthreads();
        return;
    }
    const int ti = q4_tensor_of(a, g);
    const int64_t lg = g - a.t[ti].gfirst;
    const int64_t mg = a.sel ? (int64_t)a.sel[tok] * a.t[ti].gpm : 0;  // selected matrix (MoE)
    const uint8_t *G = a.t[ti].W + (size_t)(mg + lg) * 1152 * nb;
    const uint8_t *meta = G + (size_t)16 * P * wave;
    const uint8_t *quant = G + (size_t)128 * nb + (size_t)256 * nb * wave;

    uint8_t *act = smem;
    Q4Ctx c;
    c.act = act;
    c.ad = (const float *)(act + q4_off_d(nb));
    c.abs16 = (const int16_t *)(act + q4_off_s(nb));
    c.rec = (float *)(smem + q4_act_bytes(nb) + (size_t)(4 * gsub + wave) * q4_wave_bytes(ORDER, nb));
    c.nb = nb;
    c.P = P;
    c.j = j;
    c.pl = pl;
    const int64_t lr0 = (lg % a.t[ti].gpm) * 8 + 2 * wave;
    const int64_t obase = (lg / a.t[ti].gpm) * a.t[ti].rows;
    Q4Dump dump{a.dump_s, a.dump_m, obase + lr0, a.t[ti].rows - lr0};

    // (1) x for the first quantization round, then (2) every weight load of the first chunk
    const float *x = a.x + (size_t)(tok / a.xdiv) * a.ldx;
    XRound xr;
    q8k_load(x, nb, 0, xr);
    Q4Step st[MAXS];
    auto load_steps = [&](int s0) {
#pragma unroll
        for (int k = 0; k < MAXS; ++k) {
            const int s = s0 + k;
            if (s < nsteps) {  // uniform
                const int np = min(16, P - 16 * s);
                const int pc = min(pl, np - 1);  // lanes past the last pair re-read a live one
                const uint8_t *qb = quant + (size_t)2048 * s + 16 * (4 * pc + j);
                st[k].p0 = ld16(qb);
                st[k].p1 = ld16(qb + 64 * np);
                st[k].m = ld16(meta + 16 * (16 * s + pc));
            }
        }
    };
    load_steps(0);
    // (3) quantize x into LDS while the weights are in flight (16 * GPW blocks per round)
    for (int rb = 0; rb < nb; rb += 16 * GPW) {
        if (rb > 0) q8k_load(x, nb, rb, xr);
        q8k_store(nb, rb, xr, act);
    }
    __syncthreads();

    for (int s0 = 0; s0 < nsteps; s0 += MAXS) {
        if (s0 > 0) load_steps(s0);
#pragma unroll
        for (int k = 0; k < MAXS; ++k) {
            const int s = s0 + k;
            if (s >= nsteps) break;  // uniform
            q4_step<ORDER, DUMP>(st[k], s, c, dump);
        }
    }
    wave_sync();
    q4_chain<ORDER>(c, lane, a.t[ti].y + (size_t)tok * a.ldy + obase + lr0, a.t[ti].rows - lr0);
}

#ifndef FGH_Q4_GPW
#define FGH_Q4_GPW 2
#endif
constexpr int Q4_GPW = FGH_Q4_GPW;  // 8-row groups per workgroup (sharing one quantization of x)

// groups per workgroup for a row length: Q4_GPW when its LDS fits 64 KiB, else 1
static int q4_gpw(int order, int nb) { return q4k_lds_bytes(order, nb, Q4_GPW) <= 65536 ? Q4_GPW : 1; }

template <int ORDER, int MAXS, int GPW>
static hipError_t q4_launch(const MvArgs &a, int ntok, size_t lds, hipStream_t s) {
    const unsigned wg = (unsigned)((a.groups + GPW - 1) / GPW);
    if (a.dump_s) q4k_mv_kernel<ORDER, MAXS, GPW, true><<<dim3(wg, ntok), 256 * GPW, lds, s>>>(a);
    else q4k_mv_kernel<ORDER, MAXS, GPW, false><<<dim3(wg, ntok), 256 * GPW, lds, s>>>(a);
    return hipGetLastError();
}

template <int ORDER, int GPW>
static hipError_t q4_launch_steps(const MvArgs &a, int ntok, size_t lds, hipStream_t s) {
    // registers sized to the step count; longer rows loop over chunks of Q4_MAXS steps
    const int nsteps = (2 * a.nb + 15) / 16;
    if (nsteps <= 1) return q4_launch<ORDER, 1, GPW>(a, ntok, lds, s);
    if (nsteps <= 2) return q4_launch<ORDER, 2, GPW>(a, ntok, lds, s);
    if (nsteps <= 4) return q4_launch<ORDER, 4, GPW>(a, ntok, lds, s);
    return q4_launch<ORDER, Q4_MAXS, GPW>(a, ntok, lds, s);
}

size_t q4k_lds_bytes(int order, int nb) { return q4k_lds_bytes(order, nb, q4_gpw(order, nb)); }

hipError_t launch_q4k_matvec(int order, const MvArgs &a, int ntok, int, hipStream_t s) {
    const int gpw = q4_gpw(order, a.nb);
    const size_t lds = q4k_lds_bytes(order, a.nb, gpw);
    if (lds > 65536) return hipErrorInvalidValue;
    if (order == 1) return gpw == 1 ? q4_launch_steps<1, 1>(a, ntok, lds, s) : q4_launch_steps<1, Q4_GPW>(a, ntok, lds, s);
    return gpw == 1 ? q4_launch_steps<0, 1>(a, ntok, lds, s) : q4_launch_steps<0, Q4_GPW>(a, ntok, lds, s);
}

// Q8_K images of activation rows, in the kernels' LDS layout (q4_act_bytes(nb) bytes per row): row
// r of x (stride ldx) -> img + r * q4_act_bytes(nb). SILU: the row is silu(g) * u of two fp32
// arrays (silu_f, fastgguf.c:3118: x / (1 + expf(-x))), quantized without being stored.
// 16 threads per 256-value block, 16 blocks per workgroup.
template <bool SILU>
__global__ __launch_bounds__(256) void q4_image_kernel(const float *__restrict__ x, const float *__restrict__ u,
                                                       int64_t ldx, int nb, int64_t rows, uint8_t *__restrict__ img) {
    const int64_t cb = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);  // (row, block)
    const bool live = cb < rows * nb;
    const int64_t r = live ? cb / nb : 0;
    const int b = live ? (int)(cb - r * nb) : 0;
    XRound xr;
    q8k_load_b(x + (size_t)r * ldx, b, true, xr);
    if (SILU) {
        XRound ur;
        q8k_load_b(u + (size_t)r * ldx, b, true, ur);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float4 &g = xr.v[q];
            const float4 uu = ur.v[q];
            g.x = g.x / (1.0f + expf_ref(-g.x)) * uu.x;
            g.y = g.y / (1.0f + expf_ref(-g.y)) * uu.y;
            g.z = g.z / (1.0f + expf_ref(-g.z)) * uu.z;
            g.w = g.w / (1.0f + expf_ref(-g.w)) * uu.w;
        }
    }
    q8k_store_b(nb, b, live, xr, img + (size_t)r * q4_act_bytes(nb));
}

hipError_t launch_q4_image(const float *x, const float *u, int64_t ldx, int nb, int64_t rows, uint8_t *img,
                           hipStream_t s) {
    const int64_t wg = (rows * nb + 15) / 16;
    if (u) q4_image_kernel<true><<<(unsigned)wg, 256, 0, s>>>(x, u, ldx, nb, rows, img);
    else q4_image_kernel<false><<<(unsigned)wg, 256, 0, s>>>(x, u, ldx, nb, rows, img);
    return hipGetLastError();
}
size_t q4_image_bytes(int nb) { return q4_act_bytes(nb); }

// MoE expert matvecs grouped by expert (row order, dot_q4_K_q8k): workgroup (x, y) takes 8-row group
// x of the matrix of segment y (one selected expert with its token slots, from moe_group_kernel)
// and every slot of that segment. Each wavefront loads its two rows' weights into registers once,
// then for every chunk of MOE_TC slots copies their activation images (q4_image_kernel, row
// slot / a.xdiv) into LDS and runs the same steps and chain as q4k_mv_kernel, once per slot.
// Tensor i of a.t: output rows y_i[slot * ldy]. seg: [0] = number of segments, then per segment
// {expert, first, count}.
constexpr int MOE_TC = 4;
template <int MAXS>
__global__ __launch_bounds__(256) void q4k_moe_kernel(MvArgs a, const int32_t *__restrict__ seg,
                                                      const int32_t *__restrict__ slots, const uint8_t *__restrict__ img) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 3, pl = lane >> 2;
    const int nb = a.nb, P = 2 * nb;
    const int nsteps = (P + 15) >> 4;
    const int sidx = blockIdx.y;
    if (sidx >= seg[0]) return;  // whole workgroup: fewer segments than the grid allows
    const int expert = seg[1 + 3 * sidx], first = seg[2 + 3 * sidx], count = seg[3 + 3 * sidx];
    const int64_t g = blockIdx.x;
    const int ti = q4_tensor_of(a, g);
    const int64_t lg = g - a.t[ti].gfirst;  // group within the matrix
    const uint8_t *G = a.t[ti].W + (size_t)((int64_t)expert * a.t[ti].gpm + lg) * 1152 * nb;
    const uint8_t *meta = G + (size_t)16 * P * wave;
    const uint8_t *quant = G + (size_t)128 * nb + (size_t)256 * nb * wave;
    Q4Step st[MAXS];
#pragma unroll
    for (int k = 0; k < MAXS; ++k) {
        const int s = k < nsteps ? k : nsteps - 1;
        const int np = min(16, P - 16 * s);
        const int pc = min(pl, np - 1);
        const uint8_t *qb = quant + (size_t)2048 * s + 16 * (4 * pc + j);
        st[k].p0 = ld16(qb);
        st[k].p1 = ld16(qb + 64 * np);
        st[k].m = ld16(meta + 16 * (16 * s + pc));
    }
    const size_t actb = q4_act_bytes(nb), waveb = q4_wave_bytes(0, nb);
    const int units = (int)(actb / 16);
    const int64_t lr0 = lg * 8 + 2 * wave;
    const int64_t left = a.t[ti].rows - lr0;
    float *rec0 = (float *)(smem + MOE_TC * actb + (size_t)wave * waveb);
    for (int c0 = 0; c0 < count; c0 += MOE_TC) {
        const int nc = min(MOE_TC, count - c0);
        // the chunk's activation images (rows slot / xdiv) into LDS
        for (int i = tid; i < nc * units; i += 256) {
            const int c = i / units, o = i - c * units;
            const int slot = slots[first + c0 + c];
            ((uint4 *)(smem + (size_t)c * actb))[o] = ((const uint4 *)(img + (size_t)(slot / a.xdiv) * actb))[o];
        }
        __syncthreads();
        for (int c = 0; c < nc; ++c) {
            const uint8_t *act = smem + (size_t)c * actb;
            Q4Ctx cx;
            cx.act = act;
            cx.ad = (const float *)(act + q4_off_d(nb));
            cx.abs16 = (const int16_t *)(act + q4_off_s(nb));
            cx.rec = rec0;
            cx.nb = nb;
            cx.P = P;
            cx.j = j;
            cx.pl = pl;
            Q4Dump none{nullptr, nullptr, 0, 0};
#pragma unroll
            for (int k = 0; k < MAXS; ++k)
                if (k < nsteps) q4_step<0, false>(st[k], k, cx, none);
            wave_sync();
            q4_chain<0>(cx, lane, a.t[ti].y + (size_t)slots[first + c0 + c] * a.ldy + lr0, left);
            wave_sync();  // the next slot's records reuse the area
        }
        __syncthreads();  // the next chunk reuses the activations
    }
}

size_t q4k_moe_lds_bytes(int nb) { return MOE_TC * q4_act_bytes(nb) + 4 * q4_wave_bytes(0, nb); }

// a.groups = groups of one matrix over all tensors (the launch's x extent); grid.y = max_segments
hipError_t launch_q4k_moe(const MvArgs &a, const int32_t *seg, const int32_t *slots, const uint8_t *img,
                          int max_segments, hipStream_t s) {
    const int nsteps = (2 * a.nb + 15) / 16;
    const size_t lds = q4k_moe_lds_bytes(a.nb);
    if (nsteps > 4 || lds > 65536) return hipErrorInvalidValue;
    const dim3 grid((unsigned)a.groups, (unsigned)max_segments);
    if (nsteps <= 1) q4k_moe_kernel<1><<<grid, 256, lds, s>>>(a, seg, slots, img);
    else if (nsteps <= 2) q4k_moe_kernel<2><<<grid, 256, lds, s>>>(a, seg, slots, img);
    else q4k_moe_kernel<4><<<grid, 256, lds, s>>>(a, seg, slots, img);
    return hipGetLastError();
}

// upload-time re-layout of Q4_K rows into the group layout above; one thread per destination byte
__global__ void q4k_relayout_kernel(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, int64_t rows,
                                    int nb, int64_t gpm, int64_t total, int64_t row_bytes) {
    const int64_t gbytes = (int64_t)1152 * nb;
    const int P = 2 * nb;
    for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < total; o += (int64_t)gridDim.x * blockDim.x) {
        const int64_t g = o / gbytes;
        const int64_t ob = o - g * gbytes;
        const int64_t m = g / gpm, gl = g - m * gpm;
        int w, q, byte;
        if (ob < (int64_t)128 * nb) {
            const int idx = (int)(ob >> 4);
            w = idx / P;
            q = idx - w * P;
            byte = (int)(ob & 15);
        } else {
            const int64_t o2 = ob - (int64_t)128 * nb;
            w = (int)(o2 / (256 * (int64_t)nb));
            const int o3 = (int)(o2 - (int64_t)w * 256 * nb);
            const int s = o3 >> 11, np = min(16, P - 16 * s);
            const int u = o3 - 2048 * s, h = u / (64 * np), v = u - h * 64 * np;
            const int L = v >> 4, jj = L & 3;
            q = 16 * s + (L >> 2);
            byte = 16 + 32 * jj + 16 * h + (v & 15);
        }
        const int r = 2 * w + (q >= nb), b = q - (q >= nb) * nb;
        const int64_t row = gl * 8 + r;
        dst[o] = row < rows ? src[(m * rows + row) * row_bytes + (int64_t)b * 144 + byte] : (uint8_t)0;
    }
}

hipError_t launch_q4k_relayout(const uint8_t *src, uint8_t *dst, int64_t rows, int nb, int64_t gpm, int64_t total,
                               int64_t row_bytes, hipStream_t s) {
    const int64_t want = (total + 255) / 256;
    const int grid = (int)(want < 65536 ? want : 65536);
    q4k_relayout_kernel<<<grid, 256, 0, s>>>(src, dst, rows, nb, gpm, total, row_bytes);
    return hipGetLastError();
}

}  // namespace fgh
