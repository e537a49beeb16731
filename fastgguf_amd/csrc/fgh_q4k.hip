// fgh_q4k.hip - Q4_K decode matvec for gfx950 (the dominant kernel of a Q4_K_M decode layer), the
// MoE expert kernel over the same layout, and the layout's upload transform; Q5_K on the same
// layout and kernel (row order).
//
// Device layout of a Q4_K tensor (written at upload by q4k_relayout_kernel): rows in tiles of 16
// per matrix (tpm = ceil(rows / 16) tiles, the last one zero-padded). Tile t of matrix m, block b,
// is 2304 bytes (the file's 16 x 144 bytes, rearranged) at ((m * nb + b) * tpm + t) * 2304: block-
// major, so the wavefronts of a launch, all at about the same block, read one contiguous stretch
// of HBM at a time (DRAM pages stay open) rather than one stretch per tile:
//   [0, 256)     meta: row r at 16 r, the block's first 16 bytes (fp16 d, fp16 dmin, 12 bytes of
//                6-bit scales and mins)
//   [256, 2304)  quants: slot (h, L) at 256 + 1024 h + 16 L, L = 4 r + j, holds 16-byte piece
//                h ^ (j >> 1) of chunk j of row r (block bytes 16 + 32 j + 16 (h ^ (j >> 1)) ...)
// Lane L = 4 r + j of a wavefront owns chunk j of row r (32 bytes: sub-block 2j in the low nibbles,
// 2j + 1 in the high nibbles): one step of a wavefront is one block of 16 rows, three 16-byte loads
// per lane (1 KB contiguous per quant load, 256 B for the meta). Lanes j >= 2 receive the second
// half of their chunk first and read their activation halves swapped the same way, so register k
// of the lane holds the reference's AVX2 lane k (j < 2) or lane 4 + k (j >= 2) of the block: the
// row-order reduction below needs no lane-dependent selects for that half.
//
// Decode (q4k_mv_kernel): every workgroup quantizes x into LDS (Q8_K, bit-exact with
// quantize_q8k, fastgguf.c:773-793) while its first weight steps are in flight. A wavefront walks
// the blocks of its 16-row tile through a ring of R steps in registers; the activations of a step
// are LDS broadcasts (the 4 chunks of one block: no bank conflicts). Per (row, block) the exact
// integers come from v_dot4_i32_i8 and a quad reduction; the fp32 chain runs in registers in block
// order:
//   repacked order, dot_q4Kx8 (fastgguf.c:2322-2358): acc = fma(d*yd, sumi, acc),
//                   macc = fma(dmin*yd, msum, macc), out = acc - macc
//   row order, dot_q4_K_q8k (fastgguf.c:1118-1153): lane j of a row carries the reference's lane
//                   chains 2j, 2j+1 and min chain j; out = hsum8(acc) - hsum4(macc)
// Short matrices split the blocks of a tile over S wavefronts, which write fp32 records of their
// blocks to LDS; one wavefront then runs the chains over them in block order. Repacked order:
// every wavefront records {d*yd, sumi, dmin*yd, msum} per row. Row order: wavefront 0 runs its
// chains over the first run of blocks while it streams them, the others record each lane's two
// lane partials and min partial with d*yd (and dmin*yd per row), and wavefront 0 continues.
//
// Q5_K (file block {fp16 d, fp16 dmin, 12 B scales, qh[32], ql[128]}, fastgguf.c:644-667) has the
// Q4_K block's meta and nibbles plus one fifth bit per value: bit 2j (low nibble) or 2j + 1 (high
// nibble) of qh[l] for byte l of chunk j. Its (tile, block) is 2816 bytes: [0, 2304) as Q4_K's
// (nibbles from ql), then [2304, 2816) the fifth bits, lane L = 4 r + j at 2304 + 8 L: word 0 (low
// values) and word 1 (high values), bit 8 t + d = the bit of byte t of the lane's register d. It
// runs the row order of dot_q5_K_q8k (fastgguf.c:1178-1230), whose lanes, min lanes and final
// combination are those of dot_q4_K_q8k with five-bit values.
#include "fgh_internal.h"

namespace fgh {

constexpr int RB_ROWS = 16;     // rows per tile
constexpr int RB_BYTES = 2304;  // one Q4_K (tile, block): 16 x 144
__host__ __device__ constexpr int rb_bytes(int type) { return type == T_Q5_K ? Q5K_TILE : RB_BYTES; }

// LDS records of one tile in a launch that splits its blocks over s wavefronts: repacked order,
// a float4 per (block, row); row order, for the blocks after the first wavefront's ceil(nb / s),
// a float4 per (block, lane) and a float per (block, row)
__host__ __device__ constexpr size_t q4_rec_bytes(int order, int nb, int s) {
    return s == 1 ? 0 : order == 1 ? (size_t)16 * 16 * nb : (size_t)(nb - (nb + s - 1) / s) * (64 * 16 + 16 * 4);
}

__device__ __forceinline__ void q8k_load(const float *__restrict__ x, int nb, int rb, XRound &xr) {
    const int b = rb + (threadIdx.x >> 4);
    q8k_load_b(x, b, b < nb, xr);
}

__device__ __forceinline__ float dppf_xor1(float v) { return __builtin_bit_cast(float, dpp_xor1(__builtin_bit_cast(int, v))); }
__device__ __forceinline__ float dppf_xor2(float v) { return __builtin_bit_cast(float, dpp_xor2(__builtin_bit_cast(int, v))); }

__device__ __forceinline__ void q8k_store(int nb, int rb, const XRound &xr, uint8_t *act) {
    const int b = rb + (threadIdx.x >> 4);
    q8k_store_b(nb, b, b < nb, xr, act);
}

// x = silu(x) * u, value by value (silu_f, fastgguf.c:3118: x / (1 + expf(-x))); the Q8_K
// images of h rows (q4_image_kernel) form it while they quantize
__device__ __forceinline__ void xr_silu_mul(XRound &xr, const XRound &ur) {
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

// Quantizes x (nb blocks) into act with all 64 * WPG threads: q8k_begin issues the loads of the
// first two rounds (before the caller's weight loads), q8k_finish the rest and the stores.
template <int WPG>
struct XQuant {
    static constexpr int XB = 4 * WPG;  // blocks per round
    XRound r0, r1;
};
template <int WPG>
__device__ __forceinline__ void q8k_begin(XQuant<WPG> &q, const float *x, int nb) {
    q8k_load(x, nb, 0, q.r0);
    if (nb > XQuant<WPG>::XB) q8k_load(x, nb, XQuant<WPG>::XB, q.r1);  // uniform
}
template <int WPG>
__device__ __forceinline__ void q8k_finish(XQuant<WPG> &q, const float *x, int nb, uint8_t *act) {
    constexpr int XB = XQuant<WPG>::XB;
    q8k_store(nb, 0, q.r0, act);
    if (nb > XB) q8k_store(nb, XB, q.r1, act);
    for (int rb = 2 * XB; rb < nb; rb += XB) {  // rows longer than 2 * XB blocks
        q8k_load(x, nb, rb, q.r0);
        q8k_store(nb, rb, q.r0, act);
    }
}

// A wavefront quantizes the blocks 0 .. nb - 1 of its own activation row into its own LDS region
// (the MoE down launch: one wavefront per selected expert, each with its own row): rounds of 4
// blocks, 16 lanes per block. No barrier: the wavefront's LDS reads follow its own writes in
// order. q8k_wave_begin issues the loads of the first two rounds (before the weight loads).
__device__ __forceinline__ void q8k_wave_load(const float *x, int nb, int k, XRound &xr) {
    const int b = 4 * k + ((threadIdx.x & 63) >> 4);
    q8k_load_b(x, b, b < nb, xr);
}
__device__ __forceinline__ void q8k_wave_store(int nb, int k, const XRound &xr, uint8_t *act) {
    const int b = 4 * k + ((threadIdx.x & 63) >> 4);
    q8k_store_b(nb, b, b < nb, xr, act);
}
__device__ __forceinline__ void q8k_wave_begin(XQuant<1> &q, const float *x, int nb) {
    q8k_wave_load(x, nb, 0, q.r0);
    if (nb > 4) q8k_wave_load(x, nb, 1, q.r1);  // uniform
}
__device__ __forceinline__ void q8k_wave_finish(XQuant<1> &q, const float *x, int nb, uint8_t *act) {
    q8k_wave_store(nb, 0, q.r0, act);
    if (nb > 4) q8k_wave_store(nb, 1, q.r1, act);
    for (int k = 2; 4 * k < nb; ++k) {  // rows longer than 8 blocks
        q8k_wave_load(x, nb, k, q.r0);
        q8k_wave_store(nb, k, q.r0, act);
    }
}

// one step of a lane: two 16-byte pieces of its chunk (register order), its row's meta and, Q5_K
// only, the fifth bits of its low and high values
struct RbW {
    uint4 p0, p1, m;
    uint2 h;
};
// T: the (tile, block), wavefront-uniform; live = false: a ring slot past the wavefront's blocks,
// whose loads return zeros without reading memory (a buffer of 0 bytes)
template <int TYPE = T_Q4_K>
__device__ __forceinline__ void rb_load(const uint8_t *T, uint32_t lane, RbW &w, bool live = true) {
    const BufRes r = buf_res(T, live ? rb_bytes(TYPE) : 0);
    w.p0 = bld16<WNT>(r, 256 + 16 * lane);
    w.p1 = bld16<WNT>(r, 1280 + 16 * lane);
    w.m = bld16<WNT>(r, 16 * (lane >> 2));
    if (TYPE == T_Q5_K) w.h = bld8<WNT>(r, 2304 + 8 * lane);
}

// Per-lane constants of the scale extraction: chunk j, the shift selecting bytes 2(j & 1) and
// 2(j & 1) + 1 of the scale words, and an all-ones mask for lanes j >= 2.
struct RbLane {
    int j, sh;
    uint32_t hm;
};
__device__ __forceinline__ RbLane rb_lane(int lane) {
    const int j = lane & 3;
    return RbLane{j, 16 * (j & 1), j >= 2 ? 0xFFFFFFFFu : 0u};
}

// What every order needs of one lane's chunk j of one block: its activations (register order),
// the chunk's two 6-bit sub-block scales (bytes 0 and 1 of scp), the min partial of chunk j,
// m_2j bs32_2j + m_2j+1 bs32_2j+1 (the reference's min lane p = j), and yd.
struct RbIn {
    uint32_t ylo[8], yhi[8];
    uint32_t scp;
    int mt;
    float yd;
};
__device__ __forceinline__ void rb_in(const RbW &w, const uint8_t *act, int nb, int b, const RbLane &ln, RbIn &in) {
    const int hs = 16 * (ln.j >> 1);  // lanes j >= 2: second half first
    const uint8_t *yb = act + (size_t)b * 256 + 64 * ln.j;
    const uint4 l0 = *(const uint4 *)(yb + hs), l1 = *(const uint4 *)(yb + 16 - hs);
    const uint4 h0 = *(const uint4 *)(yb + 32 + hs), h1 = *(const uint4 *)(yb + 48 - hs);
    in.ylo[0] = l0.x; in.ylo[1] = l0.y; in.ylo[2] = l0.z; in.ylo[3] = l0.w;
    in.ylo[4] = l1.x; in.ylo[5] = l1.y; in.ylo[6] = l1.z; in.ylo[7] = l1.w;
    in.yhi[0] = h0.x; in.yhi[1] = h0.y; in.yhi[2] = h0.z; in.yhi[3] = h0.w;
    in.yhi[4] = h1.x; in.yhi[5] = h1.y; in.yhi[6] = h1.z; in.yhi[7] = h1.w;
    // scales and mins of sub-blocks 2j (low nibbles) and 2j+1 (high nibbles) straight from the
    // packed words u0..u2 (scale_min_k4, fastgguf.c:466-472): for j < 2 the low 6 bits of bytes 2j,
    // 2j+1 of u0 (scales) and u1 (mins); for j >= 2 the nibbles of bytes 2j-4, 2j-3 of u2 with the
    // top 2 bits of the same bytes of u0 / u1 (both formed, the lane's one selected bitwise)
    const uint32_t A = w.m.y >> ln.sh, B = w.m.z >> ln.sh, C = w.m.w >> ln.sh;
    const uint32_t sc_lo = A & 0x3f3fu, sc_hi = (C & 0x0f0fu) | ((A >> 2) & 0x3030u);
    const uint32_t mn_lo = B & 0x3f3fu, mn_hi = ((C >> 4) & 0x0f0fu) | ((B >> 2) & 0x3030u);
    in.scp = (sc_hi & ln.hm) | (sc_lo & ~ln.hm);
    const uint32_t mnp = (mn_hi & ln.hm) | (mn_lo & ~ln.hm);
    const uint32_t bq = *(const uint32_t *)((const int16_t *)(act + q4_off_s(nb)) + 8 * b + 2 * ln.j);
    in.mt = dot2_i16(__builtin_amdgcn_perm(0u, mnp, 0x0C010C00u), bq, 0);
    in.yd = ((const float *)(act + q4_off_d(nb)))[b];
}
__device__ __forceinline__ uint32_t nib_lo(uint32_t q) { return q & 0x0F0F0F0Fu; }
__device__ __forceinline__ uint32_t nib_hi(uint32_t q) { return (q >> 4) & 0x0F0F0F0Fu; }
// the values of register d of a lane: nibbles, with (Q5_K) bit 8 t + d of the fifth-bit word moved
// to bit 4 of byte t
__device__ __forceinline__ uint32_t fifth(uint32_t h, int d) {
    return (d <= 4 ? h << (4 - d) : h >> (d - 4)) & 0x10101010u;
}
template <int TYPE>
__device__ __forceinline__ uint32_t val_lo(const RbW &w, uint32_t q, int d) {
    return TYPE == T_Q5_K ? nib_lo(q) | fifth(w.h.x, d) : nib_lo(q);
}
template <int TYPE>
__device__ __forceinline__ uint32_t val_hi(const RbW &w, uint32_t q, int d) {
    return TYPE == T_Q5_K ? nib_hi(q) | fifth(w.h.y, d) : nib_hi(q);
}

// the chunk's share of the block's sumi: sc_2j sum(lo q y) + sc_2j+1 sum(hi q y) over its 32 + 32
// values (each dot sum |.| <= 32 * 31 * 127 < 2^23: 24-bit multiplies)
template <int TYPE = T_Q4_K>
__device__ __forceinline__ int rb_sumi_part(const RbW &w, const RbIn &in) {
    const uint32_t qd[8] = {w.p0.x, w.p0.y, w.p0.z, w.p0.w, w.p1.x, w.p1.y, w.p1.z, w.p1.w};
    int il = 0, ih = 0;
#pragma unroll
    for (int d = 0; d < 8; ++d) {
        il = dot4((int)val_lo<TYPE>(w, qd[d], d), (int)in.ylo[d], il);
        ih = dot4((int)val_hi<TYPE>(w, qd[d], d), (int)in.yhi[d], ih);
    }
    return __mul24((int)(in.scp & 0xFFu), il) + __mul24((int)(in.scp >> 8), ih);
}

// Row order: the reference's lane partials 2j and 2j+1 of the block (each summed over the row's
// four chunks), for lane j. Register k of a lane holds lane k (j < 2) or 4 + k (j >= 2) of its
// chunk: one exchange with lane j ^ 2 leaves lanes 0..3 (j < 2) or 4..7 summed over two chunks,
// one exchange with lane j ^ 1 the lane's own pair summed over all four.
template <int TYPE = T_Q4_K>
__device__ __forceinline__ void rb_row_lanes(const RbW &w, const RbIn &in, int j, int &u0, int &u1) {
    const uint32_t qd[8] = {w.p0.x, w.p0.y, w.p0.z, w.p0.w, w.p1.x, w.p1.y, w.p1.z, w.p1.w};
    const uint32_t sc2 = __builtin_amdgcn_perm(0u, in.scp, 0x0C010C00u);  // (sc_2j, sc_2j+1) as int16
    int lv[8];
#pragma unroll
    for (int d = 0; d < 8; ++d)  // each dot4 is at most 4 * 31 * 127 = 15748 in magnitude: an int16 pair
        lv[d] = dot2_i16(sc2, pack_i16(dot4((int)val_lo<TYPE>(w, qd[d], d), (int)in.ylo[d], 0),
                                          dot4((int)val_hi<TYPE>(w, qd[d], d), (int)in.yhi[d], 0)), 0);
    int t[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) t[k] = lv[k] + dpp_xor2(lv[4 + k]);
    const bool odd = (j & 1) != 0;
    const int k0 = odd ? t[2] : t[0], k1 = odd ? t[3] : t[1];
    const int s0 = odd ? t[0] : t[2], s1 = odd ? t[1] : t[3];
    u0 = k0 + dpp_xor1(s0);
    u1 = k1 + dpp_xor1(s1);
}

// Row order's final combination over the row's four lanes (lane j holds chains 2j, 2j+1 and min
// chain j): hsum8(acc) - hsum4(macc), fastgguf.c:797-806 and 1089-1095; valid in lane j == 0
__device__ __forceinline__ float rb_row_final(float acc_a, float acc_b, float macc) {
    const float ea = acc_a + dppf_xor2(acc_a), eb = acc_b + dppf_xor2(acc_b);  // (v0+v4), (v1+v5) | (v2+v6), (v3+v7)
    const float f = ea + eb;
    const float h8 = f + dppf_xor1(f);
    const float g = macc + dppf_xor1(macc);  // (m0+m1) | (m2+m3)
    const float h4 = g + dppf_xor2(g);
    return h8 - h4;
}

// the tensor of global tile g in a multi-tensor launch
__device__ __forceinline__ int q4_tensor_of(const MvArgs &a, int64_t g) {
    int ti = 0;
#pragma unroll
    for (int k = 1; k < 4; ++k)
        if (k < a.nt && g >= a.t[k].gfirst) ti = k;
    return ti;
}

// Decode matvec. Workgroup = TPW tiles x S wavefronts per tile (wavefront ks of a tile takes its
// ks-th run of ceil(nb / S) blocks); grid = (tiles over all tensors / TPW, tokens).
template <int ORDER, int R, int TPW, int S, bool DUMP, int TYPE = T_Q4_K, int MODE = MV_PLAIN>
__global__ __launch_bounds__(64 * TPW * S) void q4k_mv_kernel(MvArgs a) {
    constexpr bool PAIR = MODE != MV_PLAIN, ROUTE = MODE == MV_ROUTE;
    static_assert(TYPE == T_Q4_K || ORDER == 0, "Q5_K runs the row order");
    constexpr int WPG = TPW * S;
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ts = wave / S, ks = wave - ts * S;
    const int j = lane & 3, rr = lane >> 2;
    const int nb = a.nb;
    const int tok = blockIdx.y;
    // PAIR: the workgroup holds TPW / 2 row tiles of gate (a.t[0]) and up (a.t[1]), tile slots
    // 2 i (gate) and 2 i + 1 (up) over the same rows, and writes h = silu(g) * u of them
    int64_t tile;
    bool live;
    int ti;
    uint32_t lt, gpm;
    if (PAIR) {
        gpm = (uint32_t)a.t[0].gpm;
        const uint32_t rt = blockIdx.x * (TPW / 2) + (ts >> 1);
        live = rt < gpm;
        ti = ts & 1;
        lt = live ? rt : gpm - 1;
        tile = lt;
    } else {
        tile = (int64_t)blockIdx.x * TPW + ts;
        live = tile < a.groups;
        const int64_t tc = live ? tile : a.groups - 1;
        ti = q4_tensor_of(a, tc);
        lt = (uint32_t)(tc - a.t[ti].gfirst);
        gpm = (uint32_t)a.t[ti].gpm;
    }
    // (1) x for the first quantization rounds (independent of the expert)
    const float *x = a.x + (size_t)(tok / a.xdiv) * a.ldx;
    XQuant<WPG> xq;
    q8k_begin(xq, x, nb);
    // the expert of this token slot: from sel, or routed here (every wavefront routes its token
    // itself, in its own LDS buffer: no barrier; workgroup 0 of the token's first slot publishes
    // the token's experts and weights)
    int esel = 0;
    if (ROUTE) {
        const int t = tok / a.xdiv, jj = tok - t * a.xdiv;
        const bool pub = blockIdx.x == 0 && jj == 0 && wave == 0 && a.sel_out;
        float *ps = (float *)(smem + a.route_off) + (size_t)wave * 64 * MOE_EPL;
        esel = __builtin_amdgcn_readfirstlane(moe_route_wave(a.logits + (size_t)t * a.n_expert, a.n_expert, a.xdiv, ps,
                                                             pub ? a.sel_out + (size_t)t * a.xdiv : nullptr,
                                                             pub ? a.w_out + (size_t)t * a.xdiv : nullptr, jj));
    } else if (a.sel) {
        esel = a.sel[tok];
    }
    const uint32_t mi = (uint32_t)esel + lt / gpm, tt = lt % gpm;  // matrix (MoE: selected), tile
    const int nbw = (nb + S - 1) / S, bb0 = ks * nbw;
    const int nbl = max(0, min(nb, bb0 + nbw) - bb0), bl = max(nbl - 1, 0);
    const size_t bstride = (size_t)gpm * rb_bytes(TYPE);
    const uint8_t *T0 = a.t[ti].W + (((size_t)mi * nb + min(bb0, nb - 1)) * gpm + tt) * rb_bytes(TYPE);

    // (2) the ring's first R steps
    RbW ring[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rb_load<TYPE>(T0 + (size_t)min(r, bl) * bstride, lane, ring[r]);
    // (3) quantize x into LDS while the weights are in flight
    uint8_t *act = smem;
    q8k_finish(xq, x, nb, act);
    __syncthreads();

    const int64_t mrow = (int64_t)tt * RB_ROWS;  // first row of the tile in its matrix
    const int64_t obase = (int64_t)(lt / gpm) * a.t[ti].rows;
    const int64_t rows = a.t[ti].rows;
    // S > 1: records of this tile after the activations; repacked order [b][row] float4, row order
    // [b - nbw][lane] float4 {u0, u1, mt, d*yd} then [b - nbw][row] dmin*yd
    uint8_t *recb = smem + q4_act_bytes(nb) + (size_t)ts * q4_rec_bytes(ORDER, nb, S);
    float4 *rec = (float4 *)recb;
    float *recm = (float *)(recb + (size_t)(nb - nbw) * 1024);
    const RbLane ln = rb_lane(lane);
    float acc = 0.0f, acc2 = 0.0f, macc = 0.0f;
    // one block b from ring slot r
    auto step = [&](const RbW &w, int b) {
        RbIn in;
        rb_in(w, act, nb, b, ln, in);
        const float fd = fp16_bits_to_f32(w.m.x & 0xFFFF) * in.yd;
        const float fdm = fp16_bits_to_f32(w.m.x >> 16) * in.yd;
        int sumi = 0, msum = 0;
        if (ORDER == 1 || DUMP) {
            sumi = sum4_i32(rb_sumi_part<TYPE>(w, in));
            msum = sum4_i32(in.mt);
        }
        if (ORDER == 1) {
            if (S == 1) {
                acc = __builtin_fmaf(fd, (float)sumi, acc);
                macc = __builtin_fmaf(fdm, (float)msum, macc);
            } else if (j == 0) {
                rec[(size_t)b * RB_ROWS + rr] = make_float4(fd, (float)sumi, fdm, (float)msum);
            }
        } else {
            int u0, u1;
            rb_row_lanes<TYPE>(w, in, j, u0, u1);
            if (S == 1 || ks == 0) {
                acc = __builtin_fmaf(fd, (float)u0, acc);
                acc2 = __builtin_fmaf(fd, (float)u1, acc2);
                macc = __builtin_fmaf(fdm, (float)in.mt, macc);
            } else {
                rec[(size_t)(b - nbw) * 64 + lane] = make_float4((float)u0, (float)u1, (float)in.mt, fd);
                if (j == 0) recm[(size_t)(b - nbw) * RB_ROWS + rr] = fdm;
            }
        }
        if (DUMP && live && j == 0 && mrow + rr < rows) {
            const size_t di = (size_t)(obase + mrow + rr) * nb + b;
            a.dump_s[di] = sumi;
            a.dump_m[di] = msum;
        }
    };
    // whole rounds of R blocks as straight-line code (the steps interleave), refilling the ring
    // (a refill past the wavefront's last block loads nothing: re-reading the last block missed
    // the caches under nontemporal loads, 2 % more HBM traffic and 1.5-2 % longer launches); then
    // the last nbl % R blocks already in the ring
    int b0 = 0;
    for (; b0 + R <= nbl; b0 += R) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            step(ring[r], bb0 + b0 + r);
            rb_load<TYPE>(T0 + (size_t)min(b0 + r + R, bl) * bstride, lane, ring[r], b0 + r + R <= bl);
        }
    }
#pragma unroll
    for (int r = 0; r < R - 1; ++r)
        if (b0 + r < nbl) step(ring[r], bb0 + b0 + r);  // uniform
    // the row results: lane ri(lane) holds row `row` of the tile when has
    float out = 0.0f;
    bool has;
    int row;
    if (S > 1) {
        __syncthreads();
        if (ORDER == 1) {
            has = ks == 0 && lane < RB_ROWS;
            row = lane;
            if (has) {
                const float4 *rr4 = rec + lane;
                int b = 0;
                for (; b + 4 <= nb; b += 4) {
                    float4 p[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) p[u] = rr4[(size_t)(b + u) * RB_ROWS];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        acc = __builtin_fmaf(p[u].x, p[u].y, acc);
                        macc = __builtin_fmaf(p[u].z, p[u].w, macc);
                    }
                }
                for (; b < nb; ++b) {
                    const float4 p = rr4[(size_t)b * RB_ROWS];
                    acc = __builtin_fmaf(p.x, p.y, acc);
                    macc = __builtin_fmaf(p.z, p.w, macc);
                }
                out = acc - macc;
            }
        } else {  // the row chains over the other wavefronts' blocks
            has = ks == 0 && j == 0;
            row = rr;
            if (ks == 0) {
                int b = nbw;
                for (; b + 4 <= nb; b += 4) {
                    float4 p[4];
                    float m[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        p[u] = rec[(size_t)(b + u - nbw) * 64 + lane];
                        m[u] = recm[(size_t)(b + u - nbw) * RB_ROWS + rr];
                    }
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        acc = __builtin_fmaf(p[u].w, p[u].x, acc);
                        acc2 = __builtin_fmaf(p[u].w, p[u].y, acc2);
                        macc = __builtin_fmaf(m[u], p[u].z, macc);
                    }
                }
                for (; b < nb; ++b) {
                    const float4 p = rec[(size_t)(b - nbw) * 64 + lane];
                    const float m = recm[(size_t)(b - nbw) * RB_ROWS + rr];
                    acc = __builtin_fmaf(p.w, p.x, acc);
                    acc2 = __builtin_fmaf(p.w, p.y, acc2);
                    macc = __builtin_fmaf(m, p.z, macc);
                }
                out = rb_row_final(acc, acc2, macc);
            }
        }
    } else {
        has = j == 0;
        row = rr;
        out = ORDER == 1 ? acc - macc : rb_row_final(acc, acc2, macc);
    }
    const bool store = has && live && mrow + row < rows;
    if (PAIR) {
        // gate tile -> LDS (with routing, its buffers are free: every wavefront routed before the
        // barrier after the quantization); up tile: h = silu(g) * u (silu_f, fastgguf.c:3118)
        float *pg = (float *)(smem + a.route_off) + (ts >> 1) * RB_ROWS;
        if (ti == 0 && has) pg[row] = out;
        __syncthreads();
        if (ti == 1 && store) {
            const float g = pg[row];
            a.t[0].y[(size_t)tok * a.ldy + mrow + row] = g / (1.0f + expf_ref(-g)) * out;
        }
    } else if (store) {
        a.t[ti].y[(size_t)tok * a.ldy + obase + mrow + row] = out;
    }
}

template <int ORDER, int R, int TPW, int S, int TYPE>
static hipError_t q4_launch(const MvArgs &a, int ntok, size_t lds, hipStream_t s) {
    const unsigned wg = (unsigned)((a.groups + TPW - 1) / TPW);
    if (a.dump_s) {
        q4k_mv_kernel<ORDER, R, TPW, S, true, TYPE><<<dim3(wg, ntok), 64 * TPW * S, lds, s>>>(a);
        return hipGetLastError();
    }
    if (a.logits) {
        q4k_mv_kernel<ORDER, R, TPW, S, false, TYPE, MV_ROUTE><<<dim3(wg, ntok), 64 * TPW * S, lds, s>>>(a);
        return hipGetLastError();
    }
    if (a.pair) {
        q4k_mv_kernel<ORDER, R, TPW, S, false, TYPE, MV_PAIR><<<dim3(wg, ntok), 64 * TPW * S, lds, s>>>(a);
        return hipGetLastError();
    }
    q4k_mv_kernel<ORDER, R, TPW, S, false, TYPE><<<dim3(wg, ntok), 64 * TPW * S, lds, s>>>(a);
    return hipGetLastError();
}
template <int ORDER, int TPW, int S, int TYPE = T_Q4_K>
static hipError_t q4_launch_r(int R, const MvArgs &a, int ntok, size_t lds, hipStream_t s) {
    return R == 2 ? q4_launch<ORDER, 2, TPW, S, TYPE>(a, ntok, lds, s) : q4_launch<ORDER, 4, TPW, S, TYPE>(a, ntok, lds, s);
}

// LDS of a launch: the activations, and with a block split the records of TPW tiles
static size_t q4_lds(int order, int nb, int tpw, int s) { return q4_act_bytes(nb) + (size_t)tpw * q4_rec_bytes(order, nb, s); }
static int q4_tpw(int s) { return s == 1 ? 4 : s == 2 ? 2 : 1; }

size_t q4k_lds_bytes(int order, int nb) { return q4_lds(order, nb, 4, 1); }

// Launch shape (measured on MI355X at the decode-layer shapes). Wavefronts per tile S: launches of
// at most 768 tiles (tiles x tokens) split the blocks of a tile over up to 8 wavefronts, as many
// as keep the launch within 2048 wavefronts with 2 blocks or more each, or (Q4_K) within 3072 with
// 4 blocks or more each (repacked 11008 x 4096, 688 tiles: 4 ways, 7.30 -> 6.87 us against 2;
// 5120 x 13824, 320 tiles: 8 ways, 12.7 -> 11.6 us against 4; Q5_K does better without), the LDS within
// the 160 KiB of a workgroup and every workgroup resident at once; larger launches keep one
// wavefront per tile. Tiles per workgroup: 4, 2 or 1 for S = 1, 2 or more, and 2 for a 4-way
// split of 9/8 to 2 tiles per compute unit. Ring depth R: 2 steps
// for split launches (the repacked down projection 14336 -> 4096 alone runs 1 % faster at depth 4,
// 9.09 against 9.19 us, and 5120 x 13824 9 % slower) and for unsplit ones of 1024 tiles or more
// over rows shorter than 32 blocks (enough loads in flight across the chip), 4 otherwise.
// (Before, splits kept 4 blocks per
// wavefront and depth 4 unless the launch had 1024 wavefronts over short rows; measured, graph of
// back-to-back launches: O 4096 x 4096 4.78 -> 4.59 us, 2048 x 2048 4.41 -> 3.59, 4096 x 8192
// 6.97 -> 6.02, the row order's down 4096 x 14336 10.1 -> 9.6, Q5_K's 11.4 -> 10.7; QKV, gate,
// the repacked down and the paired launches unchanged.)
template <int ORDER, int TYPE>
static hipError_t q4_launch_s(int S, int TPW, int R, const MvArgs &a, int ntok, size_t lds, hipStream_t s) {
    switch (S) {
    case 1: return q4_launch_r<ORDER, 4, 1, TYPE>(R, a, ntok, lds, s);
    case 2: return q4_launch_r<ORDER, 2, 2, TYPE>(R, a, ntok, lds, s);
    case 4:
        return TPW == 2 ? q4_launch_r<ORDER, 2, 4, TYPE>(R, a, ntok, lds, s)
                        : q4_launch_r<ORDER, 1, 4, TYPE>(R, a, ntok, lds, s);
    default: return q4_launch_r<ORDER, 1, 8, TYPE>(R, a, ntok, lds, s);
    }
}
MvShape q4k_matvec_shape(int type, int order, int64_t tiles, int nb, int num_cu) {
    if (type == T_Q5_K) order = 0;  // no repacked order for Q5_K
    int S = 1;
    if (tiles <= 768)  // (the MoE batch-1 gate/up launch has 768: 14.98 -> 14.33 us with S = 2)
        while (S < 8 &&
               ((tiles * 2 * S <= 2048 && nb >= 4 * S) || (type == T_Q4_K && tiles * 2 * S <= 3072 && nb >= 8 * S)) &&
               q4_lds(order, nb, q4_tpw(2 * S), 2 * S) <= GEMM_LDS_MAX &&
               all_resident((tiles + q4_tpw(2 * S) - 1) / q4_tpw(2 * S), 2 * S * q4_tpw(2 * S),
                            q4_lds(order, nb, q4_tpw(2 * S), 2 * S), num_cu))
            S *= 2;
    const int R = S > 1 || (nb < 32 && tiles >= 1024) ? 2 : 4;
    // a 4-way split of 9/8 to 2 tiles per compute unit holds 2 tiles per workgroup (Q4_K repacked
    // 5120 x 5120, 320 tiles: 6.78 -> 5.96 us, Q5_K 7.45 -> 6.76; 4608 x 5120 6.78 -> 5.91; rows
    // of 16 blocks within 2 % either way from 288 tiles up; 257 tiles 6 % slower)
    int tpw = q4_tpw(S);
    if (S == 4 && tiles * 8 >= 9 * (int64_t)num_cu && tiles <= 2 * num_cu &&
        q4_lds(order, nb, 2, 4) <= GEMM_LDS_MAX && all_resident((tiles + 1) / 2, 8, q4_lds(order, nb, 2, 4), num_cu))
        tpw = 2;
    return MvShape{S, R, tpw, q4_lds(order, nb, tpw, S)};
}

// paired launches: after the activations and records, with routing each wavefront's routing
// buffer, without it the gate tiles' rows
static uint32_t q4_route_off(const MvShape &sh) { return (uint32_t)((sh.lds + 15) & ~(size_t)15); }
static size_t q4_route_lds(const MvShape &sh) { return q4_route_off(sh) + (size_t)sh.S * sh.TPW * 64 * MOE_EPL * 4; }
static size_t q4_pair_lds(const MvShape &sh) { return q4_route_off(sh) + (size_t)sh.TPW / 2 * RB_ROWS * 4; }

// paired launches hold gate and up tiles in one workgroup: at most 2 wavefronts per tile
static MvShape q4_pair_shape(int type, int order, int64_t tiles, int nb, int num_cu) {
    MvShape sh = q4k_matvec_shape(type, type == T_Q5_K ? 0 : order, tiles, nb, num_cu);
    if (sh.S > 2) {
        sh.S = 2;
        sh.TPW = q4_tpw(2);
        sh.lds = q4_lds(type == T_Q5_K ? 0 : order, nb, sh.TPW, sh.S);
    }
    return sh;
}

bool q4k_route_fits(int type, int order, int64_t tiles, int nb, int num_cu) {
    const MvShape sh = q4_pair_shape(type, order, tiles, nb, num_cu);
    return sh.lds <= (sh.S == 1 ? (size_t)65536 : GEMM_LDS_MAX) && q4_route_lds(sh) <= GEMM_LDS_MAX;
}

hipError_t launch_q4k_matvec(int type, int order, const MvArgs &a, int ntok, int num_cu, hipStream_t s) {
    if (type == T_Q5_K) order = 0;
    const bool pair = a.logits || a.pair;
    const MvShape sh = pair ? q4_pair_shape(type, order, a.groups * ntok, a.nb, num_cu)
                            : q4k_matvec_shape(type, order, a.groups * ntok, a.nb, num_cu);
    if (sh.lds > (sh.S == 1 ? (size_t)65536 : GEMM_LDS_MAX)) return hipErrorInvalidValue;
    MvArgs b = a;
    size_t lds = sh.lds;
    if (pair) {  // gate and up (of the selected experts), h = silu(g) * u into a.t[0].y
        if (a.nt != 2 || a.t[0].gpm != a.t[1].gpm || a.t[0].rows != a.t[1].rows || a.dump_s)
            return hipErrorInvalidValue;
        if (a.logits && (a.sel || !a.sel_out || !a.w_out || a.n_expert < 1 || a.n_expert > 64 * MOE_EPL ||
                         a.xdiv < 1 || a.xdiv > a.n_expert || a.xdiv > 64 || ntok % a.xdiv))
            return hipErrorInvalidValue;
        b.route_off = q4_route_off(sh);
        b.groups = 2 * a.t[0].gpm;  // TPW / 2 row tiles per workgroup
        lds = a.logits ? q4_route_lds(sh) : q4_pair_lds(sh);
        if (lds > GEMM_LDS_MAX) return hipErrorInvalidValue;
    }
    if (type == T_Q5_K) return q4_launch_s<0, T_Q5_K>(sh.S, sh.TPW, sh.R, b, ntok, lds, s);
    if (order == 0) return q4_launch_s<0, T_Q4_K>(sh.S, sh.TPW, sh.R, b, ntok, lds, s);
    return q4_launch_s<1, T_Q4_K>(sh.S, sh.TPW, sh.R, b, ntok, lds, s);
}

// MoE down projection and combine of one token in one launch (moe_ffn, fastgguf.c:4620-4635):
// workgroup = one 16-row tile of the output x the token's k selected experts, wavefront j = expert
// sel[t k + j]. Wavefront j quantizes its own row h_j (a.x = the h rows of the token's slots) into
// its own LDS region, runs the row order of dot_q4_K_q8k (or dot_q5_K_q8k)
// over the expert's blocks and parks each row's dot product in LDS; wavefront 0 then forms
// y = fma(w_j, d_j, s) over j in order, the reference's sum (gcc contracts `s += w * dot`).
// grid = (16-row tiles of one expert matrix, tokens); a.t[0] = {down, y}, a.ldy = y's token stride.
template <int R, int TYPE>
__global__ __launch_bounds__(512) void q4k_moe_down_kernel(MvArgs a, const float *__restrict__ wts, int k) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int jw = __builtin_amdgcn_readfirstlane(tid >> 6);  // the selected expert of this wavefront
    const int j = lane & 3, rr = lane >> 2;
    const int nb = a.nb, tok = blockIdx.y, slot = tok * k + jw;
    const uint32_t tt = blockIdx.x, gpm = (uint32_t)a.t[0].gpm;
    const uint32_t mi = (uint32_t)a.sel[slot];
    const size_t bstride = (size_t)gpm * rb_bytes(TYPE);
    const uint8_t *T0 = a.t[0].W + ((size_t)mi * nb * gpm + tt) * rb_bytes(TYPE);
    uint8_t *act = smem + (size_t)jw * q4_act_bytes(nb);
    float *dots = (float *)(smem + (size_t)k * q4_act_bytes(nb));  // [k][16]
    const float *x = a.x + (size_t)slot * a.ldx;
    XQuant<1> xq;
    q8k_wave_begin(xq, x, nb);
    const int bl = nb - 1;
    RbW ring[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rb_load<TYPE>(T0 + (size_t)min(r, bl) * bstride, lane, ring[r], r < nb);
    q8k_wave_finish(xq, x, nb, act);
    const RbLane ln = rb_lane(lane);
    float acc = 0.0f, acc2 = 0.0f, macc = 0.0f;
    auto step = [&](const RbW &w, int b) {
        RbIn in;
        rb_in(w, act, nb, b, ln, in);
        const float fd = fp16_bits_to_f32(w.m.x & 0xFFFF) * in.yd;
        const float fdm = fp16_bits_to_f32(w.m.x >> 16) * in.yd;
        int u0, u1;
        rb_row_lanes<TYPE>(w, in, j, u0, u1);
        acc = __builtin_fmaf(fd, (float)u0, acc);
        acc2 = __builtin_fmaf(fd, (float)u1, acc2);
        macc = __builtin_fmaf(fdm, (float)in.mt, macc);
    };
    int b0 = 0;
    for (; b0 + R <= nb; b0 += R) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            step(ring[r], b0 + r);
            rb_load<TYPE>(T0 + (size_t)min(b0 + r + R, bl) * bstride, lane, ring[r], b0 + r + R < nb);
        }
    }
#pragma unroll
    for (int r = 0; r < R - 1; ++r)
        if (b0 + r < nb) step(ring[r], b0 + r);  // uniform
    const float out = rb_row_final(acc, acc2, macc);
    if (j == 0) dots[jw * 16 + rr] = out;
    __syncthreads();
    if (jw == 0 && lane < RB_ROWS) {
        const int64_t row = (int64_t)tt * RB_ROWS + lane;
        float sum = 0.0f;
        for (int jj = 0; jj < k; ++jj) sum = __builtin_fmaf(wts[(size_t)tok * k + jj], dots[jj * 16 + lane], sum);
        if (row < a.t[0].rows) a.t[0].y[(size_t)tok * a.ldy + row] = sum;
    }
}

size_t q4k_moe_down_lds(int nb, int k) { return (size_t)k * q4_act_bytes(nb) + (size_t)k * RB_ROWS * 4; }

hipError_t launch_q4k_moe_down(int type, const MvArgs &a, const float *wts, int k, int ntok, hipStream_t s) {
    const size_t lds = q4k_moe_down_lds(a.nb, k);
    if (!a.sel || !a.x || k < 1 || k > 8 || ntok < 1 || lds > GEMM_LDS_MAX || a.t[0].gpm < 1)
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)a.t[0].gpm, (unsigned)ntok);
    if (type == T_Q5_K) q4k_moe_down_kernel<4, T_Q5_K><<<grid, 64 * k, lds, s>>>(a, wts, k);
    else q4k_moe_down_kernel<4, T_Q4_K><<<grid, 64 * k, lds, s>>>(a, wts, k);
    return hipGetLastError();
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

// The grouped MoE path's first launch, one workgroup of two wavefronts per token t: wavefront 1
// forms the Q8_K image of x row t (q4_image_kernel's blocks, 8 at a time: the loads of two rounds
// in flight before the barrier, so they overlap the routing), wavefront 0 routes the token
// (moe_route_wave: sel, w) and, after the barrier (which also makes its sel stores visible to its
// own lanes), files each selected slot t k + j in its expert's bucket: bucket[e * cap + position],
// cnt[e] counting. cap = tokens * k: a token whose probabilities are not all finite (NaN or
// infinite logits) can select one expert several times, as the reference's repeated argmax does,
// so a bucket holds up to every slot of the call. The order inside a bucket is whatever the
// atomics give; no result depends on it. cnt starts at zero and moe_combine_kernel, the path's
// last launch, clears it. (One wavefront doing both, its quantization rounds one after another:
// 7.4 us at config 5.)
__global__ __launch_bounds__(128) void moe_prep_kernel(const float *__restrict__ x, int64_t ldx, int nb,
                                                       uint8_t *__restrict__ img, const float *__restrict__ logits,
                                                       int n_expert, int k, int32_t *__restrict__ sel,
                                                       float *__restrict__ w, int32_t *__restrict__ cnt,
                                                       int32_t *__restrict__ bucket, int cap) {
    __shared__ __align__(16) float ps[64 * MOE_EPL];
    const int t = blockIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6), lane = (int)threadIdx.x & 63;
    const float *xr = x + (size_t)t * ldx;
    uint8_t *ir = img + (size_t)t * q4_act_bytes(nb);
    const int bl = lane >> 4;  // this lane's block of a round of 4
    XRound xa, xb;
    if (wave == 1) {
        q8k_load_b(xr, bl, bl < nb, xa);
        q8k_load_b(xr, 4 + bl, 4 + bl < nb, xb);
    } else {
        moe_route_wave(logits + (size_t)t * n_expert, n_expert, k, ps, sel + (size_t)t * k, w + (size_t)t * k, 0);
    }
    __syncthreads();
    if (wave == 0) {
        if (lane < k) {
            const int slot = t * k + lane, e = sel[slot];
            bucket[(size_t)e * cap + atomicAdd(&cnt[e], 1)] = slot;
        }
        return;
    }
    q8k_store_b(nb, bl, bl < nb, xa, ir);
    q8k_store_b(nb, 4 + bl, 4 + bl < nb, xb, ir);
    for (int b0 = 8; b0 < nb; b0 += 8) {  // rows of more than 8 blocks
        q8k_load_b(xr, b0 + bl, b0 + bl < nb, xa);
        q8k_load_b(xr, b0 + 4 + bl, b0 + 4 + bl < nb, xb);
        q8k_store_b(nb, b0 + bl, b0 + bl < nb, xa, ir);
        q8k_store_b(nb, b0 + 4 + bl, b0 + 4 + bl < nb, xb, ir);
    }
}

hipError_t launch_moe_prep(const float *x, int64_t ldx, int nb, uint8_t *img, const float *logits, int n_expert,
                           int k, int n_tok, int32_t *sel, float *w, int32_t *cnt, int32_t *bucket, hipStream_t s) {
    if (n_expert < 1 || n_expert > 64 * MOE_EPL || k < 1 || k > n_expert || k > 64 || nb < 1 || n_tok < 1)
        return hipErrorInvalidValue;
    moe_prep_kernel<<<n_tok, 128, 0, s>>>(x, ldx, nb, img, logits, n_expert, k, sel, w, cnt, bucket, n_tok * k);
    return hipGetLastError();
}

// MoE expert matvecs grouped by expert (row order, dot_q4_K_q8k): workgroup (x, y) takes tiles
// 4x..4x+3 (one per wavefront, over the launch's tensors) of the matrix of expert y and every
// slot in its bucket (moe_prep_kernel; a workgroup of an expert no token selected exits). For every
// chunk of MOE_TC slots the workgroup copies their activation images (q4_image_kernel, row
// slot / a.xdiv) into LDS; each wavefront then walks the blocks of its tile through a ring of
// MOE_R steps, forms a block's weight-side values once (nibbles, scale and min pairs, d, dmin) and
// runs the decode kernel's row-order lane sums and fp32 chains for every slot of the chunk (the
// chains of a slot in block order, as the per-token matvec does). Tensor i of a.t: output rows
// y_i[slot * ldy].
constexpr int MOE_TC = 8, MOE_R = 2;

// the weight side of one (tile, block) for the row order: chunk j's nibbles, its (sc_2j, sc_2j+1)
// and (m_2j, m_2j+1) as int16 pairs, d and dmin
struct RbWSide {
    uint32_t lo[8], hi[8];
    uint32_t sc2, mn2;
    float d, dmin;
};
__device__ __forceinline__ void rb_wside(const RbW &w, const RbLane &ln, RbWSide &ws) {
    const uint32_t qd[8] = {w.p0.x, w.p0.y, w.p0.z, w.p0.w, w.p1.x, w.p1.y, w.p1.z, w.p1.w};
#pragma unroll
    for (int d = 0; d < 8; ++d) {
        ws.lo[d] = nib_lo(qd[d]);
        ws.hi[d] = nib_hi(qd[d]);
    }
    const uint32_t A = w.m.y >> ln.sh, B = w.m.z >> ln.sh, C = w.m.w >> ln.sh;  // as rb_in
    const uint32_t sc_lo = A & 0x3f3fu, sc_hi = (C & 0x0f0fu) | ((A >> 2) & 0x3030u);
    const uint32_t mn_lo = B & 0x3f3fu, mn_hi = ((C >> 4) & 0x0f0fu) | ((B >> 2) & 0x3030u);
    ws.sc2 = __builtin_amdgcn_perm(0u, (sc_hi & ln.hm) | (sc_lo & ~ln.hm), 0x0C010C00u);
    ws.mn2 = __builtin_amdgcn_perm(0u, (mn_hi & ln.hm) | (mn_lo & ~ln.hm), 0x0C010C00u);
    ws.d = fp16_bits_to_f32(w.m.x & 0xFFFF);
    ws.dmin = fp16_bits_to_f32(w.m.x >> 16);
}

template <int TC>
__global__ __launch_bounds__(256) void q4k_moe_kernel(MvArgs a, const int32_t *__restrict__ cnt,
                                                      const int32_t *__restrict__ slots, int cap,
                                                      const uint8_t *__restrict__ img) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 3, rr = lane >> 2;
    const int nb = a.nb;
    const int expert = blockIdx.y, count = cnt[expert];
    if (count == 0) return;  // whole workgroup: no token selected this expert
    const int first = expert * cap;
    const int64_t tile = (int64_t)blockIdx.x * 4 + wave;
    const bool live = tile < a.groups;
    const int64_t tc = live ? tile : a.groups - 1;
    const int ti = q4_tensor_of(a, tc);
    const int64_t lt = tc - a.t[ti].gfirst;  // tile within the matrix
    const size_t bstride = (size_t)a.t[ti].gpm * RB_BYTES;
    const uint8_t *T0 = a.t[ti].W + (size_t)expert * nb * bstride + (size_t)lt * RB_BYTES;
    const int bl = nb - 1;
    const size_t actb = q4_act_bytes(nb);
    const int units = (int)(actb / 16);
    const int64_t row = lt * RB_ROWS + rr;
    const bool store = live && j == 0 && row < a.t[ti].rows;
    const RbLane ln = rb_lane(lane);
    const int hs = 16 * (j >> 1);  // lanes j >= 2: second half of their activations first (as rb_in)
    RbW ring[MOE_R];
    for (int c0 = 0; c0 < count; c0 += TC) {
        const int nc = min(TC, count - c0);
#pragma unroll
        for (int r = 0; r < MOE_R; ++r) rb_load(T0 + (size_t)min(r, bl) * bstride, lane, ring[r]);
        // the chunk's activation images (rows slot / xdiv) into LDS
        for (int i = tid; i < nc * units; i += 256) {
            const int c = i / units, o = i - c * units;
            const int slot = slots[first + c0 + c];
            ((uint4 *)(smem + (size_t)c * actb))[o] = ((const uint4 *)(img + (size_t)(slot / a.xdiv) * actb))[o];
        }
        __syncthreads();
        float acc[TC], acc2[TC], macc[TC];
#pragma unroll
        for (int c = 0; c < TC; ++c) acc[c] = acc2[c] = macc[c] = 0.0f;
        auto blk = [&](const RbW &w, int b) {
            RbWSide ws;
            rb_wside(w, ln, ws);
#pragma unroll
            for (int c = 0; c < TC; ++c) {
                if (c < nc) {  // uniform
                    const uint8_t *act = smem + (size_t)c * actb;
                    const uint8_t *yb = act + (size_t)b * 256 + 64 * j;
                    const uint4 l0 = *(const uint4 *)(yb + hs), l1 = *(const uint4 *)(yb + 16 - hs);
                    const uint4 h0 = *(const uint4 *)(yb + 32 + hs), h1 = *(const uint4 *)(yb + 48 - hs);
                    const uint32_t ylo[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
                    const uint32_t yhi[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
                    const uint32_t bq = *(const uint32_t *)((const int16_t *)(act + q4_off_s(nb)) + 8 * b + 2 * j);
                    const float yd = ((const float *)(act + q4_off_d(nb)))[b];
                    int lv[8];
#pragma unroll
                    for (int d = 0; d < 8; ++d)
                        lv[d] = dot2_i16(ws.sc2, pack_i16(dot4((int)ws.lo[d], (int)ylo[d], 0),
                                                          dot4((int)ws.hi[d], (int)yhi[d], 0)), 0);
                    // the row order's lane pairs (as rb_row_lanes)
                    int t4[4];
#pragma unroll
                    for (int k = 0; k < 4; ++k) t4[k] = lv[k] + dpp_xor2(lv[4 + k]);
                    const bool odd = (j & 1) != 0;
                    const int k0 = odd ? t4[2] : t4[0], k1 = odd ? t4[3] : t4[1];
                    const int s0 = odd ? t4[0] : t4[2], s1 = odd ? t4[1] : t4[3];
                    const int u0 = k0 + dpp_xor1(s0), u1 = k1 + dpp_xor1(s1);
                    const int mt = dot2_i16(ws.mn2, bq, 0);
                    const float fd = ws.d * yd, fdm = ws.dmin * yd;
                    acc[c] = __builtin_fmaf(fd, (float)u0, acc[c]);
                    acc2[c] = __builtin_fmaf(fd, (float)u1, acc2[c]);
                    macc[c] = __builtin_fmaf(fdm, (float)mt, macc[c]);
                }
            }
        };
        int b0 = 0;
        for (; b0 + MOE_R <= nb; b0 += MOE_R) {
#pragma unroll
            for (int r = 0; r < MOE_R; ++r) {
                blk(ring[r], b0 + r);
                rb_load(T0 + (size_t)min(b0 + r + MOE_R, bl) * bstride, lane, ring[r]);
            }
        }
#pragma unroll
        for (int r = 0; r < MOE_R - 1; ++r)
            if (b0 + r < nb) blk(ring[r], b0 + r);  // uniform
#pragma unroll
        for (int c = 0; c < TC; ++c) {
            if (c < nc) {  // uniform
                const float out = rb_row_final(acc[c], acc2[c], macc[c]);
                if (store) a.t[ti].y[(size_t)slots[first + c0 + c] * a.ldy + row] = out;
            }
        }
        __syncthreads();  // the next chunk reuses the activations
    }
}

size_t q4k_moe_lds_bytes(int nb) { return MOE_TC * q4_act_bytes(nb); }
// the widest rows whose chunk of activation images fits 64 KiB of LDS
int q4k_moe_max_blocks() {
    int nb = 1;
    while (q4k_moe_lds_bytes(nb + 1) <= 65536) ++nb;
    return nb;
}

// a.groups = tiles of one matrix over all tensors; grid.y = experts
hipError_t launch_q4k_moe(const MvArgs &a, const int32_t *cnt, const int32_t *buckets, int cap, int n_expert,
                          const uint8_t *img, hipStream_t s) {
    const size_t lds = q4k_moe_lds_bytes(a.nb);
    if (a.nb < 1 || lds > 65536 || n_expert < 1 || cap < 1) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((a.groups + 3) / 4), (unsigned)n_expert);
    q4k_moe_kernel<MOE_TC><<<grid, 256, lds, s>>>(a, cnt, buckets, cap, img);
    return hipGetLastError();
}

// upload-time re-layout of Q4_K / Q5_K rows into the tile layout above; one thread per destination
// byte (a Q5_K fifth-bit byte gathers bit 2j or 2j + 1 of 8 bytes of the block's qh)
__global__ void q4k_relayout_kernel(int type, const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, int64_t rows,
                                    int nb, int64_t tpm, int64_t total, int64_t row_bytes) {
    const int TB = rb_bytes(type), BB = type == T_Q5_K ? 176 : 144, QOFF = type == T_Q5_K ? 48 : 16;
    for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < total; o += (int64_t)gridDim.x * blockDim.x) {
        const int64_t tb = o / TB;
        const int ob = (int)(o - tb * TB);
        const int64_t mb = tb / tpm, tl = tb - mb * tpm;  // (matrix, block), tile
        const int64_t m = mb / nb;
        const int b = (int)(mb - m * nb);
        int r, byte = -1, jj = 0, bi = 0;
        if (ob < 256) {
            r = ob >> 4;
            byte = ob & 15;
        } else if (ob < 2304) {
            const int u = ob - 256, hh = u >> 10, L = (u >> 4) & 63;
            jj = L & 3;
            r = L >> 2;
            byte = QOFF + 32 * jj + 16 * (hh ^ (jj >> 1)) + (u & 15);
        } else {  // Q5_K: byte bi of lane L's fifth bits (word bi >> 2: low / high values, byte t = bi & 3)
            const int u = ob - 2304, L = u >> 3;
            jj = L & 3;
            r = L >> 2;
            bi = u & 7;
        }
        const int64_t row = tl * RB_ROWS + r;
        int v = 0;
        if (row < rows) {
            const uint8_t *p = src + (m * rows + row) * row_bytes + (int64_t)b * BB;
            if (byte >= 0) {
                v = p[byte];
            } else {  // bit d: the fifth bit of byte t of register d, chunk byte 16 ((d >> 2) ^ (j >> 1)) + 4 (d & 3) + t
                const int sh = 2 * jj + (bi >> 2), t = bi & 3;
#pragma unroll
                for (int d = 0; d < 8; ++d) v |= ((p[16 + 16 * ((d >> 2) ^ (jj >> 1)) + 4 * (d & 3) + t] >> sh) & 1) << d;
            }
        }
        dst[o] = (uint8_t)v;
    }
}

hipError_t launch_q4k_relayout(int type, const uint8_t *src, uint8_t *dst, int64_t rows, int nb, int64_t tpm,
                               int64_t total, int64_t row_bytes, hipStream_t s) {
    const int64_t want = (total + 255) / 256;
    const int grid = (int)(want < 65536 ? want : 65536);
    q4k_relayout_kernel<<<grid, 256, 0, s>>>(type, src, dst, rows, nb, tpm, total, row_bytes);
    return hipGetLastError();
}

}  // namespace fgh
