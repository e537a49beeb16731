// fgh_moemm.hip - MoE expert matvecs grouped by expert on int8 MFMA (the several-token path of
// moe_ffn, fastgguf.c:4588-4642, whose expert rows the reference reads token by token through
// dot_row -> dot_q4_K_q8k, 5088-5091 and 1118-1153).
//
// Bit-exact row order on MFMA. dot_q4_K_q8k's fp32 result is not a function of a block's total
// integer: its AVX2 accumulator lane k (k = 0..7) sums sumi_k = sum_g sc_g * (sum of q * y over
// positions 4k..4k+3 of sub-block g), one fp32 chain per lane (acc_k = fma(d * yd, sumi_k, acc_k)),
// four min chains (macc_p = fma(dmin * yd, m_2p bs_2p + m_2p+1 bs_2p+1, macc_p)), then
// hsum_ps(acc) - hsum128_ps(macc). So the MFMA has to deliver the eight lane partials separately.
// v_mfma_i32_16x16x64_i8 with
//   A = activations: row m = 4 s + q holds slot s (of a group of 4 slots) restricted to the
//       positions of lane group 4 h + q, zeros elsewhere, for the two halves h of the block
//   B = weights: column n = row n of the 16-row tile, the decode layout's 16-byte pieces,
//       pre-scaled by the split sub-block scales (sc = 8 sh + sl, the prompt GEMM's two chains:
//       isum = 8 C_h + C_l, every product within int8)
// makes D_h[4 s + q][n] = the lane-(4 h + q) partial of (slot s, row n), exactly. K-step (h, i):
// lane (kg, m / n) takes piece h (positions 16 h .. 16 h + 15) of sub-block 2 kg + i (chunk kg,
// low or high nibbles): its register e covers positions 16 h + 4 e .. + 3, i.e. lane group 4 h + e,
// and the A lane keeps only register e = q. Two halves x two nibble steps x two chains = 8 MFMAs
// per (4 slots, 16 rows, block); the output lane l = 16 s + n then holds all eight lane partials
// and, from two int16 dot products per pair, the four min partials of its (slot, row), so the
// reference's chains and final horizontal sums run in that one lane, in block order: bit for bit
// the per-token matvec's result.
//
// The masked A fragments are built once per workgroup and chunk of slots in LDS from the slots'
// Q8_K images (q4_image_kernel / moe_prep_kernel layout): per (block, group of 4 slots, K-step)
// the 4 activation bytes of each lane and as many zeros, from which each lane reads its register q
// and three zero registers with one 4-byte read each (lane-contiguous, conflict-free), plus each
// slot's yd and 32-value sums.
//
// Launch: grid (tile groups, experts, slot chunks). A workgroup of 4 wavefronts takes an expert, a
// chunk of up to 8 of its slots (chunks side by side in grid.z, so a popular expert's slots run in
// parallel workgroups) and 4 x tt consecutive 16-row tiles of the launch's matrices (gate then up:
// y_0 = g, y_1 = u; or down: y_0), tt sized for three wavefronts per SIMD over all experts, every
// workgroup resident at once. A wavefront streams its tiles block by block through a ring of R
// steps in registers that runs on across tile boundaries, forms each block's weight side
// (nibbles, split scales, d, dmin, mins) once and runs every slot group of the chunk on it.
// Measured and kept out (config 5, 64 tokens, kernel trace; same bits in every form): a gate / up
// launch whose 8-wavefront workgroups cover 256 rows of gate and up and form the Q8_K images of
// h = silu(g) * u themselves (no g / u stores, no image launch): 73 us against 62-67 us plus the
// 4.9 us image launch, since its 384 workgroups, one per CU, take two rounds of which the second
// fills half the chip; A fragments expanded to 16 bytes per lane (one 16-byte read, 4x the LDS):
// two wavefronts per SIMD instead of three, slower; 4 slots per chunk: 37 % of the experts then
// stream their weights twice; ring depths 2, 6 and 8. A copy whose blocks only load (no compute)
// streams the same weights in 47 us (gate / up) and 27 us (down), about 4.7 and 4.1 TB/s: the
// rest is the per-block VALU work (about 150 instructions per wavefront and block at one group).
#include <algorithm>

#include "fgh_internal.h"

namespace fgh {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

namespace {

// A fragments of one (block, group): 4 K-steps x {64 lanes x 4 B of activations, 64 lanes x 4 B of
// zeros}; lane l reads register e of its fragment from the first half when e is its lane group q,
// else from the second (4 ds_read_b32, no VALU)
constexpr int MM_FRAG = 2048;
constexpr int MM_TPW = 4;  // wavefronts per workgroup

// LDS of a chunk of NSG groups (4 slots each) over nb blocks: fragments [b][g], then yd [g][b][s]
// fp32, 32-value sums [g][b][s] (8 int16), the slots' ids and image rows
__host__ __device__ constexpr size_t mm_off_yd(int nsg, int nb) { return (size_t)nsg * nb * MM_FRAG; }
__host__ __device__ constexpr size_t mm_off_bs(int nsg, int nb) { return mm_off_yd(nsg, nb) + (size_t)nsg * nb * 16; }
__host__ __device__ constexpr size_t mm_off_sl(int nsg, int nb) { return mm_off_bs(nsg, nb) + (size_t)nsg * nb * 64; }
__host__ __device__ constexpr size_t mm_lds(int nsg, int nb) { return mm_off_sl(nsg, nb) + (size_t)nsg * 4 * 8; }

// bytes of q (each <= 15) times a small factor (<= 7) in both 16-bit lanes: no carry between bytes
__device__ __forceinline__ uint32_t bmul(uint32_t q, uint32_t f2) {
    const u16x2 r = __builtin_bit_cast(u16x2, q) * __builtin_bit_cast(u16x2, f2);
    return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ v4i u4v(uint4 u) { return v4i{(int)u.x, (int)u.y, (int)u.z, (int)u.w}; }

// one lane's weights of one block: pieces 0 and 1 of its chunk and its row's meta; live = false:
// zeros without a memory access (a ring slot past the wavefront's last step). The decode layout
// keeps piece h of chunk kg in slot h ^ (kg >> 1) (1024-byte halves from byte 256): o0 / o1, the
// lane's byte offsets of pieces 0 / 1, undo that swap in the addresses, not in registers.
struct MmW {
    uint4 p0, p1, m;
};
__device__ __forceinline__ void mm_wload(const uint8_t *blk, uint32_t o0, uint32_t o1, uint32_t n, bool live, MmW &w) {
    const BufRes r = buf_res(blk, live ? Q4K_TILE : 0);
    w.p0 = bld16<WNT>(r, o0);
    w.p1 = bld16<WNT>(r, o1);
    w.m = bld16<WNT>(r, 16 * n);
}

struct MmArgs {
    const uint8_t *W[2];         // gate, up (or down alone): tile layout, matrices of one shape
    int nw;                      // tensors (1 or 2), their tiles concatenated
    int64_t rows, gpm;           // rows and 16-row tiles per matrix
    int nb;                      // blocks per row
    const int32_t *cnt, *slots;  // per-expert slot counts and buckets (cap entries each)
    int cap;
    const uint8_t *img;          // activation images, image row = slot / xdiv
    int xdiv;
    float *y[2];                 // y_i[slot * ldy + row] of tensor i
    int64_t ldy;
    int tt;                      // tiles per wavefront
    int32_t *dump_s, *dump_m;    // test hook: tensor 0's integers [slot][rows][nb]
};

__device__ __forceinline__ const uint8_t *img_row(const MmArgs &a, int r, size_t actb) { return a.img + (size_t)r * actb; }

template <int NSG, int R, bool DUMP>
__global__ __launch_bounds__(64 * MM_TPW) void q4k_moe_mfma_kernel(MmArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int TPW = MM_TPW, NTH = 64 * TPW, CH = 4 * NSG;  // threads, slots per chunk
    static_assert(TPW % 4 == 0, "the fragment build gives each thread one K-step: 256 threads per block");
    const int tid = threadIdx.x, l = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nb = a.nb;
    const int expert = blockIdx.y, count = a.cnt[expert];
    if (count <= (int)blockIdx.z * CH) return;  // whole workgroup: no slot of this chunk
    const int first = expert * a.cap;
    // this wavefront's tiles [t0, t0 + ntl) of the launch's tiles (those of W[0], then of W[1])
    const int64_t gpm = a.gpm, ntile = a.nw * gpm;
    const int64_t t0 = ((int64_t)blockIdx.x * TPW + wave) * a.tt;
    const int ntl = (int)max((int64_t)0, min((int64_t)a.tt, ntile - t0));
    const int kg = l >> 4, n = l & 15;  // B operand: chunk kg of row n (decode lane 4 n + kg)
    const uint32_t L = 4 * n + kg;
    const uint32_t o0 = (kg >= 2 ? 1280u : 256u) + 16 * L, o1 = (kg >= 2 ? 256u : 1280u) + 16 * L;
    const int s = l >> 4;               // output: slot s of a group, row n
    const size_t actb = q4_act_bytes(nb);
    uint8_t *frag = smem;
    float *yds = (float *)(smem + mm_off_yd(NSG, nb));
    uint4 *bss = (uint4 *)(smem + mm_off_bs(NSG, nb));
    int32_t *sl_id = (int32_t *)(smem + mm_off_sl(NSG, nb)), *sl_row = sl_id + CH;
    // (tile t of the launch, block b) of this expert
    auto step_ptr = [&](int64_t t, int b) {
        const int ti = t >= gpm ? 1 : 0;
        return a.W[ti] + (((size_t)expert * nb + b) * gpm + (size_t)(t - ti * gpm)) * Q4K_TILE;
    };

    for (int c0 = (int)blockIdx.z * CH; c0 < count; c0 += CH * (int)gridDim.z) {
        const int ns = min(CH, count - c0);
        // (1) the ring's first R steps
        MmW ring[R];
        int rj = 0, rb = 0;  // the next step to load: tile t0 + rj, block rb
#pragma unroll
        for (int r = 0; r < R; ++r) {
            mm_wload(step_ptr(t0 + min(rj, max(ntl - 1, 0)), rb), o0, o1, n, rj < ntl, ring[r]);
            if (++rb == nb) { rb = 0; ++rj; }
        }
        // (2) the chunk's slots, then its fragments, yd and sums
        if (tid < CH) {
            const int slot = tid < ns ? a.slots[first + c0 + tid] : -1;
            sl_id[tid] = slot;
            sl_row[tid] = slot >= 0 ? slot / a.xdiv : 0;
        }
        __syncthreads();
        {
            constexpr int BS = NTH >> 8;  // blocks built side by side
            const int kap = (tid >> 6) & 3, h = kap >> 1, i = kap & 1;  // this thread's K-step
            const int fk = l >> 4, fm = l & 15, fs = fm >> 2, fq = fm & 3;
            const uint32_t pos = 32 * (2 * fk + i) + 16 * h + 4 * fq;
#pragma unroll
            for (int g = 0; g < NSG; ++g) {
                const int c = 4 * g + fs;
                const uint8_t *src = img_row(a, sl_row[c], actb);
                for (int b0 = tid >> 8; b0 < nb; b0 += 4 * BS) {  // 4 loads in flight, then 4 stores
                    uint32_t v[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const int b = b0 + u * BS;
                        v[u] = c < ns && b < nb ? *(const uint32_t *)(src + (size_t)b * 256 + pos) : 0u;
                    }
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const int b = b0 + u * BS;
                        if (b < nb) {
                            uint32_t *f = (uint32_t *)(frag + ((size_t)b * NSG + g) * MM_FRAG + 512 * kap);
                            f[l] = v[u];
                            if (c0 == (int)blockIdx.z * CH) f[64 + l] = 0u;  // the zero half: the first chunk
                        }
                    }
                }
            }
            for (int e = tid; e < NSG * nb * 4; e += NTH) {
                const int gb = e >> 2, es = e & 3, g = gb / nb, b = gb - g * nb, c = 4 * g + es;
                const uint8_t *src = img_row(a, sl_row[c], actb);
                const bool ok = c < ns;
                yds[e] = ok ? ((const float *)(src + q4_off_d(nb)))[b] : 0.0f;
                bss[e] = ok ? *(const uint4 *)(src + q4_off_s(nb) + (size_t)b * 16) : make_uint4(0, 0, 0, 0);
            }
        }
        __syncthreads();

        const int ngr = (ns + 3) >> 2;  // groups with a slot (uniform)
        float acc[NSG][8], macc[NSG][4];
        auto reset = [&]() {
#pragma unroll
            for (int g = 0; g < NSG; ++g) {
#pragma unroll
                for (int k = 0; k < 8; ++k) acc[g][k] = 0.0f;
#pragma unroll
                for (int p = 0; p < 4; ++p) macc[g][p] = 0.0f;
            }
        };
        // lane offsets of the 4 registers of the A fragment: its own 4 bytes for register q (the
        // lane group of its row m = l & 15), the zero half for the other three
        const int aq = l & 3;
        uint32_t aoff[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) aoff[e] = (e == aq ? 0u : 256u) + 4u * (uint32_t)l;
        // one block b of launch tile t from ring slot w
        auto blk = [&](const MmW &w, int b, int64_t t) {
            // pieces 0 and 1 of the chunk (the loads undid the layout's swap)
            const bool sw = kg >= 2;
            const uint32_t X[2][4] = {{w.p0.x, w.p0.y, w.p0.z, w.p0.w}, {w.p1.x, w.p1.y, w.p1.z, w.p1.w}};
            // sub-block scales 2 kg and 2 kg + 1 as bytes 0 and 1 of scp (scale_min_k4, fastgguf.c:466-472)
            const int shs = 16 * (kg & 1);
            const uint32_t A = w.m.y >> shs, C = w.m.w >> shs;
            const uint32_t sc_lo = A & 0x3f3fu, sc_hi = (C & 0x0f0fu) | ((A >> 2) & 0x3030u);
            const uint32_t scp = sw ? sc_hi : sc_lo;
            const uint32_t fh[2] = {((scp >> 3) & 7u) * 0x10001u, ((scp >> 11) & 7u) * 0x10001u};
            const uint32_t fl[2] = {(scp & 7u) * 0x10001u, ((scp >> 8) & 7u) * 0x10001u};
            v4i BH[4], BL[4];
#pragma unroll
            for (int kap = 0; kap < 4; ++kap) {
                const int h = kap >> 1, i = kap & 1;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t v = i == 0 ? X[h][e] & 0x0F0F0F0Fu : (X[h][e] >> 4) & 0x0F0F0F0Fu;
                    BH[kap][e] = (int)bmul(v, fh[i]);
                    BL[kap][e] = (int)bmul(v, fl[i]);
                }
            }
            const float d = fp16_bits_to_f32(w.m.x & 0xFFFF), dmin = fp16_bits_to_f32(w.m.x >> 16);
            // the row's eight mins as int16 pairs (m_2p, m_2p+1), the reference's k4_min_vec lanes
            const uint32_t mn_lo = w.m.z & 0x3f3f3f3fu;
            const uint32_t mn_hi = ((w.m.w >> 4) & 0x0f0f0f0fu) | (((w.m.z >> 6) & 0x03030303u) << 4);
            const uint32_t MP[4] = {__builtin_amdgcn_perm(0u, mn_lo, 0x0C010C00u), __builtin_amdgcn_perm(0u, mn_lo, 0x0C030C02u),
                                    __builtin_amdgcn_perm(0u, mn_hi, 0x0C010C00u), __builtin_amdgcn_perm(0u, mn_hi, 0x0C030C02u)};
#pragma unroll
            for (int g = 0; g < NSG; ++g) {
                if (g < ngr) {  // uniform
                    const uint8_t *fb = frag + ((size_t)b * NSG + g) * MM_FRAG;
                    v4i AF[4];
#pragma unroll
                    for (int kap = 0; kap < 4; ++kap)
#pragma unroll
                        for (int e = 0; e < 4; ++e) AF[kap][e] = *(const int *)(fb + 512 * kap + aoff[e]);
                    v4i ch[2], cl[2];
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        ch[h] = __builtin_amdgcn_mfma_i32_16x16x64_i8(AF[2 * h], BH[2 * h], v4i{0, 0, 0, 0}, 0, 0, 0);
                        cl[h] = __builtin_amdgcn_mfma_i32_16x16x64_i8(AF[2 * h], BL[2 * h], v4i{0, 0, 0, 0}, 0, 0, 0);
                        ch[h] = __builtin_amdgcn_mfma_i32_16x16x64_i8(AF[2 * h + 1], BH[2 * h + 1], ch[h], 0, 0, 0);
                        cl[h] = __builtin_amdgcn_mfma_i32_16x16x64_i8(AF[2 * h + 1], BL[2 * h + 1], cl[h], 0, 0, 0);
                    }
                    const int e = (g * nb + b) * 4 + s;
                    const float yd = yds[e];
                    const uint4 bq = bss[e];
                    const uint32_t BQ[4] = {bq.x, bq.y, bq.z, bq.w};
                    const float fd = d * yd, fdm = dmin * yd;
                    int ssum = 0, msum = 0;
#pragma unroll
                    for (int h = 0; h < 2; ++h)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int isum = (ch[h][r] << 3) + cl[h][r];  // lane partial 4 h + r
                            acc[g][4 * h + r] = __builtin_fmaf(fd, (float)isum, acc[g][4 * h + r]);
                            if (DUMP) ssum += isum;
                        }
#pragma unroll
                    for (int p = 0; p < 4; ++p) {
                        const int mt = dot2_i16(MP[p], BQ[p], 0);
                        macc[g][p] = __builtin_fmaf(fdm, (float)mt, macc[g][p]);
                        if (DUMP) msum += mt;
                    }
                    const int64_t row = (t % gpm) * Q4K_TILE_ROWS + n;
                    if (DUMP && t < gpm && 4 * g + s < ns && row < a.rows) {
                        const size_t di = ((size_t)sl_id[4 * g + s] * a.rows + row) * nb + b;
                        a.dump_s[di] = ssum;
                        a.dump_m[di] = msum;
                    }
                }
            }
        };
        // the reference's final sums in each (slot, row) lane: hsum_ps(acc) - hsum128_ps(macc)
        // (fastgguf.c:797-806, 1089-1095), then the tile's outputs
        auto finish = [&](int j) {
            const int64_t t = t0 + j;
            const int ti = t >= gpm ? 1 : 0;
            const int64_t row = (t - ti * gpm) * Q4K_TILE_ROWS + n;
#pragma unroll
            for (int g = 0; g < NSG; ++g) {
                const int c = 4 * g + s;
                if (g < ngr && c < ns) {
                    const float *v = acc[g], *m = macc[g];
                    const float h8 = ((v[0] + v[4]) + (v[1] + v[5])) + ((v[2] + v[6]) + (v[3] + v[7]));
                    const float h4 = (m[0] + m[1]) + (m[2] + m[3]);
                    if (row < a.rows) a.y[ti][(size_t)sl_id[c] * a.ldy + row] = h8 - h4;
                }
            }
        };
        // the wavefront's steps (tile j, block b) in order, R at a time from the ring; each ring
        // slot refills with the step R ahead (a slot past the last step loads nothing)
        reset();
        int j = 0, b = 0;
        const int total = ntl * nb;
        auto step = [&](int r) {
            blk(ring[r], b, t0 + j);
            mm_wload(step_ptr(t0 + min(rj, ntl - 1), rb), o0, o1, n, rj < ntl, ring[r]);
            if (++rb == nb) { rb = 0; ++rj; }
            if (++b == nb) {  // uniform: the tile's last block
                finish(j);
                reset();
                b = 0;
                ++j;
            }
        };
        int k0 = 0;
        for (; k0 + R <= total; k0 += R) {
#pragma unroll
            for (int r = 0; r < R; ++r) step(r);
        }
#pragma unroll
        for (int r = 0; r < R - 1; ++r)
            if (k0 + r < total) step(r);  // uniform
        __syncthreads();  // the next chunk rebuilds the fragments and slot lists
    }
}

template <int NSG, int R>
hipError_t mm_launch(const MmArgs &a, dim3 grid, hipStream_t s) {
    const size_t lds = mm_lds(NSG, a.nb);
    if (a.dump_s) q4k_moe_mfma_kernel<NSG, R, true><<<grid, 64 * MM_TPW, lds, s>>>(a);
    else q4k_moe_mfma_kernel<NSG, R, false><<<grid, 64 * MM_TPW, lds, s>>>(a);
    return hipGetLastError();
}
template <int NSG>
hipError_t mm_launch_r(int r, const MmArgs &a, dim3 grid, hipStream_t s) {
    switch (r) {
    case 2: return mm_launch<NSG, 2>(a, grid, s);
    case 4: return mm_launch<NSG, 4>(a, grid, s);
    default: return mm_launch<NSG, 3>(a, grid, s);
    }
}
hipError_t mm_launch_g(int nsg, int r, const MmArgs &a, dim3 grid, hipStream_t s) {
    switch (nsg) {
    case 1: return mm_launch_r<1>(r, a, grid, s);
    case 2: return mm_launch_r<2>(r, a, grid, s);
    default: return mm_launch_r<4>(r, a, grid, s);
    }
}

// chunks of 4 nsg slots side by side (grid.z): the most slots an expert gets from tokens that
// pick it once each is n_tok; the chunks past that (repeated picks) loop in the last z
unsigned mm_zchunks(int n_tok, int nsg) { return (unsigned)std::max(1, (n_tok + 4 * nsg - 1) / (4 * nsg)); }

// tiles per wavefront: about three wavefronts per SIMD over all experts' tiles, at least one
int mm_tiles_per_wave(int64_t tiles, int n_expert, int num_cu) {
    const int64_t waves = 3 * 4 * (int64_t)num_cu;
    return (int)std::max<int64_t>(1, (tiles * n_expert + waves - 1) / waves);
}

}  // namespace

size_t q4k_moe_mfma_lds(int nsg, int nb) { return mm_lds(nsg, nb); }

hipError_t launch_q4k_moe_mfma(const MoeMmShape &sh, const uint8_t *w0, const uint8_t *w1, int64_t rows, int64_t gpm,
                               int nb, const int32_t *cnt, const int32_t *buckets, int cap, int n_expert, int n_tok,
                               const uint8_t *img, int xdiv, float *y0, float *y1, int64_t ldy, int32_t *dump_s,
                               int32_t *dump_m, int num_cu, hipStream_t s) {
    const int nw = w1 ? 2 : 1;
    if (nb < 1 || n_expert < 1 || cap < 1 || xdiv < 1 || rows < 1 || gpm < 1 || gpm * 16 < rows || !w0 || !y0 ||
        (w1 && !y1) || (sh.nsg != 1 && sh.nsg != 2 && sh.nsg != 4) || mm_lds(sh.nsg, nb) > GEMM_LDS_MAX)
        return hipErrorInvalidValue;
    MmArgs a = {};
    a.W[0] = w0;
    a.W[1] = w1;
    a.nw = nw;
    a.rows = rows;
    a.gpm = gpm;
    a.nb = nb;
    a.cnt = cnt;
    a.slots = buckets;
    a.cap = cap;
    a.img = img;
    a.xdiv = xdiv;
    a.y[0] = y0;
    a.y[1] = y1;
    a.ldy = ldy;
    a.dump_s = dump_s;
    a.dump_m = dump_m;
    a.tt = sh.tt > 0 ? sh.tt : mm_tiles_per_wave(nw * gpm, n_expert, num_cu);
    const int64_t wg = (nw * gpm + (int64_t)MM_TPW * a.tt - 1) / ((int64_t)MM_TPW * a.tt);
    return mm_launch_g(sh.nsg, sh.r, a, dim3((unsigned)wg, (unsigned)n_expert, mm_zchunks(n_tok, sh.nsg)), s);
}

}  // namespace fgh
