// fgh_float.hip - the decode matvec for the float weight types F32, F16 and BF16 on fp32
// activations (dot_row fastgguf.c:2207-2214: dot_f32v 1618-1632, dot_f16_row 1645-1656 and the
// BF16 loop 2209-2213; the reference's own GPU path runs these types too, gpu_kernel_for 1745).
//
// Each row kernel runs C fp32 fma chains over the row, chain k over the values C j + k in order
// (no quantization of x), then sums the chains with a fixed tree and runs the last values one
// fma each:
//   F32:  C = 16 (dot_f32v's two 8-lane accumulators s0 = chains 0..7, s1 = chains 8..15), one
//         more 8-value group into s0 when 8 values remain, hsum_ps(s0 + s1), then the last n % 8
//         values (gcc's contraction of `s += a[i] * b[i]`)
//   F16:  C = 8, the values converted exactly (vcvtph2ps), hsum_ps, then the last n % 8 values
//   BF16: C = 1, one chain over the whole row (the value is its 16 bits above 16 zero bits)
// hsum_ps(v) = ((v0 + v4) + (v1 + v5)) + ((v2 + v6) + (v3 + v7)) (fastgguf.c:797-806).
//
// A wavefront holds one row tile, lane L = C r + k taking chain k of tile row r (64 / C rows per
// tile), and walks the row's steps in order through a ring of R 16-byte loads. A step is 1 KB:
// V = 16 / value bytes values per lane, lane L's values u = 0..V-1 of step s being the row's
// values C (V s + u) + k (tile layout below), so a step is V consecutive values of each chain.
// x is staged once per workgroup in LDS in the same order (value C (V s + u) + k at float
// (C s + k) V + u), so a lane reads its step's V activations with one or two 16-byte LDS reads
// (the rows of a wavefront read the same addresses). The last, partial step runs each value on
// the chain its position takes in the reference, and the lane of chain 0 runs the scalar tail
// from the tile in global memory after the tree. Rows are independent, and every row's fp32
// operations are the reference's, in its order: the outputs are bit-identical.
//
// BF16's one chain per row makes its launch latency-bound: about 11 ns per value of the row on
// MI355X (46 us at 4096 values) whatever the row count, against 9.9 us for F16 at 4096 x 4096.
//
// Tiles (upload, fl_relayout_kernel): step s of row tile t of matrix m at
// ((m * steps + s) * tiles per matrix + t) * 1 KB, lane L's 16 bytes at 16 L; values past the
// row's end and rows past the matrix's end are zeros (never on a chain).
#include "fgh_internal.h"

namespace fgh {

namespace {

template <int TYPE>
struct Fl {
    static constexpr int C = TYPE == T_F32 ? 16 : TYPE == T_F16 ? 8 : 1;  // chains per row
    static constexpr int V = TYPE == T_F32 ? 4 : 8;                      // values per lane and step
    static constexpr int CV = C * V;                                     // a row's values per step
    static constexpr int TR = 64 / C;                                    // rows per tile
};
static_assert(Fl<T_F32>::CV == fl_step_elems(T_F32) && Fl<T_F16>::CV == fl_step_elems(T_F16) &&
                  Fl<T_BF16>::CV == fl_step_elems(T_BF16),
              "step geometry");
static_assert(Fl<T_F32>::TR == fl_tile_rows(T_F32) && Fl<T_F16>::TR == fl_tile_rows(T_F16) &&
                  Fl<T_BF16>::TR == fl_tile_rows(T_BF16),
              "tile geometry");

// DPP row_shl:k, the value of lane + k within its 16-lane row (lanes without a source read 0)
__device__ __forceinline__ float shl(float v, int k) {
    const int iv = __builtin_bit_cast(int, v);
    int o;
    switch (k) {
    case 1: o = __builtin_amdgcn_update_dpp(0, iv, 0x101, 0xF, 0xF, true); break;
    case 2: o = __builtin_amdgcn_update_dpp(0, iv, 0x102, 0xF, 0xF, true); break;
    case 4: o = __builtin_amdgcn_update_dpp(0, iv, 0x104, 0xF, 0xF, true); break;
    default: o = __builtin_amdgcn_update_dpp(0, iv, 0x108, 0xF, 0xF, true); break;
    }
    return __builtin_bit_cast(float, o);
}

// a lane's 16 bytes of one step; live = false: zeros without a memory access
__device__ __forceinline__ uint4 fl_load(const uint8_t *step, uint32_t lane, bool live) {
    return bld16<WNT>(buf_res(step, live ? FL_TILE : 0), 16 * lane);
}

// value u of a lane's 16 bytes, as fp32 (each conversion exact)
template <int TYPE>
__device__ __forceinline__ float fl_val(const uint4 &w, int u) {
    const uint32_t d[4] = {w.x, w.y, w.z, w.w};
    if (TYPE == T_F32) return __builtin_bit_cast(float, d[u]);
    const uint32_t p = d[u >> 1];
    if (TYPE == T_BF16) return __builtin_bit_cast(float, (u & 1) ? p & 0xFFFF0000u : p << 16);
    return fp16_bits_to_f32((u & 1) ? p >> 16 : p & 0xFFFFu);
}
// one value of the row in the tile layout (the scalar tail), by its position e
template <int TYPE>
__device__ __forceinline__ float fl_val_at(const uint8_t *T0, size_t sstride, int r, int e) {
    using F = Fl<TYPE>;
    const int s = e / F::CV, rem = e - s * F::CV, u = rem / F::C, kk = rem - u * F::C;
    const uint8_t *p = T0 + (size_t)s * sstride + 16 * (F::C * r + kk) + fl_value_bytes(TYPE) * u;
    if (TYPE == T_F32) return *(const float *)p;
    const uint32_t h = *(const uint16_t *)p;
    return TYPE == T_BF16 ? __builtin_bit_cast(float, h << 16) : fp16_bits_to_f32(h);
}

// where value e of the row sits in the LDS copy of x (and in a lane's step: lane C r + kk, value u)
template <int TYPE>
__device__ __forceinline__ int fl_xpos(int e) {
    using F = Fl<TYPE>;
    const int s = e / F::CV, rem = e - s * F::CV, u = rem / F::C, kk = rem - u * F::C;
    return (s * F::C + kk) * F::V + u;
}

// is value u of chain k in step s on its chain (and not in the scalar tail or past the row)?
template <int TYPE>
__device__ __forceinline__ bool on_chain(int s, int u, int k, int n) {
    using F = Fl<TYPE>;
    const int j = F::V * s + u;  // the chain's j-th value: position C j + k
    if (TYPE == T_F32) return 16 * j + 16 <= n || (k < 8 && 16 * j + 8 <= n);
    if (TYPE == T_F16) return 8 * j + 8 <= n;
    return j < n;
}

__device__ __forceinline__ int fl_tensor_of(const MvArgs &a, int64_t g) {
    int ti = 0;
#pragma unroll
    for (int q = 1; q < 4; ++q)
        if (q < a.nt && g >= a.t[q].gfirst) ti = q;
    return ti;
}

}  // namespace

// Workgroup = TPW row tiles, one wavefront each; grid = (tiles over all tensors / TPW, token
// slots). a.nb = the row's values n, a.ntile = its steps.
template <int TYPE, int R, int TPW>
__global__ __launch_bounds__(64 * TPW) void fl_mv_kernel(MvArgs a) {
    using F = Fl<TYPE>;
    extern __shared__ __align__(16) uint8_t smem[];
    float *xs = (float *)smem;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane / F::C, k = lane - r * F::C;
    const int n = a.nb, nst = a.ntile;
    const int tok = blockIdx.y;
    const int64_t tile = (int64_t)blockIdx.x * TPW + wave;
    const bool live = tile < a.groups;
    const int64_t tc = live ? tile : a.groups - 1;
    const int ti = fl_tensor_of(a, tc);
    const uint32_t lt = (uint32_t)(tc - a.t[ti].gfirst), tpm = (uint32_t)a.t[ti].gpm;
    const uint32_t mi = (a.sel ? (uint32_t)a.sel[tok] : 0u) + lt / tpm, tt = lt % tpm;
    const size_t sstride = (size_t)tpm * FL_TILE;
    const uint8_t *T0 = a.t[ti].W + ((size_t)mi * nst * tpm + tt) * FL_TILE;

    // (1) the ring's first R steps, (2) x into LDS in the lanes' order while they load
    uint4 ring[R];
#pragma unroll
    for (int q = 0; q < R; ++q) ring[q] = fl_load(T0 + (size_t)min(q, nst - 1) * sstride, (uint32_t)lane, q < nst);
    const float *x = a.x + (size_t)(tok / a.xdiv) * a.ldx;
    const int npad = nst * F::CV;
    for (int e0 = tid; e0 < npad; e0 += 4 * 64 * TPW) {
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int e = e0 + q * 64 * TPW;
            v[q] = e < n ? x[e] : 0.0f;
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int e = e0 + q * 64 * TPW;
            if (e < npad) xs[fl_xpos<TYPE>(e)] = v[q];
        }
    }
    __syncthreads();

    float acc = 0.0f;
    const int nwhole = n / F::CV;  // steps whose every value is on its chain (nst - 1 or nst)
    // the activations of step s from LDS (the last step's for s past it)
    auto xload = [&](int s, float (&xv)[8]) {
        const float4 *xp = (const float4 *)(xs + (size_t)(min(s, nst - 1) * F::C + k) * F::V);
        const float4 x0 = xp[0];
        xv[0] = x0.x, xv[1] = x0.y, xv[2] = x0.z, xv[3] = x0.w;
        if (F::V == 8) {
            const float4 x1 = xp[1];
            xv[4] = x1.x, xv[5] = x1.y, xv[6] = x1.z, xv[7] = x1.w;
        } else {
            xv[4] = xv[5] = xv[6] = xv[7] = 0.0f;
        }
    };
    // whole rounds of R whole steps, refilling the ring (a refill past the last step loads
    // nothing), straight-line code without a test; then the last steps (at most R, already in the
    // ring), each value tested against its chain. Step s's activations are in xb[s % XD], loaded
    // XD steps ahead (one step ahead left each step waiting for its LDS reads: BF16's one chain
    // ran 28 cycles per value).
    constexpr int XD = 4;
    static_assert(R % XD == 0, "the activation buffers rotate within a round");
    float xb[XD][8];
#pragma unroll
    for (int q = 0; q < XD; ++q) xload(q, xb[q]);
    int b0 = 0;
    for (; b0 + R <= nwhole; b0 += R) {
#pragma unroll
        for (int q = 0; q < R; ++q) {
#pragma unroll
            for (int u = 0; u < F::V; ++u) acc = __builtin_fmaf(fl_val<TYPE>(ring[q], u), xb[q % XD][u], acc);
            ring[q] = fl_load(T0 + (size_t)min(b0 + q + R, nst - 1) * sstride, (uint32_t)lane, b0 + q + R < nst);
            xload(b0 + q + XD, xb[q % XD]);
        }
    }
#pragma unroll
    for (int q = 0; q < R; ++q)
        if (b0 + q < nst) {  // uniform
            const int st = b0 + q;
#pragma unroll
            for (int u = 0; u < F::V; ++u)
                if (on_chain<TYPE>(st, u, k, n)) acc = __builtin_fmaf(fl_val<TYPE>(ring[q], u), xb[q % XD][u], acc);
            xload(st + XD, xb[q % XD]);
        }

    // the chains' tree (hsum_ps of s0 + s1 for F32, of the 8 chains for F16), then the scalar tail
    float res = acc;
    if (TYPE == T_F32) res = res + shl(res, 8);  // v_k = s0_k + s1_k
    if (TYPE != T_BF16) {
        res = res + shl(res, 4);  // (v_k + v_k+4), k < 4
        res = res + shl(res, 1);  // (v0 + v4) + (v1 + v5) at k = 0, the other pair at k = 2
        res = res + shl(res, 2);
    }
    const int64_t rows = a.t[ti].rows, row = (int64_t)tt * F::TR + r;
    if (live && k == 0 && row < rows) {
        if (TYPE != T_BF16) {
            const int t0 = TYPE == T_F32 ? 16 * (n / 16) + (n % 16 >= 8 ? 8 : 0) : 8 * (n / 8);
            for (int e = t0; e < n; ++e) res = __builtin_fmaf(fl_val_at<TYPE>(T0, sstride, r, e), xs[fl_xpos<TYPE>(e)], res);
        }
        a.t[ti].y[(size_t)tok * a.ldy + (int64_t)(lt / tpm) * rows + row] = res;
    }
}

// ---- upload: file rows -> tiles, one thread per destination 16 bytes ----
__global__ void fl_relayout_kernel(int type, const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, int64_t rows,
                                   int64_t cols, int steps, int64_t gpm, int64_t units) {
    const int C = type == T_F32 ? 16 : type == T_F16 ? 8 : 1, V = type == T_F32 ? 4 : 8, TR = 64 / C;
    const int vb = fl_value_bytes(type);
    for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < units; o += (int64_t)gridDim.x * blockDim.x) {
        const int64_t t = o >> 6;  // = (m * steps + s) * gpm + gl
        const int L = (int)(o & 63);
        const int64_t mt = t / gpm, gl = t - mt * gpm;
        const int64_t m = mt / steps;
        const int s = (int)(mt - m * steps);
        const int r = L / C, k = L - r * C;
        const int64_t row = gl * TR + r;
        uint8_t b[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) b[q] = 0;
        if (row < rows)
            for (int u = 0; u < V; ++u) {
                const int64_t e = (int64_t)C * (V * s + u) + k;
                if (e < cols) {
                    const uint8_t *p = src + ((m * rows + row) * cols + e) * vb;
                    for (int q = 0; q < vb; ++q) b[vb * u + q] = p[q];
                }
            }
        uint4 w;
        __builtin_memcpy(&w, b, 16);
        ((uint4 *)dst)[o] = w;
    }
}

// ---- host side ----
size_t fl_lds_bytes(int type, int64_t cols) {
    const int64_t steps = (cols + fl_step_elems(type) - 1) / fl_step_elems(type);
    return (size_t)steps * fl_step_elems(type) * 4;
}
// One wavefront per tile (the chains are serial), a ring of 16 steps (16 KB in flight per
// wavefront). Tiles per workgroup: F16 4, BF16 2, F32 4 from 2 to 8 tiles per compute unit and 2
// otherwise. Measured (graph of back-to-back launches over >= 512 MB of copies, rings of 8, 16
// and 32 x 1, 2 and 4 tiles per workgroup, at 14336 x 4096, 4096 x 4096, 4096 x 14336 and
// 1024 x 4096): a ring of 16 was the fastest or within 2 % everywhere; F32 4096 x 4096 (1024
// tiles) 13.2 us with 4 tiles against 14.9 with 2, 14336 x 4096 (3584) 37.3 with 2 against 38.5,
// 1024 x 4096 (256) 8.3 with 2 against 9.2 and 10.5 with 1.
MvShape fl_matvec_shape(int type, int64_t tiles, int64_t cols, int num_cu) {
    const int tpw = type == T_F16    ? 4
                    : type == T_BF16 ? 2
                    : tiles >= 2 * (int64_t)num_cu && tiles <= 8 * (int64_t)num_cu ? 4
                                                                                   : 2;
    return MvShape{1, 16, tpw, fl_lds_bytes(type, cols)};
}

template <int TYPE, int R, int TPW>
static hipError_t fl_launch(const MvArgs &a, int ntok, size_t lds, hipStream_t s) {
    const unsigned wg = (unsigned)((a.groups + TPW - 1) / TPW);
    fl_mv_kernel<TYPE, R, TPW><<<dim3(wg, ntok), 64 * TPW, lds, s>>>(a);
    return hipGetLastError();
}
template <int TYPE, int R>
static hipError_t fl_launch_r(const MvShape &sh, const MvArgs &a, int ntok, hipStream_t s) {
    switch (sh.TPW) {
    case 4: return fl_launch<TYPE, R, 4>(a, ntok, sh.lds, s);
    case 2: return fl_launch<TYPE, R, 2>(a, ntok, sh.lds, s);
    default: return fl_launch<TYPE, R, 1>(a, ntok, sh.lds, s);
    }
}
template <int TYPE>
static hipError_t fl_launch_type(const MvArgs &a, int ntok, int num_cu, hipStream_t s) {
    const MvShape sh = fl_matvec_shape(TYPE, a.groups * ntok, a.nb, num_cu);
    if (sh.lds > GEMM_LDS_MAX || sh.R != 16) return hipErrorInvalidValue;
    return fl_launch_r<TYPE, 16>(sh, a, ntok, s);
}
hipError_t launch_fl_matvec(int type, const MvArgs &a, int ntok, int num_cu, hipStream_t s) {
    if (a.nb < 1 || a.ntile != (a.nb + fl_step_elems(type) - 1) / fl_step_elems(type) || a.dump_s)
        return hipErrorInvalidValue;
    switch (type) {
    case T_F32: return fl_launch_type<T_F32>(a, ntok, num_cu, s);
    case T_F16: return fl_launch_type<T_F16>(a, ntok, num_cu, s);
    case T_BF16: return fl_launch_type<T_BF16>(a, ntok, num_cu, s);
    default: return hipErrorInvalidValue;
    }
}
hipError_t launch_fl_relayout(int type, const uint8_t *src, uint8_t *dst, int64_t rows, int64_t cols, int steps,
                              int64_t gpm, int64_t total, hipStream_t s) {
    if (!fl_kind(type) || total % 16) return hipErrorInvalidValue;
    const int64_t units = total / 16, want = (units + 255) / 256;
    const unsigned grid = (unsigned)(want < 65536 ? want : 65536);
    fl_relayout_kernel<<<grid, 256, 0, s>>>(type, src, dst, rows, cols, steps, gpm, units);
    return hipGetLastError();
}

}  // namespace fgh
