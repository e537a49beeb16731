// fgh_moe.hip - the MoE FFN around the expert matvecs (moe_ffn, fastgguf.c:4588-4642), per token:
//   route:    p = softmax(logits) (softmax_inplace 3147-3156), top-k by repeated argmax (3328-3332,
//             first index on ties), w_j = p_j / max(sum_j p_j, 2^-14) (4594-4604)
//   gate, up: expert sel_j's rows of gate / up times Q8_K(x) (the decode kernels with an expert
//             index read on the device)
//   h_j     = silu(g_j) * u_j, silu(x) = x / (1 + expf(-x)) (silu_f 3118): formed inside the
//             gate / up launch (one token), by the launch that quantizes the down projection's
//             inputs (the grouped path), or by silu_mul_kernel (the generic path)
//   down:     d_j = expert sel_j's rows of down times Q8_K(h_j)
//   y_i     = sum over j in order of fma(w_j, d_j[i], s)  (4626-4635; gcc contracts s += w*dot)
// Every dot product runs the reference's own per-row order (dot_q4_K_q8k and friends), so the
// integers are bit-exact and, given the same expf, so is everything else.
#include "fgh_internal.h"

namespace fgh {

// one wavefront per token (moe_route_wave, fgh_internal.h)
__global__ __launch_bounds__(64) void moe_route_kernel(const float *__restrict__ logits, int n_expert, int k,
                                                       int32_t *__restrict__ sel, float *__restrict__ w) {
    __shared__ __align__(16) float ps[64 * MOE_EPL];
    const int t = blockIdx.x;
    moe_route_wave(logits + (size_t)t * n_expert, n_expert, k, ps, sel + (size_t)t * k, w + (size_t)t * k, 0);
}

// y[t][i] = sum_j fma(w[t][j], d[t k + j][i], s), j ascending
// (cnt: the grouped path's bucket counts, cleared here for its next call: this launch runs after
// every kernel that reads them)
__global__ void moe_combine_kernel(const float *__restrict__ d, const float *__restrict__ w, float *__restrict__ y,
                                   int n_embd, int k, int64_t ldy, int32_t *__restrict__ cnt, int n_expert) {
    const int t = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (cnt && blockIdx.x == 0 && t == 0)
        for (int e = threadIdx.x; e < n_expert; e += blockDim.x) cnt[e] = 0;
    if (i >= n_embd) return;
    float s = 0.0f;
    for (int j0 = 0; j0 < k; j0 += 8) {  // 8 experts' loads in flight, then their fmas in order
        float dv[8], wv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int jj = min(j0 + u, k - 1);
            wv[u] = w[(size_t)t * k + jj];
            dv[u] = d[((size_t)t * k + jj) * n_embd + i];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (j0 + u < k) s = __builtin_fmaf(wv[u], dv[u], s);
    }
    y[(size_t)t * ldy + i] = s;
}

__global__ void expf_kernel(const float *__restrict__ x, float *__restrict__ y, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = expf_ref(x[i]);
}

hipError_t launch_expf(const float *x, float *y, int n, hipStream_t s) {
    expf_kernel<<<(n + 255) / 256, 256, 0, s>>>(x, y, n);
    return hipGetLastError();
}

// four values per thread, 1024 per workgroup; each value is read before its h is written, so h
// may be g (or u)
__global__ __launch_bounds__(256) void silu_mul_kernel(const float *g, const float *u, float *h, int64_t n) {
    const int64_t i0 = (int64_t)blockIdx.x * 1024 + threadIdx.x;
    float gv[4], uv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int64_t i = min(i0 + 256 * q, n - 1);
        gv[q] = g[i];
        uv[q] = u[i];
    }
#pragma unroll
    for (int q = 0; q < 4; ++q)
        if (i0 + 256 * q < n) h[i0 + 256 * q] = gv[q] / (1.0f + expf_ref(-gv[q])) * uv[q];
}

hipError_t launch_silu_mul(const float *g, const float *u, float *h, int64_t n, hipStream_t s) {
    if (n < 1) return hipErrorInvalidValue;
    silu_mul_kernel<<<(unsigned)((n + 1023) / 1024), 256, 0, s>>>(g, u, h, n);
    return hipGetLastError();
}

hipError_t launch_moe_route(const float *logits, int n_expert, int k, int n_tok, int32_t *sel, float *w,
                            hipStream_t s) {
    if (n_expert < 1 || n_expert > 64 * MOE_EPL || k < 1 || k > n_expert || k > 64) return hipErrorInvalidValue;
    moe_route_kernel<<<n_tok, 64, 0, s>>>(logits, n_expert, k, sel, w);
    return hipGetLastError();
}

__global__ void zero_i32_kernel(int32_t *__restrict__ p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

hipError_t launch_zero_i32(int32_t *p, int n, hipStream_t s) {
    if (n < 1) return hipSuccess;
    zero_i32_kernel<<<(n + 255) / 256, 256, 0, s>>>(p, n);
    return hipGetLastError();
}

hipError_t launch_moe_combine(const float *d, const float *w, float *y, int n_embd, int k, int n_tok, int64_t ldy,
                              int32_t *cnt, int n_expert, hipStream_t s) {
    moe_combine_kernel<<<dim3((n_embd + 255) / 256, n_tok), 256, 0, s>>>(d, w, y, n_embd, k, ldy, cnt, n_expert);
    return hipGetLastError();
}

}  // namespace fgh
