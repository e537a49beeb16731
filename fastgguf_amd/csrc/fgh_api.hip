// fgh_api.hip - the C ABI (include/fastgguf_hip.h): context, upload, dispatch and helpers.
// No entry point aborts or falls back to a CPU computation: failures return a negative status and
// leave a message in the context, and the caller decides (fastgguf.c:2577-2581 recomputes on its
// own CPU kernels).
#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdlib.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/fastgguf_hip.h"
#include "fgh_internal.h"

static const int FG_BATCH = 64;  // prompt batch limit (fastgguf.c:2139)

struct DevBuf {
    void *p = nullptr;
    size_t cap = 0;
};

struct fgh_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    uint64_t vram = 0, budget = 0, used = 0;
    int n_offloaded = 0, n_skip_type = 0, n_skip_mem = 0;
    char name[96] = {0};
    std::string err = "ok";
    // scratch, grown on demand (gpu_grow_buf, fastgguf.c:2083-2091)
    DevBuf x, y, aqs, ad, abs;
    DevBuf gq;          // prompt-GEMM activation records (launch_gemm_quant layout)
    DevBuf as;          // attention scores / weights
    DevBuf kqr, kor;    // TurboQuant attention: rotated queries, rotated outputs
    DevBuf msel, mw, mg, mu, md, mlog;  // MoE: selection, weights, gate / up / down outputs
    DevBuf mseg, mslot, mimx, mimh;         // MoE: per-expert slot counts and buckets, Q8_K images of x and h
    DevBuf ck;                              // fgh_checksum_dev: per-workgroup partial sums
    DevBuf h;                               // fgh_matvec_silu_dev: silu(g) * u
    int num_cu = 256;         // compute units (sizes the persistent decode grid)
    bool capturing = false;   // inside fgh_graph_begin / fgh_graph_end
    // Instantiated graphs not yet destroyed hold the scratch addresses they were captured with:
    // while any is alive, a buffer that grows keeps its old allocation here, freed when the last
    // graph is destroyed or the context closes.
    int live_graphs = 0;
    std::vector<void *> retired;
    // failure injection (FGH_FAIL_AT=n at fgh_open): the n-th compute call on this context fails
    // with FGH_ERR before it launches anything, so a caller's CPU fallback can be tested
    int64_t calls = 0, fail_at = 0;
    void *noalloc = nullptr;  // this device's address of the static scratch (null: unavailable)
    // the grouped MoE path's expert kernel (FGH_MOE_KERNEL at fgh_open): int8 MFMA (default) or
    // the VALU lane chains ("valu"); both are bit-identical. moe_nsg: slots per chunk / 4 of the
    // MFMA kernel (FGH_MOE_NSG: 1, 2 or 4; 0 picks by the slots per expert)
    bool moe_valu = false;
    int moe_nsg = 0;
    fgh::MoeMmShape moe_shape;  // FGH_MOE_R / FGH_MOE_TT at fgh_open (ring depth, tiles per wavefront)
    // fgh_moe_block_ints: device dumps of the grouped kernels' integers (gate sumi / msum, down
    // sumi / msum), null otherwise
    int32_t *moe_dump[4] = {nullptr, nullptr, nullptr, nullptr};
};

// fgh_matmul_dev_noalloc's scratch: a static array, one copy per device. Every prompt GEMM keeps
// its activation records here (Q4_K, Q6_K, Q8_0, Q4_0, Q4_1, Q5_0, Q5_1), and the K-split ones
// (Q4_K, Q6_K, Q8_0) their counters and partials after them (prompt_gemm_bytes sizes both). In
// host code its name is only a host-side stand-in; kernels get the device address that
// hipGetSymbolAddress returns with the device current, taken once per device at its first
// fgh_open and kept here.
static __device__ __align__(256) uint8_t scratch[FGH_NOALLOC_SCRATCH_BYTES];
constexpr int MAX_DEVICES = 64;
static std::mutex scratch_mu;
static void *scratch_addr[MAX_DEVICES];
static bool scratch_tried[MAX_DEVICES];

// the device address of scratch on the current device (null if it cannot be had)
static void *scratch_on(int device) {
    if (device < 0 || device >= MAX_DEVICES) return nullptr;
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (!scratch_tried[device]) {
        scratch_tried[device] = true;
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) == hipSuccess) scratch_addr[device] = p;
        else (void)hipGetLastError();
    }
    return scratch_addr[device];
}

// counts one compute call; true (with the context's message set) when it is the injected failure
static bool injected_failure(fgh_ctx *c);

static void free_retired(fgh_ctx *c) {
    if (c->retired.empty()) return;
    (void)hipStreamSynchronize(c->stream);
    for (void *p : c->retired) (void)hipFree(p);
    c->retired.clear();
}

struct fgh_tensor {
    fgh_ctx *ctx;
    uint32_t type;
    int64_t cols, rows, n_mats;
    int order;     // FGH_ORDER_ROW / FGH_ORDER_REPACKED (Q4_K); ROW otherwise
    int nb;        // blocks per row (256-blocks for K-quants, 32-blocks for Q8_0)
    int ntile;     // tiles per row group
    int64_t gpm;   // row tiles per matrix (16 rows for Q4_K, Q5_K, Q2_K, Q3_K and IQ4_XS, 8 otherwise)
    int64_t groups;
    uint8_t *dev;
    uint64_t dev_bytes;
};

static int fail(fgh_ctx *c, int code, const char *fmt, ...) {
    if (c) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof(buf), fmt, ap);
        va_end(ap);
        c->err = buf;
    }
    return code;
}

#define HIP_TRY(ctx, call)                                                                        \
    do {                                                                                          \
        hipError_t e_ = (call);                                                                   \
        if (e_ != hipSuccess) return fail((ctx), FGH_ERR_DEVICE, "%s: %s", #call, hipGetErrorString(e_)); \
    } while (0)

static int grow(fgh_ctx *c, DevBuf &b, size_t need) {
    if (need <= b.cap) return FGH_OK;
    if (c->capturing) return fail(c, FGH_ERR, "a scratch buffer would grow during graph capture");
    if (b.p) {
        if (c->live_graphs > 0) {
            c->retired.push_back(b.p);  // a live graph may still read or write it
        } else {
            HIP_TRY(c, hipStreamSynchronize(c->stream));
            HIP_TRY(c, hipFree(b.p));
        }
        b.p = nullptr;
        b.cap = 0;
    }
    size_t cap = std::max(need, (size_t)1 << 16);
    HIP_TRY(c, hipMalloc(&b.p, cap));
    b.cap = cap;
    return FGH_OK;
}

static bool type_supported(uint32_t t) {
    return fgh::q8_kind((int)t) || t == FGH_T_Q4_K || t == FGH_T_Q6_K || t == FGH_T_Q5_K || fgh::kq_kind((int)t) ||
           fgh::fl_kind((int)t);
}
static bool q16_rows(uint32_t t) { return t == FGH_T_Q4_K || t == FGH_T_Q5_K; }  // 16-row tiles
static int block_elems(uint32_t t) { return fgh::fl_kind((int)t) ? 1 : fgh::q8_kind((int)t) ? 32 : 256; }
static int block_bytes(uint32_t t) {
    switch (t) {
    case FGH_T_Q8_0: return 34;
    case FGH_T_Q5_0: return 22;
    case FGH_T_Q4_0: case FGH_T_IQ4_NL: return 18;
    case FGH_T_Q4_1: return 20;
    case FGH_T_Q5_1: return 24;
    case FGH_T_Q4_K: return 144;
    case FGH_T_Q5_K: return 176;
    case FGH_T_Q2_K: case FGH_T_Q3_K: case FGH_T_IQ4_XS: return fgh::kq_block_bytes((int)t);
    case FGH_T_F32: case FGH_T_F16: case FGH_T_BF16: return fgh::fl_value_bytes((int)t);
    default: return 210;
    }
}
static int tile_bytes(uint32_t t) {
    switch (t) {
    case FGH_T_Q8_0: return fgh::Q80_TILE;
    case FGH_T_Q4_K: return fgh::Q4K_TILE;
    case FGH_T_Q5_K: return fgh::Q5K_TILE;
    case FGH_T_Q6_K: return fgh::Q6K_TILE;
    case FGH_T_Q2_K: case FGH_T_Q3_K: case FGH_T_IQ4_XS: return fgh::kq_tile((int)t);
    case FGH_T_F32: case FGH_T_F16: case FGH_T_BF16: return fgh::FL_TILE;
    default: return fgh::q32_layout((int)t).tile;  // the nibble types
    }
}

// activation buffers for ntok tokens of `cols` values, for the tensor's type
static int ensure_act(fgh_ctx *c, uint32_t type, int64_t cols, int ntok) {
    const int64_t nbk = cols / block_elems(type);
    int rc;
    if (fgh::q8_kind((int)type)) {
        if ((rc = grow(c, c->aqs, (size_t)ntok * nbk * 32)) || (rc = grow(c, c->ad, (size_t)ntok * nbk * 4)) ||
            (rc = grow(c, c->abs, (size_t)ntok * nbk * 4)))
            return rc;
    } else {
        if ((rc = grow(c, c->aqs, (size_t)ntok * nbk * 256)) || (rc = grow(c, c->ad, (size_t)ntok * nbk * 4)) ||
            (rc = grow(c, c->abs, (size_t)ntok * nbk * 32)))
            return rc;
    }
    return FGH_OK;
}

// quantize ntok rows of x (device, row stride ldx) for the type into the context's buffers
static int quantize_dev(fgh_ctx *c, uint32_t type, int64_t cols, const float *x, int64_t ldx, int ntok) {
    int rc = ensure_act(c, type, cols, ntok);
    if (rc) return rc;
    if (fgh::q8_kind((int)type)) {
        fgh::ActQ8 a{(int8_t *)c->aqs.p, (float *)c->ad.p, (int16_t *)c->abs.p};
        HIP_TRY(c, fgh::launch_quant_q8(x, ldx, (int)(cols / 32), ntok, a, c->stream));
    } else {
        fgh::ActQ8K a{(int8_t *)c->aqs.p, (float *)c->ad.p, (int16_t *)c->abs.p};
        HIP_TRY(c, fgh::launch_quant_q8k(x, ldx, (int)(cols / 256), ntok, a, c->stream));
    }
    return FGH_OK;
}

// one decode launch over n tensors that share type, order and width; x: ntok fp32 vectors
// (device, stride ldx); y[i]: outputs of tensor i (token stride ldy)
static int matvec_launch(fgh_ctx *c, int n, const fgh_tensor *const *t, const float *x, int64_t ldx,
                         float *const *y, int64_t ldy, int ntok, int32_t *ds, int32_t *dm,
                         const int32_t *sel = nullptr, int xdiv = 1) {
    fgh::MvArgs a;
    memset(&a, 0, sizeof(a));
    int64_t g = 0;
    for (int i = 0; i < n; i++) {
        a.t[i] = fgh::MvT{t[i]->dev, y[i], t[i]->rows, t[i]->gpm, g};
        g += sel ? t[i]->gpm : t[i]->groups;  // with an expert index: the tiles of one matrix
    }
    a.sel = sel;
    a.xdiv = xdiv;
    a.nt = n;
    a.groups = g;
    a.x = x;
    a.ldx = ldx;
    a.ldy = ldy;
    a.nb = t[0]->nb;
    a.ntile = t[0]->ntile;
    a.dump_s = ds;
    a.dump_m = dm;
    HIP_TRY(c, fgh::launch_matvec2((int)t[0]->type, t[0]->order, a, ntok, c->num_cu, c->stream));
    return FGH_OK;
}

// the prompt GEMM for a Q4_K tensor: quantize T tokens (device X, stride ldx) into the GEMM's
// activation records (buffer act, at least gemm_act_bytes), then one MFMA launch; ds / dm:
// optional [T][rows * n_mats][nb] integer dump
static int gemm_q4k_into(fgh_ctx *c, const fgh_tensor *t, const float *X, int64_t ldx, float *Y, int64_t ldy, int T,
                         uint8_t *act, int32_t *ds, int32_t *dm) {
    const int Tp = (T + 15) / 16 * 16;
    const fgh::GemmScratch gs = fgh::gemm_scratch(t->groups, t->nb, T, c->num_cu);
    int32_t *cnt = gs.ks > 1 ? (int32_t *)(act + gs.cnt_off) : nullptr;
    HIP_TRY(c, fgh::launch_gemm_quant(X, ldx, t->nb, T, Tp, act, cnt, gs.ncnt, c->stream));
    fgh::GemmArgs a;
    memset(&a, 0, sizeof(a));
    a.ks = gs.ks;
    a.cnt = cnt;
    a.part = gs.ks > 1 ? (float *)(act + gs.part_off) : nullptr;
    a.W = t->dev;
    a.Y = Y;
    a.rows = t->rows;
    a.gpm = t->gpm;
    a.groups = t->groups;
    a.nrows = t->rows * t->n_mats;
    a.nb = t->nb;
    a.act = act;
    a.Tp = Tp;
    a.T = T;
    a.ldy = ldy;
    a.dump_s = ds;
    a.dump_m = dm;
    HIP_TRY(c, fgh::launch_q4k_gemm(a, c->stream));
    return FGH_OK;
}
// the prompt GEMM for a Q8_0 tensor (gemm_q32, fastgguf.c:2856-2999): Q8 records of T tokens, then
// one MFMA launch on the decode tiles; ds: optional [T][rows * n_mats][nb] integer dump
// the Q8_0 GEMM's scratch: workgroups of 2 groups of 32 rows, splits of at least 8 tile steps
static fgh::GemmScratch q80_scratch(const fgh_ctx *c, const fgh_tensor *t, int T) {
    const int64_t groups = (t->gpm + 3) / 4 * t->n_mats;
    const int Tp = T <= 32 ? 32 : 64;
    return fgh::gemm_split_scratch(fgh::gemm32_act_bytes(t->nb, Tp), fgh::gemm32_workgroups(groups), (int)t->ntile, 8,
                                   Tp, c->num_cu);
}
static int gemm_q80_into(fgh_ctx *c, const fgh_tensor *t, const float *X, int64_t ldx, float *Y, int64_t ldy, int T,
                         uint8_t *act, int32_t *ds) {
    const int Tp = T <= 32 ? 32 : 64;
    const fgh::GemmScratch gs = q80_scratch(c, t, T);
    int32_t *cnt = gs.ks > 1 ? (int32_t *)(act + gs.cnt_off) : nullptr;
    HIP_TRY(c, fgh::launch_gemm32_quant(X, ldx, t->nb, T, Tp, act, cnt, gs.ncnt, c->stream));
    fgh::Gemm32Args a;
    memset(&a, 0, sizeof(a));
    a.ks = gs.ks;
    a.cnt = cnt;
    a.part = gs.ks > 1 ? (float *)(act + gs.part_off) : nullptr;
    a.W = t->dev;
    a.Y = Y;
    a.rows = t->rows;
    a.tpm = t->gpm;
    a.gpm32 = (t->gpm + 3) / 4;
    a.groups = a.gpm32 * t->n_mats;
    a.nrows = t->rows * t->n_mats;
    a.nb = t->nb;
    a.nsteps = t->ntile;
    a.act = act;
    a.Tp = Tp;
    a.T = T;
    a.ldy = ldy;
    a.dump_s = ds;
    HIP_TRY(c, fgh::launch_q80_gemm(a, c->stream));
    return FGH_OK;
}

// the prompt GEMM for a Q4_0 / Q4_1 / Q5_0 / Q5_1 tensor (gemm_q32, fastgguf.c:2856-2999, in its fp32
// order): Q8 records of T tokens, then one MFMA launch on the decode tiles; ds: optional
// [T][rows * n_mats][nb] dump of the unsigned-weight integers sum u * xq
static int gemm_q32n_into(fgh_ctx *c, const fgh_tensor *t, const float *X, int64_t ldx, float *Y, int64_t ldy, int T,
                          uint8_t *act, int32_t *ds) {
    const int Tp = (T + 15) / 16 * 16;
    HIP_TRY(c, fgh::launch_gemmn_quant(X, ldx, t->nb, T, Tp, act, c->stream));
    fgh::GemmNArgs a;
    memset(&a, 0, sizeof(a));
    a.W = t->dev;
    a.Y = Y;
    a.rows = t->rows;
    a.tpm = t->gpm;
    a.ppm = (t->gpm + 1) / 2;
    a.groups = a.ppm * t->n_mats;
    a.nrows = t->rows * t->n_mats;
    a.nb = t->nb;
    a.nsteps = t->ntile;
    a.act = act;
    a.Tp = Tp;
    a.T = T;
    a.ldy = ldy;
    a.dump_s = ds;
    a.type = (int)t->type;
    HIP_TRY(c, fgh::launch_q32n_gemm(a, c->stream));
    return FGH_OK;
}
static bool q32n_type(uint32_t type) {
    return type == FGH_T_Q4_0 || type == FGH_T_Q4_1 || type == FGH_T_Q5_0 || type == FGH_T_Q5_1;
}

// the prompt GEMM for a Q6_K tensor (gemm_kquant's Q6_K branch, fastgguf.c:2704-2725, 2818-2854):
// Q8_K records of T tokens, then one MFMA launch on the decode tiles; ds / dm: optional
// [T][rows * n_mats][nb] integer dump
// the Q6_K GEMM's scratch (16-row tiles: pairs of the decode layout's 8-row tiles)
static fgh::GemmScratch q6k_scratch(const fgh_ctx *c, const fgh_tensor *t, int T) {
    const int64_t groups16 = (t->gpm + 1) / 2 * t->n_mats;  // 4 per workgroup, splits of >= 4 blocks
    const int Tp = (T + 15) / 16 * 16;
    return fgh::gemm_split_scratch(fgh::gemm6_act_bytes(t->nb, Tp), (groups16 + 3) / 4, t->nb, 4, Tp, c->num_cu);
}
static int gemm_q6k_into(fgh_ctx *c, const fgh_tensor *t, const float *X, int64_t ldx, float *Y, int64_t ldy, int T,
                         uint8_t *act, int32_t *ds, int32_t *dm) {
    const int Tp = (T + 15) / 16 * 16;
    const fgh::GemmScratch gs = q6k_scratch(c, t, T);
    int32_t *cnt = gs.ks > 1 ? (int32_t *)(act + gs.cnt_off) : nullptr;
    HIP_TRY(c, fgh::launch_gemm6_quant(X, ldx, t->nb, T, Tp, act, cnt, gs.ncnt, c->stream));
    fgh::Gemm6Args a;
    memset(&a, 0, sizeof(a));
    a.ks = gs.ks;
    a.cnt = cnt;
    a.part = gs.ks > 1 ? (float *)(act + gs.part_off) : nullptr;
    a.W = t->dev;
    a.Y = Y;
    a.rows = t->rows;
    a.tpm = t->gpm;
    a.gpm16 = (t->gpm + 1) / 2;
    a.groups = a.gpm16 * t->n_mats;
    a.nrows = t->rows * t->n_mats;
    a.nb = t->nb;
    a.act = act;
    a.Tp = Tp;
    a.T = T;
    a.ldy = ldy;
    a.dump_s = ds;
    a.dump_m = dm;
    HIP_TRY(c, fgh::launch_q6k_gemm(a, c->stream));
    return FGH_OK;
}

// the types and token counts that take a prompt GEMM (matmul, fastgguf.c:3018-3031), and the
// activation-record bytes it needs (0: the per-token decode kernels, which need no scratch)
static size_t prompt_gemm_bytes(const fgh_ctx *c, const fgh_tensor *t, int T) {
    if (T < 8) return 0;
    if (t->type == FGH_T_Q4_K) return fgh::gemm_scratch(t->groups, t->nb, T, c->num_cu).bytes;
    if (t->type == FGH_T_Q8_0) return q80_scratch(c, t, T).bytes;
    if (t->type == FGH_T_Q6_K) return q6k_scratch(c, t, T).bytes;
    if (q32n_type(t->type)) return fgh::gemmn_act_bytes(t->nb, (T + 15) / 16 * 16);
    return 0;
}
// the prompt GEMM with its records in act (at least prompt_gemm_bytes)
static int prompt_gemm_into(fgh_ctx *c, const fgh_tensor *t, const float *X, int64_t ldx, float *Y, int64_t ldy,
                            int T, uint8_t *act, int32_t *ds, int32_t *dm) {
    if (t->type == FGH_T_Q8_0) return gemm_q80_into(c, t, X, ldx, Y, ldy, T, act, ds);
    if (t->type == FGH_T_Q6_K) return gemm_q6k_into(c, t, X, ldx, Y, ldy, T, act, ds, dm);
    if (q32n_type(t->type)) return gemm_q32n_into(c, t, X, ldx, Y, ldy, T, act, ds);
    return gemm_q4k_into(c, t, X, ldx, Y, ldy, T, act, ds, dm);
}
static int prompt_gemm(fgh_ctx *c, const fgh_tensor *t, const float *X, int64_t ldx, float *Y, int64_t ldy, int T,
                       int32_t *ds, int32_t *dm) {
    int rc;
    if ((rc = grow(c, c->gq, prompt_gemm_bytes(c, t, T)))) return rc;
    return prompt_gemm_into(c, t, X, ldx, Y, ldy, T, (uint8_t *)c->gq.p, ds, dm);
}

// host-synchronous and allocating calls cannot be recorded into a graph
#define NO_CAPTURE(c) \
    do { \
        if ((c)->capturing) return fail((c), FGH_ERR, "%s: not allowed while capturing a graph", __func__); \
    } while (0)

static bool injected_failure(fgh_ctx *c) {
    if (c->fail_at <= 0 || ++c->calls != c->fail_at) return false;
    char buf[96];
    snprintf(buf, sizeof(buf), "injected failure at compute call %lld (FGH_FAIL_AT)", (long long)c->fail_at);
    c->err = buf;
    return true;
}
#define INJECT(c) \
    do { \
        if (injected_failure(c)) return FGH_ERR; \
    } while (0)

static int check_tensor(fgh_ctx *c, const fgh_tensor *t) {
    if (!c) return FGH_ERR_ARG;
    if (!t || t->ctx != c || !t->dev) return fail(c, FGH_ERR_ARG, "invalid tensor handle");
    return FGH_OK;
}

extern "C" {

static int selfcheck(fgh_ctx *c);

int fgh_open(int device, uint64_t budget_bytes, fgh_ctx **out) {
    if (!out) return FGH_ERR_ARG;
    *out = nullptr;
    // FASTGGUF_GPU=off / 0 / cpu / none keeps the caller on its CPU path without touching a
    // device, and FASTGGUF_GPU_DEVICE picks the device when the caller passes device < 0
    // (fg_gpu_init_ex, fastgguf.c:1972-1982)
    if (const char *env = getenv("FASTGGUF_GPU"))
        if (!strcmp(env, "off") || !strcmp(env, "0") || !strcmp(env, "cpu") || !strcmp(env, "none"))
            return FGH_ERR_DEVICE;
    if (device < 0)
        if (const char *dev = getenv("FASTGGUF_GPU_DEVICE")) device = atoi(dev);
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return FGH_ERR_DEVICE;
    if (device < 0) device = 0;
    if (device >= n) return FGH_ERR_ARG;
    if (hipSetDevice(device) != hipSuccess) return FGH_ERR_DEVICE;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) return FGH_ERR_DEVICE;
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) return FGH_ERR_DEVICE;  // kernels are built for gfx950 only
    fgh_ctx *c = new fgh_ctx();
    c->device = device;
    snprintf(c->name, sizeof(c->name), "%s (%s)", prop.name, prop.gcnArchName);
    c->vram = prop.totalGlobalMem;
    c->budget = budget_bytes ? budget_bytes : c->vram - c->vram / 8;
    c->num_cu = std::max(1, prop.multiProcessorCount);
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return FGH_ERR_DEVICE;
    }
    c->noalloc = scratch_on(device);  // the device is current
    if (selfcheck(c) != FGH_OK) {  // gpu_selfcheck gates use (fastgguf.c:2048-2052)
        fgh_close(c);
        return FGH_ERR_DEVICE;
    }
    if (const char *f = getenv("FGH_FAIL_AT")) c->fail_at = atoll(f);
    if (const char *m = getenv("FGH_MOE_KERNEL")) c->moe_valu = !strcmp(m, "valu");
    if (const char *m = getenv("FGH_MOE_NSG")) c->moe_nsg = atoi(m);
    if (const char *m = getenv("FGH_MOE_R")) c->moe_shape.r = atoi(m);
    if (const char *m = getenv("FGH_MOE_TT")) c->moe_shape.tt = atoi(m);
    *out = c;
    return FGH_OK;
}

void fgh_close(fgh_ctx *c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);
    for (DevBuf *b : {&c->x, &c->y, &c->aqs, &c->ad, &c->abs, &c->gq, &c->msel, &c->mw, &c->mg,
                      &c->mu, &c->md, &c->mlog, &c->mseg, &c->mslot, &c->mimx, &c->mimh, &c->ck, &c->as, &c->kqr,
                      &c->kor, &c->h})
        if (b->p) (void)hipFree(b->p);
    free_retired(c);
    (void)hipStreamDestroy(c->stream);
    delete c;
}

int fgh_info(const fgh_ctx *c, fgh_info_t *out) {
    if (!c || !out) return FGH_ERR_ARG;
    memset(out, 0, sizeof(*out));
    out->vram = c->vram;
    out->budget = c->budget;
    out->used = c->used;
    out->n_offloaded = c->n_offloaded;
    out->n_skip_type = c->n_skip_type;
    out->n_skip_mem = c->n_skip_mem;
    out->device = c->device;
    snprintf(out->name, sizeof(out->name), "%s", c->name);
    return FGH_OK;
}

const char *fgh_last_error(const fgh_ctx *c) { return c ? c->err.c_str() : "no context"; }

int fgh_upload(fgh_ctx *c, uint32_t type, int64_t cols, int64_t rows, int64_t n_mats, int order,
               const void *host, uint64_t nbytes, fgh_tensor **out) {
    if (!c || !out) return FGH_ERR_ARG;
    NO_CAPTURE(c);
    *out = nullptr;
    if (!host || rows <= 0 || n_mats <= 0 || cols <= 0) return fail(c, FGH_ERR_ARG, "upload: bad shape");
    // the order the tensor will use: the reference repacks 2-D Q4_K and Q4_0 matrices with
    // rows % 8 == 0 (repack_tensor, 2486-2489)
    const int ord = (type == FGH_T_Q4_K || type == FGH_T_Q4_0) &&
                            (order == FGH_ORDER_REPACKED || (order == FGH_ORDER_AUTO && n_mats == 1 && rows % 8 == 0))
                        ? FGH_ORDER_REPACKED
                        : FGH_ORDER_ROW;
    // the decode kernels stage x in LDS: up to 64 KiB (the float types, whose x stays fp32: 160 KiB)
    const size_t lds_max = fgh::fl_kind((int)type) ? fgh::GEMM_LDS_MAX : 65536;
    if (!type_supported(type) || cols % block_elems(type) != 0 ||
        fgh::matvec_lds_bytes((int)type, ord, (int)std::min<int64_t>(cols / block_elems(type), 1 << 20)) > lds_max) {
        c->n_skip_type++;
        return fail(c, FGH_SKIP_TYPE, "upload: type %u with %lld cols is not supported", type, (long long)cols);
    }
    const int64_t row_bytes = cols / block_elems(type) * block_bytes(type);
    int64_t want = 0;
    if (__builtin_mul_overflow(row_bytes, rows, &want) || __builtin_mul_overflow(want, n_mats, &want))
        return fail(c, FGH_ERR_ARG, "upload: the tensor's byte count overflows");
    if ((uint64_t)want != nbytes)
        return fail(c, FGH_ERR_ARG, "upload: nbytes %llu != %lld", (unsigned long long)nbytes, (long long)want);
    HIP_TRY(c, hipSetDevice(c->device));
    fgh_tensor *t = new fgh_tensor();
    t->ctx = c;
    t->type = type;
    t->cols = cols;
    t->rows = rows;
    t->n_mats = n_mats;
    t->nb = (int)(cols / block_elems(type));
    t->ntile = fgh::fl_kind((int)type) ? (int)((cols + fgh::fl_step_elems((int)type) - 1) / fgh::fl_step_elems((int)type))
               : fgh::q8_kind((int)type) ? (t->nb + 3) / 4
                                          : t->nb;
    const int tile_rows = q16_rows(type)               ? fgh::Q4K_TILE_ROWS
                          : fgh::kq_kind((int)type) ? fgh::KQ_TILE_ROWS
                          : fgh::fl_kind((int)type) ? fgh::fl_tile_rows((int)type)
                                                    : 8;
    t->gpm = (rows + tile_rows - 1) / tile_rows;
    t->groups = t->gpm * n_mats;
    t->order = ord;
    int64_t dev_bytes = 0;
    if (__builtin_mul_overflow(t->groups, (int64_t)t->ntile * tile_bytes(type), &dev_bytes)) {
        delete t;
        return fail(c, FGH_ERR_ARG, "upload: the device copy's byte count overflows");
    }
    t->dev_bytes = (uint64_t)dev_bytes;
    if (t->dev_bytes > c->budget || c->used + t->dev_bytes > c->budget) {
        delete t;
        c->n_skip_mem++;
        return fail(c, FGH_SKIP_MEM, "upload: budget exceeded");
    }
    void *stage = nullptr;
    if (hipMalloc(&t->dev, t->dev_bytes) != hipSuccess || hipMalloc(&stage, nbytes) != hipSuccess) {
        if (t->dev) (void)hipFree(t->dev);
        delete t;
        c->n_skip_mem++;
        (void)hipGetLastError();
        return fail(c, FGH_SKIP_MEM, "upload: device allocation failed");
    }
    hipError_t e = hipMemcpy(stage, host, nbytes, hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = q16_rows(type)
                ? fgh::launch_q4k_relayout((int)type, (const uint8_t *)stage, t->dev, rows, t->nb, t->gpm,
                                           (int64_t)t->dev_bytes, row_bytes, c->stream)
            : fgh::kq_kind((int)type)
                ? fgh::launch_kq_relayout((int)type, (const uint8_t *)stage, t->dev, rows, t->nb, t->gpm,
                                          (int64_t)t->dev_bytes, row_bytes, c->stream)
            : fgh::fl_kind((int)type)
                ? fgh::launch_fl_relayout((int)type, (const uint8_t *)stage, t->dev, rows, cols, t->ntile, t->gpm,
                                          (int64_t)t->dev_bytes, c->stream)
                : fgh::launch_relayout((const uint8_t *)stage, t->dev, (int)type, rows, t->nb, t->ntile, t->gpm,
                                       (int64_t)t->dev_bytes, row_bytes, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    (void)hipFree(stage);
    if (e != hipSuccess) {
        (void)hipFree(t->dev);
        delete t;
        return fail(c, FGH_ERR_DEVICE, "upload: %s", hipGetErrorString(e));
    }
    c->used += t->dev_bytes;
    c->n_offloaded++;
    *out = t;
    return FGH_OK;
}

void fgh_tensor_free(fgh_tensor *t) {
    if (!t) return;
    if (t->dev) {
        (void)hipSetDevice(t->ctx->device);
        (void)hipStreamSynchronize(t->ctx->stream);
        (void)hipFree(t->dev);
        t->ctx->used -= t->dev_bytes;
    }
    delete t;
}

// ---- device-resident entry points ----

int fgh_matvec_multi_dev(fgh_ctx *c, int n, const fgh_tensor *const *t, const float *x, float *const *y) {
    if (!c || !t || !x || !y || n < 1 || n > 4) return fail(c, FGH_ERR_ARG, "matvec_multi: bad arguments");
    int rc;
    for (int i = 0; i < n; i++) {
        if ((rc = check_tensor(c, t[i]))) return rc;
        if (!y[i]) return fail(c, FGH_ERR_ARG, "matvec_multi: null output");
        if (t[i]->cols != t[0]->cols) return fail(c, FGH_ERR_ARG, "matvec_multi: tensors differ in cols");
    }
    INJECT(c);
    HIP_TRY(c, hipSetDevice(c->device));
    // tensors of the same type and order run in one launch (matvec_multi, fastgguf.c:2552-2572)
    bool done[4] = {false, false, false, false};
    for (int i = 0; i < n; i++) {
        if (done[i]) continue;
        const fgh_tensor *grp[4];
        float *ys[4];
        int m = 0;
        for (int j = i; j < n; j++)
            if (!done[j] && t[j]->type == t[i]->type && t[j]->order == t[i]->order) {
                grp[m] = t[j];
                ys[m++] = y[j];
                done[j] = true;
            }
        if ((rc = matvec_launch(c, m, grp, x, t[0]->cols, ys, 0, 1, nullptr, nullptr))) return rc;
    }
    return FGH_OK;
}

int fgh_matvec_dev(fgh_ctx *c, const fgh_tensor *t, const float *x, float *y) {
    const fgh_tensor *tt[1] = {t};
    float *yy[1] = {y};
    return fgh_matvec_multi_dev(c, 1, tt, x, yy);
}

int fgh_matvec_silu_dev(fgh_ctx *c, const fgh_tensor *t, const float *g, const float *u, float *y) {
    int rc = check_tensor(c, t);
    if (rc) return rc;
    if (!g || !u || !y) return fail(c, FGH_ERR_ARG, "matvec_silu: null pointer");
    INJECT(c);
    HIP_TRY(c, hipSetDevice(c->device));
    // h once (one short launch), then the plain matvec: forming h inside the matvec's quantization
    // would repeat its expf in every workgroup
    if ((rc = grow(c, c->h, (size_t)t->cols * 4))) return rc;
    float *h = (float *)c->h.p;
    HIP_TRY(c, fgh::launch_silu_mul(g, u, h, t->cols, c->stream));
    float *yy[1] = {y};
    return matvec_launch(c, 1, &t, h, t->cols, yy, t->rows * t->n_mats, 1, nullptr, nullptr);
}

int fgh_matvec_gate_up_silu_dev(fgh_ctx *c, const fgh_tensor *gate, const fgh_tensor *up, const float *x, float *h) {
    int rc;
    if ((rc = check_tensor(c, gate)) || (rc = check_tensor(c, up))) return rc;
    if (!x || !h) return fail(c, FGH_ERR_ARG, "matvec_gate_up_silu: null pointer");
    if (gate->cols != up->cols || gate->rows != up->rows || gate->n_mats != 1 || up->n_mats != 1)
        return fail(c, FGH_ERR_ARG, "matvec_gate_up_silu: gate and up must be single matrices of one shape");
    INJECT(c);
    HIP_TRY(c, hipSetDevice(c->device));
    const int64_t rows = gate->rows;
    if (q16_rows(gate->type) && gate->type == up->type && gate->order == up->order) {
        // one launch: a workgroup holds gate and up tiles of the same rows and writes their h
        fgh::MvArgs a;
        memset(&a, 0, sizeof(a));
        a.t[0] = fgh::MvT{gate->dev, h, rows, gate->gpm, 0};
        a.t[1] = fgh::MvT{up->dev, nullptr, rows, up->gpm, gate->gpm};
        a.nt = 2;
        a.groups = gate->gpm + up->gpm;
        a.x = x;
        a.ldx = gate->cols;
        a.ldy = rows;
        a.nb = gate->nb;
        a.ntile = gate->ntile;
        a.xdiv = 1;
        a.pair = 1;
        HIP_TRY(c, fgh::launch_matvec2((int)gate->type, gate->order, a, 1, c->num_cu, c->stream));
        return FGH_OK;
    }
    // other types: g into h and u into scratch (one launch when their type and order agree),
    // then h = silu(h) * u
    if ((rc = grow(c, c->h, (size_t)rows * 4))) return rc;
    float *u = (float *)c->h.p;
    if (gate->type == up->type && gate->order == up->order) {
        const fgh_tensor *gu[2] = {gate, up};
        float *ys[2] = {h, u};
        if ((rc = matvec_launch(c, 2, gu, x, gate->cols, ys, rows, 1, nullptr, nullptr))) return rc;
    } else {
        float *yg[1] = {h}, *yu[1] = {u};
        if ((rc = matvec_launch(c, 1, &gate, x, gate->cols, yg, rows, 1, nullptr, nullptr)) ||
            (rc = matvec_launch(c, 1, &up, x, up->cols, yu, rows, 1, nullptr, nullptr)))
            return rc;
    }
    HIP_TRY(c, fgh::launch_silu_mul(h, u, h, rows, c->stream));
    return FGH_OK;
}

int fgh_ffn_dev(fgh_ctx *c, const fgh_tensor *gate, const fgh_tensor *up, const fgh_tensor *down, const float *x,
                float *h, float *y) {
    int rc;
    if ((rc = check_tensor(c, gate)) || (rc = check_tensor(c, up)) || (rc = check_tensor(c, down))) return rc;
    if (!x || !h || !y) return fail(c, FGH_ERR_ARG, "ffn: null pointer");
    if (down->n_mats != 1 || down->cols != gate->rows)
        return fail(c, FGH_ERR_ARG, "ffn: down must be one matrix whose columns are gate's rows");
    // the paired gate / up launch writes h (or the matvecs and the silu launch), then down reads it
    if ((rc = fgh_matvec_gate_up_silu_dev(c, gate, up, x, h))) return rc;
    return fgh_matvec_dev(c, down, h, y);
}

int fgh_matmul_dev(fgh_ctx *c, const fgh_tensor *t, const float *X, int ldx, float *Y, int ldy, int nb) {
    int rc = check_tensor(c, t);
    if (rc) return rc;
    if (!X || !Y || nb < 1 || nb > FG_BATCH || ldx < t->cols || ldy < t->rows * t->n_mats)
        return fail(c, FGH_ERR_ARG, "matmul: bad arguments");
    INJECT(c);
    HIP_TRY(c, hipSetDevice(c->device));
    // nb >= 8: the prompt GEMMs (matmul 3018-3031) on int8 MFMA for Q4_K, Q6_K, Q8_0 and the nibble
    // types Q4_0 / Q4_1 / Q5_0 / Q5_1; Q5_K, IQ4_NL, Q2_K, Q3_K and IQ4_XS, which have no GEMM in the
    // reference, run the per-token decode kernels as its matmul does
    if (prompt_gemm_bytes(c, t, nb)) return prompt_gemm(c, t, X, ldx, Y, ldy, nb, nullptr, nullptr);
    float *ys[1] = {Y};
    return matvec_launch(c, 1, &t, X, ldx, ys, ldy, nb, nullptr, nullptr);
}

int fgh_matmul_dev_noalloc(fgh_ctx *c, const fgh_tensor *t, const float *X, int ldx, float *Y, int ldy, int nb) {
    int rc = check_tensor(c, t);
    if (rc) return rc;
    if (!X || !Y || nb < 1 || nb > FG_BATCH || ldx < t->cols || ldy < t->rows * t->n_mats)
        return fail(c, FGH_ERR_ARG, "matmul_dev_noalloc: bad arguments");
    const size_t need = prompt_gemm_bytes(c, t, nb);  // the prompt GEMMs are the paths with scratch
    const bool gemm = need > 0;
    if (gemm) {
        if (need > FGH_NOALLOC_SCRATCH_BYTES)
            return fail(c, FGH_ERR_ARG,
                        "matmul_dev_noalloc: %d tokens x %lld columns need %zu bytes of scratch, more than its %u",
                        nb, (long long)t->cols, need, FGH_NOALLOC_SCRATCH_BYTES);
        if (!c->noalloc)
            return fail(c, FGH_ERR_DEVICE, "matmul_dev_noalloc: no device address for the static scratch");
    }
    INJECT(c);
    HIP_TRY(c, hipSetDevice(c->device));
    if (gemm) return prompt_gemm_into(c, t, X, ldx, Y, ldy, nb, (uint8_t *)c->noalloc, nullptr, nullptr);
    float *ys[1] = {Y};
    return matvec_launch(c, 1, &t, X, ldx, ys, ldy, nb, nullptr, nullptr);
}

int fgh_moe_ffn_dev(fgh_ctx *c, const fgh_tensor *gate, const fgh_tensor *up, const fgh_tensor *down, int k,
                    const float *logits, const float *X, float *Y, int n_tok) {
    int rc;
    if ((rc = check_tensor(c, gate)) || (rc = check_tensor(c, up)) || (rc = check_tensor(c, down))) return rc;
    const int64_t E = gate->n_mats, n_embd = gate->cols, ff = gate->rows;
    if (up->n_mats != E || up->cols != n_embd || up->rows != ff || down->n_mats != E || down->cols != ff ||
        down->rows != n_embd)
        return fail(c, FGH_ERR_ARG, "moe_ffn: gate/up must be [E][ff][n_embd] and down [E][n_embd][ff]");
    if (!logits || !X || !Y || n_tok < 1 || n_tok > FG_BATCH || k < 1 || k > E || k > 64 || E > 512)
        return fail(c, FGH_ERR_ARG, "moe_ffn: bad arguments (k %d, experts %lld, tokens %d)", k, (long long)E, n_tok);
    INJECT(c);
    HIP_TRY(c, hipSetDevice(c->device));
    const int64_t np = (int64_t)n_tok * k;  // (token, selected expert) slots
    if ((rc = grow(c, c->msel, (size_t)np * 4)) || (rc = grow(c, c->mw, (size_t)np * 4)) ||
        (rc = grow(c, c->mg, (size_t)np * ff * 4)) || (rc = grow(c, c->mu, (size_t)np * ff * 4)) ||
        (rc = grow(c, c->md, (size_t)np * n_embd * 4)))
        return rc;
    int32_t *sel = (int32_t *)c->msel.p;
    float *w = (float *)c->mw.p, *G = (float *)c->mg.p, *U = (float *)c->mu.p,
          *D = (float *)c->md.p;
    // several tokens, Q4_K experts: the slots grouped by expert, each expert's rows read once, on
    // int8 MFMA (or, FGH_MOE_KERNEL=valu, the VALU lane chains; same bits)
    const bool q4row = n_tok > 1 && gate->type == FGH_T_Q4_K && up->type == FGH_T_Q4_K && down->type == FGH_T_Q4_K &&
                       gate->order == FGH_ORDER_ROW && up->order == FGH_ORDER_ROW && down->order == FGH_ORDER_ROW;
    // MFMA chunks: 4 slots per group, 2 groups (an expert with more slots gets more workgroups)
    int nsg = c->moe_nsg == 1 || c->moe_nsg == 2 || c->moe_nsg == 4 ? c->moe_nsg : 2;
    const int nbx = std::max(gate->nb, down->nb);
    while (nsg > 1 && fgh::q4k_moe_mfma_lds(nsg, nbx) > fgh::GEMM_LDS_MAX) nsg /= 2;
    const bool mfma_fits = fgh::q4k_moe_mfma_lds(nsg, nbx) <= fgh::GEMM_LDS_MAX && gate->gpm == up->gpm;
    const bool valu_fits = gate->nb <= fgh::q4k_moe_max_blocks() && down->nb <= fgh::q4k_moe_max_blocks() &&
                           fgh::q4k_moe_lds_bytes(gate->nb) <= 65536 && fgh::q4k_moe_lds_bytes(down->nb) <= 65536;
    const bool use_valu = c->moe_valu ? valu_fits : !mfma_fits;
    const bool grouped = q4row && (use_valu ? valu_fits : mfma_fits);
    // Q4_K / Q5_K experts otherwise: two launches. Gate and up route each token inside the
    // launch (every wavefront routes its own token: the weights it streams depend on the choice),
    // publish sel / w and write h = silu(g) * u (a workgroup holds the gate and up tiles of the
    // same rows); down quantizes each slot's h and sums the k experts' rows in order (the
    // combine), so neither the routing nor the down rows take a launch of their own.
    const bool kq = (gate->type == FGH_T_Q4_K || gate->type == FGH_T_Q5_K) &&
                    (down->type == FGH_T_Q4_K || down->type == FGH_T_Q5_K);
    const bool fold = kq && !grouped && gate->type == up->type && gate->order == up->order &&
                      down->order == FGH_ORDER_ROW && k <= 8 &&
                      fgh::q4k_moe_down_lds(down->nb, k) <= fgh::GEMM_LDS_MAX &&
                      fgh::q4k_route_fits((int)gate->type, gate->order, (gate->gpm + up->gpm) * np, gate->nb, c->num_cu);
    if (fold) {
        fgh::MvArgs a;
        memset(&a, 0, sizeof(a));
        a.t[0] = fgh::MvT{gate->dev, G, gate->rows, gate->gpm, 0};
        a.t[1] = fgh::MvT{up->dev, U, up->rows, up->gpm, gate->gpm};
        a.nt = 2;
        a.groups = gate->gpm + up->gpm;
        a.x = X;
        a.ldx = n_embd;
        a.ldy = ff;
        a.nb = gate->nb;
        a.ntile = gate->ntile;
        a.xdiv = k;
        a.logits = logits;
        a.n_expert = (int)E;
        a.sel_out = sel;
        a.w_out = w;
        HIP_TRY(c, fgh::launch_matvec2((int)gate->type, gate->order, a, (int)np, c->num_cu, c->stream));
        memset(&a, 0, sizeof(a));
        a.t[0] = fgh::MvT{down->dev, Y, down->rows, down->gpm, 0};
        a.nt = 1;
        a.groups = down->gpm;
        a.x = G;  // h
        a.ldx = ff;
        a.ldy = n_embd;
        a.nb = down->nb;
        a.sel = sel;
        HIP_TRY(c, fgh::launch_q4k_moe_down((int)down->type, a, w, k, n_tok, c->stream));
        return FGH_OK;
    }
    if (grouped) {
        // one launch for the x images, the routing and the slots filed by expert; the grouped
        // kernels read the buckets; the combine clears their counts for the next call
        const size_t ibx = fgh::q4_image_bytes(gate->nb), ibh = fgh::q4_image_bytes(down->nb);
        void *cnt_before = c->mseg.p;
        // a bucket holds every slot of the call (a token may pick one expert more than once)
        const int cap = (int)np;
        if ((rc = grow(c, c->mseg, (size_t)E * 4)) || (rc = grow(c, c->mslot, (size_t)E * cap * 4)) ||
            (rc = grow(c, c->mimx, (size_t)n_tok * ibx)) || (rc = grow(c, c->mimh, (size_t)np * ibh)))
            return rc;
        int32_t *cnt = (int32_t *)c->mseg.p, *buckets = (int32_t *)c->mslot.p;
        if (c->mseg.p != cnt_before) HIP_TRY(c, fgh::launch_zero_i32(cnt, (int)(c->mseg.cap / 4), c->stream));  // new: zero once
        uint8_t *imx = (uint8_t *)c->mimx.p, *imh = (uint8_t *)c->mimh.p;
        HIP_TRY(c, fgh::launch_moe_prep(X, n_embd, gate->nb, imx, logits, (int)E, k, n_tok, sel, w, cnt, buckets,
                                        c->stream));
        // from here the counts are non-zero until the combine clears them: a failed launch clears
        // them itself, so the next call starts from zero
        auto fail_reset = [&](const char *what, hipError_t e) {
            (void)fgh::launch_zero_i32(cnt, (int)E, c->stream);
            return fail(c, FGH_ERR_DEVICE, "moe_ffn: %s: %s", what, hipGetErrorString(e));
        };
        hipError_t e;
        if (!use_valu) {
            // gate / up on MFMA, writing the h images; down on MFMA; the ordered combine
            fgh::MoeMmShape sh = c->moe_shape;
            sh.nsg = nsg;
            if ((e = fgh::launch_q4k_moe_mfma(sh, gate->dev, up->dev, ff, gate->gpm, gate->nb, cnt, buckets, cap, (int)E,
                                               n_tok, imx, k, G, U, ff, c->moe_dump[0], c->moe_dump[1], c->num_cu,
                                               c->stream)) != hipSuccess)
                return fail_reset("gate / up experts", e);
            // h = silu(g) * u, quantized straight into its images (never stored as fp32)
            if ((e = fgh::launch_q4_image(G, U, ff, down->nb, np, imh, c->stream)) != hipSuccess)
                return fail_reset("silu images", e);
            if ((e = fgh::launch_q4k_moe_mfma(sh, down->dev, nullptr, n_embd, down->gpm, down->nb, cnt, buckets, cap,
                                               (int)E, n_tok, imh, 1, D, nullptr, n_embd, c->moe_dump[2], c->moe_dump[3],
                                               c->num_cu, c->stream)) != hipSuccess)
                return fail_reset("down experts", e);
            if ((e = fgh::launch_moe_combine(D, w, Y, (int)n_embd, k, n_tok, n_embd, cnt, (int)E, c->stream)) != hipSuccess)
                return fail_reset("combine", e);
            return FGH_OK;
        }
        auto experts = [&](const fgh::MvArgs &aa, const uint8_t *img) {
            return fgh::launch_q4k_moe(aa, cnt, buckets, cap, (int)E, img, c->stream);
        };
        fgh::MvArgs a;
        memset(&a, 0, sizeof(a));
        a.t[0] = fgh::MvT{gate->dev, G, gate->rows, gate->gpm, 0};
        a.t[1] = fgh::MvT{up->dev, U, up->rows, up->gpm, gate->gpm};
        a.nt = 2;
        a.groups = gate->gpm + up->gpm;
        a.x = X;
        a.ldx = n_embd;
        a.ldy = ff;
        a.nb = gate->nb;
        a.xdiv = k;
        if ((e = experts(a, imx)) != hipSuccess) return fail_reset("gate / up experts", e);
        // h = silu(g) * u, quantized straight into its images (never stored as fp32)
        if ((e = fgh::launch_q4_image(G, U, ff, down->nb, np, imh, c->stream)) != hipSuccess)
            return fail_reset("silu images", e);
        a.t[0] = fgh::MvT{down->dev, D, down->rows, down->gpm, 0};
        a.nt = 1;
        a.groups = down->gpm;
        a.x = nullptr;
        a.ldy = n_embd;
        a.nb = down->nb;
        a.xdiv = 1;
        if ((e = experts(a, imh)) != hipSuccess) return fail_reset("down experts", e);
        if ((e = fgh::launch_moe_combine(D, w, Y, (int)n_embd, k, n_tok, n_embd, cnt, (int)E, c->stream)) != hipSuccess)
            return fail_reset("combine", e);
        return FGH_OK;
    }
    HIP_TRY(c, fgh::launch_moe_route(logits, (int)E, k, n_tok, sel, w, c->stream));
    // gate and up: one launch when their type and order agree (both read the same x row)
    if (gate->type == up->type && gate->order == up->order) {
        const fgh_tensor *gu[2] = {gate, up};
        float *ys[2] = {G, U};
        if ((rc = matvec_launch(c, 2, gu, X, n_embd, ys, ff, (int)np, nullptr, nullptr, sel, k))) return rc;
    } else {
        float *yg[1] = {G}, *yu[1] = {U};
        if ((rc = matvec_launch(c, 1, &gate, X, n_embd, yg, ff, (int)np, nullptr, nullptr, sel, k)) ||
            (rc = matvec_launch(c, 1, &up, X, n_embd, yu, ff, (int)np, nullptr, nullptr, sel, k)))
            return rc;
    }
    // down on h = silu(g) * u (formed in place of g)
    HIP_TRY(c, fgh::launch_silu_mul(G, U, G, np * ff, c->stream));
    float *yd[1] = {D};
    if ((rc = matvec_launch(c, 1, &down, G, ff, yd, n_embd, (int)np, nullptr, nullptr, sel, 1))) return rc;
    HIP_TRY(c, fgh::launch_moe_combine(D, w, Y, (int)n_embd, k, n_tok, n_embd, nullptr, 0, c->stream));
    return FGH_OK;
}

int fgh_attention_dev(fgh_ctx *c, int n_tok, int n_head, int n_head_kv, int hd, const float *q, float *o,
                      const float *k_cache, const float *v_cache, int kv_dim, int cap, const int32_t *st,
                      const int32_t *en, int max_len, float scale) {
    if (!c) return FGH_ERR_ARG;
    if (!q || !o || !k_cache || !v_cache || !st || !en || n_tok < 1 || n_head < 1 || n_head_kv < 1 ||
        n_head % n_head_kv != 0 || hd < 1 || hd > 256 || (int64_t)n_head_kv * hd > kv_dim || cap < 1 || max_len < 1)
        return fail(c, FGH_ERR_ARG, "attention: bad arguments");
    // the vector path (hd % 32 == 0) reads q and the caches 16 bytes at a time
    if (hd % 32 == 0 && (kv_dim % 4 != 0 || ((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache) % 16 != 0))
        return fail(c, FGH_ERR_ARG, "attention: for hd %% 32 == 0, kv_dim %% 4 == 0 and 16-byte aligned q and caches");
    if (((uintptr_t)q | (uintptr_t)o | (uintptr_t)k_cache | (uintptr_t)v_cache) % 4 != 0)
        return fail(c, FGH_ERR_ARG, "attention: q, o and the caches must be 4-byte aligned");
    if ((n_tok * (n_head / n_head_kv) + 3) / 4 > 65535 || n_head_kv > 65535 || (int64_t)n_tok * n_head > INT32_MAX / 2)
        return fail(c, FGH_ERR_ARG, "attention: too many rows");
    INJECT(c);
    HIP_TRY(c, hipSetDevice(c->device));
    int rc;
    if ((rc = grow(c, c->as, (size_t)n_tok * n_head * max_len * 4))) return rc;
    fgh::AttnArgs a{q, o, k_cache, v_cache, (float *)c->as.p, st, en, n_head, n_head_kv, hd, kv_dim, cap, max_len,
                    scale};
    HIP_TRY(c, fgh::launch_attention(a, n_tok, c->stream));
    return FGH_OK;
}

static bool kvq_shape_ok(int hd, int kbits, int vbits) {
    return hd >= 32 && hd <= 256 && (hd & (hd - 1)) == 0 && (kbits == 4 || kbits == 8) &&
           (vbits == 2 || vbits == 4 || vbits == 8);
}

int fgh_kvq_store_dev(fgh_ctx *c, int n_tok, int n_head_kv, int hd, int kbits, int vbits, const float *k,
                      const float *v, int stride, uint8_t *kq, uint8_t *vq, int cap, const int32_t *pos) {
    if (!c) return FGH_ERR_ARG;
    if (!k || !v || !kq || !vq || !pos || n_tok < 1 || n_tok > 65535 || n_head_kv < 1 || n_head_kv > 65535 ||
        cap < 1 || !kvq_shape_ok(hd, kbits, vbits) || (int64_t)n_head_kv * hd > stride)
        return fail(c, FGH_ERR_ARG, "kvq_store: bad arguments");
    if (((uintptr_t)kq | (uintptr_t)vq) % 16 != 0)
        return fail(c, FGH_ERR_ARG, "kvq_store: the caches must be 16-byte aligned");
    INJECT(c);
    HIP_TRY(c, hipSetDevice(c->device));
    fgh::KvqStoreArgs a{k, v, kq, vq, pos, stride, n_head_kv, hd, kbits, vbits, cap};
    HIP_TRY(c, fgh::launch_kvq_store(a, n_tok, c->stream));
    return FGH_OK;
}

int fgh_kvq_attention_dev(fgh_ctx *c, int n_tok, int n_head, int n_head_kv, int hd, int kbits, int vbits,
                          const float *q, float *o, const uint8_t *kq, const uint8_t *vq, int cap, const int32_t *st,
                          const int32_t *en, int max_len, float scale) {
    if (!c) return FGH_ERR_ARG;
    if (!q || !o || !kq || !vq || !st || !en || n_tok < 1 || n_head < 1 || n_head_kv < 1 ||
        n_head % n_head_kv != 0 || cap < 1 || max_len < 1 || !kvq_shape_ok(hd, kbits, vbits) ||
        (int64_t)n_tok * n_head > 65535)
        return fail(c, FGH_ERR_ARG, "kvq_attention: bad arguments");
    if (((uintptr_t)q | (uintptr_t)kq | (uintptr_t)vq) % 16 != 0)
        return fail(c, FGH_ERR_ARG, "kvq_attention: q and the caches must be 16-byte aligned");
    INJECT(c);
    HIP_TRY(c, hipSetDevice(c->device));
    const size_t rows = (size_t)n_tok * n_head;
    int rc;
    if ((rc = grow(c, c->as, rows * max_len * 4)) || (rc = grow(c, c->kqr, rows * hd * 4)) ||
        (rc = grow(c, c->kor, rows * hd * 4)))
        return rc;
    fgh::KvqAttnArgs a{q,  o,  (float *)c->kqr.p, (float *)c->kor.p, (float *)c->as.p, kq, vq, st, en,
                       n_head, n_head_kv, hd, kbits, vbits, cap, max_len, scale};
    HIP_TRY(c, fgh::launch_kvq_attention(a, n_tok, c->stream));
    return FGH_OK;
}

// ---- host-pointer entry points (synchronous) ----

int fgh_matvec_multi(fgh_ctx *c, int n, const fgh_tensor *const *t, const float *x, float *const *y) {
    if (!c || !t || !x || !y || n < 1 || n > 4) return fail(c, FGH_ERR_ARG, "matvec_multi: bad arguments");
    NO_CAPTURE(c);
    int rc;
    int64_t total = 0;
    for (int i = 0; i < n; i++) {
        if ((rc = check_tensor(c, t[i]))) return rc;
        total += t[i]->rows * t[i]->n_mats;
    }
    HIP_TRY(c, hipSetDevice(c->device));
    if ((rc = grow(c, c->x, (size_t)t[0]->cols * 4)) || (rc = grow(c, c->y, (size_t)total * 4))) return rc;
    HIP_TRY(c, hipMemcpyAsync(c->x.p, x, (size_t)t[0]->cols * 4, hipMemcpyHostToDevice, c->stream));
    float *yd[4];
    int64_t off = 0;
    for (int i = 0; i < n; i++) {
        yd[i] = (float *)c->y.p + off;
        off += t[i]->rows * t[i]->n_mats;
    }
    if ((rc = fgh_matvec_multi_dev(c, n, t, (const float *)c->x.p, yd))) return rc;
    for (int i = 0; i < n; i++)
        HIP_TRY(c, hipMemcpyAsync(y[i], yd[i], (size_t)(t[i]->rows * t[i]->n_mats) * 4, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    return FGH_OK;
}

int fgh_matvec(fgh_ctx *c, const fgh_tensor *t, const float *x, float *y) {
    const fgh_tensor *tt[1] = {t};
    float *yy[1] = {y};
    return fgh_matvec_multi(c, 1, tt, x, yy);
}

int fgh_matmul(fgh_ctx *c, const fgh_tensor *t, const float *X, int ldx, float *Y, int ldy, int nb) {
    int rc = check_tensor(c, t);
    if (rc) return rc;
    NO_CAPTURE(c);
    const int64_t nout = t->rows * t->n_mats;
    if (!X || !Y || nb < 1 || nb > FG_BATCH || ldx < t->cols || ldy < nout)
        return fail(c, FGH_ERR_ARG, "matmul: bad arguments");
    HIP_TRY(c, hipSetDevice(c->device));
    if ((rc = grow(c, c->x, (size_t)nb * t->cols * 4)) || (rc = grow(c, c->y, (size_t)nb * nout * 4))) return rc;
    HIP_TRY(c, hipMemcpy2DAsync(c->x.p, (size_t)t->cols * 4, X, (size_t)ldx * 4, (size_t)t->cols * 4, nb,
                                hipMemcpyHostToDevice, c->stream));
    if ((rc = fgh_matmul_dev(c, t, (const float *)c->x.p, (int)t->cols, (float *)c->y.p, (int)nout, nb))) return rc;
    HIP_TRY(c, hipMemcpy2DAsync(Y, (size_t)ldy * 4, c->y.p, (size_t)nout * 4, (size_t)nout * 4, nb,
                                hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    return FGH_OK;
}

int fgh_attention(fgh_ctx *c, int n_tok, int n_head, int n_head_kv, int hd, const float *q, float *o,
                  const float *k_cache, const float *v_cache, int kv_dim, int cap, const int32_t *st, const int32_t *en,
                  float scale) {
    if (!c) return FGH_ERR_ARG;
    NO_CAPTURE(c);
    if (!q || !o || !k_cache || !v_cache || !st || !en || n_tok < 1 || n_head < 1 || cap < 1 || kv_dim < 1)
        return fail(c, FGH_ERR_ARG, "attention: bad arguments");
    int max_len = 1;
    for (int t = 0; t < n_tok; t++) {
        const int n = en[t] - st[t] + 1;
        if (n < 1 || n > cap) return fail(c, FGH_ERR_ARG, "attention: token %d range %d..%d", t, st[t], en[t]);
        max_len = std::max(max_len, n);
    }
    HIP_TRY(c, hipSetDevice(c->device));
    const size_t nq = (size_t)n_tok * n_head * hd * 4, nc = (size_t)cap * kv_dim * 4, nr = (size_t)n_tok * 4;
    void *dq = nullptr, *dk = nullptr, *dv = nullptr, *dr = nullptr;
    int rc = FGH_OK;
    hipError_t e = hipMalloc(&dq, 2 * nq);
    if (e == hipSuccess) e = hipMalloc(&dk, nc);
    if (e == hipSuccess) e = hipMalloc(&dv, nc);
    if (e == hipSuccess) e = hipMalloc(&dr, 2 * nr);
    if (e == hipSuccess) e = hipMemcpyAsync(dq, q, nq, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(dk, k_cache, nc, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(dv, v_cache, nc, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(dr, st, nr, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync((char *)dr + nr, en, nr, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) {
        rc = fgh_attention_dev(c, n_tok, n_head, n_head_kv, hd, (const float *)dq, (float *)((char *)dq + nq),
                               (const float *)dk, (const float *)dv, kv_dim, cap, (const int32_t *)dr,
                               (const int32_t *)((char *)dr + nr), max_len, scale);
        if (rc == FGH_OK) e = hipMemcpyAsync(o, (char *)dq + nq, nq, hipMemcpyDeviceToHost, c->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    }
    (void)hipStreamSynchronize(c->stream);
    for (void *p : {dq, dk, dv, dr})
        if (p) (void)hipFree(p);
    if (rc) return rc;
    if (e != hipSuccess) return fail(c, FGH_ERR_DEVICE, "attention: %s", hipGetErrorString(e));
    return FGH_OK;
}

int fgh_moe_ffn(fgh_ctx *c, const fgh_tensor *gate, const fgh_tensor *up, const fgh_tensor *down, int k,
                const float *logits, const float *X, float *Y, int n_tok, int32_t *sel_out, float *w_out) {
    int rc = check_tensor(c, gate);
    if (rc) return rc;
    NO_CAPTURE(c);
    if (!logits || !X || !Y || n_tok < 1 || n_tok > FG_BATCH) return fail(c, FGH_ERR_ARG, "moe_ffn: bad arguments");
    const int64_t E = gate->n_mats, n_embd = gate->cols;
    HIP_TRY(c, hipSetDevice(c->device));
    if ((rc = grow(c, c->x, (size_t)n_tok * n_embd * 4)) || (rc = grow(c, c->y, (size_t)n_tok * n_embd * 4)) ||
        (rc = grow(c, c->mlog, (size_t)n_tok * E * 4)))
        return rc;
    HIP_TRY(c, hipMemcpyAsync(c->x.p, X, (size_t)n_tok * n_embd * 4, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(c, hipMemcpyAsync(c->mlog.p, logits, (size_t)n_tok * E * 4, hipMemcpyHostToDevice, c->stream));
    if ((rc = fgh_moe_ffn_dev(c, gate, up, down, k, (const float *)c->mlog.p, (const float *)c->x.p, (float *)c->y.p,
                              n_tok)))
        return rc;
    HIP_TRY(c, hipMemcpyAsync(Y, c->y.p, (size_t)n_tok * n_embd * 4, hipMemcpyDeviceToHost, c->stream));
    if (sel_out) HIP_TRY(c, hipMemcpyAsync(sel_out, c->msel.p, (size_t)n_tok * k * 4, hipMemcpyDeviceToHost, c->stream));
    if (w_out) HIP_TRY(c, hipMemcpyAsync(w_out, c->mw.p, (size_t)n_tok * k * 4, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    return FGH_OK;
}

// ---- memory, stream, events ----

int fgh_dev_alloc(fgh_ctx *c, uint64_t bytes, void **ptr) {
    if (!c || !ptr) return FGH_ERR_ARG;
    NO_CAPTURE(c);
    HIP_TRY(c, hipSetDevice(c->device));
    HIP_TRY(c, hipMalloc(ptr, bytes ? bytes : 1));
    return FGH_OK;
}
int fgh_dev_free(fgh_ctx *c, void *p) {
    if (!c) return FGH_ERR_ARG;
    NO_CAPTURE(c);
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    HIP_TRY(c, hipFree(p));
    return FGH_OK;
}
int fgh_copy_h2d(fgh_ctx *c, void *dst, const void *src, uint64_t bytes) {
    if (!c) return FGH_ERR_ARG;
    NO_CAPTURE(c);
    HIP_TRY(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    return FGH_OK;
}
int fgh_copy_d2h(fgh_ctx *c, void *dst, const void *src, uint64_t bytes) {
    if (!c) return FGH_ERR_ARG;
    NO_CAPTURE(c);
    HIP_TRY(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    return FGH_OK;
}
int fgh_copy_d2d(fgh_ctx *c, void *dst, const void *src, uint64_t bytes) {
    if (!c) return FGH_ERR_ARG;
    if (!dst || !src || bytes % 16 != 0) return fail(c, FGH_ERR_ARG, "copy_d2d: null pointer or bytes % 16 != 0");
    HIP_TRY(c, hipSetDevice(c->device));
    if (bytes) HIP_TRY(c, fgh::launch_copy16(src, dst, (int64_t)(bytes / 16), c->stream));
    return FGH_OK;
}
int fgh_checksum_dev(fgh_ctx *c, const void *src, uint64_t bytes, uint32_t *out) {
    if (!c) return FGH_ERR_ARG;
    if ((bytes && !src) || bytes % 16 != 0) return fail(c, FGH_ERR_ARG, "checksum_dev: null source or bytes % 16 != 0");
    HIP_TRY(c, hipSetDevice(c->device));
    const int np = fgh::checksum_parts(c->num_cu);
    int rc;
    if ((rc = grow(c, c->ck, (size_t)np * 4))) return rc;
    HIP_TRY(c, fgh::launch_checksum(src, (int64_t)(bytes / 16), (uint32_t *)c->ck.p, c->num_cu, out, c->stream));
    return FGH_OK;
}
int fgh_memcpy_dev(fgh_ctx *c, void *dst, const void *src, uint64_t bytes) {
    if (!c) return FGH_ERR_ARG;
    if (!dst || !src) return fail(c, FGH_ERR_ARG, "memcpy_dev: null pointer");
    HIP_TRY(c, hipSetDevice(c->device));
    if (bytes) HIP_TRY(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, c->stream));
    return FGH_OK;
}

int fgh_mfma_peak_dev(fgh_ctx *c, int iters, uint64_t *ops) {
    if (!c) return FGH_ERR_ARG;
    if (iters < 1 || iters > (1 << 20) || !ops) return fail(c, FGH_ERR_ARG, "mfma_peak_dev: iters 1..2^20 and ops");
    HIP_TRY(c, hipSetDevice(c->device));
    int rc;
    if ((rc = grow(c, c->ck, (size_t)fgh::mfma_peak_blocks(c->num_cu) * 4))) return rc;
    HIP_TRY(c, fgh::launch_mfma_peak(iters, (uint32_t *)c->ck.p, c->num_cu, c->stream));
    *ops = fgh::mfma_peak_ops(c->num_cu, iters);
    return FGH_OK;
}

int fgh_sync(fgh_ctx *c) {
    if (!c) return FGH_ERR_ARG;
    NO_CAPTURE(c);
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    return FGH_OK;
}
int fgh_event_create(fgh_ctx *c, void **ev) {
    if (!c || !ev) return FGH_ERR_ARG;
    HIP_TRY(c, hipEventCreate((hipEvent_t *)ev));
    return FGH_OK;
}
int fgh_event_record(fgh_ctx *c, void *ev) {
    if (!c || !ev) return FGH_ERR_ARG;
    HIP_TRY(c, hipEventRecord((hipEvent_t)ev, c->stream));
    return FGH_OK;
}
int fgh_event_elapsed_ms(fgh_ctx *c, void *a, void *b, float *ms) {
    if (!c || !a || !b || !ms) return FGH_ERR_ARG;
    NO_CAPTURE(c);
    HIP_TRY(c, hipEventSynchronize((hipEvent_t)b));
    HIP_TRY(c, hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b));
    return FGH_OK;
}
int fgh_event_destroy(fgh_ctx *c, void *ev) {
    if (!c || !ev) return FGH_ERR_ARG;
    HIP_TRY(c, hipEventDestroy((hipEvent_t)ev));
    return FGH_OK;
}

// ---- graphs ----

int fgh_graph_begin(fgh_ctx *c) {
    if (!c) return FGH_ERR_ARG;
    if (c->capturing) return fail(c, FGH_ERR, "graph_begin: already capturing");
    HIP_TRY(c, hipSetDevice(c->device));
    HIP_TRY(c, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
    c->capturing = true;
    return FGH_OK;
}

int fgh_graph_end(fgh_ctx *c, void **graph) {
    if (!c || !graph) return FGH_ERR_ARG;
    *graph = nullptr;
    if (!c->capturing) return fail(c, FGH_ERR, "graph_end: not capturing");
    c->capturing = false;
    hipGraph_t g = nullptr;
    HIP_TRY(c, hipStreamEndCapture(c->stream, &g));
    hipGraphExec_t ge = nullptr;
    hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return fail(c, FGH_ERR_DEVICE, "graph instantiate: %s", hipGetErrorString(e));
    *graph = ge;
    c->live_graphs++;
    return FGH_OK;
}

int fgh_graph_launch(fgh_ctx *c, void *graph) {
    if (!c || !graph) return FGH_ERR_ARG;
    if (c->capturing) return fail(c, FGH_ERR, "graph_launch: capturing");
    HIP_TRY(c, hipGraphLaunch((hipGraphExec_t)graph, c->stream));
    return FGH_OK;
}

int fgh_graph_destroy(fgh_ctx *c, void *graph) {
    if (!c || !graph) return FGH_ERR_ARG;
    NO_CAPTURE(c);
    HIP_TRY(c, hipSetDevice(c->device));
    HIP_TRY(c, hipStreamSynchronize(c->stream));  // no replay of it is still running
    HIP_TRY(c, hipGraphExecDestroy((hipGraphExec_t)graph));
    if (c->live_graphs > 0 && --c->live_graphs == 0) free_retired(c);
    return FGH_OK;
}

// ---- test hooks ----

int fgh_quantize(fgh_ctx *c, int kind, const float *x, int n, void *out_blocks) {
    if (!c || !x || !out_blocks || n <= 0) return FGH_ERR_ARG;
    NO_CAPTURE(c);
    const uint32_t type = kind == FGH_ACT_Q8 ? FGH_T_Q8_0 : kind == FGH_ACT_Q8K ? FGH_T_Q4_K : 0;
    if (!type) return fail(c, FGH_ERR_ARG, "quantize: bad kind");
    const int be = block_elems(type), nbk = n / be;
    if (nbk == 0) return FGH_OK;  // tails shorter than a block are ignored (n/32, n/256)
    int rc;
    HIP_TRY(c, hipSetDevice(c->device));
    if ((rc = grow(c, c->x, (size_t)nbk * be * 4))) return rc;
    HIP_TRY(c, hipMemcpyAsync(c->x.p, x, (size_t)nbk * be * 4, hipMemcpyHostToDevice, c->stream));
    if ((rc = quantize_dev(c, type, (int64_t)nbk * be, (const float *)c->x.p, (int64_t)nbk * be, 1))) return rc;
    const size_t qb = (size_t)nbk * (kind == FGH_ACT_Q8 ? 32 : 256), sb = (size_t)nbk * (kind == FGH_ACT_Q8 ? 2 : 16);
    std::string qs(qb, '\0'), bs(sb * 2, '\0');
    std::string d((size_t)nbk * 4, '\0');
    HIP_TRY(c, hipMemcpyAsync(&qs[0], c->aqs.p, qb, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(c, hipMemcpyAsync(&d[0], c->ad.p, (size_t)nbk * 4, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(c, hipMemcpyAsync(&bs[0], c->abs.p, sb * 2, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    uint8_t *o = (uint8_t *)out_blocks;
    for (int b = 0; b < nbk; b++) {
        if (kind == FGH_ACT_Q8) {  // {f32 d; i8 qs[32]; i16 s16[2]}
            uint8_t *blk = o + (size_t)b * 40;
            memcpy(blk, &d[(size_t)b * 4], 4);
            memcpy(blk + 4, &qs[(size_t)b * 32], 32);
            memcpy(blk + 36, &bs[(size_t)b * 4], 4);
        } else {  // {f32 d; i8 qs[256]; i16 bsums[16]}, undoing the lane permutation
            uint8_t *blk = o + (size_t)b * 292;
            memcpy(blk, &d[(size_t)b * 4], 4);
            for (int e = 0; e < 256; e++) {
                const int cc = e >> 5, i = (e >> 2) & 7, k = e & 3;
                blk[4 + e] = (uint8_t)qs[(size_t)b * 256 + 32 * i + 4 * cc + k];
            }
            memcpy(blk + 260, &bs[(size_t)b * 32], 32);
        }
    }
    return FGH_OK;
}

int fgh_block_ints(fgh_ctx *c, const fgh_tensor *t, const float *x, int32_t *sumi, int32_t *msum) {
    int rc = check_tensor(c, t);
    if (rc) return rc;
    NO_CAPTURE(c);
    if (!x || !sumi || !msum) return fail(c, FGH_ERR_ARG, "block_ints: null pointer");
    if (fgh::fl_kind((int)t->type)) return fail(c, FGH_ERR_ARG, "block_ints: a float tensor has no integer parts");
    const int64_t nout = t->rows * t->n_mats;
    // per (row, block); Q2_K / Q3_K / IQ4_XS: per (row, 32-value block), the units of their chains
    const size_t nint = (size_t)nout * t->nb * (fgh::kq_kind((int)t->type) ? 8 : 1);
    HIP_TRY(c, hipSetDevice(c->device));
    void *ds = nullptr;
    if ((rc = grow(c, c->x, (size_t)t->cols * 4)) || (rc = grow(c, c->y, (size_t)nout * 4))) return rc;
    HIP_TRY(c, hipMalloc(&ds, nint * 8));
    int32_t *dsi = (int32_t *)ds, *dmi = dsi + nint;
    hipError_t e = hipMemcpyAsync(c->x.p, x, (size_t)t->cols * 4, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) {
        float *ys[1] = {(float *)c->y.p};
        rc = matvec_launch(c, 1, &t, (const float *)c->x.p, t->cols, ys, 0, 1, dsi, dmi);
        if (!rc) {
            e = hipMemcpyAsync(sumi, dsi, nint * 4, hipMemcpyDeviceToHost, c->stream);
            if (e == hipSuccess) e = hipMemcpyAsync(msum, dmi, nint * 4, hipMemcpyDeviceToHost, c->stream);
            if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
        }
    }
    (void)hipStreamSynchronize(c->stream);
    (void)hipFree(ds);
    if (rc) return rc;
    if (e != hipSuccess) return fail(c, FGH_ERR_DEVICE, "block_ints: %s", hipGetErrorString(e));
    return FGH_OK;
}

int fgh_moe_block_ints(fgh_ctx *c, const fgh_tensor *gate, const fgh_tensor *up, const fgh_tensor *down, int k,
                       const float *logits, const float *X, int n_tok, int32_t *gate_sumi, int32_t *gate_msum,
                       int32_t *down_sumi, int32_t *down_msum) {
    int rc;
    if ((rc = check_tensor(c, gate)) || (rc = check_tensor(c, up)) || (rc = check_tensor(c, down))) return rc;
    NO_CAPTURE(c);
    if (!logits || !X || !gate_sumi || !gate_msum || !down_sumi || !down_msum || n_tok < 2 || n_tok > FG_BATCH ||
        k < 1 || k > gate->n_mats)
        return fail(c, FGH_ERR_ARG, "moe_block_ints: bad arguments");
    if (c->moe_valu || gate->type != FGH_T_Q4_K || up->type != FGH_T_Q4_K || down->type != FGH_T_Q4_K ||
        gate->order != FGH_ORDER_ROW || up->order != FGH_ORDER_ROW || down->order != FGH_ORDER_ROW)
        return fail(c, FGH_ERR_ARG, "moe_block_ints: the grouped MFMA path takes Q4_K row-order experts");
    const int64_t np = (int64_t)n_tok * k;
    const size_t ng = (size_t)np * gate->rows * gate->nb, nd = (size_t)np * down->rows * down->nb;
    HIP_TRY(c, hipSetDevice(c->device));
    void *buf = nullptr;
    HIP_TRY(c, hipMalloc(&buf, (ng + nd) * 8));
    int32_t *d0 = (int32_t *)buf;
    c->moe_dump[0] = d0;
    c->moe_dump[1] = d0 + ng;
    c->moe_dump[2] = d0 + 2 * ng;
    c->moe_dump[3] = d0 + 2 * ng + nd;
    std::vector<float> Y((size_t)n_tok * down->rows);
    rc = fgh_moe_ffn(c, gate, up, down, k, logits, X, Y.data(), n_tok, nullptr, nullptr);
    hipError_t e = hipSuccess;
    if (!rc) {
        int32_t *outs[4] = {gate_sumi, gate_msum, down_sumi, down_msum};
        const size_t cnts[4] = {ng, ng, nd, nd};
        for (int i = 0; i < 4 && e == hipSuccess; ++i)
            e = hipMemcpyAsync(outs[i], c->moe_dump[i], cnts[i] * 4, hipMemcpyDeviceToHost, c->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    }
    (void)hipStreamSynchronize(c->stream);
    for (auto &p : c->moe_dump) p = nullptr;
    (void)hipFree(buf);
    if (rc) return rc;
    if (e != hipSuccess) return fail(c, FGH_ERR_DEVICE, "moe_block_ints: %s", hipGetErrorString(e));
    return FGH_OK;
}

int fgh_gemm_block_ints(fgh_ctx *c, const fgh_tensor *t, const float *X, int ldx, int nb, int32_t *sumi,
                        int32_t *msum) {
    int rc = check_tensor(c, t);
    if (rc) return rc;
    NO_CAPTURE(c);
    if (!X || !sumi || !msum || nb < 1 || nb > FG_BATCH || ldx < t->cols)
        return fail(c, FGH_ERR_ARG, "gemm_block_ints: bad arguments");
    if (!prompt_gemm_bytes(c, t, 8))
        return fail(c, FGH_ERR_ARG, "gemm_block_ints: the MFMA GEMMs take Q4_K, Q6_K, Q8_0, Q4_0, Q4_1, Q5_0 and Q5_1 tensors");
    if (nb < 8) return fail(c, FGH_ERR_ARG, "gemm_block_ints: the prompt GEMM runs 8..64 tokens");
    const int64_t nout = t->rows * t->n_mats;
    const size_t nint = (size_t)nb * nout * t->nb;
    HIP_TRY(c, hipSetDevice(c->device));
    if ((rc = grow(c, c->x, (size_t)nb * t->cols * 4)) || (rc = grow(c, c->y, (size_t)nb * nout * 4))) return rc;
    void *ds = nullptr;
    HIP_TRY(c, hipMalloc(&ds, nint * 8));
    int32_t *dsi = (int32_t *)ds, *dmi = dsi + nint;
    hipError_t e = hipMemcpy2DAsync(c->x.p, (size_t)t->cols * 4, X, (size_t)ldx * 4, (size_t)t->cols * 4, nb,
                                    hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) {
        // the 32-value types have no min integer: their msum are zeros, as the oracle's
        if (t->type == FGH_T_Q8_0 || q32n_type(t->type)) e = hipMemsetAsync(dmi, 0, nint * 4, c->stream);
        if (e == hipSuccess) rc = prompt_gemm(c, t, (const float *)c->x.p, t->cols, (float *)c->y.p, nout, nb, dsi, dmi);
        if (!rc) {
            e = hipMemcpyAsync(sumi, dsi, nint * 4, hipMemcpyDeviceToHost, c->stream);
            if (e == hipSuccess) e = hipMemcpyAsync(msum, dmi, nint * 4, hipMemcpyDeviceToHost, c->stream);
            if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
        }
    }
    (void)hipStreamSynchronize(c->stream);
    (void)hipFree(ds);
    if (rc) return rc;
    if (e != hipSuccess) return fail(c, FGH_ERR_DEVICE, "gemm_block_ints: %s", hipGetErrorString(e));
    return FGH_OK;
}

int fgh_matvec_shape(fgh_ctx *c, uint32_t type, int order, int64_t cols, int64_t row_tiles, int ntok,
                     int32_t *shape) {
    if (!c || !shape || row_tiles < 1 || ntok < 1 || cols < 1 || !type_supported(type) ||
        cols % block_elems(type) != 0)
        return fail(c, FGH_ERR_ARG, "matvec_shape: bad arguments");
    const int ord = (type == FGH_T_Q4_K || type == FGH_T_Q4_0) && order == FGH_ORDER_REPACKED ? 1 : 0;
    const fgh::MvShape sh = fgh::matvec_shape((int)type, ord, row_tiles * ntok, (int)(cols / block_elems(type)),
                                              c->num_cu);
    shape[0] = sh.S;
    shape[1] = sh.R;
    shape[2] = sh.TPW;
    shape[3] = (int32_t)sh.lds;
    return FGH_OK;
}

int fgh_expf(fgh_ctx *c, const float *x, int n, float *out) {
    if (!c || !x || !out || n <= 0) return FGH_ERR_ARG;
    NO_CAPTURE(c);
    HIP_TRY(c, hipSetDevice(c->device));
    int rc;
    if ((rc = grow(c, c->x, (size_t)n * 4)) || (rc = grow(c, c->y, (size_t)n * 4))) return rc;
    HIP_TRY(c, hipMemcpyAsync(c->x.p, x, (size_t)n * 4, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(c, fgh::launch_expf((const float *)c->x.p, (float *)c->y.p, n, c->stream));
    HIP_TRY(c, hipMemcpyAsync(out, c->y.p, (size_t)n * 4, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    return FGH_OK;
}

int fgh_fp16_to_f32(fgh_ctx *c, const uint16_t *h, int n, float *out) {
    if (!c || !h || !out || n <= 0) return FGH_ERR_ARG;
    NO_CAPTURE(c);
    HIP_TRY(c, hipSetDevice(c->device));
    int rc;
    if ((rc = grow(c, c->x, (size_t)n * 2)) || (rc = grow(c, c->y, (size_t)n * 4))) return rc;
    HIP_TRY(c, hipMemcpyAsync(c->x.p, h, (size_t)n * 2, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(c, fgh::launch_fp16((const uint16_t *)c->x.p, (float *)c->y.p, n, c->stream));
    HIP_TRY(c, hipMemcpyAsync(out, c->y.p, (size_t)n * 4, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    return FGH_OK;
}

}  // extern "C"

// ---- self-check at open (the role of gpu_selfcheck, fastgguf.c:1898-1965) ----
// Every weight type goes through upload and matvec (Q4_K in both orders, and the prompt GEMM)
// on cases whose results are exact integers in fp32 whatever the order of the sums: x = 127
// everywhere (quantized to d = 1, q = 127 exactly), unit fp16 scales, and row r of a 16 x 512
// tensor holding one code c = 1 + r % 15 (Q2_K: 1 + r % 3) in every element. Then
// y_r = 65024 (v - m): v the element value (Q8_0, Q5_0, Q4_1, Q6_K, Q4_K, Q2_K, F16: c; Q5_K:
// c + 16) and m the min term (1 for Q4_K and Q5_K, whose mins are 1). Rows differ, so a row or
// tile mix-up shows as well as a dead kernel. One type per kernel family: the 8-row-tile kernel
// (Q8_0, Q5_0, Q4_1's min chain, Q6_K), the Q4_K / Q5_K kernel in both orders and the prompt
// GEMM, the low-bit kernel (Q2_K) and the float kernel (F16).
static void selfcheck_block(uint32_t type, int c, uint8_t *p) {
    const uint8_t nib2 = (uint8_t)(c | c << 4);
    const uint16_t one = 0x3C00;  // fp16 1.0
    switch (type) {
    case FGH_T_Q8_0:
        memcpy(p, &one, 2);
        memset(p + 2, c, 32);
        break;
    case FGH_T_Q5_0:  // nibble c with the fifth bit set: q5 - 16 = c
        memcpy(p, &one, 2);
        memset(p + 2, 0xFF, 4);
        memset(p + 6, nib2, 16);
        break;
    case FGH_T_Q6_K:  // q = c + 32 (low nibble c, high bits 2): q - 32 = c
        memset(p, nib2, 128);
        memset(p + 128, 0xAA, 64);
        memset(p + 192, 1, 16);
        memcpy(p + 208, &one, 2);
        break;
    case FGH_T_Q4_1:  // d = 1, m = 0, nibble c
        memcpy(p, &one, 2);
        memset(p + 2, 0, 2);
        memset(p + 4, nib2, 16);
        break;
    case FGH_T_Q2_K: {  // 16 scale bytes: scale 1, min 0; every 2-bit value c (c <= 3); d = 1, dmin = 0
        memset(p, 1, 16);
        memset(p + 16, c * 0x55, 64);
        memcpy(p + 80, &one, 2);
        memset(p + 82, 0, 2);
        break;
    }
    case FGH_T_F16: {  // one value: c
        const uint16_t h = (uint16_t)(0x3C00 + ((31 - __builtin_clz((unsigned)c)) << 10) +
                                      ((c << (10 - (31 - __builtin_clz((unsigned)c)))) & 0x3FF));
        memcpy(p, &h, 2);
        break;
    }
    default: {  // Q4_K / Q5_K: d = dmin = 1, the 8 scales and 8 mins all 1
        memcpy(p, &one, 2);
        memcpy(p + 2, &one, 2);
        memset(p + 4, 1, 8);
        memset(p + 12, 0x11, 4);
        if (type == FGH_T_Q5_K) {
            memset(p + 16, 0xFF, 32);
            memset(p + 48, nib2, 128);
        } else {
            memset(p + 16, nib2, 128);
        }
    }
    }
}

static int selfcheck(fgh_ctx *c) {
    const int cols = 512, rows = 16, ntok = 8;
    const struct { uint32_t type; int order, be, bb, v16, m, mod; } cases[] = {
        {FGH_T_Q8_0, FGH_ORDER_ROW, 32, 34, 0, 0, 15},    {FGH_T_Q5_0, FGH_ORDER_ROW, 32, 22, 0, 0, 15},
        {FGH_T_Q4_K, FGH_ORDER_ROW, 256, 144, 0, 1, 15},  {FGH_T_Q4_K, FGH_ORDER_REPACKED, 256, 144, 0, 1, 15},
        {FGH_T_Q5_K, FGH_ORDER_ROW, 256, 176, 16, 1, 15}, {FGH_T_Q6_K, FGH_ORDER_ROW, 256, 210, 0, 0, 15},
        {FGH_T_Q4_1, FGH_ORDER_ROW, 32, 20, 0, 0, 15},    {FGH_T_Q2_K, FGH_ORDER_ROW, 256, 84, 0, 0, 3},
        {FGH_T_F16, FGH_ORDER_ROW, 1, 2, 0, 0, 15},
    };
    std::vector<float> x((size_t)ntok * cols, 127.0f), y((size_t)ntok * rows);
    int rc = FGH_OK;
    for (const auto &k : cases) {
        const int nb = cols / k.be;
        std::vector<uint8_t> w((size_t)rows * nb * k.bb);
        for (int r = 0; r < rows; r++)
            for (int b = 0; b < nb; b++) selfcheck_block(k.type, 1 + r % k.mod, w.data() + ((size_t)r * nb + b) * k.bb);
        fgh_tensor *t = nullptr;
        if ((rc = fgh_upload(c, k.type, cols, rows, 1, k.order, w.data(), w.size(), &t)) != FGH_OK) break;
        // one token through matvec; for Q4_K also 8 tokens through matmul (the prompt GEMM)
        const int nt = k.type == FGH_T_Q4_K ? ntok : 1;
        rc = nt == 1 ? fgh_matvec(c, t, x.data(), y.data()) : fgh_matmul(c, t, x.data(), cols, y.data(), rows, nt);
        fgh_tensor_free(t);
        if (rc != FGH_OK) break;
        for (int i = 0; i < nt * rows && rc == FGH_OK; i++) {
            const float want = 65024.0f * (float)(1 + (i % rows) % k.mod + k.v16 - k.m);
            if (y[(size_t)i] != want) {
                fprintf(stderr, "[fastgguf_hip] self-check type %u order %d row %d: %g, want %g\n", k.type, k.order,
                        i % rows, (double)y[(size_t)i], (double)want);
                rc = FGH_ERR_DEVICE;
            }
        }
        if (rc != FGH_OK) break;
    }
    c->n_offloaded = c->n_skip_type = c->n_skip_mem = 0;
    return rc;
}
