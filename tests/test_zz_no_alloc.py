"""fgh_matmul_dev_noalloc: the prompt matmul with its GEMM scratch in the library's static
per-device array instead of context buffers. Through the C ABI, its outputs equal fgh_matmul_dev's
bit for bit (the same kernels on the same inputs), over two calls in a row with the second one
smaller, on a fresh context as well as on one that has already run other work; a call whose
scratch would exceed FGH_NOALLOC_SCRATCH_BYTES fails with FGH_ERR_ARG before launching anything."""
import numpy as np
import pytest
from conftest import bits_equal

from fastgguf_amd import synth as S
from fastgguf_amd.backend import Backend, BackendError

pytestmark = pytest.mark.gpu

FGH_ERR_ARG = -2
SCRATCH_BYTES = 8 << 20  # FGH_NOALLOC_SCRATCH_BYTES


def run_both(be, t, X):
    """(noalloc output, matmul_dev output) for the tokens X on tensor t, both on the device"""
    T = X.shape[0]
    xd = be.dev_alloc(X.nbytes)
    ya, yb = be.dev_alloc(4 * T * t.nout), be.dev_alloc(4 * T * t.nout)
    be.h2d(xd, X)
    poison = np.full(T * t.nout, np.nan, np.float32)
    be.h2d(ya, poison)
    be.h2d(yb, poison)
    be.matmul_dev_noalloc(t, xd, ya, T)
    be.matmul_dev(t, xd, yb, T)
    be.sync()
    got, want = np.empty((T, t.nout), np.float32), np.empty((T, t.nout), np.float32)
    be.d2h(got, ya)
    be.d2h(want, yb)
    for p in (xd, ya, yb):
        be.dev_free(p)
    return got, want


# (type, rows, cols, tokens): the first two take the prompt GEMM (Q4_K, >= 8 tokens), the larger
# one first, so the second call reuses the array with a smaller input; the third runs the decode
# kernels, which need no scratch; then the Q6_K GEMM with a 4-way K split (4096 output rows: 64
# row groups) and without, the Q8_0 GEMM with a K split and without (smaller), and the nibble-type
# GEMM (Q5_1, then Q4_0 smaller); last an F16 tensor, whose per-token decode kernel needs no scratch
CALLS = [(S.T_Q4_K, 1024, 8192, 64), (S.T_Q4_K, 272, 2048, 9), (S.T_Q4_K, 128, 2048, 5),
         (S.T_Q6_K, 4096, 14336, 64), (S.T_Q6_K, 96, 1024, 12),
         (S.T_Q8_0, 4096, 14336, 64), (S.T_Q8_0, 512, 2048, 16),
         (S.T_Q5_1, 200, 4096, 40), (S.T_Q4_0, 64, 1024, 8), (S.T_F16, 300, 1000, 24)]


@pytest.mark.parametrize("fresh", [True, False], ids=["fresh_context", "shared_context"])
def test_noalloc_matches_matmul_dev(backend, fresh):
    be = Backend(0) if fresh else backend
    try:
        for i, (ty, rows, cols, T) in enumerate(CALLS):
            w = S.weights(ty, rows, cols, 700 + i)
            X = S.activations(cols, 710 + i, rows=T)
            t = be.upload(ty, cols, w)
            got, want = run_both(be, t, X)
            assert not np.isnan(want).any()
            assert bits_equal(got, want), f"call {i}: {S.TYPE_NAME[ty]} {rows}x{cols}, {T} tokens"
            t.free()
    finally:
        if fresh:
            be.close()


def _up(n, m=256):
    return -(-n // m) * m


def gemm_scratch(type_, rows, cols, T, num_cu=256):
    """bytes of a prompt GEMM's scratch (Q4_K, Q6_K, Q8_0): the activation records, and with a K
    split (few 64-row groups) the arrival counters and ks partials of 64 rows x Tp tokens of fp32
    per workgroup"""
    wg = -(-rows // 64)
    if type_ == S.T_Q8_0:
        Tp = 32 if T <= 32 else 64
        steps = -(-(cols // 32) // 4)
        rec = (steps + (4 if steps >= 4 else 2 if steps >= 2 else 1)) * 144 * Tp
        units, min_units = steps, 8
    else:  # Q4_K, Q6_K: one 292-byte Q8_K record per 256-block and token, one of slack
        Tp = -(-T // 16) * 16
        rec = (cols // 256 + 1) * 292 * Tp
        units, min_units = cols // 256, 4
    ks = 1
    while ks < 4 and wg * (ks + 1) <= num_cu and units // (ks + 1) >= min_units:
        ks += 1
    return rec if ks == 1 else _up(rec) + _up(4 * wg) + ks * wg * 64 * Tp * 4


@pytest.mark.parametrize("type_,largest", [(S.T_Q4_K, 223), (S.T_Q6_K, 223), (S.T_Q8_0, 1804)],
                         ids=["Q4_K", "Q6_K", "Q8_0"])
def test_noalloc_refuses_more_than_its_scratch(backend, type_, largest):
    """4096 rows at 64 tokens (the down projection's output width, a 4-way K split): the largest K
    whose records fit beside the split's counters and 4 MiB of partials within 8 MiB runs; one
    block more is refused, nothing launched, and the context still works"""
    rows = 4096
    blk = 32 if type_ == S.T_Q8_0 else 256
    for nbk, ok in ((largest, True), (largest + 1, False)):
        cols = blk * nbk
        assert (gemm_scratch(type_, rows, cols, 64) <= SCRATCH_BYTES) == ok
        print(f"noalloc {S.TYPE_NAME[type_]} {rows}x{cols} 64 tokens ({'fits' if ok else 'refused'})", flush=True)
        t = backend.upload(type_, cols, S.weights(type_, rows, cols, 720 + nbk))
        X = S.activations(cols, 730, rows=64)
        if ok:
            got, want = run_both(backend, t, X)
            assert bits_equal(got, want)
        else:
            xd, yd = backend.dev_alloc(X.nbytes), backend.dev_alloc(4 * 64 * rows)
            with pytest.raises(BackendError) as e:
                backend.matmul_dev_noalloc(t, xd, yd, 64)
            assert e.value.status == FGH_ERR_ARG and "scratch" in str(e.value)
            backend.dev_free(xd)
            backend.dev_free(yd)
            # the context still works after the refusal
            got, want = run_both(backend, t, X[:8])
            assert bits_equal(got, want)
        t.free()
