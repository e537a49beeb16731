"""Pins the oracle's F32 / F16 / BF16 row kernels (fgo_dot_float; dot_row 2207-2214 of fastgguf.c:
dot_f32v 1618-1632, dot_f16_row 1645-1656, the BF16 loop 2209-2213).

* golden vectors of the reference's compiled kernels (tests/golden/float.npz, AVX-512-VNNI build):
  matvec at widths with and without each kernel's tail, on N(0, 0.02) rows and on random finite bit
  patterns (subnormals and zeros included), and matmul at 3 and 9 tokens, bit for bit;
* the compiled reference itself on fresh shapes and seeds, where oracle/_ref is built: both builds
  for F16 and BF16; for F32 the AVX2 build only at widths with n % 8 < 4 (see
  test_avx2_build_f32_tail_differs);
* the mathematics: exact integer dots (small integer values, every partial sum exact, so any
  order gives the integer: no value dropped, doubled or misdecoded); dequantize_row against numpy's
  own conversions; the dot against the float64 sum of the values' products.
"""
import numpy as np
import pytest
from conftest import bits_equal, golden

from fastgguf_amd import synth as S
from oracle import Reference

FLOAT = {"f32": S.T_F32, "f16": S.T_F16, "bf16": S.T_BF16}
WIDTHS = (3, 8, 100, 776, 1024)


def to_type(t, v):
    """fp32 values (exactly representable in the type) -> the type's bytes"""
    v = np.ascontiguousarray(v, np.float32)
    if t == S.T_F16:
        return v.astype(np.float16).view(np.uint8).reshape(v.shape[0], -1)
    if t == S.T_BF16:
        return (v.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).reshape(v.shape[0], -1)
    return v.view(np.uint8).reshape(v.shape[0], -1)


def values(t, w, cols):
    """the weights as fp32 by numpy's own conversions"""
    w = np.ascontiguousarray(w, np.uint8)
    if t == S.T_F32:
        return w.view(np.float32).reshape(-1, cols)
    if t == S.T_F16:
        return w.view(np.float16).astype(np.float32).reshape(-1, cols)
    return (w.view(np.uint16).astype(np.uint32) << 16).view(np.float32).reshape(-1, cols)


@pytest.mark.parametrize("name", list(FLOAT))
@pytest.mark.parametrize("gen", ["synth", "bytes"])
@pytest.mark.parametrize("cols", WIDTHS)
def test_matvec_matches_golden(oracle, name, gen, cols):
    g = golden("float.npz")
    w, x = g[f"{name}_{gen}_{cols}_w"], g[f"{name}_{gen}_{cols}_x"]
    assert bits_equal(oracle.matvec(FLOAT[name], w, cols, x), g[f"{name}_{gen}_{cols}_y"])


@pytest.mark.parametrize("name", list(FLOAT))
@pytest.mark.parametrize("nb", [3, 9])
def test_matmul_matches_golden(oracle, name, nb):
    g = golden("float.npz")
    w, X = g[f"{name}_mm_w"], g[f"{name}_mm_X{nb}"]
    assert bits_equal(oracle.matmul(FLOAT[name], w, X.shape[1], X), g[f"{name}_mm_Y{nb}"])


@pytest.mark.parametrize("variant", ["avx2", "vnni"])
def test_matches_compiled_reference_random(oracle, reference, variant):
    ref = reference if reference.variant == variant else Reference(variant)
    rng = np.random.Generator(np.random.PCG64(17))
    for case in range(18):
        t = list(FLOAT.values())[case % 3]
        cols = int(rng.integers(1, 600))
        if t == S.T_F32 and variant == "avx2" and cols % 8 >= 4:
            cols -= cols % 8  # the AVX2 build's own F32 tail: test_avx2_build_f32_tail_differs
        cols = max(cols, 1)
        rows = int(rng.integers(1, 12))
        w = (S.weights if case % 2 else S.random_bytes_weights)(t, rows, cols, 1400 + case)
        x = S.activations(cols, 1500 + case) * float(rng.uniform(0.1, 10))
        assert bits_equal(oracle.matvec(t, w, cols, x), ref.matvec(t, w, cols, x)), (S.TYPE_NAME[t], cols)
        X = S.activations(cols, 1600 + case, rows=int(rng.integers(2, 12)))
        assert bits_equal(oracle.matmul(t, w, cols, X), ref.matmul(t, w, cols, X)), (S.TYPE_NAME[t], cols)


def test_avx2_build_f32_tail_differs(oracle, reference):
    """gcc's x86-64-v3 code for dot_f32v's scalar tail multiplies 4 values at once and adds the 4
    products in order (no fused multiply-add) when 4 or more values remain, where the AVX-512 build
    runs one fma per value as the source's contraction reads; the two builds then differ by
    rounding. The oracle (and the GPU) follow the AVX-512 build, the golden vectors' source. Rows
    of whole 8-value groups, the models' widths, agree in both builds."""
    try:
        avx2 = reference if reference.variant == "avx2" else Reference("avx2")
    except FileNotFoundError:
        pytest.skip("the AVX2 reference build is not built")
    w = S.random_bytes_weights(S.T_F32, 16, 15, 5)
    x = S.activations(15, 6) * np.float32(2.5)
    assert not bits_equal(avx2.matvec(S.T_F32, w, 15, x), oracle.matvec(S.T_F32, w, 15, x))
    w = S.random_bytes_weights(S.T_F32, 16, 96, 7)
    x = S.activations(96, 8)
    assert bits_equal(avx2.matvec(S.T_F32, w, 96, x), oracle.matvec(S.T_F32, w, 96, x))


@pytest.mark.parametrize("t", list(FLOAT.values()))
@pytest.mark.parametrize("cols", [1, 7, 15, 16, 17, 100, 1000])
def test_integer_dot_is_exact(oracle, t, cols):
    """Integer weights in [-8, 8] and activations in [-16, 16]: every product and partial sum is an
    integer far below 2^24, so whatever the order the result is the exact integer dot."""
    rng = np.random.Generator(np.random.PCG64(cols + t))
    wv = rng.integers(-8, 9, size=(6, cols)).astype(np.float32)
    xv = rng.integers(-16, 17, size=cols).astype(np.float32)
    want = (wv.astype(np.int64) @ xv.astype(np.int64)).astype(np.float32)
    assert bits_equal(oracle.matvec(t, to_type(t, wv), cols, xv), want)


@pytest.mark.parametrize("t", list(FLOAT.values()))
def test_dequantize_row_matches_numpy(oracle, t):
    cols = 333
    w = S.random_bytes_weights(t, 4, cols, 40 + t)
    want = values(t, w, cols)
    for r in range(4):
        assert bits_equal(oracle.dequantize_row(t, w[r], cols), want[r])


@pytest.mark.parametrize("t", list(FLOAT.values()))
def test_dot_vs_float64(oracle, t):
    cols = 2048
    for seed in range(3):
        w = S.weights(t, 8, cols, 60 + seed)
        x = S.activations(cols, 70 + seed)
        terms = values(t, w, cols).astype(np.float64) * x.astype(np.float64)
        y = oracle.matvec(t, w, cols, x).astype(np.float64)
        assert (np.abs(y - terms.sum(1)) <= 1e-5 * np.abs(terms).sum(1) + 1e-30).all()
