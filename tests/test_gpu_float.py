"""GPU parity of the F32 / F16 / BF16 decode kernel (fastgguf_amd/csrc/fgh_float.hip) through the C
ABI: matvec, matvec_multi, per-token matmul and the generic MoE path, against the reference's
golden vectors and the oracle.

Bar: bit-exact. The kernel runs the fp32 operations of dot_f32v / dot_f16_row / the BF16 loop
(fastgguf.c:1618-1656, 2209-2213) in their order, so the outputs are compared bit for bit (the
1e-5 per-vector tolerance of the north star is checked too).
"""
import numpy as np
import pytest
from conftest import bits_equal, golden, rel_err

from fastgguf_amd import synth as S

pytestmark = pytest.mark.gpu

FLOAT = {"f32": S.T_F32, "f16": S.T_F16, "bf16": S.T_BF16}
TILE_ROWS = {S.T_F32: 4, S.T_F16: 8, S.T_BF16: 64}
TOL = 1e-5


def check_vec(y, ref):
    assert rel_err(y, ref) <= TOL
    assert bits_equal(y, ref), f"not bit-exact: rel {rel_err(y, ref):.3e}"


@pytest.mark.parametrize("name", list(FLOAT))
@pytest.mark.parametrize("gen", ["synth", "bytes"])
@pytest.mark.parametrize("cols", [3, 8, 100, 776, 1024])
def test_matvec_matches_golden(backend, name, gen, cols):
    g = golden("float.npz")
    w, x = g[f"{name}_{gen}_{cols}_w"], g[f"{name}_{gen}_{cols}_x"]
    print(f"golden matvec {name} {gen} {cols}", flush=True)
    t = backend.upload(FLOAT[name], cols, w)
    check_vec(backend.matvec(t, x), g[f"{name}_{gen}_{cols}_y"])
    t.free()


# widths: one value, every tail length of the 16- and 8-value steps around a step of 64, the
# largest (40960: x fills 160 KiB of LDS); rows: partly filled last tiles, and F32 launches with
# 4 tiles per workgroup (512 to 2048 tiles) and 2 (fewer or more)
SHAPES = [(1, 1), (5, 3), (9, 15), (33, 24), (70, 63), (64, 65), (130, 127), (300, 776), (1000, 4096), (2048, 1000),
          (4096, 512), (8200, 256), (7, 40960), (50, 14336)]


@pytest.mark.parametrize("t", list(FLOAT.values()))
@pytest.mark.parametrize("rows,cols", SHAPES)
def test_matvec_matches_oracle(backend, oracle, t, rows, cols):
    gen = S.random_bytes_weights if (rows + cols) % 2 else S.weights
    w = gen(t, rows, cols, rows + 3 * cols + t)
    x = S.activations(cols, cols + t) * np.float32(2.5)
    tiles = (rows + TILE_ROWS[t] - 1) // TILE_ROWS[t]
    print(f"matvec {S.TYPE_NAME[t]} {rows}x{cols} shape {backend.matvec_shape(t, 0, cols, tiles)}", flush=True)
    tt = backend.upload(t, cols, w)
    check_vec(backend.matvec(tt, x), oracle.matvec(t, w, cols, x))
    tt.free()


def test_launch_forms_are_all_taken(backend):
    """Every instantiation: ring depth 16; F32 with 2 and 4 tiles per workgroup (both reached by
    the shapes above), F16 with 4, BF16 with 2."""
    want = {S.T_F32: {2, 4}, S.T_F16: {4}, S.T_BF16: {2}}
    for t in FLOAT.values():
        shapes = {backend.matvec_shape(t, 0, c, (r + TILE_ROWS[t] - 1) // TILE_ROWS[t])[1:3] for r, c in SHAPES}
        assert shapes == {(16, p) for p in want[t]}, (S.TYPE_NAME[t], shapes)


def test_bf16_many_tiles(backend, oracle):
    """BF16 at 1024 tiles of 64 rows."""
    rows, cols = 65536, 64
    w = S.random_bytes_weights(S.T_BF16, rows, cols, 91)
    x = S.activations(cols, 92)
    tt = backend.upload(S.T_BF16, cols, w)
    check_vec(backend.matvec(tt, x), oracle.matvec(S.T_BF16, w, cols, x))
    tt.free()


def test_matvec_multi_groups_by_type(backend, oracle):
    """F16, F32, F16, Q4_K over one x: the two F16 matrices share a launch."""
    cols = 1024
    types, rows = [S.T_F16, S.T_F32, S.T_F16, S.T_Q4_K], [1000, 300, 24, 512]
    ws = [S.weights(t, r, cols, 90 + i) for i, (t, r) in enumerate(zip(types, rows))]
    x = S.activations(cols, 99)
    ts = [backend.upload(t, cols, w) for t, w in zip(types, ws)]
    for y, t, w in zip(backend.matvec_multi(ts, x), types, ws):
        order = 1 if t == S.T_Q4_K else 0  # a 2-D Q4_K with rows % 8 == 0 is repacked
        check_vec(y, oracle.matvec(t, w, cols, x, order))
    for t in ts:
        t.free()


@pytest.mark.parametrize("name", list(FLOAT))
@pytest.mark.parametrize("nb", [3, 9])
def test_matmul_matches_golden(backend, name, nb):
    g = golden("float.npz")
    w, X = g[f"{name}_mm_w"], g[f"{name}_mm_X{nb}"]
    t = backend.upload(FLOAT[name], X.shape[1], w)
    Y = backend.matmul(t, X)
    for b in range(nb):
        check_vec(Y[b], g[f"{name}_mm_Y{nb}"][b])
    t.free()


@pytest.mark.parametrize("t", list(FLOAT.values()))
@pytest.mark.parametrize("nb", [2, 16, 64])
def test_matmul_per_token_matches_oracle(backend, oracle, t, nb):
    rows, cols = 520, 1000
    w = S.random_bytes_weights(t, rows, cols, 60 + nb)
    X = S.activations(cols, 61 + nb, rows=nb)
    tt = backend.upload(t, cols, w)
    Y = backend.matmul(tt, X)
    Yo = oracle.matmul(t, w, cols, X)
    for b in range(nb):
        check_vec(Y[b], Yo[b])
    tt.free()


@pytest.mark.parametrize("types", [(S.T_F16, S.T_F16, S.T_BF16), (S.T_F32, S.T_BF16, S.T_F16),
                                   (S.T_BF16, S.T_BF16, S.T_Q4_K)])
def test_moe_matches_oracle(backend, oracle, types):
    """The generic expert path with float experts: routing, gate / up with an expert index per
    token slot, silu, down and the ordered weighted sum; one token and several per call."""
    E, K, D, F, T = 8, 2, 256, 200 if types[2] != S.T_Q4_K else 256, 5
    gw = S.weights(types[0], E * F, D, 340)
    uw = S.weights(types[1], E * F, D, 341)
    dw = S.weights(types[2], E * D, F, 342)
    X = S.activations(D, 343, rows=T)
    logits = S.router_logits(T, E, 344)
    gate = backend.upload(types[0], D, gw, rows=F, n_mats=E)
    up = backend.upload(types[1], D, uw, rows=F, n_mats=E)
    down = backend.upload(types[2], F, dw, rows=D, n_mats=E)
    for n in (1, T):
        Yo, so, wo = oracle.moe_ffn(types, gw, uw, dw, E, K, D, F, logits[:n], X[:n])
        Y, sel, w = backend.moe_ffn(gate, up, down, K, logits[:n], X[:n])
        assert np.array_equal(sel, so)
        assert bits_equal(w, wo)
        assert bits_equal(Y, Yo)
    for t in (gate, up, down):
        t.free()


def test_block_ints_refused(backend):
    from fastgguf_amd.backend import BackendError
    tt = backend.upload(S.T_F16, 64, S.weights(S.T_F16, 8, 64, 1))
    with pytest.raises(BackendError):
        backend.block_ints(tt, S.activations(64, 2))
    tt.free()


def test_graph_replays_match_eager(backend, oracle):
    """Two captured matvecs (F32, BF16) replay to the eager results, with eager calls and host
    synchronizations between the replays and the outputs overwritten before each."""
    cols = 1000
    cases = [(S.T_F32, 2048), (S.T_BF16, 300)]
    ws = [S.random_bytes_weights(t, r, cols, 70 + i) for i, (t, r) in enumerate(cases)]
    x = S.activations(cols, 71)
    ts = [backend.upload(t, cols, w) for (t, _), w in zip(cases, ws)]
    want = [oracle.matvec(t, w, cols, x) for (t, _), w in zip(cases, ws)]
    xd = backend.dev_alloc(4 * cols)
    yds = [backend.dev_alloc(4 * r) for _, r in cases]
    backend.h2d(xd, x)
    for tt, yd in zip(ts, yds):  # eager first
        backend.matvec_dev(tt, xd, yd)
    backend.sync()
    backend.graph_begin()
    for tt, yd in zip(ts, yds):
        backend.matvec_dev(tt, xd, yd)
    g = backend.graph_end()
    try:
        for rep in range(4):
            for (_, r), yd in zip(cases, yds):
                backend.h2d(yd, np.full(r, np.nan, np.float32))
            backend.graph_launch(g)
            backend.sync()
            for (_, r), yd, yw in zip(cases, yds, want):
                y = np.empty(r, np.float32)
                backend.d2h(y, yd)
                assert bits_equal(y, yw), f"replay {rep}"
            check_vec(backend.matvec(ts[0], x), want[0])  # eager work between replays
    finally:
        backend.graph_destroy(g)
    for p in [xd] + yds:
        backend.dev_free(p)
    for tt in ts:
        tt.free()
