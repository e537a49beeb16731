"""GPU parity of the Q2_K / Q3_K / IQ4_XS decode kernel (fastgguf_amd/csrc/fgh_kq.hip) through the
C ABI: matvec, matvec_multi, per-token matmul and the generic MoE path, against the reference's
golden vectors and the oracle.

Bar: bit-exact. The integers of each 32-value block are exact, and the fp32 chain of each row
follows dot_q2_K_q8 / dot_q3_K_q8 / dot_iq4_xs_q8 (fastgguf.c:1426-1614) step for step, so the
outputs are compared bit for bit (the 1e-5 per-vector tolerance of the north star is checked too).
"""
import numpy as np
import pytest
from conftest import bits_equal, golden, rel_err

from fastgguf_amd import synth as S

pytestmark = pytest.mark.gpu

LOWBIT = {"q2_k": S.T_Q2_K, "q3_k": S.T_Q3_K, "iq4_xs": S.T_IQ4_XS}
TOL = 1e-5


def check_vec(y, ref):
    assert rel_err(y, ref) <= TOL
    assert bits_equal(y, ref), f"not bit-exact: rel {rel_err(y, ref):.3e}"


@pytest.mark.parametrize("name", list(LOWBIT))
@pytest.mark.parametrize("gen", ["synth", "bytes"])
def test_matvec_matches_golden(backend, name, gen):
    g = golden("lowbit.npz")
    w, x = g[f"{name}_{gen}_w"], g[f"{name}_{gen}_x"]
    print(f"golden matvec {name} {gen}", flush=True)
    t = backend.upload(LOWBIT[name], x.size, w)
    check_vec(backend.matvec(t, x), g[f"{name}_{gen}_y"])
    t.free()


# shapes that take every launch form: 8 wavefronts per tile (up to a few thousand rows of 16 blocks
# or more), 4 (8200 rows, or 8 blocks), 2 (20000 rows, or 4 blocks), 1 (rows of 1 block); ragged
# row counts (a partly filled last tile)
SHAPES = [(64, 16384), (13, 2048), (512, 4096), (200, 8192), (4096, 4096), (8200, 4096), (9, 256), (1000, 256),
          (2048, 14336), (100, 1024), (20000, 2048)]


@pytest.mark.parametrize("t", list(LOWBIT.values()))
@pytest.mark.parametrize("rows,cols", SHAPES)
def test_matvec_matches_oracle(backend, oracle, t, rows, cols):
    gen = S.random_bytes_weights if (rows + cols) % 2 else S.weights
    w = gen(t, rows, cols, rows + 7 * t)
    x = S.activations(cols, cols + t) * np.float32(2.5)
    print(f"matvec {S.TYPE_NAME[t]} {rows}x{cols} shape {backend.matvec_shape(t, 0, cols, (rows + 15) // 16)}",
          flush=True)
    tt = backend.upload(t, cols, w)
    check_vec(backend.matvec(tt, x), oracle.matvec(t, w, cols, x))
    tt.free()


@pytest.mark.parametrize("t", list(LOWBIT.values()))
def test_widest_row(backend, oracle, t):
    """204 blocks (K = 52224), the widest row the kernel accepts (its quantized x fills 64 KiB of
    LDS less 256 bytes); one block more is refused at upload (test_gpu_matvec)."""
    rows, cols = 40, 204 * 256
    w = S.random_bytes_weights(t, rows, cols, 80 + t)
    x = S.activations(cols, 81 + t)
    print(f"widest {S.TYPE_NAME[t]} {rows}x{cols}", flush=True)
    tt = backend.upload(t, cols, w)
    check_vec(backend.matvec(tt, x), oracle.matvec(t, w, cols, x))
    tt.free()


def test_launch_forms_are_all_taken(backend):
    """The shapes above cover 1, 2, 4 and 8 wavefronts per tile (ring depth 4 for whole rows, 2
    for split launches)."""
    seen = {backend.matvec_shape(S.T_Q2_K, 0, cols, (rows + 15) // 16)[:2] for rows, cols in SHAPES}
    assert seen == {(1, 4), (2, 2), (4, 2), (8, 2)}, seen


@pytest.mark.parametrize("t", list(LOWBIT.values()))
def test_block_ints_match_oracle(backend, oracle, t):
    rows, cols = 24, 1024
    w = S.random_bytes_weights(t, rows, cols, 50 + t)
    x = S.activations(cols, 51 + t)
    tt = backend.upload(t, cols, w)
    s, m = backend.block_ints(tt, x)
    act = oracle.quantize_q8(x)
    for r in range(rows):
        so, mo = oracle.block_ints(t, w[r], act)
        assert np.array_equal(s[r], so) and np.array_equal(m[r], mo), r
    tt.free()


def test_matvec_multi_groups_by_type(backend, oracle):
    """Q2_K, Q2_K, IQ4_XS, Q3_K over one x: the two Q2_K matrices share a launch."""
    cols = 4096
    types, rows = [S.T_Q2_K, S.T_Q2_K, S.T_IQ4_XS, S.T_Q3_K], [4096, 1024, 1024, 2048]
    ws = [S.weights(t, r, cols, 90 + i) for i, (t, r) in enumerate(zip(types, rows))]
    x = S.activations(cols, 99)
    ts = [backend.upload(t, cols, w) for t, w in zip(types, ws)]
    for y, t, w in zip(backend.matvec_multi(ts, x), types, ws):
        check_vec(y, oracle.matvec(t, w, cols, x))
    for t in ts:
        t.free()


@pytest.mark.parametrize("name", list(LOWBIT))
@pytest.mark.parametrize("nb", [3, 8, 45])
def test_matmul_matches_golden(backend, name, nb):
    g = golden("lowbit.npz")
    w, X = g[f"{name}_mm_w"], g[f"{name}_mm_X{nb}"]
    t = backend.upload(LOWBIT[name], X.shape[1], w)
    Y = backend.matmul(t, X)
    for b in range(nb):
        check_vec(Y[b], g[f"{name}_mm_Y{nb}"][b])
    t.free()


@pytest.mark.parametrize("t", list(LOWBIT.values()))
@pytest.mark.parametrize("nb", [2, 16, 64])
def test_matmul_per_token_matches_oracle(backend, oracle, t, nb):
    rows, cols = 1536, 4096
    w = S.random_bytes_weights(t, rows, cols, 60 + nb)
    X = S.activations(cols, 61 + nb, rows=nb)
    tt = backend.upload(t, cols, w)
    Y = backend.matmul(tt, X)
    Yo = oracle.matmul(t, w, cols, X)
    for b in range(nb):
        check_vec(Y[b], Yo[b])
    tt.free()


@pytest.mark.parametrize("types", [(S.T_Q2_K, S.T_Q2_K, S.T_Q3_K), (S.T_IQ4_XS, S.T_IQ4_XS, S.T_IQ4_XS),
                                   (S.T_Q3_K, S.T_Q3_K, S.T_Q4_K), (S.T_Q4_K, S.T_Q4_K, S.T_Q2_K)])
def test_moe_matches_oracle(backend, oracle, types):
    """The generic expert path: routing, gate / up with an expert index per token slot, silu, down
    and the ordered weighted sum; one token and several per call."""
    E, K, D, F, T = 16, 4, 512, 512, 6
    gw = S.random_bytes_weights(types[0], E * F, D, 330)
    uw = S.random_bytes_weights(types[1], E * F, D, 331)
    dw = S.random_bytes_weights(types[2], E * D, F, 332)
    X = S.activations(D, 333, rows=T)
    logits = S.router_logits(T, E, 334)
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


def test_graph_replays_match_eager(backend, oracle):
    """Two captured matvecs (Q3_K, IQ4_XS) replay to the eager results, with eager calls and host
    synchronizations between the replays and the outputs overwritten before each."""
    cols = 4096
    cases = [(S.T_Q3_K, 2048), (S.T_IQ4_XS, 512)]
    ws = [S.weights(t, r, cols, 70 + i) for i, (t, r) in enumerate(cases)]
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
