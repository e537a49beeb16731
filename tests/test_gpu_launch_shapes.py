"""Every decode-kernel instantiation the launchers can pick runs, bit-exact against the oracle.

The decode launchers choose a launch shape per call from the row tiles of the launch, the row
width and the device's compute units: S wavefronts per tile (a block split for short matrices),
a register ring of R steps, TPW tiles per workgroup. Each (type, order, S, R, TPW) is a separate kernel
instantiation, and so is its integer-dump form. fgh_matvec_shape reports the shape a call would
take (the same function the launchers call), so these tests

  1. scan row widths and tile counts to find every shape each weight type and order can take, and
  2. run, for each reachable shape, the smallest tensor that takes it: the matvec bit for bit
     against the oracle's restatement of the reference kernel (dot_q4Kx8 / dot_q4_K_q8k /
     dot_q6_K_q8k / dot_q8_0_q8 / ... orders), its per-block integers (the dump form) against the
     oracle's, and the silu entry (a short silu launch, then the same kernel) bit for bit
     against the same matvec of silu(g) * u.

The benchmark's dominant launch (gate and up 4096 -> 14336 in one matvec_multi, both orders) is
tested at its own size as well, and so is the paired gate / up form that writes h = silu(g) * u.
"""
import numpy as np
import pytest
from conftest import bits_equal

from fastgguf_amd import synth as S
from fastgguf_amd.backend import ORDER_REPACKED, ORDER_ROW
from oracle import ORDER_REPACKED as O_RP
from oracle import ORDER_ROW as O_ROW

pytestmark = pytest.mark.gpu

FAMILIES = [(S.T_Q4_K, ORDER_REPACKED), (S.T_Q4_K, ORDER_ROW), (S.T_Q5_K, ORDER_ROW), (S.T_Q6_K, ORDER_ROW),
            (S.T_Q8_0, ORDER_ROW), (S.T_Q5_0, ORDER_ROW), (S.T_Q4_0, ORDER_REPACKED), (S.T_Q4_0, ORDER_ROW),
            (S.T_Q4_1, ORDER_ROW), (S.T_Q5_1, ORDER_ROW), (S.T_IQ4_NL, ORDER_ROW), (S.T_Q2_K, ORDER_ROW),
            (S.T_Q3_K, ORDER_ROW), (S.T_IQ4_XS, ORDER_ROW)]
TILES = [1, 2, 3, 4, 6, 8, 12, 16, 24, 32, 48, 64, 96, 100, 128, 160, 192, 200, 256, 257, 300, 384, 448, 511, 512,
         513, 600, 700, 767, 768, 900, 1000, 1023, 1024, 1100, 1536, 1792, 2048]
NB_K = [1, 2, 3, 4, 7, 8, 12, 15, 16, 17, 24, 31, 32, 33, 40, 56, 64, 100, 128, 200, 237]
NB_32 = [1, 3, 4, 8, 12, 16, 28, 29, 32, 60, 64, 96, 124, 125, 128, 160, 200, 256, 448, 800, 1600, 1820]


def tile_rows(t):
    return 16 if t in (S.T_Q4_K, S.T_Q5_K) or t in S.K256Q8_TYPES else 8


def block_elems(t):
    return 256 if t in S.K256Q8_TYPES or not S.uses_q8(t) else 32


def reachable(backend, t, order):
    """{(S, R, TPW): (nb, tiles)} over the scan, the case with the fewest weight bytes for each shape"""
    found = {}
    for nb in (NB_32 if block_elems(t) == 32 else NB_K):
        for tiles in TILES:
            s, r, tpw, lds = backend.matvec_shape(t, order, nb * block_elems(t), tiles)
            if s == 0 or lds > (65536 if s == 1 else 163840):
                continue  # such a tensor is refused at upload, or the launch refuses it
            key = (s, r, tpw)
            if key not in found or nb * tiles < found[key][0] * found[key][1]:
                found[key] = (nb, tiles)
    return found


def family_id(f):
    return f"{S.TYPE_NAME[f[0]]}_{'rp' if f[1] == ORDER_REPACKED else 'row'}"


@pytest.mark.parametrize("fam", FAMILIES, ids=family_id)
def test_every_launch_shape_bit_exact(backend, oracle, fam):
    t, order = fam
    shapes = reachable(backend, t, order)
    # the forms the launchers are written for: one wavefront per tile at ring depth 4, and block
    # splits; Q4_K and the 32-value types also reach ring depth 2 on large launches
    assert any(k[:2] == (1, 4) for k in shapes) and any(k[0] > 1 for k in shapes), shapes
    o_order = O_RP if order == ORDER_REPACKED else O_ROW
    for (s, r, tpw), (nb, tiles) in sorted(shapes.items()):
        rows = tiles * tile_rows(t)
        cols = nb * block_elems(t)
        seed = 1000 + 13 * s + r + nb
        w = S.random_bytes_weights(t, rows, cols, seed)
        x = S.activations(cols, seed + 1)
        tt = backend.upload(t, cols, w, order=order)
        assert backend.matvec_shape(t, order, cols, tiles)[:3] == (s, r, tpw)
        y = backend.matvec(tt, x)
        assert bits_equal(y, oracle.matvec(t, w, cols, x, o_order)), \
            f"matvec S={s} R={r} TPW={tpw} nb={nb} tiles={tiles}"
        # the integer-dump form of the same shape: a sample of rows against the oracle
        si, mi = backend.block_ints(tt, x)
        act = oracle.quantize_for(t, x)
        for row in sorted({0, 1, rows // 2, rows - 1}):
            os_, om = oracle.block_ints(t, w[row], act)
            assert np.array_equal(si[row], os_) and np.array_equal(mi[row], om), f"ints S={s} R={r} row {row}"
        # the silu entry on the same shape
        g = S.activations(cols, seed + 2) * np.float32(2.0)
        u = S.activations(cols, seed + 3)
        h = (g / (np.float32(1.0) + oracle.libm_expf(-g)) * u).astype(np.float32)
        assert bits_equal(backend.matvec_silu(tt, g, u), oracle.matvec(t, w, cols, h, o_order)), \
            f"silu S={s} R={r} nb={nb} tiles={tiles}"
        tt.free()


@pytest.mark.parametrize("fam", FAMILIES[:3], ids=family_id)
@pytest.mark.parametrize("rows,cols", [(5120, 5120), (6144, 4096), (4616, 4096)])
def test_two_tiles_per_workgroup_split(backend, oracle, fam, rows, cols):
    """4-way splits of 9/8 to 2 tiles per compute unit hold 2 tiles per workgroup: 5120 x 5120
    (320 tiles), QKV 6144 x 4096 (384), 4616 x 4096 (289 tiles: a partly filled last tile and
    workgroup), bit for bit against the oracle."""
    t, order = fam
    tiles = (rows + 15) // 16
    shape = backend.matvec_shape(t, order, cols, tiles)
    print(f"{S.TYPE_NAME[t]} order {order} {rows}x{cols} shape {shape}", flush=True)
    assert shape[:3] == (4, 2, 2), shape  # MI355X: 256 compute units
    w = S.random_bytes_weights(t, rows, cols, rows + cols + t)
    x = S.activations(cols, rows + 1)
    tt = backend.upload(t, cols, w, order=order)
    o_order = O_RP if order == ORDER_REPACKED else O_ROW
    assert bits_equal(backend.matvec(tt, x), oracle.matvec(t, w, cols, x, o_order))
    tt.free()


@pytest.mark.parametrize("fam", FAMILIES[3:], ids=family_id)
@pytest.mark.parametrize("rows,nb32,nb256", [(512, 163, 43), (4096, 451, 57)])
def test_split_chain_long_tail(backend, oracle, fam, rows, nb32, nb256):
    """Block splits whose final chain runs many whole batches of records before the tested last
    batch: rows of 163 / 451 32-value blocks (a last step of 3 blocks) or 43 / 57 256-value
    blocks, 512 rows and the down projection's 4096, bit for bit against the oracle."""
    t, order = fam
    nb = nb32 if block_elems(t) == 32 else nb256
    tiles, cols = rows // tile_rows(t), nb * block_elems(t)
    shape = backend.matvec_shape(t, order, cols, tiles)
    print(f"{S.TYPE_NAME[t]} order {order} {rows}x{cols} shape {shape}", flush=True)
    assert shape[0] > 1, shape
    w = S.random_bytes_weights(t, rows, cols, rows + nb + t)
    x = S.activations(cols, rows + 2)
    tt = backend.upload(t, cols, w, order=order)
    o_order = O_RP if order == ORDER_REPACKED else O_ROW
    assert bits_equal(backend.matvec(tt, x), oracle.matvec(t, w, cols, x, o_order))
    tt.free()


@pytest.mark.parametrize("order", [ORDER_REPACKED, ORDER_ROW], ids=["rp", "row"])
def test_gate_up_one_launch_at_benchmark_size(backend, oracle, order):
    """The benchmark's dominant launch: gate and up (4096 -> 14336 each, benchmark distributions)
    in one matvec_multi (the reference's forward, fastgguf.c:4870-4872; matvec_multi 2552-2572),
    both outputs bit for bit against the oracle (dot_q4Kx8, fastgguf.c:2322-2358, or
    dot_q4_K_q8k, 1118-1176)."""
    rows, cols = 14336, 4096
    wg = S.weights(S.T_Q4_K, rows, cols, 901)
    wu = S.weights(S.T_Q4_K, rows, cols, 902)
    tg = backend.upload(S.T_Q4_K, cols, wg, order=order)
    tu = backend.upload(S.T_Q4_K, cols, wu, order=order)
    # one launch over both tensors' 2 x 896 tiles of 16 rows: one wavefront per tile, ring depth 2
    assert backend.matvec_shape(S.T_Q4_K, order, cols, 2 * rows // 16)[:3] == (1, 2, 4)
    o_order = O_RP if order == ORDER_REPACKED else O_ROW
    for seed in (903, 904):
        x = S.activations(cols, seed)
        yg, yu = backend.matvec_multi([tg, tu], x)
        assert bits_equal(yg, oracle.matvec(S.T_Q4_K, wg, cols, x, o_order))
        assert bits_equal(yu, oracle.matvec(S.T_Q4_K, wu, cols, x, o_order))
    tg.free()
    tu.free()


GATE_UP_CASES = [  # type, order, rows, cols: one tile pair to the benchmark shape, odd tile counts,
    # the split (2 wavefronts per tile) and unsplit forms; Q6_K / Q8_0: matvecs then the silu launch
    (S.T_Q4_K, ORDER_REPACKED, 14336, 4096), (S.T_Q4_K, ORDER_ROW, 14336, 4096),
    (S.T_Q4_K, ORDER_REPACKED, 16, 256), (S.T_Q4_K, ORDER_REPACKED, 48, 4096), (S.T_Q4_K, ORDER_ROW, 208, 14336),
    (S.T_Q4_K, ORDER_REPACKED, 3200, 512), (S.T_Q5_K, ORDER_ROW, 1040, 2048), (S.T_Q5_K, ORDER_ROW, 7168, 768),
    (S.T_Q6_K, ORDER_ROW, 1000, 2048), (S.T_Q8_0, ORDER_ROW, 1000, 4096),
]


@pytest.mark.parametrize("case", GATE_UP_CASES, ids=lambda c: f"{S.TYPE_NAME[c[0]]}_{c[1]}_{c[2]}x{c[3]}")
def test_gate_up_silu_bit_exact(backend, oracle, case):
    """fgh_matvec_gate_up_silu_dev: h = silu_f(g) * u with g, u the gate and up matvecs (forward,
    fastgguf.c:4870-4876), bit for bit against the oracle's matvecs followed by the reference's
    loop (libm expf, fp32), and against fgh_matvec_multi followed by the same loop."""
    t, order, rows, cols = case
    wg = S.random_bytes_weights(t, rows, cols, 700 + rows)
    wu = S.random_bytes_weights(t, rows, cols, 701 + rows)
    x = S.activations(cols, 702) * np.float32(2.0)
    tg = backend.upload(t, cols, wg, order=order)
    tu = backend.upload(t, cols, wu, order=order)
    o_order = O_RP if order == ORDER_REPACKED else O_ROW
    g = oracle.matvec(t, wg, cols, x, o_order)
    u = oracle.matvec(t, wu, cols, x, o_order)
    want = (g / (np.float32(1.0) + oracle.libm_expf(-g)) * u).astype(np.float32)
    h = backend.matvec_gate_up_silu(tg, tu, x)
    assert bits_equal(h, want)
    gm, um = backend.matvec_multi([tg, tu], x)
    assert bits_equal(gm, g) and bits_equal(um, u)
    for tt in (tg, tu):
        tt.free()


def test_split_launches_graph_replays(backend, oracle):
    """Q4_0 (repacked), Q8_0 and Q2_K matvecs over 4096 x 14336 (block splits with long final
    chains) captured in one HIP graph: every replay, with eager calls and host synchronizations
    between the replays and the outputs overwritten before each, gives the oracle's bits."""
    rows, cols = 4096, 14336
    cases = [(S.T_Q4_0, ORDER_REPACKED, O_RP), (S.T_Q8_0, ORDER_ROW, O_ROW), (S.T_Q2_K, ORDER_ROW, O_ROW)]
    ws = [S.random_bytes_weights(t, rows, cols, 80 + i) for i, (t, _, _) in enumerate(cases)]
    x = S.activations(cols, 81)
    ts = [backend.upload(t, cols, w, order=o) for (t, o, _), w in zip(cases, ws)]
    for (t, o, _), tt in zip(cases, ts):
        assert backend.matvec_shape(t, o, cols, rows // tile_rows(t))[0] > 1
    want = [oracle.matvec(t, w, cols, x, oo) for (t, _, oo), w in zip(cases, ws)]
    xd = backend.dev_alloc(4 * cols)
    yds = [backend.dev_alloc(4 * rows) for _ in cases]
    backend.h2d(xd, x)
    for tt, yd in zip(ts, yds):  # eager first
        backend.matvec_dev(tt, xd, yd)
    backend.sync()
    backend.graph_begin()
    for tt, yd in zip(ts, yds):
        backend.matvec_dev(tt, xd, yd)
    g = backend.graph_end()
    try:
        for rep in range(3):
            for yd in yds:
                backend.h2d(yd, np.full(rows, np.nan, np.float32))
            backend.graph_launch(g)
            backend.sync()
            for (t, _, _), yd, yw in zip(cases, yds, want):
                y = np.empty(rows, np.float32)
                backend.d2h(y, yd)
                assert bits_equal(y, yw), f"{S.TYPE_NAME[t]} replay {rep}"
            assert bits_equal(backend.matvec(ts[1], x), want[1])  # eager work between replays
    finally:
        backend.graph_destroy(g)
    for p in [xd] + yds:
        backend.dev_free(p)
    for tt in ts:
        tt.free()


DEEP = [(S.T_Q4_0, ORDER_REPACKED), (S.T_Q4_0, ORDER_ROW), (S.T_Q8_0, ORDER_ROW), (S.T_Q4_1, ORDER_ROW),
        (S.T_Q5_0, ORDER_ROW), (S.T_Q5_1, ORDER_ROW), (S.T_IQ4_NL, ORDER_ROW)]


@pytest.mark.parametrize("fam", DEEP, ids=family_id)
@pytest.mark.parametrize("rows,nb", [(5123, 451), (6401, 161)])
def test_deep_ring_unsplit_ragged(backend, oracle, fam, rows, nb):
    """Unsplit launches with rings of 8 or 16 steps (at most 1024 tiles over rows of 32 steps or
    more) on ragged shapes: a partly filled last tile (rows % 8 != 0) and a last step of 3 or 1
    blocks, bit for bit against the oracle. 6401 rows are 801 tiles, which the types with 2-way
    splits up to 1536 tiles (Q4_0, Q5_0, IQ4_NL) split instead."""
    t, order = fam
    cols, tiles = nb * 32, (rows + 7) // 8
    shape = backend.matvec_shape(t, order, cols, tiles)
    print(f"{S.TYPE_NAME[t]} order {order} {rows}x{cols} shape {shape}", flush=True)
    nib = t in (S.T_Q4_0, S.T_Q5_0, S.T_IQ4_NL)
    if rows == 5123 or not nib:
        assert shape[0] == 1 and shape[1] in (8, 16), shape
    w = S.random_bytes_weights(t, rows, cols, rows + nb + t)
    x = S.activations(cols, rows + 3)
    tt = backend.upload(t, cols, w, order=order)
    o_order = O_RP if order == ORDER_REPACKED else O_ROW
    assert bits_equal(backend.matvec(tt, x), oracle.matvec(t, w, cols, x, o_order))
    tt.free()


@pytest.mark.parametrize("fam", [(S.T_Q8_0, ORDER_ROW), (S.T_Q4_1, ORDER_ROW), (S.T_Q5_1, ORDER_ROW)], ids=family_id)
def test_deep_ring_per_token_matmul(backend, oracle, fam):
    """The per-token matmul (3 tokens: the decode kernel with grid.y = tokens) over 256 tiles of
    rows of 33 steps: 768 tile-token launches, unsplit with a ring of 8, each token's row bit for
    bit against the oracle."""
    t, order = fam
    rows, cols, nt = 2048, 32 * 131, 3
    shape = backend.matvec_shape(t, order, cols, rows // 8, nt)
    print(f"{S.TYPE_NAME[t]} {rows}x{cols} x {nt} tokens shape {shape}", flush=True)
    assert shape[:2] == (1, 8), shape
    w = S.random_bytes_weights(t, rows, cols, 77 + t)
    X = S.activations(cols, 78 + t, rows=nt)
    tt = backend.upload(t, cols, w, order=order)
    Y = backend.matmul(tt, X)
    Yo = oracle.matmul(t, w, cols, X, O_ROW)
    for b in range(nt):
        assert bits_equal(Y[b], Yo[b]), f"token {b}"
    tt.free()
