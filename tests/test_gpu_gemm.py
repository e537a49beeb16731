"""GPU parity of the prompt-batch matmul (nb = 8..64 tokens, the reference's gemm_kquant path,
fastgguf.c:3018-3031) through the C ABI.

Bar:
  - Q4_K runs the int8 MFMA GEMM. Its per-(token, row, block) integers sumi / msum are compared bit
    for bit with the oracle's (dot_q4_K_q8k's integers on each token's Q8_K activations). Its fp32
    outputs use a different summation order from gemmk_kern, so they are compared with the
    reference's own tolerance: max|y - y_ref| / max|y_ref| <= 1e-5 per token (fastgguf.c:5723-5733),
    against the oracle's restatement of gemm_kquant and against the reference's golden outputs.
  - Q6_K runs its int8 MFMA GEMM (three chains over balanced base-8 digits of the scales): its
    per-block integers (dot_q6_K_q8k's sumi over the unsigned quants, and msum) bit for bit
    against the oracle's, its fp32 outputs within the same tolerance of gemm_kquant's order.
  - Q8_0 runs its int8 MFMA GEMM (one 32-value block per v_mfma_i32_32x32x32_i8, K split in up to 4
    parts): its per-block integers (dot_q8_0_q8's sum of q * xq) bit for bit against the oracle's,
    its fp32 outputs within the same tolerance of the oracle's GEMM order (gemm_q32).
  - Q4_0, Q4_1, Q5_0 and Q5_1 run the nibble-type MFMA GEMM in gemm_q32's own order (no K split):
    its per-block integers (gemm_q32's sum of unsigned weight times quant) bit for bit against the
    oracle's row integers plus offset times the quant sum, and its fp32 outputs bit for bit against
    the oracle's gemm_q32 and the reference's golden outputs (both orders of Q4_0: the reference's
    GEMM unpacks the repacked rows to the same values).
  - Q5_K and IQ4_NL have no prompt GEMM in the reference: their matmul is the row kernel per token
    there and here, so they are compared bit for bit.
"""
import numpy as np
import pytest
from conftest import bits_equal, golden, rel_err

from fastgguf_amd import synth as S
from fastgguf_amd.backend import ORDER_REPACKED, ORDER_ROW
from oracle import ORDER_REPACKED as O_RP
from oracle import ORDER_ROW as O_ROW

pytestmark = pytest.mark.gpu

TOL = 1e-5


def check_tokens(Y, Yref):
    assert Y.shape == Yref.shape
    for t in range(Y.shape[0]):
        e = rel_err(Y[t], Yref[t])
        assert e <= TOL, f"token {t}: rel err {e:.3e}"


@pytest.mark.parametrize("name,t", [("q8_0", S.T_Q8_0), ("q4_k", S.T_Q4_K), ("q6_k", S.T_Q6_K),
                                    ("q5_0", S.T_Q5_0), ("q5_k", S.T_Q5_K), ("q4_0", S.T_Q4_0),
                                    ("q4_1", S.T_Q4_1), ("q5_1", S.T_Q5_1), ("iq4_nl", S.T_IQ4_NL)])
@pytest.mark.parametrize("nb", [8, 45])
def test_matmul_matches_golden(backend, name, t, nb):
    g = golden("matmul.npz")
    w, X = g[f"{name}_w"], g[f"{name}_X{nb}"]
    for order, key in ((ORDER_ROW, f"{name}_Y{nb}"), (ORDER_REPACKED, f"{name}_Y{nb}_rp")):
        if order == ORDER_REPACKED and t not in (S.T_Q4_K, S.T_Q4_0):
            continue
        tt = backend.upload(t, X.shape[1], w, order=order)
        Y = backend.matmul(tt, X)
        check_tokens(Y, g[key])
        # no prompt GEMM in the reference (its row kernel per token), or gemm_q32's own order
        if t in (S.T_Q5_K, S.T_IQ4_NL, S.T_Q4_0, S.T_Q4_1, S.T_Q5_0, S.T_Q5_1):
            assert bits_equal(Y, g[key])
        tt.free()


GEMM_CASES = [  # (rows, cols, n_mats, tokens); K splits (few row groups) as noted
    (64, 256, 1, 8),        # one block, one workgroup
    (100, 512, 1, 31),      # ragged rows, one token tile
    (128, 1024, 1, 32),
    (72, 768, 1, 33),       # odd block count, two token tiles
    (21, 2048, 3, 45),      # 3-D, ragged rows per matrix; 2 K splits of 4 blocks
    (48, 3072, 1, 17),      # 3 K splits of 4 blocks
    (64, 4096, 1, 64),      # 4 K splits of 4 blocks
    (16, 14336, 1, 64),     # 56 blocks, 4 K splits of 14
]


@pytest.mark.parametrize("case", GEMM_CASES, ids=lambda c: f"{c[0]}x{c[1]}x{c[2]}_T{c[3]}")
def test_gemm_block_ints_exact(backend, oracle, case):
    rows, cols, n_mats, T = case
    w = S.random_bytes_weights(S.T_Q4_K, rows * n_mats, cols, 70 + rows)
    X = S.activations(cols, 71 + T, rows=T) * np.float32(2.0)
    tt = backend.upload(S.T_Q4_K, cols, w, rows=rows, n_mats=n_mats)
    s, m = backend.gemm_block_ints(tt, X)
    for tok in (0, T // 2, T - 1):
        act = oracle.quantize_for(S.T_Q4_K, X[tok])
        for r in range(rows * n_mats):
            os_, om = oracle.block_ints(S.T_Q4_K, w[r], act)
            assert np.array_equal(s[tok, r], os_), f"sumi token {tok} row {r}"
            assert np.array_equal(m[tok, r], om), f"msum token {tok} row {r}"
    Y = backend.matmul(tt, X)
    order = O_RP if (n_mats == 1 and rows % 8 == 0) else O_ROW
    check_tokens(Y, oracle.matmul(S.T_Q4_K, w, cols, X, order))
    tt.free()


Q80_CASES = [  # (rows, cols, n_mats, tokens): K-parts 1 (1 tile step), 2 (2-3 steps, one with an
    # Edge step), 4; partial last steps (blocks % 4 != 0); ragged rows; 3-D; both token tiles
    (64, 128, 1, 8),
    (40, 256, 1, 32),
    (100, 416, 1, 31),      # 13 blocks: 4 tile steps, the last with one block
    (72, 384, 3, 45),       # 3 steps (K-parts 2, one idle in the last step), 9 tiles per matrix
    (256, 4096, 1, 64),     # 4 K splits of 8 tile steps (few row groups)
    (24, 14336, 1, 33),     # 448 blocks, 4 K splits of 28 tile steps
    (8, 2080, 2, 9),        # 65 blocks, one 8-row tile per matrix, 2 K splits (9 and 8 steps)
    (40, 3072, 1, 20),      # 3 K splits of 8 tile steps
]


@pytest.mark.parametrize("case", Q80_CASES, ids=lambda c: f"{c[0]}x{c[1]}x{c[2]}_T{c[3]}")
def test_q80_gemm_block_ints_exact(backend, oracle, case):
    rows, cols, n_mats, T = case
    w = S.random_bytes_weights(S.T_Q8_0, rows * n_mats, cols, 170 + rows)
    X = S.activations(cols, 171 + T, rows=T) * np.float32(2.0)
    tt = backend.upload(S.T_Q8_0, cols, w, rows=rows, n_mats=n_mats)
    s, m = backend.gemm_block_ints(tt, X)
    assert not m.any()  # no min term
    for tok in (0, T // 2, T - 1):
        act = oracle.quantize_for(S.T_Q8_0, X[tok])
        for r in range(rows * n_mats):
            os_, _ = oracle.block_ints(S.T_Q8_0, w[r], act)
            assert np.array_equal(s[tok, r], os_), f"sumi token {tok} row {r}"
    check_tokens(backend.matmul(tt, X), oracle.matmul(S.T_Q8_0, w, cols, X, O_ROW))
    tt.free()


def test_q80_prefill_down_shape(backend, oracle):
    """The FFN down projection, 64 tokens x K=14336 -> N=4096, Q8_0: 4 K splits, within tolerance
    of the oracle's GEMM order, the same bits on every call; then 9 tokens"""
    rows, cols = 4096, 14336
    w = S.weights(S.T_Q8_0, rows, cols, 192)
    X = S.activations(cols, 193, rows=64)
    tt = backend.upload(S.T_Q8_0, cols, w)
    Y = backend.matmul(tt, X)
    check_tokens(Y, oracle.matmul(S.T_Q8_0, w, cols, X, O_ROW))
    assert bits_equal(backend.matmul(tt, X), Y)
    check_tokens(backend.matmul(tt, X[:9]), oracle.matmul(S.T_Q8_0, w, cols, X[:9], O_ROW))
    tt.free()


def test_q80_prefill_config_shape(backend, oracle):
    """64 tokens x K=4096 -> N=14336, Q8_0 (benchmark distributions), then 9 tokens (one token
    tile) reusing the buffers"""
    rows, cols = 14336, 4096
    w = S.weights(S.T_Q8_0, rows, cols, 190)
    X = S.activations(cols, 191, rows=64)
    tt = backend.upload(S.T_Q8_0, cols, w)
    check_tokens(backend.matmul(tt, X), oracle.matmul(S.T_Q8_0, w, cols, X, O_ROW))
    check_tokens(backend.matmul(tt, X[:9]), oracle.matmul(S.T_Q8_0, w, cols, X[:9], O_ROW))
    tt.free()


# the dumped integer minus the oracle's row integer, in units of the block's quant sum: gemm_q32's
# unsigned weights are value + 8 (Q4_0) / + 16 (Q5_0)
Q32N_OFF = {S.T_Q4_0: 8, S.T_Q4_1: 0, S.T_Q5_0: 16, S.T_Q5_1: 0}
Q32N_CASES = [  # (rows, cols, n_mats, tokens): one token tile (8, 16 tokens), 2 and 3 tiles
    # (ragged), 4 tiles; a partial last tile step (blocks % 4 != 0); an odd number of 8-row tiles (a
    # half-empty last pair); ragged rows; 3-D; long rows; launches of ~600 to ~1500 wavefronts, the
    # last with two token tiles per wavefront
    (16, 128, 1, 8),
    (40, 288, 1, 16),       # 9 blocks: 3 tile steps, the last with one block; 5 tiles
    (100, 416, 1, 31),      # 13 blocks; 13 tiles
    (21, 1056, 3, 45),      # 33 blocks, 3-D, 3 tiles per matrix
    (64, 4096, 1, 64),
    (24, 14336, 1, 33),     # 448 blocks
    (4792, 160, 1, 32),     # 300 row pairs x 2 token tiles; ragged rows
    (9600, 96, 1, 32),      # 600 x 2
    (12288, 256, 1, 64),    # 768 x 2 pairs of token tiles
]


@pytest.mark.parametrize("t", [S.T_Q4_0, S.T_Q4_1, S.T_Q5_0, S.T_Q5_1], ids=["q4_0", "q4_1", "q5_0", "q5_1"])
@pytest.mark.parametrize("case", Q32N_CASES, ids=lambda c: f"{c[0]}x{c[1]}x{c[2]}_T{c[3]}")
def test_q32n_gemm_exact(backend, oracle, t, case):
    rows, cols, n_mats, T = case
    w = S.random_bytes_weights(t, rows * n_mats, cols, 270 + rows + t)
    X = S.activations(cols, 271 + T, rows=T) * np.float32(2.0)
    tt = backend.upload(t, cols, w, rows=rows, n_mats=n_mats)
    s, m = backend.gemm_block_ints(tt, X)
    assert not m.any()  # no min integer
    check_rows = range(rows * n_mats) if rows * n_mats <= 256 else range(0, rows * n_mats, 97)
    for tok in (0, T // 2, T - 1):
        act = oracle.quantize_for(t, X[tok])
        qsum = act["s16"].astype(np.int64).sum(axis=1)
        for r in check_rows:
            os_, _ = oracle.block_ints(t, w[r], act)
            assert np.array_equal(s[tok, r], os_ + Q32N_OFF[t] * qsum), f"sumi token {tok} row {r}"
    Y = backend.matmul(tt, X)
    assert bits_equal(Y, oracle.matmul(t, w, cols, X, O_ROW))
    tt.free()


def test_q32n_prefill_config_shape(backend, oracle):
    """64 tokens x K=4096 -> N=14336 and 14336 -> 4096 (benchmark distributions), Q4_0 and Q5_1,
    bit for bit with gemm_q32; then 9 tokens (one token tile) reusing the buffers"""
    for t, seed in ((S.T_Q4_0, 290), (S.T_Q5_1, 291)):
        for rows, cols in ((14336, 4096), (4096, 14336)):
            w = S.weights(t, rows, cols, seed)
            X = S.activations(cols, seed + 1, rows=64)
            tt = backend.upload(t, cols, w)
            assert bits_equal(backend.matmul(tt, X), oracle.matmul(t, w, cols, X, O_ROW))
            assert bits_equal(backend.matmul(tt, X[:9]), oracle.matmul(t, w, cols, X[:9], O_ROW))
            tt.free()


Q6K_CASES = [  # (rows, cols, n_mats, tokens): K-halves 1 (one block) and 2 (odd and even block
    # counts); an odd number of 8-row tiles (a half-empty last pair); ragged rows; 3-D; 1..4 token tiles
    (16, 256, 1, 8),
    (40, 512, 1, 16),
    (100, 768, 1, 31),      # 13 tiles: the last pair has one tile
    (24, 2048, 3, 45),      # 3 tiles per matrix; 2 K splits (few row groups)
    (48, 3072, 1, 17),      # 3 K splits
    (64, 4096, 1, 64),      # 4 K splits
    (8, 14336, 1, 33),      # 56 blocks, one tile, 4 K splits of 14
]


@pytest.mark.parametrize("case", Q6K_CASES, ids=lambda c: f"{c[0]}x{c[1]}x{c[2]}_T{c[3]}")
def test_q6k_gemm_block_ints_exact(backend, oracle, case):
    rows, cols, n_mats, T = case
    w = S.random_bytes_weights(S.T_Q6_K, rows * n_mats, cols, 270 + rows)
    X = S.activations(cols, 271 + T, rows=T) * np.float32(2.0)
    tt = backend.upload(S.T_Q6_K, cols, w, rows=rows, n_mats=n_mats)
    s, m = backend.gemm_block_ints(tt, X)
    for tok in (0, T // 2, T - 1):
        act = oracle.quantize_for(S.T_Q6_K, X[tok])
        for r in range(rows * n_mats):
            os_, om = oracle.block_ints(S.T_Q6_K, w[r], act)
            assert np.array_equal(s[tok, r], os_), f"sumi token {tok} row {r}"
            assert np.array_equal(m[tok, r], om), f"msum token {tok} row {r}"
    check_tokens(backend.matmul(tt, X), oracle.matmul(S.T_Q6_K, w, cols, X, O_ROW))
    tt.free()


def test_q6k_prefill_down_shape(backend, oracle):
    """The FFN down projection (Q6_K in Q4_K_M files), 64 tokens x K=14336 -> N=4096: 4 K splits,
    within tolerance of gemm_kquant, the same bits on every call; then 9 tokens."""
    rows, cols = 4096, 14336
    w = S.weights(S.T_Q6_K, rows, cols, 292)
    X = S.activations(cols, 293, rows=64)
    tt = backend.upload(S.T_Q6_K, cols, w)
    Y = backend.matmul(tt, X)
    check_tokens(Y, oracle.matmul(S.T_Q6_K, w, cols, X, O_ROW))
    assert bits_equal(backend.matmul(tt, X), Y)
    check_tokens(backend.matmul(tt, X[:9]), oracle.matmul(S.T_Q6_K, w, cols, X[:9], O_ROW))
    tt.free()


def test_q6k_prefill_config_shape(backend, oracle):
    """64 tokens x K=4096 -> N=14336, Q6_K (benchmark distributions), then 9 tokens"""
    rows, cols = 14336, 4096
    w = S.weights(S.T_Q6_K, rows, cols, 290)
    X = S.activations(cols, 291, rows=64)
    tt = backend.upload(S.T_Q6_K, cols, w)
    check_tokens(backend.matmul(tt, X), oracle.matmul(S.T_Q6_K, w, cols, X, O_ROW))
    check_tokens(backend.matmul(tt, X[:9]), oracle.matmul(S.T_Q6_K, w, cols, X[:9], O_ROW))
    tt.free()


@pytest.mark.parametrize("t", [S.T_Q8_0, S.T_Q6_K, S.T_Q5_0, S.T_Q5_K, S.T_Q4_0, S.T_Q4_1, S.T_Q5_1, S.T_IQ4_NL])
@pytest.mark.parametrize("nb", [8, 64])
def test_matmul_other_types(backend, oracle, t, nb):
    cols, rows = 2048, 200
    w = S.weights(t, rows, cols, 80 + nb)
    X = S.activations(cols, 81 + nb, rows=nb)
    tt = backend.upload(t, cols, w)
    check_tokens(backend.matmul(tt, X), oracle.matmul(t, w, cols, X, O_RP if t == S.T_Q4_0 else O_ROW))
    tt.free()


def test_prefill_config_shape(backend, oracle):
    """Benchmark config 4: 64 tokens x K=4096 -> N=14336, Q4_K (benchmark distributions)."""
    rows, cols, T = 14336, 4096, 64
    w = S.weights(S.T_Q4_K, rows, cols, 90)
    X = S.activations(cols, 91, rows=T)
    tt = backend.upload(S.T_Q4_K, cols, w)
    Y = backend.matmul(tt, X)
    check_tokens(Y, oracle.matmul(S.T_Q4_K, w, cols, X, O_RP))
    # a second call with fewer tokens reuses the buffers
    Y2 = backend.matmul(tt, X[:9])
    check_tokens(Y2, oracle.matmul(S.T_Q4_K, w, cols, X[:9], O_RP))
    tt.free()


def test_prefill_down_shape(backend, oracle):
    """The FFN down projection of a 64-token prompt, 64 tokens x K=14336 -> N=4096 (Q4_K): 64 row
    groups for 256 compute units, so the GEMM runs 4 K splits whose last arriver adds the partials
    in split order; within tolerance of gemm_kquant, and every call gives the same bits (the
    arrival order does not enter the sum)."""
    rows, cols, T = 4096, 14336, 64
    w = S.weights(S.T_Q4_K, rows, cols, 92)
    X = S.activations(cols, 93, rows=T)
    tt = backend.upload(S.T_Q4_K, cols, w)
    Y = backend.matmul(tt, X)
    check_tokens(Y, oracle.matmul(S.T_Q4_K, w, cols, X, O_RP))
    for _ in range(3):
        assert bits_equal(backend.matmul(tt, X), Y)
    check_tokens(backend.matmul(tt, X[:9]), oracle.matmul(S.T_Q4_K, w, cols, X[:9], O_RP))
    tt.free()


def test_matmul_wide_q4k(backend, oracle):
    """K = 116 blocks (29696), the widest Q4_K rows in use (Llama-70B-like FFN down projections are
    28672): the GEMM with 40 tokens (two token tiles) and 9 tokens, within tolerance of gemm_kquant,
    and its integers exact."""
    rows, cols = 16, 256 * 116
    w = S.random_bytes_weights(S.T_Q4_K, rows, cols, 95)
    tt = backend.upload(S.T_Q4_K, cols, w)
    X = S.activations(cols, 96, rows=40)
    check_tokens(backend.matmul(tt, X), oracle.matmul(S.T_Q4_K, w, cols, X, O_RP))
    check_tokens(backend.matmul(tt, X[:9]), oracle.matmul(S.T_Q4_K, w, cols, X[:9], O_RP))
    s_, m_ = backend.gemm_block_ints(tt, X[:33])
    for tok in (0, 32):
        act = oracle.quantize_for(S.T_Q4_K, X[tok])
        for r in range(rows):
            os_, om = oracle.block_ints(S.T_Q4_K, w[r], act)
            assert np.array_equal(s_[tok, r], os_) and np.array_equal(m_[tok, r], om), f"token {tok} row {r}"
    tt.free()


def test_graph_keeps_scratch_across_a_larger_eager_call(oracle):
    """A graph captured with the prompt GEMM's activation scratch at one size, then an eager call
    that needs more (the scratch grows), then replays: the graph still owns the buffers it was
    captured with (the context retires, not frees, a grown buffer while a graph is alive), so
    every replay equals the eager result bit for bit. A fresh context starts with no scratch."""
    from fastgguf_amd.backend import Backend
    be = Backend(0)
    try:
        cols, rows = 2048, 128
        w = S.weights(S.T_Q4_K, rows, cols, 501)
        t = be.upload(S.T_Q4_K, cols, w)
        wide = be.upload(S.T_Q4_K, 8192, S.weights(S.T_Q4_K, 64, 8192, 502))
        X = S.activations(cols, 503, rows=9)
        Xw = S.activations(8192, 504, rows=64)
        xd, yd = be.dev_alloc(X.nbytes), be.dev_alloc(4 * 9 * rows)
        xwd, ywd = be.dev_alloc(Xw.nbytes), be.dev_alloc(4 * 64 * 64)
        be.h2d(xd, X)
        be.h2d(xwd, Xw)
        want = be.matmul(t, X)  # grows the scratch to this call's size before capture
        be.graph_begin()
        be.matmul_dev(t, xd, yd, 9)
        g = be.graph_end()
        for rep in range(3):
            be.matmul_dev(wide, xwd, ywd, 64)  # 64 tokens x 8192: every GEMM scratch buffer grows
            be.h2d(yd, np.full(9 * rows, np.nan, np.float32))
            be.graph_launch(g)
            be.sync()
            got = np.empty((9, rows), np.float32)
            be.d2h(got, yd)
            assert bits_equal(got, want), f"replay {rep}"
            check_tokens(got, oracle.matmul(S.T_Q4_K, w, cols, X, O_RP))
        be.graph_destroy(g)
        for p in (xd, yd, xwd, ywd):
            be.dev_free(p)
        t.free()
        wide.free()
    finally:
        be.close()


@pytest.mark.parametrize("ty", [S.T_Q4_K, S.T_Q6_K, S.T_Q8_0], ids=["q4_k", "q6_k", "q8_0"])
def test_split_gemm_graph_replays(oracle, ty):
    """The K-split GEMMs inside a HIP graph: the arrival counters are zeroed by the call's own
    quantizer launch (no memset node), so replays with eager calls of another shape in between
    give the eager result bit for bit, every time."""
    from fastgguf_amd.backend import Backend
    be = Backend(0)
    try:
        rows, cols, T = 64, 8192, 40  # one workgroup of rows, K split 4 ways
        w = S.weights(ty, rows, cols, 511)
        t = be.upload(ty, cols, w)
        other = be.upload(ty, 2048, S.weights(ty, 256, 2048, 512))
        X = S.activations(cols, 513, rows=T)
        Xo = S.activations(2048, 514, rows=64)
        xd, yd = be.dev_alloc(X.nbytes), be.dev_alloc(4 * T * rows)
        xod, yod = be.dev_alloc(Xo.nbytes), be.dev_alloc(4 * 64 * 256)
        be.h2d(xd, X)
        be.h2d(xod, Xo)
        want = be.matmul(t, X)
        check_tokens(want, oracle.matmul(ty, w, cols, X, O_RP if ty == S.T_Q4_K else O_ROW))
        be.graph_begin()
        be.matmul_dev(t, xd, yd, T)
        g = be.graph_end()
        for rep in range(4):
            be.h2d(yd, np.full(T * rows, np.nan, np.float32))
            be.graph_launch(g)
            be.matmul_dev(other, xod, yod, 64)
            be.sync()
            got = np.empty((T, rows), np.float32)
            be.d2h(got, yd)
            assert bits_equal(got, want), f"replay {rep}"
        be.graph_destroy(g)
        for p in (xd, yd, xod, yod):
            be.dev_free(p)
        t.free()
        other.free()
    finally:
        be.close()
