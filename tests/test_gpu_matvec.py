"""GPU parity of the decode path: device quantizers, per-block integers and matvec outputs against
the oracle (and the reference's golden vectors), through the C ABI.

Bar: bit-exact. Activation quants, scales and sums, and per-block integer dot products are
integer work; the fp32 matvec outputs reproduce the reference kernels' accumulation order
(dot_q8_0_q8 / dot_q4_K_q8k / dot_q4Kx8 / dot_q6_K_q8k / dot_q5_0_q8 / dot_q5_K_q8k), so they are
compared bit for bit too
(stronger than the 1e-5 per-vector tolerance the north star allows, which is also checked).
"""
import numpy as np
import pytest
from conftest import bits_equal, golden, rel_err

from fastgguf_amd import synth as S
from fastgguf_amd.backend import ORDER_REPACKED, ORDER_ROW, SKIP_MEM, SKIP_TYPE, BackendError
from oracle import ORDER_REPACKED as O_RP
from oracle import ORDER_ROW as O_ROW

pytestmark = pytest.mark.gpu

TOL = 1e-5  # max|y - y_ref| / max|y_ref| per output vector (fastgguf.c:5723-5733)


def check_vec(y, ref):
    assert rel_err(y, ref) <= TOL
    assert bits_equal(y, ref), f"not bit-exact: rel {rel_err(y, ref):.3e}"


def test_open_self_check_leaves_no_trace():
    """fgh_open runs the closed-form self-check of every type (the role of gpu_selfcheck,
    fastgguf.c:1898-1965) and hands over a context with nothing allocated or counted."""
    from fastgguf_amd.backend import Backend
    b = Backend(0)
    i = b.info()
    assert (i["used"], i["n_offloaded"], i["n_skip_type"], i["n_skip_mem"]) == (0, 0, 0, 0)
    b.close()


def test_fp16_decode_exhaustive(backend, oracle):
    """fp16 -> fp32 of all 65536 codes (the reference selftest's table check, fastgguf.c:6022-6031)."""
    h = np.arange(65536, dtype=np.uint16)
    got = backend.fp16_to_f32(h)
    want = np.array([oracle.lib.fgo_fp16(int(v)) for v in h], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_quantizers_match_golden(backend):
    g = golden("quantize.npz")
    for r, x in enumerate(g["quant_x"]):
        assert backend.quantize_q8(x).view(np.uint8).tobytes() == g["quant_q8"][r].tobytes(), f"q8 row {r}"
        assert backend.quantize_q8k(x).view(np.uint8).tobytes() == g["quant_q8k"][r].tobytes(), f"q8k row {r}"


@pytest.mark.parametrize("n", [256, 4096, 14336, 768, 2048, 4096 + 100])
def test_quantizers_bit_exact(backend, oracle, n):
    x = S.activations(n, 40 + n) * np.float32(3.0)
    assert backend.quantize_q8(x).tobytes() == oracle.quantize_q8(x).tobytes()
    assert backend.quantize_q8k(x).tobytes() == oracle.quantize_q8k(x).tobytes()


NAMED = [("q8_0", S.T_Q8_0), ("q4_k", S.T_Q4_K), ("q6_k", S.T_Q6_K), ("q5_0", S.T_Q5_0), ("q5_k", S.T_Q5_K),
         ("q4_0", S.T_Q4_0), ("q4_1", S.T_Q4_1), ("q5_1", S.T_Q5_1), ("iq4_nl", S.T_IQ4_NL)]
REPACKABLE = (S.T_Q4_K, S.T_Q4_0)  # the types the reference repacks (repack_tensor, fastgguf.c:2486)


@pytest.mark.parametrize("name,t", NAMED)
@pytest.mark.parametrize("gen", ["synth", "bytes"])
def test_matvec_matches_golden(backend, name, t, gen):
    g = golden("matvec.npz")
    w, x = g[f"{name}_{gen}_w"], g[f"{name}_{gen}_x"]
    tt = backend.upload(t, x.size, w, order=ORDER_ROW)
    check_vec(backend.matvec(tt, x), g[f"{name}_{gen}_y"])
    tt.free()
    if t in REPACKABLE:
        tt = backend.upload(t, x.size, w, order=ORDER_REPACKED)
        check_vec(backend.matvec(tt, x), g[f"{name}_{gen}_y_rp"])
        tt.free()


CASES = [  # (type, rows, cols, n_mats, order)
    (S.T_Q8_0, 64, 512, 1, ORDER_ROW),
    (S.T_Q8_0, 20, 96, 1, ORDER_ROW),          # 3 blocks: a tile with a padding block
    (S.T_Q8_0, 37, 4096 + 32, 2, ORDER_ROW),   # ragged rows, 3-D
    (S.T_Q4_K, 64, 768, 1, ORDER_REPACKED),
    (S.T_Q4_K, 64, 768, 1, ORDER_ROW),
    (S.T_Q4_K, 21, 256, 3, ORDER_ROW),         # ragged rows, 3-D, one block
    (S.T_Q4_K, 16, 14336, 1, ORDER_REPACKED),  # many chunks
    (S.T_Q4_K, 16, 14336, 1, ORDER_ROW),
    (S.T_Q6_K, 64, 512, 1, ORDER_ROW),
    (S.T_Q6_K, 13, 4608, 2, ORDER_ROW),        # ragged rows, 18 blocks (2 chunks)
    (S.T_Q5_0, 64, 544, 1, ORDER_ROW),         # 17 blocks: a last step of one block
    (S.T_Q5_0, 20, 96, 1, ORDER_ROW),          # 3 blocks: one step with a padding block
    (S.T_Q5_0, 37, 4096 + 64, 2, ORDER_ROW),   # ragged rows, 3-D, a last step of two blocks
    (S.T_Q5_K, 64, 768, 1, ORDER_ROW),
    (S.T_Q5_K, 21, 256, 3, ORDER_ROW),         # ragged rows, 3-D, one block
    (S.T_Q5_K, 16, 14336, 1, ORDER_ROW),       # many blocks (row-order block split over 8 wavefronts)
    (S.T_Q4_K, 21, 4096, 3, ORDER_ROW),        # row-order split over 4 wavefronts, 3-D, ragged rows
    (S.T_Q5_K, 40, 2304, 1, ORDER_ROW),        # row-order split of 9 blocks: runs of 5 and 4
    (S.T_Q4_0, 64, 544, 1, ORDER_REPACKED),    # dot_q40x8's order, a last step of one block
    (S.T_Q4_0, 64, 544, 1, ORDER_ROW),
    (S.T_Q4_0, 37, 4096 + 64, 2, ORDER_ROW),   # 3-D, ragged rows, split launch
    (S.T_Q4_0, 16, 4096 + 96, 1, ORDER_REPACKED),  # repacked order through a split launch
    (S.T_Q4_1, 64, 544, 1, ORDER_ROW),
    (S.T_Q4_1, 20, 96, 1, ORDER_ROW),          # 3 blocks: the min chain over a padding block
    (S.T_Q4_1, 37, 4096 + 64, 2, ORDER_ROW),   # the min chain through split records
    (S.T_Q5_1, 64, 544, 1, ORDER_ROW),
    (S.T_Q5_1, 37, 4096 + 96, 2, ORDER_ROW),
    (S.T_IQ4_NL, 64, 544, 1, ORDER_ROW),
    (S.T_IQ4_NL, 37, 4096 + 32, 2, ORDER_ROW),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"t{c[0]}_{c[1]}x{c[2]}x{c[3]}_o{c[4]}")
def test_block_ints_and_matvec_exact(backend, oracle, case):
    t, rows, cols, n_mats, order = case
    w = S.random_bytes_weights(t, rows * n_mats, cols, 5 + rows)
    x = S.activations(cols, 6 + rows)
    tt = backend.upload(t, cols, w, rows=rows, n_mats=n_mats, order=order)
    act = oracle.quantize_for(t, x)
    s, m = backend.block_ints(tt, x)
    for r in range(rows * n_mats):
        os_, om = oracle.block_ints(t, w[r], act)
        assert np.array_equal(s[r], os_), f"sumi row {r}"
        assert np.array_equal(m[r], om), f"msum row {r}"
    check_vec(backend.matvec(tt, x), oracle.matvec(t, w, cols, x, O_RP if order == ORDER_REPACKED else O_ROW))
    tt.free()


@pytest.mark.parametrize("cfg", ["cfg1_q8_0", "gate_q4k_rp", "gate_q4k_row", "down_q4k_rp", "lmhead_q6k",
                                 "gate_q5k", "down_q5_0", "down_q5k", "down_q4k_row", "down_q8_0", "gate_q4_0_rp",
                                 "down_q4_1", "gate_iq4_nl"])
def test_matvec_config_shapes(backend, oracle, cfg):
    """The benchmark configs' shapes with the benchmark's weight distributions (and the same FFN shapes
    for Q5_K and Q5_0)."""
    t, rows, cols, order = {
        "cfg1_q8_0": (S.T_Q8_0, 4096, 4096, ORDER_ROW),
        "gate_q4k_rp": (S.T_Q4_K, 14336, 4096, ORDER_REPACKED),
        "gate_q4k_row": (S.T_Q4_K, 14336, 4096, ORDER_ROW),
        "down_q4k_rp": (S.T_Q4_K, 4096, 14336, ORDER_REPACKED),
        "lmhead_q6k": (S.T_Q6_K, 128256, 4096, ORDER_ROW),
        "gate_q5k": (S.T_Q5_K, 14336, 4096, ORDER_ROW),
        "down_q5_0": (S.T_Q5_0, 4096, 14336, ORDER_ROW),
        "down_q5k": (S.T_Q5_K, 4096, 14336, ORDER_ROW),
        "down_q4k_row": (S.T_Q4_K, 4096, 14336, ORDER_ROW),
        "down_q8_0": (S.T_Q8_0, 4096, 14336, ORDER_ROW),
        "gate_q4_0_rp": (S.T_Q4_0, 14336, 4096, ORDER_REPACKED),
        "down_q4_1": (S.T_Q4_1, 4096, 14336, ORDER_ROW),
        "gate_iq4_nl": (S.T_IQ4_NL, 14336, 4096, ORDER_ROW),
    }[cfg]
    w = S.weights(t, rows, cols, 11)
    x = S.activations(cols, 12)
    tt = backend.upload(t, cols, w, order=order)
    y = backend.matvec(tt, x)
    check_vec(y, oracle.matvec(t, w, cols, x, O_RP if order == ORDER_REPACKED else O_ROW))
    # a second call on the same tensor with another x (buffers reused)
    x2 = S.activations(cols, 13)
    check_vec(backend.matvec(tt, x2), oracle.matvec(t, w, cols, x2, O_RP if order == ORDER_REPACKED else O_ROW))
    tt.free()


def test_matvec_multi_qkv(backend, oracle):
    """matvec_multi (fastgguf.c:2552): Q, K, V of one layer read one quantized x."""
    cols = 4096
    ws = [S.weights(S.T_Q4_K, r, cols, 20 + i) for i, r in enumerate((4096, 1024, 1024))]
    ts = [backend.upload(S.T_Q4_K, cols, w) for w in ws]
    x = S.activations(cols, 23)
    ys = backend.matvec_multi(ts, x)
    for w, y in zip(ws, ys):
        check_vec(y, oracle.matvec(S.T_Q4_K, w, cols, x, O_RP))
    for t in ts:
        t.free()


@pytest.mark.parametrize("t", [v for _, v in NAMED])
@pytest.mark.parametrize("nb", [2, 3, 7])
def test_matmul_small_batch(backend, oracle, t, nb):
    """nb < 8: the per-token decode kernel (matmul 3006-3009 for repacked tensors; the x4 tiles
    otherwise, which equal the single-row kernels)."""
    cols, rows = 1024, 72
    w = S.weights(t, rows, cols, 30 + nb)
    X = S.activations(cols, 31 + nb, rows=nb)
    tt = backend.upload(t, cols, w)
    Y = backend.matmul(tt, X)
    order = O_RP if t in REPACKABLE else O_ROW
    Yo = oracle.matmul(t, w, cols, X, order)
    for b in range(nb):
        check_vec(Y[b], Yo[b])
    tt.free()


def test_upload_refusals(backend):
    info0 = backend.info()
    with pytest.raises(BackendError) as e:
        backend.upload(S.T_Q4_K, 300, np.zeros(8 * 144 * 2, np.uint8), rows=8)  # cols % 256 != 0
    assert e.value.status == SKIP_TYPE
    with pytest.raises(BackendError) as e:
        backend.upload(15, 256, np.zeros(8 * 292, np.uint8), rows=8)  # Q8_K: not a weight type here
    assert e.value.status == SKIP_TYPE
    with pytest.raises(BackendError) as e:  # F32 / F16 / BF16 past 40960 values: x past 160 KiB of LDS
        backend.upload(S.T_F16, 40961, np.zeros(8 * 40961 * 2, np.uint8), rows=8)
    assert e.value.status == SKIP_TYPE
    with pytest.raises(BackendError) as e:  # Q2_K needs cols % 256 == 0
        backend.upload(S.T_Q2_K, 288, np.zeros(8 * 84, np.uint8), rows=8)
    assert e.value.status == SKIP_TYPE
    with pytest.raises(BackendError) as e:  # Q2_K / Q3_K / IQ4_XS past 204 blocks: x past 64 KiB of LDS
        backend.upload(S.T_IQ4_XS, 205 * 256, np.zeros(8 * 205 * 136, np.uint8), rows=8)
    assert e.value.status == SKIP_TYPE
    with pytest.raises(BackendError) as e:  # 238 blocks: the quantized x no longer fits 64 KiB of LDS
        backend.upload(S.T_Q4_K, 238 * 256, np.zeros(16 * 238 * 144, np.uint8), rows=16)
    assert e.value.status == SKIP_TYPE
    with pytest.raises(BackendError) as e:  # the same for Q6_K past 224 blocks and Q8_0 past 1820
        backend.upload(S.T_Q6_K, 225 * 256, np.zeros(8 * 225 * 210, np.uint8), rows=8)
    assert e.value.status == SKIP_TYPE
    with pytest.raises(BackendError) as e:
        backend.upload(S.T_Q8_0, 1821 * 32, np.zeros(8 * 1821 * 34, np.uint8), rows=8)
    assert e.value.status == SKIP_TYPE
    with pytest.raises(BackendError) as e:  # Q5_K as Q4_K (238 blocks), Q5_0 as Q8_0 (1821)
        backend.upload(S.T_Q5_K, 238 * 256, np.zeros(16 * 238 * 176, np.uint8), rows=16)
    assert e.value.status == SKIP_TYPE
    with pytest.raises(BackendError) as e:
        backend.upload(S.T_Q5_0, 1821 * 32, np.zeros(8 * 1821 * 22, np.uint8), rows=8)
    assert e.value.status == SKIP_TYPE
    with pytest.raises(BackendError) as e:  # Q4_1 past 1636 blocks (its block sums share the LDS)
        backend.upload(S.T_Q4_1, 1637 * 32, np.zeros(8 * 1637 * 20, np.uint8), rows=8)
    assert e.value.status == SKIP_TYPE
    with pytest.raises(BackendError) as e:  # Q5_0 cols % 32 != 0
        backend.upload(S.T_Q5_0, 48, np.zeros(8 * 22, np.uint8), rows=8)
    assert e.value.status == SKIP_TYPE
    info1 = backend.info()
    assert info1["n_skip_type"] == info0["n_skip_type"] + 12
    from fastgguf_amd.backend import Backend
    small = Backend(0, budget_bytes=1 << 20)
    with pytest.raises(BackendError) as e:
        small.upload(S.T_Q4_K, 4096, S.weights(S.T_Q4_K, 512, 4096, 1))  # 1.2 MB > 1 MB budget
    assert e.value.status == SKIP_MEM and small.info()["n_skip_mem"] == 1
    small.close()


@pytest.mark.parametrize("order", [ORDER_REPACKED, ORDER_ROW])
def test_widest_q4k_rows(backend, oracle, order):
    """237 blocks (K = 60672), the widest Q4_K row the decode kernel accepts, in both orders."""
    rows, cols = 24, 237 * 256
    w = S.random_bytes_weights(S.T_Q4_K, rows, cols, 131)
    x = S.activations(cols, 132)
    tt = backend.upload(S.T_Q4_K, cols, w, order=order)
    y = backend.matvec(tt, x)
    yo = oracle.matvec(S.T_Q4_K, w, cols, x, O_RP if order == ORDER_REPACKED else O_ROW)
    assert bits_equal(y, yo)
    tt.free()


@pytest.mark.parametrize("t,nb", [(S.T_Q6_K, 224), (S.T_Q8_0, 1820), (S.T_Q8_0, 1819), (S.T_Q5_0, 1820),
                                  (S.T_Q5_0, 1817), (S.T_Q5_K, 237), (S.T_Q4_1, 1636), (S.T_Q4_0, 1818)])
def test_widest_q6k_q80_rows(backend, oracle, t, nb):
    """The widest Q6_K (K = 57344), Q8_0 / Q5_0 / Q4_0 (K = 58240), Q4_1 (K = 52352, its block sums
    beside the quantized x) and Q5_K (K = 60672) rows the decode kernels accept, and widths whose
    last 4-block step is ragged."""
    rows, cols = 20, nb * (32 if S.uses_q8(t) else 256)
    w = S.random_bytes_weights(t, rows, cols, 133 + nb)
    x = S.activations(cols, 134)
    tt = backend.upload(t, cols, w)
    # AUTO keeps the row order here: 20 rows are not a multiple of 8 (repack_tensor, fastgguf.c:2487)
    assert bits_equal(backend.matvec(tt, x), oracle.matvec(t, w, cols, x, O_ROW))
    tt.free()


SILU_CASES = [  # (type, rows, cols, order): split launches (S > 1) and one-wavefront tiles
    (S.T_Q4_K, 48, 14336, ORDER_REPACKED),
    (S.T_Q4_K, 4096, 14336, ORDER_REPACKED),  # the Llama-3-8B down projection
    (S.T_Q4_K, 40, 2048, ORDER_ROW),
    (S.T_Q6_K, 13, 4608, ORDER_ROW),
    (S.T_Q8_0, 37, 4128, ORDER_ROW),
    (S.T_Q5_K, 40, 2048, ORDER_ROW),
    (S.T_Q5_0, 37, 4128, ORDER_ROW),
    (S.T_Q4_0, 48, 4128, ORDER_REPACKED),
    (S.T_Q4_1, 37, 4128, ORDER_ROW),
    (S.T_IQ4_NL, 37, 4128, ORDER_ROW),
]


@pytest.mark.parametrize("case", SILU_CASES, ids=lambda c: f"t{c[0]}_{c[1]}x{c[2]}_o{c[3]}")
def test_matvec_silu_fused(backend, oracle, case):
    """fgh_matvec_silu_dev: y = W * Q8(silu(g) * u) equals the reference's loop (silu_f with
    libm expf, times up, in fp32) followed by the matvec, bit for bit."""
    t, rows, cols, order = case
    w = S.random_bytes_weights(t, rows, cols, 141 + rows)
    g = S.activations(cols, 142) * np.float32(3.0)
    u = S.activations(cols, 143)
    h = (g / (np.float32(1.0) + oracle.libm_expf(-g)) * u).astype(np.float32)
    tt = backend.upload(t, cols, w, order=order)
    y = backend.matvec_silu(tt, g, u)
    assert bits_equal(y, backend.matvec(tt, h))
    assert bits_equal(y, oracle.matvec(t, w, cols, h, O_RP if order == ORDER_REPACKED else O_ROW))
    tt.free()


def test_graph_replay_matches_eager(backend, oracle):
    """A captured layer (QKV, gate+up in one launch) replayed several times, with eager work and
    synchronizations between replays: every replay equals the eager result and the oracle."""
    cols = 4096
    ws = {n: S.weights(S.T_Q4_K, r, cols, 60 + i) for i, (n, r) in enumerate((("qkv", 1536), ("gate", 2048), ("up", 2048)))}
    ts = {n: backend.upload(S.T_Q4_K, cols, w) for n, w in ws.items()}
    x = S.activations(cols, 64)
    xd = backend.dev_alloc(4 * cols)
    backend.h2d(xd, x)
    yd = {n: backend.dev_alloc(4 * w.shape[0]) for n, w in ws.items()}
    backend.graph_begin()
    backend.matvec_dev(ts["qkv"], xd, yd["qkv"])
    backend.matvec_multi_dev([ts["gate"], ts["up"]], xd, [yd["gate"], yd["up"]])
    g = backend.graph_end()
    want = {n: oracle.matvec(S.T_Q4_K, w, cols, x, O_RP) for n, w in ws.items()}
    for rep in range(4):
        for n in yd:  # clobber the outputs eagerly between replays
            backend.h2d(yd[n], np.full(ws[n].shape[0], np.nan, np.float32))
        backend.graph_launch(g)
        backend.sync()
        for n in yd:
            got = np.empty(ws[n].shape[0], np.float32)
            backend.d2h(got, yd[n])
            check_vec(got, want[n])
        check_vec(backend.matvec(ts["qkv"], x), want["qkv"])  # eager call between replays
    backend.graph_destroy(g)
    with pytest.raises(BackendError):  # host-synchronous calls are refused while capturing
        backend.graph_begin()
        try:
            backend.matvec(ts["qkv"], x)
        finally:
            backend.graph_destroy(backend.graph_end())
    for p in list(yd.values()) + [xd]:
        backend.dev_free(p)
    for t in ts.values():
        t.free()


@pytest.mark.parametrize("nbytes", [0, 16, 4096 + 48, (1 << 24) + 16 * 7])
def test_checksum_dev(backend, nbytes):
    """The streaming checksum: the wrapping sum of the buffer's 32-bit words, against numpy."""
    a = np.random.default_rng(nbytes).integers(0, 1 << 32, nbytes // 4, dtype=np.uint64).astype(np.uint32)
    src = backend.dev_alloc(max(nbytes, 16))
    if nbytes:
        backend.h2d(src, a)
    want = int(np.sum(a, dtype=np.uint64) & 0xFFFFFFFF)
    assert backend.checksum(src, nbytes) == want
    backend.dev_free(src)


def test_copy_d2d(backend):
    """The plain copy kernel (device-to-device; also the HBM-counter calibration kernel)."""
    a = np.arange(1 << 20, dtype=np.uint32)
    src, dst = backend.dev_alloc(a.nbytes), backend.dev_alloc(a.nbytes)
    backend.h2d(src, a)
    backend.d2d(dst, src, a.nbytes)
    b = np.empty_like(a)
    backend.d2h(b, dst)
    assert np.array_equal(a, b)
    backend.dev_free(src)
    backend.dev_free(dst)
