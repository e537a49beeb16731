"""GPU parity of the MoE FFN (moe_ffn, fastgguf.c:4588-4642) through the C ABI.

Every dot product runs the reference's own per-row order, so expert selection, weights and outputs
are compared bit for bit: against the reference's golden outputs (including tied router logits)
and against the oracle on random and benchmark config-5 shapes. The one function outside the
integer and IEEE-basic arithmetic is expf (softmax and silu): the device restates glibc's expf
method, checked bit for bit against the host libm here and over every float in test_oracle.
"""
import numpy as np
import pytest
from conftest import bits_equal, golden, rel_err

from fastgguf_amd import synth as S

pytestmark = pytest.mark.gpu


def test_device_expf_matches_libm(backend, oracle):
    """The device expf (softmax, silu) against this host's libm expf, bit for bit: the inputs where
    only a fused evaluation rounds as glibc does, special values, and 4M float bit patterns across
    the range where expf is neither 0 nor infinite."""
    from test_oracle import EXPF_HARD, EXPF_SPECIAL
    rng = np.random.default_rng(7)
    lo = np.float32(-104.0).view(np.uint32)
    bits_pos = rng.integers(0, np.float32(89.0).view(np.uint32), 2_000_000, dtype=np.uint32)
    bits_neg = rng.integers(0x80000000, lo, 2_000_000, dtype=np.uint32)
    xs = np.concatenate([np.array(EXPF_HARD + EXPF_SPECIAL, np.float32), bits_pos.view(np.float32),
                         bits_neg.view(np.float32)])
    got = backend.expf(xs)
    want = oracle.libm_expf(xs)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.isnan(backend.expf(np.array([np.nan, -np.nan], np.float32))).all()


def upload_experts(backend, w, cols, rows, n_exp):
    return backend.upload(S.T_Q4_K, cols, w, rows=rows, n_mats=n_exp)


def test_moe_matches_golden(backend):
    g = golden("moe.npz")
    E, K, D, F, T = (int(v) for v in g["dims"])
    gate = upload_experts(backend, g["gate"], D, F, E)
    up = upload_experts(backend, g["up"], D, F, E)
    down = upload_experts(backend, g["down"], F, D, E)
    Y, sel, w = backend.moe_ffn(gate, up, down, K, g["logits"], g["X"])
    assert np.array_equal(sel, g["sel"])  # ties on token 2 (experts 3, 7) and token 3 (all equal)
    assert bits_equal(w, g["w"])
    assert bits_equal(Y, g["Y"])
    # one token per call: the launch that routes inside the gate / up matvec
    for i in range(T):
        Y1, sel1, w1 = backend.moe_ffn(gate, up, down, K, g["logits"][i:i + 1], g["X"][i:i + 1])
        assert np.array_equal(sel1, g["sel"][i:i + 1])
        assert bits_equal(w1, g["w"][i:i + 1])
        assert bits_equal(Y1, g["Y"][i:i + 1])
    for t in (gate, up, down):
        t.free()


def test_moe_q5_matches_golden(backend):
    """Q5_K gate / up and a Q5_0 down projection over ff = 160 (a K-quant file's fallback types):
    the generic expert path (decode kernels with an expert index), bit for bit."""
    g = golden("moe_q5.npz")
    E, K, D, F, T = (int(v) for v in g["dims"])
    tg, tu, td = (int(v) for v in g["types"])
    gate = backend.upload(tg, D, g["gate"], rows=F, n_mats=E)
    up = backend.upload(tu, D, g["up"], rows=F, n_mats=E)
    down = backend.upload(td, F, g["down"], rows=D, n_mats=E)
    for n in (1, T):  # one token, and every token in one call
        Y, sel, w = backend.moe_ffn(gate, up, down, K, g["logits"][:n], g["X"][:n])
        assert np.array_equal(sel, g["sel"][:n])
        assert bits_equal(w, g["w"][:n])
        assert bits_equal(Y, g["Y"][:n])
    for t in (gate, up, down):
        t.free()


@pytest.mark.parametrize("types", [(S.T_Q5_K, S.T_Q5_K, S.T_Q5_K), (S.T_Q4_K, S.T_Q4_K, S.T_Q5_0),
                                   (S.T_Q5_0, S.T_Q5_0, S.T_Q6_K), (S.T_Q4_0, S.T_Q4_1, S.T_Q5_1),
                                   (S.T_IQ4_NL, S.T_IQ4_NL, S.T_Q4_1)])
def test_moe_mixed_types_match_oracle(backend, oracle, types):
    # ff = 352 (11 blocks of 32, a last step of 3 blocks) where the down projection takes Q8
    # activations; a K-quant down projection needs ff % 256 == 0
    E, K, D, F, T = 16, 4, 512, 352 if S.uses_q8(types[2]) else 512, 6
    gw = S.random_bytes_weights(types[0], E * F, D, 230)
    uw = S.random_bytes_weights(types[1], E * F, D, 231)
    dw = S.random_bytes_weights(types[2], E * D, F, 232)
    X = S.activations(D, 233, rows=T)
    logits = S.router_logits(T, E, 234)
    Yo, so, wo = oracle.moe_ffn(types, gw, uw, dw, E, K, D, F, logits, X)
    gate = backend.upload(types[0], D, gw, rows=F, n_mats=E)
    up = backend.upload(types[1], D, uw, rows=F, n_mats=E)
    down = backend.upload(types[2], F, dw, rows=D, n_mats=E)
    Y, sel, w = backend.moe_ffn(gate, up, down, K, logits, X)
    assert np.array_equal(sel, so)
    assert bits_equal(w, wo)
    assert bits_equal(Y, Yo)
    for t in (gate, up, down):
        t.free()


@pytest.mark.parametrize("E,K,D,F,T", [(16, 4, 512, 256, 1), (16, 4, 512, 256, 5), (32, 8, 768, 512, 9)])
def test_moe_matches_oracle(backend, oracle, E, K, D, F, T):
    gw = S.random_bytes_weights(S.T_Q4_K, E * F, D, 200 + E)
    uw = S.random_bytes_weights(S.T_Q4_K, E * F, D, 201 + E)
    dw = S.random_bytes_weights(S.T_Q4_K, E * D, F, 202 + E)
    X = S.activations(D, 203 + T, rows=T)
    logits = S.router_logits(T, E, 204 + T)
    Yo, so, wo = oracle.moe_ffn((S.T_Q4_K,) * 3, gw, uw, dw, E, K, D, F, logits, X)
    gate, up, down = (upload_experts(backend, a, c, r, E) for a, c, r in ((gw, D, F), (uw, D, F), (dw, F, D)))
    Y, sel, w = backend.moe_ffn(gate, up, down, K, logits, X)
    assert np.array_equal(sel, so)
    assert bits_equal(w, wo)
    for t in range(T):
        assert rel_err(Y[t], Yo[t]) <= 1e-5
    assert bits_equal(Y, Yo)
    for t in (gate, up, down):
        t.free()


@pytest.mark.parametrize("E,K,T,D,F", [(200, 8, 1, 256, 256), (512, 8, 1, 256, 256), (96, 10, 1, 256, 256),
                                       (70, 1, 1, 256, 256), (200, 8, 3, 256, 256), (32, 4, 1, 2048, 256),
                                       (16, 2, 2, 4096, 512)])
def test_moe_routing_shapes(backend, oracle, E, K, T, D, F):
    """Expert counts that fill several 64-expert slots of a wavefront (and 512, the most), k above
    the 8 experts the fused down launch takes (the separate routing launch), k = 1, and long rows
    over few tiles, where the routing launch splits each tile's blocks over two wavefronts."""
    gw = S.random_bytes_weights(S.T_Q4_K, E * F, D, 400 + E)
    uw = S.random_bytes_weights(S.T_Q4_K, E * F, D, 401 + E)
    dw = S.random_bytes_weights(S.T_Q4_K, E * D, F, 402 + E)
    X = S.activations(D, 403 + K, rows=T)
    logits = S.router_logits(T, E, 404 + K)
    Yo, so, wo = oracle.moe_ffn((S.T_Q4_K,) * 3, gw, uw, dw, E, K, D, F, logits, X)
    gate, up, down = (upload_experts(backend, a, c, r, E) for a, c, r in ((gw, D, F), (uw, D, F), (dw, F, D)))
    Y, sel, w = backend.moe_ffn(gate, up, down, K, logits, X)
    assert np.array_equal(sel, so)
    assert bits_equal(w, wo)
    assert bits_equal(Y, Yo)
    for t in (gate, up, down):
        t.free()


@pytest.mark.parametrize("T", [1, 64])
def test_moe_config5(backend, oracle, T):
    """Benchmark config 5: Qwen3-30B-A3B-shaped layer, 128 experts, top-8, hidden 2048, ff 768."""
    E, K, D, F = 128, 8, 2048, 768
    gw = S.q4_k_weights(E * F, D, seed=300)
    uw = S.q4_k_weights(E * F, D, seed=301)
    dw = S.q4_k_weights(E * D, F, seed=302)
    X = S.activations(D, 303, rows=T)
    logits = S.router_logits(T, E, 304)
    Yo, so, wo = oracle.moe_ffn((S.T_Q4_K,) * 3, gw, uw, dw, E, K, D, F, logits, X)
    gate, up, down = (upload_experts(backend, a, c, r, E) for a, c, r in ((gw, D, F), (uw, D, F), (dw, F, D)))
    Y, sel, w = backend.moe_ffn(gate, up, down, K, logits, X)
    assert np.array_equal(sel, so)
    assert bits_equal(w, wo)
    for t in range(T):
        assert rel_err(Y[t], Yo[t]) <= 1e-5
    assert bits_equal(Y, Yo)
    # repeated call (scratch reuse) gives the same bits
    Y2, _, _ = backend.moe_ffn(gate, up, down, K, logits, X)
    assert bits_equal(Y2, Y)
    for t in (gate, up, down):
        t.free()


def test_moe_grouped_graph_replays(backend, oracle):
    """The several-token path (the slots filed in per-expert buckets whose counts the path's last
    launch clears) captured in a graph: every replay, with eager MoE calls of another expert count
    and token count between them, equals the oracle bit for bit, and so do the eager calls."""
    E, K, D, F, T = 32, 4, 512, 256, 9
    gw = S.random_bytes_weights(S.T_Q4_K, E * F, D, 510)
    uw = S.random_bytes_weights(S.T_Q4_K, E * F, D, 511)
    dw = S.random_bytes_weights(S.T_Q4_K, E * D, F, 512)
    X = S.activations(D, 513, rows=T)
    logits = S.router_logits(T, E, 514)
    Yo, _, _ = oracle.moe_ffn((S.T_Q4_K,) * 3, gw, uw, dw, E, K, D, F, logits, X)
    gate, up, down = (upload_experts(backend, a, c, r, E) for a, c, r in ((gw, D, F), (uw, D, F), (dw, F, D)))
    E2, T2 = 16, 5  # the eager calls between the replays
    gw2 = S.random_bytes_weights(S.T_Q4_K, E2 * F, D, 520)
    uw2 = S.random_bytes_weights(S.T_Q4_K, E2 * F, D, 521)
    dw2 = S.random_bytes_weights(S.T_Q4_K, E2 * D, F, 522)
    X2 = S.activations(D, 523, rows=T2)
    logits2 = S.router_logits(T2, E2, 524)
    Yo2, _, _ = oracle.moe_ffn((S.T_Q4_K,) * 3, gw2, uw2, dw2, E2, K, D, F, logits2, X2)
    g2, u2, d2 = (upload_experts(backend, a, c, r, E2) for a, c, r in ((gw2, D, F), (uw2, D, F), (dw2, F, D)))
    xd, ld, yd = backend.dev_alloc(X.nbytes), backend.dev_alloc(logits.nbytes), backend.dev_alloc(4 * T * D)
    backend.h2d(xd, X)
    backend.h2d(ld, np.ascontiguousarray(logits, np.float32))
    backend.moe_ffn_dev(gate, up, down, K, ld, xd, yd, T)  # eager first: the scratch exists
    backend.sync()
    backend.graph_begin()
    backend.moe_ffn_dev(gate, up, down, K, ld, xd, yd, T)
    g = backend.graph_end()
    for rep in range(3):
        backend.h2d(yd, np.full(T * D, np.nan, np.float32))
        backend.graph_launch(g)
        backend.sync()
        Y = np.empty((T, D), np.float32)
        backend.d2h(Y, yd)
        assert bits_equal(Y, Yo), f"replay {rep}"
        Y2, _, _ = backend.moe_ffn(g2, u2, d2, K, logits2, X2)
        assert bits_equal(Y2, Yo2), f"eager call after replay {rep}"
    backend.graph_destroy(g)
    for p in (xd, ld, yd):
        backend.dev_free(p)
    for t in (gate, up, down, g2, u2, d2):
        t.free()


def _backend_with(env):
    """A second context whose MoE kernel choice comes from the environment at fgh_open."""
    import os

    from fastgguf_amd.backend import Backend
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        return Backend(0)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


@pytest.mark.parametrize("E,K,D,F,T", [(8, 4, 512, 256, 64), (128, 8, 2048, 768, 64), (16, 2, 4096, 512, 33)])
def test_moe_grouped_kernels_match_oracle(backend, oracle, E, K, D, F, T):
    """The grouped path's expert kernels: int8 MFMA (the default) with chunks of 4, 8 and 16 slots,
    ring depths 2, 3 and 4 and other tile counts per wavefront, and the VALU lane chains, each bit
    for bit equal to the oracle. E = 8 at 64 tokens puts about 32 slots on every expert, so every
    chunk size runs several chunks per expert side by side; 128 experts is config 5; 4096 columns
    is 16 blocks per row."""
    gw = S.random_bytes_weights(S.T_Q4_K, E * F, D, 600 + E)
    uw = S.random_bytes_weights(S.T_Q4_K, E * F, D, 601 + E)
    dw = S.random_bytes_weights(S.T_Q4_K, E * D, F, 602 + E)
    X = S.activations(D, 603 + T, rows=T)
    logits = S.router_logits(T, E, 604 + T)
    Yo, so, wo = oracle.moe_ffn((S.T_Q4_K,) * 3, gw, uw, dw, E, K, D, F, logits, X)
    for env in ({}, {"FGH_MOE_NSG": "1"}, {"FGH_MOE_NSG": "4"}, {"FGH_MOE_R": "2"}, {"FGH_MOE_R": "4", "FGH_MOE_TT": "1"},
                {"FGH_MOE_NSG": "1", "FGH_MOE_R": "4", "FGH_MOE_TT": "3"}, {"FGH_MOE_KERNEL": "valu"}):
        be = backend if not env else _backend_with(env)
        try:
            gate, up, down = (upload_experts(be, a, c, r, E) for a, c, r in ((gw, D, F), (uw, D, F), (dw, F, D)))
            Y, sel, w = be.moe_ffn(gate, up, down, K, logits, X)
            assert np.array_equal(sel, so), env
            assert bits_equal(w, wo), env
            assert bits_equal(Y, Yo), env
            for t in (gate, up, down):
                t.free()
        finally:
            if be is not backend:
                be.close()


def test_moe_grouped_block_ints_match_oracle(backend, oracle):
    """The MFMA expert kernels' per (slot, row, block) integers: gate's against the oracle's
    integers of the selected expert's rows and Q8_K(x_t), down's against those of Q8_K(h), h the
    oracle's silu(g) * u (bit-identical to the device's)."""
    E, K, D, F, T = 16, 4, 512, 256, 12
    gw = S.random_bytes_weights(S.T_Q4_K, E * F, D, 700)
    uw = S.random_bytes_weights(S.T_Q4_K, E * F, D, 701)
    dw = S.random_bytes_weights(S.T_Q4_K, E * D, F, 702)
    X = S.activations(D, 703, rows=T)
    logits = S.router_logits(T, E, 704)
    Yo, so, wo, ho = oracle.moe_ffn((S.T_Q4_K,) * 3, gw, uw, dw, E, K, D, F, logits, X, want_h=True)
    gate, up, down = (upload_experts(backend, a, c, r, E) for a, c, r in ((gw, D, F), (uw, D, F), (dw, F, D)))
    gs, gm, ds, dm = backend.moe_block_ints(gate, up, down, K, logits, X)
    rbg, rbd = S.row_bytes(S.T_Q4_K, D), S.row_bytes(S.T_Q4_K, F)
    gw2, dw2 = gw.reshape(E * F, rbg), dw.reshape(E * D, rbd)
    for t in range(T):
        ax = oracle.quantize_q8k(X[t])
        for j in range(K):
            e, slot = int(so[t, j]), t * K + j
            ah = oracle.quantize_q8k(ho[t, j])
            for r in range(F):
                s, m = oracle.block_ints(S.T_Q4_K, gw2[e * F + r], ax)
                assert np.array_equal(gs[slot, r], s) and np.array_equal(gm[slot, r], m), (t, j, r)
            for r in range(D):
                s, m = oracle.block_ints(S.T_Q4_K, dw2[e * D + r], ah)
                assert np.array_equal(ds[slot, r], s) and np.array_equal(dm[slot, r], m), (t, j, r)
    for t_ in (gate, up, down):
        t_.free()


def test_moe_grouped_nonfinite_logits(backend, oracle):
    """Tokens whose router probabilities are not all finite pick one expert several times, as the
    reference's repeated argmax does (a picked probability becomes -1 and stays a candidate): one
    token with only two finite logits for k = 4, one all NaN, one with +inf. The other tokens of the
    same batch keep their results bit for bit (each expert's bucket holds every slot of the call),
    and the next call starts from cleared counts."""
    E, K, D, F, T = 16, 4, 512, 256, 8
    gw = S.random_bytes_weights(S.T_Q4_K, E * F, D, 710)
    uw = S.random_bytes_weights(S.T_Q4_K, E * F, D, 711)
    dw = S.random_bytes_weights(S.T_Q4_K, E * D, F, 712)
    X = S.activations(D, 713, rows=T)
    logits = S.router_logits(T, E, 714)
    logits[2, 2:] = np.nan
    logits[4, :] = np.nan
    logits[6, 5] = np.inf
    Yo, so, wo = oracle.moe_ffn((S.T_Q4_K,) * 3, gw, uw, dw, E, K, D, F, logits, X)
    gate, up, down = (upload_experts(backend, a, c, r, E) for a, c, r in ((gw, D, F), (uw, D, F), (dw, F, D)))
    for rep in range(2):
        Y, sel, w = backend.moe_ffn(gate, up, down, K, logits, X)
        assert np.array_equal(sel, so), rep
        assert np.array_equal(np.isnan(w), np.isnan(wo)) and bits_equal(np.nan_to_num(w), np.nan_to_num(wo)), rep
        assert np.array_equal(np.isnan(Y), np.isnan(Yo)), rep
        assert bits_equal(np.where(np.isnan(Y), 0, Y), np.where(np.isnan(Yo), 0, Yo)), rep
    assert (so[2, 2:] == so[2, 1]).all() or len(set(so[2])) < K  # the duplicate picks happened
    for t_ in (gate, up, down):
        t_.free()
