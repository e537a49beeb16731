"""Pins the CPU oracle (oracle/fg_oracle.c) before it is trusted as the GPU parity checker.

* golden vectors written by the reference's own compiled kernels (tests/golden/make_golden.py):
  the restatement must reproduce them bit for bit;
* what the mathematics fixes independently of the reference code: quantizer special cases and
  invariants, integer block sums against brute force over independently decoded codes
  (numpy, from the byte layouts), and the dequantized-float relation of the reference selftest;
* the reference selftest's relations between kernels (batch GEMM vs single kernel, repacked vs
  row kernel: rel < 1e-5, fastgguf.c:5690-5785);
* planted mistakes: the oracle rebuilt with one mistake (FGO_MUTATE) must fail the golden vectors.
"""
import os
import subprocess

import numpy as np
import pytest
from conftest import ROOT, bits_equal, golden, rel_err

from fastgguf_amd import synth as S
from oracle import ORDER_REPACKED, ORDER_ROW, Oracle, Reference

TYPES = {"q8_0": S.T_Q8_0, "q4_k": S.T_Q4_K, "q6_k": S.T_Q6_K, "q5_0": S.T_Q5_0, "q5_k": S.T_Q5_K,
         "q4_0": S.T_Q4_0, "q4_1": S.T_Q4_1, "q5_1": S.T_Q5_1, "iq4_nl": S.T_IQ4_NL}
ALL = list(TYPES.values())
LOWBIT = {"q2_k": S.T_Q2_K, "q3_k": S.T_Q3_K, "iq4_xs": S.T_IQ4_XS}
FLOAT = {"f32": S.T_F32, "f16": S.T_F16, "bf16": S.T_BF16}
REPACKABLE = (S.T_Q4_K, S.T_Q4_0)  # the types the reference repacks (repack_tensor, fastgguf.c:2486)


# ---------------------------------------------------------------- golden vectors (reference)

def test_quantizers_match_golden(oracle):
    g = golden("quantize.npz")
    for r, x in enumerate(g["quant_x"]):
        assert oracle.quantize_q8(x).view(np.uint8).tobytes() == g["quant_q8"][r].tobytes(), f"q8 row {r}"
        assert oracle.quantize_q8k(x).view(np.uint8).tobytes() == g["quant_q8k"][r].tobytes(), f"q8k row {r}"


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("gen", ["synth", "bytes"])
def test_matvec_matches_golden(oracle, name, gen):
    g = golden("matvec.npz")
    t = TYPES[name]
    w, x = g[f"{name}_{gen}_w"], g[f"{name}_{gen}_x"]
    cols = x.size
    assert bits_equal(oracle.matvec(t, w, cols, x, ORDER_ROW), g[f"{name}_{gen}_y"])
    if t in REPACKABLE:
        assert bits_equal(oracle.matvec(t, w, cols, x, ORDER_REPACKED), g[f"{name}_{gen}_y_rp"])


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("nb", [3, 8, 45])
def test_matmul_matches_golden(oracle, name, nb):
    g = golden("matmul.npz")
    t = TYPES[name]
    w, X = g[f"{name}_w"], g[f"{name}_X{nb}"]
    cols = X.shape[1]
    assert bits_equal(oracle.matmul(t, w, cols, X, ORDER_ROW), g[f"{name}_Y{nb}"])
    if t in REPACKABLE:
        assert bits_equal(oracle.matmul(t, w, cols, X, ORDER_REPACKED), g[f"{name}_Y{nb}_rp"])


def test_moe_matches_golden(oracle):
    g = golden("moe.npz")
    E, K, D, F, T = (int(v) for v in g["dims"])
    Y, sel, w = oracle.moe_ffn((S.T_Q4_K,) * 3, g["gate"], g["up"], g["down"], E, K, D, F, g["logits"], g["X"])
    assert np.array_equal(sel, g["sel"])
    assert bits_equal(w, g["w"])
    assert bits_equal(Y, g["Y"])
    assert list(g["sel"][2][:2]) == [3, 7]      # tie on top keeps the lower index first
    assert list(g["sel"][3]) == [0, 1, 2]       # all-equal logits


def test_moe_q5_matches_golden(oracle):
    """Q5_K gate / up with a Q5_0 down projection over ff = 160 (a K-quant file's fallback types)."""
    g = golden("moe_q5.npz")
    E, K, D, F, T = (int(v) for v in g["dims"])
    types = tuple(int(v) for v in g["types"])
    assert types == (S.T_Q5_K, S.T_Q5_K, S.T_Q5_0)
    Y, sel, w = oracle.moe_ffn(types, g["gate"], g["up"], g["down"], E, K, D, F, g["logits"], g["X"])
    assert np.array_equal(sel, g["sel"])
    assert bits_equal(w, g["w"])
    assert bits_equal(Y, g["Y"])


# expf inputs where a separately rounded r = x N / ln 2 - k gives another float than glibc's
# fused evaluation (found by sweeping every float); and special values
EXPF_HARD = [float.fromhex("0x1.04845ep+5"), float.fromhex("-0x1.f8cbb2p+5")]
EXPF_SPECIAL = [0.0, -0.0, 1.0, -1.0, 88.72283, 88.72284, 100.0, -87.33654, -103.97207, -103.97208, -150.0,
                float("inf"), float("-inf"), 1e-30, -1e-30, 127.99999, 128.0, -128.0, -127.99999, 200.0,
                -200.0, 1e30, -1e30]


def test_expf_restatement_matches_libm(oracle):
    """The MoE's expf, restated from its published method and run by the GPU: equal to this host's
    libm expf on every 31st float bit pattern (the full sweep of all 2^32 also passes), on the two
    inputs that only the fused evaluation rounds right, and on special values."""
    bad, n, max_ulp = oracle.expf_compare(float("-inf"), float("inf"), 31)
    assert n > 130_000_000
    assert bad == 0, f"{bad} of {n} differ (max {max_ulp} ulp)"
    xs = np.array(EXPF_HARD + EXPF_SPECIAL, np.float32)
    want = oracle.libm_expf(xs)
    got = np.array([oracle.expf(float(x)) for x in xs], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_oracle_matches_compiled_reference_random(oracle, reference):
    """Fresh random shapes and seeds against the reference's kernels (where oracle/_ref is built)."""
    rng = np.random.Generator(np.random.PCG64(7))
    for case in range(18):
        t = ALL[case % len(ALL)]
        cols = int(rng.integers(1, 5)) * 256
        rows = 8 * int(rng.integers(1, 5))
        w = (S.weights if case % 2 else S.random_bytes_weights)(t, rows, cols, 1000 + case)
        x = S.activations(cols, 2000 + case)
        assert bits_equal(oracle.matvec(t, w, cols, x), reference.matvec(t, w, cols, x))
        if t in REPACKABLE:
            assert bits_equal(oracle.matvec(t, w, cols, x, ORDER_REPACKED), reference.matvec(t, w, cols, x, True))
        nb = int(rng.integers(8, 20))
        X = S.activations(cols, 3000 + case, rows=nb)
        if reference.variant == "vnni" or t != S.T_Q8_0:  # AVX2 builds have no Q8_0 GEMM
            assert bits_equal(oracle.matmul(t, w, cols, X), reference.matmul(t, w, cols, X))
        if S.uses_q8(t):  # rows of 32-blocks that are not 256-multiples (a tail step of 1..3 blocks)
            c2 = 32 * int(rng.integers(1, 40))
            w2 = S.weights(t, rows, c2, 4000 + case)
            x2 = S.activations(c2, 5000 + case)
            assert bits_equal(oracle.matvec(t, w2, c2, x2), reference.matvec(t, w2, c2, x2))


# ---------------------------------------------------------------- what the mathematics fixes

def test_quantizer_invariants(oracle):
    x = S.activations(4096, 11)
    x[:256] = 0.0
    for blocks, bsz, sums in ((oracle.quantize_q8k(x), 256, "bsums"), (oracle.quantize_q8(x), 32, "s16")):
        xb = x[: blocks.size * bsz].reshape(blocks.size, bsz)
        amax = np.abs(xb).max(axis=1)
        # d is the IEEE quotient amax / 127 (numpy float32 division is correctly rounded)
        assert np.array_equal(blocks["d"], (amax / np.float32(127)).astype(np.float32))
        q = blocks["qs"].astype(np.int32)
        assert np.abs(q).max() <= 127
        nz = amax > 0
        # the largest magnitude maps to +-127 exactly
        assert np.all(np.abs(q[nz]).max(axis=1) == 127)
        assert np.all(q[~nz] == 0) and np.all(blocks["d"][~nz] == 0)
        # sums of every 16 quants
        s = q.reshape(blocks.size, -1, 16).sum(axis=2)
        assert np.array_equal(blocks[sums].astype(np.int32), s)
        # dequantized values within half a step of x
        err = np.abs(q * blocks["d"][:, None] - xb)
        assert np.all(err <= blocks["d"][:, None] * 0.5 * (1 + 1e-5) + 1e-30)
    # a tail shorter than a block is ignored (n / 32, n / 256)
    assert oracle.quantize_q8(x[:63]).size == 1 and oracle.quantize_q8k(x[:511]).size == 1


def test_quantizer_rounds_half_to_even(oracle):
    # amax = 127 -> d = 1, id = 1: x * id = x exactly, so the .5 cases must round to even
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, 126.5]
    q = oracle.quantize_q8(x)["qs"][0][:9]
    assert list(q) == [127, 0, 2, 2, 0, -2, -2, 4, 126]


def _decode_codes(t, w_row, cols):
    """Independent numpy decode of one row into (integer codes, integer scale per element,
    integer min per element, block index); from the byte layouts, not from the oracle."""
    nb = cols // S.BLOCK[t][0]
    blk = w_row.reshape(nb, S.BLOCK[t][1])
    if t == S.T_Q8_0:
        q = blk[:, 2:34].view(np.int8).astype(np.int64).reshape(-1)
        return q, np.ones_like(q), np.zeros_like(q)
    if t in (S.T_Q5_0, S.T_Q5_1, S.T_Q4_0, S.T_Q4_1, S.T_IQ4_NL):
        # element j: nibble j of qs (low nibbles, then high), with bit j of qh as bit 4 (Q5)
        qoff = {S.T_Q5_0: 6, S.T_Q5_1: 8, S.T_Q4_0: 2, S.T_Q4_1: 4, S.T_IQ4_NL: 2}[t]
        qs = blk[:, qoff:qoff + 16].astype(np.int64)
        q = np.concatenate([qs & 15, qs >> 4], axis=1)
        if t in (S.T_Q5_0, S.T_Q5_1):
            h = 2 if t == S.T_Q5_0 else 4
            qh = blk[:, h:h + 4].copy().view("<u4").astype(np.int64)  # [nb, 1]
            q = q | (((qh >> np.arange(32)) & 1) << 4)
        if t == S.T_IQ4_NL:  # the published IQ4_NL values (llama.cpp's kvalues_iq4nl)
            q = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113])[q]
        q = q - {S.T_Q5_0: 16, S.T_Q4_0: 8}.get(t, 0)
        return q.reshape(-1), np.ones(nb * 32, np.int64), np.zeros(nb * 32, np.int64)
    if t in (S.T_Q4_K, S.T_Q5_K):
        s12 = blk[:, 4:16].astype(np.int64)
        sc = np.zeros((nb, 8), np.int64)
        mn = np.zeros((nb, 8), np.int64)
        for j in range(4):
            sc[:, j] = s12[:, j] & 63
            mn[:, j] = s12[:, j + 4] & 63
            sc[:, j + 4] = (s12[:, j + 8] & 15) | ((s12[:, j] >> 6) << 4)
            mn[:, j + 4] = (s12[:, j + 8] >> 4) | ((s12[:, j + 4] >> 6) << 4)
        qs = blk[:, 16:144] if t == S.T_Q4_K else blk[:, 48:176]
        qs = qs.astype(np.int64).reshape(nb, 4, 32)
        q = np.stack([qs & 15, qs >> 4], axis=2)  # [nb][j][lo/hi][32]
        if t == S.T_Q5_K:  # chunk j, half h: bit 2j + h of qh[l] is bit 4 of element l
            qh = blk[:, 16:48].astype(np.int64)
            for j in range(4):
                for h in range(2):
                    q[:, j, h] |= ((qh >> (2 * j + h)) & 1) << 4
        q = q.reshape(nb, 256)
        sub = np.arange(256) // 32
        return q.reshape(-1), sc[:, sub].reshape(-1), mn[:, sub].reshape(-1)
    ql = blk[:, 0:128].astype(np.int64).reshape(nb, 2, 64)
    qh = blk[:, 128:192].astype(np.int64).reshape(nb, 2, 32)
    sc = blk[:, 192:208].view(np.int8).astype(np.int64)
    q = np.zeros((nb, 2, 4, 32), np.int64)
    q[:, :, 0] = (ql[:, :, :32] & 15) | ((qh & 3) << 4)
    q[:, :, 1] = (ql[:, :, 32:] & 15) | (((qh >> 2) & 3) << 4)
    q[:, :, 2] = (ql[:, :, :32] >> 4) | (((qh >> 4) & 3) << 4)
    q[:, :, 3] = (ql[:, :, 32:] >> 4) | (((qh >> 6) & 3) << 4)
    return q.reshape(-1), sc[:, np.arange(256) // 16].reshape(-1), np.zeros(nb * 256, np.int64)


@pytest.mark.parametrize("t", ALL)
def test_block_ints_brute_force(oracle, t):
    cols = 1024
    w = S.random_bytes_weights(t, 4, cols, 77)
    x = S.activations(cols, 78)
    act = oracle.quantize_for(t, x)
    y = act["qs"].astype(np.int64).reshape(-1)
    bsz = S.BLOCK[t][0]
    for r in range(4):
        q, sc, mn = _decode_codes(t, w[r], cols)
        s, m = oracle.block_ints(t, w[r], act)
        if t == S.T_Q6_K:
            want_s = (sc * q * y).reshape(-1, bsz).sum(1)
            want_m = (sc * y).reshape(-1, bsz).sum(1)
        else:
            want_s = (sc * q * y).reshape(-1, bsz).sum(1)
            want_m = (mn * y).reshape(-1, bsz).sum(1)
        assert np.array_equal(s, want_s) and np.array_equal(m, want_m)


@pytest.mark.parametrize("t", ALL)
def test_dot_vs_dequantized_double(oracle, t):
    """test_kquant (fastgguf.c:5379-5411): kernel vs double sum of dequantized weights times
    dequantized activations, relative to sum |term| < 1e-4."""
    n = 1024
    for seed in range(4):
        w = S.random_bytes_weights(t, 1, n, 90 + seed)[0]
        x = S.activations(n, 95 + seed) * 2.0
        act = oracle.quantize_for(t, x)
        fast = oracle.dot(t, w, act)
        dq = oracle.dequantize_row(t, w, n).astype(np.float64)
        xd = (act["qs"].astype(np.float64) * act["d"][:, None].astype(np.float64)).reshape(-1)
        terms = dq * xd
        assert abs(fast - terms.sum()) / (np.abs(terms).sum() + 1e-9) < 1e-4


@pytest.mark.parametrize("t", ALL)
def test_selftest_relations(oracle, t):
    """matmul vs the single-row kernel and repacked vs row (fastgguf.c:5690-5785): < 1e-5."""
    cols, rows, nbt = 512, 37, 45
    w = S.random_bytes_weights(t, rows, cols, 55)
    X = S.activations(cols, 56, rows=nbt)
    Y = oracle.matmul(t, w, cols, X)
    for b in range(nbt):
        act = oracle.quantize_for(t, X[b])
        ref = np.array([oracle.dot(t, w[r], act) for r in range(rows)], np.float32)
        assert rel_err(Y[b], ref) < 1e-5
    if t in REPACKABLE:
        w = S.random_bytes_weights(t, 16, 768, 57)
        x = S.activations(768, 58)
        assert rel_err(oracle.matvec(t, w, 768, x, ORDER_REPACKED), oracle.matvec(t, w, 768, x, ORDER_ROW)) < 1e-5


# ---------------------------------------------------------------- planted mistakes

MUTANTS = {1: "hsum8 order", 2: "MoE accumulate without fma", 3: "reciprocal instead of division",
           4: "Q6_K half-lane scale", 5: "Q4_K repacked single chain", 6: "Q4_K GEMM integer epilogue",
           7: "Q5_0 fifth bit from the wrong half of qh", 8: "Q5_K qh bit pairing",
           9: "Q4_1 / Q5_1 min term without the fused multiply-add",
           10: "attention score lanes added in sequence", 11: "softmax tail through exp_neg_ps",
           12: "TurboQuant key dot without the contraction", 13: "TurboQuant scale from an fma chain",
           14: "per-row attention score tail without the contraction",
           15: "Q2_K chain without gcc's contractions", 16: "Q3_K hmask bit of the other half",
           17: "IQ4_XS high scale bits at the wrong shift", 18: "F16 row in dot_f32v's two accumulators",
           19: "BF16 chain without the contraction"}


@pytest.fixture(scope="module")
def mutant_dir(tmp_path_factory):
    return tmp_path_factory.mktemp("mutants")


def _golden_failures(o: Oracle) -> int:
    fails = 0
    g = golden("quantize.npz")
    for r, x in enumerate(g["quant_x"]):
        fails += o.quantize_q8(x).view(np.uint8).tobytes() != g["quant_q8"][r].tobytes()
    g = golden("matvec.npz")
    for name, t in TYPES.items():
        for gen in ("synth", "bytes"):
            x = g[f"{name}_{gen}_x"]
            fails += not bits_equal(o.matvec(t, g[f"{name}_{gen}_w"], x.size, x), g[f"{name}_{gen}_y"])
            if t in REPACKABLE:
                fails += not bits_equal(o.matvec(t, g[f"{name}_{gen}_w"], x.size, x, ORDER_REPACKED),
                                        g[f"{name}_{gen}_y_rp"])
    g = golden("matmul.npz")
    for name, t in TYPES.items():
        X = g[f"{name}_X45"]
        fails += not bits_equal(o.matmul(t, g[f"{name}_w"], X.shape[1], X), g[f"{name}_Y45"])
    g = golden("moe.npz")
    E, K, D, F, T = (int(v) for v in g["dims"])
    Y, _, _ = o.moe_ffn((S.T_Q4_K,) * 3, g["gate"], g["up"], g["down"], E, K, D, F, g["logits"], g["X"])
    fails += not bits_equal(Y, g["Y"])
    g = golden("moe_q5.npz")
    E, K, D, F, T = (int(v) for v in g["dims"])
    Y, _, _ = o.moe_ffn(tuple(int(v) for v in g["types"]), g["gate"], g["up"], g["down"], E, K, D, F,
                        g["logits"], g["X"])
    fails += not bits_equal(Y, g["Y"])
    for c in attn_golden():
        fails += not bits_equal(o.attn_rows(c["q"], c["st"], c["en"], c["ck"], c["cv"], [c["kvo"]] * len(c["st"]),
                                            c["hd"], c["scale"]), c["o"])
    fails += kvq_golden_failures(o)
    g = golden("lowbit.npz")
    for name, t in LOWBIT.items():
        for gen in ("synth", "bytes"):
            x = g[f"{name}_{gen}_x"]
            fails += not bits_equal(o.matvec(t, g[f"{name}_{gen}_w"], x.size, x), g[f"{name}_{gen}_y"])
    g = golden("float.npz")
    for name, t in FLOAT.items():
        for gen in ("synth", "bytes"):
            for cols in (3, 100, 1024):
                x = g[f"{name}_{gen}_{cols}_x"]
                fails += not bits_equal(o.matvec(t, g[f"{name}_{gen}_{cols}_w"], cols, x), g[f"{name}_{gen}_{cols}_y"])
    return fails


def kvq_attn_golden() -> list[dict]:
    g = golden("kvq.npz")
    out = []
    for i in range(int(g["n_attn"][0])):
        hd, nkv, kb, vb = (int(v) for v in g[f"a{i}_meta"])
        out.append(dict(q=g[f"a{i}_q"], kq=g[f"a{i}_kq"], vq=g[f"a{i}_vq"], st=g[f"a{i}_st"], en=g[f"a{i}_en"],
                        kvh=g[f"a{i}_kvh"], o=g[f"a{i}_o"], hd=hd, nkv=nkv, kbits=kb, vbits=vb,
                        scale=float(g[f"a{i}_scale"][0])))
    return out


def kvq_golden_failures(o: Oracle) -> int:
    g = golden("kvq.npz")
    fails = int(not np.array_equal(o.kvq_signs(1024), g["signs"].astype(np.float32)))
    for hd in (64, 128, 256):
        fails += not bits_equal(o.kvq_rotate(g[f"rot{hd}_x"]), g[f"rot{hd}_y"])
        fails += not bits_equal(o.kvq_rotate(g[f"rot{hd}_x"], inverse=True), g[f"rot{hd}_inv"])
    for bits in (8, 4, 2):
        for x, rec in zip(g["quant_x"], g[f"quant_rec{bits}"]):
            fails += not np.array_equal(o.kvq_quant(x, bits), rec)
    for c in kvq_attn_golden():
        fails += not bits_equal(o.kvq_attn_rows(c["q"], c["st"], c["en"], c["kq"], c["vq"], c["kvh"], c["hd"],
                                                c["kbits"], c["vbits"], c["scale"]), c["o"])
    return fails


def test_kvq_golden(oracle):
    """TurboQuant restated (signs, rotation, slice records, attention step), bit for bit against
    the compiled reference's outputs."""
    assert kvq_golden_failures(oracle) == 0


def test_kvq_against_the_mathematics(oracle):
    """The reference's own selftest relations (fastgguf.c:6035-6105) and what the mathematics
    fixes: the rotation is orthogonal (norms and dot products kept, the inverse undoes it within
    1e-5), the signs are +-1, K4 / V2 / K8 reconstruction errors stay within the selftest's
    bounds (0.15 / 0.45 / 0.01), and a record decodes to the scale times the centroid of each code."""
    rng = np.random.default_rng(21)
    assert set(np.unique(oracle.kvq_signs(1024))) == {-1.0, 1.0}
    for hd in (32, 128, 1024):
        x, y = (rng.standard_normal(hd).astype(np.float32) for _ in range(2))
        rx, ry = oracle.kvq_rotate(x), oracle.kvq_rotate(y)
        assert abs(np.linalg.norm(rx) - np.linalg.norm(x)) < 1e-5 * np.linalg.norm(x)
        assert abs(float(rx @ ry) - float(x @ y)) < 1e-4 * np.linalg.norm(x) * np.linalg.norm(y)
        back = oracle.kvq_rotate(rx, inverse=True)
        assert np.linalg.norm(back - x) < 1e-5 * np.linalg.norm(x)
        # one basis vector: R e_j = sign_j * (column j of H) / sqrt(n), every entry +-1/sqrt(n)
        e = np.zeros(hd, np.float32)
        e[3] = 1.0
        assert np.allclose(np.abs(oracle.kvq_rotate(e)), 1 / np.sqrt(hd), rtol=1e-6)
    c4 = np.array([-2.7326, -2.0690, -1.6181, -1.2562, -0.9424, -0.6568, -0.3881, -0.1284,
                   0.1284, 0.3881, 0.6568, 0.9424, 1.2562, 1.6181, 2.0690, 2.7326], np.float32)
    c2 = np.array([-1.5104, -0.4528, 0.4528, 1.5104], np.float32)
    for bits, bound in ((4, 0.15), (2, 0.45), (8, 0.01)):
        x = oracle.kvq_rotate(rng.standard_normal(128).astype(np.float32))
        rec = oracle.kvq_quant(x, bits)
        s = rec[:4].view(np.float32)[0]
        q = rec[4:]
        if bits == 8:
            dq = s * q.view(np.int8).astype(np.float32)
        elif bits == 4:
            dq = s * c4[np.stack([q & 15, q >> 4], 1).reshape(-1)]
        else:
            dq = s * c2[np.stack([(q >> (2 * k)) & 3 for k in range(4)], 1).reshape(-1)]
            # every code is the nearest centroid of x / s
            assert np.all(np.abs(x / s - dq / s) <= np.min(np.abs((x / s)[:, None] - c2[None, :]), 1) + 1e-6)
        assert np.linalg.norm(dq - x) / np.linalg.norm(x) < bound


def test_fp16_against_numpy_exhaustive(oracle):
    """fgo_fp16 (the reference's FP16() table, fastgguf.c:94-122) against numpy's IEEE half ->
    float over all 65536 codes: normals, subnormals, signed zeros, infinities and NaNs (any NaN
    code gives a NaN; the others must match bit for bit)."""
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([oracle.lib.fgo_fp16(int(v)) for v in h], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def attn_golden() -> list[dict]:
    g = golden("attn.npz")
    out = []
    for i in range(int(g["n_cases"][0])):
        hd, kvo = (int(v) for v in g[f"c{i}_meta"])
        out.append(dict(q=g[f"c{i}_q"], ck=g[f"c{i}_ck"], cv=g[f"c{i}_cv"], st=g[f"c{i}_st"], en=g[f"c{i}_en"],
                        o=g[f"c{i}_o"], hd=hd, kvo=kvo, scale=float(g[f"c{i}_scale"][0])))
    return out


def test_attention_golden(oracle):
    """attn_rows restated, bit for bit against the compiled reference's outputs."""
    for c in attn_golden():
        o = oracle.attn_rows(c["q"], c["st"], c["en"], c["ck"], c["cv"], [c["kvo"]] * len(c["st"]), c["hd"],
                             c["scale"])
        assert bits_equal(o, c["o"])


def test_exp_neg_against_the_mathematics(oracle):
    """exp_neg_ps restated: exactly 1 at 0, exactly 0 at and below -87, within 3e-7 relative of
    e^x (float64) over (-87, 0], and never above 1."""
    x = np.concatenate([-np.logspace(-8, np.log10(86.999), 20000), -np.linspace(0, 86.99, 20000)]).astype(np.float32)
    e = np.array([oracle.exp_neg(v) for v in x[::7]], np.float64)
    ref = np.exp(x[::7].astype(np.float64))
    assert np.max(np.abs(e - ref) / ref) < 3e-7
    assert oracle.exp_neg(0.0) == 1.0 and oracle.exp_neg(-87.0) == 0.0 and oracle.exp_neg(-1000.0) == 0.0
    assert np.all(e <= 1.0)


def test_attention_against_float64(oracle):
    """The restated attention is softmax(q k^T * scale) v within fp32 rounding (float64 math),
    per row, with GQA head offsets and ring wrap."""
    rng = np.random.default_rng(5)
    hd, kv_dim, cap = 64, 256, 50
    ck = rng.standard_normal((cap, kv_dim)).astype(np.float32)
    cv = rng.standard_normal((cap, kv_dim)).astype(np.float32)
    q = rng.standard_normal((6, hd)).astype(np.float32)
    st, en, kvo = [0, 10, 40, 45, 3, 20], [0, 17, 70, 94, 52, 20], [0, 64, 128, 192, 64, 0]
    o = oracle.attn_rows(q, st, en, ck, cv, kvo, hd, 0.125)
    for r in range(6):
        pos = np.arange(st[r], en[r] + 1) % cap
        k = ck[pos, kvo[r]:kvo[r] + hd].astype(np.float64)
        v = cv[pos, kvo[r]:kvo[r] + hd].astype(np.float64)
        s = k @ q[r].astype(np.float64) * 0.125
        w = np.exp(s - s.max())
        ref = (w / w.sum()) @ v
        assert np.max(np.abs(o[r] - ref)) < 1e-5 * max(1.0, np.abs(ref).max())


def test_attention_matches_compiled_reference(oracle):
    """Random cases against the compiled reference (where it is built): 4-row calls sharing a
    head offset, ranges of every length mod 8, ring wrap, hd 32 .. 256."""
    try:
        ref = Reference()
    except (OSError, FileNotFoundError):
        pytest.skip("reference build absent")
    rng = np.random.default_rng(9)
    for case in range(24):
        hd = int(rng.choice([32, 64, 96, 128, 256]))
        cap = int(rng.integers(8, 80))
        kv_dim = hd * int(rng.integers(1, 3))
        kvo = int(rng.integers(0, kv_dim // hd)) * hd
        nr = int(rng.integers(1, 5))
        st = rng.integers(0, 200, nr)
        en = st + rng.integers(0, cap, nr)
        ck = rng.standard_normal((cap, kv_dim)).astype(np.float32)
        cv = rng.standard_normal((cap, kv_dim)).astype(np.float32)
        q = (rng.standard_normal((nr, hd)) * (1 + 10 * (case % 3 == 2))).astype(np.float32)
        scale = float(np.float32(1 / np.sqrt(hd)))
        a = ref.attn_rows(q, st, en, ck, cv, kvo, hd, scale)
        b = oracle.attn_rows(q, st, en, ck, cv, [kvo] * nr, hd, scale)
        assert bits_equal(a, b), (case, hd, cap, st, en)


@pytest.mark.parametrize("mutant", sorted(MUTANTS))
def test_planted_mistake_is_caught(mutant, mutant_dir):
    so = os.path.join(str(mutant_dir), f"liboracle_m{mutant}.so")
    src = os.path.join(ROOT, "oracle", "fg_oracle.c")
    subprocess.run(["gcc", "-O2", "-march=x86-64-v3", "-ffp-contract=off", "-fPIC", "-fopenmp", "-std=c11",
                    f"-DFGO_MUTATE={mutant}", "-shared", "-o", so, src, "-lm"], check=True)
    assert _golden_failures(Oracle(so)) > 0, f"golden vectors did not catch: {MUTANTS[mutant]}"


def test_real_oracle_passes_golden_check(oracle):
    assert _golden_failures(oracle) == 0
