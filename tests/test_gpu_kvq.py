"""GPU parity of the TurboQuant KV cache (fastgguf.c:3341-3513; forward's cache write 4726-4735
and attention step 4760-4846) through the C ABI.

Records and outputs are compared bit for bit: records written on the device against the
oracle's rotation + slice quantizer (pinned to the compiled reference), the attention step
against the reference's golden outputs and against the oracle on decode and prompt-batch ranges,
GQA head groups, ring wrap, hd 32 .. 256 and every K / V bit width.
"""
import numpy as np
import pytest
from conftest import bits_equal

from fastgguf_amd.backend import BackendError

pytestmark = pytest.mark.gpu


def rec_bytes(hd, bits):
    return 4 + hd * bits // 8


def oracle_cache(oracle, k, v, pos, cap, kbits, vbits):
    """Caches written by the oracle: rows k / v [n][n_kv][hd] at positions pos."""
    n, nkv, hd = k.shape
    kq = np.zeros((cap, nkv * rec_bytes(hd, kbits)), np.uint8)
    vq = np.zeros((cap, nkv * rec_bytes(hd, vbits)), np.uint8)
    for t in range(n):
        for h in range(nkv):
            rk, rv = rec_bytes(hd, kbits), rec_bytes(hd, vbits)
            kq[pos[t] % cap, h * rk:(h + 1) * rk] = oracle.kvq_quant(oracle.kvq_rotate(k[t, h]), kbits)
            vq[pos[t] % cap, h * rv:(h + 1) * rv] = oracle.kvq_quant(oracle.kvq_rotate(v[t, h]), vbits)
    return kq, vq


def oracle_attention(oracle, q, kq, vq, st, en, n_kv, kbits, vbits, scale):
    n_tok, n_head, hd = q.shape
    g = n_head // n_kv
    kvh = np.tile(np.arange(n_head) // g, n_tok)
    return oracle.kvq_attn_rows(q.reshape(-1, hd), np.repeat(st, n_head), np.repeat(en, n_head), kq, vq, kvh, hd,
                                kbits, vbits, scale).reshape(q.shape)


@pytest.mark.parametrize("hd,kbits,vbits", [(32, 4, 4), (64, 8, 4), (128, 4, 2), (256, 8, 8), (128, 4, 4)])
def test_store_matches_oracle(backend, oracle, hd, kbits, vbits):
    rng = np.random.default_rng(hd + kbits + vbits)
    nkv, cap, n = 3, 20, 7
    k = (rng.standard_normal((n, nkv, hd)) * rng.uniform(0.01, 50, (n, nkv, 1))).astype(np.float32)
    v = (rng.standard_normal((n, nkv, hd)) * rng.uniform(0.01, 50, (n, nkv, 1))).astype(np.float32)
    k[0, 0] = 0.0  # a zero slice: scale 0, every code the one for 0
    pos = np.array([0, 1, 5, 19, 20, 33, 58], np.int32)  # slots 0, 1, 5, 19, 0 (overwrite), 13, 18
    kq0 = np.zeros((cap, nkv * rec_bytes(hd, kbits)), np.uint8)
    vq0 = np.zeros((cap, nkv * rec_bytes(hd, vbits)), np.uint8)
    kq, vq = backend.kvq_store(k, v, pos, kq0, vq0, kbits, vbits)
    # the oracle writes in token order too: token 4 overwrites token 0's slot
    wk, wv = oracle_cache(oracle, k, v, pos, cap, kbits, vbits)
    assert np.array_equal(kq, wk)
    assert np.array_equal(vq, wv)


def test_attention_matches_golden(backend):
    """The reference's own attention step over its own quantized caches: row r as a token whose
    head kvh[r] carries the golden query."""
    from test_oracle import kvq_attn_golden
    rng = np.random.default_rng(4)
    for c in kvq_attn_golden():
        hd, nkv = c["hd"], c["nkv"]
        nr = len(c["st"])
        q = rng.standard_normal((nr, nkv, hd)).astype(np.float32)
        for r in range(nr):
            q[r, c["kvh"][r]] = c["q"][r]
        o = backend.kvq_attention(q, c["kq"], c["vq"], c["st"], c["en"], nkv, c["kbits"], c["vbits"], c["scale"])
        got = np.stack([o[r, c["kvh"][r]] for r in range(nr)])
        assert bits_equal(got, c["o"]), (hd, c["kbits"], c["vbits"])


CASES = [  # (n_tok, n_head, n_head_kv, hd, cap, first position, kbits, vbits)
    (1, 4, 4, 32, 64, 0, 4, 4),
    (1, 8, 2, 64, 100, 90, 8, 4),
    (9, 8, 2, 128, 200, 180, 4, 2),
    (3, 4, 1, 256, 70, 60, 4, 4),
    (5, 6, 3, 128, 40, 33, 8, 8),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"t{c[0]}h{c[1]}kv{c[2]}d{c[3]}k{c[6]}v{c[7]}")
def test_attention_matches_oracle(backend, oracle, case):
    """Caches written on the device (checked against the oracle's), then the attention step."""
    n_tok, n_head, n_kv, hd, cap, p0, kbits, vbits = case
    rng = np.random.default_rng(hd + cap + kbits)
    n_fill = cap
    k = rng.standard_normal((n_fill, n_kv, hd)).astype(np.float32)
    v = rng.standard_normal((n_fill, n_kv, hd)).astype(np.float32)
    pos = np.arange(p0, p0 + n_fill, dtype=np.int32)
    kq0 = np.zeros((cap, n_kv * rec_bytes(hd, kbits)), np.uint8)
    vq0 = np.zeros((cap, n_kv * rec_bytes(hd, vbits)), np.uint8)
    kq, vq = backend.kvq_store(k, v, pos, kq0, vq0, kbits, vbits)
    wk, wv = oracle_cache(oracle, k, v, pos, cap, kbits, vbits)
    assert np.array_equal(kq, wk) and np.array_equal(vq, wv)
    q = (rng.standard_normal((n_tok, n_head, hd)) * 3).astype(np.float32)
    en = (p0 + n_fill - n_tok + np.arange(n_tok)).astype(np.int32)
    st = np.maximum(en - (cap - 1), p0).astype(np.int32)
    if n_tok > 1:
        st[:] = st[0]
    scale = float(np.float32(1 / np.sqrt(hd)))
    o = backend.kvq_attention(q, kq, vq, st, en, n_kv, kbits, vbits, scale)
    assert bits_equal(o, oracle_attention(oracle, q, kq, vq, st, en, n_kv, kbits, vbits, scale))


def test_attention_long_decode(backend, oracle):
    """Llama-3-8B shape (32 heads over 8 K / V heads, hd 128), K4 / V4 over a full 2048-slot ring,
    and an 8-token prompt batch at its end."""
    rng = np.random.default_rng(31)
    cap, hd, n_head, n_kv, kb, vb = 2048, 128, 32, 8, 4, 4
    kq = rng.integers(0, 256, (cap, n_kv * rec_bytes(hd, kb)), dtype=np.uint8)
    vq = rng.integers(0, 256, (cap, n_kv * rec_bytes(hd, vb)), dtype=np.uint8)
    for cache in (kq, vq):  # positive finite scales
        for h in range(n_kv):
            cache[:, h * 68:h * 68 + 4] = rng.uniform(0.5, 2.0, (cap, 1)).astype(np.float32).view(np.uint8)
    scale = float(np.float32(1 / np.sqrt(hd)))
    for n_tok in (1, 8):
        q = rng.standard_normal((n_tok, n_head, hd)).astype(np.float32)
        en = (5000 + np.arange(n_tok)).astype(np.int32)
        st = np.full(n_tok, en[-1] - cap + 1, np.int32)
        o = backend.kvq_attention(q, kq, vq, st, en, n_kv, kb, vb, scale)
        assert bits_equal(o, oracle_attention(oracle, q, kq, vq, st, en, n_kv, kb, vb, scale))


def test_attention_dev_bad_rows_are_nan(backend, oracle):
    """On device pointers a token whose range is empty or longer than max_len gets NaN outputs;
    the other tokens are unaffected."""
    rng = np.random.default_rng(41)
    cap, hd, n_head, n_kv, kb, vb = 64, 64, 4, 2, 4, 4
    k = rng.standard_normal((cap, n_kv, hd)).astype(np.float32)
    kq0 = np.zeros((cap, n_kv * rec_bytes(hd, kb)), np.uint8)
    kq, vq = backend.kvq_store(k, k[::-1].copy(), np.arange(cap, dtype=np.int32), kq0, kq0.copy(), kb, vb)
    q = rng.standard_normal((4, n_head, hd)).astype(np.float32)
    st = np.array([0, 10, 20, 5], np.int32)
    en = np.array([9, 9, 60, 30], np.int32)  # token 1 empty, token 2 longer than max_len 32
    bufs = [backend.dev_alloc(a.nbytes) for a in (q, q, kq, vq, st, en)]
    try:
        for b, a in zip(bufs, (q, q, kq, vq, st, en)):
            backend.h2d(b, a)
        backend.kvq_attention_dev(4, n_head, n_kv, hd, kb, vb, bufs[0], bufs[1], bufs[2], bufs[3], cap, bufs[4],
                                  bufs[5], 32, 0.125)
        o = np.empty_like(q)
        backend.d2h(o, bufs[1])
    finally:
        for b in bufs:
            backend.dev_free(b)
    assert np.all(np.isnan(o[1])) and np.all(np.isnan(o[2]))
    for t in (0, 3):
        want = oracle_attention(oracle, q[t:t + 1], kq, vq, st[t:t + 1], en[t:t + 1], n_kv, kb, vb, 0.125)
        assert bits_equal(o[t:t + 1], want)


def test_refusals(backend):
    rng = np.random.default_rng(5)
    k = rng.standard_normal((1, 1, 96)).astype(np.float32)
    with pytest.raises(BackendError):  # hd not a power of 2
        backend.kvq_store(k, k, [0], np.zeros((4, 52), np.uint8), np.zeros((4, 52), np.uint8), 4, 4)
    k = rng.standard_normal((1, 1, 64)).astype(np.float32)
    with pytest.raises(BackendError):  # 2-bit keys: the reference has none
        backend.kvq_store(k, k, [0], np.zeros((4, 20), np.uint8), np.zeros((4, 20), np.uint8), 2, 2)


def test_attention_graph_replays(backend, oracle):
    """fp32 and TurboQuant attention captured in one HIP graph: every replay, with eager calls in
    between, equals the eager result bit for bit (no entry point records a memset)."""
    rng = np.random.default_rng(51)
    cap, hd, n_head, n_kv, kb, vb = 256, 64, 8, 2, 4, 2
    kv_dim = n_kv * hd
    ck = rng.standard_normal((cap, kv_dim)).astype(np.float32)
    cv = rng.standard_normal((cap, kv_dim)).astype(np.float32)
    q = rng.standard_normal((3, n_head, hd)).astype(np.float32)
    st = np.array([100, 100, 100], np.int32)
    en = np.array([300, 301, 302], np.int32)
    pos = np.arange(103, 103 + cap, dtype=np.int32)
    kq0 = np.zeros((cap, n_kv * rec_bytes(hd, kb)), np.uint8)
    vq0 = np.zeros((cap, n_kv * rec_bytes(hd, vb)), np.uint8)
    kq, vq = backend.kvq_store(ck.reshape(cap, n_kv, hd), cv.reshape(cap, n_kv, hd), pos, kq0, vq0, kb, vb)
    arrays = (q, q, q, ck, cv, kq, vq, st, en)
    b = [backend.dev_alloc(a.nbytes) for a in arrays]
    try:
        for d, a in zip(b, arrays):
            backend.h2d(d, a)
        max_len = int((en - st).max()) + 1

        def calls():
            backend.attention_dev(3, n_head, n_kv, hd, b[0], b[1], b[3], b[4], kv_dim, cap, b[7], b[8], max_len, 0.125)
            backend.kvq_attention_dev(3, n_head, n_kv, hd, kb, vb, b[0], b[2], b[5], b[6], cap, b[7], b[8], max_len,
                                      0.125)

        calls()  # eager: grows the scratch buffers before capture
        backend.sync()
        want1, want2 = np.empty_like(q), np.empty_like(q)
        backend.d2h(want1, b[1])
        backend.d2h(want2, b[2])
        assert bits_equal(want1, oracle_attention_fp32(oracle, q, ck, cv, st, en, n_kv, 0.125))
        assert bits_equal(want2, oracle_attention(oracle, q, kq, vq, st, en, n_kv, kb, vb, 0.125))
        backend.graph_begin()
        calls()
        g = backend.graph_end()
        try:
            for _ in range(3):
                zero = np.zeros_like(q)
                backend.h2d(b[1], zero)
                backend.h2d(b[2], zero)
                backend.graph_launch(g)
                backend.sync()
                got1, got2 = np.empty_like(q), np.empty_like(q)
                backend.d2h(got1, b[1])
                backend.d2h(got2, b[2])
                assert bits_equal(got1, want1) and bits_equal(got2, want2)
                calls()  # eager work between replays
                backend.sync()
        finally:
            backend.graph_destroy(g)
    finally:
        for d in b:
            backend.dev_free(d)


def oracle_attention_fp32(oracle, q, ck, cv, st, en, n_kv, scale):
    n_tok, n_head, hd = q.shape
    kvo = np.tile(np.arange(n_head) // (n_head // n_kv) * hd, n_tok)
    return oracle.attn_rows(q.reshape(-1, hd), np.repeat(st, n_head), np.repeat(en, n_head), ck, cv, kvo, hd,
                            scale).reshape(q.shape)


def test_attention_zero_weight_inf_v_scale(backend, oracle):
    """kvq_axpy_v skips a position whose weight is 0 (fastgguf.c:4829-4831): a V record with an
    infinite scale at such a position leaves the output finite. Position 0's key record scale is
    +1e6 and position 1's -1e6 (same codes), so one score dominates and every other weight
    underflows to exactly 0; every V record but those two has scale +inf."""
    rng = np.random.default_rng(77)
    cap, hd, n_kv, kb, vb = 16, 64, 1, 4, 4
    rk, rv = rec_bytes(hd, kb), rec_bytes(hd, vb)
    kq = rng.integers(0, 256, (cap, rk), dtype=np.uint8)
    vq = rng.integers(0, 256, (cap, rv), dtype=np.uint8)
    kq[:, :4] = np.full((cap, 1), 1.0, np.float32).view(np.uint8)
    kq[1, 4:] = kq[0, 4:]
    kq[0, :4] = np.array([1e6], np.float32).view(np.uint8)
    kq[1, :4] = np.array([-1e6], np.float32).view(np.uint8)
    vq[:, :4] = np.full((cap, 1), np.inf, np.float32).view(np.uint8)
    vq[0:2, :4] = np.full((2, 1), 0.75, np.float32).view(np.uint8)
    q = rng.standard_normal((1, 2, hd)).astype(np.float32)
    st, en = np.array([0], np.int32), np.array([cap - 1], np.int32)
    scale = float(np.float32(1 / np.sqrt(hd)))
    want = oracle_attention(oracle, q, kq, vq, st, en, n_kv, kb, vb, scale)
    assert np.isfinite(want).all()  # the oracle (the reference's skip) stays finite
    assert bits_equal(backend.kvq_attention(q, kq, vq, st, en, n_kv, kb, vb, scale), want)
