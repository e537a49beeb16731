"""GPU parity of attention over the KV ring cache (attn_rows, fastgguf.c:3273-3326) through the C ABI.

Every output is compared bit for bit: against the compiled reference's golden outputs and against
the oracle's restatement (pinned to those outputs) on decode and prompt-batch ranges, GQA head
groups, ring wrap, head sizes 32 .. 256, every range length mod 8 (the softmax tail), and scores
spread past exp_neg_ps's -87 cut-off. Head sizes that are not multiples of 32 (the reference's
per-row path, dot_f32v's score order) run with 16-value chunks only, an extra group of 8, a
scalar tail, and odd sizes whose rows are not 16-byte aligned.
"""
import numpy as np
import pytest
from conftest import bits_equal, bits_equal_or_nan

from fastgguf_amd.backend import BackendError

pytestmark = pytest.mark.gpu


def oracle_attention(oracle, q, ck, cv, st, en, n_head_kv, scale):
    n_tok, n_head, hd = q.shape
    g = n_head // n_head_kv
    rows_st = np.repeat(np.asarray(st, np.int32), n_head)
    rows_en = np.repeat(np.asarray(en, np.int32), n_head)
    kvo = np.tile(np.arange(n_head) // g * hd, n_tok).astype(np.int32)
    return oracle.attn_rows(q.reshape(-1, hd), rows_st, rows_en, ck, cv, kvo, hd, scale).reshape(q.shape)


def test_attention_matches_golden(backend):
    """The golden calls (up to 4 rows sharing a head offset) as one head of kv_dim / hd heads."""
    from test_oracle import attn_golden
    rng = np.random.default_rng(3)
    for c in attn_golden():
        hd, kvo = c["hd"], c["kvo"]
        n_head = c["ck"].shape[1] // hd
        q = rng.standard_normal((len(c["st"]), n_head, hd)).astype(np.float32)
        q[:, kvo // hd] = c["q"]
        o = backend.attention(q, c["ck"], c["cv"], c["st"], c["en"], n_head, c["scale"])
        assert bits_equal_or_nan(o[:, kvo // hd], c["o"]), (hd, kvo, c["st"], c["en"])


CASES = [  # (n_tok, n_head, n_head_kv, hd, cap, first position, magnitude)
    (1, 4, 4, 32, 64, 0, 1.0),        # one position
    (1, 8, 2, 64, 100, 90, 1.0),      # decode over a wrapped ring
    (9, 8, 2, 128, 200, 180, 1.0),    # causal prompt batch over a wrapped ring, every length mod 8
    (5, 6, 3, 96, 40, 33, 1.0),       # hd 96, ring shorter than the range start
    (3, 4, 1, 256, 70, 60, 1.0),      # hd 256, multi-query
    (4, 2, 2, 32, 50, 10, 30.0),      # scores past the -87 cut-off
    (1, 32, 32, 80, 300, 250, 1.0),   # per-row path: hd 80 decode (five 16-value chunks)
    (9, 8, 2, 112, 60, 50, 1.0),      # hd 112: chunks and one group of 8, prompt batch, GQA
    (5, 6, 3, 100, 40, 33, 1.0),      # hd 100: a scalar tail of 4
    (70, 4, 2, 72, 100, 20, 1.0),     # hd 72, 70 tokens x 2 heads per K head: the 16-row value kernel
    (3, 5, 5, 13, 30, 25, 2.0),       # odd hd: unaligned rows, values read one by one
    (66, 2, 1, 6, 80, 0, 1.0),        # tiny hd: the tail only; 66 rows per K head
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"t{c[0]}h{c[1]}kv{c[2]}d{c[3]}cap{c[4]}")
def test_attention_matches_oracle(backend, oracle, case):
    n_tok, n_head, n_kv, hd, cap, p0, mag = case
    rng = np.random.default_rng(hd + cap)
    kv_dim = n_kv * hd
    ck = rng.standard_normal((cap, kv_dim)).astype(np.float32)
    cv = rng.standard_normal((cap, kv_dim)).astype(np.float32)
    q = (rng.standard_normal((n_tok, n_head, hd)) * mag).astype(np.float32)
    en = p0 + np.arange(n_tok, dtype=np.int32) + min(cap - n_tok, 30)
    st = np.maximum(en - (cap - 1), p0).astype(np.int32)  # as long as the cache allows
    if n_tok > 1:
        st[:] = p0  # causal: token t sees p0 .. p0 + (offset) + t
    scale = float(np.float32(1 / np.sqrt(hd)))
    o = backend.attention(q, ck, cv, st, en, n_kv, scale)
    assert bits_equal(o, oracle_attention(oracle, q, ck, cv, st, en, n_kv, scale))


@pytest.mark.parametrize("case", [(70, 4, 2, 72, 100, 20), (66, 2, 1, 6, 80, 0), (3, 5, 5, 13, 30, 25)],
                         ids=["d72_16row", "d6_16row_unaligned", "d13_4row_unaligned"])
def test_attention_per_row_path_nonfinite_v(backend, oracle, case):
    """The per-row path (hd % 32 != 0) walks each row's own positions only (fastgguf.c:3318-3323):
    inf and NaN in V at the last position of a causal batch, which only the last token attends,
    leave every other token's outputs finite, in the value kernel's 16-row and 4-row groups alike.
    (The vector path walks its call's whole span, with NaN where fma(0, inf) falls: the golden
    case with hd 64 covers that.)"""
    n_tok, n_head, n_kv, hd, cap, p0 = case
    rng = np.random.default_rng(hd + 7)
    kv_dim = n_kv * hd
    ck = rng.standard_normal((cap, kv_dim)).astype(np.float32)
    cv = rng.standard_normal((cap, kv_dim)).astype(np.float32)
    q = rng.standard_normal((n_tok, n_head, hd)).astype(np.float32)
    en = (p0 + 5 + np.arange(n_tok)).astype(np.int32)
    st = np.full(n_tok, p0, np.int32)
    last = int(en[-1]) % cap
    cv[last, 0] = np.inf
    cv[last, kv_dim - 1] = np.nan
    scale = float(np.float32(1 / np.sqrt(hd)))
    o = backend.attention(q, ck, cv, st, en, n_kv, scale)
    want = oracle_attention(oracle, q, ck, cv, st, en, n_kv, scale)
    assert np.isfinite(want[:-1]).all() and not np.isfinite(want[-1]).all()
    assert bits_equal_or_nan(o, want)


def test_attention_long_decode(backend, oracle):
    """A Llama-3-8B-shaped decode step (32 heads over 8 KV heads, hd 128) at 4096 positions of a
    wrapped 4096-slot ring, and a 64-token prompt batch at the end of the same cache."""
    rng = np.random.default_rng(11)
    cap, hd, n_head, n_kv = 4096, 128, 32, 8
    ck = rng.standard_normal((cap, n_kv * hd)).astype(np.float32)
    cv = rng.standard_normal((cap, n_kv * hd)).astype(np.float32)
    scale = float(np.float32(1 / np.sqrt(hd)))
    q = rng.standard_normal((1, n_head, hd)).astype(np.float32)
    st, en = np.array([5000], np.int32), np.array([5000 + cap - 1], np.int32)
    o = backend.attention(q, ck, cv, st, en, n_kv, scale)
    assert bits_equal(o, oracle_attention(oracle, q, ck, cv, st, en, n_kv, scale))
    q = rng.standard_normal((64, n_head, hd)).astype(np.float32)
    en = (2000 + np.arange(64)).astype(np.int32)
    st = np.zeros(64, np.int32)
    o = backend.attention(q, ck, cv, st, en, n_kv, scale)
    assert bits_equal(o, oracle_attention(oracle, q, ck, cv, st, en, n_kv, scale))


def test_attention_dev_bad_rows_are_nan(backend, oracle):
    """On device pointers the ranges are not checked on the host: a token whose range is empty or
    longer than max_len gets NaN outputs and the other tokens are unaffected."""
    rng = np.random.default_rng(12)
    cap, hd, n_head, n_kv = 64, 64, 4, 2
    ck = rng.standard_normal((cap, n_kv * hd)).astype(np.float32)
    cv = rng.standard_normal((cap, n_kv * hd)).astype(np.float32)
    q = rng.standard_normal((4, n_head, hd)).astype(np.float32)
    st = np.array([0, 10, 20, 5], np.int32)
    en = np.array([9, 9, 60, 30], np.int32)  # token 1 empty, token 2 longer than max_len 32
    scale = 0.125
    bufs = [backend.dev_alloc(a.nbytes) for a in (q, q, ck, cv, st, en)]
    try:
        for b, a in zip(bufs, (q, q, ck, cv, st, en)):
            backend.h2d(b, a)
        backend.attention_dev(4, n_head, n_kv, hd, bufs[0], bufs[1], bufs[2], bufs[3], n_kv * hd, cap, bufs[4],
                              bufs[5], 32, scale)
        o = np.empty_like(q)
        backend.d2h(o, bufs[1])
    finally:
        for b in bufs:
            backend.dev_free(b)
    assert np.all(np.isnan(o[1])) and np.all(np.isnan(o[2]))
    for t in (0, 3):
        want = oracle_attention(oracle, q[t:t + 1], ck, cv, st[t:t + 1], en[t:t + 1], n_kv, scale)
        assert bits_equal(o[t:t + 1], want)


def test_attention_refusals(backend):
    rng = np.random.default_rng(13)
    ck = rng.standard_normal((16, 96)).astype(np.float32)
    q = rng.standard_normal((1, 1, 288)).astype(np.float32)
    with pytest.raises(BackendError):  # hd above 256
        backend.attention(q, np.zeros((16, 288), np.float32), np.zeros((16, 288), np.float32), [0], [3], 1, 0.1)
    q = rng.standard_normal((1, 3, 32)).astype(np.float32)
    with pytest.raises(BackendError):  # 3 heads over 2 KV heads
        backend.attention(q, ck, ck, [0], [3], 2, 0.1)
    q = rng.standard_normal((1, 2, 32)).astype(np.float32)
    with pytest.raises(BackendError):  # range longer than the cache
        backend.attention(q, ck, ck, [0], [16], 2, 0.1)
    with pytest.raises(BackendError):  # empty range
        backend.attention(q, ck, ck, [5], [4], 2, 0.1)
