"""fgh_ffn_dev: the dense SiLU FFN of one token (forward, fastgguf.c:4870-4877: matvec_multi of
ffn_gate and ffn_up, `gate[i] = silu_f(gate[i]) * up[i]`, matvec of ffn_down) through the C ABI.

h and y are compared bit for bit with the oracle's matvecs and the reference's loop (libm expf), at
the benchmark's shape and at small and odd ones, over back-to-back calls and graph replays, for
repacked Q4_K (the paired gate / up launch, then the down matvec) and for types that take the
matvecs and the silu launch."""
import numpy as np
import pytest
from conftest import bits_equal

from fastgguf_amd import synth as S
from oracle import ORDER_REPACKED as O_RP
from oracle import ORDER_ROW as O_ROW

pytestmark = pytest.mark.gpu


def _reference(oracle, types, ws, n_embd, ff, x, order=O_RP):
    """h and y of the reference's FFN (the oracle's matvecs in the CPU path's order, the loop)"""
    g = oracle.matvec(types[0], ws[0], n_embd, x, order)
    u = oracle.matvec(types[1], ws[1], n_embd, x, order)
    h = (g / (np.float32(1.0) + oracle.libm_expf(-g)) * u).astype(np.float32)
    o_down = order if types[2] in (S.T_Q4_K, S.T_Q4_0) else O_ROW
    return h, oracle.matvec(types[2], ws[2], ff, h, o_down)


class Ffn:
    """device buffers and tensors of one FFN on one context"""

    def __init__(self, be, types, n_embd, ff, seed):
        self.be, self.n_embd, self.ff = be, n_embd, ff
        self.ws = [S.random_bytes_weights(types[0], ff, n_embd, seed), S.random_bytes_weights(types[1], ff, n_embd, seed + 1),
                   S.random_bytes_weights(types[2], n_embd, ff, seed + 2)]
        self.ts = [be.upload(types[0], n_embd, self.ws[0]), be.upload(types[1], n_embd, self.ws[1]),
                   be.upload(types[2], ff, self.ws[2])]
        self.xd, self.hd, self.yd = be.dev_alloc(4 * n_embd), be.dev_alloc(4 * ff), be.dev_alloc(4 * n_embd)

    def run(self, x, calls=1):
        self.be.h2d(self.xd, x)
        for _ in range(calls):
            self.be.ffn_dev(*self.ts, self.xd, self.hd, self.yd)
        self.be.sync()
        return self.read()

    def read(self):
        h, y = np.empty(self.ff, np.float32), np.empty(self.n_embd, np.float32)
        self.be.d2h(h, self.hd)
        self.be.d2h(y, self.yd)
        return h, y

    def free(self):
        for t in self.ts:
            t.free()
        for p in (self.xd, self.hd, self.yd):
            self.be.dev_free(p)


Q4K3 = (S.T_Q4_K,) * 3
CASES = [  # types, n_embd, ff: the benchmark's FFN, one-block rows, odd tile counts, a short down
    (Q4K3, 4096, 14336), (Q4K3, 256, 256), (Q4K3, 512, 768), (Q4K3, 2048, 5632), (Q4K3, 256, 4096),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[1]}x{c[2]}")
def test_ffn_bit_exact(backend, oracle, case):
    types, n_embd, ff = case
    f = Ffn(backend, types, n_embd, ff, 900 + ff)
    x = S.activations(n_embd, 901) * np.float32(2.0)
    print(f"ffn {n_embd}x{ff}", flush=True)
    h, y = f.run(x, calls=3)  # back-to-back calls
    hr, yr = _reference(oracle, types, f.ws, n_embd, ff, x)
    assert bits_equal(h, hr)
    assert bits_equal(y, yr)
    f.free()


def test_ffn_graph_replays(backend, oracle):
    """Three FFNs (different x) captured in one graph, replayed four times with eager calls and
    host synchronizations between the replays: every replay gives the eager results."""
    n_embd, ff = 4096, 14336
    f = Ffn(backend, Q4K3, n_embd, ff, 960)
    xs = [S.activations(n_embd, 961 + i) for i in range(3)]
    xds = [backend.dev_alloc(4 * n_embd) for _ in xs]
    outs = [(backend.dev_alloc(4 * ff), backend.dev_alloc(4 * n_embd)) for _ in xs]
    for xd, x in zip(xds, xs):
        backend.h2d(xd, x)
    want = [_reference(oracle, Q4K3, f.ws, n_embd, ff, x) for x in xs]
    f.run(xs[0])  # an eager call before the capture sizes any scratch
    backend.graph_begin()
    for xd, (hd, yd) in zip(xds, outs):
        backend.ffn_dev(*f.ts, xd, hd, yd)
    g = backend.graph_end()
    try:
        for rep in range(4):
            backend.graph_launch(g)
            backend.sync()
            for (hd, yd), (hr, yr) in zip(outs, want):
                h, y = np.empty(ff, np.float32), np.empty(n_embd, np.float32)
                backend.d2h(h, hd)
                backend.d2h(y, yd)
                assert bits_equal(h, hr) and bits_equal(y, yr), f"replay {rep}"
            h, y = f.run(xs[1])  # eager work between replays
            assert bits_equal(y, want[1][1])
    finally:
        backend.graph_destroy(g)
    for p in xds + [p for o in outs for p in o]:
        backend.dev_free(p)
    f.free()


@pytest.mark.parametrize("types", [(S.T_Q4_K, S.T_Q4_K, S.T_Q6_K), (S.T_Q6_K,) * 3, (S.T_Q5_K, S.T_Q5_K, S.T_Q4_K)],
                         ids=["down_Q6_K", "Q6_K", "Q5_K_gate_up"])
def test_ffn_other_types(backend, oracle, types):
    """A Q6_K down, Q6_K gate and up (the matvecs, then the silu launch) and Q5_K gate and up (its
    row order): the same bits as the reference's sequence."""
    n_embd, ff = 2048, 5632
    f = Ffn(backend, types, n_embd, ff, 970)
    x = S.activations(n_embd, 971)
    h, y = f.run(x)
    order = O_ROW if types[0] == S.T_Q5_K else O_RP
    g = oracle.matvec(types[0], f.ws[0], n_embd, x, order)
    u = oracle.matvec(types[1], f.ws[1], n_embd, x, order)
    hr = (g / (np.float32(1.0) + oracle.libm_expf(-g)) * u).astype(np.float32)
    yr = oracle.matvec(types[2], f.ws[2], ff, hr, O_RP if types[2] == S.T_Q4_K else O_ROW)
    assert bits_equal(h, hr) and bits_equal(y, yr)
    f.free()
