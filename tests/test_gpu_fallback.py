"""The caller's fallback when a device call fails (fastgguf.c:2577-2581): matvec reports the
failure, sets g_gpu.state = -1, and recomputes on its CPU kernels for the rest of the process.

FGH_FAIL_AT=n (read by fgh_open) makes the n-th compute call of that context return FGH_ERR
before it launches anything, so no kernel is disturbed. A caller written like the reference's
matvec then gets, call for call, the same outputs whether the device or its CPU path computed them:
the device results are bit-identical to the reference CPU kernels (the oracle stands in for them
here)."""
import os

import numpy as np
import pytest
from conftest import bits_equal

from fastgguf_amd import synth as S
from fastgguf_amd.backend import ERR, Backend, BackendError
from oracle import ORDER_REPACKED as O_RP

pytestmark = pytest.mark.gpu


class Caller:
    """The reference's matvec driver (fastgguf.c:2575-2581) over this backend."""

    def __init__(self, backend, oracle):
        self.be, self.oracle, self.gpu_state = backend, oracle, 1
        self.failures = []

    def matvec(self, t, w, cols, x):
        if t is not None and self.gpu_state == 1:
            try:
                return self.be.matvec(t, x), "gpu"
            except BackendError as e:
                self.failures.append(e)  # "[gpu] matvec failed on ... - falling back to CPU"
                self.gpu_state = -1
        return self.oracle.matvec(S.T_Q4_K, w, cols, x, O_RP), "cpu"


def test_injected_failure_falls_back_with_identical_results(oracle):
    old = os.environ.get("FGH_FAIL_AT")
    os.environ["FGH_FAIL_AT"] = "3"
    try:
        be = Backend(0)  # the self-check at open does not count
    finally:
        if old is None:
            del os.environ["FGH_FAIL_AT"]
        else:
            os.environ["FGH_FAIL_AT"] = old
    try:
        cols = 2048
        ws = [S.weights(S.T_Q4_K, 256, cols, 600 + i) for i in range(5)]
        ts = [be.upload(S.T_Q4_K, cols, w) for w in ws]
        caller = Caller(be, oracle)
        where = []
        for i, (t, w) in enumerate(zip(ts, ws)):
            x = S.activations(cols, 610 + i)
            y, dev = caller.matvec(t, w, cols, x)
            where.append(dev)
            assert bits_equal(y, oracle.matvec(S.T_Q4_K, w, cols, x, O_RP)), f"call {i} on {dev}"
        assert where == ["gpu", "gpu", "cpu", "cpu", "cpu"]
        assert len(caller.failures) == 1 and caller.failures[0].status == ERR
        assert "injected failure" in str(caller.failures[0])
        # the failed call launched nothing: the context is still usable
        x = S.activations(cols, 620)
        assert bits_equal(be.matvec(ts[0], x), oracle.matvec(S.T_Q4_K, ws[0], cols, x, O_RP))
        for t in ts:
            t.free()
    finally:
        be.close()
