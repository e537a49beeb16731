"""Tensors uploaded from a mapped GGUF file (fgh_upload_gguf) compute what the same bytes uploaded
directly compute, bit for bit, and equal the oracle: 2-D tensors of the five quantized device
types, a 3-D expert tensor, and F32 tensors (a 2-D one, and a 1-D one taken as one row), which the
reference's GPU path takes too (gpu_kernel_for, fastgguf.c:1745); a tensor of a type the device
path does not take would be refused (FGH_SKIP_TYPE)."""
import os

import numpy as np
import pytest
from conftest import ROOT, bits_equal

import gguf_write as GW
from fastgguf_amd import synth as S
from fastgguf_amd.backend import SKIP_TYPE, BackendError, Gguf
from oracle import ORDER_REPACKED, ORDER_ROW

pytestmark = pytest.mark.gpu

TINY = os.path.join(ROOT, "tests", "golden", "tiny.gguf")


def test_upload_from_gguf_matches_oracle(backend, oracle):
    kvs, tensors = GW.tiny_model()
    with Gguf(TINY) as f:
        for name, ty, dims, data in tensors:
            if ty not in S.BLOCK:
                with pytest.raises(BackendError) as e:
                    backend.upload_gguf(f, name)
                assert e.value.status == SKIP_TYPE
                continue
            t = backend.upload_gguf(f, name)
            cols = dims[0]
            rows = (dims[1] if len(dims) > 1 else 1) * (dims[2] if len(dims) > 2 else 1)
            w = np.frombuffer(data, np.uint8).reshape(rows, -1)
            x = S.activations(cols, 800 + ty)
            y = backend.matvec(t, x)
            # 2-D Q4_K with rows % 8 == 0 is repacked, as the reference's loader repacks it
            order = ORDER_REPACKED if ty == S.T_Q4_K and len(dims) == 2 and dims[1] % 8 == 0 else ORDER_ROW
            assert bits_equal(y, oracle.matvec(ty, w, cols, x, order)), name
            mrows = dims[1] if len(dims) > 1 else 1
            t2 = backend.upload(ty, cols, w, rows=mrows, n_mats=rows // mrows)
            assert bits_equal(backend.matvec(t2, x), y), name
            t.free()
            t2.free()
