"""GGUF ingestion (fgh_gguf_*, the reference's gguf_open / kv_num / tensor_find, fastgguf.c:342-454)
on the CPU: the library parses tests/golden/tiny.gguf to the same summary, tensor table and
metadata answers as the reference's own gguf_open did (tests/golden/gguf.npz, written by the
compiled reference), accepts and refuses the same broken variants, and survives corrupted files.
No device is needed."""
import os

import numpy as np
import pytest
from conftest import ROOT, golden

import gguf_write as GW
from fastgguf_amd import synth as S
from fastgguf_amd.backend import BackendError, Gguf

TINY = os.path.join(ROOT, "tests", "golden", "tiny.gguf")


def test_tiny_table_matches_reference():
    g = golden("gguf.npz")
    with Gguf(TINY) as f:
        s = f.summary()
        assert (s["version"], s["alignment"], s["n_kvs"], s["n_tensors"]) == \
            (int(g["version"][0]), int(g["alignment"][0]), int(g["n_kvs"][0]), int(g["n_tensors"][0]))
        for i, t in enumerate(f.tensors()):
            assert t["name"] == bytes(g["names"][i]).rstrip(b"\0").decode()
            assert t["type"] == int(g["types"][i]) and t["n_dims"] == int(g["n_dims"][i])
            assert t["ne"] == [int(v) for v in g["ne"][i][: t["n_dims"]]]
            assert t["offset"] == int(g["offsets"][i]) and t["nbytes"] == int(g["nbytes"][i])
        for key, want in zip(g["kv_keys"], g["kv_vals"]):
            assert f.kv_num(str(key), -1.0) == want, key
        assert f.kv_str("general.architecture") == "llama"
        assert f.kv_str("llama.block_count") is None and f.kv_str("no.such.key") is None


def test_tiny_data_and_lookup():
    kvs, tensors = GW.tiny_model()
    with Gguf(TINY) as f:
        for i, (name, ty, dims, data) in enumerate(tensors):
            assert f.find(name) == i
            assert f.data(i).tobytes() == data
        assert f.find("blk.0.ffn_up.weight") == -1
        # the stored key is the reader's first 95 characters (the reference's kv_t key buffer)
        assert f.kv_num(GW.LONG_KEY[:95], -1.0) == 77.0 and f.kv_num(GW.LONG_KEY, -1.0) == -1.0


def test_broken_files_as_the_reference(tmp_path):
    g = golden("gguf.npz")
    want = dict(zip([str(n) for n in g["variant_names"]], [int(r) for r in g["variant_rc"]]))
    good = open(TINY, "rb").read()
    variants = GW.variants(good)
    assert set(variants) == set(want)
    for name, data in variants.items():
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(data)
        try:
            Gguf(str(p)).close()
            got = 0
        except BackendError:
            got = -1
        assert got == want[name], name


def test_missing_file_and_bad_arguments(tmp_path):
    with pytest.raises(BackendError) as e:
        Gguf(str(tmp_path / "nope.gguf"))
    assert "cannot open" in str(e.value)
    from fastgguf_amd.backend import load_library
    L = load_library()
    assert L.fgh_gguf_open(None, None, None, 0) < 0
    assert L.fgh_gguf_find(None, b"x") == -1
    assert L.fgh_gguf_kv_str(None, b"x") is None
    assert L.fgh_gguf_data(None, 0) is None
    L.fgh_gguf_close(None)


def test_corrupted_headers_never_crash(tmp_path):
    """Random byte changes and truncations inside the header and tables: every open either
    succeeds with tensors inside the file or fails with a status."""
    good = bytearray(open(TINY, "rb").read())
    rng = np.random.default_rng(5)
    head = 1088  # the data section of tiny.gguf starts here
    for k in range(300):
        b = bytearray(good)
        for _ in range(int(rng.integers(1, 4))):
            b[int(rng.integers(4, head))] = int(rng.integers(0, 256))
        if k % 3 == 0:
            b = b[: int(rng.integers(4, len(b)))]
        p = tmp_path / "c.gguf"
        p.write_bytes(bytes(b))
        try:
            f = Gguf(str(p))
        except BackendError:
            continue
        for t in f.tensors():
            assert t["offset"] + t["nbytes"] <= len(b)
        f.close()


def test_overflowing_dims_and_alignment_refused(tmp_path):
    """Headers the reference would mis-read: dims whose element product wraps a u64 (here
    256 x 2^60 x 16 = 2^72, which wraps to 0 and would pass the end-of-file check with a 0-byte
    tensor), a byte count that wraps after the block division, and general.alignment values
    below 1 (a division by zero in the reference) or past 2^32. Each is refused with a status."""
    blk = bytes(144)
    cases = {
        "dims_wrap": GW.gguf_bytes([("general.alignment", GW.U32, 32)],
                                   [("w", S.T_Q4_K, [256, 1 << 60, 16], blk)]),
        "bytes_wrap": GW.gguf_bytes([("general.alignment", GW.U32, 32)],
                                    [("w", S.T_Q4_K, [1 << 62, 2], blk)]),
        "align_half": GW.gguf_bytes([("general.alignment", GW.F32, 0.5)], [("w", S.T_Q4_K, [256, 1], blk)]),
        "align_huge": GW.gguf_bytes([("general.alignment", GW.U64, 1 << 40)], [("w", S.T_Q4_K, [256, 1], blk)]),
    }
    for name, data in cases.items():
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(data)
        with pytest.raises(BackendError):
            Gguf(str(p)).close()
    # the same files with sane values open
    ok = GW.gguf_bytes([("general.alignment", GW.U32, 32)], [("w", S.T_Q4_K, [256, 1], blk)])
    p = tmp_path / "ok.gguf"
    p.write_bytes(ok)
    with Gguf(str(p)) as f:
        assert f.tensors()[0]["nbytes"] == 144
