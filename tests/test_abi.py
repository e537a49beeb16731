"""The C ABI library loads and exports every entry point include/fastgguf_hip.h declares, and its
argument checks and no-device path work without a GPU (no compute calls here)."""
import ctypes as C
import os
import re

import pytest
from conftest import ROOT

from fastgguf_amd import backend as B

HEADER = os.path.join(ROOT, "include", "fastgguf_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fgh_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert declared_functions() == sorted(B.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = B.load_library()
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_library_exports_nothing_else():
    out = os.popen(f"nm -D --defined-only {B.LIB_PATH}").read()
    syms = {l.split()[-1] for l in out.splitlines() if " T " in l}
    assert {s for s in syms if s.startswith("fgh_")} == set(B.EXPORTS)


def test_null_arguments_are_rejected():
    lib = B.load_library()
    h = C.c_void_p()
    assert lib.fgh_upload(None, 12, 256, 8, 1, -1, None, 0, C.byref(h)) == B.ERR_ARG
    assert lib.fgh_matvec(None, None, None, None) == B.ERR_ARG
    assert lib.fgh_matvec_multi(None, 1, None, None, None) == B.ERR_ARG
    assert lib.fgh_matmul(None, None, None, 0, None, 0, 1) == B.ERR_ARG
    assert lib.fgh_info(None, None) == B.ERR_ARG
    assert lib.fgh_open(0, 0, None) == B.ERR_ARG
    assert lib.fgh_last_error(None) == b"no context"
    lib.fgh_close(None)
    lib.fgh_tensor_free(None)


def _has_gpu():
    return os.path.exists("/dev/kfd")


@pytest.mark.skipif(_has_gpu(), reason="checks the no-device path")
def test_open_without_device_fails_cleanly():
    """Like fg_gpu_init without a usable GPU (fastgguf.c:1984-1995): an error status, no abort,
    and the caller stays on its CPU path."""
    lib = B.load_library()
    h = C.c_void_p(1234)
    rc = lib.fgh_open(0, 0, C.byref(h))
    assert rc == B.ERR_DEVICE and not h.value
    with pytest.raises(B.BackendError):
        B.Backend(0)


def test_gpu_off_env_keeps_the_caller_on_cpu(monkeypatch):
    """FASTGGUF_GPU=off (or 0, cpu, none) makes fgh_open fail without touching a device, as
    fg_gpu_init_ex returns with g_gpu.state = -1 (fastgguf.c:1972-1976)."""
    lib = B.load_library()
    for v in ("off", "0", "cpu", "none"):
        monkeypatch.setenv("FASTGGUF_GPU", v)
        h = C.c_void_p(1234)
        assert lib.fgh_open(0, 0, C.byref(h)) == B.ERR_DEVICE and not h.value


def test_c_caller_compiles_links_and_runs(tmp_path):
    """A C program built with gcc against include/fastgguf_hip.h and linked with the library: the
    header is valid C99, the exports resolve, and the program runs (GGUF parse; without a device
    fgh_open fails cleanly and it stays on its CPU path)."""
    import subprocess
    exe = tmp_path / "abi_smoke"
    src = os.path.join(ROOT, "tests", "c_abi", "abi_smoke.c")
    libdir = os.path.dirname(B.LIB_PATH)
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"), src, "-o",
                        str(exe), "-L", libdir, "-lfastgguf_hip", f"-Wl,-rpath,{libdir}"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe), os.path.join(ROOT, "tests", "golden", "tiny.gguf")], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "output.weight 32 x 64 Q8_0" in r.stdout
    assert ("staying on the CPU path" in r.stdout) != ("matvec: ok" in r.stdout)
