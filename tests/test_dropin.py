"""The drop-in at the reference's own call sites, without a device: include/fastgguf_c_hip.patch,
applied to a copy of fastgguf.c, only adds FG_HIP blocks; it applies without offset or fuzz; the
patched program compiles and links against include/fastgguf_hip.h and the library; and, with no
usable device, it stays on its CPU path with the reference's messages and results
(fg_gpu_init_ex 1968-2057, gpu_upload_tensor 2060-2081, fg_gpu_matvec 2114-2120, cmd_gpuinfo
2123-2128, matvec_multi 2552, matmul 3004-3009, model_load 4509-4528, moe_ffn 4588-4642).

The patch needs the reference source: where /root/reference is absent (the GPU box) those tests
skip, and tests/test_gpu_dropin.py runs the builds made here on the device."""
import os
import re
import shutil
import subprocess

import numpy as np
import pytest
from conftest import ROOT, bits_equal

from fastgguf_amd import synth as S
from fastgguf_amd.backend import LIB_PATH

REF = "/root/reference/fastgguf.c"
PATCH = os.path.join(ROOT, "include", "fastgguf_c_hip.patch")
needs_ref = pytest.mark.skipif(not os.path.exists(REF), reason="needs the reference source /root/reference")
no_device = pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="checks the no-device path")


def _hunks(text):
    return re.split(r"^@@ .* @@.*\n", text, flags=re.M)[1:]


def test_patch_only_adds_fg_hip_blocks():
    """Every changed line is an addition, and the additions are whole #ifdef FG_HIP ... #endif blocks,
    so a build without FG_HIP is the reference's own program."""
    text = open(PATCH).read()
    hunks = _hunks(text)
    assert len(hunks) == 8
    for h in hunks:
        lines = h.splitlines()
        assert not [l for l in lines if l.startswith("-")]
        added = [l[1:] for l in lines if l.startswith("+")]
        blanks = [l for l in added if not l.strip()]
        body = [l for l in added if l.strip()]
        assert body[0] == "#ifdef FG_HIP" and body[-1] == "#endif", body[:1] + body[-1:]
        depth = 0
        for l in body:
            depth += l.startswith("#if")
            depth -= l.startswith("#endif")
            assert depth >= 0
        assert depth == 0 and len(blanks) <= 2


def _apply(tmp_path):
    d = tmp_path / "src"
    d.mkdir()
    shutil.copy(REF, d / "fastgguf.c")
    r = subprocess.run(["patch", "-p1", "--fuzz=0", "--no-backup-if-mismatch", "-d", str(d), "-i", PATCH],
                       capture_output=True, text=True)
    return d / "fastgguf.c", r


@needs_ref
def test_patch_applies_without_offset_or_fuzz(tmp_path):
    src, r = _apply(tmp_path)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "offset" not in r.stdout and "fuzz" not in r.stdout, r.stdout
    assert open(src).read().count("#ifdef FG_HIP") == 8


@needs_ref
@no_device
def test_patched_program_links_and_stays_on_cpu_without_device(tmp_path):
    """The console program (FG_CONSOLE_MAIN) with the patch: `gpu` probes the device through
    fgh_open, fails cleanly and reports the CPU, as the OpenCL build does without a GPU; the
    reference's own CPU self-test still passes."""
    src, r = _apply(tmp_path)
    assert r.returncode == 0, r.stderr
    exe = tmp_path / "fastgguf_hip"
    libdir = os.path.dirname(LIB_PATH)
    r = subprocess.run(["gcc", "-O1", "-fopenmp", "-march=x86-64-v3", "-Wall", "-Wno-unused-function", "-DFG_HIP",
                        "-DFG_CONSOLE_MAIN", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe),
                        "-L", libdir, "-lfastgguf_hip", f"-Wl,-rpath,{libdir}", "-lm", "-ldl"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-4000:]
    assert "fgh_" not in r.stderr, r.stderr[-4000:]  # no warning in the added code
    nm = subprocess.run(["nm", "-D", "--undefined-only", str(exe)], capture_output=True, text=True).stdout
    for sym in ("fgh_open", "fgh_upload", "fgh_matvec", "fgh_matvec_multi", "fgh_matmul", "fgh_moe_ffn"):
        assert sym in nm, sym
    r = subprocess.run([str(exe), "gpu"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 1, r.stdout + r.stderr
    assert "no usable HIP device" in r.stderr and "[gpu] no usable GPU - CPU only" in r.stdout
    r = subprocess.run([str(exe), "selftest"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and "ALL TESTS PASSED" in r.stdout, r.stdout[-2000:]


@pytest.fixture(scope="module")
def patched_pair():
    from oracle import Reference
    try:
        return Reference("hip"), Reference("avx2")
    except FileNotFoundError:
        pytest.skip("oracle/_ref not built (needs /root/reference at build time)")


@no_device
def test_patched_call_sites_keep_cpu_results_without_device(patched_pair):
    """With fgh_open failing, the patched build's matvec, matvec_multi, matmul and moe_ffn are the
    reference's CPU kernels: outputs equal the unpatched build's bit for bit."""
    hip, cpu = patched_pair
    assert hip.hip_init(0) == -1
    assert hip.hip_state() == (-1, 0, 0, 0)
    cols = 1024
    for t, rp in ((S.T_Q4_K, True), (S.T_Q6_K, False), (S.T_Q8_0, False)):
        w = S.weights(t, 64, cols, 11)
        x = S.activations(cols, 12)
        assert bits_equal(hip.matvec(t, w, cols, x, rp), cpu.matvec(t, w, cols, x, rp))
        X = np.stack([S.activations(cols, 20 + b) for b in range(8)])
        assert bits_equal(hip.matmul(t, w, cols, X, rp), cpu.matmul(t, w, cols, X, rp))
    n_expert, k, n_embd, ff = 8, 2, 256, 256
    g, u = (S.weights(S.T_Q4_K, n_expert * ff, n_embd, s) for s in (31, 32))
    d = S.weights(S.T_Q4_K, n_expert * n_embd, ff, 33)
    X = np.stack([S.activations(n_embd, 40 + t) for t in range(3)])
    X[:, 0] = 1.0
    logits = np.random.default_rng(5).standard_normal((3, n_expert)).astype(np.float32)
    a = hip.moe_ffn((S.T_Q4_K,) * 3, g, u, d, n_expert, k, n_embd, ff, logits, X)
    b = cpu.moe_ffn((S.T_Q4_K,) * 3, g, u, d, n_expert, k, n_embd, ff, logits, X)
    assert all(bits_equal(p, q) for p, q in zip(a, b))
    assert hip.hip_state() == (-1, 0, 0, 0)  # nothing was uploaded
