"""The drop-in on the device, driven from C: the reference's own call sites, patched by
include/fastgguf_c_hip.patch (fg_gpu_init_ex 1968, gpu_upload_tensor 2060, fg_gpu_matvec 2114,
matvec_multi 2552, matvec 2575-2581, matmul 3004-3009, moe_ffn 4588), run through the gfx950
library and return what the unpatched reference computes on its CPU; the patched console program
and the plain C caller of the ABI find and use the device.

The patched builds are made where the reference source is (oracle/_ref/libfgref_hip.so: the
reference's harness on the patched copy; oracle/_ref/fastgguf_hip: the patched console program;
tests/c_abi/_build/abi_smoke: the C caller) and travel with the tree. The unpatched AVX2 build
(oracle/_ref/libfgref_avx2.so, the same -march) is the checker. Tolerance: bit-exact, except the
64-token prompt GEMMs of Q4_K, Q6_K and Q8_0, whose fp32 sums run in another order than the
reference's gemm_kquant / gemm_q32: max |y - y_ref| / max |y_ref| <= 1e-5 per token, the
reference's own selftest bound (5723-5733)."""
import json
import os
import subprocess
import sys

import numpy as np
import pytest
from conftest import ROOT, bits_equal, rel_err

from fastgguf_amd import synth as S

pytestmark = pytest.mark.gpu

HIP_SO = os.path.join(ROOT, "oracle", "_ref", "libfgref_hip.so")
CONSOLE = os.path.join(ROOT, "oracle", "_ref", "fastgguf_hip")
C_CALLER = os.path.join(ROOT, "tests", "c_abi", "_build", "abi_smoke")
TOL = 1e-5
REPACKS = (S.T_Q4_K, S.T_Q4_0)  # the types model_load repacks (repack_tensor 2486-2489)


def _need(path):
    if not os.path.exists(path):
        pytest.skip(f"{os.path.relpath(path, ROOT)} not built (build() makes it where /root/reference is)")


@pytest.fixture(scope="module")
def pair():
    _need(HIP_SO)
    from oracle import Reference
    hip, cpu = Reference("hip"), Reference("avx2")
    assert hip.hip_init(0) == 1, "the patched fg_gpu_init_ex did not open the device"
    return hip, cpu


def test_c_caller_runs_on_the_device():
    """tests/c_abi/abi_smoke.c, built with gcc against the header: its device branch (closed-form
    Q8_0 matvec, the 16-token prompt GEMM, the upload counters)."""
    _need(C_CALLER)
    print("abi_smoke device branch", flush=True)
    r = subprocess.run([C_CALLER, os.path.join(ROOT, "tests", "golden", "tiny.gguf")], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    for line in ("matvec: ok", "matmul: ok", "info: ok"):
        assert line in r.stdout, r.stdout


def test_patched_console_program_reports_the_device():
    """`fastgguf gpu` (cmd_gpuinfo 2123-2128) of the patched program: fg_gpu_init_ex opens the
    device through fgh_open (and its self-check) and the probe succeeds."""
    _need(CONSOLE)
    print("patched console: gpu", flush=True)
    r = subprocess.run([CONSOLE, "gpu"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "[gpu] using " in r.stdout and "[gpu] READY: " in r.stdout, r.stdout


@pytest.mark.parametrize("type_", [S.T_Q4_K, S.T_Q4_0, S.T_Q6_K, S.T_Q8_0, S.T_Q5_K, S.T_Q5_0, S.T_Q4_1, S.T_Q5_1,
                                   S.T_IQ4_NL, S.T_Q2_K, S.T_Q3_K, S.T_IQ4_XS, S.T_F32, S.T_F16, S.T_BF16])
def test_matvec_call_site(pair, type_):
    """matvec (2575): the tensor uploaded by gpu_upload_tensor runs on the device in the order the
    CPU path would have used (Q4_K / Q4_0 repacked, as model_load does), bit for bit. Q2_K, Q3_K
    and IQ4_XS, which the reference's own GPU path leaves on the CPU (gpu_kernel_for 1744-1751),
    are offloaded too; F32, F16 and BF16 run there in both (1745), here with the CPU kernels'
    bits."""
    hip, cpu = pair
    rows, cols = 2048, 4096
    w = S.weights(type_, rows, cols, 100 + type_)
    x = S.activations(cols, 200 + type_)
    st0 = hip.hip_state()
    print(f"matvec {S.TYPE_NAME[type_]} {rows}x{cols}", flush=True)
    y = hip.matvec(type_, w, cols, x, True)
    st1 = hip.hip_state()
    assert st1[0] == 1 and st1[1] == st0[1] + 1, (st0, st1)  # offloaded, not skipped
    assert bits_equal(y, cpu.matvec(type_, w, cols, x, type_ in REPACKS))


def test_matvec_row_order_with_repack_off(pair, monkeypatch):
    """FASTGGUF_REPACK=0 keeps the CPU path on file-layout rows (4543): the upload then picks the
    row order too."""
    hip, cpu = pair
    monkeypatch.setenv("FASTGGUF_REPACK", "0")
    w = S.weights(S.T_Q4_K, 1024, 4096, 300)
    x = S.activations(4096, 301)
    assert bits_equal(hip.matvec(S.T_Q4_K, w, 4096, x, True), cpu.matvec(S.T_Q4_K, w, 4096, x, False))


def test_matvec_multi_call_site(pair):
    """matvec_multi (2552) over Q, K, V of a Q4_K_M file (Q4_K, Q4_K, Q6_K): one device call."""
    hip, cpu = pair
    cols = 4096
    types = [S.T_Q4_K, S.T_Q4_K, S.T_Q6_K]
    rows = [4096, 1024, 1024]
    ws = [S.weights(t, r, cols, 400 + i) for i, (t, r) in enumerate(zip(types, rows))]
    x = S.activations(cols, 410)
    outs = []
    for ref, rp in ((hip, [1, 1, 1]), (cpu, [1, 1, 0])):
        import ctypes as C
        ys = [np.zeros(r, np.float32) for r in rows]
        tarr = (C.c_uint32 * 3)(*types)
        rarr = (C.c_int * 3)(*rp)
        warr = (C.c_void_p * 3)(*[w.ctypes.data for w in ws])
        narr = (C.c_int64 * 3)(*rows)
        yarr = (C.c_void_p * 3)(*[y.ctypes.data for y in ys])
        assert ref.lib.fgr_matvec_multi(3, tarr, rarr, warr, narr, cols, x.ctypes.data, yarr) == 0
        outs.append(ys)
    for a, b in zip(*outs):
        assert bits_equal(a, b)


@pytest.mark.parametrize("type_", [S.T_Q4_K, S.T_Q6_K, S.T_Q8_0, S.T_Q4_0, S.T_Q3_K, S.T_F16])
@pytest.mark.parametrize("nb", [4, 64])
def test_matmul_call_site(pair, type_, nb):
    """matmul (3004): under 8 tokens the reference runs matvec per token (bit-exact); at 64 the
    device's prompt GEMM replaces gemm_kquant / gemm_q32 (Q4_0: bit-exact with gemm_q32's order);
    Q3_K and F16 have no GEMM: the row kernel per token on both sides, bit-exact at every batch."""
    hip, cpu = pair
    rows, cols = 1024, 4096
    w = S.weights(type_, rows, cols, 500 + type_)
    X = np.stack([S.activations(cols, 600 + b) for b in range(nb)])
    print(f"matmul {S.TYPE_NAME[type_]} nb={nb}", flush=True)
    Y = hip.matmul(type_, w, cols, X, True)
    Yref = cpu.matmul(type_, w, cols, X, type_ in REPACKS)
    if nb < 8 or type_ in (S.T_Q4_0, S.T_Q3_K, S.T_F16):
        assert bits_equal(Y, Yref)
    else:
        for t in range(nb):
            e = rel_err(Y[t], Yref[t])
            assert e <= TOL, f"token {t}: rel err {e:.3e}"


@pytest.mark.parametrize("types", [(S.T_Q4_K,) * 3, (S.T_Q4_K, S.T_Q4_K, S.T_Q6_K)])
def test_moe_ffn_call_site(pair, types):
    """moe_ffn (4588): after the router matvec, the patched call hands routing, experts and the
    weighted sum to fgh_moe_ffn, token by token as forward_chunk calls it (5089-5091)."""
    hip, cpu = pair
    n_expert, k, n_embd, ff, n_tok = 32, 4, 1024, 512, 6
    g = S.weights(types[0], n_expert * ff, n_embd, 700)
    u = S.weights(types[1], n_expert * ff, n_embd, 701)
    d = S.weights(types[2], n_expert * n_embd, ff, 702)
    X = np.stack([S.activations(n_embd, 710 + t) for t in range(n_tok)])
    X[:, 0] = 1.0
    logits = np.random.default_rng(7).standard_normal((n_tok, n_expert)).astype(np.float32)
    st0 = hip.hip_state()
    a = hip.moe_ffn(types, g, u, d, n_expert, k, n_embd, ff, logits, X)
    st1 = hip.hip_state()
    assert st1[0] == 1 and st1[1] == st0[1] + 3, (st0, st1)
    b = cpu.moe_ffn(types, g, u, d, n_expert, k, n_embd, ff, logits, X)
    for name, p, q in zip(("Y", "sel", "w"), a, b):
        assert np.array_equal(p, q) and bits_equal(p, q), name


FALLBACK = r"""
import json, sys
sys.path.insert(0, sys.argv[1]); sys.path.insert(0, sys.argv[1] + "/oracle")
import numpy as np
from fastgguf_amd import synth as S
from oracle import Reference
hip, cpu = Reference("hip"), Reference("avx2")
out = {"init": hip.hip_init(0), "calls": []}
w = S.weights(S.T_Q4_K, 512, 2048, 800)
for i in range(3):
    x = S.activations(2048, 810 + i)
    y = hip.matvec(S.T_Q4_K, w, 2048, x, True)
    st = hip.hip_state()[0]
    same_rp = bool(np.array_equal(y.view(np.uint32), cpu.matvec(S.T_Q4_K, w, 2048, x, True).view(np.uint32)))
    same_row = bool(np.array_equal(y.view(np.uint32), cpu.matvec(S.T_Q4_K, w, 2048, x, False).view(np.uint32)))
    out["calls"].append([st, same_rp, same_row])
print(json.dumps(out))
"""


def test_failed_device_call_falls_back_to_the_cpu():
    """A device call that fails (FGH_FAIL_AT=2 makes the second compute call fail before it
    launches) takes the reference's own fallback (2577-2581): the message, g_gpu.state = -1, and the
    CPU kernels from then on. A tensor on the device was never repacked (repack_tensor skips it,
    2487), so the failed call's CPU recomputation runs the row order, as the reference's does; the
    harness makes a fresh tensor per call, and the next one, made with the device off, is repacked
    for the CPU as at load."""
    _need(HIP_SO)
    env = dict(os.environ, FGH_FAIL_AT="2")
    print("fallback subprocess (FGH_FAIL_AT=2)", flush=True)
    r = subprocess.run([sys.executable, "-c", FALLBACK, ROOT], capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["init"] == 1
    assert out["calls"] == [[1, True, False], [-1, False, True], [-1, True, False]], out
    assert "matvec failed on harness - falling back to CPU" in r.stderr and "injected failure" in r.stderr
