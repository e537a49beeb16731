"""Builds the gfx950 HIP library of the backend in-tree (fastgguf_amd/libfastgguf_hip.so).

    python -m fastgguf_amd.build          # or __graft_entry__.build()

hipcc cross-compiles for gfx950 without a GPU. Flags that matter for results:
  -ffp-contract=off   no fused multiply-add except where written (__builtin_fmaf), so the fp32
                      chains match the reference's evaluation order
  -Xclang -target-feature -Xclang -packed-fp32-ops
                      no packed fp32 instructions (the host pass warns it does not know the
                      feature; that is expected)
  -Xclang -target-feature -Xclang -dot6-insts  (and -dot4-insts)
                      no v_dot4c_i32_i8 / v_dot2c_i32_i16, the dot products whose accumulator is
                      the destination: the compiler then uses the three-operand v_dot4_i32_i8 /
                      v_dot2_i32_i16 (same values), whose accumulator can be the inline constant
                      0, instead of copying a zero into a register before every product that
                      starts a sum (the grouped MoE kernel: 2373 -> 1774 VALU instructions), and
                      inserts the wait states those need itself.

Division and square root stay IEEE-correct (hipcc's default), which the bit-exact quantizers need.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libfastgguf_hip.so")
SOURCES = ["fgh_api.hip", "fgh_kernels.hip", "fgh_matvec.hip", "fgh_q4k.hip", "fgh_moemm.hip", "fgh_gemm.hip", "fgh_gemm32.hip",
           "fgh_gemm32n.hip", "fgh_gemm6.hip", "fgh_moe.hip", "fgh_gguf.hip", "fgh_attn.hip", "fgh_kvq.hip",
           "fgh_kq.hip", "fgh_float.hip"]
# per-source additions: the nibble-type GEMM converts every MFMA result with a VALU instruction, so
# its results go to VGPRs (without the flag the compiler writes them to AGPRs and copies each out)
FILE_FLAGS = {"fgh_gemm32n.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"], "fgh_moemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
             "-ffp-contract=off", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Xclang", "-target-feature", "-Xclang", "-dot6-insts", "-Xclang", "-target-feature", "-Xclang",
             "-dot4-insts", "-Wall", "-Wno-unused-function", "-fvisibility=hidden",
             "-I", os.path.join(ROOT, "include")]
_NOISE = ("packed-fp32-ops", "dot6-insts", "dot4-insts")


def _run(cmd: list[str]) -> tuple[int, str]:
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if not any(f in l for f in _NOISE) and l.strip())
    return r.returncode, err


def build(verbose: bool = True, jobs: int | None = None) -> str:
    """Compiles each source to an object in parallel (every kernel is launched from its own
    translation unit, so no device code crosses files), then links the shared library."""
    from concurrent.futures import ThreadPoolExecutor
    odir = os.path.join(HERE, "_build")
    os.makedirs(odir, exist_ok=True)
    objs = [os.path.join(odir, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    cmds = [[HIPCC] + HIP_FLAGS + FILE_FLAGS.get(s, []) + ["-c", "-o", o, os.path.join(CSRC, s)]
            for s, o in zip(SOURCES, objs)]
    if verbose:
        print(" ".join(cmds[0][:-3]) + " -c <each source>", flush=True)
    jobs = jobs or min(len(cmds), max(1, int(os.environ.get("MAX_JOBS", "0")) or (os.cpu_count() or 4)))
    with ThreadPoolExecutor(jobs) as ex:
        results = list(ex.map(_run, cmds))
    for (rc, err), s in zip(results, SOURCES):
        if rc != 0:
            raise RuntimeError(f"hipcc failed on {s} ({rc}):\n{err}")
        if verbose and err:
            print(err, file=sys.stderr)
    tmp = LIB + ".tmp"
    rc, err = _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-Wl,-z,defs", "-o", tmp] + objs)
    if rc != 0:
        raise RuntimeError(f"link failed ({rc}):\n{err}")
    os.replace(tmp, LIB)
    return LIB


def build_oracle(verbose: bool = True) -> None:
    """Builds oracle/liboracle.so (the CPU parity checker) and, where /root/reference exists, the
    reference kernels into oracle/_ref/."""
    odir = os.path.join(ROOT, "oracle")
    targets = ["all"]
    if os.path.exists("/root/reference/fastgguf.c"):
        targets += ["ref", "ref-hip"]
    r = subprocess.run(["make", "-C", odir, "-B"] + targets, capture_output=True, text=True)
    if verbose:
        print(r.stdout[-2000:], flush=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{r.stderr[-4000:]}")


C_CALLER = os.path.join(ROOT, "tests", "c_abi", "_build", "abi_smoke")


def build_c_caller() -> str:
    """Builds the plain C caller of the ABI (tests/c_abi/abi_smoke.c) with gcc against the header
    and the library, as fastgguf.c would link it; its device branch runs in the GPU suite."""
    os.makedirs(os.path.dirname(C_CALLER), exist_ok=True)
    rc, err = _run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "c_abi", "abi_smoke.c"), "-o", C_CALLER, "-L", HERE,
                    "-lfastgguf_hip", "-Wl,-rpath,$ORIGIN/../../../fastgguf_amd"])
    if rc != 0:
        raise RuntimeError(f"C caller build failed ({rc}):\n{err}")
    return C_CALLER


if __name__ == "__main__":
    build()
    build_oracle()
    build_c_caller()
