"""Python binding of the C ABI in include/fastgguf_hip.h (ctypes; no torch).

The class and method names mirror the reference engine's offload and dispatch surface
(fastgguf.c): `Backend` plays g_gpu (fg_gpu_init 2057, gpu_upload_tensor 2060), and
`matvec` / `matvec_multi` / `matmul` / `moe_ffn` take the arguments of the reference functions
of the same names (2575, 2552, 3004, 4588). Every method raises `BackendError` carrying the
library's status and message when the device call fails; nothing here computes on the CPU.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from .synth import BLOCK, K256Q8_TYPES, Q8_BLK, Q8K_BLK, T_Q4_K, T_Q5_0, T_Q5_K, T_Q6_K, T_Q8_0, row_bytes

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libfastgguf_hip.so")

OK, ERR, ERR_ARG, SKIP_TYPE, SKIP_MEM, ERR_DEVICE = 0, -1, -2, -3, -4, -5
ORDER_AUTO, ORDER_ROW, ORDER_REPACKED = -1, 0, 1
ACT_Q8, ACT_Q8K = 1, 2

#: every symbol include/fastgguf_hip.h declares
EXPORTS = (
    "fgh_open", "fgh_close", "fgh_info", "fgh_last_error", "fgh_upload", "fgh_tensor_free",
    "fgh_matvec", "fgh_matvec_multi", "fgh_matmul", "fgh_moe_ffn", "fgh_attention",
    "fgh_matvec_dev", "fgh_matvec_multi_dev", "fgh_matvec_silu_dev", "fgh_matvec_gate_up_silu_dev", "fgh_ffn_dev", "fgh_matmul_dev", "fgh_matmul_dev_noalloc", "fgh_moe_ffn_dev",
    "fgh_attention_dev", "fgh_kvq_store_dev", "fgh_kvq_attention_dev",
    "fgh_graph_begin", "fgh_graph_end", "fgh_graph_launch", "fgh_graph_destroy",
    "fgh_dev_alloc", "fgh_dev_free", "fgh_copy_h2d", "fgh_copy_d2h", "fgh_copy_d2d", "fgh_checksum_dev", "fgh_memcpy_dev", "fgh_mfma_peak_dev", "fgh_sync",
    "fgh_event_create", "fgh_event_record", "fgh_event_elapsed_ms", "fgh_event_destroy",
    "fgh_quantize", "fgh_block_ints", "fgh_gemm_block_ints", "fgh_moe_block_ints", "fgh_expf", "fgh_fp16_to_f32", "fgh_matvec_shape",
    "fgh_gguf_open", "fgh_gguf_close", "fgh_gguf_summary", "fgh_gguf_tensor", "fgh_gguf_find",
    "fgh_gguf_kv_num", "fgh_gguf_kv_str", "fgh_gguf_data", "fgh_upload_gguf",
)


class BackendError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"fastgguf_hip status {status}: {msg}")
        self.status = status


class GgufTensorT(C.Structure):
    _fields_ = [("name", C.c_char * 128), ("type", C.c_uint32), ("n_dims", C.c_int32), ("ne", C.c_uint64 * 4),
                ("offset", C.c_uint64), ("nbytes", C.c_uint64)]


class InfoT(C.Structure):
    _fields_ = [("vram", C.c_uint64), ("budget", C.c_uint64), ("used", C.c_uint64),
                ("n_offloaded", C.c_int32), ("n_skip_type", C.c_int32), ("n_skip_mem", C.c_int32),
                ("device", C.c_int32), ("name", C.c_char * 96)]


_LIB = None


def load_library(path: str = LIB_PATH) -> C.CDLL:
    """Loads the built HIP library. Raises if it is missing: there is no fallback path."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built; run `python -m fastgguf_amd.build`")
    L = C.CDLL(path)
    vp, i32, i64, u32, u64, f32p = C.c_void_p, C.c_int, C.c_int64, C.c_uint32, C.c_uint64, C.c_void_p
    sig = {
        "fgh_open": (i32, [i32, u64, C.POINTER(vp)]),
        "fgh_close": (None, [vp]),
        "fgh_info": (i32, [vp, C.POINTER(InfoT)]),
        "fgh_last_error": (C.c_char_p, [vp]),
        "fgh_upload": (i32, [vp, u32, i64, i64, i64, i32, vp, u64, C.POINTER(vp)]),
        "fgh_tensor_free": (None, [vp]),
        "fgh_matvec": (i32, [vp, vp, f32p, f32p]),
        "fgh_matvec_multi": (i32, [vp, i32, vp, f32p, vp]),
        "fgh_matmul": (i32, [vp, vp, f32p, i32, f32p, i32, i32]),
        "fgh_moe_ffn": (i32, [vp, vp, vp, vp, i32, f32p, f32p, f32p, i32, vp, vp]),
        "fgh_matvec_dev": (i32, [vp, vp, vp, vp]),
        "fgh_matvec_multi_dev": (i32, [vp, i32, vp, vp, vp]),
        "fgh_matvec_silu_dev": (i32, [vp, vp, vp, vp, vp]),
        "fgh_matvec_gate_up_silu_dev": (i32, [vp, vp, vp, vp, vp]),
        "fgh_ffn_dev": (i32, [vp, vp, vp, vp, vp, vp, vp]),
        "fgh_matmul_dev": (i32, [vp, vp, vp, i32, vp, i32, i32]),
        "fgh_matmul_dev_noalloc": (i32, [vp, vp, vp, i32, vp, i32, i32]),
        "fgh_moe_ffn_dev": (i32, [vp, vp, vp, vp, i32, vp, vp, vp, i32]),
        "fgh_attention": (i32, [vp, i32, i32, i32, i32, vp, vp, vp, vp, i32, i32, vp, vp, C.c_float]),
        "fgh_attention_dev": (i32, [vp, i32, i32, i32, i32, vp, vp, vp, vp, i32, i32, vp, vp, i32, C.c_float]),
        "fgh_kvq_store_dev": (i32, [vp, i32, i32, i32, i32, i32, vp, vp, i32, vp, vp, i32, vp]),
        "fgh_kvq_attention_dev": (i32, [vp, i32, i32, i32, i32, i32, i32, vp, vp, vp, vp, i32, vp, vp, i32,
                                        C.c_float]),
        "fgh_graph_begin": (i32, [vp]),
        "fgh_graph_end": (i32, [vp, C.POINTER(vp)]),
        "fgh_graph_launch": (i32, [vp, vp]),
        "fgh_graph_destroy": (i32, [vp, vp]),
        "fgh_dev_alloc": (i32, [vp, u64, C.POINTER(vp)]),
        "fgh_dev_free": (i32, [vp, vp]),
        "fgh_copy_h2d": (i32, [vp, vp, vp, u64]),
        "fgh_copy_d2h": (i32, [vp, vp, vp, u64]),
        "fgh_copy_d2d": (i32, [vp, vp, vp, u64]),
        "fgh_checksum_dev": (i32, [vp, vp, u64, vp]),
        "fgh_memcpy_dev": (i32, [vp, vp, vp, u64]),
        "fgh_mfma_peak_dev": (i32, [vp, i32, C.POINTER(u64)]),
        "fgh_sync": (i32, [vp]),
        "fgh_event_create": (i32, [vp, C.POINTER(vp)]),
        "fgh_event_record": (i32, [vp, vp]),
        "fgh_event_elapsed_ms": (i32, [vp, vp, vp, C.POINTER(C.c_float)]),
        "fgh_event_destroy": (i32, [vp, vp]),
        "fgh_quantize": (i32, [vp, i32, f32p, i32, vp]),
        "fgh_block_ints": (i32, [vp, vp, f32p, vp, vp]),
        "fgh_gemm_block_ints": (i32, [vp, vp, f32p, i32, i32, vp, vp]),
        "fgh_moe_block_ints": (i32, [vp, vp, vp, vp, i32, f32p, f32p, i32, vp, vp, vp, vp]),
        "fgh_fp16_to_f32": (i32, [vp, vp, i32, vp]),
        "fgh_expf": (i32, [vp, f32p, i32, vp]),
        "fgh_matvec_shape": (i32, [vp, u32, i32, i64, i64, i32, vp]),
        "fgh_gguf_open": (i32, [C.c_char_p, C.POINTER(vp), C.c_char_p, C.c_size_t]),
        "fgh_gguf_close": (None, [vp]),
        "fgh_gguf_summary": (i32, [vp, C.POINTER(u32), C.POINTER(u64), C.POINTER(i64), C.POINTER(i64)]),
        "fgh_gguf_tensor": (i32, [vp, i64, C.POINTER(GgufTensorT)]),
        "fgh_gguf_find": (i64, [vp, C.c_char_p]),
        "fgh_gguf_kv_num": (i32, [vp, C.c_char_p, C.c_double, C.POINTER(C.c_double)]),
        "fgh_gguf_kv_str": (C.c_char_p, [vp, C.c_char_p]),
        "fgh_gguf_data": (vp, [vp, i64]),
        "fgh_upload_gguf": (i32, [vp, vp, i64, i32, C.POINTER(vp)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = L
    return L


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


class Tensor:
    """A device copy of one GGUF tensor (the reference's tensor_t.gpu, fastgguf.c:274)."""

    def __init__(self, backend: "Backend", handle: int, type_: int, cols: int, rows: int, n_mats: int):
        self.backend, self.handle = backend, handle
        self.type, self.cols, self.rows, self.n_mats = type_, cols, rows, n_mats

    @property
    def nout(self) -> int:
        return self.rows * self.n_mats

    @property
    def nblocks(self) -> int:
        return self.cols // BLOCK[self.type][0]

    def free(self):
        if self.handle:
            self.backend.lib.fgh_tensor_free(self.handle)
            self.handle = None


class Gguf:
    """A mapped GGUF file (gguf_open, fastgguf.c:342-440); needs no device."""

    def __init__(self, path: str):
        self.lib = load_library()
        h = C.c_void_p()
        err = C.create_string_buffer(256)
        rc = self.lib.fgh_gguf_open(os.fsencode(path), C.byref(h), err, len(err))
        if rc != OK:
            raise BackendError(rc, err.value.decode(errors="replace"))
        self.handle = h

    def close(self):
        if self.handle:
            self.lib.fgh_gguf_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def summary(self) -> dict:
        v, a, nk, nt = C.c_uint32(), C.c_uint64(), C.c_int64(), C.c_int64()
        self.lib.fgh_gguf_summary(self.handle, C.byref(v), C.byref(a), C.byref(nk), C.byref(nt))
        return {"version": v.value, "alignment": a.value, "n_kvs": nk.value, "n_tensors": nt.value}

    def tensor(self, i: int) -> dict:
        t = GgufTensorT()
        if self.lib.fgh_gguf_tensor(self.handle, i, C.byref(t)) != OK:
            raise IndexError(i)
        return {"name": t.name.decode(errors="replace"), "type": t.type, "n_dims": t.n_dims, "ne": list(t.ne)[: t.n_dims],
                "offset": t.offset, "nbytes": t.nbytes}

    def tensors(self) -> list[dict]:
        return [self.tensor(i) for i in range(self.summary()["n_tensors"])]

    def find(self, name: str) -> int:
        return self.lib.fgh_gguf_find(self.handle, name.encode())

    def kv_num(self, key: str, default: float = 0.0) -> float:
        out = C.c_double()
        self.lib.fgh_gguf_kv_num(self.handle, key.encode(), default, C.byref(out))
        return out.value

    def kv_str(self, key: str) -> str | None:
        v = self.lib.fgh_gguf_kv_str(self.handle, key.encode())
        return None if v is None else v.decode()

    def data(self, i: int) -> np.ndarray:
        """A tensor's bytes, read from the mapping (a copy)."""
        info = self.tensor(i)
        p = self.lib.fgh_gguf_data(self.handle, i)
        return np.ctypeslib.as_array((C.c_uint8 * info["nbytes"]).from_address(p)).copy()


class Backend:
    """One device context (fg_gpu_init, fastgguf.c:1968-2057)."""

    def __init__(self, device: int = 0, budget_bytes: int = 0):
        self.lib = load_library()
        h = C.c_void_p()
        rc = self.lib.fgh_open(device, budget_bytes, C.byref(h))
        if rc != OK:
            raise BackendError(rc, "fgh_open failed (no usable gfx950 device)")
        self.ctx = h

    def close(self):
        if self.ctx:
            self.lib.fgh_close(self.ctx)
            self.ctx = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _check(self, rc: int):
        if rc != OK:
            raise BackendError(rc, self.lib.fgh_last_error(self.ctx).decode())

    def info(self) -> dict:
        i = InfoT()
        self._check(self.lib.fgh_info(self.ctx, C.byref(i)))
        return {f: (getattr(i, f).decode() if f == "name" else getattr(i, f)) for f, _ in InfoT._fields_}

    # -- gpu_upload_tensor (2060)
    def upload(self, type_: int, cols: int, data: np.ndarray, rows: int | None = None, n_mats: int = 1,
               order: int = ORDER_AUTO) -> Tensor:
        data = np.ascontiguousarray(data, np.uint8)
        if rows is None:
            rows = data.size // (row_bytes(type_, cols) * n_mats)
        h = C.c_void_p()
        self._check(self.lib.fgh_upload(self.ctx, type_, cols, rows, n_mats, order, _p(data), data.size,
                                        C.byref(h)))
        return Tensor(self, h.value, type_, cols, rows, n_mats)

    # -- gpu_upload_tensor (2060) on a tensor of a mapped GGUF file
    def upload_gguf(self, g: Gguf, name_or_index, order: int = ORDER_AUTO) -> Tensor:
        i = g.find(name_or_index) if isinstance(name_or_index, str) else int(name_or_index)
        if i < 0:
            raise KeyError(name_or_index)
        info = g.tensor(i)
        ne = info["ne"] + [1] * (4 - len(info["ne"]))
        h = C.c_void_p()
        self._check(self.lib.fgh_upload_gguf(self.ctx, g.handle, i, order, C.byref(h)))
        return Tensor(self, h.value, info["type"], ne[0], ne[1], ne[2] * ne[3])

    # -- matvec (2575)
    def matvec(self, t: Tensor, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        if x.size != t.cols:
            raise ValueError("x length != cols")
        y = np.empty(t.nout, np.float32)
        self._check(self.lib.fgh_matvec(self.ctx, t.handle, _p(x), _p(y)))
        return y

    # -- matvec_multi (2552)
    def matvec_multi(self, ts: list[Tensor], x: np.ndarray) -> list[np.ndarray]:
        x = np.ascontiguousarray(x, np.float32)
        ys = [np.empty(t.nout, np.float32) for t in ts]
        th = (C.c_void_p * len(ts))(*[t.handle for t in ts])
        yp = (C.c_void_p * len(ts))(*[y.ctypes.data for y in ys])
        self._check(self.lib.fgh_matvec_multi(self.ctx, len(ts), th, _p(x), yp))
        return ys

    # -- matmul (3004): X [nb, cols] -> Y [nb, rows]
    def matmul(self, t: Tensor, X: np.ndarray) -> np.ndarray:
        X = np.ascontiguousarray(X, np.float32)
        nb = X.shape[0]
        Y = np.empty((nb, t.nout), np.float32)
        self._check(self.lib.fgh_matmul(self.ctx, t.handle, _p(X), t.cols, _p(Y), t.nout, nb))
        return Y

    # -- moe_ffn (4588) for n_tok tokens
    def moe_ffn(self, gate: Tensor, up: Tensor, down: Tensor, k: int, logits: np.ndarray, X: np.ndarray):
        X = np.ascontiguousarray(X, np.float32)
        logits = np.ascontiguousarray(logits, np.float32)
        n_tok = X.shape[0]
        Y = np.empty((n_tok, down.rows), np.float32)
        sel = np.empty((n_tok, k), np.int32)
        w = np.empty((n_tok, k), np.float32)
        self._check(self.lib.fgh_moe_ffn(self.ctx, gate.handle, up.handle, down.handle, k, _p(logits), _p(X),
                                         _p(Y), n_tok, _p(sel), _p(w)))
        return Y, sel, w

    # -- test hooks
    def quantize_q8(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros(x.size // 32, Q8_BLK)
        self._check(self.lib.fgh_quantize(self.ctx, ACT_Q8, _p(x), x.size, _p(out)))
        return out

    def quantize_q8k(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros(x.size // 256, Q8K_BLK)
        self._check(self.lib.fgh_quantize(self.ctx, ACT_Q8K, _p(x), x.size, _p(out)))
        return out

    def block_ints(self, t: Tensor, x: np.ndarray):
        """Per (row, block) integers of the decode kernel: sumi, msum [nout][blocks]; Q2_K, Q3_K and
        IQ4_XS per 32-value block, the units of their chains."""
        x = np.ascontiguousarray(x, np.float32)
        nbk = t.cols // 32 if t.type in K256Q8_TYPES else t.nblocks
        s = np.empty((t.nout, nbk), np.int32)
        m = np.empty((t.nout, nbk), np.int32)
        self._check(self.lib.fgh_block_ints(self.ctx, t.handle, _p(x), _p(s), _p(m)))
        return s, m

    def gemm_block_ints(self, t: Tensor, X: np.ndarray):
        """Per (token, row, block) integers of the prompt GEMM (Q4_K, Q6_K or Q8_0, 8..64 tokens): sumi, msum
        [nb][nout][blocks] (msum zeros for Q8_0)."""
        X = np.ascontiguousarray(X, np.float32)
        nb = X.shape[0]
        s = np.empty((nb, t.nout, t.nblocks), np.int32)
        m = np.empty((nb, t.nout, t.nblocks), np.int32)
        self._check(self.lib.fgh_gemm_block_ints(self.ctx, t.handle, _p(X), t.cols, nb, _p(s), _p(m)))
        return s, m

    def moe_block_ints(self, gate: Tensor, up: Tensor, down: Tensor, k: int, logits: np.ndarray, X: np.ndarray):
        """The grouped MoE path's per (slot, row, block) integers: gate sumi / msum [n_tok * k][ff][blocks],
        down sumi / msum [n_tok * k][n_embd][blocks] (slot t * k + j: token t's j-th expert)."""
        X = np.ascontiguousarray(X, np.float32)
        logits = np.ascontiguousarray(logits, np.float32)
        np_ = X.shape[0] * k
        gs = np.empty((np_, gate.rows, gate.nblocks), np.int32)
        gm = np.empty_like(gs)
        ds = np.empty((np_, down.rows, down.nblocks), np.int32)
        dm = np.empty_like(ds)
        self._check(self.lib.fgh_moe_block_ints(self.ctx, gate.handle, up.handle, down.handle, k, _p(logits), _p(X),
                                                X.shape[0], _p(gs), _p(gm), _p(ds), _p(dm)))
        return gs, gm, ds, dm

    def expf(self, x: np.ndarray) -> np.ndarray:
        """The device's expf (MoE softmax and silu) of every value of x."""
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(x.size, np.float32)
        self._check(self.lib.fgh_expf(self.ctx, _p(x), x.size, _p(out)))
        return out

    def matvec_shape(self, ggml_type: int, order: int, cols: int, row_tiles: int, ntok: int = 1) -> tuple:
        """(wavefronts per tile, ring depth, tiles per workgroup, LDS bytes) of the decode launch over
        row_tiles row tiles (all tensors of the launch) and ntok tokens."""
        out = np.zeros(4, np.int32)
        self._check(self.lib.fgh_matvec_shape(self.ctx, ggml_type, order, cols, row_tiles, ntok, _p(out)))
        return tuple(int(v) for v in out)

    def fp16_to_f32(self, h: np.ndarray) -> np.ndarray:
        h = np.ascontiguousarray(h, np.uint16)
        out = np.empty(h.size, np.float32)
        self._check(self.lib.fgh_fp16_to_f32(self.ctx, _p(h), h.size, _p(out)))
        return out

    # -- device memory / events (device-resident callers, benchmarks)
    def dev_alloc(self, nbytes: int) -> int:
        p = C.c_void_p()
        self._check(self.lib.fgh_dev_alloc(self.ctx, nbytes, C.byref(p)))
        return p.value

    def dev_free(self, p: int):
        self._check(self.lib.fgh_dev_free(self.ctx, p))

    def h2d(self, dst: int, a: np.ndarray):
        a = np.ascontiguousarray(a)
        self._check(self.lib.fgh_copy_h2d(self.ctx, dst, _p(a), a.nbytes))

    def d2h(self, a: np.ndarray, src: int):
        self._check(self.lib.fgh_copy_d2h(self.ctx, _p(a), src, a.nbytes))

    def d2d(self, dst: int, src: int, nbytes: int):
        self._check(self.lib.fgh_copy_d2d(self.ctx, dst, src, nbytes))

    def memcpy_dev(self, dst: int, src: int, nbytes: int):
        """hipMemcpyAsync device to device on the context stream (the runtime's copy)."""
        self._check(self.lib.fgh_memcpy_dev(self.ctx, dst, src, nbytes))

    def checksum_dev(self, src: int, nbytes: int, out: int):
        """Wrapping 32-bit word sum of nbytes at src, into the device word at out (asynchronous)."""
        self._check(self.lib.fgh_checksum_dev(self.ctx, src, nbytes, out))

    def mfma_peak_dev(self, iters: int) -> int:
        """One launch of the MFMA-only rate probe (asynchronous); returns its int8 operations."""
        ops = C.c_uint64()
        self._check(self.lib.fgh_mfma_peak_dev(self.ctx, iters, C.byref(ops)))
        return ops.value

    def checksum(self, src: int, nbytes: int) -> int:
        out = self.dev_alloc(16)
        try:
            self.checksum_dev(src, nbytes, out)
            v = np.zeros(4, dtype=np.uint32)
            self.d2h(v, out)
            return int(v[0])
        finally:
            self.dev_free(out)

    def sync(self):
        self._check(self.lib.fgh_sync(self.ctx))

    def event(self) -> int:
        e = C.c_void_p()
        self._check(self.lib.fgh_event_create(self.ctx, C.byref(e)))
        return e.value

    def record(self, ev: int):
        self._check(self.lib.fgh_event_record(self.ctx, ev))

    def elapsed_ms(self, a: int, b: int) -> float:
        ms = C.c_float()
        self._check(self.lib.fgh_event_elapsed_ms(self.ctx, a, b, C.byref(ms)))
        return ms.value

    def event_destroy(self, ev: int):
        self._check(self.lib.fgh_event_destroy(self.ctx, ev))

    def matvec_dev(self, t: Tensor, x_dev: int, y_dev: int):
        self._check(self.lib.fgh_matvec_dev(self.ctx, t.handle, x_dev, y_dev))

    def matvec_silu_dev(self, t: Tensor, g_dev: int, u_dev: int, y_dev: int):
        """y = t * Q8(silu(g) * u), the dense FFN's down projection (device pointers)."""
        self._check(self.lib.fgh_matvec_silu_dev(self.ctx, t.handle, g_dev, u_dev, y_dev))

    def matvec_silu(self, t: Tensor, g: np.ndarray, u: np.ndarray) -> np.ndarray:
        """The same from host arrays (copies in and out; for tests)."""
        g = np.ascontiguousarray(g, dtype=np.float32)
        u = np.ascontiguousarray(u, dtype=np.float32)
        nout = t.rows * t.n_mats
        gd, ud, yd = self.dev_alloc(g.nbytes), self.dev_alloc(u.nbytes), self.dev_alloc(4 * nout)
        try:
            self.h2d(gd, g)
            self.h2d(ud, u)
            self.matvec_silu_dev(t, gd, ud, yd)
            y = np.empty(nout, dtype=np.float32)
            self.d2h(y, yd)
            return y
        finally:
            for p in (gd, ud, yd):
                self.dev_free(p)

    def matvec_gate_up_silu_dev(self, gate: Tensor, up: Tensor, x_dev: int, h_dev: int):
        """h = silu(gate * Q(x)) * (up * Q(x)), the dense FFN's gate / up and the loop before
        its down projection (device pointers)."""
        self._check(self.lib.fgh_matvec_gate_up_silu_dev(self.ctx, gate.handle, up.handle, x_dev, h_dev))

    def ffn_dev(self, gate: Tensor, up: Tensor, down: Tensor, x_dev: int, h_dev: int, y_dev: int) -> None:
        """The dense SiLU FFN of one token (fgh_ffn_dev): h = silu(gate x) * (up x), y = down h."""
        self._check(self.lib.fgh_ffn_dev(self.ctx, gate.handle, up.handle, down.handle, x_dev, h_dev, y_dev))

    def matvec_gate_up_silu(self, gate: Tensor, up: Tensor, x: np.ndarray) -> np.ndarray:
        """The same from a host array (copies in and out; for tests)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        xd, hd = self.dev_alloc(x.nbytes), self.dev_alloc(4 * gate.rows)
        try:
            self.h2d(xd, x)
            self.matvec_gate_up_silu_dev(gate, up, xd, hd)
            h = np.empty(gate.rows, dtype=np.float32)
            self.d2h(h, hd)
            return h
        finally:
            for p in (xd, hd):
                self.dev_free(p)

    def matvec_multi_dev(self, ts: list[Tensor], x_dev: int, y_devs: list[int]):
        th = (C.c_void_p * len(ts))(*[t.handle for t in ts])
        yp = (C.c_void_p * len(ts))(*y_devs)
        self._check(self.lib.fgh_matvec_multi_dev(self.ctx, len(ts), th, x_dev, yp))

    def graph_begin(self):
        self._check(self.lib.fgh_graph_begin(self.ctx))

    def graph_end(self) -> int:
        g = C.c_void_p()
        self._check(self.lib.fgh_graph_end(self.ctx, C.byref(g)))
        return g.value

    def graph_launch(self, g: int):
        self._check(self.lib.fgh_graph_launch(self.ctx, g))

    def graph_destroy(self, g: int):
        self._check(self.lib.fgh_graph_destroy(self.ctx, g))

    def matmul_dev(self, t: Tensor, X_dev: int, Y_dev: int, nb: int):
        self._check(self.lib.fgh_matmul_dev(self.ctx, t.handle, X_dev, t.cols, Y_dev, t.nout, nb))

    def matmul_dev_noalloc(self, t: Tensor, X_dev: int, Y_dev: int, nb: int):
        """matmul_dev with the prompt GEMM's scratch in the library's static per-device array"""
        self._check(self.lib.fgh_matmul_dev_noalloc(self.ctx, t.handle, X_dev, t.cols, Y_dev, t.nout, nb))

    def moe_ffn_dev(self, gate: Tensor, up: Tensor, down: Tensor, k: int, logits_dev: int, X_dev: int,
                    Y_dev: int, n_tok: int):
        self._check(self.lib.fgh_moe_ffn_dev(self.ctx, gate.handle, up.handle, down.handle, k, logits_dev, X_dev,
                                             Y_dev, n_tok))

    def attention(self, q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, st, en, n_head_kv: int,
                  scale: float) -> np.ndarray:
        """attn_rows over every (token, head): q [n_tok][n_head][hd], caches [cap][kv_dim], st / en
        position ranges per token (slot = position % cap). Returns o shaped like q."""
        q = np.ascontiguousarray(q, dtype=np.float32)
        k_cache = np.ascontiguousarray(k_cache, dtype=np.float32)
        v_cache = np.ascontiguousarray(v_cache, dtype=np.float32)
        if q.ndim != 3 or k_cache.ndim != 2 or k_cache.shape != v_cache.shape:
            raise ValueError("attention: q is [n_tok][n_head][hd], caches are [cap][kv_dim]")
        n_tok, n_head, hd = q.shape
        st = np.ascontiguousarray(st, dtype=np.int32)
        en = np.ascontiguousarray(en, dtype=np.int32)
        if st.shape != (n_tok,) or en.shape != (n_tok,):
            raise ValueError("attention: st and en hold one position per token")
        o = np.empty_like(q)
        self._check(self.lib.fgh_attention(self.ctx, n_tok, n_head, n_head_kv, hd, q.ctypes.data, o.ctypes.data,
                                           k_cache.ctypes.data, v_cache.ctypes.data, k_cache.shape[1],
                                           k_cache.shape[0], st.ctypes.data, en.ctypes.data, scale))
        return o

    def attention_dev(self, n_tok: int, n_head: int, n_head_kv: int, hd: int, q_dev: int, o_dev: int,
                      k_dev: int, v_dev: int, kv_dim: int, cap: int, st_dev: int, en_dev: int, max_len: int,
                      scale: float):
        self._check(self.lib.fgh_attention_dev(self.ctx, n_tok, n_head, n_head_kv, hd, q_dev, o_dev, k_dev, v_dev,
                                               kv_dim, cap, st_dev, en_dev, max_len, scale))

    def kvq_store_dev(self, n_tok, n_head_kv, hd, kbits, vbits, k_dev, v_dev, stride, kq_dev, vq_dev, cap, pos_dev):
        self._check(self.lib.fgh_kvq_store_dev(self.ctx, n_tok, n_head_kv, hd, kbits, vbits, k_dev, v_dev, stride,
                                               kq_dev, vq_dev, cap, pos_dev))

    def kvq_attention_dev(self, n_tok, n_head, n_head_kv, hd, kbits, vbits, q_dev, o_dev, kq_dev, vq_dev, cap,
                          st_dev, en_dev, max_len, scale):
        self._check(self.lib.fgh_kvq_attention_dev(self.ctx, n_tok, n_head, n_head_kv, hd, kbits, vbits, q_dev,
                                                   o_dev, kq_dev, vq_dev, cap, st_dev, en_dev, max_len, scale))

    def kvq_store(self, k, v, pos, kq, vq, kbits: int, vbits: int):
        """Writes rows k / v ([n_tok][n_head_kv][hd]) at positions pos into host copies of the
        quantized caches kq / vq ([cap][slot bytes]), on the device; returns the new caches."""
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        n_tok, nkv, hd = k.shape
        pos = np.ascontiguousarray(pos, np.int32)
        kq = np.ascontiguousarray(kq, np.uint8)
        vq = np.ascontiguousarray(vq, np.uint8)
        bufs = [self.dev_alloc(a.nbytes) for a in (k, v, pos, kq, vq)]
        try:
            for b, a in zip(bufs, (k, v, pos, kq, vq)):
                self.h2d(b, a)
            self.kvq_store_dev(n_tok, nkv, hd, kbits, vbits, bufs[0], bufs[1], nkv * hd, bufs[3], bufs[4],
                               kq.shape[0], bufs[2])
            kq2, vq2 = np.empty_like(kq), np.empty_like(vq)
            self.d2h(kq2, bufs[3])
            self.d2h(vq2, bufs[4])
            return kq2, vq2
        finally:
            for b in bufs:
                self.dev_free(b)

    def kvq_attention(self, q, kq, vq, st, en, n_head_kv: int, kbits: int, vbits: int, scale: float):
        """TurboQuant attention over host copies of the quantized caches: q [n_tok][n_head][hd]."""
        q = np.ascontiguousarray(q, np.float32)
        n_tok, n_head, hd = q.shape
        st = np.ascontiguousarray(st, np.int32)
        en = np.ascontiguousarray(en, np.int32)
        kq = np.ascontiguousarray(kq, np.uint8)
        vq = np.ascontiguousarray(vq, np.uint8)
        max_len = int(max(1, (en - st).max() + 1))
        bufs = [self.dev_alloc(a.nbytes) for a in (q, q, kq, vq, st, en)]
        try:
            for b, a in zip(bufs, (q, q, kq, vq, st, en)):
                self.h2d(b, a)
            self.kvq_attention_dev(n_tok, n_head, n_head_kv, hd, kbits, vbits, bufs[0], bufs[1], bufs[2], bufs[3],
                                   kq.shape[0], bufs[4], bufs[5], max_len, scale)
            o = np.empty_like(q)
            self.d2h(o, bufs[1])
            return o
        finally:
            for b in bufs:
                self.dev_free(b)


__all__ = ["Backend", "BackendError", "Gguf", "Tensor", "load_library", "EXPORTS", "T_Q4_K", "T_Q5_0", "T_Q5_K", "T_Q6_K", "T_Q8_0",
           "ORDER_AUTO", "ORDER_ROW", "ORDER_REPACKED"]
