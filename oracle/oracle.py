"""ctypes loader for the CPU parity oracle (test infrastructure only).

`Oracle` wraps liboracle.so, the clean-room C restatement of the reference kernels (fg_oracle.c).
`Reference` wraps oracle/_ref/libfgref_*.so, the reference's own kernels compiled from
/root/reference (built only where the reference is present; the built .so travels with the repo).
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module.
"""
from __future__ import annotations

import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
from fastgguf_amd.synth import BLOCK, FLOAT_TYPES, K256Q8_TYPES, Q8_BLK, Q8K_BLK, uses_q8  # noqa: E402

ORDER_ROW = 0
ORDER_REPACKED = 1

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def act_dtype(type_: int):
    return Q8_BLK if uses_q8(type_) else Q8K_BLK


class Oracle:
    """The restatement (fg_oracle.c)."""

    def __init__(self, path: str | None = None):
        path = path or os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} not built (run make -C oracle)")
        L = self.lib = C.CDLL(path)
        L.fgo_fp16.restype = C.c_float
        L.fgo_fp16.argtypes = [C.c_uint16]
        for n in ("fgo_quantize_q8", "fgo_quantize_q8k"):
            getattr(L, n).argtypes = [C.c_void_p, C.c_void_p, C.c_int]
            getattr(L, n).restype = None
        for n in ("fgo_dot_q8_0", "fgo_dot_q4_K", "fgo_dot_q4_K_rp", "fgo_dot_q6_K", "fgo_dot_q5_0", "fgo_dot_q5_K",
                  "fgo_dot_q4_0_rp"):
            getattr(L, n).argtypes = [C.c_void_p, C.c_void_p, C.c_int]
            getattr(L, n).restype = C.c_float
        L.fgo_dot_q32.argtypes = [C.c_uint32, C.c_void_p, C.c_void_p, C.c_int]
        L.fgo_dot_q32.restype = C.c_float
        L.fgo_dot_k256q8.argtypes = [C.c_uint32, C.c_void_p, C.c_void_p, C.c_int]
        L.fgo_dot_k256q8.restype = C.c_float
        L.fgo_dot_float.argtypes = [C.c_uint32, C.c_void_p, C.c_void_p, C.c_int]
        L.fgo_dot_float.restype = C.c_float
        L.fgo_block_ints.argtypes = [C.c_uint32, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p]
        L.fgo_matvec.argtypes = [C.c_uint32, C.c_int, C.c_void_p, C.c_int64, C.c_int, C.c_void_p, C.c_void_p]
        L.fgo_matmul.argtypes = [C.c_uint32, C.c_int, C.c_void_p, C.c_int64, C.c_int, C.c_void_p, C.c_int,
                                 C.c_void_p, C.c_int, C.c_int]
        L.fgo_gemm.argtypes = [C.c_uint32, C.c_void_p, C.c_int64, C.c_int, C.c_void_p, C.c_int, C.c_void_p,
                               C.c_int, C.c_int]
        L.fgo_moe_ffn.argtypes = [C.c_uint32] * 3 + [C.c_void_p] * 3 + [C.c_int] * 4 + \
            [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
        L.fgo_moe_down.argtypes = [C.c_uint32, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p,
                                   C.c_void_p, C.c_void_p]
        L.fgo_moe_route.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p]
        L.fgo_moe_route.restype = None
        L.fgo_silu.argtypes = [C.c_float]
        L.fgo_silu.restype = C.c_float
        L.fgo_expf_restated.argtypes = [C.c_float]
        L.fgo_expf_restated.restype = C.c_float
        L.fgo_expf_compare.argtypes = [C.c_float, C.c_float, C.c_uint32, C.POINTER(C.c_uint64), C.POINTER(C.c_int)]
        L.fgo_expf_compare.restype = C.c_uint64
        L.fgo_dequantize_row.argtypes = [C.c_uint32, C.c_void_p, C.c_void_p, C.c_int]
        L.fgo_attn_rows.argtypes = [C.c_int] + [C.c_void_p] * 6 + [C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_float]
        L.fgo_kvq_signs.argtypes = [C.c_void_p, C.c_int]
        L.fgo_kvq_rotate.argtypes = [C.c_void_p, C.c_int, C.c_int]
        L.fgo_kvq_quant.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_int]
        L.fgo_kvq_attn_rows.argtypes = [C.c_int] + [C.c_void_p] * 6 + [C.c_int, C.c_int, C.c_void_p] + \
            [C.c_int] * 4 + [C.c_float]
        L.fgo_exp_neg.argtypes = [C.c_float]
        L.fgo_exp_neg.restype = C.c_float

    # -- quantizers
    def quantize_q8(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros(x.size // 32, Q8_BLK)
        self.lib.fgo_quantize_q8(_ptr(x), _ptr(out), x.size)
        return out

    def quantize_q8k(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros(x.size // 256, Q8K_BLK)
        self.lib.fgo_quantize_q8k(_ptr(x), _ptr(out), x.size)
        return out

    def quantize_for(self, type_: int, x: np.ndarray) -> np.ndarray:
        """the activations the type's row kernel reads: x itself for the float types"""
        if type_ in FLOAT_TYPES:
            return np.ascontiguousarray(x, np.float32).copy()
        return self.quantize_q8(x) if uses_q8(type_) else self.quantize_q8k(x)

    # -- row kernels
    def dot(self, type_: int, row: np.ndarray, act: np.ndarray, order: int = ORDER_ROW) -> float:
        row = np.ascontiguousarray(row, np.uint8)
        if type_ in FLOAT_TYPES:  # act: x in fp32
            act = np.ascontiguousarray(act, np.float32)
            return self.lib.fgo_dot_float(type_, _ptr(row), _ptr(act), act.size)
        eb, _ = BLOCK[type_]
        nb = act.size
        if type_ == 2 and order == ORDER_REPACKED:
            return self.lib.fgo_dot_q4_0_rp(_ptr(row), _ptr(act), nb)
        if type_ in K256Q8_TYPES:
            return self.lib.fgo_dot_k256q8(type_, _ptr(row), _ptr(act), nb // 8)
        if uses_q8(type_):
            return self.lib.fgo_dot_q32(type_, _ptr(row), _ptr(act), nb)
        name = {12: "fgo_dot_q4_K_rp" if order == ORDER_REPACKED else "fgo_dot_q4_K",
                14: "fgo_dot_q6_K", 13: "fgo_dot_q5_K"}[type_]
        return getattr(self.lib, name)(_ptr(row), _ptr(act), nb)

    def block_ints(self, type_: int, row: np.ndarray, act: np.ndarray):
        row = np.ascontiguousarray(row, np.uint8)
        nb = act.size
        s = np.zeros(nb, np.int32)
        m = np.zeros(nb, np.int32)
        self.lib.fgo_block_ints(type_, _ptr(row), _ptr(act), nb, _ptr(s), _ptr(m))
        return s, m

    def dequantize_row(self, type_: int, raw: np.ndarray, n: int) -> np.ndarray:
        out = np.zeros(n, np.float32)
        raw = np.ascontiguousarray(raw, np.uint8)
        if self.lib.fgo_dequantize_row(type_, _ptr(raw), _ptr(out), n) != 0:
            raise ValueError("dequantize_row failed")
        return out

    # -- drivers
    def matvec(self, type_: int, w: np.ndarray, cols: int, x: np.ndarray, order: int = ORDER_ROW) -> np.ndarray:
        w = np.ascontiguousarray(w, np.uint8)
        x = np.ascontiguousarray(x, np.float32)
        rows = w.shape[0]
        y = np.zeros(rows, np.float32)
        if self.lib.fgo_matvec(type_, order, _ptr(w), rows, cols, _ptr(x), _ptr(y)) != 0:
            raise ValueError("fgo_matvec failed")
        return y

    def matmul(self, type_: int, w: np.ndarray, cols: int, X: np.ndarray, order: int = ORDER_ROW) -> np.ndarray:
        w = np.ascontiguousarray(w, np.uint8)
        X = np.ascontiguousarray(X, np.float32)
        rows, nb = w.shape[0], X.shape[0]
        Y = np.zeros((nb, rows), np.float32)
        if self.lib.fgo_matmul(type_, order, _ptr(w), rows, cols, _ptr(X), cols, _ptr(Y), rows, nb) != 0:
            raise ValueError("fgo_matmul failed")
        return Y

    def gemm(self, type_: int, w: np.ndarray, cols: int, act: np.ndarray) -> np.ndarray:
        """act: [nb, blocks] structured activation blocks."""
        w = np.ascontiguousarray(w, np.uint8)
        act = np.ascontiguousarray(act)
        rows, nb = w.shape[0], act.shape[0]
        Y = np.zeros((nb, rows), np.float32)
        if self.lib.fgo_gemm(type_, _ptr(w), rows, cols, _ptr(act), act.shape[1], _ptr(Y), rows, nb) != 0:
            raise ValueError("fgo_gemm failed")
        return Y

    def moe_route(self, logits: np.ndarray, k: int):
        logits = np.ascontiguousarray(logits, np.float32)
        sel = np.zeros(k, np.int32)
        w = np.zeros(k, np.float32)
        self.lib.fgo_moe_route(_ptr(logits), logits.size, k, _ptr(sel), _ptr(w))
        return sel, w

    def silu(self, x: float) -> float:
        return self.lib.fgo_silu(x)

    def exp_neg(self, x: float) -> float:
        """exp_neg_ps (fastgguf.c:3168-3184) on one value."""
        return float(self.lib.fgo_exp_neg(float(x)))

    def expf(self, x: float) -> float:
        return self.lib.fgo_expf_restated(x)

    def libm_expf(self, x: np.ndarray) -> np.ndarray:
        """This host's libm expf of every value (what the reference's softmax and silu call)."""
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(x.size, np.float32)
        self.lib.fgo_expf_n(_ptr(x), x.size, _ptr(out))
        return out

    def expf_compare(self, lo: float, hi: float, stride: int):
        """(mismatches, checked, max ulps) of the restated expf against libm's expf."""
        n, mu = C.c_uint64(), C.c_int()
        bad = self.lib.fgo_expf_compare(lo, hi, stride, C.byref(n), C.byref(mu))
        return int(bad), int(n.value), int(mu.value)

    def moe_ffn(self, types, gate, up, down, n_expert, k, n_embd, ff, logits, X, want_h=False):
        X = np.ascontiguousarray(X, np.float32)
        logits = np.ascontiguousarray(logits, np.float32)
        n_tok = X.shape[0]
        Y = np.zeros((n_tok, n_embd), np.float32)
        sel = np.zeros((n_tok, k), np.int32)
        w = np.zeros((n_tok, k), np.float32)
        h = np.zeros((n_tok, k, ff), np.float32) if want_h else None
        g, u, d = (np.ascontiguousarray(a, np.uint8) for a in (gate, up, down))
        rc = self.lib.fgo_moe_ffn(types[0], types[1], types[2], _ptr(g), _ptr(u), _ptr(d), n_expert, k, n_embd,
                                  ff, _ptr(logits), _ptr(X), _ptr(Y), n_tok, _ptr(sel), _ptr(w),
                                  _ptr(h) if want_h else None)
        if rc != 0:
            raise ValueError("fgo_moe_ffn failed")
        return (Y, sel, w, h) if want_h else (Y, sel, w)

    def attn_rows(self, q, st, en, ck, cv, kvo, hd, scale):
        """attn_rows restated: q [nr][hd] rows over positions st[r]..en[r] of the ring caches ck / cv
        [cap][kv_dim] at head offsets kvo[r]; returns o [nr][hd]."""
        q = np.ascontiguousarray(q, np.float32).reshape(-1, hd)
        ck = np.ascontiguousarray(ck, np.float32)
        cv = np.ascontiguousarray(cv, np.float32)
        st, en, kvo = (np.ascontiguousarray(a, np.int32) for a in (st, en, kvo))
        o = np.zeros_like(q)
        if self.lib.fgo_attn_rows(q.shape[0], _ptr(q), _ptr(o), _ptr(st), _ptr(en), _ptr(ck), _ptr(cv), ck.shape[1],
                                  _ptr(kvo), ck.shape[0], hd, scale) != 0:
            raise ValueError("fgo_attn_rows failed")
        return o

    def kvq_signs(self, n: int) -> np.ndarray:
        out = np.zeros(n, np.float32)
        self.lib.fgo_kvq_signs(_ptr(out), n)
        return out

    def kvq_rotate(self, x, inverse: bool = False) -> np.ndarray:
        x = np.array(x, np.float32, copy=True)
        if self.lib.fgo_kvq_rotate(_ptr(x), x.size, int(inverse)) != 0:
            raise ValueError("fgo_kvq_rotate failed")
        return x

    def kvq_quant(self, x, bits: int) -> np.ndarray:
        """One head slice (already rotated) as a TurboQuant record."""
        x = np.ascontiguousarray(x, np.float32)
        rec = np.zeros(4 + x.size * bits // 8, np.uint8)
        if self.lib.fgo_kvq_quant(_ptr(x), x.size, _ptr(rec), bits) != 0:
            raise ValueError("fgo_kvq_quant failed")
        return rec

    def kvq_attn_rows(self, q, st, en, kq, vq, kvh, hd, kbits, vbits, scale):
        """TurboQuant attention rows: q [nr][hd] unrotated; kq / vq [cap][slot bytes]."""
        q = np.ascontiguousarray(q, np.float32).reshape(-1, hd)
        kq = np.ascontiguousarray(kq, np.uint8)
        vq = np.ascontiguousarray(vq, np.uint8)
        st, en, kvh = (np.ascontiguousarray(a, np.int32) for a in (st, en, kvh))
        o = np.zeros_like(q)
        if self.lib.fgo_kvq_attn_rows(q.shape[0], _ptr(q), _ptr(o), _ptr(st), _ptr(en), _ptr(kq), _ptr(vq),
                                      kq.shape[1], vq.shape[1], _ptr(kvh), kq.shape[0], hd, kbits, vbits,
                                      scale) != 0:
            raise ValueError("fgo_kvq_attn_rows failed")
        return o

    def moe_down(self, type_down, down, n_embd, ff, sel, w, h):
        sel = np.ascontiguousarray(sel, np.int32)
        w = np.ascontiguousarray(w, np.float32)
        h = np.ascontiguousarray(h, np.float32)
        out = np.zeros(n_embd, np.float32)
        d = np.ascontiguousarray(down, np.uint8)
        if self.lib.fgo_moe_down(type_down, _ptr(d), n_embd, ff, sel.size, _ptr(sel), _ptr(w), _ptr(h),
                                 _ptr(out)) != 0:
            raise ValueError("fgo_moe_down failed")
        return out


def _cpu_has_vnni() -> bool:
    try:
        with open("/proc/cpuinfo") as f:
            flags = f.read()
        return " avx512_vnni" in flags and " avx512vl" in flags
    except OSError:
        return False


class Reference:
    """The reference's own kernels, compiled from /root/reference (oracle/_ref). Variant "hip" is the
    harness on the copy of fastgguf.c that include/fastgguf_c_hip.patch patches: its matvec,
    matvec_multi, matmul and moe_ffn are the reference's call sites, routed to the gfx950 library
    once hip_init() has opened a device (the drop-in test's caller, not a checker)."""

    def __init__(self, variant: str | None = None):
        if variant is None:
            variant = "vnni" if _cpu_has_vnni() else "avx2"
        path = os.path.join(HERE, "_ref", f"libfgref_{variant}.so")
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        self.variant = variant
        L = self.lib = C.CDLL(path)
        L.fgr_build.restype = C.c_char_p
        L.fgr_init.argtypes = [C.c_int]
        L.fgr_threads.restype = C.c_int
        for n in ("fgr_quantize_q8", "fgr_quantize_q8k"):
            getattr(L, n).argtypes = [C.c_void_p, C.c_void_p, C.c_int]
            getattr(L, n).restype = None
        for n in ("fgr_dot_q8_0", "fgr_dot_q4_K", "fgr_dot_q6_K", "fgr_dot_q5_0", "fgr_dot_q5_K"):
            getattr(L, n).argtypes = [C.c_void_p, C.c_void_p, C.c_int]
            getattr(L, n).restype = C.c_float
        L.fgr_dot_q32.argtypes = [C.c_uint32, C.c_void_p, C.c_void_p, C.c_int]
        L.fgr_dot_q32.restype = C.c_float
        L.fgr_matvec.argtypes = [C.c_uint32, C.c_int, C.c_void_p, C.c_int64, C.c_int, C.c_void_p, C.c_void_p]
        L.fgr_matvec_multi.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int,
                                       C.c_void_p, C.c_void_p]
        L.fgr_matmul.argtypes = [C.c_uint32, C.c_int, C.c_void_p, C.c_int64, C.c_int, C.c_void_p, C.c_int,
                                 C.c_void_p, C.c_int, C.c_int]
        L.fgr_moe_ffn.argtypes = [C.c_uint32] * 3 + [C.c_void_p] * 3 + [C.c_int] * 4 + \
            [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p]
        L.fgr_tensor_new.restype = C.c_void_p
        L.fgr_tensor_new.argtypes = [C.c_uint32, C.c_int, C.c_void_p, C.c_int64, C.c_int]
        L.fgr_tensor_free.argtypes = [C.c_void_p]
        L.fgr_tensor_free.restype = None
        L.fgr_tensor_matvec_multi.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
        L.fgr_attn_rows.argtypes = [C.c_int] + [C.c_void_p] * 6 + [C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]
        L.fgr_kvq_signs.argtypes = [C.c_void_p, C.c_int]
        L.fgr_kvq_rotate.argtypes = [C.c_void_p, C.c_int, C.c_int]
        L.fgr_kvq_quant.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_int]
        L.fgr_kvq_dequant.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int]
        L.fgr_kvq_attn_rows.argtypes = [C.c_int] + [C.c_void_p] * 6 + [C.c_int, C.c_int, C.c_void_p] + \
            [C.c_int] * 4 + [C.c_float]
        L.fgr_gguf_table.argtypes = [C.c_char_p] + [C.c_void_p] * 10 + [C.c_int64, C.c_char_p, C.c_int, C.c_void_p]
        if variant == "hip":
            L.fgr_hip_init.argtypes = [C.c_int]
            L.fgr_hip_state.argtypes = [C.c_void_p]
        L.fgr_init(256)

    def hip_init(self, mode: int = 0) -> int:
        """The patched build only (variant "hip"): its fg_gpu_init_ex(mode); 1 = on the device."""
        return self.lib.fgr_hip_init(mode)

    def hip_state(self):
        """(g_gpu.state, n_offloaded, n_skip_type, n_skip_mem) of the patched build."""
        c = np.zeros(3, np.int32)
        st = self.lib.fgr_hip_state(_ptr(c))
        return (st, int(c[0]), int(c[1]), int(c[2]))

    @property
    def build(self) -> str:
        return self.lib.fgr_build().decode()

    def threads(self) -> int:
        return self.lib.fgr_threads()

    def quantize_q8(self, x):
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros(x.size // 32, Q8_BLK)
        self.lib.fgr_quantize_q8(_ptr(x), _ptr(out), x.size)
        return out

    def quantize_q8k(self, x):
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros(x.size // 256, Q8K_BLK)
        self.lib.fgr_quantize_q8k(_ptr(x), _ptr(out), x.size)
        return out

    def dot(self, type_, row, act):
        row = np.ascontiguousarray(row, np.uint8)
        if uses_q8(type_):
            return self.lib.fgr_dot_q32(type_, _ptr(row), _ptr(act), act.size)
        name = {12: "fgr_dot_q4_K", 14: "fgr_dot_q6_K", 13: "fgr_dot_q5_K"}[type_]
        return getattr(self.lib, name)(_ptr(row), _ptr(act), act.size)

    def matvec(self, type_, w, cols, x, repack=False):
        w = np.ascontiguousarray(w, np.uint8)
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros(w.shape[0], np.float32)
        if self.lib.fgr_matvec(type_, int(repack), _ptr(w), w.shape[0], cols, _ptr(x), _ptr(y)) != 0:
            raise ValueError("fgr_matvec failed")
        return y

    def matmul(self, type_, w, cols, X, repack=False):
        w = np.ascontiguousarray(w, np.uint8)
        X = np.ascontiguousarray(X, np.float32)
        rows, nb = w.shape[0], X.shape[0]
        Y = np.zeros((nb, rows), np.float32)
        if self.lib.fgr_matmul(type_, int(repack), _ptr(w), rows, cols, _ptr(X), cols, _ptr(Y), rows, nb) != 0:
            raise ValueError("fgr_matmul failed")
        return Y

    def tensor(self, type_, w, cols, repack=False):
        """A persistent reference tensor (repacked once); returns an opaque handle."""
        w = np.ascontiguousarray(w, np.uint8)
        h = self.lib.fgr_tensor_new(type_, int(repack), _ptr(w), w.shape[0], cols)
        if not h:
            raise ValueError("fgr_tensor_new failed")
        return h

    def tensor_free(self, h):
        self.lib.fgr_tensor_free(h)

    def tensor_matvec_multi(self, hs, x, ys):
        arr = (C.c_void_p * len(hs))(*hs)
        yp = (C.c_void_p * len(ys))(*[y.ctypes.data for y in ys])
        if self.lib.fgr_tensor_matvec_multi(len(hs), arr, _ptr(x), yp) != 0:
            raise ValueError("fgr_tensor_matvec_multi failed")

    def attn_rows(self, q, st, en, ck, cv, kvo, hd, scale):
        """The reference's attn_rows on up to 4 rows sharing the head offset kvo."""
        q = np.ascontiguousarray(q, np.float32).reshape(-1, hd)
        ck = np.ascontiguousarray(ck, np.float32)
        cv = np.ascontiguousarray(cv, np.float32)
        st, en = (np.ascontiguousarray(a, np.int32) for a in (st, en))
        o = np.zeros_like(q)
        if self.lib.fgr_attn_rows(q.shape[0], _ptr(q), _ptr(o), _ptr(st), _ptr(en), _ptr(ck), _ptr(cv), ck.shape[1],
                                  int(kvo), ck.shape[0], hd, scale) != 0:
            raise ValueError("fgr_attn_rows failed")
        return o

    def kvq_signs(self, n: int) -> np.ndarray:
        out = np.zeros(n, np.float32)
        self.lib.fgr_kvq_signs(_ptr(out), n)
        return out

    def kvq_rotate(self, x, inverse: bool = False) -> np.ndarray:
        x = np.array(x, np.float32, copy=True)
        self.lib.fgr_kvq_rotate(_ptr(x), x.size, int(inverse))
        return x

    def kvq_quant(self, x, bits: int) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        rec = np.zeros(4 + x.size * bits // 8, np.uint8)
        self.lib.fgr_kvq_quant(_ptr(x), x.size, _ptr(rec), bits)
        return rec

    def kvq_dequant(self, rec, hd: int, bits: int) -> np.ndarray:
        rec = np.ascontiguousarray(rec, np.uint8)
        out = np.zeros(hd, np.float32)
        self.lib.fgr_kvq_dequant(_ptr(rec), _ptr(out), hd, bits)
        return out

    def kvq_attn_rows(self, q, st, en, kq, vq, kvh, hd, kbits, vbits, scale):
        q = np.ascontiguousarray(q, np.float32).reshape(-1, hd)
        kq = np.ascontiguousarray(kq, np.uint8)
        vq = np.ascontiguousarray(vq, np.uint8)
        st, en, kvh = (np.ascontiguousarray(a, np.int32) for a in (st, en, kvh))
        o = np.zeros_like(q)
        if self.lib.fgr_kvq_attn_rows(q.shape[0], _ptr(q), _ptr(o), _ptr(st), _ptr(en), _ptr(kq), _ptr(vq),
                                      kq.shape[1], vq.shape[1], _ptr(kvh), kq.shape[0], hd, kbits, vbits,
                                      scale) != 0:
            raise ValueError("fgr_kvq_attn_rows failed")
        return o

    def gguf_table(self, path, keys, cap=64):
        """gguf_open on a file: its summary, tensor table and kv_num(key, -1) answers, or None if the
        reference refuses the file."""
        v, a, nk, nt = (np.zeros(1, t) for t in (np.uint32, np.uint64, np.int64, np.int64))
        names = np.zeros((cap, 128), np.uint8)
        types, nd = np.zeros(cap, np.uint32), np.zeros(cap, np.int32)
        ne, off, nb = np.zeros((cap, 4), np.uint64), np.zeros(cap, np.uint64), np.zeros(cap, np.uint64)
        kv = np.zeros(len(keys), np.float64)
        kb = b"".join(k.encode() + b"\0" for k in keys)
        rc = self.lib.fgr_gguf_table(os.fsencode(path), *(_ptr(x) for x in (v, a, nk, nt, names, types, nd, ne, off, nb)),
                                     cap, kb, len(keys), _ptr(kv))
        if rc != 0:
            return None
        n = int(nt[0])
        return {"version": v, "alignment": a, "n_kvs": nk, "n_tensors": nt, "names": names[:n], "types": types[:n],
                "n_dims": nd[:n], "ne": ne[:n], "offsets": off[:n], "nbytes": nb[:n], "kv_keys": np.array(keys),
                "kv_vals": kv}

    def moe_ffn(self, types, gate, up, down, n_expert, k, n_embd, ff, logits, X):
        X = np.ascontiguousarray(X, np.float32)
        logits = np.ascontiguousarray(logits, np.float32)
        n_tok = X.shape[0]
        Y = np.zeros((n_tok, n_embd), np.float32)
        sel = np.zeros((n_tok, k), np.int32)
        w = np.zeros((n_tok, k), np.float32)
        g, u, d = (np.ascontiguousarray(a, np.uint8) for a in (gate, up, down))
        rc = self.lib.fgr_moe_ffn(types[0], types[1], types[2], _ptr(g), _ptr(u), _ptr(d), n_expert, k, n_embd,
                                  ff, _ptr(logits), _ptr(X), _ptr(Y), n_tok, _ptr(sel), _ptr(w))
        if rc != 0:
            raise ValueError(f"fgr_moe_ffn failed ({rc})")
        return Y, sel, w
