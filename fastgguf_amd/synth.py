"""Seeded synthetic GGUF weight blocks and activations, in the reference's file layout.

Byte layouts follow fastgguf.c (lawnak/FastGGUF):
  Q8_0  34 B / 32 weights   fp16 d @0, int8 q[32] @2                       (fastgguf.c:552-562)
  Q4_K 144 B / 256 weights  fp16 d @0, fp16 dmin @2, 12 B scales @4, 128 B nibbles @16
                            (fastgguf.c:622-643; scale unpack scale_min_k4 466-472)
  Q6_K 210 B / 256 weights  ql[128] @0, qh[64] @128, int8 sc[16] @192, fp16 d @208
                            (fastgguf.c:669-693)
  Q5_0  22 B / 32 weights   fp16 d @0, u32 qh @2 (bit j = bit 4 of element j), nibbles qs[16] @6
                            (fastgguf.c:518-532, element order q5_elem 939-942)
  Q5_K 176 B / 256 weights  fp16 d @0, fp16 dmin @2, 12 B scales @4, qh[32] @16, ql[128] @48
                            (fastgguf.c:644-667)
  Q4_0  18 B / 32 weights   fp16 d @0, nibbles qs[16] @2; value d (q - 8)    (fastgguf.c:485-497)
  Q4_1  20 B / 32 weights   fp16 d @0, fp16 m @2, nibbles @4; value d q + m  (fastgguf.c:499-516)
  Q5_1  24 B / 32 weights   fp16 d @0, fp16 m @2, u32 qh @4, nibbles @8      (fastgguf.c:534-550)
  IQ4_NL 18 B / 32 weights  fp16 d @0, nibbles @2; value d kvalues[q]        (fastgguf.c:694-706)
  (32-value types: element j is nibble j of qs, low nibbles of qs[0..15] first, then the high ones)
  F32 / F16 / BF16: one value per element, 4 / 2 / 2 bytes; BF16 = the high 16 bits of an fp32
                            (dequantize_row 481-489, bf16_to_float 124-127)
Value distributions are the benchmark's: Q4_K nibbles uniform, 6-bit scales and mins uniform in
[0, 63], d and dmin = fp16(|N(0,1)| * 0.005); Q6_K quant bytes uniform, int8 scales uniform in
[-64, 63], d = fp16(|N(0,1)| * 0.002); Q8_0 quants uniform in [-127, 127], d = fp16(|N(0,1)| * 0.01);
Q5_0 and Q5_K quant bytes uniform, d = fp16(|N(0,1)| * 0.01) (Q5_0) or as Q4_K (Q5_K); the other
32-value types quant bytes uniform, d = fp16(|N(0,1)| * 0.01), m = fp16(N(0,1) * 0.05); the float
types N(0,1) * 0.02 (F16 rounded to nearest even, BF16 rounded to nearest even on the high half).
fp16 conversion rounds to nearest even (numpy astype).
"""
from __future__ import annotations

import numpy as np

T_F32 = 0
T_F16 = 1
T_BF16 = 30
T_Q4_0 = 2
T_Q4_1 = 3
T_Q5_0 = 6
T_Q5_1 = 7
T_Q8_0 = 8
T_Q2_K = 10
T_Q3_K = 11
T_Q4_K = 12
T_Q5_K = 13
T_Q6_K = 14
T_IQ4_NL = 20
T_IQ4_XS = 23

#: (elements per block, bytes per block), block_size_of (fastgguf.c:235-253)
BLOCK = {T_Q8_0: (32, 34), T_Q4_K: (256, 144), T_Q6_K: (256, 210), T_Q5_0: (32, 22), T_Q5_K: (256, 176),
         T_Q4_0: (32, 18), T_Q4_1: (32, 20), T_Q5_1: (32, 24), T_IQ4_NL: (32, 18),
         T_Q2_K: (256, 84), T_Q3_K: (256, 110), T_IQ4_XS: (256, 136), T_F32: (1, 4), T_F16: (1, 2),
         T_BF16: (1, 2)}
TYPE_NAME = {T_Q8_0: "Q8_0", T_Q4_K: "Q4_K", T_Q6_K: "Q6_K", T_Q5_0: "Q5_0", T_Q5_K: "Q5_K", T_Q4_0: "Q4_0",
             T_Q4_1: "Q4_1", T_Q5_1: "Q5_1", T_IQ4_NL: "IQ4_NL", T_Q2_K: "Q2_K", T_Q3_K: "Q3_K",
             T_IQ4_XS: "IQ4_XS", T_F32: "F32", T_F16: "F16", T_BF16: "BF16"}
Q32_TYPES = (T_Q8_0, T_Q5_0, T_Q4_0, T_Q4_1, T_Q5_1, T_IQ4_NL)
#: 256-value blocks whose row kernels take Q8 (32-value) activations
K256Q8_TYPES = (T_Q2_K, T_Q3_K, T_IQ4_XS)
#: one value per element; the row kernels take x in fp32 (no quantization)
FLOAT_TYPES = (T_F32, T_F16, T_BF16)


def uses_q8(type_: int) -> bool:
    """Activation kind (type_uses_q8, fastgguf.c:2167-2173): Q8 blocks of 32 for the 32-value
    types and for Q2_K / Q3_K / IQ4_XS, Q8_K blocks of 256 for the other K-quants."""
    return type_ in Q32_TYPES or type_ in K256Q8_TYPES

#: activation blocks, the reference's structs q8_blk_t (743) and q8k_blk_t (771)
Q8_BLK = np.dtype([("d", "<f4"), ("qs", "i1", 32), ("s16", "<i2", 2)])
Q8K_BLK = np.dtype([("d", "<f4"), ("qs", "i1", 256), ("bsums", "<i2", 16)])
assert Q8_BLK.itemsize == 40 and Q8K_BLK.itemsize == 292


def row_bytes(type_: int, cols: int) -> int:
    eb, bb = BLOCK[type_]
    if cols % eb:
        raise ValueError(f"{TYPE_NAME[type_]}: cols {cols} is not a multiple of {eb}")
    return cols // eb * bb


def _fp16_abs_normal(rng: np.random.Generator, n: int, scale: float) -> np.ndarray:
    return (np.abs(rng.standard_normal(n)) * scale).astype(np.float16)


def pack_q4k_scales(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """Inverse of scale_min_k4 (fastgguf.c:466-472): 8 six-bit scales and mins -> 12 bytes."""
    sc = sc.astype(np.uint8)
    mn = mn.astype(np.uint8)
    out = np.empty(sc.shape[:-1] + (12,), np.uint8)
    for j in range(4):
        out[..., j] = sc[..., j] | ((sc[..., j + 4] >> 4) << 6)
        out[..., 4 + j] = mn[..., j] | ((mn[..., j + 4] >> 4) << 6)
        out[..., 8 + j] = (sc[..., j + 4] & 15) | ((mn[..., j + 4] & 15) << 4)
    return out


def q4_k_weights(rows: int, cols: int, seed: int) -> np.ndarray:
    """rows x cols Q4_K matrix, returned as uint8 [rows, cols/256*144]."""
    rng = np.random.Generator(np.random.PCG64(seed))
    nb = rows * (cols // 256)
    if cols % 256:
        raise ValueError("Q4_K needs cols % 256 == 0")
    blk = np.empty((nb, 144), np.uint8)
    blk[:, 0:2] = _fp16_abs_normal(rng, nb, 0.005).view(np.uint8).reshape(nb, 2)
    blk[:, 2:4] = _fp16_abs_normal(rng, nb, 0.005).view(np.uint8).reshape(nb, 2)
    sc = rng.integers(0, 64, size=(nb, 8), dtype=np.uint8)
    mn = rng.integers(0, 64, size=(nb, 8), dtype=np.uint8)
    blk[:, 4:16] = pack_q4k_scales(sc, mn)
    blk[:, 16:144] = rng.integers(0, 256, size=(nb, 128), dtype=np.uint8)
    return blk.reshape(rows, -1)


def q6_k_weights(rows: int, cols: int, seed: int) -> np.ndarray:
    """rows x cols Q6_K matrix, returned as uint8 [rows, cols/256*210]."""
    rng = np.random.Generator(np.random.PCG64(seed))
    if cols % 256:
        raise ValueError("Q6_K needs cols % 256 == 0")
    nb = rows * (cols // 256)
    blk = np.empty((nb, 210), np.uint8)
    blk[:, 0:192] = rng.integers(0, 256, size=(nb, 192), dtype=np.uint8)
    blk[:, 192:208] = rng.integers(-64, 64, size=(nb, 16), dtype=np.int8).view(np.uint8)
    blk[:, 208:210] = _fp16_abs_normal(rng, nb, 0.002).view(np.uint8).reshape(nb, 2)
    return blk.reshape(rows, -1)


def q8_0_weights(rows: int, cols: int, seed: int) -> np.ndarray:
    """rows x cols Q8_0 matrix, returned as uint8 [rows, cols/32*34]."""
    rng = np.random.Generator(np.random.PCG64(seed))
    if cols % 32:
        raise ValueError("Q8_0 needs cols % 32 == 0")
    nb = rows * (cols // 32)
    blk = np.empty((nb, 34), np.uint8)
    blk[:, 0:2] = _fp16_abs_normal(rng, nb, 0.01).view(np.uint8).reshape(nb, 2)
    blk[:, 2:34] = rng.integers(-127, 128, size=(nb, 32), dtype=np.int8).view(np.uint8)
    return blk.reshape(rows, -1)


def q5_0_weights(rows: int, cols: int, seed: int) -> np.ndarray:
    """rows x cols Q5_0 matrix, returned as uint8 [rows, cols/32*22]."""
    rng = np.random.Generator(np.random.PCG64(seed))
    if cols % 32:
        raise ValueError("Q5_0 needs cols % 32 == 0")
    nb = rows * (cols // 32)
    blk = np.empty((nb, 22), np.uint8)
    blk[:, 0:2] = _fp16_abs_normal(rng, nb, 0.01).view(np.uint8).reshape(nb, 2)
    blk[:, 2:22] = rng.integers(0, 256, size=(nb, 20), dtype=np.uint8)
    return blk.reshape(rows, -1)


def q5_k_weights(rows: int, cols: int, seed: int) -> np.ndarray:
    """rows x cols Q5_K matrix, returned as uint8 [rows, cols/256*176]."""
    rng = np.random.Generator(np.random.PCG64(seed))
    if cols % 256:
        raise ValueError("Q5_K needs cols % 256 == 0")
    nb = rows * (cols // 256)
    blk = np.empty((nb, 176), np.uint8)
    blk[:, 0:2] = _fp16_abs_normal(rng, nb, 0.005).view(np.uint8).reshape(nb, 2)
    blk[:, 2:4] = _fp16_abs_normal(rng, nb, 0.005).view(np.uint8).reshape(nb, 2)
    sc = rng.integers(0, 64, size=(nb, 8), dtype=np.uint8)
    mn = rng.integers(0, 64, size=(nb, 8), dtype=np.uint8)
    blk[:, 4:16] = pack_q4k_scales(sc, mn)
    blk[:, 16:176] = rng.integers(0, 256, size=(nb, 160), dtype=np.uint8)
    return blk.reshape(rows, -1)


def q32_weights(type_: int, rows: int, cols: int, seed: int) -> np.ndarray:
    """rows x cols of Q4_0 / Q4_1 / Q5_1 / IQ4_NL: fp16 d (and m), uniform quant bytes."""
    rng = np.random.Generator(np.random.PCG64(seed))
    if cols % 32:
        raise ValueError(f"{TYPE_NAME[type_]} needs cols % 32 == 0")
    nb = rows * (cols // 32)
    bb = BLOCK[type_][1]
    blk = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    blk[:, 0:2] = _fp16_abs_normal(rng, nb, 0.01).view(np.uint8).reshape(nb, 2)
    if type_ in (T_Q4_1, T_Q5_1):
        blk[:, 2:4] = (rng.standard_normal(nb) * 0.05).astype(np.float16).view(np.uint8).reshape(nb, 2)
    return blk.reshape(rows, -1)


#: byte offsets of the fp16 scales in a 256-value block of the low-bit types: d (and dmin)
_K256Q8_D = {T_Q2_K: (80, 82), T_Q3_K: (108,), T_IQ4_XS: (0,)}


def k256q8_weights(type_: int, rows: int, cols: int, seed: int) -> np.ndarray:
    """rows x cols of Q2_K / Q3_K / IQ4_XS: uniform quant and scale bytes, fp16 d (Q2_K: and
    dmin) of the magnitudes the other generators use."""
    rng = np.random.Generator(np.random.PCG64(seed))
    if cols % 256:
        raise ValueError(f"{TYPE_NAME[type_]} needs cols % 256 == 0")
    nb = rows * (cols // 256)
    bb = BLOCK[type_][1]
    blk = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    for o, scale in zip(_K256Q8_D[type_], (0.004, 0.002)):
        blk[:, o:o + 2] = _fp16_abs_normal(rng, nb, scale).view(np.uint8).reshape(nb, 2)
    return blk.reshape(rows, -1)


def _bf16_bits(v: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, rounded to nearest even on the dropped 16 bits (finite inputs)"""
    u = np.ascontiguousarray(v, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def float_weights(type_: int, rows: int, cols: int, seed: int) -> np.ndarray:
    rng = np.random.Generator(np.random.PCG64(seed))
    v = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    if type_ == T_F16:
        v = v.astype(np.float16)
    elif type_ == T_BF16:
        v = _bf16_bits(v)
    return np.ascontiguousarray(v).view(np.uint8).reshape(rows, -1)


def random_float_bits(type_: int, rows: int, cols: int, seed: int) -> np.ndarray:
    """Random finite values of every exponent that keeps products with N(0, 1) activations finite:
    F16 every exponent (subnormals included, no inf / NaN), F32 and BF16 exponents 2^-40 .. 2^10,
    and about one value in 16 a zero or a subnormal, with random signs."""
    rng = np.random.Generator(np.random.PCG64(seed))
    n = rows * cols
    if type_ == T_F16:
        b = rng.integers(0, 1 << 16, size=n, dtype=np.uint32)
        e = (b >> 10) & 31
        b = np.where(e == 31, b & ~np.uint32(1 << 14), b).astype(np.uint16)  # exponent 31 -> 15
    else:
        man = rng.integers(0, 1 << 23, size=n, dtype=np.uint32)
        ex = rng.integers(127 - 40, 127 + 11, size=n).astype(np.uint32)
        ex = np.where(rng.integers(0, 16, size=n) == 0, 0, ex).astype(np.uint32)  # zeros / subnormals
        sg = rng.integers(0, 2, size=n, dtype=np.uint32)
        b = (sg << 31) | (ex << 23) | man
        if type_ == T_BF16:
            b = (b >> 16).astype(np.uint16)
    return np.ascontiguousarray(b).view(np.uint8).reshape(rows, -1)


def weights(type_: int, rows: int, cols: int, seed: int) -> np.ndarray:
    if type_ in FLOAT_TYPES:
        return float_weights(type_, rows, cols, seed)
    if type_ in K256Q8_TYPES:
        return k256q8_weights(type_, rows, cols, seed)
    if type_ in (T_Q4_0, T_Q4_1, T_Q5_1, T_IQ4_NL):
        return q32_weights(type_, rows, cols, seed)
    if type_ == T_Q5_0:
        return q5_0_weights(rows, cols, seed)
    if type_ == T_Q5_K:
        return q5_k_weights(rows, cols, seed)
    if type_ == T_Q4_K:
        return q4_k_weights(rows, cols, seed)
    if type_ == T_Q6_K:
        return q6_k_weights(rows, cols, seed)
    if type_ == T_Q8_0:
        return q8_0_weights(rows, cols, seed)
    raise ValueError(f"unsupported type {type_}")


def random_bytes_weights(type_: int, rows: int, cols: int, seed: int) -> np.ndarray:
    """Uniform random bytes with sane fp16 scales, as the reference selftest builds its rows
    (fastgguf.c:5701-5710): d in 0x2C00..0x2FFF, dmin in 0x2400..0x27FF."""
    if type_ in FLOAT_TYPES:
        return random_float_bits(type_, rows, cols, seed)
    rng = np.random.Generator(np.random.PCG64(seed))
    eb, bb = BLOCK[type_]
    nb = rows * (cols // eb)
    blk = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    d = (0x2C00 + rng.integers(0, 0x400, size=nb)).astype(np.uint16)
    dm = (0x2400 + rng.integers(0, 0x400, size=nb)).astype(np.uint16)
    if type_ == T_Q6_K:
        blk[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    elif type_ in K256Q8_TYPES:   # the reference selftest's Q2_K / Q3_K / IQ4_XS rows (5612-5676)
        o = _K256Q8_D[type_]
        blk[:, o[0]:o[0] + 2] = d.view(np.uint8).reshape(nb, 2)
        if len(o) > 1:
            blk[:, o[1]:o[1] + 2] = (0x2800 + rng.integers(0, 0x400, size=nb)).astype(np.uint16).view(
                np.uint8).reshape(nb, 2)
    else:
        blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        if type_ in (T_Q4_K, T_Q5_K, T_Q4_1, T_Q5_1):
            blk[:, 2:4] = dm.view(np.uint8).reshape(nb, 2)
    return blk.reshape(rows, -1)


def activations(n: int, seed: int, rows: int | None = None) -> np.ndarray:
    """fp32 N(0, 1) activations: shape [n] or [rows, n]."""
    rng = np.random.Generator(np.random.PCG64(seed))
    shape = (n,) if rows is None else (rows, n)
    return rng.standard_normal(shape).astype(np.float32)


def router_logits(n_tok: int, n_expert: int, seed: int) -> np.ndarray:
    rng = np.random.Generator(np.random.PCG64(seed))
    return rng.standard_normal((n_tok, n_expert)).astype(np.float32)
