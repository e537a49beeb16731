"""Writes GGUF files for the tests (test infrastructure): the v3 layout that gguf_open
(fastgguf.c:342-440) reads. Little-endian: "GGUF", u32 version, u64 tensor count, u64 metadata
count; metadata {u64-length key, u32 value type, value}; tensor infos {u64-length name, u32 n_dims,
u64 dims (ne[0] first), u32 type, u64 offset into the data section}; the data section at the next
multiple of the alignment, each tensor at an aligned offset."""
from __future__ import annotations

import struct

import numpy as np

from fastgguf_amd import synth as S

# value types of the GGUF metadata
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
        I64: "<q", F64: "<d"}


def _str(s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _value(vt: int, v) -> bytes:
    if vt == STR:
        return _str(v)
    if vt == ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_value(et, x) for x in items)
    return struct.pack(_FMT[vt], v)


def gguf_bytes(kvs, tensors, alignment: int = 32, version: int = 3) -> bytes:
    """kvs: [(key, value type, value)] (arrays: (element type, items)); tensors: [(name, ggml type,
    dims with ne[0] first, data bytes)]. general.alignment is not added: pass it in kvs."""
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs))
    head += b"".join(_str(k) + struct.pack("<I", vt) + _value(vt, v) for k, vt, v in kvs)
    off, infos, blobs = 0, [], []
    for name, ty, dims, data in tensors:
        infos.append(_str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims) +
                     struct.pack("<IQ", ty, off))
        pad = (-len(data)) % alignment
        blobs.append(bytes(data) + b"\0" * pad)
        off += len(data) + pad
    head += b"".join(infos)
    head += b"\0" * ((-len(head)) % alignment)
    return head + b"".join(blobs)


LONG_KEY = "llama.a_key_longer_than_the_readers_buffer_" + "x" * 57  # 100 characters


def tiny_model() -> tuple[list, list]:
    """The metadata and tensors of tests/golden/tiny.gguf: every value kind the reader handles (a
    string, numbers of several types, integer / string / float arrays, a key longer than 95
    characters), general.alignment = 64, and tensors of five quantized types (2-D, 3-D experts)
    plus F32 tensors (2-D and 1-D)."""
    kvs = [("general.architecture", STR, "llama"), ("general.alignment", U32, 64),
           ("llama.block_count", U32, 1), ("llama.embedding_length", U64, 256),
           ("llama.rope.freq_base", F32, 500000.0), ("llama.attention.head_count", I32, -8),
           ("llama.flag", BOOL, 1), ("llama.scale", F64, 0.125),
           ("tokenizer.ggml.tokens", ARR, (STR, ["<s>", "a", "bc"])),
           ("llama.int_array", ARR, (I32, [7, -8, 9])), ("llama.float_array", ARR, (F32, [1.5, 2.5])),
           (LONG_KEY, U16, 77)]
    t = [("blk.0.ffn_gate.weight", S.T_Q4_K, [512, 24], S.weights(S.T_Q4_K, 24, 512, 701)),
         ("blk.0.ffn_down.weight", S.T_Q6_K, [256, 40], S.weights(S.T_Q6_K, 40, 256, 702)),
         ("blk.0.attn_v.weight", S.T_Q5_0, [160, 16], S.weights(S.T_Q5_0, 16, 160, 703)),
         ("blk.0.attn_k.weight", S.T_Q5_K, [256, 16], S.weights(S.T_Q5_K, 16, 256, 704)),
         ("output.weight", S.T_Q8_0, [64, 32], S.weights(S.T_Q8_0, 32, 64, 705)),
         ("blk.0.ffn_gate_exps.weight", S.T_Q4_K, [256, 16, 4], S.weights(S.T_Q4_K, 64, 256, 706)),
         ("token_embd.weight", 0, [8, 4], np.arange(32, dtype=np.float32).view(np.uint8)),
         ("blk.0.attn_norm.weight", 0, [16], np.ones(16, np.float32).view(np.uint8))]
    return kvs, [(n, ty, d, np.ascontiguousarray(a).view(np.uint8).tobytes()) for n, ty, d, a in t]


KV_QUERIES = ["general.alignment", "llama.block_count", "llama.embedding_length", "llama.rope.freq_base",
              "llama.attention.head_count", "llama.flag", "llama.scale", "tokenizer.ggml.tokens",
              "llama.int_array", "llama.float_array", "general.architecture", "no.such.key", LONG_KEY,
              LONG_KEY[:95]]


def variants(good: bytes) -> dict:
    """Files the reader must refuse or accept the way the reference does, derived from tiny.gguf."""
    kvs, tensors = tiny_model()
    bad_type = [(n, 99 if i == 2 else ty, d, b) for i, (n, ty, d, b) in enumerate(tensors)]
    return {
        "bad_magic": b"GGUX" + good[4:],
        "short": good[:15],
        "trunc_meta": good[:60],
        "trunc_table": good[:good.index(b"blk.0.attn_k.weight") + 8],
        "past_eof": good[:-100],
        "bad_type": gguf_bytes(kvs, bad_type, alignment=64),
        "bad_value_type": b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + _str("k") + struct.pack("<I", 13) + b"\0" * 8,
        "no_alignment_key": gguf_bytes([kv for kv in kvs if kv[0] != "general.alignment"], tensors, alignment=32),
        "empty": b"GGUF" + struct.pack("<IQQ", 3, 0, 0),
    }
