"""Writes the golden vectors in tests/golden/*.npz with the reference's own kernels.

Run in a container where lawnak/FastGGUF is mounted at /root/reference:

    make -C oracle ref && python tests/golden/make_golden.py [attn | lowbit | float]

It loads oracle/_ref/libfgref_vnni.so (fastgguf.c compiled from where it lies, AVX-512-VNNI
build; ref_harness.c exports its static kernels) and records inputs and outputs only: weight
bytes, activations, quantized blocks, outputs. The fixtures are data; no reference source or
binary is stored. Seeds are fixed, so re-running reproduces the same files.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))

sys.path.insert(0, os.path.dirname(HERE))

import gguf_write as GW  # noqa: E402
from fastgguf_amd import synth as S  # noqa: E402
from oracle import Reference  # noqa: E402


def quant_inputs() -> np.ndarray:
    """Activation rows for the quantizer fixtures: normal values plus the edge cases the
    quantizers must get right (all-zero block, exact .5 ties after scaling, a single huge value,
    negative-zero, subnormals where 1/d overflows, infinities and NaN)."""
    rng = np.random.Generator(np.random.PCG64(101))
    x = rng.standard_normal((7, 1024)).astype(np.float32)
    x[1, :256] = 0.0                          # all-zero Q8_K block -> d = id = 0, q = 0
    x[1, 256:288] = 0.0                       # all-zero Q8 block
    x[2, :256] = np.arange(256) - 127.5       # amax 128 -> halfway cases
    x[2, 256:512] = (np.arange(256) % 64 - 32) * 0.5 + 0.25
    x[3, :] *= 1e3
    x[3, 5] = 3e4                             # one dominant value per block
    x[4, :] = -0.0
    x[4, 512:] = rng.standard_normal(512).astype(np.float32) * 1e-39  # subnormals
    x[5, :] = np.float32(127.0) * (rng.integers(-3, 4, 1024) / 2.0)   # exact ties x*id = k + .5
    x[6, 3] = np.inf                          # non-finite inputs: d = inf, id = 0
    x[6, 300] = -np.inf
    x[6, 600] = np.nan                        # NaN is skipped by the amax compare, quantizes to 0
    x[6, 900] = 3.4e38                        # near the top of the range
    return x


#: (hd, kv_dim, kvo, cap, st, en, q magnitude): one position, a tail of 7, whole groups of 8 plus
#: tails, causal prefill rows over a wrapped ring, a full cache, hd 32 .. 256, and scores spread
#: past exp_neg_ps's -87 cut-off; then head sizes that are not multiples of 32, which take the
#: per-row path and dot_f32v's order: 16-value chunks only (80), one more group of 8 (72, 120),
#: a scalar tail (100, 36), and an odd size at an odd offset (13)
ATTN_CASES = [
    (32, 64, 32, 40, [0], [0], 1.0),
    (64, 128, 0, 40, [3], [9], 1.0),
    (64, 128, 64, 40, [30, 30, 30, 30], [45, 46, 47, 48], 1.0),
    (128, 128, 0, 64, [50, 52, 10, 37], [100, 101, 73, 100], 1.0),
    (256, 256, 0, 24, [5, 7], [28, 20], 1.0),
    (32, 32, 0, 40, [2], [34], 30.0),
    (80, 160, 80, 40, [3, 5], [20, 33], 1.0),
    (72, 144, 0, 30, [0], [25], 1.0),
    (100, 200, 100, 24, [1, 2, 3], [23, 10, 15], 1.0),
    (36, 36, 0, 20, [0], [19], 4.0),
    (13, 26, 13, 16, [2, 4], [9, 15], 1.0),
    (120, 240, 0, 50, [10, 11, 12, 13], [40, 41, 42, 43], 1.0),
]


#: non-finite V at positions that only one row of the call covers, (position, column of the head,
#: value) each: the per-row path walks each row's own positions only, so the other row stays finite
#: (aligned hd 36, and hd 13 read value by value); the vector path walks the call's whole span with
#: zero weights outside a row's range, so fma(0, inf) makes the other row's column NaN there
ATTN_NONFINITE = [
    (36, 36, 0, 20, [0, 8], [5, 15], 1.0, [(12, 3, np.inf), (13, 7, np.nan)]),
    (13, 26, 13, 16, [2, 9], [6, 14], 1.0, [(11, 0, np.inf), (3, 12, -np.inf)]),
    (64, 128, 64, 32, [0, 8], [5, 15], 1.0, [(12, 3, np.inf), (2, 9, -np.inf)]),
]


def attn_cases(ref) -> dict:
    rng = np.random.default_rng(77)
    out = {}
    cases = [c + ([],) for c in ATTN_CASES] + ATTN_NONFINITE
    for i, (hd, kv_dim, kvo, cap, st, en, mag, plants) in enumerate(cases):
        q = (rng.standard_normal((len(st), hd)) * mag).astype(np.float32)
        ck = rng.standard_normal((cap, kv_dim)).astype(np.float32)
        cv = rng.standard_normal((cap, kv_dim)).astype(np.float32)
        for p, col, v in plants:
            cv[p % cap, kvo + col] = v
        scale = np.float32(1.0 / np.sqrt(hd))
        o = ref.attn_rows(q, st, en, ck, cv, kvo, hd, float(scale))
        out.update({f"c{i}_q": q, f"c{i}_ck": ck, f"c{i}_cv": cv, f"c{i}_st": np.array(st, np.int32),
                    f"c{i}_en": np.array(en, np.int32), f"c{i}_o": o,
                    f"c{i}_meta": np.array([hd, kvo], np.int32), f"c{i}_scale": np.array([scale], np.float32)})
    out["n_cases"] = np.array([len(cases)], np.int32)
    return out


#: (hd, K / V heads, cap, K bits, V bits, st, en, K / V head of each row)
KVQ_ATTN = [
    (64, 2, 24, 4, 4, [3, 3, 10], [20, 25, 10], [0, 1, 1]),
    (128, 1, 40, 8, 4, [30, 31], [60, 69], [0, 0]),
    (128, 2, 17, 4, 2, [0, 5], [16, 9], [1, 0]),
]


def kvq_slot_bytes(hd, nkv, bits):
    return nkv * (4 + hd * bits // 8)


def kvq_cases(ref) -> dict:
    rng = np.random.default_rng(88)
    out = {"signs": ref.kvq_signs(1024).astype(np.int8)}
    for hd in (64, 128, 256):
        x = (rng.standard_normal(hd) * 3).astype(np.float32)
        out[f"rot{hd}_x"] = x
        out[f"rot{hd}_y"] = ref.kvq_rotate(x)
        out[f"rot{hd}_inv"] = ref.kvq_rotate(x, inverse=True)
    xs = [ref.kvq_rotate((rng.standard_normal(128) * s).astype(np.float32)) for s in (0.01, 1.0, 40.0)]
    xs += [np.zeros(128, np.float32), (np.eye(1, 128, 7, dtype=np.float32)[0] * -5.0)]
    xs += [ref.kvq_rotate((rng.standard_normal(128) * (1 + k)).astype(np.float32)) for k in range(40)]
    out["quant_x"] = np.stack(xs)
    for bits in (8, 4, 2):
        out[f"quant_rec{bits}"] = np.stack([ref.kvq_quant(x, bits) for x in xs])
    for i, (hd, nkv, cap, kb, vb, st, en, kvh) in enumerate(KVQ_ATTN):
        kq = np.zeros((cap, kvq_slot_bytes(hd, nkv, kb)), np.uint8)
        vq = np.zeros((cap, kvq_slot_bytes(hd, nkv, vb)), np.uint8)
        for sl in range(cap):
            for h in range(nkv):
                k = ref.kvq_rotate(rng.standard_normal(hd).astype(np.float32))
                v = ref.kvq_rotate(rng.standard_normal(hd).astype(np.float32))
                kq[sl, h * (4 + hd * kb // 8):(h + 1) * (4 + hd * kb // 8)] = ref.kvq_quant(k, kb)
                vq[sl, h * (4 + hd * vb // 8):(h + 1) * (4 + hd * vb // 8)] = ref.kvq_quant(v, vb)
        q = (rng.standard_normal((len(st), hd)) * 2).astype(np.float32)
        scale = np.float32(1.0 / np.sqrt(hd))
        o = ref.kvq_attn_rows(q, st, en, kq, vq, kvh, hd, kb, vb, float(scale))
        out.update({f"a{i}_q": q, f"a{i}_kq": kq, f"a{i}_vq": vq, f"a{i}_st": np.array(st, np.int32),
                    f"a{i}_en": np.array(en, np.int32), f"a{i}_kvh": np.array(kvh, np.int32), f"a{i}_o": o,
                    f"a{i}_meta": np.array([hd, nkv, kb, vb], np.int32), f"a{i}_scale": np.array([scale])})
    out["n_attn"] = np.array([len(KVQ_ATTN)], np.int32)
    return out


def lowbit_cases(ref) -> dict:
    """Q2_K / Q3_K / IQ4_XS rows on Q8 activations: matvec on synthetic and selftest-style byte
    rows (dot_q2_K_q8 1426, dot_q3_K_q8 1481, dot_iq4_xs_q8 1580 through dot_row) and matmul at
    3, 8 and 45 tokens (no GEMM for these types: the row kernel per token, 3004-3093)."""
    out = {}
    for name, t in (("q2_k", S.T_Q2_K), ("q3_k", S.T_Q3_K), ("iq4_xs", S.T_IQ4_XS)):
        for gname, gen, rows, cols in (("synth", S.weights, 24, 768), ("bytes", S.random_bytes_weights, 24, 1024)):
            w = gen(t, rows, cols, 700 + t)
            xv = S.activations(cols, 710 + t)
            out[f"{name}_{gname}_w"] = w
            out[f"{name}_{gname}_x"] = xv
            out[f"{name}_{gname}_y"] = ref.matvec(t, w, cols, xv)
        w = S.weights(t, 20, 512, 720 + t)
        out[f"{name}_mm_w"] = w
        for nb in (3, 8, 45):
            X = S.activations(512, 730 + nb, rows=nb)
            out[f"{name}_mm_X{nb}"] = X
            out[f"{name}_mm_Y{nb}"] = ref.matmul(t, w, 512, X)
    return out


def float_cases(ref) -> dict:
    """F32 / F16 / BF16 rows on fp32 activations (dot_row 2207-2214: dot_f32v 1618, dot_f16_row 1645,
    the BF16 loop 2209): matvec on N(0, 0.02) rows and on random finite bit patterns, at widths
    with and without a tail (the 16-, 8- and 1-value steps of each kernel), and matmul at 3 and 9
    tokens (no GEMM for these types: dot_row per token, 3033-3093)."""
    out = {}
    for name, t in (("f32", S.T_F32), ("f16", S.T_F16), ("bf16", S.T_BF16)):
        for cols in (3, 8, 100, 776, 1024):
            for gname, gen in (("synth", S.weights), ("bytes", S.random_bytes_weights)):
                w = gen(t, 12, cols, 800 + 3 * t + cols)
                xv = S.activations(cols, 810 + t + cols) * np.float32(2.5)
                out[f"{name}_{gname}_{cols}_w"] = w
                out[f"{name}_{gname}_{cols}_x"] = xv
                out[f"{name}_{gname}_{cols}_y"] = ref.matvec(t, w, cols, xv)
        w = S.weights(t, 20, 264, 820 + t)
        out[f"{name}_mm_w"] = w
        for nb in (3, 9):
            X = S.activations(264, 830 + nb, rows=nb)
            out[f"{name}_mm_X{nb}"] = X
            out[f"{name}_mm_Y{nb}"] = ref.matmul(t, w, 264, X)
    return out


def main() -> None:
    ref = Reference("vnni")
    print("reference build:", ref.build, "threads:", ref.threads())
    if sys.argv[1:] == ["attn"]:  # only the attention vectors
        np.savez_compressed(os.path.join(HERE, "attn.npz"), **attn_cases(ref))
        return
    if sys.argv[1:] == ["float"]:  # only the F32 / F16 / BF16 vectors
        np.savez_compressed(os.path.join(HERE, "float.npz"), **float_cases(ref))
        return
    if sys.argv[1:] == ["lowbit"]:  # only the Q2_K / Q3_K / IQ4_XS vectors
        np.savez_compressed(os.path.join(HERE, "lowbit.npz"), **lowbit_cases(ref))
        return
    out = {}

    x = quant_inputs()
    out["quant_x"] = x
    out["quant_q8"] = np.stack([ref.quantize_q8(r) for r in x]).view(np.uint8)
    out["quant_q8k"] = np.stack([ref.quantize_q8k(r) for r in x]).view(np.uint8)
    np.savez_compressed(os.path.join(HERE, "quantize.npz"), **out)

    # single-token matvecs: per type, synthetic (benchmark distributions) and random-byte rows
    mv = {}
    cases = [("q8_0", S.T_Q8_0, 24, 512), ("q4_k", S.T_Q4_K, 24, 768), ("q6_k", S.T_Q6_K, 24, 512),
             ("q5_0", S.T_Q5_0, 24, 544), ("q5_k", S.T_Q5_K, 24, 768), ("q4_0", S.T_Q4_0, 24, 544),
             ("q4_1", S.T_Q4_1, 24, 544), ("q5_1", S.T_Q5_1, 24, 544), ("iq4_nl", S.T_IQ4_NL, 24, 544)]
    for name, t, rows, cols in cases:
        for gname, gen in (("synth", S.weights), ("bytes", S.random_bytes_weights)):
            w = gen(t, rows, cols, 200 + t)
            xv = S.activations(cols, 300 + t)
            key = f"{name}_{gname}"
            mv[f"{key}_w"] = w
            mv[f"{key}_x"] = xv
            mv[f"{key}_y"] = ref.matvec(t, w, cols, xv)
            if t in (S.T_Q4_K, S.T_Q4_0):
                mv[f"{key}_y_rp"] = ref.matvec(t, w, cols, xv, repack=True)
    np.savez_compressed(os.path.join(HERE, "matvec.npz"), **mv)

    # prompt batches through matmul: 3 tokens (x4 tiles / repacked per-token) and 8, 45 (GEMM)
    mm = {}
    for name, t, rows, cols in [("q8_0", S.T_Q8_0, 20, 512), ("q4_k", S.T_Q4_K, 24, 512), ("q6_k", S.T_Q6_K, 20, 512),
                                ("q5_0", S.T_Q5_0, 20, 544), ("q5_k", S.T_Q5_K, 20, 512),
                                ("q4_0", S.T_Q4_0, 24, 544), ("q4_1", S.T_Q4_1, 20, 544),
                                ("q5_1", S.T_Q5_1, 20, 544), ("iq4_nl", S.T_IQ4_NL, 20, 544)]:
        w = S.weights(t, rows, cols, 400 + t)
        mm[f"{name}_w"] = w
        for nb in (3, 8, 45):
            X = S.activations(cols, 500 + nb, rows=nb)
            mm[f"{name}_X{nb}"] = X
            mm[f"{name}_Y{nb}"] = ref.matmul(t, w, cols, X)
            if t in (S.T_Q4_K, S.T_Q4_0):
                mm[f"{name}_Y{nb}_rp"] = ref.matmul(t, w, cols, X, repack=True)
    np.savez_compressed(os.path.join(HERE, "matmul.npz"), **mm)

    # MoE: 8 experts, top-3 (the reference selftest's shape, 5938-6020), n_embd 256, ff 256,
    # 4 tokens, Q4_K experts. X[:, 0] = 1 lets the harness reproduce the given router logits
    # through the reference's own router matvec.
    E, K, D, F, T = 8, 3, 256, 256, 4
    g = S.weights(S.T_Q4_K, E * F, D, 601)
    u = S.weights(S.T_Q4_K, E * F, D, 602)
    d = S.weights(S.T_Q4_K, E * D, F, 603)
    X = S.activations(D, 604, rows=T)
    X[:, 0] = 1.0
    L = S.router_logits(T, E, 605)
    L[2, 3] = L[2, 7] = L[2].max() + 1.0     # a tie on top: argmax keeps the lower index
    L[3, :] = 0.0                            # all equal: selection 0, 1, 2
    Y, sel, w = ref.moe_ffn((S.T_Q4_K,) * 3, g, u, d, E, K, D, F, L, X)
    np.savez_compressed(os.path.join(HERE, "moe.npz"), gate=g, up=u, down=d, X=X, logits=L, Y=Y, sel=sel, w=w,
                        dims=np.array([E, K, D, F, T]))

    # MoE with the fallback types of a K-quant file: Q5_K gate / up, Q5_0 down over ff = 160
    # (5 blocks of 32: not a multiple of 256, the reason a file falls back to Q5_0)
    E, K, D, F, T = 4, 2, 256, 160, 4
    types = (S.T_Q5_K, S.T_Q5_K, S.T_Q5_0)
    g = S.weights(types[0], E * F, D, 611)
    u = S.weights(types[1], E * F, D, 612)
    d = S.weights(types[2], E * D, F, 613)
    X = S.activations(D, 614, rows=T)
    X[:, 0] = 1.0
    L = S.router_logits(T, E, 615)
    Y, sel, w = ref.moe_ffn(types, g, u, d, E, K, D, F, L, X)
    np.savez_compressed(os.path.join(HERE, "moe_q5.npz"), gate=g, up=u, down=d, X=X, logits=L, Y=Y, sel=sel, w=w,
                        dims=np.array([E, K, D, F, T]), types=np.array(types))
    # GGUF ingestion: tiny.gguf (tests/gguf_write.py's tiny model) and the reference's gguf_open of
    # it (summary, tensor table, kv_num answers), and its outcome on each broken variant
    kvs, tensors = GW.tiny_model()
    good = GW.gguf_bytes(kvs, tensors, alignment=64)
    path = os.path.join(HERE, "tiny.gguf")
    with open(path, "wb") as f:
        f.write(good)
    tab = ref.gguf_table(path, GW.KV_QUERIES)
    rcs = {}
    for name, data in GW.variants(good).items():
        vp = os.path.join(HERE, f"_variant_{name}.gguf")
        with open(vp, "wb") as f:
            f.write(data)
        rcs[name] = 0 if ref.gguf_table(vp, GW.KV_QUERIES) is not None else -1
        os.remove(vp)
    np.savez_compressed(os.path.join(HERE, "gguf.npz"), **tab, variant_names=np.array(list(rcs)),
                        variant_rc=np.array(list(rcs.values()), np.int32))
    # attention: the reference's attn_rows on up to 4 rows sharing one head offset, over ring caches
    np.savez_compressed(os.path.join(HERE, "attn.npz"), **attn_cases(ref))
    # TurboQuant KV cache: the reference's rotation signs, rotations, slice records and its
    # attention step over quantized ring caches
    np.savez_compressed(os.path.join(HERE, "kvq.npz"), **kvq_cases(ref))
    np.savez_compressed(os.path.join(HERE, "lowbit.npz"), **lowbit_cases(ref))
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz") or f.endswith(".gguf"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
