#!/usr/bin/env python3
"""Benchmark of the quantized weight x Q8-activation hot path on one MI355X.

Workload: one Llama-3-8B-shaped decode layer as Q4_K matvecs at batch 1:
fused QKV 4096->6144, O 4096->4096, and the SiLU FFN: gate and up 4096->14336 (one shared
activation), h = silu(gate) * up, down 14336->h->4096 (forward, fastgguf.c:4870-4877, through
fgh_ffn_dev: the paired gate / up launch writes h, the down matvec reads it). A step quantizes each
input vector on the device (bit-exact Q8_K) and runs the five matvecs in four launches. Weights are
seeded synthetic Q4_K blocks with the benchmark's distributions; inputs are
fp32 N(0,1) vectors already resident in HBM. To measure HBM and not the 256 MB Infinity Cache,
steps rotate over COPIES distinct device copies of the layer (>= 512 MB in total). Steps are
recorded as a real decode replays them: one HIP graph holds GRAPH_LAYERS consecutive layers
(32, Llama-3-8B's depth), so the per-graph launch cost is spread over the layers it holds.

value  = whole-layer algorithmic bytes (weights + fp32 x in + fp32 y out of the five matvecs) /
         step time, in GB/s.
roofline: the dominant kernel of the step is the Q4_K decode launch of the FFN gate and up
         projections paired (4096->2x14336 in one launch that writes h = silu(g) * u); its duration
         is the mean over back-to-back launches captured in one HIP graph and timed with HIP events
         on the library's stream. The matvec_multi launch of gate and up (g and u stored) is
         reported beside it. Every per-kernel timing rotates over at least 512 MB of distinct
         weight copies.
prefill: BASELINE config 4 (64 tokens x 4096 -> 14336, Q4_K) on the int8 MFMA GEMM, timed the
         same way, cold (rotating weights) and Infinity-Cache hot, as TOPS and fraction of 5 POPS;
         the same shape in Q8_0, Q6_K and Q4_0 on their MFMA GEMMs, and the FFN down projection
         of the same tokens (14336 -> 4096, where the GEMMs split K) in Q4_K, Q6_K and Q8_0,
         against their HBM floors.
other configs: BASELINE configs 1, 3 and 5 (Q8_0 matvec, Q6_K LM head, the MoE FFN at 1 and 64
         tokens), the low-bit types Q2_K, Q3_K and IQ4_XS and the float types F32, F16 and BF16
         at the gate shape 4096 -> 14336, against the same HBM peak.
cpu_baseline: the reference's own CPU kernels (oracle/_ref, compiled from fastgguf.c) on the same
         layer's five matvecs with its default repacked Q4_K path (its silu loop, 14336 expf, is
         not in the sample), on this host's physical cores, over weight copies beyond the host's
         L3, for a bounded sample.
Prints one JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Q4_K decode matvec HBM GB/s (%peak); 64-tok prefill int8 TOPS (%MFMA peak)"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0  # dense int8 MFMA, MI355X
LAYER = [  # name, rows (outputs), cols (inputs)
    ("qkv", 6144, 4096),
    ("o", 4096, 4096),
    ("gate", 14336, 4096),
    ("up", 14336, 4096),
    ("down", 4096, 14336),
]


def algo_bytes(rows: int, cols: int) -> int:
    """weight bytes of the Q4_K blocks read + fp32 x in + fp32 y out"""
    return rows * (cols // 256) * 144 + 4 * cols + 4 * rows


# the gate and up projections in one launch: both matrices, x read once, both outputs
GATE_UP_BYTES = 2 * algo_bytes(14336, 4096) - 4 * 4096
# the same paired into one launch that writes h = silu(g) * u: one output instead of two
GATE_UP_SILU_BYTES = GATE_UP_BYTES - 4 * 14336


ROT_BYTES = 512e6  # a per-kernel timing rotates over at least this many bytes of weights


def copies_for(nbytes: int, least: int = 1) -> int:
    return max(least, -(-int(ROT_BYTES) // nbytes))


def host_cpu() -> dict:
    """This process's CPUs: model, sockets, physical cores and logical CPUs it may run on, and the
    total L3 over the sockets (sysfs and /proc/cpuinfo). Taken before the GPU is initialised: the
    runtime may pin the calling thread afterwards."""
    cpus = sorted(os.sched_getaffinity(0))
    cores, pkgs, l3 = set(), set(), {}
    for c in cpus:
        base = f"/sys/devices/system/cpu/cpu{c}"
        try:
            pkg = int(open(f"{base}/topology/physical_package_id").read())
            core = int(open(f"{base}/topology/core_id").read())
        except OSError:
            pkg, core = 0, c
        pkgs.add(pkg)
        cores.add((pkg, core))
        try:
            shared = open(f"{base}/cache/index3/shared_cpu_list").read().strip()
            size = open(f"{base}/cache/index3/size").read().strip()
            l3[shared] = int(size[:-1]) * (1024 if size.endswith("K") else 1024 * 1024 if size.endswith("M") else 1)
        except (OSError, ValueError):
            pass
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"model": model, "sockets": len(pkgs), "physical_cores": len(cores), "logical_cpus": len(cpus),
            "l3_bytes": sum(l3.values()), "l3_instances": len(l3)}


def counted_traffic(kernel: str):
    """HBM bytes per launch measured by the rocprofv3 FETCH_SIZE / WRITE_SIZE passes recorded in
    profiles/ (scaled by a plain copy kernel of known size), or None if not recorded."""
    path = os.path.join(ROOT, "profiles", "q4k_gate_up_decode_prefill_gemm_hbm_counters.md")
    try:
        for line in open(path):
            f = line.split()
            if len(f) == 3 and f[0] == "traffic_bytes_per_launch" and f[1] == kernel:
                return int(f[2])
    except OSError:
        pass
    return None


GRAPH_LAUNCHES = 50  # back-to-back launches of one kernel per timed HIP graph


def kernel_time_on(be, launch, reps: int) -> float:
    """GRAPH_LAUNCHES back-to-back launches of one call (rotating over weight copies) captured in
    one HIP graph, replayed and timed with HIP events on the library's stream: us per launch (the
    kernel's duration plus the in-graph gap between launches)."""
    launch(0)  # grows any scratch before capture
    be.graph_begin()
    for i in range(GRAPH_LAUNCHES):
        launch(i)
    gr = be.graph_end()
    be.graph_launch(gr)
    be.sync()
    a, b = be.event(), be.event()
    n = max(1, reps // GRAPH_LAUNCHES)
    be.record(a)
    for _ in range(n):
        be.graph_launch(gr)
    be.record(b)
    be.sync()
    t = be.elapsed_ms(a, b)
    be.event_destroy(a)
    be.event_destroy(b)
    be.graph_destroy(gr)
    return t * 1e3 / (n * GRAPH_LAUNCHES)  # us


def other_configs(be, S, kernel_time, enabled: int) -> dict | None:
    """BASELINE configs 1 (Q8_0 4096^2 matvec), 3 (Q6_K LM head 128256 x 4096) and 5 (MoE, 128
    experts, top-8, hidden 2048, ff 768: batch 1 and 64 tokens), each timed like the kernels above,
    and the other weight types' decode lines (low-bit and float types at the gate shape, Q4_0 and
    Q8_0 at two long-row down shapes).
    Weight sets rotate where one copy would stay in the Infinity Cache."""
    if not enabled:
        return None
    import numpy as np
    out = {}
    # config 1: Q8_0 4096 x 4096, 32 copies (571 MB)
    w = S.q8_0_weights(4096, 4096, seed=110)
    ts = [be.upload(S.T_Q8_0, 4096, w) for _ in range(32)]
    x, y = be.dev_alloc(4 * 4096), be.dev_alloc(4 * 4096)
    be.h2d(x, S.activations(4096, 111))
    us = kernel_time(lambda i: be.matvec_dev(ts[i % 32], x, y), 200)
    nbytes = 4096 * 128 * 34 + 4 * 8192
    out["cfg1_q8_0_matvec"] = {"us": round(us, 3), "GB/s": round(nbytes / us / 1e3, 1),
                               "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "bytes": nbytes}
    for t in ts:
        t.free()
    be.dev_free(y)
    # config 3: Q6_K LM head, one copy (431 MB: beyond the Infinity Cache by itself)
    w = S.q6_k_weights(128256, 4096, seed=120)
    t = be.upload(S.T_Q6_K, 4096, w)
    del w
    y = be.dev_alloc(4 * 128256)
    us = kernel_time(lambda i: be.matvec_dev(t, x, y), 50)
    nbytes = 128256 * 16 * 210 + 4 * (4096 + 128256)
    out["cfg3_q6_k_lm_head"] = {"us": round(us, 3), "GB/s": round(nbytes / us / 1e3, 1),
                                "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "bytes": nbytes}
    t.free()
    be.dev_free(y)
    # the low-bit types (Q2_K, Q3_K, IQ4_XS; fgh_kq.hip) at the gate shape 4096 -> 14336, weight
    # copies rotating past the Infinity Cache
    for name, ty in (("q2_k", S.T_Q2_K), ("q3_k", S.T_Q3_K), ("iq4_xs", S.T_IQ4_XS)):
        wb = 14336 * S.row_bytes(ty, 4096)
        n = copies_for(wb)
        w = S.weights(ty, 14336, 4096, 130 + ty)
        ts = [be.upload(ty, 4096, w) for _ in range(n)]
        del w
        y = be.dev_alloc(4 * 14336)
        us = kernel_time(lambda i: be.matvec_dev(ts[i % n], x, y), 200)
        nbytes = wb + 4 * (4096 + 14336)
        out[f"lowbit_{name}_gate_matvec"] = {"us": round(us, 3), "GB/s": round(nbytes / us / 1e3, 1),
                                              "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "bytes": nbytes,
                                              "copies": n}
        for t in ts:
            t.free()
        be.dev_free(y)
    # the float types (F32, F16, BF16; fgh_float.hip) at the same shape: x in fp32, no quantization
    for name, ty in (("f32", S.T_F32), ("f16", S.T_F16), ("bf16", S.T_BF16)):
        wb = 14336 * S.row_bytes(ty, 4096)
        n = copies_for(wb)
        w = S.weights(ty, 14336, 4096, 140 + ty)
        ts = [be.upload(ty, 4096, w) for _ in range(n)]
        del w
        y = be.dev_alloc(4 * 14336)
        us = kernel_time(lambda i: be.matvec_dev(ts[i % n], x, y), 100)
        nbytes = wb + 4 * (4096 + 14336)
        out[f"float_{name}_gate_matvec"] = {"us": round(us, 3), "GB/s": round(nbytes / us / 1e3, 1),
                                             "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "bytes": nbytes,
                                             "copies": n}
        for t in ts:
            t.free()
        be.dev_free(y)
    be.dev_free(x)
    # two 32-value types over long rows (Q4_0 in its repacked order): the down projection
    # 14336 -> 4096 (512 tiles: the launches split each tile's steps over wavefronts) and
    # Llama-2-13B's down projection 13824 -> 5120 (640 tiles: unsplit, with deep rings)
    x = be.dev_alloc(4 * 14336)
    be.h2d(x, S.activations(14336, 150))
    for tag, rows, cols in (("down", 4096, 14336), ("13b_down", 5120, 13824)):
        for name, ty in (("q4_0", S.T_Q4_0), ("q8_0", S.T_Q8_0)):
            wb = rows * S.row_bytes(ty, cols)
            n = copies_for(wb)
            w = S.weights(ty, rows, cols, 150 + ty)
            ts = [be.upload(ty, cols, w) for _ in range(n)]
            del w
            y = be.dev_alloc(4 * rows)
            us = kernel_time(lambda i: be.matvec_dev(ts[i % n], x, y), 100)
            nbytes = wb + 4 * (rows + cols)
            out[f"long_rows_{name}_{tag}_matvec"] = {"us": round(us, 3), "GB/s": round(nbytes / us / 1e3, 1),
                                                     "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4),
                                                     "bytes": nbytes, "copies": n}
            for t in ts:
                t.free()
            be.dev_free(y)
    be.dev_free(x)
    # config 5: MoE FFN, 2 expert sets (531 MB)
    E, K, D, F = 128, 8, 2048, 768
    sets = []
    for c in range(2):
        g = be.upload(S.T_Q4_K, D, S.q4_k_weights(E * F, D, seed=300 + 3 * c), rows=F, n_mats=E)
        u = be.upload(S.T_Q4_K, D, S.q4_k_weights(E * F, D, seed=301 + 3 * c), rows=F, n_mats=E)
        d = be.upload(S.T_Q4_K, F, S.q4_k_weights(E * D, F, seed=302 + 3 * c), rows=D, n_mats=E)
        sets.append((g, u, d))
    expert_bytes = 2 * F * (D // 256) * 144 + D * (F // 256) * 144
    for T, NL in ((1, 16), (64, 1)):
        # batch 1: 16 logits rows in turn, so that successive calls select other experts (each
        # call's 8 experts come from HBM, not from the cache a previous call filled)
        X = S.activations(D, 310, rows=T)
        L = S.router_logits(T * NL, E, 311)
        xd, ld, yd = be.dev_alloc(X.nbytes), be.dev_alloc(L.nbytes), be.dev_alloc(X.nbytes)
        be.h2d(xd, X)
        be.h2d(ld, L)
        us = kernel_time(lambda i: be.moe_ffn_dev(*sets[i % 2], K, ld + ((i // 2) % NL) * T * E * 4, xd, yd, T), 100)
        # distinct experts a call's tokens select (the oracle's routing, same as the device's),
        # averaged over the logits rows
        nsel = []
        for c in range(NL):
            sel = set()
            for r in range(c * T, (c + 1) * T):
                p = np.exp(L[r] - L[r].max())
                sel.update(np.argsort(-p, kind="stable")[:K].tolist())
            nsel.append(len(sel))
        sel = range(round(sum(nsel) / NL))
        nbytes = len(sel) * expert_bytes + 4 * T * (2 * D + E)
        ops = 2.0 * T * K * (2 * F * D + D * F)
        out[f"cfg5_moe_{T}tok"] = {"us": round(us, 3), "GB/s": round(nbytes / us / 1e3, 1),
                                   "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "bytes": nbytes,
                                   "distinct_experts": len(sel), "logits_rows": NL, "TOPS": round(ops / us / 1e6, 3)}
        for p_ in (xd, ld, yd):
            be.dev_free(p_)
    for st in sets:
        for t in st:
            t.free()
    # config 5 at 64 tokens on the grouped path's other expert kernel (the VALU lane chains,
    # FGH_MOE_KERNEL=valu; same bits), beside the default int8 MFMA kernels above
    os.environ["FGH_MOE_KERNEL"] = "valu"
    try:
        from fastgguf_amd.backend import Backend
        bv = Backend(0)
    finally:
        os.environ.pop("FGH_MOE_KERNEL", None)
    vsets = [(bv.upload(S.T_Q4_K, D, S.q4_k_weights(E * F, D, seed=300 + 3 * c), rows=F, n_mats=E),
              bv.upload(S.T_Q4_K, D, S.q4_k_weights(E * F, D, seed=301 + 3 * c), rows=F, n_mats=E),
              bv.upload(S.T_Q4_K, F, S.q4_k_weights(E * D, F, seed=302 + 3 * c), rows=D, n_mats=E)) for c in range(2)]
    T = 64
    X = S.activations(D, 310, rows=T)
    L = S.router_logits(T, E, 311)
    xd, ld, yd = bv.dev_alloc(X.nbytes), bv.dev_alloc(L.nbytes), bv.dev_alloc(X.nbytes)
    bv.h2d(xd, X)
    bv.h2d(ld, L)
    us = kernel_time_on(bv, lambda i: bv.moe_ffn_dev(*vsets[i % 2], K, ld, xd, yd, T), 100)
    m = out["cfg5_moe_64tok"]
    out["cfg5_moe_64tok_valu_kernel"] = {"us": round(us, 3), "GB/s": round(m["bytes"] / us / 1e3, 1),
                                         "frac": round(m["bytes"] / us / 1e3 / HBM_PEAK_GBS, 4),
                                         "TOPS": round(m["TOPS"] * m["us"] / us, 3)}
    m["kernel"] = "int8 MFMA (default)"
    m["frac_mfma_peak"] = round(m["TOPS"] / (INT8_PEAK_TOPS), 5)
    out["cfg5_moe_64tok_valu_kernel"]["frac_mfma_peak"] = round(out["cfg5_moe_64tok_valu_kernel"]["TOPS"] / INT8_PEAK_TOPS, 5)
    for p_ in (xd, ld, yd):
        bv.dev_free(p_)
    for st in vsets:
        for t in st:
            t.free()
    bv.close()
    return out


def attention_config(be, kernel_time, enabled: int, cpu_in: dict) -> dict | None:
    """Attention over the fp32 KV ring cache (attn_rows, fastgguf.c:3273-3326) at Llama-3-8B's shape
    (32 query heads over 8 K / V heads, hd 128): one decode token over 4096 positions, and a 64-token
    prompt batch at the end of a 4096-position context; then the same over TurboQuant K4 / V4 caches
    (fastgguf.c:3341-3513) written from the same rows. cpu_in receives the decode cases' host
    inputs, for the reference's CPU timing in cpu_baseline."""
    if not enabled:
        return None
    import numpy as np
    rng = np.random.default_rng(400)
    cap, hd, nh, nkv = 4096, 128, 32, 8
    kv_dim = nkv * hd
    ck = rng.standard_normal((cap, kv_dim)).astype(np.float32)
    cv = rng.standard_normal((cap, kv_dim)).astype(np.float32)
    kd, vd = be.dev_alloc(ck.nbytes), be.dev_alloc(cv.nbytes)
    be.h2d(kd, ck)
    be.h2d(vd, cv)
    scale = float(np.float32(1 / np.sqrt(hd)))
    out = {"shape": "32 heads over 8 K/V heads, hd 128, fp32 cache of 4096 positions"}
    for name, nt in (("decode_4096", 1), ("prefill_64_at_4096", 64)):
        q = rng.standard_normal((nt, nh, hd)).astype(np.float32)
        en = (10000 + np.arange(nt)).astype(np.int32)
        st = (en[-1] - cap + 1) * np.ones(nt, np.int32)
        bufs = [be.dev_alloc(a.nbytes) for a in (q, q, st, en)]
        for b, a in zip(bufs, (q, q, st, en)):
            be.h2d(b, a)
        n_max = int((en - st).max()) + 1
        us = kernel_time(lambda i: be.attention_dev(nt, nh, nkv, hd, bufs[0], bufs[1], kd, vd, kv_dim, cap, bufs[2],
                                                    bufs[3], n_max, scale), 100)
        kv_bytes = 2 * n_max * kv_dim * 4
        fmas = 2 * int((en - st + 1).sum()) * nh * hd
        out[name] = {"us": round(us, 2), "kv_bytes": kv_bytes, "kv_GB/s": round(kv_bytes / us / 1e3, 1),
                     "fma_G/s": round(fmas / us / 1e3, 1)}
        if nt == 1:
            cpu_in.update(q=q[0], st=st, en=en, ck=ck, cv=cv, hd=hd, nh=nh, nkv=nkv, scale=scale)
        for b in bufs:
            be.dev_free(b)
    # TurboQuant K4 / V4 caches written from the same K / V rows (the cache write timed per token
    # and per 64-token batch), then the same two attention calls over them
    kb, vb = 4, 4
    kqs, vqs = nkv * (4 + hd * kb // 8), nkv * (4 + hd * vb // 8)
    kqd, vqd = be.dev_alloc(cap * kqs), be.dev_alloc(cap * vqs)
    posd = be.dev_alloc(4 * cap)
    be.h2d(posd, np.arange(cap, dtype=np.int32))
    be.kvq_store_dev(cap, nkv, hd, kb, vb, kd, vd, kv_dim, kqd, vqd, cap, posd)
    for nt in (1, 64):
        us = kernel_time(lambda i: be.kvq_store_dev(nt, nkv, hd, kb, vb, kd, vd, kv_dim, kqd, vqd, cap, posd), 100)
        out[f"turbo_k4v4_store_{nt}tok"] = {"us": round(us, 2)}
    for name, nt in (("turbo_k4v4_decode_4096", 1), ("turbo_k4v4_prefill_64_at_4096", 64)):
        q = rng.standard_normal((nt, nh, hd)).astype(np.float32)
        en = (10000 + np.arange(nt)).astype(np.int32)
        st = (en[-1] - cap + 1) * np.ones(nt, np.int32)
        bufs = [be.dev_alloc(a.nbytes) for a in (q, q, st, en)]
        for b, a in zip(bufs, (q, q, st, en)):
            be.h2d(b, a)
        n_max = int((en - st).max()) + 1
        us = kernel_time(lambda i: be.kvq_attention_dev(nt, nh, nkv, hd, kb, vb, bufs[0], bufs[1], kqd, vqd, cap,
                                                        bufs[2], bufs[3], n_max, scale), 100)
        out[name] = {"us": round(us, 2), "cache_bytes": n_max * (kqs + vqs)}
        if nt == 1:
            kq, vq = np.zeros((cap, kqs), np.uint8), np.zeros((cap, vqs), np.uint8)
            be.d2h(kq, kqd)
            be.d2h(vq, vqd)
            cpu_in.update(tq=q[0], kq=kq, vq=vq, kbits=kb, vbits=vb)
        for b in bufs:
            be.dev_free(b)
    for b in (kqd, vqd, posd, kd, vd):
        be.dev_free(b)
    return out


def cpu_attention(ref, a: dict) -> dict:
    """The reference's attention on the bench's decode cases, one thread: attn_rows in 4-row calls
    per K / V head as its forward makes, and its TurboQuant attention step per head."""
    import numpy as np
    out = {}
    if "q" in a:
        t0 = time.perf_counter()
        for _ in range(5):
            for h in range(a["nkv"]):
                ref.attn_rows(a["q"][4 * h:4 * h + 4], np.repeat(a["st"], 4), np.repeat(a["en"], 4), a["ck"], a["cv"],
                              h * a["hd"], a["hd"], a["scale"])
        out["attention_decode_4096_1thread_us"] = round((time.perf_counter() - t0) / 5 * 1e6, 1)
    if "tq" in a:
        nh = a["nh"]
        kvh = np.arange(nh) // (nh // a["nkv"])
        t0 = time.perf_counter()
        for _ in range(3):
            ref.kvq_attn_rows(a["tq"], np.repeat(a["st"], nh), np.repeat(a["en"], nh), a["kq"], a["vq"], kvh, a["hd"],
                              a["kbits"], a["vbits"], a["scale"])
        out["turbo_k4v4_decode_4096_1thread_us"] = round((time.perf_counter() - t0) / 3 * 1e6, 1)
    return out


def cpu_baseline(layer_w: dict, xs: dict, budget_s: float, cpu: dict, attn_in: dict | None = None) -> dict | None:
    """The reference's CPU path on the same layer (oracle/_ref), median over a bounded sample; and
    on the bench's attention decode cases (attn_in, from attention_config)."""
    try:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        from oracle import Reference
        ref = Reference()
    except (FileNotFoundError, OSError) as e:
        print(f"[bench] cpu baseline skipped: {e}", file=sys.stderr)
        return None
    import numpy as np

    from fastgguf_amd.synth import T_Q4_K
    per_copy = sum(r * (c // 256) * 144 for _, r, c in LAYER)
    copies = max(3, -(-int(1.5 * cpu["l3_bytes"]) // per_copy))  # the weights stream past the L3
    hs = [{n: ref.tensor(T_Q4_K, layer_w[n], c, repack=True) for n, r, c in LAYER} for _ in range(copies)]
    ys = {n: np.zeros(r, np.float32) for n, r, c in LAYER}

    def layer(k: int):
        h = hs[k % copies]
        ref.tensor_matvec_multi([h["qkv"]], xs["x"], [ys["qkv"]])
        ref.tensor_matvec_multi([h["o"]], xs["a"], [ys["o"]])
        ref.tensor_matvec_multi([h["gate"], h["up"]], xs["x2"], [ys["gate"], ys["up"]])  # forward 4870-4872
        ref.tensor_matvec_multi([h["down"]], xs["h"], [ys["down"]])

    for k in range(3):
        layer(k)
    times = []
    t_end = time.perf_counter() + budget_s
    k = 0
    while (time.perf_counter() < t_end and k < 5000) or k < 20:
        t0 = time.perf_counter()
        layer(k)
        times.append(time.perf_counter() - t0)
        k += 1
    for h in hs:
        for v in h.values():
            ref.tensor_free(v)
    med = float(np.median(times))
    total = sum(algo_bytes(r, c) for _, r, c in LAYER)
    return {"value": round(total / med / 1e9, 2), "unit": "GB/s", "cores": ref.threads(), "kind": "reference",
            "sample": f"{len(times)} decode layers (median {med * 1e6:.0f} us/layer), fastgguf.c matvec/"
                      f"matvec_multi on repacked Q4_K, {ref.build} build, {copies} rotating weight copies "
                      f"({copies * per_copy / 1e6:.0f} MB, 1.5x the L3 or more)",
            "ms_per_step": round(med * 1e3, 3), "cpu": cpu, "omp_places": os.environ.get("OMP_PLACES"),
            "omp_proc_bind": os.environ.get("OMP_PROC_BIND"),
            "numa": "one process, no numactl in this image (no --interleave=all run)",
            **cpu_attention(ref, attn_in or {})}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--copies", type=int, default=5, help="distinct device copies of the layer")
    ap.add_argument("--graph-layers", type=int, default=32, help="decode layers per replayed HIP graph")
    ap.add_argument("--kernel-reps", type=int, default=200, help="individually timed gate matvecs")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline sample budget (0 = skip)")
    ap.add_argument("--configs", type=int, default=1, help="also time BASELINE configs 1, 3 and 5 (0 = skip)")
    ap.add_argument("--attention", type=int, default=1, help="also time the attention calls (0 = skip)")
    ap.add_argument("--profile-kernels", action="store_true",
                    help="only run 20 gate matvecs, 20 copies of the same byte count by a plain copy kernel, "
                         "and 20 prefill GEMMs, eagerly (for rocprofv3 --pmc counter passes)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (this build has no multi-GPU "
              "path: every GPU box here has one GPU)", file=sys.stderr)
        return 2
    # the CPU leg: one thread per physical core this process may use, pinned to cores
    host = host_cpu()
    os.environ.setdefault("OMP_NUM_THREADS", str(max(1, host["physical_cores"])))
    os.environ.setdefault("OMP_PROC_BIND", "close")
    os.environ.setdefault("OMP_PLACES", "cores")

    import numpy as np

    from fastgguf_amd import synth as S
    from fastgguf_amd.backend import Backend

    be = Backend(0)
    layer_w = {n: S.q4_k_weights(r, c, seed=100 + i) for i, (n, r, c) in enumerate(LAYER)}
    tensors = [{n: be.upload(S.T_Q4_K, c, layer_w[n]) for n, r, c in LAYER} for _ in range(args.copies)]
    xs = {"x": S.activations(4096, 1), "a": S.activations(4096, 2), "x2": S.activations(4096, 3),
          "h": S.activations(14336, 4)}
    xd = {k: be.dev_alloc(v.nbytes) for k, v in xs.items()}
    for k, v in xs.items():
        be.h2d(xd[k], v)
    yd = {n: be.dev_alloc(4 * r) for n, r, c in LAYER}
    yd["h"] = be.dev_alloc(4 * 14336)

    if args.profile_kernels:
        gu_bytes = GATE_UP_BYTES
        cbytes = (gu_bytes + 15) // 16 * 16
        src, dst = be.dev_alloc(cbytes), be.dev_alloc(cbytes)
        Xp = S.activations(4096, 5, rows=64)
        xpd, ypd = be.dev_alloc(Xp.nbytes), be.dev_alloc(4 * 64 * 14336)
        be.h2d(xpd, Xp)
        for i in range(20):
            t = tensors[i % args.copies]
            be.matvec_multi_dev([t["gate"], t["up"]], xd["x2"], [yd["gate"], yd["up"]])
        for i in range(20):
            t = tensors[i % args.copies]
            be.matvec_gate_up_silu_dev(t["gate"], t["up"], xd["x2"], yd["h"])
        for i in range(20):
            be.d2d(dst, src, cbytes)
        for i in range(20):
            be.matmul_dev(tensors[i % args.copies]["up"], xpd, ypd, 64)
        be.sync()
        print(json.dumps({"profile_kernels": True, "gate_up_bytes": gu_bytes, "copy_bytes": cbytes,
                          "gemm_ops": 2 * 64 * 4096 * 14336}), flush=True)
        be.close()
        return 0

    def record_layer(t):
        be.matvec_dev(t["qkv"], xd["x"], yd["qkv"])
        be.matvec_dev(t["o"], xd["a"], yd["o"])
        be.ffn_dev(t["gate"], t["up"], t["down"], xd["x2"], yd["h"], yd["down"])  # forward 4870-4877

    # a step is one decode layer (5 matvecs and the silu loop in 4 launches, each quantizing its input on the
    # device); GRAPH_LAYERS consecutive layers (cycling the weight copies) form one HIP graph, as a
    # whole decode step of the model is one graph; K steps replay K / L graphs plus one graph of
    # the remaining K % L layers, so exactly K layers are timed
    L = max(1, args.graph_layers)

    def layer_graph(first: int, n: int):
        be.graph_begin()
        for j in range(n):
            record_layer(tensors[(first + j) % args.copies])
        return be.graph_end()

    graphs = [layer_graph(i * L, L) for i in range(args.copies)]
    rest = layer_graph(0, args.steps % L) if args.steps % L else None
    for k in range(max(1, -(-args.warmup // L))):
        be.graph_launch(graphs[k % args.copies])
    be.sync()
    e0, e1 = be.event(), be.event()
    be.sync()
    be.record(e0)
    for k in range(args.steps // L):
        be.graph_launch(graphs[k % args.copies])
    if rest is not None:
        be.graph_launch(rest)
    be.record(e1)
    ms = be.elapsed_ms(e0, e1)
    be.sync()
    ms_step = ms / args.steps
    # the same layers one graph each (the per-graph launch cost included), for comparison
    g1 = [layer_graph(i, 1) for i in range(args.copies)]
    n1 = min(args.steps, 100)
    be.record(e0)
    for k in range(n1):
        be.graph_launch(g1[k % args.copies])
    be.record(e1)
    be.sync()
    ms_step_1 = be.elapsed_ms(e0, e1) / n1
    for g in graphs + g1 + ([rest] if rest is not None else []):
        be.graph_destroy(g)
    layer_bytes = sum(algo_bytes(r, c) for _, r, c in LAYER)
    value = layer_bytes / (ms_step * 1e-3) / 1e9

    # per-kernel durations (kernel_time_on): graphs of back-to-back launches of one kernel
    def kernel_time(launch, reps: int) -> float:
        return kernel_time_on(be, launch, reps)

    nc = args.copies
    # per-kernel rotations: the layer copies plus more of each matrix, at least ROT_BYTES each
    rot = {}
    for n, r, c in LAYER:
        rot[n] = [t[n] for t in tensors]
        while len(rot[n]) < copies_for(r * (c // 256) * 144):
            rot[n].append(be.upload(S.T_Q4_K, c, layer_w[n]))
    extra = [t for n in rot for t in rot[n][nc:]]
    ngu = min(len(rot["gate"]), len(rot["up"]))
    launches = {
        "qkv": (lambda i: be.matvec_dev(rot["qkv"][i % len(rot["qkv"])], xd["x"], yd["qkv"]), algo_bytes(6144, 4096)),
        "o": (lambda i: be.matvec_dev(rot["o"][i % len(rot["o"])], xd["a"], yd["o"]), algo_bytes(4096, 4096)),
        "gate": (lambda i: be.matvec_dev(rot["gate"][i % len(rot["gate"])], xd["x2"], yd["gate"]),
                 algo_bytes(14336, 4096)),
        "gate+up": (lambda i: be.matvec_multi_dev([rot["gate"][i % ngu], rot["up"][i % ngu]], xd["x2"],
                                                 [yd["gate"], yd["up"]]), GATE_UP_BYTES),
        "down": (lambda i: be.matvec_dev(rot["down"][i % len(rot["down"])], xd["h"], yd["down"]),
                 algo_bytes(4096, 14336)),
        # gate and up paired in one launch that writes h = silu(g) * u (the loop between the FFN's
        # matvecs): the layer's FFN launch and its dominant kernel
        "gate+up+silu": (lambda i: be.matvec_gate_up_silu_dev(rot["gate"][i % ngu], rot["up"][i % ngu], xd["x2"],
                                                             yd["gate"]), GATE_UP_SILU_BYTES),
        "ffn": (lambda i: be.ffn_dev(rot["gate"][i % ngu], rot["up"][i % ngu], rot["down"][i % len(rot["down"])],
                                     xd["x2"], yd["h"], yd["down"]),
                GATE_UP_SILU_BYTES + algo_bytes(4096, 14336)),
    }
    kernels = {}
    for n, (fn, nbytes) in launches.items():
        us = kernel_time(fn, args.kernel_reps)
        gbs = nbytes / (us * 1e-6) / 1e9
        kernels[n] = {"us": round(us, 3), "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                      "rotation_MB": round(nbytes * (ngu if n.startswith("gate+up") else
                                                     min(ngu, len(rot["down"])) if n == "ffn" else len(rot[n])) / 1e6)}
    # the HBM rate this box delivers to a plain stream (fgh_checksum_dev: each workgroup reads one
    # contiguous share with nontemporal 16-byte loads, a sum and nothing else, the fastest read of a
    # sweep of shapes), at the gate+up byte count and at 1 GB, each rotating over at least 2 GB of
    # buffers; and the HIP runtime's own device-to-device copy of 1 GB (hipMemcpyAsync, read plus
    # write bytes), an independent figure
    def read_rate(nbytes: int, reps: int):
        nbytes = (nbytes + 15) // 16 * 16
        n = max(2, -(-int(4 * ROT_BYTES) // nbytes))
        bufs = [be.dev_alloc(nbytes) for _ in range(n)]
        us = kernel_time(lambda i: be.checksum_dev(bufs[i % n], nbytes, 0), reps)  # streaming pass only
        for p in bufs:
            be.dev_free(p)
        return nbytes, us, n
    rbytes, rus, nr = read_rate(GATE_UP_BYTES, args.kernel_reps)
    rgbs = rbytes / (rus * 1e-6) / 1e9
    gbytes, gus, ngb = read_rate(1 << 30, 50)
    ggbs = gbytes / (gus * 1e-6) / 1e9
    cbytes = 1 << 30
    cbufs = [be.dev_alloc(cbytes) for _ in range(4)]
    cus = kernel_time(lambda i: be.memcpy_dev(cbufs[2 * (i % 2) + 1], cbufs[2 * (i % 2)], cbytes), 50)
    for p in cbufs:
        be.dev_free(p)
    cgbs = 2 * cbytes / (cus * 1e-6) / 1e9
    read_reference = {"kernel": "checksum_part_kernel (plain streaming read: contiguous share per workgroup, "
                                "nontemporal 16-byte loads)",
                      "bytes": rbytes, "us": round(rus, 3), "GB/s": round(rgbs, 1), "frac": round(rgbs / HBM_PEAK_GBS, 4),
                      "rotation_MB": round(nr * rbytes / 1e6),
                      "at_1GB": {"bytes": gbytes, "us": round(gus, 3), "GB/s": round(ggbs, 1),
                                 "frac": round(ggbs / HBM_PEAK_GBS, 4), "rotation_MB": round(ngb * gbytes / 1e6)},
                      "hipMemcpyAsync_1GB": {"bytes_read_plus_written": 2 * cbytes, "us": round(cus, 3),
                                             "GB/s": round(cgbs, 1), "frac": round(cgbs / HBM_PEAK_GBS, 4)}}

    # the int8 MFMA rate a kernel that runs nothing but MFMA chains gets on this box: the attainable
    # peak beside the published 5.0 POPS (fgh_mfma_peak_dev, 2000 rounds per launch)
    mops = be.mfma_peak_dev(2000)
    mus = kernel_time(lambda i: be.mfma_peak_dev(2000), 40)
    mtops = mops / (mus * 1e-6) / 1e12
    mfma_reference = {"kernel": "mfma_peak_kernel (8 independent v_mfma_i32_16x16x64_i8 chains per wavefront, "
                                "8 wavefronts per compute unit, no memory traffic)",
                      "ops": mops, "us": round(mus, 3), "TOPS": round(mtops, 1),
                      "frac": round(mtops / INT8_PEAK_TOPS, 4)}

    g = kernels["gate+up+silu"]
    roofline = {"bound": "hbm", "achieved": g["GB/s"], "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": g["frac"],
                "traffic": counted_traffic("gate_up_silu"),
                "kernel": "q4k_mv_kernel<repacked, 1 wavefront per 16-row tile, gate/up paired> (Q4_K decode matvec, "
                          "FFN gate + up 4096->2x14336 in one launch writing h = silu(g) * u)",
                "bytes_per_launch": GATE_UP_SILU_BYTES, "us_per_launch": g["us"],
                "frac_of_read_reference": round(g["GB/s"] / rgbs, 4),
                "frac_of_read_reference_1GB": round(g["GB/s"] / ggbs, 4)}

    # prefill: 64 tokens x 4096 -> 14336 Q4_K on the int8 MFMA GEMM; one launch
    # = device Q8_K quantization of X + the GEMM. Cold: rotating over the 2 * COPIES distinct
    # gate/up matrices; hot: one matrix (Infinity-Cache resident).
    T = 64
    Xp = S.activations(4096, 5, rows=T)
    xpd = be.dev_alloc(Xp.nbytes)
    be.h2d(xpd, Xp)
    ypd = be.dev_alloc(4 * T * 14336)
    mats = [m for i in range(ngu) for m in (rot["gate"][i], rot["up"][i])]
    ops = 2.0 * T * 4096 * 14336
    prefill = {}
    for kind, pick in (("cold", lambda i: mats[i % len(mats)]), ("hot", lambda i: mats[0])):
        us = kernel_time(lambda i: be.matmul_dev(pick(i), xpd, ypd, T), args.kernel_reps)
        tops = ops / (us * 1e-6) / 1e12
        prefill[kind] = {"us": round(us, 3), "TOPS": round(tops, 2), "frac": round(tops / INT8_PEAK_TOPS, 4),
                         "frac_of_mfma_reference": round(tops / mtops, 4)}
    wq4 = 14336 * 16 * 144
    prefill.update({"workload": "cfg4: 64 tokens x K=4096 -> N=14336, Q4_K x Q8_K (quantization of X included)",
                    "ops_per_launch": ops, "peak_TOPS": INT8_PEAK_TOPS,
                    "kernel": "gemm_quant_kernel + q4k_gemm_kernel (int8 MFMA 16x16x64, split sub-block scales)",
                    "hbm_floor_us": round((wq4 + 4 * T * (4096 + 14336)) / HBM_PEAK_GBS / 1e3, 3),
                    "traffic": counted_traffic("prefill_gemm")})
    # the same shape in Q8_0, Q6_K and Q4_0 on their MFMA GEMMs (gemm_q32's and gemm_kquant's roles),
    # and the FFN down projection 14336 -> 4096 of the same 64 tokens (Q4_K on the layer's own down
    # copies; Q6_K, the down type of Q4_K_M files, and Q8_0: the GEMMs split K there), cold over
    # >= 512 MB of rotating copies and hot, against the HBM floor of their weights
    Xd = S.activations(14336, 6, rows=T)
    xdd = be.dev_alloc(Xd.nbytes)
    be.h2d(xdd, Xd)
    kname = {"q8_0": "q80_gemm_kernel (int8 MFMA 32x32x32, one block per K step)",
             "q6_k": "q6k_gemm_kernel (int8 MFMA 16x16x64, three scale-digit chains)",
             "q4_0": "q32n_gemm_kernel (int8 MFMA 16x16x32 per block, gemm_q32's fp32 order, bit-exact)",
             "q4_k": "gemm_quant_kernel + q4k_gemm_kernel (int8 MFMA 16x16x64, split sub-block scales)"}

    def prefill_line(name, ts, wbytes, rows, cols, xin):
        line = {}
        for kind, pick in (("cold", lambda i: ts[i % len(ts)]), ("hot", lambda i: ts[0])):
            us = kernel_time(lambda i: be.matmul_dev(pick(i), xin, ypd, T), args.kernel_reps)
            nbytes = wbytes + 4 * T * (rows + cols)
            line[kind] = {"us": round(us, 3), "GB/s": round(nbytes / us / 1e3, 1),
                          "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "TOPS": round(ops / us / 1e6, 2)}
        split = " (4 K splits)" if rows == 4096 else ""
        line.update({"workload": f"64 tokens x K={cols} -> N={rows}, {name.upper()}{split} (quantization of X included)",
                     "hbm_floor_us": round((wbytes + 4 * T * (rows + cols)) / HBM_PEAK_GBS / 1e3, 3),
                     "rotation_MB": round(len(ts) * wbytes / 1e6),
                     "kernel": kname[name]})
        return line

    prefill["q4_k_down"] = prefill_line("q4_k", rot["down"], 4096 * 56 * 144, 4096, 14336, xdd)
    for name, ty, wgen, bpr in (("q8_0", S.T_Q8_0, S.q8_0_weights, 34 / 32), ("q6_k", S.T_Q6_K, S.q6_k_weights, 210 / 256),
                                ("q4_0", S.T_Q4_0, lambda r, c, seed: S.weights(S.T_Q4_0, r, c, seed), 18 / 32)):
        for rows, cols, key, xin in ((14336, 4096, name, xpd), (4096, 14336, name + "_down", xdd)):
            if key == "q4_0_down":
                continue
            wbytes = int(rows * cols * bpr)
            w = wgen(rows, cols, seed=130)
            ts = [be.upload(ty, cols, w) for _ in range(copies_for(wbytes))]
            del w
            prefill[key] = prefill_line(name, ts, wbytes, rows, cols, xin)
            for t in ts:
                t.free()
    be.dev_free(xdd)
    for t in extra:
        t.free()
    be.dev_free(xpd)
    be.dev_free(ypd)

    others = other_configs(be, S, kernel_time, args.configs)
    attn_in = {}
    attention = attention_config(be, kernel_time, args.configs and args.attention, attn_in)

    cpu = cpu_baseline(layer_w, xs, args.cpu_seconds, host, attn_in) if args.cpu_seconds > 0 else None
    info = be.info()
    be.close()
    out = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 5),
        "ms_per_step_one_layer_graphs": round(ms_step_1, 5), "graph_layers": L, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "cfg2: Llama-3-8B decode layer as Q4_K matvecs at batch 1 (QKV 4096->6144, "
                               "O 4096->4096, gate/up 4096->14336 in one launch writing h = silu(g) * u, down "
                               "14336->4096 on h), device Q8_K quantization of each input included",
                   "layer_bytes": layer_bytes, "weight_copies": args.copies,
                   "weight_set_MB": round(args.copies * sum(r * (c // 256) * 144 for _, r, c in LAYER) / 1e6, 1),
                   "device": info["name"], "hbm_frac": round(value / HBM_PEAK_GBS, 4)},
        "roofline": roofline,
        "read_reference": read_reference,
        "mfma_reference": mfma_reference,
        "cpu_baseline": cpu,
        "kernels": kernels,
        "prefill": prefill,
        "other_configs": others,
        "attention": attention,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
