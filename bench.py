#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-matmul hot path (one GPU).

Workload: decode MoE expert block: int8 router
[128 x 2816] + softmax top-8, then 8 int4 g64 experts (gate/up [704 x 2816],
GeGLU, down [2816 x 704]) weighted-summed, one token at a time. All 128
experts (430 MB) are resident in HBM. A step is one batch of 64 decode
tokens (64 distinct hidden states, so the selected experts change and
mostly miss the 256 MB last-level cache), replayed from one HIP graph (3
kernels per token: router GEMV, phase 1 with the top-k selection folded in,
phase 2). --warmup W replays run untimed, then exactly --steps K replays
are timed; value = us per token = time / (64 K).

Also measured (extra fields): BASELINE config 0, the int4 g64 GEMV
[2816 x 2816], cold (rotating through 256 weight copies, 1.14 GB) and warm,
per-launch with HIP events; config 2, the bf16 prefill GEMM; the 2- and
3-bit expert / GEMV variants; config 4, the full Gemma 4 decoder layer for one token at position 4095 (context 4096),
chained through 8 resident copies of the layer so that every token reads
cold weights and KV cache, as consecutive layers of a model do.

Prints ONE JSON line on stdout. Data are synthetic (seeded SplitMix64, see
edgeexpert_amd/synth.py).
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
E, D, F, K = 128, 2816, 704, 8
TOKENS = 64


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def moe_bytes():
    """Algorithmic HBM bytes of one decode token (fp16 scale+bias)."""
    router = E * D + 2 * E * (D // 64) * 2                  # 360,448 + 22,528
    proj = F * D // 2 + 2 * F * (D // 64) * 2               # 991,232 + 123,904 per projection
    phase1 = K * 2 * proj                                   # gate + up of 8 experts
    phase2 = K * proj                                       # down of 8 experts
    acts = K * F * 2                                        # fp16 activations
    return {"router": router + 2 * D, "phase1": phase1 + 2 * D + acts,
            "phase2": phase2 + acts + 2 * D, "total": router + phase1 + phase2 + 2 * D * 2}


C4 = dict(d=2816, nq=16, nkv=8, hd=256, rotated_pairs=128, window=0, f=704, fs=2112, k=8,
          eps=1e-6, theta=10000.0, scale=1.0)
# Gemma 4's full-attention layer form at the config-4 sizes: head_dim 512,
# 2 kv heads, rope theta 1e6, partial rotary 0.25, no v projection
C4_FULL = dict(C4, nkv=2, hd=512, rotated_pairs=64, theta=1e6, full=True)
C4_CTX = 4096
C4_LAYERS = 8


def c4_bytes(shared_bits=4, shape=C4):
    """Algorithmic HBM bytes of one config-4 layer token (weights fp16 scale+bias,
    fp16 KV cache read once; activations and norm vectors are a few KB)."""
    d, qd, kvd = shape["d"], shape["nq"] * shape["hd"], shape["nkv"] * shape["hd"]
    q4 = lambda m, n: m * n // 2 + 2 * m * (n // 64) * 2
    qs = (lambda m, n: m * n + 2 * m * (n // 64) * 2) if shared_bits == 8 else q4
    parts = {
        "qkv": q4(qd + (1 if shape.get("full") else 2) * kvd, d),
        "attention_kv": 2 * C4_CTX * kvd * 2,
        "o_proj": q4(d, qd),
        "router": E * d + 2 * E * (d // 64) * 2,
        "routed": shape["k"] * 3 * q4(shape["f"], d),
        "shared": 2 * qs(shape["fs"], d) + qs(d, shape["fs"]),
    }
    parts["total"] = sum(parts.values())
    return parts


def bench_c3(ctx, stream, batch_avg_us, bits=4):
    """Config 3: 512 tokens x top-8 of 128 experts with Zipf(1.1) popularity;
    device grouping -> grouped gate/up + GeGLU -> grouped down -> token-major
    combine (4 launches), timed back to back over rotated hidden states.
    bits: code width of the experts (4, or the 2/3-bit variants)."""
    from edgeexpert_amd import ops, synth
    from edgeexpert_amd.runtime import DeviceBuffer
    T, k = 512, 8
    label = "c1/experts" if bits == 4 else f"c1b{bits}/experts"
    pool_bytes, offs, stride = synth.expert_pool(0, label, E, D, F, bits=bits)
    pool = ops.ExpertPool(DeviceBuffer.from_array(pool_bytes), stride, E, offs, weight_bits=bits)
    idx, w16 = synth.zipf_routing(0, "c3/route", T, E, k)
    active = np.unique(idx)
    n_hidden = 4
    hid = DeviceBuffer.from_array(np.stack([synth.f16_vector(0, f"c3/x{i}", T * D) for i in range(n_hidden)]))
    n, mt = T * k, ops.max_tiles(T, k, E)
    sorted_p = DeviceBuffer(n * 16)
    offsets, counts = DeviceBuffer(E * 4), DeviceBuffer(E * 4)
    tiles, n_tiles, status = DeviceBuffer(mt * 16), DeviceBuffer(ops.GROUP_STATE_BYTES), DeviceBuffer(4)
    act, partials, h2 = DeviceBuffer(n * F * 2), DeviceBuffer(n * D * 2), DeviceBuffer(T * D * 2)
    idx_b, w_b = DeviceBuffer.from_array(idx), DeviceBuffer.from_array(w16)
    grouping, grouped = ops.PrefillMoEGrouping(ctx), ops.PrefillGroupedRoutedMoE(ctx)

    def chunk(i):
        grouping.encode(stream, idx_b, w_b, T, k, E, sorted_p, offsets, counts, tiles, n_tiles, status)
        grouped.encode(stream, pool, sorted_p, tiles, n_tiles, mt, hid.ptr((i % n_hidden) * T * D * 2), D, D, F,
                       k, act, partials)
        grouped.encode_reduce_token_major(stream, partials, w_b, h2, T, k, D)

    us = batch_avg_us(chunk, 8, reps_=3)
    flop = 2.0 * n * 3 * D * F
    wbytes = len(active) * 3 * (F * D * bits // 8 + 2 * F * (D // 64) * 2)
    nbytes = wbytes + 2 * T * D * 2
    log(f"grouped MoE prefill C3 ({bits}-bit experts): {us:.1f} us per 512-token chunk ({flop / (us * 1e-6) / 1e12:.1f} TFLOP/s, "
        f"{nbytes / (us * 1e-6) / 1e9:.0f} GB/s of {len(active)} active experts' weights)")
    return {"us_per_chunk": round(us, 2), "tokens": T, "top_k": k, "active_experts": int(len(active)),
            "tflops": round(flop / (us * 1e-6) / 1e12, 1), "weight_bytes": wbytes,
            "gbs": round(nbytes / (us * 1e-6) / 1e9, 1), "us_per_token": round(us / T, 3),
            "kernels": "moe_group, moe_grouped_gate_up, moe_grouped_down, moe_combine"}


def bench_bits(ctx, stream, batch_avg_us, router, hbuf):
    """The 2- and 3-bit variants: config 1's decode token over 128 experts of
    2/3-bit rows (router + phase 1 with selection + phase 2, back to back
    over the 64 rotated tokens; per-kernel averages), and the 3-bit GEMV at
    the LM-head shape (262144 x 2816, 277 MB)."""
    from edgeexpert_amd import ops, synth
    from edgeexpert_amd._lib import ROUTER_WORKSPACE_BYTES
    from edgeexpert_amd.runtime import DeviceBuffer
    out = {}
    moe = ops.MoE(ctx)
    ws = DeviceBuffer(ROUTER_WORKSPACE_BYTES)
    ws.fill(0)
    y = DeviceBuffer(TOKENS * D * 2)
    idx, w16 = DeviceBuffer(TOKENS * K * 4), DeviceBuffer(TOKENS * K * 2)
    acts, logits = DeviceBuffer(TOKENS * K * F * 2), DeviceBuffer(TOKENS * E * 4)
    rW, rS, rB = router.weights, router.scales, router.biases
    for bits in (3, 2):
        pool_bytes, offs, stride = synth.expert_pool(0, f"c1b{bits}/experts", E, D, F, bits=bits)
        pool = ops.ExpertPool(DeviceBuffer.from_array(pool_bytes), stride, E, offs, weight_bits=bits)
        del pool_bytes
        token_us = batch_avg_us(lambda t: ops.moe_decode_token(
            ctx, stream, router, pool, hbuf.ptr(t * D * 2), None, y.ptr(t * D * 2), D, F, K, idx.ptr(t * K * 4),
            w16.ptr(t * K * 2), acts.ptr(t * K * F * 2), ws), TOKENS)
        for t in range(TOKENS):
            moe.encode_router_logits(stream, rW, rS, rB, hbuf.ptr(t * D * 2), None, logits.ptr(t * E * 4), E, D)
        p1 = batch_avg_us(lambda t: moe.encode_routed_phase1_with_selection(
            stream, pool, logits.ptr(t * E * 4), None, E, idx.ptr(t * K * 4), w16.ptr(t * K * 2),
            hbuf.ptr(t * D * 2), acts.ptr(t * K * F * 2), D, F, K), TOKENS)
        p2 = batch_avg_us(lambda t: moe.encode_routed_phase2(
            stream, pool, idx.ptr(t * K * 4), acts.ptr(t * K * F * 2), w16.ptr(t * K * 2), None,
            y.ptr(t * D * 2), D, F, K), TOKENS)
        proj = F * D * bits // 8 + 2 * F * (D // 64) * 2
        p1_bytes = K * 2 * proj + 2 * D + K * F * 2
        p1_gbs = p1_bytes / (p1 * 1e-6) / 1e9
        log(f"{bits}-bit experts: decode token {token_us:.2f} us (back-to-back), phase1 {p1:.2f} us "
            f"({p1_gbs:.0f} GB/s), phase2 {p2:.2f} us")
        out[f"moe_decode_b{bits}"] = {"us_per_token": round(token_us, 3), "phase1_us": round(p1, 3),
                                      "phase2_us": round(p2, 3), "phase1_bytes": p1_bytes,
                                      "phase1_gbs": round(p1_gbs, 1),
                                      "phase1_frac": round(p1_gbs / HBM_PEAK_GBS, 4)}
        del pool
    # 3-bit GEMV streaming rate at the LM-head shape
    Ml, n = 262144, 2816
    rb = n * 3 // 8
    Wl, Sl, Bl = synth.affine_matrix(0, "lmhead/w3", 4096, n, 3)
    big, sb, bb = DeviceBuffer(Ml * rb), DeviceBuffer(Ml * 88), DeviceBuffer(Ml * 88)
    for r0 in range(0, Ml, 4096):
        big.upload(Wl, r0 * rb)
        sb.upload(Sl, r0 * 88)
        bb.upload(Bl, r0 * 88)
    x = DeviceBuffer.from_array(synth.f16_vector(0, "c0/x", n))
    yl = DeviceBuffer(Ml * 2)
    gemv = ops.DequantInt4GEMV(ctx)
    us = batch_avg_us(lambda i: gemv.encode(stream, big, sb, bb, x, yl, Ml, n, bits=3), 8, reps_=3)
    nbytes = Ml * rb + 2 * Ml * 88 + n * 2 + Ml * 2
    gbs = nbytes / (us * 1e-6) / 1e9
    log(f"3-bit GEMV {Ml}x{n}: {us:.1f} us ({gbs:.0f} GB/s, {gbs / HBM_PEAK_GBS * 100:.1f}% of 8 TB/s)")
    out["gemv_b3_lmhead"] = {"shape": [Ml, n], "bytes": nbytes, "us": round(us, 2), "gbs": round(gbs, 1),
                             "frac": round(gbs / HBM_PEAK_GBS, 4)}
    del big, sb, bb, yl
    # 3-bit prefill GEMM at config 2's shape (bf16 activations)
    from edgeexpert_amd._lib import DTYPE_BF16
    Mg, Ng, Kg = 512, 8192, 2816
    Wg, Sg, Bg = synth.affine_matrix(0, "c2/w3", Ng, Kg, 3)
    gW, gS, gB = (DeviceBuffer.from_array(a) for a in (Wg, Sg, Bg))
    gX = DeviceBuffer.from_array(synth.bf16_vector(0, "c2/x", Mg * Kg))
    gY = DeviceBuffer(Mg * Ng * 2)
    qmm = ops.PrefillInt4QMM(ctx)
    g_us = batch_avg_us(lambda i: qmm.encode(stream, gW, gS, gB, gX, gY, Mg, Ng, Kg, DTYPE_BF16, bits=3), 20)
    tf = 2.0 * Mg * Ng * Kg / (g_us * 1e-6) / 1e12
    log(f"3-bit GEMM C2 (bf16): {g_us:.2f} us -> {tf:.1f} TFLOP/s")
    out["gemm_b3_c2"] = {"shape": [Mg, Ng, Kg], "us": round(g_us, 3), "tflops": round(tf, 1)}
    return out


def bench_c4(ctx, stream, launch, batch_avg_us, shared_bits=4, shape=C4):
    """Config 4's decoder layer; shared_bits 8 runs the shared expert at
    8 bits (the reference's default width) instead of 4; shape C4_FULL runs
    the full-attention layer form."""
    from edgeexpert_amd import ops, synth
    from edgeexpert_amd.runtime import DeviceBuffer, Event, Graph
    t0 = time.time()
    C = shape
    tag = "c4full" if C.get("full") else "c4"
    w = synth.decode_layer(0, tag, C["d"], C["nq"], C["nkv"], C["hd"], E, C["f"], C["fs"],
                           shared_bits=shared_bits, v_proj=not C.get("full", False))
    kvd = C["nkv"] * C["hd"]
    kc = synth.f16_vector(0, tag + "/kc", C4_CTX * kvd)
    vc = synth.f16_vector(0, tag + "/vc", C4_CTX * kvd)
    spec = ops.DecodeLayerShapeSpec(d=C["d"], num_q_heads=C["nq"], num_kv_heads=C["nkv"],
                                    head_dim=C["hd"], expert_f=C["f"], shared_f=C["fs"], top_k=C["k"],
                                    rotated_pairs=C["rotated_pairs"], window=C["window"], eps=C["eps"],
                                    rope_theta=C["theta"], attn_scale=C["scale"])
    # distinct device copies (same values, different addresses): each token's
    # layer reads weights and KV that the previous layers evicted from L2/MALL
    layers, caches = [], []
    for _ in range(C4_LAYERS):
        layers.append(ops.DecodeLayer(ctx, ops.DecodeLayerWeightsSpec.upload(w), spec))
        caches.append((DeviceBuffer.from_array(kc), DeviceBuffer.from_array(vc)))
    ws_bytes = ops.decode_layer_workspace_bytes(spec, C4_CTX)
    ws = DeviceBuffer(ws_bytes)
    hid = DeviceBuffer.from_array(synth.f16_vector(0, tag + "/hidden", C["d"]))
    log(f"config 4 ({tag}): {C4_LAYERS} layer copies resident, set up in {time.time() - t0:.1f}s")
    pos = C4_CTX - 1

    def stack():
        for L in range(C4_LAYERS):
            kb, vb = caches[L]
            layers[L].encode(stream, hid, hid, kb, vb, pos, ws, ws_bytes)

    # the same 8 layers as one tfq_decode_layers call: each layer's tail is
    # formed inside the next layer's QKV launch
    chain = ops.DecodeLayers(ctx, [L.keep for L in layers], [spec] * C4_LAYERS)
    cws_bytes = chain.workspace_bytes(C4_CTX)
    cws = DeviceBuffer(cws_bytes)
    hiddens = DeviceBuffer(C4_LAYERS * C["d"] * 2)

    def chained():
        chain.encode(stream, hid, hiddens, [c[0] for c in caches], [c[1] for c in caches], pos, cws, cws_bytes)

    def time_per_layer(fn):
        run = fn
        if launch == "graph":
            g = Graph(stream, fn)
            run = lambda: g.launch(stream)
        for _ in range(4):
            run()
        stream.sync()
        reps = 32
        a, b = Event(), Event()
        a.record(stream)
        for _ in range(reps):
            run()
        b.record(stream)
        stream.sync()
        return a.elapsed_ms(b) * 1e3 / (reps * C4_LAYERS)

    us_calls = time_per_layer(stack)
    us = time_per_layer(chained)
    nb = c4_bytes(shared_bits, C)
    gbs = nb["total"] / (us * 1e-6) / 1e9
    floor_us = nb["total"] / (HBM_PEAK_GBS * 1e9) * 1e6
    # attention alone (split-K partial + combine over the 4096-key cache), back to back
    att = ops.Attention(ctx)
    q = DeviceBuffer.from_array(synth.f16_vector(0, tag + "/q", C["nq"] * C["hd"]))
    out = DeviceBuffer(C["nq"] * C["hd"] * 2)
    aws = ops.Attention.workspace_bytes(C["hd"], C["nq"], C4_CTX)
    awsb = DeviceBuffer(aws)
    attn_us = batch_avg_us(lambda i: att.encode(stream, q, caches[i % C4_LAYERS][0], caches[i % C4_LAYERS][1],
                                                out, C["hd"], C["nq"], C["nkv"], C4_CTX, awsb, aws,
                                                scale=1.0), 64)
    attn_gbs = nb["attention_kv"] / (attn_us * 1e-6) / 1e9
    log(f"decode layer {tag} ({launch}, {shared_bits}-bit shared expert): {us:.2f} us/token per layer of a "
        f"{C4_LAYERS}-layer chain ({gbs:.0f} GB/s of {nb['total']} B; 8 TB/s floor {floor_us:.2f} us), "
        f"{us_calls:.2f} us as one call per layer; attention alone {attn_us:.2f} us ({attn_gbs:.0f} GB/s)")
    return {"us_per_token": round(us, 3), "us_per_token_layer_calls": round(us_calls, 3),
            "measure": f"per layer of {C4_LAYERS} resident layer copies chained in one tfq_decode_layers call "
                       f"(each tail formed in the next layer's QKV launch, the last one by the tail kernel); "
                       f"us_per_token_layer_calls: one tfq_decode_layer call per layer",
            "shared_expert_bits": shared_bits, "bytes_per_token": nb["total"],
            "attention_form": ("full: head_dim 512, 16 q / 2 kv heads, V from the k projection, rope theta 1e6, "
                               "64 rotated pairs") if C.get("full") else "sliding: head_dim 256, 16 q / 8 kv heads",
            "gbs": round(gbs, 1),
            "hbm_floor_us": round(floor_us, 3), "frac_of_floor": round(floor_us / us, 4),
            "bytes": {k: v for k, v in nb.items() if k != "total"}, "layers_rotated": C4_LAYERS,
            "context": C4_CTX, "position": pos, "launch": launch,
            "attention_us": round(attn_us, 3), "attention_gbs": round(attn_gbs, 1)}


def host_cpu():
    """(lscpu model name, logical CPUs visible, threads this job may use)."""
    model = "unknown"
    fields = {}
    try:
        for line in subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout.splitlines():
            key, _, val = line.partition(":")
            fields.setdefault(key.strip(), val.strip())
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    fields.setdefault("cpuinfo model name", line.split(":", 1)[1].strip())
                    break
    except OSError:
        pass
    # a virtualised host may print only "AMD EPYC": keep the BIOS name and
    # the family/model numbers (family 26 = Zen 5) beside it
    names = [fields.get(k) for k in ("Model name", "cpuinfo model name", "BIOS Model name")]
    names = [n for i, n in enumerate(names) if n and n not in names[:i]]
    if names:
        model = " / ".join(names)
    if fields.get("CPU family") or fields.get("Model"):
        model += f" (family {fields.get('CPU family', '?')}, model {fields.get('Model', '?')})"
    visible = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS", "")
    usable = min(visible, int(omp)) if omp.isdigit() and int(omp) > 0 else visible
    return model, visible, usable


def cpu_baseline(Wr, Sr, Br, pool_bytes, stride, offs, H, W0, S0, B0):
    """The reference's CPU path (oracle/cpu_baseline.c: the oracle's row
    arithmetic, -O3 -march=native built on this host, rows split over
    threads) timed on the host cores at 1 thread and at every usable core:
    config 1 (one decode token: router + 8 experts) and config 0 (the int4
    GEMV). Medians of >= 20 runs after warmup."""
    import oracle   # the checker, timed as the CPU restatement of the reference path
    from edgeexpert_amd import synth
    model, visible, usable = host_cpu()
    oracle.baseline_lib(rebuild=True)       # -march=native for this host
    hs = [H[t].view(np.float16).astype(np.float32) for t in range(TOKENS)]
    x0 = synth.f16_to_f32(synth.f16_vector(0, "c0/x", 2816))

    def median_us(fn, n, warm=2):
        for i in range(warm):
            fn(i)
        ts = []
        for i in range(n):
            t0 = time.perf_counter()
            fn(i)
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts)) * 1e6

    # config 2: the GEMM reference (MPPPrefillInt4QMMTests.cpuReference) over
    # a bounded sample of token rows (16 per thread), scaled to the 512 rows
    W2, S2, B2 = synth.int4_matrix(0, "c2/w", 8192, 2816)
    X2 = synth.bf16_to_f32(synth.bf16_vector(0, "c2/x", 512 * 2816)).reshape(512, 2816)
    # config 3: the grouped reference (cpuSyntheticRoutePartials) over a
    # bounded sample of the 4096 sorted pairs (8 per thread; every pair costs
    # one full expert FFN), scaled to 4096, plus the token-major combine
    T3, k3 = 512, 8
    idx3, w3 = synth.zipf_routing(0, "c3/route", T3, E, k3)
    pairs = np.array([(t, int(idx3[t, r]), r, 4) for t in range(T3) for r in range(k3)], oracle.PAIR_DTYPE)
    sorted3 = oracle.group_pairs(pairs, T3, k3, E)["sorted"]
    hid3 = synth.f16_vector(0, "c3/x0", T3 * D)
    o3 = oracle.ExpertOffsets(*[int(offs[n]) for n in synth.OFFSET_ORDER])
    parts3 = np.zeros(T3 * k3 * D, np.uint16)
    # config 4: the decoder layer (oracle tfo_decode_layer) at position 4095
    w4 = synth.decode_layer(0, "c4", C4["d"], C4["nq"], C4["nkv"], C4["hd"], E, C4["f"], C4["fs"])
    kvd = C4["nkv"] * C4["hd"]
    kc4, vc4 = synth.f16_vector(0, "c4/kc", C4_CTX * kvd), synth.f16_vector(0, "c4/vc", C4_CTX * kvd)
    h4 = synth.f16_vector(0, "c4/hidden", C4["d"])

    res = {}
    for threads in sorted({1, usable}):
        tok = median_us(lambda i: oracle.baseline_moe_decode_token(Wr, Sr, Br, pool_bytes, stride, offs,
                                                                   hs[i % TOKENS], D, F, K, threads), 20)
        gemv = median_us(lambda i: oracle.baseline_gemv_int4(W0, S0, B0, x0, threads), 40)
        rows2 = min(512, 16 * threads)
        t0 = time.perf_counter()
        oracle.gemm_int4(W2, S2, B2, X2, rows=(0, rows2), threads=threads)
        gemm = (time.perf_counter() - t0) * 1e6 * 512 / rows2
        n3 = min(len(sorted3), 8 * threads)
        t0 = time.perf_counter()
        oracle.grouped_route_partials(sorted3[:n3], hid3, D, pool_bytes, stride, o3, k3, D, F, T3, threads=threads)
        grouped = (time.perf_counter() - t0) * 1e6 * len(sorted3) / n3
        t0 = time.perf_counter()
        oracle.reduce_token_major(parts3, w3, T3, k3, D)
        grouped += (time.perf_counter() - t0) * 1e6
        layer = median_us(lambda i: oracle.decode_layer(w4, C4, h4, kc4, vc4, C4_CTX - 1, threads=threads), 20,
                          warm=1)
        res[threads] = dict(config1_us_per_token=round(tok, 1), config0_gemv_us=round(gemv, 1),
                            config2_gemm_us=round(gemm, 1), config2_rows_timed=rows2,
                            config3_us_per_chunk=round(grouped, 1), config3_pairs_timed=n3,
                            config4_us_per_token=round(layer, 1))
        log(f"CPU baseline, {threads} thread(s): config 1 {tok:.0f} us/token, config 0 GEMV {gemv:.0f} us, "
            f"config 2 GEMM {gemm / 1e6:.2f} s ({rows2} of 512 rows timed), config 3 {grouped / 1e6:.2f} s per "
            f"512-token chunk ({n3} of {len(sorted3)} pairs timed), config 4 layer {layer / 1e3:.1f} ms/token")
    return {"value": res[usable]["config1_us_per_token"], "unit": "us/token", "cores": usable, "kind": "port",
            "sample": f"config 1: median of 20 decode tokens (router + 8 experts; 64 rotated hidden states), "
                      f"rows split over {usable} threads; config 0: median of 40 GEMVs; config 2: "
                      f"16 token rows per thread of the 512 timed once, scaled to 512; config 3: 8 sorted "
                      f"pairs per thread of the 4096 timed once (each pair one whole expert FFN), scaled to "
                      f"4096, plus the whole token-major combine; config 4: median of 20 layers at position "
                      f"4095 (GEMV rows and attention heads split over the threads); oracle/cpu_baseline.c + "
                      f"tfq_oracle.c, gcc -O3 -march=native -ffp-contract=off -fopenmp",
            "cpu_model": model, "logical_cpus_visible": visible, "threads_all_cores": usable,
            "one_thread": res[1], "all_cores": res[usable]}


def trace_summary(csv_path, out=sys.stdout, b2b_gap_us=None):
    """Per (kernel, grid, workgroup) dispatch statistics of a rocprofv3
    --kernel-trace CSV: the same kernel launched at several shapes (the
    int4 GEMV at config 0 and at the LM-head shape, say) is reported once
    per shape. b2b_gap_us: keep only dispatches that start within that many
    microseconds of the previous dispatch's end (launched back to back, as
    in bench.py's per-kernel batches)."""
    import csv
    rows = []
    with open(csv_path, newline="") as fh:
        for row in csv.DictReader(fh):
            rows.append((int(row["Start_Timestamp"]), int(row["End_Timestamp"]), row["Kernel_Name"],
                         tuple(int(row[f"Grid_Size_{a}"]) for a in "XYZ"),
                         tuple(int(row[f"Workgroup_Size_{a}"]) for a in "XYZ")))
    rows.sort()
    groups = {}
    prev_end = None
    for start, end, name, grid, wg in rows:
        keep = b2b_gap_us is None or (prev_end is not None and start - prev_end <= b2b_gap_us * 1e3)
        prev_end = end if prev_end is None else max(prev_end, end)
        if keep:
            groups.setdefault((name, grid, wg), []).append((end - start) / 1e3)
    total = sum(sum(v) for v in groups.values()) or 1.0
    out.write(f"{'kernel':44s} {'grid (threads)':>20s} {'wg':>5s} {'calls':>6s} {'avg us':>9s} "
              f"{'median':>9s} {'min us':>8s} {'max us':>9s} {'% time':>7s}\n")
    for (name, grid, wg), v in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
        a = np.array(v)
        g = "x".join(str(d) for d in grid if d > 1) or "1"
        out.write(f"{name[:44]:44s} {g:>20s} {wg[0]:>5d} {len(a):>6d} {a.mean():>9.2f} {np.median(a):>9.2f} "
                  f"{a.min():>8.2f} {a.max():>9.2f} {100 * a.sum() / total:>7.2f}\n")


def pmc_summary(csv_path, out=sys.stdout, simds=1024, xcds=8):
    """Per (kernel, grid) averages of the counters in a rocprofv3 --pmc
    counter_collection CSV, per dispatch, with the matrix-core busy fraction
    of rocprofv3's MfmaUtil: SQ_VALU_MFMA_BUSY_CYCLES / (cycles x SIMDs),
    cycles = GRBM_GUI_ACTIVE / XCDs (MI355X: 8 XCDs, whose GUI_ACTIVE counts
    the profiler sums; 1024 SIMDs). A busy cycle is 1024 fp16 FLOP of one
    SIMD, so the fraction equals achieved / dense-peak FLOP/s, which
    SQ_INSTS_VALU_MFMA_MOPS_F16 x 512 (the dispatch's MFMA FLOP) cross-checks."""
    import csv
    acc = {}
    with open(csv_path, newline="") as fh:
        for row in csv.DictReader(fh):
            key = (row["Kernel_Name"], int(row["Grid_Size"]), int(row["Workgroup_Size"]))
            d = acc.setdefault(key, {})
            d.setdefault(row["Counter_Name"], {})[row["Dispatch_Id"]] = float(row["Counter_Value"])
            d.setdefault("_dur", {})[row["Dispatch_Id"]] = (int(row["End_Timestamp"]) -
                                                            int(row["Start_Timestamp"])) / 1e3
    for (name, grid, wg), d in sorted(acc.items(), key=lambda kv: -sum(kv[1]["_dur"].values())):
        n = len(d["_dur"])
        mean = {c: sum(v.values()) / len(v) for c, v in d.items()}
        line = f"{name[:40]:40s} grid {grid:>8d} wg {wg:>4d} n {n:>5d} avg {mean['_dur']:8.2f} us"
        for c in sorted(k for k in mean if not k.startswith("_")):
            line += f" {c}={mean[c]:.4g}"
        gui = mean.get("GRBM_GUI_ACTIVE")
        if gui and "SQ_VALU_MFMA_BUSY_CYCLES" in mean:
            line += f" | MFMA busy {100 * mean['SQ_VALU_MFMA_BUSY_CYCLES'] * xcds / (gui * simds):.1f}%"
        if "SQ_INSTS_VALU_MFMA_MOPS_F16" in mean and mean["_dur"] > 0:
            tf = mean["SQ_INSTS_VALU_MFMA_MOPS_F16"] * 512 / (mean["_dur"] * 1e-6) / 1e12
            line += f" | MFMA {tf:.0f} TFLOP/s"
        out.write(line + "\n")


# Algorithmic bytes per launch of the kernels the traffic summary compares:
# weights + scales/biases + activations read + outputs written, per bench.py
# unit of work. By kernel name, or by (name, blocks) for kernels launched at
# several shapes.
TRAFFIC_ALG = {
    "tfq_moe_phase1_routed_s32_p3": 17859072,
    "tfq_moe_phase2_p3": 8 * 1115136 + 8 * 704 * 2 + 8 * 2 + 8 * 4 + 2816 * 2,
    "tfq_router_logits_s64_p3": 128 * 2816 + 4 * 128 * 44 + 2816 * 2 + 128 * 4,
    "tfq_attn_partial_h256_g2": 33554432,
    "tfq_lm_head_greedy_s32_p3": 262144 * 1408 + 2 * 262144 * 88 + 2 * 2816 * 2,
}
TRAFFIC_ALG_GRID = {
    ("tfq_q4_gemv_s32_p3", 352): 4471808,                                                   # config 0
    ("tfq_gemm_q4_bf16", 256): 11534336 + 1441792 + 2883584 + 8388608,                      # config 2
    ("tfq_q4_gemv_s32_p3", 1792): 262144 * 1408 + 2 * 262144 * 88 + 2816 * 2 + 262144 * 2,  # LM-head shape
}


def traffic_summary(fetch_csv, write_csv, out=sys.stdout):
    """HBM bytes per launch from two rocprofv3 --pmc runs of this script
    (FETCH_SIZE, then WRITE_SIZE), by (kernel, blocks). The counters are
    scaled to bytes by what they read for the calibration kernels this
    script launches once: tfq_read_ceiling over 64 MiB (its largest-grid
    dispatch) and tfq_convert_bf16_f16 (32 MiB in, 32 MiB out). Ends with the
    `traffic <kernel family> <bytes>` lines read_traffic() takes."""
    import csv
    import re

    def load(path, counter):
        acc, n, sizes = {}, {}, {}
        for r in csv.DictReader(open(path, newline="")):
            if r["Counter_Name"] != counter:
                continue
            name = r["Kernel_Name"].split("(")[0].strip()
            k = (name if name in ("tfq_read_ceiling", "tfq_convert_bf16_f16") or name.startswith("__amd")
                 else f"{name}@{int(r['Grid_Size']) // int(r['Workgroup_Size'])}")
            v = float(r["Counter_Value"])
            acc[k] = acc.get(k, 0.0) + v
            n[k] = n.get(k, 0) + 1
            sizes.setdefault(k, []).append(v)
        return acc, n, sizes
    f, nf, fs = load(fetch_csv, "FETCH_SIZE")
    w, nw, ws = load(write_csv, "WRITE_SIZE")
    cal = max((int(r["Grid_Size"]), float(r["Counter_Value"])) for r in csv.DictReader(open(fetch_csv, newline=""))
              if r["Counter_Name"] == "FETCH_SIZE" and r["Kernel_Name"].startswith("tfq_read_ceiling"))
    rc = cal[1] / (64 * 1024)
    cv_f = max(fs["tfq_convert_bf16_f16"]) / (32 * 1024)
    cv_w = max(ws["tfq_convert_bf16_f16"]) / (32 * 1024)
    fetch_scale = (rc + cv_f) / 2
    rows = []
    for k in f:
        if k.startswith("__amd") or k in ("tfq_read_ceiling", "tfq_convert_bf16_f16"):
            continue
        fk = f[k] / nf[k]
        wk = w.get(k, 0.0) / max(nw.get(k, 1), 1)
        rows.append((fk * 1024 / fetch_scale + wk * 1024 / cv_w, k, nf[k], fk, wk))
    rows.sort(reverse=True)
    out.write("Calibration (kernels of known size launched by bench.py in the same run):\n"
              f"    tfq_read_ceiling, 64 MiB read (its largest-grid dispatch): FETCH_SIZE = {rc:.4f} KiB per KiB read\n"
              f"    tfq_convert_bf16_f16, 32 MiB in / 32 out: FETCH_SIZE = {cv_f:.4f} KiB per KiB read, "
              f"WRITE_SIZE = {cv_w:.4f} KiB per KiB written\n"
              f"    traffic (bytes) = FETCH_SIZE[KiB] * 1024 / {fetch_scale:.4f} + WRITE_SIZE[KiB] * 1024 / {cv_w:.4f}\n\n")
    out.write(f"{'kernel@blocks':39s} {'dispatches':>10s} {'FETCH KiB':>11s} {'WRITE KiB':>10s} {'traffic B':>12s}  "
              f"{'algorithmic B':>13s}  ratio\n")
    for traffic, k, n, fk, wk in rows:
        name, blocks = k.split("@")
        alg = TRAFFIC_ALG.get(name) or TRAFFIC_ALG_GRID.get((name, int(blocks)))
        ratio = f"{traffic / alg:6.2f}" if alg else ""
        out.write(f"{k:39s} {n:10d} {fk:11.1f} {wk:10.1f} {traffic:12.0f}  {alg if alg else '':>13}  {ratio}\n")
    out.write("\nMachine-readable lines (bench.py reads `traffic <kernel family> <bytes>`):\n")
    seen = set()
    c0 = [t for t, k, *_ in rows if k == "tfq_q4_gemv_s32_p3@352"]
    if c0:
        out.write(f"traffic tfq_q4_gemv_c0 {c0[0]:.0f}\n")
    for traffic, k, *_ in rows:
        fam = re.sub(r"(_s\d+_p\d+|_p\d+|_h\d+_g\d+|_h\d+)$", "", k.split("@")[0])
        if fam not in seen:
            seen.add(fam)
            out.write(f"traffic {fam} {traffic:.0f}\n")


def layer_summary(trace_csv, out=sys.stdout):
    """Per-kernel durations of the config-4 decoder layers in a rocprofv3
    --kernel-trace CSV of this script: the window from the first norm-staged
    QKV GEMV (1024 blocks: the _rms form, or _norm) to the last layer tail, grouped by (kernel, grid,
    queue), median and minimum over the layers."""
    import csv
    import statistics
    rows = sorted((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"],
                   int(r["Grid_Size_X"]) // int(r["Workgroup_Size_X"]), int(r["Grid_Size_Y"]), int(r["Queue_Id"]))
                  for r in csv.DictReader(open(trace_csv, newline="")))
    t0 = min(s for s, e, n, gx, gy, q in rows
             if n.startswith(("tfq_q4_gemv_rms_s32_p3", "tfq_q4_gemv_norm_s32_p3")) and gx == 1024)
    t1 = max(e for s, e, n, gx, gy, q in rows if n.startswith("tfq_layer_tail"))
    win = [r for r in rows if t0 <= r[0] and r[1] <= t1]
    layers = sum(1 for r in win if r[2].startswith("tfq_layer_tail"))
    groups = {}
    for s, e, n, gx, gy, q in win:
        groups.setdefault((n, gx, gy, q), []).append((e - s) / 1e3)
    out.write(f"layers in the window: {layers}\n\n"
              f"{'kernel':44s} {'grid':>9s} {'queue':>5s} {'median us':>10s} {'min us':>8s}\n")
    for (n, gx, gy, q), v in groups.items():
        if len(v) >= layers // 2:
            out.write(f"{n[:44]:44s} {gx:5d}x{gy:<3d} {q:5d} {statistics.median(v):10.2f} {min(v):8.2f}\n")
    # one chained layer of the first leg (the 4-bit shared expert): the
    # dispatches from a tail-forming QKV GEMV to the next, median over the
    # middle layers of its chains
    tails = [i for i, r in enumerate(rows) if r[2].startswith("tfq_q4_gemv_tail_")]
    seqs = []
    for a, b in zip(tails, tails[1:]):
        seq = rows[a:b]
        if seqs and [r[2] for r in seq] != [r[2] for r in seqs[0]]:
            break
        seqs.append(seq)
    if seqs:
        out.write(f"\none chained layer (tfq_decode_layers, {len(seqs)} layers of the first leg; median per position):\n"
                  f"{'kernel':44s} {'grid':>9s} {'median us':>10s} {'gap before us':>14s}\n")
        total = 0.0
        for j, r in enumerate(seqs[0]):
            dur = statistics.median((sq[j][1] - sq[j][0]) / 1e3 for sq in seqs)
            gap = statistics.median((sq[j][0] - sq[j - 1][1]) / 1e3 for sq in seqs) if j else 0.0
            total += dur
            out.write(f"{r[2][:44]:44s} {r[3]:5d}x{r[4]:<3d} {dur:10.2f} {gap:14.2f}\n")
        out.write(f"sum of the kernel medians: {total:.1f} us\n")


def bench_gemm_policy(ctx, stream, batch_avg_us):
    """The prefill GEMM's kernel choice by token count (config 2's weights,
    N 8192 x K 2816, bf16): the library's choice at token counts on both
    sides of its crossover (80 tokens at this N), and both kernels forced at
    the two counts next to it."""
    from edgeexpert_amd import ops, synth
    from edgeexpert_amd._lib import DTYPE_BF16, GEMM_PATH_SKINNY32, GEMM_PATH_TILE
    from edgeexpert_amd.runtime import DeviceBuffer
    N, Kd = 8192, 2816
    W, S, B = synth.int4_matrix(0, "c2/w", N, Kd)
    copies = 8                 # rotate weight copies: each launch reads weights the last ones evicted
    bufs = [tuple(DeviceBuffer.from_array(a) for a in (W, S, B)) for _ in range(copies)]
    X = DeviceBuffer.from_array(synth.bf16_vector(0, "c2/x", 512 * Kd))
    Y = DeviceBuffer(512 * N * 2)
    q = ops.PrefillInt4QMM(ctx)
    wbytes = N * Kd // 2 + 2 * N * (Kd // 64) * 2
    out = {"shape": [None, N, Kd], "crossover_tokens": 80, "auto": {}, "forced": {}}

    def run(m, path):
        return batch_avg_us(lambda i: q.encode(stream, *bufs[i % copies], X, Y, m, N, Kd, DTYPE_BF16, path=path),
                            32, reps_=3)
    for m in (1, 16, 64, 80, 96, 128, 512):
        us = run(m, None)
        out["auto"][str(m)] = {"us": round(us, 2), "tflops": round(2.0 * m * N * Kd / (us * 1e-6) / 1e12, 1),
                               "weight_gbs": round(wbytes / (us * 1e-6) / 1e9, 1),
                               "kernel": "gemv" if m == 1 else "skinny" if m <= 80 else "tile"}
    for m in (64, 96):
        out["forced"][str(m)] = {"skinny32_us": round(run(m, GEMM_PATH_SKINNY32), 2),
                                 "tile_us": round(run(m, GEMM_PATH_TILE), 2)}
    # few tokens: the decode GEMV once per token against the weight stream
    # (the reference's repeated GEMV below 32 tokens), N 2048 and 8192
    from edgeexpert_amd._lib import GEMM_PATH_GEMV, GEMM_PATH_SKINNY
    out["gemv_vs_skinny"] = {}
    for n in (2048, 8192):
        Wn, Sn, Bn = synth.int4_matrix(0, f"c2/w{n}", n, Kd) if n != N else (W, S, B)
        bn = [tuple(DeviceBuffer.from_array(a) for a in (Wn, Sn, Bn)) for _ in range(copies)]
        for m in (1, 2, 3, 4):
            row = {}
            for name, path in (("gemv", GEMM_PATH_GEMV), ("skinny", GEMM_PATH_SKINNY), ("auto", None)):
                row[name + "_us"] = round(batch_avg_us(
                    lambda i: q.encode(stream, *bn[i % copies], X, Y, m, n, Kd, DTYPE_BF16, path=path), 32, reps_=3), 2)
            out["gemv_vs_skinny"][f"n{n}_m{m}"] = row
        del bn
    log("GEMM by token count (N 8192, K 2816, bf16): " +
        ", ".join(f"M={m} {v['us']:.1f} us ({v['kernel']})" for m, v in out["auto"].items()) +
        "; forced " + ", ".join(f"M={m}: skinny {v['skinny32_us']:.1f} / tile {v['tile_us']:.1f} us"
                                for m, v in out["forced"].items()) +
        "; GEMV vs skinny " + ", ".join(f"{key}: {v['gemv_us']:.2f} / {v['skinny_us']:.2f} (auto {v['auto_us']:.2f})"
                                         for key, v in out["gemv_vs_skinny"].items()))
    return out


TRAFFIC_FILE = "profiles/hbm_traffic_moe_decode_c1.txt"


def read_traffic():
    """HBM bytes per launch measured by two rocprofv3 --pmc runs of this
    script (FETCH_SIZE, WRITE_SIZE), scaled by the calibration kernels; read
    from the committed summary. Lines: `traffic <kernel> <bytes>`."""
    path = os.path.join(ROOT, TRAFFIC_FILE)
    if not os.path.exists(path):
        return None
    out = {}
    for line in open(path):
        f = line.split()
        if len(f) == 3 and f[0] == "traffic":
            out[f[1]] = int(float(f[2]))
    return out or None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64, help="timed 64-token graph replays")
    ap.add_argument("--warmup", type=int, default=8, help="untimed replays before them")
    ap.add_argument("--legs", default="all",
                    help="comma list of the extra legs to run besides the headline: c0, c2, lmhead, c3, c4, "
                         "c4full, policy, bits, cpu (default all)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--launch", choices=("graph", "stream"), default="graph",
                    help="replay the 64-token step from a HIP graph, or issue it from the host")
    ap.add_argument("--trace-summary", metavar="CSV",
                    help="print per (kernel, grid) statistics of a rocprofv3 kernel-trace CSV and exit")
    ap.add_argument("--b2b-gap-us", type=float, default=None,
                    help="with --trace-summary: only dispatches starting within this gap of the previous end")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="print HBM bytes per launch from FETCH_SIZE / WRITE_SIZE counter CSVs and exit")
    ap.add_argument("--layer-summary", metavar="CSV",
                    help="print the config-4 layer's per-kernel durations from a kernel-trace CSV and exit")
    ap.add_argument("--pmc-summary", metavar="CSV",
                    help="print per (kernel, grid) averages of a rocprofv3 --pmc counter CSV and exit")
    args = ap.parse_args()
    if args.pmc_summary:
        pmc_summary(args.pmc_summary)
        return
    if args.traffic_summary:
        traffic_summary(*args.traffic_summary)
        return
    if args.layer_summary:
        layer_summary(args.layer_summary)
        return
    if args.trace_summary:
        trace_summary(args.trace_summary, b2b_gap_us=args.b2b_gap_us)
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); the multi-GPU "
              "sharding of this path is a design note, not a measured configuration.",
              file=sys.stderr)
        sys.exit(2)

    from edgeexpert_amd import ops, synth
    from edgeexpert_amd._lib import LM_HEAD_WORKSPACE_BYTES, ROUTER_WORKSPACE_BYTES
    from edgeexpert_amd.runtime import DeviceBuffer, Event, Graph, Stream, device_info, synchronize

    legs = set(args.legs.split(","))

    def want(leg):
        return ("all" in legs or leg in legs) and not (leg == "cpu" and args.no_cpu)

    name, arch = device_info()
    log(f"device {name} {arch}")
    ctx = ops.Context()
    stream = Stream()

    # ------------------------------------------------------------ inputs ----
    t0 = time.time()
    pool_bytes, offs, stride = synth.expert_pool(0, "c1/experts", E, D, F)
    Wr, Sr, Br = synth.int8_matrix(0, "c1/router", E, D)
    H = np.stack([synth.f16_vector(0, f"c1/h{t}", D) for t in range(TOKENS)])
    log(f"inputs generated in {time.time() - t0:.1f}s (pool {pool_bytes.nbytes / 1e6:.0f} MB)")
    pool = ops.ExpertPool(DeviceBuffer.from_array(pool_bytes), stride, E, offs)
    rW, rS, rB = (DeviceBuffer.from_array(a) for a in (Wr, Sr, Br))
    hbuf = DeviceBuffer.from_array(H)
    ybuf = DeviceBuffer(TOKENS * D * 2)
    ws = DeviceBuffer(ROUTER_WORKSPACE_BYTES)
    ws.fill(0)

    router = ops.Router(rW, rS, rB, E)
    idx_all = DeviceBuffer(TOKENS * K * 4)
    w16_all = DeviceBuffer(TOKENS * K * 2)
    acts_all = DeviceBuffer(TOKENS * K * F * 2)

    def token(t):
        ops.moe_decode_token(ctx, stream, router, pool, hbuf.ptr(t * D * 2), None,
                             ybuf.ptr(t * D * 2), D, F, K, idx_all.ptr(t * K * 4),
                             w16_all.ptr(t * K * 2), acts_all.ptr(t * K * F * 2), ws)

    def all_tokens():
        for t in range(TOKENS):
            token(t)

    reps_w = max(0, args.warmup)
    reps = max(1, args.steps)
    steps = reps
    if args.launch == "graph":
        graph = Graph(stream, all_tokens)
        run = lambda: graph.launch(stream)
    else:
        run = all_tokens
    for _ in range(reps_w):
        run()
    stream.sync()

    # -------------------------------------------------------- timed region ----
    e0, e1 = Event(), Event()
    synchronize()
    wall0 = time.perf_counter()
    e0.record(stream)
    for _ in range(reps):
        run()
    e1.record(stream)
    stream.sync()
    synchronize()
    wall = time.perf_counter() - wall0
    gpu_ms = e0.elapsed_ms(e1)
    us_per_token = gpu_ms * 1e3 / (steps * TOKENS)
    log(f"MoE decode ({args.launch}): {steps} steps x {TOKENS} tokens in {gpu_ms:.2f} ms (events), wall "
        f"{wall * 1e3:.2f} ms -> {us_per_token:.2f} us/token")

    # ------------------------------ per-kernel durations (HIP events) ----
    # Each kernel of the block, launched back to back for the 64 tokens (whose
    # routing is already in idx_all / w16_all) between two events on `stream`;
    # the average includes the launch gap between consecutive kernels.
    nb = moe_bytes()
    moe = ops.MoE(ctx)

    # A one-block read of 256 MiB (a few ms of GPU time, one launch) queued ahead
    # of every timed batch: the host enqueues the whole batch while the GPU is
    # still busy with it, so the events see kernels back to back with no
    # host launch gaps (also under a profiler, where launches are slower).
    pad_bytes = 256 << 20
    pad_buf = DeviceBuffer(pad_bytes)
    pad_buf.fill(0)
    pad_sink = DeviceBuffer(256)

    def pad():
        ops.read_ceiling(ctx, stream, pad_buf, pad_bytes, pad_sink, 1)

    def batch_avg_us(launch_one, count, reps_=5):
        best = []
        for _ in range(reps_):
            a, b = Event(), Event()
            pad()
            a.record(stream)
            for t in range(count):
                launch_one(t)
            b.record(stream)
            stream.sync()
            best.append(a.elapsed_ms(b) * 1e3 / count)
        return float(np.median(best))

    logits_all = DeviceBuffer(TOKENS * E * 4)
    k_us = {
        "router_logits": batch_avg_us(lambda t: moe.encode_router_logits(
            stream, rW, rS, rB, hbuf.ptr(t * D * 2), None, logits_all.ptr(t * E * 4), E, D), TOKENS),
        "phase1": batch_avg_us(lambda t: moe.encode_routed_phase1_with_selection(
            stream, pool, logits_all.ptr(t * E * 4), None, E, idx_all.ptr(t * K * 4), w16_all.ptr(t * K * 2),
            hbuf.ptr(t * D * 2), acts_all.ptr(t * K * F * 2), D, F, K), TOKENS),
        "phase2": batch_avg_us(lambda t: moe.encode_routed_phase2(
            stream, pool, idx_all.ptr(t * K * 4), acts_all.ptr(t * K * F * 2), w16_all.ptr(t * K * 2),
            None, ybuf.ptr(t * D * 2), D, F, K), TOKENS),
    }
    p1_us = k_us["phase1"]
    p1_gbs = nb["phase1"] / (p1_us * 1e-6) / 1e9
    log("kernel avg (back-to-back): " + ", ".join(f"{k} {v:.2f} us" for k, v in k_us.items())
        + f"; phase1 {p1_gbs:.0f} GB/s ({nb['phase1']} B/launch)")

    W0, S0, B0 = synth.int4_matrix(0, "c0/w", 2816, 2816)
    x0 = DeviceBuffer.from_array(synth.f16_vector(0, "c0/x", 2816))
    gemv = ops.DequantInt4GEMV(ctx)

    def leg_c0():
        """Config 0: the int4 GEMV [2816 x 2816], cold (256 rotating weight
        copies, 1.1 GB) and warm, back to back."""
        n_copies = 256
        y0 = DeviceBuffer(2816 * 2)
        wsz, ssz = W0.nbytes, S0.nbytes
        big = DeviceBuffer(n_copies * (wsz + 2 * ssz))
        for i in range(n_copies):
            base = i * (wsz + 2 * ssz)
            big.upload(W0, base)
            big.upload(S0, base + wsz)
            big.upload(B0, base + wsz + ssz)
        gemv_bytes = wsz + 2 * ssz + 2 * 2816 * 2

        def gemv_launch(copy):
            base = copy * (wsz + 2 * ssz)
            gemv.encode(stream, big, big, big, x0, y0, 2816, 2816, weights_offset=base,
                        scales_offset=base + wsz, biases_offset=base + wsz + ssz)

        cold_us = batch_avg_us(gemv_launch, n_copies)
        warm_us = batch_avg_us(lambda i: gemv_launch(0), n_copies)
        # the same 256 cold launches replayed from one HIP graph (the kernel
        # boundary of a graph instead of a host launch each)
        g0 = Graph(stream, lambda: [gemv_launch(i) for i in range(n_copies)])
        g0.launch(stream)
        stream.sync()
        cold_graph_us = batch_avg_us(lambda i: g0.launch(stream), 4) / n_copies
        cold_gbs = gemv_bytes / (cold_us * 1e-6) / 1e9
        warm_gbs = gemv_bytes / (warm_us * 1e-6) / 1e9
        graph_gbs = gemv_bytes / (cold_graph_us * 1e-6) / 1e9
        # the read ceiling of the same cold bytes: one pure 128-bit read pass
        # over each copy's weights + scales + biases, the same rotation
        sink0 = DeviceBuffer(4 * 8192)
        rbytes = (wsz + 2 * ssz) // 16 * 16
        ceil_us = batch_avg_us(lambda i: ops.read_ceiling(ctx, stream, big, rbytes, sink0, 8192,
                                                          src_offset=(i % n_copies) * (wsz + 2 * ssz)), n_copies)
        # the launch floor: the same kernel reading one 16-byte chunk (one
        # block), from the rotated copies (cold) and from one address (warm),
        # back to back and replayed from a graph
        def one_block(i, cold=True):
            ops.read_ceiling(ctx, stream, big, 16, sink0, 8192,
                             src_offset=(i % n_copies) * (wsz + 2 * ssz) if cold else 0)

        floor_us = batch_avg_us(one_block, n_copies)
        floor_warm_us = batch_avg_us(lambda i: one_block(i, False), n_copies)
        g1 = Graph(stream, lambda: [one_block(i) for i in range(n_copies)])
        g2 = Graph(stream, lambda: [one_block(i, False) for i in range(n_copies)])
        for g in (g1, g2):
            g.launch(stream)
        stream.sync()
        floor_graph_us = batch_avg_us(lambda i: g1.launch(stream), 4) / n_copies
        floor_graph_warm_us = batch_avg_us(lambda i: g2.launch(stream), 4) / n_copies
        # the int8 GEMV (tfq_gemv_q8g64) at the same shape: 128 rotating
        # copies of its 8.4 MB (cold) and one copy (warm)
        W8, S8, B8 = synth.int8_matrix(0, "c0/w8", 2816, 2816)
        w8sz, s8sz = W8.nbytes, S8.nbytes
        n8 = 128
        big8 = DeviceBuffer(n8 * (w8sz + 2 * s8sz))
        for i in range(n8):
            base = i * (w8sz + 2 * s8sz)
            big8.upload(W8, base)
            big8.upload(S8, base + w8sz)
            big8.upload(B8, base + w8sz + s8sz)
        gemv8 = ops.DequantInt8GEMV(ctx)

        def gemv8_launch(copy):
            base = copy * (w8sz + 2 * s8sz)
            gemv8.encode(stream, big8, big8, big8, x0, y0, 2816, 2816, weights_offset=base,
                         scales_offset=base + w8sz, biases_offset=base + w8sz + s8sz)

        gemv8_bytes = w8sz + 2 * s8sz + 2 * 2816 * 2
        cold8_us = batch_avg_us(gemv8_launch, n8)
        warm8_us = batch_avg_us(lambda i: gemv8_launch(0), n8)
        del big8
        log(f"int8 GEMV 2816x2816 (back-to-back): cold {cold8_us:.2f} us "
            f"({gemv8_bytes / (cold8_us * 1e-6) / 1e9:.0f} GB/s), warm {warm8_us:.2f} us")
        log(f"GEMV C0 (back-to-back): cold {cold_us:.2f} us ({cold_gbs:.0f} GB/s), warm {warm_us:.2f} us "
            f"({warm_gbs:.0f} GB/s); cold from a graph {cold_graph_us:.2f} us ({graph_gbs:.0f} GB/s); "
            f"cold read of the same bytes {ceil_us:.2f} us (GEMV at {ceil_us / cold_us:.2f} of it); "
            f"one-block launch reading 16 B: cold {floor_us:.2f} / warm {floor_warm_us:.2f} us back to back, "
            f"{floor_graph_us:.2f} / {floor_graph_warm_us:.2f} us from a graph")
        return {"shape": [2816, 2816], "bytes": gemv_bytes, "cold_us": round(cold_us, 3),
                "cold_gbs": round(cold_gbs, 1), "cold_frac": round(cold_gbs / HBM_PEAK_GBS, 4),
                "cold_read_ceiling_us": round(ceil_us, 3),
                "cold_frac_of_read_ceiling": round(ceil_us / cold_us, 4),
                "launch_floor_us": {"cold": round(floor_us, 3), "warm": round(floor_warm_us, 3),
                                    "cold_graph": round(floor_graph_us, 3), "warm_graph": round(floor_graph_warm_us, 3),
                                    "measure": "tfq_read_ceiling over 16 bytes (one block): the rotated copies' "
                                               "first chunk (cold) or one address (warm)"},
                "warm_us": round(warm_us, 3), "warm_gbs": round(warm_gbs, 1),
                "cold_graph_us": round(cold_graph_us, 3), "cold_graph_frac": round(graph_gbs / HBM_PEAK_GBS, 4),
                "copies_rotated": n_copies,
                "int8_gemv": {"shape": [2816, 2816], "bytes": gemv8_bytes, "cold_us": round(cold8_us, 3),
                              "cold_gbs": round(gemv8_bytes / (cold8_us * 1e-6) / 1e9, 1),
                              "warm_us": round(warm8_us, 3), "copies_rotated": n8}}

    def leg_c2():
        """Config 2: the bf16 prefill GEMM 512 x 8192 x 2816."""
        from edgeexpert_amd._lib import DTYPE_BF16
        qmm = ops.PrefillInt4QMM(ctx)
        Mg, Ng, Kg = 512, 8192, 2816
        Wg, Sg, Bg = synth.int4_matrix(0, "c2/w", Ng, Kg)
        gW, gS, gB = (DeviceBuffer.from_array(a) for a in (Wg, Sg, Bg))
        gX = DeviceBuffer.from_array(synth.bf16_vector(0, "c2/x", Mg * Kg))
        gY = DeviceBuffer(Mg * Ng * 2)
        gemm_us = batch_avg_us(lambda i: qmm.encode(stream, gW, gS, gB, gX, gY, Mg, Ng, Kg, DTYPE_BF16), 20)
        gemm_tflops = 2.0 * Mg * Ng * Kg / (gemm_us * 1e-6) / 1e12
        log(f"GEMM C2 (bf16, back-to-back): {gemm_us:.2f} us -> {gemm_tflops:.1f} TFLOP/s "
            f"({gemm_tflops / 2500.0 * 100:.1f}% of 2.5 PFLOP/s dense fp16/bf16)")
        return {"shape": [Mg, Ng, Kg], "dtype": "bf16 in/out, fp16 MFMA, fp32 acc", "us": round(gemm_us, 3),
                "tflops": round(gemm_tflops, 1), "frac_of_dense_peak": round(gemm_tflops / 2500.0, 4)}

    def leg_lmhead():
        """262144 x 2816 int4 (415 MB, larger than every cache): the steady-state
        streaming rate of the decode GEMV, and the greedy decode head over the
        same rows (RMSNorm folded into the staging, per-block argmax, one-block
        reduce: 2 launches), back to back."""
        Ml = 262144
        Wl, Sl, Bl = synth.int4_matrix(0, "lmhead/w", 4096, 2816)        # 4096-row tile, replicated
        big_l = DeviceBuffer(Ml * 1408)
        sl_b, bl_b = DeviceBuffer(Ml * 88), DeviceBuffer(Ml * 88)
        for r0 in range(0, Ml, 4096):
            big_l.upload(Wl, r0 * 1408)
            sl_b.upload(Sl, r0 * 88)
            bl_b.upload(Bl, r0 * 88)
        yl = DeviceBuffer(Ml * 2)
        lm_bytes = Ml * 1408 + 2 * Ml * 88 + 2816 * 2 + Ml * 2
        lm_us = batch_avg_us(lambda i: gemv.encode(stream, big_l, sl_b, bl_b, x0, yl, Ml, 2816), 8, reps_=3)
        lm_gbs = lm_bytes / (lm_us * 1e-6) / 1e9
        log(f"GEMV LM-head shape {Ml}x2816: {lm_us:.1f} us ({lm_gbs:.0f} GB/s, "
            f"{lm_gbs / HBM_PEAK_GBS * 100:.1f}% of 8 TB/s)")
        head = ops.LMHeadGreedyInt4(ctx)
        tok_b, lm_ws = DeviceBuffer(4), DeviceBuffer(LM_HEAD_WORKSPACE_BYTES)
        norm_w = DeviceBuffer.from_array(synth.f16_vector(0, "lmhead/norm", 2816, std=0.5))
        greedy_us = batch_avg_us(lambda i: head.encode_greedy_decode(stream, x0, norm_w, big_l, sl_b, bl_b, tok_b,
                                                                     2816, Ml, lm_ws), 8, reps_=3)
        greedy_bytes = Ml * 1408 + 2 * Ml * 88 + 2 * 2816 * 2 + 4
        greedy_gbs = greedy_bytes / (greedy_us * 1e-6) / 1e9
        log(f"greedy LM head {Ml}x2816 (norm + rows + argmax, 2 launches): {greedy_us:.1f} us "
            f"({greedy_gbs:.0f} GB/s, {greedy_gbs / HBM_PEAK_GBS * 100:.1f}% of 8 TB/s)")
        return ({"shape": [Ml, 2816], "bytes": lm_bytes, "us": round(lm_us, 2), "gbs": round(lm_gbs, 1),
                 "frac": round(lm_gbs / HBM_PEAK_GBS, 4)},
                {"shape": [Ml, 2816], "bytes": greedy_bytes, "us": round(greedy_us, 2), "gbs": round(greedy_gbs, 1),
                 "frac": round(greedy_gbs / HBM_PEAK_GBS, 4),
                 "kernels": "lm_head_greedy (norm staging + rows + block argmax), lm_head_reduce"})

    gemv_c0 = leg_c0() if want("c0") else None
    gemm_c2 = leg_c2() if want("c2") else None
    gemv_lmhead, lm_head_greedy = leg_lmhead() if want("lmhead") else (None, None)
    c3 = bench_c3(ctx, stream, batch_avg_us) if want("c3") else None
    c4 = bench_c4(ctx, stream, args.launch, batch_avg_us) if want("c4") else None
    c4_s8 = bench_c4(ctx, stream, args.launch, batch_avg_us, shared_bits=8) if want("c4") else None
    c4_full = bench_c4(ctx, stream, args.launch, batch_avg_us, shape=C4_FULL) if want("c4full") else None
    gemm_policy = bench_gemm_policy(ctx, stream, batch_avg_us) if want("policy") else None
    bits_legs = bench_bits(ctx, stream, batch_avg_us, router, hbuf) if want("bits") else None
    if bits_legs is not None and want("c3"):
        bits_legs["grouped_prefill_c3_b3"] = bench_c3(ctx, stream, batch_avg_us, bits=3)

    # -------------------------------------- HBM counter calibration kernels ----
    # One plain read (64 MiB) and one plain copy (32 MiB in, 32 MiB out) of
    # known size, launched once so that a rocprofv3 --pmc run of this command
    # can scale FETCH_SIZE / WRITE_SIZE of the other kernels to bytes.
    cal_bytes = 64 << 20
    cal = DeviceBuffer(cal_bytes)
    cal.fill(0)
    sink = DeviceBuffer(4 * 8192)
    ops.read_ceiling(ctx, stream, cal, cal_bytes, sink, 8192)
    ops.convert_bf16_to_f16(ctx, stream, cal, cal.ptr(cal_bytes // 2), cal_bytes // 4)
    stream.sync()
    traffic = read_traffic()

    # ------------------------------------------------------ CPU baseline ----
    cpu = cpu_baseline(Wr, Sr, Br, pool_bytes, stride, offs, H, W0, S0, B0) if want("cpu") else None
    out = {
        "metric": "MoE decode layer us/token (BASELINE config 1: int8 router + top-8 of 128 int4 g64 experts)",
        "value": round(us_per_token, 3),
        "unit": "us/token",
        "n_gpus": 1,
        "steps": steps,
        "warmup": reps_w,
        "ms_per_step": round(gpu_ms / steps, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4/int8 weights x fp16 activations, fp32 accumulate",
        "data": "synthetic (seeded SplitMix64, BASELINE distributions)",
        "config": {"workload": "config1_moe_decode", "experts": E, "top_k": K, "d": D, "f": F,
                   "tokens_per_step": TOKENS, "tokens_rotated": TOKENS, "launch": args.launch,
                   "kernels_per_token": "router_logits, moe_phase1_routed (top-k selection + gate/up), "
                                        "moe_phase2"},
        "roofline": {"kernel": "tfq_moe_phase1_routed (top-8 selection + gate/up of 8 experts)",
                     "bound": "hbm",
                     "achieved": round(p1_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(p1_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic.get("tfq_moe_phase1_routed") if traffic else None,
                     "traffic_source": TRAFFIC_FILE if traffic else None,
                     "algorithmic_bytes": nb["phase1"], "avg_launch_us": round(p1_us, 3),
                     "kernel_avg_us": {k: round(v, 3) for k, v in k_us.items()}},
        "cpu_baseline": cpu,
        "token_bytes": nb["total"],
        "token_gbs": round(nb["total"] / (us_per_token * 1e-6) / 1e9, 1),
        "gemv_c0": gemv_c0,
        "gemm_c2": gemm_c2,
        "gemv_lmhead": gemv_lmhead,
        "lm_head_greedy": lm_head_greedy,
        "grouped_prefill_c3": c3,
        "decode_layer_c4": c4,
        "decode_layer_c4_int8_shared": c4_s8,
        "decode_layer_c4_full_attention": c4_full,
        "gemm_by_token_count": gemm_policy,
        "bit_variants": bits_legs,
        "wall_s": round(wall, 4),
        "device": f"{name} {arch}",
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
