#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-matmul hot path (one GPU).

Workload: decode MoE expert block, one token per
step: int8 router [128 x 2816] + softmax top-8, then 8 int4 g64 experts
(gate/up [704 x 2816], GeGLU, down [2816 x 704]) weighted-summed. All 128
experts (430 MB) are resident in HBM; the token changes every step (64
distinct hidden states, rotated) so the selected experts change and mostly
miss the 256 MB last-level cache. Steps are replayed from a HIP graph that
holds 64 tokens (3 kernels each: router GEMV, phase 1 with the top-k
selection folded in, phase 2).

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
C4_CTX = 4096
C4_LAYERS = 8


def c4_bytes():
    """Algorithmic HBM bytes of one config-4 layer token (weights fp16 scale+bias,
    fp16 KV cache read once; activations and norm vectors are a few KB)."""
    d, qd, kvd = C4["d"], C4["nq"] * C4["hd"], C4["nkv"] * C4["hd"]
    q4 = lambda m, n: m * n // 2 + 2 * m * (n // 64) * 2
    parts = {
        "qkv": q4(qd + 2 * kvd, d),
        "attention_kv": 2 * C4_CTX * kvd * 2,
        "o_proj": q4(d, qd),
        "router": E * d + 2 * E * (d // 64) * 2,
        "routed": C4["k"] * 3 * q4(C4["f"], d),
        "shared": 2 * q4(C4["fs"], d) + q4(d, C4["fs"]),
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
    tiles, n_tiles, status = DeviceBuffer(mt * 16), DeviceBuffer(4), DeviceBuffer(4)
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


def bench_c4(ctx, stream, launch, batch_avg_us):
    from edgeexpert_amd import ops, synth
    from edgeexpert_amd.runtime import DeviceBuffer, Event, Graph
    t0 = time.time()
    w = synth.decode_layer(0, "c4", C4["d"], C4["nq"], C4["nkv"], C4["hd"], E, C4["f"], C4["fs"])
    kvd = C4["nkv"] * C4["hd"]
    kc = synth.f16_vector(0, "c4/kc", C4_CTX * kvd)
    vc = synth.f16_vector(0, "c4/vc", C4_CTX * kvd)
    spec = ops.DecodeLayerShapeSpec(d=C4["d"], num_q_heads=C4["nq"], num_kv_heads=C4["nkv"],
                                    head_dim=C4["hd"], expert_f=C4["f"], shared_f=C4["fs"], top_k=C4["k"],
                                    rotated_pairs=C4["rotated_pairs"], window=C4["window"], eps=C4["eps"],
                                    rope_theta=C4["theta"], attn_scale=C4["scale"])
    # distinct device copies (same values, different addresses): each token's
    # layer reads weights and KV that the previous layers evicted from L2/MALL
    layers, caches = [], []
    for _ in range(C4_LAYERS):
        layers.append(ops.DecodeLayer(ctx, ops.DecodeLayerWeightsSpec.upload(w), spec))
        caches.append((DeviceBuffer.from_array(kc), DeviceBuffer.from_array(vc)))
    ws_bytes = ops.decode_layer_workspace_bytes(spec, C4_CTX)
    ws = DeviceBuffer(ws_bytes)
    hid = DeviceBuffer.from_array(synth.f16_vector(0, "c4/hidden", C4["d"]))
    log(f"config 4: {C4_LAYERS} layer copies resident, set up in {time.time() - t0:.1f}s")
    pos = C4_CTX - 1

    def stack():
        for L in range(C4_LAYERS):
            kb, vb = caches[L]
            layers[L].encode(stream, hid, hid, kb, vb, pos, ws, ws_bytes)

    run = stack
    if launch == "graph":
        g = Graph(stream, stack)
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
    us = a.elapsed_ms(b) * 1e3 / (reps * C4_LAYERS)
    nb = c4_bytes()
    gbs = nb["total"] / (us * 1e-6) / 1e9
    floor_us = nb["total"] / (HBM_PEAK_GBS * 1e9) * 1e6
    # attention alone (split-K partial + combine over the 4096-key cache), back to back
    att = ops.Attention(ctx)
    q = DeviceBuffer.from_array(synth.f16_vector(0, "c4/q", C4["nq"] * C4["hd"]))
    out = DeviceBuffer(C4["nq"] * C4["hd"] * 2)
    aws = ops.Attention.workspace_bytes(C4["hd"], C4["nq"], C4_CTX)
    awsb = DeviceBuffer(aws)
    attn_us = batch_avg_us(lambda i: att.encode(stream, q, caches[i % C4_LAYERS][0], caches[i % C4_LAYERS][1],
                                                out, C4["hd"], C4["nq"], C4["nkv"], C4_CTX, awsb, aws,
                                                scale=1.0), 64)
    attn_gbs = nb["attention_kv"] / (attn_us * 1e-6) / 1e9
    log(f"decode layer C4 ({launch}): {us:.2f} us/token ({gbs:.0f} GB/s of {nb['total']} B; "
        f"8 TB/s floor {floor_us:.2f} us); attention alone {attn_us:.2f} us ({attn_gbs:.0f} GB/s)")
    return {"us_per_token": round(us, 3), "bytes_per_token": nb["total"], "gbs": round(gbs, 1),
            "hbm_floor_us": round(floor_us, 3), "frac_of_floor": round(floor_us / us, 4),
            "bytes": {k: v for k, v in nb.items() if k != "total"}, "layers_rotated": C4_LAYERS,
            "context": C4_CTX, "position": pos, "launch": launch,
            "attention_us": round(attn_us, 3), "attention_gbs": round(attn_gbs, 1)}


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
    ap.add_argument("--steps", type=int, default=4096)
    ap.add_argument("--warmup", type=int, default=256)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-c4", action="store_true", help="skip the config-4 decode-layer leg")
    ap.add_argument("--no-c3", action="store_true", help="skip the config-3 grouped-prefill leg")
    ap.add_argument("--no-bits", action="store_true", help="skip the 2/3-bit variant legs")
    ap.add_argument("--launch", choices=("graph", "stream"), default="graph",
                    help="replay the 64-token step from a HIP graph, or issue it from the host")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); the multi-GPU "
              "sharding of this path is a design note, not a measured configuration.",
              file=sys.stderr)
        sys.exit(2)

    from edgeexpert_amd import ops, synth
    from edgeexpert_amd._lib import LM_HEAD_WORKSPACE_BYTES, ROUTER_WORKSPACE_BYTES
    from edgeexpert_amd.runtime import DeviceBuffer, Event, Graph, Stream, device_info, synchronize

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

    reps_w = max(1, args.warmup // TOKENS)
    reps = max(1, args.steps // TOKENS)
    steps = reps * TOKENS
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
    us_per_token = gpu_ms * 1e3 / steps
    log(f"MoE decode ({args.launch}): {steps} tokens in {gpu_ms:.2f} ms (events), wall "
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

    # ------------------------------------------------ GEMV config 0 (extra) ----
    gemv = ops.DequantInt4GEMV(ctx)
    n_copies = 256
    W0, S0, B0 = synth.int4_matrix(0, "c0/w", 2816, 2816)
    x0 = DeviceBuffer.from_array(synth.f16_vector(0, "c0/x", 2816))
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
    cold_gbs = gemv_bytes / (cold_us * 1e-6) / 1e9
    warm_gbs = gemv_bytes / (warm_us * 1e-6) / 1e9
    log(f"GEMV C0 (back-to-back): cold {cold_us:.2f} us ({cold_gbs:.0f} GB/s), warm {warm_us:.2f} us "
        f"({warm_gbs:.0f} GB/s)")

    # ------------------------------------------------ GEMM config 2 (extra) ----
    qmm = ops.PrefillInt4QMM(ctx)
    from edgeexpert_amd._lib import DTYPE_BF16
    Mg, Ng, Kg = 512, 8192, 2816
    Wg, Sg, Bg = synth.int4_matrix(0, "c2/w", Ng, Kg)
    gW, gS, gB = (DeviceBuffer.from_array(a) for a in (Wg, Sg, Bg))
    gX = DeviceBuffer.from_array(synth.bf16_vector(0, "c2/x", Mg * Kg))
    gY = DeviceBuffer(Mg * Ng * 2)
    gemm_us = batch_avg_us(lambda i: qmm.encode(stream, gW, gS, gB, gX, gY, Mg, Ng, Kg, DTYPE_BF16), 20)
    gemm_flop = 2.0 * Mg * Ng * Kg
    gemm_tflops = gemm_flop / (gemm_us * 1e-6) / 1e12
    log(f"GEMM C2 (bf16, back-to-back): {gemm_us:.2f} us -> {gemm_tflops:.1f} TFLOP/s "
        f"({gemm_tflops / 2500.0 * 100:.1f}% of 2.5 PFLOP/s dense fp16/bf16)")

    # ------------------------------------ large GEMV: LM-head shape (extra) ----
    # 262144 x 2816 int4 (415 MB, larger than every cache): the steady-state
    # streaming rate of the decode GEMV, launched back to back.
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
    # the greedy decode head over the same rows: RMSNorm folded into the
    # activation staging, per-block argmax, one-block reduce (2 launches)
    head = ops.LMHeadGreedyInt4(ctx)
    tok_b, lm_ws = DeviceBuffer(4), DeviceBuffer(LM_HEAD_WORKSPACE_BYTES)
    norm_w = DeviceBuffer.from_array(synth.f16_vector(0, "lmhead/norm", 2816, std=0.5))
    greedy_us = batch_avg_us(lambda i: head.encode_greedy_decode(stream, x0, norm_w, big_l, sl_b, bl_b, tok_b,
                                                                 2816, Ml, lm_ws), 8, reps_=3)
    greedy_bytes = Ml * 1408 + 2 * Ml * 88 + 2 * 2816 * 2 + 4
    greedy_gbs = greedy_bytes / (greedy_us * 1e-6) / 1e9
    log(f"greedy LM head {Ml}x2816 (norm + rows + argmax, 2 launches): {greedy_us:.1f} us "
        f"({greedy_gbs:.0f} GB/s, {greedy_gbs / HBM_PEAK_GBS * 100:.1f}% of 8 TB/s)")
    del big_l, sl_b, bl_b, yl, lm_ws

    # ----------------------------------------- grouped MoE prefill, config 3 ----
    c3 = None if args.no_c3 else bench_c3(ctx, stream, batch_avg_us)

    # ------------------------------------------------ decode layer config 4 ----
    c4 = None if args.no_c4 else bench_c4(ctx, stream, args.launch, batch_avg_us)

    # ------------------------------------------------- 2/3-bit variants ----
    bits_legs = None if args.no_bits else bench_bits(ctx, stream, batch_avg_us, router, hbuf)
    if bits_legs is not None and not args.no_c3:
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
    cpu = None
    if not args.no_cpu:
        import oracle   # the checker, timed as the CPU restatement of the reference path
        hs = [H[t].view(np.float16).astype(np.float32) for t in range(TOKENS)]
        done, c0 = 0, time.perf_counter()
        while (time.perf_counter() - c0 < 10.0 and done < 200) or done < 3:
            h = hs[done % TOKENS]
            ridx, rw = oracle.topk_softmax(oracle.router_logits(Wr, Sr, Br, h), K)
            oracle.moe_routed(pool_bytes, stride, offs, h, ridx, rw, D, F)
            done += 1
        cpu_us = (time.perf_counter() - c0) / done * 1e6
        cpu = {"value": round(cpu_us, 1), "unit": "us/token", "cores": 1, "kind": "port",
               "sample": f"{done} tokens of config 1 (router + 8 experts), oracle/tfq_oracle.c, "
                         f"1 thread, host {os.cpu_count()} logical CPUs"}
        log(f"CPU baseline: {cpu_us:.0f} us/token over {done} tokens")

    out = {
        "metric": "MoE decode layer us/token (BASELINE config 1: int8 router + top-8 of 128 int4 g64 experts)",
        "value": round(us_per_token, 3),
        "unit": "us/token",
        "n_gpus": 1,
        "steps": steps,
        "warmup": reps_w * TOKENS,
        "ms_per_step": round(gpu_ms / steps, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4/int8 weights x fp16 activations, fp32 accumulate",
        "data": "synthetic (seeded SplitMix64, BASELINE distributions)",
        "config": {"workload": "config1_moe_decode", "experts": E, "top_k": K, "d": D, "f": F,
                   "tokens_rotated": TOKENS, "launch": args.launch,
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
        "gemv_c0": {"shape": [2816, 2816], "bytes": gemv_bytes, "cold_us": round(cold_us, 3),
                    "cold_gbs": round(cold_gbs, 1), "cold_frac": round(cold_gbs / HBM_PEAK_GBS, 4),
                    "warm_us": round(warm_us, 3), "warm_gbs": round(warm_gbs, 1),
                    "copies_rotated": n_copies},
        "gemm_c2": {"shape": [Mg, Ng, Kg], "dtype": "bf16 in/out, fp16 MFMA, fp32 acc",
                    "us": round(gemm_us, 3), "tflops": round(gemm_tflops, 1),
                    "frac_of_dense_peak": round(gemm_tflops / 2500.0, 4)},
        "gemv_lmhead": {"shape": [Ml, 2816], "bytes": lm_bytes, "us": round(lm_us, 2),
                        "gbs": round(lm_gbs, 1), "frac": round(lm_gbs / HBM_PEAK_GBS, 4)},
        "lm_head_greedy": {"shape": [Ml, 2816], "bytes": greedy_bytes, "us": round(greedy_us, 2),
                           "gbs": round(greedy_gbs, 1), "frac": round(greedy_gbs / HBM_PEAK_GBS, 4),
                           "kernels": "lm_head_greedy (norm staging + rows + block argmax), lm_head_reduce"},
        "grouped_prefill_c3": c3,
        "decode_layer_c4": c4,
        "bit_variants": bits_legs,
        "wall_s": round(wall, 4),
        "device": f"{name} {arch}",
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
