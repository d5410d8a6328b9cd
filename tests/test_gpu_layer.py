"""GPU parity of the config-4 decode layer: split-K GQA decode attention and
the whole Gemma 4 decoder layer (tfq_decode_layer) against the CPU oracle,
through libtfq's C ABI.

Bars: routing indices bit-exact; every stage's output (the intermediate
buffers are read back from the documented workspace layout) within
rel_error 1e-3 (north star) of the oracle fed with the GPU's own stored
inputs of that stage. The whole chain (ten fp16-stored stages) against the
pure oracle: rel_error below 1e-3, or, where the oracle's own chain moves
further than that when its arithmetic is perturbed at fp32 size before every
fp16 rounding point (layer_chain.chain_floor: the spread of two exact chains
that differ only in summation order), no further from the oracle than the
oracle is from itself; and always below the reference's bar for chained fp16
reductions (Tolerance.fp16ChainedReduction = 1e-2,
V/Tolerance/Tolerances.swift:12-15)."""
import numpy as np
import pytest

import oracle
from edgeexpert_amd import ops, synth
from edgeexpert_amd._lib import TfqError
from edgeexpert_amd.runtime import DeviceBuffer, Graph
from helpers import f16_round, from_f16_bits
from layer_chain import chain_floor

pytestmark = pytest.mark.gpu
TOL = oracle.Tolerance.north_star


def _dev(a):
    return DeviceBuffer.from_array(np.ascontiguousarray(a))


# ---------------------------------------------------------------- attention ----

def _run_attention(ctx, stream, q16, k16, v16, hd, nq, nkv, seq, window, scale):
    ws_bytes = ops.Attention.workspace_bytes(hd, nq, seq, window)
    ws = DeviceBuffer(ws_bytes)
    out = _dev(np.full(nq * hd, 0x7E00, np.uint16))
    ops.Attention(ctx).encode(stream, _dev(q16), _dev(k16), _dev(v16), out, hd, nq, nkv, seq, ws, ws_bytes,
                              window=window, scale=scale)
    stream.sync()
    return from_f16_bits(out.download(np.uint16, nq * hd))


@pytest.mark.parametrize("hd,nq,nkv,seq,window,scale", [
    (256, 16, 8, 4096, 0, None),        # config 4 attention at full context
    (256, 16, 8, 8192, 0, None),        # 128 chunks: the combine's general (m, l) loops and chunk loop
    (128, 8, 2, 5000, 0, None),         # 79 chunks, ragged last one
    (256, 16, 8, 4096, 0, 1.0),         # Gemma 4 scale 1.0
    (256, 16, 8, 1000, 512, None),      # sliding window (encodeSWA)
    (256, 16, 4, 300, 0, None),         # GQA group 4
    (256, 4, 4, 1, 0, None),            # one key
    (128, 8, 2, 77, 0, None),           # ragged last chunk
    (128, 8, 8, 64, 0, 1.0),            # exactly one chunk
    (128, 4, 1, 129, 100, None),        # window cuts a chunk boundary
    (512, 16, 2, 4096, 0, 1.0),         # full-attention layers: head_dim 512, group 8
    (512, 16, 2, 77, 0, None),          # ... ragged last chunk
    (512, 8, 2, 130, 0, None),          # head_dim 512, group 4
    (512, 2, 2, 64, 0, None),           # head_dim 512, group 1
])
def test_attention_matches_reference(ctx, stream, hd, nq, nkv, seq, window, scale):
    tag = f"attn-h{hd}-q{nq}-kv{nkv}-T{seq}-w{window}"
    q16 = synth.f16_vector(0, tag + "/q", nq * hd)
    k16 = synth.f16_vector(0, tag + "/k", seq * nkv * hd)
    v16 = synth.f16_vector(0, tag + "/v", seq * nkv * hd)
    got = _run_attention(ctx, stream, q16, k16, v16, hd, nq, nkv, seq, window, scale)
    ref = oracle.attention(from_f16_bits(q16), from_f16_bits(k16), from_f16_bits(v16), hd, nq, nkv, seq,
                           window, scale)
    rel = oracle.rel_error(got, ref)
    assert rel < TOL, f"{tag}: rel={rel}"


def test_attention_is_deterministic(ctx, stream):
    hd, nq, nkv, seq = 256, 16, 8, 2048
    q16 = synth.f16_vector(1, "det/q", nq * hd)
    k16 = synth.f16_vector(1, "det/k", seq * nkv * hd)
    v16 = synth.f16_vector(1, "det/v", seq * nkv * hd)
    a = _run_attention(ctx, stream, q16, k16, v16, hd, nq, nkv, seq, 0, None)
    b = _run_attention(ctx, stream, q16, k16, v16, hd, nq, nkv, seq, 0, None)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_attention_rejects_bad_contract(ctx, stream):
    att = ops.Attention(ctx)
    ws = DeviceBuffer(1 << 20)
    buf = DeviceBuffer(1 << 20)
    bad = [dict(hd=64, nq=4, nkv=2, seq=8), dict(hd=128, nq=6, nkv=2, seq=8),
           dict(hd=128, nq=4, nkv=3, seq=8), dict(hd=128, nq=4, nkv=2, seq=0)]
    for b in bad:
        with pytest.raises(TfqError):
            att.encode(stream, buf, buf, buf, buf, b["hd"], b["nq"], b["nkv"], b["seq"], ws, 1 << 20)
    with pytest.raises(TfqError):       # workspace too small
        att.encode(stream, buf, buf, buf, buf, 256, 16, 8, 4096, ws, 1024)


# -------------------------------------------------------------------- layer ----

def _layout(shape, seq):
    """Mirror of DecodeLayer::layout (edgeexpert_amd/csrc/host/ops.hpp): 256-byte
    aligned segments o, h1, h2, hmid, inv (the vectors a chained layer leaves
    for the next, first), q, attn, parts, logits, idx, w, acts, sact, kv (the
    staged raw k/v rows)."""
    up = lambda v: (v + 255) // 256 * 256
    qd = shape["nq"] * shape["hd"]
    sizes = [("o", shape["d"] * 2), ("h1", shape["d"] * 2), ("h2", shape["d"] * 2), ("hmid", shape["d"] * 2),
             ("inv", 4), ("q", qd * 2), ("attn", qd * 2),
             ("parts", ops.Attention.workspace_bytes(shape["hd"], shape["nq"], seq, shape["window"])),
             ("logits", 4096), ("idx", shape["k"] * 4), ("w", shape["k"] * 2),
             ("acts", shape["k"] * shape["f"] * 2), ("sact", shape["fs"] * 2),
             ("kv", 2 * shape["nkv"] * shape["hd"] * 2)]
    off, L = 0, {}
    for n, sz in sizes:
        L[n] = off
        off += up(sz)
    L["total"] = off
    return L


def _spec(shape):
    return ops.DecodeLayerShapeSpec(d=shape["d"], num_q_heads=shape["nq"], num_kv_heads=shape["nkv"],
                                    head_dim=shape["hd"], expert_f=shape["f"], shared_f=shape["fs"],
                                    top_k=shape["k"], rotated_pairs=shape["rotated_pairs"],
                                    window=shape["window"], eps=shape["eps"], rope_theta=shape["theta"],
                                    attn_scale=shape["scale"])


def _layer_case(ctx, stream, shape, E, pos, cap, seed, label, in_place=False, expert_bits=4, shared_bits=4):
    w = synth.decode_layer(seed, label, shape["d"], shape["nq"], shape["nkv"], shape["hd"], E, shape["f"],
                           shape["fs"], expert_bits=expert_bits, shared_bits=shared_bits,
                           v_proj=not shape.get("full", False))
    kvd = shape["nkv"] * shape["hd"]
    kc = synth.f16_vector(seed, label + "/kc", cap * kvd)
    vc = synth.f16_vector(seed, label + "/vc", cap * kvd)
    hidden = synth.f16_vector(seed, label + "/hidden", shape["d"])
    print(f"[layer] {label} pos={pos} E={E} shape={shape}", flush=True)
    spec = _spec(shape)
    L = _layout(shape, pos + 1)
    ws_bytes = ops.decode_layer_workspace_bytes(spec, pos + 1)
    assert ws_bytes == L["total"]
    ws = DeviceBuffer(ws_bytes)
    ws.fill(0)
    kb, vb, hb = _dev(kc), _dev(vc), _dev(hidden)
    ob = hb if in_place else _dev(np.full(shape["d"], 0x7E00, np.uint16))
    layer = ops.DecodeLayer(ctx, ops.DecodeLayerWeightsSpec.upload(w), spec)
    layer.encode(stream, hb, ob, kb, vb, pos, ws, ws_bytes)
    stream.sync()
    kc_ref, vc_ref = kc.copy(), vc.copy()
    out_ref, idx_ref, w_ref, tr = oracle.decode_layer(w, shape, hidden, kc_ref, vc_ref, pos, trace=True)
    got = {
        "out": from_f16_bits(ob.download(np.uint16, shape["d"])),
        "idx": ws.download(np.uint32, shape["k"], offset=L["idx"]),
        "w": from_f16_bits(ws.download(np.uint16, shape["k"], offset=L["w"])),
        "attn": from_f16_bits(ws.download(np.uint16, shape["nq"] * shape["hd"], offset=L["attn"])),
        "o": from_f16_bits(ws.download(np.uint16, shape["d"], offset=L["o"])),
        "h1": from_f16_bits(ws.download(np.uint16, shape["d"], offset=L["h1"])),
        "h2": from_f16_bits(ws.download(np.uint16, shape["d"], offset=L["h2"])),
        "kslot": from_f16_bits(kb.download(np.uint16, kvd, offset=pos * kvd * 2)),
        "vslot": from_f16_bits(vb.download(np.uint16, kvd, offset=pos * kvd * 2)),
        "kcache": kb.download(np.uint16, cap * kvd),
        "vcache": vb.download(np.uint16, cap * kvd),
        "q_raw": from_f16_bits(ws.download(np.uint16, shape["nq"] * shape["hd"], offset=L["q"])),
        "pos": pos,
    }
    ref = {"out": from_f16_bits(out_ref), "idx": idx_ref, "w": w_ref,
           "attn": from_f16_bits(tr["attn"]), "o": from_f16_bits(tr["o"]), "h1": from_f16_bits(tr["h1"]),
           "h2": from_f16_bits(tr["h2"]),
           "kslot": from_f16_bits(kc_ref[pos * kvd:(pos + 1) * kvd]),
           "vslot": from_f16_bits(vc_ref[pos * kvd:(pos + 1) * kvd])}
    # slots other than `pos` are untouched
    assert np.array_equal(np.delete(got["kcache"].reshape(cap, kvd), pos, 0),
                          np.delete(kc.reshape(cap, kvd), pos, 0))
    got["kc_in"], got["vc_in"] = kc, vc
    return got, ref, w, hidden


def _n16(x, w16, eps=1e-6):
    return f16_round(oracle.rmsnorm(x, None if w16 is None else from_f16_bits(w16), eps))


def _check_layer(got, ref, w, shape, hidden, label):
    """Each stage against the oracle fed with the GPU's own stored inputs
    then the whole chain against the pure oracle."""
    assert list(got["idx"]) == list(ref["idx"]), f"{label}: routing differs"
    d, eps = shape["d"], shape["eps"]
    h_in = from_f16_bits(hidden)
    # the projection (with its fused input norm) and the k/v epilogue, fed by `hidden`
    for key in ("kslot", "vslot"):
        rel = oracle.rel_error(got[key], ref[key])
        assert rel < TOL, f"{label}: {key} rel={rel}"
    stage = {}
    # attention: the GPU's raw q through the oracle epilogue, the GPU's caches
    hd, nq, nkv, pos = shape["hd"], shape["nq"], shape["nkv"], got["pos"]
    qn = np.concatenate([_n16(got["q_raw"][h * hd:(h + 1) * hd], w["q_norm"], eps) for h in range(nq)])
    q = f16_round(oracle.rope_neox(qn, nq, hd, shape["rotated_pairs"], pos, shape["theta"]))
    kvd = nkv * hd
    K = from_f16_bits(got["kcache"][:(pos + 1) * kvd])
    V = from_f16_bits(got["vcache"][:(pos + 1) * kvd])
    stage["attn"] = f16_round(oracle.attention(q, K, V, hd, nq, nkv, pos + 1, shape["window"], shape["scale"]))
    stage["o"] = f16_round(oracle.gemv_int4(*w["o"], got["attn"]))
    h = f16_round(h_in + _n16(got["o"], w["post_attention_norm"], eps))
    logits = oracle.router_logits(w["router_w"], w["router_s"], w["router_b"], _n16(h, None, eps),
                                  from_f16_bits(w["router_eff"]))
    ridx, rw = oracle.topk_softmax(logits, shape["k"], from_f16_bits(w["router_gain"]))
    assert list(ridx) == list(got["idx"]), f"{label}: routing of the GPU's h differs"
    stage["w"] = f16_round(rw)
    sh = (w["shared_gate"], w["shared_up"], w["shared_down"])
    shared = oracle.shared_expert_int8 if w.get("shared_bits", 4) == 8 else oracle.shared_expert_int4
    stage["h1"] = f16_round(shared(*sh, _n16(h, w["pre_ffn_norm"], eps), d, shape["fs"]))
    stage["h2"] = f16_round(oracle.moe_routed(w["pool"], w["stride"], w["off"], _n16(h, w["pre_ffn2_norm"], eps),
                                              ridx, got["w"], d, shape["f"], bits=w.get("expert_bits", 4)))
    h12 = f16_round(_n16(got["h1"], w["post_ffn1_norm"], eps) + _n16(got["h2"], w["post_ffn2_norm"], eps))
    stage["out"] = f16_round(f16_round(h + _n16(h12, w["post_ffn_norm"], eps)) *
                             f16_round(np.float32(w["layer_scalar"])))
    for key, expect in stage.items():
        rel = oracle.rel_error(got[key], expect)
        assert rel < TOL, f"{label}: stage {key} rel={rel}"
    chained = oracle.rel_error(got["out"], ref["out"])
    floor, trials = chain_floor(w, shape, hidden, got["kc_in"], got["vc_in"], pos, trials=12)
    msg = (f"{label}: end-to-end rel={chained:.4g}; oracle against itself perturbed at fp32 size: "
           f"max {floor:.4g} over {[float(f'{t:.3g}') for t in trials]}")
    print(f"[layer] {msg}", flush=True)
    assert chained < TOL or chained <= floor, msg
    assert chained < oracle.Tolerance.fp16_chained_reduction, msg

SMALL = dict(d=256, nq=4, nkv=2, hd=128, rotated_pairs=64, window=0, f=128, fs=192, k=2,
             eps=1e-6, theta=10000.0, scale=1.0)
CONFIG4 = dict(d=2816, nq=16, nkv=8, hd=256, rotated_pairs=128, window=0, f=704, fs=2112, k=8,
               eps=1e-6, theta=10000.0, scale=1.0)


@pytest.mark.parametrize("pos", [0, 70, 130])
def test_layer_small_matches_reference(ctx, stream, pos):
    got, ref, w, hid = _layer_case(ctx, stream, SMALL, 8, pos, 160, 3, f"small-{pos}")
    _check_layer(got, ref, w, SMALL, hid, f"small pos={pos}")


def test_layer_small_window_and_partial_rotary(ctx, stream):
    shape = dict(SMALL, window=64, rotated_pairs=16, theta=1e6)
    got, ref, w, hid = _layer_case(ctx, stream, shape, 8, 200, 256, 4, "small-swa")
    _check_layer(got, ref, w, shape, hid, "small window")


@pytest.mark.parametrize("bits", [2, 3])
def test_layer_small_with_2_3_bit_experts(ctx, stream, bits):
    # the routed experts of the layer at 2/3 bits (the pool's weight_bits;
    # quant.routedExpert.weightBits, Model.swift:61-63)
    got, ref, w, hid = _layer_case(ctx, stream, SMALL, 8, 70, 160, 7, f"small-b{bits}", expert_bits=bits)
    _check_layer(got, ref, w, SMALL, hid, f"small {bits}-bit experts")


def test_layer_small_with_int8_shared_expert(ctx, stream):
    # the shared expert at 8 bits, the reference's default width when the
    # manifest has no quant block (Model.swift:59)
    got, ref, w, hid = _layer_case(ctx, stream, SMALL, 8, 70, 160, 8, "small-s8", shared_bits=8)
    _check_layer(got, ref, w, SMALL, hid, "small int8 shared")


def test_layer_in_place_equals_out_of_place(ctx, stream):
    a = _layer_case(ctx, stream, SMALL, 8, 33, 64, 5, "inplace")[0]
    b = _layer_case(ctx, stream, SMALL, 8, 33, 64, 5, "inplace", in_place=True)[0]
    assert np.array_equal(a["out"].view(np.uint32), b["out"].view(np.uint32))


def test_layer_config4_full_context(ctx, stream):
    # d 2816, 16 q / 8 kv heads x 256, context 4096 (the
    # new token at position 4095), shared expert 2112, top-8 of 128 experts
    got, ref, w, hid = _layer_case(ctx, stream, CONFIG4, 128, 4095, 4096, 0, "c4")
    _check_layer(got, ref, w, CONFIG4, hid, "config 4")


def test_layer_config4_int8_shared_expert(ctx, stream):
    # config 4 with the shared expert [2112 x 2816] at 8 bits
    got, ref, w, hid = _layer_case(ctx, stream, CONFIG4, 128, 4095, 4096, 9, "c4-s8", shared_bits=8)
    _check_layer(got, ref, w, CONFIG4, hid, "config 4, int8 shared")


# Gemma 4's full-attention layers (every sixth, ModelTypes.swift:84-105):
# head_dim 512, 2 kv heads (group 8), rope theta 1e6, partial rotary 0.25
# (rotated pairs 512·0.25/2 = 64), no v projection: V is the k projection
# (RealForwardRunner.swift:2252-2255, 2303).
SMALL_FULL = dict(d=256, nq=8, nkv=1, hd=512, rotated_pairs=64, window=0, f=128, fs=192, k=2,
                  eps=1e-6, theta=1e6, scale=1.0, full=True)
CONFIG4_FULL = dict(CONFIG4, nkv=2, hd=512, rotated_pairs=64, theta=1e6, full=True)


@pytest.mark.parametrize("pos", [0, 70, 130])
def test_layer_small_full_attention(ctx, stream, pos):
    got, ref, w, hid = _layer_case(ctx, stream, SMALL_FULL, 8, pos, 160, 10, f"small-full-{pos}")
    _check_layer(got, ref, w, SMALL_FULL, hid, f"small full pos={pos}")


def test_layer_config4_full_attention(ctx, stream):
    # a full-attention layer at the config-4 sizes: 16 q / 2 kv heads x 512,
    # the new token at position 4095
    got, ref, w, hid = _layer_case(ctx, stream, CONFIG4_FULL, 128, 4095, 4096, 11, "c4-full")
    _check_layer(got, ref, w, CONFIG4_FULL, hid, "config 4, full attention")


def test_layer_graph_replays_match_eager(ctx, stream):
    shape, E, pos, cap = SMALL, 8, 90, 128
    w = synth.decode_layer(6, "graph", shape["d"], shape["nq"], shape["nkv"], shape["hd"], E, shape["f"],
                           shape["fs"])
    kvd = shape["nkv"] * shape["hd"]
    kb = _dev(synth.f16_vector(6, "graph/kc", cap * kvd))
    vb = _dev(synth.f16_vector(6, "graph/vc", cap * kvd))
    hb = _dev(synth.f16_vector(6, "graph/hidden", shape["d"]))
    spec = _spec(shape)
    ws_bytes = ops.decode_layer_workspace_bytes(spec, pos + 1)
    ws = DeviceBuffer(ws_bytes)
    ob = _dev(np.zeros(shape["d"], np.uint16))
    layer = ops.DecodeLayer(ctx, ops.DecodeLayerWeightsSpec.upload(w), spec)
    layer.encode(stream, hb, ob, kb, vb, pos, ws, ws_bytes)
    stream.sync()
    eager = ob.download(np.uint16, shape["d"]).copy()
    g = Graph(stream, lambda: layer.encode(stream, hb, ob, kb, vb, pos, ws, ws_bytes))
    for r in range(3):
        ob.fill(0)
        ws.fill(0xFF)
        g.launch(stream)
        stream.sync()
        assert np.array_equal(ob.download(np.uint16, shape["d"]), eager), f"replay {r}"


# ------------------------------------------------------------ layer chains ----
#
# tfq_decode_layers: n layers per call, layer i's tail formed inside layer
# i+1's QKV launch (kStageTail). At d = 256 each thread of the QKV staging
# owns the same 16-byte chunk as in the tail kernel, so the fused tail's sums
# are the tail kernel's and the chain equals per-layer calls bit for bit; at
# the config-4 sizes every layer's output is held to the oracle layer fed the
# chain's previous output, as the single-layer test holds the end-to-end one.

def _chain_case(ctx, stream, shapes, E, pos, cap, seed, label):
    ws_list, specs, caches = [], [], []
    for i, sh in enumerate(shapes):
        w = synth.decode_layer(seed + i, f"{label}/L{i}", sh["d"], sh["nq"], sh["nkv"], sh["hd"], E, sh["f"], sh["fs"],
                               v_proj=not sh.get("full", False))
        kvd = sh["nkv"] * sh["hd"]
        caches.append((synth.f16_vector(seed + i, f"{label}/L{i}/kc", cap * kvd),
                       synth.f16_vector(seed + i, f"{label}/L{i}/vc", cap * kvd)))
        ws_list.append(w)
        specs.append(_spec(sh))
    return ws_list, specs, caches


def _run_chain(ctx, stream, ws_list, specs, caches, hidden, pos, d):
    n = len(ws_list)
    up = [ops.DecodeLayerWeightsSpec.upload(w) for w in ws_list]
    chain = ops.DecodeLayers(ctx, up, specs)
    wsb = chain.workspace_bytes(pos + 1)
    ws = DeviceBuffer(wsb)
    kb = [_dev(kc) for kc, _ in caches]
    vb = [_dev(vc) for _, vc in caches]
    hs = _dev(np.full(n * d, 0x7E00, np.uint16))
    chain.encode(stream, _dev(hidden), hs, kb, vb, pos, ws, wsb)
    stream.sync()
    return from_f16_bits(hs.download(np.uint16, n * d)).reshape(n, d), hs.download(np.uint16, n * d).reshape(n, d)


def test_layer_chain_equals_layer_calls_small(ctx, stream):
    shapes = [SMALL, SMALL_FULL, dict(SMALL, window=64, rotated_pairs=16, theta=1e6)]
    pos, cap, d = 70, 160, SMALL["d"]
    ws_list, specs, caches = _chain_case(ctx, stream, shapes, 8, pos, cap, 12, "chain")
    hidden = synth.f16_vector(12, "chain/hidden", d)
    print(f"[chain] small 3 layers pos={pos}", flush=True)
    _, got = _run_chain(ctx, stream, ws_list, specs, caches, hidden, pos, d)
    h = _dev(hidden)
    for i, (w, spec, (kc, vc)) in enumerate(zip(ws_list, specs, caches)):
        layer = ops.DecodeLayer(ctx, ops.DecodeLayerWeightsSpec.upload(w), spec)
        wsb = ops.decode_layer_workspace_bytes(spec, pos + 1)
        out = _dev(np.zeros(d, np.uint16))
        layer.encode(stream, h, out, _dev(kc), _dev(vc), pos, DeviceBuffer(wsb), wsb)
        stream.sync()
        ref = out.download(np.uint16, d)
        assert np.array_equal(got[i], ref), f"layer {i}: {np.count_nonzero(got[i] != ref)} words differ"
        h = out


def test_layer_chain_config4_sliding_and_full(ctx, stream):
    shapes = [CONFIG4, CONFIG4_FULL]
    pos, cap, d = 4095, 4096, CONFIG4["d"]
    ws_list, specs, caches = _chain_case(ctx, stream, shapes, 128, pos, cap, 13, "c4chain")
    hidden = synth.f16_vector(13, "c4chain/hidden", d)
    print(f"[chain] config 4 sliding + full pos={pos}", flush=True)
    outs, _ = _run_chain(ctx, stream, ws_list, specs, caches, hidden, pos, d)
    inp = hidden
    for i, (w, sh, (kc, vc)) in enumerate(zip(ws_list, shapes, caches)):
        ref = from_f16_bits(oracle.decode_layer(w, sh, inp, kc.copy(), vc.copy(), pos)[0])
        rel = oracle.rel_error(outs[i], ref)
        floor, trials = chain_floor(w, sh, inp, kc, vc, pos, trials=12)
        msg = f"chain layer {i}: rel={rel:.4g}, oracle spread {floor:.4g}"
        print(f"[chain] {msg}", flush=True)
        assert rel < TOL or rel <= floor, msg
        inp = synth.f16_bits(outs[i])
