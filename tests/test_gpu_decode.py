"""GPU parity of the decode path (GEMVs, router top-k, routed MoE, shared
expert) against the CPU oracle, through libtfq's C ABI.

Test names and inputs mirror the reference's kernel tests
(T/ = Tests/TurboFieldfare/Core/ in the reference checkout). Tolerances:
north-star bar max relative error (RelError.compute) <= 1e-3 for every
floating-point output, tighter than the reference's own 5e-3 / 1e-2;
top-k indices and expert order bit-exact.
"""
import numpy as np
import pytest

import oracle
from edgeexpert_amd import ops, synth
from edgeexpert_amd._lib import ROUTER_WORKSPACE_BYTES, TfqError, TFQ_E_INVAL
from edgeexpert_amd.runtime import DeviceBuffer
from helpers import bf16_to_f16_exact, f16_bits, f16_round, from_f16_bits, ref_int4_rows, ref_int8_rows

pytestmark = pytest.mark.gpu
TOL = oracle.Tolerance.north_star
GROUP_SWEEP = [64, 128, 192, 256, 320, 512]     # OffByMultiples.multiplesOfGroup ≤ 512


def _dev(a, pad_to=0):
    return DeviceBuffer.from_array(np.ascontiguousarray(a), pad_to=pad_to)


def _run_q4(ctx, stream, W, S16, B16, x16, m, n, weight_offset=0):
    wbuf = DeviceBuffer(W.nbytes + weight_offset)
    wbuf.upload(W, offset=weight_offset)
    sb, bb, xb = _dev(S16), _dev(B16), _dev(x16)
    yb = _dev(np.full(m, 0x7E00, np.uint16))            # NaN sentinel
    ops.DequantInt4GEMV(ctx).encode(stream, wbuf, sb, bb, xb, yb, m, n, weights_offset=weight_offset)
    stream.sync()
    return from_f16_bits(yb.download(np.uint16, m))


# ---------------------------------------------------------- int4 GEMV ----

def _q4_run_and_compare(ctx, stream, m, n, seed, weight_offset=0):
    # T/Kernels/Quant/DequantInt4GEMVTests.swift:41-100
    W, S, B, xr = ref_int4_rows(seed, f"int4-gemv-kernel-m{m}-n{n}", m, n, -0.5, 0.5, extra=n)
    x16 = f16_bits(xr)
    y = _run_q4(ctx, stream, W, bf16_to_f16_exact(S), bf16_to_f16_exact(B), x16, m, n, weight_offset)
    ref = oracle.gemv_int4(W, S, B, f16_round(xr), oracle.FMT_BF16)
    rel = oracle.rel_error(y, ref)
    assert rel < TOL, f"M={m} N={n}: rel={rel}"


@pytest.mark.parametrize("m,n,seed", [(128, 128, 0xC1), (1024, 2816, 0xC2), (64, 64, 0xC3)])
def test_gemv_q4_reference_shapes(ctx, stream, m, n, seed):
    _q4_run_and_compare(ctx, stream, m, n, seed)


@pytest.mark.parametrize("m", [64, 65, 128, 129])
@pytest.mark.parametrize("n", GROUP_SWEEP)
def test_gemv_q4_sweep(ctx, stream, m, n):
    _q4_run_and_compare(ctx, stream, m, n, (m * 0x9E37 + n) & 0xFFFFFFFFFFFFFFFF)


# the last two: more rows than one round of resident blocks covers, so every
# wavefront runs several row groups (two in flight; odd counts for some)
@pytest.mark.parametrize("m,n", [(2816, 4096), (4096, 2816), (2816, 2112), (2816, 704), (2048, 8192),
                                 (40000, 2816), (30001, 512)])
def test_gemv_q4_production_shapes(ctx, stream, m, n):
    W, S, B = synth.int4_matrix(1, f"prod/{m}x{n}", m, n)
    x16 = synth.f16_vector(1, f"prod/x{n}", n)
    y = _run_q4(ctx, stream, W, S, B, x16, m, n)
    ref = oracle.gemv_int4(W, S, B, from_f16_bits(x16))
    assert oracle.rel_error(y, ref) < TOL


@pytest.mark.parametrize("m,n", [(256, 2816), (256, 8192), (128, 192)])
def test_gemv_q4_staging_forms_agree(ctx, stream, m, n):
    # a 16-byte aligned x takes the form whose staging mode is fixed at
    # compile time (plain up to n = 4096, wide up to 8192), a 2-byte aligned x
    # the form that reads the mode: the same arithmetic, so the same bits
    W, S, B = synth.int4_matrix(3, f"forms/{m}x{n}", m, n)
    x16 = synth.f16_vector(3, f"forms/x{n}", n)
    wb, sb, bb = _dev(W), _dev(S), _dev(B)
    outs = []
    for off in (0, 2):
        xb = DeviceBuffer(n * 2 + 16)
        xb.upload(x16, offset=off)
        yb = _dev(np.full(m, 0x7E00, np.uint16))
        ops.DequantInt4GEMV(ctx).encode(stream, wb, sb, bb, xb, yb, m, n, x_offset=off)
        stream.sync()
        outs.append(yb.download(np.uint16, m))
    assert np.array_equal(outs[0], outs[1])
    assert oracle.rel_error(from_f16_bits(outs[0]), oracle.gemv_int4(W, S, B, from_f16_bits(x16))) < TOL


@pytest.mark.parametrize("E,d,with_eff", [(128, 2816, False), (128, 2816, True), (8, 256, True)])
def test_router_logits_staging_forms_agree(ctx, stream, E, d, with_eff):
    # 16-byte aligned h (and effective scale) takes the router form whose
    # staging mode is fixed at compile time, a 2-byte aligned h the form that
    # reads the mode: the same logits, bit for bit
    rW, rS, rB = synth.int8_matrix(4, f"rforms/{E}x{d}", E, d)
    h16 = synth.f16_vector(4, f"rforms/h{d}", d)
    eff = synth.f16_vector(4, f"rforms/eff{d}", d) if with_eff else None
    rb = tuple(_dev(a) for a in (rW, rS, rB))
    effb = _dev(eff) if with_eff else None
    moe = ops.MoE(ctx)
    outs = []
    for off in (0, 2):
        hb = DeviceBuffer(d * 2 + 16)
        hb.upload(h16, offset=off)
        lb = _dev(np.full(E, np.nan, np.float32))
        moe.encode_router_logits(stream, *rb, hb.ptr(off), effb, lb, E, d)
        stream.sync()
        outs.append(lb.download(np.float32, E))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    ref = oracle.router_logits(rW, rS, rB, from_f16_bits(h16), None if eff is None else from_f16_bits(eff))
    assert oracle.rel_error(outs[0], ref) < 1e-5


def test_gemv_q4_baseline_config0(ctx, stream):
    # W[2816, 2816] int4 g64, fp16 scale/bias, x ~ N(0,1), seed 0.
    W, S, B = synth.int4_matrix(0, "c0/w", 2816, 2816)
    x16 = synth.f16_vector(0, "c0/x", 2816)
    y = _run_q4(ctx, stream, W, S, B, x16, 2816, 2816)
    x = from_f16_bits(x16)
    ref = oracle.gemv_int4(W, S, B, x)
    ref64 = oracle.gemv_int4_f64(W, S, B, x)
    assert oracle.rel_error(y, ref) < TOL
    assert oracle.rel_error(y, ref64) < TOL


def test_gemv_q4_weight_offset_16_works_and_2_is_rejected(ctx, stream):
    # T/Kernels/Quant/DequantInt4GEMVTests.swift:114-121 binds weights at +2. The
    # MI355X kernel loads 128-bit chunks, so a 16-byte aligned offset is required
    # and anything else is rejected with TFQ_E_INVAL instead of trapping.
    _q4_run_and_compare(ctx, stream, 128, 2816, 0xC4, weight_offset=16)
    with pytest.raises(TfqError) as ei:
        _q4_run_and_compare(ctx, stream, 128, 2816, 0xC4, weight_offset=2)
    assert ei.value.status == TFQ_E_INVAL


def test_gemv_q4_rejects_bad_shapes(ctx, stream):
    b = DeviceBuffer(4096)
    g = ops.DequantInt4GEMV(ctx)
    for m, n in [(4, 100), (0, 64), (4, 0)]:
        with pytest.raises(TfqError) as ei:
            g.encode(stream, b, b, b, b, b, m, n)
        assert ei.value.status == TFQ_E_INVAL


def test_gemv_q4_is_deterministic(ctx, stream):
    W, S, B = synth.int4_matrix(2, "det/w", 512, 2816)
    x16 = synth.f16_vector(2, "det/x", 2816)
    a = _run_q4(ctx, stream, W, S, B, x16, 512, 2816)
    b = _run_q4(ctx, stream, W, S, B, x16, 512, 2816)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_fused_qkv_equals_three_gemvs(ctx, stream):
    # FusedQKVGEMV (S/Kernels/Fusions/FusedQKVGEMV.swift:92-156); C4 shapes.
    n, mq, mkv = 2816, 4096, 2048
    mats = {k: synth.int4_matrix(4, f"qkv/{k}", r, n) for k, r in (("q", mq), ("k", mkv), ("v", mkv))}
    x16 = synth.f16_vector(4, "qkv/x", n)
    dev = {k: tuple(_dev(a) for a in v) for k, v in mats.items()}
    ys = {k: _dev(np.zeros(r, np.uint16)) for k, r in (("q", mq), ("k", mkv), ("v", mkv))}
    proj = {k: ops.Q4Projection(*dev[k], rows=r, cols=n) for k, r in (("q", mq), ("k", mkv), ("v", mkv))}
    xb = _dev(x16)
    ops.DequantInt4GEMV(ctx).encode_qkv(stream, proj["q"], proj["k"], proj["v"], xb, ys["q"], ys["k"],
                                        ys["v"], mq, mkv, n)
    stream.sync()
    x = from_f16_bits(x16)
    for k, r in (("q", mq), ("k", mkv), ("v", mkv)):
        got = from_f16_bits(ys[k].download(np.uint16, r))
        single = _run_q4(ctx, stream, *mats[k], x16, r, n)
        assert np.array_equal(got.view(np.uint32), single.view(np.uint32))
        assert oracle.rel_error(got, oracle.gemv_int4(*mats[k], x)) < TOL


# ---------------------------------------------------------- int8 GEMV ----

def _q8_run_and_compare(ctx, stream, m, n, seed):
    # T/Kernels/Quant/DequantInt8GEMVTests.swift:16-54
    W, S, B, xr = ref_int8_rows(seed, f"int8-gemv-m{m}-n{n}", m, n, -1.0, 1.0, extra=n)
    x16 = f16_bits(xr)
    bufs = [_dev(W), _dev(bf16_to_f16_exact(S)), _dev(bf16_to_f16_exact(B)), _dev(x16)]
    yb = _dev(np.full(m, 0x7E00, np.uint16))
    ops.DequantInt8GEMV(ctx).encode(stream, *bufs, yb, m, n)
    stream.sync()
    y = from_f16_bits(yb.download(np.uint16, m))
    ref = oracle.gemv_int8(W, S, B, f16_round(xr), oracle.FMT_BF16)
    rel = oracle.rel_error(y, ref)
    assert rel < TOL, f"M={m} N={n}: rel={rel}"


@pytest.mark.parametrize("m,n,seed", [(128, 2816, 0x151), (1024, 2816, 0x152)])
def test_gemv_q8_reference_shapes(ctx, stream, m, n, seed):
    _q8_run_and_compare(ctx, stream, m, n, seed)


@pytest.mark.parametrize("m", [128, 256, 1024])
@pytest.mark.parametrize("n", GROUP_SWEEP)
def test_gemv_q8_sweep(ctx, stream, m, n):
    _q8_run_and_compare(ctx, stream, m, n, m * 1000 + n)


@pytest.mark.parametrize("m,n", [(128, 2816), (1024, 4096), (96, 192)])
def test_gemv_q8_staging_forms_agree(ctx, stream, m, n):
    # a 16-byte aligned x takes the int8 GEMV form whose copy staging is
    # fixed at compile time, a 2-byte aligned x the form that reads the
    # staging mode: the same arithmetic, so the same bits (and the oracle's)
    W, S, B, xr = ref_int8_rows(0x160 + m, f"int8-forms-m{m}-n{n}", m, n, -1.0, 1.0, extra=n)
    x16 = f16_bits(xr)
    wb, sb, bb = _dev(W), _dev(bf16_to_f16_exact(S)), _dev(bf16_to_f16_exact(B))
    outs = []
    for off in (0, 2):
        xb = DeviceBuffer(n * 2 + 16)
        xb.upload(x16, offset=off)
        yb = _dev(np.full(m, 0x7E00, np.uint16))
        ops.DequantInt8GEMV(ctx).encode(stream, wb, sb, bb, xb, yb, m, n, x_offset=off)
        stream.sync()
        outs.append(yb.download(np.uint16, m))
    assert np.array_equal(outs[0], outs[1])
    ref = oracle.gemv_int8(W, S, B, f16_round(xr), oracle.FMT_BF16)
    assert oracle.rel_error(from_f16_bits(outs[0]), ref) < TOL


# ------------------------------------------------------------- router ----

def _run_router(ctx, stream, W, S16, B16, h16, eff16, gain16, E, d, k, ws=None):
    if ws is None:
        ws = DeviceBuffer(ROUTER_WORKSPACE_BYTES)
        ws.fill(0)
    bufs = [_dev(W), _dev(S16), _dev(B16), _dev(h16)]
    effb = _dev(eff16) if eff16 is not None else None
    gb = _dev(gain16) if gain16 is not None else None
    idx = _dev(np.full(k, 0xFFFFFFFF, np.uint32))
    w16 = _dev(np.zeros(k, np.uint16))
    w32 = _dev(np.zeros(k, np.float32))
    logits = _dev(np.zeros(E, np.float32))
    ops.MoE(ctx).encode_router_gemma4(stream, *bufs, effb, gb, idx, w16, E, d, k, ws,
                                      out_weights_f32=w32, out_logits=logits)
    stream.sync()
    return (idx.download(np.uint32, k), from_f16_bits(w16.download(np.uint16, k)),
            w32.download(np.float32, k), logits.download(np.float32, E), ws)


def test_router_production_matches_reference(ctx, stream):
    # T/Kernels/MoE/RouterTopKTests.swift:17-44
    E, D, K = 16, 128, 8
    r = oracle.SplitMix64(0xA5B61234)
    weights = np.stack([r.uniforms(D, -0.05, 0.05) + np.float32(e * 0.01) for e in range(E)])
    hidden = r.uniforms(D, -1.0, 1.0)
    inv = np.float32(1.0) / np.sqrt(np.float32(D))
    eff = (r.uniforms(D, 0.5, 1.5) * inv).astype(np.float32)
    gain = r.uniforms(E, 0.6, 1.4)
    W, S, B = oracle.quantize_int8_matrix(weights)
    h16, eff16, gain16 = f16_bits(hidden), f16_bits(eff), f16_bits(gain)
    idx, w, wf, logits, _ = _run_router(ctx, stream, W, bf16_to_f16_exact(S), bf16_to_f16_exact(B),
                                        h16, eff16, gain16, E, D, K)
    # the oracle sees exactly the values the device buffers hold
    ref_logits = oracle.router_logits(W, S, B, from_f16_bits(h16), from_f16_bits(eff16), oracle.FMT_BF16)
    ref_idx, ref_w = oracle.topk_softmax(ref_logits, K, from_f16_bits(gain16))
    assert list(idx) == list(ref_idx)
    assert oracle.rel_error(logits, ref_logits) < 1e-5
    assert np.max(np.abs(wf - ref_w)) < 1e-5
    assert np.max(np.abs(w - ref_w)) < 5e-3 * 0.2      # fp16 rounding of weights ≤ 1 half-ulp


def test_router_near_tie_like_reference(ctx, stream):
    # T/Kernels/MoE/RouterTopKTests.swift:46-70
    E, D, K = 16, 128, 8
    r = oracle.SplitMix64(0x71E0F4A)
    pattern = r.uniforms(D, 0.2, 1.0)
    hidden = r.uniforms(D, 0.5, 1.5)
    gains = np.zeros(E, np.float32)
    for e in range(7):
        gains[e] = 1.0 - e * 0.05
    gains[7] = 0.5
    gains[8] = 0.5 * (1.0 + 1e-4)
    for e in range(9, E):
        gains[e] = 0.4 - (e - 9) * 0.02
    W, S, B = oracle.quantize_int8_matrix(np.outer(gains, pattern).astype(np.float32))
    h16 = f16_bits(hidden)
    idx, _, _, logits, _ = _run_router(ctx, stream, W, bf16_to_f16_exact(S), bf16_to_f16_exact(B), h16,
                                       None, None, E, D, K)
    ref_logits = oracle.router_logits(W, S, B, from_f16_bits(h16), None, oracle.FMT_BF16)
    ref_idx, _ = oracle.topk_softmax(ref_logits, K)
    assert list(idx) == list(ref_idx)


def test_router_baseline_config1_and_workspace_reuse(ctx, stream):
    # BASELINE config 1 router: int8 g64 [128 x 2816], eff = gain = 1; several tokens.
    E, D, K = 128, 2816, 8
    W, S, B = synth.int8_matrix(0, "c1/router", E, D)
    ws = None
    for t in range(4):
        h16 = synth.f16_vector(0, f"c1/h{t}", D)
        idx, w, wf, logits, ws = _run_router(ctx, stream, W, S, B, h16, None, None, E, D, K, ws)
        ref_logits = oracle.router_logits(W, S, B, from_f16_bits(h16))
        ref_idx, ref_w = oracle.topk_softmax(ref_logits, K)
        srt = np.sort(ref_logits)[::-1]
        assert srt[K - 1] - srt[K] > 1e-3, "ambiguous 8th/9th margin"
        assert list(idx) == list(ref_idx)
        assert np.max(np.abs(wf - ref_w)) < 1e-5


@pytest.mark.parametrize("E,k", [(256, 64), (64, 1), (128, 16)])
def test_router_topk_sizes(ctx, stream, E, k):
    D = 512
    W, S, B = synth.int8_matrix(7, f"rt/{E}", E, D)
    h16 = synth.f16_vector(7, f"rt/h{E}", D)
    idx, _, wf, logits, _ = _run_router(ctx, stream, W, S, B, h16, None, None, E, D, k)
    ref_idx, ref_w = oracle.topk_softmax(logits, k)     # selection pinned on the device logits
    assert list(idx) == list(ref_idx)
    assert np.max(np.abs(wf - ref_w)) < 1e-5


# ---------------------------------------------------------- routed MoE ----

def _pool_from_blobs(blobs):
    stride = blobs[0][0].size
    return np.concatenate([b for b, _ in blobs]), stride


def _make_ref_blob(gates, ups, downs, align=16):
    """Blob like MoEFusedFFNTests.makeBlob (T/Kernels/MoE/MoEFusedFFNTests.swift:161-197)
    with weights padded to 16-byte boundaries and fp16 scale/bias words."""
    parts, offs, cur = [], {}, 0
    for proj, rows in (("gate", gates), ("up", ups), ("down", downs)):
        W, S, B = oracle.quantize_int4_matrix(rows)
        for part, arr in (("w", W), ("s", bf16_to_f16_exact(S)), ("b", bf16_to_f16_exact(B))):
            pad = (-cur) % align
            parts.append(np.zeros(pad, np.uint8))
            cur += pad
            offs[f"{proj}_{part}"] = cur
            raw = np.ascontiguousarray(arr).view(np.uint8).ravel()
            parts.append(raw)
            cur += raw.size
    pad = (-cur) % 256
    parts.append(np.zeros(pad, np.uint8))
    return np.concatenate(parts), offs


def test_routed_pipeline_and_hit_split_match_reference(ctx, stream):
    # T/Kernels/MoE/MoEFusedFFNTests.swift:17-159
    D, F, K = 128, 64, 8
    key = synth.seed_key(0x2D3, "production-routed-moe")
    u = synth.uniform24(key, K * (2 * F * D + D * F) + 2 * D, -0.4, 0.4)
    pos = 0
    blobs = []
    for _ in range(K):
        g = u[pos:pos + F * D].reshape(F, D); pos += F * D
        up = u[pos:pos + F * D].reshape(F, D); pos += F * D
        dn = u[pos:pos + D * F].reshape(D, F); pos += D * F
        blobs.append(_make_ref_blob(g, up, dn))
    # x, residual: uniform(-0.5, 0.5) drawn after the weights, rounded to fp16
    tail = synth.uniform24(key, K * (2 * F * D + D * F) + 2 * D, -0.5, 0.5)[pos:]
    x16, res16 = f16_bits(tail[:D]), f16_bits(tail[D:])
    rw16 = f16_bits(np.array([0.04 + s * 0.015 for s in range(K)], np.float32))
    offs = blobs[0][1]
    pool_bytes = np.concatenate([b for b, _ in blobs])
    stride = blobs[0][0].size
    pool = ops.ExpertPool(_dev(pool_bytes), stride, K, offs)
    idx = _dev(np.arange(K, dtype=np.uint32))
    xb, resb, rwb = _dev(x16), _dev(res16), _dev(rw16)
    moe = ops.MoE(ctx)
    full_acts = _dev(np.full(K * F, 0x7E00, np.uint16))      # fp16 NaN sentinels
    split_acts = _dev(np.full(K * F, 0x7E00, np.uint16))
    yf = _dev(np.zeros(D, np.uint16))
    ys = _dev(np.zeros(D, np.uint16))
    moe.encode_routed_phase1(stream, pool, idx, xb, full_acts, D, F, K)
    moe.encode_routed_phase2(stream, pool, idx, full_acts, rwb, resb, yf, D, F, K)
    low, high = _dev(np.arange(0, 4, dtype=np.uint32)), _dev(np.arange(4, 8, dtype=np.uint32))
    moe.encode_routed_phase1_subset(stream, pool, idx, xb, split_acts, low, 4, D, F, K)
    moe.encode_routed_phase1_subset(stream, pool, idx, xb, split_acts, high, 4, D, F, K)
    moe.encode_routed_phase2(stream, pool, idx, split_acts, rwb, resb, ys, D, F, K)
    stream.sync()
    full = from_f16_bits(yf.download(np.uint16, D))
    split = from_f16_bits(ys.download(np.uint16, D))
    assert np.array_equal(full.view(np.uint32), split.view(np.uint32))
    expected = oracle.moe_routed(pool_bytes, stride, offs, from_f16_bits(x16), np.arange(K),
                                 from_f16_bits(rw16), D, F, residual=from_f16_bits(res16))
    rel = oracle.rel_error(full, expected)
    assert rel < TOL, f"rel={rel}"


@pytest.mark.parametrize("F", [4096, 3968])
def test_moe_phase1_many_row_groups_per_wave(ctx, stream, F):
    # 8 slots x F gate/up rows: more rows than one round of resident phase-1
    # blocks covers, so every wavefront runs several row groups (two in
    # flight), their count even everywhere at F = 4096 and odd for some
    # wavefronts at F = 3968. Reference: g and u from the float64 GEMV
    # oracle, act = gelu_tanh(g)·u
    E, D, K = 12, 256, 8
    pool_bytes, offs, stride = synth.expert_pool(0x7A1, f"groups/experts/{F}", E, D, F)
    pool = ops.ExpertPool(_dev(pool_bytes), stride, E, offs)
    sel = np.array([11, 3, 7, 0, 9, 5, 2, 8], np.uint32)
    x16 = synth.f16_vector(0x7A2, f"groups/x/{F}", D)
    acts = _dev(np.full(K * F, 0x7E00, np.uint16))       # fp16 NaN sentinels
    ops.MoE(ctx).encode_routed_phase1(stream, pool, _dev(sel), _dev(x16), acts, D, F, K)
    stream.sync()
    got = from_f16_bits(acts.download(np.uint16, K * F)).reshape(K, F)
    x = from_f16_bits(x16)
    for s, e in enumerate(sel):
        blob = pool_bytes[int(e) * stride:(int(e) + 1) * stride]
        g = oracle.gemv_int4_f64(*synth.blob_views(blob, offs, D, F, "gate"), x)
        u = oracle.gemv_int4_f64(*synth.blob_views(blob, offs, D, F, "up"), x)
        ref = 0.5 * g * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (g + 0.044715 * g ** 3))) * u
        assert not np.isnan(got[s]).any(), f"F={F} slot {s}: a row was not written"
        rel = oracle.rel_error(got[s], ref)
        assert rel < TOL, f"F={F} slot {s}: rel={rel}"


def test_moe_baseline_config1_router_to_experts(ctx, stream):
    # 1 token, h ~ N(0,1) [2816], int8 router [128 x 2816],
    # softmax top-8, 128 int4 experts (gate/up [704 x 2816], down [2816 x 704])
    # resident in HBM; routing stays on the device.
    E, D, F, K = 128, 2816, 704, 8
    pool_bytes, offs, stride = synth.expert_pool(0, "c1/experts", E, D, F)
    Wr, Sr, Br = synth.int8_matrix(0, "c1/router", E, D)
    pool = ops.ExpertPool(_dev(pool_bytes), stride, E, offs)
    moe = ops.MoE(ctx)
    ws = DeviceBuffer(ROUTER_WORKSPACE_BYTES)
    ws.fill(0)
    rb = [_dev(Wr), _dev(Sr), _dev(Br)]
    idx, w16, wf = _dev(np.zeros(K, np.uint32)), _dev(np.zeros(K, np.uint16)), _dev(np.zeros(K, np.float32))
    acts = _dev(np.zeros(K * F, np.uint16))
    for t in range(3):
        h16 = synth.f16_vector(0, f"c1/h{t}", D)
        hb = _dev(h16)
        y = _dev(np.full(D, 0x7E00, np.uint16))
        moe.encode_router_gemma4(stream, *rb, hb, None, None, idx, w16, E, D, K, ws, out_weights_f32=wf)
        moe.encode_routed(stream, pool, idx, w16, hb, None, y, D, F, K, acts)
        stream.sync()
        got = from_f16_bits(y.download(np.uint16, D))
        h = from_f16_bits(h16)
        ref_idx, ref_w = oracle.topk_softmax(oracle.router_logits(Wr, Sr, Br, h), K)
        assert list(idx.download(np.uint32, K)) == list(ref_idx)
        # the expert block consumes the fp16 routing weights the router emits
        w_dev = from_f16_bits(w16.download(np.uint16, K))
        assert np.max(np.abs(w_dev - ref_w)) <= np.abs(ref_w).max() * 2.0 ** -11
        expected = oracle.moe_routed(pool_bytes, stride, offs, h, ref_idx, w_dev, D, F)
        rel = oracle.rel_error(got, expected)
        assert rel < TOL, f"token {t}: rel={rel}"


def test_moe_phase1_rejects_bad_contract(ctx, stream):
    E, D, F = 4, 128, 64
    pool_bytes, offs, stride = synth.expert_pool(0, "bad", E, D, F)
    pool = ops.ExpertPool(_dev(pool_bytes), stride, E, offs)
    b = _dev(np.zeros(4096, np.uint8))
    moe = ops.MoE(ctx)
    with pytest.raises(TfqError):
        moe.encode_routed_phase1(stream, pool, b, b, b, D, F, 9)          # topK > 8
    with pytest.raises(TfqError):
        moe.encode_routed_phase1(stream, pool, b, b, b, D + 32, F, 8)     # D % 64
    bad = ops.ExpertPool(pool.buffer, stride, E, dict(offs, down_w=offs["down_w"] + 2))
    with pytest.raises(TfqError):
        moe.encode_routed_phase2(stream, bad, b, b, b, None, b, D, F, 8)


# --------------------------------------------------------- shared expert ----

@pytest.mark.parametrize("d,f,seed,label", [(128, 64, 0x604, "shared-expert-int4"),
                                            (2816, 2112, 0, "c4/shared")])
def test_shared_expert_int4_matches_reference(ctx, stream, d, f, seed, label):
    # T/Kernels/MoE/SharedExpertInt4Tests.swift:11-53 (reference shapes) and the C4 shape
    if d == 128:
        key = synth.seed_key(seed, label)
        u = synth.uniform24(key, d + 2 * f * d + d * f, -0.4, 0.4)
        x = u[:d]
        gate = oracle.quantize_int4_matrix(u[d:d + f * d].reshape(f, d))
        up = oracle.quantize_int4_matrix(u[d + f * d:d + 2 * f * d].reshape(f, d))
        down = oracle.quantize_int4_matrix(u[d + 2 * f * d:].reshape(d, f))
        conv = lambda m: (m[0], bf16_to_f16_exact(m[1]), bf16_to_f16_exact(m[2]))
        gate, up, down = conv(gate), conv(up), conv(down)
    else:
        x = synth.normal(synth.seed_key(seed, label + "/x"), d)
        gate = synth.int4_matrix(seed, label + "/gate", f, d)
        up = synth.int4_matrix(seed, label + "/up", f, d)
        down = synth.int4_matrix(seed, label + "/down", d, f)
    x16 = f16_bits(x)
    proj = lambda m, r, c: ops.Q4Projection(_dev(m[0]), _dev(m[1]), _dev(m[2]), rows=r, cols=c)
    y = _dev(np.full(d, 0x7E00, np.uint16))
    act = _dev(np.zeros(f, np.uint16))
    ops.SharedExpertInt4(ctx).encode(stream, _dev(x16), proj(gate, f, d), proj(up, f, d),
                                     proj(down, d, f), y, act)
    stream.sync()
    got = from_f16_bits(y.download(np.uint16, d))
    ref = oracle.shared_expert_int4(gate, up, down, from_f16_bits(x16), d, f)
    rel = oracle.rel_error(got, ref)
    assert rel < TOL, f"rel={rel}"


def test_shared_expert_int4_staging_forms_agree(ctx, stream):
    # a 16-byte aligned x takes the gate/up form whose copy staging is fixed
    # at compile time, a 2-byte aligned x the form that reads the mode: the
    # same bits
    d, f, label = 2816, 2112, "c4/shared"
    x16 = f16_bits(synth.normal(synth.seed_key(3, label + "/x"), d))
    mats = [synth.int4_matrix(3, label + n, r, c) for n, r, c in (("/gate", f, d), ("/up", f, d), ("/down", d, f))]
    proj = lambda m, r, c: ops.Q4Projection(_dev(m[0]), _dev(m[1]), _dev(m[2]), rows=r, cols=c)
    gate, up, down = proj(mats[0], f, d), proj(mats[1], f, d), proj(mats[2], d, f)
    outs = []
    for off in (0, 2):
        xb = DeviceBuffer(d * 2 + 16)
        xb.upload(x16, offset=off)
        y = _dev(np.full(d, 0x7E00, np.uint16))
        act = _dev(np.zeros(f, np.uint16))
        ops.SharedExpertInt4(ctx).encode(stream, xb.ptr(off), gate, up, down, y, act)
        stream.sync()
        outs.append(y.download(np.uint16, d))
    assert np.array_equal(outs[0], outs[1])
    ref = oracle.shared_expert_int4(*mats, from_f16_bits(x16), d, f)
    assert oracle.rel_error(from_f16_bits(outs[0]), ref) < TOL


# -------------------------------------------------------------- loader ----

def test_convert_bf16_to_f16_exact_and_counts_inexact(ctx, stream):
    vals = np.array([1.0, -0.5, 0.02, 1e-3, 65280.0, 2.0 ** -14, 1e-30, 1e6, -3.0e5], np.float32)
    bits = synth.bf16_bits(vals)
    src, dst, cnt = _dev(bits), _dev(np.zeros(vals.size, np.uint16)), _dev(np.zeros(1, np.uint32))
    ops.convert_bf16_to_f16(ctx, stream, src, dst, vals.size, cnt)
    stream.sync()
    out = from_f16_bits(dst.download(np.uint16, vals.size))
    exact = synth.bf16_to_f32(bits)
    assert np.array_equal(out[:6], exact[:6])
    assert cnt.download(np.uint32, 1)[0] == 3


def test_phase1_with_selection_equals_router_select_then_phase1(ctx, stream):
    # the selection folded into phase 1 must give the routing of
    # tfq_router_topk and the activations of tfq_moe_phase1, bit for bit
    E, D, F, K = 128, 2816, 704, 8
    pool_bytes, offs, stride = synth.expert_pool(3, "sel/experts", E, D, F)
    Wr, Sr, Br = synth.int8_matrix(3, "sel/router", E, D)
    gain16 = f16_bits(synth.uniform24(synth.seed_key(3, "sel/gain"), E, 0.5, 1.5))
    pool = ops.ExpertPool(_dev(pool_bytes), stride, E, offs)
    moe = ops.MoE(ctx)
    rb = [_dev(Wr), _dev(Sr), _dev(Br)]
    gb = _dev(gain16)
    for t in range(3):
        h16 = synth.f16_vector(3, f"sel/h{t}", D)
        hb = _dev(h16)
        ws = DeviceBuffer(ROUTER_WORKSPACE_BYTES)
        ws.fill(0)
        logits_a, logits_b = _dev(np.zeros(E, np.float32)), _dev(np.zeros(E, np.float32))
        i1, w1, f1 = _dev(np.zeros(K, np.uint32)), _dev(np.zeros(K, np.uint16)), _dev(np.zeros(K, np.float32))
        i2, w2, f2 = _dev(np.zeros(K, np.uint32)), _dev(np.zeros(K, np.uint16)), _dev(np.zeros(K, np.float32))
        a1, a2 = _dev(np.zeros(K * F, np.uint16)), _dev(np.full(K * F, 0x7E00, np.uint16))
        moe.encode_router_gemma4(stream, *rb, hb, None, gb, i1, w1, E, D, K, ws, out_weights_f32=f1,
                                 out_logits=logits_a)
        moe.encode_routed_phase1(stream, pool, i1, hb, a1, D, F, K)
        moe.encode_router_logits(stream, *rb, hb, None, logits_b, E, D)
        moe.encode_routed_phase1_with_selection(stream, pool, logits_b, gb, E, i2, w2, hb, a2, D, F, K,
                                                out_weights_f32=f2)
        stream.sync()
        assert np.array_equal(logits_a.download(np.float32, E).view(np.uint32),
                              logits_b.download(np.float32, E).view(np.uint32))
        assert np.array_equal(i1.download(np.uint32, K), i2.download(np.uint32, K))
        assert np.array_equal(w1.download(np.uint16, K), w2.download(np.uint16, K))
        assert np.array_equal(f1.download(np.float32, K).view(np.uint32), f2.download(np.float32, K).view(np.uint32))
        assert np.array_equal(a1.download(np.uint16, K * F), a2.download(np.uint16, K * F))
        ref_idx, _ = oracle.topk_softmax(oracle.router_logits(Wr, Sr, Br, from_f16_bits(h16)), K,
                                         from_f16_bits(gain16))
        assert list(i2.download(np.uint32, K)) == list(ref_idx)



@pytest.mark.parametrize("with_inf", [False, True])
def test_phase1_selection_nan_signed_zero_and_infinities(ctx, stream, with_inf):
    # router_topk_select_k8 (moe.metal:152-168) never prefers a NaN score,
    # never takes -inf, and -0 == +0 ties by the lower index. Fed straight
    # into tfq_moe_phase1_routed's selection; indices bit-exact with the
    # oracle, weights equal where finite and NaN where the oracle's are
    # (a +inf logit makes every softmax weight inf - inf = NaN).
    E, D, F, K = 128, 256, 128, 8
    pool_bytes, offs, stride = synth.expert_pool(4, "nan/experts", E, D, F)
    pool = ops.ExpertPool(_dev(pool_bytes), stride, E, offs)
    logits = (-1.0 - synth.uniform24(synth.seed_key(4, "nan/logits"), E)).astype(np.float32)
    logits[3], logits[12] = 1.0, 0.5
    logits[[7, 64]] = 0.0
    logits[[40, 100]] = -0.0
    logits[[2, 9, 127]] = np.nan
    logits[[50, 51]] = -np.inf
    if with_inf:
        logits[20] = np.inf
    gain16 = f16_bits(synth.uniform24(synth.seed_key(4, "nan/gain"), E, 0.5, 1.5))
    idx, w16, wf = _dev(np.zeros(K, np.uint32)), _dev(np.zeros(K, np.uint16)), _dev(np.zeros(K, np.float32))
    acts = _dev(np.zeros(K * F, np.uint16))
    h16 = synth.f16_vector(4, "nan/h", D)
    ops.MoE(ctx).encode_routed_phase1_with_selection(stream, pool, _dev(logits), _dev(gain16), E, idx, w16, _dev(h16),
                                                     acts, D, F, K, out_weights_f32=wf)
    stream.sync()
    ref_idx, ref_w = oracle.topk_softmax(logits, K, from_f16_bits(gain16))
    got_idx = list(idx.download(np.uint32, K))
    assert got_idx == list(ref_idx)
    assert got_idx[:6] == ([20] if with_inf else []) + [3, 12, 7, 40, 64, 100][:6 - int(with_inf)]
    assert not set(got_idx) & {2, 9, 127, 50, 51}
    got_w = wf.download(np.float32, K)
    assert np.array_equal(np.isnan(got_w), np.isnan(ref_w)) and (np.all(np.isnan(ref_w)) == with_inf)
    fin = ~np.isnan(ref_w)
    assert np.all(np.abs(got_w[fin] - ref_w[fin]) <= 1e-6 * np.abs(ref_w[fin]))
    assert np.array_equal(np.isnan(from_f16_bits(w16.download(np.uint16, K))), np.isnan(ref_w))


# --------------------------------------------- fused decode token (C ABI) ----
#
# tfq_moe_decode_token: router GEMV (each router block also publishes its
# best 8 keys) -> phase 1 ranking those candidate lists -> phase 2. The
# selection must equal the oracle's top-k over all logits bit for bit,
# including ties that span router blocks (lower expert index first).

def _decode_token(ctx, stream, Wr, Sr, Br, h16, E, D, F, K, seed, label, gain16=None):
    pool_bytes, offs, stride = synth.expert_pool(seed, label, E, D, F)
    pool = ops.ExpertPool(_dev(pool_bytes), stride, E, offs)
    router = ops.Router(_dev(Wr), _dev(Sr), _dev(Br), E, None, None if gain16 is None else _dev(gain16))
    y = _dev(np.full(D, 0x7E00, np.uint16))
    idx, w16 = _dev(np.full(K, 0xFFFFFFFF, np.uint32)), _dev(np.zeros(K, np.uint16))
    acts = _dev(np.full(K * F, 0x7E00, np.uint16))
    ws = DeviceBuffer(ROUTER_WORKSPACE_BYTES)
    ws.fill(0xFF)
    ops.moe_decode_token(ctx, stream, router, pool, _dev(h16), None, y, D, F, K, idx, w16, acts, ws)
    stream.sync()
    h = from_f16_bits(h16)
    gain = None if gain16 is None else from_f16_bits(gain16)
    ref_idx, ref_w = oracle.topk_softmax(oracle.router_logits(Wr, Sr, Br, h), K, gain)
    got_idx = idx.download(np.uint32, K)
    assert list(got_idx) == list(ref_idx), f"{label}: {list(got_idx)} != {list(ref_idx)}"
    w_dev = from_f16_bits(w16.download(np.uint16, K))
    assert np.max(np.abs(w_dev - ref_w)) < 2e-3
    ref = oracle.moe_routed(pool_bytes, stride, offs, h, ref_idx, w_dev, D, F)
    rel = oracle.rel_error(from_f16_bits(y.download(np.uint16, D)), ref)
    assert rel < TOL, f"{label}: rel={rel}"
    return list(got_idx)


def test_decode_token_baseline_config1(ctx, stream):
    E, D, F, K = 128, 2816, 704, 8
    W, S, B = synth.int8_matrix(0, "c1/router", E, D)
    for t in range(2):
        _decode_token(ctx, stream, W, S, B, synth.f16_vector(0, f"c1/h{t}", D), E, D, F, K, 0, "c1/experts")


def test_decode_token_all_logits_equal(ctx, stream):
    # every router row identical: 128 equal logits across all router blocks
    E, D, F, K = 128, 512, 128, 8
    W, S, B = synth.int8_matrix(11, "tie/router", E, D)
    W[:], S[:], B[:] = W[0], S[0], B[0]
    got = _decode_token(ctx, stream, W, S, B, synth.f16_vector(11, "tie/h", D), E, D, F, K, 11, "tie/experts")
    assert got == list(range(K))


def test_decode_token_ties_across_router_blocks(ctx, stream):
    # copies of the best row in several router blocks (16 rows per block at
    # d = 512): the equal logits must come out in expert-index order
    E, D, F, K = 128, 512, 128, 8
    W, S, B = synth.int8_matrix(12, "tie2/router", E, D)
    h16 = synth.f16_vector(12, "tie2/h", D)
    best = int(np.argmax(oracle.router_logits(W, S, B, from_f16_bits(h16))))
    for e in (100, 3, 50, 19, 120, 64):
        W[e], S[e], B[e] = W[best], S[best], B[best]
    got = _decode_token(ctx, stream, W, S, B, h16, E, D, F, K, 12, "tie2/experts")
    tied = sorted({best, 100, 3, 50, 19, 120, 64})
    assert got[:len(tied)] == tied


@pytest.mark.parametrize("E,D,K", [(100, 256, 6), (40, 2816, 8), (256, 1024, 8)])
def test_decode_token_odd_shapes(ctx, stream, E, D, K):
    F = 128
    W, S, B = synth.int8_matrix(13, f"odd/router{E}", E, D)
    gain16 = f16_bits(synth.uniform24(synth.seed_key(13, f"odd/gain{E}"), E, 0.5, 1.5))
    _decode_token(ctx, stream, W, S, B, synth.f16_vector(13, f"odd/h{E}", D), E, D, F, K, 13,
                  f"odd/experts{E}", gain16)
