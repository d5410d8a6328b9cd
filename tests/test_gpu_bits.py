"""GPU parity of the 2- and 3-bit affine variants (the reference's
TurboFieldfareRebits experts and 3-bit attention rows) against the oracle,
through libtfq's C ABI.

Reference kernels: 3-bit GEMV and fused QKV (S/Metal/Quant/dequant_int4.metal:
512-717, selected by `bits:` in DequantInt4GEMV.swift:140-180 and
FusedQKVGEMV.swift:100-156); 2/3-bit routed experts (S/Metal/MoE/moe.metal:
644-1180, MoE.swift:234-375). The reference has no tests for these paths;
the oracle they are checked against is pinned in test_oracle_bits.py.
Tolerance: RelError <= 1e-3; selections bit-exact.
"""
import numpy as np
import pytest

import oracle
from edgeexpert_amd import ops, synth
from edgeexpert_amd._lib import DTYPE_BF16, DTYPE_F16, ROUTER_WORKSPACE_BYTES, TfqError, TFQ_E_INVAL
from edgeexpert_amd.runtime import DeviceBuffer
from helpers import from_f16_bits

pytestmark = pytest.mark.gpu
TOL = oracle.Tolerance.north_star


def _dev(a):
    return DeviceBuffer.from_array(np.ascontiguousarray(a))


# ------------------------------------------------------------ dense GEMV ----

def _gemv(ctx, stream, W, S, B, x16, m, n, bits):
    y = _dev(np.full(m, 0x7E00, np.uint16))
    ops.DequantInt4GEMV(ctx).encode(stream, _dev(W), _dev(S), _dev(B), _dev(x16), y, m, n, bits=bits)
    stream.sync()
    return from_f16_bits(y.download(np.uint16, m))


# the last two shapes have more rows than one round of resident blocks
# covers (40000 and 30001 rows: every wavefront runs several row groups,
# their count odd for some wavefronts and even for others), which runs the
# 3-bit GEMV's two-groups-in-flight loop and its last odd group
@pytest.mark.parametrize("m,n", [(64, 64), (65, 128), (129, 320), (1024, 2816), (512, 4096), (96, 8192),
                                 (2048, 2816), (40000, 2816), (30001, 512)])
def test_gemv_b3(ctx, stream, m, n):
    W, S, B = synth.affine_matrix(3, f"b3/gemv/{m}x{n}", m, n, 3)
    x16 = synth.f16_vector(3, f"b3/x/{n}", n)
    got = _gemv(ctx, stream, W, S, B, x16, m, n, 3)
    ref = oracle.gemv_affine(W, S, B, from_f16_bits(x16), 3)
    rel = oracle.rel_error(got, ref)
    assert rel < TOL, f"m={m} n={n}: rel={rel}"


def test_gemv_b3_extreme_codes(ctx, stream):
    # every code 0 or 7 in alternating groups, unit scales: exercises the top
    # bit of each 3-bit field and fields straddling the 32-bit words
    m, n = 32, 512
    codes = np.zeros((m, n), np.uint32)
    codes[:, ::2] = 7
    codes[::3, 64:128] = 7
    W = np.stack([oracle.pack_affine_codes(r, 3) for r in codes])
    S = synth.f16_bits(np.full((m, n // 64), 0.5, np.float32))
    B = synth.f16_bits(np.full((m, n // 64), -1.0, np.float32))
    x16 = synth.f16_vector(4, "b3/extreme/x", n)
    got = _gemv(ctx, stream, W, S, B, x16, m, n, 3)
    ref = oracle.gemv_affine(W, S, B, from_f16_bits(x16), 3)
    assert oracle.rel_error(got, ref) < TOL


@pytest.mark.parametrize("mq,mkv", [(2048, 512), (16384, 8192)])
def test_qkv_b3(ctx, stream, mq, mkv):
    n = 2816
    mats = {k: synth.affine_matrix(6, f"b3/qkv/{k}", rows, n, 3) for k, rows in (("q", mq), ("k", mkv), ("v", mkv))}
    x16 = synth.f16_vector(6, "b3/qkv/x", n)
    projs = {k: ops.Q4Projection(_dev(W), _dev(S), _dev(B), W.shape[0], n) for k, (W, S, B) in mats.items()}
    ys = {k: _dev(np.full(W.shape[0], 0x7E00, np.uint16)) for k, (W, _, _) in mats.items()}
    ops.DequantInt4GEMV(ctx).encode_qkv(stream, projs["q"], projs["k"], projs["v"], _dev(x16), ys["q"], ys["k"],
                                        ys["v"], mq, mkv, n, bits=3)
    stream.sync()
    for k, (W, S, B) in mats.items():
        got = from_f16_bits(ys[k].download(np.uint16, W.shape[0]))
        ref = oracle.gemv_affine(W, S, B, from_f16_bits(x16), 3)
        assert oracle.rel_error(got, ref) < TOL, (mq, mkv, k)


@pytest.mark.parametrize("bits", [2, 5, 0])
def test_gemv_rejects_other_widths(ctx, stream, bits):
    # DequantInt4GEMV.swift:149-150: attention weights are 3 or 4 bits
    W, S, B = synth.affine_matrix(1, "b3/bad", 64, 128, 3)
    with pytest.raises(TfqError) as e:
        _gemv(ctx, stream, W, S, B, synth.f16_vector(1, "b3/bad/x", 128), 64, 128, bits)
    assert e.value.status == TFQ_E_INVAL


# ------------------------------------------------------- routed experts ----

def _pool(bits, E, D, F, label, seed=21):
    pool_bytes, offs, stride = synth.expert_pool(seed, label, E, D, F, bits=bits)
    return pool_bytes, ops.ExpertPool(_dev(pool_bytes), stride, E, offs, weight_bits=bits), offs, stride


@pytest.mark.parametrize("bits", [2, 3])
@pytest.mark.parametrize("E,D,F,K", [(16, 2816, 704, 8), (8, 128, 64, 8), (12, 512, 1024, 6), (4, 8192, 64, 2)])
def test_moe_phases(ctx, stream, bits, E, D, F, K):
    pool_bytes, pool, offs, stride = _pool(bits, E, D, F, f"b{bits}/moe/{E}x{D}x{F}")
    rng = np.random.default_rng(bits * 100 + D)
    idx16 = rng.permutation(E).astype(np.uint32)[:K]
    x16 = synth.f16_vector(bits, f"b{bits}/x/{D}", D)
    res16 = synth.f16_vector(bits, f"b{bits}/res/{D}", D, 0.1)
    rw16 = synth.f16_bits(rng.dirichlet(np.ones(K)).astype(np.float32))
    moe = ops.MoE(ctx)
    idx, xb, rw, res = _dev(idx16), _dev(x16), _dev(rw16), _dev(res16)
    acts = _dev(np.full(K * F, 0x7E00, np.uint16))
    split = _dev(np.full(K * F, 0x7E00, np.uint16))
    y, ys = _dev(np.zeros(D, np.uint16)), _dev(np.zeros(D, np.uint16))
    moe.encode_routed_phase1(stream, pool, idx, xb, acts, D, F, K)
    moe.encode_routed_phase2(stream, pool, idx, acts, rw, res, y, D, F, K)
    half = K // 2
    moe.encode_routed_phase1_subset(stream, pool, idx, xb, split, _dev(np.arange(half, dtype=np.uint32)), half,
                                    D, F, K)
    moe.encode_routed_phase1_subset(stream, pool, idx, xb, split, _dev(np.arange(half, K, dtype=np.uint32)),
                                    K - half, D, F, K)
    moe.encode_routed_phase2(stream, pool, idx, split, rw, res, ys, D, F, K)
    stream.sync()
    got = from_f16_bits(y.download(np.uint16, D))
    assert np.array_equal(y.download(np.uint16, D), ys.download(np.uint16, D))
    ref = oracle.moe_routed(pool_bytes, stride, offs, from_f16_bits(x16), idx16, from_f16_bits(rw16), D, F,
                            residual=from_f16_bits(res16), bits=bits)
    rel = oracle.rel_error(got, ref)
    assert rel < TOL, f"bits={bits} D={D} F={F}: rel={rel}"


@pytest.mark.parametrize("bits", [2, 3])
def test_moe_decode_token_baseline_config1(ctx, stream, bits):
    # BASELINE config 1 at 2/3 bits: int8 router [128 x 2816] -> top-8 ->
    # experts of 2/3-bit rows, routing kept on the device (tfq_moe_decode_token)
    E, D, F, K = 128, 2816, 704, 8
    pool_bytes, pool, offs, stride = _pool(bits, E, D, F, f"c1b{bits}/experts", seed=0)
    Wr, Sr, Br = synth.int8_matrix(0, "c1/router", E, D)
    router = ops.Router(_dev(Wr), _dev(Sr), _dev(Br), E)
    ws = DeviceBuffer(ROUTER_WORKSPACE_BYTES)
    for t in range(2):
        h16 = synth.f16_vector(0, f"c1/h{t}", D)
        y = _dev(np.full(D, 0x7E00, np.uint16))
        idx, w16 = _dev(np.full(K, 0xFFFFFFFF, np.uint32)), _dev(np.zeros(K, np.uint16))
        acts = _dev(np.full(K * F, 0x7E00, np.uint16))
        ws.fill(0xFF)
        ops.moe_decode_token(ctx, stream, router, pool, _dev(h16), None, y, D, F, K, idx, w16, acts, ws)
        stream.sync()
        h = from_f16_bits(h16)
        ref_idx, _ = oracle.topk_softmax(oracle.router_logits(Wr, Sr, Br, h), K)
        assert list(idx.download(np.uint32, K)) == list(ref_idx)
        w_dev = from_f16_bits(w16.download(np.uint16, K))
        ref = oracle.moe_routed(pool_bytes, stride, offs, h, ref_idx, w_dev, D, F, bits=bits)
        rel = oracle.rel_error(from_f16_bits(y.download(np.uint16, D)), ref)
        assert rel < TOL, f"bits={bits} token {t}: rel={rel}"


@pytest.mark.parametrize("bits", [2, 3])
def test_moe_bad_expert_index_poisons(ctx, stream, bits):
    E, D, F, K = 4, 256, 128, 2
    _, pool, _, _ = _pool(bits, E, D, F, f"b{bits}/nan")
    acts = _dev(np.zeros(K * F, np.uint16))
    ops.MoE(ctx).encode_routed_phase1(stream, pool, _dev(np.array([1, E + 3], np.uint32)),
                                      _dev(synth.f16_vector(2, "nan/x", D)), acts, D, F, K)
    stream.sync()
    a = from_f16_bits(acts.download(np.uint16, K * F)).reshape(K, F)
    assert np.isfinite(a[0]).all() and np.isnan(a[1]).all()


def test_pool_width_checks(ctx, stream):
    E, D, F, K = 4, 256, 128, 2
    pool_bytes, pool, offs, stride = _pool(3, E, D, F, "b3/checks")
    moe = ops.MoE(ctx)
    x, acts = _dev(synth.f16_vector(2, "chk/x", D)), _dev(np.zeros(K * F, np.uint16))
    idx = _dev(np.arange(K, dtype=np.uint32))
    for bad in (1, 5, 8):
        p = ops.ExpertPool(pool.buffer, stride, E, offs, weight_bits=bad)
        with pytest.raises(TfqError) as e:
            moe.encode_routed_phase1(stream, p, idx, x, acts, D, F, K)
        assert e.value.status == TFQ_E_INVAL
    # a tightly packed 3-bit pool declared 4-bit no longer fits its stride
    _, toffs, tstride = synth.expert_pool(21, "b3/tight", E, D, F, align=256, bits=3)
    small = ops.ExpertPool(pool.buffer, tstride, E, toffs, weight_bits=4)
    with pytest.raises(TfqError) as e:
        moe.encode_routed_phase1(stream, small, idx, x, acts, D, F, K)
    assert e.value.status == TFQ_E_INVAL


# ---------------------------------------------------------------- prefill ----

@pytest.mark.parametrize("t,n,k,dtype", [(1, 64, 64, DTYPE_F16), (37, 300, 320, DTYPE_BF16),
                                         (512, 8192, 2816, DTYPE_BF16), (130, 1024, 8192, DTYPE_F16)])
def test_prefill_gemm_b3(ctx, stream, t, n, k, dtype):
    # PrefillInt4QMM.encode(..., bits: 3) (prefill.metal:711-757); config 2's
    # shape among them, rows checked on a sample of tokens
    W, S, B = synth.affine_matrix(7, f"b3/gemm/{n}x{k}", n, k, 3)
    xf = synth.normal(synth.seed_key(7, f"b3/gemm/x{t}x{k}"), t * k)
    xbits = synth.bf16_bits(xf) if dtype == DTYPE_BF16 else synth.f16_bits(xf)
    xr = (synth.bf16_to_f32(xbits) if dtype == DTYPE_BF16 else from_f16_bits(xbits)).reshape(t, k)
    y = _dev(np.full(t * n, 0x7E00, np.uint16))
    ops.PrefillInt4QMM(ctx).encode(stream, _dev(W), _dev(S), _dev(B), _dev(xbits), y, t, n, k, dtype, bits=3)
    stream.sync()
    yb = y.download(np.uint16).reshape(t, n)
    got = synth.bf16_to_f32(yb) if dtype == DTYPE_BF16 else from_f16_bits(yb)
    rows = (0, t) if t <= 64 else (t - 40, t)
    ref = oracle.gemm_int4(W, S, B, xr, rows=rows, bits=3)[rows[0]:rows[1]]
    got = got[rows[0]:rows[1]]
    if dtype == DTYPE_F16:
        rel = oracle.rel_error(got, ref)
        assert rel < TOL, f"t={t} n={n} k={k}: rel={rel}"
    else:   # bf16 output: the bar plus bf16's own rounding (2^-8 relative), as for the int4 QMM
        bound = TOL * np.abs(ref).max() + 2.0 ** -8 * np.abs(ref)
        assert np.all(np.abs(got - ref) <= bound), f"max excess {np.max(np.abs(got - ref) - bound)}"


def test_prefill_gemm_rejects_other_widths(ctx, stream):
    W, S, B = synth.affine_matrix(7, "b3/gemm/bad", 64, 64, 2)
    with pytest.raises(TfqError) as e:
        ops.PrefillInt4QMM(ctx).encode(stream, _dev(W), _dev(S), _dev(B), _dev(np.zeros(64, np.uint16)),
                                       _dev(np.zeros(64, np.uint16)), 1, 64, 64, DTYPE_F16, bits=2)
    assert e.value.status == TFQ_E_INVAL


@pytest.mark.parametrize("bits", [2, 3])
def test_moe_prefill_end_to_end_bits(ctx, stream, bits):
    # router -> grouping -> grouped 2/3-bit experts -> combine (tfq_moe_prefill;
    # prefill.metal:1304-1450 for the reference's 2/3-bit grouped experts)
    T, k, E, d, f = 96, 8, 32, 512, 256
    pool_bytes, pool, offs, stride = _pool(bits, E, d, f, f"pf{bits}/experts", seed=1)
    Wr, Sr, Br = synth.int8_matrix(1, "pf/router", E, d)
    hidden = synth.f16_vector(1, f"pf{bits}/x", T * d)
    router = ops.Router(_dev(Wr), _dev(Sr), _dev(Br), E)
    wsb = ops.moe_prefill_workspace_bytes(T, k, E, d, f)
    idx, w16 = _dev(np.zeros(T * k, np.uint32)), _dev(np.zeros(T * k, np.uint16))
    h2 = _dev(np.zeros(T * d, np.uint16))
    ops.moe_prefill(ctx, stream, router, pool, _dev(hidden), d, T, d, f, k, h2, idx, w16, DeviceBuffer(wsb), wsb)
    stream.sync()
    got_idx = idx.download(np.uint32).reshape(T, k)
    ref_idx, _ = oracle.prefill_router(Wr, Sr, Br, from_f16_bits(hidden).reshape(T, d), k)
    assert np.array_equal(got_idx, ref_idx)
    w_dev = w16.download(np.uint16)
    pairs = ops.PrefillRouter.make_token_expert_pairs(got_idx, w_dev, T, k)
    grp = oracle.group_pairs(pairs.astype(oracle.PAIR_DTYPE), T, k, E, 16)
    o = oracle.ExpertOffsets(*[int(offs[n]) for n in synth.OFFSET_ORDER])
    ref = oracle.grouped_route_partials(grp["sorted"], hidden, d, pool_bytes, stride, o, k, d, f, T, bits=bits)
    ref_h2 = from_f16_bits(oracle.reduce_token_major(ref, w_dev, T, k, d))
    rel = oracle.rel_error(from_f16_bits(h2.download(np.uint16)), ref_h2)
    assert rel < TOL, f"bits={bits}: rel={rel}"


@pytest.mark.parametrize("bits", [2, 3])
def test_grouped_experts_config3_shape_sampled(ctx, stream, bits):
    # config 3's shape (512 tokens x top-8 of 128 experts, Zipf routing) with
    # 2/3-bit experts: the grouped partials of 8 sampled tokens
    T, k, E, d, f = 512, 8, 128, 2816, 704
    pool_bytes, pool, offs, stride = _pool(bits, E, d, f, f"c3b{bits}/experts", seed=0)
    idx, w16 = synth.zipf_routing(0, "c3/route", T, E, k)
    hidden = synth.f16_vector(0, "c3/x", T * d)
    n, mt = T * k, ops.max_tiles(T, k, E)
    b = {n_: DeviceBuffer(sz) for n_, sz in (("sorted", n * 16), ("offsets", E * 4), ("counts", E * 4),
                                            ("tiles", mt * 16), ("n_tiles", ops.GROUP_STATE_BYTES), ("status", 4))}
    ops.PrefillMoEGrouping(ctx).encode(stream, _dev(idx), _dev(w16), T, k, E, b["sorted"], b["offsets"],
                                       b["counts"], b["tiles"], b["n_tiles"], b["status"])
    act = _dev(np.zeros(n * f, np.uint16))
    parts = _dev(np.zeros(n * d, np.uint16))
    ops.PrefillGroupedRoutedMoE(ctx).encode(stream, pool, b["sorted"], b["tiles"], b["n_tiles"], mt, _dev(hidden),
                                            d, d, f, k, act, parts)
    stream.sync()
    sorted_p = np.frombuffer(b["sorted"].download(np.uint8, n * 16).tobytes(), oracle.PAIR_DTYPE)
    toks = np.array([0, 5, 100, 255, 256, 400, 500, 511])
    sel = sorted_p[np.isin(sorted_p["token"], toks)]
    o = oracle.ExpertOffsets(*[int(offs[n_]) for n_ in synth.OFFSET_ORDER])
    ref = oracle.grouped_route_partials(sel, hidden, d, pool_bytes, stride, o, k, d, f, T, bits=bits)
    gp = from_f16_bits(parts.download(np.uint16)).reshape(T, k, d)
    rp = from_f16_bits(ref).reshape(T, k, d)
    rel = oracle.rel_error(gp[toks], rp[toks])
    assert rel < TOL, f"bits={bits}: rel={rel}"
