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
from edgeexpert_amd._lib import ROUTER_WORKSPACE_BYTES, TfqError, TFQ_E_INVAL, TFQ_E_UNSUPPORTED
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


@pytest.mark.parametrize("m,n", [(64, 64), (65, 128), (129, 320), (1024, 2816), (512, 4096), (96, 8192),
                                 (2048, 2816)])
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


def test_qkv_b3(ctx, stream):
    mq, mkv, n = 2048, 512, 2816
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
        assert oracle.rel_error(got, ref) < TOL, k


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
    # the grouped prefill kernels are 4-bit only
    ws_bytes = ops.moe_prefill_workspace_bytes(4, K, E, D, F)
    Wr, Sr, Br = synth.int8_matrix(3, "chk/router", E, D)
    router = ops.Router(_dev(Wr), _dev(Sr), _dev(Br), E)
    with pytest.raises(TfqError) as e:
        ops.moe_prefill(ctx, stream, router, pool, _dev(np.zeros(4 * D, np.uint16)), D, 4, D, F, K,
                        _dev(np.zeros(4 * D, np.uint16)), _dev(np.zeros(4 * K, np.uint32)),
                        _dev(np.zeros(4 * K, np.uint16)), DeviceBuffer(ws_bytes), ws_bytes)
    assert e.value.status == TFQ_E_UNSUPPORTED
