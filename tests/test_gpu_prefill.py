"""GPU parity of the prefill dequant-fused GEMM (MFMA) against the CPU oracle.

Mirrors T/Kernels/TensorCore/MPPPrefillInt4QMMTests.swift and
T/Kernels/Prefill/PrefillAffineTests.swift (reference checkout). Tolerance:
max relative error (RelError.compute) <= 1e-3 against the fp32 oracle for
fp16 outputs; for bf16 outputs the one final rounding to bf16 is allowed on
top, exactly half a bf16 ulp of the value (bf16 keeps 8 significant bits, so
half an ulp is between 2^-9 and 2^-8 of |v|):
|y - ref| <= 1e-3 * max|ref| + halfulp_bf16(max(|ref|, |y|)).
"""
import numpy as np
import pytest

import oracle
from edgeexpert_amd import ops, synth
from edgeexpert_amd._lib import DTYPE_BF16, DTYPE_F16, TFQ_E_INVAL, TfqError
from edgeexpert_amd.runtime import DeviceBuffer
from helpers import bf16_half_ulp, from_f16_bits

pytestmark = pytest.mark.gpu
TOL = oracle.Tolerance.north_star


def _dev(a):
    return DeviceBuffer.from_array(np.ascontiguousarray(a))


def _run(ctx, stream, W, S, B, xbits, t, n, k, dtype):
    y = _dev(np.full(t * n, 0x7FC0 if dtype == DTYPE_BF16 else 0x7E00, np.uint16))
    ops.PrefillInt4QMM(ctx).encode(stream, _dev(W), _dev(S), _dev(B), _dev(xbits), y, t, n, k, dtype)
    stream.sync()
    bits = y.download(np.uint16, t * n)
    out = synth.bf16_to_f32(bits) if dtype == DTYPE_BF16 else from_f16_bits(bits)
    return out.reshape(t, n)


def _check(y, ref, dtype):
    if dtype == DTYPE_F16:
        rel = oracle.rel_error(y, ref)
        assert rel < TOL, f"rel={rel}"
    else:
        bound = TOL * np.abs(ref).max() + bf16_half_ulp(np.maximum(np.abs(ref), np.abs(y)))
        assert np.all(np.abs(y - ref) <= bound), f"max excess {np.max(np.abs(y - ref) - bound)}"


def _mpp_inputs(t, n, k, adversarial=False):
    # MPPPrefillInt4QMMTests.makeInputs (MPPPrefillInt4QMMTests.swift:20-62)
    groups = k // 64
    idx = np.arange(n * k // 2, dtype=np.int64)
    packed = ((idx * 37 + 0x29) & 0xFF).astype(np.uint8).reshape(n, k // 2)
    r = np.arange(n)[:, None]
    g = np.arange(groups)[None, :]
    if adversarial:
        sv = np.array([oracle.f32_to_bf16(0.001), oracle.f32_to_bf16(-0.0015), 0x0001, 0x8001], np.uint16)
        bv = np.array([oracle.f32_to_bf16(-0.01), oracle.f32_to_bf16(0.006), 0x0001, 0x8001], np.uint16)
        S = sv[(r + g) % 4]
        B = bv[(r * 3 + g) % 4]
    else:
        S = synth.bf16_bits(0.001 + ((r + g) % 5) * 0.00025 + 0 * g)
        B = synth.bf16_bits(-0.01 + ((r * 3 + g) % 7) * 0.002 + 0 * g)
    x = (((np.arange(t * k) * 11) % 29 - 14) / 64.0).astype(np.float16).reshape(t, k)
    # BF16 scale words become fp16 words (the adversarial subnormals flush to 0 in fp16)
    S16 = synth.bf16_to_f32(S).astype(np.float16).view(np.uint16)
    B16 = synth.bf16_to_f32(B).astype(np.float16).view(np.uint16)
    return packed, S16, B16, x


@pytest.mark.parametrize("t,n,k,adv", [(64, 32, 64, False), (64, 32, 128, True), (17, 35, 64, False),
                                       (17, 35, 128, True)])
@pytest.mark.parametrize("dtype", [DTYPE_F16, DTYPE_BF16])
def test_qmm_matches_fp32_affine_reference(ctx, stream, t, n, k, adv, dtype):
    # MPPPrefillInt4QMMTests.swift:85-104 (the reference's bound: <= 0.03 abs and <= 1e-3 rel)
    W, S, B, x = _mpp_inputs(t, n, k, adv)
    xbits = x.view(np.uint16) if dtype == DTYPE_F16 else synth.bf16_bits(x.astype(np.float32))
    xin = x.astype(np.float32) if dtype == DTYPE_F16 else synth.bf16_to_f32(xbits)
    y = _run(ctx, stream, W, S, B, xbits, t, n, k, dtype)
    ref = oracle.gemm_int4(W, S, B, xin.reshape(t, k))
    assert np.max(np.abs(y - ref)) <= 0.03
    _check(y, ref, dtype)


@pytest.mark.parametrize("t,n,k", [(1, 64, 64), (2, 129, 128), (3, 65, 192), (7, 256, 128), (32, 64, 64),
                                   (1, 4096, 2816), (2, 2048, 2816), (2, 8192, 2816), (2, 2816, 8192),
                                   (129, 704, 2816), (33, 2112, 2816), (200, 2816, 2112)])
def test_qmm_matches_repeated_gemv_and_oracle(ctx, stream, t, n, k):
    # PrefillAffineTests.swift:176-209: QMM == repeated GEMV within 1e-3
    W, S, B = synth.int4_matrix(5, f"qmm/{t}x{n}x{k}", n, k)
    x16 = synth.f16_vector(5, f"qmm/x{t}x{k}", t * k).reshape(t, k)
    y = _run(ctx, stream, W, S, B, x16, t, n, k, DTYPE_F16)
    xf = from_f16_bits(x16)
    gemv = ops.DequantInt4GEMV(ctx)
    wb, sb, bb = _dev(W), _dev(S), _dev(B)
    for tok in range(min(t, 3)):
        yv = _dev(np.zeros(n, np.uint16))
        gemv.encode(stream, wb, sb, bb, _dev(x16[tok]), yv, n, k)
        stream.sync()
        rel = oracle.rel_error(y[tok], from_f16_bits(yv.download(np.uint16, n)))
        assert rel < TOL, f"token {tok}: QMM vs GEMV rel={rel}"
    rows = (0, min(t, 8))
    ref = oracle.gemm_int4(W, S, B, xf, rows=rows)
    rel = oracle.rel_error(y[rows[0]:rows[1]], ref[rows[0]:rows[1]])
    assert rel < TOL, f"rel={rel}"


def test_qmm_baseline_config2_bf16(ctx, stream):
    # X[512, 2816] bf16 ~ N(0,1), W[8192, 2816] int4 g64, Y bf16.
    # The fp32 oracle is evaluated on token rows in every 64-token tile: both
    # edges of each tile (rows 64i and 64i+63, the two 32-row MFMA sub-tiles'
    # outer rows) and one row inside each 32-row sub-tile, all 8192 outputs.
    t, n, k = 512, 8192, 2816
    W, S, B = synth.int4_matrix(0, "c2/w", n, k)
    xb = synth.bf16_vector(0, "c2/x", t * k).reshape(t, k)
    y = _run(ctx, stream, W, S, B, xb, t, n, k, DTYPE_BF16)
    xf = synth.bf16_to_f32(xb)
    rows = sorted({r for i in range(t // 64) for r in (64 * i, 64 * i + 13, 64 * i + 45, 64 * i + 63)})
    for r in rows:
        ref = oracle.gemm_int4(W, S, B, xf, rows=(r, r + 1))
        _check(y[r:r + 1], ref[r:r + 1], DTYPE_BF16)


def test_qmm_is_byte_stable_across_dispatches(ctx, stream):
    # MPPPrefillInt4QMMTests.swift:131-181 (32 dispatches, identical bytes)
    t, n, k = 64, 2048, 2816
    W, S, B, x = _mpp_inputs(t, n, k)
    bufs = [_dev(a) for a in (W, S, B, x.view(np.uint16))]
    outs = [_dev(np.zeros(t * n, np.uint16)) for _ in range(8)]
    q = ops.PrefillInt4QMM(ctx)
    for rep in range(32):
        q.encode(stream, *bufs, outs[rep % 8], t, n, k, DTYPE_F16)
    stream.sync()
    first = outs[0].download(np.uint16)
    for o in outs[1:]:
        assert np.array_equal(o.download(np.uint16), first)


def test_qmm_rejects_bad_contract(ctx, stream):
    b = _dev(np.zeros(1 << 16, np.uint8))
    q = ops.PrefillInt4QMM(ctx)
    for args in [(4, 64, 100, DTYPE_F16), (0, 64, 64, DTYPE_F16), (4, 64, 64, 7)]:
        with pytest.raises(TfqError) as ei:
            q.encode(stream, b, b, b, b, b, *args)
        assert ei.value.status == TFQ_E_INVAL
