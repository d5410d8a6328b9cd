"""GPU parity of the int8 shared expert (tfq_shared_expert_q8) and of the
prefill shared expert over a block of rows (tfq_prefill_shared_expert, int4
and int8), through libtfq's C ABI.

Mirrors T/Kernels/MoE/SharedExpertInt8Tests.swift (reference inputs:
SeedTree(0x601).key("shared-expert-int8"), d 128, f 64) and
T/Kernels/Prefill/PrefillSharedExpertTests.swift (4 rows, x stride 144, y
stride 137, sentinel -7.25 between rows). Bar: RelError <= 1e-3 against the
CPU oracle (the reference's own bound is 4 x Tolerance.quantInt8).
"""
import numpy as np
import pytest

import oracle
from edgeexpert_amd import ops, synth
from edgeexpert_amd._lib import TfqError
from edgeexpert_amd.runtime import DeviceBuffer
from helpers import bf16_to_f16_exact, f16_bits, from_f16_bits

pytestmark = pytest.mark.gpu
TOL = oracle.Tolerance.north_star
SENTINEL = np.float16(-7.25).view(np.uint16)


def _dev(a):
    return DeviceBuffer.from_array(np.ascontiguousarray(a))


def _reference_inputs(seed, label, d, f, bits):
    """The reference test's draw (x, gate, up, down), quantised, BF16 words -> fp16."""
    u = synth.uniform24(synth.seed_key(seed, label), d + 3 * f * d, -0.4, 0.4)
    q = oracle.quantize_int4_matrix if bits == 4 else oracle.quantize_int8_matrix
    conv = lambda m: (m[0], bf16_to_f16_exact(m[1]), bf16_to_f16_exact(m[2]))
    gate = conv(q(u[d:d + f * d].reshape(f, d)))
    up = conv(q(u[d + f * d:d + 2 * f * d].reshape(f, d)))
    down = conv(q(u[d + 2 * f * d:].reshape(d, f)))
    return u[:d], gate, up, down


def _synthetic(seed, label, d, f, bits):
    mat = synth.int4_matrix if bits == 4 else synth.int8_matrix
    return (mat(seed, label + "/gate", f, d), mat(seed, label + "/up", f, d), mat(seed, label + "/down", d, f))


def _proj(m, rows, cols):
    return ops.Q4Projection(_dev(m[0]), _dev(m[1]), _dev(m[2]), rows=rows, cols=cols)


@pytest.mark.parametrize("d,f,seed,label", [(128, 64, 0x601, "shared-expert-int8"),
                                            (2816, 2112, 0, "c4/shared8")])
def test_shared_expert_int8_matches_reference(ctx, stream, d, f, seed, label):
    print(f"[shared8] d={d} f={f}", flush=True)
    if d == 128:
        x, gate, up, down = _reference_inputs(seed, label, d, f, 8)
    else:
        x = synth.normal(synth.seed_key(seed, label + "/x"), d)
        gate, up, down = _synthetic(seed, label, d, f, 8)
    x16 = f16_bits(x)
    y = _dev(np.full(d, 0x7E00, np.uint16))
    act = _dev(np.zeros(f, np.uint16))
    ops.SharedExpertInt8(ctx).encode(stream, _dev(x16), _proj(gate, f, d), _proj(up, f, d), _proj(down, d, f),
                                     y, act)
    stream.sync()
    got = from_f16_bits(y.download(np.uint16, d))
    ref = oracle.shared_expert_int8(gate, up, down, from_f16_bits(x16), d, f)
    rel = oracle.rel_error(got, ref)
    assert rel < TOL, f"rel={rel}"
    # the fused gate/up/act: act = fp16(gelu(g) * u), g and u in fp32
    g = oracle.gemv_int8(*gate, from_f16_bits(x16))
    u = oracle.gemv_int8(*up, from_f16_bits(x16))
    act_ref = np.array([oracle.gelu_tanh(float(v)) for v in g], np.float32) * u
    rel_act = oracle.rel_error(from_f16_bits(act.download(np.uint16, f)), act_ref)
    assert rel_act < TOL, f"act rel={rel_act}"


def test_shared_expert_int8_staging_forms_agree(ctx, stream):
    # a 16-byte aligned x takes the int8 gate/up form whose copy staging is
    # fixed at compile time, a 2-byte aligned x the form that reads the mode:
    # the same bits (act and output)
    d, f = 2816, 2112
    x16 = f16_bits(synth.normal(synth.seed_key(5, "forms8/x"), d))
    gate, up, down = _synthetic(5, "forms8", d, f, 8)
    pg, pu, pd = _proj(gate, f, d), _proj(up, f, d), _proj(down, d, f)
    outs = []
    for off in (0, 2):
        xb = DeviceBuffer(d * 2 + 16)
        xb.upload(x16, offset=off)
        y = _dev(np.full(d, 0x7E00, np.uint16))
        act = _dev(np.zeros(f, np.uint16))
        ops.SharedExpertInt8(ctx).encode(stream, xb.ptr(off), pg, pu, pd, y, act)
        stream.sync()
        outs.append((y.download(np.uint16, d), act.download(np.uint16, f)))
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
    ref = oracle.shared_expert_int8(gate, up, down, from_f16_bits(x16), d, f)
    assert oracle.rel_error(from_f16_bits(outs[0][0]), ref) < TOL


def test_shared_expert_int8_rejects_bad_contract(ctx, stream):
    b = _dev(np.zeros(1 << 16, np.uint8))
    p = ops.Q4Projection(b, b, b, rows=64, cols=100)
    with pytest.raises(TfqError):                # d not a multiple of 64
        ops.SharedExpertInt8(ctx).encode(stream, b, p, p, p, b, b)
    big = ops.Q4Projection(b, b, b, rows=8192, cols=4160)
    with pytest.raises(TfqError):                # d beyond 4096
        ops.SharedExpertInt8(ctx).encode(stream, b, big, big, big, b, b)


def _prefill_case(ctx, stream, bits, rows, d, f, x_stride, y_stride, mats, seed):
    x = synth.f16_vector(seed, f"pshared/x{bits}", rows * x_stride).reshape(rows, x_stride)
    xb = _dev(x)
    y = _dev(np.full(rows * y_stride, SENTINEL, np.uint16))
    ws_bytes = ops.prefill_shared_expert_workspace_bytes(bits, rows, f)
    ws = DeviceBuffer(ws_bytes)
    gate, up, down = mats
    ps = ops.PrefillSharedExpert(ctx, weight_bits=bits)
    ps.encode_block(stream, xb, y, _proj(gate, f, d), _proj(up, f, d), _proj(down, d, f), ws, ws_bytes,
                    rows, d, f, x_stride, y_stride)
    stream.sync()
    out = y.download(np.uint16, rows * y_stride).reshape(rows, y_stride)
    # the padding between rows is untouched
    assert np.all(out[:, d:] == SENTINEL)
    return x, from_f16_bits(out[:, :d])


@pytest.mark.parametrize("bits,xs", [(8, 144), (4, 144), (8, 139)])
def test_prefill_shared_expert_block_matches_rows(ctx, stream, bits, xs):
    # PrefillSharedExpertTests.swift:7-13: 4 rows, d 128, f 64, x stride 144, y stride 137;
    # int8 also at x stride 139 (2-byte aligned rows: the block takes the
    # staging form that reads its mode, the single rows the fixed one)
    rows, d, f, ys = 4, 128, 64, 137
    _, gate, up, down = _reference_inputs(0xC0FFEE + bits, "prefill-shared-expert", d, f, bits)
    x, got = _prefill_case(ctx, stream, bits, rows, d, f, xs, ys, (gate, up, down), 11)
    run = oracle.shared_expert_int8 if bits == 8 else oracle.shared_expert_int4
    single = ops.SharedExpertInt8(ctx) if bits == 8 else ops.SharedExpertInt4(ctx)
    for r in range(rows):
        xr = from_f16_bits(x[r, :d])
        ref = run(gate, up, down, xr, d, f)
        rel = oracle.rel_error(got[r], ref)
        assert rel < TOL, f"row {r}: rel={rel}"
        # the decode form on the same row (PrefillSharedExpertTests: block == repeated scalar rows)
        y1 = _dev(np.zeros(d, np.uint16))
        single.encode(stream, _dev(x[r, :d]), _proj(gate, f, d), _proj(up, f, d), _proj(down, d, f), y1,
                      _dev(np.zeros(f, np.uint16)))
        stream.sync()
        one = from_f16_bits(y1.download(np.uint16, d))
        if bits == 8:
            assert np.array_equal(got[r].view(np.uint32), one.view(np.uint32)), f"row {r}: block != row"
        else:
            # int4 rows run the prefill GEMM (fp16 weight tiles) instead of the GEMV
            assert oracle.rel_error(got[r], one) < TOL, f"row {r}: block vs row"


@pytest.mark.parametrize("bits,rows", [(8, 24), (4, 24), (4, 80)])
def test_prefill_shared_expert_config4_shape(ctx, stream, bits, rows):
    # the C4 shared expert (d 2816, f 2112) over a block of rows; int4 at 24 rows
    # takes the few-token GEMM, at 80 rows the MFMA tile
    d, f = 2816, 2112
    print(f"[pshared] bits={bits} rows={rows}", flush=True)
    mats = _synthetic(3, f"pshared{bits}", d, f, bits)
    x, got = _prefill_case(ctx, stream, bits, rows, d, f, d + 64, d + 8, mats, 12)
    run = oracle.shared_expert_int8 if bits == 8 else oracle.shared_expert_int4
    for r in sorted({0, 1, rows // 2, rows - 1}):
        ref = run(*mats, from_f16_bits(x[r, :d]), d, f)
        rel = oracle.rel_error(got[r], ref)
        assert rel < TOL, f"row {r}: rel={rel}"


def test_prefill_shared_expert_rejects_bad_contract(ctx, stream):
    b = _dev(np.zeros(1 << 16, np.uint8))
    p = ops.Q4Projection(b, b, b, rows=64, cols=128)
    ws = DeviceBuffer(1 << 16)
    with pytest.raises(TfqError):                # weight bits
        ops.PrefillSharedExpert(ctx, weight_bits=3).encode_block(stream, b, b, p, p, p, ws, 1 << 16, 2, 128, 64,
                                                                  128, 128)
    with pytest.raises(TfqError):                # x stride below d
        ops.PrefillSharedExpert(ctx).encode_block(stream, b, b, p, p, p, ws, 1 << 16, 2, 128, 64, 120, 128)
    with pytest.raises(TfqError):                # workspace too small
        ops.PrefillSharedExpert(ctx, weight_bits=4).encode_block(stream, b, b, p, p, p, ws, 64, 2, 128, 64,
                                                                  128, 128)
