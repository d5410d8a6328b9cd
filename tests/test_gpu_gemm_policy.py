"""GPU parity of the prefill GEMM's kernel choice by token count (the role of
PrefillProjectionDispatchPolicy, S/Runtime/Inference/RealForwardRunner.swift:
217-230, 1411-1492): the few-token weight stream (gemm_skinny.hpp) and the
64-token MFMA tile (gemm.hpp) against the CPU oracle
(MPPPrefillInt4QMMTests.cpuReference) and against each other, through the
C ABI (tfq_gemm_q4g64 / tfq_gemm_qg64 choose; tfq_gemm_qg64_path forces).

Bar: RelError <= 1e-3 against the fp32 oracle for fp16 outputs; bf16 outputs
may add one final rounding (half a bf16 ulp of the value). The two kernels
multiply the same fp16 weights, so they agree far inside the bar.
"""
import numpy as np
import pytest

import oracle
from edgeexpert_amd import ops, synth
from edgeexpert_amd._lib import (DTYPE_BF16, DTYPE_F16, GEMM_PATH_GEMV, GEMM_PATH_SKINNY, GEMM_PATH_SKINNY32,
                                 GEMM_PATH_TILE)
from edgeexpert_amd.runtime import DeviceBuffer
from helpers import bf16_half_ulp, from_f16_bits

pytestmark = pytest.mark.gpu
TOL = oracle.Tolerance.north_star
PATHS = {"skinny": GEMM_PATH_SKINNY, "skinny32": GEMM_PATH_SKINNY32, "tile": GEMM_PATH_TILE,
         "gemv": GEMM_PATH_GEMV}


def _dev(a):
    return DeviceBuffer.from_array(np.ascontiguousarray(a))


def _gemm(ctx, stream, bufs, t, n, k, dtype, bits=4, path=None):
    W, S, B, X = bufs
    y = _dev(np.full(t * n, 0x7FC0 if dtype == DTYPE_BF16 else 0x7E00, np.uint16))
    ops.PrefillInt4QMM(ctx).encode(stream, W, S, B, X, y, t, n, k, dtype, bits=bits, path=path)
    stream.sync()
    out = y.download(np.uint16, t * n)
    return (synth.bf16_to_f32(out) if dtype == DTYPE_BF16 else from_f16_bits(out)).reshape(t, n)


def _check(y, ref, dtype, label):
    if dtype == DTYPE_F16:
        rel = oracle.rel_error(y, ref)
        assert rel < TOL, f"{label}: rel={rel}"
    else:
        bound = TOL * np.abs(ref).max() + bf16_half_ulp(np.maximum(np.abs(ref), np.abs(y)))
        assert np.all(np.abs(y - ref) <= bound), f"{label}: max excess {np.max(np.abs(y - ref) - bound)}"


M_SWEEP = [1, 2, 3, 4, 5, 7, 8, 9, 15, 16, 17, 24, 31, 32, 33, 47, 48, 63, 64, 65, 66, 96, 129]


@pytest.mark.parametrize("n", [2048, 8192])
def test_auto_path_over_token_counts(ctx, stream, n):
    # M = 1 ... past the crossover on both sides, every output row of every token
    k = 2816
    W, S, B = synth.int4_matrix(21, f"policy/w{n}", n, k)
    X = synth.f16_vector(21, "policy/x", max(M_SWEEP) * k).reshape(-1, k)
    bufs = (_dev(W), _dev(S), _dev(B), _dev(X))
    ref_all = oracle.gemm_int4(W, S, B, from_f16_bits(X))
    for t in M_SWEEP:
        print(f"[policy] n={n} m={t}", flush=True)
        y = _gemm(ctx, stream, bufs, t, n, k, DTYPE_F16)
        _check(y, ref_all[:t], DTYPE_F16, f"n={n} m={t}")


@pytest.mark.parametrize("n", [2048, 2816, 4096, 8192])
@pytest.mark.parametrize("t", [1, 16, 33])
def test_forced_paths_agree(ctx, stream, n, t):
    k = 2816
    W, S, B = synth.int4_matrix(22, f"paths/w{n}", n, k)
    X = synth.bf16_vector(22, f"paths/x{t}", t * k).reshape(t, k)
    bufs = (_dev(W), _dev(S), _dev(B), _dev(X))
    rows = (0, min(t, 4))
    ref = oracle.gemm_int4(W, S, B, synth.bf16_to_f32(X), rows=rows)
    outs = {}
    for name, path in PATHS.items():
        outs[name] = _gemm(ctx, stream, bufs, t, n, k, DTYPE_BF16, path=path)
        _check(outs[name][rows[0]:rows[1]], ref[rows[0]:rows[1]], DTYPE_BF16, f"{name} n={n} t={t}")
    # the paths multiply the same fp16 weights and differ by fp32 summation
    # order only: at most one bf16 ulp apart after the final rounding, plus
    # the order difference itself where a sum cancels to near zero (fp32
    # rounding of ~K terms of the row's magnitude: 1e-4 of the largest output)
    for a, b in (("skinny", "tile"), ("skinny32", "skinny")):
        ulp = 2 * bf16_half_ulp(np.maximum(np.abs(outs[a]), np.abs(outs[b])))
        slack = 1e-4 * np.abs(outs[b]).max()
        assert np.all(np.abs(outs[a] - outs[b]) <= ulp + slack), f"{a} vs {b}: more than one bf16 ulp apart"


@pytest.mark.parametrize("t,n,k", [(1, 100, 64), (3, 17, 704), (5, 300, 2112), (16, 64, 128), (20, 2816, 4096),
                                   (2, 96, 8192), (7, 33, 1088)])
@pytest.mark.parametrize("path", ["skinny", "skinny32", "gemv"])
def test_skinny_ragged_shapes(ctx, stream, t, n, k, path):
    # half-filled last 128-code tiles (k % 128 == 64), row counts off the
    # 16/32-row tiles, token counts off the 16-token tile, every tile count 1..8
    W, S, B = synth.int4_matrix(23, f"ragged/{t}x{n}x{k}", n, k)
    X = synth.f16_vector(23, f"ragged/x{t}x{k}", t * k).reshape(t, k)
    y = _gemm(ctx, stream, (_dev(W), _dev(S), _dev(B), _dev(X)), t, n, k, DTYPE_F16, path=PATHS[path])
    _check(y, oracle.gemm_int4(W, S, B, from_f16_bits(X)), DTYPE_F16, f"{path} {t}x{n}x{k}")


@pytest.mark.parametrize("t", [1, 9, 40])
def test_skinny_3bit(ctx, stream, t):
    n, k = 2048, 2816
    W, S, B = synth.affine_matrix(24, "skinny3/w", n, k, 3)
    X = synth.f16_vector(24, f"skinny3/x{t}", t * k).reshape(t, k)
    bufs = (_dev(W), _dev(S), _dev(B), _dev(X))
    ref = oracle.gemm_int4(W, S, B, from_f16_bits(X), bits=3)
    for path in (None, GEMM_PATH_SKINNY, GEMM_PATH_TILE, GEMM_PATH_GEMV):
        y = _gemm(ctx, stream, bufs, t, n, k, DTYPE_F16, bits=3, path=path)
        _check(y, ref, DTYPE_F16, f"3-bit t={t} path={path}")


def test_skinny_is_byte_stable_across_dispatches(ctx, stream):
    t, n, k = 12, 4096, 2816
    W, S, B = synth.int4_matrix(25, "stable/w", n, k)
    X = synth.f16_vector(25, "stable/x", t * k)
    bufs = (_dev(W), _dev(S), _dev(B), _dev(X))
    first = _gemm(ctx, stream, bufs, t, n, k, DTYPE_F16, path=GEMM_PATH_SKINNY)
    for _ in range(5):
        again = _gemm(ctx, stream, bufs, t, n, k, DTYPE_F16, path=GEMM_PATH_SKINNY)
        assert np.array_equal(again.view(np.uint32), first.view(np.uint32))


@pytest.mark.parametrize("dtype", [DTYPE_F16, DTYPE_BF16])
def test_gemv_path_equals_decode_gemv(ctx, stream, dtype):
    # the one-token path is the decode GEMV: on fp16 input its output equals
    # tfq_gemv_q4g64's bit for bit; on bf16 input, that of the fp16-converted
    # row, stored as bf16 (both against the oracle too)
    t, n, k = 3, 2048, 2816
    W, S, B = synth.int4_matrix(26, "gemvpath/w", n, k)
    X16 = synth.f16_vector(26, "gemvpath/x", t * k)
    Xb = synth.bf16_vector(26, "gemvpath/xb", t * k)
    Wd, Sd, Bd = _dev(W), _dev(S), _dev(B)
    X = X16 if dtype == DTYPE_F16 else Xb
    y = _gemm(ctx, stream, (Wd, Sd, Bd, _dev(X)), t, n, k, dtype, path=GEMM_PATH_GEMV)
    xf = from_f16_bits(X16) if dtype == DTYPE_F16 else synth.bf16_to_f32(Xb)
    x16 = xf.astype(np.float16).view(np.uint16)
    g = ops.DequantInt4GEMV(ctx)
    yd = _dev(np.zeros(t * n, np.uint16))
    xd = _dev(x16)
    for i in range(t):
        g.encode(stream, Wd, Sd, Bd, xd, yd, n, k, x_offset=2 * i * k, y_offset=2 * i * n)
    stream.sync()
    ref16 = from_f16_bits(yd.download(np.uint16, t * n)).reshape(t, n)
    if dtype == DTYPE_F16:
        assert np.array_equal(y.view(np.uint32), ref16.view(np.uint32))
    else:
        # same fp32 sums rounded to bf16 instead of fp16: within one fp16 ulp + half a bf16 ulp
        bound = np.abs(ref16) * 2.0 ** -11 + bf16_half_ulp(np.maximum(np.abs(ref16), np.abs(y)))
        assert np.all(np.abs(y - ref16) <= bound)
    _check(y, oracle.gemm_int4(W, S, B, xf.reshape(t, k)), dtype, f"gemv path dtype={dtype}")
