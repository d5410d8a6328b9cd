"""Bit-exact checks of the code unpack on the GPU (the north star's
"bit-exact for unpacking"): with a one-hot activation e_j every kernel's
output is a single dequantised weight of column j, so each output word can be
compared with the weight's exact value bit for bit, for every code of every
width at every position.

* GEMV family (decode): y[r] = fp16(fp32(q[r][j]·s + b)) — the GEMV forms
  s·Σq·x + b·Σx in fp32 (q·s is exact in fp32) and rounds once to fp16; the
  reference's DequantInt4GemvRef dequantises to fp32 first, then dots, which
  gives the same word.
* Routed phase 2 (down + weighted sum) with one slot active at weight 1:
  the same word.
* Prefill GEMM (both kernels): Y[j][r] = fp16(q·s + b) rounded once — the
  fp16 weight tile the reference's tensor-op path stages
  (S/Metal/TensorCore/tensorops.metal:57-80) — times 1 accumulated in fp32.

Rows hold every code of their width at many positions (code (7j + 5r) mod
2^bits at column j); scales and biases follow the BASELINE distributions.
Expected words are computed in float64 (exact) and rounded by numpy.
"""
import numpy as np
import pytest

import oracle
from edgeexpert_amd import ops, synth
from edgeexpert_amd._lib import DTYPE_F16, GEMM_PATH_SKINNY, GEMM_PATH_TILE
from edgeexpert_amd.runtime import DeviceBuffer

pytestmark = pytest.mark.gpu
ONE = np.float16(1.0).view(np.uint16)


def _dev(a):
    return DeviceBuffer.from_array(np.ascontiguousarray(a))


def _rows(bits, m, k, seed):
    codes = ((7 * np.arange(k)[None, :] + 5 * np.arange(m)[:, None]) % (1 << bits)).astype(np.uint32)
    if bits == 4:
        W = synth.pack_int4(codes)
    else:
        W = np.stack([oracle.pack_affine_codes(codes[r], bits) for r in range(m)])
    g = m * (k // 64)
    s16 = synth.f16_bits(np.abs(synth.normal(synth.seed_key(seed, f"bx{bits}/s"), g, 0.02)) * (16 >> bits))
    b = -(1 << (bits - 1)) * synth.f16_to_f32(s16) + synth.normal(synth.seed_key(seed, f"bx{bits}/b"), g, 0.002)
    S, B = s16.reshape(m, -1), synth.f16_bits(b).reshape(m, -1)
    # exact q·s + b per (row, column), in float64
    w64 = (codes.astype(np.float64) * np.repeat(synth.f16_to_f32(S).astype(np.float64), 64, axis=1)
           + np.repeat(synth.f16_to_f32(B).astype(np.float64), 64, axis=1))
    return W, S, B, codes, w64


def _identity(k):
    x = np.zeros((k, k), np.uint16)
    x[np.arange(k), np.arange(k)] = ONE
    return x


@pytest.mark.parametrize("bits", [4, 3])
def test_gemv_one_hot_is_bit_exact(ctx, stream, bits):
    # tfq_gemv_q4g64 / tfq_gemv_qg64 (3-bit): every column j of a K = 512 row
    m, k = 64, 512
    W, S, B, codes, w64 = _rows(bits, m, k, 1)
    assert set(np.unique(codes)) == set(range(1 << bits))
    expect = w64.astype(np.float32).astype(np.float16).view(np.uint16)      # fp16(fp32(q·s + b))
    bufs = [_dev(a) for a in (W, S, B)]
    X = _dev(_identity(k))
    Y = _dev(np.zeros(k * m, np.uint16))
    g = ops.DequantInt4GEMV(ctx)
    for j in range(k):
        g.encode(stream, *bufs, X, Y, m, k, x_offset=2 * j * k, y_offset=2 * j * m, bits=bits)
    stream.sync()
    got = Y.download(np.uint16, k * m).reshape(k, m).T
    bad = np.argwhere(got != expect)
    assert bad.size == 0, f"{len(bad)} words differ, first (row, col) {tuple(bad[0])}: " \
                          f"{got[tuple(bad[0])]:#06x} != {expect[tuple(bad[0])]:#06x}"


@pytest.mark.parametrize("bits", [4, 3, 2])
def test_phase2_one_hot_is_bit_exact(ctx, stream, bits):
    # tfq_moe_phase2 over experts of `bits`-bit rows: slot 0 active with weight
    # 1 and a one-hot activation, the other slots weight 0 and zero activations
    E, D, F, K = 4, 64, 128, 8
    offs, stride = synth.expert_layout(D, F, bits=bits)
    pool = np.zeros(E * stride, np.uint8)
    W, S, B, _, w64 = _rows(bits, D, F, 2)
    e = 2
    blob = pool[e * stride:(e + 1) * stride]
    blob[offs["down_w"]:offs["down_w"] + W.size] = W.reshape(-1)
    blob[offs["down_s"]:offs["down_s"] + 2 * S.size] = S.reshape(-1).view(np.uint8)
    blob[offs["down_b"]:offs["down_b"] + 2 * B.size] = B.reshape(-1).view(np.uint8)
    expect = w64.astype(np.float32).astype(np.float16).view(np.uint16)      # [D][F]
    p = ops.ExpertPool(_dev(pool), stride, E, offs, weight_bits=bits)
    idx = _dev(np.array([e, 0, 1, 3, 0, 1, 2, 3], np.uint32))
    rw = np.zeros(K, np.uint16)
    rw[0] = ONE
    rwb = _dev(rw)
    acts = np.zeros((F, K, F), np.uint16)
    acts[np.arange(F), 0, np.arange(F)] = ONE
    ab = _dev(acts)
    Y = _dev(np.zeros(F * D, np.uint16))
    moe = ops.MoE(ctx)
    for j in range(F):
        moe.encode_routed_phase2(stream, p, idx, ab.ptr(j * K * F * 2), rwb, None, Y.ptr(j * D * 2), D, F, K)
    stream.sync()
    got = Y.download(np.uint16, F * D).reshape(F, D).T
    assert np.array_equal(got, expect), f"{np.count_nonzero(got != expect)} words differ"


@pytest.mark.parametrize("bits", [4, 3])
@pytest.mark.parametrize("path", [GEMM_PATH_TILE, GEMM_PATH_SKINNY])
def test_gemm_one_hot_is_bit_exact(ctx, stream, bits, path):
    # the prefill GEMM on the identity: token j reads column j of every row
    m, k = 96, 512
    W, S, B, _, w64 = _rows(bits, m, k, 3)
    expect = w64.astype(np.float16).view(np.uint16).T                      # fp16(q·s + b), one rounding
    Y = _dev(np.zeros(k * m, np.uint16))
    ops.PrefillInt4QMM(ctx).encode(stream, _dev(W), _dev(S), _dev(B), _dev(_identity(k)), Y, k, m, k, DTYPE_F16,
                                   bits=bits, path=path)
    stream.sync()
    got = Y.download(np.uint16, k * m).reshape(k, m)
    assert np.array_equal(got, expect), f"{np.count_nonzero(got != expect)} words differ"


def _affine_rows(codes, bits):
    if bits == 4:
        return synth.pack_int4(codes)
    return np.stack([oracle.pack_affine_codes(codes[r], bits) for r in range(codes.shape[0])])


@pytest.mark.parametrize("bits", [4, 3, 2])
def test_grouped_down_one_hot_is_bit_exact(ctx, stream, bits):
    # tfq_moe_grouped (gate/up then down units). Token t's hidden row is e_t;
    # every gate weight is 16 and up row f is 1/16 at column f only, so the
    # gate/up units give act = fp16(gelu(16)·u) = e_t exactly (gelu(16) = 16:
    # e^(-2z) underflows) and each down partial of a pair of token t is the
    # expert's dequantised down weight of column t: fp16(q·s + b), one
    # rounding. Routing: rank 0 -> expert 0 (128 pairs: two 64-pair halves on
    # wide units), rank 1 -> experts 1..15 (8-9 pairs: stream units), rank 2 ->
    # experts 16..18 (42-43 pairs: one partly filled wide half); expert 19 idle.
    T, k, E, D, F = 128, 3, 20, 256, 128
    offs, stride = synth.expert_layout(D, F, align=256, bits=bits)
    pool = np.zeros(E * stride, np.uint8)
    gq, gs = {4: (8, 2.0), 3: (4, 4.0), 2: (2, 8.0)}[bits]
    gate_codes = np.full((F, D), gq, np.uint32)
    up_codes = np.zeros((F, D), np.uint32)
    up_codes[np.arange(F), np.arange(F)] = 1
    f16 = lambda v, shape: np.full(shape, np.float16(v).view(np.uint16), np.uint16)
    expect = {}
    for e in range(E):
        codes = ((7 * np.arange(F)[None, :] + 5 * np.arange(D)[:, None] + 3 * e) % (1 << bits)).astype(np.uint32)
        g = D * (F // 64)
        s16 = synth.f16_bits(np.abs(synth.normal(synth.seed_key(e, f"gd{bits}/s"), g, 0.02)) * (16 >> bits))
        b = -(1 << (bits - 1)) * synth.f16_to_f32(s16) + synth.normal(synth.seed_key(e, f"gd{bits}/b"), g, 0.002)
        S, B = s16.reshape(D, -1), synth.f16_bits(b).reshape(D, -1)
        w64 = (codes.astype(np.float64) * np.repeat(synth.f16_to_f32(S).astype(np.float64), 64, axis=1)
               + np.repeat(synth.f16_to_f32(B).astype(np.float64), 64, axis=1))
        expect[e] = w64.astype(np.float16).view(np.uint16)                     # [D][F], one rounding
        parts = {"gate_w": _affine_rows(gate_codes, bits), "gate_s": f16(gs, (F, D // 64)),
                 "gate_b": f16(0.0, (F, D // 64)), "up_w": _affine_rows(up_codes, bits),
                 "up_s": f16(0.0625, (F, D // 64)), "up_b": f16(0.0, (F, D // 64)),
                 "down_w": _affine_rows(codes, bits), "down_s": S, "down_b": B}
        for name, arr in parts.items():
            raw = np.ascontiguousarray(arr).view(np.uint8).ravel()
            o = e * stride + offs[name]
            pool[o:o + raw.size] = raw
    t = np.arange(T)
    idx = np.stack([np.zeros(T, np.int64), 1 + t % 15, 16 + t % 3], axis=1).astype(np.uint32)
    w16 = f16(1.0, (T, k))
    hidden = np.zeros((T, D), np.uint16)
    hidden[t, t] = ONE
    got, bufs = _group_on_device(ctx, stream, idx, w16, T, k, E)
    p = ops.ExpertPool(_dev(pool), stride, E, offs, weight_bits=bits)
    act = _dev(np.full(T * k * F, 0x7FFF, np.uint16))
    partials = _dev(np.full(T * k * D, 0x7FFF, np.uint16))
    ops.PrefillGroupedRoutedMoE(ctx).encode(stream, p, bufs["sorted"], bufs["tiles"], bufs["n_tiles"],
                                            ops.max_tiles(T, k, E), _dev(hidden), D, D, F, k, act, partials)
    stream.sync()
    parts = partials.download(np.uint16).reshape(T, k, D)
    for tok in range(T):
        for r in range(k):
            want = expect[int(idx[tok, r])][:, tok]
            bad = np.flatnonzero(parts[tok, r] != want)
            assert bad.size == 0, (f"{bits}-bit token {tok} rank {r} expert {idx[tok, r]}: {bad.size} words differ, "
                                   f"first d={bad[0]}: {parts[tok, r, bad[0]]:#06x} != {want[bad[0]]:#06x}")


def _group_on_device(ctx, stream, idx, w16, T, k, E):
    n = T * k
    mt = ops.max_tiles(T, k, E)
    bufs = dict(sorted=_dev(np.zeros(n, ops.PAIR_DTYPE)), offsets=_dev(np.zeros(E, np.uint32)),
                counts=_dev(np.zeros(E, np.uint32)), tiles=_dev(np.zeros(mt, ops.TILE_DTYPE)),
                n_tiles=_dev(np.zeros(ops.GROUP_STATE_BYTES // 4, np.uint32)), status=_dev(np.zeros(1, np.uint32)))
    ops.PrefillMoEGrouping(ctx).encode(stream, _dev(idx), _dev(w16), T, k, E, bufs["sorted"], bufs["offsets"],
                                       bufs["counts"], bufs["tiles"], bufs["n_tiles"], bufs["status"])
    stream.sync()
    assert int(bufs["status"].download(np.uint32, 1)[0]) == 0
    counts = bufs["counts"].download(np.uint32, E)
    assert counts[0] == T and counts[19] == 0 and set(counts[1:16]) <= {8, 9} and set(counts[16:19]) <= {42, 43}
    return None, bufs
