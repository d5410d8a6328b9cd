"""Pins the CPU oracle (oracle/tfq_oracle.c) before it is trusted as the checker.

Each check is chosen so that a plausible slip in the restatement (wrong
nibble order, dropped bias term, swapped operands, wrong tie rule, wrong
rounding) fails it: published known-answer values, the reference's own
known-answer tests (transcribed), closed forms, independent numpy
recomputation, and float64 brute force.
"""
import math

import numpy as np
import pytest

import oracle
from edgeexpert_amd import synth
from helpers import dequant_int4_np, ref_int4_rows

L = oracle.lib


# ------------------------------------------------------------- PRNG ----

def test_splitmix64_published_vector():
    # SplitMix64 seeded with 0: the generator's published first outputs.
    r = oracle.SplitMix64(0)
    assert [r.next() for _ in range(3)] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4,
                                            0x06C45D188009454F]


def test_seedtree_is_fnv1a64_xor_root():
    # FNV-1a 64 published vectors: "" -> offset basis, "a" -> 0xaf63dc4c8601ec8c.
    assert L().tfo_seedtree_key(0, b"") == 0xCBF29CE484222325
    assert L().tfo_seedtree_key(0, b"a") == 0xAF63DC4C8601EC8C
    assert L().tfo_seedtree_key(0x1234, b"a") == 0xAF63DC4C8601EC8C ^ 0x1234
    assert synth.seed_key(0x1234, "a") == 0xAF63DC4C8601EC8C ^ 0x1234


def test_uniform_is_24bit_and_host_generator_agrees():
    key = synth.seed_key(0xC1, "int4-gemv-kernel-m128-n128")
    r = oracle.SplitMix64(key)
    raw = oracle.SplitMix64(key)
    for _ in range(100):
        u = r.uniform(0.0, 1.0)
        assert u == (raw.next() >> 40) / float(1 << 24)
    r = oracle.SplitMix64(key)
    assert np.array_equal(r.uniforms(4096, -0.5, 0.5), synth.uniform24(key, 4096, -0.5, 0.5))


# ------------------------------------------------------ conversions ----

@pytest.mark.parametrize("value,bits", [
    (1.0, 0x3F80), (-1.0, 0xBF80), (0.5, 0x3F00), (1.0 / 3.0, 0x3EAB), (12345.0, 0x4641),
    (0.0, 0x0000),
])
def test_bf16_known_values(value, bits):
    assert oracle.f32_to_bf16(value) == bits


def test_bf16_round_half_even():
    f = lambda u: np.array([u], np.uint32).view(np.float32)[0]
    assert oracle.f32_to_bf16(f(0x3F808000)) == 0x3F80     # tie, even stays
    assert oracle.f32_to_bf16(f(0x3F818000)) == 0x3F82     # tie, odd rounds up
    assert oracle.f32_to_bf16(f(0x3F808001)) == 0x3F81


def test_f16_matches_ieee_numpy():
    rng = np.random.RandomState(7)
    xs = np.concatenate([rng.randn(20000) * 1000, rng.randn(20000) * 1e-5, rng.randn(2000) * 7e4,
                         [65504, 65519.99, 65520, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, -0.0]])
    xs = xs.astype(np.float32)
    got = np.array([oracle.f32_to_f16(float(v)) for v in xs], np.uint16)
    with np.errstate(over="ignore"):
        assert np.array_equal(got, xs.astype(np.float16).view(np.uint16))
    bits = np.arange(0, 65536, 97, dtype=np.uint16)
    back = np.array([oracle.f16_to_f32(int(b)) for b in bits], np.float32)
    ref = bits.view(np.float16).astype(np.float32)
    ok = ~np.isnan(ref)
    assert np.array_equal(back[ok].view(np.uint32), ref[ok].view(np.uint32))


# ------------------------------------------------------------ format ----

def test_int4_code_layout_brute_force():
    # every byte value: element 2k = low nibble, 2k+1 = high nibble
    row = np.arange(256, dtype=np.uint8)
    for j in range(512):
        b = int(row[j // 2])
        assert oracle.int4_code(row, j) == ((b >> 4) if j & 1 else (b & 0xF))
    # the same bits read as 8 nibbles per little-endian u32 word
    words = row.view("<u4")
    for j in range(0, 512, 37):
        assert oracle.int4_code(row, j) == (int(words[j // 8]) >> (4 * (j % 8))) & 0xF


def test_nibble_layout_low_even_high_odd():
    # T/Infrastructure/ModelIO/QuantizationTests.swift:35-50
    row = np.arange(64, dtype=np.float32) - 31.5
    p, s, b = oracle.quantize_int4_row(row)
    scale, bias = oracle.bf16_to_f32(int(s[0])), oracle.bf16_to_f32(int(b[0]))
    lo, hi = int(p[0]) & 0xF, int(p[0]) >> 4
    assert abs(lo * scale + bias - row[0]) <= scale + 1e-3
    assert abs(hi * scale + bias - row[1]) <= scale + 1e-3


def test_int4_round_trip_bound():
    # QuantizationTests.swift:8-33 (bound amax/7 + 1e-3) and
    # DequantInt4GEMVReferenceTests.swift:55-76 (bound scale + 1e-4)
    key = synth.seed_key(0x51A71001, "int4-affine-round-trip")
    row = synth.uniform24(key, 256, -1.0, 1.0)
    p, s, b = oracle.quantize_int4_row(row)
    rec = oracle.dequantize_int4_row(p, s, b, oracle.FMT_BF16, 256)
    for g in range(4):
        seg = slice(64 * g, 64 * g + 64)
        amax = np.abs(row[seg]).max()
        assert np.all(np.abs(rec[seg] - row[seg]) <= amax / 7.0 + 1e-3)
        assert np.all(np.abs(rec[seg] - row[seg]) <= oracle.bf16_to_f32(int(s[g])) + 1e-4)


def test_quantization_affine_known_answers():
    # T/Infrastructure/ModelIO/QuantizationAffineTests.swift:7-88
    row = np.array([0.10 + k * 0.01 for k in range(64)] + [-0.50 - k * 0.005 for k in range(64)],
                   np.float32)
    p, s, b = oracle.quantize_int4_row(row)
    assert p.size == 64 and s.size == 2 and b.size == 2
    rec = oracle.dequantize_int4_row(p, s, b, oracle.FMT_BF16, 128)
    assert np.all(np.abs(rec - row) < 0.025)

    row8 = np.array([-0.3 + k * 0.02 for k in range(64)], np.float32)
    p8, s8, b8 = oracle.quantize_int8_row(row8)
    rec8 = oracle.dequantize_int8_row(p8, s8, b8, oracle.FMT_BF16, 64)
    assert np.all(np.abs(rec8 - row8) < 0.008)

    const = np.full(64, 0.42, np.float32)
    pc, sc, bc = oracle.quantize_int4_row(const)
    recc = oracle.dequantize_int4_row(pc, sc, bc, oracle.FMT_BF16, 64)
    assert np.all(np.abs(recc - oracle.bf16_to_f32(oracle.f32_to_bf16(0.42))) < 1e-6)
    assert oracle.bf16_to_f32(int(sc[0])) == 1.0

    pos = (np.arange(64, dtype=np.float32) / 63.0 + 1.0).astype(np.float32)
    pp, _, _ = oracle.quantize_int4_row(pos)
    codes = synth.unpack_int4(pp)
    assert codes.min() == 0 and codes.max() == 15


def test_dequantize_matches_numpy_bit_exact():
    W, S, B, _ = ref_int4_rows(3, "deq", 16, 512, -1.0, 1.0)
    ref = dequant_int4_np(W, S, B, oracle.FMT_BF16)
    for r in range(16):
        got = oracle.dequantize_int4_row(W[r], S[r], B[r], oracle.FMT_BF16, 512)
        assert np.array_equal(got, ref[r])
    # fp16 scale words decode differently from BF16 words (the format switch is live)
    f16 = oracle.dequantize_int4_row(W[0], S[0], B[0], oracle.FMT_F16, 512)
    assert not np.array_equal(f16, ref[0])


# -------------------------------------------------------------- GEMV ----

@pytest.mark.parametrize("m,n,seed", [(4, 128, 0xF1), (8, 256, 0xF2), (16, 512, 0xF3), (32, 2816, 0xF4)])
def test_gemv_int4_vs_float64_and_numpy(m, n, seed):
    # DequantInt4GEMVReferenceTests.swift:38-53: the fp32 path within 1e-5 of an
    # independent computation.
    W, S, B, x = ref_int4_rows(seed, f"int4-gemv-ref-m{m}-n{n}", m, n, -1.0, 1.0, extra=n)
    y = oracle.gemv_int4(W, S, B, x, oracle.FMT_BF16)
    y64 = oracle.gemv_int4_f64(W, S, B, x, oracle.FMT_BF16)
    ynp = dequant_int4_np(W, S, B, oracle.FMT_BF16).astype(np.float64) @ x.astype(np.float64)
    assert oracle.rel_error(y, ynp) < oracle.Tolerance.identity
    assert np.allclose(y64, ynp, rtol=0, atol=1e-9 * max(1.0, np.abs(ynp).max()))
    # a transposed / mis-ordered unpack must be caught by this comparison
    Wswap = ((W >> 4) | (W << 4)).astype(np.uint8)
    bad = oracle.gemv_int4(Wswap, S, B, x, oracle.FMT_BF16)
    assert oracle.rel_error(bad, ynp) > 1e-2


def test_gemv_int4_multithreaded_matches_serial():
    W, S, B, x = ref_int4_rows(9, "mt", 100, 704, -1.0, 1.0, extra=704)
    assert np.array_equal(oracle.gemv_int4(W, S, B, x), oracle.gemv_int4_mt(W, S, B, x, threads=7))


def test_gemv_int8_vs_numpy():
    key = synth.seed_key(0x151, "int8-gemv-m128-n2816")
    u = synth.uniform24(key, 128 * 2816 + 2816, -1.0, 1.0)
    W, S, B = oracle.quantize_int8_matrix(u[:128 * 2816].reshape(128, 2816))
    x = u[128 * 2816:]
    y = oracle.gemv_int8(W, S, B, x, oracle.FMT_BF16)
    deq = (W.astype(np.float32) * np.repeat(synth.bf16_to_f32(S), 64, axis=1)
           + np.repeat(synth.bf16_to_f32(B), 64, axis=1)).astype(np.float32)
    ynp = deq.astype(np.float64) @ x.astype(np.float64)
    assert oracle.rel_error(y, ynp) < oracle.Tolerance.identity
    assert np.allclose(oracle.gemv_int8_f64(W, S, B, x, oracle.FMT_BF16), ynp, rtol=1e-12, atol=1e-9)


def test_gemv_closed_form_constant_codes():
    # all codes q, scale s, bias b: y = Σ (q s + b) x = (q s + b) Σ x exactly for small ints
    n = 256
    W = np.full((2, n // 2), 0x77, np.uint8)         # q = 7 everywhere
    S = np.full((2, n // 64), np.float16(0.5).view(np.uint16), np.uint16)
    B = np.full((2, n // 64), np.float16(-1.0).view(np.uint16), np.uint16)
    x = np.arange(n, dtype=np.float32) % 5
    y = oracle.gemv_int4(W, S, B, x)
    assert np.all(y == np.float32(2.5 * x.sum()))


# ------------------------------------------------------ router/top-k ----

def _topk_brute(logits, k):
    order = np.lexsort((np.arange(logits.size), -logits.astype(np.float64)))
    return order[:k]


def test_topk_matches_sort_brute_force_with_ties():
    rng = np.random.RandomState(11)
    for trial in range(50):
        E = rng.choice([16, 128, 256])
        logits = np.round(rng.randn(E) * 2, 1).astype(np.float32)   # many exact ties
        k = int(rng.choice([1, 8, 16]))
        idx, w = oracle.topk_softmax(logits, k)
        assert list(idx) == list(_topk_brute(logits, k))
        sel = logits[idx].astype(np.float64)
        ref = np.exp(sel - sel.max())
        ref /= ref.sum()
        assert np.allclose(w, ref, rtol=1e-6, atol=1e-7)
        assert abs(w.sum() - 1.0) < 1e-5


def test_topk_equal_logits_gives_lowest_indices_and_uniform_weights():
    idx, w = oracle.topk_softmax(np.zeros(32, np.float32), 8)
    assert list(idx) == list(range(8))
    assert np.allclose(w, 1.0 / 8)


def test_router_near_tie_resolves_by_logit():
    # T/Kernels/MoE/RouterTopKTests.swift:46-70: expert 8's gain is 1e-4 above
    # expert 7's, so 8 ranks ahead of 7; both are in the top 8 minus one of them.
    E, D = 16, 128
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
    logits = oracle.router_logits(W, S, B, hidden, fmt=oracle.FMT_BF16)
    idx, _ = oracle.topk_softmax(logits, 8)
    assert list(idx) == list(_topk_brute(logits, 8))
    assert list(idx[:7]) == list(range(7))


def test_router_logits_equal_int8_gemv_of_scaled_hidden():
    W, S, B, tail = (lambda k: (lambda u: (*oracle.quantize_int8_matrix(u[:16 * 128].reshape(16, 128)),
                                           u[16 * 128:]))(synth.uniform24(k, 16 * 128 + 256, -1, 1)))(
        synth.seed_key(5, "router"))
    h, eff = tail[:128], tail[128:] + np.float32(2.0)
    a = oracle.router_logits(W, S, B, h, eff, fmt=oracle.FMT_BF16)
    b = oracle.gemv_int8(W, S, B, (h * eff).astype(np.float32), oracle.FMT_BF16)
    assert np.array_equal(a, b)


# --------------------------------------------------------------- MoE ----

def test_gelu_reference_points():
    # T/Validation/Reference/MoEReferenceTests.swift:8-17
    g = oracle.gelu_tanh
    assert abs(g(0.0)) < 1e-7
    expected = 0.5 * (1 + math.tanh(0.7978845608028654 * (1 + 0.044715)))
    assert abs(g(1.0) - expected) < 1e-5
    assert g(1.0) > 0 and g(-1.0) < 0 and g(2.0) > g(1.0)
    # the tanh form approximates the erf GELU within 1e-3 on [-5, 5]
    for v in np.linspace(-5, 5, 101):
        assert abs(g(float(v)) - 0.5 * v * (1 + math.erf(v / math.sqrt(2)))) < 1e-3


def _small_pool(num_experts, d, f, seed):
    offsets, stride = synth.expert_layout(d, f, align=256)
    pool = np.zeros(num_experts * stride, np.uint8)
    for e in range(num_experts):
        pool[e * stride:(e + 1) * stride] = synth.expert_blob(seed, f"e{e}", d, f, offsets, stride)
    return pool, offsets, stride


def test_ffn_matches_independent_numpy():
    d, f = 128, 64
    pool, off, stride = _small_pool(2, d, f, 21)
    x = synth.normal(synth.seed_key(21, "x"), d)
    out = oracle.ffn_int4(pool[:stride], off, x, d, f)
    gw, gs, gb = synth.blob_views(pool[:stride], off, d, f, "gate")
    uw, us, ub = synth.blob_views(pool[:stride], off, d, f, "up")
    dw, dsc, db = synth.blob_views(pool[:stride], off, d, f, "down")
    g = dequant_int4_np(gw, gs, gb).astype(np.float64) @ x
    u = dequant_int4_np(uw, us, ub).astype(np.float64) @ x
    act = 0.5 * g * (1 + np.tanh(0.7978845608028654 * (g + 0.044715 * g ** 3))) * u
    ref = dequant_int4_np(dw, dsc, db).astype(np.float64) @ act
    assert oracle.rel_error(out, ref) < 1e-5


def test_moe_routed_is_linear_in_routing_weights():
    d, f = 128, 64
    pool, off, stride = _small_pool(4, d, f, 33)
    x = synth.normal(synth.seed_key(33, "x"), d)
    res = synth.normal(synth.seed_key(33, "r"), d)
    o1 = oracle.ffn_int4(pool[stride:2 * stride], off, x, d, f)
    o3 = oracle.ffn_int4(pool[3 * stride:], off, x, d, f)
    w = np.array([0.25, 0.75], np.float32)
    y = oracle.moe_routed(pool, stride, off, x, np.array([1, 3], np.uint32), w, d, f, residual=res)
    expect = (res + o1 * w[0]).astype(np.float32) + (o3 * w[1]).astype(np.float32)
    assert np.array_equal(y, expect)


# ---------------------------------------------------------- grouping ----

def _pairs(rows):
    a = np.zeros(len(rows), oracle.PAIR_DTYPE)
    for i, (t, e, r, w) in enumerate(rows):
        a[i] = (t, e, r, w)
    return a


def test_grouping_known_answer():
    # T/Kernels/Prefill/PrefillMoEGroupingTests.swift:5-53
    rows = [(0, 3, 0, 10), (0, 1, 1, 11), (0, 4, 2, 12), (1, 1, 0, 13), (1, 3, 1, 14), (1, 2, 2, 15),
            (2, 4, 0, 16), (2, 3, 1, 17), (2, 1, 2, 18), (3, 5, 0, 19), (3, 1, 1, 20), (3, 4, 2, 21)]
    g = oracle.group_pairs(_pairs(rows[::-1]), 4, 3, 6, 2)
    assert list(g["sorted"]["expert"]) == [1, 1, 1, 1, 2, 3, 3, 3, 4, 4, 4, 5]
    assert [[int(p["token"]), int(p["rank"])] for p in g["sorted"]] == [
        [0, 1], [1, 0], [2, 2], [3, 1], [1, 2], [0, 0], [1, 1], [2, 1], [0, 2], [2, 0], [3, 2], [3, 0]]
    assert list(g["offsets"]) == [0xFFFFFFFF, 0, 4, 5, 8, 11]
    assert list(g["counts"]) == [0, 4, 1, 3, 3, 1]
    assert [tuple(int(v) for v in x) for x in g["groups"]] == [
        (1, 0, 4), (2, 4, 1), (3, 5, 3), (4, 8, 3), (5, 11, 1)]
    assert [tuple(int(v) for v in x) for x in g["tiles"]] == [(0, 2, 0, 5), (2, 2, 5, 6), (4, 1, 11, 1)]
    assert max(g["groups"]["pair_count"]) == 4
    assert max(g["tiles"]["pair_count"]) == 6
    assert max(g["tiles"]["group_count"]) == 2


def test_grouping_deterministic_and_preserves_weight_bits():
    # PrefillMoEGroupingTests.swift:55-82
    tm = [(0, 2, 0, 101), (0, 1, 1, 102), (1, 2, 0, 103), (1, 0, 1, 104), (2, 1, 0, 105), (2, 2, 1, 106)]
    sh = [tm[5], tm[1], tm[3], tm[0], tm[4], tm[2]]
    a = oracle.group_pairs(_pairs(tm), 3, 2, 3, 2)
    b = oracle.group_pairs(_pairs(sh), 3, 2, 3, 2)
    for k in ("sorted", "offsets", "counts", "groups", "tiles"):
        assert np.array_equal(a[k], b[k])
    assert list(a["sorted"]["weight_bits"]) == [104, 102, 105, 101, 103, 106]


def test_grouping_sort_keys():
    # PrefillMoEGroupingTests.swift:84-115
    rows = [(0, 1, 0, 10), (0, 2, 1, 20), (1, 3, 0, 30), (1, 1, 1, 11), (2, 2, 0, 21), (2, 3, 1, 31)]
    g = oracle.group_pairs(_pairs(rows), 3, 2, 4, 2, sort_keys=[0, 30, 10, 20])
    assert list(g["groups"]["expert"]) == [2, 3, 1]
    assert list(g["sorted"]["expert"]) == [2, 2, 3, 3, 1, 1]
    assert list(g["offsets"]) == [0xFFFFFFFF, 4, 0, 2]
    assert [tuple(int(v) for v in x) for x in g["tiles"]] == [(0, 2, 0, 4), (2, 1, 4, 2)]


@pytest.mark.parametrize("pairs,args,name,values", [
    ([(0, 0, 0, 1)], (1, 1, 1, 17), "invalidTileExpertCount", (17, 0)),
    ([(0, 2, 0, 1)], (1, 1, 2, 1), "expertOutOfRange", (2, 0)),
    ([(0, 0, 0, 1), (0, 1, 0, 2)], (1, 2, 2, 1), "duplicateTokenRank", (0, 0)),
])
def test_grouping_rejects_invalid_metadata(pairs, args, name, values):
    # PrefillMoEGroupingTests.swift:117-173
    with pytest.raises(oracle.GroupingError) as ei:
        oracle.group_pairs(_pairs(pairs), *args)
    assert ei.value.name == name and ei.value.values == values


def test_grouping_rejects_sort_key_count():
    with pytest.raises(oracle.GroupingError) as ei:
        oracle.group_pairs(_pairs([(0, 0, 0, 1)]), 1, 1, 2, 1, sort_keys=[0])
    assert ei.value.name == "expertSortKeyCountMismatch" and ei.value.values == (2, 1)


def test_grouping_t32_pressure():
    # PrefillMoEGroupingTests.swift:175-203
    rows = [(t, (t + r * 7) % 74, r, t * 8 + r) for t in range(32) for r in range(8)]
    g = oracle.group_pairs(_pairs(rows), 32, 8, 128, 16)
    assert g["sorted"].size == 256 and g["groups"].size <= 74
    assert all(t["group_count"] <= 16 and t["pair_count"] > 0 for t in g["tiles"])


# ------------------------------------------------- reduce / partials ----

def test_reduce_token_major_matches_numpy():
    # PrefillMoETests.swift:8-44 inputs (SplitMix64 seed 0x4D0E2026)
    rows, k, d = 3, 8, 64
    r = oracle.SplitMix64(0x4D0E2026)
    partials = r.uniforms(rows * k * d, -2.0, 2.0).astype(np.float16)
    weights = r.uniforms(rows * k, -1.0, 1.0).astype(np.float16)
    got = oracle.reduce_token_major(partials.view(np.uint16), weights.view(np.uint16), rows, k, d)
    p = partials.astype(np.float32).reshape(rows, k, d)
    w = weights.astype(np.float32).reshape(rows, k, 1)
    acc = np.zeros((rows, d), np.float32)
    for rr in range(k):
        acc = (acc + (w[:, rr] * p[:, rr])).astype(np.float32)
    assert np.array_equal(got.view(np.float16), acc.astype(np.float16).ravel())


def test_grouped_partials_match_per_pair_ffn():
    d, f, E, T, k = 64, 64, 4, 3, 2
    pool, off, stride = _small_pool(E, d, f, 44)
    rows = [(0, 2, 0, 0), (0, 0, 1, 0), (1, 1, 0, 0), (1, 2, 1, 0), (2, 0, 0, 0), (2, 1, 1, 0)]
    g = oracle.group_pairs(_pairs(rows), T, k, E, 16)
    hidden = (((np.arange(T * d) % 17) - 8) * 0.01).astype(np.float16)
    parts = oracle.grouped_route_partials(g["sorted"], hidden.view(np.uint16), d, pool, stride, off, k,
                                          d, f, T).view(np.float16).astype(np.float32)
    for (t, e, r, _) in rows:
        out = oracle.ffn_int4(pool[e * stride:(e + 1) * stride], off, hidden[t * d:(t + 1) * d]
                              .astype(np.float32), d, f)
        got = parts[(t * k + r) * d:(t * k + r + 1) * d]
        # the grouped reference rounds act and output to fp16
        assert np.max(np.abs(got - out)) <= 2e-3 * max(1.0, np.abs(out).max())


# -------------------------------------------------------------- GEMM ----

def test_gemm_matches_float64():
    M, N, K = 5, 48, 256
    W, S, B = synth.int4_matrix(3, "gemm", N, K)
    X = synth.normal(synth.seed_key(3, "X"), M * K).reshape(M, K)
    Y = oracle.gemm_int4(W, S, B, X)
    ref = X.astype(np.float64) @ dequant_int4_np(W, S, B).astype(np.float64).T
    assert oracle.rel_error(Y, ref) < 1e-5
    part = oracle.gemm_int4(W, S, B, X, rows=(1, 3))
    assert np.array_equal(part[1:3], Y[1:3]) and not part[0].any() and not part[3:].any()


def test_rel_error_definition():
    # V/Tolerance/RelError.swift:7-16
    assert oracle.rel_error([1.0, 2.0], [1.0, 2.5]) == pytest.approx(0.2)
    assert oracle.rel_error([1e-9], [0.0]) == pytest.approx(1e-3)


# ------------------------------------------------ greedy LM head (argmax) ----
# logit.metal:706-787: the largest finite row value wins, the lowest row among
# equal values (v == best, so -0 ties with +0), token 0 when nothing is finite.

def _argmax_brute(z):
    best, best_i = None, None
    for i, v in enumerate(z):
        if not math.isfinite(v):
            continue
        if best is None or v > best:
            best, best_i = v, i
    return 0 if best_i is None else best_i


def test_greedy_argmax_brute_force_with_nonfinite_and_ties():
    rng = np.random.default_rng(7)
    for trial in range(300):
        n = int(rng.integers(1, 40))
        z = rng.integers(-3, 4, n).astype(np.float32)       # many exact ties
        for _ in range(int(rng.integers(0, 4))):
            z[int(rng.integers(0, n))] = rng.choice([np.nan, np.inf, -np.inf])
        assert oracle.greedy_argmax(z) == _argmax_brute(z), z


def test_greedy_argmax_special_cases():
    assert oracle.greedy_argmax(np.array([np.nan, np.inf, -np.inf], np.float32)) == 0
    assert oracle.greedy_argmax(np.array([-np.inf, 5.0, np.nan, 5.0], np.float32)) == 1
    assert oracle.greedy_argmax(np.array([1.0, -0.0, 0.0, -1.0], np.float32)) == 0
    assert oracle.greedy_argmax(np.array([-2.0, -0.0, 0.0, -1.0], np.float32)) == 1   # -0 == +0
    assert oracle.greedy_argmax(np.array([-3.0e38, -1.0e38], np.float32)) == 1
    # numpy's first-occurrence argmax over the finite values
    z = np.random.default_rng(8).standard_normal(10000).astype(np.float32)
    z[::97] = np.nan
    assert oracle.greedy_argmax(z) == int(np.argmax(np.where(np.isfinite(z), z, -np.inf)))


def test_lm_head_greedy_is_norm_then_rows_then_argmax():
    d, vocab = 256, 777
    W, S, B = synth.int4_matrix(3, "pin/lmhead", vocab, d)
    h16 = synth.f16_vector(3, "pin/lmhead/h", d)
    w16 = synth.f16_vector(3, "pin/lmhead/w", d, std=0.5)
    tok, z = oracle.lm_head_greedy(h16, w16, W, S, B, eps=1e-6)
    # independent numpy: RMSNorm (float64 sum of squares, as RmsNorm.swift), fp16 rounding,
    # then the dequantised rows in float64
    h = h16.view(np.float16).astype(np.float32)
    w = w16.view(np.float16).astype(np.float32)
    inv = np.float32(1.0) / np.sqrt(np.float32(np.sum(h.astype(np.float64) ** 2) / d) + np.float32(1e-6))
    x = ((h * w) * inv).astype(np.float16).astype(np.float64)
    z64 = dequant_int4_np(W, S, B).astype(np.float64) @ x
    assert np.max(np.abs(z - z64)) <= 1e-5 * max(1.0, np.max(np.abs(z64)))
    order = np.argsort(-z64)
    assert z64[order[0]] - z64[order[1]] > 1e-3             # no near tie at this seed
    assert tok == int(order[0])
    # no scale: the same rows over the unweighted norm
    tok0, z0 = oracle.lm_head_greedy(h16, None, W, S, B)
    x0 = (h * inv).astype(np.float16).astype(np.float64)
    assert tok0 == int(np.argmax(dequant_int4_np(W, S, B).astype(np.float64) @ x0))
