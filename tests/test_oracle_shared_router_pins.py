"""Pins of the shared-expert oracles (int4 and int8) and of the prefill router
oracle, each against an independent computation.

Shared expert (T/Kernels/MoE/SharedExpertInt4Tests.swift:13-28,
SharedExpertInt8Tests.swift:46-68): the inputs are the reference tests' own
(SeedTree(seed).key(label) uniforms in (-0.4, 0.4), drawn x, gate, up, down
in that order, quantised with quantizeInt4Affine / quantizeInt8Affine). The
independent side dequantises with numpy, forms gate and up in float64, the
GELU in float64, rounds act to fp16 and runs the down projection in float64.
Two planted mistakes must fail the same bound: gate and up swapped, and the
fp16 rounding of act left out.

Prefill router (PrefillRouter.encodeGemma4Block's reference, the per-token
router of RouterTopKTests.swift:72-97 applied to every row of a strided
hidden block): equal to per-row router_logits + topk_softmax, and to a
float64 numpy + sort brute force; reading the rows with the wrong stride
must change the result.
"""
import numpy as np
import pytest

import oracle
from edgeexpert_amd import synth
from helpers import dequant_int4_np

C_GELU = 0.7978845608028654


def _gelu64(g):
    return 0.5 * g * (1.0 + np.tanh(C_GELU * (g + 0.044715 * g ** 3)))


def _dequant_int8_np(W, S, B, fmt):
    to32 = synth.f16_to_f32 if fmt == oracle.FMT_F16 else synth.bf16_to_f32
    return (W.astype(np.float32) * np.repeat(to32(S), 64, axis=-1)
            + np.repeat(to32(B), 64, axis=-1)).astype(np.float32)


def _reference_inputs(seed, label, d, f, bits):
    """The reference test's draw: x[d], gate[f][d], up[f][d], down[d][f]."""
    u = synth.uniform24(synth.seed_key(seed, label), d + 3 * f * d, -0.4, 0.4)
    x = u[:d]
    gate = u[d:d + f * d].reshape(f, d)
    up = u[d + f * d:d + 2 * f * d].reshape(f, d)
    down = u[d + 2 * f * d:].reshape(d, f)
    q = oracle.quantize_int4_matrix if bits == 4 else oracle.quantize_int8_matrix
    return x, q(gate), q(up), q(down)


def _independent(gate, up, down, x16, bits, fmt, round_act=True, swap=False, round_gu=False):
    deq = (lambda t: dequant_int4_np(*t, fmt)) if bits == 4 else (lambda t: _dequant_int8_np(*t, fmt))
    g = deq(gate).astype(np.float64) @ x16.astype(np.float64)
    u = deq(up).astype(np.float64) @ x16.astype(np.float64)
    if round_gu:
        g = g.astype(np.float32).astype(np.float16).astype(np.float64)
        u = u.astype(np.float32).astype(np.float16).astype(np.float64)
    if swap:
        g, u = u, g
    act = _gelu64(g) * u
    if round_act:
        act = act.astype(np.float32).astype(np.float16).astype(np.float64)
    return deq(down).astype(np.float64) @ act


@pytest.mark.parametrize("bits,seed,label,d,f", [
    (4, 0x604, "shared-expert-int4", 128, 64),      # SharedExpertInt4Tests.swift:13-14
    (8, 0x601, "shared-expert-int8", 128, 64),      # SharedExpertInt8Tests.swift:46-47
    (4, 0x61, "shared-expert-int4-wide", 512, 256),
    (8, 0x62, "shared-expert-int8-wide", 512, 256),
])
def test_shared_expert_oracle_matches_independent_float64(bits, seed, label, d, f):
    x, gate, up, down = _reference_inputs(seed, label, d, f, bits)
    x16 = x.astype(np.float16).astype(np.float32)           # Float(Float16(x)), as the test feeds it
    run = oracle.shared_expert_int4 if bits == 4 else oracle.shared_expert_int8
    y = run(gate, up, down, x16, d, f, oracle.FMT_BF16)
    ref = _independent(gate, up, down, x16, bits, oracle.FMT_BF16)
    bound = 1e-5
    assert oracle.rel_error(y, ref) < bound
    # planted mistakes that the same bound must catch
    no_round = _independent(gate, up, down, x16, bits, oracle.FMT_BF16, round_act=False)
    swapped = _independent(gate, up, down, x16, bits, oracle.FMT_BF16, swap=True)
    assert oracle.rel_error(no_round, ref) > bound
    assert oracle.rel_error(swapped, ref) > 100 * bound
    # the generic form with round_gu: gate and up rounded to fp16 before the activation
    assert np.array_equal(oracle.shared_expert(gate, up, down, x16, d, f, bits, False, oracle.FMT_BF16), y)
    y_gu = oracle.shared_expert(gate, up, down, x16, d, f, bits, True, oracle.FMT_BF16)
    ref_gu = _independent(gate, up, down, x16, bits, oracle.FMT_BF16, round_gu=True)
    assert oracle.rel_error(y_gu, ref_gu) < bound
    assert oracle.rel_error(ref, ref_gu) > bound        # the rounding is visible at this bound


def _router_inputs(T, E, d, stride, seed):
    key = synth.seed_key(seed, "prefill-router-pin")
    u = synth.uniform24(key, E * d + T * stride, -1.0, 1.0)
    W, S, B = oracle.quantize_int8_matrix(u[:E * d].reshape(E, d))
    hidden = u[E * d:].reshape(T, stride).astype(np.float16).astype(np.float32)
    return W, S, B, hidden


@pytest.mark.parametrize("T,E,d,stride,k", [(6, 32, 256, 272, 4), (5, 128, 512, 576, 8)])
def test_prefill_router_oracle_is_per_row_router(T, E, d, stride, k):
    W, S, B, hidden = _router_inputs(T, E, d, stride, 0x7E + k)
    idx, w = oracle.prefill_router(W, S, B, hidden, k, fmt=oracle.FMT_BF16)
    deq = _dequant_int8_np(W, S, B, oracle.FMT_BF16).astype(np.float64)
    for t in range(T):
        row = hidden[t, :d]
        logits = oracle.router_logits(W, S, B, row, fmt=oracle.FMT_BF16)
        ridx, rw = oracle.topk_softmax(logits, k)
        assert list(idx[t]) == list(ridx)
        assert np.array_equal(w[t], rw)
        # independent: float64 logits, sort by (value desc, index asc)
        l64 = deq @ row.astype(np.float64)
        assert np.allclose(logits, l64, rtol=0, atol=1e-5 * np.abs(l64).max())
        order = np.lexsort((np.arange(E), -l64))[:k]
        assert list(idx[t]) == list(order)
        sel = l64[order]
        soft = np.exp(sel - sel.max())
        assert np.allclose(w[t], soft / soft.sum(), rtol=1e-5, atol=1e-7)
    # rows read with stride d instead of `stride` (a dropped stride) route differently
    flat = np.ascontiguousarray(hidden).reshape(-1)[:T * d].reshape(T, d)
    bad_idx, _ = oracle.prefill_router(W, S, B, flat, k, fmt=oracle.FMT_BF16)
    assert not np.array_equal(bad_idx[1:], idx[1:])


def test_topk_nan_ranks_last_and_signed_zeros_tie_by_index():
    # router_topk_select_k8 (moe.metal:152-168) never prefers NaN; -0 == +0
    logits = np.array([np.nan, -0.0, 1.0, 0.0, np.nan, -1.0], np.float32)
    idx, w = oracle.topk_softmax(logits, 4)
    assert list(idx) == [2, 1, 3, 5]
    assert np.all(np.isfinite(w))
    idx6, _ = oracle.topk_softmax(logits, 6)
    assert list(idx6) == [2, 1, 3, 5, 0, 4]
