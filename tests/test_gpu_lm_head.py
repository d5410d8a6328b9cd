"""GPU parity of the greedy int4 LM head (tfq_lm_head_greedy) against the CPU
oracle: LMHeadChainInt4.encodeGreedyDecode
(S/Kernels/Fusions/LMHeadChainInt4.swift:62-135; logit.metal:688-787).

The token is an index: it must equal the oracle's bit for bit. Where two
rows' logits are closer than the fp32 accumulation-order difference between
the GPU and the oracle could flip (never at these seeds: the tests assert a
clear gap first), the exact-tie cases below pin the tie rule with rows whose
logits are equal bit for bit on both sides (identical row data).
"""
import numpy as np
import pytest

import oracle
from edgeexpert_amd import ops, synth
from edgeexpert_amd._lib import LM_HEAD_WORKSPACE_BYTES, TfqError, TFQ_E_INVAL, TFQ_E_UNSUPPORTED
from edgeexpert_amd.runtime import DeviceBuffer

pytestmark = pytest.mark.gpu


def _dev(a):
    return DeviceBuffer.from_array(np.ascontiguousarray(a))


def _greedy(ctx, stream, h16, w16, W, S, B, eps=1e-6):
    vocab, d = W.shape[0], h16.size
    out = _dev(np.full(1, 0xDEADBEEF, np.uint32))
    ws = DeviceBuffer(LM_HEAD_WORKSPACE_BYTES)
    ws.fill(0xFF)
    ops.LMHeadGreedyInt4(ctx).encode_greedy_decode(stream, _dev(h16), None if w16 is None else _dev(w16),
                                                   _dev(W), _dev(S), _dev(B), out, d, vocab, ws, eps)
    stream.sync()
    return int(out.download(np.uint32, 1)[0])


def _inputs(seed, d, vocab):
    W, S, B = synth.int4_matrix(seed, f"lmhead/{d}x{vocab}", vocab, d)
    h16 = synth.f16_vector(seed, f"lmhead/h{d}", d)
    w16 = synth.f16_vector(seed, f"lmhead/w{d}", d, std=0.5)
    return W, S, B, h16, w16


def _clear_winner(z):
    zf = np.where(np.isfinite(z), z, -np.inf)
    if zf.size < 2:
        return True
    top2 = np.sort(zf)[-2:]
    return top2[1] - top2[0] > 1e-4 * max(1.0, abs(top2[1]))


@pytest.mark.parametrize("d,vocab,seed", [(2816, 4099, 1), (2816, 32768, 2), (256, 1, 3), (512, 777, 4),
                                          (4096, 10000, 5), (64, 300, 6)])
def test_lm_head_greedy_matches_oracle(ctx, stream, d, vocab, seed):
    W, S, B, h16, w16 = _inputs(seed, d, vocab)
    ref, z = oracle.lm_head_greedy(h16, w16, W, S, B)
    assert _clear_winner(z)
    assert _greedy(ctx, stream, h16, w16, W, S, B) == ref


@pytest.mark.parametrize("d,vocab,seed", [(2816, 4099, 12), (4096, 3000, 13), (6144, 2000, 14)])
def test_lm_head_greedy_staging_forms_agree(ctx, stream, d, vocab, seed):
    # a 16-byte aligned hidden state and norm weight take the rows form whose
    # RMSNorm staging is fixed at compile time (d <= 4096), a 2-byte aligned
    # hidden state the form that reads the mode (and d 6144 both): the
    # oracle's token either way
    W, S, B, h16, w16 = _inputs(seed, d, vocab)
    ref, z = oracle.lm_head_greedy(h16, w16, W, S, B)
    assert _clear_winner(z)
    bufs = [_dev(a) for a in (w16, W, S, B)]
    toks = []
    for off in (0, 2):
        hb = DeviceBuffer(d * 2 + 16)
        hb.upload(h16, offset=off)
        out = _dev(np.full(1, 0xDEADBEEF, np.uint32))
        ws = DeviceBuffer(LM_HEAD_WORKSPACE_BYTES)
        ws.fill(0xFF)
        ops.LMHeadGreedyInt4(ctx).encode_greedy_decode(stream, hb, *bufs, out, d, vocab, ws, 1e-6,
                                                       hidden_offset=off)
        stream.sync()
        toks.append(int(out.download(np.uint32, 1)[0]))
    assert toks == [ref, ref]


def test_lm_head_greedy_without_norm_weight(ctx, stream):
    W, S, B, h16, _ = _inputs(7, 2816, 5000)
    ref, z = oracle.lm_head_greedy(h16, None, W, S, B)
    assert _clear_winner(z)
    assert _greedy(ctx, stream, h16, None, W, S, B) == ref


def test_lm_head_greedy_ties_take_the_lowest_row(ctx, stream):
    d, vocab = 2816, 6000
    W, S, B, h16, w16 = _inputs(8, d, vocab)
    ref, _ = oracle.lm_head_greedy(h16, w16, W, S, B)
    # copies of the winning row before and after it: equal logits bit for bit
    for dst in (5, ref + 1 if ref + 1 < vocab else ref - 1, vocab - 1):
        W2, S2, B2 = W.copy(), S.copy(), B.copy()
        W2[dst], S2[dst], B2[dst] = W[ref], S[ref], B[ref]
        tok, z = oracle.lm_head_greedy(h16, w16, W2, S2, B2)
        assert tok == min(dst, ref) and z[dst] == z[ref]
        assert _greedy(ctx, stream, h16, w16, W2, S2, B2) == tok


def test_lm_head_greedy_skips_nonfinite_rows(ctx, stream):
    d, vocab = 2816, 3000
    W, S, B, h16, w16 = _inputs(9, d, vocab)
    ref, _ = oracle.lm_head_greedy(h16, w16, W, S, B)
    S2 = S.copy()
    S2[ref, 3] = 0x7E00                   # NaN scale: the best row's logit is NaN
    S2[ref // 2, 0] = 0x7C00              # +inf scale: +inf or NaN, skipped either way
    tok, z = oracle.lm_head_greedy(h16, w16, W, S2, B)
    assert not np.isfinite(z[ref]) and tok != ref and _clear_winner(z)
    assert _greedy(ctx, stream, h16, w16, W, S2, B) == tok


def test_lm_head_greedy_all_nonfinite_gives_token_zero(ctx, stream):
    d, vocab = 512, 900
    W, S, B, h16, w16 = _inputs(10, d, vocab)
    S2 = np.full_like(S, 0x7E00)
    tok, _ = oracle.lm_head_greedy(h16, w16, W, S2, B)
    assert tok == 0
    assert _greedy(ctx, stream, h16, w16, W, S2, B) == 0


def test_lm_head_greedy_contract(ctx, stream):
    W, S, B, h16, w16 = _inputs(11, 256, 100)
    head = ops.LMHeadGreedyInt4(ctx)
    out, ws = _dev(np.zeros(1, np.uint32)), DeviceBuffer(LM_HEAD_WORKSPACE_BYTES)
    bufs = [_dev(a) for a in (h16, w16, W, S, B)]
    with pytest.raises(TfqError) as e:
        head.encode_greedy_decode(stream, *bufs, out, 200, 100, ws)          # d % 64 != 0
    assert e.value.status == TFQ_E_INVAL
    with pytest.raises(TfqError) as e:
        head.encode_greedy_decode(stream, *bufs, out, 256, 0, ws)            # empty vocab
    assert e.value.status == TFQ_E_INVAL
    with pytest.raises(TfqError) as e:
        head.encode_greedy_decode(stream, *bufs, out, 8256, 100, ws)         # d > 8192
    assert e.value.status == TFQ_E_UNSUPPORTED
    with pytest.raises(TfqError) as e:
        head.encode_greedy_decode(stream, *bufs, out, 256, 100, ws, rms_eps=0.0)
    assert e.value.status == TFQ_E_INVAL
