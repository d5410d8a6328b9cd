"""GPU check of the allocation-free decode entry point
(tfq_moe_decode_token_noalloc): through the C ABI, its outputs equal those
of tfq_moe_decode_token (caller-provided scratch) bit for bit — same kernels,
same inputs — on two calls in a row, the second with a smaller shape, and it
rejects a shape beyond its fixed scratch."""
import ctypes as C

import numpy as np
import pytest

import oracle
from edgeexpert_amd import ops, synth
from edgeexpert_amd._lib import ROUTER_WORKSPACE_BYTES, TFQ_E_INVAL, TfqError, lib
from edgeexpert_amd.runtime import DeviceBuffer

pytestmark = pytest.mark.gpu


def _dev(a):
    return DeviceBuffer.from_array(np.ascontiguousarray(a))


def _case(ctx, stream, E, D, F, K, seed):
    print(f"[noalloc] E={E} D={D} F={F} K={K}", flush=True)
    pool_bytes, offs, stride = synth.expert_pool(seed, f"noalloc{E}", E, D, F)
    pool = ops.ExpertPool(_dev(pool_bytes), stride, E, offs)
    W, S, B = synth.int8_matrix(seed, f"noalloc{E}/router", E, D)
    router = ops.Router(_dev(W), _dev(S), _dev(B), E)
    h16 = synth.f16_vector(seed, f"noalloc{E}/h", D)
    res16 = synth.f16_vector(seed, f"noalloc{E}/r", D, std=0.1)
    x, res = _dev(h16), _dev(res16)
    outs = {}
    for mode in ("scratch", "noalloc"):
        y = _dev(np.full(D, 0x7E00, np.uint16))
        idx, w16 = _dev(np.full(K, 0xFFFFFFFF, np.uint32)), _dev(np.zeros(K, np.uint16))
        if mode == "scratch":
            acts, ws = DeviceBuffer(K * F * 2), DeviceBuffer(ROUTER_WORKSPACE_BYTES)
            ops.moe_decode_token(ctx, stream, router, pool, x, res, y, D, F, K, idx, w16, acts, ws)
        else:
            ops.moe_decode_token_noalloc(ctx, stream, router, pool, x, res, y, D, F, K, idx, w16)
        stream.sync()
        outs[mode] = (y.download(np.uint16, D), idx.download(np.uint32, K), w16.download(np.uint16, K))
    for a, b in zip(outs["scratch"], outs["noalloc"]):
        assert np.array_equal(a, b)
    # and both against the oracle (routing bit-exact, output within 1e-3)
    h = h16.view(np.float16).astype(np.float32)
    ridx, _ = oracle.topk_softmax(oracle.router_logits(W, S, B, h), K)
    assert list(outs["noalloc"][1]) == list(ridx)
    wdev = outs["noalloc"][2].view(np.float16).astype(np.float32)
    ref = oracle.moe_routed(pool_bytes, stride, offs, h, ridx, wdev, D, F,
                            residual=res16.view(np.float16).astype(np.float32))
    got = outs["noalloc"][0].view(np.float16).astype(np.float32)
    assert oracle.rel_error(got, ref) < oracle.Tolerance.north_star


def test_noalloc_decode_token_equals_scratch_form_twice(ctx, stream):
    _case(ctx, stream, 128, 2816, 704, 8, 1)      # config 1
    _case(ctx, stream, 16, 512, 256, 4, 2)        # a smaller second call on the same scratch


def test_noalloc_rejects_shape_beyond_scratch(ctx, stream):
    E, D, F, K = 8, 128, 1088, 8                  # 8 * 1088 * 2 > 16384 bytes
    pool_bytes, offs, stride = synth.expert_pool(3, "noalloc-big", E, D, F)
    pool = ops.ExpertPool(_dev(pool_bytes), stride, E, offs)
    W, S, B = synth.int8_matrix(3, "noalloc-big/router", E, D)
    router = ops.Router(_dev(W), _dev(S), _dev(B), E)
    b = _dev(np.zeros(4096, np.uint8))
    with pytest.raises(TfqError) as ei:
        ops.moe_decode_token_noalloc(ctx, stream, router, pool, b, None, b, D, F, K, b, b)
    assert ei.value.status == TFQ_E_INVAL
    assert b"scratch" in lib().tfq_last_error_message()


def test_noalloc_decode_token_replays_from_a_captured_graph(ctx, stream):
    # the allocation-free call captured into a HIP graph (stream capture: a
    # hipMalloc, or a memset node, inside it would break or corrupt the
    # replays) and replayed three times, with eager calls of both forms
    # between the replays; every replay equals the eager call bit for bit
    from edgeexpert_amd.runtime import Graph
    E, D, F, K = 128, 2816, 704, 8
    print(f"[noalloc] graph E={E} D={D} F={F} K={K}", flush=True)
    pool_bytes, offs, stride = synth.expert_pool(4, "noalloc-g", E, D, F)
    pool = ops.ExpertPool(_dev(pool_bytes), stride, E, offs)
    W, S, B = synth.int8_matrix(4, "noalloc-g/router", E, D)
    router = ops.Router(_dev(W), _dev(S), _dev(B), E)
    x, res = _dev(synth.f16_vector(4, "noalloc-g/h", D)), _dev(synth.f16_vector(4, "noalloc-g/r", D, std=0.1))
    x2 = _dev(synth.f16_vector(5, "noalloc-g/h2", D))
    y, idx, w16 = DeviceBuffer(D * 2), DeviceBuffer(K * 4), DeviceBuffer(K * 2)
    y2, idx2, w2 = DeviceBuffer(D * 2), DeviceBuffer(K * 4), DeviceBuffer(K * 2)
    acts, ws = DeviceBuffer(K * F * 2), DeviceBuffer(ROUTER_WORKSPACE_BYTES)

    def call():
        ops.moe_decode_token_noalloc(ctx, stream, router, pool, x, res, y, D, F, K, idx, w16)

    call()
    stream.sync()
    eager = (y.download(np.uint16, D).copy(), idx.download(np.uint32, K).copy(), w16.download(np.uint16, K).copy())
    g = Graph(stream, call)
    for r in range(3):
        y.fill(0)
        idx.fill(0xFF)
        w16.fill(0)
        g.launch(stream)
        stream.sync()
        got = (y.download(np.uint16, D), idx.download(np.uint32, K), w16.download(np.uint16, K))
        for a, b in zip(got, eager):
            assert np.array_equal(a, b), f"replay {r}"
        # eager work on the same scratch and on caller scratch between replays
        ops.moe_decode_token_noalloc(ctx, stream, router, pool, x2, None, y2, D, F, K, idx2, w2)
        ops.moe_decode_token(ctx, stream, router, pool, x2, None, y2, D, F, K, idx2, w2, acts, ws)
        stream.sync()
