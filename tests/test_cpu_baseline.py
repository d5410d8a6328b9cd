"""The CPU baseline (oracle/cpu_baseline.c, timed by bench.py) computes the
oracle's arithmetic exactly: at any thread count its outputs equal the serial
oracle's bit for bit (threads only split the rows), for BASELINE config 0's
GEMV and a config-1-shaped decode token."""
import numpy as np
import pytest

import oracle
from edgeexpert_amd import synth


@pytest.mark.parametrize("threads", [1, 3, 8])
def test_baseline_gemv_equals_oracle(threads):
    W, S, B = synth.int4_matrix(0, "c0/w", 2816, 2816)
    x = synth.f16_to_f32(synth.f16_vector(0, "c0/x", 2816))
    assert np.array_equal(oracle.baseline_gemv_int4(W, S, B, x, threads), oracle.gemv_int4(W, S, B, x))


@pytest.mark.parametrize("threads", [1, 4])
def test_baseline_decode_token_equals_oracle(threads):
    E, D, F, K = 16, 512, 256, 8
    pool, offs, stride = synth.expert_pool(0, "cpub/experts", E, D, F)
    rW, rS, rB = synth.int8_matrix(0, "cpub/router", E, D)
    h = synth.f16_to_f32(synth.f16_vector(0, "cpub/h", D))
    y, idx, w = oracle.baseline_moe_decode_token(rW, rS, rB, pool, stride, offs, h, D, F, K, threads)
    ridx, rw = oracle.topk_softmax(oracle.router_logits(rW, rS, rB, h), K)
    assert list(idx) == list(ridx) and np.array_equal(w, rw)
    assert np.array_equal(y, oracle.moe_routed(pool, stride, offs, h, ridx, rw, D, F))
