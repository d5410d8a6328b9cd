"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_fixtures.py) against the CPU oracle: recomputing every
stored output from the stored inputs must reproduce it bit for bit. CPU only."""
import os

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def h2f(b):
    return np.asarray(b, np.uint16).view(np.float16).astype(np.float32)


def test_fixtures_present():
    names = {f[:-4] for f in os.listdir(GOLDEN) if f.endswith(".npz")}
    assert {"gemv_q4_m96_n448", "router_topk_e48_d320_k6", "moe_decode_e6_d256_f128_k3",
            "grouping_t40_k4_e12", "attention_h128_q4_kv2_t150_w96", "gemm_q4_m40_n96_k256"} <= names


def test_gemv_fixture():
    z = load("gemv_q4_m96_n448")
    y = oracle.gemv_int4(z["W"], z["S"], z["B"], h2f(z["x"]))
    assert np.array_equal(y.view(np.uint32), z["y"].view(np.uint32))


def test_router_fixture():
    z = load("router_topk_e48_d320_k6")
    logits = oracle.router_logits(z["W"], z["S"], z["B"], h2f(z["h"]), h2f(z["eff"]))
    assert np.array_equal(logits.view(np.uint32), z["logits"].view(np.uint32))
    idx, w = oracle.topk_softmax(logits, int(z["k"]), h2f(z["gain"]))
    assert np.array_equal(idx, z["idx"]) and np.array_equal(w.view(np.uint32), z["w"].view(np.uint32))


def test_moe_fixture():
    z = load("moe_decode_e6_d256_f128_k3")
    y = oracle.moe_routed(z["pool"], int(z["stride"]), [int(v) for v in z["offsets"]], h2f(z["x"]), z["idx"],
                          h2f(z["w_f16"]), 256, 128)
    assert np.array_equal(y.view(np.uint32), z["y"].view(np.uint32))


def test_grouping_fixture():
    z = load("grouping_t40_k4_e12")
    T, k, E = int(z["T"]), int(z["k"]), int(z["E"])
    pairs = np.zeros(T * k, oracle.PAIR_DTYPE)
    pairs["token"] = np.repeat(np.arange(T, dtype=np.uint32), k)
    pairs["rank"] = np.tile(np.arange(k, dtype=np.uint32), T)
    pairs["expert"] = z["idx"].ravel()
    pairs["weight_bits"] = z["w16"].ravel()
    res = oracle.group_pairs(pairs, T, k, E)
    assert np.array_equal(res["sorted"].view(np.uint32).reshape(-1, 4), z["sorted"])
    assert np.array_equal(res["offsets"], z["offsets"]) and np.array_equal(res["counts"], z["counts"])


def test_attention_fixture():
    z = load("attention_h128_q4_kv2_t150_w96")
    out = oracle.attention(h2f(z["q"]), h2f(z["k"]), h2f(z["v"]), int(z["hd"]), int(z["nq"]), int(z["nkv"]),
                           int(z["seq"]), int(z["window"]))
    assert np.array_equal(out.view(np.uint32), z["out"].view(np.uint32))


def test_gemm_fixture():
    z = load("gemm_q4_m40_n96_k256")
    Y = oracle.gemm_int4(z["W"], z["S"], z["B"], h2f(z["X"]))
    assert np.array_equal(Y.view(np.uint32), z["Y"].view(np.uint32))
