"""The HIP path against the committed golden fixtures (tests/golden/*.npz):
the same bars as the other parity tests — bit-exact for indices and
grouping, RelError <= 1e-3 for floating-point outputs."""
import os

import numpy as np
import pytest

import oracle
from edgeexpert_amd import ops
from edgeexpert_amd._lib import DTYPE_F16, ROUTER_WORKSPACE_BYTES
from edgeexpert_amd.runtime import DeviceBuffer

pytestmark = pytest.mark.gpu
TOL = oracle.Tolerance.north_star
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def dev(a):
    return DeviceBuffer.from_array(np.ascontiguousarray(a))


def h2f(b):
    return np.asarray(b, np.uint16).view(np.float16).astype(np.float32)


def test_gemv_golden(ctx, stream):
    z = load("gemv_q4_m96_n448")
    y = dev(np.zeros(96, np.uint16))
    ops.DequantInt4GEMV(ctx).encode(stream, dev(z["W"]), dev(z["S"]), dev(z["B"]), dev(z["x"]), y, 96, 448)
    stream.sync()
    assert oracle.rel_error(h2f(y.download(np.uint16, 96)), z["y"]) < TOL


def test_router_golden(ctx, stream):
    z = load("router_topk_e48_d320_k6")
    E, d, k = 48, 320, int(z["k"])
    ws = DeviceBuffer(ROUTER_WORKSPACE_BYTES)
    ws.fill(0)
    idx, w16, wf = dev(np.zeros(k, np.uint32)), dev(np.zeros(k, np.uint16)), dev(np.zeros(k, np.float32))
    ops.MoE(ctx).encode_router_gemma4(stream, dev(z["W"]), dev(z["S"]), dev(z["B"]), dev(z["h"]), dev(z["eff"]),
                                      dev(z["gain"]), idx, w16, E, d, k, ws, out_weights_f32=wf)
    stream.sync()
    assert np.array_equal(idx.download(np.uint32, k), z["idx"])
    assert np.max(np.abs(wf.download(np.float32, k) - z["w"])) < 1e-5


def test_moe_decode_golden(ctx, stream):
    z = load("moe_decode_e6_d256_f128_k3")
    d, f, k = 256, 128, 3
    offs = dict(zip(("gate_w", "gate_s", "gate_b", "up_w", "up_s", "up_b", "down_w", "down_s", "down_b"),
                    [int(v) for v in z["offsets"]]))
    pool = ops.ExpertPool(dev(z["pool"]), int(z["stride"]), 6, offs)
    y, acts = dev(np.zeros(d, np.uint16)), dev(np.zeros(k * f, np.uint16))
    ops.MoE(ctx).encode_routed(stream, pool, dev(z["idx"]), dev(z["w_f16"]), dev(z["x"]), None, y, d, f, k, acts)
    stream.sync()
    assert oracle.rel_error(h2f(y.download(np.uint16, d)), z["y"]) < TOL


def test_grouping_golden(ctx, stream):
    z = load("grouping_t40_k4_e12")
    T, k, E = int(z["T"]), int(z["k"]), int(z["E"])
    n, mt = T * k, ops.max_tiles(T, k, E)
    sp, offsets, counts = dev(np.zeros(n, ops.PAIR_DTYPE)), dev(np.zeros(E, np.uint32)), dev(np.zeros(E, np.uint32))
    tiles, nt, st = dev(np.zeros(mt, ops.TILE_DTYPE)), dev(np.zeros(1, np.uint32)), dev(np.full(1, 9, np.uint32))
    ops.PrefillMoEGrouping(ctx).encode(stream, dev(z["idx"]), dev(z["w16"]), T, k, E, sp, offsets, counts, tiles,
                                       nt, st)
    stream.sync()
    assert st.download(np.uint32, 1)[0] == 0
    assert np.array_equal(sp.download(np.uint32, n * 4).reshape(-1, 4), z["sorted"])
    assert np.array_equal(counts.download(np.uint32, E), z["counts"])
    got_off = offsets.download(np.uint32, E)
    assert np.array_equal(got_off, z["offsets"])


def test_attention_golden(ctx, stream):
    z = load("attention_h128_q4_kv2_t150_w96")
    hd, nq, nkv, seq, window = (int(z[k_]) for k_ in ("hd", "nq", "nkv", "seq", "window"))
    wsb = ops.Attention.workspace_bytes(hd, nq, seq, window)
    ws, out = DeviceBuffer(wsb), dev(np.zeros(nq * hd, np.uint16))
    ops.Attention(ctx).encode(stream, dev(z["q"]), dev(z["k"]), dev(z["v"]), out, hd, nq, nkv, seq, ws, wsb,
                              window=window)
    stream.sync()
    assert oracle.rel_error(h2f(out.download(np.uint16, nq * hd)), z["out"]) < TOL


def test_gemm_golden(ctx, stream):
    z = load("gemm_q4_m40_n96_k256")
    M, N, K = 40, 96, 256
    Y = dev(np.zeros(M * N, np.uint16))
    ops.PrefillInt4QMM(ctx).encode(stream, dev(z["W"]), dev(z["S"]), dev(z["B"]), dev(z["X"]), Y, M, N, K,
                                   dtype=DTYPE_F16)
    stream.sync()
    assert oracle.rel_error(h2f(Y.download(np.uint16, M * N)).reshape(M, N), z["Y"]) < TOL
