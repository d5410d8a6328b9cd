"""Loading a repacked (.gturbo) checkpoint into device memory
(tfq_expert_pool_load, tfq_resident_load) on the GPU: the pool holds each
logical expert's weights bit for bit and its BF16 scales/biases as fp16 (the
exact conversion), whatever the file's physical order; the MoE decode phases
run on the loaded pool and match the oracle; missing, short and mismatched
files fail with the documented status."""
import os

import numpy as np
import pytest

import gturbo
import oracle
from edgeexpert_amd import ops, synth
from edgeexpert_amd._lib import TfqError, TFQ_E_INVAL, TFQ_E_IO, TFQ_E_UNSUPPORTED
from edgeexpert_amd.runtime import DeviceBuffer
from helpers import from_f16_bits

pytestmark = pytest.mark.gpu
TOL = oracle.Tolerance.north_star


def _dev(a):
    return DeviceBuffer.from_array(np.ascontiguousarray(a))


def _bf16_to_f16(bits):
    return synth.bf16_to_f32(bits).astype(np.float16).view(np.uint16)


def _load(ctx, stream, root, layer, d, f):
    L = ops.PackedExpertsLayout(root)
    stride, total = L.pool_bytes(d, f)
    pool = DeviceBuffer(total)
    pool.fill(0xFF)
    inexact = _dev(np.zeros(1, np.uint32))
    p = L.load_pool(ctx, stream, layer, d, f, pool, inexact)
    stream.sync()
    return L, p, int(inexact.download(np.uint32, 1)[0])


@pytest.mark.parametrize("d,f,experts,order,bits", [(256, 128, 4, [3, 1, 0, 2], 4),
                                                    (2816, 704, 8, [5, 2, 7, 0, 1, 6, 4, 3], 4),
                                                    (256, 128, 4, [2, 3, 1, 0], 3), (320, 192, 3, [1, 2, 0], 2)])
def test_pool_holds_each_logical_expert(ctx, stream, tmp_path, d, f, experts, order, bits):
    data, _ = gturbo.write_model(str(tmp_path), d, f, experts, layers=2, physical_order=order, bits=bits)
    L, pool, inexact = _load(ctx, stream, str(tmp_path), 1, d, f)
    assert inexact == 0
    assert pool.num_experts == experts and pool.stride % 256 == 0 and pool.weight_bits == bits
    assert all(pool.offsets[k] % 16 == 0 for k in ("gate_w", "up_w", "down_w"))
    raw = pool.buffer.download(np.uint8, pool.stride * experts)
    for e in range(experts):
        blob = raw[e * pool.stride:(e + 1) * pool.stride]
        for role in ("gate", "up", "down"):
            W, s, b = data[(1, e)][role]
            w_off = pool.offsets[role + "_w"]
            assert np.array_equal(blob[w_off:w_off + W.size], W.ravel()), (e, role)
            for key, bf in (("_s", s), ("_b", b)):
                off = pool.offsets[role + key]
                got = blob[off:off + 2 * bf.size].view(np.uint16)
                assert np.array_equal(got, _bf16_to_f16(bf.ravel())), (e, role + key)


@pytest.mark.parametrize("bits", [4, 3, 2])
def test_loaded_pool_runs_the_decode_phases(ctx, stream, tmp_path, bits):
    D, F, E, K = 2816, 704, 8, 8
    gturbo.write_model(str(tmp_path), D, F, E, physical_order=[1, 0, 3, 2, 5, 4, 7, 6], bits=bits)
    L, pool, _ = _load(ctx, stream, str(tmp_path), 0, D, F)
    pool_bytes = pool.buffer.download(np.uint8, pool.stride * E)
    rng = np.random.default_rng(3)
    idx16 = rng.permutation(E).astype(np.uint32)[:K]
    x16 = synth.f16_vector(3, "gturbo/x", D)
    rw16 = synth.f16_bits(rng.dirichlet(np.ones(K)).astype(np.float32))
    acts = _dev(np.full(K * F, 0x7E00, np.uint16))
    y = _dev(np.zeros(D, np.uint16))
    idx = _dev(idx16)
    moe = ops.MoE(ctx)
    moe.encode_routed_phase1(stream, pool, idx, _dev(x16), acts, D, F, K)
    moe.encode_routed_phase2(stream, pool, idx, acts, _dev(rw16), None, y, D, F, K)
    stream.sync()
    got = from_f16_bits(y.download(np.uint16, D))
    ref = oracle.moe_routed(pool_bytes, pool.stride, pool.offsets, from_f16_bits(x16), idx16,
                            from_f16_bits(rw16), D, F, bits=bits)
    assert oracle.rel_error(got, ref) < TOL


def test_pool_load_errors(ctx, stream, tmp_path):
    root = str(tmp_path)
    gturbo.write_model(root, 256, 128, 2)
    L = ops.PackedExpertsLayout(root)
    stride, total = L.pool_bytes(256, 128)
    pool = DeviceBuffer(total)
    for d, f, status in ((256, 192, TFQ_E_INVAL), (320, 128, TFQ_E_INVAL), (250, 128, TFQ_E_INVAL)):
        with pytest.raises(TfqError) as e:
            L.load_pool(ctx, stream, 0, d, f, pool)
        assert e.value.status == status
    with pytest.raises(TfqError) as e:                     # pool too small
        L.load_pool(ctx, stream, 0, 256, 128, DeviceBuffer(total - 256))
    assert e.value.status == TFQ_E_INVAL
    with pytest.raises(TfqError) as e:                     # no such layer entry
        L.load_pool(ctx, stream, 1, 256, 128, pool)
    assert e.value.status == TFQ_E_INVAL
    # a short layer file
    path = os.path.join(root, "packed_experts", "layer_00.bin")
    full = open(path, "rb").read()
    open(path, "wb").write(full[:len(full) - 100])
    with pytest.raises(TfqError) as e:
        L.load_pool(ctx, stream, 0, 256, 128, pool)
    assert e.value.status == TFQ_E_IO
    os.remove(path)                                        # and a missing one
    with pytest.raises(TfqError) as e:
        L.load_pool(ctx, stream, 0, 256, 128, pool)
    assert e.value.status == TFQ_E_IO and "packed_experts/layer_00.bin" in str(e.value)


def test_pool_load_checks_the_tensors(ctx, stream, tmp_path):
    root = str(tmp_path)
    _, layout = gturbo.write_model(root, 256, 128, 2)
    pool = DeviceBuffer(ops.PackedExpertsLayout(root).pool_bytes(256, 128)[1])
    cases = [
        (lambda t: t["up"].update(bits=3), TFQ_E_UNSUPPORTED),          # widths mixed in one layer
        (lambda t: t["gate"].update(bits=8), TFQ_E_UNSUPPORTED),        # not 2, 3 or 4 bits
        (lambda t: t["down"].update(dtype="U8"), TFQ_E_UNSUPPORTED),    # not U32 words
        (lambda t: t["down_scales"].update(dtype="F16"), TFQ_E_INVAL),  # scales not BF16
        (lambda t: t["gate"].update(shape=[128, 128]), TFQ_E_INVAL),    # shape vs d, f
        (lambda t: t["up_biases"].update(offset=10 ** 9), TFQ_E_INVAL), # outside the blob
        (lambda t: t.pop("down_biases"), TFQ_E_INVAL),                  # missing sub-tensor
    ]
    import copy
    for mutate, status in cases:
        lay = copy.deepcopy(layout)
        mutate(lay["layers"][0]["experts"][1]["tensors"])
        gturbo.write_layout(root, lay)
        L = ops.PackedExpertsLayout(root)
        with pytest.raises(TfqError) as e:
            L.load_pool(ctx, stream, 0, 256, 128, pool)
        assert e.value.status == status, mutate


def test_resident_load(ctx, stream, tmp_path):
    path = str(tmp_path / "model_weights.bin")
    blob = np.random.default_rng(5).integers(0, 256, 3 * (1 << 20) + 77, dtype=np.uint8)
    blob.tofile(path)
    dst = DeviceBuffer(1 << 21)
    ops.resident_load(stream, path, 12345, (1 << 21) - 3, dst)
    got = dst.download(np.uint8, (1 << 21) - 3)
    assert np.array_equal(got, blob[12345:12345 + (1 << 21) - 3])
    with pytest.raises(TfqError) as e:
        ops.resident_load(stream, path, blob.size - 10, 11, dst)
    assert e.value.status == TFQ_E_IO
    with pytest.raises(TfqError) as e:
        ops.resident_load(stream, str(tmp_path / "absent.bin"), 0, 1, dst)
    assert e.value.status == TFQ_E_IO
