"""The packed-experts layout reader (tfq_expert_layout_load) on the CPU:
the reference reader's contract (S/Infrastructure/ModelIO/PackedExpertsLayout.swift:55-137)
on layouts written as the repacker writes them (gturbo.py), and each of its
error cases. Loading into device memory is covered by test_gpu_loader.py."""
import copy
import json

import pytest

import gturbo
from edgeexpert_amd import ops
from edgeexpert_amd._lib import TfqError, TFQ_E_INVAL, TFQ_E_IO


def _layout(tmp_path, d=128, f=64, experts=4, layers=2, order=None):
    return gturbo.write_model(str(tmp_path), d, f, experts, layers=layers, physical_order=order)


def test_reads_the_repacker_layout(tmp_path):
    _, layout = _layout(tmp_path, order=[2, 0, 3, 1])
    L = ops.PackedExpertsLayout(str(tmp_path))
    assert (L.expert_stride, L.num_layers, L.experts_per_layer, L.layer_entries) == (
        layout["expertStride"], 2, 4, 2)
    for e in range(4):
        rank, off, size = L.expert(1, e)
        assert rank == [2, 0, 3, 1].index(e) and off == rank * L.expert_stride and size == L.expert_stride
    offs, name = L.routed_expert_offsets(0)
    plan, _ = gturbo.blob_plan(128, 64)
    want = {k: off for k, off, *_ in plan}
    assert name == "layer_00.bin"
    assert offs == {"gate_w": want["gate"], "gate_s": want["gate_scales"], "gate_b": want["gate_biases"],
                    "up_w": want["up"], "up_s": want["up_scales"], "up_b": want["up_biases"],
                    "down_w": want["down"], "down_s": want["down_scales"], "down_b": want["down_biases"]}
    with pytest.raises(TfqError) as e:
        L.expert(2, 0)
    assert e.value.status == TFQ_E_INVAL
    L.close()


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_pool_bytes_follow_the_code_width(tmp_path, bits):
    d, f, E = 256, 128, 4
    gturbo.write_model(str(tmp_path), d, f, E, bits=bits)
    L = ops.PackedExpertsLayout(str(tmp_path))
    stride, total = L.pool_bytes(d, f)
    blob = 3 * f * d * bits // 8 + 4 * f * (d // 64) * 2 + 2 * d * (f // 64) * 2
    assert stride == (blob + 255) // 256 * 256 and total == E * stride
    offs, _ = L.routed_expert_offsets(0)
    plan, _ = gturbo.blob_plan(d, f, bits)
    assert offs["up_w"] == dict((k, o) for k, o, *_ in plan)["up"]


def test_missing_expert_and_rank_keys_take_the_reader_defaults(tmp_path):
    _, layout = _layout(tmp_path, layers=1)
    lay = copy.deepcopy(layout)
    for ex in lay["layers"][0]["experts"]:
        del ex["expert"], ex["physicalRank"]          # ids = entries placed so far, rank = id
    gturbo.write_layout(str(tmp_path), lay)
    L = ops.PackedExpertsLayout(str(tmp_path))
    assert [L.expert(0, e)[0] for e in range(4)] == [0, 1, 2, 3]


def test_missing_layout_is_an_io_error(tmp_path):
    with pytest.raises(TfqError) as e:
        ops.PackedExpertsLayout(str(tmp_path))
    assert e.value.status == TFQ_E_IO and "packed_experts/layout.json" in str(e.value)


def test_size_cap(tmp_path):
    _layout(tmp_path, layers=1)
    with pytest.raises(TfqError) as e:
        ops.PackedExpertsLayout(str(tmp_path), max_bytes=100)
    assert e.value.status == TFQ_E_INVAL and "exceeds metadata cap 100" in str(e.value)


def _mutated(tmp_path, mutate):
    _, layout = _layout(tmp_path, layers=1)
    lay = copy.deepcopy(layout)
    mutate(lay)
    gturbo.write_layout(str(tmp_path), lay)
    with pytest.raises(TfqError) as e:
        ops.PackedExpertsLayout(str(tmp_path))
    assert e.value.status == TFQ_E_INVAL
    return str(e.value)


def _ex(lay, i=0):
    return lay["layers"][0]["experts"][i]


@pytest.mark.parametrize("mutate,detail", [
    (lambda l: l.pop("expertStride"), "missing top-level keys"),
    (lambda l: l.update(numLayers="2"), "missing top-level keys"),
    (lambda l: l.update(layers=[1]), "missing top-level keys"),
    (lambda l: l["layers"][0].pop("file"), "malformed layer entry"),
    (lambda l: l["layers"][0].update(layer=1.5), "malformed layer entry"),
    (lambda l: _ex(l).pop("tensors"), "malformed expert entry"),
    (lambda l: _ex(l).update(offset="0"), "malformed expert entry"),
    (lambda l: _ex(l)["tensors"]["up"].pop("dtype"), "malformed tensor up"),
    (lambda l: _ex(l)["tensors"]["down_scales"].update(shape=[64, 1.5]), "malformed tensor down_scales"),
    (lambda l: _ex(l)["tensors"]["gate"].update(bits="4"), "malformed tensor bits gate"),
    (lambda l: _ex(l).update(expert=4), "expert id out of range"),
    (lambda l: _ex(l).update(expert=-1), "expert id out of range"),
    (lambda l: _ex(l).update(physicalRank=4), "physicalRank out of range"),
    (lambda l: _ex(l, 1).update(expert=0), "missing expert entries"),
    (lambda l: l["layers"][0]["experts"].pop(), "missing expert entries"),
])
def test_malformed_layouts(tmp_path, mutate, detail):
    assert detail in _mutated(tmp_path, mutate)


def test_not_json(tmp_path):
    gturbo.write_layout(str(tmp_path), '{"expertStride": 16384, "layers": [')
    with pytest.raises(TfqError) as e:
        ops.PackedExpertsLayout(str(tmp_path))
    assert e.value.status == TFQ_E_INVAL and "layout.json:" in str(e.value)


def test_json_reader_edge_cases(tmp_path):
    # integral floats are integers (NSNumber bridging), strings with escapes are fine
    text = json.dumps({"expertStride": 16384.0, "numLayers": 1, "expertsPerLayer": 1, "layers": [
        {"layer": 0, "file": "layer_é.bin", "experts": [
            {"offset": 0, "size": 16384, "tensors": {"gate": {"offset": 0, "size": 8, "dtype": "U32",
                                                            "shape": [1, 16], "bits": 4}}}]}]})
    gturbo.write_layout(str(tmp_path), text)
    L = ops.PackedExpertsLayout(str(tmp_path))
    assert L.expert_stride == 16384 and L.routed_expert_offsets(0)[1] == "layer_é.bin"
