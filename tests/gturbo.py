"""Writes small repacked (.gturbo) model directories for the loader tests, in
the reference's on-disk form: packed_experts/layout.json as
GTurboJSON.swift:90-155 writes it and one file per layer whose expert blobs
follow RepackPlanner.planLayerFile (RepackPlanner.swift:363-438): for role
gate, up, down the U32 weights, then BF16 scales, then BF16 biases, the blob
padded to 16 KiB pages, expert e at physicalRank(e) * stride. bits 2 / 3
write weights as TurboFieldfareRebits does (Rebits/main.swift:418-441): same
U32 dtype and logical shape, `bits` set, rows of cols*bits/8 bytes."""
import json
import os

import numpy as np

from edgeexpert_amd import synth

PAGE = 16384                   # Layout.pageBytes (RepackPlanner.swift:5-7)
ROLES = ("gate", "up", "down")


def expert_tensors(seed, layer, e, d, f, bits=4):
    """(packed u8 weights, bf16 scales, bf16 biases) per role of one expert."""
    out = {}
    for role in ROLES:
        rows, cols = (f, d) if role != "down" else (d, f)
        W, S16, B16 = synth.affine_matrix(seed, f"gturbo/l{layer}/e{e}/{role}", rows, cols, bits)
        # the checkpoint keeps BF16 scales/biases: the values of the fp16 draws,
        # rounded to BF16 (fp16 holds every BF16 value in this range exactly)
        s = synth.bf16_bits(synth.f16_to_f32(S16))
        b = synth.bf16_bits(synth.f16_to_f32(B16))
        out[role] = (W, s.reshape(rows, cols // 64), b.reshape(rows, cols // 64))
    return out


def blob_plan(d, f, bits=4):
    """[(key, offset, size, dtype, shape, bits)] in blob order, and the stride."""
    plan, cur = [], 0
    for role in ROLES:
        rows, cols = (f, d) if role != "down" else (d, f)
        wsz, ssz = rows * cols * bits // 8, rows * (cols // 64) * 2
        plan.append((role, cur, wsz, "U32", [rows, cols], bits))
        cur += wsz
        plan.append((role + "_scales", cur, ssz, "BF16", [rows, cols // 64], None))
        cur += ssz
        plan.append((role + "_biases", cur, ssz, "BF16", [rows, cols // 64], None))
        cur += ssz
    return plan, (cur + PAGE - 1) // PAGE * PAGE


def write_model(root, d, f, experts, layers=1, seed=7, physical_order=None, bits=4):
    """Writes root/packed_experts/{layout.json, layer_XX.bin}; returns
    {(layer, expert): tensors} and the layout dict."""
    pe = os.path.join(root, "packed_experts")
    os.makedirs(pe, exist_ok=True)
    plan, stride = blob_plan(d, f, bits)
    order = list(physical_order) if physical_order is not None else list(range(experts))
    rank = {e: r for r, e in enumerate(order)}            # logical expert -> physical rank
    data, layers_json = {}, []
    for layer in range(layers):
        name = f"layer_{layer:02d}.bin"
        buf = np.zeros(experts * stride, np.uint8)
        entries = []
        for e in range(experts):
            t = expert_tensors(seed, layer, e, d, f, bits)
            data[(layer, e)] = t
            base = rank[e] * stride
            tensors = {}
            for key, off, size, dtype, shape, tbits in plan:
                role = key.split("_")[0]
                arr = t[role][0] if dtype == "U32" else t[role][1 if key.endswith("scales") else 2]
                raw = np.ascontiguousarray(arr).view(np.uint8).ravel()
                assert raw.size == size
                buf[base + off:base + off + size] = raw
                entry = {"offset": off, "size": size, "dtype": dtype, "shape": shape}
                if tbits is not None:
                    entry["bits"] = tbits
                tensors[key] = entry
            entries.append({"expert": e, "physicalRank": rank[e], "offset": base, "size": stride,
                            "tensors": tensors})
        buf.tofile(os.path.join(pe, name))
        layers_json.append({"layer": layer, "file": name, "experts": entries})
    layout = {"expertStride": stride, "numLayers": layers, "expertsPerLayer": experts, "layers": layers_json}
    with open(os.path.join(pe, "layout.json"), "w") as fh:
        json.dump(layout, fh)
    return data, layout


def write_layout(root, layout_obj_or_text):
    pe = os.path.join(root, "packed_experts")
    os.makedirs(pe, exist_ok=True)
    with open(os.path.join(pe, "layout.json"), "w") as fh:
        fh.write(layout_obj_or_text if isinstance(layout_obj_or_text, str) else json.dumps(layout_obj_or_text))
