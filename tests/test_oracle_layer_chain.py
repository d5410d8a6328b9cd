"""The stage-by-stage restatement of the oracle's decoder layer
(tests/layer_chain.py) against tfo_decode_layer, and the spread of the
oracle's own chain under fp32-sized perturbations (CPU only).

The restatement must equal the oracle bit for bit without perturbation, or
the spread it measures would belong to some other chain. The spread at
config 4 with the int8 shared expert exceeds 1e-3 end to end while the
perturbation is ~2 fp32 ulps: the end-to-end RelError of any implementation
that rounds at the reference's ten fp16 points is only defined to within
that spread (the GPU layer test allows exactly it)."""
import numpy as np
import pytest

import oracle
from edgeexpert_amd import synth
from helpers import from_f16_bits
from layer_chain import chain, chain_floor

SMALL = dict(d=256, nq=4, nkv=2, hd=128, rotated_pairs=64, window=0, f=128, fs=192, k=2,
             eps=1e-6, theta=10000.0, scale=1.0)
CONFIG4 = dict(d=2816, nq=16, nkv=8, hd=256, rotated_pairs=128, window=0, f=704, fs=2112, k=8,
               eps=1e-6, theta=10000.0, scale=1.0)
SMALL_FULL = dict(d=256, nq=8, nkv=1, hd=512, rotated_pairs=64, window=0, f=128, fs=192, k=2,
                  eps=1e-6, theta=1e6, scale=1.0)


def _case(shape, E, pos, cap, seed, label, **kw):
    w = synth.decode_layer(seed, label, shape["d"], shape["nq"], shape["nkv"], shape["hd"], E, shape["f"],
                           shape["fs"], **kw)
    kvd = shape["nkv"] * shape["hd"]
    kc = synth.f16_vector(seed, label + "/kc", cap * kvd)
    vc = synth.f16_vector(seed, label + "/vc", cap * kvd)
    hidden = synth.f16_vector(seed, label + "/hidden", shape["d"])
    return w, kc, vc, hidden


@pytest.mark.parametrize("shape,pos,kw", [
    (SMALL, 70, {}),
    (SMALL, 0, {}),
    (dict(SMALL, window=64, rotated_pairs=16, theta=1e6), 200, {}),
    (SMALL, 70, dict(shared_bits=8)),
    (SMALL, 70, dict(expert_bits=3)),
    (SMALL, 70, dict(expert_bits=2)),
    (SMALL_FULL, 70, dict(v_proj=False)),
])
def test_chain_equals_oracle_layer(shape, pos, kw):
    w, kc, vc, hidden = _case(shape, 8, pos, max(pos + 1, 160), 3, f"chain-{pos}", **kw)
    kc_ref, vc_ref = kc.copy(), vc.copy()
    out, idx, wts, tr = oracle.decode_layer(w, shape, hidden, kc_ref, vc_ref, pos, trace=True)
    c = chain(w, shape, hidden, kc, vc, pos)
    kvd = shape["nkv"] * shape["hd"]
    assert list(c["idx"]) == list(idx)
    assert np.array_equal(c["rw"], wts)
    for key in ("attn", "o", "h", "h1", "h2"):
        assert np.array_equal(c[key], from_f16_bits(tr[key])), key
    assert np.array_equal(c["kslot"], from_f16_bits(kc_ref[pos * kvd:(pos + 1) * kvd]))
    assert np.array_equal(c["vslot"], from_f16_bits(vc_ref[pos * kvd:(pos + 1) * kvd]))
    assert np.array_equal(c["out"], from_f16_bits(out))
    # the inputs are left as they were
    assert np.array_equal(kc, synth.f16_vector(3, f"chain-{pos}/kc", kc.size))


def test_perturbation_moves_the_chain_by_fp16_flips():
    # perturbed at fp32 size, the first stage (the new k slot) moves by at
    # most one fp16 ulp per element, and some seed moves the output
    w, kc, vc, hidden = _case(SMALL, 8, 70, 160, 3, "chain-70")
    base = chain(w, SMALL, hidden, kc, vc, 70)
    moved = False
    for t in range(6):
        p = chain(w, SMALL, hidden, kc, vc, 70, np.random.default_rng(t))
        ulp = np.abs(np.nextafter(base["kslot"].astype(np.float16), np.float16(np.inf)).astype(np.float32)
                     - base["kslot"])
        assert np.all(np.abs(p["kslot"] - base["kslot"]) <= ulp)
        moved |= not np.array_equal(p["out"], base["out"])
    assert moved


def test_config4_chain_spread_exceeds_the_north_star_bar():
    # config 4, int8 shared expert (seed/label as test_gpu_layer.py): the
    # oracle's chain against itself, 12 perturbations of ~2 fp32 ulps
    w, kc, vc, hidden = _case(CONFIG4, 128, 4095, 4096, 9, "c4-s8", shared_bits=8)
    floor, trials = chain_floor(w, CONFIG4, hidden, kc, vc, 4095, trials=12)
    assert floor > 1e-3, trials
    assert floor < oracle.Tolerance.fp16_chained_reduction, trials


def test_layer_without_v_projection_equals_k_proj_as_v():
    # the full-attention layers run the fused QKV with k_proj as the v
    # projection (RealForwardRunner.swift:2252-2255): the oracle without a v
    # matrix must equal the oracle given k's matrix as v, bit for bit, and
    # differ from a layer with a v matrix of its own (position 0: the new
    # token is the only key, so the output is its V)
    for pos in (0, 70):
        w, kc, vc, hidden = _case(SMALL_FULL, 8, pos, 160, 3, "full-v", v_proj=False)
        a = oracle.decode_layer(w, SMALL_FULL, hidden, kc.copy(), vc.copy(), pos)[0]
        b = oracle.decode_layer(dict(w, v=w["k"]), SMALL_FULL, hidden, kc.copy(), vc.copy(), pos)[0]
        assert np.array_equal(a, b)
    w, kc, vc, hidden = _case(SMALL_FULL, 8, 0, 160, 3, "full-v", v_proj=False)
    wv = synth.decode_layer(3, "full-v", SMALL_FULL["d"], SMALL_FULL["nq"], SMALL_FULL["nkv"], SMALL_FULL["hd"], 8,
                            SMALL_FULL["f"], SMALL_FULL["fs"])
    a = oracle.decode_layer(w, SMALL_FULL, hidden, kc.copy(), vc.copy(), 0)[0]
    c = oracle.decode_layer(wv, SMALL_FULL, hidden, kc.copy(), vc.copy(), 0)[0]
    assert not np.array_equal(a, c)
