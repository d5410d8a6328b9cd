"""The decoder-layer chain of the CPU oracle restated stage by stage from the
oracle's primitives, with an optional perturbation of fp32 size before every
fp16 rounding point.

Unperturbed, `chain` equals `oracle.decode_layer` bit for bit (checked in
test_oracle_layer_chain.py). Perturbed, it measures how far the oracle's own
chain moves when its arithmetic changes at the level of a different fp32
summation order: `chain_floor` is the largest end-to-end RelError over a few
seeded perturbations. The decode layer stores ten fp16 intermediates (the
reference's rounding points), and a rounding that flips one fp16 ulp early in
the chain (h, the post-attention residual) passes through the routed experts'
gain (outputs ~60 from inputs ~1 with the config-0 weight distributions), so
the end-to-end RelError of two exact-arithmetic chains that differ only in
summation order is itself 7e-4 .. 1.4e-3 at config 4.

Stages follow tfo_decode_layer (oracle/tfq_oracle.c), which cites
RealForwardRunner.swift:2273-2440 and fused.metal:86-375 for each step.
"""
from __future__ import annotations

import numpy as np

import oracle
from helpers import f16_round, from_f16_bits

# relative size of the perturbation: ~2 fp32 ulps (a changed summation order
# of a well-conditioned fp32 sum); attention's softmax-weighted sums get 1e-6
# (hardware exp2 and a chunked softmax).
REL = 2e-7
REL_ATTENTION = 1e-6


def chain(w: dict, s: dict, hidden16, kc16, vc16, pos: int, rng=None):
    """One decoder layer; returns a dict of the fp16-valued stages (as float32)
    out, h, h1, h2, attn, o, kslot, vslot, and the routing idx / rw.
    kc16 / vc16 are not modified (the new slot is applied to copies)."""
    def nz(x, rel=REL):
        x = np.asarray(x, np.float32)
        if rng is None:
            return x
        return (x * (1.0 + rel * rng.standard_normal(x.shape))).astype(np.float32)

    eps, d, hd, nq, nkv = s["eps"], s["d"], s["hd"], s["nq"], s["nkv"]
    v_from_k = w.get("v") is None       # full-attention layers: V from the k projection

    def n16(x, w16):
        return f16_round(nz(oracle.rmsnorm(x, None if w16 is None else from_f16_bits(w16), eps)))

    hid = from_f16_bits(hidden16)
    xn = n16(hid, w["input_norm"])
    q = f16_round(nz(oracle.gemv_int4(*w["q"], xn)))
    k = f16_round(nz(oracle.gemv_int4(*w["k"], xn)))
    v = k if v_from_k else f16_round(nz(oracle.gemv_int4(*w["v"], xn)))
    q = np.concatenate([n16(q[h * hd:(h + 1) * hd], w["q_norm"]) for h in range(nq)])
    vn = np.concatenate([n16(v[h * hd:(h + 1) * hd], None) for h in range(nkv)])
    kn = np.concatenate([n16(k[h * hd:(h + 1) * hd], w["k_norm"]) for h in range(nkv)])
    q = f16_round(nz(oracle.rope_neox(q, nq, hd, s["rotated_pairs"], pos, s["theta"])))
    kn = f16_round(nz(oracle.rope_neox(kn, nkv, hd, s["rotated_pairs"], pos, s["theta"])))
    kvd = nkv * hd
    K = from_f16_bits(kc16[:(pos + 1) * kvd]).copy()
    V = from_f16_bits(vc16[:(pos + 1) * kvd]).copy()
    K[pos * kvd:] = kn
    V[pos * kvd:] = vn
    attn = f16_round(nz(oracle.attention(q, K, V, hd, nq, nkv, pos + 1, s["window"], s["scale"]),
                        REL_ATTENTION))
    o = f16_round(nz(oracle.gemv_int4(*w["o"], attn)))
    h = f16_round(hid + n16(o, w["post_attention_norm"]))
    logits = nz(oracle.router_logits(w["router_w"], w["router_s"], w["router_b"], n16(h, None),
                                     from_f16_bits(w["router_eff"])))
    idx, rw = oracle.topk_softmax(logits, s["k"], from_f16_bits(w["router_gain"]))
    rw = f16_round(nz(rw))
    sh = (w["shared_gate"], w["shared_up"], w["shared_down"])
    h1 = f16_round(nz(oracle.shared_expert(*sh, n16(h, w["pre_ffn_norm"]), d, s["fs"],
                                           bits=w.get("shared_bits", 4))))
    h2 = f16_round(nz(oracle.moe_routed(w["pool"], w["stride"], w["off"], n16(h, w["pre_ffn2_norm"]), idx, rw,
                                        d, s["f"], bits=w.get("expert_bits", 4))))
    h12 = f16_round(n16(h1, w["post_ffn1_norm"]) + n16(h2, w["post_ffn2_norm"]))
    out = f16_round(f16_round(h + n16(h12, w["post_ffn_norm"])) * f16_round(np.float32(w["layer_scalar"])))
    return dict(out=out, h=h, h1=h1, h2=h2, attn=attn, o=o, kslot=kn, vslot=vn, idx=idx, rw=rw)


def chain_floor(w: dict, s: dict, hidden16, kc16, vc16, pos: int, trials: int = 6):
    """End-to-end RelError of the oracle's chain against itself perturbed by
    fp32-sized noise (seeds 0..trials-1): the spread any implementation that
    rounds at the same points has to be allowed. Returns (max, per-trial list)."""
    base = chain(w, s, hidden16, kc16, vc16, pos)["out"]
    errs = [oracle.rel_error(chain(w, s, hidden16, kc16, vc16, pos, np.random.default_rng(t))["out"], base)
            for t in range(trials)]
    return max(errs), errs
