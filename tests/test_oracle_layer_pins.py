"""Pins of the decode-layer part of the CPU oracle (RMSNorm, NeoX RoPE,
attention, and the layer composition) against what fixes them independently:
the reference's own cross-check shapes (an independent scalar formulation,
as T/Validation/Reference/{RMSNorm,Attention}ReferenceTests.swift do), closed
forms and invariants chosen so that a dropped term, a wrong index or a
transposed head mapping fails one of them. CPU only."""
import numpy as np
import pytest

import oracle
from edgeexpert_amd import synth
from helpers import f16_round, from_f16_bits

IDENTITY = oracle.Tolerance.identity


def _uniform(seed, label, n, lo, hi):
    return synth.uniform24(synth.seed_key(seed, label), n, lo, hi)


# ------------------------------------------------------------------ RMSNorm ----

@pytest.mark.parametrize("d,seed", [(256, 0xA1), (512, 0xB2), (2816, 0xC3)])
def test_rmsnorm_matches_scalar_formulation(d, seed):
    # RMSNormReferenceTests.acceleratedMatchesScalar: x ~ U(-1,1), w ~ U(0.5,1.5), eps 1e-6
    u = _uniform(seed, "rmsnorm-ref", 2 * d, -1.0, 1.0)
    x = u[:d]
    w = (u[d:] + 1.0) / 2.0 + 0.5
    y = oracle.rmsnorm(x, w, 1e-6)
    ss = 0.0
    for v in x.astype(np.float64):
        ss += v * v
    inv = 1.0 / np.sqrt(ss / d + 1e-6)
    ref = np.array([x[i] * inv * w[i] for i in range(d)], np.float32)
    assert oracle.rel_error(y, ref) < IDENTITY


def test_rmsnorm_one_hot_closed_form():
    # x = a·e_j: mean(x²) = a²/n, so y_j = a·w_j / sqrt(a²/n + eps) and y_i = 0 elsewhere;
    # a weight read from the wrong index, or a sum/mean mix-up, breaks it
    n, j, a, eps = 64, 17, 3.0, 1e-6
    x = np.zeros(n, np.float32)
    x[j] = a
    w = np.linspace(0.5, 1.5, n).astype(np.float32)
    y = oracle.rmsnorm(x, w, eps)
    expect = a * w[j] / np.sqrt(a * a / n + eps)
    assert abs(y[j] - expect) <= 1e-6 * abs(expect)
    assert np.all(y[np.arange(n) != j] == 0)


def test_rmsnorm_constant_and_no_scale():
    x = np.full(128, -2.5, np.float32)
    y = oracle.rmsnorm(x, None, 1e-6)
    assert np.allclose(y, -2.5 / np.sqrt(6.25 + 1e-6), rtol=1e-6)
    small = np.array([1e-4, -1e-4, 2e-4, -2e-4] * 2, np.float32)   # smallMagnitudes
    assert np.all(np.isfinite(oracle.rmsnorm(small, np.ones(8, np.float32), 1e-6)))


# --------------------------------------------------------------------- RoPE ----

def test_rope_position_zero_is_identity():
    x = _uniform(1, "rope", 3 * 64, -1, 1)
    assert np.array_equal(oracle.rope_neox(x, 3, 64, 32, 0, 10000.0), x)


def test_rope_pair_zero_rotates_by_position_radians():
    # pair 0 has frequency theta^0 = 1: a rotation by `position` radians of (x[0], x[half])
    hd, pos = 256, 4095
    x = np.zeros(hd, np.float32)
    x[0], x[128] = 0.6, -0.8
    y = oracle.rope_neox(x, 1, hd, 128, pos, 10000.0)
    c, s = np.cos(float(pos)), np.sin(float(pos))
    assert abs(y[0] - (0.6 * c + 0.8 * s)) < 1e-6
    assert abs(y[128] - (0.6 * s - 0.8 * c)) < 1e-6
    assert np.all(y[np.r_[1:128, 129:256]] == 0)


def test_rope_neox_pairs_preserve_norm_and_pass_through():
    hd, rp = 128, 40
    x = _uniform(2, "rope-norm", 2 * hd, -1, 1)
    y = oracle.rope_neox(x, 2, hd, rp, 777, 1e6)
    for h in range(2):
        b = h * hd
        n0 = np.hypot(x[b:b + rp], x[b + 64:b + 64 + rp])
        n1 = np.hypot(y[b:b + rp], y[b + 64:b + 64 + rp])
        assert np.allclose(n0, n1, rtol=1e-6, atol=1e-7)
        # pairs >= rotated_pairs pass through unchanged (partial rotary)
        assert np.array_equal(y[b + rp:b + 64], x[b + rp:b + 64])
        assert np.array_equal(y[b + 64 + rp:b + hd], x[b + 64 + rp:b + hd])


def test_rope_angles_add():
    # rope(rope(x, a), b) == rope(x, a + b): pins the frequency of every pair
    x = _uniform(3, "rope-add", 256, -1, 1)
    ab = oracle.rope_neox(oracle.rope_neox(x, 1, 256, 128, 1000, 10000.0), 1, 256, 128, 2000, 10000.0)
    direct = oracle.rope_neox(x, 1, 256, 128, 3000, 10000.0)
    assert np.max(np.abs(ab - direct)) < 2e-6


def test_rope_frequencies_divide_by_head_dim():
    # pair i rotates by pos * theta^(-2i/hd) (proportional RoPE, RoPE.swift:73-76)
    hd, i, pos, theta = 256, 37, 100, 10000.0
    x = np.zeros(hd, np.float32)
    x[i] = 1.0
    y = oracle.rope_neox(x, 1, hd, 64, pos, theta)
    ang = pos * theta ** (-2.0 * i / hd)
    assert abs(y[i] - np.cos(ang)) < 1e-6 and abs(y[i + 128] - np.sin(ang)) < 1e-6


# ---------------------------------------------------------------- attention ----

def _attn_np(q, k, v, hd, nq, nkv, seq, window, scale):
    """Independent formulation: vectorised float64 softmax per head."""
    g = nq // nkv
    start = max(0, seq - window) if window else 0
    K = k.reshape(seq, nkv, hd).astype(np.float64)[start:]
    V = v.reshape(seq, nkv, hd).astype(np.float64)[start:]
    out = np.zeros((nq, hd))
    for h in range(nq):
        s = K[:, h // g, :] @ q.reshape(nq, hd)[h].astype(np.float64) * scale
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ V[:, h // g, :]
    return out.reshape(-1).astype(np.float32)


@pytest.mark.parametrize("hd,nq,nkv,seq,window,seed", [
    (64, 4, 2, 128, 64, 0x161), (64, 4, 2, 32, 128, 0x162), (64, 8, 1, 128, 0, 0x163),
    (128, 8, 4, 64, 0, 0x164)])
def test_attention_matches_scalar_formulation(hd, nq, nkv, seq, window, seed):
    # AttentionReferenceTests.vDSPMatchesScalar shapes and U(-0.5, 0.5) inputs
    u = _uniform(seed, f"attention-ref-h{nq}-d{hd}-T{seq}", nq * hd + 2 * seq * nkv * hd, -0.5, 0.5)
    q, k, v = u[:nq * hd], u[nq * hd:nq * hd + seq * nkv * hd], u[nq * hd + seq * nkv * hd:]
    got = oracle.attention(q, k, v, hd, nq, nkv, seq, window)
    ref = _attn_np(q, k, v, hd, nq, nkv, seq, window, 1 / np.sqrt(hd))
    assert oracle.rel_error(got, ref) < IDENTITY


def test_attention_single_key_returns_its_value():
    hd, nq, nkv = 32, 4, 2
    q = _uniform(4, "q", nq * hd, -1, 1)
    k = _uniform(4, "k", nkv * hd, -1, 1)
    v = _uniform(4, "v", nkv * hd, -1, 1)
    out = oracle.attention(q, k, v, hd, nq, nkv, 1).reshape(nq, hd)
    for h in range(nq):
        assert np.allclose(out[h], v.reshape(nkv, hd)[h // 2], atol=1e-7)


def test_attention_gqa_head_mapping_and_window():
    # V constant per (position, kv head): out[h] = Σ_j p_j c[j][h // G]; with
    # equal keys p is uniform over the window -> mean of the visible c[j][h//G]
    hd, nq, nkv, seq, window = 16, 8, 2, 50, 20
    c = _uniform(5, "c", seq * nkv, -1, 1).reshape(seq, nkv)
    v = np.repeat(c[:, :, None], hd, axis=2).reshape(-1).astype(np.float32)
    k = np.zeros(seq * nkv * hd, np.float32)
    q = _uniform(5, "q", nq * hd, -1, 1)
    out = oracle.attention(q, k, v, hd, nq, nkv, seq, window).reshape(nq, hd)
    for h in range(nq):
        assert np.allclose(out[h], c[seq - window:, h // (nq // nkv)].mean(), atol=1e-6)
    full = oracle.attention(q, k, v, hd, nq, nkv, seq, 0).reshape(nq, hd)
    assert np.allclose(full[:, 0], [c[:, h // 4].mean() for h in range(nq)], atol=1e-6)
    assert np.array_equal(oracle.attention(q, k, v, hd, nq, nkv, seq, seq), oracle.attention(q, k, v, hd, nq, nkv, seq, 0))


def test_attention_dominant_key():
    hd, seq = 64, 40
    q = np.zeros(hd, np.float32)
    q[3] = 1.0
    k = np.zeros(seq * hd, np.float32)
    k[7 * hd + 3] = 60.0           # score 60·scale for key 7, 0 elsewhere
    v = _uniform(6, "v", seq * hd, -1, 1)
    out = oracle.attention(q, k, v, hd, 1, 1, seq, 0, scale=1.0)
    assert np.allclose(out, v.reshape(seq, hd)[7], atol=1e-20 + 1e-12 * seq)


# ------------------------------------------------------------ layer (oracle) ----

SMALL = dict(d=256, nq=4, nkv=2, hd=128, rotated_pairs=64, window=0, f=128, fs=192, k=2,
             eps=1e-6, theta=10000.0, scale=1.0)


def _small_layer(scalar=0.75):
    s = SMALL
    w = synth.decode_layer(9, "pin-layer", s["d"], s["nq"], s["nkv"], s["hd"], 8, s["f"], s["fs"], scalar)
    return w


def _run(w, pos=70, cap=96, shape=SMALL):
    kvd = shape["nkv"] * shape["hd"]
    kc = synth.f16_vector(9, "kc", cap * kvd)
    vc = synth.f16_vector(9, "vc", cap * kvd)
    hidden = synth.f16_vector(9, "hidden", shape["d"])
    kc0, vc0 = kc.copy(), vc.copy()
    out, idx, wts, tr = oracle.decode_layer(w, shape, hidden, kc, vc, pos, trace=True)
    return hidden, kc0, vc0, kc, vc, out, idx, wts, tr


def _n16(x, w16, eps=1e-6):
    return f16_round(oracle.rmsnorm(x, None if w16 is None else from_f16_bits(w16), eps))


def test_layer_composition_wiring():
    """Every stage of tfo_decode_layer equals the separately pinned primitive
    applied to the previous stage's stored (fp16) buffer."""
    s = SMALL
    w = _small_layer()
    pos = 70
    hidden, kc0, vc0, kc, vc, out, idx, wts, tr = _run(w, pos)
    d, hd, nq, nkv = s["d"], s["hd"], s["nq"], s["nkv"]
    kvd = nkv * hd
    h_in = from_f16_bits(hidden)
    # only slot `pos` of the caches changes
    assert np.array_equal(np.delete(kc.reshape(-1, kvd), pos, 0), np.delete(kc0.reshape(-1, kvd), pos, 0))
    assert np.array_equal(np.delete(vc.reshape(-1, kvd), pos, 0), np.delete(vc0.reshape(-1, kvd), pos, 0))
    normed = _n16(h_in, w["input_norm"])
    q_raw = f16_round(oracle.gemv_int4(*w["q"], normed))
    k_raw = f16_round(oracle.gemv_int4(*w["k"], normed))
    v_raw = f16_round(oracle.gemv_int4(*w["v"], normed))
    qn = np.concatenate([_n16(q_raw[h * hd:(h + 1) * hd], w["q_norm"]) for h in range(nq)])
    kn = np.concatenate([_n16(k_raw[h * hd:(h + 1) * hd], w["k_norm"]) for h in range(nkv)])
    vn = np.concatenate([_n16(v_raw[h * hd:(h + 1) * hd], None) for h in range(nkv)])
    q = f16_round(oracle.rope_neox(qn, nq, hd, s["rotated_pairs"], pos, s["theta"]))
    k = f16_round(oracle.rope_neox(kn, nkv, hd, s["rotated_pairs"], pos, s["theta"]))
    assert np.array_equal(from_f16_bits(tr["q"]), q)
    assert np.array_equal(from_f16_bits(kc.reshape(-1, kvd)[pos]), k)
    assert np.array_equal(from_f16_bits(vc.reshape(-1, kvd)[pos]), vn)
    K, V = from_f16_bits(kc[:(pos + 1) * kvd]), from_f16_bits(vc[:(pos + 1) * kvd])
    attn = f16_round(oracle.attention(q, K, V, hd, nq, nkv, pos + 1, 0, s["scale"]))
    assert np.array_equal(from_f16_bits(tr["attn"]), attn)
    o = f16_round(oracle.gemv_int4(*w["o"], attn))
    assert np.array_equal(from_f16_bits(tr["o"]), o)
    h = f16_round(h_in + _n16(o, w["post_attention_norm"]))
    assert np.array_equal(from_f16_bits(tr["h"]), h)
    logits = oracle.router_logits(w["router_w"], w["router_s"], w["router_b"], _n16(h, None),
                                  from_f16_bits(w["router_eff"]))
    ridx, rw = oracle.topk_softmax(logits, s["k"], from_f16_bits(w["router_gain"]))
    assert list(idx) == list(ridx)
    assert np.array_equal(wts, f16_round(rw))
    sh = (w["shared_gate"], w["shared_up"], w["shared_down"])
    h1 = f16_round(oracle.shared_expert_int4(*sh, _n16(h, w["pre_ffn_norm"]), d, s["fs"]))
    assert np.array_equal(from_f16_bits(tr["h1"]), h1)
    h2 = f16_round(oracle.moe_routed(w["pool"], w["stride"], w["off"], _n16(h, w["pre_ffn2_norm"]), ridx,
                                     f16_round(rw), d, s["f"]))
    assert np.array_equal(from_f16_bits(tr["h2"]), h2)
    h12 = f16_round(_n16(h1, w["post_ffn1_norm"]) + _n16(h2, w["post_ffn2_norm"]))
    res = f16_round(h + _n16(h12, w["post_ffn_norm"]))
    expect = f16_round(res * f16_round(np.float32(w["layer_scalar"])))
    assert np.array_equal(from_f16_bits(out), expect)


def test_layer_scalar_zero_and_zero_ffn_norm():
    w = _small_layer(scalar=0.0)
    out = _run(w)[5]
    assert np.all(from_f16_bits(out) == 0)
    w = _small_layer(scalar=1.0)
    w["post_ffn_norm"] = np.zeros_like(w["post_ffn_norm"])      # FFN branch contributes 0
    _, _, _, _, _, out, _, _, tr = _run(w)
    assert np.array_equal(out, tr["h"])                          # out = h·1


def test_layer_position_zero_attends_to_itself():
    # at position 0 the only key is the new token: attn[h] = v_new[h // G]
    w = _small_layer()
    _, _, _, kc, vc, _, _, _, tr = _run(w, pos=0)
    kvd = SMALL["nkv"] * SMALL["hd"]
    vnew = from_f16_bits(vc[:kvd]).reshape(SMALL["nkv"], SMALL["hd"])
    attn = from_f16_bits(tr["attn"]).reshape(SMALL["nq"], SMALL["hd"])
    for h in range(SMALL["nq"]):
        assert np.array_equal(attn[h], f16_round(vnew[h // 2]))
