"""Seeded synthetic inputs for the BASELINE configurations (host side, numpy).

The streams are the reference's own test PRNG: SplitMix64 seeded through
SeedTree's FNV-1a label hash (V/PRNG/SplitMix64.swift:11-23,
V/PRNG/SeedTree.swift:12-19 in the reference checkout). SplitMix64 is a
counter-based generator — output i of a stream seeded with `key` is
mix(key + (i + 1) * GAMMA) — so a whole stream is produced with one vectorised
numpy expression instead of a Python loop.

Tensor streams are named "<config>/<tensor>" under SeedTree(seed), so each
tensor can be regenerated independently and the GPU and the CPU see the same
bits. Distributions follow BASELINE.json:
  int4 weights: q ~ U{0..15} (each SplitMix64 output supplies 8 packed
                bytes, i.e. 16 codes, little-endian); scale = |N(0, 0.02)| (fp16);
                bias = -8*scale + N(0, 0.002) (fp16), one pair per 64 along K.
  int8 router:  q ~ U{0..255} (8 codes per output); scale = |N(0, 0.02)|/16; bias = -128*scale + N(0, 0.002).
  activations:  N(0, 1), rounded to fp16 (or bf16 for the prefill GEMM).
Normals use Box–Muller on two 24-bit uniforms, evaluated in float64.
"""
from __future__ import annotations

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
MASK64 = (1 << 64) - 1
GROUP = 64


def seed_key(root: int, label: str) -> int:
    """SeedTree(root).key(label) -> initial SplitMix64 state."""
    h = 0xCBF29CE484222325
    for byte in label.encode():
        h ^= byte
        h = (h * 0x100000001B3) & MASK64
    return (root ^ h) & MASK64


def splitmix64(key: int, n: int, start: int = 0) -> np.ndarray:
    """Outputs start .. start+n-1 of the SplitMix64 stream seeded with `key`."""
    with np.errstate(over="ignore"):
        i = np.arange(start + 1, start + n + 1, dtype=np.uint64)
        z = np.uint64(key) + i * GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform24(key: int, n: int, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    """SplitMix64.uniform(lo, hi): lo + (hi - lo) * (next() >> 40) / 2^24, in float32."""
    u = (splitmix64(key, n) >> np.uint64(40)).astype(np.float32) / np.float32(1 << 24)
    return np.float32(lo) + (np.float32(hi) - np.float32(lo)) * u


def normal(key: int, n: int, std: float = 1.0) -> np.ndarray:
    """Box–Muller over output pairs (2i, 2i+1); float32 result."""
    r = splitmix64(key, 2 * n) >> np.uint64(40)
    u1 = (r[0::2].astype(np.float64) + 1.0) / float(1 << 24)      # (0, 1]
    u2 = r[1::2].astype(np.float64) / float(1 << 24)              # [0, 1)
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return (z * std).astype(np.float32)


def f16_bits(x) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def bf16_bits(x) -> np.ndarray:
    """Round-half-even to bfloat16 (Quantization.swift:16-23 rounding)."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    lsb = (u >> np.uint64(16)) & np.uint64(1)
    return ((u + np.uint64(0x7FFF) + lsb) >> np.uint64(16)).astype(np.uint16)


def bf16_to_f32(bits) -> np.ndarray:
    return (np.asarray(bits, np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def f16_to_f32(bits) -> np.ndarray:
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


def pack_int4(q: np.ndarray) -> np.ndarray:
    """Codes [..., K] (0..15) -> bytes [..., K/2]; low nibble = even element.
    Equivalently 8 nibbles per little-endian uint32 word along K."""
    q = np.asarray(q, np.uint8)
    return (q[..., 0::2] | (q[..., 1::2] << 4)).astype(np.uint8)


def unpack_int4(packed: np.ndarray) -> np.ndarray:
    p = np.asarray(packed, np.uint8)
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), np.uint8)
    out[..., 0::2] = p & 0x0F
    out[..., 1::2] = p >> 4
    return out


def int4_matrix(seed: int, label: str, rows: int, k: int):
    """Affine int4 g64 matrix [rows][k] with the BASELINE distributions.
    Returns (packed u8 [rows][k/2], scales fp16 bits [rows][k/64], biases fp16 bits)."""
    assert k % GROUP == 0
    # Each 64-bit output is 8 packed bytes = 16 uniform codes, in memory order.
    packed = splitmix64(seed_key(seed, label + "/q"), rows * k // 16).view(np.uint8)
    packed = packed.reshape(rows, k // 2)
    g = rows * (k // GROUP)
    s = np.abs(normal(seed_key(seed, label + "/s"), g, 0.02))
    s16 = f16_bits(s)
    b = np.float32(-8.0) * f16_to_f32(s16) + normal(seed_key(seed, label + "/b"), g, 0.002)
    return packed, s16.reshape(rows, -1), f16_bits(b).reshape(rows, -1)


def affine_matrix(seed: int, label: str, rows: int, k: int, bits: int):
    """Affine g64 matrix of `bits`-bit codes (2, 3 or 4; rows of k*bits/8 bytes,
    codes packed from the least significant bit). bits == 4 is int4_matrix.
    Uniform random bytes are uniform codes at every width; scale =
    |N(0,0.02)|·16/2^bits and bias = -2^(bits-1)·scale + N(0, 0.002) keep the
    weights' spread that of the int4 matrices."""
    if bits == 4:
        return int4_matrix(seed, label, rows, k)
    assert bits in (2, 3) and k % GROUP == 0
    nbytes = rows * k * bits // 8
    packed = splitmix64(seed_key(seed, label + "/q"), (nbytes + 7) // 8).view(np.uint8)[:nbytes]
    g = rows * (k // GROUP)
    s = np.abs(normal(seed_key(seed, label + "/s"), g, 0.02)) * np.float32(16 >> bits)
    s16 = f16_bits(s)
    b = np.float32(-(1 << (bits - 1))) * f16_to_f32(s16) + normal(seed_key(seed, label + "/b"), g, 0.002)
    return packed.reshape(rows, -1), s16.reshape(rows, -1), f16_bits(b).reshape(rows, -1)


def int8_matrix(seed: int, label: str, rows: int, k: int):
    """Affine int8 g64 router matrix: q ~ U{0..255}, scale = |N(0,0.02)|/16,
    bias = -128*scale + N(0, 0.002) (fp16)."""
    assert k % GROUP == 0
    # Each 64-bit output is 8 uniform byte codes, in memory order.
    q = splitmix64(seed_key(seed, label + "/q"), rows * k // 8).view(np.uint8)
    g = rows * (k // GROUP)
    s = np.abs(normal(seed_key(seed, label + "/s"), g, 0.02)) / np.float32(16.0)
    s16 = f16_bits(s)
    b = np.float32(-128.0) * f16_to_f32(s16) + normal(seed_key(seed, label + "/b"), g, 0.002)
    return q.reshape(rows, k), s16.reshape(rows, -1), f16_bits(b).reshape(rows, -1)


def f16_vector(seed: int, label: str, n: int, std: float = 1.0) -> np.ndarray:
    return f16_bits(normal(seed_key(seed, label), n, std))


def bf16_vector(seed: int, label: str, n: int, std: float = 1.0) -> np.ndarray:
    return bf16_bits(normal(seed_key(seed, label), n, std))


# ------------------------------------------------------------------ experts ----

def expert_layout(d: int, f: int, align: int = 16384, bits: int = 4):
    """Blob layout of one routed expert: [gateW, gateS, gateB, upW, upS, upB,
    downW, downS, downB], each sub-tensor contiguous, blob padded to `align`
    (the repacker's 16 KiB expert stride); weights of `bits`-bit codes.
    Returns (offsets dict, stride)."""
    gw = f * d * bits // 8
    gs = f * (d // GROUP) * 2
    dw = d * f * bits // 8
    ds = d * (f // GROUP) * 2
    o = {}
    cur = 0
    for name, size in (("gate_w", gw), ("gate_s", gs), ("gate_b", gs), ("up_w", gw), ("up_s", gs),
                       ("up_b", gs), ("down_w", dw), ("down_s", ds), ("down_b", ds)):
        o[name] = cur
        cur += size
    stride = (cur + align - 1) // align * align
    return o, stride


OFFSET_ORDER = ("gate_w", "gate_s", "gate_b", "up_w", "up_s", "up_b", "down_w", "down_s", "down_b")


def expert_blob(seed: int, label: str, d: int, f: int, offsets: dict, stride: int,
                bits: int = 4) -> np.ndarray:
    """One expert blob of `stride` bytes with BASELINE-distributed gate/up/down."""
    blob = np.zeros(stride, np.uint8)
    for proj, rows, cols in (("gate", f, d), ("up", f, d), ("down", d, f)):
        w, s, b = affine_matrix(seed, f"{label}/{proj}", rows, cols, bits)
        for part, arr in (("w", w), ("s", s), ("b", b)):
            raw = np.ascontiguousarray(arr).view(np.uint8).ravel()
            off = offsets[f"{proj}_{part}"]
            blob[off:off + raw.size] = raw
    return blob


def expert_pool(seed: int, label: str, num_experts: int, d: int, f: int, align: int = 16384,
                bits: int = 4):
    """All experts of one layer, concatenated at a fixed stride."""
    offsets, stride = expert_layout(d, f, align, bits)
    pool = np.zeros(num_experts * stride, np.uint8)
    for e in range(num_experts):
        pool[e * stride:(e + 1) * stride] = expert_blob(seed, f"{label}/e{e}", d, f, offsets, stride, bits)
    return pool, offsets, stride


def blob_views(blob: np.ndarray, offsets: dict, d: int, f: int, proj: str, bits: int = 4):
    """(W u8 [rows][cols*bits/8], S u16 [rows][cols/64], B u16) views into one expert blob."""
    rows, cols = (f, d) if proj in ("gate", "up") else (d, f)
    rb = cols * bits // 8
    w = blob[offsets[f"{proj}_w"]:offsets[f"{proj}_w"] + rows * rb].reshape(rows, rb)
    ng = rows * (cols // GROUP)
    s = blob[offsets[f"{proj}_s"]:offsets[f"{proj}_s"] + 2 * ng].view(np.uint16).reshape(rows, -1)
    b = blob[offsets[f"{proj}_b"]:offsets[f"{proj}_b"] + 2 * ng].view(np.uint16).reshape(rows, -1)
    return w, s, b


# ---------------------------------------------------------------- routing ----

def zipf_routing(seed: int, label: str, tokens: int, num_experts: int, top_k: int, s: float = 1.1):
    """Skewed prefill routing: expert popularity p ∝ r^-s
    over a seeded rank permutation; each token takes top_k distinct experts
    by Gumbel-top-k over log p, ties to the lower expert index; its weights are
    the softmax of the selected perturbed logits, rounded to fp16.
    Returns (indices u32 [tokens][top_k], weights fp16 bits [tokens][top_k])."""
    perm = np.argsort(uniform24(seed_key(seed, label + "/perm"), num_experts), kind="stable")
    rank_of = np.empty(num_experts, np.int64)
    rank_of[perm] = np.arange(num_experts)
    logp = -s * np.log(rank_of + 1.0)
    u = (splitmix64(seed_key(seed, label + "/gumbel"), tokens * num_experts) >> np.uint64(11))
    u = (u.astype(np.float64) + 0.5) / float(1 << 53)                 # (0, 1)
    z = logp[None, :] + (-np.log(-np.log(u))).reshape(tokens, num_experts)
    order = np.lexsort((np.broadcast_to(np.arange(num_experts), z.shape), -z), axis=1)
    idx = order[:, :top_k].astype(np.uint32)
    sel = np.take_along_axis(z, order[:, :top_k], axis=1)
    w = np.exp(sel - sel[:, :1])
    w = (w / w.sum(axis=1, keepdims=True)).astype(np.float32)
    return idx, f16_bits(w)


def norm_weight(seed: int, label: str, n: int, lo: float = 0.5, hi: float = 1.5) -> np.ndarray:
    """RMSNorm weight vector (fp16 bits), uniform in [lo, hi)."""
    return f16_bits(uniform24(seed_key(seed, label), n, lo, hi))


def decode_layer(seed: int, label: str, d: int, nq: int, nkv: int, hd: int, num_experts: int,
                 f: int, fs: int, layer_scalar: float = 0.75, expert_bits: int = 4,
                 shared_bits: int = 4, v_proj: bool = True) -> dict:
    """Weights of one Gemma 4 decoder layer with the BASELINE distributions:
    int4 g64 projections as in config 0, an int8 g64 router, num_experts
    routed experts in one pool, a shared expert of int4 (config 0
    distributions) or int8 rows (shared_bits 8, the router's distributions),
    and RMSNorm weights uniform in [0.5, 1.5) (so that a weight applied to
    the wrong element is visible). Keys follow the CPU oracle's
    tfo_layer_weights."""
    shared = int4_matrix if shared_bits == 4 else int8_matrix
    L = label
    qd, kvd = nq * hd, nkv * hd
    w = {
        "input_norm": norm_weight(seed, L + "/input_norm", d),
        "q": int4_matrix(seed, L + "/q", qd, d),
        "k": int4_matrix(seed, L + "/k", kvd, d),
        "v": int4_matrix(seed, L + "/v", kvd, d) if v_proj else None,
        "o": int4_matrix(seed, L + "/o", d, qd),
        "q_norm": norm_weight(seed, L + "/q_norm", hd),
        "k_norm": norm_weight(seed, L + "/k_norm", hd),
        "post_attention_norm": norm_weight(seed, L + "/post_attention_norm", d),
        "pre_ffn_norm": norm_weight(seed, L + "/pre_ffn_norm", d),
        "pre_ffn2_norm": norm_weight(seed, L + "/pre_ffn2_norm", d),
        "post_ffn1_norm": norm_weight(seed, L + "/post_ffn1_norm", d),
        "post_ffn2_norm": norm_weight(seed, L + "/post_ffn2_norm", d),
        "post_ffn_norm": norm_weight(seed, L + "/post_ffn_norm", d),
        "shared_gate": shared(seed, L + "/shared_gate", fs, d),
        "shared_up": shared(seed, L + "/shared_up", fs, d),
        "shared_down": shared(seed, L + "/shared_down", d, fs),
        "shared_bits": shared_bits,
        "num_experts": num_experts,
        "layer_scalar": layer_scalar,
    }
    rw, rs, rb = int8_matrix(seed, L + "/router", num_experts, d)
    w.update(router_w=rw, router_s=rs, router_b=rb,
             router_eff=norm_weight(seed, L + "/router_eff", d),
             router_gain=norm_weight(seed, L + "/router_gain", num_experts))
    pool, offsets, stride = expert_pool(seed, L + "/experts", num_experts, d, f, bits=expert_bits)
    w.update(pool=pool, off=offsets, stride=stride, expert_bits=expert_bits)
    return w
