"""ctypes front end of the CPU oracle (tfq_oracle.c).

TEST INFRASTRUCTURE ONLY: this is the checker. Only tests/, the smoke() of
__graft_entry__ and the cpu_baseline leg of bench.py may import it; the
product (edgeexpert_amd, libtfq) never does.

Each wrapper names the reference function it restates (paths relative to the
reference checkout; S/ = Sources/TurboFieldfare/, V/ =
Sources/TurboFieldfareValidation/Support/, T/ = Tests/TurboFieldfare/Core/).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libtfq_oracle.so")

FMT_F16 = 0
FMT_BF16 = 1
GROUP = 64

# PrefillMoEGroupingError cases (S/Kernels/Prefill/MoE/PrefillMoEGrouping.swift:52-88)
GROUP_ERRORS = {
    1: "invalidQueryCount",
    2: "invalidTopK",
    3: "invalidNumExperts",
    4: "invalidTileExpertCount",
    5: "pairCountMismatch",
    6: "tokenOutOfRange",
    7: "rankOutOfRange",
    8: "expertOutOfRange",
    9: "duplicateTokenRank",
    10: "expertSortKeyCountMismatch",
}


def build() -> str:
    """Compile the oracle with its Makefile (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = C.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


class ExpertOffsets(C.Structure):
    """MoEExpertOffsets (S/Kernels/MoE/MoE.swift:4-29)."""
    _fields_ = [(n, C.c_uint32) for n in (
        "gate_w", "gate_s", "gate_b", "up_w", "up_s", "up_b", "down_w", "down_s", "down_b")]


PAIR_DTYPE = np.dtype([("token", "<u4"), ("expert", "<u4"), ("rank", "<u4"), ("weight_bits", "<u4")])
GROUP_DTYPE = np.dtype([("expert", "<u4"), ("pair_start", "<u4"), ("pair_count", "<u4")])
TILE_DTYPE = np.dtype([("group_start", "<u4"), ("group_count", "<u4"),
                       ("pair_start", "<u4"), ("pair_count", "<u4")])

_P = C.c_void_p


class Q4(C.Structure):
    _fields_ = [("w", _P), ("s", _P), ("b", _P)]


class LayerWeights(C.Structure):
    """tfo_layer_weights (tfq_oracle.h)."""
    _fields_ = [("input_norm", _P), ("q", Q4), ("k", Q4), ("v", Q4), ("o", Q4),
                ("q_norm", _P), ("k_norm", _P), ("post_attention_norm", _P), ("pre_ffn_norm", _P),
                ("pre_ffn2_norm", _P), ("router_w", _P), ("router_s", _P), ("router_b", _P),
                ("router_eff", _P), ("router_gain", _P), ("num_experts", C.c_int),
                ("pool", _P), ("stride", C.c_uint64), ("off", ExpertOffsets),
                ("shared_gate", Q4), ("shared_up", Q4), ("shared_down", Q4),
                ("post_ffn1_norm", _P), ("post_ffn2_norm", _P), ("post_ffn_norm", _P),
                ("layer_scalar", C.c_float), ("expert_bits", C.c_int), ("shared_bits", C.c_int)]


class LayerShape(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("d", "nq", "nkv", "hd", "rotated_pairs", "window", "f", "fs", "k")] + \
               [(n, C.c_float) for n in ("eps", "theta", "scale")]


class LayerTrace(C.Structure):
    _fields_ = [(n, _P) for n in ("q", "attn", "o", "h", "h1", "h2")]


def _declare(L):
    def d(name, res, *args):
        f = getattr(L, name)
        f.restype = res
        f.argtypes = list(args)
    u64p = C.POINTER(C.c_uint64)
    d("tfo_set_threads", None, C.c_int)
    d("tfo_splitmix64_next", C.c_uint64, u64p)
    d("tfo_splitmix64_uniform", C.c_float, u64p, C.c_float, C.c_float)
    d("tfo_seedtree_key", C.c_uint64, C.c_uint64, C.c_char_p)
    d("tfo_f32_to_bf16", C.c_uint16, C.c_float)
    d("tfo_bf16_to_f32", C.c_float, C.c_uint16)
    d("tfo_f32_to_f16", C.c_uint16, C.c_float)
    d("tfo_f16_to_f32", C.c_float, C.c_uint16)
    d("tfo_quantize_int4_row", None, _P, C.c_int, _P, _P, _P)
    d("tfo_quantize_int8_row", None, _P, C.c_int, _P, _P, _P)
    d("tfo_dequantize_int4_row", None, _P, _P, _P, C.c_int, C.c_int, _P)
    d("tfo_dequantize_int8_row", None, _P, _P, _P, C.c_int, C.c_int, _P)
    d("tfo_int4_code", C.c_uint32, _P, C.c_size_t)
    d("tfo_affine_row_bytes", C.c_size_t, C.c_size_t, C.c_int)
    d("tfo_pack_affine_code", None, _P, C.c_size_t, C.c_uint32, C.c_size_t, C.c_int)
    d("tfo_affine_code", C.c_uint32, _P, C.c_size_t, C.c_size_t, C.c_int)
    d("tfo_quantize_affine_row", None, _P, C.c_int, C.c_int, _P, _P, _P)
    d("tfo_dequantize_affine_row", None, _P, _P, _P, C.c_int, C.c_int, C.c_int, _P)
    d("tfo_gemv_affine", None, _P, _P, _P, C.c_int, C.c_int, _P, C.c_int, C.c_int, _P)
    for n in ("tfo_gemv_int4", "tfo_gemv_int8", "tfo_gemv_int4_f64", "tfo_gemv_int8_f64"):
        d(n, None, _P, _P, _P, C.c_int, _P, C.c_int, C.c_int, _P)
    d("tfo_gemv_int4_mt", None, _P, _P, _P, C.c_int, _P, C.c_int, C.c_int, _P, C.c_int)
    d("tfo_router_logits", None, _P, _P, _P, C.c_int, _P, _P, C.c_int, C.c_int, _P)
    d("tfo_topk_softmax", C.c_int, _P, C.c_int, C.c_int, _P, _P, _P)
    d("tfo_gelu_tanh", C.c_float, C.c_float)
    d("tfo_ffn_int4", None, _P, C.POINTER(ExpertOffsets), C.c_int, _P, C.c_int, C.c_int, _P)
    d("tfo_moe_routed", None, _P, C.c_uint64, C.POINTER(ExpertOffsets), C.c_int, _P, _P, _P, _P,
      C.c_int, C.c_int, C.c_int, _P)
    d("tfo_moe_routed_bits", None, _P, C.c_uint64, C.POINTER(ExpertOffsets), C.c_int, C.c_int, _P, _P, _P,
      _P, C.c_int, C.c_int, C.c_int, _P)
    for n in ("tfo_shared_expert_int4", "tfo_shared_expert_int8"):
        d(n, None, _P, _P, _P, _P, _P, _P, _P, _P, _P, C.c_int, _P, C.c_int, C.c_int, _P)
    d("tfo_shared_expert", None, _P, _P, _P, _P, _P, _P, _P, _P, _P, C.c_int, C.c_int, C.c_int, _P, C.c_int,
      C.c_int, _P)
    d("tfo_group_pairs", C.c_int, _P, C.c_int64, C.c_int64, C.c_int64, C.c_int64, C.c_int64,
      _P, C.c_int64, _P, _P, _P, _P, C.POINTER(C.c_int64), _P, C.POINTER(C.c_int64),
      C.POINTER(C.c_int64))
    d("tfo_prefill_router", C.c_int, _P, _P, _P, C.c_int, _P, C.c_int, _P, _P, C.c_int, C.c_int,
      C.c_int, C.c_int, _P, _P)
    d("tfo_grouped_route_partials", None, _P, C.c_int64, _P, C.c_int, _P, C.c_uint64,
      C.POINTER(ExpertOffsets), C.c_int, C.c_int, C.c_int, C.c_int, _P)
    d("tfo_grouped_route_partials_bits", None, _P, C.c_int64, _P, C.c_int, _P, C.c_uint64,
      C.POINTER(ExpertOffsets), C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _P)
    d("tfo_reduce_token_major", None, _P, _P, C.c_int, C.c_int, C.c_int, _P)
    d("tfo_gemm_int4", None, _P, _P, _P, C.c_int, _P, C.c_int, C.c_int, C.c_int, _P, C.c_int,
      C.c_int)
    d("tfo_gemm_affine", None, _P, _P, _P, C.c_int, C.c_int, _P, C.c_int, C.c_int, C.c_int, _P, C.c_int,
      C.c_int)
    d("tfo_rmsnorm", None, _P, _P, C.c_int, C.c_float, _P)
    d("tfo_greedy_argmax", C.c_uint32, _P, C.c_int)
    d("tfo_lm_head_greedy", C.c_uint32, _P, _P, _P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_float, _P)
    d("tfo_rope_neox", None, _P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float)
    d("tfo_attention", None, _P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, _P)
    d("tfo_decode_layer", None, C.POINTER(LayerWeights), C.POINTER(LayerShape), _P, _P, _P, C.c_int,
      _P, _P, _P, C.POINTER(LayerTrace))
    d("tfo_rel_error", C.c_float, _P, _P, C.c_size_t)
    d("tfo_max_abs_diff", C.c_float, _P, _P, C.c_size_t)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---------------------------------------------------------------- PRNG ----

class SplitMix64:
    """V/PRNG/SplitMix64.swift:4-25."""

    def __init__(self, seed: int):
        self.state = C.c_uint64(seed & 0xFFFFFFFFFFFFFFFF)

    def next(self) -> int:
        return lib().tfo_splitmix64_next(C.byref(self.state))

    def uniform(self, lo: float, hi: float) -> float:
        return lib().tfo_splitmix64_uniform(C.byref(self.state), lo, hi)

    def uniforms(self, n: int, lo: float, hi: float) -> np.ndarray:
        f = lib().tfo_splitmix64_uniform
        return np.array([f(C.byref(self.state), lo, hi) for _ in range(n)], dtype=np.float32)


def seed_tree_key(root: int, label: str) -> SplitMix64:
    """V/PRNG/SeedTree.swift:12-19."""
    return SplitMix64(lib().tfo_seedtree_key(root & 0xFFFFFFFFFFFFFFFF, label.encode()))


# --------------------------------------------------------- conversions ----

def f32_to_bf16(x: float) -> int:
    return lib().tfo_f32_to_bf16(x)


def bf16_to_f32(b: int) -> float:
    return lib().tfo_bf16_to_f32(b)


def f32_to_f16(x: float) -> int:
    return lib().tfo_f32_to_f16(x)


def f16_to_f32(h: int) -> float:
    return lib().tfo_f16_to_f32(h)


# ------------------------------------------------------------- format ----

def quantize_int4_row(row):
    """Quantization.quantizeInt4Affine (Quantization.swift:50-102) -> (packed u8[n/2], s bf16, b bf16)."""
    row = _c(row, np.float32)
    n = row.size
    packed = np.zeros(n // 2, np.uint8)
    s = np.zeros(n // GROUP, np.uint16)
    b = np.zeros(n // GROUP, np.uint16)
    lib().tfo_quantize_int4_row(_ptr(row), n, _ptr(packed), _ptr(s), _ptr(b))
    return packed, s, b


def quantize_int8_row(row):
    """Quantization.quantizeInt8Affine (Quantization.swift:135-177)."""
    row = _c(row, np.float32)
    n = row.size
    packed = np.zeros(n, np.uint8)
    s = np.zeros(n // GROUP, np.uint16)
    b = np.zeros(n // GROUP, np.uint16)
    lib().tfo_quantize_int8_row(_ptr(row), n, _ptr(packed), _ptr(s), _ptr(b))
    return packed, s, b


def quantize_int4_matrix(rows):
    rows = _c(rows, np.float32)
    out = [quantize_int4_row(r) for r in rows]
    return (np.stack([o[0] for o in out]), np.stack([o[1] for o in out]),
            np.stack([o[2] for o in out]))


def quantize_int8_matrix(rows):
    rows = _c(rows, np.float32)
    out = [quantize_int8_row(r) for r in rows]
    return (np.stack([o[0] for o in out]), np.stack([o[1] for o in out]),
            np.stack([o[2] for o in out]))


def dequantize_int4_row(packed, s, b, fmt, n):
    out = np.zeros(n, np.float32)
    lib().tfo_dequantize_int4_row(_ptr(_c(packed, np.uint8)), _ptr(_c(s, np.uint16)),
                                  _ptr(_c(b, np.uint16)), fmt, n, _ptr(out))
    return out


def dequantize_int8_row(packed, s, b, fmt, n):
    out = np.zeros(n, np.float32)
    lib().tfo_dequantize_int8_row(_ptr(_c(packed, np.uint8)), _ptr(_c(s, np.uint16)),
                                  _ptr(_c(b, np.uint16)), fmt, n, _ptr(out))
    return out


def int4_code(packed_row, j: int) -> int:
    return lib().tfo_int4_code(_ptr(_c(packed_row, np.uint8)), j)


# 2-, 3- and 4-bit rows (QuantizedAffineRow, Quantization.swift:195-349)

def affine_row_bytes(n: int, bits: int) -> int:
    return lib().tfo_affine_row_bytes(n, bits)


def pack_affine_codes(codes, bits: int):
    """packCode (Quantization.swift:295-320) of every code in order -> u8[packedRowBytes]."""
    codes = _c(codes, np.uint32)
    nbytes = affine_row_bytes(codes.size, bits)
    buf = np.zeros(max(nbytes, 1), np.uint8)
    L = lib()
    for j, q in enumerate(codes.tolist()):
        L.tfo_pack_affine_code(_ptr(buf), nbytes, q, j, bits)
    return buf[:nbytes]


def affine_codes(row, n: int, bits: int):
    """unpackCode (Quantization.swift:322-349) of codes 0..n-1."""
    row = _c(row, np.uint8)
    L = lib()
    return np.array([L.tfo_affine_code(_ptr(row), row.size, j, bits) for j in range(n)], np.uint32)


def quantize_affine_row(row, bits: int):
    """quantizeAffine (Quantization.swift:229-273) -> (packed, s bf16, b bf16)."""
    row = _c(row, np.float32)
    n = row.size
    packed = np.zeros(affine_row_bytes(n, bits), np.uint8)
    s = np.zeros(n // GROUP, np.uint16)
    b = np.zeros(n // GROUP, np.uint16)
    lib().tfo_quantize_affine_row(_ptr(row), n, bits, _ptr(packed), _ptr(s), _ptr(b))
    return packed, s, b


def dequantize_affine_row(packed, s, b, fmt, bits: int, n: int):
    """dequantizeAffine (Quantization.swift:275-293)."""
    out = np.zeros(n, np.float32)
    lib().tfo_dequantize_affine_row(_ptr(_c(packed, np.uint8)), _ptr(_c(s, np.uint16)),
                                    _ptr(_c(b, np.uint16)), fmt, bits, n, _ptr(out))
    return out


# --------------------------------------------------------------- GEMV ----

def _gemv(name, W, S, B, fmt, x, m, n, out_dtype):
    W = _c(W, np.uint8); S = _c(S, np.uint16); B = _c(B, np.uint16); x = _c(x, np.float32)
    y = np.zeros(m, out_dtype)
    getattr(lib(), name)(_ptr(W), _ptr(S), _ptr(B), fmt, _ptr(x), m, n, _ptr(y))
    return y


def gemv_int4(W, S, B, x, fmt=FMT_F16):
    """DequantInt4GemvRef.apply (V/Reference/Quant/DequantInt4Gemv.swift:12-42). W: [m][n/2] u8."""
    m, n = W.shape[0], np.asarray(x).size
    return _gemv("tfo_gemv_int4", W, S, B, fmt, x, m, n, np.float32)


def gemv_affine(W, S, B, x, bits, fmt=FMT_F16):
    """gemv_int4 over bits-bit rows (W: [m][n*bits/8] u8)."""
    W = _c(W, np.uint8); S = _c(S, np.uint16); B = _c(B, np.uint16); x = _c(x, np.float32)
    m, n = W.shape[0], x.size
    y = np.zeros(m, np.float32)
    lib().tfo_gemv_affine(_ptr(W), _ptr(S), _ptr(B), fmt, bits, _ptr(x), m, n, _ptr(y))
    return y


def gemv_int4_f64(W, S, B, x, fmt=FMT_F16):
    m, n = W.shape[0], np.asarray(x).size
    return _gemv("tfo_gemv_int4_f64", W, S, B, fmt, x, m, n, np.float64)


def gemv_int4_mt(W, S, B, x, fmt=FMT_F16, threads=1):
    W = _c(W, np.uint8); S = _c(S, np.uint16); B = _c(B, np.uint16); x = _c(x, np.float32)
    m, n = W.shape[0], x.size
    y = np.zeros(m, np.float32)
    lib().tfo_gemv_int4_mt(_ptr(W), _ptr(S), _ptr(B), fmt, _ptr(x), m, n, _ptr(y), threads)
    return y


def gemv_int8(W, S, B, x, fmt=FMT_F16):
    """DequantInt8GemvRef.apply (V/Reference/Quant/DequantInt8Gemv.swift:12-40)."""
    m, n = W.shape[0], np.asarray(x).size
    return _gemv("tfo_gemv_int8", W, S, B, fmt, x, m, n, np.float32)


def gemv_int8_f64(W, S, B, x, fmt=FMT_F16):
    m, n = W.shape[0], np.asarray(x).size
    return _gemv("tfo_gemv_int8_f64", W, S, B, fmt, x, m, n, np.float64)


# ------------------------------------------------------------- router ----

def router_logits(W, S, B, h, eff=None, fmt=FMT_F16):
    """RouterTopKTests.reference, logits part (T/Kernels/MoE/RouterTopKTests.swift:76-80)."""
    W = _c(W, np.uint8); S = _c(S, np.uint16); B = _c(B, np.uint16); h = _c(h, np.float32)
    E, D = W.shape
    e = None if eff is None else _c(eff, np.float32)
    out = np.zeros(E, np.float32)
    lib().tfo_router_logits(_ptr(W), _ptr(S), _ptr(B), fmt, _ptr(h), _ptr(e), E, D, _ptr(out))
    return out


def topk_softmax(logits, k, expert_scale=None):
    """RouterTopKTests.reference, selection part (RouterTopKTests.swift:81-96)."""
    logits = _c(logits, np.float32)
    es = None if expert_scale is None else _c(expert_scale, np.float32)
    idx = np.zeros(k, np.uint32)
    w = np.zeros(k, np.float32)
    rc = lib().tfo_topk_softmax(_ptr(logits), logits.size, k, _ptr(es), _ptr(idx), _ptr(w))
    if rc != 0:
        raise ValueError("k out of range")
    return idx, w


def prefill_router(W, S, B, hidden, k, eff=None, expert_scale=None, fmt=FMT_F16):
    W = _c(W, np.uint8); S = _c(S, np.uint16); B = _c(B, np.uint16)
    hidden = _c(hidden, np.float32)
    T, stride = hidden.shape
    E, D = W.shape
    e = None if eff is None else _c(eff, np.float32)
    es = None if expert_scale is None else _c(expert_scale, np.float32)
    idx = np.zeros((T, k), np.uint32)
    w = np.zeros((T, k), np.float32)
    rc = lib().tfo_prefill_router(_ptr(W), _ptr(S), _ptr(B), fmt, _ptr(hidden), stride, _ptr(e),
                                  _ptr(es), T, E, D, k, _ptr(idx), _ptr(w))
    if rc != 0:
        raise ValueError("k out of range")
    return idx, w


# ---------------------------------------------------------------- MoE ----

def gelu_tanh(x: float) -> float:
    return lib().tfo_gelu_tanh(x)


def _offsets(off) -> ExpertOffsets:
    if isinstance(off, ExpertOffsets):
        return off
    if isinstance(off, dict):
        return ExpertOffsets(**off)
    return ExpertOffsets(*[int(v) for v in off])


def ffn_int4(blob, off, x, d, f, fmt=FMT_F16):
    blob = _c(blob, np.uint8); x = _c(x, np.float32)
    out = np.zeros(d, np.float32)
    o = _offsets(off)
    lib().tfo_ffn_int4(_ptr(blob), C.byref(o), fmt, _ptr(x), d, f, _ptr(out))
    return out


def moe_routed(pool, stride, off, x, idx, w, d, f, residual=None, fmt=FMT_F16, bits=4):
    """MoeRef.applyStreamedRouted (V/Reference/MoE/Moe.swift:58-88); experts of
    `bits`-bit rows (2, 3, 4)."""
    pool = _c(pool, np.uint8); x = _c(x, np.float32)
    idx = _c(idx, np.uint32); w = _c(w, np.float32)
    r = None if residual is None else _c(residual, np.float32)
    y = np.zeros(d, np.float32)
    o = _offsets(off)
    lib().tfo_moe_routed_bits(_ptr(pool), int(stride), C.byref(o), fmt, bits, _ptr(x), _ptr(r), _ptr(idx),
                              _ptr(w), idx.size, d, f, _ptr(y))
    return y


def _shared_expert(name, gate, up, down, x, d, f, fmt):
    args = []
    for (W, S, B) in (gate, up, down):
        args += [_c(W, np.uint8), _c(S, np.uint16), _c(B, np.uint16)]
    x = _c(x, np.float32)
    y = np.zeros(d, np.float32)
    getattr(lib(), name)(*[_ptr(a) for a in args], fmt, _ptr(x), d, f, _ptr(y))
    return y


def shared_expert(gate, up, down, x, d, f, bits=4, round_gu=False, fmt=FMT_F16):
    """The shared expert at `bits` 4 or 8; round_gu rounds gate and up to fp16
    first (the reference's GPU storage points, tfo_shared_expert)."""
    args = []
    for (W, S, B) in (gate, up, down):
        args += [_c(W, np.uint8), _c(S, np.uint16), _c(B, np.uint16)]
    x = _c(x, np.float32)
    y = np.zeros(d, np.float32)
    lib().tfo_shared_expert(*[_ptr(a) for a in args], fmt, bits, int(round_gu), _ptr(x), d, f, _ptr(y))
    return y


def shared_expert_int4(gate, up, down, x, d, f, fmt=FMT_F16):
    """SharedExpertInt4Tests reference (T/Kernels/MoE/SharedExpertInt4Tests.swift:21-28).
    gate/up/down: (W, S, B) tuples."""
    return _shared_expert("tfo_shared_expert_int4", gate, up, down, x, d, f, fmt)


def shared_expert_int8(gate, up, down, x, d, f, fmt=FMT_F16):
    """SharedExpertInt8Tests reference (T/Kernels/MoE/SharedExpertInt8Tests.swift:57-68).
    gate/up/down: (W, S, B) tuples of int8 rows (W [rows][cols] u8)."""
    return _shared_expert("tfo_shared_expert_int8", gate, up, down, x, d, f, fmt)


# ------------------------------------------------------- decode layer ----

def rmsnorm(x, w, eps):
    """RmsNormRef.apply (V/Reference/Primitives/RmsNorm.swift:14-44); w None: no scale."""
    x = _c(x, np.float32)
    wv = None if w is None else _c(w, np.float32)
    y = np.zeros_like(x)
    lib().tfo_rmsnorm(_ptr(x), _ptr(wv), x.size, eps, _ptr(y))
    return y


def greedy_argmax(z) -> int:
    """logit.metal:706-784: largest finite value, lowest index on ties, 0 if none finite."""
    z = _c(z, np.float32)
    return int(lib().tfo_greedy_argmax(_ptr(z), z.size))


def lm_head_greedy(hidden_f16, norm_w_f16, W, S, B, eps=1e-6, fmt=FMT_F16):
    """LMHeadChainInt4.encodeGreedyDecode (LMHeadChainInt4.swift:62-135): (token, z)."""
    h = _c(hidden_f16, np.uint16); w = None if norm_w_f16 is None else _c(norm_w_f16, np.uint16)
    W = _c(W, np.uint8); S = _c(S, np.uint16); B = _c(B, np.uint16)
    vocab, d = W.shape[0], h.size
    z = np.zeros(vocab, np.float32)
    tok = lib().tfo_lm_head_greedy(_ptr(h), _ptr(w), _ptr(W), _ptr(S), _ptr(B), fmt, d, vocab, eps, _ptr(z))
    return int(tok), z


def rope_neox(x, num_heads, head_dim, rotated_pairs, position, theta):
    """RopeRef.applyNeox (V/Reference/Attention/RoPE.swift:70-110) on a copy of x."""
    y = _c(x, np.float32).copy()
    lib().tfo_rope_neox(_ptr(y), num_heads, head_dim, rotated_pairs, position, theta)
    return y


def attention(q, k, v, head_dim, nq, nkv, seq_len, window=0, scale=None):
    """AttentionRef.apply (V/Reference/Attention/Attention.swift:14-104)."""
    if scale is None:
        scale = 1.0 / float(np.sqrt(head_dim))
    q = _c(q, np.float32); k = _c(k, np.float32); v = _c(v, np.float32)
    out = np.zeros(nq * head_dim, np.float32)
    lib().tfo_attention(_ptr(q), _ptr(k), _ptr(v), head_dim, nq, nkv, seq_len, window or 0, scale,
                        _ptr(out))
    return out



def decode_layer(w: dict, shape: dict, hidden_f16, k_cache_f16, v_cache_f16, position, trace=False, threads=None):
    """One Gemma 4 decoder layer (tfo_decode_layer). w: dict of numpy arrays
    (fp16 bits for norms; (W, S, B) tuples for int4 matrices, "v" None for a
    layer without a v projection; 'pool', 'stride', 'off' for the routed
    experts; router_* arrays). The caches are updated in place at slot
    `position`. threads: run the CPU-baseline build with that many row
    threads (same results). Returns (out_f16, idx, weights, trace dict)."""
    keep = []

    def arr(a, dt):
        if a is None:
            return None
        a = _c(a, dt)
        keep.append(a)
        return _ptr(a)

    def q4(t):
        if t is None:       # no v projection: V from the k projection (full-attention layers)
            return Q4(None, None, None)
        W, S, B = (_c(t[0], np.uint8), _c(t[1], np.uint16), _c(t[2], np.uint16))
        keep.extend([W, S, B])
        return Q4(_ptr(W), _ptr(S), _ptr(B))

    lw = LayerWeights(
        input_norm=arr(w["input_norm"], np.uint16), q=q4(w["q"]), k=q4(w["k"]), v=q4(w.get("v")), o=q4(w["o"]),
        q_norm=arr(w["q_norm"], np.uint16), k_norm=arr(w["k_norm"], np.uint16),
        post_attention_norm=arr(w["post_attention_norm"], np.uint16),
        pre_ffn_norm=arr(w["pre_ffn_norm"], np.uint16), pre_ffn2_norm=arr(w["pre_ffn2_norm"], np.uint16),
        router_w=arr(w["router_w"], np.uint8), router_s=arr(w["router_s"], np.uint16),
        router_b=arr(w["router_b"], np.uint16), router_eff=arr(w.get("router_eff"), np.uint16),
        router_gain=arr(w.get("router_gain"), np.uint16), num_experts=int(w["num_experts"]),
        pool=arr(w["pool"], np.uint8), stride=int(w["stride"]), off=_offsets(w["off"]),
        shared_gate=q4(w["shared_gate"]), shared_up=q4(w["shared_up"]), shared_down=q4(w["shared_down"]),
        post_ffn1_norm=arr(w["post_ffn1_norm"], np.uint16), post_ffn2_norm=arr(w["post_ffn2_norm"], np.uint16),
        post_ffn_norm=arr(w["post_ffn_norm"], np.uint16), layer_scalar=float(w["layer_scalar"]),
        expert_bits=int(w.get("expert_bits", 4)), shared_bits=int(w.get("shared_bits", 4)))
    ls = LayerShape(**{k_: shape[k_] for k_ in ("d", "nq", "nkv", "hd", "rotated_pairs", "window", "f", "fs",
                                                 "k", "eps", "theta", "scale")})
    d, qd = shape["d"], shape["nq"] * shape["hd"]
    hidden = _c(hidden_f16, np.uint16)
    assert k_cache_f16.dtype == np.uint16 and k_cache_f16.flags.c_contiguous
    assert v_cache_f16.dtype == np.uint16 and v_cache_f16.flags.c_contiguous
    out = np.zeros(d, np.uint16)
    idx = np.zeros(shape["k"], np.uint32)
    wts = np.zeros(shape["k"], np.float32)
    tr = {"q": np.zeros(qd, np.uint16), "attn": np.zeros(qd, np.uint16), "o": np.zeros(d, np.uint16),
          "h": np.zeros(d, np.uint16), "h1": np.zeros(d, np.uint16), "h2": np.zeros(d, np.uint16)}
    lt = LayerTrace(**{n: _ptr(a) for n, a in tr.items()})
    _lib_for(threads).tfo_decode_layer(C.byref(lw), C.byref(ls), _ptr(hidden), _ptr(k_cache_f16), _ptr(v_cache_f16),
                           int(position), _ptr(out), _ptr(idx), _ptr(wts), C.byref(lt) if trace else None)
    return out, idx, wts, (tr if trace else None)


# ------------------------------------------------------------ prefill ----

class GroupingError(Exception):
    def __init__(self, code, a, b):
        self.code = code
        self.name = GROUP_ERRORS.get(code, str(code))
        self.values = (a, b)
        super().__init__(f"{self.name}{self.values}")


def group_pairs(pairs, query_count, top_k, num_experts, tile_expert_count=16, sort_keys=None):
    """PrefillMoEGrouping.groupTokenExpertPairs (PrefillMoEGrouping.swift:91-192).
    pairs: structured array of PAIR_DTYPE. Returns dict of sorted/offsets/counts/groups/tiles."""
    pairs = np.ascontiguousarray(pairs, dtype=PAIR_DTYPE)
    n = pairs.size
    sorted_ = np.zeros(max(n, 1), PAIR_DTYPE)
    ne = max(int(num_experts), 1)
    offsets = np.zeros(ne, np.uint32)
    counts = np.zeros(ne, np.uint32)
    groups = np.zeros(ne, GROUP_DTYPE)
    tiles = np.zeros(ne, TILE_DTYPE)
    ng = C.c_int64(0)
    nt = C.c_int64(0)
    err = (C.c_int64 * 2)()
    sk = None if sort_keys is None else _c(sort_keys, np.uint64)
    rc = lib().tfo_group_pairs(_ptr(pairs), n, query_count, top_k, num_experts, tile_expert_count,
                               _ptr(sk), 0 if sk is None else sk.size, _ptr(sorted_),
                               _ptr(offsets), _ptr(counts), _ptr(groups), C.byref(ng),
                               _ptr(tiles), C.byref(nt), err)
    if rc != 0:
        raise GroupingError(rc, err[0], err[1])
    return {
        "sorted": sorted_[:n], "offsets": offsets[:num_experts], "counts": counts[:num_experts],
        "groups": groups[:ng.value], "tiles": tiles[:nt.value], "query_count": query_count,
    }


def grouped_route_partials(sorted_pairs, hidden_f16, hidden_stride, pool, stride, off, top_k, d, f,
                           query_count, fmt=FMT_F16, bits=4, threads=None):
    """cpuSyntheticRoutePartials (T/Kernels/Prefill/PrefillGroupedRoutedMoETests.swift:229-279).
    Unwritten (token, rank) slots keep the sentinel -99 as in the reference."""
    sp = np.ascontiguousarray(sorted_pairs, dtype=PAIR_DTYPE)
    hidden_f16 = _c(hidden_f16, np.uint16)
    pool = _c(pool, np.uint8)
    out = np.full(query_count * top_k * d, np.float16(-99).view(np.uint16), np.uint16)
    o = _offsets(off)
    _lib_for(threads).tfo_grouped_route_partials_bits(_ptr(sp), sp.size, _ptr(hidden_f16), hidden_stride,
                                          _ptr(pool), int(stride), C.byref(o), fmt, bits, top_k, d, f,
                                          _ptr(out))
    return out


def reduce_token_major(partials_f16, weights_f16, rows, top_k, d):
    """cpuReduce (T/Kernels/Prefill/PrefillMoETests.swift:46-58). fp16 bits in and out."""
    p = _c(partials_f16, np.uint16); w = _c(weights_f16, np.uint16)
    out = np.zeros(rows * d, np.uint16)
    lib().tfo_reduce_token_major(_ptr(p), _ptr(w), rows, top_k, d, _ptr(out))
    return out


def gemm_int4(W, S, B, X, fmt=FMT_F16, rows=None, bits=4, threads=None):
    """MPPPrefillInt4QMMTests.cpuReference (T/Kernels/TensorCore/MPPPrefillInt4QMMTests.swift:80-105),
    fp32 accumulator (unrounded). rows=(r0, r1) computes a bounded sample of token rows."""
    W = _c(W, np.uint8); S = _c(S, np.uint16); B = _c(B, np.uint16); X = _c(X, np.float32)
    M, K = X.shape
    N = W.shape[0]
    r0, r1 = (0, M) if rows is None else rows
    Y = np.zeros((M, N), np.float32)
    _lib_for(threads).tfo_gemm_affine(_ptr(W), _ptr(S), _ptr(B), fmt, bits, _ptr(X), M, N, K, _ptr(Y), r0, r1)
    return Y


def rel_error(actual, reference) -> float:
    """RelError.compute (V/Tolerance/RelError.swift:7-16)."""
    a = _c(actual, np.float32).ravel(); r = _c(reference, np.float32).ravel()
    assert a.size == r.size
    return lib().tfo_rel_error(_ptr(a), _ptr(r), a.size)


def max_abs_diff(a, b) -> float:
    a = _c(a, np.float32).ravel(); b = _c(b, np.float32).ravel()
    return lib().tfo_max_abs_diff(_ptr(a), _ptr(b), a.size)


class Tolerance:
    """V/Tolerance/Tolerances.swift:4-21, plus the north-star bar."""
    identity = 1e-5
    fp16_reduction = 5e-3
    fp16_chained_reduction = 1e-2
    quant_int4 = 1.5e-3
    quant_int8 = 1e-3
    north_star = 1e-3     # max relative error for floating-point outputs


# ------------------------------------------------------- CPU baseline ----
#
# oracle/libtfq_cpu_baseline.so: the same row arithmetic split over host
# threads (cpu_baseline.c), built -O3 -march=native on the host that times it.

_BASELINE_PATH = os.path.join(_HERE, "libtfq_cpu_baseline.so")
_baseline = None


def baseline_lib(rebuild: bool = False):
    """Builds (make cpu_baseline, on this host) and loads the CPU baseline library."""
    global _baseline
    if _baseline is None or rebuild:
        subprocess.run(["make", "-s"] + (["-B"] if rebuild else []) + ["-C", _HERE, "cpu_baseline"], check=True)
        L = C.CDLL(_BASELINE_PATH)
        _declare(L)             # the oracle's functions, built -O3 -march=native -fopenmp
        L.tfb_gemv_int4.restype = None
        L.tfb_gemv_int4.argtypes = [_P, _P, _P, C.c_int, _P, C.c_int, C.c_int, _P, C.c_int]
        L.tfb_moe_decode_token.restype = None
        L.tfb_moe_decode_token.argtypes = [_P, _P, _P, C.c_int, _P, C.c_uint64, C.POINTER(ExpertOffsets), C.c_int,
                                           _P, _P, C.c_int, C.c_int, C.c_int, _P, _P, _P, C.c_int]
        _baseline = L
    return _baseline


def _lib_for(threads):
    """The checker (threads None), or the CPU-baseline build of the same
    functions with their row loops split over `threads` (identical results)."""
    if threads is None:
        return lib()
    L = baseline_lib()
    L.tfo_set_threads(int(threads))
    return L


def baseline_gemv_int4(W, S, B, x, threads=1, fmt=FMT_F16):
    """tfb_gemv_int4: DequantInt4GemvRef.apply with the rows split over `threads`."""
    W = _c(W, np.uint8); S = _c(S, np.uint16); B = _c(B, np.uint16); x = _c(x, np.float32)
    m, n = W.shape[0], W.shape[1] * 2
    y = np.zeros(m, np.float32)
    baseline_lib().tfo_set_threads(1)       # tfb_* split the rows themselves
    baseline_lib().tfb_gemv_int4(_ptr(W), _ptr(S), _ptr(B), fmt, _ptr(x), m, n, _ptr(y), int(threads))
    return y


def baseline_moe_decode_token(rW, rS, rB, pool, stride, off, h, d, f, k, threads=1, residual=None, fmt=FMT_F16):
    """tfb_moe_decode_token: router -> top-k -> routed experts for one token,
    rows split over `threads`. Returns (y, idx, weights)."""
    rW = _c(rW, np.uint8); rS = _c(rS, np.uint16); rB = _c(rB, np.uint16)
    pool = _c(pool, np.uint8); h = _c(h, np.float32)
    r = None if residual is None else _c(residual, np.float32)
    idx = np.zeros(k, np.uint32)
    w = np.zeros(k, np.float32)
    y = np.zeros(d, np.float32)
    o = _offsets(off)
    baseline_lib().tfo_set_threads(1)
    baseline_lib().tfb_moe_decode_token(_ptr(rW), _ptr(rS), _ptr(rB), rW.shape[0], _ptr(pool), int(stride),
                                        C.byref(o), fmt, _ptr(h), _ptr(r), d, f, k, _ptr(idx), _ptr(w), _ptr(y),
                                        int(threads))
    return y, idx, w
