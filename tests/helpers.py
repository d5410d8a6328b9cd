"""Input builders shared by the tests.

`ref_*` builders reproduce the reference tests' own inputs: SeedTree(seed)
.key(label) -> SplitMix64 uniforms -> Quantization.quantizeInt4Affine (BF16
scale/bias), exactly as e.g. T/Kernels/Quant/DequantInt4GEMVTests.swift:41-60
draws them. The BF16 words are converted to the library's fp16 format with an
exactness check (every value these tests produce is exactly representable).
"""
from __future__ import annotations

import numpy as np

import oracle
from edgeexpert_amd import synth


def bf16_to_f16_exact(bits: np.ndarray) -> np.ndarray:
    f = synth.bf16_to_f32(bits)
    h = f.astype(np.float16)
    assert np.array_equal(h.astype(np.float32), f), "BF16 value not exactly representable in fp16"
    return h.view(np.uint16)


def ref_int4_rows(seed: int, label: str, m: int, n: int, lo: float, hi: float, extra: int = 0):
    """m rows of n uniforms quantised with quantizeInt4Affine, then `extra`
    more uniforms from the same stream. Returns (W u8 [m][n/2], S bf16 [m][n/64],
    B bf16, tail float32[extra])."""
    key = synth.seed_key(seed, label)
    u = synth.uniform24(key, m * n + extra, lo, hi)
    rows = u[: m * n].reshape(m, n)
    W, S, B = oracle.quantize_int4_matrix(rows)
    return W, S, B, u[m * n:]


def ref_int8_rows(seed: int, label: str, m: int, n: int, lo: float, hi: float, extra: int = 0):
    key = synth.seed_key(seed, label)
    u = synth.uniform24(key, m * n + extra, lo, hi)
    W, S, B = oracle.quantize_int8_matrix(u[: m * n].reshape(m, n))
    return W, S, B, u[m * n:]


def f16_round(x) -> np.ndarray:
    """Float(Float16(x)) — the value a fp16 buffer holds."""
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def f16_bits(x) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def from_f16_bits(bits) -> np.ndarray:
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


def dequant_int4_np(W, S, B, scale_fmt=oracle.FMT_F16):
    """Independent numpy dequantisation (used to pin the C oracle)."""
    q = synth.unpack_int4(W).astype(np.float32)
    to32 = synth.f16_to_f32 if scale_fmt == oracle.FMT_F16 else synth.bf16_to_f32
    s = np.repeat(to32(S), 64, axis=-1)
    b = np.repeat(to32(B), 64, axis=-1)
    return (q * s + b).astype(np.float32)


def bf16_half_ulp(v) -> np.ndarray:
    """Half a bf16 ulp at |v|: bf16 keeps 8 significant bits, so a value in
    [2^e, 2^(e+1)) rounds to within 2^(e-8) (between 2^-9 and 2^-8 of |v|)."""
    a = np.abs(np.asarray(v, np.float64))
    e = np.floor(np.log2(np.where(a > 0, a, 2.0 ** -126)))
    return np.ldexp(1.0, (e - 8).astype(np.int64))
