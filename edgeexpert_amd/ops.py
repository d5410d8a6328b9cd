"""Python mirror of the reference operator API over libtfq's C ABI.

Class and method names follow the reference's Swift wrappers (S/ =
Sources/TurboFieldfare/ in the reference checkout) so that tests read like
the reference's own: a Stream replaces the MTLCommandBuffer, a
(DeviceBuffer, byte offset) pair replaces (MTLBuffer, offset). Every call
goes to the HIP kernels in libtfq; a non-OK status raises TfqError.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

from ._lib import (CODE_OBJECT_PATH, ExpertOffsets, ExpertPoolDesc, Q4Matrix, RouterDesc, check,
                   lib)
from .runtime import DeviceBuffer, Stream


def _addr(buf, offset: int = 0):
    """Device address of buf+offset; None stays None (NULL)."""
    if buf is None:
        return None
    if isinstance(buf, DeviceBuffer):
        return buf.ptr(offset)
    return int(buf) + int(offset)


def _s(stream):
    return None if stream is None else (stream.handle if isinstance(stream, Stream) else stream)


class Context:
    """Loaded gfx950 code object (replaces MetalContext, S/Infrastructure/Metal/MetalContext.swift)."""

    def __init__(self, code_object: str | None = None):
        h = C.c_void_p()
        path = (code_object or CODE_OBJECT_PATH).encode()
        check(lib().tfq_create(C.byref(h), path), "tfq_create")
        self.handle = h.value

    def close(self):
        if getattr(self, "handle", None):
            lib().tfq_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


@dataclass
class Q4Projection:
    """One int4 matrix: weights/scales/biases buffers with byte offsets
    (SharedExpertProjection, S/Kernels/MoE/SharedExpertRuntime)."""
    weights: object
    scales: object
    biases: object
    rows: int
    cols: int
    weights_offset: int = 0
    scales_offset: int = 0
    biases_offset: int = 0

    def desc(self) -> Q4Matrix:
        return Q4Matrix(_addr(self.weights, self.weights_offset), _addr(self.scales, self.scales_offset),
                        _addr(self.biases, self.biases_offset))


class DequantInt4GEMV:
    """S/Kernels/Quant/DequantInt4GEMV.swift:5-181."""

    def __init__(self, context: Context):
        self.ctx = context

    def encode(self, stream, weights, scales, biases, x, y, m, n, weights_offset=0,
               scales_offset=0, biases_offset=0, x_offset=0, y_offset=0):
        check(lib().tfq_gemv_q4g64(self.ctx.handle, _s(stream), _addr(weights, weights_offset),
                                   _addr(scales, scales_offset), _addr(biases, biases_offset),
                                   _addr(x, x_offset), _addr(y, y_offset), m, n),
              "DequantInt4GEMV.encode")

    encode_tgx = encode   # x always staged in LDS: encodeTgx is the same launch

    def encode_qkv(self, stream, q: Q4Projection, k: Q4Projection, v: Q4Projection, x, yq, yk, yv,
                   mq, mkv, n):
        """FusedQKVGEMV.encode (S/Kernels/Fusions/FusedQKVGEMV.swift:92-156)."""
        qd, kd, vd = q.desc(), k.desc(), v.desc()
        check(lib().tfq_gemv_q4g64_qkv(self.ctx.handle, _s(stream), C.byref(qd), C.byref(kd),
                                       C.byref(vd), _addr(x), _addr(yq), _addr(yk), _addr(yv), mq,
                                       mkv, n), "FusedQKVGEMV.encode")


class DequantInt8GEMV:
    """S/Kernels/Quant/DequantInt8GEMV.swift:16-82."""

    def __init__(self, context: Context):
        self.ctx = context

    def encode(self, stream, weights, scales, biases, x, y, m, n, weights_offset=0,
               scales_offset=0, biases_offset=0, x_offset=0, y_offset=0):
        check(lib().tfq_gemv_q8g64(self.ctx.handle, _s(stream), _addr(weights, weights_offset),
                                   _addr(scales, scales_offset), _addr(biases, biases_offset),
                                   _addr(x, x_offset), _addr(y, y_offset), m, n),
              "DequantInt8GEMV.encode")


class PrefillInt4QMM:
    """S/Kernels/Prefill/Primitives/PrefillPrimitives.swift:73-123 and
    S/Kernels/TensorCore/MPPPrefillInt4QMM.swift:4-83 (one MFMA kernel)."""

    def __init__(self, context: Context):
        self.ctx = context

    def encode(self, stream, weights, scales, biases, x, y, t, n, k, dtype=0, weights_offset=0,
               scales_offset=0, biases_offset=0, x_offset=0, y_offset=0):
        check(lib().tfq_gemm_q4g64(self.ctx.handle, _s(stream), _addr(weights, weights_offset),
                                   _addr(scales, scales_offset), _addr(biases, biases_offset),
                                   _addr(x, x_offset), _addr(y, y_offset), t, n, k, dtype),
              "PrefillInt4QMM.encode")


MPPPrefillInt4QMM = PrefillInt4QMM


@dataclass
class ExpertPool:
    """All routed experts of a layer resident in one device buffer:
    expert e = buffer + base_offset + e*stride (replaces MoE's argument buffer)."""
    buffer: object
    stride: int
    num_experts: int
    offsets: dict
    base_offset: int = 0

    def desc(self) -> ExpertPoolDesc:
        o = ExpertOffsets(*[int(self.offsets[k]) for k in (
            "gate_w", "gate_s", "gate_b", "up_w", "up_s", "up_b", "down_w", "down_s", "down_b")])
        return ExpertPoolDesc(_addr(self.buffer, self.base_offset), self.stride, self.num_experts, o)


class MoE:
    """S/Kernels/MoE/MoE.swift:31-414."""
    max_streamed_experts = 8

    def __init__(self, context: Context):
        self.ctx = context

    def encode_router_gemma4(self, stream, weights, scales, biases, hidden, effective_scale,
                             per_expert_scale, out_indices, out_weights, num_experts, d, top_k,
                             workspace, out_weights_f32=None, out_logits=None, weights_offset=0,
                             scales_offset=0, biases_offset=0, hidden_offset=0):
        check(lib().tfq_router_topk(self.ctx.handle, _s(stream), _addr(weights, weights_offset),
                                    _addr(scales, scales_offset), _addr(biases, biases_offset),
                                    _addr(hidden, hidden_offset), _addr(effective_scale),
                                    _addr(per_expert_scale), _addr(out_indices), _addr(out_weights),
                                    _addr(out_weights_f32), _addr(out_logits), num_experts, d, top_k,
                                    _addr(workspace)), "MoE.encodeRouterGemma4")

    def encode_routed_phase1(self, stream, pool: ExpertPool, indices, x, acts, d, f, top_k):
        p = pool.desc()
        check(lib().tfq_moe_phase1(self.ctx.handle, _s(stream), C.byref(p), _addr(indices),
                                   _addr(x), _addr(acts), d, f, top_k),
              "MoE.encodeRoutedPersistentPhase1U16Load")

    def encode_routed_phase1_subset(self, stream, pool: ExpertPool, indices, x, acts, active_slots,
                                    active_count, d, f, top_k):
        p = pool.desc()
        check(lib().tfq_moe_phase1_subset(self.ctx.handle, _s(stream), C.byref(p), _addr(indices),
                                          _addr(x), _addr(acts), _addr(active_slots), active_count,
                                          d, f, top_k),
              "MoE.encodeRoutedPersistentPhase1SubsetU16Load")

    def encode_routed_phase2(self, stream, pool: ExpertPool, indices, acts, routing_weights,
                             residual, y, d, f, top_k):
        p = pool.desc()
        check(lib().tfq_moe_phase2(self.ctx.handle, _s(stream), C.byref(p), _addr(indices),
                                   _addr(acts), _addr(routing_weights), _addr(residual), _addr(y), d,
                                   f, top_k), "MoE.encodeRoutedPersistentPhase2Reduce")

    def encode_routed(self, stream, pool: ExpertPool, indices, routing_weights, x, residual, y, d,
                      f, top_k, acts):
        p = pool.desc()
        check(lib().tfq_moe_decode(self.ctx.handle, _s(stream), C.byref(p), _addr(indices),
                                   _addr(routing_weights), _addr(x), _addr(residual), _addr(y), d, f,
                                   top_k, _addr(acts)), "tfq_moe_decode")


@dataclass
class Router:
    """int8 router of one layer (weights [num_experts][d]); eff / gain may be None."""
    weights: object
    scales: object
    biases: object
    num_experts: int
    effective_scale: object = None
    per_expert_scale: object = None

    def desc(self) -> RouterDesc:
        return RouterDesc(_addr(self.weights), _addr(self.scales), _addr(self.biases),
                          _addr(self.effective_scale), _addr(self.per_expert_scale), self.num_experts)


def moe_decode_token(context: Context, stream, router: Router, pool: ExpertPool, x, residual, y, d,
                     f, top_k, out_indices, out_weights, acts, workspace):
    """Router -> top-k -> phase 1 -> phase 2 for one token, indices kept on the device."""
    r, p = router.desc(), pool.desc()
    check(lib().tfq_moe_decode_token(context.handle, _s(stream), C.byref(r), C.byref(p), _addr(x),
                                     _addr(residual), _addr(y), d, f, top_k, _addr(out_indices),
                                     _addr(out_weights), _addr(acts), _addr(workspace)),
          "tfq_moe_decode_token")


class SharedExpertInt4:
    """S/Kernels/MoE/SharedExpertInt4.swift:21-95."""

    def __init__(self, context: Context):
        self.ctx = context

    def encode(self, stream, x, gate: Q4Projection, up: Q4Projection, down: Q4Projection, y,
               scratch_act):
        g, u, dn = gate.desc(), up.desc(), down.desc()
        check(lib().tfq_shared_expert_q4(self.ctx.handle, _s(stream), C.byref(g), C.byref(u),
                                         C.byref(dn), _addr(x), _addr(y), gate.cols, gate.rows,
                                         _addr(scratch_act)), "SharedExpertInt4.encode")


def convert_bf16_to_f16(context: Context, stream, src, dst, count, inexact_counter=None):
    """Exact BF16 -> fp16 conversion of scale/bias words at load time."""
    check(lib().tfq_convert_bf16_to_f16(context.handle, _s(stream), _addr(src), _addr(dst), count,
                                        _addr(inexact_counter)), "tfq_convert_bf16_to_f16")


def read_ceiling(context: Context, stream, src, nbytes: int, sink, sink_blocks: int, src_offset=0):
    """HBM read-ceiling probe (one pass over nbytes with 128-bit loads)."""
    check(lib().tfq_read_ceiling(context.handle, _s(stream), _addr(src, src_offset), nbytes,
                                 _addr(sink), sink_blocks), "tfq_read_ceiling")
