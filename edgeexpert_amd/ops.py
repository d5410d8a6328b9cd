"""Python mirror of the reference operator API over libtfq's C ABI.

Class and method names follow the reference's Swift wrappers (S/ =
Sources/TurboFieldfare/ in the reference checkout) so that tests read like
the reference's own: a Stream replaces the MTLCommandBuffer, a
(DeviceBuffer, byte offset) pair replaces (MTLBuffer, offset). Every call
goes to the HIP kernels in libtfq; a non-OK status raises TfqError.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

from ._lib import (CODE_OBJECT_PATH, DecodeLayerShape, DecodeLayerWeights, ExpertOffsets,
                   ExpertPoolDesc, Q4Matrix, RouterDesc, check, lib)
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
               scales_offset=0, biases_offset=0, x_offset=0, y_offset=0, bits=4):
        """bits: 4, or 3 for the 3-bit rows (DequantInt4GEMV.swift:140-180)."""
        args = (self.ctx.handle, _s(stream), _addr(weights, weights_offset), _addr(scales, scales_offset),
                _addr(biases, biases_offset), _addr(x, x_offset), _addr(y, y_offset), m, n)
        if bits == 4:
            check(lib().tfq_gemv_q4g64(*args), "DequantInt4GEMV.encode")
        else:
            check(lib().tfq_gemv_qg64(*args, bits), "DequantInt4GEMV.encode")

    encode_tgx = encode   # x always staged in LDS: encodeTgx is the same launch

    def encode_qkv(self, stream, q: Q4Projection, k: Q4Projection, v: Q4Projection, x, yq, yk, yv,
                   mq, mkv, n, bits=4):
        """FusedQKVGEMV.encode (S/Kernels/Fusions/FusedQKVGEMV.swift:92-156)."""
        qd, kd, vd = q.desc(), k.desc(), v.desc()
        args = (self.ctx.handle, _s(stream), C.byref(qd), C.byref(kd), C.byref(vd), _addr(x), _addr(yq),
                _addr(yk), _addr(yv), mq, mkv, n)
        if bits == 4:
            check(lib().tfq_gemv_q4g64_qkv(*args), "FusedQKVGEMV.encode")
        else:
            check(lib().tfq_gemv_qg64_qkv(*args, bits), "FusedQKVGEMV.encode")


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
               scales_offset=0, biases_offset=0, x_offset=0, y_offset=0, bits=4, path=None):
        """bits: 4, or 3 for 3-bit rows (PrefillPrimitives.swift:91-99). path:
        None (the library's choice by token count) or a GEMM_PATH_* kernel."""
        args = (self.ctx.handle, _s(stream), _addr(weights, weights_offset), _addr(scales, scales_offset),
                _addr(biases, biases_offset), _addr(x, x_offset), _addr(y, y_offset), t, n, k, dtype)
        if path is not None:
            check(lib().tfq_gemm_qg64_path(*args, bits, path), "PrefillInt4QMM.encode")
        elif bits == 4:
            check(lib().tfq_gemm_q4g64(*args), "PrefillInt4QMM.encode")
        else:
            check(lib().tfq_gemm_qg64(*args, bits), "PrefillInt4QMM.encode")


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
    weight_bits: int = 4      # code width of the rows: 2, 3 or 4 (MoE.swift:244 bits:)

    def desc(self) -> ExpertPoolDesc:
        o = ExpertOffsets(*[int(self.offsets[k]) for k in (
            "gate_w", "gate_s", "gate_b", "up_w", "up_s", "up_b", "down_w", "down_s", "down_b")])
        return ExpertPoolDesc(_addr(self.buffer, self.base_offset), self.stride, self.num_experts, o,
                              self.weight_bits)


class PackedExpertsLayout:
    """packed_experts/layout.json of a repacked model directory
    (S/Infrastructure/ModelIO/PackedExpertsLayout.swift:38-150), parsed by
    libtfq with the reader's checks (tfq_loader.h)."""

    def __init__(self, model_dir: str, max_bytes: int = 0):
        h = C.c_void_p()
        check(lib().tfq_expert_layout_load(os.fsencode(model_dir), max_bytes, C.byref(h)),
              "PackedExpertsLayoutReader.load")
        self.handle = h
        self.model_dir = model_dir
        stride, nl, epl, entries = C.c_uint64(), C.c_uint32(), C.c_uint32(), C.c_uint32()
        check(lib().tfq_expert_layout_info(h, C.byref(stride), C.byref(nl), C.byref(epl), C.byref(entries)),
              "tfq_expert_layout_info")
        self.expert_stride, self.num_layers = stride.value, nl.value
        self.experts_per_layer, self.layer_entries = epl.value, entries.value

    def expert(self, layer: int, expert: int):
        """(physicalRank, offset, size) of layout.expert(layer:expert:)."""
        r, off, size = C.c_uint32(), C.c_uint64(), C.c_uint64()
        check(lib().tfq_expert_layout_expert(self.handle, layer, expert, C.byref(r), C.byref(off),
                                             C.byref(size)), "PackedExpertsLayout.expert")
        return r.value, off.value, size.value

    def routed_expert_offsets(self, layer: int):
        """Model.routedExpertOffsets (ModelExpertIO.swift:40-61) and the layer's file name."""
        o = ExpertOffsets()
        name = C.create_string_buffer(4096)
        check(lib().tfq_expert_layout_offsets(self.handle, layer, C.byref(o), name, len(name)),
              "routedExpertOffsets")
        return {k: getattr(o, k) for k, _ in ExpertOffsets._fields_}, name.value.decode()

    def pool_bytes(self, d: int, f: int):
        stride, total = C.c_uint64(), C.c_uint64()
        check(lib().tfq_expert_pool_bytes(self.handle, d, f, C.byref(stride), C.byref(total)),
              "tfq_expert_pool_bytes")
        return stride.value, total.value

    def load_pool(self, context, stream, layer: int, d: int, f: int, pool, inexact_counter=None):
        """Loads one layer's experts into the device buffer `pool`; returns the ExpertPool."""
        desc = ExpertPoolDesc()
        check(lib().tfq_expert_pool_load(context.handle, _s(stream), self.handle, os.fsencode(self.model_dir),
                                         layer, d, f, _addr(pool), pool.nbytes, C.byref(desc),
                                         _addr(inexact_counter)), "tfq_expert_pool_load")
        offs = {k: getattr(desc.offsets, k) for k, _ in ExpertOffsets._fields_}
        return ExpertPool(pool, desc.stride, desc.num_experts, offs, weight_bits=desc.weight_bits)

    def close(self):
        if self.handle:
            lib().tfq_expert_layout_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def resident_load(stream, path: str, file_offset: int, size: int, dst):
    """The resident tensor bytes [file_offset, file_offset + size) of `path` into device memory
    (ResidentBuffer.init, S/Infrastructure/ModelIO/ResidentBuffer.swift:15-57)."""
    check(lib().tfq_resident_load(_s(stream), os.fsencode(path), file_offset, size, _addr(dst)),
          "tfq_resident_load")


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

    def encode_router_logits(self, stream, weights, scales, biases, hidden, effective_scale, logits,
                             num_experts, d):
        """The router GEMV alone (router_gemv_gemma4_r4)."""
        check(lib().tfq_router_logits(self.ctx.handle, _s(stream), _addr(weights), _addr(scales),
                                      _addr(biases), _addr(hidden), _addr(effective_scale), _addr(logits),
                                      num_experts, d), "MoE.encodeRouterLogits")

    def encode_routed_phase1_with_selection(self, stream, pool: ExpertPool, logits, per_expert_scale,
                                            num_experts, out_indices, out_weights, x, acts, d, f, top_k,
                                            out_weights_f32=None):
        """Top-k selection folded into phase 1 (every block selects; block 0 publishes)."""
        p = pool.desc()
        check(lib().tfq_moe_phase1_routed(self.ctx.handle, _s(stream), C.byref(p), _addr(logits),
                                          _addr(per_expert_scale), num_experts, _addr(out_indices),
                                          _addr(out_weights), _addr(out_weights_f32), _addr(x), _addr(acts),
                                          d, f, top_k), "MoE.encodeRoutedPhase1WithSelection")

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


class LMHeadGreedyInt4:
    """S/Kernels/Fusions/LMHeadChainInt4.swift:5-136 (encodeGreedyDecode)."""

    def __init__(self, context: Context):
        self.ctx = context

    def encode_greedy_decode(self, stream, hidden, norm_weight, weights, scales, biases, out_token, d,
                             vocab, workspace, rms_eps=1e-6, hidden_offset=0, out_token_offset=0):
        check(lib().tfq_lm_head_greedy(self.ctx.handle, _s(stream), _addr(hidden, hidden_offset),
                                       _addr(norm_weight), _addr(weights), _addr(scales), _addr(biases),
                                       _addr(out_token, out_token_offset), d, vocab, rms_eps,
                                       _addr(workspace)), "LMHeadChainInt4.encodeGreedyDecode")


def moe_decode_token(context: Context, stream, router: Router, pool: ExpertPool, x, residual, y, d,
                     f, top_k, out_indices, out_weights, acts, workspace):
    """Router -> top-k -> phase 1 -> phase 2 for one token, indices kept on the device."""
    r, p = router.desc(), pool.desc()
    check(lib().tfq_moe_decode_token(context.handle, _s(stream), C.byref(r), C.byref(p), _addr(x),
                                     _addr(residual), _addr(y), d, f, top_k, _addr(out_indices),
                                     _addr(out_weights), _addr(acts), _addr(workspace)),
          "tfq_moe_decode_token")


def moe_decode_token_noalloc(context: Context, stream, router: Router, pool: ExpertPool, x, residual, y, d,
                             f, top_k, out_indices, out_weights):
    """moe_decode_token with its scratch in libtfq's fixed device array (no allocation)."""
    r, p = router.desc(), pool.desc()
    check(lib().tfq_moe_decode_token_noalloc(context.handle, _s(stream), C.byref(r), C.byref(p), _addr(x),
                                             _addr(residual), _addr(y), d, f, top_k, _addr(out_indices),
                                             _addr(out_weights)), "tfq_moe_decode_token_noalloc")


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


class SharedExpertInt8:
    """S/Kernels/MoE/SharedExpertInt8.swift:55-210 (int8 rows: Q4Projection
    descriptors whose weights hold one byte per code)."""

    def __init__(self, context: Context):
        self.ctx = context

    def encode(self, stream, x, gate: Q4Projection, up: Q4Projection, down: Q4Projection, y,
               scratch_act):
        g, u, dn = gate.desc(), up.desc(), down.desc()
        check(lib().tfq_shared_expert_q8(self.ctx.handle, _s(stream), C.byref(g), C.byref(u),
                                         C.byref(dn), _addr(x), _addr(y), gate.cols, gate.rows,
                                         _addr(scratch_act)), "SharedExpertInt8.encode")


def prefill_shared_expert_workspace_bytes(weight_bits: int, tokens: int, f: int) -> int:
    return lib().tfq_prefill_shared_expert_workspace_bytes(weight_bits, tokens, f)


class PrefillSharedExpert:
    """S/Kernels/Prefill/MoE/PrefillSharedExpert.swift:4-60 (weightBits 8 by default)."""

    def __init__(self, context: Context, weight_bits: int = 8):
        self.ctx = context
        self.weight_bits = weight_bits

    def encode_block(self, stream, x, y, gate: Q4Projection, up: Q4Projection, down: Q4Projection,
                     workspace, workspace_bytes, query_count, d, intermediate, x_stride_elements,
                     y_stride_elements, x_offset=0, y_offset=0):
        g, u, dn = gate.desc(), up.desc(), down.desc()
        check(lib().tfq_prefill_shared_expert(self.ctx.handle, _s(stream), self.weight_bits, C.byref(g),
                                              C.byref(u), C.byref(dn), _addr(x, x_offset), x_stride_elements,
                                              _addr(y, y_offset), y_stride_elements, query_count, d,
                                              intermediate, _addr(workspace), workspace_bytes),
              "PrefillSharedExpert.encodeBlock")


def convert_bf16_to_f16(context: Context, stream, src, dst, count, inexact_counter=None):
    """Exact BF16 -> fp16 conversion of scale/bias words at load time."""
    check(lib().tfq_convert_bf16_to_f16(context.handle, _s(stream), _addr(src), _addr(dst), count,
                                        _addr(inexact_counter)), "tfq_convert_bf16_to_f16")


def read_ceiling(context: Context, stream, src, nbytes: int, sink, sink_blocks: int, src_offset=0):
    """HBM read-ceiling probe (one pass over nbytes with 128-bit loads)."""
    check(lib().tfq_read_ceiling(context.handle, _s(stream), _addr(src, src_offset), nbytes,
                                 _addr(sink), sink_blocks), "tfq_read_ceiling")


# ----------------------------------------------------------------- prefill ----

PAIR_DTYPE = np.dtype([("token", "<u4"), ("expert", "<u4"), ("rank", "<u4"), ("weight_bits", "<u4")])
TILE_DTYPE = np.dtype([("expert", "<u4"), ("start", "<u4"), ("count", "<u4"), ("reserved", "<u4")])
GROUP_DTYPE = np.dtype([("expert", "<u4"), ("pair_start", "<u4"), ("pair_count", "<u4")])
GROUP_TILE_DTYPE = np.dtype([("group_start", "<u4"), ("group_count", "<u4"), ("pair_start", "<u4"),
                             ("pair_count", "<u4")])
GROUP_ERRORS = {1: "invalidQueryCount", 2: "invalidTopK", 3: "invalidNumExperts",
                4: "invalidTileExpertCount", 5: "pairCountMismatch", 6: "tokenOutOfRange",
                7: "rankOutOfRange", 8: "expertOutOfRange", 9: "duplicateTokenRank",
                10: "expertSortKeyCountMismatch"}


# Bytes of the device grouping state (TFQ_MOE_GROUP_STATE_WORDS words): the
# tile count, then the grouped launches' work counters.
GROUP_STATE_BYTES = 16


def max_tiles(T: int, k: int, num_experts: int) -> int:
    n = T * k
    return (n + 127) // 128 + min(num_experts, n)


class PrefillRouter:
    """S/Kernels/Prefill/MoE/PrefillRouter.swift:30-112."""

    def __init__(self, context: Context):
        self.ctx = context

    def encode_gemma4_block(self, stream, router: "Router", hidden, hidden_stride, query_count, d,
                            top_k, out_indices, out_weights, logits_scratch, out_weights_f32=None):
        r = router.desc()
        check(lib().tfq_prefill_router(self.ctx.handle, _s(stream), C.byref(r), _addr(hidden),
                                       hidden_stride, query_count, d, top_k, _addr(out_indices),
                                       _addr(out_weights), _addr(out_weights_f32),
                                       _addr(logits_scratch)), "PrefillRouter.encodeGemma4Block")

    @staticmethod
    def make_token_expert_pairs(indices, weights_f16_bits, query_count, top_k):
        """makeTokenExpertPairs (PrefillRouter.swift:91-111): token-major pairs."""
        idx = np.asarray(indices, np.uint32).reshape(query_count, top_k)
        wb = np.asarray(weights_f16_bits, np.uint16).reshape(query_count, top_k)
        pairs = np.zeros(query_count * top_k, PAIR_DTYPE)
        pairs["token"] = np.repeat(np.arange(query_count, dtype=np.uint32), top_k)
        pairs["rank"] = np.tile(np.arange(top_k, dtype=np.uint32), query_count)
        pairs["expert"] = idx.ravel()
        pairs["weight_bits"] = wb.ravel()
        return pairs


class GroupingError(Exception):
    def __init__(self, code, a, b):
        self.code = code
        self.name = GROUP_ERRORS.get(code, str(code))
        self.values = (a, b)
        super().__init__(f"{self.name}{self.values}")


class PrefillMoEGrouping:
    """PrefillMoEGrouping (S/Kernels/Prefill/MoE/PrefillMoEGrouping.swift:90-193):
    group_token_expert_pairs runs the host restatement in libtfq; encode runs
    the device counting sort."""

    def __init__(self, context: Context | None = None):
        self.ctx = context

    @staticmethod
    def group_token_expert_pairs(pairs, query_count, top_k, num_experts, tile_expert_count=16,
                                 expert_sort_keys=None):
        pairs = np.ascontiguousarray(pairs, dtype=PAIR_DTYPE)
        n = pairs.size
        ne = max(int(num_experts), 1)
        sorted_ = np.zeros(max(n, 1), PAIR_DTYPE)
        offsets = np.zeros(ne, np.uint32)
        counts = np.zeros(ne, np.uint32)
        groups = np.zeros(ne, GROUP_DTYPE)
        tiles = np.zeros(ne, GROUP_TILE_DTYPE)
        ng, nt = C.c_int64(0), C.c_int64(0)
        err = (C.c_int64 * 2)()
        sk = None if expert_sort_keys is None else np.ascontiguousarray(expert_sort_keys, np.uint64)
        rc = lib().tfq_group_pairs_host(
            pairs.ctypes.data, n, query_count, top_k, num_experts, tile_expert_count,
            None if sk is None else sk.ctypes.data, 0 if sk is None else sk.size,
            sorted_.ctypes.data, offsets.ctypes.data, counts.ctypes.data, groups.ctypes.data,
            C.byref(ng), tiles.ctypes.data, C.byref(nt), err)
        if rc != 0:
            raise GroupingError(rc, err[0], err[1])
        return {"sorted": sorted_[:n], "offsets": offsets[:num_experts],
                "counts": counts[:num_experts], "groups": groups[:ng.value],
                "tiles": tiles[:nt.value], "query_count": query_count}

    def encode(self, stream, indices, weights, query_count, top_k, num_experts, sorted_pairs,
               offsets, counts, tiles, n_tiles, status):
        check(lib().tfq_moe_group(self.ctx.handle, _s(stream), _addr(indices), _addr(weights),
                                  query_count, top_k, num_experts, _addr(sorted_pairs),
                                  _addr(offsets), _addr(counts), _addr(tiles), _addr(n_tiles),
                                  _addr(status)), "tfq_moe_group")


class PrefillGroupedRoutedMoE:
    """S/Kernels/Prefill/MoE/PrefillGroupedRoutedMoE.swift:390-529 and
    S/Kernels/Prefill/MoE/PrefillMoE.swift:4-40."""

    def __init__(self, context: Context):
        self.ctx = context

    def encode(self, stream, pool: "ExpertPool", sorted_pairs, tiles, n_tiles, max_tiles_, hidden,
               hidden_stride, d, f, top_k, act_scratch, route_partials):
        p = pool.desc()
        check(lib().tfq_moe_grouped(self.ctx.handle, _s(stream), C.byref(p), _addr(sorted_pairs),
                                    _addr(tiles), _addr(n_tiles), max_tiles_, _addr(hidden),
                                    hidden_stride, d, f, top_k, _addr(act_scratch),
                                    _addr(route_partials)), "PrefillGroupedRoutedMoE.encode")

    def encode_reduce_token_major(self, stream, route_partials, route_weights, h2, query_count,
                                  top_k, d):
        check(lib().tfq_moe_combine(self.ctx.handle, _s(stream), _addr(route_partials),
                                    _addr(route_weights), _addr(h2), query_count, top_k, d),
              "PrefillMoE.encodeReduceTokenMajor")


def moe_prefill_workspace_bytes(T, top_k, num_experts, d, f) -> int:
    return lib().tfq_moe_prefill_workspace_bytes(T, top_k, num_experts, d, f)


def moe_prefill(context: Context, stream, router: "Router", pool: "ExpertPool", hidden, hidden_stride,
                T, d, f, top_k, h2, out_indices, out_weights, workspace, workspace_bytes):
    """Router -> device grouping -> grouped experts -> combine for T tokens."""
    r, p = router.desc(), pool.desc()
    check(lib().tfq_moe_prefill(context.handle, _s(stream), C.byref(r), C.byref(p), _addr(hidden),
                                hidden_stride, T, d, f, top_k, _addr(h2), _addr(out_indices),
                                _addr(out_weights), _addr(workspace), workspace_bytes),
          "tfq_moe_prefill")


# -------------------------------------------------------------- decode layer --

class Attention:
    """S/Kernels/Attention/Attention.swift:26-420 (encodeFull / encodeSWA)."""

    def __init__(self, context: Context):
        self.ctx = context

    @staticmethod
    def workspace_bytes(head_dim, num_q_heads, seq_len, window=0) -> int:
        return lib().tfq_attention_workspace_bytes(head_dim, num_q_heads, seq_len, window)

    def encode(self, stream, q, k, v, out, head_dim, num_q_heads, num_kv_heads, seq_len, workspace,
               workspace_bytes, window=0, scale=None):
        """window 0 = encodeFull; scale None = 1/sqrt(head_dim) (Attention.defaultScale)."""
        if scale is None:
            scale = 1.0 / float(np.sqrt(head_dim))
        check(lib().tfq_attention_decode(self.ctx.handle, _s(stream), _addr(q), _addr(k), _addr(v),
                                         _addr(out), head_dim, num_q_heads, num_kv_heads, seq_len,
                                         window, scale, _addr(workspace), workspace_bytes),
              "Attention.encode")


@dataclass
class DecodeLayerShapeSpec:
    d: int
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    expert_f: int
    shared_f: int
    top_k: int
    rotated_pairs: int | None = None
    window: int = 0
    eps: float = 1e-6
    rope_theta: float = 10000.0
    attn_scale: float = 1.0

    def desc(self) -> DecodeLayerShape:
        rp = self.head_dim // 2 if self.rotated_pairs is None else self.rotated_pairs
        return DecodeLayerShape(self.d, self.num_q_heads, self.num_kv_heads, self.head_dim, rp,
                                self.window, self.expert_f, self.shared_f, self.top_k, self.eps,
                                self.rope_theta, self.attn_scale)


@dataclass
class DecodeLayerWeightsSpec:
    """Device buffers of one Gemma 4 decoder layer (norm weights fp16)."""
    input_norm: object
    q_proj: Q4Projection
    k_proj: Q4Projection
    v_proj: Q4Projection
    q_norm: object
    k_norm: object
    o_proj: Q4Projection
    post_attention_norm: object
    pre_ffn_norm: object
    pre_ffn2_norm: object
    router: "Router"
    experts: "ExpertPool"
    shared_gate: Q4Projection
    shared_up: Q4Projection
    shared_down: Q4Projection
    post_ffn1_norm: object
    post_ffn2_norm: object
    post_ffn_norm: object
    layer_scalar: float = 1.0
    shared_bits: int = 4

    @classmethod
    def upload(cls, w: dict) -> "DecodeLayerWeightsSpec":
        """Copies host arrays (the keys of edgeexpert_amd.synth.decode_layer)
        into device buffers that this spec keeps alive."""
        def buf(a):
            return DeviceBuffer.from_array(np.ascontiguousarray(a))

        def q4(t, bits=4):
            if t is None:       # no v projection (full-attention layers): null matrix
                return Q4Projection(None, None, None, 0, 0)
            W, S, B = t
            rows, cols = W.shape[0], W.shape[1] * 8 // bits
            return Q4Projection(buf(W), buf(S), buf(B), rows, cols)

        sb = int(w.get("shared_bits", 4))

        E = int(w["num_experts"])
        router = Router(buf(w["router_w"]), buf(w["router_s"]), buf(w["router_b"]), E,
                        buf(w["router_eff"]) if w.get("router_eff") is not None else None,
                        buf(w["router_gain"]) if w.get("router_gain") is not None else None)
        pool = ExpertPool(buf(w["pool"]), int(w["stride"]), E, dict(w["off"]),
                          weight_bits=int(w.get("expert_bits", 4)))
        return cls(buf(w["input_norm"]), q4(w["q"]), q4(w["k"]), q4(w.get("v")), buf(w["q_norm"]),
                   buf(w["k_norm"]), q4(w["o"]), buf(w["post_attention_norm"]), buf(w["pre_ffn_norm"]),
                   buf(w["pre_ffn2_norm"]), router, pool, q4(w["shared_gate"], sb), q4(w["shared_up"], sb),
                   q4(w["shared_down"], sb), buf(w["post_ffn1_norm"]), buf(w["post_ffn2_norm"]),
                   buf(w["post_ffn_norm"]), float(w["layer_scalar"]), sb)

    def desc(self) -> DecodeLayerWeights:
        return DecodeLayerWeights(
            _addr(self.input_norm), self.q_proj.desc(), self.k_proj.desc(), self.v_proj.desc(),
            _addr(self.q_norm), _addr(self.k_norm), self.o_proj.desc(), _addr(self.post_attention_norm),
            _addr(self.pre_ffn_norm), _addr(self.pre_ffn2_norm), self.router.desc(), self.experts.desc(),
            self.shared_gate.desc(), self.shared_up.desc(), self.shared_down.desc(),
            _addr(self.post_ffn1_norm), _addr(self.post_ffn2_norm), _addr(self.post_ffn_norm),
            float(self.layer_scalar), int(self.shared_bits))


def decode_layer_workspace_bytes(shape: DecodeLayerShapeSpec, max_seq_len: int) -> int:
    sd = shape.desc()
    return lib().tfq_decode_layer_workspace_bytes(C.byref(sd), max_seq_len)


class DecodeLayer:
    """One decoder layer per call: the per-layer decode sequence of
    RealForwardRunner (S/Runtime/Inference/RealForwardRunner.swift:2265-2862)."""

    def __init__(self, context: Context, weights: DecodeLayerWeightsSpec, shape: DecodeLayerShapeSpec):
        self.ctx = context
        self._w = weights.desc()
        self._s = shape.desc()
        self.keep = weights

    def encode(self, stream, hidden_in, hidden_out, k_cache, v_cache, position, workspace, workspace_bytes,
               out_indices=None, out_weights=None):
        check(lib().tfq_decode_layer(self.ctx.handle, _s(stream), C.byref(self._w), C.byref(self._s),
                                     _addr(hidden_in), _addr(hidden_out), _addr(k_cache), _addr(v_cache),
                                     position, _addr(out_indices), _addr(out_weights), _addr(workspace),
                                     workspace_bytes), "DecodeLayer.encode")


class DecodeLayers:
    """Consecutive decoder layers per call (tfq_decode_layers): the per-token
    loop over layers of RealForwardRunner (RealForwardRunner.swift:2239-2862)
    with each layer's tail formed inside the next layer's QKV launch."""

    def __init__(self, context: Context, weights: list, shapes: list):
        assert len(weights) == len(shapes) and weights
        self.ctx = context
        self.n = len(weights)
        self._w = (DecodeLayerWeights * self.n)(*[w.desc() for w in weights])
        self._s = (DecodeLayerShape * self.n)(*[s.desc() for s in shapes])
        self.keep = weights

    def workspace_bytes(self, max_seq_len: int) -> int:
        return lib().tfq_decode_layers_workspace_bytes(self._s, self.n, max_seq_len)

    def encode(self, stream, hidden_in, hiddens, k_caches, v_caches, position, workspace, workspace_bytes):
        """hiddens: device buffer [n][d] receiving every layer's output;
        k_caches / v_caches: one device buffer per layer."""
        kc = (C.c_void_p * self.n)(*[_addr(b) for b in k_caches])
        vc = (C.c_void_p * self.n)(*[_addr(b) for b in v_caches])
        check(lib().tfq_decode_layers(self.ctx.handle, _s(stream), self.n, self._w, self._s, _addr(hidden_in),
                                      _addr(hiddens), kc, vc, position, _addr(workspace), workspace_bytes),
              "DecodeLayers.encode")
