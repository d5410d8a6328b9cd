"""ctypes binding of libtfq (include/tfq.h, include/tfq_runtime.h).

The shared library is built in-tree by edgeexpert_amd.build into
edgeexpert_amd/lib/. There is no fallback: if libtfq.so or its code object is
missing, loading raises TfqNotBuilt.
"""
from __future__ import annotations

import ctypes as C
import os

LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib")
LIB_PATH = os.path.join(LIB_DIR, "libtfq.so")
# the code objects edgeexpert_amd.build writes (one per kernel translation unit)
CODE_OBJECT_UNITS = ("tfq_gemv", "tfq_int8", "tfq_phase1", "tfq_phase1_routed", "tfq_moe", "tfq_gemm",
                     "tfq_prefill", "tfq_attention", "tfq_layer_moe")
CODE_OBJECT_PATHS = [os.path.join(LIB_DIR, u + ".co") for u in CODE_OBJECT_UNITS]
CODE_OBJECT_PATH = LIB_DIR

ABI_VERSION = 4          # TFQ_ABI_VERSION of include/tfq.h this binding follows
TFQ_OK = 0
TFQ_E_INVAL = 1
TFQ_E_UNSUPPORTED = 2
TFQ_E_HIP = 3
TFQ_E_NOT_LOADED = 4
TFQ_E_IO = 5
ROUTER_WORKSPACE_BYTES = 4096
LM_HEAD_WORKSPACE_BYTES = 65536
NOALLOC_SCRATCH_BYTES = 16384 + ROUTER_WORKSPACE_BYTES
DTYPE_F16 = 0
DTYPE_BF16 = 1
GEMM_PATH_AUTO = 0
GEMM_PATH_TILE = 1
GEMM_PATH_SKINNY = 2
GEMM_PATH_SKINNY32 = 3
GEMM_PATH_GEMV = 4


class TfqNotBuilt(RuntimeError):
    pass


class TfqError(RuntimeError):
    def __init__(self, status: int, where: str):
        lib = _load()
        self.status = status
        self.hip_error = lib.tfq_last_hip_error()
        msg = lib.tfq_last_error_message().decode(errors="replace")
        super().__init__(f"{where}: {lib.tfq_status_string(status).decode()} ({msg})")


class Q4Matrix(C.Structure):
    _fields_ = [("weights", C.c_void_p), ("scales", C.c_void_p), ("biases", C.c_void_p)]


class ExpertOffsets(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in (
        "gate_w", "gate_s", "gate_b", "up_w", "up_s", "up_b", "down_w", "down_s", "down_b")]


class ExpertPoolDesc(C.Structure):
    _fields_ = [("base", C.c_void_p), ("stride", C.c_uint64), ("num_experts", C.c_uint32),
                ("offsets", ExpertOffsets), ("weight_bits", C.c_uint32)]


class RouterDesc(C.Structure):
    _fields_ = [("weights", C.c_void_p), ("scales", C.c_void_p), ("biases", C.c_void_p),
                ("effective_scale", C.c_void_p), ("per_expert_scale", C.c_void_p),
                ("num_experts", C.c_uint32)]


class PairT(C.Structure):
    _fields_ = [("token", C.c_uint32), ("expert", C.c_uint32), ("rank", C.c_uint32),
                ("weight_bits", C.c_uint32)]


class DecodeLayerWeights(C.Structure):
    """tfq_decode_layer_weights (include/tfq.h)."""
    _fields_ = [("input_norm", C.c_void_p), ("q_proj", Q4Matrix), ("k_proj", Q4Matrix),
                ("v_proj", Q4Matrix), ("q_norm", C.c_void_p), ("k_norm", C.c_void_p),
                ("o_proj", Q4Matrix), ("post_attention_norm", C.c_void_p), ("pre_ffn_norm", C.c_void_p),
                ("pre_ffn2_norm", C.c_void_p), ("router", RouterDesc), ("experts", ExpertPoolDesc),
                ("shared_gate", Q4Matrix), ("shared_up", Q4Matrix), ("shared_down", Q4Matrix),
                ("post_ffn1_norm", C.c_void_p), ("post_ffn2_norm", C.c_void_p),
                ("post_ffn_norm", C.c_void_p), ("layer_scalar", C.c_float), ("shared_bits", C.c_uint32)]


class DecodeLayerShape(C.Structure):
    """tfq_decode_layer_shape (include/tfq.h)."""
    _fields_ = [(n, C.c_uint32) for n in ("d", "num_q_heads", "num_kv_heads", "head_dim", "rotated_pairs",
                                          "window", "expert_f", "shared_f", "top_k")] + \
               [(n, C.c_float) for n in ("eps", "rope_theta", "attn_scale")]


_P = C.c_void_p
_U32 = C.c_uint32
_I = C.c_int

# name -> argtypes (restype int unless listed in _RES)
SIGNATURES = {
    "tfq_create": [C.POINTER(C.c_void_p), C.c_char_p],
    "tfq_destroy": [_P],
    "tfq_status_string": [_I],
    "tfq_last_hip_error": [],
    "tfq_last_error_message": [],
    "tfq_gemv_q4g64": [_P, _P, _P, _P, _P, _P, _P, _U32, _U32],
    "tfq_gemv_q4g64_qkv": [_P, _P, C.POINTER(Q4Matrix), C.POINTER(Q4Matrix), C.POINTER(Q4Matrix),
                           _P, _P, _P, _P, _U32, _U32, _U32],
    "tfq_gemv_qg64": [_P, _P, _P, _P, _P, _P, _P, _U32, _U32, _U32],
    "tfq_gemv_qg64_qkv": [_P, _P, C.POINTER(Q4Matrix), C.POINTER(Q4Matrix), C.POINTER(Q4Matrix),
                          _P, _P, _P, _P, _U32, _U32, _U32, _U32],
    "tfq_gemv_q8g64": [_P, _P, _P, _P, _P, _P, _P, _U32, _U32],
    "tfq_lm_head_greedy": [_P, _P, _P, _P, _P, _P, _P, _P, _U32, _U32, C.c_float, _P],
    "tfq_expert_layout_load": [C.c_char_p, C.c_uint64, C.POINTER(C.c_void_p)],
    "tfq_expert_layout_free": [_P],
    "tfq_expert_layout_info": [_P, C.POINTER(C.c_uint64), C.POINTER(C.c_uint32), C.POINTER(C.c_uint32),
                               C.POINTER(C.c_uint32)],
    "tfq_expert_layout_expert": [_P, _U32, _U32, C.POINTER(C.c_uint32), C.POINTER(C.c_uint64),
                                 C.POINTER(C.c_uint64)],
    "tfq_expert_layout_offsets": [_P, _U32, C.POINTER(ExpertOffsets), C.c_char_p, C.c_size_t],
    "tfq_expert_pool_bytes": [_P, _U32, _U32, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)],
    "tfq_expert_pool_load": [_P, _P, _P, C.c_char_p, _U32, _U32, _U32, _P, C.c_uint64,
                             C.POINTER(ExpertPoolDesc), _P],
    "tfq_resident_load": [_P, C.c_char_p, C.c_uint64, C.c_uint64, _P],
    "tfq_router_topk": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _U32, _U32, _U32, _P],
    "tfq_moe_phase1": [_P, _P, C.POINTER(ExpertPoolDesc), _P, _P, _P, _U32, _U32, _U32],
    "tfq_router_logits": [_P, _P, _P, _P, _P, _P, _P, _P, _U32, _U32],
    "tfq_moe_phase1_routed": [_P, _P, C.POINTER(ExpertPoolDesc), _P, _P, _U32, _P, _P, _P, _P, _P, _U32,
                              _U32, _U32],
    "tfq_moe_phase1_subset": [_P, _P, C.POINTER(ExpertPoolDesc), _P, _P, _P, _P, _U32, _U32, _U32,
                              _U32],
    "tfq_moe_phase2": [_P, _P, C.POINTER(ExpertPoolDesc), _P, _P, _P, _P, _P, _U32, _U32, _U32],
    "tfq_moe_decode": [_P, _P, C.POINTER(ExpertPoolDesc), _P, _P, _P, _P, _P, _U32, _U32, _U32, _P],
    "tfq_moe_decode_token": [_P, _P, C.POINTER(RouterDesc), C.POINTER(ExpertPoolDesc), _P, _P, _P,
                             _U32, _U32, _U32, _P, _P, _P, _P],
    "tfq_moe_decode_token_noalloc": [_P, _P, C.POINTER(RouterDesc), C.POINTER(ExpertPoolDesc), _P, _P, _P,
                                     _U32, _U32, _U32, _P, _P],
    "tfq_shared_expert_q4": [_P, _P, C.POINTER(Q4Matrix), C.POINTER(Q4Matrix), C.POINTER(Q4Matrix),
                             _P, _P, _U32, _U32, _P],
    "tfq_shared_expert_q8": [_P, _P, C.POINTER(Q4Matrix), C.POINTER(Q4Matrix), C.POINTER(Q4Matrix),
                             _P, _P, _U32, _U32, _P],
    "tfq_prefill_shared_expert_workspace_bytes": [_U32, _U32, _U32],
    "tfq_prefill_shared_expert": [_P, _P, _U32, C.POINTER(Q4Matrix), C.POINTER(Q4Matrix), C.POINTER(Q4Matrix),
                                  _P, _U32, _P, _U32, _U32, _U32, _U32, _P, C.c_size_t],
    "tfq_convert_bf16_to_f16": [_P, _P, _P, _P, C.c_uint64, _P],
    "tfq_read_ceiling": [_P, _P, _P, C.c_uint64, _P, _U32],
    "tfq_gemm_q4g64": [_P, _P, _P, _P, _P, _P, _P, _U32, _U32, _U32, _I],
    "tfq_gemm_qg64": [_P, _P, _P, _P, _P, _P, _P, _U32, _U32, _U32, _I, _U32],
    "tfq_gemm_qg64_path": [_P, _P, _P, _P, _P, _P, _P, _U32, _U32, _U32, _I, _U32, _I],
    "tfq_prefill_router": [_P, _P, C.POINTER(RouterDesc), _P, _U32, _U32, _U32, _U32, _P, _P, _P, _P],
    "tfq_moe_group": [_P, _P, _P, _P, _U32, _U32, _U32, _P, _P, _P, _P, _P, _P],
    "tfq_group_pairs_host": [_P, C.c_int64, C.c_int64, C.c_int64, C.c_int64, C.c_int64, _P,
                             C.c_int64, _P, _P, _P, _P, C.POINTER(C.c_int64), _P,
                             C.POINTER(C.c_int64), C.POINTER(C.c_int64)],
    "tfq_moe_grouped": [_P, _P, C.POINTER(ExpertPoolDesc), _P, _P, _P, _U32, _P, _U32, _U32, _U32,
                        _U32, _P, _P],
    "tfq_moe_combine": [_P, _P, _P, _P, _P, _U32, _U32, _U32],
    "tfq_moe_prefill_workspace_bytes": [_U32, _U32, _U32, _U32, _U32],
    "tfq_moe_prefill": [_P, _P, C.POINTER(RouterDesc), C.POINTER(ExpertPoolDesc), _P, _U32, _U32,
                        _U32, _U32, _U32, _P, _P, _P, _P, C.c_size_t],
    "tfq_attention_workspace_bytes": [_U32, _U32, _U32, _U32],
    "tfq_attention_decode": [_P, _P, _P, _P, _P, _P, _U32, _U32, _U32, _U32, _U32, C.c_float, _P,
                             C.c_size_t],
    "tfq_decode_layer_workspace_bytes": [C.POINTER(DecodeLayerShape), _U32],
    "tfq_decode_layers_workspace_bytes": [C.POINTER(DecodeLayerShape), _U32, _U32],
    "tfq_decode_layers": [_P, _P, _U32, C.POINTER(DecodeLayerWeights), C.POINTER(DecodeLayerShape), _P, _P,
                          C.POINTER(_P), C.POINTER(_P), _U32, _P, C.c_size_t],
    "tfq_decode_layer": [_P, _P, C.POINTER(DecodeLayerWeights), C.POINTER(DecodeLayerShape), _P, _P, _P,
                         _P, _U32, _P, _P, _P, C.c_size_t],
    "tfq_abi_version": [],
    "tfq_rt_device_count": [C.POINTER(_I)],
    "tfq_rt_set_device": [_I],
    "tfq_rt_device_info": [C.c_char_p, C.c_size_t, C.c_char_p, C.c_size_t],
    "tfq_rt_malloc": [C.POINTER(C.c_void_p), C.c_size_t],
    "tfq_rt_free": [_P],
    "tfq_rt_memcpy_htod": [_P, _P, C.c_size_t],
    "tfq_rt_memcpy_dtoh": [_P, _P, C.c_size_t],
    "tfq_rt_memcpy_dtod": [_P, _P, C.c_size_t, _P],
    "tfq_rt_memset": [_P, _I, C.c_size_t],
    "tfq_rt_stream_create": [C.POINTER(C.c_void_p)],
    "tfq_rt_stream_destroy": [_P],
    "tfq_rt_stream_sync": [_P],
    "tfq_rt_device_sync": [],
    "tfq_rt_event_create": [C.POINTER(C.c_void_p)],
    "tfq_rt_event_destroy": [_P],
    "tfq_rt_event_record": [_P, _P],
    "tfq_rt_event_sync": [_P],
    "tfq_rt_event_elapsed_ms": [C.POINTER(C.c_float), _P, _P],
    "tfq_rt_capture_begin": [_P],
    "tfq_rt_capture_end": [_P, C.POINTER(C.c_void_p)],
    "tfq_rt_graph_launch": [_P, _P],
    "tfq_rt_graph_destroy": [_P],
}
_RES = {"tfq_destroy": None, "tfq_status_string": C.c_char_p, "tfq_expert_layout_free": None,
        "tfq_moe_prefill_workspace_bytes": C.c_size_t,
        "tfq_attention_workspace_bytes": C.c_size_t,
        "tfq_decode_layer_workspace_bytes": C.c_size_t,
        "tfq_decode_layers_workspace_bytes": C.c_size_t,
        "tfq_prefill_shared_expert_workspace_bytes": C.c_size_t,
        "tfq_last_error_message": C.c_char_p}

_lib = None


def _load():
    global _lib
    if _lib is None:
        missing = [p for p in [LIB_PATH, *CODE_OBJECT_PATHS] if not os.path.exists(p)]
        if missing:
            raise TfqNotBuilt(f"{', '.join(missing)} missing: run `python -m edgeexpert_amd.build` first")
        lib = C.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            f = getattr(lib, name)
            f.argtypes = args
            f.restype = _RES.get(name, C.c_int)
        if lib.tfq_abi_version() != ABI_VERSION:
            raise TfqNotBuilt(f"{LIB_PATH} has ABI version {lib.tfq_abi_version()}, this binding expects "
                              f"{ABI_VERSION}: rebuild with `python -m edgeexpert_amd.build`")
        _lib = lib
    return _lib


def lib():
    return _load()


def check(status: int, where: str):
    if status != TFQ_OK:
        raise TfqError(status, where)
