"""CPU checks of the drop-in boundary: libtfq loads, exports every function
declared in include/*.h, and its code object holds every kernel the host
resolves. No GPU work is launched here."""
import ctypes as C
import os
import re
import shutil
import subprocess

import pytest

from edgeexpert_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in sorted(os.listdir(os.path.join(ROOT, "include")))
           if h.endswith(".h")]


def declared_functions():
    names = set()
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(tfq_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return sorted(names)


def test_headers_declare_the_boundary():
    names = declared_functions()
    for required in ("tfq_create", "tfq_gemv_q4g64", "tfq_gemv_q8g64", "tfq_router_topk",
                     "tfq_moe_phase1", "tfq_moe_phase2", "tfq_shared_expert_q4"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"
    # and the Python binding covers them all
    assert not [n for n in declared_functions() if n not in _lib.SIGNATURES]


def test_status_strings_and_null_context_without_gpu():
    lib = _lib.lib()
    for s in range(5):
        assert lib.tfq_status_string(s)
    # a null context is rejected before any HIP call
    assert lib.tfq_gemv_q4g64(None, None, None, None, None, None, None, 1, 64) == _lib.TFQ_E_INVAL
    assert b"context" in lib.tfq_last_error_message()


@pytest.mark.skipif(not shutil.which("gcc"), reason="no C compiler")
def test_struct_layouts_match_header(tmp_path):
    # compile the header with the system C compiler and compare with the ctypes mirror
    src = tmp_path / "layout.c"
    fields = ["sizeof(tfq_expert_offsets)", "sizeof(tfq_expert_pool)", "offsetof(tfq_expert_pool, offsets)",
              "sizeof(tfq_q4_matrix)", "offsetof(tfq_expert_pool, num_experts)", "sizeof(tfq_router)",
              "sizeof(tfq_decode_layer_weights)", "offsetof(tfq_decode_layer_weights, router)",
              "offsetof(tfq_decode_layer_weights, experts)", "offsetof(tfq_decode_layer_weights, shared_gate)",
              "offsetof(tfq_decode_layer_weights, layer_scalar)", "sizeof(tfq_decode_layer_shape)",
              "offsetof(tfq_decode_layer_shape, eps)"]
    body = "".join(f'printf("%zu\\n", (size_t)({f}));' for f in fields)
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "tfq.h"\n'
                   'int main(void){' + body + 'return 0;}\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True).stdout.split()]
    W, S = _lib.DecodeLayerWeights, _lib.DecodeLayerShape
    assert got == [C.sizeof(_lib.ExpertOffsets), C.sizeof(_lib.ExpertPoolDesc),
                   _lib.ExpertPoolDesc.offsets.offset, C.sizeof(_lib.Q4Matrix),
                   _lib.ExpertPoolDesc.num_experts.offset, C.sizeof(_lib.RouterDesc),
                   C.sizeof(W), W.router.offset, W.experts.offset, W.shared_gate.offset,
                   W.layer_scalar.offset, C.sizeof(S), S.eps.offset]


@pytest.mark.skipif(not shutil.which("/opt/rocm/llvm/bin/llvm-readelf"), reason="no llvm-readelf")
def test_code_object_is_gfx950_and_holds_all_kernels():
    out = "".join(subprocess.run(["/opt/rocm/llvm/bin/llvm-readelf", "--symbols", "--notes", p],
                                 capture_output=True, text=True, check=True).stdout
                  for p in _lib.CODE_OBJECT_PATHS)
    assert out.count("gfx950") >= len(_lib.CODE_OBJECT_PATHS)
    assert "gfx950" in out
    src = open(os.path.join(ROOT, "edgeexpert_amd", "csrc", "host", "tfq.cpp")).read()
    assert "kernel_names" in src
    for fam in ("tfq_q4_gemv_s64_p2", "tfq_moe_phase1_s64_p2", "tfq_moe_phase2_p3",
                "tfq_router_logits_s64_p3", "tfq_router_select", "tfq_gate_up_act_s64_p2",
                "tfq_convert_bf16_f16", "tfq_attn_partial_h256_g2", "tfq_attn_combine_h256",
                "tfq_layer_tail", "tfq_gemm_skinny_q4_bf16_r1_c3", "tfq_q8_gate_up_act_norm_s64_p3",
                "tfq_gelu_mul_f16"):
        assert fam in out
