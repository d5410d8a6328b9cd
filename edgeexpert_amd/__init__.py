"""edgeexpert_amd — MI355X (gfx950) quantized-matmul hot path of the
TurboFieldfare / edgeexpert runtime: MLX-affine int4/int8 GEMVs, the fused
router top-k, the routed top-k MoE decode block and the shared expert,
exposed through the C ABI in include/tfq.h (libtfq) and mirrored here with
the reference's operator names.
"""
from ._lib import TfqError, TfqNotBuilt  # noqa: F401

__all__ = ["TfqError", "TfqNotBuilt"]
