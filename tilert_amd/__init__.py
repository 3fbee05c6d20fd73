"""tilert_amd: MI355X (gfx950) FP8 decode hot path of TileRT, from scratch.

Block-scaled FP8 linears (act_quant + fp8_gemm), the MoE expert layer with fused
SwiGLU, and the DSA lightning indexer + exact top-k, as hand-written HIP kernels behind
a C ABI (``include/tilert_amd.h``), with Python wrappers that keep the reference's
operator signatures.
"""
from .kernel import act_quant, fp8_gemm, weight_dequant, weight_quant  # noqa: F401
from .common import linear  # noqa: F401
from .utils import cosine_similarity, relative_l2_error  # noqa: F401

__version__ = "0.1.0"
