"""DeepSeek-style FP8 linear, ``tilert/models/common.py:57-89`` (FP8 branch)."""
from __future__ import annotations

import torch

from .kernel import PackedFP8Weight, act_quant, fp8_gemm


def linear(x_in: torch.Tensor, weight, weight_scale: torch.Tensor | None = None,
           bias: torch.Tensor | None = None, scale_fmt: str | None = None) -> torch.Tensor:
    """``y = x W^T (+ b)``: act_quant(x) per 1x128, then the block-scaled FP8 GEMM.

    The reference attaches the scale to the weight tensor (``_get_scale_tensor``); here it
    is an explicit argument.  Output bf16.
    """
    if not isinstance(weight, PackedFP8Weight) and weight.dtype != torch.float8_e4m3fn:
        raise ValueError("linear: weight must be float8_e4m3fn (bf16 weights use F.linear)")
    x_q, scale = act_quant(x_in.contiguous(), 128, scale_fmt)
    y = fp8_gemm(x_q, scale, weight, weight_scale)
    if bias is not None:
        y += bias
    return y
