"""``unproj_o_allreduce`` with the reference operator's signature
(tilert/models/deepseek_v3_2/ops/unproj_o_allreduce.py:23-58) on the gfx950 HIP library:
the attention output projection over the device's heads, y = o_flat . wo_shard^T with bf16
activations (golden :480-498), plus the residual ``x_in``: the single-GPU form of the
allreduce-add epilogue (padded_allreduce_add.py:100-114); ``flag`` is unused."""
from __future__ import annotations

import torch

from .projq_wqb import HeadWeights, head_gemm


def convert_unproj_o(wo: torch.Tensor, wo_scales: torch.Tensor) -> HeadWeights:
    """The device's o_proj shard [dim, local_heads * v_dim] (+ fp32 block scales) as one
    head weight."""
    return HeadWeights(wo[None].contiguous(), wo_scales.float()[None].contiguous())


def unproj_o_allreduce(vec_in: torch.Tensor, mat_in: HeadWeights, mat_scale: torch.Tensor | None,
                       x_in: torch.Tensor | None, flag: int, vec_out: torch.Tensor,
                       profile_logs: torch.Tensor | None = None, model_arch: str = "deepseek_v3_2",
                       compute_kernel_type: str = "bf16") -> None:
    """vec_in bf16 [1, s, heads, v_dim] (or [1, s, heads * v_dim]); mat_in =
    ``convert_unproj_o(wo_shard, scales)``; x_in bf16 [1, s, dim] or None; vec_out bf16
    [1, s, dim]."""
    if model_arch not in ("deepseek_v3_2", "glm_5"):
        raise ValueError(f"Unsupported architecture: {model_arch}")
    if compute_kernel_type not in ("bf16", "fp16mma", "bf16mma"):
        raise ValueError(f"Unsupported compute_kernel_type: {compute_kernel_type}")
    if mat_in.H != 1:
        raise ValueError("mat_in must be one weight (convert_unproj_o)")
    if vec_in.numel() % mat_in.K:
        raise ValueError(f"vec_in must hold [1, s, {mat_in.K}] values")
    head_gemm(vec_in, mat_in, vec_out, x_in)
