"""``projo_wkvb`` with the reference operator's signature
(tilert/models/deepseek_v3_2/ops/projo_wkvb.py:24-54) on the gfx950 HIP library: the
absorbed value projection of MLA, o[t, h, :] = o_lat[t, h, :] . wkv_b[h, nope:, :]^T
(golden ``einsum("bshc,hdc->bshd")``, :465-467), for the device's local heads, through the
per-head GEMV (``tl_head_gemm_bf16``)."""
from __future__ import annotations

import torch

from .projq_wqb import BLOCK, HeadWeights, head_gemm


def convert_projo_wkvb(wkv_b: torch.Tensor, wkv_b_scales: torch.Tensor, n_heads: int, nope_dim: int = 128,
                       v_dim: int = 128) -> HeadWeights:
    """The device's kv_b_proj shard [n_heads * (nope + v), kv_lora] (+ fp32 block scales)
    -> each head's value block [v, kv_lora] (rows nope .. nope + v of the head)."""
    hd = nope_dim + v_dim
    kv = wkv_b.shape[1]
    if wkv_b.shape[0] != n_heads * hd or nope_dim % BLOCK or hd % BLOCK:
        raise ValueError("wkv_b must be [n_heads * (nope + v), kv_lora] with 128-aligned head blocks")
    w = wkv_b.view(torch.uint8).reshape(n_heads, hd, kv)[:, nope_dim:].contiguous()
    s = wkv_b_scales.float().reshape(n_heads, hd // BLOCK, kv // BLOCK)[:, nope_dim // BLOCK:]
    return HeadWeights(w.view(torch.float8_e4m3fn), s.contiguous())


def projo_wkvb(o_in: torch.Tensor, wkv_b_b: HeadWeights, wkv_b_scales: torch.Tensor | None, output: torch.Tensor,
               profile_logs: torch.Tensor | None = None, model_arch: str = "deepseek_v3_2",
               compute_kernel_type: str = "fp16mma") -> None:
    """o_in bf16 [b, s, heads, kv_lora] (the attention output in the latent space); wkv_b_b =
    ``convert_projo_wkvb(...)`` (scales ride along); output bf16 [b, s, heads, v_dim]."""
    if model_arch not in ("deepseek_v3_2", "glm_5"):
        raise ValueError(f"Unsupported architecture: {model_arch}")
    if compute_kernel_type not in ("fp16mma", "bf16mma"):
        raise ValueError(f"Unsupported compute_kernel_type: {compute_kernel_type}")
    if o_in.shape[-2:] != (wkv_b_b.H, wkv_b_b.K):
        raise ValueError(f"o_in must be [b, s, {wkv_b_b.H}, {wkv_b_b.K}]")
    head_gemm(o_in, wkv_b_b, output)
