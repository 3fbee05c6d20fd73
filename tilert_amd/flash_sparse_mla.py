"""Sparse MLA decode attention over the indexer's top-k selection, with the reference
operator's shape (tilert/models/deepseek_v3_2/ops/flash_sparse_mla.py:18-93; golden
FlashSparseMLACombine.golden_forward :152-196): split-K over 64-position splits, the
per-split ``output_acc`` / ``lse_acc`` and the total ``lse`` returned as the reference's
function returns them."""
from __future__ import annotations

import math

import torch

from . import _lib
from .kernel import _require_cuda, _stream

MAX_SPLITS = 32
_ARCH_ATTN = {"deepseek_v3_2": (128, 64, 40.0), "glm_5": (192, 64, None)}


def softmax_scale(model_arch: str) -> float:
    """FlashSparseMLACombine.softmax_scale (ops/flash_sparse_mla.py:125-130) for the model's
    head dims and rope factor (deepseek_v3_2/model_args.py:76-82, glm_5/model_args.py:42-48)."""
    if model_arch not in _ARCH_ATTN:
        raise ValueError(f"unsupported model_arch {model_arch!r}")
    nope, rope, factor = _ARCH_ATTN[model_arch]
    mscale = 1.0 if factor is None else 0.1 * math.log(factor) + 1.0
    return (nope + rope) ** -0.5 * mscale * mscale


def flash_sparse_mla(query: torch.Tensor, query_pe: torch.Tensor, key_value: torch.Tensor,
                     key_pe: torch.Tensor, indices: torch.Tensor, cur_pos: torch.Tensor,
                     output: torch.Tensor, profile_logs: torch.Tensor | None, split_size: int = 64,
                     compute_kernel_type: str = "bf16mma", *, model_arch: str,
                     scale: float | None = None) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """query bf16 [1, s, heads, 512], query_pe bf16 [1, s, heads, 64], key_value bf16
    [1, T, 512], key_pe bf16 [1, T, 64], indices int32 [1, s, topk] (distinct positions;
    entries outside [0, T) are ignored, e.g. top-k's -1 padding), cur_pos int32 [1] on the
    device; ``output`` bf16 [1, s, heads, 512] is filled.  Returns (lse [1, s, heads],
    lse_acc [1, s, heads, 32], output_acc [1, s, heads, 32, 512]), fp32.  ``scale``
    overrides the model's softmax scale."""
    batch, seqlen, heads, hidden_dim = query.shape
    if split_size != 64:
        raise ValueError("The current implementation of flash_sparse_mla_op only supports split_size=64")
    if batch != 1:
        raise ValueError("The current implementation of flash_sparse_mla_op only supports batch=1")
    if seqlen > 4:
        raise ValueError("The current implementation of flash_sparse_mla_op only supports seqlen<=4")
    seqlen_kv = key_value.shape[1]
    index_len = indices.shape[-1]
    if index_len > seqlen_kv:
        raise ValueError("index_len must be less than or equal to seqlen_kv")
    if heads not in (8, 10, 16, 20):
        raise ValueError(f"Unsupported heads: {heads}")
    if compute_kernel_type != "bf16mma":
        raise ValueError(f"unsupported compute_kernel_type {compute_kernel_type!r}")
    if hidden_dim != 512 or key_value.shape[-1] != 512 or query_pe.shape[-1] != 64 or key_pe.shape[-1] != 64:
        raise ValueError("flash_sparse_mla expects a 512-wide latent and 64-wide rope part")
    for name, t in (("query", query), ("query_pe", query_pe), ("key_value", key_value), ("key_pe", key_pe),
                    ("output", output)):
        if t.dtype != torch.bfloat16 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous bfloat16 tensor")
    if indices.dtype != torch.int32 or not indices.is_contiguous():
        raise ValueError("indices must be a contiguous int32 tensor")
    if cur_pos.dtype != torch.int32:
        raise ValueError("cur_pos must be an int32 tensor")
    if output.numel() != seqlen * heads * 512:
        raise ValueError("output must hold [1, seqlen, heads, 512]")
    device = query.device
    if any(t.device != device for t in (query_pe, key_value, key_pe, indices, cur_pos, output)):
        raise RuntimeError("flash_sparse_mla inputs must be on the same device")
    _require_cuda("flash_sparse_mla", query)
    sm = softmax_scale(model_arch) if scale is None else float(scale)
    lse = torch.empty(batch, seqlen, heads, device=device, dtype=torch.float32)
    lse_acc = torch.empty(batch, seqlen, heads, MAX_SPLITS, device=device, dtype=torch.float32)
    output_acc = torch.empty(batch, seqlen, heads, MAX_SPLITS, 512, device=device, dtype=torch.float32)
    _lib.call("tl_flash_sparse_mla", query.data_ptr(), query_pe.data_ptr(), key_value.data_ptr(), key_pe.data_ptr(),
              indices.data_ptr(), cur_pos.data_ptr(), seqlen, heads, index_len, seqlen_kv, sm, output.data_ptr(),
              output_acc.data_ptr(), lse.data_ptr(), lse_acc.data_ptr(), _stream(query))
    return lse, lse_acc, output_acc
