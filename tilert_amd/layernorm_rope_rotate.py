"""Indexer key producer with the reference operator's shape
(tilert/models/deepseek_v3_2/ops/layernorm_rope_rotate.py:23-82; golden_forward :206-220):
LayerNorm -> non-interleaved RoPE on dims 0..63 -> 128-point Hadamard (scale 128^-1/2),
written to the bf16 key cache at ``cur_pos``; and its fused variant that quantises the
keys straight into the fp8 KI page cache the paged indexer reads."""
from __future__ import annotations

import torch

from . import _lib
from .kernel import SCALE_MODES, _require_cuda, _stream
from .sparse_index import KI_PAGE_BYTES

LN_EPS = 1e-6  # golden_forward's F.layer_norm eps (ops/layernorm_rope_rotate.py:207-213)


def _check(input_raw, cur_pos, weight, bias, freqs_cis):
    if input_raw.dtype != torch.bfloat16:
        raise ValueError("input must be a bfloat16 tensor.")
    if cur_pos.dtype != torch.int32:
        raise ValueError("cur_pos must be a int32 tensor.")
    if weight.dtype != torch.float32:
        raise ValueError("weight must be a float32 tensor.")
    if bias.dtype != torch.float32:
        raise ValueError("bias must be a float32 tensor.")
    if freqs_cis.dtype != torch.float32:
        raise ValueError("freqs_cis must be a float32 tensor.")
    batch, seq, dim = input_raw.shape
    if dim != 128:
        raise ValueError("dim must be 128, as we precompute scale inner kernel")
    if batch != 1:
        raise ValueError("batch must be 1 in this version")
    if weight.numel() != 128 or bias.numel() != 128:
        raise ValueError("weight and bias must hold 128 values")
    if freqs_cis.numel() != seq * 64:
        raise ValueError("freqs_cis must be the fp32 [seq, 1, 64] (cos, sin) view of the seq tokens' freqs")
    tensors = (input_raw, cur_pos, weight, bias, freqs_cis)
    if any(t.device != input_raw.device for t in tensors):
        raise ValueError("layernorm_rope_rotate inputs must be on the same device")
    if not all(t.is_contiguous() for t in tensors):
        raise ValueError("layernorm_rope_rotate inputs must be contiguous")
    _require_cuda("layernorm_rope_rotate", input_raw)
    return seq


def layernorm_rope_rotate(input_raw: torch.Tensor, cur_pos: torch.Tensor, k_cache_raw: torch.Tensor,
                          weight: torch.Tensor, bias: torch.Tensor, freqs_cis: torch.Tensor,
                          profile_logs: torch.Tensor | None, model_arch: str,
                          compute_kernel_type: str = "general") -> None:
    """input_raw bf16 [1, seq, 128]; cur_pos int32 [1] (device); k_cache_raw bf16
    [1, rows, 128] receives key t at row cur_pos + t (rows outside the cache are dropped);
    weight, bias fp32 [128]; freqs_cis fp32 [seq, 1, 64] (the op's view_as_real of the
    seq tokens' freqs_cis, layernorm_rope_rotate.py:224-226).  ``profile_logs`` is
    accepted and left untouched."""
    seq = _check(input_raw, cur_pos, weight, bias, freqs_cis)
    if compute_kernel_type != "general":
        raise ValueError(f"unsupported compute_kernel_type {compute_kernel_type!r}")
    if k_cache_raw.dtype != torch.bfloat16:
        raise ValueError("k_cache must be a bfloat16 tensor.")
    if k_cache_raw.shape[-1] != 128 or not k_cache_raw.is_contiguous() or k_cache_raw.device != input_raw.device:
        raise ValueError("k_cache must be a contiguous [1, rows, 128] tensor on the input's device")
    rows = k_cache_raw.numel() // 128
    _lib.call("tl_layernorm_rope_rotate", input_raw.data_ptr(), seq, cur_pos.data_ptr(), k_cache_raw.data_ptr(),
              rows, weight.data_ptr(), bias.data_ptr(), freqs_cis.data_ptr(), LN_EPS, _stream(input_raw))


def layernorm_rope_rotate_ki(input_raw: torch.Tensor, cur_pos: torch.Tensor, ki_pages: torch.Tensor,
                             weight: torch.Tensor, bias: torch.Tensor, freqs_cis: torch.Tensor,
                             scale_fmt: str | None = "div") -> None:
    """The same keys, quantised per key (``act_quant`` of the bf16 result with ``scale_fmt``)
    into the KI pages (uint8 [n_pages, 8448]) at positions cur_pos + t: byte-identical to
    ``layernorm_rope_rotate`` followed by ``ki_cache_write``, in one launch."""
    seq = _check(input_raw, cur_pos, weight, bias, freqs_cis)
    if ki_pages.dtype != torch.uint8 or ki_pages.dim() != 2 or ki_pages.shape[1] != KI_PAGE_BYTES \
            or not ki_pages.is_contiguous() or ki_pages.device != input_raw.device:
        raise ValueError(f"ki_pages must be a contiguous uint8 [n_pages, {KI_PAGE_BYTES}] tensor on the input's device")
    _lib.call("tl_layernorm_rope_rotate_ki", input_raw.data_ptr(), seq, cur_pos.data_ptr(), ki_pages.data_ptr(),
              ki_pages.shape[0], weight.data_ptr(), bias.data_ptr(), freqs_cis.data_ptr(), LN_EPS,
              SCALE_MODES.get(scale_fmt, 1), _stream(input_raw))
