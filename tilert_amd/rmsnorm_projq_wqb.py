"""RMSNorm of the q latent fused with the wq_b projection, with the reference operator's
signature (tilert/models/deepseek_v3_2/ops/rmsnorm_projq_wqb.py:20-44; golden
RmsnormProjqWqb.golden_forward :496-512): bf16 activations times the fp8 weight dequantised
to bf16 (BF16MMA), one launch."""
from __future__ import annotations

import torch

from . import _lib
from .kernel import PackedFP8Weight, _require_cuda, _stream

EPS = {"deepseek_v3_2": 1e-6, "glm_5": 1e-5}  # model_args.eps (deepseek_v3_2/model_args.py:95, glm_5/model_args.py:59)
_HEAD_DIMS = {"deepseek_v3_2": (128, 64), "glm_5": (192, 64)}  # (qk_nope_head_dim, qk_rope_head_dim)


def rmsnorm_projq_wqb_op(q: torch.Tensor, wq_b: PackedFP8Weight, wq_b_scales: torch.Tensor | None,
                         q_norm_weight: torch.Tensor, q_nope: torch.Tensor, q_pe: torch.Tensor,
                         profile_logs: torch.Tensor | None, algorithm: str, model_arch: str) -> None:
    """q bf16 [1, s, q_rank]; wq_b the [heads * (nope + rope), q_rank] e4m3fn weight packed
    with ``pack_weight`` (its scales are used when ``wq_b_scales`` is None); q_norm_weight
    fp32 [q_rank]; q_nope bf16 [1, s, heads, nope] and q_pe bf16 [1, s, heads, rope] are
    filled.  ``algorithm`` must be "bf16mma" (the golden's numerics); ``profile_logs`` is
    accepted and left untouched."""
    if algorithm not in ("bf16mma", "bf16"):
        raise ValueError(f"unsupported algorithm {algorithm!r} (this op runs BF16MMA)")
    if model_arch not in _HEAD_DIMS:
        raise ValueError(f"unsupported model_arch {model_arch!r}")
    nope_dim, rope_dim = _HEAD_DIMS[model_arch]
    if not isinstance(wq_b, PackedFP8Weight):
        raise ValueError("wq_b must be a PackedFP8Weight (tilert_amd.kernel.pack_weight)")
    bsz, seqlen, q_rank = q.shape
    if bsz != 1 or seqlen not in (1, 2, 4):
        raise ValueError(f"Invalid batch size or sequence length: bsz={bsz}, seqlen={seqlen}")
    if q.dtype != torch.bfloat16 or q_nope.dtype != torch.bfloat16 or q_pe.dtype != torch.bfloat16:
        raise ValueError("q, q_nope and q_pe must be bfloat16 tensors")
    if q_norm_weight.dtype != torch.float32 or q_norm_weight.numel() != q_rank:
        raise ValueError("q_norm_weight must be a float32 [q_rank] tensor")
    scales = wq_b.scale if wq_b_scales is None else wq_b_scales
    if scales.dtype != torch.float32:
        raise ValueError("wq_b_scales must be float32")
    heads = wq_b.N // (nope_dim + rope_dim)
    if wq_b.K != q_rank or heads * (nope_dim + rope_dim) != wq_b.N:
        raise ValueError("wq_b must be [heads * (nope + rope), q_rank]")
    if q_nope.shape != (1, seqlen, heads, nope_dim) or q_pe.shape != (1, seqlen, heads, rope_dim):
        raise ValueError("q_nope / q_pe must be [1, s, heads, nope] / [1, s, heads, rope]")
    tensors = (q, q_norm_weight, scales, q_nope, q_pe)
    if not all(t.is_contiguous() for t in tensors):
        raise ValueError("rmsnorm_projq_wqb inputs must be contiguous")
    _require_cuda("rmsnorm_projq_wqb", q, q_norm_weight, wq_b.data, scales, q_nope, q_pe)
    _lib.call("tl_rmsnorm_projq_wqb", q.data_ptr(), q_norm_weight.data_ptr(), EPS[model_arch], wq_b.data.data_ptr(),
              scales.data_ptr(), q_nope.data_ptr(), q_pe.data_ptr(), seqlen, heads, q_rank, nope_dim, rope_dim,
              _stream(q))
