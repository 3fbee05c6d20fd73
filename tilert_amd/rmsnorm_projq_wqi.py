"""The indexer's query projection with the reference operator's signature
(tilert/models/deepseek_v3_2/ops/rmsnorm_projq_wqi.py:17-37; golden
RmsnormProjqWqi.golden_forward :301-314): RMSNorm of the q latent, rounded to bf16, times
the fp8 wq_b of the indexer (index_n_heads * index_head_dim rows) dequantised to bf16, as
iq [1, s, heads, head_dim].  The same one-launch kernel as ``rmsnorm_projq_wqb`` with no
rope split."""
from __future__ import annotations

import torch

from . import _lib
from .kernel import PackedFP8Weight, _require_cuda, _stream

EPS = {"deepseek_v3_2": 1e-6, "glm_5": 1e-5}
HEAD_DIM = 128  # index_head_dim (deepseek_v3_2/model_args.py)


def rmsnorm_projq_wqi_op(q: torch.Tensor, wqi: PackedFP8Weight, wqi_scale: torch.Tensor | None,
                         rmsnorm_gamma: torch.Tensor, iq: torch.Tensor, profile_logs: torch.Tensor | None,
                         algorithm: str, model_arch: str) -> None:
    """q bf16 [1, s, q_rank] (s in 1, 2, 4, 8); wqi = ``pack_weight`` of the [heads * 128,
    q_rank] e4m3fn weight (its scales are used when ``wqi_scale`` is None); rmsnorm_gamma
    fp32 [q_rank]; iq bf16 [1, s, heads, 128].  ``algorithm`` "fp16mma" / "bf16mma": the
    kernel runs bf16 MMA on the golden's bf16 operands."""
    if algorithm not in ("fp16mma", "bf16mma"):
        raise ValueError(f"unsupported algorithm {algorithm!r}")
    if model_arch not in EPS:
        raise ValueError(f"unsupported model_arch {model_arch!r}")
    if not isinstance(wqi, PackedFP8Weight):
        raise ValueError("wqi must be a PackedFP8Weight (tilert_amd.kernel.pack_weight)")
    bsz, seqlen, q_rank = q.shape
    if bsz != 1 or seqlen not in (1, 2, 4, 8):
        raise ValueError(f"Invalid batch size or sequence length: bsz={bsz}, seqlen={seqlen}")
    if q.dtype != torch.bfloat16 or iq.dtype != torch.bfloat16:
        raise ValueError("q and iq must be bfloat16 tensors")
    gamma = rmsnorm_gamma.reshape(-1).to(torch.float32).contiguous()
    if gamma.numel() != q_rank:
        raise ValueError("rmsnorm_gamma must be [q_rank]")
    scales = wqi.scale if wqi_scale is None else wqi_scale.float().contiguous()
    heads = wqi.N // HEAD_DIM
    if wqi.K != q_rank or heads * HEAD_DIM != wqi.N:
        raise ValueError("wqi must be [heads * 128, q_rank]")
    if iq.shape != (1, seqlen, heads, HEAD_DIM) or not iq.is_contiguous() or not q.is_contiguous():
        raise ValueError(f"iq must be a contiguous [1, s, {heads}, {HEAD_DIM}] tensor")
    _require_cuda("rmsnorm_projq_wqi", q, gamma, wqi.data, scales, iq)
    _lib.call("tl_rmsnorm_projq_wqb", q.data_ptr(), gamma.data_ptr(), EPS[model_arch], wqi.data.data_ptr(),
              scales.data_ptr(), iq.data_ptr(), None, seqlen, heads, q_rank, HEAD_DIM, 0, _stream(q))
