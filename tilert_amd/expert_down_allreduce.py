"""``expert_down_allreduce`` with the reference operator's signature
(tilert/models/deepseek_v3_2/ops/expert_down_allreduce.py:23-63) on the gfx950 HIP library:
the down projection of the shared expert and each token's selected experts, each term
weighted by its routing probability (the shared one by 1) and rounded to bf16, summed in
fp32 (golden :445-468), plus the residual ``x_in``.

One device's share of the tensor-parallel split: the cross-device sum (the allreduce) is
the identity on one GPU, so the result is ``bf16(partial + x_in)``, the single-GPU form of
the reference's allreduce-add epilogue (padded_allreduce_add.py:100-114).  ``flag`` (the
allreduce's synchronisation flag) is accepted and unused.
"""
from __future__ import annotations

import torch

from . import _lib
from .kernel import _require_cuda, _stream
from .moe import pack_moe_weight

BLOCK = 128


class DownExperts:
    """Stacked down weights of ``n_local`` experts (or dense-MLP chunks): e4m3fn
    [n_local, D, I] with scales [n_local, D/128, I/128], packed tile-major for the kernels
    (the role of ``ExpertDownAllReduceWeightsConverter``, :112-229)."""

    def __init__(self, down: torch.Tensor, down_s: torch.Tensor) -> None:
        if down.dtype != torch.float8_e4m3fn or down.dim() != 3:
            raise ValueError("down weights must be 3-D float8_e4m3fn [n_local, D, I]")
        E, D, I = down.shape
        if I % BLOCK or D % BLOCK:
            raise ValueError("I and D must be multiples of 128")
        if down_s.shape != (E, D // BLOCK, I // BLOCK):
            raise ValueError("scales must be [n_local, D/128, I/128]")
        _require_cuda("DownExperts", down, down_s)
        self.n_local, self.D, self.I = E, D, I
        self.w2 = pack_moe_weight(down.reshape(E * D, I).contiguous())
        self.s2 = down_s.float().contiguous()

    @property
    def device(self) -> torch.device:
        return self.w2.device


def _check_out(vec_out: torch.Tensor, x_in: torch.Tensor | None, s: int, D: int, who: str) -> None:
    if vec_out.dtype != torch.bfloat16 or vec_out.numel() != s * D or not vec_out.is_contiguous():
        raise ValueError(f"{who}: vec_out must be a contiguous bfloat16 [1, s, {D}] tensor")
    if x_in is not None and (x_in.dtype != torch.bfloat16 or x_in.numel() != s * D or not x_in.is_contiguous()):
        raise ValueError(f"{who}: x_in must be a contiguous bfloat16 [1, s, {D}] tensor")


def expert_down_allreduce(vec_in: torch.Tensor, mat_in: DownExperts, mat_scale: torch.Tensor | None,
                          indices: torch.Tensor, scores: torch.Tensor, x_in: torch.Tensor | None, flag: int,
                          vec_out: torch.Tensor, profile_logs: torch.Tensor | None = None,
                          model_arch: str = "deepseek_v3_2", compute_kernel_type: str = "bf16") -> None:
    """vec_in bf16 [1, s, 1 + topk, I] (``expert_select_up_gate_silu``'s hidden_out);
    mat_in = ``DownExperts`` of the shared expert then the routed experts (its scales ride
    along, so ``mat_scale`` may be None); indices int32 / scores fp32 [1, s, topk] (the
    routing outputs); x_in bf16 [1, s, D] residual or None; vec_out bf16 [1, s, D]."""
    if model_arch not in ("deepseek_v3_2", "glm_5"):
        raise ValueError(f"Unsupported architecture: {model_arch}")
    if compute_kernel_type not in ("bf16", "bf16mma", "general"):
        raise ValueError(f"Unsupported compute_kernel_type: {compute_kernel_type}")
    ex = mat_in
    if vec_in.dtype != torch.bfloat16 or vec_in.dim() != 4 or vec_in.shape[0] != 1 or vec_in.shape[-1] != ex.I:
        raise ValueError(f"vec_in must be bfloat16 [1, s, 1 + topk, {ex.I}]")
    s, P = vec_in.shape[1], vec_in.shape[2]
    topk = P - 1
    if indices.dtype != torch.int32 or indices.numel() != s * topk:
        raise ValueError(f"indices must be int32 [1, s, {topk}]")
    if scores.dtype != torch.float32 or scores.numel() != s * topk:
        raise ValueError(f"scores must be float32 [1, s, {topk}]")
    _check_out(vec_out, x_in, s, ex.D, "expert_down_allreduce")
    ts = (vec_in, indices, scores, x_in, vec_out)
    if not all(t.is_contiguous() for t in ts if t is not None):
        raise ValueError("expert_down_allreduce tensors must be contiguous")
    _require_cuda("expert_down_allreduce", *ts, ex.w2, ex.s2)
    _lib.call("tl_expert_down_allreduce", vec_in.data_ptr(), ex.w2.data_ptr(), ex.s2.data_ptr(), indices.data_ptr(),
              scores.data_ptr(), x_in.data_ptr() if x_in is not None else None, s, ex.n_local - 1, topk, ex.D,
              ex.I, vec_out.data_ptr(), _stream(vec_in))


def device_down_shard(down: torch.Tensor, down_s: torch.Tensor, device_id: int, num_devices: int
                      ) -> tuple[torch.Tensor, torch.Tensor]:
    """One device's slice of full down weights [n_local, D, moe_inter] (+ scales): columns
    ``device_id * moe_inter / num_devices ..`` of every expert (``process_down_weights``,
    :325-352)."""
    inter = down.shape[2]
    if inter % (num_devices * BLOCK):
        raise ValueError("moe_inter_dim must split into 128-column blocks per device")
    per = inter // num_devices
    c = slice(device_id * per, (device_id + 1) * per)
    cs = slice(device_id * per // BLOCK, (device_id + 1) * per // BLOCK)
    return down[:, :, c].contiguous(), down_s[:, :, cs].contiguous()
