"""``expert_select_up_gate_silu`` with the reference operator's signature
(tilert/models/deepseek_v3_2/ops/expert_sel_up_gate_silu.py:23-48) on the gfx950 HIP library:
the router's top-k on the device, then gate/up + SwiGLU of the shared expert and each
token's selected experts, at one device's share of the tensor-parallel split of the
experts' intermediate dim.

The weight converter (the role of ``ExpertSelectUpGateSiLUWeightsConverter``, :107-334) is
``UpGateExperts``: the device's stacked gate/up slices -- expert 0 the shared expert, then
the routed experts (``device_sharding``, :478-512) -- packed once into the MoE kernels'
fragment layout with their fp32 128x128 block scales.
"""
from __future__ import annotations

import torch

from . import _lib
from .kernel import _require_cuda, _stream
from .moe import pack_moe_weight

BLOCK = 128

# (n_expert_groups, n_limited_groups, n_activated_experts, route_scale) per model_arch:
# deepseek_v3_2/model_args.py:66-72; GLM-5 routes without groups
# (deepseek_v3_2/ops/expert_sel_up_gate_silu.py:641-652, glm_5/model_args.py:32-38)
ROUTING = {
    "deepseek_v3_2": (8, 4, 8, 2.5),
    "glm_5": (1, 1, 8, 2.5),
}


class UpGateExperts:
    """Stacked gate/up weights of ``n_local`` experts (or dense-MLP chunks): gate, up
    e4m3fn [n_local, I, D] with scales [n_local, I/128, D/128] (fp32 or bf16), packed
    tile-major ([I gate rows, I up rows] per expert) for the HIP kernels."""

    def __init__(self, gate: torch.Tensor, gate_s: torch.Tensor, up: torch.Tensor, up_s: torch.Tensor) -> None:
        if gate.dtype != torch.float8_e4m3fn or up.dtype != torch.float8_e4m3fn or gate.dim() != 3:
            raise ValueError("gate/up weights must be 3-D float8_e4m3fn [n_local, I, D]")
        if up.shape != gate.shape:
            raise ValueError("gate and up shapes differ")
        E, I, D = gate.shape
        if I % BLOCK or D % BLOCK:
            raise ValueError("I and D must be multiples of 128")
        if gate_s.shape != (E, I // BLOCK, D // BLOCK) or up_s.shape != gate_s.shape:
            raise ValueError("scales must be [n_local, I/128, D/128]")
        _require_cuda("UpGateExperts", gate, gate_s, up, up_s)
        self.n_local, self.I, self.D = E, I, D
        self.w13 = pack_moe_weight(torch.cat([gate, up], dim=1).reshape(E * 2 * I, D).contiguous())
        self.s13 = torch.cat([gate_s, up_s], dim=1).float().contiguous()

    @property
    def device(self) -> torch.device:
        return self.w13.device


def expert_select_up_gate_silu(hidden_in: torch.Tensor, scores_in: torch.Tensor, bias_in: torch.Tensor | None,
                               experts_weights_in: UpGateExperts, hidden_out: torch.Tensor,
                               expert_probs_out: torch.Tensor, expert_indices_out: torch.Tensor,
                               profile_logs: torch.Tensor | None = None, algorithm: str = "bf16mma", *,
                               model_arch: str) -> None:
    """hidden_in bf16 [1, s, D]; scores_in fp32 [1, s, n_routed] router logits; bias_in fp32
    [n_routed] (the e_score_correction_bias, or None); experts_weights_in = ``UpGateExperts``
    of the shared expert then the n_routed experts; hidden_out bf16 [1, s, 1 + topk, I]
    (position 0 the shared expert, then the selected experts in descending routing score);
    expert_probs_out fp32 [1, s, topk] (normalised, times route_scale); expert_indices_out
    int32 [1, s, topk].  ``algorithm``: the kernel computes with bf16 activations and the
    bf16-rounded dequantised weights of the golden whatever the name ("fp8mma", "fp16mma"
    and "bf16mma" are accepted); ``profile_logs`` is accepted and left untouched."""
    if model_arch not in ROUTING:
        raise ValueError(f"Unsupported architecture: {model_arch}")
    if algorithm not in ("fp8mma", "fp16mma", "bf16mma"):
        raise ValueError(f"Unsupported algorithm: {algorithm}")
    n_groups, topk_groups, topk, route_scale = ROUTING[model_arch]
    ex = experts_weights_in
    if hidden_in.dtype != torch.bfloat16 or hidden_in.shape[-1] != ex.D:
        raise ValueError("hidden_in must be bfloat16 [1, s, dim]")
    if hidden_in.dim() != 3 or hidden_in.shape[0] != 1:
        raise ValueError("hidden_in must be [1, s, dim] (batch 1)")
    s = hidden_in.shape[1]
    n_routed = ex.n_local - 1
    if scores_in.dtype != torch.float32 or scores_in.numel() != s * n_routed:
        raise ValueError(f"scores_in must be float32 [1, s, {n_routed}]")
    if bias_in is not None and (bias_in.dtype != torch.float32 or bias_in.numel() != n_routed):
        raise ValueError(f"bias_in must be float32 [{n_routed}]")
    if hidden_out.dtype != torch.bfloat16 or hidden_out.numel() != s * (1 + topk) * ex.I:
        raise ValueError(f"hidden_out must be bfloat16 [1, s, {1 + topk}, {ex.I}]")
    if expert_probs_out.dtype != torch.float32 or expert_probs_out.numel() != s * topk:
        raise ValueError(f"expert_probs_out must be float32 [1, s, {topk}]")
    if expert_indices_out.dtype != torch.int32 or expert_indices_out.numel() != s * topk:
        raise ValueError(f"expert_indices_out must be int32 [1, s, {topk}]")
    ts = (hidden_in, scores_in, bias_in, hidden_out, expert_probs_out, expert_indices_out)
    if not all(t.is_contiguous() for t in ts if t is not None):
        raise ValueError("expert_select_up_gate_silu tensors must be contiguous")
    _require_cuda("expert_select_up_gate_silu", *ts, ex.w13, ex.s13)
    _lib.call("tl_expert_select_up_gate_silu", hidden_in.data_ptr(), scores_in.data_ptr(),
              bias_in.data_ptr() if bias_in is not None else None, ex.w13.data_ptr(), ex.s13.data_ptr(), s,
              n_routed, topk, n_groups, topk_groups, route_scale, ex.D, ex.I, hidden_out.data_ptr(),
              expert_probs_out.data_ptr(), expert_indices_out.data_ptr(), _stream(hidden_in))


def expert_select(scores_in: torch.Tensor, bias_in: torch.Tensor | None, expert_probs_out: torch.Tensor,
                  expert_indices_out: torch.Tensor, *, model_arch: str) -> None:
    """The routing alone (``_ref_expert_select_ds`` / ``_ref_expert_select_glm5``):
    scores_in fp32 [..., n_routed] -> expert_probs_out fp32 / expert_indices_out int32
    [..., topk]."""
    if model_arch not in ROUTING:
        raise ValueError(f"Unsupported architecture: {model_arch}")
    n_groups, topk_groups, topk, route_scale = ROUTING[model_arch]
    n_routed = scores_in.shape[-1]
    T = scores_in.numel() // n_routed
    if scores_in.dtype != torch.float32 or not scores_in.is_contiguous():
        raise ValueError("scores_in must be a contiguous float32 tensor")
    if expert_probs_out.numel() != T * topk or expert_indices_out.numel() != T * topk or \
            expert_probs_out.dtype != torch.float32 or expert_indices_out.dtype != torch.int32:
        raise ValueError(f"outputs must be float32 / int32 [..., {topk}]")
    if bias_in is not None and (bias_in.dtype != torch.float32 or bias_in.numel() != n_routed):
        raise ValueError(f"bias_in must be float32 [{n_routed}]")
    _require_cuda("expert_select", scores_in, bias_in, expert_probs_out, expert_indices_out)
    _lib.call("tl_moe_route", scores_in.data_ptr(), bias_in.data_ptr() if bias_in is not None else None, T,
              n_routed, topk, n_groups, topk_groups, route_scale, expert_probs_out.data_ptr(),
              expert_indices_out.data_ptr(), _stream(scores_in))


def device_gate_up_shard(gate: torch.Tensor, gate_s: torch.Tensor, up: torch.Tensor, up_s: torch.Tensor,
                         device_id: int, num_devices: int) -> tuple[torch.Tensor, ...]:
    """One device's slice of full expert weights [n_local, moe_inter, D] (+ scales): rows
    ``device_id * moe_inter / num_devices ..`` of every expert, as the reference's
    ``process_gate_up_weights`` / ``device_sharding`` cut them (:430-512)."""
    inter = gate.shape[1]
    if inter % (num_devices * BLOCK):
        raise ValueError("moe_inter_dim must split into 128-row blocks per device")
    per = inter // num_devices
    r = slice(device_id * per, (device_id + 1) * per)
    rs = slice(device_id * per // BLOCK, (device_id + 1) * per // BLOCK)
    return (gate[:, r].contiguous(), gate_s[:, rs].contiguous(), up[:, r].contiguous(), up_s[:, rs].contiguous())
