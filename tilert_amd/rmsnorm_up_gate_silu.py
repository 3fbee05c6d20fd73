"""``rmsnorm_up_gate_silu`` with the reference operator's signature
(tilert/models/deepseek_v3_2/ops/rmsnorm_up_gate_silu.py:26-44) on the gfx950 HIP library:
RMSNorm of the hidden state, then gate/up + SwiGLU of the dense MLP's device share, in one
launch.  The share is ``n_chunks`` chunks of I rows (the reference's pseudo-experts:
inter_dim / num_devices rows cut into moe_inter_dim / num_devices blocks, :110-120),
written to hidden_out [1, s, n_chunks, I] (golden :318-347).

Numerics: the normalised rows are rounded to bf16 and the dequantised weights to bf16
(bf16 MMA, fp32 accumulation); the golden keeps both in fp32, so results agree with it to
about one bf16 step (checked at rel-L2 <= 1e-2), and with the bf16-operand restatement at
the GEMM bar.
"""
from __future__ import annotations

import torch

from . import _lib
from .expert_sel_up_gate_silu import UpGateExperts
from .kernel import _require_cuda, _stream

BLOCK = 128
EPS = {"deepseek_v3_2": 1e-6, "glm_5": 1e-5}  # model_args.py eps (deepseek_v3_2:95, glm_5:59)


def rmsnorm_up_gate_silu(hidden_in: torch.Tensor, gamma_in: torch.Tensor, weights_in: UpGateExperts,
                         hidden_out: torch.Tensor, profile_logs: torch.Tensor | None = None,
                         model_arch: str = "deepseek_v3_2", compute_kernel_type: str = "fp8mma") -> None:
    """hidden_in bf16 [1, s, D]; gamma_in fp32 [D] (bf16 is widened); weights_in =
    ``UpGateExperts`` of the device's chunks; hidden_out bf16 [1, s, n_chunks, I].
    ``compute_kernel_type`` ("fp8mma", "fp16mma", "bf16mma") is accepted; the kernel runs
    bf16 MMA (see the module notes)."""
    if model_arch not in EPS:
        raise ValueError(f"Unsupported architecture: {model_arch}")
    if compute_kernel_type not in ("fp8mma", "fp16mma", "bf16mma"):
        raise ValueError(f"Unsupported compute_kernel_type: {compute_kernel_type}")
    w = weights_in
    if hidden_in.dtype != torch.bfloat16 or hidden_in.shape[-1] != w.D or not hidden_in.is_contiguous():
        raise ValueError(f"hidden_in must be a contiguous bfloat16 [1, s, {w.D}] tensor")
    s = hidden_in.numel() // w.D
    if gamma_in.numel() != w.D:
        raise ValueError(f"gamma_in must be [{w.D}]")
    if hidden_out.dtype != torch.bfloat16 or hidden_out.numel() != s * w.n_local * w.I or not hidden_out.is_contiguous():
        raise ValueError(f"hidden_out must be a contiguous bfloat16 [1, s, {w.n_local}, {w.I}] tensor")
    gamma = gamma_in.reshape(w.D).to(torch.float32).contiguous()
    _require_cuda("rmsnorm_up_gate_silu", hidden_in, gamma, hidden_out, w.w13, w.s13)
    _lib.call("tl_rmsnorm_up_gate_silu", hidden_in.data_ptr(), gamma.data_ptr(), EPS[model_arch], w.w13.data_ptr(),
              w.s13.data_ptr(), s, w.n_local, w.D, w.I, hidden_out.data_ptr(), _stream(hidden_in))


def device_chunks(w: torch.Tensor, w_s: torch.Tensor, device_id: int, num_devices: int, n_chunks: int,
                  rows: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
    """The reference's cut of a dense weight into one device's chunks
    (rmsnorm_up_gate_silu.py:110-160, down_allreduce.py:165-212): for gate/up
    [inter, D] (``rows``), chunk i of device d is rows i * inter / n_chunks + d * c ..
    (c = inter / (n_chunks * num_devices)); for down [D, inter] (``rows=False``) the same
    columns.  Returns ([n_chunks, c, D] or [n_chunks, D, c], scales)."""
    inter = w.shape[0] if rows else w.shape[1]
    c = inter // (n_chunks * num_devices)
    if c * n_chunks * num_devices != inter or c % BLOCK:
        raise ValueError("inter_dim must split into 128-aligned chunks per device")
    parts, sparts = [], []
    for i in range(n_chunks):
        a = i * (inter // n_chunks) + device_id * c
        if rows:
            parts.append(w[a:a + c])
            sparts.append(w_s[a // BLOCK:(a + c) // BLOCK])
        else:
            parts.append(w[:, a:a + c])
            sparts.append(w_s[:, a // BLOCK:(a + c) // BLOCK])
    return torch.stack(parts).contiguous(), torch.stack(sparts).contiguous()
