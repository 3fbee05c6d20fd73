"""Shared tolerance checks (the bars are the workload's stated ones)."""
import math

import torch


def bf16_ulp_at(x: float) -> float:
    """Spacing of bf16 numbers at magnitude x (8 significant bits)."""
    if x == 0:
        return 2.0 ** -133
    return 2.0 ** (math.floor(math.log2(abs(x))) - 7)


def assert_gemm_close(out: torch.Tensor, ref: torch.Tensor, what: str = "") -> None:
    """relative L2 <= 5e-3 and max-abs <= 2 bf16 ulp of the output scale (max |ref|)."""
    out = out.detach().float().cpu()
    ref = ref.detach().float().cpu()
    assert out.shape == ref.shape, (out.shape, ref.shape)
    assert torch.isfinite(out).all(), f"{what}: non-finite output"
    rel = (torch.norm(out - ref) / torch.norm(ref).clamp_min(1e-30)).item()
    scale = ref.abs().max().item()
    maxabs = (out - ref).abs().max().item()
    lim = 2 * bf16_ulp_at(scale)
    assert rel <= 5e-3, f"{what}: rel L2 {rel:.3e} > 5e-3"
    assert maxabs <= lim, f"{what}: max-abs {maxabs:.3e} > 2 bf16 ulp of {scale:.3e} ({lim:.3e})"
