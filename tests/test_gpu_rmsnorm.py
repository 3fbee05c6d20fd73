"""GPU parity of the fused RMSNorm + act_quant (rmsnorm_quant_op) against the CPU oracle."""
import pytest
import torch

from oracle import reference as ref
from tilert_amd import kernel as K
from tilert_amd import synth
from tilert_amd.rmsnorm import rmsnorm_quant

pytestmark = pytest.mark.gpu

LOGS = torch.zeros(1)  # the reference op requires a profile_logs tensor


def _bf16_ulps(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Distance in bf16 steps (sign-magnitude bit patterns as integers)."""
    def key(t):
        i = t.view(torch.int16).to(torch.int32)
        return torch.where(i < 0, -(i & 0x7fff), i)
    return (key(a) - key(b)).abs()


@pytest.mark.parametrize("rows,dim,scale_fmt", [
    (4, 7168, None),     # DeepSeek-V3.2 hidden size, decode M = 4
    (7, 6144, "div"),    # GLM-5 hidden size
    (1, 128, "ue8m0"),
    (33, 16384, None),   # the largest supported row
    (2, 2176, None),     # 272 chunks: a second row slice with 16 live chunks
    (3, 10240, "ue8m0"),  # 1280 chunks: the first 256 virtual threads sum two chunks
])
def test_rmsnorm_quant_vs_oracle(cuda, rows, dim, scale_fmt):
    g = synth.gen(rows * 1000 + dim)
    x = (torch.randn(rows, dim, generator=g) * 2).to(torch.bfloat16)
    x[0, :128] = 0.0                      # an all-zero quantisation group
    w = 1 + 0.1 * torch.randn(dim, generator=g)
    xd, wd = x.to(cuda), w.to(cuda)
    y = torch.empty_like(xd)
    q = torch.empty(rows, dim, dtype=torch.float8_e4m3fn, device=cuda)
    s = torch.empty(rows, dim // 128, dtype=torch.float32, device=cuda)
    rmsnorm_quant(xd, wd, y, q, s, LOGS, model_arch="deepseek_v3_2", scale_fmt=scale_fmt)
    want = ref.rmsnorm(x, w)
    d = _bf16_ulps(y.cpu(), want)
    # fp32 sums in a different order: at most one bf16 step, and almost always none
    assert d.max() <= 1 and (d > 0).float().mean() < 1e-3
    # the quantised outputs are act_quant of the kernel's own bf16 norm, bit for bit
    mode = {None: ref.SCALE_MODE_REFERENCE, "ue8m0": ref.SCALE_MODE_UE8M0, "div": 2}[scale_fmt]
    q_ref, s_ref = ref.act_quant(y.cpu(), 128, mode)
    assert torch.equal(q.cpu().view(torch.uint8), q_ref.view(torch.uint8))
    assert torch.equal(s.cpu(), s_ref)
    q2, s2 = K.act_quant(y, scale_fmt=scale_fmt)
    assert torch.equal(q.view(torch.uint8), q2.view(torch.uint8)) and torch.equal(s, s2)


def test_rmsnorm_without_quant_outputs(cuda):
    g = synth.gen(9)
    x = torch.randn(5, 7168, generator=g).to(torch.bfloat16).to(cuda)
    w = torch.rand(7168, generator=g).to(cuda) + 0.5
    y1, y2 = torch.empty_like(x), torch.empty_like(x)
    q = torch.empty(5, 7168, dtype=torch.float8_e4m3fn, device=cuda)
    s = torch.empty(5, 56, dtype=torch.float32, device=cuda)
    rmsnorm_quant(x, w, y1, profile_logs=LOGS, model_arch="deepseek_v3_2")
    rmsnorm_quant(x, w, y2, q, s, LOGS, model_arch="deepseek_v3_2")
    assert torch.equal(y1, y2)


def test_rmsnorm_quant_argument_errors(cuda):
    x = torch.zeros(2, 7168, dtype=torch.bfloat16, device=cuda)
    w = torch.ones(7168, device=cuda)
    y = torch.empty_like(x)
    with pytest.raises(ValueError, match="profile_logs"):
        rmsnorm_quant(x, w, y, model_arch="deepseek_v3_2")
    with pytest.raises(ValueError, match="go together"):
        rmsnorm_quant(x, w, y, torch.empty(2, 7168, dtype=torch.float8_e4m3fn, device=cuda), None, LOGS,
                      model_arch="deepseek_v3_2")
