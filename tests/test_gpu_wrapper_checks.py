"""Every tensor a wrapper hands to a kernel must be on the GPU: a host tensor among the
outputs or the weights is rejected with ValueError before anything is launched."""
import pytest
import torch

from tilert_amd import kernel as K
from tilert_amd import moe
from tilert_amd.rmsnorm import rmsnorm_quant

pytestmark = pytest.mark.gpu


def test_rmsnorm_quant_rejects_host_tensors(cuda):
    x = torch.randn(2, 256, device=cuda).to(torch.bfloat16)
    gamma = torch.ones(256, device=cuda)
    out = torch.empty_like(x)
    q = torch.empty(2, 256, dtype=torch.float8_e4m3fn, device=cuda)
    s = torch.empty(2, 2, device=cuda)
    logs = torch.zeros(1, device=cuda)
    rmsnorm_quant(x, gamma, out, q, s, logs, model_arch="deepseek_v3_2")  # all on the GPU: fine
    for args in ((x, gamma.cpu(), out, q, s), (x, gamma, out.cpu(), q, s), (x, gamma, out, q.cpu(), s),
                 (x, gamma, out, q, s.cpu())):
        with pytest.raises(ValueError):
            rmsnorm_quant(*args, logs, model_arch="deepseek_v3_2")


def _experts(cuda):
    E, D, I = 2, 256, 128
    g = torch.zeros(E, I, D, dtype=torch.float8_e4m3fn, device=cuda)
    d = torch.zeros(E, D, I, dtype=torch.float8_e4m3fn, device=cuda)
    return moe.LocalExperts(g, torch.ones(E, 1, 2, device=cuda), g.clone(), torch.ones(E, 1, 2, device=cuda),
                            d, torch.ones(E, 2, 1, device=cuda))


def test_moe_rejects_host_outputs(cuda):
    ex = _experts(cuda)
    x = torch.zeros(1, 256, dtype=torch.bfloat16, device=cuda)
    idx = torch.zeros(1, 2, dtype=torch.int32, device=cuda)
    w = torch.ones(1, 2, device=cuda)
    with pytest.raises(ValueError):
        moe.ep_gate_up_swiglu(x, idx, ex, torch.empty(2, 1, 128, dtype=torch.bfloat16))
    h = moe.ep_gate_up_swiglu(x, idx, ex)
    with pytest.raises(ValueError):
        moe.ep_down_combine(h, ex, idx, w, vec_out=torch.empty(1, 256, dtype=torch.bfloat16))
    ex.w2 = ex.w2.cpu()
    with pytest.raises(ValueError):
        moe.ep_down_combine(h, ex, idx, w)


def test_fp8_gemm_rejects_host_output(cuda):
    a = torch.zeros(1, 512, dtype=torch.float8_e4m3fn, device=cuda)
    b = torch.zeros(128, 512, dtype=torch.float8_e4m3fn, device=cuda)
    with pytest.raises(ValueError):
        K.fp8_gemm(a, torch.ones(1, 4, device=cuda), b, torch.ones(1, 4, device=cuda),
                   out=torch.empty(1, 128, dtype=torch.bfloat16))
