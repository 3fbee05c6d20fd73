"""GPU parity of ``rmsnorm_projx_wqkva`` (the DECOUPLED RMSNormProjxWqkva,
rmsnorm_projx_wqkva.py:473-509): byte-identical to calling ``rmsnorm_quant`` then
``projx_wqkva`` by hand, and within the GEMM tolerance of the oracle's golden chain
(rms_norm, then the three projections)."""
import pytest
import torch

from oracle import reference as ref
from tests._tol import assert_gemm_close
from tilert_amd import synth
from tilert_amd.projx import ARCH_DIMS, pack_wqkva, projx_wqkva, rmsnorm_projx_wqkva
from tilert_amd.rmsnorm import rmsnorm_quant

pytestmark = pytest.mark.gpu
LOGS = torch.zeros(1)
SENTINEL = -12352.0


def _case(cuda, batch, seq, arch, max_len, pos, scale_fmt, seed):
    dim, q_rank, kv_rank, rope = ARCH_DIMS[arch]
    g = synth.gen(seed)
    wq, wqs = ref.weight_quant(synth.weight_fp32(q_rank, dim, g))
    wkv, wkvs = ref.weight_quant(synth.weight_fp32(kv_rank + rope, dim, g))
    x = (torch.randn(batch, seq, dim, generator=g) * 2).to(torch.bfloat16)
    x[0, 0, :128] = 0.0  # an all-zero quantisation group
    gamma = 1 + 0.1 * torch.randn(dim, generator=g)
    w = pack_wqkva(wq.to(cuda), wqs.to(cuda), wkv.to(cuda), wkvs.to(cuda), kv_rank)
    cur = torch.tensor([pos], dtype=torch.int32, device=cuda)
    xd, gd = x.to(cuda), gamma.to(cuda)

    def outs():
        return (torch.empty(batch, seq, q_rank, dtype=torch.bfloat16, device=cuda),
                torch.empty(batch, seq, kv_rank, dtype=torch.bfloat16, device=cuda),
                torch.full((batch, max_len, rope), SENTINEL, dtype=torch.bfloat16, device=cuda))
    # the two-launch composition
    y = torch.empty_like(xd)
    xq = torch.empty(batch, seq, dim, dtype=torch.float8_e4m3fn, device=cuda)
    xs = torch.empty(batch, seq, dim // 128, dtype=torch.float32, device=cuda)
    rmsnorm_quant(xd, gd, y, xq, xs, LOGS, model_arch=arch, scale_fmt=scale_fmt)
    two = outs()
    projx_wqkva(xq, xs, w, cur, *two, LOGS, model_arch=arch)
    # the module entry point (the same two launches, behind one call)
    one = outs()
    y1 = torch.empty_like(xd)
    rmsnorm_projx_wqkva(xd, gd, w, cur, *one, y1, LOGS, model_arch=arch, scale_fmt=scale_fmt)
    torch.cuda.synchronize()
    return x, gamma, (wq, wqs, wkv, wkvs, kv_rank), (y, xq, xs, two), (y1, one)


@pytest.mark.parametrize("batch,seq,arch,max_len,pos,scale_fmt", [
    (1, 4, "deepseek_v3_2", 128, 0, None),
    (4, 1, "deepseek_v3_2", 64, 17, "ue8m0"),
    (1, 3, "deepseek_v3_2", 32, 30, None),   # 3 tokens, one past the cache end
    (2, 8, "deepseek_v3_2", 40, 3, "div"),
    (1, 1, "glm_5", 32, 5, "div"),
    (3, 3, "glm_5", 16, 2, None),
])
def test_module_equals_rmsnorm_quant_then_projx(cuda, batch, seq, arch, max_len, pos, scale_fmt):
    x, gamma, wts, (y, xq, xs, two), (y1, one) = _case(cuda, batch, seq, arch, max_len, pos, scale_fmt,
                                                       900 + batch * 10 + seq)
    assert torch.equal(y1, y), "normalised rows differ from rmsnorm_quant's"
    for a, b, name in zip(one, two, ("q", "kv", "pe cache")):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"{name} differs from the two-launch path"
    # the oracle's golden chain, on the kernel's own quantised activations
    wq_, wkv_, wpe_ = ref.projx_wqkva(xq.cpu(), xs.cpu(), *wts)
    assert_gemm_close(one[0], wq_, "q")
    assert_gemm_close(one[1], wkv_, "kv")


def test_fused_is_close_to_the_fp32_golden(cuda):
    """Against rms_norm in fp32 and the dequantised weights (golden_forward, :450-471):
    the activation quantisation is the only extra error."""
    x, gamma, (wq, wqs, wkv, wkvs, kv_rank), _, (y1, one) = _case(cuda, 1, 4, "deepseek_v3_2", 8, 0, None, 77)
    xn = ref.rmsnorm(x.reshape(4, -1), gamma).float()
    q = xn @ ref.weight_dequant(wq, wqs).T
    rel = (one[0].cpu().float().reshape(4, -1) - q).norm() / q.norm()
    assert rel < 3e-2, rel



def test_rejects_bad_arguments(cuda):
    dim, q_rank, kv_rank, rope = ARCH_DIMS["deepseek_v3_2"]
    w = pack_wqkva(torch.zeros(q_rank, dim, dtype=torch.float8_e4m3fn, device=cuda),
                   torch.ones(q_rank // 128, dim // 128, device=cuda),
                   torch.zeros(kv_rank + rope, dim, dtype=torch.float8_e4m3fn, device=cuda),
                   torch.ones(5, dim // 128, device=cuda), kv_rank)
    cur = torch.zeros(1, dtype=torch.int32, device=cuda)
    q = torch.empty(1, 4, q_rank, dtype=torch.bfloat16, device=cuda)
    kv = torch.empty(1, 4, kv_rank, dtype=torch.bfloat16, device=cuda)
    pe = torch.empty(1, 32, rope, dtype=torch.bfloat16, device=cuda)
    with pytest.raises(ValueError, match="bfloat16"):
        rmsnorm_projx_wqkva(torch.zeros(1, 4, dim, device=cuda), torch.ones(dim, device=cuda), w, cur, q, kv, pe,
                            model_arch="deepseek_v3_2")
    with pytest.raises(ValueError, match="does not match"):
        rmsnorm_projx_wqkva(torch.zeros(1, 4, 6144, dtype=torch.bfloat16, device=cuda), torch.ones(6144, device=cuda),
                            w, cur, q, kv, pe, model_arch="deepseek_v3_2")
