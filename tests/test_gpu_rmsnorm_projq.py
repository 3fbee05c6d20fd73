"""GPU parity of the fused q RMSNorm + wq_b projection (RmsnormProjqWqb, BF16MMA) against
the CPU oracle restatement of its golden (ops/rmsnorm_projq_wqb.py:496-512)."""
import pytest
import torch

from oracle import reference as ref
from tests._tol import assert_gemm_close
from tilert_amd import kernel as K
from tilert_amd import synth
from tilert_amd.rmsnorm_projq_wqb import rmsnorm_projq_wqb_op

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("s,heads,rank,arch", [
    (4, 16, 1536, "deepseek_v3_2"),  # the TP=8 share of DeepSeek-V3.2: wq_b 3072 x 1536
    (1, 16, 1536, "deepseek_v3_2"),
    (2, 8, 2048, "glm_5"),           # GLM-5 head dims (192 + 64), q_lora_rank 2048
    (4, 3, 512, "deepseek_v3_2"),    # one K group, a head count that is not a multiple of 8
])
def test_rmsnorm_projq_wqb_vs_oracle(cuda, s, heads, rank, arch):
    g = synth.gen(60 + heads + rank)
    nope, rope = (128, 64) if arch == "deepseek_v3_2" else (192, 64)
    q = (torch.randn(1, s, rank, generator=g) * 3).to(torch.bfloat16)
    gamma = torch.rand(rank, generator=g) + 0.5
    wq, ws = ref.weight_quant(synth.weight_fp32(heads * (nope + rope), rank, g))
    packed = K.pack_weight(wq.to(cuda), ws.to(cuda))
    q_nope = torch.zeros(1, s, heads, nope, dtype=torch.bfloat16, device=cuda)
    q_pe = torch.zeros(1, s, heads, rope, dtype=torch.bfloat16, device=cuda)
    rmsnorm_projq_wqb_op(q.to(cuda), packed, None, gamma.to(cuda), q_nope, q_pe, None, "bf16mma", arch)
    eps = 1e-6 if arch == "deepseek_v3_2" else 1e-5
    want_nope, want_pe = ref.rmsnorm_projq_wqb(q[0], gamma, wq, ws, heads, nope, rope, eps)
    assert_gemm_close(q_nope[0], want_nope, "q_nope")
    assert_gemm_close(q_pe[0], want_pe, "q_pe")


def test_rmsnorm_projq_wqb_rejects_fp16mma(cuda):
    wq, ws = ref.weight_quant(synth.weight_fp32(192, 512, synth.gen(1)))
    packed = K.pack_weight(wq.to(cuda), ws.to(cuda))
    q = torch.zeros(1, 1, 512, dtype=torch.bfloat16, device=cuda)
    with pytest.raises(ValueError, match="BF16MMA"):
        rmsnorm_projq_wqb_op(q, packed, None, torch.ones(512, device=cuda), torch.zeros(1, 1, 1, 128, device=cuda),
                             torch.zeros(1, 1, 1, 64, device=cuda), None, "fp16mma", "deepseek_v3_2")
