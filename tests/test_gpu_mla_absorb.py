"""GPU parity of the absorbed MLA projections -- projq_wqb, projo_wkvb and
unproj_o_allreduce -- against the oracle's restated goldens at the device share of 16 heads
(DeepSeek-V3.2: nope 128, v 128, kv_lora 512, dim 7168; GLM-5: dim 6144), M = 1..4: the
bf16-weight restatement at the GEMM bar, the fp32-weight golden at rel-L2 1e-2."""
import pytest
import torch

from oracle import reference as ref
from tests._tol import assert_gemm_close
from tilert_amd import kernel as K
from tilert_amd import synth
from tilert_amd.projo_wkvb import convert_projo_wkvb, projo_wkvb
from tilert_amd.projq_wqb import convert_projq_wqb, projq_wqb
from tilert_amd.unproj_o_allreduce import convert_unproj_o, unproj_o_allreduce

pytestmark = pytest.mark.gpu

H, NOPE, V, KV = 16, 128, 128, 512


def _rel(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    return (torch.norm(a - b) / torch.norm(b)).item()


@pytest.fixture(scope="module")
def wkv_b(cuda):
    g = torch.Generator(device=cuda).manual_seed(31)
    q, s = K.weight_quant(torch.randn(H * (NOPE + V), KV, device=cuda, generator=g) * 0.02)
    return q, s


@pytest.mark.parametrize("M", [1, 2, 4])
def test_projq_wqb_vs_oracle(cuda, wkv_b, M):
    q, s = wkv_b
    x = synth.activations(M, H * NOPE, synth.gen(40 + M)).reshape(1, M, H, NOPE)
    out = torch.empty(1, M, H, KV, dtype=torch.bfloat16, device=cuda)
    projq_wqb(x.to(cuda), convert_projq_wqb(q, s, H), None, out, None, model_arch="deepseek_v3_2")
    qc, sc = q.cpu(), s.cpu()
    assert_gemm_close(out, ref.projq_wqb(x, qc, sc, H, NOPE, bf16_weights=True), f"projq_wqb M={M}")
    assert _rel(out, ref.projq_wqb(x, qc, sc, H, NOPE, bf16_weights=False)) <= 1e-2


@pytest.mark.parametrize("M", [1, 3, 4])
def test_projo_wkvb_vs_oracle(cuda, wkv_b, M):
    q, s = wkv_b
    o = synth.activations(M, H * KV, synth.gen(50 + M)).reshape(1, M, H, KV)
    out = torch.empty(1, M, H, V, dtype=torch.bfloat16, device=cuda)
    projo_wkvb(o.to(cuda), convert_projo_wkvb(q, s, H), None, out, None, "deepseek_v3_2")
    qc, sc = q.cpu(), s.cpu()
    assert_gemm_close(out, ref.projo_wkvb(o, qc, sc, H, V, bf16_weights=True), f"projo_wkvb M={M}")
    assert _rel(out, ref.projo_wkvb(o, qc, sc, H, V, bf16_weights=False)) <= 1e-2


@pytest.mark.parametrize("D,M,residual", [(7168, 4, True), (7168, 1, False), (6144, 2, True)])
def test_unproj_o_allreduce_vs_oracle(cuda, D, M, residual):
    g = torch.Generator(device=cuda).manual_seed(32 + D)
    wo, wos = K.weight_quant(torch.randn(D, H * V, device=cuda, generator=g) * 0.02)
    x = synth.activations(M, H * V, synth.gen(60 + M)).reshape(1, M, H, V)
    xin = synth.activations(M, D, synth.gen(70 + M)).reshape(1, M, D) if residual else None
    out = torch.empty(1, M, D, dtype=torch.bfloat16, device=cuda)
    unproj_o_allreduce(x.to(cuda), convert_unproj_o(wo, wos), None, xin.to(cuda) if residual else None, 0, out, None,
                       "deepseek_v3_2")
    woc, wosc = wo.cpu(), wos.cpu()
    assert_gemm_close(out, ref.unproj_o_allreduce(x, woc, wosc, True, xin), f"unproj_o D={D} M={M}")
    assert _rel(out, ref.unproj_o_allreduce(x, woc, wosc, False, xin)) <= 1e-2


def test_head_weights_conversion_matches_manual_slices(cuda, wkv_b):
    """The converters' head blocks: projq's is the transposed nope block, projo's the value
    block, with their 128x128 scales."""
    q, s = wkv_b
    wq = convert_projq_wqb(q, s, H)
    wo = convert_projo_wkvb(q, s, H)
    assert (wq.N, wq.K, wo.N, wo.K) == (KV, NOPE, V, KV)
    sc = s.cpu().reshape(H, 2, KV // 128)
    assert torch.equal(wq.s.cpu(), sc[:, :1].transpose(1, 2))
    assert torch.equal(wo.s.cpu(), sc[:, 1:])
