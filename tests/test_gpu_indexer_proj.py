"""GPU parity of the indexer's input projections against the oracle:

* ``projx_wqaki``: x_q . [wq_a; wk]^T routed to q and ki -- each output equals the FP8 GEMM
  oracle on its own weight at the GEMM bar;
* ``projx_wis``: the bf16 weights_proj GEMV at the GEMM bar;
* ``rmsnorm_projx_wqakis`` (decoupled): q and ki at the GEMM bar against the oracle chain
  that the module runs (``rmsnorm_quant``: bf16 norm, act_quant; then the FP8 GEMM),
  idx_scores at the GEMM bar against ``projx_wis`` of the oracle's bf16 norm; and the three
  outputs against the module's fp32 golden (rms_norm, then fp32 matmuls) at rel-L2 3e-2 --
  the kernels quantise the normalised rows to fp8 for wq_a / wk, which the golden does not;
* ``rmsnorm_projq_wqi_op``: the golden (bf16 normalised q, bf16 weights) at the GEMM bar,
  64 heads x 128 at q_lora 1536 (DeepSeek-V3.2) and 2048 (GLM-5), s in 1, 2, 4, 8."""
import pytest
import torch

from oracle import reference as ref
from tests._tol import assert_gemm_close
from tilert_amd import kernel as K
from tilert_amd import synth
from tilert_amd.projx_wqaki import pack_wqaki, projx_wis, projx_wqaki, rmsnorm_projx_wqakis
from tilert_amd.rmsnorm_projq_wqi import rmsnorm_projq_wqi_op

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    return (torch.norm(a - b) / torch.norm(b)).item()


def _weights(dim, q_rank, seed):
    g = synth.gen(seed)
    wq, wqs = ref.weight_quant(synth.weight_fp32(q_rank, dim, g))
    wk, wks = ref.weight_quant(synth.weight_fp32(128, dim, g))
    wis = (torch.randn(64, dim, generator=g) * 0.02).to(torch.bfloat16)
    return wq, wqs, wk, wks, wis


@pytest.mark.parametrize("dim,q_rank,M", [(7168, 1536, 4), (7168, 1536, 1), (6144, 2048, 2),
                                           (7168, 1536, 48)])  # M > 32: the wide MFMA GEMM, two output segments
def test_projx_wqaki_and_wis_vs_oracle(cuda, dim, q_rank, M):
    wq, wqs, wk, wks, wis = _weights(dim, q_rank, dim + M)
    x = synth.activations(M, dim, synth.gen(M))
    xq, xs = ref.act_quant(x)
    packed = pack_wqaki(wq.to(cuda), wqs.to(cuda), wk.to(cuda), wks.to(cuda))
    q = torch.empty(1, M, q_rank, dtype=torch.bfloat16, device=cuda)
    ki = torch.empty(1, M, 128, dtype=torch.bfloat16, device=cuda)
    projx_wqaki(xq.reshape(1, M, dim).to(cuda), xs.reshape(1, M, -1).to(cuda), packed, q, ki, None,
                model_arch="deepseek_v3_2")
    assert_gemm_close(q[0], ref.fp8_gemm(xq, xs, wq, wqs), "q")
    assert_gemm_close(ki[0], ref.fp8_gemm(xq, xs, wk, wks), "ki")
    if M > 16:  # projx_wis is a decode GEMV (M <= 16)
        return
    sc = torch.empty(1, M, 64, dtype=torch.bfloat16, device=cuda)
    projx_wis(x.reshape(1, M, dim).to(cuda), wis.to(cuda), sc)
    assert_gemm_close(sc[0], ref.projx_wis(x, wis), "idx_scores")


@pytest.mark.parametrize("arch,dim,q_rank,M", [("deepseek_v3_2", 7168, 1536, 4), ("glm_5", 6144, 2048, 4),
                                                 ("deepseek_v3_2", 7168, 1536, 1), ("deepseek_v3_2", 7168, 1536, 16)])
def test_rmsnorm_projx_wqakis_vs_golden(cuda, arch, dim, q_rank, M):
    wq, wqs, wk, wks, wis = _weights(dim, q_rank, 5 + dim)
    g = synth.gen(77)
    x = synth.activations(M, dim, g)
    gamma = torch.rand(dim, generator=g) + 0.5
    packed = pack_wqaki(wq.to(cuda), wqs.to(cuda), wk.to(cuda), wks.to(cuda))
    q = torch.empty(1, M, q_rank, dtype=torch.bfloat16, device=cuda)
    ki = torch.empty(1, M, 128, dtype=torch.bfloat16, device=cuda)
    sc = torch.empty(1, M, 64, dtype=torch.bfloat16, device=cuda)
    rmsnorm_projx_wqakis(x.reshape(1, M, dim).to(cuda), gamma.to(cuda), packed, wis.to(cuda), q, ki, sc,
                         model_arch=arch)
    eps = 1e-6 if arch == "deepseek_v3_2" else 1e-5
    # the chain the module runs, restated: bf16 norm + act_quant, then the FP8 GEMM / bf16 GEMV
    y, xq, xs = ref.rmsnorm_quant(x, gamma, eps)
    assert_gemm_close(q[0], ref.fp8_gemm(xq, xs, wq, wqs), f"q {arch}")
    assert_gemm_close(ki[0], ref.fp8_gemm(xq, xs, wk, wks), f"ki {arch}")
    assert_gemm_close(sc[0], ref.projx_wis(y, wis), f"idx_scores {arch}")
    # the module's fp32 golden
    rq, rki, rsc = ref.rmsnorm_projx_wqakis(x, gamma, wq, wqs, wk, wks, wis, eps)
    assert _rel(q[0], rq) <= 3e-2 and _rel(ki[0], rki) <= 3e-2
    assert _rel(sc[0], rsc) <= 1e-2  # bf16 rows, bf16 weights: no fp8 step


@pytest.mark.parametrize("arch,q_rank,s", [("deepseek_v3_2", 1536, 4), ("deepseek_v3_2", 1536, 8),
                                           ("deepseek_v3_2", 1536, 1), ("glm_5", 2048, 2)])
def test_rmsnorm_projq_wqi_vs_oracle(cuda, arch, q_rank, s):
    g = synth.gen(90 + s + q_rank)
    q = (torch.randn(1, s, q_rank, generator=g) * 3).to(torch.bfloat16)
    gamma = torch.rand(q_rank, generator=g) + 0.5
    wq, ws = ref.weight_quant(synth.weight_fp32(64 * 128, q_rank, g))
    packed = K.pack_weight(wq.to(cuda), ws.to(cuda))
    iq = torch.zeros(1, s, 64, 128, dtype=torch.bfloat16, device=cuda)
    rmsnorm_projq_wqi_op(q.to(cuda), packed, None, gamma.to(cuda), iq, None, "fp16mma", arch)
    eps = 1e-6 if arch == "deepseek_v3_2" else 1e-5
    assert_gemm_close(iq[0], ref.rmsnorm_projq_wqi(q[0], gamma, wq, ws, 64, 128, eps), f"iq {arch} s={s}")


@pytest.mark.parametrize("M,N,K", [(4, 64, 384),     # one K slice: no workspace
                                   (3, 32, 1152),    # a last slice with one live block of eight
                                   (16, 64, 7168),   # the largest M at the production width
                                   (1, 160, 2048)])
def test_bf16_gemv_slices_vs_oracle(cuda, M, N, K):
    """projx_wis's bf16 GEMV over K slices (fixed-order sum of the slices' partials),
    twice in a row on one stream (the arrival counters are left zero for the next call)."""
    g = synth.gen(M * 7 + N + K)
    x = synth.activations(M, K, g)
    w = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16)
    want = ref.projx_wis(x, w)
    for _ in range(2):
        y = torch.empty(1, M, N, dtype=torch.bfloat16, device=cuda)
        projx_wis(x.reshape(1, M, K).to(cuda), w.to(cuda), y)
        assert_gemm_close(y[0], want, f"bf16_gemv M={M} N={N} K={K}")
