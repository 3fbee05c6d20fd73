"""GPU parity of the reference-layout MoE and dense-MLP operators against the oracle's
restated goldens:

* routing (``_ref_expert_select_ds`` / ``_glm5``): the indices exactly (order included) and
  the probabilities to fp32 rounding;
* ``expert_select_up_gate_silu`` (shared expert at position 0, then the selected experts)
  and ``expert_down_allreduce`` (+ residual) at DeepSeek-V3.2 (D 7168, 256 routed experts,
  8 groups) and GLM-5 (D 6144, no groups) device shares, I = 256, M = 1, 2, 4;
* ``rmsnorm_up_gate_silu`` / ``down_allreduce`` at the dense MLP's device share (9 chunks of
  256): the bf16-operand restatement at the GEMM bar, the fp32 golden at rel-L2 1e-2.

Weights are drawn and block-quantised on the GPU (``weight_quant`` is bit-exact against the
oracle's, tests/test_gpu_linear.py); the oracle reads the same fp8 codes back.
"""
import pytest
import torch

from oracle import reference as ref
from tests._tol import assert_gemm_close
from tilert_amd import kernel as K
from tilert_amd import synth
from tilert_amd.down_allreduce import down_allreduce
from tilert_amd.expert_down_allreduce import DownExperts, expert_down_allreduce
from tilert_amd.expert_sel_up_gate_silu import ROUTING, UpGateExperts, expert_select, expert_select_up_gate_silu
from tilert_amd.rmsnorm_up_gate_silu import EPS, rmsnorm_up_gate_silu

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    return (torch.norm(a - b) / torch.norm(b)).item()


def _quant_stack(E, n, k, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    qs, ss = [], []
    for _ in range(E):
        q, s = K.weight_quant(torch.randn(n, k, device=dev, generator=g) * 0.02)
        qs.append(q)
        ss.append(s)
    return torch.stack(qs), torch.stack(ss)


class _Experts:
    """Shared + routed experts of one device share, on the GPU and packed."""

    def __init__(self, n_local, D, I, seed, dev):
        self.g = _quant_stack(n_local, I, D, seed, dev)
        self.u = _quant_stack(n_local, I, D, seed + 1, dev)
        self.d = _quant_stack(n_local, D, I, seed + 2, dev)
        self.up = UpGateExperts(*self.g, *self.u)
        self.down = DownExperts(*self.d)
        self.D, self.I = D, I

    def cpu(self, which, e):
        q, s = getattr(self, which)
        return q[e].cpu(), s[e].cpu()


_CACHE = {}


def _experts(n_local, D, I, seed, dev):
    key = (n_local, D, I, seed)
    if key not in _CACHE:
        _CACHE.clear()
        _CACHE[key] = _Experts(n_local, D, I, seed, dev)
    return _CACHE[key]


def _sub(ex, which, ids):
    """The oracle's per-expert weights for local experts ``ids`` (codes, scales), as dicts
    indexed by local expert id."""
    q, sc = {}, {}
    for e in ids:
        q[e], sc[e] = ex.cpu(which, e)
    return q, sc


@pytest.mark.parametrize("arch,M", [("deepseek_v3_2", 4), ("deepseek_v3_2", 33), ("glm_5", 4), ("glm_5", 1)])
def test_routing_vs_oracle(cuda, arch, M):
    n_groups, topk_groups, topk, scale = ROUTING[arch]
    g = synth.gen(500 + M)
    logits = torch.randn(M, 256, generator=g) * 2
    bias = torch.randn(256, generator=g) * 0.1
    probs = torch.empty(M, topk, device=cuda)
    idx = torch.empty(M, topk, dtype=torch.int32, device=cuda)
    expert_select(logits.to(cuda), bias.to(cuda), probs, idx, model_arch=arch)
    w, i = ref.expert_select(logits, bias, topk, n_groups, topk_groups, scale)
    assert torch.equal(idx.cpu().long(), i), "routing indices differ"
    assert torch.allclose(probs.cpu(), w, rtol=2e-6, atol=0)


def test_routing_without_bias_and_ties(cuda):
    """No bias: groups scored by their max; exact ties are taken lowest id first."""
    logits = torch.zeros(2, 256)
    logits[0, 40:48] = 3.0  # eight tied winners in one group
    logits[1] = torch.randn(256, generator=synth.gen(9))
    probs = torch.empty(2, 8, device=cuda)
    idx = torch.empty(2, 8, dtype=torch.int32, device=cuda)
    expert_select(logits.to(cuda), None, probs, idx, model_arch="deepseek_v3_2")
    assert idx[0].cpu().tolist() == list(range(40, 48))
    w, i = ref.expert_select(logits[1:], None, 8, 8, 4, 2.5)
    assert torch.equal(idx[1:].cpu().long(), i)
    assert torch.allclose(probs[1:].cpu(), w, rtol=2e-6)


@pytest.mark.parametrize("arch,D,M", [("deepseek_v3_2", 7168, 4), ("deepseek_v3_2", 7168, 1),
                                      ("glm_5", 6144, 2), ("deepseek_v3_2", 1024, 3),
                                      ("deepseek_v3_2", 1024, 6)])  # M > 4: every wave routes, x copied after
def test_expert_select_up_gate_silu_and_down_vs_oracle(cuda, arch, D, M):
    I, n_routed = 256, 256
    n_groups, topk_groups, topk, scale = ROUTING[arch]
    ex = _experts(1 + n_routed, D, I, 7 + D, cuda)
    g = synth.gen(600 + M + D)
    x = synth.activations(M, D, g)
    logits = torch.randn(M, n_routed, generator=g)
    bias = torch.randn(n_routed, generator=g) * 0.1
    xin = synth.activations(M, D, g)
    h = torch.empty(1, M, 1 + topk, I, dtype=torch.bfloat16, device=cuda)
    probs = torch.empty(1, M, topk, device=cuda)
    idx = torch.empty(1, M, topk, dtype=torch.int32, device=cuda)
    print(f"expert_select_up_gate_silu {arch} D={D} M={M}", flush=True)
    expert_select_up_gate_silu(x.reshape(1, M, D).to(cuda), logits.reshape(1, M, -1).to(cuda), bias.to(cuda),
                               ex.up, h, probs, idx, None, model_arch=arch)
    y = torch.empty(1, M, D, dtype=torch.bfloat16, device=cuda)
    y0 = torch.empty(1, M, D, dtype=torch.bfloat16, device=cuda)
    expert_down_allreduce(h, ex.down, None, idx, probs, xin.reshape(1, M, D).to(cuda), 0, y)
    expert_down_allreduce(h, ex.down, None, idx, probs, None, 0, y0)
    torch.cuda.synchronize()
    rw, ri = ref.expert_select(logits, bias, topk, n_groups, topk_groups, scale)
    assert torch.equal(idx[0].cpu().long(), ri)
    assert torch.allclose(probs[0].cpu(), rw, rtol=2e-6)
    used = sorted({0} | {1 + int(e) for e in ri.flatten()})
    gq, gs = _sub(ex, "g", used)
    uq, us = _sub(ex, "u", used)
    dq, ds = _sub(ex, "d", used)
    rh = ref.expert_select_up_gate_silu(x, ri, gq, gs, uq, us)
    assert_gemm_close(h[0], rh, f"hidden_out {arch} M={M}")
    # the down op on the kernel's own hidden_out isolates it from gate/up differences
    hk = h[0].cpu()
    assert_gemm_close(y0[0], ref.expert_down_allreduce(hk, ri, probs[0].cpu(), dq, ds), f"down {arch} M={M}")
    assert_gemm_close(y[0], ref.expert_down_allreduce(hk, ri, probs[0].cpu(), dq, ds, x_in=xin), "down + residual")
    # the whole chain against the oracle chain
    ry = ref.expert_down_allreduce(rh, ri, rw, dq, ds)
    assert _rel(y0[0], ry) <= 5e-3


def test_down_skips_out_of_range_ids(cuda):
    """Routed ids outside [0, n_routed) contribute nothing (no out-of-bounds weight read)."""
    D, I, M = 1024, 256, 2
    ex = _experts(257, D, I, 7 + D, cuda)
    h = (torch.randn(1, M, 9, I, generator=synth.gen(3)) * 0.1).to(torch.bfloat16)
    idx = torch.tensor([[3, 9, 300, -1, 5, 6, 7, 8], [1, 2, 3, 4, 5, 6, 7, 1000]], dtype=torch.int32)
    probs = torch.full((M, 8), 0.25)
    y = torch.empty(1, M, D, dtype=torch.bfloat16, device=cuda)
    expert_down_allreduce(h.to(cuda), ex.down, None, idx.reshape(1, M, 8).to(cuda), probs.reshape(1, M, 8).to(cuda),
                          None, 0, y)
    keep = idx.clone()
    hh = h[0].clone()
    for t in range(M):  # the oracle with the invalid positions' rows zeroed
        for j in range(8):
            if not 0 <= int(idx[t, j]) < 256:
                keep[t, j] = 0
                hh[t, 1 + j] = 0
    used = sorted({0} | {1 + int(e) for e in keep.flatten()})
    dq, ds = _sub(ex, "d", used)
    assert_gemm_close(y[0], ref.expert_down_allreduce(hh, keep, probs, dq, ds), "down with skipped ids")


@pytest.mark.parametrize("arch,D,M", [("deepseek_v3_2", 7168, 4), ("deepseek_v3_2", 7168, 1), ("glm_5", 6144, 3),
                                     ("deepseek_v3_2", 2048, 16)])
def test_dense_mlp_vs_oracle(cuda, arch, D, M):
    """M = 16 is the largest accepted token count (one 16-row MFMA tile; 4 chunks keep the
    64-pair limit): every one of its rows must be written."""
    C, I = min(9, 64 // M), 256
    gq, gs = _quant_stack(C, I, D, 70, cuda)
    uq, us = _quant_stack(C, I, D, 71, cuda)
    dq, ds = _quant_stack(C, D, I, 72, cuda)
    g = synth.gen(700 + M)
    x = synth.activations(M, D, g)
    gamma = torch.rand(D, generator=g) + 0.5
    xin = synth.activations(M, D, g)
    h = torch.empty(1, M, C, I, dtype=torch.bfloat16, device=cuda)
    rmsnorm_up_gate_silu(x.reshape(1, M, D).to(cuda), gamma.to(cuda), UpGateExperts(gq, gs, uq, us), h, None, arch)
    y = torch.empty(1, M, D, dtype=torch.bfloat16, device=cuda)
    down_allreduce(h, DownExperts(dq, ds), None, xin.reshape(1, M, D).to(cuda), 0, y, None, arch)
    torch.cuda.synchronize()
    c = [t.cpu() for t in (gq, gs, uq, us, dq, ds)]
    want16 = ref.rmsnorm_up_gate_silu(x, gamma, EPS[arch], *c[:4], bf16_operands=True)
    want32 = ref.rmsnorm_up_gate_silu(x, gamma, EPS[arch], *c[:4], bf16_operands=False)
    assert_gemm_close(h[0], want16, f"rmsnorm_up_gate_silu {arch} M={M}")
    assert _rel(h[0], want32) <= 1e-2
    hk = h[0].cpu()
    assert_gemm_close(y[0], ref.down_allreduce(hk, c[4], c[5], bf16_weights=True, x_in=xin), "down_allreduce")
    assert _rel(y[0], ref.down_allreduce(hk, c[4], c[5], bf16_weights=False, x_in=xin)) <= 1e-2


def test_reference_argument_checks(cuda):
    ex = _experts(257, 1024, 256, 7 + 1024, cuda)
    x = torch.zeros(1, 2, 1024, dtype=torch.bfloat16, device=cuda)
    sc = torch.zeros(1, 2, 256, device=cuda)
    h = torch.empty(1, 2, 9, 256, dtype=torch.bfloat16, device=cuda)
    p = torch.empty(1, 2, 8, device=cuda)
    i = torch.empty(1, 2, 8, dtype=torch.int32, device=cuda)
    with pytest.raises(ValueError):
        expert_select_up_gate_silu(x, sc, None, ex.up, h, p, i, None, model_arch="llama")
    with pytest.raises(ValueError):
        expert_select_up_gate_silu(x, sc[..., :128], None, ex.up, h, p, i, None, model_arch="deepseek_v3_2")
    with pytest.raises(ValueError):
        expert_select_up_gate_silu(x, sc, None, ex.up, h.cpu(), p, i, None, model_arch="deepseek_v3_2")
