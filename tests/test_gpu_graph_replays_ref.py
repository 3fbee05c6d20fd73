"""HIP-graph replays of the reference-layout MoE (routing fused into the gate/up launch,
then the down op with the residual) and of the dense-MLP share: captured once, replayed
with eager calls and output poisoning in between; every replay must equal the eager result
bit for bit, and the fused routing's outputs must equal the standalone routing op's.
"""
import pytest
import torch

from tilert_amd import kernel as K
from tilert_amd import synth
from tilert_amd.down_allreduce import down_allreduce
from tilert_amd.expert_down_allreduce import DownExperts, expert_down_allreduce
from tilert_amd.expert_sel_up_gate_silu import ROUTING, UpGateExperts, expert_select, expert_select_up_gate_silu
from tilert_amd.rmsnorm_up_gate_silu import rmsnorm_up_gate_silu
from tests.test_gpu_graph_replay import _check_replays

pytestmark = pytest.mark.gpu


def _stack(E, n, k, g, dev):
    qs, ss = zip(*[K.weight_quant((torch.randn(n, k, generator=g) * 0.02).to(dev)) for _ in range(E)])
    return torch.stack(qs), torch.stack(ss)


@pytest.mark.parametrize("arch,D", [("deepseek_v3_2", 2048), ("glm_5", 1024)])
def test_reference_moe_graph_replays(cuda, arch, D):
    M, I, n_routed = 4, 256, 256
    topk = ROUTING[arch][2]
    g = torch.Generator().manual_seed(77)
    up = UpGateExperts(*_stack(1 + n_routed, I, D, g, cuda), *_stack(1 + n_routed, I, D, g, cuda))
    dn = DownExperts(*_stack(1 + n_routed, D, I, g, cuda))
    x = synth.activations(M, D, g).reshape(1, M, D).to(cuda)
    xin = synth.activations(M, D, g).reshape(1, M, D).to(cuda)
    scores = torch.randn(1, M, n_routed, generator=g).to(cuda)
    bias = (torch.randn(n_routed, generator=g) * 0.1).to(cuda)
    h = torch.empty(1, M, 1 + topk, I, dtype=torch.bfloat16, device=cuda)
    probs = torch.empty(1, M, topk, device=cuda)
    idx = torch.empty(1, M, topk, dtype=torch.int32, device=cuda)
    y = torch.empty(1, M, D, dtype=torch.bfloat16, device=cuda)
    print(f"reference MoE graph replays {arch} D={D}", flush=True)

    def run():
        expert_select_up_gate_silu(x, scores, bias, up, h, probs, idx, None, model_arch=arch)
        expert_down_allreduce(h, dn, None, idx, probs, xin, 0, y)
        return [h, probs, idx, y]

    _check_replays(run)
    # the fused routing against the standalone routing op
    p2 = torch.empty_like(probs)
    i2 = torch.empty_like(idx)
    expert_select(scores, bias, p2, i2, model_arch=arch)
    torch.cuda.synchronize()
    assert torch.equal(i2, idx) and torch.equal(p2, probs), "fused routing differs from the routing op"


def test_dense_mlp_graph_replays(cuda):
    M, D, I = 4, 2048, 256
    g = torch.Generator().manual_seed(78)
    up = UpGateExperts(*_stack(9, I, D, g, cuda), *_stack(9, I, D, g, cuda))
    dn = DownExperts(*_stack(9, D, I, g, cuda))
    x = synth.activations(M, D, g).reshape(1, M, D).to(cuda)
    xin = synth.activations(M, D, g).reshape(1, M, D).to(cuda)
    gam = (torch.rand(D, generator=g) + 0.5).to(cuda)
    h = torch.empty(1, M, 9, I, dtype=torch.bfloat16, device=cuda)
    y = torch.empty(1, M, D, dtype=torch.bfloat16, device=cuda)
    print("dense MLP graph replays", flush=True)

    def run():
        rmsnorm_up_gate_silu(x, gam, up, h, None, "deepseek_v3_2")
        down_allreduce(h, dn, None, xin, 0, y, None, "deepseek_v3_2")
        return [h, y]

    _check_replays(run)
