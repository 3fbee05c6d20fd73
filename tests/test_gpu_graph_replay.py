"""HIP-graph replays of the paths that keep state in a workspace between calls (split-K
counters and partials of the GEMMs, top-k's arrival counters and candidate regions) and of
the MoE layer: each op is captured once and replayed several times, with eager calls of
the same op and output poisoning in between, and every replay must equal the eager result
bit for bit.  A counter a kernel failed to re-arm, or a partial read from the wrong call,
shows up as a changed replay.  The ops' own parity with the oracle is covered by their
test files; here the eager call is the reference.
"""
import pytest
import torch

from oracle import reference as ref
from tilert_amd import kernel as K
from tilert_amd import moe, synth
from tilert_amd import sparse_index as si
from tilert_amd.topk import topk_rows

pytestmark = pytest.mark.gpu


def _check_replays(run, replays=4):
    """run() enqueues the op on the current stream and returns its output tensors."""
    want = [t.clone() for t in run()]
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up on a side stream, as torch's capture does
        run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = run()
    for rep in range(replays):
        for o in outs:
            o.fill_(-7)
        eager = [t.clone() for t in run()]  # the same op eagerly between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, w, e in zip(outs, want, eager):
            assert torch.equal(e, w), f"eager call {rep} differs"
            assert torch.equal(o, w), f"replay {rep} differs from the eager result"


@pytest.mark.parametrize("M,N,Kd,packed", [
    (32, 576, 7168, False),    # GEMV, K split in 4 slices (partials + counters)
    (64, 2048, 7168, True),    # wide MFMA GEMM, 16 slices x 16 K ranges
    (256, 7168, 2048, True),   # wide MFMA GEMM, 2 token groups x K ranges
    (16, 7168, 1024, True),    # GEMV on the activation image
])
def test_fp8_gemm_graph_replays(cuda, M, N, Kd, packed):
    g = synth.gen(4000 + M + N)
    xq, xs = ref.act_quant(synth.activations(M, Kd, g))
    wq, ws = ref.weight_quant(synth.weight_fp32(N, Kd, g))
    xq, xs, wq, ws = xq.to(cuda), xs.to(cuda), wq.to(cuda), ws.to(cuda)
    b = K.pack_weight(wq, ws) if packed else None
    out = torch.empty(M, N, dtype=torch.bfloat16, device=cuda)

    def run():
        if packed:
            K.fp8_gemm(xq, xs, b, out=out)
        else:
            K.fp8_gemm(xq, xs, wq, ws, out=out)
        return [out]

    _check_replays(run)


def test_indexer_topk_graph_replays(cuda):
    M, H, L, k = 4, 64, 32768, 2048
    g = torch.Generator(device=cuda).manual_seed(7)
    q = torch.randn(M, H, 128, device=cuda, generator=g).to(torch.float8_e4m3fn)
    qs = torch.rand(M, device=cuda, generator=g) + 0.5
    kv = torch.randn(L, 128, device=cuda, generator=g).to(torch.float8_e4m3fn)
    ks = torch.rand(L, device=cuda, generator=g) + 0.5
    w = (torch.randn(M, H, device=cuda, generator=g) / 8).to(torch.bfloat16)
    logits = torch.empty(M, L, device=cuda)
    idx = torch.empty(M, k, dtype=torch.int32, device=cuda)

    def run():
        si.sparse_index_topk_fp8(q, qs, kv, ks, w, logits, idx, L - M)
        return [logits, idx]

    _check_replays(run)


def test_topk_rows_graph_replays(cuda):
    rows, ld, k = 4, 131072, 2048
    logits = torch.randn(rows, ld, device=cuda, generator=torch.Generator(device=cuda).manual_seed(3))
    idx = torch.empty(rows, k, dtype=torch.int32, device=cuda)

    def run():
        topk_rows(logits, ld - rows, k, out=idx)
        return [idx]

    _check_replays(run)


def test_moe_graph_replays(cuda):
    M, E, D, I, topk, n_exp = 4, 8, 1024, 512, 8, 32
    g = synth.gen(11)
    W = {}
    for name, (n, kk) in (("gate", (I, D)), ("up", (I, D)), ("down", (D, I))):
        q, s = zip(*[ref.weight_quant(synth.weight_fp32(n, kk, g)) for _ in range(E)])
        W[name] = (torch.stack(q).to(cuda), torch.stack(s).to(cuda))
    ex = moe.LocalExperts(W["gate"][0], W["gate"][1], W["up"][0], W["up"][1], W["down"][0], W["down"][1],
                          expert_begin=0)
    x = synth.activations(M, D, g).to(cuda)
    idx, w = synth.routing(M, n_exp, topk, g)
    idx, w = idx.to(cuda), w.to(cuda)
    h = torch.empty(E, M, I, dtype=torch.bfloat16, device=cuda)
    y = torch.empty(M, D, dtype=torch.bfloat16, device=cuda)

    def run():
        moe.moe_forward(x, ex, idx, w, h, y)
        return [y]

    _check_replays(run)
