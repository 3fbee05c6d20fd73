"""GPU parity of flash_sparse_mla (split-K sparse MLA decode attention) against the CPU
oracle restatement of FlashSparseMLACombine.golden_forward (ops/flash_sparse_mla.py:152-196)."""
import math

import pytest
import torch

from oracle import reference as ref
from tests._tol import assert_gemm_close
from tilert_amd import synth
from tilert_amd.flash_sparse_mla import flash_sparse_mla

pytestmark = pytest.mark.gpu


def _inputs(s, h, T, seed):
    g = synth.gen(seed)
    q = (torch.randn(1, s, h, 512, generator=g) * 0.5).to(torch.bfloat16)
    qp = (torch.randn(1, s, h, 64, generator=g) * 0.5).to(torch.bfloat16)
    kv = torch.randn(1, T, 512, generator=g).to(torch.bfloat16)
    pe = torch.randn(1, T, 64, generator=g).to(torch.bfloat16)
    return g, q, qp, kv, pe


def _run(cuda, q, qp, kv, pe, idx, cur, arch="deepseek_v3_2"):
    s, h = q.shape[1], q.shape[2]
    out = torch.zeros(1, s, h, 512, dtype=torch.bfloat16, device=cuda)
    res = flash_sparse_mla(q.to(cuda), qp.to(cuda), kv.to(cuda), pe.to(cuda), idx.to(cuda),
                           torch.tensor([cur], dtype=torch.int32, device=cuda), out, None, model_arch=arch)
    return out.cpu(), [r.cpu() for r in res]


@pytest.mark.parametrize("s,h,T,k,arch", [
    (4, 16, 8192, 2048, "deepseek_v3_2"),  # the decode shape: 16 heads at TP=8, top-2048
    (1, 16, 4096, 2048, "deepseek_v3_2"),
    (2, 20, 300, 100, "glm_5"),            # two head tiles, a partial last split
    (3, 8, 64, 64, "glm_5"),               # one split, every position selected
    (4, 10, 50, 1, "deepseek_v3_2"),       # one position per token
])
def test_flash_sparse_mla_vs_oracle(cuda, s, h, T, k, arch):
    g, q, qp, kv, pe = _inputs(s, h, T, 1000 + T + k)
    cur = T - s  # token t at position cur + t; drawn positions past it are masked for s > 1
    # (drawn from the positions every token sees when one is drawn: a token whose whole
    # selection is masked has a NaN golden -- tested separately)
    pool = T if k > 1 else cur + 1
    idx = torch.stack([torch.randperm(pool, generator=g)[:k] for _ in range(s)]).to(torch.int32)[None]
    out, (lse, lse_acc, out_acc) = _run(cuda, q, qp, kv, pe, idx, cur, arch)
    want = ref.flash_sparse_mla(q[0], qp[0], kv[0], pe[0], idx[0], cur, ref.mla_softmax_scale(arch))
    assert_gemm_close(out[0], want, f"flash_sparse_mla s={s} h={h} k={k}")
    # lse: ln sum exp of the visible scaled scores (fp64 check)
    sc = ref.mla_softmax_scale(arch)
    for t in range(s):
        sel = [int(i) for i in idx[0, t] if s == 1 or int(i) <= cur + t]
        z = (torch.einsum("hc,tc->ht", q[0, t].double(), kv[0, sel].double())
             + torch.einsum("hr,tr->ht", qp[0, t].double(), pe[0, sel].double())) * sc
        assert torch.allclose(lse[0, t].double(), torch.logsumexp(z, -1), rtol=0, atol=2e-4)


def test_padding_and_out_of_range_indices_are_ignored(cuda):
    s, h, T, k = 2, 16, 500, 300
    g, q, qp, kv, pe = _inputs(s, h, T, 77)
    idx = torch.stack([torch.randperm(T, generator=g)[:k] for _ in range(s)]).to(torch.int32)
    idx[0, 200:] = -1          # top-k's padding
    idx[1, 10:20] = T + 5      # past the cache
    out, _ = _run(cuda, q, qp, kv, pe, idx[None], T - s)
    for t in range(s):
        keep = [int(i) for i in idx[t] if 0 <= int(i) < T and int(i) <= T - s + t]
        # a seqlen-1 oracle call on the kept positions (no triu mask)
        want = ref.flash_sparse_mla(q[0, t:t + 1], qp[0, t:t + 1], kv[0], pe[0], torch.tensor([keep]), T,
                                    ref.mla_softmax_scale("deepseek_v3_2"))
        assert_gemm_close(out[0, t], want[0], f"token {t}")


def test_token_with_nothing_visible_gets_zeros(cuda):
    s, h, T = 2, 16, 64
    _, q, qp, kv, pe = _inputs(s, h, T, 80)
    idx = torch.tensor([[[63, 62], [10, 63]]], dtype=torch.int32)  # token 0 at 61 sees neither
    out, (lse, _, _) = _run(cuda, q, qp, kv, pe, idx, T - 3)
    assert torch.all(out[0, 0] == 0) and torch.isneginf(lse[0, 0]).all()
    want = ref.flash_sparse_mla(q[0, 1:], qp[0, 1:], kv[0], pe[0], torch.tensor([[10]]), T,
                                ref.mla_softmax_scale("deepseek_v3_2"))
    assert torch.equal(out[0, 1], want[0])  # one visible position: exactly its kv row


def test_nan_in_unselected_rows_does_not_leak(cuda):
    s, h, T = 1, 16, 256
    g, q, qp, kv, pe = _inputs(s, h, T, 78)
    clean_kv, clean_pe = kv.clone(), pe.clone()
    kv[0, 0] = float("nan")  # row 0 is never selected; masked slots must not read it into a product
    pe[0, 0] = float("inf")  # (the golden scores every row, so it would return NaN here)
    idx = torch.full((1, 1, 100), -1, dtype=torch.int32)
    idx[0, 0, :40] = torch.randperm(T - 1, generator=g)[:40].to(torch.int32) + 1
    out, _ = _run(cuda, q, qp, kv, pe, idx, T - 1)
    want = ref.flash_sparse_mla(q[0], qp[0], clean_kv[0], clean_pe[0], idx[0, :, :40], T - 1,
                                ref.mla_softmax_scale("deepseek_v3_2"))
    assert torch.isfinite(out).all()
    assert_gemm_close(out[0], want, "nan row")


def test_reference_argument_checks(cuda):
    _, q, qp, kv, pe = _inputs(5, 16, 64, 79)
    out = torch.zeros(1, 5, 16, 512, dtype=torch.bfloat16, device=cuda)
    idx = torch.zeros(1, 5, 8, dtype=torch.int32, device=cuda)
    pos = torch.zeros(1, dtype=torch.int32, device=cuda)
    args = (q.to(cuda), qp.to(cuda), kv.to(cuda), pe.to(cuda), idx, pos, out, None)
    with pytest.raises(ValueError, match="seqlen<=4"):
        flash_sparse_mla(*args, model_arch="deepseek_v3_2")
    with pytest.raises(ValueError, match="split_size=64"):
        flash_sparse_mla(*args, split_size=32, model_arch="deepseek_v3_2")
