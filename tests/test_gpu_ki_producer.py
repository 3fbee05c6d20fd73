"""GPU parity of the indexer key producer (LayerNorm -> RoPE -> Hadamard,
ops/layernorm_rope_rotate.py:206-220) against the CPU oracle, and of its fused KI-page
variant against the bf16 result quantised by ki_cache_write."""
import pytest
import torch

from oracle import reference as ref
from tilert_amd import synth
from tilert_amd.layernorm_rope_rotate import layernorm_rope_rotate, layernorm_rope_rotate_ki
from tilert_amd.sparse_index import KI_PAGE_BYTES, ki_cache_write

pytestmark = pytest.mark.gpu


def _inputs(seq, seed):
    g = synth.gen(seed)
    x = (torch.randn(1, seq, 128, generator=g) * 2 + 0.3).to(torch.bfloat16)
    w = torch.rand(128, generator=g) * 0.2 + 0.9
    b = torch.randn(128, generator=g) * 0.1
    theta = torch.rand(seq, 32, generator=g, dtype=torch.float64) * 6.28
    fr = torch.stack([theta.cos(), theta.sin()], dim=-1).reshape(seq, 1, 64).float()
    return x, w, b, fr


def _ulp(t):
    e = torch.floor(torch.log2(t.abs().clamp_min(2.0 ** -126)))
    return torch.pow(2.0, e - 7)


@pytest.mark.parametrize("seq,cur_pos,rows", [(1, 0, 1), (4, 3, 16), (37, 100, 200), (257, 0, 257)])
def test_layernorm_rope_rotate_vs_oracle(cuda, seq, cur_pos, rows):
    x, w, b, fr = _inputs(seq, 40 + seq)
    cache = torch.full((1, rows, 128), 7.0, dtype=torch.bfloat16, device=cuda)
    pos = torch.tensor([cur_pos], dtype=torch.int32, device=cuda)
    layernorm_rope_rotate(x.to(cuda), pos, cache, w.to(cuda), b.to(cuda), fr.to(cuda), None, "deepseek_v3_2")
    want = ref.layernorm_rope_rotate(x[0], w, b, fr.reshape(seq, 64))
    got = cache[0, cur_pos:cur_pos + seq].cpu()
    # fp32 statistics and butterfly order differ from torch's CPU kernels in the last bits:
    # every value within one bf16 step of the oracle, nearly all identical
    diff = (got.float() - want.float()).abs()
    assert torch.all(diff <= _ulp(torch.maximum(got.float().abs(), want.float().abs()))), diff.max()
    assert (got == want).float().mean().item() > 0.995
    untouched = torch.cat([cache[0, :cur_pos], cache[0, cur_pos + seq:]]).cpu()
    assert torch.all(untouched == 7.0)


def test_rows_outside_the_cache_are_dropped(cuda):
    x, w, b, fr = _inputs(6, 7)
    cache = torch.full((1, 8, 128), 7.0, dtype=torch.bfloat16, device=cuda)
    args = (w.to(cuda), b.to(cuda), fr.to(cuda), None, "deepseek_v3_2")
    layernorm_rope_rotate(x.to(cuda), torch.tensor([5], dtype=torch.int32, device=cuda), cache, *args)
    want = ref.layernorm_rope_rotate(x[0], w, b, fr.reshape(6, 64))
    got = cache[0].cpu()
    assert torch.all(got[:5] == 7.0)
    assert (got[5:] == want[:3]).float().mean() > 0.99  # keys 0..2 land on rows 5..7
    cache.fill_(7.0)
    layernorm_rope_rotate(x.to(cuda), torch.tensor([-4], dtype=torch.int32, device=cuda), cache, *args)
    got = cache[0].cpu()
    assert (got[:2] == want[4:]).float().mean() > 0.99  # keys 4, 5 land on rows 0, 1
    assert torch.all(got[2:] == 7.0)


@pytest.mark.parametrize("scale_fmt", [None, "ue8m0", "div"])
def test_ki_variant_is_ki_cache_write_of_the_bf16_keys(cuda, scale_fmt):
    seq, cur_pos, n_pages = 150, 30, 4  # keys straddle pages 0..2
    x, w, b, fr = _inputs(seq, 50)
    xd, wd, bd, fd = x.to(cuda), w.to(cuda), b.to(cuda), fr.to(cuda)
    pos = torch.tensor([cur_pos], dtype=torch.int32, device=cuda)
    pages = torch.zeros(n_pages, KI_PAGE_BYTES, dtype=torch.uint8, device=cuda)
    layernorm_rope_rotate_ki(xd, pos, pages, wd, bd, fd, scale_fmt=scale_fmt)
    cache = torch.zeros(1, seq, 128, dtype=torch.bfloat16, device=cuda)
    layernorm_rope_rotate(xd, torch.zeros(1, dtype=torch.int32, device=cuda), cache, wd, bd, fd, None, "deepseek_v3_2")
    want = torch.zeros_like(pages)
    ki_cache_write(cache[0], want, cur_pos, scale_fmt=scale_fmt)
    assert torch.equal(pages.cpu(), want.cpu())


def test_ki_variant_drops_positions_past_the_pages(cuda):
    x, w, b, fr = _inputs(10, 60)
    pages = torch.zeros(1, KI_PAGE_BYTES, dtype=torch.uint8, device=cuda)
    pos = torch.tensor([60], dtype=torch.int32, device=cuda)  # keys 0..3 fit, 4..9 do not
    layernorm_rope_rotate_ki(x.to(cuda), pos, pages, w.to(cuda), b.to(cuda), fr.to(cuda))
    p = pages.cpu()
    assert torch.all(p[0, :60 * 128] == 0) and torch.any(p[0, 60 * 128:64 * 128] != 0)
    assert torch.all(p[0, 64 * 128:64 * 128 + 60 * 4] == 0)
