"""GPU parity of act_quant, weight_quant/dequant and the block-scaled FP8 GEMM against
the CPU oracle (bit-exact for quantisation, stated tolerances for GEMM outputs)."""
import numpy as np
import pytest
import torch

from oracle import reference as ref
from tests._tol import assert_gemm_close
from tilert_amd import kernel as K
from tilert_amd import synth

pytestmark = pytest.mark.gpu


def _all_bf16_finite() -> torch.Tensor:
    bits = np.arange(65536, dtype=np.uint32)
    f = (bits << 16).view(np.float32)
    f = f[np.isfinite(f)]
    pad = (-len(f)) % 128
    f = np.concatenate([f, np.zeros(pad, np.float32)])
    return torch.from_numpy(f).to(torch.bfloat16).reshape(-1, 128)


@pytest.mark.parametrize("mode,fmt", [(0, None), (1, "ue8m0"), (2, "div")])
def test_act_quant_exhaustive_bf16(cuda, mode, fmt):
    """Every finite bf16 value, in groups mixing magnitudes (shuffled) and in sorted
    groups (so both tiny and huge amax occur): codes and scales bit-exact."""
    x = _all_bf16_finite()
    g = torch.Generator().manual_seed(0)
    xs = x.flatten()[torch.randperm(x.numel(), generator=g)].reshape(-1, 128)
    for xx in (x, xs, torch.cat([x, xs], 1)):
        y, s = K.act_quant(xx.to(cuda).contiguous(), 128, fmt)
        ry, rs = ref.act_quant(xx, 128, mode)
        assert torch.equal(s.cpu(), rs), "scales differ"
        assert torch.equal(y.cpu().view(torch.uint8), ry.view(torch.uint8)), "codes differ"


def test_act_quant_edge_groups(cuda):
    x = torch.zeros(4, 256, dtype=torch.bfloat16)
    x[1, :128] = 3.0
    x[2, 5] = -1e-30
    x[3, 130] = 448.0
    y, s = K.act_quant(x.to(cuda), 128)
    ry, rs = ref.act_quant(x, 128)
    assert torch.equal(s.cpu(), rs)
    assert torch.equal(y.cpu().view(torch.uint8), ry.view(torch.uint8))


@pytest.mark.parametrize("N,Kd", [(128, 128), (576, 7168), (300, 520), (2048, 1536)])
def test_weight_quant_bit_exact(cuda, N, Kd):
    w = synth.weight_fp32(N, Kd, synth.gen(N + Kd))
    q, s = K.weight_quant(w.to(cuda))
    rq, rs = ref.weight_quant(w)
    assert torch.equal(s.cpu(), rs)
    assert torch.equal(q.cpu().view(torch.uint8), rq.view(torch.uint8))
    d = K.weight_dequant(q, s)
    assert torch.equal(d.cpu(), ref.weight_dequant(rq, rs).to(torch.get_default_dtype()))


GEMM_CASES = [
    # (M, N, K)
    (1, 256, 512),
    (4, 576, 7168),     # wkv_a: partial last scale row
    (32, 576, 7168),    # 36 row tiles at M > 16: split-K in 4 slices
    (2, 7168, 6144),    # wide and long: 4 operand buffers per wave
    (4, 3072, 1536),    # wq_b
    (4, 4096, 512),     # wkv_b
    (4, 7168, 2048),    # wo
    (3, 1536, 7168),    # wq_a, odd M
    (16, 2048, 1024),
    (17, 512, 1024),
    (64, 1024, 2048),
    (256, 512, 1024),
    (64, 2048, 7168),   # canonical: per-row-tile kernel, 4 token tiles, split-K; packed: wide kernel
    (128, 2048, 7168),  # tiled kernel (M > 64) with split-K
    (32, 1152, 2048),
    (200, 400, 2048),   # 25 row tiles: a partly empty last 128-row group
    (100, 7168, 1024),
    # several row tiles per workgroup sharing each activation fragment
    (16, 7168, 1024),   # 2 row tiles, 1 token tile
    (16, 7168, 640),    # the same on the canonical (unpacked) layout
    (32, 18432, 512),   # 4 row tiles, 2 token tiles
    (24, 6144, 512),    # 2 row tiles, 2 token tiles
    (48, 7168, 1024),   # 2 row tiles, 4 token tiles
    (64, 12288, 512),   # 4 row tiles, 4 token tiles
    # M > 32 (or > 16 with K split in <= 2), packed: wide MFMA GEMM (F row tiles per
    # workgroup, S K ranges)
    (65, 128, 512),     # F = 4: 2 slices, each split over all 4 K blocks: 4 partials
    (192, 1024, 2048),  # F = 8: 2 token groups, the second half full; 8 tiles x 16 K ranges
    (40, 2048, 1024),   # one token group with 3 of its 8 fragments past M
    (200, 640, 2048),   # F = 5
    (200, 768, 2048),   # F = 6
    (200, 1152, 2048),  # F = 9
    (200, 4352, 1024),  # F = 8, K ranges of 3, 3 and 2 blocks
    (255, 2048, 1024),  # last token fragment 15/16 full, second token group
    (33, 7168, 512),    # 3 of 8 token fragments valid, 4 K ranges of one block
]


@pytest.mark.parametrize("M,N,Kd", GEMM_CASES)
def test_fp8_gemm_vs_oracle(cuda, M, N, Kd):
    g = synth.gen(1000 + M + N + Kd)
    x = synth.activations(M, Kd, g)
    w = synth.weight_fp32(N, Kd, g)
    wq, ws = ref.weight_quant(w)
    xq, xs = ref.act_quant(x)
    out = K.fp8_gemm(xq.to(cuda), xs.to(cuda), wq.to(cuda), ws.to(cuda))
    out2 = K.fp8_gemm(xq.to(cuda), xs.to(cuda), wq.to(cuda), ws.to(cuda))
    torch.cuda.synchronize()
    assert torch.equal(out, out2), "fp8_gemm is not deterministic"
    assert_gemm_close(out, ref.fp8_gemm(xq, xs, wq, ws), f"M={M} N={N} K={Kd}")
    if Kd % 512 == 0:
        packed = K.pack_weight(wq.to(cuda), ws.to(cuda))
        outp = K.fp8_gemm(xq.to(cuda), xs.to(cuda), packed)
        if M <= 16 or N % 128:  # the same GEMV kernel on both layouts
            assert torch.equal(outp, out), "packed-weight GEMM differs from the canonical one"
        else:  # the wide MFMA GEMM (packed) and the GEMV / tiled kernel (canonical) sum differently
            assert torch.equal(outp, K.fp8_gemm(xq.to(cuda), xs.to(cuda), packed)), "not deterministic"
            assert_gemm_close(outp, ref.fp8_gemm(xq, xs, wq, ws), f"packed M={M} N={N} K={Kd}")


def test_pack_weight_layout(cuda):
    """The K-group-major fragment layout documented in include/tilert_amd.h, byte by byte."""
    N, Kd = 48, 1024
    w = torch.randint(0, 256, (N, Kd), dtype=torch.uint8)
    p = K.pack_weight(w.view(torch.float8_e4m3fn).to(cuda), torch.ones(1, 8, device=cuda)).data.cpu()
    NT = N // 16
    for t in range(NT):
        for kb in range(Kd // 128):
            f = ((kb // 4) * NT + t) * 4 + kb % 4
            frag = p[f * 2048:(f + 1) * 2048].reshape(2, 64, 16)
            for piece in range(2):
                for lane in range(64):
                    row = 16 * t + lane % 16
                    col = 128 * kb + 64 * piece + 16 * (lane // 16)
                    assert torch.equal(frag[piece, lane], w[row, col:col + 16])


def test_fp8_gemm_one_hot_picks_column(cuda):
    """x = e_k (one nonzero) selects dequantised column k of W exactly (up to bf16)."""
    N, Kd = 256, 1024
    w = synth.weight_fp32(N, Kd, synth.gen(7))
    wq, ws = ref.weight_quant(w)
    x = torch.zeros(2, Kd, dtype=torch.bfloat16)
    x[0, 300] = 1.0
    x[1, 1023] = -2.0
    xq, xs = ref.act_quant(x)
    out = K.fp8_gemm(xq.to(cuda), xs.to(cuda), wq.to(cuda), ws.to(cuda)).cpu()
    wd = ref.weight_dequant(wq, ws)
    assert torch.equal(out[0], wd[:, 300].to(torch.bfloat16))
    assert torch.equal(out[1], (-2.0 * wd[:, 1023]).to(torch.bfloat16))


def test_linear_matches_oracle(cuda):
    from tilert_amd.common import linear
    M, N, Kd = 4, 1024, 7168
    g = synth.gen(11)
    x = synth.activations(M, Kd, g)
    wq, ws = ref.weight_quant(synth.weight_fp32(N, Kd, g))
    out = linear(x.to(cuda), wq.to(cuda), ws.to(cuda))
    assert_gemm_close(out, ref.linear(x, wq, ws), "linear")


def test_fp8_gemm_rejects_bad_shapes(cuda):
    a = torch.zeros(4, 100, dtype=torch.float8_e4m3fn, device=cuda)
    with pytest.raises((AssertionError, ValueError, RuntimeError)):
        K.fp8_gemm(a, torch.zeros(4, 1, device=cuda), a, torch.zeros(1, 1, device=cuda))


@pytest.mark.parametrize("M,N,Kd", [(32, 576, 7168), (4, 18432, 7168), (2, 7168, 2048), (64, 2048, 7168), (128, 2048, 7168)])
def test_fp8_gemm_split_k_repeatable(cuda, M, N, Kd):
    """The cross-workgroup split-K reduction must give bit-identical results on every
    call (a stale or missing partial would show up as a changed output)."""
    g = synth.gen(99 + N)
    xq, xs = ref.act_quant(synth.activations(M, Kd, g))
    wq, ws = ref.weight_quant(synth.weight_fp32(N, Kd, g))
    xq, xs, wq, ws = xq.to(cuda), xs.to(cuda), wq.to(cuda), ws.to(cuda)
    packed = K.pack_weight(wq, ws)
    first = K.fp8_gemm(xq, xs, packed)
    first_c = K.fp8_gemm(xq, xs, wq, ws)
    outs = [K.fp8_gemm(xq, xs, packed) for _ in range(30)]
    outs_c = [K.fp8_gemm(xq, xs, wq, ws) for _ in range(10)]
    torch.cuda.synchronize()
    for o in outs:
        assert torch.equal(o, first)
    for o in outs_c:  # packed M > 16 with N % 128 = 0 may run the wide kernel; canonical: another one
        assert torch.equal(o, first if (M <= 16 or N % 128) else first_c)
