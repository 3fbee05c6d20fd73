"""GPU parity of the block-scaled FP8 GEMM at the workload's full shapes against the CPU
oracle (the projection goldens' fp32 ``x_deq @ W_deq^T -> bf16``, refs/kernel.py:282-306,
projx_wqkva.py:503-529):

* config 0: one linear 7168 -> 18432 at M = 1, seed 0;
* config 3: the dense MLP's up 7168 -> 18432 and down 18432 -> 7168 at
  M in {1, 4, 16, 64, 256} (seeds 1..5), on both weight layouts.  On packed weights M = 64
  and 256 run the wide MFMA GEMM (up: 128 slices of 9 row tiles x 2 token groups at M =
  256; down: 64 slices of 7 row tiles split over K), canonical weights run the GEMV at
  M <= 64 and the tiled kernel at M = 256; M <= 16 runs the GEMV on both.

The bar is the workload's: relative L2 <= 5e-3 and max-abs <= 2 bf16 ulp of the output
scale (``tests/_tol.py``).
"""
import pytest
import torch

from oracle import reference as ref
from tests._tol import assert_gemm_close
from tilert_amd import kernel as K
from tilert_amd import synth

pytestmark = pytest.mark.gpu

SWEEP_M = (1, 4, 16, 64, 256)


class _Layer:
    """One full-size weight: CPU codes + dequantised fp32 copy for the oracle, the GPU
    canonical and packed forms for the kernels."""

    def __init__(self, N, Kd, seed, dev):
        w = synth.weight_fp32(N, Kd, synth.gen(seed))
        self.q, self.s = ref.weight_quant(w)
        del w
        self.wd = ref.weight_dequant(self.q, self.s)
        self.qg, self.sg = self.q.to(dev), self.s.to(dev)
        self.packed = K.pack_weight(self.qg, self.sg)
        self.N, self.K = N, Kd

    def check(self, M, seed, dev):
        x = synth.activations(M, self.K, synth.gen(seed))
        xq, xs = ref.act_quant(x)
        want = (ref.act_dequant(xq, xs) @ self.wd.T).to(torch.bfloat16)
        xg, xsg = xq.to(dev), xs.to(dev)
        out_c = K.fp8_gemm(xg, xsg, self.qg, self.sg)
        out_p = K.fp8_gemm(xg, xsg, self.packed)
        out_p2 = K.fp8_gemm(xg, xsg, self.packed)
        torch.cuda.synchronize()
        what = f"M={M} N={self.N} K={self.K} seed={seed}"
        print(what, flush=True)
        assert_gemm_close(out_c, want, "canonical " + what)
        assert_gemm_close(out_p, want, "packed " + what)
        assert torch.equal(out_p, out_p2), "packed GEMM not deterministic: " + what
        if M <= 16:  # the same GEMV on both layouts
            assert torch.equal(out_c, out_p), "layouts differ: " + what


@pytest.fixture(scope="module")
def up(cuda):
    return _Layer(18432, 7168, 0, cuda)


@pytest.fixture(scope="module")
def down(cuda):
    return _Layer(7168, 18432, 100, cuda)


def test_config0_single_linear_M1(cuda, up):
    up.check(1, 0, cuda)


@pytest.mark.parametrize("i,M", list(enumerate(SWEEP_M)))
def test_config3_up_7168x18432(cuda, up, i, M):
    up.check(M, 1 + i, cuda)


@pytest.mark.parametrize("i,M", list(enumerate(SWEEP_M)))
def test_config3_down_18432x7168(cuda, down, i, M):
    down.check(M, 1 + i, cuda)


@pytest.mark.parametrize("M", [200, 129])
def test_one_tile_per_workgroup_partial_token_group(cuda, up, M):
    """>= 256 output tiles with a partly empty second 128-token group."""
    up.check(M, 50 + M, cuda)


@pytest.mark.parametrize("M,N,Kd", [(256, 16384, 512), (200, 16384, 512), (130, 32768, 512)])
def test_many_tiles_small_k(cuda, M, N, Kd):
    """The one-tile-per-workgroup MFMA GEMM at a short K (4 blocks: ring prologue only)."""
    g = synth.gen(M + N + Kd)
    xq, xs = ref.act_quant(synth.activations(M, Kd, g))
    wq, ws = ref.weight_quant(synth.weight_fp32(N, Kd, g))
    packed = K.pack_weight(wq.to(cuda), ws.to(cuda))
    out = K.fp8_gemm(xq.to(cuda), xs.to(cuda), packed)
    assert_gemm_close(out, ref.fp8_gemm(xq, xs, wq, ws), f"M={M} N={N} K={Kd}")
