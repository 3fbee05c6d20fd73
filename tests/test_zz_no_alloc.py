"""The allocation-free entry point ``tl_fp8_gemm_packed_static`` (scratch in a static device
array) against ``tl_fp8_gemm_packed`` with a caller workspace, through the C ABI: bit-identical
on two calls in a row (the second smaller, so it runs over the first call's leftover scratch),
and a clear error for a shape whose scratch exceeds the static maximum."""
import pytest
import torch

from oracle import reference as ref
from tilert_amd import _lib
from tilert_amd import kernel as K
from tilert_amd import synth

pytestmark = pytest.mark.gpu

def _case(M, N, Kd, seed, dev):
    g = synth.gen(seed)
    xq, xs = ref.act_quant(synth.activations(M, Kd, g))
    wq, ws = ref.weight_quant(synth.weight_fp32(N, Kd, g))
    packed = K.pack_weight(wq.to(dev), ws.to(dev))
    return xq.to(dev), xs.to(dev), packed


def _with_workspace(xq, xs, packed, M, N, Kd, dev):
    lib = _lib.load()
    need = lib.tl_fp8_gemm_workspace_bytes(M, N, Kd)
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=dev)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    st = torch.cuda.current_stream(dev).cuda_stream
    rc = lib.tl_fp8_gemm_packed(xq.data_ptr(), xs.data_ptr(), packed.data.data_ptr(), packed.scale.data_ptr(),
                                out.data_ptr(), M, N, Kd, ws.data_ptr() if need else None, need, st)
    assert rc == 0, lib.tl_last_error()
    return out


def _static(xq, xs, packed, M, N, Kd, dev):
    lib = _lib.load()
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    st = torch.cuda.current_stream(dev).cuda_stream
    rc = lib.tl_fp8_gemm_packed_static(xq.data_ptr(), xs.data_ptr(), packed.data.data_ptr(), packed.scale.data_ptr(),
                                       out.data_ptr(), M, N, Kd, st)
    assert rc == 0, lib.tl_last_error()
    return out


@pytest.mark.parametrize("first,second", [
    # the wide MFMA GEMM with a K split (fp32 partials), then the split-K GEMV over its leftovers
    ((256, 7168, 4096), (40, 576, 7168)),
    # GEMV with the activation image and 4 row tiles, then a plain M = 4 GEMV (no scratch)
    ((64, 18432, 7168), (4, 1024, 2048)),
    # split-K GEMV at M > 16, then a smaller split-K GEMV: the counters must be zero again
    ((48, 1024, 7168), (17, 512, 2048)),
    # the largest dense-MLP shapes of the M sweep (down 18432 -> 7168 at M = 256 has the
    # largest scratch of the sweep), then up at M = 64
    ((256, 7168, 18432), (64, 18432, 7168)),
])
def test_static_matches_workspace_entry_point(cuda, first, second):
    for i, (M, N, Kd) in enumerate((first, second)):
        print(f"static scratch case {i}: M={M} N={N} K={Kd}", flush=True)
        xq, xs, packed = _case(M, N, Kd, 7 * M + N + Kd, cuda)
        want = _with_workspace(xq, xs, packed, M, N, Kd, cuda)
        got = _static(xq, xs, packed, M, N, Kd, cuda)
        again = _static(xq, xs, packed, M, N, Kd, cuda)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"static scratch differs from the workspace call at {(M, N, Kd)}"
        assert torch.equal(again, want), f"repeated static call differs at {(M, N, Kd)}"


def test_static_rejects_shapes_beyond_the_maximum(cuda):
    lib = _lib.load()
    dev = cuda
    # M = 64 over K = 655360: the GEMV's activation image (64 x K bytes + scales) exceeds 40 MiB
    M, N, Kd = 64, 16, 655360
    a = torch.zeros(M, Kd, dtype=torch.float8_e4m3fn, device=dev)
    a_s = torch.ones(M, Kd // 128, device=dev)
    b = torch.zeros(N * Kd, dtype=torch.uint8, device=dev)
    b_s = torch.ones((N + 127) // 128, Kd // 128, device=dev)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    rc = lib.tl_fp8_gemm_packed_static(a.data_ptr(), a_s.data_ptr(), b.data_ptr(), b_s.data_ptr(), out.data_ptr(),
                                       M, N, Kd, torch.cuda.current_stream(dev).cuda_stream)
    assert rc == 3
    assert b"static maximum" in lib.tl_last_error()
