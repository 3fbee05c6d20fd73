"""FP8 block-scaled primitives with the signatures of the reference's
``tilert/models/deepseek_v3_2/refs/kernel.py`` (act_quant :252-279, fp8_gemm :282-306,
weight_dequant :97-129), running on the gfx950 HIP library.

All tensors live on the GPU.  fp8 tensors are ``torch.float8_e4m3fn`` (OCP e4m3fn, the
format gfx950's MFMA consumes natively).
"""
from __future__ import annotations

import torch

from . import _lib

BLOCK = 128
SCALE_MODES = {None: 0, "ue8m0": 1, "div": 2}


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _require_cuda(name: str, *ts: torch.Tensor | None) -> None:
    """Every tensor that reaches a kernel must live on the same GPU (None = not passed)."""
    ts = tuple(t for t in ts if t is not None)
    for t in ts:
        if not t.is_cuda:
            raise ValueError(f"{name}: all tensors must be on a GPU (got {t.device})")
    dev = ts[0].device
    for t in ts:
        if t.device != dev:
            raise ValueError(f"{name}: tensors on different devices ({dev} vs {t.device})")


def act_quant(x: torch.Tensor, block_size: int = 128, scale_fmt: str | None = None
              ) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantise ``x`` (bf16, [..., K]) per 1x128 group to e4m3fn with fp32 scales.

    ``scale_fmt=None``: s = max(amax,1e-4) * fp32(1/448) (refs/kernel.py:191);
    any other value selects the power-of-two "ue8m0" scale (refs/kernel.py:140-151,189),
    except ``"div"`` which selects s = max(amax,1e-4)/448.
    Returns (y float8_e4m3fn [..., K], s float32 [..., K/128]).
    """
    if not x.is_contiguous():
        raise AssertionError("Input tensor must be contiguous")
    if x.size(-1) % block_size != 0:
        raise AssertionError(f"Last dimension size must be divisible by block_size (block_size={block_size})")
    if x.dtype != torch.bfloat16:
        raise ValueError(f"act_quant: x must be bfloat16 (got {x.dtype})")
    _require_cuda("act_quant", x)
    mode = SCALE_MODES.get(scale_fmt, 1)
    N = x.size(-1)
    y = torch.empty_like(x, dtype=torch.float8_e4m3fn)
    s = x.new_empty(*x.size()[:-1], N // block_size, dtype=torch.float32)
    rows = x.numel() // N if N else 0
    _lib.call("tl_act_quant", x.data_ptr(), y.data_ptr(), s.data_ptr(), rows, N, block_size,
              mode, _stream(x))
    return y, s


def weight_quant(w: torch.Tensor, block_size: int = 128) -> tuple[torch.Tensor, torch.Tensor]:
    """128x128 block quantisation of an fp32/bf16 weight [N, K] -> (e4m3fn [N,K], fp32 scales
    [ceil(N/128), ceil(K/128)]), s = block_amax / 448."""
    if block_size != BLOCK:
        raise ValueError("weight_quant: block_size must be 128")
    if w.dim() != 2 or not w.is_contiguous():
        raise AssertionError("Input tensors must be contiguous and have 2 dimensions")
    if w.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"weight_quant: unsupported dtype {w.dtype}")
    _require_cuda("weight_quant", w)
    N, K = w.shape
    q = torch.empty(N, K, dtype=torch.float8_e4m3fn, device=w.device)
    s = torch.empty((N + BLOCK - 1) // BLOCK, (K + BLOCK - 1) // BLOCK, dtype=torch.float32, device=w.device)
    _lib.call("tl_weight_quant", w.data_ptr(), int(w.dtype == torch.bfloat16), q.data_ptr(),
              s.data_ptr(), N, K, _stream(w))
    return q, s


def weight_dequant(x_in: torch.Tensor, s_in: torch.Tensor, block_size: int = 128) -> torch.Tensor:
    """``W = fp32(Wq) * S`` per 128x128 block, returned in ``torch.get_default_dtype()``
    when that is fp32 or bf16 (refs/kernel.py:97-129)."""
    if not (x_in.is_contiguous() and s_in.is_contiguous()):
        raise AssertionError("Input tensors must be contiguous")
    if x_in.dim() != 2 or s_in.dim() != 2:
        raise AssertionError("Input tensors must have 2 dimensions")
    if block_size != BLOCK:
        raise ValueError("weight_dequant: block_size must be 128")
    if x_in.dtype != torch.float8_e4m3fn or s_in.dtype != torch.float32:
        raise ValueError("weight_dequant: expects float8_e4m3fn weights and float32 scales")
    _require_cuda("weight_dequant", x_in, s_in)
    dt = torch.get_default_dtype()
    if dt not in (torch.float32, torch.bfloat16):
        raise ValueError(f"weight_dequant: default dtype {dt} not supported")
    N, K = x_in.shape
    y = torch.empty(N, K, dtype=dt, device=x_in.device)
    _lib.call("tl_weight_dequant", x_in.data_ptr(), s_in.data_ptr(), y.data_ptr(),
              int(dt == torch.bfloat16), N, K, _stream(x_in))
    return y


class _Workspace:
    """Per-(device, stream) zero-initialised scratch for split-K GEMMs.

    The kernels leave the counter region zeroed after every call, so the buffer is only
    zero-filled when it is (re)allocated.  Calls on one stream are ordered, which is what
    makes sharing one buffer per stream safe.
    """

    def __init__(self) -> None:
        self._bufs: dict[tuple[int, int], torch.Tensor] = {}
        # Buffers replaced by a larger one stay allocated until the process ends: a HIP
        # graph captured while one of them was current still addresses it on replay, so
        # freeing it would hand its (no longer zeroed) memory to another tensor.
        self._retired: list[torch.Tensor] = []

    def get(self, device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
        key = (device.index, stream)
        buf = self._bufs.get(key)
        if buf is None or buf.numel() < nbytes:
            if buf is not None:
                self._retired.append(buf)
            buf = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
            self._bufs[key] = buf
        return buf


_WS = _Workspace()


class PackedFP8Weight:
    """A block-scaled fp8 weight [N, K] repacked into MFMA operand fragments.

    Built once at weight-load time (the role of the reference's per-op weight converters,
    e.g. ``RMSNormProjQKVAFP8MMAWeightsConverter``); ``fp8_gemm``/``linear`` accept it in
    place of the canonical weight and give bit-identical results, streaming ~25% faster.
    """

    def __init__(self, data: torch.Tensor, scale: torch.Tensor, N: int, K: int) -> None:
        self.data, self.scale, self.N, self.K = data, scale, N, K

    @property
    def shape(self) -> tuple[int, int]:
        return (self.N, self.K)

    @property
    def device(self) -> torch.device:
        return self.data.device


def pack_weight(b: torch.Tensor, b_s: torch.Tensor) -> PackedFP8Weight:
    """Repack a canonical e4m3fn weight [N, K] (+ its [ceil(N/128), K/128] scales)."""
    if b.dtype != torch.float8_e4m3fn or b.dim() != 2 or not b.is_contiguous():
        raise ValueError("pack_weight: expects a contiguous 2-D float8_e4m3fn weight")
    _require_cuda("pack_weight", b)
    N, K = b.shape
    out = torch.empty(N * K, dtype=torch.uint8, device=b.device)
    _lib.call("tl_fp8_pack_weight", b.data_ptr(), out.data_ptr(), N, K, _stream(b))
    return PackedFP8Weight(out, b_s.contiguous(), N, K)


def fp8_gemm(a: torch.Tensor, a_s: torch.Tensor, b, b_s: torch.Tensor | None = None,
             out: torch.Tensor | None = None) -> torch.Tensor:
    """``C = A . B^T`` with per-128-block scales; A e4m3fn [..., K] + a_s [..., K/128],
    B e4m3fn [N, K] (or a ``PackedFP8Weight``) + b_s [ceil(N/128), K/128].  Returns bf16
    [..., N] (refs/kernel.py:282-306; bf16 is DeepSeek inference's default dtype)."""
    packed = isinstance(b, PackedFP8Weight)
    if packed:
        b_s = b.scale if b_s is None else b_s
        bt = b.data
    else:
        bt = b
    if not (a.is_contiguous() and bt.is_contiguous()):
        raise AssertionError("Input tensors must be contiguous")
    if not (a_s.is_contiguous() and b_s.is_contiguous()):
        raise AssertionError("Scaling factor tensors must be contiguous")
    if a.dtype != torch.float8_e4m3fn or (not packed and b.dtype != torch.float8_e4m3fn):
        raise ValueError("fp8_gemm: a and b must be float8_e4m3fn")
    if a_s.dtype != torch.float32 or b_s.dtype != torch.float32:
        raise ValueError("fp8_gemm: scales must be float32")
    _require_cuda("fp8_gemm", a, a_s, bt, b_s)
    K = a.size(-1)
    M = a.numel() // K
    N = b.shape[0]
    if b.shape[1] != K:
        raise ValueError(f"fp8_gemm: K mismatch ({K} vs {b.shape[1]})")
    if a_s.numel() != M * (K // BLOCK) or b_s.shape != ((N + BLOCK - 1) // BLOCK, K // BLOCK):
        raise ValueError("fp8_gemm: scale shapes do not match the operands")
    if out is None:
        out = a.new_empty(*a.size()[:-1], N, dtype=torch.bfloat16)
    elif out.dtype != torch.bfloat16 or not out.is_contiguous() or out.numel() != M * N:
        raise ValueError("fp8_gemm: out must be a contiguous bf16 tensor of M*N elements")
    _require_cuda("fp8_gemm", a, out)
    st = _stream(a)
    nbytes = _lib.query("tl_fp8_gemm_workspace_bytes", M, N, K)
    ws_ptr, ws_len = None, 0
    if nbytes:
        ws = _WS.get(a.device, st, nbytes)
        ws_ptr, ws_len = ws.data_ptr(), ws.numel()
    _lib.call("tl_fp8_gemm_packed" if packed else "tl_fp8_gemm", a.data_ptr(), a_s.data_ptr(),
              bt.data_ptr(), b_s.data_ptr(), out.data_ptr(), M, N, K, ws_ptr, ws_len, st)
    return out
