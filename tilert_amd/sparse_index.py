"""DSA lightning indexer with the reference's operators (ops/sparse_index.py:11-128):
``sparse_index`` fills the logits, ``sparse_index_topk`` also selects the exact top-k key
positions per token (one call: the scoring launch, then the top-k launch on the same stream
with a workspace kept per device and stream).

``sparse_index`` / ``sparse_index_topk`` keep the reference's signatures: bf16 q
[.., s, H, 128], bf16 index-key cache kv [.., L, 128], bf16 head weights [.., s, H],
fp32 logits [.., s, ld >= L], int32 indices [.., s, k]; cur_pos is the first token's
position and token t sees keys 0 .. cur_pos + t.  Scores are
``score_scale * sum_h w[t,h] * ReLU(q[t,h] . k[l])`` with score_scale = (128 H)^-1/2 applied
inside the kernel (the wrapper's "we precompute scale inner kernel": DeepSeek-V3.2's
indexer scales the head weights by H^-1/2 and the dot products by head_dim^-1/2; a
positive constant, so the selection does not depend on it).

``sparse_index_fp8`` / ``sparse_index_topk_fp8`` are the fp8 variant of the workload: q
e4m3fn with a per-token (or per-(token, head)) fp32 scale, keys e4m3fn [L, 128] with a
per-key fp32 scale (the fp8 KI cache of pd_vllm/profiles/mla_nsa.py:17-41,211-228,
flattened), scores ``sum_h w * ReLU(q . k)`` on the dequantised values.
"""
from __future__ import annotations

import torch

from . import _lib
from .kernel import SCALE_MODES, _Workspace, _require_cuda, _stream

_WS = _Workspace()


def score_scale(heads: int, dim: int = 128) -> float:
    """The bf16 operators' in-kernel score scale, (dim * heads)^-1/2."""
    return float((dim * heads) ** -0.5)


def _topk_workspace(dev: torch.device, st: int, M: int, ld: int, k: int) -> torch.Tensor:
    nbytes = _lib.query("tl_indexer_topk_workspace_bytes", M, ld, k)
    if nbytes == 0:
        raise ValueError(f"sparse_index_topk: {M} tokens x {ld} logits columns is beyond the top-k's limits")
    return _WS.get(dev, st, nbytes)

# The KI page format of pd_vllm/profiles/mla_nsa.py:17-41 (PAGE_SIZE, KI_PAGE_BYTES).
KI_PAGE_KEYS = 64
KI_PAGE_BYTES = KI_PAGE_KEYS * 128 + KI_PAGE_KEYS * 4  # 8448


def _check(q, q_scale, kv, k_scale, weights, logits, heads=(32, 64)):
    if q.dtype != torch.float8_e4m3fn:
        raise ValueError("q must be a float8_e4m3fn tensor.")
    if kv.dtype != torch.float8_e4m3fn:
        raise ValueError("kv must be a float8_e4m3fn tensor.")
    if weights.dtype != torch.bfloat16:
        raise ValueError("weights must be a bfloat16 tensor.")
    if logits.dtype != torch.float32:
        raise ValueError("logits must be a float32 tensor.")
    if q_scale.dtype != torch.float32 or k_scale.dtype != torch.float32:
        raise ValueError("q_scale and k_scale must be float32 tensors.")
    head, dim = q.shape[-2], q.shape[-1]
    if head not in heads:
        raise ValueError(f"Unsupported head size: {head}. Sparse index op currently only "
                         f"supports a head number of {' or '.join(map(str, heads))}.")
    if dim != 128 or kv.shape[-1] != 128:
        raise ValueError("dim must be 128, as we precompute scale inner kernel")
    device = q.device
    if any(t.device != device for t in (q_scale, kv, k_scale, weights, logits)):
        raise ValueError("sparse_index inputs must be on the same device")
    _require_cuda("sparse_index", q)
    for t in (q, q_scale, kv, k_scale, weights, logits):
        if not t.is_contiguous():
            raise ValueError("sparse_index inputs must be contiguous")


def sparse_index_fp8(q: torch.Tensor, q_scale: torch.Tensor, kv: torch.Tensor, k_scale: torch.Tensor,
                     weights: torch.Tensor, logits: torch.Tensor, cur_pos: int,
                     profile_logs: torch.Tensor | None = None, compute_kernel_type: str = "fp8", *,
                     model_arch: str = "deepseek_v3_2") -> None:
    """logits[t, l] = sum_h weights[t,h] * ReLU(q[t,h] . kv[l]) (dequantised), for the
    token at position ``cur_pos + t`` and keys l <= cur_pos + t; -inf for later keys.

    q [.., M, H, 128] e4m3fn; q_scale [M] or [M, H]; kv [L, 128] e4m3fn; k_scale [L];
    weights [M, H] bf16; logits [M, ld] fp32 (ld >= L; columns >= L are not written).
    """
    if compute_kernel_type != "fp8":
        raise ValueError(f"unsupported compute_kernel_type {compute_kernel_type!r}")
    _check(q, q_scale, kv, k_scale, weights, logits)
    H = q.shape[-2]
    M = q.numel() // (H * 128)
    L = kv.numel() // 128
    if weights.numel() != M * H:
        raise ValueError("weights must be [M, H]")
    per_head = q_scale.numel() == M * H and H > 1
    if not per_head and q_scale.numel() != M:
        raise ValueError("q_scale must be [M] or [M, H]")
    if k_scale.numel() != L:
        raise ValueError("k_scale must be [L]")
    ld = logits.shape[-1]
    if logits.numel() != M * ld or ld < L:
        raise ValueError("logits must be [M, ld] with ld >= L")
    _lib.call("tl_indexer_fp8_scores", q.data_ptr(), q_scale.data_ptr(), int(per_head), kv.data_ptr(),
              k_scale.data_ptr(), weights.data_ptr(), logits.data_ptr(), M, H, L, ld, int(cur_pos), _stream(q))


def sparse_index_topk_fp8(q: torch.Tensor, q_scale: torch.Tensor, kv: torch.Tensor,
                          k_scale: torch.Tensor, weights: torch.Tensor, logits: torch.Tensor,
                          indices: torch.Tensor, cur_pos: int,
                          profile_logs: torch.Tensor | None = None) -> None:
    """``sparse_index_fp8`` and the exact top-k of every token's visible keys (token t sees
    keys 0 .. cur_pos + t), one call.  indices int32 [M, k] (k = 2048 in DSA) receives
    the selected key positions in ascending order, -1 past the visible count."""
    if q.shape[-2] != 64:
        raise ValueError(f"Unsupported head size: {q.shape[-2]}. Sparse index topk fused op "
                         "supports head number of 64 (DSV3.2).")
    _check(q, q_scale, kv, k_scale, weights, logits)
    H = q.shape[-2]
    M = q.numel() // (H * 128)
    L = kv.numel() // 128
    per_head = q_scale.numel() == M * H and H > 1
    if not per_head and q_scale.numel() != M:
        raise ValueError("q_scale must be [M] or [M, H]")
    if weights.numel() != M * H or k_scale.numel() != L:
        raise ValueError("weights must be [M, H] and k_scale [L]")
    ld = logits.shape[-1]
    if logits.numel() != M * ld or ld < L:
        raise ValueError("logits must be [M, ld] with ld >= L")
    if indices.dtype != torch.int32 or indices.numel() % M or not indices.is_contiguous():
        raise ValueError("indices must be a contiguous int32 [M, k] tensor")
    k = indices.numel() // M
    st = _stream(q)
    ws = _topk_workspace(q.device, st, M, ld, k)
    _lib.call("tl_indexer_fp8_topk", q.data_ptr(), q_scale.data_ptr(), int(per_head), kv.data_ptr(),
              k_scale.data_ptr(), weights.data_ptr(), logits.data_ptr(), M, H, L, ld, int(cur_pos), k,
              indices.data_ptr(), ws.data_ptr(), ws.numel(), st)


# ------------------------------------------------ the reference's bf16 operators
def _check_bf16(q, kv, weights, logits, profile_logs, extra=()):
    """The reference wrapper's checks (ops/sparse_index.py:40-66), then this build's
    layout requirements."""
    if q.dtype != torch.bfloat16:
        raise ValueError("input must be a bfloat16 tensor.")
    if kv.dtype != torch.bfloat16:
        raise ValueError("kv must be a bfloat16 tensor.")
    if weights.dtype != torch.bfloat16:
        raise ValueError("weights must be a bfloat16 tensor.")
    if logits.dtype != torch.float32:
        raise ValueError("logits must be a float32 tensor.")
    head, dim = q.shape[-2], q.shape[-1]
    if dim != 128 or kv.shape[-1] != 128:
        raise ValueError("dim must be 128, as we precompute scale inner kernel")
    device = q.device
    others = (kv, weights, logits, *extra) + ((profile_logs,) if profile_logs is not None else ())
    if any(t.device != device for t in others):
        raise ValueError("sparse_index inputs must be on the same device: "
                         f"q={device}, kv={kv.device}, weights={weights.device}, logits={logits.device}")
    _require_cuda("sparse_index", q)
    for t in (q, kv, weights, logits, *extra):
        if not t.is_contiguous():
            raise ValueError("sparse_index inputs must be contiguous")
    M = q.numel() // (head * 128)
    L = kv.numel() // 128
    if weights.numel() != M * head:
        raise ValueError("weights must be [.., s, heads]")
    ld = logits.shape[-1]
    if logits.numel() != M * ld or ld < L:
        raise ValueError("logits must be [.., s, ld] with ld >= the cache length")
    return head, M, L, ld


def sparse_index(q: torch.Tensor, kv: torch.Tensor, weights: torch.Tensor, logits: torch.Tensor, cur_pos: int,
                 profile_logs: torch.Tensor | None = None, compute_kernel_type: str = "bf16", *,
                 model_arch: str = "deepseek_v3_2") -> None:
    """``sparse_index`` (ops/sparse_index.py:11-69): logits[t, l] = score_scale * sum_h
    weights[t,h] * ReLU(q[t,h] . kv[l]) for keys l <= cur_pos + t, -inf after."""
    if compute_kernel_type != "bf16":
        raise ValueError(f"Unsupported compute_kernel_type: {compute_kernel_type}")
    if model_arch not in ("deepseek_v3_2", "glm_5"):
        raise ValueError(f"Unsupported architecture: {model_arch}")
    head = q.shape[-2]
    if head != 64 and head != 32:
        raise ValueError(f"Unsupported head size: {head}. Sparse index op currently only "
                         "supports a head number of 64 or 32.")
    H, M, L, ld = _check_bf16(q, kv, weights, logits, profile_logs)
    _lib.call("tl_indexer_bf16_scores", q.data_ptr(), kv.data_ptr(), weights.data_ptr(), score_scale(H),
              logits.data_ptr(), M, H, L, ld, int(cur_pos), _stream(q))


def _bf16_topk(q, kv, weights, logits, indices, cur_pos, profile_logs):
    H, M, L, ld = _check_bf16(q, kv, weights, logits, profile_logs, (indices,))
    if indices.dtype != torch.int32 or indices.numel() % M:
        raise ValueError("indices must be an int32 [.., s, k] tensor")
    k = indices.numel() // M
    st = _stream(q)
    ws = _topk_workspace(q.device, st, M, ld, k)
    _lib.call("tl_indexer_bf16_topk", q.data_ptr(), kv.data_ptr(), weights.data_ptr(), score_scale(H),
              logits.data_ptr(), M, H, L, ld, int(cur_pos), k, indices.data_ptr(), ws.data_ptr(), ws.numel(), st)


def sparse_index_topk(q: torch.Tensor, kv: torch.Tensor, weights: torch.Tensor, logits: torch.Tensor,
                      indices: torch.Tensor, cur_pos: int, profile_logs: torch.Tensor | None = None) -> None:
    """``sparse_index_topk`` (ops/sparse_index.py:72-128, the DeepSeek-V3.2 fused op):
    ``sparse_index``'s logits and the exact top-k per token into ``indices`` [.., s, k]
    (ascending key positions, -1 past the visible count), one call.  The workspace the
    reference allocates per call is kept per device and stream (its counters are left
    zeroed by every call)."""
    head = q.shape[-2]
    if head != 64:
        raise ValueError(f"Unsupported head size: {head}. Sparse index topk fused op "
                         "supports head number of 64 (DSV3.2).")
    _bf16_topk(q, kv, weights, logits, indices, cur_pos, profile_logs)


def ki_pages_from_flat(kv: torch.Tensor, k_scale: torch.Tensor) -> torch.Tensor:
    """The KI page image of a flat fp8 cache: kv e4m3fn [L, 128] and k_scale fp32 [L] ->
    uint8 [ceil(L/64), 8448]; page p holds keys 64p .. 64p+63 (fp8 rows, then their
    scales), the layout ``MlaNsaProfile._dequant_ki`` reads (mla_nsa.py:211-228).  Rows
    past L are zero.  A layout conversion in torch (load time), not a hot-path op."""
    if kv.dtype != torch.float8_e4m3fn or kv.dim() != 2 or kv.shape[1] != 128:
        raise ValueError("kv must be a float8_e4m3fn [L, 128] tensor")
    if k_scale.dtype != torch.float32 or k_scale.numel() != kv.shape[0]:
        raise ValueError("k_scale must be a float32 [L] tensor")
    L = kv.shape[0]
    n_pages = (L + KI_PAGE_KEYS - 1) // KI_PAGE_KEYS
    pages = torch.zeros(n_pages, KI_PAGE_BYTES, dtype=torch.uint8, device=kv.device)
    full = torch.zeros(n_pages * KI_PAGE_KEYS, 128, dtype=torch.uint8, device=kv.device)
    full[:L] = kv.view(torch.uint8)
    sc = torch.zeros(n_pages * KI_PAGE_KEYS, dtype=torch.float32, device=kv.device)
    sc[:L] = k_scale.reshape(-1)
    pages[:, :KI_PAGE_KEYS * 128] = full.reshape(n_pages, KI_PAGE_KEYS * 128)
    pages[:, KI_PAGE_KEYS * 128:] = sc.reshape(n_pages, KI_PAGE_KEYS).view(torch.uint8).reshape(n_pages, -1)
    return pages


def ki_cache_write(keys: torch.Tensor, ki_pages: torch.Tensor, pos: int, scale_fmt: str | None = "div") -> None:
    """Quantise ``keys`` (bf16 [n, 128]) per key to e4m3fn with an fp32 scale and store them
    at positions pos .. pos+n-1 of ``ki_pages`` (uint8 [n_pages, 8448]).  ``scale_fmt`` as in
    ``act_quant``; the default "div" is the per-token amax / 448 of the
    workload's key cache."""
    if keys.dtype != torch.bfloat16 or keys.dim() != 2 or keys.shape[1] != 128 or not keys.is_contiguous():
        raise ValueError("keys must be a contiguous bfloat16 [n, 128] tensor")
    if ki_pages.dtype != torch.uint8 or ki_pages.dim() != 2 or ki_pages.shape[1] != KI_PAGE_BYTES \
            or not ki_pages.is_contiguous():
        raise ValueError(f"ki_pages must be a contiguous uint8 [n_pages, {KI_PAGE_BYTES}] tensor")
    if keys.device != ki_pages.device:
        raise ValueError("keys and ki_pages must be on the same device")
    _require_cuda("ki_cache_write", keys)
    _lib.call("tl_ki_cache_write", keys.data_ptr(), keys.shape[0], ki_pages.data_ptr(), ki_pages.shape[0],
              int(pos), SCALE_MODES.get(scale_fmt, 1), _stream(keys))


def sparse_index_paged(q: torch.Tensor, q_scale: torch.Tensor, ki_pages: torch.Tensor,
                       weights: torch.Tensor, logits: torch.Tensor, cur_pos: int, seq_len: int) -> None:
    """``sparse_index`` over the paged KI cache (uint8 [n_pages, 8448], keys 0 .. seq_len-1):
    bit-identical to ``sparse_index`` on the equivalent flat cache."""
    if ki_pages.dtype != torch.uint8 or ki_pages.dim() != 2 or ki_pages.shape[1] != KI_PAGE_BYTES \
            or not ki_pages.is_contiguous():
        raise ValueError(f"ki_pages must be a contiguous uint8 [n_pages, {KI_PAGE_BYTES}] tensor")
    L = int(seq_len)
    if L < 0 or L > ki_pages.shape[0] * KI_PAGE_KEYS:
        raise ValueError("seq_len exceeds the pages' capacity")
    # validate q / weights / logits exactly as the flat op does (a [L, 128] view stands in
    # for the cache in the shape checks)
    _check(q, q_scale, torch.empty(0, 128, dtype=torch.float8_e4m3fn, device=q.device),
           torch.empty(0, dtype=torch.float32, device=q.device), weights, logits)
    if ki_pages.device != q.device:
        raise ValueError("sparse_index inputs must be on the same device")
    H = q.shape[-2]
    M = q.numel() // (H * 128)
    if weights.numel() != M * H:
        raise ValueError("weights must be [M, H]")
    per_head = q_scale.numel() == M * H and H > 1
    if not per_head and q_scale.numel() != M:
        raise ValueError("q_scale must be [M] or [M, H]")
    ld = logits.shape[-1]
    if logits.numel() != M * ld or ld < L:
        raise ValueError("logits must be [M, ld] with ld >= seq_len")
    _lib.call("tl_indexer_fp8_scores_paged", q.data_ptr(), q_scale.data_ptr(), int(per_head), ki_pages.data_ptr(),
              ki_pages.shape[0], weights.data_ptr(), logits.data_ptr(), M, H, L, ld, int(cur_pos), _stream(q))
