"""ctypes binding of ``libtilert_amd.so`` (the C ABI in ``include/tilert_amd.h``).

The library is loaded lazily on first use.  There is no fallback: if the shared library
is missing or fails to load, every op raises ``RuntimeError`` -- the product path is the
HIP path or nothing.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

_PKG = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("TILERT_AMD_LIB", _PKG / "libtilert_amd.so"))

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_size = ctypes.c_size_t

# name -> (restype, argtypes)
SIGNATURES: dict[str, tuple] = {
    "tl_last_error": (ctypes.c_char_p, []),
    "tl_version": (ctypes.c_char_p, []),
    "tl_act_quant": (_int, [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _int, _c_void_p]),
    "tl_weight_quant": (_int, [_c_void_p, _int, _c_void_p, _c_void_p, _i64, _i64, _c_void_p]),
    "tl_weight_dequant": (_int, [_c_void_p, _c_void_p, _c_void_p, _int, _i64, _i64, _c_void_p]),
    "tl_fp8_gemm_workspace_bytes": (_size, [_i64, _i64, _i64]),
    "tl_fp8_gemm": (_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                           _i64, _i64, _i64, _c_void_p, _size, _c_void_p]),
    "tl_fp8_pack_weight": (_int, [_c_void_p, _c_void_p, _i64, _i64, _c_void_p]),
    "tl_moe_pack_weight": (_int, [_c_void_p, _c_void_p, _i64, _i64, _c_void_p]),
    "tl_fp8_gemm_packed": (_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                  _i64, _i64, _i64, _c_void_p, _size, _c_void_p]),
    "tl_fp8_gemm_packed_static": (_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                         _i64, _i64, _i64, _c_void_p]),
    "tl_projx_wqkva": (_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                              _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                              _c_void_p, _size, _c_void_p]),
    "tl_moe_gate_up_swiglu": (_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64,
                                     _i64, _i64, _i64, _i64, _c_void_p, _c_void_p]),
    "tl_moe_down_combine": (_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                   _i64, _i64, _i64, _i64, _i64, _i64, _c_void_p, _c_void_p]),
    "tl_moe_route": (_int, [_c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, _c_void_p,
                            _c_void_p, _c_void_p]),
    "tl_expert_select_up_gate_silu": (_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64,
                                             _i64, _i64, ctypes.c_float, _i64, _i64, _c_void_p, _c_void_p,
                                             _c_void_p, _c_void_p]),
    "tl_expert_down_allreduce": (_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64,
                                        _i64, _i64, _i64, _i64, _c_void_p, _c_void_p]),
    "tl_rmsnorm_up_gate_silu": (_int, [_c_void_p, _c_void_p, ctypes.c_float, _c_void_p, _c_void_p, _i64, _i64,
                                       _i64, _i64, _c_void_p, _c_void_p]),
    "tl_down_allreduce": (_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _c_void_p,
                                 _c_void_p]),
    "tl_head_gemm_bf16": (_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _c_void_p,
                                 _c_void_p]),
    "tl_projx_wqaki": (_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64,
                              _i64, _c_void_p, _size, _c_void_p]),
    "tl_bf16_gemv": (_int, [_c_void_p, _c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p, _size, _c_void_p]),
    "tl_bf16_gemv_workspace_bytes": (_size, [_i64, _i64, _i64]),
    "tl_rmsnorm_quant": (_int, [_c_void_p, _c_void_p, ctypes.c_float, _i64, _i64, _c_void_p, _c_void_p,
                                _c_void_p, _int, _c_void_p]),
    "tl_indexer_fp8_scores": (_int, [_c_void_p, _c_void_p, _int, _c_void_p, _c_void_p,
                                     _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i64,
                                     _c_void_p]),
    "tl_indexer_fp8_scores_paged": (_int, [_c_void_p, _c_void_p, _int, _c_void_p, _i64,
                                           _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i64,
                                           _c_void_p]),
    "tl_indexer_topk_workspace_bytes": (_size, [_i64, _i64, _i64]),
    "tl_indexer_fp8_topk": (_int, [_c_void_p, _c_void_p, _int, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                   _i64, _i64, _i64, _i64, _i64, _i64, _c_void_p, _c_void_p, _size, _c_void_p]),
    "tl_indexer_bf16_scores": (_int, [_c_void_p, _c_void_p, _c_void_p, ctypes.c_float, _c_void_p, _i64, _i64,
                                      _i64, _i64, _i64, _c_void_p]),
    "tl_indexer_bf16_topk": (_int, [_c_void_p, _c_void_p, _c_void_p, ctypes.c_float, _c_void_p, _i64, _i64,
                                    _i64, _i64, _i64, _i64, _c_void_p, _c_void_p, _size, _c_void_p]),
    "tl_ki_cache_write": (_int, [_c_void_p, _i64, _c_void_p, _i64, _i64, _int, _c_void_p]),
    "tl_layernorm_rope_rotate": (_int, [_c_void_p, _i64, _c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p,
                                        _c_void_p, ctypes.c_float, _c_void_p]),
    "tl_layernorm_rope_rotate_ki": (_int, [_c_void_p, _i64, _c_void_p, _c_void_p, _i64, _c_void_p,
                                           _c_void_p, _c_void_p, ctypes.c_float, _int, _c_void_p]),
    "tl_flash_sparse_mla": (_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                   _i64, _i64, _i64, _i64, ctypes.c_float, _c_void_p, _c_void_p,
                                   _c_void_p, _c_void_p, _c_void_p]),
    "tl_rmsnorm_projq_wqb": (_int, [_c_void_p, _c_void_p, ctypes.c_float, _c_void_p, _c_void_p, _c_void_p,
                                    _c_void_p, _i64, _i64, _i64, _i64, _i64, _c_void_p]),
    "tl_topk_workspace_bytes": (_size, [_i64, _i64, _i64]),
    "tl_topk_rows": (_int, [_c_void_p, _i64, _i64, _i64, _i64, _c_void_p, _c_void_p, _size,
                            _c_void_p]),
}

_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raise RuntimeError if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"tilert_amd: HIP library not found at {LIB_PATH}; build it with "
                "`python -m tilert_amd.build` (there is no CPU fallback)")
        lib = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_LOCAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name, None)
            if fn is None:  # reported by exported_symbols(); raises when called
                continue
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def exported_symbols() -> set[str]:
    """Names from SIGNATURES that the loaded library actually exports."""
    lib = load()
    return {n for n in SIGNATURES if getattr(lib, n, None) is not None}


def call(name: str, *args) -> None:
    """Invoke ``name``; a nonzero status raises RuntimeError(tl_last_error())."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.tl_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed (status {rc}): {msg}")


def query(name: str, *args):
    return getattr(load(), name)(*args)
