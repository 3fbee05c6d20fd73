"""The C ABI boundary: the library loads, exports every entry point include/tilert_amd.h
declares, and the Python wrappers fail loudly (no CPU fallback).  CPU only."""
import re
import subprocess
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "tilert_amd.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(tl_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_expected_entry_points():
    names = declared_symbols()
    for n in ("tl_act_quant", "tl_fp8_gemm", "tl_fp8_gemm_packed", "tl_moe_gate_up_swiglu",
              "tl_moe_down_combine", "tl_indexer_fp8_scores", "tl_topk_rows", "tl_last_error",
              "tl_layernorm_rope_rotate", "tl_layernorm_rope_rotate_ki"):
        assert n in names


def test_library_exports_every_declared_symbol():
    from tilert_amd import _lib
    lib = _lib.load()
    missing = [n for n in declared_symbols() if getattr(lib, n, None) is None]
    assert not missing, f"not exported: {missing}"
    assert set(declared_symbols()) == set(_lib.SIGNATURES), "ctypes table out of sync with the header"
    assert lib.tl_version().startswith(b"tilert_amd")


def test_nm_shows_extern_c_exports():
    out = subprocess.run(["nm", "-D", "--defined-only", str(ROOT / "tilert_amd" / "libtilert_amd.so")],
                         capture_output=True, text=True).stdout
    for n in declared_symbols():
        assert re.search(rf"\bT {n}$", out, re.M), n


def test_argument_errors_need_no_gpu():
    """Status codes and messages come back through the ABI before any launch."""
    from tilert_amd import _lib
    lib = _lib.load()
    assert lib.tl_fp8_gemm(None, None, None, None, None, 4, 100, 7168, None, 0, None) == 1
    assert b"multiple of 16" in lib.tl_last_error()
    assert lib.tl_fp8_gemm(None, None, None, None, None, 4, 128, 7168, None, 0, None) == 1
    assert b"null pointer" in lib.tl_last_error()
    assert lib.tl_fp8_gemm(None, None, None, None, None, 300, 128, 7168, None, 0, None) == 3
    assert lib.tl_indexer_fp8_scores(None, None, 0, None, None, None, None, 4, 48, 10, 10, 0, None) == 3
    assert lib.tl_topk_rows(None, 4, 131072, 0, 9000, None, None, 0, None) == 3
    assert lib.tl_moe_gate_up_swiglu(None, None, None, None, 17, 8, 0, 32, 7168, 2048, None, None) == 3
    assert lib.tl_act_quant(None, None, None, 4, 100, 128, 0, None) == 1
    assert lib.tl_layernorm_rope_rotate(None, 4, None, None, 8, None, None, None, 1e-6, None) == 1
    assert b"null pointer" in lib.tl_last_error()
    assert lib.tl_layernorm_rope_rotate_ki(None, 0, None, None, 1, None, None, None, 1e-6, 5, None) == 1
    assert lib.tl_fp8_gemm_workspace_bytes(32, 576, 7168) > 0  # narrow layer at M > 16: split K
    # the allocation-free GEMM rejects a shape whose scratch exceeds its static array before
    # touching the device (pointers are only checked for null and alignment)
    assert lib.tl_fp8_gemm_packed_static(256, 256, 256, 256, 256, 64, 16, 655360, None) == 3
    assert b"static maximum" in lib.tl_last_error()
    assert lib.tl_fp8_gemm_workspace_bytes(4, 576, 7168) == 0  # GEMV: never split
    assert lib.tl_fp8_gemm_workspace_bytes(4, 18432, 7168) == 0
    assert lib.tl_fp8_gemm_workspace_bytes(16, 18432, 7168) > 0  # activation image
    # projx_wqkva: q_rank not a multiple of 128, then more than 64 tokens
    assert lib.tl_projx_wqkva(None, None, None, None, None, None, None, None, 1, 4, 128, 7168, 1000, 512, 64, None, 0, None) == 1
    assert lib.tl_projx_wqkva(None, None, None, None, None, None, None, None, 2, 40, 128, 7168, 1536, 512, 64, None, 0, None) == 3


def test_reference_layout_moe_rejects_more_than_one_row_tile():
    """The reference-layout gate/up and down kernels compute one 16-token MFMA tile: M > 16
    must fail before any launch (M = 32 at 2 chunks is within the 64-pair limit)."""
    from tilert_amd import _lib
    lib = _lib.load()
    assert lib.tl_down_allreduce(None, None, None, None, 32, 2, 7168, 256, None, None) == 3
    assert b"> 16 tokens" in lib.tl_last_error()
    assert lib.tl_rmsnorm_up_gate_silu(None, None, 1e-6, None, None, 17, 1, 7168, 256, None, None) == 3
    assert lib.tl_expert_down_allreduce(None, None, None, None, None, None, 32, 256, 1, 7168, 256, None, None) == 3
    assert lib.tl_expert_select_up_gate_silu(None, None, None, None, None, 21, 256, 2, 8, 4, 2.5, 7168, 256,
                                             None, None, None, None) == 3
    # M = 16 passes the shape checks and stops at the null pointers
    assert lib.tl_down_allreduce(None, None, None, None, 16, 2, 7168, 256, None, None) == 1
    assert b"null pointer" in lib.tl_last_error()


def test_routing_with_bias_needs_two_experts_per_group():
    """With a bias a group scores as its two best experts' sum: one-expert groups are rejected
    (the reference's topk(2) over a group would raise); without a bias they are fine."""
    import ctypes
    from tilert_amd import _lib
    lib = _lib.load()
    bias = ctypes.c_void_p(16)  # any non-null value: validation happens before any device access
    assert lib.tl_moe_route(None, bias, 4, 8, 2, 8, 4, 1.0, None, None, None) == 1
    assert b">= 2 experts" in lib.tl_last_error()
    assert lib.tl_moe_route(None, None, 4, 8, 2, 8, 4, 1.0, None, None, None) == 1
    assert b"null pointer" in lib.tl_last_error()


def test_wrappers_reject_cpu_tensors():
    from tilert_amd import kernel as K
    from tilert_amd.topk import topk_accurate
    with pytest.raises(ValueError, match="GPU"):
        K.act_quant(torch.zeros(2, 128, dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        K.act_quant(torch.zeros(2, 128))  # wrong dtype
    with pytest.raises(AssertionError):
        K.act_quant(torch.zeros(2, 100, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="topk must be"):
        topk_accurate(torch.zeros(1, 2, 8), 8, 100)
    # layernorm_rope_rotate keeps the reference op's checks (ops/layernorm_rope_rotate.py:34-56)
    from tilert_amd.layernorm_rope_rotate import layernorm_rope_rotate
    x = torch.zeros(1, 2, 128, dtype=torch.bfloat16)
    pos = torch.zeros(1, dtype=torch.int32)
    cache = torch.zeros(1, 4, 128, dtype=torch.bfloat16)
    w, b, f = torch.ones(128), torch.zeros(128), torch.zeros(2, 1, 64)
    with pytest.raises(ValueError, match="input must be a bfloat16 tensor"):
        layernorm_rope_rotate(x.float(), pos, cache, w, b, f, None, "deepseek_v3_2")
    with pytest.raises(ValueError, match="cur_pos must be a int32 tensor"):
        layernorm_rope_rotate(x, pos.long(), cache, w, b, f, None, "deepseek_v3_2")
    with pytest.raises(ValueError, match="dim must be 128"):
        layernorm_rope_rotate(torch.zeros(1, 2, 64, dtype=torch.bfloat16), pos, cache, w, b, f, None, "deepseek_v3_2")
    with pytest.raises(ValueError, match="batch must be 1"):
        layernorm_rope_rotate(torch.zeros(2, 2, 128, dtype=torch.bfloat16), pos, cache, w, b, f, None, "deepseek_v3_2")
    with pytest.raises(ValueError, match="GPU"):
        layernorm_rope_rotate(x, pos, cache, w, b, f, None, "deepseek_v3_2")


def test_missing_library_fails_loudly(tmp_path):
    code = ("import tilert_amd._lib as l\n"
            "try:\n    l.load()\nexcept RuntimeError as e:\n    print('RAISED', e)\n")
    env = {"TILERT_AMD_LIB": str(tmp_path / "nope.so"), "PATH": "/usr/bin:/bin"}
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, cwd=ROOT, env=env).stdout
    assert "RAISED" in out and "no CPU fallback" in out


def test_bench_refuses_multi_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True)
    assert r.returncode == 2 and "one GPU" in r.stderr
