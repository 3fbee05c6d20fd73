"""Checkpoint loading (HF safetensors -> one GPU's TP/EP share): slicing on the CPU."""
import pytest
import torch
from safetensors.torch import save_file

from tests import _mini_ckpt as mini
from tilert_amd.checkpoint import Checkpoint


@pytest.fixture(scope="module")
def ckpt_dir(tmp_path_factory):
    d = tmp_path_factory.mktemp("ckpt")
    return str(d), mini.write(str(d))


def test_index_resolves_tensors_across_shards(ckpt_dir):
    path, t = ckpt_dir
    c = Checkpoint(path)
    for name in ("model.layers.3.self_attn.q_a_proj.weight", "model.layers.4.mlp.down_proj.weight_scale_inv"):
        assert name in c
        got = c.get(name)
        assert got.dtype == t[name].dtype and torch.equal(got.view(torch.uint8) if got.dtype == torch.float8_e4m3fn
                                                          else got, t[name].view(torch.uint8)
                                                          if got.dtype == torch.float8_e4m3fn else t[name])


def test_fp8_slices_match_manual_slices_with_their_scale_blocks(ckpt_dir):
    path, t = ckpt_dir
    c = Checkpoint(path)
    p = "model.layers.3.self_attn."
    w, s = c.fp8(p + "q_b_proj", rows=(768, 1536))      # heads 4..7 (rank 1 of 8)
    assert torch.equal(w.view(torch.uint8), t[p + "q_b_proj.weight"][768:1536].view(torch.uint8))
    assert torch.equal(s, t[p + "q_b_proj.weight_scale_inv"][6:12])
    w, s = c.fp8(p + "o_proj", cols=(3584, 4096))       # the last rank's columns
    assert torch.equal(w.view(torch.uint8), t[p + "o_proj.weight"][:, 3584:].view(torch.uint8))
    assert torch.equal(s, t[p + "o_proj.weight_scale_inv"][:, 28:32])
    with pytest.raises(ValueError, match="boundary"):
        c.fp8(p + "q_b_proj", rows=(100, 200))
    with pytest.raises(KeyError):
        c.get("model.layers.9.mlp.gate_proj.weight")


def test_single_file_and_directory_without_index(tmp_path):
    x = torch.arange(12, dtype=torch.float32).reshape(3, 4)
    save_file({"a": x}, str(tmp_path / "one.safetensors"))
    assert torch.equal(Checkpoint(str(tmp_path / "one.safetensors")).get("a", cols=(1, 3)), x[:, 1:3])
    assert torch.equal(Checkpoint(str(tmp_path)).get("a", rows=(1, 2)), x[1:2])
