"""Checkpoint upload (gpt-oss-tvm_amd/weights.py) on the CPU.

The reference's TVMCheckpoint (weights.py:70-122) reads safetensors, casts
MXFP4 blocks and scales to uint8 and maps parameter names with four rules.
These tests write checkpoint-named safetensors files (the names the real
gpt-oss checkpoint uses: block.N.mlp.mlp1_weight.blocks, norm.scale, ...),
load them into MLPBlocks held in host memory, and cover the error paths:
a missing file or tensor, a shape or dtype mismatch, and E8M0 scale bytes
outside the range the fused matmuls reproduce exactly (loaded, with a
warning that counts the blocks concerned).
"""
import os

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from oracle import moe_oracle as O

E, H, INTER, LAYERS = 4, 64, 64, 3


def _bf16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


def _layer_tensors(layer: int, seed: int) -> dict:
    p = O.make_params(seed, num_experts=E, hidden=H, inter=INTER)
    pre = f"block.{layer}.mlp."
    return {
        pre + "norm.scale": _bf16(p.norm_w), pre + "gate.weight": _bf16(p.gate_w),
        pre + "gate.bias": _bf16(p.gate_b),
        pre + "mlp1_weight.blocks": torch.from_numpy(p.mlp1_blocks),
        pre + "mlp1_weight.scales": torch.from_numpy(p.mlp1_scales),
        pre + "mlp1_bias": _bf16(p.mlp1_bias),
        pre + "mlp2_weight.blocks": torch.from_numpy(p.mlp2_blocks),
        pre + "mlp2_weight.scales": torch.from_numpy(p.mlp2_scales),
        pre + "mlp2_bias": _bf16(p.mlp2_bias),
    }


@pytest.fixture()
def modules():
    import weights as W
    from model.config import GPTOssConfig
    from model.mlp import MLPBlock
    cfg = GPTOssConfig(num_experts=E, hidden_size=H, intermediate_size=INTER,
                       num_hidden_layers=LAYERS)
    return W, cfg, MLPBlock


@pytest.fixture()
def ckpt_dir(tmp_path):
    tensors = {}
    for i in range(LAYERS):
        tensors.update(_layer_tensors(i, 50 + i))
    # an unrelated tensor of the real checkpoint is ignored
    tensors["embedding.weight"] = torch.zeros(8, H, dtype=torch.bfloat16)
    save_file(tensors, os.path.join(tmp_path, "model.safetensors"))
    return tmp_path, tensors


def test_convert_key_rules(modules):
    """weights.py:103-113: the four renames, in order."""
    W, _, _ = modules
    assert W.convert_key("model.block.3.mlp.norm.weight") == "block.3.mlp.norm.scale"
    assert W.convert_key("model.block.0.mlp.mlp1_weight_blocks") == "block.0.mlp.mlp1_weight.blocks"
    assert W.convert_key("model.block.0.mlp.mlp2_weight_scales") == "block.0.mlp.mlp2_weight.scales"
    assert W.convert_key("model.block.0.mlp.gate.weight") == "block.0.mlp.gate.weight"
    assert W.convert_key("model.block.0.mlp.mlp1_bias") == "block.0.mlp.mlp1_bias"
    assert W.mlp_prefix(7) == "model.block.7.mlp."


def test_load_every_layer(modules, ckpt_dir):
    W, cfg, _ = modules
    path, tensors = ckpt_dir
    for where in (path, os.path.join(path, "model.safetensors")):  # directory or file
        ck = W.TorchCheckpoint(where, "cpu")
        blocks = W.load_mlp_blocks(ck, cfg)
        assert len(blocks) == LAYERS
        for i, blk in enumerate(blocks):
            for name, p in blk.named_parameters():
                src = tensors[W.convert_key(W.mlp_prefix(i) + name)]
                assert p.dtype == src.dtype and torch.equal(p.detach(), src), (i, name)
            # packed: blocks stay uint8 [E, 2I, H/32, 16], no bf16 expansion
            assert blk.mlp1_weight_blocks.dtype == torch.uint8
            assert tuple(blk.mlp1_weight_blocks.shape) == (E, 2 * INTER, H // 32, 16)
            assert W.scale_range(blk) == (118, 122)


def test_blocks_cast_to_uint8(modules, tmp_path):
    """weights.py:88-89: blocks and scales stored with another integer dtype
    are cast to uint8 on load (bytes kept)."""
    W, cfg, MLPBlock = modules
    t = _layer_tensors(0, 60)
    t["block.0.mlp.mlp1_weight.blocks"] = t["block.0.mlp.mlp1_weight.blocks"].view(torch.int8)
    save_file(t, os.path.join(tmp_path, "model.safetensors"))
    blk = MLPBlock(cfg, device="cpu")
    W.TorchCheckpoint(tmp_path, "cpu").load_into(blk, prefix=W.mlp_prefix(0))
    ref = _layer_tensors(0, 60)["block.0.mlp.mlp1_weight.blocks"]
    assert torch.equal(blk.mlp1_weight_blocks.detach(), ref)


def test_missing_file_and_tensor(modules, tmp_path, ckpt_dir):
    W, cfg, MLPBlock = modules
    with pytest.raises(FileNotFoundError):
        W.TorchCheckpoint(tmp_path / "nowhere", "cpu")
    path, _ = ckpt_dir
    blk = MLPBlock(cfg, device="cpu")
    with pytest.raises(KeyError, match="block.9.mlp"):
        W.TorchCheckpoint(path, "cpu").load_into(blk, prefix=W.mlp_prefix(9))


@pytest.mark.parametrize("what", ["shape", "dtype"])
def test_shape_and_dtype_mismatch(modules, tmp_path, what):
    W, cfg, MLPBlock = modules
    t = _layer_tensors(0, 61)
    key = "block.0.mlp.mlp2_bias"
    if what == "shape":
        t[key] = t[key][:, :-1].contiguous()
    else:
        t[key] = t[key].float()
    save_file(t, os.path.join(tmp_path, "model.safetensors"))
    blk = MLPBlock(cfg, device="cpu")
    before = blk.gate.weight.detach().clone()
    with pytest.raises(ValueError, match="mlp2_bias"):
        W.TorchCheckpoint(tmp_path, "cpu").load_into(blk, prefix=W.mlp_prefix(0))
    # nothing was copied: validation runs before any parameter changes
    assert torch.equal(blk.gate.weight.detach(), before)


@pytest.mark.parametrize("bad", [0, 1, 253, 254, 255])
def test_scale_bytes_outside_range_loaded_with_warning(modules, tmp_path, bad):
    """Scale bytes where the fused MFMA path and the reference dequant can
    differ (s = 255: +inf in the reference, NaN in E8M0 hardware; 0, 1:
    subnormal weights; 253, 254: overflow) are loaded, as the reference loads
    them, with a warning that counts the blocks."""
    W, cfg, MLPBlock = modules
    t = _layer_tensors(0, 62)
    key = "block.0.mlp.mlp1_weight.scales"
    t[key][1, 2, 1] = bad
    t["block.0.mlp.mlp1_weight.blocks"][1, 2, 1, 0] = 0x21      # the block holds nonzero values
    save_file(t, os.path.join(tmp_path, "model.safetensors"))
    blk = MLPBlock(cfg, device="cpu")
    with pytest.warns(RuntimeWarning, match=r"mlp1_weight.scales: 1 MXFP4 blocks .*outside \[2, 252\]"):
        W.TorchCheckpoint(tmp_path, "cpu").load_into(blk, prefix=W.mlp_prefix(0))
    assert int(blk.mlp1_weight_scales[1, 2, 1]) == bad
    assert torch.equal(blk.mlp1_weight_blocks.detach(), t["block.0.mlp.mlp1_weight.blocks"])


@pytest.mark.parametrize("bad", [0, 1, 253, 254])
def test_zero_blocks_outside_range_are_exact(modules, tmp_path, bad):
    """A block of zeros (codes 0 and 8, +-0) contributes exactly zero at any
    scale byte but 255: no warning."""
    import warnings
    W, cfg, MLPBlock = modules
    t = _layer_tensors(0, 64)
    t["block.0.mlp.mlp2_weight.scales"][3, 5, 0] = bad
    t["block.0.mlp.mlp2_weight.blocks"][3, 5, 0, :] = torch.tensor([0x00, 0x80, 0x08, 0x88] * 4,
                                                                  dtype=torch.uint8)
    save_file(t, os.path.join(tmp_path, "model.safetensors"))
    blk = MLPBlock(cfg, device="cpu")
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        W.TorchCheckpoint(tmp_path, "cpu").load_into(blk, prefix=W.mlp_prefix(0))
    assert W.scale_range(blk)[0 if bad < 2 else 1] == bad
    assert W.blocks_outside_range(blk.mlp2_weight_blocks, blk.mlp2_weight_scales) == 0
    blk.mlp2_weight_scales.data[3, 5, 0] = 255                     # 0 x inf: NaN in the reference
    assert W.blocks_outside_range(blk.mlp2_weight_blocks, blk.mlp2_weight_scales) == 1


@pytest.mark.parametrize("edge", [2, 252])
def test_scale_range_edges_accepted(modules, tmp_path, edge):
    W, cfg, MLPBlock = modules
    t = _layer_tensors(0, 63)
    t["block.0.mlp.mlp2_weight.scales"][0, 0, 0] = edge
    save_file(t, os.path.join(tmp_path, "model.safetensors"))
    blk = MLPBlock(cfg, device="cpu")
    W.TorchCheckpoint(tmp_path, "cpu").load_into(blk, prefix=W.mlp_prefix(0))
    assert edge in W.scale_range(blk)
