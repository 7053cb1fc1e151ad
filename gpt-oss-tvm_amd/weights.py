"""Packed MXFP4 weight upload from a gpt-oss safetensors checkpoint.

Mirrors the reference's ``TVMCheckpoint`` (weights.py:70-122): tensors are
read with safetensors straight onto the device, MXFP4 blocks and scales are
kept as uint8 (weights.py:88-89) -- packed, with no bf16 expansion -- and
parameter names are mapped to checkpoint names with the same rules
(weights.py:102-113): drop ``model.``, ``norm.weight`` -> ``norm.scale``,
``weight_blocks`` -> ``weight.blocks``, ``weight_scales`` -> ``weight.scales``.
A layer's MoE parameters live under ``block.{i}.mlp.`` (the reference's
``GPTOssForCausalLM.model.block[i].mlp``, model/transformer.py:41-42, with
``model.`` dropped by the first rule).

Tensors land in torch-ROCm device memory; no DLPack hop is needed because the
kernels take raw device pointers.

Loading is checked before anything is copied: every tensor must exist, match
its parameter's shape and dtype, and every E8M0 scale byte must lie in
[2, 252].  Inside that range the expert matmuls (which feed the scale bytes
to the block-scaled MFMA) give exactly the reference's dequantised weights
(model/mlp.py:297-298, ``exp2(s - 127)``); outside it they do not (s = 255
is +inf in the reference and NaN in the hardware's E8M0; s in {0, 1, 253,
254} reach fp32 subnormals or overflow), so such a checkpoint is refused.
"""
from __future__ import annotations

from pathlib import Path
from typing import Iterable

import torch
from safetensors import safe_open

# Bytes per MXFP4 block: 32 e2m1 values packed in 16 bytes (weights.py:35).
BYTES_PER_BLOCK = 16

# E8M0 scale bytes for which the fused matmuls reproduce the reference exactly.
SCALE_MIN, SCALE_MAX = 2, 252

_RENAMES = (
    ("model.", ""),
    ("norm.weight", "norm.scale"),
    ("weight_blocks", "weight.blocks"),
    ("weight_scales", "weight.scales"),
)


def convert_key(name: str) -> str:
    """Parameter name -> checkpoint name (weights.py:103-113)."""
    for old, new in _RENAMES:
        name = name.replace(old, new)
    return name


def mlp_prefix(layer: int) -> str:
    """Parameter-name prefix of layer ``layer``'s MoE block (before convert_key)."""
    return f"model.block.{layer}.mlp."


class TorchCheckpoint:
    """safetensors -> device tensors, MXFP4 blocks/scales as uint8."""

    def __init__(self, path: str | Path, target_device: str | torch.device = "cuda"):
        self.path = Path(path)
        self.device = torch.device(target_device)
        self.params = self._load_safetensors()

    def _load_safetensors(self) -> dict[str, torch.Tensor]:
        st_path = self.path / "model.safetensors" if self.path.suffix != ".safetensors" else self.path
        if not st_path.exists():
            raise FileNotFoundError(f"safetensor not found: {st_path}")
        params: dict[str, torch.Tensor] = {}
        dev = "cpu" if self.device.type == "cpu" else f"{self.device.type}:{self.device.index or 0}"
        with safe_open(str(st_path), framework="pt", device=dev) as f:
            for name in f.keys():
                t = f.get_tensor(name)
                if "blocks" in name or "scales" in name:
                    t = t.to(torch.uint8)
                params[name] = t
        return params

    def get_tensor(self, name: str) -> torch.Tensor:
        if name not in self.params:
            raise KeyError(f"Tensor {name} not found in checkpoint {self.path}")
        return self.params[name]

    def load_packed_params(self, params: Iterable[tuple[str, object]]) -> list[torch.Tensor]:
        """Checkpoint tensors for (parameter name, parameter) pairs, in order (weights.py:102-122)."""
        return [self.get_tensor(convert_key(name)) for name, _ in params]

    def load_into(self, module: torch.nn.Module, prefix: str = "") -> None:
        """Copy the checkpoint tensors of ``module``'s parameters into them.

        ``prefix`` is prepended to each parameter name before the mapping
        (``mlp_prefix(i)`` for layer i's MoE block).  Everything is validated
        first -- presence (KeyError), shape and dtype (ValueError), the E8M0
        scale range (ValueError) -- so a refused checkpoint leaves the module
        untouched.
        """
        named = [(prefix + name, p) for name, p in module.named_parameters()]
        srcs = self.load_packed_params(named)
        for (name, p), src in zip(named, srcs):
            if tuple(src.shape) != tuple(p.shape) or src.dtype != p.dtype:
                raise ValueError(f"{convert_key(name)}: checkpoint has {tuple(src.shape)} "
                                 f"{src.dtype}, parameter is {tuple(p.shape)} {p.dtype}")
            if name.endswith("weight_scales") and src.numel():
                lo, hi = int(src.min()), int(src.max())
                if lo < SCALE_MIN or hi > SCALE_MAX:
                    raise ValueError(
                        f"{convert_key(name)}: E8M0 scale bytes span [{lo}, {hi}], outside "
                        f"[{SCALE_MIN}, {SCALE_MAX}] where the MXFP4 matmuls reproduce the "
                        "reference dequantisation (model/mlp.py:297-298)")
        with torch.no_grad():
            for (_, p), src in zip(named, srcs):
                p.copy_(src)


def load_mlp_blocks(ckpt: TorchCheckpoint, config, layers: Iterable[int] | None = None,
                    device: str | torch.device | None = None) -> list:
    """One MLPBlock per layer (all ``config.num_hidden_layers`` by default),
    parameters loaded from ``block.{i}.mlp.*`` of the checkpoint."""
    from model.mlp import MLPBlock

    dev = ckpt.device if device is None else torch.device(device)
    out = []
    for i in (range(config.num_hidden_layers) if layers is None else layers):
        blk = MLPBlock(config, device=dev)
        ckpt.load_into(blk, prefix=mlp_prefix(i))
        out.append(blk)
    return out


def scale_range(module: torch.nn.Module) -> tuple[int, int]:
    """(min, max) E8M0 scale byte over a block's MXFP4 weights.

    The fused matmuls dequantise exactly while 2 <= s <= 252 (every e2m1 value
    times 2^(s-127) is a normal bf16); load_into refuses checkpoints outside.
    """
    lo, hi = 255, 0
    for name, p in module.named_parameters():
        if name.endswith("weight_scales"):
            lo = min(lo, int(p.min()))
            hi = max(hi, int(p.max()))
    return lo, hi
