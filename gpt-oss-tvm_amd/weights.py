"""Packed MXFP4 weight upload from a gpt-oss safetensors checkpoint.

Mirrors the reference's ``TVMCheckpoint`` (weights.py:70-122): tensors are
read with safetensors straight onto the device, MXFP4 blocks and scales are
kept as uint8 (weights.py:88-89) -- packed, with no bf16 expansion -- and
parameter names are mapped to checkpoint names with the same rules
(weights.py:102-113): drop ``model.``, ``norm.weight`` -> ``norm.scale``,
``weight_blocks`` -> ``weight.blocks``, ``weight_scales`` -> ``weight.scales``.

Tensors land in torch-ROCm device memory; no DLPack hop is needed because the
kernels take raw device pointers.
"""
from __future__ import annotations

from pathlib import Path
from typing import Iterable

import torch
from safetensors import safe_open

# Bytes per MXFP4 block: 32 e2m1 values packed in 16 bytes (weights.py:35).
BYTES_PER_BLOCK = 16

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
        """Copy the checkpoint tensors of ``module``'s parameters into them (shape/dtype checked)."""
        named = [(prefix + name, p) for name, p in module.named_parameters()]
        for (name, p), src in zip(named, self.load_packed_params(named)):
            if tuple(src.shape) != tuple(p.shape) or src.dtype != p.dtype:
                raise ValueError(f"{name}: checkpoint has {tuple(src.shape)} {src.dtype}, "
                                 f"parameter is {tuple(p.shape)} {p.dtype}")
            with torch.no_grad():
                p.copy_(src)


def scale_range(module: torch.nn.Module) -> tuple[int, int]:
    """(min, max) E8M0 scale byte over a block's MXFP4 weights.

    The fused matmuls dequantise exactly while 2 <= s <= 252 (every e2m1 value
    times 2^(s-127) is a normal bf16); real checkpoints can be checked with this.
    """
    lo, hi = 255, 0
    for name, p in module.named_parameters():
        if name.endswith("weight_scales"):
            lo = min(lo, int(p.min()))
            hi = max(hi, int(p.max()))
    return lo, hi
