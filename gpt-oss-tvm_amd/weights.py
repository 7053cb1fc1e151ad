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

Loading is checked before anything is copied: every tensor must exist and
match its parameter's shape and dtype.  Every E8M0 scale byte is accepted, as
the reference accepts it.  Inside [2, 252] the expert matmuls (which feed the
scale bytes to the block-scaled MFMA) use exactly the reference's dequantised
weights (model/mlp.py:297-298, ``exp2(s - 127)``).  Outside it a block that
holds only zeros (every e2m1 code +-0) still contributes exactly zero, except
at s = 255.  A block with a nonzero value can differ:
  * s in {0, 1}: the weights are fp32 subnormals or the smallest normals
    (2^-128 ... 6 x 2^-126), whose products the matrix cores may flush, an
    absolute difference below 2^-120 per product;
  * s in {253, 254}: the weights are 2^125 or more (+-inf in the reference
    for the larger codes), so any dot product that uses them overflows in both;
  * s = 255: +inf in the reference, NaN in the hardware's E8M0.
Such blocks are counted and reported with a RuntimeWarning, not refused.
"""
from __future__ import annotations

import warnings
from pathlib import Path
from typing import Iterable

import torch
from safetensors import safe_open

# Bytes per MXFP4 block: 32 e2m1 values packed in 16 bytes (weights.py:35).
BYTES_PER_BLOCK = 16

# E8M0 scale bytes for which the fused matmuls reproduce the reference exactly.
SCALE_MIN, SCALE_MAX = 2, 252


def blocks_outside_range(blocks: torch.Tensor, scales: torch.Tensor) -> int:
    """MXFP4 blocks ([..., G, 16] u8 codes, [..., G] E8M0 bytes) on which the
    fused matmuls may differ from the reference dequantisation: a scale byte
    outside [SCALE_MIN, SCALE_MAX] on a block with a nonzero value, or 255 on
    any block (0 x inf is NaN in the reference)."""
    out = (scales < SCALE_MIN) | (scales > SCALE_MAX)
    if not bool(out.any()):
        return 0
    nonzero = ((blocks & 0x77) != 0).any(dim=-1)   # e2m1 magnitude bits of both nibbles
    return int((out & (nonzero | (scales == 255))).sum())

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
        first -- presence (KeyError), shape and dtype (ValueError) -- so a
        refused checkpoint leaves the module untouched.  MXFP4 blocks whose
        scale byte lies outside [2, 252] (``blocks_outside_range``) are
        loaded and reported with a RuntimeWarning.
        """
        named = [(prefix + name, p) for name, p in module.named_parameters()]
        srcs = self.load_packed_params(named)
        by_name = dict(zip((n for n, _ in named), srcs))
        for (name, p), src in zip(named, srcs):
            if tuple(src.shape) != tuple(p.shape) or src.dtype != p.dtype:
                raise ValueError(f"{convert_key(name)}: checkpoint has {tuple(src.shape)} "
                                 f"{src.dtype}, parameter is {tuple(p.shape)} {p.dtype}")
        for name, src in by_name.items():
            if name.endswith("weight_scales") and src.numel():
                blocks = by_name.get(name[:-len("scales")] + "blocks")
                bad = blocks_outside_range(blocks, src) if blocks is not None else 0
                if bad:
                    lo, hi = int(src.min()), int(src.max())
                    warnings.warn(
                        f"{convert_key(name)}: {bad} MXFP4 blocks with nonzero values have E8M0 "
                        f"scale bytes outside [{SCALE_MIN}, {SCALE_MAX}] (bytes span [{lo}, {hi}]);"
                        " on them the matmuls may differ from the reference dequantisation "
                        "(model/mlp.py:297-298): flushed subnormal products at 0 and 1, "
                        "overflow at 253 and 254, NaN instead of inf at 255", RuntimeWarning)
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
    times 2^(s-127) is a normal bf16); load_into warns about blocks outside.
    """
    lo, hi = 255, 0
    for name, p in module.named_parameters():
        if name.endswith("weight_scales"):
            lo = min(lo, int(p.min()))
            hi = max(hi, int(p.max()))
    return lo, hi
