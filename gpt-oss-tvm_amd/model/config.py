"""gpt-oss configuration fields read by the MoE block.

Mirrors ``GPTOssConfig`` of the reference (model/config.py:12-38): the same
field names and defaults.  Only the fields the MoE block reads
(model/mlp.py:73-80) affect this package; the others are kept so that a
reference ``config.json`` loads unchanged.  The context-window logic of
model/config.py:56-77 belongs to attention and is not restated.
"""
from __future__ import annotations

import dataclasses
import json
from pathlib import Path
from typing import Any


@dataclasses.dataclass
class GPTOssConfig:
    context_window_size: int = 0
    prefill_chunk_size: int = 8192
    tensor_parallel_shards: int = 1
    pipeline_parallel_stages: int = 1
    dtype: str = "bfloat16"
    kwargs: dict[str, Any] = dataclasses.field(default_factory=dict)

    num_hidden_layers: int = 36
    num_experts: int = 128
    num_experts_per_tok: int = 4
    vocab_size: int = 201088
    hidden_size: int = 2880
    intermediate_size: int = 2880
    head_dim: int = 64
    num_attention_heads: int = 64
    num_key_value_heads: int = 8
    sliding_window_size: int = 128
    rope_theta: int | float = 150000
    rope_scaling: dict | None = None
    swiglu_limit: float = 7.0
    sliding_window_pattern: int = 2

    # gpt-oss config.json spellings of the same fields
    _ALIASES = {"experts_per_token": "num_experts_per_tok"}

    @classmethod
    def from_dict(cls, source: dict[str, Any]) -> "GPTOssConfig":
        names = {f.name for f in dataclasses.fields(cls)}
        known, extra = {}, {}
        for key, value in source.items():
            key = cls._ALIASES.get(key, key)
            (known if key in names and key != "kwargs" else extra)[key] = value
        return cls(**known, kwargs=extra)

    @classmethod
    def from_file(cls, path: str | Path) -> "GPTOssConfig":
        with open(path, encoding="utf-8") as f:
            return cls.from_dict(json.load(f))


def gpt_oss_20b() -> GPTOssConfig:
    """The 20B shape: 24 layers, 32 experts (4)."""
    return GPTOssConfig(num_hidden_layers=24, num_experts=32)


def gpt_oss_120b() -> GPTOssConfig:
    """The 120B shape: 36 layers, 128 experts."""
    return GPTOssConfig(num_hidden_layers=36, num_experts=128)
