"""gpt-oss AttentionBlock on the gfx950 kernels.

Mirror of the reference's ``AttentionBlock`` (model/attention.py:68-256):
the same parameter names and shapes (``sinks`` [64], ``norm.weight`` [H],
``qkv.weight`` [5120, H], ``qkv.bias``, ``out.weight`` [H, 4096],
``out.bias``), the same forward (pre-norm, fused QKV, YaRN RoPE on q and k,
KV append, attention over the paged cache, sink scaling, output projection,
residual) and the alternating sliding window (even layers, attention.py:87).

The dense projections round once to bf16 after fp32 accumulation, as the
reference's matmul, and add their biases as separate bf16 ops (``nn.Linear``'s
second op): for up to 8 tokens (decode) in hand-written GEMV kernels with the
bias, RoPE and cache append (QKV) or the bias and residual (output) fused; for
prefill-sized inputs as library GEMMs (``torch.nn.functional.linear`` without
bias, hipBLASLt) followed by the HIP epilogue kernels.  Everything else runs in the HIP
kernels of libmoe_gfx950 (attn_native): there is no other path.
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

import attn_native as A

from .config import GPTOssConfig
from .kv_cache import PagedKVCache


def yarn_rope_tables(config: GPTOssConfig) -> tuple[np.ndarray, float]:
    """(inv_freq [head_dim / 2] fp32, concentration) of YaRN RoPE
    (model/attention.py:15-66, 103-148), from the config's rope_scaling."""
    rs = config.rope_scaling or {}
    theta = float(rs.get("rope_theta", config.rope_theta))
    factor = float(rs.get("factor", 32.0))
    beta_fast = float(rs.get("beta_fast", 32.0))
    beta_slow = float(rs.get("beta_slow", 1.0))
    orig = int(rs.get("original_max_position_embeddings", 4096))
    dim = config.head_dim
    half = dim // 2

    def corr(rot):  # inverse of the rotation count of a dim (attention.py:15-22)
        return dim * math.log(orig / (rot * 2 * math.pi)) / (2 * math.log(theta))

    low = np.float32(max(corr(beta_fast), 0.0))
    high = np.float32(min(corr(beta_slow), dim - 1))
    if low == high:
        high = np.float32(high + np.float32(0.001))
    one = np.float32(1.0)
    d = np.arange(half)
    power = np.power(np.float32(theta), (d * 2 % dim).astype(np.float32) / np.float32(dim))
    power = power.astype(np.float32)
    extra = (one / power).astype(np.float32)
    inter = (one / (np.float32(factor) * power)).astype(np.float32)
    t = ((d.astype(np.float32) - low) / (high - low)).astype(np.float32)
    keep = (one - np.minimum(np.maximum(t, np.float32(0.0)), one)).astype(np.float32)
    inv_freq = (inter * (one - keep) + extra * keep).astype(np.float32)
    conc = 0.1 * math.log(factor) + 1.0 if factor > 1.0 else 1.0
    return inv_freq, float(np.float32(conc))


class _Norm(torch.nn.Module):
    def __init__(self, hidden: int, device, dtype):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.ones(hidden, device=device, dtype=dtype),
                                         requires_grad=False)


class _Linear(torch.nn.Module):
    def __init__(self, fin: int, fout: int, bias: bool, device, dtype):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.zeros((fout, fin), device=device, dtype=dtype),
                                         requires_grad=False)
        self.bias = (torch.nn.Parameter(torch.zeros(fout, device=device, dtype=dtype),
                                        requires_grad=False) if bias else None)


class AttentionBlock(torch.nn.Module):
    """x [1, n, H] -> x + attention(x) (model/attention.py:182-256)."""

    def __init__(self, config: GPTOssConfig, layer_idx: int = 0, device="cuda",
                 dtype=torch.bfloat16, eps: float = 1e-5):
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.head_dim = config.head_dim
        self.num_attention_heads = config.num_attention_heads
        self.num_key_value_heads = config.num_key_value_heads
        if (self.head_dim, self.num_attention_heads, self.num_key_value_heads) != (
                A.HEAD_DIM, A.Q_HEADS, A.KV_HEADS):
            raise ValueError("the attention kernels are built for head_dim 64, 64 query heads "
                             "and 8 key/value heads (gpt-oss)")
        self.sliding_window = config.sliding_window_size if layer_idx % 2 == 0 else 0
        self.sm_scale = 1.0 / math.sqrt(config.head_dim)
        self.eps = eps
        H = config.hidden_size
        qkv_dim = config.head_dim * (config.num_attention_heads + 2 * config.num_key_value_heads)
        self.sinks = torch.nn.Parameter(torch.zeros(config.num_attention_heads, device=device,
                                                    dtype=dtype), requires_grad=False)
        self.norm = _Norm(H, device, dtype)
        self.qkv = _Linear(H, qkv_dim, True, device, dtype)
        self.out = _Linear(config.head_dim * config.num_attention_heads, H, True, device, dtype)
        inv_freq, self.concentration = yarn_rope_tables(config)
        self.register_buffer("inv_freq", torch.from_numpy(inv_freq).to(device), persistent=False)

    def _window(self, tables) -> int:
        if self.sliding_window <= 0:
            return 0
        w = set(tables.windows)
        if len(w) != 1:
            raise ValueError("sequences of one forward must share the sliding-window setting")
        return min(self.sliding_window, w.pop()) if 0 not in tables.windows else 0

    def forward(self, x: torch.Tensor, cache: PagedKVCache) -> torch.Tensor:
        tables = cache.tables
        if tables is None:
            raise RuntimeError("call cache.begin_forward(...) before the forward")
        H = x.shape[-1]
        x2 = x.reshape(-1, H)
        n = x2.shape[0]
        if n != tables.num_tokens:
            raise ValueError(f"{n} tokens in x, {tables.num_tokens} in the forward's tables")
        q = torch.empty((n, A.Q_HEADS, A.HEAD_DIM), dtype=x.dtype, device=x.device)
        layer = cache.layer(self.layer_idx)
        small = n <= A.GEMV_MAX_TOKENS  # decode-sized: GEMV kernels with fused norm / epilogues
        if small:
            A.qkv_gemv_rope_append(x2, self.qkv.weight, self.qkv.bias, tables.positions,
                                   tables.slots, self.inv_freq, self.concentration, layer, q,
                                   norm_w=self.norm.weight, eps=self.eps)
        else:
            t = A.rms_norm(x2, self.norm.weight, self.eps)
            qkv = F.linear(t, self.qkv.weight)
            A.qkv_rope_append(qkv, self.qkv.bias, tables.positions, tables.slots, self.inv_freq,
                              self.concentration, layer, q)
        o = torch.empty_like(q)
        window = self._window(tables)
        if tables.is_decode:
            span = cache.static_span or tables.max_kv_len
            span = min(span, window) if window > 0 else span
            ws = cache.decode_workspace(tables.batch, span)
            A.decode(q, layer, tables.page_indptr, tables.page_indices, tables.kv_len, span,
                     window, self.sm_scale, self.sinks, o, ws)
        else:
            A.prefill(q, tables.q_indptr, tables.max_q_len, layer, tables.page_indptr,
                      tables.page_indices, tables.kv_len, window, self.sm_scale, self.sinks, o)
        o2 = o.view(n, A.Q_HEADS * A.HEAD_DIM)
        if small:
            return A.gemv_bias_residual(o2, self.out.weight, self.out.bias, x2).view(x.shape)
        y = F.linear(o2, self.out.weight)
        return A.bias_residual(x2, y, self.out.bias).view(x.shape)
