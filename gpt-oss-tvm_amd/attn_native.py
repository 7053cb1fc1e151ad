"""ctypes binding of the attention-block entry points of libmoe_gfx950.so
(include/attn_gfx950.h).

Same rules as ``moe_native``: GPU tensors only, dtype / shape / contiguity
checked before anything is launched, torch's current stream, RuntimeError on
a non-zero status, no fallback when the library is missing.
"""
from __future__ import annotations

import ctypes

import torch

import moe_native
from moe_native import _check, _expect, _ptr, _stream

_lib = moe_native.lib()

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_F = ctypes.c_float
_INT = ctypes.c_int
_SZ = ctypes.c_size_t

_SIGS = {
    "attn_rms_norm": ([_P, _I64, _I64, _P, _F, _P, _P], _INT),
    "attn_qkv_rope_append": ([_P, _P, _I64, _P, _P, _P, _F, _P, _I64, _P, _P], _INT),
    "attn_decode_workspace_bytes": ([_I64, _I64], _SZ),
    "attn_decode": ([_P, _I64, _P, _I64, _P, _P, _P, _I64, _I32, _F, _P, _P, _P, _SZ, _P], _INT),
    "attn_prefill": ([_P, _P, _I64, _I64, _P, _I64, _P, _P, _P, _I32, _F, _P, _P, _P], _INT),
    "attn_bias_residual": ([_P, _P, _P, _I64, _I64, _P, _P], _INT),
    "attn_embedding": ([_P, _I64, _P, _I64, _I64, _P, _P], _INT),
    "attn_gemv": ([_P, _I64, _I64, _P, _I64, _P, _F, _P, _P], _INT),
    "attn_gemv_bias_residual": ([_P, _I64, _I64, _P, _I64, _P, _P, _P, _P], _INT),
    "attn_qkv_gemv_rope_append": ([_P, _I64, _I64, _P, _P, _F, _P, _P, _P, _P, _F, _P, _I64, _P,
                                   _P], _INT),
    "attn_sample_workspace_bytes": ([_I64], _SZ),
    "attn_sample_top_p": ([_P, _I64, _I64, _F, _F, _F, _P, _P, _SZ, _P], _INT),
}
for _name, (_args, _ret) in _SIGS.items():
    _fn = getattr(_lib, _name)
    _fn.argtypes = _args
    _fn.restype = _ret

EXPORTED = tuple(_SIGS)

HEAD_DIM, Q_HEADS, KV_HEADS, PAGE = 64, 64, 8, 16
QKV_DIM = HEAD_DIM * (Q_HEADS + 2 * KV_HEADS)


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float, out: torch.Tensor | None = None):
    """[n, H] bf16 -> [n, H] bf16 (nn.RMSNorm, model/attention.py:80)."""
    _expect(x, "x", torch.bfloat16)
    H = x.shape[-1]
    _expect(w, "w", torch.bfloat16, (H,))
    if out is None:
        out = torch.empty_like(x)
    _expect(out, "out", torch.bfloat16, tuple(x.shape))
    n = x.numel() // H
    _check(_lib.attn_rms_norm(_ptr(x), n, H, _ptr(w), eps, _ptr(out), _stream()), "attn_rms_norm")
    return out


def qkv_rope_append(qkv: torch.Tensor, bias: torch.Tensor, positions: torch.Tensor,
                    slots: torch.Tensor, inv_freq: torch.Tensor, concentration: float,
                    kv_cache: torch.Tensor, q_out: torch.Tensor) -> torch.Tensor:
    """qkv [n, 5120] bf16 (matmul output) -> q_out [n, 64, 64]; k, v to the cache."""
    _expect(qkv, "qkv", torch.bfloat16)
    if qkv.dim() != 2 or qkv.shape[1] != QKV_DIM:
        raise ValueError(f"qkv: expected [n, {QKV_DIM}], got {tuple(qkv.shape)}")
    n = qkv.shape[0]
    _expect(bias, "bias", torch.bfloat16, (QKV_DIM,))
    _expect(positions, "positions", torch.int32, (n,))
    _expect(slots, "slots", torch.int32, (n,))
    _expect(inv_freq, "inv_freq", torch.float32, (HEAD_DIM // 2,))
    _expect(kv_cache, "kv_cache", torch.bfloat16)
    if tuple(kv_cache.shape[1:]) != (2, KV_HEADS, PAGE, HEAD_DIM):
        raise ValueError(f"kv_cache: expected [pages, 2, {KV_HEADS}, {PAGE}, {HEAD_DIM}], "
                         f"got {tuple(kv_cache.shape)}")
    _expect(q_out, "q_out", torch.bfloat16, (n, Q_HEADS, HEAD_DIM))
    _check(_lib.attn_qkv_rope_append(_ptr(qkv), _ptr(bias), n, _ptr(positions), _ptr(slots),
                                     _ptr(inv_freq), concentration, _ptr(kv_cache),
                                     kv_cache.shape[0], _ptr(q_out), _stream()),
           "attn_qkv_rope_append")
    return q_out


def decode_workspace_bytes(batch: int, max_span: int) -> int:
    return int(_lib.attn_decode_workspace_bytes(batch, max_span))


def decode_workspace(batch: int, max_span: int, device="cuda") -> torch.Tensor:
    """A zeroed attn_decode workspace (its arrival counts must be zero before
    the first call; every call leaves them zero)."""
    return torch.zeros(max(decode_workspace_bytes(batch, max_span), 256), dtype=torch.uint8,
                       device=device)


def _tables(kv_cache, page_indptr, page_indices, kv_len, batch):
    _expect(kv_cache, "kv_cache", torch.bfloat16)
    _expect(page_indptr, "page_indptr", torch.int32, (batch + 1,))
    _expect(page_indices, "page_indices", torch.int32)
    _expect(kv_len, "kv_len", torch.int32, (batch,))


def decode(q: torch.Tensor, kv_cache: torch.Tensor, page_indptr: torch.Tensor,
           page_indices: torch.Tensor, kv_len: torch.Tensor, max_span: int, window: int,
           sm_scale: float, sinks: torch.Tensor, out: torch.Tensor,
           workspace: torch.Tensor) -> torch.Tensor:
    """One query token per sequence over its cached keys (cross_attention);
    ``workspace`` from ``decode_workspace`` (reused across calls)."""
    _expect(q, "q", torch.bfloat16)
    batch = q.shape[0]
    _expect(q, "q", torch.bfloat16, (batch, Q_HEADS, HEAD_DIM))
    _tables(kv_cache, page_indptr, page_indices, kv_len, batch)
    _expect(sinks, "sinks", torch.bfloat16, (Q_HEADS,))
    _expect(out, "out", torch.bfloat16, (batch, Q_HEADS, HEAD_DIM))
    _expect(workspace, "workspace", torch.uint8)
    _check(_lib.attn_decode(_ptr(q), batch, _ptr(kv_cache), kv_cache.shape[0], _ptr(page_indptr),
                            _ptr(page_indices), _ptr(kv_len), max_span, window, sm_scale,
                            _ptr(sinks), _ptr(out), _ptr(workspace), workspace.numel(), _stream()),
           "attn_decode")
    return out


def prefill(q: torch.Tensor, q_indptr: torch.Tensor, max_q_len: int, kv_cache: torch.Tensor,
            page_indptr: torch.Tensor, page_indices: torch.Tensor, kv_len: torch.Tensor,
            window: int, sm_scale: float, sinks: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """Causal (sliding-window) attention of each sequence's new tokens over its cache."""
    _expect(q, "q", torch.bfloat16)
    n = q.shape[0]
    _expect(q, "q", torch.bfloat16, (n, Q_HEADS, HEAD_DIM))
    batch = q_indptr.numel() - 1
    _expect(q_indptr, "q_indptr", torch.int32, (batch + 1,))
    _tables(kv_cache, page_indptr, page_indices, kv_len, batch)
    _expect(sinks, "sinks", torch.bfloat16, (Q_HEADS,))
    _expect(out, "out", torch.bfloat16, (n, Q_HEADS, HEAD_DIM))
    _check(_lib.attn_prefill(_ptr(q), _ptr(q_indptr), batch, max_q_len, _ptr(kv_cache),
                             kv_cache.shape[0], _ptr(page_indptr), _ptr(page_indices),
                             _ptr(kv_len), window, sm_scale, _ptr(sinks), _ptr(out), _stream()),
           "attn_prefill")
    return out


def bias_residual(x: torch.Tensor, y: torch.Tensor, bias: torch.Tensor,
                  out: torch.Tensor | None = None) -> torch.Tensor:
    """bf16(x + bf16(y + bias)) (model/attention.py:254-256)."""
    _expect(x, "x", torch.bfloat16)
    H = x.shape[-1]
    _expect(y, "y", torch.bfloat16, tuple(x.shape))
    _expect(bias, "bias", torch.bfloat16, (H,))
    if out is None:
        out = torch.empty_like(x)
    _expect(out, "out", torch.bfloat16, tuple(x.shape))
    _check(_lib.attn_bias_residual(_ptr(x), _ptr(y), _ptr(bias), x.numel() // H, H, _ptr(out),
                                   _stream()), "attn_bias_residual")
    return out


def embedding(ids: torch.Tensor, table: torch.Tensor, out: torch.Tensor | None = None):
    """ids [n] int32 -> [n, H] rows of table [vocab, H] (nn.Embedding)."""
    _expect(ids, "ids", torch.int32)
    _expect(table, "table", torch.bfloat16)
    vocab, H = table.shape
    n = ids.numel()
    if out is None:
        out = torch.empty((n, H), dtype=torch.bfloat16, device=table.device)
    _expect(out, "out", torch.bfloat16, (n, H))
    _check(_lib.attn_embedding(_ptr(ids), n, _ptr(table), vocab, H, _ptr(out), _stream()),
           "attn_embedding")
    return out


def sample_workspace(batch: int, device="cuda") -> torch.Tensor:
    """A zeroed sampling workspace (each call leaves it zeroed)."""
    return torch.zeros(int(_lib.attn_sample_workspace_bytes(batch)), dtype=torch.uint8,
                       device=device)


def sample_top_p(logits: torch.Tensor, temperature: float, top_p: float, uniform: float,
                 workspace: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """bf16 logits [batch, vocab] -> token ids [batch] int32 (TVM's top-p sampler)."""
    _expect(logits, "logits", torch.bfloat16)
    if logits.dim() == 1:
        logits = logits.view(1, -1)
    batch, vocab = logits.shape
    if out is None:
        out = torch.empty(batch, dtype=torch.int32, device=logits.device)
    _expect(out, "out", torch.int32, (batch,))
    _expect(workspace, "workspace", torch.uint8)
    _check(_lib.attn_sample_top_p(_ptr(logits), batch, vocab, temperature, top_p, uniform,
                                  _ptr(out), _ptr(workspace), workspace.numel(), _stream()),
           "attn_sample_top_p")
    return out


GEMV_MAX_TOKENS = 8


def gemv(x: torch.Tensor, W: torch.Tensor, out: torch.Tensor | None = None,
         norm_w: torch.Tensor | None = None, eps: float = 1e-5) -> torch.Tensor:
    """bf16(t @ W^T) for at most 8 token rows (decode-sized nn.Linear matmul),
    t = x or RMSNorm(x) with weight norm_w."""
    _expect(x, "x", torch.bfloat16)
    _expect(W, "W", torch.bfloat16)
    N, K = W.shape
    M = x.numel() // K
    if norm_w is not None:
        _expect(norm_w, "norm_w", torch.bfloat16, (K,))
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    _expect(out, "out", torch.bfloat16, (M, N))
    _check(_lib.attn_gemv(_ptr(x), M, K, _ptr(W), N, _ptr(norm_w), eps, _ptr(out), _stream()),
           "attn_gemv")
    return out


def gemv_bias_residual(x: torch.Tensor, W: torch.Tensor, bias: torch.Tensor,
                       residual: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """bf16(residual + bf16(bf16(x @ W^T) + bias)) for at most 8 token rows."""
    _expect(x, "x", torch.bfloat16)
    _expect(W, "W", torch.bfloat16)
    N, K = W.shape
    M = x.numel() // K
    _expect(bias, "bias", torch.bfloat16, (N,))
    _expect(residual, "residual", torch.bfloat16)
    if residual.numel() != M * N:
        raise ValueError(f"residual: expected {M * N} elements, got {residual.numel()}")
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    _expect(out, "out", torch.bfloat16)
    _check(_lib.attn_gemv_bias_residual(_ptr(x), M, K, _ptr(W), N, _ptr(bias), _ptr(residual),
                                        _ptr(out), _stream()), "attn_gemv_bias_residual")
    return out


def qkv_gemv_rope_append(x: torch.Tensor, W: torch.Tensor, bias: torch.Tensor,
                         positions: torch.Tensor, slots: torch.Tensor, inv_freq: torch.Tensor,
                         concentration: float, kv_cache: torch.Tensor, q_out: torch.Tensor,
                         norm_w: torch.Tensor | None = None, eps: float = 1e-5) -> torch.Tensor:
    """The decode QKV projection with bias, RoPE and the cache append fused
    (and the block's pre-norm when norm_w is given)."""
    _expect(x, "x", torch.bfloat16)
    _expect(W, "W", torch.bfloat16)
    N, K = W.shape
    if N != QKV_DIM:
        raise ValueError(f"W: expected {QKV_DIM} rows, got {N}")
    M = x.numel() // K
    _expect(bias, "bias", torch.bfloat16, (QKV_DIM,))
    _expect(positions, "positions", torch.int32, (M,))
    _expect(slots, "slots", torch.int32, (M,))
    _expect(inv_freq, "inv_freq", torch.float32, (HEAD_DIM // 2,))
    _expect(kv_cache, "kv_cache", torch.bfloat16)
    _expect(q_out, "q_out", torch.bfloat16, (M, Q_HEADS, HEAD_DIM))
    if norm_w is not None:
        _expect(norm_w, "norm_w", torch.bfloat16, (K,))
    _check(_lib.attn_qkv_gemv_rope_append(_ptr(x), M, K, _ptr(W), _ptr(norm_w), eps, _ptr(bias),
                                          _ptr(positions),
                                          _ptr(slots), _ptr(inv_freq), concentration,
                                          _ptr(kv_cache), kv_cache.shape[0], _ptr(q_out),
                                          _stream()), "attn_qkv_gemv_rope_append")
    return q_out
