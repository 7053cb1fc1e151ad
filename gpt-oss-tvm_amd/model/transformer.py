"""gpt-oss transformer around the MoE block: the decode loop's model.

Mirror of the reference's model/transformer.py:13-133: ``TransformerBlock``
(attention block then MoE block, each with its residual), ``Transformer``
(the blocks and the final RMSNorm; the embedding lives here as in the
reference), and ``GPTOssForCausalLM`` with ``embed``, ``prefill`` (logits
of the last token), ``decode`` and ``extend`` over a paged KV cache, and the
unembedding whose bf16 output is returned as fp32 logits (``_get_logits``).
Parameter names follow the reference's modules, so a gpt-oss checkpoint
loads through ``weights.TorchCheckpoint.load_into`` (embedding.weight,
block.N.attn.*, block.N.mlp.*, norm.scale, unembedding.weight).

Every operator is a HIP kernel of libmoe_gfx950; the dense bf16 projections
(QKV, attention output, unembedding) are HIP GEMVs for up to 8 tokens and
library GEMMs for more.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

import attn_native as A

from .attention import AttentionBlock
from .config import GPTOssConfig
from .kv_cache import PagedKVCache
from .mlp import MLPBlock


class _Weight(torch.nn.Module):
    def __init__(self, shape, device, dtype, fill=0.0):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.full(shape, fill, device=device, dtype=dtype),
                                         requires_grad=False)


class TransformerBlock(torch.nn.Module):
    """model/transformer.py:13-31."""

    def __init__(self, config: GPTOssConfig, layer_idx: int, device="cuda"):
        super().__init__()
        self.attn = AttentionBlock(config, layer_idx, device=device)
        self.mlp = MLPBlock(config, device=device)

    def forward(self, x: torch.Tensor, cache: PagedKVCache) -> torch.Tensor:
        x = self.attn(x, cache)
        return self.mlp(x)


class Transformer(torch.nn.Module):
    """model/transformer.py:34-66 (embedding, blocks, final norm)."""

    def __init__(self, config: GPTOssConfig, device="cuda", eps: float = 1e-5):
        super().__init__()
        self.eps = eps
        self.embedding = _Weight((config.vocab_size, config.hidden_size), device, torch.bfloat16)
        self.block = torch.nn.ModuleList(
            [TransformerBlock(config, i, device) for i in range(config.num_hidden_layers)])
        self.norm = _Weight((config.hidden_size,), device, torch.bfloat16, fill=1.0)

    def layers(self, x: torch.Tensor, cache: PagedKVCache) -> torch.Tensor:
        for blk in self.block:
            x = blk(x, cache)
        return x

    def forward(self, x: torch.Tensor, cache: PagedKVCache) -> torch.Tensor:
        x = self.layers(x, cache)
        H = x.shape[-1]
        return A.rms_norm(x.reshape(-1, H), self.norm.weight, self.eps).view(x.shape)


class GPTOssForCausalLM(torch.nn.Module):
    """model/transformer.py:69-133."""

    def __init__(self, config: GPTOssConfig, device="cuda"):
        super().__init__()
        self.config = config
        self.model = Transformer(config, device)
        self.unembedding = _Weight((config.vocab_size, config.hidden_size), device, torch.bfloat16)
        self.hidden_size = config.hidden_size
        self.num_hidden_layers = config.num_hidden_layers
        self.sw_pattern = config.sliding_window_pattern

    def _logits_bf16(self, h: torch.Tensor) -> torch.Tensor:
        h2 = h.reshape(-1, self.hidden_size)
        if h2.shape[0] <= A.GEMV_MAX_TOKENS:  # decode-sized: the GEMV kernel
            return A.gemv(h2.contiguous(), self.unembedding.weight)
        return F.linear(h2, self.unembedding.weight)

    def _get_logits(self, h: torch.Tensor) -> torch.Tensor:
        """bf16 logits of the unembedding, as fp32 (model/transformer.py:95-100)."""
        return self._logits_bf16(h).float()

    def embed(self, input_ids: torch.Tensor) -> torch.Tensor:
        """int32 ids [n] -> [1, n, H] (model/transformer.py:101-105)."""
        return A.embedding(input_ids.to(torch.int32).reshape(-1),
                           self.model.embedding.weight).view(1, -1, self.hidden_size)

    def prefill(self, input_embed: torch.Tensor, cache: PagedKVCache) -> torch.Tensor:
        """Logits [1, 1, vocab] of the last token (model/transformer.py:107-119)."""
        h = self.model(input_embed, cache)
        return self._get_logits(h[:, -1:, :]).view(1, 1, -1)

    def decode_logits_bf16(self, input_embed: torch.Tensor, cache: PagedKVCache) -> torch.Tensor:
        """The unembedding's bf16 logits [b, vocab] of one new token per
        sequence (``decode`` returns them as fp32).  Up to 8 sequences the
        final norm runs inside the unembedding GEMV."""
        if input_embed.numel() // self.hidden_size > A.GEMV_MAX_TOKENS:
            h = self.model(input_embed, cache)
            return self._logits_bf16(h)
        x = self.model.layers(input_embed, cache)
        return A.gemv(x.reshape(-1, self.hidden_size), self.unembedding.weight,
                      norm_w=self.model.norm.weight, eps=self.model.eps)

    def decode(self, input_embed: torch.Tensor, cache: PagedKVCache) -> torch.Tensor:
        """Logits [1, b, vocab] of one new token per sequence (model/transformer.py:121-126)."""
        return self.decode_logits_bf16(input_embed, cache).float().view(1, -1,
                                                                        self.config.vocab_size)

    def extend(self, input_embed: torch.Tensor, cache: PagedKVCache) -> torch.Tensor:
        """Prefill of new tokens over a cached prefix (model/transformer.py:128-140)."""
        return self.prefill(input_embed, cache)

    def create_paged_kv_cache(self, max_batch_size: int, max_total_seq_len: int,
                              prefill_chunk_size: int, page_size: int = 16,
                              device="cuda") -> PagedKVCache:
        """model/transformer.py:153-175: one page pool for every layer."""
        if page_size != 16:
            raise ValueError("the attention kernels use pages of 16 tokens")
        pages = -(-max_total_seq_len // page_size) + max_batch_size
        return PagedKVCache(self.num_hidden_layers, pages, max_batch_size,
                            max(prefill_chunk_size, max_batch_size), device=device)
