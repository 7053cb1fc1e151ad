"""Decode-loop engine on MI355X: the reference's ``Engine`` (engine.py:14-183)
without the TVM compile step.

The model runs eagerly on torch's current stream through the HIP kernels of
libmoe_gfx950; the KV cache is ``model.kv_cache.PagedKVCache``; sampling is
the GPU top-p sampler (``attn_sample_top_p``) with the reference's fixed
parameters (temperature 0.7, top_p 0.9, uniform sample 0.5: engine.py:40).
A chat loop drives it exactly as the reference's chat.py does: ``prefill``
(or ``extend``) the prompt, ``sample``, then ``decode`` + ``sample`` per
generated token, ``popn`` to roll the cache back.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

import attn_native as A
from model.config import GPTOssConfig
from model.transformer import GPTOssForCausalLM


class Engine:
    next_seq_id = 0

    def __init__(self, model_path: str | Path | None = None, config: GPTOssConfig | None = None,
                 device: str = "cuda", max_total_seq_len: int | None = None):
        if model_path is not None:
            self.model_path = Path(model_path)
            self.config = config or GPTOssConfig.from_file(self.model_path / "config.json")
        elif config is not None:
            self.model_path, self.config = None, config
        else:
            raise ValueError("give a checkpoint directory or a config")
        self.device = torch.device(device)
        self.model = GPTOssForCausalLM(self.config, device=self.device)
        if self.model_path is not None:
            import weights
            weights.TorchCheckpoint(self.model_path, self.device).load_into(self.model)
        cw = self.config.context_window_size or 40960
        self.paged_kv_cache = self.model.create_paged_kv_cache(
            1, max_total_seq_len or cw, self.config.prefill_chunk_size, 16, self.device)
        self.sample_parameters = {"temperature": 0.7, "top_p": 0.9, "random_seed": 0.5}
        self._sample_ws = A.sample_workspace(1, self.device)
        self._token = torch.zeros(1, dtype=torch.int32, device=self.device)

    # -- sequences (engine.py:109-131) ---------------------------------------------
    def clear_kv_cache(self) -> None:
        self.paged_kv_cache.clear()

    def begin_sequence(self, sliding_window_size: int | None = None,
                       sink_size: int | None = None) -> int:
        seq_id = self.__class__.next_seq_id
        self.__class__.next_seq_id += 1
        self.paged_kv_cache.add_sequence(seq_id)
        sliding_window_size = sliding_window_size or self.config.sliding_window_size
        if sliding_window_size > 0:
            self.paged_kv_cache.enable_sliding_window(seq_id, sliding_window_size, sink_size or 0)
        return seq_id

    def popn(self, seq_id: int, n: int) -> None:
        self.paged_kv_cache.popn(seq_id, n)

    def get_kv_total_seq_len(self) -> int:
        return self.paged_kv_cache.total_sequence_length()

    # -- forward passes (engine.py:133-174) --------------------------------------------
    def _ids(self, input_tokens) -> torch.Tensor:
        if isinstance(input_tokens, torch.Tensor):
            return input_tokens.to(device=self.device, dtype=torch.int32).reshape(-1)
        return torch.from_numpy(np.ascontiguousarray(input_tokens, dtype=np.int32).reshape(-1)).to(
            self.device)

    def _run(self, fn, input_tokens, sequence_id: int) -> torch.Tensor:
        ids = self._ids(input_tokens)
        embed = self.model.embed(ids)
        self.paged_kv_cache.begin_forward([sequence_id], [ids.numel()])
        try:
            return fn(embed, self.paged_kv_cache)
        finally:
            self.paged_kv_cache.end_forward()

    @torch.no_grad()
    def prefill(self, input_tokens, sequence_id: int = 0) -> torch.Tensor:
        return self._run(self.model.prefill, input_tokens, sequence_id)

    @torch.no_grad()
    def decode(self, input_tokens, sequence_id: int = 0) -> torch.Tensor:
        return self._run(self.model.decode, input_tokens, sequence_id)

    @torch.no_grad()
    def extend(self, input_tokens, sequence_id: int = 0) -> torch.Tensor:
        return self._run(self.model.extend, input_tokens, sequence_id)

    # -- the decode step in one HIP graph ---------------------------------------------
    def _step_body(self) -> None:
        embed = self.model.embed(self._token)
        lb = self.model.decode_logits_bf16(embed, self.paged_kv_cache)
        self._graph_logits_bf16 = lb
        p = self.sample_parameters
        A.sample_top_p(lb[-1:], p["temperature"], p["top_p"], p["random_seed"], self._sample_ws,
                       self._token)

    @property
    def graph_logits(self) -> torch.Tensor:
        """fp32 logits [1, 1, vocab] of the last captured decode step (its bf16
        logits, converted on request)."""
        return self._graph_logits_bf16.float().view(1, -1, self.config.vocab_size)

    @torch.no_grad()
    def capture_decode(self, sequence_id: int) -> None:
        """Capture one decode step of ``sequence_id`` -- embedding of the last
        sampled token, every layer, final norm, unembedding, sampling into the
        same token buffer -- in a HIP graph (``decode_sample`` replays it).

        Nothing is allocated inside the step: the KV cache's forward tables
        are fixed device buffers refreshed by ``begin_forward`` before each
        replay, every MoE block's workspace is reserved for one token, and the
        decode attention's split count is fixed at the pool's capacity
        (``static_span``).  The workspaces the graph captures are held for the
        life of the model, so a later, longer prefill or extend (which grows
        the eager workspaces) leaves them in place.  The warm-up and capture
        steps are rolled back."""
        c = self.paged_kv_cache
        c.static_span = c.num_pages * 16
        c.reserve_decode(1, c.static_span, for_graph=True)
        for blk in self.model.model.block:
            blk.mlp.reserve(1, for_graph=True)
        token = self._token.clone()  # the warm-up step samples over it
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            c.begin_forward([sequence_id], [1])
            self._step_body()
            c.end_forward()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        c.popn(sequence_id, 1)
        self._token.copy_(token)
        c.begin_forward([sequence_id], [1])
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            self._step_body()
        c.end_forward()
        c.popn(sequence_id, 1)
        self._graph, self._graph_seq = graph, sequence_id

    def decode_sample(self, sequence_id: int) -> torch.Tensor:
        """One captured decode step fed with the last sampled token
        (``sample_device`` / ``sample`` wrote it): the next token, as the
        1-element device tensor the following step reads; its logits are in
        ``graph_logits``."""
        if getattr(self, "_graph", None) is None or self._graph_seq != sequence_id:
            raise RuntimeError(f"capture_decode({sequence_id}) first")
        self.paged_kv_cache.begin_forward([sequence_id], [1])
        self._graph.replay()
        self.paged_kv_cache.end_forward()
        return self._token

    def sample_device(self, logits: torch.Tensor) -> torch.Tensor:
        """The sampled token id as a 1-element int32 device tensor (no host sync).

        The logits are the unembedding's bf16 values in fp32; they go back to
        bf16 exactly for the sampler."""
        p = self.sample_parameters
        lb = logits.reshape(-1, logits.shape[-1])[-1:].to(torch.bfloat16)
        return A.sample_top_p(lb, p["temperature"], p["top_p"], p["random_seed"],
                              self._sample_ws, self._token)

    def sample(self, logits: torch.Tensor) -> int:
        """engine.py:165-167: one token id from the last row of ``logits``."""
        return int(self.sample_device(logits).item())
