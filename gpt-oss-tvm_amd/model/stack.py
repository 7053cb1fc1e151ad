"""Layers of MoE blocks applied in sequence, ready for graph capture.

The reference runs its layers in a Python loop, ``for block in self.block:
x = block(x)`` (model/transformer.py:59-60), each TransformerBlock applying
attention and then ``self.mlp(x)`` (transformer.py:21-31), i.e.
MLPBlock.forward (model/mlp.py:371-402: RMSNorm -> MoE -> residual add).
MoEStack chains only the MoE half: x <- block_l(x) for l = 0 .. L-1.

A step may carry several token groups (a mixed step: decode tokens and a
prefill chunk), each with its own block per layer -- views that share a
layer's expert weights (MLPBlock.with_gate_bias) -- run layer by layer:
layer l applies its blocks to every group before layer l + 1 starts.

Everything a call needs is allocated by ``reserve``: one block workspace
shared by every call (they run one after another on one stream) and two
activation buffers per group that the layers write in turn.  ``forward``
then allocates nothing and launches only kernels, so a whole step can be
captured in one HIP graph (torch.cuda.CUDAGraph) and replayed.
"""
from __future__ import annotations

import torch

from .mlp import MLPBlock


class MoEStack(torch.nn.Module):
    """layers: one MLPBlock per layer, or one tuple of MLPBlocks (one per token
    group) per layer."""

    def __init__(self, layers):
        super().__init__()
        if not layers:
            raise ValueError("MoEStack needs at least one layer")
        self.layers = [tuple(l) if isinstance(l, (list, tuple)) else (l,) for l in layers]
        self.groups = len(self.layers[0])
        if any(len(l) != self.groups for l in self.layers):
            raise ValueError("every layer needs one block per token group")
        self.blocks = torch.nn.ModuleList([b for l in self.layers for b in l])
        self.hidden_size = self.layers[0][0].hidden_size
        self._n: tuple[int, ...] = ()
        self._ws: torch.Tensor | None = None
        self._bufs: list[torch.Tensor] = []

    def workspace_bytes(self, *ns: int) -> int:
        return max(b.workspace_bytes(n) for l in self.layers for b, n in zip(l, ns))

    def reserve(self, *ns: int) -> None:
        """Allocate for calls of up to ns[g] tokens in group g."""
        if len(ns) != self.groups:
            raise ValueError(f"reserve needs {self.groups} token counts, got {len(ns)}")
        dev = self.layers[0][0].mlp1_weight_blocks.device
        self._ws = torch.zeros(max(self.workspace_bytes(*ns), 256), dtype=torch.uint8, device=dev)
        self._bufs = [torch.empty((2, max(n, 1), self.hidden_size), dtype=torch.bfloat16, device=dev)
                      for n in ns]
        self._n = tuple(ns)

    def forward(self, *xs: torch.Tensor):
        """xs[g]: [b, s, hidden] bf16 with b * s <= the reserved count.  Returns
        the last layer's output per group (a tensor for one group, else a
        tuple): views of internal buffers, valid until the next call."""
        if len(xs) != self.groups:
            raise ValueError(f"forward needs {self.groups} token groups, got {len(xs)}")
        shapes = [x.shape for x in xs]
        cur = []
        for g, x in enumerate(xs):
            b, s, h = x.shape
            if not self._bufs or b * s > self._n[g]:
                raise RuntimeError(f"MoEStack.reserve must cover {b * s} tokens in group {g} "
                                   "before forward")
            cur.append(x.reshape(b * s, h))
        for i, layer in enumerate(self.layers):
            for g, blk in enumerate(layer):
                nxt = self._bufs[g][i & 1, :cur[g].shape[0]]
                blk.forward_into(cur[g], nxt, self._ws)
                cur[g] = nxt
        outs = tuple(c.view(sh) for c, sh in zip(cur, shapes))
        return outs[0] if self.groups == 1 else outs
