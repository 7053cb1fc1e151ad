"""gpt-oss MXFP4 mixture-of-experts MLP block on MI355X (gfx950).

Drop-in for the reference's ``MLPBlock`` (model/mlp.py:63-402, wired in by
model/transformer.py:10,19,29): same constructor arguments, the same nine
parameters under the same names and checkpoint layout, and ``forward(x)`` on
``x [b, s, hidden]`` bf16 returning ``x + MoE(RMSNorm(x))`` in bf16.  The
reference's operator methods ``run_einsum`` and ``run_gating`` and the
``swiglu`` function keep their names and argument meaning.

Every operator runs as a hand-written HIP kernel of libmoe_gfx950.so through
its C ABI (moe_native); there is no PyTorch or CPU fallback.  The MXFP4
weights stay packed in HBM (uint8 blocks + E8M0 scales) and are dequantised
inside the expert matmuls.
"""
from __future__ import annotations

import torch

import moe_native as _native

from .config import GPTOssConfig

# e2m1 code -> value, model/mlp.py:9-26
FP4_VALUES = [
    +0.0, +0.5, +1.0, +1.5, +2.0, +3.0, +4.0, +6.0,
    -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0,
]

SWIGLU_ALPHA = 1.702


def swiglu(x: torch.Tensor, alpha: float = SWIGLU_ALPHA, limit: float = 7.0,
           out_dtype: str = "float32") -> torch.Tensor:
    """Interleaved clamped SwiGLU (model/mlp.py:29-60).

    Even features are the gate (clamped above at ``limit``), odd features the
    linear part (clamped to [-limit, limit]); out = g * sigmoid(alpha*g) * (l + 1).
    The block calls it with out_dtype "float32" (model/mlp.py:390), the only
    dtype this kernel computes in.
    """
    if out_dtype != "float32":
        raise NotImplementedError("swiglu computes in float32 only (the MoE block's call)")
    return _native.swiglu(x, alpha, limit)


def _dtype(name: str) -> torch.dtype:
    if name != "bfloat16":
        raise NotImplementedError(f"dtype {name!r}: the MoE kernels take bfloat16 activations")
    return torch.bfloat16


class RMSNorm(torch.nn.Module):
    """Parameter holder for the block's norm (``nn.RMSNorm``, model/mlp.py:81-87)."""

    def __init__(self, hidden_size: int, epsilon: float, dtype: torch.dtype, device=None):
        super().__init__()
        self.epsilon = epsilon
        self.weight = torch.nn.Parameter(torch.ones(hidden_size, dtype=dtype, device=device),
                                         requires_grad=False)


class Linear(torch.nn.Module):
    """Parameter holder for the router (``nn.Linear``, model/mlp.py:88-92)."""

    def __init__(self, in_features: int, out_features: int, dtype: torch.dtype, device=None):
        super().__init__()
        self.weight = torch.nn.Parameter(
            torch.zeros(out_features, in_features, dtype=dtype, device=device), requires_grad=False)
        self.bias = torch.nn.Parameter(torch.zeros(out_features, dtype=dtype, device=device),
                                       requires_grad=False)


class MLPBlock(torch.nn.Module):
    """MXFP4 MoE block; parameters in checkpoint layout (model/mlp.py:63-144)."""

    def __init__(self, config: GPTOssConfig, rms_norm_eps: float = 1e-5, dtype: str | None = None,
                 device: str | torch.device = "cuda"):
        super().__init__()
        assert config
        self.config = config
        self.rms_norm_eps = rms_norm_eps
        if dtype is None:
            dtype = config.dtype
        self.dtype = dtype
        tdt = _dtype(dtype)
        self.num_experts = config.num_experts
        self.experts_per_token = config.num_experts_per_tok
        self.swiglu_limit = config.swiglu_limit
        self.world_size = 1
        self.hidden_size = config.hidden_size
        self.intermediate_size = config.intermediate_size
        self.norm = RMSNorm(config.hidden_size, rms_norm_eps, tdt, device)
        self.gate = Linear(config.hidden_size, self.num_experts, tdt, device)
        assert config.intermediate_size % self.world_size == 0

        self.mxfp4_dtype = "uint8"
        self.mxfp4_group_size = config.hidden_size // 32
        self.mxfp4_block_length = 16
        E, H, I = self.num_experts, config.hidden_size, config.intermediate_size // self.world_size

        def packed(*shape, dt=torch.uint8):
            return torch.nn.Parameter(torch.zeros(shape, dtype=dt, device=device),
                                      requires_grad=False)

        self.mlp1_weight_blocks = packed(E, 2 * I, H // 32, 16)
        self.mlp1_weight_scales = packed(E, 2 * I, H // 32)
        self.mlp2_weight_blocks = packed(E, H, I // 32, 16)
        self.mlp2_weight_scales = packed(E, H, I // 32)
        self.mlp1_bias = packed(E, 2 * I, dt=tdt)
        self.mlp2_bias = packed(E, H, dt=tdt)
        self._ws: torch.Tensor | None = None
        self._ws_held: list = []
        self._ws_need: dict = {}  # workspace bytes by token count

    # -- parameters ---------------------------------------------------------

    def packed_params(self) -> dict[str, torch.Tensor]:
        """The nine parameters by reference name (norm.weight is ``norm.scale`` on disk)."""
        return {
            "norm.weight": self.norm.weight, "gate.weight": self.gate.weight,
            "gate.bias": self.gate.bias,
            "mlp1_weight_blocks": self.mlp1_weight_blocks,
            "mlp1_weight_scales": self.mlp1_weight_scales, "mlp1_bias": self.mlp1_bias,
            "mlp2_weight_blocks": self.mlp2_weight_blocks,
            "mlp2_weight_scales": self.mlp2_weight_scales, "mlp2_bias": self.mlp2_bias,
        }

    def with_gate_bias(self, bias: torch.Tensor) -> "MLPBlock":
        """A block that shares every parameter of this one except the router
        bias (``gate.bias`` [E] bf16, copied): a view of the same layer whose
        tokens route differently.  Used to build synthetic workloads whose token
        groups have different routing profiles; allocates only the bias."""
        twin = MLPBlock(self.config, self.rms_norm_eps, self.dtype, device="meta")
        twin.norm.weight = self.norm.weight
        twin.gate.weight = self.gate.weight
        for name in ("mlp1_weight_blocks", "mlp1_weight_scales", "mlp2_weight_blocks",
                     "mlp2_weight_scales", "mlp1_bias", "mlp2_bias"):
            setattr(twin, name, getattr(self, name))
        b = bias.to(device=self.gate.bias.device, dtype=self.gate.bias.dtype)
        if tuple(b.shape) != tuple(self.gate.bias.shape):
            raise ValueError(f"gate bias: expected shape {tuple(self.gate.bias.shape)}")
        twin.gate.bias = torch.nn.Parameter(b.clone().contiguous(), requires_grad=False)
        return twin

    # -- reference operator methods -----------------------------------------

    def run_einsum(self, input_tensor: torch.Tensor, expert_indices: torch.Tensor,
                   weight_blocks: torch.Tensor, weight_scales: torch.Tensor,
                   bias_tensor: torch.Tensor) -> torch.Tensor:
        """Fused MXFP4 expert matmul, fp32 out [n, k, N] (model/mlp.py:238-326).

        input_tensor is bf16 [n, K] (the mlp1 call) or fp32 [n, k, K] (mlp2).
        """
        return _native.einsum_fused(input_tensor, expert_indices, weight_blocks, weight_scales,
                                    bias_tensor)

    def run_gating(self, input_tensor: torch.Tensor, expert_weights: torch.Tensor,
                   out_dtype: str | None = None) -> torch.Tensor:
        """Weighted sum over the k experts, fp32 -> bf16 (model/mlp.py:328-369)."""
        if out_dtype not in (None, self.dtype):
            raise NotImplementedError("run_gating writes the block dtype (bfloat16)")
        return _native.gemv_gating(input_tensor, expert_weights)

    def route(self, x2d: torch.Tensor):
        """norm -> gate -> top-k -> softmax (model/mlp.py:375-382): (t, indices, weights)."""
        return _native.router_topk(x2d, self.norm.weight, self.gate.weight, self.gate.bias,
                                   self.experts_per_token, self.norm.epsilon)

    # -- forward --------------------------------------------------------------

    def workspace_bytes(self, n: int) -> int:
        """Bytes of block workspace a call on n tokens needs (moe_workspace_bytes)."""
        need = self._ws_need.get(n)
        if need is None:
            need = _native.workspace_bytes(n, self.num_experts, self.experts_per_token,
                                           self.hidden_size, self.intermediate_size)
            self._ws_need[n] = need
        return need

    def _workspace(self, n: int, device) -> torch.Tensor:
        need = self.workspace_bytes(n)
        if self._ws is None or self._ws.numel() < need or self._ws.device != device:
            # A buffer that a captured graph holds stays alive in _ws_held;
            # eager calls that need more get a new one.  Zero-filled: the
            # block's counters must start at zero (every call leaves them so).
            self._ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=device)
        return self._ws

    def reserve(self, n: int, for_graph: bool = False) -> None:
        """Size the module's workspace for calls of up to n tokens now, so that
        forward() allocates no workspace later (e.g. under graph capture).

        With ``for_graph`` the buffer is also kept alive for as long as the
        module lives: a graph captured after this call holds its raw address,
        and a later, larger eager call replaces ``_ws`` with a new buffer
        instead of freeing the captured one."""
        ws = self._workspace(n, self.mlp1_weight_blocks.device)
        if for_graph and all(h is not ws for h in self._ws_held):
            self._ws_held.append(ws)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """x [b, s, hidden] bf16 -> x + MoE(RMSNorm(x)) (model/mlp.py:371-402).

        One C call chains router, grouping, mlp1 + SwiGLU, mlp2 and the gated
        combine + residual on the current stream.  The module's workspace is
        reused across calls, so concurrent calls on one module must not overlap.
        """
        b, seq_len, dim = x.shape
        x2 = x.reshape(b * seq_len, dim)
        if not x2.is_contiguous():
            x2 = x2.contiguous()
        ws = self._workspace(x2.shape[0], x2.device)
        out = _native.block_forward(x2, self._param_seq(), self.experts_per_token,
                                    self.norm.epsilon, SWIGLU_ALPHA, self.swiglu_limit, ws)
        return out.reshape(b, seq_len, dim)

    def _param_seq(self) -> tuple:
        """The nine parameters in moe_native.BLOCK_PARAM_NAMES order, read from
        the modules' parameter dicts (attribute lookups on a module cost
        microseconds of host time per call)."""
        p, nm, g = self._parameters, self._modules["norm"]._parameters, \
            self._modules["gate"]._parameters
        return (nm["weight"], g["weight"], g["bias"], p["mlp1_weight_blocks"],
                p["mlp1_weight_scales"], p["mlp1_bias"], p["mlp2_weight_blocks"],
                p["mlp2_weight_scales"], p["mlp2_bias"])

    def forward_into(self, x2d: torch.Tensor, out: torch.Tensor, workspace: torch.Tensor) -> torch.Tensor:
        """forward on x2d [n, hidden] into the caller's ``out`` [n, hidden] with the
        caller's ``workspace`` (uint8, at least workspace_bytes(n), 256-byte
        aligned, zero-filled when allocated: every call leaves its counters at
        zero): nothing is allocated, so the call can be captured in a graph.
        Calls that share a workspace must not overlap (one stream, in order)."""
        n = x2d.shape[0]
        if workspace.numel() < self.workspace_bytes(n):
            raise ValueError(f"workspace: need {self.workspace_bytes(n)} bytes, "
                             f"got {workspace.numel()}")
        return _native.block_forward(x2d, self.packed_params(), self.experts_per_token,
                                     self.norm.epsilon, SWIGLU_ALPHA, self.swiglu_limit,
                                     workspace, out=out)

    def forward_marked(self, x: torch.Tensor, events) -> tuple[torch.Tensor, list[str]]:
        """forward with ``events`` (8 torch.cuda.Event) recorded on the current
        stream around the block's own launches: events[0] before the first,
        events[i] after stage i.  Returns (output, the stage names that
        events[1:] close).  The kernels and results are forward's."""
        b, seq_len, dim = x.shape
        x2 = x.reshape(b * seq_len, dim).contiguous()
        ws = self._workspace(x2.shape[0], x2.device)
        out = torch.empty_like(x2)
        names = _native.block_forward_marked(x2, self.packed_params(), self.experts_per_token,
                                             self.norm.epsilon, SWIGLU_ALPHA, self.swiglu_limit,
                                             ws, out, events)
        return out.reshape(b, seq_len, dim), names[1:]

    def forward_staged(self, x: torch.Tensor, events: dict | None = None,
                       fused_decode: bool = False, pieces_epilogue: bool = False) -> dict:
        """The same chain, one C call per stage, returning every intermediate.

        ``events`` (optional) maps stage names to (start, end) torch.cuda.Event
        pairs recorded around that stage on the current stream; the stages are
        "router", "permute", "pieces_t", "mlp1", "pieces_act", "mlp2", "combine",
        or with ``fused_decode`` (the decode chain in one launch, mlp_decode;
        at most 128 tokens) "mlp_decode" in place of the middle three, and
        "act" is None.  With ``pieces_epilogue`` mlp1 writes act's fp8 pieces
        itself (mlp1_swiglu_pieces, the block's prefill kernels): "pieces_act"
        is then empty and "act" None.
        """
        b, seq_len, dim = x.shape
        n = b * seq_len
        x2 = x.reshape(n, dim).contiguous()
        k = self.experts_per_token

        def rec(name, i):
            if events and name in events:
                events[name][i].record()

        rec("router", 0)
        t, idx, w = self.route(x2)
        rec("router", 1)
        rec("permute", 0)
        perm = _native.permute(idx, self.num_experts)
        rec("permute", 1)
        rec("pieces_t", 0)
        t_pk = _native.quantize_pieces(t, 2)
        rec("pieces_t", 1)
        if fused_decode:
            done = torch.zeros(self.num_experts + 1, dtype=torch.int32, device=x.device)
            rec("mlp_decode", 0)
            y, act_pk = _native.mlp_decode(
                t_pk, n, perm["indptr"], perm["sorted_pairs"], k, self.mlp1_weight_blocks,
                self.mlp1_weight_scales, self.mlp1_bias, self.mlp2_weight_blocks,
                self.mlp2_weight_scales, self.mlp2_bias, SWIGLU_ALPHA, self.swiglu_limit,
                done=done)
            rec("mlp_decode", 1)
            rec("combine", 0)
            out = _native.gemv_gating(y.view(n, k, self.hidden_size), w, x2)
            rec("combine", 1)
            return {"t": t, "idx": idx, "w": w, "perm": perm, "act": None,
                    "act_pieces": act_pk, "y": y, "out": out.reshape(b, seq_len, dim)}
        rec("mlp1", 0)
        if pieces_epilogue:
            act_pk, _ = _native.mlp1_swiglu_pieces(
                t_pk, n, dim, perm["indptr"], perm["sorted_pairs"], k, self.mlp1_weight_blocks,
                self.mlp1_weight_scales, self.mlp1_bias, SWIGLU_ALPHA, self.swiglu_limit)
            act = None
            rec("mlp1", 1)
            rec("pieces_act", 0)
        else:
            act = _native.mlp1_swiglu(t_pk, n, dim, perm["indptr"], perm["sorted_pairs"], k,
                                      self.mlp1_weight_blocks, self.mlp1_weight_scales,
                                      self.mlp1_bias, SWIGLU_ALPHA, self.swiglu_limit)
            rec("mlp1", 1)
            rec("pieces_act", 0)
            act_pk = _native.quantize_pieces(act, 3)
        rec("pieces_act", 1)
        rec("mlp2", 0)
        y = _native.mlp2(act_pk, perm["indptr"], perm["sorted_pairs"], n, k,
                         self.mlp2_weight_blocks, self.mlp2_weight_scales, self.mlp2_bias)
        rec("mlp2", 1)
        rec("combine", 0)
        out = _native.gemv_gating(y.view(n, k, self.hidden_size), w, x2)
        rec("combine", 1)
        return {"t": t, "idx": idx, "w": w, "perm": perm, "act": act, "act_pieces": act_pk,
                "y": y, "out": out.reshape(b, seq_len, dim)}
