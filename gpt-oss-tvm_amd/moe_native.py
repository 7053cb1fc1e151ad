"""ctypes binding of libmoe_gfx950.so (the C ABI declared in include/moe_gfx950.h).

Every wrapper takes torch tensors that already live on the GPU, checks dtype,
shape, device and contiguity the way the reference's ``T.match_buffer`` does
(a mismatch raises before anything is launched), and launches on torch's
current HIP stream.  A non-zero status from the library raises RuntimeError.

There is no fallback: if the library is missing this module raises on import.
"""
from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmoe_gfx950.so")

if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"{LIB_PATH} is missing: build it with `python gpt-oss-tvm_amd/build_native.py` "
        "(or __graft_entry__.build()); the MoE block has no non-HIP fallback")

_lib = ctypes.CDLL(LIB_PATH)

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_F = ctypes.c_float
_INT = ctypes.c_int
_SZ = ctypes.c_size_t

_SIGS = {
    "moe_version": ([], _INT),
    "moe_status_string": ([_INT], ctypes.c_char_p),
    "moe_dequant_mxfp4": ([_P, _P, _P, _I64, _P], _INT),
    "moe_dequant_mxfp4_fast": ([_P, _P, _P, _I64, _P], _INT),
    "moe_router_topk": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _F, _P, _P, _P, _P], _INT),
    "moe_permute": ([_P, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P], _INT),
    "moe_einsum_workspace_bytes": ([_I64, _I64, _I64, _I64, _INT], _SZ),
    "moe_einsum_fused": ([_P, _INT, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _SZ, _P],
                         _INT),
    "moe_pieces_bytes": ([_I64, _I64, _INT], _SZ),
    "moe_quantize_pieces": ([_P, _INT, _I64, _I64, _INT, _P, _P], _INT),
    "moe_mlp1_swiglu": ([_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _F, _F, _P, _P],
                        _INT),
    "moe_mlp1_swiglu_pieces": ([_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _F, _F, _P,
                                _P, _P], _INT),
    "moe_mlp2": ([_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P], _INT),
    "moe_mlp_decode": ([_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _F, _F,
                        _P, _P, _P, _P], _INT),
    "moe_gemv_gating": ([_P, _P, _P, _I64, _I64, _I64, _P, _P], _INT),
    "moe_swiglu": ([_P, _I64, _I64, _F, _F, _P, _P], _INT),
    "moe_workspace_bytes": ([_I64, _I64, _I64, _I64, _I64], _SZ),
    "moe_workspace_layout": ([_I64, _I64, _I64, _I64, _I64, ctypes.POINTER(_SZ)], _INT),
    "moe_block_forward": ([_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                           _F, _F, _F, _P, _P, _SZ, _P], _INT),
    "moe_block_status": ([_P, _I64, _I64, _I64, _I64, _I64, _P], _INT),
    "moe_block_forward_noalloc": ([_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P,
                                   _P, _F, _F, _F, _P, _P], _INT),
    "moe_set_decode_spin_limit": ([_INT], _INT),
    "moe_hbm_read": ([_P, _SZ, _INT, _INT, _P, _P], _INT),
    "moe_block_forward_marked": ([_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P,
                                  _P, _F, _F, _F, _P, _P, _SZ, _P, _INT, _P, _P, _P], _INT),
}

# MOE_STAGE_* of include/moe_gfx950.h
STAGE_NAMES = ("start", "router_logits", "select", "decode", "mlp1", "act_pieces", "mlp2",
               "gating", "router")
for _name, (_args, _ret) in _SIGS.items():
    _fn = getattr(_lib, _name)
    _fn.argtypes = _args
    _fn.restype = _ret

EXPORTED = tuple(_SIGS)


def lib():
    return _lib


def status_string(code: int) -> str:
    return _lib.moe_status_string(code).decode()


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed: {status_string(rc)} ({rc})")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream():
    # (the raw handle of the current stream; the public call builds a Stream
    # object first, a few microseconds of host time per block call)
    if _raw_stream is not None:
        return _raw_stream(torch.cuda.current_device())
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None):
    # plain ints: the argtypes (c_void_p) convert them
    return None if t is None else t.data_ptr()


def _expect(t: torch.Tensor, name: str, dtype: torch.dtype, shape: tuple | None = None) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a torch.Tensor, got {type(t).__name__}")
    if t.dtype != dtype:
        raise TypeError(f"{name}: expected dtype {dtype}, got {t.dtype}")
    if not t.is_cuda:
        raise ValueError(f"{name}: expected a GPU tensor, got device {t.device}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: expected a contiguous tensor")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: expected shape {tuple(shape)}, got {tuple(t.shape)}")


# ---------------------------------------------------------------------------
# Operators (one per C entry point)
# ---------------------------------------------------------------------------

def dequant_mxfp4(blocks: torch.Tensor, scales: torch.Tensor, fast: bool = False) -> torch.Tensor:
    """[..., 16] u8 blocks + [...] u8 scales -> [..., 32] bf16 (model/mlp.py:172-234)."""
    _expect(blocks, "blocks", torch.uint8)
    _expect(scales, "scales", torch.uint8, tuple(blocks.shape[:-1]))
    if blocks.shape[-1] != 16:
        raise ValueError(f"blocks: last dim must be 16, got {blocks.shape[-1]}")
    rows = scales.numel()
    out = torch.empty(tuple(blocks.shape[:-1]) + (32,), dtype=torch.bfloat16, device=blocks.device)
    fn = _lib.moe_dequant_mxfp4_fast if fast else _lib.moe_dequant_mxfp4
    _check(fn(_ptr(blocks), _ptr(scales), _ptr(out), rows, _stream()), "moe_dequant_mxfp4")
    return out


def router_topk(x, norm_w, gate_w, gate_b, k: int, eps: float = 1e-5):
    """x [n, H] -> (t [n, H] bf16, idx [n, k] int32, w [n, k] bf16); model/mlp.py:375-382."""
    n, H = x.shape
    E = gate_w.shape[0]
    _expect(x, "x", torch.bfloat16)
    _expect(norm_w, "norm.weight", torch.bfloat16, (H,))
    _expect(gate_w, "gate.weight", torch.bfloat16, (E, H))
    _expect(gate_b, "gate.bias", torch.bfloat16, (E,))
    t = torch.empty_like(x)
    idx = torch.empty((n, k), dtype=torch.int32, device=x.device)
    w = torch.empty((n, k), dtype=torch.bfloat16, device=x.device)
    _check(_lib.moe_router_topk(_ptr(x), _ptr(norm_w), _ptr(gate_w), _ptr(gate_b), n, H, E, k, eps,
                                _ptr(t), _ptr(idx), _ptr(w), _stream()), "moe_router_topk")
    return t, idx, w


def permute(idx: torch.Tensor, num_experts: int) -> dict:
    """Group (token, slot) pairs by expert; model/mlp_optimized.py:119-148."""
    _expect(idx, "expert_indices", torch.int32)
    n, k = idx.shape
    dev = idx.device
    nk = n * k
    res = {
        "indptr": torch.empty(num_experts + 1, dtype=torch.int32, device=dev),
        "sorted_pairs": torch.empty(nk, dtype=torch.int32, device=dev),
        "token_indices": torch.empty(nk, dtype=torch.int32, device=dev),
        "expert_ids": torch.empty(nk, dtype=torch.int32, device=dev),
        "pair_pos": torch.empty(nk, dtype=torch.int32, device=dev),
    }
    _check(_lib.moe_permute(_ptr(idx), n, k, num_experts, _ptr(res["indptr"]),
                            _ptr(res["sorted_pairs"]), _ptr(res["token_indices"]),
                            _ptr(res["expert_ids"]), _ptr(res["pair_pos"]), _stream()),
           "moe_permute")
    return res


def einsum_fused(x, expert_indices, blocks, scales, bias) -> torch.Tensor:
    """moe_einsum_fused (model/mlp.py:267-326): fp32 out [n, k, N]."""
    _expect(expert_indices, "expert_indices", torch.int32)
    n, k = expert_indices.shape
    E, N, G, _ = blocks.shape
    K = G * 32
    x3 = x.dim() == 3
    if x3:
        _expect(x, "x", torch.float32, (n, k, K))
    else:
        _expect(x, "x", torch.bfloat16, (n, K))
    _expect(blocks, "weight_blocks", torch.uint8, (E, N, G, 16))
    _expect(scales, "weight_scales", torch.uint8, (E, N, G))
    _expect(bias, "bias", torch.bfloat16, (E, N))
    out = torch.empty((n, k, N), dtype=torch.float32, device=x.device)
    wsb = _lib.moe_einsum_workspace_bytes(n, k, E, K, int(x3))
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=x.device)
    _check(_lib.moe_einsum_fused(_ptr(x), int(x3), _ptr(expert_indices), n, k, E, N, K, _ptr(blocks),
                                 _ptr(scales), _ptr(bias), _ptr(out), _ptr(ws), wsb, _stream()),
           "moe_einsum_fused")
    return out


def pieces_bytes(rows: int, K: int, pieces: int) -> int:
    return int(_lib.moe_pieces_bytes(rows, K, pieces))


def quantize_pieces(x: torch.Tensor, pieces: int, packed: torch.Tensor | None = None) -> torch.Tensor:
    """x [rows, K] bf16 or fp32 -> packed fp8 pieces (u8 buffer of pieces_bytes(rows, K, pieces)).

    Layout: q [rows, pieces, ceil(K/128)*128] e4m3 codes, then (256-byte aligned)
    qs [rows, pieces, 4, 28] E8M0 bytes with qs[.., g, c] the scale of block 4c + g.
    """
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"x: expected bfloat16 or float32, got {x.dtype}")
    _expect(x, "x", x.dtype)
    if x.dim() != 2:
        raise ValueError(f"x: expected [rows, K], got shape {tuple(x.shape)}")
    rows, K = x.shape
    nbytes = pieces_bytes(rows, K, pieces)
    if nbytes == 0 and rows > 0:
        raise ValueError(f"quantize_pieces: unsupported K={K} or pieces={pieces}")
    if packed is None:
        packed = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=x.device)
    elif packed.numel() < nbytes:
        raise ValueError(f"packed: need {nbytes} bytes, got {packed.numel()}")
    _check(_lib.moe_quantize_pieces(_ptr(x), int(x.dtype == torch.float32), rows, K, pieces,
                                    _ptr(packed), _stream()), "moe_quantize_pieces")
    return packed


def unpack_pieces(packed: torch.Tensor, rows: int, K: int, pieces: int):
    """Views (q [rows, pieces, Kp] u8, qs [rows, pieces, 4, 28] u8) of a packed buffer."""
    kp = (K + 127) // 128 * 128
    qb = (rows * pieces * kp + 255) // 256 * 256
    q = packed[: rows * pieces * kp].view(rows, pieces, kp)
    qs = packed[qb: qb + rows * pieces * 112].view(rows, pieces, 4, 28)
    return q, qs


def mlp1_swiglu(t_pieces, n, H, indptr, sorted_pairs, k, blocks, scales, bias, alpha, limit,
                act=None):
    """mlp1 + SwiGLU over grouped pairs -> act fp32 [n*k, I] (row = sorted position).

    t_pieces: quantize_pieces(t, 2) of the normalised tokens t [n, H].
    """
    E, N2, G, _ = blocks.shape
    inter = N2 // 2
    _expect(t_pieces, "t_pieces", torch.uint8)
    if t_pieces.numel() < pieces_bytes(n, H, 2):
        raise ValueError("t_pieces: buffer smaller than pieces_bytes(n, H, 2)")
    _expect(blocks, "mlp1_weight_blocks", torch.uint8, (E, 2 * inter, H // 32, 16))
    _expect(scales, "mlp1_weight_scales", torch.uint8, (E, 2 * inter, H // 32))
    _expect(bias, "mlp1_bias", torch.bfloat16, (E, 2 * inter))
    if act is None:
        act = torch.empty((n * k, inter), dtype=torch.float32, device=blocks.device)
    _check(_lib.moe_mlp1_swiglu(_ptr(t_pieces), _ptr(indptr), _ptr(sorted_pairs), n, k, E, H,
                                inter, _ptr(blocks), _ptr(scales), _ptr(bias), alpha, limit,
                                _ptr(act), _stream()), "moe_mlp1_swiglu")
    return act


def mlp1_swiglu_pieces(t_pieces, n, H, indptr, sorted_pairs, k, blocks, scales, bias, alpha,
                       limit, act=None, act_pieces=None):
    """mlp1 + SwiGLU -> act's three fp8 pieces (the block's prefill form).

    Returns (act_pieces, act): act [n*k, I] fp32 is scratch, written only when
    the grouped GEMV runs (fewer than 48 pairs per expert on average).
    """
    E, N2, G, _ = blocks.shape
    inter = N2 // 2
    _expect(t_pieces, "t_pieces", torch.uint8)
    if t_pieces.numel() < pieces_bytes(n, H, 2):
        raise ValueError("t_pieces: buffer smaller than pieces_bytes(n, H, 2)")
    _expect(blocks, "mlp1_weight_blocks", torch.uint8, (E, 2 * inter, H // 32, 16))
    _expect(scales, "mlp1_weight_scales", torch.uint8, (E, 2 * inter, H // 32))
    _expect(bias, "mlp1_bias", torch.bfloat16, (E, 2 * inter))
    if act is None:
        act = torch.empty((n * k, inter), dtype=torch.float32, device=blocks.device)
    if act_pieces is None:
        act_pieces = torch.empty(pieces_bytes(n * k, inter, 3), dtype=torch.uint8,
                                 device=blocks.device)
    _check(_lib.moe_mlp1_swiglu_pieces(_ptr(t_pieces), _ptr(indptr), _ptr(sorted_pairs), n, k, E,
                                       H, inter, _ptr(blocks), _ptr(scales), _ptr(bias), alpha,
                                       limit, _ptr(act), _ptr(act_pieces), _stream()),
           "moe_mlp1_swiglu_pieces")
    return act_pieces, act


def mlp2(act_pieces, indptr, sorted_pairs, n, k, blocks, scales, bias, y=None):
    """mlp2 over grouped pairs -> y fp32 [n*k, H] by pair.

    act_pieces: quantize_pieces(act, 3) of mlp1_swiglu's output (sorted rows).
    """
    E, H, G, _ = blocks.shape
    inter = G * 32
    _expect(act_pieces, "act_pieces", torch.uint8)
    if act_pieces.numel() < pieces_bytes(n * k, inter, 3):
        raise ValueError("act_pieces: buffer smaller than pieces_bytes(n*k, I, 3)")
    _expect(blocks, "mlp2_weight_blocks", torch.uint8, (E, H, G, 16))
    _expect(scales, "mlp2_weight_scales", torch.uint8, (E, H, G))
    _expect(bias, "mlp2_bias", torch.bfloat16, (E, H))
    if y is None:
        y = torch.empty((n * k, H), dtype=torch.float32, device=blocks.device)
    _check(_lib.moe_mlp2(_ptr(act_pieces), _ptr(indptr), _ptr(sorted_pairs), n, k, E, H, inter,
                         _ptr(blocks), _ptr(scales), _ptr(bias), _ptr(y), _stream()), "moe_mlp2")
    return y


def mlp_decode(t_pieces, n, indptr, sorted_pairs, k, w1, s1, b1, w2, s2, b2, alpha, limit,
               act_pieces=None, done=None, y=None):
    """mlp1 + SwiGLU + act pieces + mlp2 in one launch (n <= 128) -> (y, act_pieces).

    Same results as mlp1_swiglu -> quantize_pieces(act, 3) -> mlp2.  Raises
    RuntimeError ("unsupported parameter value") where the launch does not apply.
    done: int32 [E + 1], zero on entry; afterwards done[:E] holds the per-expert
    mlp1 tile counts and done[E] the status word (nonzero: a bounded wait gave
    up and y is incomplete).
    """
    E, N2, G, _ = w1.shape
    inter, H = N2 // 2, G * 32
    _expect(t_pieces, "t_pieces", torch.uint8)
    if t_pieces.numel() < pieces_bytes(n, H, 2):
        raise ValueError("t_pieces: buffer smaller than pieces_bytes(n, H, 2)")
    _expect(w1, "mlp1_weight_blocks", torch.uint8, (E, 2 * inter, H // 32, 16))
    _expect(s1, "mlp1_weight_scales", torch.uint8, (E, 2 * inter, H // 32))
    _expect(b1, "mlp1_bias", torch.bfloat16, (E, 2 * inter))
    _expect(w2, "mlp2_weight_blocks", torch.uint8, (E, H, inter // 32, 16))
    _expect(s2, "mlp2_weight_scales", torch.uint8, (E, H, inter // 32))
    _expect(b2, "mlp2_bias", torch.bfloat16, (E, H))
    dev = w1.device
    if act_pieces is None:
        act_pieces = torch.empty(pieces_bytes(n * k, inter, 3), dtype=torch.uint8, device=dev)
    if done is None:
        done = torch.zeros(E + 1, dtype=torch.int32, device=dev)
    _expect(done, "done", torch.int32, (E + 1,))
    if y is None:
        y = torch.empty((n * k, H), dtype=torch.float32, device=dev)
    _check(_lib.moe_mlp_decode(_ptr(t_pieces), _ptr(indptr), _ptr(sorted_pairs), n, k, E, H,
                               inter, _ptr(w1), _ptr(s1), _ptr(b1), _ptr(w2), _ptr(s2), _ptr(b2),
                               alpha, limit, _ptr(act_pieces), _ptr(done), _ptr(y), _stream()),
           "moe_mlp_decode")
    return y, act_pieces


def gemv_gating(y: torch.Tensor, w: torch.Tensor, x: torch.Tensor | None = None, out=None):
    """moe_gemv_gating (model/mlp.py:340-369) [+ residual, mlp.py:402]."""
    n, k, N = y.shape
    _expect(y, "x", torch.float32)
    _expect(w, "e_weights", torch.bfloat16, (n, k))
    if x is not None:
        _expect(x, "residual", torch.bfloat16, (n, N))
    if out is None:
        out = torch.empty((n, N), dtype=torch.bfloat16, device=y.device)
    _check(_lib.moe_gemv_gating(_ptr(y), _ptr(w), _ptr(x), n, k, N, _ptr(out), _stream()),
           "moe_gemv_gating")
    return out


def swiglu(x: torch.Tensor, alpha: float, limit: float) -> torch.Tensor:
    """Interleaved clamped SwiGLU, fp32 (model/mlp.py:29-60)."""
    _expect(x, "x", torch.float32)
    if x.shape[-1] % 2:
        raise ValueError("swiglu: last dim must be even")
    d = x.shape[-1] // 2
    rows = x.numel() // max(x.shape[-1], 1)
    out = torch.empty(tuple(x.shape[:-1]) + (d,), dtype=torch.float32, device=x.device)
    _check(_lib.moe_swiglu(_ptr(x), rows, d, alpha, limit, _ptr(out), _stream()), "moe_swiglu")
    return out


def workspace_bytes(n, E, k, H, inter) -> int:
    return int(_lib.moe_workspace_bytes(n, E, k, H, inter))


WORKSPACE_REGIONS = ("t", "idx", "w", "indptr", "sorted_pairs", "token_indices", "expert_ids",
                     "pair_pos", "t_pieces", "act", "act_pieces", "y", "logits", "counts", "sync")


def workspace_layout(n, E, k, H, inter) -> list[int]:
    offs = (_SZ * len(WORKSPACE_REGIONS))()
    _check(_lib.moe_workspace_layout(n, E, k, H, inter, offs), "moe_workspace_layout")
    return list(offs)


BLOCK_PARAM_NAMES = ("norm.weight", "gate.weight", "gate.bias", "mlp1_weight_blocks",
                     "mlp1_weight_scales", "mlp1_bias", "mlp2_weight_blocks",
                     "mlp2_weight_scales", "mlp2_bias")


def block_forward(x, params, k, eps, alpha, limit, workspace, out=None):
    """Whole block in one C call (model/mlp.py:371-402).  x [n, H] bf16;
    params: the nine parameters by reference name, or as a sequence in
    BLOCK_PARAM_NAMES order."""
    p = params if isinstance(params, (tuple, list)) else [params[nm] for nm in BLOCK_PARAM_NAMES]
    n, H = x.shape
    E = p[1].shape[0]
    inter = p[6].shape[2] * 32
    _expect(x, "x", torch.bfloat16)
    if out is None:
        out = torch.empty_like(x)
    _expect(out, "out", torch.bfloat16, (n, H))
    _expect(workspace, "workspace", torch.uint8)
    _check(_lib.moe_block_forward(
        x.data_ptr(), n, E, k, H, inter, p[0].data_ptr(), p[1].data_ptr(), p[2].data_ptr(),
        p[3].data_ptr(), p[4].data_ptr(), p[5].data_ptr(), p[6].data_ptr(), p[7].data_ptr(),
        p[8].data_ptr(), eps, alpha, limit, out.data_ptr(), workspace.data_ptr(),
        workspace.numel(), _stream()), "moe_block_forward")
    return out


def block_forward_marked(x, params: dict, k, eps, alpha, limit, workspace, out, events):
    """block_forward with ``events`` (at least 8 torch.cuda.Event) recorded on
    the current stream before the block's first launch and after each of its
    stages.  Returns the stage names the recorded events close, in order:
    events[i - 1] -> events[i] times stage i (i >= 1)."""
    n, H = x.shape
    E = params["gate.weight"].shape[0]
    inter = params["mlp2_weight_blocks"].shape[2] * 32
    _expect(x, "x", torch.bfloat16)
    _expect(out, "out", torch.bfloat16, (n, H))
    _expect(workspace, "workspace", torch.uint8)
    if len(events) < 8:
        raise ValueError("block_forward_marked needs 8 events")
    for ev in events:
        if ev.cuda_event == 0:
            ev.record()          # torch creates its events on first record
    handles = (ctypes.c_void_p * len(events))(*[ev.cuda_event for ev in events])
    stages = (ctypes.c_int32 * 8)()
    used = ctypes.c_int32(0)
    _check(_lib.moe_block_forward_marked(
        _ptr(x), n, E, k, H, inter, _ptr(params["norm.weight"]), _ptr(params["gate.weight"]),
        _ptr(params["gate.bias"]), _ptr(params["mlp1_weight_blocks"]),
        _ptr(params["mlp1_weight_scales"]), _ptr(params["mlp1_bias"]),
        _ptr(params["mlp2_weight_blocks"]), _ptr(params["mlp2_weight_scales"]),
        _ptr(params["mlp2_bias"]), eps, alpha, limit, _ptr(out), _ptr(workspace),
        workspace.numel(), handles, len(events), stages, ctypes.byref(used), _stream()),
        "moe_block_forward_marked")
    return [STAGE_NAMES[stages[i]] for i in range(used.value)]


def block_forward_noalloc(x, params: dict, k, eps, alpha, limit, out):
    """The block with the library's static scratch as workspace (no allocation
    by the library; ``out`` [n, H] bf16 is the caller's).  Same results as
    block_forward."""
    n, H = x.shape
    E = params["gate.weight"].shape[0]
    inter = params["mlp2_weight_blocks"].shape[2] * 32
    _expect(x, "x", torch.bfloat16)
    _expect(out, "out", torch.bfloat16, (n, H))
    _check(_lib.moe_block_forward_noalloc(
        _ptr(x), n, E, k, H, inter, _ptr(params["norm.weight"]), _ptr(params["gate.weight"]),
        _ptr(params["gate.bias"]), _ptr(params["mlp1_weight_blocks"]),
        _ptr(params["mlp1_weight_scales"]), _ptr(params["mlp1_bias"]),
        _ptr(params["mlp2_weight_blocks"]), _ptr(params["mlp2_weight_scales"]),
        _ptr(params["mlp2_bias"]), eps, alpha, limit, _ptr(out), _stream()),
        "moe_block_forward_noalloc")
    return out


def block_status(workspace, n, E, k, H, inter) -> int:
    """Status of the last block_forward on this workspace: 0, or the negative
    MOE_ERR_INCOMPLETE code when its decode launch's bounded wait gave up (its
    outputs are NaN).  Synchronises the current stream."""
    return int(_lib.moe_block_status(_ptr(workspace), n, E, k, H, inter, _stream()))


def set_decode_spin_limit(polls: int) -> int:
    """Bound of the decode launch's wait in polls (negative: the default); returns
    the previous bound.  Tests set 0 to force the reported give-up path."""
    return int(_lib.moe_set_decode_spin_limit(polls))


def hbm_read(src: torch.Tensor, grid: int, unroll: int, sink: torch.Tensor) -> None:
    """Streaming read of every byte of ``src`` (the HBM calibration kernel);
    ``sink`` holds at least ``grid`` int32."""
    if not src.is_cuda or not src.is_contiguous():
        raise ValueError("src: a contiguous device tensor")
    _expect(sink, "sink", torch.int32)
    if sink.numel() < grid:
        raise ValueError(f"sink: need {grid} ints")
    _check(_lib.moe_hbm_read(_ptr(src), src.numel() * src.element_size(), grid, unroll,
                             _ptr(sink), _stream()), "moe_hbm_read")
