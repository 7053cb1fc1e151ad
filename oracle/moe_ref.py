"""ctypes binding of the C restatement (``moe_ref.c``) -- TEST INFRASTRUCTURE ONLY.

Loaded by tests/ and by bench.py's cpu_baseline leg; never by the product path.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libmoe_oracle.so")
_lib = None


def build() -> str:
    """Compile libmoe_oracle.so from moe_ref.c (gcc, no GPU needed)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        i, f = ctypes.c_int, ctypes.c_float
        L.moe_ref_block_forward.argtypes = [P, i, i, i, i, i, P, P, P, P, P, P, P, P, P, f, f, f, i,
                                            P, P, P, P]
        L.moe_ref_block_forward.restype = i
        L.moe_ref_einsum.argtypes = [P, i, P, i, i, i, i, P, P, P, P, i]
        L.moe_ref_einsum.restype = None
        L.moe_ref_swiglu.argtypes = [P, ctypes.c_long, f, f, P]
        L.moe_ref_swiglu.restype = None
        L.moe_ref_gating.argtypes = [P, P, P, i, i, i, P]
        L.moe_ref_gating.restype = None
        L.moe_ref_route.argtypes = [P, i, i, i, i, P, P, P, f, P, P, P]
        L.moe_ref_route.restype = None
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def block_forward(x, p, k=4, eps=1e-5, limit=7.0, alpha=1.702, nthreads=1):
    """Serial (nthreads=1) restatement of MLPBlock.forward; returns (out, t, idx, w)."""
    n, H = x.shape
    E = p.gate_w.shape[0]
    inter = p.mlp2_blocks.shape[2] * 32
    out = np.empty((n, H), np.uint16)
    t = np.empty((n, H), np.uint16)
    idx = np.empty((n, k), np.int32)
    w = np.empty((n, k), np.uint16)
    arrs = [np.ascontiguousarray(a) for a in (x, p.norm_w, p.gate_w, p.gate_b, p.mlp1_blocks,
                                             p.mlp1_scales, p.mlp1_bias, p.mlp2_blocks,
                                             p.mlp2_scales, p.mlp2_bias)]
    rc = lib().moe_ref_block_forward(_p(arrs[0]), n, H, inter, E, k, *[_p(a) for a in arrs[1:]],
                                     eps, limit, alpha, nthreads, _p(out), _p(t), _p(idx), _p(w))
    if rc != 0:
        raise ValueError(f"moe_ref_block_forward failed ({rc})")
    return out, t, idx, w


def einsum(x, idx, blocks, scales, bias, nthreads=1):
    """Serial-order fp32 ``moe_einsum_fused`` (model/mlp.py:238-326)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    n, k = idx.shape
    E, N, G, _ = blocks.shape
    out = np.empty((n, k, N), np.float32)
    lib().moe_ref_einsum(_p(x), int(x.ndim == 3), _p(idx), n, k, N, G * 32,
                         _p(np.ascontiguousarray(blocks)), _p(np.ascontiguousarray(scales)),
                         _p(np.ascontiguousarray(bias)), _p(out), nthreads)
    return out


def swiglu(x, alpha=1.702, limit=7.0):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape[:-1] + (x.shape[-1] // 2,), np.float32)
    lib().moe_ref_swiglu(_p(x), out.size, alpha, limit, _p(out))
    return out


def gating(y, w, x=None):
    y = np.ascontiguousarray(y, dtype=np.float32)
    n, k, N = y.shape
    out = np.empty((n, N), np.uint16)
    xp = _p(np.ascontiguousarray(x)) if x is not None else None
    lib().moe_ref_gating(_p(y), _p(np.ascontiguousarray(w)), xp, n, k, N, _p(out))
    return out


def route(x, p, k=4, eps=1e-5):
    n, H = x.shape
    E = p.gate_w.shape[0]
    t = np.empty((n, H), np.uint16)
    idx = np.empty((n, k), np.int32)
    w = np.empty((n, k), np.uint16)
    lib().moe_ref_route(_p(np.ascontiguousarray(x)), n, H, E, k, _p(p.norm_w), _p(p.gate_w),
                        _p(p.gate_b), eps, _p(t), _p(idx), _p(w))
    return t, idx, w
