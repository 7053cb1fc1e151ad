"""Helpers shared by the GPU parity tests: numpy (oracle) <-> torch device tensors."""
import numpy as np
import torch

from oracle import moe_oracle as O


def bf16_dev(a: np.ndarray) -> torch.Tensor:
    """uint16 bf16 bit patterns -> torch.bfloat16 on cuda:0."""
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).cuda()


def u8_dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).cuda()


def i32_dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).cuda()


def f32_dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


def host_bf16(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def host(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def make_block(p: O.BlockParams, k: int = 4):
    """An MLPBlock holding the oracle's parameters on cuda:0."""
    from model.config import GPTOssConfig
    from model.mlp import MLPBlock
    E, H = p.gate_w.shape
    inter = p.mlp2_blocks.shape[2] * 32
    cfg = GPTOssConfig(num_experts=E, num_experts_per_tok=k, hidden_size=H, intermediate_size=inter)
    blk = MLPBlock(cfg, device="cuda")
    with torch.no_grad():
        blk.norm.weight.copy_(bf16_dev(p.norm_w))
        blk.gate.weight.copy_(bf16_dev(p.gate_w))
        blk.gate.bias.copy_(bf16_dev(p.gate_b))
        blk.mlp1_weight_blocks.copy_(u8_dev(p.mlp1_blocks))
        blk.mlp1_weight_scales.copy_(u8_dev(p.mlp1_scales))
        blk.mlp1_bias.copy_(bf16_dev(p.mlp1_bias))
        blk.mlp2_weight_blocks.copy_(u8_dev(p.mlp2_blocks))
        blk.mlp2_weight_scales.copy_(u8_dev(p.mlp2_scales))
        blk.mlp2_bias.copy_(bf16_dev(p.mlp2_bias))
    return blk


def params_from_npz(z) -> O.BlockParams:
    return O.BlockParams(z["norm_w"], z["gate_w"], z["gate_b"], z["mlp1_blocks"],
                         z["mlp1_scales"], z["mlp1_bias"], z["mlp2_blocks"], z["mlp2_scales"],
                         z["mlp2_bias"])


def norm_rel(a: np.ndarray, b: np.ndarray) -> float:
    """max |a - b| / max |b| (infinity-norm relative error)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))
