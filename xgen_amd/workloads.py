"""Seeded synthetic inputs for the W8A8 DiT linear configurations.

Shapes are the measured configurations of the path (one SP8 rank's token
share at d=3072): QKV [9216,3072], out-proj [3072,3072], FFN up [12288,3072]
with GELU-tanh, FFN down [3072,12288]; M = 15,624 tokens (5 s clip) or 31,248
(10 s clip); plus a CPU-sized case M=256, K=N=1024.

Draw order from one generator seeded per call: x, outlier channels, W, bias,
AdaLN tables.  x ~ N(0,1) bf16 with round(0.001*K) channels (seeded randperm)
scaled x50; W ~ N(0, 0.02) bf16; bias ~ N(0, 0.01) bf16; AdaLN shift/scale
tables ~ N(0, 0.1) bf16 [T=20, d].
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

D_MODEL = 3072
M_5S = 15624   # 31*48*84 / 8
M_10S = 31248  # 2 * 15624

LINEARS = {
    "qkv": (3 * D_MODEL, D_MODEL),
    "out": (D_MODEL, D_MODEL),
    "ffn_up": (4 * D_MODEL, D_MODEL),
    "ffn_down": (D_MODEL, 4 * D_MODEL),
}


@dataclass
class LinearInputs:
    x: torch.Tensor
    weight: torch.Tensor
    bias: torch.Tensor
    outlier_channels: torch.Tensor


def generator(seed: int, device="cpu") -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def activations(M: int, K: int, g: torch.Generator, device="cpu", outliers: bool = True):
    x = torch.randn((M, K), generator=g, device=device, dtype=torch.float32).to(torch.bfloat16)
    n_out = round(0.001 * K) if outliers else 0
    ids = torch.randperm(K, generator=g, device=device)[:n_out]
    if n_out:
        x[:, ids] = (x[:, ids].float() * 50.0).to(torch.bfloat16)
    return x, ids


def linear_inputs(M: int, K: int, N: int, seed: int = 0, device="cpu", outliers: bool = True) -> LinearInputs:
    g = generator(seed, device)
    x, ids = activations(M, K, g, device, outliers)
    w = (torch.randn((N, K), generator=g, device=device) * 0.02).to(torch.bfloat16)
    b = (torch.randn((N,), generator=g, device=device) * 0.01).to(torch.bfloat16)
    return LinearInputs(x, w, b, ids)


def adaln_tables(rows: int, width: int, g: torch.Generator, device="cpu"):
    shift = (torch.randn((rows, width), generator=g, device=device) * 0.1).to(torch.bfloat16)
    scale = (torch.randn((rows, width), generator=g, device=device) * 0.1).to(torch.bfloat16)
    return shift, scale


def weight(name: str, g: torch.Generator, device="cpu") -> tuple[torch.Tensor, torch.Tensor]:
    N, K = LINEARS[name]
    w = (torch.randn((N, K), generator=g, device=device) * 0.02).to(torch.bfloat16)
    b = (torch.randn((N,), generator=g, device=device) * 0.01).to(torch.bfloat16)
    return w, b


# Head-parallel attention geometry of the FP8 wire codec: 24 heads x 128 (d = 3072), 8 peers.
HEADS, HEAD_DIM, SP_PEERS = 24, 128, 8


def qkv_head_views(fused: torch.Tensor, heads: int = HEADS, head_dim: int = HEAD_DIM, peers: int = SP_PEERS):
    """Q, K, V of a fused [M, 3 * heads * head_dim] projection output as in-place
    [peers, M, 1, heads / peers, head_dim] views (peer p holds heads p*H/P .. (p+1)*H/P - 1)."""
    M = fused.shape[0]
    return tuple(t.unflatten(-1, (peers, heads // peers, head_dim)).reshape(M, 1, peers, heads // peers, head_dim)
                 .permute(2, 0, 1, 3, 4) for t in fused.chunk(3, dim=-1))
