"""Gated multi-head attention parameters used by triangle attention.

Same parameter names and shapes as boltz_mlx/layers/triangular_attention/primitives.py:20-38 (linear_q/k/v/o/g,
no biases; c_hidden is the per-head width). The arithmetic runs in the bzpf triangle-attention kernels; this
module only holds the weights.
"""

from __future__ import annotations

import torch

from boltz_mlx_amd.layers.norm import LayerNorm as _LN

Linear = torch.nn.Linear


def LayerNorm(c_in: int, eps: float = 1e-5) -> _LN:  # noqa: N802
    return _LN(c_in, eps=eps)


class Attention(torch.nn.Module):
    def __init__(self, c_q: int, c_k: int, c_v: int, c_hidden: int, no_heads: int, gating: bool = True):
        super().__init__()
        if not gating:
            raise NotImplementedError("triangle attention is always gated")
        self.c_q, self.c_k, self.c_v = c_q, c_k, c_v
        self.c_hidden = c_hidden
        self.no_heads = no_heads
        self.gating = gating
        self.linear_q = torch.nn.Linear(c_q, c_hidden * no_heads, bias=False)
        self.linear_k = torch.nn.Linear(c_k, c_hidden * no_heads, bias=False)
        self.linear_v = torch.nn.Linear(c_v, c_hidden * no_heads, bias=False)
        self.linear_o = torch.nn.Linear(c_hidden * no_heads, c_q, bias=False)
        self.linear_g = torch.nn.Linear(c_q, c_hidden * no_heads, bias=False)
