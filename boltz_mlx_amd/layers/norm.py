"""LayerNorm with torch.nn.LayerNorm's parameters, computed by the bzpf LayerNorm kernel.

Mirrors boltz_mlx/layers/norm.py:8-17 (``__call__`` in fp32, ``.f16(x, eps_scale)`` with a fused fp16 cast).
"""

from __future__ import annotations

import torch

from boltz_mlx_amd import kernels as K


class LayerNorm(torch.nn.LayerNorm):
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return K.layer_norm(x, self.weight, self.bias, self.eps)

    def f16(self, x: torch.Tensor, eps_scale: float = 1.0) -> torch.Tensor:
        """Normalised output in fp16 (fp32 statistics). eps_scale multiplies eps: LN(c x) with eps c^2 == LN(x)
        (norm.py:12-17)."""
        return K.layer_norm(x, self.weight, self.bias, self.eps * eps_scale, out_dtype=torch.float16)

    def to_storage(self, x: torch.Tensor) -> torch.Tensor:
        """LN(x) in the pair path's storage dtype (fp32, or fp16 in f16 mode)."""
        return K.layer_norm(x, self.weight, self.bias, self.eps, out_dtype=K.storage_dtype())
