"""AttentionPairBias (v2) on the bzpf kernels: the s track's pair-biased attention.

Same constructor, parameters and call signature as boltz_mlx/layers/attentionv2.py:12-86
(``AttentionPairBias(c_s, c_z, num_heads, inf=1e6, compute_pair_bias=True)(s, z, mask, k_in, multiplicity=1,
pair_bias=None)``). proj_z is Sequential(LayerNorm, Linear) as in the PyTorch checkpoint (names proj_z.0.*,
proj_z.1.*); its [N, N, H] -> [H, N, N] rearrangement is folded into the pair-bias kernel's output layout.
"""

from __future__ import annotations

from typing import Optional

import torch

from boltz_mlx_amd import kernels as K
from boltz_mlx_amd.layers.norm import LayerNorm


class AttentionPairBias(torch.nn.Module):
    def __init__(self, c_s: int, c_z: Optional[int] = None, num_heads: Optional[int] = None, inf: float = 1e6,
                 compute_pair_bias: bool = True) -> None:
        super().__init__()
        assert c_s % num_heads == 0
        self.c_s = c_s
        self.num_heads = num_heads
        self.head_dim = c_s // num_heads
        self.inf = inf
        self.proj_q = torch.nn.Linear(c_s, c_s)
        self.proj_k = torch.nn.Linear(c_s, c_s, bias=False)
        self.proj_v = torch.nn.Linear(c_s, c_s, bias=False)
        self.proj_g = torch.nn.Linear(c_s, c_s, bias=False)
        self.compute_pair_bias = compute_pair_bias
        if compute_pair_bias:
            self.proj_z = torch.nn.Sequential(LayerNorm(c_z), torch.nn.Linear(c_z, num_heads, bias=False))
        self.proj_o = torch.nn.Linear(c_s, c_s, bias=False)

    def pair_bias(self, z: torch.Tensor) -> torch.Tensor:
        """proj_z(z) as [H, N, N] in the storage dtype, from z [N, N, c_z] fp32."""
        return K.pair_bias(z, self.proj_z[0], K.wcache(self, "w_z", self.proj_z[1].weight))

    def forward(self, s: torch.Tensor, z: torch.Tensor, mask: torch.Tensor, k_in: torch.Tensor,
                multiplicity: int = 1, pair_bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        """s, k_in: [B, N, c_s]; z: [B, N, N, c_z] fp32 (or, without compute_pair_bias, the bias [B, N, N, H]);
        mask: [B, N]; pair_bias: proj_z(z) already computed as [B, H, N, N]. Returns the update [B, N, c_s] fp32."""
        B, N, _ = s.shape
        out = torch.empty((B, N, self.c_s), dtype=torch.float32, device=s.device)
        dt = K.storage_dtype()
        mask = mask.to(torch.float32).contiguous()
        for b in range(B):
            zb = b // multiplicity
            if pair_bias is not None:
                bias = pair_bias[zb].to(dt).contiguous()
            elif self.compute_pair_bias:
                bias = self.pair_bias(z[zb].contiguous())
            else:
                bias = z[zb].permute(2, 0, 1).to(dt).contiguous()
            self.fused(s[b].to(dt).contiguous(), k_in[b].to(dt).contiguous(), bias, mask[b], out[b],
                       accumulate=False)
        return out

    def fused(self, s: torch.Tensor, k_in: torch.Tensor, bias: torch.Tensor, mask: torch.Tensor, out: torch.Tensor,
              accumulate: bool = True) -> None:
        """out (+)= attention(s, k_in) for one batch element: s, k_in [N, c_s] and bias [H, N, N] in the storage
        dtype, mask [N] fp32, out [N, c_s] fp32."""
        q = K.linear(s, K.wcache(self, "w_q", self.proj_q.weight), bias=self.proj_q.bias)
        k = K.linear(k_in, K.wcache(self, "w_k", self.proj_k.weight))
        v = K.linear(k_in, K.wcache(self, "w_v", self.proj_v.weight))
        g = K.linear(s, K.wcache(self, "w_g", self.proj_g.weight))
        o = K.seq_attention(q, k, v, g, bias, mask, self.inf, self.num_heads)
        K.linear(o, K.wcache(self, "w_o", self.proj_o.weight), out=out, accumulate=accumulate)
