"""MSALayer on the bzpf kernels: same constructor, parameter names and call signature as
boltz_mlx/modules/trunkv2.py:205-247 (inference):
  m += PairWeightedAveraging(m, z, pair_mask); m += Transition(m); z += OuterProductMean(m, msa_mask);
  z = PairformerNoSeqLayer(z, pair_mask)
with the residual adds fused into the producing GEMMs' epilogues (fp32 accumulate).
"""

from __future__ import annotations

import torch

from boltz_mlx_amd.layers.outer_product_mean import OuterProductMean
from boltz_mlx_amd.layers.pair_averaging import PairWeightedAveraging
from boltz_mlx_amd.layers.pairformer import PairformerNoSeqLayer
from boltz_mlx_amd.layers.transition import Transition


class MSALayer(torch.nn.Module):
    def __init__(self, msa_s: int, token_z: int, msa_dropout: float = 0.0, z_dropout: float = 0.0,
                 pairwise_head_width: int = 32, pairwise_num_heads: int = 4) -> None:
        super().__init__()
        self.msa_dropout = msa_dropout
        self.msa_transition = Transition(dim=msa_s, hidden=msa_s * 4)
        self.pair_weighted_averaging = PairWeightedAveraging(c_m=msa_s, c_z=token_z, c_h=32, num_heads=8)
        self.pairformer_layer = PairformerNoSeqLayer(token_z=token_z, dropout=z_dropout,
                                                     pairwise_head_width=pairwise_head_width,
                                                     pairwise_num_heads=pairwise_num_heads)
        self.outer_product_mean = OuterProductMean(c_in=msa_s, c_hidden=32, c_out=token_z)

    def forward(self, z: torch.Tensor, m: torch.Tensor, token_mask: torch.Tensor, msa_mask: torch.Tensor,
                **unused) -> tuple[torch.Tensor, torch.Tensor]:
        """z [B, N, N, token_z], m [B, S, N, msa_s], token_mask: the pair mask [B, N, N], msa_mask [B, S, N] ->
        (z, m) fp32. The reference's chunk_* / use_kernels keywords are accepted and ignored."""
        # the first update of each stream is written out of place (input + update), so the inputs are not copied
        z_in = z.to(torch.float32).contiguous()
        m_in = m.to(torch.float32).contiguous()
        z = torch.empty_like(z_in)
        m = torch.empty_like(m_in)
        pm = token_mask.to(torch.float32).contiguous()
        S, N, D = m.shape[1:]
        for b in range(z.shape[0]):
            self.pair_weighted_averaging.accumulate(m[b], m_in[b], z_in[b], pm[b], resid=m_in[b])
            m2 = m[b].view(S * N, D)
            self.msa_transition.inplace(m2)
            self.outer_product_mean.accumulate(z[b], m[b], msa_mask[b], resid=z_in[b])
        self.pairformer_layer.inplace(z, pm)
        return z, m
