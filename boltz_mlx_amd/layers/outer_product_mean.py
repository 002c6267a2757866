"""OuterProductMean on the bzpf kernels: same constructor, parameter names and call signature as
boltz_mlx/layers/outer_product_mean.py:12-50 (inference).

  x = mask * (LN(m) [W_a; W_b]^T) as three bf16 parts      bzpf_opm_ln_split (one kernel, fp32 accuracy)
  num = mask^T mask                                        bzpf_linear (fp32, the pair counts)
  z16 = (sum_s mask_si mask_sj a_si (x) b_sj) / max(num, 1)  bzpf_opm_outer (fp32-accurate: six bf16 part products
                                                           per product, fp32 sums; fp16 out in f16 mode)
  out (+)= z16 W_o^T + bias                                bzpf_linear (fp16 GEMM in f16 mode, fp32 accumulate)
The outer sum runs over all MSA rows in one kernel per block of token rows i (at most OPM_PAIRS_PER_CHUNK pairs),
as the reference's fused f16 path does (outer_product_mean.py:52-84); the reference's re-associated form for very
few MSA rows (outer_product_mean.py:86-114) computes the same linear map and is not separate here.
"""

from __future__ import annotations

import torch

from boltz_mlx_amd import kernels as K
from boltz_mlx_amd.layers.norm import LayerNorm

OPM_PAIRS_PER_CHUNK = 1 << 20  # (i, j) pairs per outer-sum launch: 2 GiB of fp16 z rows of 1024


class OuterProductMean(torch.nn.Module):
    def __init__(self, c_in: int, c_hidden: int, c_out: int) -> None:
        super().__init__()
        if c_hidden != 32:
            raise NotImplementedError("the outer-sum kernel is built for c_hidden = 32 (the model's value)")
        self.c_hidden = c_hidden
        self.norm = LayerNorm(c_in)
        self.proj_a = torch.nn.Linear(c_in, c_hidden, bias=False)
        self.proj_b = torch.nn.Linear(c_in, c_hidden, bias=False)
        self.proj_o = torch.nn.Linear(c_hidden * c_hidden, c_out)

    def kernel_weights(self):
        """[proj_a; proj_b] in fp32 (the MSA-side projection keeps fp32 in both modes) and proj_o in the storage
        dtype."""
        return (K.KernelWeight("w_ab", ("proj_a.weight", "proj_b.weight"), half=False),
                K.KernelWeight("w_o", ("proj_o.weight",)))

    def forward(self, m: torch.Tensor, mask: torch.Tensor, chunk_size=None) -> torch.Tensor:
        """m [B, S, N, c_in], mask [B, S, N] -> [B, N, N, c_out] fp32. chunk_size is accepted and ignored."""
        B, S, N, _ = m.shape
        out = torch.empty((B, N, N, self.proj_o.out_features), dtype=torch.float32, device=m.device)
        for b in range(B):
            self.accumulate(out[b], m[b], mask[b], accumulate=False)
        return out

    def accumulate(self, z: torch.Tensor, m: torch.Tensor, mask: torch.Tensor, accumulate: bool = True,
                   resid: torch.Tensor | None = None) -> None:
        """z [N, N, c_out] fp32 contiguous (+)= the layer's output for one MSA m [S, N, c_in], mask [S, N]; with
        resid (fp32 [N, N, c_out], not overlapping z) z = resid + the output instead."""
        S, N, c_in = m.shape
        co = self.proj_o.out_features
        w_ab, w_o = K.kernel_weight(self, "w_ab"), K.kernel_weight(self, "w_o")
        mk = mask.to(torch.float32).reshape(S, N).contiguous()
        m3 = m.to(torch.float32).reshape(S, N, c_in)
        if c_in == 64 and self.c_hidden == 32:
            planes = K.opm_ln_split(m3.contiguous(), self.norm, w_ab, mk)
        else:
            mn = K.layer_norm(m3.reshape(S * N, c_in), self.norm.weight, self.norm.bias, self.norm.eps)
            planes = K.opm_split(K.linear(mn, w_ab).view(S, N, 2 * self.c_hidden), mk)
        z2 = z.view(N * N, co)
        num = K.opm_counts(mk)
        step = max(1, min(N, OPM_PAIRS_PER_CHUNK // N))
        for i0 in range(0, N, step):
            n = min(step, N - i0)
            zz = K.opm_outer_planes(planes, num, S, N, i0, n, out_dtype=w_o.dtype)
            if resid is not None:
                r2 = resid.reshape(N * N, co)[i0 * N:(i0 + n) * N]
                K.linear_residual(zz, w_o, r2, z2[i0 * N:(i0 + n) * N], bias=self.proj_o.bias)
            else:
                K.linear(zz, w_o, bias=self.proj_o.bias, out=z2[i0 * N:(i0 + n) * N], accumulate=accumulate)
