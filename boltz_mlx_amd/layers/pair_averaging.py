"""PairWeightedAveraging on the bzpf kernels: same constructor, parameter names and call signature as
boltz_mlx/layers/pair_averaging.py:10-59 (inference).

  v | g = LN(m) [W_m; W_g]^T                              bzpf_ln_linear_f32 (one kernel; fp32 accuracy)
  logits = LN(z) W_z^T                                      bzpf_pair_bias (fp32 statistics and logits)
  w = softmax_j(logits + (1 - pair_mask) * -inf)            bzpf_pwa_softmax
  o = sigmoid(g) * sum_j w[h, i, j] v[s, j, h]              bzpf_pwa_wsplit + bzpf_pwa_avg (fp32 accuracy on the
                                                            bf16 matrix cores: three exact parts per operand)
  out (+)= o W_o^T                                          bzpf_linear (fp32)
In f16 mode W_z is the fp16 weight copy (upcast; the logits stay fp32) and proj_m / proj_g / proj_o stay fp32, as in
the reference's fused path (pair_averaging.py:61-77).
"""

from __future__ import annotations

import torch

from boltz_mlx_amd import kernels as K
from boltz_mlx_amd.layers.norm import LayerNorm


class PairWeightedAveraging(torch.nn.Module):
    def __init__(self, c_m: int, c_z: int, c_h: int, num_heads: int, inf: float = 1e6) -> None:
        super().__init__()
        if c_h != 32 or c_z != 128:
            raise NotImplementedError("the averaging kernels are built for c_h = 32 and c_z = 128 (the model's)")
        self.c_m, self.c_z, self.c_h, self.num_heads, self.inf = c_m, c_z, c_h, num_heads, inf
        self.norm_m = LayerNorm(c_m)
        self.norm_z = LayerNorm(c_z)
        self.proj_m = torch.nn.Linear(c_m, c_h * num_heads, bias=False)
        self.proj_g = torch.nn.Linear(c_m, c_h * num_heads, bias=False)
        self.proj_z = torch.nn.Linear(c_z, num_heads, bias=False)
        self.proj_o = torch.nn.Linear(c_h * num_heads, c_m, bias=False)

    def kernel_weights(self):
        """[proj_m; proj_g] and proj_o in fp32 (both modes); proj_z in the storage dtype (its fp16 copy is upcast for
        the fp32 logits, as the reference's fused path does)."""
        return (K.KernelWeight("w_mg", ("proj_m.weight", "proj_g.weight"), half=False),
                K.KernelWeight("w_o", ("proj_o.weight",), half=False), K.KernelWeight("w_z", ("proj_z.weight",)))

    def forward(self, m: torch.Tensor, z: torch.Tensor, mask: torch.Tensor, chunk_heads: bool = False) -> torch.Tensor:
        """m [B, S, N, c_m], z [B, N, N, c_z], mask [B, N, N] -> [B, S, N, c_m] fp32 (chunk_heads is ignored)."""
        out = torch.empty(m.shape, dtype=torch.float32, device=m.device)
        for b in range(m.shape[0]):
            self.accumulate(out[b], m[b], z[b], mask[b], accumulate=False)
        return out

    def accumulate(self, out: torch.Tensor, m: torch.Tensor, z: torch.Tensor, pair_mask: torch.Tensor,
                   accumulate: bool = True, resid: torch.Tensor | None = None) -> None:
        """out [S, N, c_m] fp32 contiguous (+)= the layer's output for one MSA m [S, N, c_m] and z [N, N, c_z];
        with resid (fp32 [S, N, c_m], not overlapping out) out = resid + the output instead."""
        S, N, _ = m.shape
        HC = self.c_h * self.num_heads
        w_mg, w_o = K.kernel_weight(self, "w_mg"), K.kernel_weight(self, "w_o")
        w_z = K.kernel_weight(self, "w_z").float()
        m2 = m.reshape(S * N, self.c_m).to(torch.float32)
        if self.c_m == 64 and (2 * HC) % 256 == 0:
            vg = K.ln_linear_f32(m2.contiguous(), self.norm_m, w_mg)
        else:
            vg = K.linear(K.layer_norm(m2, self.norm_m.weight, self.norm_m.bias, self.norm_m.eps), w_mg)
        logits = K.pair_bias(z.to(torch.float32).contiguous(), self.norm_z, w_z)
        w = K.pwa_softmax(logits, pair_mask.to(torch.float32).contiguous(), self.inf)
        og = K.pwa_avg(w, vg[:, :HC], vg[:, HC:], S, N)
        if resid is not None:
            K.linear_residual(og, w_o, resid.reshape(S * N, self.c_m), out.view(S * N, self.c_m))
        else:
            K.linear(og, w_o, out=out.view(S * N, self.c_m), accumulate=accumulate)
