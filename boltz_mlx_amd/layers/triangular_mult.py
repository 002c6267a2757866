"""Triangle multiplication (outgoing / incoming) on the bzpf kernels.

Same constructor, parameters and call signature as boltz_mlx/layers/triangular_mult.py:27-65, 190-195
(``TriangleMultiplicationOutgoing(dim)(x, mask, use_kernels=False, xn=None)`` returns the update, not the
residual sum). The computation is three kernels per batch element: projection + gate + mask into channel-major
a|b, the per-channel N x N x N contraction, and the fused tail (norm_out, p_out, g_out gate, residual, next LN).
"""

from __future__ import annotations

import torch

from boltz_mlx_amd import kernels as K
from boltz_mlx_amd.layers.norm import LayerNorm


class _TriangleMultiplication(torch.nn.Module):
    outgoing: bool = True

    def __init__(self, dim: int = 128) -> None:
        super().__init__()
        self.norm_in = LayerNorm(dim, eps=1e-5)
        self.p_in = torch.nn.Linear(dim, 2 * dim, bias=False)
        self.g_in = torch.nn.Linear(dim, 2 * dim, bias=False)
        self.norm_out = LayerNorm(dim)
        self.p_out = torch.nn.Linear(dim, dim, bias=False)
        self.g_out = torch.nn.Linear(dim, dim, bias=False)

    def forward(self, x: torch.Tensor, mask: torch.Tensor, use_kernels: bool = False,
                xn: torch.Tensor | None = None) -> torch.Tensor:
        """x: [B, N, N, D] fp32; mask: [B, N, N]. `use_kernels` is accepted and ignored. xn: norm_in(x) already
        computed, used as the reference uses it (triangular_mult.py:23-29): in f16 mode with B = 1 (fp16
        [1, N, N, D]); otherwise the LayerNorm is computed from x."""
        B, N, M, D = x.shape
        if N != M:
            raise ValueError("triangle multiplication needs a square pair representation")
        out = torch.empty(x.shape, dtype=torch.float32, device=x.device)
        mask = mask.to(torch.float32).contiguous()
        use_xn = xn is not None and B == 1 and K.f16()
        if use_xn and (tuple(xn.shape) != tuple(x.shape) or xn.dtype != K.storage_dtype()):
            raise ValueError(f"xn must be the fp16 norm_in output of shape {tuple(x.shape)}, got "
                             f"{tuple(xn.shape)} {xn.dtype}")
        for b in range(B):
            xb = xn[b].contiguous() if use_xn else self.norm_in.to_storage(x[b])
            self.fused(xb.reshape(N * N, D), mask[b], out[b], accumulate=False)
        return out

    def fused(self, xn: torch.Tensor, mask: torch.Tensor, z: torch.Tensor, accumulate: bool = True,
              next_ln=None):
        """z (+)= self(z) from xn = norm_in(z) ([N*N, D], storage dtype) and mask [N, N] fp32; returns
        next_ln(z_new) in the storage dtype when next_ln is given."""
        N, D = z.shape[0], z.shape[-1]
        kexp = K.TRIMULT_K if K.f16() else 0
        w_pg, w_po, w_go = self.prepare()
        if D != 128:  # the projection and tail kernels are built for 128 channels: GEMMs plus layout kernels
            ab = K.trimul_pack(K.linear(xn, w_pg), mask, 2.0 ** -kexp, not self.outgoing, N)
            o = K.trimul_contract(ab, N)
            del ab
            on = K.layer_norm(K.channels_to_rows(o, N), self.norm_out.weight, self.norm_out.bias,
                              self.norm_out.eps * 2.0 ** (-4 * kexp), out_dtype=K.storage_dtype())
            del o
            z2 = z.view(N * N, D)
            if not accumulate:
                z2.zero_()
            K.linear_gated(on, w_po, K.linear(xn, w_go, out_dtype=torch.float32), z2)
            return None if next_ln is None else next_ln.to_storage(z).reshape(N * N, D)
        ab = K.trimul_proj(xn, w_pg, mask, 2.0 ** -kexp, not self.outgoing, N)
        o = K.trimul_contract(ab, N, K.key_extent(mask, N, not self.outgoing))
        del ab
        return K.trimul_tail(o, self.norm_out, self.norm_out.eps * 2.0 ** (-4 * kexp), w_po, xn, w_go, z,
                             accumulate, next_ln, N)

    def kernel_weights(self):
        """[p_in; g_in] (the projection kernel's 4·128 rows), p_out and g_out (the tail), all in the storage dtype."""
        return (K.KernelWeight("w_pg", ("p_in.weight", "g_in.weight")), K.KernelWeight("w_po", ("p_out.weight",)),
                K.KernelWeight("w_go", ("g_out.weight",)))

    def prepare(self):
        """The kernel weights ([p_in; g_in], p_out, g_out), cached on the module."""
        return tuple(K.kernel_weight(self, n) for n in ("w_pg", "w_po", "w_go"))


class TriangleMultiplicationOutgoing(_TriangleMultiplication):
    outgoing = True


class TriangleMultiplicationIncoming(_TriangleMultiplication):
    outgoing = False
