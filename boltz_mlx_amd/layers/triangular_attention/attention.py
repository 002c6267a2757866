"""Triangle attention (starting / ending node) on the bzpf kernels.

Same constructor, parameters and call signature as boltz_mlx/layers/triangular_attention/attention.py:12-35,
193-200 (``TriangleAttention(c_in, c_hidden, no_heads, starting=True, inf=1e9)(x, mask=None, chunk_size=None,
use_kernels=False, xn=None, keep_t=False)`` returns the update). Three kernels per batch element: the fused
q|k|v|g|tri-bias projection (reading positions transposed for the ending node), the flash core, and linear_o +
residual (+ next LN) writing back at the un-transposed position.

``xn`` follows the reference's contract (attention.py:95-100): it is used in f16 mode only (the fp32 path computes
the LayerNorm itself), and for the ending node it is the LayerNorm output already transposed, so its projection
reads it in place. Inside the layer chain (``fused``) the carried LayerNorm output stays in the natural layout and
the projection kernel reads the ending node's positions transposed instead.
"""

from __future__ import annotations

from typing import Optional

import torch

from boltz_mlx_amd import kernels as K
from boltz_mlx_amd.layers.triangular_attention.primitives import Attention, LayerNorm


class TriangleAttention(torch.nn.Module):
    def __init__(self, c_in: int, c_hidden: int, no_heads: int, starting: bool = True, inf: float = 1e9) -> None:
        super().__init__()
        self.c_in = c_in
        self.c_hidden = c_hidden
        self.no_heads = no_heads
        self.starting = starting
        self.inf = inf
        self.layer_norm = LayerNorm(c_in)
        self.linear = torch.nn.Linear(c_in, no_heads, bias=False)
        self.mha = Attention(c_in, c_in, c_in, c_hidden, no_heads)

    def forward(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None, chunk_size: Optional[int] = None,
                use_kernels: bool = False, xn: Optional[torch.Tensor] = None, keep_t: bool = False) -> torch.Tensor:
        """x: [B, I, J, C_in] fp32; mask: [B, I, J]. chunk_size / use_kernels are accepted and ignored (the core is
        flash-style and never materialises the logits). xn (f16 mode): layer_norm(x) in fp16, for the ending node
        transposed ([B, J, I, C_in]), as the reference's f16 path takes it; outside f16 mode it is ignored."""
        B, N, M, D = x.shape
        if N != M:
            raise ValueError("triangle attention needs a square pair representation")
        if mask is None:
            mask = torch.ones(x.shape[:-1], dtype=torch.float32, device=x.device)
        mask = mask.to(torch.float32).contiguous()
        out = torch.empty(x.shape, dtype=torch.float32, device=x.device)
        use_xn = xn is not None and K.f16()
        if use_xn and (tuple(xn.shape) != tuple(x.shape) or xn.dtype != K.storage_dtype()):
            raise ValueError(f"xn must be the fp16 layer_norm output of shape {tuple(x.shape)}, got "
                             f"{tuple(xn.shape)} {xn.dtype}")
        for b in range(B):
            xb = xn[b].contiguous() if use_xn else self.layer_norm.to_storage(x[b])
            self.fused(xb.reshape(N * N, D), mask[b], out[b], accumulate=False, xn_transposed=use_xn)
        # keep_t (the ending node's update left in its attention frame, [B, J, I, C]) is an f16-path option of the
        # reference (attention.py:130-131); its fp32 path always returns the natural layout (attention.py:45-46, 91-92)
        if keep_t and not self.starting and K.f16():
            out = out.transpose(1, 2).contiguous()
        return out

    def fused(self, xn: torch.Tensor, mask: torch.Tensor, z: torch.Tensor, accumulate: bool = True, next_ln=None,
              before_core=None, xn_transposed: bool = False):
        """z (+)= self(z) from xn = layer_norm(z) ([N*N, D], storage dtype; natural layout, or for the ending node
        transposed when xn_transposed) and the pair mask [N, N] fp32 (natural layout); returns next_ln(z_new) when
        next_ln is given. before_core() is called after the projection is enqueued and before the attention core
        (the point where independent work on another stream overlaps the core rather than a persistent kernel)."""
        N, D = z.shape[0], z.shape[-1]
        H, C = self.no_heads, self.mha.c_hidden
        w, w_o = self.prepare()
        trans = not self.starting
        # the projection reads xn at the attention frame's position: transposed for the ending node unless the
        # caller already transposed it
        proj_trans = trans and not xn_transposed
        if D != 128 or H * C != D:  # the fused projection / output kernels are built for 128 = H * C channels:
            # otherwise GEMMs plus layout kernels (the core takes C = 16, 32 or 64)
            qkg, vt, tb = K.triattn_pack(K.linear(xn, w), proj_trans, N, H, C)
            if before_core is not None:
                before_core()
            core = K.triattn_core(qkg, vt, tb, mask, trans, self.inf, N, H, C)
            del qkg, vt, tb
            y = K.linear(core, w_o, out_dtype=torch.float32).view(N, N, D)
            if not accumulate:
                z.zero_()
            nxt = K.add_ln(z, y, ln=next_ln, trans_y=trans, out_dtype=K.storage_dtype())
            return None if nxt is None else nxt.view(N * N, D)
        core = self._core_128(xn, mask, N, before_core, proj_trans)
        return K.linear_resid_ln(core, w_o, trans, z, accumulate, next_ln, N)

    def fused_core(self, xn: torch.Tensor, mask: torch.Tensor, before_core=None):
        """The 128-channel path of fused() without its output stage, for a consumer that applies linear_o and the
        residual itself (K.attn_out_transition): returns (core output [N*N, 128] in the storage dtype, in this node's
        attention frame, linear_o's kernel weight), or None where fused() takes the generic path."""
        N, D = mask.shape[0], xn.shape[-1]
        if D != 128 or self.no_heads * self.mha.c_hidden != D:
            return None
        return self._core_128(xn, mask, N, before_core, not self.starting), self.prepare()[1]

    def _core_128(self, xn, mask, N: int, before_core, proj_trans: bool):
        H, C = self.no_heads, self.mha.c_hidden
        w = self.prepare()[0]
        qkg, vt, tb = K.triattn_proj(xn, w, proj_trans, N, H, C)
        if before_core is not None:
            before_core()
        core = K.triattn_core(qkg, vt, tb, mask, not self.starting, self.inf, N, H, C)
        del qkg, vt, tb
        return core

    def kernel_weights(self):
        """[q; k; v; g; triangle bias] (the projection's 4·H·C + H rows) and linear_o, in the storage dtype."""
        return (K.KernelWeight("w_qkvgb", ("mha.linear_q.weight", "mha.linear_k.weight", "mha.linear_v.weight",
                                           "mha.linear_g.weight", "linear.weight")),
                K.KernelWeight("w_o", ("mha.linear_o.weight",)))

    def prepare(self):
        """The kernel weights ([q; k; v; g; triangle bias] and linear_o), cached on the module."""
        return K.kernel_weight(self, "w_qkvgb"), K.kernel_weight(self, "w_o")


TriangleAttentionStartingNode = TriangleAttention


class TriangleAttentionEndingNode(TriangleAttention):
    def __init__(self, c_in: int, c_hidden: int, no_heads: int, inf: float = 1e9) -> None:
        super().__init__(c_in, c_hidden, no_heads, starting=False, inf=inf)
