"""SwiGLU Transition on the bzpf kernels.

Same constructor, parameters and call signature as boltz_mlx/layers/transition.py:12-54
(``Transition(dim=128, hidden=512, out_dim=None)(x, chunk_size=None, xn=None)``; fc1 is the SiLU branch,
148-154). For the pair width (dim 128, out_dim 128) one fused kernel does LN -> fc1|fc2 -> SwiGLU -> fc3 with the
hidden activations kept on chip; other widths (the s track, dim 384) run LN, the up-projection, SwiGLU and the
down-projection as separate bzpf kernels.
"""

from __future__ import annotations

from typing import Optional

import torch

from boltz_mlx_amd import kernels as K
from boltz_mlx_amd.layers.norm import LayerNorm


FUSED_MIN_ROWS = 16384  # rows from which the fp16 up-projection carries the SwiGLU product (bzpf_linear_swiglu)


class Transition(torch.nn.Module):
    def __init__(self, dim: int = 128, hidden: int = 512, out_dim: Optional[int] = None) -> None:
        super().__init__()
        if out_dim is None:
            out_dim = dim
        self.norm = LayerNorm(dim, eps=1e-5)
        self.fc1 = torch.nn.Linear(dim, hidden, bias=False)
        self.fc2 = torch.nn.Linear(dim, hidden, bias=False)
        self.fc3 = torch.nn.Linear(hidden, out_dim, bias=False)
        self.hidden = hidden

    def _pair_kernel(self) -> bool:
        return self.fc1.in_features == 128 and self.fc3.out_features == 128 and self.hidden % 64 == 0

    def forward(self, x: torch.Tensor, chunk_size: Optional[int] = None,
                xn: Optional[torch.Tensor] = None) -> torch.Tensor:
        """x: [..., dim] fp32 -> [..., out_dim] fp32. chunk_size is accepted and ignored (the fused kernel keeps
        no [rows, hidden] intermediate). xn: norm(x) already computed, used in f16 mode only, as the reference
        uses it (transition.py:27-31, 56-60); otherwise the LayerNorm is computed from x."""
        use_xn = xn is not None and K.f16()
        if use_xn and (tuple(xn.shape) != tuple(x.shape) or xn.dtype != K.storage_dtype()):
            raise ValueError(f"xn must be the fp16 norm output of shape {tuple(x.shape)}, got "
                             f"{tuple(xn.shape)} {xn.dtype}")
        xn = xn.contiguous() if use_xn else self.norm.to_storage(x)
        if self._pair_kernel():
            out = torch.empty(x.shape, dtype=torch.float32, device=x.device)
            self.fused(xn, out, accumulate=False)
            return out
        return self.unfused(xn)

    def kernel_weights(self):
        """[fc1; fc2] (the up-projection, SiLU branch first) and fc3, in the storage dtype."""
        return K.KernelWeight("w12", ("fc1.weight", "fc2.weight")), K.KernelWeight("w3", ("fc3.weight",))

    def prepare(self):
        """The kernel weights in the storage dtype ([fc1; fc2] and fc3), cached on the module. In f16 mode at 64
        channels the hidden activations are scaled by 2^-TRANS64_K before their fp16 store and the output by
        2^TRANS64_K (the reference's fp16 overflow margin, boltz_mlx/kernels.py:1327, layers/transition.py:60-92):
        folded exactly into the weights as fc2 * 2^-k and fc3 * 2^k."""
        w12, w3 = K.kernel_weight(self, "w12"), K.kernel_weight(self, "w3")
        k = K.TRANS64_K if (K.f16() and self.fc1.in_features == 64) else 0
        if not k:
            return w12, w3
        hit = self.__dict__.get("_bzpf_scaled")
        if hit is None or hit[0] is not w12 or hit[1] is not w3 or hit[2] != k:
            w12s = w12.clone()
            w12s[self.hidden:] *= 2.0 ** -k
            hit = (w12, w3, k, w12s, (w3 * 2.0 ** k).contiguous())
            self.__dict__["_bzpf_scaled"] = hit
        return hit[3], hit[4]

    def fused(self, xn: torch.Tensor, z: torch.Tensor, accumulate: bool = True, next_ln=None, pair_bias=None):
        """z (+)= transition from xn = norm(z) (storage dtype); returns next_ln(z_new) when next_ln is given. With
        pair_bias = (LayerNorm, weight [H, D]) it also returns Linear(LN(z_new)) as [H, N, N]: (next_ln(z_new), bias)."""
        if not self._pair_kernel():  # other channel counts: GEMMs + SwiGLU, residual in the second GEMM
            if pair_bias is not None:
                raise NotImplementedError("the pair-bias epilogue needs the 128-channel transition kernel")
            z2 = z.view(-1, z.shape[-1])
            if accumulate and self._fused64_ok(z2):  # xn = norm(z): the kernel recomputes it from z
                w12, w3 = self.prepare()
                K.transition64_f16(z2, self.norm, w12, w3)
            else:
                self.unfused(xn, out=z2, accumulate=accumulate)
            return None if next_ln is None else next_ln.to_storage(z2).reshape(z2.shape)
        w12, w3 = self.prepare()
        return K.transition(xn, w12, w3, z, accumulate, next_ln, pair_bias)

    def fused_after_attention_ok(self, z: torch.Tensor) -> bool:
        """Whether fused_after_attention applies: fp16 mode, the 128-channel pair kernel, z [N, N, 128]."""
        return K.f16() and self._pair_kernel() and z.dim() == 3 and z.shape[0] == z.shape[1]

    def fused_after_attention(self, o: torch.Tensor, w_o: torch.Tensor, trans: bool, z: torch.Tensor, next_ln=None,
                              pair_bias=None):
        """z += o' w_o^T (a triangle attention's output stage: o' = its core output o at the transposed position
        when trans), then z += self(z) in one fp16 kernel (fused_after_attention_ok(z) must hold); returns what
        fused() returns."""
        w12, w3 = self.prepare()
        return K.attn_out_transition(o, w_o, trans, z, self.norm, w12, w3, next_ln, pair_bias)

    def _fused64_ok(self, x: torch.Tensor) -> bool:
        """Whether x (fp32 [rows, dim]) takes bzpf_transition64_f16: f16 mode, 64 channels, hidden a multiple of 64
        up to 384, and the large row counts (the MSA track, the template stack's pairs)."""
        return (K.f16() and self.fc1.in_features == 64 and self.fc3.out_features == 64 and self.hidden % 64 == 0
                and self.hidden <= 384 and x.dtype == torch.float32 and x.is_contiguous()
                and x.shape[0] >= FUSED_MIN_ROWS)

    def inplace(self, x: torch.Tensor) -> None:
        """x (fp32 [rows, dim], contiguous) += self(x). At 64 channels in f16 mode over many rows (the MSA track) one
        kernel computes the LayerNorm, both projections and the residual (bzpf_transition64_f16); otherwise
        norm + unfused."""
        if self._fused64_ok(x):
            w12, w3 = self.prepare()
            K.transition64_f16(x, self.norm, w12, w3)
            return
        self.unfused(self.norm.to_storage(x), out=x, accumulate=True)

    def unfused(self, xn: torch.Tensor, out: Optional[torch.Tensor] = None, accumulate: bool = False):
        """fc3(SwiGLU(xn fc12^T)) as row GEMMs (in fp16 the up-projection carries the SwiGLU product in its
        epilogue); accumulate adds into the fp32 `out`."""
        w12, w3 = self.prepare()
        # fused for the large row counts (MSA rows x tokens, pairs); the s track's N rows run on a side stream next
        # to the triangle core, where the separate small kernels find free slots more easily
        if xn.dtype == torch.float16 and xn.shape[-1] % 64 == 0 and self.hidden % 32 == 0 \
                and xn.numel() // xn.shape[-1] >= FUSED_MIN_ROWS:
            hit = self.__dict__.get("_bzpf_w12g")
            if hit is None or hit[0] is not w12:
                hit = (w12, K.group_swiglu_rows(w12[:self.hidden], w12[self.hidden:]))
                self.__dict__["_bzpf_w12g"] = hit
            a = K.linear_swiglu(xn.contiguous(), hit[1])
        else:
            a = K.swiglu(K.linear(xn, w12))
        return K.linear(a, w3, out=out, out_dtype=torch.float32, accumulate=accumulate)
