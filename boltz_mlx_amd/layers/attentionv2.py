"""AttentionPairBias (v2) on the bzpf kernels: the s track's pair-biased attention.

Same constructor, parameters and call signature as boltz_mlx/layers/attentionv2.py:12-86
(``AttentionPairBias(c_s, c_z, num_heads, inf=1e6, compute_pair_bias=True)(s, z, mask, k_in, multiplicity=1,
pair_bias=None)``). proj_z is Sequential(LayerNorm, Linear) as in the PyTorch checkpoint (names proj_z.0.*,
proj_z.1.*); its [N, N, H] -> [H, N, N] rearrangement is folded into the pair-bias kernel's output layout.

Precision follows the reference's f16 mode (attentionv2.py:50-84 with the fp16 weight set of its
fp16_manifest.json): proj_q / proj_k / proj_v / proj_g / proj_o, the logits, the softmax and the weighted sum stay
fp32 in both modes; only the pair bias proj_z(z) is computed and stored in fp16 in f16 mode (fp16 proj_z.1 weight),
and the fp32 logits add it as it is.
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

    def kernel_weights(self):
        """[proj_q; proj_k; proj_v; proj_g] and proj_o in fp32 (both modes), proj_z's linear in the storage dtype."""
        kws = (K.KernelWeight("w_qkvg", ("proj_q.weight", "proj_k.weight", "proj_v.weight", "proj_g.weight"),
                              half=False),
               K.KernelWeight("w_o", ("proj_o.weight",), half=False))
        return kws + ((K.KernelWeight("w_z", ("proj_z.1.weight",)),) if self.compute_pair_bias else ())

    def qkvg_bias(self) -> torch.Tensor:
        """fp32 [4 c_s]: proj_q's bias, then zeros (the bias of the fused q | k | v | g GEMM), cached."""
        bq = self.proj_q.bias
        key = (bq.data_ptr(), bq._version, bq.device)
        hit = self.__dict__.get("_bzpf_b_qkvg")
        if hit is None or hit[0] != key:
            full = torch.zeros(4 * self.c_s, dtype=torch.float32, device=bq.device)
            with torch.no_grad():
                full[: self.c_s] = bq.detach().float()
            hit = (key, full)
            self.__dict__["_bzpf_b_qkvg"] = hit
        return hit[1]

    def prepare(self):
        """The kernel weights, cached on the module: [proj_q; proj_k; proj_v; proj_g] (fp32) with the matching bias
        (fp32), proj_o (fp32), and proj_z's linear in the storage dtype when the module computes it (else None)."""
        w_z = K.kernel_weight(self, "w_z") if self.compute_pair_bias else None
        return K.kernel_weight(self, "w_qkvg"), self.qkvg_bias(), K.kernel_weight(self, "w_o"), w_z

    def pair_bias(self, z: torch.Tensor) -> torch.Tensor:
        """proj_z(z) as [H, N, N] in the storage dtype, from z [N, N, c_z] fp32."""
        return K.pair_bias(z, self.proj_z[0], self.prepare()[3])

    def forward(self, s: torch.Tensor, z: torch.Tensor, mask: torch.Tensor, k_in: torch.Tensor,
                multiplicity: int = 1, pair_bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        """s, k_in: [B, N, c_s]; z: [B, N, N, c_z] fp32 (or, without compute_pair_bias, the bias [B, N, N, H]);
        mask: [B, N]; pair_bias: proj_z(z) already computed as [B, H, N, N]. Returns the update [B, N, c_s] fp32."""
        B, N, _ = s.shape
        out = torch.empty((B, N, self.c_s), dtype=torch.float32, device=s.device)
        mask = mask.to(torch.float32).contiguous()

        def as_bias(t):  # fp32 or fp16 as given (the logits are fp32 and add it as it is)
            return t.contiguous() if t.dtype in (torch.float32, torch.float16) else t.float().contiguous()

        for b in range(B):
            zb = b // multiplicity
            if pair_bias is not None:
                bias = as_bias(pair_bias[zb])
            elif self.compute_pair_bias:
                bias = self.pair_bias(z[zb].contiguous())
            else:
                bias = as_bias(z[zb].permute(2, 0, 1))
            self.fused(s[b].float().contiguous(), k_in[b].float().contiguous(), bias, mask[b], out[b],
                       accumulate=False)
        return out

    def fused(self, s: torch.Tensor, k_in: torch.Tensor, bias: torch.Tensor, mask: torch.Tensor, out: torch.Tensor,
              accumulate: bool = True) -> None:
        """out (+)= attention(s, k_in) for one batch element: s, k_in [N, c_s] fp32, bias [H, N, N] (fp32, or fp16
        in f16 mode), mask [N] fp32, out [N, c_s] fp32."""
        if s.dtype != torch.float32 or k_in.dtype != torch.float32:
            raise ValueError("AttentionPairBias.fused: s and k_in must be fp32 (the s track's projections are fp32)")
        w_qkvg, b_qkvg, w_o, _ = self.prepare()
        c = self.c_s
        if k_in is s:  # one GEMM for q, k, v, g (the Pairformer's self-attention): [N, 4 c_s]
            qkvg = K.linear(s, w_qkvg, bias=b_qkvg)
            o = K.seq_attention_packed(qkvg, bias, mask, self.inf, self.num_heads)
        else:
            q = K.linear(s, w_qkvg[:c], bias=b_qkvg[:c])
            k = K.linear(k_in, w_qkvg[c:2 * c])
            v = K.linear(k_in, w_qkvg[2 * c:3 * c])
            g = K.linear(s, w_qkvg[3 * c:])
            o = K.seq_attention(q, k, v, g, bias, mask, self.inf, self.num_heads)
        K.linear(o, w_o, out=out, accumulate=accumulate)
