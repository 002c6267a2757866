"""PairformerLayer / PairformerModule (and the no-sequence variants) on the bzpf kernels.

Same constructors, parameter names and call signatures as boltz_mlx/layers/pairformer.py:23-153 (v2 layers,
inference only). The layer runs the reference order (pairformer.py:84-93, strict path 238-247 of the MLX port):
z += tri_mul_out; z += tri_mul_in; z += tri_att_start; z += tri_att_end; z += transition_z; then
s += attention(pre_norm_s(s), z, mask, k_in=pre_norm_s(s)); s += transition_s(s).

Each pair update is one fused kernel chain that adds its result into z in place and writes the next module's
LayerNorm output (the reference's add_ln / *_addln epilogues, kernels_nax3.py), so z is read and written once
per update. PairformerModule clones its inputs once and carries the next layer's norm_in output from each
layer's transition (the reference's PAIRLNX carry, pairformer.py:145-148, 243-246).
"""

from __future__ import annotations

import sys
from typing import Optional

import torch

from boltz_mlx_amd import kernels as K
from boltz_mlx_amd.layers.attentionv2 import AttentionPairBias as AttentionPairBiasV2
from boltz_mlx_amd.layers.norm import LayerNorm
from boltz_mlx_amd.layers.transition import Transition
from boltz_mlx_amd.layers.triangular_attention.attention import (
    TriangleAttentionEndingNode,
    TriangleAttentionStartingNode,
)
from boltz_mlx_amd.layers.triangular_mult import TriangleMultiplicationIncoming, TriangleMultiplicationOutgoing


def _pair_chain(layer, z: torch.Tensor, pm: torch.Tensor, xn_in: Optional[torch.Tensor], next_ln, hooks=(None, None),
                pair_bias=None):
    """The five pair updates on one batch element z [N, N, D] (fp32, updated in place) with pair mask pm [N, N]
    fp32. Returns next_ln(z_new) in the storage dtype (or None); with pair_bias = (LayerNorm, weight) the
    transition also returns the s track's pair bias of z_new: (next_ln(z_new), bias [H, N, N]). hooks[0] / hooks[1]
    are called just before the starting / ending node's attention core is enqueued."""
    N, D = z.shape[0], z.shape[-1]
    xn = layer.tri_mul_out.norm_in.to_storage(z).reshape(N * N, D) if xn_in is None else xn_in
    xn = layer.tri_mul_out.fused(xn, pm, z, True, next_ln=layer.tri_mul_in.norm_in)
    xn = layer.tri_mul_in.fused(xn, pm, z, True, next_ln=layer.tri_att_start.layer_norm)
    xn = layer.tri_att_start.fused(xn, pm, z, True, next_ln=layer.tri_att_end.layer_norm, before_core=hooks[0])
    tr = layer.transition_z
    if K.f16() and tr.fused_after_attention_ok(z):
        # the ending node's output stage (linear_o + residual) runs inside the transition kernel
        core = layer.tri_att_end.fused_core(xn, pm, before_core=hooks[1])
        if core is not None:
            return tr.fused_after_attention(core[0], core[1], True, z, next_ln=next_ln, pair_bias=pair_bias)
    xn = layer.tri_att_end.fused(xn, pm, z, True, next_ln=tr.norm, before_core=hooks[1])
    return tr.fused(xn, z, True, next_ln=next_ln, pair_bias=pair_bias)


def _guarded(owner: torch.nn.Module, run, outs: tuple, ins: tuple) -> None:
    """run() writes the fp32 streams `outs` in place, starting from copies of `ins`. In f16 with the guard on, the
    streams are checked for inf / nan afterwards (one device count, one sync) and, if any is found, the pass is
    recomputed with the fp32 kernels from `ins` (the reference's per-recycle fallback, boltz_mlx/model.py:176-193,
    with its stderr line and fallback counter)."""
    run()
    if not (K.f16() and K.GUARDS):
        return
    if int(K.count_nonfinite(*outs).item()) == 0:
        return
    owner.fp16_fallbacks += 1
    print(f"boltz_mlx_amd: fp16 overflow guard hit; pass recomputed in fp32 (fallback {owner.fp16_fallbacks})",
          file=sys.stderr)
    for o, i in zip(outs, ins):
        o.copy_(i)
    K.set_precision("fp32")
    try:
        run()
    finally:
        K.set_precision("f16")


class PairformerLayer(torch.nn.Module):
    def __init__(self, token_s: int, token_z: int, num_heads: int = 16, dropout: float = 0.25,
                 pairwise_head_width: int = 32, pairwise_num_heads: int = 4, post_layer_norm: bool = False,
                 v2: bool = True) -> None:
        super().__init__()
        if not v2:
            raise NotImplementedError("only the v2 pairformer layer is provided")
        self.token_z = token_z
        self.dropout = dropout  # unused at inference
        self.num_heads = num_heads
        self.post_layer_norm = post_layer_norm
        self.pre_norm_s = LayerNorm(token_s)
        self.attention = AttentionPairBiasV2(token_s, token_z, num_heads)
        self.tri_mul_out = TriangleMultiplicationOutgoing(token_z)
        self.tri_mul_in = TriangleMultiplicationIncoming(token_z)
        self.tri_att_start = TriangleAttentionStartingNode(token_z, pairwise_head_width, pairwise_num_heads, inf=1e9)
        self.tri_att_end = TriangleAttentionEndingNode(token_z, pairwise_head_width, pairwise_num_heads, inf=1e9)
        self.transition_s = Transition(token_s, token_s * 4)
        self.transition_z = Transition(token_z, token_z * 4)
        self.s_post_norm = LayerNorm(token_s) if post_layer_norm else torch.nn.Identity()

    def forward(self, s: torch.Tensor, z: torch.Tensor, mask: torch.Tensor, pair_mask: torch.Tensor,
                chunk_size_tri_attn: Optional[int] = None, use_kernels: bool = False, use_cuequiv_mul: bool = False,
                use_cuequiv_attn: bool = False, xn_in: Optional[torch.Tensor] = None,
                next_ln=None) -> tuple[torch.Tensor, torch.Tensor]:
        """s [B, N, token_s], z [B, N, N, token_z], mask [B, N], pair_mask [B, N, N] -> (s, z) (new tensors).
        chunk_size_tri_attn / use_* are accepted and ignored. xn_in: tri_mul_out.norm_in(z) in the storage dtype
        ([N*N, D], B = 1) as carried by PairformerModule."""
        s = s.to(torch.float32).clone().contiguous()
        z = z.to(torch.float32).clone().contiguous()
        self.inplace(s, z, mask.to(torch.float32).contiguous(), pair_mask.to(torch.float32).contiguous(),
                     xn_in=xn_in, next_ln=None)
        return s, z

    def inplace(self, s: torch.Tensor, z: torch.Tensor, mask: torch.Tensor, pair_mask: torch.Tensor,
                xn_in: Optional[torch.Tensor] = None, next_ln=None) -> Optional[torch.Tensor]:
        """Update fp32 s and z in place (masks fp32 contiguous). Returns next_ln(z_new) for B = 1, else None."""
        B = z.shape[0]
        xn_next = None
        for b in range(B):
            xn_next, bias = _pair_chain(self, z[b], pair_mask[b], xn_in if B == 1 else None,
                                        next_ln if B == 1 else None, pair_bias=self._pair_bias_args())
            self._s_update(s[b], bias, mask[b])
        return xn_next

    def _pair_bias_args(self):
        """(LayerNorm, weight) of the attention's proj_z, for the transition's pair-bias epilogue."""
        return self.attention.proj_z[0], self.attention.prepare()[3]

    def prepare(self) -> None:
        """Cache every kernel weight of the layer in the storage dtype (a one-time conversion per precision; the
        module does it for all layers before the first block, outside the steady-state block loop)."""
        for mod in (self.attention, self.tri_mul_out, self.tri_mul_in, self.tri_att_start, self.tri_att_end,
                    self.transition_s, self.transition_z):
            mod.prepare()

    def _s_update(self, s: torch.Tensor, bias: torch.Tensor, mask: torch.Tensor) -> None:
        """s += attention(pre_norm_s(s), pair bias) then s += transition_s(s), in place (one batch element)."""
        self._s_attention(s, bias, mask)
        self._s_transition(s)

    def _s_attention(self, s: torch.Tensor, bias: torch.Tensor, mask: torch.Tensor) -> None:
        # fp32 in both modes (the reference's f16 mode keeps the s attention's projections and softmax in fp32; the
        # pair bias is fp16 there)
        s_n = K.layer_norm(s, self.pre_norm_s.weight, self.pre_norm_s.bias, self.pre_norm_s.eps,
                           out_dtype=torch.float32)
        self.attention.fused(s_n, s_n, bias, mask, s, accumulate=True)

    def _s_transition(self, s: torch.Tensor) -> None:
        self.transition_s.unfused(self.transition_s.norm.to_storage(s), out=s, accumulate=True)
        if not isinstance(self.s_post_norm, torch.nn.Identity):
            s.copy_(self.s_post_norm(s))


class PairformerModule(torch.nn.Module):
    def __init__(self, token_s: int, token_z: int, num_blocks: int, num_heads: int = 16, dropout: float = 0.25,
                 pairwise_head_width: int = 32, pairwise_num_heads: int = 4, post_layer_norm: bool = False,
                 activation_checkpointing: bool = False, v2: bool = True, **kwargs) -> None:
        super().__init__()
        self.token_z = token_z
        self.num_blocks = num_blocks
        self.dropout = dropout
        self.num_heads = num_heads
        self.post_layer_norm = post_layer_norm
        self.fp16_fallbacks = 0  # passes the fp16 overflow guard recomputed in fp32
        self.layers = torch.nn.ModuleList([
            PairformerLayer(token_s, token_z, num_heads, dropout, pairwise_head_width, pairwise_num_heads,
                            post_layer_norm, v2)
            for _ in range(num_blocks)
        ])

    def forward(self, s: torch.Tensor, z: torch.Tensor, mask: torch.Tensor, pair_mask: torch.Tensor,
                use_kernels: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
        """All layers on copies of s, z; in f16 the fp16 overflow guard checks the result and recomputes the pass
        in fp32 if it holds inf / nan (fp16_fallbacks counts those)."""
        s_in, z_in = s, z
        s = s.to(torch.float32).clone().contiguous()
        z = z.to(torch.float32).clone().contiguous()
        m, pm = mask.to(torch.float32).contiguous(), pair_mask.to(torch.float32).contiguous()
        _guarded(self, lambda: self.inplace(s, z, m, pm), (s, z), (s_in, z_in))
        return s, z

    def inplace(self, s: torch.Tensor, z: torch.Tensor, mask: torch.Tensor, pair_mask: torch.Tensor) -> None:
        """Run every layer on fp32 s, z in place (masks fp32 contiguous)."""
        self.run(s, z, mask, pair_mask, 0, len(self.layers))

    def run(self, s: torch.Tensor, z: torch.Tensor, mask: torch.Tensor, pair_mask: torch.Tensor, start: int,
            count: int, xn: Optional[torch.Tensor] = None, cycle: bool = False) -> Optional[torch.Tensor]:
        """Apply layers start, start + 1, ... (count of them, wrapping modulo the depth when cycle) to fp32 s, z
        in place; xn is the first layer's tri_mul_out.norm_in(z) when already computed (B = 1). Returns the next
        layer's norm_in(z) for B = 1 (the carry; None after the last layer unless cycle).

        The z updates of layer i + 1 read only z, so the s track of layer i (attention with the pair bias of layer
        i's z, then transition_s) runs on a second stream beside the pair kernels of layer i + 1: its attention half
        is released when layer i + 1's starting-node attention core starts and its transition half when the
        ending-node core starts, so it shares the GPU with those two (non-persistent) kernels rather than with the
        persistent row kernels, whose grids assume the whole GPU. (Measured at N = 400 and 1000, this takes the same
        block time as running the same kernels in series at those points: the s track's cost is its chain of small
        kernels, not the lack of overlap.) The pair bias is computed on the main
        stream (by the transition's epilogue) before z moves on; the main stream waits for the side stream once at
        the end. (The reference
        pipelines the same way by submitting layer i + 1 while layer i's tail runs, pairformer.py:145-148.)"""
        n, B = len(self.layers), z.shape[0]
        if self.__dict__.get("_bzpf_prepared") != K.storage_dtype():
            # first run in this precision: convert every layer's weights now; the per-call caches in the layers
            # still rebuild any weight that changes afterwards
            for layer in self.layers:
                layer.prepare()
            self.__dict__["_bzpf_prepared"] = K.storage_dtype()
        main = torch.cuda.current_stream(z.device)
        side = torch.cuda.Stream(device=z.device)
        side.wait_stream(main)  # s, the masks and the weights are ready

        def release(work):
            ready = torch.cuda.Event()
            ready.record(main)
            side.wait_event(ready)
            with torch.cuda.stream(side):
                work()

        def hooks_for(pending):
            if not pending:
                return (None, None)
            return (lambda: release(lambda: [lay._s_attention(sb, bias, mb) for lay, sb, bias, mb in pending]),
                    lambda: release(lambda: [lay._s_transition(sb) for lay, sb, _, _ in pending]))

        with K.pair_mask_scope():  # the mask-derived values are made once for all the layers
            xn = xn if B == 1 else None
            pending = []  # s-track work of the previous layer: (layer, s[b], pair bias, mask[b])
            for k in range(count):
                i = (start + k) % n
                layer = self.layers[i]
                nxt = self.layers[(i + 1) % n].tri_mul_out.norm_in if (i + 1 < n or cycle) else None
                done = []
                for b in range(B):
                    hooks = hooks_for(pending) if b == 0 else (None, None)
                    xn, bias = _pair_chain(layer, z[b], pair_mask[b], xn if B == 1 else None,
                                           nxt if B == 1 else None, hooks, pair_bias=layer._pair_bias_args())
                    bias.record_stream(side)  # allocated on the main stream, read on the side stream
                    done.append((layer, s[b], bias, mask[b]))
                pending = done
        hooks = hooks_for(pending)
        hooks[0]()
        hooks[1]()
        main.wait_stream(side)
        return xn if B == 1 else None


class PairformerNoSeqLayer(torch.nn.Module):
    def __init__(self, token_z: int, dropout: float = 0.25, pairwise_head_width: int = 32,
                 pairwise_num_heads: int = 4, post_layer_norm: bool = False) -> None:
        super().__init__()
        self.token_z = token_z
        self.dropout = dropout
        self.post_layer_norm = post_layer_norm
        self.tri_mul_out = TriangleMultiplicationOutgoing(token_z)
        self.tri_mul_in = TriangleMultiplicationIncoming(token_z)
        self.tri_att_start = TriangleAttentionStartingNode(token_z, pairwise_head_width, pairwise_num_heads, inf=1e9)
        self.tri_att_end = TriangleAttentionEndingNode(token_z, pairwise_head_width, pairwise_num_heads, inf=1e9)
        self.transition_z = Transition(token_z, token_z * 4)

    def forward(self, z: torch.Tensor, pair_mask: torch.Tensor, chunk_size_tri_attn: Optional[int] = None,
                use_kernels: bool = False, use_cuequiv_mul: bool = False, use_cuequiv_attn: bool = False,
                xn_in: Optional[torch.Tensor] = None, next_ln=None) -> torch.Tensor:
        z = z.to(torch.float32).clone().contiguous()
        self.inplace(z, pair_mask.to(torch.float32).contiguous(), xn_in=xn_in)
        return z

    def inplace(self, z: torch.Tensor, pair_mask: torch.Tensor, xn_in=None, next_ln=None):
        B = z.shape[0]
        xn_next = None
        for b in range(B):
            xn_next = _pair_chain(self, z[b], pair_mask[b], xn_in if B == 1 else None, next_ln if B == 1 else None)
        return xn_next


class PairformerNoSeqModule(torch.nn.Module):
    def __init__(self, token_z: int, num_blocks: int, dropout: float = 0.25, pairwise_head_width: int = 32,
                 pairwise_num_heads: int = 4, post_layer_norm: bool = False, activation_checkpointing: bool = False,
                 **kwargs) -> None:
        super().__init__()
        self.token_z = token_z
        self.num_blocks = num_blocks
        self.dropout = dropout
        self.post_layer_norm = post_layer_norm
        self.fp16_fallbacks = 0  # passes the fp16 overflow guard recomputed in fp32
        self.layers = torch.nn.ModuleList([
            PairformerNoSeqLayer(token_z, dropout, pairwise_head_width, pairwise_num_heads, post_layer_norm)
            for _ in range(num_blocks)
        ])

    def forward(self, z: torch.Tensor, pair_mask: torch.Tensor, use_kernels: bool = False) -> torch.Tensor:
        z_in = z
        z = z.to(torch.float32).clone().contiguous()
        pm = pair_mask.to(torch.float32).contiguous()

        def run():
            n, xn = len(self.layers), None
            with K.pair_mask_scope():
                for i, layer in enumerate(self.layers):
                    nxt = self.layers[i + 1].tri_mul_out.norm_in if i + 1 < n else None
                    xn = layer.inplace(z, pm, xn_in=xn, next_ln=nxt)

        _guarded(self, run, (z,), (z_in,))
        return z
