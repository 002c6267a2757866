"""Diffusion token transformer (AdaLN, ConditionedTransitionBlock, DiffusionTransformerLayer, DiffusionTransformer)
on the bzpf kernels.

Same constructors, parameter names and call signatures as boltz_mlx/modules/transformersv2.py:15-297 (inference,
full attention; the windowed ``to_keys`` form of the atom transformer is not built here). The output projection of
a layer is one Linear registered under two names (``output_projection_linear`` and ``output_projection.0``), as in
the PyTorch checkpoint.

Forward pass (the reference's fast path, transformersv2.py:199-264 and 376-420): the s-side projections of every
layer are computed once per call in two GEMMs (the s_norm weight folded into the AdaLN linears); each layer then runs
  b = sigmoid(attn_scale) * LN(a) + attn_shift                         bzpf_adaln
  q|k|v|g = b W_qkvg^T (+ q bias)                                      bzpf_linear
  o = sigmoid(g) * softmax(q k^T / sqrt(hd) + bias + mask) v            bzpf_seq_attention_batched
  a += sigmoid(out_gate) * (o W_o^T)                                   bzpf_linear_gated
  t = sigmoid(tr_scale) * LN(a) + tr_shift                             bzpf_adaln
  u = silu(t W_g^T) * (t W_x^T) * (t W_ab^T)                           bzpf_linear_swiglu3 (fp16; else
                                                                       bzpf_linear + bzpf_swiglu3)
  a += sigmoid(tr_gate) * (u W_ba^T)                                   bzpf_linear_gated
with a fp32 throughout; in f16 mode the GEMM operands and intermediates are fp16 (fp32 accumulation, LayerNorm
statistics and softmax).
"""

from __future__ import annotations

import torch

from boltz_mlx_amd import kernels as K
from boltz_mlx_amd.layers.attentionv2 import AttentionPairBias
from boltz_mlx_amd.layers.norm import LayerNorm


class SwiGLU(torch.nn.Module):
    """x, gates = split(h, 2); silu(gates) * x (transformersv2.py:15-18)."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x, gates = torch.chunk(x, 2, dim=-1)
        return torch.nn.functional.silu(gates) * x


class AdaLN(torch.nn.Module):
    """Algorithm 26 (transformersv2.py:27-41): sigmoid(s_scale(s_norm(s))) * a_norm(a) + s_bias(s_norm(s))."""

    def __init__(self, dim: int, dim_single_cond: int) -> None:
        super().__init__()
        self.a_norm = LayerNorm(dim, elementwise_affine=False)
        self.s_norm = LayerNorm(dim_single_cond, bias=False)
        self.s_scale = torch.nn.Linear(dim_single_cond, dim)
        self.s_bias = torch.nn.Linear(dim_single_cond, dim, bias=False)


class ConditionedTransitionBlock(torch.nn.Module):
    """Algorithm 25 (transformersv2.py:44-66)."""

    def __init__(self, dim_single: int, dim_single_cond: int, expansion_factor: int = 2) -> None:
        super().__init__()
        self.adaln = AdaLN(dim_single, dim_single_cond)
        dim_inner = int(dim_single * expansion_factor)
        self.swish_gate = torch.nn.Sequential(torch.nn.Linear(dim_single, dim_inner * 2, bias=False), SwiGLU())
        self.a_to_b = torch.nn.Linear(dim_single, dim_inner, bias=False)
        self.b_to_a = torch.nn.Linear(dim_inner, dim_single, bias=False)
        self.output_projection = torch.nn.Sequential(torch.nn.Linear(dim_single_cond, dim_single), torch.nn.Sigmoid())


class DiffusionTransformerLayer(torch.nn.Module):
    """Algorithm 23, one layer (transformersv2.py:69-108)."""

    def __init__(self, heads: int, dim: int = 384, dim_single_cond: int | None = None,
                 post_layer_norm: bool = False) -> None:
        super().__init__()
        dim_single_cond = dim if dim_single_cond is None else dim_single_cond
        self.adaln = AdaLN(dim, dim_single_cond)
        self.pair_bias_attn = AttentionPairBias(c_s=dim, num_heads=heads, compute_pair_bias=False)
        self.output_projection_linear = torch.nn.Linear(dim_single_cond, dim)
        self.output_projection = torch.nn.Sequential(self.output_projection_linear, torch.nn.Sigmoid())
        self.transition = ConditionedTransitionBlock(dim_single=dim, dim_single_cond=dim_single_cond)
        self.post_layer_norm = post_layer_norm
        if post_layer_norm:
            self.post_lnorm = LayerNorm(dim)

    def kernel_weights(self):
        """In the storage dtype: the attention's [proj_q; proj_k; proj_v; proj_g] and proj_o (fp16 GEMMs in f16 mode,
        unlike the Pairformer's s track), the transition's [swish_gate; a_to_b] rows (x, then the SiLU gates, then
        a_to_b: swish_gate's two halves in checkpoint order) and b_to_a."""
        return (K.KernelWeight("w_qkvg", ("pair_bias_attn.proj_q.weight", "pair_bias_attn.proj_k.weight",
                                          "pair_bias_attn.proj_v.weight", "pair_bias_attn.proj_g.weight")),
                K.KernelWeight("w_o", ("pair_bias_attn.proj_o.weight",)),
                K.KernelWeight("w_ff", ("transition.swish_gate.0.weight", "transition.a_to_b.weight")),
                K.KernelWeight("w_ba", ("transition.b_to_a.weight",)))

    def prepare(self):
        """The layer's kernel weights, cached: q|k|v|g with proj_q's bias (fp32), proj_o, the transition's
        [x; gates; a_to_b] rows and b_to_a."""
        w_qkvg, w_o, w_ff, w_ba = (K.kernel_weight(self, n) for n in ("w_qkvg", "w_o", "w_ff", "w_ba"))
        return w_qkvg, self.pair_bias_attn.qkvg_bias(), w_o, w_ff, w_ba

    def _ff_derived(self, w_ff, grouped: bool):
        """w_ff's rows for the feed-forward kernels, cached with its source: the SiLU gates first, then x, then a_to_b
        (the unfused GEMM + K.swiglu3), or those three regrouped per 32 output columns (K.linear_swiglu3)."""
        key = "_bzpf_ffg" if grouped else "_bzpf_ffr"
        hit = self.__dict__.get(key)
        if hit is None or hit[0] is not w_ff:
            H = w_ff.shape[0] // 3
            x, gates, ab = w_ff[:H], w_ff[H:2 * H], w_ff[2 * H:]
            w = K.group_swiglu3_rows(gates, x, ab) if grouped else torch.cat([gates, x, ab], 0).contiguous()
            hit = (w_ff, w)
            self.__dict__[key] = hit
        return hit[1]

    def ff_grouped(self, w_ff):
        """w_ff regrouped for the fused fp16 feed-forward kernel (K.linear_swiglu3)."""
        return self._ff_derived(w_ff, True)

    def forward(self, a, s, bias=None, mask=None, to_keys=None, multiplicity: int = 1, cond=None, attn_bias=None):
        """One layer on its own (a [B*mult, N, D], s [B*mult, N, Dc], bias [B, N, N, H], mask [B*mult, N])."""
        if to_keys is not None:
            raise NotImplementedError("windowed (to_keys) attention is not built")
        h1, h2 = _precompute_cond([self], s)
        out = a.to(torch.float32).clone().contiguous()
        _layer_fast(self, out, h1, h2, 0, 1, _layer_bias(bias, 0, 1, self.pair_bias_attn.num_heads),
                    mask.to(torch.float32).contiguous(), multiplicity)
        return out


def _cond_weights(layers, dtype, w_gates=None):
    """[s_scale g; s_bias g; s_scale' g'; s_bias' g'] per layer with g the s_norm weight folded into the columns (the
    product in fp32, then the storage dtype), their biases, and [output_projection; transition output_projection]
    with biases (transformersv2.py:376-420). w_gates: the latter rows already built (the stack's kernel weight)."""
    w1, b1, w2, b2 = [], [], [], []
    for layer in layers:
        for ad in (layer.adaln, layer.transition.adaln):
            g = ad.s_norm.weight.detach().float()[None, :]
            w1 += [ad.s_scale.weight.detach().float() * g, ad.s_bias.weight.detach().float() * g]
            b1 += [ad.s_scale.bias.detach().float(), torch.zeros_like(ad.s_scale.bias, dtype=torch.float32)]
        op = layer.transition.output_projection[0]
        w2 += [layer.output_projection_linear.weight.detach(), op.weight.detach()]
        b2 += [layer.output_projection_linear.bias.detach().float(), op.bias.detach().float()]
    w2 = torch.cat(w2, 0).to(dtype).contiguous() if w_gates is None else w_gates
    return torch.cat(w1, 0).to(dtype).contiguous(), torch.cat(b1, 0).contiguous(), w2, torch.cat(b2, 0).contiguous()


def _precompute_cond(layers, s, weights=None):
    """h1 [rows, L * 4 * D] and h2 [rows, L * 2 * D] (fp32, before any sigmoid) for s [..., Dc]."""
    dt = K.storage_dtype()
    w1, b1, w2, b2 = weights if weights is not None else _cond_weights(layers, dt)
    s2 = s.reshape(-1, s.shape[-1]).to(torch.float32).contiguous()
    sn = K.layer_norm(s2, None, None, 1e-5, out_dtype=dt)
    h1 = K.linear(sn, w1, bias=b1, out_dtype=torch.float32)
    h2 = K.linear(s2.to(dt).contiguous(), w2, bias=b2, out_dtype=torch.float32)
    return h1, h2


def _layer_bias(bias, i: int, L: int, H: int):
    """Layer i's pair bias as [B, H, N, M] in the storage dtype from bias [B, N, M, L * H] (transformersv2.py:284-292)."""
    B, N, M, _ = bias.shape
    return bias.reshape(B, N, M, L, H)[:, :, :, i].permute(0, 3, 1, 2).to(K.storage_dtype()).contiguous()


def _layer_fast(layer, a, h1, h2, i: int, L: int, bias_l, mask, multiplicity: int) -> None:
    """Layer i of L on a [B*mult, N, D] fp32 in place from the precomputed conditioning h1, h2."""
    Bm, N, D = a.shape
    rows_c = h1.shape[0]
    if rows_c not in (N, Bm * N):
        # the kernels pair row r with conditioning row r % rows_c: valid for one shared group or one per sample
        raise ValueError(f"conditioning s must have 1 or {Bm} samples of {N} tokens (a is [{Bm}, {N}, {D}]); got "
                         f"{rows_c} rows")
    dt = K.storage_dtype()
    at = layer.pair_bias_attn
    H = at.num_heads
    w_qkvg, b_qkvg, w_o, w_ff, w_ba = layer.prepare()
    rows = Bm * N
    a2 = a.view(rows, D)
    c1 = h1.view(-1, L, 4, D)[:, i]
    c2 = h2.view(-1, L, 2, D)[:, i]
    b = K.adaln(a2, c1[:, 0], c1[:, 1], dt)
    qkvg = K.linear(b, w_qkvg, bias=b_qkvg)
    o = K.seq_attention_packed(qkvg.view(Bm, N, 4 * D), bias_l, mask, at.inf, H, multiplicity=multiplicity)
    K.linear_gated(o.view(rows, D), w_o, c2[:, 0], a2)
    t = K.adaln(a2, c1[:, 2], c1[:, 3], dt)
    H3 = w_ff.shape[0]
    if dt == torch.float16 and D % 64 == 0 and (H3 // 3) % 32 == 0:
        u = K.linear_swiglu3(t, layer.ff_grouped(w_ff))
    else:
        u = K.swiglu3(K.linear(t, layer._ff_derived(w_ff, False)))
    K.linear_gated(u, w_ba, c2[:, 1], a2)
    if layer.post_layer_norm:
        a2.copy_(layer.post_lnorm(a2))


class DiffusionTransformer(torch.nn.Module):
    """Algorithm 23 (transformersv2.py:259-297)."""

    def __init__(self, depth: int, heads: int, dim: int = 384, dim_single_cond: int | None = None,
                 pair_bias_attn: bool = True, activation_checkpointing: bool = False,
                 post_layer_norm: bool = False) -> None:
        super().__init__()
        dim_single_cond = dim if dim_single_cond is None else dim_single_cond
        self.pair_bias_attn = pair_bias_attn
        self.layers = torch.nn.ModuleList([
            DiffusionTransformerLayer(heads, dim, dim_single_cond, post_layer_norm) for _ in range(depth)
        ])

    def kernel_weights(self):
        """The output gates of every layer in the storage dtype: [output_projection; transition output_projection]
        per layer (one GEMM per call over the conditioning s)."""
        srcs = []
        for i in range(len(self.layers)):
            srcs += [f"layers.{i}.output_projection_linear.weight", f"layers.{i}.transition.output_projection.0.weight"]
        return (K.KernelWeight("w_gates", tuple(srcs)),)

    def precompute_cond(self, s):
        """(h1, h2): every layer's s-side projections for s [..., Dc] (cached weights per storage dtype)."""
        dt = K.storage_dtype()
        w_gates = K.kernel_weight(self, "w_gates")
        key = (dt, w_gates.data_ptr()) + tuple((p.data_ptr(), p._version) for p in self.parameters())
        hit = self.__dict__.get("_bzpf_cond_w")
        if hit is None or hit[0] != key:
            hit = (key, _cond_weights(self.layers, dt, w_gates))
            self.__dict__["_bzpf_cond_w"] = hit
        return _precompute_cond(self.layers, s, hit[1])

    def prepare(self, bias):
        """The step-invariant per-layer pair biases [B, H, N, M] in the storage dtype from bias [B, N, M, L * H]
        (transformersv2.py:267-282)."""
        L = len(self.layers)
        H = self.layers[0].pair_bias_attn.num_heads
        return [_layer_bias(bias, i, L, H) for i in range(L)]

    def forward(self, a, s, bias=None, mask=None, to_keys=None, multiplicity: int = 1, cond=None, fast: bool = True,
                prepared=None):
        """a [B*mult, N, D], s [B*mult, N, Dc] (or [B', N, Dc] shared by consecutive groups of rows), bias
        [B, N, N, L * H] (shared by `multiplicity` consecutive samples), mask [B*mult, N]. Returns the new a (fp32).
        `cond` may hold a precomputed (h1, h2) from precompute_cond and `prepared` the per-layer biases from
        prepare(bias), as the reference's step loop does."""
        if to_keys is not None or not self.pair_bias_attn:
            raise NotImplementedError("only the full-attention token transformer with pair bias is built")
        L = len(self.layers)
        h1, h2 = cond if cond is not None else self.precompute_cond(s)
        biases = prepared if prepared is not None else self.prepare(bias)
        out = a.to(torch.float32).clone().contiguous()
        m = mask.to(torch.float32).contiguous()
        for i, layer in enumerate(self.layers):
            _layer_fast(layer, out, h1, h2, i, L, biases[i], m, multiplicity)
        return out


class DiffusionStepGraph:
    """One pass of a DiffusionTransformer over fixed conditioning (cond from precompute_cond, per-layer biases from
    prepare, mask, multiplicity) captured in a HIP graph and replayed per sampler step, so the twelve launches of each
    layer run without host work between them (the reference compiles its step loop instead,
    boltz_mlx/modules/transformersv2.py:259-297). The graph holds the weights, conditioning and work buffers of the
    capture: build a new one after any of them changes. __call__(a) copies a [B*mult, N, D] into the graph's input
    and replays; the result is the graph's output buffer, overwritten by the next call."""

    def __init__(self, module: DiffusionTransformer, a, cond, prepared, mask, multiplicity: int = 1) -> None:
        self.a_in = a.to(torch.float32).clone().contiguous()
        self.mask = mask.to(torch.float32).contiguous()

        def run():
            return module(self.a_in, None, None, self.mask, multiplicity=multiplicity, cond=cond, prepared=prepared)

        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            run()  # weight caches and the library are set up outside the capture
        torch.cuda.current_stream().wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.out = run()

    def __call__(self, a: torch.Tensor) -> torch.Tensor:
        self.a_in.copy_(a)
        self.graph.replay()
        return self.out
