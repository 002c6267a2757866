"""numpy restatement of the reference's diffusion token transformer (test infrastructure: the reference results the tests
compare against, never the product).

Like oracle/pairformer.py, every function computes in the dtype of its inputs (float64 pins the parity tests) and
takes parameter dicts keyed by the reference's PyTorch qualified names relative to the module.

Sources restated (paths relative to the reference checkout):
- AdaLN (Algorithm 26): boltz_mlx/modules/transformersv2.py:27-41 (a_norm: LayerNorm without affine; s_norm:
  LayerNorm with weight and no bias; sigmoid(s_scale(s)) * a + s_bias(s)).
- ConditionedTransitionBlock (Algorithm 25): transformersv2.py:44-66 (SwiGLU splits [x, gates] and applies silu to
  the gates, transformersv2.py:15-18).
- DiffusionTransformerLayer (Algorithm 23, one layer): transformersv2.py:69-108 (the module-level path without the
  precomputed conditioning), attention through AttentionPairBias(compute_pair_bias=False) (attentionv2.py:43-86).
- DiffusionTransformer: transformersv2.py:259-297 (the pair bias [B, N, M, L * H] split per layer).

Parity status: pinned by tests/test_oracle_diffusion.py against torch float64 formulations (layer_norm,
scaled_dot_product_attention), the fast path with the s-side conditioning precomputed for all layers
(transformersv2.py:376-420, restated independently below in precompute_cond / layer_fast), and closed forms
(zero output gates' linears give the identity update scaled by 1/2, zero b_to_a gives no transition update).
"""

from __future__ import annotations

import numpy as np

from oracle.pairformer import layer_norm, linear, sigmoid, silu, softmax, sub

__all__ = ["adaln", "conditioned_transition", "pair_bias_attention", "diffusion_layer", "diffusion_transformer",
           "precompute_cond", "diffusion_layer_fast"]


def adaln(a, s, p: dict):
    """AdaLN (transformersv2.py:36-41): sigmoid(s_scale(LN_w(s))) * LN(a) + s_bias(LN_w(s))."""
    an = layer_norm(a, None, None, 1e-5)
    sn = layer_norm(s, p["s_norm.weight"], None, 1e-5)
    return sigmoid(linear(sn, p["s_scale.weight"], p["s_scale.bias"])) * an + linear(sn, p["s_bias.weight"])


def conditioned_transition(a, s, p: dict):
    """ConditionedTransitionBlock (transformersv2.py:55-66): a' = AdaLN(a, s); h = swish_gate.0(a') split [x, gates];
    b = silu(gates) * x * a_to_b(a'); out = sigmoid(output_projection.0(s)) * b_to_a(b)."""
    a = adaln(a, s, sub(p, "adaln"))
    h = linear(a, p["swish_gate.0.weight"])
    inner = h.shape[-1] // 2
    x, gates = h[..., :inner], h[..., inner:]
    b = silu(gates) * x * linear(a, p["a_to_b.weight"])
    o = sigmoid(linear(s, p["output_projection.0.weight"], p["output_projection.0.bias"]))
    return o * linear(b, p["b_to_a.weight"])


def pair_bias_attention(s, bias, mask, k_in, p: dict, num_heads: int, multiplicity: int = 1, inf: float = 1e6):
    """AttentionPairBias with compute_pair_bias=False (attentionv2.py:43-86): bias [B, N, M, H] is given (repeated
    over `multiplicity` consecutive samples); logits = q k^T / sqrt(hd) + bias + (1 - mask) * (-inf);
    y = proj_o(sigmoid(proj_g(s)) * softmax(logits) v)."""
    Bm, N, Cs = s.shape
    H = num_heads
    hd = Cs // H
    q = linear(s, p["proj_q.weight"], p["proj_q.bias"]).reshape(Bm, N, H, hd).transpose(0, 2, 1, 3)
    k = linear(k_in, p["proj_k.weight"]).reshape(Bm, -1, H, hd).transpose(0, 2, 3, 1)
    v = linear(k_in, p["proj_v.weight"]).reshape(Bm, -1, H, hd).transpose(0, 2, 1, 3)
    b = np.repeat(bias.transpose(0, 3, 1, 2), multiplicity, axis=0)  # [B * mult, H, N, M]
    g = sigmoid(linear(s, p["proj_g.weight"]))
    att = (q @ k) / s.dtype.type(hd ** 0.5) + b
    att = att + (1 - mask[:, None, None, :].astype(s.dtype)) * s.dtype.type(-inf)
    o = (softmax(att, -1) @ v).transpose(0, 2, 1, 3).reshape(Bm, N, Cs)
    return linear(g * o, p["proj_o.weight"])


def diffusion_layer(a, s, bias, mask, p: dict, num_heads: int, multiplicity: int = 1, post_layer_norm: bool = False):
    """DiffusionTransformerLayer.__call__ without precomputed conditioning (transformersv2.py:88-108)."""
    b = adaln(a, s, sub(p, "adaln"))
    b = pair_bias_attention(b, bias, mask, b, sub(p, "pair_bias_attn"), num_heads, multiplicity)
    b = sigmoid(linear(s, p["output_projection_linear.weight"], p["output_projection_linear.bias"])) * b
    a = a + b
    a = a + conditioned_transition(a, s, sub(p, "transition"))
    if post_layer_norm:
        a = layer_norm(a, p["post_lnorm.weight"], p["post_lnorm.bias"], 1e-5)
    return a


def diffusion_transformer(a, s, bias, mask, p: dict, depth: int, num_heads: int, multiplicity: int = 1):
    """DiffusionTransformer.__call__ (transformersv2.py:284-297): bias [B, N, M, L * H] viewed as [B, N, M, L, H],
    layer i taking bias[..., i, :]; params under ``layers.{i}.``."""
    B, N, M, D = bias.shape
    bias = bias.reshape(B, N, M, depth, D // depth)
    for i in range(depth):
        a = diffusion_layer(a, s, bias[:, :, :, i], mask, sub(p, f"layers.{i}"), num_heads, multiplicity)
    return a


def precompute_cond(s, p: dict, depth: int):
    """The s-side projections of every layer in two products (the fast path, transformersv2.py:376-420): with g the
    s_norm weight folded into the columns of s_scale / s_bias, h1 = LN(s) . [s_scale g; s_bias g; s_scale' g';
    s_bias' g']^T + [s_scale.b; 0; s_scale'.b; 0] and h2 = s . [out_proj; transition out_proj]^T + biases, per layer.
    Returns (h1 [..., L, 4, D], h2 [..., L, 2, D]) before any sigmoid."""
    w1, b1, w2, b2 = [], [], [], []
    for i in range(depth):
        q = sub(p, f"layers.{i}")
        for ad in ("adaln", "transition.adaln"):
            g = q[f"{ad}.s_norm.weight"][None, :]
            w1 += [q[f"{ad}.s_scale.weight"] * g, q[f"{ad}.s_bias.weight"] * g]
            b1 += [q[f"{ad}.s_scale.bias"], np.zeros_like(q[f"{ad}.s_scale.bias"])]
        w2 += [q["output_projection_linear.weight"], q["transition.output_projection.0.weight"]]
        b2 += [q["output_projection_linear.bias"], q["transition.output_projection.0.bias"]]
    h1 = linear(layer_norm(s, None, None, 1e-5), np.concatenate(w1, 0), np.concatenate(b1, 0))
    h2 = linear(s, np.concatenate(w2, 0), np.concatenate(b2, 0))
    D = h1.shape[-1] // (4 * depth)
    return h1.reshape(*s.shape[:-1], depth, 4, D), h2.reshape(*s.shape[:-1], depth, 2, D)


def diffusion_layer_fast(a, h1, h2, bias, mask, p: dict, num_heads: int, multiplicity: int = 1):
    """One layer from the precomputed conditioning of that layer, h1 [..., 4, D] and h2 [..., 2, D]
    (transformersv2.py:199-264: attn_scale * LN(a) + attn_shift, one q|k|v|g product, a + out_gate * o; then
    tr_scale * LN(a) + tr_shift, the [x, gates, a_to_b] product, a + tr_gate * b_to_a(silu(gates) x ab))."""
    at, tr = sub(p, "pair_bias_attn"), sub(p, "transition")
    b = sigmoid(h1[..., 0, :]) * layer_norm(a, None, None, 1e-5) + h1[..., 1, :]
    o = pair_bias_attention(b, bias, mask, b, at, num_heads, multiplicity)
    a = a + sigmoid(h2[..., 0, :]) * o
    t = sigmoid(h1[..., 2, :]) * layer_norm(a, None, None, 1e-5) + h1[..., 3, :]
    h = linear(t, tr["swish_gate.0.weight"])
    inner = h.shape[-1] // 2
    u = silu(h[..., inner:]) * h[..., :inner] * linear(t, tr["a_to_b.weight"])
    return a + sigmoid(h2[..., 1, :]) * linear(u, tr["b_to_a.weight"])
