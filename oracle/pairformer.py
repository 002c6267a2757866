"""numpy restatement of the reference's Pairformer pair path (test infrastructure: the reference results the tests
compare against, never the product).

Every function computes in the dtype of its inputs: float64 pins the parity tests, float32 is the
reference-equivalent CPU path timed beside the GPU (the reference's own CPU path is MLX fp32; MLX is not
installed here, so this restatement stands in for it).

Parameters are plain dicts keyed by the reference's PyTorch/MLX qualified names relative to the module
(``norm_in.weight``, ``p_in.weight``, ``mha.linear_q.weight`` ...); ``nn.Linear.weight`` is [out, in].

Sources restated (paths relative to the reference checkout):
- LayerNorm: boltz_mlx/layers/norm.py:8-17, boltz_mlx/kernels.py:438-507 (two-pass fp32 statistics, rsqrt).
- Triangle multiplication: boltz_mlx/layers/triangular_mult.py:23-65 (generic path), 67-105 (B=1 layout).
- Triangle attention: boltz_mlx/layers/triangular_attention/attention.py:27-93 and primitives.py:40-75
  (q scaled by 1/sqrt(c) before q.k; logits + mask_bias, then + tri_bias; sigmoid gate; linear_o).
- Transition: boltz_mlx/layers/transition.py:27-54, 148-154 (fc1 is the SiLU branch).
- AttentionPairBias (s track): boltz_mlx/layers/attentionv2.py:43-86.
- PairformerLayer / PairformerModule: boltz_mlx/layers/pairformer.py:59-94, 135-153.

Parity status: every function here is pinned by tests/test_oracle.py against independent formulations
(torch float64 layer_norm / scaled_dot_product_attention, explicit loops, einsum), invariants
(incoming == transposed outgoing, ending == transposed starting) and closed forms (fully masked rows,
zero masks, zero weights).
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "sub",
    "layer_norm",
    "linear",
    "sigmoid",
    "silu",
    "softmax",
    "tri_mul",
    "tri_att",
    "transition",
    "attention_pair_bias",
    "pairformer_layer",
    "pairformer_module",
    "metrics",
]


def sub(params: dict, prefix: str) -> dict:
    """The entries of `params` under `prefix.` with the prefix removed (weights.py:20-22 subtree)."""
    p = prefix.rstrip(".") + "."
    return {k[len(p):]: v for k, v in params.items() if k.startswith(p)}


def layer_norm(x, w=None, b=None, eps=1e-5):
    """Row LayerNorm over the last axis: two-pass mean/variance, (x - mean) * rsqrt(var + eps) * w + b
    (kernels.py:438-462; norm.py:8-17)."""
    # computed in the promoted type of the arguments (float32 x with float64 parameters gives float64, as
    # (x - mean) * w would)
    dt = np.result_type(x, *(a for a in (w, b) if a is not None))
    x = np.asarray(x, dtype=dt)
    mean = x.mean(axis=-1, keepdims=True)
    d = x - mean
    var = (d * d).mean(axis=-1, keepdims=True)
    # in place from here (the values equal d / sqrt(var + eps) * w + b; fewer large temporaries at N^2 rows)
    d /= np.sqrt(var + dt.type(eps))
    if w is not None:
        d *= w
    if b is not None:
        d += b
    return d


def linear(x, w, b=None):
    """nn.Linear: x @ w.T (+ b), w is [out, in]."""
    y = x @ w.T
    return y if b is None else y + b


def sigmoid(x):
    """1 / (1 + exp(-x)), evaluated in place on one temporary."""
    e = np.negative(x)
    np.exp(e, out=e)
    e += 1.0
    return np.divide(1.0, e, out=e)


def silu(x):
    return x * sigmoid(x)


def softmax(a, axis=-1):
    m = a.max(axis=axis, keepdims=True)
    e = np.subtract(a, m)
    np.exp(e, out=e)
    e /= e.sum(axis=axis, keepdims=True)
    return e


def tri_mul(x, mask, p: dict, outgoing: bool):
    """Triangle multiplication update (not the residual sum) for x [B, N, N, D], mask [B, N, N]
    (triangular_mult.py:40-65): xn = norm_in(x); a|b = (xn p_in^T) * sigmoid(xn g_in^T) * mask;
    outgoing o[i,j,d] = sum_k a[i,k,d] b[j,k,d]; incoming o[i,j,d] = sum_k a[k,i,d] b[k,j,d];
    out = p_out(norm_out(o)) * sigmoid(g_out(xn))."""
    D = p["p_out.weight"].shape[0]
    xn = layer_norm(x, p["norm_in.weight"], p["norm_in.bias"], 1e-5)
    ab = linear(xn, p["p_in.weight"])
    ab *= sigmoid(linear(xn, p["g_in.weight"]))
    ab *= mask[..., None]
    a, b = ab[..., :D], ab[..., D:]
    at = np.ascontiguousarray(a.transpose(0, 3, 1, 2))  # [B, D, N, N]
    bt = np.ascontiguousarray(b.transpose(0, 3, 1, 2))
    if outgoing:
        o = at @ bt.transpose(0, 1, 3, 2)  # [B, D, i, j] = sum_k a[d,i,k] b[d,j,k]
    else:
        o = at.transpose(0, 1, 3, 2) @ bt  # sum_k a[d,k,i] b[d,k,j]
    o = o.transpose(0, 2, 3, 1)
    g_out = sigmoid(linear(xn, p["g_out.weight"]))
    out = linear(layer_norm(o, p["norm_out.weight"], p["norm_out.bias"], 1e-5), p["p_out.weight"])
    out *= g_out
    return out


def tri_att(x, mask, p: dict, starting: bool, inf: float = 1e9, row_chunk: int = 64, rows=None):
    """Triangle attention update for x [B, I, J, C_in], mask [B, I, J] (attention.py:27-93; primitives.py:40-75).
    For row i, head h: logits[j,k] = (q[i,j]/sqrt(c)) . k[i,k] + inf*(mask[i,k]-1) + tri_bias[h,j,k],
    tri_bias = linear(xn)[j,k,h]; out = linear_o(sigmoid(g) * softmax(logits) v). The ending node runs the same
    on x and mask with the two token axes swapped and swaps the output back (attention.py:40-42, 91-92).
    Rows are processed `row_chunk` at a time (same math; bounds the [rows, H, J, K] logits). `rows` (a count)
    restricts the attention to the first `rows` rows of the (swapped) frame and returns only those, the tri bias
    still coming from every row: rows are independent, so this times a sample of a large case."""
    if mask is None:
        mask = np.ones(x.shape[:-1], dtype=x.dtype)
    if not starting:
        x = x.swapaxes(-2, -3)
        mask = mask.swapaxes(-1, -2)
    Hq = p["mha.linear_q.weight"]
    H = p["linear.weight"].shape[0]
    HC = Hq.shape[0]
    C = HC // H
    xn = layer_norm(x, p["layer_norm.weight"], p["layer_norm.bias"], 1e-5)
    B, I, J, _ = x.shape
    tri_bias = linear(xn, p["linear.weight"]).transpose(0, 3, 1, 2)  # [B, H, J, K]
    if rows is not None:
        if not starting:
            raise ValueError("a row sample is defined for the starting node's frame")
        I = min(I, int(rows))
    scale = x.dtype.type(1.0 / np.sqrt(C))
    out = np.empty((B, I, J, HC), dtype=x.dtype)
    for b in range(B):
        for i0 in range(0, I, row_chunk):
            xs = xn[b, i0:min(i0 + row_chunk, I)]  # [r, J, Cin]
            r = xs.shape[0]
            q = linear(xs, Hq).reshape(r, J, H, C).transpose(0, 2, 1, 3) * scale
            k = linear(xs, p["mha.linear_k.weight"]).reshape(r, J, H, C).transpose(0, 2, 1, 3)
            v = linear(xs, p["mha.linear_v.weight"]).reshape(r, J, H, C).transpose(0, 2, 1, 3)
            g = sigmoid(linear(xs, p["mha.linear_g.weight"]))  # [r, J, HC]
            a = q @ k.transpose(0, 1, 3, 2)  # [r, H, J, K]
            a = a + (x.dtype.type(inf) * (mask[b, i0:i0 + r] - 1))[:, None, None, :]
            a = a + tri_bias[b][None]
            o = softmax(a, -1) @ v  # [r, H, J, C]
            out[b, i0:i0 + r] = o.transpose(0, 2, 1, 3).reshape(r, J, HC) * g
    y = linear(out, p["mha.linear_o.weight"])
    if not starting:
        y = y.swapaxes(-2, -3)
    return y


def transition(x, p: dict):
    """SwiGLU transition fc3(silu(fc1(LN(x))) * fc2(LN(x))) (transition.py:27-54, 148-154)."""
    xn = layer_norm(x, p["norm.weight"], p["norm.bias"], 1e-5)
    return linear(silu(linear(xn, p["fc1.weight"])) * linear(xn, p["fc2.weight"]), p["fc3.weight"])


def attention_pair_bias(s, z, mask, k_in, p: dict, num_heads: int, inf: float = 1e6):
    """AttentionPairBias v2 (attentionv2.py:43-86): q = proj_q(s) (biased), k, v from k_in; bias = proj_z(z) =
    Linear(LN(z)) as [B, H, N, N]; logits = q k^T / sqrt(hd) + bias + (1 - mask) * (-inf);
    y = proj_o(sigmoid(proj_g(s)) * softmax(logits) v)."""
    B, N, Cs = s.shape
    H = num_heads
    hd = Cs // H
    q = linear(s, p["proj_q.weight"], p["proj_q.bias"]).reshape(B, N, H, hd).transpose(0, 2, 1, 3)
    k = linear(k_in, p["proj_k.weight"]).reshape(B, N, H, hd).transpose(0, 2, 3, 1)
    v = linear(k_in, p["proj_v.weight"]).reshape(B, N, H, hd).transpose(0, 2, 1, 3)
    bias = linear(layer_norm(z, p["proj_z.0.weight"], p["proj_z.0.bias"], 1e-5), p["proj_z.1.weight"])
    bias = bias.transpose(0, 3, 1, 2)  # [B, H, N, N]
    g = sigmoid(linear(s, p["proj_g.weight"]))
    a = (q @ k) / s.dtype.type(hd ** 0.5) + bias
    a = a + (1 - mask[:, None, None, :].astype(s.dtype)) * s.dtype.type(-inf)
    o = (softmax(a, -1) @ v).transpose(0, 2, 1, 3).reshape(B, N, Cs)
    return linear(g * o, p["proj_o.weight"])


def pairformer_layer(s, z, mask, pair_mask, p: dict, num_heads: int = 16):
    """One PairformerLayer (pairformer.py:59-94 strict path): five residual pair updates in order, then the
    s track (pre_norm_s, AttentionPairBias with k_in = pre_norm_s(s), transition_s); s_post_norm = Identity."""
    z = z + tri_mul(z, pair_mask, sub(p, "tri_mul_out"), True)
    z = z + tri_mul(z, pair_mask, sub(p, "tri_mul_in"), False)
    z = z + tri_att(z, pair_mask, sub(p, "tri_att_start"), True)
    z = z + tri_att(z, pair_mask, sub(p, "tri_att_end"), False)
    z = z + transition(z, sub(p, "transition_z"))
    s_n = layer_norm(s, p["pre_norm_s.weight"], p["pre_norm_s.bias"], 1e-5)
    s = s + attention_pair_bias(s_n, z, mask, s_n, sub(p, "attention"), num_heads)
    s = s + transition(s, sub(p, "transition_s"))
    return s, z


def pairformer_module(s, z, mask, pair_mask, p: dict, num_blocks: int, num_heads: int = 16):
    """PairformerModule: num_blocks layers in sequence (pairformer.py:135-153), params under ``layers.{i}.``."""
    for i in range(num_blocks):
        s, z = pairformer_layer(s, z, mask, pair_mask, sub(p, f"layers.{i}"), num_heads)
    return s, z


def metrics(ours, ref) -> dict:
    """Parity metrics in float64 (compare.py:14-34): max_abs, max_rel = max|d| / max|ref|, cosine, and
    rel_fro = ||d||_F / ||ref||_F."""
    a = np.asarray(ours, dtype=np.float64)
    b = np.asarray(ref, dtype=np.float64)
    if a.shape != b.shape:
        raise ValueError(f"shape mismatch {a.shape} vs {b.shape}")
    d = np.abs(a - b)
    scale = max(float(np.abs(b).max(initial=0.0)), 1e-12)
    na, nb = np.linalg.norm(a), np.linalg.norm(b)
    cos = float(a.ravel() @ b.ravel() / (na * nb)) if na * nb > 0 else (1.0 if d.max(initial=0) == 0 else 0.0)
    return {
        "max_abs": float(d.max(initial=0.0)),
        "max_rel": float(d.max(initial=0.0) / scale),
        "rel_fro": float(np.linalg.norm(d) / max(nb, 1e-300)),
        "cos": cos,
        "finite": bool(np.isfinite(a).all()),
    }
