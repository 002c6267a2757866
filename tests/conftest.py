"""Shared test helpers: the `gpu` marker, the reference's parameter layout and seeded inputs.

The parameter names and shapes below are the reference checkpoint layout of one PairformerLayer
(nn.Linear.weight is [out, in]; boltz_mlx/layers/pairformer.py:23-57, triangular_mult.py:10-17,
triangular_attention/attention.py:15-25 with primitives.py:20-38, transition.py:15-25, attentionv2.py:15-41).
"""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C-ABI library)")


# ----------------------------------------------------------------------------------------------------------------
# reference parameter layout
# ----------------------------------------------------------------------------------------------------------------

def shapes_tri_mul(D: int) -> dict:
    return {
        "norm_in.weight": (D,), "norm_in.bias": (D,),
        "p_in.weight": (2 * D, D), "g_in.weight": (2 * D, D),
        "norm_out.weight": (D,), "norm_out.bias": (D,),
        "p_out.weight": (D, D), "g_out.weight": (D, D),
    }


def shapes_tri_att(c_in: int, c_hidden: int, heads: int) -> dict:
    hc = c_hidden * heads
    return {
        "layer_norm.weight": (c_in,), "layer_norm.bias": (c_in,),
        "linear.weight": (heads, c_in),
        "mha.linear_q.weight": (hc, c_in), "mha.linear_k.weight": (hc, c_in),
        "mha.linear_v.weight": (hc, c_in), "mha.linear_o.weight": (c_in, hc),
        "mha.linear_g.weight": (hc, c_in),
    }


def shapes_transition(dim: int, hidden: int) -> dict:
    return {
        "norm.weight": (dim,), "norm.bias": (dim,),
        "fc1.weight": (hidden, dim), "fc2.weight": (hidden, dim), "fc3.weight": (dim, hidden),
    }


def shapes_attention(c_s: int, c_z: int, heads: int) -> dict:
    return {
        "proj_q.weight": (c_s, c_s), "proj_q.bias": (c_s,),
        "proj_k.weight": (c_s, c_s), "proj_v.weight": (c_s, c_s), "proj_g.weight": (c_s, c_s),
        "proj_z.0.weight": (c_z,), "proj_z.0.bias": (c_z,), "proj_z.1.weight": (heads, c_z),
        "proj_o.weight": (c_s, c_s),
    }


def _prefixed(prefix: str, d: dict) -> dict:
    return {f"{prefix}.{k}": v for k, v in d.items()}


def shapes_layer(token_s: int, token_z: int, heads: int = 16, pw: int = 32, pheads: int = 4) -> dict:
    out = {"pre_norm_s.weight": (token_s,), "pre_norm_s.bias": (token_s,)}
    out.update(_prefixed("attention", shapes_attention(token_s, token_z, heads)))
    out.update(_prefixed("tri_mul_out", shapes_tri_mul(token_z)))
    out.update(_prefixed("tri_mul_in", shapes_tri_mul(token_z)))
    out.update(_prefixed("tri_att_start", shapes_tri_att(token_z, pw, pheads)))
    out.update(_prefixed("tri_att_end", shapes_tri_att(token_z, pw, pheads)))
    out.update(_prefixed("transition_s", shapes_transition(token_s, 4 * token_s)))
    out.update(_prefixed("transition_z", shapes_transition(token_z, 4 * token_z)))
    return out


def shapes_adaln(dim: int, dim_cond: int) -> dict:
    return {"s_norm.weight": (dim_cond,), "s_scale.weight": (dim, dim_cond), "s_scale.bias": (dim,),
            "s_bias.weight": (dim, dim_cond)}


def shapes_diffusion_layer(dim: int, dim_cond: int | None = None, expansion: int = 2) -> dict:
    """One DiffusionTransformerLayer (transformersv2.py:69-86). The output projection is one Linear registered under
    two names (output_projection_linear and output_projection.0); only the first is listed here, and
    with_shared_alias() adds the second with the same values."""
    dc = dim if dim_cond is None else dim_cond
    inner = dim * expansion
    out = _prefixed("adaln", shapes_adaln(dim, dc))
    out.update(_prefixed("pair_bias_attn", {
        "proj_q.weight": (dim, dim), "proj_q.bias": (dim,), "proj_k.weight": (dim, dim),
        "proj_v.weight": (dim, dim), "proj_g.weight": (dim, dim), "proj_o.weight": (dim, dim)}))
    out.update({"output_projection_linear.weight": (dim, dc), "output_projection_linear.bias": (dim,)})
    out.update(_prefixed("transition.adaln", shapes_adaln(dim, dc)))
    out.update({"transition.swish_gate.0.weight": (2 * inner, dim), "transition.a_to_b.weight": (inner, dim),
                "transition.b_to_a.weight": (dim, inner), "transition.output_projection.0.weight": (dim, dc),
                "transition.output_projection.0.bias": (dim,)})
    return out


def shapes_opm(c_in: int = 64, c_hidden: int = 32, c_out: int = 128) -> dict:
    """OuterProductMean (outer_product_mean.py:15-21)."""
    return {"norm.weight": (c_in,), "norm.bias": (c_in,), "proj_a.weight": (c_hidden, c_in),
            "proj_b.weight": (c_hidden, c_in), "proj_o.weight": (c_out, c_hidden * c_hidden), "proj_o.bias": (c_out,)}


def shapes_pwa(c_m: int = 64, c_z: int = 128, c_h: int = 32, heads: int = 8) -> dict:
    """PairWeightedAveraging (pair_averaging.py:13-28)."""
    return {"norm_m.weight": (c_m,), "norm_m.bias": (c_m,), "norm_z.weight": (c_z,), "norm_z.bias": (c_z,),
            "proj_m.weight": (c_h * heads, c_m), "proj_g.weight": (c_h * heads, c_m), "proj_z.weight": (heads, c_z),
            "proj_o.weight": (c_m, c_h * heads)}


def shapes_noseq_layer(token_z: int, pw: int = 32, pheads: int = 4) -> dict:
    out = {}
    out.update(_prefixed("tri_mul_out", shapes_tri_mul(token_z)))
    out.update(_prefixed("tri_mul_in", shapes_tri_mul(token_z)))
    out.update(_prefixed("tri_att_start", shapes_tri_att(token_z, pw, pheads)))
    out.update(_prefixed("tri_att_end", shapes_tri_att(token_z, pw, pheads)))
    out.update(_prefixed("transition_z", shapes_transition(token_z, 4 * token_z)))
    return out


def shapes_msa_layer(msa_s: int = 64, token_z: int = 128) -> dict:
    """MSALayer (trunkv2.py:205-227)."""
    out = {}
    out.update(_prefixed("msa_transition", shapes_transition(msa_s, 4 * msa_s)))
    out.update(_prefixed("pair_weighted_averaging", shapes_pwa(msa_s, token_z)))
    out.update(_prefixed("pairformer_layer", shapes_noseq_layer(token_z)))
    out.update(_prefixed("outer_product_mean", shapes_opm(msa_s, 32, token_z)))
    return out


def with_shared_alias(params: dict) -> dict:
    """Adds `...output_projection.0.*` = `...output_projection_linear.*` (the shared Linear's second name)."""
    out = dict(params)
    for k, v in params.items():
        if "output_projection_linear." in k:
            out[k.replace("output_projection_linear.", "output_projection.0.")] = v
    return out


def rand_params(shapes: dict, seed: int, std: float = 0.02, ln_random: bool = True,
                dtype=np.float64) -> dict:
    """Seeded parameters in sorted-name order: matrices and biases ~ N(0, std); LayerNorm weights
    1 + N(0, 0.1) and biases N(0, 0.1) when `ln_random` (so a swapped or dropped affine term shows), else 1 / 0."""
    rng = np.random.default_rng(seed)
    out = {}
    for name in sorted(shapes):
        shp = shapes[name]
        is_ln = len(shp) == 1 and not name.endswith("proj_q.bias")
        if is_ln and name.endswith("weight"):
            v = 1.0 + 0.1 * rng.standard_normal(shp) if ln_random else np.ones(shp)
        elif is_ln:
            v = 0.1 * rng.standard_normal(shp) if ln_random else np.zeros(shp)
        else:
            v = std * rng.standard_normal(shp)
        out[name] = v.astype(dtype)
    return out


def pair_inputs(N: int, D: int, seed: int, n_pad: int = 0, B: int = 1, dtype=np.float64):
    """z ~ N(0,1) [B, N, N, D]; token mask with the last n_pad tokens padded; pair_mask = tok_i * tok_j
    (the trunk's mask construction, model.py:171-172)."""
    rng = np.random.default_rng(seed)
    z = rng.standard_normal((B, N, N, D)).astype(dtype)
    tok = np.ones((B, N), dtype=dtype)
    if n_pad:
        tok[:, N - n_pad:] = 0
    pm = tok[:, :, None] * tok[:, None, :]
    return z, tok, pm


@pytest.fixture
def rng():
    return np.random.default_rng(1234)
