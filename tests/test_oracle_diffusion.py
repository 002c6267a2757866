"""Pins the diffusion-transformer oracle (oracle/diffusion.py) against independent torch float64 formulations,
the fast-path algebra (conditioning folded and precomputed for all layers) and closed forms.

The torch references below are written from torch.nn.functional (layer_norm, silu, scaled_dot_product_attention)
rather than from the oracle's helpers, so a dropped term, a swapped SwiGLU half, a wrong bias slice or a missing
gate in either would show.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import rand_params, shapes_diffusion_layer
from oracle import diffusion as OD


def T(x):
    return torch.from_numpy(np.asarray(x, dtype=np.float64))


def _sub(p, prefix):
    return {k[len(prefix) + 1:]: v for k, v in p.items() if k.startswith(prefix + ".")}


def _torch_adaln(a, s, p):
    D, Ds = a.shape[-1], s.shape[-1]
    an = F.layer_norm(a, (D,), None, None, 1e-5)
    sn = F.layer_norm(s, (Ds,), T(p["s_norm.weight"]), None, 1e-5)
    return torch.sigmoid(F.linear(sn, T(p["s_scale.weight"]), T(p["s_scale.bias"]))) * an + F.linear(
        sn, T(p["s_bias.weight"]))


def _torch_transition(a, s, p):
    a = _torch_adaln(a, s, _sub(p, "adaln"))
    x, gates = torch.chunk(F.linear(a, T(p["swish_gate.0.weight"])), 2, dim=-1)
    b = F.silu(gates) * x * F.linear(a, T(p["a_to_b.weight"]))
    gate = torch.sigmoid(F.linear(s, T(p["output_projection.0.weight"]), T(p["output_projection.0.bias"])))
    return gate * F.linear(b, T(p["b_to_a.weight"]))


def _torch_attention(x, bias, mask, p, H, mult):
    Bm, N, D = x.shape
    hd = D // H
    q = F.linear(x, T(p["proj_q.weight"]), T(p["proj_q.bias"])).view(Bm, N, H, hd).transpose(1, 2)
    k = F.linear(x, T(p["proj_k.weight"])).view(Bm, N, H, hd).transpose(1, 2)
    v = F.linear(x, T(p["proj_v.weight"])).view(Bm, N, H, hd).transpose(1, 2)
    outs = []
    for b in range(Bm):
        m = bias[b // mult].permute(2, 0, 1) + (1 - mask[b])[None, None, :] * -1e6
        outs.append(F.scaled_dot_product_attention(q[b:b + 1], k[b:b + 1], v[b:b + 1], attn_mask=m[None]))
    o = torch.cat(outs, 0).transpose(1, 2).reshape(Bm, N, D)
    g = torch.sigmoid(F.linear(x, T(p["proj_g.weight"])))
    return F.linear(g * o, T(p["proj_o.weight"]))


def _torch_layer(a, s, bias, mask, p, H, mult):
    b = _torch_adaln(a, s, _sub(p, "adaln"))
    b = _torch_attention(b, bias, mask, _sub(p, "pair_bias_attn"), H, mult)
    a = a + torch.sigmoid(F.linear(s, T(p["output_projection_linear.weight"]),
                                   T(p["output_projection_linear.bias"]))) * b
    return a + _torch_transition(a, s, _sub(p, "transition"))


def _inputs(B, mult, N, D, H, seed):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((B * mult, N, D))
    s = rng.standard_normal((B * mult, N, D))
    bias = rng.standard_normal((B, N, N, H))
    mask = np.ones((B * mult, N))
    mask[:, -2:] = 0
    return a, s, bias, mask


def test_adaln_vs_torch():
    D = 64
    p = _sub(rand_params(shapes_diffusion_layer(D), seed=1, std=0.2), "adaln")
    a, s, _, _ = _inputs(1, 1, 5, D, 4, 2)
    ref = _torch_adaln(T(a), T(s), p).numpy()
    assert np.abs(OD.adaln(a, s, p) - ref).max() < 1e-12


def test_conditioned_transition_vs_torch_and_gate_half():
    D = 64
    p = _sub(rand_params(shapes_diffusion_layer(D), seed=3, std=0.2), "transition")
    a, s, _, _ = _inputs(1, 1, 6, D, 4, 4)
    ref = _torch_transition(T(a), T(s), p).numpy()
    got = OD.conditioned_transition(a, s, p)
    assert np.abs(got - ref).max() < 1e-12
    # silu acts on the second half of swish_gate (the gates): swapping the halves must change the result
    w = p["swish_gate.0.weight"]
    q = dict(p, **{"swish_gate.0.weight": np.concatenate([w[w.shape[0] // 2:], w[:w.shape[0] // 2]], 0)})
    assert np.abs(OD.conditioned_transition(a, s, q) - got).max() > 1e-3


@pytest.mark.parametrize("mult", [1, 2])
def test_pair_bias_attention_vs_sdpa(mult):
    D, H = 64, 4
    p = _sub(rand_params(shapes_diffusion_layer(D), seed=5, std=0.3), "pair_bias_attn")
    a, _, bias, mask = _inputs(2, mult, 7, D, H, 6)
    ref = _torch_attention(T(a), T(bias), T(mask), p, H, mult).numpy()
    assert np.abs(OD.pair_bias_attention(a, bias, mask, a, p, H, mult) - ref).max() < 1e-12


@pytest.mark.parametrize("mult", [1, 2])
def test_diffusion_layer_vs_torch(mult):
    D, H = 64, 4
    p = rand_params(shapes_diffusion_layer(D), seed=7, std=0.2)
    a, s, bias, mask = _inputs(1, mult, 6, D, H, 8)
    ref = _torch_layer(T(a), T(s), T(bias), T(mask), p, H, mult).numpy()
    assert np.abs(OD.diffusion_layer(a, s, bias, mask, p, H, mult) - ref).max() < 1e-12


def test_layer_closed_forms():
    """Zero b_to_a: no transition update, the layer is a + gate * attention. Zero proj_o as well: the layer is the
    identity."""
    D, H = 64, 4
    p = rand_params(shapes_diffusion_layer(D), seed=9, std=0.2)
    a, s, bias, mask = _inputs(1, 1, 5, D, H, 10)
    p0 = dict(p, **{"transition.b_to_a.weight": np.zeros_like(p["transition.b_to_a.weight"])})
    gate = OD.sigmoid(OD.linear(s, p["output_projection_linear.weight"], p["output_projection_linear.bias"]))
    b = OD.adaln(a, s, _sub(p, "adaln"))
    att = OD.pair_bias_attention(b, bias, mask, b, _sub(p, "pair_bias_attn"), H)
    assert np.abs(OD.diffusion_layer(a, s, bias, mask, p0, H) - (a + gate * att)).max() < 1e-12
    p00 = dict(p0, **{"pair_bias_attn.proj_o.weight": np.zeros_like(p["pair_bias_attn.proj_o.weight"])})
    assert np.abs(OD.diffusion_layer(a, s, bias, mask, p00, H) - a).max() == 0


@pytest.mark.parametrize("mult", [1, 3])
def test_fast_path_equals_module_path(mult):
    """The precomputed conditioning with the s_norm weight folded into the linears (what the GPU path runs) equals
    the module path layer by layer, and the bias [B, N, M, L * H] is split per layer in the reference's order."""
    D, H, L = 64, 4, 3
    p = {}
    for i in range(L):
        p.update({f"layers.{i}.{k}": v for k, v in rand_params(shapes_diffusion_layer(D), seed=20 + i, std=0.2).items()})
    a, s, _, mask = _inputs(1, mult, 6, D, H, 11)
    bias = np.random.default_rng(12).standard_normal((1, 6, 6, L * H))
    ref = OD.diffusion_transformer(a, s, bias, mask, p, L, H, mult)
    h1, h2 = OD.precompute_cond(s, p, L)
    x = a
    for i in range(L):
        x = OD.diffusion_layer_fast(x, h1[..., i, :, :], h2[..., i, :, :], bias[..., i * H:(i + 1) * H], mask,
                                    _sub(p, f"layers.{i}"), H, mult)
    assert np.abs(x - ref).max() < 1e-10
    # a different split of the bias (heads interleaved across layers) must not match
    wrong = bias.reshape(1, 6, 6, H, L).transpose(0, 1, 2, 4, 3).reshape(1, 6, 6, L * H)
    assert np.abs(OD.diffusion_transformer(a, s, wrong, mask, p, L, H, mult) - ref).max() > 1e-4
