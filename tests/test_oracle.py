"""Pins the CPU oracle (oracle/pairformer.py) against independent formulations, invariants and closed forms.

Nothing here retypes the oracle's formulas: LayerNorm is checked against torch's layer_norm, attention against
torch's scaled_dot_product_attention and explicit per-element loops, the triangle contraction against einsum and
loops, and each module against invariants (transposition symmetry, masks, zero weights) that a dropped term,
a wrong sign/index or a transposed operand would break.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from conftest import (pair_inputs, rand_params, shapes_attention, shapes_layer, shapes_transition,
                      shapes_tri_att, shapes_tri_mul)




def T(x):
    return torch.from_numpy(np.asarray(x, dtype=np.float64))


# ---------------------------------------------------------------- LayerNorm

@pytest.mark.parametrize("D", [32, 128, 384])
def test_layer_norm_vs_torch(D):
    rng = np.random.default_rng(D)
    x = rng.standard_normal((7, D)) * 3 + 1.5
    w, b = 1 + 0.1 * rng.standard_normal(D), 0.1 * rng.standard_normal(D)
    ref = F.layer_norm(T(x), (D,), T(w), T(b), 1e-5).numpy()
    assert np.abs(O.layer_norm(x, w, b, 1e-5) - ref).max() < 1e-12


def test_layer_norm_invariants():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 128))
    y = O.layer_norm(x)
    assert np.abs(y.mean(-1)).max() < 1e-12
    assert np.abs((y * y).mean(-1) - 1).max() < 1e-3  # var / (var + eps)
    # LN(c x) with eps c^2 == LN(x) with eps (the power-of-two pre-scale trick, norm.py:12-17)
    c = 2.0 ** -8
    assert np.abs(O.layer_norm(c * x, eps=1e-5 * c * c) - y).max() < 1e-12
    # a zero row normalises to the bias
    b = rng.standard_normal(128)
    assert np.abs(O.layer_norm(np.zeros((1, 128)), None, b) - b).max() == 0


# ---------------------------------------------------------------- triangle multiplication

def _tri_mul_loops(x, mask, p, outgoing):
    """Per-element loops over (i, j, d, k) for the contraction; torch for LN/linear."""
    D = p["p_out.weight"].shape[0]
    xt = T(x[0])
    xn = F.layer_norm(xt, (D,), T(p["norm_in.weight"]), T(p["norm_in.bias"]), 1e-5)
    ab = (xn @ T(p["p_in.weight"]).T) * torch.sigmoid(xn @ T(p["g_in.weight"]).T) * T(mask[0])[..., None]
    a, b = ab[..., :D].numpy(), ab[..., D:].numpy()
    N = x.shape[1]
    o = np.zeros((N, N, D))
    for i in range(N):
        for j in range(N):
            for d in range(D):
                s = 0.0
                for k in range(N):
                    s += a[i, k, d] * b[j, k, d] if outgoing else a[k, i, d] * b[k, j, d]
                o[i, j, d] = s
    on = F.layer_norm(T(o), (D,), T(p["norm_out.weight"]), T(p["norm_out.bias"]), 1e-5)
    return ((on @ T(p["p_out.weight"]).T) * torch.sigmoid(xn @ T(p["g_out.weight"]).T)).numpy()[None]


@pytest.mark.parametrize("outgoing", [True, False])
def test_tri_mul_vs_loops(outgoing):
    D, N = 8, 5
    p = rand_params(shapes_tri_mul(D), seed=3)
    x, _, pm = pair_inputs(N, D, seed=4, n_pad=1)
    pm[0, 1, 2] = 0  # an asymmetric hole: a transposed mask would show
    ref = _tri_mul_loops(x, pm, p, outgoing)
    assert np.abs(O.tri_mul(x, pm, p, outgoing) - ref).max() < 1e-12


def test_tri_mul_einsum_and_symmetry():
    D, N = 16, 9
    p = rand_params(shapes_tri_mul(D), seed=5)
    x, _, pm = pair_inputs(N, D, seed=6, n_pad=2)
    pm[0, 3, 4] = 0
    out = O.tri_mul(x, pm, p, True)
    inc = O.tri_mul(x, pm, p, False)
    # The contractions satisfy o_in(x, m)[i, j] = o_out(x^T, m^T)[i, j]; the output gate reads xn at the
    # un-transposed position, so with a constant gate (g_out = 0) incoming(x, m) == outgoing(x^T, m^T).
    q = dict(p)
    q["g_out.weight"] = np.zeros_like(p["g_out.weight"])
    inc2 = O.tri_mul(x, pm, q, False)
    out2 = O.tri_mul(x.swapaxes(1, 2), pm.swapaxes(1, 2), q, True)
    assert np.abs(inc2 - out2).max() < 1e-12
    assert np.abs(inc2 - out2.swapaxes(1, 2)).max() > 1e-3  # and not its transpose
    assert np.abs(out - inc).max() > 1e-3  # the two directions differ on a non-symmetric input
    # einsum form of the outgoing contraction
    xn = O.layer_norm(x, p["norm_in.weight"], p["norm_in.bias"])
    ab = (xn @ p["p_in.weight"].T) * O.sigmoid(xn @ p["g_in.weight"].T) * pm[..., None]
    o = np.einsum("bikd,bjkd->bijd", ab[..., :D], ab[..., D:])
    ref = O.layer_norm(o, p["norm_out.weight"], p["norm_out.bias"]) @ p["p_out.weight"].T
    ref = ref * O.sigmoid(xn @ p["g_out.weight"].T)
    assert np.abs(out - ref).max() < 1e-12


def test_tri_mul_zero_mask_closed_form():
    D, N = 16, 6
    p = rand_params(shapes_tri_mul(D), seed=7)
    x, _, _ = pair_inputs(N, D, seed=8)
    pm = np.zeros((1, N, N))
    xn = O.layer_norm(x, p["norm_in.weight"], p["norm_in.bias"])
    # o = 0 -> norm_out(0) = norm_out.bias
    ref = (p["norm_out.bias"] @ p["p_out.weight"].T) * O.sigmoid(xn @ p["g_out.weight"].T)
    for outgoing in (True, False):
        assert np.abs(O.tri_mul(x, pm, p, outgoing) - ref).max() < 1e-12


# ---------------------------------------------------------------- triangle attention

def _tri_att_sdpa(x, mask, p, starting, inf=1e9):
    """torch SDPA with the explicit additive mask (tri bias + key mask bias)."""
    if not starting:
        x = x.swapaxes(1, 2)
        mask = mask.swapaxes(1, 2)
    H = p["linear.weight"].shape[0]
    HC = p["mha.linear_q.weight"].shape[0]
    C = HC // H
    xt = T(x[0])
    I, J, Cin = xt.shape
    xn = F.layer_norm(xt, (Cin,), T(p["layer_norm.weight"]), T(p["layer_norm.bias"]), 1e-5)

    def heads(w):
        return (xn @ T(p[w]).T).reshape(I, J, H, C).permute(0, 2, 1, 3)

    q, k, v = heads("mha.linear_q.weight"), heads("mha.linear_k.weight"), heads("mha.linear_v.weight")
    tb = (xn @ T(p["linear.weight"]).T).permute(2, 0, 1)  # [H, J, K]
    mb = inf * (T(mask[0]) - 1)  # [I, K]
    bias = mb[:, None, None, :] + tb[None]
    o = F.scaled_dot_product_attention(q, k, v, attn_mask=bias, scale=C ** -0.5)
    o = o.permute(0, 2, 1, 3).reshape(I, J, HC) * torch.sigmoid(xn @ T(p["mha.linear_g.weight"]).T)
    y = (o @ T(p["mha.linear_o.weight"]).T).numpy()[None]
    return y.swapaxes(1, 2) if not starting else y


@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("N", [1, 2, 9, 17])
def test_tri_att_vs_sdpa(starting, N):
    p = rand_params(shapes_tri_att(32, 8, 3), seed=11, std=0.3)
    x, _, pm = pair_inputs(N, 32, seed=N, n_pad=N // 4)
    if N > 3:
        pm[0, 1, 2] = 0
    ref = _tri_att_sdpa(x, pm, p, starting)
    got = O.tri_att(x, pm, p, starting, row_chunk=4)
    assert np.abs(got - ref).max() < 1e-11


def test_tri_att_loops_tiny():
    """Explicit per-logit loops with the reference's summation order ((q/sqrt c).k + mask_bias) + tri_bias."""
    N, Cin, C, H = 4, 8, 2, 2
    p = rand_params(shapes_tri_att(Cin, C, H), seed=12, std=0.5)
    x, _, pm = pair_inputs(N, Cin, seed=13)
    pm[0, 0, 3] = 0
    pm[0, 2, :] = 0  # a fully masked row
    xn = O.layer_norm(x[0], p["layer_norm.weight"], p["layer_norm.bias"])
    q = xn @ p["mha.linear_q.weight"].T
    k = xn @ p["mha.linear_k.weight"].T
    v = xn @ p["mha.linear_v.weight"].T
    g = xn @ p["mha.linear_g.weight"].T
    tb = xn @ p["linear.weight"].T
    o = np.zeros((N, N, H * C))
    for i in range(N):
        for h in range(H):
            for j in range(N):
                lg = []
                for kk in range(N):
                    s = sum((q[i, j, h * C + c] / np.sqrt(C)) * k[i, kk, h * C + c] for c in range(C))
                    lg.append((s + 1e9 * (pm[0, i, kk] - 1)) + tb[j, kk, h])
                lg = np.array(lg)
                w = np.exp(lg - lg.max())
                w /= w.sum()
                for c in range(C):
                    o[i, j, h * C + c] = (w * v[i, :, h * C + c]).sum() / (1 + np.exp(-g[i, j, h * C + c]))
    ref = o @ p["mha.linear_o.weight"].T
    assert np.abs(O.tri_att(x, pm, p, True)[0] - ref).max() < 1e-12


def test_tri_att_symmetry_and_masks():
    N, Cin, C, H = 12, 32, 8, 4
    p = rand_params(shapes_tri_att(Cin, C, H), seed=14, std=0.3)
    x, _, pm = pair_inputs(N, Cin, seed=15, n_pad=3)
    pm[0, 2, 5] = 0
    end = O.tri_att(x, pm, p, False)
    end2 = O.tri_att(x.swapaxes(1, 2), pm.swapaxes(1, 2), p, True).swapaxes(1, 2)
    assert np.abs(end - end2).max() < 1e-12
    start = O.tri_att(x, pm, p, True)
    assert np.abs(start - end).max() > 1e-3
    # fully masked row i (padded token): every logit rounds to -1e9 in the reference order -> uniform weights
    # (in float64 the logits differ by the O(1) terms, so compare in float32 like the reference)
    x32, pm32 = x.astype(np.float32), pm.astype(np.float32)
    p32 = {k: v.astype(np.float32) for k, v in p.items()}
    out32 = O.tri_att(x32, pm32, p32, True)
    i = N - 1
    xn = O.layer_norm(x32[0, i], p32["layer_norm.weight"], p32["layer_norm.bias"])
    v = xn @ p32["mha.linear_v.weight"].T  # [K, HC]
    g = O.sigmoid(xn @ p32["mha.linear_g.weight"].T)  # [J, HC]
    closed = (g * v.mean(0)[None]) @ p32["mha.linear_o.weight"].T
    assert np.abs(out32[0, i] - closed).max() < 1e-5
    # masked keys get exactly zero weight in rows with some unmasked key: perturbing x at a masked key changes
    # only that key's own query/gate terms, so compare a query column that is unchanged
    x2 = x.copy()
    x2[0, 0, N - 1] += 5.0  # row 0, key N-1 is masked (padded token)
    a = O.tri_att(x, pm, p, True)[0, 0, : N - 1]
    b = O.tri_att(x2, pm, p, True)[0, 0, : N - 1]
    # the tri bias of pair (0, N-1) feeds only queries j=0 (bias[h, 0, N-1]) on masked key N-1: weight 0 anyway
    assert np.abs(a - b).max() < 1e-12


def test_tri_att_row_sample():
    """The row sample used to time large cases is the first rows of the full result (rows are independent; the tri
    bias comes from every row)."""
    p = rand_params(shapes_tri_att(16, 4, 2), seed=16, std=0.3)
    x, _, pm = pair_inputs(11, 16, seed=17, n_pad=2)
    full = O.tri_att(x, pm, p, True, row_chunk=4)
    part = O.tri_att(x, pm, p, True, row_chunk=4, rows=6)
    assert part.shape == (1, 6, 11, 16)
    assert np.abs(part - full[:, :6]).max() < 1e-13


# ---------------------------------------------------------------- transition

def test_transition_vs_torch():
    rng = np.random.default_rng(20)
    p = rand_params(shapes_transition(16, 64), seed=21, std=0.2)
    x = rng.standard_normal((3, 5, 16))
    xn = F.layer_norm(T(x), (16,), T(p["norm.weight"]), T(p["norm.bias"]), 1e-5)
    ref = F.linear(F.silu(F.linear(xn, T(p["fc1.weight"]))) * F.linear(xn, T(p["fc2.weight"])), T(p["fc3.weight"]))
    got = O.transition(x, p)
    assert np.abs(got - ref.numpy()).max() < 1e-13
    # the SiLU branch is fc1: swapping fc1 / fc2 changes the result
    q = dict(p)
    q["fc1.weight"], q["fc2.weight"] = p["fc2.weight"], p["fc1.weight"]
    assert np.abs(O.transition(x, q) - got).max() > 1e-3


# ---------------------------------------------------------------- attention with pair bias (s track)

def test_attention_pair_bias_vs_sdpa():
    B, N, Cs, Cz, H = 1, 11, 48, 16, 4
    p = rand_params(shapes_attention(Cs, Cz, H), seed=30, std=0.2)
    rng = np.random.default_rng(31)
    s = rng.standard_normal((B, N, Cs))
    z = rng.standard_normal((B, N, N, Cz))
    mask = np.ones((B, N))
    mask[:, -3:] = 0
    got = O.attention_pair_bias(s, z, mask, s, p, H)
    st, zt = T(s), T(z)
    hd = Cs // H
    q = F.linear(st, T(p["proj_q.weight"]), T(p["proj_q.bias"])).reshape(B, N, H, hd).transpose(1, 2)
    k = F.linear(st, T(p["proj_k.weight"])).reshape(B, N, H, hd).transpose(1, 2)
    v = F.linear(st, T(p["proj_v.weight"])).reshape(B, N, H, hd).transpose(1, 2)
    zb = F.linear(F.layer_norm(zt, (Cz,), T(p["proj_z.0.weight"]), T(p["proj_z.0.bias"]), 1e-5), T(p["proj_z.1.weight"]))
    bias = zb.permute(0, 3, 1, 2) + (1 - T(mask))[:, None, None, :] * -1e6
    o = F.scaled_dot_product_attention(q, k, v, attn_mask=bias).transpose(1, 2).reshape(B, N, Cs)
    ref = F.linear(torch.sigmoid(F.linear(st, T(p["proj_g.weight"]))) * o, T(p["proj_o.weight"]))
    assert np.abs(got - ref.numpy()).max() < 1e-12


# ---------------------------------------------------------------- layer / module

def test_layer_zero_weights_identity():
    p = rand_params(shapes_layer(48, 32, heads=4, pw=8, pheads=2), seed=40)
    for k in p:
        if p[k].ndim == 2 or k.endswith("proj_q.bias"):
            p[k] = np.zeros_like(p[k])
    z, tok, pm = pair_inputs(6, 32, seed=41, n_pad=1)
    s = np.random.default_rng(42).standard_normal((1, 6, 48))
    s2, z2 = O.pairformer_layer(s, z, tok, pm, p, num_heads=4)
    assert np.array_equal(z2, z) and np.array_equal(s2, s)


PAIR_MODULES = ("tri_mul_out", "tri_mul_in", "tri_att_start", "tri_att_end", "transition_z")


def _tri_mul_torch(x, mask, p, outgoing):
    """torch einsum form of a triangle multiplication (float64)."""
    D = p["p_out.weight"].shape[0]
    xt = T(x[0])
    xn = F.layer_norm(xt, (D,), T(p["norm_in.weight"]), T(p["norm_in.bias"]), 1e-5)
    ab = (xn @ T(p["p_in.weight"]).T) * torch.sigmoid(xn @ T(p["g_in.weight"]).T) * T(mask[0])[..., None]
    a, b = ab[..., :D], ab[..., D:]
    o = torch.einsum("ikd,jkd->ijd", a, b) if outgoing else torch.einsum("kid,kjd->ijd", a, b)
    on = F.layer_norm(o, (D,), T(p["norm_out.weight"]), T(p["norm_out.bias"]), 1e-5)
    return ((on @ T(p["p_out.weight"]).T) * torch.sigmoid(xn @ T(p["g_out.weight"]).T)).numpy()[None]


def _torch_transition(x, p):
    xn = F.layer_norm(x, (x.shape[-1],), T(p["norm.weight"]), T(p["norm.bias"]), 1e-5)
    return F.linear(F.silu(F.linear(xn, T(p["fc1.weight"]))) * F.linear(xn, T(p["fc2.weight"])), T(p["fc3.weight"]))


def _torch_apb(s_n, z, mask, p, H, inf=1e6):
    """AttentionPairBias on torch SDPA: q from s_n (biased), k / v from k_in = s_n, pair bias Linear(LN(z))."""
    B, N, Cs = s_n.shape
    hd = Cs // H
    q = F.linear(s_n, T(p["proj_q.weight"]), T(p["proj_q.bias"])).reshape(B, N, H, hd).transpose(1, 2)
    k = F.linear(s_n, T(p["proj_k.weight"])).reshape(B, N, H, hd).transpose(1, 2)
    v = F.linear(s_n, T(p["proj_v.weight"])).reshape(B, N, H, hd).transpose(1, 2)
    zb = F.linear(F.layer_norm(z, (z.shape[-1],), T(p["proj_z.0.weight"]), T(p["proj_z.0.bias"]), 1e-5),
                  T(p["proj_z.1.weight"]))
    bias = zb.permute(0, 3, 1, 2) + (1 - mask)[:, None, None, :] * -inf
    o = F.scaled_dot_product_attention(q, k, v, attn_mask=bias).transpose(1, 2).reshape(B, N, Cs)
    return F.linear(torch.sigmoid(F.linear(s_n, T(p["proj_g.weight"]))) * o, T(p["proj_o.weight"]))


def _pair_module_torch(name, z, pm, q):
    """The torch formulation of one pair module of the layer (the wiring pairformer.py:84-88 gives it)."""
    if name.startswith("tri_mul"):
        return _tri_mul_torch(z, pm, q, name == "tri_mul_out")
    if name.startswith("tri_att"):
        return _tri_att_sdpa(z, pm, q, name == "tri_att_start")
    return _torch_transition(T(z), q).numpy()


def _only(base, keep):
    """The layer's parameters with every matrix outside the modules `keep` zeroed (their updates vanish)."""
    return {k: (v if (k.startswith(keep) or v.ndim == 1 and not k.endswith("proj_q.bias")) else np.zeros_like(v))
            for k, v in base.items()}


def _layer_case():
    base = rand_params(shapes_layer(48, 32, heads=4, pw=8, pheads=2), seed=43, std=0.3)
    z, tok, pm = pair_inputs(6, 32, seed=44, n_pad=1)
    pm[0, 1, 3] = 0  # an asymmetric hole: a transposed mask or a swapped node would show
    s = np.random.default_rng(45).standard_normal((1, 6, 48))
    return base, z, tok, pm, s


@pytest.mark.parametrize("keep", PAIR_MODULES)
def test_layer_order(keep):
    """With one pair module live the layer's z update is that module alone, in its own wiring (direction, node)."""
    base, z, tok, pm, s = _layer_case()
    p = _only(base, (keep,))
    _, z2 = O.pairformer_layer(s, z, tok, pm, p, num_heads=4)
    ref = z + _pair_module_torch(keep, z, pm, O.sub(p, keep))
    assert np.abs(z2 - ref).max() < 1e-12
    # the other wiring of the same weights (incoming for outgoing, ending for starting) gives another result
    other = {"tri_mul_out": "tri_mul_in", "tri_mul_in": "tri_mul_out", "tri_att_start": "tri_att_end",
             "tri_att_end": "tri_att_start"}.get(keep)
    if other is not None:
        assert np.abs(z + _pair_module_torch(other, z, pm, O.sub(p, keep)) - z2).max() > 1e-4


@pytest.mark.parametrize("first,second", [(a, b) for i, a in enumerate(PAIR_MODULES) for b in PAIR_MODULES[i + 1:]])
def test_layer_two_live_modules_in_reference_order(first, second):
    """Two live pair modules compose in the reference order (pairformer.py:84-88): the later one reads the z the
    earlier one updated; the reversed order gives another result."""
    base, z, tok, pm, s = _layer_case()
    p = _only(base, (first, second))
    _, z2 = O.pairformer_layer(s, z, tok, pm, p, num_heads=4)
    qa, qb = O.sub(p, first), O.sub(p, second)
    z1 = z + _pair_module_torch(first, z, pm, qa)
    ref = z1 + _pair_module_torch(second, z1, pm, qb)
    assert np.abs(z2 - ref).max() < 1e-12
    zr = z + _pair_module_torch(second, z, pm, qb)
    rev = zr + _pair_module_torch(first, zr, pm, qa)
    assert np.abs(rev - ref).max() > 1e-6


def test_layer_s_track_composition():
    """The s track reads the pair bias from the z every pair update has produced, takes q and k_in from
    pre_norm_s(s), and runs transition_s on s after the attention residual (pairformer.py:90-93). transition_z is
    the only non-zero pair module, so the pre- and post-update z differ; a bias from the old z, transition_s on
    pre_norm_s(s) or on the pre-attention s would each fail."""
    cs, cz, H = 48, 32, 4
    base = rand_params(shapes_layer(cs, cz, heads=H, pw=8, pheads=2), seed=46, std=0.3)
    keep = ("attention", "transition_s", "transition_z")
    p = {k: (v if (k.startswith(keep) or v.ndim == 1 and not k.endswith("proj_q.bias")) else np.zeros_like(v))
         for k, v in base.items()}
    z, tok, pm = pair_inputs(7, cz, seed=47, n_pad=2)
    s = np.random.default_rng(48).standard_normal((1, 7, cs)) * 2 + 0.5
    s2, z2 = O.pairformer_layer(s, z, tok, pm, p, num_heads=H)
    zt, st, mt = T(z), T(s), T(tok)
    z1 = zt + _torch_transition(zt, O.sub(p, "transition_z"))
    s_n = F.layer_norm(st, (cs,), T(p["pre_norm_s.weight"]), T(p["pre_norm_s.bias"]), 1e-5)
    s1 = st + _torch_apb(s_n, z1, mt, O.sub(p, "attention"), H)
    ref_s = s1 + _torch_transition(s1, O.sub(p, "transition_s"))
    assert np.abs(z2 - z1.numpy()).max() < 1e-12
    assert np.abs(s2 - ref_s.numpy()).max() < 1e-11
    # the alternatives a misreading would compute are far from it
    wrong_bias = st + _torch_apb(s_n, zt, mt, O.sub(p, "attention"), H)
    wrong_bias = wrong_bias + _torch_transition(wrong_bias, O.sub(p, "transition_s"))
    wrong_tr = s1 + _torch_transition(s_n, O.sub(p, "transition_s"))
    for w in (wrong_bias, wrong_tr):
        assert np.abs(s2 - w.numpy()).max() > 1e-4


def test_layer_transition_s_alone():
    """Only transition_s non-zero: s' = s + transition(s) on the un-normalised s, z unchanged."""
    cs, cz, H = 48, 32, 4
    base = rand_params(shapes_layer(cs, cz, heads=H, pw=8, pheads=2), seed=49, std=0.3)
    p = {k: (v if (k.startswith("transition_s") or v.ndim == 1 and not k.endswith("proj_q.bias"))
             else np.zeros_like(v)) for k, v in base.items()}
    z, tok, pm = pair_inputs(5, cz, seed=50)
    s = np.random.default_rng(51).standard_normal((1, 5, cs)) * 3 - 1
    s2, z2 = O.pairformer_layer(s, z, tok, pm, p, num_heads=H)
    ref = T(s) + _torch_transition(T(s), O.sub(p, "transition_s"))
    assert np.array_equal(z2, z)
    assert np.abs(s2 - ref.numpy()).max() < 1e-12


def _zeroed(p):
    return {k: (np.zeros_like(v) if (v.ndim == 2 or k.endswith("proj_q.bias")) else v) for k, v in p.items()}


def test_module_runs_layers_in_order():
    """PairformerModule applies layers.0, then layers.1, ... (pairformer.py:145-148): with block 1 zeroed the
    module equals layer 0 alone, with block 0 zeroed it equals layer 1 alone, and with both live it is layer 1 after
    layer 0 (which differs from the reverse order)."""
    cs, cz, H = 48, 32, 4
    p0 = rand_params(shapes_layer(cs, cz, heads=H, pw=8, pheads=2), seed=52, std=0.2)
    p1 = rand_params(shapes_layer(cs, cz, heads=H, pw=8, pheads=2), seed=53, std=0.2)
    z, tok, pm = pair_inputs(6, cz, seed=54, n_pad=1)
    s = np.random.default_rng(55).standard_normal((1, 6, cs))

    def stack(a, b):
        out = {f"layers.0.{k}": v for k, v in a.items()}
        out.update({f"layers.1.{k}": v for k, v in b.items()})
        return out

    one = O.pairformer_layer(s, z, tok, pm, p0, H)
    got = O.pairformer_module(s, z, tok, pm, stack(p0, _zeroed(p1)), 2, H)
    assert all(np.abs(g - r).max() < 1e-12 for g, r in zip(got, one))
    one = O.pairformer_layer(s, z, tok, pm, p1, H)
    got = O.pairformer_module(s, z, tok, pm, stack(_zeroed(p0), p1), 2, H)
    assert all(np.abs(g - r).max() < 1e-12 for g, r in zip(got, one))
    fwd = O.pairformer_layer(*O.pairformer_layer(s, z, tok, pm, p0, H), tok, pm, p1, H)
    rev = O.pairformer_layer(*O.pairformer_layer(s, z, tok, pm, p1, H), tok, pm, p0, H)
    got = O.pairformer_module(s, z, tok, pm, stack(p0, p1), 2, H)
    assert all(np.abs(g - r).max() < 1e-12 for g, r in zip(got, fwd))
    assert np.abs(got[1] - rev[1]).max() > 1e-4


def test_metrics_definition():
    m = O.metrics(np.array([1.0, 2.0, 3.5]), np.array([1.0, 2.0, 4.0]))
    assert m["max_abs"] == 0.5 and m["max_rel"] == 0.125


def test_layer_norm_promotes_like_its_formula():
    """A float32 input with float64 parameters is normalised in float64 (as (x - mean) * w + b promotes), not in
    the input's float32."""
    rng = np.random.default_rng(60)
    x = rng.standard_normal((3, 128)).astype(np.float32)
    w, b = 1 + 0.1 * rng.standard_normal(128), 0.1 * rng.standard_normal(128)
    got = O.layer_norm(x, w, b)
    assert got.dtype == np.float64
    ref = F.layer_norm(T(x), (128,), T(w), T(b), 1e-5).numpy()
    assert np.abs(got - ref).max() < 1e-12
    assert O.layer_norm(x, w.astype(np.float32), b.astype(np.float32)).dtype == np.float32
