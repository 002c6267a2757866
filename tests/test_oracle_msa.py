"""Pins the MSA-block oracle (oracle/msa.py) against torch float64 formulations written from the definitions
(einsum outer sums and weighted averages, torch layer_norm / softmax), brute-force loops on tiny inputs and closed
forms. A dropped mask factor, a transposed (c, d) flattening, a missing clamp of the pair counts, a softmax over the
wrong axis or a gate on the wrong projection fails one of them."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import pair_inputs, rand_params, shapes_layer, shapes_msa_layer, shapes_opm, shapes_pwa
from oracle import msa as OM
from oracle import pairformer as OP


def T(x):
    return torch.from_numpy(np.asarray(x, dtype=np.float64))


def _torch_opm(m, mask, p):
    mn = F.layer_norm(T(m), (m.shape[-1],), T(p["norm.weight"]), T(p["norm.bias"]), 1e-5)
    mk = T(mask)[..., None]
    a = F.linear(mn, T(p["proj_a.weight"])) * mk
    b = F.linear(mn, T(p["proj_b.weight"])) * mk
    num = torch.clamp((mk[:, :, None, :, :] * mk[:, :, :, None, :]).sum(1), min=1)
    z = torch.einsum("bsic,bsjd->bijcd", a, b).flatten(-2) / num
    return F.linear(z, T(p["proj_o.weight"]), T(p["proj_o.bias"])).numpy()


def _torch_pwa(m, z, pm, p, H=8, ch=32, inf=1e6):
    mn = F.layer_norm(T(m), (m.shape[-1],), T(p["norm_m.weight"]), T(p["norm_m.bias"]), 1e-5)
    B, S, N, _ = m.shape
    v = F.linear(mn, T(p["proj_m.weight"])).view(B, S, N, H, ch).permute(0, 3, 1, 2, 4)
    zn = F.layer_norm(T(z), (z.shape[-1],), T(p["norm_z.weight"]), T(p["norm_z.bias"]), 1e-5)
    logits = F.linear(zn, T(p["proj_z.weight"])).permute(0, 3, 1, 2) + (1 - T(pm))[:, None] * -inf
    w = torch.softmax(logits, dim=-1)
    o = torch.matmul(w[:, :, None], v).permute(0, 2, 3, 1, 4).reshape(B, S, N, H * ch)
    g = torch.sigmoid(F.linear(mn, T(p["proj_g.weight"])))
    return F.linear(g * o, T(p["proj_o.weight"])).numpy()


def _msa_inputs(S, N, seed, p_mask=0.2):
    rng = np.random.default_rng(seed)
    m = rng.standard_normal((1, S, N, 64))
    mask = (rng.random((1, S, N)) > p_mask).astype(np.float64)
    return m, mask


@pytest.mark.parametrize("S,N", [(7, 5), (1, 6), (23, 4)])
def test_opm_vs_torch(S, N):
    p = rand_params(shapes_opm(), seed=S, std=0.1)
    m, mask = _msa_inputs(S, N, S + N)
    assert np.abs(OM.outer_product_mean(m, mask, p) - _torch_opm(m, mask, p)).max() < 1e-12


def test_opm_outer_brute_force_and_layout():
    """z[i, j, c * 32 + d] = sum_s mask_si mask_sj a[s, i, c] b[s, j, d] / max(count, 1) by plain loops, with one
    pair (i, j) whose tokens never share an unmasked row (count 0 -> divided by 1)."""
    rng = np.random.default_rng(2)
    S, N, c = 4, 3, 32
    ab = rng.standard_normal((S, N, 2 * c))
    mask = np.ones((S, N))
    mask[:, 0] = [1, 0, 1, 0]
    mask[:, 2] = [0, 1, 0, 1]
    got = OM.opm_outer(ab, mask, c)
    for i in range(N):
        for j in range(N):
            cnt = sum(mask[s, i] * mask[s, j] for s in range(S))
            for ca in (0, 5, 31):
                for d in (0, 7, 31):
                    ref = sum(mask[s, i] * mask[s, j] * ab[s, i, ca] * ab[s, j, c + d] for s in range(S)) / max(cnt, 1)
                    assert abs(got[i, j, ca * c + d] - ref) < 1e-12
    assert (mask[:, 0] * mask[:, 2]).sum() == 0 and np.all(got[0, 2] == 0)


def test_opm_all_masked_gives_bias():
    p = rand_params(shapes_opm(), seed=3, std=0.1)
    m, _ = _msa_inputs(5, 4, 4)
    out = OM.outer_product_mean(m, np.zeros((1, 5, 4)), p)
    assert np.abs(out - p["proj_o.bias"]).max() == 0


@pytest.mark.parametrize("S,N", [(3, 5), (1, 7)])
def test_pwa_vs_torch(S, N):
    p = rand_params(shapes_pwa(), seed=10 + S, std=0.2)
    m, _ = _msa_inputs(S, N, 11)
    z, _, pm = pair_inputs(N, 128, seed=12, n_pad=1)
    pm = pm.copy()
    pm[0, 1, 3] = 0
    assert np.abs(OM.pair_weighted_averaging(m, z, pm, p) - _torch_pwa(m, z, pm, p)).max() < 1e-12


def test_pwa_weight_closed_forms():
    """Zero proj_z: w is the uniform average over the unmasked keys of each row; a row with one unmasked key puts
    weight 1 on it; weights sum to 1."""
    N = 6
    p = rand_params(shapes_pwa(), seed=13, std=0.2)
    z, _, _ = pair_inputs(N, 128, seed=14)
    pm = np.ones((N, N))
    pm[0, 2:] = 0
    pm[1, :] = 0
    pm[1, 4] = 1
    w0 = OM.pwa_weights(z[0], pm, dict(p, **{"proj_z.weight": np.zeros_like(p["proj_z.weight"])}))
    assert np.abs(w0[:, 0, :2] - 0.5).max() < 1e-15 and np.abs(w0[:, 0, 2:]).max() < 1e-15
    w = OM.pwa_weights(z[0], pm, p)
    assert np.abs(w[:, 1, 4] - 1).max() < 1e-15
    assert np.abs(w.sum(-1) - 1).max() < 1e-12
    assert np.abs(w0[:, 2] - 1 / N).max() < 1e-15


def test_pwa_avg_brute_force():
    rng = np.random.default_rng(15)
    S, N, H, ch = 2, 3, 8, 32
    w = rng.random((H, N, N))
    v, g = rng.standard_normal((S, N, H * ch)), rng.standard_normal((S, N, H * ch))
    got = OM.pwa_avg(w, v, g, ch)
    for s, i, h, d in [(0, 0, 0, 0), (1, 2, 7, 31), (0, 1, 3, 17)]:
        ref = sum(w[h, i, j] * v[s, j, h * ch + d] for j in range(N)) / (1 + np.exp(-g[s, i, h * ch + d]))
        assert abs(got[s, i, h * ch + d] - ref) < 1e-12


def test_msa_layer_order_and_noseq():
    """The MSA layer is PWA -> transition on m -> OPM into z -> the NoSeq pair layer, which is PairformerLayer's
    pair part: checked against the pieces composed by hand and against pairformer_layer's z output."""
    N, S = 5, 3
    p = rand_params(shapes_msa_layer(), seed=20, std=0.05)
    z, tok, pm = pair_inputs(N, 128, seed=21, n_pad=1)
    m, msa_mask = _msa_inputs(S, N, 22)
    zo, mo = OM.msa_layer(z, m, pm, msa_mask, p)
    m1 = m + OM.pair_weighted_averaging(m, z, pm, OP.sub(p, "pair_weighted_averaging"))
    m2 = m1 + OP.transition(m1, OP.sub(p, "msa_transition"))
    z1 = z + OM.outer_product_mean(m2, msa_mask, OP.sub(p, "outer_product_mean"))
    assert np.abs(mo - m2).max() == 0
    pl = rand_params(shapes_layer(384, 128), seed=23)
    pl.update({k[len("pairformer_layer."):]: v for k, v in p.items() if k.startswith("pairformer_layer.")})
    s = np.random.default_rng(24).standard_normal((1, N, 384))
    _, z_ref = OP.pairformer_layer(s, z1, tok, pm, pl)
    assert np.abs(zo - z_ref).max() < 1e-12
