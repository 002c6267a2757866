"""numpy restatement of the reference's MSA-block pair kernels (test infrastructure: the reference results the tests
compare against, never the product).

Like oracle/pairformer.py, every function computes in the dtype of its inputs (float64 pins the parity tests) and
takes parameter dicts keyed by the reference's PyTorch qualified names relative to the module.

Sources restated (paths relative to the reference checkout):
- OuterProductMean: boltz_mlx/layers/outer_product_mean.py:24-50 (module path): LN(m), a = proj_a * mask,
  b = proj_b * mask, z[i, j, c, d] = sum_s a[s, i, c] b[s, j, d] / max(sum_s mask[s, i] mask[s, j], 1), proj_o
  over the flattened (c, d) with c major; the fused path's pieces (outer_product_mean.py:52-84 and
  kernels_msa.py:322-343: [W_a; W_b] in one GEMM, the mask applied to the outer-sum operands, num = mask^T mask)
  are restated in opm_outer.
- PairWeightedAveraging: boltz_mlx/layers/pair_averaging.py:30-59: v = proj_m(LN(m)) per head, logits
  proj_z(LN(z)) + (1 - pair_mask) * -inf, softmax over j, o[s, i] = sum_j w[h, i, j] v[s, j], gate
  sigmoid(proj_g(LN(m))), proj_o; the fused path's split (pwa_weights then pwa_avg with the gate in its epilogue,
  kernels_msa.py:461-500, 620-653) in pwa_weights / pwa_avg.
- MSALayer: boltz_mlx/modules/trunkv2.py:205-247 (m += PWA(m, z, token pair mask); m += Transition(m);
  z += OPM(m, msa_mask); z = PairformerNoSeqLayer(z)), PairformerNoSeqLayer: boltz_mlx/layers/pairformer.py:156-203
  (the five pair updates of PairformerLayer without the s track).

Parity status: pinned by tests/test_oracle_msa.py against torch float64 formulations written from the definitions
(einsum outer sums, torch.softmax), the fused-path split against the module path, closed forms (an all-masked MSA
gives num = 1 and z = bias; one unmasked key gives w = 1 on it; zero proj_z weights give the masked uniform
average) and brute-force loops on tiny inputs.
"""

from __future__ import annotations

import numpy as np

from oracle.pairformer import layer_norm, linear, sigmoid, softmax, sub, transition, tri_att, tri_mul

__all__ = ["opm_outer", "outer_product_mean", "pwa_weights", "pwa_avg", "pair_weighted_averaging",
           "pairformer_noseq_layer", "msa_layer"]


def opm_outer(ab, mask, c: int = 32):
    """z / num for one MSA (ab [S, N, 2c] = LN(m) [W_a; W_b]^T, unmasked; mask [S, N]) as [N, N, c * c] with
    column index c_a * c + d (outer_product_mean.py:37-45; kernels_msa.py:322-343)."""
    a = ab[..., :c] * mask[..., None]
    b = ab[..., c:2 * c] * mask[..., None]
    num = np.maximum(mask.T @ mask, 1.0)
    z = np.einsum("sic,sjd->ijcd", a, b)
    N = ab.shape[1]
    return z.reshape(N, N, c * c) / num[:, :, None]


def outer_product_mean(m, mask, p: dict, c: int = 32):
    """OuterProductMean (outer_product_mean.py:24-50) for m [B, S, N, c_in], mask [B, S, N] -> [B, N, N, c_out]."""
    mn = layer_norm(m, p["norm.weight"], p["norm.bias"], 1e-5)
    w_ab = np.concatenate([p["proj_a.weight"], p["proj_b.weight"]], 0)
    out = []
    for b in range(m.shape[0]):
        z = opm_outer(linear(mn[b], w_ab), mask[b].astype(m.dtype), c)
        out.append(linear(z, p["proj_o.weight"], p["proj_o.bias"]))
    return np.stack(out)


def pwa_weights(z, pair_mask, p: dict, inf: float = 1e6):
    """softmax_j(proj_z(norm_z(z)) + (1 - pair_mask) * -inf) as [H, N, N] for one z [N, N, c_z]
    (pair_averaging.py:43-49; kernels_msa.py:485-500)."""
    zn = layer_norm(z, p["norm_z.weight"], p["norm_z.bias"], 1e-5)
    logits = linear(zn, p["proj_z.weight"]).transpose(2, 0, 1)
    return softmax(logits + (1 - pair_mask)[None] * -inf, -1)


def pwa_avg(w, v, g, c_h: int = 32):
    """sigmoid(g) * o with o[s, i, h c_h + d] = sum_j w[h, i, j] v[s, j, h c_h + d] (v, g [S, N, H c_h])
    (pair_averaging.py:50-57; kernels_msa.py:645-653)."""
    S, N, HC = v.shape
    H = HC // c_h
    vh = v.reshape(S, N, H, c_h)
    o = np.einsum("hij,sjhd->sihd", w, vh).reshape(S, N, HC)
    return sigmoid(g) * o


def pair_weighted_averaging(m, z, pair_mask, p: dict, num_heads: int = 8, c_h: int = 32, inf: float = 1e6):
    """PairWeightedAveraging (pair_averaging.py:30-59): m [B, S, N, c_m], z [B, N, N, c_z], pair_mask [B, N, N]."""
    mn = layer_norm(m, p["norm_m.weight"], p["norm_m.bias"], 1e-5)
    out = []
    for b in range(m.shape[0]):
        w = pwa_weights(z[b], pair_mask[b], p, inf)
        og = pwa_avg(w, linear(mn[b], p["proj_m.weight"]), linear(mn[b], p["proj_g.weight"]), c_h)
        out.append(linear(og, p["proj_o.weight"]))
    return np.stack(out)


def pairformer_noseq_layer(z, pair_mask, p: dict):
    """PairformerNoSeqLayer (pairformer.py:156-203): the pair updates of PairformerLayer, z [B, N, N, c_z]."""
    z = z + tri_mul(z, pair_mask, sub(p, "tri_mul_out"), True)
    z = z + tri_mul(z, pair_mask, sub(p, "tri_mul_in"), False)
    z = z + tri_att(z, pair_mask, sub(p, "tri_att_start"), True)
    z = z + tri_att(z, pair_mask, sub(p, "tri_att_end"), False)
    return z + transition(z, sub(p, "transition_z"))


def msa_layer(z, m, pair_mask, msa_mask, p: dict):
    """MSALayer (trunkv2.py:229-247) -> (z, m)."""
    m = m + pair_weighted_averaging(m, z, pair_mask, sub(p, "pair_weighted_averaging"))
    m = m + transition(m, sub(p, "msa_transition"))
    z = z + outer_product_mean(m, msa_mask, sub(p, "outer_product_mean"))
    z = pairformer_noseq_layer(z, pair_mask, sub(p, "pairformer_layer"))
    return z, m
