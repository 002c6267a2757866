"""Writes the golden fixtures in this folder from the CPU oracle (float64 arithmetic on float32-representable
inputs and weights).

The reference commits no golden vectors for this path (its module dumps are generated from upstream torch and
git-ignored), so these fixtures pin the oracle against regressions and give the GPU tests fixed vectors. Every row
and every column of every pair mask keeps at least one unmasked entry, so neither the starting node (rows) nor the
ending node (columns) sees a fully masked row, and fp32 evaluation agrees with these float64 outputs to ~1e-6. (On
a fully masked row the fp32 reference rounds every logit to -inf * 1 and averages uniformly; float64 does not.)

Run: python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, os.path.dirname(HERE))

import oracle as O  # noqa: E402
from conftest import rand_params, shapes_attention, shapes_transition, shapes_tri_att, shapes_tri_mul  # noqa: E402


def f32(d):
    return {k: np.asarray(v, dtype=np.float32) for k, v in d.items()}


def pair(N, D, seed):
    rng = np.random.default_rng(seed)
    z = rng.standard_normal((1, N, N, D)).astype(np.float32)
    tok = np.ones((1, N), np.float32)
    tok[:, -2:] = 0
    pm = tok[:, :, None] * tok[:, None, :]
    pm[:, -2:, 0] = 1  # padded rows keep one key: no fully masked row in the starting frame
    pm[:, 0, -2:] = 1  # padded columns keep one entry: none in the ending frame either
    pm[0, 3, 5] = 0
    return z, pm


def save(name, **arrays):
    np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrays)
    print("wrote", name, {k: v.shape for k, v in arrays.items()})


def main():
    N, D = 12, 128
    p = f32(rand_params(shapes_tri_mul(D), seed=901, std=0.1))
    z, pm = pair(N, D, 902)
    f64 = {k: v.astype(np.float64) for k, v in p.items()}
    out = O.tri_mul(z.astype(np.float64), pm.astype(np.float64), f64, True)
    inc = O.tri_mul(z.astype(np.float64), pm.astype(np.float64), f64, False)
    save("tri_mul_N12", z=z, pair_mask=pm, out_outgoing=out, out_incoming=inc, **{"p." + k: v for k, v in p.items()})

    p = f32(rand_params(shapes_tri_att(D, 32, 4), seed=911, std=0.1))
    z, pm = pair(N, D, 912)
    f64 = {k: v.astype(np.float64) for k, v in p.items()}
    st = O.tri_att(z.astype(np.float64), pm.astype(np.float64), f64, True)
    en = O.tri_att(z.astype(np.float64), pm.astype(np.float64), f64, False)
    save("tri_att_N12", z=z, pair_mask=pm, out_starting=st, out_ending=en, **{"p." + k: v for k, v in p.items()})

    p = f32(rand_params(shapes_transition(D, 4 * D), seed=921, std=0.1))
    x = np.random.default_rng(922).standard_normal((37, D)).astype(np.float32)
    y = O.transition(x.astype(np.float64), {k: v.astype(np.float64) for k, v in p.items()})
    save("transition_R37", x=x, out=y, **{"p." + k: v for k, v in p.items()})

    cs, H = 64, 4
    p = f32(rand_params(shapes_attention(cs, D, H), seed=931, std=0.1))
    rng = np.random.default_rng(932)
    s = rng.standard_normal((1, N, cs)).astype(np.float32)
    zz = rng.standard_normal((1, N, N, D)).astype(np.float32)
    mask = np.ones((1, N), np.float32)
    mask[:, -3:] = 0
    y = O.attention_pair_bias(s.astype(np.float64), zz.astype(np.float64), mask.astype(np.float64),
                              s.astype(np.float64), {k: v.astype(np.float64) for k, v in p.items()}, H)
    save("attention_pair_bias_N12", s=s, z=zz, mask=mask, out=y, **{"p." + k: v for k, v in p.items()})


if __name__ == "__main__":
    main()
