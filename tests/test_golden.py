"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py from the oracle): the oracle must keep
reproducing them (CPU), and the GPU modules in fp32 must match them to the fp32 parity bound (gpu)."""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    d = dict(np.load(os.path.join(GOLDEN, name + ".npz")))
    params = {k[2:]: v for k, v in d.items() if k.startswith("p.")}
    return d, params


def f64(p):
    return {k: v.astype(np.float64) for k, v in p.items()}


def test_oracle_reproduces_golden():
    d, p = load("tri_mul_N12")
    z, pm = d["z"].astype(np.float64), d["pair_mask"].astype(np.float64)
    assert np.abs(O.tri_mul(z, pm, f64(p), True) - d["out_outgoing"]).max() < 1e-12
    assert np.abs(O.tri_mul(z, pm, f64(p), False) - d["out_incoming"]).max() < 1e-12
    d, p = load("tri_att_N12")
    z, pm = d["z"].astype(np.float64), d["pair_mask"].astype(np.float64)
    assert np.abs(O.tri_att(z, pm, f64(p), True) - d["out_starting"]).max() < 1e-12
    assert np.abs(O.tri_att(z, pm, f64(p), False) - d["out_ending"]).max() < 1e-12
    d, p = load("transition_R37")
    assert np.abs(O.transition(d["x"].astype(np.float64), f64(p)) - d["out"]).max() < 1e-12
    d, p = load("attention_pair_bias_N12")
    s = d["s"].astype(np.float64)
    got = O.attention_pair_bias(s, d["z"].astype(np.float64), d["mask"].astype(np.float64), s, f64(p), 4)
    assert np.abs(got - d["out"]).max() < 1e-12


def test_golden_holds_in_fp32():
    """The fixtures are float64 outputs; the GPU bound below compares fp32 arithmetic against them, which is only
    meaningful where fp32 evaluation of the same function lands within that bound. A fully masked attention row
    (starting frame: a row of the mask; ending frame: a column) breaks this, since fp32 rounds all of its logits to
    the same -inf value, so the masks must keep one entry in every row and column."""
    def f32(p):
        return {k: v.astype(np.float32) for k, v in p.items()}

    def rel(got, ref):
        return O.metrics(got, ref)["max_rel"]

    d, p = load("tri_mul_N12")
    pm = d["pair_mask"]
    for ax in (1, 2):
        assert (pm.max(axis=ax) > 0).all()
    assert rel(O.tri_mul(d["z"], pm, f32(p), True), d["out_outgoing"]) <= 2e-6
    assert rel(O.tri_mul(d["z"], pm, f32(p), False), d["out_incoming"]) <= 2e-6
    d, p = load("tri_att_N12")
    pm = d["pair_mask"]
    for ax in (1, 2):
        assert (pm.max(axis=ax) > 0).all()
    assert rel(O.tri_att(d["z"], pm, f32(p), True), d["out_starting"]) <= 2e-6
    assert rel(O.tri_att(d["z"], pm, f32(p), False), d["out_ending"]) <= 2e-6
    d, p = load("transition_R37")
    assert rel(O.transition(d["x"], f32(p)), d["out"]) <= 2e-6
    d, p = load("attention_pair_bias_N12")
    assert rel(O.attention_pair_bias(d["s"], d["z"], d["mask"], d["s"], f32(p), 4), d["out"]) <= 2e-6


@pytest.mark.gpu
def test_gpu_modules_match_golden_fp32():
    from boltz_mlx_amd import kernels as K
    from boltz_mlx_amd.layers.attentionv2 import AttentionPairBias
    from boltz_mlx_amd.layers.transition import Transition
    from boltz_mlx_amd.layers.triangular_attention.attention import (TriangleAttentionEndingNode,
                                                                     TriangleAttentionStartingNode)
    from boltz_mlx_amd.layers.triangular_mult import TriangleMultiplicationIncoming, TriangleMultiplicationOutgoing
    from boltz_mlx_amd.weights import load_module

    assert torch.cuda.is_available()
    old = K.PRECISION
    K.set_precision("fp32")
    try:
        def dev(x):
            return torch.tensor(x, dtype=torch.float32, device="cuda")

        def check(got, ref, name):
            m = O.metrics(got.cpu().numpy(), ref)
            print(f"golden {name}: max_rel={m['max_rel']:.2e}", flush=True)
            assert m["max_rel"] <= 1e-5, (name, m)

        d, p = load("tri_mul_N12")
        for cls, key in ((TriangleMultiplicationOutgoing, "out_outgoing"), (TriangleMultiplicationIncoming, "out_incoming")):
            mod = load_module(cls(128), p).cuda()
            check(mod(dev(d["z"]), dev(d["pair_mask"])), d[key], key)
        d, p = load("tri_att_N12")
        for cls, key in ((TriangleAttentionStartingNode, "out_starting"), (TriangleAttentionEndingNode, "out_ending")):
            mod = load_module(cls(128, 32, 4), p).cuda()
            check(mod(dev(d["z"]), dev(d["pair_mask"])), d[key], key)
        d, p = load("transition_R37")
        check(load_module(Transition(128, 512), p).cuda()(dev(d["x"])), d["out"], "transition")
        d, p = load("attention_pair_bias_N12")
        mod = load_module(AttentionPairBias(64, 128, 4), p).cuda()
        check(mod(dev(d["s"]), dev(d["z"]), dev(d["mask"]), dev(d["s"])), d["out"], "attention_pair_bias")
    finally:
        K.set_precision(old)
