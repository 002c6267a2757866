"""The pair updates at 64 channels (the template stack's PairformerNoSeqLayer / Module, c_z = 64) on the GEMM +
layout-kernel path (csrc/bzpf_pack.hip), against the oracle (oracle/msa.py::pairformer_noseq_layer, which is
generic in the channel count). The layout kernels are also pinned at 128 channels against the fused projection
kernels they stand in for: the same buffers from the same inputs."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from conftest import pair_inputs, rand_params, shapes_noseq_layer
from oracle import msa as OM
from oracle.pairformer import sub

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _device():
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    from boltz_mlx_amd import _lib

    _lib.load()
    yield


@pytest.fixture
def precision(request):
    from boltz_mlx_amd import kernels as K

    old = K.PRECISION
    K.set_precision(request.param)
    yield request.param
    K.set_precision(old)


def dev(x, dtype=torch.float32):
    return torch.tensor(np.asarray(x), dtype=dtype, device="cuda")


@pytest.mark.parametrize("trans", [False, True])
@pytest.mark.parametrize("N", [37, 70])
def test_triattn_pack_matches_fused_projection(trans, N):
    from boltz_mlx_amd import kernels as K

    H, C, D = 4, 32, 128
    rng = np.random.default_rng(N + trans)
    xn = dev(rng.standard_normal((N * N, D)))
    w = dev(rng.standard_normal((4 * H * C + H, D)) / np.sqrt(D))
    q1, v1, t1 = K.triattn_proj(xn, w, trans, N, H, C)
    q2, v2, t2 = K.triattn_pack(K.linear(xn, w), trans, N, H, C)
    idx = torch.tensor(K.tri_bias_offsets(N, H).ravel(), device="cuda")
    ldk = K.row_pitch(N)
    for a, b in ((q1, q2), (v1[..., :N], v2[..., :N]), (t1[idx], t2[idx])):
        m = O.metrics(b.cpu().numpy(), a.cpu().numpy())
        assert m["max_rel"] < 1e-5, m
    assert torch.all(v2[..., N:ldk] == 0)


@pytest.mark.parametrize("incoming", [False, True])
def test_trimul_pack_matches_fused_projection(incoming):
    from boltz_mlx_amd import kernels as K

    N, D = 45, 128
    rng = np.random.default_rng(7 + incoming)
    xn = dev(rng.standard_normal((N * N, D)))
    w = dev(rng.standard_normal((4 * D, D)) / np.sqrt(D))
    mask = (rng.random((N, N)) > 0.2).astype(np.float32)
    a1 = K.trimul_proj(xn, w, dev(mask), 0.25, incoming, N)
    a2 = K.trimul_pack(K.linear(xn, w), dev(mask), 0.25, incoming, N)
    m = O.metrics(a2[..., :N].cpu().numpy(), a1[..., :N].cpu().numpy())
    assert m["max_rel"] < 1e-5, m
    assert torch.all(a2[..., N:] == 0)


def test_channels_to_rows():
    from boltz_mlx_amd import kernels as K

    N, D = 70, 64
    ld = K.row_pitch(N)
    o = torch.randn((D, N, ld), device="cuda")
    got = K.channels_to_rows(o, N).view(N, N, D)
    assert torch.equal(got, o[..., :N].permute(1, 2, 0))


@pytest.mark.parametrize("precision", ["fp32", "f16"], indirect=True)
@pytest.mark.parametrize("N,n_pad", [(24, 2), (70, 5), (260, 6)])
def test_noseq_layer_c64(precision, N, n_pad):
    from boltz_mlx_amd.layers.pairformer import PairformerNoSeqLayer
    from boltz_mlx_amd.weights import load_module

    p = rand_params(shapes_noseq_layer(64), seed=N, std=0.1)
    z, _, pm = pair_inputs(N, 64, seed=N + 1, n_pad=n_pad)
    mod = load_module(PairformerNoSeqLayer(64), p).cuda()
    got = mod(dev(z), dev(pm)).cpu().numpy()
    # the oracle in float32: padded tokens' fully-masked attention rows (inf = 1e9) round every logit to one value,
    # the reference's fp32 semantics (uniform weights), which float64 does not reproduce
    f = lambda x: np.asarray(x, np.float32)  # noqa: E731
    ref = OM.pairformer_noseq_layer(f(z), f(pm), {k: f(v) for k, v in p.items()})
    mt = O.metrics(got - z, ref - z)
    print(f"noseq c_z=64 N={N} [{precision}]: {mt}", flush=True)
    assert mt["finite"]
    if precision == "fp32":
        assert mt["max_rel"] <= 1e-5, mt
    else:
        assert mt["max_rel"] <= 3e-2 and mt["rel_fro"] <= 1e-2, mt


@pytest.mark.parametrize("N,n_pad", [(24, 2), (70, 5)])
def test_noseq_layer_c64_fused_transition(monkeypatch, N, n_pad):
    """f16 with the pair transition on the fused 64-channel kernel (taken from 16,384 pairs; forced here)."""
    from boltz_mlx_amd import kernels as K
    from boltz_mlx_amd.layers import transition as T
    from boltz_mlx_amd.layers.pairformer import PairformerNoSeqLayer
    from boltz_mlx_amd.weights import load_module

    monkeypatch.setattr(T, "FUSED_MIN_ROWS", 1)
    p = rand_params(shapes_noseq_layer(64), seed=N, std=0.1)
    z, _, pm = pair_inputs(N, 64, seed=N + 1, n_pad=n_pad)
    old = K.PRECISION
    K.set_precision("f16")
    try:
        mod = load_module(PairformerNoSeqLayer(64), p).cuda()
        got = mod(dev(z), dev(pm)).cpu().numpy()
    finally:
        K.set_precision(old)
    f = lambda x: np.asarray(x, np.float32)  # noqa: E731 (float32 oracle: see test_noseq_layer_c64)
    ref = OM.pairformer_noseq_layer(f(z), f(pm), {k: f(v) for k, v in p.items()})
    mt = O.metrics(got - z, ref - z)
    assert mt["finite"] and mt["max_rel"] <= 3e-2 and mt["rel_fro"] <= 1e-2, mt


@pytest.mark.parametrize("precision", ["fp32", "f16"], indirect=True)
def test_noseq_module_c64_two_blocks(precision):
    """The template stack's shape: two NoSeq blocks at c_z = 64 (trunkv2.py:64-71)."""
    from boltz_mlx_amd.layers.pairformer import PairformerNoSeqModule
    from boltz_mlx_amd.weights import load_module

    N = 40
    p = {}
    for i in range(2):
        p.update({f"layers.{i}.{k}": v for k, v in rand_params(shapes_noseq_layer(64), seed=50 + i, std=0.1).items()})
    z, _, pm = pair_inputs(N, 64, seed=52, n_pad=3)
    mod = load_module(PairformerNoSeqModule(64, 2), p).cuda()
    got = mod(dev(z), dev(pm)).cpu().numpy()
    f = lambda x: np.asarray(x, np.float32)  # noqa: E731 (float32 oracle: see test_noseq_layer_c64)
    ref = f(z)
    for i in range(2):
        ref = OM.pairformer_noseq_layer(ref, f(pm), {k: f(v) for k, v in sub(p, f"layers.{i}").items()})
    mt = O.metrics(got - z, ref - z)
    print(f"noseq module c_z=64 [{precision}]: {mt}", flush=True)
    assert mt["finite"]
    if precision == "fp32":
        assert mt["max_rel"] <= 1e-5, mt
    else:
        assert mt["max_rel"] <= 3e-2 and mt["rel_fro"] <= 1e-2, mt
