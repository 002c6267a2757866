"""GPU parity at the benchmark configurations' own sizes, with the reference's dense random masks, B = 2 batches and
the reference's f16 ``xn`` contract.

- C1: one PairformerLayer, fp32, N = 128 (z, s ~ N(0, 1), weights ~ N(0, 0.02), LayerNorm gamma 1 / beta 0, all-ones
  mask) against the float32 oracle at max|d| / max|ref| <= 1e-5.
- C2: triangle attention, N = 400, the last 40 tokens padded, starting and ending node, fp32 (1e-5) and f16 (the
  module gate) against the oracle.
- C3: triangle multiplication, N = 800, outgoing and incoming, f16 against the oracle; plus a coherent input whose
  contraction peaks above the fp16 range (the 2^-K operand pre-scale keeps it finite).
- C4: the 64-block trunk at N = 1000 and N = 400 (5 % padded tokens) in f16 against the same trunk in fp32 (the mode pinned to
  the oracle at 1e-5 above), with a stated rel_fro bound, and the size-independent padding property: the outputs at
  unpadded positions do not depend on the values at padded positions, bit for bit.
- C5: one diffusion-transformer layer (D 768, 16 heads, N 400, 5 samples sharing one pair bias) against the oracle,
  and the 24-layer stack in f16 against fp32.

The float32 oracle stands in for the reference's fp32 CPU path (MLX fp32); f16 gates are the module / layer gates of
test_gpu_parity.py (max_rel, rel_fro) = (2e-2, 5e-3) / (3e-2, 1e-2).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from conftest import (pair_inputs, rand_params, shapes_diffusion_layer, shapes_layer, shapes_tri_att, shapes_tri_mul,
                      with_shared_alias)
from oracle import diffusion as OD

pytestmark = pytest.mark.gpu

F16_MODULE = (2e-2, 5e-3)
F16_LAYER = (3e-2, 1e-2)
# f16 against fp32 after many blocks / layers: the per-block fp16 storage rounding compounds through the residual
# streams. Measured on MI355X (printed by the tests): 64-block trunk at N = 1000, rel_fro of the z update 1.1e-3 and of
# the s update 6.7e-4; 24-layer diffusion stack 7.0e-4. The bounds leave about 4x margin.
TRUNK_REL_FRO = 5e-3
DIFF_STACK_REL_FRO = 3e-3


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


def load(mod, params):
    from boltz_mlx_amd.weights import load_module

    load_module(mod, params)
    return mod.cuda()


def cast(d, dt):
    return {k: np.asarray(v, dtype=dt) for k, v in d.items()}


def check(name, got, ref, prec, gate=F16_MODULE):
    m = O.metrics(got, ref)
    print(f"{name} [{prec}]: max_rel={m['max_rel']:.3e} rel_fro={m['rel_fro']:.3e} max_abs={m['max_abs']:.3e}",
          flush=True)
    assert m["finite"], name
    if prec == "fp32":
        assert m["max_rel"] <= 1e-5, (name, m)
    else:
        assert m["max_rel"] <= gate[0] and m["rel_fro"] <= gate[1], (name, m)


def rand_mask(rng, shape):
    """The reference's dense random mask (tests/test_triatt_mma.py:14-19): keep with probability 0.7, plus fully
    masked rows 3 and 7 and a masked key column 5."""
    m = (rng.random(shape) > 0.3).astype(np.float64)
    m[..., 3, :] = 0.0
    m[..., :, 5] = 0.0
    m[..., 7, :] = 0.0
    return m


# ------------------------------------------------------------------------------------------------ C1

@pytest.mark.timeout(300)
@pytest.mark.parametrize("precision", ["fp32", "f16"], indirect=True)
def test_c1_block_N128(precision):
    from boltz_mlx_amd.layers.pairformer import PairformerLayer

    N, cs, cz, H = 128, 384, 128, 16
    p = rand_params(shapes_layer(cs, cz, H), seed=1001, std=0.02, ln_random=False)
    z, tok, pm = pair_inputs(N, cz, seed=1002)
    s = np.random.default_rng(1003).standard_normal((1, N, cs))
    f32 = np.float32
    s_r, z_r = O.pairformer_layer(s.astype(f32), z.astype(f32), tok.astype(f32), pm.astype(f32), cast(p, f32), H)
    layer = load(PairformerLayer(cs, cz, H), p)
    s_g, z_g = layer(dev(s), dev(z), dev(tok), dev(pm))
    # the update, not the sum, carries the comparison (z + update is dominated by z)
    check("C1 block z update", (z_g.cpu().numpy() - z), z_r - z, precision, F16_LAYER)
    check("C1 block s update", (s_g.cpu().numpy() - s), s_r - s, precision, F16_LAYER)
    check("C1 block z", z_g.cpu().numpy(), z_r, precision, F16_LAYER)
    check("C1 block s", s_g.cpu().numpy(), s_r, precision, F16_LAYER)


# ------------------------------------------------------------------------------------------------ C2

@pytest.mark.timeout(400)
@pytest.mark.parametrize("precision", ["fp32", "f16"], indirect=True)
@pytest.mark.parametrize("starting", [True, False])
def test_c2_tri_att_N400(precision, starting):
    from boltz_mlx_amd.layers.triangular_attention.attention import (TriangleAttentionEndingNode,
                                                                     TriangleAttentionStartingNode)

    N, D, C, H = 400, 128, 32, 4
    p = rand_params(shapes_tri_att(D, C, H), seed=1100, std=0.1, ln_random=False)
    x, _, pm = pair_inputs(N, D, seed=1101, n_pad=40)
    f32 = np.float32
    ref = O.tri_att(x.astype(f32), pm.astype(f32), cast(p, f32), starting, row_chunk=16)
    mod = load(TriangleAttentionStartingNode(D, C, H) if starting else TriangleAttentionEndingNode(D, C, H), p)
    got = mod(dev(x), dev(pm)).cpu().numpy()
    check(f"C2 tri_att_{'start' if starting else 'end'} N=400", got, ref, precision)


# ------------------------------------------------------------------------------------------------ C3

@pytest.mark.timeout(600)
@pytest.mark.parametrize("precision", ["fp32", "f16"], indirect=True)
@pytest.mark.parametrize("outgoing", [True, False])
def test_c3_tri_mul_N800(precision, outgoing):
    from boltz_mlx_amd.layers.triangular_mult import TriangleMultiplicationIncoming, TriangleMultiplicationOutgoing

    N, D = 800, 128
    p = rand_params(shapes_tri_mul(D), seed=1200, std=0.1, ln_random=False)
    x, _, pm = pair_inputs(N, D, seed=1201)
    f32 = np.float32
    ref = O.tri_mul(x.astype(f32), pm.astype(f32), cast(p, f32), outgoing)
    mod = load((TriangleMultiplicationOutgoing if outgoing else TriangleMultiplicationIncoming)(D), p)
    got = mod(dev(x), dev(pm)).cpu().numpy()
    check(f"C3 tri_mul_{'out' if outgoing else 'in'} N=800", got, ref, precision)


@pytest.mark.timeout(600)
@pytest.mark.parametrize("precision", ["f16"], indirect=True)
def test_c3_tri_mul_N800_beyond_fp16_range(precision):
    """Every position near one direction u and p_in / g_in aligned with LN(u): a, b ~ 6..18 (a per-channel factor)
    with gates ~ 1, so the contraction o = sum_k a b reaches 3e4..2.6e5, mostly above fp16's 65504. The 2^-4 pre-scale
    of a and b (o carries 2^-8) keeps every fp16 intermediate finite and norm_out's eps * 2^-16 undoes the scale."""
    from boltz_mlx_amd.layers.triangular_mult import TriangleMultiplicationOutgoing

    N, D = 800, 128
    rng = np.random.default_rng(1210)
    u = rng.standard_normal(D)
    x = u[None, None, None, :] + 0.3 * rng.standard_normal((1, N, N, D))
    ln_u = (u - u.mean()) / u.std()
    p = rand_params(shapes_tri_mul(D), seed=1211, std=0.05, ln_random=False)
    alpha = 12.0 * (1.0 + 0.5 * rng.uniform(-1.0, 1.0, size=(2 * D, 1)))
    p["p_in.weight"] = p["p_in.weight"] + alpha * ln_u[None, :] / D
    p["g_in.weight"] = p["g_in.weight"] + 6.0 * ln_u[None, :] / D
    pm = np.ones((1, N, N))
    f32 = np.float32
    xn = O.layer_norm(x[0, :4, :4].astype(np.float64))
    a = (xn @ p["p_in.weight"].T) * O.sigmoid(xn @ p["g_in.weight"].T)
    assert (a * a).mean() * N > 7e4  # the contraction peak is above the fp16 range
    ref = O.tri_mul(x.astype(f32), pm.astype(f32), cast(p, f32), True)
    got = load(TriangleMultiplicationOutgoing(D), p)(dev(x), dev(pm)).cpu().numpy()
    check("C3 tri_mul_out N=800 beyond fp16 range", got, ref, precision)


# ------------------------------------------------------------------------------------------------ C4

def _trunk(N, blocks, seed):
    from boltz_mlx_amd.layers.pairformer import PairformerModule
    from boltz_mlx_amd.weights import load_module, synthetic_state

    m = PairformerModule(384, 128, blocks, 16)
    load_module(m, synthetic_state(m, seed))
    m = m.cuda()
    rng = np.random.default_rng(seed + 1)
    z = torch.tensor(rng.standard_normal((1, N, N, 128), dtype=np.float32), device="cuda")
    s = torch.tensor(rng.standard_normal((1, N, 384), dtype=np.float32), device="cuda")
    tok = torch.ones((1, N), dtype=torch.float32, device="cuda")
    tok[:, N - int(round(0.05 * N)):] = 0
    pm = (tok[:, :, None] * tok[:, None, :]).contiguous()
    return m, s, z, tok, pm


def _rel_fro(a, b):
    d = (a.double() - b.double()).norm().item()
    return d / max(b.double().norm().item(), 1e-300)


@pytest.mark.timeout(900)
@pytest.mark.parametrize("N", [400, 1000])
def test_c4_trunk_f16_vs_fp32_and_padding(N):
    """The benchmark's trunk at both of its sizes (N = 1000 is C4; N = 400 is the metric's second size)."""
    from boltz_mlx_amd import kernels as K

    blocks = 64
    n_real = N - int(round(0.05 * N))
    old = K.PRECISION
    try:
        m, s, z, tok, pm = _trunk(N, blocks, seed=0)
        K.set_precision("f16")
        with torch.no_grad():
            s16, z16 = m(s, z, tok, pm)
        torch.cuda.synchronize()
        assert m.fp16_fallbacks == 0
        assert torch.isfinite(z16).all() and torch.isfinite(s16).all()
        print(f"C4 f16 trunk done: |z| max {z16.abs().max().item():.3e}", flush=True)
        # padding property: new values at the padded positions change nothing at the unpadded ones
        z2, s2 = z.clone(), s.clone()
        g = torch.Generator(device="cuda").manual_seed(5)
        z2[:, n_real:] = 4 * torch.randn(z2[:, n_real:].shape, generator=g, device="cuda")
        z2[:, :, n_real:] = 4 * torch.randn(z2[:, :, n_real:].shape, generator=g, device="cuda")
        s2[:, n_real:] = 4 * torch.randn(s2[:, n_real:].shape, generator=g, device="cuda")
        with torch.no_grad():
            s16b, z16b = m(s2, z2, tok, pm)
        torch.cuda.synchronize()
        assert torch.equal(z16b[:, :n_real, :n_real], z16[:, :n_real, :n_real])
        assert torch.equal(s16b[:, :n_real], s16[:, :n_real])
        print("C4 padding invariance: bit-exact", flush=True)
        del z2, s2, s16b, z16b
        K.set_precision("fp32")
        with torch.no_grad():
            s32, z32 = m(s, z, tok, pm)
        torch.cuda.synchronize()
        rz = _rel_fro(z16[:, :n_real, :n_real] - z[:, :n_real, :n_real], z32[:, :n_real, :n_real] - z[:, :n_real, :n_real])
        rs = _rel_fro(s16[:, :n_real] - s[:, :n_real], s32[:, :n_real] - s[:, :n_real])
        rz_all = _rel_fro(z16, z32)
        print(f"C4 64-block trunk N={N} f16 vs fp32: rel_fro(z update)={rz:.3e} rel_fro(s update)={rs:.3e} "
              f"rel_fro(z)={rz_all:.3e}", flush=True)
        assert rz <= TRUNK_REL_FRO and rs <= TRUNK_REL_FRO
    finally:
        K.set_precision(old)


@pytest.mark.timeout(600)
def test_trunk_blocks_N1537_f16_vs_fp32():
    """Beyond the benchmark's sizes: two blocks at N = 1537 (rows padded to 1600, a partial 256-wide contraction tile
    and query block, 13 query blocks per attention row) with 3% padded tokens; f16 against the fp32 kernels, both on
    the GPU (the float64 oracle at this size would take minutes), and padding invariance bit for bit."""
    from boltz_mlx_amd import kernels as K

    N, blocks = 1537, 2
    n_real = N - 46
    old = K.PRECISION
    try:
        m, s, z, tok, pm = _trunk(N, blocks, seed=7)
        tok.fill_(1.0)
        tok[:, n_real:] = 0
        pm.copy_(tok[:, :, None] * tok[:, None, :])
        K.set_precision("f16")
        with torch.no_grad():
            s16, z16 = m(s, z, tok, pm)
            z2 = z.clone()
            z2[:, n_real:] = 3 * torch.randn_like(z2[:, n_real:])
            s16b, z16b = m(s, z2, tok, pm)
        torch.cuda.synchronize()
        assert torch.isfinite(z16).all() and torch.isfinite(s16).all() and m.fp16_fallbacks == 0
        assert torch.equal(z16b[:, :n_real, :n_real], z16[:, :n_real, :n_real])
        assert torch.equal(s16b[:, :n_real], s16[:, :n_real])
        del z2, s16b, z16b
        K.set_precision("fp32")
        with torch.no_grad():
            s32, z32 = m(s, z, tok, pm)
        torch.cuda.synchronize()
        rz = _rel_fro(z16[:, :n_real, :n_real] - z[:, :n_real, :n_real], z32[:, :n_real, :n_real] - z[:, :n_real, :n_real])
        rs = _rel_fro(s16[:, :n_real] - s[:, :n_real], s32[:, :n_real] - s[:, :n_real])
        print(f"N={N} two blocks f16 vs fp32: rel_fro(z update)={rz:.3e} rel_fro(s update)={rs:.3e}", flush=True)
        assert rz <= TRUNK_REL_FRO and rs <= TRUNK_REL_FRO
    finally:
        K.set_precision(old)


# ------------------------------------------------------------------------------------------------ C5

def _diff_params(D, depth, std, seed):
    p = {}
    for i in range(depth):
        p.update({f"layers.{i}.{k}": v
                  for k, v in with_shared_alias(rand_params(shapes_diffusion_layer(D), seed=seed + i, std=std)).items()})
    return p


@pytest.mark.timeout(400)
@pytest.mark.parametrize("precision", ["fp32", "f16"], indirect=True)
def test_c5_diffusion_layer_D768_N400_5_samples(precision):
    from boltz_mlx_amd.layers.transformersv2 import DiffusionTransformer
    from boltz_mlx_amd.weights import load_module

    D, H, N, mult = 768, 16, 400, 5
    p = _diff_params(D, 1, 0.02, seed=1300)
    rng = np.random.default_rng(1301)
    a = rng.standard_normal((mult, N, D))
    s = rng.standard_normal((mult, N, D))
    bias = rng.standard_normal((1, N, N, H))
    mask = np.ones((mult, N))
    mask[:, N - N // 20:] = 0
    odt = np.float32 if precision == "fp32" else np.float64
    ref = OD.diffusion_transformer(a.astype(odt), s.astype(odt), bias.astype(odt), mask.astype(odt),
                                   cast(p, odt), 1, H, mult)
    m = load_module(DiffusionTransformer(depth=1, heads=H, dim=D), p).cuda()
    got = m(dev(a), dev(s), dev(bias), dev(mask), multiplicity=mult).cpu().numpy()
    check("C5 diffusion layer update", got - a, ref - a, precision)


@pytest.mark.timeout(600)
def test_c5_diffusion_stack_24_layers_f16_vs_fp32():
    from boltz_mlx_amd import kernels as K
    from boltz_mlx_amd.layers.transformersv2 import DiffusionTransformer
    from boltz_mlx_amd.weights import load_module, synthetic_state

    N, D, H, L, S = 400, 768, 16, 24, 5
    m = DiffusionTransformer(depth=L, heads=H, dim=D)
    load_module(m, synthetic_state(m, seed=5, std=0.02))
    m = m.cuda()
    g = torch.Generator(device="cuda").manual_seed(5)
    a = torch.randn((S, N, D), generator=g, device="cuda")
    s = torch.randn((S, N, D), generator=g, device="cuda")
    bias = 0.5 * torch.randn((1, N, N, L * H), generator=g, device="cuda")
    mask = torch.ones((S, N), device="cuda")
    mask[:, N - N // 20:] = 0
    old = K.PRECISION
    outs = {}
    try:
        for prec in ("fp32", "f16"):
            K.set_precision(prec)
            with torch.no_grad():
                outs[prec] = m(a, s, bias, mask, multiplicity=S)
            torch.cuda.synchronize()
    finally:
        K.set_precision(old)
    r = _rel_fro(outs["f16"] - a, outs["fp32"] - a)
    print(f"C5 24-layer stack f16 vs fp32: rel_fro(update)={r:.3e}", flush=True)
    assert torch.isfinite(outs["f16"]).all()
    assert r <= DIFF_STACK_REL_FRO


# ------------------------------------------------------------------------------------------------ dense masks, B = 2

@pytest.mark.timeout(300)
@pytest.mark.parametrize("precision", ["fp32", "f16"], indirect=True)
@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("N", [37, 200])
def test_tri_att_dense_random_mask_B2(precision, starting, N):
    """Two batch elements with independent dense random masks: the core's masked branch in almost every key block,
    fully masked rows 3 and 7, a masked key column."""
    from boltz_mlx_amd.layers.triangular_attention.attention import (TriangleAttentionEndingNode,
                                                                     TriangleAttentionStartingNode)

    D, C, H = 128, 32, 4
    rng = np.random.default_rng(1400 + N)
    p = rand_params(shapes_tri_att(D, C, H), seed=1401 + N, std=0.1)
    x = rng.standard_normal((2, N, N, D))
    mask = rand_mask(rng, (2, N, N))
    f32 = np.float32
    ref = O.tri_att(x.astype(f32), mask.astype(f32), cast(p, f32), starting, row_chunk=16)
    mod = load(TriangleAttentionStartingNode(D, C, H) if starting else TriangleAttentionEndingNode(D, C, H), p)
    got = mod(dev(x), dev(mask)).cpu().numpy()
    check(f"tri_att_{'start' if starting else 'end'} dense mask B=2 N={N}", got, ref, precision)


@pytest.mark.parametrize("precision", ["fp32", "f16"], indirect=True)
@pytest.mark.parametrize("outgoing", [True, False])
def test_tri_mul_dense_random_mask_B2(precision, outgoing):
    from boltz_mlx_amd.layers.triangular_mult import TriangleMultiplicationIncoming, TriangleMultiplicationOutgoing

    N, D = 67, 128
    rng = np.random.default_rng(1500)
    p = rand_params(shapes_tri_mul(D), seed=1501, std=0.1)
    x = rng.standard_normal((2, N, N, D))
    mask = rand_mask(rng, (2, N, N))
    odt = np.float32 if precision == "fp32" else np.float64
    ref = O.tri_mul(x.astype(odt), mask.astype(odt), cast(p, odt), outgoing)
    mod = load((TriangleMultiplicationOutgoing if outgoing else TriangleMultiplicationIncoming)(D), p)
    got = mod(dev(x), dev(mask)).cpu().numpy()
    check(f"tri_mul_{'out' if outgoing else 'in'} dense mask B=2", got, ref, precision)


@pytest.mark.parametrize("precision", ["fp32", "f16"], indirect=True)
def test_pairformer_layer_B2(precision):
    from boltz_mlx_amd.layers.pairformer import PairformerLayer

    N, cs, cz, H = 33, 384, 128, 16
    p = rand_params(shapes_layer(cs, cz, H), seed=1600, std=0.05)
    rng = np.random.default_rng(1601)
    z = rng.standard_normal((2, N, N, cz))
    s = rng.standard_normal((2, N, cs))
    tok = np.ones((2, N))
    tok[0, -4:] = 0
    tok[1, -9:] = 0
    pm = tok[:, :, None] * tok[:, None, :]
    f32 = np.float32
    s_r, z_r = O.pairformer_layer(s.astype(f32), z.astype(f32), tok.astype(f32), pm.astype(f32), cast(p, f32), H)
    s_g, z_g = load(PairformerLayer(cs, cz, H), p)(dev(s), dev(z), dev(tok), dev(pm))
    check("pairformer_layer B=2 z", z_g.cpu().numpy(), z_r, precision, F16_LAYER)
    check("pairformer_layer B=2 s", s_g.cpu().numpy(), s_r, precision, F16_LAYER)


@pytest.mark.parametrize("precision", ["fp32", "f16"], indirect=True)
def test_pairformer_module_B2(precision):
    """Two blocks over a batch of two with different padding: the module's schedule for B > 1 (each element's s track
    on the side stream, no norm_in carry between layers)."""
    from boltz_mlx_amd.layers.pairformer import PairformerModule

    N, cs, cz, H, nb = 29, 384, 128, 16, 2
    p = {}
    for i in range(nb):
        p.update({f"layers.{i}.{k}": v for k, v in rand_params(shapes_layer(cs, cz, H), seed=1700 + i, std=0.05).items()})
    rng = np.random.default_rng(1702)
    z = rng.standard_normal((2, N, N, cz))
    s = rng.standard_normal((2, N, cs))
    tok = np.ones((2, N))
    tok[0, -2:] = 0
    tok[1, -7:] = 0
    pm = tok[:, :, None] * tok[:, None, :]
    f32 = np.float32
    s_r, z_r = O.pairformer_module(s.astype(f32), z.astype(f32), tok.astype(f32), pm.astype(f32), cast(p, f32), nb, H)
    s_g, z_g = load(PairformerModule(cs, cz, nb, H), p)(dev(s), dev(z), dev(tok), dev(pm))
    check("pairformer_module B=2 z", z_g.cpu().numpy(), z_r, precision, F16_LAYER)
    check("pairformer_module B=2 s", s_g.cpu().numpy(), s_r, precision, F16_LAYER)


# ------------------------------------------------------------------------------------------------ xn contract

@pytest.mark.parametrize("starting", [True, False])
def test_tri_att_xn_reference_layout(starting):
    """f16: xn is the fp16 LayerNorm output, for the ending node already transposed (the reference's
    attention.py:95-100 contract); the result equals the call without xn bit for bit. fp32 ignores xn."""
    from boltz_mlx_amd import kernels as K
    from boltz_mlx_amd.layers.triangular_attention.attention import (TriangleAttentionEndingNode,
                                                                     TriangleAttentionStartingNode)

    N, D, C, H = 70, 128, 32, 4
    p = rand_params(shapes_tri_att(D, C, H), seed=1700, std=0.1)
    x, _, pm = pair_inputs(N, D, seed=1701, n_pad=5)
    pm[0, 2, 9] = 0
    mod = load(TriangleAttentionStartingNode(D, C, H) if starting else TriangleAttentionEndingNode(D, C, H), p)
    old = K.PRECISION
    try:
        K.set_precision("f16")
        xg, mg = dev(x), dev(pm)
        xn = mod.layer_norm.to_storage(xg)
        if not starting:
            xn = xn.transpose(1, 2).contiguous()
        a = mod(xg, mg)
        b = mod(xg, mg, xn=xn)
        torch.cuda.synchronize()
        assert torch.equal(a, b)
        if not starting:  # the natural layout is a different input for the ending node
            c = mod(xg, mg, xn=mod.layer_norm.to_storage(xg))
            assert not torch.equal(a, c)
        with pytest.raises(ValueError):
            mod(xg, mg, xn=xn.float())
        K.set_precision("fp32")
        a32 = mod(xg, mg)
        b32 = mod(xg, mg, xn=torch.zeros_like(xn))
        torch.cuda.synchronize()
        assert torch.equal(a32, b32)
    finally:
        K.set_precision(old)


@pytest.mark.parametrize("starting", [True, False])
def test_tri_att_keep_t(starting):
    """keep_t is an f16-path option of the reference (attention.py:130-131): in f16 the ending node returns its
    update in the attention frame (the transpose of keep_t=False's); the fp32 path ignores it and always returns the
    natural layout (attention.py:45-46, 91-92), as does the starting node in both modes."""
    from boltz_mlx_amd import kernels as K
    from boltz_mlx_amd.layers.triangular_attention.attention import (TriangleAttentionEndingNode,
                                                                     TriangleAttentionStartingNode)

    N, D, C, H = 45, 128, 32, 4
    p = rand_params(shapes_tri_att(D, C, H), seed=1710, std=0.1)
    x, _, pm = pair_inputs(N, D, seed=1711, n_pad=4)
    pm[0, 3, 11] = 0
    mod = load(TriangleAttentionStartingNode(D, C, H) if starting else TriangleAttentionEndingNode(D, C, H), p)
    old = K.PRECISION
    try:
        xg, mg = dev(x), dev(pm)
        K.set_precision("fp32")
        a32, b32 = mod(xg, mg), mod(xg, mg, keep_t=True)
        K.set_precision("f16")
        a16, b16 = mod(xg, mg), mod(xg, mg, keep_t=True)
        torch.cuda.synchronize()
        assert torch.equal(a32, b32)
        if starting:
            assert torch.equal(a16, b16)
        else:
            assert torch.equal(b16, a16.transpose(1, 2)) and not torch.equal(b16, a16)
    finally:
        K.set_precision(old)


def test_tri_mul_and_transition_xn():
    """f16 with B = 1: a given xn is used as the norm_in / norm output (equal to the call without it); fp32 ignores
    it (triangular_mult.py:23-29, transition.py:27-31)."""
    from boltz_mlx_amd import kernels as K
    from boltz_mlx_amd.layers.transition import Transition
    from boltz_mlx_amd.layers.triangular_mult import TriangleMultiplicationIncoming
    from conftest import shapes_transition

    N, D = 40, 128
    x, _, pm = pair_inputs(N, D, seed=1800, n_pad=3)
    tm = load(TriangleMultiplicationIncoming(D), rand_params(shapes_tri_mul(D), seed=1801, std=0.1))
    tr = load(Transition(D, 4 * D), rand_params(shapes_transition(D, 4 * D), seed=1802, std=0.1))
    old = K.PRECISION
    try:
        xg, mg = dev(x), dev(pm)
        for prec in ("f16", "fp32"):
            K.set_precision(prec)
            for mod, ln, args in ((tm, tm.norm_in, (mg,)), (tr, tr.norm, ())):
                xn = ln.to_storage(xg) if prec == "f16" else torch.zeros(xg.shape, dtype=torch.float16,
                                                                          device="cuda")
                a = mod(xg, *args)
                b = mod(xg, *args, xn=xn)
                torch.cuda.synchronize()
                assert torch.equal(a, b), (type(mod).__name__, prec)
    finally:
        K.set_precision(old)
