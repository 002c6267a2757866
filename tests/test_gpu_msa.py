"""GPU parity of the MSA-block kernels and modules (boltz_mlx_amd/layers/outer_product_mean.py, pair_averaging.py,
msa.py) against the numpy oracle (oracle/msa.py). Gates follow the reference's own MSA kernel tests
(tests/test_msa_kernels.py): the fp32 reductions within 1e-5 (relative Frobenius) / 1e-4 (max) of float64 on the
same fp32 operands, the fp16-stored outer sum within one fp16 rounding (2^-10 of the largest value), modules in fp32
within 1e-5 relative Frobenius and in f16 mode within 3e-3."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from conftest import pair_inputs, rand_params, shapes_msa_layer, shapes_opm, shapes_pwa
from oracle import msa as OM

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


def _opm_inputs(S, N, seed):
    rng = np.random.default_rng(seed)
    ab = rng.standard_normal((S, N, 64)).astype(np.float32)
    mask = (rng.random((S, N)) > 0.2).astype(np.float32)
    mask[0] = 1
    return ab, mask


@pytest.mark.parametrize("S,N,i_base,n_i", [(249, 37, 0, 37), (40, 13, 3, 7), (33, 5, 0, 5), (64, 70, 64, 6),
                                            (17, 130, 5, 120)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16])
def test_opm_outer(S, N, i_base, n_i, out_dtype):
    from boltz_mlx_amd import kernels as K

    ab, mask = _opm_inputs(S, N, S + N)
    got = K.opm_outer(dev(ab), dev(mask), i_base, n_i, out_dtype=out_dtype).double().cpu().numpy()
    ref = OM.opm_outer(ab.astype(np.float64), mask.astype(np.float64))[i_base:i_base + n_i].reshape(n_i * N, 1024)
    m = O.metrics(got, ref)
    assert m["finite"]
    if out_dtype == torch.float32:
        assert m["rel_fro"] < 1e-5 and m["max_rel"] < 1e-5, m
    else:
        assert np.abs(got - ref).max() <= np.abs(ref).max() * 2.0 ** -10, m


@pytest.mark.parametrize("S,N", [(37, 5), (16, 3), (1, 2)])
def test_opm_split_parts_and_layout(S, N):
    """The split planes hold x = fp32(mask * ab) as x1 = bf16(x), x2 = bf16(x - x1), x3 = x - x1 - x2 (exact),
    chunk (g, n, p, h) = part p of channels 32 h .. + 31 of token n over MSA rows 16 g .. + 15, zeros past S."""
    from boltz_mlx_amd import kernels as K

    ab, mask = _opm_inputs(S, N, 7 * S + N)
    ab[0, 0, :4] = [1e-30, -3e38, 1.0 + 2.0 ** -20, 0.0]  # tiny, huge, a value needing all three parts, zero
    got = K.opm_split(dev(ab), dev(mask)).cpu()
    G = (S + 15) // 16
    assert got.shape == (G, N, 3, 2, 32, 16) and got.dtype == torch.bfloat16
    x = np.zeros((G * 16, N, 64), np.float32)
    x[:S] = ab * mask[:, :, None]  # the fp32 products
    xt = torch.from_numpy(x)
    p1 = xt.to(torch.bfloat16)  # round to nearest even
    p2 = (xt - p1.float()).to(torch.bfloat16)
    p3 = (xt - p1.float() - p2.float()).to(torch.bfloat16)
    assert torch.equal(p3.float(), xt - p1.float() - p2.float())  # the third part is exact
    # [G * 16, N, 2 * 32] -> [G, N, part, h, c, k]
    want = torch.stack([p1, p2, p3]).view(3, G, 16, N, 2, 32).permute(1, 3, 0, 4, 5, 2)
    assert torch.equal(got.view(torch.int16), want.contiguous().view(torch.int16))


@pytest.mark.parametrize("S,N", [(37, 5), (64, 130), (17, 9)])
def test_opm_ln_split(S, N):
    """The planes from the MSA itself: their three parts add up to mask * (LN(m) W_ab^T) (LN as bzpf_layernorm, the
    product fp32-accurate), in the opm_split layout, zeros past S; the outer sum over them matches the oracle."""
    from boltz_mlx_amd import kernels as K

    rng = np.random.default_rng(S * N)
    m = (rng.standard_normal((S, N, 64)) * 1.5 + 0.2).astype(np.float32)
    mask = (rng.random((S, N)) > 0.2).astype(np.float32)
    w_ab = (rng.standard_normal((64, 64)) / 8).astype(np.float32)

    class LN:
        weight = dev(1 + 0.1 * rng.standard_normal(64))
        bias = dev(0.1 * rng.standard_normal(64))
        eps = 1e-5

    planes = K.opm_ln_split(dev(m), LN, dev(w_ab), dev(mask))
    G = (S + 15) // 16
    x = planes.float().sum(2).double().cpu().numpy()  # [G, N, 2, 32, 16]: the parts' sum is exact
    got = x.transpose(0, 4, 1, 2, 3).reshape(G * 16, N, 64)
    mn = K.layer_norm(dev(m.reshape(S * N, 64)), LN.weight, LN.bias, LN.eps).cpu().numpy().astype(np.float64)
    ab = (mn @ w_ab.astype(np.float64).T).reshape(S, N, 64)
    ref = np.zeros((G * 16, N, 64))
    ref[:S] = ab * mask[:, :, None]
    assert np.all(got[S:] == 0)
    assert O.metrics(got[:S], ref[:S])["max_rel"] <= 1e-6
    num = K.opm_counts(dev(mask))
    out = K.opm_outer_planes(planes, num, S, N, out_dtype=torch.float32).double().cpu().numpy()
    oref = OM.opm_outer(ab, mask.astype(np.float64)).reshape(N * N, 1024)
    assert O.metrics(out, oref)["max_rel"] < 1e-5


def test_opm_outer_zero_count_pair():
    """Two tokens that never share an unmasked MSA row: their pair's count is 0, clamped to 1, and z is 0."""
    from boltz_mlx_amd import kernels as K

    ab, mask = _opm_inputs(20, 9, 3)
    mask[:, 2] = np.arange(20) % 2
    mask[:, 6] = 1 - np.arange(20) % 2
    got = K.opm_outer(dev(ab), dev(mask), out_dtype=torch.float32).cpu().numpy().reshape(9, 9, 1024)
    ref = OM.opm_outer(ab.astype(np.float64), mask.astype(np.float64))
    assert np.all(got[2, 6] == 0) and np.all(got[6, 2] == 0)
    assert O.metrics(got, ref)["max_rel"] < 1e-5


@pytest.mark.parametrize("N", [5, 37, 130])
@pytest.mark.parametrize("wdt", [torch.float16, torch.float32])
def test_pwa_weights(N, wdt):
    from boltz_mlx_amd import kernels as K

    rng = np.random.default_rng(N)
    z = (rng.standard_normal((N, N, 128)) * 3 + 1).astype(np.float32)
    pm = (rng.random((N, N)) > 0.2).astype(np.float32)
    pm[:, 0] = 1
    pm[1] = 0  # a row with every key masked
    p = rand_params(shapes_pwa(), seed=N, std=128 ** -0.5)
    wz = torch.tensor(p["proj_z.weight"], dtype=wdt).float()

    class LN:
        weight, bias, eps = dev(p["norm_z.weight"]), dev(p["norm_z.bias"]), 1e-5

    logits = K.pair_bias(dev(z), LN, wz.cuda())
    w = K.pwa_softmax(logits, dev(pm), 1e6).cpu().numpy()
    ref = OM.pwa_weights(z.astype(np.float64), pm.astype(np.float64),
                         {**p, "proj_z.weight": wz.double().numpy()})
    assert w.shape == (8, N, (N + 15) // 16 * 16) and np.all(w[:, :, N:] == 0)
    assert np.isfinite(w).all() and np.abs(w.sum(-1) - 1).max() < 1e-5
    # row 1 masks every key: its fp32 logits - 1e6 round to multiples of 1/16 (as the reference's fp32 logits do),
    # which the float64 definition does not; the other rows are compared exactly
    keep = np.arange(N) != 1
    m = O.metrics(w[:, keep, :N], ref[:, keep])
    assert m["rel_fro"] < 1e-5 and m["max_rel"] < 1e-5, m


@pytest.mark.parametrize("N", [37, 64, 130])
def test_pwa_wsplit_parts_and_layout(N):
    """The weight chunks hold w = w1 + w2 + w3 (w1 = bf16(w), w2 = bf16(w - w1), w3 the exact rest) with chunk
    (h, ib, jg, p) = part p of rows 32 ib .. + 31 and tokens 16 jg .. + 15, zeros past N and in the padding stage."""
    from boltz_mlx_amd import kernels as K

    rng = np.random.default_rng(N)
    H, ldw = 8, (N + 15) // 16 * 16
    w = np.zeros((H, N, ldw), np.float32)
    x = rng.random((H, N, N)).astype(np.float32)
    w[:, :, :N] = x / x.sum(-1, keepdims=True)
    got = K.pwa_wsplit(dev(w)).cpu()
    nib, G = (N + 31) // 32, (ldw // 16 + 1) // 2 * 2
    assert got.shape == (H, nib, G, 3, 32, 16)
    full = torch.zeros((H, nib * 32, G * 16))
    full[:, :N, :ldw] = torch.from_numpy(w)
    p1 = full.to(torch.bfloat16)
    p2 = (full - p1.float()).to(torch.bfloat16)
    p3 = (full - p1.float() - p2.float()).to(torch.bfloat16)
    assert torch.equal(p1.float() + p2.float() + p3.float(), full)
    # [H, nib * 32, G * 16] per part -> [H, ib, jg, part, row, token]
    want = torch.stack([p1, p2, p3]).view(3, H, nib, 32, G, 16).permute(1, 2, 4, 0, 3, 5)
    assert torch.equal(got.view(torch.int16), want.contiguous().view(torch.int16))


@pytest.mark.parametrize("rows,M", [(1, 256), (300, 512), (4100, 512), (129, 768)])
def test_ln_linear_f32(rows, M):
    """The fused LayerNorm + projection against bzpf_layernorm's fp32 output times W in float64: the LayerNorm is the
    same arithmetic, the product fp32-accurate (row tiles cut short, one to three column blocks)."""
    from boltz_mlx_amd import kernels as K

    rng = np.random.default_rng(rows + M)
    x = (rng.standard_normal((rows, 64)) * 2 + 0.3).astype(np.float32)
    w = (rng.standard_normal((M, 64)) / 8).astype(np.float32)

    class LN:
        weight = dev(1 + 0.1 * rng.standard_normal(64))
        bias = dev(0.1 * rng.standard_normal(64))
        eps = 1e-5

    got = K.ln_linear_f32(dev(x), LN, dev(w)).cpu().numpy()
    xn = K.layer_norm(dev(x), LN.weight, LN.bias, LN.eps).cpu().numpy().astype(np.float64)
    assert O.metrics(got, xn @ w.astype(np.float64).T)["max_rel"] <= 1e-6


@pytest.mark.parametrize("S,N", [(249, 37), (1, 130), (7, 64), (6, 200)])
def test_pwa_avg(S, N):
    from boltz_mlx_amd import kernels as K

    rng = np.random.default_rng(S * N)
    H = 8
    ldw = (N + 15) // 16 * 16
    w = np.zeros((H, N, ldw), np.float32)
    x = rng.random((H, N, N)).astype(np.float32)
    w[:, :, :N] = x / x.sum(-1, keepdims=True)
    vg = rng.standard_normal((S * N, 2 * H * 32)).astype(np.float32)
    vgd = dev(vg)
    got = K.pwa_avg(dev(w), vgd[:, :256], vgd[:, 256:], S, N).cpu().numpy()
    ref = OM.pwa_avg(w[:, :, :N].astype(np.float64), vg[:, :256].reshape(S, N, 256).astype(np.float64),
                     vg[:, 256:].reshape(S, N, 256).astype(np.float64)).reshape(S * N, 256)
    m = O.metrics(got, ref)
    assert m["rel_fro"] < 1e-5 and m["max_rel"] < 1e-4, m


@pytest.mark.parametrize("precision", ["fp32", "f16"], indirect=True)
@pytest.mark.parametrize("S,N", [(249, 37), (64, 130)])
def test_opm_module(precision, S, N):
    from boltz_mlx_amd.layers.outer_product_mean import OuterProductMean
    from boltz_mlx_amd.weights import load_module

    p = rand_params(shapes_opm(), seed=S + N, std=0.1)
    rng = np.random.default_rng(S)
    m = rng.standard_normal((1, S, N, 64))
    mask = (rng.random((1, S, N)) > 0.2).astype(np.float64)
    mask[:, 0] = 1
    mod = load_module(OuterProductMean(64, 32, 128), p).cuda()
    got = mod(dev(m), dev(mask)).cpu().numpy()
    ref = OM.outer_product_mean(m, mask, p)
    mt = O.metrics(got, ref)
    assert mt["finite"]
    assert mt["rel_fro"] < (1e-5 if precision == "fp32" else 3e-3), mt


@pytest.mark.parametrize("precision", ["fp32", "f16"], indirect=True)
@pytest.mark.parametrize("S,N", [(249, 37), (1, 130), (17, 64)])
def test_pwa_module(precision, S, N):
    from boltz_mlx_amd.layers.pair_averaging import PairWeightedAveraging
    from boltz_mlx_amd.weights import load_module

    p = rand_params(shapes_pwa(), seed=S * 7 + N, std=0.1)
    rng = np.random.default_rng(S + 1)
    m = rng.standard_normal((1, S, N, 64))
    z = rng.standard_normal((1, N, N, 128)) * 3
    pm = (rng.random((1, N, N)) > 0.15).astype(np.float64)
    pm[:, :, 0] = 1
    mod = load_module(PairWeightedAveraging(64, 128, 32, 8), p).cuda()
    got = mod(dev(m), dev(z), dev(pm)).cpu().numpy()
    if precision == "f16":
        p = {**p, "proj_z.weight": p["proj_z.weight"].astype(np.float16).astype(np.float64)}
    ref = OM.pair_weighted_averaging(m, z, pm, p)
    mt = O.metrics(got, ref)
    assert mt["finite"] and mt["rel_fro"] < 1e-5, mt


@pytest.mark.parametrize("precision", ["fp32", "f16"], indirect=True)
def test_msa_layer(precision):
    from boltz_mlx_amd.layers.msa import MSALayer
    from boltz_mlx_amd.weights import load_module

    N, S = 40, 23
    p = rand_params(shapes_msa_layer(), seed=31, std=0.05)
    z, _, pm = pair_inputs(N, 128, seed=32, n_pad=3)
    rng = np.random.default_rng(33)
    m = rng.standard_normal((1, S, N, 64))
    msa_mask = (rng.random((1, S, N)) > 0.1).astype(np.float64)
    mod = load_module(MSALayer(64, 128), p).cuda()
    zg, mg = mod(dev(z), dev(m), dev(pm), dev(msa_mask))
    zr, mr = OM.msa_layer(z, m, pm, msa_mask, p)
    # the 3 padded tokens mask every key of their PWA rows, whose fp32 logits - 1e6 round to multiples of 1/16 (as
    # the reference's do); the masked pair updates keep that out of the valid tokens, which are compared
    v = N - 3
    zg, mg = zg.cpu().numpy(), mg.cpu().numpy()
    assert np.isfinite(zg).all() and np.isfinite(mg).all()
    mz = O.metrics(zg[:, :v, :v] - z[:, :v, :v], zr[:, :v, :v] - z[:, :v, :v])
    mm = O.metrics(mg[:, :, :v] - m[:, :, :v], mr[:, :, :v] - m[:, :, :v])
    print(f"msa layer [{precision}]: z {mz} m {mm}", flush=True)
    assert mz["finite"] and mm["finite"]
    if precision == "fp32":
        assert mz["rel_fro"] < 1e-5 and mm["rel_fro"] < 1e-5, (mz, mm)
    else:
        assert mz["rel_fro"] < 5e-3 and mm["rel_fro"] < 5e-3, (mz, mm)


@pytest.mark.timeout(600)
@pytest.mark.parametrize("precision", ["fp32", "f16"], indirect=True)
def test_msa_layer_N260(precision):
    """The MSA layer at N = 260 (67,600 pairs: the outer product mean's output projection on the 128-column
    LDS-direct tiles for 65,536+ rows, the fused 64-channel kernels on full tiles) with 48 MSA rows, 6 padded tokens
    and a random MSA mask, against the oracle."""
    from boltz_mlx_amd.layers.msa import MSALayer
    from boltz_mlx_amd.weights import load_module

    N, S, npad = 260, 48, 6
    p = rand_params(shapes_msa_layer(), seed=41, std=0.05)
    z, _, pm = pair_inputs(N, 128, seed=42, n_pad=npad)
    rng = np.random.default_rng(43)
    m = rng.standard_normal((1, S, N, 64))
    msa_mask = (rng.random((1, S, N)) > 0.1).astype(np.float64)
    mod = load_module(MSALayer(64, 128), p).cuda()
    zg, mg = mod(dev(z), dev(m), dev(pm), dev(msa_mask))
    zr, mr = OM.msa_layer(z, m, pm, msa_mask, p)
    v = N - npad
    zg, mg = zg.cpu().numpy(), mg.cpu().numpy()
    assert np.isfinite(zg).all() and np.isfinite(mg).all()
    mz = O.metrics(zg[:, :v, :v] - z[:, :v, :v], zr[:, :v, :v] - z[:, :v, :v])
    mm = O.metrics(mg[:, :, :v] - m[:, :, :v], mr[:, :, :v] - m[:, :, :v])
    print(f"msa layer N={N} S={S} [{precision}]: z {mz} m {mm}", flush=True)
    if precision == "fp32":
        assert mz["rel_fro"] < 1e-5 and mm["rel_fro"] < 1e-5, (mz, mm)
    else:
        assert mz["rel_fro"] < 5e-3 and mm["rel_fro"] < 5e-3, (mz, mm)


@pytest.mark.parametrize("rows,H", [(300, 256), (5000, 256), (257, 128), (20000, 384)])
def test_transition64_f16(rows, H):
    """The fused 64-channel transition against the float64 formula on the same fp16 weights, with xn and the SwiGLU
    product rounded to fp16 as the kernel's operands (the reference's f16 transition), and against the unfused
    kernels (LayerNorm, GEMM with the SwiGLU epilogue, GEMM): the update within fp16 operand rounding."""
    from boltz_mlx_amd import kernels as K

    rng = np.random.default_rng(rows + H)
    x = (rng.standard_normal((rows, 64)) * 1.3 + 0.1).astype(np.float32)
    w12 = torch.tensor(rng.standard_normal((2 * H, 64)) / 8, dtype=torch.float16)
    w3 = torch.tensor(rng.standard_normal((64, H)) / 16, dtype=torch.float16)

    class LN:
        weight = dev(1 + 0.1 * rng.standard_normal(64))
        bias = dev(0.1 * rng.standard_normal(64))
        eps = 1e-5

    xg = dev(x)
    K.transition64_f16(xg, LN, w12.cuda(), w3.cuda())
    got = xg.cpu().numpy().astype(np.float64) - x
    xn = torch.tensor(O.layer_norm(x.astype(np.float64), LN.weight.double().cpu().numpy(),
                                   LN.bias.double().cpu().numpy())).half().double().numpy()
    h = xn @ w12.double().numpy().T
    a = torch.tensor(h[:, :H] / (1 + np.exp(-h[:, :H])) * h[:, H:]).half().double().numpy()
    ref = a @ w3.double().numpy().T
    m = O.metrics(got, ref)
    assert m["max_rel"] < 1e-2 and m["rel_fro"] < 2e-3, m
    xu = dev(x)
    xnu = K.layer_norm(xu, LN.weight, LN.bias, LN.eps, out_dtype=torch.float16)
    a16 = K.swiglu(K.linear(xnu, w12.cuda()))
    K.linear(a16, w3.cuda(), out=xu, out_dtype=torch.float32, accumulate=True)
    mu = O.metrics(got, xu.cpu().numpy().astype(np.float64) - x)
    assert mu["max_rel"] < 1e-2 and mu["rel_fro"] < 2e-3, mu


def test_msa_layer_fused_transition(monkeypatch):
    """The MSA layer in f16 mode with the m transition on the fused 64-channel kernel (taken from 16,384 rows; forced
    here at 23 x 40) against the oracle, at the f16 layer gate."""
    from boltz_mlx_amd import kernels as K
    from boltz_mlx_amd.layers import transition as T
    from boltz_mlx_amd.layers.msa import MSALayer
    from boltz_mlx_amd.weights import load_module

    monkeypatch.setattr(T, "FUSED_MIN_ROWS", 1)
    old = K.PRECISION
    K.set_precision("f16")
    try:
        N, S = 40, 23
        p = rand_params(shapes_msa_layer(), seed=31, std=0.05)
        z, _, pm = pair_inputs(N, 128, seed=32, n_pad=3)
        rng = np.random.default_rng(33)
        m = rng.standard_normal((1, S, N, 64))
        msa_mask = (rng.random((1, S, N)) > 0.1).astype(np.float64)
        mod = load_module(MSALayer(64, 128), p).cuda()
        zg, mg = mod(dev(z), dev(m), dev(pm), dev(msa_mask))
    finally:
        K.set_precision(old)
    zr, mr = OM.msa_layer(z, m, pm, msa_mask, p)
    v = N - 3
    zg, mg = zg.cpu().numpy(), mg.cpu().numpy()
    mz = O.metrics(zg[:, :v, :v] - z[:, :v, :v], zr[:, :v, :v] - z[:, :v, :v])
    mm = O.metrics(mg[:, :, :v] - m[:, :, :v], mr[:, :, :v] - m[:, :, :v])
    assert mz["rel_fro"] < 5e-3 and mm["rel_fro"] < 5e-3, (mz, mm)


@pytest.mark.parametrize("precision", ["fp32", "f16"], indirect=True)
def test_msa_layer_batch2(precision):
    """Two batch elements through the MSA layer (its first updates written out of place onto each element's inputs,
    the inputs left unchanged) against the oracle."""
    from boltz_mlx_amd.layers.msa import MSALayer
    from boltz_mlx_amd.weights import load_module

    N, S = 24, 19
    p = rand_params(shapes_msa_layer(), seed=41, std=0.05)
    z, _, pm = pair_inputs(N, 128, seed=42, n_pad=2, B=2)
    rng = np.random.default_rng(43)
    m = rng.standard_normal((2, S, N, 64))
    msa_mask = (rng.random((2, S, N)) > 0.1).astype(np.float64)
    mod = load_module(MSALayer(64, 128), p).cuda()
    zd, md = dev(z), dev(m)
    zg, mg = mod(zd, md, dev(pm), dev(msa_mask))
    assert torch.equal(zd, dev(z)) and torch.equal(md, dev(m))  # inputs untouched
    zr, mr = OM.msa_layer(z, m, pm, msa_mask, p)
    v = N - 2
    zg, mg = zg.cpu().numpy(), mg.cpu().numpy()
    mz = O.metrics(zg[:, :v, :v] - z[:, :v, :v], zr[:, :v, :v] - z[:, :v, :v])
    mm = O.metrics(mg[:, :, :v] - m[:, :, :v], mr[:, :, :v] - m[:, :, :v])
    assert mz["finite"] and mm["finite"]
    tol = 1e-5 if precision == "fp32" else 5e-3
    assert mz["rel_fro"] < tol and mm["rel_fro"] < tol, (mz, mm)
