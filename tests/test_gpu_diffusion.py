"""GPU parity of the diffusion token transformer (boltz_mlx_amd/layers/transformersv2.py) and its kernels against
the numpy oracle (oracle/diffusion.py): fp32 within 1e-5 of the float32 oracle, f16 within the module gate of the
float64 oracle (max_rel 2e-2, rel_fro 5e-3)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from conftest import rand_params, shapes_diffusion_layer, with_shared_alias
from oracle import diffusion as OD

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


@pytest.mark.parametrize("D", [384, 768])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16])
def test_adaln_kernel(D, out_dtype):
    """sigmoid(scale) * LN(a) + shift with scale/shift strided views of a wider conditioning buffer whose rows are
    shared by consecutive groups of rows (row r uses r % rows_c)."""
    from boltz_mlx_amd import kernels as K

    rng = np.random.default_rng(D)
    rows, rows_c = 60, 20
    a = 2 * rng.standard_normal((rows, D)) + 0.5
    cond = rng.standard_normal((rows_c, 3, 2, D))
    c = dev(cond)
    got = K.adaln(dev(a), c[:, 1, 0], c[:, 1, 1], out_dtype).float().cpu().numpy()
    q = np.arange(rows) % rows_c
    ref = OD.sigmoid(cond[q, 1, 0]) * O.layer_norm(a) + cond[q, 1, 1]
    tol = 1e-5 if out_dtype == torch.float32 else 2e-3
    assert O.metrics(got, ref)["max_rel"] <= tol


@pytest.mark.parametrize("dt", [torch.float32, torch.float16])
def test_linear_gated_and_swiglu3(dt):
    from boltz_mlx_amd import kernels as K

    rng = np.random.default_rng(3)
    rows, Kd, M, rows_g = 70, 96, 80, 35
    x = rng.standard_normal((rows, Kd))
    w = 0.1 * rng.standard_normal((M, Kd))
    b = rng.standard_normal(M)
    gate = rng.standard_normal((rows_g, 2, M))
    y0 = rng.standard_normal((rows, M))
    y = dev(y0)
    g = dev(gate)
    xg, wg = dev(x, dt), dev(w, dt)
    K.linear_gated(xg, wg, g[:, 1], y, bias=dev(b))
    xr, wr = xg.double().cpu().numpy(), wg.double().cpu().numpy()
    ref = y0 + OD.sigmoid(gate[np.arange(rows) % rows_g, 1]) * (xr @ wr.T + b)
    assert O.metrics(y.cpu().numpy(), ref)["max_rel"] <= (1e-5 if dt == torch.float32 else 2e-3)
    h = dev(rng.standard_normal((rows, 3 * 48)), dt)
    hr = h.double().cpu().numpy()
    ref3 = OD.silu(hr[:, :48]) * hr[:, 48:96] * hr[:, 96:]
    got3 = K.swiglu3(h).double().cpu().numpy()
    assert O.metrics(got3, ref3)["max_rel"] <= (1e-5 if dt == torch.float32 else 3e-3)


@pytest.mark.parametrize("R,Kd,M", [(1, 64, 4), (130, 192, 260), (300, 768, 132), (257, 1536, 388)])
def test_gemm_f16_tiles(R, Kd, M):
    """The fp16 128 x 128 GEMM (K % 64 == 0, 16-byte aligned operands; odd and even K-stage counts, row and column
    tiles cut short) in all four epilogues against float64 on the same fp16 values, and against the fp32-operand
    kernel on those values."""
    from boltz_mlx_amd import kernels as K

    rng = np.random.default_rng(R + Kd + M)
    x = dev(rng.standard_normal((R, Kd)), torch.float16)
    w = dev(rng.standard_normal((M, Kd)) / np.sqrt(Kd), torch.float16)
    b = rng.standard_normal(M)
    gate = rng.standard_normal((7, 2, M))
    y0 = rng.standard_normal((R, M))
    xr, wr = x.double().cpu().numpy(), w.double().cpu().numpy()
    ref = xr @ wr.T + b
    sig = OD.sigmoid(gate[np.arange(R) % 7, 0])
    g = dev(gate)
    outs = []
    for x_in, w_in in ((x, w), (x.float(), w.float())):
        y16 = K.linear(x_in, w_in, bias=dev(b), out_dtype=torch.float16)
        y32 = K.linear(x_in, w_in, bias=dev(b), out_dtype=torch.float32)
        yacc = dev(y0)
        K.linear(x_in, w_in, bias=dev(b), out=yacc, accumulate=True)
        ygat = dev(y0)
        K.linear_gated(x_in, w_in, g[:, 0], ygat, bias=dev(b))
        torch.cuda.synchronize()
        assert O.metrics(y16.double().cpu().numpy(), ref)["max_rel"] <= 2e-3
        assert O.metrics(y32.cpu().numpy(), ref)["max_rel"] <= 1e-5
        assert O.metrics(yacc.cpu().numpy(), y0 + ref)["max_rel"] <= 1e-5
        assert O.metrics(ygat.cpu().numpy(), y0 + sig * ref)["max_rel"] <= 1e-5
        outs.append((y16, y32, yacc, ygat))
    for f, s in zip(*outs):
        assert O.metrics(f.double().cpu().numpy(), s.double().cpu().numpy())["max_rel"] <= 2e-3


@pytest.mark.parametrize("R,Kd,M", [(1, 16, 1), (129, 48, 64), (4100, 64, 512), (3000, 256, 64), (257, 32, 200)])
def test_linear_fp32_accuracy(R, Kd, M):
    """fp32 linear (the fp32-MFMA kernel for K % 32 == 0, the generic one otherwise; row and column tiles cut short)
    against float64 on the same fp32 values at fp32 accuracy, plain, with bias and accumulated; 0/1 operands (the
    pair counts' mask^T mask) give exact integers."""
    from boltz_mlx_amd import kernels as K

    rng = np.random.default_rng(R * Kd + M)
    x = rng.standard_normal((R, Kd)).astype(np.float32)
    w = (rng.standard_normal((M, Kd)) / np.sqrt(Kd)).astype(np.float32)
    b = rng.standard_normal(M).astype(np.float32)
    y0 = rng.standard_normal((R, M)).astype(np.float32)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    y = K.linear(dev(x), dev(w)).cpu().numpy()
    yb = K.linear(dev(x), dev(w), bias=dev(b)).cpu().numpy()
    yacc = dev(y0)
    K.linear(dev(x), dev(w), out=yacc, accumulate=True)
    assert O.metrics(y, ref)["max_rel"] <= 1e-6
    assert O.metrics(yb, ref + b)["max_rel"] <= 1e-6
    assert O.metrics(yacc.cpu().numpy(), ref + y0)["max_rel"] <= 1e-6
    xm = (rng.random((R, Kd)) > 0.3).astype(np.float32)
    wm = (rng.random((M, Kd)) > 0.3).astype(np.float32)
    assert np.array_equal(K.linear(dev(xm), dev(wm)).cpu().numpy(), xm @ wm.T)


@pytest.mark.parametrize("dt,R,Kd,M", [(torch.float32, 300, 64, 64), (torch.float32, 129, 48, 20),
                                       (torch.float16, 2100, 1024, 128), (torch.float16, 130, 192, 260)])
def test_linear_residual_equals_copy_and_accumulate(dt, R, Kd, M):
    """out = res + x w^T + bias written out of place equals copying res and accumulating, bit for bit, on the
    fp32-MFMA, generic, LDS-direct and register-staged fp16 kernels; res may be a strided row view."""
    from boltz_mlx_amd import kernels as K

    rng = np.random.default_rng(R + Kd + M)
    x = dev(rng.standard_normal((R, Kd)), dt)
    w = dev(rng.standard_normal((M, Kd)) / np.sqrt(Kd), dt)
    b = dev(rng.standard_normal(M))
    big = dev(rng.standard_normal((R, M + 12)))
    res = big[:, 4:4 + M]
    got = torch.empty((R, M), device="cuda")
    K.linear_residual(x, w, res, got, bias=b)
    want = res.contiguous().clone()
    K.linear(x, w, bias=b, out=want, accumulate=True)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_gemm_f16_large_grid_tiles():
    """A grid of 2048+ 128 x 128 tiles takes the 128 x 128 kernel (smaller grids the 64 x 64 one): its rows equal
    the 64 x 64 kernel's on the same rows bit for bit (same k order per element), and the last row tile, cut short,
    and a gated update match float64."""
    from boltz_mlx_amd import kernels as K

    R, Kd, M = 4000, 192, 8192
    rng = np.random.default_rng(21)
    x = dev(rng.standard_normal((R, Kd)), torch.float16)
    w = dev(rng.standard_normal((M, Kd)) / np.sqrt(Kd), torch.float16)
    b = dev(rng.standard_normal(M))
    big = K.linear(x, w, bias=b, out_dtype=torch.float32)
    small = K.linear(x[:100].contiguous(), w, bias=b, out_dtype=torch.float32)
    gate = dev(rng.standard_normal((3, M)))
    y = torch.ones((R, M), device="cuda")
    K.linear_gated(x, w, gate, y, bias=b)
    torch.cuda.synchronize()
    assert torch.equal(big[:100], small)
    xr, wr = x[-72:].double().cpu().numpy(), w.double().cpu().numpy()
    ref = xr @ wr.T + b.double().cpu().numpy()
    assert O.metrics(big[-72:].cpu().numpy(), ref)["max_rel"] <= 1e-5
    g = OD.sigmoid(gate.double().cpu().numpy()[np.arange(R - 72, R) % 3])
    assert O.metrics(y[-72:].cpu().numpy(), 1 + g * ref)["max_rel"] <= 1e-5


def _params(D, depth, std, seed):
    p = {}
    for i in range(depth):
        p.update({f"layers.{i}.{k}": v
                  for k, v in with_shared_alias(rand_params(shapes_diffusion_layer(D), seed=seed + i, std=std)).items()})
    return p


@pytest.mark.parametrize("precision", ["fp32", "f16"], indirect=True)
@pytest.mark.parametrize("D,H,N,mult,std", [(64, 4, 13, 2, 0.2), (768, 16, 24, 2, 0.04)])
def test_diffusion_transformer(precision, D, H, N, mult, std):
    from boltz_mlx_amd.layers.transformersv2 import DiffusionTransformer
    from boltz_mlx_amd.weights import load_module

    depth, B = 2, 1
    p = _params(D, depth, std, seed=D)
    rng = np.random.default_rng(N)
    a = rng.standard_normal((B * mult, N, D))
    s = rng.standard_normal((B * mult, N, D))
    bias = rng.standard_normal((B, N, N, depth * H))
    mask = np.ones((B * mult, N))
    mask[:, -3:] = 0
    mask[1, 2] = 0
    odt = np.float32 if precision == "fp32" else np.float64
    ref = OD.diffusion_transformer(a.astype(odt), s.astype(odt), bias.astype(odt), mask.astype(odt),
                                   {k: v.astype(odt) for k, v in p.items()}, depth, H, mult)
    m = load_module(DiffusionTransformer(depth=depth, heads=H, dim=D), p).cuda()
    got = m(dev(a), dev(s), dev(bias), dev(mask), multiplicity=mult).cpu().numpy()
    # compare the updates (the residual a dominates the output)
    mt = O.metrics(got - a, ref - a)
    print(f"diffusion transformer D={D} [{precision}]: {mt}", flush=True)
    assert mt["finite"]
    if precision == "fp32":
        assert mt["max_rel"] <= 1e-5, mt
    else:
        assert mt["max_rel"] <= 2e-2 and mt["rel_fro"] <= 5e-3, mt


@pytest.mark.parametrize("precision", ["fp32"], indirect=True)
def test_diffusion_layer_forward_and_shared_conditioning(precision):
    """A layer called on its own equals layer 0 of the stack, and conditioning s shared by the samples (one row
    group) gives the same result as s repeated per sample."""
    from boltz_mlx_amd.layers.transformersv2 import DiffusionTransformer
    from boltz_mlx_amd.weights import load_module

    D, H, N, mult = 64, 4, 9, 3
    p = _params(D, 1, 0.2, seed=5)
    rng = np.random.default_rng(6)
    a = rng.standard_normal((mult, N, D))
    s1 = rng.standard_normal((1, N, D))
    bias = rng.standard_normal((1, N, N, H))
    mask = np.ones((mult, N))
    m = load_module(DiffusionTransformer(depth=1, heads=H, dim=D), p).cuda()
    full = m(dev(a), dev(np.repeat(s1, mult, 0)), dev(bias), dev(mask), multiplicity=mult)
    shared = m(dev(a), dev(np.repeat(s1, mult, 0)), dev(bias), dev(mask), multiplicity=mult,
               cond=m.precompute_cond(dev(s1)))
    one = m.layers[0](dev(a), dev(np.repeat(s1, mult, 0)), dev(bias), dev(mask), multiplicity=mult)
    torch.cuda.synchronize()
    assert torch.equal(full, shared)
    assert torch.equal(full, one)


@pytest.mark.parametrize("hd", [16, 24, 32, 48, 64])
@pytest.mark.parametrize("N", [64, 132])
@pytest.mark.parametrize("all_masked", [False, True])
def test_seq_attention_mfma_vs_valu(hd, N, all_masked):
    """The fp16 MFMA sequence attention (head widths 16-64, N % 4 == 0, 16-byte rows; 24 as 32 with zero dims) against the VALU kernel on the
    same fp16 values (the VALU kernel is forced by a row pitch that is not a multiple of 8), within the reference's
    MMA-vs-scalar gate (5e-3), and against the float64 definition. Keys past N - 3 are masked; all_masked masks
    every key, which leaves the softmax of the unmasked logits (checked against the float64 definition only)."""
    from boltz_mlx_amd import kernels as K

    H = 3
    HD = H * hd
    rng = np.random.default_rng(hd * 1000 + N)
    qkvg = rng.standard_normal((N, 4 * HD)).astype(np.float16)
    bias = (2 * rng.standard_normal((H, N, N))).astype(np.float16)
    mask = np.ones(N, np.float32)
    mask[-3:] = 0
    if all_masked:
        mask[:] = 0
    a, bg, mg = dev(qkvg, torch.float16), dev(bias, torch.float16), dev(mask)
    fast = K.seq_attention_packed(a, bg, mg, 1e6, H)
    wide = torch.zeros((N, 4 * HD + 4), dtype=torch.float16, device="cuda")
    wide[:, :4 * HD] = a
    base, es = wide.data_ptr(), wide.element_size()
    slow = torch.empty((N, HD), dtype=torch.float16, device="cuda")
    K.call("bzpf_seq_attention", base, base + HD * es, base + 2 * HD * es, base + 3 * HD * es, 4 * HD + 4,
           bg.data_ptr(), mg.data_ptr(), 1e6, slow.data_ptr(), HD, K.F16, K.F16, N, H, hd,
           K._stream())
    torch.cuda.synchronize()
    f, sl = fast.float().cpu().numpy(), slow.float().cpu().numpy()
    if not all_masked:  # all keys masked: the fp32 VALU kernel keeps the rounding of logits near -1e6
        m = O.metrics(f, sl)
        assert m["finite"] and m["max_rel"] <= 5e-3, m
    x = qkvg.astype(np.float64)
    ref = np.empty((N, HD))
    for h in range(H):
        q, k, v, g = (x[:, c * HD + h * hd: c * HD + (h + 1) * hd] for c in range(4))
        lg = q @ k.T / np.sqrt(hd) + bias[h].astype(np.float64) + (1 - mask.astype(np.float64))[None, :] * -1e6
        ref[:, h * hd:(h + 1) * hd] = OD.sigmoid(g) * (O.softmax(lg, -1) @ v)
    m2 = O.metrics(f, ref)
    assert m2["max_rel"] <= 1e-2, m2


@pytest.mark.parametrize("hd", [16, 24, 32, 48, 64])
@pytest.mark.parametrize("N", [1, 37, 64, 130])
@pytest.mark.parametrize("bias16", [False, True])
def test_seq_attention_f32_mfma(hd, N, bias16):
    """fp32 sequence attention on the fp32 matrix cores (fp32 q / k / v / g, an fp32 or fp16 bias: the s track's
    arithmetic in both precision modes) against the float64 definition at the fp32 gate (1e-5 of the largest
    output) and against the VALU kernel on the same values (forced by a row pitch that is not a multiple of 4).
    Every seventh key and, for N > 4, the last two are masked."""
    from boltz_mlx_amd import kernels as K

    H = 3
    HD = H * hd
    rng = np.random.default_rng(hd * 7 + N)
    qkvg = rng.standard_normal((N, 4 * HD)).astype(np.float32)
    bias = (2 * rng.standard_normal((H, N, N))).astype(np.float16 if bias16 else np.float32)
    mask = np.ones(N, np.float32)
    mask[3::7] = 0
    if N > 4:
        mask[-2:] = 0
    a, bg, mg = dev(qkvg), dev(bias, torch.float16 if bias16 else torch.float32), dev(mask)
    fast = K.seq_attention_packed(a, bg, mg, 1e6, H)
    wide = torch.zeros((N, 4 * HD + 1), dtype=torch.float32, device="cuda")
    wide[:, :4 * HD] = a
    base, es = wide.data_ptr(), wide.element_size()
    slow = torch.empty((N, HD), dtype=torch.float32, device="cuda")
    K.call("bzpf_seq_attention", base, base + HD * es, base + 2 * HD * es, base + 3 * HD * es, 4 * HD + 1,
           bg.data_ptr(), mg.data_ptr(), 1e6, slow.data_ptr(), HD, K.F32, K.F16 if bias16 else K.F32, N, H, hd,
           K._stream())
    torch.cuda.synchronize()
    f, sl = fast.cpu().numpy(), slow.cpu().numpy()
    x = qkvg.astype(np.float64)
    ref = np.empty((N, HD))
    for h in range(H):
        q, k, v, g = (x[:, c * HD + h * hd: c * HD + (h + 1) * hd] for c in range(4))
        lg = q @ k.T / np.sqrt(hd) + bias[h].astype(np.float64) + (1 - mask.astype(np.float64))[None, :] * -1e6
        ref[:, h * hd:(h + 1) * hd] = OD.sigmoid(g) * (O.softmax(lg, -1) @ v)
    m, mv = O.metrics(f, ref), O.metrics(f, sl)
    print(f"seq_attention f32 hd={hd} N={N} bias16={bias16}: vs float64 {m['max_rel']:.2e}, vs VALU "
          f"{mv['max_rel']:.2e}", flush=True)
    assert m["finite"] and m["max_rel"] <= 1e-5, m
    assert mv["max_rel"] <= 1e-5, mv


def test_seq_attention_f32_mfma_all_keys_masked():
    """A sequence whose keys are all masked: the mask term is one shift of every logit, which the softmax cancels;
    the fp32 kernel leaves it out (as the fp16 one does), so the output is the unmasked softmax."""
    from boltz_mlx_amd import kernels as K

    N, H, hd = 70, 2, 24
    HD = H * hd
    rng = np.random.default_rng(5)
    qkvg = rng.standard_normal((N, 4 * HD)).astype(np.float32)
    bias = rng.standard_normal((H, N, N)).astype(np.float32)
    out = K.seq_attention_packed(dev(qkvg), dev(bias), dev(np.zeros(N, np.float32)), 1e6, H)
    x = qkvg.astype(np.float64)
    ref = np.empty((N, HD))
    for h in range(H):
        q, k, v, g = (x[:, c * HD + h * hd: c * HD + (h + 1) * hd] for c in range(4))
        ref[:, h * hd:(h + 1) * hd] = OD.sigmoid(g) * (O.softmax(q @ k.T / np.sqrt(hd) + bias[h], -1) @ v)
    m = O.metrics(out.cpu().numpy(), ref)
    assert m["finite"] and m["max_rel"] <= 1e-5, m


@pytest.mark.parametrize("dt,N", [(torch.float16, 68), (torch.float32, 68), (torch.float16, 67)])
def test_seq_attention_batched_samples(dt, N):
    """All samples in one launch (sample groups of `multiplicity` sharing a bias, a mask row each) equal one call per
    sample: the MFMA kernels in fp16 and fp32 (one grid over the samples), the VALU kernel for N % 4 != 0 in fp16
    (one launch per sample)."""
    from boltz_mlx_amd import kernels as K

    S, mult, H, hd = 6, 3, 4, 48
    rng = np.random.default_rng(11)
    qkvg = dev(rng.standard_normal((S, N, 4 * H * hd)), dt)
    bias = dev(2 * rng.standard_normal((S // mult, H, N, N)), dt)
    mask = np.ones((S, N), np.float32)
    mask[:, -5:] = 0
    mask[1, :7] = 0
    mask[4, :] = 0
    mg = dev(mask)
    batched = K.seq_attention_packed(qkvg, bias, mg, 1e6, H, multiplicity=mult)
    single = torch.stack([K.seq_attention_packed(qkvg[i], bias[i // mult], mg[i], 1e6, H) for i in range(S)])
    torch.cuda.synchronize()
    assert torch.equal(batched, single)


@pytest.mark.parametrize("precision", ["fp32", "f16"], indirect=True)
def test_step_graph_replays_equal_eager(precision):
    """The captured step replayed several times, with eager work and synchronisations between the replays and the
    output fed back as the next input, equals the eager forward bit for bit on every replay."""
    from boltz_mlx_amd.layers.transformersv2 import DiffusionStepGraph, DiffusionTransformer
    from boltz_mlx_amd.weights import load_module

    D, H, N, mult, depth = 128, 4, 36, 3, 2
    p = _params(D, depth, 0.1, seed=9)
    rng = np.random.default_rng(12)
    a = dev(rng.standard_normal((mult, N, D)))
    s = dev(rng.standard_normal((mult, N, D)))
    bias = dev(rng.standard_normal((1, N, N, depth * H)))
    mask = np.ones((mult, N))
    mask[:, -4:] = 0
    mk = dev(mask)
    m = load_module(DiffusionTransformer(depth=depth, heads=H, dim=D), p).cuda()
    cond, prepared = m.precompute_cond(s), m.prepare(bias)
    step = DiffusionStepGraph(m, a, cond, prepared, mk, multiplicity=mult)
    x_graph, x_eager = a.clone(), a.clone()
    for it in range(4):
        x_eager = m(x_eager, s, bias, mk, multiplicity=mult, cond=cond, prepared=prepared)
        torch.cuda.synchronize()
        x_graph = step(x_graph).clone()
        torch.cuda.synchronize()
        assert torch.equal(x_graph, x_eager), f"replay {it}"
        _ = (torch.randn(1000, device="cuda") * 2).sum().item()  # unrelated eager work between replays


@pytest.mark.parametrize("R,Kd,M", [(1537, 64, 132), (1600, 192, 2052), (2000, 768, 3072), (2100, 768, 772),
                                    (65600, 128, 128)])
def test_gemm_lds_direct_paths(R, Kd, M):
    """The LDS-direct GEMM (1536+ rows: 64 x 64 tiles, 192 x 128 for 2048+ output columns, 128 x 128 for 128 columns
    over 65,536+ rows; tiles dealt to the XCDs in contiguous ranges, ragged tile counts) in all four epilogues against
    float64, and bit for bit against the register-staged kernel on the first 100 rows (same k order per element)."""
    from boltz_mlx_amd import kernels as K

    rng = np.random.default_rng(R + Kd + M)
    x = dev(rng.standard_normal((R, Kd)), torch.float16)
    w = dev(rng.standard_normal((M, Kd)) / np.sqrt(Kd), torch.float16)
    b = dev(rng.standard_normal(M))
    gate = rng.standard_normal((400, M))
    y0 = rng.standard_normal((R, M))
    y16 = K.linear(x, w, bias=b, out_dtype=torch.float16)
    y32 = K.linear(x, w, bias=b, out_dtype=torch.float32)
    yacc = dev(y0)
    K.linear(x, w, bias=b, out=yacc, accumulate=True)
    ygat = dev(y0)
    K.linear_gated(x, w, dev(gate), ygat, bias=b)
    small16 = K.linear(x[:100].contiguous(), w, bias=b, out_dtype=torch.float16)
    small32 = K.linear(x[:100].contiguous(), w, bias=b, out_dtype=torch.float32)
    sgat = dev(y0[:100])
    K.linear_gated(x[:100].contiguous(), w, dev(gate), sgat, bias=b)
    torch.cuda.synchronize()
    assert torch.equal(y16[:100], small16) and torch.equal(y32[:100], small32) and torch.equal(ygat[:100], sgat)
    rows = np.r_[0:64, R - 70:R]  # the first tile and the ragged last ones
    ref = x[rows].double().cpu().numpy() @ w.double().cpu().numpy().T + b.double().cpu().numpy()
    assert O.metrics(y16[rows].double().cpu().numpy(), ref)["max_rel"] <= 2e-3
    assert O.metrics(y32[rows].cpu().numpy(), ref)["max_rel"] <= 1e-5
    assert O.metrics(yacc[rows].cpu().numpy(), y0[rows] + ref)["max_rel"] <= 1e-5
    sig = OD.sigmoid(gate[rows % 400])
    assert O.metrics(ygat[rows].cpu().numpy(), y0[rows] + sig * ref)["max_rel"] <= 1e-5


@pytest.mark.parametrize("np_,R,Kd,H", [(3, 1600, 768, 1536), (3, 1537, 64, 64), (2, 2000, 192, 256),
                                        (2, 1600, 128, 96)])
def test_linear_swiglu_lds_direct(np_, R, Kd, H):
    """The gated product as the LDS-direct GEMM's epilogue (1536+ rows, H a multiple of 64; H = 96 keeps the
    register-staged kernel) against float64, and bit for bit against the register-staged kernel on 100 rows."""
    from boltz_mlx_amd import kernels as K

    rng = np.random.default_rng(np_ * R + H)
    x = dev(rng.standard_normal((R, Kd)), torch.float16)
    w = dev(rng.standard_normal((np_ * H, Kd)) / np.sqrt(Kd), torch.float16)
    if np_ == 3:
        wg = K.group_swiglu3_rows(w[:H], w[H:2 * H], w[2 * H:])
        run = K.linear_swiglu3
    else:
        wg = K.group_swiglu_rows(w[:H], w[H:])
        run = K.linear_swiglu
    fused = run(x, wg)
    small = run(x[:100].contiguous(), wg)
    torch.cuda.synchronize()
    assert torch.equal(fused[:100], small)
    rows = np.r_[0:40, R - 40:R]
    h = x[rows].double().cpu().numpy() @ w.double().cpu().numpy().T
    ref = OD.silu(h[:, :H]) * h[:, H:2 * H]
    if np_ == 3:
        ref = ref * h[:, 2 * H:]
    assert O.metrics(fused[rows].double().cpu().numpy(), ref)["max_rel"] <= 2e-3


@pytest.mark.parametrize("R,Kd,H", [(70, 64, 32), (300, 768, 1536), (129, 192, 96)])
def test_linear_swiglu3_fused(R, Kd, H):
    """The fused feed-forward GEMM (gated product in the epilogue, grouped weight rows) against float64 on the same
    fp16 values, and against the unfused linear + swiglu3 (which rounds the [R, 3H] product to fp16 first)."""
    from boltz_mlx_amd import kernels as K

    rng = np.random.default_rng(R + H)
    x = dev(rng.standard_normal((R, Kd)), torch.float16)
    w = dev(rng.standard_normal((3 * H, Kd)) / np.sqrt(Kd), torch.float16)
    fused = K.linear_swiglu3(x, K.group_swiglu3_rows(w[:H], w[H:2 * H], w[2 * H:]))
    unfused = K.swiglu3(K.linear(x, w))
    torch.cuda.synchronize()
    h = x.double().cpu().numpy() @ w.double().cpu().numpy().T
    ref = OD.silu(h[:, :H]) * h[:, H:2 * H] * h[:, 2 * H:]
    assert O.metrics(fused.double().cpu().numpy(), ref)["max_rel"] <= 2e-3
    assert O.metrics(fused.double().cpu().numpy(), unfused.double().cpu().numpy())["max_rel"] <= 5e-3


@pytest.mark.parametrize("R,Kd,H", [(70, 64, 32), (300, 384, 1536), (257, 64, 256)])
def test_linear_swiglu_fused(R, Kd, H):
    """The two-factor form (Transition's SwiGLU, 64-row weight groups) against float64 and the unfused kernels."""
    from boltz_mlx_amd import kernels as K

    rng = np.random.default_rng(R * 3 + H)
    x = dev(rng.standard_normal((R, Kd)), torch.float16)
    w = dev(rng.standard_normal((2 * H, Kd)) / np.sqrt(Kd), torch.float16)
    fused = K.linear_swiglu(x, K.group_swiglu_rows(w[:H], w[H:]))
    unfused = K.swiglu(K.linear(x, w))
    torch.cuda.synchronize()
    h = x.double().cpu().numpy() @ w.double().cpu().numpy().T
    ref = OD.silu(h[:, :H]) * h[:, H:]
    assert O.metrics(fused.double().cpu().numpy(), ref)["max_rel"] <= 2e-3
    assert O.metrics(fused.double().cpu().numpy(), unfused.double().cpu().numpy())["max_rel"] <= 5e-3


def test_seq_attention_wave_count_variants_agree():
    """A grid of 512+ 128-query blocks runs 4-wave workgroups, a smaller one 2-wave workgroups; a query's result does
    not depend on how many query tiles share its workgroup: 32 samples in one call equal 32 single-sample calls
    bit for bit."""
    from boltz_mlx_amd import kernels as K

    S, mult, N, H, hd = 32, 4, 200, 8, 32
    rng = np.random.default_rng(31)
    qkvg = dev(rng.standard_normal((S, N, 4 * H * hd)), torch.float16)
    bias = dev(rng.standard_normal((S // mult, H, N, N)), torch.float16)
    mask = np.ones((S, N), np.float32)
    mask[:, -9:] = 0
    mg = dev(mask)
    batched = K.seq_attention_packed(qkvg, bias, mg, 1e6, H, multiplicity=mult)
    single = torch.stack([K.seq_attention_packed(qkvg[i], bias[i // mult], mg[i], 1e6, H) for i in range(S)])
    torch.cuda.synchronize()
    assert torch.equal(batched, single)
