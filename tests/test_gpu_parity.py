"""GPU parity: every bzpf module and kernel against the CPU oracle on the same seeded inputs.

fp32 mode is the parity build: max|d| / max|ref| <= 1e-5 against the oracle evaluated in float32 (the
reference's own CPU path is MLX fp32; float32 also reproduces its rounding of fully masked attention rows, where
every logit rounds to -1e9 and the softmax is uniform).

f16 mode (fp16 operands and intermediates, fp32 accumulation, statistics and softmax, fp32 residuals) is checked
against the float64 oracle with the tolerances F16_TOL below, in the spirit of the reference's fp16 gates
(tests/test_nax2_kernels.py: rel_fro <= 2e-3 / max_rel <= 1e-2 against same-rounding references; here the
reference is full precision, so the fp16 storage rounding of every intermediate counts too).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from conftest import pair_inputs, rand_params, shapes_attention, shapes_layer, shapes_transition, shapes_tri_att, shapes_tri_mul

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5
# (max_rel, rel_fro) for f16 mode vs the float64 oracle
F16_TOL = {"module": (2e-2, 5e-3), "layer": (3e-2, 1e-2)}


@pytest.fixture(scope="module", autouse=True)
def _device():
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    from boltz_mlx_amd import _lib

    _lib.load()
    torch.backends.cuda.matmul.allow_tf32 = False
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


def check(name, got, ref, prec, level="module"):
    m = O.metrics(got, ref)
    print(f"{name} [{prec}]: max_rel={m['max_rel']:.3e} rel_fro={m['rel_fro']:.3e} max_abs={m['max_abs']:.3e}",
          flush=True)
    assert m["finite"], name
    if prec == "fp32":
        assert m["max_rel"] <= FP32_TOL, (name, m)
    else:
        mr, rf = F16_TOL[level]
        assert m["max_rel"] <= mr and m["rel_fro"] <= rf, (name, m)


def oracle_dtype(prec):
    return np.float32 if prec == "fp32" else np.float64


def cast(d, dt):
    return {k: np.asarray(v, dtype=dt) for k, v in d.items()}


# ------------------------------------------------------------------------------------------------ LayerNorm

@pytest.mark.parametrize("D", [128, 384])
@pytest.mark.parametrize("io", [("f32", "f32"), ("f32", "f16"), ("f16", "f32")])
def test_layernorm(D, io):
    from boltz_mlx_amd import kernels as K

    rng = np.random.default_rng(D)
    rows = 1037
    x = rng.standard_normal((rows, D)) * 2 + 0.5
    w, b = 1 + 0.1 * rng.standard_normal(D), 0.1 * rng.standard_normal(D)
    tin = torch.float16 if io[0] == "f16" else torch.float32
    tout = torch.float16 if io[1] == "f16" else torch.float32
    xg = dev(x, tin)
    y = K.layer_norm(xg, dev(w), dev(b), 1e-5, out_dtype=tout).float().cpu().numpy()
    ref = O.layer_norm(xg.float().cpu().numpy().astype(np.float64), w, b, 1e-5)
    tol = 1e-5 if io == ("f32", "f32") else 2e-3
    assert O.metrics(y, ref)["max_rel"] <= tol


@pytest.mark.parametrize("trans_y,trans_out", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_add_ln(trans_y, trans_out):
    from boltz_mlx_amd import kernels as K
    from boltz_mlx_amd.layers.norm import LayerNorm

    N, D = 19, 128
    rng = np.random.default_rng(5)
    z = rng.standard_normal((N, N, D))
    y = rng.standard_normal((N, N, D))
    ln = LayerNorm(D).cuda()
    with torch.no_grad():
        ln.weight.copy_(dev(1 + 0.1 * rng.standard_normal(D)))
        ln.bias.copy_(dev(0.1 * rng.standard_normal(D)))
    zg = dev(z)
    out = K.add_ln(zg, dev(y), ln, scale=0.5, trans_y=bool(trans_y), trans_out=bool(trans_out),
                   out_dtype=torch.float32)
    yy = y.swapaxes(0, 1) if trans_y else y
    zr = z + 0.5 * yy
    lr = O.layer_norm(zr, ln.weight.detach().cpu().numpy(), ln.bias.detach().cpu().numpy())
    if trans_out:
        lr = lr.swapaxes(0, 1)
    assert O.metrics(zg.cpu().numpy(), zr)["max_rel"] <= 1e-6
    assert O.metrics(out.cpu().numpy(), lr)["max_rel"] <= 1e-5


# ------------------------------------------------------------------------------------------------ raw contraction

@pytest.mark.parametrize("N", [1, 63, 64, 65, 130])
@pytest.mark.parametrize("dt", [torch.float32, torch.float16])
def test_trimul_contract_raw(N, dt):
    from boltz_mlx_amd import kernels as K

    D = 8
    ld = K.row_pitch(N)
    rng = np.random.default_rng(N)
    ab = np.zeros((2 * D, N, ld))
    ab[:, :, :N] = rng.integers(-3, 4, size=(2 * D, N, N))  # small integers: exact in fp16 with fp32 accumulation
    o = K.trimul_contract(dev(ab, dt), N).float().cpu().numpy()[:, :, :N]
    ref = np.einsum("dik,djk->dij", ab[:D, :, :N], ab[D:, :, :N])
    if dt == torch.float16:
        ref = ref.astype(np.float16).astype(np.float64)  # the store rounds to fp16
    assert np.array_equal(o, ref)


@pytest.mark.parametrize("N", [130, 300])
@pytest.mark.parametrize("dt", [torch.float32, torch.float16])
def test_trimul_contract_key_extent_exact(N, dt):
    """With columns k >= k_len of ab zero (trailing padded tokens), the contraction stopped at k_len (rounded up to
    64) equals the full one bit for bit, for extents inside a stage, on a stage edge and of one key; 0 and N mean
    every key. Random fp16/fp32 values (not exact integers), so any change in the summed terms would show."""
    from boltz_mlx_amd import kernels as K

    D = 8
    ld = K.row_pitch(N)
    rng = np.random.default_rng(4100 + N)
    for k_len in (1, 64, N - 37, N - 1, 0, N):
        ab = np.zeros((2 * D, N, ld))
        kk = k_len if 0 < k_len < N else N
        ab[:, :, :kk] = rng.standard_normal((2 * D, N, kk))
        abd = dev(ab, dt)
        full = K.trimul_contract(abd, N)
        part = K.trimul_contract(abd, N, k_len)
        torch.cuda.synchronize()
        assert torch.equal(part[:, :, :N], full[:, :, :N]), (N, k_len)


@pytest.mark.parametrize("precision", ["f16"], indirect=True)
@pytest.mark.parametrize("outgoing", [True, False])
def test_tri_mul_in_mask_scope_equals_plain(precision, outgoing):
    """Inside pair_mask_scope the module contracts only up to the key extent of its (asymmetric, trailing-padded)
    mask; the update equals the call outside a scope (every key) bit for bit, in f16."""
    from boltz_mlx_amd import kernels as K
    from boltz_mlx_amd.layers.triangular_mult import TriangleMultiplicationIncoming, TriangleMultiplicationOutgoing

    N, D = 200, 128
    torch.manual_seed(3)
    m = (TriangleMultiplicationOutgoing if outgoing else TriangleMultiplicationIncoming)(D).cuda()
    with torch.no_grad():
        for prm in m.parameters():
            prm.normal_(0.0, 0.05)
    rng = np.random.default_rng(7)
    z = dev(rng.standard_normal((N, N, D)))
    tok = np.ones(N)
    tok[N - 70:] = 0
    mask = dev((tok[:, None] * tok[None, :] * (rng.random((N, N)) > 0.1)).astype(np.float32))
    xn = m.norm_in.to_storage(z).reshape(N * N, D)
    z1, z2 = z.clone(), z.clone()
    m.fused(xn, mask, z1, True)
    with K.pair_mask_scope():
        assert K.key_extent(mask, N, not outgoing) <= N - 70
        m.fused(xn, mask, z2, True)
    torch.cuda.synchronize()
    assert torch.equal(z1, z2)


# ------------------------------------------------------------------------------------------------ modules

TRI_N = [1, 2, 17, 33, 70, 130]


@pytest.mark.parametrize("precision", ["fp32", "f16"], indirect=True)
@pytest.mark.parametrize("outgoing", [True, False])
@pytest.mark.parametrize("N", TRI_N)
def test_tri_mul(precision, outgoing, N):
    from boltz_mlx_amd.layers.triangular_mult import TriangleMultiplicationIncoming, TriangleMultiplicationOutgoing

    D = 128
    p = rand_params(shapes_tri_mul(D), seed=100 + N, std=0.1)
    x, _, pm = pair_inputs(N, D, seed=N, n_pad=N // 5)
    if N > 3:
        pm[0, 1, 2] = 0
    odt = oracle_dtype(precision)
    ref = O.tri_mul(x.astype(odt), pm.astype(odt), cast(p, odt), outgoing)
    mod = load((TriangleMultiplicationOutgoing if outgoing else TriangleMultiplicationIncoming)(D), p)
    got = mod(dev(x), dev(pm)).cpu().numpy()
    check(f"tri_mul_{'out' if outgoing else 'in'} N={N}", got, ref, precision)


@pytest.mark.parametrize("precision", ["fp32", "f16"], indirect=True)
@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("N", [1, 2, 9, 33, 65, 100])
def test_tri_att(precision, starting, N):
    from boltz_mlx_amd.layers.triangular_attention.attention import (TriangleAttentionEndingNode,
                                                                     TriangleAttentionStartingNode)

    D, C, H = 128, 32, 4
    p = rand_params(shapes_tri_att(D, C, H), seed=200 + N, std=0.1)
    x, _, pm = pair_inputs(N, D, seed=N + 7, n_pad=N // 5)
    if N > 3:
        pm[0, 2, 1] = 0
    odt = np.float32  # fully masked rows follow the fp32 rounding (see the module docstring)
    ref = O.tri_att(x.astype(odt), pm.astype(odt), cast(p, odt), starting, row_chunk=16)
    mod = load(TriangleAttentionStartingNode(D, C, H) if starting else TriangleAttentionEndingNode(D, C, H), p)
    got = mod(dev(x), dev(pm)).cpu().numpy()
    check(f"tri_att_{'start' if starting else 'end'} N={N}", got, ref, precision)


@pytest.mark.parametrize("precision", ["fp32", "f16"], indirect=True)
@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("N", [17, 117])
def test_tri_att_other_head_shape(precision, starting, N):
    """3 heads of 16 channels at c_in = 128 (H * C != c_in, as in the reference's layer test,
    tests/test_triatt_mma.py:98): the GEMM + layout path and the VALU core (C = 16)."""
    from boltz_mlx_amd.layers.triangular_attention.attention import (TriangleAttentionEndingNode,
                                                                     TriangleAttentionStartingNode)

    D, C, H = 128, 16, 3
    p = rand_params(shapes_tri_att(D, C, H), seed=300 + N, std=0.1)
    x, _, pm = pair_inputs(N, D, seed=N + 9, n_pad=N // 6)
    pm[0, 3, 1] = 0
    ref = O.tri_att(x.astype(np.float32), pm.astype(np.float32), cast(p, np.float32), starting, row_chunk=16)
    mod = load(TriangleAttentionStartingNode(D, C, H) if starting else TriangleAttentionEndingNode(D, C, H), p)
    got = mod(dev(x), dev(pm)).cpu().numpy()
    check(f"tri_att_H3C16_{'start' if starting else 'end'} N={N}", got, ref, precision)


@pytest.mark.parametrize("precision", ["fp32", "f16"], indirect=True)
@pytest.mark.parametrize("dim,rows", [(128, 1), (128, 37), (128, 4111), (384, 5), (384, 300)])
def test_transition(precision, dim, rows):
    from boltz_mlx_amd.layers.transition import Transition

    p = rand_params(shapes_transition(dim, 4 * dim), seed=300 + rows, std=0.1)
    x = np.random.default_rng(rows).standard_normal((rows, dim))
    odt = oracle_dtype(precision)
    ref = O.transition(x.astype(odt), cast(p, odt))
    got = load(Transition(dim, 4 * dim), p)(dev(x)).cpu().numpy()
    check(f"transition dim={dim} rows={rows}", got, ref, precision)


@pytest.mark.parametrize("precision", ["fp32", "f16"], indirect=True)
@pytest.mark.parametrize("N", [5, 40, 129])
def test_attention_pair_bias(precision, N):
    from boltz_mlx_amd.layers.attentionv2 import AttentionPairBias

    cs, cz, H = 384, 128, 16
    p = rand_params(shapes_attention(cs, cz, H), seed=400 + N, std=0.1)
    rng = np.random.default_rng(N)
    s = rng.standard_normal((1, N, cs))
    z = rng.standard_normal((1, N, N, cz))
    mask = np.ones((1, N))
    mask[:, -(N // 5):] = 0 if N >= 5 else 1
    odt = np.float32
    ref = O.attention_pair_bias(s.astype(odt), z.astype(odt), mask.astype(odt), s.astype(odt), cast(p, odt), H)
    got = load(AttentionPairBias(cs, cz, H), p)(dev(s), dev(z), dev(mask), dev(s)).cpu().numpy()
    check(f"attention_pair_bias N={N}", got, ref, precision)


@pytest.mark.parametrize("N", [7, 64, 200])
def test_attention_pair_bias_f16_keeps_fp32_projections(N):
    """The reference's f16 mode keeps AttentionPairBias's projections, logits and softmax in fp32 and only computes
    the pair bias in fp16 (attentionv2.py:50-84; proj_z.1 is its one fp16 weight of the module). So f16 mode with a
    given pair bias computes exactly what fp32 mode computes with it, and without one it differs from the fp32
    oracle only by the fp16 bias: bounds 4e-3 max_rel and 1e-3 rel_fro, against the module gate's 2e-2 / 5e-3."""
    from boltz_mlx_amd import kernels as K
    from boltz_mlx_amd.layers.attentionv2 import AttentionPairBias

    cs, cz, H = 384, 128, 16
    p = rand_params(shapes_attention(cs, cz, H), seed=470 + N, std=0.1)
    rng = np.random.default_rng(471 + N)
    s, z = rng.standard_normal((1, N, cs)), rng.standard_normal((1, N, N, cz))
    mask = np.ones((1, N))
    mask[:, -(N // 6):] = 0 if N >= 6 else 1
    mod = load(AttentionPairBias(cs, cz, H), p)
    bias16 = dev(rng.standard_normal((1, H, N, N)), torch.float16)
    old = K.PRECISION
    try:
        out = {}
        for prec in ("fp32", "f16"):
            K.set_precision(prec)
            out[prec] = (mod(dev(s), dev(z), dev(mask), dev(s), pair_bias=bias16),
                         mod(dev(s), dev(z), dev(mask), dev(s), pair_bias=bias16.float()),
                         mod(dev(s), dev(z), dev(mask), dev(s)))
        torch.cuda.synchronize()
    finally:
        K.set_precision(old)
    assert torch.equal(out["fp32"][0], out["f16"][0]) and torch.equal(out["fp32"][1], out["f16"][1])
    assert torch.equal(out["f16"][0], out["f16"][1])  # the fp16 bias is added as it is
    ref = O.attention_pair_bias(s, z, mask, s, cast(p, np.float64), H)
    m = O.metrics(out["f16"][2].cpu().numpy(), ref)
    print(f"attention_pair_bias f16 N={N}: max_rel={m['max_rel']:.3e} rel_fro={m['rel_fro']:.3e}", flush=True)
    assert m["finite"] and m["max_rel"] <= 4e-3 and m["rel_fro"] <= 1e-3, m


@pytest.mark.parametrize("precision", ["fp32", "f16"], indirect=True)
@pytest.mark.parametrize("N,n_pad", [(1, 0), (2, 1), (24, 3), (50, 0), (65, 6)])
def test_pairformer_layer(precision, N, n_pad):
    from boltz_mlx_amd.layers.pairformer import PairformerLayer

    cs, cz, H = 384, 128, 16
    p = rand_params(shapes_layer(cs, cz, H), seed=500 + N, std=0.05)
    z, tok, pm = pair_inputs(N, cz, seed=N, n_pad=n_pad)
    s = np.random.default_rng(N + 1).standard_normal((1, N, cs))
    odt = np.float32
    s_r, z_r = O.pairformer_layer(s.astype(odt), z.astype(odt), tok.astype(odt), pm.astype(odt), cast(p, odt), H)
    layer = load(PairformerLayer(cs, cz, H), p)
    s_g, z_g = layer(dev(s), dev(z), dev(tok), dev(pm))
    check(f"pairformer_layer z N={N}", z_g.cpu().numpy(), z_r, precision, "layer")
    check(f"pairformer_layer s N={N}", s_g.cpu().numpy(), s_r, precision, "layer")


@pytest.mark.parametrize("precision", ["fp32", "f16"], indirect=True)
def test_pairformer_module_two_blocks(precision):
    from boltz_mlx_amd.layers.pairformer import PairformerModule

    N, cs, cz, H, nb = 20, 384, 128, 16, 2
    m = PairformerModule(cs, cz, nb, H)
    p = {}
    for i in range(nb):
        p.update({f"layers.{i}.{k}": v for k, v in rand_params(shapes_layer(cs, cz, H), seed=600 + i, std=0.05).items()})
    z, tok, pm = pair_inputs(N, cz, seed=61, n_pad=2)
    s = np.random.default_rng(62).standard_normal((1, N, cs))
    odt = np.float32
    s_r, z_r = O.pairformer_module(s.astype(odt), z.astype(odt), tok.astype(odt), pm.astype(odt), cast(p, odt), nb, H)
    m = load(m, p)
    s_g, z_g = m(dev(s), dev(z), dev(tok), dev(pm))
    check("pairformer_module z", z_g.cpu().numpy(), z_r, precision, "layer")
    check("pairformer_module s", s_g.cpu().numpy(), s_r, precision, "layer")


# ------------------------------------------------------------------------------------------------ fast vs slow core

def _tb_index(N, H):
    """Offsets of (h, j, k) for k < row_pitch(N) (the padded key range) in the fragment-ordered bias layout."""
    from boltz_mlx_amd import kernels as K

    ldk = K.row_pitch(N)
    njt, nkb = (N + 31) // 32, ldk // 64
    h = np.arange(H)[:, None, None]
    j = np.arange(N)[None, :, None]
    k = np.arange(ldk)[None, None, :]
    jt, q, kb, kk = j >> 5, j & 31, k >> 6, k & 63
    kt, p, hl, e = kk >> 5, (kk >> 3) & 3, (kk >> 2) & 1, kk & 3
    x = kt * 16 + p * 4 + e
    return ((h * njt + jt) * nkb + kb) * 2048 + (x >> 3) * 512 + (hl * 32 + q) * 8 + (x & 7)


@pytest.mark.parametrize("trans", [False, True])
def test_tri_bias_layout_matches_projection(trans):
    """The projection writes the bias at tri_bias_offsets and zero-fills keys past N (read back from the buffer)."""
    from boltz_mlx_amd import kernels as K

    N, H, C = 70, 4, 32
    rng = np.random.default_rng(3)
    xn = dev(rng.standard_normal((N * N, 128)), torch.float16)
    w = dev(0.1 * rng.standard_normal((4 * H * C + H, 128)), torch.float16)
    _, _, tb = K.triattn_proj(xn, w, trans, N, H, C)
    got = tb.float().cpu().numpy()
    ref = (xn.float() @ w[4 * H * C:].float().T).cpu().numpy() * K.LOG2E  # bias of position (a, b) = [a*N + b]
    ref = ref.reshape(N, N, H).transpose(2, 0, 1)
    if trans:  # the ending node's bias for (query j, key k) is the projection at (k, j)
        ref = ref.transpose(0, 2, 1)
    assert np.allclose(got[K.tri_bias_offsets(N, H)], ref, rtol=4e-3, atol=4e-3)
    assert np.all(got[_tb_index(N, H)[:, :, N:].ravel()] == 0)


@pytest.mark.parametrize("N", [1, 2, 17, 64, 65, 130])
@pytest.mark.parametrize("trans", [False, True])
def test_triattn_core_mfma_vs_valu(N, trans):
    """The fp16 MFMA flash core against the VALU reference kernel on identical fp16 inputs (the reference's own gate
    for its fp16 core against the fp32-softmax kernel: <= 5e-3, tests/test_triatt_nax.py). Rows with padded keys, a
    fully masked row and an asymmetric hole are included; trans reads the mask transposed (ending node)."""
    from boltz_mlx_amd import kernels as K

    H, C = 4, 32
    rng = np.random.default_rng(N)
    ldk = K.row_pitch(N)
    qkg = dev(rng.standard_normal((3 * H, N * N, C)), torch.float16)
    vt = dev(rng.standard_normal((H, N, C, ldk)), torch.float16)
    # bias in the fragment-ordered layout: keys past N are 0 (as the projection writes them); slots of queries past N
    # are never read for a valid query and hold NaN here to prove it
    tb_np = np.full(K.tri_bias_numel(N, H), np.nan, dtype=np.float32)
    dense = np.zeros((H, N, ldk), dtype=np.float32)
    dense[:, :, :N] = 2 * rng.standard_normal((H, N, N))
    tb_np[_tb_index(N, H).ravel()] = dense.ravel()
    tb = dev(tb_np, torch.float16)
    # V^T padding is never written by the projection: NaN there proves it is never used
    vt[..., N:] = float("nan")
    mask = np.ones((N, N), np.float32)
    if N > 4:
        mask[:, -2:] = 0
        mask[3, :] = 0
        mask[1, 2] = 0
    if N > 100:
        mask[5, :70] = 0  # a whole leading key block masked: the running maximum starts from masked logits
    mg = dev(mask)
    fast = K.triattn_core(qkg, vt, tb, mg, trans, 1e9, N, H, C, impl=2).float().cpu().numpy()
    slow = K.triattn_core(qkg, vt, tb, mg, trans, 1e9, N, H, C, impl=1).float().cpu().numpy()
    m = O.metrics(fast, slow)
    print(f"core mfma vs valu N={N} trans={trans}: {m}", flush=True)
    assert m["finite"] and m["max_rel"] <= 5e-3 and m["rel_fro"] <= 2e-3, m


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("n", [1, 7, 4099, 1_000_003])
def test_count_nonfinite(dtype, n):
    """bzpf_count_nonfinite against numpy on +inf, -inf and nan planted at seeded positions (the tail past the last
    16-byte vector and the very last element included), and on a clean tensor."""
    from boltz_mlx_amd import kernels as K

    rng = np.random.default_rng(n)
    x = (100 * rng.standard_normal(n)).astype(np.float32)
    assert int(K.count_nonfinite(dev(x, dtype)).item()) == 0
    pos = np.unique(np.concatenate([rng.integers(0, n, size=min(n, 37)), [n - 1]]))
    x[pos] = rng.choice([np.inf, -np.inf, np.nan], size=pos.size)
    if dtype == torch.float16:
        x[0] = 7e4 if 0 not in pos else x[0]  # rounds to +inf in fp16
    with np.errstate(over="ignore"):
        ref = int((~np.isfinite(x.astype(np.float16 if dtype == torch.float16 else np.float32))).sum())
    t = dev(x, dtype)
    assert int(K.count_nonfinite(t).item()) == ref
    assert int(K.count_nonfinite(t, t).item()) == 2 * ref


def test_fp16_guard_recomputes_in_fp32():
    """A transition whose fp16 hidden activations overflow (fc1/fc2 scaled up): the f16 pass leaves inf/nan in z,
    the guard sees them and recomputes the pass with the fp32 kernels, so forward returns exactly the fp32 result and
    counts one fallback (boltz_mlx/model.py:176-193). With the guard off, the f16 result is not finite."""
    from boltz_mlx_amd import kernels as K
    from boltz_mlx_amd.layers.pairformer import PairformerModule

    N, cs, cz, H = 24, 384, 128, 16
    p = {f"layers.0.{k}": v for k, v in rand_params(shapes_layer(cs, cz, H), seed=77, std=0.05).items()}
    for k in ("layers.0.transition_z.fc1.weight", "layers.0.transition_z.fc2.weight"):
        p[k] = 300.0 * p[k]
    z, tok, pm = pair_inputs(N, cz, seed=78, n_pad=2)
    s = np.random.default_rng(79).standard_normal((1, N, cs))
    args = (dev(s), dev(z), dev(tok), dev(pm))
    prev, prev_guard = K.PRECISION, K.GUARDS
    try:
        K.set_precision("fp32")
        ref = load(PairformerModule(cs, cz, 1, H), p)
        s32, z32 = ref(*args)
        assert torch.isfinite(z32).all() and torch.isfinite(s32).all()
        K.set_precision("f16")
        m = load(PairformerModule(cs, cz, 1, H), p)
        K.GUARDS = False
        _, z16 = m(*args)
        assert not torch.isfinite(z16).all()
        K.GUARDS = True
        s_g, z_g = m(*args)
        assert m.fp16_fallbacks == 1
        assert K.PRECISION == "f16"
        assert torch.equal(z_g, z32) and torch.equal(s_g, s32)
    finally:
        K.set_precision(prev)
        K.GUARDS = prev_guard


@pytest.mark.parametrize("N", [40, 129])
def test_triattn_core_ignores_padded_query_slots(N):
    """The bias slots of the padded queries past N (up to the 32-query tile) are never written by the projection. A
    real query's output must not depend on them: the core's lazy-rescale decision is taken over the real queries
    only. Large finite values there (which raise the maximum of the padded lanes in many key blocks) must give the
    same bits as zeros."""
    from boltz_mlx_amd import kernels as K

    H, C = 4, 32
    rng = np.random.default_rng(1000 + N)
    ldk = K.row_pitch(N)
    qkg = dev(rng.standard_normal((3 * H, N * N, C)), torch.float16)
    vt = dev(rng.standard_normal((H, N, C, ldk)), torch.float16)
    dense = np.zeros((H, N, ldk), dtype=np.float32)
    dense[:, :, :N] = 2 * rng.standard_normal((H, N, N))
    outs = []
    for big in (False, True):
        tb_np = rng.uniform(-6e4, 6e4, K.tri_bias_numel(N, H)).astype(np.float32) if big else np.zeros(
            K.tri_bias_numel(N, H), np.float32)
        tb_np[_tb_index(N, H).ravel()] = dense.ravel()
        mask = np.ones((N, N), np.float32)
        mask[:, -3:] = 0
        outs.append(K.triattn_core(qkg, vt, dev(tb_np, torch.float16), dev(mask), False, 1e9, N, H, C, impl=2))
    torch.cuda.synchronize()
    assert torch.isfinite(outs[0]).all()
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("precision", ["f16"], indirect=True)
def test_pairformer_module_overlap_matches_sequential(precision):
    """The module runs each block's s track on a second stream, overlapped with the next block's pair kernels; the
    result must equal running the layers one after the other on one stream, bit for bit (same kernels, same
    order on each tensor)."""
    import torch

    from boltz_mlx_amd.layers.pairformer import PairformerModule

    N, cs, cz, H, nb = 40, 384, 128, 16, 3
    m = PairformerModule(cs, cz, nb, H)
    p = {}
    for i in range(nb):
        p.update({f"layers.{i}.{k}": v for k, v in rand_params(shapes_layer(cs, cz, H), seed=700 + i, std=0.05).items()})
    m = load(m, p)
    z, tok, pm = pair_inputs(N, cz, seed=71, n_pad=3)
    s = np.random.default_rng(72).standard_normal((1, N, cs))
    s1, z1 = dev(s).float().clone(), dev(z).float().clone()
    s2, z2 = s1.clone(), z1.clone()
    tk, pmk = dev(tok).float().contiguous(), dev(pm).float().contiguous()
    m.run(s1, z1, tk, pmk, 0, nb)
    xn = None
    for i, layer in enumerate(m.layers):
        nxt = m.layers[i + 1].tri_mul_out.norm_in if i + 1 < nb else None
        xn = layer.inplace(s2, z2, tk, pmk, xn_in=xn, next_ln=nxt)
    torch.cuda.synchronize()
    assert torch.equal(z1, z2)
    assert torch.equal(s1, s2)


@pytest.mark.parametrize("precision", ["fp32", "f16"], indirect=True)
@pytest.mark.parametrize("N", [5, 40, 129])
def test_transition_pair_bias(precision, N):
    """The transition with the s track's pair bias in its epilogue (bzpf_transition_pb) against the transition
    followed by the pair-bias kernel on the same z: z and the next LN bit for bit; the bias within the fp16 storage
    rounding (gamma folded into the fp16 weights), and against Linear(LN(z_new)) in float64."""
    import torch

    from boltz_mlx_amd import kernels as K
    from boltz_mlx_amd.layers.norm import LayerNorm
    from boltz_mlx_amd.layers.transition import Transition

    D, H = 128, 16
    rng = np.random.default_rng(900 + N)
    tr = load(Transition(D, 4 * D), rand_params(shapes_transition(D, 4 * D), seed=910 + N, std=0.1))
    ln_next, ln_pb = LayerNorm(D).cuda(), LayerNorm(D).cuda()
    with torch.no_grad():
        for ln in (ln_next, ln_pb):
            ln.weight.copy_(torch.tensor(1 + 0.3 * rng.standard_normal(D)))
            ln.bias.copy_(torch.tensor(0.3 * rng.standard_normal(D)))
    w_pb = dev(0.2 * rng.standard_normal((H, D)), K.storage_dtype())
    z0 = dev(3 * rng.standard_normal((N, N, D)))
    xn = tr.norm.to_storage(z0).reshape(N * N, D)
    z1, z2 = z0.clone(), z0.clone()
    xn1, bias1 = tr.fused(xn, z1, True, next_ln=ln_next, pair_bias=(ln_pb, w_pb))
    xn2 = tr.fused(xn, z2, True, next_ln=ln_next)
    bias2 = K.pair_bias(z2, ln_pb, w_pb)
    torch.cuda.synchronize()
    assert torch.equal(z1, z2)
    assert torch.equal(xn1, xn2)
    assert bias1.shape == (H, N, N) and bias1.dtype == bias2.dtype
    b1, b2 = bias1.float().cpu().numpy(), bias2.float().cpu().numpy()
    scale = np.abs(b2).max()
    tol = 1e-6 if precision == "fp32" else 4e-3
    assert np.abs(b1 - b2).max() <= tol * scale
    zn = z2.double().cpu().numpy()
    mu, var = zn.mean(-1, keepdims=True), zn.var(-1, keepdims=True)
    gam, bet = ln_pb.weight.detach().double().cpu().numpy(), ln_pb.bias.detach().double().cpu().numpy()
    lnz = (zn - mu) / np.sqrt(var + ln_pb.eps) * gam + bet
    ref = np.einsum("ijc,hc->hij", lnz, w_pb.double().cpu().numpy())
    assert np.abs(b1 - ref).max() <= (1e-5 if precision == "fp32" else 6e-3) * np.abs(ref).max()


@pytest.mark.parametrize("precision", ["f16"], indirect=True)
@pytest.mark.parametrize("N", [1, 5, 37, 130])
@pytest.mark.parametrize("trans", [False, True])
@pytest.mark.parametrize("with_pb", [False, True])
def test_attn_out_transition_equals_two_stages(precision, N, trans, with_pb):
    """bzpf_attn_out_transition (the ending node's linear_o + residual run in the transition kernel, the
    intermediate LayerNorm kept in registers) against bzpf_linear_resid_ln followed by bzpf_transition(_pb) on the
    same inputs: z, the next LayerNorm and the pair bias bit for bit."""
    import torch

    from boltz_mlx_amd import kernels as K
    from boltz_mlx_amd.layers.norm import LayerNorm
    from boltz_mlx_amd.layers.transition import Transition

    D, H = 128, 16
    rng = np.random.default_rng(1300 + N + 7 * trans + 3 * with_pb)
    tr = load(Transition(D, 4 * D), rand_params(shapes_transition(D, 4 * D), seed=1310 + N, std=0.1))
    ln_next, ln_pb = LayerNorm(D).cuda(), LayerNorm(D).cuda()
    with torch.no_grad():
        for ln in (ln_next, ln_pb):
            ln.weight.copy_(torch.tensor(1 + 0.3 * rng.standard_normal(D)))
            ln.bias.copy_(torch.tensor(0.3 * rng.standard_normal(D)))
    w_o = dev(0.1 * rng.standard_normal((D, D)), torch.float16)
    o = dev(rng.standard_normal((N * N, D)), torch.float16)
    w_pb = dev(0.2 * rng.standard_normal((H, D)), torch.float16)
    z0 = dev(3 * rng.standard_normal((N, N, D)))
    pb = (ln_pb, w_pb) if with_pb else None
    z1, z2 = z0.clone(), z0.clone()
    r1 = tr.fused_after_attention(o, w_o, trans, z1, next_ln=ln_next, pair_bias=pb)
    xn = K.linear_resid_ln(o, w_o, trans, z2, True, tr.norm, N)
    r2 = tr.fused(xn, z2, True, next_ln=ln_next, pair_bias=pb)
    torch.cuda.synchronize()
    print(f"attn_out_transition N={N} trans={trans} pb={with_pb}: max|dz|="
          f"{float((z1 - z2).abs().max()):.3e}", flush=True)
    assert torch.equal(z1, z2)
    if with_pb:
        assert torch.equal(r1[0], r2[0]) and torch.equal(r1[1], r2[1])
    else:
        assert torch.equal(r1, r2)


@pytest.mark.parametrize("impl", [1, 2])
@pytest.mark.parametrize("N", [7, 70, 200])
def test_triattn_core_strided_mask(impl, N):
    """bzpf_triattn_core reading the natural-orientation mask with strides (mask_si = 1, mask_sk = N), as a C caller
    may pass it for the ending node, equals the call on the transposed copy (the path the module takes), bit for
    bit, for both cores."""
    import torch

    from boltz_mlx_amd import _lib
    from boltz_mlx_amd import kernels as K

    H, C = 4, 32
    rng = np.random.default_rng(1500 + N + impl)
    ldk = K.row_pitch(N)
    qkg = dev(rng.standard_normal((3 * H, N * N, C)), torch.float16)
    vt = dev(rng.standard_normal((H, N, C, ldk)), torch.float16)
    vt[..., N:] = 0
    tb = dev(rng.standard_normal(K.tri_bias_numel(N, H)), torch.float16)
    mask = (rng.random((N, N)) > 0.3).astype(np.float32)
    mask[:, 0] = 1  # no fully masked row of the ending frame
    mg = dev(mask)
    ref = K.triattn_core(qkg, vt, tb, mg, True, 1e9, N, H, C, impl=impl)
    out = torch.empty_like(ref)
    rc = _lib.load().bzpf_triattn_core(qkg.data_ptr(), vt.data_ptr(), tb.data_ptr(), mg.data_ptr(), 1, N, 1e9,
                                       out.data_ptr(), K._dt(qkg), N, ldk, H, C, impl,
                                       torch.cuda.current_stream().cuda_stream)
    assert rc == 0, _lib.load().bzpf_last_error()
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


@pytest.mark.gpu
@pytest.mark.parametrize("N,n_pad", [(200, 33), (300, 50), (700, 116), (700, 330)])
def test_triattn_core_trailing_block_skip_exact(N, n_pad):
    """The MFMA core skips the key blocks after a row's last unmasked key (found by a backward scan in 256-key steps)
    when inf >= 1e6, since those keys' probabilities are exactly zero. Pinned bit for bit against the same call with
    inf = 5e5 (no skip; the masked probabilities are zero there too): trailing padding that covers whole blocks,
    more than 256 padded tokens, rows whose last unmasked key lies far before the end, rows masked at the start,
    interior holes and fully masked rows."""
    import torch

    from boltz_mlx_amd import kernels as K

    H, C = 4, 32
    rng = np.random.default_rng(2600 + N)
    ldk = K.row_pitch(N)
    qkg = dev(rng.standard_normal((3 * H, N * N, C)), torch.float16)
    vt = dev(rng.standard_normal((H, N, C, ldk)), torch.float16)
    vt[..., N:] = 0
    tb = dev(rng.standard_normal(K.tri_bias_numel(N, H)), torch.float16)
    tok = np.ones(N, np.float32)
    tok[N - n_pad:] = 0  # trailing padding: whole 64-key blocks for N = 700, 300
    mask = tok[:, None] * tok[None, :] * (rng.random((N, N)) > 0.2)
    mask[:, 0] = np.where(tok > 0, 1.0, 0.0)  # rows of real tokens keep key 0
    if N > 256:
        mask[3, N // 4:] = 0  # last unmasked key before the scanned range
    mask[5, : N // 2] = 0  # masked at the start (the maximum is set late)
    mask[5, N // 2] = 1
    mg = dev(mask.astype(np.float32))
    for trans in (False, True):
        skip = K.triattn_core(qkg, vt, tb, mg, trans, 1e9, N, H, C, impl=2)
        full = K.triattn_core(qkg, vt, tb, mg, trans, 5e5, N, H, C, impl=2)
        torch.cuda.synchronize()
        assert torch.equal(skip, full), (N, trans)
