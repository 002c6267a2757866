"""torch-facing wrappers of the bzpf C ABI, plus the precision policy of the pair path.

Every wrapper checks devices, dtypes, shapes and contiguity on the host, then calls the C entry point on torch's
current HIP stream with raw device pointers. Outputs and intermediates are allocated here with torch (the C side
never allocates). There is no CPU path: a CPU tensor or a missing library raises.

Precision (mirrors the reference's BOLTZ_MLX_PRECISION, boltz_mlx/kernels.py:1212-1220): "fp32" keeps every
operand in fp32 (the parity build); "f16" stores GEMM operands, LayerNorm outputs and intermediates in fp16 with
fp32 accumulation, fp32 LayerNorm statistics and softmax, and fp32 residual streams. In f16 the triangle
multiplication operands a, b are pre-scaled by 2^-TRIMULT_K and norm_out's eps by 2^-4K, which cancels exactly
(boltz_mlx/kernels.py:1393-1396, layers/norm.py:12-17).
"""

from __future__ import annotations

import contextlib
import os
from typing import NamedTuple

import torch

from boltz_mlx_amd import _lib
from boltz_mlx_amd._lib import F16, F32
from boltz_mlx_amd._lib import call as _call

PRECISION = os.environ.get("BOLTZ_MLX_PRECISION", "fp32")
# fp16 overflow guard (boltz_mlx/kernels.py:1230-1236): after an f16 pass over the trunk, the fp32 residual streams
# are checked for inf / nan (one count per stream) and the pass is recomputed in fp32 when any is found.
# BOLTZ_MLX_GUARDS=0 or BOLTZ_MLX_GUARD_MODE=off turns it off.
GUARDS = os.environ.get("BOLTZ_MLX_GUARDS", "1") == "1" and os.environ.get("BOLTZ_MLX_GUARD_MODE", "residual") != "off"
TRIMULT_K = int(os.environ.get("BOLTZ_MLX_TRIMULT_K", "4"))
# fp16 transition hidden down-scale exponent at 64 channels (boltz_mlx/kernels.py:1327, layers/transition.py:60-92)
TRANS64_K = int(os.environ.get("BOLTZ_MLX_TRANS64_K", "2"))


# Per-entry-point HIP event timing (off unless a dict is installed with start_timing()).
_TIMING: dict | None = None
_TIMING_STREAM = None
SIDE = " (side stream)"


def start_timing() -> None:
    """Record a start/end torch.cuda.Event pair on the current stream around every bzpf launch from now on; launches
    issued on another stream than the current one at this call are keyed `name + SIDE` (their intervals overlap the
    main stream's and include the wait for free compute units)."""
    global _TIMING, _TIMING_STREAM
    _TIMING = {}
    _TIMING_STREAM = torch.cuda.current_stream()


def stop_timing() -> dict:
    """Synchronise and return {entry point: [milliseconds per launch, ...]}; stops recording."""
    global _TIMING
    t, _TIMING = _TIMING, None
    if not t:
        return {}
    torch.cuda.synchronize()
    return {name: [a.elapsed_time(b) for a, b in pairs] for name, pairs in t.items()}


def call(name: str, *args) -> None:
    if _TIMING is None:
        _call(name, *args)
        return
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    _call(name, *args)
    b.record()
    key = name if torch.cuda.current_stream() == _TIMING_STREAM else name + SIDE
    _TIMING.setdefault(key, []).append((a, b))


def set_precision(mode: str) -> None:
    """"fp32" or "f16" (process-wide, like the reference's environment switch)."""
    global PRECISION
    if mode not in ("fp32", "f16"):
        raise ValueError(f"precision must be 'fp32' or 'f16', got {mode!r}")
    PRECISION = mode


def f16() -> bool:
    return PRECISION == "f16"


def storage_dtype() -> torch.dtype:
    return torch.float16 if f16() else torch.float32


def _dt(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return F32
    if t.dtype == torch.float16:
        return F16
    raise TypeError(f"unsupported dtype {t.dtype}")


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _p(t):
    return None if t is None else t.data_ptr()


def _dev(*ts):
    for t in ts:
        if t is not None and (not t.is_cuda or not t.is_contiguous()):
            raise ValueError("bzpf kernels need contiguous ROCm device tensors")


def row_pitch(N: int) -> int:
    return int(_lib.load().bzpf_row_pitch(N))


# ------------------------------------------------------------------------------------------------ weight caches

class KernelWeight(NamedTuple):
    """A weight matrix a kernel reads, as its module declares it (``kernel_weights()``): the row concatenation of the
    module's parameters at the paths ``srcs`` (relative to the module), kept in the storage dtype when ``half`` (fp16
    in f16 mode), else always in fp32. The declarations are the one place that says which parameters f16 mode reads
    only as fp16: the mixed-checkpoint manifest (boltz_mlx_amd/mixed.py) is read off them."""

    name: str
    srcs: tuple
    half: bool = True


def declared_weights(owner: torch.nn.Module) -> dict:
    """{name: KernelWeight} of a module that declares kernel weights (else empty)."""
    fn = getattr(owner, "kernel_weights", None)
    return {} if fn is None else {kw.name: kw for kw in fn()}


def kernel_weight(owner: torch.nn.Module, name: str) -> torch.Tensor:
    """The declared kernel weight `name` of `owner` in its dtype, cached on the module (wcache)."""
    kw = declared_weights(owner).get(name)
    if kw is None:
        raise KeyError(f"{type(owner).__name__} declares no kernel weight {name!r}")
    params = [owner.get_parameter(p) for p in kw.srcs]
    return wcache(owner, name, *params, dtype=storage_dtype() if kw.half else torch.float32)


def _wkey(dtype, params) -> tuple:
    return (dtype,) + tuple((p.data_ptr(), p._version, p.device) for p in params)


def wcache_seed(owner: torch.nn.Module, name: str, params, w: torch.Tensor) -> None:
    """Install `w` (already concatenate(params, 0) in w's dtype, e.g. the buffer the parameters are views of) as the
    cache entry wcache(owner, name, *params, dtype=w.dtype) returns."""
    owner.__dict__.setdefault("_bzpf_cache", {})[name] = (_wkey(w.dtype, params), w)


def wcache(owner: torch.nn.Module, name: str, *params: torch.Tensor, dtype=None) -> torch.Tensor:
    """concatenate(params, 0) in `dtype` (default: the storage dtype), cached on `owner` and rebuilt when a source
    parameter changes (data pointer or in-place version). Mirrors the reference's w16 cache
    (boltz_mlx/kernels.py:1330-1357)."""
    dtype = dtype or storage_dtype()
    key = _wkey(dtype, params)
    hit = owner.__dict__.get("_bzpf_cache", {}).get(name)
    if hit is not None and hit[0] == key:
        return hit[1]
    with torch.no_grad():
        w = params[0] if len(params) == 1 else torch.cat(list(params), 0)
        w = w.detach().to(dtype).contiguous()
    owner.__dict__.setdefault("_bzpf_cache", {})[name] = (key, w)
    return w


def f32c(t: torch.Tensor) -> torch.Tensor:
    return t.detach().float().contiguous()


# ------------------------------------------------------------------------------------------------ wrappers

def layer_norm(x: torch.Tensor, weight, bias, eps: float = 1e-5, out_dtype=torch.float32) -> torch.Tensor:
    """LayerNorm over the last axis (boltz_mlx/kernels.py:482-507)."""
    x = x.contiguous()
    _dev(x)
    D = x.shape[-1]
    y = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    w = None if weight is None else f32c(weight)
    b = None if bias is None else f32c(bias)
    call("bzpf_layernorm", _p(x), _dt(x), _p(w), _p(b), float(eps), _p(y), _dt(y), x.numel() // D, D, _stream())
    return y


def count_nonfinite(*tensors: torch.Tensor) -> torch.Tensor:
    """Device int32 [1]: the number of inf / nan elements over the given fp32 / fp16 tensors, without a host sync
    (the residual-mode overflow guard, boltz_mlx/kernels.py:1262-1282)."""
    _dev(*tensors)
    count = torch.zeros((1,), dtype=torch.int32, device=tensors[0].device)
    for t in tensors:
        call("bzpf_count_nonfinite", _p(t), _dt(t), t.numel(), _p(count), _stream())
    return count


def add_ln(z: torch.Tensor, y: torch.Tensor, ln=None, scale: float = 1.0, trans_y: bool = False,
           trans_out: bool = False, out_dtype=torch.float16):
    """In place z += y * scale over [N, N, D] (y optionally read transposed); returns LN(z) (optionally transposed)
    when `ln` (a LayerNorm module) is given (boltz_mlx/kernels.py:1448-1480)."""
    _dev(z, y)
    if z.dtype != torch.float32 or z.shape != y.shape:
        raise ValueError("add_ln: z must be fp32 and y the same shape")
    N, D = z.shape[-2], z.shape[-1]
    if z.dim() != 3 or z.shape[0] != N:
        raise ValueError("add_ln: z must be [N, N, D]")
    out = None
    w = b = None
    eps = 1e-5
    if ln is not None:
        out = torch.empty(z.shape, dtype=out_dtype, device=z.device)
        w, b, eps = f32c(ln.weight), f32c(ln.bias), ln.eps
    call("bzpf_add_ln", _p(z), _p(y), _dt(y), float(scale), int(trans_y), _p(w), _p(b), float(eps), _p(out),
         _dt(out) if out is not None else F32, int(trans_out), N, D, _stream())
    return out


def trimul_proj(xn, w_pg, mask, scale: float, incoming: bool, N: int) -> torch.Tensor:
    _dev(xn, w_pg, mask)
    if mask.dtype != torch.float32 or mask.numel() != N * N:
        raise ValueError("trimul_proj: mask must be fp32 [N, N]")
    D = xn.shape[-1]
    if w_pg.shape != (4 * D, D) or w_pg.dtype != xn.dtype or xn.numel() != N * N * D:
        raise ValueError("trimul_proj: shape/dtype mismatch")
    ld = row_pitch(N)
    ab = torch.empty((2 * D, N, ld), dtype=xn.dtype, device=xn.device)
    call("bzpf_trimul_proj", _p(xn), _p(w_pg), _p(mask), float(scale), int(incoming), _p(ab), _dt(xn), N, ld, D,
         _stream())
    return ab


def trimul_pack(P: torch.Tensor, mask: torch.Tensor, scale: float, incoming: bool, N: int) -> torch.Tensor:
    """ab [2D, N, ld] from P = xn [p_in; g_in]^T ([N*N, 4D]) at any D (the fused trimul_proj is built for 128)."""
    _dev(P, mask)
    D = P.shape[-1] // 4
    if P.shape != (N * N, 4 * D) or mask.dtype != torch.float32 or mask.numel() != N * N:
        raise ValueError("trimul_pack: need P [N*N, 4D] and an fp32 mask [N, N]")
    ld = row_pitch(N)
    ab = torch.empty((2 * D, N, ld), dtype=P.dtype, device=P.device)
    call("bzpf_trimul_pack", _p(P), _p(mask), float(scale), int(incoming), _p(ab), _dt(P), N, ld, D, _stream())
    return ab


def channels_to_rows(o: torch.Tensor, N: int, out_dtype=None) -> torch.Tensor:
    """[N*N, D] rows from the contraction output o [D, N, ld]."""
    _dev(o)
    D = o.shape[0]
    ld = row_pitch(N)
    if o.shape != (D, N, ld):
        raise ValueError("channels_to_rows: o must be [D, N, ld]")
    out = torch.empty((N * N, D), dtype=out_dtype or o.dtype, device=o.device)
    call("bzpf_channels_to_rows", _p(o), _dt(o), _p(out), _dt(out), N, ld, D, _stream())
    return out


def triattn_pack(P: torch.Tensor, trans: bool, N: int, H: int, C: int):
    """(qkg, vt, tb) as triattn_proj returns them, from P = xn [q; k; v; g; bias]^T ([N*N, 4HC + H]) at any c_in."""
    _dev(P)
    if P.shape != (N * N, 4 * H * C + H):
        raise ValueError("triattn_pack: P must be [N*N, 4HC + H]")
    ldk = row_pitch(N)
    qkg = torch.empty((3 * H, N * N, C), dtype=P.dtype, device=P.device)
    vt = torch.empty((H, N, C, ldk), dtype=P.dtype, device=P.device)
    tb = torch.zeros((tri_bias_numel(N, H),), dtype=P.dtype, device=P.device)
    call("bzpf_triattn_pack", _p(P), int(trans), LOG2E / C ** 0.5, LOG2E, _p(qkg), _p(vt), _p(tb), _dt(P), N, ldk, H,
         C, _stream())
    return qkg, vt, tb


def trimul_contract(ab: torch.Tensor, N: int, k_len: int = 0) -> torch.Tensor:
    """o [D, N, ld] = per-channel a b^T; k_len > 0: columns k >= k_len of ab are zero and the sum stops there (the
    trailing padded tokens; key_extent gives it for a pair mask)."""
    _dev(ab)
    D = ab.shape[0] // 2
    ld = row_pitch(N)
    if ab.shape != (2 * D, N, ld):
        raise ValueError("trimul_contract: ab must be [2D, N, ld]")
    o = torch.empty((D, N, ld), dtype=ab.dtype, device=ab.device)
    call("bzpf_trimul_contract", _p(ab), _p(o), _dt(ab), N, ld, D, int(k_len), _stream())
    return o


# Per-mask values derived once inside pair_mask_scope(): {key: {"t": transposed copy, ("ext", incoming): k_len}}
_MASK_SCOPE: dict | None = None


@contextlib.contextmanager
def pair_mask_scope():
    """Inside the block, the values derived from a pair mask (the ending-node core's transposed copy, the
    contraction's key extent) are computed once per mask (keyed by its storage, shape, strides and version) and
    reused by every later call with the same mask: a module run derives them once instead of once per layer.
    Outside a scope each call transposes for itself and the contraction runs over every key."""
    global _MASK_SCOPE
    prev, _MASK_SCOPE = _MASK_SCOPE, {}
    try:
        yield
    finally:
        _MASK_SCOPE = prev


def _mask_entry(mask: torch.Tensor):
    if _MASK_SCOPE is None:
        return None
    key = (mask.data_ptr(), tuple(mask.shape), tuple(mask.stride()), mask._version)
    return _MASK_SCOPE.setdefault(key, {})


def mask_transposed(mask: torch.Tensor, N: int) -> torch.Tensor:
    """The pair mask [N, N] transposed, contiguous (cached inside pair_mask_scope)."""
    ent = _mask_entry(mask)
    if ent is None:
        return mask.reshape(N, N).t().contiguous()
    if "t" not in ent:
        ent["t"] = mask.reshape(N, N).t().contiguous()
    return ent["t"]


def key_extent(mask: torch.Tensor, N: int, incoming: bool) -> int:
    """1 + the last token k whose pair-mask column (outgoing; row for incoming) is not all zero: bzpf_trimul_proj
    writes zeros in ab for every k past it. Computed (one host sync) only inside pair_mask_scope, once per mask;
    0 (every key) outside, and during stream capture (no sync there)."""
    ent = _mask_entry(mask)
    if ent is None or (mask.is_cuda and torch.cuda.is_current_stream_capturing()):
        return 0
    if ("ext", incoming) not in ent:
        m = mask.reshape(N, N) != 0
        live = m.any(dim=1 if incoming else 0)
        idx = torch.nonzero(live)
        ent[("ext", incoming)] = int(idx[-1, 0].item()) + 1 if idx.numel() else N
    return ent[("ext", incoming)]


def trimul_tail(o, norm_out, eps_out: float, w_po, xn, w_go, z, accumulate: bool, next_ln=None, N: int = 0):
    """z (+)= p_out(LN_out(o)) * sigmoid(g_out(xn)); returns next_ln(z) in the storage dtype when next_ln is given."""
    _dev(o, w_po, xn, w_go, z)
    D = o.shape[0]
    ld = row_pitch(N)
    if z.dtype != torch.float32 or z.numel() != N * N * D or o.shape != (D, N, ld):
        raise ValueError("trimul_tail: shape/dtype mismatch")
    nxt = nw = nb = None
    neps = 1e-5
    if next_ln is not None:
        nxt = torch.empty((N * N, D), dtype=xn.dtype, device=xn.device)
        nw, nb, neps = f32c(next_ln.weight), f32c(next_ln.bias), next_ln.eps
    call("bzpf_trimul_tail", _p(o), _p(f32c(norm_out.weight)), _p(f32c(norm_out.bias)), float(eps_out), _p(w_po),
         _p(xn), _p(w_go), _p(z), int(accumulate), _p(nw), _p(nb), float(neps), _p(nxt), _dt(xn), N, ld, D,
         _stream())
    return nxt


LOG2E = 1.4426950408889634


def triattn_proj(xn, w, trans: bool, N: int, H: int, C: int):
    """-> (qkg [3H, N*N, C], vt [H, N, C, ldk], tb flat in the fragment-ordered layout of tri_bias_offsets) in
    xn's dtype, q scaled by log2(e)/sqrt(C) and the bias by log2(e) (the base-2 logits the core expects)."""
    _dev(xn, w)
    D = xn.shape[-1]
    if w.shape != (4 * H * C + H, D) or w.dtype != xn.dtype or xn.numel() != N * N * D:
        raise ValueError("triattn_proj: shape/dtype mismatch")
    ldk = row_pitch(N)
    qkg = torch.empty((3 * H, N * N, C), dtype=xn.dtype, device=xn.device)
    vt = torch.empty((H, N, C, ldk), dtype=xn.dtype, device=xn.device)
    tb = torch.empty((tri_bias_numel(N, H),), dtype=xn.dtype, device=xn.device)
    call("bzpf_triattn_proj", _p(xn), _p(w), int(trans), LOG2E / C ** 0.5, LOG2E, _p(qkg), _p(vt), _p(tb), _dt(xn),
         N, ldk, D, H, C, _stream())
    return qkg, vt, tb


def tri_bias_numel(N: int, H: int) -> int:
    """Elements of the fragment-ordered triangle-bias buffer: H * (N rounded up to 32) * row_pitch(N)."""
    return H * ((N + 31) // 32) * 32 * row_pitch(N)


def tri_bias_offsets(N: int, H: int):
    """Index of element (h, j, k) of a dense [H, N, N] bias in the fragment-ordered layout the attention core reads
    (32-query tile, 64-key block, lane 32*hl + q owning keys 32*kt + 8*p + 4*hl + e, stored so that each of a
    lane's four 16-byte loads is contiguous across the wave), as an int64 array."""
    import numpy as np

    ldk = row_pitch(N)
    njt, nkb = (N + 31) // 32, ldk // 64
    h = np.arange(H)[:, None, None]
    j = np.arange(N)[None, :, None]
    k = np.arange(N)[None, None, :]
    jt, q, kb, kk = j >> 5, j & 31, k >> 6, k & 63
    kt, p, hl, e = kk >> 5, (kk >> 3) & 3, (kk >> 2) & 1, kk & 3
    x = kt * 16 + p * 4 + e
    return ((h * njt + jt) * nkb + kb) * 2048 + (x >> 3) * 512 + (hl * 32 + q) * 8 + (x & 7)


TRIATT_IMPL = {"auto": 0, "scalar": 1, "mma": 2}[os.environ.get("BOLTZ_MLX_TRIATT_IMPL", "auto")]


def triattn_core(qkg, vt, tb, mask, trans: bool, inf: float, N: int, H: int, C: int, impl: int | None = None):
    """mask: the pair mask [N, N] fp32 in the natural orientation; the ending node (trans) reads it transposed (from
    a transposed copy).
    impl: 0 auto, 1 VALU kernel, 2 MFMA kernel (default from BOLTZ_MLX_TRIATT_IMPL = auto | scalar | mma)."""
    _dev(qkg, vt, tb, mask)
    if mask.dtype != torch.float32 or mask.numel() != N * N:
        raise ValueError("triattn_core: mask must be fp32 [N, N]")
    ldk = row_pitch(N)
    if qkg.shape != (3 * H, N * N, C) or vt.shape != (H, N, C, ldk) or tb.numel() != tri_bias_numel(N, H):
        raise ValueError("triattn_core: buffers must come from triattn_proj")
    out = torch.empty((N * N, H * C), dtype=qkg.dtype, device=qkg.device)
    if trans:
        # the ending node's row i reads column i of the mask: a transposed copy makes the kernel's per-block mask
        # loads contiguous (strided, every lane touched its own cache line: 13% of the core at N = 1000)
        mask = mask_transposed(mask, N)
    call("bzpf_triattn_core", _p(qkg), _p(vt), _p(tb), _p(mask), N, 1, float(inf), _p(out), _dt(qkg), N, ldk, H, C,
         TRIATT_IMPL if impl is None else int(impl), _stream())
    return out


def linear_resid_ln(x, w, trans: bool, z, accumulate: bool, next_ln=None, N: int = 0):
    _dev(x, w, z)
    D = z.shape[-1]
    if z.dtype != torch.float32 or x.numel() != N * N * D or w.shape != (D, D):
        raise ValueError("linear_resid_ln: shape/dtype mismatch")
    nxt = nw = nb = None
    neps = 1e-5
    if next_ln is not None:
        nxt = torch.empty((N * N, D), dtype=x.dtype, device=x.device)
        nw, nb, neps = f32c(next_ln.weight), f32c(next_ln.bias), next_ln.eps
    call("bzpf_linear_resid_ln", _p(x), _p(w), int(trans), _p(z), int(accumulate), _p(nw), _p(nb), float(neps),
         _p(nxt), _dt(x), N, D, _stream())
    return nxt


def transition(xn, w12, w3, z, accumulate: bool, next_ln=None, pair_bias=None):
    """z (+)= fc3(silu(xn fc1^T) * (xn fc2^T)); returns next_ln(z_new) (or None). pair_bias = (ln, w) also computes
    Linear(ln(z_new)) as [H, rows] in w's dtype (the s track's pair bias, z being [N, N, D]) and returns
    (next_ln(z_new), bias)."""
    _dev(xn, w12, w3, z)
    D = z.shape[-1]
    rows = z.numel() // D
    hidden = w3.shape[1]
    if xn.numel() != rows * D or w12.shape != (2 * hidden, D) or w3.shape != (D, hidden):
        raise ValueError("transition: shape mismatch")
    nxt = nw = nb = None
    neps = 1e-5
    if next_ln is not None:
        nxt = torch.empty((rows, D), dtype=xn.dtype, device=xn.device)
        nw, nb, neps = f32c(next_ln.weight), f32c(next_ln.bias), next_ln.eps
    if pair_bias is None:
        call("bzpf_transition", _p(xn), _p(w12), _p(w3), _p(z), int(accumulate), _p(nw), _p(nb), float(neps),
             _p(nxt), _dt(xn), rows, D, hidden, _stream())
        return nxt
    ln, w = pair_bias
    _dev(w)
    H = w.shape[0]
    if w.shape != (H, D) or w.dtype != xn.dtype:
        raise ValueError("transition: pair-bias weight must be [H, D] in the storage dtype")
    N = z.shape[0]
    bias = torch.empty((H, N, rows // N), dtype=w.dtype, device=z.device)
    call("bzpf_transition_pb", _p(xn), _p(w12), _p(w3), _p(z), int(accumulate), _p(nw), _p(nb), float(neps),
         _p(nxt), _p(w), _p(f32c(ln.weight)), _p(f32c(ln.bias)), float(ln.eps), _p(bias), H, _dt(xn), rows, D, hidden,
         _stream())
    return nxt, bias


def attn_out_transition(o, w_o, trans: bool, z, ln, w12, w3, next_ln=None, pair_bias=None):
    """fp16: z += o' w_o^T (o' = o at the transposed position when trans: the ending-node attention's output stage),
    then z += transition(ln(z)) in the same kernel (the intermediate LayerNorm stays in registers); returns
    next_ln(z_new) (or None), with pair_bias = (ln_pb, w) also the s track's pair bias: (next_ln(z_new), bias). Equals
    linear_resid_ln(o, w_o, trans, z, True, ln) followed by transition(.., z, True, next_ln, pair_bias) bit for bit."""
    _dev(o, w_o, w12, w3, z)
    N, D = z.shape[0], z.shape[-1]
    rows = z.numel() // D
    hidden = w3.shape[1]
    if z.dtype != torch.float32 or o.dtype != torch.float16 or o.numel() != rows * D or rows != N * N or \
            w_o.shape != (D, D) or w12.shape != (2 * hidden, D) or w3.shape != (D, hidden):
        raise ValueError("attn_out_transition: shape/dtype mismatch")
    nxt = nw = nb = None
    neps = 1e-5
    if next_ln is not None:
        nxt = torch.empty((rows, D), dtype=o.dtype, device=o.device)
        nw, nb, neps = f32c(next_ln.weight), f32c(next_ln.bias), next_ln.eps
    pw = plw = plb = bias = None
    peps, H = 1e-5, 0
    if pair_bias is not None:
        ln_pb, pw = pair_bias
        _dev(pw)
        H = pw.shape[0]
        if pw.shape != (H, D) or pw.dtype != o.dtype:
            raise ValueError("attn_out_transition: pair-bias weight must be [H, D] in fp16")
        plw, plb, peps = f32c(ln_pb.weight), f32c(ln_pb.bias), ln_pb.eps
        bias = torch.empty((H, N, N), dtype=pw.dtype, device=z.device)
    call("bzpf_attn_out_transition", _p(o), _p(w_o), int(trans), _p(f32c(ln.weight)), _p(f32c(ln.bias)),
         float(ln.eps), _p(w12), _p(w3), _p(z), _p(nw), _p(nb), float(neps), _p(nxt), _p(pw), _p(plw), _p(plb),
         float(peps), _p(bias), H, _dt(o), N, D, hidden, _stream())
    return nxt if pair_bias is None else (nxt, bias)


def linear(x, w, bias=None, out=None, out_dtype=None, accumulate: bool = False) -> torch.Tensor:
    """y = x w^T + bias over the rows of x (w [M, K] in x's dtype); accumulate adds into the fp32 `out`."""
    _dev(x, w)
    K = x.shape[-1]
    M = w.shape[0]
    rows = x.numel() // K
    if w.shape[1] != K or w.dtype != x.dtype:
        raise ValueError("linear: shape/dtype mismatch")
    if out is None:
        out = torch.empty(x.shape[:-1] + (M,), dtype=out_dtype or x.dtype, device=x.device)
    _dev(out)
    b = None if bias is None else f32c(bias)
    call("bzpf_linear", _p(x), _p(w), _p(b), _p(out), _dt(x), _dt(out), rows, K, M, int(accumulate), _stream())
    return out


def linear_residual(x, w, res: torch.Tensor, out: torch.Tensor, bias=None) -> torch.Tensor:
    """out (fp32) = res + x w^T + bias over the rows of x, for an fp32 res [rows, M] with unit column stride (a
    residual update written out of place: the same sums as copying res into out and accumulating)."""
    _dev(x, w, out)
    K = x.shape[-1]
    M = w.shape[0]
    rows = x.numel() // K
    if w.shape[1] != K or w.dtype != x.dtype or out.dtype != torch.float32 or out.numel() != rows * M \
            or not res.is_cuda or res.dtype != torch.float32 or res.dim() != 2 or res.shape != (rows, M) \
            or res.stride(1) != 1:
        raise ValueError("linear_residual: shape/dtype mismatch")
    b = None if bias is None else f32c(bias)
    call("bzpf_linear_residual", _p(x), _p(w), _p(b), _p(res), res.stride(0), _p(out), _dt(x), rows, K, M, _stream())
    return out


def linear_gated(x, w, gate: torch.Tensor, out: torch.Tensor, bias=None) -> torch.Tensor:
    """out (fp32) += sigmoid(gate) * (x w^T + bias) over the rows of x; gate is an fp32 [rows_g, M] view whose
    rows may have a pitch (a slice of the precomputed conditioning), row r using gate row r % rows_g
    (transformersv2.py:96-99, 63-66)."""
    _dev(x, w, out)
    K = x.shape[-1]
    M = w.shape[0]
    rows = x.numel() // K
    if w.shape[1] != K or w.dtype != x.dtype or out.dtype != torch.float32 or out.numel() != rows * M:
        raise ValueError("linear_gated: shape/dtype mismatch")
    if not gate.is_cuda or gate.dtype != torch.float32 or gate.dim() != 2 or gate.shape[1] != M or gate.stride(1) != 1:
        raise ValueError("linear_gated: gate must be an fp32 [rows, M] view with unit column stride")
    b = None if bias is None else f32c(bias)
    call("bzpf_linear_gated", _p(x), _p(w), _p(b), _p(gate), gate.stride(0), gate.shape[0], _p(out), _dt(x), rows,
         K, M, _stream())
    return out


def linear_swiglu3(x: torch.Tensor, w_grouped: torch.Tensor) -> torch.Tensor:
    """silu(x Wg^T) * (x Wx^T) * (x Wab^T) in one fp16 GEMM for w_grouped from group_swiglu3_rows (fp16 only)."""
    _dev(x, w_grouped)
    Kd = x.shape[-1]
    H = w_grouped.shape[0] // 3
    rows = x.numel() // Kd
    if x.dtype != torch.float16 or w_grouped.dtype != torch.float16 or w_grouped.shape != (3 * H, Kd):
        raise ValueError("linear_swiglu3: need fp16 x [rows, K] and grouped fp16 w [3H, K]")
    u = torch.empty(x.shape[:-1] + (H,), dtype=torch.float16, device=x.device)
    call("bzpf_linear_swiglu3", _p(x), _p(w_grouped), _p(u), rows, Kd, H, _stream())
    return u


def linear_swiglu(x: torch.Tensor, w_grouped: torch.Tensor) -> torch.Tensor:
    """silu(x W1^T) * (x W2^T) in one fp16 GEMM for w_grouped = group_swiglu_rows(W1, W2) (fp16 only)."""
    _dev(x, w_grouped)
    Kd = x.shape[-1]
    H = w_grouped.shape[0] // 2
    rows = x.numel() // Kd
    if x.dtype != torch.float16 or w_grouped.dtype != torch.float16 or w_grouped.shape != (2 * H, Kd):
        raise ValueError("linear_swiglu: need fp16 x [rows, K] and grouped fp16 w [2H, K]")
    u = torch.empty(x.shape[:-1] + (H,), dtype=torch.float16, device=x.device)
    call("bzpf_linear_swiglu", _p(x), _p(w_grouped), _p(u), rows, Kd, H, _stream())
    return u


def group_swiglu_rows(*ws: torch.Tensor) -> torch.Tensor:
    """[W_0; W_1 (; W_2)] regrouped as blocks [W_0[32q:32q+32]; W_1[..] (; W_2[..])] per 32 output columns q (the
    fused kernels' layout)."""
    H, Kd = ws[0].shape
    return torch.stack([w.view(H // 32, 32, Kd) for w in ws], 1).reshape(len(ws) * H, Kd).contiguous()


def group_swiglu3_rows(wg: torch.Tensor, wx: torch.Tensor, wab: torch.Tensor) -> torch.Tensor:
    return group_swiglu_rows(wg, wx, wab)


def adaln(a: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor, out_dtype, eps: float = 1e-5) -> torch.Tensor:
    """sigmoid(scale) * LN(a) + shift (LN without affine) for fp32 a [rows, D]; scale and shift are fp32 [rows_c, D]
    views of one pitch (slices of the precomputed conditioning), row r using row r % rows_c
    (transformersv2.py:27-41, 218, 252)."""
    _dev(a)
    D = a.shape[-1]
    rows = a.numel() // D
    if a.dtype != torch.float32 or scale.shape != shift.shape or scale.dim() != 2 or scale.shape[1] != D:
        raise ValueError("adaln: shape/dtype mismatch")
    if (not scale.is_cuda or not shift.is_cuda or scale.stride() != shift.stride() or scale.stride(1) != 1
            or scale.dtype != torch.float32 or shift.dtype != torch.float32):
        raise ValueError("adaln: scale and shift must be fp32 views with one row pitch and unit column stride")
    out = torch.empty(a.shape, dtype=out_dtype, device=a.device)
    call("bzpf_adaln", _p(a), _p(scale), _p(shift), scale.stride(0), scale.shape[0], float(eps), _p(out), _dt(out),
         rows, D, _stream())
    return out


def swiglu3(h: torch.Tensor) -> torch.Tensor:
    """silu(h[:, :H]) * h[:, H:2H] * h[:, 2H:] for h [rows, 3H] (the conditioned transition's gated product)."""
    _dev(h)
    H = h.shape[-1] // 3
    rows = h.numel() // (3 * H)
    a = torch.empty(h.shape[:-1] + (H,), dtype=h.dtype, device=h.device)
    call("bzpf_swiglu3", _p(h), _p(a), _dt(h), rows, H, _stream())
    return a


def swiglu(h: torch.Tensor) -> torch.Tensor:
    _dev(h)
    H = h.shape[-1] // 2
    rows = h.numel() // (2 * H)
    a = torch.empty(h.shape[:-1] + (H,), dtype=h.dtype, device=h.device)
    call("bzpf_swiglu", _p(h), _p(a), _dt(h), rows, H, _stream())
    return a


def seq_attention(q, k, v, g, bias, mask, inf: float, H: int) -> torch.Tensor:
    """q/k/v/g [N, H*hd], bias [H, N, N] (fp32 or fp16, independently of q's dtype), mask [N] fp32 -> [N, H*hd]."""
    _dev(q, k, v, g, bias, mask)
    N, HD = q.shape
    hd = HD // H
    if bias.shape != (H, N, N) or mask.numel() != N or mask.dtype != torch.float32:
        raise ValueError("seq_attention: bias must be [H, N, N] and mask fp32 [N]")
    out = torch.empty_like(q)
    call("bzpf_seq_attention", _p(q), _p(k), _p(v), _p(g), HD, _p(bias), _p(mask), float(inf), _p(out), HD,
         _dt(q), _dt(bias), N, H, hd, _stream())
    return out


def seq_attention_packed(qkvg, bias, mask, inf: float, H: int, out=None, multiplicity: int = 1) -> torch.Tensor:
    """seq_attention over [N, 4*H*hd] or [S, N, 4*H*hd] buffers holding q | k | v | g per row (the fused
    projection's output), one launch for all S samples; bias [H, N, N] or [S / multiplicity, H, N, N] (consecutive
    groups of `multiplicity` samples share one; fp32 or fp16, independently of qkvg's dtype), mask [N] or [S, N] fp32.
    Writes `out` [(S,) N, H*hd] when given."""
    _dev(qkvg, bias, mask)
    batched = qkvg.dim() == 3
    q3 = qkvg if batched else qkvg[None]
    S, N, HD4 = q3.shape
    HD = HD4 // 4
    hd = HD // H
    b4 = bias if bias.dim() == 4 else bias[None]
    m2 = mask.reshape(S, N) if mask.numel() == S * N else mask
    if (b4.shape[1:] != (H, N, N) or b4.shape[0] * multiplicity != S or m2.shape != (S, N)
            or mask.dtype != torch.float32 or not (q3.is_contiguous() and b4.is_contiguous() and m2.is_contiguous())):
        raise ValueError("seq_attention: need contiguous qkvg [S, N, 4HD], bias [S / multiplicity, H, N, N] and "
                         "mask fp32 [S, N]")
    shape = (S, N, HD) if batched else (N, HD)
    if out is None:
        out = torch.empty(shape, dtype=qkvg.dtype, device=qkvg.device)
    elif out.shape != shape or out.dtype != qkvg.dtype or not out.is_contiguous():
        raise ValueError("seq_attention: out must be a contiguous [(S,) N, H*hd] tensor of qkvg's dtype")
    base, es = q3.data_ptr(), q3.element_size()
    call("bzpf_seq_attention_batched", base, base + HD * es, base + 2 * HD * es, base + 3 * HD * es, HD4, N * HD4,
         _p(b4), H * N * N, int(multiplicity), _p(m2), N, float(inf), _p(out), HD, N * HD, _dt(qkvg), _dt(b4), S, N,
         H, hd, _stream())
    return out


def opm_counts(mask: torch.Tensor) -> torch.Tensor:
    """num = mask^T mask ([N, N] fp32: the pair counts sum_s mask_si mask_sj, exact integers) for mask fp32 [S, N],
    as one fp32 GEMM over the transposed mask (MSA rows padded with zeros to a multiple of 32)."""
    S, N = mask.shape
    mt = torch.zeros((N, (S + 31) // 32 * 32), dtype=torch.float32, device=mask.device)
    mt[:, :S] = mask.t()
    return linear(mt, mt)


def opm_split(ab: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
    """The masked outer-product-mean operands x = mask[s, n] * ab[s, n, ch] as three exact bf16 parts, in the chunk
    layout bzpf_opm_outer loads ([ceil(S / 16), N, 3, 2, 32, 16] bf16: stage, token, part, a | b, channel, MSA row
    within the stage; zeros past S) for ab fp32 [S, N, 64], mask fp32 [S, N] (outer_product_mean.py:37-45)."""
    _dev(ab, mask)
    S, N, C2 = ab.shape
    if ab.dtype != torch.float32 or C2 < 64 or not ab.is_contiguous() or mask.shape != (S, N) \
            or mask.dtype != torch.float32 or not mask.is_contiguous():
        raise ValueError("opm_split: need contiguous fp32 ab [S, N, 64] and mask [S, N]")
    planes = torch.empty(((S + 15) // 16, N, 3, 2, 32, 16), dtype=torch.bfloat16, device=ab.device)
    call("bzpf_opm_split", _p(ab), C2, _p(mask), _p(planes), S, N, _stream())
    return planes


def opm_ln_split(m: torch.Tensor, ln, w_ab: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
    """The opm_split planes straight from the MSA: mask[s, n] * (LN(m[s, n]) w_ab^T) for m fp32 [S, N, 64], w_ab fp32
    [64, 64] ([proj_a; proj_b]), mask fp32 [S, N], in one kernel (outer_product_mean.py:37-45)."""
    _dev(m, w_ab, mask)
    S, N, C = m.shape
    if m.dtype != torch.float32 or C != 64 or not m.is_contiguous() or w_ab.shape != (64, 64) \
            or w_ab.dtype != torch.float32 or not w_ab.is_contiguous() or mask.shape != (S, N) \
            or mask.dtype != torch.float32 or not mask.is_contiguous():
        raise ValueError("opm_ln_split: need contiguous fp32 m [S, N, 64], w_ab [64, 64] and mask [S, N]")
    lw, lb = f32c(ln.weight), f32c(ln.bias)
    planes = torch.empty(((S + 15) // 16, N, 3, 2, 32, 16), dtype=torch.bfloat16, device=m.device)
    call("bzpf_opm_ln_split", _p(m), _p(lw), _p(lb), float(ln.eps), _p(w_ab), _p(mask), _p(planes), S, N, _stream())
    return planes


def opm_outer_planes(planes: torch.Tensor, num: torch.Tensor, S: int, N: int, i_base: int = 0,
                     n_i: int | None = None, out_dtype=torch.float16) -> torch.Tensor:
    """The outer sum over opm_split / opm_ln_split planes for S MSA rows and N tokens: [n_i * N, 1024], row
    (i - i_base) * N + j, column c * 32 + d, divided by max(num[i, j], 1) (outer_product_mean.py:37-45)."""
    _dev(planes, num)
    n_i = N - i_base if n_i is None else n_i
    if planes.shape != ((S + 15) // 16, N, 3, 2, 32, 16) or planes.dtype != torch.bfloat16 \
            or not planes.is_contiguous():
        raise ValueError("opm_outer: planes must be the contiguous output of opm_split for S, N")
    if num.shape != (N, N) or num.dtype != torch.float32 or not num.is_contiguous():
        raise ValueError("opm_outer: num must be the contiguous fp32 [N, N] pair counts")
    out = torch.empty((n_i * N, 1024), dtype=out_dtype, device=planes.device)
    call("bzpf_opm_outer", _p(planes), _p(num), _p(out), _dt(out), S, N, int(i_base), int(n_i), _stream())
    return out


def opm_outer(ab: torch.Tensor, mask: torch.Tensor, i_base: int = 0, n_i: int | None = None,
              out_dtype=torch.float16, num: torch.Tensor | None = None) -> torch.Tensor:
    """OuterProductMean's outer sum for one MSA: ab fp32 [S, N, 64] (LN(m) [W_a; W_b]^T, unmasked), mask fp32
    [S, N] -> [n_i * N, 1024] with row (i - i_base) * N + j and column c * 32 + d holding
    sum_s mask_si mask_sj a[s, i, c] b[s, j, d] / max(sum_s mask_si mask_sj, 1) (outer_product_mean.py:37-45):
    opm_split, then opm_outer_planes."""
    S, N, _ = ab.shape
    num = opm_counts(mask) if num is None else num
    return opm_outer_planes(opm_split(ab, mask), num, S, N, i_base, n_i, out_dtype)


def transition64_f16(x: torch.Tensor, ln, w12: torch.Tensor, w3: torch.Tensor) -> None:
    """x (fp32 [rows, 64], in place) += fc3(silu(xn fc1^T) * (xn fc2^T)), xn = fp16(LN(x)), for fp16 w12 [2H, 64]
    ([fc1; fc2]) and w3 [64, H] in one kernel (transition.py:27-92 at 64 channels)."""
    _dev(x, w12, w3)
    rows, Dx = x.shape
    H = w3.shape[1]
    if x.dtype != torch.float32 or Dx != 64 or not x.is_contiguous() or w12.shape != (2 * H, 64) \
            or w3.shape != (64, H) or w12.dtype != torch.float16 or w3.dtype != torch.float16 \
            or not w12.is_contiguous() or not w3.is_contiguous():
        raise ValueError("transition64_f16: need contiguous fp32 x [rows, 64], fp16 w12 [2H, 64] and w3 [64, H]")
    call("bzpf_transition64_f16", _p(x), _p(f32c(ln.weight)), _p(f32c(ln.bias)), float(ln.eps), _p(w12), _p(w3),
         rows, H, _stream())


def ln_linear_f32(x: torch.Tensor, ln, w: torch.Tensor) -> torch.Tensor:
    """LN(x; ln.weight, ln.bias, ln.eps) w^T for fp32 x [rows, 64] and fp32 w [M, 64] (M a multiple of 256) in one
    kernel (the LayerNorm of bzpf_layernorm, the product at fp32 accuracy) -> [rows, M] fp32
    (pair_averaging.py:36-41)."""
    _dev(x, w)
    rows, Kd = x.shape
    M = w.shape[0]
    if x.dtype != torch.float32 or w.dtype != torch.float32 or Kd != 64 or w.shape[1] != 64 or M % 256 \
            or not x.is_contiguous() or not w.is_contiguous():
        raise ValueError("ln_linear_f32: need contiguous fp32 x [rows, 64] and w [M, 64] with M % 256 == 0")
    lw, lb = f32c(ln.weight), f32c(ln.bias)
    y = torch.empty((rows, M), dtype=torch.float32, device=x.device)
    call("bzpf_ln_linear_f32", _p(x), _p(lw), _p(lb), float(ln.eps), _p(w), _p(y), rows, 64, M, _stream())
    return y


def pwa_softmax(logits: torch.Tensor, pair_mask: torch.Tensor, inf: float) -> torch.Tensor:
    """softmax_j(logits[h, i, j] + (1 - pair_mask[i, j]) * -inf) for fp32 logits [H, N, N] as [H, N, ldw] with
    ldw = N rounded up to 16 and zeros past N (pair_averaging.py:43-49)."""
    _dev(logits, pair_mask)
    H, N, _ = logits.shape
    if logits.dtype != torch.float32 or not logits.is_contiguous() or pair_mask.shape != (N, N) \
            or pair_mask.dtype != torch.float32 or not pair_mask.is_contiguous():
        raise ValueError("pwa_softmax: need contiguous fp32 logits [H, N, N] and pair_mask [N, N]")
    ldw = (N + 15) // 16 * 16
    w = torch.empty((H, N, ldw), dtype=torch.float32, device=logits.device)
    call("bzpf_pwa_softmax", _p(logits), _p(pair_mask), float(inf), _p(w), N, ldw, H, _stream())
    return w


def pwa_avg(w: torch.Tensor, v: torch.Tensor, g: torch.Tensor, S: int, N: int) -> torch.Tensor:
    """sigmoid(g) * (sum_j w[h, i, j] v[s, j, h*32 + d]) for w [H, N, ldw] from pwa_softmax and fp32 v, g
    [S * N, >= 32 H] row views with unit column stride (pair_averaging.py:50-57) -> [S * N, 32 H] fp32."""
    _dev(w)
    H, Nw, ldw = w.shape
    HC = 32 * H
    for t in (v, g):
        if not t.is_cuda or t.dtype != torch.float32 or t.dim() != 2 or t.shape[0] != S * N or t.shape[1] < HC or t.stride(1) != 1:
            raise ValueError("pwa_avg: v and g must be fp32 [S * N, >= 32 H] views with unit column stride")
    if Nw != N or not w.is_contiguous():
        raise ValueError("pwa_avg: w must be the contiguous [H, N, ldw] output of pwa_softmax")
    wp = pwa_wsplit(w)
    out = torch.empty((S * N, HC), dtype=torch.float32, device=v.device)
    call("bzpf_pwa_avg", _p(wp), ldw, _p(v), v.stride(0), _p(g), g.stride(0), _p(out), HC, S, N, H, _stream())
    return out


def pwa_wsplit(w: torch.Tensor) -> torch.Tensor:
    """The weights w [H, N, ldw] of pwa_softmax as three exact bf16 parts in the chunks pwa_avg loads
    ([H, ceil(N / 32), G, 3, 32, 16] bf16: head, 32-row block, 16-token stage (G = ldw / 16 rounded up to even, zeros
    past N), part, row, token)."""
    _dev(w)
    H, N, ldw = w.shape
    if w.dtype != torch.float32 or not w.is_contiguous() or ldw % 16 or ldw < N:
        raise ValueError("pwa_wsplit: w must be the contiguous fp32 [H, N, ldw] output of pwa_softmax")
    wp = torch.empty((H, (N + 31) // 32, (ldw // 16 + 1) // 2 * 2, 3, 32, 16), dtype=torch.bfloat16, device=w.device)
    assert wp.numel() * 2 == _lib.load().bzpf_pwa_wsplit_bytes(N, ldw, H)
    call("bzpf_pwa_wsplit", _p(w), ldw, _p(wp), N, H, _stream())
    return wp


def pair_bias(z: torch.Tensor, ln, w: torch.Tensor) -> torch.Tensor:
    """Linear(LN(z)) for z fp32 [N, N, D] as [H, N, N] in w's dtype."""
    _dev(z, w)
    N, D = z.shape[0], z.shape[-1]
    H = w.shape[0]
    out = torch.empty((H, N, N), dtype=w.dtype, device=z.device)
    call("bzpf_pair_bias", _p(z), _p(f32c(ln.weight)), _p(f32c(ln.bias)), float(ln.eps), _p(w), _p(out), _dt(w),
         N * N, D, H, _stream())
    return out
