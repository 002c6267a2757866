"""Pairformer trunk benchmark on one MI355X: Pairformer blocks/s at N=1000 (and N=400), fp16 mixed precision.

Workload (the 64-block trunk configuration): PairformerModule(token_s=384, token_z=128, 64 blocks, 16 s-heads,
triangle attention 4 x 32), synthetic seeded inputs z ~ N(0,1) [1, N, N, 128], s ~ N(0,1) [1, N, 384], 5% of the
tokens padded (pair_mask = tok_i tok_j), random-init weights ~ N(0, 0.02) with LayerNorm gamma=1 beta=0. A step is
one Pairformer block (layer i % 64 of the trunk, applied in place to the resident z and s), so --steps 64 is one
full trunk pass. Inputs and weights are resident in HBM before the timed region.

Prints one JSON line. `roofline` is for the kernel with the largest share of the timed region, from HIP events
recorded around every launch on the launch stream, against the published peaks (`frac`) and against the GEMM and
copy rates measured in the same run (`frac_measured`, `measured_ceilings`); `cpu_baseline` times the numpy oracle
(reference-equivalent fp32 CPU path) on the N=128 block, N=400 triangle attention, N=800 triangle multiplication and
one diffusion-transformer layer, and estimates one N=1000 block from row samples and FLOP ratios (see cpu_baseline).
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0


def block_flops(N: int) -> float:
    """Algorithmic FLOP of one Pairformer block (triangle ops, transitions, s track)."""
    return 1536.0 * N ** 3 + 1121792.0 * N ** 2 + 5013504.0 * N


def kernel_work(name: str, N: int, H: int = 4, C: int = 32, D: int = 128) -> tuple[float, float]:
    """(algorithmic FLOP, algorithmic HBM bytes) of one launch of a pair-track entry point at N tokens, fp16
    storage, fp32 z: the per-unit figures times the units one launch processes."""
    R = N * N
    if name == "bzpf_trimul_contract":   # 128 channels of N x N x N; read a, b, write o (fp16)
        return 2.0 * D * N ** 3, 6.0 * D * N ** 2
    if name == "bzpf_triattn_core":      # QK^T and PV per (row, head); q|k|v|g + bias + mask read, out written
        return 4.0 * H * C * N ** 3, (2 * 4 * H * C + 2 * H + 4 + 2 * H * C) * float(R)
    if name == "bzpf_transition":        # 128 -> 2x512 -> 128 per row; xn in, z r/w, next LN out
        return 393216.0 * R, R * D * (2 + 4 + 4 + 2.0)
    if name == "bzpf_transition_pb":     # the transition plus the s track's 128 -> 16 pair bias (16 fp16 out)
        return (393216.0 + 2.0 * 128 * 16) * R, R * (D * (2 + 4 + 4 + 2.0) + 32.0)
    if name == "bzpf_attn_out_transition":  # linear_o + residual, then the transition with the pair bias: o in, z r/w,
        # next LN and the 16-head pair bias out (the intermediate z, written and read back, is not algorithmic)
        return (2.0 * 128 * 128 + 393216.0 + 2.0 * 128 * 16) * R, R * (256 + 1024 + 256 + 32.0)
    if name == "bzpf_trimul_proj":       # 128 -> 512 per row; xn in, a|b (256 ch) out
        return 131072.0 * R, R * (D * 2 + 256 * 2.0)
    if name == "bzpf_trimul_tail":       # two 128 x 128 GEMMs per row; o, xn in, z r/w, next LN out
        return 65536.0 * R, R * (256 + 256 + 1024 + 256.0)
    if name == "bzpf_triattn_proj":      # 128 -> 516 per row; xn in, q|k|v|g + bias out
        return 2.0 * 128 * (4 * H * C + H) * R, R * (D * 2 + (4 * H * C + H) * 2.0)
    if name == "bzpf_linear_resid_ln":   # 128 x 128 per row; x in, z r/w, next LN out
        return 2.0 * 128 * 128 * R, R * (256 + 1024 + 256.0)
    if name == "bzpf_pair_bias":         # LN + 128 -> 16 per row; z in, bias out
        return 2.0 * 128 * 16 * R, R * (512 + 32.0)
    return 0.0, 0.0


def profiled_traffic(name: str, N: int):
    """HBM bytes per launch of `name` at N from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary
    (profiles/traffic_N{N}_fp16.json, counters scaled by the copy-kernel calibration), or None."""
    path = os.path.join(ROOT, "profiles", f"traffic_N{N}_fp16.json")
    try:
        with open(path) as f:
            return json.load(f)["kernels"][name]["traffic_bytes"]
    except (OSError, KeyError, ValueError):
        return None


def roofline_for(name: str, ms: float, N: int, ceilings: dict | None = None) -> dict:
    """Roofline of one launch against the published peaks; with `ceilings` (measured_ceilings) also the fraction of
    the rate measured in the same run (frac_measured)."""
    fl, by = kernel_work(name, N)
    traffic = profiled_traffic(name, N)
    t_fl = fl / (MFMA_F16_PEAK_TFLOPS * 1e12)
    t_by = by / (HBM_PEAK_GBS * 1e9)
    if t_fl >= t_by:
        ach = fl / (ms * 1e-3) / 1e12
        out = {"kernel": name, "bound": "mfma", "achieved": round(ach, 2), "peak": MFMA_F16_PEAK_TFLOPS,
               "unit": "TFLOP/s", "frac": round(ach / MFMA_F16_PEAK_TFLOPS, 4), "traffic": traffic,
               "avg_ms": round(ms, 4), "algorithmic_flop": fl, "algorithmic_bytes": by}
        if ceilings:
            out["frac_measured"] = round(ach / ceilings["gemm_f16_tflops"], 4)
        return out
    ach = by / (ms * 1e-3) / 1e9
    out = {"kernel": name, "bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
           "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic, "avg_ms": round(ms, 4),
           "algorithmic_flop": fl, "algorithmic_bytes": by}
    if ceilings:
        out["frac_measured"] = round(ach / ceilings["copy_gbs"], 4)
    return out


def measured_ceilings(device) -> dict:
    """Attainable rates measured in the same run: a plain fp16 GEMM through torch (hipBLASLt / rocBLAS), 8192^3,
    and a 1 GiB device-to-device copy (bytes read + written); best of 10 after 3 warm-ups each."""
    import torch

    def best_ms(fn, reps=10):
        for _ in range(3):
            fn()
        best = float("inf")
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            torch.cuda.synchronize()
            best = min(best, a.elapsed_time(b))
        return best

    n = 8192
    g = torch.Generator(device=device).manual_seed(3)
    x = torch.randn((n, n), generator=g, device=device).half()
    y = torch.randn((n, n), generator=g, device=device).half()
    c = torch.empty((n, n), dtype=torch.float16, device=device)
    t_gemm = best_ms(lambda: torch.matmul(x, y, out=c))
    del x, y, c
    src = torch.empty(256 << 20, dtype=torch.float32, device=device).fill_(1.0)
    dst = torch.empty_like(src)
    t_copy = best_ms(lambda: dst.copy_(src))
    nbytes = 2.0 * src.numel() * 4
    del src, dst
    torch.cuda.empty_cache()
    return {"gemm_f16_tflops": round(2.0 * n ** 3 / (t_gemm * 1e-3) / 1e12, 1),
            "copy_gbs": round(nbytes / (t_copy * 1e-3) / 1e9, 1),
            "how": "torch fp16 matmul 8192^3 (hipBLASLt/rocBLAS) and a 1 GiB device copy, best of 10"}


def make_trunk(N: int, blocks: int, seed: int, device):
    import numpy as np
    import torch

    from boltz_mlx_amd.layers.pairformer import PairformerModule
    from boltz_mlx_amd.weights import load_module, synthetic_state

    m = PairformerModule(384, 128, blocks, 16)
    load_module(m, synthetic_state(m, seed))
    m = m.to(device)
    rng = np.random.default_rng(seed + 1)
    z = torch.tensor(rng.standard_normal((1, N, N, 128), dtype=np.float32), device=device)
    s = torch.tensor(rng.standard_normal((1, N, 384), dtype=np.float32), device=device)
    tok = torch.ones((1, N), dtype=torch.float32, device=device)
    tok[:, N - int(round(0.05 * N)):] = 0
    pm = (tok[:, :, None] * tok[:, None, :]).contiguous()
    return m, s, z, tok, pm


def run_blocks(m, s, z, tok, pm, start: int, count: int, xn=None):
    """Apply `count` consecutive blocks of the trunk (cycling) in place, as PairformerModule runs them (the s track
    of each block overlapped with the next block's pair kernels); carries the next norm_in output."""
    return m.run(s, z, tok, pm, start, count, xn=xn, cycle=True)


def c5_flops_per_step(N: int = 400, samples: int = 5, depth: int = 24, D: int = 768) -> float:
    """Diffusion token transformer, one step: per layer and sample 2 N D (4D + D + 6D) + 2 N 2D D + 4 N^2 D
    (q|k|v|g, output, [gates; x; a_to_b] and b_to_a GEMMs, q k^T and P v); the conditioning GEMMs are step-invariant."""
    return float(depth * samples * (2 * N * D * (4 * D + D + 6 * D) + 2 * N * 2 * D * D + 4 * N * N * D))


def diffusion_transformer_leg(steps: int, device) -> dict:
    """The diffusion-transformer stack (24 layers, D 768, 16 heads x 48, N 400, 5 samples sharing one pair bias)
    timed over `steps` sampler steps, each a full pass of the stack with the output fed back as the next input,
    eagerly and replayed from a captured HIP graph (ms_per_step); the pair bias (LN(z) W, z [400, 400, 128] -> 24 x 16 heads, laid out per layer) and the s conditioning are
    computed once."""
    import torch

    from boltz_mlx_amd import kernels as K
    from boltz_mlx_amd.layers.transformersv2 import DiffusionStepGraph, DiffusionTransformer
    from boltz_mlx_amd.weights import load_module, synthetic_state

    N, D, H, L, S = 400, 768, 16, 24, 5
    m = DiffusionTransformer(depth=L, heads=H, dim=D)
    load_module(m, synthetic_state(m, seed=5, std=0.02))
    m = m.to(device)
    g = torch.Generator(device=device).manual_seed(5)
    a = torch.randn((S, N, D), generator=g, device=device)
    s = torch.randn((S, N, D), generator=g, device=device)
    z = torch.randn((N * N, 128), generator=g, device=device)
    w_z = (0.02 * torch.randn((L * H, 128), generator=g, device=device)).to(K.storage_dtype())
    bias = K.linear(K.layer_norm(z, None, None, 1e-5, out_dtype=K.storage_dtype()), w_z).view(1, N, N, L * H)
    mask = torch.ones((S, N), device=device)
    mask[:, N - N // 20:] = 0
    cond = m.precompute_cond(s)
    prepared = m.prepare(bias)
    for _ in range(2):
        a = m(a, s, bias, mask, multiplicity=S, cond=cond, prepared=prepared)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        a = m(a, s, bias, mask, multiplicity=S, cond=cond, prepared=prepared)
    torch.cuda.synchronize()
    dt_eager = time.perf_counter() - t0
    # the same steps replayed from one captured HIP graph (the sampler's loop: conditioning fixed, a fed back)
    step = DiffusionStepGraph(m, a, cond, prepared, mask, multiplicity=S)
    for _ in range(2):
        a = step(a)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        a = step(a)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    fl = c5_flops_per_step(N, S, L, D)
    return {"workload": "diffusion_transformer_24L_D768_N400_5samples_fp16", "steps": steps,
            "steps_per_s": round(steps / dt, 3), "ms_per_step": round(1e3 * dt / steps, 3),
            "ms_per_step_eager": round(1e3 * dt_eager / steps, 3),
            "tflops_effective": round(fl * steps / dt / 1e12, 2), "flop_per_step": fl,
            "finite": bool(torch.isfinite(a).all().item())}


def msa_layer_leg(steps: int, device, N: int = 400, S: int = 1024) -> dict:
    """One MSA block (MSALayer: pair-weighted averaging, transition on m, outer-product mean, NoSeq pair layer) at
    N tokens and S MSA rows (5 % padded tokens, 10 % masked MSA entries), random-init weights, timed over `steps`
    layer calls. The outer sum and the weighted average are fp32-accurate reductions (the reference's numerics
    policy) on the bf16 matrix cores (three exact bf16 parts per fp32 operand); their fp32 FLOPs are reported."""
    import torch

    from boltz_mlx_amd.layers.msa import MSALayer
    from boltz_mlx_amd.weights import load_module, synthetic_state

    m = MSALayer(64, 128)
    load_module(m, synthetic_state(m, seed=7, std=0.02))
    m = m.to(device)
    g = torch.Generator(device=device).manual_seed(7)
    z = torch.randn((1, N, N, 128), generator=g, device=device)
    msa = torch.randn((1, S, N, 64), generator=g, device=device)
    tok = torch.ones((1, N), device=device)
    tok[:, N - N // 20:] = 0
    pm = tok[:, :, None] * tok[:, None, :]
    msa_mask = (torch.rand((1, S, N), generator=g, device=device) > 0.1).float() * tok[:, None, :]
    for _ in range(2):
        zo, mo = m(z, msa, pm, msa_mask)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        zo, mo = m(z, msa, pm, msa_mask)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    fl_opm = 2.0 * (32 * N) ** 2 * S
    fl_pwa = 2.0 * 8 * N * N * S * 32
    return {"workload": f"msa_layer_N{N}_S{S}_fp16", "steps": steps, "ms_per_layer": round(1e3 * dt, 3),
            "fp32_reduction_flop": fl_opm + fl_pwa,
            "finite": bool(torch.isfinite(zo).all().item() and torch.isfinite(mo).all().item())}


def config_legs(device) -> dict:
    """The module-level configurations on the GPU, each through the reference's module API with random-init weights
    and seeded inputs: C1 one PairformerLayer in fp32 at N = 128 (all-ones mask); C2 triangle attention, starting +
    ending node, N = 400 with the last 40 tokens padded, fp16; C3 triangle multiplication, outgoing + incoming,
    N = 800, fp16. Each: 3 warm-up calls, then the best of 5 timed batches of 5 calls (HIP events); TFLOP/s from the
    algorithmic counts (C1: the block FLOP; C2: per node 512 N^3 + 164,864 N^2 (core, projection, linear_o);
    C3: per direction 256 N^3 + 196,608 N^2)."""
    import torch

    from boltz_mlx_amd import kernels as K
    from boltz_mlx_amd.layers.pairformer import PairformerLayer
    from boltz_mlx_amd.layers.triangular_attention.attention import (TriangleAttentionEndingNode,
                                                                     TriangleAttentionStartingNode)
    from boltz_mlx_amd.layers.triangular_mult import TriangleMultiplicationIncoming, TriangleMultiplicationOutgoing
    from boltz_mlx_amd.weights import load_module, synthetic_state

    def best_ms(fn, calls=5, reps=5):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        best = float("inf")
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(calls):
                fn()
            b.record()
            torch.cuda.synchronize()
            best = min(best, a.elapsed_time(b) / calls)
        return best

    def module(m, seed):
        load_module(m, synthetic_state(m, seed))
        return m.to(device)

    g = torch.Generator(device=device).manual_seed(11)
    out = {}
    old = K.PRECISION
    try:
        K.set_precision("fp32")
        N = 128
        layer = module(PairformerLayer(384, 128, 16), 21)
        z = torch.randn((1, N, N, 128), generator=g, device=device)
        s = torch.randn((1, N, 384), generator=g, device=device)
        tok = torch.ones((1, N), device=device)
        pm = tok[:, :, None] * tok[:, None, :]
        ms = best_ms(lambda: layer(s, z, tok, pm))
        out["C1_block_N128_fp32"] = {"ms": round(ms, 4), "blocks_per_s": round(1e3 / ms, 1),
                                     "tflops": round(block_flops(N) / (ms * 1e-3) / 1e12, 2)}
        K.set_precision("f16")
        N = 400
        ts, te = module(TriangleAttentionStartingNode(128, 32, 4), 22), module(TriangleAttentionEndingNode(128, 32, 4), 23)
        z = torch.randn((1, N, N, 128), generator=g, device=device)
        tok = torch.ones((1, N), device=device)
        tok[:, N - 40:] = 0
        pm = tok[:, :, None] * tok[:, None, :]
        ms = best_ms(lambda: (ts(z, pm), te(z, pm)))
        fl = 2 * (512.0 * N ** 3 + 164864.0 * N ** 2)
        out["C2_tri_att_N400_start_end_f16"] = {"ms": round(ms, 4), "tflops": round(fl / (ms * 1e-3) / 1e12, 2)}
        N = 800
        mo, mi = module(TriangleMultiplicationOutgoing(128), 24), module(TriangleMultiplicationIncoming(128), 25)
        z = torch.randn((1, N, N, 128), generator=g, device=device)
        pm = torch.ones((1, N, N), device=device)
        ms = best_ms(lambda: (mo(z, pm), mi(z, pm)))
        fl = 2 * (256.0 * N ** 3 + 196608.0 * N ** 2)
        out["C3_tri_mul_N800_out_in_f16"] = {"ms": round(ms, 4), "tflops": round(fl / (ms * 1e-3) / 1e12, 2)}
        del z, pm
        torch.cuda.empty_cache()
    finally:
        K.set_precision(old)
    return out


def _median_time(fn, reps: int, budget_s: float):
    """1 warm-up call, then up to `reps` timed calls (fewer when the warm-up shows they would exceed budget_s;
    at least 1); returns (median seconds, timed calls)."""
    import statistics

    t0 = time.perf_counter()
    fn()
    warm = time.perf_counter() - t0
    n = max(1, min(reps, int(budget_s / max(warm, 1e-9))))
    ts = []
    for _ in range(n):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts), n


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(budget_s: float = 25.0) -> dict:
    """The numpy float32 oracle (reference-equivalent fp32 CPU path) on the host cores: each configuration gets
    1 warm-up and the median of up to 5 timed runs (fewer if 5 would exceed budget_s), on the BLAS thread pool the
    environment gives (OMP_NUM_THREADS; numpy's elementwise work is single-threaded).
      C1: one PairformerLayer, N = 128;  C2: triangle attention N = 400 (last 40 padded), starting + ending node;
      C3: triangle multiplication N = 800, outgoing + incoming;  C5: one diffusion-transformer layer (D 768,
      16 heads, N = 400, 5 samples), with a sampler-step ESTIMATE of 24 layers.
    value: blocks/s at N = 1000 (ESTIMATE): triangle attention from a row sample at N = 1000 (rows are independent:
    fixed + per-row cost from two sample sizes, times 1000 rows, both nodes), triangle multiplication from C3 scaled
    by its module FLOP ratio 800 -> 1000, the pair transition from a 10^5-row sample (row-wise, times 10), and the s
    track (pre-norm, AttentionPairBias with the pair bias from z, transition_s) timed at N = 1000."""
    import numpy as np

    import oracle as O
    from boltz_mlx_amd.layers.pairformer import PairformerLayer
    from boltz_mlx_amd.weights import synthetic_state

    try:
        from threadpoolctl import threadpool_info
        threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:  # threadpoolctl absent: report the visible cores
        threads = os.cpu_count()
    f32 = np.float32
    p = synthetic_state(PairformerLayer(384, 128, 16), seed=0)
    rng = np.random.default_rng(1)

    def inputs(N, n_pad):
        z = rng.standard_normal((1, N, N, 128), dtype=f32)
        tok = np.ones((1, N), f32)
        if n_pad:
            tok[:, N - n_pad:] = 0
        return z, tok, tok[:, :, None] * tok[:, None, :]

    cfg = {}
    z, tok, pm = inputs(128, 0)
    s = rng.standard_normal((1, 128, 384), dtype=f32)
    t, n = _median_time(lambda: O.pairformer_layer(s, z, tok, pm, p, 16), 5, budget_s)
    cfg["C1_block_N128_fp32"] = {"s": round(t, 4), "runs": n}
    z, tok, pm = inputs(400, 40)
    pa, pe = O.sub(p, "tri_att_start"), O.sub(p, "tri_att_end")
    t, n = _median_time(lambda: (O.tri_att(z, pm, pa, True), O.tri_att(z, pm, pe, False)), 5, budget_s)
    cfg["C2_tri_att_N400_start_end"] = {"s": round(t, 4), "runs": n}
    z, tok, pm = inputs(800, 0)
    po, pi = O.sub(p, "tri_mul_out"), O.sub(p, "tri_mul_in")
    t_c3, n = _median_time(lambda: (O.tri_mul(z, pm, po, True), O.tri_mul(z, pm, pi, False)), 5, budget_s)
    cfg["C3_tri_mul_N800_out_in"] = {"s": round(t_c3, 4), "runs": n}
    del z, tok, pm
    # C4 estimate at N = 1000
    N = 1000
    z, tok, pm = inputs(N, 50)
    r1, r2 = 8, 24
    t1 = min(_time_once(lambda: O.tri_att(z, pm, pa, True, row_chunk=8, rows=r1)) for _ in range(2))
    t2 = min(_time_once(lambda: O.tri_att(z, pm, pa, True, row_chunk=8, rows=r2)) for _ in range(2))
    per_row = max(t2 - t1, 0.0) / (r2 - r1)
    t_att = 2 * (max(t1 - r1 * per_row, 0.0) + N * per_row)
    fl = lambda n: 256.0 * n ** 3 + 196608.0 * n ** 2  # noqa: E731  (module FLOP per direction)
    t_mul = t_c3 * fl(N) / fl(800)
    rows = 100_000
    xr = z.reshape(-1, 128)[:rows]
    t_tr = min(_time_once(lambda: O.transition(xr, O.sub(p, "transition_z"))) for _ in range(2)) * (N * N / rows)
    s = rng.standard_normal((1, N, 384), dtype=f32)

    def s_track():
        s_n = O.layer_norm(s, p["pre_norm_s.weight"], p["pre_norm_s.bias"])
        s1 = s + O.attention_pair_bias(s_n, z, tok, s_n, O.sub(p, "attention"), 16)
        return s1 + O.transition(s1, O.sub(p, "transition_s"))

    t_s = _time_once(s_track)
    t_block = t_att + t_mul + t_tr + t_s
    del z, xr
    # C5: one diffusion-transformer layer (D 768, 16 heads x 48) over 5 samples at N = 400; a sampler step is 24 layers
    from boltz_mlx_amd.layers.transformersv2 import DiffusionTransformer
    from oracle import diffusion as OD

    pd = synthetic_state(DiffusionTransformer(depth=1, heads=16, dim=768), seed=2, std=0.02)
    a5 = rng.standard_normal((5, 400, 768), dtype=f32)
    s5 = rng.standard_normal((5, 400, 768), dtype=f32)
    b5 = rng.standard_normal((1, 400, 400, 16), dtype=f32)
    m5 = np.ones((5, 400), f32)
    m5[:, 380:] = 0
    t_c5, n = _median_time(lambda: OD.diffusion_transformer(a5, s5, b5, m5, pd, 1, 16, 5), 5, budget_s)
    cfg["C5_diffusion_layer_N400_5samples"] = {"s": round(t_c5, 4), "runs": n,
                                               "step_estimate_s": round(24 * t_c5, 3)}
    return {"value": round(1.0 / t_block, 6), "unit": "blocks/s", "cores": int(threads), "kind": "port",
            "cpu_model": _cpu_model(), "os_cpu_count": os.cpu_count(),
            "sample": (f"numpy float32 oracle, {threads} BLAS threads; configs (1 warm-up + median): "
                       + ", ".join(f"{k} {v['s']} s (median of {v['runs']})" for k, v in cfg.items())
                       + f"; value = ESTIMATE of one N=1000 block ({t_block:.1f} s): tri-att {t_att:.1f} s "
                         f"(rows {r1}/{r2} sampled), tri-mul {t_mul:.1f} s (C3 x FLOP ratio), transition "
                         f"{t_tr:.1f} s (1e5-row sample), s track {t_s:.1f} s; C5 step ESTIMATE = 24 x one "
                         f"layer ({24 * t_c5:.2f} s)"),
            "configs": cfg}


def _time_once(fn) -> float:
    t0 = time.perf_counter()
    fn()
    return time.perf_counter() - t0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64, help="timed Pairformer blocks at N")
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--n", type=int, default=1000)
    ap.add_argument("--n-small", type=int, default=400)
    ap.add_argument("--small-warmup", type=int, default=64,
                    help="untimed blocks before the N=400 figure (at least, and at least 0.5 s of them)")
    ap.add_argument("--small-steps", type=int, default=128, help="timed blocks per window for the N=400 figure")
    ap.add_argument("--small-windows", type=int, default=3,
                    help="timed windows at N=400 (at least; more, up to 3x as many, until three of them agree "
                         "within 3%%); the figure is the median window")
    ap.add_argument("--cpu-budget", type=float, default=25.0,
                    help="seconds per CPU-baseline configuration (bounds the timed runs after the warm-up)")
    ap.add_argument("--blocks", type=int, default=64)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--c5-steps", type=int, default=20,
                    help="diffusion-transformer sampler steps timed after the trunk (0: skip)")
    ap.add_argument("--msa-steps", type=int, default=5, help="MSA-block layer calls timed after the trunk (0: skip)")
    ap.add_argument("--no-configs", action="store_true", help="skip the C1 / C2 / C3 module timings")
    ap.add_argument("--no-ceilings", action="store_true", help="skip the measured GEMM / copy ceilings")
    ap.add_argument("--msa-only", action="store_true", help="time only the MSA-block leg and print its JSON line")
    ap.add_argument("--c5-only", action="store_true",
                    help="time only the diffusion-transformer leg (for profiling it) and print its JSON line")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="end with one 512 MiB device-to-device copy (the known-size kernel that scales the "
                         "FETCH_SIZE / WRITE_SIZE counters of rocprofv3 --pmc); skips the measured ceilings")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the library has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        return 2

    import torch

    from boltz_mlx_amd import kernels as K

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm device", file=sys.stderr)
        return 1
    K.set_precision("f16")
    dev = torch.device("cuda:0")
    torch.backends.cuda.matmul.allow_tf32 = False
    if args.c5_only:
        with torch.no_grad():
            print(json.dumps({"diffusion_transformer": diffusion_transformer_leg(args.c5_steps, dev)}), flush=True)
        return 0
    if args.msa_only:
        with torch.no_grad():
            print(json.dumps({"msa_layer": msa_layer_leg(args.msa_steps, dev)}), flush=True)
        return 0
    result_small, small_windows, times_small = None, None, None
    with torch.no_grad():
        # N = 400 blocks/s (secondary figure)
        if args.n_small:
            m, s, z, tok, pm = make_trunk(args.n_small, args.blocks, 0, dev)
            # warm-up: at least small_warmup blocks and 0.5 s of them (clocks settle), then the median of the
            # timed windows
            done, t0 = 0, time.perf_counter()
            xn = None
            while done < args.small_warmup or time.perf_counter() - t0 < 0.5:
                xn = run_blocks(m, s, z, tok, pm, done, 16, xn)
                done += 16
                torch.cuda.synchronize()
            windows = []
            nmin = max(1, args.small_windows)

            def settled(ws):  # three windows within 3% of each other
                w = sorted(ws)
                return any(w[i + 2] <= 1.03 * w[i] for i in range(len(w) - 2))

            while len(windows) < nmin or (len(windows) < 3 * nmin and not settled(windows)):
                t0 = time.perf_counter()
                xn = run_blocks(m, s, z, tok, pm, done, args.small_steps, xn)
                torch.cuda.synchronize()
                windows.append(args.small_steps / (time.perf_counter() - t0))
                done += args.small_steps
            result_small = float(statistics.median(windows))
            small_windows = [round(w, 1) for w in windows]
            # per-kernel event times at N = 400 over one more window
            K.start_timing()
            run_blocks(m, s, z, tok, pm, done, args.small_steps, xn)
            torch.cuda.synchronize()
            times_small = K.stop_timing()
            del m, s, z, tok, pm
            torch.cuda.empty_cache()
        m, s, z, tok, pm = make_trunk(args.n, args.blocks, 0, dev)
        xn = run_blocks(m, s, z, tok, pm, 0, args.warmup)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        run_blocks(m, s, z, tok, pm, args.warmup, args.steps, xn)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        finite = bool(torch.isfinite(z).all().item() and torch.isfinite(s).all().item())
        # per-kernel breakdown: HIP events around every launch on the launch stream, over the same number of blocks
        K.start_timing()
        t1 = time.perf_counter()
        run_blocks(m, s, z, tok, pm, args.warmup + args.steps, args.steps, xn)
        torch.cuda.synchronize()
        dt_ev = time.perf_counter() - t1
        times = K.stop_timing()
        if args.calibrate_copy:
            a = torch.empty(128 << 20, dtype=torch.float32, device=dev).fill_(1.0)
            b = torch.empty_like(a)
            torch.cuda.synchronize()
            b.copy_(a)
            torch.cuda.synchronize()
            del a, b
    ceilings = None
    if not (args.calibrate_copy or args.no_ceilings):  # a counter run keeps the calibration copy the only large copy
        with torch.no_grad():
            ceilings = measured_ceilings(dev)
    total = {k: sum(v) for k, v in times.items()}
    main = {k: v for k, v in total.items() if not k.endswith(K.SIDE)}
    dom = max(main, key=main.get)
    roof = roofline_for(dom, total[dom] / len(times[dom]), args.n, ceilings)
    # shares over the main stream's launches; the s track's launches on the side stream overlap them (their event
    # intervals include the wait for compute units the attention core holds) and carry no share
    breakdown = {k: {"ms_total": round(v, 3), "launches": len(times[k]),
                     "share": None if k.endswith(K.SIDE) else round(v / sum(main.values()), 4)}
                 for k, v in sorted(total.items(), key=lambda kv: (kv[0].endswith(K.SIDE), -kv[1]))}
    per_kernel_roof = {k: roofline_for(k, total[k] / len(times[k]), args.n, ceilings) for k in total
                       if kernel_work(k, args.n)[0] > 0}
    roof_small = None
    if times_small:
        roof_small = {k: roofline_for(k, sum(v) / len(v), args.n_small, ceilings) for k, v in times_small.items()
                      if not k.endswith(K.SIDE) and kernel_work(k, args.n_small)[0] > 0}
    value = args.steps / dt
    out = {
        "metric": f"Pairformer blocks/sec at N={args.n} fp16",
        "value": round(value, 4),
        "unit": "blocks/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * dt / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded N(0,1) z and s, random-init weights N(0,0.02), 5% padded tokens)",
        "config": {"workload": f"pairformer_trunk_{args.blocks}blocks_N{args.n}_fp16", "N": args.n,
                   "blocks": args.blocks, "token_s": 384, "token_z": 128, "s_heads": 16,
                   "tri_heads": 4, "tri_head_dim": 32, "pad_frac": 0.05, "parallelism": "none (1 GPU)"},
        "blocks_per_s_n400": None if result_small is None else round(result_small, 4),
        "n400_windows": small_windows,
        "tflops_effective": round(value * block_flops(args.n) / 1e12, 2),
        "finite": finite,
        "roofline": roof,
        "kernel_breakdown": breakdown,
        "kernel_roofline": per_kernel_roof,
        "kernel_roofline_n400": roof_small,
        "timed_with_events_s": round(dt_ev, 4),
        "measured_ceilings": ceilings,
    }
    if args.c5_steps:
        with torch.no_grad():
            out["diffusion_transformer"] = diffusion_transformer_leg(args.c5_steps, dev)
    if args.msa_steps:
        with torch.no_grad():
            out["msa_layer"] = msa_layer_leg(args.msa_steps, dev)
    if not args.no_configs and not args.calibrate_copy:
        with torch.no_grad():
            out["config_legs"] = config_legs(dev)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.cpu_budget)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
