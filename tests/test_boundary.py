"""CPU checks of the drop-in boundary: the C-ABI library loads and exports every symbol include/bzpf.h declares,
the ctypes signatures cover the header, and the modules carry the reference checkpoint's parameter names and
shapes (so a converted checkpoint loads with strict=True). No device calls."""

from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest
import torch

from conftest import (ROOT, rand_params, shapes_attention, shapes_layer, shapes_transition, shapes_tri_att,
                      shapes_tri_mul)

HEADER = os.path.join(ROOT, "include", "bzpf.h")


def header_symbols() -> set:
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return set(re.findall(r"\b(bzpf_\w+)\s*\(", txt))


def test_library_exports_header_symbols():
    from boltz_mlx_amd import _lib

    _lib.load()  # maps torch's HIP runtime first
    lib = ctypes.CDLL(_lib.LIB_PATH)
    syms = header_symbols()
    assert len(syms) >= 15
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, missing
    assert set(_lib.SIGNATURES) == syms


def test_library_host_only_calls():
    from boltz_mlx_amd import _lib

    lib = _lib.load()
    assert lib.bzpf_version().decode().startswith("bzpf")
    assert lib.bzpf_row_pitch(1) == 64 and lib.bzpf_row_pitch(64) == 64 and lib.bzpf_row_pitch(65) == 128
    # argument validation happens on the host, before any launch
    rc = lib.bzpf_trimul_proj(None, None, None, 1.0, 0, None, 0, 10, 64, 128, None)
    assert rc == -1 and b"xn" in lib.bzpf_last_error()
    rc = lib.bzpf_triattn_proj(None, None, 0, 1.0, 1.0, None, None, None, 0, 10, 64, 128, 4, 32, None)
    assert rc == -1
    # the weight-split size: 3 KB per (head, 32-row block, 16-token stage), stages rounded up to even
    assert lib.bzpf_pwa_wsplit_bytes(400, 400, 8) == 8 * 13 * 26 * 3072
    assert lib.bzpf_pwa_wsplit_bytes(37, 48, 8) == 8 * 2 * 4 * 3072
    assert lib.bzpf_pwa_wsplit_bytes(37, 40, 8) == -1 and lib.bzpf_pwa_wsplit_bytes(50, 48, 8) == -1
    rc = lib.bzpf_opm_split(None, 64, None, None, 10, 10, None)
    assert rc == -1 and b"NULL" in lib.bzpf_last_error()


def test_header_signatures_match_ctypes():
    """Argument counts of the ctypes table equal the header prototypes."""
    from boltz_mlx_amd import _lib

    txt = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    for name, args in _lib.SIGNATURES.items():
        m = re.search(r"\b" + name + r"\s*\(([^)]*)\)", txt)
        assert m, name
        params = [p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"]
        assert len(params) == len(args), (name, len(params), len(args))


def _names_shapes(mod):
    return {k: tuple(v.shape) for k, v in mod.state_dict().items()}


def test_module_parameter_layout():
    from boltz_mlx_amd.layers.attentionv2 import AttentionPairBias
    from boltz_mlx_amd.layers.pairformer import PairformerLayer, PairformerModule
    from boltz_mlx_amd.layers.transition import Transition
    from boltz_mlx_amd.layers.triangular_attention.attention import TriangleAttentionEndingNode
    from boltz_mlx_amd.layers.triangular_mult import TriangleMultiplicationIncoming

    assert _names_shapes(TriangleMultiplicationIncoming(128)) == shapes_tri_mul(128)
    assert _names_shapes(TriangleAttentionEndingNode(128, 32, 4)) == shapes_tri_att(128, 32, 4)
    assert _names_shapes(Transition(128, 512)) == shapes_transition(128, 512)
    assert _names_shapes(AttentionPairBias(384, 128, 16)) == shapes_attention(384, 128, 16)
    assert _names_shapes(PairformerLayer(384, 128, 16)) == shapes_layer(384, 128, 16)
    m = PairformerModule(384, 128, 2, 16)
    want = {f"layers.{i}.{k}": v for i in range(2) for k, v in shapes_layer(384, 128, 16).items()}
    assert _names_shapes(m) == want


def test_strict_load_and_synthetic_state():
    from boltz_mlx_amd.layers.pairformer import PairformerLayer
    from boltz_mlx_amd.weights import load_module, synthetic_state

    layer = PairformerLayer(64, 128, 4)
    st = rand_params(shapes_layer(64, 128, 4), seed=1)
    load_module(layer, st)
    assert torch.equal(layer.tri_mul_out.p_in.weight, torch.tensor(st["tri_mul_out.p_in.weight"], dtype=torch.float32))
    bad = dict(st)
    bad.pop("tri_att_end.linear.weight")
    with pytest.raises(ValueError):
        load_module(layer, bad)
    syn = synthetic_state(layer, seed=3)
    assert set(syn) == set(st)
    assert np.all(syn["pre_norm_s.weight"] == 1) and np.all(syn["tri_mul_in.norm_out.bias"] == 0)
    assert abs(float(np.std(syn["tri_mul_out.p_in.weight"])) - 0.02) < 0.002


def test_safetensors_roundtrip(tmp_path):
    from safetensors.numpy import save_file

    from boltz_mlx_amd.layers.transition import Transition
    from boltz_mlx_amd.weights import load_safetensors

    st = {f"pairformer_module.layers.0.transition_z.{k}": v.astype(np.float32)
          for k, v in rand_params(shapes_transition(128, 512), seed=2).items()}
    p = tmp_path / "w.safetensors"
    save_file(st, str(p))
    t = Transition(128, 512)
    load_safetensors(t, str(p), prefix="pairformer_module.layers.0.transition_z")
    assert torch.equal(t.fc3.weight, torch.tensor(st["pairformer_module.layers.0.transition_z.fc3.weight"]))


def test_mixed_fp16_checkpoint_loads_exactly(tmp_path):
    """A mixed checkpoint (the reference's boltz_mlx/mixed.py: fp16 copies of the GEMM weights, fp32 for the rest)
    loads through the same strict loader: the fp16 tensors become fp32 parameters exactly, so the fp16 operands the
    kernels build from them are the file's fp16 bits."""
    from safetensors.numpy import save_file

    from boltz_mlx_amd.layers.transition import Transition
    from boltz_mlx_amd.weights import load_safetensors

    full = {k: v.astype(np.float32) for k, v in rand_params(shapes_transition(128, 512), seed=5).items()}
    mixed = {k: (v.astype(np.float16) if k.endswith("weight") and v.ndim == 2 else v) for k, v in full.items()}
    p = tmp_path / "mixed.safetensors"
    save_file(mixed, str(p))
    t = load_safetensors(Transition(128, 512), str(p))
    for k, v in mixed.items():
        got = dict(t.named_parameters())[k].detach()
        assert got.dtype == torch.float32
        if v.dtype == np.float16:
            assert np.array_equal(got.half().numpy().view(np.uint16), v.view(np.uint16)), k
        else:
            assert torch.equal(got, torch.tensor(v)), k


def test_no_cpu_compute_path():
    """The product path refuses CPU tensors instead of computing them some other way."""
    from boltz_mlx_amd import _lib
    from boltz_mlx_amd import kernels as K

    _lib.load()
    x = torch.zeros(4, 128)
    with pytest.raises(ValueError):
        K.layer_norm(x, None, None)
