"""Mixed fp16 / fp32 checkpoints (boltz_mlx_amd/mixed.py): the manifest derived from the modules' kernel-weight
groups, the conversion's overflow check, the format / manifest check on load, and fp16 weights held once (the
parameters of a multi-parameter group are views of the cached kernel weight). CPU only; the GPU test that a mixed
load computes bit for bit what the runtime-cast path computes is in test_gpu_mixed.py."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from boltz_mlx_amd import kernels as K
from boltz_mlx_amd import mixed as M
from boltz_mlx_amd.layers.pairformer import PairformerModule
from boltz_mlx_amd.weights import load_module, synthetic_state


def small_trunk(seed=0):
    m = PairformerModule(48, 32, 2, 4)
    load_module(m, synthetic_state(m, seed, std=0.1))
    return m


def test_manifest_lists_the_gemm_weights():
    m = small_trunk()
    entry = M.manifest_entry(m)
    params = set(entry["params"])
    for i in range(2):
        pre = f"layers.{i}."
        for name in ("tri_mul_out.p_in.weight", "tri_mul_out.g_in.weight", "tri_mul_in.g_out.weight",
                     "tri_att_start.mha.linear_q.weight", "tri_att_end.linear.weight", "tri_att_end.mha.linear_o.weight",
                     "transition_z.fc1.weight", "transition_z.fc3.weight", "transition_s.fc2.weight",
                     "attention.proj_q.weight", "attention.proj_o.weight", "attention.proj_z.1.weight"):
            assert pre + name in params, name
        for name in ("tri_mul_out.norm_in.weight", "attention.proj_q.bias", "pre_norm_s.weight",
                     "attention.proj_z.0.weight", "transition_z.norm.bias"):
            assert pre + name not in params, name
    groups = {(g["owner"], g["cache"]): g for g in entry["groups"]}
    g = groups[("layers.0.tri_mul_out", "w_pg")]
    assert g["srcs"] == ["p_in.weight", "g_in.weight"] and g["storable"] and g["shape"] == [128, 32]
    # the hash is a function of the entry alone
    assert M.entry_sha(entry) == M.entry_sha(M.manifest_entry(small_trunk(seed=3)))
    assert M.entry_sha(entry) != M.entry_sha({**entry, "params": entry["params"][1:]})


def test_to_mixed_overflow_and_missing():
    m = small_trunk()
    entry = M.manifest_entry(m)
    state = {k: v.detach().clone() for k, v in m.state_dict().items()}
    state["layers.0.tri_mul_out.p_in.weight"][0, 0] = 1e6
    with pytest.raises(OverflowError):
        M.to_mixed(state, entry)
    del state["layers.0.tri_mul_out.p_in.weight"]
    with pytest.raises(KeyError):
        M.to_mixed(state, entry)


def test_mixed_round_trip_holds_fp16_once(tmp_path):
    src = small_trunk(seed=1)
    entry = M.manifest_entry(src)
    path = str(tmp_path / "trunk_mixed.safetensors")
    M.save_mixed(path, src.state_dict(), entry)
    dst = M.load_mixed(small_trunk(seed=2), path, entry)
    sd_src, fp16 = src.state_dict(), set(entry["params"])
    for k, v in dst.state_dict().items():
        if k in fp16:
            assert v.dtype == torch.float16, k
            assert torch.equal(v, sd_src[k].to(torch.float16)), k
        else:
            assert v.dtype == torch.float32 and torch.equal(v, sd_src[k]), k
    tm = dst.layers[0].tri_mul_out
    # p_in and g_in are views of one buffer, which is the cached [p_in; g_in] kernel weight
    assert tm.p_in.weight.untyped_storage().data_ptr() == tm.g_in.weight.untyped_storage().data_ptr()
    old = K.PRECISION
    K.set_precision("f16")
    try:
        w_pg, w_po, _ = tm.prepare()
        assert w_pg.data_ptr() == tm.p_in.weight.data_ptr()
        assert w_pg.data_ptr() + tm.p_in.weight.numel() * 2 == tm.g_in.weight.data_ptr()
        assert w_po.data_ptr() == tm.p_out.weight.data_ptr()  # one source: the parameter itself
        assert tm.prepare()[0] is w_pg
        assert torch.equal(w_pg, torch.cat([sd_src["layers.0.tri_mul_out.p_in.weight"],
                                            sd_src["layers.0.tri_mul_out.g_in.weight"]]).to(torch.float16))
    finally:
        K.set_precision(old)


def test_load_rejects_stale_or_foreign_files(tmp_path):
    from safetensors.torch import save_file

    src = small_trunk()
    entry = M.manifest_entry(src)
    path = str(tmp_path / "m.safetensors")
    M.save_mixed(path, src.state_dict(), entry)
    stale = {**entry, "groups": entry["groups"][1:]}
    with pytest.raises(ValueError, match="manifest"):
        M.load_mixed(small_trunk(), path, stale)
    plain = str(tmp_path / "plain.safetensors")
    save_file({k: v.contiguous() for k, v in src.state_dict().items()}, plain)
    with pytest.raises(ValueError, match="format"):
        M.load_mixed(small_trunk(), plain, entry)
    # a file for another model (missing parameters) fails the strict name check
    other = PairformerModule(48, 32, 1, 4)
    load_module(other, synthetic_state(other, 0))
    one = str(tmp_path / "one.safetensors")
    M.save_mixed(one, other.state_dict(), M.manifest_entry(other))
    with pytest.raises(ValueError, match="missing"):
        M.load_mixed(small_trunk(), one, M.manifest_entry(other))


def test_prefuse_keeps_shared_sources_apart():
    """A parameter listed in two groups keeps its own buffer (views of one group would be wrong for the other)."""
    m = small_trunk()
    entry = M.manifest_entry(m)
    tm = m.layers[0].tri_mul_out
    with torch.no_grad():
        for name in ("p_in", "g_in", "g_out"):
            w = getattr(tm, name).weight
            setattr(getattr(tm, name), "weight", torch.nn.Parameter(w.to(torch.float16), requires_grad=False))
    groups = [g for g in entry["groups"] if g["owner"] == "layers.0.tri_mul_out"]
    shared = {"groups": groups + [{"owner": "layers.0.tri_mul_out", "cache": "w_extra", "srcs": ["g_in.weight",
                                                                                                   "g_out.weight"],
                                   "storable": True, "shape": [96, 32]}], "params": []}
    before = tm.g_in.weight.data_ptr()
    M.prefuse(m, shared)
    assert tm.g_in.weight.data_ptr() == before  # not turned into a view
    assert np.isfinite(tm.p_in.weight.float().numpy()).all()
