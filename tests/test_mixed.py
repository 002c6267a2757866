"""Mixed fp16 / fp32 checkpoints (boltz_mlx_amd/mixed.py), CPU only.

The fp16 parameter set and the kernel-weight partition are pinned against the reference's committed manifest
(tests/golden/fp16_manifest_layers.json, written from boltz_mlx/fp16_manifest.json by make_manifest_fixture.py):
per Pairformer layer 27 parameters, per MSA layer 28, per diffusion token-transformer layer 11. A file converted with
the reference's manifest entry for the whole checkpoint loads into a sub-model here. The GPU test that a mixed load
computes bit for bit what the runtime-cast path computes is in test_gpu_mixed.py."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

from boltz_mlx_amd import kernels as K
from boltz_mlx_amd import mixed as M
from boltz_mlx_amd.layers.pairformer import PairformerModule
from boltz_mlx_amd.weights import load_module, synthetic_state

FIXTURE = os.path.join(os.path.dirname(__file__), "golden", "fp16_manifest_layers.json")


@pytest.fixture(scope="module")
def ref_manifest():
    with open(FIXTURE) as f:
        return json.load(f)


def small_trunk(seed=0, blocks=2):
    m = PairformerModule(48, 32, blocks, 4)
    load_module(m, synthetic_state(m, seed, std=0.1))
    return m


def _under(entry: dict, prefix: str) -> set:
    return {p[len(prefix):] for p in entry["params"] if p.startswith(prefix)}


def _source_tuples(groups: list, layer_prefix: str = "") -> set:
    """(full source names, shape) of each storable group; owners relative to the layer."""
    out = set()
    for g in groups:
        if not g["storable"]:
            continue
        owner = g["owner"][len(layer_prefix):] if g["owner"].startswith(layer_prefix) else g["owner"]
        out.add((tuple(f"{owner}.{s}" if owner else s for s in g["srcs"]), tuple(g["shape"])))
    return out


def _layer_groups(entry: dict, layer: str) -> list:
    return [g for g in entry["groups"] if g["owner"] == layer or g["owner"].startswith(layer + ".")]


def test_pairformer_layer_matches_reference_manifest(ref_manifest):
    """The Boltz-2 trunk layer (token_s 384, token_z 128, 16 heads): same 27 fp16 parameters in every layer, and the
    same kernel-weight partition (sources and shapes) as the reference's manifest."""
    ref = ref_manifest["pairformer_layer"]
    entry = M.manifest_entry(PairformerModule(384, 128, 2, 16))
    for i in range(2):
        assert _under(entry, f"layers.{i}.") == set(ref["params"]), i
    assert len(ref["params"]) == 27
    ours = {(tuple(s[len("layers.0."):] for s in srcs), shape)
            for srcs, shape in _source_tuples(_layer_groups(entry, "layers.0"))}
    assert ours == _source_tuples(ref["groups"])
    # the s track's attention projections are fp32 in f16 mode, as in the reference
    assert "attention.proj_q.weight" not in ref["params"] and "attention.proj_z.1.weight" in ref["params"]


def test_msa_layer_matches_reference_manifest(ref_manifest):
    from boltz_mlx_amd.layers.msa import MSALayer

    ref = ref_manifest["msa_layer"]
    layer = MSALayer(64, 128)
    entry = M.manifest_entry(layer)
    assert set(entry["params"]) == set(ref["params"]) and len(ref["params"]) == 28
    assert _source_tuples(entry["groups"]) == _source_tuples(ref["groups"])


def test_token_transformer_layer_matches_reference_manifest(ref_manifest):
    """The diffusion token transformer (24 x 768, 16 heads; two layers here): the layer's four groups, the stack's
    output-gate group, and the 11 fp16 parameters per layer (output_projection registered under two names)."""
    from boltz_mlx_amd.layers.transformersv2 import DiffusionTransformer

    ref = ref_manifest["token_transformer_layer"]
    entry = M.manifest_entry(DiffusionTransformer(2, 16, 768, 768))
    assert _under(entry, "layers.0.") == set(ref["params"]) and len(ref["params"]) == 11
    ours = {(tuple(s[len("layers.0."):] for s in srcs), shape)
            for srcs, shape in _source_tuples(_layer_groups(entry, "layers.0"))}
    assert ours == _source_tuples(ref["groups"])
    stack = [g for g in entry["groups"] if g["owner"] == ""]
    ref_stack = [g for g in ref_manifest["token_transformer_stack_groups_layer0"] if g["storable"]]
    assert len(stack) == 1 and len(ref_stack) == 1
    assert stack[0]["srcs"][:2] == ref_stack[0]["srcs"]


def test_manifest_is_a_function_of_the_architecture():
    entry = M.manifest_entry(small_trunk())
    assert M.entry_sha(entry) == M.entry_sha(M.manifest_entry(small_trunk(seed=3)))
    assert M.entry_sha(entry) != M.entry_sha({**entry, "params": entry["params"][1:]})
    g = {(r["owner"], r["cache"]): r for r in entry["groups"]}[("layers.0.tri_mul_out", "w_pg")]
    assert g == {"owner": "layers.0.tri_mul_out", "cache": "w_pg", "srcs": ["p_in.weight", "g_in.weight"],
                 "shape": [128, 32], "storable": True}


def test_convert_checks_range_dtype_and_presence():
    m = small_trunk()
    entry = M.manifest_entry(m)
    state = {k: v.detach().clone() for k, v in m.state_dict().items()}
    name = "layers.0.tri_mul_out.p_in.weight"
    state[name][0, 0] = 65519.0  # rounds to 65504: representable
    state[name][0, 1] = -3e-8  # just above half the smallest subnormal: rounds to -2^-24, not to zero
    state[name][0, 2] = 1e-9  # flushes to zero
    mixed, report = M.convert(state, entry)
    assert mixed[name].dtype == torch.float16 and float(mixed[name][0, 0]) == 65504.0
    assert report[name]["overflow"] == 0 and report[name]["flushed"] >= 1
    assert float(mixed[name][0, 1]) == -2.0 ** -24 and float(mixed[name][0, 2]) == 0.0
    assert mixed["layers.0.tri_mul_out.norm_in.weight"].dtype == torch.float32
    state[name][1, 0] = 65520.0  # rounds to inf
    with pytest.raises(OverflowError, match="fp16 range"):
        M.convert(state, entry)
    state[name] = state[name].double()
    with pytest.raises(TypeError):
        M.convert(state, entry)
    del state[name]
    with pytest.raises(KeyError):
        M.convert(state, entry)


def test_round_trip_binds_kernel_weights(tmp_path):
    src = small_trunk(seed=1)
    entry = M.manifest_entry(src)
    path = str(tmp_path / "trunk_mixed.safetensors")
    M.save_mixed(path, src.state_dict(), entry)
    dst = M.load_mixed(small_trunk(seed=2), path)
    sd_src, half = src.state_dict(), set(entry["params"])
    for k, v in dst.state_dict().items():
        if k in half:
            assert v.dtype == torch.float16 and torch.equal(v, sd_src[k].to(torch.float16)), k
        else:
            assert v.dtype == torch.float32 and torch.equal(v, sd_src[k]), k
    tm = dst.layers[0].tri_mul_out
    assert tm.p_in.weight.untyped_storage().data_ptr() == tm.g_in.weight.untyped_storage().data_ptr()
    old = K.PRECISION
    K.set_precision("f16")
    try:
        w_pg, w_po, _ = tm.prepare()
        assert w_pg.data_ptr() == tm.p_in.weight.data_ptr()
        assert w_pg.data_ptr() + tm.p_in.weight.numel() * 2 == tm.g_in.weight.data_ptr()
        assert w_po.data_ptr() == tm.p_out.weight.data_ptr()  # one source: the parameter itself
        assert tm.prepare()[0] is w_pg
        ta = dst.layers[1].tri_att_end
        assert ta.prepare()[0].data_ptr() == ta.mha.linear_q.weight.data_ptr()
        # the s track's attention projections stay fp32 parameters and fp32 kernel weights
        at = dst.layers[0].attention
        assert at.proj_q.weight.dtype == torch.float32 and at.prepare()[0].dtype == torch.float32
    finally:
        K.set_precision(old)


def test_load_rejects_stale_or_foreign_files(tmp_path):
    from safetensors.torch import save_file

    src = small_trunk()
    entry = M.manifest_entry(src)
    path = str(tmp_path / "m.safetensors")
    M.save_mixed(path, src.state_dict(), entry)
    stale = {**entry, "groups": entry["groups"][1:]}
    with pytest.raises(ValueError, match="convert the checkpoint again"):
        M.load_mixed(small_trunk(), path, stale)
    plain = str(tmp_path / "plain.safetensors")
    save_file({k: v.contiguous() for k, v in src.state_dict().items()}, plain)
    with pytest.raises(ValueError, match="not a mixed checkpoint"):
        M.load_mixed(small_trunk(), plain, entry)
    other = small_trunk(blocks=1)
    one = str(tmp_path / "one.safetensors")
    M.save_mixed(one, other.state_dict(), M.manifest_entry(other))
    with pytest.raises(ValueError, match="absent from the file"):
        M.load_mixed(small_trunk(), one, M.manifest_entry(other))


def test_reference_format_file_loads_into_a_sub_model(ref_manifest, tmp_path):
    """A whole-checkpoint file converted with the reference's manifest entry (its cache names, its owners, other
    stacks' tensors beside the trunk's) loads into a PairformerModule by prefix, and its groups are laid out as this
    library's kernel weights (matched by their sources)."""
    blocks, pre = 2, "pairformer_module."
    ref = ref_manifest["pairformer_layer"]
    groups, params = [], []
    for i in range(blocks):
        lp = f"{pre}layers.{i}"
        groups += [{**g, "owner": f"{lp}.{g['owner']}" if g["owner"] else lp} for g in ref["groups"]]
        params += [f"{lp}.{p}" for p in ref["params"]]
    foreign = "msa_module.layers.0.outer_product_mean.proj_o.weight"
    groups.append({"cache": "_w16", "owner": "msa_module.layers.0.outer_product_mean.proj_o", "shape": [128, 1024],
                   "srcs": ["weight"], "storable": True})
    params.append(foreign)
    entry = {"groups": sorted(groups, key=lambda g: (g["owner"], g["cache"])), "params": sorted(params)}

    src = PairformerModule(384, 128, blocks, 16)
    load_module(src, synthetic_state(src, 5, std=0.05))
    state = {pre + k: v for k, v in src.state_dict().items()}
    state[foreign] = torch.tensor(np.random.default_rng(0).standard_normal((128, 1024)) * 0.02, dtype=torch.float32)
    path = str(tmp_path / "boltz2_conf_mixed.safetensors")
    M.save_mixed(path, state, entry)

    dst = M.load_mixed(PairformerModule(384, 128, blocks, 16), path, entry, prefix=pre)
    half = set(M.restrict(entry, pre)["params"])
    assert len(half) == 27 * blocks
    sd = src.state_dict()
    for k, v in dst.state_dict().items():
        want = sd[k].to(torch.float16) if k in half else sd[k]
        assert v.dtype == want.dtype and torch.equal(v, want), k
    old = K.PRECISION
    K.set_precision("f16")
    try:
        for layer in dst.layers:
            for mod, first in ((layer.tri_mul_in, layer.tri_mul_in.p_in.weight),
                               (layer.tri_att_start, layer.tri_att_start.mha.linear_q.weight),
                               (layer.transition_z, layer.transition_z.fc1.weight),
                               (layer.transition_s, layer.transition_s.fc1.weight)):
                assert mod.prepare()[0].data_ptr() == first.data_ptr(), type(mod).__name__
    finally:
        K.set_precision(old)


class _Overlapping(torch.nn.Module):
    """Three declared fp16 groups; the first two share w2."""

    def __init__(self):
        super().__init__()
        for i in range(1, 6):
            self.register_parameter(f"w{i}", torch.nn.Parameter(torch.full((2, 3), float(i), dtype=torch.float16),
                                                                requires_grad=False))

    def kernel_weights(self):
        return (K.KernelWeight("a", ("w1", "w2")), K.KernelWeight("b", ("w2", "w3")), K.KernelWeight("c", ("w4", "w5")))


def test_bind_keeps_shared_sources_apart():
    """A parameter that two laid-out groups would share keeps its own buffer (views for one group would be wrong for
    the other); a group with sources of its own is still laid out, and groups of other models are skipped."""
    m = _Overlapping()
    entry = M.manifest_entry(m)
    entry["groups"].append({"owner": "elsewhere", "cache": "x", "srcs": ["w1", "w2"], "shape": [4, 3],
                            "storable": True})
    before = {n: p.data_ptr() for n, p in m.named_parameters()}
    assert M.bind_groups(m, entry) == 1
    for n in ("w1", "w2", "w3"):
        assert m.get_parameter(n).data_ptr() == before[n], n
    assert m.w4.data_ptr() + 12 == m.w5.data_ptr() and m.w4.untyped_storage().data_ptr() == m.w5.untyped_storage().data_ptr()
    old = K.PRECISION
    K.set_precision("f16")
    try:
        c = K.kernel_weight(m, "c")
        assert c.data_ptr() == m.w4.data_ptr() and torch.equal(c, torch.cat([m.w4, m.w5]))
        assert torch.equal(K.kernel_weight(m, "b"), torch.cat([m.w2, m.w3]))
    finally:
        K.set_precision(old)
