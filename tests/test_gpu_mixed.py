"""A trunk loaded from a mixed fp16 checkpoint computes, in f16 mode, exactly what the same weights loaded in fp32 and
cast at first use compute (the fp32 -> fp16 cast is deterministic, so the fp16 kernel operands are the same bits), and
holds its GEMM weights once, in fp16."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from boltz_mlx_amd import kernels as K
from boltz_mlx_amd import mixed as M

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _device():
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    from boltz_mlx_amd import _lib

    _lib.load()
    old = K.PRECISION
    K.set_precision("f16")
    yield
    K.set_precision(old)


def test_mixed_trunk_equals_runtime_cast(tmp_path):
    from boltz_mlx_amd.layers.pairformer import PairformerModule
    from boltz_mlx_amd.weights import load_module, synthetic_state

    N, blocks = 40, 2
    ref = PairformerModule(384, 128, blocks, 16)
    state = synthetic_state(ref, 11, std=0.05)
    load_module(ref, state)
    ref = ref.cuda()
    entry = M.manifest_entry(ref)
    path = str(tmp_path / "trunk_mixed.safetensors")
    M.save_mixed(path, {k: torch.as_tensor(v) for k, v in state.items()}, entry)
    mix = M.load_mixed(PairformerModule(384, 128, blocks, 16), path, entry, device="cuda")
    rng = np.random.default_rng(12)
    z = torch.tensor(rng.standard_normal((1, N, N, 128)), dtype=torch.float32, device="cuda")
    s = torch.tensor(rng.standard_normal((1, N, 384)), dtype=torch.float32, device="cuda")
    tok = torch.ones((1, N), device="cuda")
    tok[:, -3:] = 0
    pm = tok[:, :, None] * tok[:, None, :]
    with torch.no_grad():
        s1, z1 = ref(s, z, tok, pm)
        s2, z2 = mix(s, z, tok, pm)
    torch.cuda.synchronize()
    assert torch.equal(z1, z2) and torch.equal(s1, s2)
    # the manifest's parameters are held once, in fp16, and every other parameter in fp32
    half = set(entry["params"])
    want = sum(p.numel() * (2 if n in half else 4) for n, p in ref.named_parameters())
    assert sum(p.numel() * p.element_size() for p in mix.parameters()) == want
