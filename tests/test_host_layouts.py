"""Host-side layout helpers of the fused kernels (CPU): the weight-row regrouping of the SwiGLU GEMMs."""

from __future__ import annotations

import torch


def test_group_swiglu_rows():
    """Block q of the grouped matrix is [W_0 rows 32q..32q+31; W_1 same (; W_2 same)], every source row once."""
    from boltz_mlx_amd import kernels as K

    H, Kd = 96, 5
    ws = [torch.arange(H * Kd, dtype=torch.float32).view(H, Kd) + 1000 * p for p in range(3)]
    g3 = K.group_swiglu3_rows(*ws)
    assert g3.shape == (3 * H, Kd)
    for q in range(H // 32):
        for p in range(3):
            assert torch.equal(g3[96 * q + 32 * p:96 * q + 32 * (p + 1)], ws[p][32 * q:32 * (q + 1)])
    g2 = K.group_swiglu_rows(ws[0], ws[1])
    for q in range(H // 32):
        assert torch.equal(g2[64 * q:64 * q + 32], ws[0][32 * q:32 * (q + 1)])
        assert torch.equal(g2[64 * q + 32:64 * (q + 1)], ws[1][32 * q:32 * (q + 1)])
    assert torch.equal(torch.sort(g3.flatten())[0], torch.sort(torch.cat(ws).flatten())[0])
