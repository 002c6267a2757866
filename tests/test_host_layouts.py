"""Host-side layout helpers of the fused kernels (CPU): the weight-row regrouping of the SwiGLU GEMMs, the pair-mask
scope, and the kernels' own index maps and 32-bit buffer ranges built on the host."""

from __future__ import annotations

import pytest
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


def test_pair_mask_scope_extent_and_transpose():
    """key_extent / mask_transposed: nothing is derived outside a scope (extent 0 = every key, a fresh transposed
    copy per call); inside, the extent is 1 + the last live token (columns for outgoing, rows for incoming, checked
    by brute force on an asymmetric mask), each value is made once per mask, and an in-place change of the mask
    (a new version) is seen."""
    from boltz_mlx_amd import kernels as K

    N = 70
    g = torch.Generator().manual_seed(5)
    m = (torch.rand((N, N), generator=g) > 0.4).float()
    m[:, 61:] = 0  # columns past 60 dead (outgoing extent 61)
    m[55:, :] = 0  # rows past 54 dead (incoming extent 55)
    brute_out = 1 + max(k for k in range(N) if any(m[i, k] != 0 for i in range(N)))
    brute_in = 1 + max(k for k in range(N) if any(m[k, i] != 0 for i in range(N)))
    assert (brute_out, brute_in) == (61, 55)
    assert K.key_extent(m, N, False) == 0 and K.key_extent(m, N, True) == 0
    t0 = K.mask_transposed(m, N)
    assert torch.equal(t0, m.t()) and t0.is_contiguous() and K.mask_transposed(m, N) is not t0
    with K.pair_mask_scope():
        assert K.key_extent(m, N, False) == brute_out and K.key_extent(m, N, True) == brute_in
        t1 = K.mask_transposed(m, N)
        assert torch.equal(t1, m.t()) and K.mask_transposed(m.view(N, N), N) is t1  # a view of the same storage
        m[:, 69] = 1  # in place: a new version
        assert K.key_extent(m, N, False) == N and K.key_extent(m, N, True) == N
        assert torch.equal(K.mask_transposed(m, N), m.t())
        with K.pair_mask_scope():  # nested scopes start empty and restore the outer one
            assert K.key_extent(torch.zeros(N, N), N, False) == N
        assert K.mask_transposed(m, N) is K.mask_transposed(m, N)
    assert K.key_extent(m, N, False) == 0


# ---------------------------------------------------------------- kernel index maps and buffer ranges (host build)

@pytest.fixture(scope="module")
def layout_lib(tmp_path_factory):
    """tests/layout_check.cpp built with g++ against boltz_mlx_amd/csrc/bzpf_layout.h (the header the kernels and
    their launchers use; it needs no HIP)."""
    import ctypes
    import os
    import subprocess

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    out = str(tmp_path_factory.mktemp("layout") / "layout_check.so")
    subprocess.run(["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-I", os.path.join(root, "boltz_mlx_amd", "csrc"),
                    os.path.join(root, "tests", "layout_check.cpp"), "-o", out], check=True)
    lib = ctypes.CDLL(out)
    lib.lc_check.argtypes = [ctypes.c_char_p, ctypes.c_int]
    lib.lc_tb_offsets.argtypes = [ctypes.c_int64, ctypes.c_int, ctypes.c_void_p]
    return lib


def test_kernel_layouts_and_buffer_ranges(layout_lib):
    """The fragment-ordered triangle bias is a bijection onto its buffer with the core's 1 KB load runs; the
    contraction's LDS swizzle permutes each row and makes the fragment reads conflict-free; every buffer resource of
    the attention core, the contraction and the fp16 sequence attention keeps its extent and largest offset below
    2^31 at the launchers' size limits, which refuse the first size past them."""
    import ctypes

    buf = ctypes.create_string_buffer(1 << 17)
    failures = layout_lib.lc_check(buf, len(buf))
    report = buf.value.decode()
    print(report)
    assert failures == 0, [line for line in report.splitlines() if line.startswith("FAIL")]
    assert report.count("ok") > 100


@pytest.mark.parametrize("N,H", [(1, 1), (37, 4), (130, 3), (257, 4)])
def test_tb_offset_matches_the_host_wrapper(layout_lib, N, H):
    """The kernels' tb_offset (bzpf_layout.h) and kernels.tri_bias_offsets (the host's map of a dense bias into the
    layout, used by the tests and the layout kernels' callers) agree element for element."""
    import numpy as np

    from boltz_mlx_amd import kernels as K

    got = np.empty((H, N, N), dtype=np.int64)
    layout_lib.lc_tb_offsets(N, H, got.ctypes.data)
    assert np.array_equal(got, K.tri_bias_offsets(N, H))
