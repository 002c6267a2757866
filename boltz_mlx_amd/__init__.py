"""boltz_mlx_amd — MI355X-native Pairformer pair path (bzpf).

Hand-written gfx950 HIP kernels behind a C ABI (include/bzpf.h, built into boltz_mlx_amd/libbzpf.so) and
torch.nn.Modules with the reference's call signatures and checkpoint names (boltz_mlx/layers/*.py of
jackryan225/boltz-mlx), so the path drops in for the reference's kernels*.py path.
"""

__version__ = "0.1.0"
