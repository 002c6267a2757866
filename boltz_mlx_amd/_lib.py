"""ctypes binding of libbzpf.so (the C ABI declared in include/bzpf.h).

The library is built in-tree by ``boltz_mlx_amd/build.py`` (``__graft_entry__.build()``). There is no fallback:
importing the compute path without the library, or calling it without a ROCm device, raises.
"""

from __future__ import annotations

import ctypes as C
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libbzpf.so")

F32, F16 = 0, 1

vp, i32, i64, f32 = C.c_void_p, C.c_int, C.c_int64, C.c_float

# name -> argtypes (restype is int unless listed in _RESTYPES)
SIGNATURES = {
    "bzpf_version": [],
    "bzpf_last_error": [],
    "bzpf_row_pitch": [i64],
    "bzpf_layernorm": [vp, i32, vp, vp, f32, vp, i32, i64, i32, vp],
    "bzpf_add_ln": [vp, vp, i32, f32, i32, vp, vp, f32, vp, i32, i32, i64, i32, vp],
    "bzpf_count_nonfinite": [vp, i32, i64, vp, vp],
    "bzpf_linear_gated": [vp, vp, vp, vp, i64, i64, vp, i32, i64, i32, i32, vp],
    "bzpf_swiglu3": [vp, vp, i32, i64, i32, vp],
    "bzpf_adaln": [vp, vp, vp, i64, i64, f32, vp, i32, i64, i32, vp],
    "bzpf_trimul_proj": [vp, vp, vp, f32, i32, vp, i32, i64, i64, i32, vp],
    "bzpf_trimul_contract": [vp, vp, i32, i64, i64, i32, i64, vp],
    "bzpf_trimul_tail": [vp, vp, vp, f32, vp, vp, vp, vp, i32, vp, vp, f32, vp, i32, i64, i64, i32, vp],
    "bzpf_triattn_proj": [vp, vp, i32, f32, f32, vp, vp, vp, i32, i64, i64, i32, i32, i32, vp],
    "bzpf_triattn_core": [vp, vp, vp, vp, i64, i64, f32, vp, i32, i64, i64, i32, i32, i32, vp],
    "bzpf_linear_resid_ln": [vp, vp, i32, vp, i32, vp, vp, f32, vp, i32, i64, i32, vp],
    "bzpf_transition": [vp, vp, vp, vp, i32, vp, vp, f32, vp, i32, i64, i32, i32, vp],
    "bzpf_transition_pb": [vp, vp, vp, vp, i32, vp, vp, f32, vp, vp, vp, vp, f32, vp, i32, i32, i64, i32, i32, vp],
    "bzpf_attn_out_transition": [vp, vp, i32, vp, vp, f32, vp, vp, vp, vp, vp, f32, vp, vp, vp, vp, f32, vp, i32, i32,
                                 i64, i32, i32, vp],
    "bzpf_linear": [vp, vp, vp, vp, i32, i32, i64, i32, i32, i32, vp],
    "bzpf_linear_residual": [vp, vp, vp, vp, i64, vp, i32, i64, i32, i32, vp],
    "bzpf_swiglu": [vp, vp, i32, i64, i32, vp],
    "bzpf_seq_attention": [vp, vp, vp, vp, i64, vp, vp, f32, vp, i64, i32, i32, i64, i32, i32, vp],
    "bzpf_linear_swiglu3": [vp, vp, vp, i64, i32, i32, vp],
    "bzpf_linear_swiglu": [vp, vp, vp, i64, i32, i32, vp],
    "bzpf_trimul_pack": [vp, vp, f32, i32, vp, i32, i64, i64, i32, vp],
    "bzpf_channels_to_rows": [vp, i32, vp, i32, i64, i64, i32, vp],
    "bzpf_triattn_pack": [vp, i32, f32, f32, vp, vp, vp, i32, i64, i64, i32, i32, vp],
    "bzpf_opm_split": [vp, i64, vp, vp, i32, i32, vp],
    "bzpf_opm_ln_split": [vp, vp, vp, f32, vp, vp, vp, i32, i32, vp],
    "bzpf_opm_outer": [vp, vp, vp, i32, i32, i32, i32, i32, vp],
    "bzpf_pwa_softmax": [vp, vp, f32, vp, i32, i64, i32, vp],
    "bzpf_transition64_f16": [vp, vp, vp, f32, vp, vp, i64, i32, vp],
    "bzpf_ln_linear_f32": [vp, vp, vp, f32, vp, vp, i64, i32, i32, vp],
    "bzpf_pwa_wsplit_bytes": [i32, i64, i32],
    "bzpf_pwa_wsplit": [vp, i64, vp, i32, i32, vp],
    "bzpf_pwa_avg": [vp, i64, vp, i64, vp, i64, vp, i64, i32, i32, i32, vp],
    "bzpf_seq_attention_batched": [vp, vp, vp, vp, i64, i64, vp, i64, i32, vp, i64, f32, vp, i64, i64, i32, i32, i32,
                                   i64, i32, i32, vp],
    "bzpf_pair_bias": [vp, vp, vp, f32, vp, vp, i32, i64, i32, i32, vp],
}
_RESTYPES = {"bzpf_version": C.c_char_p, "bzpf_last_error": C.c_char_p, "bzpf_row_pitch": i64,
             "bzpf_pwa_wsplit_bytes": i64}

_lib = None


class BzpfError(RuntimeError):
    pass


def load(path: str | None = None):
    """Load (once) and return the library with argtypes set (default path: LIB_PATH as it is at the first call).
    Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    path = path or LIB_PATH
    # torch first: its HIP runtime (torch/lib/libamdhip64.so, soname libamdhip64.so.7) must be the one mapped
    # when the library resolves libamdhip64.so.7, so that the process holds a single runtime instance.
    import torch  # noqa: F401

    if not os.path.exists(path):
        raise BzpfError(f"{path} not found: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                        "(or python boltz_mlx_amd/build.py)")
    lib = C.CDLL(path)
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _RESTYPES.get(name, i32)
    _lib = lib
    return lib


def call(name: str, *args) -> None:
    """Call an entry point; a non-zero status raises BzpfError with the library's message."""
    rc = getattr(load(), name)(*args)
    if rc != 0:
        msg = load().bzpf_last_error().decode()
        raise BzpfError(f"{name} failed ({rc}): {msg}")
