"""Builds libbzpf.so (the gfx950 HIP kernels behind the C ABI in include/bzpf.h) in-tree with hipcc.

Each .hip source under csrc/ is compiled to an object in parallel, then linked into boltz_mlx_amd/libbzpf.so.
Packed-FP32 instruction selection is disabled for the device code.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libbzpf.so")
ARCH = os.environ.get("BZPF_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: the kernels read every accumulator back with VALU ops (softmax, epilogues),
    # which the AGPR form would route through v_accvgpr moves
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-munsafe-fp-atomics", f"-I{INCLUDE}", f"-I{CSRC}",
]


def torch_lib_dir() -> str:
    import importlib.util

    spec = importlib.util.find_spec("torch")
    if spec is None or not spec.submodule_search_locations:
        raise RuntimeError("torch (ROCm build) is required to link against its HIP runtime")
    d = os.path.join(list(spec.submodule_search_locations)[0], "lib")
    if not os.path.exists(os.path.join(d, "libamdhip64.so")):
        raise RuntimeError(f"{d}/libamdhip64.so not found (torch must be a ROCm build)")
    return d


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


# Per-source additions. The fp16 attention core is VALU-bound; without NaN semantics its fmaxf reductions over MFMA
# results need no canonicalising v_max_f32 per logit (its inputs are finite or -inf by construction).
FILE_FLAGS = {"bzpf_triattn_mfma.hip": ["-fno-honor-nans"]}


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *CFLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in (r.stderr or "").splitlines() if noise not in line)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {os.path.basename(src)}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    # Link against the HIP runtime that torch loads (torch/lib/libamdhip64.so), so that the library and torch
    # share one runtime instance (and one device context) in the process.
    tlib = torch_lib_dir()
    r = subprocess.run(["g++", "-shared", "-fPIC", *objs, "-o", tmp, f"-L{tlib}", f"-Wl,-rpath,{tlib}",
                        "-l:libamdhip64.so"], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    return LIB


if __name__ == "__main__":
    build()
