"""Weight I/O for the bzpf modules: converted checkpoints and seeded synthetic weights.

The modules use the reference's PyTorch qualified names (boltz_mlx/weights.py:27-36 loads converted safetensors
under those names with a strict name check), so a converted Boltz-2 checkpoint loads with ``strict=True``.
"""

from __future__ import annotations

import numpy as np
import torch


def subtree(state: dict, prefix: str) -> dict:
    """Entries of `state` under `prefix.` with the prefix removed (boltz_mlx/weights.py:20-22)."""
    p = prefix.rstrip(".") + "."
    return {k[len(p):]: v for k, v in state.items() if k.startswith(p)}


def load_module(module: torch.nn.Module, state: dict, prefix: str = "", strict: bool = True) -> torch.nn.Module:
    """Load `state` (names relative to `prefix`; any tensor / array values) into `module` with a strict name and
    shape check (boltz_mlx/weights.py:27-36)."""
    w = subtree(state, prefix) if prefix else dict(state)
    ours = module.state_dict()
    if strict:
        missing, extra = set(ours) - set(w), set(w) - set(ours)
        if missing or extra:
            raise ValueError(f"{prefix or 'module'}: missing={sorted(missing)[:10]} unexpected={sorted(extra)[:10]}")
    conv = {}
    for k, v in w.items():
        t = torch.as_tensor(np.asarray(v)) if not isinstance(v, torch.Tensor) else v
        if k in ours and tuple(t.shape) != tuple(ours[k].shape):
            raise ValueError(f"{k}: shape {tuple(t.shape)} != {tuple(ours[k].shape)}")
        conv[k] = t.to(ours[k].dtype) if k in ours else t
    module.load_state_dict(conv, strict=strict)
    return module


def load_safetensors(module: torch.nn.Module, path: str, prefix: str = "", strict: bool = True) -> torch.nn.Module:
    """Load a converted safetensors checkpoint (PyTorch names) into `module` (safe loader: no pickle)."""
    from safetensors.numpy import load_file

    return load_module(module, load_file(path), prefix, strict)


def synthetic_state(module: torch.nn.Module, seed: int, std: float = 0.02) -> dict:
    """Seeded random-init weights in sorted-name order: every Linear weight and bias ~ N(0, std), LayerNorm weight
    1 and bias 0 (numpy default_rng; the synthetic-weight convention of the benchmark configs)."""
    rng = np.random.default_rng(seed)
    out = {}
    ln_params = set()
    for name, mod in module.named_modules():
        if isinstance(mod, torch.nn.LayerNorm):
            ln_params.update({f"{name}.weight" if name else "weight", f"{name}.bias" if name else "bias"})
    for name, t in sorted(module.state_dict().items()):
        if name in ln_params:
            v = np.ones(t.shape) if name.endswith("weight") else np.zeros(t.shape)
        else:
            v = std * rng.standard_normal(t.shape)
        out[name] = v.astype(np.float32)
    return out
