"""Mixed fp16 / fp32 checkpoints for f16 mode: fp16 GEMM weights stored once, checked against a manifest.

A mixed checkpoint holds, under the PyTorch names of the fp32 checkpoint, fp16 copies of exactly the parameters that
f16 mode consumes only through fp16 kernel weights, and the fp32 values of everything else; its safetensors metadata
carries ``format`` and ``manifest_sha``. Loading checks both (a stale or partially converted file raises), keeps the
fp16 tensors in fp16, builds each multi-parameter kernel weight once and makes its source parameters views into it,
so no fp32 copy of a GEMM weight exists and no second fp16 copy is made at first use.

Which parameters are fp16 is derived from the code: every kernel weight is built by ``kernels.wcache(owner, name,
*params)``; with ``kernels.WCACHE_TRACE`` set, each module's ``prepare()`` reports (owner, cache name, sources) and
sources that are parameters (by identity) map to their qualified names. A group whose sources are all parameters is
"storable". The manifest entry is {"groups": [...], "params": [...]}, hashed by ``entry_sha``.

Kept alike with the reference on purpose (boltz_mlx/mixed.py:49-60, 216-287), so that files its converter wrote for
the same parameter set validate here: the format string, the entry hash (sha256 of the sorted-key JSON, 16 hex
digits), the metadata keys, the overflow check of the conversion and the prefuse of multi-parameter groups.
"""

from __future__ import annotations

import hashlib
import json

import numpy as np
import torch

from boltz_mlx_amd import kernels as K

FORMAT = "boltz-mlx-mixed-v1"
FP16_MAX = 65504.0


def entry_sha(entry: dict) -> str:
    """Hash of a manifest entry (stored in the mixed file; a mismatch at load means a stale file)."""
    return hashlib.sha256(json.dumps(entry, sort_keys=True).encode()).hexdigest()[:16]


def _param_names(model: torch.nn.Module) -> dict:
    """id(parameter) -> its qualified names (a module registered twice gives two names for one tensor)."""
    out: dict = {}
    for n, p in model.named_parameters(remove_duplicate=False):
        out.setdefault(id(p), []).append(n)
    return out


def trace_groups(model: torch.nn.Module) -> list:
    """The fp16 kernel-weight groups of `model`, from every submodule's argument-free prepare() run in f16 mode (on
    any device: the weight caches are torch casts and concatenations)."""
    paths = {id(m): p for p, m in model.named_modules()}
    names = _param_names(model)
    groups: dict = {}

    def hook(owner, name, params, dtype):
        if dtype != torch.float16:
            return
        op = paths.get(id(owner))
        if op is None:
            raise RuntimeError(f"kernel weight {name!r}: owner {type(owner).__name__} is not a submodule")
        pre = op + "." if op else ""
        srcs = []
        for t in params:
            ns = [n for n in names.get(id(t), []) if n.startswith(pre)]
            srcs.append(ns[0][len(pre):] if ns else None)
        groups[(op, name)] = {"owner": op, "cache": name, "srcs": srcs, "storable": all(s is not None for s in srcs),
                              "shape": [int(sum(t.shape[0] for t in params)), *map(int, params[0].shape[1:])]}

    old_trace, old_prec = K.WCACHE_TRACE, K.PRECISION
    K.WCACHE_TRACE = hook
    K.set_precision("f16")
    try:
        with torch.no_grad():
            for m in model.modules():
                prep = getattr(type(m), "prepare", None)
                if prep is None:
                    continue
                try:
                    m.prepare()
                except TypeError:  # prepare(...) that needs arguments (per-call inputs): no weight group
                    continue
    finally:
        K.WCACHE_TRACE = old_trace
        K.set_precision(old_prec)
    return sorted(groups.values(), key=lambda g: (g["owner"], g["cache"]))


def manifest_entry(model: torch.nn.Module, groups: list | None = None) -> dict:
    """{"groups": [...], "params": [every qualified name of a storable group's sources, aliases included]}."""
    groups = trace_groups(model) if groups is None else groups
    names = _param_names(model)
    by_name = {n: ns for ns in names.values() for n in ns}
    params = set()
    for g in groups:
        if g["storable"]:
            for s in g["srcs"]:
                params.update(by_name[f"{g['owner']}.{s}" if g["owner"] else s])
    return {"groups": groups, "params": sorted(params)}


def to_mixed(state: dict, entry: dict) -> tuple:
    """fp32 state dict -> (mixed state dict, per-tensor fp16 range stats). Raises on a missing manifest parameter, a
    non-fp32 source or any fp16 overflow."""
    params = set(entry["params"])
    missing = params - set(state)
    if missing:
        raise KeyError(f"manifest parameters missing from the checkpoint: {sorted(missing)[:5]}")
    out, stats, bad = {}, {}, {}
    for k, v in state.items():
        t = torch.as_tensor(np.asarray(v)) if not isinstance(v, torch.Tensor) else v.detach().cpu()
        if k in params:
            if t.dtype != torch.float32:
                raise TypeError(f"{k}: expected an fp32 source, got {t.dtype}")
            a = t.abs()
            h = t.to(torch.float16)
            stats[k] = {"n": t.numel(), "max_abs": float(a.max()) if t.numel() else 0.0,
                        "overflow": int((~torch.isfinite(h) & torch.isfinite(t)).sum()),
                        "flushed": int(((t != 0) & (h == 0)).sum())}
            if stats[k]["overflow"]:
                bad[k] = stats[k]["overflow"]
            out[k] = h
        else:
            out[k] = t
    if bad:
        raise OverflowError(f"fp16 overflow (|w| > {FP16_MAX}) in {len(bad)} tensors: {bad}")
    return out, stats


def save_mixed(path: str, state: dict, entry: dict) -> None:
    """Write a mixed checkpoint (to_mixed of an fp32 state) with its format and manifest hash."""
    from safetensors.torch import save_file

    mixed, _ = to_mixed(state, entry)
    save_file({k: v.contiguous() for k, v in mixed.items()}, path,
              metadata={"format": FORMAT, "manifest_sha": entry_sha(entry)})


def _resolve(model: torch.nn.Module, path: str):
    m = model
    for part in path.split(".") if path else []:
        m = getattr(m, part, None)
        if m is None:
            return None
    return m


def prefuse(model: torch.nn.Module, entry: dict) -> int:
    """After a mixed load: build each storable multi-parameter group's fp16 kernel weight once, put it in the
    module's weight cache, and make the source parameters views into it (their own buffers are freed), so the
    concatenated fp16 weight exists once. A parameter shared by two groups keeps its own buffer. Returns the number of
    groups seeded. Owners missing from the model are skipped."""
    groups = [g for g in entry["groups"] if g["storable"]]
    count: dict = {}
    for g in groups:
        for s in g["srcs"]:
            key = f"{g['owner']}.{s}"
            count[key] = count.get(key, 0) + 1
    n = 0
    with torch.no_grad():
        for g in groups:
            owner = _resolve(model, g["owner"])
            if owner is None:
                continue
            leaves = []
            for s in g["srcs"]:
                *pp, leaf = s.split(".")
                parent = _resolve(owner, ".".join(pp))
                leaves.append((parent, leaf, getattr(parent, leaf)))
            if any(t.dtype != torch.float16 for _, _, t in leaves):
                continue  # not stored in fp16 in this file: the cache casts at first use
            if len(leaves) > 1 and all(count[f"{g['owner']}.{s}"] == 1 for s in g["srcs"]):
                w = torch.cat([t.detach() for _, _, t in leaves], 0).contiguous()
                r = 0
                for parent, leaf, t in leaves:
                    setattr(parent, leaf, torch.nn.Parameter(w[r:r + t.shape[0]], requires_grad=False))
                    r += t.shape[0]
                K.wcache_seed(owner, g["cache"], [getattr(parent, leaf) for parent, leaf, _ in leaves], w)
            else:  # one source (the cache is the parameter itself) or a shared source (the cache concatenates)
                K.wcache(owner, g["cache"], *[getattr(parent, leaf) for parent, leaf, _ in leaves],
                         dtype=torch.float16)
            n += 1
    return n


def load_mixed(model: torch.nn.Module, path: str, entry: dict, device=None) -> torch.nn.Module:
    """Load a mixed checkpoint into `model` (strict names and shapes) after checking its format and manifest hash
    against `entry` (this build's manifest_entry(model), or the manifest entry the file was converted with). fp16
    tensors stay fp16 (the parameter changes dtype); the model is placed on `device`, then prefused."""
    from safetensors import safe_open

    with safe_open(path, framework="pt") as f:
        meta = f.metadata() or {}
        if meta.get("format") != FORMAT or meta.get("manifest_sha") != entry_sha(entry):
            raise ValueError(f"{path}: format {meta.get('format')!r} / manifest {meta.get('manifest_sha')!r} do not "
                             f"match this manifest ({FORMAT} / {entry_sha(entry)}); convert the checkpoint again")
        state = {k: f.get_tensor(k) for k in f.keys()}
    ours = dict(model.named_parameters(remove_duplicate=False))
    ours.update(dict(model.named_buffers()))
    missing, extra = set(ours) - set(state), set(state) - set(ours)
    if missing or extra:
        raise ValueError(f"{path}: missing={sorted(missing)[:10]} unexpected={sorted(extra)[:10]}")
    if device is not None:
        model.to(device)
    fp16 = set(entry["params"])
    replaced: dict = {}  # id(old parameter) -> its fp16 replacement (a tensor registered under two names stays one)
    with torch.no_grad():
        for k, v in state.items():
            *pp, leaf = k.split(".")
            parent = _resolve(model, ".".join(pp))
            cur = getattr(parent, leaf)
            if tuple(v.shape) != tuple(cur.shape):
                raise ValueError(f"{k}: shape {tuple(v.shape)} != {tuple(cur.shape)}")
            if k in fp16:
                if v.dtype != torch.float16:
                    raise ValueError(f"{k}: the manifest lists it as fp16, the file holds {v.dtype}")
                new = replaced.get(id(cur))
                if new is None:
                    new = replaced[id(cur)] = torch.nn.Parameter(v.to(cur.device), requires_grad=False)
                setattr(parent, leaf, new)
            elif id(cur) not in replaced:
                cur.copy_(v.to(cur.dtype))
    prefuse(model, entry)
    return model
