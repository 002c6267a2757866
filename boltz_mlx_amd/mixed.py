"""Mixed fp16 / fp32 checkpoints for f16 mode.

A mixed checkpoint holds every parameter of the model under its checkpoint name. The parameters that f16 mode reads
only as fp16 kernel weights are stored in fp16 (the round-to-nearest-even value of the fp32 one); all others stay
fp32. Loading one keeps those parameters in fp16 on the device and lays each multi-parameter kernel weight out once,
with its source parameters as views into it, so the model never holds an fp32 copy of an fp16 GEMM weight and the
first f16 call builds no second copy.

Which parameters are fp16 is read off the modules' declarations: a module that feeds a kernel lists its weight
matrices in ``kernel_weights()`` (``kernels.KernelWeight``: cache name, source parameter paths, ``half``), and its
``prepare()`` reads exactly those through ``kernels.kernel_weight``. The ``half`` declarations of a model, with their
owners, make the manifest entry:
    {"groups": [{"owner", "cache", "srcs", "shape", "storable"}, ...], "params": [every name of every source]}.

The file contract is shared with the reference's converter on purpose (boltz_mlx/mixed.py:49-60, 143-153, 216-287),
so that files converted on either side load on the other: the format tag, the safetensors metadata keys ``format``
and ``manifest_sha``, the entry hash (sha256 of the entry's sorted-key JSON, first 16 hex digits) and the fields of a
group record. A file the reference converted is loaded with the reference's manifest entry (``load_mixed(...,
entry=its entry, prefix=...)`` for a sub-model of the whole Boltz-2 checkpoint); its groups are matched to this
library's kernel weights by their source parameters, since the two libraries name their caches differently.
"""

from __future__ import annotations

import hashlib
import json

import torch

from boltz_mlx_amd import kernels as K

FORMAT = "boltz-mlx-mixed-v1"
META_FORMAT, META_SHA = "format", "manifest_sha"
# fp16's largest finite value is 65504; under round to nearest even everything from 65520 up becomes inf
HALF_OVERFLOW = 65520.0


def entry_sha(entry: dict) -> str:
    """The manifest hash written into a mixed file (a different hash at load time means a stale file)."""
    blob = json.dumps(entry, sort_keys=True).encode()
    return hashlib.sha256(blob).hexdigest()[:16]


def _join(path: str, name: str) -> str:
    return f"{path}.{name}" if path else name


def _names_by_tensor(model: torch.nn.Module) -> dict:
    """id(parameter) -> all of its qualified names (a module registered under two names gives a tensor two)."""
    names: dict = {}
    for name, p in model.named_parameters(remove_duplicate=False):
        names.setdefault(id(p), []).append(name)
    return names


def half_groups(model: torch.nn.Module) -> list:
    """Group records of every kernel weight the model's modules declare as fp16-in-f16-mode, sorted by (owner,
    cache). Each source is a parameter of its owner, so every record is storable."""
    records = []
    for path, mod in model.named_modules():
        for kw in K.declared_weights(mod).values():
            if not kw.half:
                continue
            params = [mod.get_parameter(src) for src in kw.srcs]
            rows = sum(int(p.shape[0]) for p in params)
            records.append({"owner": path, "cache": kw.name, "srcs": list(kw.srcs),
                            "shape": [rows, *(int(d) for d in params[0].shape[1:])], "storable": True})
    records.sort(key=lambda r: (r["owner"], r["cache"]))
    return records


def manifest_entry(model: torch.nn.Module) -> dict:
    """This library's manifest entry for `model`: its fp16 groups and the sorted names (aliases included) of their
    source parameters."""
    groups = half_groups(model)
    aliases = _names_by_tensor(model)
    params = set()
    for g in groups:
        owner = model.get_submodule(g["owner"])
        for src in g["srcs"]:
            params.update(aliases[id(owner.get_parameter(src))])
    return {"groups": groups, "params": sorted(params)}


def restrict(entry: dict, prefix: str) -> dict:
    """The part of a manifest entry that lies under `prefix` (a sub-model's checkpoint prefix such as
    "pairformer_module."), with the prefix removed from owners and parameter names."""
    if not prefix:
        return entry
    root = prefix[:-1] if prefix.endswith(".") else prefix
    groups = []
    for g in entry["groups"]:
        owner = g["owner"]
        if owner == root:
            groups.append({**g, "owner": ""})
        elif owner.startswith(prefix):
            groups.append({**g, "owner": owner[len(prefix):]})
    params = [p[len(prefix):] for p in entry["params"] if p.startswith(prefix)]
    return {"groups": groups, "params": params}


def convert(state: dict, entry: dict) -> tuple:
    """fp32 state dict -> (mixed state dict, {name: range report} for the fp16 tensors).

    Raises KeyError when the state lacks a parameter the entry lists, TypeError when such a parameter is not fp32,
    and OverflowError when any of them holds a finite value that fp16 cannot represent."""
    half = set(entry["params"])
    absent = sorted(half.difference(state))
    if absent:
        raise KeyError(f"{len(absent)} fp16 parameters of the manifest are not in the state dict, e.g. {absent[:3]}")
    mixed, report, too_large = {}, {}, []
    for name, value in state.items():
        t = value.detach().cpu() if isinstance(value, torch.Tensor) else torch.as_tensor(value)
        if name not in half:
            mixed[name] = t
            continue
        if t.dtype != torch.float32:
            raise TypeError(f"{name}: the fp16 conversion takes fp32 values, got {t.dtype}")
        h = t.to(torch.float16)
        mag = t.abs()
        rep = {"n": t.numel(), "max_abs": float(mag.max()) if t.numel() else 0.0,
               "overflow": int((torch.isfinite(t) & (mag >= HALF_OVERFLOW)).sum()),
               "flushed": int(((t != 0) & (h == 0)).sum())}
        report[name] = rep
        if rep["overflow"]:
            too_large.append(f"{name} ({rep['overflow']} values)")
        mixed[name] = h
    if too_large:
        raise OverflowError(f"values beyond the fp16 range (|w| >= {HALF_OVERFLOW:g}) in {len(too_large)} tensors: "
                            + ", ".join(too_large[:5]))
    return mixed, report


def save_mixed(path: str, state: dict, entry: dict) -> dict:
    """Convert an fp32 state dict and write it as a mixed safetensors file; returns the range report."""
    from safetensors.torch import save_file

    mixed, report = convert(state, entry)
    save_file({k: v.contiguous() for k, v in mixed.items()}, path,
              metadata={META_FORMAT: FORMAT, META_SHA: entry_sha(entry)})
    return report


def _places(model: torch.nn.Module) -> dict:
    """id(parameter) -> every (module, attribute) it is registered at."""
    places: dict = {}
    for path, mod in model.named_modules(remove_duplicate=False):
        for leaf, p in mod.named_parameters(recurse=False):
            places.setdefault(id(p), []).append((mod, leaf))
    return places


def _rebind(places: dict, old: torch.Tensor, new: torch.nn.Parameter) -> None:
    for mod, leaf in places.get(id(old), []):
        setattr(mod, leaf, new)


def bind_groups(model: torch.nn.Module, entry: dict) -> int:
    """Lay out every multi-parameter fp16 kernel weight of `model` that `entry` also groups (same source parameters,
    whatever the entry calls the cache) as one buffer: the buffer becomes the owner's cached kernel weight and the
    source parameters become views into it. A source that two such groups share keeps its own buffer (the cache then
    concatenates at first use). Returns the number of buffers laid out."""
    declared = {}  # tuple(id of each source) -> (owner module, kernel weight)
    for path, mod in model.named_modules():
        for kw in K.declared_weights(mod).values():
            if kw.half and len(kw.srcs) > 1:
                declared[tuple(id(mod.get_parameter(s)) for s in kw.srcs)] = (mod, kw)
    matched = []
    for g in entry["groups"]:
        if not g.get("storable") or len(g["srcs"]) < 2:
            continue
        try:
            ids = tuple(id(model.get_parameter(_join(g["owner"], s))) for s in g["srcs"])
        except AttributeError:  # a module of another model (e.g. outside this sub-model)
            continue
        if ids in declared and declared[ids] not in [m for m, _ in matched]:
            matched.append((declared[ids], ids))
    uses: dict = {}
    for _, ids in matched:
        for i in ids:
            uses[i] = uses.get(i, 0) + 1
    places = _places(model)
    laid = 0
    with torch.no_grad():
        for (mod, kw), ids in matched:
            params = [mod.get_parameter(s) for s in kw.srcs]
            if any(uses[i] > 1 for i in ids) or any(p.dtype != torch.float16 for p in params):
                continue
            buf = torch.empty((sum(p.shape[0] for p in params), *params[0].shape[1:]), dtype=torch.float16,
                              device=params[0].device)
            row, views = 0, []
            for p in params:
                n = p.shape[0]
                buf[row:row + n].copy_(p)
                view = torch.nn.Parameter(buf[row:row + n], requires_grad=False)
                _rebind(places, p, view)
                views.append(view)
                row += n
            K.wcache_seed(mod, kw.name, views, buf)
            laid += 1
    return laid


def load_mixed(model: torch.nn.Module, path: str, entry: dict | None = None, prefix: str = "",
               device=None) -> torch.nn.Module:
    """Load a mixed checkpoint into `model` and lay out its fp16 kernel weights (bind_groups).

    entry: the manifest entry the file was converted with: this library's manifest_entry(model) (the default), or
    another converter's entry for the whole checkpoint. prefix: the checkpoint prefix of `model` inside the file
    ("" when the file holds this model alone); tensors outside it are not read. The file's format tag and manifest
    hash must match, and its tensors under the prefix must be exactly the model's parameters and buffers, with the
    same shapes; the entry's fp16 parameters must be fp16 in the file."""
    from safetensors import safe_open

    entry = manifest_entry(model) if entry is None else entry
    want = entry_sha(entry)
    with safe_open(path, framework="pt") as f:
        meta = f.metadata() or {}
        if meta.get(META_FORMAT) != FORMAT:
            raise ValueError(f"{path}: not a mixed checkpoint (format tag {meta.get(META_FORMAT)!r}, expected "
                             f"{FORMAT!r})")
        if meta.get(META_SHA) != want:
            raise ValueError(f"{path}: converted with manifest {meta.get(META_SHA)!r}, but the given entry hashes to "
                             f"{want!r}; convert the checkpoint again")
        state = {k[len(prefix):]: f.get_tensor(k) for k in f.keys() if k.startswith(prefix)}
    if device is not None:
        model.to(device)
    own = dict(model.named_parameters(remove_duplicate=False))
    own.update(model.named_buffers(remove_duplicate=False))
    lacking, extra = sorted(set(own) - set(state)), sorted(set(state) - set(own))
    if lacking or extra:
        raise ValueError(f"{path}: tensors do not match the model (absent from the file: {lacking[:8]}; not in the "
                         f"model: {extra[:8]})")
    half = set(restrict(entry, prefix)["params"])
    places = _places(model)
    done: dict = {}  # id(old parameter) -> its replacement (a tensor with two names is replaced once)
    with torch.no_grad():
        for name, value in state.items():
            cur = own[name]
            if tuple(value.shape) != tuple(cur.shape):
                raise ValueError(f"{path}: {name} has shape {tuple(value.shape)}, the model {tuple(cur.shape)}")
            if name in half:
                if value.dtype != torch.float16:
                    raise ValueError(f"{path}: {name} is an fp16 parameter of the manifest but the file holds "
                                     f"{value.dtype}")
                if id(cur) not in done:
                    done[id(cur)] = torch.nn.Parameter(value.to(cur.device), requires_grad=False)
                    _rebind(places, cur, done[id(cur)])
            elif id(cur) not in done:
                cur.copy_(value.to(device=cur.device, dtype=cur.dtype))
    bind_groups(model, restrict(entry, prefix))
    return model
