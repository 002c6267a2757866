"""Writes fp16_manifest_layers.json: the per-layer part of the reference's committed fp16 manifest
(boltz_mlx/fp16_manifest.json, entry "conf"), the one reference-held fixture of the mixed-checkpoint contract.

For each stack below, the group records owned by layer 0 (or by its submodules) and the fp16 parameter names under
layer 0, both relative to the layer; for the token transformer also the stack-level groups, with their sources
limited to layer 0's. Data only: names, shapes, cache names and flags as the reference's file lists them.

Run (in a checkout that has the reference next to it): python tests/golden/make_manifest_fixture.py
"""

from __future__ import annotations

import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = "/root/reference/boltz_mlx/fp16_manifest.json"
STACKS = {
    "pairformer_layer": "pairformer_module.layers.0",
    "msa_layer": "msa_module.layers.0",
    "token_transformer_layer": "structure_module.score_model.token_transformer.layers.0",
}
TOKEN_STACK = "structure_module.score_model.token_transformer"


def main() -> None:
    with open(SRC) as f:
        conf = json.load(f)["conf"]
    out = {"source": "boltz_mlx/fp16_manifest.json (conf)"}
    for key, layer in STACKS.items():
        pre = layer + "."
        groups = []
        for g in conf["groups"]:
            if g["owner"] == layer or g["owner"].startswith(pre):
                groups.append({**g, "owner": g["owner"][len(pre):] if g["owner"] != layer else ""})
        params = sorted(p[len(pre):] for p in conf["params"] if p.startswith(pre))
        out[key] = {"groups": groups, "params": params}
    stack_groups = []
    for g in conf["groups"]:
        if g["owner"] == TOKEN_STACK:
            srcs = [s for s in g["srcs"] if s is None or s.startswith("layers.0.")]
            stack_groups.append({**g, "owner": "", "srcs": srcs})
    out["token_transformer_stack_groups_layer0"] = stack_groups
    with open(os.path.join(HERE, "fp16_manifest_layers.json"), "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
        f.write("\n")


if __name__ == "__main__":
    main()
