"""Write the converted-checkpoint tensor names of one MoE block from the reference
itself (run in the build container only).

What this pins: the names wanferenz_amd/loader.py reads.  A converted
``model*-mp1.safetensors`` file holds each tensor under the module path of the
reference model (the partition loader loads it by those names), and the
converter derives those names from the Hugging Face names with ``_rename``
(wanferenz/model/conversion.py:15-29, which looks the key up in
``tensor_layout.mapping``, wanferenz/model/tensor_layout.py:74-84).  This
script:

* builds the reference's own ``MoE`` module (architecture.py:744-794, loaded as
  make_golden.py loads it) for a routed layer and a hash-routed layer and lists
  ``state_dict()`` names under ``layers.<L>.ffn.``: the names a converted file
  must hold;
* writes, for each, the Hugging Face source name (``model.`` prefix, ``mlp``,
  ``weight_scale_inv``, ``e_score_correction_bias``: the renames ``_rename``
  undoes) and checks that the reference's ``_rename`` maps it back exactly.

Only names are written, to tests/golden/ckpt_names.json.

Usage:  python tests/golden/make_names.py [/root/reference]
"""

from __future__ import annotations

import json
import os
import sys

sys.dont_write_bytecode = True

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))


def hf_name(converted: str) -> str:
    """The Hugging Face name the converter turns into ``converted``."""
    n = "model." + converted.replace(".ffn.", ".mlp.")
    if n.endswith(".scale"):
        n = n[: -len(".scale")] + ".weight_scale_inv"
    if n.endswith(".gate.bias"):
        n = n[: -len(".bias")] + ".e_score_correction_bias"
    return n


def main():
    import torch

    from tests.golden.make_golden import load_reference

    ref_root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    mod = load_reference(ref_root, True)
    from wanferenz.model.conversion import _rename

    out = {"source": "architecture.py MoE.state_dict() under layers.<L>.ffn.; conversion._rename of the HF name",
           "layers": {}}
    for label, layer, n_hash in (("routed", 3, 0), ("hash", 0, 1)):
        args = mod.ModelArgs(dim=256, moe_inter_dim=128, n_routed_experts=4, n_activated_experts=2,
                             n_shared_experts=1, n_hash_layers=n_hash, expert_dtype="fp4", vocab_size=64)
        with mod.set_dtype(torch.bfloat16):
            moe = mod.MoE(layer, args)
        names = {}
        for k in sorted(moe.state_dict()):
            conv = f"layers.{layer}.ffn.{k}"
            src = hf_name(conv)
            back = _rename(src)
            if back != conv:
                raise SystemExit(f"_rename({src!r}) = {back!r}, expected {conv!r}")
            names[conv] = src
        out["layers"][label] = {"layer": layer, "n_experts": 4, "names": names}
        print(f"{label}: {len(names)} names, e.g. {next(iter(names.items()))}")
    with open(os.path.join(HERE, "ckpt_names.json"), "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()
