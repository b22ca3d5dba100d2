"""Write a golden case's weights as a converted checkpoint (test fixture helper).

Tensor names, dtypes and shapes follow the converter's output
(wanferenz/model/conversion.py:15-29 renaming, :71-80 fp4 experts) and the
module paths of the model (architecture.py:674-794): the file a
LayerPartition would load (partition.py:759-773).
"""

from __future__ import annotations

import json
import os

import numpy as np
import torch


def _t(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    return t.view(dtype) if dtype is not None else t


def write_case_checkpoint(case, inp, path, layer=3, split_files=True, extra_layer=True):
    from safetensors.torch import save_file

    os.makedirs(path, exist_ok=True)
    I, E = case.inter, case.n_experts
    nb = I // 128
    p = f"layers.{layer}.ffn."
    st = {p + "gate.weight": _t(inp.gate_w.view(np.int16), torch.bfloat16)}
    if inp.tid2eid is not None:
        st[p + "gate.tid2eid"] = _t(inp.tid2eid.astype(np.int32))
    else:
        st[p + "gate.bias"] = _t(inp.gate_bias.astype(np.float32))
    for e in range(E):
        q = f"{p}experts.{e}."
        st[q + "w1.weight"] = _t(inp.w13[e, :I], torch.float4_e2m1fn_x2)
        st[q + "w1.scale"] = _t(inp.w13_s[e, :I], torch.float8_e8m0fnu)
        st[q + "w3.weight"] = _t(inp.w13[e, I:], torch.float4_e2m1fn_x2)
        st[q + "w3.scale"] = _t(inp.w13_s[e, I:], torch.float8_e8m0fnu)
        st[q + "w2.weight"] = _t(inp.w2[e], torch.float4_e2m1fn_x2)
        st[q + "w2.scale"] = _t(inp.w2_s[e], torch.float8_e8m0fnu)
    q = p + "shared_experts."
    st[q + "w1.weight"] = _t(inp.sh_w13[:I], torch.float8_e4m3fn)
    st[q + "w1.scale"] = _t(inp.sh_w13_s[:nb], torch.float8_e8m0fnu)
    st[q + "w3.weight"] = _t(inp.sh_w13[I:], torch.float8_e4m3fn)
    st[q + "w3.scale"] = _t(inp.sh_w13_s[nb:], torch.float8_e8m0fnu)
    st[q + "w2.weight"] = _t(inp.sh_w2, torch.float8_e4m3fn)
    st[q + "w2.scale"] = _t(inp.sh_w2_s, torch.float8_e8m0fnu)
    if extra_layer:  # a neighbouring block's tensor, which the loader must ignore
        st[f"layers.{layer + 1}.attn_norm.weight"] = torch.ones(case.dim, dtype=torch.float32)
    names = sorted(st)
    if split_files:  # tensors of one block spread over two files, as a converted release has
        half = len(names) // 2
        parts = [names[:half], names[half:]]
    else:
        parts = [names]
    for i, part in enumerate(parts):
        save_file({n: st[n].contiguous() for n in part}, os.path.join(path, f"model{i:05d}-mp1.safetensors"))
    cfg = {"dim": case.dim, "moe_inter_dim": case.inter, "n_routed_experts": E,
           "n_activated_experts": case.topk, "score_func": case.score_func,
           "route_scale": case.route_scale, "swiglu_limit": case.swiglu_limit,
           "scale_fmt": "ue8m0" if case.round_pow2 else None,
           "n_hash_layers": layer + 1 if inp.tid2eid is not None else 0}
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(cfg, f)
    return path
