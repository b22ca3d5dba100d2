"""Converted checkpoint -> expert bank -> packed HIP layer, for one MoE layer.

The reference serves from the OUTPUT of its converter (wanferenz/model/
conversion.py:89-140): ``model*-mp1.safetensors`` files whose tensor names are
the module paths of the model (``_rename``, conversion.py:15-29), read by name
(partition.py:69-97) and loaded per block with ``load_state_dict``
(partition.py:759-773), after which ``_relayout_moe`` turns the per-expert
parameters into views of one bank (fp4_grouped.py:142-188).

This module reads the same files directly into the bank layout on the device
(no per-expert module, no second copy of the reference layout) and returns the
:class:`~wanferenz_amd.moe.MoEWeights` that :class:`~wanferenz_amd.moe.HipMoE`
packs into MFMA-ready tiles once.  Names read for block ``li`` (the state-dict
keys of MoE / Gate / Expert, architecture.py:674-794):

* ``layers.{li}.ffn.gate.weight`` bf16 [E, D]; ``.gate.bias`` fp32 [E] or, on
  a hash-routed layer, ``.gate.tid2eid`` int32 [vocab, k];
* ``layers.{li}.ffn.experts.{e}.{w1,w3,w2}.weight`` float4_e2m1fn_x2 [N, K/2]
  with ``.scale`` float8_e8m0fnu [N, K/32] (the converter's fp4 expert dtype,
  conversion.py:71-80);
* ``layers.{li}.ffn.shared_experts.{w1,w3,w2}.weight`` float8_e4m3fn [N, K]
  with ``.scale`` [N/128, K/128] (e8m0 or float32).

``config.json`` (ModelArgs keys, partition.py:60-66) supplies top-k, the score
function, route scale, SwiGLU limit and the hash-layer count.
"""

from __future__ import annotations

import glob
import json
import os
from typing import Dict, List, Optional, Tuple

import torch

from . import _native as N
from .moe import MoEConfig, MoEWeights

_FP4 = torch.float4_e2m1fn_x2
_E8M0 = torch.float8_e8m0fnu
_E4M3 = torch.float8_e4m3fn


class CheckpointError(RuntimeError):
    pass


class Checkpoint:
    """Name -> file index of a converted checkpoint directory (the reference's
    tensor_locations / raw, partition.py:69-97), with open handles kept per file."""

    def __init__(self, path: str):
        from safetensors import safe_open

        self.path = path
        files = sorted(glob.glob(os.path.join(path, "model*-mp*.safetensors")))
        if not files:
            raise CheckpointError(f"no model*-mp*.safetensors in {path!r} (a converted checkpoint is expected)")
        self._open = safe_open
        self._where: Dict[str, str] = {}
        self._handles = {}
        for f in files:
            with safe_open(f, "pt", device="cpu") as h:
                for n in h.keys():
                    self._where[n] = f
        cfg = os.path.join(path, "config.json")
        self.args = json.load(open(cfg)) if os.path.exists(cfg) else {}

    def names(self, prefix: str) -> List[str]:
        return [n for n in self._where if n.startswith(prefix)]

    def has(self, name: str) -> bool:
        return name in self._where

    def get(self, name: str) -> torch.Tensor:
        f = self._where.get(name)
        if f is None:
            raise CheckpointError(f"{name!r} is not in {self.path!r}")
        h = self._handles.get(f)
        if h is None:
            h = self._handles[f] = self._open(f, "pt", device="cpu")
        return h.get_tensor(name)

    def close(self):
        self._handles.clear()


def _expect(t: torch.Tensor, name: str, dtype, shape) -> torch.Tensor:
    if t.dtype != dtype:
        raise CheckpointError(f"{name}: dtype {t.dtype}, expected {dtype}")
    if tuple(t.shape) != tuple(shape):
        raise CheckpointError(f"{name}: shape {tuple(t.shape)}, expected {tuple(shape)}")
    return t


def moe_config(ck: Checkpoint, layer: int, dim: int, inter: int, n_experts: int) -> MoEConfig:
    a = ck.args
    topk = int(a.get("n_activated_experts", a.get("num_experts_per_tok", 0)))
    if topk <= 0:
        raise CheckpointError("config.json gives no n_activated_experts")
    scale_fmt = a.get("scale_fmt", "ue8m0")
    return MoEConfig(dim, inter, n_experts, topk,
                     a.get("score_func", a.get("scoring_func", "sqrtsoftplus")),
                     float(a.get("route_scale", a.get("routed_scaling_factor", 1.0))),
                     float(a.get("swiglu_limit", 0.0)),
                     N.WZ_SCALE_F32 if scale_fmt is None else N.WZ_SCALE_UE8M0,
                     N.WZ_WSCALE_E8M0)


def load_moe_layer(path_or_ck, layer: int, device="cuda") -> Tuple[MoEConfig, MoEWeights]:
    """Read block ``layer``'s MoE from a converted checkpoint into bank tensors on
    ``device``: w13 [E, 2I, D/2] (w1 rows, then w3 rows), w2 [E, D, I/2] and their
    e8m0 scales, the shared expert and the gate, each byte copied once from the
    file into its slot of the bank."""
    ck = path_or_ck if isinstance(path_or_ck, Checkpoint) else Checkpoint(path_or_ck)
    p = f"layers.{layer}.ffn."
    if not ck.has(p + "gate.weight"):
        raise CheckpointError(f"no {p}gate.weight in {ck.path!r}")
    gw = ck.get(p + "gate.weight")
    if gw.dtype != torch.bfloat16 or gw.dim() != 2:
        raise CheckpointError(f"{p}gate.weight: bf16 [E, D] expected, got {gw.dtype} {tuple(gw.shape)}")
    E, D = gw.shape
    experts = sorted({int(n[len(p + "experts."):].split(".")[0]) for n in ck.names(p + "experts.")})
    if experts != list(range(E)):
        raise CheckpointError(f"{p}experts: indices {experts[:4]}.. do not cover 0..{E - 1} "
                              "(a partial expert range is not served)")
    w1_0 = ck.get(p + "experts.0.w1.weight")
    if w1_0.dtype != _FP4:
        raise CheckpointError(f"{p}experts.0.w1.weight: {w1_0.dtype}; the MXFP4 expert bank expects "
                              f"{_FP4} (convert with expert_dtype fp4)")
    I = w1_0.shape[0]
    cfg = moe_config(ck, layer, D, I, E)

    dev = torch.device(device)
    u8 = dict(dtype=torch.uint8, device=dev)
    w13 = torch.empty(E, 2 * I, D // 2, **u8)
    w13_s = torch.empty(E, 2 * I, D // 32, **u8)
    w2 = torch.empty(E, D, I // 2, **u8)
    w2_s = torch.empty(E, D, I // 32, **u8)
    for e in range(E):
        q = f"{p}experts.{e}."
        for j, kind in enumerate(("w1", "w3")):
            w = _expect(ck.get(q + kind + ".weight"), q + kind + ".weight", _FP4, (I, D // 2))
            s = _expect(ck.get(q + kind + ".scale"), q + kind + ".scale", _E8M0, (I, D // 32))
            w13[e, j * I:(j + 1) * I].copy_(w.view(torch.uint8))
            w13_s[e, j * I:(j + 1) * I].copy_(s.view(torch.uint8))
        w = _expect(ck.get(q + "w2.weight"), q + "w2.weight", _FP4, (D, I // 2))
        s = _expect(ck.get(q + "w2.scale"), q + "w2.scale", _E8M0, (D, I // 32))
        w2[e].copy_(w.view(torch.uint8))
        w2_s[e].copy_(s.view(torch.uint8))

    sh = {}
    for kind, shape in (("w1", (I, D)), ("w3", (I, D)), ("w2", (D, I))):
        name = f"{p}shared_experts.{kind}.weight"
        w = _expect(ck.get(name), name, _E4M3, shape)
        s = ck.get(f"{p}shared_experts.{kind}.scale")
        sshape = ((shape[0] + 127) // 128, (shape[1] + 127) // 128)
        if tuple(s.shape) != sshape or s.dtype not in (_E8M0, torch.float32):
            raise CheckpointError(f"{p}shared_experts.{kind}.scale: {s.dtype} {tuple(s.shape)}, expected "
                                  f"e8m0 or float32 {sshape}")
        sh[kind] = (w.view(torch.uint8).to(dev), (s.view(torch.uint8) if s.dtype == _E8M0 else s).to(dev))
    kinds = {s.dtype for _, s in sh.values()}
    if len(kinds) != 1:
        raise CheckpointError(f"{p}shared_experts: mixed scale dtypes {kinds}")
    if torch.float32 in kinds:
        cfg.shared_w_scale_kind = N.WZ_WSCALE_F32

    bias = tid2eid = None
    if ck.has(p + "gate.tid2eid"):
        tid2eid = ck.get(p + "gate.tid2eid")
        if tid2eid.dtype != torch.int32 or tid2eid.dim() != 2 or tid2eid.shape[1] != cfg.topk:
            raise CheckpointError(f"{p}gate.tid2eid: int32 [vocab, {cfg.topk}] expected, got "
                                  f"{tid2eid.dtype} {tuple(tid2eid.shape)}")
        tid2eid = tid2eid.to(dev)
    else:
        bias = _expect(ck.get(p + "gate.bias"), p + "gate.bias", torch.float32, (E,)).to(dev)
    w = MoEWeights(gate_w=gw.to(dev), gate_bias=bias, w13=w13, w13_s=w13_s, w2=w2, w2_s=w2_s,
                   sh_w1=sh["w1"][0], sh_w1_s=sh["w1"][1], sh_w3=sh["w3"][0], sh_w3_s=sh["w3"][1],
                   sh_w2=sh["w2"][0], sh_w2_s=sh["w2"][1], tid2eid=tid2eid)
    return cfg, w


def hip_moe_layer(path_or_ck, layer: int, device="cuda", max_tokens: int = 16):
    """The packed HIP layer of block ``layer`` (HipMoE over the loaded bank)."""
    from .moe import HipMoE

    cfg, w = load_moe_layer(path_or_ck, layer, device)
    return HipMoE(cfg, w, max_tokens=max_tokens)
