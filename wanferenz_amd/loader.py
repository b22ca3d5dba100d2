"""Converted checkpoint -> expert bank -> packed HIP layer, for one MoE layer.

The reference serves from the OUTPUT of its converter (wanferenz/model/
conversion.py:89-140): ``model*-mp1.safetensors`` files whose tensor names are
the module paths of the model (``_rename``, conversion.py:15-29), read by name
(partition.py:69-97) and loaded per block with ``load_state_dict``
(partition.py:759-773), after which ``_relayout_moe`` turns the per-expert
parameters into views of one bank (fp4_grouped.py:142-188).

This module reads the same files by name.  :func:`hip_moe_layer` (the serving
path) copies one expert at a time to the device and packs it straight into the
MFMA-ready banks of :class:`~wanferenz_amd.moe.HipMoE`, so the layer never
holds a second, reference-layout copy of its experts (the packed banks play the
part of the reference's bank, loaded in place with ``preserve=False``,
partition.py:398-405).  :func:`load_moe_layer` reads the reference-layout bank
itself (inspection and tests).  Names read for block ``li`` (the state-dict
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


class _Layer:
    """What one block's MoE needs besides the routed experts, on the device."""

    def __init__(self, ck: "Checkpoint", layer: int, device):
        p = self.prefix = f"layers.{layer}.ffn."
        self.ck = ck
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
        cfg = self.cfg = moe_config(ck, layer, D, I, E)
        self.dev = dev = torch.device(device)
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
        self.shared = sh
        self.gate_w = gw.to(dev)
        self.gate_bias = self.tid2eid = None
        if ck.has(p + "gate.tid2eid"):
            t = ck.get(p + "gate.tid2eid")
            if t.dtype != torch.int32 or t.dim() != 2 or t.shape[1] != cfg.topk:
                raise CheckpointError(f"{p}gate.tid2eid: int32 [vocab, {cfg.topk}] expected, got "
                                      f"{t.dtype} {tuple(t.shape)}")
            self.tid2eid = t.to(dev)
        else:
            self.gate_bias = _expect(ck.get(p + "gate.bias"), p + "gate.bias", torch.float32, (E,)).to(dev)

    def expert(self, e: int):
        """Expert e's (w1, w1_s, w3, w3_s, w2, w2_s) as byte tensors on the device."""
        D, I = self.cfg.dim, self.cfg.inter
        q = f"{self.prefix}experts.{e}."
        out = []
        for kind, shape in (("w1", (I, D)), ("w3", (I, D)), ("w2", (D, I))):
            w = _expect(self.ck.get(q + kind + ".weight"), q + kind + ".weight", _FP4, (shape[0], shape[1] // 2))
            s = _expect(self.ck.get(q + kind + ".scale"), q + kind + ".scale", _E8M0, (shape[0], shape[1] // 32))
            out += [w.view(torch.uint8).to(self.dev), s.view(torch.uint8).to(self.dev)]
        return tuple(out)

    def shared_tuple(self):
        sh = self.shared
        return (sh["w1"][0], sh["w1"][1], sh["w3"][0], sh["w3"][1], sh["w2"][0], sh["w2"][1])


def _checkpoint(path_or_ck) -> "Checkpoint":
    return path_or_ck if isinstance(path_or_ck, Checkpoint) else Checkpoint(path_or_ck)


def load_moe_layer(path_or_ck, layer: int, device="cuda") -> Tuple[MoEConfig, MoEWeights]:
    """Read block ``layer``'s MoE from a converted checkpoint into reference-layout bank
    tensors on ``device``: w13 [E, 2I, D/2] (w1 rows, then w3 rows), w2 [E, D, I/2] and
    their e8m0 scales, the shared expert and the gate (for inspection; the serving path,
    :func:`hip_moe_layer`, never builds this bank)."""
    L = _Layer(_checkpoint(path_or_ck), layer, device)
    cfg = L.cfg
    E, D, I = cfg.n_experts, cfg.dim, cfg.inter
    u8 = dict(dtype=torch.uint8, device=L.dev)
    w13 = torch.empty(E, 2 * I, D // 2, **u8)
    w13_s = torch.empty(E, 2 * I, D // 32, **u8)
    w2 = torch.empty(E, D, I // 2, **u8)
    w2_s = torch.empty(E, D, I // 32, **u8)
    for e in range(E):
        w1, s1, w3, s3, wb, sb = L.expert(e)
        torch.cat([w1, w3], out=w13[e])
        torch.cat([s1, s3], out=w13_s[e])
        w2[e].copy_(wb)
        w2_s[e].copy_(sb)
    sh = L.shared_tuple()
    w = MoEWeights(gate_w=L.gate_w, gate_bias=L.gate_bias, w13=w13, w13_s=w13_s, w2=w2, w2_s=w2_s,
                   sh_w1=sh[0], sh_w1_s=sh[1], sh_w3=sh[2], sh_w3_s=sh[3], sh_w2=sh[4], sh_w2_s=sh[5],
                   tid2eid=L.tid2eid)
    return cfg, w


def hip_moe_layer(path_or_ck, layer: int, device="cuda", max_tokens: int = 16):
    """The packed HIP layer of block ``layer``, read expert by expert from the
    checkpoint and packed in place (HipMoE.from_experts): the device holds one
    expert's reference-layout tensors at a time, never the whole bank."""
    from .moe import HipMoE

    L = _Layer(_checkpoint(path_or_ck), layer, device)
    return HipMoE.from_experts(L.cfg, L.gate_w, L.gate_bias, L.expert, L.shared_tuple(), tid2eid=L.tid2eid,
                               max_tokens=max_tokens)
