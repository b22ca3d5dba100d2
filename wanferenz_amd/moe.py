"""MoE layer on the HIP library: the drop-in for the reference's MoE dispatch chain.

Two ways in:

* :class:`HipMoE` — a standalone layer over expert-bank tensors
  (w13 ``[E, 2I, D/2]`` packed e2m1 + ``[E, 2I, D/32]`` e8m0, w2 ``[E, D, I/2]``
  + ``[E, D, I/32]``, the bank layout of wanferenz/kernels/fp4_grouped.py:142-188)
  with an FP8 shared expert and a bf16 gate.  ``forward(x, input_ids)`` is one
  stream-ordered sequence of launches with no host sync and no allocation
  besides its output, so a decode step can be captured in a HIP graph.
* :func:`install` — replaces ``MoE.forward`` of a loaded reference model module
  at class level, following the reference's install protocol
  (fp4_grouped.py:339-351): the previous forward is kept in ``_REF_FORWARD``,
  the new function carries a ``_v4_hip_moe`` marker and installing twice is a
  no-op.  A layer the HIP path cannot serve (``world_size > 1``, an expert
  dtype other than MXFP4, a shared expert other than FP8) declines to
  ``_REF_FORWARD`` with a reason tally in ``moe._hip_declined``, as
  fp4_grouped._decline does (fp4_grouped.py:256-262).  The declined path still
  runs on the HIP library when :func:`wanferenz_amd.kernels.install` has
  rebound the module's act_quant / fp8_gemm / fp4_gemm.
"""

from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass, field
from typing import Optional

import torch

from . import _native as N
from . import kernels

SCORE_FUNCS = {"softmax": N.WZ_SCORE_SOFTMAX, "sigmoid": N.WZ_SCORE_SIGMOID,
               "sqrtsoftplus": N.WZ_SCORE_SQRTSOFTPLUS}


class WzMoeDesc(ctypes.Structure):
    """ctypes mirror of ``wz_moe_desc`` (include/wanferenz_amd.h)."""

    _fields_ = [
        ("dim", ctypes.c_int32), ("inter", ctypes.c_int32), ("n_experts", ctypes.c_int32),
        ("topk", ctypes.c_int32), ("score_func", ctypes.c_int32),
        ("act_scale_kind", ctypes.c_int32), ("shared_w_scale_kind", ctypes.c_int32),
        ("route_scale", ctypes.c_float), ("swiglu_limit", ctypes.c_float),
        ("vocab", ctypes.c_int64),
        ("gate_w", ctypes.c_void_p), ("gate_bias", ctypes.c_void_p), ("tid2eid", ctypes.c_void_p),
        ("w13", ctypes.c_void_p), ("w13_s", ctypes.c_void_p),
        ("w2", ctypes.c_void_p), ("w2_s", ctypes.c_void_p),
        ("sh_w1", ctypes.c_void_p), ("sh_w1_s", ctypes.c_void_p),
        ("sh_w3", ctypes.c_void_p), ("sh_w3_s", ctypes.c_void_p),
        ("sh_w2", ctypes.c_void_p), ("sh_w2_s", ctypes.c_void_p),
        ("w13p", ctypes.c_void_p), ("w13p_s", ctypes.c_void_p),
        ("w2p", ctypes.c_void_p), ("w2p_s", ctypes.c_void_p),
        ("sh13p", ctypes.c_void_p), ("sh2p", ctypes.c_void_p),
    ]

PACKED_NAMES = ("w13p", "w13p_s", "w2p", "w2p_s", "sh13p", "sh2p")


@dataclass
class MoEConfig:
    dim: int
    inter: int
    n_experts: int
    topk: int
    score_func: str = "sqrtsoftplus"
    route_scale: float = 1.0
    swiglu_limit: float = 0.0
    act_scale_kind: int = N.WZ_SCALE_UE8M0       # reference scale_fmt="ue8m0"
    shared_w_scale_kind: int = N.WZ_WSCALE_E8M0


@dataclass
class MoEWeights:
    """Device tensors of one MoE layer (byte views; formats in the module docstring)."""

    gate_w: torch.Tensor                  # bf16 [E, D]
    gate_bias: Optional[torch.Tensor]     # fp32 [E], None for hash-routed layers
    w13: torch.Tensor                     # uint8 [E, 2I, D/2]
    w13_s: torch.Tensor                   # uint8 [E, 2I, D/32]
    w2: torch.Tensor                      # uint8 [E, D, I/2]
    w2_s: torch.Tensor                    # uint8 [E, D, I/32]
    sh_w1: torch.Tensor                   # uint8 (e4m3) [I, D]
    sh_w1_s: torch.Tensor                 # [I/128, D/128] e8m0 bytes or fp32
    sh_w3: torch.Tensor
    sh_w3_s: torch.Tensor
    sh_w2: torch.Tensor                   # [D, I]
    sh_w2_s: torch.Tensor                 # [D/128, I/128]
    tid2eid: Optional[torch.Tensor] = None  # int32 [vocab, k]


_BYTE_TYPES = (torch.uint8, torch.float4_e2m1fn_x2, torch.float8_e8m0fnu, torch.float8_e4m3fn, torch.int8)


def _need(name, t, shape, dtypes=None):
    if t is None:
        raise ValueError(f"MoE weights: {name} missing")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"MoE weights: {name} has shape {tuple(t.shape)}, want {tuple(shape)}")
    if not t.is_contiguous():
        raise ValueError(f"MoE weights: {name} must be contiguous")
    if not t.is_cuda:
        raise RuntimeError(f"MoE weights: {name} must be on the GPU (no CPU fallback)")
    if dtypes and t.dtype not in dtypes:
        raise TypeError(f"MoE weights: {name} dtype {t.dtype} not in {dtypes}")


def _check_gate(cfg: MoEConfig, gate_w, gate_bias, tid2eid):
    E, D, k = cfg.n_experts, cfg.dim, cfg.topk
    _need("gate_w", gate_w, (E, D), (torch.bfloat16,))
    if tid2eid is None:
        if gate_bias is not None:
            _need("gate_bias", gate_bias, (E,), (torch.float32,))
    elif (tid2eid.dim() != 2 or tid2eid.size(1) != k or tid2eid.dtype != torch.int32 or not tid2eid.is_cuda
          or not tid2eid.is_contiguous()):
        raise ValueError("MoE weights: tid2eid must be a contiguous int32 [vocab, k] GPU tensor")


def _shared_scale_types(cfg: MoEConfig):
    return (torch.float32,) if cfg.shared_w_scale_kind == N.WZ_WSCALE_F32 else _BYTE_TYPES


def _check_shared(cfg: MoEConfig, sh):
    """sh = (w1, w1_s, w3, w3_s, w2, w2_s) of the FP8 shared expert; weights may be None
    (only the scales are checked then)."""
    D, I = cfg.dim, cfg.inter
    nb = lambda n: (n + 127) // 128  # noqa: E731
    shapes = ((I, D), (nb(I), nb(D)), (I, D), (nb(I), nb(D)), (D, I), (nb(D), nb(I)))
    for j, (name, t, shape) in enumerate(zip(("sh_w1", "sh_w1_s", "sh_w3", "sh_w3_s", "sh_w2", "sh_w2_s"), sh, shapes)):
        if j % 2 == 0 and t is None:
            continue
        _need(name, t, shape, _BYTE_TYPES if j % 2 == 0 else _shared_scale_types(cfg))


def _check_expert(cfg: MoEConfig, e, ex):
    D, I = cfg.dim, cfg.inter
    shapes = ((I, D // 2), (I, D // 32), (I, D // 2), (I, D // 32), (D, I // 2), (D, I // 32))
    for name, t, shape in zip(("w1", "w1_s", "w3", "w3_s", "w2", "w2_s"), ex, shapes):
        _need(f"expert {e} {name}", t, shape, _BYTE_TYPES)


def _check_layout(cfg: MoEConfig, w: MoEWeights):
    D, I, E = cfg.dim, cfg.inter, cfg.n_experts
    _check_gate(cfg, w.gate_w, w.gate_bias, w.tid2eid)
    _need("w13", w.w13, (E, 2 * I, D // 2), _BYTE_TYPES)
    _need("w13_s", w.w13_s, (E, 2 * I, D // 32), _BYTE_TYPES)
    _need("w2", w.w2, (E, D, I // 2), _BYTE_TYPES)
    _need("w2_s", w.w2_s, (E, D, I // 32), _BYTE_TYPES)
    _check_shared(cfg, (w.sh_w1, w.sh_w1_s, w.sh_w3, w.sh_w3_s, w.sh_w2, w.sh_w2_s))


def _ptr(t):
    return None if t is None else t.data_ptr()


class HipMoE:
    """One MoE layer served by the HIP library (see module docstring).

    The layer holds the packed expert banks (the only copy the kernels read),
    the gate, the tid2eid table of a hash layer and the shared expert's block
    scales.  ``HipMoE(cfg, weights)`` packs a reference-layout bank and keeps
    ``weights`` (``self.weights``) unless ``keep_reference=False``;
    :meth:`from_experts` packs expert by expert and never holds a
    reference-layout bank.
    """

    def __init__(self, cfg: MoEConfig, weights: MoEWeights, max_tokens: int = 16, keep_reference: bool = True):
        if cfg.score_func not in SCORE_FUNCS:
            raise ValueError(f"unknown score_func {cfg.score_func!r}")
        _check_layout(cfg, weights)
        w = weights
        self._setup(cfg, w.gate_w, w.gate_bias, w.tid2eid, (w.sh_w1_s, w.sh_w3_s, w.sh_w2_s))
        d = self.desc
        for name in ("w13", "w13_s", "w2", "w2_s", "sh_w1", "sh_w3", "sh_w2"):
            setattr(d, name, getattr(w, name).data_ptr())
        self._alloc_packed()
        N.call("wz_moe_pack", ctypes.byref(d), *(self.packed[n].data_ptr() for n in PACKED_NAMES),
               N.stream_handle(self.device))
        self.weights = weights if keep_reference else None
        if not keep_reference:
            self._forget_reference()
        self._ws = None
        self._ws_tokens = 0
        self.reserve(max_tokens)

    @classmethod
    def from_experts(cls, cfg: MoEConfig, gate_w, gate_bias, experts, shared, tid2eid=None,
                     max_tokens: int = 16) -> "HipMoE":
        """Build the layer one expert at a time, with no reference-layout bank.

        ``experts(e)`` returns expert e's ``(w1, w1_s, w3, w3_s, w2, w2_s)`` device
        tensors (e2m1x2 / e8m0 bytes, shapes of one reference Expert); each is
        packed into its slot (wz_moe_pack_expert) and may be dropped by the caller
        right after.  ``shared`` is ``(w1, w1_s, w3, w3_s, w2, w2_s)`` of the FP8
        shared expert; only its scales are kept.
        """
        if cfg.score_func not in SCORE_FUNCS:
            raise ValueError(f"unknown score_func {cfg.score_func!r}")
        _check_gate(cfg, gate_w, gate_bias, tid2eid)
        _check_shared(cfg, shared)
        self = object.__new__(cls)
        self._setup(cfg, gate_w, gate_bias, tid2eid, (shared[1], shared[3], shared[5]))
        self._alloc_packed()
        stream = N.stream_handle(self.device)
        for e in range(cfg.n_experts):
            ex = experts(e)
            _check_expert(cfg, e, ex)
            N.call("wz_moe_pack_expert", ctypes.byref(self.desc), e, *(t.data_ptr() for t in ex), stream)
        N.call("wz_moe_pack_shared", ctypes.byref(self.desc), shared[0].data_ptr(), shared[2].data_ptr(),
               shared[4].data_ptr(), stream)
        self.weights = None
        self._ws = None
        self._ws_tokens = 0
        self.reserve(max_tokens)
        return self

    def _setup(self, cfg, gate_w, gate_bias, tid2eid, shared_scales):
        self.cfg = cfg
        self.gate_w, self.tid2eid = gate_w, tid2eid
        self.gate_bias = None if tid2eid is not None else gate_bias
        self.shared_scales = tuple(shared_scales)
        self.device = gate_w.device
        d = WzMoeDesc()
        d.dim, d.inter, d.n_experts, d.topk = cfg.dim, cfg.inter, cfg.n_experts, cfg.topk
        d.score_func = SCORE_FUNCS[cfg.score_func]
        d.act_scale_kind = cfg.act_scale_kind
        d.shared_w_scale_kind = cfg.shared_w_scale_kind
        d.route_scale = cfg.route_scale
        d.swiglu_limit = cfg.swiglu_limit
        d.vocab = 0 if tid2eid is None else tid2eid.size(0)
        d.gate_w = gate_w.data_ptr()
        d.gate_bias = _ptr(self.gate_bias)
        d.tid2eid = _ptr(tid2eid)
        d.sh_w1_s, d.sh_w3_s, d.sh_w2_s = (t.data_ptr() for t in self.shared_scales)
        self.desc = d

    def _alloc_packed(self):
        d = self.desc
        self.packed = {}
        for i, name in enumerate(PACKED_NAMES):
            n = int(N.lib().wz_moe_packed_bytes(ctypes.byref(d), i))
            self.packed[name] = torch.empty(n, dtype=torch.uint8, device=self.device)
            setattr(d, name, self.packed[name].data_ptr())

    def _forget_reference(self):
        for name in ("w13", "w13_s", "w2", "w2_s", "sh_w1", "sh_w3", "sh_w2"):
            setattr(self.desc, name, None)

    def with_gate_bias(self, bias: torch.Tensor, max_tokens: int = 16) -> "HipMoE":
        """A layer over the same expert banks (packed once) with another fp32 gate bias [E]."""
        import dataclasses

        if self.tid2eid is not None:
            raise ValueError("HipMoE: a hash-routed layer has no gate bias")
        bias = bias.to(device=self.device, dtype=torch.float32).contiguous()
        if bias.shape != (self.cfg.n_experts,):
            raise ValueError(f"HipMoE: gate bias must be [{self.cfg.n_experts}], got {tuple(bias.shape)}")
        other = object.__new__(HipMoE)
        other.cfg = self.cfg
        other.gate_w, other.tid2eid, other.gate_bias = self.gate_w, None, bias
        other.shared_scales = self.shared_scales
        other.weights = None if self.weights is None else dataclasses.replace(self.weights, gate_bias=bias)
        other.desc = WzMoeDesc()
        ctypes.memmove(ctypes.byref(other.desc), ctypes.byref(self.desc), ctypes.sizeof(WzMoeDesc))
        other.desc.gate_bias = bias.data_ptr()
        other.device = self.device
        other.packed = self.packed
        other._ws = None
        other._ws_tokens = 0
        other.reserve(max_tokens)
        return other

    # -- workspace -----------------------------------------------------------
    def workspace_bytes(self, T: int) -> int:
        return int(N.lib().wz_moe_workspace_bytes(ctypes.byref(self.desc), T))

    def reserve(self, T: int):
        """Allocate scratch for up to T tokens (outside any graph capture)."""
        if T <= self._ws_tokens and self._ws is not None:
            return
        nbytes = max(self.workspace_bytes(T), 256)
        self._ws = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        N.call("wz_moe_workspace_init", self._ws.data_ptr(), nbytes, N.stream_handle(self.device))
        self._ws_tokens = T

    def _ws_for(self, T: int):
        if T > self._ws_tokens:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(
                    f"HipMoE: T={T} exceeds the reserved workspace ({self._ws_tokens} tokens) "
                    "inside graph capture; call reserve() before capturing")
            self.reserve(T)
        return self._ws

    # -- compute -------------------------------------------------------------
    def _tokens(self, x: torch.Tensor) -> torch.Tensor:
        if x.dtype != torch.bfloat16:
            raise TypeError(f"HipMoE: x must be bf16, got {x.dtype}")
        if x.device != self.device:
            raise RuntimeError(f"HipMoE: x is on {x.device}, the layer on {self.device} (no CPU fallback)")
        if x.size(-1) != self.cfg.dim:
            raise ValueError(f"HipMoE: x has rows of {x.size(-1)}, the layer dim is {self.cfg.dim}")
        return x.reshape(-1, self.cfg.dim).contiguous()

    def _ids(self, input_ids, T: int):
        """int64 ids on the layer's device for a hash-routed layer, else None.

        Ids given on the host are range-checked there (IndexError, as the
        reference's ``tid2eid[input_ids]`` raises); device ids are not read back:
        an id outside the table gives that token NaN routing weights and a NaN
        output row instead (the kernels never read outside the table)."""
        if self.tid2eid is None:
            return None
        if input_ids is None:
            raise ValueError("HipMoE: a hash-routed layer needs input_ids")
        ids = input_ids.reshape(-1)
        if ids.numel() != T:
            raise ValueError(f"HipMoE: input_ids has {ids.numel()} ids for {T} tokens")
        if not ids.is_cuda and T:
            lo, hi = int(ids.min()), int(ids.max())
            if lo < 0 or hi >= self.tid2eid.size(0):
                raise IndexError(f"HipMoE: input id {lo if lo < 0 else hi} outside the tid2eid table "
                                 f"of {self.tid2eid.size(0)} rows")
        return ids.to(self.device, torch.int64).contiguous()

    def _check_out(self, t, shape, dtype, what):
        if t.dtype != dtype or t.device != self.device or not t.is_contiguous() or t.numel() != shape[0] * shape[1]:
            raise ValueError(f"HipMoE: {what} must be a contiguous {dtype} tensor of {shape[0]}x{shape[1]} "
                             f"elements on {self.device}, got {t.dtype} {tuple(t.shape)} on {t.device}")

    def forward(self, x: torch.Tensor, input_ids: Optional[torch.Tensor] = None,
                out: Optional[torch.Tensor] = None, routing_out=None) -> torch.Tensor:
        """x [..., D] bf16 -> y [..., D] bf16 (MoE.forward, architecture.py:777-794), any number of tokens.

        ``out`` (bf16, T*D elements) receives y when given; ``routing_out`` =
        (weights fp32 [T, k], indices int64 [T, k]) receives the routing."""
        xv = self._tokens(x)
        T, D, k = xv.size(0), self.cfg.dim, self.cfg.topk
        ids = self._ids(input_ids, T)
        if out is not None:
            self._check_out(out, (T, D), torch.bfloat16, "out")
        y = out if out is not None else torch.empty_like(xv)
        wp = ip = None
        if routing_out is not None:
            self._check_out(routing_out[0], (T, k), torch.float32, "routing weights")
            self._check_out(routing_out[1], (T, k), torch.int64, "routing indices")
            wp, ip = routing_out[0].data_ptr(), routing_out[1].data_ptr()
        ws = self._ws_for(T)
        N.call("wz_moe_forward", ctypes.byref(self.desc), xv.data_ptr(), _ptr(ids), T, y.data_ptr(), wp, ip,
               ws.data_ptr(), ws.numel(), N.stream_handle(self.device))
        return y.view(x.shape)

    __call__ = forward

    # widths the routing launch normalises itself (wz_moe_forward_norm)
    NORM_MAX_T, NORM_MAX_D = 8, 4096

    def forward_norm(self, h: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                     input_ids: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
                     routing_out=None) -> torch.Tensor:
        """forward(RMSNorm(h)): ``x = self.ffn_norm(x); x = self.ffn(x, input_ids)`` of
        Block.forward (architecture.py:871-872) in one call, bit for bit the norm
        (kernels.rms_norm) followed by forward().  For decode widths (T <= 8,
        D <= 4096) the routing launch normalises the rows it reads, so no norm
        launch runs; other widths run the norm, then forward."""
        hv = self._tokens(h)
        T, D, k = hv.size(0), self.cfg.dim, self.cfg.topk
        nw = norm_weight.detach()
        if nw.dtype != torch.float32 or nw.numel() != D or not nw.is_contiguous() or nw.device != hv.device:
            raise ValueError(f"HipMoE.forward_norm: norm weight must be a contiguous fp32 [{D}] tensor on {hv.device}")
        if T > self.NORM_MAX_T or D > self.NORM_MAX_D:
            from . import kernels
            return self.forward(kernels.rms_norm(h, norm_weight, eps), input_ids, out=out, routing_out=routing_out)
        ids = self._ids(input_ids, T)
        if out is not None:
            self._check_out(out, (T, D), torch.bfloat16, "out")
        y = out if out is not None else torch.empty_like(hv)
        wp = ip = None
        if routing_out is not None:
            self._check_out(routing_out[0], (T, k), torch.float32, "routing weights")
            self._check_out(routing_out[1], (T, k), torch.int64, "routing indices")
            wp, ip = routing_out[0].data_ptr(), routing_out[1].data_ptr()
        ws = self._ws_for(T)
        N.call("wz_moe_forward_norm", ctypes.byref(self.desc), hv.data_ptr(), nw.data_ptr(), float(eps),
               _ptr(ids), T, y.data_ptr(), wp, ip, ws.data_ptr(), ws.numel(), N.stream_handle(self.device))
        return y.view(h.shape)

    def replay_stage(self, x: torch.Tensor, stage: int, out: torch.Tensor,
                     input_ids: Optional[torch.Tensor] = None) -> None:
        """Re-launch one stage (N.WZ_STAGE_*) of the preceding forward(x, input_ids, out) call.

        The workspace still holds that call's routing tables and intermediates;
        this is for timing a stage alone (eagerly or captured in a graph).
        """
        xv = self._tokens(x)
        T = xv.size(0)
        if T > self._ws_tokens or T * self.cfg.topk > 16384:
            raise RuntimeError("HipMoE.replay_stage: no preceding single-chunk forward with this many tokens")
        self._check_out(out, (T, self.cfg.dim), torch.bfloat16, "out")
        ids = self._ids(input_ids, T)
        N.call("wz_moe_replay_stage", ctypes.byref(self.desc), xv.data_ptr(), _ptr(ids), T, int(stage),
               out.data_ptr(), self._ws.data_ptr(), self._ws.numel(), N.stream_handle(self.device))

    def route(self, x: torch.Tensor, input_ids: Optional[torch.Tensor] = None):
        """Gate.forward + canonical permutation: (weights, indices, offsets, perm_token, perm_slot)."""
        D, E, k = self.cfg.dim, self.cfg.n_experts, self.cfg.topk
        xv = self._tokens(x)
        T = xv.size(0)
        ids = self._ids(input_ids, T)
        dev = self.device
        weights = torch.empty(T, k, dtype=torch.float32, device=dev)
        indices = torch.empty(T, k, dtype=torch.int64, device=dev)
        offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
        ptok = torch.empty(T * k, dtype=torch.int32, device=dev)
        pslot = torch.empty(T * k, dtype=torch.int32, device=dev)
        ws = self._ws_for(T)
        N.call("wz_moe_route", ctypes.byref(self.desc), xv.data_ptr(), _ptr(ids), T, weights.data_ptr(),
               indices.data_ptr(), offsets.data_ptr(), ptok.data_ptr(), pslot.data_ptr(), ws.data_ptr(),
               ws.numel(), N.stream_handle(dev))
        return weights, indices, offsets, ptok, pslot


# ---------------------------------------------------------------- drop-in -----

_REF_FORWARD = None
_MOD = None
# hip_moe_of's default: empty the module's expert weights once packed (one copy in HBM)
RELEASE_EXPERTS = True


def _act_kind_of_module(mod) -> int:
    scale_fmt = getattr(mod, "scale_fmt", None)
    scale_dtype = getattr(mod, "scale_dtype", torch.float32)
    if scale_fmt is None:
        return N.WZ_SCALE_F32
    return N.WZ_SCALE_UE8M0 if scale_dtype == torch.float8_e8m0fnu else N.WZ_SCALE_UE8M0_F32


def _bytes(p) -> torch.Tensor:
    return p.detach().view(torch.uint8)


def _release(params):
    """Point each parameter at an empty tensor of its dtype: the packed banks are the
    layer's only copy from here on (the reference's bank layout with preserve=False,
    serving/partition.py:398-405, likewise leaves no per-expert storage behind)."""
    empty = {}
    for p in params:
        key = (p.dtype, p.device)
        if key not in empty:
            empty[key] = torch.empty(0, dtype=p.dtype, device=p.device)
        p.data = empty[key]
        # a packed-tile record of the FP8 linear path (kernels._packed_of) names
        # storage that is gone
        p.__dict__.pop("_wz_packed", None)


def hip_moe_of(moe, mod=None, release: Optional[bool] = None) -> Optional[HipMoE]:
    """Build (once) and cache the HipMoE view of a reference MoE module.

    Each routed expert's w1/w3/w2 parameters are packed straight into the packed
    banks (wz_moe_pack_expert), and the shared expert's into its FP8 tiles.  With
    ``release`` (default: the module flag ``RELEASE_EXPERTS``, on) the packed
    weight parameters are emptied afterwards, so the layer holds one copy of its
    experts; the gate and the block scales of the shared expert stay.  A released
    layer cannot be served by the kept reference forward any more.
    """
    h = getattr(moe, "_hip_moe", None)
    if h is not None:
        return h
    mod = mod or _MOD
    release = RELEASE_EXPERTS if release is None else release
    lo, hi = moe.experts_start_idx, moe.experts_end_idx
    if hi - lo <= 0 or moe.experts[lo].w1.weight.dtype != torch.float4_e2m1fn_x2:
        return None
    sh = moe.shared_experts
    if sh.w1.weight.dtype != torch.float8_e4m3fn:
        return None
    e0 = moe.experts[lo]
    gate = moe.gate
    cfg = MoEConfig(
        dim=moe.dim, inter=e0.w1.weight.shape[0], n_experts=moe.n_routed_experts,
        topk=moe.n_activated_experts, score_func=gate.score_func,
        route_scale=float(gate.route_scale), swiglu_limit=float(e0.swiglu_limit),
        act_scale_kind=_act_kind_of_module(mod),
        shared_w_scale_kind=N.WZ_WSCALE_E8M0 if sh.w1.scale.dtype == torch.float8_e8m0fnu else N.WZ_WSCALE_F32,
    )

    def expert(e):
        ex = moe.experts[e]
        return tuple(_bytes(getattr(getattr(ex, kind), attr)) for kind in ("w1", "w3", "w2")
                     for attr in ("weight", "scale"))

    def scale(lin):
        return lin.scale.detach() if lin.scale.dtype == torch.float32 else _bytes(lin.scale)

    with torch.no_grad():
        # the shared expert's linears may have run through the installed FP8 path,
        # which packs weights in their own storage; the bank packer reads row-major
        for lin in (sh.w1, sh.w3, sh.w2):
            kernels.unpack_fp8_in_place(lin.weight)
        shared = (_bytes(sh.w1.weight), scale(sh.w1), _bytes(sh.w3.weight), scale(sh.w3), _bytes(sh.w2.weight),
                  scale(sh.w2))
        h = HipMoE.from_experts(
            cfg, gate.weight.detach(), None if gate.bias is None else gate.bias.detach(), expert, shared,
            tid2eid=gate.tid2eid.detach() if getattr(gate, "hash", False) else None)
        if release:
            # the pack kernels read the module's storage on the current stream; the
            # caching allocator may hand freed blocks to another stream (the
            # reference warms its graphs up on a side stream), so they finish first
            torch.cuda.current_stream(gate.weight.device).synchronize()
            # the reference's relayout may have left a bank the experts' views point into
            moe._grouped_bank = None
            _release([getattr(getattr(moe.experts[e], kind), "weight") for e in range(lo, hi)
                      for kind in ("w1", "w3", "w2")] + [sh.w1.weight, sh.w3.weight, sh.w2.weight])
            _release([getattr(getattr(moe.experts[e], kind), "scale") for e in range(lo, hi)
                      for kind in ("w1", "w3", "w2")])
            moe._hip_released = True
    moe._hip_moe = h
    return h


def _servable(moe, mod) -> Optional[str]:
    """Why the HIP layer cannot serve ``moe`` (a decline reason), or None."""
    if int(getattr(mod, "world_size", 1) or 1) > 1:
        return "world_size>1"
    if moe.experts_start_idx != 0 or moe.experts_end_idx != moe.n_routed_experts:
        return "partial-experts"
    return None


def prepare(module, mod=None, max_tokens: int = 16) -> int:
    """Pack every MoE layer of ``module`` that the HIP path serves, now (at load,
    before any graph capture), with a workspace for ``max_tokens``: the role of
    the reference's load-time bank layout (serving/partition.py:398-405), so the
    first captured step allocates nothing.  Returns the number of layers packed."""
    mod = mod or _MOD
    n = 0
    for m in module.modules():
        if hasattr(m, "experts") and hasattr(m, "experts_start_idx") and _servable(m, mod) is None:
            h = hip_moe_of(m, mod)
            if h is not None:
                h.reserve(max_tokens)
                n += 1
    return n


def _decline(moe, why, x, input_ids):
    tally = getattr(moe, "_hip_declined", None)
    if tally is None:
        tally = moe._hip_declined = {}
    tally[why] = tally.get(why, 0) + 1
    return _REF_FORWARD(moe, x, input_ids)


def hip_forward(self, x, input_ids):
    """Replacement for MoE.forward(self, x, input_ids) (architecture.py:777-794)."""
    why = _servable(self, _MOD)
    if why is not None:
        return _decline(self, why, x, input_ids)
    h = hip_moe_of(self)
    if h is None:
        return _decline(self, "not-mxfp4-bank", x, input_ids)
    y = h.forward(x, input_ids)
    self._hip_steps = getattr(self, "_hip_steps", 0) + 1
    return y


hip_forward._v4_hip_moe = True


def install(mod) -> bool:
    """Replace mod.MoE.forward with the HIP layer (idempotent, marker ``_v4_hip_moe``)."""
    global _REF_FORWARD, _MOD
    _MOD = mod
    if getattr(mod.MoE.forward, "_v4_hip_moe", False):
        return False
    _REF_FORWARD = mod.MoE.forward
    mod.MoE.forward = hip_forward
    return True


def uninstall(mod) -> bool:
    global _REF_FORWARD
    if _REF_FORWARD is None or not getattr(mod.MoE.forward, "_v4_hip_moe", False):
        return False
    mod.MoE.forward = _REF_FORWARD
    _REF_FORWARD = None
    return True


# ------------------------------------------------------------- the drafter ----
#
# The DSpark drafter's MTP blocks get their MoE forward bound per instance
# (decoding/expert_bank.py:167-191, called from decoding/dspark.py:450-452 when
# V4_DSPARK_MOE is set): an instance attribute, which a class-level
# MoE.forward replacement never reaches.  install_drafter binds the HIP layer
# the same way, so the drafter's MoE runs here instead of the reference's
# TileLang grouped kernel (expert_bank.py:38-60).

V4_DSPARK_MOE = os.environ.get("V4_DSPARK_MOE", "0") not in ("", "0")


def _draft_decline(self, why, x, input_ids):
    """The reference drafter's decline (expert_bank.py:99-105): tally the reason,
    run the class-level forward."""
    tally = getattr(self, "_draft_declined", None)
    if tally is None:
        tally = self._draft_declined = {}
    tally[why] = tally.get(why, 0) + 1
    return type(self).forward(self, x, input_ids)


def hip_draft_forward(self, x, input_ids):
    """Per-instance MoE forward of a drafter MTP block (expert_bank.draft_forward,
    expert_bank.py:108-164): the same routing, experts, shared expert and combine
    as MoE.forward, on the HIP layer.  The HIP layer serves every token count,
    so the reference's width limits (T > 1, T * k <= its 32-row tile) do not
    apply; what it cannot serve declines as the reference's does."""
    if int(getattr(_DRAFT_MOD, "world_size", 1) or 1) > 1:
        return _draft_decline(self, "world_size>1", x, input_ids)
    if self.gate.hash:
        return _draft_decline(self, "hash-routed", x, input_ids)
    if self.experts_start_idx != 0 or self.experts_end_idx != self.n_routed_experts:
        return _draft_decline(self, "partial-experts", x, input_ids)
    h = hip_moe_of(self, _DRAFT_MOD)
    if h is None:
        return _draft_decline(self, "not-mxfp4-bank", x, input_ids)
    y = h.forward(x, input_ids)
    self._draft_steps = getattr(self, "_draft_steps", 0) + 1
    return y


hip_draft_forward._v4_hip_draft = True
_DRAFT_MOD = None


def install_drafter(dstail, mod=None, force: bool = False) -> int:
    """Bind :func:`hip_draft_forward` on each non-hash MoE of ``dstail.mtp`` (the
    reference's install_drafter, expert_bank.py:167-191): only when V4_DSPARK_MOE
    is set, as there, unless ``force``.  ``mod`` is the model module (its
    scale_fmt / scale_dtype / world_size; the reference takes partition.ref()).
    Each bound layer is packed now (its expert weights released, as the
    reference's relayout with preserve=False does).  Returns the number bound."""
    global _DRAFT_MOD
    if not (V4_DSPARK_MOE or force):
        return 0
    _DRAFT_MOD = mod or _MOD
    took = 0
    for blk in dstail.mtp:
        moe = getattr(blk, "ffn", None)
        if moe is None or moe.gate.hash:
            continue
        e0 = moe.experts[moe.experts_start_idx]
        if e0.w1.weight.dtype != torch.float4_e2m1fn_x2 and getattr(moe, "_hip_moe", None) is None:
            continue
        if getattr(moe.forward, "_v4_hip_draft", False):
            continue
        if hip_moe_of(moe, _DRAFT_MOD) is None:
            continue
        moe.forward = hip_draft_forward.__get__(moe, type(moe))
        took += 1
    return took


def uninstall_drafter(dstail) -> int:
    """Remove the per-instance binding (the class-level forward is used again)."""
    n = 0
    for blk in dstail.mtp:
        moe = getattr(blk, "ffn", None)
        if moe is not None and getattr(moe.__dict__.get("forward"), "_v4_hip_draft", False):
            del moe.forward
            n += 1
    return n


def drafter_coverage(dstail) -> dict:
    """Per-layer (steps served, declines by reason) of the drafter's MoEs
    (expert_bank.coverage, expert_bank.py:194-203)."""
    out = {}
    for blk in dstail.mtp:
        moe = blk.ffn
        out[moe.layer_id] = (getattr(moe, "_draft_steps", 0), dict(getattr(moe, "_draft_declined", {})))
    return out


def coverage(module) -> dict:
    """Per-layer (steps served, declines by reason), like fp4_grouped.coverage (:327-336)."""
    out = {}
    mods = module.modules() if hasattr(module, "modules") else [module]
    for m in mods:
        if hasattr(m, "experts") and hasattr(m, "experts_start_idx"):
            out[getattr(m, "layer_id", len(out))] = (
                getattr(m, "_hip_steps", 0), dict(getattr(m, "_hip_declined", {})))
    return out


# Install markers of the MoE.forward replacements the reference ships
# (serving/controls.py:38-42), with the labels its moe_chain prints.
_CHAIN_MARKERS = (("_v4_hip_moe", "hip"), ("_v4_multi", "multi"), ("_v4_grouped", "grouped"),
                  ("_v4_decode_fast", "decode"))


def moe_chain(mod) -> list:
    """The installed MoE.forward chain, outermost first (controls.moe_chain,
    serving/controls.py:45-68): each replacement is recognised by its marker and
    followed to the forward it kept (``_REF_FORWARD`` of the module that defines
    it); the chain ends at ``"ref"``, ``"ORPHAN"`` (a marked forward whose module
    is gone) or ``"CYCLE"``."""
    import sys

    fn = getattr(getattr(mod, "MoE", None), "forward", None)
    out, seen = [], set()
    while fn is not None:
        if id(fn) in seen:
            out.append("CYCLE")
            break
        seen.add(id(fn))
        label = next((lab for marker, lab in _CHAIN_MARKERS if getattr(fn, marker, False)), None)
        if label is None:
            out.append("ref")
            break
        out.append(label)
        owner = sys.modules.get(getattr(fn, "__module__", "") or "")
        if owner is None:
            out.append("ORPHAN")
            break
        fn = getattr(owner, "_REF_FORWARD", None)
    return out
