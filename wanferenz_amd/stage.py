"""A decode stage: blocks of FP8 projections + RMSNorm + residual around the MoE layer.

The step on either side of the MoE in a decoder block (Block.forward,
architecture.py:853-874): the pre-norms (RMSNorm, :217-230), the FP8 linears of
the attention side (linear(), :121-132) and the MoE (:777-794), chained over a
stack of blocks and captured as one HIP graph per step, the way the reference
captures its decode step (decoder.py:465-488).  Two simplifications keep this
to the kernels on the measured path: the hyper-connection mixing
(hc_pre / hc_post, :821-850) is a plain residual add, and attention itself
(sparse_attn) is not run — its projections are, with their outputs feeding the
chain where the shapes allow.

Per block, with h the [T, D] residual stream (bf16):

    a = rms_norm(h, attn_norm)
    u = P_down(a)            N x K = q_dim x D     (e.g. 1024 x 4096)
    v = P_up(u)              D x q_dim             (4096 x 1024)
    w = P_sq(v)              D x D                 (4096 x 4096)
    z = P_wide(a)            wide x D              (16384 x 4096; consumed by attention)
    h = h + w
    m = rms_norm(h, ffn_norm)
    h = h + moe(m)

Every buffer is allocated once, so a step is a fixed sequence of launches.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Sequence

import torch

from . import kernels
from . import synth


@dataclass
class StageBlock:
    attn_norm: torch.Tensor          # fp32 [D]
    ffn_norm: torch.Tensor           # fp32 [D]
    p_down: kernels.PackedFp8Linear  # [q, D]
    p_up: kernels.PackedFp8Linear    # [D, q]
    p_sq: kernels.PackedFp8Linear    # [D, D]
    p_wide: kernels.PackedFp8Linear  # [wide, D]
    moe: object                      # HipMoE


def synthetic_linear(N: int, K: int, seed: int, device, fp32_scales: bool = True):
    """(e4m3 weight [N, K], scales [N/128, K/128]) on the device: NaN codes replaced,
    float32 scales U[0.5, 1.5) (fp8_vector.py:185-232) or e8m0 2^-15..2^-11."""
    w = torch.empty(N, K, dtype=torch.uint8, device=device)
    synth.device_fill(w, synth.stream_key(seed, synth.S_FP8_W), synth.FILL_E4M3)
    nb, kb = (N + 127) // 128, (K + 127) // 128
    if fp32_scales:
        s = torch.empty(nb, kb, dtype=torch.float32, device=device)
        synth.device_fill(s, synth.stream_key(seed, synth.S_FP8_W_S), synth.FILL_F32_UNIFORM, 0.5, 1.5)
    else:
        s = torch.empty(nb, kb, dtype=torch.uint8, device=device)
        synth.device_fill(s, synth.stream_key(seed, synth.S_FP8_W_S), synth.FILL_E8M0, 112, 116)
        s = s.view(torch.float8_e8m0fnu)
    return w.view(torch.float8_e4m3fn), s


def synthetic_block(moe, D: int, q_dim: int, wide: int, seed: int, device) -> StageBlock:
    """Projections with e8m0 block scales (the model's FP8 weights carry e8m0 scales,
    architecture.py:158-168); 2^-15..2^-11 keeps a K = 4096 product of uniform e4m3
    codes O(1), so the residual stream keeps its scale block after block."""
    lins = []
    for j, (N, K) in enumerate(((q_dim, D), (D, q_dim), (D, D), (wide, D))):
        w, s = synthetic_linear(N, K, seed * 16 + j, device, fp32_scales=False)
        lins.append(kernels.PackedFp8Linear(w, s, "ue8m0"))
    norms = []
    for j in range(2):
        t = torch.empty(D, dtype=torch.float32, device=device)
        synth.device_fill(t, synth.stream_key(seed * 16 + 8 + j, synth.S_NORM), synth.FILL_F32_UNIFORM, 0.5, 1.5)
        norms.append(t)
    return StageBlock(norms[0], norms[1], *lins, moe)


class DecodeStage:
    """A stack of StageBlocks at a fixed token count T; ``step`` runs it eagerly,
    ``capture`` records one step as a graph, ``replay`` runs the graph."""

    def __init__(self, blocks: Sequence[StageBlock], T: int, eps: float = 1e-6):
        self.blocks: List[StageBlock] = list(blocks)
        self.T, self.eps = T, eps
        b0 = self.blocks[0]
        D, dev = b0.p_sq.N, b0.p_sq.packed.device
        self.D = D
        bf = dict(dtype=torch.bfloat16, device=dev)
        self.x_in = torch.zeros(T, D, **bf)
        self.h = torch.zeros(T, D, **bf)
        self.a = torch.empty(T, D, **bf)
        self.u = torch.empty(T, b0.p_down.N, **bf)
        self.v = torch.empty(T, D, **bf)
        self.w = torch.empty(T, D, **bf)
        self.z = torch.empty(T, b0.p_wide.N, **bf)
        self.m = torch.empty(T, D, **bf)
        self.e = torch.empty(T, D, **bf)
        for b in self.blocks:
            for lin in (b.p_down, b.p_up, b.p_sq, b.p_wide):
                lin.reserve(T)
            b.moe.reserve(T)
        self.graph = None

    def _run(self, routing=None, trace=None):
        T, eps = self.T, self.eps
        self.h.copy_(self.x_in)
        for i, b in enumerate(self.blocks):
            h_in = None if trace is None else self.h.clone()
            kernels.rms_norm(self.h, b.attn_norm, eps, out=self.a)
            b.p_down(self.a, out=self.u)
            b.p_up(self.u, out=self.v)
            b.p_sq(self.v, out=self.w)
            b.p_wide(self.a, out=self.z)
            kernels.add(self.h, self.w, out=self.h)
            h_mid = None if trace is None else self.h.clone()
            kernels.rms_norm(self.h, b.ffn_norm, eps, out=self.m)
            b.moe.forward(self.m, out=self.e, routing_out=None if routing is None else routing[i])
            kernels.add(self.h, self.e, out=self.h)
            if trace is not None:
                trace.append({"h_in": h_in, "a": self.a.clone(), "u": self.u.clone(), "v": self.v.clone(),
                              "w": self.w.clone(), "z": self.z.clone(), "h_mid": h_mid, "m": self.m.clone(),
                              "e": self.e.clone(), "h_out": self.h.clone()})
        return self.h

    def step(self, x: torch.Tensor, routing=None, trace=None) -> torch.Tensor:
        """One eager step.  ``routing``: optional per-block (weights [T, k] fp32,
        indices [T, k] int64) buffers that receive each MoE's routing; ``trace``:
        optional list that receives a dict of every block's intermediates."""
        self.x_in.copy_(x)
        return self._run(routing, trace)

    def capture(self):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self._run()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._run()
        self.graph = g
        return g

    def replay(self, x: torch.Tensor) -> torch.Tensor:
        self.x_in.copy_(x)
        self.graph.replay()
        return self.h
