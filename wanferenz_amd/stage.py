"""A decode stage: V4 decoder blocks' FP8 projections, norms and residuals around the MoE.

The step on either side of the MoE in a decoder block (Block.forward,
architecture.py:853-874) at the V4-Flash projection shapes, chained over a
stack of blocks and captured as one HIP graph per step, the way the reference
captures its decode step (decoder.py:465-488).  The attention side runs every
FP8 projection of Attention.forward (architecture.py:611-672) and of the
indexer on its real input: wq_a and wkv on the normed hidden state, q_norm,
then wq_b and the indexer's wq_b on the normed query latent (fp8_vector.py:505-513
lists the same five shapes).  Attention itself, its rotary embedding and the
bf16 grouped wo_a product are not run (sparse_attn is measured on its own), so
the input of wo_b — [T, n_groups * o_lora_rank] — is taken from the indexer's
query projection, which has that width at V4 (8192).  The hyper-connection
mixing (hc_pre / hc_post, :821-850) is a plain residual add.

Per block, with h the [T, D] residual stream (bf16):

    (h, hq) = add_rms_norm_quant(h, e_prev, attn_norm)   # block 0: rms_norm_quant(h)
    qa = wq_a(hq)                 q_lora x D        (1024 x 4096)
    kv = wkv(hq)                  head_dim x D      (512 x 4096)
    qq = rms_norm_quant(qa, q_norm)
    q  = wq_b(qq)                 heads*hd x q_lora (32768 x 1024)
    iq = idx_wq_b(qq)             idx x q_lora      (8192 x 1024)
    h1 = h + wo_b(iq)             D x o             (4096 x 8192), residual in the epilogue
    m  = rms_norm(h1, ffn_norm)
    e  = moe(m)
    (after the last block: h = h1 + e)

The two projections that read one input run as one launch (wq_a with wkv,
wq_b with the indexer's wq_b: kernels.PackedFp8Pair), and the norm that feeds
them (attn_norm with the previous block's MoE residual, q_norm) runs inside
that launch (PackedFp8Pair.norm_gemm: the rms_norm_quant codes, bit for bit)
when T fits its rows (T <= 4); otherwise each FP8 input is produced quantised
by the norm that precedes it (rms_norm_quant).  With the fused norms the
ffn_norm runs inside the MoE layer's routing launch as well
(HipMoE.forward_norm: the rms_norm output, bit for bit).  The residual add of the
attention side sits in wo_b's epilogue and that of the MoE side in the next
block's norm.  Every buffer is allocated once, so a step is a fixed sequence of
launches.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Sequence

import torch

from . import kernels
from . import synth

# V4-Flash attention-side widths (architecture.py ModelArgs): q_lora_rank,
# head_dim, n_heads * head_dim, index_n_heads * index_head_dim.
V4_DIMS = dict(q_lora=1024, head_dim=512, q_width=32768, idx_width=8192)


@dataclass
class StageBlock:
    attn_norm: torch.Tensor              # fp32 [D]
    q_norm: torch.Tensor                 # fp32 [q_lora]
    ffn_norm: torch.Tensor               # fp32 [D]
    qa_kv: kernels.PackedFp8Pair         # wq_a [q_lora, D] and wkv [head_dim, D], one launch
    q_idx: kernels.PackedFp8Pair         # wq_b [q_width, q_lora] and idx wq_b [idx_width, q_lora]
    wo_b: kernels.PackedFp8Linear        # [D, idx_width]
    moe: object                          # HipMoE


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


def projection_shapes(D: int, q_lora: int, head_dim: int, q_width: int, idx_width: int):
    """(N, K) of wq_a, wkv, wq_b, idx_wq_b, wo_b."""
    return ((q_lora, D), (head_dim, D), (q_width, q_lora), (idx_width, q_lora), (D, idx_width))


def synthetic_block(moe, D: int, seed: int, device, q_lora: int = 1024, head_dim: int = 512,
                    q_width: int = 32768, idx_width: int = 8192) -> StageBlock:
    """Projections with e8m0 block scales (the model's FP8 weights carry e8m0 scales,
    architecture.py:158-168); 2^-15..2^-11 keeps a K = 4096 product of uniform e4m3
    codes O(1), so the residual stream keeps its scale block after block."""
    ws = [synthetic_linear(N, K, seed * 16 + j, device, fp32_scales=False)
          for j, (N, K) in enumerate(projection_shapes(D, q_lora, head_dim, q_width, idx_width))]
    norms = []
    for j, n in enumerate((D, q_lora, D)):
        t = torch.empty(n, dtype=torch.float32, device=device)
        synth.device_fill(t, synth.stream_key(seed * 16 + 8 + j, synth.S_NORM), synth.FILL_F32_UNIFORM, 0.5, 1.5)
        norms.append(t)
    return StageBlock(norms[0], norms[1], norms[2], kernels.PackedFp8Pair(*ws[0], *ws[1], "ue8m0"),
                      kernels.PackedFp8Pair(*ws[2], *ws[3], "ue8m0"), kernels.PackedFp8Linear(*ws[4], "ue8m0"), moe)


class DecodeStage:
    """A stack of StageBlocks at a fixed token count T; ``step`` runs it eagerly,
    ``capture`` records one step as a graph, ``replay`` runs the graph."""

    def __init__(self, blocks: Sequence[StageBlock], T: int, eps: float = 1e-6, fused_norms: bool = True):
        self.blocks: List[StageBlock] = list(blocks)
        self.T, self.eps = T, eps
        b0 = self.blocks[0]
        D, dev = b0.wo_b.N, b0.wo_b.packed.device
        self.D = D
        bf = dict(dtype=torch.bfloat16, device=dev)

        def q8(n):
            return (torch.empty(T, n, dtype=kernels._E4M3, device=dev),
                    torch.empty(T, n // 128, dtype=kernels._E8M0, device=dev))

        self.x_in = torch.zeros(T, D, **bf)
        # the residual stream: each new value goes to the next of three buffers, so
        # no kernel writes the buffer it reads
        self.h = [torch.zeros(T, D, **bf) for _ in range(3)]
        self.hq = q8(D)
        self.qa = torch.empty(T, b0.qa_kv.N0, **bf)
        self.kv = torch.empty(T, b0.qa_kv.N1, **bf)
        self.qq = q8(b0.qa_kv.N0)
        self.q = torch.empty(T, b0.q_idx.N0, **bf)
        self.iq = torch.empty(T, b0.q_idx.N1, **bf)
        self.m = torch.empty(T, D, **bf)
        self.e = torch.empty(T, D, **bf)
        self.y = torch.empty(T, D, **bf)
        for b in self.blocks:
            for lin in (b.qa_kv, b.q_idx, b.wo_b):
                lin.reserve(T)
            b.moe.reserve(T)
        # the norms ride in the projections' launches when T fits the fused path
        self.fused_norms = fused_norms and all(
            T <= kernels.norm_linear_rows(lin.K) for b in self.blocks for lin in (b.qa_kv, b.q_idx))
        self.graph = None

    def _run(self, routing=None, trace=None):
        eps = self.eps
        h = self.x_in
        nxt = iter(self.h * (2 * len(self.blocks)))
        for i, b in enumerate(self.blocks):
            h_in, e_in = (None, None) if trace is None else (h.clone(), None if i == 0 else self.e.clone())
            if self.fused_norms:
                # attn_norm (with the previous block's MoE residual) and q_norm run
                # inside the projections' launches, on the codes the unfused norms
                # give; a trace records those codes from the unfused kernels
                if i == 0:
                    b.qa_kv.norm_gemm(h, b.attn_norm, eps, out=(self.qa, self.kv))
                else:
                    hs = next(nxt)
                    b.qa_kv.norm_gemm(h, b.attn_norm, eps, b=self.e, sum_out=hs, out=(self.qa, self.kv))
                    h = hs
                b.q_idx.norm_gemm(self.qa, b.q_norm, eps, out=(self.q, self.iq))
                if trace is not None:
                    kernels.rms_norm_quant(h, b.attn_norm, eps, out=self.hq)
                    kernels.rms_norm_quant(self.qa, b.q_norm, eps, out=self.qq)
            else:
                if i == 0:
                    kernels.rms_norm_quant(h, b.attn_norm, eps, out=self.hq)
                else:
                    # the previous block's MoE residual, fused into this block's norm
                    hs = next(nxt)
                    kernels.add_rms_norm_quant(h, self.e, b.attn_norm, eps, sum_out=hs, out=self.hq)
                    h = hs
                b.qa_kv.gemm(*self.hq, out=(self.qa, self.kv))
                kernels.rms_norm_quant(self.qa, b.q_norm, eps, out=self.qq)
                b.q_idx.gemm(*self.qq, out=(self.q, self.iq))
            h1 = next(nxt)
            b.wo_b(self.iq, out=h1, residual=h)
            ro = None if routing is None else routing[i]
            if self.fused_norms and trace is None:
                b.moe.forward_norm(h1, b.ffn_norm, eps, out=self.e, routing_out=ro)
            else:
                kernels.rms_norm(h1, b.ffn_norm, eps, out=self.m)
                b.moe.forward(self.m, out=self.e, routing_out=ro)
            if trace is not None:
                trace.append({"h_in": h_in, "e_in": e_in, "h": h.clone(), "hq": self.hq[0].clone(),
                              "hs": self.hq[1].clone(), "qa": self.qa.clone(), "kv": self.kv.clone(),
                              "qq": self.qq[0].clone(), "qs": self.qq[1].clone(), "q": self.q.clone(),
                              "iq": self.iq.clone(), "h1": h1.clone(), "m": self.m.clone(), "e": self.e.clone()})
            h = h1
        kernels.add(h, self.e, out=self.y)
        return self.y

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
        return self.y
