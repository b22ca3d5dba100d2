"""Torch float32 restatement of the reference's CPU path for one MoE layer.

Test and benchmark infrastructure (the CPU baseline and a second checker),
never the product path.  It follows, op for op in torch CPU ops:

- wanferenz/kernels/torch_ops.py:17-49 (``_round_scale``, ``act_quant``),
  :79-108 (``_dequant``, ``unpack_fp4``, ``fp8_gemm``, ``fp4_gemm``);
- wanferenz/model/architecture.py:121-132 (``linear``), :696-718
  (``Gate.forward``), :729-741 (``Expert.forward``), :777-794
  (``MoE.forward``).

Pinned by tests/test_oracle_torch.py against the golden vectors that
tests/golden/make_golden.py wrote from the reference's own CPU path, and
against the numpy oracle (oracle/moe.py) on the same inputs.

Weights are held as the checkpoint stores them: FP4 experts as packed e2m1
bytes with per-32 e8m0 scales (decoded to float32 here), the FP8 shared expert
as e4m3 bytes with 128 x 128 block scales.  Every call dequantises the weights
it multiplies, as torch_ops.fp4_gemm / fp8_gemm do.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F

FP8_MAX = 448.0
_E2M1 = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)
_FP4_TABLE = torch.tensor(_E2M1 + tuple(-v for v in _E2M1), dtype=torch.float32)


def round_scale(amax: torch.Tensor, max_inv: float) -> torch.Tensor:
    """2^ceil(log2(amax * max_inv)) by frexp (torch_ops.py:17-21)."""
    x = amax * max_inv
    mant, exp = torch.frexp(x)
    return torch.ldexp(torch.ones_like(x), torch.where(mant == 0.5, exp - 1, exp))


def act_quant(x: torch.Tensor, round_pow2: bool, block: int = 128) -> Tuple[torch.Tensor, torch.Tensor]:
    """torch_ops.py:33-49: per-row, per-128 e4m3 codes (float8 tensor) and float32 scales."""
    n = x.size(-1)
    z = x.contiguous().float().unflatten(-1, (n // block, block))
    amax = z.abs().amax(-1, keepdim=True).clamp_min(1e-4)
    s = round_scale(amax, 1.0 / FP8_MAX) if round_pow2 else amax * (1.0 / FP8_MAX)
    q = (z / s).clamp(-FP8_MAX, FP8_MAX)
    return q.to(torch.float8_e4m3fn).flatten(-2), s.squeeze(-1)


def _dequant(v: torch.Tensor, s: torch.Tensor, block: int) -> torch.Tensor:
    return v.float() * s.float().repeat_interleave(block, -1)[..., : v.size(-1)]


def unpack_fp4(b: torch.Tensor) -> torch.Tensor:
    """torch_ops.py:84-92: packed e2m1 bytes [N, K/2] -> float32 [N, K], low nibble first."""
    u = b.view(torch.uint8)
    t = _FP4_TABLE.to(u.device)
    return torch.stack([t[(u & 0x0F).long()], t[(u >> 4).long()]], dim=-1).flatten(-2)


def fp8_gemm(a, a_s, w_codes, w_s, out_dtype=torch.bfloat16) -> torch.Tensor:
    """torch_ops.py:93-99 with the weight as e4m3 bytes [N, K] and float32 block scales."""
    k, n = a.size(-1), w_codes.size(0)
    da = _dequant(a.reshape(-1, k), a_s.reshape(-1, a_s.size(-1)), 128)
    db = _dequant(w_codes.view(torch.float8_e4m3fn), w_s.repeat_interleave(128, 0)[:n], 128)
    return (da @ db.t()).view(*a.shape[:-1], n).to(out_dtype)


def fp4_gemm(a, a_s, w_packed, w_s, out_dtype=torch.bfloat16) -> torch.Tensor:
    """torch_ops.py:102-108 with float32 per-32 weight scales [N, K/32]."""
    k, n = a.size(-1), w_packed.size(0)
    da = _dequant(a.reshape(-1, k), a_s.reshape(-1, a_s.size(-1)), 128)
    db = unpack_fp4(w_packed) * w_s.float().repeat_interleave(32, -1)[:, :k]
    return (da @ db.t()).view(*a.shape[:-1], n).to(out_dtype)


@dataclass
class QLinear:
    """A quantised weight: kind "fp4" (packed bytes [N, K/2], scales [N, K/32]) or
    "fp8" (e4m3 bytes [N, K], scales [ceil(N/128), K/128]); scales are float32."""
    kind: str
    weight: torch.Tensor
    scale: torch.Tensor


def linear(x: torch.Tensor, w: QLinear, round_pow2: bool) -> torch.Tensor:
    """architecture.py:121-132 for a quantised weight: act_quant, then the scaled GEMM."""
    q, s = act_quant(x, round_pow2)
    return (fp4_gemm if w.kind == "fp4" else fp8_gemm)(q, s, w.weight, w.scale)


def expert_forward(ws: Sequence[QLinear], x: torch.Tensor, weights: Optional[torch.Tensor],
                   swiglu_limit: float, round_pow2: bool) -> torch.Tensor:
    """architecture.py:729-741: clamp-SwiGLU on w1/w3, the routing weight, then w2."""
    w1, w3, w2 = ws
    dtype = x.dtype
    gate = linear(x, w1, round_pow2).float()
    up = linear(x, w3, round_pow2).float()
    if swiglu_limit > 0:
        up = torch.clamp(up, min=-swiglu_limit, max=swiglu_limit)
        gate = torch.clamp(gate, max=swiglu_limit)
    h = F.silu(gate) * up
    if weights is not None:
        h = weights * h
    return linear(h.to(dtype), w2, round_pow2)


def gate_forward(x: torch.Tensor, gate_w: torch.Tensor, bias: Optional[torch.Tensor], topk: int,
                 score_func: str, route_scale: float, tid2eid: Optional[torch.Tensor] = None,
                 input_ids: Optional[torch.Tensor] = None):
    """architecture.py:696-718 -> (weights, indices, biased scores)."""
    scores = F.linear(x.float(), gate_w.float())
    if score_func == "softmax":
        scores = scores.softmax(dim=-1)
    elif score_func == "sigmoid":
        scores = scores.sigmoid()
    else:
        scores = F.softplus(scores).sqrt()
    original = scores
    if bias is not None:
        scores = scores + bias
    if tid2eid is not None:
        indices = tid2eid[input_ids]
    else:
        indices = scores.topk(topk, dim=-1)[1]
    weights = original.gather(1, indices.long())
    if score_func != "softmax":
        weights /= weights.sum(dim=-1, keepdim=True)
    weights *= route_scale
    return weights, indices, scores


@dataclass
class MoELayer:
    gate_w: torch.Tensor                  # bf16 [E, D]
    gate_bias: Optional[torch.Tensor]     # float32 [E]
    experts: Dict[int, Sequence[QLinear]]  # the routed experts present (w1, w3, w2)
    shared: Sequence[QLinear]             # FP8 (w1, w3, w2)
    n_experts: int
    topk: int
    score_func: str = "sqrtsoftplus"
    route_scale: float = 1.5
    swiglu_limit: float = 10.0
    round_pow2: bool = True
    tid2eid: Optional[torch.Tensor] = None


def moe_forward(p: MoELayer, x: torch.Tensor, input_ids: Optional[torch.Tensor] = None):
    """architecture.py:777-794 -> (y bf16 [T, D], weights, indices).  A routed expert
    missing from ``p.experts`` raises (the caller supplies every selected one)."""
    weights, indices, _ = gate_forward(x, p.gate_w, p.gate_bias, p.topk, p.score_func, p.route_scale,
                                       p.tid2eid, input_ids)
    y = torch.zeros_like(x, dtype=torch.float32)
    counts = torch.bincount(indices.flatten().long(), minlength=p.n_experts).tolist()
    for i in range(p.n_experts):
        if counts[i] == 0:
            continue
        idx, top = torch.where(indices == i)
        y[idx] += expert_forward(p.experts[i], x[idx], weights[idx, top, None], p.swiglu_limit, p.round_pow2)
    y += expert_forward(p.shared, x, None, p.swiglu_limit, p.round_pow2)
    return y.type_as(x), weights, indices


def near_ties(biased_scores: torch.Tensor, topk: int, rel: float = 2.0 ** -20) -> list:
    """Tokens whose k-th and (k+1)-th selection keys differ by at most ``rel`` of the
    k-th: a one-ulp difference in the logits may swap the last expert."""
    top = biased_scores.float().topk(topk + 1, dim=-1)[0]
    gap = (top[:, topk - 1] - top[:, topk]).abs()
    return torch.nonzero(gap <= rel * top[:, topk - 1].abs()).flatten().tolist()
