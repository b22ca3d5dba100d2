"""ORACLE (test infrastructure only): CPU restatement of the reference MoE + FP8-linear path.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this module, and only as the checker: the product never calls it.

Each function restates the reference's CPU semantics (wanferenz/kernels/
torch_ops.py and wanferenz/model/architecture.py) with numpy, keeping the
reference's rounding points (fp32 intermediates, bf16 outputs of every
linear).  Matrix products are accumulated in float64 and rounded to float32
once, which is the exactly-rounded value every fp32 accumulation order
approximates; the tests therefore compare floating outputs by tolerance and
integer outputs (expert ids, permutation) bit-exactly.

Parity status per function (how each is pinned; see tests/test_oracle_*.py):

* act_quant            known answers + brute force over e4m3 + reference golden vectors
* fp8_gemm / fp4_gemm  exactness-constructed cases (bit-exact) + float64 brute force
                       + reference golden vectors
* gate                 closed form + reference golden vectors (indices bit-exact,
                       near-tie margins recorded)
* permutation          stable counting sort == brute-force sort by (expert, token, slot)
* expert / moe_forward reference golden vectors (end-to-end MoE.forward of the
                       reference CPU path, toy config and hash-routed layer)
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import numpy as np

from .numerics import (
    FP8_MAX,
    bf16_round,
    e2m1_decode_nibbles,
    e4m3_decode,
    e4m3_encode,
    e8m0_decode,
)

F32_INV448 = np.float32(1.0 / 448.0)


def round_scale(x: np.ndarray) -> np.ndarray:
    """2^ceil(log2(x)) for float32 x > 0 (torch_ops.py:17-21, frexp form).

    frexp gives x = m * 2^e with m in [0.5, 1); an exact power of two has
    m == 0.5 and keeps its exponent, anything else rounds up.
    """
    x = np.asarray(x, dtype=np.float32)
    m, e = np.frexp(x)
    e = np.where(m == 0.5, e - 1, e)
    # frexp of NaN / inf: torch returns exponent 0, so the scale is 1 (numpy's
    # exponent for them is platform-defined; fix it here)
    e = np.where(np.isfinite(x), e, 0)
    return np.ldexp(np.float32(1.0), e).astype(np.float32)


def act_quant(x: np.ndarray, block: int = 128, round_pow2: bool = True):
    """Per-row, per-``block`` dynamic FP8 quantisation (torch_ops.py:33-49).

    x: float32 array [..., K] holding bf16 values.  Returns (q uint8 e4m3
    codes [..., K], s float32 [..., K/block]).  ``round_pow2`` is the
    reference's ``scale_fmt is not None`` (ue8m0 scales).
    """
    x = np.asarray(x, dtype=np.float32)
    K = x.shape[-1]
    if K % block:
        raise ValueError(f"act_quant: last dim {K} not a multiple of {block}")
    z = x.reshape(x.shape[:-1] + (K // block, block))
    amax = np.maximum(np.abs(z).max(axis=-1, keepdims=True), np.float32(1e-4))  # both keep NaN, as torch
    s = round_scale(amax * F32_INV448) if round_pow2 else (amax * F32_INV448).astype(np.float32)
    q = np.clip(z / s, np.float32(-FP8_MAX), np.float32(FP8_MAX)).astype(np.float32)
    codes = e4m3_encode(q).reshape(x.shape)
    return codes, s[..., 0].astype(np.float32)


BF16_MAX = np.float32(3.3895313892515355e38)


def wire_pack(x: np.ndarray):
    """The FP8 wire format of a stage boundary (_pack_t, serving/chain.py:208-217).

    Per row (last dim): scale = bf16(clamp(amax / 448, 1e-8, bf16 max)) in fp32
    arithmetic, q = e4m3(clamp(x / scale, +-448)).  Returns (q uint8 codes, scale
    float32 holding bf16 values [...]).
    """
    f = np.asarray(x, dtype=np.float32)
    amax = np.abs(f).max(axis=-1, keepdims=True)
    scale = bf16_round(np.clip(amax / np.float32(448.0), np.float32(1e-8), BF16_MAX).astype(np.float32))
    q = np.clip(f / scale, np.float32(-FP8_MAX), np.float32(FP8_MAX)).astype(np.float32)
    return e4m3_encode(q), scale[..., 0]


def wire_unpack(q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """_unpack_t (chain.py:220-222): bf16(q) * scale in bf16 -> bf16 values as float32."""
    v = e4m3_decode(q).astype(np.float32)
    return bf16_round((v * np.asarray(scale, np.float32)[..., None]).astype(np.float32))


def dequant_act(q: np.ndarray, s: np.ndarray, block: int = 128) -> np.ndarray:
    v = e4m3_decode(q).astype(np.float64)
    return v * np.repeat(np.asarray(s, dtype=np.float64), block, axis=-1)[..., : v.shape[-1]]


def dequant_fp8_weight(w: np.ndarray, w_s: np.ndarray, block: int = 128) -> np.ndarray:
    """e4m3 [N, K] with block scales [ceil(N/128), ceil(K/128)] -> float64 [N, K]."""
    N, K = w.shape
    s = np.asarray(w_s, dtype=np.float64)
    s = np.repeat(np.repeat(s, block, axis=0)[:N], block, axis=1)[:, :K]
    return e4m3_decode(w).astype(np.float64) * s


def dequant_fp4_weight(w: np.ndarray, w_s: np.ndarray, block: int = 32) -> np.ndarray:
    """packed e2m1 [N, K/2] with e8m0-valued scales [N, K/32] -> float64 [N, K]."""
    v = e2m1_decode_nibbles(w).astype(np.float64)
    return v * np.repeat(np.asarray(w_s, dtype=np.float64), block, axis=-1)[:, : v.shape[-1]]


def _to_bf16(c64: np.ndarray) -> np.ndarray:
    return bf16_round(c64.astype(np.float32))


def fp8_gemm(a, a_s, w, w_s) -> np.ndarray:
    """C = dequant(a) @ dequant(w)^T -> bf16 values as float32 (torch_ops.py:93-99)."""
    da = dequant_act(a, a_s)
    return _to_bf16(da @ dequant_fp8_weight(w, w_s).T)


def fp4_gemm(a, a_s, w, w_s) -> np.ndarray:
    """C = dequant(a) @ (unpack_fp4(w) * w_s)^T -> bf16 values (torch_ops.py:102-108)."""
    da = dequant_act(a, a_s)
    return _to_bf16(da @ dequant_fp4_weight(w, w_s).T)


# ---------------------------------------------------------------- gate --------


def softplus_f32(a32: np.ndarray) -> np.ndarray:
    """torch F.softplus(beta=1, threshold=20) evaluated exactly, rounded to fp32."""
    a = np.asarray(a32, dtype=np.float64)
    out = np.where(a > 20.0, a, np.log1p(np.exp(np.minimum(a, 20.0))))
    return out.astype(np.float32)


def gate_scores(x: np.ndarray, W: np.ndarray, score_func: str = "sqrtsoftplus") -> np.ndarray:
    """Routing scores before the bias (architecture.py:696-705).

    x: [T, D] bf16 values, W: [E, D] bf16 values.  The product is exact in
    float64 (bf16 x bf16 fits 16 bits) and the 4096-term sum is rounded once
    to float32.
    """
    a32 = (np.asarray(x, np.float64) @ np.asarray(W, np.float64).T).astype(np.float32)
    if score_func == "softmax":
        a = a32.astype(np.float64)
        e = np.exp(a - a.max(-1, keepdims=True))
        return (e / e.sum(-1, keepdims=True)).astype(np.float32)
    if score_func == "sigmoid":
        return (1.0 / (1.0 + np.exp(-a32.astype(np.float64)))).astype(np.float32)
    sp = softplus_f32(a32)
    return np.sqrt(sp.astype(np.float64)).astype(np.float32)


def topk_desc(b: np.ndarray, k: int) -> np.ndarray:
    """Indices of the k largest values per row, descending; ties -> lower index."""
    T, E = b.shape
    order = np.lexsort((np.broadcast_to(np.arange(E), (T, E)), -b.astype(np.float64)), axis=-1)
    return order[:, :k].astype(np.int64)


@dataclass
class GateResult:
    weights: np.ndarray   # [T, k] float32
    indices: np.ndarray   # [T, k] int64
    scores: np.ndarray    # [T, E] float32 (after score_func, before bias)
    biased: np.ndarray    # [T, E] float32 (selection scores)
    margin: np.ndarray    # [T] float32: k-th minus (k+1)-th biased score (inf for hash)


def gate(
    x,
    W,
    bias: Optional[np.ndarray],
    k: int,
    score_func: str = "sqrtsoftplus",
    route_scale: float = 1.0,
    tid2eid: Optional[np.ndarray] = None,
    input_ids: Optional[np.ndarray] = None,
) -> GateResult:
    """Gate.forward (architecture.py:696-718)."""
    s = gate_scores(x, W, score_func)
    b = s + np.asarray(bias, np.float32) if bias is not None else s
    b = b.astype(np.float32)
    T, E = s.shape
    if tid2eid is not None:
        idx = np.asarray(tid2eid)[np.asarray(input_ids).reshape(-1)].astype(np.int64)
        margin = np.full(T, np.inf, np.float32)
    else:
        idx = topk_desc(b, k)
        srt = np.sort(b, axis=-1)[:, ::-1]
        margin = (srt[:, k - 1] - srt[:, k]) if E > k else np.full(T, np.inf, np.float32)
    w = np.take_along_axis(s, idx, axis=1).astype(np.float32)
    if score_func != "softmax":
        tot = np.zeros(T, np.float32)
        for j in range(idx.shape[1]):
            tot = (tot + w[:, j]).astype(np.float32)
        w = (w / tot[:, None]).astype(np.float32)
    w = (w * np.float32(route_scale)).astype(np.float32)
    return GateResult(w, idx, s, b, np.asarray(margin, np.float32))


# ---------------------------------------------------------- permutation --------


def permutation(indices: np.ndarray, n_experts: int):
    """Canonical expert-major order of (token, slot) pairs (expert_batch.py:24-37).

    Experts ascending; within an expert, tokens ascending, then slot.  Returns
    (counts [E], offsets [E+1], perm_token [P], perm_slot [P]).
    """
    idx = np.asarray(indices, dtype=np.int64)
    T, k = idx.shape
    counts = np.bincount(idx.reshape(-1), minlength=n_experts).astype(np.int32)
    offsets = np.zeros(n_experts + 1, np.int32)
    offsets[1:] = np.cumsum(counts)
    cursor = offsets[:-1].copy()
    perm_token = np.empty(T * k, np.int32)
    perm_slot = np.empty(T * k, np.int32)
    for t in range(T):
        for j in range(k):
            e = idx[t, j]
            p = cursor[e]
            perm_token[p] = t
            perm_slot[p] = j
            cursor[e] += 1
    return counts, offsets, perm_token, perm_slot


# -------------------------------------------------------------- experts --------


@dataclass
class Fp4Linear:
    weight: np.ndarray   # uint8 [N, K/2] packed e2m1
    scale: np.ndarray    # float32 [N, K/32] powers of two (e8m0 values)

    def __call__(self, x, round_pow2):
        q, s = act_quant(x, 128, round_pow2)
        return fp4_gemm(q, s, self.weight, self.scale)


@dataclass
class Fp8Linear:
    weight: np.ndarray   # uint8 [N, K] e4m3
    scale: np.ndarray    # float32 [ceil(N/128), ceil(K/128)]

    def __call__(self, x, round_pow2):
        q, s = act_quant(x, 128, round_pow2)
        return fp8_gemm(q, s, self.weight, self.scale)


def silu_f32(g: np.ndarray) -> np.ndarray:
    g64 = np.asarray(g, np.float64)
    return (g64 / (1.0 + np.exp(-g64))).astype(np.float32)


def expert_forward(x, w1, w3, w2, weights=None, swiglu_limit=0.0, round_pow2=True):
    """Expert.forward (architecture.py:729-741); x: [n, D] bf16 values."""
    g = w1(x, round_pow2).astype(np.float32)
    u = w3(x, round_pow2).astype(np.float32)
    if swiglu_limit > 0:
        L = np.float32(swiglu_limit)
        u = np.clip(u, -L, L)
        g = np.minimum(g, L)
    h = (silu_f32(g) * u).astype(np.float32)
    if weights is not None:
        h = (np.asarray(weights, np.float32) * h).astype(np.float32)
    return w2(bf16_round(h), round_pow2)


@dataclass
class MoEParams:
    dim: int
    inter: int
    n_experts: int
    topk: int
    gate_w: np.ndarray                 # [E, D] bf16 values (float32)
    gate_bias: Optional[np.ndarray]    # [E] float32 or None for hash layers
    experts: list                      # list of (w1, w3, w2) Fp4Linear (or Fp8Linear)
    shared: tuple                      # (w1, w3, w2) Fp8Linear
    score_func: str = "sqrtsoftplus"
    route_scale: float = 1.0
    swiglu_limit: float = 0.0
    round_pow2: bool = True
    tid2eid: Optional[np.ndarray] = None


@dataclass
class MoEResult:
    y: np.ndarray           # [T, D] bf16 values (float32)
    gate: GateResult
    counts: np.ndarray
    offsets: np.ndarray
    perm_token: np.ndarray
    perm_slot: np.ndarray


def moe_forward(p: MoEParams, x: np.ndarray, input_ids: Optional[np.ndarray] = None,
                experts_subset=None) -> MoEResult:
    """MoE.forward (architecture.py:777-794).

    Experts run in ascending id; each adds its bf16 output into an fp32
    accumulator for its tokens.  A token that lists one expert twice (hash
    layers) receives that expert once: ``y[idx] += out`` is a non-accumulating
    index_put, so the last slot's write wins (architecture.py:790).  The
    shared expert's bf16 output is added last, then the sum is rounded to bf16.
    """
    x = np.asarray(x, np.float32)
    T = x.shape[0]
    g = gate(x, p.gate_w, p.gate_bias, p.topk, p.score_func, p.route_scale,
             p.tid2eid, input_ids)
    counts, offsets, ptok, pslot = permutation(g.indices, p.n_experts)
    y = np.zeros((T, p.dim), np.float32)
    for e in range(p.n_experts):
        if counts[e] == 0:
            continue
        toks = ptok[offsets[e]:offsets[e + 1]]
        slots = pslot[offsets[e]:offsets[e + 1]]
        w1, w3, w2 = p.experts[e]
        out = expert_forward(x[toks], w1, w3, w2, g.weights[toks, slots][:, None],
                             p.swiglu_limit, p.round_pow2)
        # non-accumulating index_put: for a repeated token keep the last row
        upd = {}
        for r, t in enumerate(toks):
            upd[int(t)] = r
        for t, r in upd.items():
            y[t] = (y[t] + out[r]).astype(np.float32)
    s1, s3, s2 = p.shared
    y = (y + expert_forward(x, s1, s3, s2, None, p.swiglu_limit, p.round_pow2)).astype(np.float32)
    return MoEResult(bf16_round(y), g, counts, offsets, ptok, pslot)


def rmsnorm(x: np.ndarray, weight: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """RMSNorm (architecture.py:217-230): fp32 x * rsqrt(mean(x^2) + eps) * w -> bf16."""
    x64 = np.asarray(x, np.float64)
    var = (x64 * x64).mean(-1, keepdims=True).astype(np.float32)
    r = (1.0 / np.sqrt(var.astype(np.float64) + eps)).astype(np.float32)
    y = (np.asarray(x, np.float32) * r).astype(np.float32)
    return bf16_round((np.asarray(weight, np.float32) * y).astype(np.float32))


def cosine(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    na, nb = np.linalg.norm(a), np.linalg.norm(b)
    if na == 0 and nb == 0:
        return 1.0
    return float(a @ b / (na * nb))


def max_rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    """max |got - ref| / max |ref| (bf16 outputs are compared this way)."""
    ref = np.asarray(ref, np.float64)
    d = np.abs(np.asarray(got, np.float64) - ref).max() if ref.size else 0.0
    m = np.abs(ref).max() if ref.size else 0.0
    return float(d / m) if m > 0 else float(d)


__all__ = [n for n in dir() if not n.startswith("_") and n not in ("annotations", "math")]


def sparse_attn(q: np.ndarray, kv: np.ndarray, attn_sink: np.ndarray, topk_idxs: np.ndarray,
                softmax_scale: float, block: int = 64) -> np.ndarray:
    """Sparse attention over gathered rows (torch_ops.py:114-146), float32 as the
    reference's CPU path: blockwise online softmax with the sink term in the
    denominator, K = V = kv.  q [b, s, h, d], kv [b, n, d] (float32 holding bf16
    values), attn_sink [h], topk_idxs [b, s, topk] (-1 = unused).  Returns bf16
    values as float32 [b, s, h, d]."""
    q = np.asarray(q, np.float32)
    kv = np.asarray(kv, np.float32)
    b, s, h, d = q.shape
    topk = topk_idxs.shape[-1]
    acc = np.zeros((b, s, h, d), np.float32)
    sum_exp = np.zeros((b, s, h), np.float32)
    m = np.full((b, s, h), -np.inf, np.float32)
    bi = np.arange(b)[:, None, None]
    with np.errstate(invalid="ignore", over="ignore"):
        for t in range(0, max(topk, 1), block):
            n = min(block, topk - t)
            idx = np.full((b, s, block), -1, np.int64)
            if n > 0:
                idx[..., :n] = topk_idxs[..., t:t + n]
            valid = idx >= 0
            g = kv[bi, np.maximum(idx, 0)]
            g = np.where(valid[..., None], g, np.float32(0))
            sc = (np.einsum("bshd,bstd->bsht", q, g).astype(np.float32) * np.float32(softmax_scale))
            sc = np.where(valid[:, :, None, :], sc, -np.inf).astype(np.float32)
            m_prev = m
            m = np.maximum(m, sc.max(-1))
            resc = np.exp(m_prev - m).astype(np.float32)
            resc = np.where(np.isnan(resc), np.float32(1), resc)
            p = np.exp(sc - m[..., None]).astype(np.float32)
            sum_exp = (sum_exp * resc + p.sum(-1)).astype(np.float32)
            acc = (acc * resc[..., None] + np.einsum("bsht,bstd->bshd", p, g)).astype(np.float32)
        sum_exp = (sum_exp + np.exp(np.asarray(attn_sink, np.float32).reshape(1, 1, h) - m)).astype(np.float32)
        return bf16_round((acc / sum_exp[..., None]).astype(np.float32))

