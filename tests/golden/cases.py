"""Seeded MoE cases shared by the golden-vector writer, the oracle tests and the GPU parity tests.

Inputs are regenerated from ``(seed, stream)`` by wanferenz_amd.synth; the
committed fixtures under tests/golden/ hold only the reference's outputs.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import numpy as np

from wanferenz_amd import synth


@dataclass(frozen=True)
class MoECase:
    name: str
    dim: int
    inter: int
    n_experts: int
    topk: int
    T: int
    seed: int = 0
    layer: int = 0
    hash_layer: bool = False
    vocab: int = 64
    score_func: str = "sqrtsoftplus"
    route_scale: float = 1.5
    swiglu_limit: float = 10.0
    round_pow2: bool = True          # reference scale_fmt == "ue8m0"
    hash_patterns: tuple = ()        # rows of tid2eid overwritten (token id -> experts)


CASES = {
    # The toy layer the reference's CPU path runs (hidden 1024, 16 routed + 1 shared,
    # top-2, intermediate 512, T=4).
    "toy_t4": MoECase("toy_t4", 1024, 512, 16, 2, 4),
    "toy_t1": MoECase("toy_t1", 1024, 512, 16, 2, 1, seed=1),
    "toy_t4_fp32scale": MoECase("toy_t4_fp32scale", 1024, 512, 16, 2, 4, seed=2, round_pow2=False),
    "toy_t37": MoECase("toy_t37", 1024, 512, 16, 2, 37, seed=3),
    # top-6 over 32 experts, T=8 (decode verify width) — exercises the k=6 renormalisation.
    "top6_t8": MoECase("top6_t8", 512, 256, 32, 6, 8, seed=4),
    # hash-routed layer with repeated experts inside a token's list
    "hash_t3": MoECase("hash_t3", 1024, 512, 32, 6, 3, seed=5, hash_layer=True,
                       hash_patterns=((7, (3, 3, 17, 3, 20, 17)), (9, (1, 2, 3, 4, 5, 6)),
                                      (11, (31, 31, 31, 31, 31, 31)))),
}


def hash_input_ids(case: MoECase) -> np.ndarray:
    key = synth.stream_key(case.seed, synth.layer_stream(case.layer, synth.S_INPUT_IDS))
    ids = (synth.draws(key, 0, case.T) % np.uint64(case.vocab)).astype(np.int64)
    if case.hash_patterns:
        pat_ids = [p[0] for p in case.hash_patterns]
        for i in range(min(case.T, len(pat_ids))):
            ids[i] = pat_ids[i]
    return ids


@dataclass
class MoEInputs:
    x: np.ndarray            # uint16 bf16 bits [T, D]
    gate_w: np.ndarray       # uint16 bf16 bits [E, D]
    gate_bias: Optional[np.ndarray]  # float32 [E]
    w13: np.ndarray          # uint8 [E, 2I, D/2] packed e2m1 (w1 rows then w3 rows)
    w13_s: np.ndarray        # uint8 [E, 2I, D/32] e8m0
    w2: np.ndarray           # uint8 [E, D, I/2]
    w2_s: np.ndarray         # uint8 [E, D, I/32]
    sh_w13: np.ndarray       # uint8 [2I, D] e4m3 (w1 rows then w3 rows)
    sh_w13_s: np.ndarray     # uint8 [2I/128, D/128] e8m0
    sh_w2: np.ndarray        # uint8 [D, I] e4m3
    sh_w2_s: np.ndarray      # uint8 [D/128, I/128] e8m0
    input_ids: np.ndarray    # int64 [T]
    tid2eid: Optional[np.ndarray] = None  # int32 [vocab, k]


def make_inputs(case: MoECase) -> MoEInputs:
    s, L = case.seed, case.layer
    D, I, E, k, T = case.dim, case.inter, case.n_experts, case.topk, case.T

    def key(stream):
        return synth.stream_key(s, synth.layer_stream(L, stream))

    x = synth.normal_bf16(key(synth.S_X), (T, D), 1.0)
    gw = synth.normal_bf16(key(synth.S_GATE_W), (E, D), 0.02)
    bias = None if case.hash_layer else synth.normal_f32(key(synth.S_GATE_BIAS), (E,), 0.01)
    lo, hi = synth.ROUTED_E8M0
    w13 = synth.fill_u8(key(synth.S_W13), 0, E * 2 * I * D // 2).reshape(E, 2 * I, D // 2)
    w13_s = synth.fill_e8m0(key(synth.S_W13_S), 0, E * 2 * I * D // 32, lo, hi).reshape(E, 2 * I, D // 32)
    w2 = synth.fill_u8(key(synth.S_W2), 0, E * D * I // 2).reshape(E, D, I // 2)
    w2_s = synth.fill_e8m0(key(synth.S_W2_S), 0, E * D * I // 32, lo, hi).reshape(E, D, I // 32)
    slo, shi = synth.SHARED_E8M0
    sh13 = synth.fill_e4m3(key(synth.S_SH_W13), 0, 2 * I * D).reshape(2 * I, D)
    sh13_s = synth.fill_e8m0(key(synth.S_SH_W13_S), 0, (2 * I // 128) * (D // 128), slo, shi).reshape(2 * I // 128, D // 128)
    sh2 = synth.fill_e4m3(key(synth.S_SH_W2), 0, D * I).reshape(D, I)
    sh2_s = synth.fill_e8m0(key(synth.S_SH_W2_S), 0, (D // 128) * (I // 128), slo, shi).reshape(D // 128, I // 128)
    ids = hash_input_ids(case)
    tid2eid = None
    if case.hash_layer:
        tid2eid = (synth.draws(key(synth.S_TID2EID), 0, case.vocab * k) % np.uint64(E)).astype(np.int32).reshape(case.vocab, k)
        for tok, experts in case.hash_patterns:
            tid2eid[tok] = np.asarray(experts, np.int32)
    return MoEInputs(x, gw, bias, w13, w13_s, w2, w2_s, sh13, sh13_s, sh2, sh2_s, ids, tid2eid)


def oracle_params(case: MoECase, inp: MoEInputs):
    """Build oracle.moe.MoEParams from the synthetic inputs (test-side only)."""
    from oracle import moe as om
    from oracle.numerics import e8m0_decode, from_bf16_bits

    I = case.inter
    experts = []
    for e in range(case.n_experts):
        w1 = om.Fp4Linear(inp.w13[e, :I], e8m0_decode(inp.w13_s[e, :I]))
        w3 = om.Fp4Linear(inp.w13[e, I:], e8m0_decode(inp.w13_s[e, I:]))
        w2 = om.Fp4Linear(inp.w2[e], e8m0_decode(inp.w2_s[e]))
        experts.append((w1, w3, w2))
    nb = I // 128
    shared = (
        om.Fp8Linear(inp.sh_w13[:I], e8m0_decode(inp.sh_w13_s[:nb])),
        om.Fp8Linear(inp.sh_w13[I:], e8m0_decode(inp.sh_w13_s[nb:])),
        om.Fp8Linear(inp.sh_w2, e8m0_decode(inp.sh_w2_s)),
    )
    return om.MoEParams(
        dim=case.dim, inter=I, n_experts=case.n_experts, topk=case.topk,
        gate_w=from_bf16_bits(inp.gate_w), gate_bias=inp.gate_bias,
        experts=experts, shared=shared, score_func=case.score_func,
        route_scale=case.route_scale, swiglu_limit=case.swiglu_limit,
        round_pow2=case.round_pow2, tid2eid=inp.tid2eid,
    )
