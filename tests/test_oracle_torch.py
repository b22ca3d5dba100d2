"""The torch float32 restatement (oracle/torch_ref.py) against the reference's own
CPU outputs (tests/golden/*.npz) and against the numpy oracle.

The golden vectors were written by the reference's CPU path (torch_ops.py over
architecture.py's MoE.forward), so an op-for-op torch restatement reproduces
them bit for bit; a dropped clamp, a transposed scale or a wrong nibble order
fails the indices, the weights or the bf16 output bits.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe as om
from oracle import torch_ref as tr
from oracle.numerics import e8m0_decode, from_bf16_bits
from tests.golden.cases import CASES, make_inputs, oracle_params


def _bf16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


def torch_layer(case, inp) -> tr.MoELayer:
    I = case.inter
    nb = I // 128
    u8 = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    f32 = lambda a: torch.from_numpy(np.ascontiguousarray(e8m0_decode(a), dtype=np.float32))
    experts = {}
    for e in range(case.n_experts):
        experts[e] = (tr.QLinear("fp4", u8(inp.w13[e, :I]), f32(inp.w13_s[e, :I])),
                      tr.QLinear("fp4", u8(inp.w13[e, I:]), f32(inp.w13_s[e, I:])),
                      tr.QLinear("fp4", u8(inp.w2[e]), f32(inp.w2_s[e])))
    shared = (tr.QLinear("fp8", u8(inp.sh_w13[:I]), f32(inp.sh_w13_s[:nb])),
              tr.QLinear("fp8", u8(inp.sh_w13[I:]), f32(inp.sh_w13_s[nb:])),
              tr.QLinear("fp8", u8(inp.sh_w2), f32(inp.sh_w2_s)))
    return tr.MoELayer(
        gate_w=_bf16(inp.gate_w),
        gate_bias=None if inp.gate_bias is None else torch.from_numpy(inp.gate_bias),
        experts=experts, shared=shared, n_experts=case.n_experts, topk=case.topk,
        score_func=case.score_func, route_scale=case.route_scale, swiglu_limit=case.swiglu_limit,
        round_pow2=case.round_pow2,
        tid2eid=None if inp.tid2eid is None else torch.from_numpy(inp.tid2eid))


@pytest.mark.parametrize("name", list(CASES))
def test_torch_restatement_matches_reference_golden(name):
    case = CASES[name]
    inp = make_inputs(case)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        y, w, idx = tr.moe_forward(torch_layer(case, inp), _bf16(inp.x), torch.from_numpy(inp.input_ids))
    finally:
        torch.set_default_dtype(prev)
    g = np.load(f"tests/golden/{name}.npz")
    assert np.array_equal(idx.numpy().astype(np.int64), g["indices"].astype(np.int64))
    assert np.allclose(w.numpy(), g["weights"], rtol=1e-6, atol=0)
    ybits = y.view(torch.int16).numpy().view(np.uint16)
    assert np.mean(ybits == g["y_bf16"]) >= 0.999, np.mean(ybits == g["y_bf16"])


@pytest.mark.parametrize("name", ["toy_t4", "top6_t8"])
def test_torch_restatement_agrees_with_numpy_oracle(name):
    case = CASES[name]
    inp = make_inputs(case)
    y, _, idx = tr.moe_forward(torch_layer(case, inp), _bf16(inp.x), torch.from_numpy(inp.input_ids))
    r = om.moe_forward(oracle_params(case, inp), from_bf16_bits(inp.x), inp.input_ids)
    assert np.array_equal(idx.numpy().astype(np.int64), r.gate.indices.astype(np.int64))
    yf = y.float().numpy()
    assert om.max_rel_err(yf, r.y) <= 1e-2 and om.cosine(yf, r.y) >= 0.9999


def test_act_quant_matches_numpy_oracle_on_edge_blocks():
    """Zero, power-of-two, tiny and huge blocks give the oracle's codes and scales."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, 512)).astype(np.float32)
    x[0, :128] = 0.0
    x[1, 128:256] = 0.0
    x[1, 130] = 448.0 * 4
    x[2, 256:384] *= np.float32(1e-30)
    x[3, 384:] *= np.float32(1e30)
    xb = torch.from_numpy(x).to(torch.bfloat16)
    for pow2 in (True, False):
        q, s = tr.act_quant(xb, pow2)
        rq, rs = om.act_quant(xb.float().numpy(), 128, pow2)
        assert np.array_equal(q.view(torch.uint8).numpy(), rq)
        assert np.array_equal(s.numpy(), rs)


def test_unpack_fp4_nibble_order():
    """Low nibble is the even element; code 8 + c is -value(c)."""
    b = torch.tensor([[0x21, 0x9F]], dtype=torch.uint8)
    got = tr.unpack_fp4(b).tolist()[0]
    assert got == [0.5, 1.0, -6.0, -0.5]


def test_near_ties_flags_exact_and_close_gaps():
    s = torch.tensor([[5.0, 4.0, 3.0, 3.0, 1.0],
                      [5.0, 4.0, 3.0, 2.0, 1.0],
                      [5.0, 4.0, 3.0, 3.0 * (1 - 2.0 ** -22), 1.0]])
    assert tr.near_ties(s, 3) == [0, 2]
