"""CPU pins of the oracle's gate, permutation and MoE layer.

* Golden vectors: the reference's own CPU MoE.forward (architecture.py:777-794
  over torch_ops.py) on the committed cases (tests/golden/*.npz, written by
  tests/golden/make_golden.py): expert indices bit-exact, routing weights
  within 1e-6 relative (the reference's fp32 gate GEMM sums in its own order,
  so its logits can sit a few ulp from the correctly rounded ones), layer
  outputs within the bf16 tolerance (and in practice bit-equal but for single
  elements).
* Permutation: counting sort == brute-force sort by (expert, token, slot).
* Gate: invariants the definition fixes (renormalised weights sum to
  route_scale, selection in descending biased order with ties to the lower
  index, weights gathered from the unbiased scores, hash rows read tid2eid).
* Hash keep-last: a token that lists an expert twice receives it once.
"""

import numpy as np
import pytest

from oracle import moe as om
from oracle.numerics import from_bf16_bits
from tests.golden.cases import CASES, make_inputs, oracle_params

TOL_REL = 1e-2
TOL_COS = 0.9999


@pytest.mark.parametrize("name", list(CASES))
def test_oracle_matches_reference_golden(name):
    case = CASES[name]
    inp = make_inputs(case)
    r = om.moe_forward(oracle_params(case, inp), from_bf16_bits(inp.x), inp.input_ids)
    g = np.load(f"tests/golden/{name}.npz")
    assert np.array_equal(r.gate.indices, g["indices"])
    assert np.allclose(r.gate.weights, g["weights"], rtol=1e-6, atol=0)
    y = from_bf16_bits(g["y_bf16"])
    assert om.max_rel_err(r.y, y) <= TOL_REL and om.cosine(r.y, y) >= TOL_COS
    assert np.mean(r.y == y) >= 0.999, np.mean(r.y == y)


def test_golden_cases_are_not_near_ties():
    """Every score-routed golden token has a clear k-th vs (k+1)-th margin."""
    for name, case in CASES.items():
        if case.hash_layer:
            continue
        inp = make_inputs(case)
        r = om.gate(from_bf16_bits(inp.x), from_bf16_bits(inp.gate_w), inp.gate_bias, case.topk,
                    case.score_func, case.route_scale)
        rel = r.margin / np.abs(r.biased).max(axis=1)
        assert rel.min() > 1e-4, (name, rel.min())


@pytest.mark.parametrize("seed,T,E,k", [(0, 1, 4, 1), (1, 13, 16, 2), (2, 40, 32, 6), (3, 7, 8, 8)])
def test_permutation_matches_brute_force_sort(seed, T, E, k):
    rng = np.random.default_rng(seed)
    idx = rng.integers(0, E, (T, k))  # repeats allowed (hash layers)
    counts, offsets, ptok, pslot = om.permutation(idx, E)
    pairs = sorted((int(idx[t, j]), t, j) for t in range(T) for j in range(k))
    assert [p[1] for p in pairs] == ptok.tolist()
    assert [p[2] for p in pairs] == pslot.tolist()
    assert counts.tolist() == np.bincount(idx.ravel(), minlength=E).tolist()
    assert offsets[0] == 0 and offsets[-1] == T * k and (np.diff(offsets) == counts).all()


def test_gate_invariants():
    rng = np.random.default_rng(4)
    T, D, E, k = 16, 256, 32, 6
    x = from_bf16_bits((rng.standard_normal((T, D)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16))
    W = from_bf16_bits(((rng.standard_normal((E, D)) * 0.02).astype(np.float32).view(np.uint32) >> 16)
                       .astype(np.uint16))
    bias = (rng.standard_normal(E) * 0.01).astype(np.float32)
    for sf in ("sqrtsoftplus", "sigmoid", "softmax"):
        g = om.gate(x, W, bias, k, sf, 1.5)
        b = g.biased
        for t in range(T):
            sel = g.indices[t]
            assert len(set(sel.tolist())) == k
            assert all(b[t, sel[j]] >= b[t, sel[j + 1]] for j in range(k - 1))
            rest = np.setdiff1d(np.arange(E), sel)
            assert b[t, rest].max() <= b[t, sel[-1]]
        w = g.weights / np.float32(1.5)
        if sf != "softmax":
            assert np.allclose(w.sum(1), 1.0, atol=4e-7)
            assert np.allclose(w * np.take_along_axis(g.scores, g.indices, 1).sum(1, keepdims=True),
                               np.take_along_axis(g.scores, g.indices, 1), rtol=1e-6)
        else:
            assert np.allclose(w, np.take_along_axis(g.scores, g.indices, 1), rtol=1e-6)


def test_gate_ties_go_to_lower_index():
    x = np.ones((1, 128), np.float32)
    W = np.zeros((8, 128), np.float32)
    bias = np.float32([0.0, 0.5, 0.5, 0.0, 0.5, 0.0, 0.0, 0.0])
    g = om.gate(x, W, bias, 3, "sigmoid", 1.0)
    assert g.indices.tolist() == [[1, 2, 4]]
    g = om.gate(x, W, None, 3, "sigmoid", 1.0)
    assert g.indices.tolist() == [[0, 1, 2]]


def test_hash_routing_reads_table_and_keeps_repeats_once():
    case = CASES["hash_t3"]
    inp = make_inputs(case)
    p = oracle_params(case, inp)
    r = om.moe_forward(p, from_bf16_bits(inp.x), inp.input_ids)
    assert np.array_equal(r.gate.indices, inp.tid2eid[inp.input_ids])
    # token 0 lists (3, 3, 17, 3, 20, 17): the layer equals one pass per distinct expert
    t = 0
    x0 = from_bf16_bits(inp.x[t:t + 1])
    acc = np.zeros((1, case.dim), np.float32)
    seen = {}
    for j, e in enumerate(r.gate.indices[t].tolist()):
        seen[e] = j  # the last slot of a repeated expert is the one kept
    for e in sorted(seen):
        w1, w3, w2 = p.experts[e]
        acc = (acc + om.expert_forward(x0, w1, w3, w2, r.gate.weights[t:t + 1, seen[e]][:, None],
                                       p.swiglu_limit, p.round_pow2)).astype(np.float32)
    s1, s3, s2 = p.shared
    acc = (acc + om.expert_forward(x0, s1, s3, s2, None, p.swiglu_limit, p.round_pow2)).astype(np.float32)
    assert np.array_equal(om.bf16_round(acc), r.y[t:t + 1])


def test_gate_scores_match_torch_for_every_score_function():
    """Gate.forward (architecture.py:699-705) in torch fp32 against the oracle: the
    oracle rounds each score once from float64 (so do the HIP kernels); torch's
    fp32 sigmoid / softplus land within 2 ulp of that, its fp32 softmax within 8
    (6 measured here: an fp32 sum of fp32 exponentials).  The selection agrees
    wherever the k-th vs (k+1)-th margin is not within that noise."""
    import torch
    import torch.nn.functional as F

    rng = np.random.default_rng(11)
    T, D, E, k = 64, 512, 64, 6
    x = from_bf16_bits((rng.standard_normal((T, D)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16))
    W = from_bf16_bits(((rng.standard_normal((E, D)) * 0.05).astype(np.float32).view(np.uint32) >> 16)
                       .astype(np.uint16))
    bias = (rng.standard_normal(E) * 0.01).astype(np.float32)
    logits = torch.from_numpy(x).double() @ torch.from_numpy(W).double().T
    logits = logits.float()
    for sf, fn, ulps in (("softmax", lambda a: a.softmax(dim=-1), 8), ("sigmoid", torch.sigmoid, 2),
                         ("sqrtsoftplus", lambda a: F.softplus(a).sqrt(), 2)):
        g = om.gate(x, W, bias, k, sf, 1.5)
        ts = fn(logits).numpy()
        assert np.all(np.abs(g.scores - ts) <= ulps * np.spacing(np.abs(ts))), sf
        tb = torch.from_numpy(ts) + torch.from_numpy(bias)
        tidx = tb.topk(k, dim=-1)[1].numpy()
        close = g.margin <= 2 * ulps * np.spacing(np.abs(g.biased).max(1))
        assert np.array_equal(g.indices[~close], tidx[~close]), sf
