"""CPU pins of the oracle's sparse attention (oracle.moe.sparse_attn, restating
torch_ops.py:114-146) against a direct float64 softmax and closed forms."""

import numpy as np

from oracle import moe as om
from oracle.numerics import bf16_round
from wanferenz_amd import synth


def _direct(q, kv, sink, idx, scale):
    """softmax with the sink logit in the denominator, one max subtraction, float64"""
    b, s, h, d = q.shape
    out = np.zeros((b, s, h, d))
    for bb in range(b):
        for ss in range(s):
            sel = [i for i in idx[bb, ss] if i >= 0]
            g = kv[bb, sel].astype(np.float64)
            for hh in range(h):
                lg = g @ q[bb, ss, hh].astype(np.float64) * scale
                m = max(lg.max() if len(sel) else -np.inf, sink[hh])
                w = np.exp(lg - m)
                out[bb, ss, hh] = (w @ g) / (w.sum() + np.exp(sink[hh] - m))
    return out


def _inputs(seed, b, s, h, d, n, topk, invalid=0.2):
    k = synth.stream_key(seed, 60)
    q = bf16_round(synth.f32_from_bf16_bits(synth.normal_bf16(k, (b, s, h, d), 1.0)))
    kv = bf16_round(synth.f32_from_bf16_bits(synth.normal_bf16(synth.stream_key(seed, 61), (b, n, d), 1.0)))
    sink = synth.fill_f32_uniform(synth.stream_key(seed, 62), 0, h, -1.0, 1.0)
    r = synth.draws(synth.stream_key(seed, 63), 0, b * s * topk)
    idx = (r % np.uint64(n)).astype(np.int32).reshape(b, s, topk)
    idx[(r % np.uint64(1000)).reshape(b, s, topk) < invalid * 1000] = -1
    return q, kv, sink, idx


def test_matches_direct_softmax():
    """Blocks of 64 with a running max (topk 150 = 3 blocks, the last partial, 20 %
    unused slots) against the one-pass float64 formula: within one bf16 ulp."""
    q, kv, sink, idx = _inputs(1, 2, 3, 4, 64, 200, 150)
    got = om.sparse_attn(q, kv, sink, idx, 0.125)
    ref = _direct(q, kv, sink, idx, 0.125)
    assert np.all(np.abs(got - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-30 + 2.0 ** -133)


def test_closed_forms():
    d = 32
    kv = bf16_round(np.linspace(-2, 2, 10 * d).reshape(1, 10, d).astype(np.float32))
    sink = np.array([0.5], np.float32)
    # q = 0: every valid row weighs 1, the sink e^0.5: mean of rows * n / (n + e^0.5)
    q = np.zeros((1, 1, 1, d), np.float32)
    idx = np.array([[[3, -1, 7, 9, -1]]], np.int32)
    got = om.sparse_attn(q, kv, sink, idx, 1.0)
    want = kv[0, [3, 7, 9]].astype(np.float64).sum(0) / (3 + np.exp(0.5))
    assert np.allclose(got[0, 0, 0], want, rtol=2.0 ** -8, atol=1e-6)
    # no valid row in the first block of 64: the reference's running max is still -inf
    # there, exp(-inf - -inf) is NaN and stays in the sums -> NaN output; a fully
    # unused later block after a valid one contributes nothing
    got = om.sparse_attn(q + 1, kv, sink, np.full((1, 1, 5), -1, np.int32), 1.0)
    assert np.isnan(got).all()
    idx2 = np.full((1, 1, 130), -1, np.int32)
    idx2[0, 0, 5] = 4
    got = om.sparse_attn(q, kv, sink, idx2, 1.0)
    assert np.allclose(got[0, 0, 0], kv[0, 4] / (1 + np.exp(0.5)), rtol=2.0 ** -8, atol=1e-6)
