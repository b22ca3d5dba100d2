"""Portable, counter-based synthetic inputs for the MoE / FP8-linear workloads.

Every tensor is a pure function of ``(seed, stream, flat index)`` so that any
slice of a multi-GB expert bank can be regenerated independently on the CPU
(numpy here) or on the GPU (``wz_synth_fill`` in the HIP library, which uses
the same integer hash).  Only integer arithmetic feeds the bytes that are
generated on the GPU; Gaussian tensors (activations, gate weights) are drawn
on the host with float64 Box-Muller and rounded to bf16 with round-to-nearest-
even, then uploaded.

The generators follow the recipes of the reference's own tests and probes:

* MXFP4 expert weights: e2m1 codes uniform over all 16 values, ue8m0 scale
  bytes uniform in a stated exponent window (reference expert weights are
  ``float4_e2m1fn_x2`` + ``float8_e8m0fnu`` per 32 K-elements,
  wanferenz/model/architecture.py:146-157).
* FP8 weights: e4m3 bytes uniform with the two NaN codes replaced by zero,
  as in wanferenz/kernels/fp8_vector.py:195-197; fp32 block scales uniform in
  [0.5, 1.5) as in fp8_vector.py:216-231.
"""

from __future__ import annotations

import json
import os

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_MASK64 = (1 << 64) - 1

# Fill modes shared with the HIP generator (wz_synth_fill).
FILL_U8 = 0          # low byte of the draw
FILL_E8M0 = 1        # lo + draw % (hi - lo + 1)
FILL_E4M3 = 2        # low byte, NaN codes (0x7F, 0xFF) -> 0x00
FILL_F32_UNIFORM = 3  # lo + (draw >> 41) * 2^-23 * (hi - lo), lo/hi floats


def _mix64_int(z: int) -> int:
    z &= _MASK64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _MASK64
    return z ^ (z >> 31)


def stream_key(seed: int, stream: int) -> int:
    """64-bit key of one named stream (splitmix64 finaliser of seed*phi+stream+1)."""
    return _mix64_int(seed * 0x9E3779B97F4A7C15 + stream + 1)


def draws(key: int, start: int, count: int) -> np.ndarray:
    """uint64 draws ``mix64(key + (i + 1) * phi)`` for i in [start, start+count)."""
    with np.errstate(over="ignore"):
        i = np.arange(start + 1, start + count + 1, dtype=np.uint64)
        z = np.uint64(key) + i * GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def fill_u8(key: int, start: int, count: int) -> np.ndarray:
    return (draws(key, start, count) & np.uint64(0xFF)).astype(np.uint8)


def fill_e8m0(key: int, start: int, count: int, lo: int, hi: int) -> np.ndarray:
    span = np.uint64(hi - lo + 1)
    return (np.uint64(lo) + draws(key, start, count) % span).astype(np.uint8)


def fill_e4m3(key: int, start: int, count: int) -> np.ndarray:
    b = fill_u8(key, start, count)
    b[(b & 0x7F) == 0x7F] = 0
    return b


def fill_f32_uniform(key: int, start: int, count: int, lo: float, hi: float) -> np.ndarray:
    k = (draws(key, start, count) >> np.uint64(41)).astype(np.float64)
    return (np.float32(lo) + (k * 2.0**-23).astype(np.float32) * np.float32(hi - lo)).astype(np.float32)


def bf16_bits_from_f32(x: np.ndarray) -> np.ndarray:
    """Round float32 to bfloat16 (round-to-nearest-even) and return the uint16 bits."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    bias = np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))
    r = ((u + bias) >> np.uint32(16)).astype(np.uint16)
    r[nan] = ((u[nan] >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16)
    return r


def f32_from_bf16_bits(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def normal_bf16(key: int, shape, sigma: float = 1.0, mean: float = 0.0) -> np.ndarray:
    """N(mean, sigma) drawn by float64 Box-Muller, cast to float32, then bf16 RNE.

    Returns uint16 bf16 bits of ``shape``.
    """
    n = int(np.prod(shape))
    d = draws(key, 0, 2 * n)
    u1 = ((d[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * 2.0**-53
    u2 = (d[1::2] >> np.uint64(11)).astype(np.float64) * 2.0**-53
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    v = (z * sigma + mean).astype(np.float32)
    return bf16_bits_from_f32(v).reshape(shape)


def normal_f32(key: int, shape, sigma: float = 1.0, mean: float = 0.0) -> np.ndarray:
    n = int(np.prod(shape))
    d = draws(key, 0, 2 * n)
    u1 = ((d[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * 2.0**-53
    u2 = (d[1::2] >> np.uint64(11)).astype(np.float64) * 2.0**-53
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return (z * sigma + mean).astype(np.float32).reshape(shape)


# Stream identifiers.  A layer's streams are offset by ``layer * 64`` so that
# stacked layers never share bytes.
S_X = 1
S_GATE_W = 2
S_GATE_BIAS = 3
S_W13 = 4
S_W13_S = 5
S_W2 = 6
S_W2_S = 7
S_SH_W13 = 8
S_SH_W13_S = 9
S_SH_W2 = 10
S_SH_W2_S = 11
S_TID2EID = 12
S_INPUT_IDS = 13
S_FP8_W = 20
S_FP8_W_S = 21
S_FP8_X = 22
S_NORM = 23


def layer_stream(layer: int, stream: int) -> int:
    return layer * 64 + stream


# Exponent windows (ue8m0 byte values) of the synthetic scales.
ROUTED_E8M0 = (119, 123)   # 2^-8 .. 2^-4 per 32-element block
SHARED_E8M0 = (112, 116)   # 2^-15 .. 2^-11 per 128x128 block (keeps the shared
                           # expert's pre-activations O(1) for uniform e4m3 codes)


# ------------------------------------------------------------ device fills ----


def device_fill(t, key: int, mode: int, lo: float = 0.0, hi: float = 0.0, start: int = 0):
    """Fill a contiguous device tensor (bytes, or float32 for mode 3) with the hash stream."""
    from . import _native as N

    if not t.is_contiguous():
        raise ValueError("device_fill: tensor must be contiguous")
    n = t.numel() if mode != FILL_F32_UNIFORM else t.numel()
    N.call("wz_synth_fill", t.data_ptr(), n, key & 0xFFFFFFFFFFFFFFFF, start, mode, float(lo), float(hi),
           N.stream_handle(t.device))
    return t


def synthetic_moe(cfg, seed: int = 0, layer: int = 0, device="cuda", hash_layer: bool = False,
                  vocab: int = 64, bias_sigma: float = 0.01, bias=None):
    """MoEWeights of one synthetic layer (streams as tests/golden/cases.make_inputs).

    Expert banks and the FP8 shared expert are generated on the device by the
    integer hash; the bf16 gate weight and fp32 bias are drawn on the host
    (Box-Muller) and uploaded.  Returns (weights, host) where host holds the
    host-side gate weight bits and bias.
    """
    import torch

    from .moe import MoEWeights

    D, I, E, k = cfg.dim, cfg.inter, cfg.n_experts, cfg.topk

    def key(stream):
        return stream_key(seed, layer_stream(layer, stream))

    u8 = dict(dtype=torch.uint8, device=device)
    lo, hi = ROUTED_E8M0
    w13 = device_fill(torch.empty(E, 2 * I, D // 2, **u8), key(S_W13), FILL_U8)
    w13_s = device_fill(torch.empty(E, 2 * I, D // 32, **u8), key(S_W13_S), FILL_E8M0, lo, hi)
    w2 = device_fill(torch.empty(E, D, I // 2, **u8), key(S_W2), FILL_U8)
    w2_s = device_fill(torch.empty(E, D, I // 32, **u8), key(S_W2_S), FILL_E8M0, lo, hi)
    slo, shi = SHARED_E8M0
    sh13 = device_fill(torch.empty(2 * I, D, **u8), key(S_SH_W13), FILL_E4M3)
    sh13_s = device_fill(torch.empty(2 * I // 128, D // 128, **u8), key(S_SH_W13_S), FILL_E8M0, slo, shi)
    sh2 = device_fill(torch.empty(D, I, **u8), key(S_SH_W2), FILL_E4M3)
    sh2_s = device_fill(torch.empty(D // 128, I // 128, **u8), key(S_SH_W2_S), FILL_E8M0, slo, shi)
    gw_bits = normal_bf16(key(S_GATE_W), (E, D), 0.02)
    gate_w = torch.from_numpy(gw_bits.view(np.int16)).view(torch.bfloat16).to(device)
    host = {"gate_w": gw_bits}
    gate_bias = None
    tid2eid = None
    if hash_layer:
        t2e = (draws(key(S_TID2EID), 0, vocab * k) % np.uint64(E)).astype(np.int32).reshape(vocab, k)
        host["tid2eid"] = t2e
        tid2eid = torch.from_numpy(t2e).to(device)
    else:
        b = normal_f32(key(S_GATE_BIAS), (E,), bias_sigma) if bias is None else np.asarray(bias, np.float32)
        host["gate_bias"] = b
        gate_bias = torch.from_numpy(b).to(device)
    nb = I // 128
    w = MoEWeights(gate_w=gate_w, gate_bias=gate_bias, w13=w13, w13_s=w13_s, w2=w2, w2_s=w2_s,
                   sh_w1=sh13[:I], sh_w1_s=sh13_s[:nb], sh_w3=sh13[I:], sh_w3_s=sh13_s[nb:],
                   sh_w2=sh2, sh_w2_s=sh2_s, tid2eid=tid2eid)
    return w, host


def zipf_bias(n_experts: int, s: float = 1.1, beta: float = 0.05, seed: int = 1) -> np.ndarray:
    """Gate bias that skews expert popularity towards a Zipf(s) law.

    bias_e = beta * log(p_e) with p_e proportional to rank_e^-s, where rank is a
    seeded random permutation of the experts; beta sets the strength
    (:func:`calibrate_zipf` finds the beta at which the routed popularity is
    Zipf(s); the V4 value is in ``zipf_v4.json``).
    """
    d = draws(stream_key(seed, 77), 0, n_experts)
    rank = np.argsort(np.argsort(d)) + 1
    p = rank.astype(np.float64) ** (-s)
    p /= p.sum()
    return (beta * np.log(p)).astype(np.float32)


def zipf_exponent(counts) -> float:
    """Maximum-likelihood exponent of a finite Zipf law over len(counts) ranks fitted to
    the rank-frequency data ``counts`` (selections per expert, any order).

    The likelihood of s is prod_r (r^-s / H(s))^c_r with H(s) = sum_r r^-s; its
    stationary point equates the observed mean of log(rank) with the model's,
    sum_r c_r log r / C = sum_r r^-s log r / H(s), whose right side falls as s
    grows, so bisection finds it."""
    c = np.sort(np.asarray(counts, np.float64))[::-1]
    r = np.arange(1, c.size + 1, dtype=np.float64)
    target = float((c * np.log(r)).sum() / c.sum())
    lo, hi = 0.0, 8.0
    for _ in range(60):
        m = 0.5 * (lo + hi)
        w = r ** -m
        if (w * np.log(r)).sum() / w.sum() > target:
            lo = m
        else:
            hi = m
    return 0.5 * (lo + hi)


def route_counts(x_bits: np.ndarray, gate_w_bits: np.ndarray, bias: np.ndarray, k: int) -> np.ndarray:
    """Selections per expert of the biased sqrt-softplus top-k gate (Gate.forward,
    architecture.py:696-718, routing only) over tokens x: workload synthesis, in
    float64 products rounded to float32 scores; lower index first on ties."""
    a = (f32_from_bf16_bits(x_bits).astype(np.float64) @ f32_from_bf16_bits(gate_w_bits).astype(np.float64).T)
    a = a.astype(np.float32).astype(np.float64)
    sc = np.sqrt(np.where(a > 20.0, a, np.log1p(np.exp(np.minimum(a, 20.0)))).astype(np.float32).astype(np.float64))
    key = (sc.astype(np.float32) + bias.astype(np.float32)).astype(np.float32)
    idx = np.argsort(-key.astype(np.float64), axis=1, kind="stable")[:, :k]
    return np.bincount(idx.ravel(), minlength=gate_w_bits.shape[0])


ZIPF_V4_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "zipf_v4.json")


def zipf_v4_calibration_batch(T: int = 2048):
    """The calibration inputs of the V4 prefill workload: the gate of synthetic layer 0
    (seed 0, N(0, 0.02) bf16 [256, 4096]) and T tokens of N(0, 1) bf16 (seed 2)."""
    E, D = 256, 4096
    gw = normal_bf16(stream_key(0, layer_stream(0, S_GATE_W)), (E, D), 0.02)
    x = normal_bf16(stream_key(2, S_X), (T, D), 1.0)
    return x, gw


def calibrate_zipf(s: float = 1.1, k: int = 6, T: int = 2048, iters: int = 40) -> dict:
    """Bisection on beta so that the top-k routing of the calibration batch has a
    Zipf exponent (``zipf_exponent``) of s; returns beta, the fitted exponent and
    the achieved selections per expert."""
    x, gw = zipf_v4_calibration_batch(T)
    E = gw.shape[0]

    def fit(beta):
        c = route_counts(x, gw, zipf_bias(E, s, beta), k)
        return zipf_exponent(c), c

    lo, hi = 0.0, 2.0
    for _ in range(iters):
        mid = 0.5 * (lo + hi)
        if fit(mid)[0] < s:
            lo = mid
        else:
            hi = mid
    beta = float(np.float32(0.5 * (lo + hi)))
    got, counts = fit(beta)
    return {"s": s, "k": k, "T": T, "beta": beta, "fitted_exponent": got,
            "counts_per_expert": counts.astype(int).tolist(),
            "max_expert_rows": int(counts.max()), "experts_unused": int((counts == 0).sum())}


def zipf_v4_beta() -> float:
    """The committed calibration's beta (``python -m wanferenz_amd.synth calibrate`` writes it)."""
    with open(ZIPF_V4_FILE) as f:
        return float(json.load(f)["beta"])


if __name__ == "__main__":
    import sys

    if sys.argv[1:] == ["calibrate"]:
        r = calibrate_zipf()
        with open(ZIPF_V4_FILE, "w") as f:
            json.dump(r, f, indent=1)
        print(f"beta {r['beta']:.6f} fitted exponent {r['fitted_exponent']:.4f} max rows {r['max_expert_rows']} "
              f"unused {r['experts_unused']} -> {ZIPF_V4_FILE}")
