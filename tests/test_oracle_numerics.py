"""CPU pins of the oracle's number codecs and act_quant (no GPU).

Each codec is checked against an independent source: torch's own dtype casts
(a library routine, over every code or a dense sweep that includes every
rounding midpoint), hand-computed known answers, or the format definition
evaluated with Python's exact float arithmetic.  A plausible slip — a wrong
exponent bias, ties rounded away from even, the nibble order swapped, a
saturation bound off by one code — fails at least one of these.
"""

import math

import numpy as np
import pytest
import torch

from oracle import moe as om
from oracle.numerics import (
    E2M1_TABLE,
    E4M3_TABLE,
    bf16_round,
    e2m1_decode_nibbles,
    e4m3_decode,
    e4m3_encode,
    e8m0_decode,
    e8m0_encode_pow2,
)


def _torch_e4m3_codes(v: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(v, np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_e4m3_decode_matches_torch_every_code():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    ref = codes.view(torch.float8_e4m3fn).float().numpy()
    got = e4m3_decode(codes.numpy())
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(got[ok], ref[ok])
    assert np.array_equal(np.signbit(got[ok]), np.signbit(ref[ok]))


def test_e4m3_known_answers():
    # definition: bias 7, 3 mantissa bits, no infinities, S.1111.111 is NaN
    assert E4M3_TABLE[0x7E] == 448.0            # max finite
    assert E4M3_TABLE[0x38] == 1.0              # exponent 7 -> 2^0
    assert E4M3_TABLE[0x01] == 2.0 ** -9        # smallest subnormal
    assert E4M3_TABLE[0x08] == 2.0 ** -6        # smallest normal
    assert np.isnan(E4M3_TABLE[0x7F]) and np.isnan(E4M3_TABLE[0xFF])
    # ties go to the even code: 1.0625 is halfway between 1.0 (0x38) and 1.125 (0x39)
    assert e4m3_encode(np.float32([1.0625]))[0] == 0x38
    # 1.1875 is halfway between 1.125 (0x39) and 1.25 (0x3A)
    assert e4m3_encode(np.float32([1.1875]))[0] == 0x3A
    # half the smallest subnormal rounds to zero (even), a hair above rounds up
    assert e4m3_encode(np.float32([2.0 ** -10]))[0] == 0x00
    assert e4m3_encode(np.nextafter(np.float32([2.0 ** -10]), np.float32(1)))[0] == 0x01
    assert e4m3_encode(np.float32([-0.0]))[0] == 0x80
    assert e4m3_encode(np.float32([-448.0]))[0] == 0xFE


def test_e4m3_encode_matches_torch_dense_sweep():
    pos = E4M3_TABLE[:0x7F].astype(np.float64)
    mids = (pos[:-1] + pos[1:]) / 2.0
    mids32 = mids.astype(np.float32)
    assert np.array_equal(mids32.astype(np.float64), mids)  # midpoints are exact in fp32
    above = np.nextafter(mids32, np.float32(np.inf))
    below = np.nextafter(mids32, np.float32(0))
    rng = np.random.default_rng(0)
    rand = np.exp(rng.uniform(np.log(2.0 ** -12), np.log(448.0), 20000)).astype(np.float32)
    v = np.concatenate([pos.astype(np.float32), mids32, above, below, rand,
                        np.float32([0.0, 2.0 ** -12, 447.99])])
    v = np.concatenate([v, -v])
    v = v[np.abs(v) <= 448.0]
    got = e4m3_encode(v)
    ref = _torch_e4m3_codes(v)
    bad = np.nonzero(got != ref)[0]
    assert bad.size == 0, f"{bad.size} mismatches, e.g. {v[bad[:5]]} -> {got[bad[:5]]} vs torch {ref[bad[:5]]}"


def test_e4m3_encode_rejects_out_of_range():
    with pytest.raises(ValueError):
        e4m3_encode(np.float32([448.5]))


def test_e4m3_encode_nan_is_torchs_nan_code():
    v = np.float32([np.nan, -np.nan, 1.0])
    got = e4m3_encode(v)
    want = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert got.tolist() == want.tolist() == [0x7F, 0xFF, 0x38]


def test_e2m1_from_definition_and_nibble_order():
    # e2m1: sign, 2 exponent bits (bias 1), 1 mantissa bit; exponent 0 is subnormal
    for c in range(16):
        s = -1.0 if c & 8 else 1.0
        e, m = (c >> 1) & 3, c & 1
        v = s * (m * 0.5 if e == 0 else (1.0 + m / 2.0) * 2.0 ** (e - 1))
        assert E2M1_TABLE[c] == v and math.copysign(1.0, E2M1_TABLE[c]) == s
    # low nibble is the even element (torch_ops.py:72-74, 82-90)
    out = e2m1_decode_nibbles(np.uint8([[0x21, 0xF7]]))
    assert out.tolist() == [[0.5, 1.0, 6.0, -6.0]]


def test_e8m0_decode_matches_torch_every_code():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    ref = codes.view(torch.float8_e8m0fnu).float().numpy()
    got = e8m0_decode(codes.numpy())
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(got[ok], ref[ok])
    for b in (1, 100, 127, 128, 200, 254):
        assert e8m0_encode_pow2(np.float32([2.0 ** (b - 127)]))[0] == b


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(50000).astype(np.float32) * np.float32(3.0)
    u = x.view(np.uint32)
    ties = ((u & np.uint32(0xFFFF0000)) | np.uint32(0x8000)).view(np.float32)  # exact halfway cases
    x = np.concatenate([x, ties, np.float32([0.0, -0.0, 1e-40, 3.4e38])])
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(bf16_round(x).view(np.uint32), ref.view(np.uint32))


def test_round_scale_is_pow2_ceiling():
    rng = np.random.default_rng(2)
    x = np.exp(rng.uniform(-30, 10, 5000)).astype(np.float32)
    x = np.concatenate([x, np.float32([2.0 ** -20, 0.25, 1.0, 8.0])])  # exact powers keep their value
    got = om.round_scale(x)
    for xi, gi in zip(x.tolist(), got.tolist()):
        e = math.ceil(math.log2(xi))
        if 2.0 ** (e - 1) >= xi:  # guard log2 rounding at the boundary
            e -= 1
        assert gi == 2.0 ** e, (xi, gi)


def test_act_quant_known_answers():
    # zero block: amax floors at 1e-4, every code is +0
    q, s = om.act_quant(np.zeros((1, 128), np.float32), round_pow2=False)
    assert s[0, 0] == np.float32(np.float32(1e-4) * np.float32(1.0 / 448.0)) and not q.any()
    q, s = om.act_quant(np.zeros((1, 128), np.float32), round_pow2=True)
    assert s[0, 0] == 2.0 ** math.ceil(math.log2(1e-4 / 448.0))
    # amax = 448 * 2^-3 = 56: both scale kinds give s = 0.125, the max element maps to 448 (0x7E)
    x = np.zeros((1, 256), np.float32)
    x[0, 5], x[0, 200] = -56.0, 3.0
    x[0, 130] = 56.0
    for pow2 in (False, True):
        q, s = om.act_quant(x, round_pow2=pow2)
        assert s.tolist() == [[0.125, 0.125]]
        assert q[0, 5] == 0xFE and q[0, 130] == 0x7E
    # non-power-of-two amax with pow2 scales: 100 -> s = 2^ceil(log2(100/448)) = 0.25; 100/0.25 = 400
    # lies halfway between 384 (0x7C) and 416 (0x7D) and goes to the even code
    x = np.zeros((1, 128), np.float32)
    x[0, 0] = 100.0
    q, s = om.act_quant(x, round_pow2=True)
    assert s[0, 0] == 0.25 and q[0, 0] == 0x7C


def test_act_quant_error_bound():
    """|x - dequant(q)| <= half an e4m3 step at |x/s|, times s (RNE), for every element."""
    rng = np.random.default_rng(3)
    x = bf16_round(rng.standard_normal((16, 512)).astype(np.float32) * np.float32(4.0))
    for pow2 in (False, True):
        q, s = om.act_quant(x, round_pow2=pow2)
        sr = np.repeat(s, 128, axis=1).astype(np.float64)
        y = np.clip(x / sr, -448.0, 448.0)
        dq = e4m3_decode(q).astype(np.float64)
        a = np.abs(y)
        # e4m3 spacing at magnitude a: 2^(floor(log2 a) - 3) for normals, 2^-9 below 2^-6
        ex = np.floor(np.log2(np.maximum(a, 2.0 ** -6)))
        step = 2.0 ** (ex - 3)
        assert (np.abs(dq - y) <= step / 2 + a * 2.0 ** -22).all()  # + the fp32 rounding of x / s
        assert (np.abs(dq) <= 448.0).all()


def test_rmsnorm_matches_torch():
    """oracle.rmsnorm (architecture.py:217-230) vs torch's own F.rms_norm in float32, then bf16."""
    rng = np.random.default_rng(5)
    x = bf16_round(rng.standard_normal((6, 4096)).astype(np.float32) * np.float32(2.0))
    w = bf16_round(rng.uniform(0.5, 1.5, 4096).astype(np.float32))
    ref = torch.nn.functional.rms_norm(torch.from_numpy(x), (4096,), torch.from_numpy(w), eps=1e-6)
    ref = ref.to(torch.bfloat16).float().numpy()
    got = om.rmsnorm(x, w, 1e-6)
    # fp32 reductions differ in order: equal up to one bf16 step at rounding boundaries
    step = np.spacing(np.abs(ref).astype(np.float32)) * 65536
    assert (np.abs(got - ref) <= step).all() and np.mean(got == ref) > 0.99


def _torch_act_quant(x, scale_fmt):
    """The reference's CPU act_quant (torch_ops.py:15-49) evaluated by torch itself."""
    import torch

    def round_scale(amax, max_inv):
        mant, exp = torch.frexp(amax * max_inv)
        return torch.ldexp(torch.ones_like(amax), torch.where(mant == 0.5, exp - 1, exp))

    z = torch.from_numpy(x).float().unflatten(-1, (-1, 128))
    amax = z.abs().amax(-1, keepdim=True).clamp_min(1e-4)
    s = round_scale(amax, 1.0 / 448.0) if scale_fmt is not None else amax * (1.0 / 448.0)
    q = (z / s).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).flatten(-2)
    return q.view(torch.uint8).numpy(), s.squeeze(-1).numpy()


def _special_blocks():
    """Rows of 128-blocks holding NaN, +inf, -inf, all of them, and ordinary values."""
    base = np.linspace(-3.0, 3.0, 128, dtype=np.float32)
    rows = []
    for spec in ([], [(5, np.nan)], [(0, np.inf)], [(127, -np.inf)], [(3, np.nan), (9, np.inf)],
                 [(i, np.nan) for i in range(128)]):
        r = base.copy()
        for i, v in spec:
            r[i] = v
        rows.append(r)
    return np.stack(rows)


def _same_codes(a, b):
    """e4m3 codes equal, with any two NaN codes (0x7F / 0xFF) counted equal."""
    a, b = np.asarray(a, np.uint8), np.asarray(b, np.uint8)
    nan_a, nan_b = (a & 0x7F) == 0x7F, (b & 0x7F) == 0x7F
    return np.array_equal(nan_a, nan_b) and np.array_equal(a[~nan_a], b[~nan_b])


@pytest.mark.parametrize("round_pow2", [True, False])
def test_act_quant_non_finite_blocks_follow_torch(round_pow2):
    """NaN / inf inside a block: torch's amax and clamp keep NaN, the fp32 scale is
    NaN or inf, and the ue8m0 rule gives scale 1 (frexp's exponent for a
    non-finite value is 0); the oracle must do the same."""
    x = _special_blocks()
    q, s = om.act_quant(x, 128, round_pow2)
    tq, ts = _torch_act_quant(x, "ue8m0" if round_pow2 else None)
    assert _same_codes(q, tq)
    assert np.array_equal(s, ts, equal_nan=True)
    if round_pow2:
        assert (s[1:] == 1.0).all()


def test_wire_pack_non_finite_rows_follow_torch():
    """_pack_t (serving/chain.py:208-217) on NaN / inf rows, evaluated by torch."""
    import torch

    x = _special_blocks()
    q, scale = om.wire_pack(x)
    f = torch.from_numpy(x)
    ts = (f.abs().amax(-1, keepdim=True) / 448.0).clamp(min=1e-8, max=torch.finfo(torch.bfloat16).max)
    ts = ts.to(torch.bfloat16)
    tq = (f / ts.float()).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    assert _same_codes(q, tq.view(torch.uint8).numpy())
    assert np.array_equal(scale, ts.float().squeeze(-1).numpy(), equal_nan=True)
