"""CPU pins of the oracle's FP8 wire format (oracle.moe.wire_pack / wire_unpack,
restating serving/chain.py:208-222) by closed forms and an error bound."""

import numpy as np

from oracle import moe as om
from oracle.numerics import bf16_round, e4m3_decode
from wanferenz_amd import synth


def test_power_of_two_row_is_exact():
    """amax = 448 * 2^k gives scale 2^k exactly (bf16-exact), so e4m3-representable
    multiples of 2^k come back unchanged."""
    for k in (-20, -3, 0, 5, 60):
        row = np.array([448.0, -448.0, 1.5, -0.25, 0.0, 3.5, -96.0, 2.0 ** -9], np.float32) * np.float32(2.0 ** k)
        q, s = om.wire_pack(row[None])
        assert s[0] == np.float32(2.0 ** k)
        assert np.array_equal(e4m3_decode(q[0]) * np.float32(2.0 ** k), row)
        assert np.array_equal(om.wire_unpack(q, s)[0], row)


def test_zero_row_and_amax_maps_to_448():
    q, s = om.wire_pack(np.zeros((1, 64), np.float32))
    assert not q.any() and s[0] > 0 and s[0] == bf16_round(np.float32(1e-8))
    x = bf16_round(synth.f32_from_bf16_bits(synth.normal_bf16(synth.stream_key(5, 40), (16, 512), 3.0)))
    q, s = om.wire_pack(x)
    # the row maximum lands on the e4m3 maximum (a scale of amax/240 or amax/224 would not)
    assert np.all(np.abs(e4m3_decode(q)).max(axis=-1) == 448.0)


def test_round_trip_error_bound():
    """|unpack(pack(x)) - x| <= (2^-4 + 2^-8) |x| + 2^-10 scale: e4m3 keeps 3 mantissa
    bits (half-ulp 2^-4 relative, 2^-10 absolute below 2^-6), bf16 output rounding 2^-9."""
    x = bf16_round(synth.f32_from_bf16_bits(synth.normal_bf16(synth.stream_key(6, 41), (32, 1024), 1.0)))
    x[3] *= np.float32(1e-30)
    x[4] *= np.float32(1e30)
    q, s = om.wire_pack(x)
    y = om.wire_unpack(q, s).astype(np.float64)
    bound = (2.0 ** -4 + 2.0 ** -8) * np.abs(x) + 2.0 ** -10 * s[:, None].astype(np.float64)
    assert np.all(np.abs(y - x) <= bound)
