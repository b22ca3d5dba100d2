"""CPU checks of the synthetic-input generator (wanferenz_amd/synth.py).

The byte streams are SplitMix64 outputs (Steele, Lea and Flood, OOPSLA 2014;
Vigna's reference C code): the first outputs for states 0 and 1234567 are the
published test values.  The GPU fill (wz_synth_fill) is checked against the
same host stream in tests/test_gpu_moe.py.
"""

import numpy as np

from wanferenz_amd import synth


def test_splitmix64_known_answers():
    assert int(synth.draws(0, 0, 1)[0]) == 0xE220A8397B1DCDAF
    assert [int(v) for v in synth.draws(1234567, 0, 5)] == [
        6457827717110365317, 3203168211198807973, 9817491932198370423,
        4593380528125082431, 16408922859458223821]
    # counter-based: any window equals the same slice of a longer run
    assert np.array_equal(synth.draws(99, 1000, 7), synth.draws(99, 0, 2000)[1000:1007])


def test_fills_follow_their_recipes():
    k = synth.stream_key(0, synth.layer_stream(3, synth.S_W13))
    e = synth.fill_e8m0(k, 0, 100000, 119, 123)
    assert e.min() == 119 and e.max() == 123
    f8 = synth.fill_e4m3(k, 0, 100000)
    assert not np.any((f8 & 0x7F) == 0x7F)  # NaN codes replaced (fp8_vector.py:195-197)
    u = synth.fill_f32_uniform(k, 0, 100000, 0.5, 1.5)
    assert u.min() >= 0.5 and u.max() < 1.5
    x = synth.f32_from_bf16_bits(synth.normal_bf16(k, (200000,), 1.0))
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01
    # different layers never share a stream
    assert synth.stream_key(0, synth.layer_stream(0, synth.S_W13)) != synth.stream_key(
        0, synth.layer_stream(1, synth.S_W13))


def test_zipf_bias_orders_popularity():
    b = synth.zipf_bias(256, s=1.1, beta=0.05)
    assert b.shape == (256,) and b.dtype == np.float32
    # bias_e = beta * log p_e, p_e ~ rank^-1.1: consecutive ranks differ by beta * 1.1 * log((r+1)/r)
    srt = np.sort(b)[::-1]
    r = np.arange(1, 256)
    assert np.allclose(srt[:-1] - srt[1:], 0.05 * 1.1 * np.log((r + 1) / r), rtol=1e-4, atol=1e-7)


def test_zipf_exponent_recovers_known_laws():
    """The MLE of a finite Zipf law returns s for expected counts proportional to r^-s
    (the stationary point is exact there), in any order, and grows with the skew."""
    r = np.arange(1, 257, dtype=np.float64)
    for s in (0.5, 1.1, 2.0):
        c = 1e6 * r ** -s
        assert abs(synth.zipf_exponent(c) - s) < 1e-9
        assert abs(synth.zipf_exponent(c[::-1].copy()) - s) < 1e-9
    assert abs(synth.zipf_exponent(np.ones(256))) < 1e-9


def test_committed_zipf_calibration_reproduces():
    """wanferenz_amd/zipf_v4.json: the committed beta routes the calibration batch to
    the committed histogram, whose fitted exponent is the Zipf(1.1) target."""
    import json

    with open(synth.ZIPF_V4_FILE) as f:
        cal = json.load(f)
    x, gw = synth.zipf_v4_calibration_batch(cal["T"])
    counts = synth.route_counts(x, gw, synth.zipf_bias(256, cal["s"], cal["beta"]), cal["k"])
    assert counts.tolist() == cal["counts_per_expert"]
    assert counts.sum() == cal["T"] * cal["k"] and counts.max() <= cal["T"]
    assert abs(synth.zipf_exponent(counts) - 1.1) < 2e-3
    # the strength found by bisection is where the fit crosses s: either side falls short / overshoots
    lo = synth.route_counts(x, gw, synth.zipf_bias(256, 1.1, cal["beta"] * 0.9), 6)
    hi = synth.route_counts(x, gw, synth.zipf_bias(256, 1.1, cal["beta"] * 1.1), 6)
    assert synth.zipf_exponent(lo) < 1.1 < synth.zipf_exponent(hi)
