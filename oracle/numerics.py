"""ORACLE (test infrastructure only): number-format codecs written from their definitions.

Nothing in the product imports this package.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg use it, as the
checker.

Formats (OCP MX / OCP FP8 definitions):

* e4m3fn: 1 sign, 4 exponent (bias 7), 3 mantissa bits; no infinities; codes
  0x7F/0xFF are NaN; max finite 448.  Subnormals are m * 2^-9.
* e2m1: 1 sign, 2 exponent (bias 1), 1 mantissa bit -> {0, .5, 1, 1.5, 2, 3, 4, 6}
  (table in wanferenz/model/tensor_layout.py:11-31, wanferenz/kernels/torch_ops.py:13).
  Two codes per byte, low nibble = even element (torch_ops.py:72-74, 82-90).
* e8m0: unsigned exponent byte e -> 2^(e-127); 0xFF is NaN.
* bf16: top 16 bits of an IEEE float32, rounded to nearest even.

Parity status: every codec here is pinned by tests/test_oracle_numerics.py
against torch's own dtype casts over every code / a dense sweep (library
routine) and against hand-computed known answers.
"""

from __future__ import annotations

import numpy as np

FP8_MAX = 448.0
FP4_MAX = 6.0


def _e4m3_table() -> np.ndarray:
    t = np.zeros(256, dtype=np.float32)
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e = (c >> 3) & 0xF
        m = c & 0x7
        if (c & 0x7F) == 0x7F:
            t[c] = np.nan
        elif e == 0:
            t[c] = s * m * 2.0**-9
        else:
            t[c] = s * 2.0 ** (e - 7) * (1.0 + m / 8.0)
    return t


E4M3_TABLE = _e4m3_table()
E2M1_TABLE = np.array(
    [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0],
    dtype=np.float32,
)
# Non-negative finite e4m3 values, ascending with the code (codes 0x00..0x7E).
_E4M3_POS = E4M3_TABLE[:0x7F].astype(np.float64)
_E4M3_MID = (_E4M3_POS[:-1] + _E4M3_POS[1:]) / 2.0


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    return E4M3_TABLE[np.asarray(codes, dtype=np.uint8)]


def e4m3_encode(v: np.ndarray) -> np.ndarray:
    """float32 -> e4m3fn byte, round-to-nearest-even on the magnitude.

    Inputs must already be clamped to [-448, 448] (the reference clamps before
    the cast, torch_ops.py:44); NaN encodes as the e4m3fn NaN 0x7F with the
    float's sign (torch's cast does the same).  The sign bit is taken from the
    float's sign, so -0.0 and negative values that round to zero give 0x80.
    """
    v = np.asarray(v, dtype=np.float32)
    a = np.abs(v).astype(np.float64)
    nan = np.isnan(a)
    if np.any(a[~nan] > FP8_MAX):
        raise ValueError("e4m3_encode: input outside [-448, 448]")
    a = np.where(nan, 0.0, a)
    lo = np.searchsorted(_E4M3_MID, a, side="left")
    hi = np.searchsorted(_E4M3_MID, a, side="right")
    code = lo + ((hi != lo) & (lo % 2 == 1))
    code = np.where(nan, 0x7F, code).astype(np.uint8)
    return code | (np.signbit(v).astype(np.uint8) << 7)


def e2m1_decode_nibbles(packed: np.ndarray) -> np.ndarray:
    """uint8 [..., K/2] -> float32 [..., K]; low nibble is the even element."""
    u = np.asarray(packed, dtype=np.uint8)
    out = np.empty(u.shape[:-1] + (u.shape[-1] * 2,), dtype=np.float32)
    out[..., 0::2] = E2M1_TABLE[u & 0x0F]
    out[..., 1::2] = E2M1_TABLE[u >> 4]
    return out


def e8m0_decode(b: np.ndarray) -> np.ndarray:
    b = np.asarray(b, dtype=np.uint8)
    with np.errstate(over="ignore"):  # code 0xFF overflows before it is set to NaN
        out = np.ldexp(np.float32(1.0), b.astype(np.int32) - 127).astype(np.float32)
    out[b == 0xFF] = np.nan
    return out


def e8m0_encode_pow2(s: np.ndarray) -> np.ndarray:
    """Exact power-of-two float32 -> e8m0 byte (raises if not a power of two)."""
    s = np.asarray(s, dtype=np.float32)
    m, e = np.frexp(s)
    if np.any(m != 0.5):
        raise ValueError("e8m0_encode_pow2: not a power of two")
    return (e - 1 + 127).astype(np.uint8)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest-even bfloat16 value, returned as float32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    bias = np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))
    r = ((u + bias) >> np.uint32(16)) << np.uint32(16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = np.where(nan, u | np.uint32(0x00400000), r).astype(np.uint32)
    return r.view(np.float32).reshape(np.shape(x))


def bf16_bits(x: np.ndarray) -> np.ndarray:
    return (bf16_round(x).view(np.uint32) >> np.uint32(16)).astype(np.uint16)


def from_bf16_bits(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float64).astype(np.float32)
