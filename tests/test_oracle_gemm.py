"""CPU pins of the oracle's fp8_gemm / fp4_gemm (torch_ops.py:93-108).

* Exactness-constructed cases: small integer codes and power-of-two scales
  make every partial sum exactly representable, so the result is fixed
  independently of summation order; it is computed here with Python integers
  and rounded to bf16 by torch.
* Brute force: explicit per-element loops over independently decoded
  operands (nibbles unpacked by hand, scales indexed [n // 128][k // 128] and
  [n][k // 32] element by element), float64 sums, bf16 by torch.  A transposed
  operand, a swapped nibble or a wrong scale index fails these.
"""

import math

import numpy as np
import torch

from oracle import moe as om
from oracle.numerics import E2M1_TABLE, E4M3_TABLE


def _bf16(x64) -> np.ndarray:
    return torch.tensor(np.asarray(x64, np.float64), dtype=torch.float64).to(torch.float32).to(
        torch.bfloat16).float().numpy()


def _e4m3_code_of(v: float) -> int:
    return int(np.nonzero(E4M3_TABLE == np.float32(v))[0][0])


def _e2m1_code_of(v: float) -> int:
    return int(np.nonzero(E2M1_TABLE == np.float32(v))[0][0])


def test_fp8_gemm_exact_integers():
    rng = np.random.default_rng(10)
    M, N, K = 3, 256, 256
    vals = [0.0, 1.0, 2.0, 3.0, 4.0, -1.0, -2.0, -3.0]
    ai = rng.integers(0, len(vals), (M, K))
    wi = rng.integers(0, len(vals), (N, K))
    a = np.vectorize(lambda i: _e4m3_code_of(vals[i]))(ai).astype(np.uint8)
    w = np.vectorize(lambda i: _e4m3_code_of(vals[i]))(wi).astype(np.uint8)
    a_s = np.float32([[1.0, 2.0]] * M)                 # per 128-block of K
    w_s = np.float32([[0.5, 4.0], [1.0, 0.25]])        # [N/128, K/128]
    got = om.fp8_gemm(a, a_s, w, w_s)
    for m in range(M):
        for n in range(N):
            acc = 0.0
            for k in range(K):
                acc += vals[ai[m, k]] * a_s[m, k // 128] * vals[wi[n, k]] * w_s[n // 128, k // 128]
            assert got[m, n] == _bf16([acc])[0], (m, n)


def test_fp4_gemm_exact_integers():
    rng = np.random.default_rng(11)
    M, N, K = 2, 64, 128
    fp4 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -1.0, -6.0]
    av = [0.0, 1.0, -2.0, 4.0]
    ai = rng.integers(0, len(av), (M, K))
    wi = rng.integers(0, len(fp4), (N, K))
    a = np.vectorize(lambda i: _e4m3_code_of(av[i]))(ai).astype(np.uint8)
    codes = np.vectorize(lambda i: _e2m1_code_of(fp4[i]))(wi).astype(np.uint8)
    w = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)  # low nibble = even k
    w_s = 2.0 ** rng.integers(-2, 3, (N, K // 32)).astype(np.float32)
    a_s = np.float32([[0.5]] * M)
    got = om.fp4_gemm(a, a_s, w, w_s)
    for m in range(M):
        for n in range(N):
            acc = sum(av[ai[m, k]] * 0.5 * fp4[wi[n, k]] * float(w_s[n, k // 32]) for k in range(K))
            assert got[m, n] == _bf16([acc])[0], (m, n)


def test_fp4_gemm_brute_force_random():
    rng = np.random.default_rng(12)
    M, N, K = 4, 32, 256
    a = rng.integers(0, 256, (M, K), dtype=np.uint8)
    a[(a & 0x7F) == 0x7F] = 0
    a_s = np.exp(rng.uniform(-3, 1, (M, K // 128))).astype(np.float32)
    w = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    w_s = (2.0 ** rng.integers(-6, 2, (N, K // 32))).astype(np.float32)
    got = om.fp4_gemm(a, a_s, w, w_s)
    ref = np.empty((M, N))
    for m in range(M):
        for n in range(N):
            acc = 0.0
            for k in range(K):
                byte = int(w[n, k // 2])
                nib = byte & 0xF if k % 2 == 0 else byte >> 4
                sgn = -1.0 if nib & 8 else 1.0
                e, mm = (nib >> 1) & 3, nib & 1
                wv = sgn * (mm * 0.5 if e == 0 else (1 + mm / 2) * 2.0 ** (e - 1))
                acc += float(E4M3_TABLE[a[m, k]]) * float(a_s[m, k // 128]) * wv * float(w_s[n, k // 32])
            ref[m, n] = acc
    ref = _bf16(ref)
    # both sums are float64 of exact products: the fp32 results agree except at
    # a rounding boundary, where they may differ by one bf16 step
    ulp = np.spacing(np.abs(ref).astype(np.float32)) * 65536
    assert (np.abs(got - ref) <= ulp).all()
    assert np.mean(got == ref) > 0.99


def test_fp8_gemm_brute_force_block_scales():
    rng = np.random.default_rng(13)
    M, N, K = 2, 256, 384
    a = rng.integers(0, 256, (M, K), dtype=np.uint8)
    w = rng.integers(0, 256, (N, K), dtype=np.uint8)
    a[(a & 0x7F) == 0x7F] = 0
    w[(w & 0x7F) == 0x7F] = 0
    a_s = rng.uniform(0.1, 2.0, (M, K // 128)).astype(np.float32)
    w_s = rng.uniform(0.5, 1.5, (2, 3)).astype(np.float32)  # distinct per (n // 128, k // 128)
    got = om.fp8_gemm(a, a_s, w, w_s)
    ref = np.empty((M, N))
    for m in range(M):
        for n in range(N):
            ref[m, n] = math.fsum(float(E4M3_TABLE[a[m, k]]) * float(a_s[m, k // 128]) *
                                  float(E4M3_TABLE[w[n, k]]) * float(w_s[n // 128, k // 128]) for k in range(K))
    ref = _bf16(ref)
    ulp = np.spacing(np.abs(ref).astype(np.float32)) * 65536
    assert (np.abs(got - ref) <= ulp).all()
    assert np.mean(got == ref) > 0.99
