"""GPU parity of the HIP act_quant / fp8_gemm / fp4_gemm / fp8_linear against the oracle.

Bar: act_quant bit-exact (codes and scales); GEMMs bit-exact on exactness-
constructed inputs (every partial sum representable in fp32, so any
accumulation order gives the same fp32 and hence the same bf16), and within
max|d|/max|ref| <= 1e-2 and cosine >= 0.9999 on random inputs.
"""

import numpy as np
import pytest
import torch

from oracle import moe as om
from oracle.numerics import e8m0_decode, from_bf16_bits
from tests.helpers import bf16_tensor, bits16, bytes8, f32_of_bf16, f32_tensor, u8_tensor
from wanferenz_amd import kernels, synth

pytestmark = pytest.mark.gpu

TOL_REL = 1e-2
TOL_COS = 0.9999


@pytest.fixture(autouse=True)
def _bf16_default():
    """The model runs with torch's default dtype set to bf16 (fp4_grouped.py:451)."""
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    yield
    torch.set_default_dtype(prev)


def _x(seed, M, K, sigma=1.0):
    return synth.normal_bf16(synth.stream_key(seed, synth.S_FP8_X), (M, K), sigma)


def _special_rows(bits):
    """Overwrite blocks with edge cases: all-zero, exact power-of-two amax, tiny, huge."""
    from oracle.numerics import bf16_bits

    b = bits.copy()
    K = b.shape[1]
    if b.shape[0] >= 4 and K >= 256:
        b[0, :128] = 0
        b[1, :128] = bf16_bits(np.full(128, 0.5, np.float32))
        b[1, 5] = bf16_bits(np.float32(448.0 * 2.0))   # amax exactly 2 * 448 -> s = 2
        b[2, 128:256] = bf16_bits(np.linspace(-1e-6, 1e-6, 128).astype(np.float32))
        b[3, :128] = bf16_bits(np.linspace(-3e4, 3e4, 128).astype(np.float32))
        b[3, 130] = bf16_bits(np.float32(-0.0))
    return b


@pytest.mark.parametrize("scale_fmt,scale_dtype", [
    ("ue8m0", torch.float8_e8m0fnu), (None, torch.float32), ("ue8m0", torch.float32)])
@pytest.mark.parametrize("M,K", [(1, 4096), (4, 1024), (37, 2048), (128, 512)])
def test_act_quant_bit_exact(gpu, scale_fmt, scale_dtype, M, K):
    xb = _special_rows(_x(M * 7 + K, M, K))
    x = bf16_tensor(xb, gpu)
    q, s = kernels.act_quant(x, 128, scale_fmt, scale_dtype)
    torch.cuda.synchronize()
    rq, rs = om.act_quant(from_bf16_bits(xb), 128, round_pow2=scale_fmt is not None)
    got_q = bytes8(q)
    assert np.array_equal(got_q, rq), f"{(got_q != rq).sum()} code mismatches"
    if scale_dtype == torch.float8_e8m0fnu:
        got_s = e8m0_decode(bytes8(s))
    else:
        got_s = s.cpu().numpy()
    assert np.array_equal(got_s.view(np.uint32), rs.view(np.uint32))


def _fp4_weight(seed, N, K, e_lo=119, e_hi=123):
    key = synth.stream_key(seed, synth.S_W13)
    w = synth.fill_u8(key, 0, N * K // 2).reshape(N, K // 2)
    ws = synth.fill_e8m0(synth.stream_key(seed, synth.S_W13_S), 0, N * K // 32, e_lo, e_hi).reshape(N, K // 32)
    return w, ws


def _fp8_weight(seed, N, K, fp32_scales):
    w = synth.fill_e4m3(synth.stream_key(seed, synth.S_FP8_W), 0, N * K).reshape(N, K)
    nb, kb = (N + 127) // 128, (K + 127) // 128
    if fp32_scales:
        ws = synth.fill_f32_uniform(synth.stream_key(seed, synth.S_FP8_W_S), 0, nb * kb, 0.5, 1.5).reshape(nb, kb)
    else:
        ws = synth.fill_e8m0(synth.stream_key(seed, synth.S_FP8_W_S), 0, nb * kb, 112, 116).reshape(nb, kb)
    return w, ws


def _close(got, ref):
    return om.max_rel_err(got, ref), om.cosine(got, ref)


@pytest.mark.parametrize("act_fmt", ["ue8m0", None])
@pytest.mark.parametrize("M,N,K", [(1, 256, 1024), (4, 512, 4096), (8, 128, 2048), (33, 256, 512), (130, 128, 1024)])
def test_fp4_gemm_random(gpu, act_fmt, M, N, K):
    xb = _x(M + N + K, M, K)
    sd = torch.float8_e8m0fnu if act_fmt else torch.float32
    x = bf16_tensor(xb, gpu)
    q, s = kernels.act_quant(x, 128, act_fmt, sd)
    w, ws = _fp4_weight(N * 3 + K, N, K)
    c = kernels.fp4_gemm(q, s, u8_tensor(w, gpu, torch.float4_e2m1fn_x2), u8_tensor(ws, gpu, torch.float8_e8m0fnu), sd)
    got = f32_of_bf16(c)
    rq, rs = om.act_quant(from_bf16_bits(xb), 128, act_fmt is not None)
    ref = om.fp4_gemm(rq, rs, w, e8m0_decode(ws))
    rel, cos = _close(got, ref)
    assert rel <= TOL_REL and cos >= TOL_COS, (rel, cos)
    assert (got == ref).mean() > 0.9, (got == ref).mean()


@pytest.mark.parametrize("w_fp32", [False, True])
@pytest.mark.parametrize("act_fmt", ["ue8m0", None])
@pytest.mark.parametrize("M,N,K", [(1, 256, 1024), (4, 1024, 4096), (8, 384, 2048), (20, 128, 512), (128, 256, 1024)])
def test_fp8_gemm_random(gpu, w_fp32, act_fmt, M, N, K):
    xb = _x(M + 2 * N + K, M, K)
    sd = torch.float8_e8m0fnu if act_fmt else torch.float32
    x = bf16_tensor(xb, gpu)
    q, s = kernels.act_quant(x, 128, act_fmt, sd)
    w, ws = _fp8_weight(N + K, N, K, w_fp32)
    wst = f32_tensor(ws, gpu) if w_fp32 else u8_tensor(ws, gpu, torch.float8_e8m0fnu)
    c = kernels.fp8_gemm(q, s, u8_tensor(w, gpu, torch.float8_e4m3fn), wst, sd)
    got = f32_of_bf16(c)
    rq, rs = om.act_quant(from_bf16_bits(xb), 128, act_fmt is not None)
    ref = om.fp8_gemm(rq, rs, w, ws if w_fp32 else e8m0_decode(ws))
    rel, cos = _close(got, ref)
    assert rel <= TOL_REL and cos >= TOL_COS, (rel, cos)
    # fused act_quant: same codes, same math
    y = kernels.fp8_linear(x, u8_tensor(w, gpu, torch.float8_e4m3fn), wst, act_fmt, sd)
    got2 = f32_of_bf16(y)
    rel2, cos2 = _close(got2, ref)
    assert rel2 <= TOL_REL and cos2 >= TOL_COS, (rel2, cos2)


def _exact_codes(seed, n, table_codes):
    d = synth.draws(synth.stream_key(seed, 99), 0, n)
    return np.asarray(table_codes, np.uint8)[(d % np.uint64(len(table_codes))).astype(np.int64)]


@pytest.mark.parametrize("M,N,K", [(1, 128, 1024), (5, 256, 2048), (16, 64, 4096), (40, 128, 512)])
def test_fp4_gemm_exact(gpu, M, N, K):
    """Small codes and unit scales: every partial sum is exact in fp32 -> bit-exact bf16."""
    # e4m3 codes of 0, +-0.5, +-1, +-1.5, +-2 and e2m1 codes 0..15 (|v| <= 6)
    a_codes = _exact_codes(M * K, M * K, [0x00, 0x30, 0xB0, 0x38, 0xB8, 0x3C, 0xBC, 0x40, 0xC0]).reshape(M, K)
    w = synth.fill_u8(synth.stream_key(N, 7), 0, N * K // 2).reshape(N, K // 2)
    ws = np.full((N, K // 32), 127, np.uint8)
    a_s = np.full((M, K // 128), 127, np.uint8)
    c = kernels.fp4_gemm(u8_tensor(a_codes, gpu, torch.float8_e4m3fn), u8_tensor(a_s, gpu, torch.float8_e8m0fnu),
                         u8_tensor(w, gpu, torch.float4_e2m1fn_x2), u8_tensor(ws, gpu, torch.float8_e8m0fnu))
    got = bits16(c)
    ref = om.fp4_gemm(a_codes, e8m0_decode(a_s), w, e8m0_decode(ws))
    from oracle.numerics import bf16_bits
    assert np.array_equal(got, bf16_bits(ref))


@pytest.mark.parametrize("act_fmt", ["ue8m0", None])
@pytest.mark.parametrize("M,N,K", [(20, 256, 1024), (130, 128, 2048), (200, 384, 4096), (64, 16, 512),
                                   (300, 256, 1024), (512, 512, 2048), (256, 768, 1536), (384, 512, 4096)])
def test_fp4_gemm_packed_random(gpu, act_fmt, M, N, K):
    """fp4_gemm on the packed weight against the oracle: the prefill tile GEMM, and
    at M >= 256 with N a multiple of 256 and power-of-two activation scales the
    128 x 256 big-tile kernel (ragged M; K = 1536 leaves the last scale dword half
    used)."""
    xb = _x(M + 5 * N + K, M, K)
    sd = torch.float8_e8m0fnu if act_fmt else torch.float32
    x = bf16_tensor(xb, gpu)
    q, s = kernels.act_quant(x, 128, act_fmt, sd)
    w, ws = _fp4_weight(N * 5 + K, N, K)
    lin = kernels.PackedFp4Linear(u8_tensor(w, gpu, torch.float4_e2m1fn_x2), u8_tensor(ws, gpu, torch.float8_e8m0fnu))
    got = f32_of_bf16(lin.gemm(q, s))
    rq, rs = om.act_quant(from_bf16_bits(xb), 128, act_fmt is not None)
    ref = om.fp4_gemm(rq, rs, w, e8m0_decode(ws))
    rel, cos = _close(got, ref)
    assert rel <= TOL_REL and cos >= TOL_COS, (rel, cos)
    assert (got == ref).mean() > 0.9, (got == ref).mean()


@pytest.mark.parametrize("M,N,K", [(17, 128, 1024), (100, 256, 2048), (64, 128, 4096), (260, 256, 2048),
                                   (512, 512, 1024)])
def test_fp4_gemm_packed_exact(gpu, M, N, K):
    """Small codes and unit scales through the packed tile GEMM (and the big-tile
    kernel at M >= 256): bit-exact bf16."""
    a_codes = _exact_codes(M * K + 3, M * K, [0x00, 0x30, 0xB0, 0x38, 0xB8, 0x3C, 0xBC, 0x40, 0xC0]).reshape(M, K)
    w = synth.fill_u8(synth.stream_key(N + 3, 7), 0, N * K // 2).reshape(N, K // 2)
    ws = np.full((N, K // 32), 127, np.uint8)
    a_s = np.full((M, K // 128), 127, np.uint8)
    lin = kernels.PackedFp4Linear(u8_tensor(w, gpu, torch.float4_e2m1fn_x2), u8_tensor(ws, gpu, torch.float8_e8m0fnu))
    c = lin.gemm(u8_tensor(a_codes, gpu, torch.float8_e4m3fn), u8_tensor(a_s, gpu, torch.float8_e8m0fnu))
    from oracle.numerics import bf16_bits
    ref = om.fp4_gemm(a_codes, e8m0_decode(a_s), w, e8m0_decode(ws))
    assert np.array_equal(bits16(c), bf16_bits(ref))


@pytest.mark.parametrize("M,N,K", [(1, 128, 1024), (7, 256, 2048), (16, 128, 4096)])
def test_fp8_gemm_exact(gpu, M, N, K):
    codes = [0x00, 0x30, 0xB0, 0x38, 0xB8, 0x3C, 0xBC, 0x40, 0xC0]
    a_codes = _exact_codes(M * K + 1, M * K, codes).reshape(M, K)
    w = _exact_codes(N * K + 2, N * K, codes).reshape(N, K)
    ws = np.full(((N + 127) // 128, K // 128), 127, np.uint8)
    a_s = np.full((M, K // 128), 127, np.uint8)
    c = kernels.fp8_gemm(u8_tensor(a_codes, gpu, torch.float8_e4m3fn), u8_tensor(a_s, gpu, torch.float8_e8m0fnu),
                         u8_tensor(w, gpu, torch.float8_e4m3fn), u8_tensor(ws, gpu, torch.float8_e8m0fnu))
    from oracle.numerics import bf16_bits
    ref = om.fp8_gemm(a_codes, e8m0_decode(a_s), w, e8m0_decode(ws))
    assert np.array_equal(bits16(c), bf16_bits(ref))


def test_fp4_gemm_single_nonzero_layout(gpu):
    """One nonzero weight nibble at a time: pins row/column/K placement and nibble order."""
    M, N, K = 16, 16, 128
    a = np.zeros((M, K), np.uint8)
    rng = np.random.default_rng(0)
    for m in range(M):
        a[m] = np.where(rng.random(K) < 0.5, 0x38, 0x40)  # 1.0 or 2.0
    a_s = np.full((M, 1), 127, np.uint8)
    ws = np.full((N, K // 32), 127, np.uint8)
    for (n, k) in [(0, 0), (0, 1), (3, 37), (15, 127), (9, 64), (4, 95)]:
        w = np.zeros((N, K // 2), np.uint8)
        w[n, k // 2] = (0x2 << (4 * (k % 2)))  # e2m1 code 2 = 1.0 at element k
        c = kernels.fp4_gemm(u8_tensor(a, gpu, torch.float8_e4m3fn), u8_tensor(a_s, gpu, torch.float8_e8m0fnu),
                             u8_tensor(w, gpu, torch.float4_e2m1fn_x2), u8_tensor(ws, gpu, torch.float8_e8m0fnu))
        got = f32_of_bf16(c)
        exp = np.zeros((M, N), np.float32)
        exp[:, n] = np.where(a[:, k] == 0x38, 1.0, 2.0)
        assert np.array_equal(got, exp), (n, k)


def test_fp8_gemm_single_nonzero_layout(gpu):
    """One nonzero FP8 weight at a time: pins row/column/K placement of the FP8 operands."""
    M, N, K = 16, 16, 128
    rng = np.random.default_rng(1)
    a = np.where(rng.random((M, K)) < 0.5, 0x38, 0x40).astype(np.uint8)
    a_s = np.full((M, 1), 127, np.uint8)
    ws = np.full((1, 1), 127, np.uint8)
    for (n, k) in [(0, 0), (0, 1), (3, 37), (15, 127), (9, 64), (4, 95)]:
        w = np.zeros((N, K), np.uint8)
        w[n, k] = 0x38
        c = kernels.fp8_gemm(u8_tensor(a, gpu, torch.float8_e4m3fn), u8_tensor(a_s, gpu, torch.float8_e8m0fnu),
                             u8_tensor(w, gpu, torch.float8_e4m3fn), u8_tensor(ws, gpu, torch.float8_e8m0fnu))
        got = f32_of_bf16(c)
        exp = np.zeros((M, N), np.float32)
        exp[:, n] = np.where(a[:, k] == 0x38, 1.0, 2.0)
        assert np.array_equal(got, exp), (n, k, got[:, n], np.nonzero(got))


def test_fp4_gemm_k_mapping(gpu):
    """Map each weight element k to the activation column it meets (bits of k' in rows 0..6)."""
    M, N, K = 16, 16, 128
    a = np.zeros((M, K), np.uint8)
    for m in range(7):
        a[m] = np.where((np.arange(K) >> m) & 1, 0x38, 0x00)
    a[7] = 0x38
    a_s = np.full((M, 1), 127, np.uint8)
    ws = np.full((N, K // 32), 127, np.uint8)
    bad = []
    for k in range(K):
        w = np.zeros((N, K // 2), np.uint8)
        w[5, k // 2] = (0x2 << (4 * (k % 2)))
        c = kernels.fp4_gemm(u8_tensor(a, gpu, torch.float8_e4m3fn), u8_tensor(a_s, gpu, torch.float8_e8m0fnu),
                             u8_tensor(w, gpu, torch.float4_e2m1fn_x2), u8_tensor(ws, gpu, torch.float8_e8m0fnu))
        got = f32_of_bf16(c)
        cols = np.nonzero(got[7])[0].tolist()
        kk = int(sum(int(got[m, 5] != 0) << m for m in range(7)))
        if cols != [5] or kk != k:
            bad.append((k, kk, cols))
    assert not bad, f"k -> (k', cols): {bad}"


@pytest.mark.parametrize("T,D", [(1, 4096), (4, 4096), (37, 1024), (3, 7168)])
def test_rms_norm_matches_oracle(gpu, T, D):
    """RMSNorm (architecture.py:217-230) vs the oracle: the fp32 sum of squares runs in
    a different order, so outputs may differ by one bf16 ulp where the fp32 product
    lands next to a rounding boundary; nearly all elements are bit-equal."""
    xb = _x(11 + T, T, D, 3.0)
    wgt = synth.fill_f32_uniform(synth.stream_key(12, synth.S_FP8_X), 0, D, 0.5, 1.5)
    y = kernels.rms_norm(bf16_tensor(xb, gpu).view(T, D), f32_tensor(wgt, gpu), 1e-6)
    torch.cuda.synchronize()
    got = f32_of_bf16(y)
    ref = om.rmsnorm(from_bf16_bits(xb).reshape(T, D), wgt, 1e-6)
    rel = np.abs(got - ref) / np.maximum(np.abs(ref), 1e-30)
    assert rel.max() <= 2.0 ** -7, rel.max()          # at most one bf16 ulp
    assert (got == ref).mean() >= 0.99


def test_rms_norm_closed_forms(gpu):
    """An all-zero row gives zeros (rsqrt(eps) * 0); a constant row of +-c with unit
    weight gives c / sqrt(c^2 + eps) = 1 - O(1e-7), which rounds to exactly +-1 in bf16."""
    from oracle.numerics import bf16_bits

    D = 2048
    xf = np.zeros((4, D), np.float32)
    xf[1] = 0.5
    xf[2] = -3.0
    xf[3, : D // 2] = 2.0
    xf[3, D // 2:] = -2.0
    y = kernels.rms_norm(bf16_tensor(bf16_bits(xf), gpu), f32_tensor(np.ones(D, np.float32), gpu))
    torch.cuda.synchronize()
    got = f32_of_bf16(y)
    assert not got[0].any()
    assert np.all(got[1] == 1.0) and np.all(got[2] == -1.0)
    assert np.all(got[3, : D // 2] == 1.0) and np.all(got[3, D // 2:] == -1.0)


def test_add_bf16_is_one_rounding(gpu):
    """a + b as one IEEE fp32 add (round to nearest even) and one bf16 rounding, the
    same two steps numpy's float32 add and the oracle's bf16_round take: bit-equal."""
    n = 4096 * 5
    a = _x(31, 1, n)
    b = _x(32, 1, n)
    out = kernels.add(bf16_tensor(a, gpu), bf16_tensor(b, gpu))
    torch.cuda.synchronize()
    from oracle.numerics import bf16_round

    ref = bf16_round((from_bf16_bits(a) + from_bf16_bits(b)).astype(np.float32))
    assert np.array_equal(f32_of_bf16(out).ravel(), ref.ravel())


# the dense projections of the decode block: cfg-3 widths, then the V4 attention
# projections wq_a, wkv, wq_b, wo_b and the indexer's wq_b (fp8_vector.py:505-510)
PROJ_SHAPES = [(4096, 1024), (1024, 4096), (4096, 4096), (16384, 4096),
               (512, 4096), (32768, 1024), (4096, 8192), (8192, 1024)]


@pytest.mark.parametrize("w_fp32", [True, False])
@pytest.mark.parametrize("N,K", PROJ_SHAPES)
@pytest.mark.parametrize("M", [1, 4, 8, 17, 32, 128])
def test_fp8_linear_projection_shapes(gpu, w_fp32, N, K, M):
    """fp8_linear (act_quant fused) at the dense projection shapes, weights generated on
    the device by the same hash stream as the host generator; the oracle checks three
    128-row weight blocks (first, middle, last) of every output."""
    w = torch.empty(N, K, dtype=torch.uint8, device=gpu)
    synth.device_fill(w, synth.stream_key(N + K, synth.S_FP8_W), synth.FILL_E4M3)
    nb, kb = N // 128, K // 128
    if w_fp32:
        ws = torch.empty(nb, kb, dtype=torch.float32, device=gpu)
        synth.device_fill(ws, synth.stream_key(N + K, synth.S_FP8_W_S), synth.FILL_F32_UNIFORM, 0.5, 1.5)
    else:
        ws = torch.empty(nb, kb, dtype=torch.uint8, device=gpu)
        synth.device_fill(ws, synth.stream_key(N + K, synth.S_FP8_W_S), synth.FILL_E8M0, 112, 116)
        ws = ws.view(torch.float8_e8m0fnu)
    xb = _x(M * 7 + K, M, K)
    y = kernels.fp8_linear(bf16_tensor(xb, gpu), w.view(torch.float8_e4m3fn), ws, "ue8m0", torch.float32)
    torch.cuda.synchronize()
    got = f32_of_bf16(y)
    blocks = sorted({0, nb // 2, nb - 1})
    rows = np.concatenate([np.arange(b * 128, b * 128 + 128) for b in blocks])
    w_sub = bytes8(w[torch.from_numpy(rows).to(gpu)])
    ws_sub = ws[blocks].cpu()
    ws_sub = ws_sub.numpy() if w_fp32 else e8m0_decode(ws_sub.view(torch.uint8).numpy())
    rq, rs = om.act_quant(from_bf16_bits(xb), 128, True)
    ref = om.fp8_gemm(rq, rs, w_sub, ws_sub)
    rel, cos = _close(got[:, rows], ref)
    assert rel <= TOL_REL and cos >= TOL_COS, (rel, cos)
    # the packed-weight path (GEMV at M <= 16, act_quant + tile GEMM above)
    lin = kernels.PackedFp8Linear(w.view(torch.float8_e4m3fn), ws, "ue8m0")
    y2 = lin(bf16_tensor(xb, gpu))
    torch.cuda.synchronize()
    rel2, cos2 = _close(f32_of_bf16(y2)[:, rows], ref)
    assert rel2 <= TOL_REL and cos2 >= TOL_COS, (rel2, cos2)


@pytest.mark.parametrize("M,N,K", [(1, 256, 4096), (5, 512, 1024), (16, 128, 2048), (40, 256, 4096),
                                   (3, 128, 1536), (1, 512, 8192), (16, 384, 8192), (2, 4096, 1024),
                                   (4, 256, 4096), (9, 256, 4096), (12, 128, 1024), (5, 256, 8192),
                                   (6, 256, 8192), (8, 256, 8192), (12, 128, 4096), (24, 256, 1024),
                                   (33, 256, 8192), (64, 256, 4096), (130, 384, 1024), (200, 128, 2048),
                                   (257, 128, 1536)])
def test_fp8_linear_packed_exact(gpu, M, N, K):
    """x in {0, +-0.5, +-1, +-1.5} with one 2.0 per 128-block quantises exactly (ue8m0
    scale 2^-7), weight codes of the same values with unit scales: every partial sum
    is exact in fp32, so the packed linear must equal the oracle bit for bit, on the
    GEMV path (M <= 16) and the quantise + tile GEMM path (M = 40, K = 1536).  The
    one-tile GEMV quantises x in LDS in 1, 2, 4 or 8 passes per wave by M x K / 128
    (M = 1, 4, 12, 9 / 5 at K = 4096 / 8192); M = 6, 8 at K = 8192 and 12 at 4096 hold
    more than 64 KB of LDS; M = 16 at K = 8192 needs more passes and runs the ring
    kernel."""
    from oracle.numerics import bf16_bits

    vals = np.array([0.0, 0.5, -0.5, 1.0, -1.0, 1.5, -1.5], np.float32)
    d = synth.draws(synth.stream_key(M * N + K, 98), 0, M * K)
    xf = vals[(d % np.uint64(len(vals))).astype(np.int64)].reshape(M, K)
    xf[:, ::128] = 2.0
    codes = [0x00, 0x30, 0xB0, 0x38, 0xB8, 0x3C, 0xBC, 0x40, 0xC0]
    w = _exact_codes(N * K + 3, N * K, codes).reshape(N, K)
    ws = np.full(((N + 127) // 128, K // 128), 127, np.uint8)
    wt = u8_tensor(w, gpu, torch.float8_e4m3fn)
    wst = u8_tensor(ws, gpu, torch.float8_e8m0fnu)
    lin = kernels.PackedFp8Linear(wt, wst, "ue8m0")
    y = lin(bf16_tensor(bf16_bits(xf), gpu))
    torch.cuda.synchronize()
    rq, rs = om.act_quant(xf, 128, True)
    ref = om.fp8_gemm(rq, rs, w, e8m0_decode(ws))
    assert np.array_equal(bits16(y), bf16_bits(ref))



@pytest.mark.parametrize("N,K", [(16 * (1024 * 9 + 8), 1024), (16 * (1024 * 5 + 8), 2048),
                                 (16 * (512 * 5 + 8), 4096), (16 * (256 * 5 + 8), 8192)])
def test_fp8_gemv_ring_every_tile(gpu, N, K):
    """The packed GEMV at an N where every workgroup (at most 4 per CU) streams more than
    twice its ring depth of 16-column tiles, with a ragged last round: every tile of the
    output is compared with a float32 torch statement of fp8_gemm on the dequantised
    operands (act_quant by the oracle), row block by row block."""
    M = 3
    w = torch.empty(N, K, dtype=torch.uint8, device=gpu)
    synth.device_fill(w, synth.stream_key(N + K + 1, synth.S_FP8_W), synth.FILL_E4M3)
    ws = torch.empty(N // 128, K // 128, dtype=torch.uint8, device=gpu)
    synth.device_fill(ws, synth.stream_key(N + K + 1, synth.S_FP8_W_S), synth.FILL_E8M0, 112, 116)
    ws = ws.view(torch.float8_e8m0fnu)
    xb = _x(N + K, M, K)
    lin = kernels.PackedFp8Linear(w.view(torch.float8_e4m3fn), ws, "ue8m0")
    y = f32_of_bf16(lin(bf16_tensor(xb, gpu)))
    rq, rs = om.act_quant(from_bf16_bits(xb), 128, True)
    xd = torch.from_numpy(np.ascontiguousarray(om.dequant_act(rq, rs), dtype=np.float32)).to(gpu)
    wsf = ws.view(torch.uint8).to(torch.int32)
    wsf = torch.ldexp(torch.ones_like(wsf, dtype=torch.float32), wsf - 127)
    ref = torch.empty(M, N, dtype=torch.float32, device=gpu)
    for r0 in range(0, N, 8192):
        wd = w[r0:r0 + 8192].view(torch.float8_e4m3fn).float().view(-1, K // 128, 128)
        wd = (wd * wsf[r0 // 128:(r0 + 8192) // 128].repeat_interleave(128, 0)[:, :, None]).view(-1, K)
        ref[:, r0:r0 + 8192] = xd @ wd.T
    torch.cuda.synchronize()
    ref = ref.cpu().numpy()
    for r0 in range(0, N, 16 * 512):
        rel, cos = _close(y[:, r0:r0 + 16 * 512], ref[:, r0:r0 + 16 * 512])
        assert rel <= TOL_REL and cos >= TOL_COS, (r0, rel, cos)

def _wire_rows(seed, M, D):
    from oracle.numerics import bf16_bits

    x = from_bf16_bits(_x(seed, M, D, 2.0)).reshape(M, D)
    if M >= 4:
        x[0] = 0.0
        x[1] *= np.float32(1e-33)   # scales near the 1e-8 floor
        x[2] = np.float32(448.0 * 2.0 ** 7) * np.sign(x[2])
        x[3, 7] = np.float32(3.0e38)
    return bf16_bits(x.astype(np.float32))


@pytest.mark.parametrize("M,D", [(1, 4096), (5, 1024), (33, 7168), (8, 520)])
def test_wire_pack_unpack_bit_exact(gpu, M, D):
    """The FP8 stage-boundary format (serving/chain.py:208-222) vs the oracle: codes,
    bf16 scales and the unpacked bf16 values bit for bit."""
    xb = _wire_rows(41 + M, M, D)
    q, s = kernels.wire_pack(bf16_tensor(xb, gpu).view(M, D))
    y = kernels.wire_unpack(q, s)
    torch.cuda.synchronize()
    rq, rs = om.wire_pack(from_bf16_bits(xb).reshape(M, D))
    assert np.array_equal(bytes8(q), rq)
    assert np.array_equal(f32_of_bf16(s), rs)
    assert np.array_equal(f32_of_bf16(y).reshape(M, D), om.wire_unpack(rq, rs))


@pytest.mark.parametrize("scale_fmt,scale_dtype", [("ue8m0", torch.float8_e8m0fnu), (None, torch.float32)])
@pytest.mark.parametrize("T,D", [(1, 4096), (4, 7168), (37, 1024)])
def test_rms_norm_quant_is_norm_then_act_quant(gpu, scale_fmt, scale_dtype, T, D):
    """The fused producer equals rms_norm followed by act_quant bit for bit (same
    arithmetic), and the oracle's act_quant of that normalised row."""
    xb = _x(51 + T, T, D, 2.0)
    wgt = synth.fill_f32_uniform(synth.stream_key(52, synth.S_NORM), 0, D, 0.5, 1.5)
    x, w = bf16_tensor(xb, gpu).view(T, D), f32_tensor(wgt, gpu)
    q, s = kernels.rms_norm_quant(x, w, 1e-6, scale_fmt, scale_dtype)
    y = kernels.rms_norm(x, w, 1e-6)
    q2, s2 = kernels.act_quant(y, 128, scale_fmt, scale_dtype)
    torch.cuda.synchronize()
    assert torch.equal(q.view(torch.uint8), q2.view(torch.uint8))
    assert torch.equal(s.view(torch.uint8), s2.view(torch.uint8))
    rq, rs = om.act_quant(f32_of_bf16(y).reshape(T, D), 128, scale_fmt is not None)
    assert np.array_equal(bytes8(q).reshape(T, D), rq)
    got_s = e8m0_decode(bytes8(s)) if scale_fmt else s.cpu().numpy()
    assert np.array_equal(got_s.reshape(rs.shape), rs)


@pytest.mark.parametrize("T,D", [(4, 4096), (3, 1024), (16, 256)])
def test_add_rms_norm_quant_is_add_then_norm_quant(gpu, T, D):
    """The residual step fused into the norm: h equals the bf16 add of x and b bit for
    bit (the oracle's fp32 sum rounded once), and (q, s) equal rms_norm_quant of h."""
    from oracle.numerics import bf16_round

    xb, bb = _x(61 + T, T, D, 2.0), _x(62 + T, T, D, 1.0)
    wgt = synth.fill_f32_uniform(synth.stream_key(63, synth.S_NORM), 0, D, 0.5, 1.5)
    x, b, w = bf16_tensor(xb, gpu).view(T, D), bf16_tensor(bb, gpu).view(T, D), f32_tensor(wgt, gpu)
    h, q, s = kernels.add_rms_norm_quant(x, b, w, 1e-6)
    q2, s2 = kernels.rms_norm_quant(h, w, 1e-6)
    torch.cuda.synchronize()
    ref = bf16_round((from_bf16_bits(xb) + from_bf16_bits(bb)).astype(np.float32)).reshape(T, D)
    assert np.array_equal(f32_of_bf16(h), ref)
    assert torch.equal(q.view(torch.uint8), q2.view(torch.uint8))
    assert torch.equal(s.view(torch.uint8), s2.view(torch.uint8))


@pytest.mark.parametrize("M,N,K", [(4, 4096, 8192), (1, 1024, 4096), (16, 512, 1024), (40, 256, 1024),
                                   (3, 128, 1536), (24, 1024, 1024), (33, 1024, 4096), (128, 4096, 4096)])
def test_fp8_linear_residual_epilogue(gpu, M, N, K):
    """y = residual + linear(x): the GEMV epilogue (M <= 16, K in the GEMV set) and the
    tile GEMM followed by an add both give bf16(bf16(linear(x)) + residual), i.e. the
    packed linear's own output added to the residual as a bf16 tensor add, bit for bit;
    the pre-quantised entry (gemm) does the same from rms_norm_quant-style input."""
    from oracle.numerics import bf16_round

    w, ws = __import__("wanferenz_amd.stage", fromlist=["synthetic_linear"]).synthetic_linear(
        N, K, M * 7 + N + K, gpu, fp32_scales=False)
    lin = kernels.PackedFp8Linear(w, ws, "ue8m0")
    xb, rb = _x(M * 3 + K, M, K), _x(M * 5 + N, M, N, 4.0)
    x, r = bf16_tensor(xb, gpu).view(M, K), bf16_tensor(rb, gpu).view(M, N)
    plain = lin(x)
    fused = lin(x, residual=r)
    q, qs = kernels.act_quant(x, 128, "ue8m0", torch.float8_e8m0fnu)
    plain_q = lin.gemm(q, qs)
    fused_q = lin.gemm(q, qs, residual=r)
    torch.cuda.synchronize()
    ref = bf16_round((f32_of_bf16(plain) + from_bf16_bits(rb).reshape(M, N)).astype(np.float32))
    assert np.array_equal(f32_of_bf16(fused), ref)
    assert torch.equal(plain_q, plain)
    assert torch.equal(fused_q, fused)
    with pytest.raises(Exception):
        lin(x, out=r, residual=r)  # the residual may not be the output


@pytest.mark.parametrize("M,N0,N1,K", [(4, 1024, 512, 4096), (4, 32768, 8192, 1024), (1, 256, 128, 8192),
                                        (24, 256, 384, 1024), (3, 128, 48, 256), (40, 1024, 512, 4096),
                                        (128, 32768, 8192, 1024), (17, 256, 384, 8192)])
def test_fp8_pair_equals_two_linears(gpu, M, N0, N1, K):
    """Two stacked projections in one launch give each projection's own output bit
    for bit (GEMV path at M <= 16 and K in its set, the two tile GEMMs otherwise)."""
    from wanferenz_amd import stage

    w0, s0 = stage.synthetic_linear(N0, K, N0 + K, gpu, fp32_scales=False)
    w1, s1 = stage.synthetic_linear(N1, K, N1 + K + 1, gpu, fp32_scales=False)
    pair = kernels.PackedFp8Pair(w0, s0, w1, s1)
    l0, l1 = kernels.PackedFp8Linear(w0, s0), kernels.PackedFp8Linear(w1, s1)
    q, qs = kernels.act_quant(bf16_tensor(_x(M + K, M, K), gpu).view(M, K), 128, "ue8m0", torch.float8_e8m0fnu)
    y0, y1 = pair.gemm(q, qs)
    torch.cuda.synchronize()
    assert torch.equal(y0, l0.gemm(q, qs)) and torch.equal(y1, l1.gemm(q, qs))


@pytest.mark.parametrize("M,N,K", [(1, 1024, 4096), (4, 256, 8192), (8, 512, 1024), (16, 128, 2048),
                                   (3, 40960, 1024), (24, 512, 1024), (40, 1024, 4096), (128, 512, 8192)])
def test_fp8_linear_packed_float_act_scales(gpu, M, N, K):
    """The packed linear with non-power-of-two activation scales (scale_fmt None:
    amax / 448 as float32, applied on the VALU per K-block), on the one-tile GEMV
    (its LDS quantisation) and the ring kernel (N = 40960), against the oracle's
    act_quant(round_pow2=False) and fp8_gemm."""
    from wanferenz_amd import stage

    w, ws = stage.synthetic_linear(N, K, N + K + 11, gpu, fp32_scales=True)
    xb = _x(M * 11 + K, M, K)
    lin = kernels.PackedFp8Linear(w, ws, None)
    got = f32_of_bf16(lin(bf16_tensor(xb, gpu).view(M, K)))
    rq, rs = om.act_quant(from_bf16_bits(xb), 128, False)
    rows = np.arange(min(N, 1024))
    ref = om.fp8_gemm(rq, rs, bytes8(w[:rows.size]).reshape(rows.size, K), ws[: (rows.size + 127) // 128].cpu().numpy())
    rel, cos = _close(got[:, rows], ref)
    assert rel <= TOL_REL and cos >= TOL_COS, (rel, cos)


def test_pair_outputs_are_checked(gpu):
    """Outputs of the wrong size, dtype or layout are refused before any launch."""
    from wanferenz_amd import stage

    w0, s0 = stage.synthetic_linear(256, 1024, 31, gpu, fp32_scales=False)
    w1, s1 = stage.synthetic_linear(128, 1024, 32, gpu, fp32_scales=False)
    pair = kernels.PackedFp8Pair(w0, s0, w1, s1)
    x = bf16_tensor(_x(5, 4, 1024), gpu).view(4, 1024)
    nw = torch.ones(1024, dtype=torch.float32, device=gpu)
    y0 = torch.empty(4, 256, dtype=torch.bfloat16, device=gpu)
    y1 = torch.empty(4, 128, dtype=torch.bfloat16, device=gpu)
    for bad in ((y0[:1], y1), (y0, y1.float()), (y0.t(), y1)):
        with pytest.raises(ValueError):
            pair.norm_gemm(x, nw, out=bad)
    with pytest.raises(ValueError):
        pair.norm_gemm(x, nw, b=x.clone(), sum_out=torch.empty(2, 1024, dtype=torch.bfloat16, device=gpu))
    q, qs = kernels.rms_norm_quant(x, nw)
    with pytest.raises(ValueError):
        pair.gemm(q, qs, out=(y0[:2], y1))
    pair.norm_gemm(x, nw, out=(y0, y1))
    torch.cuda.synchronize()


@pytest.mark.parametrize("with_b", [False, True])
@pytest.mark.parametrize("M,K,N0", [(4, 4096, 256), (3, 1024, 256), (3, 1024, 8192)])
def test_fused_norm_pair_float_act_scales(gpu, with_b, M, K, N0):
    """norm_gemm with non-power-of-two activation scales (scale_fmt None, float32
    scales) = rms_norm_quant / add_rms_norm_quant with the same scales, then the
    pair's GEMV, bit for bit; N0 = 8192 at K = 1024: more than 512 tiles (the
    projection of the normed query latent is that wide)."""
    from wanferenz_amd import stage

    w0, s0 = stage.synthetic_linear(N0, K, K + 21, gpu, fp32_scales=True)
    w1, s1 = stage.synthetic_linear(128, K, K + 22, gpu, fp32_scales=True)
    pair = kernels.PackedFp8Pair(w0, s0, w1, s1, None)
    x = bf16_tensor(_x(M * 7 + K, M, K), gpu).view(M, K)
    nw = torch.from_numpy(np.linspace(0.25, 2.0, K, dtype=np.float32)).to(gpu)
    f32 = dict(scale_fmt=None, scale_dtype=torch.float32)
    if with_b:
        b = bf16_tensor(_x(M * 9 + K, M, K), gpu).view(M, K)
        h, q, qs = kernels.add_rms_norm_quant(x, b, nw, 1e-6, **f32)
        hf, y0, y1 = pair.norm_gemm(x, nw, 1e-6, b=b, **f32)
        torch.cuda.synchronize()
        assert torch.equal(hf, h)
    else:
        q, qs = kernels.rms_norm_quant(x, nw, 1e-6, **f32)
        y0, y1 = pair.norm_gemm(x, nw, 1e-6, **f32)
    r0, r1 = pair.gemm(q, qs)
    torch.cuda.synchronize()
    assert torch.equal(y0, r0) and torch.equal(y1, r1)


@pytest.mark.parametrize("with_b", [False, True])
@pytest.mark.parametrize("M,N0,N1,K,wfp32", [(4, 1024, 512, 4096, False), (1, 1024, 512, 4096, True),
                                              (3, 32768, 8192, 1024, False), (4, 256, 128, 1024, True),
                                              (2, 256, 48, 2048, False), (4, 128, 64, 8192, False),
                                              (2, 128, 16, 8192, True)])
def test_fused_norm_pair_equals_unfused(gpu, with_b, M, N0, N1, K, wfp32):
    """PackedFp8Pair.norm_gemm (RMSNorm, with b the residual step first, quantised
    inside the projections' launch) gives the unfused ops' outputs bit for bit:
    add_rms_norm_quant / rms_norm_quant, then the pair's GEMV; the sum output equals
    the add's.  Rows include a zero row (the norm's eps floor), a row of tiny values
    and a row of large ones; M above norm_linear_rows(K) is refused."""
    from oracle.numerics import bf16_bits
    from wanferenz_amd import stage

    w0, s0 = stage.synthetic_linear(N0, K, N0 + K + 7, gpu, fp32_scales=wfp32)
    w1, s1 = stage.synthetic_linear(N1, K, N1 + K + 8, gpu, fp32_scales=wfp32)
    pair = kernels.PackedFp8Pair(w0, s0, w1, s1)
    xf = from_bf16_bits(_x(M * 3 + K, M, K)).reshape(M, K)
    if M >= 2:
        xf[0] = 0.0
        xf[1] *= np.float32(1e-30)
    if M >= 3:
        xf[2] *= np.float32(3e4)
    x = bf16_tensor(bf16_bits(xf), gpu).view(M, K)
    nw = torch.from_numpy(np.linspace(0.5, 1.5, K, dtype=np.float32)).to(gpu)
    b = bf16_tensor(_x(M * 5 + K + 1, M, K), gpu).view(M, K) if with_b else None
    if with_b:
        h, q, qs = kernels.add_rms_norm_quant(x, b, nw, 1e-6)
        hf, y0, y1 = pair.norm_gemm(x, nw, 1e-6, b=b)
        torch.cuda.synchronize()
        assert torch.equal(hf, h)
    else:
        q, qs = kernels.rms_norm_quant(x, nw, 1e-6)
        y0, y1 = pair.norm_gemm(x, nw, 1e-6)
    r0, r1 = pair.gemm(q, qs)
    torch.cuda.synchronize()
    assert torch.equal(y0, r0) and torch.equal(y1, r1)
    rows = kernels.norm_linear_rows(K)
    assert rows >= M
    with pytest.raises(Exception):
        big = bf16_tensor(_x(9, rows + 1, K), gpu).view(rows + 1, K)
        pair.norm_gemm(big, nw, 1e-6)


@pytest.mark.parametrize("act_fmt", ["ue8m0", None])
@pytest.mark.parametrize("G,N,K", [(6, 4096, 4096), (6, 4096, 2048), (1, 256, 1024), (40, 128, 512)])
def test_grouped_fp4_gemm(gpu, act_fmt, G, N, K):
    """grouped_fp4_gemm (fp4_grouped.py:96-128): row g against its own expert weight.
    Bit-equal to fp4_gemm of that row (the reference's CPU path computes it that way,
    fp4_grouped.py:112-121) and to the oracle's fp4_gemm within the bf16 bar."""
    xb = _x(G * 13 + N + K, G, K)
    sd = torch.float8_e8m0fnu if act_fmt else torch.float32
    q, s = kernels.act_quant(bf16_tensor(xb, gpu), 128, act_fmt, sd)
    ws_ = [_fp4_weight(N * 5 + K + g, N, K) for g in range(G)]
    w = np.stack([a for a, _ in ws_])
    wsc = np.stack([b for _, b in ws_])
    wt, wst = u8_tensor(w, gpu, torch.float4_e2m1fn_x2), u8_tensor(wsc, gpu, torch.float8_e8m0fnu)
    c = kernels.grouped_fp4_gemm(q, s, wt, wst, sd)
    got = f32_of_bf16(c)
    rows = torch.cat([kernels.fp4_gemm(q[g:g + 1].contiguous(), s[g:g + 1].contiguous(), wt[g], wst[g], sd)
                      for g in range(G)])
    assert np.array_equal(bits16(c), bits16(rows))
    rq, rs = om.act_quant(from_bf16_bits(xb), 128, act_fmt is not None)
    ref = np.concatenate([om.fp4_gemm(rq[g:g + 1], rs[g:g + 1], w[g], e8m0_decode(wsc[g])) for g in range(G)])
    rel, cos = _close(got, ref)
    assert rel <= TOL_REL and cos >= TOL_COS, (rel, cos)


def _nonfinite_rows(K):
    """bf16 rows whose 128-blocks hold NaN, +-inf, both, all-NaN, or ordinary values."""
    from oracle.numerics import bf16_bits

    base = np.linspace(-3.0, 3.0, K, dtype=np.float32)
    rows = []
    for spec in ([], [(5, np.nan)], [(0, np.inf)], [(K - 1, -np.inf)], [(3, np.nan), (9, np.inf)],
                 [(i, np.nan) for i in range(128)]):
        r = base.copy()
        for i, v in spec:
            r[i] = v
        rows.append(r)
    return bf16_bits(np.stack(rows))


def _same_codes(a, b):
    a, b = np.asarray(a, np.uint8), np.asarray(b, np.uint8)
    nan_a, nan_b = (a & 0x7F) == 0x7F, (b & 0x7F) == 0x7F
    return np.array_equal(nan_a, nan_b) and np.array_equal(a[~nan_a], b[~nan_b])


@pytest.mark.parametrize("scale_fmt,scale_dtype", [
    ("ue8m0", torch.float8_e8m0fnu), ("ue8m0", torch.float32), (None, torch.float32)])
def test_act_quant_non_finite_blocks(gpu, scale_fmt, scale_dtype):
    """NaN / inf in a block quantise as the reference's torch act_quant does
    (torch_ops.py:33-49): NaN survives the amax and the clamp, the fp32 scale
    is NaN or inf, the ue8m0 scale is 1; other blocks are untouched."""
    xb = _nonfinite_rows(512)
    q, s = kernels.act_quant(bf16_tensor(xb, gpu), 128, scale_fmt, scale_dtype)
    torch.cuda.synchronize()
    rq, rs = om.act_quant(from_bf16_bits(xb), 128, scale_fmt is not None)
    assert _same_codes(bytes8(q), rq)
    got_s = e8m0_decode(bytes8(s)) if scale_dtype == torch.float8_e8m0fnu else s.cpu().numpy()
    assert np.array_equal(got_s, rs, equal_nan=True)


def test_nan_in_x_gives_nan_rows_through_the_fused_linear(gpu):
    """A NaN activation makes its output row NaN on the packed GEMV (act_quant fused)
    and the other rows are unchanged."""
    from oracle.numerics import bf16_bits

    N, K, M = 256, 1024, 4
    w, ws = _fp8_weight(3, N, K, False)
    lin = kernels.PackedFp8Linear(u8_tensor(w, gpu, torch.float8_e4m3fn), u8_tensor(ws, gpu, torch.float8_e8m0fnu))
    xb = _x(77, M, K)
    y0 = lin(bf16_tensor(xb, gpu))
    xb2 = xb.copy()
    xb2[2, 700] = bf16_bits(np.float32(np.nan))
    y1 = lin(bf16_tensor(xb2, gpu))
    torch.cuda.synchronize()
    f1 = f32_of_bf16(y1)
    assert np.isnan(f1[2]).all()
    keep = [0, 1, 3]
    assert np.array_equal(bits16(y1)[keep], bits16(y0)[keep])


def test_wire_pack_non_finite_rows(gpu):
    """_pack_t (serving/chain.py:208-217) on NaN / inf rows: NaN rows give a NaN scale
    and NaN codes, an inf row the bf16-max scale, as torch computes them."""
    xb = _nonfinite_rows(1024)
    q, sc = kernels.wire_pack(bf16_tensor(xb, gpu))
    torch.cuda.synchronize()
    rq, rs = om.wire_pack(from_bf16_bits(xb))
    assert _same_codes(bytes8(q), rq)
    assert np.array_equal(f32_of_bf16(sc), rs, equal_nan=True)


# the M values the reference's invariance probe covers (fp8_vector.py:235-252),
# either side of each switch between kernels (16 | 17, 32 | 33), and a prefill width
INVARIANT_M = [1, 4, 8, 16, 17, 24, 32, 33, 64, 128]


@pytest.mark.parametrize("w_fp32", [False, True])
@pytest.mark.parametrize("act", ["ue8m0", "float"])
@pytest.mark.parametrize("N,K", PROJ_SHAPES)
def test_fp8_linear_batch_invariant(gpu, w_fp32, act, N, K):
    """A row's output does not depend on how many rows share the call: the packed
    linear at M = 1 .. 128 (one-tile GEMV, ring GEMV and tile GEMM, whichever serves
    each M) gives every row the bits it has at M = 128, torch.equal as the reference
    requires before it enables its decode GEMV (fp8_vector.py:235-252).  Both weight
    scale kinds, power-of-two and float activation scales, bf16 input (act_quant
    fused) and pre-quantised input (fp8_gemm on the packed weight)."""
    from wanferenz_amd import stage

    w, ws = stage.synthetic_linear(N, K, N + 5 * K, gpu, fp32_scales=w_fp32)
    lin = kernels.PackedFp8Linear(w, ws, "ue8m0" if act == "ue8m0" else None)
    Mmax = max(INVARIANT_M)
    x = bf16_tensor(_x(N + K + 3, Mmax, K), gpu).view(Mmax, K)
    ref = lin(x)
    sdt = torch.float8_e8m0fnu if act == "ue8m0" else torch.float32
    q, qs = kernels.act_quant(x, 128, "ue8m0" if act == "ue8m0" else None, sdt)
    ref_q = lin.gemm(q, qs)
    torch.cuda.synchronize()
    assert torch.equal(ref, ref_q)
    for M in INVARIANT_M[:-1]:
        y = lin(x[:M].contiguous())
        yq = lin.gemm(q[:M].contiguous(), qs[:M].contiguous())
        torch.cuda.synchronize()
        assert torch.equal(y, ref[:M]), f"M={M}: bf16 input differs from M={Mmax}"
        assert torch.equal(yq, ref[:M]), f"M={M}: pre-quantised input differs from M={Mmax}"
