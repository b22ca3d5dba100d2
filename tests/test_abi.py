"""CPU checks of the C-ABI library (no GPU calls).

The shared library must load on a host without a GPU, export every entry
point include/wanferenz_amd.h declares, size its workspace and packed banks
as documented, and reject bad arguments with an error code and message before
it touches the device (argument checks never reach a launch).
"""

import ctypes
import math
import os
import re

import pytest

from wanferenz_amd import _native as N
from wanferenz_amd.moe import WzMoeDesc

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "wanferenz_amd.h")


def header_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(wz_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_header_symbol():
    syms = header_symbols()
    assert len(syms) >= 18, syms
    L = N.lib()
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, f"declared in the header but not exported: {missing}"
    # the Python binding covers the same set
    assert sorted(N.SIGNATURES) == syms


def _desc(D=4096, I=2048, E=256, k=6):
    d = WzMoeDesc()
    d.dim, d.inter, d.n_experts, d.topk = D, I, E, k
    d.score_func = N.WZ_SCORE_SQRTSOFTPLUS
    d.act_scale_kind = N.WZ_SCALE_UE8M0
    d.shared_w_scale_kind = N.WZ_WSCALE_E8M0
    d.route_scale, d.swiglu_limit = 1.5, 10.0
    d.gate_w = 0x1000  # never dereferenced by the host-side checks below
    return d


def test_workspace_serves_every_smaller_call():
    L = N.lib()
    for D, I, E, k in ((4096, 2048, 256, 6), (1024, 512, 16, 2), (512, 256, 32, 6)):
        d = _desc(D, I, E, k)
        sizes = [L.wz_moe_workspace_bytes(ctypes.byref(d), T) for T in range(0, 300)]
        # wz_moe_workspace_bytes(T) covers every call with 1..T tokens
        for T in range(1, 300):
            assert sizes[T] >= max(sizes[1:T + 1]), (D, T)
        assert all(s % 256 == 0 for s in sizes)


def test_packed_bank_sizes():
    L = N.lib()
    D, I, E = 4096, 2048, 256
    d = _desc(D, I, E)
    got = [L.wz_moe_packed_bytes(ctypes.byref(d), i) for i in range(6)]
    KG13, KG2 = math.ceil(D / 512), math.ceil(I / 512)
    want = [E * I * D,                      # w13p: E x 2I x D e2m1 = E*I*D bytes
            E * (I // 16) * KG13 * 2 * 256,  # w13p_s: dword of 4 e8m0 per lane
            E * D * I // 2,                  # w2p
            E * (D // 16) * KG2 * 256,       # w2p_s
            2 * I * D,                       # sh13p (e4m3 w1 | w3)
            D * I]                           # sh2p
    assert got == want
    # the packed routed bank holds the same bytes as the reference-layout bank (no padding)
    assert got[0] + got[2] == E * (2 * I * D // 2 + D * I // 2)


def _err():
    return N.lib().wz_last_error().decode()


def test_argument_errors_are_reported_without_a_device():
    L = N.lib()
    assert L.wz_act_quant_fp8(None, 4, 100, None, None, 1, None) == -1
    assert "multiple of 128" in _err()
    assert L.wz_act_quant_fp8(None, 4, 128, None, None, 7, None) == -1
    assert "scale kind" in _err()
    assert L.wz_fp4_gemm(None, None, None, None, None, 1, 100, 128, 1, None) != 0
    d = _desc()
    d.dim = 100
    assert L.wz_moe_forward(ctypes.byref(d), None, None, 4, None, None, None, None, 0, None) == -1
    assert "multiples of 128" in _err()
    d = _desc(k=300)
    assert L.wz_moe_forward(ctypes.byref(d), None, None, 4, None, None, None, None, 0, None) == -1
    assert "topk" in _err()
    d = _desc()
    need = L.wz_moe_workspace_bytes(ctypes.byref(d), 4)
    buf = ctypes.create_string_buffer(64)
    assert L.wz_moe_forward(ctypes.byref(d), None, None, 4, None, None, None, buf, 64, None) == -3
    assert str(need) in _err() or "workspace" in _err()
    d = _desc()
    d.n_experts = 100000
    assert L.wz_moe_route(ctypes.byref(d), None, None, 4, None, None, None, None, None, None, 0, None) == -1
    assert "n_experts" in _err()


def test_fused_norm_linear_limits_and_errors():
    L = N.lib()
    assert [L.wz_fp8_norm_linear_max_rows(k) for k in (1024, 2048, 4096, 8192, 1536)] == [4, 2, 4, 4, 0]
    f = L.wz_fp8_norm_linear_packed_pair
    # K outside the GEMV set
    assert f(None, None, None, ctypes.c_float(1e-6), None, None, None, None, 256, None, 1, 256, 1536, 1, 1, None) == -1
    assert "K=1536" in _err()
    # a split that is not a multiple of 128, and a sum without the addend
    assert f(None, None, None, ctypes.c_float(1e-6), None, None, None, None, 48, ctypes.c_void_p(16), 1, 256, 1024,
             1, 1, None) == -1
    assert "split" in _err()
    assert f(None, None, None, ctypes.c_float(1e-6), ctypes.c_void_p(16), None, None, None, 256, None, 1, 256, 1024,
             1, 1, None) == -1
    assert "addend" in _err()
    # zero rows: nothing to do
    assert f(None, None, None, ctypes.c_float(1e-6), None, None, None, None, 256, None, 0, 256, 1024, 1, 1, None) == 0


def test_zero_tokens_is_a_no_op():
    L = N.lib()
    d = _desc()
    assert L.wz_act_quant_fp8(None, 0, 128, None, None, 1, None) == 0
    assert L.wz_moe_forward(ctypes.byref(d), None, None, 0, None, None, None, None, 0, None) == 0


def test_last_error_is_per_thread():
    import threading

    L = N.lib()
    L.wz_act_quant_fp8(None, 4, 100, None, None, 1, None)
    mine = _err()
    seen = []

    def other():
        L.wz_act_quant_fp8(None, 4, 128, None, None, 9, None)
        seen.append(_err())

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert "scale kind" in seen[0] and _err() == mine


def test_sparse_attn_workspace_and_argument_errors():
    """wz_sparse_attn sizes its split partials on the host and rejects bad
    arguments before any launch (the pointers below are never dereferenced)."""
    L = N.lib()
    # decode (one query, 64 heads of 512, 640 indices): 10 blocks, one workgroup each,
    # partial = m[64] + l[64] + O[64][512] floats
    assert L.wz_sparse_attn_workspace_bytes(1, 1, 64, 512, 640) == 10 * (128 + 64 * 512) * 4
    assert L.wz_sparse_attn_workspace_bytes(1, 512, 64, 512, 640) == 0  # enough queries: no split
    assert L.wz_sparse_attn_workspace_bytes(1, 1, 48, 512, 640) == 10 * (128 + 64 * 512) * 4  # 48 heads: one group
    q, kv, sink, idx, o = 16, 32, 48, 64, 80  # aligned stand-ins

    def call(B=1, S=1, H=64, D=512, Nn=100, topk=640, ws=None, wsb=0, qq=q):
        return L.wz_sparse_attn(qq, kv, sink, idx, o, B, S, H, D, Nn, topk, 0.1, ws, wsb, None)

    assert call(H=40) == -1 and "multiple of 16" in _err()
    assert call(D=96) == -1 and "head dim" in _err()
    assert call(qq=17) == -1 and "16-byte aligned" in _err()
    assert call(ws=96, wsb=64) == -1 and "workspace of 64 bytes" in _err()
    assert call(topk=4096) == -1 and "needs a workspace" in _err()
    assert call(Nn=1 << 22) == -1 and "2 GiB" in _err()
    assert call(B=0) == 0 and call(S=0) == 0  # no queries: nothing to do
