"""wz_moe_forward_noalloc (the MoE layer on the library's own scratch array,
for callers that cannot allocate) against wz_moe_forward with a workspace,
both called through the C ABI.

Both run the same kernels on the same inputs, so outputs and routing must be
bit-identical.  Each case makes two calls in a row, the second with fewer
tokens, so the second call runs on scratch holding the first call's contents.
"""

import ctypes

import numpy as np
import pytest
import torch

from tests.golden.cases import CASES, make_inputs
from tests.helpers import bf16_tensor
from wanferenz_amd import _native as N
from wanferenz_amd import synth
from wanferenz_amd.moe import HipMoE, MoEConfig

pytestmark = pytest.mark.gpu


def _outs(moe, T):
    D, k, dev = moe.cfg.dim, moe.cfg.topk, moe.device
    return (torch.full((T, D), 7.0, dtype=torch.bfloat16, device=dev),
            torch.full((T, k), -1.0, dtype=torch.float32, device=dev),
            torch.full((T, k), -1, dtype=torch.int64, device=dev))


def _noalloc(moe, x, ids=None):
    T = x.size(0)
    y, w, i = _outs(moe, T)
    rc = N.lib().wz_moe_forward_noalloc(ctypes.byref(moe.desc), x.data_ptr(), None if ids is None else ids.data_ptr(),
                                        T, y.data_ptr(), w.data_ptr(), i.data_ptr(), N.stream_handle(moe.device))
    N.check(rc, "wz_moe_forward_noalloc")
    return y, w, i


def _with_workspace(moe, x, ids=None):
    T = x.size(0)
    y, w, i = _outs(moe, T)
    ws = torch.empty(max(int(N.lib().wz_moe_workspace_bytes(ctypes.byref(moe.desc), T)), 256), dtype=torch.uint8,
                     device=moe.device)
    N.call("wz_moe_workspace_init", ws.data_ptr(), ws.numel(), N.stream_handle(moe.device))
    N.call("wz_moe_forward", ctypes.byref(moe.desc), x.data_ptr(), None if ids is None else ids.data_ptr(), T,
           y.data_ptr(), w.data_ptr(), i.data_ptr(), ws.data_ptr(), ws.numel(), N.stream_handle(moe.device))
    return y, w, i


def _same(a, b):
    torch.cuda.synchronize()
    for u, v in zip(a, b):
        assert torch.equal(u, v)


def _case_layer(name, T, gpu):
    from tests.test_gpu_moe import upload_case
    import dataclasses

    case = dataclasses.replace(CASES[name], T=T)
    inp = make_inputs(case)
    moe = upload_case(case, inp, gpu)
    ids = torch.from_numpy(inp.input_ids).to(gpu) if case.hash_layer else None
    return moe, bf16_tensor(inp.x, gpu), ids


@pytest.mark.parametrize("name,T1,T2", [("toy_t4", 40, 5), ("top6_t8", 12, 3), ("hash_t3", 24, 3),
                                        ("toy_t4", 1300, 17)])
def test_noalloc_equals_forward_on_two_calls(gpu, name, T1, T2):
    moe, x, ids = _case_layer(name, T1, gpu)
    _same(_noalloc(moe, x, ids), _with_workspace(moe, x, ids))
    x2, ids2 = x[:T2].contiguous(), None if ids is None else ids[:T2].contiguous()
    _same(_noalloc(moe, x2, ids2), _with_workspace(moe, x2, ids2))


def test_noalloc_v4_decode_and_the_size_limit(gpu):
    """The V4 decode layer (T = 8, then 2) on the scratch; T = 157 needs more than
    the 16 MiB the library holds and is refused with an error before any launch."""
    cfg = MoEConfig(4096, 2048, 256, 6, "sqrtsoftplus", 1.5, 10.0, N.WZ_SCALE_UE8M0, N.WZ_WSCALE_E8M0)
    w, _ = synth.synthetic_moe(cfg, seed=3, layer=0, device=gpu)
    moe = HipMoE(cfg, w, max_tokens=8, keep_reference=False)
    del w
    for T in (8, 2):
        x = bf16_tensor(synth.normal_bf16(synth.stream_key(60 + T, synth.S_X), (T, 4096), 1.0), gpu)
        _same(_noalloc(moe, x), _with_workspace(moe, x))
    big = torch.zeros(157, 4096, dtype=torch.bfloat16, device=gpu)
    y = torch.zeros_like(big)
    rc = N.lib().wz_moe_forward_noalloc(ctypes.byref(moe.desc), big.data_ptr(), None, 157, y.data_ptr(), None,
                                        None, N.stream_handle(gpu))
    assert rc == -3 and b"16777216" in N.lib().wz_last_error()
    torch.cuda.synchronize()
    assert not y.any()
    x = bf16_tensor(synth.normal_bf16(synth.stream_key(99, synth.S_X), (156, 4096), 1.0), gpu)
    _same(_noalloc(moe, x), _with_workspace(moe, x))
