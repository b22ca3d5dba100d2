"""CPU checks of the drop-in protocol (no GPU calls).

install() follows the reference's protocol (fp4_grouped.install,
wanferenz/kernels/fp4_grouped.py:339-351; fp8_vector.install :476-491): the
previous function is kept, the new one carries a marker attribute, a second
install is a no-op, and a layer the HIP path cannot serve declines to the
kept forward with a tally by reason (fp4_grouped.py:256-262).
"""

import types

import pytest
import torch

from tests import mirror_model as mm
from wanferenz_amd import kernels
from wanferenz_amd import moe as wm


@pytest.fixture
def mod():
    """A fresh copy of the mirror module, so class-level patches do not leak."""
    m = types.ModuleType("mirror_copy")
    for k, v in vars(mm).items():
        if not k.startswith("__"):
            setattr(m, k, v)

    class MoE(mm.MoE):
        forward = mm.MoE.forward

    m.MoE = MoE
    yield m
    wm.uninstall(m)


def test_moe_install_is_idempotent_and_reversible(mod):
    ref = mod.MoE.forward
    assert wm.moe_chain(mod) == "ref"
    assert wm.install(mod) is True
    assert getattr(mod.MoE.forward, "_v4_hip_moe", False)
    assert wm.install(mod) is False  # marker seen: no double wrap
    assert wm._REF_FORWARD is ref
    assert wm.moe_chain(mod) == "hip>ref"
    assert wm.uninstall(mod) is True
    assert mod.MoE.forward is ref and wm.moe_chain(mod) == "ref"
    assert wm.uninstall(mod) is False


@pytest.mark.parametrize("why", ["world_size>1", "partial-experts", "not-mxfp4-bank"])
def test_unservable_layers_decline_to_the_kept_forward(mod, why):
    moe = mm.MoE(0, 256, 128, 8, 2, expert_dtype=torch.float4_e2m1fn_x2)
    if why == "world_size>1":
        mod.world_size = 2
    elif why == "partial-experts":
        moe.experts_end_idx = 4
    else:
        moe = mm.MoE(0, 256, 128, 8, 2, expert_dtype=torch.bfloat16)
    wm.install(mod)
    x = torch.zeros(3, 256, dtype=torch.bfloat16)
    y = mod.MoE.forward(moe, x, torch.zeros(3, dtype=torch.int64))
    assert moe.ref_calls == 1 and bool((y == mm.SENTINEL).all())
    assert moe._hip_declined == {why: 1}
    assert wm.coverage(moe) == {0: (0, {why: 1})}


def test_kernel_install_rebinds_module_globals():
    m = types.ModuleType("kernels_host")
    orig = {n: (lambda *a, **k: None) for n in ("act_quant", "fp8_gemm", "fp4_gemm", "sparse_attn")}
    for n, f in orig.items():
        setattr(m, n, f)
    assert kernels.install(m) is True
    assert m.act_quant is kernels.act_quant and m.fp8_gemm is kernels.fp8_gemm and m.fp4_gemm is kernels.fp4_gemm
    assert m.sparse_attn is kernels.sparse_attn
    assert kernels.install(m) is False
    assert kernels.uninstall(m) is True
    assert all(getattr(m, n) is f for n, f in orig.items())


def test_kernels_refuse_cpu_tensors():
    """The product has no CPU path: a CPU tensor is an error, not a fallback."""
    x = torch.zeros(2, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU only"):
        kernels.act_quant(x, 128, "ue8m0", torch.float8_e8m0fnu)
    a = torch.zeros(2, 128, dtype=torch.uint8).view(torch.float8_e4m3fn)
    s = torch.zeros(2, 1, dtype=torch.float32)
    with pytest.raises(RuntimeError, match="GPU only"):
        kernels.fp8_gemm(a, s, a, torch.ones(1, 1))
