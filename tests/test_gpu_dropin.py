"""GPU parity through the drop-in boundary: MoE.forward replaced by install().

A mirror of the reference's MoE module (tests/mirror_model.py: same
attributes, dtypes and shapes as wanferenz/model/architecture.py:674-794)
holds a golden case's weights on the GPU.  After install(), MoE.forward runs
the HIP layer: the per-expert parameters become views into one bank (the
relayout of fp4_grouped._relayout_moe, fp4_grouped.py:142-188), and the
output must match the reference's own golden vectors to the bf16 tolerance.
"""

import types

import numpy as np
import pytest
import torch

from oracle import moe as om
from oracle.numerics import from_bf16_bits
from tests import mirror_model as mm
from tests.golden.cases import CASES, make_inputs
from tests.helpers import bf16_tensor, f32_of_bf16
from wanferenz_amd import moe as wm

pytestmark = pytest.mark.gpu


@pytest.fixture
def mod():
    m = types.ModuleType("mirror_gpu")
    for k, v in vars(mm).items():
        if not k.startswith("__"):
            setattr(m, k, v)

    class MoE(mm.MoE):
        forward = mm.MoE.forward

    m.MoE = MoE
    yield m
    wm.uninstall(m)


@pytest.mark.parametrize("name", ["toy_t4", "toy_t37", "hash_t3", "top6_t8"])
def test_installed_moe_forward_matches_golden(gpu, mod, name):
    case = CASES[name]
    inp = make_inputs(case)
    moe = mm.moe_from_case(case, inp, gpu)
    wm.install(mod)
    x = bf16_tensor(inp.x, gpu).view(1, case.T, case.dim)
    ids = torch.from_numpy(inp.input_ids).to(gpu).view(1, case.T)
    y = mod.MoE.forward(moe, x, ids)
    torch.cuda.synchronize()
    assert moe.ref_calls == 0 and moe._hip_steps == 1 and not getattr(moe, "_hip_declined", {})
    assert y.shape == x.shape and y.dtype == torch.bfloat16
    got = f32_of_bf16(y.view(case.T, case.dim))
    gold = from_bf16_bits(np.load(f"tests/golden/{name}.npz")["y_bf16"])
    rel, cos = om.max_rel_err(got, gold), om.cosine(got, gold)
    assert rel <= 1e-2 and cos >= 0.9999, (rel, cos)
    # the experts' parameters now live in the bank (views, no second copy)
    bank = moe._grouped_bank
    w1 = moe.experts[3].w1.weight
    assert w1.untyped_storage().data_ptr() == bank["w13"].untyped_storage().data_ptr()
    # a second call reuses the cached layer
    y2 = mod.MoE.forward(moe, x, ids)
    assert torch.equal(y, y2) and moe._hip_steps == 2
