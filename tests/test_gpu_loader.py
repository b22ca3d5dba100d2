"""GPU: a converted checkpoint loaded by wanferenz_amd.loader straight into the bank
and packed layer reproduces the reference's golden vectors for the case it holds."""

import numpy as np
import pytest
import torch

from oracle import moe as om
from oracle.numerics import from_bf16_bits
from tests.ckpt_writer import write_case_checkpoint
from tests.golden.cases import CASES, make_inputs
from tests.helpers import bf16_tensor, f32_of_bf16
from wanferenz_amd import loader

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["toy_t4", "hash_t3", "top6_t8"])
def test_loaded_layer_matches_golden(gpu, tmp_path, name):
    case = CASES[name]
    inp = make_inputs(case)
    path = write_case_checkpoint(case, inp, str(tmp_path / name), layer=2)
    moe = loader.hip_moe_layer(path, 2, device=gpu, max_tokens=case.T)
    ids = torch.from_numpy(inp.input_ids).to(gpu)
    y = moe.forward(bf16_tensor(inp.x, gpu), ids)
    torch.cuda.synchronize()
    got = f32_of_bf16(y)
    gold = from_bf16_bits(np.load(f"tests/golden/{name}.npz")["y_bf16"])
    rel, cos = om.max_rel_err(got, gold), om.cosine(got, gold)
    assert rel <= 1e-2 and cos >= 0.9999, (rel, cos)
