"""The converted-checkpoint loader (wanferenz_amd/loader.py) on CPU: names, dtypes,
shapes and the bank bytes, against a golden case written in the converter's format."""

import numpy as np
import pytest
import torch

from tests.ckpt_writer import write_case_checkpoint
from tests.golden.cases import CASES, make_inputs
from wanferenz_amd import _native as N
from wanferenz_amd import loader


@pytest.mark.parametrize("name", ["toy_t4", "hash_t3", "toy_t4_fp32scale"])
def test_bank_bytes_match_the_case(tmp_path, name):
    case = CASES[name]
    inp = make_inputs(case)
    path = write_case_checkpoint(case, inp, str(tmp_path / name), layer=3)
    cfg, w = loader.load_moe_layer(path, 3, device="cpu")
    assert (cfg.dim, cfg.inter, cfg.n_experts, cfg.topk) == (case.dim, case.inter, case.n_experts, case.topk)
    assert cfg.score_func == case.score_func and cfg.route_scale == case.route_scale
    assert cfg.swiglu_limit == case.swiglu_limit
    assert cfg.act_scale_kind == (N.WZ_SCALE_UE8M0 if case.round_pow2 else N.WZ_SCALE_F32)
    assert np.array_equal(w.w13.numpy(), inp.w13) and np.array_equal(w.w13_s.numpy(), inp.w13_s)
    assert np.array_equal(w.w2.numpy(), inp.w2) and np.array_equal(w.w2_s.numpy(), inp.w2_s)
    I, nb = case.inter, case.inter // 128
    assert np.array_equal(w.sh_w1.numpy(), inp.sh_w13[:I]) and np.array_equal(w.sh_w3.numpy(), inp.sh_w13[I:])
    assert np.array_equal(w.sh_w1_s.numpy(), inp.sh_w13_s[:nb]) and np.array_equal(w.sh_w2_s.numpy(), inp.sh_w2_s)
    assert np.array_equal(w.gate_w.view(torch.int16).numpy().view(np.uint16), inp.gate_w)
    if case.hash_layer:
        assert w.gate_bias is None and np.array_equal(w.tid2eid.numpy(), inp.tid2eid)
    else:
        assert w.tid2eid is None and np.array_equal(w.gate_bias.numpy(), inp.gate_bias)


def test_missing_and_malformed_tensors(tmp_path):
    case = CASES["toy_t4"]
    inp = make_inputs(case)
    path = write_case_checkpoint(case, inp, str(tmp_path / "ck"), layer=0, split_files=False)
    with pytest.raises(loader.CheckpointError, match="layers.5.ffn.gate.weight"):
        loader.load_moe_layer(path, 5, device="cpu")
    with pytest.raises(loader.CheckpointError, match="model"):
        loader.load_moe_layer(str(tmp_path / "empty"), 0, device="cpu")
    # an fp8 expert bank (converter expert_dtype "fp8") is not the MXFP4 bank
    from safetensors.torch import load_file, save_file

    f = str(tmp_path / "ck" / "model00000-mp1.safetensors")
    st = load_file(f)
    st["layers.0.ffn.experts.0.w1.weight"] = torch.zeros(case.inter, case.dim, dtype=torch.float8_e4m3fn)
    save_file(st, f)
    with pytest.raises(loader.CheckpointError, match="MXFP4"):
        loader.load_moe_layer(path, 0, device="cpu")


def _pattern(name: str, layer: int) -> str:
    import re

    return re.sub(r"experts\.\d+\.", "experts.<e>.", name.replace(f"layers.{layer}.", "layers.<L>."))


@pytest.mark.parametrize("label,name", [("routed", "toy_t4"), ("hash", "hash_t3")])
def test_names_are_the_reference_converters(tmp_path, monkeypatch, label, name):
    """The tensor names the loader reads for one block are the reference's: the names
    of its own MoE module's state_dict under layers.<L>.ffn., which its converter's
    _rename produces from the Hugging Face names (tests/golden/ckpt_names.json,
    written by tests/golden/make_names.py from the reference).  Checked as patterns
    (expert index and layer abstracted): the names read == the fixture's, and the
    fixture's HF names carry the renames conversion.py:15-29 undoes."""
    import json
    import os

    fx = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "ckpt_names.json")))["layers"][label]
    want = {_pattern(n, fx["layer"]) for n in fx["names"]}
    for conv, hf in fx["names"].items():
        assert hf.startswith("model.") and ".mlp." in hf and ".ffn." in conv
        assert conv.endswith(".scale") == hf.endswith(".weight_scale_inv")
        assert conv.endswith("gate.bias") == hf.endswith("gate.e_score_correction_bias")
    case = CASES[name]
    inp = make_inputs(case)
    layer = 3
    path = write_case_checkpoint(case, inp, str(tmp_path / name), layer=layer)
    read = set()
    orig = loader.Checkpoint.get

    def get(self, n):
        read.add(n)
        return orig(self, n)

    monkeypatch.setattr(loader.Checkpoint, "get", get)
    loader.load_moe_layer(path, layer, device="cpu")
    got = {_pattern(n, layer) for n in read}
    assert got == want, (sorted(got ^ want))
    # every expert's names are read, and nothing outside this block's ffn
    assert all(n.startswith(f"layers.{layer}.ffn.") for n in read)
    assert len(read) == len(want) - 6 + 6 * case.n_experts
