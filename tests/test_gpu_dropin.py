"""GPU parity through the drop-in boundary: MoE.forward and the FP8 linears
replaced by install().

A mirror of the reference's MoE module (tests/mirror_model.py: same
attributes, dtypes and shapes as wanferenz/model/architecture.py:674-794)
holds a golden case's weights on the GPU.  After install(), MoE.forward runs
the HIP layer: each expert's parameters are packed straight into the packed
banks and then released (one copy in HBM, the reference's bank layout with
preserve=False, serving/partition.py:398-405), and the output must match the
reference's own golden vectors to the bf16 tolerance.  The FP8 linears go
through the packed GEMV once kernels.install() has rebound linear / fp8_gemm
(the reference's fp8_vector.install, fp8_vector.py:472-491), at the real V4
projection shapes (fp8_vector.py:505-513).
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
from oracle.numerics import e8m0_decode
from tests.golden.cases import oracle_params
from wanferenz_amd import kernels, synth
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
@pytest.mark.parametrize("release", [True, False])
def test_installed_moe_forward_matches_golden(gpu, mod, name, release, monkeypatch):
    monkeypatch.setattr(wm, "RELEASE_EXPERTS", release)
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
    h = moe._hip_moe
    assert h.weights is None  # the layer keeps only the packed banks
    w1 = moe.experts[3].w1.weight
    if release:
        # one copy of the experts: the module's expert weights are emptied
        assert w1.numel() == 0 and moe.experts[0].w2.scale.numel() == 0
        assert moe.shared_experts.w1.weight.numel() == 0 and moe.shared_experts.w1.scale.numel() > 0
    else:
        assert w1.numel() == case.inter * case.dim // 2
    # a second call reuses the cached layer
    y2 = mod.MoE.forward(moe, x, ids)
    assert torch.equal(y, y2) and moe._hip_steps == 2


def test_prepare_packs_at_load_and_the_step_captures(gpu, mod):
    """prepare() packs the model's MoE layers at load (the reference's load-time bank,
    partition.py:398-405); a decode step through the installed MoE.forward then
    captures in a graph whose replays equal the eager step."""
    case = CASES["top6_t8"]
    inp = make_inputs(case)
    moe = mm.moe_from_case(case, inp, gpu)
    model = torch.nn.ModuleList([moe])
    wm.install(mod)
    assert wm.prepare(model, mod, max_tokens=case.T) == 1
    assert moe._hip_moe is not None and moe.experts[0].w1.weight.numel() == 0
    x = bf16_tensor(inp.x, gpu).view(1, case.T, case.dim)
    ids = torch.from_numpy(inp.input_ids).to(gpu).view(1, case.T)
    eager = mod.MoE.forward(moe, x, ids).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            mod.MoE.forward(moe, x, ids)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = mod.MoE.forward(moe, x, ids)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        mod.MoE.forward(moe, x, ids)  # eager work between replays


def test_installed_moe_serves_any_prompt_length(gpu, mod):
    """MoE.forward takes any T (architecture.py:777-794).  At top-2, T = 8193 is
    one token past a single call's 16384 routed pairs: the layer runs it as a
    chunk of 8192 tokens and one of 1.  Rows are checked against the oracle
    (sampled), against the same tokens in shorter calls (the layer is
    token-local, and both calls of a row run the same kernels, so bit-equal),
    and the lone last token against a one-token call."""
    import dataclasses

    case = dataclasses.replace(CASES["toy_t4"], name="toy_t8193", T=8193)
    inp = make_inputs(case)
    moe = mm.moe_from_case(case, inp, gpu)
    wm.install(mod)
    x = bf16_tensor(inp.x, gpu)
    ids = torch.from_numpy(inp.input_ids).to(gpu)
    y = mod.MoE.forward(moe, x.view(1, -1, case.dim), ids.view(1, -1)).view(case.T, case.dim)
    h = moe._hip_moe
    part = torch.cat([h.forward(x[:3000]), h.forward(x[3000:8192])])
    last = h.forward(x[8192:])
    torch.cuda.synchronize()
    assert torch.equal(y[:8192], part)
    assert torch.equal(y[8192:], last)
    rows = [0, 1, 4095, 8191, 8192]
    p = oracle_params(case, inp)
    ref = om.moe_forward(p, from_bf16_bits(inp.x[rows]), inp.input_ids[rows])
    got = f32_of_bf16(y[rows])
    rel, cos = om.max_rel_err(got, ref.y), om.cosine(got, ref.y)
    assert rel <= 1e-2 and cos >= 0.9999, (rel, cos)


def test_hash_ids_outside_the_table(gpu):
    """tid2eid[input_ids] raises for an id outside the table (architecture.py:710-711).
    Host ids are checked before launch (IndexError); device ids are not read back:
    that token's row comes out NaN, the other tokens' rows are unchanged."""
    case = CASES["hash_t3"]
    inp = make_inputs(case)
    from tests.test_gpu_moe import upload_case

    moe = upload_case(case, inp, gpu)
    x = bf16_tensor(inp.x, gpu)
    good = moe.forward(x, torch.from_numpy(inp.input_ids).to(gpu))
    bad = inp.input_ids.copy()
    bad[1] = case.vocab + 5
    with pytest.raises(IndexError):
        moe.forward(x, torch.from_numpy(bad))
    for T, xs in ((case.T, x), (40, x.repeat(14, 1)[:40])):
        ids = np.resize(bad, T)
        y = moe.forward(xs, torch.from_numpy(ids).to(gpu))
        ref = moe.forward(xs, torch.from_numpy(np.resize(inp.input_ids, T)).to(gpu))
        torch.cuda.synchronize()
        hit = ids >= case.vocab
        yf = y.float().cpu().numpy()
        assert np.isnan(yf[hit]).all()
        assert torch.equal(y[torch.from_numpy(~hit).to(gpu)], ref[torch.from_numpy(~hit).to(gpu)])
    assert torch.equal(moe.forward(x, torch.from_numpy(inp.input_ids).to(gpu)), good)


# ------------------------------------------------------------- FP8 linears ---

# The decode projections the reference's GEMV serves (fp8_vector.py:505-513), N x K.
V4_PROJECTIONS = {"attn.wq_a": (1024, 4096), "attn.wkv": (512, 4096), "attn.wq_b": (32768, 1024),
                  "attn.wo_b": (4096, 8192), "idx.wq_b": (8192, 1024), "shared.w13": (4096, 4096),
                  "shared.w2": (4096, 2048)}


@pytest.fixture
def lin_mod():
    """A model module exposing the linear-path globals (architecture.py:12-19, 121-134)."""
    m = types.ModuleType("mirror_linear")
    m.block_size, m.scale_fmt, m.scale_dtype = 128, "ue8m0", torch.float8_e8m0fnu

    def unused(*a, **k):
        raise AssertionError("the replaced binding was called")

    m.act_quant = m.fp8_gemm = m.fp4_gemm = m.linear = unused
    kernels.install(m)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    yield m
    torch.set_default_dtype(prev)
    kernels.uninstall(m)


def _fp8_param(N, K, gpu, seed):
    w = torch.empty(N, K, dtype=torch.uint8, device=gpu)
    synth.device_fill(w, synth.stream_key(seed, synth.S_FP8_W), synth.FILL_E4M3)
    s = torch.empty((N + 127) // 128, (K + 127) // 128, dtype=torch.uint8, device=gpu)
    synth.device_fill(s, synth.stream_key(seed, synth.S_FP8_W_S), synth.FILL_E8M0, 112, 116)
    p = torch.nn.Parameter(w.view(torch.float8_e4m3fn), requires_grad=False)
    p.scale = torch.nn.Parameter(s.view(torch.float8_e8m0fnu), requires_grad=False)
    return p


@pytest.mark.parametrize("name", list(V4_PROJECTIONS))
@pytest.mark.parametrize("M", [1, 4, 17, 32, 40])
def test_installed_linear_runs_the_packed_path(gpu, lin_mod, name, M):
    """linear(x, W) and act_quant + fp8_gemm through the installed bindings, on a
    weight Parameter: both run on the packed copy made at first use, agree bit
    for bit (same codes, same product), and match the oracle on three 128-row
    blocks of the output."""
    N, K = V4_PROJECTIONS[name]
    w = _fp8_param(N, K, gpu, N + 3 * K)
    nb = N // 128
    blocks = sorted({0, nb // 2, nb - 1})
    rows = np.concatenate([np.arange(b * 128, b * 128 + 128) for b in blocks])
    # the row-major bytes, read before the first call packs the weight in place
    wsub = w.detach().view(torch.uint8)[torch.from_numpy(rows).to(gpu)].cpu().numpy()
    ssub = e8m0_decode(w.scale.detach().view(torch.uint8)[blocks].cpu().numpy())
    xb = synth.normal_bf16(synth.stream_key(M + N, synth.S_FP8_X), (M, K), 1.0)
    x = bf16_tensor(xb, gpu)
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated(gpu)
    y = lin_mod.linear(x, w)
    torch.cuda.synchronize()
    # one copy of the projection: the tiles sit in the Parameter's own storage
    assert kernels.is_packed(w) and tuple(w.shape) == (N, K) and w.dtype == torch.float8_e4m3fn
    assert w.untyped_storage().nbytes() == N * K
    assert torch.cuda.memory_allocated(gpu) - before < N * K // 2
    q, s = lin_mod.act_quant(x, 128, lin_mod.scale_fmt, lin_mod.scale_dtype)
    y2 = lin_mod.fp8_gemm(q, s, w, w.scale, lin_mod.scale_dtype)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    rq, rs = om.act_quant(from_bf16_bits(xb), 128, True)
    ref = om.fp8_gemm(rq, rs, wsub, ssub)
    got = f32_of_bf16(y)[:, rows]
    rel, cos = om.max_rel_err(got, ref), om.cosine(got, ref)
    assert rel <= 1e-2 and cos >= 0.9999, (rel, cos)


def test_packed_copy_follows_the_weight(gpu, lin_mod):
    """Writing the weight in place (a checkpoint load after install) makes the next
    call repack; a graph captured after a first call runs the packed GEMV."""
    N, K = 1024, 4096
    w = _fp8_param(N, K, gpu, 11)
    x = bf16_tensor(synth.normal_bf16(synth.stream_key(5, synth.S_FP8_X), (2, K), 1.0), gpu)
    y0 = lin_mod.linear(x, w)
    w2 = _fp8_param(N, K, gpu, 12)
    with torch.no_grad():
        w.copy_(w2)
        w.scale.copy_(w2.scale)
    y1 = lin_mod.linear(x, w)
    y_ref = lin_mod.linear(x, w2)
    torch.cuda.synchronize()
    assert torch.equal(y1, y_ref) and not torch.equal(y0, y1)
    out = torch.empty_like(y1)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            out.copy_(lin_mod.linear(x, w))
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out.copy_(lin_mod.linear(x, w))
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, y1)


def test_packed_weight_unpacks_and_rejects_bad_operands(gpu, lin_mod):
    """unpack_fp8_in_place restores the row-major bytes exactly; a packed weight
    refuses the calls the replaced binding would have served on row-major bytes
    (fp32 input); uninstall(mod, model) unpacks every packed weight."""
    N, K = 1024, 4096
    w = _fp8_param(N, K, gpu, 21)
    orig = w.detach().view(torch.uint8).clone()
    x = bf16_tensor(synth.normal_bf16(synth.stream_key(9, synth.S_FP8_X), (3, K), 1.0), gpu)
    y = lin_mod.linear(x, w)
    assert kernels.is_packed(w) and not torch.equal(w.detach().view(torch.uint8), orig)
    with pytest.raises(TypeError):
        lin_mod.linear(x.float(), w)
    with pytest.raises(ValueError):
        lin_mod.linear(x[:, :1024].contiguous(), w)
    assert kernels.unpack_fp8_in_place(w) and not kernels.is_packed(w)
    assert torch.equal(w.detach().view(torch.uint8), orig)
    assert torch.equal(lin_mod.linear(x, w), y)
    model = torch.nn.Module()
    model.w = w
    kernels.pack_fp8_weights(model)
    assert kernels.is_packed(w)
    kernels.uninstall(lin_mod, model)
    kernels.install(lin_mod)
    assert not kernels.is_packed(w) and torch.equal(w.detach().view(torch.uint8), orig)


def test_pack_fp8_weights_leaves_moe_layers_to_the_moe_packer(gpu, mod):
    """pack_fp8_weights skips the MoE's shared expert; and a shared expert packed in
    place by the FP8 linear path before the MoE layer is built is turned back
    before the bank packer reads it, so the layer still matches the golden vectors."""
    case = CASES["toy_t4"]
    inp = make_inputs(case)
    moe = mm.moe_from_case(case, inp, gpu)
    model = torch.nn.Module()
    model.ffn = moe
    assert kernels.pack_fp8_weights(model) == 0
    assert not kernels.is_packed(moe.shared_experts.w1.weight)
    # the shared expert's linears run through the installed FP8 path first
    for lin in (moe.shared_experts.w1, moe.shared_experts.w3, moe.shared_experts.w2):
        assert kernels._packed_of(lin.weight) is not None and kernels.is_packed(lin.weight)
    wm.install(mod)
    x = bf16_tensor(inp.x, gpu).view(1, case.T, case.dim)
    ids = torch.from_numpy(inp.input_ids).to(gpu).view(1, case.T)
    y = mod.MoE.forward(moe, x, ids)
    torch.cuda.synchronize()
    got = f32_of_bf16(y.view(case.T, case.dim))
    gold = from_bf16_bits(np.load(f"tests/golden/{case.name}.npz")["y_bf16"])
    rel, cos = om.max_rel_err(got, gold), om.cosine(got, gold)
    assert rel <= 1e-2 and cos >= 0.9999, (rel, cos)
    # released: no packed-tile record is left on the emptied parameters
    assert not hasattr(moe.shared_experts.w1.weight, "_wz_packed")


@pytest.mark.parametrize("name", ["toy_t4", "top6_t8", "toy_t1"])
def test_drafter_moe_bound_per_instance(gpu, mod, name):
    """install_drafter binds the HIP layer on each non-hash MTP block's MoE as an
    instance attribute (expert_bank.install_drafter, expert_bank.py:167-191), so the
    drafter's MoE never reaches the class-level forward or a grouped-GEMM kernel of
    the reference; the output matches the reference's golden vectors.  A hash-routed
    block is left alone, as the reference leaves it."""
    case = CASES[name]
    inp = make_inputs(case)
    moe = mm.moe_from_case(case, inp, gpu)
    hcase = CASES["hash_t3"]
    hmoe = mm.moe_from_case(hcase, make_inputs(hcase), gpu)
    hmoe.layer_id = 1
    tail = types.SimpleNamespace(mtp=[types.SimpleNamespace(ffn=moe), types.SimpleNamespace(ffn=hmoe)])
    assert wm.install_drafter(tail, mod) == 0  # V4_DSPARK_MOE is not set
    assert wm.install_drafter(tail, mod, force=True) == 1
    assert wm.install_drafter(tail, mod, force=True) == 0  # already bound
    assert "forward" in moe.__dict__ and "forward" not in hmoe.__dict__
    x = bf16_tensor(inp.x, gpu).view(1, case.T, case.dim)
    ids = torch.from_numpy(inp.input_ids).to(gpu).view(1, case.T)
    y = moe(x, ids)  # nn.Module.__call__ finds the instance binding, as the model's block does
    torch.cuda.synchronize()
    assert moe.ref_calls == 0 and getattr(moe, "_draft_steps", 0) == 1
    got = f32_of_bf16(y.view(case.T, case.dim))
    gold = from_bf16_bits(np.load(f"tests/golden/{name}.npz")["y_bf16"])
    rel, cos = om.max_rel_err(got, gold), om.cosine(got, gold)
    assert rel <= 1e-2 and cos >= 0.9999, (rel, cos)
    assert wm.drafter_coverage(tail) == {0: (1, {}), 1: (0, {})}
    # a layer the HIP path cannot serve declines to the class-level forward, tallied
    mod.world_size = 2
    try:
        yd = moe(x, ids)
    finally:
        mod.world_size = 1
    assert moe.ref_calls == 1 and float(yd.flatten()[0]) == mm.SENTINEL
    assert moe._draft_declined == {"world_size>1": 1}
    assert wm.uninstall_drafter(tail) == 1 and "forward" not in moe.__dict__
