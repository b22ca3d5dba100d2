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
    assert wm.moe_chain(mod) == ["ref"]
    assert wm.install(mod) is True
    assert getattr(mod.MoE.forward, "_v4_hip_moe", False)
    assert wm.install(mod) is False  # marker seen: no double wrap
    assert wm._REF_FORWARD is ref
    assert wm.moe_chain(mod) == ["hip", "ref"]
    assert wm.uninstall(mod) is True
    assert mod.MoE.forward is ref and wm.moe_chain(mod) == ["ref"]
    assert wm.uninstall(mod) is False


def _marked_layer(name, marker, kept):
    """A module shaped like one of the reference's MoE replacements
    (expert_batch / fp4_grouped / expert_dispatch): a forward carrying the
    install marker and a module-level _REF_FORWARD."""
    import sys

    m = types.ModuleType(name)

    def fwd(self, x, input_ids):
        return m._REF_FORWARD(self, x, input_ids)

    fwd.__module__ = name
    setattr(fwd, marker, True)
    m.forward, m._REF_FORWARD = fwd, kept
    sys.modules[name] = m
    return m


def test_moe_chain_walks_every_kept_forward(mod):
    """moe_chain follows each marked forward to the one it kept, as the reference's
    controls.moe_chain does (serving/controls.py:45-68)."""
    import sys

    ref = mod.MoE.forward
    grouped = _marked_layer("fake_fp4_grouped", "_v4_grouped", ref)
    multi = _marked_layer("fake_expert_batch", "_v4_multi", grouped.forward)
    try:
        mod.MoE.forward = multi.forward
        assert wm.moe_chain(mod) == ["multi", "grouped", "ref"]
        wm.install(mod)
        assert wm.moe_chain(mod) == ["hip", "multi", "grouped", "ref"]
        wm.uninstall(mod)
        grouped._REF_FORWARD = multi.forward  # a loop
        assert wm.moe_chain(mod) == ["multi", "grouped", "CYCLE"]
        del sys.modules["fake_fp4_grouped"]
        assert wm.moe_chain(mod) == ["multi", "grouped", "ORPHAN"]
    finally:
        sys.modules.pop("fake_fp4_grouped", None)
        sys.modules.pop("fake_expert_batch", None)


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
    orig = {n: (lambda *a, **k: None) for n in ("act_quant", "fp8_gemm", "fp4_gemm", "sparse_attn", "linear")}
    for n, f in orig.items():
        setattr(m, n, f)
    assert kernels.install(m) is True
    assert m.act_quant is kernels.act_quant and m.fp8_gemm is kernels.fp8_gemm and m.fp4_gemm is kernels.fp4_gemm
    assert m.sparse_attn is kernels.sparse_attn and m.linear is kernels.linear
    assert kernels.install(m) is False
    assert kernels.uninstall(m) is True
    assert all(getattr(m, n) is f for n, f in orig.items())


def _torch_act_quant(x, block_size=128, scale_fmt=None, scale_dtype=torch.float32, inplace=False):
    """The reference's CPU act_quant statement (torch_ops.py:33-49), written out
    here as the binding install() replaces."""
    z = x.float().unflatten(-1, (-1, block_size))
    amax = z.abs().amax(-1, keepdim=True).clamp_min(1e-4)
    s = amax / 448.0
    if scale_fmt is not None:
        s = torch.exp2(torch.ceil(torch.log2(s)))
    q = (z / s).clamp(-448, 448).to(torch.float8_e4m3fn)
    if inplace:
        x.copy_((q.float() * s).flatten(-2).to(x.dtype))
        return x
    return q.flatten(-2), s.squeeze(-1).to(scale_dtype)


def test_act_quant_outside_the_path_goes_to_the_replaced_binding():
    """The attention calls act_quant(kv, 64, ..., True) (architecture.py:470, 632):
    after install() that call must reach the replaced act_quant, not fail."""
    m = types.ModuleType("model_host")
    m.act_quant = _torch_act_quant
    kernels.install(m)
    try:
        x = torch.randn(3, 256).to(torch.bfloat16)
        want = _torch_act_quant(x.clone(), 64, "ue8m0", torch.float32, True)
        got = m.act_quant(x.clone(), 64, "ue8m0", torch.float32, True)
        assert torch.equal(got, want)
        q1, s1 = m.act_quant(x, 64, None, torch.float32)
        q0, s0 = _torch_act_quant(x, 64, None, torch.float32)
        assert torch.equal(q1.view(torch.uint8), q0.view(torch.uint8)) and torch.equal(s1, s0)
    finally:
        kernels.uninstall(m)
    with pytest.raises(NotImplementedError):
        kernels.act_quant(torch.zeros(2, 128, dtype=torch.bfloat16), 64)


def test_installed_linear_passes_non_fp8_weights_through():
    """linear() for a bf16 weight is the replaced linear's result (F.linear)."""
    import torch.nn.functional as F

    m = types.ModuleType("model_linear")
    m.linear = lambda x, w, bias=None: F.linear(x, w)
    kernels.install(m)
    try:
        x, w = torch.randn(2, 64), torch.randn(8, 64)
        assert torch.equal(m.linear(x, w), F.linear(x, w))
    finally:
        kernels.uninstall(m)


def test_kernels_refuse_cpu_tensors():
    """The product has no CPU path: a CPU tensor is an error, not a fallback."""
    x = torch.zeros(2, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU only"):
        kernels.act_quant(x, 128, "ue8m0", torch.float8_e8m0fnu)
    a = torch.zeros(2, 128, dtype=torch.uint8).view(torch.float8_e4m3fn)
    s = torch.zeros(2, 1, dtype=torch.float32)
    with pytest.raises(RuntimeError, match="GPU only"):
        kernels.fp8_gemm(a, s, a, torch.ones(1, 1))


def test_installed_linear_rejects_mismatched_fp8_operands_before_launch():
    """An FP8 weight whose K or block-scale grid does not match x raises ValueError
    in linear() before any packing or launch (the packed kernels read K and the
    scale grid from these; a wider x would read past the weight)."""
    m = types.ModuleType("model_linear_fp8")
    m.block_size, m.scale_fmt, m.scale_dtype = 128, "ue8m0", torch.float8_e8m0fnu

    def unused(*a, **k):
        raise AssertionError("the replaced binding was called")

    m.linear = unused
    kernels.install(m)
    try:
        w = torch.nn.Parameter(torch.zeros(256, 512, dtype=torch.uint8).view(torch.float8_e4m3fn),
                               requires_grad=False)
        w.scale = torch.nn.Parameter(torch.zeros(2, 4, dtype=torch.uint8).view(torch.float8_e8m0fnu),
                                     requires_grad=False)
        for K in (640, 384):
            with pytest.raises(ValueError, match="K="):
                m.linear(torch.zeros(3, K, dtype=torch.bfloat16), w)
        w.scale = torch.nn.Parameter(torch.zeros(2, 3, dtype=torch.uint8).view(torch.float8_e8m0fnu),
                                     requires_grad=False)
        with pytest.raises(ValueError, match="block scales"):
            m.linear(torch.zeros(3, 512, dtype=torch.bfloat16), w)
        assert not hasattr(w, "_wz_packed")
    finally:
        kernels.uninstall(m)


def _pack_statement(w: torch.Tensor) -> torch.Tensor:
    """The FP8 tile layout wz_fp8_pack writes (pack.hip, mode 3): [N/16][K/128][2 halves]
    [64 lanes][16 B], lane l = 16 g + r of half h holding row r, K [64 h + 16 g, +16);
    written out here element by element."""
    N_, K = w.shape
    out = torch.empty(N_ * K, dtype=torch.uint8)
    u = w.view(torch.uint8)
    i = 0
    for nt in range(N_ // 16):
        for kb in range(K // 128):
            for h in range(2):
                for ln in range(64):
                    r, g = ln & 15, ln >> 4
                    c = kb * 128 + 64 * h + 16 * g
                    out[i:i + 16] = u[nt * 16 + r, c:c + 16]
                    i += 16
    return out


def test_unpack_in_place_inverts_the_tile_layout():
    """unpack_fp8_in_place restores the row-major bytes from the packed tiles (CPU
    tensors: the permutation is torch's, no kernel)."""
    g = torch.Generator().manual_seed(3)
    rowmajor = torch.randint(0, 256, (32, 256), generator=g, dtype=torch.uint8)
    p = torch.nn.Parameter(_pack_statement(rowmajor).view(32, 256).view(torch.float8_e4m3fn), requires_grad=False)
    assert kernels.unpack_fp8_in_place(p) is False  # not marked packed: left alone
    p._wz_packed = (p.data_ptr(), p._version)
    assert kernels.is_packed(p)
    assert kernels.unpack_fp8_in_place(p) is True
    assert torch.equal(p.detach().view(torch.uint8), rowmajor) and not kernels.is_packed(p)


def test_drafter_install_needs_the_flag_and_skips_hash_layers():
    """install_drafter binds nothing unless V4_DSPARK_MOE is set (or forced), and never
    a hash-routed block's MoE (expert_bank.py:167-191)."""
    hmoe = mm.MoE(0, 256, 128, 8, 2, hash_layer=True)
    tail = types.SimpleNamespace(mtp=[types.SimpleNamespace(ffn=hmoe), types.SimpleNamespace(ffn=None)])
    assert wm.install_drafter(tail, types.ModuleType("m")) == 0
    assert wm.install_drafter(tail, types.ModuleType("m"), force=True) == 0
    assert "forward" not in hmoe.__dict__
    assert wm.uninstall_drafter(tail) == 0
