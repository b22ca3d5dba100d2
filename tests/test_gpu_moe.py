"""GPU parity of the HIP MoE layer (routing, permutation, experts, combine).

Bar (stated here, applied below):
  * expert indices and their order: bit-exact vs the oracle, except tokens
    whose k-th vs (k+1)-th biased-score margin is below NEAR_TIE (reported);
  * canonical permutation (offsets, perm_token, perm_slot): bit-exact;
  * routing weights: |d| <= 4 fp32 ulp;
  * layer output (bf16): max|d|/max|ref| <= 1e-2 and cosine >= 0.9999 vs the
    oracle and vs the reference's own golden vectors.
"""

import numpy as np
import pytest
import torch

from oracle import moe as om
from oracle.numerics import e8m0_decode, from_bf16_bits
from tests.golden.cases import CASES, make_inputs, oracle_params
from tests.helpers import bf16_tensor, bits16, f32_of_bf16, u8_tensor
from wanferenz_amd import synth
from wanferenz_amd.moe import HipMoE, MoEConfig, MoEWeights
from wanferenz_amd import _native as N

pytestmark = pytest.mark.gpu

TOL_REL = 1e-2
TOL_COS = 0.9999
NEAR_TIE = 1e-6   # relative margin below which a top-k flip is reported, not failed


def upload_case(case, inp, dev):
    cfg = MoEConfig(case.dim, case.inter, case.n_experts, case.topk, case.score_func,
                    case.route_scale, case.swiglu_limit,
                    N.WZ_SCALE_UE8M0 if case.round_pow2 else N.WZ_SCALE_F32, N.WZ_WSCALE_E8M0)
    I, nb = case.inter, case.inter // 128
    w = MoEWeights(
        gate_w=bf16_tensor(inp.gate_w, dev),
        gate_bias=None if inp.gate_bias is None else torch.from_numpy(inp.gate_bias).to(dev),
        w13=u8_tensor(inp.w13, dev), w13_s=u8_tensor(inp.w13_s, dev),
        w2=u8_tensor(inp.w2, dev), w2_s=u8_tensor(inp.w2_s, dev),
        sh_w1=u8_tensor(inp.sh_w13[:I], dev), sh_w1_s=u8_tensor(inp.sh_w13_s[:nb], dev),
        sh_w3=u8_tensor(inp.sh_w13[I:], dev), sh_w3_s=u8_tensor(inp.sh_w13_s[nb:], dev),
        sh_w2=u8_tensor(inp.sh_w2, dev), sh_w2_s=u8_tensor(inp.sh_w2_s, dev),
        tid2eid=None if inp.tid2eid is None else torch.from_numpy(inp.tid2eid).to(dev),
    )
    return HipMoE(cfg, w, max_tokens=case.T)


def check_routing(moe, x, ids, gate, E):
    """Routing of all rows vs the oracle's GateResult; returns the near-tie tokens."""
    w, idx, off, ptok, pslot = moe.route(x, ids)
    torch.cuda.synchronize()
    idx = idx.cpu().numpy()
    near = []
    for t in range(idx.shape[0]):
        if not np.array_equal(idx[t], gate.indices[t]):
            rel = gate.margin[t] / max(abs(gate.biased[t]).max(), 1e-30)
            assert rel < NEAR_TIE, f"token {t}: {idx[t]} != {gate.indices[t]} (margin {gate.margin[t]})"
            near.append(t)
    if near:
        print(f"near-tie tokens (margin < {NEAR_TIE} rel): {near}")
        return near
    wd = np.abs(w.cpu().numpy() - gate.weights)
    ulp = np.spacing(np.abs(gate.weights).astype(np.float32))
    assert (wd <= 4 * ulp).all(), wd.max()
    counts, offsets, rt, rs = om.permutation(gate.indices, E)
    assert np.array_equal(off.cpu().numpy(), offsets)
    assert np.array_equal(ptok.cpu().numpy(), rt)
    assert np.array_equal(pslot.cpu().numpy(), rs)
    return near


@pytest.mark.parametrize("name", list(CASES))
def test_moe_golden_cases(gpu, name):
    case = CASES[name]
    inp = make_inputs(case)
    moe = upload_case(case, inp, gpu)
    x = bf16_tensor(inp.x, gpu)
    ids = torch.from_numpy(inp.input_ids).to(gpu)
    ref = om.moe_forward(oracle_params(case, inp), from_bf16_bits(inp.x), inp.input_ids)
    near = check_routing(moe, x, ids, ref.gate, case.n_experts)
    y = moe.forward(x, ids)
    got = f32_of_bf16(y)
    rel, cos = om.max_rel_err(got, ref.y), om.cosine(got, ref.y)
    assert rel <= TOL_REL and cos >= TOL_COS, (rel, cos)
    gold = from_bf16_bits(np.load(f"tests/golden/{name}.npz")["y_bf16"])
    rel_g, cos_g = om.max_rel_err(got, gold), om.cosine(got, gold)
    assert rel_g <= TOL_REL and cos_g >= TOL_COS, (rel_g, cos_g)
    print(f"{name}: rel {rel:.2e} cos {cos:.8f}  vs golden rel {rel_g:.2e}; "
          f"bit-equal {np.mean(got == ref.y):.4f}; near-ties {near}")


V4 = dict(dim=4096, inter=2048, n_experts=256, topk=6)


def _v4_cfg():
    return MoEConfig(V4["dim"], V4["inter"], V4["n_experts"], V4["topk"], "sqrtsoftplus", 1.5, 10.0,
                     N.WZ_SCALE_UE8M0, N.WZ_WSCALE_E8M0)


@pytest.fixture(scope="module")
def v4_layer(gpu):
    cfg = _v4_cfg()
    w, host = synth.synthetic_moe(cfg, seed=0, layer=0, device=gpu)
    moe = HipMoE(cfg, w, max_tokens=64)
    return cfg, w, host, moe


def _oracle_params_from_device(cfg, w, host, experts, bias=None, round_pow2=True):
    """Oracle parameters for the experts a routing touched, copied back from HBM."""
    I = cfg.inter
    ex = [None] * cfg.n_experts
    for e in experts:
        w13 = w.w13[e].cpu().numpy()
        w13s = e8m0_decode(w.w13_s[e].cpu().numpy())
        ex[e] = (om.Fp4Linear(w13[:I], w13s[:I]), om.Fp4Linear(w13[I:], w13s[I:]),
                 om.Fp4Linear(w.w2[e].cpu().numpy(), e8m0_decode(w.w2_s[e].cpu().numpy())))
    shared = (om.Fp8Linear(w.sh_w1.cpu().numpy(), e8m0_decode(w.sh_w1_s.cpu().numpy())),
              om.Fp8Linear(w.sh_w3.cpu().numpy(), e8m0_decode(w.sh_w3_s.cpu().numpy())),
              om.Fp8Linear(w.sh_w2.cpu().numpy(), e8m0_decode(w.sh_w2_s.cpu().numpy())))
    return om.MoEParams(cfg.dim, I, cfg.n_experts, cfg.topk, from_bf16_bits(host["gate_w"]),
                        host.get("gate_bias") if bias is None else bias, ex, shared, cfg.score_func,
                        cfg.route_scale,
                        cfg.swiglu_limit, round_pow2, None)


def test_v4_device_fill_matches_host_generator(v4_layer):
    cfg, w, host, moe = v4_layer
    e = 137
    key = synth.stream_key(0, synth.layer_stream(0, synth.S_W13))
    n = 2 * cfg.inter * cfg.dim // 2
    ref = synth.fill_u8(key, e * n, n)
    assert np.array_equal(w.w13[e].cpu().numpy().ravel(), ref)
    key = synth.stream_key(0, synth.layer_stream(0, synth.S_W2_S))
    n = cfg.dim * cfg.inter // 32
    ref = synth.fill_e8m0(key, e * n, n, *synth.ROUTED_E8M0)
    assert np.array_equal(w.w2_s[e].cpu().numpy().ravel(), ref)


def _v4_decode_check(cfg, w, host, moe, T, round_pow2=True):
    xb = synth.normal_bf16(synth.stream_key(100 + T, synth.S_X), (T, cfg.dim), 1.0)
    x = bf16_tensor(xb, "cuda")
    g = om.gate(from_bf16_bits(xb), from_bf16_bits(host["gate_w"]), host["gate_bias"], cfg.topk,
                cfg.score_func, cfg.route_scale)
    p = _oracle_params_from_device(cfg, w, host, sorted(set(g.indices.ravel().tolist())), round_pow2=round_pow2)
    ref = om.moe_forward(p, from_bf16_bits(xb))
    near = check_routing(moe, x, None, ref.gate, cfg.n_experts)
    # the decode kernels route on their own (route_decode_kernel): check what they export
    rw = torch.empty(T, cfg.topk, dtype=torch.float32, device="cuda")
    ri = torch.empty(T, cfg.topk, dtype=torch.int64, device="cuda")
    y = moe.forward(x, routing_out=(rw, ri))
    if not near:
        assert np.array_equal(ri.cpu().numpy(), ref.gate.indices)
        wd = np.abs(rw.cpu().numpy() - ref.gate.weights)
        assert (wd <= 4 * np.spacing(np.abs(ref.gate.weights).astype(np.float32))).all(), wd.max()
    got = f32_of_bf16(y)
    rel, cos = om.max_rel_err(got, ref.y), om.cosine(got, ref.y)
    assert rel <= TOL_REL and cos >= TOL_COS, (rel, cos)
    print(f"V4 T={T} pow2 {round_pow2}: rel {rel:.2e} cos {cos:.8f} bit-equal {np.mean(got == ref.y):.4f} "
          f"near-ties {near}")


@pytest.mark.parametrize("T", [1, 2, 4, 5, 8])
def test_v4_decode_parity(v4_layer, T):
    cfg, w, host, moe = v4_layer
    _v4_decode_check(cfg, w, host, moe, T)


def _norm_weight(D, seed, dev):
    rng = np.random.default_rng(seed)
    return torch.from_numpy(rng.uniform(0.5, 1.5, D).astype(np.float32)).to(dev)


def _forward_norm_check(moe, cfg, h, nw, ids=None):
    """forward_norm(h) against rms_norm(h) then forward(): output and routing torch.equal."""
    from wanferenz_amd import kernels

    T, k = h.size(0), cfg.topk
    dev = h.device
    r1 = (torch.empty(T, k, dtype=torch.float32, device=dev), torch.empty(T, k, dtype=torch.int64, device=dev))
    r2 = (torch.empty_like(r1[0]), torch.empty_like(r1[1]))
    y1 = moe.forward_norm(h, nw, 1e-6, ids, routing_out=r1).clone()
    m = kernels.rms_norm(h, nw, 1e-6)
    y2 = moe.forward(m, ids, routing_out=r2).clone()
    torch.cuda.synchronize()
    assert torch.equal(r1[1], r2[1]), "routing indices differ"
    assert torch.equal(r1[0], r2[0]), "routing weights differ"
    assert torch.equal(y1, y2), f"output differs at T={T}"
    assert torch.isfinite(y1.float()).all()


@pytest.mark.parametrize("T", [1, 2, 3, 4, 5, 7, 8, 9, 16])
def test_v4_forward_norm_equals_norm_then_forward(v4_layer, T):
    """The block's ffn RMSNorm folded into the layer's routing launch (every gate
    and shared-expert workgroup normalises the rows it reads; T <= 8) gives the
    bits of kernels.rms_norm followed by forward(), at every decode width (T = 9
    and 16 run the norm launch first), on a residual-stream-sized h (std 3) and a
    non-trivial norm weight."""
    cfg, w, host, moe = v4_layer
    dev = w.gate_w.device
    h = bf16_tensor(synth.normal_bf16(synth.stream_key(900 + T, synth.S_X), (T, cfg.dim), 3.0), dev)
    _forward_norm_check(moe, cfg, h, _norm_weight(cfg.dim, T, dev))


@pytest.mark.parametrize("name", ["toy_t4", "hash_t3", "toy_t4_fp32scale", "top6_t8"])
def test_forward_norm_golden_shapes(gpu, name):
    """forward_norm at the golden cases' shapes: D = 1024 and 512, a hash-routed
    layer (ids on the device), float activation scales, top-6 of 32 experts."""
    case = CASES[name]
    inp = make_inputs(case)
    moe = upload_case(case, inp, gpu)
    cfg = moe.cfg
    h = bf16_tensor(synth.normal_bf16(synth.stream_key(77, synth.S_X), (case.T, case.dim), 2.0), gpu)
    ids = torch.from_numpy(inp.input_ids).to(gpu)
    _forward_norm_check(moe, cfg, h, _norm_weight(case.dim, 5, gpu), ids)


def test_forward_norm_wide_batch_runs_the_norm_first(v4_layer):
    """Above the decode widths forward_norm runs the norm launch, then forward."""
    cfg, w, host, moe = v4_layer
    dev = w.gate_w.device
    h = bf16_tensor(synth.normal_bf16(synth.stream_key(901, synth.S_X), (24, cfg.dim), 3.0), dev)
    _forward_norm_check(moe, cfg, h, _norm_weight(cfg.dim, 24, dev))


def test_v4_decode_parity_fp32_act_scales(v4_layer):
    """Float (non power-of-two) activation scales at the V4 shape: the decode
    w2 then runs w2_combine_kernel (the LDS-staged kernel serves K-blocks of 16
    only with power-of-two scales)."""
    cfg, w, host, _ = v4_layer
    cfg32 = MoEConfig(V4["dim"], V4["inter"], V4["n_experts"], V4["topk"], "sqrtsoftplus", 1.5, 10.0,
                      N.WZ_SCALE_F32, N.WZ_WSCALE_E8M0)
    moe32 = HipMoE(cfg32, w, max_tokens=8)
    _v4_decode_check(cfg32, w, host, moe32, 3, round_pow2=False)


def test_v4_decode_routing_publication_over_many_steps(v4_layer):
    """The decode routing launch hands the gate scores of its 128 gate
    workgroups to the last one to arrive through relaxed agent-scope stores, a
    drained wait and an agent-scope add (moe_common.h).  Over 96 distinct inputs
    (T = 1, 2, 4, 8; eager calls and replays of one captured graph, the input
    changed in place between replays, with eager work in between) the routing it
    exports equals the oracle's gate every time: indices exactly, weights within
    4 fp32 ulp (a top-k flip is allowed only at a relative key margin below
    NEAR_TIE)."""
    cfg, w, host, moe = v4_layer
    gw = from_bf16_bits(host["gate_w"])
    flips = 0
    for T in (1, 2, 4, 8):
        x = torch.empty(T, cfg.dim, dtype=torch.bfloat16, device="cuda")
        out = torch.empty_like(x)
        rw = torch.empty(T, cfg.topk, dtype=torch.float32, device="cuda")
        ri = torch.empty(T, cfg.topk, dtype=torch.int64, device="cuda")
        x.copy_(bf16_tensor(synth.normal_bf16(synth.stream_key(4000 + T, synth.S_X), (T, cfg.dim), 1.0), "cuda"))
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(2):
                moe.forward(x, out=out, routing_out=(rw, ri))
        torch.cuda.current_stream().wait_stream(s)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            moe.forward(x, out=out, routing_out=(rw, ri))
        for step in range(24):
            xb = synth.normal_bf16(synth.stream_key(5000 + 100 * T + step, synth.S_X), (T, cfg.dim), 1.0)
            x.copy_(bf16_tensor(xb, "cuda"))
            ri.fill_(-1)
            if step % 2:
                graph.replay()
            else:
                moe.forward(x, out=out, routing_out=(rw, ri))
            torch.cuda.synchronize()
            g = om.gate(from_bf16_bits(xb), gw, host["gate_bias"], cfg.topk, cfg.score_func, cfg.route_scale)
            got_i, got_w = ri.cpu().numpy(), rw.cpu().numpy()
            for t in range(T):
                if not np.array_equal(got_i[t], g.indices[t]):
                    rel = g.margin[t] / max(abs(g.biased[t]).max(), 1e-30)
                    assert rel < NEAR_TIE, f"T={T} step {step} token {t}: {got_i[t]} != {g.indices[t]}"
                    flips += 1
                    continue
                wd = np.abs(got_w[t] - g.weights[t])
                assert (wd <= 4 * np.spacing(np.abs(g.weights[t]).astype(np.float32))).all(), (T, step, t)
        del graph
    print(f"96 decode routings checked, near-tie flips {flips}")


def test_v4_decode_graph_replay(v4_layer):
    """A captured decode step replays to the eager result, replay after replay."""
    cfg, w, host, moe = v4_layer
    T = 4
    x = bf16_tensor(synth.normal_bf16(synth.stream_key(7, synth.S_X), (T, cfg.dim), 1.0), "cuda")
    eager = moe.forward(x).clone()
    out = torch.empty_like(x)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            moe.forward(x, out=out)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        moe.forward(x, out=out)
    for i in range(4):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i} differs from eager"
        _ = moe.forward(x)  # eager work between replays


def _expected_pack_w13(w13, w13_s, D, I):
    """numpy statement of the packed w13 layout (pack.hip): [E][I/16][D/128][2][64 lanes][16 B]."""
    E = w13.shape[0]
    KB = D // 128
    out = np.empty((E, I // 16, KB, 2, 64, 16), np.uint8)
    lanes = np.arange(64)
    r, g = lanes & 15, lanes >> 4
    for m in range(2):
        rows = w13[:, m * I:(m + 1) * I].reshape(E, I // 16, 16, D // 2)  # [E, FT, 16, D/2]
        for kb in range(KB):
            for ln in range(64):
                out[:, :, kb, m, ln] = rows[:, :, r[ln], kb * 64 + g[ln] * 16: kb * 64 + g[ln] * 16 + 16]
    KG = (KB + 3) // 4
    sc = np.zeros((E, I // 16, KG, 2, 64, 4), np.uint8)
    for m in range(2):
        srows = w13_s[:, m * I:(m + 1) * I].reshape(E, I // 16, 16, D // 32)
        for kg in range(KG):
            for j in range(4):
                kb = kg * 4 + j
                if kb < KB:
                    for ln in range(64):
                        sc[:, :, kg, m, ln, j] = srows[:, :, r[ln], kb * 4 + g[ln]]
    return out.reshape(-1), sc.reshape(-1)


def test_pack_layout_matches_statement(gpu):
    case = CASES["toy_t4"]
    inp = make_inputs(case)
    moe = upload_case(case, inp, gpu)
    torch.cuda.synchronize()
    exp_w, exp_s = _expected_pack_w13(inp.w13, inp.w13_s, case.dim, case.inter)
    assert np.array_equal(moe.packed["w13p"].cpu().numpy(), exp_w)
    assert np.array_equal(moe.packed["w13p_s"].cpu().numpy(), exp_s)


# ------------------------------------------------------------------ prefill ---
# T > 16 runs the expert-grouped MFMA GEMM path (moe_prefill.hip).  The layer is
# token-local, so at large T the oracle is evaluated on sampled rows (all
# routing is still checked in full), and every row is compared with the decode
# path run over 16-token chunks of the same input.

PREFILL_CASES = {
    # oracle-only cases (no reference golden at these T): fp32 scales, hash routing, top-6
    "toy_t40_fp32scale": dict(case="toy_t4_fp32scale", T=40),
    "hash_t48": dict(case="hash_t3", T=48),
    "top6_t100": dict(case="top6_t8", T=100),
}


@pytest.mark.parametrize("name", list(PREFILL_CASES))
def test_moe_prefill_oracle_cases(gpu, name):
    import dataclasses
    spec = PREFILL_CASES[name]
    case = dataclasses.replace(CASES[spec["case"]], name=name, T=spec["T"])
    inp = make_inputs(case)
    moe = upload_case(case, inp, gpu)
    x = bf16_tensor(inp.x, gpu)
    ids = torch.from_numpy(inp.input_ids).to(gpu)
    ref = om.moe_forward(oracle_params(case, inp), from_bf16_bits(inp.x), inp.input_ids)
    near = check_routing(moe, x, ids, ref.gate, case.n_experts)
    rw = torch.empty(case.T, case.topk, dtype=torch.float32, device=gpu)
    ri = torch.empty(case.T, case.topk, dtype=torch.int64, device=gpu)
    y = moe.forward(x, ids, routing_out=(rw, ri))
    if not near:
        assert np.array_equal(ri.cpu().numpy(), ref.gate.indices)
    got = f32_of_bf16(y)
    rel, cos = om.max_rel_err(got, ref.y), om.cosine(got, ref.y)
    assert rel <= TOL_REL and cos >= TOL_COS, (rel, cos)
    print(f"{name}: rel {rel:.2e} cos {cos:.8f} bit-equal {np.mean(got == ref.y):.4f} near-ties {near}")


def test_prefill_gate_wide_batch(gpu):
    """T >= 1024 takes the 32-token x 64-expert MFMA gate (at this width its rolled K
    loop; 1100 leaves a ragged last token group) and the many-workgroup permutation:
    every token's routing against the oracle's exact gate, the weights within 4 ulp,
    and the offsets and permutation tables exact (check_routing), then the forward's
    exported routing equal to it."""
    import dataclasses
    case = dataclasses.replace(CASES["top6_t8"], name="top6_t1100", T=1100)
    inp = make_inputs(case)
    moe = upload_case(case, inp, gpu)
    x = bf16_tensor(inp.x, gpu)
    g = om.gate(from_bf16_bits(inp.x), from_bf16_bits(inp.gate_w), inp.gate_bias, case.topk, case.score_func,
                case.route_scale)
    near = check_routing(moe, x, None, g, case.n_experts)
    rw = torch.empty(case.T, case.topk, dtype=torch.float32, device=gpu)
    ri = torch.empty(case.T, case.topk, dtype=torch.int64, device=gpu)
    moe.forward(x, routing_out=(rw, ri))
    if not near:
        assert np.array_equal(ri.cpu().numpy(), g.indices)
    print(f"{case.name}: routing of {case.T} tokens exact; near-ties {near}")


def _torch_oracle_rows(cfg, w, xb, g, dev):
    """Every row of the layer by the torch float32 restatement of the reference CPU
    path (oracle/torch_ref.py: act_quant, dequantised fp4/fp8 GEMMs, clamp-SwiGLU,
    the non-accumulating y[idx] += per expert, then the shared expert), run on the
    device over the numpy oracle's exact routing ``g``, the weights read back from
    the layer's reference-layout bank."""
    from oracle import torch_ref as tr

    I, D = cfg.inter, cfg.dim

    def e8m0(t):
        return torch.ldexp(torch.ones(t.shape, device=dev), t.to(torch.int32).float() - 127.0)

    x = torch.from_numpy(from_bf16_bits(xb).reshape(-1, D)).to(dev).to(torch.bfloat16)
    idx = torch.from_numpy(g.indices).to(dev)
    wts = torch.from_numpy(g.weights).to(dev)
    y = torch.zeros(x.shape, dtype=torch.float32, device=dev)
    for e in sorted(set(g.indices.ravel().tolist())):
        w13, s13 = w.w13[e], e8m0(w.w13_s[e])
        ws = (tr.QLinear("fp4", w13[:I], s13[:I]), tr.QLinear("fp4", w13[I:], s13[I:]),
              tr.QLinear("fp4", w.w2[e], e8m0(w.w2_s[e])))
        rows, slot = torch.where(idx == e)
        y[rows] += tr.expert_forward(ws, x[rows], wts[rows, slot, None], cfg.swiglu_limit, True).float()
    shared = tuple(tr.QLinear("fp8", a, e8m0(b)) for a, b in
                   ((w.sh_w1, w.sh_w1_s), (w.sh_w3, w.sh_w3_s), (w.sh_w2, w.sh_w2_s)))
    y += tr.expert_forward(shared, x, None, cfg.swiglu_limit, True).float()
    return f32_of_bf16(y.to(torch.bfloat16))


@pytest.mark.parametrize("T", [12, 16, 17, 24, 32])
def test_v4_multi_token_parity(v4_layer, T):
    """The multi-token widths of the reference's decode paths (expert_batch.py:14-53
    serves T in [2, 32], the drafter T * k <= 32, expert_bank.py:108-164) at the
    V4 shape, each against the oracle directly: routing of every token bit-exact
    (the exported tables too), every output row against the torch float32
    restatement of the reference's CPU path over the oracle's routing, and four
    rows (the first, the last and two of the most loaded expert's) against the
    numpy oracle."""
    cfg, w, host, moe = v4_layer
    xb = synth.normal_bf16(synth.stream_key(300 + T, synth.S_X), (T, cfg.dim), 1.0)
    x = bf16_tensor(xb, "cuda")
    b = host["gate_bias"]
    g = om.gate(from_bf16_bits(xb), from_bf16_bits(host["gate_w"]), b, cfg.topk, cfg.score_func, cfg.route_scale)
    near = check_routing(moe, x, None, g, cfg.n_experts)
    rw = torch.empty(T, cfg.topk, dtype=torch.float32, device="cuda")
    ri = torch.empty(T, cfg.topk, dtype=torch.int64, device="cuda")
    y = moe.forward(x, routing_out=(rw, ri))
    if not near:
        assert np.array_equal(ri.cpu().numpy(), g.indices)
        wd = np.abs(rw.cpu().numpy() - g.weights)
        assert (wd <= 4 * np.spacing(np.abs(g.weights).astype(np.float32))).all(), wd.max()
    got = f32_of_bf16(y)
    full = _torch_oracle_rows(cfg, w, xb, g, x.device)
    rel_t, cos_t = om.max_rel_err(got, full), om.cosine(got, full)
    assert rel_t <= TOL_REL and cos_t >= TOL_COS, (rel_t, cos_t)
    counts = np.bincount(g.indices.ravel(), minlength=cfg.n_experts)
    hot_rows = np.nonzero((g.indices == int(counts.argmax())).any(1))[0]
    rows = sorted({0, T - 1} | set(hot_rows[:2].tolist()))
    gs = om.gate(from_bf16_bits(xb[rows]), from_bf16_bits(host["gate_w"]), b, cfg.topk, cfg.score_func,
                 cfg.route_scale)
    p = _oracle_params_from_device(cfg, w, host, sorted(set(gs.indices.ravel().tolist())))
    ref = om.moe_forward(p, from_bf16_bits(xb[rows]))
    rel, cos = om.max_rel_err(got[rows], ref.y), om.cosine(got[rows], ref.y)
    assert rel <= TOL_REL and cos >= TOL_COS, (rel, cos)
    print(f"V4 T={T}: all rows vs torch oracle rel {rel_t:.2e} cos {cos_t:.8f} bit-equal {np.mean(got == full):.4f};"
          f" rows {rows} vs oracle rel {rel:.2e} cos {cos:.8f}; near-ties {near}")


def _decode_chunks(moe, x, chunk=16):
    return torch.cat([moe.forward(x[i:i + chunk]) for i in range(0, x.size(0), chunk)])


@pytest.mark.parametrize("T,bias", [(64, "normal"), (128, "normal"), (128, "zipf"), (300, "normal"),
                                    (512, "normal"), (512, "zipf"), (2048, "zipf")])
def test_v4_prefill_parity(v4_layer, T, bias):
    """Prefill at the V4 shape; "zipf" is the calibrated Zipf(1.1) gate bias of the
    prefill workload (wanferenz_amd/zipf_v4.json).  All routing is checked in full;
    every output row against the torch float32 restatement of the reference's CPU
    path (on the device, over the oracle's exact routing), 16 sampled rows
    (including rows of the most loaded expert) against the numpy oracle, and every
    row against the decode path run over 16-token chunks."""
    import dataclasses
    cfg, w, host, moe = v4_layer
    b = host["gate_bias"]
    if bias == "zipf":
        b = synth.zipf_bias(cfg.n_experts, beta=synth.zipf_v4_beta())
        w = dataclasses.replace(w, gate_bias=torch.from_numpy(b).to("cuda"))
        moe = moe.with_gate_bias(w.gate_bias, max_tokens=T)
    xb = synth.normal_bf16(synth.stream_key(500 + T, synth.S_X), (T, cfg.dim), 1.0)
    x = bf16_tensor(xb, "cuda")
    g = om.gate(from_bf16_bits(xb), from_bf16_bits(host["gate_w"]), b, cfg.topk, cfg.score_func,
                cfg.route_scale)
    counts = np.bincount(g.indices.ravel(), minlength=cfg.n_experts)
    near = check_routing(moe, x, None, g, cfg.n_experts)
    y = moe.forward(x)
    got = f32_of_bf16(y)
    # oracle on sampled rows: spread over the batch plus tokens of the most loaded expert
    hot = int(counts.argmax())
    hot_rows = np.nonzero((g.indices == hot).any(1))[0]
    rng = np.random.default_rng(T)
    rows = sorted(set(rng.choice(T, size=min(T, 10), replace=False).tolist()) | {0, T - 1}
                  | set(hot_rows[:4].tolist()))
    xs = xb[rows]
    gs = om.gate(from_bf16_bits(xs), from_bf16_bits(host["gate_w"]), b, cfg.topk, cfg.score_func,
                 cfg.route_scale)
    p = _oracle_params_from_device(cfg, w, host, sorted(set(gs.indices.ravel().tolist())), bias=b)
    ref = om.moe_forward(p, from_bf16_bits(xs))
    rel, cos = om.max_rel_err(got[rows], ref.y), om.cosine(got[rows], ref.y)
    assert rel <= TOL_REL and cos >= TOL_COS, (rel, cos)
    # every row against the torch restatement of the reference path
    full = _torch_oracle_rows(cfg, w, xb, g, x.device)
    rel_t, cos_t = om.max_rel_err(got, full), om.cosine(got, full)
    assert rel_t <= TOL_REL and cos_t >= TOL_COS, (rel_t, cos_t)
    # every row against the decode path on 16-token chunks
    dec = f32_of_bf16(_decode_chunks(moe, x))
    rel_d, cos_d = om.max_rel_err(got, dec), om.cosine(got, dec)
    assert rel_d <= TOL_REL and cos_d >= TOL_COS, (rel_d, cos_d)
    print(f"V4 prefill T={T} ({bias} bias, experts hit {int((counts > 0).sum())}, max rows "
          f"{int(counts.max())}): all rows vs torch oracle rel {rel_t:.2e} cos {cos_t:.8f} bit-equal "
          f"{np.mean(got == full):.4f}; {len(rows)} sampled rows vs oracle rel {rel:.2e} cos {cos:.8f}; vs decode "
          f"rel {rel_d:.2e} cos {cos_d:.8f} bit-equal {np.mean(got == dec):.4f}; near-ties {near}")


# Gate score functions other than the V4 sqrt-softplus (Gate.forward, architecture.py:700-705):
# softmax (weights not renormalised) and sigmoid, on the decode (T <= 16) and prefill paths.
SCORE_CASES = [(case, sf, T) for sf in ("softmax", "sigmoid")
               for case, T in (("toy_t4", 4), ("top6_t8", 8), ("top6_t8", 100), ("toy_t37", 37))]


@pytest.mark.parametrize("name,score_func,T", SCORE_CASES)
def test_score_functions(gpu, name, score_func, T):
    import dataclasses

    case = dataclasses.replace(CASES[name], name=f"{name}_{score_func}", T=T, score_func=score_func)
    inp = make_inputs(case)
    moe = upload_case(case, inp, gpu)
    x = bf16_tensor(inp.x, gpu)
    ref = om.moe_forward(oracle_params(case, inp), from_bf16_bits(inp.x))
    near = check_routing(moe, x, None, ref.gate, case.n_experts)
    rw = torch.empty(T, case.topk, dtype=torch.float32, device=gpu)
    ri = torch.empty(T, case.topk, dtype=torch.int64, device=gpu)
    y = moe.forward(x, routing_out=(rw, ri))
    if not near:
        assert np.array_equal(ri.cpu().numpy(), ref.gate.indices)
        wd = np.abs(rw.cpu().numpy() - ref.gate.weights)
        assert (wd <= 4 * np.spacing(np.abs(ref.gate.weights).astype(np.float32))).all(), wd.max()
    got = f32_of_bf16(y)
    rel, cos = om.max_rel_err(got, ref.y), om.cosine(got, ref.y)
    assert rel <= TOL_REL and cos >= TOL_COS, (rel, cos)
    print(f"{case.name} T={T}: rel {rel:.2e} cos {cos:.8f} near-ties {near}")


@pytest.mark.parametrize("score_func,T", [("sigmoid", 4), ("sigmoid", 128), ("softmax", 4), ("softmax", 128)])
def test_v4_score_functions(v4_layer, score_func, T):
    """The V4 shape with the other score functions: decode (route_decode_kernel) and
    prefill (MFMA gate with exact refinement for sigmoid; the fp64 dot gate for
    softmax)."""
    cfg, w, host, _ = v4_layer
    cfg2 = MoEConfig(V4["dim"], V4["inter"], V4["n_experts"], V4["topk"], score_func, 1.5, 10.0,
                     N.WZ_SCALE_UE8M0, N.WZ_WSCALE_E8M0)
    moe = HipMoE(cfg2, w, max_tokens=T)
    xb = synth.normal_bf16(synth.stream_key(900 + T, synth.S_X), (T, cfg.dim), 1.0)
    x = bf16_tensor(xb, "cuda")
    g = om.gate(from_bf16_bits(xb), from_bf16_bits(host["gate_w"]), host["gate_bias"], cfg.topk, score_func,
                cfg.route_scale)
    near = check_routing(moe, x, None, g, cfg.n_experts)
    y = moe.forward(x)
    rows = sorted({0, 1, T // 2, T - 1})
    xs = xb[rows]
    gs = om.gate(from_bf16_bits(xs), from_bf16_bits(host["gate_w"]), host["gate_bias"], cfg.topk, score_func,
                 cfg.route_scale)
    p = _oracle_params_from_device(cfg2, w, host, sorted(set(gs.indices.ravel().tolist())))
    ref = om.moe_forward(p, from_bf16_bits(xs))
    got = f32_of_bf16(y)[rows]
    rel, cos = om.max_rel_err(got, ref.y), om.cosine(got, ref.y)
    assert rel <= TOL_REL and cos >= TOL_COS, (rel, cos)
    print(f"V4 {score_func} T={T}: rel {rel:.2e} cos {cos:.8f} near-ties {near}")


@pytest.mark.parametrize("score_func,T", [("sqrtsoftplus", 1), ("sqrtsoftplus", 4), ("sqrtsoftplus", 16),
                                          ("softmax", 4), ("sigmoid", 11)])
def test_decode_exact_ties(gpu, score_func, T):
    """256 experts whose gate rows and biases come in groups of four equal ones
    (e, e ^ 1, e + 128, (e ^ 1) + 128): every selection key ties exactly with
    three others, in two lanes and two slots of a lane, and the top-k must take
    the lower expert id first (torch.topk's order, the oracle's lexsort).
    T = 16 (96 pairs) runs the decode routing's general table path, the others
    its one-lane-per-pair path."""
    import dataclasses

    case = dataclasses.replace(CASES["top6_t8"], name=f"ties_{score_func}_t{T}", dim=512, inter=256,
                               n_experts=256, T=T, seed=7, score_func=score_func)
    inp = make_inputs(case)
    grp = (np.arange(256) % 128) // 2
    inp.gate_w = np.ascontiguousarray(inp.gate_w[grp])
    inp.gate_bias = np.ascontiguousarray(inp.gate_bias[grp])
    moe = upload_case(case, inp, gpu)
    x = bf16_tensor(inp.x, gpu)
    ref = om.moe_forward(oracle_params(case, inp), from_bf16_bits(inp.x))
    rw = torch.empty(T, case.topk, dtype=torch.float32, device=gpu)
    ri = torch.empty(T, case.topk, dtype=torch.int64, device=gpu)
    y = moe.forward(x, routing_out=(rw, ri))
    got_i = ri.cpu().numpy()
    assert np.array_equal(got_i, ref.gate.indices), (got_i, ref.gate.indices)
    # every token's top group of four is taken whole, in ascending id
    for r in got_i:
        assert r[0] % 2 == 0 and list(r[:4]) == [r[0], r[0] + 1, r[0] + 128, r[0] + 129], r
    wd = np.abs(rw.cpu().numpy() - ref.gate.weights)
    assert (wd <= 4 * np.spacing(np.abs(ref.gate.weights).astype(np.float32))).all(), wd.max()
    got = f32_of_bf16(y)
    rel, cos = om.max_rel_err(got, ref.y), om.cosine(got, ref.y)
    assert rel <= TOL_REL and cos >= TOL_COS, (rel, cos)
    print(f"{case.name}: rel {rel:.2e} cos {cos:.8f}")


@pytest.mark.parametrize("name,T", [("top6_t8", 4), ("toy_t4", 4), ("toy_t4", 16), ("top6_t8", 40)])
def test_replay_stages_reproduce_the_forward(gpu, name, T):
    """wz_moe_replay_stage re-runs a stage of the last forward on its workspace state."""
    import dataclasses
    case = dataclasses.replace(CASES[name], T=T)
    inp = make_inputs(case)
    moe = upload_case(case, inp, gpu)
    x = bf16_tensor(inp.x, gpu)
    y = moe.forward(x).clone()
    out = torch.zeros_like(y)
    for st in (N.WZ_STAGE_ROUTE, N.WZ_STAGE_W13, N.WZ_STAGE_HQUANT, N.WZ_STAGE_W2, N.WZ_STAGE_COMBINE):
        moe.replay_stage(x, st, out)
    torch.cuda.synchronize()
    assert torch.equal(out, y)
    out.zero_()
    moe.replay_stage(x, N.WZ_STAGE_W2, out)
    moe.replay_stage(x, N.WZ_STAGE_COMBINE, out)
    torch.cuda.synchronize()
    assert torch.equal(out, y)
