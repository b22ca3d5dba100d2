"""GPU parity of the decode stage (wanferenz_amd/stage.py): V4 decoder blocks' FP8
projections, fused norms, residual adds and the MoE layer, run eagerly and as one
captured graph.

Bar: every op of the chain vs its restatement in oracle/, fed the stage's own input
to that op (residual adds bit-exact, norms within one bf16 ulp, projections and the
MoE within max|d|/max|ref| <= 1e-2 and cosine >= 0.9999, routing bit-exact); graph
replays equal the eager step bit for bit.
"""

import numpy as np
import pytest
import torch

from oracle import moe as om
from oracle.numerics import bf16_round, e8m0_decode, from_bf16_bits
from tests.helpers import bf16_tensor, bytes8, f32_of_bf16
from tests.test_gpu_moe import _oracle_params_from_device
from wanferenz_amd import _native as N
from wanferenz_amd import kernels, stage, synth
from wanferenz_amd.moe import HipMoE, MoEConfig

pytestmark = pytest.mark.gpu

TOL_REL = 1e-2
TOL_COS = 0.9999


def _close(got, ref):
    return om.max_rel_err(got, ref), om.cosine(got, ref)


def _oracle_linear_q(q, qs, n, k, seed, blocks=None):
    """The oracle's fp8_gemm of pre-quantised activations (the stage's own codes);
    with ``blocks``, only those 128-row blocks of the weight (their output columns)."""
    w, s = stage.synthetic_linear(n, k, seed, "cuda", fp32_scales=False)
    if blocks is None:
        return om.fp8_gemm(q, qs, bytes8(w), e8m0_decode(bytes8(s).reshape(s.shape)))
    rows = torch.from_numpy(np.concatenate([np.arange(b * 128, b * 128 + 128) for b in blocks])).to(w.device)
    return om.fp8_gemm(q, qs, bytes8(w.view(torch.uint8)[rows]), e8m0_decode(bytes8(s).reshape(s.shape)[blocks]))


def _cols(blocks):
    return slice(None) if blocks is None else np.concatenate([np.arange(b * 128, b * 128 + 128) for b in blocks])


def _some_blocks(n, sample):
    nb = n // 128
    return sorted({0, nb // 2, nb - 1}) if sample else None


STAGE_SHAPES = {
    # D, MoE (E, top-k, I), attention widths; "sample": projections checked on three
    # 128-column blocks of the output (first, middle, last)
    "toy": dict(cfg=(1024, 512, 16, 2), dims=dict(q_lora=256, head_dim=128, q_width=2048, idx_width=1024),
                sample=False),
    "v4": dict(cfg=(4096, 2048, 256, 6), dims=dict(q_lora=1024, head_dim=512, q_width=32768, idx_width=8192),
               sample=True),
}


@pytest.mark.parametrize("shape", list(STAGE_SHAPES))
def test_stage_ops_match_oracle(gpu, shape):
    """Two blocks of the stage, every op checked against the oracle fed the stage's
    own input to that op, since each FP8 re-quantisation turns a one-ulp bf16
    difference upstream into an e4m3 rounding flip downstream.  "toy": D 1024, 16
    experts top-2; q_lora 256, head_dim 128, q width 2048, indexer width 1024 (wq_a,
    wkv and wo_b at K = 1024 run the GEMV, wq_b and the indexer at K = 256 the tile
    GEMM).  "v4": the V4-Flash shapes (D 4096, 256 MXFP4 experts top-6, wq_a 1024 x
    4096, wkv 512 x 4096, wq_b 32768 x 1024, indexer wq_b 8192 x 1024, wo_b 4096 x
    8192).  wo_b carries the residual in its epilogue and the second block's norm
    carries the first block's MoE residual.  Residual adds bit-exact, the fused norm
    + act_quant equal to rms_norm then act_quant on the device and to the oracle's
    act_quant of that row, the norms within one bf16 ulp of the oracle's,
    projections and the MoE to the bf16 tolerance, the routing of each MoE the
    oracle's on the stage's input."""
    spec = STAGE_SHAPES[shape]
    D, I_, E_, k_ = spec["cfg"]
    dims, sample = spec["dims"], spec["sample"]
    cfg = MoEConfig(D, I_, E_, k_, "sqrtsoftplus", 1.5, 10.0, N.WZ_SCALE_UE8M0, N.WZ_WSCALE_E8M0)
    T = 4
    layers = [synth.synthetic_moe(cfg, seed=0, layer=l, device=gpu) for l in range(2)]
    blocks = [stage.synthetic_block(HipMoE(cfg, w, max_tokens=T), D, seed=l, device=gpu, **dims)
              for l, (w, _) in enumerate(layers)]
    st = stage.DecodeStage(blocks, T)
    xb = synth.normal_bf16(synth.stream_key(7, synth.S_X), (T, D), 1.0)
    trace = []
    rts = [(torch.empty(T, cfg.topk, dtype=torch.float32, device=gpu),
            torch.empty(T, cfg.topk, dtype=torch.int64, device=gpu)) for _ in blocks]
    y = st.step(bf16_tensor(xb, gpu), routing=rts, trace=trace)
    torch.cuda.synchronize()
    assert np.array_equal(f32_of_bf16(trace[0]["h_in"]), from_bf16_bits(xb).reshape(T, D))

    def close(name, got, ref):
        rel, cos = _close(got, ref)
        assert rel <= TOL_REL and cos >= TOL_COS, (name, rel, cos)

    def one_ulp(name, got, ref):
        rel = np.abs(got - ref) / np.maximum(np.abs(ref), 1e-30)
        assert rel.max() <= 2.0 ** -7, (name, rel.max())

    def norm_quant(name, q_t, s_t, x_t, wgt):
        """The fused norm + act_quant = rms_norm then act_quant on the device, bit for
        bit; that act_quant = the oracle's of the same row; the norm within one bf16
        ulp of the oracle's."""
        yv = kernels.rms_norm(x_t, wgt, 1e-6)
        q2, s2 = kernels.act_quant(yv, 128, "ue8m0", torch.float8_e8m0fnu)
        torch.cuda.synchronize()
        assert torch.equal(q_t.view(torch.uint8), q2.view(torch.uint8)), name
        assert torch.equal(s_t.view(torch.uint8), s2.view(torch.uint8)), name
        yf = f32_of_bf16(yv)
        rq, rs = om.act_quant(yf, 128, True)
        assert np.array_equal(bytes8(q_t).reshape(rq.shape), rq), name
        one_ulp(name, yf, om.rmsnorm(f32_of_bf16(x_t), wgt.cpu().numpy()))

    def dq(t):
        return bytes8(t).reshape(t.shape)

    ql, qw, idw = dims["q_lora"], dims["q_width"], dims["idx_width"]
    for l, ((w, host), b, tr, (_, ri)) in enumerate(zip(layers, blocks, trace, rts)):
        g = {k: f32_of_bf16(v) for k, v in tr.items() if v is not None and v.dtype == torch.bfloat16}
        if l > 0:
            assert np.array_equal(g["h"], bf16_round((g["h_in"] + g["e_in"]).astype(np.float32)))
        hq, hs = dq(tr["hq"]), e8m0_decode(dq(tr["hs"]))
        norm_quant("attn_norm", tr["hq"], tr["hs"], tr["h"], b.attn_norm)
        bl = _some_blocks(ql, sample)
        close("wq_a", g["qa"][:, _cols(bl)], _oracle_linear_q(hq, hs, ql, D, l * 16 + 0, bl))
        bl = _some_blocks(dims["head_dim"], sample)
        close("wkv", g["kv"][:, _cols(bl)], _oracle_linear_q(hq, hs, dims["head_dim"], D, l * 16 + 1, bl))
        qq, qs = dq(tr["qq"]), e8m0_decode(dq(tr["qs"]))
        norm_quant("q_norm", tr["qq"], tr["qs"], tr["qa"], b.q_norm)
        bl = _some_blocks(qw, sample)
        close("wq_b", g["q"][:, _cols(bl)], _oracle_linear_q(qq, qs, qw, ql, l * 16 + 2, bl))
        bl = _some_blocks(idw, sample)
        close("idx_wq_b", g["iq"][:, _cols(bl)], _oracle_linear_q(qq, qs, idw, ql, l * 16 + 3, bl))
        rq, rs = om.act_quant(g["iq"], 128, True)
        bl = _some_blocks(D, sample)
        wo = _oracle_linear_q(rq, rs, D, idw, l * 16 + 4, bl)
        c = _cols(bl)
        close("wo_b + residual", g["h1"][:, c], bf16_round((g["h"][:, c] + wo).astype(np.float32)))
        one_ulp("ffn_norm", g["m"], om.rmsnorm(g["h1"], b.ffn_norm.cpu().numpy()))
        gate = om.gate(g["m"], from_bf16_bits(host["gate_w"]), host["gate_bias"], cfg.topk, cfg.score_func,
                       cfg.route_scale)
        assert np.array_equal(ri.cpu().numpy(), gate.indices)
        p = _oracle_params_from_device(cfg, w, host, sorted(set(gate.indices.ravel().tolist())))
        close("moe", g["e"], om.moe_forward(p, g["m"]).y)
    last = {k: f32_of_bf16(v) for k, v in trace[-1].items() if v is not None and v.dtype == torch.bfloat16}
    assert np.array_equal(f32_of_bf16(y), bf16_round((last["h1"] + last["e"]).astype(np.float32)))


def test_stage_graph_replays_equal_eager(gpu):
    """Two V4-shaped blocks (D 4096, 256 MXFP4 experts top-6; wq_a 1024 x 4096, wkv
    512 x 4096, wq_b 32768 x 1024, indexer wq_b 8192 x 1024, wo_b 4096 x 8192) at T = 4:
    every replay of the captured step equals an eager step on the same input, with
    eager work between replays."""
    cfg = MoEConfig(4096, 2048, 256, 6, "sqrtsoftplus", 1.5, 10.0, N.WZ_SCALE_UE8M0, N.WZ_WSCALE_E8M0)
    T = 4
    blocks = []
    for l in range(2):
        w, _ = synth.synthetic_moe(cfg, seed=0, layer=l, device=gpu)
        blocks.append(stage.synthetic_block(HipMoE(cfg, w, max_tokens=T), 4096, seed=l, device=gpu))
    st = stage.DecodeStage(blocks, T)
    st.capture()
    for s in range(3):
        xb = synth.normal_bf16(synth.stream_key(s, synth.S_X), (T, 4096), 1.0)
        x = bf16_tensor(xb, gpu)
        y_graph = st.replay(x).clone()
        torch.cuda.synchronize()
        y_eager = st.step(x).clone()
        torch.cuda.synchronize()
        assert torch.equal(y_graph, y_eager), f"replay {s}"
        assert torch.isfinite(y_graph.float()).all()


def test_stage_fused_norms_equal_unfused(gpu):
    """The stage with every norm fused (attn_norm and q_norm in the projection
    pairs, ffn_norm in the MoE layer's routing launch) gives the unfused stage's
    bits (rms_norm_quant / rms_norm launches, then the layers), two V4 blocks at
    T = 4, three inputs."""
    cfg = MoEConfig(4096, 2048, 256, 6, "sqrtsoftplus", 1.5, 10.0, N.WZ_SCALE_UE8M0, N.WZ_WSCALE_E8M0)
    T = 4
    blocks = []
    for l in range(2):
        w, _ = synth.synthetic_moe(cfg, seed=0, layer=l, device=gpu)
        blocks.append(stage.synthetic_block(HipMoE(cfg, w, max_tokens=T), 4096, seed=l, device=gpu))
    fused, plain = stage.DecodeStage(blocks, T), stage.DecodeStage(blocks, T, fused_norms=False)
    assert fused.fused_norms and not plain.fused_norms
    for s in range(3):
        x = bf16_tensor(synth.normal_bf16(synth.stream_key(40 + s, synth.S_X), (T, 4096), 1.0), gpu)
        y0 = fused.step(x).clone()
        y1 = plain.step(x).clone()
        torch.cuda.synchronize()
        assert torch.equal(y0, y1), f"input {s}"

