"""GPU parity of the decode stage (wanferenz_amd/stage.py): blocks of RMSNorm, FP8
projections, residual adds and the MoE layer, run eagerly and as one captured graph.

Bar: the stage output vs the oracle run of the same chain (every op restated in
oracle/, each fed the oracle's own previous output) within max|d|/max|ref| <= 1e-2
and cosine >= 0.9999 after two blocks; graph replays equal the eager step bit for bit.
"""

import numpy as np
import pytest
import torch

from oracle import moe as om
from oracle.numerics import bf16_round, e8m0_decode, from_bf16_bits
from tests.helpers import bf16_tensor, bytes8, f32_of_bf16
from tests.test_gpu_moe import _oracle_params_from_device
from wanferenz_amd import _native as N
from wanferenz_amd import stage, synth
from wanferenz_amd.moe import HipMoE, MoEConfig

pytestmark = pytest.mark.gpu

TOL_REL = 1e-2
TOL_COS = 0.9999


def _oracle_linear(x, n, k, seed):
    w, s = stage.synthetic_linear(n, k, seed, "cuda", fp32_scales=False)
    rq, rs = om.act_quant(x, 128, True)
    return om.fp8_gemm(rq, rs, bytes8(w), e8m0_decode(bytes8(s).reshape(s.shape)))


def _close(got, ref):
    return om.max_rel_err(got, ref), om.cosine(got, ref)


def test_stage_ops_match_oracle(gpu):
    """Two toy blocks (D 1024, 16 experts top-2, projections 256 / 1024 / 1024 / 2048
    wide): the GEMV path (K = 1024) and the quantise + tile GEMM path (K = 256) both
    run.  Every op of every block is checked against the oracle fed the stage's own
    input to that op, since each FP8 re-quantisation turns a one-ulp bf16 difference
    upstream into an e4m3 rounding flip (a 6 % step) downstream: the residual adds
    bit-exact, norms within one bf16 ulp, projections and the MoE to the bf16
    tolerance; the routing of each MoE is the oracle's on the stage's input."""
    cfg = MoEConfig(1024, 512, 16, 2, "sqrtsoftplus", 1.5, 10.0, N.WZ_SCALE_UE8M0, N.WZ_WSCALE_E8M0)
    T, D, q, wide = 4, 1024, 256, 2048
    layers = [synth.synthetic_moe(cfg, seed=0, layer=l, device=gpu) for l in range(2)]
    blocks = [stage.synthetic_block(HipMoE(cfg, w, max_tokens=T), D, q, wide, seed=l, device=gpu)
              for l, (w, _) in enumerate(layers)]
    st = stage.DecodeStage(blocks, T)
    xb = synth.normal_bf16(synth.stream_key(7, synth.S_X), (T, D), 1.0)
    trace = []
    rts = [(torch.empty(T, cfg.topk, dtype=torch.float32, device=gpu),
            torch.empty(T, cfg.topk, dtype=torch.int64, device=gpu)) for _ in blocks]
    st.step(bf16_tensor(xb, gpu), routing=rts, trace=trace)
    torch.cuda.synchronize()
    assert np.array_equal(f32_of_bf16(trace[0]["h_in"]), from_bf16_bits(xb).reshape(T, D))

    def one_ulp(got, ref):
        rel = np.abs(got - ref) / np.maximum(np.abs(ref), 1e-30)
        assert rel.max() <= 2.0 ** -7, rel.max()

    def close(name, got, ref):
        rel, cos = _close(got, ref)
        assert rel <= TOL_REL and cos >= TOL_COS, (name, rel, cos)

    for l, ((w, host), b, tr, (_, ri)) in enumerate(zip(layers, blocks, trace, rts)):
        g = {k: f32_of_bf16(v) for k, v in tr.items()}
        one_ulp(g["a"], om.rmsnorm(g["h_in"], b.attn_norm.cpu().numpy()))
        close("p_down", g["u"], _oracle_linear(g["a"], q, D, l * 16 + 0))
        close("p_up", g["v"], _oracle_linear(g["u"], D, q, l * 16 + 1))
        close("p_sq", g["w"], _oracle_linear(g["v"], D, D, l * 16 + 2))
        if l == len(blocks) - 1:
            close("p_wide", g["z"], _oracle_linear(g["a"], wide, D, l * 16 + 3))
        assert np.array_equal(g["h_mid"], bf16_round((g["h_in"] + g["w"]).astype(np.float32)))
        one_ulp(g["m"], om.rmsnorm(g["h_mid"], b.ffn_norm.cpu().numpy()))
        gate = om.gate(g["m"], from_bf16_bits(host["gate_w"]), host["gate_bias"], cfg.topk, cfg.score_func,
                       cfg.route_scale)
        assert np.array_equal(ri.cpu().numpy(), gate.indices)
        p = _oracle_params_from_device(cfg, w, host, sorted(set(gate.indices.ravel().tolist())))
        close("moe", g["e"], om.moe_forward(p, g["m"]).y)
        assert np.array_equal(g["h_out"], bf16_round((g["h_mid"] + g["e"]).astype(np.float32)))


def test_stage_graph_replays_equal_eager(gpu):
    """Two V4-shaped blocks (D 4096, 256 MXFP4 experts top-6, projections 1024 x 4096,
    4096 x 1024, 4096 x 4096, 16384 x 4096) at T = 4: every replay of the captured
    step equals an eager step on the same input, with eager work between replays."""
    cfg = MoEConfig(4096, 2048, 256, 6, "sqrtsoftplus", 1.5, 10.0, N.WZ_SCALE_UE8M0, N.WZ_WSCALE_E8M0)
    T = 4
    blocks = []
    for l in range(2):
        w, _ = synth.synthetic_moe(cfg, seed=0, layer=l, device=gpu)
        blocks.append(stage.synthetic_block(HipMoE(cfg, w, max_tokens=T), 4096, 1024, 16384, seed=l, device=gpu))
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
