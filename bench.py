"""Benchmark: DeepSeek-V4-Flash-shape MoE layer, decode, on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--T 4] [--layers 12] [--no-cpu]

A step is one MoE layer forward (gate + top-6 routing + permute + MXFP4 routed
experts + FP8 shared expert + combine) over T synthetic tokens.  Steps rotate
over ``--layers`` independent layers (12 x 3.45 GB of expert banks resident in
HBM) with a different input per layer, so the 256 MB Infinity Cache cannot
serve repeated expert reads.  The layers are captured in rotation order as
one HIP graph, as a decode step captures its layers (no graph-launch gap
between layers); K steps replay it K // L times, then a graph of the first
K % L layers.

Printed JSON line (one):
  value       algorithmic HBM GB/s of the layer = sum over steps of
              (U*13,369,344 + 25,167,360 + 2,098,176 + 4*T*D) bytes / time,
              U = distinct experts the step's routing selected
  ms_per_step layer latency (µs/layer = 1000 * ms_per_step)
  roofline    the dominant kernel (w13: routed w1/w3 + shared w1/w3 + SwiGLU),
              algorithmic bytes per launch / its mean launch duration, measured
              live: the stage replayed alone for all layers from a captured
              graph, HIP events on the replay stream (stage_times)
  stage_us    the same per-launch measurement for every stage of the layer
  fp8_gemv    the FP8 linear at the dense projection shapes (packed and row-major)
  grouped_fp4 the grouped MXFP4 GEMM of the banked decode path (6 experts' w1|w3, w2)
  sparse_attn sparse attention at 64 heads of 512, topk 640: decode B = 1, 4, 8
              (µs, gathered-row GB/s) and prefill S = 512, 2048 (bf16 MFMA
              utilisation)
  decode_stage 12 V4 blocks (fused norms, the five FP8 attention-side projections,
              residuals, MoE) in one graph per step
  prefill_detail  the layer at T = 128, 512, 2048 with the calibrated Zipf(1.1)
              gate bias (beta in wanferenz_amd/zipf_v4.json; the fitted exponent
              of each batch's routing is reported): µs/layer, tokens/s,
              algorithmic HBM GB/s, and MFMA utilisation = 6*D*I*(T*k + T) flops /
              time against the dense FP8 (5.0 PFLOP/s, the rate of an e4m3 x e2m1
              scaled MFMA) and FP4 (10.1 PFLOP/s) peaks
  prefill_hot_experts  T = 2048 with every token on experts 0..5 (2048 rows
              each): the w13 / w2 launches' MFMA rate on full tiles
  fp4_gemm_m2048  one expert's w1|w3 and w2 GEMMs alone at M = 2048
  per_T_stage_us  the per-launch stage times of the decode sweep
The last three keys hold the whole metric in scalars:
  cpu_baseline the torch float32 restatement of the reference CPU path
              (oracle/torch_ref.py) on layer 0 at T tokens, all cores (<= 16) and
              one core on the same tokens, median of 6 after 2 warm-ups, CPU
              model, the HIP layer's agreement on the same tokens, near-tie tokens
  prefill     the prefill half flat: T = 2048 µs/layer, HBM fraction and MFMA
              rate, T = 128 / 512, the hot-expert tiles, the M = 2048 GEMMs and the
              committed MFMA-busy counters
  per_T       the decode layer at T = 1, 2, 4, 8 (µs/layer, HBM fraction)
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MoE layer µs + HBM GB/s (decode T=1-8); FP4 MFMA util (prefill T=2048)"
HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5000.0
FP4_PEAK_TFLOPS = 10100.0
BF16_PEAK_TFLOPS = 2500.0
D, I, E, K_TOP = 4096, 2048, 256, 6
ROUTED_EXPERT_BYTES = 3 * (I * D // 2) + 3 * (I * D // 32)          # 13,369,344
SHARED_BYTES = 3 * I * D + 3 * (I // 128) * (D // 128)              # 25,167,360
GATE_BYTES = E * D * 2 + E * 4                                       # 2,098,176
W13_ROUTED_BYTES = 2 * (I * D // 2) + 2 * (I * D // 32)             # 8,912,896


def committed_traffic(T: int):
    """HBM bytes per launch of the w13 stage at this T from the committed rocprofv3 counter
    summary (FETCH_SIZE + WRITE_SIZE, copy-calibrated), or None when none was recorded."""
    import re

    path = os.path.join(ROOT, "profiles", "hbm_traffic_pmc.md")
    if not os.path.exists(path):
        return None
    m = re.search(rf"traffic_bytes_per_launch w13 decode T={T} = (\d+)", open(path).read())
    return int(m.group(1)) if m else None


def layer_bytes(U: int, T: int) -> int:
    return U * ROUTED_EXPERT_BYTES + SHARED_BYTES + GATE_BYTES + 4 * T * D


def w13_bytes(U: int, T: int) -> int:
    # the w13 launch streams the routed experts' w1|w3 (the shared expert's run in the
    # route launch): weights + the quantized x read (e4m3 + fp32 scales) + h written
    # (bf16, one row per routed (token, expert) pair)
    return U * W13_ROUTED_BYTES + T * D + 4 * T * (D // 128) + 2 * T * K_TOP * I


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=240)
    ap.add_argument("--warmup", type=int, default=24)
    ap.add_argument("--T", type=int, default=4)
    ap.add_argument("--layers", type=int, default=12)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-stage", action="store_true",
                    help="skip the decode stage (MoE + FP8 projections + norms, one graph per step)")
    ap.add_argument("--no-gemv", action="store_true",
                    help="skip the FP8 linear (dense projection shapes) measurement")
    ap.add_argument("--no-attn", action="store_true",
                    help="skip the sparse attention measurement")
    ap.add_argument("--prefill", default="128,512,2048",
                    help="comma-separated prefill T values ('' to skip)")
    ap.add_argument("--prefill-layers", type=int, default=3)
    ap.add_argument("--prefill-legs", default="zipf,hot,gemm",
                    help="prefill legs to run: zipf (calibrated skew), hot (every token on experts "
                         "0..5), gemm (one expert's GEMMs alone at M = 2048)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 1 GiB device-to-device copy 5 times (the reference kernel of "
                         "known traffic for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE) and exit")
    return ap.parse_args()


def build_layers(n_layers, dev, tmax):
    from wanferenz_amd import _native as N
    from wanferenz_amd import synth
    from wanferenz_amd.moe import HipMoE, MoEConfig

    cfg = MoEConfig(D, I, E, K_TOP, "sqrtsoftplus", 1.5, 10.0, N.WZ_SCALE_UE8M0, N.WZ_WSCALE_E8M0)
    layers = []
    for l in range(n_layers):
        w, host = synth.synthetic_moe(cfg, seed=0, layer=l, device=dev)
        layers.append((HipMoE(cfg, w, max_tokens=tmax), host))
    return cfg, layers


def make_inputs(n_layers, T, dev, salt=0):
    import torch

    from wanferenz_amd import synth

    xs = []
    for l in range(n_layers):
        bits = synth.normal_bf16(synth.stream_key(1000 + salt, synth.layer_stream(l, synth.S_X)), (T, D), 1.0)
        xs.append((bits, torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).to(dev)))
    return xs


def distinct_experts(layers, xs):
    import torch

    Us = []
    for (moe, _), (_, x) in zip(layers, xs):
        _, idx, _, _, _ = moe.route(x)
        torch.cuda.synchronize()
        Us.append(len(set(idx.cpu().numpy().ravel().tolist())))
    return Us


def capture(layers, xs, steps):
    """One graph of every layer in rotation order (as a decode step captures
    its layers: no graph-launch gap between layers), plus a graph of the first
    steps % L layers, so that exactly `steps` layer forwards can be timed."""
    import torch

    outs = []
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for (moe, _), (_, x) in zip(layers, xs):
            out = torch.empty_like(x)
            for _ in range(2):
                moe.forward(x, out=out)
            outs.append(out)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()

    def graph_of(n):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for (moe, _), (_, x), out in list(zip(layers, xs, outs))[:n]:
                moe.forward(x, out=out)
        return g

    L = len(layers)
    full = graph_of(L)
    tail = graph_of(steps % L) if steps % L else None
    torch.cuda.synchronize()
    return (full, tail), outs


def time_steps(graphs, steps, warmup, L):
    """Seconds for exactly `steps` layer forwards in rotation order
    (steps // L replays of the all-layer graph, then the tail graph)."""
    import torch

    full, tail = graphs
    for _ in range(-(-warmup // L)):
        full.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps // L):
        full.replay()
    if tail is not None:
        tail.replay()
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return start.elapsed_time(end) / 1000.0, wall


STAGES = (("route", 0), ("w13", 1), ("hquant", 2), ("w2", 3), ("combine", 4))  # WZ_STAGE_*


def stage_times(layers, xs, outs, reps=20):
    """Mean µs per launch of each stage of the layer.

    Each stage alone (wz_moe_replay_stage: the same kernels on the state the
    last forward left in the workspace) that launches anything is captured for all layers into one
    graph, so its launches run back to back with no launch gaps and no event
    packets between kernels; HIP events on the replay stream bracket ``reps``
    replays.  Rotating over all layers keeps the weights out of the caches as
    in the timed run.
    """
    import torch

    from wanferenz_amd import _native as N

    T = xs[0][1].size(0)
    res = {}
    lib = N.lib()
    for name, st in STAGES:
        # a stage that launches nothing on this path (hquant and combine when w2
        # quantises and combines itself) has no time of its own
        lib.wz_prof_begin(64)
        layers[0][0].replay_stage(xs[0][1], st, outs[0])
        n_launch = lib.wz_prof_end()
        if n_launch <= 0:
            continue
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for (moe, _), (_, x), out in zip(layers, xs, outs):
                moe.replay_stage(x, st, out)
        g.replay()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            g.replay()
        end.record()
        torch.cuda.synchronize()
        res[name] = start.elapsed_time(end) * 1000.0 / (reps * len(layers))
        del g
    return res


def measure_T(layers, T, steps, warmup, dev, salt):
    xs = make_inputs(len(layers), T, dev, salt)
    Us = distinct_experts(layers, xs)
    graphs, outs = capture(layers, xs, steps)
    L = len(layers)
    secs, wall = time_steps(graphs, steps, warmup, L)
    total_bytes = sum(layer_bytes(Us[i % L], T) for i in range(steps))
    kt = stage_times(layers, xs, outs)
    return dict(T=T, secs=secs, wall=wall, Us=Us, total_bytes=total_bytes, kernels=kt, xs=xs)


# (N, K): the cfg-3 projection widths, then the V4 attention projections wkv, wq_b,
# wo_b and the indexer's wq_b (fp8_vector.py:505-510; wq_a is 1024 x 4096)
GEMV_SHAPES = ((4096, 1024), (1024, 4096), (4096, 4096), (16384, 4096), (512, 4096), (32768, 1024), (4096, 8192),
               (8192, 1024))
GEMV_TS = (1, 4, 8, 16, 32, 128)
GEMV_ROTATE_BYTES = 640 << 20   # weight copies per shape: more than the 256 MB Infinity Cache


def graph_timed(launches, reps):
    """Mean µs of one replay of a graph holding ``launches()`` (warmed eagerly on a
    side stream, captured, replayed once), HIP events around ``reps`` replays."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        launches()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        launches()
    g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1000.0 / reps


def gemv_bytes(N: int, K: int, T: int) -> int:
    # e4m3 weight + fp32 128x128 block scales + bf16 x read + bf16 y written
    return N * K + 4 * ((N + 127) // 128) * ((K + 127) // 128) + 2 * T * K + 2 * T * N


def measure_gemv(dev, reps=5):
    """FP8 block-scaled linear (act_quant fused) at the dense-projection shapes.

    Weights: e4m3 codes with NaN codes replaced, fp32 128x128 block scales
    U[0.5, 1.5) (the probe recipe of fp8_vector.py:185-232); per-token ue8m0
    activation quantisation.  "packed": the weight relaid once into MFMA tiles
    (kernels.PackedFp8Linear: GEMV at T <= 16, act_quant + tile GEMM above);
    "rowmajor": the reference layout as fp8_gemm receives it (wz_fp8_linear).
    Each shape rotates over enough weight copies (>= 640 MB) that every launch
    streams its weight from HBM; one graph holds one launch per copy, HIP
    events bracket ``reps`` replays.
    """
    import torch

    from wanferenz_amd import _native as N
    from wanferenz_amd import kernels, synth

    res = {}
    for Nn, K in GEMV_SHAPES:
        R = max(2, -(-GEMV_ROTATE_BYTES // (Nn * K)))
        pool = torch.empty(R, Nn, K, dtype=torch.uint8, device=dev)
        synth.device_fill(pool, synth.stream_key(0, synth.S_FP8_W), synth.FILL_E4M3)
        sc = torch.empty(R, (Nn + 127) // 128, (K + 127) // 128, dtype=torch.float32, device=dev)
        synth.device_fill(sc, synth.stream_key(0, synth.S_FP8_W_S), synth.FILL_F32_UNIFORM, 0.5, 1.5)
        lins = [kernels.PackedFp8Linear(pool[r].view(torch.float8_e4m3fn), sc[r], "ue8m0") for r in range(R)]
        entry = {"weight_copies": R}
        for layout in ("packed", "rowmajor"):
            row = {}
            for T in GEMV_TS:
                xb = synth.normal_bf16(synth.stream_key(T, synth.S_FP8_X), (T, K), 1.0)
                x = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).to(dev)
                y = torch.empty(T, Nn, dtype=torch.bfloat16, device=dev)
                if layout == "packed":
                    for lin in lins:
                        lin.reserve(T)

                    def launches():
                        for lin in lins:
                            lin(x, out=y)
                else:
                    def launches():
                        st = N.stream_handle(dev)
                        for r in range(R):
                            N.call("wz_fp8_linear", N.ptr(x), N.ptr(pool[r]), N.ptr(sc[r]), N.ptr(y), T, Nn, K,
                                   N.WZ_SCALE_UE8M0_F32, N.WZ_WSCALE_F32, st)
                us = graph_timed(launches, reps) / R
                gbs = gemv_bytes(Nn, K, T) / (us * 1e-6) / 1e9
                row[str(T)] = {"us": round(us, 2), "GB_s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                               "TFLOP_s": round(2.0 * T * Nn * K / (us * 1e-6) / 1e12, 2)}
            entry[layout] = row
        res[f"{Nn}x{K}"] = entry
        del pool, sc, lins
        torch.cuda.empty_cache()
    return res


def measure_grouped_fp4(dev, reps=10):
    """grouped_fp4_gemm at the banked decode shapes (fp4_grouped.py:297, 312):
    G = 6 experts' w1|w3 (N = 2I, K = D) and w2 (N = D, K = I), one e4m3 row each,
    rotating over >= 640 MB of weight copies.  Bytes: the G weight slices with
    their e8m0 scales + the rows in and out."""
    import torch

    from wanferenz_amd import _native as N
    from wanferenz_amd import synth

    res = {}
    G = K_TOP
    for name, Nn, K in (("w13", 2 * I, D), ("w2", D, I)):
        per = G * (Nn * K // 2 + Nn * K // 32)
        R = max(2, -(-GEMV_ROTATE_BYTES // per))
        w = torch.empty(R, G, Nn, K // 2, dtype=torch.uint8, device=dev)
        synth.device_fill(w, synth.stream_key(1, synth.S_W13), synth.FILL_U8)
        ws = torch.full((R, G, Nn, K // 32), 121, dtype=torch.uint8, device=dev)
        a = torch.full((G, K), 0x38, dtype=torch.uint8, device=dev)  # e4m3 1.0
        a_s = torch.ones(G, K // 128, dtype=torch.float32, device=dev)
        c = torch.empty(G, Nn, dtype=torch.bfloat16, device=dev)

        def launches():
            st = N.stream_handle(dev)
            for r in range(R):
                N.call("wz_grouped_fp4_gemm", N.ptr(a), N.ptr(a_s), N.ptr(w[r]), N.ptr(ws[r]), N.ptr(c), G, Nn, K,
                       N.WZ_SCALE_F32, st)

        us = graph_timed(launches, reps) / R
        byts = per + G * K + 4 * G * (K // 128) + 2 * G * Nn
        res[name] = {"G": G, "N": Nn, "K": K, "us": round(us, 2), "GB_s": round(byts / (us * 1e-6) / 1e9, 1),
                     "hbm_frac": round(byts / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        del w, ws
        torch.cuda.empty_cache()
    return res


def stage_proj_bytes(T: int) -> int:
    """FP8 projection bytes of one V4 stage block (wq_a, wkv, wq_b, indexer wq_b, wo_b):
    e4m3 weights + e8m0 128x128 scales + the activations in (e4m3 for the four fed by a
    fused norm, bf16 for wo_b) and out (bf16), + wo_b's residual read."""
    from wanferenz_amd import stage

    tot = 0
    shapes = stage.projection_shapes(D, **stage.V4_DIMS)
    for j, (Nn, K) in enumerate(shapes):
        a_in = (2 if j == len(shapes) - 1 else 1) * T * K + (T * K // 128)
        tot += Nn * K + ((Nn + 127) // 128) * ((K + 127) // 128) + a_in + 2 * T * Nn
    return tot + 2 * T * D


def measure_stage(layers, dev, T=4, steps=256, warmup=16):
    """The decode stage: every MoE layer as one V4 block with the five FP8 projections
    of its attention side, fused norms and residual adds, one hipGraph per step
    (wanferenz_amd/stage.py).

    A fresh x ~ N(0, 1) per step (seed = step), staged into the graph's input
    buffer by a device copy inside the timed region.  Bytes per step: each
    block's projections + its MoE layer with the distinct experts U_b of that
    block's routing, counted on eager steps over the same inputs.
    """
    import torch

    from wanferenz_amd import stage, synth

    blocks = [stage.synthetic_block(moe, D, seed=100 + l, device=dev) for l, (moe, _) in enumerate(layers)]
    st = stage.DecodeStage(blocks, T)
    xs = np.stack([synth.normal_bf16(synth.stream_key(s, synth.S_X), (T, D), 1.0) for s in range(steps)])
    xg = torch.from_numpy(xs.view(np.int16)).view(torch.bfloat16).to(dev)
    # routing of every block on a sample of the steps' inputs (eager, outside the timing)
    rts = [(torch.empty(T, K_TOP, dtype=torch.float32, device=dev),
            torch.empty(T, K_TOP, dtype=torch.int64, device=dev)) for _ in blocks]
    Us = []
    for s in range(0, steps, max(1, steps // 16)):
        st.step(xg[s], routing=rts)
        torch.cuda.synchronize()
        Us.append([len(set(ri.cpu().numpy().ravel().tolist())) for _, ri in rts])
    U_mean = float(np.mean(Us))
    st.capture()
    for s in range(warmup):
        st.replay(xg[s % steps])
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for s in range(steps):
        st.replay(xg[s])
    end.record()
    torch.cuda.synchronize()
    secs = start.elapsed_time(end) / 1000.0
    nb = len(blocks)
    step_bytes = nb * (stage_proj_bytes(T) + layer_bytes(1, T)) + (U_mean - 1) * nb * ROUTED_EXPERT_BYTES
    us = secs / steps * 1e6
    gbs = step_bytes / (us * 1e-6) / 1e9
    del st, blocks
    torch.cuda.empty_cache()
    dims = stage.V4_DIMS
    return {"workload": f"decode stage: {nb} V4 blocks x (add + RMSNorm + act_quant, FP8 wq_a "
                        f"{dims['q_lora']}x{D} with wkv {dims['head_dim']}x{D} in one launch, q_norm + act_quant, "
                        f"wq_b {dims['q_width']}x{dims['q_lora']} with indexer wq_b "
                        f"{dims['idx_width']}x{dims['q_lora']} in one launch, "
                        f"wo_b {D}x{dims['idx_width']} with the residual in its epilogue, RMSNorm, MoE layer), "
                        f"T={T}, one hipGraph per step, fresh x per step",
            "T": T, "blocks": nb, "steps": steps, "us_per_step": round(us, 1),
            "us_per_block": round(us / nb, 2), "tokens_per_s": round(T * steps / secs, 1),
            "mean_distinct_experts": round(U_mean, 2), "bytes_per_step": int(step_bytes),
            "GB_s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}


ATTN_H, ATTN_D, ATTN_TOPK, ATTN_WIN = 64, 512, 640, 128
ATTN_CACHE = ATTN_WIN + 65536 // 4   # window + compressed rows of a 64K context at ratio 4


def measure_attn(dev, reps=10):
    """sparse_attn at the V4-Flash attention shape: 64 heads of 512, 640 gathered
    rows per query (the 128-row window + 512 selected compressed rows).

    decode: B sequences x 1 query over a cache of 128 + 16384 rows; the window
    indices are the 128 window rows, the selected ones 512 distinct random rows
    of the compressed part.  Enough (kv, index) copies rotate that their caches
    total >= 640 MB.  Algorithmic bytes per query: the 640 gathered rows + q + o
    + the indices.  prefill: one sequence of S queries over S + S/4 rows, every
    query with 640 valid random indices (no causal -1 entries: the full work).
    FLOPs per query: 4 * H * D * topk (S = QK^T and O = PV).
    """
    import torch

    from wanferenz_amd import _native as N
    from wanferenz_amd import kernels

    g = torch.Generator().manual_seed(7)
    H, Dh, K, W = ATTN_H, ATTN_D, ATTN_TOPK, ATTN_WIN

    def case(B, S, n, R, prefill):
        q = (torch.randn(B, S, H, Dh, generator=g) * 0.5).to(torch.bfloat16).to(dev)
        sink = torch.randn(H, generator=g).to(dev)
        o = torch.empty_like(q)
        kvs, idxs = [], []
        for _ in range(R):
            kvs.append((torch.randn(B, n, Dh, generator=g)).to(torch.bfloat16).to(dev))
            if prefill:
                ix = torch.stack([torch.randperm(n, generator=g)[:K] for _ in range(B * S)])
            else:
                ix = torch.stack([torch.cat([torch.arange(W), W + torch.randperm(n - W, generator=g)[:K - W]])
                                  for _ in range(B * S)])
            idxs.append(ix.view(B, S, K).to(torch.int32).to(dev))

        wsb = kernels.sparse_attn_workspace_bytes(B, S, H, Dh, K)
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)

        def launches():
            st = N.stream_handle(dev)
            for kv, ix in zip(kvs, idxs):
                N.call("wz_sparse_attn", N.ptr(q), N.ptr(kv), N.ptr(sink), N.ptr(ix), N.ptr(o), B, S, H, Dh, n, K,
                       Dh ** -0.5, N.ptr(ws) if wsb else None, wsb, st)

        us = graph_timed(launches, reps) / R
        nq = B * S
        byts = (n * B * Dh * 2 if prefill else nq * K * Dh * 2) + nq * (4 * H * Dh + 4 * K)
        fl = 4.0 * H * Dh * K * nq
        return {"us": round(us, 2), "workgroups_per_query": max(1, wsb // max(1, B * S * (H // 64) * (128 + 64 * Dh) * 4)),
                "GB_s": round(byts / (us * 1e-6) / 1e9, 1),
                "hbm_frac": round(byts / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                "TFLOP_s": round(fl / (us * 1e-6) / 1e12, 2),
                "mfma_frac_bf16": round(fl / (us * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, 4)}

    res = {"shape": f"H={H} D={Dh} topk={K} (window {W} + {K - W} selected)"}
    for B in (1, 4, 8):
        per = B * ATTN_CACHE * Dh * 2
        res[f"decode_B{B}"] = case(B, 1, ATTN_CACHE, max(2, -(-GEMV_ROTATE_BYTES // per)), False)
    for S in (512, 2048):
        res[f"prefill_S{S}"] = case(1, S, S + S // 4, 2, True)
    torch.cuda.empty_cache()
    return res


def prefill_flops(T: int) -> float:
    return 6.0 * D * I * (T * K_TOP + T)


def measure_prefill(layers, Ts, dev):
    """Prefill T-token layers with the calibrated Zipf(1.1) gate bias (beta from
    wanferenz_amd/zipf_v4.json) over the first layers' banks."""
    import torch

    from wanferenz_amd import synth

    beta = synth.zipf_v4_beta()
    zb = torch.from_numpy(synth.zipf_bias(E, 1.1, beta)).to(dev)
    tmax = max(Ts)
    players = [(moe.with_gate_bias(zb, max_tokens=tmax), host) for moe, host in layers]
    res = {}
    for T in Ts:
        xs = make_inputs(len(players), T, dev, salt=5000 + T)
        loads = []
        for (moe, _), (_, x) in zip(players, xs):
            _, idx, _, _, _ = moe.route(x)
            torch.cuda.synchronize()
            loads.append(np.bincount(idx.cpu().numpy().ravel(), minlength=E))
        steps = max(6, min(60, 24576 // T))
        graphs, outs = capture(players, xs, steps)
        secs, _ = time_steps(graphs, steps, max(2, steps // 4), len(players))
        kt = stage_times(players, xs, outs, reps=max(2, steps // 3))
        L = len(players)
        nbytes = sum(layer_bytes(int((loads[i % L] > 0).sum()), T) for i in range(steps))
        us = secs / steps * 1e6
        tflops = prefill_flops(T) / (us * 1e-6) / 1e12
        res[str(T)] = {"us_per_layer": round(us, 1), "tokens_per_s": round(T / (us * 1e-6), 1),
                       "GB_s": round(nbytes / secs / 1e9, 1),
                       "hbm_frac": round(nbytes / secs / 1e9 / HBM_PEAK_GBS, 4),
                       "TFLOP_s": round(tflops, 1),
                       "mfma_frac_fp8": round(tflops / FP8_PEAK_TFLOPS, 4),
                       "mfma_frac_fp4": round(tflops / FP4_PEAK_TFLOPS, 4),
                       "max_expert_rows": int(max(l.max() for l in loads)),
                       "zipf_beta": round(beta, 6),
                       "zipf_exponent": round(float(np.mean([synth.zipf_exponent(l) for l in loads])), 3),
                       "mean_active_experts": round(float(np.mean([(l > 0).sum() for l in loads])), 1),
                       "steps": steps,
                       "stage_us": {k: round(v, 2) for k, v in kt.items()}}
    return res


def measure_hot_experts(layers, dev, T=2048):
    """Hot-expert tiles: the prefill layer at T tokens with a gate bias that sends
    every token to experts 0..5, so each of the six holds T rows (the M = 2048
    expert of a skewed batch) and every w1/w3 and w2 tile is full.  MFMA rate of
    the w13 and w2 launches = 2 * rows * N * K flops (routed rows T*k, plus the T
    shared-expert rows) / the launch's mean duration (stage replay)."""
    import torch

    bias = torch.zeros(E, dtype=torch.float32, device=dev)
    bias[:K_TOP] = 100.0
    players = [(moe.with_gate_bias(bias, max_tokens=T), host) for moe, host in layers]
    xs = make_inputs(len(players), T, dev, salt=7000)
    steps = max(6, min(60, 24576 // T))
    graphs, outs = capture(players, xs, steps)
    secs, _ = time_steps(graphs, steps, max(2, steps // 4), len(players))
    kt = stage_times(players, xs, outs, reps=max(2, steps // 3))
    rows = T * K_TOP + T
    res = {"T": T, "rows_per_expert": T, "us_per_layer": round(secs / steps * 1e6, 1),
           "stage_us": {k: round(v, 2) for k, v in kt.items()}}
    for st, flops in (("w13", 2.0 * rows * (2 * I) * D), ("w2", 2.0 * rows * D * I)):
        tf = flops / (kt[st] * 1e-6) / 1e12
        res[st] = {"TFLOP_s": round(tf, 1), "mfma_frac_fp8_rate": round(tf / FP8_PEAK_TFLOPS, 4),
                   "mfma_frac_fp4_peak": round(tf / FP4_PEAK_TFLOPS, 4)}
    return res


def measure_fp4_gemm_2048(dev, reps=10):
    """One expert's GEMMs alone at M = 2048 rows (e4m3 activations with ue8m0 block
    scales x MXFP4 weights): w1|w3 (N = 2I, K = D) and w2 (N = D, K = I), through the
    packed-weight tile GEMM (wz_fp4_gemm_packed, the weight relaid once by
    wz_fp4_pack) and through the row-major wz_fp4_gemm.  Two weight copies
    alternate; flops = 2 M N K; rate against the e4m3 x e2m1 scaled-MFMA rate (the
    FP8 rate, 5.0 PFLOP/s) and the FP4 peak."""
    import torch

    from wanferenz_amd import kernels, synth

    M = 2048
    res = {}
    for name, Nn, K in (("w13", 2 * I, D), ("w2", D, I)):
        xb = synth.normal_bf16(synth.stream_key(M + K, synth.S_FP8_X), (M, K), 1.0)
        x = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).to(dev)
        q, qs = kernels.act_quant(x, 128, "ue8m0", torch.float8_e8m0fnu)
        ws = []
        for r in range(2):
            w = torch.empty(Nn, K // 2, dtype=torch.uint8, device=dev)
            synth.device_fill(w, synth.stream_key(r, synth.S_W13), synth.FILL_U8)
            s = torch.empty(Nn, K // 32, dtype=torch.uint8, device=dev)
            synth.device_fill(s, synth.stream_key(r, synth.S_W13_S), synth.FILL_E8M0, 118, 122)
            ws.append((w.view(torch.float4_e2m1fn_x2), s.view(torch.float8_e8m0fnu)))
        packed = [kernels.PackedFp4Linear(w, s).reserve(M, torch.float8_e8m0fnu) for w, s in ws]
        out = torch.empty(M, Nn, dtype=torch.bfloat16, device=dev)

        def launches_packed():
            for lin in packed:
                lin.gemm(q, qs, out=out)

        def launches_rowmajor():
            for w, s in ws:
                kernels.fp4_gemm(q, qs, w, s, torch.float8_e8m0fnu)

        entry = {"M": M, "N": Nn, "K": K}
        for tag, fn in (("packed", launches_packed), ("rowmajor", launches_rowmajor)):
            us = graph_timed(fn, reps) / len(ws)
            tf = 2.0 * M * Nn * K / (us * 1e-6) / 1e12
            entry[tag] = {"us": round(us, 2), "TFLOP_s": round(tf, 1),
                          "mfma_frac_fp8_rate": round(tf / FP8_PEAK_TFLOPS, 4),
                          "mfma_frac_fp4_peak": round(tf / FP4_PEAK_TFLOPS, 4)}
        res[name] = entry
    return res


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def _torch_layer(moe, used):
    """The layer's touched routed experts and its shared expert, copied to host
    memory in the checkpoint's formats, for the torch restatement."""
    import torch

    from oracle import torch_ref as tr

    w = moe.weights

    def e8m0(t):
        return torch.ldexp(torch.ones(t.shape), t.cpu().to(torch.int32).float() - 127.0)

    experts = {}
    for e in used:
        w13, s13 = w.w13[e].cpu(), e8m0(w.w13_s[e])
        experts[e] = (tr.QLinear("fp4", w13[:I], s13[:I]), tr.QLinear("fp4", w13[I:], s13[I:]),
                      tr.QLinear("fp4", w.w2[e].cpu(), e8m0(w.w2_s[e])))
    shared = tuple(tr.QLinear("fp8", a.cpu(), e8m0(b)) for a, b in
                   ((w.sh_w1, w.sh_w1_s), (w.sh_w3, w.sh_w3_s), (w.sh_w2, w.sh_w2_s)))
    return tr.MoELayer(w.gate_w.cpu(), w.gate_bias.cpu(), experts, shared, E, K_TOP,
                       "sqrtsoftplus", 1.5, 10.0, True)


def cpu_baseline(layers, cfg, T, dev):
    """The torch float32 restatement of the reference CPU path (oracle/torch_ref.py,
    op for op after torch_ops.py and architecture.py) on layer 0 of the benchmark,
    on the T-token step: all cores (at most 16, the box's CPU share) and one core
    (the reference's OMP_NUM_THREADS=1) on the same tokens; 2 warm-up runs, then
    the median of 6.  Each run dequantises the weights it multiplies, as the
    reference CPU path does.  The same inputs go through the HIP layer: expert
    indices must match, outputs within 1e-2 relative / 0.9999 cosine; near-tie
    tokens are listed.  The result is flat (scalars) first, the two legs after."""
    import torch

    from oracle import torch_ref as tr
    from wanferenz_amd import synth

    moe, _ = layers[0]
    n_all = max(1, min(16, len(os.sched_getaffinity(0))))
    legs = {}
    prev_threads, prev_dtype = torch.get_num_threads(), torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        bits = synth.normal_bf16(synth.stream_key(1000, synth.layer_stream(0, synth.S_X)), (T, D), 1.0)
        xc = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)
        _, idx_c, scores = tr.gate_forward(xc, moe.weights.gate_w.cpu(), moe.weights.gate_bias.cpu(), K_TOP,
                                           "sqrtsoftplus", 1.5)
        used = sorted(set(idx_c.flatten().tolist()))
        p = _torch_layer(moe, used)
        # the HIP layer on the same tokens
        out = torch.empty(T, D, dtype=torch.bfloat16, device=dev)
        moe.forward(xc.to(dev), out=out)
        _, idx_g, _, _, _ = moe.route(xc.to(dev))
        torch.cuda.synchronize()
        nbytes = layer_bytes(len(used), T)
        for leg, nt in (("all_cores", n_all), ("one_core", 1)):
            torch.set_num_threads(nt)
            times = []
            for i in range(8):
                t0 = time.perf_counter()
                y_c, _, idx_c = tr.moe_forward(p, xc)
                times.append(time.perf_counter() - t0)
            med = float(np.median(times[2:]))
            yg, yc = out.float().cpu().numpy(), y_c.float().numpy()
            legs[leg] = {"threads": nt, "us_per_layer": round(med * 1e6, 1), "tokens_per_s": round(T / med, 2),
                         "GB_s": round(nbytes / med / 1e9, 4), "runs": len(times) - 2, "warmup": 2,
                         "max_rel_err": round(float(np.abs(yg - yc).max() / max(np.abs(yc).max(), 1e-30)), 6),
                         "cosine": round(float((yg * yc).sum() / max(np.linalg.norm(yg) * np.linalg.norm(yc),
                                                                    1e-30)), 7),
                         "indices_match": bool(torch.equal(idx_g.cpu().long(), idx_c.long()))}
    finally:
        torch.set_num_threads(prev_threads)
        torch.set_default_dtype(prev_dtype)
    a, o = legs["all_cores"], legs["one_core"]
    return {"value": a["GB_s"], "unit": "GB/s", "cores": a["threads"], "kind": "port",
            "sample": f"one V4 MoE layer (layer 0 of the benchmark, T={T}, U={len(used)}) through the torch "
                      f"float32 restatement of the reference CPU path, {a['threads']} threads and 1 thread on "
                      f"the same tokens: median of 6 after 2 warm-ups each",
            "cpu_model": _cpu_model(), "T": T, "distinct_experts": len(used),
            "us_per_layer": a["us_per_layer"], "tokens_per_s": a["tokens_per_s"],
            "one_core_us_per_layer": o["us_per_layer"], "one_core_GB_s": o["GB_s"],
            "one_core_tokens_per_s": o["tokens_per_s"],
            "indices_match": a["indices_match"] and o["indices_match"],
            "max_rel_err": max(a["max_rel_err"], o["max_rel_err"]), "cosine": min(a["cosine"], o["cosine"]),
            "near_tie_tokens": len(tr.near_ties(scores, K_TOP)),
            "legs": legs}


def committed_mfma_busy():
    """MFMA busy (%) of the prefill w1/w3 and w2 launches at T = 2048 from the committed
    rocprofv3 counter summary: the calibrated Zipf batch, then the hot-expert batch."""
    import re

    path = os.path.join(ROOT, "profiles", "moe_prefill_T2048_mfma_pmc.md")
    if not os.path.exists(path):
        return {}
    rows = re.findall(r"^\| `(\w+)<([^>]*)>` \|(?:[^|]*\|){4} ([\d.]+) % \|", open(path).read(), re.M)
    if len(rows) < 4:
        return {}
    return {"counter_mfma_busy_w13_zipf": float(rows[0][2]), "counter_mfma_busy_w2_zipf": float(rows[1][2]),
            "counter_mfma_busy_w13_hot": float(rows[2][2]), "counter_mfma_busy_w2_hot": float(rows[3][2]),
            "counter_source": "profiles/moe_prefill_T2048_mfma_pmc.md (SQ_VALU_MFMA_BUSY_CYCLES)"}


def flat_prefill(detail, hot, gemm):
    """The prefill half of the metric as one flat block of scalars: T = 2048 with the
    calibrated skew (µs per layer, HBM fraction, MFMA rate), the other T, the hot-expert
    tiles, one expert's GEMMs at M = 2048, and the committed counter figures."""
    out = {}
    if "2048" in detail:
        d = detail["2048"]
        out.update({"T": 2048, "us_per_layer": d["us_per_layer"], "tokens_per_s": d["tokens_per_s"],
                    "GB_s": d["GB_s"], "hbm_frac": d["hbm_frac"], "TFLOP_s": d["TFLOP_s"],
                    "mfma_frac_fp4_peak": d["mfma_frac_fp4"], "mfma_frac_fp8_rate": d["mfma_frac_fp8"],
                    "zipf_exponent": d["zipf_exponent"], "max_expert_rows": d["max_expert_rows"]})
    for T, d in detail.items():
        if T != "2048":
            out[f"T{T}_us_per_layer"] = d["us_per_layer"]
            out[f"T{T}_hbm_frac"] = d["hbm_frac"]
    if hot:
        out["hot_us_per_layer"] = hot["us_per_layer"]
        for st in ("w13", "w2"):
            out[f"hot_{st}_TFLOP_s"] = hot[st]["TFLOP_s"]
            out[f"hot_{st}_mfma_frac_fp8_rate"] = hot[st]["mfma_frac_fp8_rate"]
            out[f"hot_{st}_mfma_frac_fp4_peak"] = hot[st]["mfma_frac_fp4_peak"]
    if gemm:
        for st in ("w13", "w2"):
            g = gemm[st]["packed"]
            out[f"m2048_{st}_us"] = g["us"]
            out[f"m2048_{st}_mfma_frac_fp8_rate"] = g["mfma_frac_fp8_rate"]
            out[f"m2048_{st}_mfma_frac_fp4_peak"] = g["mfma_frac_fp4_peak"]
    out.update(committed_mfma_busy())
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(no multi-GPU path is built)", file=sys.stderr)
        sys.exit(2)
    import torch

    from wanferenz_amd import _native

    if args.copy_calibration:
        src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        src.fill_(1)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": 1 << 30, "launches": 5}), flush=True)
        return
    _native.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg, layers = build_layers(args.layers, dev, 16)
    torch.cuda.synchronize()
    main_run = measure_T(layers, args.T, args.steps, args.warmup, dev, 0)
    secs, T = main_run["secs"], args.T
    value = main_run["total_bytes"] / secs / 1e9
    ms = secs / args.steps * 1000.0
    Umean = float(np.mean(main_run["Us"]))
    kt = main_run["kernels"]
    w13_us = kt["w13"]
    w13_b = float(np.mean([w13_bytes(u, T) for u in main_run["Us"]]))
    achieved = w13_b / (w13_us * 1e-6) / 1e9
    out = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "mxfp4(e2m1)*fp8(e4m3)->fp32", "data": "synthetic",
        "config": {"workload": f"DeepSeek-V4-Flash MoE layer decode, T={T} tokens: hidden 4096, "
                               f"256 routed MXFP4 experts + 1 FP8 shared, top-6, intermediate 2048; "
                               f"{args.layers} layers rotated in one hipGraph",
                   "T": T, "layers": args.layers, "mean_distinct_experts": Umean},
        "us_per_layer": round(ms * 1000.0, 2),
        "tokens_per_s": round(T * args.steps / secs, 1),
        "hbm_frac_layer": round(value / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "kernel": "moe_w13", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": committed_traffic(T),
                     "traffic_source": "profiles/hbm_traffic_pmc.md: rocprofv3 FETCH_SIZE + WRITE_SIZE "
                                       "per launch of the w13 kernel, copy-calibrated",
                     "bytes_per_launch": round(w13_b),
                     "mean_us": round(w13_us, 2)},
        "stage_us": {k: round(v, 2) for k, v in kt.items()},
    }
    sweep = {}
    if not args.no_sweep:
        for Ts in (1, 2, 4, 8):
            r = main_run if Ts == T else measure_T(layers, Ts, 120, 12, dev, Ts)
            v = r["total_bytes"] / r["secs"] / 1e9
            n = 120 if Ts != T else args.steps
            sweep[str(Ts)] = {"us_per_layer": round(r["secs"] / n * 1e6, 2), "GB_s": round(v, 1),
                              "hbm_frac": round(v / HBM_PEAK_GBS, 4),
                              "mean_U": round(float(np.mean(r["Us"])), 1),
                              "stage_us": {k: round(x, 2) for k, x in r["kernels"].items()}}
    detail, hot, gemm = {}, None, None
    if args.prefill:
        Ts = [int(t) for t in args.prefill.split(",") if t]
        legs = set(args.prefill_legs.split(","))
        if "zipf" in legs:
            detail = measure_prefill(layers[:max(1, args.prefill_layers)], Ts, dev)
        if "hot" in legs:
            hot = measure_hot_experts(layers[:max(1, args.prefill_layers)], dev)
        if "gemm" in legs:
            gemm = measure_fp4_gemm_2048(dev)
    if not args.no_gemv:
        out["fp8_gemv"] = measure_gemv(dev)
        out["grouped_fp4"] = measure_grouped_fp4(dev)
    if not args.no_attn:
        out["sparse_attn"] = measure_attn(dev)
    if not args.no_stage:
        out["decode_stage"] = measure_stage(layers, dev, T=args.T)
    if detail:
        out["prefill_detail"] = detail
    if hot:
        out["prefill_hot_experts"] = hot
    if gemm:
        out["fp4_gemm_m2048"] = gemm
    # the last keys of the line: the CPU baseline, the flat prefill block and the
    # decode sweep, so a reader of the line's tail finds the whole metric there
    if sweep:
        out["per_T_stage_us"] = {k: v["stage_us"] for k, v in sweep.items()}
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(layers, cfg, T, dev)
    if detail or hot or gemm:
        out["prefill"] = flat_prefill(detail, hot, gemm)
    if sweep:
        out["per_T"] = {k: {"us_per_layer": v["us_per_layer"], "hbm_frac": v["hbm_frac"], "GB_s": v["GB_s"],
                            "mean_U": v["mean_U"]} for k, v in sweep.items()}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
