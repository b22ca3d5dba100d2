"""Stand-in for the reference model module's MoE classes (test infrastructure only).

``wanferenz_amd.moe.install(mod)`` rebinds ``mod.MoE.forward`` on the
reference's loaded model module and reads the attributes its MoE / Gate /
Expert / Linear objects carry (wanferenz/model/architecture.py:137-180 for
Linear, :674-794 for Gate, Expert and MoE), plus the module globals
``world_size``, ``scale_fmt`` and ``scale_dtype``.  The reference cannot be
imported where the GPU tests run, so this module provides classes with the
same attribute names, parameter dtypes and shapes.  Their own ``forward``
computes nothing: ``MoE.forward`` counts the call and returns a sentinel, so a
test can tell the reference path (a decline) from the HIP path.
"""

from __future__ import annotations

import torch
from torch import nn

world_size, rank = 1, 0
scale_fmt, scale_dtype = "ue8m0", torch.float8_e8m0fnu
block_size, fp4_block_size = 128, 32
SENTINEL = 7.0


def _param(shape, dtype, device):
    return nn.Parameter(torch.zeros(shape, dtype=torch.uint8, device=device).view(dtype), requires_grad=False)


class Linear(nn.Module):
    def __init__(self, in_features, out_features, dtype, device="cpu"):
        super().__init__()
        self.in_features, self.out_features = in_features, out_features
        if dtype == torch.float4_e2m1fn_x2:
            self.weight = _param((out_features, in_features // 2), dtype, device)
            self.scale = _param((out_features, in_features // fp4_block_size), torch.float8_e8m0fnu, device)
        elif dtype == torch.float8_e4m3fn:
            self.weight = _param((out_features, in_features), dtype, device)
            nb = lambda n: (n + block_size - 1) // block_size  # noqa: E731
            self.scale = _param((nb(out_features), nb(in_features)), torch.float8_e8m0fnu, device)
        else:
            self.weight = nn.Parameter(torch.zeros(out_features, in_features, dtype=dtype, device=device),
                                       requires_grad=False)
            self.scale = None
        self.weight.scale = self.scale


class Expert(nn.Module):
    def __init__(self, dim, inter_dim, dtype, swiglu_limit=0.0, device="cpu"):
        super().__init__()
        self.w1 = Linear(dim, inter_dim, dtype, device)
        self.w2 = Linear(inter_dim, dim, dtype, device)
        self.w3 = Linear(dim, inter_dim, dtype, device)
        self.swiglu_limit = swiglu_limit


class Gate(nn.Module):
    def __init__(self, dim, n_experts, topk, score_func, route_scale, hash_layer, vocab, device="cpu"):
        super().__init__()
        self.dim, self.topk = dim, topk
        self.score_func, self.route_scale = score_func, route_scale
        self.hash = hash_layer
        self.weight = nn.Parameter(torch.zeros(n_experts, dim, dtype=torch.bfloat16, device=device),
                                   requires_grad=False)
        if hash_layer:
            self.tid2eid = nn.Parameter(torch.zeros(vocab, topk, dtype=torch.int32, device=device),
                                        requires_grad=False)
            self.bias = None
        else:
            self.bias = nn.Parameter(torch.zeros(n_experts, dtype=torch.float32, device=device),
                                     requires_grad=False)


class MoE(nn.Module):
    def __init__(self, layer_id, dim, inter, n_experts, topk, score_func="sqrtsoftplus", route_scale=1.0,
                 swiglu_limit=0.0, hash_layer=False, vocab=64, expert_dtype=torch.float4_e2m1fn_x2,
                 device="cpu"):
        super().__init__()
        self.layer_id, self.dim = layer_id, dim
        self.n_routed_experts = n_experts
        self.n_local_experts = n_experts // world_size
        self.n_activated_experts = topk
        self.experts_start_idx = rank * self.n_local_experts
        self.experts_end_idx = self.experts_start_idx + self.n_local_experts
        self.gate = Gate(dim, n_experts, topk, score_func, route_scale, hash_layer, vocab, device)
        self.experts = nn.ModuleList([Expert(dim, inter, expert_dtype, swiglu_limit, device)
                                      for _ in range(n_experts)])
        self.shared_experts = Expert(dim, inter, torch.float8_e4m3fn, swiglu_limit, device)
        self.ref_calls = 0

    def forward(self, x, input_ids):
        self.ref_calls += 1
        return torch.full_like(x, SENTINEL)


def moe_from_case(case, inp, device):
    """A mirror MoE holding the weights of a tests/golden/cases.py case."""
    moe = MoE(0, case.dim, case.inter, case.n_experts, case.topk, case.score_func, case.route_scale,
              case.swiglu_limit, case.hash_layer, case.vocab, device=device)

    def put(p, a):
        p.data.view(torch.uint8).copy_(torch.from_numpy(a).view(torch.uint8).reshape(p.shape))

    I, nb = case.inter, case.inter // 128
    g = moe.gate
    g.weight.data.copy_(torch.from_numpy(inp.gate_w.view("int16")).view(torch.bfloat16))
    if case.hash_layer:
        g.tid2eid.data.copy_(torch.from_numpy(inp.tid2eid))
    else:
        g.bias.data.copy_(torch.from_numpy(inp.gate_bias))
    for e, ex in enumerate(moe.experts):
        put(ex.w1.weight, inp.w13[e, :I])
        put(ex.w3.weight, inp.w13[e, I:])
        put(ex.w1.scale, inp.w13_s[e, :I])
        put(ex.w3.scale, inp.w13_s[e, I:])
        put(ex.w2.weight, inp.w2[e])
        put(ex.w2.scale, inp.w2_s[e])
    sh = moe.shared_experts
    put(sh.w1.weight, inp.sh_w13[:I])
    put(sh.w3.weight, inp.sh_w13[I:])
    put(sh.w1.scale, inp.sh_w13_s[:nb])
    put(sh.w3.scale, inp.sh_w13_s[nb:])
    put(sh.w2.weight, inp.sh_w2)
    put(sh.w2.scale, inp.sh_w2_s)
    return moe
