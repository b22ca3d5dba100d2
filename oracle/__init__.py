"""ORACLE — test infrastructure, not product.

A CPU restatement (numpy) of the reference's MoE + FP8-linear path, used only
by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
as the checker.  The product package ``wanferenz_amd`` never imports it.

Modules:
  numerics  number-format codecs (e4m3fn, e2m1, e8m0, bf16) from their definitions
  moe       act_quant, fp8_gemm, fp4_gemm, gate, permutation, expert, moe_forward, rmsnorm,
            wire_pack / wire_unpack (the FP8 stage-boundary format), sparse_attn

The reference's own path (wanferenz/kernels/torch_ops.py + the hot subset of
wanferenz/model/architecture.py) is Python, so there is no C/C++ reference to
compile into ``oracle/_ref``.
"""
