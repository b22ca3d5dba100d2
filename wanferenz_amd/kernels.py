"""Drop-in kernel functions with the reference's signatures, running on the HIP library.

The reference model imports ``act_quant, fp4_act_quant, fp8_gemm, fp4_gemm,
sparse_attn, hc_split_sinkhorn`` from ``wanferenz.kernels.reference``
(wanferenz/model/architecture.py:12-19) and resolves them as module globals
at call time, so rebinding them on the loaded model module redirects every
FP8 / FP4 linear (the precedent is wanferenz/kernels/fp8_vector.py:476-485).
:func:`install` does that for the three functions on this path.

Signatures, argument meaning and error behaviour follow
wanferenz/kernels/reference.py:117-146 (act_quant), :292-311 (fp8_gemm) and
:572-591 (fp4_gemm): inputs must be contiguous (AssertionError otherwise),
outputs are new tensors in ``torch.get_default_dtype()`` (bf16 in the model).
"""

from __future__ import annotations

import torch

from . import _native as N

_E8M0 = torch.float8_e8m0fnu
_E4M3 = torch.float8_e4m3fn
_FP4X2 = torch.float4_e2m1fn_x2


def _act_kind(scale_fmt, scale_dtype) -> int:
    if scale_fmt is None:
        if scale_dtype != torch.float32:
            raise ValueError(
                "act_quant: scale_fmt=None gives non-power-of-two scales, which only a float32 "
                f"scale_dtype can hold (got {scale_dtype})"
            )
        return N.WZ_SCALE_F32
    return N.WZ_SCALE_UE8M0 if scale_dtype == _E8M0 else N.WZ_SCALE_UE8M0_F32


def _scale_kind_of(s: torch.Tensor) -> int:
    """Activation scale kind read off the scale tensor's dtype."""
    if s.dtype == _E8M0:
        return N.WZ_SCALE_UE8M0
    if s.dtype == torch.float32:
        return N.WZ_SCALE_F32
    raise TypeError(f"activation scales must be float32 or float8_e8m0fnu, got {s.dtype}")


def _wscale_kind_of(s: torch.Tensor) -> int:
    if s.dtype == _E8M0:
        return N.WZ_WSCALE_E8M0
    if s.dtype == torch.float32:
        return N.WZ_WSCALE_F32
    raise TypeError(f"weight scales must be float32 or float8_e8m0fnu, got {s.dtype}")


def _require_cuda(*ts):
    for t in ts:
        if not t.is_cuda:
            raise RuntimeError(
                "wanferenz_amd kernels run on the GPU only (got a CPU tensor); "
                "there is no CPU fallback in this package"
            )


def _finish(c: torch.Tensor) -> torch.Tensor:
    dt = torch.get_default_dtype()
    return c if dt == torch.bfloat16 else c.to(dt)


def act_quant(x, block_size=128, scale_fmt=None, scale_dtype=torch.float32, inplace=False):
    """x [..., K] bf16 -> (e4m3 [..., K], scales [..., K/128]); reference.py:117-146."""
    N_ = x.size(-1)
    assert N_ % block_size == 0
    if block_size != 128:
        raise NotImplementedError("act_quant: only the 128-element activation block is on this path")
    if inplace:
        raise NotImplementedError(
            "act_quant(inplace=True) is the attention QAT round trip (torch_ops.py:44-47), "
            "outside the MoE/FP8-linear path"
        )
    if x.dtype != torch.bfloat16:
        raise TypeError(f"act_quant: expected bf16 activations, got {x.dtype}")
    _require_cuda(x)
    kind = _act_kind(scale_fmt, scale_dtype)
    z = x.contiguous()
    y = torch.empty_like(z, dtype=_E4M3)
    s = z.new_empty(*z.size()[:-1], N_ // block_size, dtype=scale_dtype)
    M = z.numel() // N_
    N.call("wz_act_quant_fp8", N.ptr(z), M, N_, N.ptr(y), N.ptr(s), kind, N.stream_handle(z.device))
    return y, s


def fp8_gemm(a, a_s, b, b_s, scale_dtype=torch.float32):
    """C[..., N] = dequant(a) @ dequant(b)^T in bf16; reference.py:292-311."""
    assert a.is_contiguous() and b.is_contiguous(), "Input tensors must be contiguous"
    assert a_s.is_contiguous() and b_s.is_contiguous(), "Scaling factor tensors must be contiguous"
    _require_cuda(a, a_s, b, b_s)
    K = a.size(-1)
    M = a.numel() // K
    Nn = b.size(0)
    if b.size(1) != K:
        raise ValueError(f"fp8_gemm: a has K={K}, b has K={b.size(1)}")
    c = torch.empty(*a.size()[:-1], Nn, dtype=torch.bfloat16, device=a.device)
    N.call("wz_fp8_gemm", N.ptr(a), N.ptr(a_s), N.ptr(b), N.ptr(b_s), N.ptr(c), M, Nn, K,
           _scale_kind_of(a_s), _wscale_kind_of(b_s), N.stream_handle(a.device))
    return _finish(c)


def fp4_gemm(a, a_s, b, b_s, scale_dtype=torch.float32):
    """C[..., N] = dequant(a) @ (e2m1(b) * b_s)^T in bf16; reference.py:572-591."""
    assert a.is_contiguous() and b.is_contiguous(), "Input tensors must be contiguous"
    assert a_s.is_contiguous() and b_s.is_contiguous(), "Scaling factor tensors must be contiguous"
    _require_cuda(a, a_s, b, b_s)
    if b_s.dtype != _E8M0:
        raise TypeError(f"fp4_gemm: MXFP4 weight scales are e8m0, got {b_s.dtype}")
    K = a.size(-1)
    M = a.numel() // K
    Nn = b.size(0)
    if b.size(1) * 2 != K:
        raise ValueError(f"fp4_gemm: a has K={K}, b packs K={b.size(1) * 2}")
    c = torch.empty(*a.size()[:-1], Nn, dtype=torch.bfloat16, device=a.device)
    N.call("wz_fp4_gemm", N.ptr(a), N.ptr(a_s), N.ptr(b), N.ptr(b_s), N.ptr(c), M, Nn, K,
           _scale_kind_of(a_s), N.stream_handle(a.device))
    return _finish(c)


def fp8_linear(x, weight, weight_scale, scale_fmt="ue8m0", scale_dtype=_E8M0):
    """linear() for an FP8 weight with act_quant fused into the GEMM (architecture.py:121-132)."""
    assert x.is_contiguous() and weight.is_contiguous() and weight_scale.is_contiguous()
    _require_cuda(x, weight, weight_scale)
    K = x.size(-1)
    M = x.numel() // K
    Nn = weight.size(0)
    y = torch.empty(*x.size()[:-1], Nn, dtype=torch.bfloat16, device=x.device)
    N.call("wz_fp8_linear", N.ptr(x), N.ptr(weight), N.ptr(weight_scale), N.ptr(y), M, Nn, K,
           _act_kind(scale_fmt, scale_dtype), _wscale_kind_of(weight_scale), N.stream_handle(x.device))
    return _finish(y)


_fp8_gemm_marker = "_v4_hip_fp8_gemm"
fp8_gemm._v4_hip_fp8_gemm = True
fp4_gemm._v4_hip_fp4_gemm = True
act_quant._v4_hip_act_quant = True

_REF = {}


def install(mod) -> bool:
    """Rebind act_quant / fp8_gemm / fp4_gemm on a loaded reference model module.

    Idempotent via the marker attributes; the replaced functions are kept in
    ``_REF`` (the reference's _REF_FP8_GEMM pattern, fp8_vector.py:472-491).
    """
    took = False
    for name, fn in (("act_quant", act_quant), ("fp8_gemm", fp8_gemm), ("fp4_gemm", fp4_gemm)):
        cur = getattr(mod, name, None)
        if cur is fn:
            continue
        _REF.setdefault(name, cur)
        setattr(mod, name, fn)
        took = True
    return took


def uninstall(mod) -> bool:
    """Restore the functions install() replaced on ``mod``."""
    took = False
    for name, fn in (("act_quant", act_quant), ("fp8_gemm", fp8_gemm), ("fp4_gemm", fp4_gemm)):
        if getattr(mod, name, None) is fn and name in _REF:
            setattr(mod, name, _REF.pop(name))
            took = True
    return took
