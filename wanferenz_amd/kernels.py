"""Drop-in kernel functions with the reference's signatures, running on the HIP library.

The reference model imports ``act_quant, fp4_act_quant, fp8_gemm, fp4_gemm,
sparse_attn, hc_split_sinkhorn`` from ``wanferenz.kernels.reference``
(wanferenz/model/architecture.py:12-19) and resolves them as module globals
at call time, so rebinding them on the loaded model module redirects every
FP8 / FP4 linear (the precedent is wanferenz/kernels/fp8_vector.py:476-485).
:func:`install` does that for the four functions on this path (all but
hc_split_sinkhorn).

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
    """x [..., K] bf16 -> (e4m3 [..., K], scales [..., K/128]); reference.py:117-146.

    The MoE / FP8-linear path quantises in 128-element blocks.  The model also
    calls act_quant on the attention path with other block sizes and with
    ``inplace=True`` (the QAT round trip of torch_ops.py:44-47, e.g.
    architecture.py:470, 632): once :func:`install` has rebound act_quant,
    those calls go to the binding it replaced, unchanged."""
    N_ = x.size(-1)
    if block_size != 128 or inplace:
        prev = _REF.get("act_quant")
        if prev is not None:
            return prev(x, block_size, scale_fmt, scale_dtype, inplace)
        raise NotImplementedError(
            "act_quant: only block_size=128 with inplace=False runs on this path; other forms go to the "
            "binding install() replaced, and none was installed")
    assert N_ % block_size == 0
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


# Pack FP8 weight Parameters into the GEMV tile format on their first use outside
# graph capture, in their own storage (fp8_gemm / linear then read the tiles).
PACK_FP8_WEIGHTS = True


def _tile_view(b) -> torch.Tensor:
    return b.detach().view(torch.uint8).view(-1)


def is_packed(b) -> bool:
    """True when FP8 weight ``b`` holds the packed tiles (wz_fp8_pack's format) in
    its own storage: packed at this address and not written since."""
    got = getattr(b, "_wz_packed", None)
    return got is not None and got == (b.data_ptr(), b._version)


def _packed_of(b):
    """The packed tiles of FP8 weight ``b`` ([N, K] e4m3 Parameter), packing it once.

    The tiles hold the same N*K bytes as the row-major weight, so they are
    written over it: the Parameter keeps its shape, dtype and storage, and the
    model holds one copy of each projection (the reference's decode retile reads
    its weights in place as well, fp8_vector.py:316-351).  ``b._wz_packed``
    records the storage address and version the tiles were written at; a later
    write into the Parameter (a checkpoint load bumps its version) holds
    row-major bytes again, and the next call repacks.  Returns None where the
    tile format does not apply (N % 16, K % 128, a CPU or non-contiguous
    tensor), for tensors that are not Parameters, or while a graph is being
    captured and the weight is not packed yet; the caller then reads the
    row-major bytes."""
    if not PACK_FP8_WEIGHTS or not isinstance(b, torch.nn.Parameter) or b.dim() != 2:
        return None
    Nn, K = b.shape
    if Nn % 16 or K % 128 or b.dtype not in (_E4M3, torch.uint8) or not b.is_cuda:
        return None
    if is_packed(b):
        return _tile_view(b)
    if torch.cuda.is_current_stream_capturing() or not b.is_contiguous():
        return None
    tmp = torch.empty(Nn * K, dtype=torch.uint8, device=b.device)
    N.call("wz_fp8_pack", N.ptr(b), Nn, K, N.ptr(tmp), N.stream_handle(b.device))
    # .data: the copy is not an autograd write, so the version stays the one recorded
    b.data.view(torch.uint8).view(-1).copy_(tmp)
    b._wz_packed = (b.data_ptr(), b._version)
    return _tile_view(b)


def unpack_fp8_in_place(b) -> bool:
    """Turn a weight packed by :func:`_packed_of` back into row-major bytes (for a
    consumer that reads the reference layout, e.g. the MoE bank packer).  The
    tile of 16 rows x 128 K is two 1-KB halves; lane l = 16 g + r of half h holds
    row r, K [64 h + 16 g, +16).  Returns whether anything was done."""
    if not is_packed(b):
        return False
    Nn, K = b.shape
    t = _tile_view(b).view(Nn // 16, K // 128, 2, 4, 16, 16)
    rows = t.permute(0, 4, 1, 2, 3, 5).contiguous().view(-1)
    b.data.view(torch.uint8).view(-1).copy_(rows)
    del b._wz_packed
    return True


def _moe_param_ids(module) -> set:
    """ids of the parameters inside MoE layers (modules with experts and a shared
    expert): the MoE packer turns those into its own banks."""
    out = set()
    for m in module.modules():
        if hasattr(m, "experts") and hasattr(m, "shared_experts"):
            out.update(id(p) for p in m.parameters())
    return out


def pack_fp8_weights(module) -> int:
    """Pack every FP8 weight Parameter of ``module`` in place now (before a graph
    capture, so captured steps find the packed tiles); returns how many are packed.
    The MoE layers' weights are left to the MoE packer (moe.prepare)."""
    skip = _moe_param_ids(module)
    n = 0
    for p in module.parameters():
        if p.dtype == _E4M3 and p.is_cuda and id(p) not in skip and _packed_of(p) is not None:
            n += 1
    return n


def fp8_gemm(a, a_s, b, b_s, scale_dtype=torch.float32):
    """C[..., N] = dequant(a) @ dequant(b)^T in bf16; reference.py:292-311.

    A weight Parameter is served from its packed copy (GEMV for up to 16 rows,
    the dense tile GEMM above), as the reference's decode retile serves it
    (fp8_vector.py:289-297); any other weight from its row-major bytes."""
    assert a.is_contiguous() and b.is_contiguous(), "Input tensors must be contiguous"
    assert a_s.is_contiguous() and b_s.is_contiguous(), "Scaling factor tensors must be contiguous"
    _require_cuda(a, a_s, b, b_s)
    K = a.size(-1)
    M = a.numel() // K
    Nn = b.size(0)
    if b.size(1) != K:
        raise ValueError(f"fp8_gemm: a has K={K}, b has K={b.size(1)}")
    c = torch.empty(*a.size()[:-1], Nn, dtype=torch.bfloat16, device=a.device)
    akind, wkind = _scale_kind_of(a_s), _wscale_kind_of(b_s)
    packed = _packed_of(b)
    if packed is not None:
        need = int(N.lib().wz_fp8_gemm_packed_workspace_bytes(M, K, akind))
        ws = torch.empty(need, dtype=torch.uint8, device=a.device) if need else None
        N.call("wz_fp8_gemm_packed", N.ptr(a), N.ptr(a_s), N.ptr(packed), N.ptr(b_s), N.ptr(c), M, Nn, K, akind,
               wkind, N.ptr(ws), need, N.stream_handle(a.device))
    else:
        N.call("wz_fp8_gemm", N.ptr(a), N.ptr(a_s), N.ptr(b), N.ptr(b_s), N.ptr(c), M, Nn, K, akind, wkind,
               N.stream_handle(a.device))
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


def grouped_fp4_gemm(a, a_s, w, w_s, scale_dtype=torch.float32):
    """C[g, :] = dequant(a[g]) @ (e2m1(w[g]) * w_s[g])^T in bf16; fp4_grouped.py:96-128.

    a [G, K] e4m3 with a_s [G, K/128], w [G, N, K/2] e2m1x2 with w_s [G, N, K/32]
    e8m0 (the gathered bank slices of the banked decode path).  The contiguity
    and N-tile assertions are the reference's; the reference's G <= 32 bound
    (its A tile) does not apply here."""
    assert a.is_contiguous() and w.is_contiguous(), "grouped fp4: a and w must be contiguous"
    assert a_s.is_contiguous() and w_s.is_contiguous(), "grouped fp4: scales must be contiguous"
    assert w.size(1) % 128 == 0, f"grouped fp4: N={w.size(1)} is not a whole number of 128-wide tiles"
    _require_cuda(a, a_s, w, w_s)
    if w_s.dtype != _E8M0:
        raise TypeError(f"grouped_fp4_gemm: MXFP4 weight scales are e8m0, got {w_s.dtype}")
    G, K = a.shape
    Nn = w.size(1)
    if w.size(0) != G or w.size(2) * 2 != K:
        raise ValueError(f"grouped_fp4_gemm: a [{G}, {K}] against w {tuple(w.shape)}")
    c = torch.empty(G, Nn, dtype=torch.bfloat16, device=a.device)
    N.call("wz_grouped_fp4_gemm", N.ptr(a), N.ptr(a_s), N.ptr(w), N.ptr(w_s), N.ptr(c), G, Nn, K,
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


class PackedFp4Linear:
    """An MXFP4 weight (e2m1x2 [N, K/2] with e8m0 scales [N, K/32]) relaid once into
    the expert banks' tile format (wz_fp4_pack), for fp4_gemm at row counts past
    decode: ``gemm(q, q_s)`` = fp4_gemm(q, q_s, weight, scale) (reference.py:572-591)
    -> bf16 [..., N] on the tile GEMM of the MoE prefill."""

    def __init__(self, weight, weight_scale):
        assert weight.is_contiguous() and weight_scale.is_contiguous()
        _require_cuda(weight, weight_scale)
        if weight_scale.dtype != _E8M0:
            raise TypeError(f"PackedFp4Linear: MXFP4 weight scales are e8m0, got {weight_scale.dtype}")
        self.N, self.K = weight.size(0), weight.size(1) * 2
        dev = weight.device
        self.packed = torch.empty(self.N * self.K // 2, dtype=torch.uint8, device=dev)
        self.packed_s = torch.empty(int(N.lib().wz_fp4_packed_scale_bytes(self.N, self.K)), dtype=torch.uint8,
                                    device=dev)
        N.call("wz_fp4_pack", N.ptr(weight), N.ptr(weight_scale), self.N, self.K, N.ptr(self.packed),
               N.ptr(self.packed_s), N.stream_handle(dev))
        self._ws = None

    def reserve(self, M: int, scale_dtype=torch.float32):
        kind = N.WZ_SCALE_UE8M0 if scale_dtype == _E8M0 else N.WZ_SCALE_F32
        need = int(N.lib().wz_fp4_gemm_packed_workspace_bytes(M, self.K, kind))
        if need and (self._ws is None or self._ws.numel() < need):
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(f"PackedFp4Linear: reserve({M}) before capturing a graph")
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.packed.device)
        return self

    def gemm(self, q, q_s, out=None):
        assert q.is_contiguous() and q_s.is_contiguous() and q.size(-1) == self.K
        _require_cuda(q, q_s)
        M = q.numel() // self.K
        self.reserve(M, q_s.dtype)
        y = torch.empty(*q.size()[:-1], self.N, dtype=torch.bfloat16, device=q.device) if out is None else out
        ws = self._ws
        N.call("wz_fp4_gemm_packed", N.ptr(q), N.ptr(q_s), N.ptr(self.packed), N.ptr(self.packed_s), N.ptr(y), M,
               self.N, self.K, _scale_kind_of(q_s), N.ptr(ws), 0 if ws is None else ws.numel(),
               N.stream_handle(q.device))
        return _finish(y)


class PackedFp8Linear:
    """An FP8 linear whose weight is relaid once into MFMA-ready tiles (wz_fp8_pack).

    ``__call__(x)`` is linear(x, weight) for the FP8 weight (architecture.py:121-132:
    act_quant with the module's scale rule, then fp8_gemm) -> bf16 [..., N].  The
    packed copy holds the same N*K bytes as the weight; the scale tensor is used as
    given (float32 or e8m0 [ceil(N/128), K/128]).  ``reserve(M)`` sizes the workspace
    for row counts above the GEMV range before a graph capture.
    """

    def __init__(self, weight, weight_scale, scale_fmt="ue8m0"):
        assert weight.is_contiguous() and weight_scale.is_contiguous()
        _require_cuda(weight, weight_scale)
        if weight.dtype not in (_E4M3, torch.uint8):
            raise TypeError(f"PackedFp8Linear: e4m3 weight expected, got {weight.dtype}")
        self.N, self.K = weight.shape
        self.w_kind = _wscale_kind_of(weight_scale)
        self.act_kind = N.WZ_SCALE_F32 if scale_fmt is None else N.WZ_SCALE_UE8M0_F32
        self.scale = weight_scale
        self.packed = torch.empty(self.N * self.K, dtype=torch.uint8, device=weight.device)
        N.call("wz_fp8_pack", N.ptr(weight), self.N, self.K, N.ptr(self.packed), N.stream_handle(weight.device))
        self._ws = None

    def workspace_bytes(self, M: int) -> int:
        return int(N.lib().wz_fp8_linear_workspace_bytes(M, self.K))

    def reserve(self, M: int):
        need = self.workspace_bytes(M)
        if need and (self._ws is None or self._ws.numel() < need):
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(f"PackedFp8Linear: reserve({M}) before capturing a graph")
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.packed.device)
        return self

    def _out(self, lead, M, out, residual, device):
        y = torch.empty(*lead, self.N, dtype=torch.bfloat16, device=device) if out is None else out
        if residual is not None:
            assert residual.is_contiguous() and residual.dtype == torch.bfloat16
            if residual.numel() != M * self.N:
                raise ValueError(f"PackedFp8Linear: residual has {residual.numel()} elements for [{M}, {self.N}]")
        return y

    def __call__(self, x, out=None, residual=None):
        """linear(x, weight); with ``residual``, residual + linear(x, weight) in one
        launch (the block's bf16 residual add fused into the epilogue)."""
        assert x.is_contiguous() and x.size(-1) == self.K
        _require_cuda(x)
        if x.dtype != torch.bfloat16:
            raise TypeError(f"PackedFp8Linear: bf16 input expected, got {x.dtype}")
        M = x.numel() // self.K
        self.reserve(M)
        y = self._out(x.size()[:-1], M, out, residual, x.device)
        ws = self._ws
        tail = (M, self.N, self.K, self.act_kind, self.w_kind, N.ptr(ws), 0 if ws is None else ws.numel(),
                N.stream_handle(x.device))
        if residual is None:
            N.call("wz_fp8_linear_packed", N.ptr(x), N.ptr(self.packed), N.ptr(self.scale), N.ptr(y), *tail)
        else:
            N.call("wz_fp8_linear_packed_add", N.ptr(x), N.ptr(self.packed), N.ptr(self.scale), N.ptr(residual),
                   N.ptr(y), *tail)
        return y

    def gemm(self, q, q_s, out=None, residual=None):
        """fp8_gemm(q, q_s, weight, scale) from pre-quantised activations (e4m3 [..., K]
        with scales [..., K/128], e.g. from rms_norm_quant), optionally + residual."""
        assert q.is_contiguous() and q_s.is_contiguous() and q.size(-1) == self.K
        _require_cuda(q, q_s)
        M = q.numel() // self.K
        kind = _scale_kind_of(q_s)
        need = int(N.lib().wz_fp8_gemm_packed_workspace_bytes(M, self.K, kind))
        if need and (self._ws is None or self._ws.numel() < need):
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("PackedFp8Linear.gemm: workspace needed during a graph capture")
            self._ws = torch.empty(need, dtype=torch.uint8, device=q.device)
        y = self._out(q.size()[:-1], M, out, residual, q.device)
        ws = self._ws
        tail = (M, self.N, self.K, kind, self.w_kind, N.ptr(ws), 0 if ws is None else ws.numel(),
                N.stream_handle(q.device))
        if residual is None:
            N.call("wz_fp8_gemm_packed", N.ptr(q), N.ptr(q_s), N.ptr(self.packed), N.ptr(self.scale), N.ptr(y), *tail)
        else:
            N.call("wz_fp8_gemm_packed_add", N.ptr(q), N.ptr(q_s), N.ptr(self.packed), N.ptr(self.scale),
                   N.ptr(residual), N.ptr(y), *tail)
        return y


class PackedFp8Pair:
    """Two FP8 linears that read the same input (wq_a and wkv of the attention side,
    wq_b and the indexer's wq_b; architecture.py:611-672), their weights stacked
    row-wise and packed once, served by one launch (wz_fp8_gemm_packed_pair).
    ``gemm(q, q_s)`` -> (fp8_gemm(q, q_s, w0, s0), fp8_gemm(q, q_s, w1, s1)).  The
    first weight's rows must be a multiple of 128 (its block scales end on a row)."""

    def __init__(self, w0, s0, w1, s1, scale_fmt="ue8m0"):
        for t in (w0, s0, w1, s1):
            assert t.is_contiguous()
        _require_cuda(w0, s0, w1, s1)
        if w0.size(1) != w1.size(1) or w0.size(0) % 128 or s0.dtype != s1.dtype:
            raise ValueError("PackedFp8Pair: weights must share K, the first must have a multiple of 128 rows, "
                             "and the scales one dtype")
        self.N0, self.N1, self.K = w0.size(0), w1.size(0), w0.size(1)
        self.N = self.N0 + self.N1
        self.w_kind = _wscale_kind_of(s0)
        self.scale = torch.cat([s0.view(torch.uint8) if s0.dtype == _E8M0 else s0,
                                s1.view(torch.uint8) if s1.dtype == _E8M0 else s1]).contiguous()
        w = torch.cat([w0.view(torch.uint8), w1.view(torch.uint8)]).contiguous()
        self.packed = torch.empty(self.N * self.K, dtype=torch.uint8, device=w0.device)
        N.call("wz_fp8_pack", N.ptr(w), self.N, self.K, N.ptr(self.packed), N.stream_handle(w0.device))
        torch.cuda.current_stream(w0.device).synchronize()  # the stacked copy is freed on return
        self._ws = None

    def reserve(self, M: int, q_dtype=_E8M0):
        kind = N.WZ_SCALE_UE8M0 if q_dtype == _E8M0 else N.WZ_SCALE_F32
        need = int(N.lib().wz_fp8_gemm_packed_workspace_bytes(M, self.K, kind))
        if need and (self._ws is None or self._ws.numel() < need):
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(f"PackedFp8Pair: reserve({M}) before capturing a graph")
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.packed.device)
        return self

    def _outs(self, lead, M, out, device):
        if out is None:
            return (torch.empty(*lead, self.N0, dtype=torch.bfloat16, device=device),
                    torch.empty(*lead, self.N1, dtype=torch.bfloat16, device=device))
        for y, n in zip(out, (self.N0, self.N1)):
            if y.dtype != torch.bfloat16 or not y.is_contiguous() or y.numel() != M * n or y.device != device:
                raise ValueError(f"PackedFp8Pair: an output must be a contiguous bf16 tensor of {M}x{n} "
                                 f"elements on {device}, got {y.dtype} {tuple(y.shape)} on {y.device}")
        return out

    def gemm(self, q, q_s, out=None):
        assert q.is_contiguous() and q_s.is_contiguous() and q.size(-1) == self.K
        _require_cuda(q, q_s)
        M = q.numel() // self.K
        self.reserve(M, q_s.dtype)
        y0, y1 = self._outs(q.size()[:-1], M, out, q.device)
        ws = self._ws
        N.call("wz_fp8_gemm_packed_pair", N.ptr(q), N.ptr(q_s), N.ptr(self.packed), N.ptr(self.scale), N.ptr(y0),
               self.N0, N.ptr(y1), M, self.N, self.K, _scale_kind_of(q_s), self.w_kind, N.ptr(ws),
               0 if ws is None else ws.numel(), N.stream_handle(q.device))
        return y0, y1

    def norm_gemm(self, x, weight, eps=1e-6, b=None, sum_out=None, out=None, scale_fmt="ue8m0",
                  scale_dtype=_E8M0):
        """``gemm(*rms_norm_quant(x, weight, eps))``, or with ``b`` the residual step
        first (``add_rms_norm_quant(x, b, ...)``, h written to ``sum_out``), in one
        launch (wz_fp8_norm_linear_packed_pair): the same codes, so the same outputs
        bit for bit.  At most ``norm_linear_rows(K)`` rows."""
        assert x.is_contiguous() and weight.is_contiguous() and x.size(-1) == self.K
        _require_cuda(x, weight)
        if x.dtype != torch.bfloat16 or weight.dtype != torch.float32 or weight.numel() != self.K:
            raise TypeError("norm_gemm: x must be bf16 [..., K] and weight float32 [K]")
        if b is not None:
            assert b.is_contiguous() and b.shape == x.shape and b.dtype == torch.bfloat16
            _require_cuda(b)
        elif sum_out is not None:
            raise ValueError("norm_gemm: sum_out needs b")
        M = x.numel() // self.K
        kind = _act_kind(scale_fmt, scale_dtype)
        y0, y1 = self._outs(x.size()[:-1], M, out, x.device)
        if b is not None and sum_out is None:
            sum_out = torch.empty_like(x)
        if sum_out is not None and (sum_out.dtype != torch.bfloat16 or not sum_out.is_contiguous()
                                    or sum_out.numel() != x.numel() or sum_out.device != x.device):
            raise ValueError("norm_gemm: sum_out must be a contiguous bf16 tensor of x's size on x's device")
        N.call("wz_fp8_norm_linear_packed_pair", N.ptr(x), None if b is None else N.ptr(b), N.ptr(weight),
               float(eps), None if sum_out is None else N.ptr(sum_out), N.ptr(self.packed), N.ptr(self.scale),
               N.ptr(y0), self.N0, N.ptr(y1), M, self.N, self.K, kind, self.w_kind, N.stream_handle(x.device))
        return (y0, y1) if b is None else (sum_out, y0, y1)


def norm_linear_rows(K: int) -> int:
    """Rows the fused norm + FP8 projections (``PackedFp8Pair.norm_gemm``) serve at K."""
    return int(N.lib().wz_fp8_norm_linear_max_rows(int(K)))


def rms_norm(x, weight, eps=1e-6, out=None):
    """RMSNorm.forward (architecture.py:217-230): bf16(weight * (x * rsqrt(mean(x^2) + eps))),
    fp32 math, one row per token; weight is the module's fp32 parameter."""
    assert x.is_contiguous() and weight.is_contiguous()
    _require_cuda(x, weight)
    if x.dtype != torch.bfloat16 or weight.dtype != torch.float32:
        raise TypeError(f"rms_norm: x must be bf16 and weight float32 (got {x.dtype}, {weight.dtype})")
    D = x.size(-1)
    if weight.numel() != D:
        raise ValueError(f"rms_norm: weight has {weight.numel()} elements for rows of {D}")
    y = torch.empty_like(x) if out is None else out
    N.call("wz_rmsnorm", N.ptr(x), N.ptr(weight), N.ptr(y), x.numel() // D, D, float(eps),
           N.stream_handle(x.device))
    return y


def _norm_quant_out(x, scale_fmt, scale_dtype, out):
    D = x.size(-1)
    kind = _act_kind(scale_fmt, scale_dtype)
    if out is None:
        q = torch.empty(x.shape, dtype=_E4M3, device=x.device)
        s = torch.empty(*x.shape[:-1], D // 128, dtype=_E8M0 if kind == N.WZ_SCALE_UE8M0 else torch.float32,
                        device=x.device)
    else:
        q, s = out
    return kind, q, s


def rms_norm_quant(x, weight, eps=1e-6, scale_fmt="ue8m0", scale_dtype=_E8M0, out=None):
    """act_quant(rms_norm(x, weight, eps)) in one pass (architecture.py:217-230 then
    reference.py:117-146): -> (e4m3 [..., D], scales [..., D/128]); ``out``: (q, s)
    buffers to fill."""
    assert x.is_contiguous() and weight.is_contiguous()
    _require_cuda(x, weight)
    if x.dtype != torch.bfloat16 or weight.dtype != torch.float32:
        raise TypeError(f"rms_norm_quant: x must be bf16 and weight float32 (got {x.dtype}, {weight.dtype})")
    D = x.size(-1)
    kind, q, s = _norm_quant_out(x, scale_fmt, scale_dtype, out)
    N.call("wz_rmsnorm_quant", N.ptr(x), N.ptr(weight), N.ptr(q), N.ptr(s), x.numel() // D, D, float(eps), kind,
           N.stream_handle(x.device))
    return q, s


def add_rms_norm_quant(x, b, weight, eps=1e-6, scale_fmt="ue8m0", scale_dtype=_E8M0, sum_out=None, out=None):
    """The residual step h = x + b (bf16 add) fused with rms_norm_quant(h, weight):
    -> (h, e4m3 [..., D], scales [..., D/128]).  h is written to ``sum_out`` (a new
    tensor when None)."""
    assert x.is_contiguous() and b.is_contiguous() and weight.is_contiguous() and x.shape == b.shape
    _require_cuda(x, b, weight)
    if x.dtype != torch.bfloat16 or b.dtype != torch.bfloat16 or weight.dtype != torch.float32:
        raise TypeError("add_rms_norm_quant: x and b must be bf16 and weight float32")
    D = x.size(-1)
    h = torch.empty_like(x) if sum_out is None else sum_out
    kind, q, s = _norm_quant_out(x, scale_fmt, scale_dtype, out)
    N.call("wz_add_rmsnorm_quant", N.ptr(x), N.ptr(b), N.ptr(weight), N.ptr(h), N.ptr(q), N.ptr(s),
           x.numel() // D, D, float(eps), kind, N.stream_handle(x.device))
    return h, q, s


def sparse_attn(q, kv, attn_sink, topk_idxs, softmax_scale, workspace=None):
    """sparse_attn (torch_ops.py:114-146, reference.py:397-418): q [b, s, h, d] bf16,
    kv [b, n, d] bf16, attn_sink [h] fp32, topk_idxs [b, s, topk] int32 -> [b, s, h, d]
    in q's dtype.  Head counts that are not a multiple of 16 are padded with zero
    heads, as the reference's GPU wrapper does (reference.py:406-416).  With few
    queries the index blocks are split over workgroups whose partials need
    ``sparse_attn_workspace_bytes`` of device memory: ``workspace`` (a uint8 tensor
    at least that large) is used when given, else one is allocated."""
    _require_cuda(q, kv, attn_sink, topk_idxs)
    b, s, h, d = q.shape
    if q.dtype != torch.bfloat16 or kv.dtype != torch.bfloat16:
        raise TypeError(f"sparse_attn: bf16 q and kv expected (got {q.dtype}, {kv.dtype})")
    hp = (h + 15) // 16 * 16
    if hp != h:
        q = torch.cat([q, q.new_zeros(b, s, hp - h, d)], dim=2)
        attn_sink = torch.cat([attn_sink, attn_sink.new_zeros(hp - h)])
    q = q.contiguous()
    kv = kv.contiguous()
    sink = attn_sink.float().contiguous()
    idx = topk_idxs.to(torch.int32).contiguous()
    topk = idx.size(-1)
    o = torch.empty_like(q)
    need = sparse_attn_workspace_bytes(b, s, hp, d, topk)
    if need and (workspace is None or workspace.numel() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    ws, wsb = (N.ptr(workspace), workspace.numel()) if need else (None, 0)
    N.call("wz_sparse_attn", N.ptr(q), N.ptr(kv), N.ptr(sink), N.ptr(idx), N.ptr(o), b, s, hp, d, kv.size(1),
           topk, float(softmax_scale), ws, wsb, N.stream_handle(q.device))
    return o if hp == h else o.narrow(2, 0, h).contiguous()


def sparse_attn_workspace_bytes(b, s, h, d, topk) -> int:
    """Device bytes of the split partials of a sparse_attn call (0: not split)."""
    return int(N.lib().wz_sparse_attn_workspace_bytes(b, s, h, d, topk))


def wire_pack(t):
    """_pack_t (serving/chain.py:208-217): bf16 [..., D] -> (e4m3 [..., D], bf16 scale [...])."""
    assert t.is_contiguous()
    _require_cuda(t)
    if t.dtype != torch.bfloat16:
        raise TypeError(f"wire_pack: bf16 input expected, got {t.dtype}")
    D = t.size(-1)
    q = torch.empty(t.shape, dtype=_E4M3, device=t.device)
    scale = torch.empty(t.shape[:-1], dtype=torch.bfloat16, device=t.device)
    N.call("wz_fp8_wire_pack", N.ptr(t), N.ptr(q), N.ptr(scale), t.numel() // D, D, N.stream_handle(t.device))
    return q, scale


def wire_unpack(q, scale):
    """_unpack_t (serving/chain.py:220-222): bf16(q) * scale -> bf16 [..., D]."""
    assert q.is_contiguous() and scale.is_contiguous()
    _require_cuda(q, scale)
    D = q.size(-1)
    y = torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)
    N.call("wz_fp8_wire_unpack", N.ptr(q), N.ptr(scale), N.ptr(y), q.numel() // D, D, N.stream_handle(q.device))
    return y


def add(a, b, out=None):
    """Elementwise a + b of two bf16 tensors of one shape, fp32 sum rounded once to bf16:
    the plain residual step (x + f(x)) of a decoder stage.  The model's own blocks mix
    the residual through hyper-connections (Block.hc_post, architecture.py:839-850),
    which this function does not implement."""
    assert a.is_contiguous() and b.is_contiguous() and a.shape == b.shape
    _require_cuda(a, b)
    if a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16:
        raise TypeError(f"add: bf16 operands expected (got {a.dtype}, {b.dtype})")
    out = torch.empty_like(a) if out is None else out
    N.call("wz_add_bf16", N.ptr(a), N.ptr(b), N.ptr(out), a.numel(), N.stream_handle(a.device))
    return out


def _model_module_of(fn):
    import sys

    return sys.modules.get(getattr(fn, "__module__", "") or "")


def linear(x, weight, bias=None):
    """linear() of the model (architecture.py:121-134) with the FP8 case fused:
    act_quant of x runs inside the GEMV / GEMM prologue on the packed weight
    (the same codes and scales as act_quant, so the same product).  The block
    size and scale format are the model module's globals, read at call time as
    the reference reads them; an FP4 weight runs act_quant + fp4_gemm, anything
    else F.linear, as in the reference."""
    assert bias is None
    mod = _LINEAR_MOD
    if weight.dtype == _E4M3:
        _check_fp8_operands(x, weight)
    if weight.dtype == _E4M3 and x.dtype == torch.bfloat16 and getattr(mod, "block_size", 128) == 128:
        packed = _packed_of(weight)
        if packed is not None:
            _require_cuda(x)
            x = x.contiguous()
            scale_fmt = getattr(mod, "scale_fmt", None)
            K = x.size(-1)
            M = x.numel() // K
            Nn = weight.size(0)
            akind = N.WZ_SCALE_F32 if scale_fmt is None else N.WZ_SCALE_UE8M0_F32
            y = torch.empty(*x.size()[:-1], Nn, dtype=torch.bfloat16, device=x.device)
            need = int(N.lib().wz_fp8_linear_workspace_bytes(M, K))
            ws = torch.empty(need, dtype=torch.uint8, device=x.device) if need else None
            N.call("wz_fp8_linear_packed", N.ptr(x), N.ptr(packed), N.ptr(weight.scale), N.ptr(y), M, Nn, K,
                   akind, _wscale_kind_of(weight.scale), N.ptr(ws), need, N.stream_handle(x.device))
            return _finish(y)
    if weight.dtype == _E4M3 and is_packed(weight):
        # the replaced binding would read the tiles as row-major bytes
        raise TypeError(f"linear: the FP8 weight is packed in place; its input must be bf16 (got {x.dtype}) "
                        f"with 128-element quantisation blocks (got {getattr(mod, 'block_size', 128)})")
    return _REF["linear"](x, weight, bias)


def _check_fp8_operands(x, weight):
    """The shapes linear() on an FP8 weight needs (architecture.py:158-168): x
    [..., K] against weight [N, K] and its block scales [ceil(N/128), ceil(K/128)].
    The packed kernels read K and the scale grid from these, so a mismatch would
    read past the weight; it raises here, before any launch, as the reference's
    fp8_gemm rejects it."""
    Nn, K = weight.shape
    if x.size(-1) != K:
        raise ValueError(f"linear: x has K={x.size(-1)}, the FP8 weight [{Nn}, {K}] needs K={K}")
    s = getattr(weight, "scale", None)
    want = ((Nn + 127) // 128, (K + 127) // 128)
    if s is None or tuple(s.shape) != want:
        raise ValueError(f"linear: the FP8 weight [{Nn}, {K}] needs block scales {list(want)}, "
                         f"got {None if s is None else list(s.shape)}")


fp8_gemm._v4_hip_fp8_gemm = True
fp4_gemm._v4_hip_fp4_gemm = True
act_quant._v4_hip_act_quant = True
linear._v4_hip_linear = True

_REF = {}
_LINEAR_MOD = None


def _installed():
    return (("act_quant", act_quant), ("fp8_gemm", fp8_gemm), ("fp4_gemm", fp4_gemm), ("sparse_attn", sparse_attn),
            ("linear", linear))


def install(mod, model=None) -> bool:
    """Rebind act_quant / fp8_gemm / fp4_gemm / sparse_attn / linear on a loaded
    reference model module (each one the module has).

    Idempotent via the marker attributes; the replaced functions are kept in
    ``_REF`` (the reference's _REF_FP8_GEMM pattern, fp8_vector.py:472-491).
    With ``model`` given, its FP8 weights are packed in place now
    (pack_fp8_weights), so a graph captured afterwards runs the packed GEMV from
    the first step and the model holds one copy of each projection.
    """
    global _LINEAR_MOD
    took = False
    for name, fn in _installed():
        if not hasattr(mod, name):
            continue
        cur = getattr(mod, name)
        if cur is fn:
            continue
        _REF.setdefault(name, cur)
        setattr(mod, name, fn)
        took = True
    if hasattr(mod, "linear"):
        _LINEAR_MOD = mod
    if model is not None:
        pack_fp8_weights(model)
    return took


def uninstall(mod, model=None) -> bool:
    """Restore the functions install() replaced on ``mod``.  The restored bindings
    read FP8 weights row-major, so with ``model`` given every weight packed in
    place is turned back (unpack_fp8_in_place) first."""
    if model is not None:
        for p in model.parameters():
            unpack_fp8_in_place(p)
    took = False
    for name, fn in _installed():
        if getattr(mod, name, None) is fn and name in _REF:
            setattr(mod, name, _REF.pop(name))
            took = True
    return took
