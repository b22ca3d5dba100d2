"""ctypes binding of libwanferenz_amd.so (the C ABI in include/wanferenz_amd.h).

The library is built in-tree by ``python -m wanferenz_amd.build``.  Loading
fails loudly when it is missing: there is no CPU fallback in the product.
"""

from __future__ import annotations

import ctypes
import os
import threading

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libwanferenz_amd.so")

# Symbols declared in include/wanferenz_amd.h, with their ctypes signatures.
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float
SIGNATURES = {
    "wz_last_error": (ctypes.c_char_p, []),
    "wz_device_info": (_I, [ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "wz_act_quant_fp8": (_I, [_P, _I64, _I64, _P, _P, _I, _P]),
    "wz_fp8_gemm": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _P]),
    "wz_fp8_linear": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _P]),
    "wz_fp4_gemm": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _P]),
    "wz_grouped_fp4_gemm": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _P]),
    "wz_fp4_packed_scale_bytes": (ctypes.c_size_t, [_I64, _I64]),
    "wz_fp4_pack": (_I, [_P, _P, _I64, _I64, _P, _P, _P]),
    "wz_fp4_gemm_packed_workspace_bytes": (ctypes.c_size_t, [_I64, _I64, _I]),
    "wz_fp4_gemm_packed": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _P, ctypes.c_size_t, _P]),
    "wz_fp8_pack": (_I, [_P, _I64, _I64, _P, _P]),
    "wz_fp8_linear_workspace_bytes": (ctypes.c_size_t, [_I64, _I64]),
    "wz_fp8_linear_packed": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _P, ctypes.c_size_t, _P]),
    "wz_fp8_gemm_packed_workspace_bytes": (ctypes.c_size_t, [_I64, _I64, _I]),
    "wz_fp8_gemm_packed": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _P, ctypes.c_size_t, _P]),
    "wz_fp8_linear_packed_add": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _P, ctypes.c_size_t, _P]),
    "wz_fp8_gemm_packed_add": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _P, ctypes.c_size_t, _P]),
    "wz_fp8_gemm_packed_pair": (_I, [_P, _P, _P, _P, _P, _I64, _P, _I64, _I64, _I64, _I, _I, _P, ctypes.c_size_t,
                                     _P]),
    "wz_moe_workspace_bytes": (ctypes.c_size_t, [_P, _I64]),
    "wz_moe_packed_bytes": (ctypes.c_size_t, [_P, _I]),
    "wz_moe_pack": (_I, [_P, _P, _P, _P, _P, _P, _P, _P]),
    "wz_moe_pack_expert": (_I, [_P, _I64, _P, _P, _P, _P, _P, _P, _P]),
    "wz_moe_pack_shared": (_I, [_P, _P, _P, _P, _P]),
    "wz_moe_workspace_init": (_I, [_P, ctypes.c_size_t, _P]),
    "wz_moe_forward": (_I, [_P, _P, _P, _I64, _P, _P, _P, _P, ctypes.c_size_t, _P]),
    "wz_moe_forward_norm": (_I, [_P, _P, _P, _F, _P, _I64, _P, _P, _P, _P, ctypes.c_size_t, _P]),
    "wz_moe_forward_noalloc": (_I, [_P, _P, _P, _I64, _P, _P, _P, _P]),
    "wz_moe_route": (_I, [_P, _P, _P, _I64, _P, _P, _P, _P, _P, _P, ctypes.c_size_t, _P]),
    "wz_moe_replay_stage": (_I, [_P, _P, _P, _I64, _I, _P, _P, ctypes.c_size_t, _P]),
    "wz_rmsnorm": (_I, [_P, _P, _P, _I64, _I64, _F, _P]),
    "wz_add_bf16": (_I, [_P, _P, _P, _I64, _P]),
    "wz_rmsnorm_quant": (_I, [_P, _P, _P, _P, _I64, _I64, _F, _I, _P]),
    "wz_add_rmsnorm_quant": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _F, _I, _P]),
    "wz_fp8_norm_linear_packed_pair": (_I, [_P, _P, _P, _F, _P, _P, _P, _P, _I64, _P, _I64, _I64, _I64, _I, _I,
                                            _P]),
    "wz_fp8_norm_linear_max_rows": (_I, [_I64]),
    "wz_fp8_wire_pack": (_I, [_P, _P, _P, _I64, _I64, _P]),
    "wz_sparse_attn_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64, _I64]),
    "wz_sparse_attn": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _F, _P, _I64, _P]),
    "wz_fp8_wire_unpack": (_I, [_P, _P, _P, _I64, _I64, _P]),
    "wz_synth_fill": (_I, [_P, _I64, ctypes.c_uint64, _I64, _I, ctypes.c_double, ctypes.c_double, _P]),
    "wz_prof_begin": (_I, [_I]),
    "wz_prof_end": (_I, []),
    "wz_prof_get": (_I, [_I, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_F)]),
}

# Scale / format constants (mirrors of the header's #defines).
WZ_SCALE_F32 = 0
WZ_SCALE_UE8M0 = 1
WZ_SCALE_UE8M0_F32 = 2
WZ_WSCALE_F32 = 0
WZ_WSCALE_E8M0 = 1
WZ_SCORE_SOFTMAX = 0
WZ_SCORE_SIGMOID = 1
WZ_SCORE_SQRTSOFTPLUS = 2
WZ_STAGE_ROUTE = 0
WZ_STAGE_W13 = 1
WZ_STAGE_HQUANT = 2
WZ_STAGE_W2 = 3
WZ_STAGE_COMBINE = 4

_LIB = None
_LOCK = threading.Lock()


class WzError(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is None:
            if not os.path.exists(LIB_PATH):
                raise WzError(
                    f"{LIB_PATH} is not built — run `python -m wanferenz_amd.build` "
                    "(there is no CPU fallback)"
                )
            L = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                if not hasattr(L, name):
                    continue
                fn = getattr(L, name)
                fn.restype = res
                fn.argtypes = args
            _LIB = L
    return _LIB


def missing_symbols() -> list:
    L = lib()
    return [n for n in SIGNATURES if not hasattr(L, n)]


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        msg = lib().wz_last_error().decode(errors="replace")
        raise WzError(f"{what}: {msg}" if what else msg)


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)


def ptr(t) -> int:
    """Device (or host) address of a torch tensor, or None."""
    return None if t is None else t.data_ptr()


def stream_handle(device=None) -> int:
    import torch

    return torch.cuda.current_stream(device).cuda_stream


class KernelTimer:
    """Live per-launch timing of the library's kernels with HIP events.

    Usage: ``with KernelTimer(max_launches) as kt: ...`` then ``kt.records``
    holds (kernel name, milliseconds) for every launch made inside the block
    (graph captures are never instrumented).
    """

    def __init__(self, max_launches: int = 4096):
        self.max_launches = max_launches
        self.records = []

    def __enter__(self):
        check(lib().wz_prof_begin(self.max_launches), "wz_prof_begin")
        return self

    def __exit__(self, *exc):
        n = lib().wz_prof_end()
        name = ctypes.c_char_p()
        ms = ctypes.c_float()
        for i in range(n):
            check(lib().wz_prof_get(i, ctypes.byref(name), ctypes.byref(ms)), "wz_prof_get")
            self.records.append((name.value.decode(), float(ms.value)))
        return False

    def mean_ms(self) -> dict:
        out = {}
        for n, ms in self.records:
            out.setdefault(n, []).append(ms)
        return {n: sum(v) / len(v) for n, v in out.items()}
