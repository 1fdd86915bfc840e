"""ctypes binding of ``liblaplace_hip.so`` (the C ABI of include/laplace_hip.h).

Loading fails loudly: if the library has not been built there is no CPU
fallback in this package, by design. Build it with
``python -m laplace_amd.build``.
"""
from __future__ import annotations

import ctypes as C
import os

# LAPLACE_HIP_LIB: load another build of the library (side-by-side timing runs)
LIB_PATH = os.environ.get("LAPLACE_HIP_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                             "liblaplace_hip.so")

LP_OK, LP_UNSUPPORTED, LP_EINVAL, LP_EHIP, LP_ENODEV = 0, 1, 2, 3, 4
STATUS_NAMES = {0: "LP_OK", 1: "LP_UNSUPPORTED", 2: "LP_EINVAL", 3: "LP_EHIP", 4: "LP_ENODEV"}

# Every symbol the header declares, with (restype, argtypes).
_vp, _i, _u32, _sz, _b = C.c_void_p, C.c_int, C.c_uint32, C.c_size_t, C.c_bool


class BatchSpec(C.Structure):
    """lp_batch_spec of include/laplace_hip.h."""
    _fields_ = [("x", _vp), ("w", _vp), ("type", _u32), ("y", _vp), ("K", _i), ("N", _i)]


SIGNATURES = {
    "lp_gemm": (_b, [_vp, _vp, _u32, _vp, _i, _i, _i]),
    "lp_moe_gemv": (_b, [_vp, _vp, _u32, _vp, _i, _vp, _i, _i]),
    "lp_moe_gemv_multi": (_b, [_vp, _vp, _u32, _vp, _i, _vp, _i, _i]),
    "lp_get_gemm": (_vp, []),
    "lp_get_moe_gemv": (_vp, []),
    "lp_get_moe_gemv_multi": (_vp, []),
    "lp_register_weights": (_i, [_vp, _sz]),
    "lp_release_weights": (None, []),
    "lp_release_region": (_i, [_vp]),
    "lp_quantize_act": (_i, [_vp, _i, _i, _vp, _vp, _vp, _vp, _vp]),
    "lp_act_workspace_bytes": (_sz, [_i, _i]),
    "lp_quantize_act_dev": (_i, [_vp, _i, _i, _vp, _sz, _vp]),
    "lp_act_unpack_dev": (_i, [_vp, _i, _i, _vp, _vp, _vp, _vp, _vp]),
    "lp_gemm_dev": (_i, [_vp, _vp, _u32, _vp, _i, _i, _i, _vp, _sz, _vp]),
    "lp_gemm_q_dev": (_i, [_vp, _vp, _u32, _vp, _i, _i, _i, _vp]),
    "lp_gemm_route": (C.c_char_p, [_u32, _i, _i, _i, _vp]),
    "lp_set_gemm_kernel": (_i, [_i]),
    "lp_mfma_probe_dev": (_i, [_i, _i, _i, _i, _vp, _vp]),
    "lp_gemm_dev_noalloc": (_i, [_vp, _vp, _u32, _vp, _i, _i, _i, _vp]),
    "lp_block_sums_dev": (_i, [_vp, _vp, _u32, _vp, _i, _i, _i, _vp]),
    "lp_moe_grouped_dev": (_i, [_vp, _i, _vp, _vp, _u32, _vp, _i, _i, _i, _i, _i, _vp, _sz, _vp]),
    "lp_moe_workspace_bytes": (_sz, [_i, _i, _i, _i, _i]),
    "lp_moe_grouped": (_b, [_vp, _i, _vp, _vp, _u32, _vp, _i, _i, _i, _i, _i]),
    "lp_dequantize": (_i, [_vp, _u32, _vp, C.c_long]),
    "lp_dequantize_dev": (_i, [_vp, _u32, _vp, C.c_long, _vp]),
    "lp_moe_ffn_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _u32]),
    "lp_moe_ffn_dev": (_i, [_vp, _i, _i, _vp, _u32, _vp, _vp, C.c_float, _vp, _u32, _vp, _u32, _vp,
                            _i, _i, _i, _vp, _vp, _vp, _vp, _sz, _vp]),
    "lp_gemm_batch": (_b, [C.POINTER(BatchSpec), _i]),
    "lp_gemm_batch_workspace_bytes": (_sz, [C.POINTER(BatchSpec), _i]),
    "lp_gemm_batch_dev": (_i, [C.POINTER(BatchSpec), _i, _vp, _sz, _vp]),
    "lp_read_probe_dev": (_i, [_vp, _sz, _i, _i, _i, _vp, _vp]),
    "lp_last_error": (C.c_char_p, []),
    "lp_device_ok": (_i, []),
    "lp_device_info": (_i, [_vp, _vp, _vp, _vp]),
}

_lib = None


class LaplaceHipError(RuntimeError):
    pass


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built: run `python -m laplace_amd.build`")
        # PyTorch-ROCm ships its own libamdhip64 with the same soname as the
        # system one this library links. Whichever loads first serves both;
        # if the system runtime came first, torch's HIP would not initialise.
        # Load torch (when installed) first so the process has one runtime.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name, None)
            if fn is None:
                continue
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int, what: str) -> None:
    if rc != LP_OK:
        msg = lib().lp_last_error().decode(errors="replace")
        raise LaplaceHipError(f"{what}: {STATUS_NAMES.get(rc, rc)}: {msg}")
