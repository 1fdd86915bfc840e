"""Host-side mirror of the reference's matmul front-end (src/matmul.h:18-54)
over the gfx950 C ABI.

Same entry points, argument meaning and output layout as the reference:

  matmul_row(x, w, y, K, N)            y[j] = sum_k x[k] W[k, j]
  matmul_rows(x, w, y, M, K, N)        y[m*N + j], x[m*K + k]
  fused_moe_gemm_idx(x, w, y, idx, n, K, N)    y[k*N + j] = expert idx[k] on x
  fused_moe_gemm_multi(x, w, y, idx, n, K, N)  y[k*N + j] = expert idx[k] on x[k]
  matmul_register_weights(buf)         device residency for a weight region
  dequantize(w, dst, n)                dst[i] = element i of w as fp32

``x``/``y`` are either numpy float32 arrays (host path: the C ABI stages
them through pinned memory and returns synchronously, like the reference)
or torch tensors on the GPU (device path: stream-ordered on torch's current
stream, no host round trip). A weight is a :class:`Tensor` whose ``data``
holds the GGUF blocks, as a numpy uint8 array or a uint8 device tensor.

Where the reference falls back to its scalar CPU code for a type the SIMD
back-end does not handle (src/matmul.cpp:426-432), this package raises
:class:`NotImplementedError`: it has no CPU path of its own.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from enum import IntEnum

import numpy as np

from ._lib import LP_OK, LP_UNSUPPORTED, LaplaceHipError, check, lib


class GGMLType(IntEnum):
    """src/tensor.h:11-34 (values are the GGUF type ids)."""
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q8_1 = 9
    Q2_K = 10
    Q3_K = 11
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    Q8_K = 15
    BF16 = 30


_BPB = {GGMLType.F32: 4, GGMLType.F16: 2, GGMLType.BF16: 2, GGMLType.Q4_0: 18,
        GGMLType.Q4_1: 20, GGMLType.Q5_0: 22, GGMLType.Q5_1: 24, GGMLType.Q8_0: 34,
        GGMLType.Q8_1: 36, GGMLType.Q2_K: 84, GGMLType.Q3_K: 110, GGMLType.Q4_K: 144,
        GGMLType.Q5_K: 176, GGMLType.Q6_K: 210}
_EPB = {GGMLType.F32: 1, GGMLType.F16: 1, GGMLType.BF16: 1}

# int8-activation types (gemm_int in the reference's SIMD back-end, src/matmul_simd.cpp:484-488)
GPU_TYPES = (GGMLType.Q8_0, GGMLType.Q4_0, GGMLType.Q5_0, GGMLType.Q4_K, GGMLType.Q6_K)
# fp32-activation types (its fp32 dots, :489-493, and the scalar gemm_fallback,
# src/matmul.cpp:331-353)
GPU_FP32_TYPES = (GGMLType.F32, GGMLType.F16, GGMLType.BF16, GGMLType.Q2_K, GGMLType.Q3_K,
                  GGMLType.Q5_K)


def bytes_per_block(t: int) -> int:
    """src/tensor.h:41-67 (0 for types without a block size)."""
    return _BPB.get(GGMLType(t), 0)


def elements_per_block(t: int) -> int:
    """src/tensor.h:69-100."""
    t = GGMLType(t)
    if t in _EPB:
        return 1
    if t in (GGMLType.Q4_0, GGMLType.Q4_1, GGMLType.Q5_0, GGMLType.Q5_1, GGMLType.Q8_0,
             GGMLType.Q8_1):
        return 32
    if t in (GGMLType.Q2_K, GGMLType.Q3_K, GGMLType.Q4_K, GGMLType.Q5_K, GGMLType.Q6_K,
             GGMLType.Q8_K):
        return 256
    return 0


def row_bytes(t: int, K: int) -> int:
    """Bytes of one weight row: K / epb * bpb (src/matmul_simd.cpp:482)."""
    epb = elements_per_block(t)
    return (K // epb) * bytes_per_block(t) if epb else 0


@dataclass
class Tensor:
    """The parts of the reference's Tensor view (src/tensor.h:130-163) the
    matmul path reads: type, dims ([K, N], dims[0] innermost) and data."""
    type: int
    dims: tuple
    data: object
    name: str = "w"
    extra: dict = field(default_factory=dict)


def _is_torch(a) -> bool:
    return type(a).__module__.startswith("torch")


def _ptr(a) -> int:
    if _is_torch(a):
        return a.data_ptr()
    return a.ctypes.data


def _stream_ptr():
    import torch
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _workspace(M: int, K: int, device):
    import torch
    nbytes = int(lib().lp_act_workspace_bytes(M, K))
    return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device), nbytes


def matmul_rows(x, w: Tensor, y, M: int, K: int, N: int) -> None:
    """src/matmul.cpp:408-433: int8-activation semantics for GPU_TYPES, the
    scalar path's fp32-activation semantics for GPU_FP32_TYPES."""
    if _is_torch(x):
        ws, nb = _workspace(M, K, x.device)
        rc = lib().lp_gemm_dev(_ptr(x), _ptr(w.data), int(w.type), _ptr(y), M, K, N,
                               _ptr(ws), nb, _stream_ptr())
        if rc == LP_UNSUPPORTED:
            raise NotImplementedError(lib().lp_last_error().decode())
        check(rc, "lp_gemm_dev")
        return
    assert x.dtype == np.float32 and y.dtype == np.float32
    ok = lib().lp_gemm(_ptr(x), _ptr(w.data), int(w.type), _ptr(y), M, K, N)
    if not ok:
        raise NotImplementedError(f"lp_gemm: {lib().lp_last_error().decode()}")


def matmul_row(x, w: Tensor, y, K: int, N: int) -> None:
    """src/matmul.cpp:435-437."""
    matmul_rows(x, w, y, 1, K, N)


def matmul_lm_head(x, w: Tensor, y, M: int, K: int, N: int) -> None:
    """src/matmul.cpp:439-444: the vocabulary projection goes through the same GPU path."""
    matmul_rows(x, w, y, M, K, N)


def matmul_register_weights(buf: np.ndarray) -> None:
    """src/matmul.cpp:446-448: make a host weight region device-resident."""
    check(lib().lp_register_weights(_ptr(buf), buf.nbytes), "lp_register_weights")


def _moe(x, w: Tensor, y, expert_idx, n_experts: int, K: int, N: int, multi: bool) -> None:
    if _is_torch(x):
        raise TypeError("device MoE goes through laplace_amd.moe.moe_grouped (T = 1)")
    idx = np.ascontiguousarray(expert_idx, dtype=np.int32)
    fn = lib().lp_moe_gemv_multi if multi else lib().lp_moe_gemv
    if not fn(_ptr(x), _ptr(w.data), int(w.type), idx.ctypes.data, n_experts, _ptr(y), K, N):
        raise NotImplementedError(lib().lp_last_error().decode())


def fused_moe_gemm_idx(x, w: Tensor, y, expert_idx, n_experts: int, K: int, N: int) -> None:
    """src/matmul.cpp:456-477."""
    _moe(x, w, y, expert_idx, n_experts, K, N, False)


def fused_moe_gemm_multi(x, w: Tensor, y, expert_idx, n_experts: int, K: int, N: int) -> None:
    """src/matmul.cpp:479-500."""
    _moe(x, w, y, expert_idx, n_experts, K, N, True)


def dequantize(w: Tensor, dst, n: int) -> None:
    """src/matmul.cpp:504-675: the first n elements of w as fp32 into dst."""
    if _is_torch(dst):
        rc = lib().lp_dequantize_dev(_ptr(w.data), int(w.type), _ptr(dst), n, _stream_ptr())
    else:
        assert dst.dtype == np.float32
        rc = lib().lp_dequantize(_ptr(w.data), int(w.type), _ptr(dst), n)
    if rc == LP_UNSUPPORTED:
        raise NotImplementedError(lib().lp_last_error().decode())
    check(rc, "lp_dequantize")


def matmul_gemm_batch(specs) -> bool:
    """src/matmul.h:46-54, src/matmul.cpp:450-454: each spec (x, w, y, K, N)
    is an M = 1 matmul. One C-ABI call for the whole batch (lp_gemm_batch /
    lp_gemm_batch_dev): consecutive Q4_K specs sharing x and K run as one
    launch. All x/y are numpy arrays (host path) or all torch GPU tensors."""
    from ._lib import BatchSpec
    specs = list(specs)
    if not specs:
        return True
    arr = (BatchSpec * len(specs))()
    dev = _is_torch(specs[0][0])
    for i, (x, w, y, K, N) in enumerate(specs):
        if _is_torch(x) != dev or _is_torch(y) != dev:
            raise TypeError("a batch is all host arrays or all device tensors")
        if not dev:
            assert x.dtype == np.float32 and y.dtype == np.float32
        arr[i] = BatchSpec(_ptr(x), _ptr(w.data), int(w.type), _ptr(y), K, N)
    L = lib()
    if dev:
        import torch
        nb = int(L.lp_gemm_batch_workspace_bytes(arr, len(specs)))
        ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=specs[0][0].device)
        rc = L.lp_gemm_batch_dev(arr, len(specs), ws.data_ptr(), nb, _stream_ptr())
        if rc == LP_UNSUPPORTED:
            raise NotImplementedError(L.lp_last_error().decode())
        check(rc, "lp_gemm_batch_dev")
        return True
    if not L.lp_gemm_batch(arr, len(specs)):
        raise NotImplementedError(f"lp_gemm_batch: {L.lp_last_error().decode()}")
    return True


def quantize_act(x: np.ndarray):
    """Host-pointer quantizer: (d, sum, sum_lo, sum_hi, qs) of x[M, K]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.ndim == 1:
        x = x[None, :]
    M, K = x.shape
    nb = K // 32
    d = np.zeros((M, nb), np.float32)
    s = np.zeros((M, nb), np.float32)
    lo = np.zeros((M, nb), np.int16)
    hi = np.zeros((M, nb), np.int16)
    qs = np.zeros((M, K), np.int8)
    check(lib().lp_quantize_act(_ptr(x), M, K, _ptr(d), _ptr(s), _ptr(lo), _ptr(hi), _ptr(qs)),
          "lp_quantize_act")
    return d, s, lo, hi, qs


__all__ = ["GGMLType", "Tensor", "matmul_row", "matmul_rows", "matmul_lm_head",
           "matmul_register_weights", "fused_moe_gemm_idx", "fused_moe_gemm_multi",
           "matmul_gemm_batch", "quantize_act", "dequantize", "bytes_per_block", "elements_per_block",
           "row_bytes", "GPU_TYPES", "GPU_FP32_TYPES", "LaplaceHipError", "LP_OK"]
