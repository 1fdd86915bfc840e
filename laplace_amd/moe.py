"""Grouped MoE dispatch over the gfx950 C ABI.

The reference's MoE layer (src/arch_gemma4.cpp:507-641) loops over tokens
and calls ``fused_moe_gemm_idx`` (gate/up, one activation row per token,
:604) and ``fused_moe_gemm_multi`` (down, one activation row per selected
expert, :626) once per token. :func:`moe_grouped` takes the whole batch of
T tokens at once: pair ``p = t*topk + j`` uses expert ``topk_idx[t, j]`` and
writes ``y[p]``, with the same values the per-token calls produce
(src/matmul.cpp:456-500). On the device the pairs are grouped by expert so
each expert's weights are streamed once per group of pairs.
"""
from __future__ import annotations

import numpy as np

from ._lib import LP_UNSUPPORTED, check, lib
from .matmul import Tensor, _is_torch, _ptr, _stream_ptr


def moe_workspace_bytes(T: int, topk: int, n_experts: int, K: int, multi: bool) -> int:
    return int(lib().lp_moe_workspace_bytes(T, topk, n_experts, K, 1 if multi else 0))


def moe_grouped(x, w: Tensor, y, topk_idx, T: int, topk: int, n_experts: int, K: int, N: int,
                multi: bool = False, ws=None) -> None:
    """y[(t*topk + j)*N + n] = dot(x_row, expert topk_idx[t, j] row n).

    x_row is x[t] (multi=False, x is [T, K]) or x[t*topk + j] (multi=True, x is
    [T*topk, K]). ``w.data`` stacks n_experts weight matrices of N rows each.
    numpy arguments take the synchronous host path; torch CUDA tensors the
    stream-ordered device path (``ws`` optional workspace tensor).
    """
    m = 1 if multi else 0
    if _is_torch(x):
        import torch
        nb = moe_workspace_bytes(T, topk, n_experts, K, multi)
        if ws is None:
            ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=x.device)
        rc = lib().lp_moe_grouped_dev(_ptr(x), m, _ptr(topk_idx), _ptr(w.data), int(w.type), _ptr(y),
                                      T, topk, n_experts, K, N, _ptr(ws), ws.numel(), _stream_ptr())
        if rc == LP_UNSUPPORTED:
            raise NotImplementedError(lib().lp_last_error().decode())
        check(rc, "lp_moe_grouped_dev")
        return
    idx = np.ascontiguousarray(topk_idx, dtype=np.int32)
    assert x.dtype == np.float32 and y.dtype == np.float32
    if not lib().lp_moe_grouped(_ptr(x), m, idx.ctypes.data, _ptr(w.data), int(w.type), _ptr(y),
                                T, topk, n_experts, K, N):
        raise ValueError(lib().lp_last_error().decode())


def moe_ffn(x, router: Tensor, router_scale, pre_norm, rms_eps: float, gate_up: Tensor, down: Tensor,
            down_scale, n_experts: int, top_k: int, inter: int, out=None, return_routing: bool = False):
    """Gemma4Arch::moe_ffn (src/arch_gemma4.cpp:507-641) for all rows of x
    [T, H] on the device (torch CUDA tensors): router norm/scale/matmul,
    softmax, top-k, renormalised weights, expert norm, grouped gate/up and
    down GEMVs, GeGLU, weighted sum with the per-expert down scales."""
    import torch
    T, H = x.shape
    if out is None:
        out = torch.empty((T, H), dtype=torch.float32, device=x.device)
    idx = torch.empty((T, top_k), dtype=torch.int32, device=x.device)
    wts = torch.empty((T, top_k), dtype=torch.float32, device=x.device)
    nb = int(lib().lp_moe_ffn_workspace_bytes(T, H, n_experts, top_k, inter, int(router.type)))
    ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=x.device)
    rc = lib().lp_moe_ffn_dev(_ptr(x), T, H, _ptr(router.data), int(router.type), _ptr(router_scale),
                              _ptr(pre_norm), float(rms_eps), _ptr(gate_up.data), int(gate_up.type),
                              _ptr(down.data), int(down.type), _ptr(down_scale), n_experts, top_k, inter,
                              _ptr(out), _ptr(idx), _ptr(wts), _ptr(ws), ws.numel(), _stream_ptr())
    if rc == LP_UNSUPPORTED:
        raise NotImplementedError(lib().lp_last_error().decode())
    check(rc, "lp_moe_ffn_dev")
    return (out, idx, wts) if return_routing else out


__all__ = ["moe_grouped", "moe_workspace_bytes", "moe_ffn"]
