"""Helpers for the GPU tests: device buffers through torch, calls through
the C ABI of liblaplace_hip.so, seeded synthetic weights.

Torch is used only to hold device memory and the stream; every computation
under test runs in the HIP library.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from laplace_amd import _lib
from laplace_amd.matmul import row_bytes

Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14
TYPES = (Q8_0, Q4_0, Q4_K, Q6_K)
NAMES = {Q4_0: "Q4_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q6_K: "Q6_K"}


def L():
    return _lib.lib()


def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    return torch


def to_dev(a: np.ndarray):
    torch = torch_dev()
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def stream():
    torch = torch_dev()
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def workspace(M: int, K: int):
    torch = torch_dev()
    nb = int(L().lp_act_workspace_bytes(M, K))
    return torch.empty(nb, dtype=torch.uint8, device="cuda"), nb


def quantize_dev(x: np.ndarray):
    """(d, sum, sums16, qs) of x[M, K] computed on the GPU."""
    torch = torch_dev()
    M, K = x.shape
    xd = to_dev(x.astype(np.float32))
    ws, nb = workspace(M, K)
    _lib.check(L().lp_quantize_act_dev(xd.data_ptr(), M, K, ws.data_ptr(), nb, stream()),
               "lp_quantize_act_dev")
    nbk = M * (K // 32)
    d = torch.empty(nbk, dtype=torch.float32, device="cuda")
    s = torch.empty(nbk, dtype=torch.float32, device="cuda")
    s16 = torch.empty(nbk, dtype=torch.int32, device="cuda")
    qs = torch.empty(M * K, dtype=torch.int8, device="cuda")
    _lib.check(L().lp_act_unpack_dev(ws.data_ptr(), M, K, d.data_ptr(), s.data_ptr(),
                                     s16.data_ptr(), qs.data_ptr(), stream()), "lp_act_unpack_dev")
    torch.cuda.synchronize()
    return (d.cpu().numpy().reshape(M, -1), s.cpu().numpy().reshape(M, -1),
            s16.cpu().numpy().reshape(M, -1), qs.cpu().numpy().reshape(M, K))


def gemm_dev(t: int, x: np.ndarray, w: np.ndarray, N: int) -> np.ndarray:
    torch = torch_dev()
    x = np.ascontiguousarray(x, np.float32)
    if x.ndim == 1:
        x = x[None]
    M, K = x.shape
    xd, wd = to_dev(x), to_dev(w)
    y = torch.empty(M * N, dtype=torch.float32, device="cuda")
    ws, nb = workspace(M, K)
    _lib.check(L().lp_gemm_dev(xd.data_ptr(), wd.data_ptr(), t, y.data_ptr(), M, K, N,
                               ws.data_ptr(), nb, stream()), "lp_gemm_dev")
    torch.cuda.synchronize()
    return y.cpu().numpy().reshape(M, N)


def block_sums_dev(t: int, x: np.ndarray, w: np.ndarray, N: int) -> np.ndarray:
    torch = torch_dev()
    M, K = x.shape
    xd, wd = to_dev(x.astype(np.float32)), to_dev(w)
    ws, nb = workspace(M, K)
    _lib.check(L().lp_quantize_act_dev(xd.data_ptr(), M, K, ws.data_ptr(), nb, stream()), "q")
    S = K // 16 if t == Q6_K else K // 32
    out = torch.empty(M * N * S, dtype=torch.int32, device="cuda")
    _lib.check(L().lp_block_sums_dev(ws.data_ptr(), wd.data_ptr(), t, out.data_ptr(), M, K, N,
                                     stream()), "lp_block_sums_dev")
    torch.cuda.synchronize()
    return out.cpu().numpy().reshape(M, N, S)


def synth_weights(t: int, K: int, N: int, seed: int) -> np.ndarray:
    """Seeded GGUF blocks with the distributions of BASELINE.json's configs:
    codes uniform, fp16 scales |N(0,1)| * 0.01 (Q4_0: * 0.02), K-quant
    6-bit scale/min fields uniform (uniform bytes), Q6_K int8 scales
    uniform in [-32, 31]."""
    rng = np.random.default_rng(seed)
    nbytes = row_bytes(t, K) * N
    w = rng.integers(0, 256, nbytes, dtype=np.uint8)
    if t == Q8_0:
        b = w.reshape(-1, 34)
        b[:, 2:] = rng.integers(-127, 128, (b.shape[0], 32), dtype=np.int8).view(np.uint8)
        b[:, 0:2] = (np.abs(rng.standard_normal(b.shape[0])) * 0.01).astype(np.float16).view(np.uint8).reshape(-1, 2)
    elif t == Q4_0:
        b = w.reshape(-1, 18)
        b[:, 0:2] = (np.abs(rng.standard_normal(b.shape[0])) * 0.02).astype(np.float16).view(np.uint8).reshape(-1, 2)
    elif t == Q4_K:
        b = w.reshape(-1, 144)
        b[:, 0:2] = (np.abs(rng.standard_normal(b.shape[0])) * 0.01).astype(np.float16).view(np.uint8).reshape(-1, 2)
        b[:, 2:4] = (np.abs(rng.standard_normal(b.shape[0])) * 0.01).astype(np.float16).view(np.uint8).reshape(-1, 2)
    elif t == Q6_K:
        b = w.reshape(-1, 210)
        b[:, 192:208] = rng.integers(-32, 32, (b.shape[0], 16), dtype=np.int8).view(np.uint8)
        b[:, 208:210] = (np.abs(rng.standard_normal(b.shape[0])) * 0.01).astype(np.float16).view(np.uint8).reshape(-1, 2)
    return w


def synth_x(M: int, K: int, seed: int, outliers: float = 0.0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K)).astype(np.float32)
    if outliers:
        x[rng.random((M, K)) < outliers] *= 20.0
    return x


def normwise(y, ref) -> float:
    """max |y - ref| / max |ref| (the reference's GPU tolerance form,
    tests/test_metal.cpp:200-203)."""
    den = float(np.abs(ref).max())
    return float(np.abs(y - ref).max()) / (den if den > 0 else 1.0)


def moe_dev(t: int, x: np.ndarray, w: np.ndarray, idx: np.ndarray, n_experts: int, N: int,
            multi: bool) -> np.ndarray:
    """Grouped MoE on device pointers: y[T*topk, N]."""
    torch = torch_dev()
    T, topk = idx.shape
    x = np.ascontiguousarray(x, np.float32)
    K = x.shape[1]
    xd, wd = to_dev(x), to_dev(w)
    idd = to_dev(np.ascontiguousarray(idx, np.int32))
    y = torch.full((T * topk * N,), float("nan"), dtype=torch.float32, device="cuda")
    nb = int(L().lp_moe_workspace_bytes(T, topk, n_experts, K, 1 if multi else 0))
    ws = torch.empty(max(nb, 1), dtype=torch.uint8, device="cuda")
    _lib.check(L().lp_moe_grouped_dev(xd.data_ptr(), 1 if multi else 0, idd.data_ptr(), wd.data_ptr(), t,
                                      y.data_ptr(), T, topk, n_experts, K, N, ws.data_ptr(), nb,
                                      stream()), "lp_moe_grouped_dev")
    torch.cuda.synchronize()
    return y.cpu().numpy().reshape(T * topk, N)


def routing(T: int, topk: int, n_experts: int, seed: int) -> np.ndarray:
    """Top-k expert choice per token: distinct experts, uniform without
    replacement (the MoE benchmark configuration's routing)."""
    rng = np.random.default_rng(seed)
    return np.stack([rng.choice(n_experts, topk, replace=False) for _ in range(T)]).astype(np.int32)
