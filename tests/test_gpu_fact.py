"""GEMV with fp32 activations for F32, F16, BF16 (the reference's fp32 dots,
src/matmul_simd.cpp:489-493) and Q2_K, Q3_K, Q5_K (its scalar fallback,
src/matmul.cpp:331-353), against the oracle's restatement of
gemm_scalar<dot_row_*> (src/matmul.cpp:63-314). The GPU reassociates the fp32
sums, so the bar is normwise 2e-5 (fp32 rounding over K <= 4096), not bit
equality. Q5_0, which the reference's int8 back-end takes
(src/matmul_simd.cpp:486), is tested on the int8 path against gemm_int."""
import numpy as np
import pytest

from hip_util import L, normwise, to_dev, stream

pytestmark = pytest.mark.gpu

F32, F16, Q5_0, Q2_K, Q3_K, Q5_K, BF16 = 0, 1, 6, 10, 11, 13, 30
FACT = {"F32": F32, "F16": F16, "BF16": BF16, "Q2_K": Q2_K, "Q3_K": Q3_K, "Q5_K": Q5_K}
BLOCK = {Q5_0: (32, 22, [0]), Q2_K: (256, 84, [80, 82]), Q3_K: (256, 110, [108]), Q5_K: (256, 176, [0, 2])}
TOL = 2e-5


def fact_weights(t, K, N, seed):
    """Finite weights: fp32/fp16/bf16 from N(0,1) * 0.05; quantized blocks of
    uniform bytes with fp16 scales |N(0,1)| * 0.01."""
    rng = np.random.default_rng(seed)
    if t in (F32, F16, BF16):
        v = (rng.standard_normal(K * N) * 0.05).astype(np.float32)
        if t == F32:
            return v.view(np.uint8).copy()
        if t == F16:
            return v.astype(np.float16).view(np.uint8).copy()
        return (v.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).copy()
    epb, bpb, scales = BLOCK[t]
    nblk = K // epb * N
    w = rng.integers(0, 256, nblk * bpb, dtype=np.uint8).reshape(nblk, bpb)
    for off in scales:
        w[:, off:off + 2] = (np.abs(rng.standard_normal(nblk)) * 0.01).astype(np.float16).view(np.uint8).reshape(-1, 2)
    return w.reshape(-1)


def gemm_dev(t, x, w, N):
    import torch
    M, K = x.shape
    xd, wd = to_dev(x), to_dev(w)
    y = torch.empty(M * N, dtype=torch.float32, device="cuda")
    from hip_util import workspace
    ws, nb = workspace(M, K)
    rc = L().lp_gemm_dev(xd.data_ptr(), wd.data_ptr(), t, y.data_ptr(), M, K, N, ws.data_ptr(), nb, stream())
    assert rc == 0, L().lp_last_error().decode()
    torch.cuda.synchronize()
    return y.cpu().numpy().reshape(M, N)


@pytest.mark.parametrize("name", list(FACT))
@pytest.mark.parametrize("K,N,M", [(256, 7, 1), (512, 65, 3), (2816, 128, 1), (4096, 300, 5), (1024, 64, 8)])
def test_fact_gemv_matches_scalar_path(orc, name, K, N, M):
    t = FACT[name]
    w = fact_weights(t, K, N, seed=K + N + t)
    x = np.random.default_rng(M + K).standard_normal((M, K)).astype(np.float32)
    ref = orc.gemm_scalar(t, x, w, N)
    y = gemm_dev(t, x, w, N)
    assert np.isfinite(y).all()
    assert normwise(y, ref) <= TOL


@pytest.mark.parametrize("name", ["F32", "Q5_K", "Q3_K"])
def test_fact_host_api(orc, name):
    """The drop-in lp_gemm takes these types (the reference would have run its
    scalar fallback): same result as the device entry."""
    t = FACT[name]
    K, N, M = 2816 if t == F32 else 2048, 96, 2
    w = fact_weights(t, K, N, seed=7 + t)
    x = np.random.default_rng(9).standard_normal((M, K)).astype(np.float32)
    y = np.zeros((M, N), np.float32)
    assert L().lp_gemm(x.ctypes.data, w.ctypes.data, t, y.ctypes.data, M, K, N)
    assert np.array_equal(y, gemm_dev(t, x, w, N))
    assert normwise(y, orc.gemm_scalar(t, x, w, N)) <= TOL
    L().lp_release_weights()


def test_fact_types_unsupported_where_int8_only():
    """Quantized-activation and grouped-MoE entries report LP_UNSUPPORTED for
    these types, so the caller's per-expert fallback (src/matmul.cpp:467-479)
    runs each expert through lp_gemm."""
    import torch
    from laplace_amd import _lib
    K, N = 512, 16
    w = to_dev(fact_weights(Q5_K, K, N, seed=1))
    ws = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    y = torch.zeros(N, dtype=torch.float32, device="cuda")
    assert L().lp_gemm_q_dev(ws.data_ptr(), w.data_ptr(), Q5_K, y.data_ptr(), 1, K, N, stream()) == _lib.LP_UNSUPPORTED
    x = np.zeros(K, np.float32)
    idx = np.array([0], np.int32)
    yh = np.zeros(N, np.float32)
    wh = fact_weights(Q5_K, K, N, seed=1)
    assert not L().lp_moe_gemv(x.ctypes.data, wh.ctypes.data, Q5_K, idx.ctypes.data, 1, yh.ctypes.data, K, N)
    # K not a whole number of super-blocks: unsupported (the scalar path keeps it)
    assert not L().lp_gemm(x.ctypes.data, wh.ctypes.data, Q5_K, yh.ctypes.data, 1, 320, N)


@pytest.mark.parametrize("K,N,M", [(32, 5, 1), (512, 65, 3), (2048, 300, 5), (4096, 64, 8)])
def test_q5_0_int8_path(orc, K, N, M):
    """Q5_0 (dot_row_q5_0_int_neon, src/matmul_simd.cpp:184-224): int8
    activations, exact per-block integer sums of (code - 16) * q; against the
    oracle's gemm_int, and bit-identical to quantize + lp_gemm_q_dev."""
    import torch
    from hip_util import workspace
    w = fact_weights(Q5_0, K, N, seed=K + N)
    x = np.random.default_rng(M + K).standard_normal((M, K)).astype(np.float32)
    x[0, :8] = [127.0, -127.0, 0.5, -0.5, 1.5, 2.5, 0.0, 3.0]
    y = gemm_dev(Q5_0, x, w, N)
    assert normwise(y, orc.gemm_int(Q5_0, x, w, N)) <= 1e-4
    xd, wd = to_dev(x), to_dev(w)
    ws, nb = workspace(M, K)
    y2 = torch.empty(M * N, dtype=torch.float32, device="cuda")
    assert L().lp_quantize_act_dev(xd.data_ptr(), M, K, ws.data_ptr(), nb, stream()) == 0
    assert L().lp_gemm_q_dev(ws.data_ptr(), wd.data_ptr(), Q5_0, y2.data_ptr(), M, K, N, stream()) == 0
    torch.cuda.synchronize()
    assert np.array_equal(y2.cpu().numpy().reshape(M, N).view(np.uint32), y.view(np.uint32))
