"""Q4_K and Q6_K at one activation row on the flat super-block kernels (gemv_q4k_flat,
gemv_q6k_flat, lp_gemv.hip): a workgroup owns whole rows, a wave 64 consecutive
super-blocks of them whatever row they fall in, and each row's per-lane sums
are added afterwards. Against the oracle's gemm_int (dot_row_q4_k_int,
src/matmul_simd.cpp:226-283), and bit-identical between the single-call
path (x quantized inside the kernel) and the quantizer-fed path, at the
shapes the library routes to it (rows straddling waves; a last workgroup
with fewer rows; the quantizer-fed form at K >= 12288)."""
import numpy as np
import pytest

from hip_util import Q4_K, gemm_dev, normwise, synth_weights, synth_x

pytestmark = pytest.mark.gpu

TOL = 1e-4


@pytest.mark.parametrize("K,N", [(3584, 18944), (3584, 18901), (12288, 5000), (2304, 17000)])
def test_flat_q4k(orc, K, N):
    print(f"flat Q4_K K={K} N={N}", flush=True)
    import torch
    from hip_util import L, stream, to_dev, workspace
    from laplace_amd import _lib
    w = synth_weights(Q4_K, K, N, seed=K + N)
    x = synth_x(1, K, seed=K + 5, outliers=0.01)
    wd = to_dev(w)
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert L().lp_gemm_route(Q4_K, 1, K, N, wd.data_ptr()).decode() == "flat"
    y = gemm_dev(Q4_K, x, w, N)
    assert normwise(y, orc.gemm_int(Q4_K, x, w, N)) <= TOL
    xd = to_dev(x)
    ws, nb = workspace(1, K)
    y2 = torch.empty(N, dtype=torch.float32, device="cuda")
    _lib.check(L().lp_quantize_act_dev(xd.data_ptr(), 1, K, ws.data_ptr(), nb, stream()), "q")
    _lib.check(L().lp_gemm_q_dev(ws.data_ptr(), wd.data_ptr(), Q4_K, y2.data_ptr(), 1, K, N, stream()), "g")
    torch.cuda.synchronize()
    assert np.array_equal(y2.cpu().numpy().reshape(1, N).view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("K,N", [(18944, 1024), (14336, 1001), (32768, 300), (5120, 77)])
def test_flat_q6k(orc, K, N):
    """Q6_K at one activation row on gemv_q6k_flat (few rows of long K): rows
    of 56..128 super-blocks spread over the waves of one workgroup per CU,
    2-byte aligned 210-byte blocks per lane, against the oracle."""
    print(f"flat Q6_K K={K} N={N}", flush=True)
    import torch
    from hip_util import L, Q6_K, to_dev
    w = synth_weights(Q6_K, K, N, seed=K + 2 * N)
    x = synth_x(1, K, seed=K + 9, outliers=0.01)
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert L().lp_gemm_route(Q6_K, 1, K, N, to_dev(w).data_ptr()).decode() == "q6flat"
    y = gemm_dev(Q6_K, x, w, N)
    assert normwise(y, orc.gemm_int(Q6_K, x, w, N)) <= TOL
