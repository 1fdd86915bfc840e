"""lp_gemm_dev_noalloc (the entry point that allocates nothing: its
workspace is the library's static device array) against lp_gemm_dev with a
caller workspace: the same kernels on the same inputs, so the outputs are
bit-identical. Two calls in a row, the second on a smaller input, for the
routes that use the workspace (quantized activations; split-precision
planes for the prefill GEMM), plus the size limit."""
import ctypes as C

import numpy as np
import pytest

from hip_util import Q4_K, Q6_K, Q8_0, L, stream, synth_weights, synth_x, to_dev, torch_dev
from laplace_amd import _lib

pytestmark = pytest.mark.gpu


def _pair(t, M, K, N, seed):
    torch = torch_dev()
    w = synth_weights(t, K, N, seed=seed)
    x = synth_x(M, K, seed=seed + 1, outliers=0.01)
    xd, wd = to_dev(x), to_dev(w)
    route = L().lp_gemm_route(t, M, K, N, wd.data_ptr()).decode()
    y0 = torch.full((M * N,), float("nan"), dtype=torch.float32, device="cuda")
    y1 = torch.full((M * N,), float("nan"), dtype=torch.float32, device="cuda")
    nb = int(L().lp_act_workspace_bytes(M, K))
    ws = torch.empty(max(nb, 1), dtype=torch.uint8, device="cuda")
    _lib.check(L().lp_gemm_dev(xd.data_ptr(), wd.data_ptr(), t, y0.data_ptr(), M, K, N, ws.data_ptr(), nb,
                               stream()), "lp_gemm_dev")
    _lib.check(L().lp_gemm_dev_noalloc(xd.data_ptr(), wd.data_ptr(), t, y1.data_ptr(), M, K, N, stream()),
               "lp_gemm_dev_noalloc")
    torch.cuda.synchronize()
    return y0.cpu().numpy(), y1.cpu().numpy(), route


@pytest.mark.parametrize("t,big,small", [
    (Q4_K, (96, 2048, 512), (8, 1024, 256)),        # GEMM planes, then the int8 MFMA kernel
    (Q4_K, (16, 4096, 768), (3, 1024, 256)),        # small-M MFMA, then the dot4 GEMV
    (Q6_K, (12, 2048, 640), (2, 1024, 256)),
    # K-split Q6_K row quads: partial sums in the workspace's tail region
    (Q6_K, (8, 18944, 512), (3, 8448, 256)),
    (Q8_0, (40, 1024, 384), (5, 512, 128)),         # row chunks
], ids=["q4k_gemm", "q4k_small", "q6k", "q6k_rq_split", "q80"])
def test_noalloc_matches_workspace_entry(t, big, small):
    for i, (M, K, N) in enumerate((big, small)):
        y0, y1, route = _pair(t, M, K, N, seed=100 * t + i)
        if t == Q6_K and K > 4096 and 3 <= M <= 8:
            assert route == "q6rq", (M, K, N, route)
        assert np.isfinite(y0).all()
        assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32)), (t, M, K, N)


def test_noalloc_rejects_oversized_workspace():
    """A shape whose workspace exceeds the 8 MiB scratch is refused before
    any launch, with the reason in lp_last_error."""
    M, K, N = 2048, 4096, 256
    assert int(L().lp_act_workspace_bytes(M, K)) > (8 << 20)
    torch = torch_dev()
    xd = torch.zeros(M * K, dtype=torch.float32, device="cuda")
    wd = torch.zeros((K // 256) * 144 * N, dtype=torch.uint8, device="cuda")
    yd = torch.zeros(M * N, dtype=torch.float32, device="cuda")
    rc = L().lp_gemm_dev_noalloc(xd.data_ptr(), wd.data_ptr(), Q4_K, yd.data_ptr(), M, K, N, stream())
    assert rc == 2 and b"no-alloc scratch" in L().lp_last_error()
