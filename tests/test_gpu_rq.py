"""Q4_K at 2..8 activation rows on the row-quad int8 MFMA kernel (lp_rq.hip:
4x4x4 int8 blocks, a weight row quad per wave, K <= 4096) against the
oracle's gemm_int (dot_row_q4_k_int, src/matmul_simd.cpp:226-283): every M
of both token groups, K from one super-block to sixteen (lanes of absent
super-blocks must add nothing), ragged N (a partial last row quad, waves
with several row quads, waves with none), activation outliers."""
import numpy as np
import pytest

from hip_util import Q4_K, gemm_dev, normwise, synth_weights, synth_x

pytestmark = pytest.mark.gpu

TOL = 1e-4


# (M, N) where the library routes Q4_K to this kernel (rq_preferred): M = 4 at
# any N, M = 3 from 12288 rows, M = 5..8 from 2048 rows
CASES = [(4, 1), (4, 6), (4, 333), (4, 5000), (3, 12290), (5, 2048), (6, 2051), (7, 3001), (8, 4999)]


@pytest.mark.parametrize("K", [256, 512, 768, 1280, 2048, 3584, 4096])
@pytest.mark.parametrize("M,N", CASES)
def test_rq_q4k(orc, K, N, M):
    print(f"rq Q4_K M={M} K={K} N={N}", flush=True)
    import torch
    from hip_util import L, to_dev
    w = synth_weights(Q4_K, K, N, seed=K + 3 * N + M)
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert L().lp_gemm_route(Q4_K, M, K, N, to_dev(w).data_ptr()).decode() == "rq"
    x = synth_x(M, K, seed=M * 5 + 1, outliers=0.01)
    y = gemm_dev(Q4_K, x, w, N)
    ref = orc.gemm_int(Q4_K, x, w, N)
    assert np.isfinite(y).all()
    assert normwise(y, ref) <= TOL


def test_rq_q4k_config3(orc):
    """Config 3's Q4_K gate/up (18944 x 3584) at M = 4 and 8, on a sample
    of 512 rows checked against the oracle (the GPU computes all rows)."""
    K, N = 3584, 18944
    w = synth_weights(Q4_K, K, N, seed=99)
    rb = K // 256 * 144
    rows = np.sort(np.random.default_rng(5).choice(N, 512, replace=False))
    ws = np.concatenate([w[r * rb:(r + 1) * rb] for r in rows])
    for M in (4, 8):
        print(f"rq config3 M={M}", flush=True)
        x = synth_x(M, K, seed=M)
        y = gemm_dev(Q4_K, x, w, N)
        assert normwise(y[:, rows], orc.gemm_int(Q4_K, x, ws, len(rows))) <= TOL
