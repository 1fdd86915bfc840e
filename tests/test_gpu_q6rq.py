"""Q6_K at 3..8 activation rows (1..2 when K <= 4096) on the row-quad int8 MFMA kernel
(lp_q6rq.hip: 4x4x4 int8 blocks, a weight row quad per wave, K in chunks of
16 super-blocks) against the oracle's gemm_int (dot_row_q6_k_int,
src/matmul_simd.cpp:285-342): both token groups, K from one super-block
(lanes of absent super-blocks must add nothing) through one full chunk to
several chunks with a ragged last one (the coalesced chunk-copy path),
2-byte aligned rows (odd super-block counts), ragged N (a partial last row
quad, workgroups with idle waves), activation outliers."""
import numpy as np
import pytest

from hip_util import Q6_K, gemm_dev, normwise, synth_weights, synth_x

pytestmark = pytest.mark.gpu

TOL = 1e-4

CASES = [(3, 5), (4, 1), (4, 333), (5, 130), (6, 17), (7, 1001), (8, 4096)]


@pytest.mark.parametrize("K", [256, 1280, 4096, 4352, 8448, 18944])
@pytest.mark.parametrize("M,N", CASES)
def test_q6rq(orc, K, N, M):
    print(f"q6rq Q6_K M={M} K={K} N={N}", flush=True)
    from hip_util import L, to_dev
    w = synth_weights(Q6_K, K, N, seed=K + 7 * N + M)
    assert L().lp_gemm_route(Q6_K, M, K, N, to_dev(w).data_ptr()).decode() == "q6rq"
    x = synth_x(M, K, seed=M * 3 + 2, outliers=0.01)
    y = gemm_dev(Q6_K, x, w, N)
    ref = orc.gemm_int(Q6_K, x, w, N)
    assert np.isfinite(y).all()
    assert normwise(y, ref) <= TOL


@pytest.mark.parametrize("M,N", [(1, 7), (1, 4096), (2, 130), (2, 1001)])
@pytest.mark.parametrize("K", [256, 3584, 4096])
def test_q6rq_one_two_rows(orc, K, N, M):
    """One and two activation rows in one chunk (K <= 4096) also run here."""
    print(f"q6rq Q6_K M={M} K={K} N={N}", flush=True)
    from hip_util import L, to_dev
    w = synth_weights(Q6_K, K, N, seed=K + 5 * N + M)
    assert L().lp_gemm_route(Q6_K, M, K, N, to_dev(w).data_ptr()).decode() == "q6rq"
    x = synth_x(M, K, seed=M * 7 + 3, outliers=0.01)
    y = gemm_dev(Q6_K, x, w, N)
    assert normwise(y, orc.gemm_int(Q6_K, x, w, N)) <= TOL


def test_q6rq_config3(orc):
    """Config 3's Q6_K down projection (3584 x 18944) at M = 4 and 8, on a
    sample of 256 rows checked against the oracle (the GPU computes all)."""
    K, N = 18944, 3584
    w = synth_weights(Q6_K, K, N, seed=98)
    rb = K // 256 * 210
    rows = np.sort(np.random.default_rng(6).choice(N, 256, replace=False))
    ws = np.concatenate([w[r * rb:(r + 1) * rb] for r in rows])
    for M in (4, 8):
        print(f"q6rq config3 M={M}", flush=True)
        x = synth_x(M, K, seed=M + 40)
        y = gemm_dev(Q6_K, x, w, N)
        assert normwise(y[:, rows], orc.gemm_int(Q6_K, x, ws, len(rows))) <= TOL


def test_q6rq_unsplit_long_k(orc):
    """Long K whose partial sums exceed the workspace's scratch (8 rows x
    5 chunks x 13200 outputs > 2 MiB): the chunk loop with coalesced chunk
    copies; a sample of 128 rows against the oracle."""
    K, N, M = 18944, 13200, 8
    w = synth_weights(Q6_K, K, N, seed=97)
    rb = K // 256 * 210
    rows = np.sort(np.random.default_rng(8).choice(N, 128, replace=False))
    ws = np.concatenate([w[r * rb:(r + 1) * rb] for r in rows])
    x = synth_x(M, K, seed=77)
    y = gemm_dev(Q6_K, x, w, N)
    assert normwise(y[:, rows], orc.gemm_int(Q6_K, x, ws, len(rows))) <= TOL
