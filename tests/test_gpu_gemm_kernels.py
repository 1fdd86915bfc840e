"""The Q4_K prefill GEMM kernel families (lp_set_gemm_kernel 1-5:
split-precision fp16/fp8 MFMA on row-major planes, the same arithmetic on
MFMA-fragment-order planes, int8 MFMA with a per-block fp32 epilogue, and
the wide-token kernel with 128 x 256 and 256 x 256 tiles), each
against the oracle's gemm_int (src/matmul_simd.cpp:226-283, 432-455) within
1e-4 normwise, and each bit-identical between the one-call path
(lp_gemm_dev: quantize and planes from fp32 x) and the two-step path
(lp_quantize_act_dev + lp_gemm_q_dev: planes from the stored blocks).
Shapes cover partial token and row tiles and the K-split tail round (tiles
of two workgroups adding into a zeroed y)."""
import numpy as np
import pytest

from hip_util import L, Q4_K, gemm_dev, normwise, stream, synth_weights, synth_x, to_dev, workspace
from laplace_amd import _lib

pytestmark = pytest.mark.gpu

# (K, N, M); K > 4096 takes the two-launch planes from fp32 x
SHAPES = [(512, 300, 130), (4096, 512, 257), (2816, 200, 129), (1024, 4096, 384), (4096, 14336, 128),
          (5120, 264, 160)]


@pytest.fixture
def kernel_family():
    def use(k):
        _lib.check(L().lp_set_gemm_kernel(k), "lp_set_gemm_kernel")
    yield use
    _lib.check(L().lp_set_gemm_kernel(0), "lp_set_gemm_kernel")


@pytest.mark.parametrize("kern", [1, 2, 3, 4, 5])
@pytest.mark.parametrize("K,N,M", SHAPES, ids=lambda v: str(v))
def test_gemm_kernel_family(orc, kernel_family, kern, K, N, M):
    import torch
    print(f"gemm kernel {kern} K={K} N={N} M={M}", flush=True)
    kernel_family(kern)
    w = synth_weights(Q4_K, K, N, seed=K + N + kern)
    x = synth_x(M, K, seed=M + 3, outliers=0.01)
    y = gemm_dev(Q4_K, x, w, N)
    assert np.isfinite(y).all()
    rng = np.random.default_rng(M + N)
    toks = np.sort(rng.choice(M, min(M, 40), replace=False))
    rows = np.sort(rng.choice(N, min(N, 64), replace=False))
    rb = len(w) // N
    wsub = np.concatenate([w[r * rb:(r + 1) * rb] for r in rows])
    ref = orc.gemm_int(Q4_K, x[toks], wsub, len(rows))
    assert normwise(y[np.ix_(toks, rows)], ref) <= 1e-4
    xd, wd = to_dev(x), to_dev(w)
    ws, nb = workspace(M, K)
    y2 = torch.empty(M * N, dtype=torch.float32, device="cuda")
    assert L().lp_quantize_act_dev(xd.data_ptr(), M, K, ws.data_ptr(), nb, stream()) == 0
    assert L().lp_gemm_q_dev(ws.data_ptr(), wd.data_ptr(), Q4_K, y2.data_ptr(), M, K, N, stream()) == 0
    torch.cuda.synchronize()
    assert np.array_equal(y2.cpu().numpy().reshape(M, N).view(np.uint32), y.view(np.uint32))


def test_gemm_kernel_rejects_unknown():
    assert L().lp_set_gemm_kernel(6) == _lib.LP_EINVAL
    assert L().lp_set_gemm_kernel(-1) == _lib.LP_EINVAL


@pytest.mark.parametrize("kern", [2, 4, 5])
def test_gemm_kernel_scale_edge_cases(orc, kernel_family, kern):
    """Super-block scales the wide-token kernel's per-super-block units treat
    specially: d = 0 (the unit stays, V decodes as zero, only the min term
    counts), subnormal fp16 d and dmin, and dmin far larger than d (the unit
    ratio d_old / d_new spans many binades). Against the oracle's gemm_int
    (src/matmul_simd.cpp:226-283) within 1e-4 normwise, row by row."""
    print(f"gemm scale edge cases kernel {kern}", flush=True)
    kernel_family(kern)
    K, N, M = 2048, 512, 300
    w = synth_weights(Q4_K, K, N, seed=77).reshape(N, K // 256, 144)
    rng = np.random.default_rng(78)
    f16 = lambda v: np.array([v], np.float16).view(np.uint8)
    w[0:8, 1, 0:2] = f16(0.0)                                 # d = 0 in one super-block
    w[8:16, :, 0:2] = f16(0.0)                                # d = 0 everywhere (min terms only)
    w[16:24, 3, 0:2] = np.frombuffer(np.uint16(3).tobytes(), np.uint8)     # subnormal d
    w[24:32, 5, 2:4] = np.frombuffer(np.uint16(7).tobytes(), np.uint8)     # subnormal dmin
    w[32:40, 2, 0:2] = f16(1e-5)                              # dmin / d ~ 1e3 ...
    w[32:40, 2, 2:4] = f16(0.02)
    w[40:48, ::2, 0:2] = f16(30.0)                            # ... and d jumping between binades
    w = w.reshape(-1)
    x = synth_x(M, K, seed=79, outliers=0.01)
    y = gemm_dev(Q4_K, x, w, N)
    toks = np.sort(rng.choice(M, 48, replace=False))
    rows = np.arange(0, 56)
    rb = len(w) // N
    wsub = np.concatenate([w[r * rb:(r + 1) * rb] for r in rows])
    ref = orc.gemm_int(Q4_K, x[toks], wsub, len(rows))
    got = y[np.ix_(toks, rows)]
    assert np.isfinite(got).all()
    for j in range(0, 56, 8):
        assert normwise(got[:, j:j + 8], ref[:, j:j + 8]) <= 1e-4, f"rows {j}..{j + 7}"


@pytest.mark.parametrize("kern", [0, 1, 2, 4, 5])
def test_gemm_kernel_activation_edge_rows(orc, kernel_family, kern):
    """Activation rows the row exponent treats specially, through the
    one-call path (planes from fp32 x: one launch for K <= 4096) and the
    two-step path (planes from the stored blocks), bit for bit: a row of
    zeros (exponent 0), a row of subnormals, a row whose only large block
    holds a NaN (the NaN block's scale is skipped), rows with +-inf, a row
    with one huge block. Finite rows also against the oracle within 1e-4;
    the subnormal row's exponent is clamped, so its outputs stay finite."""
    import torch
    print(f"gemm activation edge rows kernel {kern}", flush=True)
    kernel_family(kern)
    K, N, M = 1024, 256, 160
    w = synth_weights(Q4_K, K, N, seed=91)
    x = synth_x(M, K, seed=92, outliers=0.01)
    x[5] = 0.0
    x[6] = np.float32(1e-40) * np.sign(x[6])
    x[7, 64:96] *= 1e6
    x[7, 70] = np.nan
    x[8, 300] = np.inf
    x[9, 900] = -np.inf
    x[10, 512:544] *= 1e30
    y = gemm_dev(Q4_K, x, w, N)
    xd, wd = to_dev(x), to_dev(w)
    ws, nb = workspace(M, K)
    y2 = torch.empty(M * N, dtype=torch.float32, device="cuda")
    assert L().lp_quantize_act_dev(xd.data_ptr(), M, K, ws.data_ptr(), nb, stream()) == 0
    assert L().lp_gemm_q_dev(ws.data_ptr(), wd.data_ptr(), Q4_K, y2.data_ptr(), M, K, N, stream()) == 0
    torch.cuda.synchronize()
    assert np.array_equal(y2.cpu().numpy().reshape(M, N).view(np.uint32), y.view(np.uint32))
    assert np.isfinite(y[[0, 5, 6, 10, 11, 159]]).all()
    # the subnormal row (6) is left out here: the reference's own products
    # of subnormal block scales (d * xd, src/matmul_simd.cpp:226-283) keep a
    # few significant bits, so the oracle is no yardstick for it
    fin = [0, 5, 10, 11, 159]
    ref = orc.gemm_int(Q4_K, x[fin], w, N)
    for i, r in enumerate(fin):
        assert normwise(y[r], ref[i]) <= 1e-4, f"row {r}"


@pytest.mark.parametrize("kern", [0, 5])
def test_gemm_planes_grid_stride(orc, kernel_family, kern):
    """More token pairs than the one-launch planes kernel has workgroups (4
    per CU): its workgroups take a second pair, whose rows were requested
    while the first was processed. One-call path against the two-step
    path bit for bit, sampled rows against the oracle."""
    import torch
    print(f"gemm planes grid stride kernel {kern}", flush=True)
    kernel_family(kern)
    K, N, M = 512, 256, 2 * 4 * 256 + 100
    w = synth_weights(Q4_K, K, N, seed=95)
    x = synth_x(M, K, seed=96, outliers=0.01)
    y = gemm_dev(Q4_K, x, w, N)
    xd, wd = to_dev(x), to_dev(w)
    ws, nb = workspace(M, K)
    y2 = torch.empty(M * N, dtype=torch.float32, device="cuda")
    assert L().lp_quantize_act_dev(xd.data_ptr(), M, K, ws.data_ptr(), nb, stream()) == 0
    assert L().lp_gemm_q_dev(ws.data_ptr(), wd.data_ptr(), Q4_K, y2.data_ptr(), M, K, N, stream()) == 0
    torch.cuda.synchronize()
    assert np.array_equal(y2.cpu().numpy().reshape(M, N).view(np.uint32), y.view(np.uint32))
    toks = np.array([0, 1, 2047, 2048, 2049, 2100, M - 1])
    ref = orc.gemm_int(Q4_K, x[toks], w, N)
    assert normwise(y[toks], ref) <= 1e-4
