"""GPU parity: the HIP path through the C ABI against the CPU oracle on the
same seeded inputs.

Bars (from the reference's int8 path, src/matmul_simd.cpp):
  * quantized activation blocks (d, sum, sum_lo, sum_hi, codes): bit-exact;
  * per-sub-block int32 dot sums: bit-exact;
  * fp32 outputs: normwise max|dy| / max|y| <= 1e-4 (TOL below), plus the
    reference's own per-element acceptance (tests/test_matmul.cpp:88-97).
"""
import numpy as np
import pytest

from hip_util import (Q4_0, Q4_K, Q6_K, Q8_0, TYPES, NAMES, block_sums_dev, gemm_dev, normwise,
                      quantize_dev, synth_weights, synth_x)

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _flush(msg):
    print(msg, flush=True)


# ---------------------------------------------------------------------------
# quantizer


def _edge_rows(K):
    rows = []
    x = np.zeros(K, np.float32)
    rows.append(x.copy())                                   # all zero
    x = np.ones(K, np.float32)
    x[3] = np.nan
    x[40] = np.inf
    x[70] = -np.inf
    rows.append(x)
    x = np.zeros(K, np.float32)                             # ties at d = id = 1
    x[0] = 127.0
    x[1:11] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, 100.5, -100.5, 126.5]
    rows.append(x)
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(K) * 1e-39).astype(np.float32)   # subnormal inputs
    x[32:64] *= 1e-5
    rows.append(x)
    x = (rng.standard_normal(K) * 1e30).astype(np.float32)
    rows.append(x)
    return np.stack(rows)


@pytest.mark.parametrize("M,K", [(1, 4096), (8, 3584), (5, 2048), (64, 768)])
def test_quantizer_bit_exact(orc, M, K):
    _flush(f"quantizer M={M} K={K}")
    x = synth_x(M, K, seed=M * 7 + K, outliers=0.01)
    d, s, s16, qs = quantize_dev(x)
    rd, rs, rlo, rhi, rqs = orc.quantize_act(x)
    assert np.array_equal(qs, rqs)
    assert np.array_equal(d.view(np.uint32), rd.view(np.uint32))
    assert np.array_equal(s.view(np.uint32), rs.view(np.uint32))
    lo = (s16 & 0xffff).astype(np.uint16).view(np.int16)
    hi = ((s16.view(np.uint32) >> 16) & 0xffff).astype(np.uint16).view(np.int16)
    assert np.array_equal(lo, rlo) and np.array_equal(hi, rhi)


def test_quantizer_edge_cases_bit_exact(orc):
    _flush("quantizer edge cases")
    x = _edge_rows(256)
    d, s, s16, qs = quantize_dev(x)
    rd, rs, rlo, rhi, rqs = orc.quantize_act(x)
    assert np.array_equal(qs, rqs)
    # NaN blocks: compare NaN-ness, other values by bits
    for a, b in ((d, rd), (s, rs)):
        na, nb = np.isnan(a), np.isnan(b)
        assert np.array_equal(na, nb)
        assert np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))
    lo = (s16 & 0xffff).astype(np.uint16).view(np.int16)
    assert np.array_equal(lo, rlo)


def test_quantizer_host_api(orc):
    _flush("quantizer host api")
    from laplace_amd import quantize_act
    x = synth_x(3, 1024, seed=5, outliers=0.01)
    got = quantize_act(x)
    want = orc.quantize_act(x)
    for g, w_ in zip(got, want):
        assert np.array_equal(np.asarray(g).view(np.uint8), np.asarray(w_).view(np.uint8))


# ---------------------------------------------------------------------------
# integer block sums


@pytest.mark.parametrize("t", TYPES, ids=lambda t: NAMES[t])
@pytest.mark.parametrize("K", [512, 2816, 4096])
def test_block_sums_bit_exact(orc, t, K):
    if t in (Q4_0, Q8_0) and K % 64:
        pytest.skip("legacy chunk is 64 elements")
    _flush(f"block sums {NAMES[t]} K={K}")
    M, N = 3, 33
    rng = np.random.default_rng(K + t)
    w = rng.integers(0, 256, (K // (256 if t in (Q4_K, Q6_K) else 32)) * N *
                     {Q4_0: 18, Q8_0: 34, Q4_K: 144, Q6_K: 210}[t], dtype=np.uint8)
    x = synth_x(M, K, seed=K, outliers=0.01)
    got = block_sums_dev(t, x, w, N)
    _, _, _, _, qs = orc.quantize_act(x)
    want = orc.block_sums(t, w, qs, K, N)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------------------
# GEMV against the oracle's gemm_int


def _check_against_oracle(orc, t, x, w, N, y):
    ref = orc.gemm_int(t, x, w, N)
    err = normwise(y, ref)
    assert err <= TOL, f"normwise {err:.3g}"
    diff = np.abs(y - ref)
    ok = (diff <= 1e-3) | (diff <= 1e-3 * np.maximum(np.abs(y), np.abs(ref)))
    assert ok.all(), f"{(~ok).sum()} outputs outside rel/abs 1e-3"


REF_SHAPES = [(t, 512, n) for n in (1, 8, 33, 256) for t in TYPES] + \
             [(t, 2816, n) for n in (1, 8, 256, 4096) for t in (Q4_K, Q6_K)]


@pytest.mark.parametrize("t,K,N", REF_SHAPES, ids=lambda v: str(v))
def test_gemv_reference_test_shapes(orc, t, K, N):
    """The reference's matmul test inputs (tests/test_matmul.cpp:272-291)."""
    _flush(f"gemv ref-shape {NAMES[t]} K={K} N={N}")
    w = orc.ref_test_weights(t, K, N)
    x = orc.ref_test_x(t, K)[None, :]
    y = gemm_dev(t, x, w, N)
    _check_against_oracle(orc, t, x, w, N, y)


CONFIG_SHAPES = [
    (Q8_0, 4096, 4096, 1),
    (Q4_0, 4096, 14336, 1), (Q4_0, 14336, 4096, 1),
    (Q4_K, 4096, 14336, 1),
    (Q4_K, 3584, 18944, 1), (Q4_K, 3584, 18944, 4), (Q4_K, 3584, 18944, 8),
    (Q6_K, 18944, 3584, 1), (Q6_K, 18944, 3584, 4), (Q6_K, 18944, 3584, 8),
    # LM head of the reference's GPU benchmark (tests/bench_cpu_gpu.cpp:58)
    (Q4_K, 2816, 262144, 1),
]


@pytest.mark.parametrize("t,K,N,M", CONFIG_SHAPES, ids=lambda v: str(v))
def test_gemv_baseline_configs(orc, t, K, N, M):
    """BASELINE.json configs 1-3 at full size; the oracle checks a seeded
    sample of 256 rows (rows are independent), the GPU computes all N."""
    _flush(f"gemv config {NAMES[t]} K={K} N={N} M={M}")
    w = synth_weights(t, K, N, seed=K * 3 + N)
    x = synth_x(M, K, seed=K + M)
    y = gemm_dev(t, x, w, N)
    assert np.isfinite(y).all()
    rb = len(w) // N
    rows = np.sort(np.random.default_rng(N).choice(N, 256, replace=False))
    ws = np.concatenate([w[r * rb:(r + 1) * rb] for r in rows])
    _check_against_oracle(orc, t, x, ws, len(rows), y[:, rows])


@pytest.mark.parametrize("t", TYPES, ids=lambda t: NAMES[t])
def test_batched_rows_equal_single(t):
    """tests/test_matmul.cpp:217-250: matmul_rows(M=7) equals M matmul_row
    calls within 1e-4 (almost_equal, absolute or relative). As in the
    reference, Q8_0 and Q4_K use random bytes as weights (NaN skipped); the
    reference does not test Q4_0 / Q6_K this way - with random fp16 scales
    up to 65504 their rows cancel to a few units out of ~1e6-sized terms, and
    two correct summation orders differ by more than 1e-4 (the oracle
    differs from both as well) - so they use the synthetic weight
    distribution."""
    _flush(f"batched vs single {NAMES[t]}")
    M, K, N = 7, 512, 64
    rng = np.random.default_rng(41 + t)
    if t in (Q8_0, Q4_K):
        w = rng.integers(0, 256, (K // (256 if t == Q4_K else 32)) * N * {Q8_0: 34, Q4_K: 144}[t],
                         dtype=np.uint8)
    else:
        w = synth_weights(t, K, N, seed=41 + t)
    x = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    yb = gemm_dev(t, x, w, N)
    for m in range(M):
        ys = gemm_dev(t, x[m:m + 1], w, N)[0]
        a, b = yb[m], ys
        both_nan = np.isnan(a) & np.isnan(b)
        diff = np.abs(a - b)
        ok = both_nan | (diff <= 1e-4) | (diff <= 1e-4 * np.maximum(np.abs(a), np.abs(b)))
        assert ok.all()


def test_subnormal_weight_scales(orc):
    """fp16 scales that are all subnormal must not be flushed to zero."""
    _flush("subnormal scales")
    t, K, N = Q8_0, 512, 16
    w = synth_weights(t, K, N, seed=3).reshape(-1, 34)
    rng = np.random.default_rng(4)
    w[:, 0:2] = rng.integers(1, 0x3ff, (w.shape[0], 1), dtype=np.uint16).view(np.uint8).reshape(-1, 2)
    w = w.reshape(-1)
    x = synth_x(1, K, seed=9)
    y = gemm_dev(t, x, w, N)
    ref = orc.gemm_int(t, x, w, N)
    assert np.abs(ref).max() > 0
    assert normwise(y, ref) <= TOL


def test_host_api_matches_device_api(orc):
    _flush("host api vs device api")
    from laplace_amd import GGMLType, Tensor, matmul_rows
    t, K, N, M = Q4_K, 2048, 384, 3
    w = synth_weights(t, K, N, seed=77)
    x = synth_x(M, K, seed=78)
    y = np.zeros((M, N), np.float32)
    matmul_rows(x, Tensor(GGMLType.Q4_K, (K, N), w), y, M, K, N)
    yd = gemm_dev(t, x, w, N)
    assert np.array_equal(y.view(np.uint32), yd.view(np.uint32))
    _check_against_oracle(orc, t, x, w, N, y)


def test_unsupported_type_is_reported():
    from laplace_amd import _lib
    import ctypes as C
    x = np.zeros(256, np.float32)
    w = np.zeros(256 * 2, np.uint8)
    y = np.zeros(1, np.float32)
    # Q4_1 (3): neither the reference's back-ends nor this library take it
    ok = _lib.lib().lp_gemm(x.ctypes.data, w.ctypes.data, 3, y.ctypes.data, 1, 256, 1)
    assert ok is False
    assert b"not handled" in _lib.lib().lp_last_error()
    # F16 (1) is taken (fp32-activation path): zero weights give zero
    y[:] = 1.0
    assert _lib.lib().lp_gemm(x.ctypes.data, w.ctypes.data, 1, y.ctypes.data, 1, 256, 1) is True
    assert y[0] == 0.0
    _lib.lib().lp_release_weights()


# ---------------------------------------------------------------------------
# prefill GEMM (Q4_K, M > 8): MFMA path against the oracle's gemm_int


GEMM_SHAPES = [(512, 256, 9), (512, 300, 49), (512, 256, 130), (2816, 300, 65), (4096, 512, 257)]


@pytest.mark.parametrize("K,N,M", GEMM_SHAPES, ids=lambda v: str(v))
def test_gemm_q4k_small(orc, K, N, M):
    _flush(f"gemm Q4_K K={K} N={N} M={M}")
    w = synth_weights(Q4_K, K, N, seed=K + N)
    x = synth_x(M, K, seed=M, outliers=0.01)
    y = gemm_dev(Q4_K, x, w, N)
    ref = orc.gemm_int(Q4_K, x, w, N)
    err = normwise(y, ref)
    assert err <= TOL, f"normwise {err:.3g}"
    # these shapes have few tiles, so K is split over two workgroups whose
    # halves are added into y: the result must not depend on their order
    assert np.array_equal(gemm_dev(Q4_K, x, w, N).view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("N,M", [(4096, 512), (4096, 2048), (14336, 512), (14336, 2048)],
                         ids=lambda v: str(v))
def test_gemm_q4k_prefill_configs(orc, N, M):
    """BASELINE.json config 4 at full size (x N(0,1) with 1% outliers x20):
    the GPU computes the whole [M, N]; the oracle checks 48 sampled tokens
    x 96 sampled rows (outputs are independent)."""
    K = 4096
    _flush(f"gemm prefill N={N} M={M}")
    w = synth_weights(Q4_K, K, N, seed=N)
    x = synth_x(M, K, seed=M + 1, outliers=0.01)
    y = gemm_dev(Q4_K, x, w, N)
    assert np.isfinite(y).all()
    rng = np.random.default_rng(M + N)
    toks = np.sort(rng.choice(M, 48, replace=False))
    rows = np.sort(rng.choice(N, 96, replace=False))
    rb = len(w) // N
    ws = np.concatenate([w[r * rb:(r + 1) * rb] for r in rows])
    ref = orc.gemm_int(Q4_K, x[toks], ws, len(rows))
    err = normwise(y[np.ix_(toks, rows)], ref)
    assert err <= TOL, f"normwise {err:.3g}"


@pytest.mark.parametrize("K,N,M", [(512, 300, 17), (1024, 256, 24), (512, 300, 33), (2816, 4096, 48)],
                         ids=lambda v: str(v))
def test_gemm_q4k_small_prefill_chunks(orc, K, N, M):
    """Q4_K at 17..48 rows (the GEMM's 64-token tiles would be mostly empty)
    runs as 16-row chunks on the int8 MFMA kernel plus a GEMV remainder:
    against the oracle's gemm_int, rows 16 apart are independent."""
    _flush(f"gemm chunks Q4_K K={K} N={N} M={M}")
    w = synth_weights(Q4_K, K, N, seed=K + M)
    x = synth_x(M, K, seed=M + 7, outliers=0.01)
    y = gemm_dev(Q4_K, x, w, N)
    assert normwise(y, orc.gemm_int(Q4_K, x, w, N)) <= TOL
    for m0 in range(0, M, 16):
        part = gemm_dev(Q4_K, x[m0:m0 + 16], w, N)
        assert np.array_equal(part.view(np.uint32), y[m0:m0 + 16].view(np.uint32))


# (N, K) -> kernel at M = 3 and M = 4 on a 256-CU part (lp_gemm_route)
THREE_FOUR = {(256, 14336): ("i8mf", "i8mf"), (256, 16384): ("i8mf", "i8mf"),
              (8192, 512): ("sbm", "rq"), (256, 512): ("sbm", "rq"), (12288, 1024): ("rq", "rq")}


@pytest.mark.parametrize("N,K", list(THREE_FOUR), ids=[f"{n}x{k}" for n, k in THREE_FOUR])
@pytest.mark.parametrize("M", [3, 4])
def test_q4k_three_four_rows(orc, M, N, K):
    """Q4_K at M = 3, 4, each case on the kernel named in THREE_FOUR (checked
    through the routing probe): the 16x16 int8 MFMA kernel when its 16-row
    workgroups apply and K is long (N = 256, K = 14336, and K = 16384, the
    last K whose block scales fit its LDS), the dot4 GEMV or the row-quad
    kernel otherwise; all against the oracle's gemm_int."""
    import torch
    from hip_util import L, to_dev
    _flush(f"Q4_K M={M} N={N} K={K}")
    w = synth_weights(Q4_K, K, N, seed=M + N)
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        route = L().lp_gemm_route(Q4_K, M, K, N, to_dev(w).data_ptr()).decode()
        assert route == THREE_FOUR[(N, K)][M - 3]
    x = synth_x(M, K, seed=M + 3, outliers=0.01)
    y = gemm_dev(Q4_K, x, w, N)
    assert normwise(y, orc.gemm_int(Q4_K, x, w, N)) <= TOL


def test_gemm_matches_gemv_rows(orc):
    """The MFMA GEMM (M = 16) and the GEMV (M = 8, twice) agree per row."""
    _flush("gemm vs gemv")
    K, N = 4096, 768
    w = synth_weights(Q4_K, K, N, seed=5)
    x = synth_x(16, K, seed=6, outliers=0.01)
    yg = gemm_dev(Q4_K, x, w, N)
    yv = np.concatenate([gemm_dev(Q4_K, x[:8], w, N), gemm_dev(Q4_K, x[8:], w, N)])
    assert normwise(yg, yv) <= TOL


@pytest.mark.parametrize("t", TYPES, ids=[NAMES[t] for t in TYPES])
@pytest.mark.parametrize("M", [1, 2, 3, 5, 8, 16])
def test_gemm_dev_equals_two_step(t, M):
    """lp_gemm_dev (quantize + GEMV in one call) is bit-identical to
    lp_quantize_act_dev + lp_gemm_q_dev on the stored blocks, including
    blocks with zeros, exact ties, infinities and NaNs."""
    import torch
    from hip_util import L, stream, to_dev, workspace
    from laplace_amd import _lib
    K, N = 1024, 200
    w = synth_weights(t, K, N, seed=300 + t)
    x = synth_x(M, K, seed=301, outliers=0.01)
    x[0, 32:64] = 0.0
    x[0, 64:96] = np.array([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5] * 4, np.float32)
    if M > 1:
        x[1, 100] = np.inf
        x[1, 300] = np.nan
    y1 = gemm_dev(t, x, w, N)
    xd, wd = to_dev(x), to_dev(w)
    ws, nb = workspace(M, K)
    y2 = torch.empty(M * N, dtype=torch.float32, device="cuda")
    _lib.check(L().lp_quantize_act_dev(xd.data_ptr(), M, K, ws.data_ptr(), nb, stream()), "q")
    _lib.check(L().lp_gemm_q_dev(ws.data_ptr(), wd.data_ptr(), t, y2.data_ptr(), M, K, N, stream()), "g")
    torch.cuda.synchronize()
    y2 = y2.cpu().numpy().reshape(M, N)
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))


@pytest.mark.parametrize("K", [2048, 2304, 5120, 14336, 18944, 21760])
@pytest.mark.parametrize("N", [1, 5, 77, 1000])
def test_q4k_stream_gemv_shapes(orc, K, N):
    """The M=1 Q4_K GEMV streams whole rows per wave (R rows, I loads per
    lane, both depending on K): every K it accepts, ragged N (partial last
    wave, waves with no rows), against the oracle."""
    t = Q4_K
    w = synth_weights(t, K, N, seed=K + N)
    x = synth_x(1, K, seed=7, outliers=0.01)
    y = gemm_dev(t, x, w, N)
    ref = orc.gemm_int(t, x, w, N)
    assert normwise(y, ref) <= 1e-4


@pytest.mark.parametrize("K,N", [(256, 17), (512, 40), (2048, 1000), (3584, 333), (4096, 64), (18944, 48)])
@pytest.mark.parametrize("M", [5, 9, 16])
def test_q4k_small_m_mfma(orc, K, N, M):
    """5 <= M <= 16 Q4_K products run on the small-M MFMA kernel (planes from
    x in one pass, 32 weight rows x 8 K-slices per workgroup): K with fewer
    super-blocks than K-slices, ragged N, M up to the tile height. The
    K=3584 cases hold an fp16 rounding tie of d*q (hi and lo must come from
    the same fp32 product)."""
    t = Q4_K
    w = synth_weights(t, K, N, seed=K * 7 + N + M)
    x = synth_x(M, K, seed=M + 11, outliers=0.01)
    y = gemm_dev(t, x, w, N)
    ref = orc.gemm_int(t, x, w, N)
    assert np.isfinite(y).all()
    assert normwise(y, ref) <= 1e-4


@pytest.mark.parametrize("t", [Q8_0, Q4_0, Q6_K], ids=["Q8_0", "Q4_0", "Q6_K"])
@pytest.mark.parametrize("K,N", [(256, 7), (768, 100), (3584, 257), (4096, 1001), (2048, 4095), (14336, 33),
                                 (18944, 40), (32768, 9)])
def test_m1_gemv_shapes(orc, t, K, N):
    """M=1 GEMV for Q8_0 / Q4_0 / Q6_K over a range of K (rows that are not
    16-byte multiples for Q6_K, K up to the 32768 limit), ragged N (Q8_0 at
    K 2048-4096 with few rows runs one row per wave, idle lanes past it): the
    single-call path (lp_gemm_dev) against the oracle and bit-identical to
    the quantizer-fed path (lp_gemm_q_dev)."""
    import torch
    from hip_util import L, stream, to_dev, workspace
    from laplace_amd import _lib
    w = synth_weights(t, K, N, seed=K + 3 * N + t)
    x = synth_x(1, K, seed=K + t, outliers=0.01)
    ref = orc.gemm_int(t, x, w, N)
    y = gemm_dev(t, x, w, N)
    assert normwise(y, ref) <= 1e-4
    xd, wd = to_dev(x), to_dev(w)
    ws, nb = workspace(1, K)
    y2 = torch.empty(N, dtype=torch.float32, device="cuda")
    _lib.check(L().lp_quantize_act_dev(xd.data_ptr(), 1, K, ws.data_ptr(), nb, stream()), "q")
    _lib.check(L().lp_gemm_q_dev(ws.data_ptr(), wd.data_ptr(), t, y2.data_ptr(), 1, K, N, stream()), "g")
    torch.cuda.synchronize()
    assert np.array_equal(y2.cpu().numpy().reshape(1, N).view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("M", [2, 3, 4, 5, 8, 13, 16])
@pytest.mark.parametrize("K,N", [(256, 7), (3584, 65), (18944, 40), (32768, 5)])
def test_q6k_multi_row_gemv(orc, K, N, M):
    """Q6_K for 2..16 activation rows over ragged N against the oracle, with
    activation outliers: dot4 GEMV (4 rows per weight pass) up to M = 4, int8
    MFMA from 5 (odd super-block counts give 2-byte aligned rows)."""
    _flush(f"q6k multi-row K={K} N={N} M={M}")
    w = synth_weights(Q6_K, K, N, seed=K + 7 * N + M)
    x = synth_x(M, K, seed=K + M, outliers=0.01)
    y = gemm_dev(Q6_K, x, w, N)
    assert normwise(y, orc.gemm_int(Q6_K, x, w, N)) <= 1e-4


@pytest.mark.parametrize("t", [Q8_0, Q4_0, Q6_K], ids=["Q8_0", "Q4_0", "Q6_K"])
@pytest.mark.parametrize("M", [21, 37, 64])
def test_prefill_rows_other_types(orc, t, M):
    """Prefill-sized M for the types without a GEMM kernel: chunks of rows
    (16 on the int8 MFMA kernel for Q6_K, 8 on the GEMV otherwise, remainders
    below 5 rows on the GEMV) against the oracle."""
    _flush(f"prefill rows {NAMES[t]} M={M}")
    K, N = 1024, 96
    w = synth_weights(t, K, N, seed=500 + M + t)
    x = synth_x(M, K, seed=501 + M, outliers=0.01)
    y = gemm_dev(t, x, w, N)
    assert normwise(y, orc.gemm_int(t, x, w, N)) <= TOL


@pytest.mark.parametrize("t", [Q8_0, Q6_K, Q4_0], ids=["Q8_0", "Q6_K", "Q4_0"])
@pytest.mark.parametrize("M", [17, 40, 70])
@pytest.mark.parametrize("N", [12288, 3000])
def test_i8_prefill_chunks(orc, t, M, N):
    """Q8_0, Q6_K and Q4_0 rows beyond 16 run in chunks of 32 on the int8 MFMA
    kernels with two token tiles per workgroup (one weight pass per chunk):
    sampled outputs against the oracle, and the first 16 rows bit-identical
    to a 16-row call (same per-output arithmetic; Q4_0's 16-row call runs on
    the dot4 GEMV, so within 1e-5 there)."""
    from hip_util import L, to_dev
    K = 1024
    w = synth_weights(t, K, N, seed=500 + M + t)
    assert L().lp_gemm_route(t, M, K, N, to_dev(w).data_ptr()).decode() == "i8mf"
    x = synth_x(M, K, seed=501, outliers=0.01)
    y = gemm_dev(t, x, w, N)
    assert np.isfinite(y).all()
    rng = np.random.default_rng(M)
    rows = np.sort(rng.choice(N, 48, replace=False))
    rb = len(w) // N
    wsub = np.concatenate([w[r * rb:(r + 1) * rb] for r in rows])
    ref = orc.gemm_int(t, x, wsub, len(rows))
    assert normwise(y[:, rows], ref) <= 1e-4
    y16 = gemm_dev(t, x[:16], w, N)
    if t == Q4_0 or (t == Q8_0 and N < 12288):
        # 16 rows run on another kernel (Q4_0: the dot4 GEMV; Q8_0 with few
        # rows: 16-row workgroups of 16 K-slices): another fp32 order
        assert normwise(y[:16], y16) <= 1e-5
    else:
        assert np.array_equal(y[:16].view(np.uint32), y16.view(np.uint32))
