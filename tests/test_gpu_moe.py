"""Grouped MoE dispatch on the GPU against the CPU oracle.

The oracle is the reference's per-token call (moe_gemv_int /
moe_gemv_multi_int, src/matmul_simd.cpp:506-544, as called per token from
src/arch_gemma4.cpp:604 and :626): for every token t the grouped result rows
y[t*topk .. t*topk + topk) must equal the oracle's call for that token with
expert list topk_idx[t]. Tolerance: normwise 1e-4 (fp32 outputs of int8
block dots; tests/test_metal.cpp:200-203 form). Grouping must not change the
arithmetic, so the grouped rows are also compared bit for bit with the
M = 1 GEMV on the selected expert's slice.
"""
import numpy as np
import pytest

from hip_util import (Q4_K, Q6_K, TYPES, NAMES, L, gemm_dev, moe_dev, normwise, routing,
                      synth_weights, synth_x)
from laplace_amd.matmul import row_bytes

pytestmark = pytest.mark.gpu

TOL = 1e-4


def oracle_grouped(orc, t, x, w, idx, K, N, multi):
    T, topk = idx.shape
    out = np.zeros((T * topk, N), np.float32)
    for tok in range(T):
        xt = x[tok * topk:(tok + 1) * topk] if multi else x[tok]
        out[tok * topk:(tok + 1) * topk] = orc.moe_gemv_int(t, xt, w, idx[tok], K, N, multi)
    return out


@pytest.mark.parametrize("multi", [False, True])
@pytest.mark.parametrize("t", TYPES, ids=[NAMES[t] for t in TYPES])
def test_moe_small(orc, t, multi):
    E, T, topk, K, N = 16, 10, 4, 512, 72
    w = synth_weights(t, K, N * E, seed=100 + t)
    idx = routing(T, topk, E, seed=5 + t)
    x = synth_x(T * topk if multi else T, K, seed=9 + t)
    y = moe_dev(t, x, w, idx, E, N, multi)
    ref = oracle_grouped(orc, t, x, w, idx, K, N, multi)
    assert np.isfinite(y).all()
    assert normwise(y, ref) <= TOL


@pytest.mark.parametrize("t", TYPES, ids=[NAMES[t] for t in TYPES])
def test_moe_grouped_equals_gemv(t):
    """Each pair's row equals the M=1 GEMV on its expert to fp32 rounding:
    the Q4_K groups run on the fp16-MFMA kernel (exact operand folding, fp32
    accumulation in another order), the other types on the same integer
    block dots in another summation order (1e-5 normwise)."""
    E, T, topk, K, N = 8, 6, 3, 1024, 40
    w = synth_weights(t, K, N * E, seed=200 + t)
    idx = routing(T, topk, E, seed=11)
    x = synth_x(T, K, seed=12)
    y = moe_dev(t, x, w, idx, E, N, False)
    eb = row_bytes(t, K) * N
    for tok in range(T):
        for j in range(topk):
            e = int(idx[tok, j])
            g = gemm_dev(t, x[tok], w[e * eb:(e + 1) * eb], N)[0]
            assert normwise(y[tok * topk + j], g) <= 1e-5, (tok, j, e)


def test_moe_skewed_and_duplicates(orc):
    """All tokens on one expert (many groups of one expert), repeated experts
    within a token, and a group count that is not a multiple of the group size."""
    t, E, T, topk, K, N = Q4_K, 6, 23, 3, 512, 48
    w = synth_weights(t, K, N * E, seed=31)
    x = synth_x(T, K, seed=32)
    idx = np.full((T, topk), 4, np.int32)
    idx[::5, 1] = 0
    idx[3] = [2, 2, 2]
    y = moe_dev(t, x, w, idx, E, N, False)
    assert normwise(y, oracle_grouped(orc, t, x, w, idx, K, N, False)) <= TOL


@pytest.mark.parametrize("multi,N,K", [(False, 1536, 2048), (True, 2048, 768)],
                         ids=["gate_up", "down"])
def test_moe_baseline_config(orc, multi, N, K):
    """The MoE benchmark configuration: 128 experts, 64 tokens, top-8, Q4_K
    gate/up (N=1536, K=2048) and down (N=2048, K=768); every pair checked
    against the oracle."""
    t, E, T, topk = Q4_K, 128, 64, 8
    w = synth_weights(t, K, N * E, seed=41 if multi else 42)
    idx = routing(T, topk, E, seed=43)
    x = synth_x(T * topk if multi else T, K, seed=44)
    y = moe_dev(t, x, w, idx, E, N, multi)
    assert np.isfinite(y).all()
    ref = oracle_grouped(orc, t, x, w, idx, K, N, multi)
    assert normwise(y, ref) <= TOL


def test_moe_host_api_matches_device(orc):
    """lp_moe_grouped (host pointers) and lp_moe_gemv / lp_moe_gemv_multi (the
    reference's per-token ABI) give the device path's values."""
    import ctypes as C
    t, E, T, topk, K, N = Q4_K, 12, 5, 4, 512, 64
    w = synth_weights(t, K, N * E, seed=51)
    idx = routing(T, topk, E, seed=52)
    for multi in (0, 1):
        x = synth_x(T * topk if multi else T, K, seed=53 + multi)
        yd = moe_dev(t, x, w, idx, E, N, bool(multi))
        yh = np.zeros((T * topk, N), np.float32)
        assert L().lp_moe_grouped(x.ctypes.data, multi, idx.ctypes.data, w.ctypes.data, t,
                                  yh.ctypes.data, T, topk, E, K, N)
        assert np.array_equal(yh, yd)
        fn = L().lp_moe_gemv_multi if multi else L().lp_moe_gemv
        for tok in range(T):
            xt = np.ascontiguousarray(x[tok * topk:(tok + 1) * topk] if multi else x[tok])
            it = np.ascontiguousarray(idx[tok])
            yt = np.zeros((topk, N), np.float32)
            assert fn(xt.ctypes.data, w.ctypes.data, t, it.ctypes.data, topk, yt.ctypes.data, K, N)
            assert np.array_equal(yt, yd[tok * topk:(tok + 1) * topk])
    L().lp_release_weights()


def test_moe_host_rejects_bad_index():
    t, E, T, topk, K, N = Q4_K, 4, 2, 2, 256, 16
    w = synth_weights(t, K, N * E, seed=61)
    x = synth_x(T, K, seed=62)
    idx = np.array([[0, 1], [4, 2]], np.int32)
    y = np.zeros((T * topk, N), np.float32)
    assert not L().lp_moe_grouped(x.ctypes.data, 0, idx.ctypes.data, w.ctypes.data, t,
                                  y.ctypes.data, T, topk, E, K, N)
    assert b"outside" in L().lp_last_error()


def test_moe_device_drops_bad_index(orc):
    """Device path: a pair naming an expert outside [0, E) is dropped (its y
    row keeps its previous contents), the others are computed."""
    t, E, T, topk, K, N = Q4_K, 4, 3, 2, 256, 16
    w = synth_weights(t, K, N * E, seed=71)
    x = synth_x(T, K, seed=72)
    idx = np.array([[0, 1], [9, 2], [3, -1]], np.int32)
    y = moe_dev(t, x, w, idx, E, N, False)
    assert np.isnan(y[2]).all() and np.isnan(y[5]).all()
    ok = [0, 1, 3, 4]
    good = idx.copy()
    good[good < 0] = 0
    good[good >= E] = 0
    ref = oracle_grouped(orc, t, x, w, good, K, N, False)
    assert normwise(y[ok], ref[ok]) <= TOL


def test_moe_empty():
    t = Q4_K
    w = synth_weights(t, 256, 16, seed=1)
    x = np.zeros((1, 256), np.float32)
    idx = np.zeros((0, 8), np.int32)
    assert L().lp_moe_grouped(x.ctypes.data, 0, idx.ctypes.data, w.ctypes.data, t,
                              x.ctypes.data, 0, 8, 1, 256, 16)


@pytest.mark.parametrize("multi", [False, True])
def test_moe_many_pairs_per_expert_mfma(orc, multi):
    """When experts average more than 8 pairs (prefill-sized batches), Q4_K groups of
    up to 16 pairs run on the small-M MFMA kernel: 8 experts, 96 tokens,
    top-2, ragged groups, against the oracle."""
    t, E, T, topk, K, N = Q4_K, 8, 96, 2, 1024, 80
    w = synth_weights(t, K, N * E, seed=81 + multi)
    idx = routing(T, topk, E, seed=82)
    x = synth_x(T * topk if multi else T, K, seed=83, outliers=0.01)
    y = moe_dev(t, x, w, idx, E, N, multi)
    assert np.isfinite(y).all()
    assert normwise(y, oracle_grouped(orc, t, x, w, idx, K, N, multi)) <= TOL


@pytest.mark.parametrize("K,N", [(256, 300), (768, 200), (2048, 96), (3072, 40)], ids=lambda v: str(v))
def test_moe_mfma_row_sets(orc, K, N):
    """The MFMA groups' workgroups take several row sets in turn, and at
    short K split their waves into fewer K-slices and more row groups (K 256:
    1 slice x 8 row groups, 768: 2 x 4, 2048: 8 x 1, 3072: 8 x 1 over 12
    super-blocks): ragged N (a partial last row set, workgroups with fewer
    sets), 6 experts, 64 tokens, top-2 (about 21 pairs per expert, so some
    experts take two groups), against the oracle."""
    t, E, T, topk = Q4_K, 6, 64, 2
    w = synth_weights(t, K, N * E, seed=K + N)
    idx = routing(T, topk, E, seed=K)
    x = synth_x(T, K, seed=N, outliers=0.01)
    y = moe_dev(t, x, w, idx, E, N, False)
    assert np.isfinite(y).all()
    assert normwise(y, oracle_grouped(orc, t, x, w, idx, K, N, False)) <= TOL
