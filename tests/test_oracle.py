"""Pins the CPU oracle (oracle/lp_oracle.c) before it is trusted as the
checker for the HIP path.

Each check ties the restatement to something it did not derive from:
  * the reference's fp16 known-answer tests (tests/test_matmul.cpp:252-268);
  * the reference's own fp16.h, kernels.h and tests/quant_ref.h, compiled in
    place into oracle/_ref (bit-exact comparisons);
  * one-hot probes: with unit scales, the integer block sums of a one-hot
    activation must reproduce the reference dequantizer's value of that
    element, which fixes the element-to-code mapping of every decoder;
  * the reference's dual-reference acceptance test (tests/test_matmul.cpp:
    57-108): the int8 path against the fp64 product of the reference
    dequantizer with the Q8 round-trip of x, the scalar path against the
    exact fp64 product, at the reference's seeds and shapes (:272-291);
  * closed-form quantizer properties, including round-half-to-even ties.
"""
import numpy as np
import pytest

from oracle.oracle import F16, BF16, Q4_0, Q8_0, Q4_K, Q6_K, Q5_0, Q2_K, Q3_K, Q5_K, F32

REF_TYPES = (Q8_0, Q4_0, Q4_K, Q6_K)


def _u16_bits(f):
    return np.frombuffer(np.float32(f).tobytes(), np.uint32)[0]


# ---------------------------------------------------------------------------
# fp16 / bf16


def test_fp16_known_answers(orc):
    """tests/test_matmul.cpp:252-268, verbatim constants."""
    L = orc.lib()
    assert L.or_fp16_to_fp32(0x3C00) == 1.0
    assert L.or_fp16_to_fp32(0xC000) == -2.0
    assert L.or_fp16_to_fp32(0x0000) == 0.0
    assert L.or_fp16_to_fp32(0x7BFF) == 65504.0
    assert L.or_fp16_to_fp32(0x0001) == 5.9604644775390625e-08
    assert L.or_fp32_to_fp16(1.0) == 0x3C00
    assert L.or_fp32_to_fp16(-2.0) == 0xC000
    for h in range(0, 0x7C00, 7):
        assert L.or_fp32_to_fp16(L.or_fp16_to_fp32(h)) == h


def test_fp16_exhaustive_against_reference(orc, ref):
    L = orc.lib()
    for h in range(65536):
        a, b = L.or_fp16_to_fp32(h), ref.ref_fp16_to_fp32(h)
        assert _u16_bits(a) == _u16_bits(b), hex(h)


def test_fp16_bf16_rounding_against_reference(orc, ref):
    L = orc.lib()
    rng = np.random.default_rng(5)
    bits = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)
    vals = bits.view(np.float32)
    extra = np.array([0.0, -0.0, 1e-8, 6e-8, 3e-8, 65504.0, 65520.0, 1e6, np.inf, -np.inf,
                      np.nan, 0.5, 2049.0, 6.1e-5, 6.09e-5], np.float32)
    for v in np.concatenate([vals, extra, (rng.standard_normal(50000) * 0.02).astype(np.float32)]):
        v = float(v)
        assert L.or_fp32_to_fp16(v) == ref.ref_fp32_to_fp16(v), v
        assert L.or_fp32_to_bf16(v) == ref.ref_fp32_to_bf16(v), v
    for h in range(0, 65536, 3):
        assert _u16_bits(L.or_bf16_to_fp32(h)) == _u16_bits(ref.ref_bf16_to_fp32(h))


def test_get_scale_min_k4_against_reference(orc, ref):
    import ctypes as C
    rng = np.random.default_rng(11)
    for _ in range(2000):
        q = rng.integers(0, 256, 12, dtype=np.uint8)
        for j in range(8):
            d1, m1, d2, m2 = C.c_uint8(), C.c_uint8(), C.c_uint8(), C.c_uint8()
            orc.lib().or_get_scale_min_k4(j, q, C.byref(d1), C.byref(m1))
            ref.ref_get_scale_min_k4(j, q, C.byref(d2), C.byref(m2))
            assert (d1.value, m1.value) == (d2.value, m2.value)


# ---------------------------------------------------------------------------
# block layouts


def _random_blocks(t, nblk, rng, sane_scales=True):
    """Random blocks; fp16 scales drawn finite when sane_scales."""
    bpb = {Q4_0: 18, Q8_0: 34, Q4_K: 144, Q6_K: 210}[t]
    w = rng.integers(0, 256, nblk * bpb, dtype=np.uint8).reshape(nblk, bpb)
    if sane_scales:
        d = (np.abs(rng.standard_normal(nblk)) * 0.02 + 1e-3).astype(np.float16).view(np.uint8).reshape(nblk, 2)
        dm = (np.abs(rng.standard_normal(nblk)) * 0.02 + 1e-3).astype(np.float16).view(np.uint8).reshape(nblk, 2)
        if t in (Q4_0, Q8_0, Q4_K):
            w[:, 0:2] = d
        if t == Q4_K:
            w[:, 2:4] = dm
        if t == Q6_K:
            w[:, 208:210] = d
    return w.reshape(-1)


@pytest.mark.parametrize("t", REF_TYPES)
def test_dequantize_bit_exact_against_quant_ref(orc, ref, t):
    rng = np.random.default_rng(100 + t)
    epb = orc.block_elems(t)
    for sane in (True, False):
        nblk = 64
        w = _random_blocks(t, nblk, rng, sane)
        mine = orc.dequantize(t, w, nblk * epb)
        theirs = np.zeros(nblk * epb, np.float32)
        assert ref.ref_dequant(t, w, nblk, theirs) == 0
        assert np.array_equal(mine.view(np.uint32), theirs.view(np.uint32))


def _unit_scale_blocks(t, nblk, rng):
    """Random codes with every scale set to 1 and every min to 0, so the
    reference dequantizer returns the (offset) integer code itself."""
    w = _random_blocks(t, nblk, rng).reshape(nblk, -1)
    one = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    if t in (Q4_0, Q8_0):
        w[:, 0:2] = one
    elif t == Q4_K:
        w[:, 0:2] = one
        w[:, 2:4] = 0
        w[:, 4:16] = np.array([1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1], np.uint8)
    elif t == Q6_K:
        w[:, 192:208] = 1
        w[:, 208:210] = one
    return w.reshape(-1)


@pytest.mark.parametrize("t", REF_TYPES)
def test_block_sums_one_hot_probe(orc, ref, t):
    """Integer sums of a one-hot activation return each element's code; with
    unit scales the reference dequantizer returns the same code (minus the
    fixed offset of Q4_0's unsigned nibble path)."""
    rng = np.random.default_rng(7 + t)
    K = 512
    epb = orc.block_elems(t)
    nblk = K // epb
    w = _unit_scale_blocks(t, nblk, rng)
    deq = np.zeros(K, np.float32)
    assert ref.ref_dequant(t, w, nblk, deq) == 0
    sub = 16 if t == Q6_K else 32
    qs = np.zeros((K, K), np.int8)
    qs[np.arange(K), np.arange(K)] = 1
    sums = orc.block_sums(t, w, qs, K, 1)[:, 0, :]        # [K probes, n_sub]
    codes = sums[np.arange(K), np.arange(K) // sub]
    others = sums.copy()
    others[np.arange(K), np.arange(K) // sub] = 0
    assert not others.any()
    expect = deq.astype(np.int64) + (8 if t == Q4_0 else 0)
    assert np.array_equal(codes.astype(np.int64), expect)


# ---------------------------------------------------------------------------
# quantizer


def test_quantizer_closed_form_properties(orc):
    rng = np.random.default_rng(3)
    M, K = 16, 4096
    x = rng.standard_normal((M, K)).astype(np.float32)
    mask = rng.random((M, K)) < 0.01
    x[mask] *= 20
    x[3, 64:96] = 0.0
    d, s, lo, hi, qs = orc.quantize_act(x)
    xb = x.reshape(M, K // 32, 32)
    qb = qs.reshape(M, K // 32, 32).astype(np.int32)
    amax = np.abs(xb).max(axis=2)
    assert np.array_equal(d, (amax / np.float32(127.0)).astype(np.float32))
    assert np.abs(qb).max() <= 127
    # the largest-magnitude element maps to +-127
    arg = np.abs(xb).argmax(axis=2)
    top = np.take_along_axis(qb, arg[..., None], axis=2)[..., 0]
    nz = amax > 0
    assert np.array_equal(np.abs(top[nz]), np.full(nz.sum(), 127))
    assert not qb[~nz].any() and not d[~nz].any() and not s[~nz].any()
    assert np.array_equal(lo.astype(np.int32), qb[..., :16].sum(axis=2))
    assert np.array_equal(hi.astype(np.int32), qb[..., 16:].sum(axis=2))
    assert np.array_equal(s, (d * (lo.astype(np.int32) + hi).astype(np.float32)).astype(np.float32))
    # |q*d - x| <= d/2 up to fp32 rounding of id
    err = np.abs(qb * d[..., None] - xb)
    assert (err <= d[..., None] * 0.5000001 + 1e-30).all()


def test_quantizer_round_half_even(orc):
    """amax = 127 gives d = id = 1 exactly, so x itself is rounded: ties go
    to even (vcvtnq_s32_f32), not away from zero."""
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    ties = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, 100.5, -100.5, 126.5], np.float32)
    x[1:1 + ties.size] = ties
    d, s, lo, hi, qs = orc.quantize_act(x)
    assert d[0, 0] == 1.0
    assert list(qs[0, 1:1 + ties.size]) == [0, 2, 2, 0, -2, -2, 4, 100, -100, 126]


def test_quantizer_nonfinite_blocks(orc):
    x = np.ones((1, 96), np.float32)
    x[0, 5] = np.nan
    x[0, 40] = np.inf
    d, s, lo, hi, qs = orc.quantize_act(x)
    assert np.isnan(d[0, 0]) and not qs[0, :32].any()     # NaN amax: id = 0
    assert np.isinf(d[0, 1]) and not qs[0, 32:64].any()   # inf amax: id = 0, inf*0 -> 0
    assert d[0, 2] == np.float32(1.0) / np.float32(127.0)
    assert (qs[0, 64:] == 127).all()


# ---------------------------------------------------------------------------
# the reference's dual-reference acceptance test


def _ref_rows(orc, ref, t, w, K, N):
    epb = orc.block_elems(t)
    out = np.zeros(K * N, np.float32)
    assert ref.ref_dequant(t, w, (K // epb) * N, out) == 0
    return out.reshape(N, K)


def _q8_roundtrip(orc, x):
    d, s, lo, hi, qs = orc.quantize_act(x)
    return (qs.reshape(x.shape[0], -1, 32).astype(np.float32) * d[..., None]).reshape(x.shape)


def _almost_equal(a, b, rel, abs_tol):
    diff = np.abs(a - b)
    return (diff <= abs_tol) | (diff <= rel * np.maximum(np.abs(a), np.abs(b)))


CASES = [(t, 512, n) for n in (1, 8, 33, 256) for t in REF_TYPES] + \
        [(t, 2816, n) for n in (1, 8, 256, 4096) for t in (Q4_K, Q6_K)]


@pytest.mark.parametrize("t,K,N", CASES)
def test_dual_reference(orc, ref, t, K, N):
    w = orc.ref_test_weights(t, K, N)
    x = orc.ref_test_x(t, K)[None, :]
    rows = _ref_rows(orc, ref, t, w, K, N).astype(np.float64)
    y_exact = (x.astype(np.float64) @ rows.T)[0]
    y_q8 = (_q8_roundtrip(orc, x).astype(np.float64) @ rows.T)[0]

    y_int = orc.gemm_int(t, x, w, N)[0]
    y_sc = orc.gemm_scalar(t, x, w, N)[0]
    # the reference's own acceptance (either reference, rel 1e-3 / abs 1e-3)
    ok = _almost_equal(y_int, y_exact, 1e-3, 1e-3) | _almost_equal(y_int, y_q8, 1e-3, 1e-3)
    assert ok.all()
    # The scalar path's sequential fp32 sum misses the per-element criterion
    # at heavy cancellation only (Q6_K K=2816 N=4096, output 2642: -0.079195
    # vs exact -0.078987 with max|y| = 439; an fp32 emulation of the
    # reference's loop order in numpy gives the same -0.07919508), so
    # outputs below 1e-3 of the row maximum are judged normwise instead.
    ok = _almost_equal(y_sc, y_exact, 1e-3, 1e-4) | (np.abs(y_exact) < 1e-3 * np.abs(y_exact).max())
    assert ok.all()
    # tighter: the int path IS the Q8 round-trip product up to fp32 rounding
    scale = np.abs(y_q8).max()
    assert np.abs(y_int - y_q8).max() <= 2e-6 * scale
    assert np.abs(y_sc - y_exact).max() <= 2e-6 * np.abs(y_exact).max()


def test_batched_rows_equal_single(orc):
    """tests/test_matmul.cpp:217-250 shape (M=7, K=512, N=64), random bytes."""
    M, K, N = 7, 512, 64
    for t in (Q8_0, Q4_K, Q4_0, Q6_K):
        rng = np.random.default_rng(41 + t)
        w = rng.integers(0, 256, orc.row_bytes(t, K) * N, dtype=np.uint8)
        x = rng.uniform(-1, 1, (M, K)).astype(np.float32)
        yb = orc.gemm_int(t, x, w, N)
        for m in range(M):
            ys = orc.gemm_int(t, x[m], w, N)[0]
            assert np.array_equal(yb[m].view(np.uint32), ys.view(np.uint32))
        ys1 = orc.gemm_scalar(t, x, w, N, nthreads=1)
        ys8 = orc.gemm_scalar(t, x, w, N, nthreads=8)
        assert np.array_equal(ys1.view(np.uint32), ys8.view(np.uint32))


@pytest.mark.parametrize("multi", [False, True])
def test_moe_equals_per_expert_gemm(orc, multi):
    """moe_gemv_int equals the sequential fallback of src/matmul.cpp:469-476
    (/:493-499): matmul_row on each selected expert's slice."""
    t, E, K, N = Q4_K, 6, 512, 40
    rng = np.random.default_rng(9)
    rb = orc.row_bytes(t, K)
    w = _random_blocks(t, E * N * (K // 256), rng)
    idx = np.array([4, 1, 5, 1], np.int32)
    x = rng.standard_normal((idx.size if multi else 1, K)).astype(np.float32)
    y = orc.moe_gemv_int(t, x, w, idx, K, N, multi)
    for k, e in enumerate(idx):
        sl = w[e * N * rb:(e + 1) * N * rb]
        yk = orc.gemm_int(t, x[k if multi else 0], sl, N)[0]
        assert np.array_equal(y[k].view(np.uint32), yk.view(np.uint32))


@pytest.mark.parametrize("t", [Q5_0, Q2_K, Q3_K, Q5_K, F16, BF16, F32])
def test_scalar_dot_matches_own_dequantize(orc, t):
    """Types outside quant_ref.h: the scalar dot and dequantize of the same
    blocks agree. This is a consistency check only; the field layouts are
    pinned by the closed-form probes in test_oracle_probes.py, and the GPU
    kernels for these types are checked against the oracle in
    test_gpu_fact.py."""
    K, N = 512, 16
    rng = np.random.default_rng(200 + t)
    nbytes = orc.row_bytes(t, K) * N
    if t in (F32,):
        w = rng.standard_normal(K * N).astype(np.float32).view(np.uint8).copy()
    elif t in (F16,):
        w = rng.standard_normal(K * N).astype(np.float16).view(np.uint8).copy()
    elif t in (BF16,):
        w = (rng.standard_normal(K * N).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).copy()
    else:
        w = rng.integers(0, 256, nbytes, dtype=np.uint8)
        bpb = int(orc.lib().or_bytes_per_block(t))
        blocks = w.reshape(-1, bpb)
        dd = (np.abs(rng.standard_normal(blocks.shape[0])) * 0.02 + 1e-3).astype(np.float16).view(np.uint8).reshape(-1, 2)
        off = {Q5_0: [0], Q2_K: [80, 82], Q3_K: [108], Q5_K: [0, 2]}[t]
        for o in off:
            blocks[:, o:o + 2] = dd
    x = rng.uniform(-1, 1, (1, K)).astype(np.float32)
    rows = orc.dequantize(t, w, K * N).reshape(N, K).astype(np.float64)
    y = orc.gemm_scalar(t, x, w, N)[0]
    exact = (x.astype(np.float64) @ rows.T)[0]
    assert np.abs(y - exact).max() <= 1e-5 * max(np.abs(exact).max(), 1e-3)


from moe_layer import moe_layer_inputs as _moe_layer_inputs  # noqa: E402


def test_moe_ffn_restatement_against_float64(orc):
    """or_moe_ffn (Gemma4Arch::moe_ffn, src/arch_gemma4.cpp:507-641) against
    an independent float64 evaluation of the same mathematics, with the
    expert GEMVs taken from the oracle's moe_gemv_int (pinned separately):
    router norm and scale, softmax, top-k, renormalised weights (checked
    against argsort), expert norm, GeGLU with gate = the first `inter`
    outputs, weighted sum with down_scale."""
    rng = np.random.default_rng(5)
    T, H, n_exp, top_k, inter = 3, 512, 16, 4, 256
    p = _moe_layer_inputs(rng, H, n_exp, inter, Q4_K, Q4_K)
    x = (rng.standard_normal((T, H)) * 2.0).astype(np.float32)
    out, idx, wts = orc.moe_ffn(x, p["router_w"], F32, p["router_scale"], p["pre_norm"], p["eps"],
                                p["gu_w"], Q4_K, p["dn_w"], Q4_K, p["down_scale"], n_exp, top_k, inter)
    rw = p["router_w"].view(np.float32).reshape(n_exp, H).astype(np.float64)
    for t in range(T):
        xr = x[t].astype(np.float64)
        inv = 1.0 / np.sqrt(np.mean(xr * xr) + p["eps"])
        logits = (xr * inv * p["router_scale"] / np.sqrt(H)) @ rw.T
        prob = np.exp(logits - logits.max())
        prob /= prob.sum()
        order = np.argsort(-prob, kind="stable")[:top_k]
        assert np.array_equal(idx[t], order)
        wk = prob[order] / prob[order].sum()
        assert np.allclose(wts[t], wk, rtol=1e-5, atol=1e-7)
        ein = (xr * inv * p["pre_norm"]).astype(np.float32)
        gu = orc.moe_gemv_int(Q4_K, ein[None, :], p["gu_w"], idx[t], H, 2 * inter, False).astype(np.float64)
        g, u = gu[:, :inter], gu[:, inter:]
        hidden = 0.5 * g * (1.0 + np.tanh(0.7978845608028654 * (g + 0.044715 * g ** 3))) * u
        eo = orc.moe_gemv_int(Q4_K, hidden.astype(np.float32), p["dn_w"], idx[t], inter, H, True).astype(np.float64)
        ref = ((wk * p["down_scale"][idx[t]])[:, None] * eo).sum(axis=0)
        assert np.abs(out[t] - ref).max() <= 1e-4 * np.abs(ref).max()
