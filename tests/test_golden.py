"""Committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py): the oracle must reproduce them bit for bit
(CPU), and the GPU path must match them - activation blocks and per-block
int32 sums bit-exact, fp32 outputs within normwise 1e-4 of the int8-path
result (tests/test_metal.cpp:200-203 form)."""
import glob
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURES = sorted(glob.glob(os.path.join(HERE, "golden", "*.npz")))
IDS = [os.path.basename(p)[:-4] for p in FIXTURES]


def load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_fixtures_present():
    assert len(FIXTURES) == 4


@pytest.mark.parametrize("path", FIXTURES, ids=IDS)
def test_oracle_reproduces_fixture(orc, path):
    f = load(path)
    t, K, N = int(f["type"]), int(f["K"]), int(f["N"])
    w, x = f["w"], f["x"]
    assert np.array_equal(orc.ref_test_weights(t, K, N), w)
    for M in (1, 4):
        xm = x[:M]
        d, s, lo, hi, qs = orc.quantize_act(xm)
        for name, got in (("d", d), ("sum", s), ("sum_lo", lo), ("sum_hi", hi), ("qs", qs)):
            assert np.array_equal(got.view(np.uint8), f[f"{name}_m{M}"].view(np.uint8)), name
        assert np.array_equal(orc.block_sums(t, w, qs, K, N), f[f"bsum_m{M}"])
        assert np.array_equal(orc.gemm_int(t, xm, w, N).view(np.uint32), f[f"y_int_m{M}"].view(np.uint32))
        assert np.array_equal(orc.gemm_scalar(t, xm, w, N).view(np.uint32),
                              f[f"y_scalar_m{M}"].view(np.uint32))
    assert np.array_equal(orc.dequantize(t, w, N * K).view(np.uint32), f["deq"].view(np.uint32))


@pytest.mark.parametrize("path", FIXTURES, ids=IDS)
def test_fixture_invariants(path):
    """Closed-form properties the fixture itself must satisfy."""
    f = load(path)
    for M in (1, 4):
        qs = f[f"qs_m{M}"].astype(np.int32).reshape(M, -1, 32)
        assert np.abs(qs).max() <= 127
        lo, hi = f[f"sum_lo_m{M}"].astype(np.int32), f[f"sum_hi_m{M}"].astype(np.int32)
        assert np.array_equal(lo, qs[:, :, :16].sum(-1)) and np.array_equal(hi, qs[:, :, 16:].sum(-1))
        d = f[f"d_m{M}"]
        assert (qs[d == 0] == 0).all()
        # the amax element of every non-zero block maps to +-127
        assert (np.abs(qs).max(-1)[d > 0] == 127).all()
    if f["x"].shape[0] >= 3:
        # exact ties of row 2, block 2 (d = 1): 0.5 -> 0, 1.5 -> 2, 2.5 -> 2, 3.5 -> 4
        q = f["qs_m4"][2, 64:72].astype(int)
        assert list(q) == [127, 0, 2, 2, 0, -2, -2, 4]


@pytest.mark.gpu
@pytest.mark.parametrize("path", FIXTURES, ids=IDS)
def test_gpu_matches_fixture(path):
    from hip_util import block_sums_dev, gemm_dev, normwise, quantize_dev
    f = load(path)
    t, K, N = int(f["type"]), int(f["K"]), int(f["N"])
    w, x = f["w"], f["x"]
    for M in (1, 4):
        xm = np.ascontiguousarray(x[:M])
        d, s, s16, qs = quantize_dev(xm)
        assert np.array_equal(d.view(np.uint32), f[f"d_m{M}"].view(np.uint32))
        assert np.array_equal(s.view(np.uint32), f[f"sum_m{M}"].view(np.uint32))
        assert np.array_equal(qs, f[f"qs_m{M}"])
        lo = (s16.astype(np.uint32) & 0xFFFF).astype(np.uint16).view(np.int16)
        hi = (s16.astype(np.uint32) >> 16).astype(np.uint16).view(np.int16)
        assert np.array_equal(lo, f[f"sum_lo_m{M}"]) and np.array_equal(hi, f[f"sum_hi_m{M}"])
        assert np.array_equal(block_sums_dev(t, xm, w, N), f[f"bsum_m{M}"])
        y = gemm_dev(t, xm, w, N)
        assert normwise(y, f[f"y_int_m{M}"]) <= 1e-4
