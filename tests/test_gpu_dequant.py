"""GPU dequantize (lp_dequantize / lp_dequantize_dev) against the oracle's
restatement of src/matmul.cpp:504-675, which is itself checked bit for bit
against the reference's quant_ref dequantizers on the CPU. Bar: bit-exact
(NaN outputs from NaN/Inf block scales compare as NaN)."""
import numpy as np
import pytest

from hip_util import L, stream, to_dev, torch_dev
from laplace_amd import _lib

pytestmark = pytest.mark.gpu

TYPES = {"F32": (0, 1, 4), "F16": (1, 1, 2), "BF16": (30, 1, 2), "Q4_0": (2, 32, 18),
         "Q5_0": (6, 32, 22), "Q8_0": (8, 32, 34), "Q2_K": (10, 256, 84), "Q3_K": (11, 256, 110),
         "Q4_K": (12, 256, 144), "Q5_K": (13, 256, 176), "Q6_K": (14, 256, 210)}


def same(a, b):
    a32, b32 = a.view(np.uint32), b.view(np.uint32)
    nan = np.isnan(a) & np.isnan(b)
    return bool(((a32 == b32) | nan).all())


def dequant_dev(t, w, n):
    torch = torch_dev()
    wd = to_dev(w)
    out = torch.empty(max(n, 1), dtype=torch.float32, device="cuda")
    _lib.check(L().lp_dequantize_dev(wd.data_ptr(), t, out.data_ptr(), n, stream()), "dequantize_dev")
    torch.cuda.synchronize()
    return out.cpu().numpy()[:n]


@pytest.mark.parametrize("name", list(TYPES))
def test_dequant_random_bytes(orc, name):
    t, epb, bpb = TYPES[name]
    nblk = 4096 // epb if epb > 1 else 20000
    rng = np.random.default_rng(t)
    w = rng.integers(0, 256, nblk * bpb, dtype=np.uint8)
    n = nblk * epb
    got = dequant_dev(t, w, n)
    assert same(got, orc.dequantize(t, w, n))


@pytest.mark.parametrize("name", ["Q4_0", "Q8_0", "Q4_K", "Q6_K", "Q5_K", "Q3_K", "Q2_K", "Q5_0"])
def test_dequant_finite_scales_exact(orc, name):
    """Realistic blocks (finite small fp16 scales): every output bit-exact and finite."""
    t, epb, bpb = TYPES[name]
    from laplace_amd.matmul import row_bytes  # noqa: F401
    rng = np.random.default_rng(100 + t)
    nblk = 512
    w = rng.integers(0, 256, nblk * bpb, dtype=np.uint8).reshape(nblk, bpb)
    scale_at = {2: [0], 6: [0], 8: [0], 10: [80, 82], 11: [108], 12: [0, 2], 13: [0, 2], 14: [208]}[t]
    for off in scale_at:
        w[:, off:off + 2] = (np.abs(rng.standard_normal(nblk)) * 0.01).astype(np.float16).view(np.uint8).reshape(-1, 2)
    w = w.reshape(-1)
    got = dequant_dev(t, w, nblk * epb)
    ref = orc.dequantize(t, w, nblk * epb)
    assert np.isfinite(got).all()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_dequant_f16_exhaustive(orc):
    w = np.arange(65536, dtype=np.uint16).view(np.uint8)
    assert same(dequant_dev(1, w, 65536), orc.dequantize(1, w, 65536))


def test_dequant_host_api_and_errors(orc):
    t, n = 12, 256 * 8
    rng = np.random.default_rng(3)
    w = rng.integers(0, 256, 8 * 144, dtype=np.uint8)
    out = np.zeros(n, np.float32)
    assert L().lp_dequantize(w.ctypes.data, t, out.ctypes.data, n) == _lib.LP_OK
    assert same(out, dequant_dev(t, w, n))
    assert L().lp_dequantize(w.ctypes.data, 9, out.ctypes.data, 32) == _lib.LP_UNSUPPORTED
    assert L().lp_dequantize(w.ctypes.data, t, out.ctypes.data, 100) == _lib.LP_EINVAL
    assert L().lp_dequantize(w.ctypes.data, t, out.ctypes.data, 0) == _lib.LP_OK
    L().lp_release_weights()


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("shift", [1, 2, 4, 8])
def test_dequant_unaligned_weights(orc, name, shift):
    """Weights at an offset from the allocation (1, 2, 4 or 8 bytes): the
    types whose eight-output path needs an aligned pointer (16 bytes for
    F32/F16/BF16, 8 for Q4_K/Q5_K, 2 for Q4_0/Q5_0/Q8_0/Q6_K) fall back to
    the per-element decode; every output bit-exact."""
    torch = torch_dev()
    t, epb, bpb = TYPES[name]
    nblk = 2048 // epb if epb > 1 else 2048
    rng = np.random.default_rng(7 * t + shift)
    w = rng.integers(0, 256, nblk * bpb, dtype=np.uint8)
    n = nblk * epb
    buf = torch.zeros(len(w) + 16, dtype=torch.uint8, device="cuda")
    buf[shift:shift + len(w)] = torch.from_numpy(w).to("cuda")
    out = torch.empty(n, dtype=torch.float32, device="cuda")
    _lib.check(L().lp_dequantize_dev(buf.data_ptr() + shift, t, out.data_ptr(), n, stream()), "dequantize_dev")
    torch.cuda.synchronize()
    assert same(out.cpu().numpy(), orc.dequantize(t, w, n))
