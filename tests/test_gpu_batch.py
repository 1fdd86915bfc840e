"""GPU parity of the batched M=1 matmuls (lp_gemm_batch / lp_gemm_batch_dev),
the drop-in for matmul_gemm_batch (src/matmul.h:46-54,
src/matmul.cpp:450-454): each spec's y must equal the single-spec GEMV of
the same inputs bit for bit (a multi-matrix launch runs the same per-row
arithmetic) and the oracle's int8-path result within the fp32 bar."""
import ctypes as C

import numpy as np
import pytest

from hip_util import (Q4_0, Q4_K, Q6_K, Q8_0, L, gemm_dev, normwise, stream, synth_weights, synth_x,
                      to_dev, torch_dev)
from laplace_amd import _lib
from laplace_amd._lib import BatchSpec

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _run_dev(specs):
    """specs: list of (x[K] numpy, w numpy, type, N). Device path, one call."""
    torch = torch_dev()
    keep, arr = [], (BatchSpec * len(specs))()
    xs = {}
    ys = []
    for i, (x, w, t, N) in enumerate(specs):
        key = id(x)
        if key not in xs:
            xs[key] = to_dev(np.ascontiguousarray(x, np.float32))
        xd, wd = xs[key], to_dev(w)
        y = torch.full((max(N, 1),), float("nan"), dtype=torch.float32, device="cuda")
        keep += [xd, wd]
        ys.append(y)
        arr[i] = BatchSpec(xd.data_ptr(), wd.data_ptr(), t, y.data_ptr(), x.shape[-1], N)
    nb = int(L().lp_gemm_batch_workspace_bytes(arr, len(specs)))
    ws = torch.empty(max(nb, 1), dtype=torch.uint8, device="cuda")
    _lib.check(L().lp_gemm_batch_dev(arr, len(specs), ws.data_ptr(), nb, stream()), "lp_gemm_batch_dev")
    torch.cuda.synchronize()
    return [y.cpu().numpy()[:N] for y, (_, _, _, N) in zip(ys, specs)]


def _run_host(specs):
    arr = (BatchSpec * len(specs))()
    ys = []
    for i, (x, w, t, N) in enumerate(specs):
        y = np.full(max(N, 1), np.nan, np.float32)
        ys.append(y)
        arr[i] = BatchSpec(x.ctypes.data, w.ctypes.data, t, y.ctypes.data, x.shape[-1], N)
    assert L().lp_gemm_batch(arr, len(specs)), L().lp_last_error()
    return [y[:N] for y, (_, _, _, N) in zip(ys, specs)]


def _check(orc, specs, outs):
    for (x, w, t, N), y in zip(specs, outs):
        if N == 0:
            continue
        single = gemm_dev(t, x, w, N)[0]
        assert np.array_equal(y.view(np.uint32), single.view(np.uint32)), f"type {t} N {N}"
        assert normwise(y, orc.gemm_int(t, x[None], w, N)[0]) <= TOL


def test_qkv_batch_one_launch(orc):
    """Q/K/V of a shared x (src/arch_gemma4.cpp:318-327): three Q4_K specs."""
    print("batch qkv K=2048", flush=True)
    K = 2048
    x = synth_x(1, K, seed=3)[0]
    specs = [(x, synth_weights(Q4_K, K, N, seed=10 + i), Q4_K, N) for i, N in enumerate([512, 128, 128])]
    _check(orc, specs, _run_dev(specs))


def test_gate_up_batch_ragged_rows(orc):
    """gate/up of a shared x (src/arch_gemma4.cpp:694-700) with row counts that
    are not multiples of a wave's row group, at the headline K."""
    print("batch gate/up K=4096", flush=True)
    K = 4096
    x = synth_x(1, K, seed=5, outliers=0.01)[0]
    specs = [(x, synth_weights(Q4_K, K, 301, seed=21), Q4_K, 301),
             (x, synth_weights(Q4_K, K, 77, seed=22), Q4_K, 77)]
    _check(orc, specs, _run_dev(specs))


def test_batch_longer_than_one_launch_and_empty_spec(orc):
    """Six Q4_K specs on one x (split 4 + 2), one of them with N = 0."""
    print("batch six specs K=3584", flush=True)
    K = 3584
    x = synth_x(1, K, seed=7)[0]
    Ns = [64, 0, 33, 128, 5, 96]
    specs = [(x, synth_weights(Q4_K, K, max(N, 1), seed=30 + i), Q4_K, N) for i, N in enumerate(Ns)]
    _check(orc, specs, _run_dev(specs))


def test_mixed_batch_falls_back_per_spec(orc):
    """Other types and distinct activation rows run one spec at a time."""
    print("batch mixed types", flush=True)
    K = 1024
    x1, x2 = synth_x(1, K, seed=8)[0], synth_x(1, K, seed=9)[0]
    specs = [(x1, synth_weights(Q6_K, K, 40, seed=41), Q6_K, 40),
             (x1, synth_weights(Q4_K, K, 64, seed=42), Q4_K, 64),
             (x2, synth_weights(Q4_K, K, 64, seed=43), Q4_K, 64),
             (x2, synth_weights(Q8_0, K, 48, seed=44), Q8_0, 48),
             (x2, synth_weights(Q4_0, K, 16, seed=45), Q4_0, 16)]
    _check(orc, specs, _run_dev(specs))


def test_host_batch_matches_device_batch(orc):
    """The synchronous host-pointer entry (the drop-in) returns what the device
    form computes."""
    print("batch host path", flush=True)
    K = 2048
    x = synth_x(1, K, seed=11)[0]
    x2 = synth_x(1, K, seed=12)[0]
    specs = [(x, synth_weights(Q4_K, K, 256, seed=51), Q4_K, 256),
             (x, synth_weights(Q4_K, K, 64, seed=52), Q4_K, 64),
             (x2, synth_weights(Q6_K, K, 32, seed=53), Q6_K, 32)]
    host = _run_host(specs)
    dev = _run_dev(specs)
    for a, b in zip(host, dev):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_batch_rejects_bad_spec():
    """A spec with an unsupported type is LP_UNSUPPORTED before anything runs."""
    x = synth_x(1, 256, seed=1)[0]
    w = np.zeros(20 * 16, np.uint8)
    arr = (BatchSpec * 1)(BatchSpec(x.ctypes.data, w.ctypes.data, 3, x.ctypes.data, 256, 16))
    assert not L().lp_gemm_batch(arr, 1)
    assert L().lp_gemm_batch_dev(arr, 1, None, 0, None) == _lib.LP_UNSUPPORTED


def test_host_batch_shared_weight_different_n(orc):
    """Two specs read the same host weight pointer over different lengths
    (the second spec's N is larger). The batch resolves the pointer once for
    the longer span, so the first spec does not read a freed device copy."""
    K, Nbig, Nsmall = 1024, 384, 128
    w = synth_weights(Q4_K, K, Nbig, seed=71)
    x = synth_x(1, K, 72)[0]
    L().lp_release_weights()
    specs = [(x, w, Q4_K, Nsmall), (x, w, Q4_K, Nbig)]
    outs = _run_host(specs)
    L().lp_release_weights()
    ref = orc.gemm_int(Q4_K, x[None], w, Nbig)[0]
    assert normwise(outs[1], ref) <= TOL
    assert normwise(outs[0], ref[:Nsmall]) <= TOL
    assert np.array_equal(outs[0].view(np.uint32), outs[1][:Nsmall].view(np.uint32))


def test_registered_region_unaligned_base(orc):
    """A region registered at a base that is not 256-byte aligned: its
    device copy keeps the host alignment modulo 256, so a 16-byte-aligned
    Q4_K tensor inside it runs on the aligned kernels and matches the
    oracle; lp_release_region drops only that region."""
    K, N = 1024, 256
    w = synth_weights(Q4_K, K, N, seed=73)
    x = synth_x(1, K, 74)
    buf = np.zeros(w.nbytes + 512, np.uint8)
    base = buf[48:]                      # base % 256 != 0 in general
    pad = (-(base.ctypes.data + 16)) % 16
    tensor = base[16 + pad:16 + pad + w.nbytes]
    tensor[:] = w
    _lib.check(L().lp_register_weights(base.ctypes.data, base.nbytes), "lp_register_weights")
    y = np.zeros(N, np.float32)
    assert L().lp_gemm(x.ctypes.data, tensor.ctypes.data, Q4_K, y.ctypes.data, 1, K, N), L().lp_last_error()
    assert normwise(y, orc.gemm_int(Q4_K, x, w, N)[0]) <= TOL
    assert L().lp_release_region(base.ctypes.data) == 0
    assert L().lp_release_region(base.ctypes.data) != 0   # already dropped
