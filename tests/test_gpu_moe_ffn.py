"""The MoE feed-forward layer on the device (lp_moe_ffn_dev) against the
oracle's restatement of Gemma4Arch::moe_ffn (src/arch_gemma4.cpp:507-641):
same routing (expert ids exactly, weights to fp32 rounding) and outputs
within 1e-4 normwise (int8 expert GEMVs as the reference's back-end; the
norms, softmax and GeGLU reassociate fp32 sums and use the device's
exp/tanh)."""
import numpy as np
import pytest

from moe_layer import moe_layer_inputs
from hip_util import normwise, to_dev

pytestmark = pytest.mark.gpu

F32, Q4_0, Q8_0, Q4_K, Q6_K = 0, 2, 8, 12, 14


def run_both(orc, T, H, n_exp, top_k, inter, gu_t, dn_t, router_t, seed, paired_router=False, nan_row=None):
    import torch
    from laplace_amd.matmul import Tensor
    from laplace_amd.moe import moe_ffn
    rng = np.random.default_rng(seed)
    p = moe_layer_inputs(rng, H, n_exp, inter, gu_t, dn_t, router_t)
    if paired_router:
        # F32 router rows 2i and 2i+1 identical: every logit appears twice
        r = p["router_w"].view(np.float32).reshape(n_exp, H)
        r[1::2] = r[0::2]
    if nan_row is not None:
        # one F32 router row of NaN: that expert's logit is NaN for every token
        p["router_w"].view(np.float32).reshape(n_exp, H)[nan_row] = np.nan
    x = (rng.standard_normal((T, H)) * 2.0).astype(np.float32)
    ref, ridx, rw = orc.moe_ffn(x, p["router_w"], router_t, p["router_scale"], p["pre_norm"], p["eps"],
                                p["gu_w"], gu_t, p["dn_w"], dn_t, p["down_scale"], n_exp, top_k, inter)
    out, idx, wts = moe_ffn(to_dev(x), Tensor(router_t, (H, n_exp), to_dev(p["router_w"])),
                            to_dev(p["router_scale"]), to_dev(p["pre_norm"]), p["eps"],
                            Tensor(gu_t, (H, 2 * inter), to_dev(p["gu_w"])),
                            Tensor(dn_t, (inter, H), to_dev(p["dn_w"])), to_dev(p["down_scale"]),
                            n_exp, top_k, inter, return_routing=True)
    torch.cuda.synchronize()
    return (out.cpu().numpy(), idx.cpu().numpy(), wts.cpu().numpy()), (ref, ridx, rw)


@pytest.mark.parametrize("T,H,n_exp,top_k,inter,gu_t,dn_t,router_t", [
    (1, 512, 16, 4, 256, Q4_K, Q4_K, F32),
    (4, 512, 32, 8, 256, Q4_K, Q6_K, F32),
    # 32 pairs over 8 experts: both passes on the row-quad group kernel, the
    # down pass quantizing GeGLU(gate|up) while it stages its activations
    (4, 512, 8, 8, 256, Q4_K, Q4_K, F32),
    (7, 1024, 64, 2, 512, Q8_0, Q4_0, Q8_0),
    # Gemma4 26B layer shape (tests/bench_cpu_gpu.cpp:55-57): H 2816, 128
    # experts, top-8, expert inter 704 (down K = 704: a Q8_0 tensor)
    (2, 2816, 128, 8, 704, Q4_K, Q8_0, F32),
    # 144 pairs over 16 experts (9 per expert): both expert passes on the MFMA
    # group kernel
    (72, 512, 16, 2, 256, Q4_K, Q4_K, F32),
], ids=lambda v: str(v))
def test_moe_ffn_matches_oracle(orc, T, H, n_exp, top_k, inter, gu_t, dn_t, router_t):
    (out, idx, wts), (ref, ridx, rw) = run_both(orc, T, H, n_exp, top_k, inter, gu_t, dn_t, router_t,
                                                seed=T + H + n_exp)
    assert np.array_equal(idx, ridx)
    assert np.allclose(wts, rw, rtol=1e-5, atol=1e-7)
    assert np.isfinite(out).all()
    assert normwise(out, ref) <= 1e-4


@pytest.mark.parametrize("T,top_k", [(1, 3), (3, 5), (9, 3)])
def test_moe_ffn_router_ties(orc, T, top_k):
    """Experts in pairs with identical router rows, so the logits tie exactly:
    the top-k takes the lower expert index first (the reference's strict '>'
    scan, src/arch_gemma4.cpp:546-563) in both the one-launch top-k and route
    kernel (T <= 4) and the separate top-k kernel."""
    (out, idx, wts), (ref, ridx, rw) = run_both(orc, T, 512, 32, top_k, 256, Q4_K, Q4_K, F32,
                                                seed=100 + T, paired_router=True)
    assert np.array_equal(idx, ridx)
    assert np.allclose(wts, rw, rtol=1e-5, atol=1e-7)
    assert normwise(out, ref) <= 1e-4


@pytest.mark.parametrize("T,nan_row", [(1, 5), (3, 0), (9, 17)])
def test_moe_ffn_nan_router(orc, T, nan_row):
    """A NaN router logit makes every softmax probability NaN. The
    reference's scan (best = 0, strict '>', src/arch_gemma4.cpp:555-559) then
    picks expert 0 for every k, so every pick must stay in range and equal the
    oracle's (all zero), in both top-k kernels (T <= 4 and beyond); the
    weights and outputs are NaN on both sides."""
    (out, idx, wts), (ref, ridx, rw) = run_both(orc, T, 512, 32, 4, 256, Q4_K, Q4_K, F32,
                                                seed=300 + T, nan_row=nan_row)
    assert (ridx == 0).all()
    assert np.array_equal(idx, ridx)
    assert np.array_equal(np.isnan(wts), np.isnan(rw))
    assert np.array_equal(np.isnan(out), np.isnan(ref))


def test_moe_ffn_rejects_bad_shapes():
    """top_k beyond 16 or n_exp, and more than 1024 experts, are LP_EINVAL."""
    from laplace_amd import _lib
    L = _lib.lib()
    for n_exp, top_k in [(8, 9), (32, 17), (2048, 4), (8, 0)]:
        rc = L.lp_moe_ffn_dev(None, 1, 256, None, 0, None, None, 1e-6, None, 12, None, 12, None,
                              n_exp, top_k, 256, None, None, None, None, 0, None)
        assert rc == _lib.LP_EINVAL
