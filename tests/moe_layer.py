"""Seeded inputs of a small Gemma4-style MoE layer (shared by the oracle and
GPU tests): router weights, router and pre-norm scales, quantized gate/up and
down experts with finite small fp16 scales, per-expert down scales."""
import numpy as np

import oracle.oracle as orc_mod
from oracle.oracle import F32, Q4_0, Q4_K, Q6_K, Q8_0


def moe_layer_inputs(rng, H, n_exp, inter, gu_t, dn_t, router_t=F32):
    """Weights of a small MoE layer: F32 router, quantized experts with
    finite small scales, router/pre-norm scales and per-expert down scales."""
    def blocks(t, K, N, n_mat):
        nb = orc_mod.row_bytes(t, K) * N * n_mat
        w = rng.integers(0, 256, nb, dtype=np.uint8)
        bpb = int(orc_mod.lib().or_bytes_per_block(t))
        b = w.reshape(-1, bpb)
        off = {Q4_K: [0, 2], Q8_0: [0], Q4_0: [0], Q6_K: [208]}[t]
        for o in off:
            b[:, o:o + 2] = (np.abs(rng.standard_normal(b.shape[0])) * 0.01).astype(np.float16).view(np.uint8).reshape(-1, 2)
        if t == Q8_0:
            b[:, 2:] = rng.integers(-127, 128, (b.shape[0], 32), dtype=np.int8).view(np.uint8)
        return w
    if router_t == F32:
        router = (rng.standard_normal(n_exp * H) * 0.5).astype(np.float32).view(np.uint8).copy()
    else:
        router = blocks(router_t, H, n_exp, 1)
    return dict(router_w=router, router_type=router_t,
                router_scale=(1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32),
                pre_norm=(1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32), eps=1e-6,
                gu_w=blocks(gu_t, H, 2 * inter, n_exp), gu_type=gu_t,
                dn_w=blocks(dn_t, inter, H, n_exp), dn_type=dn_t,
                down_scale=(0.5 + rng.random(n_exp)).astype(np.float32),
                n_exp=n_exp, inter=inter)
