"""Writes the small golden fixtures tests/golden/<TYPE>_K512_N8.npz.

Inputs: the weights come from the reference test suite's own generator and
seeds (XorShift32, tests/test_util.h:49-61, tests/test_matmul.cpp:272-291,
as restated in oracle/lp_oracle.c:or_ref_test_weights); the activations are
4 rows of length 512: row 0 is the reference's test vector for the type
(tests/test_matmul.cpp:272-291), rows 1-3 are seeded N(0,1) with edge cases
(an all-zero block, a block with exact .5 ties after scaling, a large
outlier, a negative-only block).

Expected outputs, per M in {1, 4} (M=1 uses row 0):
  d, sum, sum_lo, sum_hi, qs   ActQ8 blocks (src/matmul_simd.cpp:348-410)
  bsum                          per-sub-block int32 dots [M, N, S]
  y_int                         int8-activation GEMM (src/matmul_simd.cpp:432-455)
  y_scalar                      fp32 scalar GEMM (src/matmul.cpp:320-334)
  deq                           dequantized weights [N*K]
All from oracle/liboracle.so. `deq` is also produced by the reference's own
dequantizers (tests/quant_ref.h:47-110, built as oracle/_ref/libref.so from
the reference's sources) and the script refuses to write a fixture where
the two disagree.

Run from the repository root: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import oracle as orc  # noqa: E402

TYPES = {"Q8_0": 8, "Q4_0": 2, "Q4_K": 12, "Q6_K": 14}
K, N = 512, 8
OUT = os.path.dirname(os.path.abspath(__file__))


def activations(t: int) -> np.ndarray:
    rng = np.random.default_rng(1000 + t)
    x = rng.standard_normal((4, K)).astype(np.float32)
    x[0] = orc.ref_test_x(t, K)
    x[1, 32:64] = 0.0                                  # d = 0 block
    # ties: amax 127 makes id = 1, so the halves round to even
    x[2, 64:96] = np.array([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5] * 4, np.float32)
    x[3, 5] = 400.0                                    # outlier
    x[3, 96:128] = -np.abs(x[3, 96:128])               # negative-only block
    return x


def main():
    orc.build()
    have_ref = orc.ref_available()
    for name, t in TYPES.items():
        w = orc.ref_test_weights(t, K, N)
        x = activations(t)
        arrays = {"w": w, "x": x, "type": np.int32(t), "K": np.int32(K), "N": np.int32(N)}
        for M in (1, 4):
            xm = x[:M]
            d, s, lo, hi, qs = orc.quantize_act(xm)
            arrays.update({f"d_m{M}": d, f"sum_m{M}": s, f"sum_lo_m{M}": lo, f"sum_hi_m{M}": hi,
                           f"qs_m{M}": qs,
                           f"bsum_m{M}": orc.block_sums(t, w, qs, K, N),
                           f"y_int_m{M}": orc.gemm_int(t, xm, w, N, nthreads=1),
                           f"y_scalar_m{M}": orc.gemm_scalar(t, xm, w, N, nthreads=1)})
        deq = orc.dequantize(t, w, N * K)
        if have_ref:
            import ctypes as C
            ref = np.zeros(N * K, np.float32)
            nblocks = w.nbytes // orc.lib().or_bytes_per_block(t)
            if orc.ref().ref_dequant(t, w, nblocks, ref) != 0:
                raise SystemExit(f"reference dequantizer rejected {name}")
            if not np.array_equal(ref.view(np.uint32), deq.view(np.uint32)):
                raise SystemExit(f"{name}: oracle dequantize differs from the reference's")
        else:
            print("oracle/_ref not built: dequantize not cross-checked", file=sys.stderr)
        arrays["deq"] = deq
        path = os.path.join(OUT, f"{name}_K{K}_N{N}.npz")
        np.savez_compressed(path, **arrays)
        print(f"wrote {os.path.relpath(path, ROOT)} ({os.path.getsize(path)} B)")


if __name__ == "__main__":
    main()
