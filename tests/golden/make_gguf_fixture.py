"""Writes tests/golden/ref_writer_weights.gguf with the reference's own GGUF
test writer (tests/gguf_writer.h, compiled unmodified into oracle/_ref by
oracle/Makefile). The file is data: three weight tensors (Q4_K, Q6_K, Q8_0,
K 1024 x N 32, seeded random blocks with small fp16 scales) and a little
metadata. The GPU test test_gguf.py::test_registered_file_matmul reads it
with laplace_amd.gguf, registers its data section and runs lp_gemm on the
tensors in place; the reference itself never travels to the GPU box.

Run from the repository root:  python tests/golden/make_gguf_fixture.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as orc  # noqa: E402

Q8_0, Q4_K, Q6_K = 8, 12, 14
K, N = 1024, 32
OUT = os.path.join(HERE, "ref_writer_weights.gguf")


def blocks(t, seed):
    rng = np.random.default_rng(seed)
    rb = orc.row_bytes(t, K)
    w = rng.integers(0, 256, rb * N, dtype=np.uint8)
    bpb = {Q8_0: 34, Q4_K: 144, Q6_K: 210}[t]
    b = w.reshape(-1, bpb)
    f16 = lambda: (np.abs(rng.standard_normal(b.shape[0])) * 0.01).astype(np.float16).view(np.uint8).reshape(-1, 2)
    if t == Q8_0:
        b[:, 0:2] = f16()
    elif t == Q4_K:
        b[:, 0:2] = f16()
        b[:, 2:4] = f16()
    else:
        b[:, 208:210] = f16()
    return w


def main():
    orc.build()
    w = orc.RefGGUFWriter()
    w.kv("str", "general.architecture", "laplace-test")
    w.kv("u32", "test.k", K)
    for name, t, seed in (("w.q4k", Q4_K, 1), ("w.q6k", Q6_K, 2), ("w.q80", Q8_0, 3)):
        w.tensor(name, (K, N), t, blocks(t, seed))
    w.write(OUT)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
