"""Build the gfx950 shared library ``laplace_amd/liblaplace_hip.so`` in-tree.

Every source under ``laplace_amd/csrc`` is compiled with hipcc for gfx950
only and linked into one library that exports the C ABI of
``include/laplace_hip.h``. Run ``python -m laplace_amd.build`` (or
``__graft_entry__.build()``); it always recompiles.

Flags: ``-O3``; no fast-math (the activation quantizer must be bit-exact:
IEEE division and round-half-even); packed-fp32 instructions disabled
(``-target-feature -packed-fp32-ops``).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
ROOT = os.path.dirname(PKG)
LIB = os.path.join(PKG, "liblaplace_hip.so")
OBJ = os.path.join(ROOT, "_build", "obj")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

SOURCES = ["lp_gemv.hip", "lp_gemm.hip", "lp_gemm_fr.hip", "lp_gemm_i8.hip", "lp_dequant.hip", "lp_moe_ffn.hip", "lp_rq.hip", "lp_q6rq.hip", "lp_api.cpp"]

CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    f"-I{os.path.join(ROOT, 'include')}",
]


# Per-source additions. lp_rq.hip: MFMA results in VGPRs (its int8 block sums
# feed VALU at once; the AGPR form costs a v_accvgpr_read per value).
SRC_FLAGS = {"lp_gemm_fr.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"], "lp_gemm_i8.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"], "lp_rq.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"], "lp_q6rq.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _compile(src: str) -> str:
    path = os.path.join(CSRC, src)
    obj = os.path.join(OBJ, src.rsplit(".", 1)[0] + ".o")
    cmd = [HIPCC, *CFLAGS, *SRC_FLAGS.get(src, []), "-x", "hip", "-c", path, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(OBJ, exist_ok=True)
    srcs = list(SOURCES)
    missing = [s for s in srcs if not os.path.exists(os.path.join(CSRC, s))]
    if missing:
        raise FileNotFoundError(f"missing sources: {missing}")
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
