"""The reference-side binding (integration/kernels_hip.cpp) as a compiled
artefact: compiled against the reference's own headers (src/kernels.h,
src/matmul.h, src/tensor.h, in place under /root/reference) and
include/laplace_hip.h, then linked with liblaplace_hip.so into a program
that binds the getters the way src/matmul.cpp does. Without a usable GPU
(this container) the getters must return nullptr and the hooks false, which
is the reference's fall-back contract (src/kernels.h:114-119,
src/matmul.cpp:426-432). Skipped where the reference tree is absent."""
import os
import subprocess
import textwrap

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = os.environ.get("LAPLACE_REF", "/root/reference")
LIB = os.path.join(ROOT, "laplace_amd", "liblaplace_hip.so")

needs_ref = pytest.mark.skipif(not os.path.isfile(os.path.join(REF, "src", "kernels.h")),
                               reason="reference headers not present")

MAIN = textwrap.dedent("""
    #include <cstdio>
    #include "kernels.h"
    #include "kernels_hip.h"
    using namespace Laplace;
    int main() {
        kernels::gemm_fn g = kernels::get_simd_gemm();
        kernels::moe_gemv_fn m = kernels::get_simd_moe_gemv();
        kernels::moe_gemv_multi_fn mm = kernels::get_simd_moe_gemv_multi();
        Tensor t;
        t.type = GGMLType::Q4_K;
        float x[256] = {0}, y[1] = {0};
        MatmulBatchSpec s = {x, &t, y, 256, 1};
        bool b = kernels::hip_gemm_batch(&s, 1);
        bool d = kernels::hip_dequantize(t, y, 0);
        kernels::hip_register_weights(x, sizeof x);
        std::printf("%d %d %d %d %d\\n", g != nullptr, m != nullptr, mm != nullptr, (int)b, (int)d);
        return 0;
    }
""")


def _cxx(args, cwd):
    r = subprocess.run(["g++", "-std=c++20", "-Wall", "-Werror"] + args, cwd=cwd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return r


@needs_ref
def test_binding_compiles_against_reference_headers(tmp_path):
    inc = ["-I" + os.path.join(REF, "src"), "-I" + os.path.join(ROOT, "include"),
           "-I" + os.path.join(ROOT, "integration")]
    _cxx(inc + ["-fsyntax-only", os.path.join(ROOT, "integration", "kernels_hip.cpp")], tmp_path)


@needs_ref
@pytest.mark.skipif(not os.path.isfile(LIB), reason="liblaplace_hip.so not built")
def test_binding_links_and_falls_back_without_gpu(tmp_path):
    inc = ["-I" + os.path.join(REF, "src"), "-I" + os.path.join(ROOT, "include"),
           "-I" + os.path.join(ROOT, "integration")]
    (tmp_path / "main.cpp").write_text(MAIN)
    libdir = os.path.dirname(LIB)
    _cxx(inc + ["-o", "bind", "main.cpp", os.path.join(ROOT, "integration", "kernels_hip.cpp"),
                "-L" + libdir, "-llaplace_hip", "-Wl,-rpath," + libdir], tmp_path)
    env = dict(os.environ, HIP_VISIBLE_DEVICES="", ROCR_VISIBLE_DEVICES="")
    r = subprocess.run([str(tmp_path / "bind")], capture_output=True, text=True, env=env, timeout=120)
    assert r.returncode == 0, r.stderr
    assert r.stdout.split() == ["0", "0", "0", "0", "0"], r.stdout
