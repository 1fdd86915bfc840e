// kernels_hip.cpp - MI355X back-end for the reference's kernels.h ABI.
//
// Added to the reference tree as src/kernels_hip.cpp and compiled on x86-64
// in place of the non-AArch64 stubs of src/matmul_simd.cpp:627-637: the
// getters of src/kernels.h:114-119 return the entry points of
// liblaplace_hip.so (include/laplace_hip.h), whose signatures are the
// back-end ABI's (src/kernels.h:94-112) with GGMLType passed as its uint32_t
// value. Nothing above kernels.h changes; LAPLACE_NOSIMD=1 still forces the
// scalar path (src/matmul.cpp:47-54), and a false return still falls back
// to it (src/matmul.cpp:426-432).
//
// tests/test_integration.py compiles this file against the reference's own
// headers and links it with the library.
#include "kernels_hip.h"

#include <cstdint>
#include <cstdlib>
#include <vector>

#include "kernels.h"
#include "laplace_hip.h"

namespace Laplace {
namespace kernels {

static_assert(sizeof(GGMLType) == sizeof(uint32_t), "GGMLType travels as its uint32_t value");

static bool hip_gemm(const float* x, const uint8_t* w, GGMLType t, float* y, int M, int K, int N) {
    return lp_gemm(x, w, static_cast<uint32_t>(t), y, M, K, N);
}
static bool hip_moe(const float* x, const uint8_t* w, GGMLType t, const int* idx, int n, float* y,
                    int K, int N) {
    return lp_moe_gemv(x, w, static_cast<uint32_t>(t), idx, n, y, K, N);
}
static bool hip_moe_multi(const float* x, const uint8_t* w, GGMLType t, const int* idx, int n,
                          float* y, int K, int N) {
    return lp_moe_gemv_multi(x, w, static_cast<uint32_t>(t), idx, n, y, K, N);
}

// nullptr when no gfx950 device is usable: the front-end keeps its scalar path.
gemm_fn get_simd_gemm() { return lp_get_gemm() ? hip_gemm : nullptr; }
moe_gemv_fn get_simd_moe_gemv() { return lp_get_moe_gemv() ? hip_moe : nullptr; }
moe_gemv_multi_fn get_simd_moe_gemv_multi() { return lp_get_moe_gemv_multi() ? hip_moe_multi : nullptr; }

static bool hip_usable() { return !std::getenv("LAPLACE_NOSIMD") && lp_get_gemm() != nullptr; }

void hip_register_weights(const void* base, size_t size) {
    if (hip_usable()) lp_register_weights(base, size);
}

bool hip_gemm_batch(const MatmulBatchSpec* specs, int n) {
    if (n <= 0 || !hip_usable()) return false;
    std::vector<lp_batch_spec> b(static_cast<size_t>(n));
    for (int i = 0; i < n; i++)
        b[i] = {specs[i].x, specs[i].w->data, static_cast<uint32_t>(specs[i].w->type), specs[i].y, specs[i].K,
                specs[i].N};
    return lp_gemm_batch(b.data(), n);
}

bool hip_dequantize(const Tensor& w, float* dst, int n) {
    if (!hip_usable()) return false;
    return lp_dequantize(w.data, static_cast<uint32_t>(w.type), dst, n) == 0;
}

}  // namespace kernels
}  // namespace Laplace
