// kernels_hip.h - the three hooks the reference's matmul front-end calls
// besides the kernels.h getters, for the MI355X back-end (liblaplace_hip.so).
//
// Each is one added line in src/matmul.cpp:
//   matmul_register_weights (src/matmul.cpp:446-448): hip_register_weights(base, size);
//   matmul_gemm_batch       (src/matmul.cpp:450-454): if (hip_gemm_batch(specs, n)) return true;
//   dequantize              (src/matmul.cpp:504):     if (hip_dequantize(w, dst, n)) return;
// and every path keeps its existing CPU code when the hook returns false.
#pragma once

#include <cstddef>

#include "matmul.h"   // MatmulBatchSpec, Tensor (reference src/)

namespace Laplace {
namespace kernels {

// Copies the mmap'd GGUF region to the GPU once; later weight pointers inside
// it resolve to the device copy. No-op without a usable device.
void hip_register_weights(const void* base, size_t size);

// The whole batch of M=1 matmuls on the GPU (specs sharing x in one launch).
// false: LAPLACE_NOSIMD set, no device, or a type the back-end does not take;
// nothing was written and the caller runs its per-spec loop.
bool hip_gemm_batch(const MatmulBatchSpec* specs, int n);

// Dequantize on the GPU; false leaves dst to the caller's CPU loop.
bool hip_dequantize(const Tensor& w, float* dst, int n);

}  // namespace kernels
}  // namespace Laplace
