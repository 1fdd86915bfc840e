// ref_glue.cpp - C-callable wrappers around the reference's own header-only
// GGUF layout oracle, compiled in place from /root/reference (see Makefile).
//
// TEST INFRASTRUCTURE ONLY. The wrapped sources are the reference's:
//   src/fp16.h:9-85          fp16/bf16 conversions
//   src/kernels.h:82-90      get_scale_min_k4
//   tests/quant_ref.h:47-110 independent GGUF dequantizers (Q4_0, Q8_0, Q4_K, Q6_K)
//   tests/test_util.h:49-61  XorShift32
// Nothing here re-implements them; this file only exposes them to ctypes so
// the oracle's restatement can be checked against the reference itself.
#include <cstdint>
#include <cstring>

#include "fp16.h"
#include "kernels.h"
#include "quant_ref.h"
#include "test_util.h"

extern "C" {

float ref_fp16_to_fp32(uint16_t h) { return Laplace::fp16_to_fp32(h); }
uint16_t ref_fp32_to_fp16(float f) { return Laplace::fp32_to_fp16(f); }
float ref_bf16_to_fp32(uint16_t h) { return Laplace::bf16_to_fp32(h); }
uint16_t ref_fp32_to_bf16(float f) { return Laplace::fp32_to_bf16(f); }

void ref_get_scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
    Laplace::kernels::get_scale_min_k4(j, q, d, m);
}

// Dequantize n_blocks consecutive blocks of `type` (GGMLType value).
int ref_dequant(int type, const uint8_t* w, long n_blocks, float* out) {
    for (long i = 0; i < n_blocks; i++) {
        switch (type) {
            case 2: {
                quant_ref::block_q4_0 b; std::memcpy(&b, w + i * 18, 18);
                quant_ref::dequant_q4_0(&b, out + i * 32); break;
            }
            case 8: {
                quant_ref::block_q8_0 b; std::memcpy(&b, w + i * 34, 34);
                quant_ref::dequant_q8_0(&b, out + i * 32); break;
            }
            case 12: {
                quant_ref::block_q4_K b; std::memcpy(&b, w + i * 144, 144);
                quant_ref::dequant_q4_K(&b, out + i * 256); break;
            }
            case 14: {
                quant_ref::block_q6_K b; std::memcpy(&b, w + i * 210, 210);
                quant_ref::dequant_q6_K(&b, out + i * 256); break;
            }
            default: return -1;
        }
    }
    return 0;
}

void ref_xorshift_u32(uint32_t seed, long n, uint32_t* out) {
    XorShift32 r(seed);
    for (long i = 0; i < n; i++) out[i] = r.next();
}

void ref_xorshift_float(uint32_t seed, long n, float* out) {
    XorShift32 r(seed);
    for (long i = 0; i < n; i++) out[i] = r.next_float();
}

}  // extern "C"
