// ref_glue.cpp - C-callable wrappers around the reference's own header-only
// GGUF layout oracle, compiled in place from /root/reference (see Makefile).
//
// TEST INFRASTRUCTURE ONLY. The wrapped sources are the reference's:
//   src/fp16.h:9-85          fp16/bf16 conversions
//   src/kernels.h:82-90      get_scale_min_k4
//   tests/quant_ref.h:47-110 independent GGUF dequantizers (Q4_0, Q8_0, Q4_K, Q6_K)
//   tests/test_util.h:49-61  XorShift32
//   tests/gguf_writer.h      the GGUF v3 test-file writer (Writer, TensorDecl)
// Nothing here re-implements them; this file only exposes them to ctypes so
// the oracle's restatement can be checked against the reference itself.
#include <cstdint>
#include <cstring>

#include "fp16.h"
#include "gguf_writer.h"
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

// The reference's GGUF writer behind a handle: metadata and tensors are
// added one call at a time, then written (optionally truncated) to a path.
void* ref_gguf_new(void) { return new gguf_writer::Writer(); }
void ref_gguf_free(void* h) { delete static_cast<gguf_writer::Writer*>(h); }
void ref_gguf_kv_u32(void* h, const char* k, uint32_t v) { static_cast<gguf_writer::Writer*>(h)->kv_u32(k, v); }
void ref_gguf_kv_i32(void* h, const char* k, int32_t v) { static_cast<gguf_writer::Writer*>(h)->kv_i32(k, v); }
void ref_gguf_kv_f32(void* h, const char* k, float v) { static_cast<gguf_writer::Writer*>(h)->kv_f32(k, v); }
void ref_gguf_kv_bool(void* h, const char* k, int v) { static_cast<gguf_writer::Writer*>(h)->kv_bool(k, v != 0); }
void ref_gguf_kv_str(void* h, const char* k, const char* v) { static_cast<gguf_writer::Writer*>(h)->kv_str(k, v); }
void ref_gguf_kv_arr_str(void* h, const char* k, const char* const* v, long n) {
    std::vector<std::string> a(v, v + n);
    static_cast<gguf_writer::Writer*>(h)->kv_arr_str(k, a);
}
void ref_gguf_kv_arr_u8(void* h, const char* k, const uint8_t* v, long n) {
    static_cast<gguf_writer::Writer*>(h)->kv_arr_u8(k, std::vector<uint8_t>(v, v + n));
}
void ref_gguf_kv_arr_i16(void* h, const char* k, const int16_t* v, long n) {
    static_cast<gguf_writer::Writer*>(h)->kv_arr_i16(k, std::vector<int16_t>(v, v + n));
}
void ref_gguf_kv_arr_bool(void* h, const char* k, const uint8_t* v, long n) {
    std::vector<bool> a(n);
    for (long i = 0; i < n; i++) a[i] = v[i] != 0;
    static_cast<gguf_writer::Writer*>(h)->kv_arr_bool(k, a);
}
void ref_gguf_kv_arr_i32(void* h, const char* k, const int32_t* v, long n) {
    static_cast<gguf_writer::Writer*>(h)->kv_arr_i32(k, std::vector<int32_t>(v, v + n));
}
void ref_gguf_add_tensor(void* h, const char* name, const uint64_t* dims, int ndims, uint32_t type,
                         const uint8_t* data, long nbytes) {
    gguf_writer::TensorDecl t;
    t.name = name;
    t.dims.assign(dims, dims + ndims);
    t.type = type;
    t.data.assign(data, data + nbytes);
    static_cast<gguf_writer::Writer*>(h)->add_tensor(std::move(t));
}
int ref_gguf_write(void* h, const char* path, long truncate_bytes) {
    return static_cast<gguf_writer::Writer*>(h)->write_file(path, (size_t)truncate_bytes) ? 0 : 1;
}

}  // extern "C"
