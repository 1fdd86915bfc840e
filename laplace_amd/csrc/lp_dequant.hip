// lp_dequant.hip - GGUF blocks to fp32 (src/matmul.cpp:504-675) for gfx950.
//
// One thread per output element; the block header is re-read by the 32/256
// threads of a block and served from cache. Every formula keeps the
// reference's operation order with contraction disabled, so each output is
// the same fp32 value the reference's scalar loop produces.
#include <hip/hip_runtime.h>

#include "lp_internal.h"

namespace lp {

namespace {

__device__ __forceinline__ uint32_t rd16(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

__device__ __forceinline__ float h2f(uint32_t h) { return fp16_bits_to_f32(h); }

__device__ __forceinline__ void scale_min(int j, const uint8_t* q, int& d, int& m) {
    // get_scale_min_k4 (src/kernels.h:82-90)
    if (j < 4) {
        d = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// 6-bit Q3_K scale j of the 12 packed bytes (src/matmul.cpp:236-282 unpack).
__device__ __forceinline__ int q3k_scale(const uint8_t* s, int j) {
    const int lo = (j < 8) ? (s[j] & 0xF) : (s[j - 8] >> 4);
    const int hi = (s[8 + (j & 3)] >> (2 * (j >> 2))) & 3;
    return lo | (hi << 4);
}

#pragma clang fp contract(off)
__device__ float dequant_one(uint32_t type, const uint8_t* __restrict__ w, long i) {
    switch (type) {
        case T_F32: return reinterpret_cast<const float*>(w)[i];
        case T_F16: return h2f(rd16(w + 2 * i));
        case T_BF16: return __uint_as_float(rd16(w + 2 * i) << 16);
        case T_Q4_0: {
            const uint8_t* b = w + (i >> 5) * 18;
            const int l = (int)(i & 31);
            const int q = l < 16 ? (b[2 + l] & 0xF) : (b[2 + l - 16] >> 4);
            return h2f(rd16(b)) * (float)(q - 8);
        }
        case T_Q5_0: {
            const uint8_t* b = w + (i >> 5) * 22;
            const int l = (int)(i & 31);
            const uint32_t qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) | ((uint32_t)b[5] << 24);
            const int q = l < 16 ? ((b[6 + l] & 0xF) | (int)(((qh >> l) & 1u) << 4))
                                 : ((b[6 + l - 16] >> 4) | (int)(((qh >> l) & 1u) << 4));
            return h2f(rd16(b)) * (float)(q - 16);
        }
        case T_Q8_0: {
            const uint8_t* b = w + (i >> 5) * 34;
            return h2f(rd16(b)) * (float)(int8_t)b[2 + (i & 31)];
        }
        case T_Q2_K: {
            const uint8_t* b = w + (i >> 8) * 84;
            const int e = (int)(i & 255), j = e >> 4, l = e & 15;
            const float d = h2f(rd16(b + 80)), dmin = h2f(rd16(b + 82));
            const float sc = (float)(b[j] & 0xF), mn = (float)(b[j] >> 4);
            const int half = j >> 3, jj = j & 7, group = jj >> 1, lo = jj & 1;
            const int q = (b[16 + half * 32 + lo * 16 + l] >> (group * 2)) & 3;
            const float a = d * sc;
            const float c = dmin * mn;
            return a * (float)q - c;
        }
        case T_Q3_K: {
            const uint8_t* b = w + (i >> 8) * 110;
            const int e = (int)(i & 255), j = e >> 4;
            const float d = h2f(rd16(b + 108));
            const float sc = (float)q3k_scale(b + 96, j) - 32;
            const int g = e >> 5, li = e & 31;
            const int low2 = (b[32 + (g >> 2) * 32 + li] >> ((g & 3) * 2)) & 3;
            const int hbit = (b[li] >> g) & 1;
            const float a = d * sc;
            return a * (float)(low2 - 4 + 4 * hbit);
        }
        case T_Q4_K: {
            const uint8_t* b = w + (i >> 8) * 144;
            const int e = (int)(i & 255), jb = e >> 6, hi = (e >> 5) & 1, l = e & 31;
            int sc, m;
            scale_min(2 * jb + hi, b + 4, sc, m);
            const float d1 = h2f(rd16(b)) * (float)sc, m1 = h2f(rd16(b + 2)) * (float)m;
            const uint8_t q = b[16 + 32 * jb + l];
            return d1 * (float)(hi ? (q >> 4) : (q & 0xF)) - m1;
        }
        case T_Q5_K: {
            const uint8_t* b = w + (i >> 8) * 176;
            const int e = (int)(i & 255), jb = e >> 6, hi = (e >> 5) & 1, l = e & 31;
            int sc, m;
            scale_min(2 * jb + hi, b + 4, sc, m);
            const float d1 = h2f(rd16(b)) * (float)sc, m1 = h2f(rd16(b + 2)) * (float)m;
            const uint8_t q = b[48 + 32 * jb + l];
            const int v = (hi ? (q >> 4) : (q & 0xF)) + 16 * ((b[16 + l] >> (2 * jb + hi)) & 1);
            return d1 * (float)v - m1;
        }
        case T_Q6_K: {
            const uint8_t* b = w + (i >> 8) * 210;
            const int e = (int)(i & 255), h = e >> 7, r = e & 127, g = r >> 5, l = r & 31;
            const uint8_t* ql = b + 64 * h;
            const uint8_t* qh = b + 128 + 32 * h;
            const int8_t* sc = reinterpret_cast<const int8_t*>(b + 192 + 8 * h);
            const int nib = (g & 1) ? ((g & 2) ? (ql[l + 32] >> 4) : (ql[l + 32] & 0xF))
                                    : ((g & 2) ? (ql[l] >> 4) : (ql[l] & 0xF));
            const int q = (nib | (((qh[l] >> (2 * g)) & 3) << 4)) - 32;
            const float a = h2f(rd16(b + 208)) * (float)sc[(l >> 4) + 2 * g];
            return a * (float)q;
        }
        default: return 0.0f;
    }
}
#pragma clang fp contract(on)

__global__ void __launch_bounds__(256)
dequant_kernel(uint32_t type, const uint8_t* __restrict__ w, float* __restrict__ dst, long n) {
    const long stride = (long)gridDim.x * blockDim.x;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        dst[i] = dequant_one(type, w, i);
}

}  // namespace

int dequant_block_elems(uint32_t type) {
    switch (type) {
        case T_F32: case T_F16: case T_BF16: return 1;
        case T_Q4_0: case T_Q5_0: case T_Q8_0: return 32;
        case T_Q2_K: case T_Q3_K: case T_Q4_K: case T_Q5_K: case T_Q6_K: return 256;
        default: return 0;
    }
}

size_t dequant_src_bytes(uint32_t type, long n) {
    const int epb = dequant_block_elems(type);
    if (epb == 0) return 0;
    long bpb;
    switch (type) {
        case T_F32: bpb = 4; break;
        case T_F16: case T_BF16: bpb = 2; break;
        case T_Q4_0: bpb = 18; break;
        case T_Q5_0: bpb = 22; break;
        case T_Q8_0: bpb = 34; break;
        case T_Q2_K: bpb = 84; break;
        case T_Q3_K: bpb = 110; break;
        case T_Q4_K: bpb = 144; break;
        case T_Q5_K: bpb = 176; break;
        default: bpb = 210; break;
    }
    return (size_t)(n / epb) * (size_t)bpb;
}

hipError_t launch_dequant(uint32_t type, const uint8_t* w, float* dst, long n, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    long grid = (n + 255) / 256;
    if (grid > 65536) grid = 65536;
    hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)grid), dim3(256), 0, st, type, w, dst, n);
    return hipGetLastError();
}

}  // namespace lp
