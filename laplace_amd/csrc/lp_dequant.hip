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
__device__ __forceinline__ float dequant_one(uint32_t type, const uint8_t* __restrict__ w, long i) {
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
// Q4_K, eight consecutive outputs from i0 (8 | i0): one 32-element block,
// so one scale pair and eight consecutive code bytes (an 8-byte load; w
// 8-byte aligned), the arithmetic of dequant_one.
__device__ __forceinline__ void dequant8_q4k(const uint8_t* __restrict__ w, long i0, float (&v)[8]) {
    const uint8_t* b = w + (i0 >> 8) * 144;
    const int e = (int)(i0 & 255), jb = e >> 6, hi = (e >> 5) & 1, l0 = e & 31;
    int sc, m;
    scale_min(2 * jb + hi, b + 4, sc, m);
    const float d1 = h2f(rd16(b)) * (float)sc, m1 = h2f(rd16(b + 2)) * (float)m;
    const uint2 q8 = *reinterpret_cast<const uint2*>(b + 16 + 32 * jb + l0);
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t q = ((k < 4 ? q8.x : q8.y) >> (8 * (k & 3))) & 0xffu;
        v[k] = d1 * (float)(hi ? (q >> 4) : (q & 0xF)) - m1;
    }
}
// Eight bytes at a 2-byte aligned address (four 16-bit loads).
__device__ __forceinline__ uint2 ld8_h(const uint8_t* p) {
    const uint16_t* h = reinterpret_cast<const uint16_t*>(p);
    return make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16));
}
__device__ __forceinline__ uint32_t byte_of(uint2 u, int k) { return ((k < 4 ? u.x : u.y) >> (8 * (k & 3))) & 0xffu; }

// Eight consecutive outputs from i0 (8 | i0) of the types whose eight
// elements share their block header and sit in consecutive bytes, with
// dequant_one's arithmetic; false: not one of them (the caller decodes
// element by element). Alignment of w: 16 bytes for F32/F16/BF16, 8 for
// Q4_K/Q5_K, 2 for Q4_0/Q5_0/Q8_0/Q6_K (dequant_wide_ok).
template <uint32_t T>
__device__ __forceinline__ bool dequant8_wide(const uint8_t* __restrict__ w, long i0, float (&v)[8]) {
    if constexpr (T == T_F32) {
        const float4 a = reinterpret_cast<const float4*>(w)[i0 / 4], c = reinterpret_cast<const float4*>(w)[i0 / 4 + 1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = c.x; v[5] = c.y; v[6] = c.z; v[7] = c.w;
        return true;
    } else if constexpr (T == T_F16 || T == T_BF16) {
        const u32x4 q = reinterpret_cast<const u32x4*>(w)[i0 / 8];
        const uint32_t u[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            if constexpr (T == T_F16) {
                v[2 * k] = h2f(u[k] & 0xffffu);
                v[2 * k + 1] = h2f(u[k] >> 16);
            } else {
                v[2 * k] = __uint_as_float((u[k] & 0xffffu) << 16);
                v[2 * k + 1] = __uint_as_float(u[k] & 0xffff0000u);
            }
        }
        return true;
    } else if constexpr (T == T_Q4_0) {
        const uint8_t* b = w + (i0 >> 5) * 18;
        const int l0 = (int)(i0 & 31);
        const float d = h2f(rd16(b));
        const uint2 q8 = ld8_h(b + 2 + (l0 & 15));
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t q = byte_of(q8, k);
            v[k] = d * (float)((int)(l0 < 16 ? (q & 0xF) : (q >> 4)) - 8);
        }
        return true;
    } else if constexpr (T == T_Q8_0) {
        const uint8_t* b = w + (i0 >> 5) * 34;
        const float d = h2f(rd16(b));
        const uint2 q8 = ld8_h(b + 2 + (i0 & 31));
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = d * (float)(int8_t)byte_of(q8, k);
        return true;
    } else if constexpr (T == T_Q4_K) {
        dequant8_q4k(w, i0, v);
        return true;
    } else if constexpr (T == T_Q5_0) {
        const uint8_t* b = w + (i0 >> 5) * 22;
        const int l0 = (int)(i0 & 31);
        const uint16_t* hp = reinterpret_cast<const uint16_t*>(b + 2);
        const uint32_t qh = (uint32_t)hp[0] | ((uint32_t)hp[1] << 16);
        const float d = h2f(rd16(b));
        const uint2 q8 = ld8_h(b + 6 + (l0 & 15));
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t q = byte_of(q8, k);
            const int l = l0 + k;
            const int v5 = (int)(l0 < 16 ? (q & 0xF) : (q >> 4)) | (int)(((qh >> l) & 1u) << 4);
            v[k] = d * (float)(v5 - 16);
        }
        return true;
    } else if constexpr (T == T_Q5_K) {
        const uint8_t* b = w + (i0 >> 8) * 176;
        const int e = (int)(i0 & 255), jb = e >> 6, hi = (e >> 5) & 1, l0 = e & 31;
        int sc, m;
        scale_min(2 * jb + hi, b + 4, sc, m);
        const float d1 = h2f(rd16(b)) * (float)sc, m1 = h2f(rd16(b + 2)) * (float)m;
        const uint2 q8 = *reinterpret_cast<const uint2*>(b + 48 + 32 * jb + l0);
        const uint2 h8 = *reinterpret_cast<const uint2*>(b + 16 + l0);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t q = byte_of(q8, k);
            const int v5 = (int)(hi ? (q >> 4) : (q & 0xF)) + 16 * (int)((byte_of(h8, k) >> (2 * jb + hi)) & 1u);
            v[k] = d1 * (float)v5 - m1;
        }
        return true;
    } else if constexpr (T == T_Q6_K) {
        const uint8_t* b = w + (i0 >> 8) * 210;
        const int e = (int)(i0 & 255), h = e >> 7, r = e & 127, g = r >> 5, l0 = r & 31;
        const uint2 ql = ld8_h(b + 64 * h + l0 + ((g & 1) ? 32 : 0));
        const uint2 qh = ld8_h(b + 128 + 32 * h + l0);
        const int8_t* sc = reinterpret_cast<const int8_t*>(b + 192 + 8 * h);
        const float a = h2f(rd16(b + 208)) * (float)sc[(l0 >> 4) + 2 * g];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t lb = byte_of(ql, k);
            const int nib = (g & 2) ? (int)(lb >> 4) : (int)(lb & 0xF);
            const int q = (nib | (int)(((byte_of(qh, k) >> (2 * g)) & 3u) << 4)) - 32;
            v[k] = a * (float)q;
        }
        return true;
    } else {
        return false;
    }
}
#pragma clang fp contract(on)

__global__ void __launch_bounds__(256)
dequant_kernel(uint32_t type, const uint8_t* __restrict__ w, float* __restrict__ dst, long n) {
    const long stride = (long)gridDim.x * blockDim.x;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        dst[i] = dequant_one(type, w, i);
}

// w's alignment for dequant8_wide
static bool dequant_wide_ok(uint32_t type, const uint8_t* w) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(w);
    switch (type) {
        case T_F32: case T_F16: case T_BF16: return a % 16 == 0;
        case T_Q4_K: case T_Q5_K: return a % 8 == 0;
        case T_Q4_0: case T_Q5_0: case T_Q8_0: case T_Q6_K: return a % 2 == 0;
        default: return false;
    }
}

// Eight consecutive outputs per thread (two 16-byte stores; the type is a
// template constant, so the eight inlined decodes share their block-header
// loads). n % 8 == 0 and dst 16-byte aligned.
template <uint32_t T, bool WIDE>
__global__ void __launch_bounds__(256)
dequant8_kernel(const uint8_t* __restrict__ w, float* __restrict__ dst, long n8) {
    const long stride = (long)gridDim.x * blockDim.x;
    for (long j = (long)blockIdx.x * blockDim.x + threadIdx.x; j < n8; j += stride) {
        float v[8];
        if (!(WIDE && dequant8_wide<T>(w, 8 * j, v))) {
#pragma unroll
            for (int k = 0; k < 8; k++) v[k] = dequant_one(T, w, 8 * j + k);
        }
        float4* o = reinterpret_cast<float4*>(dst + 8 * j);
        o[0] = make_float4(v[0], v[1], v[2], v[3]);
        o[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
}

// ---------------------------------------------------------------------------
// GEMV with fp32 activations for the types the reference's int8 back-end does
// not take (F32, F16, BF16, Q5_0, Q2_K, Q3_K, Q5_K): the reference then runs
// gemm_scalar<dot_row_*> (src/matmul.cpp:320-353, dots at :63-314), fp32 x
// against the decoded weights. One wave per weight row at a time, lane l
// taking the 32-element chunks l, l+64, ...: it decodes the chunk once
// (dequant_one, the dequantize arithmetic, with the block header loads shared
// by the 32 inlined calls) and dots it with the MR activation rows; a
// butterfly sum over the wave. The fp32 sums are reassociated against the
// reference's sequential loop, so results agree to fp32 rounding.
// One 32-element chunk c of a row: codes q[32] and, per 16-element half h,
// (a[h], b[h]) with chunk value = sum_h a[h] * sum(x * q) + b[h] * sum(x).
// Generic form: q = the dequantized values, a = 1, b = 0. The K-quants load
// their chunk's code bytes as whole dwords and keep the reference's integer
// codes (Q2_K: 2-bit q with d*sc and -dmin*m per 16; Q3_K: signed 3-bit a
// with d*(sc-32) per 16; Q5_K: 5-bit v with d*sc and -dmin*m per 32).
template <uint32_t T>
__device__ __forceinline__ void chunk_decode(const uint8_t* __restrict__ wr, int c, float (&q)[32], float (&a)[2],
                                             float (&b)[2]) {
    if constexpr (T == T_Q5_K) {
        const uint8_t* blk = wr + (size_t)(c >> 3) * 176;
        const int j = c & 7, jb = j >> 1, hi = j & 1;
        const uint32_t* qs = reinterpret_cast<const uint32_t*>(blk + 48 + 32 * jb);
        const uint32_t* qh = reinterpret_cast<const uint32_t*>(blk + 16);
        const int bit = 2 * jb + hi;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t v = ((qs[k] >> (4 * hi)) & 0x0f0f0f0fu) | (((qh[k] >> bit) & 0x01010101u) << 4);
            q[4 * k] = (float)(v & 0xff);
            q[4 * k + 1] = (float)((v >> 8) & 0xff);
            q[4 * k + 2] = (float)((v >> 16) & 0xff);
            q[4 * k + 3] = (float)(v >> 24);
        }
        int sc, m;
        scale_min(j, blk + 4, sc, m);
        const float d1 = h2f(rd16(blk)) * (float)sc, m1 = h2f(rd16(blk + 2)) * (float)m;
        a[0] = a[1] = d1;
        b[0] = b[1] = -m1;
    } else if constexpr (T == T_Q2_K) {
        const uint8_t* blk = wr + (size_t)(c >> 3) * 84;
        const int j = c & 7;
        const uint32_t* qs = reinterpret_cast<const uint32_t*>(blk + 16 + 32 * (j >> 2));
        const int sh = 2 * (j & 3);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t v = (qs[k] >> sh) & 0x03030303u;
            q[4 * k] = (float)(v & 0xff);
            q[4 * k + 1] = (float)((v >> 8) & 0xff);
            q[4 * k + 2] = (float)((v >> 16) & 0xff);
            q[4 * k + 3] = (float)(v >> 24);
        }
        const float d = h2f(rd16(blk + 80)), dmin = h2f(rd16(blk + 82));
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint8_t s = blk[2 * j + h];
            a[h] = d * (float)(s & 0xF);
            b[h] = -(dmin * (float)(s >> 4));
        }
    } else if constexpr (T == T_Q3_K) {
        // The 110-byte block is 2-byte aligned: its 32 hmask bytes and the 32
        // code bytes of chunk g are read as dwords from the aligned-down
        // address and funnel-shifted. Per byte u = low2 | hbit << 2 (0..7),
        // the reference's code being u - 4: chunk = a * sum(x*u) - 4a * sum(x).
        const uint8_t* blk = wr + (size_t)(c >> 3) * 110;
        const int g = c & 7;
        const uintptr_t ab = reinterpret_cast<uintptr_t>(blk);
        const uint32_t sh = (uint32_t)(ab & 3);
        const uint32_t* hp = reinterpret_cast<const uint32_t*>(ab - sh);
        const uint32_t* qp = reinterpret_cast<const uint32_t*>(ab - sh + 32 + 32 * (g >> 2));
        uint32_t hw_[9], qw_[9];
#pragma unroll
        for (int k = 0; k < 9; k++) {
            hw_[k] = hp[k];
            qw_[k] = qp[k];
        }
        const int s2 = 2 * (g & 3);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t hv = alignb(hw_[k + 1], hw_[k], sh), qv = alignb(qw_[k + 1], qw_[k], sh);
            const uint32_t u = ((qv >> s2) & 0x03030303u) | (((hv >> g) & 0x01010101u) << 2);
            q[4 * k] = (float)(u & 0xff);
            q[4 * k + 1] = (float)((u >> 8) & 0xff);
            q[4 * k + 2] = (float)((u >> 16) & 0xff);
            q[4 * k + 3] = (float)(u >> 24);
        }
        const float d = h2f(rd16(blk + 108));
#pragma unroll
        for (int h = 0; h < 2; h++) {
            a[h] = d * (float)(q3k_scale(blk + 96, 2 * g + h) - 32);
            b[h] = -4.0f * a[h];
        }
    } else {
#pragma unroll
        for (int l = 0; l < 32; l++) q[l] = dequant_one(T, wr, 32 * c + l);
        a[0] = a[1] = 1.0f;
        b[0] = b[1] = 0.0f;
    }
}

template <uint32_t T, int MR>
__global__ void __launch_bounds__(256)
gemv_fact_kernel(const uint8_t* __restrict__ w, size_t rb, const float* __restrict__ x, float* __restrict__ y,
                 int K, int N, int ldy) {
    // blockIdx.y: which group of MR activation rows
    x += (size_t)blockIdx.y * MR * K;
    y += (size_t)blockIdx.y * MR * ldy;
    const int lane = threadIdx.x & 63;
    const long nwaves = ((long)gridDim.x * blockDim.x) >> 6;
    const int nch = K >> 5;
    for (long row = ((long)blockIdx.x * blockDim.x + threadIdx.x) >> 6; row < N; row += nwaves) {
        const uint8_t* wr = w + (size_t)row * rb;
        float acc[MR];
#pragma unroll
        for (int m = 0; m < MR; m++) acc[m] = 0.0f;
        for (int c = lane; c < nch; c += 64) {
            float wv[32], ca[2], cb[2];
            chunk_decode<T>(wr, c, wv, ca, cb);
            const bool need_x = cb[0] != 0.0f || cb[1] != 0.0f;
#pragma unroll
            for (int m = 0; m < MR; m++) {
                const float4* xp = reinterpret_cast<const float4*>(x + (size_t)m * K + 32 * c);
                float t = acc[m];
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    float s = 0.0f, xs = 0.0f;
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const float4 v = xp[4 * h + q];
                        const float* wq = wv + 16 * h + 4 * q;
                        s = fmaf(v.x, wq[0], s);
                        s = fmaf(v.y, wq[1], s);
                        s = fmaf(v.z, wq[2], s);
                        s = fmaf(v.w, wq[3], s);
                        xs += (v.x + v.y) + (v.z + v.w);
                    }
                    t = fmaf(ca[h], s, t);
                    if (need_x) t = fmaf(cb[h], xs, t);
                }
                acc[m] = t;
            }
        }
#pragma unroll
        for (int m = 0; m < MR; m++) {
            float v = acc[m];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
            if (lane == 0) y[(size_t)m * ldy + row] = v;
        }
    }
}

// Q5_0 with int8 activations (dot_row_q5_0_int_neon, src/matmul_simd.cpp:184-224):
// per 32-element block the exact integer sum of (code - 16) * q, scaled by
// fp16(d) * xd. Same layout as gemv_fact_kernel: one wave per row at a time,
// lane l taking blocks l, l+64, ...; the 22-byte blocks are 2-byte aligned
// (16-bit loads); the activation codes are 16-byte aligned rows of K.
__device__ __forceinline__ int dot4s(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

template <int MR>
__global__ void __launch_bounds__(256)
gemv_q50_kernel(const uint8_t* __restrict__ w, size_t rb, ActView A, float* __restrict__ y, int K, int N) {
    const int lane = threadIdx.x & 63;
    const long nwaves = ((long)gridDim.x * blockDim.x) >> 6;
    const int nb = K >> 5;
    // blockIdx.y: which group of MR activation rows
    A.qs += (size_t)blockIdx.y * MR * K;
    A.d += (size_t)blockIdx.y * MR * nb;
    y += (size_t)blockIdx.y * MR * N;
    for (long row = ((long)blockIdx.x * blockDim.x + threadIdx.x) >> 6; row < N; row += nwaves) {
        const uint8_t* wr = w + (size_t)row * rb;
        float acc[MR];
#pragma unroll
        for (int m = 0; m < MR; m++) acc[m] = 0.0f;
        for (int b = lane; b < nb; b += 64) {
            const uint16_t* h = reinterpret_cast<const uint16_t*>(wr + (size_t)b * 22);
            const float d = h2f(h[0]);
            const uint32_t qh = (uint32_t)h[1] | ((uint32_t)h[2] << 16);
            uint32_t qs[4];
#pragma unroll
            for (int k = 0; k < 4; k++) qs[k] = (uint32_t)h[3 + 2 * k] | ((uint32_t)h[4 + 2 * k] << 16);
            // codes of elements 4k..4k+3 (low nibbles) and 16+4k.. (high nibbles), minus 16
            uint32_t c[8];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t hb_lo = (qh >> (4 * k)) & 0xfu, hb_hi = (qh >> (16 + 4 * k)) & 0xfu;
                // spread 4 bits into bit 4 of 4 bytes
                const uint32_t s_lo = ((hb_lo & 1u) | ((hb_lo & 2u) << 7) | ((hb_lo & 4u) << 14) | ((hb_lo & 8u) << 21)) << 4;
                const uint32_t s_hi = ((hb_hi & 1u) | ((hb_hi & 2u) << 7) | ((hb_hi & 4u) << 14) | ((hb_hi & 8u) << 21)) << 4;
                // (v - 16) per byte: v in [0, 31] -> v ^ 16 flips bit 4; sign-extend 5 bits
                const uint32_t lo = (qs[k] & 0x0f0f0f0fu) | s_lo;
                const uint32_t hi = ((qs[k] >> 4) & 0x0f0f0f0fu) | s_hi;
                // v - 16 in two's complement bytes: (v ^ 0x10) - 0x10 per byte, done as
                // (v ^ 0x10) | (0xe0 where bit 4 of v ^ 0x10 is set)
                const uint32_t lx = lo ^ 0x10101010u, hx = hi ^ 0x10101010u;
                c[k] = lx | ((lx & 0x10101010u) * 0x0eu);
                c[4 + k] = hx | ((hx & 0x10101010u) * 0x0eu);
            }
#pragma unroll
            for (int m = 0; m < MR; m++) {
                const uint4* aq = reinterpret_cast<const uint4*>(A.qs + (size_t)m * K + 32 * b);
                const uint4 a0 = aq[0], a1 = aq[1];
                int s0 = 0;
                s0 = dot4s(c[0], a0.x, s0); s0 = dot4s(c[1], a0.y, s0);
                s0 = dot4s(c[2], a0.z, s0); s0 = dot4s(c[3], a0.w, s0);
                s0 = dot4s(c[4], a1.x, s0); s0 = dot4s(c[5], a1.y, s0);
                s0 = dot4s(c[6], a1.z, s0); s0 = dot4s(c[7], a1.w, s0);
                acc[m] = fmaf(d * A.d[(size_t)m * nb + b], (float)s0, acc[m]);
            }
        }
#pragma unroll
        for (int m = 0; m < MR; m++) {
            float v = acc[m];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
            if (lane == 0) y[(size_t)m * N + row] = v;
        }
    }
}

// The K-quant types with LDS staging: per-lane loads of a chunk's scattered
// fields (scales, code bytes, high bits) and of its 32 x values are bound by
// the texture-address unit. Instead each wave loads its row with coalesced
// 16-byte loads (lane l: bytes 16l of each KiB), writes it to a per-wave LDS
// buffer and decodes its chunks from there (chunk_decode on LDS pointers);
// the workgroup stages the MR activation rows in LDS once (144-byte stride
// per 32-element chunk, so the 8 float4 reads of a chunk are conflict-free
// across lanes). The next row's bytes are requested before the current row is
// computed. Same per-chunk arithmetic and wave sum as gemv_fact_kernel.
constexpr int kFactLdsPieces = 11;          // row <= 11 KiB: Q5_K K <= 16384
constexpr int kFactChunkStride = 144;       // LDS bytes per 32-element x chunk

template <uint32_t T, int MR>
__global__ void __launch_bounds__(256)
gemv_fact_lds(const uint8_t* __restrict__ w, size_t rb, const float* __restrict__ x, float* __restrict__ y,
              int K, int N, int ldy) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    x += (size_t)blockIdx.y * MR * K;
    y += (size_t)blockIdx.y * MR * ldy;
    const int lane = threadIdx.x & 63;
    const int nch = K >> 5;
    const size_t xrow = (size_t)nch * kFactChunkStride;
    // activation rows -> LDS; each chunk's 16-element half sums go into the
    // chunk's 16 padding bytes (the same for every weight row)
    for (int m = 0; m < MR; m++) {
        for (int i = threadIdx.x; i < (K >> 2); i += blockDim.x) {
            const float4 v = reinterpret_cast<const float4*>(x + (size_t)m * K)[i];
            *reinterpret_cast<float4*>(smem + m * xrow + (i >> 3) * kFactChunkStride + (i & 7) * 16) = v;
        }
    }
    __syncthreads();
    for (int m = 0; m < MR; m++) {
        for (int i = threadIdx.x; i < 2 * nch; i += blockDim.x) {
            const float4* xp = reinterpret_cast<const float4*>(smem + m * xrow + (i >> 1) * kFactChunkStride) + 4 * (i & 1);
            float xs = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float4 xv = xp[q];
                xs += (xv.x + xv.y) + (xv.z + xv.w);
            }
            reinterpret_cast<float*>(smem + m * xrow + (i >> 1) * kFactChunkStride + 128)[i & 1] = xs;
        }
    }
    const size_t rbuf = (rb + 1023) & ~size_t(1023);
    uint8_t* wb = smem + MR * xrow + (threadIdx.x >> 6) * rbuf;
    const int nld = (int)((rb + 1023) / 1024);
    const long nwaves = ((long)gridDim.x * blockDim.x) >> 6;
    long row = (long)blockIdx.x * (blockDim.x >> 6) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    u32x4 v[kFactLdsPieces];
    auto load_row = [&](long r) {
        const uint8_t* src = w + (size_t)r * rb;
#pragma unroll
        for (int k = 0; k < kFactLdsPieces; k++) {
            if (k < nld) {
                size_t o = 1024 * (size_t)k + 16 * lane;
                o = o + 16 <= rb ? o : rb - 16;
                v[k] = *reinterpret_cast<const u32x4*>(src + o);
            }
        }
    };
    if (row < N) load_row(row);
    __syncthreads();
    for (; row < N; row += nwaves) {
        // a piece clamped to the row's last 16 bytes goes back to where it came
        // from (rows need not be a multiple of 16 bytes)
#pragma unroll
        for (int k = 0; k < kFactLdsPieces; k++) {
            if (k < nld) {
                size_t o = 1024 * (size_t)k + 16 * lane;
                if (o + 16 <= rb) {
                    *reinterpret_cast<u32x4*>(wb + o) = v[k];
                } else {
                    o = rb - 16;                            // 4-byte aligned (rb % 4 == 0)
                    uint32_t* d4 = reinterpret_cast<uint32_t*>(wb + o);
                    d4[0] = v[k].x; d4[1] = v[k].y; d4[2] = v[k].z; d4[3] = v[k].w;
                }
            }
        }
        if (row + nwaves < N) load_row(row + nwaves);
        float acc[MR];
#pragma unroll
        for (int m = 0; m < MR; m++) acc[m] = 0.0f;
        for (int c = lane; c < nch; c += 64) {
            float wv[32], ca[2], cb[2];
            chunk_decode<T>(wb, c, wv, ca, cb);
            const bool need_x = cb[0] != 0.0f || cb[1] != 0.0f;
#pragma unroll
            for (int m = 0; m < MR; m++) {
                const float4* xp = reinterpret_cast<const float4*>(smem + m * xrow + (size_t)c * kFactChunkStride);
                const float2 xsum = *reinterpret_cast<const float2*>(smem + m * xrow + (size_t)c * kFactChunkStride + 128);
                float t = acc[m];
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    float sx = 0.0f;
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const float4 xv = xp[4 * h + q];
                        const float* wq = wv + 16 * h + 4 * q;
                        sx = fmaf(xv.x, wq[0], sx);
                        sx = fmaf(xv.y, wq[1], sx);
                        sx = fmaf(xv.z, wq[2], sx);
                        sx = fmaf(xv.w, wq[3], sx);
                    }
                    t = fmaf(ca[h], sx, t);
                    if (need_x) t = fmaf(cb[h], h ? xsum.y : xsum.x, t);
                }
                acc[m] = t;
            }
        }
#pragma unroll
        for (int m = 0; m < MR; m++) {
            float s2 = acc[m];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) s2 += __shfl_xor(s2, off, 64);
            if (lane == 0) y[(size_t)m * ldy + row] = s2;
        }
    }
}

// F32 / F16 / BF16 weights: a lane takes 8 consecutive elements of every
// 512-element slab of the row (16-byte loads for the 2-byte types, two for
// F32; x the same way), so each wave streams its row with fully coalesced
// loads, eight slabs in flight; fp32 products summed per lane, then over the
// wave (dot_row_f16 / dot_row_bf16 / dot_row_f32, src/matmul.cpp:63-101,
// reassociated).
template <uint32_t T>
__device__ __forceinline__ void dense8(const uint8_t* __restrict__ p, float (&o)[8]) {
    if constexpr (T == T_F32) {
        const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
        o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
    } else {
        const u32x4 v = *reinterpret_cast<const u32x4*>(p);
        const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            if constexpr (T == T_F16) {
                o[2 * k] = h2f(u[k] & 0xffffu);
                o[2 * k + 1] = h2f(u[k] >> 16);
            } else {
                o[2 * k] = __uint_as_float(u[k] << 16);
                o[2 * k + 1] = __uint_as_float(u[k] & 0xffff0000u);
            }
        }
    }
}

// U slabs in flight per lane
template <uint32_t T, int MR, int U>
__global__ void __launch_bounds__(256)
gemv_dense_kernel(const uint8_t* __restrict__ w, const float* __restrict__ x, float* __restrict__ y, int K,
                  int N, int ldy) {
    constexpr int EB = T == T_F32 ? 4 : 2;        // bytes per element
    x += (size_t)blockIdx.y * MR * K;
    y += (size_t)blockIdx.y * MR * ldy;
    const int lane = threadIdx.x & 63;
    const long nwaves = ((long)gridDim.x * blockDim.x) >> 6;
    for (long row = ((long)blockIdx.x * blockDim.x + threadIdx.x) >> 6; row < N; row += nwaves) {
        const uint8_t* wr = w + (size_t)row * K * EB;
        float acc[MR];
#pragma unroll
        for (int m = 0; m < MR; m++) acc[m] = 0.0f;
        for (int e0 = 8 * lane; e0 < K; e0 += U * 512) {
            float wv[U][8];
#pragma unroll
            for (int u = 0; u < U; u++)
                if (e0 + 512 * u < K) dense8<T>(wr + (size_t)(e0 + 512 * u) * EB, wv[u]);
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int e = e0 + 512 * u;
                if (e < K) {
#pragma unroll
                    for (int m = 0; m < MR; m++) {
                        const float4* xp = reinterpret_cast<const float4*>(x + (size_t)m * K + e);
                        const float4 a = xp[0], b = xp[1];
                        float t = acc[m];
                        t = fmaf(a.x, wv[u][0], t); t = fmaf(a.y, wv[u][1], t);
                        t = fmaf(a.z, wv[u][2], t); t = fmaf(a.w, wv[u][3], t);
                        t = fmaf(b.x, wv[u][4], t); t = fmaf(b.y, wv[u][5], t);
                        t = fmaf(b.z, wv[u][6], t); t = fmaf(b.w, wv[u][7], t);
                        acc[m] = t;
                    }
                }
            }
        }
#pragma unroll
        for (int m = 0; m < MR; m++) {
            float s2 = acc[m];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) s2 += __shfl_xor(s2, off, 64);
            if (lane == 0) y[(size_t)m * ldy + row] = s2;
        }
    }
}

// LDS bytes of gemv_fact_lds for MR activation rows; 0 when it does not apply.
static size_t fact_lds_bytes(uint32_t T, int MR, int K, size_t rb) {
    if (!(T == T_Q2_K || T == T_Q3_K || T == T_Q5_K)) return 0;
    if (rb % 4 != 0 || rb < 16 || (rb + 1023) / 1024 > kFactLdsPieces) return 0;
    const size_t b = (size_t)MR * (K / 32) * kFactChunkStride + 4 * ((rb + 1023) & ~size_t(1023));
    return b <= 160 * 1024 ? b : 0;
}

template <uint32_t T>
static hipError_t launch_fact_t(const uint8_t* w, const float* x, float* y, int M, int K, int N, hipStream_t st) {
    const size_t rb = fact_row_bytes(T, K);
    if constexpr (T == T_Q2_K || T == T_Q3_K || T == T_Q5_K) {
        // one row group of up to 4 activation rows per launch (grid.y = group)
        if (reinterpret_cast<uintptr_t>(w) % 4 == 0 && fact_lds_bytes(T, M < 4 ? M : 4, K, rb)) {
            const long cap = (long)device_cu_count() * 12;    // 3 workgroups per CU
            const long waves = N < cap ? N : cap;
            const unsigned gx = (unsigned)((waves + 3) / 4);
            // full groups of 4 activation rows in one launch (grid.y = group),
            // the remainder in a second
            const int full = M / 4, rest = M % 4;
            if (full)
                hipLaunchKernelGGL((gemv_fact_lds<T, 4>), dim3(gx, full), dim3(256), fact_lds_bytes(T, 4, K, rb), st,
                                   w, rb, x, y, K, N, N);
            if (rest) {
                const float* xm = x + (size_t)full * 4 * K;
                float* ym = y + (size_t)full * 4 * N;
                const size_t shm = fact_lds_bytes(T, rest, K, rb);
                switch (rest) {
                    case 1: hipLaunchKernelGGL((gemv_fact_lds<T, 1>), dim3(gx), dim3(256), shm, st, w, rb, xm, ym, K, N, N); break;
                    case 2: hipLaunchKernelGGL((gemv_fact_lds<T, 2>), dim3(gx), dim3(256), shm, st, w, rb, xm, ym, K, N, N); break;
                    default: hipLaunchKernelGGL((gemv_fact_lds<T, 3>), dim3(gx), dim3(256), shm, st, w, rb, xm, ym, K, N, N); break;
                }
            }
            return hipGetLastError();
        }
    }
    if constexpr (T == T_F32 || T == T_F16 || T == T_BF16) {
        if (reinterpret_cast<uintptr_t>(w) % 16 == 0 && K % 8 == 0) {
            const long cap = (long)device_cu_count() * 32;
            const long waves = N < cap ? N : cap;
            const unsigned gx = (unsigned)((waves + 3) / 4);
            const int full = M / 4, rest = M % 4;
            // eight slabs per lane while the rows fit 16 waves per CU; four
            // (fewer registers, all 32 waves per CU resident) beyond (BF16,
            // K 4096: 4096 rows 10.5 / 10.75 us with 8 / 4, 14336 rows 34.3 /
            // 28.0; 16 slabs 15.4 / 35.1)
            const bool u8 = N <= (long)device_cu_count() * 16;
#define LP_DN(MR, G, XM, YM)                                                                                  \
    if (u8) hipLaunchKernelGGL((gemv_dense_kernel<T, MR, 8>), G, dim3(256), 0, st, w, XM, YM, K, N, N);       \
    else hipLaunchKernelGGL((gemv_dense_kernel<T, MR, 4>), G, dim3(256), 0, st, w, XM, YM, K, N, N)
            if (full) LP_DN(4, dim3(gx, full), x, y);
            if (rest) {
                const float* xm = x + (size_t)full * 4 * K;
                float* ym = y + (size_t)full * 4 * N;
                switch (rest) {
                    case 1: LP_DN(1, dim3(gx), xm, ym); break;
                    case 2: LP_DN(2, dim3(gx), xm, ym); break;
                    default: LP_DN(3, dim3(gx), xm, ym); break;
                }
            }
#undef LP_DN
            return hipGetLastError();
        }
    }
    // one launch for the full groups of 4 activation rows (grid.y = group),
    // one for the remainder
    const int full = M / 4, rest = M % 4;
    long waves = (long)N * (full + (rest ? 1 : 0));
    const long cap = (long)device_cu_count() * 32;
    const long per = waves > cap ? (cap + (full ? full : 1) - 1) / (full ? full : 1) : N;
    const unsigned gx = (unsigned)((per + 3) / 4);
    if (full) hipLaunchKernelGGL((gemv_fact_kernel<T, 4>), dim3(gx, full), dim3(256), 0, st, w, rb, x, y, K, N, N);
    if (rest) {
        const float* xm = x + (size_t)full * 4 * K;
        float* ym = y + (size_t)full * 4 * N;
        const unsigned g1 = (unsigned)(((N < cap ? N : cap) + 3) / 4);
        switch (rest) {
            case 1: hipLaunchKernelGGL((gemv_fact_kernel<T, 1>), dim3(g1), dim3(256), 0, st, w, rb, xm, ym, K, N, N); break;
            case 2: hipLaunchKernelGGL((gemv_fact_kernel<T, 2>), dim3(g1), dim3(256), 0, st, w, rb, xm, ym, K, N, N); break;
            default: hipLaunchKernelGGL((gemv_fact_kernel<T, 3>), dim3(g1), dim3(256), 0, st, w, rb, xm, ym, K, N, N); break;
        }
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemv_q50(const uint8_t* w, const ActView& A, float* y, int M, int K, int N, hipStream_t st) {
    if (M <= 0 || N <= 0) return hipSuccess;
    const size_t rb = (size_t)(K / 32) * 22;
    long waves = N;
    const long cap = (long)device_cu_count() * 32;
    if (waves > cap) waves = cap;
    const unsigned grid = (unsigned)((waves + 3) / 4);
    const int nb = K / 32;
    // full groups of 4 activation rows in one launch (grid.y = group), the
    // remainder in a second
    const int full = M / 4, rest = M % 4;
    if (full) hipLaunchKernelGGL((gemv_q50_kernel<4>), dim3(grid, full), dim3(256), 0, st, w, rb, A, y, K, N);
    if (rest) {
        ActView Am = A;
        Am.qs = A.qs + (size_t)full * 4 * K;
        Am.d = A.d + (size_t)full * 4 * nb;
        float* ym = y + (size_t)full * 4 * N;
        switch (rest) {
            case 1: hipLaunchKernelGGL((gemv_q50_kernel<1>), dim3(grid), dim3(256), 0, st, w, rb, Am, ym, K, N); break;
            case 2: hipLaunchKernelGGL((gemv_q50_kernel<2>), dim3(grid), dim3(256), 0, st, w, rb, Am, ym, K, N); break;
            default: hipLaunchKernelGGL((gemv_q50_kernel<3>), dim3(grid), dim3(256), 0, st, w, rb, Am, ym, K, N); break;
        }
    }
    return hipGetLastError();
}

bool fact_type(uint32_t type) {
    // Q5_0 is not among them: the reference's int8 back-end takes it
    // (gemm_simd, src/matmul_simd.cpp:486)
    switch (type) {
        case T_F32: case T_F16: case T_BF16: case T_Q2_K: case T_Q3_K: case T_Q5_K: return true;
        default: return false;
    }
}

size_t fact_row_bytes(uint32_t type, int K) {
    switch (type) {
        case T_F32: return (size_t)K * 4;
        case T_F16: case T_BF16: return (size_t)K * 2;
        case T_Q5_0: return (size_t)(K / 32) * 22;
        case T_Q2_K: return (size_t)(K / 256) * 84;
        case T_Q3_K: return (size_t)(K / 256) * 110;
        case T_Q5_K: return (size_t)(K / 256) * 176;
        default: return 0;
    }
}

hipError_t launch_gemv_fact(uint32_t type, const uint8_t* w, const float* x, float* y, int M, int K, int N,
                            hipStream_t st) {
    if (M <= 0 || N <= 0) return hipSuccess;
    switch (type) {
        case T_F32: return launch_fact_t<T_F32>(w, x, y, M, K, N, st);
        case T_F16: return launch_fact_t<T_F16>(w, x, y, M, K, N, st);
        case T_BF16: return launch_fact_t<T_BF16>(w, x, y, M, K, N, st);
        case T_Q5_0: return launch_fact_t<T_Q5_0>(w, x, y, M, K, N, st);
        case T_Q2_K: return launch_fact_t<T_Q2_K>(w, x, y, M, K, N, st);
        case T_Q3_K: return launch_fact_t<T_Q3_K>(w, x, y, M, K, N, st);
        case T_Q5_K: return launch_fact_t<T_Q5_K>(w, x, y, M, K, N, st);
        default: return hipErrorInvalidValue;
    }
}

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
    if (n % 8 == 0 && reinterpret_cast<uintptr_t>(dst) % 16 == 0) {
        const long n8 = n / 8;
        long g8 = (n8 + 255) / 256;
        if (g8 > 65536) g8 = 65536;
        const dim3 grid((unsigned)g8);
        const bool wide = dequant_wide_ok(type, w);
        switch (type) {
#define LP_D(TT)                                                                                          \
    case TT:                                                                                              \
        if (wide) hipLaunchKernelGGL((dequant8_kernel<TT, true>), grid, dim3(256), 0, st, w, dst, n8);    \
        else hipLaunchKernelGGL((dequant8_kernel<TT, false>), grid, dim3(256), 0, st, w, dst, n8);        \
        return hipGetLastError();
            LP_D(T_F32) LP_D(T_F16) LP_D(T_BF16) LP_D(T_Q4_0) LP_D(T_Q5_0) LP_D(T_Q8_0) LP_D(T_Q2_K) LP_D(T_Q3_K)
            LP_D(T_Q4_K) LP_D(T_Q5_K) LP_D(T_Q6_K)
#undef LP_D
            default: break;
        }
    }
    long grid = (n + 255) / 256;
    if (grid > 65536) grid = 65536;
    hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)grid), dim3(256), 0, st, type, w, dst, n);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Byte copy by a kernel (16-byte pieces where both ends allow, else 4 bytes):
// for small transfers between device memory and device-mapped pinned host
// memory, where a kernel's PCIe reads and posted writes finish sooner than a
// DMA copy is set up.
__global__ void __launch_bounds__(256) copy_kernel(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src,
                                                   size_t bytes, int wide) {
    const size_t n16 = wide ? bytes / 16 : 0;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
        reinterpret_cast<u32x4*>(dst)[i] = reinterpret_cast<const u32x4*>(src)[i];
    for (size_t i = n16 * 4 + (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < bytes / 4; i += stride)
        reinterpret_cast<uint32_t*>(dst)[i] = reinterpret_cast<const uint32_t*>(src)[i];
}

hipError_t launch_copy(void* dst, const void* src, size_t bytes, hipStream_t st) {
    if (bytes == 0) return hipSuccess;
    if (bytes % 4 != 0 || reinterpret_cast<uintptr_t>(dst) % 4 != 0 || reinterpret_cast<uintptr_t>(src) % 4 != 0)
        return hipErrorInvalidValue;
    const int wide = reinterpret_cast<uintptr_t>(dst) % 16 == 0 && reinterpret_cast<uintptr_t>(src) % 16 == 0;
    size_t blocks = (bytes + 4095) / 4096;
    if (blocks > 256) blocks = 256;
    hipLaunchKernelGGL(copy_kernel, dim3((unsigned)blocks), dim3(256), 0, st, static_cast<uint8_t*>(dst),
                       static_cast<const uint8_t*>(src), bytes, wide);
    return hipGetLastError();
}

}  // namespace lp
