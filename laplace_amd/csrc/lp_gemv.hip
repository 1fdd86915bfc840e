// lp_gemv.hip - activation quantizer, decode GEMV (M <= 8) and the
// per-block integer-sum probe, for gfx950.
//
// Reference behaviour followed:
//   quantize_act_q8_neon   src/matmul_simd.cpp:348-410
//   gemm_int<dot_row_*>    src/matmul_simd.cpp:432-455 (+ dots :143-342)
//
// GEMV design (HBM-bound: ~0.56-1.06 B of weight per element, no reuse):
//   * one lane owns one 64-element chunk of K; a row is handled by LPR
//     lanes (LPR = next power of two >= K/64, so 64 lanes at K = 4096);
//   * the lane's quantized activations (M rows x 64 codes + scales) are
//     loaded once into registers and reused for every weight row the lane
//     visits, so HBM traffic is the weight stream plus one activation read
//     per workgroup;
//   * weights are read once, as nontemporal dword loads of the packed
//     blocks, unpacked in registers and dotted with v_dot4_i32_i8; R rows are
//     loaded before any is reduced to keep several KB in flight per wave;
//   * the LPR partial sums of a row are combined with cross-lane shuffles,
//     and through LDS when LPR spans several waves.
#include <hip/hip_runtime.h>

#include "lp_chunks.h"
#include "lp_internal.h"

namespace lp {

// ---------------------------------------------------------------------------
// Quantizer: 8 lanes per 32-element block, one float4 per lane.

__device__ __forceinline__ int32_t cvt_rne_sat(float v) {
    // vcvtnq_s32_f32: ties to even, saturating, NaN -> 0.
    const float r = __builtin_rintf(v);
    if (r != r) return 0;
    if (r >= 2147483648.0f) return 2147483647;
    if (r < -2147483648.0f) return (int32_t)0x80000000u;
    return (int32_t)r;
}

__global__ void __launch_bounds__(256)
quantize_act_kernel(const float* __restrict__ x, int M, int K, ActView A) {
    const int nb = K >> 5;
    const long total = (long)M * nb;
    const int g = threadIdx.x & 7;                       // lane within the block's group
    const long stride = (long)gridDim.x * (blockDim.x >> 3);
    for (long blk = (long)blockIdx.x * (blockDim.x >> 3) + (threadIdx.x >> 3); blk < total;
         blk += stride) {
        const long m = blk / nb, b = blk - m * nb;
        const float4 v = *reinterpret_cast<const float4*>(x + m * K + 32 * b + 4 * g);
        float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
        int nan = (v.x != v.x) | (v.y != v.y) | (v.z != v.z) | (v.w != v.w);
#pragma unroll
        for (int off = 1; off < 8; off <<= 1) {
            amax = fmaxf(amax, __shfl_xor(amax, off, 8));
            nan |= __shfl_xor(nan, off, 8);
        }
        if (nan) amax = __builtin_nanf("");                // FMAX propagates NaN
        const float d = amax / 127.0f;
        const float id = d > 0.0f ? 1.0f / d : 0.0f;
        const int32_t q0 = cvt_rne_sat(v.x * id), q1 = cvt_rne_sat(v.y * id);
        const int32_t q2 = cvt_rne_sat(v.z * id), q3 = cvt_rne_sat(v.w * id);
        // int32 sums wrap modulo 2^32 as the NEON lane adds do.
        uint32_t s = (uint32_t)q0 + (uint32_t)q1 + (uint32_t)q2 + (uint32_t)q3;
        s += __shfl_xor(s, 1, 8);
        s += __shfl_xor(s, 2, 8);                          // lanes 0-3: elems 0-15, 4-7: 16-31
        const uint32_t s_hi = __shfl_xor(s, 4, 8);
        auto sat8 = [](int32_t q) -> uint32_t {
            q = q > 127 ? 127 : (q < -128 ? -128 : q);
            return (uint32_t)(q & 0xff);
        };
        const uint32_t packed = sat8(q0) | (sat8(q1) << 8) | (sat8(q2) << 16) | (sat8(q3) << 24);
        *reinterpret_cast<uint32_t*>(A.qs + m * K + 32 * b + 4 * g) = packed;
        if (g == 0) {
            const int16_t lo = (int16_t)(uint16_t)s;
            const int16_t hi = (int16_t)(uint16_t)s_hi;
            A.d[blk] = d;
            A.sum[blk] = d * (float)((int32_t)lo + (int32_t)hi);
            A.s16[blk] = (int32_t)(((uint32_t)(uint16_t)lo) | ((uint32_t)(uint16_t)hi << 16));
        }
    }
}

hipError_t launch_quantize(const float* x, int M, int K, const ActView& A, hipStream_t st) {
    const long blocks = (long)M * (K >> 5);
    if (blocks == 0) return hipSuccess;
    long grid = (blocks + 31) / 32;
    if (grid > 8192) grid = 8192;
    hipLaunchKernelGGL(quantize_act_kernel, dim3((unsigned)grid), dim3(256), 0, st, x, M, K, A);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// GEMV.
//
// Grid: each workgroup of WG = max(256, LPR) lanes holds SPW = WG / LPR row
// slots. Slot s of workgroup b owns rows (b*SPW + s)*R + i*(gridDim*SPW*R)
// + r for r < R, i = 0, 1, ...; every lane of the workgroup runs the same
// number of iterations so the LDS barriers (LPR > 64) stay uniform.

template <uint32_t T, int M, int R>
__global__ void __launch_bounds__(512)
gemv_kernel(const uint8_t* __restrict__ w, size_t rb, ActView A, float* __restrict__ y,
            int K, int N, int lpr, int iters) {
    using C = Chunk<T>;
    extern __shared__ float red[];                      // [WG/64][R*M] when lpr > 64
    const int tid = threadIdx.x;
    const int lane_in_row = tid & (lpr - 1);
    const int slot = tid / lpr;
    const int spw = blockDim.x / lpr;
    const int nchunks = K >> 6;
    const bool active = lane_in_row < nchunks;
    const int c = active ? lane_in_row : 0;

    typename C::Act act[M];
#pragma unroll
    for (int m = 0; m < M; m++) load_act<T>(A, K, m, c, act[m]);

    const long gstride = (long)gridDim.x * spw * R;
    long row0 = ((long)blockIdx.x * spw + slot) * R;
    for (int it = 0; it < iters; it++, row0 += gstride) {
        typename C::Wt wt[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const long row = row0 + r;
            if (active && row < N) C::load_w(w + row * rb, c, wt[r]);
        }
        float part[R][M];
#pragma unroll
        for (int r = 0; r < R; r++) {
#pragma unroll
            for (int m = 0; m < M; m++) {
                float p = 0.0f;
                if (active && row0 + r < N) {
                    int is[C::NSUB];
                    C::isums(wt[r], act[m], is);
                    p = C::partial(wt[r], act[m], is, c);
                }
                part[r][m] = p;
            }
        }
        // reduce over the lpr lanes of the row (within a wave first)
        const int wl = lpr < 64 ? lpr : 64;
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int m = 0; m < M; m++)
                for (int off = wl >> 1; off >= 1; off >>= 1)
                    part[r][m] += __shfl_xor(part[r][m], off, 64);
        if (lpr <= 64) {
            if (lane_in_row == 0) {
#pragma unroll
                for (int r = 0; r < R; r++)
                    if (row0 + r < N)
#pragma unroll
                        for (int m = 0; m < M; m++) y[(size_t)m * N + row0 + r] = part[r][m];
            }
        } else {
            const int wave = tid >> 6, nw = lpr >> 6;
            if ((tid & 63) == 0) {
#pragma unroll
                for (int r = 0; r < R; r++)
#pragma unroll
                    for (int m = 0; m < M; m++) red[wave * R * M + r * M + m] = part[r][m];
            }
            __syncthreads();
            // one lane per (r, m) of this slot's first wave finishes the sum
            const int first = slot * nw;
            if (wave == first && (tid & 63) < R * M) {
                const int rm = tid & 63;
                float s = 0.0f;
                for (int i = 0; i < nw; i++) s += red[(first + i) * R * M + rm];
                const int r = rm / M, m = rm % M;
                if (row0 + r < N) y[(size_t)m * N + row0 + r] = s;
            }
            __syncthreads();
        }
    }
}

template <uint32_t T, int M, int R>
static hipError_t launch_gemv_t(const uint8_t* w, const ActView& A, float* y, int K, int N,
                                hipStream_t st) {
    const int nchunks = K >> 6;
    int lpr = 1;
    while (lpr < nchunks) lpr <<= 1;
    if (lpr > 512) return hipErrorInvalidValue;   // K > 32768: not handled here
    const int wg = lpr > 256 ? lpr : 256;
    const int spw = wg / lpr;
    const long groups = ((long)N + R - 1) / R;           // R-row groups
    long want = (groups + spw - 1) / spw;                // workgroups for one pass
    const long cap = (long)device_cu_count() * (2048 / wg);   // ~8 waves per CU resident
    const long grid = want < cap ? want : cap;
    const int iters = (int)((groups + grid * spw - 1) / (grid * spw));
    const size_t rb = row_bytes(T, K);
    const size_t shm = lpr > 64 ? sizeof(float) * (wg / 64) * R * M : 0;
    hipLaunchKernelGGL((gemv_kernel<T, M, R>), dim3((unsigned)grid), dim3(wg), shm, st,
                       w, rb, A, y, K, N, lpr, iters);
    return hipGetLastError();
}

template <uint32_t T>
static hipError_t launch_gemv_type(const uint8_t* w, const ActView& A, float* y, int M, int K,
                                   int N, hipStream_t st) {
    switch (M) {
        case 1: return launch_gemv_t<T, 1, 4>(w, A, y, K, N, st);
        case 2: return launch_gemv_t<T, 2, 4>(w, A, y, K, N, st);
        case 3: return launch_gemv_t<T, 3, 2>(w, A, y, K, N, st);
        case 4: return launch_gemv_t<T, 4, 2>(w, A, y, K, N, st);
        case 5: return launch_gemv_t<T, 5, 2>(w, A, y, K, N, st);
        case 6: return launch_gemv_t<T, 6, 2>(w, A, y, K, N, st);
        case 7: return launch_gemv_t<T, 7, 1>(w, A, y, K, N, st);
        case 8: return launch_gemv_t<T, 8, 1>(w, A, y, K, N, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv(uint32_t type, const uint8_t* w, const ActView& A, float* y, int M, int K,
                       int N, hipStream_t st) {
    if (M <= 0 || N <= 0) return hipSuccess;
    switch (type) {
        case T_Q8_0: return launch_gemv_type<T_Q8_0>(w, A, y, M, K, N, st);
        case T_Q4_0: return launch_gemv_type<T_Q4_0>(w, A, y, M, K, N, st);
        case T_Q4_K: return launch_gemv_type<T_Q4_K>(w, A, y, M, K, N, st);
        case T_Q6_K: return launch_gemv_type<T_Q6_K>(w, A, y, M, K, N, st);
        default: return hipErrorInvalidValue;
    }
}

// ---------------------------------------------------------------------------
// Integer sub-block sums through the same chunk decoders (test probe):
// out[(m*N + row) * nsub + s], nsub = K/32 (K/16 for Q6_K).

template <uint32_t T>
__global__ void __launch_bounds__(256)
block_sums_kernel(const uint8_t* __restrict__ w, size_t rb, ActView A, int32_t* __restrict__ out,
                  int M, int K, int N) {
    using C = Chunk<T>;
    const int nchunks = K >> 6;
    const long total = (long)M * N * nchunks;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (long)gridDim.x * blockDim.x) {
        const int c = (int)(i % nchunks);
        const long mr = i / nchunks;
        const int row = (int)(mr % N), m = (int)(mr / N);
        typename C::Act a;
        load_act<T>(A, K, m, c, a);
        typename C::Wt wt;
        C::load_w(w + (size_t)row * rb, c, wt);
        int is[C::NSUB];
        C::isums(wt, a, is);
        const int nsub = nchunks * C::NSUB;
#pragma unroll
        for (int s = 0; s < C::NSUB; s++) out[mr * nsub + C::sub_index(c, s)] = is[s];
    }
}

hipError_t launch_block_sums(uint32_t type, const uint8_t* w, const ActView& A, int32_t* out,
                             int M, int K, int N, hipStream_t st) {
    const long total = (long)M * N * (K >> 6);
    if (total == 0) return hipSuccess;
    long grid = (total + 255) / 256;
    if (grid > 65536) grid = 65536;
    const size_t rb = row_bytes(type, K);
    switch (type) {
        case T_Q8_0: hipLaunchKernelGGL(block_sums_kernel<T_Q8_0>, dim3(grid), dim3(256), 0, st, w, rb, A, out, M, K, N); break;
        case T_Q4_0: hipLaunchKernelGGL(block_sums_kernel<T_Q4_0>, dim3(grid), dim3(256), 0, st, w, rb, A, out, M, K, N); break;
        case T_Q4_K: hipLaunchKernelGGL(block_sums_kernel<T_Q4_K>, dim3(grid), dim3(256), 0, st, w, rb, A, out, M, K, N); break;
        case T_Q6_K: hipLaunchKernelGGL(block_sums_kernel<T_Q6_K>, dim3(grid), dim3(256), 0, st, w, rb, A, out, M, K, N); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace lp
