// lp_gemm.hip - prefill GEMM for Q4_K weights (M > 8 tokens) on gfx950 MFMA.
//
// Reference semantics: gemm_int<dot_row_q4_k_int_neon> row by row
// (src/matmul_simd.cpp:226-283, 432-455):
//   y[m,n] = sum_sb [ d_n * sum_{b in sb} sc_nb * xd_mb * P_mnb
//                     - dmin_n * sum_{b in sb} mn_nb * xs_mb ]
// with P_mnb = sum_{k in b} nib_nk * q_mk, xd/xs/q the ActQ8 activation
// blocks (src/matmul_simd.cpp:348-410).
//
// Why not int8 MFMA: the activation scale xd_mb changes every 32 elements,
// so an int8 MFMA per 32-K block must be followed by >= 3 VALU operations
// per output (int->float, scale, accumulate). At M=2048, N=14336, K=4096
// that is 3.8e9 element-blocks per op, ~96 us of VALU per op on 256 CUs,
// which caps the int8 route far below the MFMA rate. Instead the block
// scale is folded into the operands, exactly:
//   A[m,k] = xd_mb * q_mk  (fp32 product) split as hi = fp16(A), lo = fp16(A - hi)
//   V[n,k] = sc_nb * nib_nk   (an integer <= 945: exact in fp16)
// so sum_k A*V over a super-block is two fp16 MFMA streams (hi, lo) with
// fp32 accumulation, and the only per-output epilogue is per super-block
// (x d_n). The min term sum_b mn_nb*xs_mb is a second, K = 8 per
// super-block, fp16 MFMA (xs split hi/lo; the 6-bit mn exact). Every
// activation row is pre-scaled by an exact power of two (undone in the
// epilogue) so its values sit well inside fp16 range. The result equals the
// reference's within fp32 rounding (relative error ~1e-6).
//
// Tiling: workgroup = 8 waves, output tile 128 tokens x 256 weight rows,
// K step 64 (a quarter super-block). Each wave owns 64 x 64 = 2 x 2 MFMA
// tiles of 32 x 32 (v_mfma_f32_32x32x16_f16). Per K step, the activation
// hi/lo planes (32 KB) and the raw 4-bit codes of the weight rows (8 KB)
// are copied into LDS with global_load_lds_dwordx4 (1 KiB per wave
// instruction), double buffered; super-block headers and activation sums
// are staged once per super-block. The 4-bit codes are turned into fp16 V
// in registers (v_perm + magic-number packed-fp16 FMA).
#include <hip/hip_runtime.h>

#include "lp_device.h"
#include "lp_internal.h"

namespace lp {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f16v __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------------------
// Activation planes for the GEMM, built from the quantized activations.
//   hi, lo : fp16 [M][K]        xd*q*2^-E_m split into two fp16
//   shi, slo : fp16 [M][K/32]   xs*2^-E_m split likewise
//   escale : f32 [M]            2^E_m (applied to the row's outputs)
// E_m = exponent of max_b xd_mb, so |xd*q*2^-E| <= 127.

__global__ void __launch_bounds__(256)
gemm_prep_kernel(ActView A, int K, _Float16* __restrict__ hi, _Float16* __restrict__ lo,
                 _Float16* __restrict__ shi, _Float16* __restrict__ slo,
                 float* __restrict__ escale) {
    const int m = blockIdx.x;
    const int nb = K >> 5;
    const float* d = A.d + (size_t)m * nb;
    const float* s = A.sum + (size_t)m * nb;
    __shared__ float red[256];
    float mx = 0.0f;
    for (int b = threadIdx.x; b < nb; b += blockDim.x) mx = fmaxf(mx, fabsf(d[b]));
    red[threadIdx.x] = mx;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (threadIdx.x < o) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + o]);
        __syncthreads();
    }
    mx = red[0];
    int e = 0;
    if (mx > 0.0f && mx == mx && mx < 3.0e38f) (void)frexpf(mx, &e);   // mx = f * 2^e, f in [0.5, 1)
    const float inv = ldexpf(1.0f, -e);
    if (threadIdx.x == 0) escale[m] = ldexpf(1.0f, e);
    const int8_t* q = A.qs + (size_t)m * K;
    for (int k = threadIdx.x; k < K; k += blockDim.x) {
        const float v = (d[k >> 5] * inv) * (float)q[k];
        const _Float16 h = (_Float16)v;
        hi[(size_t)m * K + k] = h;
        lo[(size_t)m * K + k] = (_Float16)(v - (float)h);
    }
    for (int b = threadIdx.x; b < nb; b += blockDim.x) {
        const float v = s[b] * inv;
        const _Float16 h = (_Float16)v;
        shi[(size_t)m * nb + b] = h;
        slo[(size_t)m * nb + b] = (_Float16)(v - (float)h);
    }
}

// ---------------------------------------------------------------------------

constexpr int BM = 128, BN = 256, BK = 64;
constexpr int kGemmThreads = 512;
constexpr int A_PLANE = BM * BK * 2;          // 16 KB per plane per stage
constexpr int B_TILE = BN * 32;               // 8 KB of codes per stage
constexpr int STAGE = 2 * A_PLANE + B_TILE;   // 40 KB
constexpr int HDR = BN * 16;                  // 4 KB super-block headers
constexpr int XS = BM * 16;                   // 2 KB per xs plane
constexpr int SB_STAGE = HDR + 2 * XS;        // 8 KB
constexpr int GEMM_LDS = 2 * STAGE + 2 * SB_STAGE;   // 96 KB

__device__ __forceinline__ void dma16(const void* g, uint8_t* lds) {
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

struct GemmArgs {
    const _Float16* hi;
    const _Float16* lo;
    const _Float16* shi;
    const _Float16* slo;
    const float* escale;
    const uint8_t* w;
    size_t rb;
    float* y;
    int M, N, K;
};

// Copies for K step kt of tile (m0, n0) into stage buffer `st` (and, at a
// super-block start, its headers and activation sums into `sbb`). Returns
// the number of DMA instructions this wave issued.
__device__ __forceinline__ int issue_kstep(const GemmArgs& g, int m0, int n0, int kt, uint8_t* st,
                                           uint8_t* sbb, int wave, int lane) {
    const int k0 = kt * BK;
    const int sb = kt >> 2, jb = kt & 3;
    int n = 0;
    // activation planes: 16 instructions each, 8 rows x 128 B per instruction,
    // 16-byte pieces XOR-swizzled by (row & 7)
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int p = wave * 4 + i;                  // 0..31
        const int plane = p >> 4, pp = p & 15;
        const int row = pp * 8 + (lane >> 3);
        const int piece = (lane & 7) ^ (row & 7);
        int gm = m0 + row;
        gm = gm < g.M ? gm : g.M - 1;
        const _Float16* src = (plane ? g.lo : g.hi) + (size_t)gm * g.K + k0 + piece * 8;
        dma16(src, st + plane * A_PLANE + pp * 1024);
        n++;
    }
    // weight codes: 32 rows x 32 B per instruction
    {
        const int row = wave * 32 + (lane >> 1);
        int gn = n0 + row;
        gn = gn < g.N ? gn : g.N - 1;
        const uint8_t* src = g.w + (size_t)gn * g.rb + (size_t)sb * 144 + 16 + 32 * jb + 16 * (lane & 1);
        dma16(src, st + 2 * A_PLANE + wave * 1024);
        n++;
    }
    if (jb == 0) {
        if (wave < 4) {                              // headers: 64 rows x 16 B
            int gn = n0 + wave * 64 + lane;
            gn = gn < g.N ? gn : g.N - 1;
            dma16(g.w + (size_t)gn * g.rb + (size_t)sb * 144, sbb + wave * 1024);
        } else {                                     // xs hi/lo: 64 tokens x 16 B
            const int plane = (wave - 4) >> 1, part = (wave - 4) & 1;
            int gm = m0 + part * 64 + lane;
            gm = gm < g.M ? gm : g.M - 1;
            const _Float16* src = (plane ? g.slo : g.shi) + (size_t)gm * (g.K >> 5) + sb * 8;
            dma16(src, sbb + HDR + plane * XS + part * 1024);
        }
        n++;
    }
    return n;
}

__device__ __forceinline__ void wait_dma(int outstanding) {
    // gfx9 s_waitcnt: vmcnt[3:0] | expcnt 7 << 4 | lgkmcnt 15 << 8 | vmcnt[5:4] << 14
    if (outstanding >= 6) __builtin_amdgcn_s_waitcnt(6 | (7 << 4) | (15 << 8));
    else if (outstanding == 5) __builtin_amdgcn_s_waitcnt(5 | (7 << 4) | (15 << 8));
    else __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ uint32_t pick2(uint32_t u, int a) {
    // bytes a and a+1 of u into bits 0-7 and 16-23 (others zero)
    return __builtin_amdgcn_perm(0u, u, (uint32_t)a | (4u << 8) | ((uint32_t)(a + 1) << 16) | (4u << 24));
}

// 8 codes (bytes b0..b7 in u0,u1; nibble half `hi`) -> 8 fp16 V = sc * nibble.
__device__ __forceinline__ h8 decode_v(uint32_t u0, uint32_t u1, bool hi_nib, h2 mul, h2 add) {
    const uint32_t mask = hi_nib ? 0x00f000f0u : 0x000f000fu;
    h8 out;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const uint32_t x = pick2(t < 2 ? u0 : u1, (2 * t) & 3);
        const uint32_t mg = (x & mask) | 0x64006400u;          // fp16 1024 + n (or 1024 + 16n)
        const h2 hv = __builtin_bit_cast(h2, mg);
        const h2 v = __builtin_elementwise_fma(hv, mul, add);  // (h - 1024) * scale, exact
        out[2 * t] = v[0];
        out[2 * t + 1] = v[1];
    }
    return out;
}

__global__ void __launch_bounds__(kGemmThreads)
gemm_q4k_kernel(GemmArgs g, int ntn) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 2, wn = wave & 3;
    const int tile = blockIdx.x;
    const int m0 = (tile / ntn) * BM, n0 = (tile % ntn) * BN;
    // stage buffer i at smem + i * STAGE; super-block buffer i after them
    auto stage = [&](int i) { return smem + i * STAGE; };
    auto sbuf = [&](int i) { return smem + 2 * STAGE + i * SB_STAGE; };
    const int nk = g.K / BK;

    f16v acc[2][2], main_[2][2];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int r = 0; r < 16; r++) { acc[a][b][r] = 0.0f; main_[a][b][r] = 0.0f; }

    // per super-block weight scales of this lane's two weight rows
    h2 vmul[2][8], vadd[2][8];
    h8 bmin[2];
    float dsc[2], dmn[2];

    (void)issue_kstep(g, m0, n0, 0, stage(0), sbuf(0), wave, lane);
    const int nsb = nk >> 2;
    for (int sb = 0; sb < nsb; sb++) {
        // jb unrolled so every register-array index below is a constant
#pragma unroll
        for (int jb = 0; jb < 4; jb++) {
        const int kt = 4 * sb + jb;
        int nnext = 0;
        if (kt + 1 < nk)
            nnext = issue_kstep(g, m0, n0, kt + 1, stage((jb + 1) & 1), sbuf(((kt + 1) >> 2) & 1), wave, lane);
        wait_dma(nnext);
        __builtin_amdgcn_s_barrier();
        const uint8_t* st = stage(jb & 1);
        const uint8_t* sbb = sbuf(sb & 1);
        if (jb == 0) {
            // decode the two weight rows' headers: d, dmin, 8 x (sc, m)
#pragma unroll
            for (int ct = 0; ct < 2; ct++) {
                const int row = wn * 64 + ct * 32 + (lane & 31);
                const u32x4 h = *reinterpret_cast<const u32x4*>(sbb + row * 16);
                dsc[ct] = fp16_bits_to_f32(h.x);
                dmn[ct] = fp16_bits_to_f32(h.x >> 16);
                h8 mm;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    uint32_t sc, mn;
                    if (j < 4) {
                        sc = __builtin_amdgcn_ubfe(h.y, 8 * j, 6);
                        mn = __builtin_amdgcn_ubfe(h.z, 8 * j, 6);
                    } else {
                        sc = __builtin_amdgcn_ubfe(h.w, 8 * (j - 4), 4) | (__builtin_amdgcn_ubfe(h.y, 8 * (j - 4) + 6, 2) << 4);
                        mn = __builtin_amdgcn_ubfe(h.w, 8 * (j - 4) + 4, 4) | (__builtin_amdgcn_ubfe(h.z, 8 * (j - 4) + 6, 2) << 4);
                    }
                    // even blocks use low nibbles (1024 + n), odd high (1024 + 16n)
                    const _Float16 s = (j & 1) ? (_Float16)((float)sc * 0.0625f) : (_Float16)(float)sc;
                    vmul[ct][j] = h2{s, s};
                    vadd[ct][j] = h2{(_Float16)(-1024.0f) * s, (_Float16)(-1024.0f) * s};
                    mm[j] = (_Float16)(float)mn;
                }
                // lanes 32..63 supply k = 8..15 of the K=16 min MFMA: zero
                bmin[ct] = lane < 32 ? mm : h8{0, 0, 0, 0, 0, 0, 0, 0};
            }
        }

        // four K=16 sub-steps
#pragma unroll
        for (int s = 0; s < 4; s++) {
            h8 ahi[2], alo[2];
#pragma unroll
            for (int tt = 0; tt < 2; tt++) {
                const int row = wm * 64 + tt * 32 + (lane & 31);
                const int piece = (2 * s + (lane >> 5)) ^ (row & 7);
                ahi[tt] = *reinterpret_cast<const h8*>(st + row * 128 + piece * 16);
                alo[tt] = *reinterpret_cast<const h8*>(st + A_PLANE + row * 128 + piece * 16);
            }
            const int blk = 2 * jb + (s >> 1);          // block within the super-block
            const bool hi_nib = (s >> 1) != 0;
            const int half = s & 1;
#pragma unroll
            for (int ct = 0; ct < 2; ct++) {
                const int row = wn * 64 + ct * 32 + (lane & 31);
                const uint2 u = *reinterpret_cast<const uint2*>(st + 2 * A_PLANE + row * 32 + 16 * half + 8 * (lane >> 5));
                const h8 v = decode_v(u.x, u.y, hi_nib, vmul[ct][blk], vadd[ct][blk]);
#pragma unroll
                for (int tt = 0; tt < 2; tt++) {
                    main_[tt][ct] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ahi[tt], v, main_[tt][ct], 0, 0, 0);
                    main_[tt][ct] = __builtin_amdgcn_mfma_f32_32x32x16_f16(alo[tt], v, main_[tt][ct], 0, 0, 0);
                }
            }
        }

        if (jb == 3) {
            // min term of this super-block and the per-super-block epilogue
#pragma unroll
            for (int tt = 0; tt < 2; tt++) {
                const int tok = wm * 64 + tt * 32 + (lane & 31);
                h8 shv = *reinterpret_cast<const h8*>(sbb + HDR + tok * 16);
                h8 slv = *reinterpret_cast<const h8*>(sbb + HDR + XS + tok * 16);
                if (lane >= 32) { shv = h8{0, 0, 0, 0, 0, 0, 0, 0}; slv = shv; }
#pragma unroll
                for (int ct = 0; ct < 2; ct++) {
                    f16v mn = {0};
                    mn = __builtin_amdgcn_mfma_f32_32x32x16_f16(shv, bmin[ct], mn, 0, 0, 0);
                    mn = __builtin_amdgcn_mfma_f32_32x32x16_f16(slv, bmin[ct], mn, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        acc[tt][ct][r] = fmaf(dsc[ct], main_[tt][ct][r], acc[tt][ct][r]);
                        acc[tt][ct][r] = fmaf(-dmn[ct], mn[r], acc[tt][ct][r]);
                        main_[tt][ct][r] = 0.0f;
                    }
                }
            }
        }
        // every wave is done reading this stage before it is refilled
        __builtin_amdgcn_s_waitcnt(0xc07f);           // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        }
    }

    // store: D[token][row] -> y[token * N + row] * 2^E_token
#pragma unroll
    for (int tt = 0; tt < 2; tt++)
#pragma unroll
        for (int ct = 0; ct < 2; ct++) {
            const int n = n0 + wn * 64 + ct * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + wm * 64 + tt * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < g.M && n < g.N) g.y[(size_t)m * g.N + n] = acc[tt][ct][r] * g.escale[m];
            }
        }
}

size_t gemm_planes_bytes(int M, int K) {
    const size_t up = 256;
    auto r = [&](size_t v) { return (v + up - 1) / up * up; };
    return 2 * r((size_t)M * K * 2) + 2 * r((size_t)M * (K / 32) * 2) + r((size_t)M * 4);
}

bool gemm_supported(uint32_t type, int M, int K) {
    return type == T_Q4_K && M > 8 && K % 256 == 0;
}

hipError_t launch_gemm(uint32_t type, const uint8_t* w, const ActView& A, void* planes, float* y,
                       int M, int K, int N, hipStream_t st) {
    if (!gemm_supported(type, M, K)) return hipErrorInvalidValue;
    if (M <= 0 || N <= 0) return hipSuccess;
    auto r = [](size_t v) { return (v + 255) / 256 * 256; };
    uint8_t* p = static_cast<uint8_t*>(planes);
    _Float16* hi = reinterpret_cast<_Float16*>(p);
    p += r((size_t)M * K * 2);
    _Float16* lo = reinterpret_cast<_Float16*>(p);
    p += r((size_t)M * K * 2);
    _Float16* shi = reinterpret_cast<_Float16*>(p);
    p += r((size_t)M * (K / 32) * 2);
    _Float16* slo = reinterpret_cast<_Float16*>(p);
    p += r((size_t)M * (K / 32) * 2);
    float* escale = reinterpret_cast<float*>(p);
    hipLaunchKernelGGL(gemm_prep_kernel, dim3(M), dim3(256), 0, st, A, K, hi, lo, shi, slo, escale);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    GemmArgs g{hi, lo, shi, slo, escale, w, row_bytes(type, K), y, M, N, K};
    const int ntn = (N + BN - 1) / BN, ntm = (M + BM - 1) / BM;
    hipLaunchKernelGGL(gemm_q4k_kernel, dim3(ntn * ntm), dim3(kGemmThreads), GEMM_LDS, st, g, ntn);
    return hipGetLastError();
}

}  // namespace lp
