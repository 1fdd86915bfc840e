// lp_moe_ffn.hip - the element-wise and per-token parts of the Gemma4 MoE
// feed-forward (src/arch_gemma4.cpp:507-641) around the grouped expert GEMVs:
// router input and expert input norms, softmax + top-k + renormalisation,
// GeGLU, and the weighted combine with the per-expert down scales.
#include <hip/hip_runtime.h>

#include "lp_chunks.h"
#include "lp_internal.h"
#include "lp_route.h"

namespace lp {

namespace {

// Sum over a workgroup of 256 threads (fixed order: wave partials by
// butterfly, then the 4 wave sums in index order).
__device__ __forceinline__ float block_sum256(float v, float* red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// The 8 threads of a 32-element block quantize it as quantize_act_kernel does
// (same arithmetic, same stores).
__device__ __forceinline__ void store_q8_block(const ActView& A, long m, int K, int i4, float4 v) {
    const Q8Group q = quant_group8(v);
    *reinterpret_cast<uint32_t*>(A.qs + m * K + 4 * i4) = q.packed;
    if ((i4 & 7) == 0) {
        const long blk = m * (K >> 5) + (i4 >> 3);
        A.d[blk] = q.d;
        A.sum[blk] = q.sum;
        A.s16[blk] = q.s16;
    }
}

// Per token t (one workgroup): ms = sum x^2, inv = 1 / sqrt(ms / H + eps);
//   router input  r[i] = (x[i] * inv) * (gate_scale[i] * inv_sqrt_h)
//     (rmsnorm_no_scale, src/arch_gemma4.cpp:24-29, then :540-541)
//   expert input  e[i] = x[i] * inv * pre_norm[i]   (ops::rmsnorm, src/ops.cpp:35-74)
// Both norms of the reference sum the same squares in the same order, so
// they share inv.
__global__ void __launch_bounds__(256)
moe_norms_kernel(const float* __restrict__ x, int H, const float* __restrict__ gate_scale,
                 const float* __restrict__ pre_norm, float inv_sqrt_h, float eps, float* __restrict__ rin,
                 float* __restrict__ ein, ActView Aq) {
#pragma clang fp contract(off)
    __shared__ float red[4];
    const float* xr = x + (size_t)blockIdx.x * H;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < H; i += 256) ss += xr[i] * xr[i];
    const float ms = block_sum256(ss, red);
    const float inv = 1.0f / sqrtf(ms / (float)H + eps);
    float* rr = rin + (size_t)blockIdx.x * H;
    float* er = ein + (size_t)blockIdx.x * H;
    if (Aq.qs) {
        // float4 per thread; H % 32 == 0, so a block's 8 threads are all in or all out
        for (int i4 = threadIdx.x; i4 < (H >> 2); i4 += 256) {
            const float4 xv = reinterpret_cast<const float4*>(xr)[i4];
            const float4 gs = reinterpret_cast<const float4*>(gate_scale)[i4];
            const float4 pn = reinterpret_cast<const float4*>(pre_norm)[i4];
            const float v0 = xv.x * inv, v1 = xv.y * inv, v2 = xv.z * inv, v3 = xv.w * inv;
            reinterpret_cast<float4*>(rr)[i4] = make_float4(v0 * (gs.x * inv_sqrt_h), v1 * (gs.y * inv_sqrt_h),
                                                            v2 * (gs.z * inv_sqrt_h), v3 * (gs.w * inv_sqrt_h));
            const float4 e = make_float4(v0 * pn.x, v1 * pn.y, v2 * pn.z, v3 * pn.w);
            reinterpret_cast<float4*>(er)[i4] = e;
            store_q8_block(Aq, blockIdx.x, H, i4, e);
        }
    } else {
        for (int i = threadIdx.x; i < H; i += 256) {
            const float v = xr[i] * inv;
            rr[i] = v * (gate_scale[i] * inv_sqrt_h);
            er[i] = v * pre_norm[i];
        }
    }
}

// A few tokens (MR <= 4) with an F32 router: the two norms and the router
// products in one launch. Every workgroup recomputes each token's inv from x
// (the same sum in the same order as moe_norms_kernel), quantizes its slice
// of the expert input (32-element blocks, 8 threads each), and its waves take
// router rows as gemv_dense_kernel<F32, MR> does (lane: 8 consecutive
// elements of each 512-element slab, 8 slabs in flight, then the wave sum),
// with the router input r[i] = (x[i] * inv) * (gate_scale[i] * inv_sqrt_h)
// formed on the fly: logits bit-identical to the two-kernel path.
template <int MR>
__global__ void __launch_bounds__(256)
moe_norm_router_kernel(const float* __restrict__ x, int H, const float* __restrict__ gate_scale,
                       const float* __restrict__ pre_norm, float inv_sqrt_h, float eps,
                       const float* __restrict__ router, int n_exp, float* __restrict__ logits,
                       float* __restrict__ ein, ActView Aq) {
#pragma clang fp contract(off)
    __shared__ float red[4];
    float inv[MR];
#pragma unroll
    for (int t = 0; t < MR; t++) {
        const float* xr = x + (size_t)t * H;
        float ss = 0.0f;
        for (int i = threadIdx.x; i < H; i += 256) ss += xr[i] * xr[i];
        const float ms = block_sum256(ss, red);
        inv[t] = 1.0f / sqrtf(ms / (float)H + eps);
    }
    // this workgroup's share of the expert input (whole 32-element blocks)
    const int h4 = H >> 2;
    for (int i4 = blockIdx.x * 256 + threadIdx.x; i4 < MR * h4; i4 += gridDim.x * 256) {
        const int t = i4 / h4, c4 = i4 - t * h4;
        float it = inv[0];
#pragma unroll
        for (int u = 1; u < MR; u++) it = t == u ? inv[u] : it;
        const float4 xv = reinterpret_cast<const float4*>(x + (size_t)t * H)[c4];
        const float4 pn = reinterpret_cast<const float4*>(pre_norm)[c4];
        const float4 e = make_float4((xv.x * it) * pn.x, (xv.y * it) * pn.y, (xv.z * it) * pn.z,
                                     (xv.w * it) * pn.w);
        reinterpret_cast<float4*>(ein + (size_t)t * H)[c4] = e;
        store_q8_block(Aq, t, H, c4, e);
    }
    // router rows, one per wave
    const int lane = threadIdx.x & 63;
    const int row = (blockIdx.x * 256 + threadIdx.x) >> 6;
    if (row >= n_exp) return;
    const float* wr = router + (size_t)row * H;
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; m++) acc[m] = 0.0f;
    constexpr int U = 8;
    for (int e0 = 8 * lane; e0 < H; e0 += U * 512) {
        float wv[U][8];
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (e0 + 512 * u < H) {
                const float4 a = reinterpret_cast<const float4*>(wr + e0 + 512 * u)[0];
                const float4 b = reinterpret_cast<const float4*>(wr + e0 + 512 * u)[1];
                wv[u][0] = a.x; wv[u][1] = a.y; wv[u][2] = a.z; wv[u][3] = a.w;
                wv[u][4] = b.x; wv[u][5] = b.y; wv[u][6] = b.z; wv[u][7] = b.w;
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int e = e0 + 512 * u;
            if (e < H) {
                const float4 g0 = reinterpret_cast<const float4*>(gate_scale + e)[0];
                const float4 g1 = reinterpret_cast<const float4*>(gate_scale + e)[1];
                const float gs[8] = {g0.x * inv_sqrt_h, g0.y * inv_sqrt_h, g0.z * inv_sqrt_h, g0.w * inv_sqrt_h,
                                     g1.x * inv_sqrt_h, g1.y * inv_sqrt_h, g1.z * inv_sqrt_h, g1.w * inv_sqrt_h};
#pragma unroll
                for (int m = 0; m < MR; m++) {
                    const float4 a = reinterpret_cast<const float4*>(x + (size_t)m * H + e)[0];
                    const float4 b = reinterpret_cast<const float4*>(x + (size_t)m * H + e)[1];
                    const float xv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
                    float t = acc[m];
#pragma unroll
                    for (int j = 0; j < 8; j++) t = fmaf((xv[j] * inv[m]) * gs[j], wv[u][j], t);
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
        if (lane == 0) logits[(size_t)m * n_exp + row] = s2;
    }
}

// Wave-wide reductions with DPP lane moves (the pattern of group_sum: the
// result lands in lane 63, read back as a wave-uniform value). A lane with no
// source in a step keeps its own value, the identity of max / arg-max.
template <int CTRL, int ROWMASK>
__device__ __forceinline__ float dpp_max_step(float v) {
    const int b = __builtin_bit_cast(int, v);
    return fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(b, b, CTRL, ROWMASK, 0xf, false)));
}
__device__ __forceinline__ float wave_max(float v) {
    v = dpp_max_step<0xb1, 0xf>(v);
    v = dpp_max_step<0x4e, 0xf>(v);
    v = dpp_max_step<0x114, 0xf>(v);
    v = dpp_max_step<0x118, 0xf>(v);
    v = dpp_max_step<0x142, 0xa>(v);
    v = dpp_max_step<0x143, 0xc>(v);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
// Arg-max over the wave of 64-bit keys (order-preserving bits of the value
// above the complemented index: the larger value wins, the lower index on
// equal values), one compare and two selects per step. A lane with no source
// in a step keeps its own key.
template <int CTRL, int ROWMASK>
__device__ __forceinline__ void dpp_kmax_step(uint64_t& k) {
    const int lo = (int)(uint32_t)k, hi = (int)(uint32_t)(k >> 32);
    const uint32_t olo = (uint32_t)__builtin_amdgcn_update_dpp(lo, lo, CTRL, ROWMASK, 0xf, false);
    const uint32_t ohi = (uint32_t)__builtin_amdgcn_update_dpp(hi, hi, CTRL, ROWMASK, 0xf, false);
    const uint64_t o = ((uint64_t)ohi << 32) | olo;
    k = o > k ? o : k;
}
__device__ __forceinline__ uint64_t wave_kmax(uint64_t k) {
    dpp_kmax_step<0xb1, 0xf>(k);
    dpp_kmax_step<0x4e, 0xf>(k);
    dpp_kmax_step<0x114, 0xf>(k);
    dpp_kmax_step<0x118, 0xf>(k);
    dpp_kmax_step<0x142, 0xa>(k);
    dpp_kmax_step<0x143, 0xc>(k);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)k, 63);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(k >> 32), 63);
    return ((uint64_t)hi << 32) | lo;
}
// Key of candidate (v, e): the float's bits mapped so unsigned order is
// numeric order (v + 0.0f first: -0 and +0 compare equal, as in the float
// scan), then ~e; 0 for no candidate (NaN, or no expert), below every key.
__device__ __forceinline__ uint64_t topk_key(float v, int e) {
    v = v + 0.0f;
    const uint32_t b = __builtin_bit_cast(uint32_t, v);
    const uint32_t m = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return v != v ? 0ull : ((uint64_t)m << 32) | (uint32_t)~e;
}
__device__ __forceinline__ float key_value(uint64_t k) {
    const uint32_t m = (uint32_t)(k >> 32);
    return __builtin_bit_cast(float, (m & 0x80000000u) ? (m & 0x7fffffffu) : ~m);
}

// Per token (one wave): softmax over the n_exp router logits, top-k by
// repeated arg-max (the lower index wins a tie, as the reference's strict
// '>' scan; a pick is then set to -1e30 as the reference does), and the k
// weights divided by their sum (src/arch_gemma4.cpp:546-563). The sum of
// exponentials is a wave reduction (reassociated against the reference's
// loop); the k-weight sum runs in pick order. n_exp <= 64 * PER (PER
// logits per lane, the smallest power of two that holds them, up to
// kTopkPer).
constexpr int kTopkPer = 16;

// Token t's top-k by one wave (lane = its lane); the picks also go to
// lidx (LDS) when given.
template <int PER>
__device__ __forceinline__ void topk_token(const float* __restrict__ logits, int t, int n_exp, int top_k,
                                           int* __restrict__ idx, float* __restrict__ wts, int* lidx) {
    const int lane = threadIdx.x & 63;
    const float* l = logits + (size_t)t * n_exp;
    float v[PER];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int e = lane + 64 * j;
        v[j] = e < n_exp ? l[e] : -INFINITY;
        mx = fmaxf(mx, v[j]);
    }
    mx = wave_max(mx);
    float sm = 0.0f;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        v[j] = lane + 64 * j < n_exp ? expf(v[j] - mx) : 0.0f;
        sm += v[j];
    }
    sm = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, group_sum(sm, 64)), 63));
#pragma unroll
    for (int j = 0; j < PER; j++) v[j] = lane + 64 * j < n_exp ? v[j] / sm : -INFINITY;
    float mine = 0.0f;
    int mine_i = 0;
    for (int k = 0; k < top_k; k++) {     // top_k <= 16 (the reference's top_idx[16])
        uint64_t key = 0;
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const int e = lane + 64 * j;
            const uint64_t kj = e < n_exp ? topk_key(v[j], e) : 0ull;
            key = kj > key ? kj : key;
        }
        key = wave_kmax(key);
        // The reference's scan starts at best = 0 and moves only on a strict
        // '>', so a NaN held by expert 0 is never beaten, and NaNs elsewhere
        // never win (they carry key 0 here). A NaN or +inf logit makes every
        // probability NaN, and the reference then picks expert 0 for every k
        // (its -1e30 after the first pick still beats the NaNs).
        const float v0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v[0]), 0));
        const bool take0 = v0 != v0 || key == 0ull;
        const float bv = take0 ? v0 : key_value(key);
        const int bi = take0 ? 0 : (int)~(uint32_t)key;
        if (lane == k) {
            mine = bv;
            mine_i = bi;
        }
        if ((bi & 63) == lane) {
#pragma unroll
            for (int j = 0; j < PER; j++)
                if (lane + 64 * j == bi) v[j] = -1e30f;
        }
    }
    float wsum = 0.0f;
    for (int k = 0; k < top_k; k++)
        wsum += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mine), k));
    if (lane < top_k) {
        idx[(size_t)t * top_k + lane] = mine_i;
        wts[(size_t)t * top_k + lane] = mine / wsum;
        if (lidx) lidx[t * top_k + lane] = mine_i;
    }
}

template <int PER>
__global__ void __launch_bounds__(64)
moe_topk_kernel(const float* __restrict__ logits, int n_exp, int top_k, int* __restrict__ idx,
                float* __restrict__ wts) {
    topk_token<PER>(logits, blockIdx.x, n_exp, top_k, idx, wts, nullptr);
}

// A few tokens (T <= 4): one workgroup does every token's top-k (a wave
// each) and then its first wave builds the route table of the grouped expert
// passes from the picks in LDS: one launch instead of two.
template <int PER>
__global__ void __launch_bounds__(1024)
moe_topk_route_kernel(const float* __restrict__ logits, int T, int n_exp, int top_k, int* __restrict__ idx,
                      float* __restrict__ wts, uint8_t* __restrict__ route, int max_groups, int gsize) {
    extern __shared__ int tsm[];
    int* lidx = tsm;                                   // T * top_k picks
    const int wave = threadIdx.x >> 6;
    if (wave < T) topk_token<PER>(logits, wave, n_exp, top_k, idx, wts, lidx);
    __syncthreads();
    // one wave up to 16 pairs; the workgroup's scans beyond (measured, us per
    // layer at 128 experts, top-8: T=1 32.3 -> 30.9, T=2 36.5 -> 35.4 with
    // one wave; T=4 46.7 -> 47.6)
    const int P = T * top_k;
    if (P <= 16) {
        if (wave == 0) build_route_wave(lidx, P, n_exp, route, max_groups, gsize);
    } else {
        build_route(lidx, P, n_exp, route, max_groups, gsize, tsm + ((P + 3) & ~3));
    }
}

// hidden[p][i] = gelu_tanh(gate[p][i]) * up[p][i], gate|up = gu row p
// (gelu_tanh_mul)
__global__ void __launch_bounds__(256)
geglu_kernel(const float* __restrict__ gu, int inter, long n, float* __restrict__ hidden) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const long p = i / inter, c = i - p * inter;
    hidden[i] = gelu_tanh_mul(gu[p * 2 * inter + c], gu[p * 2 * inter + inter + c]);
}

// The same, four outputs per thread, and each 32-element block quantized
// (inter % 32 == 0).
__global__ void __launch_bounds__(256)
geglu_q_kernel(const float* __restrict__ gu, int inter, long n4, float* __restrict__ hidden, ActView Aq) {
    const long i4 = (long)blockIdx.x * 256 + threadIdx.x;
    if (i4 >= n4) return;                                // n4 % 8 == 0: whole blocks
    const int q4 = inter >> 2;
    const long p = i4 / q4, c4 = i4 - p * q4;
    const float4 g = reinterpret_cast<const float4*>(gu + p * 2 * inter)[c4];
    const float4 u = reinterpret_cast<const float4*>(gu + p * 2 * inter + inter)[c4];
    const float4 h = make_float4(gelu_tanh_mul(g.x, u.x), gelu_tanh_mul(g.y, u.y), gelu_tanh_mul(g.z, u.z),
                                 gelu_tanh_mul(g.w, u.w));
    reinterpret_cast<float4*>(hidden)[i4] = h;
    store_q8_block(Aq, p, inter, (int)c4, h);
}

// out[t][i] = sum_k (w[t,k] * down_scale[idx[t,k]]) * eo[t*k_ + k][i], k in
// order from 0 (src/arch_gemma4.cpp:632-639).
__global__ void __launch_bounds__(256)
moe_combine_kernel(const float* __restrict__ eo, const int* __restrict__ idx, const float* __restrict__ wts,
                   const float* __restrict__ down_scale, int top_k, int H, float* __restrict__ out) {
    const int t = blockIdx.y;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= H) return;
    float acc = 0.0f;
    for (int k = 0; k < top_k; k++) {
        const float wgt = wts[(size_t)t * top_k + k] * down_scale[idx[(size_t)t * top_k + k]];
        acc = fmaf(wgt, eo[((size_t)t * top_k + k) * H + i], acc);
    }
    out[(size_t)t * H + i] = acc;
}

}  // namespace

int moe_topk_max_experts() { return 64 * kTopkPer; }

// logits per lane of the top-k wave
static int topk_per(int n_exp) {
    int per = 1;
    while (64 * per < n_exp) per <<= 1;
    return per;
}

hipError_t launch_moe_norms(const float* x, int T, int H, const float* gate_scale, const float* pre_norm,
                            float eps, float* rin, float* ein, const ActView& Aq, hipStream_t st) {
    if (T <= 0) return hipSuccess;
    if (Aq.qs && H % 32 != 0) return hipErrorInvalidValue;
    const float inv_sqrt_h = 1.0f / sqrtf((float)H);
    hipLaunchKernelGGL(moe_norms_kernel, dim3(T), dim3(256), 0, st, x, H, gate_scale, pre_norm, inv_sqrt_h, eps,
                       rin, ein, Aq);
    return hipGetLastError();
}

bool moe_norm_router_supported(int T, int H, uint32_t router_type, const void* router, const void* gate_scale,
                               const void* pre_norm) {
    return T >= 1 && T <= 4 && router_type == T_F32 && H % 32 == 0 &&
           reinterpret_cast<uintptr_t>(router) % 16 == 0 && reinterpret_cast<uintptr_t>(gate_scale) % 16 == 0 &&
           reinterpret_cast<uintptr_t>(pre_norm) % 16 == 0;
}

hipError_t launch_moe_norm_router(const float* x, int T, int H, const float* gate_scale, const float* pre_norm,
                                  float eps, const float* router, int n_exp, float* logits, float* ein,
                                  const ActView& Aq, hipStream_t st) {
    if (T < 1 || T > 4 || H % 32 != 0 || !Aq.qs) return hipErrorInvalidValue;
    const float inv_sqrt_h = 1.0f / sqrtf((float)H);
    const dim3 grid((unsigned)((n_exp + 3) / 4));
#define LP_NR(MRV) hipLaunchKernelGGL(moe_norm_router_kernel<MRV>, grid, dim3(256), 0, st, x, H, gate_scale, pre_norm, \
                                      inv_sqrt_h, eps, router, n_exp, logits, ein, Aq)
    switch (T) {
        case 1: LP_NR(1); break;
        case 2: LP_NR(2); break;
        case 3: LP_NR(3); break;
        default: LP_NR(4); break;
    }
#undef LP_NR
    return hipGetLastError();
}

hipError_t launch_moe_topk(const float* logits, int T, int n_exp, int top_k, int* idx, float* wts,
                           hipStream_t st) {
    if (T <= 0) return hipSuccess;
#define LP_TK(PV) hipLaunchKernelGGL(moe_topk_kernel<PV>, dim3(T), dim3(64), 0, st, logits, n_exp, top_k, idx, wts)
    switch (topk_per(n_exp)) {
        case 1: LP_TK(1); break;
        case 2: LP_TK(2); break;
        case 4: LP_TK(4); break;
        case 8: LP_TK(8); break;
        default: LP_TK(16); break;
    }
#undef LP_TK
    return hipGetLastError();
}

// measured at 128 experts, top-8 (us per layer, separate kernels vs one):
// T=1 37.4 / 36.9, T=4 51.5 / 50.2, T=16 85.3 / 89.0 (one wave per token
// on one CU loses to a workgroup per token)
bool moe_topk_route_supported(int T) { return T >= 1 && T <= 4; }

hipError_t launch_moe_topk_route(const float* logits, int T, int n_exp, int top_k, int* idx, float* wts,
                                 void* route, int gsize, hipStream_t st) {
    // one wave per token (at most 64 pairs)
    if (T < 1 || top_k < 1 || T * top_k > 64 || n_exp > kMoeMaxExperts || gsize < 4) return hipErrorInvalidValue;
    const int P = T * top_k;
    const int mg = moe_max_groups(P, n_exp);
    const size_t shm = sizeof(int) * ((size_t)((P + 3) & ~3) + (P <= 16 ? 0 : 3 * (size_t)n_exp + 2 * 16));
#define LP_TKR(PV) hipLaunchKernelGGL(moe_topk_route_kernel<PV>, dim3(1), dim3(64 * T), shm, st, logits, T, n_exp, \
                                      top_k, idx, wts, static_cast<uint8_t*>(route), mg, gsize)
    switch (topk_per(n_exp)) {
        case 1: LP_TKR(1); break;
        case 2: LP_TKR(2); break;
        case 4: LP_TKR(4); break;
        case 8: LP_TKR(8); break;
        default: LP_TKR(16); break;
    }
#undef LP_TKR
    return hipGetLastError();
}

hipError_t launch_geglu(const float* gu, int P, int inter, float* hidden, const ActView& Aq, hipStream_t st) {
    const long n = (long)P * inter;
    if (n <= 0) return hipSuccess;
    if (Aq.qs) {
        if (inter % 32 != 0) return hipErrorInvalidValue;
        const long n4 = n / 4;
        hipLaunchKernelGGL(geglu_q_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st, gu, inter, n4,
                           hidden, Aq);
    } else {
        hipLaunchKernelGGL(geglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, gu, inter, n, hidden);
    }
    return hipGetLastError();
}

hipError_t launch_moe_combine(const float* eo, const int* idx, const float* wts, const float* down_scale, int T,
                              int top_k, int H, float* out, hipStream_t st) {
    if (T <= 0) return hipSuccess;
    hipLaunchKernelGGL(moe_combine_kernel, dim3((H + 255) / 256, T), dim3(256), 0, st, eo, idx, wts, down_scale,
                       top_k, H, out);
    return hipGetLastError();
}

}  // namespace lp
