// lp_internal.h - launchers shared between the kernel translation units and
// the C-ABI layer (lp_api.cpp). Not part of the public interface.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "lp_device.h"

namespace lp {

// Bytes of one weight row of K elements: K / epb * bpb, as the reference
// computes rb (src/matmul_simd.cpp:482). 0 for types this library does not
// decode.
inline size_t row_bytes(uint32_t type, int K) {
    switch (type) {
        case T_Q8_0: return (size_t)(K / 32) * 34;
        case T_Q4_0: return (size_t)(K / 32) * 18;
        case T_Q5_0: return (size_t)(K / 32) * 22;
        case T_Q4_K: return (size_t)(K / 256) * 144;
        case T_Q6_K: return (size_t)(K / 256) * 210;
        default: return 0;
    }
}

// Multiprocessor count of the current device (cached per device).
int device_cu_count();

// Gemma4 MoE feed-forward pieces (lp_moe_ffn.hip).
int moe_topk_max_experts();
// norms of x [T, H]; when Aq.qs is set, ein is also quantized into Aq (H % 32 == 0)
hipError_t launch_moe_norms(const float* x, int T, int H, const float* gate_scale, const float* pre_norm,
                            float eps, float* rin, float* ein, const ActView& Aq, hipStream_t st);
// Both norms, the expert input's quantization and the F32 router products in
// one launch for 1..4 tokens (moe_norm_router_supported); logits equal to
// launch_moe_norms + the F32 router GEMV bit for bit.
bool moe_norm_router_supported(int T, int H, uint32_t router_type, const void* router, const void* gate_scale,
                               const void* pre_norm);
hipError_t launch_moe_norm_router(const float* x, int T, int H, const float* gate_scale, const float* pre_norm,
                                  float eps, const float* router, int n_exp, float* logits, float* ein,
                                  const ActView& Aq, hipStream_t st);
// Top-k and the route table in one launch (up to 16 tokens; preferred for
// T <= 4: moe_topk_route_supported).
bool moe_topk_route_supported(int T);
hipError_t launch_moe_topk_route(const float* logits, int T, int n_exp, int top_k, int* idx, float* wts,
                                 void* route, int gsize, hipStream_t st);
hipError_t launch_moe_topk(const float* logits, int T, int n_exp, int top_k, int* idx, float* wts,
                           hipStream_t st);
// hidden [P, inter]; when Aq.qs is set, also quantized into Aq (inter % 32 == 0)
hipError_t launch_geglu(const float* gu, int P, int inter, float* hidden, const ActView& Aq, hipStream_t st);
hipError_t launch_moe_combine(const float* eo, const int* idx, const float* wts, const float* down_scale, int T,
                              int top_k, int H, float* out, hipStream_t st);

// Types the reference's int8 back-end leaves to its scalar fp32 path (F32,
// F16, BF16, Q5_0, Q2_K, Q3_K, Q5_K): GEMV with fp32 activations (lp_dequant.hip).
bool fact_type(uint32_t type);
// Q5_0 with int8 activations (lp_dequant.hip)
hipError_t launch_gemv_q50(const uint8_t* w, const ActView& A, float* y, int M, int K, int N, hipStream_t st);
size_t fact_row_bytes(uint32_t type, int K);
hipError_t launch_gemv_fact(uint32_t type, const uint8_t* w, const float* x, float* y, int M, int K, int N,
                            hipStream_t st);

hipError_t launch_quantize(const float* x, int M, int K, const ActView& A, hipStream_t st);
hipError_t launch_gemv(uint32_t type, const uint8_t* w, const ActView& A, float* y, int M, int K,
                       int N, hipStream_t st);
// The kernel launch_gemv picks for these operands (routing probe).
const char* gemv_route_name(uint32_t type, int M, int K, int N, const uint8_t* w);
// Single-launch quantize + GEMV from fp32 x (M == 1, Q4_K): the workgroups
// quantize x themselves, bit-identically to launch_quantize.
bool gemv_fused_supported(uint32_t type, int M, int K, const uint8_t* w);
hipError_t launch_gemv_fused(uint32_t type, const uint8_t* w, const float* x, float* y, int M, int K,
                             int N, hipStream_t st);
// Q4_K weight matrices of one multi-matrix GEMV launch (same K, same
// activation row): matrix i is n[i] rows at w[i], output y[i], and owns the
// row groups [gstart[i], gstart[i+1]) of the launch (gstart[count..] = total).
constexpr int kBatchMax = 4;
struct SbBatch {
    const uint8_t* w[kBatchMax];
    float* y[kBatchMax];
    int n[kBatchMax];
    int gstart[kBatchMax + 1];
    int count;
};
// One launch of quantize + Q4_K GEMV over count <= kBatchMax matrices sharing x
// (each supported by gemv_fused_supported).
hipError_t launch_gemv_fused_batch(const uint8_t* const* w, float* const* y, const int* n, int count,
                                   const float* x, int K, hipStream_t st);
// Q4_K products for M >= 2 activation rows (lp_gemm.hip), on the fp16
// "planes" of the activations (gemm_planes_bytes(M, K) bytes of scratch):
// M <= 16 on the small-M MFMA kernel, larger M on the tiled GEMM.
bool gemm_supported(uint32_t type, int M, int K);
// Small M on int8 MFMA straight from the quantized blocks (no planes):
// Q4_K and Q6_K for 5 <= M <= 16 (Q4_K from M = 3 when N < 32 x CUs and K >= 14336),
// Q8_0 for 9 <= M <= 16.
bool i8mf_supported(uint32_t type, int M, int K, int N, const uint8_t* w);
// Q8_0 / Q6_K rows beyond 16 in chunks of i8_chunk_rows() on the int8 MFMA
// kernels with several token tiles per workgroup (lp_gemm.hip).
bool i8_chunk_supported(uint32_t type, int K, int N, const uint8_t* w);
int i8_chunk_rows();
hipError_t launch_i8_chunk(uint32_t type, const uint8_t* w, const ActView& A, float* y, int M, int K, int N,
                            hipStream_t st);
hipError_t launch_gemv_i8mf(uint32_t type, const uint8_t* w, const ActView& A, float* y, int M, int K, int N,
                            hipStream_t st);
// Q4_K for 1 <= M <= 8 on 4x4 int8 MFMA blocks, a row quad per wave
// (lp_rq.hip); K <= 4096. rq_preferred: the shapes where it is the fastest
// kernel.
bool rq_supported(uint32_t type, int M, int K, int N, const uint8_t* w);
bool rq_preferred(uint32_t type, int M, int K, int N, const uint8_t* w);
hipError_t launch_gemv_rq(const uint8_t* w, const ActView& A, float* y, int M, int K, int N, hipStream_t st);

// Q6_K GEMV for 1 <= M <= 8 on 4x4x4 int8 MFMA blocks (lp_q6rq.hip), any K.
bool q6rq_supported(uint32_t type, int M, int K, int N, const uint8_t* w);
bool q6rq_preferred(uint32_t type, int M, int K, int N, const uint8_t* w);
hipError_t launch_gemv_q6rq(const uint8_t* w, const ActView& A, float* y, int M, int K, int N, hipStream_t st);
size_t gemm_planes_bytes(int M, int K);
// Fragment-order planes and the prefill GEMM on them (lp_gemm_fr.hip);
// launch_planes_from_x / launch_gemm_planes / launch_gemm take this route
// where gemm_fr_preferred says so.
size_t gemm_fr_planes_bytes(int M, int K);
// Int8-MFMA prefill GEMM from the quantized blocks (lp_gemm_i8.hip): its
// scale planes take gemm_i8_planes_bytes of the planes area; launch_gemm
// takes this route where gemm_i8_preferred says so.
size_t gemm_i8_planes_bytes(int M, int K);
bool gemm_i8_supported(uint32_t type, int M, int K);
bool gemm_i8_preferred(uint32_t type, int M, int K, int N);
// Prefill GEMM kernel family (0 by shape, 1 split-precision, 2 fragment-order, 3 int8, 4/5 wide-token 128/256-token tiles).
void set_gemm_kernel(int k);
hipError_t launch_gemm_i8(const uint8_t* w, const ActView& A, void* planes, float* y, int M, int K, int N,
                          hipStream_t st);
bool gemm_fr_supported(uint32_t type, int M, int K);
hipError_t launch_fr_planes(const float* x, const ActView& A, void* planes, int M, int K, hipStream_t st);
// MFMA throughput probe (lp_mfma_probe_dev): grid x 512 threads, `out` grid*512 floats.
hipError_t launch_mfma_probe(int kind, int rnd_ops, int iters, int grid, float* out, hipStream_t st);
hipError_t launch_fr_gemm(const uint8_t* w, void* planes, float* y, int M, int K, int N, hipStream_t st);
hipError_t launch_wt_gemm(const uint8_t* w, void* planes, float* y, int M, int K, int N, hipStream_t st, int cfg);
// Wide-token GEMM configuration by shape: 1 (256 x 256 tiles, two waves per
// SIMD), 0 (128 x 256 tiles, one wave per SIMD), or -1 (too few tiles for
// either to fill the CUs).
int wt_auto_cfg(int M, int K, int N);
// planes from fp32 x (quantize + planes in one pass); with y given, also the
// zeroing of y that the product below needs at some shapes, which then runs
// with y_zeroed = true
hipError_t launch_planes_from_x(const float* x, void* planes, int M, int K, hipStream_t st, int N,
                                float* y = nullptr);
hipError_t launch_gemm_planes(uint32_t type, const uint8_t* w, void* planes, float* y, int M, int K, int N,
                              hipStream_t st, bool y_zeroed = false);
// planes from quantized activations A, then the product
hipError_t launch_gemm(uint32_t type, const uint8_t* w, const ActView& A, void* planes, float* y,
                       int M, int K, int N, hipStream_t st);
// grouped MoE on the int8 small-M MFMA kernel (groups of <= 16 pairs) from
// the quantized activation rows A; route from launch_moe_route with group
// size 16.
bool moe_mf_supported(uint32_t type, int K);
hipError_t launch_moe_i8mf(const uint8_t* w, const ActView& A, const void* route, int max_groups, int multi,
                           int topk, float* y, int K, int N, hipStream_t st);
// Grouped MoE dispatch (lp_gemv.hip). P = T * topk pairs, E experts stacked
// in w (E x N rows). `route` is scratch of moe_route_bytes(P, E) bytes.
// gsize: pairs per group (the group is the activation-row count of one
// workgroup): 16 for the 16x16 int8 MFMA kernel (Q4_K), 8 for the row-quad
// kernel (Q4_K, rq_moe_supported), 4 for the GEMV kernels (any type; Q4_K on
// the row-quad kernel where supported).
constexpr int kMoeMaxExperts = 8192;
constexpr int kRqMoeGroup = 8;
int moe_max_groups(int P, int E);
size_t moe_route_bytes(int P, int E);
hipError_t launch_moe_grouped(uint32_t type, const uint8_t* w, const ActView& A, int gsize,
                              int rows, const int* idx, int P, int E, int multi, int topk, void* route,
                              float* y, int K, int N, hipStream_t st);
// The two halves of launch_moe_grouped: the route table of the pairs (groups
// of <= gsize pairs), and the grouped products on a route table built for the
// same pairs and group size.
hipError_t launch_moe_route(const int* idx, int P, int E, void* route, int gsize, hipStream_t st);
// launch_quantize(x, rows, K, A) and launch_moe_route(idx, P, E, route, gsize)
// in one launch
hipError_t launch_moe_quant_route(const float* x, int rows, int K, const ActView& A, const int* idx, int P, int E,
                                  void* route, int gsize, hipStream_t st);
// gu (the MoE layer's down pass): the activations are GeGLU of the pairs'
// gate|up rows (2 K floats each), quantized while the GEMV stages them, where
// moe_geglu_fusable says the kernel for (type, K, gsize, w) does that.
hipError_t launch_moe_grouped_routed(uint32_t type, const uint8_t* w, const ActView& A, int gsize,
                                     int rows, int P, int E, int multi, int topk, const void* route, float* y,
                                     int K, int N, hipStream_t st, const float* gu = nullptr);
bool moe_geglu_fusable(uint32_t type, int K, int gsize, const uint8_t* w);
// Q4_K MoE groups of <= 8 pairs on the row-quad kernel (lp_rq.hip)
bool rq_moe_supported(uint32_t type, int K);
hipError_t launch_moe_rq(const uint8_t* w, const ActView& A, const void* route, int max_groups, int gsize,
                         int multi, int topk, float* y, int K, int N, hipStream_t st, const float* gu = nullptr);
// dequantize (lp_dequant.hip): elements per block (0 = type not handled)
// and source bytes of n elements.
int dequant_block_elems(uint32_t type);
size_t dequant_src_bytes(uint32_t type, long n);
hipError_t launch_dequant(uint32_t type, const uint8_t* w, float* dst, long n, hipStream_t st);
// Byte copy by a kernel (bytes, dst and src multiples of 4): small transfers
// to and from device-mapped pinned host memory.
hipError_t launch_copy(void* dst, const void* src, size_t bytes, hipStream_t st);
// streaming-read probe (measurement): unroll in {1, 4, 9}
hipError_t launch_read_probe(const void* buf, size_t bytes, int grid, int block, int unroll, uint32_t* sink,
                             hipStream_t st);
hipError_t launch_block_sums(uint32_t type, const uint8_t* w, const ActView& A, int32_t* out,
                             int M, int K, int N, hipStream_t st);

}  // namespace lp
