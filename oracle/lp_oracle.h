/*
 * lp_oracle.h - CPU restatement of Laplace's GGUF quantized-matmul arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP product
 * path: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it. Nothing in laplace_amd/ links or calls it.
 *
 * Two arithmetics are restated, each function citing the reference lines it
 * follows (paths are relative to the Laplace source tree):
 *
 *   1. The int8-activation path of src/matmul_simd.cpp (the parity oracle):
 *      ActQ8 activation quantizer (:348-410), per-type integer block dots and
 *      fp32 block-scale epilogue (:143-342), gemm_int row loop (:432-455),
 *      MoE GEMVs (:506-544). The NEON lane structure (4 int32 lanes per
 *      16-element dot, lane-wise fused multiply-add, pairwise final sum) is
 *      emulated so the fp32 results follow the reference's rounding as far as
 *      it is determined by the source (see lp_oracle.c for the one place where
 *      floating-point contraction had to be assumed).
 *
 *   2. The portable scalar fp32 path of src/matmul.cpp (the CPU throughput
 *      baseline): dot_row_* (:63-314), gemm_scalar with ThreadPool's static
 *      contiguous chunking (:320-334, src/threadpool.h:229-258,:310-320),
 *      dequantize (:504-675).
 *
 * Activation blocks are returned structure-of-arrays: per 32-element block
 * b of row m, d[m*nb+b], sum[m*nb+b], sum_lo/sum_hi[m*nb+b] and
 * qs[m*K + 32*b + l]. The values equal the fields of the reference's ActQ8
 * struct (src/matmul_simd.cpp:26-32).
 *
 * Parity pins (each checked in tests/test_oracle.py): fp16 known answers and
 * an exhaustive comparison against the reference's own fp16.h; block layouts
 * against the reference's independent GGUF dequantizers (tests/quant_ref.h)
 * built into oracle/_ref; integer block sums against one-hot probes and the
 * fp64 product of those dequantized rows; the quantizer against closed-form
 * invariants and round-half-even ties; committed golden fixtures.
 * The fp32 rounding of the NEON path as executed on Apple hardware is pinned
 * only by tolerance (1e-4), as the reference path cannot run on x86.
 */
#ifndef LP_ORACLE_H
#define LP_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGMLType values (src/tensor.h:11-34). */
enum {
    OR_F32 = 0, OR_F16 = 1, OR_Q4_0 = 2, OR_Q5_0 = 6, OR_Q8_0 = 8,
    OR_Q2_K = 10, OR_Q3_K = 11, OR_Q4_K = 12, OR_Q5_K = 13, OR_Q6_K = 14,
    OR_BF16 = 30
};

size_t or_bytes_per_block(int type);    /* src/tensor.h:41-67 */
int    or_elements_per_block(int type); /* src/tensor.h:69-100 */
size_t or_row_bytes(int type, int K);   /* K / epb * bpb, as the reference computes rb */

float    or_fp16_to_fp32(uint16_t h);   /* src/fp16.h:9-38 */
uint16_t or_fp32_to_fp16(float f);      /* src/fp16.h:40-69 */
float    or_bf16_to_fp32(uint16_t b);   /* src/fp16.h:71-76 */
uint16_t or_fp32_to_bf16(float f);      /* src/fp16.h:78-85 */
void     or_get_scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m); /* src/kernels.h:82-90 */

/* ActQ8 quantizer for M rows of K floats (src/matmul_simd.cpp:348-410, 418-427). */
void or_quantize_act(const float* x, int M, int K, float* d, float* sum,
                     int16_t* sum_lo, int16_t* sum_hi, int8_t* qs);

/* Number of integer sub-block sums per row: K/32, or K/16 for Q6_K. */
int or_n_subsums(int type, int K);

/* Per-sub-block int32 dots of one weight row with one quantized activation
 * row, exactly the integers the NEON kernels form before their fp32 epilogue:
 *   Q8_0  : sum w*q over each 32-block                         (:143-160)
 *   Q4_0  : sum nibble*q (unsigned nibble) over each 32-block  (:162-182)
 *   Q5_0  : sum (v5-16)*q over each 32-block                   (:184-224)
 *   Q4_K  : sum nibble*q over each 32-element sub-block        (:226-283)
 *   Q6_K  : sum (v6-32)*q over each 16 elements                (:285-342)
 * Returns 0 on success, -1 for an unsupported type. */
int or_block_sums_row(int type, const uint8_t* wrow, const int8_t* qs, int K, int32_t* out);

/* Int8-activation dot of one weight row (fp32 result, NEON lane emulation). */
float or_dot_int_row(int type, const uint8_t* wrow, const float* d, const float* sum,
                     const int8_t* qs, int K);

/* gemm_int: y[m*N+j] = dot_int(quantize(x[m]), row j)   (src/matmul_simd.cpp:432-455).
 * nthreads <= 1 runs serially. Returns 0, or -1 for an unsupported type. */
int or_gemm_int(int type, const float* x, const uint8_t* w, float* y,
                int M, int K, int N, int nthreads);

/* moe_gemv_int / moe_gemv_multi_int (src/matmul_simd.cpp:506-544):
 *   y[k*N+j] = dot_int(xa_k, w + expert_idx[k]*N*rb + j*rb)
 * xa_k is quantize(x) for every k when multi == 0, quantize(x + k*K) when
 * multi != 0. */
int or_moe_gemv_int(int type, const float* x, const uint8_t* w, const int* expert_idx,
                    int n_experts, float* y, int K, int N, int multi, int nthreads);

/* Scalar fp32 dot of one row (src/matmul.cpp:63-314). */
float or_dot_scalar_row(int type, const float* x, const uint8_t* wrow, int K);

/* gemm_scalar (src/matmul.cpp:320-353) with ThreadPool::parallel_for's static
 * contiguous chunking over N; serial when M == 1 and N < 128, as the
 * reference. Returns 0, or -1 for an unsupported type. */
int or_gemm_scalar(int type, const float* x, const uint8_t* w, float* y,
                   int M, int K, int N, int nthreads);

/* dequantize (src/matmul.cpp:504-675). Returns 0, or -1 if unsupported. */
int or_dequantize(int type, const uint8_t* w, float* dst, int n);

/* Seeded inputs of the reference's matmul test (tests/test_matmul.cpp):
 * XorShift32 (tests/test_util.h:49-61) with the per-type seeds and field
 * order of test_q4_0/test_q8_0/test_q4_k/test_q6_k (:142-212) and
 * small_fp16 (:51-55). or_ref_test_x gives random_x with seed 7 + type
 * (:59-60). Returns 0, or -1 for a type the reference test does not cover. */
int  or_ref_test_weights(int type, int K, int N, uint8_t* out);
void or_ref_test_x(int type, int K, float* out);

/* Gemma4Arch::moe_ffn (src/arch_gemma4.cpp:507-641) for T tokens of H:
 * router rmsnorm + scale + matmul, softmax, top-k, renormalised weights,
 * expert rmsnorm, gate/up and down expert GEMVs (int8 path), GeGLU, weighted
 * sum with down_scale. out is T x H; idx_out / w_out (T x top_k) may be NULL.
 * Returns 0, or -1 for an unsupported type or top_k. */
int or_moe_ffn(const float* x, int T, int H, const uint8_t* router_w, int router_type,
               const float* router_scale, const float* pre_norm, float eps,
               const uint8_t* gu_w, int gu_type, const uint8_t* dn_w, int dn_type,
               const float* down_scale, int n_exp, int top_k, int inter,
               float* out, int* idx_out, float* w_out);

#ifdef __cplusplus
}
#endif
#endif
