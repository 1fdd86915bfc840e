/*
 * laplace_hip.h - C ABI of the MI355X (gfx950) GGUF quantized-matmul back-end.
 *
 * The functions below are what the Laplace C++ engine binds to replace its
 * CPU matmul back-end. Plain pointers and sizes only; no HIP or torch types.
 * `type` is a GGMLType value (reference src/tensor.h:11-34). The matmul
 * entries (lp_gemm, lp_gemm_dev, lp_gemm_batch) handle F32 = 0, F16 = 1,
 * Q4_0 = 2, Q5_0 = 6, Q8_0 = 8, Q2_K = 10, Q3_K = 11, Q4_K = 12, Q5_K = 13,
 * Q6_K = 14 and BF16 = 30; lp_gemm_q_dev takes the int8-activation types
 * (Q4_0, Q5_0, Q8_0, Q4_K, Q6_K) and the grouped-MoE entries Q4_0, Q8_0,
 * Q4_K and Q6_K. Any other type
 * makes the call return "not handled" so the caller falls back to its CPU
 * path.
 *
 * Two families:
 *   1. Host-pointer, synchronous entry points with the exact signatures of
 *      the reference's back-end function-pointer types (src/kernels.h:94-119):
 *      x, w, y live in host memory; y is complete when the call returns;
 *      false means "type or shape not handled here, fall back". Weights are
 *      served from device copies made by lp_register_weights (or a copy
 *      cached by host pointer on first use, as the reference's Metal back-end
 *      does, src/metal.mm:601-621).
 *   2. Device-pointer, stream-ordered entry points (suffix _dev) for callers
 *      that keep x, w, y in HBM. They never allocate: scratch for quantized
 *      activations is a caller-provided workspace sized by
 *      lp_act_workspace_bytes. They return an lp_status code.
 *
 * Numerics follow the reference's int8-activation path
 * (src/matmul_simd.cpp): activations are quantized to 32-element int8
 * blocks exactly as quantize_act_q8_neon does (:348-410, bit-exact), the
 * per-block int32 dot sums equal the NEON kernels' (:143-342, bit-exact),
 * and fp32 outputs agree with the reference within 1e-4 normwise relative
 * error (fp32 accumulation order differs).
 */
#ifndef LAPLACE_HIP_H
#define LAPLACE_HIP_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    LP_OK = 0,
    LP_UNSUPPORTED = 1,  /* type/shape/alignment not handled: caller falls back */
    LP_EINVAL = 2,       /* bad argument (null pointer, short workspace, ...) */
    LP_EHIP = 3,         /* a HIP runtime call failed; see lp_last_error() */
    LP_ENODEV = 4        /* no usable gfx950 device */
} lp_status;

/* ---- 1. drop-in back-end ABI (host pointers, synchronous) ---------------- */

/* y[M,N] = X[M,K] @ W^T, W = N contiguous rows of K elements of `type`.
 * Replaces gemm_fn (src/kernels.h:97-98) / gemm_simd (src/matmul_simd.cpp:480-496). */
bool lp_gemm(const float* x, const uint8_t* w, uint32_t type, float* y, int M, int K, int N);

/* y[k*N + j] = dot(x, W_{expert_idx[k]} row j), one shared activation row.
 * Replaces moe_gemv_fn (src/kernels.h:100-105) / moe_gemv_simd (src/matmul_simd.cpp:580-596). */
bool lp_moe_gemv(const float* x, const uint8_t* w, uint32_t type, const int* expert_idx,
                 int n_experts, float* y, int K, int N);

/* y[k*N + j] = dot(x + k*K, W_{expert_idx[k]} row j).
 * Replaces moe_gemv_multi_fn (src/kernels.h:107-112) / moe_gemv_multi_simd (:598-614). */
bool lp_moe_gemv_multi(const float* x, const uint8_t* w, uint32_t type, const int* expert_idx,
                       int n_experts, float* y, int K, int N);

typedef bool (*lp_gemm_fn)(const float*, const uint8_t*, uint32_t, float*, int, int, int);
typedef bool (*lp_moe_gemv_fn)(const float*, const uint8_t*, uint32_t, const int*, int,
                               float*, int, int);

/* Getters in the style of get_simd_gemm (src/kernels.h:114-119): NULL when
 * no gfx950 device is usable, so the caller keeps its scalar path. */
lp_gemm_fn     lp_get_gemm(void);
lp_moe_gemv_fn lp_get_moe_gemv(void);
lp_moe_gemv_fn lp_get_moe_gemv_multi(void);

/* Copies [base, base+size) of host memory (e.g. the mmap'd GGUF file) to the
 * current device once; host weight pointers inside it then resolve to the
 * device copy. Mirrors matmul_register_weights (src/matmul.h:47-48) and the
 * Metal registration it forwards to (src/metal.mm:581-599). */
int lp_register_weights(const void* base, size_t size);
/* Drops every registered region and cached weight copy of the current device. */
void lp_release_weights(void);
/* Drops the one region registered at `base` (other regions and cached copies
 * stay). LP_EINVAL if no region starts there. No reference counterpart: the
 * reference never unregisters; this is for a file that is closed while
 * others stay open. */
int lp_release_region(const void* base);

/* Host-pointer quantizer, the ActQ8 fields as separate arrays (test hook):
 * d, sum, sum_lo, sum_hi hold M*K/32 values, qs M*K codes. K % 32 == 0. */
int lp_quantize_act(const float* x, int M, int K, float* d, float* sum, int16_t* sum_lo,
                    int16_t* sum_hi, int8_t* qs);

/* dst[0..n) = the first n elements of w, dequantized to fp32. Types: F32,
 * F16, BF16, Q4_0, Q5_0, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K; n a multiple of
 * the block size. Each value equals the reference's scalar dequantize
 * (same operation order, no contraction). Replaces Laplace::dequantize
 * (src/matmul.h:44, src/matmul.cpp:504-675); host pointers, synchronous; the
 * weights resolve through lp_register_weights like the matmul entries. */
int lp_dequantize(const uint8_t* w, uint32_t type, float* dst, long n);

/* ---- 2. device-pointer, stream-ordered API ------------------------------- */

/* Bytes of workspace holding M rows of quantized activations of length K,
 * plus the scratch of the kernels that run on them (fp16 planes of the
 * prefill GEMM for M >= 5, 2 MiB of partial sums for 3 <= M <= 8). */
size_t lp_act_workspace_bytes(int M, int K);

/* Quantize x[M,K] (device) into the workspace (codes, scales, sums). */
int lp_quantize_act_dev(const float* x, int M, int K, void* ws, size_t ws_bytes, void* stream);

/* Read back the quantized activations held in a workspace into device
 * arrays in the host-API layout (test hook). */
int lp_act_unpack_dev(const void* ws, int M, int K, float* d, float* sum, int32_t* sums16,
                      int8_t* qs, void* stream);

/* y[M,N] = X[M,K] @ W^T on device pointers: quantize, then GEMV (M <= 8)
 * or GEMM. x, w, y and ws are device pointers; `stream` is a hipStream_t
 * (NULL = default stream). Asynchronous with respect to the host. */
int lp_gemm_dev(const float* x, const uint8_t* w, uint32_t type, float* y, int M, int K, int N,
                void* ws, size_t ws_bytes, void* stream);

/* Same product from activations already quantized into ws. ws must be the
 * buffer lp_quantize_act_dev filled for the same M and K, of at least
 * lp_act_workspace_bytes(M, K) bytes: besides the quantized blocks, the
 * kernels chosen here use its tail (the GEMM planes for M >= 5, partial sums
 * for 3 <= M <= 8), and this call takes no size to check it against. */
int lp_gemm_q_dev(const void* ws, const uint8_t* w, uint32_t type, float* y, int M, int K, int N,
                  void* stream);

/* lp_gemm_dev without a workspace argument: the workspace is a static
 * device array of the library (8 MiB per device), so the call allocates
 * nothing, for callers that cannot allocate (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). No counterpart in
 * the reference. Shapes whose workspace (lp_act_workspace_bytes(M, K))
 * exceeds 8 MiB return LP_EINVAL. Calls that overlap on one device race on
 * the shared array; serialise them (one stream, or events). */
int lp_gemm_dev_noalloc(const float* x, const uint8_t* w, uint32_t type, float* y, int M, int K, int N,
                        void* stream);

/* Per-sub-block int32 dots through the GEMV decoders (test hook):
 * out[(m*N + j)*S + s], S = K/32 (K/16 for Q6_K). */
int lp_block_sums_dev(const void* ws, const uint8_t* w, uint32_t type, int32_t* out, int M,
                      int K, int N, void* stream);

/* Device-pointer dequantize, stream-ordered. */
int lp_dequantize_dev(const uint8_t* w, uint32_t type, float* dst, long n, void* stream);

/* ---- 2b. batched M=1 matmuls ------------------------------------------------ */

/* One M=1 matmul of a batch: y[N] = x[K] @ W^T. Mirrors MatmulBatchSpec
 * (src/matmul.h:46-53) with the Tensor replaced by (w, type). */
typedef struct lp_batch_spec {
    const float* x;
    const uint8_t* w;
    uint32_t type;
    float* y;
    int K, N;
} lp_batch_spec;

/* n matmuls, host pointers, synchronous. Replaces matmul_gemm_batch
 * (src/matmul.h:54, src/matmul.cpp:450-454). Consecutive Q4_K specs with the
 * same x and K (the Q/K/V and gate/up batches of src/arch_gemma4.cpp:318-327,
 * :694-700) run as one launch of up to 4 matrices. false = not handled
 * (caller loops over matmul_rows). */
bool lp_gemm_batch(const lp_batch_spec* specs, int n);

/* Device-pointer form (x, w, y device pointers; the specs array itself in
 * host memory), stream-ordered; ws of lp_gemm_batch_workspace_bytes. */
size_t lp_gemm_batch_workspace_bytes(const lp_batch_spec* specs, int n);
int lp_gemm_batch_dev(const lp_batch_spec* specs, int n, void* ws, size_t ws_bytes, void* stream);

/* ---- 3. grouped MoE dispatch ---------------------------------------------- */

/* The MoE layer of T tokens, each routed to topk experts of a stacked weight
 * tensor w = n_experts x (N rows of K elements of `type`). Pair
 * p = t*topk + j uses expert topk_idx[p] and writes y[p*N .. p*N + N):
 *   multi == 0: y[p*N + n] = dot(x[t*K ..], W_{topk_idx[p]} row n)     (x is T x K)
 *   multi != 0: y[p*N + n] = dot(x[p*K ..], W_{topk_idx[p]} row n)     (x is T*topk x K)
 * Each pair's result equals the reference's per-token call for that token:
 * fused_moe_gemm_idx / fused_moe_gemm_multi (src/matmul.cpp:456-500, called
 * per token from src/arch_gemma4.cpp:604 and :626), i.e. moe_gemv_int /
 * moe_gemv_multi_int (src/matmul_simd.cpp:506-544). Pairs are grouped by
 * expert on the device so an expert's weights are streamed once per group
 * instead of once per pair. No reference counterpart as a single entry: the
 * reference loops over tokens. */
size_t lp_moe_workspace_bytes(int T, int topk, int n_experts, int K, int multi);

/* Device pointers, stream-ordered. Indices outside [0, n_experts) are
 * dropped on the device (their y rows are left unwritten). */
int lp_moe_grouped_dev(const float* x, int multi, const int* topk_idx, const uint8_t* w,
                       uint32_t type, float* y, int T, int topk, int n_experts, int K, int N,
                       void* ws, size_t ws_bytes, void* stream);

/* Host pointers, synchronous; false (with lp_last_error) on a bad index. */
bool lp_moe_grouped(const float* x, int multi, const int* topk_idx, const uint8_t* w,
                    uint32_t type, float* y, int T, int topk, int n_experts, int K, int N);

/* ---- 4. MoE feed-forward layer (router, experts, combine) ----------------- */

/* The whole MoE feed-forward of Gemma4Arch::moe_ffn (src/arch_gemma4.cpp:507-641)
 * for T tokens on the device:
 *   router in  r = rmsnorm_no_scale(x) * router_scale / sqrt(H)     (:537-541)
 *   logits     = r @ router_w^T  (n_exp rows of H, router_type)      (:543-544)
 *   softmax, top-k (lowest index wins a tie), weights / their sum    (:546-563)
 *   expert in  e = rmsnorm(x, pre_norm, rms_eps)                     (:567-571)
 *   gu[p]      = e_t @ gate_up_w[idx[p]]^T   (2*inter rows of H)     (:598-605)
 *   hidden[p]  = gelu_tanh(gu[p][0:inter]) * gu[p][inter:2*inter]    (:613-620)
 *   eo[p]      = hidden[p] @ down_w[idx[p]]^T (H rows of inter)      (:623-628)
 *   out[t]     = sum_k (w[t,k] * down_scale[idx[t,k]]) * eo[t*top_k + k]  (:632-639)
 * x and out are T x H; p = t*top_k + k. The expert GEMVs are the grouped
 * dispatch of section 3 (int8 types); the router takes every type lp_gemm
 * takes. topk_idx / topk_w (T x top_k) receive the routing when not NULL.
 * Constraints: n_exp <= 1024, 1 <= top_k <= min(16, n_exp). No single
 * reference counterpart: the reference runs these steps per token on the CPU. */
size_t lp_moe_ffn_workspace_bytes(int T, int H, int n_exp, int top_k, int inter, uint32_t router_type);

int lp_moe_ffn_dev(const float* x, int T, int H, const uint8_t* router_w, uint32_t router_type,
                   const float* router_scale, const float* pre_norm, float rms_eps,
                   const uint8_t* gate_up_w, uint32_t gate_up_type, const uint8_t* down_w,
                   uint32_t down_type, const float* down_scale, int n_exp, int top_k, int inter,
                   float* out, int* topk_idx, float* topk_w, void* ws, size_t ws_bytes, void* stream);

/* ---- diagnostics ----------------------------------------------------------- */

/* Kernel-family switch for the Q4_K prefill GEMM (M > 64), no reference
 * counterpart; for comparison runs and tests. 0: chosen by shape (default);
 * 1: split-precision fp16/fp8 MFMA on row-major planes; 2: fp16/fp8 MFMA on
 * MFMA-fragment-order planes; 3: int8 MFMA with a per-block fp32 epilogue;
 * 4 and 5: the wide-token kernel (128-token wave tiles on fragment-order
 * planes) with 128 x 256 and 256 x 256 workgroup tiles. All meet the same
 * parity bar. Process-wide; not thread-safe against
 * concurrent matmul calls. Returns LP_EINVAL for other values. */
int lp_set_gemm_kernel(int kernel);

/* Routing probe, no reference counterpart: the name of the kernel family
 * lp_gemm_q_dev runs for these operands (with a workspace of
 * lp_act_workspace_bytes(M, K) bytes; the first chunk's kernel when M rows
 * are split into chunks): "sb", "b32_sb", "sbm", "q6k_sbm", "rq", "i8mf",
 * "gemm", "tile", "fact" (fp32-activation types); "" when the shape or
 * type is rejected. The choice depends on the device (CU count): tests use
 * it to show which kernel a parity case exercised. */
const char* lp_gemm_route(uint32_t type, int M, int K, int N, const void* w);

/* Measurement hook, no reference counterpart: streams `bytes` (a multiple
 * of 16) from device memory with `grid` x `block` threads and `unroll`
 * (1, 4 or 9) independent 16-byte non-temporal loads in flight per thread,
 * the GEMV's load form; `sink` (4 bytes of device memory) is written only on
 * an impossible checksum. Its time per launch is the read ceiling the
 * weight-streaming kernels are compared with (bench.py's roofline field). */
int lp_read_probe_dev(const void* buf, size_t bytes, int grid, int block, int unroll, uint32_t* sink,
                      void* stream);

/* Measurement hook, no reference counterpart: `grid` workgroups of 8 waves
 * issue `iters` times the MFMA sequence of one 64-element K step of the
 * prefill GEMM (kind 0: 16 fp16 32x32x16 + 4 fp8 32x32x64 products on a 2 x 2
 * tile set; kind 1: 8 int8 32x32x32 products) on register operands, either
 * near-constant (random_operands = 0) or random values of the GEMM's ranges;
 * `out` takes grid * 512 floats. Its time against the nominal rate is how
 * much of the MFMA peak the part sustains on such data. Kinds 2-9: 32 fp16
 * 32x32x16 products per iteration with 0, 1, 3 or 6 independent VALU
 * operations after each, in 8-wave (2-5) or 4-wave (6-9) workgroups: how
 * much of the matrix pipe's rate survives VALU work issued by the same wave
 * (random_operands ignored). */
int lp_mfma_probe_dev(int kind, int random_operands, int iters, int grid, float* out, void* stream);

/* Text of the last error on this thread ("" if none). */
const char* lp_last_error(void);
/* 1 if the current device is usable (gfx950), 0 otherwise. */
int lp_device_ok(void);
/* Measurement aid, no reference counterpart: the current device's compute
 * unit count, peak shader clock (kHz), memory clock (kHz) and memory bus
 * width (bits), as the runtime reports them (0 where it reports nothing);
 * bench.py records them next to the peaks it divides by. Null pointers are
 * skipped. */
int lp_device_info(int* cus, int* clock_khz, int* mem_clock_khz, int* mem_bus_bits);

#ifdef __cplusplus
}
#endif
#endif
