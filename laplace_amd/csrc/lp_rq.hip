// lp_rq.hip - Q4_K GEMV for 1..8 activation rows on 4x4 int8 MFMA blocks.
//
// dot_row_q4_k_int (src/matmul_simd.cpp:226-283) for a few activation rows
// at once: per 32-element block b of weight row n and token m the exact
// integer sum P = sum_k q_mk * nib_nk, then
//   y[m, n] += (d_n * sc_nb) * xd_mb * P  -  (dmin_n * m_nb) * xs_mb
// with xd / xs the token's block scale and scaled block sum.
//
// Layout: a wave owns G = 16 / S row quads (4 consecutive weight rows each)
// at a time, with all of K (K <= 4096: at most 16 super-blocks; S = the
// super-block count rounded up to a power of two). Lane l = 4q + j: weight
// row j of row quad q / S, super-block q % S. Each lane loads its
// super-block (144 bytes: header + codes) with nine 16-byte loads.
//
// v_mfma_i32_4x4x4_16b_i8 is 16 independent 4x4x4 products; block q of the
// instruction is lane quad q (lanes 4q..4q+3): A row i = lane 4q+i, B column
// j = lane 4q+j, D[q][i][j] in lane 4q+j element i (layout checked on the
// device). A = four tokens' activation codes, B = the four rows' 4-bit codes
// (one byte per code, 4 consecutive K per lane), so every quad sums its own
// super-block: one instruction covers 4 tokens x 4 rows x 16 super-blocks x
// 4 K. Eight instructions give the 32-element block sums P of a block for
// all sixteen super-blocks at once, one output per lane and token: the fp32
// epilogue is 3 VALU operations per token and 32 weight elements (against
// 16 tokens' worth of outputs per 32 elements on a 16x16 tile).
// The min term sum_b m_nb * xs_mb runs on v_mfma_f32_4x4x1_16b_f32 (A = the
// tokens' xs, B = the rows' m), one per block, scaled by -dmin once per
// super-block.
// TG groups of 4 tokens (M <= 4 TG); unused token rows are zero.
//
// The partial sums of the S super-block lanes of a row are added with
// cross-lane shuffles (fixed order) when the row quads are done. Each wave
// handles `per_wave` consecutive units of G row quads; the next unit's loads
// are issued before the current one is computed.
// MOE: blockIdx.y is a routed group (expert, first pair, n <= 8 pairs, from
// the route table of the grouped dispatch): the group's activation rows
// (token, or pair in the multi form) and output rows (pairs) replace rows
// 0..M-1, and the weights are the group's expert.
//
// LDS (per workgroup): the tokens' codes, token stride = 272 bytes per
// super-block rounded to 64 mod 256 (lanes 4q+j of a 16-lane read phase then
// hit 16 distinct 16-byte bank groups: super-block q at +68q dwords, token j
// at +16j dwords mod 64); per super-block and block the tokens' xd and xs.

#include "lp_chunks.h"
#include "lp_internal.h"

namespace lp {

typedef int i4v __attribute__((ext_vector_type(4)));
typedef float f4v __attribute__((ext_vector_type(4)));

constexpr int kRqWaves = 4;      // waves per workgroup (8 for large dense two-group products)
constexpr int kRqMaxSb = 16;

struct RqArgs {
    const uint8_t* w;
    long rb;             // bytes per weight row
    ActView A;
    float* y;
    int M, K, N;
    long nunits;         // units of G row quads
    int per_wave;        // units per wave
    int tok_stride;      // LDS bytes per token's codes
    int sc_stride;       // LDS floats per super-block of scales (8 blocks x 4 TG tokens, padded)
    // MOE
    const uint8_t* route;
    long ebytes;         // bytes per expert
    int max_groups, multi, topk;
    const float* gu;     // MOE: when set, the activations are GeGLU(gu rows) quantized while staged
};

struct RqTile {
    u32x4 h;             // d, dmin, scales[12]
    u32x4 c[8];          // codes: bytes 16 i .. 16 i + 15
};

template <int TG, int S, bool MOE, int W = kRqWaves>
__global__ void __launch_bounds__(64 * W)
gemv_q4k_rq(RqArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr int MP = 4 * TG;
    constexpr int G = 16 / S;                 // row quads per wave unit
    constexpr int L = S == 1 ? 0 : S == 2 ? 1 : S == 4 ? 2 : S == 8 ? 3 : 4;
    const int K = a.K, N = a.N;
    int M = a.M;
    const uint8_t* w = a.w;
    const int* pairs = nullptr;
    int first = 0;
    if constexpr (MOE) {
        if ((int)blockIdx.y >= *reinterpret_cast<const int*>(a.route)) return;
        const int4 gd = reinterpret_cast<const int4*>(a.route + 16)[blockIdx.y];
        pairs = reinterpret_cast<const int*>(a.route + 16 + (size_t)a.max_groups * 16);
        first = gd.y;
        M = gd.z;
        w += (size_t)gd.x * a.ebytes;
    }
    auto act_row = [&](int m) -> size_t {
        if constexpr (MOE) {
            const int p = pairs[first + m];
            return (size_t)(a.multi ? p : p / a.topk);
        } else {
            return (size_t)m;
        }
    };
    const int nsb = K >> 8, nb = K >> 5;
    uint8_t* sq = smem;                                                   // [MP][tok_stride]
    float* sxd = reinterpret_cast<float*>(smem + (size_t)MP * a.tok_stride);   // [nsb][sc_stride]
    float* sxs = sxd + (size_t)nsb * a.sc_stride;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int q = lane >> 2, j = lane & 3;
    const int sub = q / S, sq_raw = q % S;
    const bool qv = sq_raw < nsb;
    const int sbq = qv ? sq_raw : nsb - 1;
    const int tga = (M + 3) >> 2;             // token groups in use

    const long gw = (long)blockIdx.x * W + __builtin_amdgcn_readfirstlane(wave);
    const long u0 = gw * a.per_wave;
    const long u1 = u0 + a.per_wave < a.nunits ? u0 + a.per_wave : a.nunits;
    const uint32_t lane_off = (uint32_t)((4 * sub + j) * a.rb + sbq * 144);

    auto load = [&](long u, RqTile& t) {
        // wave-uniform unit base; the last unit clamps rows past N
        const uint8_t* p;
        if ((u + 1) * 4 * G <= N) {
            p = w + u * 4 * G * a.rb + lane_off;
        } else {
            long row = (u * G + sub) * 4 + j;
            row = row < N ? row : N - 1;
            p = w + row * a.rb + (long)sbq * 144;
        }
        // plain loads: each 128-byte line is read by several of the nine
        // instructions (nontemporal loads measured 1.9x slower)
        t.h = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
        for (int i = 0; i < 8; i++) t.c[i] = reinterpret_cast<const u32x4*>(p + 16)[i];
    };

    RqTile ta, tb;
    if (u0 < u1) load(u0, ta);

    // stage the tokens' codes and block scales (zero for padding tokens)
    const int kp = K >> 4;                    // 16-byte pieces per token
    const int mq = MOE && a.gu ? M : 0;       // rows quantized from GeGLU(gu) below
    for (int i = threadIdx.x; i < MP * kp; i += blockDim.x) {
        const int m = i / kp, c = i - m * kp;
        if (m < mq) continue;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (m < M) v = reinterpret_cast<const u32x4*>(a.A.qs + act_row(m) * K)[c];
        *reinterpret_cast<u32x4*>(sq + (size_t)m * a.tok_stride + (c >> 4) * 272 + (c & 15) * 16) = v;
    }
    for (int i = threadIdx.x; i < MP * nb; i += blockDim.x) {
        const int m = i / nb, b = i - m * nb;
        if (m < mq) continue;
        const int o = (b >> 3) * a.sc_stride + (b & 7) * MP + m;
        const size_t r = m < M ? act_row(m) : 0;
        sxd[o] = m < M ? a.A.d[r * nb + b] : 0.0f;
        sxs[o] = m < M ? a.A.sum[r * nb + b] : 0.0f;
    }
    if constexpr (MOE) {
        for (int m = 0; m < mq; m++)
            stage_geglu_row(a.gu + act_row(m) * 2 * K, K, sq + (size_t)m * a.tok_stride, sxd + m, a.sc_stride, MP,
                            nsb * a.sc_stride, threadIdx.x, blockDim.x);
    }
    __syncthreads();

    const uint8_t* aq = sq + (size_t)j * a.tok_stride + sbq * 272;      // token j (+4t) of super-block sbq
    const float* xdq = sxd + (size_t)sbq * a.sc_stride;
    const float* xsq = sxs + (size_t)sbq * a.sc_stride;
    const i4v zi = {0, 0, 0, 0};
    const f4v z4 = {0.0f, 0.0f, 0.0f, 0.0f};

    // one unit of G row quads from its loaded tile
    auto compute = [&](long u, const RqTile& T) {
        const u32x4 h = T.h;
        const float d = qv ? fp16_bits_to_f32(h.x) : 0.0f;
        const float dmin = qv ? fp16_bits_to_f32(h.x >> 16) : 0.0f;
        f4v acc[TG], mn[TG];
#pragma unroll
        for (int t = 0; t < TG; t++) {
            acc[t] = z4;
            mn[t] = z4;
        }
#pragma unroll
        for (int jb = 0; jb < 4; jb++) {
            uint32_t sc0, m0, sc1, m1;
            scale_min_k4(2 * jb, h.y, h.z, h.w, sc0, m0);
            scale_min_k4(2 * jb + 1, h.y, h.z, h.w, sc1, m1);
            const float ds0 = d * (float)sc0, ds1 = d * (float)sc1;
            const float fm0 = (float)m0, fm1 = (float)m1;
            // 4-bit codes as bytes: low nibbles (block 2jb), high nibbles (2jb+1);
            // the high ones shifted two dwords at a time
            const u32x4 c0 = T.c[2 * jb], c1 = T.c[2 * jb + 1];
            const uint64_t wv[4] = {(uint64_t)c0.y << 32 | c0.x, (uint64_t)c0.w << 32 | c0.z,
                                    (uint64_t)c1.y << 32 | c1.x, (uint64_t)c1.w << 32 | c1.z};
            uint32_t bl[8], bh[8];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint64_t lo = wv[i] & 0x0f0f0f0f0f0f0f0full, hi = (wv[i] >> 4) & 0x0f0f0f0f0f0f0f0full;
                bl[2 * i] = (uint32_t)lo;
                bl[2 * i + 1] = (uint32_t)(lo >> 32);
                bh[2 * i] = (uint32_t)hi;
                bh[2 * i + 1] = (uint32_t)(hi >> 32);
            }
#pragma unroll
            for (int t = 0; t < TG; t++) {
                if (t < tga) {
                    const uint8_t* at = aq + (size_t)4 * t * a.tok_stride + 64 * jb;
                    const u32x4 l0 = *reinterpret_cast<const u32x4*>(at);
                    const u32x4 l1 = *reinterpret_cast<const u32x4*>(at + 16);
                    const u32x4 g0 = *reinterpret_cast<const u32x4*>(at + 32);
                    const u32x4 g1 = *reinterpret_cast<const u32x4*>(at + 48);
                    const uint32_t al[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
                    const uint32_t ah[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
                    i4v p0 = zi, p1 = zi;
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        p0 = __builtin_amdgcn_mfma_i32_4x4x4i8((int)al[i], (int)bl[i], p0, 0, 0, 0);
                        p1 = __builtin_amdgcn_mfma_i32_4x4x4i8((int)ah[i], (int)bh[i], p1, 0, 0, 0);
                    }
                    const f4v xd0 = *reinterpret_cast<const f4v*>(xdq + (2 * jb) * MP + 4 * t);
                    const f4v xd1 = *reinterpret_cast<const f4v*>(xdq + (2 * jb + 1) * MP + 4 * t);
                    const float xs0 = xsq[(2 * jb) * MP + 4 * t + j];
                    const float xs1 = xsq[(2 * jb + 1) * MP + 4 * t + j];
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        acc[t][r] = fmaf((float)p0[r] * xd0[r], ds0, acc[t][r]);
                        acc[t][r] = fmaf((float)p1[r] * xd1[r], ds1, acc[t][r]);
                    }
                    mn[t] = __builtin_amdgcn_mfma_f32_4x4x1f32(xs0, fm0, mn[t], 0, 0, 0);
                    mn[t] = __builtin_amdgcn_mfma_f32_4x4x1f32(xs1, fm1, mn[t], 0, 0, 0);
                }
                // keep the next step's LDS reads behind this one (without it:
                // 219 / 372 registers, 10-40 % slower)
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        // Sum over the S super-block lanes of each row (lane bits 2 .. L+1).
        // With two or more levels the 4 tokens are spread over the lanes on
        // the way: the exchanges over the top two levels leave token
        // 2*b(L+1) + b(L) in each lane, the lower levels are plain sums, and
        // the lanes with those lower bits clear store.
        const long row = (u * G + sub) * 4 + j;
#pragma unroll
        for (int t = 0; t < TG; t++) {
            if (t < tga) {
                float v[4];
#pragma unroll
                for (int r = 0; r < 4; r++) v[r] = fmaf(-dmin, mn[t][r], acc[t][r]);
                if constexpr (L >= 2) {
                    const bool bh = (lane >> (L + 1)) & 1, bl = (lane >> L) & 1;
                    const float k0 = bh ? v[2] : v[0], k1 = bh ? v[3] : v[1];
                    const float s0 = bh ? v[0] : v[2], s1 = bh ? v[1] : v[3];
                    const float w0 = k0 + __shfl_xor(s0, 2 << L), w1 = k1 + __shfl_xor(s1, 2 << L);
                    float uu = (bl ? w1 : w0) + __shfl_xor(bl ? w0 : w1, 1 << L);
#pragma unroll
                    for (int b = L - 1; b >= 2; b--) uu += __shfl_xor(uu, 1 << b);
                    const int m = 4 * t + 2 * bh + bl;
                    const bool st = ((lane >> 2) & ((1 << (L - 2)) - 1)) == 0;
                    if (st && m < M && row < N) {
                        size_t yr = (size_t)m;
                        if constexpr (MOE) yr = (size_t)pairs[first + m];
                        a.y[yr * N + row] = uu;
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        if constexpr (L == 1) v[r] += __shfl_xor(v[r], 4);
                        const int m = 4 * t + r;
                        if ((L == 0 || (q & 1) == 0) && m < M && row < N) {
                            size_t yr = (size_t)m;
                            if constexpr (MOE) yr = (size_t)pairs[first + m];
                            a.y[yr * N + row] = v[r];
                        }
                    }
                }
            }
        }
    };

    // units in pairs: each tile buffer is loaded while the other is computed
    for (long u = u0; u < u1; u += 2) {
        if (u + 1 < u1) load(u + 1, tb);
        compute(u, ta);
        if (u + 1 >= u1) break;
        if (u + 2 < u1) load(u + 2, ta);
        compute(u + 1, tb);
    }
}

static size_t rq_tok_stride(int K) {
    size_t s = (size_t)(K / 256) * 272;
    s = (s + 255) & ~size_t(255);
    return s + 64;                       // 64 mod 256
}

static int rq_tg(int M) { return M <= 4 ? 1 : 2; }

static size_t rq_lds(int M, int K) {
    const int MP = 4 * rq_tg(M);
    const size_t sc_stride = (size_t)8 * MP + 4;
    return (size_t)MP * rq_tok_stride(K) + 2 * (size_t)(K / 256) * sc_stride * 4;
}

bool rq_supported(uint32_t type, int M, int K, int N, const uint8_t* w) {
    return type == T_Q4_K && M >= 1 && M <= 8 && K % 256 == 0 && K / 256 <= kRqMaxSb && N > 0 &&
           reinterpret_cast<uintptr_t>(w) % 16 == 0 && rq_lds(M, K) <= 64 * 1024;
}

// Where it beats the dot4 GEMV (M <= 4) and the 16x16 int8 MFMA kernel
// (M >= 5), measured on MI355X against them (us, K 4096 unless noted):
//   M=3: 18944x3584 13.8 vs 16.5, 14336 12.8 vs 13.8; 8192 8.8 vs 8.0, 4096 6.6 vs 6.2
//   M=4: 18944x3584 13.9 vs 18.2, 14336 12.9 vs 15.6, 4096 6.7 vs 7.0, 1536x2048 5.1 vs 6.0
//   M=5: 14336 15.5 vs 17.8, 2048 7.6 vs 7.8; 1536x2048 6.2 vs 5.7
//   M=8: 18944x3584 17.9 vs 20.6, 14336 16.2 vs 19.1, 4096 8.6 vs 9.0; 1536x2048 6.3 vs 6.2
//   M=2: slower everywhere measured (14336: 13.8 vs 13.1)
bool rq_preferred(uint32_t type, int M, int K, int N, const uint8_t* w) {
    if (!rq_supported(type, M, K, N, w)) return false;
    return M == 4 || (M == 3 && N >= 12288) || (M >= 5 && N >= 2048);
}

static int rq_span(int K) {
    const int nsb = K / 256;
    int S = 1;
    while (S < nsb) S <<= 1;
    return S;
}

template <bool MOE>
static hipError_t launch_rq(const RqArgs& a0, int TG, int groups, hipStream_t st) {
    RqArgs a = a0;
    const int S = rq_span(a.K);
    const int G = 16 / S;
    a.nunits = ((long)a.N + 4 * G - 1) / (4 * G);
    a.tok_stride = (int)rq_tok_stride(a.K);
    a.sc_stride = 8 * 4 * TG + 4;
    if (MOE) {
        // four units per wave: the group's activation staging then serves
        // four units' weights (measured at 128 experts, 64 tokens, top-8:
        // 135 / 123 / 122 / 125 / 148 us at 1 / 2 / 4 / 8 / 16)
        a.per_wave = 4;
    } else {
        // whole units per wave, as few per wave as lets every workgroup be
        // resident at once (register-limited: 12 waves per CU at TG 1, 8 at TG 2)
        const long target = (long)device_cu_count() * (TG == 1 ? 12 : 8);
        a.per_wave = (int)((a.nunits + target - 1) / target);
    }
    // Two token groups over many rows: 8-wave workgroups (one per CU at the
    // 8-waves target), whose activation staging serves twice the waves
    // (us, 4 vs 8 waves: 18944x3584 M=5 17.7 / 16.6, M=8 18.8 / 17.2;
    // 14336x4096 M=5 16.5 / 15.7, M=8 16.9 / 16.2; but 4096x4096 M=8 9.2 /
    // 9.6, and one token group mixed: 18944x3584 M=4 14.3 / 17.8)
    const int W = (!MOE && TG == 2 && a.N >= 8192) ? 8 : kRqWaves;
    const long waves = (a.nunits + a.per_wave - 1) / a.per_wave;
    const dim3 grid((unsigned)((waves + W - 1) / W), (unsigned)groups);
    const size_t shm = rq_lds(4 * TG, a.K);
#define LP_RQ(TGV, SV)                                                                                        \
    if (W == 8) hipLaunchKernelGGL((gemv_q4k_rq<TGV, SV, MOE, (TGV == 2 && !MOE) ? 8 : kRqWaves>), grid,         \
                                   dim3(64 * W), shm, st, a);                                                 \
    else hipLaunchKernelGGL((gemv_q4k_rq<TGV, SV, MOE>), grid, dim3(64 * kRqWaves), shm, st, a)
#define LP_RQS(TGV)                     \
    switch (S) {                        \
        case 1: LP_RQ(TGV, 1); break;   \
        case 2: LP_RQ(TGV, 2); break;   \
        case 4: LP_RQ(TGV, 4); break;   \
        case 8: LP_RQ(TGV, 8); break;   \
        default: LP_RQ(TGV, 16); break; \
    }
    if (TG == 1) {
        LP_RQS(1)
    } else {
        LP_RQS(2)
    }
#undef LP_RQS
#undef LP_RQ
    return hipGetLastError();
}

hipError_t launch_gemv_rq(const uint8_t* w, const ActView& A, float* y, int M, int K, int N, hipStream_t st) {
    if (M <= 0 || N <= 0) return hipSuccess;
    if (!rq_supported(T_Q4_K, M, K, N, w)) return hipErrorInvalidValue;
    RqArgs a{};
    a.w = w;
    a.rb = (long)row_bytes(T_Q4_K, K);
    a.A = A;
    a.y = y;
    a.M = M;
    a.K = K;
    a.N = N;
    return launch_rq<false>(a, rq_tg(M), 1, st);
}

bool rq_moe_supported(uint32_t type, int K) { return rq_supported(type, kRqMoeGroup, K, 1, nullptr); }

hipError_t launch_moe_rq(const uint8_t* w, const ActView& A, const void* route, int max_groups, int gsize,
                         int multi, int topk, float* y, int K, int N, hipStream_t st, const float* gu) {
    if (N <= 0 || max_groups <= 0) return hipSuccess;
    if (!rq_supported(T_Q4_K, kRqMoeGroup, K, N, w)) return hipErrorInvalidValue;
    RqArgs a{};
    a.w = w;
    a.rb = (long)row_bytes(T_Q4_K, K);
    a.A = A;
    a.y = y;
    a.M = kRqMoeGroup;
    a.K = K;
    a.N = N;
    a.route = static_cast<const uint8_t*>(route);
    a.ebytes = a.rb * N;
    a.max_groups = max_groups;
    a.multi = multi;
    a.topk = topk;
    a.gu = gu;
    if (gsize != kRqMoeGroup) return hipErrorInvalidValue;
    return launch_rq<true>(a, 2, max_groups, st);
}

}  // namespace lp
