// lp_rq.hip - Q4_K GEMV for 1..8 activation rows on 4x4 int8 MFMA blocks.
//
// dot_row_q4_k_int (src/matmul_simd.cpp:226-283) for a few activation rows
// at once: per 32-element block b of weight row n and token m the exact
// integer sum P = sum_k q_mk * nib_nk, then
//   y[m, n] += (d_n * sc_nb) * xd_mb * P  -  (dmin_n * m_nb) * xs_mb
// with xd / xs the token's block scale and scaled block sum.
//
// Layout: a wave owns a row quad (4 consecutive weight rows) at a time, with
// all of K (K <= 4096: at most 16 super-blocks). Lane l = 4q + j: weight row
// j of the quad, super-block q. Each lane loads its super-block (144 bytes:
// header + codes) with nine 16-byte loads; for a fixed row the 16 lanes read
// 2.3 KB of one row, so an instruction touches 4 row spans.
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
// The partial sums of the 16 super-block lanes of a row are added with
// cross-lane shuffles (fixed order) when the row quad is done. Each wave
// handles `per_wave` consecutive row quads; the next quad's loads are issued
// before the current one is computed.
//
// LDS (per workgroup): the tokens' codes, token stride = 272 bytes per
// super-block rounded to 64 mod 256 (lanes 4q+j of a 16-lane read phase then
// hit 16 distinct 16-byte bank groups: super-block q at +68q dwords, token j
// at +16j dwords mod 64); per super-block and block the tokens' xd and xs.

#include "lp_internal.h"

namespace lp {

typedef int i4v __attribute__((ext_vector_type(4)));
typedef float f4v __attribute__((ext_vector_type(4)));

constexpr int kRqWaves = 4;
constexpr int kRqMaxSb = 16;

struct RqArgs {
    const uint8_t* w;
    long rb;             // bytes per weight row
    ActView A;
    float* y;
    int M, K, N;
    long nrq;            // row quads
    int per_wave;        // row quads per wave
    int tok_stride;      // LDS bytes per token's codes
    int sc_stride;       // LDS floats per super-block of scales (8 blocks x 4 TG tokens, padded)
};

struct RqTile {
    u32x4 h;             // d, dmin, scales[12]
    u32x4 c[8];          // codes: bytes 16 i .. 16 i + 15
};

template <int TG>
__global__ void __launch_bounds__(64 * kRqWaves)
gemv_q4k_rq(RqArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr int MP = 4 * TG;
    const int K = a.K, N = a.N, M = a.M;
    const int nsb = K >> 8, nb = K >> 5;
    uint8_t* sq = smem;                                                   // [MP][tok_stride]
    float* sxd = reinterpret_cast<float*>(smem + (size_t)MP * a.tok_stride);   // [nsb][sc_stride]
    float* sxs = sxd + (size_t)nsb * a.sc_stride;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int q = lane >> 2, j = lane & 3;
    const bool qv = q < nsb;
    const int sbq = qv ? q : nsb - 1;

    const long gw = (long)blockIdx.x * kRqWaves + __builtin_amdgcn_readfirstlane(wave);
    const long rq0 = gw * a.per_wave;
    const long rq1 = rq0 + a.per_wave < a.nrq ? rq0 + a.per_wave : a.nrq;
    const uint32_t lane_off = (uint32_t)(j * a.rb + sbq * 144);

    auto load = [&](long rq, RqTile& t) {
        // wave-uniform row-quad base; the last quad clamps rows past N
        const uint8_t* p;
        if (rq * 4 + 4 <= N) {
            p = a.w + rq * 4 * a.rb + lane_off;
        } else {
            long row = rq * 4 + j;
            row = row < N ? row : N - 1;
            p = a.w + row * a.rb + (long)sbq * 144;
        }
        // plain loads: each 128-byte line is read by several of the nine
        // instructions (nontemporal loads measured 1.9x slower)
        t.h = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
        for (int i = 0; i < 8; i++) t.c[i] = reinterpret_cast<const u32x4*>(p + 16)[i];
    };

    RqTile ta, tb;
    if (rq0 < rq1) load(rq0, ta);

    // stage the tokens' codes and block scales (zero for padding tokens)
    for (int i = threadIdx.x; i < MP * (K >> 4); i += blockDim.x) {
        const int m = i / (K >> 4), c = i % (K >> 4);        // 16-byte piece c of token m
        u32x4 v = {0u, 0u, 0u, 0u};
        if (m < M) v = reinterpret_cast<const u32x4*>(a.A.qs + (size_t)m * K)[c];
        *reinterpret_cast<u32x4*>(sq + (size_t)m * a.tok_stride + (c >> 4) * 272 + (c & 15) * 16) = v;
    }
    for (int i = threadIdx.x; i < MP * nb; i += blockDim.x) {
        const int m = i / nb, b = i % nb;
        const int o = (b >> 3) * a.sc_stride + (b & 7) * MP + m;
        sxd[o] = m < M ? a.A.d[(size_t)m * nb + b] : 0.0f;
        sxs[o] = m < M ? a.A.sum[(size_t)m * nb + b] : 0.0f;
    }
    __syncthreads();

    const uint8_t* aq = sq + (size_t)j * a.tok_stride + sbq * 272;      // token j (+4t) of super-block sbq
    const float* xdq = sxd + (size_t)sbq * a.sc_stride;
    const float* xsq = sxs + (size_t)sbq * a.sc_stride;
    const i4v zi = {0, 0, 0, 0};
    const f4v z4 = {0.0f, 0.0f, 0.0f, 0.0f};

    // one row quad from its loaded tile
    auto compute = [&](long rq, const RqTile& T) {
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
                // keep the next step's LDS reads behind this one (without it:
                // 219 / 372 registers, 10-40 % slower)
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        // Sum over the 16 super-block lanes of each row (lanes j + 4q) while
        // spreading the 4 tokens over the lanes: after the xor-32 and xor-16
        // exchanges lane bits 5..4 select the token, and the xor-8 and xor-4
        // sums finish; lanes with bits 3..2 clear store.
        const bool b5 = (lane & 32) != 0, b4 = (lane & 16) != 0;
        const long row = rq * 4 + j;
#pragma unroll
        for (int t = 0; t < TG; t++) {
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; r++) v[r] = fmaf(-dmin, mn[t][r], acc[t][r]);
            const float k0 = b5 ? v[2] : v[0], k1 = b5 ? v[3] : v[1];
            const float s0 = b5 ? v[0] : v[2], s1 = b5 ? v[1] : v[3];
            const float w0 = k0 + __shfl_xor(s0, 32), w1 = k1 + __shfl_xor(s1, 32);
            float u = (b4 ? w1 : w0) + __shfl_xor(b4 ? w0 : w1, 16);
            u += __shfl_xor(u, 8);
            u += __shfl_xor(u, 4);
            const int m = 4 * t + (lane >> 4);
            if ((lane & 12) == 0 && m < M && row < N) a.y[(size_t)m * N + row] = u;
        }
    };

    // row quads in pairs: each tile buffer is loaded while the other is computed
    for (long rq = rq0; rq < rq1; rq += 2) {
        if (rq + 1 < rq1) load(rq + 1, tb);
        compute(rq, ta);
        if (rq + 1 >= rq1) break;
        if (rq + 2 < rq1) load(rq + 2, ta);
        compute(rq + 1, tb);
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
    a.nrq = ((long)N + 3) / 4;
    const int TG = rq_tg(M);
    a.tok_stride = (int)rq_tok_stride(K);
    a.sc_stride = 8 * 4 * TG + 4;
    // whole row quads per wave, as few per wave as lets every workgroup be
    // resident at once (register-limited: 12 waves per CU at TG 1, 8 at TG 2)
    const long target = (long)device_cu_count() * (TG == 1 ? 12 : 8);
    a.per_wave = (int)((a.nrq + target - 1) / target);
    const long waves = (a.nrq + a.per_wave - 1) / a.per_wave;
    const unsigned grid = (unsigned)((waves + kRqWaves - 1) / kRqWaves);
    const size_t shm = rq_lds(M, K);
    if (TG == 1) hipLaunchKernelGGL(gemv_q4k_rq<1>, dim3(grid), dim3(64 * kRqWaves), shm, st, a);
    else hipLaunchKernelGGL(gemv_q4k_rq<2>, dim3(grid), dim3(64 * kRqWaves), shm, st, a);
    return hipGetLastError();
}

}  // namespace lp
