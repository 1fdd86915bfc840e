// lp_gemm_i8.hip - prefill GEMM for Q4_K weights on int8 MFMA (M >= 128).
//
// Reference semantics: gemm_int<dot_row_q4_k_int_neon> row by row
// (src/matmul_simd.cpp:226-283, 432-455):
//   y[m,n] = sum_sb [ sum_{b in sb} (d_n sc_nb) * xd_mb * P_mnb
//                     - dmin_n * sum_{b in sb} mn_nb * xs_mb ]
// with P_mnb = sum_{k in b} nib_nk * q_mk the exact int32 block sum of the
// ActQ8 codes q (src/matmul_simd.cpp:348-410) against the weight nibbles.
//
// P is what v_mfma_i32_32x32x32_i8 computes for one 32-element block (A =
// the tokens' int8 codes, B = the weights' 4-bit codes as int8, D lane =
// weight row n, 16 tokens), bit-exact. The block scales are applied by the
// VALU per output and block: acc += float(P) * (xd' * d sc) (three
// operations), with xd' = xd * 2^-E_m (E_m the exponent of the row's largest
// block scale, a power-of-two shift that keeps the min term's fp16 operands in
// range). The min term is one fp16 MFMA per super-block (xs' = xs 2^-E_m as
// an fp16 hi + lo pair against the exact 6-bit m), and y = acc * 2^E_m. So
// the products are the reference's integers and only the fp32 accumulation
// order differs.
//
// Operands in HBM: the ActQ8 codes qs [M][K] as the quantizer wrote them
// (lane l of a block's A fragment takes bytes 16(l/32)..+16 of the block for
// token l%32: the nibble order of the 32-byte code chunk, low nibbles block
// 2jb, high 2jb+1); XD [K/64][2][Mp] f32 (xd' of the step's two blocks, token
// fastest); SX [K/256][Mp][2][8] fp16 (xs' hi, lo of the super-block's 8
// blocks); escale [Mp].
//
// Tiling: 4 waves, tile 128 tokens x 128 weight rows, wave (th, rq) = (w&1,
// w>>1) takes tokens 64th..+64 and rows 64rq..+64 (2 x 2 MFMA tiles); two
// workgroups per CU. Per 64-element K step the workgroup copies the 8 KiB of
// codes of its tokens, the 4 KiB of weight codes and 1 KiB of block scales
// into LDS (buffer_load_dwordx4 ... lds, NS stages), headers and min-term
// operands once per super-block.
#include <hip/hip_runtime.h>

#include "lp_chunks.h"
#include "lp_internal.h"

namespace lp {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef int i16v __attribute__((ext_vector_type(16)));
typedef int i4v __attribute__((ext_vector_type(4)));
typedef float f4v __attribute__((ext_vector_type(4)));

constexpr int kBm = 128, kBn = 128, kNw = 4;
constexpr int kQ = 8192, kCodes = 4096, kXd = 1024;
constexpr int kStage = kQ + kCodes + kXd;              // 13 KiB
constexpr int kHdr = kBn * 16, kSx = 4 * 1024;
constexpr int kSbuf = kHdr + kSx;                      // 6 KiB
constexpr int kNs = 4;
constexpr int kLds = kNs * kStage + 2 * kSbuf + kNw * 64 * 4;

struct I8Args {
    const int8_t* qs;
    const uint8_t* xd;        // XD plane
    const uint8_t* sx;        // SX plane
    const float* escale;
    const uint8_t* w;
    size_t rb;
    float* y;
    int M, N, K, Mp;
    int ntm, ntn;
    int nfull;                // tiles [0, nfull) whole; later tiles split in two halves of K
};

__device__ __forceinline__ uint32_t lds_addr(const uint8_t* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint8_t*)p;
}
// LDS reads as inline assembly with explicit lgkmcnt waits (a compiler-
// generated ds_read after direct-to-LDS copies waits for every copy in flight).
template <int OFF>
__device__ __forceinline__ void rd128(u32x4& o, uint32_t a) {
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(o) : "v"(a), "n"(OFF));
}
template <int OFF>
__device__ __forceinline__ void rd128f(f4v& o, uint32_t a) {
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(o) : "v"(a), "n"(OFF));
}
template <int N>
__device__ __forceinline__ void lgkm() {
    asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ uint32_t sc6(uint32_t hy, uint32_t hw, int j) {
    return j < 4 ? __builtin_amdgcn_ubfe(hy, 8 * j, 6)
                 : __builtin_amdgcn_ubfe(hw, 8 * (j - 4), 4) | (__builtin_amdgcn_ubfe(hy, 8 * (j - 4) + 6, 2) << 4);
}
__device__ __forceinline__ uint32_t m6(uint32_t hz, uint32_t hw, int j) {
    return j < 4 ? __builtin_amdgcn_ubfe(hz, 8 * j, 6)
                 : __builtin_amdgcn_ubfe(hw, 8 * (j - 4) + 4, 4) | (__builtin_amdgcn_ubfe(hz, 8 * (j - 4) + 6, 2) << 4);
}

struct I8Plan {
    Rsrc rs_q, rs_w, rs_xd, rs_sx;
    uint32_t q_off[2], code_off, hdr_off, xd_off, sx_off;
};

// Copies of wave w (step kt): the codes of token tile w (two blocks, 2 KiB),
// row tile w's weight codes (1 KiB), and on wave 0 the step's block scales;
// per super-block token tile w's min-term operands and, on waves 0-1, the
// headers of rows 64w..+64. i = 0..3 step copies, 4..5 super-block copies.
__device__ __forceinline__ void i8_issue(const I8Plan& d, int wave, int kt, int Mp, uint8_t* st, uint8_t* sbb,
                                         int i) {
    const int sb = kt >> 2, jb = kt & 3;
    if (i < 2) dma16(d.rs_q, d.q_off[i], (uint32_t)(kt * 64), st + (wave * 2 + i) * 1024);
    else if (i == 2) dma16(d.rs_w, d.code_off, (uint32_t)(sb * 144 + 32 * jb), st + kQ + wave * 1024);
    else if (i == 3) {
        if (wave == 0) dma16(d.rs_xd, d.xd_off, (uint32_t)(kt * 2 * Mp * 4), st + kQ + kCodes);
    } else if (jb == 0) {
        if (i == 4) dma16(d.rs_sx, d.sx_off, (uint32_t)(sb * Mp * 32), sbb + kHdr + wave * 1024);
        else if (wave < 2) dma16(d.rs_w, d.hdr_off, (uint32_t)(sb * 144), sbb + wave * 1024);
    }
}
__device__ __forceinline__ int i8_count(int k, int nk, int wave) {
    if (k >= nk) return 0;
    return 3 + (wave == 0) + ((k & 3) == 0 ? 1 + (wave < 2) : 0);
}

__global__ void __launch_bounds__(256, 2) __attribute__((amdgpu_waves_per_eu(2, 2)))
gemm_q4k_i8(I8Args g) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int th = wave & 1, rq = wave >> 1;
    const int bid = blockIdx.x;
    int tile, part = 0, ksplit = 1;
    if (bid < g.nfull) {
        tile = (g.nfull & 7) == 0 ? (bid & 7) * (g.nfull >> 3) + (bid >> 3) : bid;
    } else {
        tile = g.nfull + ((bid - g.nfull) >> 1);
        part = (bid - g.nfull) & 1;
        ksplit = 2;
    }
    // pairs of token tiles walk the weight tiles together (shared in L2)
    int tm, tn;
    {
        const int per = 2 * g.ntn, grp = tile / per, in = tile % per;
        const int gm = g.ntm - grp * 2 < 2 ? g.ntm - grp * 2 : 2;
        tm = grp * 2 + in % gm;
        tn = in / gm;
    }
    const int m0 = tm * kBm, n0 = tn * kBn;
    const int nsb_all = g.K >> 8;
    const int sb_beg = part * nsb_all / ksplit, sb_end = (part + 1) * nsb_all / ksplit;
    const int kt0 = 4 * sb_beg, nk = 4 * sb_end;

    I8Plan d;
    {
        const int mt = g.M - m0 < kBm ? g.M - m0 : kBm;
        const int nt = g.N - n0 < kBn ? g.N - n0 : kBn;
        d.rs_q = make_rsrc(g.qs + (size_t)m0 * g.K, (uint32_t)((size_t)mt * g.K));
        d.rs_w = make_rsrc(g.w + (size_t)n0 * g.rb, (uint32_t)((size_t)nt * g.rb));
        d.rs_xd = make_rsrc(g.xd, (uint32_t)((size_t)(g.K >> 6) * 2 * g.Mp * 4));
        d.rs_sx = make_rsrc(g.sx, (uint32_t)((size_t)nsb_all * g.Mp * 32));
        int tok = wave * 32 + (lane & 31);
        tok = tok < mt ? tok : mt - 1;
#pragma unroll
        for (int h = 0; h < 2; h++) d.q_off[h] = (uint32_t)(tok * g.K + 32 * h + 16 * (lane >> 5));
        int row = wave * 32 + (lane & 31);
        row = row < nt ? row : nt - 1;
        d.code_off = (uint32_t)((size_t)row * g.rb) + 16 + 16 * (lane >> 5);
        int hrow = (wave & 1) * 64 + lane;
        hrow = hrow < nt ? hrow : nt - 1;
        d.hdr_off = (uint32_t)((size_t)hrow * g.rb);
        d.xd_off = (uint32_t)((((lane >> 5) * g.Mp) + m0 + 4 * (lane & 31)) * 4);
        d.sx_off = (uint32_t)((m0 + wave * 32 + (lane & 31)) * 32 + 16 * (lane >> 5));
    }
    auto stage = [&](int i) { return smem + i * kStage; };
    auto sbuf = [&](int i) { return smem + kNs * kStage + i * kSbuf; };

    const uint32_t lds0 = lds_addr(smem);
    const int gl = lane >> 5;
    const uint32_t aq = lds0 + lane * 16 + th * 4096;                 // + t*2048 + h*1024
    const uint32_t ac = lds0 + kQ + lane * 16 + rq * 2048;            // + r*1024
    const uint32_t ax = lds0 + kQ + kCodes + (th * 64 + 4 * gl) * 4;   // + h*512 + t*128 + q*32
    const uint32_t ah = lds0 + kNs * kStage + (rq * 64 + (lane & 31)) * 16;   // + r*512
    const uint32_t as = lds0 + kNs * kStage + kHdr + th * 2048 + lane * 16;   // + t*1024

    f16v acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[a][b][r] = 0.0f;
    uint32_t hy[2], hz[2], hw[2];
    float dd[2], dmn[2];

#pragma unroll
    for (int i = 0; i < kNs - 1; i++)
        if (kt0 + i < nk)
#pragma unroll
            for (int p = 0; p < 6; p++) i8_issue(d, wave, kt0 + i, g.Mp, stage(i), sbuf(((kt0 + i) >> 2) & 1), p);

    for (int sb = sb_beg; sb < sb_end; sb++) {
        const uint32_t sbo = (uint32_t)((sb & 1) * kSbuf);
#pragma unroll 1
        for (int jb = 0; jb < 4; jb++) {
            const int kt = 4 * sb + jb;
            int later = 0;
#pragma unroll
            for (int i = 1; i < kNs - 1; i++) later += i8_count(kt + i, nk, wave);
            wait_dma(later);
            __builtin_amdgcn_s_barrier();
            const bool pf = kt + kNs - 1 < nk;
            uint8_t* const pst = stage((kt + kNs - 1 - kt0) % kNs);
            uint8_t* const psb = sbuf(((kt + kNs - 1) >> 2) & 1);
            const uint32_t so = (uint32_t)(((kt - kt0) % kNs) * kStage);

            if (jb == 0) {
                u32x4 h0, h1;
                rd128<0>(h0, ah + sbo);
                rd128<512>(h1, ah + sbo);
                lgkm<0>();
                asm volatile("" : "+v"(h0), "+v"(h1));
                const u32x4 hh[2] = {h0, h1};
#pragma unroll
                for (int r = 0; r < 2; r++) {
                    dd[r] = fp16_bits_to_f32(hh[r].x);
                    dmn[r] = fp16_bits_to_f32(hh[r].x >> 16);
                    hy[r] = hh[r].y;
                    hz[r] = hh[r].z;
                    hw[r] = hh[r].w;
                }
            }
            // per block scale d*sc of this lane's rows (the reference's d * sc1)
            float dsc[2][2];
#pragma unroll
            for (int r = 0; r < 2; r++)
#pragma unroll
                for (int h = 0; h < 2; h++) dsc[r][h] = dd[r] * (float)sc6(hy[r], hw[r], 2 * jb + h);

            u32x4 Q[2][2], C[2];
            rd128<0>(C[0], ac + so);
            rd128<1024>(C[1], ac + so);
            rd128<0>(Q[0][0], aq + so);
            rd128<1024>(Q[0][1], aq + so);
            rd128<2048>(Q[1][0], aq + so);
            rd128<3072>(Q[1][1], aq + so);
            lgkm<0>();
#pragma unroll
            for (int r = 0; r < 2; r++) asm volatile("" : "+v"(C[r]));
#pragma unroll
            for (int t = 0; t < 2; t++) asm volatile("" : "+v"(Q[t][0]), "+v"(Q[t][1]));

#pragma unroll
            for (int h = 0; h < 2; h++) {
                // block scales of this lane's 16 tokens per tile for block h:
                // tokens 8q + 4(l/32) + i, four float4 reads each
                f4v X[2][4];
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const uint32_t xa = ax + so + h * 512 + t * 128;
                    rd128f<0>(X[t][0], xa);
                    rd128f<32>(X[t][1], xa);
                    rd128f<64>(X[t][2], xa);
                    rd128f<96>(X[t][3], xa);
                }
                lgkm<0>();
#pragma unroll
                for (int t = 0; t < 2; t++)
#pragma unroll
                    for (int q = 0; q < 4; q++) asm volatile("" : "+v"(X[t][q]));
#pragma unroll
                for (int r = 0; r < 2; r++) {
                    // block 2jb: low nibbles; 2jb+1: high nibbles (as int8 0..15)
                    i4v B;
#pragma unroll
                    for (int c = 0; c < 4; c++)
                        B[c] = (int)((h ? (C[r][c] >> 4) : C[r][c]) & 0x0f0f0f0fu);
#pragma unroll
                    for (int t = 0; t < 2; t++) {
                        const i4v A = __builtin_bit_cast(i4v, Q[t][h]);
                        const i16v P = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, i16v{}, 0, 0, 0);
#pragma unroll
                        for (int i = 0; i < 16; i++)
                            acc[t][r][i] = fmaf((float)P[i], X[t][i >> 2][i & 3] * dsc[r][h], acc[t][r][i]);
                        // one block product in flight per wave: its 16 sums are
                        // consumed before the next MFMA (the other wave on the
                        // SIMD fills the MFMA's latency)
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
            }
            if (pf) {
#pragma unroll
                for (int i = 0; i < 6; i++) i8_issue(d, wave, kt + kNs - 1, g.Mp, pst, psb, i);
            }
            if (jb == 3) {
                // min term: sum_b m_b * (xs'_hi + xs'_lo)_b, one K = 16 fp16 product
                u32x4 S0, S1;
                rd128<0>(S0, as + sbo);
                rd128<1024>(S1, as + sbo);
                h8 mb[2];
#pragma unroll
                for (int r = 0; r < 2; r++)
#pragma unroll
                    for (int j = 0; j < 8; j++) mb[r][j] = (_Float16)(float)m6(hz[r], hw[r], j);
                lgkm<0>();
                asm volatile("" : "+v"(S0), "+v"(S1));
                const h8 S[2] = {__builtin_bit_cast(h8, S0), __builtin_bit_cast(h8, S1)};
#pragma unroll
                for (int r = 0; r < 2; r++)
#pragma unroll
                    for (int t = 0; t < 2; t++) {
                        const f16v mm = __builtin_amdgcn_mfma_f32_32x32x16_f16(S[t], mb[r], f16v{}, 0, 0, 0);
#pragma unroll
                        for (int i = 0; i < 16; i++) acc[t][r][i] = fmaf(-dmn[r], mm[i], acc[t][r][i]);
                    }
            }
        }
    }

    // D[token][row] -> y[token * N + row] * 2^E_token
    const int mw = m0 + th * 64;
    float* esl = reinterpret_cast<float*>(smem + kNs * kStage + 2 * kSbuf) + wave * 64;
    esl[lane] = mw + lane < g.M ? g.escale[mw + lane] : 0.0f;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const int n = n0 + rq * 64 + r * 32 + (lane & 31);
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int ml = t * 32 + 8 * (i >> 2) + 4 * gl + (i & 3);
                const int m = mw + ml;
                if (m < g.M && n < g.N) {
                    const float val = acc[t][r][i] * esl[ml];
                    if (ksplit == 1) g.y[(size_t)m * g.N + n] = val;
                    else atomicAdd(&g.y[(size_t)m * g.N + n], val);
                }
            }
    }
}

// Scale planes from the quantized blocks, one wave per token row (rows
// M..Mp-1: zeros, escale 1): E from the largest block scale (fmaxf skips a
// NaN block's scale), XD[ks][h][m] = d * 2^-E, SX[sb][m] = fp16 hi/lo of
// xs * 2^-E for the 8 blocks.
__global__ void __launch_bounds__(256) i8_prep_kernel(ActView A, int M, int Mp, int K, float* __restrict__ xd,
                                                      _Float16* __restrict__ sx, float* __restrict__ escale) {
#pragma clang fp contract(off)
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (m >= Mp) return;
    const int lane = threadIdx.x & 63, nb = K >> 5;
    const float* dr = A.d + (size_t)m * nb;
    const float* sr = A.sum + (size_t)m * nb;
    float mx = 0.0f;
    if (m < M) {
        for (int b = lane; b < nb; b += 64) mx = fmaxf(mx, fabsf(dr[b]));
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    }
    const int e = row_exponent(mx);
    const float inv = ldexpf(1.0f, -e);
    if (lane == 0) escale[m] = ldexpf(1.0f, e);
    for (int b = lane; b < nb; b += 64) {
        const float dv = m < M ? dr[b] * inv : 0.0f;
        float xs = m < M ? sr[b] * inv : 0.0f;
        xd[((size_t)(b >> 1) * 2 + (b & 1)) * Mp + m] = dv;
        asm volatile("" : "+v"(xs));
        const _Float16 hi = (_Float16)xs;
        const size_t o = ((size_t)(b >> 3) * Mp + m) * 16 + (b & 7);
        sx[o] = hi;
        sx[o + 8] = (_Float16)(xs - (float)hi);
    }
}

__global__ void __launch_bounds__(256) i8_zero_kernel(float* __restrict__ y, size_t n) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) y[i] = 0.0f;
}

size_t up256(size_t v) { return (v + 255) & ~size_t(255); }

}  // namespace

static int i8_mp(int M) { return (M + kBm - 1) / kBm * kBm; }

size_t gemm_i8_planes_bytes(int M, int K) {
    const size_t Mp = (size_t)i8_mp(M);
    return up256(Mp * (K / 32) * 4) + up256(Mp * (K / 256) * 32) + up256(Mp * 4);
}

bool gemm_i8_supported(uint32_t type, int M, int K) {
    return type == T_Q4_K && M >= kBm && K % 256 == 0 && K <= 32768;
}

hipError_t launch_gemm_i8(const uint8_t* w, const ActView& A, void* planes, float* y, int M, int K, int N,
                          hipStream_t st) {
    if (M <= 0 || N <= 0) return hipSuccess;
    const int Mp = i8_mp(M);
    uint8_t* p = static_cast<uint8_t*>(planes);
    float* xd = reinterpret_cast<float*>(p);
    p += up256((size_t)Mp * (K / 32) * 4);
    _Float16* sx = reinterpret_cast<_Float16*>(p);
    p += up256((size_t)Mp * (K / 256) * 32);
    float* es = reinterpret_cast<float*>(p);
    hipLaunchKernelGGL(i8_prep_kernel, dim3(Mp / 4), dim3(256), 0, st, A, M, Mp, K, xd, sx, es);

    const int ntm = Mp / kBm, ntn = (N + kBn - 1) / kBn, ntiles = ntm * ntn;
    // tiles beyond the last full round of two workgroups per CU, when at most
    // half a round, are split in K (their halves fill that round)
    const int slots = 2 * device_cu_count();
    const int rem = slots > 0 ? ntiles % slots : 0;
    const int nfull = (rem > 0 && 2 * rem <= slots && (K >> 8) >= 2) ? ntiles - rem : ntiles;
    if (nfull < ntiles) {
        const size_t first = (size_t)(nfull / ntn) * kBm * N, n = (size_t)M * N - first;
        hipLaunchKernelGGL(i8_zero_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, y + first, n);
    }
    I8Args g{A.qs, reinterpret_cast<const uint8_t*>(xd), reinterpret_cast<const uint8_t*>(sx), es, w,
             row_bytes(T_Q4_K, K), y, M, N, K, Mp, ntm, ntn, nfull};
    const long nblk = (long)nfull + 2L * (ntiles - nfull);
    hipLaunchKernelGGL(gemm_q4k_i8, dim3((unsigned)nblk), dim3(256), kLds, st, g);
    return hipGetLastError();
}

}  // namespace lp
