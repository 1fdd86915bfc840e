// lp_gemm_fr.hip - prefill GEMM for Q4_K weights (M >= 128 tokens) on planes
// stored in MFMA fragment order.
//
// Reference semantics: gemm_int<dot_row_q4_k_int_neon> row by row
// (src/matmul_simd.cpp:226-283, 432-455):
//   y[m,n] = sum_sb [ d_n * sum_{b in sb} sc_nb * xd_mb * P_mnb
//                     - dmin_n * sum_{b in sb} mn_nb * xs_mb ]
// with P_mnb = sum_{k in b} nib_nk * q_mk and xd/xs/q the ActQ8 activation
// blocks (src/matmul_simd.cpp:348-410).
//
// Operands (the split-precision folding of the block scales):
//   t[m,k]  = xd_mb * q_mk * 2^(9 - E_m)   (E_m: exponent of the row's largest
//             block scale, so |t| <= 65024)
//   hi      = fp16(t),  lo = e4m3(t - hi)      (activation planes)
//   V[n,k]  = sc_nb * nib_nk / 4  (exact in fp16),  V8 = e4m3(V)
// main_sb = sum_k hi*V (fp16 MFMA, exact products) + sum_k lo*V8 (fp8 MFMA),
// and per super-block acc += d_n * 2^-7 * main_sb - dmin_n * min_sb with
// min_sb = sum_b m_nb * xs_mb * 2^-E_m (xs split into fp16 hi + lo, one fp16
// MFMA against the exact 6-bit m). y = acc * 2^E_m. The residual term leaves
// a per-product error below 2^-14 of |t*V|.
//
// Fragment-order planes. The activation planes are written by this file's
// planes kernel in the exact order the MFMA lanes read them, so every copy is
// a contiguous 1 KiB piece and every LDS read is lane-linear (no swizzle, no
// bank conflicts). Within a 64-element K step, lane half g (lane / 32),
// sub-step s (0..3) and position p (0..7) hold element
//   e(g, s, p) = 16g + 4s + perm(p & 3) + (p >= 4 ? 32 : 0),  perm = {0,2,1,3}
// which is what the weight decode produces from the 16 code bytes 16g..16g+15
// of the step's 32-byte code chunk (dword s of them: low nibbles are elements
// 0..31 of the step, high nibbles 32..63, src/matmul_simd.cpp:240-262). The
// MFMAs pair A and B values of the same lane half and position, so the sums
// are those of the natural order.
//   HI [T][ks][s][lane][8 fp16]       T = 32-token tile, ks = 64-element K step
//   LO [T][ks][h][lane][16 e4m3]      byte 8s + p of a lane's 32, half h = byte/16
//   SX [T][sb][lane][8 fp16]          lanes 0-31: fp16(xs 2^-E) of the token's
//                                     8 blocks of super-block sb; 32-63: residuals
//   escale [Mp]                       2^E_m
//
// GEMM tiling: a workgroup is 4 waves and a tile of 128 tokens x 256 weight
// rows; wave w owns every token of the tile and weight rows 64w..64w+63
// (4 x 2 MFMA tiles of 32 x 32: A = activations, B = weights, D lane = weight
// row). Each wave decodes only its own rows and reads the shared activation
// tile from LDS: 96 B of LDS per token per K step against 1536 MFMA cycles,
// half of the LDS bytes per MFMA of a 32-row wave. Per K step the wave copies
// one token tile's planes (6 KiB) and its two row tiles' codes (2 KiB) into
// LDS with buffer_load_dwordx4 ... lds; headers and min-term planes once per
// super-block. NS stages in flight, one barrier per K step, one workgroup per
// CU (LDS NS x 32 KiB + 16 KiB).
#include <hip/hip_runtime.h>

#include "lp_chunks.h"
#include "lp_internal.h"

namespace lp {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef int i8x32 __attribute__((ext_vector_type(8)));   // 32 fp8 bytes

constexpr int kTm = 4;            // 32-token tiles per workgroup
constexpr int kTmW = 2;           // 32-token tiles per wave (token half th = wave & 1)
constexpr int kRt = 2;            // 32-row tiles per wave (row half rq = wave >> 1)
constexpr int kNw = 4;            // waves; two workgroups per CU
constexpr int kBm = 32 * kTm, kBn = 32 * kRt * (kNw * kTmW / kTm);
constexpr int kHi = kTm * 4096, kLo = kTm * 2048, kCodes = (kBn / 32) * 1024;
constexpr int kStage = kHi + kLo + kCodes;                   // 28 KiB
constexpr int kHdr = kBn * 16, kSx = kTm * 1024;
constexpr int kSbuf = kHdr + kSx;                            // 6 KiB
constexpr int kDmaStep = 7;                                  // per wave and K step
static_assert(kHi / 1024 + kLo / 1024 + kCodes / 1024 == kNw * kDmaStep, "copies split evenly");
static_assert(kSx / 1024 == kNw && kHdr / 1024 == 2, "super-block copies: one min-term piece per wave, "
                                                      "headers on waves 0-1");

struct FrArgs {
    const uint8_t* hi;
    const uint8_t* lo;
    const uint8_t* sx;
    const float* escale;
    const uint8_t* w;
    size_t rb;
    float* y;
    int M, N, K;
    int ntm, ntn;       // token / row tiles of the grid
    int tiles_pad;      // 32-token tiles of the planes (Mp / 32)
    int nfull;          // tiles [0, nfull) run whole; each later tile is two workgroups,
                        // one per half of K, adding into a zeroed y (two fp32 additions
                        // onto 0 give the same sum in either order)
};

__device__ __forceinline__ uint32_t lds_addr(const uint8_t* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint8_t*)p;
}
// LDS reads as inline assembly with explicit lgkmcnt waits: a compiler-
// generated ds_read after direct-to-LDS copies makes the compiler wait for
// every copy in flight (vmcnt(0)), the prefetches of later steps included.
template <int OFF>
__device__ __forceinline__ void rd128(u32x4& o, uint32_t a) {
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(o) : "v"(a), "n"(OFF));
}
template <int OFF>
__device__ __forceinline__ void rd128h(h8& o, uint32_t a) {
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(o) : "v"(a), "n"(OFF));
}
template <int N, typename V, int T>
__device__ __forceinline__ void lgkm(V (&a)[T]) {
    asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N) : "memory");
#pragma unroll
    for (int i = 0; i < T; i++) asm volatile("" : "+v"(a[i]));
}

// One dword of codes (bytes b0..b3) -> 8 fp16 V in positions
// [lo b0, lo b2, lo b1, lo b3, hi b0, hi b2, hi b1, hi b3]: masking nibbles
// into fp16 1024 + n (low) or 1024 + 16n (high) and one packed fma each,
// (h - 1024) * sc/4 (or sc/64), exact.
__device__ __forceinline__ h8 decode4(uint32_t u, h2 ml, h2 al, h2 mh, h2 ah) {
    const uint32_t u8 = u >> 8;
    uint32_t a, b, c, d;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(a) : "v"(0x000f000fu), "v"(u), "s"(0x64006400u));
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(b) : "v"(0x000f000fu), "v"(u8), "s"(0x64006400u));
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(c) : "v"(0x00f000f0u), "v"(u), "s"(0x64006400u));
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(d) : "v"(0x00f000f0u), "v"(u8), "s"(0x64006400u));
    const h2 va = __builtin_elementwise_fma(__builtin_bit_cast(h2, a), ml, al);
    const h2 vb = __builtin_elementwise_fma(__builtin_bit_cast(h2, b), ml, al);
    const h2 vc = __builtin_elementwise_fma(__builtin_bit_cast(h2, c), mh, ah);
    const h2 vd = __builtin_elementwise_fma(__builtin_bit_cast(h2, d), mh, ah);
    return h8{va[0], va[1], vb[0], vb[1], vc[0], vc[1], vd[0], vd[1]};
}

__device__ __forceinline__ uint32_t e4m3x4(uint32_t h01, uint32_t h23) {
    uint32_t w;
    asm("v_cvt_scalef32_pk_fp8_f16 %0, %1, 1.0\n\tv_cvt_scalef32_pk_fp8_f16 %0, %2, 1.0 op_sel:[0,0,1]"
        : "=&v"(w) : "v"(h01), "v"(h23));
    return w;
}

// 6-bit scale j of a Q4_K header (words hy = scales[0..3], hz = [4..7],
// hw = [8..11]); get_scale_min_k4 (src/kernels.h:82-90).
__device__ __forceinline__ uint32_t q4k_sc(uint32_t hy, uint32_t hw, int j) {
    return j < 4 ? __builtin_amdgcn_ubfe(hy, 8 * j, 6)
                 : __builtin_amdgcn_ubfe(hw, 8 * (j - 4), 4) | (__builtin_amdgcn_ubfe(hy, 8 * (j - 4) + 6, 2) << 4);
}
__device__ __forceinline__ uint32_t q4k_m(uint32_t hz, uint32_t hw, int j) {
    return j < 4 ? __builtin_amdgcn_ubfe(hz, 8 * j, 6)
                 : __builtin_amdgcn_ubfe(hw, 8 * (j - 4) + 4, 4) | (__builtin_amdgcn_ubfe(hz, 8 * (j - 4) + 6, 2) << 4);
}

// Per wave: copy sources fixed for the tile; a step changes scalar offsets.
// Wave w copies token tile w's hi (four 1 KiB pieces per step) and lo (two)
// planes and row tile w's codes (one), and per super-block token tile w's
// min-term planes; waves 0-1 also the headers of rows 64w..+64.
struct FrPlan {
    Rsrc rs_hi, rs_lo, rs_w, rs_sx;
    uint32_t code_off, hdr_off;
};

// Copy i of K step kt into stage `st` (i = 0..6), or of the super-block that
// kt starts into `sbb` (i = 7: min-term planes, 8: headers). The copies move
// through the CU's vector-memory path at ~64 B per clock and a wave's issue
// waits for it, so the compute loop spreads them over its fp8 MFMAs.
__device__ __forceinline__ void fr_issue(const FrPlan& d, int wave, int kt, uint8_t* st, uint8_t* sbb, int i) {
    const uint32_t lane16 = (threadIdx.x & 63) * 16;
    const int sb = kt >> 2, jb = kt & 3;
    if (i < 4) dma16(d.rs_hi, lane16, (uint32_t)(kt * 4096 + i * 1024), st + wave * 4096 + i * 1024);
    else if (i < 6) dma16(d.rs_lo, lane16, (uint32_t)(kt * 2048 + (i - 4) * 1024), st + kHi + wave * 2048 + (i - 4) * 1024);
    else if (i == 6) dma16(d.rs_w, d.code_off, (uint32_t)(sb * 144 + 32 * jb), st + kHi + kLo + wave * 1024);
    else if (jb == 0) {
        if (i == 7) dma16(d.rs_sx, lane16, (uint32_t)(sb * 1024), sbb + kHdr + wave * 1024);
        else if (wave < 2) dma16(d.rs_w, d.hdr_off, (uint32_t)(sb * 144), sbb + wave * 1024);
    }
}

__device__ __forceinline__ int fr_count(int k, int nk, int wave) {
    return k < nk ? kDmaStep + ((k & 3) == 0 ? (wave < 2 ? 2 : 1) : 0) : 0;
}

template <int NS>
__global__ void __launch_bounds__(64 * kNw, 2) __attribute__((amdgpu_waves_per_eu(2, 2)))
gemm_q4k_fr(FrArgs g) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int th = wave & 1, rq = wave >> 1;
    // blocks are dealt to the 8 XCDs round-robin, so each XCD gets a
    // contiguous run of whole tiles (the workgroups in flight on one XCD share
    // operands in its L2); split tiles (g.nfull == 0) come in K-half pairs.
    const int bid = blockIdx.x;
    int tile, part = 0, ksplit = 1;
    if (bid < g.nfull) {
        tile = (g.nfull & 7) == 0 ? (bid & 7) * (g.nfull >> 3) + (bid >> 3) : bid;
    } else {
        tile = g.nfull + ((bid - g.nfull) >> 1);
        part = (bid - g.nfull) & 1;
        ksplit = 2;
    }
    // pairs of token tiles walk the weight tiles together (the workgroups in
    // flight share both operands in L2)
    constexpr int GM = 2;
    int tm, tn;
    {
        const int per = GM * g.ntn, grp = tile / per, in = tile % per;
        const int gm = g.ntm - grp * GM < GM ? g.ntm - grp * GM : GM;
        tm = grp * GM + in % gm;
        tn = in / gm;
    }
    const int m0 = tm * kBm, n0 = tn * kBn;
    const int nsb_all = g.K >> 8, ks_all = g.K >> 6;
    const int sb_beg = part * nsb_all / ksplit, sb_end = (part + 1) * nsb_all / ksplit;
    const int kt0 = 4 * sb_beg, nk = 4 * sb_end;

    FrPlan d;
    {
        int T = tm * kTm + wave;                               // token tile this wave copies
        T = T < g.tiles_pad ? T : g.tiles_pad - 1;
        const int nt = g.N - n0 < kBn ? g.N - n0 : kBn;
        d.rs_w = make_rsrc(g.w + (size_t)n0 * g.rb, (uint32_t)((size_t)nt * g.rb));
        d.rs_hi = make_rsrc(g.hi + (size_t)T * ks_all * 4096, (uint32_t)(ks_all * 4096));
        d.rs_lo = make_rsrc(g.lo + (size_t)T * ks_all * 2048, (uint32_t)(ks_all * 2048));
        d.rs_sx = make_rsrc(g.sx + (size_t)T * nsb_all * 1024, (uint32_t)(nsb_all * 1024));
        int row = wave * 32 + (lane & 31);
        row = row < nt ? row : nt - 1;
        d.code_off = (uint32_t)((size_t)row * g.rb) + 16 + 16 * (lane >> 5);
        int hrow = (wave & 1) * 64 + lane;
        hrow = hrow < nt ? hrow : nt - 1;
        d.hdr_off = (uint32_t)((size_t)hrow * g.rb);
    }
    auto stage = [&](int i) { return smem + i * kStage; };
    auto sbuf = [&](int i) { return smem + NS * kStage + i * kSbuf; };

    const uint32_t lds0 = lds_addr(smem);
    const uint32_t l16 = lds0 + lane * 16 + th * (kTmW * 4096);     // + this wave's token tiles
    const uint32_t l16lo = lds0 + lane * 16 + kHi + th * (kTmW * 2048);
    const uint32_t l16c = lds0 + lane * 16 + kHi + kLo + rq * (kRt * 1024);
    const uint32_t hdr_a = lds0 + NS * kStage + (rq * 64 + (lane & 31)) * 16;   // + r * 512
    const uint32_t sx_a = lds0 + NS * kStage + kHdr + th * (kTmW * 1024) + lane * 16;

    f16v acc[kTmW][kRt], mn[kTmW][kRt];
#pragma unroll
    for (int a = 0; a < kTmW; a++)
#pragma unroll
        for (int b = 0; b < kRt; b++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[a][b][r] = 0.0f;

    uint32_t hy[kRt], hz[kRt], hw[kRt];
    float dsc[kRt], dmn[kRt];

    // prologue: steps kt0 .. kt0+NS-2 in flight
#pragma unroll
    for (int i = 0; i < NS - 1; i++)
        if (kt0 + i < nk)
#pragma unroll
            for (int p = 0; p < 9; p++) fr_issue(d, wave, kt0 + i, stage(i), sbuf(((kt0 + i) >> 2) & 1), p);

    for (int sb = sb_beg; sb < sb_end; sb++) {
        const uint32_t sbo = (uint32_t)((sb & 1) * kSbuf);
#pragma unroll
        for (int jb = 0; jb < 4; jb++) {
            const int kt = 4 * sb + jb;
            int later = 0;                       // copies of steps kt+1 .. kt+NS-2 (may stay in flight)
#pragma unroll
            for (int i = 1; i < NS - 1; i++) later += fr_count(kt + i, nk, wave);
            wait_dma(later);
            // after this barrier every wave has finished step kt-1, whose
            // stage is the one step kt+NS-1 is copied into
            __builtin_amdgcn_s_barrier();
            const bool pf = kt + NS - 1 < nk;
            uint8_t* const pst = stage((kt + NS - 1 - kt0) % NS);
            uint8_t* const psb = sbuf(((kt + NS - 1) >> 2) & 1);
            const uint32_t so = (uint32_t)(((kt - kt0) % NS) * kStage);

            if (jb == 0) {
                u32x4 h[kRt];
                rd128<0>(h[0], hdr_a + sbo);
                rd128<512>(h[1], hdr_a + sbo);
                lgkm<0>(h);
#pragma unroll
                for (int r = 0; r < kRt; r++) {
                    dsc[r] = fp16_bits_to_f32(h[r].x) * 0.0078125f;   // d * 2^-7 (main carries 2^7)
                    dmn[r] = fp16_bits_to_f32(h[r].x >> 16);
                    hy[r] = h[r].y;
                    hz[r] = h[r].z;
                    hw[r] = h[r].w;
                }
            }
            // decode constants: low nibbles block 2jb (sc/4), high 2jb+1 (sc/64)
            h2 ml[kRt], al[kRt], mh[kRt], ah[kRt];
#pragma unroll
            for (int r = 0; r < kRt; r++) {
                const float sl = (float)q4k_sc(hy[r], hw[r], 2 * jb) * 0.25f;
                const float sh = (float)q4k_sc(hy[r], hw[r], 2 * jb + 1) * (0.25f * 0.0625f);
                const _Float16 a = (_Float16)sl, b = (_Float16)(-1024.0f * sl);
                const _Float16 c = (_Float16)sh, e = (_Float16)(-1024.0f * sh);
                ml[r] = h2{a, a};
                al[r] = h2{b, b};
                mh[r] = h2{c, c};
                ah[r] = h2{e, e};
            }

            const uint32_t b = l16 + so;
            u32x4 cw[kRt];
            // the whole step's fragments are requested up front (14 LDS reads
            // in flight: codes, four hi sub-steps, the lo pair) and waited for
            // in order
            h8 A[4][kTmW];
            u32x4 L[kTmW][2];
            rd128<0>(cw[0], l16c + so);
            rd128<1024>(cw[1], l16c + so);
            rd128h<0>(A[0][0], b);
            rd128h<4096>(A[0][1], b);
            rd128h<1024>(A[1][0], b);
            rd128h<1024 + 4096>(A[1][1], b);
            rd128h<2048>(A[2][0], b);
            rd128h<2048 + 4096>(A[2][1], b);
            rd128h<3072>(A[3][0], b);
            rd128h<3072 + 4096>(A[3][1], b);
            rd128<0>(L[0][0], l16lo + so);
            rd128<1024>(L[0][1], l16lo + so);
            rd128<2048>(L[1][0], l16lo + so);
            rd128<3072>(L[1][1], l16lo + so);
            lgkm<12>(cw);
            uint32_t v8[kRt][8];
            // software-pipelined: sub-step s+1's weights are decoded (and s's
            // converted to e4m3) between sub-step s's MFMAs
            h8 Vc[kRt];
#pragma unroll
            for (int r = 0; r < kRt; r++) Vc[r] = decode4(cw[r][0], ml[r], al[r], mh[r], ah[r]);
#pragma unroll
            for (int s = 0; s < 4; s++) {
                if (s == 0) lgkm<10>(A[0]);
                else if (s == 1) lgkm<8>(A[1]);
                else if (s == 2) lgkm<6>(A[2]);
                else lgkm<4>(A[3]);
                h8 Vn[kRt];
#pragma unroll
                for (int r = 0; r < kRt; r++)
#pragma unroll
                    for (int t = 0; t < kTmW; t++)
                        mn[t][r] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[s][t], Vc[r],
                                                                          (jb == 0 && s == 0) ? f16v{} : mn[t][r],
                                                                          0, 0, 0);
                if (s < 3) {
#pragma unroll
                    for (int r = 0; r < kRt; r++) {
                        Vn[r] = decode4(cw[r][s + 1], ml[r], al[r], mh[r], ah[r]);
                    }
                }
#pragma unroll
                for (int r = 0; r < kRt; r++) {
                    const u32x4 q = __builtin_bit_cast(u32x4, Vc[r]);
                    v8[r][2 * s] = e4m3x4(q.x, q.y);
                    v8[r][2 * s + 1] = e4m3x4(q.z, q.w);
                }
#pragma unroll
                for (int i = 0; i < kRt * kTmW; i++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
                    __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);   // then up to four VALU
                }
                __builtin_amdgcn_sched_barrier(0);
                if (s < 3) {
#pragma unroll
                    for (int r = 0; r < kRt; r++) Vc[r] = Vn[r];
                }
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
            for (int t = 0; t < kTmW; t++) asm volatile("" : "+v"(L[t][0]), "+v"(L[t][1]));
#pragma unroll
            for (int r = 0; r < kRt; r++) {
                const i8x32 bv = {(int)v8[r][0], (int)v8[r][1], (int)v8[r][2], (int)v8[r][3],
                                  (int)v8[r][4], (int)v8[r][5], (int)v8[r][6], (int)v8[r][7]};
#pragma unroll
                for (int t = 0; t < kTmW; t++) {
                    const i8x32 av = {(int)L[t][0].x, (int)L[t][0].y, (int)L[t][0].z, (int)L[t][0].w,
                                      (int)L[t][1].x, (int)L[t][1].y, (int)L[t][1].z, (int)L[t][1].w};
                    mn[t][r] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, mn[t][r], 0, 0, 0, 0, 0, 0);
                    __builtin_amdgcn_sched_barrier(0);
                    if (pf) fr_issue(d, wave, kt + NS - 1, pst, psb, r * kTmW + t);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            if (pf) {
#pragma unroll
                for (int i = kRt * kTmW; i < 9; i++) fr_issue(d, wave, kt + NS - 1, pst, psb, i);
            }
            if (jb == 3) {
                // min term: sum_b m_b * (xs_hi + xs_lo)_b as one K = 16 product
                // (lanes 0-31: k = blocks 0..7 on the hi plane, 32-63: the same
                // blocks on the residual plane; B = the exact m in both halves)
                h8 S[kTmW];
                rd128h<0>(S[0], sx_a + sbo);
                rd128h<1024>(S[1], sx_a + sbo);
                h8 mb[kRt];
#pragma unroll
                for (int r = 0; r < kRt; r++)
#pragma unroll
                    for (int j = 0; j < 8; j++) mb[r][j] = (_Float16)(float)q4k_m(hz[r], hw[r], j);
                lgkm<0>(S);
#pragma unroll
                for (int r = 0; r < kRt; r++)
#pragma unroll
                    for (int t = 0; t < kTmW; t++) {
                        const f16v mm = __builtin_amdgcn_mfma_f32_32x32x16_f16(S[t], mb[r], f16v{}, 0, 0, 0);
#pragma unroll
                        for (int i = 0; i < 16; i++) {
                            acc[t][r][i] = fmaf(dsc[r], mn[t][r][i], acc[t][r][i]);
                            acc[t][r][i] = fmaf(-dmn[r], mm[i], acc[t][r][i]);
                        }
                    }
            }
        }
    }

    // D[token][row] -> y[token * N + row] * 2^E_token; the wave's 64 row
    // scales go through a wave-private LDS slot (one load wait, not one per output)
    const int mw = m0 + th * 32 * kTmW;
    float* esl = reinterpret_cast<float*>(smem + NS * kStage + 2 * kSbuf) + wave * 64;
    esl[lane] = mw + lane < g.M ? g.escale[mw + lane] : 0.0f;
    __builtin_amdgcn_wave_barrier();
    const int gl = lane >> 5;
#pragma unroll
    for (int r = 0; r < kRt; r++) {
        const int n = n0 + (rq * kRt + r) * 32 + (lane & 31);
#pragma unroll
        for (int t = 0; t < kTmW; t++)
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

// Row exponents: escale[m] = 2^E_m, E_m the exponent of fl(max_b amax_b / 127)
// over the row's blocks without a NaN (block scales are monotone in amax);
// rows M..Mp-1 get 1. One wave per row.
// From quantized blocks (ACT): the largest block scale of the row (fmaxf
// skips a NaN block's scale), the same value.
template <bool ACT>
__global__ void __launch_bounds__(256) fr_rowexp_kernel(const float* __restrict__ x, ActView Aq, int M, int Mp,
                                                        int K, float* __restrict__ escale) {
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (m >= Mp) return;
    const int lane = threadIdx.x & 63;
    float mx = 0.0f;
    if (ACT && m < M) {
        const float* dr = Aq.d + (size_t)m * (K >> 5);
        for (int b = lane; b < (K >> 5); b += 64) mx = fmaxf(mx, fabsf(dr[b]));
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    } else if (m < M) {
        const float4* xr = reinterpret_cast<const float4*>(x + (size_t)m * K);
        for (int i0 = lane; i0 < K / 4; i0 += 256) {
            // four loads in flight per lane (K / 4 is a multiple of 8; lanes past
            // the row's end take a zero)
            float4 uu[4];
#pragma unroll
            for (int c = 0; c < 4; c++) uu[c] = i0 + 64 * c < K / 4 ? xr[i0 + 64 * c] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int c = 0; c < 4; c++) {
            const float4 u = uu[c];
            float amax = fmaxf(fmaxf(fabsf(u.x), fabsf(u.y)), fmaxf(fabsf(u.z), fabsf(u.w)));
            uint32_t nan = (u.x != u.x) | (u.y != u.y) | (u.z != u.z) | (u.w != u.w);
#pragma unroll
            for (int o = 1; o < 8; o <<= 1) {
                amax = fmaxf(amax, __shfl_xor(amax, o, 8));
                nan |= __shfl_xor(nan, o, 8);
            }
            if (!nan) mx = fmaxf(mx, amax);
            }
        }
#pragma unroll
        for (int o = 8; o < 64; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    }
    if (!ACT) mx = mx / 127.0f;
    const int e = row_exponent(mx);
    if (lane == 0) escale[m] = ldexpf(1.0f, e);
}

// Planes of one 32-token tile and one super-block (grid: super-blocks x
// tiles), from fp32 x: quantize each 32-element block exactly as
// quantize_act_kernel does, form t = xd*q*2^(9-E) and its split, write the
// tile's fragment-order pieces to LDS, then copy them out with contiguous
// 16-byte stores (16 KiB HI, 8 KiB LO, 1 KiB SX). Wave w takes tokens
// 4w..4w+3, lane l elements 4l..4l+3 of the super-block (8 lanes per block).
// ACT: from the quantized blocks instead of x (codes, d and sum as stored).
template <bool ACT>
__global__ void __launch_bounds__(512) fr_planes_kernel(const float* __restrict__ x, ActView Aq, int M, int K,
                                                        const float* __restrict__ escale, uint8_t* __restrict__ hi,
                                                        uint8_t* __restrict__ lo, uint8_t* __restrict__ sx) {
#pragma clang fp contract(off)
    __shared__ __attribute__((aligned(16))) uint8_t t_hi[16384];
    __shared__ __attribute__((aligned(16))) uint8_t t_lo[8192];
    __shared__ __attribute__((aligned(16))) uint8_t t_sx[1024];
    const int sb = blockIdx.x, T = blockIdx.y;
    const int ks_all = K >> 6, nsb = K >> 8;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int ksl = lane >> 4;                    // K step within the super-block
    const int hin = (lane >> 3) & 1;              // elements 32..63 of the step (high nibbles)
    const int g = (lane >> 2) & 1, s = lane & 3;
    // the wave's four token rows requested together
    float4 xv[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int m = T * 32 + wave * 4 + j;
        xv[j] = (!ACT && m < M) ? *reinterpret_cast<const float4*>(x + (size_t)m * K + 256 * sb + 4 * lane)
                                : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int r = wave * 4 + j;               // token within the tile
        const int m = T * 32 + r;
        Q8Group q;
        if (ACT) {
            q.packed = 0;
            q.d = 0.0f;
            q.sum = 0.0f;
            if (m < M) {
                const size_t bi = (size_t)m * (K >> 5) + 8 * sb + (lane >> 3);
                q.packed = *reinterpret_cast<const uint32_t*>(Aq.qs + (size_t)m * K + 256 * sb + 4 * lane);
                q.d = Aq.d[bi];
                q.sum = Aq.sum[bi];
            }
        } else {
            q = quant_group8(xv[j]);
        }
        const float inv = 1.0f / escale[T * 32 + r];     // a power of two: exact
        const float ds = q.d * inv;
        _Float16 h[4], rl[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            float t = ds * (float)(int8_t)(q.packed >> (8 * c));
            t = t * 512.0f;
            asm volatile("" : "+v"(t));           // hi and lo both from fl32(t): no fused fp16 product
            h[c] = (_Float16)t;
            rl[c] = (_Float16)(t - (float)h[c]);
        }
        const int ln = 32 * g + r;                // fragment lane
        // positions (hin ? 4 : 0) + {0, 2, 1, 3} hold elements c = 0, 1, 2, 3 -> store c order 0 2 1 3
        typedef _Float16 h4 __attribute__((ext_vector_type(4)));
        *reinterpret_cast<h4*>(t_hi + ((ksl * 4 + s) * 64 + ln) * 16 + hin * 8) = h4{h[0], h[2], h[1], h[3]};
        typedef short s2 __attribute__((ext_vector_type(2)));
        s2 w = {0, 0};
        w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(w, h2{rl[0], rl[2]}, 1.0f, false);
        w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(w, h2{rl[1], rl[3]}, 1.0f, true);
        *reinterpret_cast<uint32_t*>(t_lo + ((ksl * 2 + (s >> 1)) * 64 + ln) * 16 + 8 * (s & 1) + 4 * hin) =
            __builtin_bit_cast(uint32_t, w);
        if ((lane & 7) == 0) {
            const int bk = lane >> 3;
            float xs = q.sum * inv;
            asm volatile("" : "+v"(xs));
            const _Float16 sh = (_Float16)xs;
            reinterpret_cast<_Float16*>(t_sx)[r * 8 + bk] = sh;
            reinterpret_cast<_Float16*>(t_sx)[(32 + r) * 8 + bk] = (_Float16)(xs - (float)sh);
        }
    }
    __syncthreads();
    const size_t tk = (size_t)T * ks_all + 4 * sb;
    u32x4* dh = reinterpret_cast<u32x4*>(hi + tk * 4096);
    u32x4* dl = reinterpret_cast<u32x4*>(lo + tk * 2048);
    const int i = threadIdx.x;
    dh[i] = reinterpret_cast<const u32x4*>(t_hi)[i];
    dh[i + 512] = reinterpret_cast<const u32x4*>(t_hi)[i + 512];
    dl[i] = reinterpret_cast<const u32x4*>(t_lo)[i];
    if (i < 64) reinterpret_cast<u32x4*>(sx + ((size_t)T * nsb + sb) * 1024)[i] = reinterpret_cast<const u32x4*>(t_sx)[i];
}

// Row exponents and planes from fp32 x in one pass, for K <= 4096: a
// workgroup takes kFxTok tokens of a 32-token tile and their whole rows,
// kFxKw waves per token (wave w: token w % kFxTok, super-blocks
// w / kFxTok + kFxKw i), lane l elements 4l..4l+3 of each of its
// super-blocks (all requested together, held in registers). The row
// exponent is the largest block scale of the quantized row (fmaxf skips a
// NaN block's scale; the scale is monotone in the block's amax, so this is
// fr_rowexp_kernel's value), and t, its split and the xs terms are
// fr_planes_kernel's arithmetic, so the planes are bit-identical. The
// tokens' pieces of every super-block go to LDS as [row][lane half][token]
// 16-byte units and are copied out in runs of kFxTok units. Workgroups
// stride over the token groups and request the next group's rows before
// processing the current one. Against fr_rowexp_kernel + fr_planes_kernel at
// K 4096: M 2048 26.8 -> 20.3 us, M 512 12.5 -> 7.5 (8 tokens x 1 wave per
// workgroup 23.6 / 17.4, 4 x 4 19.5 / 10.2, 1 x 16 28.8 / 9.2).
constexpr int kFxTok = 2;                         // tokens per workgroup
constexpr int kFxKw = 8;                          // waves per token
constexpr int kFxMaxSb = 16;                      // super-blocks per row (K <= 4096)
constexpr int kFxUnits = 50 * kFxTok;             // 16-byte units per super-block: HI 32, LO 16, SX 2 per token
constexpr int kFxWgPerCu = 4;                     // grid cap: workgroups per CU

__global__ void __launch_bounds__(64 * kFxTok * kFxKw) fr_planes_x_kernel(const float* __restrict__ x, int M, int K,
                                                                          float* __restrict__ escale,
                                                                          uint8_t* __restrict__ hi,
                                                                          uint8_t* __restrict__ lo,
                                                                          uint8_t* __restrict__ sx) {
#pragma clang fp contract(off)
    constexpr int NJ = kFxMaxSb / kFxKw;
    extern __shared__ __attribute__((aligned(16))) uint8_t st[];
    __shared__ float wmax[kFxKw][kFxTok];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rr = wave % kFxTok, kh = wave / kFxTok;
    const int nsb = K >> 8, ks_all = K >> 6;
    const int ngrp = (((M + 31) & ~31)) / kFxTok;
    const int ksl = lane >> 4, hin = (lane >> 3) & 1, g = (lane >> 2) & 1, s = lane & 3;
    auto load = [&](int grp, float4 (&xv)[NJ]) {
        const int m = grp * kFxTok + rr;
        const float* xr = x + (size_t)m * K + 4 * lane;
#pragma unroll
        for (int i = 0; i < NJ; i++) {
            const int j = kh + kFxKw * i;
            xv[i] = (grp < ngrp && m < M && j < nsb) ? *reinterpret_cast<const float4*>(xr + 256 * j)
                                                     : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    float4 xv[NJ];
    load(blockIdx.x, xv);
    // the next group's rows are requested before this group is processed
    for (int grp = blockIdx.x; grp < ngrp; grp += gridDim.x) {
        float4 xn[NJ];
        load(grp + gridDim.x, xn);
        const int m = grp * kFxTok + rr;
        const int T = (grp * kFxTok) >> 5, r0 = (grp * kFxTok) & 31;
        Q8Group q[NJ];
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < NJ; i++) {
            q[i] = quant_group8(xv[i]);
            mx = fmaxf(mx, q[i].d);
        }
#pragma unroll
        for (int o = 8; o < 64; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
        if (kFxKw > 1) {
            if (lane == 0) wmax[kh][rr] = mx;
            __syncthreads();
#pragma unroll
            for (int k = 0; k < kFxKw; k++) mx = fmaxf(mx, wmax[k][rr]);
        }
        const int e = row_exponent(mx);
        const float es = ldexpf(1.0f, e);
        if (lane == 0 && kh == 0) escale[m] = es;
        const float inv = 1.0f / es;
#pragma unroll
        for (int i = 0; i < NJ; i++) {
            const int j = kh + kFxKw * i;
            if (j >= nsb) continue;
            uint8_t* sh_hi = st + j * kFxUnits * 16;
            uint8_t* sh_lo = sh_hi + 32 * kFxTok * 16;
            uint8_t* sh_sx = sh_lo + 16 * kFxTok * 16;
            const float ds = q[i].d * inv;
            _Float16 h[4], rl[4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                float t = ds * (float)(int8_t)(q[i].packed >> (8 * c));
                t = t * 512.0f;
                asm volatile("" : "+v"(t));
                h[c] = (_Float16)t;
                rl[c] = (_Float16)(t - (float)h[c]);
            }
            typedef _Float16 h4 __attribute__((ext_vector_type(4)));
            *reinterpret_cast<h4*>(sh_hi + (((ksl * 4 + s) * 2 + g) * kFxTok + rr) * 16 + hin * 8) =
                h4{h[0], h[2], h[1], h[3]};
            typedef short s2 __attribute__((ext_vector_type(2)));
            s2 w = {0, 0};
            w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(w, h2{rl[0], rl[2]}, 1.0f, false);
            w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(w, h2{rl[1], rl[3]}, 1.0f, true);
            *reinterpret_cast<uint32_t*>(sh_lo + (((ksl * 2 + (s >> 1)) * 2 + g) * kFxTok + rr) * 16 + 8 * (s & 1) +
                                         4 * hin) = __builtin_bit_cast(uint32_t, w);
            if ((lane & 7) == 0) {
                const int bk = lane >> 3;
                float xs = q[i].sum * inv;
                asm volatile("" : "+v"(xs));
                const _Float16 xh = (_Float16)xs;
                reinterpret_cast<_Float16*>(sh_sx)[rr * 8 + bk] = xh;
                reinterpret_cast<_Float16*>(sh_sx)[(kFxTok + rr) * 8 + bk] = (_Float16)(xs - (float)xh);
            }
        }
        __syncthreads();
        // unit v of super-block j: row2 = v / kFxTok (row * 2 + lane half), token v % kFxTok
        const int nu = nsb * kFxUnits;
        for (int u = threadIdx.x; u < nu; u += 64 * kFxTok * kFxKw) {
            const int j = u / kFxUnits, v = u - j * kFxUnits;
            const u32x4 val = *reinterpret_cast<const u32x4*>(st + (size_t)u * 16);
            const int t = v % kFxTok, row2 = v / kFxTok;
            const size_t tk = (size_t)T * ks_all + 4 * j;
            uint8_t* dst;
            if (row2 < 32) dst = hi + tk * 4096 + ((row2 >> 1) * 64 + 32 * (row2 & 1) + r0 + t) * 16;
            else if (row2 < 48) dst = lo + tk * 2048 + (((row2 - 32) >> 1) * 64 + 32 * (row2 & 1) + r0 + t) * 16;
            else dst = sx + ((size_t)T * nsb + j) * 1024 + ((row2 - 48) * 32 + r0 + t) * 16;
            *reinterpret_cast<u32x4*>(dst) = val;
        }
        __syncthreads();                          // LDS and wmax free for the next group
#pragma unroll
        for (int i = 0; i < NJ; i++) xv[i] = xn[i];
    }
}

struct FrPlanes {
    uint8_t* hi;
    uint8_t* lo;
    uint8_t* sx;
    float* escale;
};

// MFMA throughput probe (measurement hook): per iteration a wave issues the
// fragment-order GEMM's products of one 64-element step on a 2 x 2 tile
// set (16 v_mfma_f32_32x32x16_f16 + 4 v_mfma_f32_32x32x64_f8f6f4, kind 0)
// or 8 v_mfma_i32_32x32x32_i8 (kind 1), operands in registers: either
// near-constant (mostly zero) or random bit patterns of the GEMM's value
// ranges, which shows how much of the nominal MFMA rate the part sustains
// on real data (clock and power).
template <int KIND>
__global__ void __launch_bounds__(512) mfma_probe_kernel(int rnd_ops, int iters, float* __restrict__ out) {
    uint32_t x = (threadIdx.x + 1) * 2654435761u + blockIdx.x * 97u;
    auto rnd = [&]() {
        x ^= x << 13;
        x ^= x >> 17;
        x ^= x << 5;
        return x;
    };
    const int lane = threadIdx.x & 63;
    h8 A[4][2], B[4][2];
    i8x32 L[2], V8[2];
    for (int s = 0; s < 4; s++)
        for (int t = 0; t < 2; t++)
            for (int j = 0; j < 8; j++) {
                A[s][t][j] = rnd_ops ? (_Float16)((int)(rnd() % 20001) - 10000) : (_Float16)(j == 0 ? lane * 0.001f : 0.0f);
                B[s][t][j] = rnd_ops ? (_Float16)((rnd() % 64) * (rnd() % 16) * 0.25f) : (_Float16)(j == 1 ? 0.5f : 0.0f);
            }
    for (int t = 0; t < 2; t++)
        for (int j = 0; j < 8; j++) {
            L[t][j] = rnd_ops ? (int)(rnd() & 0x3f3f3f3fu) : 0;
            V8[t][j] = rnd_ops ? (int)(rnd() & 0x5f5f5f5fu) : 0;
        }
    f16v acc[2][2];
    typedef int i16v __attribute__((ext_vector_type(16)));
    typedef int i4v __attribute__((ext_vector_type(4)));
    i16v iacc[2][2];
    for (int t = 0; t < 2; t++)
        for (int r = 0; r < 2; r++)
            for (int i = 0; i < 16; i++) {
                acc[t][r][i] = 0.0f;
                iacc[t][r][i] = 0;
            }
    for (int it = 0; it < iters; it++) {
        if (KIND == 0) {
#pragma unroll
            for (int s = 0; s < 4; s++)
#pragma unroll
                for (int r = 0; r < 2; r++)
#pragma unroll
                    for (int t = 0; t < 2; t++)
                        acc[t][r] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[s][t], B[s][r], acc[t][r], 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 2; r++)
#pragma unroll
                for (int t = 0; t < 2; t++)
                    acc[t][r] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(L[t], V8[r], acc[t][r], 0, 0, 0, 0, 0, 0);
        } else {
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int r = 0; r < 2; r++)
#pragma unroll
                    for (int t = 0; t < 2; t++) {
                        const i4v a = {L[t][4 * h], L[t][4 * h + 1], L[t][4 * h + 2], L[t][4 * h + 3]};
                        const i4v b = {V8[r][4 * h], V8[r][4 * h + 1], V8[r][4 * h + 2], V8[r][4 * h + 3]};
                        iacc[t][r] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, iacc[t][r], 0, 0, 0);
                    }
        }
        asm volatile("" : "+v"(A[0][0]), "+v"(B[0][0]), "+v"(L[0]), "+v"(V8[0]));
    }
    float sm = 0.0f;
    for (int t = 0; t < 2; t++)
        for (int r = 0; r < 2; r++)
            for (int i = 0; i < 16; i++) sm += acc[t][r][i] + (float)iacc[t][r][i];
    out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = sm;
}

// MFMA / VALU co-issue probe (measurement hook): per iteration a wave issues
// 32 v_mfma_f32_32x32x16_f16 on a 4 x 2 tile set (the wide-token GEMM's
// K step) with NV independent packed-fp16 VALU operations after each
// product, in workgroups of NW waves: how much of the matrix pipe's rate
// survives VALU work between the products of one wave (NW = 4: one wave per
// SIMD at one workgroup per CU) or of two (NW = 8).
template <int NV, int NW>
__global__ void __launch_bounds__(64 * NW) coissue_probe_kernel(int iters, float* __restrict__ out) {
    const int lane = threadIdx.x & 63;
    h8 A[4], B[2];
    for (int i = 0; i < 4; i++)
        for (int j = 0; j < 8; j++) A[i][j] = (_Float16)((lane * 7 + i * 13 + j) % 17 - 8);
    for (int i = 0; i < 2; i++)
        for (int j = 0; j < 8; j++) B[i][j] = (_Float16)((lane * 3 + i * 5 + j) % 11);
    h2 v[8];
    for (int i = 0; i < 8; i++) v[i] = h2{(_Float16)(lane * 0.01f + i), (_Float16)0.5f};
    const h2 m = {(_Float16)0.999f, (_Float16)0.999f}, a = {(_Float16)0.001f, (_Float16)0.001f};
    f16v acc[4][2];
    for (int t = 0; t < 4; t++)
        for (int r = 0; r < 2; r++)
            for (int i = 0; i < 16; i++) acc[t][r][i] = 0.0f;
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int s = 0; s < 4; s++) {
#pragma unroll
            for (int r = 0; r < 2; r++)
#pragma unroll
                for (int t = 0; t < 4; t++) acc[t][r] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[t], B[r], acc[t][r], 0, 0, 0);
#pragma unroll
            for (int k = 0; k < NV; k++)
#pragma unroll
                for (int i = 0; i < 8; i++) v[i] = __builtin_elementwise_fma(v[i], m, a);
            if (NV > 0) {
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, NV, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        asm volatile("" : "+v"(A[0]), "+v"(B[0]));
    }
    float sm = 0.0f;
    for (int t = 0; t < 4; t++)
        for (int r = 0; r < 2; r++)
            for (int i = 0; i < 16; i++) sm += acc[t][r][i];
    for (int i = 0; i < 8; i++) sm += (float)v[i][0];
    out[(size_t)blockIdx.x * 512 + threadIdx.x] = sm;
}

}  // namespace

hipError_t launch_mfma_probe(int kind, int rnd_ops, int iters, int grid, float* out, hipStream_t st) {
    if (kind == 0) hipLaunchKernelGGL(mfma_probe_kernel<0>, dim3(grid), dim3(512), 0, st, rnd_ops, iters, out);
    else if (kind == 1) hipLaunchKernelGGL(mfma_probe_kernel<1>, dim3(grid), dim3(512), 0, st, rnd_ops, iters, out);
    else if (kind >= 2 && kind <= 9) {
        // kinds 2-5: 8-wave workgroups, 0 / 1 / 3 / 6 VALU operations per
        // product; 6-9: the same with 4-wave workgroups
#define LP_P(NV, NW) hipLaunchKernelGGL((coissue_probe_kernel<NV, NW>), dim3(grid), dim3(64 * NW), 0, st, iters, out)
        switch (kind) {
            case 2: LP_P(0, 8); break;
            case 3: LP_P(1, 8); break;
            case 4: LP_P(3, 8); break;
            case 5: LP_P(6, 8); break;
            case 6: LP_P(0, 4); break;
            case 7: LP_P(1, 4); break;
            case 8: LP_P(3, 4); break;
            default: LP_P(6, 4); break;
        }
#undef LP_P
    } else return hipErrorInvalidValue;
    return hipGetLastError();
}

namespace {

size_t up256(size_t v) { return (v + 255) & ~size_t(255); }

FrPlanes carve_fr(void* base, int M, int K) {
    const size_t Mp = (size_t)((M + 31) & ~31);
    uint8_t* p = static_cast<uint8_t*>(base);
    FrPlanes P;
    P.hi = p;
    p += up256(Mp * K * 2);
    P.lo = p;
    p += up256(Mp * K);
    P.sx = p;
    p += up256(Mp * (K / 256) * 32);
    P.escale = reinterpret_cast<float*>(p);
    return P;
}

}  // namespace

size_t gemm_fr_planes_bytes(int M, int K) {
    const size_t Mp = (size_t)((M + 31) & ~31);
    return up256(Mp * K * 2) + up256(Mp * K) + up256(Mp * (K / 256) * 32) + up256(Mp * 4);
}

bool gemm_fr_supported(uint32_t type, int M, int K) {
    return type == T_Q4_K && M >= kBm && K % 256 == 0 && K <= 32768;
}

// Planes from fp32 x (x != nullptr) or from quantized blocks A.
hipError_t launch_fr_planes(const float* x, const ActView& A, void* planes, int M, int K, hipStream_t st) {
    if (M <= 0) return hipSuccess;
    const FrPlanes P = carve_fr(planes, M, K);
    const int Mp = (M + 31) & ~31;
    const dim3 eg((Mp + 3) / 4), pg(K / 256, Mp / 32);
    if (x && K <= 256 * kFxMaxSb) {
        const int fgrid = std::min(Mp / kFxTok, kFxWgPerCu * device_cu_count());
        hipLaunchKernelGGL(fr_planes_x_kernel, dim3(fgrid), dim3(64 * kFxTok * kFxKw),
                           (size_t)(K / 256) * kFxUnits * 16,
                           st, x, M, K, P.escale, P.hi, P.lo, P.sx);
    } else if (x) {
        hipLaunchKernelGGL(fr_rowexp_kernel<false>, eg, dim3(256), 0, st, x, A, M, Mp, K, P.escale);
        hipLaunchKernelGGL(fr_planes_kernel<false>, pg, dim3(512), 0, st, x, A, M, K, P.escale, P.hi, P.lo, P.sx);
    } else {
        hipLaunchKernelGGL(fr_rowexp_kernel<true>, eg, dim3(256), 0, st, x, A, M, Mp, K, P.escale);
        hipLaunchKernelGGL(fr_planes_kernel<true>, pg, dim3(512), 0, st, x, A, M, K, P.escale, P.hi, P.lo, P.sx);
    }
    return hipGetLastError();
}

__global__ void __launch_bounds__(256) fr_zero_kernel(float* __restrict__ y, size_t n) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) y[i] = 0.0f;
}

// Tiles of the grid that run whole: all of them when there are at least as
// many tiles as CUs (a CU's throughput was measured the same with one or two
// workgroups, so a half-full last round costs no more than split tiles, and
// splitting would need y zeroed first: 8.6 us at N 14336 M 2048); with fewer,
// each tile runs as two workgroups over the halves of K, to reach more CUs.
static int fr_nfull(int ntiles, int K) {
    return (ntiles < device_cu_count() && (K >> 8) >= 2) ? 0 : ntiles;
}

hipError_t launch_fr_gemm(const uint8_t* w, void* planes, float* y, int M, int K, int N, hipStream_t st) {
    if (M <= 0 || N <= 0) return hipSuccess;
    const FrPlanes P = carve_fr(planes, M, K);
    const int ntm = (M + kBm - 1) / kBm, ntn = (N + kBn - 1) / kBn, ntiles = ntm * ntn;
    FrArgs g{P.hi, P.lo, P.sx, P.escale, w, row_bytes(T_Q4_K, K), y, M, N, K, ntm, ntn, (M + 31) / 32,
             fr_nfull(ntiles, K)};
    if (g.nfull < ntiles) {
        // rows of the split tiles (and of whole tiles sharing those rows: they overwrite)
        const size_t first = (size_t)(g.nfull / ntn) * kBm * N, n = (size_t)M * N - first;
        hipLaunchKernelGGL(fr_zero_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, y + first, n);
    }
    constexpr int NS = 2;
    const size_t lds = (size_t)NS * kStage + 2 * kSbuf + kNw * 64 * 4;
    const long nblk = (long)g.nfull + 2L * (ntiles - g.nfull);
    hipLaunchKernelGGL((gemm_q4k_fr<NS>), dim3((unsigned)nblk), dim3(64 * kNw), lds, st, g);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Wide-token prefill GEMM (gemm_q4k_wt) on the same fragment-order planes.
//
// Same arithmetic as gemm_q4k_fr; what changes is the work split. Each wave
// owns 128 tokens and 64 weight rows (4 x 2 MFMA tiles of 32 x 32), so every
// weight element is decoded once per 128 tokens, half the decode VALU per
// MFMA of a 64-token wave tile. A workgroup is 4 * TH waves (TH token halves
// of 128 tokens, 4 row quarters of 64 rows): a tile of 128 * TH tokens x 256
// rows. TH = 2 puts two waves on each SIMD, which is what lets one wave's
// VALU work (decode, e4m3 conversion, super-block fold) issue under the other
// wave's MFMAs; with one wave per SIMD a wave's own VALU work between its
// MFMAs leaves the matrix pipe idle.
//
// The super-block scale is applied by keeping each row's accumulators in
// units u = d_sb * 2^-7 of the current super-block: the MFMAs add the
// unscaled main products straight into the accumulators, and at each
// super-block boundary acc = acc * (u_old / u_new) - (dmin_old / u_new) *
// min_old (one accumulator set instead of two). A super-block whose d is
// zero keeps the old unit and decodes its V as zero (its main term is zero);
// a non-finite d makes the row NaN.
//
// Per K step wave w copies token tile w's hi (4 x 1 KiB) and lo (2 x 1 KiB)
// pieces and code piece w (32 rows x 32 B; with TH = 1 also piece w + 4), and
// per super-block token tile w's min-term piece and (waves 0-3) the headers
// of 64 rows.
// ---------------------------------------------------------------------------
namespace {

// TM token groups of 128 x RQ row groups of 64, one wave each.
template <int TM, int RQ>
struct WtCfg {
    static constexpr int Nw = TM * RQ;                // waves
    static constexpr int TT = 4 * TM;                 // 32-token tiles per workgroup
    static constexpr int Bm = 32 * TT, Bn = 64 * RQ;
    static constexpr int Hi = TT * 4096, Lo = TT * 2048, Codes = 2 * RQ * 1024;
    static constexpr int Stage = Hi + Lo + Codes;
    static constexpr int Hdr = Bn * 16, Sx = TT * 1024;
    static constexpr int Sbuf = Hdr + Sx;
    static constexpr int NS = Nw == 4 || TM == 1 ? 3 : 2;
    static constexpr int WPT = Nw / TT;               // waves copying one token tile's pieces
    static constexpr int NA = 6 / WPT;                // hi/lo pieces per wave and step
    static constexpr int NC = 2 * RQ / Nw;            // code pieces per wave and step
    static constexpr int DmaStep = NA + NC;
    static constexpr size_t Lds = (size_t)NS * Stage + 2 * Sbuf + Nw * 128 * 4;
    static_assert(Stage / 1024 == Nw * DmaStep, "copies split evenly");
    static_assert(Lds <= 160 * 1024, "LDS");
};

struct WtArgs {
    const uint8_t* hi;
    const uint8_t* lo;
    const uint8_t* sx;
    const float* escale;
    const uint8_t* w;
    size_t rb;
    float* y;
    int M, N, K;
    int ntm, ntn;
    int tiles_pad;
    int nfull;          // tiles [0, nfull) run whole; each later one is two
                        // workgroups over the halves of K adding into a zeroed y
};

struct WtPlan {
    Rsrc rs_hi, rs_lo, rs_w, rs_sx;
    uint32_t code_off[2], hdr_off;
};

// Copy i of step kt: i < NA the wave's hi/lo pieces (wave w takes pieces
// (w % WPT) * NA .. + NA of token tile w / WPT: 4 hi then 2 lo), then its NC
// code pieces w * NC + k (32 rows x 32 B each); i = DmaStep, DmaStep + 1 on a
// super-block's first step: token tile w's min-term piece (w < TT) and the
// headers of rows 64w .. 64w + 63 (w < RQ).
template <int TM, int RQ>
__device__ __forceinline__ void wt_issue(const WtPlan& d, int wave, int kt, uint8_t* st, uint8_t* sbb, int i) {
    using C = WtCfg<TM, RQ>;
    const uint32_t lane16 = (threadIdx.x & 63) * 16;
    const int sb = kt >> 2, jb = kt & 3;
    if (i < C::NA) {
        const int tt = wave / C::WPT, j = (wave % C::WPT) * C::NA + i;
        if (j < 4) dma16(d.rs_hi, lane16, (uint32_t)(kt * 4096 + j * 1024), st + tt * 4096 + j * 1024);
        else dma16(d.rs_lo, lane16, (uint32_t)(kt * 2048 + (j - 4) * 1024), st + C::Hi + tt * 2048 + (j - 4) * 1024);
    } else if (i < C::DmaStep) {
        const int k = i - C::NA;
        dma16(d.rs_w, d.code_off[k], (uint32_t)(sb * 144 + 32 * jb), st + C::Hi + C::Lo + (wave * C::NC + k) * 1024);
    } else if (jb == 0) {
        if (i == C::DmaStep) {
            if (wave < C::TT) dma16(d.rs_sx, lane16, (uint32_t)(sb * 1024), sbb + C::Hdr + wave * 1024);
        } else if (wave < RQ) {
            dma16(d.rs_w, d.hdr_off, (uint32_t)(sb * 144), sbb + wave * 1024);
        }
    }
}

template <int TM, int RQ>
__device__ __forceinline__ int wt_count(int k, int nk, int wave) {
    using C = WtCfg<TM, RQ>;
    return k < nk ? C::DmaStep + ((k & 3) == 0 ? (wave < C::TT ? 1 : 0) + (wave < RQ ? 1 : 0) : 0) : 0;
}

template <int TM, int RQ>
__global__ void __launch_bounds__(64 * TM * RQ, 1) __attribute__((amdgpu_waves_per_eu(TM * RQ / 4, TM * RQ / 4)))
gemm_q4k_wt(WtArgs g) {
    using C = WtCfg<TM, RQ>;
    constexpr int NS = C::NS;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int th = wave / RQ, rq = wave % RQ;         // token group, row group
    const int bid = blockIdx.x;
    int tile, part = 0, ksplit = 1;
    if (bid < g.nfull) {
        tile = (g.nfull & 7) == 0 ? (bid & 7) * (g.nfull >> 3) + (bid >> 3) : bid;
    } else {
        tile = g.nfull + ((bid - g.nfull) >> 1);
        part = (bid - g.nfull) & 1;
        ksplit = 2;
    }
    constexpr int GM = 2;
    int tm, tn;
    {
        const int per = GM * g.ntn, grp = tile / per, in = tile % per;
        const int gm = g.ntm - grp * GM < GM ? g.ntm - grp * GM : GM;
        tm = grp * GM + in % gm;
        tn = in / gm;
    }
    const int m0 = tm * C::Bm, n0 = tn * C::Bn;
    const int nsb_all = g.K >> 8, ks_all = g.K >> 6;
    const int sb_beg = part * nsb_all / ksplit, sb_end = (part + 1) * nsb_all / ksplit;
    const int kt0 = 4 * sb_beg, nk = 4 * sb_end;

    WtPlan d;
    {
        auto clampT = [&](int T) { return T < g.tiles_pad ? T : g.tiles_pad - 1; };
        const int T = clampT(tm * C::TT + wave / C::WPT);
        const int Ts = clampT(tm * C::TT + (wave < C::TT ? wave : 0));
        const int nt = g.N - n0 < C::Bn ? g.N - n0 : C::Bn;
        d.rs_w = make_rsrc(g.w + (size_t)n0 * g.rb, (uint32_t)((size_t)nt * g.rb));
        d.rs_hi = make_rsrc(g.hi + (size_t)T * ks_all * 4096, (uint32_t)(ks_all * 4096));
        d.rs_lo = make_rsrc(g.lo + (size_t)T * ks_all * 2048, (uint32_t)(ks_all * 2048));
        d.rs_sx = make_rsrc(g.sx + (size_t)Ts * nsb_all * 1024, (uint32_t)(nsb_all * 1024));
#pragma unroll
        for (int c = 0; c < 2; c++) {
            int row = (wave * C::NC + (c < C::NC ? c : 0)) * 32 + (lane & 31);
            row = row < nt ? row : nt - 1;
            d.code_off[c] = (uint32_t)((size_t)row * g.rb) + 16 + 16 * (lane >> 5);
        }
        int hrow = (wave < RQ ? wave : 0) * 64 + lane;
        hrow = hrow < nt ? hrow : nt - 1;
        d.hdr_off = (uint32_t)((size_t)hrow * g.rb);
    }
    auto stage = [&](int i) { return smem + i * C::Stage; };
    auto sbuf = [&](int i) { return smem + NS * C::Stage + i * C::Sbuf; };

    const uint32_t lds0 = lds_addr(smem);
    const uint32_t l16 = lds0 + lane * 16 + th * (4 * 4096);                 // this wave's 4 token tiles
    const uint32_t l16lo = lds0 + lane * 16 + C::Hi + th * (4 * 2048);
    const uint32_t l16c = lds0 + lane * 16 + C::Hi + C::Lo + rq * (2 * 1024);   // code pieces 2rq, 2rq+1
    const uint32_t hdr_a = lds0 + NS * C::Stage + (rq * 64 + (lane & 31)) * 16;  // + r * 512
    const uint32_t sx_a = lds0 + NS * C::Stage + C::Hdr + th * (4 * 1024) + lane * 16;

    f16v acc[4][2];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[a][b][r] = 0.0f;

    uint32_t hy[2], hz[2], hw[2];
    float u[2], dmn[2], zs[2];
#pragma unroll
    for (int r = 0; r < 2; r++) {
        u[r] = 1.0f;
        dmn[r] = 0.0f;
        zs[r] = 1.0f;
        hy[r] = hz[r] = hw[r] = 0;
    }

    // min term of the previous super-block (its SX piece in buffer `sbo`, its
    // m values in hz/hw) folded into the accumulators: acc = acc * rho - kap * min
    auto fold = [&](uint32_t sbo, const float (&rho)[2], const float (&kap)[2]) {
        h8 S[4];
        rd128h<0>(S[0], sx_a + sbo);
        rd128h<1024>(S[1], sx_a + sbo);
        rd128h<2048>(S[2], sx_a + sbo);
        rd128h<3072>(S[3], sx_a + sbo);
        h8 mb[2];
#pragma unroll
        for (int r = 0; r < 2; r++)
#pragma unroll
            for (int j = 0; j < 8; j++) mb[r][j] = (_Float16)(float)q4k_m(hz[r], hw[r], j);
        lgkm<0>(S);
        // one tile's min product in registers at a time: each product's B
        // operand is tied to the previous tile's folded accumulators, so the
        // products cannot all be hoisted ahead of the folds
        f16v prev = acc[0][0];
#pragma unroll
        for (int r = 0; r < 2; r++)
#pragma unroll
            for (int t = 0; t < 4; t++) {
                h8 bm = mb[r];
                asm volatile("" : "+v"(bm) : "v"(prev));
                const f16v mm = __builtin_amdgcn_mfma_f32_32x32x16_f16(S[t], bm, f16v{}, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 16; i++) acc[t][r][i] = fmaf(-kap[r], mm[i], acc[t][r][i] * rho[r]);
                prev = acc[t][r];
            }
    };

#pragma unroll
    for (int i = 0; i < NS - 1; i++)
        if (kt0 + i < nk)
#pragma unroll
            for (int p = 0; p < C::DmaStep + 2; p++)
                wt_issue<TM, RQ>(d, wave, kt0 + i, stage(i), sbuf(((kt0 + i) >> 2) & 1), p);

    // residual (fp8) products of a step, run after the next step's barrier:
    // their operands are in registers, so they fill the time the next
    // step's first LDS reads take, and the next copies go out under them
    // (zero before the first step: its residual call adds nothing)
    u32x4 Lp[4][2];
    i8x32 bvp[2];
#pragma unroll
    for (int t = 0; t < 4; t++) Lp[t][0] = Lp[t][1] = u32x4{0, 0, 0, 0};
    bvp[0] = bvp[1] = i8x32{0, 0, 0, 0, 0, 0, 0, 0};
    auto residual = [&](bool issue, int kt, uint8_t* pst, uint8_t* psb) {
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const i8x32 av = {(int)Lp[t][0].x, (int)Lp[t][0].y, (int)Lp[t][0].z, (int)Lp[t][0].w,
                              (int)Lp[t][1].x, (int)Lp[t][1].y, (int)Lp[t][1].z, (int)Lp[t][1].w};
#pragma unroll
            for (int r = 0; r < 2; r++) {
                acc[t][r] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bvp[r], acc[t][r], 0, 0, 0, 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
                const int ci = t * 2 + r;
                if (issue && ci < C::DmaStep) wt_issue<TM, RQ>(d, wave, kt, pst, psb, ci);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if (issue) {
#pragma unroll
            for (int i = C::DmaStep < 8 ? C::DmaStep : 8; i < C::DmaStep + 2; i++) wt_issue<TM, RQ>(d, wave, kt, pst, psb, i);
        }
    };

    for (int sb = sb_beg; sb < sb_end; sb++) {
        const uint32_t sbo = (uint32_t)((sb & 1) * C::Sbuf);
#pragma unroll
        for (int jb = 0; jb < 4; jb++) {
            const int kt = 4 * sb + jb;
            int later = 0;
#pragma unroll
            for (int i = 1; i < NS - 1; i++) later += wt_count<TM, RQ>(kt + i, nk, wave);
            wait_dma(later);
            __builtin_amdgcn_s_barrier();
            const bool pf = kt + NS - 1 < nk;
            uint8_t* const pst = stage((kt + NS - 1 - kt0) % NS);
            uint8_t* const psb = sbuf(((kt + NS - 1) >> 2) & 1);
            const uint32_t so = (uint32_t)(((kt - kt0) % NS) * C::Stage);
            const uint32_t b = l16 + so;

            // this step's first reads, then the previous step's residual
            // products (and this step's copies) while they land
            u32x4 h[2];
            if (jb == 0) {
                rd128<0>(h[0], hdr_a + sbo);
                rd128<512>(h[1], hdr_a + sbo);
            }
            u32x4 cw[2];
            h8 A[2][4];
            rd128<0>(cw[0], l16c + so);
            rd128<1024>(cw[1], l16c + so);
            rd128h<0>(A[0][0], b);
            rd128h<4096>(A[0][1], b);
            rd128h<8192>(A[0][2], b);
            rd128h<12288>(A[0][3], b);
            residual(pf, kt + NS - 1, pst, psb);

            if (jb == 0) {
                if (jb == 0) lgkm<6>(h);
                float rho[2], kap[2];
#pragma unroll
                for (int r = 0; r < 2; r++) {
                    const float dn = fp16_bits_to_f32(h[r].x);
                    const float un = dn * 0.0078125f;
                    const bool ok = un != 0.0f && __builtin_isfinite(un);
                    const float unew = ok ? un : u[r];
                    rho[r] = __builtin_isfinite(dn) ? u[r] / unew : __builtin_nanf("");
                    kap[r] = dmn[r] / unew;
                    u[r] = unew;
                    zs[r] = ok ? 1.0f : 0.0f;
                }
                if (sb > sb_beg) fold(sbo ^ (uint32_t)C::Sbuf, rho, kap);
#pragma unroll
                for (int r = 0; r < 2; r++) {
                    dmn[r] = fp16_bits_to_f32(h[r].x >> 16);
                    hy[r] = h[r].y;
                    hz[r] = h[r].z;
                    hw[r] = h[r].w;
                }
            }
            h2 ml[2], al[2], mh[2], ah[2];
#pragma unroll
            for (int r = 0; r < 2; r++) {
                const float sl = (float)q4k_sc(hy[r], hw[r], 2 * jb) * (0.25f * zs[r]);
                const float sh = (float)q4k_sc(hy[r], hw[r], 2 * jb + 1) * (0.25f * 0.0625f * zs[r]);
                const _Float16 a = (_Float16)sl, b = (_Float16)(-1024.0f * sl);
                const _Float16 c = (_Float16)sh, e = (_Float16)(-1024.0f * sh);
                ml[r] = h2{a, a};
                al[r] = h2{b, b};
                mh[r] = h2{c, c};
                ah[r] = h2{e, e};
            }
            uint32_t v8[2][8];
            h8 Vc[2];
            lgkm<4>(cw);
#pragma unroll
            for (int r = 0; r < 2; r++)
                Vc[r] = decode4(cw[r][0], ml[r], al[r], mh[r], ah[r]);
#pragma unroll
            for (int s = 0; s < 4; s++) {
                h8 (&As)[4] = A[s & 1];
                h8 (&An)[4] = A[(s + 1) & 1];
                lgkm<0>(As);
                if (s == 0) {
                    rd128h<1024>(An[0], b);
                    rd128h<1024 + 4096>(An[1], b);
                    rd128h<1024 + 8192>(An[2], b);
                    rd128h<1024 + 12288>(An[3], b);
                } else if (s == 1) {
                    rd128h<2048>(An[0], b);
                    rd128h<2048 + 4096>(An[1], b);
                    rd128h<2048 + 8192>(An[2], b);
                    rd128h<2048 + 12288>(An[3], b);
                } else if (s == 2) {
                    rd128h<3072>(An[0], b);
                    rd128h<3072 + 4096>(An[1], b);
                    rd128h<3072 + 8192>(An[2], b);
                    rd128h<3072 + 12288>(An[3], b);
                } else {
                    // this step's lo pieces, for its residual products after
                    // the next barrier
                    const uint32_t bl = l16lo + so;
                    rd128<0>(Lp[0][0], bl);
                    rd128<1024>(Lp[0][1], bl);
                    rd128<2048>(Lp[1][0], bl);
                    rd128<3072>(Lp[1][1], bl);
                    rd128<4096>(Lp[2][0], bl);
                    rd128<5120>(Lp[2][1], bl);
                    rd128<6144>(Lp[3][0], bl);
                    rd128<7168>(Lp[3][1], bl);
                }
                // the next fragments' reads go out before this sub-step's
                // MFMAs (else the scheduler sinks them below the MFMAs that read
                // the registers they would reuse, and their latency is exposed)
                __builtin_amdgcn_sched_barrier(0);
                h8 Vn[2];
#pragma unroll
                for (int r = 0; r < 2; r++)
#pragma unroll
                    for (int t = 0; t < 4; t++)
                        acc[t][r] = __builtin_amdgcn_mfma_f32_32x32x16_f16(As[t], Vc[r], acc[t][r], 0, 0, 0);
                if (s < 3) {
#pragma unroll
                    for (int r = 0; r < 2; r++)
                        Vn[r] = decode4(cw[r][s + 1], ml[r], al[r], mh[r], ah[r]);
                }
#pragma unroll
                for (int r = 0; r < 2; r++) {
                    const u32x4 q = __builtin_bit_cast(u32x4, Vc[r]);
                    v8[r][2 * s] = e4m3x4(q.x, q.y);
                    v8[r][2 * s + 1] = e4m3x4(q.z, q.w);
                }
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
                if (s < 3) {
#pragma unroll
                    for (int r = 0; r < 2; r++) Vc[r] = Vn[r];
                }
            }
#pragma unroll
            for (int r = 0; r < 2; r++)
                bvp[r] = i8x32{(int)v8[r][0], (int)v8[r][1], (int)v8[r][2], (int)v8[r][3],
                               (int)v8[r][4], (int)v8[r][5], (int)v8[r][6], (int)v8[r][7]};
            // the lo pieces must be in registers before the next barrier
            // lets their stage be overwritten
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
            for (int t = 0; t < 4; t++) asm volatile("" : "+v"(Lp[t][0]), "+v"(Lp[t][1]));
        }
    }
    residual(false, 0, nullptr, nullptr);
    // the last super-block's min term; the accumulators leave in units of 1
    {
        float rho[2], kap[2];
#pragma unroll
        for (int r = 0; r < 2; r++) {
            rho[r] = u[r];
            kap[r] = dmn[r];
        }
        fold((uint32_t)(((sb_end - 1) & 1) * C::Sbuf), rho, kap);
    }

    const int mw = m0 + th * 128;
    float* esl = reinterpret_cast<float*>(smem + NS * C::Stage + 2 * C::Sbuf) + wave * 128;
    esl[lane] = mw + lane < g.M ? g.escale[mw + lane] : 0.0f;
    esl[64 + lane] = mw + 64 + lane < g.M ? g.escale[mw + 64 + lane] : 0.0f;
    __builtin_amdgcn_wave_barrier();
    const int gl = lane >> 5;
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const int n = n0 + rq * 64 + r * 32 + (lane & 31);
#pragma unroll
        for (int t = 0; t < 4; t++)
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

template <int TM, int RQ>
hipError_t launch_wt(const uint8_t* w, void* planes, float* y, int M, int K, int N, hipStream_t st) {
    using C = WtCfg<TM, RQ>;
    const FrPlanes P = carve_fr(planes, M, K);
    const int ntm = (M + C::Bm - 1) / C::Bm, ntn = (N + C::Bn - 1) / C::Bn, ntiles = ntm * ntn;
    const int cus = device_cu_count(), nsb = K >> 8;
    // one workgroup per CU: a last round that would leave at least half the
    // CUs idle runs its tiles as two workgroups over the halves of K instead
    // (two fp32 additions onto a zeroed y give the same sum in either order;
    // more parts would make the result depend on their order)
    const int rem = ntiles % cus;
    const bool split = rem > 0 && 2 * rem <= cus && nsb >= 2;
    const int nfull = split ? ntiles - rem : ntiles;
    WtArgs g{P.hi, P.lo, P.sx, P.escale, w, row_bytes(T_Q4_K, K), y, M, N, K, ntm, ntn, (M + 31) / 32, nfull};
    if (nfull < ntiles) {
        // rows of the token-tile pairs holding split tiles (whole tiles there overwrite)
        const size_t first = (size_t)(nfull / (2 * ntn)) * 2 * C::Bm * N;
        if (first < (size_t)M * N) {
            const size_t n = (size_t)M * N - first;
            hipLaunchKernelGGL(fr_zero_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, y + first, n);
        }
    }
    const long nblk = (long)nfull + 2L * (ntiles - nfull);
    hipLaunchKernelGGL((gemm_q4k_wt<TM, RQ>), dim3((unsigned)nblk), dim3(64 * C::Nw), C::Lds, st, g);
    return hipGetLastError();
}

}  // namespace

int wt_auto_cfg(int M, int K, int N) {
    const long cus = device_cu_count();
    const long t1 = (long)((M + 255) / 256) * ((N + 255) / 256);
    const long t0 = (long)((M + 127) / 128) * ((N + 255) / 256);
    // K-weighted: a K-split tile round costs less than an idle one
    if (t1 * (K / 256) >= 12L * cus) return 1;
    if (t0 * 5 >= 2 * cus) return 0;
    return -1;
}

hipError_t launch_wt_gemm(const uint8_t* w, void* planes, float* y, int M, int K, int N, hipStream_t st, int cfg) {
    if (M <= 0 || N <= 0) return hipSuccess;
    if (cfg == 1) return launch_wt<2, 4>(w, planes, y, M, K, N, st);
    return launch_wt<1, 4>(w, planes, y, M, K, N, st);
}

}  // namespace lp
