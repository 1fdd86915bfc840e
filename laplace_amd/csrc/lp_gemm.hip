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
// so an int8 MFMA per 32-K block must be followed by >= 2 VALU operations
// per output (int->float, scaled accumulate; the scale product itself is a
// third). One VALU operation per output and block already takes as long as
// the int8 MFMA producing it (a 32x32x32 int8 MFMA is 32 cycles, its 16
// outputs per lane 16 wave64 VALU operations of 4 cycles), so the int8
// route is VALU-bound at no more than half the int8 rate (a third with the
// scale product). The block scales are
// instead folded into the operands: A = xd*q (an fp32 product) as an fp16
// value plus its e4m3 residual, V = sc*nibble (exact in fp16), so the
// per-output epilogue runs once per 256-element super-block. See
// gemm_q4k_sp below for the operands, the error bound and the tiling.
//
// Small M (<= 16 rows, K beyond the int8 kernel's LDS limit) keeps the
// two-plane fp16 form (hi = fp16(xd*q), lo = fp16(xd*q - hi)) on
// v_mfma_f32_16x16x32_f16 (gemv_q4k_mf).
#include <hip/hip_runtime.h>

#include "lp_chunks.h"
#include "lp_internal.h"

namespace lp {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));

constexpr int kPlaneChunk = 1024;   // elements per workgroup in the plane kernels

// ---------------------------------------------------------------------------
// Activation planes for the GEMM, built from the quantized activations.
//   hi, lo : fp16 [M][K]        xd*q*2^-E_m split into two fp16; each group of
//                               four elements stored in the order k0 k2 k1 k3
//   shi, slo : fp16 [M][K/32]   xs*2^-E_m split likewise
//   escale : f32 [M]            2^E_m (applied to the row's outputs)
// E_m = exponent of max_b xd_mb, so |xd*q*2^-E| <= 127.

// hi = fp16(v) and lo = fp16(v - hi) must both come from the same fp32 v =
// fl(d*q): if the compiler fuses the product into the fp16 conversion of one
// use (v_fma_mix) but not the other, hi + lo misses v by an fp16 ulp at
// rounding ties. Contraction is off and v passes through an empty asm.
// Split-precision planes (SP, for the prefill GEMM) replace lo by the e4m3
// residual of hi = fp16(t * 2^9): lo8 = e4m3(t * 2^9 - hi), stored per
// 64-element chunk in the [g][s][e] order the GEMM's fp8 MFMA reads.
__device__ __forceinline__ uint32_t lo8_index(int k) {
    const int p = k & 63;
    return (uint32_t)((k & ~63) + 32 * ((p >> 3) & 1) + 8 * (p >> 4) + (p & 7));
}

// Four values of one group (in stored order k0 k2 k1 k3): hi and lo planes.
template <bool SP>
__device__ __forceinline__ void store_group(float t[4], _Float16* hi, _Float16* lo, size_t rowoff, int k) {
#pragma clang fp contract(off)
    h4 vh, vl;
    float r[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        float v = SP ? t[c] * 512.0f : t[c];
        asm volatile("" : "+v"(v));   // hi and lo both from fl32(v): no fused fp16 product
        const _Float16 h = (_Float16)v;
        vh[c] = h;
        r[c] = v - (float)h;
        vl[c] = (_Float16)r[c];
    }
    *reinterpret_cast<h4*>(hi + rowoff + k) = h4{vh[0], vh[2], vh[1], vh[3]};
    if (SP) {
        typedef short s2 __attribute__((ext_vector_type(2)));
        s2 w = {0, 0};
        w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(w, h2{vl[0], vl[2]}, 1.0f, false);
        w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(w, h2{vl[1], vl[3]}, 1.0f, true);
        *reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(lo) + rowoff + lo8_index(k)) =
            __builtin_bit_cast(uint32_t, w);
    } else {
        *reinterpret_cast<h4*>(lo + rowoff + k) = h4{vl[0], vl[2], vl[1], vl[3]};
    }
}

template <bool SP>
__global__ void __launch_bounds__(256)
gemm_prep_kernel(ActView A, int K, _Float16* __restrict__ hi, _Float16* __restrict__ lo,
                 _Float16* __restrict__ shi, _Float16* __restrict__ slo,
                 float* __restrict__ escale, float* __restrict__ yz, int N) {
#pragma clang fp contract(off)
    const int m = blockIdx.y;
    if (yz && blockIdx.x == 0)
        for (int i = threadIdx.x; i < N; i += blockDim.x) yz[(size_t)m * N + i] = 0.0f;
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
    const int e = row_exponent(mx);
    const float inv = ldexpf(1.0f, -e);
    if (threadIdx.x == 0 && blockIdx.x == 0) escale[m] = ldexpf(1.0f, e);
    // this workgroup's chunk: 4 codes per thread
    const int k = 4 * (blockIdx.x * (int)blockDim.x + (int)threadIdx.x);
    if (k < K) {
        const uint32_t qq = *reinterpret_cast<const uint32_t*>(A.qs + (size_t)m * K + k);
        const float ds = d[k >> 5] * inv;
        float t[4];
#pragma unroll
        for (int c = 0; c < 4; c++) t[c] = ds * (float)(int8_t)(qq >> (8 * c));
        store_group<SP>(t, hi, lo, (size_t)m * K, k);
        if ((k & 31) == 0) {
            const int b = k >> 5;
            float v = s[b] * inv;
            asm volatile("" : "+v"(v));
            const _Float16 h = (_Float16)v;
            shi[(size_t)m * nb + b] = h;
            slo[(size_t)m * nb + b] = (_Float16)(v - (float)h);
        }
    }
}

// 8 codes (bytes b0..b7 in u0,u1; nibble half `hi`) -> 8 fp16 V = sc * nibble,
// in the order b0 b2 b1 b3 b4 b6 b5 b7: masking a dword's nibbles into fp16
// 1024 + n (or 1024 + 16n) yields bytes 0 and 2 in one step and, after a
// shift by 8, bytes 1 and 3. The activation planes store each group of four
// elements in the same order (k0 k2 k1 k3), so every MFMA sums the same
// products as the natural order.
__device__ __forceinline__ h8 decode_v(uint32_t u0, uint32_t u1, bool hi_nib, h2 mul, h2 add) {
    const uint32_t mask = hi_nib ? 0x00f000f0u : 0x000f000fu;
    h8 out;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const uint32_t u = t < 2 ? u0 : u1;
        // (x & mask) | (0x64006400 & ~mask) in one v_bfi_b32 (the two fields are disjoint)
        uint32_t mg;
        asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(mg) : "v"(mask), "v"((t & 1) ? (u >> 8) : u), "s"(0x64006400u));
        const h2 hv = __builtin_bit_cast(h2, mg);
        const h2 v = __builtin_elementwise_fma(hv, mul, add);  // (h - 1024) * scale, exact
        out[2 * t] = v[0];
        out[2 * t + 1] = v[1];
    }
    return out;
}

// LDS reads are issued as inline assembly with explicit lgkmcnt waits. A
// compiler-generated ds_read after direct-to-LDS copies makes the compiler
// wait for every outstanding copy (vmcnt(0)), including the prefetches of
// later K steps, which serialises the copy pipeline; the copies a read
// depends on are instead waited for explicitly (wait_dma + s_barrier).
__device__ __forceinline__ uint32_t lds_addr(const uint8_t* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint8_t*)p;
}
template <int OFF>
__device__ __forceinline__ void lds_rd128(h8& out, uint32_t a) {
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(out) : "v"(a), "n"(OFF));
}
template <int OFF>
__device__ __forceinline__ void lds_rd128u(u32x4& out, uint32_t a) {
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(out) : "v"(a), "n"(OFF));
}
template <int OFF>
__device__ __forceinline__ void lds_rd64(uint2& out, uint32_t a) {
    asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(out) : "v"(a), "n"(OFF));
}

__device__ __forceinline__ h8 min_codes(uint32_t hy, uint32_t hz, uint32_t hw) {
    h8 mm;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        uint32_t mn;
        if (j < 4) mn = __builtin_amdgcn_ubfe(hz, 8 * j, 6);
        else mn = __builtin_amdgcn_ubfe(hw, 8 * (j - 4) + 4, 4) | (__builtin_amdgcn_ubfe(hz, 8 * (j - 4) + 6, 2) << 4);
        mm[j] = (_Float16)(float)mn;
    }
    return mm;
}


// ---------------------------------------------------------------------------
// Split-precision prefill GEMM (Q4_K, M > 32).
//
// Operands (per 64-element K step):
//   hi[m,k]  fp16(t),  t = xd_mb * q_mk * 2^(9 - E_m)  (|t| <= 65024)
//   lo[m,k]  e4m3(t - hi)                  (the fp16 rounding residual)
//   V[n,k]   sc_nb * nib_nk / 4            (<= 236.25: exact in fp16)
//   V8[n,k]  e4m3(V)                       (converted in registers)
// main = sum_k hi*V (v_mfma_f32_32x32x16_f16, exact products) + sum_k lo*V8
// (v_mfma_f32_32x32x64_f8f6f4, one instruction per 64-K step and tile), so
// main = 2^7 * sum_k xd*q*2^-E * sc*nib up to the residual term's error:
// |lo| <= 2^-11 |t| and the two e4m3 roundings (relative 2^-4 each) leave a
// per-product error below 2^-14 of |t*V| (2^-17 typical). The fp8 MFMA runs
// at twice the fp16 rate, so a product costs 1.5 fp16-MFMA units, against 2
// for an fp16 hi/lo pair of planes.
// Per super-block: acc += d_n * 2^-7 * main - dmin_n * sum_b m_nb * xs_mb
// (the min term: xs split into fp16 hi/lo against the exact 6-bit m).
//
// Workgroup = NW waves, tile 32*TT tokens x 32*NW weight rows; wave w owns
// every token of the tile and weight rows w*32 .. +32: TT MFMA tiles of
// 32 x 32 (A = activations, B = weights; D lane = weight row, 16 tokens).
// One decoded weight tile feeds TT token tiles, so the VALU work per MFMA
// (nibble decode, e4m3 conversion, scales) shrinks as 1/TT; the VALU is
// what bounds this kernel (fp16 and fp8 MFMAs of one wave co-issue with the
// VALU of the other wave on its SIMD only in part).
// Per K step the hi plane (128 B per token), the lo plane (64 B per token)
// and the weight codes (32 B per row) are copied into LDS with
// buffer_load_dwordx4 ... lds (1 KiB per wave instruction; scalar per-step
// offsets), NS stages in flight; headers and activation sums once per
// super-block, double-buffered. Large shapes run 4-wave workgroups of 128 x
// 128 with two stages, two workgroups per CU: each waits at its own barrier,
// so one workgroup's MFMAs fill the other's copy and barrier stalls (8 % faster
// than one 8-wave workgroup of 128 x 256 with three stages).
//
// LDS layouts (per stage):
//   hi:    token row r at r*128; its eight 16-byte pieces (piece p holds the
//          K=16 sub-step p/2, lane half p%2) at slot p ^ ((r >> 1) & 7);
//   lo:    [lane half g][token row r][2 x 16 B] at g*BM*32 + r*32, the half
//          h (sub-steps 2h, 2h+1) at slot h ^ ((r >> 3) & 1);
//   codes: 32-row groups of 1 KiB, [half 0: 32 x 16 B][half 1: 32 x 16 B].
// The swizzles make any 16 consecutive token rows read one piece from 16
// distinct 16-byte bank groups.
//
// lo byte order: each 64-element chunk is stored as [g][s][e], byte
// 32g + 8s + e holding the residual of the hi-plane position 16s + 8g + e,
// so lane half g of the fp8 MFMA reads 32 contiguous bytes that pair with
// the V values it decoded for the four fp16 sub-steps (V8 = their e4m3).

// TT: 32-token tiles per wave (the workgroup's tokens); NW: waves (32 weight
// rows each); NS: copy stages in flight.
template <int TT, int NW, int NS>
struct SpCfg {
    static constexpr int BM = 32 * TT, BN = 32 * NW;
    static constexpr int HI = BM * 128, LO = BM * 64, CODES = BN * 32;
    static constexpr int STAGE = HI + LO + CODES;
    static constexpr int HDR = BN * 16, XS = BM * 16;
    static constexpr int SBUF = HDR + 2 * XS;
    static constexpr int LDS = NS * STAGE + 2 * SBUF;
    static constexpr int N_HI = HI / 1024, N_LO = LO / 1024, N_CODES = CODES / 1024;
    static constexpr int N_HDR = HDR / 1024, N_SB = N_HDR + 2 * XS / 1024;   // per super-block
    static constexpr int H = N_HI / NW;                                      // hi copies per wave
    static constexpr int LW = (N_LO + NW - 1) / NW, SBW = (N_SB + NW - 1) / NW;
    static_assert(N_HI % NW == 0 && N_CODES == NW && N_HDR >= 1 && XS % 1024 == 0, "copy split");
    static_assert(NS == 2 || NS == 3, "two or three stages");
};

struct SpArgs {
    const _Float16* hi;
    const uint8_t* lo;
    const _Float16* shi;
    const _Float16* slo;
    const float* escale;
    const uint8_t* w;
    size_t rb;
    float* y;
    int M, N, K;
    int ksplit;           // 2: two workgroups per tile, one per half of the super-blocks,
                          // adding into a zeroed y (two fp32 adds onto 0 give the same
                          // sum in either order)
    int ntn, ntiles;      // weight-row tiles, tiles
};

// Per-lane copy sources of one wave, fixed for the whole tile; a K step
// changes only the scalar offset. Every wave issues H hi copies and one code
// copy per K step; lo copies and the per-super-block copies (headers, then
// the two activation-sum planes) are dealt round-robin over the waves, with
// wave-uniform flags. Rows past M or N are clamped to the last one (their
// results are not stored).
template <int TT, int NW, int NS>
struct SpPlan {
    using Cf = SpCfg<TT, NW, NS>;
    Rsrc rs_hi, rs_lo, rs_w, rs_sb[Cf::SBW];
    uint32_t hi_off[Cf::H], hi_lds[Cf::H], lo_off[Cf::LW], lo_lds[Cf::LW], c_off, c_lds;
    uint32_t sb_off[Cf::SBW], sb_lds[Cf::SBW];
    int has_lo[Cf::LW], sb_kind[Cf::SBW];   // sb_kind: 0 header, 1 activation sums, -1 none
};

template <int TT, int NW, int NS>
__device__ __forceinline__ SpPlan<TT, NW, NS> sp_plan(const SpArgs& g, int m0, int n0, int wave, int lane) {
    using Cf = SpCfg<TT, NW, NS>;
    SpPlan<TT, NW, NS> d;
    const int mt = g.M - m0 < Cf::BM ? g.M - m0 : Cf::BM;
    const int nt = g.N - n0 < Cf::BN ? g.N - n0 : Cf::BN;
    const int nbk = g.K >> 5;
    d.rs_hi = make_rsrc(g.hi + (size_t)m0 * g.K, (uint32_t)mt * (uint32_t)g.K * 2);
    d.rs_lo = make_rsrc(g.lo + (size_t)m0 * g.K, (uint32_t)mt * (uint32_t)g.K);
    d.rs_w = make_rsrc(g.w + (size_t)n0 * g.rb, (uint32_t)((size_t)nt * g.rb));
#pragma unroll
    for (int i = 0; i < Cf::H; i++) {
        const int j = wave * Cf::H + i;
        const int row = 8 * j + (lane >> 3);
        const int piece = (lane & 7) ^ ((row >> 1) & 7);
        const int r = row < mt ? row : mt - 1;
        d.hi_off[i] = (uint32_t)r * (uint32_t)g.K * 2 + (uint32_t)piece * 16;
        d.hi_lds[i] = (uint32_t)j * 1024;
    }
#pragma unroll
    for (int i = 0; i < Cf::LW; i++) {
        const int j = i * NW + wave;
        d.has_lo[i] = j < Cf::N_LO;
        const int o = 1024 * (j < Cf::N_LO ? j : 0) + 16 * lane;
        const int gh = o / (Cf::BM * 32), rem = o % (Cf::BM * 32);
        const int row = rem >> 5, slot = (rem >> 4) & 1;
        const int h = slot ^ ((row >> 3) & 1);
        const int r = row < mt ? row : mt - 1;
        d.lo_off[i] = (uint32_t)r * (uint32_t)g.K + (uint32_t)(32 * gh + 16 * h);
        d.lo_lds[i] = Cf::HI + (uint32_t)o;
    }
    {
        int r = 32 * wave + (lane & 31);
        r = r < nt ? r : nt - 1;
        d.c_off = (uint32_t)((size_t)r * g.rb) + 16 + 16 * (lane >> 5);
        d.c_lds = Cf::HI + Cf::LO + (uint32_t)wave * 1024;
    }
#pragma unroll
    for (int i = 0; i < Cf::SBW; i++) {
        const int j = i * NW + wave;
        d.sb_kind[i] = -1;
        d.rs_sb[i] = d.rs_w;
        d.sb_off[i] = 0;
        d.sb_lds[i] = 0;
        if (j < Cf::N_HDR) {
            int r = 64 * j + lane;
            r = r < nt ? r : nt - 1;
            d.sb_kind[i] = 0;
            d.sb_off[i] = (uint32_t)((size_t)r * g.rb);
            d.sb_lds[i] = (uint32_t)j * 1024;
        } else if (j < Cf::N_SB) {
            const int q = j - Cf::N_HDR, per = Cf::XS / 1024;
            const int pl = q / per, part = q % per;
            int r = 64 * part + lane;
            r = r < mt ? r : mt - 1;
            d.sb_kind[i] = 1;
            d.rs_sb[i] = make_rsrc((pl ? g.slo : g.shi) + (size_t)m0 * nbk, (uint32_t)(mt * nbk * 2));
            d.sb_off[i] = (uint32_t)(r * nbk * 2);
            d.sb_lds[i] = Cf::HDR + pl * Cf::XS + part * 1024;
        }
    }
    return d;
}

// Copies of K step kt into stage `st` (+ super-block data into `sbb` when kt
// starts a super-block). Returns the number of copies issued.
template <int TT, int NW, int NS>
__device__ __forceinline__ int sp_issue(const SpPlan<TT, NW, NS>& d, int kt, uint8_t* st, uint8_t* sbb) {
    using Cf = SpCfg<TT, NW, NS>;
    const int sb = kt >> 2, jb = kt & 3;
#pragma unroll
    for (int i = 0; i < Cf::H; i++) dma16(d.rs_hi, d.hi_off[i], (uint32_t)(kt * 128), st + d.hi_lds[i]);
    dma16(d.rs_w, d.c_off, (uint32_t)(sb * 144 + 32 * jb), st + d.c_lds);
    int n = Cf::H + 1;
#pragma unroll
    for (int i = 0; i < Cf::LW; i++) {
        if (d.has_lo[i]) {
            dma16(d.rs_lo, d.lo_off[i], (uint32_t)(kt * 64), st + d.lo_lds[i]);
            n++;
        }
    }
    if (jb == 0) {
#pragma unroll
        for (int i = 0; i < Cf::SBW; i++) {
            if (d.sb_kind[i] == 0) {
                dma16(d.rs_sb[i], d.sb_off[i], (uint32_t)(sb * 144), sbb + d.sb_lds[i]);
                n++;
            } else if (d.sb_kind[i] == 1) {
                dma16(d.rs_sb[i], d.sb_off[i], (uint32_t)(sb * 16), sbb + d.sb_lds[i]);
                n++;
            }
        }
    }
    return n;
}

typedef int i8x32 __attribute__((ext_vector_type(8)));   // 32 fp8 bytes

template <int N, typename V, int T>
__device__ __forceinline__ void lgkm_wait(V (&a)[T]) {
    asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N) : "memory");
#pragma unroll
    for (int i = 0; i < T; i++) asm volatile("" : "+v"(a[i]));
}

__device__ __forceinline__ uint32_t h4_to_e4m3(uint32_t h01, uint32_t h23) {
    uint32_t w;
    asm("v_cvt_scalef32_pk_fp8_f16 %0, %1, 1.0\n\tv_cvt_scalef32_pk_fp8_f16 %0, %2, 1.0 op_sel:[0,0,1]"
        : "=&v"(w) : "v"(h01), "v"(h23));
    return w;
}
__device__ __forceinline__ uint2 h8_to_e4m3(h8 v) {
    const u32x4 q = __builtin_bit_cast(u32x4, v);
    return make_uint2(h4_to_e4m3(q.x, q.y), h4_to_e4m3(q.z, q.w));
}

// Per-block decode constants for V = sc * nibble / 4: decode_v's packed fma
// (h - 1024) * mul computes it exactly (h = 1024 + n for low nibbles, 1024 +
// 16n for high ones, hence mul = sc/4 or sc/64).
__device__ __forceinline__ void scale_pair4(uint32_t hy, uint32_t hw, int j, h2& mul, h2& add) {
    uint32_t sc;
    if (j < 4) sc = __builtin_amdgcn_ubfe(hy, 8 * j, 6);
    else sc = __builtin_amdgcn_ubfe(hw, 8 * (j - 4), 4) | (__builtin_amdgcn_ubfe(hy, 8 * (j - 4) + 6, 2) << 4);
    const float s = (j & 1) ? (float)sc * (0.0625f * 0.25f) : (float)sc * 0.25f;
    const _Float16 h = (_Float16)s, a = (_Float16)(-1024.0f * s);
    mul = h2{h, h};
    add = h2{a, a};
}

template <int TT>
__device__ __forceinline__ void rd_tiles(h8 (&o)[TT], uint32_t a) {
    lds_rd128<0>(o[0], a);
    if (TT > 1) lds_rd128<4096>(o[1 % TT], a);
    if (TT > 2) lds_rd128<8192>(o[2 % TT], a);
    if (TT > 3) lds_rd128<12288>(o[3 % TT], a);
}
template <int OFF>
__device__ __forceinline__ void lds_rd_lo(i8x32& o, uint32_t a0, uint32_t a1) {
    u32x4 p0, p1;
    lds_rd128u<OFF>(p0, a0);
    lds_rd128u<OFF>(p1, a1);
    asm volatile("" : "+v"(p0), "+v"(p1));
    o = i8x32{(int)p0.x, (int)p0.y, (int)p0.z, (int)p0.w, (int)p1.x, (int)p1.y, (int)p1.z, (int)p1.w};
}
template <int TT>
__device__ __forceinline__ void rd_lo(i8x32 (&o)[TT], uint32_t a0, uint32_t a1) {
    lds_rd_lo<0>(o[0], a0, a1);
    if (TT > 1) lds_rd_lo<1024>(o[1 % TT], a0, a1);
    if (TT > 2) lds_rd_lo<2048>(o[2 % TT], a0, a1);
    if (TT > 3) lds_rd_lo<3072>(o[3 % TT], a0, a1);
}

// Tile of linear index `lin`: groups of kGroupM token tiles walk the weight
// tiles together (consecutive tiles share a weight tile, the next kGroupM
// share the next one), so the tiles in flight on one XCD reuse both operands
// in its L2. Measured (us, groups of 8 / 2): N 4096 M 512 66-69 / 63-64,
// N 14336 M 512 162 / 158-160, N 14336 M 2048 479-481 / 472-474 (4 close
// to 2, 16 slower at M 2048).
constexpr int kGroupM = 2;
__device__ __forceinline__ void sp_tile(int lin, int ntm, int ntn, int& tm, int& tn) {
    const int per_group = kGroupM * ntn;
    const int grp = lin / per_group, in = lin % per_group;
    const int gm = ntm - grp * kGroupM < kGroupM ? ntm - grp * kGroupM : kGroupM;
    tm = grp * kGroupM + in % gm;
    tn = in / gm;
}

template <int TT, int NW, int NS>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2)))
gemm_q4k_sp(SpArgs g) {
    using C = SpCfg<TT, NW, NS>;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // blocks are dealt to the 8 XCDs round-robin: give each XCD a contiguous
    // run of linear tile indices
    const int nblk = g.ntiles * g.ksplit;
    const int bid = blockIdx.x;
    const int lin = (nblk & 7) == 0 ? (bid & 7) * (nblk >> 3) + (bid >> 3) : bid;
    const int tile = lin / g.ksplit, part = lin % g.ksplit;
    int tm, tn;
    sp_tile(tile, g.ntiles / g.ntn, g.ntn, tm, tn);
    const int m0 = tm * C::BM, n0 = tn * C::BN;
    const int nsb_all = g.K >> 8;
    const int sb_beg = part * nsb_all / g.ksplit, sb_end = (part + 1) * nsb_all / g.ksplit;
    const int kt0 = 4 * sb_beg, nk = 4 * sb_end;
    const SpPlan<TT, NW, NS> plan = sp_plan<TT, NW, NS>(g, m0, n0, wave, lane);
    auto stage = [&](int i) { return smem + i * C::STAGE; };
    auto sbuf = [&](int i) { return smem + NS * C::STAGE + i * C::SBUF; };

    const uint32_t lds0 = lds_addr(smem);
    const int gl = lane >> 5, r32 = lane & 31;
    uint32_t a_s[4], lo_h[2];
    {
        const int a_x = gl ^ ((r32 >> 1) & 7);
#pragma unroll
        for (int s = 0; s < 4; s++) a_s[s] = lds0 + r32 * 128 + (uint32_t)(((2 * s) ^ a_x) * 16);
        const int x = (r32 >> 3) & 1;
        const uint32_t lb = lds0 + C::HI + gl * C::BM * 32 + r32 * 32;
        lo_h[0] = lb + 16 * x;
        lo_h[1] = lb + 16 * (x ^ 1);
    }
    // this wave's weight rows: wave*32 + lane%32 (code group `wave`)
    const uint32_t b_base = lds0 + C::HI + C::LO + wave * 1024 + (lane & 31) * 16 + 8 * gl;
    const uint32_t hdr_base = lds0 + NS * C::STAGE + (wave * 32 + (lane & 31)) * 16;
    const uint32_t xs_base = lds0 + NS * C::STAGE + C::HDR + (lane & 31) * 16;

    f16v acc[TT], main_[TT];
#pragma unroll
    for (int a = 0; a < TT; a++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[a][r] = 0.0f;

    uint32_t hy = 0, hz = 0, hw = 0;
    float dsc = 0.0f, dmn = 0.0f;

    // NS stages: steps kt+1 .. kt+NS-2 are in flight while step kt is
    // computed; cnt_next counts the copies of step kt+1 (three stages)
    int cnt_next = 0;
    (void)sp_issue<TT, NW, NS>(plan, kt0, stage(0), sbuf(sb_beg & 1));
    if (NS == 3 && kt0 + 1 < nk) cnt_next = sp_issue<TT, NW, NS>(plan, kt0 + 1, stage(1), sbuf(sb_beg & 1));
    for (int sb = sb_beg; sb < sb_end; sb++) {
        const uint32_t sb_off = (uint32_t)((sb & 1) * C::SBUF);
#pragma unroll
        for (int jb = 0; jb < 4; jb++) {
            const int kt = 4 * sb + jb;
            wait_dma(NS == 3 ? cnt_next : 0);         // step kt has landed
            // after this barrier every wave has finished step kt-1, whose
            // stage buffer is the one step kt+NS-1 is copied into
            __builtin_amdgcn_s_barrier();
            cnt_next = 0;
            if (kt + NS - 1 < nk)
                cnt_next = sp_issue<TT, NW, NS>(plan, kt + NS - 1, stage((kt + NS - 1 - kt0) % NS),
                                                sbuf(((kt + NS - 1) >> 2) & 1));
            const uint32_t st_off = (uint32_t)(((kt - kt0) % NS) * C::STAGE);

            if (jb == 0) {
                u32x4 h;
                lds_rd128u<0>(h, hdr_base + sb_off);
                asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(h));
                dsc = fp16_bits_to_f32(h.x) * 0.0078125f;   // d * 2^-7 (main carries 2^7)
                dmn = fp16_bits_to_f32(h.x >> 16);
                hy = h.y;
                hz = h.z;
                hw = h.w;
            }
            h2 vmul[2], vadd[2];
#pragma unroll
            for (int i = 0; i < 2; i++) scale_pair4(hy, hw, 2 * jb + i, vmul[i], vadd[i]);

            // Four K=16 sub-steps on the hi plane; the weight codes are two 8-byte
            // pairs (pair s&1: sub-step s low nibbles, s+2 high nibbles).
            uint2 u[2];
            h8 ah[2][TT];                               // [s & 1][token tile]
            h8 v[2];                                    // [s & 1]
            uint2 v8[4];                                // e4m3 V of the four sub-steps
            const uint32_t bq = b_base + st_off;
            lds_rd64<0>(u[0], bq);
            lds_rd64<512>(u[1], bq);
            uint32_t as[4];
#pragma unroll
            for (int q = 0; q < 4; q++) as[q] = a_s[q] + st_off;
            rd_tiles<TT>(ah[0], as[0]);
            rd_tiles<TT>(ah[1], as[1]);
            lgkm_wait<2 * TT>(u);
            v[0] = decode_v(u[0].x, u[0].y, false, vmul[0], vadd[0]);
            i8x32 al[TT];
#pragma unroll
            for (int s = 0; s < 4; s++) {
                // LDS reads in flight behind this sub-step's TT: s=0,1: the other
                // buffer's TT; s=2: sub-step 3's TT and the 2TT residual reads;
                // s=3: those 2TT
                if (s < 2) lgkm_wait<TT>(ah[s & 1]);
                else if (s == 2) lgkm_wait<3 * TT>(ah[s & 1]);
                else lgkm_wait<2 * TT>(ah[s & 1]);
                __builtin_amdgcn_sched_barrier(0);
                __builtin_amdgcn_s_setprio(1);
#pragma unroll
                for (int tt = 0; tt < TT; tt++)
                    main_[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                        ah[s & 1][tt], v[s & 1], (jb == 0 && s == 0) ? f16v{} : main_[tt], 0, 0, 0);
                v8[s] = h8_to_e4m3(v[s & 1]);
                if (s < 3) {
                    const int sn = s + 1;
                    v[sn & 1] = decode_v(u[sn & 1].x, u[sn & 1].y, sn >= 2, vmul[sn >> 1], vadd[sn >> 1]);
                }
                __builtin_amdgcn_sched_barrier(0);
                __builtin_amdgcn_s_setprio(0);
                if (s < 2) rd_tiles<TT>(ah[s & 1], as[s + 2]);
                if (s == 1) rd_lo<TT>(al, lo_h[0] + st_off, lo_h[1] + st_off);
            }
            lgkm_wait<0>(al);
            const i8x32 b8 = {(int)v8[0].x, (int)v8[0].y, (int)v8[1].x, (int)v8[1].y,
                              (int)v8[2].x, (int)v8[2].y, (int)v8[3].x, (int)v8[3].y};
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int tt = 0; tt < TT; tt++)
                main_[tt] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(al[tt], b8, main_[tt], 0, 0, 0, 0, 0, 0);
            __builtin_amdgcn_s_setprio(0);

            if (jb == 3) {
                // min term and the super-block's scale: sum_b m * xs as a K = 16
                // product (lanes 32..63 supply k = 8..15: zero)
                h8 shv[TT], slv[TT];
#pragma unroll
                for (int tt = 0; tt < TT; tt++) {
                    lds_rd128<0>(shv[tt], xs_base + sb_off + tt * 512);
                    lds_rd128<C::XS>(slv[tt], xs_base + sb_off + tt * 512);
                }
                const h8 mm = min_codes(hy, hz, hw);
                const h8 bmin = lane < 32 ? mm : h8{0, 0, 0, 0, 0, 0, 0, 0};
                lgkm_wait<0>(shv);
                lgkm_wait<0>(slv);
#pragma unroll
                for (int tt = 0; tt < TT; tt++) {
                    if (lane >= 32) { shv[tt] = h8{0, 0, 0, 0, 0, 0, 0, 0}; slv[tt] = shv[tt]; }
                    f16v mn = __builtin_amdgcn_mfma_f32_32x32x16_f16(shv[tt], bmin, f16v{}, 0, 0, 0);
                    mn = __builtin_amdgcn_mfma_f32_32x32x16_f16(slv[tt], bmin, mn, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        acc[tt][r] = fmaf(dsc, main_[tt][r], acc[tt][r]);
                        acc[tt][r] = fmaf(-dmn, mn[r], acc[tt][r]);
                    }
                }
            }
        }
    }

    // store: D[token][row] -> y[token * N + row] * 2^E_token
    const int n = n0 + wave * 32 + (lane & 31);   // D lane = weight row
#pragma unroll
    for (int tt = 0; tt < TT; tt++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int m = m0 + tt * 32 + 8 * (r >> 2) + 4 * gl + (r & 3);
            if (m < g.M && n < g.N) {
                const float val = acc[tt][r] * g.escale[m];
                if (g.ksplit == 1) g.y[(size_t)m * g.N + n] = val;
                else atomicAdd(&g.y[(size_t)m * g.N + n], val);
            }
        }
}

// ---------------------------------------------------------------------------
// Planes of M activation rows carved from one buffer (256-byte aligned).

struct Planes {
    _Float16* hi;
    _Float16* lo;
    _Float16* shi;
    _Float16* slo;
    float* escale;
};

static Planes carve_planes(void* base, int M, int K) {
    auto r = [](size_t v) { return (v + 255) / 256 * 256; };
    uint8_t* p = static_cast<uint8_t*>(base);
    Planes P;
    P.hi = reinterpret_cast<_Float16*>(p);
    p += r((size_t)M * K * 2);
    P.lo = reinterpret_cast<_Float16*>(p);
    p += r((size_t)M * K * 2);
    P.shi = reinterpret_cast<_Float16*>(p);
    p += r((size_t)M * (K / 32) * 2);
    P.slo = reinterpret_cast<_Float16*>(p);
    p += r((size_t)M * (K / 32) * 2);
    P.escale = reinterpret_cast<float*>(p);
    return P;
}

// Quantize fp32 activation rows and write their planes, one workgroup per
// row, without storing the ActQ8 blocks: the same values as
// quantize_act_kernel followed by gemm_prep_kernel. The row is read once into
// registers (NF float4 per thread, 8 consecutive threads per 32-element
// block). Pass 1: block scales and their row maximum (the exponent E); pass
// 2: codes, hi/lo and shi/slo from the registers.
template <int NF, bool SP>
__global__ void __launch_bounds__(1024)
quant_planes_kernel(const float* __restrict__ x, int K, Planes P, float* __restrict__ yz, int N) {
#pragma clang fp contract(off)
    const int m = blockIdx.x;
    if (yz)
        for (int i = threadIdx.x; i < N; i += blockDim.x) yz[(size_t)m * N + i] = 0.0f;
    const float4* xr = reinterpret_cast<const float4*>(x + (size_t)m * K);
    const int n4 = K >> 2, nb = K >> 5;
    const int nt = blockDim.x;
    float4 v[NF];
#pragma unroll
    for (int j = 0; j < NF; j++) {
        const int i = threadIdx.x + j * nt;
        v[j] = i < n4 ? xr[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    // pass 1: the largest block scale. Block scales are fl(amax_b / 127),
    // monotone in amax_b, so their maximum is fl(max amax_b / 127), over the
    // blocks without a NaN (a NaN block's scale is NaN, which the maximum skips).
    __shared__ float red[32];
    float mx = 0.0f;
#pragma unroll
    for (int j = 0; j < NF; j++) {
        const float4 u = v[j];
        float amax = fmaxf(fmaxf(fabsf(u.x), fabsf(u.y)), fmaxf(fabsf(u.z), fabsf(u.w)));
        int nan = (u.x != u.x) | (u.y != u.y) | (u.z != u.z) | (u.w != u.w);
#pragma unroll
        for (int off = 1; off < 8; off <<= 1) {
            amax = fmaxf(amax, __shfl_xor(amax, off, 8));
            nan |= __shfl_xor(nan, off, 8);
        }
        if (!nan) mx = fmaxf(mx, amax);
    }
#pragma unroll
    for (int off = 8; off < 64; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = 0.0f;
    for (int wv = 0; wv < (nt + 63) / 64; wv++) mx = fmaxf(mx, red[wv]);
    mx = mx / 127.0f;
    const int e = row_exponent(mx);
    const float inv = ldexpf(1.0f, -e);
    if (threadIdx.x == 0) P.escale[m] = ldexpf(1.0f, e);
    // pass 2
#pragma unroll
    for (int j = 0; j < NF; j++) {
        const int i = threadIdx.x + j * nt;
        const Q8Group q = quant_group8(v[j]);
        if (i < n4) {
            const float ds = q.d * inv;
            float t[4];
#pragma unroll
            for (int c = 0; c < 4; c++) t[c] = ds * (float)(int8_t)(q.packed >> (8 * c));
            store_group<SP>(t, P.hi, P.lo, (size_t)m * K, 4 * i);
            if ((i & 7) == 0) {
                const int b = i >> 3;
                float xs = q.sum * inv;
                asm volatile("" : "+v"(xs));
                const _Float16 h = (_Float16)xs;
                P.shi[(size_t)m * nb + b] = h;
                P.slo[(size_t)m * nb + b] = (_Float16)(xs - (float)h);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Small-M Q4_K product on MFMA: M <= 16 activation rows (tokens) against
// every weight row, with the prefill GEMM's exact operand folding (A = the
// tokens' hi/lo planes, B = V = sc * nibble in fp16) on
// v_mfma_f32_16x16x32_f16: one MFMA pair per 32-element sub-block, so the
// per-element VALU work is the nibble decode alone, independent of M.
//
// Workgroup = kMfTiles x 16 weight rows x kMfWaves waves; wave w takes the
// super-blocks [w*nsb/8, (w+1)*nsb/8) of all the rows (one activation load
// feeds kMfTiles MFMA pairs), and the waves' partial sums are added in a
// fixed order through LDS. Lane l: A row (token) l%16, B column
// (weight row) l%16, k = 8*(l/16) .. +8 of the sub-block; D: weight row
// l%16, tokens 4*(l/16) .. +4. Lanes load their row's super-block header
// and their 8-byte slice of each 32-byte code quarter directly (cached).
// Used for K beyond the int8 kernel's LDS limit (gemv_q4k_i8mf below).

constexpr int kMfWaves = 8;
constexpr int kMfTiles = 2;         // 16-row tiles per workgroup (every wave takes all of them)
constexpr int kI8ChunkTt = 2;      // Q8_0 / Q6_K prefill chunks: 16-token tiles per workgroup
constexpr bool kQ6Chunk = true;
constexpr bool kQ40Chunk = true;
constexpr int kMfMoeWaves = 2;      // grouped MoE: waves per workgroup
constexpr int kMfMoeRows = 64;    // grouped MoE: weight rows per workgroup (at least two sets)
constexpr int kMfMaxM = 16;
// Measured on MI355X (Q4_K 18944 x 3584): the GEMV tile kernel is faster
// up to M = 4, the small-M MFMA kernels from M = 5 to 16.
constexpr int kMfMinM = 5;
typedef float f4v __attribute__((ext_vector_type(4)));

struct MfArgs {
    const uint8_t* w;
    long rb;              // bytes per weight row
    int N, K, M;
    Planes P;
    float* y;
};

__global__ void __launch_bounds__(64 * kMfWaves)
gemv_q4k_mf(MfArgs a) {
    __shared__ f4v red[kMfWaves][kMfTiles][64];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int tok = lane & 15, g = lane >> 4;
    const int M = a.M;
    const uint8_t* w = a.w;
    const bool tv = tok < M;
    const int arow = tv ? tok : 0;
    const int row0 = blockIdx.x * (16 * kMfTiles) + (lane & 15);
    const int nsb = a.K >> 8, nb = a.K >> 5;
    const int sb0 = wv * nsb / kMfWaves, sb1 = (wv + 1) * nsb / kMfWaves;
    const uint8_t* wr[kMfTiles];
#pragma unroll
    for (int t = 0; t < kMfTiles; t++) {
        int row = row0 + 16 * t;
        row = row < a.N ? row : a.N - 1;
        wr[t] = w + (size_t)row * a.rb;
    }
    const _Float16* ahi = a.P.hi + (size_t)arow * a.K + 8 * g;
    const _Float16* alo = a.P.lo + (size_t)arow * a.K + 8 * g;
    const _Float16* xsh = a.P.shi + (size_t)arow * nb;
    const _Float16* xsl = a.P.slo + (size_t)arow * nb;
    const h8 z8 = {0, 0, 0, 0, 0, 0, 0, 0};
    const f4v z4 = {0.0f, 0.0f, 0.0f, 0.0f};

    f4v acc[kMfTiles];
#pragma unroll
    for (int t = 0; t < kMfTiles; t++) acc[t] = z4;
    for (int s = sb0; s < sb1; s++) {
        u32x4 h[kMfTiles];
        uint2 q[kMfTiles][4];
#pragma unroll
        for (int t = 0; t < kMfTiles; t++) {
            const uint8_t* blk = wr[t] + 144 * s;
            h[t] = *reinterpret_cast<const u32x4*>(blk);
#pragma unroll
            for (int jb = 0; jb < 4; jb++) q[t][jb] = *reinterpret_cast<const uint2*>(blk + 16 + 32 * jb + 8 * g);
        }
        f4v mainv[kMfTiles];
        h8 mm[kMfTiles];
#pragma unroll
        for (int t = 0; t < kMfTiles; t++) mainv[t] = z4;
#pragma unroll
        for (int b = 0; b < 8; b++) {
            const int k0 = 32 * (8 * s + b);
            const h8 vh = tv ? *reinterpret_cast<const h8*>(ahi + k0) : z8;
            const h8 vl = tv ? *reinterpret_cast<const h8*>(alo + k0) : z8;
#pragma unroll
            for (int t = 0; t < kMfTiles; t++) {
                uint32_t sc, mn;
                scale_min_k4(b, h[t].y, h[t].z, h[t].w, sc, mn);
                mm[t][b] = (_Float16)(float)mn;
                // even blocks use low nibbles (1024 + n), odd high (1024 + 16n)
                const float sf = (b & 1) ? (float)sc * 0.0625f : (float)sc;
                const _Float16 hs = (_Float16)sf, ha = (_Float16)(-1024.0f * sf);
                const h8 v = decode_v(q[t][b >> 1].x, q[t][b >> 1].y, (b & 1) != 0, h2{hs, hs}, h2{ha, ha});
                mainv[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, v, mainv[t], 0, 0, 0);
                mainv[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vl, v, mainv[t], 0, 0, 0);
            }
        }
        // min term: sum_b m_b * xs_b as a K = 8 product (k = 8g + e; only g = 0 non-zero)
        const h8 sh = (tv && g == 0) ? *reinterpret_cast<const h8*>(xsh + 8 * s) : z8;
        const h8 sl = (tv && g == 0) ? *reinterpret_cast<const h8*>(xsl + 8 * s) : z8;
#pragma unroll
        for (int t = 0; t < kMfTiles; t++) {
            const h8 mb = g == 0 ? mm[t] : z8;
            f4v mnv = __builtin_amdgcn_mfma_f32_16x16x32_f16(sh, mb, z4, 0, 0, 0);
            mnv = __builtin_amdgcn_mfma_f32_16x16x32_f16(sl, mb, mnv, 0, 0, 0);
            const float d = fp16_bits_to_f32(h[t].x), dmin = fp16_bits_to_f32(h[t].x >> 16);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                acc[t][r] = fmaf(d, mainv[t][r], acc[t][r]);
                acc[t][r] = fmaf(-dmin, mnv[r], acc[t][r]);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < kMfTiles; t++) red[wv][t][lane] = acc[t];
    __syncthreads();
    // wave t sums tile t over the K-slices in a fixed order
    if (wv < kMfTiles) {
        const int t = wv;
        f4v sum = red[0][t][lane];
#pragma unroll
        for (int i = 1; i < kMfWaves; i++) sum += red[i][t][lane];
        const int row = row0 + 16 * t;
        if (row < a.N) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int tt = 4 * g + r;
                if (tt < M) a.y[(size_t)tt * a.N + row] = sum[r] * a.P.escale[tt];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Q4_K for 5 <= M <= 16 activation rows on int8 MFMA (v_mfma_i32_16x16x32_i8,
// one 32-element block per instruction): A = the tokens' int8 codes straight
// from the quantized blocks (16 rows, unused rows zero), B = the weights'
// 4-bit codes as int8 (16 weight rows), D = the exact per-block int32 sums
// P_mnb of the reference's dot_row_q4_k_int_neon (src/matmul_simd.cpp:226-283).
// Epilogue per block: acc += P * (xd_m * d_n*sc_nb); per super-block the min
// term -dmin_n * sum_b m_nb * xs_mb. Same workgroup shape as gemv_q4k_mf
// (32 weight rows x 8 waves, each wave a K-slice of whole super-blocks, slices
// summed in a fixed order through LDS); the activation codes are read once
// per workgroup (one byte per element, a quarter of the fp16 hi/lo planes'
// traffic), and the block scales and sums are staged in LDS as [block][token]
// so a lane's four tokens come in one read. Operand layout checked on the
// device: A row = lane%16, k = 8*(lane/16)+e; B column = lane%16; D row =
// 4*(lane/16)+r, column = lane%16.
typedef int i4v __attribute__((ext_vector_type(4)));

// K-slices for a row of nsb super-blocks over nwv waves: the largest power
// of two <= min(nsb, nwv) (nwv a power of two)
__host__ __device__ inline int mf_kslices(int nsb, int nwv) {
    int k = 1;
    while (2 * k <= nsb && 2 * k <= nwv) k *= 2;
    return k;
}

// MOE: blockIdx.y is a routed group (expert, first pair, n <= 16 pairs): the
// group's activation rows (token, or pair in the multi form) and outputs
// (pair rows) replace rows 0..M-1.
// TL 16-row tiles per row set, NWV waves (K-slices); ri row sets per
// workgroup, one after another, all served by one activation staging. RWS:
// as many K-slices as the row has super-blocks (a power of two, at most
// NWV), the remaining waves on further row tiles of the set.
template <bool MOE, int TL = kMfTiles, int NWV = kMfWaves, bool RWS = false>
__global__ void __launch_bounds__(64 * NWV)
gemv_q4k_i8mf(const uint8_t* __restrict__ w, long rb, ActView A, float* __restrict__ y, int M, int K, int N,
              const uint8_t* __restrict__ route, int max_groups, int multi, int topk, long ebytes, int ri = 1) {
    __shared__ f4v red[NWV][TL][64];
    extern __shared__ __attribute__((aligned(16))) float sdx[];   // [nb][16] xd, then [nb][16] xs
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int tok = lane & 15, g = lane >> 4;
    const int nsb = K >> 8, nb = K >> 5;
    const int* pairs = nullptr;
    int first = 0;
    if constexpr (MOE) {
        if ((int)blockIdx.y >= *reinterpret_cast<const int*>(route)) return;
        const int4 gd = reinterpret_cast<const int4*>(route + 16)[blockIdx.y];
        pairs = reinterpret_cast<const int*>(route + 16 + (size_t)max_groups * 16);
        first = gd.y;
        M = gd.z;
        w += (size_t)gd.x * ebytes;
    }
    auto act_row = [&](int t) -> int {
        if constexpr (MOE) {
            const int p = pairs[first + t];
            return multi ? p : p / topk;
        } else {
            return t;
        }
    };
    float* sxs = sdx + (size_t)nb * 16;
    for (int i = threadIdx.x; i < nb * 16; i += blockDim.x) {
        const int b = i >> 4, t = i & 15;
        const size_t r = t < M ? (size_t)act_row(t) : 0;
        sdx[i] = t < M ? A.d[r * nb + b] : 0.0f;
        sxs[i] = t < M ? A.sum[r * nb + b] : 0.0f;
    }
    __syncthreads();
    const bool tv = tok < M;
    const int8_t* aq = A.qs + (size_t)act_row(tv ? tok : 0) * K + 8 * g;
    // RWS: K-slices of whole super-blocks, as many as the row has (a power of
    // two, at most NWV), the other waves on further row tiles
    const int ks_n = RWS ? mf_kslices(nsb, NWV) : NWV, rw_n = NWV / ks_n;
    const int ks = wv % ks_n, rw = wv / ks_n;
    const int sb0 = ks * nsb / ks_n, sb1 = (ks + 1) * nsb / ks_n;
    // ri consecutive row sets per workgroup: the activation staging above
    // serves all of them
    for (int it = 0; it < ri; it++) {
    const int rbase = (blockIdx.x * ri + it) * rw_n * (16 * TL);
    if (rbase >= N) break;
    const int row0 = rbase + rw * (16 * TL) + (lane & 15);
    const uint8_t* wr[TL];
#pragma unroll
    for (int t = 0; t < TL; t++) {
        int row = row0 + 16 * t;
        row = row < N ? row : N - 1;
        wr[t] = w + (size_t)row * rb;
    }
    const i4v zi = {0, 0, 0, 0};
    const f4v z4 = {0.0f, 0.0f, 0.0f, 0.0f};
    f4v acc[TL];
#pragma unroll
    for (int t = 0; t < TL; t++) acc[t] = z4;
    for (int s = sb0; s < sb1; s++) {
        u32x4 h[TL];
        uint2 q[TL][4];
#pragma unroll
        for (int t = 0; t < TL; t++) {
            const uint8_t* blk = wr[t] + 144 * s;
            h[t] = *reinterpret_cast<const u32x4*>(blk);
#pragma unroll
            for (int jb = 0; jb < 4; jb++) q[t][jb] = *reinterpret_cast<const uint2*>(blk + 16 + 32 * jb + 8 * g);
        }
        long av[8];
#pragma unroll
        for (int b = 0; b < 8; b++) av[b] = tv ? *reinterpret_cast<const long*>(aq + 32 * (8 * s + b)) : 0L;
        f4v mnacc[TL];
#pragma unroll
        for (int t = 0; t < TL; t++) mnacc[t] = z4;
#pragma unroll
        for (int b = 0; b < 8; b++) {
            const f4v xd = *reinterpret_cast<const f4v*>(sdx + (size_t)(8 * s + b) * 16 + 4 * g);
            const f4v xs = *reinterpret_cast<const f4v*>(sxs + (size_t)(8 * s + b) * 16 + 4 * g);
#pragma unroll
            for (int t = 0; t < TL; t++) {
                uint32_t sc, mn;
                scale_min_k4(b, h[t].y, h[t].z, h[t].w, sc, mn);
                const uint2 u = q[t][b >> 1];
                const uint32_t lo = (b & 1) ? (u.x >> 4) & 0x0f0f0f0fu : u.x & 0x0f0f0f0fu;
                const uint32_t hi = (b & 1) ? (u.y >> 4) & 0x0f0f0f0fu : u.y & 0x0f0f0f0fu;
                const long bw = (long)((unsigned long)lo | ((unsigned long)hi << 32));
                const i4v S = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[b], bw, zi, 0, 0, 0);
                const float dsc = fp16_bits_to_f32(h[t].x) * (float)sc;
                const float fm = (float)mn;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    acc[t][r] = fmaf((float)S[r], xd[r] * dsc, acc[t][r]);
                    mnacc[t][r] = fmaf(fm, xs[r], mnacc[t][r]);
                }
            }
        }
#pragma unroll
        for (int t = 0; t < TL; t++) {
            const float dmin = fp16_bits_to_f32(h[t].x >> 16);
#pragma unroll
            for (int r = 0; r < 4; r++) acc[t][r] = fmaf(-dmin, mnacc[t][r], acc[t][r]);
        }
    }
#pragma unroll
    for (int t = 0; t < TL; t++) red[wv][t][lane] = acc[t];
    __syncthreads();
    // each output tile summed over its K-slices in a fixed order
    for (int o = wv; o < rw_n * TL; o += NWV) {
        const int ro = o / TL, t = o % TL;
        f4v sum = red[ro * ks_n][t][lane];
        for (int i = 1; i < ks_n; i++) sum += red[ro * ks_n + i][t][lane];
        const int row = rbase + ro * (16 * TL) + 16 * t + (lane & 15);
        if (row < N) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int tt = 4 * g + r;
                if (tt < M) {
                    int yr;
                    if constexpr (MOE) yr = pairs[first + tt];
                    else yr = tt;
                    y[(size_t)yr * N + row] = sum[r];
                }
            }
        }
    }
    if (ri > 1) __syncthreads();                  // red is reused by the next row set
    }
}

// Q6_K for 5 <= M <= 16 on the same int8 MFMA: B = the 6-bit codes minus 32
// as int8 (ql nibble | qh bits << 4, then -32 per byte), so D is the exact
// sum of (code - 32) * q. The two 16-element halves of a 32-element block
// have their own int8 scale, so a block takes two MFMAs (lanes of the other
// half zeroed in B) and the epilogue adds (xd*d) * (sc0*S0 + sc1*S1)
// (dot_row_q6_k_int_neon, src/matmul_simd.cpp:285-342). The 210-byte blocks
// are 2-byte aligned: each 8-byte piece is read as three dwords from the
// aligned-down address and funnel-shifted.
// 8 bytes at a 2-byte aligned address, read without touching a byte past
// them: two dwords when 4-byte aligned, else the dwords at p-2 and p+2 and
// the halfword at p+6.
__device__ __forceinline__ uint2 ld8_a2(const uint8_t* p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    if ((a & 3) == 0) return *reinterpret_cast<const uint2*>(p);
    const uint32_t* q = reinterpret_cast<const uint32_t*>(a - 2);
    const uint32_t d0 = q[0], d1 = q[1];
    const uint32_t t = *reinterpret_cast<const uint16_t*>(p + 6);
    return make_uint2((d0 >> 16) | (d1 << 16), (d1 >> 16) | (t << 16));
}

template <int TL, int NWV, int TT = 1>
__global__ void __launch_bounds__(64 * NWV)
gemv_q6k_i8mf(const uint8_t* __restrict__ w, long rb, ActView A, float* __restrict__ y, int M, int K, int N) {
    static_assert(TL * TT <= NWV, "one wave per output tile in the final sum");
    constexpr int TK = 16 * TT;                  // tokens per workgroup (TT 16-token tiles)
    __shared__ f4v red[NWV][TL * TT][64];
    extern __shared__ __attribute__((aligned(16))) float sdx[];   // [nb][TK] xd
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int tok = lane & 15, g = lane >> 4;
    const int nsb = K >> 8, nb = K >> 5;
    for (int i = threadIdx.x; i < nb * TK; i += blockDim.x) {
        const int b = i / TK, t = i % TK;
        sdx[i] = t < M ? A.d[(size_t)t * nb + b] : 0.0f;
    }
    __syncthreads();
    bool tv[TT];
    const int8_t* aq[TT];
#pragma unroll
    for (int u = 0; u < TT; u++) {
        tv[u] = tok + 16 * u < M;
        aq[u] = A.qs + (size_t)(tv[u] ? tok + 16 * u : 0) * K + 8 * g;
    }
    const int row0 = blockIdx.x * (16 * TL) + (lane & 15);
    const int sb0 = wv * nsb / NWV, sb1 = (wv + 1) * nsb / NWV;
    const uint8_t* wr[TL];
#pragma unroll
    for (int t = 0; t < TL; t++) {
        int row = row0 + 16 * t;
        row = row < N ? row : N - 1;
        wr[t] = w + (size_t)row * rb;
    }
    const bool first_half = g < 2;                 // k 0..15 of the block
    const i4v zi = {0, 0, 0, 0};
    const f4v z4 = {0.0f, 0.0f, 0.0f, 0.0f};
    f4v acc[TL][TT];
#pragma unroll
    for (int t = 0; t < TL; t++)
#pragma unroll
        for (int u = 0; u < TT; u++) acc[t][u] = z4;
    for (int s = sb0; s < sb1; s++) {
        uint2 ql[TL][4], qh[TL][2];
        uint32_t scw[TL][4];
        float d[TL];
#pragma unroll
        for (int t = 0; t < TL; t++) {
            const uint8_t* blk = wr[t] + 210 * (size_t)s;
#pragma unroll
            for (int i = 0; i < 4; i++) ql[t][i] = ld8_a2(blk + 64 * (i >> 1) + 32 * (i & 1) + 8 * g);
#pragma unroll
            for (int i = 0; i < 2; i++) qh[t][i] = ld8_a2(blk + 128 + 32 * i + 8 * g);
            const uint2 s0 = ld8_a2(blk + 192), s1 = ld8_a2(blk + 200);
            scw[t][0] = s0.x; scw[t][1] = s0.y; scw[t][2] = s1.x; scw[t][3] = s1.y;
            d[t] = fp16_bits_to_f32(*reinterpret_cast<const uint16_t*>(blk + 208));
        }
        long av[TT][8];
#pragma unroll
        for (int u = 0; u < TT; u++)
#pragma unroll
            for (int b = 0; b < 8; b++)
                av[u][b] = tv[u] ? *reinterpret_cast<const long*>(aq[u] + 32 * (8 * s + b)) : 0L;
#pragma unroll
        for (int b = 0; b < 8; b++) {
            const int h = b >> 2, g6 = b & 3;
#pragma unroll
            for (int t = 0; t < TL; t++) {
                const uint2 l = ql[t][2 * h + (g6 & 1)], hh = qh[t][h];
                const int ns = 4 * (g6 >> 1), hs = 2 * g6;
                uint32_t c0 = ((l.x >> ns) & 0x0f0f0f0fu) | (((hh.x >> hs) & 0x03030303u) << 4);
                uint32_t c1 = ((l.y >> ns) & 0x0f0f0f0fu) | (((hh.y >> hs) & 0x03030303u) << 4);
                // code - 32 per byte (codes 0..63: no borrow across bytes)
                c0 = ((c0 | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
                c1 = ((c1 | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
                const long bw = (long)((unsigned long)c0 | ((unsigned long)c1 << 32));
                const long b0 = first_half ? bw : 0L, b1 = first_half ? 0L : bw;
                const int si = 8 * h + 2 * g6;          // scales of the block's two halves
                const float sc0 = (float)(int8_t)(scw[t][si >> 2] >> (8 * (si & 3)));
                const float sc1 = (float)(int8_t)(scw[t][(si + 1) >> 2] >> (8 * ((si + 1) & 3)));
#pragma unroll
                for (int u = 0; u < TT; u++) {
                    const f4v xd = *reinterpret_cast<const f4v*>(sdx + (size_t)(8 * s + b) * TK + 16 * u + 4 * g);
                    const i4v S0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[u][b], b0, zi, 0, 0, 0);
                    const i4v S1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[u][b], b1, zi, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const float dx = d[t] * xd[r];
                        acc[t][u][r] = fmaf(dx * sc0, (float)S0[r], acc[t][u][r]);
                        acc[t][u][r] = fmaf(dx * sc1, (float)S1[r], acc[t][u][r]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int t = 0; t < TL; t++)
#pragma unroll
        for (int u = 0; u < TT; u++) red[wv][t * TT + u][lane] = acc[t][u];
    __syncthreads();
    // wave i sums output tile i (row tile i / TT, token tile i % TT)
    if (wv < TL * TT) {
        const int t = wv / TT, u = wv % TT;
        f4v sum = red[0][wv][lane];
#pragma unroll
        for (int i = 1; i < NWV; i++) sum += red[i][wv][lane];
        const int row = row0 + 16 * t;
        if (row < N) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int tt = 16 * u + 4 * g + r;
                if (tt < M) y[(size_t)tt * N + row] = sum[r];
            }
        }
    }
}

// Q8_0 for 9 <= M <= 16 on the same int8 MFMA: one 32-element block per
// instruction, B = the int8 codes, epilogue acc += P * (xd * fp16(d))
// (dot_row_q8_0_int_neon, src/matmul_simd.cpp:143-160). Waves take K-slices
// of 8-block groups; the 34-byte blocks are 2-byte aligned.
// TT 16-token tiles per workgroup (M <= 16 TT): each weight fragment feeds
// TT MFMAs, so prefill chunks of 32-64 rows read the weights once per chunk.
template <uint32_t T, int TL, int NWV, int TT = 1>
__global__ void __launch_bounds__(64 * NWV)
gemv_b32_i8mf(const uint8_t* __restrict__ w, long rb, ActView A, float* __restrict__ y, int M, int K, int N) {
    static_assert(T == T_Q8_0 || T == T_Q4_0, "Q8_0 / Q4_0");
    static_assert(TL * TT <= NWV, "one wave per output tile in the final sum");
    constexpr int BPB = T == T_Q8_0 ? 34 : 18;
    constexpr int TK = 16 * TT;
    __shared__ f4v red[NWV][TL * TT][64];
    extern __shared__ __attribute__((aligned(16))) float sdx[];   // [nb][TK] xd
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int tok = lane & 15, g = lane >> 4;
    const int nb = K >> 5, ngr = K >> 8;
    for (int i = threadIdx.x; i < nb * TK; i += blockDim.x) {
        const int b = i / TK, t = i % TK;
        sdx[i] = t < M ? A.d[(size_t)t * nb + b] : 0.0f;
    }
    __syncthreads();
    bool tv[TT];
    const int8_t* aq[TT];
#pragma unroll
    for (int u = 0; u < TT; u++) {
        tv[u] = tok + 16 * u < M;
        aq[u] = A.qs + (size_t)(tv[u] ? tok + 16 * u : 0) * K + 8 * g;
    }
    const int row0 = blockIdx.x * (16 * TL) + (lane & 15);
    const int gr0 = wv * ngr / NWV, gr1 = (wv + 1) * ngr / NWV;
    const uint8_t* wr[TL];
#pragma unroll
    for (int t = 0; t < TL; t++) {
        int row = row0 + 16 * t;
        row = row < N ? row : N - 1;
        wr[t] = w + (size_t)row * rb;
    }
    const i4v zi = {0, 0, 0, 0};
    const f4v z4 = {0.0f, 0.0f, 0.0f, 0.0f};
    f4v acc[TL][TT];
#pragma unroll
    for (int t = 0; t < TL; t++)
#pragma unroll
        for (int u = 0; u < TT; u++) acc[t][u] = z4;
    for (int gr = gr0; gr < gr1; gr++) {
        long av[TT][8];
#pragma unroll
        for (int u = 0; u < TT; u++)
#pragma unroll
            for (int b = 0; b < 8; b++)
                av[u][b] = tv[u] ? *reinterpret_cast<const long*>(aq[u] + 32 * (8 * gr + b)) : 0L;
#pragma unroll
        for (int b = 0; b < 8; b++) {
            const int kb = 8 * gr + b;
#pragma unroll
            for (int t = 0; t < TL; t++) {
                const uint8_t* blk = wr[t] + (size_t)kb * BPB;
                const float d = fp16_bits_to_f32(*reinterpret_cast<const uint16_t*>(blk));
                uint2 c;
                if constexpr (T == T_Q8_0) {
                    c = ld8_a2(blk + 2 + 8 * g);
                } else {
                    // elements 8g..8g+7: low nibbles of bytes 8g.. (g < 2), high
                    // nibbles of bytes 8(g - 2).. ; code - 8 per byte (no borrow)
                    const uint2 r = ld8_a2(blk + 2 + 8 * (g & 1));
                    const int sh = g < 2 ? 0 : 4;
                    c.x = ((((r.x >> sh) & 0x0f0f0f0fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
                    c.y = ((((r.y >> sh) & 0x0f0f0f0fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
                }
                const long bw = (long)((unsigned long)c.x | ((unsigned long)c.y << 32));
#pragma unroll
                for (int u = 0; u < TT; u++) {
                    const f4v xd = *reinterpret_cast<const f4v*>(sdx + (size_t)kb * TK + 16 * u + 4 * g);
                    const i4v S = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[u][b], bw, zi, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[t][u][r] = fmaf(d * xd[r], (float)S[r], acc[t][u][r]);
                }
            }
        }
    }
#pragma unroll
    for (int t = 0; t < TL; t++)
#pragma unroll
        for (int u = 0; u < TT; u++) red[wv][t * TT + u][lane] = acc[t][u];
    __syncthreads();
    // wave i sums output tile i (row tile i / TT, token tile i % TT)
    if (wv < TL * TT) {
        const int t = wv / TT, u = wv % TT;
        f4v sum = red[0][wv][lane];
#pragma unroll
        for (int i = 1; i < NWV; i++) sum += red[i][wv][lane];
        const int row = row0 + 16 * t;
        if (row < N) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int tt = 16 * u + 4 * g + r;
                if (tt < M) y[(size_t)tt * N + row] = sum[r];
            }
        }
    }
}

bool i8mf_supported(uint32_t type, int M, int K, int N, const uint8_t* w) {
    // LDS: per block and token the scale (Q4_K also the sum), at most 64 KiB
    if (M > kMfMaxM || K % 256 != 0) return false;
    if (type == T_Q4_K) {
        // M = 3, 4 at long K where the 16-row workgroups apply (measured at
        // 4096 x 14336: M=3 31.1 -> 23.3 us, M=4 36.6 -> 23.8); the GEMV stays
        // faster on wide shapes (14336 x 4096: 17.4 vs 19.8) and at shorter K
        // (4096 x 8192, M=3: 12.2 vs 15.1)
        const int min_m = ((N + 31) / 32 < device_cu_count() && K >= 14336) ? 3 : kMfMinM;
        return M >= min_m && (size_t)(K / 32) * 16 * 8 <= 64 * 1024 && reinterpret_cast<uintptr_t>(w) % 16 == 0;
    }
    if (M < kMfMinM) return false;
    // Q8_0 from 9 rows (measured at 14336 x 4096: M=8 64 us vs 54 on the GEMV,
    // M=16 70 vs 104, M=64 266 vs 392); Q4_0 was no faster than the GEMV
    const bool lds_ok = (size_t)(K / 32) * 16 * 4 <= 64 * 1024 && reinterpret_cast<uintptr_t>(w) % 2 == 0;
    if (type == T_Q6_K) return lds_ok;
    if (type == T_Q8_0) return M >= 9 && lds_ok;
    return false;
}

// Q8_0, Q4_0 and Q6_K prefill rows in chunks of kI8ChunkTt * 16 tokens
// (one weight pass per chunk), 32-row workgroups of 8 waves; Q6_K only where
// those fill 1.5 rounds of CUs: 1 <= M <= 16 * kI8ChunkTt. Measured (us per
// call), Q8_0 against 16-row chunks: 14336x4096 M = 32 / 64 / 256 113 / 223
// / 884 -> 67 / 132 / 522, 4096x4096 M=128 142 -> 134 (16-row workgroups of
// 16 waves there: 151); Q4_0 against 8-row GEMV chunks: 14336x4096 M=64 262
// -> 130, 4096x4096 M=128 193 -> 131, 1024x4096 M=64 72.5 -> 65; Q6_K
// 14336x4096 M=64 156 -> 100, but 4096x4096 M=128 97.5 -> 111 (so not
// there); four token tiles slower everywhere (Q8_0 14336x4096 M=256 948)
bool i8_chunk_supported(uint32_t type, int K, int N, const uint8_t* w) {
    return (type == T_Q8_0 || (type == T_Q6_K && kQ6Chunk) || (type == T_Q4_0 && kQ40Chunk)) && K % 256 == 0 &&
           (size_t)(K / 32) * 16 * kI8ChunkTt * 4 <= 64 * 1024 && reinterpret_cast<uintptr_t>(w) % 2 == 0 &&
           (2 * ((N + 31) / 32) >= 3 * device_cu_count() || type != T_Q6_K);
}
int i8_chunk_rows() { return 16 * kI8ChunkTt; }

hipError_t launch_i8_chunk(uint32_t type, const uint8_t* w, const ActView& A, float* y, int M, int K, int N,
                            hipStream_t st) {
    if (M <= 0 || N <= 0) return hipSuccess;
    if (M > 16 * kI8ChunkTt || !i8_chunk_supported(type, K, N, w)) return hipErrorInvalidValue;
    constexpr int TT = kI8ChunkTt;
    const size_t shm = (size_t)(K / 32) * 16 * TT * 4;
    const long rbq = (long)row_bytes(type, K);
    if (type == T_Q6_K)
        hipLaunchKernelGGL((gemv_q6k_i8mf<2, 8, TT>), dim3((N + 31) / 32), dim3(512), shm, st, w, rbq, A, y, M, K, N);
    else if (type == T_Q4_0)
        hipLaunchKernelGGL((gemv_b32_i8mf<T_Q4_0, 2, 8, TT>), dim3((N + 31) / 32), dim3(512), shm, st, w, rbq, A, y,
                           M, K, N);
    else
        hipLaunchKernelGGL((gemv_b32_i8mf<T_Q8_0, 2, 8, TT>), dim3((N + 31) / 32), dim3(512), shm, st, w, rbq, A, y,
                           M, K, N);
    return hipGetLastError();
}

hipError_t launch_gemv_i8mf(uint32_t type, const uint8_t* w, const ActView& A, float* y, int M, int K, int N,
                            hipStream_t st) {
    if (M <= 0 || N <= 0) return hipSuccess;
    if (!i8mf_supported(type, M, K, N, w)) return hipErrorInvalidValue;
    if (rq_preferred(type, M, K, N, w)) return launch_gemv_rq(w, A, y, M, K, N, st);
    if (q6rq_preferred(type, M, K, N, w)) return launch_gemv_q6rq(w, A, y, M, K, N, st);
    const dim3 grid((N + 16 * kMfTiles - 1) / (16 * kMfTiles));
    if (type == T_Q8_0) {
        const size_t shm = (size_t)(K / 32) * 16 * 4;
        const long rbq = (long)row_bytes(type, K);
        if (2 * ((N + 31) / 32) >= 3 * device_cu_count())
            hipLaunchKernelGGL((gemv_b32_i8mf<T_Q8_0, 2, 8>), grid, dim3(512), shm, st, w, rbq, A, y, M, K, N);
        else
            hipLaunchKernelGGL((gemv_b32_i8mf<T_Q8_0, 1, 16>), dim3((N + 15) / 16), dim3(1024), shm, st, w, rbq, A, y,
                               M, K, N);
        return hipGetLastError();
    }
    if (type == T_Q6_K) {
        // few weight rows (e.g. a down projection, 3584 rows of K 18944): 16-row
        // workgroups of 16 waves, so the K-slices spread over twice the CUs.
        // Switch point measured for Q6_K and Q8_0, M 8..16: 14336 rows (448
        // 32-row workgroups) 10-13 % faster on the 32-row form, 10240 rows
        // (320) 10-13 % faster on the 16-row form.
        const size_t shm = (size_t)(K / 32) * 16 * 4;
        const long rbq = (long)row_bytes(T_Q6_K, K);
        if (2 * ((N + 31) / 32) >= 3 * device_cu_count())
            hipLaunchKernelGGL((gemv_q6k_i8mf<2, 8>), grid, dim3(512), shm, st, w, rbq, A, y, M, K, N);
        else
            hipLaunchKernelGGL((gemv_q6k_i8mf<1, 16>), dim3((N + 15) / 16), dim3(1024), shm, st, w, rbq, A, y, M, K, N);
    } else {
        const size_t shm = (size_t)(K / 32) * 16 * 8;
        const long rbq = (long)row_bytes(T_Q4_K, K);
        // fewer 32-row workgroups than CUs (e.g. a down projection, 4096 rows
        // of K 14336): 16-row workgroups of 16 waves (M=16 42.6 -> 34.1 us
        // there; at 14336 x 4096 the 32-row form is faster, 26.3 vs 36.7)
        if ((N + 31) / 32 < device_cu_count())
            hipLaunchKernelGGL((gemv_q4k_i8mf<false, 1, 16>), dim3((N + 15) / 16), dim3(1024), shm, st, w, rbq, A, y,
                               M, K, N, nullptr, 0, 0, 1, 0L);
        else
            hipLaunchKernelGGL(gemv_q4k_i8mf<false>, grid, dim3(64 * kMfWaves), shm, st, w, rbq, A, y, M, K, N,
                               nullptr, 0, 0, 1, 0L);
    }
    return hipGetLastError();
}

// y = 0 (a kernel, not a memset, so the sequence can be captured in a graph)
__global__ void __launch_bounds__(256) zero_f32_kernel(float* __restrict__ y, size_t n) {
    const size_t i = (size_t)blockIdx.x * 1024 + threadIdx.x;   // y may be only 4-byte aligned
#pragma unroll
    for (int k = 0; k < 4; k++)
        if (i + 256 * k < n) y[i + 256 * k] = 0.0f;
}

size_t gemm_planes_bytes(int M, int K) {
    const size_t up = 256;
    auto r = [&](size_t v) { return (v + up - 1) / up * up; };
    const size_t sp = 2 * r((size_t)M * K * 2) + 2 * r((size_t)M * (K / 32) * 2) + r((size_t)M * 4);
    const size_t fr = gemm_fr_supported(T_Q4_K, M, K) ? gemm_fr_planes_bytes(M, K) : 0;
    const size_t i8 = gemm_i8_supported(T_Q4_K, M, K) ? gemm_i8_planes_bytes(M, K) : 0;
    const size_t a = sp > fr ? sp : fr;
    return a > i8 ? a : i8;
}

// Prefill GEMM kernel family: 0 = by shape, 1 = the split-precision kernel
// on row-major planes (gemm_q4k_sp), 2 = the fragment-order kernel
// (gemm_q4k_fr), 3 = the int8-MFMA kernel (gemm_q4k_i8; measured slower,
// kept for comparison runs), 4 and 5 = the wide-token kernel on
// fragment-order planes (gemm_q4k_wt) with 128 x 256 and 256 x 256 tiles.
static int g_gemm_kernel = 0;
void set_gemm_kernel(int k) { g_gemm_kernel = k; }

bool gemm_i8_preferred(uint32_t type, int M, int K, int N) {
    return g_gemm_kernel == 3 && gemm_i8_supported(type, M, K) && N > 0;
}

// By shape (bench.py --gemm-sweep over N 2048-14336, M 128-2048, K 4096 and
// 14336): the wide-token kernel wherever its workgroups fill the CUs
// (wt_auto_cfg), the split-precision kernel elsewhere (few tiles: its
// 64-token tiles and single planes pass win). The fragment-order kernel
// measured slower than one of the two at every shape of the sweep.
static bool gemm_fr_preferred(int M, int K, int N) {
    if (!gemm_fr_supported(T_Q4_K, M, K) || N < 128) return false;
    if (g_gemm_kernel == 1 || g_gemm_kernel == 3) return false;
    if (g_gemm_kernel == 2 || g_gemm_kernel >= 4) return true;
    return wt_auto_cfg(M, K, N) >= 0;
}

bool gemm_supported(uint32_t type, int M, int K) {
    return type == T_Q4_K && M >= kMfMinM && K % 256 == 0;
}

// Planes for M rows: the fp16 hi/lo pair for the small-M MFMA kernel
// (M <= kMfMaxM), the split-precision pair for the GEMM otherwise.
static bool planes_sp(int M) { return M > kMfMaxM; }

// The split-precision GEMM splits K over two workgroups that add into a
// zeroed y when 64-token tiles leave CUs idle; the planes kernels zero y's
// rows then (one fewer launch).
static bool sp_ksplit(int M, int K, int N) {
    if (M <= kMfMaxM || gemm_fr_preferred(M, K, N)) return false;
    const long cus = device_cu_count();
    const long t128 = (long)((N + 255) / 256) * ((M + 127) / 128);
    const long t64 = (long)((N + 255) / 256) * ((M + 63) / 64);
    return t128 < cus && t64 <= cus && (K >> 8) >= 2;
}

hipError_t launch_planes_from_x(const float* x, void* planes, int M, int K, hipStream_t st, int N, float* y) {
    if (M <= 0) return hipSuccess;
    float* yz = (y && sp_ksplit(M, K, N)) ? y : nullptr;
    if (gemm_fr_preferred(M, K, N)) return launch_fr_planes(x, ActView{}, planes, M, K, st);
    // NF float4 per thread, at most 1024 threads (K <= 32768); 8 | K/4/NF since 32 | K
    const int n4 = K / 4;
    const int nf = n4 <= 1024 ? 1 : n4 <= 2048 ? 2 : n4 <= 4096 ? 4 : 8;
    const int threads = n4 / nf;
    if (threads % 8 != 0) return hipErrorInvalidValue;     // 8-thread groups must not straddle blocks
    const Planes P = carve_planes(planes, M, K);
    const bool sp = planes_sp(M);
#define LP_QP(NF)                                                                                   \
    if (sp) hipLaunchKernelGGL((quant_planes_kernel<NF, true>), dim3(M), dim3(threads), 0, st, x, K, P, yz, N); \
    else hipLaunchKernelGGL((quant_planes_kernel<NF, false>), dim3(M), dim3(threads), 0, st, x, K, P, yz, N);
    switch (nf) {
        case 1: LP_QP(1) break;
        case 2: LP_QP(2) break;
        case 4: LP_QP(4) break;
        default: LP_QP(8) break;
    }
#undef LP_QP
    return hipGetLastError();
}

static hipError_t launch_planes_from_act(const ActView& A, void* planes, int M, int K, hipStream_t st, int N,
                                         float* y) {
    float* yz = (y && sp_ksplit(M, K, N)) ? y : nullptr;
    const Planes P = carve_planes(planes, M, K);
    const dim3 grid((K + kPlaneChunk - 1) / kPlaneChunk, M);
    if (planes_sp(M))
        hipLaunchKernelGGL(gemm_prep_kernel<true>, grid, dim3(kPlaneChunk / 4), 0, st, A, K, P.hi, P.lo, P.shi,
                           P.slo, P.escale, yz, N);
    else
        hipLaunchKernelGGL(gemm_prep_kernel<false>, grid, dim3(kPlaneChunk / 4), 0, st, A, K, P.hi, P.lo, P.shi,
                           P.slo, P.escale, yz, N);
    return hipGetLastError();
}

template <int TT, int NW, int NS>
static hipError_t launch_sp(SpArgs g, hipStream_t st) {
    using C = SpCfg<TT, NW, NS>;
    g.ntn = (g.N + C::BN - 1) / C::BN;
    g.ntiles = g.ntn * ((g.M + C::BM - 1) / C::BM);
    const long nblk = (long)g.ntiles * g.ksplit;
    hipLaunchKernelGGL((gemm_q4k_sp<TT, NW, NS>), dim3((unsigned)nblk), dim3(64 * NW), C::LDS, st, g);
    return hipGetLastError();
}

hipError_t launch_gemm_planes(uint32_t type, const uint8_t* w, void* planes, float* y, int M, int K, int N,
                              hipStream_t st, bool y_zeroed) {
    if (!gemm_supported(type, M, K)) return hipErrorInvalidValue;
    if (M <= 0 || N <= 0) return hipSuccess;
    if (gemm_fr_preferred(M, K, N))
        return g_gemm_kernel == 2 ? launch_fr_gemm(w, planes, y, M, K, N, st)
                                  : launch_wt_gemm(w, planes, y, M, K, N, st,
                                                   g_gemm_kernel >= 4 ? g_gemm_kernel - 4 : wt_auto_cfg(M, K, N));
    const Planes P = carve_planes(planes, M, K);
    if (M <= kMfMaxM) {
        MfArgs a{w, (long)row_bytes(type, K), N, K, M, P, y};
        hipLaunchKernelGGL(gemv_q4k_mf, dim3((N + 16 * kMfTiles - 1) / (16 * kMfTiles)), dim3(64 * kMfWaves),
                           0, st, a);
        return hipGetLastError();
    }
    const long cus = device_cu_count();
    SpArgs g{P.hi, reinterpret_cast<const uint8_t*>(P.lo), P.shi, P.slo, P.escale, w, row_bytes(type, K), y,
             M, N, K, 1, 0, 0};
    // 128-token tiles; 64-token ones when those leave CUs idle, and then K
    // split over two workgroups that add into a zeroed y (two fp32
    // additions onto 0 give the same sum in either order)
    const long t128 = (long)((N + 255) / 256) * ((M + 127) / 128);
    if (t128 >= cus) return launch_sp<4, 4, 2>(g, st);
    const long t64 = (long)((N + 255) / 256) * ((M + 63) / 64);
    g.ksplit = (t64 <= cus && (K >> 8) >= 2) ? 2 : 1;
    if (g.ksplit == 2 && !y_zeroed) {
        const size_t n4 = (size_t)M * N;
        hipLaunchKernelGGL(zero_f32_kernel, dim3((unsigned)((n4 + 1023) / 1024)), dim3(256), 0, st, y, n4);
    }
    return launch_sp<2, 4, 2>(g, st);
}

hipError_t launch_gemm(uint32_t type, const uint8_t* w, const ActView& A, void* planes, float* y,
                       int M, int K, int N, hipStream_t st) {
    if (!gemm_supported(type, M, K)) return hipErrorInvalidValue;
    if (M <= 0 || N <= 0) return hipSuccess;
    if (gemm_i8_preferred(type, M, K, N)) return launch_gemm_i8(w, A, planes, y, M, K, N, st);
    hipError_t e = gemm_fr_preferred(M, K, N) ? launch_fr_planes(nullptr, A, planes, M, K, st)
                                              : launch_planes_from_act(A, planes, M, K, st, N, y);
    if (e != hipSuccess) return e;
    return launch_gemm_planes(type, w, planes, y, M, K, N, st, true);
}

bool moe_mf_supported(uint32_t type, int K) {
    return type == T_Q4_K && K % 256 == 0 && (size_t)(K / 32) * 16 * 8 <= 64 * 1024;
}

hipError_t launch_moe_i8mf(const uint8_t* w, const ActView& A, const void* route, int max_groups, int multi,
                           int topk, float* y, int K, int N, hipStream_t st) {
    if ((size_t)(K / 32) * 16 * 8 > 64 * 1024) return hipErrorInvalidValue;
    const long rb = (long)row_bytes(T_Q4_K, K);
    // two waves (two K-slices) per workgroup, row sets of rw rows, ri of them
    // per workgroup: kMfMoeRows rows, at least two sets. Measured at 128
    // experts, top-8, 160 / 256 / 512 tokens (us per layer): 8 waves with one
    // 32-row set and 8 K-slices for every K - / 358 / 591, 4 sets 313 / 496
    // (256 / 512), with fewer K-slices at short K 291 / 451, two sets at K 768
    // 219 / 281 / 444; 512 rows per workgroup 382 / 455 (too few
    // workgroups); then 4 waves 194-198 / 254-258 / 408-410, 2 waves with 64
    // rows 195-198 / 253 / 394-398 (32 rows: the same; 128: 271-273 at 256
    // tokens), 1 wave 193-197 / 274-277 / 404-407, 16 waves 287 / 472
    constexpr int NWM = kMfMoeWaves;
    const int rw = 16 * kMfTiles * (NWM / mf_kslices(K / 256, NWM));
    const int ri = rw < kMfMoeRows ? kMfMoeRows / rw : 2;
    const int rows = rw * ri;
    hipLaunchKernelGGL((gemv_q4k_i8mf<true, kMfTiles, NWM, true>), dim3((N + rows - 1) / rows, max_groups),
                       dim3(64 * NWM), (size_t)(K / 32) * 16 * 8, st, w, rb, A, y, 0, K, N,
                       static_cast<const uint8_t*>(route), max_groups, multi, topk, rb * N, ri);
    return hipGetLastError();
}

}  // namespace lp
