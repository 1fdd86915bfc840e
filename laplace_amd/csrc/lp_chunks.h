// lp_chunks.h - per-type decode of one 64-element "chunk" of a weight row
// against the matching 64 quantized activations.
//
// A chunk is the unit one lane owns in the GEMV: 64 consecutive elements of
// K, i.e. 2 activation blocks. For every type the same two steps run:
//   isums()   the exact int32 sub-block dots the reference's NEON kernels
//             form (src/matmul_simd.cpp:143-342): per 32-element block for
//             Q8_0/Q4_0/Q4_K, per 16 elements for Q6_K;
//   partial() the fp32 block-scale epilogue over those integers.
// Weights are read straight from HBM as dwords (nontemporal: each weight
// byte is used once per launch); activations come from registers the lane
// filled once (Act) and reuses for every row it visits.
#pragma once

#include "lp_device.h"

namespace lp {

template <uint32_t T> struct Chunk;

// ---------------------------------------------------------------------------
// Q8_0: chunk c = blocks 2c, 2c+1 = 68 bytes at row + 68c (4-byte aligned
// when the row is). Reference: dot_row_q8_0_int_neon, matmul_simd.cpp:143-160.
template <> struct Chunk<T_Q8_0> {
    static constexpr int NSUB = 2;
    __device__ static int sub_index(int c, int s) { return 2 * c + s; }
    struct Wt { uint32_t w[17]; };
    struct Act { uint32_t q[2][8]; float d[2]; float s[2]; int qsum[4]; };

    __device__ static void load_w(const uint8_t* row, int c, Wt& w) {
        const uint32_t* p = reinterpret_cast<const uint32_t*>(row + 68 * c);
#pragma unroll
        for (int i = 0; i < 17; i++) w.w[i] = __builtin_nontemporal_load(p + i);
    }
    // row: LDS address of the row copy, 4-byte aligned; results valid after wait()
    using Raw = Wt;
    __device__ static void load_w_lds(uint32_t row, int c, Raw& w) { lds_dwords<17>(row + 68 * c, w.w); }
    __device__ static void wait(Raw& r, Wt& w) { lds_wait(r.w); w = r; }
    __device__ static void isums(const Wt& w, const Act& a, int (&is)[NSUB]) {
        int s0 = 0, s1 = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) s0 = dot4(alignb(w.w[i + 1], w.w[i], 2), a.q[0][i], s0);
#pragma unroll
        for (int i = 0; i < 8; i++) s1 = dot4(w.w[9 + i], a.q[1][i], s1);
        is[0] = s0;
        is[1] = s1;
    }
    __device__ static float partial(const Wt& w, const Act& a, const int (&is)[NSUB], int) {
        float d0 = fp16_bits_to_f32(w.w[0]);
        float d1 = fp16_bits_to_f32(w.w[8] >> 16);
        float acc = (d0 * a.d[0]) * (float)is[0];
        return fmaf(d1 * a.d[1], (float)is[1], acc);
    }
};

// ---------------------------------------------------------------------------
// Q4_0: chunk c = blocks 2c, 2c+1 = 36 bytes at row + 36c.
// Reference: dot_row_q4_0_int_neon, matmul_simd.cpp:162-182: the integer is
// sum(nibble * q) with the unsigned nibble; the -8 offset is applied in fp32
// through the activation block sum.
template <> struct Chunk<T_Q4_0> {
    static constexpr int NSUB = 2;
    __device__ static int sub_index(int c, int s) { return 2 * c + s; }
    struct Wt { uint32_t w[9]; };
    struct Act { uint32_t q[2][8]; float d[2]; float s[2]; int qsum[4]; };

    __device__ static void load_w(const uint8_t* row, int c, Wt& w) {
        const uint32_t* p = reinterpret_cast<const uint32_t*>(row + 36 * c);
#pragma unroll
        for (int i = 0; i < 9; i++) w.w[i] = __builtin_nontemporal_load(p + i);
    }
    using Raw = Wt;
    __device__ static void load_w_lds(uint32_t row, int c, Raw& w) { lds_dwords<9>(row + 36 * c, w.w); }
    __device__ static void wait(Raw& r, Wt& w) { lds_wait(r.w); w = r; }
    __device__ static void isums(const Wt& w, const Act& a, int (&is)[NSUB]) {
        int s0 = 0, s1 = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint32_t q = alignb(w.w[i + 1], w.w[i], 2);
            s0 = dot4(q & 0x0f0f0f0fu, a.q[0][i], s0);
            s0 = dot4((q >> 4) & 0x0f0f0f0fu, a.q[0][4 + i], s0);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint32_t q = w.w[5 + i];
            s1 = dot4(q & 0x0f0f0f0fu, a.q[1][i], s1);
            s1 = dot4((q >> 4) & 0x0f0f0f0fu, a.q[1][4 + i], s1);
        }
        is[0] = s0;
        is[1] = s1;
    }
    __device__ static float partial(const Wt& w, const Act& a, const int (&is)[NSUB], int) {
        float d0 = fp16_bits_to_f32(w.w[0]);
        float d1 = fp16_bits_to_f32(w.w[4] >> 16);
        float acc = (d0 * a.d[0]) * (float)is[0];
        acc = fmaf(d1 * a.d[1], (float)is[1], acc);
        // - d * 8 * xa.sum per block
        acc = fmaf(-(d0 * 8.0f), a.s[0], acc);
        return fmaf(-(d1 * 8.0f), a.s[1], acc);
    }
};

// ---------------------------------------------------------------------------
// Q4_K: chunk c = super-block c>>2, quarter jb = c&3: the 32 qs bytes
// 32jb..32jb+31 whose low nibbles are sub-block 2jb and high nibbles
// sub-block 2jb+1. Reference: dot_row_q4_k_int_neon, matmul_simd.cpp:226-283.
// Super-blocks are 144 = 9*16 bytes, so every chunk is 16-byte aligned when
// the tensor base is.
template <> struct Chunk<T_Q4_K> {
    static constexpr int NSUB = 2;
    __device__ static int sub_index(int c, int s) { return 2 * c + s; }
    struct Wt { u32x4 h; u32x4 q0, q1; };
    struct Act { uint32_t q[2][8]; float d[2]; float s[2]; int qsum[4]; };

    __device__ static void load_w(const uint8_t* row, int c, Wt& w) {
        const uint8_t* blk = row + 144 * (c >> 2);
        const int jb = c & 3;
        w.h = ld_nt16(blk);
        w.q0 = ld_nt16(blk + 16 + 32 * jb);
        w.q1 = ld_nt16(blk + 32 + 32 * jb);
    }
    // row: LDS address of the row copy, 16-byte aligned
    using Raw = Wt;
    __device__ static void load_w_lds(uint32_t row, int c, Raw& w) {
        const uint32_t blk = row + 144 * (c >> 2);
        const uint32_t q = blk + 32 * (c & 3);
        lds_b128<0>(w.h, blk);
        lds_b128<16>(w.q0, q);
        lds_b128<32>(w.q1, q);
    }
    __device__ static void wait(Raw& r, Wt& w) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        lds_wait_v(r.h);
        lds_wait_v(r.q0);
        lds_wait_v(r.q1);
        w = r;
    }
    __device__ static void isums(const Wt& w, const Act& a, int (&is)[NSUB]) {
        const uint32_t q[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
        int s0 = 0, s1 = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            s0 = dot4(q[i] & 0x0f0f0f0fu, a.q[0][i], s0);
            s1 = dot4((q[i] >> 4) & 0x0f0f0f0fu, a.q[1][i], s1);
        }
        is[0] = s0;
        is[1] = s1;
    }
    __device__ static float partial(const Wt& w, const Act& a, const int (&is)[NSUB], int c) {
        const float d = fp16_bits_to_f32(w.h.x);
        const float dmin = fp16_bits_to_f32(w.h.x >> 16);
        const int jb = c & 3;
        uint32_t sc1, m1, sc2, m2;
        scale_min_k4(2 * jb, w.h.y, w.h.z, w.h.w, sc1, m1);
        scale_min_k4(2 * jb + 1, w.h.y, w.h.z, w.h.w, sc2, m2);
        float acc = ((d * (float)sc1) * a.d[0]) * (float)is[0];
        acc = fmaf((d * (float)sc2) * a.d[1], (float)is[1], acc);
        acc = fmaf(-(dmin * (float)m1), a.s[0], acc);
        return fmaf(-(dmin * (float)m2), a.s[1], acc);
    }
};

// ---------------------------------------------------------------------------
// Q6_K: chunk c = super-block c>>2, half h = (c>>1)&1, lane-half lr = c&1.
// It covers elements 128h + 32g + 16lr + l (g < 4, l < 16): four 16-element
// groups, each with its own int8 scale sc[8h + 2g + lr]. Reference:
// dot_row_q6_k_int_neon, matmul_simd.cpp:285-342. Super-blocks are 210
// bytes, so chunks are only 2-byte aligned: loads go through load_window.
// The 6-bit code v in [0, 63] is used unsigned and the -32 offset is applied
// exactly as -32 * sum(q) over the same 16 saturated activations.
template <> struct Chunk<T_Q6_K> {
    static constexpr int NSUB = 4;
    // group g of chunk c is 16-element sub-block 16sb + 8h + 2g + lr
    __device__ static int sub_index(int c, int g) {
        return 16 * (c >> 2) + 8 * ((c >> 1) & 1) + 2 * g + (c & 1);
    }
    struct Wt { uint32_t la[4], lb[4], qh[4], sc[2]; uint32_t d; };
    struct Act { uint32_t q[4][4]; float d[4]; float s[2]; int qsum[4]; };

    __device__ static void load_w(const uint8_t* row, int c, Wt& w) {
        const uint8_t* blk = row + 210 * (c >> 2);
        const int h = (c >> 1) & 1, lr = c & 1;
        load_window<4>(blk + 64 * h + 16 * lr, w.la);
        load_window<4>(blk + 64 * h + 32 + 16 * lr, w.lb);
        load_window<4>(blk + 128 + 32 * h + 16 * lr, w.qh);
        load_window<2>(blk + 192 + 8 * h, w.sc);
        w.d = load_u16(blk + 208);
    }
    // row: LDS address of the row copy, 2-byte aligned. Every field of the
    // chunk sits at a multiple of 4 bytes from ql's window start p, so all
    // windows share one byte shift sh = p & 3; the raw dwords are kept in
    // Wt::raw until wait() funnel-shifts them.
    struct Raw { uint32_t la[5], lb[5], qh[5], sc[3], d[1]; uint32_t sh; };
    __device__ static void load_w_lds(uint32_t row, int c, Raw& r) {
        const uint32_t blk = row + 210 * (c >> 2);
        const int h = (c >> 1) & 1, lr = c & 1;
        const uint32_t p = blk + 64 * h + 16 * lr;
        const uint32_t a = p & ~3u;
        r.sh = p & 3u;
        lds_dwords<5>(a, r.la);
        lds_dwords<5, 32>(a, r.lb);
        lds_dwords<5>(a + 128 - 32 * h, r.qh);
        lds_dwords<3>(a + 192 - 56 * h - 16 * lr, r.sc);
        lds_dwords<1>((blk + 208) & ~3u, r.d);   // d: same byte shift (208 = 4 * 52)
    }
    __device__ static void wait(Raw& r, Wt& w) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        lds_wait(r.la);
        lds_wait(r.lb);
        lds_wait(r.qh);
        lds_wait(r.sc);
        lds_wait(r.d);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            w.la[i] = alignb(r.la[i + 1], r.la[i], r.sh);
            w.lb[i] = alignb(r.lb[i + 1], r.lb[i], r.sh);
            w.qh[i] = alignb(r.qh[i + 1], r.qh[i], r.sh);
        }
#pragma unroll
        for (int i = 0; i < 2; i++) w.sc[i] = alignb(r.sc[i + 1], r.sc[i], r.sh);
        w.d = (r.d[0] >> (8 * r.sh)) & 0xffffu;   // sh is 0 or 2: d never straddles a dword
    }
    __device__ static void isums(const Wt& w, const Act& a, int (&is)[NSUB]) {
        int s[4] = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t hb = w.qh[i];
            const uint32_t v0 = (w.la[i] & 0x0f0f0f0fu) | ((hb & 0x03030303u) << 4);
            const uint32_t v1 = (w.lb[i] & 0x0f0f0f0fu) | (((hb >> 2) & 0x03030303u) << 4);
            const uint32_t v2 = ((w.la[i] >> 4) & 0x0f0f0f0fu) | (((hb >> 4) & 0x03030303u) << 4);
            const uint32_t v3 = ((w.lb[i] >> 4) & 0x0f0f0f0fu) | (((hb >> 6) & 0x03030303u) << 4);
            s[0] = dot4(v0, a.q[0][i], s[0]);
            s[1] = dot4(v1, a.q[1][i], s[1]);
            s[2] = dot4(v2, a.q[2][i], s[2]);
            s[3] = dot4(v3, a.q[3][i], s[3]);
        }
#pragma unroll
        for (int g = 0; g < 4; g++) is[g] = s[g] - 32 * a.qsum[g];
    }
    __device__ static float partial(const Wt& w, const Act& a, const int (&is)[NSUB], int c) {
        const float d = fp16_bits_to_f32(w.d);
        const int lr = c & 1;
        float acc = 0.0f;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int bidx = lr + 2 * g;   // byte of the 8 scale bytes of this half
            const int sc = (int)(int8_t)((w.sc[bidx >> 2] >> (8 * (bidx & 3))) & 0xffu);
            acc = fmaf((d * a.d[g]) * (float)sc, (float)is[g], acc);
        }
        return acc;
    }
};

// ---------------------------------------------------------------------------
// Activation registers for chunk c of one row of quantized activations.

__device__ __forceinline__ void load_q16(const int8_t* p, uint32_t (&q)[4]) {
    uint4 v = *reinterpret_cast<const uint4*>(p);
    q[0] = v.x; q[1] = v.y; q[2] = v.z; q[3] = v.w;
}

__device__ __forceinline__ int qsum16(const uint32_t (&q)[4]) {
    int s = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) s = dot4(q[i], 0x01010101u, s);
    return s;
}

template <uint32_t T>
__device__ __forceinline__ void load_act(const ActView& A, int K, int m, int c,
                                         typename Chunk<T>::Act& a) {
    const int nb = K >> 5;
    const int8_t* qrow = A.qs + (size_t)m * K;
    const float* drow = A.d + (size_t)m * nb;
    const float* srow = A.sum + (size_t)m * nb;
    if constexpr (T == T_Q6_K) {
        const int sb = c >> 2, h = (c >> 1) & 1, lr = c & 1;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int blk = 8 * sb + 4 * h + g;
            load_q16(qrow + 32 * blk + 16 * lr, a.q[g]);
            a.d[g] = drow[blk];
            a.qsum[g] = qsum16(a.q[g]);
        }
        a.s[0] = a.s[1] = 0.0f;
    } else {
#pragma unroll
        for (int b = 0; b < 2; b++) {
            const int blk = 2 * c + b;
            uint32_t lo[4], hi[4];
            load_q16(qrow + 32 * blk, lo);
            load_q16(qrow + 32 * blk + 16, hi);
#pragma unroll
            for (int i = 0; i < 4; i++) { a.q[b][i] = lo[i]; a.q[b][4 + i] = hi[i]; }
            a.d[b] = drow[blk];
            a.s[b] = srow[blk];
        }
#pragma unroll
        for (int i = 0; i < 4; i++) a.qsum[i] = 0;
    }
}

// The same activation registers through loads the compiler does not track
// (inline assembly), for kernels that issue direct-to-LDS copies after them:
// a compiler-tracked load would make its first use wait for every later copy
// (vmcnt(0)). Protocol: act_issue(); ...later loads...; an explicit
// s_waitcnt vmcnt(n) that covers these loads; act_finish(), which fences the
// raw registers and only then reads them.
struct ActRaw {
    u32x4 q[4];
    float d[4];
};

__device__ __forceinline__ void gld_b128(u32x4& v, const void* p) {
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(p));
}
__device__ __forceinline__ void gld_b32(float& v, const void* p) {
    asm volatile("global_load_dword %0, %1, off" : "=v"(v) : "v"(p));
}

// q[] holds the codes (Q6_K: four 16-byte halves; others: blocks 2c, 2c+1 as
// 2 x 32 bytes); d[] the block scales (Q6_K) or d0, d1, sum0, sum1.
template <uint32_t T>
__device__ __forceinline__ void act_issue(const ActView& A, int K, int m, int c, ActRaw& r) {
    const int nb = K >> 5;
    const int8_t* qrow = A.qs + (size_t)m * K;
    const float* drow = A.d + (size_t)m * nb;
    const float* srow = A.sum + (size_t)m * nb;
    if constexpr (T == T_Q6_K) {
        const int sb = c >> 2, h = (c >> 1) & 1, lr = c & 1;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int blk = 8 * sb + 4 * h + g;
            gld_b128(r.q[g], qrow + 32 * blk + 16 * lr);
            gld_b32(r.d[g], drow + blk);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) gld_b128(r.q[i], qrow + 64 * c + 16 * i);
        gld_b32(r.d[0], drow + 2 * c);
        gld_b32(r.d[1], drow + 2 * c + 1);
        gld_b32(r.d[2], srow + 2 * c);
        gld_b32(r.d[3], srow + 2 * c + 1);
    }
}

template <uint32_t T>
__device__ __forceinline__ void act_finish(ActRaw& r, typename Chunk<T>::Act& a) {
#pragma unroll
    for (int i = 0; i < 4; i++) asm volatile("" : "+v"(r.q[i]), "+v"(r.d[i]));
    if constexpr (T == T_Q6_K) {
#pragma unroll
        for (int g = 0; g < 4; g++) {
            a.q[g][0] = r.q[g].x; a.q[g][1] = r.q[g].y; a.q[g][2] = r.q[g].z; a.q[g][3] = r.q[g].w;
            a.d[g] = r.d[g];
            a.qsum[g] = qsum16(a.q[g]);
        }
        a.s[0] = a.s[1] = 0.0f;
    } else {
#pragma unroll
        for (int b = 0; b < 2; b++) {
            const u32x4 lo = r.q[2 * b], hi = r.q[2 * b + 1];
            a.q[b][0] = lo.x; a.q[b][1] = lo.y; a.q[b][2] = lo.z; a.q[b][3] = lo.w;
            a.q[b][4] = hi.x; a.q[b][5] = hi.y; a.q[b][6] = hi.z; a.q[b][7] = hi.w;
            a.d[b] = r.d[b];
            a.s[b] = r.d[2 + b];
        }
#pragma unroll
        for (int i = 0; i < 4; i++) a.qsum[i] = 0;
    }
}

// ---------------------------------------------------------------------------
// Quantizer helpers (src/matmul_simd.cpp:348-410).

__device__ __forceinline__ int32_t cvt_rne_sat(float v) {
    // vcvtnq_s32_f32: ties to even, saturating, NaN -> 0.
    const float r = __builtin_rintf(v);
    if (r != r) return 0;
    if (r >= 2147483648.0f) return 2147483647;
    if (r < -2147483648.0f) return (int32_t)0x80000000u;
    return (int32_t)r;
}

__device__ __forceinline__ uint32_t sat8_byte(int32_t q) {
    q = q > 127 ? 127 : (q < -128 ? -128 : q);
    return (uint32_t)(q & 0xff);
}

// One 32-element block quantized by 8 consecutive lanes (one float4 each,
// lane g = elements 4g..4g+3): packed codes of the lane's 4 elements, and
// the block's d, sum and (sum_lo | sum_hi << 16), valid in every lane.
struct Q8Group {
    uint32_t packed;
    float d, sum;
    int32_t s16;
};

// Lane exchanges inside 8-lane groups with DPP moves (no LDS round trip):
// X = 1 and 2 swap neighbours / pairs inside a quad, X = 4 pairs lane i with
// lane 7 - i (row_half_mirror), which for a quad-uniform value is the other
// quad's value, all a reduction over the 8 lanes needs.
template <int X>
__device__ __forceinline__ uint32_t dpp_x8(uint32_t v) {
    constexpr int ctrl = X == 1 ? 0xb1 : X == 2 ? 0x4e : 0x141;
    return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, ctrl, 0xf, 0xf, false);
}
__device__ __forceinline__ float dpp_x8f(float v, int x) {
    const uint32_t b = __float_as_uint(v);
    return __uint_as_float(x == 1 ? dpp_x8<1>(b) : x == 2 ? dpp_x8<2>(b) : dpp_x8<4>(b));
}

// Row exponent of the prefill planes: E with mx = f * 2^E, f in [0.5, 1)
// (0 for a zero, NaN or infinite mx), clamped at -100 so that 2^E and 2^-E
// are both finite normal floats: a row whose largest block scale is
// subnormal (every |x| below ~1.5e-36) then gets t = xd * q * 2^(9 + 100),
// still below 2^16 in magnitude, instead of an overflowing 2^-E.
constexpr int kRowExpMin = -100;
__device__ __forceinline__ int row_exponent(float mx) {
    int e = 0;
    if (mx > 0.0f && mx == mx && mx < 3.0e38f) (void)frexpf(mx, &e);
    return e < kRowExpMin ? kRowExpMin : e;
}

__device__ __forceinline__ Q8Group quant_group8(const float4 v) {
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    uint32_t nan = (v.x != v.x) | (v.y != v.y) | (v.z != v.z) | (v.w != v.w);
    amax = fmaxf(amax, dpp_x8f(amax, 1));
    nan |= dpp_x8<1>(nan);
    amax = fmaxf(amax, dpp_x8f(amax, 2));
    nan |= dpp_x8<2>(nan);
    amax = fmaxf(amax, dpp_x8f(amax, 4));
    nan |= dpp_x8<4>(nan);
    if (nan) amax = __builtin_nanf("");                // FMAX propagates NaN
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    const int32_t q0 = cvt_rne_sat(v.x * id), q1 = cvt_rne_sat(v.y * id);
    const int32_t q2 = cvt_rne_sat(v.z * id), q3 = cvt_rne_sat(v.w * id);
    // int32 sums wrap modulo 2^32 as the NEON lane adds do.
    uint32_t s = (uint32_t)q0 + (uint32_t)q1 + (uint32_t)q2 + (uint32_t)q3;
    s += dpp_x8<1>(s);
    s += dpp_x8<2>(s);                                 // lanes 0-3: elems 0-15, 4-7: 16-31
    const uint32_t s_other = dpp_x8<4>(s);
    const bool first_half = (threadIdx.x & 4) == 0;
    const uint32_t s_lo = first_half ? s : s_other, s_hi = first_half ? s_other : s;
    Q8Group r;
    r.packed = sat8_byte(q0) | (sat8_byte(q1) << 8) | (sat8_byte(q2) << 16) | (sat8_byte(q3) << 24);
    const int16_t lo = (int16_t)(uint16_t)s_lo;
    const int16_t hi = (int16_t)(uint16_t)s_hi;
    r.d = d;
    r.sum = d * (float)((int32_t)lo + (int32_t)hi);
    r.s16 = (int32_t)(((uint32_t)(uint16_t)lo) | ((uint32_t)(uint16_t)hi << 16));
    return r;
}


// gelu_tanh(g) * u (ops::geglu, src/ops.cpp:132-174:
// 0.5 * g * (1 + tanh(c * (g + 0.044715 g^3)))), contraction off.
__device__ __forceinline__ float gelu_tanh_mul(float g, float u) {
#pragma clang fp contract(off)
    const float g3 = (g * g) * g;
    const float cst = 0.7978845608028654f;
    const float gelu = 0.5f * g * (1.0f + tanhf(cst * (g + 0.044715f * g3)));
    return gelu * u;
}

// GeGLU of one gate|up row (gate: K floats, then up: K floats) quantized in
// 32-element blocks exactly as the MoE layer's GeGLU kernel quantizes it,
// written to a GEMV's LDS staging: codes of element e at
// codes[(e / 256) * 272 + e % 256], block b's d at
// dsc[(b / 8) * s1 + (b % 8) * s2] and its scaled sum soff floats after.
// Threads tid, tid + nt, ... (nt a multiple of 64) take one float4 each, 8
// consecutive lanes per block; K % 32 == 0.
__device__ __forceinline__ void stage_geglu_row(const float* __restrict__ gu, int K, uint8_t* codes, float* dsc,
                                                int s1, int s2, int soff, int tid, int nt) {
    for (int i4 = tid; i4 < (K >> 2); i4 += nt) {
        const float4 g = reinterpret_cast<const float4*>(gu)[i4];
        const float4 u = reinterpret_cast<const float4*>(gu + K)[i4];
        const float4 h = make_float4(gelu_tanh_mul(g.x, u.x), gelu_tanh_mul(g.y, u.y), gelu_tanh_mul(g.z, u.z),
                                     gelu_tanh_mul(g.w, u.w));
        const Q8Group q = quant_group8(h);
        const int e = 4 * i4;
        *reinterpret_cast<uint32_t*>(codes + (e >> 8) * 272 + (e & 255)) = q.packed;
        if ((i4 & 7) == 0) {
            const int b = i4 >> 3;
            float* dp = dsc + (b >> 3) * s1 + (b & 7) * s2;
            dp[0] = q.d;
            dp[soff] = q.sum;
        }
    }
}

}  // namespace lp
