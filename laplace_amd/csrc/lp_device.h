// lp_device.h - device-side building blocks shared by the gfx950 kernels:
// GGUF block geometry, fp16 decode, byte-window loads for blocks that are
// only 2-byte aligned, int8 dot helpers and wavefront reductions.
//
// Block layouts are those of the reference's src/kernels.h:21-79 (GGUF):
//   Q4_0  18 B : fp16 d, 16 B nibbles (low nibble = element l, high = l+16)
//   Q8_0  34 B : fp16 d, 32 x int8
//   Q4_K 144 B : fp16 d, fp16 dmin, 12 B packed 6-bit (scale, min) x 8, 128 B nibbles
//   Q6_K 210 B : 128 B ql, 64 B qh, 16 x int8 scales, fp16 d (last)
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lp {

// GGMLType values (reference src/tensor.h:11-34).
enum : uint32_t {
    T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q5_0 = 6, T_Q8_0 = 8,
    T_Q2_K = 10, T_Q3_K = 11, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_BF16 = 30,
};

// Quantized activations in HBM, structure-of-arrays (one ActQ8 of the
// reference, src/matmul_simd.cpp:26-32, is spread over the four arrays):
//   qs   int8 [M, K]            codes, row-major (MFMA/dot friendly)
//   d    f32  [M, K/32]         block scale amax/127
//   sum  f32  [M, K/32]         d * (sum_lo + sum_hi)
//   s16  i32  [M, K/32]         sum_lo | sum_hi << 16 (int16 each)
struct ActView {
    int8_t*  qs;
    float*   d;
    float*   sum;
    int32_t* s16;
    // scratch of the caller's workspace for partial sums of K-split kernels
    // (none when null; kernels then run unsplit)
    float*   part = nullptr;
    size_t   part_bytes = 0;
};

__device__ __forceinline__ float fp16_bits_to_f32(uint32_t h) {
    // v_cvt_f32_f16 is exact for every finite fp16 value, subnormals
    // included (fp16 denormals are not flushed on gfx950).
    _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)(h & 0xffffu));
    return (float)v;
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16-byte nontemporal load (global_load_dwordx4 nt); p must be 16-byte aligned.
__device__ __forceinline__ u32x4 ld_nt16(const void* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// int8x4 . int8x4 + acc (v_dot4_i32_i8).
__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int acc) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, acc, false);
}

// ((hi:lo) >> 8*sh)[31:0]  (v_alignbyte_b32)
__device__ __forceinline__ uint32_t alignb(uint32_t hi, uint32_t lo, uint32_t sh) {
    return __builtin_amdgcn_alignbyte(hi, lo, sh);
}

// NDW dwords of the byte window starting at p, for p only 2-byte aligned.
// Loads NDW aligned dwords, plus one more only when p is not 4-byte aligned
// (so a window ending exactly at an allocation end never reads past it by a
// whole dword), then funnel-shifts them.
template <int NDW>
__device__ __forceinline__ void load_window(const uint8_t* p, uint32_t (&out)[NDW]) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t* base = reinterpret_cast<const uint32_t*>(a & ~uintptr_t(3));
    const uint32_t sh = (uint32_t)(a & 3);
    uint32_t w[NDW + 1];
#pragma unroll
    for (int i = 0; i < NDW; i++) w[i] = __builtin_nontemporal_load(base + i);
    w[NDW] = sh ? __builtin_nontemporal_load(base + NDW) : 0u;
#pragma unroll
    for (int i = 0; i < NDW; i++) out[i] = alignb(w[i + 1], w[i], sh);
}

// Same byte window read from LDS (p 2-byte aligned; NDW + 1 aligned dwords,
// all inside the staged tile).
template <int NDW>
__device__ __forceinline__ void lds_window(const uint8_t* p, uint32_t (&out)[NDW]) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t* base = reinterpret_cast<const uint32_t*>(a & ~uintptr_t(3));
    const uint32_t sh = (uint32_t)(a & 3);
    uint32_t w[NDW + 1];
#pragma unroll
    for (int i = 0; i <= NDW; i++) w[i] = base[i];
#pragma unroll
    for (int i = 0; i < NDW; i++) out[i] = alignb(w[i + 1], w[i], sh);
}

// Sum over groups of `lpr` consecutive lanes (lpr a power of two, 2..64)
// with DPP lane moves; the group's sum lands in its last lane (lpr - 1).
template <int CTRL, int ROWMASK>
__device__ __forceinline__ float dpp_step(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                   0, __builtin_bit_cast(int, v), CTRL, ROWMASK, 0xf, false));
}
__device__ __forceinline__ float group_sum(float v, int lpr) {
    v = dpp_step<0xb1, 0xf>(v);                 // quad_perm [1,0,3,2]
    if (lpr > 2) v = dpp_step<0x4e, 0xf>(v);    // quad_perm [2,3,0,1]
    if (lpr > 4) v = dpp_step<0x114, 0xf>(v);   // row_shr:4
    if (lpr > 8) v = dpp_step<0x118, 0xf>(v);   // row_shr:8
    if (lpr > 16) v = dpp_step<0x142, 0xa>(v);  // row_bcast:15 into rows 1, 3
    if (lpr > 32) v = dpp_step<0x143, 0xc>(v);  // row_bcast:31 into rows 2, 3
    return v;
}

// Two bytes at p (2-byte aligned) as a zero-extended u32.
__device__ __forceinline__ uint32_t load_u16(const uint8_t* p) {
    return *reinterpret_cast<const uint16_t*>(p);
}

// Byte j (0..11) of the K-quant scale array held in three dwords.
__device__ __forceinline__ uint32_t byte_of3(uint32_t s0, uint32_t s1, uint32_t s2, int j) {
    uint32_t w = j < 4 ? s0 : (j < 8 ? s1 : s2);
    return (w >> (8 * (j & 3))) & 0xffu;
}

// get_scale_min_k4 (reference src/kernels.h:82-90) on the 12 scale bytes.
__device__ __forceinline__ void scale_min_k4(int j, uint32_t s0, uint32_t s1, uint32_t s2,
                                             uint32_t& sc, uint32_t& mn) {
    if (j < 4) {
        sc = byte_of3(s0, s1, s2, j) & 63u;
        mn = byte_of3(s0, s1, s2, j + 4) & 63u;
    } else {
        uint32_t hi = byte_of3(s0, s1, s2, j + 4);
        sc = (hi & 0xfu) | ((byte_of3(s0, s1, s2, j - 4) >> 6) << 4);
        mn = (hi >> 4) | ((byte_of3(s0, s1, s2, j) >> 6) << 4);
    }
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// ---------------------------------------------------------------------------
// LDS reads as inline assembly. A compiler-generated ds_read that follows
// direct-to-LDS copies (global_load_lds) makes the compiler wait for every
// copy still in flight (vmcnt(0)), so a stage of a tile could not be read
// while later stages are still arriving. These reads carry no such implicit
// wait: the caller orders them after the copies they need with an explicit
// s_waitcnt vmcnt + s_barrier, and waits for their results with lds_wait().

__device__ __forceinline__ uint32_t lds_addr_of(const void* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}
template <int OFF>
__device__ __forceinline__ void lds_b32(uint32_t& v, uint32_t a) {
    asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(v) : "v"(a), "n"(OFF));
}
template <int OFF>
__device__ __forceinline__ void lds_b128(u32x4& v, uint32_t a) {
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(a), "n"(OFF));
}
template <int N, int BASE = 0, int I = 0>
__device__ __forceinline__ void lds_dwords(uint32_t a, uint32_t (&w)[N]) {
    if constexpr (I < N) {
        lds_b32<BASE + 4 * I>(w[I], a);
        lds_dwords<N, BASE, I + 1>(a, w);
    }
}
// Wait for all of this wave's LDS reads; every register they fill is passed
// so no use is scheduled before the wait.
template <int N>
__device__ __forceinline__ void lds_wait(uint32_t (&w)[N]) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int i = 0; i < N; i++) asm volatile("" : "+v"(w[i]));
}
__device__ __forceinline__ void lds_wait_v(u32x4& v) { asm volatile("" : "+v"(v)); }

// Buffer-resource copies straight into LDS: the per-lane byte offset is fixed
// for the whole tile and a K step only changes the scalar offset, so the copy
// addresses cost no vector instructions. LDS destination: the wave-uniform
// base plus 16 bytes per lane.
typedef __amdgpu_buffer_rsrc_t Rsrc;
__device__ __forceinline__ Rsrc make_rsrc(const void* base, uint32_t bytes) {
    // 0x00020000: the raw-buffer configuration word of the gfx9 family
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ void dma16(Rsrc r, uint32_t voff, uint32_t soff, uint8_t* lds) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}


__device__ __forceinline__ void wait_dma(int outstanding) {
    // gfx9 s_waitcnt: vmcnt[3:0] | expcnt 7 << 4 | lgkmcnt 15 << 8 | vmcnt[5:4] << 14
    switch (outstanding) {
#define LP_W(i) case i: __builtin_amdgcn_s_waitcnt(((i) & 15) | (7 << 4) | (15 << 8) | (((i) >> 4) << 14)); break;
        LP_W(1) LP_W(2) LP_W(3) LP_W(4) LP_W(5) LP_W(6) LP_W(7) LP_W(8) LP_W(9) LP_W(10) LP_W(11) LP_W(12)
        LP_W(13) LP_W(14) LP_W(15) LP_W(16) LP_W(17) LP_W(18) LP_W(19) LP_W(20) LP_W(21) LP_W(22) LP_W(23)
        LP_W(24) LP_W(25) LP_W(26) LP_W(27) LP_W(28) LP_W(29) LP_W(30) LP_W(31) LP_W(32) LP_W(33) LP_W(34)
        LP_W(35) LP_W(36) LP_W(37) LP_W(38) LP_W(39) LP_W(40)
#undef LP_W
        default: __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8)); break;
    }
}

}  // namespace lp
