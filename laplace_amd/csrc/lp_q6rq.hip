// lp_q6rq.hip - Q6_K GEMV for 1..8 activation rows on 4x4 int8 MFMA blocks.
//
// dot_row_q6_k_int (src/matmul_simd.cpp:285-342) for a few activation rows
// at once. Per 16-element block of weight row n and token m the reference
// forms the integer sum sum_k v_nk * q_mk - 32 * sum_k q_mk (v = the 6-bit
// code ql | qh << 4) and adds (d_n * xd_mb) * sc_n * that in fp32. Here the
// two 16-element sums of a 32-element block are combined in int32 with their
// scales, I = sc_0 * S_0 + sc_1 * S_1 (exact), and the block adds
// xd_mb * I in fp32; d_n multiplies once per super-block.
//
// Layout: K in chunks of 16 super-blocks (4096 elements); a wave owns one
// row quad (4 consecutive weight rows). Lane l = 4q + j: weight row j of the
// quad, super-block 16c + q of chunk c.
//   One chunk per workgroup (COAL = false): K <= 4096, or K split over the
//   grid's second dimension with the chunks' partial sums in the caller's
//   workspace scratch, added in chunk order by q6rq_reduce. Each lane loads
//   its super-block (210 bytes, 2-byte aligned) as 52 dwords from the dword
//   at or below its start plus one more dword and the 16-bit d, and
//   funnel-shifts it.
//   Chunk loop (COAL = true, long K without scratch): the wave copies its
//   quad's chunk with coalesced 16-byte loads into its own LDS region and
//   each lane reads its super-block back; the next chunk's copy is requested
//   before this one is computed.

// v_mfma_i32_4x4x4_16b_i8 is 16 independent 4x4x4 products; block q of the
// instruction is lane quad q: A row i = lane 4q+i (token i's four codes),
// B column j = lane 4q+j (row j's four 6-bit codes), D[q][i][j] in lane
// 4q+j element i. Four instructions sum a 16-element block for 4 tokens x
// 4 rows x 16 super-blocks; the accumulator starts at -32 * (the token's
// 16-element code sum), so the chain ends at the reference's integer term.
//
// The workgroup's waves share the tokens' codes of the chunk in LDS,
// together with per block the tokens' xd and the two -32 * code sums (the
// chunk loop double-buffers them: the next chunk's are loaded into
// registers while this one is computed, one barrier per chunk). At the end
// the 16 super-block lanes of each row are added with cross-lane shuffles in
// fixed order, spreading the 4 tokens of a group over the lanes on the way.
//
// LDS (per buffer): tokens' codes, token stride 4416 bytes (16 x 272 rounded
// to 64 mod 256: lanes 4q+i of a 16-lane read phase hit 16 distinct 16-byte
// bank groups), then per super-block SS dwords of [block g][token group t]
// {xd x4, c0 x4, c1 x4}, SS = 96 TG + 4 (distinct bank groups over q).

#include "lp_internal.h"

namespace lp {

typedef int i4v __attribute__((ext_vector_type(4)));
typedef float f4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));

constexpr int kQ6rqWaves = 4;
constexpr int kQ6rqTok = 4416;               // LDS bytes per token per chunk
constexpr int kQ6rqRowStride = 3392;         // LDS bytes per weight row of a wave's chunk copy

struct Q6rqArgs {
    const uint8_t* w;
    long rb;             // bytes per weight row
    ActView A;
    float* y;
    int M, K, N;
    int nchunk;          // chunks of 16 super-blocks
    int buf_bytes;       // LDS bytes per chunk buffer
    float* part;         // K split: per chunk (blockIdx.y) partial sums [nchunk][M][N]; else null
};

struct Q6Tile {
    u32x4 r[13];         // dwords 0..51 from the dword at or below the block start
    uint32_t tail;       // dword 52 (block bytes 206..209) when the block starts at byte 2 of a dword
    uint32_t dh;         // d (fp16 bits)
    uint32_t sh;         // byte offset of the block start in dword 0 (0 or 2)
};

template <int TG, bool COAL>
__global__ void __launch_bounds__(64 * kQ6rqWaves)
gemv_q6k_rq(Q6rqArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr int MP = 4 * TG;
    constexpr int SS = 96 * TG + 4;           // dwords per super-block of block scales
    const int K = a.K, N = a.N, M = a.M;
    const int nsb = K >> 8, nb = K >> 5;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int q = lane >> 2, j = lane & 3;
    const int tga = (M + 3) >> 2;
    // row j of row quad qd (clamped to the last row)
    auto lane_row = [&](long qd) {
        const long r = qd * 4 + j;
        return r < N ? r : (long)N - 1;
    };

    auto load = [&](int c, long qd, Q6Tile& t) {
        int sb = 16 * c + q;
        sb = sb < nsb ? sb : nsb - 1;
        const uint8_t* blk = a.w + lane_row(qd) * a.rb + (long)sb * 210;
        const uintptr_t ab = reinterpret_cast<uintptr_t>(blk);
        const uint8_t* base = reinterpret_cast<const uint8_t*>(ab & ~uintptr_t(3));
#pragma unroll
        for (int i = 0; i < 13; i++) {
            const u32x4a4 v = *reinterpret_cast<const u32x4a4*>(base + 16 * i);
            t.r[i] = u32x4{v.x, v.y, v.z, v.w};
        }
        // dword 52 only when the block starts at byte 2 of a dword; else dword
        // 51 again, so no load passes the block's end
        t.tail = *reinterpret_cast<const uint32_t*>(base + ((ab & 3) ? 208 : 204));
        t.dh = *reinterpret_cast<const uint16_t*>(blk + 208);
        t.sh = (uint32_t)(ab & 3);
    };

    // chunk staging: tokens' codes (16-byte pieces) and per block xd, c0, c1
    constexpr int PPT = MP * 256 / (64 * kQ6rqWaves);      // code pieces per thread
    constexpr int BPT = MP * 128 / (64 * kQ6rqWaves);      // blocks per thread
    u32x4 sp[PPT];
    float sxd[BPT];
    int sc0[BPT], sc1[BPT];
    auto stage_load = [&](int c) {
#pragma unroll
        for (int k = 0; k < PPT; k++) {
            const int i = threadIdx.x + 64 * kQ6rqWaves * k;
            const int m = i >> 8, p = i & 255;
            const int sb = 16 * c + (p >> 4);
            u32x4 v = {0u, 0u, 0u, 0u};
            if (m < M && sb < nsb)
                v = reinterpret_cast<const u32x4*>(a.A.qs + (size_t)m * K + (size_t)sb * 256)[p & 15];
            sp[k] = v;
        }
#pragma unroll
        for (int k = 0; k < BPT; k++) {
            const int i = threadIdx.x + 64 * kQ6rqWaves * k;
            const int m = i >> 7, bl = i & 127;
            const int b = 128 * c + bl;
            float xd = 0.0f;
            int s = 0;
            if (m < M && b < nb) {
                xd = a.A.d[(size_t)m * nb + b];
                s = a.A.s16[(size_t)m * nb + b];
            }
            sxd[k] = xd;
            sc0[k] = -32 * (int)(int16_t)(uint16_t)((uint32_t)s & 0xffffu);
            sc1[k] = -32 * (int)(int16_t)(uint16_t)((uint32_t)s >> 16);
        }
    };
    auto stage_store = [&](int buf) {
        uint8_t* codes = smem + (size_t)buf * a.buf_bytes;
        int* sx = reinterpret_cast<int*>(codes + MP * kQ6rqTok);
#pragma unroll
        for (int k = 0; k < PPT; k++) {
            const int i = threadIdx.x + 64 * kQ6rqWaves * k;
            const int m = i >> 8, p = i & 255;
            *reinterpret_cast<u32x4*>(codes + m * kQ6rqTok + (p >> 4) * 272 + (p & 15) * 16) = sp[k];
        }
#pragma unroll
        for (int k = 0; k < BPT; k++) {
            const int i = threadIdx.x + 64 * kQ6rqWaves * k;
            const int m = i >> 7, bl = i & 127;
            const int o = (bl >> 3) * SS + (bl & 7) * 12 * TG + 12 * (m >> 2) + (m & 3);
            sx[o] = __float_as_int(sxd[k]);
            sx[o + 4] = sc0[k];
            sx[o + 8] = sc1[k];
        }
    };

    f4v tot[TG];
#pragma unroll
    for (int t = 0; t < TG; t++) tot[t] = f4v{0.0f, 0.0f, 0.0f, 0.0f};

    // the lane's super-block as dwords 0..51 (ql, qh, scales) and its d
    auto tile_words = [&](const Q6Tile& T, uint32_t (&wd)[52], uint32_t& dh) {
        uint32_t raw[53];
#pragma unroll
        for (int k = 0; k < 13; k++) {
            raw[4 * k] = T.r[k].x; raw[4 * k + 1] = T.r[k].y; raw[4 * k + 2] = T.r[k].z; raw[4 * k + 3] = T.r[k].w;
        }
        raw[52] = T.tail;
#pragma unroll
        for (int k = 0; k < 52; k++) wd[k] = alignb(raw[k + 1], raw[k], T.sh);
        dh = T.dh;
    };

    auto compute = [&](int c, const uint32_t (&wd)[52], uint32_t dh, int buf) {
        const bool qv = 16 * c + q < nsb;
        const float d = qv ? fp16_bits_to_f32(dh) : 0.0f;
        const uint8_t* codes = smem + (size_t)buf * a.buf_bytes;
        const int* sx = reinterpret_cast<const int*>(codes + MP * kQ6rqTok) + q * SS;
        const uint8_t* aq = codes + j * kQ6rqTok + q * 272;
        f4v acc[TG];
#pragma unroll
        for (int t = 0; t < TG; t++) acc[t] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int n = 0; n < 2; n++) {
#pragma unroll
            for (int gg = 0; gg < 4; gg++) {
                const int g = 4 * n + gg;
                uint32_t v[8];
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const uint32_t ql = wd[16 * n + 8 * (gg & 1) + k];
                    const uint32_t qh = wd[32 + 8 * n + k];
                    v[k] = ((ql >> (4 * (gg >> 1))) & 0x0f0f0f0fu) | (((qh >> (2 * gg)) & 0x03030303u) << 4);
                }
                const int si = 8 * n + 2 * gg;
                const int s0 = (int)(int8_t)((wd[48 + (si >> 2)] >> (8 * (si & 3))) & 0xffu);
                const int s1 = (int)(int8_t)((wd[48 + ((si + 1) >> 2)] >> (8 * ((si + 1) & 3))) & 0xffu);
#pragma unroll
                for (int t = 0; t < TG; t++) {
                    if (t < tga) {
                        const uint8_t* at = aq + (size_t)4 * t * kQ6rqTok + 128 * n + 32 * gg;
                        const u32x4 a0 = *reinterpret_cast<const u32x4*>(at);
                        const u32x4 a1 = *reinterpret_cast<const u32x4*>(at + 16);
                        const int* bs = sx + g * 12 * TG + 12 * t;
                        const f4v xd = *reinterpret_cast<const f4v*>(bs);
                        i4v p0 = *reinterpret_cast<const i4v*>(bs + 4);
                        i4v p1 = *reinterpret_cast<const i4v*>(bs + 8);
                        p0 = __builtin_amdgcn_mfma_i32_4x4x4i8((int)a0.x, (int)v[0], p0, 0, 0, 0);
                        p0 = __builtin_amdgcn_mfma_i32_4x4x4i8((int)a0.y, (int)v[1], p0, 0, 0, 0);
                        p0 = __builtin_amdgcn_mfma_i32_4x4x4i8((int)a0.z, (int)v[2], p0, 0, 0, 0);
                        p0 = __builtin_amdgcn_mfma_i32_4x4x4i8((int)a0.w, (int)v[3], p0, 0, 0, 0);
                        p1 = __builtin_amdgcn_mfma_i32_4x4x4i8((int)a1.x, (int)v[4], p1, 0, 0, 0);
                        p1 = __builtin_amdgcn_mfma_i32_4x4x4i8((int)a1.y, (int)v[5], p1, 0, 0, 0);
                        p1 = __builtin_amdgcn_mfma_i32_4x4x4i8((int)a1.z, (int)v[6], p1, 0, 0, 0);
                        p1 = __builtin_amdgcn_mfma_i32_4x4x4i8((int)a1.w, (int)v[7], p1, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            const int I = __mul24(s0, p0[r]) + __mul24(s1, p1[r]);
                            acc[t][r] = fmaf((float)I, xd[r], acc[t][r]);
                        }
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
#pragma unroll
        for (int t = 0; t < TG; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) tot[t][r] = fmaf(d, acc[t][r], tot[t][r]);
    };

    const int nc = a.nchunk;

    // Sum over the 16 super-block lanes of each row (lane bits 2..5) and
    // store row quad qd's outputs. The exchanges over bits 5 and 4 leave
    // token 2*b5 + b4 of the group in each lane, bits 3 and 2 are plain sums,
    // and the lanes with those clear store.
    auto emit = [&](long qd, float* out) {
        const long row = qd * 4 + j;
#pragma unroll
        for (int t = 0; t < TG; t++) {
            if (t < tga) {
                const f4v v = tot[t];
                const bool bh = (lane >> 5) & 1, bl = (lane >> 4) & 1;
                const float k0 = bh ? v[2] : v[0], k1 = bh ? v[3] : v[1];
                const float s0 = bh ? v[0] : v[2], s1 = bh ? v[1] : v[3];
                const float w0 = k0 + __shfl_xor(s0, 32), w1 = k1 + __shfl_xor(s1, 32);
                float uu = (bl ? w1 : w0) + __shfl_xor(bl ? w0 : w1, 16);
                uu += __shfl_xor(uu, 8);
                uu += __shfl_xor(uu, 4);
                const int m = 4 * t + 2 * bh + bl;
                if ((lane & 12) == 0 && m < M && row < N) out[(size_t)m * N + row] = uu;
            }
        }
    };

    if constexpr (COAL) {
    const long quad = (long)blockIdx.x * kQ6rqWaves + wave;
    // Coalesced weight path: the wave copies its quad's chunk (4 rows x up
    // to 3360 bytes) into its own LDS region, row stride RS, as 16-byte
    // pieces at consecutive 16-byte aligned addresses (piece P = lane + 64 k:
    // row P / 211, piece P % 211 of the aligned window holding the row's
    // chunk), and each lane then reads its super-block back from the offset
    // of the chunk in the window. An aligned 16-byte piece that holds a byte
    // of the matrix lies in that byte's page, so pieces are clamped to the
    // last one holding the matrix's last byte and no load can fault.
    constexpr int RS = kQ6rqRowStride;
    uint8_t* wreg = smem + 2 * (size_t)a.buf_bytes + (size_t)wave * 4 * RS;
    const uintptr_t wend = (reinterpret_cast<uintptr_t>(a.w) + (uintptr_t)N * a.rb - 1) & ~uintptr_t(15);
    auto row_addr = [&](int r) {
        long g = quad * 4 + r;
        g = g < N ? g : (long)N - 1;
        return reinterpret_cast<uintptr_t>(a.w) + (uintptr_t)(g * a.rb);
    };
    u32x4 cp[14];
    auto cload = [&](int c) {
#pragma unroll
        for (int k = 0; k < 14; k++) {
            const int P = lane + 64 * k;
            int r = P / 211;
            const int pc = P - 211 * r;
            r = r < 4 ? r : 3;
            uintptr_t pa = ((row_addr(r) + 3360u * (uintptr_t)c) & ~uintptr_t(15)) + 16u * (uintptr_t)pc;
            pa = pa < wend ? pa : wend;
            cp[k] = *reinterpret_cast<const u32x4*>(pa);
        }
    };
    auto cstore = [&]() {
#pragma unroll
        for (int k = 0; k < 14; k++) {
            const int P = lane + 64 * k;
            const int r = P / 211, pc = P - 211 * (P / 211);
            if (r < 4) *reinterpret_cast<u32x4*>(wreg + r * RS + 16 * pc) = cp[k];
        }
    };
    auto cwords = [&](int c, uint32_t (&wd)[52], uint32_t& dh) {
        int sbl = nsb - 16 * c;
        sbl = sbl < 16 ? sbl : 16;
        const int ql = q < sbl ? q : sbl - 1;
        const uint32_t s0 = (uint32_t)((row_addr(j) + 3360u * (uintptr_t)c) & 15);
        const uint32_t off = (uint32_t)(j * RS) + s0 + (uint32_t)(ql * 210);
        const uint32_t* base = reinterpret_cast<const uint32_t*>(wreg + (off & ~3u));
        const uint32_t sh = off & 3u;
        uint32_t raw[54];
#pragma unroll
        for (int k = 0; k < 54; k++) raw[k] = base[k];
#pragma unroll
        for (int k = 0; k < 52; k++) wd[k] = alignb(raw[k + 1], raw[k], sh);
        dh = alignb(raw[53], raw[52], sh) & 0xffffu;
    };
    cload(0);
    stage_load(0);
    stage_store(0);
    __syncthreads();
    for (int c = 0; c < nc; c++) {
        cstore();
        if (c + 1 < nc) {
            stage_load(c + 1);
            cload(c + 1);
        }
        uint32_t wd[52], dh;
        cwords(c, wd, dh);
        compute(c, wd, dh, c & 1);
        if (c + 1 < nc) {
            stage_store((c + 1) & 1);
            __syncthreads();
        }
    }
    emit(quad, a.y);
    } else {
        // one row quad per wave and one chunk per workgroup (blockIdx.y;
        // K <= 4096, or K split with the chunks' partial sums into a.part):
        // many short-lived workgroups, whose loads and compute overlap
        // across the resident ones (row quads in sequence per wave with the
        // next one's super-blocks requested early measured slower: fewer
        // resident waves at 183 VGPRs)
        const int c = blockIdx.y;
        const long qd = (long)blockIdx.x * kQ6rqWaves + wave;
        Q6Tile t0;
        // the activation rows are requested before the weights (issued after
        // them, they queue behind the weight stream); with one token group
        // the weights only after the staging barrier. us at 3584x18944, M =
        // 4 / 8: weights first 21.7 / 25.5; activations first 21.1 / 23.3;
        // weights after the barrier 19.7 / 24.2 (14336x4096 M = 8: 19.5,
        // 18.3, 17.8)
        if constexpr (TG == 1) {
            stage_load(c);
            stage_store(0);
            __syncthreads();
            load(c, qd, t0);
        } else {
            stage_load(c);
            load(c, qd, t0);
            stage_store(0);
            __syncthreads();
        }
        uint32_t wd[52], dh;
        tile_words(t0, wd, dh);
        compute(c, wd, dh, 0);
        emit(qd, a.part ? a.part + (size_t)c * M * N : a.y);
    }
}

// K split: y = the chunks' partial sums added in chunk order
__global__ void __launch_bounds__(256)
q6rq_reduce(const float* __restrict__ part, int nsplit, long mn, float* __restrict__ y) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= mn) return;
    float s = part[i];
    for (int c = 1; c < nsplit; c++) s += part[(size_t)c * mn + i];
    y[i] = s;
}

static int q6rq_tg(int M) { return M <= 4 ? 1 : 2; }

static size_t q6rq_buf(int TG) { return (size_t)4 * TG * kQ6rqTok + (size_t)16 * (96 * TG + 4) * 4; }

bool q6rq_supported(uint32_t type, int M, int K, int N, const uint8_t* w) {
    // w 4-byte aligned: a block at byte 2 of a dword is read from the dword below it
    return type == T_Q6_K && M >= 1 && M <= 8 && K % 256 == 0 && K > 0 && N > 0 &&
           reinterpret_cast<uintptr_t>(w) % 4 == 0;
}

bool q6rq_preferred(uint32_t type, int M, int K, int N, const uint8_t* w) {
    // M = 1, 2 only in one chunk: the dot4 kernel (gemv_q6k_sbm) is faster
    // at long K there (us, 3584x18944: M=1 18.0 vs 21.1; M=2 21.2 vs 21.6
    // unsplit, 20.3 split; 4096x14336 M=2 16.3 vs 18.2 split), slower in one
    // chunk (4096x4096 M=1 7.9 vs 6.9, M=2 9.5 vs 7.0; 14336x4096 M=1 15.3 vs
    // 14.1, M=2 19.1 vs 14.8)
    return q6rq_supported(type, M, K, N, w) && (M >= 3 || K <= 4096);
}

hipError_t launch_gemv_q6rq(const uint8_t* w, const ActView& A, float* y, int M, int K, int N, hipStream_t st) {
    if (M <= 0 || N <= 0) return hipSuccess;
    if (!q6rq_supported(T_Q6_K, M, K, N, w)) return hipErrorInvalidValue;
    Q6rqArgs a{};
    a.w = w;
    a.rb = (long)row_bytes(T_Q6_K, K);
    a.A = A;
    a.y = y;
    a.M = M;
    a.K = K;
    a.N = N;
    a.nchunk = (K / 256 + 15) / 16;
    const int TG = q6rq_tg(M);
    a.buf_bytes = (int)q6rq_buf(TG);
    const long quads = ((long)N + 3) / 4;
    // K over several chunks: one workgroup per (row-quad group, chunk) when
    // the caller's scratch holds the partial sums (more waves), else the
    // chunk loop with coalesced chunk copies
    const size_t part_need = (size_t)a.nchunk * M * N * sizeof(float);
    const bool split = a.nchunk > 1 && A.part && part_need <= A.part_bytes;
    const bool coal = a.nchunk > 1 && !split;
    a.part = split ? A.part : nullptr;
    const long gx = (quads + kQ6rqWaves - 1) / kQ6rqWaves;
    const dim3 grid((unsigned)gx, split ? (unsigned)a.nchunk : 1u);
    const size_t shm = coal ? 2 * q6rq_buf(TG) + (size_t)kQ6rqWaves * 4 * kQ6rqRowStride : q6rq_buf(TG);
#define LP_Q6RQ_LAUNCH(TGV, CV) hipLaunchKernelGGL((gemv_q6k_rq<TGV, CV>), grid, dim3(64 * kQ6rqWaves), shm, st, a)
    if (TG == 1) {
        if (coal) LP_Q6RQ_LAUNCH(1, true);
        else LP_Q6RQ_LAUNCH(1, false);
    } else {
        if (coal) LP_Q6RQ_LAUNCH(2, true);
        else LP_Q6RQ_LAUNCH(2, false);
    }
#undef LP_Q6RQ_LAUNCH
    if (split) {
        const long mn = (long)M * N;
        hipLaunchKernelGGL(q6rq_reduce, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, st, a.part, a.nchunk, mn, y);
    }
    return hipGetLastError();
}

}  // namespace lp
