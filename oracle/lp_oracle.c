/*
 * lp_oracle.c - CPU restatement of Laplace's quantized-matmul arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product). See
 * lp_oracle.h for the contract and the list of parity pins.
 *
 * Build: gcc -O2 -std=c11 -ffp-contract=off -fno-fast-math (oracle/Makefile).
 * -ffp-contract=off keeps every multiply and add separately rounded unless
 * this file calls fmaf() explicitly, so each fused operation below is one
 * the reference's NEON code performs (vfmaq_f32) or, in two marked places,
 * one that Apple clang's default -ffp-contract=on forms from a scalar
 * expression.
 */
#include "lp_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* Type table (src/tensor.h:41-100).                                        */

size_t or_bytes_per_block(int t) {
    switch (t) {
        case OR_F32: return 4;
        case OR_F16: case OR_BF16: return 2;
        case OR_Q4_0: return 18;
        case OR_Q5_0: return 22;
        case OR_Q8_0: return 34;
        case OR_Q2_K: return 84;
        case OR_Q3_K: return 110;
        case OR_Q4_K: return 144;
        case OR_Q5_K: return 176;
        case OR_Q6_K: return 210;
        default: return 0;
    }
}

int or_elements_per_block(int t) {
    switch (t) {
        case OR_F32: case OR_F16: case OR_BF16: return 1;
        case OR_Q4_0: case OR_Q5_0: case OR_Q8_0: return 32;
        case OR_Q2_K: case OR_Q3_K: case OR_Q4_K: case OR_Q5_K: case OR_Q6_K: return 256;
        default: return 0;
    }
}

size_t or_row_bytes(int t, int K) {
    int epb = or_elements_per_block(t);
    if (epb == 0) return 0;
    return (size_t)(K / epb) * or_bytes_per_block(t);
}

/* ------------------------------------------------------------------------ */
/* fp16 / bf16 (src/fp16.h:9-85).                                           */

static float f32_from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t bits_from_f32(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

float or_fp16_to_fp32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) & 1u;
    int32_t  e    = (h >> 10) & 0x1f;
    uint32_t man  = h & 0x3ffu;
    if (e == 0) {
        if (man == 0) return f32_from_bits(sign << 31);
        /* subnormal: value = man * 2^-24, renormalised into an fp32 normal */
        int shift = 0;
        while ((man & 0x400u) == 0) { man <<= 1; shift++; }
        man &= 0x3ffu;
        return f32_from_bits((sign << 31) | ((uint32_t)(113 - shift) << 23) | (man << 13));
    }
    if (e == 31) return f32_from_bits((sign << 31) | (0xffu << 23) | (man << 13));
    return f32_from_bits((sign << 31) | ((uint32_t)(e + 112) << 23) | (man << 13));
}

/* Round-half-up on the dropped mantissa bits (bit 12 decides), which is what
 * src/fp16.h:40-69 does; not IEEE round-to-nearest-even. */
uint16_t or_fp32_to_fp16(float f) {
    uint32_t b = bits_from_f32(f);
    uint32_t sign = (b >> 16) & 0x8000u;
    int32_t  e = (int32_t)((b >> 23) & 0xff) - 127 + 15;
    uint32_t man = b & 0x7fffffu;
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man = (man | 0x800000u) >> (1 - e);
        if (man & 0x1000u) man += 0x2000u;
        return (uint16_t)(sign | (man >> 13));
    }
    if (e == 143) { /* exponent field 0xff: inf or nan */
        return (uint16_t)(sign | 0x7c00u | (man ? (man >> 13) : 0));
    }
    if (e > 30) return (uint16_t)(sign | 0x7c00u);
    if (man & 0x1000u) {
        man += 0x2000u;
        if (man & 0x800000u) {
            man = 0;
            e += 1;
            if (e > 30) return (uint16_t)(sign | 0x7c00u);
        }
    }
    return (uint16_t)(sign | ((uint32_t)e << 10) | (man >> 13));
}

float or_bf16_to_fp32(uint16_t v) { return f32_from_bits((uint32_t)v << 16); }

uint16_t or_fp32_to_bf16(float f) {
    uint32_t b = bits_from_f32(f);
    b += 0x7fffu + ((b >> 16) & 1u);
    return (uint16_t)(b >> 16);
}

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static uint32_t rd32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* src/kernels.h:82-90: 8 (scale, min) pairs of 6 bits packed in 12 bytes. */
void or_get_scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* ------------------------------------------------------------------------ */
/* ActQ8 quantizer (src/matmul_simd.cpp:348-410).                           */

/* vcvtnq_s32_f32: round to nearest, ties to even, saturate, NaN -> 0. */
static int32_t cvtn_s32(float v) {
    if (isnan(v)) return 0;
    if (v >= 2147483648.0f) return INT32_MAX;
    if (v <= -2147483648.0f) return INT32_MIN;
    return (int32_t)nearbyintf(v);   /* default rounding mode: ties to even */
}

/* vmaxq_f32 / vmaxvq_f32 (FMAX): a NaN operand propagates. */
static float fmax_nan(float a, float b) {
    if (isnan(a) || isnan(b)) return NAN;
    return a > b ? a : b;
}

static void quantize_block(const float* xb, float* d_out, float* sum_out,
                           int16_t* lo_out, int16_t* hi_out, int8_t* qs) {
    float amax = 0.0f;
    for (int l = 0; l < 32; l++) amax = fmax_nan(amax, fabsf(xb[l]));
    float d  = amax / 127.0f;
    float id = d > 0.0f ? 1.0f / d : 0.0f;
    int32_t iv[32];
    for (int l = 0; l < 32; l++) iv[l] = cvtn_s32(xb[l] * id);
    /* int32 lane adds wrap modulo 2^32 (vaddq_s32 / vaddvq_s32); addition
     * modulo 2^32 is associative, so the lane order does not matter. */
    uint32_t s_lo = 0, s_hi = 0;
    for (int l = 0; l < 16; l++) s_lo += (uint32_t)iv[l];
    for (int l = 16; l < 32; l++) s_hi += (uint32_t)iv[l];
    int16_t lo = (int16_t)(uint16_t)s_lo;   /* static_cast<int16_t>: truncation */
    int16_t hi = (int16_t)(uint16_t)s_hi;
    *lo_out = lo;
    *hi_out = hi;
    *d_out = d;
    *sum_out = d * (float)((int32_t)lo + (int32_t)hi);
    /* vqmovn_s32 then vqmovn_s16: saturate to int16, then to int8. */
    for (int l = 0; l < 32; l++) {
        int32_t v = iv[l];
        if (v > 127) v = 127;
        if (v < -128) v = -128;
        qs[l] = (int8_t)v;
    }
}

void or_quantize_act(const float* x, int M, int K, float* d, float* sum,
                     int16_t* sum_lo, int16_t* sum_hi, int8_t* qs) {
    const int nb = K / 32;
    for (int m = 0; m < M; m++) {
        for (int b = 0; b < nb; b++) {
            size_t i = (size_t)m * nb + b;
            quantize_block(x + (size_t)m * K + 32 * b, d + i, sum + i, sum_lo + i, sum_hi + i,
                           qs + (size_t)m * K + 32 * b);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Weight decoders to signed/unsigned integer codes, one element at a time. */
/* Element e (0..epb-1) of a block maps to the code the NEON kernel pairs    */
/* with activation element e of the same block.                              */

/* Q4_0: low nibbles are elements 0..15, high nibbles 16..31 (:162-182). */
static int code_q4_0(const uint8_t* blk, int e) {
    const uint8_t* qs = blk + 2;
    return e < 16 ? (qs[e] & 0xF) : (qs[e - 16] >> 4);
}

/* Q5_0: nibble | bit e of qh << 4, minus 16 (:184-224). */
static int code_q5_0(const uint8_t* blk, int e) {
    uint32_t qh = rd32(blk + 2);
    const uint8_t* qs = blk + 6;
    int nib = e < 16 ? (qs[e] & 0xF) : (qs[e - 16] >> 4);
    return (nib | (int)(((qh >> e) & 1u) << 4)) - 16;
}

/* Q4_K: chunk jb = e/64 reads qs[32jb..32jb+31]; its low nibbles are
 * elements 64jb..64jb+31 (sub-block 2jb), high nibbles the next 32
 * (sub-block 2jb+1) (:242-280). Returns the unsigned nibble. */
static int code_q4_k(const uint8_t* blk, int e) {
    const uint8_t* qs = blk + 16;
    int jb = e / 64, r = e % 64;
    return r < 32 ? (qs[32 * jb + r] & 0xF) : (qs[32 * jb + r - 32] >> 4);
}

/* Q6_K: half h = e/128, g = (e%128)/32, l = e%32. Low 4 bits from
 * ql[64h + l + 32*(g&1)] (low nibble for g<2, high nibble for g>=2), high
 * 2 bits from (qh[32h + l] >> 2g) & 3, minus 32 (:300-323). */
static int code_q6_k(const uint8_t* blk, int e) {
    const uint8_t* ql = blk;
    const uint8_t* qh = blk + 128;
    int h = e / 128, g = (e % 128) / 32, l = e % 32;
    uint8_t qlb = ql[64 * h + l + ((g & 1) ? 32 : 0)];
    int lo = (g >= 2) ? (qlb >> 4) : (qlb & 0xF);
    int hi = (qh[32 * h + l] >> (2 * g)) & 3;
    return (lo | (hi << 4)) - 32;
}

static int code_q8_0(const uint8_t* blk, int e) { return (int8_t)blk[2 + e]; }

int or_n_subsums(int type, int K) {
    switch (type) {
        case OR_Q8_0: case OR_Q4_0: case OR_Q5_0: case OR_Q4_K: return K / 32;
        case OR_Q6_K: return (K / 256) * 16;
        default: return -1;
    }
}

static int (*code_fn(int type))(const uint8_t*, int) {
    switch (type) {
        case OR_Q8_0: return code_q8_0;
        case OR_Q4_0: return code_q4_0;
        case OR_Q5_0: return code_q5_0;
        case OR_Q4_K: return code_q4_k;
        case OR_Q6_K: return code_q6_k;
        default: return NULL;
    }
}

int or_block_sums_row(int type, const uint8_t* wrow, const int8_t* qs, int K, int32_t* out) {
    int (*code)(const uint8_t*, int) = code_fn(type);
    if (!code) return -1;
    const int epb = or_elements_per_block(type);
    const size_t bpb = or_bytes_per_block(type);
    const int sub = (type == OR_Q6_K) ? 16 : 32;
    const int nblk = K / epb;
    int idx = 0;
    for (int b = 0; b < nblk; b++) {
        const uint8_t* blk = wrow + (size_t)b * bpb;
        for (int s = 0; s < epb / sub; s++) {
            int32_t acc = 0;
            for (int l = 0; l < sub; l++) {
                int e = s * sub + l;
                acc += code(blk, e) * (int32_t)qs[b * epb + e];
            }
            out[idx++] = acc;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Int8 dots with the NEON lane structure.                                  */
/* dot16 lane i (i < 4) sums the products of elements 4i..4i+3 of a         */
/* 16-element group (vdotq_s32 / vusdotq_s32).                              */

static void dot16(int (*code)(const uint8_t*, int), const uint8_t* blk, int e0,
                  const int8_t* q, int32_t lane[4]) {
    for (int i = 0; i < 4; i++) {
        int32_t s = 0;
        for (int j = 0; j < 4; j++) s += code(blk, e0 + 4 * i + j) * (int32_t)q[4 * i + j];
        lane[i] = s;
    }
}

/* acc = vfmaq_f32(acc, vdupq_n_f32(scale), vcvtq_f32_s32(p)) */
static void fma4(float acc[4], float scale, const int32_t p[4]) {
    for (int i = 0; i < 4; i++) acc[i] = fmaf(scale, (float)p[i], acc[i]);
}

/* vaddvq_f32: pairwise (a0 + a1) + (a2 + a3). */
static float hsum4(const float a[4]) { return (a[0] + a[1]) + (a[2] + a[3]); }

static float hsum4x2(const float a[4], const float b[4]) {
    float t[4];
    for (int i = 0; i < 4; i++) t[i] = a[i] + b[i];
    return hsum4(t);
}

/* src/matmul_simd.cpp:143-160 */
static float dot_int_q8_0(const uint8_t* w, const float* xd, const int8_t* q, int K) {
    float acc0[4] = {0}, acc1[4] = {0};
    int32_t p0[4], p1[4];
    for (int b = 0; b < K / 32; b++) {
        const uint8_t* blk = w + (size_t)b * 34;
        dot16(code_q8_0, blk, 0, q + 32 * b, p0);
        dot16(code_q8_0, blk, 16, q + 32 * b + 16, p1);
        float scale = or_fp16_to_fp32(rd16(blk)) * xd[b];
        fma4(acc0, scale, p0);
        fma4(acc1, scale, p1);
    }
    return hsum4x2(acc0, acc1);
}

/* src/matmul_simd.cpp:162-182 */
static float dot_int_q4_0(const uint8_t* w, const float* xd, const float* xs,
                          const int8_t* q, int K) {
    float acc[4] = {0};
    float acc_offset = 0.0f;
    int32_t p0[4], p1[4];
    for (int b = 0; b < K / 32; b++) {
        const uint8_t* blk = w + (size_t)b * 18;
        dot16(code_q4_0, blk, 0, q + 32 * b, p0);
        dot16(code_q4_0, blk, 16, q + 32 * b + 16, p1);
        float dw = or_fp16_to_fp32(rd16(blk));
        float scale = dw * xd[b];
        fma4(acc, scale, p0);
        fma4(acc, scale, p1);
        /* `acc_offset += d * 8.0f * xa.sum`: clang -ffp-contract=on fuses the
         * outer multiply-add into one fma (assumed, not observable here). */
        acc_offset = fmaf(dw * 8.0f, xs[b], acc_offset);
    }
    return hsum4(acc) - acc_offset;
}

/* src/matmul_simd.cpp:184-224 */
static float dot_int_q5_0(const uint8_t* w, const float* xd, const int8_t* q, int K) {
    float acc[4] = {0};
    int32_t p0[4], p1[4];
    for (int b = 0; b < K / 32; b++) {
        const uint8_t* blk = w + (size_t)b * 22;
        dot16(code_q5_0, blk, 0, q + 32 * b, p0);
        dot16(code_q5_0, blk, 16, q + 32 * b + 16, p1);
        float scale = or_fp16_to_fp32(rd16(blk)) * xd[b];
        fma4(acc, scale, p0);
        fma4(acc, scale, p1);
    }
    return hsum4(acc);
}

/* src/matmul_simd.cpp:226-283 */
static float dot_int_q4_k(const uint8_t* w, const float* xd, const float* xs,
                          const int8_t* q, int K) {
    float acc0[4] = {0}, acc1[4] = {0};
    float acc_min = 0.0f;
    int32_t p10[4], p11[4], p20[4], p21[4];
    for (int b = 0; b < K / 256; b++) {
        const uint8_t* blk = w + (size_t)b * 144;
        float d = or_fp16_to_fp32(rd16(blk));
        float dmin = or_fp16_to_fp32(rd16(blk + 2));
        const uint8_t* scales = blk + 4;
        for (int jb = 0; jb < 4; jb++) {
            uint8_t sc, m;
            or_get_scale_min_k4(2 * jb, scales, &sc, &m);
            float d1 = d * (float)sc, m1 = dmin * (float)m;
            or_get_scale_min_k4(2 * jb + 1, scales, &sc, &m);
            float d2 = d * (float)sc, m2 = dmin * (float)m;
            int a1 = b * 8 + 2 * jb, a2 = a1 + 1;
            dot16(code_q4_k, blk, 64 * jb, q + 32 * a1, p10);
            dot16(code_q4_k, blk, 64 * jb + 16, q + 32 * a1 + 16, p11);
            dot16(code_q4_k, blk, 64 * jb + 32, q + 32 * a2, p20);
            dot16(code_q4_k, blk, 64 * jb + 48, q + 32 * a2 + 16, p21);
            float scale1 = d1 * xd[a1];
            float scale2 = d2 * xd[a2];
            fma4(acc0, scale1, p10);
            fma4(acc1, scale1, p11);
            fma4(acc0, scale2, p20);
            fma4(acc1, scale2, p21);
            /* `acc_min += m1 * a1.sum + m2 * a2.sum`: with clang's
             * -ffp-contract=on the inner sum becomes fma(m1, s1, m2*s2)
             * (assumed, not observable here). */
            acc_min = acc_min + fmaf(m1, xs[a1], m2 * xs[a2]);
        }
    }
    return hsum4x2(acc0, acc1) - acc_min;
}

/* src/matmul_simd.cpp:285-342 */
static float dot_int_q6_k(const uint8_t* w, const float* xd, const int8_t* q, int K) {
    float acc0[4] = {0}, acc1[4] = {0};
    int32_t p0[4], p1[4];
    for (int b = 0; b < K / 256; b++) {
        const uint8_t* blk = w + (size_t)b * 210;
        float d = or_fp16_to_fp32(rd16(blk + 208));
        const int8_t* sc = (const int8_t*)(blk + 192);
        for (int h = 0; h < 2; h++) {
            for (int g = 0; g < 4; g++) {
                int a = b * 8 + h * 4 + g;
                int e0 = 128 * h + 32 * g;
                dot16(code_q6_k, blk, e0, q + 32 * a, p0);
                dot16(code_q6_k, blk, e0 + 16, q + 32 * a + 16, p1);
                float s0 = d * xd[a] * (float)sc[8 * h + 2 * g];
                float s1 = d * xd[a] * (float)sc[8 * h + 2 * g + 1];
                fma4(acc0, s0, p0);
                fma4(acc1, s1, p1);
            }
        }
    }
    return hsum4x2(acc0, acc1);
}

float or_dot_int_row(int type, const uint8_t* wrow, const float* d, const float* sum,
                     const int8_t* qs, int K) {
    switch (type) {
        case OR_Q8_0: return dot_int_q8_0(wrow, d, qs, K);
        case OR_Q4_0: return dot_int_q4_0(wrow, d, sum, qs, K);
        case OR_Q5_0: return dot_int_q5_0(wrow, d, qs, K);
        case OR_Q4_K: return dot_int_q4_k(wrow, d, sum, qs, K);
        case OR_Q6_K: return dot_int_q6_k(wrow, d, qs, K);
        default: return NAN;
    }
}

/* ------------------------------------------------------------------------ */
/* ThreadPool::parallel_for partitioning (src/threadpool.h:229-258, 310-320): */
/* chunk = ceil(n / active); thread t runs [t*chunk, min(n, (t+1)*chunk)).    */

typedef void (*body_fn)(void* ctx, int i);
typedef struct { body_fn fn; void* ctx; int n, active, tid; } pf_task;

static void* pf_run(void* arg) {
    pf_task* t = (pf_task*)arg;
    int chunk = (t->n + t->active - 1) / t->active;
    int start = t->tid * chunk;
    int end = start + chunk;
    if (end > t->n) end = t->n;
    for (int i = start; i < end; i++) t->fn(t->ctx, i);
    return NULL;
}

static void parallel_for(int n, int active, body_fn fn, void* ctx) {
    if (n <= 0) return;
    if (active <= 1) {
        for (int i = 0; i < n; i++) fn(ctx, i);
        return;
    }
    pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)active);
    pf_task* tasks = (pf_task*)malloc(sizeof(pf_task) * (size_t)active);
    for (int t = 0; t < active; t++) {
        tasks[t] = (pf_task){fn, ctx, n, active, t};
        if (t > 0) pthread_create(&th[t], NULL, pf_run, &tasks[t]);
    }
    pf_run(&tasks[0]);   /* the calling thread is tid 0, as in the reference */
    for (int t = 1; t < active; t++) pthread_join(th[t], NULL);
    free(th);
    free(tasks);
}

/* ------------------------------------------------------------------------ */
/* gemm_int (src/matmul_simd.cpp:432-455): N_DST = 2 columns per task.      */

typedef struct {
    int type, M, K, N;
    const uint8_t* w;
    size_t rb;
    const float* d; const float* sum; const int8_t* qs;
    float* y;
} gemm_int_ctx;

static void gemm_int_body(void* p, int task) {
    gemm_int_ctx* c = (gemm_int_ctx*)p;
    const int nb = c->K / 32;
    int j0 = task * 2, j1 = j0 + 2 < c->N ? j0 + 2 : c->N;
    for (int j = j0; j < j1; j++) {
        const uint8_t* row = c->w + (size_t)j * c->rb;
        for (int m = 0; m < c->M; m++) {
            c->y[(size_t)m * c->N + j] = or_dot_int_row(
                c->type, row, c->d + (size_t)m * nb, c->sum + (size_t)m * nb,
                c->qs + (size_t)m * c->K, c->K);
        }
    }
}

typedef struct { float* d; float* sum; int16_t* lo; int16_t* hi; int8_t* qs; } act_buf;

static int act_alloc(act_buf* a, int M, int K) {
    size_t nbk = (size_t)M * (K / 32);
    a->d = (float*)malloc(sizeof(float) * (nbk ? nbk : 1));
    a->sum = (float*)malloc(sizeof(float) * (nbk ? nbk : 1));
    a->lo = (int16_t*)malloc(sizeof(int16_t) * (nbk ? nbk : 1));
    a->hi = (int16_t*)malloc(sizeof(int16_t) * (nbk ? nbk : 1));
    a->qs = (int8_t*)malloc((size_t)M * K + 1);
    return (a->d && a->sum && a->lo && a->hi && a->qs) ? 0 : -1;
}

static void act_free(act_buf* a) { free(a->d); free(a->sum); free(a->lo); free(a->hi); free(a->qs); }

int or_gemm_int(int type, const float* x, const uint8_t* w, float* y,
                int M, int K, int N, int nthreads) {
    if (!code_fn(type)) return -1;
    act_buf a;
    if (act_alloc(&a, M, K)) { act_free(&a); return -1; }
    or_quantize_act(x, M, K, a.d, a.sum, a.lo, a.hi, a.qs);
    gemm_int_ctx c = {type, M, K, N, w, or_row_bytes(type, K), a.d, a.sum, a.qs, y};
    int ntask = (N + 1) / 2;
    int active = (M > 1 || N >= 128) ? nthreads : 1;
    parallel_for(ntask, active, gemm_int_body, &c);
    act_free(&a);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* moe_gemv_int / moe_gemv_multi_int (src/matmul_simd.cpp:506-544).         */

typedef struct {
    int type, K, N, multi;
    const uint8_t* w; size_t rb, per_expert;
    const int* idx;
    const float* d; const float* sum; const int8_t* qs;
    float* y;
} moe_ctx;

static void moe_body(void* p, int i) {
    moe_ctx* c = (moe_ctx*)p;
    int k = i / c->N, j = i % c->N;
    const int nb = c->K / 32;
    size_t a = c->multi ? (size_t)k : 0;
    const uint8_t* row = c->w + (size_t)c->idx[k] * c->per_expert + (size_t)j * c->rb;
    c->y[(size_t)k * c->N + j] = or_dot_int_row(c->type, row, c->d + a * nb, c->sum + a * nb,
                                                c->qs + a * c->K, c->K);
}

int or_moe_gemv_int(int type, const float* x, const uint8_t* w, const int* expert_idx,
                    int n_experts, float* y, int K, int N, int multi, int nthreads) {
    if (!code_fn(type)) return -1;
    int rows = multi ? n_experts : 1;
    act_buf a;
    if (act_alloc(&a, rows, K)) { act_free(&a); return -1; }
    or_quantize_act(x, rows, K, a.d, a.sum, a.lo, a.hi, a.qs);
    size_t rb = or_row_bytes(type, K);
    moe_ctx c = {type, K, N, multi, w, rb, rb * (size_t)N, expert_idx, a.d, a.sum, a.qs, y};
    parallel_for(n_experts * N, nthreads, moe_body, &c);
    act_free(&a);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Scalar fp32 dots (src/matmul.cpp:63-314), sequential accumulation.       */

static float sdot_f32(const float* x, const uint8_t* row, int K) {
    float acc = 0.0f;
    for (int k = 0; k < K; k++) { float w; memcpy(&w, row + 4 * (size_t)k, 4); acc += x[k] * w; }
    return acc;
}

static float sdot_f16(const float* x, const uint8_t* row, int K) {
    float acc = 0.0f;
    for (int k = 0; k < K; k++) acc += x[k] * or_fp16_to_fp32(rd16(row + 2 * (size_t)k));
    return acc;
}

static float sdot_bf16(const float* x, const uint8_t* row, int K) {
    float acc = 0.0f;
    for (int k = 0; k < K; k++) acc += x[k] * or_bf16_to_fp32(rd16(row + 2 * (size_t)k));
    return acc;
}

static float sdot_q4_0(const float* x, const uint8_t* row, int K) {   /* :84-100 */
    float acc = 0.0f;
    for (int b = 0; b < K / 32; b++) {
        const uint8_t* blk = row + (size_t)b * 18;
        const float* xb = x + 32 * b;
        float d = or_fp16_to_fp32(rd16(blk));
        float sum = 0.0f;
        for (int l = 0; l < 16; l++) {
            sum += xb[l] * (float)((blk[2 + l] & 0xF) - 8);
            sum += xb[l + 16] * (float)((blk[2 + l] >> 4) - 8);
        }
        acc += d * sum;
    }
    return acc;
}

static float sdot_q5_0(const float* x, const uint8_t* row, int K) {   /* :102-121 */
    float acc = 0.0f;
    for (int b = 0; b < K / 32; b++) {
        const uint8_t* blk = row + (size_t)b * 22;
        const float* xb = x + 32 * b;
        float d = or_fp16_to_fp32(rd16(blk));
        uint32_t qh = rd32(blk + 2);
        float sum = 0.0f;
        for (int l = 0; l < 16; l++) {
            int lo0 = (blk[6 + l] & 0xF) | (int)(((qh >> l) & 1u) << 4);
            int lo1 = (blk[6 + l] >> 4) | (int)(((qh >> (l + 16)) & 1u) << 4);
            sum += xb[l] * (float)(lo0 - 16);
            sum += xb[l + 16] * (float)(lo1 - 16);
        }
        acc += d * sum;
    }
    return acc;
}

static float sdot_q8_0(const float* x, const uint8_t* row, int K) {   /* :123-135 */
    float acc = 0.0f;
    for (int b = 0; b < K / 32; b++) {
        const uint8_t* blk = row + (size_t)b * 34;
        const float* xb = x + 32 * b;
        float sum = 0.0f;
        for (int l = 0; l < 32; l++) sum += xb[l] * (float)(int8_t)blk[2 + l];
        acc += or_fp16_to_fp32(rd16(blk)) * sum;
    }
    return acc;
}

static float sdot_q4_k(const float* x, const uint8_t* row, int K) {   /* :137-167 */
    float acc = 0.0f;
    for (int b = 0; b < K / 256; b++) {
        const uint8_t* blk = row + (size_t)b * 144;
        const float* xb = x + 256 * b;
        float d = or_fp16_to_fp32(rd16(blk));
        float dmin = or_fp16_to_fp32(rd16(blk + 2));
        const uint8_t* q = blk + 16;
        for (int jb = 0, is = 0; jb < 256; jb += 64, is += 2, q += 32) {
            uint8_t sc, m;
            or_get_scale_min_k4(is, blk + 4, &sc, &m);
            float d1 = d * sc, m1 = dmin * m;
            or_get_scale_min_k4(is + 1, blk + 4, &sc, &m);
            float d2 = d * sc, m2 = dmin * m;
            float s1 = 0.0f, s2 = 0.0f, x1 = 0.0f, x2 = 0.0f;
            for (int l = 0; l < 32; l++) {
                s1 += xb[jb + l] * (float)(q[l] & 0xF);
                x1 += xb[jb + l];
                s2 += xb[jb + 32 + l] * (float)(q[l] >> 4);
                x2 += xb[jb + 32 + l];
            }
            acc += d1 * s1 - m1 * x1 + d2 * s2 - m2 * x2;
        }
    }
    return acc;
}

static float sdot_q6_k(const float* x, const uint8_t* row, int K) {   /* :169-198 */
    float acc = 0.0f;
    for (int b = 0; b < K / 256; b++) {
        const uint8_t* blk = row + (size_t)b * 210;
        float d = or_fp16_to_fp32(rd16(blk + 208));
        const uint8_t* ql = blk;
        const uint8_t* qh = blk + 128;
        const int8_t* sc = (const int8_t*)(blk + 192);
        const float* xb = x + 256 * b;
        for (int n_off = 0; n_off < 256; n_off += 128, ql += 64, qh += 32, sc += 8) {
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                int q1 = (int)((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                acc += xb[n_off + l] * (d * sc[is + 0] * q1);
                acc += xb[n_off + l + 32] * (d * sc[is + 2] * q2);
                acc += xb[n_off + l + 64] * (d * sc[is + 4] * q3);
                acc += xb[n_off + l + 96] * (d * sc[is + 6] * q4);
            }
        }
    }
    return acc;
}

static float sdot_q2_k(const float* x, const uint8_t* row, int K) {   /* :200-234 */
    float acc = 0.0f;
    for (int b = 0; b < K / 256; b++) {
        const uint8_t* blk = row + (size_t)b * 84;
        const float* xq = x + 256 * b;
        float d = or_fp16_to_fp32(rd16(blk + 80));
        float dmin = or_fp16_to_fp32(rd16(blk + 82));
        const uint8_t* q = blk + 16;
        const uint8_t* sc = blk;
        int is = 0;
        float isum = 0.0f, summs = 0.0f;
        for (int k = 0; k < 2; k++, q += 32) {
            for (int j = 0, shift = 0; j < 4; j++, shift += 2) {
                float s = (float)(sc[is] & 0xF), m = (float)(sc[is] >> 4);
                float suml = 0.0f, xsum = 0.0f;
                for (int l = 0; l < 16; l++) { suml += xq[l] * (float)((q[l] >> shift) & 3); xsum += xq[l]; }
                isum += s * suml; summs += m * xsum;
                xq += 16; is++;
                s = (float)(sc[is] & 0xF); m = (float)(sc[is] >> 4);
                suml = 0.0f; xsum = 0.0f;
                for (int l = 16; l < 32; l++) { suml += xq[l - 16] * (float)((q[l] >> shift) & 3); xsum += xq[l - 16]; }
                isum += s * suml; summs += m * xsum;
                xq += 16; is++;
            }
        }
        acc += d * isum - dmin * summs;
    }
    return acc;
}

/* Q3_K 6-bit scale unpack of src/matmul.cpp:246-253 (also :626-633). */
static void q3k_scales(const uint8_t* s12, uint8_t out[16]) {
    const uint32_t kmask1 = 0x03030303u, kmask2 = 0x0f0f0f0fu;
    uint32_t aux[4];
    aux[0] = rd32(s12); aux[1] = rd32(s12 + 4); aux[2] = rd32(s12 + 8);
    uint32_t tmp = aux[2];
    aux[2] = ((aux[0] >> 4) & kmask2) | (((tmp >> 4) & kmask1) << 4);
    aux[3] = ((aux[1] >> 4) & kmask2) | (((tmp >> 6) & kmask1) << 4);
    aux[0] = (aux[0] & kmask2) | (((tmp >> 0) & kmask1) << 4);
    aux[1] = (aux[1] & kmask2) | (((tmp >> 2) & kmask1) << 4);
    for (int i = 0; i < 4; i++)
        for (int j = 0; j < 4; j++) out[4 * i + j] = (uint8_t)(aux[i] >> (8 * j));
}

static float sdot_q3_k(const float* x, const uint8_t* row, int K) {   /* :236-282 */
    float acc = 0.0f;
    for (int b = 0; b < K / 256; b++) {
        const uint8_t* blk = row + (size_t)b * 110;
        const float* xq = x + 256 * b;
        float d = or_fp16_to_fp32(rd16(blk + 108));
        uint8_t scales[16];
        q3k_scales(blk + 96, scales);
        const uint8_t* q3 = blk + 32;
        const uint8_t* hm = blk;
        int is = 0;
        uint32_t m = 1;
        for (int j = 0; j < 2; j++, q3 += 32) {
            for (int s = 0; s < 4; s++) {
                int shift = 2 * s;
                float sum0 = 0.0f, sum1 = 0.0f;
                for (int l = 0; l < 16; l++) {
                    int a = (q3[l] >> shift) & 3;
                    a -= (hm[l] & m) ? 0 : 4;
                    sum0 += xq[l] * (float)a;
                }
                for (int l = 16; l < 32; l++) {
                    int a = (q3[l] >> shift) & 3;
                    a -= (hm[l] & m) ? 0 : 4;
                    sum1 += xq[l] * (float)a;
                }
                acc += d * (float)(scales[is] - 32) * sum0; is++;
                acc += d * (float)(scales[is] - 32) * sum1; is++;
                xq += 32;
                m <<= 1;
            }
        }
    }
    return acc;
}

static float sdot_q5_k(const float* x, const uint8_t* row, int K) {   /* :284-314 */
    float acc = 0.0f;
    for (int b = 0; b < K / 256; b++) {
        const uint8_t* blk = row + (size_t)b * 176;
        const float* xb = x + 256 * b;
        float d = or_fp16_to_fp32(rd16(blk));
        float dmin = or_fp16_to_fp32(rd16(blk + 2));
        const uint8_t* qh = blk + 16;
        const uint8_t* q = blk + 48;
        for (int jb = 0, is = 0; jb < 256; jb += 64, is += 2, q += 32) {
            uint8_t sc, m;
            or_get_scale_min_k4(is, blk + 4, &sc, &m);
            float d1 = d * sc, m1 = dmin * m;
            or_get_scale_min_k4(is + 1, blk + 4, &sc, &m);
            float d2 = d * sc, m2 = dmin * m;
            int bit = 2 * (jb / 64);
            float s1 = 0.0f, s2 = 0.0f, x1 = 0.0f, x2 = 0.0f;
            for (int l = 0; l < 32; l++) {
                int v1 = (q[l] & 0xF) + 16 * ((qh[l] >> bit) & 1);
                int v2 = (q[l] >> 4) + 16 * ((qh[l] >> (bit + 1)) & 1);
                s1 += xb[jb + l] * (float)v1; x1 += xb[jb + l];
                s2 += xb[jb + 32 + l] * (float)v2; x2 += xb[jb + 32 + l];
            }
            acc += d1 * s1 - m1 * x1 + d2 * s2 - m2 * x2;
        }
    }
    return acc;
}

typedef float (*sdot_fn)(const float*, const uint8_t*, int);

static sdot_fn scalar_fn(int type) {
    switch (type) {
        case OR_F32: return sdot_f32;
        case OR_F16: return sdot_f16;
        case OR_BF16: return sdot_bf16;
        case OR_Q4_0: return sdot_q4_0;
        case OR_Q5_0: return sdot_q5_0;
        case OR_Q8_0: return sdot_q8_0;
        case OR_Q4_K: return sdot_q4_k;
        case OR_Q6_K: return sdot_q6_k;
        case OR_Q2_K: return sdot_q2_k;
        case OR_Q3_K: return sdot_q3_k;
        case OR_Q5_K: return sdot_q5_k;
        default: return NULL;
    }
}

float or_dot_scalar_row(int type, const float* x, const uint8_t* wrow, int K) {
    sdot_fn f = scalar_fn(type);
    return f ? f(x, wrow, K) : NAN;
}

typedef struct {
    sdot_fn dot; const float* x; const uint8_t* w; float* y;
    int M, K, N; size_t rb;
} gemm_scalar_ctx;

static void gemm_scalar_body(void* p, int j) {   /* src/matmul.cpp:323-328 */
    gemm_scalar_ctx* c = (gemm_scalar_ctx*)p;
    const uint8_t* row = c->w + (size_t)j * c->rb;
    for (int m = 0; m < c->M; m++)
        c->y[(size_t)m * c->N + j] = c->dot(c->x + (size_t)m * c->K, row, c->K);
}

int or_gemm_scalar(int type, const float* x, const uint8_t* w, float* y,
                   int M, int K, int N, int nthreads) {
    sdot_fn f = scalar_fn(type);
    if (!f) return -1;
    gemm_scalar_ctx c = {f, x, w, y, M, K, N, or_row_bytes(type, K)};
    int active = (M > 1 || N >= 128) ? nthreads : 1;
    parallel_for(N, active, gemm_scalar_body, &c);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* dequantize (src/matmul.cpp:504-675).                                     */

int or_dequantize(int type, const uint8_t* w, float* dst, int n) {
    switch (type) {
        case OR_F32: memcpy(dst, w, sizeof(float) * (size_t)n); return 0;
        case OR_F16: for (int i = 0; i < n; i++) dst[i] = or_fp16_to_fp32(rd16(w + 2 * (size_t)i)); return 0;
        case OR_BF16: for (int i = 0; i < n; i++) dst[i] = or_bf16_to_fp32(rd16(w + 2 * (size_t)i)); return 0;
        case OR_Q4_0:
            for (int i = 0; i < n; i += 32) {
                const uint8_t* blk = w + (size_t)(i / 32) * 18;
                float d = or_fp16_to_fp32(rd16(blk));
                for (int l = 0; l < 16; l++) {
                    dst[i + l] = d * (float)((blk[2 + l] & 0xF) - 8);
                    dst[i + l + 16] = d * (float)((blk[2 + l] >> 4) - 8);
                }
            }
            return 0;
        case OR_Q5_0:
            for (int i = 0; i < n; i += 32) {
                const uint8_t* blk = w + (size_t)(i / 32) * 22;
                float d = or_fp16_to_fp32(rd16(blk));
                uint32_t qh = rd32(blk + 2);
                for (int l = 0; l < 16; l++) {
                    int lo0 = (blk[6 + l] & 0xF) | (int)(((qh >> l) & 1u) << 4);
                    int lo1 = (blk[6 + l] >> 4) | (int)(((qh >> (l + 16)) & 1u) << 4);
                    dst[i + l] = d * (float)(lo0 - 16);
                    dst[i + l + 16] = d * (float)(lo1 - 16);
                }
            }
            return 0;
        case OR_Q8_0:
            for (int i = 0; i < n; i += 32) {
                const uint8_t* blk = w + (size_t)(i / 32) * 34;
                float d = or_fp16_to_fp32(rd16(blk));
                for (int l = 0; l < 32; l++) dst[i + l] = d * (float)(int8_t)blk[2 + l];
            }
            return 0;
        case OR_Q4_K:
            for (int i = 0; i < n; i += 256) {
                const uint8_t* blk = w + (size_t)(i / 256) * 144;
                float d = or_fp16_to_fp32(rd16(blk));
                float dmin = or_fp16_to_fp32(rd16(blk + 2));
                const uint8_t* q = blk + 16;
                for (int jb = 0, is = 0; jb < 256; jb += 64, is += 2, q += 32) {
                    uint8_t sc, m;
                    or_get_scale_min_k4(is, blk + 4, &sc, &m);
                    float d1 = d * sc, m1 = dmin * m;
                    or_get_scale_min_k4(is + 1, blk + 4, &sc, &m);
                    float d2 = d * sc, m2 = dmin * m;
                    for (int l = 0; l < 32; l++) dst[i + jb + l] = d1 * (float)(q[l] & 0xF) - m1;
                    for (int l = 0; l < 32; l++) dst[i + jb + 32 + l] = d2 * (float)(q[l] >> 4) - m2;
                }
            }
            return 0;
        case OR_Q6_K:
            for (int i = 0; i < n; i += 256) {
                const uint8_t* blk = w + (size_t)(i / 256) * 210;
                float d = or_fp16_to_fp32(rd16(blk + 208));
                const uint8_t* ql = blk;
                const uint8_t* qh = blk + 128;
                const int8_t* sc = (const int8_t*)(blk + 192);
                float* y = dst + i;
                for (int n_off = 0; n_off < 256; n_off += 128, y += 128, ql += 64, qh += 32, sc += 8) {
                    for (int l = 0; l < 32; l++) {
                        int is = l / 16;
                        int q1 = (int)((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                        int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                        int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                        int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                        y[l] = d * sc[is + 0] * q1;
                        y[l + 32] = d * sc[is + 2] * q2;
                        y[l + 64] = d * sc[is + 4] * q3;
                        y[l + 96] = d * sc[is + 6] * q4;
                    }
                }
            }
            return 0;
        case OR_Q2_K:
            for (int i = 0; i < n; i += 256) {
                const uint8_t* blk = w + (size_t)(i / 256) * 84;
                float d = or_fp16_to_fp32(rd16(blk + 80)), dmin = or_fp16_to_fp32(rd16(blk + 82));
                for (int j = 0; j < 16; j++) {
                    float sc = (float)(blk[j] & 0xF), mn = (float)(blk[j] >> 4);
                    int half = j / 8, jj = j % 8, group = jj / 2, lo = jj % 2;
                    for (int l = 0; l < 16; l++) {
                        int q = (blk[16 + half * 32 + lo * 16 + l] >> (group * 2)) & 3;
                        dst[i + j * 16 + l] = d * sc * (float)q - dmin * mn;
                    }
                }
            }
            return 0;
        case OR_Q3_K:
            for (int i = 0; i < n; i += 256) {
                const uint8_t* blk = w + (size_t)(i / 256) * 110;
                float d = or_fp16_to_fp32(rd16(blk + 108));
                uint8_t scales[16];
                q3k_scales(blk + 96, scales);
                for (int j = 0; j < 16; j++) {
                    float sc = (float)scales[j] - 32;
                    for (int l = 0; l < 16; l++) {
                        int e = j * 16 + l;
                        int g = e / 32, li = e % 32;
                        int low2 = (blk[32 + (g / 4) * 32 + li] >> ((g % 4) * 2)) & 3;
                        int hbit = (blk[li] >> g) & 1;
                        int a = low2 - 4 + 4 * hbit;
                        dst[i + e] = d * sc * (float)a;
                    }
                }
            }
            return 0;
        case OR_Q5_K:
            for (int i = 0; i < n; i += 256) {
                const uint8_t* blk = w + (size_t)(i / 256) * 176;
                float d = or_fp16_to_fp32(rd16(blk)), dmin = or_fp16_to_fp32(rd16(blk + 2));
                const uint8_t* qh = blk + 16;
                const uint8_t* q = blk + 48;
                for (int jb = 0, is = 0; jb < 256; jb += 64, is += 2, q += 32) {
                    uint8_t sc, m;
                    or_get_scale_min_k4(is, blk + 4, &sc, &m); float d1 = d * sc, m1 = dmin * m;
                    or_get_scale_min_k4(is + 1, blk + 4, &sc, &m); float d2 = d * sc, m2 = dmin * m;
                    int bit = 2 * (jb / 64);
                    for (int l = 0; l < 32; l++) {
                        int v1 = (q[l] & 0xF) + 16 * ((qh[l] >> bit) & 1);
                        int v2 = (q[l] >> 4) + 16 * ((qh[l] >> (bit + 1)) & 1);
                        dst[i + jb + l] = d1 * (float)v1 - m1;
                        dst[i + jb + 32 + l] = d2 * (float)v2 - m2;
                    }
                }
            }
            return 0;
        default:
            memset(dst, 0, sizeof(float) * (size_t)n);
            return -1;
    }
}

/* ------------------------------------------------------------------------ */
/* Seeded inputs of tests/test_matmul.cpp.                                  */

typedef struct { uint32_t s; } xs32;
static uint32_t xs_next(xs32* r) { r->s ^= r->s << 13; r->s ^= r->s >> 17; r->s ^= r->s << 5; return r->s; }
static float xs_float(xs32* r) { return (float)(xs_next(r) >> 8) * (2.0f / 16777216.0f) - 1.0f; }
static uint8_t xs_byte(xs32* r) { return (uint8_t)(xs_next(r) & 0xff); }
static uint16_t small_fp16(xs32* r) {                 /* tests/test_matmul.cpp:51-55 */
    float d = 0.005f + 0.065f * (xs_float(r) * 0.5f + 0.5f);
    return or_fp32_to_fp16(d);
}
static void wr16(uint8_t* p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

int or_ref_test_weights(int type, int K, int N, uint8_t* out) {
    xs32 r;
    size_t nblk;
    switch (type) {
        case OR_Q4_0:                                       /* :142-157 */
            r.s = 17; nblk = (size_t)(K / 32) * N;
            for (size_t i = 0; i < nblk; i++) {
                uint8_t* b = out + i * 18;
                wr16(b, small_fp16(&r));
                for (int l = 0; l < 16; l++) b[2 + l] = xs_byte(&r);
            }
            return 0;
        case OR_Q8_0:                                       /* :159-174 */
            r.s = 19; nblk = (size_t)(K / 32) * N;
            for (size_t i = 0; i < nblk; i++) {
                uint8_t* b = out + i * 34;
                wr16(b, small_fp16(&r));
                for (int l = 0; l < 32; l++) b[2 + l] = xs_byte(&r);
            }
            return 0;
        case OR_Q4_K:                                       /* :176-193 */
            r.s = 23; nblk = (size_t)(K / 256) * N;
            for (size_t i = 0; i < nblk; i++) {
                uint8_t* b = out + i * 144;
                wr16(b, small_fp16(&r));
                wr16(b + 2, small_fp16(&r));
                for (int l = 0; l < 12; l++) b[4 + l] = xs_byte(&r);
                for (int l = 0; l < 128; l++) b[16 + l] = xs_byte(&r);
            }
            return 0;
        case OR_Q6_K:                                       /* :195-212 */
            r.s = 29; nblk = (size_t)(K / 256) * N;
            for (size_t i = 0; i < nblk; i++) {
                uint8_t* b = out + i * 210;
                for (int l = 0; l < 128; l++) b[l] = xs_byte(&r);
                for (int l = 0; l < 64; l++) b[128 + l] = xs_byte(&r);
                for (int l = 0; l < 16; l++) b[192 + l] = (uint8_t)(int8_t)((int)(xs_next(&r) % 17) - 8);
                wr16(b + 208, small_fp16(&r));
            }
            return 0;
        default:
            return -1;
    }
}

void or_ref_test_x(int type, int K, float* out) {   /* :45-49, :59-60 */
    xs32 r;
    r.s = 7u + (uint32_t)type;
    for (int k = 0; k < K; k++) out[k] = xs_float(&r);
}

/* ------------------------------------------------------------------------ */
/* Gemma4 MoE feed-forward (src/arch_gemma4.cpp:507-641), all T tokens.     */
/* Per token, in the reference's order:                                     */
/*   rmsnorm_no_scale (:24-29), * router scale * 1/sqrt(H) (:540-541),      */
/*   router matmul (:543-544: the int8 path for the types gemm_simd takes   */
/*   with gemm_int, src/matmul_simd.cpp:484-488, the fp32 dot otherwise),   */
/*   softmax (:546-550), top-k by strict '>' scans (:552-558), weights over */
/*   their sum (:560-562), ops::rmsnorm (src/ops.cpp:68-73), the two expert */
/*   GEMVs (moe_gemv_int / multi), ops::geglu (src/ops.cpp:165-172), the     */
/*   weighted sum (:632-639). Sequential fp32 loops as the reference's       */
/*   non-NEON code.                                                          */
static int int8_type(int t) {
    return t == OR_Q8_0 || t == OR_Q4_0 || t == OR_Q5_0 || t == OR_Q4_K || t == OR_Q6_K;
}

int or_moe_ffn(const float* x, int T, int H, const uint8_t* router_w, int router_type,
               const float* router_scale, const float* pre_norm, float eps,
               const uint8_t* gu_w, int gu_type, const uint8_t* dn_w, int dn_type,
               const float* down_scale, int n_exp, int top_k, int inter,
               float* out, int* idx_out, float* w_out) {
    if (top_k < 1 || top_k > 16 || top_k > n_exp) return -1;
    float* tmp = (float*)malloc(sizeof(float) * (size_t)H);
    float* moe_in = (float*)malloc(sizeof(float) * (size_t)H);
    float* logits = (float*)malloc(sizeof(float) * (size_t)n_exp);
    float* gu = (float*)malloc(sizeof(float) * (size_t)top_k * 2 * inter);
    float* hidden = (float*)malloc(sizeof(float) * (size_t)top_k * inter);
    float* eo = (float*)malloc(sizeof(float) * (size_t)top_k * H);
    int rc = 0;
    const float inv_sqrt_h = 1.0f / sqrtf((float)H);
    for (int m = 0; m < T && rc == 0; m++) {
        const float* xr = x + (size_t)m * H;
        float* o = out + (size_t)m * H;
        for (int i = 0; i < H; i++) o[i] = 0.0f;
        float ms = 0.0f;
        for (int i = 0; i < H; i++) ms += xr[i] * xr[i];
        float inv = 1.0f / sqrtf(ms / H + eps);
        for (int i = 0; i < H; i++) tmp[i] = xr[i] * inv;
        for (int i = 0; i < H; i++) tmp[i] *= router_scale[i] * inv_sqrt_h;
        rc = int8_type(router_type) ? or_gemm_int(router_type, tmp, router_w, logits, 1, H, n_exp, 1)
                                    : or_gemm_scalar(router_type, tmp, router_w, logits, 1, H, n_exp, 1);
        if (rc) break;
        float maxl = logits[0];
        for (int e = 1; e < n_exp; e++) if (logits[e] > maxl) maxl = logits[e];
        float suml = 0.0f;
        for (int e = 0; e < n_exp; e++) { logits[e] = expf(logits[e] - maxl); suml += logits[e]; }
        for (int e = 0; e < n_exp; e++) logits[e] /= suml;
        int idx[16];
        float wk[16];
        for (int k = 0; k < top_k; k++) {
            int best = 0;
            for (int e = 1; e < n_exp; e++) if (logits[e] > logits[best]) best = e;
            idx[k] = best;
            wk[k] = logits[best];
            logits[best] = -1e30f;
        }
        float wsum = 0.0f;
        for (int k = 0; k < top_k; k++) wsum += wk[k];
        for (int k = 0; k < top_k; k++) wk[k] /= wsum;
        /* ops::rmsnorm: its own sum of squares, the same loop */
        float ms2 = 0.0f;
        for (int i = 0; i < H; i++) ms2 += xr[i] * xr[i];
        float inv2 = 1.0f / sqrtf(ms2 / H + eps);
        for (int i = 0; i < H; i++) moe_in[i] = xr[i] * inv2 * pre_norm[i];
        rc = or_moe_gemv_int(gu_type, moe_in, gu_w, idx, top_k, gu, H, 2 * inter, 0, 1);
        if (rc) break;
        const float c = 0.7978845608028654f;
        for (int k = 0; k < top_k; k++) {
            const float* g = gu + (size_t)k * 2 * inter;
            const float* u = g + inter;
            float* hd = hidden + (size_t)k * inter;
            for (int i = 0; i < inter; i++) {
                float gg = g[i];
                float g2 = gg * gg;
                float g3 = g2 * gg;
                float gelu = 0.5f * gg * (1.0f + tanhf(c * (gg + 0.044715f * g3)));
                hd[i] = gelu * u[i];
            }
        }
        rc = or_moe_gemv_int(dn_type, hidden, dn_w, idx, top_k, eo, inter, H, 1, 1);
        if (rc) break;
        for (int k = 0; k < top_k; k++) {
            float weight = wk[k] * down_scale[idx[k]];
            const float* e = eo + (size_t)k * H;
            for (int i = 0; i < H; i++) o[i] += weight * e[i];
        }
        for (int k = 0; k < top_k; k++) {
            if (idx_out) idx_out[(size_t)m * top_k + k] = idx[k];
            if (w_out) w_out[(size_t)m * top_k + k] = wk[k];
        }
    }
    free(tmp); free(moe_in); free(logits); free(gu); free(hidden); free(eo);
    return rc;
}
