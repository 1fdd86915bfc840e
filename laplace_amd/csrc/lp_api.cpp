// lp_api.cpp - C ABI over the gfx950 kernels (declarations in
// include/laplace_hip.h).
//
// Host-pointer entry points keep the reference back-end's contract
// (src/kernels.h:94-119): synchronous, internally parallel, false when the
// type is not handled. They stage x and y through pinned host buffers on a
// library-owned stream and take weights from device copies: a registered
// region (lp_register_weights, after src/metal.mm:581-599) or a copy cached
// by host pointer on first use (after get_weight_buf, src/metal.mm:601-621).
// Calls are serialised by one mutex, as the Metal back-end does
// (src/metal.mm:646).
#include <algorithm>
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "../../include/laplace_hip.h"
#include "lp_internal.h"

namespace lp {

static thread_local char g_err[512];

static void set_err(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

#define LP_HIP(call)                                                              \
    do {                                                                          \
        hipError_t e_ = (call);                                                   \
        if (e_ != hipSuccess) {                                                   \
            set_err("%s failed: %s (%s:%d)", #call, hipGetErrorString(e_),        \
                    __FILE__, __LINE__);                                          \
            return LP_EHIP;                                                       \
        }                                                                         \
    } while (0)

struct DevInfo {
    bool probed = false;
    bool ok = false;
    int cus = 0;
};

static std::mutex g_info_mtx;
static std::unordered_map<int, DevInfo> g_info;

static DevInfo& dev_info() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = -1;
    std::lock_guard<std::mutex> lk(g_info_mtx);
    DevInfo& di = g_info[dev];
    if (!di.probed) {
        di.probed = true;
        hipDeviceProp_t p;
        if (dev >= 0 && hipGetDeviceProperties(&p, dev) == hipSuccess) {
            di.cus = p.multiProcessorCount;
            di.ok = std::strncmp(p.gcnArchName, "gfx950", 6) == 0;
        }
    }
    return di;
}

int device_cu_count() {
    int n = dev_info().cus;
    return n > 0 ? n : 256;
}

// ---------------------------------------------------------------------------
// Workspace layout for quantized activations:
//   [qs: M*K int8][d: M*nb f32][sum: M*nb f32][s16: M*nb i32], each 256-B aligned.

static size_t up256(size_t v) { return (v + 255) & ~size_t(255); }

static size_t act_bytes(int M, int K) {
    const size_t nbk = (size_t)M * (K / 32);
    return up256((size_t)M * K) + 3 * up256(nbk * 4);
}

// Scratch for the partial sums of the K-split Q6_K row-quad GEMV (3 <= M <= 8).
constexpr size_t kPartReserve = size_t(2) << 20;
static size_t part_reserve(int M) { return M >= 3 && M <= 8 ? kPartReserve : 0; }

static size_t planes_reserve(int M, int K) { return M >= 5 ? gemm_planes_bytes(M, K) : 0; }

// Activation blocks, plus the fp16 planes of the MFMA products when M >= 5,
// plus the partial-sum scratch when 3 <= M <= 8.
static size_t ws_bytes(int M, int K) {
    return act_bytes(M, K) + planes_reserve(M, K) + part_reserve(M);
}

static void* ws_planes(void* ws, int M, int K) {
    return static_cast<uint8_t*>(ws) + act_bytes(M, K);
}

static ActView ws_view(void* ws, int M, int K) {
    uint8_t* p = static_cast<uint8_t*>(ws);
    const size_t nbk = (size_t)M * (K / 32);
    ActView a;
    a.qs = reinterpret_cast<int8_t*>(p);
    p += up256((size_t)M * K);
    a.d = reinterpret_cast<float*>(p);
    p += up256(nbk * 4);
    a.sum = reinterpret_cast<float*>(p);
    p += up256(nbk * 4);
    a.s16 = reinterpret_cast<int32_t*>(p);
    return a;
}

// ws_view of a workspace of ws_bytes(M, K) bytes, with its partial-sum scratch.
static ActView ws_view_full(void* ws, int M, int K) {
    ActView a = ws_view(ws, M, K);
    if (part_reserve(M)) {
        a.part = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + act_bytes(M, K) + planes_reserve(M, K));
        a.part_bytes = part_reserve(M);
    }
    return a;
}

static bool type_handled(uint32_t t) {
    return t == T_Q8_0 || t == T_Q4_0 || t == T_Q5_0 || t == T_Q4_K || t == T_Q6_K;
}

// Shape/alignment preconditions of the kernels. Returns LP_OK or the status
// to report.
static int check_shape(uint32_t type, const void* w, int M, int K, int N) {
    if (fact_type(type)) {
        // fp32-activation path: whole 32-element chunks (whole super-blocks for K-quants)
        if (M < 0 || K <= 0 || N < 0) {
            set_err("bad shape M=%d K=%d N=%d", M, K, N);
            return LP_EINVAL;
        }
        const int need = (type == T_Q2_K || type == T_Q3_K || type == T_Q5_K) ? 256 : 32;
        if (K % need != 0) {
            set_err("K=%d must be a multiple of %d for type %u", K, need, type);
            return LP_UNSUPPORTED;
        }
        const uintptr_t align = (type == T_F32 || type == T_Q2_K || type == T_Q5_K) ? 4 : 2;
        if (reinterpret_cast<uintptr_t>(w) % align != 0) {
            set_err("weights must be %zu-byte aligned for type %u", (size_t)align, type);
            return LP_UNSUPPORTED;
        }
        return LP_OK;
    }
    if (!type_handled(type)) {
        set_err("type %u not handled on the GPU", type);
        return LP_UNSUPPORTED;
    }
    if (M < 0 || K <= 0 || N < 0) {
        set_err("bad shape M=%d K=%d N=%d", M, K, N);
        return LP_EINVAL;
    }
    const int need = (type == T_Q4_K || type == T_Q6_K) ? 256 : type == T_Q5_0 ? 32 : 64;
    if (K % need != 0 || K > 32768) {
        set_err("K=%d must be a multiple of %d and at most 32768", K, need);
        return LP_UNSUPPORTED;
    }
    const uintptr_t a = reinterpret_cast<uintptr_t>(w);
    const uintptr_t align = (type == T_Q4_K) ? 16 : type == T_Q5_0 ? 2 : 4;
    if (a % align != 0) {
        set_err("weights must be %zu-byte aligned for type %u", (size_t)align, type);
        return LP_UNSUPPORTED;
    }
    return LP_OK;
}

// Whether M > 16 rows run on the tiled GEMM. Q4_K at small prefill sizes
// runs faster as 16-row chunks on the int8 MFMA kernel (one weight pass per
// chunk) than on the GEMM's 64-token tiles (measured per call at
// N x K = 14336 x 4096 / 4096 x 14336: M=17 32 vs 49 and 52 vs 136 us;
// M=32 49 vs 54 and 82 vs 142; M=48 71 vs 59 and 122 vs 149; M=64 94 vs
// 64 and 161 vs 155).
static bool use_gemm(uint32_t type, int M, int K, int N, const uint8_t* w) {
    if (!gemm_supported(type, M, K) || i8mf_supported(type, M, K, N, w)) return false;
    if (type == T_Q4_K && i8mf_supported(type, 16, K, N, w) && (M <= 32 || (M <= 64 && N <= 4096))) return false;
    return true;
}

static int gemm_q(const ActView& A, void* planes, const uint8_t* w, uint32_t type, float* y,
                  int M, int K, int N, hipStream_t st) {
    if (i8mf_supported(type, M, K, N, w)) {
        LP_HIP(launch_gemv_i8mf(type, w, A, y, M, K, N, st));
        return LP_OK;
    }
    if (planes && use_gemm(type, M, K, N, w)) {
        LP_HIP(launch_gemm(type, w, A, planes, y, M, K, N, st));
        return LP_OK;
    }
    // no GEMM kernel for the type: chunks of rows through the widest small-M
    // path (Q8_0: several 16-token tiles per workgroup; 16 rows on int8 MFMA
    // where the type has it, else 8 on the GEMV)
    if (M > 16 && i8_chunk_supported(type, K, N, w)) {
        const int ch = i8_chunk_rows();
        for (int m0 = 0; m0 < M; m0 += ch) {
            const int mt = M - m0 < ch ? M - m0 : ch;
            ActView sub = A;
            sub.qs = A.qs + (size_t)m0 * K;
            sub.d = A.d + (size_t)m0 * (K / 32);
            sub.sum = A.sum + (size_t)m0 * (K / 32);
            sub.s16 = A.s16 + (size_t)m0 * (K / 32);
            LP_HIP(launch_i8_chunk(type, w, sub, y + (size_t)m0 * N, mt, K, N, st));
        }
        return LP_OK;
    }
    const int chunk = i8mf_supported(type, 16, K, N, w) ? 16 : 8;
    for (int m0 = 0; m0 < M; m0 += chunk) {
        const int mt = M - m0 < chunk ? M - m0 : chunk;
        ActView sub = A;                 // the partial-sum scratch is shared (stream-ordered)
        sub.qs = A.qs + (size_t)m0 * K;
        sub.d = A.d + (size_t)m0 * (K / 32);
        sub.sum = A.sum + (size_t)m0 * (K / 32);
        sub.s16 = A.s16 + (size_t)m0 * (K / 32);
        if (i8mf_supported(type, mt, K, N, w)) LP_HIP(launch_gemv_i8mf(type, w, sub, y + (size_t)m0 * N, mt, K, N, st));
        else LP_HIP(launch_gemv(type, w, sub, y + (size_t)m0 * N, mt, K, N, st));
    }
    return LP_OK;
}

// The kernel gemm_q runs for these operands (first chunk when rows are
// chunked), for the routing probe lp_gemm_route.
static const char* gemm_q_route(uint32_t type, int M, int K, int N, const uint8_t* w) {
    if (i8mf_supported(type, M, K, N, w))
        return rq_preferred(type, M, K, N, w) ? "rq" : q6rq_preferred(type, M, K, N, w) ? "q6rq" : "i8mf";
    if (use_gemm(type, M, K, N, w)) return "gemm";
    if (M > 16 && i8_chunk_supported(type, K, N, w)) return "i8mf";
    const int chunk = i8mf_supported(type, 16, K, N, w) ? 16 : 8;
    const int mt = M < chunk ? M : chunk;
    if (i8mf_supported(type, mt, K, N, w))
        return rq_preferred(type, mt, K, N, w) ? "rq" : q6rq_preferred(type, mt, K, N, w) ? "q6rq" : "i8mf";
    return gemv_route_name(type, mt, K, N, w);
}

// ---------------------------------------------------------------------------
// Host-pointer machinery.

struct Region {
    const uint8_t* host;
    size_t size;
    uint8_t* dev;   // device address of host[0]
    void* alloc;    // what hipMalloc returned (dev minus the alignment offset)
};

struct HostCtx {
    hipStream_t stream = nullptr;
    std::vector<Region> regions;                       // registered ranges
    std::unordered_map<const void*, Region> copies;    // per-pointer cache
    void* ws = nullptr;
    size_t ws_cap = 0;
    float* xd = nullptr;
    size_t xd_cap = 0;
    float* yd = nullptr;
    size_t yd_cap = 0;
    int* idx_d = nullptr;
    size_t idx_cap = 0;
    float* x_pin = nullptr;
    size_t x_pin_cap = 0;
    float* y_pin = nullptr;
    size_t y_pin_cap = 0;
};

// Transfers up to this size go by a copy kernel through the pinned buffers'
// device addresses (the kernel's PCIe reads and posted writes finish sooner
// than a DMA copy at these sizes); larger ones by DMA.
constexpr size_t kKernelCopyMax = 1u << 20;
// pin: the pinned allocation (its base, from grow_pinned), off: the bytes
// at pin + off
static int copy_h2d(HostCtx& c, void* dst_dev, void* pin, size_t off, size_t bytes) {
    uint8_t* src_pin = static_cast<uint8_t*>(pin) + off;
#ifndef LP_NO_KCOPY
    if (bytes <= kKernelCopyMax) {
        void* base = nullptr;
        LP_HIP(hipHostGetDevicePointer(&base, pin, 0));
        LP_HIP(launch_copy(dst_dev, static_cast<uint8_t*>(base) + off, bytes, c.stream));
        return LP_OK;
    }
#endif
    LP_HIP(hipMemcpyAsync(dst_dev, src_pin, bytes, hipMemcpyHostToDevice, c.stream));
    return LP_OK;
}
static int copy_d2h(HostCtx& c, void* pin, size_t off, const void* src_dev, size_t bytes) {
    uint8_t* dst_pin = static_cast<uint8_t*>(pin) + off;
#ifndef LP_NO_KCOPY
    if (bytes <= kKernelCopyMax) {
        void* base = nullptr;
        LP_HIP(hipHostGetDevicePointer(&base, pin, 0));
        LP_HIP(launch_copy(static_cast<uint8_t*>(base) + off, src_dev, bytes, c.stream));
        return LP_OK;
    }
#endif
    LP_HIP(hipMemcpyAsync(dst_pin, src_dev, bytes, hipMemcpyDeviceToHost, c.stream));
    return LP_OK;
}

static std::mutex g_host_mtx;
static std::unordered_map<int, HostCtx> g_host;

static HostCtx* host_ctx() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    HostCtx& c = g_host[dev];
    if (!c.stream && hipStreamCreate(&c.stream) != hipSuccess) return nullptr;
    return &c;
}

template <typename T>
static int grow_dev(T*& p, size_t& cap, size_t bytes) {
    if (bytes <= cap) return LP_OK;
    if (p) (void)hipFree(p);
    p = nullptr;
    cap = 0;
    LP_HIP(hipMalloc(reinterpret_cast<void**>(&p), bytes));
    cap = bytes;
    return LP_OK;
}

template <typename T>
static int grow_pinned(T*& p, size_t& cap, size_t bytes) {
    if (bytes <= cap) return LP_OK;
    if (p) (void)hipHostFree(p);
    p = nullptr;
    cap = 0;
    LP_HIP(hipHostMalloc(reinterpret_cast<void**>(&p), bytes, hipHostMallocDefault));
    cap = bytes;
    return LP_OK;
}

// Device address of `len` bytes of host weights at w.
static int resolve_weights(HostCtx& c, const uint8_t* w, size_t len, const uint8_t** out) {
    for (const Region& r : c.regions) {
        if (w >= r.host && w + len <= r.host + r.size) {
            *out = r.dev + (w - r.host);
            return LP_OK;
        }
    }
    auto it = c.copies.find(w);
    if (it != c.copies.end() && it->second.size >= len) {
        *out = it->second.dev;
        return LP_OK;
    }
    if (it != c.copies.end()) {
        (void)hipFree(it->second.alloc);
        c.copies.erase(it);
    }
    uint8_t* d = nullptr;
    LP_HIP(hipMalloc(reinterpret_cast<void**>(&d), len));
    if (hipMemcpy(d, w, len, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(d);
        set_err("weight upload failed");
        return LP_EHIP;
    }
    c.copies[w] = Region{w, len, d, d};
    *out = d;
    return LP_OK;
}

// Shared body of the host-pointer GEMM / MoE calls. rows = activation rows
// staged (M for the GEMM, 1 or n_experts for MoE).
static int host_gemm(const float* x, const uint8_t* w, uint32_t type, float* y, int M, int K,
                     int N) {
    int st = check_shape(type, w, M, K, N);
    if (st != LP_OK) return st;
    if (!dev_info().ok) {
        set_err("no gfx950 device");
        return LP_ENODEV;
    }
    if (M == 0 || N == 0) return LP_OK;
    std::lock_guard<std::mutex> lk(g_host_mtx);
    HostCtx* c = host_ctx();
    if (!c) {
        set_err("no HIP device/stream");
        return LP_ENODEV;
    }
    const size_t xb = sizeof(float) * (size_t)M * K, yb = sizeof(float) * (size_t)M * N;
    const uint8_t* wd = nullptr;
    int rc;
    const size_t rbytes = fact_type(type) ? fact_row_bytes(type, K) : row_bytes(type, K);
    if ((rc = resolve_weights(*c, w, rbytes * (size_t)N, &wd)) != LP_OK) return rc;
    if ((rc = grow_dev(c->xd, c->xd_cap, xb)) != LP_OK) return rc;
    if ((rc = grow_dev(c->yd, c->yd_cap, yb)) != LP_OK) return rc;
    if ((rc = grow_dev(c->ws, c->ws_cap, ws_bytes(M, K))) != LP_OK) return rc;
    if ((rc = grow_pinned(c->x_pin, c->x_pin_cap, xb)) != LP_OK) return rc;
    if ((rc = grow_pinned(c->y_pin, c->y_pin_cap, yb)) != LP_OK) return rc;
    std::memcpy(c->x_pin, x, xb);
    if ((rc = copy_h2d(*c, c->xd, c->x_pin, 0, xb)) != LP_OK) return rc;
    if (fact_type(type)) {
        LP_HIP(launch_gemv_fact(type, wd, c->xd, c->yd, M, K, N, c->stream));
    } else if (gemv_fused_supported(type, M, K, wd)) {
        LP_HIP(launch_gemv_fused(type, wd, c->xd, c->yd, M, K, N, c->stream));
    } else if (i8mf_supported(type, M, K, N, wd)) {
        const ActView A = ws_view_full(c->ws, M, K);
        LP_HIP(launch_quantize(c->xd, M, K, A, c->stream));
        LP_HIP(launch_gemv_i8mf(type, wd, A, c->yd, M, K, N, c->stream));
    } else if (use_gemm(type, M, K, N, wd) && !gemm_i8_preferred(type, M, K, N)) {
        void* planes = ws_planes(c->ws, M, K);
        LP_HIP(launch_planes_from_x(c->xd, planes, M, K, c->stream, N, c->yd));
        LP_HIP(launch_gemm_planes(type, wd, planes, c->yd, M, K, N, c->stream, true));
    } else {
        const ActView A = ws_view_full(c->ws, M, K);
        LP_HIP(launch_quantize(c->xd, M, K, A, c->stream));
        if ((rc = gemm_q(A, ws_planes(c->ws, M, K), wd, type, c->yd, M, K, N, c->stream)) != LP_OK)
            return rc;
    }
    if ((rc = copy_d2h(*c, c->y_pin, 0, c->yd, yb)) != LP_OK) return rc;
    LP_HIP(hipStreamSynchronize(c->stream));
    std::memcpy(y, c->y_pin, yb);
    return LP_OK;
}

// Workspace of the grouped MoE call: activation rows (T, or T*topk in the
// multi form), then the route table.
// Workspace of the grouped MoE call: activation blocks and fp16 planes of the
// activation rows (T, or T*topk in the multi form), then the route table.
static size_t moe_ws_bytes(int T, int topk, int E, int K, int multi) {
    const int P = T * topk, rows = multi ? P : T;
    return act_bytes(rows, K) + up256(moe_route_bytes(P, E));
}

static int check_moe(uint32_t type, const void* w, int T, int topk, int E, int K, int N) {
    if (fact_type(type) || type == T_Q5_0) {
        // the caller's per-expert fallback (src/matmul.cpp:467-479) then runs
        // each expert through lp_gemm, which takes these types
        set_err("type %u: grouped MoE takes the int8 types only", type);
        return LP_UNSUPPORTED;
    }
    int st = check_shape(type, w, 1, K, N);
    if (st != LP_OK) return st;
    if (T < 0 || topk < 0 || (T > 0 && topk > 0 && (E <= 0 || E > kMoeMaxExperts))) {
        set_err("bad MoE shape T=%d topk=%d n_experts=%d (at most %d experts)", T, topk, E,
                kMoeMaxExperts);
        return LP_EINVAL;
    }
    if ((long)T * topk > (1L << 24)) {
        set_err("too many (token, expert) pairs: %ld", (long)T * topk);
        return LP_EINVAL;
    }
    return LP_OK;
}

// Pairs per routed group below the 16-pair MFMA groups: 8 on the row-quad
// kernel once experts average more than 2 pairs (groups of 4 would split
// many experts into groups that each read the expert again; measured at 128
// experts, 64 tokens, top-8: 133 vs 147 us), else 4 on the GEMV kernels
// (one or two pairs per expert: 39 vs 41 us at one token, 52 vs 58 at four).
static int moe_group_size(uint32_t type, int K, int P, int E) {
    return rq_moe_supported(type, K) && P > 2 * E ? kRqMoeGroup : 4;
}

static constexpr bool kMoeFuseQuantRoute = true;

static int moe_q(const float* x, int multi, const int* idx, const uint8_t* w, uint32_t type,
                 float* y, int T, int topk, int E, int K, int N, void* ws, hipStream_t st) {
    const int P = T * topk, rows = multi ? P : T;
    const ActView A = ws_view(ws, rows, K);
    void* route = static_cast<uint8_t*>(ws) + act_bytes(rows, K);
    // groups of <= 16 pairs on the int8 MFMA kernel pay off when experts are
    // chosen by more than 8 pairs on average (prefill; at 128 experts, top-8:
    // 10 per expert 259 vs 274 us on the GEMV kernels, 8 per expert 246 vs
    // 236 us; 6 per expert 177 vs 137 us); decode-sized batches stay on the
    // GEMV kernels
    const bool mf = moe_mf_supported(type, K) && P > 8 * E;
    const int gs = mf ? 16 : moe_group_size(type, K, P, E);
    if (kMoeFuseQuantRoute) {
        // one launch for the quantization and the route table (the route
        // kernel alone is one short workgroup)
        LP_HIP(launch_moe_quant_route(x, rows, K, A, idx, P, E, route, gs, st));
        LP_HIP(launch_moe_grouped_routed(type, w, A, gs, rows, P, E, multi, topk, route, y, K, N, st));
    } else {
        LP_HIP(launch_quantize(x, rows, K, A, st));
        LP_HIP(launch_moe_grouped(type, w, A, gs, rows, idx, P, E, multi, topk, route, y, K, N, st));
    }
    return LP_OK;
}

// Host-pointer grouped MoE: T tokens x topk experts; idx[T*topk] is checked
// on the host (a pair naming an expert outside [0, E) is an error).
static int host_moe_grouped(const float* x, int multi, const int* idx, const uint8_t* w,
                            uint32_t type, float* y, int T, int topk, int E, int K, int N) {
    int st = check_moe(type, w, T, topk, E, K, N);
    if (st != LP_OK) return st;
    const int P = T * topk;
    if (P == 0 || N == 0) return LP_OK;
    for (int p = 0; p < P; p++) {
        if (idx[p] < 0 || idx[p] >= E) {
            set_err("expert index %d at pair %d outside [0, %d)", idx[p], p, E);
            return LP_EINVAL;
        }
    }
    if (!dev_info().ok) {
        set_err("no gfx950 device");
        return LP_ENODEV;
    }
    std::lock_guard<std::mutex> lk(g_host_mtx);
    HostCtx* c = host_ctx();
    if (!c) {
        set_err("no HIP device/stream");
        return LP_ENODEV;
    }
    const int rows = multi ? P : T;
    const size_t xb = sizeof(float) * (size_t)rows * K, yb = sizeof(float) * (size_t)P * N;
    const uint8_t* wd = nullptr;
    int rc;
    if ((rc = resolve_weights(*c, w, row_bytes(type, K) * (size_t)N * E, &wd)) != LP_OK) return rc;
    if ((rc = grow_dev(c->xd, c->xd_cap, xb)) != LP_OK) return rc;
    if ((rc = grow_dev(c->yd, c->yd_cap, yb)) != LP_OK) return rc;
    if ((rc = grow_dev(c->ws, c->ws_cap, moe_ws_bytes(T, topk, E, K, multi))) != LP_OK) return rc;
    if ((rc = grow_dev(c->idx_d, c->idx_cap, sizeof(int) * (size_t)P)) != LP_OK) return rc;
    if ((rc = grow_pinned(c->x_pin, c->x_pin_cap, xb + sizeof(int) * (size_t)P)) != LP_OK) return rc;
    if ((rc = grow_pinned(c->y_pin, c->y_pin_cap, yb)) != LP_OK) return rc;
    std::memcpy(c->x_pin, x, xb);
    int* idx_pin = reinterpret_cast<int*>(reinterpret_cast<uint8_t*>(c->x_pin) + xb);
    std::memcpy(idx_pin, idx, sizeof(int) * (size_t)P);
    if ((rc = copy_h2d(*c, c->xd, c->x_pin, 0, xb)) != LP_OK) return rc;
    if ((rc = copy_h2d(*c, c->idx_d, c->x_pin, xb, sizeof(int) * (size_t)P)) != LP_OK) return rc;
    if ((rc = moe_q(c->xd, multi, c->idx_d, wd, type, c->yd, T, topk, E, K, N, c->ws, c->stream)) != LP_OK)
        return rc;
    if ((rc = copy_d2h(*c, c->y_pin, 0, c->yd, yb)) != LP_OK) return rc;
    LP_HIP(hipStreamSynchronize(c->stream));
    std::memcpy(y, c->y_pin, yb);
    return LP_OK;
}

// The reference's per-token MoE entry (src/kernels.h:100-112): one token,
// n_exp selected experts. The stacked tensor's expert count is not passed,
// so the selected indices bound the device copy.
static int host_moe(const float* x, const uint8_t* w, uint32_t type, const int* idx, int n_exp,
                    float* y, int K, int N, bool multi) {
    if (fact_type(type) || type == T_Q5_0) return check_moe(type, w, 1, n_exp, 1, K, N);
    if (n_exp <= 0 || N == 0) return check_shape(type, w, 1, K, N);
    int E = 0;
    for (int k = 0; k < n_exp; k++) {
        if (idx[k] < 0) {
            set_err("negative expert index %d", idx[k]);
            return LP_EINVAL;
        }
        E = idx[k] + 1 > E ? idx[k] + 1 : E;
    }
    if (E > kMoeMaxExperts) {
        set_err("expert index %d beyond %d", E - 1, kMoeMaxExperts);
        return LP_UNSUPPORTED;
    }
    return host_moe_grouped(x, multi ? 1 : 0, idx, w, type, y, 1, n_exp, E, K, N);
}

}  // namespace lp

using namespace lp;

extern "C" {

bool lp_gemm(const float* x, const uint8_t* w, uint32_t type, float* y, int M, int K, int N) {
    int rc = host_gemm(x, w, type, y, M, K, N);
    if (rc != LP_OK && rc != LP_UNSUPPORTED) fprintf(stderr, "[laplace_hip] %s\n", g_err);
    return rc == LP_OK;
}

bool lp_moe_gemv(const float* x, const uint8_t* w, uint32_t type, const int* expert_idx,
                 int n_experts, float* y, int K, int N) {
    int rc = host_moe(x, w, type, expert_idx, n_experts, y, K, N, false);
    if (rc != LP_OK && rc != LP_UNSUPPORTED) fprintf(stderr, "[laplace_hip] %s\n", g_err);
    return rc == LP_OK;
}

bool lp_moe_gemv_multi(const float* x, const uint8_t* w, uint32_t type, const int* expert_idx,
                       int n_experts, float* y, int K, int N) {
    int rc = host_moe(x, w, type, expert_idx, n_experts, y, K, N, true);
    if (rc != LP_OK && rc != LP_UNSUPPORTED) fprintf(stderr, "[laplace_hip] %s\n", g_err);
    return rc == LP_OK;
}

lp_gemm_fn lp_get_gemm(void) { return dev_info().ok ? lp_gemm : nullptr; }
lp_moe_gemv_fn lp_get_moe_gemv(void) { return dev_info().ok ? lp_moe_gemv : nullptr; }
lp_moe_gemv_fn lp_get_moe_gemv_multi(void) { return dev_info().ok ? lp_moe_gemv_multi : nullptr; }

int lp_register_weights(const void* base, size_t size) {
    if (!base || size == 0) {
        set_err("empty region");
        return LP_EINVAL;
    }
    std::lock_guard<std::mutex> lk(g_host_mtx);
    HostCtx* c = host_ctx();
    if (!c) return LP_ENODEV;
    // The copy starts at the same offset modulo 256 as the host region, so
    // a host weight pointer and the device address it resolves to have the
    // same alignment (the kernels' 16-byte loads rely on it).
    const size_t off = reinterpret_cast<uintptr_t>(base) & 255;
    uint8_t* d = nullptr;
    LP_HIP(hipMalloc(reinterpret_cast<void**>(&d), size + off));
    if (hipMemcpy(d + off, base, size, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(d);
        set_err("weight upload failed");
        return LP_EHIP;
    }
    c->regions.push_back(Region{static_cast<const uint8_t*>(base), size, d + off, d});
    return LP_OK;
}

int lp_release_region(const void* base) {
    std::lock_guard<std::mutex> lk(g_host_mtx);
    HostCtx* c = host_ctx();
    if (!c) return LP_ENODEV;
    for (size_t i = 0; i < c->regions.size(); i++) {
        if (c->regions[i].host == base) {
            (void)hipStreamSynchronize(c->stream);
            (void)hipFree(c->regions[i].alloc);
            c->regions.erase(c->regions.begin() + i);
            return LP_OK;
        }
    }
    set_err("no registered region starts at %p", base);
    return LP_EINVAL;
}

void lp_release_weights(void) {
    std::lock_guard<std::mutex> lk(g_host_mtx);
    HostCtx* c = host_ctx();
    if (!c) return;
    (void)hipStreamSynchronize(c->stream);
    for (Region& r : c->regions) (void)hipFree(r.alloc);
    for (auto& kv : c->copies) (void)hipFree(kv.second.alloc);
    c->regions.clear();
    c->copies.clear();
}

int lp_quantize_act(const float* x, int M, int K, float* d, float* sum, int16_t* sum_lo,
                    int16_t* sum_hi, int8_t* qs) {
    if (K % 32 != 0 || M < 0) return LP_EINVAL;
    if (!dev_info().ok) return LP_ENODEV;
    if (M == 0) return LP_OK;
    std::lock_guard<std::mutex> lk(g_host_mtx);
    HostCtx* c = host_ctx();
    if (!c) return LP_ENODEV;
    const size_t xb = sizeof(float) * (size_t)M * K;
    const size_t nbk = (size_t)M * (K / 32);
    int rc;
    if ((rc = grow_dev(c->xd, c->xd_cap, xb)) != LP_OK) return rc;
    if ((rc = grow_dev(c->ws, c->ws_cap, ws_bytes(M, K))) != LP_OK) return rc;
    LP_HIP(hipMemcpyAsync(c->xd, x, xb, hipMemcpyHostToDevice, c->stream));
    const ActView A = ws_view(c->ws, M, K);
    LP_HIP(launch_quantize(c->xd, M, K, A, c->stream));
    std::vector<int32_t> s16(nbk);
    LP_HIP(hipMemcpyAsync(qs, A.qs, (size_t)M * K, hipMemcpyDeviceToHost, c->stream));
    LP_HIP(hipMemcpyAsync(d, A.d, nbk * 4, hipMemcpyDeviceToHost, c->stream));
    LP_HIP(hipMemcpyAsync(sum, A.sum, nbk * 4, hipMemcpyDeviceToHost, c->stream));
    LP_HIP(hipMemcpyAsync(s16.data(), A.s16, nbk * 4, hipMemcpyDeviceToHost, c->stream));
    LP_HIP(hipStreamSynchronize(c->stream));
    for (size_t i = 0; i < nbk; i++) {
        sum_lo[i] = (int16_t)(uint16_t)((uint32_t)s16[i] & 0xffffu);
        sum_hi[i] = (int16_t)(uint16_t)((uint32_t)s16[i] >> 16);
    }
    return LP_OK;
}

size_t lp_act_workspace_bytes(int M, int K) { return ws_bytes(M, K); }

int lp_quantize_act_dev(const float* x, int M, int K, void* ws, size_t wsb, void* stream) {
    if (K % 32 != 0 || M < 0 || (M > 0 && (!x || !ws))) return LP_EINVAL;
    if (wsb < ws_bytes(M, K)) {
        set_err("workspace %zu < %zu bytes", wsb, ws_bytes(M, K));
        return LP_EINVAL;
    }
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0) {
        set_err("x must be 16-byte aligned");
        return LP_EINVAL;
    }
    LP_HIP(launch_quantize(x, M, K, ws_view_full(ws, M, K), static_cast<hipStream_t>(stream)));
    return LP_OK;
}

int lp_act_unpack_dev(const void* ws, int M, int K, float* d, float* sum, int32_t* sums16,
                      int8_t* qs, void* stream) {
    const ActView A = ws_view(const_cast<void*>(ws), M, K);
    const size_t nbk = (size_t)M * (K / 32);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (qs) LP_HIP(hipMemcpyAsync(qs, A.qs, (size_t)M * K, hipMemcpyDeviceToDevice, st));
    if (d) LP_HIP(hipMemcpyAsync(d, A.d, nbk * 4, hipMemcpyDeviceToDevice, st));
    if (sum) LP_HIP(hipMemcpyAsync(sum, A.sum, nbk * 4, hipMemcpyDeviceToDevice, st));
    if (sums16) LP_HIP(hipMemcpyAsync(sums16, A.s16, nbk * 4, hipMemcpyDeviceToDevice, st));
    return LP_OK;
}

int lp_gemm_q_dev(const void* ws, const uint8_t* w, uint32_t type, float* y, int M, int K, int N,
                  void* stream) {
    if (fact_type(type)) {
        set_err("type %u takes fp32 activations (lp_gemm_dev), not quantized blocks", type);
        return LP_UNSUPPORTED;
    }
    int rc = check_shape(type, w, M, K, N);
    if (rc != LP_OK) return rc;
    return gemm_q(ws_view_full(const_cast<void*>(ws), M, K), ws_planes(const_cast<void*>(ws), M, K), w,
                  type, y, M, K, N, static_cast<hipStream_t>(stream));
}

const char* lp_gemm_route(uint32_t type, int M, int K, int N, const void* w) {
    if (fact_type(type)) return "fact";
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    if (check_shape(type, wb, M, K, N) != LP_OK || M <= 0 || N <= 0) return "";
    return gemm_q_route(type, M, K, N, wb);
}

int lp_gemm_dev(const float* x, const uint8_t* w, uint32_t type, float* y, int M, int K, int N,
                void* ws, size_t wsb, void* stream) {
    int rc = check_shape(type, w, M, K, N);
    if (rc != LP_OK) return rc;
    if (fact_type(type)) {
        // fp32 activations straight into the GEMV (no workspace)
        if (M > 0 && N > 0 && (!x || !y)) {
            set_err("null pointer");
            return LP_EINVAL;
        }
        if (reinterpret_cast<uintptr_t>(x) % 16 != 0) {
            set_err("x must be 16-byte aligned");
            return LP_EINVAL;
        }
        LP_HIP(launch_gemv_fact(type, w, x, y, M, K, N, static_cast<hipStream_t>(stream)));
        return LP_OK;
    }
    if (gemv_fused_supported(type, M, K, w)) {
        // one launch: the GEMV quantizes x itself (bit-identical blocks)
        if (wsb < ws_bytes(M, K) || (M > 0 && (!x || !y))) {
            set_err("workspace %zu < %zu bytes or null pointer", wsb, ws_bytes(M, K));
            return LP_EINVAL;
        }
        if (reinterpret_cast<uintptr_t>(x) % 16 != 0) {
            set_err("x must be 16-byte aligned");
            return LP_EINVAL;
        }
        LP_HIP(launch_gemv_fused(type, w, x, y, M, K, N, static_cast<hipStream_t>(stream)));
        return LP_OK;
    }
    if (use_gemm(type, M, K, N, w) && !gemm_i8_preferred(type, M, K, N)) {
        // fp16 planes straight from x (one pass), then the MFMA product
        if (wsb < ws_bytes(M, K) || (M > 0 && (!x || !y))) {
            set_err("workspace %zu < %zu bytes or null pointer", wsb, ws_bytes(M, K));
            return LP_EINVAL;
        }
        if (reinterpret_cast<uintptr_t>(x) % 16 != 0) {
            set_err("x must be 16-byte aligned");
            return LP_EINVAL;
        }
        void* planes = ws_planes(ws, M, K);
        hipStream_t hs = static_cast<hipStream_t>(stream);
        LP_HIP(launch_planes_from_x(x, planes, M, K, hs, N, y));
        LP_HIP(launch_gemm_planes(type, w, planes, y, M, K, N, hs, true));
        return LP_OK;
    }
    if ((rc = lp_quantize_act_dev(x, M, K, ws, wsb, stream)) != LP_OK) return rc;
    return lp_gemm_q_dev(ws, w, type, y, M, K, N, stream);
}

int lp_block_sums_dev(const void* ws, const uint8_t* w, uint32_t type, int32_t* out, int M, int K,
                      int N, void* stream) {
    if (fact_type(type) || type == T_Q5_0) {
        set_err("type %u: no block-sum probe", type);
        return LP_UNSUPPORTED;
    }
    int rc = check_shape(type, w, M, K, N);
    if (rc != LP_OK) return rc;
    LP_HIP(launch_block_sums(type, w, ws_view(const_cast<void*>(ws), M, K), out, M, K, N,
                             static_cast<hipStream_t>(stream)));
    return LP_OK;
}

size_t lp_moe_workspace_bytes(int T, int topk, int n_experts, int K, int multi) {
    if (T < 0 || topk < 0 || n_experts < 0 || K < 0) return 0;
    return moe_ws_bytes(T, topk, n_experts, K, multi);
}

int lp_moe_grouped_dev(const float* x, int multi, const int* topk_idx, const uint8_t* w,
                       uint32_t type, float* y, int T, int topk, int n_experts, int K, int N,
                       void* ws, size_t wsb, void* stream) {
    int rc = check_moe(type, w, T, topk, n_experts, K, N);
    if (rc != LP_OK) return rc;
    if (T == 0 || topk == 0 || N == 0) return LP_OK;
    if (!x || !topk_idx || !w || !y || !ws) {
        set_err("null pointer");
        return LP_EINVAL;
    }
    if (wsb < moe_ws_bytes(T, topk, n_experts, K, multi)) {
        set_err("workspace %zu < %zu bytes", wsb, moe_ws_bytes(T, topk, n_experts, K, multi));
        return LP_EINVAL;
    }
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0) {
        set_err("x must be 16-byte aligned");
        return LP_EINVAL;
    }
    return moe_q(x, multi ? 1 : 0, topk_idx, w, type, y, T, topk, n_experts, K, N, ws,
                 static_cast<hipStream_t>(stream));
}

// ---- MoE feed-forward --------------------------------------------------------

namespace {
struct FfnWs {
    float *rin, *ein, *logits, *wts, *gu, *hidden, *eo;
    int* idx;
    void* rws;       // router GEMV workspace (int8 router types)
    size_t rws_b;
    void* mws;       // grouped-MoE workspace
    size_t mws_b;
    ActView eq, hq;  // int8 blocks of ein [T, H] and hidden [P, inter] (fused quantization)
    void* route;     // route table shared by both expert passes
    size_t total;
};

FfnWs ffn_layout(void* base, int T, int H, int n_exp, int top_k, int inter, uint32_t router_type) {
    FfnWs f{};
    const size_t P = (size_t)T * top_k;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off += up256(bytes);
        return static_cast<uint8_t*>(base) + o;
    };
    f.rin = reinterpret_cast<float*>(take(4 * (size_t)T * H));
    f.ein = reinterpret_cast<float*>(take(4 * (size_t)T * H));
    f.logits = reinterpret_cast<float*>(take(4 * (size_t)T * n_exp));
    f.idx = reinterpret_cast<int*>(take(4 * P));
    f.wts = reinterpret_cast<float*>(take(4 * P));
    f.gu = reinterpret_cast<float*>(take(4 * P * 2 * inter));
    f.hidden = reinterpret_cast<float*>(take(4 * P * inter));
    f.eo = reinterpret_cast<float*>(take(4 * P * H));
    f.rws_b = fact_type(router_type) ? 0 : ws_bytes(T, H);
    f.rws = take(f.rws_b);
    const size_t m0 = moe_ws_bytes(T, top_k, n_exp, H, 0), m1 = moe_ws_bytes(T, top_k, n_exp, inter, 1);
    f.mws_b = m0 > m1 ? m0 : m1;
    f.mws = take(f.mws_b);
    f.eq = ws_view(take(act_bytes(T, H)), T, H);
    f.hq = ws_view(take(act_bytes((int)P, inter)), (int)P, inter);
    f.route = take(moe_route_bytes((int)P, n_exp));
    f.total = off;
    return f;
}
}  // namespace

size_t lp_moe_ffn_workspace_bytes(int T, int H, int n_exp, int top_k, int inter, uint32_t router_type) {
    if (T < 0 || H <= 0 || n_exp <= 0 || top_k <= 0 || inter <= 0) return 0;
    return ffn_layout(nullptr, T, H, n_exp, top_k, inter, router_type).total;
}

int lp_moe_ffn_dev(const float* x, int T, int H, const uint8_t* router_w, uint32_t router_type,
                   const float* router_scale, const float* pre_norm, float rms_eps,
                   const uint8_t* gate_up_w, uint32_t gate_up_type, const uint8_t* down_w,
                   uint32_t down_type, const float* down_scale, int n_exp, int top_k, int inter,
                   float* out, int* topk_idx, float* topk_w, void* ws, size_t wsb, void* stream) {
    if (T < 0 || H <= 0 || n_exp <= 0 || inter <= 0 || top_k < 1 || top_k > 16 || top_k > n_exp ||
        n_exp > moe_topk_max_experts()) {
        set_err("bad MoE layer shape T=%d H=%d n_exp=%d top_k=%d inter=%d (n_exp <= %d, top_k <= 16)", T, H,
                n_exp, top_k, inter, moe_topk_max_experts());
        return LP_EINVAL;
    }
    int rc;
    if ((rc = check_shape(router_type, router_w, T, H, n_exp)) != LP_OK) return rc;
    if ((rc = check_moe(gate_up_type, gate_up_w, T, top_k, n_exp, H, 2 * inter)) != LP_OK) return rc;
    if ((rc = check_moe(down_type, down_w, T, top_k, n_exp, inter, H)) != LP_OK) return rc;
    if (T == 0) return LP_OK;
    if (!x || !router_w || !router_scale || !pre_norm || !gate_up_w || !down_w || !down_scale || !out || !ws) {
        set_err("null pointer");
        return LP_EINVAL;
    }
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(ws) % 256 != 0) {
        set_err("x must be 16-byte and ws 256-byte aligned");
        return LP_EINVAL;
    }
    const FfnWs f = ffn_layout(ws, T, H, n_exp, top_k, inter, router_type);
    if (wsb < f.total) {
        set_err("workspace %zu < %zu bytes", wsb, f.total);
        return LP_EINVAL;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    int* idx = topk_idx ? topk_idx : f.idx;
    float* wts = topk_w ? topk_w : f.wts;
    const int P = T * top_k;
    // Decode-sized batches (neither expert pass on the MFMA kernel): the norm
    // and GeGLU kernels also write the int8 blocks the expert GEMVs read, and
    // one route table serves both passes.
    const bool fused = !(moe_mf_supported(gate_up_type, H) && P > 8 * n_exp) &&
                       !(moe_mf_supported(down_type, inter) && P > 8 * n_exp) && H % 32 == 0 &&
                       inter % 32 == 0 && reinterpret_cast<uintptr_t>(router_scale) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(pre_norm) % 16 == 0;
    if (fused && moe_norm_router_supported(T, H, router_type, router_w, router_scale, pre_norm)) {
        // few tokens: one launch for the norms and the router (measured at
        // 128 experts, top-8, us per layer: T=1 30.9 -> 28.1, T=2 35.4 ->
        // 34.6, T=4 46.5 -> 46.6)
        LP_HIP(launch_moe_norm_router(x, T, H, router_scale, pre_norm, rms_eps,
                                      reinterpret_cast<const float*>(router_w), n_exp, f.logits, f.ein, f.eq, st));
    } else {
        LP_HIP(launch_moe_norms(x, T, H, router_scale, pre_norm, rms_eps, f.rin, f.ein, fused ? f.eq : ActView{},
                                st));
        if ((rc = lp_gemm_dev(f.rin, router_w, router_type, f.logits, T, H, n_exp, f.rws, f.rws_b, stream)) != LP_OK)
            return rc;
    }
    if (fused) {
        // one route table for both products: groups of 8 only if both run on
        // the row-quad kernel; for a few tokens the top-k kernel builds it
        const int gs = std::min(moe_group_size(gate_up_type, H, P, n_exp), moe_group_size(down_type, inter, P, n_exp));
        if (moe_topk_route_supported(T)) {
            LP_HIP(launch_moe_topk_route(f.logits, T, n_exp, top_k, idx, wts, f.route, gs, st));
        } else {
            LP_HIP(launch_moe_topk(f.logits, T, n_exp, top_k, idx, wts, st));
            LP_HIP(launch_moe_route(idx, P, n_exp, f.route, gs, st));
        }
        LP_HIP(launch_moe_grouped_routed(gate_up_type, gate_up_w, f.eq, gs, T, P, n_exp, 0, top_k, f.route,
                                         f.gu, H, 2 * inter, st));
        if (T <= 4 && moe_geglu_fusable(down_type, inter, gs, down_w)) {
            // the down GEMV applies GeGLU and quantizes while staging its
            // activations (every workgroup of a group redoes its pairs' GeGLU:
            // measured faster than the separate kernel up to 4 tokens, at 128
            // experts top-8 T=1 33.5 -> 32.5 us, T=4 47.2 -> 46.5; slower from
            // 16: 82.7 -> 84.4, T=64 134 -> 139)
            LP_HIP(launch_moe_grouped_routed(down_type, down_w, f.hq, gs, P, P, n_exp, 1, top_k, f.route, f.eo,
                                             inter, H, st, f.gu));
        } else {
            LP_HIP(launch_geglu(f.gu, P, inter, f.hidden, f.hq, st));
            LP_HIP(launch_moe_grouped_routed(down_type, down_w, f.hq, gs, P, P, n_exp, 1, top_k, f.route, f.eo,
                                             inter, H, st));
        }
    } else {
        LP_HIP(launch_moe_topk(f.logits, T, n_exp, top_k, idx, wts, st));
        if ((rc = lp_moe_grouped_dev(f.ein, 0, idx, gate_up_w, gate_up_type, f.gu, T, top_k, n_exp, H, 2 * inter,
                                     f.mws, f.mws_b, stream)) != LP_OK)
            return rc;
        LP_HIP(launch_geglu(f.gu, P, inter, f.hidden, ActView{}, st));
        if ((rc = lp_moe_grouped_dev(f.hidden, 1, idx, down_w, down_type, f.eo, T, top_k, n_exp, inter, H, f.mws,
                                     f.mws_b, stream)) != LP_OK)
            return rc;
    }
    LP_HIP(launch_moe_combine(f.eo, idx, wts, down_scale, T, top_k, H, out, st));
    return LP_OK;
}

// ---- Batched M=1 matmuls (matmul_gemm_batch) ---------------------------------

// Specs i..j-1 can share one multi-matrix launch: same activation row and K,
// Q4_K weights the fused GEMV takes.
static bool batch_fusable(const lp_batch_spec& a, const lp_batch_spec& b) {
    return a.x == b.x && a.K == b.K && a.type == T_Q4_K && b.type == T_Q4_K &&
           gemv_fused_supported(T_Q4_K, 1, a.K, a.w) && gemv_fused_supported(T_Q4_K, 1, b.K, b.w);
}

static int check_batch(const lp_batch_spec* specs, int n) {
    if (n < 0 || (n > 0 && !specs)) {
        set_err("bad batch: n=%d", n);
        return LP_EINVAL;
    }
    for (int i = 0; i < n; i++) {
        const lp_batch_spec& s = specs[i];
        int rc = check_shape(s.type, s.w, 1, s.K, s.N);
        if (rc != LP_OK) return rc;
        if (s.N > 0 && (!s.x || !s.y)) {
            set_err("spec %d: null pointer", i);
            return LP_EINVAL;
        }
        if (reinterpret_cast<uintptr_t>(s.x) % 16 != 0) {
            set_err("spec %d: x must be 16-byte aligned", i);
            return LP_EINVAL;
        }
    }
    return LP_OK;
}

size_t lp_gemm_batch_workspace_bytes(const lp_batch_spec* specs, int n) {
    size_t b = 0;
    for (int i = 0; specs && i < n; i++) {
        const size_t w = specs[i].K > 0 ? ws_bytes(1, specs[i].K) : 0;
        if (w > b) b = w;
    }
    return b;
}

// Specs already validated; device pointers.
static int batch_dev(const lp_batch_spec* specs, int n, void* ws, size_t wsb, hipStream_t st) {
    int i = 0;
    while (i < n) {
        int j = i + 1;
        while (j < n && j - i < kBatchMax && batch_fusable(specs[i], specs[j])) j++;
        if (j - i >= 2) {
            const uint8_t* w[kBatchMax];
            float* y[kBatchMax];
            int nn[kBatchMax];
            for (int k = i; k < j; k++) {
                w[k - i] = specs[k].w;
                y[k - i] = specs[k].y;
                nn[k - i] = specs[k].N;
            }
            LP_HIP(launch_gemv_fused_batch(w, y, nn, j - i, specs[i].x, specs[i].K, st));
        } else {
            const lp_batch_spec& s = specs[i];
            const int rc = lp_gemm_dev(s.x, s.w, s.type, s.y, 1, s.K, s.N, ws, wsb, st);
            if (rc != LP_OK) return rc;
        }
        i = j;
    }
    return LP_OK;
}

int lp_gemm_batch_dev(const lp_batch_spec* specs, int n, void* ws, size_t wsb, void* stream) {
    int rc = check_batch(specs, n);
    if (rc != LP_OK) return rc;
    return batch_dev(specs, n, ws, wsb, static_cast<hipStream_t>(stream));
}

// Host pointers, synchronous: every spec's x is staged once (specs naming the
// same x with the same K share the staged copy), weights resolve through the
// registered regions or the per-pointer cache, all outputs come back with one
// copy.
static int host_gemm_batch(const lp_batch_spec* specs, int n) {
    int rc = check_batch(specs, n);
    if (rc != LP_OK) return rc;
    if (n == 0) return LP_OK;
    if (!dev_info().ok) {
        set_err("no gfx950 device");
        return LP_ENODEV;
    }
    std::lock_guard<std::mutex> lk(g_host_mtx);
    HostCtx* c = host_ctx();
    if (!c) {
        set_err("no HIP device/stream");
        return LP_ENODEV;
    }
    // offsets (floats, 16-byte aligned) of each spec's staged x and y
    std::vector<size_t> xo(n), yo(n);
    size_t xt = 0, yt = 0;
    for (int i = 0; i < n; i++) {
        int share = -1;
        for (int k = 0; k < i; k++)
            if (specs[k].x == specs[i].x && specs[k].K == specs[i].K) { share = k; break; }
        if (share >= 0) xo[i] = xo[share];
        else { xo[i] = xt; xt += ((size_t)specs[i].K + 3) & ~size_t(3); }
        yo[i] = yt;
        yt += ((size_t)specs[i].N + 3) & ~size_t(3);
    }
    if ((rc = grow_dev(c->xd, c->xd_cap, 4 * xt)) != LP_OK) return rc;
    if ((rc = grow_dev(c->yd, c->yd_cap, 4 * yt)) != LP_OK) return rc;
    if ((rc = grow_dev(c->ws, c->ws_cap, lp_gemm_batch_workspace_bytes(specs, n))) != LP_OK) return rc;
    if ((rc = grow_pinned(c->x_pin, c->x_pin_cap, 4 * xt)) != LP_OK) return rc;
    if ((rc = grow_pinned(c->y_pin, c->y_pin_cap, 4 * yt)) != LP_OK) return rc;
    std::vector<lp_batch_spec> ds(specs, specs + n);
    // Each distinct weight pointer is resolved once, for the longest span any
    // spec reads from it: resolving a later, longer span would replace the
    // cached copy an earlier spec already points to.
    std::vector<size_t> span(n);
    for (int i = 0; i < n; i++) {
        const lp_batch_spec& s = specs[i];
        const size_t rbytes = fact_type(s.type) ? fact_row_bytes(s.type, s.K) : row_bytes(s.type, s.K);
        span[i] = s.N > 0 ? rbytes * (size_t)s.N : 0;
    }
    for (int i = 0; i < n; i++) {
        if (span[i] == 0) continue;
        int first = i;
        for (int k = 0; k < i; k++)
            if (span[k] && specs[k].w == specs[i].w) { first = k; break; }
        if (first != i) continue;
        size_t len = span[i];
        for (int k = i + 1; k < n; k++)
            if (specs[k].w == specs[i].w && span[k] > len) len = span[k];
        const uint8_t* d = nullptr;
        if ((rc = resolve_weights(*c, specs[i].w, len, &d)) != LP_OK) return rc;
        for (int k = i; k < n; k++)
            if (span[k] && specs[k].w == specs[i].w) ds[k].w = d;
    }
    for (int i = 0; i < n; i++) {
        const lp_batch_spec& s = specs[i];
        std::memcpy(c->x_pin + xo[i], s.x, sizeof(float) * (size_t)s.K);
        ds[i].x = c->xd + xo[i];
        ds[i].y = c->yd + yo[i];
    }
    if (xt && (rc = copy_h2d(*c, c->xd, c->x_pin, 0, 4 * xt)) != LP_OK) return rc;
    if ((rc = batch_dev(ds.data(), n, c->ws, c->ws_cap, c->stream)) != LP_OK) return rc;
    if (yt && (rc = copy_d2h(*c, c->y_pin, 0, c->yd, 4 * yt)) != LP_OK) return rc;
    LP_HIP(hipStreamSynchronize(c->stream));
    for (int i = 0; i < n; i++) std::memcpy(specs[i].y, c->y_pin + yo[i], sizeof(float) * (size_t)specs[i].N);
    return LP_OK;
}

bool lp_gemm_batch(const lp_batch_spec* specs, int n) {
    int rc = host_gemm_batch(specs, n);
    if (rc != LP_OK && rc != LP_UNSUPPORTED) fprintf(stderr, "[laplace_hip] %s\n", g_err);
    return rc == LP_OK;
}

bool lp_moe_grouped(const float* x, int multi, const int* topk_idx, const uint8_t* w,
                    uint32_t type, float* y, int T, int topk, int n_experts, int K, int N) {
    int rc = host_moe_grouped(x, multi ? 1 : 0, topk_idx, w, type, y, T, topk, n_experts, K, N);
    if (rc != LP_OK && rc != LP_UNSUPPORTED) fprintf(stderr, "[laplace_hip] %s\n", g_err);
    return rc == LP_OK;
}

int lp_dequantize_dev(const uint8_t* w, uint32_t type, float* dst, long n, void* stream) {
    const int epb = dequant_block_elems(type);
    if (epb == 0) {
        set_err("type %u not handled by dequantize", type);
        return LP_UNSUPPORTED;
    }
    if (n < 0 || n % epb != 0 || (n > 0 && (!w || !dst))) {
        set_err("n=%ld must be a non-negative multiple of %d", n, epb);
        return LP_EINVAL;
    }
    LP_HIP(launch_dequant(type, w, dst, n, static_cast<hipStream_t>(stream)));
    return LP_OK;
}

int lp_dequantize(const uint8_t* w, uint32_t type, float* dst, long n) {
    const int epb = dequant_block_elems(type);
    if (epb == 0) {
        set_err("type %u not handled by dequantize", type);
        return LP_UNSUPPORTED;
    }
    if (n < 0 || n % epb != 0) {
        set_err("n=%ld must be a non-negative multiple of %d", n, epb);
        return LP_EINVAL;
    }
    if (n == 0) return LP_OK;
    if (!dev_info().ok) {
        set_err("no gfx950 device");
        return LP_ENODEV;
    }
    std::lock_guard<std::mutex> lk(g_host_mtx);
    HostCtx* c = host_ctx();
    if (!c) return LP_ENODEV;
    const size_t src = dequant_src_bytes(type, n), yb = sizeof(float) * (size_t)n;
    const uint8_t* wd = nullptr;
    int rc;
    if ((rc = resolve_weights(*c, w, src, &wd)) != LP_OK) return rc;
    if ((rc = grow_dev(c->yd, c->yd_cap, yb)) != LP_OK) return rc;
    LP_HIP(launch_dequant(type, wd, c->yd, n, c->stream));
    LP_HIP(hipMemcpyAsync(dst, c->yd, yb, hipMemcpyDeviceToHost, c->stream));
    LP_HIP(hipStreamSynchronize(c->stream));
    return LP_OK;
}

// ---- the entry point that allocates nothing -------------------------------
// lp_gemm_dev with its workspace in a file-scope device array instead of a
// caller buffer. Each device holds its own copy of the array; its device
// address is looked up once per device (hipGetSymbolAddress, with that
// device current) and kept. In host code `scratch` only names the symbol:
// kernels get the looked-up address. Nothing in the scratch needs to start
// at zero (the quantizer writes every activation block and plane the
// products read), and calls that overlap on one device race on it.
constexpr size_t kNoAllocScratch = size_t(8) << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratch];
static std::mutex g_scratch_mtx;
static void* g_scratch_dev[64];

static int scratch_ptr(void** out) {
    int dev = 0;
    LP_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) {
        set_err("device ordinal %d out of range", dev);
        return LP_ENODEV;
    }
    std::lock_guard<std::mutex> lk(g_scratch_mtx);
    if (!g_scratch_dev[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            set_err("hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
            return LP_EHIP;
        }
        g_scratch_dev[dev] = p;
    }
    *out = g_scratch_dev[dev];
    return LP_OK;
}

int lp_gemm_dev_noalloc(const float* x, const uint8_t* w, uint32_t type, float* y, int M, int K, int N,
                        void* stream) {
    int rc = check_shape(type, w, M, K, N);
    if (rc != LP_OK) return rc;
    const size_t need = fact_type(type) ? 0 : ws_bytes(M, K);
    if (need > kNoAllocScratch) {
        set_err("M=%d K=%d needs %zu bytes of workspace; the no-alloc scratch holds %zu (use lp_gemm_dev)",
                M, K, need, kNoAllocScratch);
        return LP_EINVAL;
    }
    void* ws = nullptr;
    if ((rc = scratch_ptr(&ws)) != LP_OK) return rc;
    return lp_gemm_dev(x, w, type, y, M, K, N, ws, kNoAllocScratch, stream);
}

int lp_read_probe_dev(const void* buf, size_t bytes, int grid, int block, int unroll, uint32_t* sink,
                      void* stream) {
    if (!buf || !sink) {
        set_err("null pointer");
        return LP_EINVAL;
    }
    LP_HIP(launch_read_probe(buf, bytes, grid, block, unroll, sink, static_cast<hipStream_t>(stream)));
    return LP_OK;
}

int lp_mfma_probe_dev(int kind, int random_operands, int iters, int grid, float* out, void* stream) {
    if (!out || iters < 1 || grid < 1 || kind < 0 || kind > 9) {
        set_err("bad probe arguments");
        return LP_EINVAL;
    }
    LP_HIP(launch_mfma_probe(kind, random_operands, iters, grid, out, static_cast<hipStream_t>(stream)));
    return LP_OK;
}

int lp_set_gemm_kernel(int kernel) {
    if (kernel < 0 || kernel > 5) {
        set_err("kernel %d: 0 (by shape) or 1-5", kernel);
        return LP_EINVAL;
    }
    set_gemm_kernel(kernel);
    return LP_OK;
}

const char* lp_last_error(void) { return g_err; }

int lp_device_ok(void) { return dev_info().ok ? 1 : 0; }

int lp_device_info(int* cus, int* clock_khz, int* mem_clock_khz, int* mem_bus_bits) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        set_err("no device");
        return LP_EINVAL;
    }
    int v[4] = {0, 0, 0, 0};
    const hipDeviceAttribute_t at[4] = {hipDeviceAttributeMultiprocessorCount, hipDeviceAttributeClockRate,
                                        hipDeviceAttributeMemoryClockRate, hipDeviceAttributeMemoryBusWidth};
    for (int i = 0; i < 4; i++)
        if (hipDeviceGetAttribute(&v[i], at[i], dev) != hipSuccess) v[i] = 0;
    if (cus) *cus = v[0];
    if (clock_khz) *clock_khz = v[1];
    if (mem_clock_khz) *mem_clock_khz = v[2];
    if (mem_bus_bits) *mem_bus_bits = v[3];
    return LP_OK;
}

}  // extern "C"
