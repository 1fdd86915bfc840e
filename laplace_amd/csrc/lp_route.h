// lp_route.h - the route table of the grouped MoE dispatch, built by one
// workgroup (the route kernel, and the top-k kernel of the MoE layer for a
// few tokens).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lp {

// Route table: [count: 1 int][pad to 16 B][groups: max_groups x int4
// (expert, first, n, 0)][pairs: P ints (pair ids sorted by expert)].
// One workgroup: histogram of experts (LDS atomics), exclusive scans of the
// counts and group counts, scatter of pair ids, group table. Pairs whose
// expert index is outside [0, E) are dropped (their outputs are not written).
// rs: LDS of 3 E + 2 (blockDim.x / 64) ints; idx may be in LDS.
__device__ inline void build_route(const int* idx, int P, int E, uint8_t* __restrict__ route, int max_groups,
                                   int gsize, int* rs) {
    int* cnt = rs;                 // E
    int* off = rs + E;             // E: first pair slot of expert e
    int* goff = rs + 2 * E;        // E: first group of expert e
    int* part = rs + 3 * E;        // 2 scan partials per wave
    int* ngroups = reinterpret_cast<int*>(route);
    int4* groups = reinterpret_cast<int4*>(route + 16);
    int* pairs = reinterpret_cast<int*>(route + 16 + (size_t)max_groups * 16);
    const int tid = threadIdx.x, nt = blockDim.x;
    for (int e = tid; e < E; e += nt) cnt[e] = 0;
    __syncthreads();
    for (int p = tid; p < P; p += nt) {
        const int e = idx[p];
        if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    // block scan: thread i owns experts [i*per, (i+1)*per)
    const int per = (E + nt - 1) / nt;
    const int e0 = tid * per, e1 = e0 + per < E ? e0 + per : E;
    int sc = 0, sg = 0;
    for (int e = e0; e < e1; e++) {
        sc += cnt[e];
        sg += (cnt[e] + gsize - 1) / gsize;
    }
    // inclusive scan of (sc, sg): within the wave by shuffles, then the
    // preceding waves' totals from LDS (one barrier)
    const int lane = tid & 63, wv = tid >> 6;
    int ia = sc, ib = sg;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int ta = __shfl_up(ia, o, 64), tb = __shfl_up(ib, o, 64);
        if (lane >= o) {
            ia += ta;
            ib += tb;
        }
    }
    if (lane == 63) {
        part[2 * wv] = ia;
        part[2 * wv + 1] = ib;
    }
    __syncthreads();
    for (int v = 0; v < wv; v++) {
        ia += part[2 * v];
        ib += part[2 * v + 1];
    }
    sc = ia - sc;                   // exclusive prefix
    sg = ib - sg;
    for (int e = e0; e < e1; e++) {
        off[e] = sc;
        goff[e] = sg;
        const int c = cnt[e];
        for (int g = 0; g * gsize < c; g++) {
            const int n = c - g * gsize < gsize ? c - g * gsize : gsize;
            groups[sg + g] = make_int4(e, sc + g * gsize, n, 0);
        }
        sc += c;
        sg += (c + gsize - 1) / gsize;
    }
    if (tid == nt - 1) ngroups[0] = ib;
    __syncthreads();
    // scatter: slot within the expert from a second round of atomics
    for (int e = tid; e < E; e += nt) cnt[e] = 0;
    __syncthreads();
    for (int p = tid; p < P; p += nt) {
        const int e = idx[p];
        if (e >= 0 && e < E) pairs[off[e] + atomicAdd(&cnt[e], 1)] = p;
    }
}

}  // namespace lp
