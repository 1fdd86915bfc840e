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

// The same table from one wave for P <= 64 pairs (lane p holds pair p):
// pair p's slot is its rank in (expert, pair id) order and k_p its position
// within its expert, both counted over broadcasts of every pair's expert;
// the pairs with k_p % gsize == 0 start the groups, numbered in slot order.
// No atomics or barriers; pairs within an expert come in pair-id order.
__device__ inline void build_route_wave(const int* idx, int P, int E, uint8_t* __restrict__ route, int max_groups,
                                        int gsize) {
    const int lane = threadIdx.x & 63;
    int* ngroups = reinterpret_cast<int*>(route);
    int4* groups = reinterpret_cast<int4*>(route + 16);
    int* pairs = reinterpret_cast<int*>(route + 16 + (size_t)max_groups * 16);
    const int e = lane < P ? idx[lane] : -1;
    const bool valid = lane < P && e >= 0 && e < E;
    int rank = 0, k = 0, cnt = 0;
    for (int q = 0; q < P; q++) {
        const int eq = __builtin_amdgcn_readlane(e, q);
        if (eq >= 0 && eq < E) {
            rank += (eq < e) || (eq == e && q < lane);
            k += eq == e && q < lane;
            cnt += eq == e;
        }
    }
    const bool starter = valid && k % gsize == 0;
    const uint64_t sb = __ballot(starter);
    int gi = 0;
    for (int q = 0; q < P; q++) {
        if ((sb >> q) & 1) gi += __builtin_amdgcn_readlane(rank, q) < rank;
    }
    if (valid) pairs[rank] = lane;
    if (starter) groups[gi] = make_int4(e, rank, cnt - k < gsize ? cnt - k : gsize, 0);
    if (lane == 0) ngroups[0] = (int)__popcll(sb);
}

}  // namespace lp
