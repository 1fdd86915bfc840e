"""Benchmark of the MI355X GGUF quantized-matmul path (one GPU).

Headline: Q4_K decode GEMV, W = 14336 x 4096
(N x K), M = 1, fp32 activations quantized on the fly to 32-element int8
blocks. One step = quantize x + GEMV against one weight copy; steps rotate
over >= 16 distinct device copies of the weights (> 512 MB, twice the
256 MB Infinity Cache) so every step streams its weights from HBM. Steps
are captured in a HIP graph (torch.cuda.graph around the C-ABI calls, which
launch on torch's current stream) and replayed; the timed region is
bracketed by torch.cuda.synchronize().

value = algorithmic bytes per step / time per step, in GB/s, where
algorithmic bytes = weight bytes + 4*M*K (x) + 4*M*N (y).

roofline: the GEMV kernel alone, timed with HIP events over graph replays
of back-to-back GEMV launches on pre-quantized activations; achieved =
algorithmic bytes per launch / average launch duration; peak = 8000 GB/s.
traffic: HBM bytes per launch from rocprofv3 PMC runs, read from
profiles/<workload>_traffic.json when that file exists (else null).

cpu_baseline: the reference's portable scalar path (gemm_scalar<dot_row_q4_k>,
src/matmul.cpp:137-167, :320-334) as restated in oracle/liboracle.so, on the
host cores, same weights, whole matrix, median of repeated runs.

Extra lines (also in the JSON): the other BASELINE.json GEMV configs
("extra"), the prefill GEMM ("gemm"), the grouped MoE expert GEMVs ("moe")
and the whole MoE feed-forward layer ("moe_ffn": router to combine).
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
ROTATE_MIN_BYTES = 512 << 20
KERNEL_MIN_LAUNCHES = 200
Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14
F32, F16, Q5_0, Q2_K, Q3_K, Q5_K, BF16 = 0, 1, 6, 10, 11, 13, 30
FACT_TYPES = (F32, F16, BF16, Q2_K, Q3_K, Q5_K)   # fp32-activation GEMV
TNAME = {Q4_0: "Q4_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q6_K: "Q6_K", F32: "F32", F16: "F16",
         BF16: "BF16", Q5_0: "Q5_0", Q2_K: "Q2_K", Q3_K: "Q3_K", Q5_K: "Q5_K"}


def row_bytes(t, K):
    return {Q4_0: K // 32 * 18, Q8_0: K // 32 * 34, Q4_K: K // 256 * 144, Q6_K: K // 256 * 210,
            F32: K * 4, F16: K * 2, BF16: K * 2, Q5_0: K // 32 * 22, Q2_K: K // 256 * 84,
            Q3_K: K // 256 * 110, Q5_K: K // 256 * 176}[t]


def synth_weights(t, K, N, seed):
    """Seeded blocks with BASELINE.json's distributions (uniform codes and
    6-bit fields, fp16 scales |N(0,1)| * 0.01, Q4_0 * 0.02, Q6_K int8
    scales uniform in [-32, 31])."""
    rng = np.random.default_rng(seed)
    if t in (F32, F16, BF16):
        v = (rng.standard_normal(K * N) * 0.05).astype(np.float32)
        if t == F32:
            return v.view(np.uint8).copy()
        if t == F16:
            return v.astype(np.float16).view(np.uint8).copy()
        return (v.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).copy()
    bpb = {Q4_0: 18, Q8_0: 34, Q4_K: 144, Q6_K: 210, Q5_0: 22, Q2_K: 84, Q3_K: 110, Q5_K: 176}[t]
    w = rng.integers(0, 256, row_bytes(t, K) * N, dtype=np.uint8)
    b = w.reshape(-1, bpb)
    nb = b.shape[0]

    def f16(scale):
        return (np.abs(rng.standard_normal(nb)) * scale).astype(np.float16).view(np.uint8).reshape(-1, 2)
    if t == Q8_0:
        b[:, 2:] = rng.integers(-127, 128, (nb, 32), dtype=np.int8).view(np.uint8)
        b[:, 0:2] = f16(0.01)
    elif t == Q4_0:
        b[:, 0:2] = f16(0.02)
    elif t == Q4_K:
        b[:, 0:2] = f16(0.01)
        b[:, 2:4] = f16(0.01)
    elif t == Q6_K:
        b[:, 192:208] = rng.integers(-32, 32, (nb, 16), dtype=np.int8).view(np.uint8)
        b[:, 208:210] = f16(0.01)
    else:
        # fp16 scale fields of Q5_0 / Q2_K / Q3_K / Q5_K
        for off in {Q5_0: [0], Q2_K: [80, 82], Q3_K: [108], Q5_K: [0, 2]}[t]:
            b[:, off:off + 2] = f16(0.01)
    return w


def synth_x(M, K, seed, outliers=0.0):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K)).astype(np.float32)
    if outliers:
        x[rng.random((M, K)) < outliers] *= 20.0
    return x


class Gpu:
    def __init__(self):
        import torch
        from laplace_amd import _lib
        self.torch = torch
        self.L = _lib.lib()
        self.check = _lib.check
        if not torch.cuda.is_available():
            raise SystemExit("bench.py needs a GPU (cuda:0)")
        if self.L.lp_device_ok() != 1:
            raise SystemExit("device is not gfx950")
        self.dev = torch.device("cuda:0")

    def stream(self):
        return C.c_void_p(self.torch.cuda.current_stream().cuda_stream)

    def copies(self, w_host, min_bytes=ROTATE_MIN_BYTES, min_copies=16):
        torch = self.torch
        n = max(min_copies, -(-min_bytes // w_host.nbytes))
        base = torch.from_numpy(w_host).to(self.dev)
        out = [base]
        for _ in range(n - 1):
            out.append(base.clone())
        return out


# (grid, block, loads in flight per thread); (224, 1024, 9) is the GEMV's own
# shape at 14336 x 4096 (224 workgroups of 16 waves, 9 x 16 B per lane)
READ_PROBE_SHAPES = [(224, 1024, 9), (256, 1024, 9), (512, 1024, 4), (1024, 512, 4), (2048, 256, 4),
                     (2048, 1024, 1), (4096, 512, 1), (8192, 256, 1), (16384, 128, 1), (32768, 64, 1)]


def measure_read_ceiling(g: Gpu, bufs, nbytes, reps, wreps, shapes=None):
    """The part's streaming-read ceiling for this byte count: the
    lp_read_probe_dev kernel over the same rotating weight copies, graph-
    timed like the GEMV kernel, best of READ_PROBE_SHAPES (grid, block,
    loads in flight per thread)."""
    torch = g.torch
    sink = torch.zeros(4, dtype=torch.int32, device=g.dev)
    ncp = len(bufs)
    nb = nbytes - nbytes % 16
    res = []
    for (grid, block, unroll) in (shapes or READ_PROBE_SHAPES):
        def launch(i):
            g.check(g.L.lp_read_probe_dev(bufs[i % ncp].data_ptr(), nb, grid, block, unroll, sink.data_ptr(),
                                          g.stream()), "lp_read_probe_dev")
        launch(0)
        torch.cuda.synchronize()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            launch(1)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for i in range(ncp):
                launch(i)
        for _ in range(wreps):
            gr.replay()
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        ev0.record()
        for _ in range(reps):
            gr.replay()
        ev1.record()
        torch.cuda.synchronize()
        us = ev0.elapsed_time(ev1) * 1e3 / (reps * ncp)
        res.append((us, grid, block, unroll))
    us, grid, block, unroll = min(res)
    return {"us": round(us, 3), "gbs": round(nb / (us * 1e-6) / 1e9, 1),
            "frac_of_peak": round(nb / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "best_shape": {"grid": grid, "block": block, "loads_in_flight_per_thread": unroll},
            "shapes_tried": len(res), "bytes": nb,
            "all_us": {f"{gr}x{bl}x{un}": round(u, 3) for (u, gr, bl, un) in res}}


def measure_gemv(g: Gpu, t, N, K, M, steps, warmup, seed=0, read_ceiling=False, ceiling_shapes=None):
    """Time quantize+GEMV steps over rotating weight copies; time the GEMV
    kernel alone with HIP events. Returns a dict of figures."""
    torch = g.torch
    w = synth_weights(t, K, N, seed=seed + N + K)
    x = synth_x(M, K, seed=seed + 1)
    ws_list = g.copies(w)
    ncp = len(ws_list)
    xd = torch.from_numpy(x).to(g.dev)
    y = torch.empty(M * N, dtype=torch.float32, device=g.dev)
    nbws = int(g.L.lp_act_workspace_bytes(M, K))
    ws = torch.empty(nbws, dtype=torch.uint8, device=g.dev)
    alg_bytes = w.nbytes + 4 * M * K + 4 * M * N
    # the library's fused M = 1 path (gemv_fused_supported): one launch that
    # quantizes x itself
    fused = (t in (Q4_K, Q4_0, Q8_0) and M == 1 and K % 256 == 0 and K // 256 <= 64
             and not (t in (Q4_K, Q8_0) and K >= 12288))

    def step(i):
        g.check(g.L.lp_gemm_dev(xd.data_ptr(), ws_list[i % ncp].data_ptr(), t, y.data_ptr(),
                                M, K, N, ws.data_ptr(), nbws, g.stream()), "lp_gemm_dev")

    def gemv_only(i):
        # the kernel that computes y in a step: for Q4_K at M = 1 the step is
        # one launch (the GEMV quantizes x itself); otherwise the GEMV on the
        # step's quantized activations
        if fused or t in FACT_TYPES:
            step(i)
        else:
            g.check(g.L.lp_gemm_q_dev(ws.data_ptr(), ws_list[i % ncp].data_ptr(), t, y.data_ptr(),
                                      M, K, N, g.stream()), "lp_gemm_q_dev")

    # eager reference result for the graph check
    step(ncp - 1)
    torch.cuda.synchronize()
    y_eager = y.clone()

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(2):
            step(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(ncp):
            step(i)
    # the headline window runs exactly `steps` steps: whole replays of the
    # ncp-step graph plus one graph of the remaining steps
    full, rest = divmod(steps, ncp)
    grest = None
    if rest:
        grest = torch.cuda.CUDAGraph()
        with torch.cuda.graph(grest):
            for i in range(rest):
                step(i)
    gk = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gk):
        for i in range(ncp):
            gemv_only(i)

    wreps = max(1, -(-warmup // ncp))
    for _ in range(wreps):
        graph.replay()
    torch.cuda.synchronize()
    # every replay of the graph reproduces the eager result
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(y, y_eager), "graph replay differs from eager result"

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(full):
        graph.replay()
    if grest is not None:
        grest.replay()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    nsteps = steps
    ms_step = wall * 1e3 / nsteps

    # GEMV kernel alone: HIP events on the launch stream around graph
    # replays, at least KERNEL_MIN_LAUNCHES back-to-back launches
    kreps = max(1, -(-max(steps, KERNEL_MIN_LAUNCHES) // ncp))
    for _ in range(wreps):
        gk.replay()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(kreps):
        gk.replay()
    ev1.record()
    torch.cuda.synchronize()
    us_kernel = ev0.elapsed_time(ev1) * 1e3 / (kreps * ncp)
    kernel_launches = kreps * ncp

    ceiling = None
    if read_ceiling:
        ceiling = measure_read_ceiling(g, ws_list, int(w.nbytes), kreps, wreps, ceiling_shapes)

    return {
        "read_ceiling": ceiling,
        "type": TNAME[t], "N": N, "K": K, "M": M,
        "alg_bytes": alg_bytes, "weight_bytes": int(w.nbytes),
        "copies": ncp, "rotation_bytes": int(w.nbytes) * ncp,
        "steps": nsteps, "ms_per_step": ms_step,
        "gbs_step": alg_bytes / (ms_step * 1e-3) / 1e9,
        "us_gemv": us_kernel, "kernel_launches": kernel_launches,
        "gbs_gemv": alg_bytes / (us_kernel * 1e-6) / 1e9,
        "w_host": w, "x_host": x, "fused": fused,
        # the kernel the library routes this shape to (lp_gemm_route)
        "route": g.L.lp_gemm_route(t, M, K, N, ws_list[0].data_ptr()).decode(),
    }


def measure_gemm(g: Gpu, N, K, M, reps=20, copies=2, seed=0):
    """Prefill GEMM (Q4_K, M tokens): one step = quantize x + fp16 planes +
    MFMA GEMM. Timed with HIP events over graph replays on the launch stream.
    Weight copies rotate (the weights are re-read per token tile anyway)."""
    torch = g.torch
    t = Q4_K
    w = synth_weights(t, K, N, seed=seed + N + K)
    x = synth_x(M, K, seed=seed + 2, outliers=0.01)
    ws_list = g.copies(w, min_bytes=0, min_copies=copies)
    ncp = len(ws_list)
    xd = torch.from_numpy(x).to(g.dev)
    y = torch.empty(M * N, dtype=torch.float32, device=g.dev)
    nbws = int(g.L.lp_act_workspace_bytes(M, K))
    ws = torch.empty(nbws, dtype=torch.uint8, device=g.dev)

    def step(i):
        g.check(g.L.lp_gemm_dev(xd.data_ptr(), ws_list[i % ncp].data_ptr(), t, y.data_ptr(),
                                M, K, N, ws.data_ptr(), nbws, g.stream()), "lp_gemm_dev")

    step(0)
    torch.cuda.synchronize()
    y0 = y.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(1)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(ncp):
            step(i)
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(y, y0) or ncp > 1, "graph replay differs from eager result"
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(reps):
        graph.replay()
    ev1.record()
    torch.cuda.synchronize()
    us = ev0.elapsed_time(ev1) * 1e3 / (reps * ncp)
    ops = 2.0 * M * N * K
    return {"workload": f"Q4_K prefill GEMM N={N} K={K} M={M}", "us_step": round(us, 2),
            "tops": round(ops / (us * 1e-6) / 1e12, 1),
            "frac_int8_peak": round(ops / (us * 1e-6) / 1e12 / INT8_PEAK_TOPS, 4)}


def measure_moe_ffn(g: Gpu, T, reps=20, copies=2, seed=0):
    """The whole MoE feed-forward layer on the device (lp_moe_ffn_dev) at
    BASELINE.json config 5's shapes: F32 router 128 x 2048, 128 Q4_K experts
    (gate_up 1536 x 2048, down 2048 x 768), top-8, T tokens. One step = router
    norm + matmul + softmax/top-k, expert norm, grouped gate/up, GeGLU, grouped
    down, combine; routing comes from the router, so the experts touched are
    the ones the router picks. value = (router + unique-expert weight bytes +
    x + out) / step time."""
    torch = g.torch
    E, topk, H, inter = 128, 8, 2048, 768
    rng = np.random.default_rng(seed + 91)
    router = (rng.standard_normal(E * H) * 0.5).astype(np.float32).view(np.uint8).copy()
    wgu = synth_weights(Q4_K, H, 2 * inter * E, seed=seed + 5)
    wd = synth_weights(Q4_K, inter, H * E, seed=seed + 6)
    gu_list = g.copies(wgu, min_bytes=0, min_copies=copies)
    d_list = g.copies(wd, min_bytes=0, min_copies=copies)
    ncp = len(gu_list)
    rd = torch.from_numpy(router).to(g.dev)
    rs = torch.from_numpy((1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)).to(g.dev)
    pn = torch.from_numpy((1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)).to(g.dev)
    ds = torch.from_numpy((0.5 + rng.random(E)).astype(np.float32)).to(g.dev)
    x = torch.from_numpy((rng.standard_normal((T, H)) * 2.0).astype(np.float32)).to(g.dev)
    out = torch.empty((T, H), dtype=torch.float32, device=g.dev)
    idx = torch.empty((T, topk), dtype=torch.int32, device=g.dev)
    wts = torch.empty((T, topk), dtype=torch.float32, device=g.dev)
    nb = int(g.L.lp_moe_ffn_workspace_bytes(T, H, E, topk, inter, F32))
    ws = torch.empty(nb, dtype=torch.uint8, device=g.dev)

    def step(i):
        g.check(g.L.lp_moe_ffn_dev(x.data_ptr(), T, H, rd.data_ptr(), F32, rs.data_ptr(), pn.data_ptr(), 1e-6,
                                   gu_list[i % ncp].data_ptr(), Q4_K, d_list[i % ncp].data_ptr(), Q4_K,
                                   ds.data_ptr(), E, topk, inter, out.data_ptr(), idx.data_ptr(), wts.data_ptr(),
                                   ws.data_ptr(), nb, g.stream()), "lp_moe_ffn_dev")

    step(0)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(1)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(ncp):
            step(i)
    for _ in range(3):
        graph.replay()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(reps):
        graph.replay()
    ev1.record()
    torch.cuda.synchronize()
    us = ev0.elapsed_time(ev1) * 1e3 / (reps * ncp)
    uniq = len(np.unique(idx.cpu().numpy()))
    wbytes = router.nbytes + uniq * (row_bytes(Q4_K, H) * 2 * inter + row_bytes(Q4_K, inter) * H)
    alg = wbytes + 8 * T * H
    return {"workload": f"MoE feed-forward layer (lp_moe_ffn_dev): F32 router 128x2048, 128 Q4_K experts "
                        f"(gate_up 1536x2048, down 2048x768), top-8, T={T}",
            "unique_experts": uniq, "alg_bytes": int(alg), "us_step": round(us, 2),
            "gbs": round(alg / (us * 1e-6) / 1e9, 1),
            "hbm_frac": round(alg / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


def measure_moe(g: Gpu, T=64, reps=20, copies=2, seed=0):
    """MoE layer dispatch: 128 Q4_K experts, T
    tokens (64 in the config), top-8 routing (distinct experts per token,
    uniform). One step = grouped gate/up (N=1536, K=2048, one activation row
    per token) + grouped down (N=2048, K=768, one activation row per pair),
    each with its quantization and routing. Layer copies rotate so every step
    streams its experts from HBM. value = (unique-expert weight bytes + x + y
    bytes) / step time. At T >= 128 (>= 8 pairs per expert) the groups run on
    the int8 MFMA kernel."""
    torch = g.torch
    t, E, topk = Q4_K, 128, 8
    P = T * topk
    Ngu, Kgu, Nd, Kd = 1536, 2048, 2048, 768
    rng = np.random.default_rng(seed + 77)
    idx = np.stack([rng.choice(E, topk, replace=False) for _ in range(T)]).astype(np.int32)
    wgu = synth_weights(t, Kgu, Ngu * E, seed=seed + 5)
    wd = synth_weights(t, Kd, Nd * E, seed=seed + 6)
    gu_list = g.copies(wgu, min_bytes=0, min_copies=copies)
    d_list = g.copies(wd, min_bytes=0, min_copies=copies)
    ncp = len(gu_list)
    xgu = torch.from_numpy(synth_x(T, Kgu, seed + 7)).to(g.dev)
    xdn = torch.from_numpy(synth_x(P, Kd, seed + 8)).to(g.dev)
    ygu = torch.empty(P * Ngu, dtype=torch.float32, device=g.dev)
    ydn = torch.empty(P * Nd, dtype=torch.float32, device=g.dev)
    idd = torch.from_numpy(idx).to(g.dev)
    nb1 = int(g.L.lp_moe_workspace_bytes(T, topk, E, Kgu, 0))
    nb2 = int(g.L.lp_moe_workspace_bytes(T, topk, E, Kd, 1))
    ws1 = torch.empty(nb1, dtype=torch.uint8, device=g.dev)
    ws2 = torch.empty(nb2, dtype=torch.uint8, device=g.dev)

    def step(i):
        g.check(g.L.lp_moe_grouped_dev(xgu.data_ptr(), 0, idd.data_ptr(), gu_list[i % ncp].data_ptr(), t,
                                       ygu.data_ptr(), T, topk, E, Kgu, Ngu, ws1.data_ptr(), nb1,
                                       g.stream()), "moe gate_up")
        g.check(g.L.lp_moe_grouped_dev(xdn.data_ptr(), 1, idd.data_ptr(), d_list[i % ncp].data_ptr(), t,
                                       ydn.data_ptr(), T, topk, E, Kd, Nd, ws2.data_ptr(), nb2,
                                       g.stream()), "moe down")

    step(0)
    torch.cuda.synchronize()
    y0 = (ygu.clone(), ydn.clone())
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(1)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(ncp):
            step(i)
    graph.replay()
    torch.cuda.synchronize()
    if ncp == 1:
        assert torch.equal(ygu, y0[0]) and torch.equal(ydn, y0[1]), "graph replay differs"
    for _ in range(3):
        graph.replay()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(reps):
        graph.replay()
    ev1.record()
    torch.cuda.synchronize()
    us = ev0.elapsed_time(ev1) * 1e3 / (reps * ncp)
    uniq = len(np.unique(idx))
    wbytes = uniq * (row_bytes(t, Kgu) * Ngu + row_bytes(t, Kd) * Nd)
    alg = wbytes + 4 * (T * Kgu + P * Kd) + 4 * P * (Ngu + Nd)
    per_pair = P * (row_bytes(t, Kgu) * Ngu + row_bytes(t, Kd) * Nd)
    return {"workload": f"Q4_K MoE layer: 128 experts, {T} tokens, top-8; gate_up 1536x2048 + "
                        "down 2048x768 (grouped by expert)",
            "unique_experts": uniq, "alg_bytes": int(alg), "us_step": round(us, 2),
            "gbs": round(alg / (us * 1e-6) / 1e9, 1),
            "hbm_frac": round(alg / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "per_pair_bytes_reference": int(per_pair)}


def _graph_us(g: Gpu, fn, reps=50, inner=8):
    """Average microseconds of fn() over graph replays of `inner` calls."""
    torch = g.torch
    fn()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(inner):
            fn()
    for _ in range(3):
        graph.replay()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(reps):
        graph.replay()
    ev1.record()
    torch.cuda.synchronize()
    return ev0.elapsed_time(ev1) * 1e3 / (reps * inner)


def measure_aux(g: Gpu):
    """The quantizer at prefill size (quantize_act_q8_neon over M 2048 x K
    4096: 33.5 MB of fp32 read, 8.9 MB of blocks written) and dequantize of a
    Q4_K 14336 x 4096 weight to fp32 (33 MB read, 235 MB written): both
    HBM-bound, value = bytes moved / time."""
    torch = g.torch
    out = []
    M, K = 2048, 4096
    x = torch.from_numpy(synth_x(M, K, 3)).to(g.dev)
    nb = int(g.L.lp_act_workspace_bytes(M, K))
    ws = torch.empty(nb, dtype=torch.uint8, device=g.dev)
    us = _graph_us(g, lambda: g.check(g.L.lp_quantize_act_dev(x.data_ptr(), M, K, ws.data_ptr(), nb, g.stream()),
                                      "quantize"))
    byt = 4 * M * K + M * K + M * (K // 32) * 16
    out.append({"workload": "ActQ8 quantizer M=2048 K=4096", "us": round(us, 2),
                "gbs": round(byt / (us * 1e-6) / 1e9, 1), "hbm_frac": round(byt / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
    N, K = 14336, 4096
    w = torch.from_numpy(synth_weights(Q4_K, K, N, 4)).to(g.dev)
    dst = torch.empty(N * K, dtype=torch.float32, device=g.dev)
    us = _graph_us(g, lambda: g.check(g.L.lp_dequantize_dev(w.data_ptr(), Q4_K, dst.data_ptr(), N * K, g.stream()),
                                      "dequantize"), reps=20, inner=4)
    byt = w.numel() + 4 * N * K
    out.append({"workload": "dequantize Q4_K 14336x4096 -> fp32", "us": round(us, 2),
                "gbs": round(byt / (us * 1e-6) / 1e9, 1), "hbm_frac": round(byt / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
    return out


def measure_batch(g: Gpu, copies=8):
    """matmul_gemm_batch at Llama-3-8B decode shapes (Q4_K, K 4096): Q/K/V
    (4096 + 1024 + 1024 rows) and gate/up (2 x 14336 rows), each a batch of
    specs sharing one x. One lp_gemm_batch_dev call (one launch per batch)
    against the same specs as separate lp_gemm_dev calls. Weight copies
    rotate so every launch streams from HBM. value = weight bytes + x + y per
    step / step time."""
    from laplace_amd._lib import BatchSpec
    torch = g.torch
    K = 4096
    x = torch.from_numpy(synth_x(1, K, 17)).to(g.dev)
    out = []
    for name, Ns in (("Q/K/V 4096+1024+1024", (4096, 1024, 1024)), ("gate/up 2x14336", (14336, 14336))):
        mats = [[torch.from_numpy(synth_weights(Q4_K, K, N, 60 + i)).to(g.dev) for N in Ns] for i in range(copies)]
        ys = [torch.empty(N, dtype=torch.float32, device=g.dev) for N in Ns]
        arrs = []
        for c in range(copies):
            arr = (BatchSpec * len(Ns))()
            for i, N in enumerate(Ns):
                arr[i] = BatchSpec(x.data_ptr(), mats[c][i].data_ptr(), Q4_K, ys[i].data_ptr(), K, N)
            arrs.append(arr)
        nb = int(g.L.lp_gemm_batch_workspace_bytes(arrs[0], len(Ns)))
        ws = torch.empty(nb, dtype=torch.uint8, device=g.dev)
        state = {"i": 0}

        def batched():
            c = state["i"] % copies
            state["i"] += 1
            g.check(g.L.lp_gemm_batch_dev(arrs[c], len(Ns), ws.data_ptr(), nb, g.stream()), "batch")

        def separate():
            c = state["i"] % copies
            state["i"] += 1
            for i, N in enumerate(Ns):
                g.check(g.L.lp_gemm_dev(x.data_ptr(), mats[c][i].data_ptr(), Q4_K, ys[i].data_ptr(), 1, K, N,
                                        ws.data_ptr(), nb, g.stream()), "gemm")

        us_b = _graph_us(g, batched, reps=40, inner=copies)
        us_s = _graph_us(g, separate, reps=40, inner=copies)
        byt = sum(row_bytes(Q4_K, K) * N + 4 * N for N in Ns) + 4 * K
        out.append({"workload": f"matmul_gemm_batch Q4_K {name}, K=4096", "us_batch": round(us_b, 2),
                    "us_separate": round(us_s, 2), "gbs_batch": round(byt / (us_b * 1e-6) / 1e9, 1),
                    "hbm_frac_batch": round(byt / (us_b * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
        del mats
        torch.cuda.empty_cache()
    return out


def measure_host_api(g: Gpu, w, x, t, N, K, reps=200):
    """The drop-in host-pointer entry (lp_gemm, the gemm_fn contract):
    weights registered once (device-resident), x and y staged over PCIe
    through pinned buffers, synchronous return. Median wall time per call."""
    M = x.shape[0]
    y = np.zeros((M, N), np.float32)
    g.check(g.L.lp_register_weights(w.ctypes.data, w.nbytes), "lp_register_weights")
    times = []
    for i in range(reps + 10):
        t0 = time.perf_counter()
        ok = g.L.lp_gemm(x.ctypes.data, w.ctypes.data, t, y.ctypes.data, M, K, N)
        dt = time.perf_counter() - t0
        assert ok, "lp_gemm failed"
        if i >= 10:
            times.append(dt)
    g.L.lp_release_weights()
    med = statistics.median(times)
    alg = w.nbytes + 4 * M * K + 4 * M * N
    return {"us_per_call": round(med * 1e6, 2), "gbs": round(alg / med / 1e9, 1),
            "note": "host x/y over PCIe, registered device weights, synchronous (lp_gemm)"}


def device_info(g: Gpu):
    """The box's own figures next to the published peaks the roofline uses:
    CU count, peak shader and memory clocks, memory bus width, and the
    peaks they imply (HBM3E: 4 transfers per reported memory clock over the
    bus, which gives the published 8 TB/s at 2000 MHz x 8192 bits; int8
    MFMA: 4 SIMDs x 2048 int8 ops per clock per CU on gfx950)."""
    v = [C.c_int(0) for _ in range(4)]
    g.L.lp_device_info(*[C.byref(x) for x in v])
    cus, clk, mclk, bus = (x.value for x in v)
    torch = g.torch
    return {"name": torch.cuda.get_device_properties(0).name, "cus": cus,
            "shader_clock_mhz": round(clk / 1e3, 1), "memory_clock_mhz": round(mclk / 1e3, 1),
            "memory_bus_bits": bus,
            "hbm_peak_from_clocks_gbs": round(4 * mclk * 1e3 * bus / 8 / 1e9, 1),
            "int8_peak_from_clock_tops": round(cus * 4 * 2048 * clk * 1e3 / 1e12, 1),
            "peaks_used": {"hbm_gbs": HBM_PEAK_GBS, "int8_tops": INT8_PEAK_TOPS}}


def host_cores():
    """Threads for the CPU baseline: every core this process may run on.
    The count is the CPU affinity set, lowered to the cgroup CPU quota when
    one is set (cpu.max), since threads past the quota only time-slice."""
    aff = len(os.sched_getaffinity(0))
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, p = f.read().split()[:2]
        if q != "max":
            quota = max(1, int(int(q) // int(p)))
    except (OSError, ValueError):
        pass
    n = min(aff, quota) if quota else aff
    note = f"affinity set {aff} cores" + (f", cgroup quota {quota} cores" if quota else ", no cgroup quota")
    return n, note


def cpu_baseline(t, w, x, N, K, budget_s=12.0):
    """Scalar fp32 path of the reference on the host, whole matrix."""
    from oracle import oracle as orc
    orc.build()
    threads, cores_note = host_cores()
    M = x.shape[0]
    alg = w.nbytes + 4 * M * K + 4 * M * N
    res = {}
    for nth in (threads, 1):
        times = []
        t_end = time.perf_counter() + budget_s / 2
        while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 50):
            t0 = time.perf_counter()
            orc.gemm_scalar(t, x, w, N, nthreads=nth)
            times.append(time.perf_counter() - t0)
        res[nth] = (statistics.median(times), len(times))
    med, runs = res[threads]
    med1, runs1 = res[1]
    return {
        "value": alg / med / 1e9, "unit": "GB/s", "cores": threads, "cores_note": cores_note,
        "kind": "port",
        "sample": f"{TNAME[t]} {N}x{K} M={M} whole matrix, gemm_scalar (src/matmul.cpp:320-334) "
                  f"restated in oracle/lp_oracle.c, median of {runs} runs",
        "value_1thread": alg / med1 / 1e9, "runs_1thread": runs1,
    }


def cpu_baseline_gemm(N, K, M, budget_s=15.0):
    """Scalar fp32 path of the reference for the prefill GEMM
    (gemm_scalar<dot_row_q4_k>, src/matmul.cpp:137-167, :320-353, as restated
    in oracle/liboracle.so) on the host cores: all M tokens against a sample
    of the weight rows, sized from a short calibration run to about
    budget_s seconds; ops = 2*M*rows*K over the timed run."""
    from oracle import oracle as orc
    orc.build()
    threads, cores_note = host_cores()
    w_all = synth_weights(Q4_K, K, N, seed=N + K)
    x = synth_x(M, K, seed=2, outliers=0.01)
    rb = row_bytes(Q4_K, K)

    def run(n):
        w = np.ascontiguousarray(w_all[: n * rb])
        t0 = time.perf_counter()
        orc.gemm_scalar(Q4_K, x, w, n, nthreads=threads)
        return time.perf_counter() - t0

    n0 = max(threads, 8)
    t0 = run(n0)
    n = int(min(N, max(n0, n0 * budget_s / max(t0, 1e-3))))
    n = max(threads, n - n % threads)
    dt = run(n)
    ops = 2.0 * M * n * K
    return {"value": round(ops / dt / 1e12, 6), "unit": "TOPS", "cores": threads,
            "cores_note": cores_note, "kind": "port",
            "sample": f"Q4_K gemm_scalar (src/matmul.cpp:320-353) restated in oracle/lp_oracle.c: "
                      f"all {M} tokens x K {K} against the first {n} of {N} weight rows, one run "
                      f"of {dt:.1f} s"}


def load_traffic(name):
    path = os.path.join(ROOT, "profiles", f"{name}_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("traffic_bytes_per_launch")


GEMM_SWEEP = [(n, 4096, m) for n in (2048, 4096, 8192, 14336) for m in (128, 256, 512, 1024, 2048)] + \
    [(4096, 14336, 512), (4096, 14336, 2048)]
GEMM_KERNELS = {0: "by shape", 1: "split-precision, row-major planes", 2: "fragment-order planes", 3: "int8 MFMA",
                4: "wide-token, 128 x 256 tiles", 5: "wide-token, 256 x 256 tiles"}


def gemm_sweep(g: Gpu, kernels=None, shapes=None):
    """Step time of the Q4_K prefill GEMM (quantize/planes + product) per
    kernel family over GEMM_SWEEP shapes (N, K, M); the routing table of
    lp_gemm comes from these lines."""
    for (n, k, m) in (shapes or GEMM_SWEEP):
        for kern, name in GEMM_KERNELS.items():
            if kernels and kern not in kernels:
                continue
            g.check(g.L.lp_set_gemm_kernel(kern), "lp_set_gemm_kernel")
            r = measure_gemm(g, n, k, m, reps=10)
            print(json.dumps({"kernel": kern, "family": name, **r}), flush=True)
        g.torch.cuda.empty_cache()
    g.check(g.L.lp_set_gemm_kernel(0), "lp_set_gemm_kernel")


def mfma_probe(g: Gpu, iters=20000):
    """Sustained MFMA rate of the prefill GEMM's instruction mix on register
    operands (no memory traffic), 256 workgroups x 8 waves: near-constant
    operands against random ones of the GEMM's value ranges, as a fraction of
    the nominal rate at the spec clock (fp16 2.5 PFLOP/s with the fp8 part at
    twice that; int8 5.0 POPS)."""
    torch = g.torch
    grid = 256
    out = torch.empty(grid * 512, dtype=torch.float32, device=g.dev)
    for kind, name in ((0, "fp16 32x32x16 x16 + fp8 32x32x64 x4 per step"), (1, "int8 32x32x32 x8 per step")):
        for rnd in (0, 1):
            g.check(g.L.lp_mfma_probe_dev(kind, rnd, 100, grid, out.data_ptr(), g.stream()), "probe")
            torch.cuda.synchronize()
            ev0 = torch.cuda.Event(enable_timing=True)
            ev1 = torch.cuda.Event(enable_timing=True)
            ev0.record()
            g.check(g.L.lp_mfma_probe_dev(kind, rnd, iters, grid, out.data_ptr(), g.stream()), "probe")
            ev1.record()
            torch.cuda.synchronize()
            us = ev0.elapsed_time(ev1) * 1e3
            waves = grid * 8
            # nominal cycles per iteration per SIMD (2 waves per SIMD)
            clk = (16 * 32 + 4 * 64) if kind == 0 else 8 * 32
            ideal_us = clk * iters * (waves / 1024) / 2.4e9 * 1e6
            print(json.dumps({"mfma_probe": name, "random_operands": bool(rnd), "us": round(us, 1),
                              "nominal_us_at_2.4GHz": round(ideal_us, 1),
                              "frac_of_nominal": round(ideal_us / us, 4)}), flush=True)
    # co-issue: 32 fp16 products per iteration and wave with NV VALU
    # operations after each; 256 workgroups of 8 waves (two per SIMD) or of 4
    # waves (one per SIMD)
    for kind in range(2, 10):
        nv = (0, 1, 3, 6)[(kind - 2) % 4]
        nw = 8 if kind < 6 else 4
        it = iters // 4
        g.check(g.L.lp_mfma_probe_dev(kind, 0, 100, grid, out.data_ptr(), g.stream()), "probe")
        torch.cuda.synchronize()
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        ev0.record()
        g.check(g.L.lp_mfma_probe_dev(kind, 0, it, grid, out.data_ptr(), g.stream()), "probe")
        ev1.record()
        torch.cuda.synchronize()
        us = ev0.elapsed_time(ev1) * 1e3
        ideal_us = 32 * 32 * it * (grid * nw / 1024) / 2.4e9 * 1e6
        print(json.dumps({"coissue_probe": f"{nv} VALU per fp16 product, {nw // 4} wave(s) per SIMD",
                          "us": round(us, 1), "nominal_us_at_2.4GHz": round(ideal_us, 1),
                          "frac_of_nominal": round(ideal_us / us, 4)}), flush=True)


READ_SWEEP_BYTES = [33_030_144, 49_545_216, 66_060_288, 99_090_432, 132_120_576, 198_180_864,
                    264_241_152, 330_301_440, 415_236_096]


def read_sweep(g: Gpu):
    """Streaming-read time of N bytes by the best lp_read_probe_dev launch
    shape, N from the headline Q4_K weight (14336 x 4096, 33.0 MB) to the
    LM head's (262144 x 2816 Q4_K, 415.2 MB): where the part's read rate
    crosses 70 % of the 8 TB/s spec. Rotating copies (>= 2, >= 512 MiB in
    all) so every launch reads HBM, not the 256 MB Infinity Cache."""
    torch = g.torch
    for nb in READ_SWEEP_BYTES:
        ncp = max(2, -(-ROTATE_MIN_BYTES // nb))
        bufs = [torch.randint(0, 256, (nb,), dtype=torch.uint8, device=g.dev) for _ in range(ncp)]
        reps = max(4, int(400e6 // (nb * ncp)) + 1)
        r = measure_read_ceiling(g, bufs, nb, reps, 2)
        print(json.dumps({"read_sweep_bytes": nb, "copies": ncp, **r}), flush=True)
        del bufs
        torch.cuda.empty_cache()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extra", action="store_true", help="headline workload only")
    ap.add_argument("--no-gemm", action="store_true", help="skip the prefill GEMM lines")
    ap.add_argument("--no-moe", action="store_true", help="skip the MoE dispatch line")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="first run N torch device copies of 256 MiB (a copy kernel of known "
                         "size, to scale rocprofv3 FETCH_SIZE/WRITE_SIZE readings)")
    ap.add_argument("--gemm-sweep", action="store_true",
                    help="only the Q4_K prefill GEMM, every kernel family (lp_set_gemm_kernel 1-3) over "
                         "a grid of shapes, one JSON line each")
    ap.add_argument("--sweep-kernels", default="", help="with --gemm-sweep: comma-separated families")
    ap.add_argument("--sweep-shapes", default="", help="with --gemm-sweep: NxKxM,... instead of the table")
    ap.add_argument("--mfma-probe", action="store_true",
                    help="only the MFMA throughput probe (lp_mfma_probe_dev), near-constant vs random operands")
    ap.add_argument("--read-sweep", action="store_true",
                    help="only the streaming-read ceiling (lp_read_probe_dev) over read sizes "
                         "from the headline weight (33 MB) to the LM head (415 MB), one JSON line each")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(see DESIGN.md for how the GEMV/GEMM/MoE would shard).", file=sys.stderr)
        raise SystemExit(2)

    g = Gpu()
    if args.calib_copy_mib:
        a = g.torch.empty(256 << 20, dtype=g.torch.uint8, device=g.dev)
        b = g.torch.empty_like(a)
        for _ in range(args.calib_copy_mib):
            b.copy_(a)
        g.torch.cuda.synchronize()
        del a, b
    if args.read_sweep:
        read_sweep(g)
        return
    if args.gemm_sweep:
        kern = [int(v) for v in args.sweep_kernels.split(",") if v]
        shp = [tuple(int(v) for v in t.split("x")) for t in args.sweep_shapes.split(",") if t]
        gemm_sweep(g, kern or None, shp or None)
        return
    if args.mfma_probe:
        mfma_probe(g)
        return
    t, N, K, M = Q4_K, 14336, 4096, 1
    r = measure_gemv(g, t, N, K, M, args.steps, args.warmup, read_ceiling=True)
    name = "q4k_gemv_14336x4096_m1"
    achieved = r["gbs_gemv"]
    out = {
        "metric": "Q4_K GEMV GB/s (% HBM peak) + prefill GEMM int8 TOPS (% MFMA peak)",
        "value": round(r["gbs_step"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": r["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "Q4_K decode GEMV, W 14336x4096 (N x K), M=1, fp32 x quantized "
                               "to 32-element int8 blocks in-step",
                   "N": N, "K": K, "M": M, "weight_copies": r["copies"],
                   "rotation_bytes": r["rotation_bytes"], "alg_bytes_per_step": r["alg_bytes"],
                   "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": load_traffic(name),
                     "kernel_launches_timed": r["kernel_launches"],
                     "read_ceiling": r["read_ceiling"],
                     "frac_of_read_ceiling": round(r["read_ceiling"]["us"] / r["us_gemv"], 4),
                     "kernel": "gemv_q4k_sb (quantize fused, one launch per step)" if r["fused"]
                     else "gemv_kernel<Q4_K,M=1>", "us_per_launch": round(r["us_gemv"], 3)},
    }
    out["device"] = device_info(g)
    out["host_api"] = measure_host_api(g, r["w_host"], r["x_host"], t, N, K)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(t, r["w_host"], r["x_host"], N, K)
    extra = []
    if not args.no_extra:
        cfgs = [(Q8_0, 4096, 4096, 1), (Q4_0, 14336, 4096, 1), (Q4_0, 4096, 14336, 1),
                (Q4_K, 18944, 3584, 1), (Q4_K, 18944, 3584, 4), (Q4_K, 18944, 3584, 8),
                (Q6_K, 3584, 18944, 1), (Q6_K, 3584, 18944, 4), (Q6_K, 3584, 18944, 8),
                # LM head, the largest single weight stream (tests/bench_cpu_gpu.cpp:58)
                (Q4_K, 262144, 2816, 1),
                # fp32-activation types (the reference's scalar path): MoE router, FFN
                (F32, 128, 2816, 1), (Q5_K, 14336, 4096, 1), (Q2_K, 14336, 4096, 1),
                (BF16, 4096, 4096, 1)]
        for (tt, n, k, m) in cfgs:
            # weight streams of 16 MB and more: the part's read ceiling for the
            # same bytes in the probe's best shape at these sizes
            big = row_bytes(tt, k) * n >= (16 << 20) if tt in (Q4_0, Q8_0, Q4_K, Q6_K) else False
            e = measure_gemv(g, tt, n, k, m, max(64, args.steps // 4), 16, read_ceiling=big,
                             ceiling_shapes=[(4096, 512, 1)])
            line = {"workload": f"{TNAME[tt]} GEMV {n}x{k} M={m}",
                    "gbs_step": round(e["gbs_step"], 1),
                    "gbs_gemv": round(e["gbs_gemv"], 1),
                    "hbm_frac_gemv": round(e["gbs_gemv"] / HBM_PEAK_GBS, 4),
                    "us_gemv": round(e["us_gemv"], 3), "route": e["route"]}
            if e["read_ceiling"]:
                line["read_ceiling_us"] = e["read_ceiling"]["us"]
                line["frac_of_read_ceiling"] = round(e["read_ceiling"]["us"] / e["us_gemv"], 4)
            extra.append(line)
            g.torch.cuda.empty_cache()
    out["extra"] = extra
    gemms = []
    if not args.no_gemm:
        for (n, k, m) in [(14336, 4096, 2048), (14336, 4096, 512), (4096, 4096, 2048), (4096, 4096, 512)]:
            gemms.append(measure_gemm(g, n, k, m))
            g.torch.cuda.empty_cache()
        head = gemms[0]
        out["gemm"] = {"metric": "prefill GEMM int8-equivalent TOPS (2*M*N*K / step time)",
                       "value": head["tops"], "unit": "TOPS", "workload": head["workload"],
                       "us_per_step": head["us_step"],
                       "roofline": {"bound": "mfma", "achieved": head["tops"],
                                    "peak": INT8_PEAK_TOPS, "unit": "TOPS",
                                    "frac": head["frac_int8_peak"], "traffic": None},
                       "all": gemms}
        if not args.no_cpu:
            out["gemm"]["cpu_baseline"] = cpu_baseline_gemm(14336, 4096, 2048)
    if not args.no_moe:
        out["moe"] = measure_moe(g)
        g.torch.cuda.empty_cache()
        if not args.no_extra:
            out["moe_prefill"] = measure_moe(g, T=256)
            g.torch.cuda.empty_cache()
        out["moe_ffn"] = [measure_moe_ffn(g, T) for T in (1, 64)]
    if not args.no_extra:
        g.torch.cuda.empty_cache()
        out["aux"] = measure_aux(g)
        g.torch.cuda.empty_cache()
        out["batch"] = measure_batch(g)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
