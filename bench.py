#!/usr/bin/env python3
"""Benchmark of the quantized MUL_MAT hot path on one MI355X.

Headline (`value`): Q4_K decode GEMV throughput in GB/s at N = 1 on the
27B-class FFN gate/up shape (17408 x 5120), one step = one
MUL_MAT (activation quantization + GEMV) over one of ~12 distinct weight
copies (>= 2 x the 256 MB Infinity Cache), so the bytes come from HBM.
Algorithmic bytes per step = weight block bytes + K*N*4 (x) + M*N*4 (dst).

Also reported, on the same JSON line:
  roofline      the GEMV kernel's own duration: the median over the timed
                region's launches of a HIP event pair stamped by each
                dispatch on the library's stream (a second pass of the same
                loop), cross-checked by event records placed on the stream
                around each launch -> achieved GB/s against 8 TB/s; HBM
                traffic per launch from the committed rocprofv3 PMC runs
  cpu_baseline  the CPU oracle (a C restatement of ggml-cpu's algorithm,
                kind "port") on the same op on the cores this process may use
                (at most 16, the host share of a one-GPU box), median of its
                reps, with nproc and a single-thread figure
  gemm          prefill MUL_MAT at N = 512: Q4_0 4096x4096, 11008x4096 and
                4096x11008 (config 1), Q4_K 17408x5120, Q6_K 5120x17408 and the
                Q6_K 151936x5120 head (config 2), in TOPS vs the dense int8
                MFMA peak ("secondary" repeats the first); --only adj_gemm:
                IQ4_XS 14336x4096 and Q5_K 17408x5120 at N = 512
  gemv          decode and few-column MUL_MAT of configs 0, 2 and 4: GB/s and
                the kernel's fraction of 8 TB/s
  moe           config 3's whole MoE layer at T = 1, 4, 256 tokens (router,
                gate + up + SwiGLU over 512 Q4_K experts, down, the shared
                expert, the combine), rotated over two layers' expert stacks
                (1.8 GB): GB/s of the expert weights each step touches, against
                the layer's HBM roofline, and each op's own time
  moe_grouped   MUL_MAT_ID with many tokens per expert (16 experts x 1024 tokens
                top-10, 128 experts x 512 tokens top-8; Q4_K 512x2048): op and
                kernel time, TOPS against the int8 peak; and gate + up + SwiGLU
                in one call at 16 x 1024 against the same op on GEMV tasks

    python bench.py [--steps K] [--warmup W] [--gpus 1]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
MALL_BYTES = 256 << 20


def weight_copies(be, qm, synth, qtype, M, K, seed, min_total=2 * MALL_BYTES):
    raw = synth.weights(qtype, M, K, seed)
    ncopy = max(2, -(-min_total // raw.nbytes))
    first = be.new_tensor(qtype, (K, M))
    be.set_tensor(first, raw)
    ws = [first]
    size = qm.alloc_size(qtype, (K, M))
    for _ in range(ncopy - 1):
        t = be.new_tensor(qtype, (K, M))
        be.copy(t.buf, 0, first.buf, 0, size)
        ws.append(t)
    be.synchronize()
    return raw, ws


def run_mul_mat(be, ws, xt, yt, steps):
    for i in range(steps):
        be.mul_mat(ws[i % len(ws)], xt, yt)


def kernel_medians(be, fn, steps):
    """Median main-kernel duration (ms) of `steps` calls of fn(i): stamped by each dispatch,
    then placed as event records on the stream around each launch (two more passes)."""
    out = []
    for markers in (False, True):
        be.kernel_timing(True, markers=markers)
        for i in range(steps):
            fn(i)
        t = be.kernel_times()
        be.kernel_timing(False)
        out.append(float(np.median(t)) if t.size else float("nan"))
    return out


def time_op(be, ws, xt, yt, steps, warmup):
    """Timed region: `steps` ops between a stream synchronize on both sides, uninstrumented
    (value).  Then the kernel's own median duration from two more passes (stamping every
    launch slows the host side, so it stays out of the timed region)."""
    run_mul_mat(be, ws, xt, yt, warmup)
    be.synchronize()
    t0 = time.perf_counter()
    be.timer_begin()
    run_mul_mat(be, ws, xt, yt, steps)
    dev_ms = be.timer_end()
    wall = time.perf_counter() - t0
    k_disp, k_mark = kernel_medians(be, lambda i: be.mul_mat(ws[i % len(ws)], xt, yt), steps)
    return wall, dev_ms, k_disp, k_mark


def graph_replay_us(be, fns, steps, warmup):
    """The same ops replayed from one HIP graph (qmm_capture_begin/end, qmm_graph_launch): the
    callables in fns run once eagerly (which sizes the scratch), then are captured in order into
    one graph, which is replayed (steps / len(fns) launches, at least one) between stream
    synchronizes; microseconds per callable.  The kernels and buffers are the eager ones; only
    the launches differ.  (One graph per op loses on this ROCm: a hipGraphLaunch costs ~18 us of
    host time; a graph of many ops amortizes it.)"""
    for fn in fns:
        fn()
    be.synchronize()
    be.capture_begin()
    for fn in fns:
        fn()
    g = be.capture_end()
    try:
        for _ in range(max(1, warmup // len(fns))):
            be.graph_launch(g)
        be.synchronize()
        reps = max(1, steps // len(fns))
        be.timer_begin()
        for _ in range(reps):
            be.graph_launch(g)
        return be.timer_end() * 1e3 / (reps * len(fns))
    finally:
        g.free()


def kernel_ms(k_disp, k_mark, op_ms):
    """The kernel time a roofline uses: the smaller of the two medians, each of which bounds the
    kernel's own duration from above: the stream markers take in the launch gaps, and in an op of
    two kernels (pre-pass, GEMM) the dispatch stamps at times do too (Q4_K 17408 x 5120 x 512 in
    one process: stamps 138.4 us, markers 115.9, rocprofv3's trace median 121); the op's own time
    per step caps both"""
    vals = [v for v in (k_disp, k_mark) if v == v]
    return min(vals + [op_ms]) if vals else op_ms


def profile_traffic(kernel_tag):
    """HBM bytes per launch of a kernel from the committed rocprofv3 PMC runs
    (FETCH_SIZE and WRITE_SIZE, each scaled by what the counter reads for the
    runtime's copy kernel of known size), or None."""
    p = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        d = json.load(open(p))
        return d[kernel_tag]["traffic_bytes"]
    except (OSError, ValueError, KeyError, TypeError):
        return None


def cpu_baseline(orc, qtype, raw, M, K, x, budget_s):
    """The oracle on the cores this process may use (at most 16) and on one core: median GB/s
    of its reps (at least 5, about budget_s seconds in all)."""
    nproc = os.cpu_count() or 1
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else nproc
    threads = max(1, min(16, avail))
    nbytes = raw.nbytes + K * 4 + M * 4

    def reps(nthreads, budget, at_least):
        orc.mul_mat(qtype, raw, M, K, x, threads=nthreads)    # warm
        times = []
        while len(times) < at_least or sum(times) < budget:
            t0 = time.perf_counter()
            orc.mul_mat(qtype, raw, M, K, x, threads=nthreads)
            times.append(time.perf_counter() - t0)
        return times

    tm = reps(threads, 0.8 * budget_s, 5)
    t1 = reps(1, 0.2 * budget_s, 5)
    med, med1 = float(np.median(tm)), float(np.median(t1))
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "nproc": nproc, "cores_available": avail,
            "single_thread": {"value": round(nbytes / med1 / 1e9, 3), "unit": "GB/s", "cores": 1, "reps": len(t1)},
            "sample": f"Q4_K {M}x{K} N=1 MUL_MAT, median of {len(tm)} reps ({sum(tm):.1f} s) on {threads} threads "
                      f"(nproc {nproc}, {avail} available to the process) with the C oracle (ggml-cpu's algorithm "
                      f"restated in C, -O3 -mavx2; q8_K quantization included); single thread: median of {len(t1)} reps"}


def gemm_case(be, qmm, synth, qtype, M, K, N, name, args, traffic_tag):
    """One prefill MUL_MAT (activation pre-pass + GEMM) over rotated weight
    copies: op TOPS (timed region), GEMM kernel TOPS (median dispatch-stamped
    duration) and its fraction of the dense int8 MFMA peak."""
    raw, ws = weight_copies(be, qmm, synth, qtype, M, K, seed=2)
    x = synth.activations(N, K, seed=3)
    xt = be.new_tensor(qmm.F32, (K, N))
    be.set_tensor(xt, x.view(np.uint8).ravel())
    yt = be.new_tensor(qmm.F32, (M, N))
    steps = max(20, args.steps // 10)
    wall, dev, kd, km = time_op(be, ws, xt, yt, steps, max(2, args.warmup // 4))
    op_ms = wall * 1e3 / steps
    k = kernel_ms(kd, km, op_ms)
    ops = 2.0 * M * N * K
    sec = {"workload": name, "path": be.last_path(),
           "tops": round(ops * steps / wall / 1e12, 3),
           "kernel_tops": round(ops / (k * 1e-3) / 1e12, 3),
           "frac_int8_peak": round(ops / (k * 1e-3) / 1e12 / INT8_PEAK_TOPS, 5),
           "ms_per_op": round(op_ms, 4), "kernel_ms": round(k, 4), "kernel_ms_markers": round(km, 4),
           "traffic": profile_traffic(traffic_tag)}
    for w in ws:
        be.free_buffer(w.buf)
    be.free_buffer(xt.buf)
    be.free_buffer(yt.buf)
    return sec


def gemv_case(be, qmm, synth, qtype, M, K, N, name, args):
    """One decode / few-column MUL_MAT (pre-pass + GEMV) over rotated weight
    copies: GB/s of weight block bytes + activations + dst, for the op (timed
    region) and for the GEMV kernel alone (median dispatch-stamped duration)."""
    raw, ws = weight_copies(be, qmm, synth, qtype, M, K, seed=6)
    x = synth.activations(N, K, seed=7)
    xt = be.new_tensor(qmm.F32, (K, N))
    be.set_tensor(xt, x.view(np.uint8).ravel())
    yt = be.new_tensor(qmm.F32, (M, N))
    steps = max(20, args.steps // 2)
    wall, dev, kd, km = time_op(be, ws, xt, yt, steps, max(4, args.warmup // 2))
    us = wall * 1e6 / steps
    k = kernel_ms(kd, km, us * 1e-3)
    algo = raw.nbytes + K * N * 4 + M * N * 4
    sec = {"workload": name, "path": be.last_path(), "N": N,
           "GBs": round(algo * steps / wall / 1e9, 1), "us_per_op": round(us, 3),
           "kernel_us": round(k * 1e3, 3), "kernel_us_markers": round(km * 1e3, 3),
           "kernel_GBs": round(algo / (k * 1e-3) / 1e9, 1),
           "frac_hbm": round(algo / (k * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    for w in ws:
        be.free_buffer(w.buf)
    be.free_buffer(xt.buf)
    be.free_buffer(yt.buf)
    return sec


def glu_case(be, qmm, synth, args):
    """Config 2's FFN gate/up at decode (17408 x 5120 Q4_K each, N = 1) and its SwiGLU: the
    fused call (one GEMV launch streams both images, then the GLU kernel) against the two
    MUL_MATs alone (one graph: one activation quantization, two GEMV launches, no GLU).
    GB/s counts both matrices' weight bytes."""
    M, K, N = 17408, 5120, 1
    _, wg = weight_copies(be, qmm, synth, qmm.Q4_K, M, K, seed=8)
    _, wu = weight_copies(be, qmm, synth, qmm.Q4_K, M, K, seed=9)
    x = synth.activations(N, K, seed=10)
    xt = be.new_tensor(qmm.F32, (K, N))
    be.set_tensor(xt, x.view(np.uint8).ravel())
    yt = be.new_tensor(qmm.F32, (M, N))
    yu = be.new_tensor(qmm.F32, (M, N))
    steps = max(20, args.steps // 2)
    nw = len(wg)

    def run(n, fused):
        for i in range(n):
            g, u = wg[i % nw], wu[(i + 1) % nw]
            if fused:
                be.mul_mat_glu(g, u, xt, yt, qmm.GLU_SWIGLU)
            else:
                be.graph_compute([(qmm.OP_MUL_MAT, g, xt, None, yt), (qmm.OP_MUL_MAT, u, xt, None, yu)])

    out = {"workload": "Q4_K FFN gate+up 2 x 17408x5120 N=1 + SwiGLU (config 2)"}
    for fused in (True, False):
        run(max(4, args.warmup // 2), fused)
        be.synchronize()
        t0 = time.perf_counter()
        run(steps, fused)
        be.synchronize()
        out["fused_us" if fused else "two_gemv_us"] = round((time.perf_counter() - t0) * 1e6 / steps, 3)
    run(1, True)
    out["path"] = be.last_path()
    wbytes = 2 * synth.row_bytes(qmm.Q4_K, K) * M
    out["fused_GBs"] = round(wbytes / (out["fused_us"] * 1e-6) / 1e9, 1)
    out["two_gemv_GBs"] = round(wbytes / (out["two_gemv_us"] * 1e-6) / 1e9, 1)
    for w in wg + wu:
        be.free_buffer(w.buf)
    for t in (xt, yt, yu):
        be.free_buffer(t.buf)
    return out


def moe_grouped_glu(be, qmm, synth, ws, xt, it, yt, ids, E, n_used, M, K, T, name, args, steps):
    """MUL_MAT_ID gate + up + SwiGLU in one call (qmm_mul_mat_id_glu), gate and up two of the
    rotated stacks: the op's time on its default path (the grouped GEMM past 32 pairs per expert)
    and on the 8-pair GEMV tasks (QMM_MOE_GEMM_MIN=0); TOPS = 2 products x 2 x pairs x M x K over
    the op's time."""
    def run(n):
        t0 = time.perf_counter()
        for i in range(n):
            be.mul_mat_id_glu(ws[i % len(ws)], ws[(i + 1) % len(ws)], xt, it, yt, qmm.GLU_SWIGLU)
        be.synchronize()
        return (time.perf_counter() - t0) / max(n, 1)
    run(args.warmup)
    op_s = run(steps)
    path = be.last_path()
    os.environ["QMM_MOE_GEMM_MIN"] = "0"
    try:
        run(args.warmup)
        tasks_s = run(steps)
        tasks_path = be.last_path()
    finally:
        del os.environ["QMM_MOE_GEMM_MIN"]
    ops = 2.0 * 2.0 * T * n_used * M * K
    for w in ws:
        be.free_buffer(w.buf)
    for t in (xt, it, yt):
        be.free_buffer(t.buf)
    return {"workload": name, "path": path, "experts": E, "tokens": T, "n_used": n_used, "M": M, "K": K,
            "op_us": round(op_s * 1e6, 2), "op_tops": round(ops / op_s / 1e12, 1),
            "gemv_tasks_op_us": round(tasks_s * 1e6, 2), "gemv_tasks_path": tasks_path}


def moe_grouped_case(be, qmm, synth, E, n_used, M, K, T, name, args, glu=False):
    """MUL_MAT_ID with many tokens per expert (Q4_K experts [K, M, E], src1 [K, 1, T], top-n_used
    of softmaxed random logits): one step = one op over one of several copies of the stack
    (>= 2 x the MALL).  TOPS = 2 x pairs x M x K over the main kernel's median; GB/s counts the
    touched expert bytes, the f32 activations and dst over the op's own time."""
    raw, ws = weight_copies(be, qmm, synth, qmm.Q4_K, M * E, K, seed=21)
    ws = [qmm.Tensor(w.buf, qmm.Q4_K, (K, M, E)) for w in ws]
    ids = synth.moe_ids(T, E, n_used, seed=22)
    x = synth.activations(T, K, seed=23)
    xt = be.new_tensor(qmm.F32, (K, 1, T))
    be.set_tensor(xt, x.view(np.uint8).ravel())
    it = be.new_tensor(qmm.I32, (n_used, T))
    be.set_tensor(it, ids.view(np.uint8).ravel())
    yt = be.new_tensor(qmm.F32, (M, n_used, T))
    steps = max(10, args.steps // 4)
    if glu:
        return moe_grouped_glu(be, qmm, synth, ws, xt, it, yt, ids, E, n_used, M, K, T, name, args, steps)
    for i in range(args.warmup):
        be.mul_mat_id(ws[i % len(ws)], xt, it, yt)
    be.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        be.mul_mat_id(ws[i % len(ws)], xt, it, yt)
    be.synchronize()
    op_s = (time.perf_counter() - t0) / steps
    path = be.last_path()
    be.kernel_timing(True)
    for i in range(steps):
        be.mul_mat_id(ws[i % len(ws)], xt, it, yt)
    be.synchronize()
    kt = be.kernel_times()
    be.kernel_timing(False)
    k_ms = float(np.median(kt)) if kt.size else float("nan")
    ops = 2.0 * T * n_used * M * K
    touched = len(np.unique(ids)) * synth.row_bytes(qmm.Q4_K, K) * M
    moved = touched + T * K * 4 + T * n_used * M * 4
    for w in ws:
        be.free_buffer(w.buf)
    for t in (xt, it, yt):
        be.free_buffer(t.buf)
    return {"workload": name, "path": path, "experts": E, "tokens": T, "n_used": n_used, "M": M, "K": K,
            "op_us": round(op_s * 1e6, 2), "kernel_us": round(k_ms * 1e3, 2),
            "kernel_tops": round(ops / (k_ms * 1e-3) / 1e12, 1), "frac_int8_peak": round(ops / (k_ms * 1e-3) / 1e12 / INT8_PEAK_TOPS, 4),
            "GBs": round(moved / op_s / 1e9, 1)}


class MoeLayers:
    """Config 3's MoE layer, `nl` copies: per layer the gate and up expert stacks [2048, 512, 512]
    and the down stack [512, 2048, 512] in Q4_K (906 MB), the shared expert's gate / up
    [2048, 512] and down [512, 2048], and the buffers of one layer's chain.  The layers' stacks
    hold the same bytes (device copies of one seeded stack per shape)."""
    E, K_USED, HID, FFN = 512, 10, 2048, 512

    def __init__(self, be, qmm, synth, nl):
        self.be, self.qmm, self.nl = be, qmm, nl
        E, HID, FFN = self.E, self.HID, self.FFN
        q = qmm.Q4_K
        self.ebytes = synth.row_bytes(q, HID) * FFN                # one expert matrix: 589,824 B
        self.bufs = []
        proto = {}
        for name, (rows, k, ne, seed) in {"gate": (E * FFN, HID, (HID, FFN, E), 11), "down": (E * HID, FFN, (FFN, HID, E), 13),
                                          "sgate": (FFN, HID, (HID, FFN), 14), "sdown": (HID, FFN, (FFN, HID), 16)}.items():
            t = be.new_tensor(q, ne)
            be.set_tensor(t, synth.weights(q, rows, k, seed))
            proto[name] = t
        self.layers = []
        for _ in range(nl):
            L = {}
            for name, src in (("gate", "gate"), ("up", "gate"), ("down", "down"), ("sgate", "sgate"), ("sup", "sgate"),
                              ("sdown", "sdown")):
                t = be.new_tensor(q, proto[src].ne)
                be.copy(t.buf, 0, proto[src].buf, 0, qmm.alloc_size(q, proto[src].ne))
                L[name] = t
                self.bufs.append(t.buf)
            self.layers.append(L)
        for t in proto.values():
            be.free_buffer(t.buf)
        be.synchronize()

    def close(self):
        for b in self.bufs:
            self.be.free_buffer(b)


def moe_case(be, qmm, synth, layers, T, args):
    """Config 3's whole MoE layer at T tokens, one step = one layer: the router (softmax /
    top-10 over 512 logits per token), gate + up + SwiGLU over the routed experts (one call),
    the down projection (src1 [512, 10, T]), the shared expert's gate + up + SwiGLU and down,
    and the combine with the sigmoid-gated shared expert.  Steps alternate between the layers
    and take the next of 32 router-logit sets, so the stacks (1.8 GB) rotate through HBM.  GB/s
    counts the expert weights each step touches (distinct routed experts x 3 matrices + the
    shared expert), the bytes BASELINE.md's C3 row quotes."""
    qm = qmm
    be_ = be
    E, k, HID, FFN = layers.E, layers.K_USED, layers.HID, layers.FFN
    g = np.random.default_rng(1000 + T)
    nlog = 32
    logits = [g.standard_normal((T, E)).astype(np.float32) for _ in range(nlog)]
    lts = []
    touched = []
    for lg in logits:
        t = be_.new_tensor(qm.F32, (E, T))
        be_.set_tensor(t, lg.view(np.uint8).ravel())
        lts.append(t)
        top = np.argpartition(-lg, k - 1, axis=1)[:, :k]          # the k largest logits of each token
        touched.append((len(np.unique(top)) * 3 + 3) * layers.ebytes)
    x = synth.activations(T, HID, seed=5)
    xt = be_.new_tensor(qm.F32, (HID, 1, T))
    be_.set_tensor(xt, x.view(np.uint8).ravel())
    x2 = qm.Tensor(xt.buf, qm.F32, (HID, T))
    sgl = be_.new_tensor(qm.F32, (1, T))
    be_.set_tensor(sgl, g.standard_normal(T).astype(np.float32).view(np.uint8))
    ids = be_.new_tensor(qm.I32, (k, T))
    wts = be_.new_tensor(qm.F32, (k, T))
    h = be_.new_tensor(qm.F32, (FFN, k, T))
    ex = be_.new_tensor(qm.F32, (HID, k, T))
    hs = be_.new_tensor(qm.F32, (FFN, T))
    ys = be_.new_tensor(qm.F32, (HID, T))
    out = be_.new_tensor(qm.F32, (HID, T))
    tmp = [lts, [xt, sgl, ids, wts, h, ex, hs, ys, out]]
    nl = len(layers.layers)

    def router(i):
        be_.moe_topk(lts[i % nlog], ids, wts)

    def gate_up(i):
        L = layers.layers[i % nl]
        be_.mul_mat_id_glu(L["gate"], L["up"], xt, ids, h, qm.GLU_SWIGLU)

    def down(i):
        be_.mul_mat_id(layers.layers[i % nl]["down"], h, ids, ex)

    def shared(i):
        L = layers.layers[i % nl]
        be_.mul_mat_glu(L["sgate"], L["sup"], x2, hs, qm.GLU_SWIGLU)
        be_.mul_mat(L["sdown"], hs, ys)

    def combine(i):
        be_.moe_combine(ex, wts, out, ys, sgl)

    def layer(i):
        router(i)
        gate_up(i)
        down(i)
        shared(i)
        combine(i)

    steps = max(32, args.steps // 2)
    for i in range(16):
        layer(i)
    be_.synchronize()
    t0 = time.perf_counter()
    be_.timer_begin()
    for i in range(steps):
        layer(i)
    dev_ms = be_.timer_end()
    wall = time.perf_counter() - t0
    paths = {}
    for name, fn in (("gate_up_glu", gate_up), ("down", down)):
        layer(0)
        fn(0)
        paths[name] = be_.last_path()
    times = {}
    for name, fn in (("router", router), ("gate_up_glu", gate_up), ("down", down), ("shared", shared),
                     ("combine", combine)):
        for i in range(8):
            layer(i)
        be_.synchronize()
        be_.timer_begin()
        for i in range(steps):
            fn(i)
        times[name] = be_.timer_end() * 1e3 / steps
    bytes_step = float(np.mean([touched[i % nlog] for i in range(steps)]))
    us = dev_ms * 1e3 / steps
    # the layer from one HIP graph holding the eager rotation's first nlog steps (layer copies and
    # logits sets in turn), so the replays touch the same experts and stacks as the eager steps
    g_us = graph_replay_us(be_, [lambda i=i: layer(i) for i in range(nlog)], steps, 16)
    # the same layer with the expert products, the shared expert and the combine in one call
    # (qmm_moe_ffn: two launches) after the router, where it takes the token count
    def layer_fused(i):
        L = layers.layers[i % nl]
        router(i)
        be_.moe_ffn(L["gate"], L["up"], L["down"], xt, ids, wts, out, shared=(L["sgate"], L["sup"], L["sdown"]),
                    shared_logit=sgl)

    fused = None
    try:
        layer_fused(0)
    except qm.QmmError:                                          # (more tokens than the fused block takes)
        pass
    else:
        fpath = be_.last_path()
        for i in range(16):
            layer_fused(i)
        be_.synchronize()
        be_.timer_begin()
        for i in range(steps):
            layer_fused(i)
        f_us = be_.timer_end() * 1e3 / steps
        be_.timer_begin()
        for i in range(steps):
            be_.moe_ffn(layers.layers[i % nl]["gate"], layers.layers[i % nl]["up"], layers.layers[i % nl]["down"], xt,
                        ids, wts, out, shared=(layers.layers[i % nl]["sgate"], layers.layers[i % nl]["sup"],
                                               layers.layers[i % nl]["sdown"]), shared_logit=sgl)
        ffn_us = be_.timer_end() * 1e3 / steps
        fg_us = graph_replay_us(be_, [lambda i=i: layer_fused(i) for i in range(nlog)], steps, 16)

        # the router inside the gate/up launch: the whole layer in two launches
        def layer_2(i):
            L = layers.layers[i % nl]
            be_.moe_ffn(L["gate"], L["up"], L["down"], xt, ids, wts, out, shared=(L["sgate"], L["sup"], L["sdown"]),
                        shared_logit=sgl, logits=lts[i % nlog])

        for i in range(16):
            layer_2(i)
        be_.synchronize()
        be_.timer_begin()
        for i in range(steps):
            layer_2(i)
        f2_us = be_.timer_end() * 1e3 / steps
        f2g_us = graph_replay_us(be_, [lambda i=i: layer_2(i) for i in range(nlog)], steps, 16)
        fused = {"us_per_layer": round(f2_us, 3), "GBs": round(bytes_step / (f2_us * 1e-6) / 1e9, 1),
                 "frac_hbm": round(bytes_step / (f2_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                 "us_per_layer_graph": round(f2g_us, 3), "path": be_.last_path(),
                 "note": "qmm_moe_ffn with the router's logits: router + gate/up + SwiGLU of the routed pairs and the "
                         "shared expert in one launch, down + router weights + sigmoid-gated shared + slot sum in a "
                         "second"}
        fused["router_outside"] = {"us_per_layer": round(f_us, 3), "GBs": round(bytes_step / (f_us * 1e-6) / 1e9, 1),
                 "frac_hbm": round(bytes_step / (f_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                 "op_us": {"router": round(times["router"], 3), "moe_ffn": round(ffn_us, 3)}, "path": fpath,
                 "us_per_layer_graph": round(fg_us, 3),
                 "note": "router (qmm_moe_topk) + qmm_moe_ffn: three launches"}
    res = {"workload": f"config 3 MoE layer, T={T}: router + gate/up/SwiGLU (512 Q4_K experts, top-10) + down + "
                       f"shared expert + combine, {nl} layers rotated",
           "T": T, "us_per_layer": round(us, 3), "wall_us_per_layer": round(wall * 1e6 / steps, 3),
           "weight_bytes_touched": int(bytes_step), "GBs": round(bytes_step / (us * 1e-6) / 1e9, 1),
           "frac_hbm": round(bytes_step / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
           "roofline_us": round(bytes_step / (HBM_PEAK_GBS * 1e9) * 1e6, 3),
           "op_us": {n: round(v, 3) for n, v in times.items()}, "paths": paths,
           "us_per_layer_graph": round(g_us, 3),
           "GBs_graph": round(bytes_step / (g_us * 1e-6) / 1e9, 1),
           "fused": fused}
    for t in tmp[0] + tmp[1]:
        be_.free_buffer(t.buf)
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--only", default="", help="profile one workload: q4k_gemv, q40_gemm, q4k_gemm, q6k_gemm, adj_gemm, gemv, glu, "
                                                 "moe or moe_grouped")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for {args.gpus}); "
              "MUL_MAT would shard by output rows with no reduction, see DESIGN.md", file=sys.stderr)
        sys.exit(2)

    from arcint_amd import qmm, synth

    be = qmm.Backend(0)
    out = {}
    M, K, N = 17408, 5120, 1
    if args.only in ("", "q4k_gemv"):
        raw, ws = weight_copies(be, qmm, synth, qmm.Q4_K, M, K, seed=0)
        x = synth.activations(N, K, seed=1)
        xt = be.new_tensor(qmm.F32, (K, N))
        be.set_tensor(xt, x.view(np.uint8).ravel())
        yt = be.new_tensor(qmm.F32, (M, N))
        wall, dev_ms, kd, km = time_op(be, ws, xt, yt, args.steps, args.warmup)
        path = be.last_path()
        algo = raw.nbytes + K * N * 4 + M * N * 4
        value = algo * args.steps / wall / 1e9
        k_ms = kernel_ms(kd, km, wall * 1e3 / args.steps)
        achieved = algo / (k_ms * 1e-3) / 1e9
        # one launch (the fused kernel quantizes its own activations, K over 4-wave work-groups)
        # or the q8_K pre-pass and the GEMV
        fused = path == "gemv-fq"
        tag = "q4k_gemv_fq" if fused else "q4k_gemv"
        prof = "profiles/k_gemv_fq_q4k_17408x5120_n1.md" if fused else "profiles/k_gemv_q4k_17408x5120_n1.md"
        kname = ("k_gemv_fq<12, 1> (Q4_K, 1 column, K split over 4-wave work-groups, activations quantized "
                 "in the kernel)" if fused else "k_gemv<12, 1> (Q4_K, 1 column)")
        op_desc = "MUL_MAT in one launch" if fused else "MUL_MAT incl. q8_K pre-pass"
        traffic = profile_traffic(tag)
        out.update({
            "metric": "Q4_K GEMV GB/s (% of 8 TB/s) at N=1; Q4_0 GEMM TOPS (% MFMA peak) at N=512",
            "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(wall * 1e3 / args.steps, 5), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "int8", "data": "synthetic",
            "config": {"workload": f"Q4_K GEMV 17408x5120 N=1 (config 2 ffn gate/up), {op_desc}",
                       "weights": "Q4_K", "M": M, "K": K, "N": N, "weight_copies": len(ws),
                       "rotated_bytes": int(len(ws) * raw.nbytes), "path": path,
                       "device_ms_per_step": round(dev_ms / args.steps, 5)},
            "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                         "traffic_source": f"profiles/traffic.json: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE of this "
                                           f"kernel ({prof}), scaled by the copy kernel's counts; not measured in "
                                           "this run",
                         "kernel": kname, "kernel_us": round(k_ms * 1e3, 3),
                         "kernel_us_markers": round(km * 1e3, 3), "kernel_us_stat": f"median of {args.steps} launches",
                         "algorithmic_bytes": int(algo)},
        })
        # the same ops from one HIP graph: four passes over the weight copies (the value above is
        # the eager op)
        g_us = graph_replay_us(be, [lambda w=w: be.mul_mat(w, xt, yt) for w in ws * 4], args.steps, args.warmup)
        out["graph"] = {"us_per_op": round(g_us, 3), "GBs": round(algo / (g_us * 1e-6) / 1e9, 1),
                        "frac_hbm": round(algo / (g_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                        "note": f"{4 * len(ws)} MUL_MATs ({'one launch each' if fused else 'q8_K pre-pass + GEMV'}, "
                                "the weight copies in turn) captured in one HIP graph and replayed (qmm_graph_launch); "
                                "value is the eager op"}
        if not args.no_cpu:
            import oracle
            out["cpu_baseline"] = cpu_baseline(oracle, qmm.Q4_K, raw, M, K, x, args.cpu_seconds)
        for w in ws:
            be.free_buffer(w.buf)

    if not args.no_secondary and args.only in ("", "q40_gemm", "q4k_gemm", "q6k_gemm", "adj_gemm"):
        cases = [(qmm.Q4_0, 4096, 4096, 512, "Q4_0 GEMM 4096x4096x512 (config 1 attn)", "q40_gemm", "q40_gemm"),
                 (qmm.Q4_0, 11008, 4096, 512, "Q4_0 GEMM 11008x4096x512 (config 1 ffn gate/up)", "q40_gemm",
                  "q40_gemm_11008"),
                 (qmm.Q4_K, 17408, 5120, 512, "Q4_K GEMM 17408x5120x512 (config 2 ffn gate/up)", "q4k_gemm", "q4k_gemm"),
                 (qmm.Q4_0, 4096, 11008, 512, "Q4_0 GEMM 4096x11008x512 (config 1 ffn down)", "q40_gemm",
                  "q40_gemm_down"),
                 (qmm.Q6_K, 5120, 17408, 512, "Q6_K GEMM 5120x17408x512 (config 2 ffn down)", "q6k_gemm", "q6k_gemm"),
                 (qmm.Q6_K, 151936, 5120, 512, "Q6_K GEMM 151936x5120x512 (config 2 output head)", "q6k_gemm",
                  "q6k_gemm_head"),
                 # (the adjacent types at config shapes: --only adj_gemm, not in the default run)
                 (qmm.IQ4_XS, 14336, 4096, 512, "IQ4_XS GEMM 14336x4096x512 (config 4 shape)", "adj_gemm", "iq4xs_gemm"),
                 (qmm.Q5_K, 17408, 5120, 512, "Q5_K GEMM 17408x5120x512 (config 2 shape)", "adj_gemm", "q5k_gemm")]
        secs = []
        for qtype, M2, K2, N2, name, tag, ttag in cases:
            if (args.only and args.only != tag) or (not args.only and tag == "adj_gemm"):
                continue
            secs.append(gemm_case(be, qmm, synth, qtype, M2, K2, N2, name, args, ttag))
        if out:
            out["secondary"] = secs[0]
            out["gemm"] = secs
        else:
            out = {"metric": "GEMM TOPS at N=512", "value": secs[0]["tops"], "unit": "TOPS", "gemm": secs}
    if not args.no_secondary and args.only in ("", "gemv"):
        gcases = [(qmm.Q4_0, 4096, 4096, 1, "Q4_0 GEMV 4096x4096 N=1 (config 0/1)"),
                  (qmm.Q6_K, 5120, 17408, 1, "Q6_K GEMV 5120x17408 N=1 (config 2 ffn down)"),
                  (qmm.Q4_K, 17408, 5120, 4, "Q4_K 17408x5120 N=4 (config 2)"),
                  (qmm.Q4_K, 17408, 5120, 16, "Q4_K 17408x5120 N=16 (config 2, 16-column MFMA task)"),
                  (qmm.Q4_K, 17408, 5120, 32, "Q4_K 17408x5120 N=32 (config 2, 32-column MFMA task)"),
                  (qmm.Q6_K, 5120, 17408, 8, "Q6_K 5120x17408 N=8 (config 2 ffn down, MFMA)"),
                  (qmm.Q6_K, 151936, 5120, 1, "Q6_K GEMV 151936x5120 N=1 (config 2 output head)"),
                  (qmm.Q6_K, 151936, 5120, 4, "Q6_K 151936x5120 N=4 (config 2 output head, MTP verify width)")]
        for qt, nm in ((qmm.IQ4_XS, "IQ4_XS"), (qmm.Q8_0, "Q8_0")):
            for n in (1, 2, 4, 8):
                gcases.append((qt, 14336, 4096, n, f"{nm} 14336x4096 N={n} (config 4)"))
            for n in (1, 8):
                gcases.append((qt, 4096, 14336, n, f"{nm} 4096x14336 N={n} (config 4)"))
        # the adjacent types on config shapes (no reference config quotes them)
        gcases += [(qmm.Q5_K, 17408, 5120, 1, "Q5_K GEMV 17408x5120 N=1 (config 2 shape)"),
                   (qmm.IQ4_NL, 14336, 4096, 1, "IQ4_NL GEMV 14336x4096 N=1 (config 4 shape)"),
                   (qmm.IQ4_NL, 14336, 4096, 8, "IQ4_NL 14336x4096 N=8 (config 4 shape)")]
        gem = [gemv_case(be, qmm, synth, qt, M2, K2, N2, nm, args) for qt, M2, K2, N2, nm in gcases]
        if out:
            out["gemv"] = gem
        else:
            out = {"metric": "GEMV GB/s", "value": gem[0]["GBs"], "unit": "GB/s", "gemv": gem}
    if not args.no_secondary and args.only in ("", "glu"):
        g = glu_case(be, qmm, synth, args)
        if out:
            out["glu"] = g
        else:
            out = {"metric": "FFN gate+up GB/s", "value": g["fused_GBs"], "unit": "GB/s", "glu": g}
    if not args.no_secondary and args.only in ("", "moe"):
        layers = MoeLayers(be, qmm, synth, 2)
        moe = [moe_case(be, qmm, synth, layers, T, args) for T in (1, 4, 256)]
        layers.close()
        if out:
            out["moe"] = moe
        else:
            out = {"metric": "MoE layer GB/s", "value": moe[0]["GBs"], "unit": "GB/s", "moe": moe}
    if not args.no_secondary and args.only in ("", "moe", "moe_grouped"):
        mg = [moe_grouped_case(be, qmm, synth, 16, 10, 512, 2048, 1024,
                               "MUL_MAT_ID 16 Q4_K experts 512x2048, 1024 tokens top-10 (640 pairs per expert)", args),
              moe_grouped_case(be, qmm, synth, 128, 8, 512, 2048, 512,
                               "MUL_MAT_ID 128 Q4_K experts 512x2048, 512 tokens top-8 (32 pairs per expert)", args),
              moe_grouped_case(be, qmm, synth, 16, 10, 512, 2048, 1024,
                               "MUL_MAT_ID gate + up + SwiGLU, 16 Q4_K experts 512x2048, 1024 tokens top-10", args,
                               glu=True)]
        if out:
            out["moe_grouped"] = mg
        else:
            out = {"metric": "grouped MUL_MAT_ID TOPS", "value": mg[0]["kernel_tops"], "unit": "TOPS", "moe_grouped": mg}
    be.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
