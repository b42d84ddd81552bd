#!/usr/bin/env python3
"""Benchmark of the quantized MUL_MAT hot path on one MI355X.

Headline (`value`): Q4_K decode GEMV throughput in GB/s at N = 1 on the
27B-class FFN gate/up shape (17408 x 5120), one step = one
MUL_MAT (activation quantization + GEMV) over one of ~12 distinct weight
copies (>= 2 x the 256 MB Infinity Cache), so the bytes come from HBM.
Algorithmic bytes per step = weight block bytes + K*N*4 (x) + M*N*4 (dst).

Also reported, on the same JSON line:
  roofline      the GEMV kernel's own duration (HIP events around each launch
                on the library's stream, a second pass of the same loop) ->
                achieved GB/s against 8 TB/s, plus HBM traffic per launch
                from profiles/ when the rocprofv3 PMC runs were committed
  cpu_baseline  the CPU oracle (a C restatement of ggml-cpu's algorithm,
                kind "port") on the same op, bounded to ~--cpu-seconds
  gemm          prefill MUL_MAT at N = 512: Q4_0 4096x4096 and 11008x4096
                (config 1), Q4_K 17408x5120 (config 2), in TOPS vs the dense
                int8 MFMA peak ("secondary" repeats the first)
  gemv          decode and few-column MUL_MAT: Q4_0 4096x4096 and Q6_K
                5120x17408 at N = 1, Q4_K 17408x5120 at N = 4, IQ4_XS and Q8_0
                14336x4096 at N = 2, 4, 8 (configs 0, 2, 4): GB/s and the
                kernel's fraction of 8 TB/s
  moe           MUL_MAT_ID on config 3 (512 Q4_K experts, top-10) at T = 1,
                4, 256 tokens: GB/s of the expert weights each step touches; with
                the router (softmax / top-10) and the combine (hidden 2048) per op

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


def time_op(be, ws, xt, yt, steps, warmup):
    """Timed region: `steps` ops between a stream synchronize on both sides,
    uninstrumented (value).  Then the same `steps` ops again with every main
    kernel (GEMV / GEMM) stamping a HIP event pair with its own dispatch start
    and end on the library's stream: the kernel's average duration for the
    roofline (stamping every launch slows the host side, so it stays out of
    the timed region)."""
    run_mul_mat(be, ws, xt, yt, warmup)
    be.synchronize()
    t0 = time.perf_counter()
    be.timer_begin()
    run_mul_mat(be, ws, xt, yt, steps)
    dev_ms = be.timer_end()
    wall = time.perf_counter() - t0
    be.kernel_timing(True)
    run_mul_mat(be, ws, xt, yt, steps)
    k_ms, n = be.kernel_time()
    be.kernel_timing(False)
    return wall, dev_ms, k_ms / max(n, 1)


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
    threads = min(os.cpu_count() or 1, 16)
    nbytes = raw.nbytes + K * 4 + M * 4
    orc.mul_mat(qtype, raw, M, K, x, threads=threads)     # warm
    reps, t0 = 0, time.perf_counter()
    while True:
        orc.mul_mat(qtype, raw, M, K, x, threads=threads)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return {"value": round(nbytes * reps / el / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"Q4_K {M}x{K} N=1 MUL_MAT x{reps} reps ({el:.1f} s, {threads} threads) with the C oracle "
                      f"(ggml-cpu's algorithm restated in C, -O3 -mavx2; q8_K quantization included)"}


def gemm_case(be, qmm, synth, qtype, M, K, N, name, args, traffic_tag):
    """One prefill MUL_MAT (activation pre-pass + GEMM) over rotated weight
    copies: op TOPS (timed region), GEMM kernel TOPS (dispatch-stamped) and
    its fraction of the dense int8 MFMA peak."""
    raw, ws = weight_copies(be, qmm, synth, qtype, M, K, seed=2)
    x = synth.activations(N, K, seed=3)
    xt = be.new_tensor(qmm.F32, (K, N))
    be.set_tensor(xt, x.view(np.uint8).ravel())
    yt = be.new_tensor(qmm.F32, (M, N))
    steps = max(5, args.steps // 10)
    wall, dev, k = time_op(be, ws, xt, yt, steps, max(2, args.warmup // 4))
    ops = 2.0 * M * N * K
    sec = {"workload": name, "path": be.last_path(),
           "tops": round(ops * steps / wall / 1e12, 3),
           "kernel_tops": round(ops / (k * 1e-3) / 1e12, 3),
           "frac_int8_peak": round(ops / (k * 1e-3) / 1e12 / INT8_PEAK_TOPS, 5),
           "ms_per_op": round(wall * 1e3 / steps, 4), "kernel_ms": round(k, 4),
           "traffic": profile_traffic(traffic_tag)}
    for w in ws:
        be.free_buffer(w.buf)
    be.free_buffer(xt.buf)
    be.free_buffer(yt.buf)
    return sec


def gemv_case(be, qmm, synth, qtype, M, K, N, name, args):
    """One decode / few-column MUL_MAT (pre-pass + GEMV) over rotated weight
    copies: GB/s of weight block bytes + activations + dst, for the op (timed
    region) and for the GEMV kernel alone (dispatch-stamped)."""
    raw, ws = weight_copies(be, qmm, synth, qtype, M, K, seed=6)
    x = synth.activations(N, K, seed=7)
    xt = be.new_tensor(qmm.F32, (K, N))
    be.set_tensor(xt, x.view(np.uint8).ravel())
    yt = be.new_tensor(qmm.F32, (M, N))
    steps = max(20, args.steps // 2)
    wall, dev, k = time_op(be, ws, xt, yt, steps, max(4, args.warmup // 2))
    algo = raw.nbytes + K * N * 4 + M * N * 4
    sec = {"workload": name, "path": be.last_path(), "N": N,
           "GBs": round(algo * steps / wall / 1e9, 1), "us_per_op": round(wall * 1e6 / steps, 3),
           "kernel_us": round(k * 1e3, 3), "kernel_GBs": round(algo / (k * 1e-3) / 1e9, 1),
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


def moe_case(be, qmm, synth, T, args):
    """MUL_MAT_ID on config 3's expert gate/up: 512 Q4_K experts of 512 x 2048,
    top-10 routing, T tokens sharing one activation column each (ne11 = 1).
    One step = one MUL_MAT_ID (pre-pass, on-GPU routing, expert GEMV tasks)
    with the next of 16 router id sets; GB/s counts the weight bytes of the
    experts that step touches."""
    E, n_used, M, K = 512, 10, 512, 2048
    raw = synth.weights(qmm.Q4_K, E * M, K, seed=4)
    w = be.new_tensor(qmm.Q4_K, (K, M, E))
    be.set_tensor(w, raw)
    ebytes = raw.nbytes // E
    idsets, touched = [], []
    for k in range(16):
        ids = synth.moe_ids(T, E, n_used, seed=100 + k)
        t = be.new_tensor(qmm.I32, (n_used, T))
        be.set_tensor(t, ids.view(np.uint8).ravel())
        idsets.append(t)
        touched.append(len(np.unique(ids)) * ebytes)
    x = synth.activations(T, K, seed=5)
    xt = be.new_tensor(qmm.F32, (K, 1, T))
    be.set_tensor(xt, x.view(np.uint8).ravel())
    yt = be.new_tensor(qmm.F32, (M, n_used, T))
    steps = max(16, args.steps // 2)
    for i in range(16):
        be.mul_mat_id(w, xt, idsets[i % 16], yt)
    be.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        be.mul_mat_id(w, xt, idsets[i % 16], yt)
    be.synchronize()
    wall = time.perf_counter() - t0
    be.kernel_timing(True)
    for i in range(steps):
        be.mul_mat_id(w, xt, idsets[i % 16], yt)
    k_ms, n = be.kernel_time()
    be.kernel_timing(False)
    bytes_step = float(np.mean(touched))
    us = wall * 1e6 / steps
    k_us = k_ms / max(n, 1) * 1e3
    path = be.last_path()
    # the router (softmax / top-10 over 512 logits per token) and the combine of the layer's
    # down-projection outputs (hidden 2048, 10 slots) around it, device time per op
    lg = be.new_tensor(qmm.F32, (E, T))
    be.set_tensor(lg, synth.activations(T, E, seed=6).view(np.uint8).ravel())
    rid = be.new_tensor(qmm.I32, (n_used, T))
    rw = be.new_tensor(qmm.F32, (n_used, T))
    ex = be.new_tensor(qmm.F32, (2048, n_used, T))
    be.set_tensor(ex, synth.activations(n_used * T, 2048, seed=7).view(np.uint8).ravel())
    yo = be.new_tensor(qmm.F32, (2048, T))
    # the layer's gate and up stacks with the SwiGLU in one call (one route, one GEMV launch)
    wu = be.new_tensor(qmm.Q4_K, (K, M, E))
    be.copy(wu.buf, 0, w.buf, 0, qmm.alloc_size(qmm.Q4_K, (K, M, E)))
    yg = be.new_tensor(qmm.F32, (M, n_used, T))
    state = {"i": 0}

    def glu():
        be.mul_mat_id_glu(w, wu, xt, idsets[state["i"] % 16], yg, qmm.GLU_SWIGLU)
        state["i"] += 1

    times = {}
    for name, fn in (("router", lambda: be.moe_topk(lg, rid, rw)), ("combine", lambda: be.moe_combine(ex, rw, yo)),
                     ("gate_up_glu", glu)):
        for _ in range(10):
            fn()
        be.synchronize()
        be.timer_begin()
        for _ in range(steps):
            fn()
        times[name] = be.timer_end() * 1e3 / steps
    out = {"workload": f"MUL_MAT_ID Q4_K 512 experts x (512 x 2048), top-10, T={T} (config 3 gate/up)",
           "path": path, "us_per_op": round(us, 3), "expert_bytes_touched": int(bytes_step),
           "GBs": round(bytes_step / (us * 1e-6) / 1e9, 1), "kernel_us": round(k_us, 3),
           "kernel_GBs": round(bytes_step / (k_us * 1e-6) / 1e9, 1),
           "router_us": round(times["router"], 3), "combine_us": round(times["combine"], 3),
           "gate_up_glu_us": round(times["gate_up_glu"], 3)}
    for t in (lg, rid, rw, ex, yo, wu, yg):
        be.free_buffer(t.buf)
    for t in idsets:
        be.free_buffer(t.buf)
    for t in (w, xt, yt):
        be.free_buffer(t.buf)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--only", default="", help="profile one workload: q4k_gemv, q40_gemm, q4k_gemm, gemv, glu or moe")
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
        wall, dev_ms, k_ms = time_op(be, ws, xt, yt, args.steps, args.warmup)
        path = be.last_path()
        algo = raw.nbytes + K * N * 4 + M * N * 4
        value = algo * args.steps / wall / 1e9
        achieved = algo / (k_ms * 1e-3) / 1e9
        traffic = profile_traffic("q4k_gemv")
        out.update({
            "metric": "Q4_K GEMV GB/s (% of 8 TB/s) at N=1; Q4_0 GEMM TOPS (% MFMA peak) at N=512",
            "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(wall * 1e3 / args.steps, 5), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "int8", "data": "synthetic",
            "config": {"workload": "Q4_K GEMV 17408x5120 N=1 (config 2 ffn gate/up), MUL_MAT incl. q8_K pre-pass",
                       "weights": "Q4_K", "M": M, "K": K, "N": N, "weight_copies": len(ws),
                       "rotated_bytes": int(len(ws) * raw.nbytes), "path": path,
                       "device_ms_per_step": round(dev_ms / args.steps, 5)},
            "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                         "kernel": "k_gemv<12, 1> (Q4_K, 1 column)", "kernel_us": round(k_ms * 1e3, 3),
                         "algorithmic_bytes": int(algo)},
        })
        if not args.no_cpu:
            import oracle
            out["cpu_baseline"] = cpu_baseline(oracle, qmm.Q4_K, raw, M, K, x, args.cpu_seconds)
        for w in ws:
            be.free_buffer(w.buf)

    if not args.no_secondary and args.only in ("", "q40_gemm", "q4k_gemm"):
        cases = [(qmm.Q4_0, 4096, 4096, 512, "Q4_0 GEMM 4096x4096x512 (config 1 attn)", "q40_gemm", "q40_gemm"),
                 (qmm.Q4_0, 11008, 4096, 512, "Q4_0 GEMM 11008x4096x512 (config 1 ffn gate/up)", "q40_gemm",
                  "q40_gemm_11008"),
                 (qmm.Q4_K, 17408, 5120, 512, "Q4_K GEMM 17408x5120x512 (config 2 ffn gate/up)", "q4k_gemm", "q4k_gemm")]
        secs = []
        for qtype, M2, K2, N2, name, tag, ttag in cases:
            if args.only and args.only != tag:
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
        moe = [moe_case(be, qmm, synth, T, args) for T in (1, 4, 256)]
        if out:
            out["moe"] = moe
        else:
            out = {"metric": "MUL_MAT_ID GB/s", "value": moe[-1]["GBs"], "unit": "GB/s", "moe": moe}
    be.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
