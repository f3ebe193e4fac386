#!/usr/bin/env python
"""bench.py — the quantized-linear hot path on one MI355X against its roofline.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs 1,2,3,4,5,q6k_head,m4_q4k,...] [--cpu-seconds S | --no-cpu]

A step is one pass of the hot path over one batch of synthetic input of a BASELINE config: one kernel launch for the
decode GEMV configs 1-3, the 7 projection launches of one 27B-class layer for configs 4-5. The headline (`value`) is
config 2 (GGUF Q8_0 decode GEMV, x[1,5120] @ W[17408,5120]^T), in GB/s of algorithmic bytes (packed weight bytes +
scales + x + y, never repack padding) per second, with the weights already in HBM. Weights are repacked once at load
as a load would (north star 3): single-row configs into the row-major planes of the decode GEMV, batched configs (4
int8, 5 Q4_K) into 16-row tiles, the layout ops.prepare loads by default. `q6k_head` is not a BASELINE config: it is
the shape of the reference's largest published per-call number (a 151936 x 2560 Q6_K output head at one activation
row, 369.8 us on TPU v6e-1, reference CORE-CHANGES.md:73), reported beside the configs, as are one 27B-class layer at 1,
4 and 16 activation rows (`m1_q4k` row-major, `m1_q4k_tiles`, `m4_*`, `m16_*`: the reference engine's row buckets;
Q4_K, Q8_0, Q5_K, Q6_K and int8 weights, tiles from 2 rows on) and config 5 on row-major planes (`c5_rm`). Rows
`m1_q4k_stacked`, `m4_q4k_stacked`, `m16_q4k_stacked` and `c4_stacked` time the same layer with the projections that
share an input stacked by rows at load (ops.stack_rows: q|k|v 8192 x 5120, gate|up 34816 x 5120), four launches per
layer instead of seven; the BASELINE configs 4 and 5 stay the seven launches they name. `p512_q4k` is the same Q4_K
layer at 512 rows, the reference engine's default prefill chunk (runtime/engine.py:168). `q4k_9728` and `q2k_9728` are
the shapes of the reference's other published per-call numbers (a 9728 x 2560 weight at one row: Q4_K 22.6 us, Q2_K
25.5 us on TPU v6e-1, CORE-CHANGES.md:84): Q4_K on the decode GEMV, Q2_K (no kernel planes here) on the exact path's
fused product over the file's blocks (mbq_matmul_raw).

Timing: each projection's launches are captured in a HIP graph (torch.cuda.CUDAGraph) of K launches that cycles through
>= 1 GiB of distinct weight copies (the 256 MB Infinity Cache cannot serve repeats), replayed once for warmup, then R
times (R >= 5 and R * K >= 100), each replay bracketed by torch.cuda.synchronize() and timed with HIP events on the
stream the kernels run on. A projection's launch time is the median over the R replays of (replay time / K), so every
figure is the median of >= 100 timed launches whatever K is; `mean_us` beside it is the mean over all of them. Beside
it, `eager_call_us` is the end-to-end time of back-to-back eager ctypes calls through the C ABI, timed on the host
(argument checks, plan, launch and kernel; up to 50 calls). Rows `c2_ops`, `m1_q4k_ops`, `m4_q4k_ops` and `c5_ops`
time the same work through mashbox_amd.ops.qmatmul (prepare's default layout, the result in x's dtype), the caller's
path. The CPU
baseline is the oracle's restatement of mashbox's exact path
(rebuild float32 weights per call, float32 dot; int8: float32 dot then the scales) on the host's cores, every config at
full size (a few seconds each); `cpu_baseline` is config 2's.

The one JSON line on stdout carries the contract's fields and one short summary per config (well under the 8,000
characters a driver keeps); the per-projection detail goes to the --detail file (its default: --help).

Profiling modes (rocprofv3 runs of committed files; summaries in profiles/): --pmc-probe [CONFIGS] launches each
config's projections a few times plus a calibration copy; --summarize-pmc turns a FETCH_SIZE and a WRITE_SIZE run of
it into profiles/traffic.json; --summarize-counters prints a counter run's means per kernel; --summarize-stats prints a
--kernel-trace --stats CSV.
"""
import argparse
import ctypes
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "decode GEMV HBM GB/s (% of peak) + prefill GEMM TFLOP/s (% MFMA peak)"
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E, AMD spec
PEAK_BF16_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, AMD spec (no sparsity)
HEADLINE = 2


def algorithmic_bytes(t, m, n, k):
    if t == "int8":
        w = n * k + 4 * n
    else:
        bs, ts = {8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210), 10: (256, 84)}[t]
        w = n * (k // bs) * ts
    return w + 2 * m * k + 2 * m * n


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# the configs a run without --configs times, in order
DEFAULT_CONFIGS = ("1,2,3,4,5,q6k_head,m1_q4k,m1_q4k_tiles,m4_q4k,m16_q4k,m4_q8,m16_q8,m4_q5k,m16_q5k,m4_q6k,m16_q6k,"
                   "m4_int8,m16_int8,c5_rm,c2_ops,m1_q4k_ops,m4_q4k_ops,c5_ops,m1_q4k_stacked,m4_q4k_stacked,"
                   "m16_q4k_stacked,c4_stacked,p512_q4k,q4k_9728,q2k_9728")

# rows timed through mashbox_amd.ops.qmatmul (the caller's path) instead of the C ABI: row -> the config it repeats
OPS_ROWS = {"c2_ops": 2, "c5_ops": 5, "m4_q4k_ops": "m4_q4k", "m1_q4k_ops": "m1_q4k"}


def config_of(idx):
    from mashbox_amd import synth
    idx = OPS_ROWS.get(idx, idx)
    return synth.CONFIGS[idx] if idx in synth.CONFIGS else synth.EXTRA[idx]


def setup_projection(idx, pi, rotate_bytes):
    """one projection of a config, ready to launch: seeded synthetic weights in HBM (repacked as a load would), cycled
    over >= rotate_bytes of distinct copies -> (launch(copy) -> rc, copies, weight bytes, plan text, (t, M, N, K)).
    An OPS_ROWS entry loads the GGUF blocks with ops.prepare and launches ops.qmatmul."""
    import torch
    from mashbox_amd import synth
    from mashbox_amd import _lib as LIB
    from mashbox_amd._lib import OUT_BF16, check, lib

    L = lib()
    dev = torch.device("cuda", 0)
    via_ops = idx in OPS_ROWS
    base = OPS_ROWS.get(idx, idx)
    t, M, projs = config_of(idx)
    name, N, K = projs[pi]
    seed = (1000 * base if isinstance(base, int) else 9000) + pi
    st = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    x = synth.acts(M, K, seed=seed, device=dev)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    if via_ops:
        from mashbox_amd import kernels as KQ
        from mashbox_amd import ops
        if ops.kernel_types() == frozenset():
            ops.load_kernels()
        raw = {8: synth.q8_0_raw, 12: synth.q4_k_raw, 13: synth.q5_k_raw, 14: synth.q6_k_raw}[t](N, K, seed=seed + 7, device=dev)
        h = ops.prepare(raw, t, (N, K))
        if not isinstance(h, ops.Packed):
            raise RuntimeError(f"{idx} {name}: ops.prepare gave {h!r}, not kernel planes")
        del raw
        p = h.packed
        wbytes = p.buf.numel()
        copies = max(1, math.ceil(rotate_bytes / wbytes))
        hs = [h] + [ops.Packed(KQ.Planes(p.buf.clone(), p.t, p.N, p.K, p.lead), h.t, h.shape) for _ in range(copies - 1)]

        def launch(c):
            ops.qmatmul(x, hs[c])
            return 0
        plan = "ops.qmatmul " + LIB.plan_str(p.t, M, N, K)
    elif t == 10:
        # Q2_K has no kernel planes: the exact path's fused product reads the file's blocks (mbq_matmul_raw)
        raw = synth.q2_k_raw(N, K, seed=seed + 7, device=dev)
        wbytes = raw.numel()
        copies = max(1, math.ceil(rotate_bytes / wbytes))
        bufs = [raw] + [raw.clone() for _ in range(copies - 1)]

        def launch(c):
            return L.mbq_matmul_raw(t, ctypes.c_void_p(bufs[c].data_ptr()), ctypes.c_void_p(x.data_ptr()), M, N, K,
                                    ctypes.c_void_p(y.data_ptr()), OUT_BF16, st())
        plan = "raw GEMV (exact path, file blocks)"
    elif t == "int8" and M > 1:
        # batched int8: the weights repacked once at load into 16-row tiles (MBQ_I8T planes; from 2 rows on they run
        # faster than row-major weights: MI355X, 17408 x 5120 at 4 rows 19 vs 36 us)
        q, s = synth.int8_weights(N, K, seed=seed + 7, device=dev)
        pb = check(L.mbq_plane_bytes(LIB.I8T, N, K), "int8 plane_bytes")
        planes = torch.empty(pb, dtype=torch.uint8, device=dev)
        check(L.mbq_int8_repack_dev(ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(s.data_ptr()), N, K,
                                    ctypes.c_void_p(planes.data_ptr()), st()), "int8 repack")
        del q, s
        wbytes = pb
        copies = max(1, math.ceil(rotate_bytes / wbytes))
        bufs = [planes] + [planes.clone() for _ in range(copies - 1)]

        def launch(c):
            return L.mbq_matmul(LIB.I8T, ctypes.c_void_p(bufs[c].data_ptr()), 0, None, 1, ctypes.c_void_p(x.data_ptr()),
                                M, N, K, ctypes.c_void_p(y.data_ptr()), OUT_BF16, st())
        plan = LIB.plan_str(LIB.I8T, M, N, K)
    elif t == "int8":
        # decode int8 at one row: the reference's row-major weights, run by the decode GEMV
        q, s = synth.int8_weights(N, K, seed=seed + 7, device=dev)
        wbytes = N * K + 4 * N
        copies = max(1, math.ceil(rotate_bytes / wbytes))
        bufs = [(q, s)] + [(q.clone(), s.clone()) for _ in range(copies - 1)]

        def launch(c):
            qq, ss = bufs[c]
            return L.mbq_int8_linear(ctypes.c_void_p(qq.data_ptr()), ctypes.c_void_p(ss.data_ptr()),
                                     ctypes.c_void_p(x.data_ptr()), M, N, K, ctypes.c_void_p(y.data_ptr()), OUT_BF16, st())
        plan = LIB.plan_str(LIB.INT8, M, N, K)
    else:
        raw = {8: synth.q8_0_raw, 12: synth.q4_k_raw, 13: synth.q5_k_raw, 14: synth.q6_k_raw}[t](N, K, seed=seed + 7, device=dev)
        # batched GGUF configs (2 rows and more) load the blocks as 16-row tiles, ops.prepare's default layout;
        # single-row configs keep the row-major planes of the decode GEMV; "_rm" / "_tiles" rows force one
        tiles = (M > 1 and not str(idx).endswith("_rm")) or str(idx).endswith(("_tiles", "_stacked"))
        pt = {12: LIB.Q4KT, 8: LIB.Q8T, 13: LIB.Q5KT, 14: LIB.Q6KT}.get(t, t) if tiles else t
        pb = check(L.mbq_plane_bytes(pt, N, K), "plane_bytes")
        planes = torch.empty(pb, dtype=torch.uint8, device=dev)
        check(L.mbq_repack_dev(pt, ctypes.c_void_p(raw.data_ptr()), N, K, ctypes.c_void_p(planes.data_ptr()), st()), "repack")
        del raw
        wbytes = pb
        copies = max(1, math.ceil(rotate_bytes / wbytes))
        bufs = [planes] + [planes.clone() for _ in range(copies - 1)]

        def launch(c):
            return L.mbq_matmul(pt, ctypes.c_void_p(bufs[c].data_ptr()), 0, None, 1, ctypes.c_void_p(x.data_ptr()),
                                M, N, K, ctypes.c_void_p(y.data_ptr()), OUT_BF16, st())
        plan = LIB.plan_str(pt, M, N, K)
    torch.cuda.synchronize()
    check(launch(0), f"config {idx} {name}")          # eager call: argument errors surface here, not in a capture
    torch.cuda.synchronize()
    return launch, copies, wbytes, plan, (t, M, N, K)


def time_graph(g, launches, replays):
    """-> (median, mean) microseconds per launch over `replays` replays of graph g (each holds `launches` launches),
    each replay bracketed by torch.cuda.synchronize() and timed with HIP events on the current stream"""
    import statistics
    import torch
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    per = []
    for _ in range(replays):
        torch.cuda.synchronize()
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        per.append(e0.elapsed_time(e1) * 1000.0 / launches)
    return statistics.median(per), sum(per) / len(per)


def replays_for(steps, min_launches=100, min_replays=5):
    return max(min_replays, math.ceil(min_launches / max(1, steps)))


def run_config(idx, steps, warmup, rotate_bytes):
    import torch
    from mashbox_amd import synth
    from mashbox_amd._lib import check

    t, M, projs = config_of(idx)
    base = OPS_ROWS.get(idx, idx)
    out = {"projections": {}}
    total_us = total_mean_us = total_eager_us = 0.0
    total_bytes = 0
    total_flops = 0
    replays = replays_for(steps)
    for pi, (name, N, K) in enumerate(projs):
        launch, copies, wbytes, plan, _ = setup_projection(idx, pi, rotate_bytes)

        def capture(n):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for i in range(n):
                    check(launch(i % copies), "launch")
            return g

        if warmup > 0:
            gw = capture(warmup)
            gw.replay()
        g = capture(steps)
        us, mean_us = time_graph(g, steps, replays)
        # end to end through the C ABI: back-to-back eager ctypes calls timed on the host (argument checks, plan,
        # launch, and the kernel), the caller's view when it does not capture a graph
        ne = min(steps, 50)
        rcs = 0
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(ne):
            rcs |= launch(i % copies)
        torch.cuda.synchronize()
        eager_us = (time.perf_counter() - t0) * 1e6 / ne
        check(rcs, f"config {idx} {name} eager calls")
        ab = algorithmic_bytes(t, M, N, K)
        fl = 2 * M * N * K
        out["projections"][name] = {"M": M, "N": N, "K": K, "us": round(us, 3), "mean_us": round(mean_us, 3),
                                    "GBps": round(ab / us / 1e3, 1), "TFLOPs": round(fl / us / 1e6, 2),
                                    "eager_call_us": round(eager_us, 2), "rotation_copies": copies,
                                    "rotation_MB": round(copies * wbytes / 1e6, 1), "plan": plan}
        total_eager_us += eager_us
        total_us += us
        total_mean_us += mean_us
        total_bytes += ab
        total_flops += fl
        del launch, g
        torch.cuda.empty_cache()
    gbs = total_bytes / total_us / 1e3
    tfl = total_flops / total_us / 1e6
    out.update({"type": {8: "Q8_0", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K", 10: "Q2_K"}.get(t, t), "M": M,
                "us_per_step": round(total_us, 3), "mean_us_per_step": round(total_mean_us, 3),
                "launches_timed": replays * steps, "GBps": round(gbs, 1), "hbm_frac": round(gbs / PEAK_HBM_GBS, 4),
                "TFLOPs": round(tfl, 2), "mfma_frac": round(tfl / PEAK_BF16_TFLOPS, 4),
                "eager_us_per_step": round(total_eager_us, 2), "algorithmic_bytes": total_bytes, "flops": total_flops})
    if base in synth.REF_TPU_US:
        out["reference_tpu_v6e_us"] = synth.REF_TPU_US[base]
        out["speedup_vs_reference_tpu_v6e"] = round(synth.REF_TPU_US[base] / total_us, 2)
    log(f"{idx}: {total_us:.2f} us  {gbs:.0f} GB/s {100 * gbs / PEAK_HBM_GBS:.1f}%HBM  "
        f"{tfl:.1f} TF/s {100 * tfl / PEAK_BF16_TFLOPS:.1f}%MFMA")
    return out


def measured_peaks():
    """the box's achievable rates, measured by libmbq's probes (mbq_probe.hip) and torch: HBM read (every KiB of 2 GiB
    read once by a streaming kernel), device copy (torch, read + write) and bf16 MFMA (back-to-back MFMAs on every SIMD)"""
    import torch
    from mashbox_amd._lib import check, lib

    L = lib()
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    n = (2 << 30) // 4
    a = torch.ones(n, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    sink = torch.zeros(16, dtype=torch.float32, device="cuda")
    flops = ctypes.c_int64(0)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    out = {}
    for name, fn, nbytes in (
            ("read_GBps", lambda: check(L.mbq_probe_read(ctypes.c_void_p(a.data_ptr()), 4 * n,
                                                         ctypes.c_void_p(sink.data_ptr()), st), "read probe"), 4 * n),
            ("copy_GBps", lambda: b.copy_(a), 8 * n)):
        fn()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(10):
            fn()
        e1.record()
        torch.cuda.synchronize()
        out[name] = round(nbytes * 10 / (e0.elapsed_time(e1) * 1e-3) / 1e9, 1)
    check(L.mbq_probe_mfma(20000, ctypes.c_void_p(sink.data_ptr()), ctypes.byref(flops), st), "MFMA probe")
    torch.cuda.synchronize()
    e0.record()
    check(L.mbq_probe_mfma(20000, ctypes.c_void_p(sink.data_ptr()), ctypes.byref(flops), st), "MFMA probe")
    e1.record()
    torch.cuda.synchronize()
    out["mfma_bf16_TFLOPs"] = round(flops.value / (e0.elapsed_time(e1) * 1e-3) / 1e12, 1)
    out["how"] = ("read: mbq_probe_read over 2 GiB (4 waves per CU, 16 KiB in flight each); copy: torch copy of 2 GiB "
                  "(bytes read + written); MFMA: mbq_probe_mfma, v_mfma_f32_16x16x32_bf16 x 8 independent "
                  "accumulators, 8 waves per CU")
    del a, b
    torch.cuda.empty_cache()
    return out


def _cpu_threads():
    """host threads for the CPU baselines: torch's intra-op count, which follows OMP_NUM_THREADS (the GPU box allots 16
    host cores to a one-GPU job and sets OMP_NUM_THREADS=16; the container's own count otherwise)"""
    import torch
    return max(1, torch.get_num_threads())


def _cpu_model():
    try:
        return next((l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name")), "?")
    except OSError:
        return "?"


def cpu_baselines(seconds_per_config, configs=(1, 2, 3, 4, 5), min_calls=5):
    """the oracle's restatement of mashbox's exact path (oracle/ref.py) on the host cores, per config, seed-0 inputs of
    oracle/gen.py at full size: GGUF configs rebuild float32 weights from the blocks per call (row chunks of
    exact_chunk_rows, one chunk per host thread) and multiply in float32; int8 configs take (x @ bf16(q).T) * s in
    float32 (BLAS on the host threads). Median of >= min_calls calls (more while under seconds_per_config)."""
    import numpy as np
    from threadpoolctl import threadpool_limits
    from oracle import gen as G
    from oracle import ref as R

    threads = _cpu_threads()
    res = {}
    for idx in configs:
        cfg = G.config(idx, seed=0)
        m = cfg["m"]
        times = []
        t_end = time.perf_counter() + seconds_per_config
        while len(times) < min_calls or time.perf_counter() < t_end:
            t0 = time.perf_counter()
            for name, n, k, w, xb in cfg["projections"]:
                x = R.bf16_to_f32(xb)
                if cfg["t"] == "int8":
                    q, s = w
                    with threadpool_limits(threads):
                        y = R.int8_linear(x, q, s)
                else:
                    with threadpool_limits(1):                      # one BLAS thread per chunk, chunks on `threads`
                        y = R.qmatmul_exact(x, w, cfg["t"], (n, k), threads=threads)
                R.bf16_round(y)
            times.append(time.perf_counter() - t0)
        med = float(np.median(times))
        ab = sum(algorithmic_bytes(cfg["t"] if cfg["t"] == "int8" else int(cfg["t"]), m, n, k)
                 for _, n, k, _, _ in cfg["projections"])
        fl = sum(2 * m * n * k for _, n, k, _, _ in cfg["projections"])
        res[f"c{idx}"] = {"us_per_step": round(med * 1e6, 1), "GBps": round(ab / med / 1e9, 3),
                          "TFLOPs": round(fl / med / 1e12, 4), "calls": len(times)}
        log(f"cpu baseline config {idx}: {med * 1e3:.1f} ms/step ({len(times)} calls, {threads} threads)")
        del cfg
    return res, threads


def cpu_baseline_line(per_config, threads):
    """the contract's cpu_baseline object: config 2 (the headline) from cpu_baselines"""
    c2 = per_config["c2"]
    return {"value": c2["GBps"], "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"config 2 whole (Q8_0 W[17408,5120], x[1,5120], seed 0): {c2['calls']} calls of "
                      f"oracle.ref.qmatmul_exact (float32 rebuild in 8 row chunks of 2176 + float32 dot, chunks on "
                      f"{threads} threads), median {c2['us_per_step'] / 1e3:.1f} ms/call; host CPU {_cpu_model()}, "
                      f"os.cpu_count() {os.cpu_count()}, torch threads {threads}"}


# kernels of the matmul path (dispatches the pmc probe counts; repack, zero and dequant kernels excluded)
MATMUL_KERNELS = ("gemv_kernel", "wsgemm_kernel", "kgemm_kernel", "sgemm_kernel", "gemm_kernel")


def pmc_probe(configs=(1, 2, 3, 4, 5), launches=4, copy_mib=1024, rotate_mb=1024):
    """for rocprofv3 --pmc: every projection of each config launched `launches` times eagerly over rotating weight
    copies (the bench's inputs), in config and projection order, then a plain device copy of copy_mib MiB (read and
    written once) 4 times to calibrate FETCH_SIZE / WRITE_SIZE"""
    import torch
    from mashbox_amd import synth
    from mashbox_amd._lib import check

    for idx in configs:
        _, _, projs = synth.CONFIGS[idx] if idx in synth.CONFIGS else synth.EXTRA[idx]
        for pi in range(len(projs)):
            launch, copies, _, _, _ = setup_projection(idx, pi, rotate_mb << 20)
            for i in range(launches):
                check(launch((i + 1) % copies), "launch")
            torch.cuda.synchronize()
            del launch
            torch.cuda.empty_cache()
    src = torch.ones(copy_mib << 18, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"pmc_probe": {"configs": list(configs), "launches": launches, "copy_bytes": copy_mib << 20}}),
          flush=True)


def _counter_rows(d):
    import csv
    import glob
    rows = []
    for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
        rows += list(csv.DictReader(open(f)))
    return rows


def _probe_dispatches(rows, counter):
    """(matmul dispatches in launch order, the last 4 dispatches = the calibration copies) for one counter"""
    rows = [r for r in rows if r["Counter_Name"] == counter]
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    mm = [r for r in rows if "mbq::" in r["Kernel_Name"] and any(k in r["Kernel_Name"] for k in MATMUL_KERNELS)]
    return mm, rows[-4:]


def summarize_pmc(fetch_dir, write_dir, out, configs=(1, 2, 3, 4, 5), launches=4, copy_mib=1024):
    """profiles/traffic.json from two rocprofv3 --pmc runs of --pmc-probe (FETCH_SIZE, then WRITE_SIZE): HBM bytes per
    step of each config (per projection the median of its probe launches after the first, each on a distinct weight
    copy), each counter scaled by what it reads for the calibration copy"""
    import statistics as stt
    from mashbox_amd import synth

    fm, fc = _probe_dispatches(_counter_rows(fetch_dir), "FETCH_SIZE")
    wm, wc = _probe_dispatches(_counter_rows(write_dir), "WRITE_SIZE")
    cfg = lambda idx: synth.CONFIGS[idx] if idx in synth.CONFIGS else synth.EXTRA[idx]
    plan = [(idx, name, n, k, cfg(idx)[0], cfg(idx)[1]) for idx in configs for name, n, k in cfg(idx)[2]]
    per = launches + 1                                      # setup_projection's eager check, then the probe's launches
    if len(fm) != len(plan) * per or len(wm) != len(plan) * per:
        raise SystemExit(f"expected {len(plan) * per} matmul dispatches, got fetch {len(fm)} write {len(wm)}")
    known_kib = (copy_mib << 20) / 1024.0
    ff = known_kib / stt.median(float(r["Counter_Value"]) for r in fc)
    fw = known_kib / stt.median(float(r["Counter_Value"]) for r in wc)
    rec = {"fetch_scale": round(ff, 4), "write_scale": round(fw, 4), "copy_kib": known_kib,
           "command": "rocprofv3 --pmc FETCH_SIZE (then WRITE_SIZE) -d DIR -o out --output-format csv -- "
                      "python3 bench.py --pmc-probe; python3 bench.py --summarize-pmc FETCH_DIR WRITE_DIR"}
    for idx in configs:
        fetch_b = write_b = alg = 0.0
        kernels = set()
        for p, (ci, name, n, k, t, m) in enumerate(plan):
            if ci != idx:
                continue
            # the eager check and the first probe launch also fault in code and tables: the later launches count
            fk = [float(r["Counter_Value"]) for r in fm[p * per + 2:(p + 1) * per]]
            wk = [float(r["Counter_Value"]) for r in wm[p * per + 2:(p + 1) * per]]
            fetch_b += stt.median(fk) * ff * 1024.0
            write_b += stt.median(wk) * fw * 1024.0
            alg += algorithmic_bytes(t, m, n, k)
            kernels.add(fm[p * per]["Kernel_Name"].split("(")[0])
        rec[_key(idx)] = {"hbm_bytes_per_launch": round(fetch_b + write_b), "fetch_bytes": round(fetch_b),
                          "write_bytes": round(write_b), "algorithmic_bytes": round(alg),
                          "traffic_over_algorithmic": round((fetch_b + write_b) / alg, 4), "kernels": sorted(kernels)}
    with open(out, "w") as f:
        json.dump(rec, f, indent=1)
    print(json.dumps(rec), flush=True)


def summarize_counters(d, kernel_substr=None, simds=1024, clock_ghz=2.17):
    """markdown of rocprofv3 --pmc runs of --pmc-probe (one directory per pass under d): per matmul kernel, the mean
    of each counter over its dispatches and derived shares. SQ_VALU_MFMA_BUSY_CYCLES is summed over the SIMDs (it
    reads 16 per v_mfma_f32_16x16x32_bf16), so its share of the kernel is busy / (SIMDs x dispatch ns x clock); the
    clock is the MFMA probe's (2.28 PF = 1024 SIMDs x 1024 flop/cycle x 2.17 GHz) and the dispatch time is the one the
    profiler measured, on dispatches it serializes"""
    import collections
    import statistics as stt
    rows = _counter_rows(d)
    by = collections.defaultdict(lambda: collections.defaultdict(list))
    dur = collections.defaultdict(list)
    for r in rows:
        name = r["Kernel_Name"]
        if "mbq::" not in name or not any(k in name for k in MATMUL_KERNELS):
            continue
        if kernel_substr and kernel_substr not in name:
            continue
        kern = name.split("(")[0]
        by[kern][r["Counter_Name"]].append(float(r["Counter_Value"]))
        dur[(kern, r["Counter_Name"])].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])))
    for kern, cs in sorted(by.items()):
        o = {k: sum(v) / len(v) for k, v in cs.items()}
        ns = stt.median(dur[(kern, next(iter(cs)))])
        print(f"\n`{kern}` ({len(next(iter(cs.values())))} dispatches per pass, median {ns / 1e3:.1f} us under the "
              f"profiler)\n\n| counter | mean per dispatch |\n|---|---:|")
        for k in sorted(o):
            print(f"| {k} | {o[k]:.0f} |")
        wc = o.get("SQ_WAVE_CYCLES")
        if wc:
            for k in ("SQ_WAIT_ANY", "SQ_WAIT_INST_ANY", "SQ_ACTIVE_INST_VALU", "SQ_ACTIVE_INST_LDS"):
                if k in o:
                    print(f"| {k} / SQ_WAVE_CYCLES | {o[k] / wc:.3f} |")
        if "SQ_VALU_MFMA_BUSY_CYCLES" in o:
            busy = sum(cs["SQ_VALU_MFMA_BUSY_CYCLES"])
            t_ns = sum(dur[(kern, "SQ_VALU_MFMA_BUSY_CYCLES")])
            print(f"| MFMA busy share: SQ_VALU_MFMA_BUSY_CYCLES / ({simds} SIMDs x {clock_ghz} GHz x dispatch time) | "
                  f"{busy / (simds * t_ns * clock_ghz):.3f} |")
        if "SQ_VALU_MFMA_COEXEC_CYCLES" in o and o.get("SQ_VALU_MFMA_BUSY_CYCLES"):
            print(f"| SQ_VALU_MFMA_COEXEC_CYCLES / SQ_VALU_MFMA_BUSY_CYCLES | "
                  f"{o['SQ_VALU_MFMA_COEXEC_CYCLES'] / o['SQ_VALU_MFMA_BUSY_CYCLES']:.3f} |")
        if "SQ_INSTS_VALU" in o and "SQ_INSTS_MFMA" in o and o["SQ_INSTS_MFMA"]:
            print(f"| SQ_INSTS_VALU / SQ_INSTS_MFMA | {o['SQ_INSTS_VALU'] / o['SQ_INSTS_MFMA']:.2f} |")
        if "SQ_LDS_BANK_CONFLICT" in o and "SQ_INSTS_LDS" in o and o["SQ_INSTS_LDS"]:
            print(f"| SQ_LDS_BANK_CONFLICT / SQ_INSTS_LDS | {o['SQ_LDS_BANK_CONFLICT'] / o['SQ_INSTS_LDS']:.3f} |")


def summarize_stats(csv_path, top_other=4):
    """markdown table of a rocprofv3 --kernel-trace --stats kernel_stats.csv: every mbq kernel, then the other kernels
    (torch's input generation, copies) with the most time"""
    import csv
    rows = list(csv.DictReader(open(csv_path)))
    key = lambda r: float(r.get("TotalDurationNs", 0) or 0)
    ours = [r for r in rows if "mbq::" in r["Name"]]
    other = [r for r in rows if "mbq::" not in r["Name"]]
    print("| kernel | calls | avg us | min us | max us | % time |\n|---|---:|---:|---:|---:|---:|")
    for r in sorted(ours, key=key, reverse=True) + sorted(other, key=key, reverse=True)[:top_other]:
        name = r["Name"]
        name = name[:90] + ("..." if len(name) > 90 else "")
        print(f"| `{name}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | {float(r['MinNs']) / 1e3:.2f} | "
              f"{float(r['MaxNs']) / 1e3:.2f} | {float(r['Percentage']):.1f} |")


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[1])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--configs", default=DEFAULT_CONFIGS)
    ap.add_argument("--rotate-mb", type=int, default=1024, help="distinct weight bytes cycled per projection")
    ap.add_argument("--cpu-seconds", type=float, default=4.0, help="CPU baseline time per config (at least 5 calls)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--detail", default=os.path.join(ROOT, "gpurun_out", "bench_detail.json"),
                    help="per-projection detail (JSON file; '' = none)")
    ap.add_argument("--traffic", default=os.path.join(ROOT, "profiles", "traffic.json"),
                    help="HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE, WRITE_SIZE)")
    ap.add_argument("--pmc-probe", nargs="?", const="1,2,3,4,5", default=None, metavar="CONFIGS",
                    help="only the configs' matmul launches + a calibration copy (for rocprofv3 --pmc)")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="write --traffic from the two --pmc runs of --pmc-probe")
    ap.add_argument("--pmc-configs", default="1,2,3,4,5", metavar="CONFIGS",
                    help="--summarize-pmc: the configs the --pmc-probe runs launched, in order")
    ap.add_argument("--summarize-counters", nargs="+", metavar=("DIR", "KERNEL"),
                    help="markdown of a --pmc run of --pmc-probe: counter means per matmul kernel")
    ap.add_argument("--summarize-stats", metavar="KERNEL_STATS_CSV", help="print a rocprofv3 --stats CSV as markdown")
    a = ap.parse_args()
    if a.summarize_pmc:
        return summarize_pmc(a.summarize_pmc[0], a.summarize_pmc[1], a.traffic, _configs(a.pmc_configs))
    if a.summarize_stats:
        return summarize_stats(a.summarize_stats)
    if a.summarize_counters:
        return summarize_counters(a.summarize_counters[0], a.summarize_counters[1] if len(a.summarize_counters) > 1 else None)
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py runs on one GPU: this path is measured on a single MI355X, at one GPU's share of the weights "
              "(column-parallel rows need no collective; row-parallel K splits add one reduce-scatter + all-gather "
              "of the partials). --gpus must be 1.", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    if a.pmc_probe:
        return pmc_probe(_configs(a.pmc_probe), rotate_mb=a.rotate_mb)
    configs = [int(c) if c.isdigit() else c for c in a.configs.split(",") if c]
    if HEADLINE not in configs:
        configs.insert(0, HEADLINE)
    res = {}
    for c in configs:
        res[c] = run_config(c, a.steps, a.warmup, a.rotate_mb << 20)
    try:
        with open(a.traffic) as f:
            tj = json.load(f)
    except (OSError, ValueError):
        tj = {}
    peaks = measured_peaks()
    cpu = None
    if not a.no_cpu:
        per, threads = cpu_baselines(a.cpu_seconds)
        cpu = (per, threads)
    line, detail = make_line(res, tj, peaks, cpu, a.steps, a.warmup, a.detail)
    if a.detail:
        os.makedirs(os.path.dirname(os.path.abspath(a.detail)), exist_ok=True)
        with open(a.detail, "w") as f:
            json.dump(detail, f, indent=1)
    print(json.dumps(line, separators=(",", ":")), flush=True)


def _key(c):
    return f"c{c}" if isinstance(c, int) else str(c)


def _configs(text):
    """"1,2,m1_q4k_tiles" -> (1, 2, "m1_q4k_tiles")"""
    return tuple(int(c) if c.isdigit() else c for c in text.split(",") if c)


def summary(r):
    """one config's short summary for the JSON line: microseconds per step, the rate of its bound and its fraction"""
    o = {"us": round(r["us_per_step"], 2)}
    if r["mfma_frac"] >= 0.1:                      # the prefill GEMM and config 4: MFMA rate beside the HBM rate
        o.update(TFLOPs=round(r["TFLOPs"], 1), mfma=round(r["mfma_frac"], 3))
    o.update(GBps=round(r["GBps"]), hbm=round(r["hbm_frac"], 3))
    if "traffic_over_algorithmic" in r:
        o["traffic_x"] = round(r["traffic_over_algorithmic"], 3)
    if "speedup_vs_reference_tpu_v6e" in r:        # the shapes of the reference's published per-call numbers
        o["x_ref_tpu"] = r["speedup_vs_reference_tpu_v6e"]
    return o


def make_line(res, traffic, peaks, cpu, steps, warmup, detail_path=None):
    """-> (the one JSON line of the contract, the per-projection detail). res: run_config results by config; traffic:
    profiles/traffic.json; cpu: (cpu_baselines per config, threads) or None"""
    head = res[HEADLINE]
    proj = head["projections"]["w"]
    for c, r in res.items():
        tc = traffic.get(_key(c))
        if tc and "hbm_bytes_per_launch" in tc:
            r["hbm_traffic_bytes"] = tc["hbm_bytes_per_launch"]
            r["traffic_over_algorithmic"] = round(tc["hbm_bytes_per_launch"] / r["algorithmic_bytes"], 4)
    line = {
        "metric": METRIC, "value": head["GBps"], "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(head["us_per_step"] / 1e3, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded, BASELINE config value ranges, generated on the GPU)",
        "config": {"workload": "config 2: GGUF Q8_0 decode GEMV x bf16[1,5120] @ W[17408,5120]^T, fp32 accumulate, "
                               "bf16 out", "M": 1, "N": 17408, "K": 5120, "weight_type": "Q8_0",
                   "rotation_MB": proj["rotation_MB"]},
        "timing": f"per launch: median over {replays_for(steps)} graph replays of {steps} launches "
                  f"({head['launches_timed']} launches), HIP events on the launching stream",
        "roofline": {"bound": "hbm", "achieved": head["GBps"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(head["GBps"] / PEAK_HBM_GBS, 4), "traffic": traffic.get("c2", {}).get("hbm_bytes_per_launch"),
                     "kernel": "mbq::gemv_kernel (Q8_0, 1 activation row)", "kernel_us": proj["us"],
                     "kernel_mean_us": proj["mean_us"], "algorithmic_bytes_per_launch": head["algorithmic_bytes"]},
        "configs": {_key(c): summary(r) for c, r in res.items()},
        "measured_peaks": {k: v for k, v in peaks.items() if k != "how"},
    }
    detail = {"configs": {_key(c): r for c, r in res.items()}, "measured_peaks": peaks}
    if cpu is not None:
        per, threads = cpu
        line["cpu_baseline"] = cpu_baseline_line(per, threads)
        line["cpu_baseline_us"] = {c: v["us_per_step"] for c, v in per.items()}
        detail["cpu_baseline_configs"] = per | {"threads": threads, "cpu": _cpu_model(), "os_cpu_count": os.cpu_count(),
                                                "kind": "port: oracle/ref.py restatement of mashbox's plain-JAX exact path",
                                                "inputs": "oracle/gen.py seed 0, full BASELINE sizes"}
    if detail_path:
        line["detail"] = os.path.relpath(os.path.abspath(detail_path), ROOT)
    return line, detail


if __name__ == "__main__":
    main()
