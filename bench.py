#!/usr/bin/env python
"""bench.py — the quantized-linear hot path on one MI355X against its roofline.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs 1,2,3,4,5,q6k_head] [--cpu-seconds S | --no-cpu]

A step is one pass of the hot path over one batch of synthetic input of a BASELINE config: one kernel launch for the
decode GEMV configs 1-3, the 7 projection launches of one 27B-class layer for configs 4-5. The headline (`value`) is
config 2 (GGUF Q8_0 decode GEMV, x[1,5120] @ W[17408,5120]^T), in GB/s of algorithmic bytes (packed weight bytes +
scales + x + y, never repack padding) per second, with the weights already in HBM. `q6k_head` is not a BASELINE
config: it is the shape of the reference's largest published per-call number (a 151936 x 2560 Q6_K output head at one
activation row, 369.8 us on TPU v6e-1, reference CORE-CHANGES.md:73), reported beside the configs.

Timing: each projection's launches are captured in a HIP graph (torch.cuda.CUDAGraph) that cycles through >= 1 GiB of
distinct weight copies (the 256 MB Infinity Cache cannot serve repeats), replayed once for W warmup launches, then once
for K timed launches bracketed by torch.cuda.synchronize() and HIP events on the stream the kernels run on. The kernel's
average launch duration is the event time / K. The CPU baseline is the oracle's restatement of mashbox's exact path
(rebuild float32 weights per call, float32 dot) on the host's cores, on a bounded sample of config 2.
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
        bs, ts = {8: (32, 34), 12: (256, 144), 14: (256, 210)}[t]
        w = n * (k // bs) * ts
    return w + 2 * m * k + 2 * m * n


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def run_config(idx, steps, warmup, rotate_bytes):
    import torch
    from mashbox_amd import synth
    from mashbox_amd import _lib as LIB
    from mashbox_amd._lib import OUT_BF16, check, lib

    L = lib()
    dev = torch.device("cuda", 0)
    t, M, projs = synth.CONFIGS[idx] if idx in synth.CONFIGS else synth.EXTRA[idx]
    out = {"projections": {}}
    total_us = 0.0
    total_bytes = 0
    total_flops = 0
    for pi, (name, N, K) in enumerate(projs):
        seed = (1000 * idx if isinstance(idx, int) else 9000) + pi
        x = synth.acts(M, K, seed=seed, device=dev)
        y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        if t == "int8" and M > 4:
            # batched int8: the weights repacked once at load into 16-row tiles (MBQ_I8T planes)
            q, s = synth.int8_weights(N, K, seed=seed + 7, device=dev)
            pb = check(L.mbq_plane_bytes(LIB.I8T, N, K), "int8 plane_bytes")
            planes = torch.empty(pb, dtype=torch.uint8, device=dev)
            check(L.mbq_int8_repack_dev(ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(s.data_ptr()), N, K,
                                        ctypes.c_void_p(planes.data_ptr()),
                                        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)), "int8 repack")
            del q, s
            wbytes = pb
            copies = max(1, math.ceil(rotate_bytes / wbytes))
            bufs = [planes] + [planes.clone() for _ in range(copies - 1)]

            def launch(c, bufs=bufs, x=x, y=y, M=M, N=N, K=K):
                return L.mbq_matmul(LIB.I8T, ctypes.c_void_p(bufs[c].data_ptr()), 0, None, 1,
                                    ctypes.c_void_p(x.data_ptr()), M, N, K, ctypes.c_void_p(y.data_ptr()), OUT_BF16,
                                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        elif t == "int8":
            # decode int8: the reference's row-major weights, run by the decode GEMV
            q, s = synth.int8_weights(N, K, seed=seed + 7, device=dev)
            wbytes = N * K + 4 * N
            copies = max(1, math.ceil(rotate_bytes / wbytes))
            bufs = [(q, s)] + [(q.clone(), s.clone()) for _ in range(copies - 1)]

            def launch(c, bufs=bufs, x=x, y=y, M=M, N=N, K=K):
                qq, ss = bufs[c]
                return L.mbq_int8_linear(ctypes.c_void_p(qq.data_ptr()), ctypes.c_void_p(ss.data_ptr()),
                                         ctypes.c_void_p(x.data_ptr()), M, N, K, ctypes.c_void_p(y.data_ptr()),
                                         OUT_BF16, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        else:
            raw = {8: synth.q8_0_raw, 12: synth.q4_k_raw, 14: synth.q6_k_raw}[t](N, K, seed=seed + 7, device=dev)
            pb = check(L.mbq_plane_bytes(t, N, K), "plane_bytes")
            planes = torch.empty(pb, dtype=torch.uint8, device=dev)
            check(L.mbq_repack_dev(t, ctypes.c_void_p(raw.data_ptr()), N, K, ctypes.c_void_p(planes.data_ptr()),
                                   ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)), "repack")
            del raw
            wbytes = pb
            copies = max(1, math.ceil(rotate_bytes / wbytes))
            bufs = [planes] + [planes.clone() for _ in range(copies - 1)]

            def launch(c, bufs=bufs, x=x, y=y, M=M, N=N, K=K, t=t):
                return L.mbq_matmul(t, ctypes.c_void_p(bufs[c].data_ptr()), 0, None, 1, ctypes.c_void_p(x.data_ptr()),
                                    M, N, K, ctypes.c_void_p(y.data_ptr()), OUT_BF16,
                                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        check(launch(0), f"config {idx} {name}")          # eager call: argument errors surface here, not in capture
        torch.cuda.synchronize()

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
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1000.0 / steps
        ab = algorithmic_bytes(t, M, N, K)
        fl = 2 * M * N * K
        out["projections"][name] = {"M": M, "N": N, "K": K, "us": round(us, 3), "GBps": round(ab / us / 1e3, 1),
                                    "TFLOPs": round(fl / us / 1e6, 2), "rotation_copies": copies,
                                    "rotation_MB": round(copies * wbytes / 1e6, 1),
                                    "plan": LIB.plan_str((LIB.I8T if M > 4 else LIB.INT8) if t == "int8" else t, M, N, K)}
        total_us += us
        total_bytes += ab
        total_flops += fl
        del bufs, g
        torch.cuda.empty_cache()
    gbs = total_bytes / total_us / 1e3
    tfl = total_flops / total_us / 1e6
    out.update({"type": {8: "Q8_0", 12: "Q4_K", 14: "Q6_K"}.get(t, t), "M": M, "us_per_step": round(total_us, 3),
                "GBps": round(gbs, 1), "hbm_frac": round(gbs / PEAK_HBM_GBS, 4), "TFLOPs": round(tfl, 2),
                "mfma_frac": round(tfl / PEAK_BF16_TFLOPS, 4), "algorithmic_bytes": total_bytes, "flops": total_flops})
    if idx in synth.REF_TPU_US:
        out["reference_tpu_v6e_us"] = synth.REF_TPU_US[idx]
        out["speedup_vs_reference_tpu_v6e"] = round(synth.REF_TPU_US[idx] / total_us, 2)
    log(f"config {idx}: {out['us_per_step']:.2f} us/step  {gbs:.0f} GB/s ({100 * gbs / PEAK_HBM_GBS:.1f}% HBM)  "
        f"{tfl:.1f} TFLOP/s ({100 * tfl / PEAK_BF16_TFLOPS:.1f}% MFMA)")
    return out


def measured_peaks():
    """the box's achievable HBM rates with plain torch kernels on 2 GiB: read (a float32 sum) and copy (read + write)"""
    import torch
    n = (2 << 30) // 4
    a = torch.ones(n, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    out = {}
    for name, fn, nbytes in (("read_GBps", lambda: a.sum(), 4 * n), ("copy_GBps", lambda: b.copy_(a), 8 * n)):
        fn()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(10):
            fn()
        e1.record()
        torch.cuda.synchronize()
        out[name] = round(nbytes * 10 / (e0.elapsed_time(e1) * 1e-3) / 1e9, 1)
    del a, b
    torch.cuda.empty_cache()
    return out


def cpu_baseline(seconds):
    """oracle restatement of mashbox's exact path on config 2 (Q8_0 17408 x 5120, M = 1), host cores"""
    import numpy as np
    from oracle import gen as G
    from oracle import ref as R

    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    threads = max(1, min(threads, 16))
    cfg = G.config(HEADLINE, seed=0)
    (_, n, k, raw, xb), = cfg["projections"]
    x = R.bf16_to_f32(xb)
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        y = R.qmatmul_exact(x, raw, R.Q8_0, (n, k), threads=threads)
        R.bf16_round(y)
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    ab = algorithmic_bytes(8, 1, n, k)
    try:
        model = next((l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name")), "?")
    except OSError:
        model = "?"
    return {"value": round(ab / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"config 2 whole (Q8_0 W[17408,5120], x[1,5120]): {len(times)} calls of oracle.ref.qmatmul_exact "
                      f"(float32 rebuild in 8 row chunks of 2176 + float32 dot, chunks on {threads} threads), "
                      f"median {med * 1e3:.1f} ms/call; host CPU {model}"}


def pmc_probe(launches=24, copy_mib=1024):
    """the headline kernel alone, eagerly, for rocprofv3 --pmc: `launches` config-2 GEMV launches over rotating weight
    copies, then a plain device copy of copy_mib MiB (read and written once) to calibrate the counters"""
    import torch
    from mashbox_amd import synth
    from mashbox_amd._lib import OUT_BF16, check, lib

    L = lib()
    dev = torch.device("cuda", 0)
    t, M, ((_, N, K),) = synth.CONFIGS[HEADLINE]
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    x = synth.acts(M, K, seed=1000 * HEADLINE, device=dev)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    raw = synth.q8_0_raw(N, K, seed=1000 * HEADLINE + 7, device=dev)
    pb = check(L.mbq_plane_bytes(t, N, K), "plane_bytes")
    planes = torch.empty(pb, dtype=torch.uint8, device=dev)
    check(L.mbq_repack_dev(t, ctypes.c_void_p(raw.data_ptr()), N, K, ctypes.c_void_p(planes.data_ptr()), st), "repack")
    copies = [planes] + [planes.clone() for _ in range(11)]
    for i in range(launches):
        check(L.mbq_matmul(t, ctypes.c_void_p(copies[i % len(copies)].data_ptr()), 0, None, 1,
                           ctypes.c_void_p(x.data_ptr()), M, N, K, ctypes.c_void_p(y.data_ptr()), OUT_BF16, st), "matmul")
    src = torch.ones(copy_mib << 18, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"pmc_probe": {"launches": launches, "copy_bytes": copy_mib << 20,
                                    "algorithmic_bytes": algorithmic_bytes(t, M, N, K)}}), flush=True)


def _counter_rows(d):
    import csv
    import glob
    rows = []
    for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
        rows += list(csv.DictReader(open(f)))
    return rows


def summarize_pmc(fetch_dir, write_dir, out, copy_mib=1024):
    """profiles/traffic.json from the two rocprofv3 --pmc runs of --pmc-probe (FETCH_SIZE, then WRITE_SIZE): HBM bytes
    per headline-kernel launch, each counter scaled by what it reads for the calibration copy"""
    def per(rows, counter):
        # headline-kernel dispatches, and the calibration copies: the probe's last 4 dispatches
        rows = [r for r in rows if r["Counter_Name"] == counter]
        last = sorted(int(r["Dispatch_Id"]) for r in rows)[-4:]
        k = [float(r["Counter_Value"]) for r in rows if "gemv_kernel<8, 1," in r["Kernel_Name"]]
        c = [float(r["Counter_Value"]) for r in rows if int(r["Dispatch_Id"]) in last]
        return k, c
    fk, fc = per(_counter_rows(fetch_dir), "FETCH_SIZE")
    wk, wc = per(_counter_rows(write_dir), "WRITE_SIZE")
    if not (fk and fc and wk and wc):
        raise SystemExit(f"missing dispatches: gemv fetch {len(fk)} copy fetch {len(fc)} gemv write {len(wk)} copy write {len(wc)}")
    import statistics as stt
    known_kib = (copy_mib << 20) / 1024.0
    ff, fw = known_kib / stt.median(fc), known_kib / stt.median(wc)
    fetch_b = stt.median(fk[1:] or fk) * ff * 1024.0       # the first launch also faults in code and tables
    write_b = stt.median(wk[1:] or wk) * fw * 1024.0
    rec = {"c2": {"hbm_bytes_per_launch": round(fetch_b + write_b), "fetch_bytes": round(fetch_b), "write_bytes": round(write_b),
                  "fetch_kib_raw": stt.median(fk), "write_kib_raw": stt.median(wk), "copy_fetch_kib_raw": stt.median(fc),
                  "copy_write_kib_raw": stt.median(wc), "copy_kib": known_kib, "fetch_scale": round(ff, 4),
                  "write_scale": round(fw, 4), "launches": len(fk),
                  "command": "rocprofv3 --pmc FETCH_SIZE (then WRITE_SIZE) -f csv -- python3 bench.py --pmc-probe"}}
    with open(out, "w") as f:
        json.dump(rec, f, indent=1)
    print(json.dumps(rec), flush=True)


def summarize_stats(csv_path, top=12):
    """markdown table of a rocprofv3 --kernel-trace --stats kernel_stats.csv"""
    import csv
    rows = list(csv.DictReader(open(csv_path)))
    key = lambda r: float(r.get("TotalDurationNs", 0) or 0)
    print("| kernel | calls | avg us | min us | max us | % time |\n|---|---:|---:|---:|---:|---:|")
    for r in sorted(rows, key=key, reverse=True)[:top]:
        name = r["Name"]
        name = name[:90] + ("..." if len(name) > 90 else "")
        print(f"| `{name}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | {float(r['MinNs']) / 1e3:.2f} | "
              f"{float(r['MaxNs']) / 1e3:.2f} | {float(r['Percentage']):.1f} |")


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[1])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--configs", default="1,2,3,4,5,q6k_head")
    ap.add_argument("--rotate-mb", type=int, default=1024, help="distinct weight bytes cycled per projection")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--traffic", default=os.path.join(ROOT, "profiles", "traffic.json"),
                    help="HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE, WRITE_SIZE)")
    ap.add_argument("--pmc-probe", action="store_true", help="only the headline kernel + a calibration copy (for --pmc)")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="write --traffic from the two --pmc runs of --pmc-probe")
    ap.add_argument("--summarize-stats", metavar="KERNEL_STATS_CSV", help="print a rocprofv3 --stats CSV as markdown")
    a = ap.parse_args()
    if a.summarize_pmc:
        return summarize_pmc(a.summarize_pmc[0], a.summarize_pmc[1], a.traffic)
    if a.summarize_stats:
        return summarize_stats(a.summarize_stats)
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py runs on one GPU: this path is measured on a single MI355X (its kernels shard by weight rows "
              "with no collective; see DESIGN.md). --gpus must be 1.", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    if a.pmc_probe:
        return pmc_probe()
    configs = [int(c) if c.isdigit() else c for c in a.configs.split(",") if c]
    if HEADLINE not in configs:
        configs.insert(0, HEADLINE)
    res = {}
    for c in configs:
        res[c] = run_config(c, a.steps, a.warmup, a.rotate_mb << 20)
    head = res[HEADLINE]
    proj = head["projections"]["w"]
    traffic = None
    try:
        with open(a.traffic) as f:
            traffic = json.load(f).get("c2", {}).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        traffic = None
    line = {
        "metric": METRIC, "value": head["GBps"], "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(head["us_per_step"] / 1e3, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded, BASELINE config value ranges, generated on the GPU)",
        "config": {"workload": "config 2: GGUF Q8_0 decode GEMV x bf16[1,5120] @ W[17408,5120]^T, fp32 accumulate, "
                               "bf16 out", "M": 1, "N": 17408, "K": 5120, "weight_type": "Q8_0",
                   "rotation_MB": proj["rotation_MB"]},
        "roofline": {"bound": "hbm", "achieved": head["GBps"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(head["GBps"] / PEAK_HBM_GBS, 4), "traffic": traffic,
                     "kernel": "mbq::gemv_kernel (Q8_0, 1 activation row)", "kernel_us": proj["us"],
                     "algorithmic_bytes_per_launch": head["algorithmic_bytes"]},
        "configs": {(f"c{c}" if isinstance(c, int) else c): {k: v for k, v in r.items() if k != "projections"}
                    | {"projections": r["projections"]} for c, r in res.items()},
    }
    line["measured_peaks"] = measured_peaks()
    if not a.no_cpu:
        line["cpu_baseline"] = cpu_baseline(a.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
