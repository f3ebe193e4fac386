"""bench.py's one JSON line, built on the CPU from stub results: it carries the contract's fields, stays well under the
8,000 characters a driver keeps of stdout (4,000 here, leaving room for the stderr summary after it), and every
figure is the median of at least 100 timed launches whatever --steps is."""
import json

import bench

CONFIGS = list(bench._configs(bench.DEFAULT_CONFIGS))       # every config a default run times
PROJ = ["q", "k", "v", "o", "gate", "up", "down"]


def _stub(c, steps):
    projs = {"w": None} if c in (1, 2, 3, "q6k_head", "c2_ops", "q4k_9728", "q2k_9728") else dict.fromkeys(PROJ)
    p = {name: {"M": 16, "N": 17408, "K": 5120, "us": 123.456, "mean_us": 124.5, "GBps": 1234.5, "TFLOPs": 12.34,
                "eager_call_us": 23.45, "rotation_copies": 18, "rotation_MB": 1103.0,
                "plan": "kgroup 16x68/1"} for name in projs}
    return {"projections": p, "type": "Q4_K", "M": 16, "us_per_step": 1478.612, "mean_us_per_step": 1480.1,
            "launches_timed": bench.replays_for(steps) * steps, "GBps": 4908.12, "hbm_frac": 0.61351,
            "TFLOPs": 944.03, "mfma_frac": 0.37761, "eager_us_per_step": 1500.2, "algorithmic_bytes": 94740480,
            "flops": 1396000000000,
            **({"reference_tpu_v6e_us": 369.8, "speedup_vs_reference_tpu_v6e": 6.51} if c in bench_ref() else {})}


def bench_ref():
    from mashbox_amd import synth
    return set(synth.REF_TPU_US)


def test_line_is_short_and_complete():
    for steps in (1, 20, 200):
        res = {c: _stub(c, steps) for c in CONFIGS}
        traffic = {f"c{i}": {"hbm_bytes_per_launch": 95000000} for i in range(1, 6)}
        peaks = {"read_GBps": 5745.0, "copy_GBps": 4941.6, "mfma_bf16_TFLOPs": 2275.5, "how": "x" * 300}
        per = {f"c{i}": {"us_per_step": 14731.5, "GBps": 6.431, "TFLOPs": 0.0121, "calls": 258} for i in range(1, 6)}
        line, detail = bench.make_line(res, traffic, peaks, (per, 16), steps, 5, "/tmp/bench_detail.json")
        text = json.dumps(line, separators=(",", ":"))
        assert len(text) < 4000, len(text)
        back = json.loads(text)
        for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
                  "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
            assert k in back, k
        assert back["config"]["workload"].startswith("config 2")
        assert set(back["roofline"]) >= {"bound", "achieved", "peak", "unit", "frac", "traffic"}
        assert set(back["cpu_baseline"]) >= {"value", "unit", "cores", "kind", "sample"}
        assert len(back["configs"]) == len(CONFIGS)
        assert all("x_ref_tpu" in back["configs"][c] for c in bench_ref())
        assert bench.replays_for(steps) * steps >= 100 and bench.replays_for(steps) >= 5
        assert "projections" in detail["configs"]["c4"]
