"""bench.py's host-side contract, on the CPU: a multi-GPU request exits with
a message (this build runs on one GPU); a CPU baseline record carries the
fields the bench line reports (value, unit, cores, kind, sample and the
per-op times it sets against the GPU's) and the reference's outputs the
parity leg compares with; and the stdout line stays under the size the
driver reads whole, parses, and holds every contract field, however long the
configurations' records are."""
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_cpu_baseline_record_fields():
    import bench
    rec, outs = bench.cpu_baseline_c1(reps=1)
    assert rec["unit"] == "GB/s" and rec["kind"] == "reference" and rec["cores"] == 1
    assert rec["value"] > 0 and "single-threaded" in rec["sample"]
    assert set(rec["per_op_ms_full"]) == {"add fwd", "relu fwd", "sum(1) fwd", "sum() fwd", "sum() bwd",
                                          "sum(1) bwd", "relu bwd", "add bwd"}
    assert all(v > 0 for v in rec["per_op_ms_full"].values())
    assert "sample_MiB" in rec and "sample_exceeds_llc" in rec
    # the reference's outputs on the recipe's bytes, for the parity leg
    assert outs["t"].size == 1024 * 1024 and outs["gb"].size == 1024
    assert float(outs["y"].reshape(-1)[0]) > 0


def _record(i, long=False):
    s = "x" * (600 if long else 120)
    rec = {"workload": "c%d: " % i + s, "elements": 268435456, "value": 6000.0 + i, "unit": "GB/s",
           "pct_of_peak": 75.0, "value_event": 5800.0, "basis": "trace", "ms_per_step": 1.234567,
           "roofline": {"bound": "hbm", "achieved": 6100.0, "peak": 8000.0, "unit": "GB/s", "frac": 0.7625,
                        "traffic": 1073741824, "kernel": "softmax_bwd_kernel<true, 4>" + s[:40],
                        "op": "softmax bwd", "algorithmic_bytes": 4194304000, "ms": 0.6789},
           "cpu_baseline": {"value": 1.2345, "unit": "GB/s", "cores": 1, "kind": "reference",
                            "sample": "logits[64,32000] row slice of config 4 " + s + "; median of 3 ...",
                            "per_op_ms_full": {"op%d" % k: 1.0 for k in range(20)}},
           "speedup_vs_cpu_step": 4321.0,
           "below_70pct": ["op name %d" % k for k in range(12 if long else 2)],
           "parity": {"pass": not long, "checks": 40,
                      "fail": ["a long failing check name %d" % k for k in range(30 if long else 0)]}}
    return rec


def test_bench_line_fits_and_parses():
    import argparse

    import bench
    args = argparse.Namespace(steps=20, warmup=5)
    for long in (False, True):
        recs = {nm: _record(i, long) for i, nm in enumerate(bench.ALL)}
        line = bench.bench_line(recs[bench.ALL[0]], recs, bench.ALL, args, 256, "trace",
                                {"wm_copy_kernel": 6400.0})
        text = json.dumps(line)
        assert len(text.encode()) <= bench.LINE_LIMIT, len(text)
        back = json.loads(text)
        for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                    "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
            assert key in back, key
        for key in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
            assert key in back["roofline"], key
        for key in ("value", "unit", "cores", "kind", "sample"):
            assert key in back["cpu_baseline"], key
        assert "workload" in back["config"]
        assert set(back["configs"]) == set(bench.ALL[1:])
        for rec in back["configs"].values():
            assert {"value", "pct", "ms_per_step", "roofline", "cpu_baseline", "parity"} <= set(rec)
            assert {"op", "frac", "ms", "algorithmic_bytes"} <= set(rec["roofline"])
            assert {"value", "cores"} <= set(rec["cpu_baseline"])


def test_headline_is_the_largest_config():
    import bench
    assert bench.ALL[0] == "c4"


def test_dispatch_tracer_library_exports():
    """libwm_ktrace (bench.py's trace-basis timer) loads and exports its entry
    points; registering it needs no GPU (it only configures rocprofiler-sdk),
    and an empty window takes no dispatches."""
    path = os.path.join(ROOT, "whitematter_amd", "libwm_ktrace.so")
    assert os.path.exists(path), "build() makes libwm_ktrace.so"
    r = subprocess.run([sys.executable, "-c", f"""
import ctypes
L = ctypes.CDLL({path!r})
for fn in ("wm_ktrace_init", "wm_ktrace_error", "wm_ktrace_begin", "wm_ktrace_end", "wm_ktrace_take",
           "wm_ktrace_name"):
    getattr(L, fn)
assert L.wm_ktrace_init() == 0
n = ctypes.c_int(-1)
assert L.wm_ktrace_begin() == 0 and L.wm_ktrace_end(ctypes.byref(n)) == 0 and n.value == 0
assert L.wm_ktrace_take(100, None, 0) == 0
print("ok")
"""], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stderr[-2000:]
