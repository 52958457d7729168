"""bench.py's host-side contract, on the CPU: a multi-GPU request exits with
a message (this build runs on one GPU), and a CPU baseline record carries
the fields the bench line reports (value, unit, cores, kind, sample and the
per-op times it sets against the GPU's)."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_cpu_baseline_record_fields():
    sys.path.insert(0, ROOT)
    import bench
    rec = bench.cpu_baseline_c1(reps=1)
    assert rec["unit"] == "GB/s" and rec["kind"] == "reference" and rec["cores"] == 1
    assert rec["value"] > 0 and "single-threaded" in rec["sample"]
    assert set(rec["per_op_ms_full"]) == {"add fwd", "relu fwd", "sum(1) fwd", "sum() fwd", "sum() bwd",
                                          "sum(1) bwd", "relu bwd", "add bwd"}
    assert all(v > 0 for v in rec["per_op_ms_full"].values())
