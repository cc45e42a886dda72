"""bench.py's host side without a GPU: the single-GPU rule, the configs it offers, and the
algorithmic byte counts its roofline divides by (the per-launch figures quoted for c2:
159,712,768 B for the gate/up kernel with its router rows, 74,383,360 B for the down kernel,
234,008,064 B per layer)."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout.strip() == ""


def test_configs_cover_the_baseline_workloads():
    assert {"c1", "c2", "c3", "c4", "fp4"} <= set(bench.CONFIGS)
    c2 = bench.CONFIGS["c2"]
    assert (c2["hidden"], c2["inter"], c2["E"], c2["k"], c2["shared"]) == (7168, 2048, 384, 8, 1)


def test_c2_algorithmic_bytes():
    nb = bench.algorithmic_bytes(bench.CONFIGS["c2"], None)
    assert nb["gateup"] + nb["router"] == 159_712_768
    assert nb["down"] == 74_383_360
    assert nb["layer"] == 234_008_064
