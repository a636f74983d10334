"""CPU checks of bench.py's side of the driver contract: the one-GPU rule and
the HBM-traffic figures it reads from the committed counter summary."""
import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, REPO)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0
    assert "one GPU" in r.stderr and r.stdout == ""


@pytest.mark.parametrize("op", ["gateup", "down", "head", "hybrid_gateup", "hybrid_down"])
def test_traffic_of_the_roofline_ops_is_read_from_the_profile(op):
    import bench

    t = bench.read_traffic(op)
    assert isinstance(t, int) and t > 0
    # the counters see about the algorithmic bytes (GGUF weight bytes + f32
    # vectors): within 2 % for the matvecs
    alg = {"gateup": 2 * bench.gguf_bytes(bench.Q4_K, 5120, 27648) + 2 * 5120 * 4 + 27648 * 4,
           "down": bench.gguf_bytes(bench.Q6_K, 27648, 5120) + 27648 * 4 + 2 * 5120 * 4,
           "head": bench.gguf_bytes(bench.Q6_K, 5120, 152064) + 2 * 5120 * 4 + 152064 * 4,
           "hybrid_gateup": 2 * bench.gguf_bytes(bench.Q4_K, 5120, 17408) + 2 * 5120 * 4 + 17408 * 4,
           "hybrid_down": bench.gguf_bytes(bench.Q6_K, 17408, 5120) + 17408 * 4 + 2 * 5120 * 4}[op]
    assert 1.0 <= t / alg < 1.02, (op, t, alg)


def test_unknown_op_has_no_traffic():
    import bench

    assert bench.read_traffic("no_such_op") is None


def test_cpu_baseline_uses_a_native_timing_build_and_reports_the_host():
    """The CPU baselines run the oracle sources built with -O3 -march=native
    on the timing host (in a child process: the switch is process-wide), and
    report nproc, the CPU model and the NUMA layout; the timing build agrees
    with the exact parity build to f32 rounding."""
    code = (
        "import sys, json; sys.path.insert(0, %r); sys.path.insert(0, %r)\n"
        "import numpy as np, oracle\n"
        "w = oracle.gen_weight(12, 3, 64, 1024); x = oracle.gen_normal(4, 1024)\n"
        "exact = oracle.matvec(12, w, 1024, 64, x)\n"
        "import bench\n"
        "o = bench.cpu_oracle()\n"
        "fast = o.matvec(12, w, 1024, 64, x, threads=2)\n"
        "rel = float(np.linalg.norm(fast - exact) / np.linalg.norm(exact))\n"
        "print(json.dumps(dict(path=o.LIB_PATH, rel=rel, info=bench.host_info(2))))\n"
    ) % (REPO, os.path.join(REPO, "tests"))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    import json

    d = json.loads(r.stdout.strip().splitlines()[-1])
    assert d["path"].endswith("liblrs_oracle_timing.so") and "/oracle/" not in d["path"]
    assert d["rel"] < 1e-5
    info = d["info"]
    assert info["nproc"] >= 1 and info["threads_used"] == 2 and "-march=native" in info["build"]
    assert "cpu_model" in info and isinstance(info["numa_nodes"], dict)
