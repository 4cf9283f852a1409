"""The parts of bench.py's output contract that need no GPU.

- It refuses to run on more than one GPU, before touching one.
- The algorithmic byte counts behind `value` and `roofline.achieved`.
- The dispatch statistics it reports.
- The committed counter figures it reads for `roofline.traffic`, checked
  against the summaries they come from.
"""
import json
import os
import re
import subprocess
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402


def test_refuses_more_than_one_gpu():
    for args, env in ((["--gpus", "2"], {}), ([], {"WORLD_SIZE": "2"})):
        r = subprocess.run([sys.executable, str(ROOT / "bench.py")] + args,
                           env=dict(os.environ, **env), capture_output=True, text=True,
                           timeout=120)
        assert r.returncode == 2, r.stderr
        assert "single" in r.stderr and "--gpus 1" in r.stderr
        assert r.stdout == ""  # no JSON line


def test_algorithmic_bytes():
    # K*N/2 packed nibbles + N*ceil(K/bs) fp32 scales + M*K fp32 activations
    # + M*N fp32 outputs
    head = 4096 * 4096 // 2 + 4096 * 32 * 4 + 4096 * 4 + 4096 * 4
    assert head == 8945664
    assert bench.mmnb_bytes(1, 4096, 4096, 128, False) == head
    # zero points: one nibble per (column, block), each column's padded to whole bytes
    bs32 = 4096 * 4096 // 2 + 4096 * 128 * 4 + 4096 * 4 + 4096 * 4 + 4096 * 64
    assert bench.mmnb_bytes(1, 4096, 4096, 32, True) == bs32 == 10780672
    # a ragged last block and an odd block count per column
    nb = -(-1000 // 64)
    assert bench.mmnb_bytes(3, 1000, 7, 64, True) == (
        1000 * 7 // 2 + 7 * nb * 4 + 3 * 1000 * 4 + 3 * 7 * 4 + 7 * ((nb + 1) // 2))


def test_dispatch_stats():
    s = bench.dispatch_stats([0.004, 0.002, 0.003, 0.010])  # ms
    assert s["count"] == 4
    assert np.isclose(s["median_us"], 3.5) and np.isclose(s["mean_us"], 4.75)
    assert np.isclose(s["min_us"], 2.0) and np.isclose(s["max_us"], 10.0)


def test_committed_traffic_matches_its_summaries():
    traffic = json.loads((ROOT / "profiles" / "traffic.json").read_text())
    for key in ("gemv_m1_k4096_n4096_bs128", "gemm_m512_k4096_n4096_bs32_zp"):
        t = traffic[key]
        assert bench.measured_traffic(key) == t["bytes_per_launch"]
        # bytes = (FETCH_SIZE * fetch scale + WRITE_SIZE * write scale) KiB
        want = (t["fetch_kib_raw"] * t["fetch_scale"] + t["write_kib_raw"] * t["write_scale"])
        assert abs(t["bytes_per_launch"] - want * 1024) <= 1024
        # the summary it names states the same figure (MB, two decimals)
        md = (ROOT / "profiles" / t["source"]).read_text()
        mb = [float(x) for x in re.findall(r"HBM traffic per launch: \*\*([0-9.]+) MB", md)]
        assert mb and abs(mb[0] - t["bytes_per_launch"] / 1e6) < 0.006
    assert bench.measured_traffic("no such workload") is None
