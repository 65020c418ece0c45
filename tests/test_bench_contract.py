"""bench.py's command line: one GPU only (more exits with a message and code
2 before touching a GPU), and the cost model's byte and flop counts of the
measured wave."""
import json
import subprocess
import sys
from pathlib import Path

import numpy as np

from specgrove_amd import workloads as W

ROOT = Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout.strip() == ""


def test_measured_wave_bytes_and_flops():
    wl = W.qwen3_8b_workload()
    assert wl.num_requests == 64 and wl.total_rows == 2048
    assert int(wl.prefix_len.sum()) == 138564
    # prefix K+V (512 B per token per kv head) + Q, O and tree K/V per row
    # (20,480 B) + 4-byte metadata per row and three per request
    want = 138564 * 8 * 512 + 2048 * 20480 + 4 * (2048 + 3 * 64)
    assert wl.algorithmic_bytes() == want
    depths = [W.depths_of(p) for p in wl.parents]
    visible = sum(len(p) * int(L) + sum(d + 1 for d in ds)
                  for p, L, ds in zip(wl.parents, wl.prefix_len, depths))
    assert wl.algorithmic_flops() == 4 * 32 * 128 * visible
    assert np.all(wl.prefix_len >= 512) and np.all(wl.prefix_len <= 4096)
