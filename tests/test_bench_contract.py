"""The bench's contract on the host (no GPU): one GPU only, and the roofline traffic it
reports comes from the committed rocprofv3 counter summary and matches the north-star
workload's algorithmic bytes."""

import subprocess
import sys
from pathlib import Path

import oracle
from aiproj_amd import workloads

ROOT = Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_is_refused_before_any_device_work():
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True,
                          text=True, timeout=120)
    assert proc.returncode == 2
    assert "one GPU" in proc.stderr
    assert proc.stdout == ""


def test_traffic_comes_from_the_committed_profile_and_fits_the_bytes():
    sys.path.insert(0, str(ROOT))
    import bench

    traffic = bench.traffic_for("decode_mfma_kernel", "north")
    assert isinstance(traffic, int)
    s = workloads.spec("north")
    algorithmic = oracle.decode_algorithmic_bytes(s.lengths, s.num_q_heads, s.num_kv_heads, s.head_dim,
                                                  s.block_size)
    assert algorithmic == 277_381_120
    # HBM bytes per launch: the algorithmic bytes plus the split-K partial states, q and the
    # tile prefix, a few percent more.
    assert 1.0 <= traffic / algorithmic < 1.05
    assert bench.traffic_for("decode_mfma_kernel", "no_such_workload") is None
