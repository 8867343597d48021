"""bench.py's `traffic` comes from committed rocprofv3 summaries (CPU only).

Each summary that bench.py reads must exist, state the command that produced it and carry
the `avg_kernel_ms:` and `hbm_bytes_per_launch:` lines; a run of another workload or path
reports null rather than a figure measured on something else. bench.py measures one GPU and
refuses a multi-GPU launch with exit status 2 before it touches a device.
"""
import os
import subprocess
import sys
from pathlib import Path

import pytest

import bench

PROFILES = Path(__file__).resolve().parent.parent / "profiles"
NAMES = sorted(set(bench.TRAFFIC_PROFILES.values()) | {"pq_scan_kernel_l2_1Mx16_q10k_k10.md"})


@pytest.mark.parametrize("name", NAMES)
def test_traffic_profile_is_complete(name):
    text = (PROFILES / name).read_text()
    assert "rocprofv3 --kernel-trace --stats" in text
    assert "rocprofv3 --pmc FETCH_SIZE" in text and "rocprofv3 --pmc WRITE_SIZE" in text
    lines = {ln.split(":", 1)[0]: ln.split(":", 1)[1] for ln in text.splitlines()
             if ln.startswith(("avg_kernel_ms:", "hbm_bytes_per_launch:"))}
    assert float(lines["avg_kernel_ms"]) > 0
    traffic = bench.read_traffic(name, True)
    assert traffic == int(float(lines["hbm_bytes_per_launch"])) and traffic > 0


def test_traffic_only_for_the_profiled_run():
    name = bench.TRAFFIC_PROFILES[(3, 1_000_000, 10_000, 10, "collect-bounded")]
    assert bench.read_traffic(name, False) is None
    assert bench.read_traffic("", True) is None
    assert bench.read_traffic("no_such_profile.md", True) is None
    # the headline's sampled path and other workloads have no traffic summary
    assert (3, 1_000_000, 10_000, 10, "collect-sampled") not in bench.TRAFFIC_PROFILES
    assert (3, 1_000_000, 10_000, 100, "collect-sampled") not in bench.TRAFFIC_PROFILES


@pytest.mark.parametrize("argv,env", [(["--gpus", "2"], {}), ([], {"WORLD_SIZE": "8"})])
def test_bench_refuses_more_than_one_gpu(argv, env):
    root = Path(bench.__file__).resolve().parent
    run = subprocess.run([sys.executable, str(root / "bench.py"), *argv], capture_output=True,
                         text=True, timeout=120, env={**os.environ, **env})
    assert run.returncode == 2
    assert "one GPU only" in run.stderr and run.stdout == ""
