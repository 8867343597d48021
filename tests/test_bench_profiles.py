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
NAMES = sorted(set(bench.TRAFFIC_PROFILES.values()) | set(bench.F16_PROFILES.values()) |
               {traffic for traffic, _ in bench.PQ_PROFILES.values()})


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
    # the headline's sampled path at k = 10 has no traffic summary; at k = 100 (its default
    # path there, a default-run extra) it has one
    assert (3, 1_000_000, 10_000, 10, "collect-sampled") not in bench.TRAFFIC_PROFILES
    name = bench.TRAFFIC_PROFILES[(3, 1_000_000, 10_000, 100, "collect-sampled")]
    assert bench.read_traffic(name, True) > 512_000_000


@pytest.mark.parametrize("argv,env", [(["--gpus", "2"], {}), ([], {"WORLD_SIZE": "8"})])
def test_bench_refuses_more_than_one_gpu(argv, env):
    root = Path(bench.__file__).resolve().parent
    run = subprocess.run([sys.executable, str(root / "bench.py"), *argv], capture_output=True,
                         text=True, timeout=120, env={**os.environ, **env})
    assert run.returncode == 2
    assert "one GPU only" in run.stderr and run.stdout == ""


@pytest.mark.parametrize("name", sorted(set(bench.COUNTER_PROFILES.values())))
def test_mfma_counter_profile_is_complete(name):
    text = (PROFILES / name).read_text()
    assert "rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_VALU_MFMA_MOPS_F32" in text
    ctr = bench.read_counters(name, True)
    assert 0 < ctr["mfma_busy_frac"] < 1 and ctr["mfma_flop_per_launch"] > 0
    assert 1.0 < ctr["shader_clock_ghz"] < 2.5
    assert bench.read_counters(name, False) is None


@pytest.mark.parametrize("name", sorted(set(bench.F16_PROFILES.values())))
def test_f16_counter_profile_is_complete(name):
    text = (PROFILES / name).read_text()
    assert "rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES" in text and "rocprofv3 --pmc SQ_INSTS_LDS" in text
    ctr = bench.read_counters(name, True)
    assert 0 < ctr["mfma_busy_frac"] < 1 and 0 < ctr["lds_busy_frac"] < 1
    assert 1.0 < ctr["shader_clock_ghz"] < 2.5


@pytest.mark.parametrize("masked", [False, True])
def test_lds_counter_profile_is_complete(masked):
    name = bench.PQ_PROFILES[masked][1]
    text = (PROFILES / name).read_text()
    assert "rocprofv3 --pmc SQ_INSTS_LDS SQ_LDS_BANK_CONFLICT" in text
    ctr = bench.read_counters(name, True)
    assert 0 < ctr["lds_busy_frac"] < 1 and ctr["lds_bank_conflict_per_cycle"] > 0
    assert 0 < ctr["lds_roofline_frac"] < 1


def test_lds_rate_profile_is_complete():
    # the PQ scan's roofline: the LDS read rates measured by bench.py --workload lds
    text = (PROFILES / bench.LDS_PROFILE).read_text()
    assert "python bench.py --workload lds" in text and "rocprofv3 --kernel-trace --stats" in text
    ctr = bench.read_counters(bench.LDS_PROFILE, True)
    assert ctr["lds_conflict_free_gbs"] > ctr["lds_random_gather_gbs"] > 0


def test_host_cpu_names_the_host():
    h = bench.host_cpu()
    assert h["nproc"] >= 1 and isinstance(h["cpu_model"], str) and h["cpu_model"]
