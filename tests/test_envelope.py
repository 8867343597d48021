"""Benchmark envelopes in the reference's artefact format (CPU only).

tests/golden/envelope_keys.json holds the key structure of the reference's committed
artefacts bench/results/gpu.json and bench/results/sift1m.json (written by
tests/golden/make_envelope_keys.py). This backend's envelopes must carry every key they
carry, except the CUDA-specific GPU fields, which name the HIP device instead, and the
interpreter versions, which name this build's tools.
"""
import json
from pathlib import Path

import pytest

from proxima_amd import envelope

KEYS = json.loads((Path(__file__).resolve().parent / "golden" / "envelope_keys.json").read_text())
CUDA_ONLY = {"compute_capability", "cuda_driver_version", "cuda_runtime_version"}
HIP_GPU = {"device_index", "device_count", "name", "arch", "hip_driver_version",
           "hip_runtime_version", "total_vram_bytes", "compute_units"}


def _has_keys(ours, ref, path="", skip=("versions",)):
    for key, sub in ref.items():
        if key in skip:
            continue
        assert key in ours, f"missing {path}{key}"
        if isinstance(sub, dict):
            if key == "gpu":
                continue
            _has_keys(ours[key], sub, f"{path}{key}.", skip)


def test_gpu_envelope_matches_reference_layout():
    env = envelope.gpu_envelope(n_base=1_000_000, dim=128, n_queries=10_000, k=10, metric="L2",
                                gpu_seconds=0.025, reps=5, cpu_mt_seconds=12.5,
                                topk_agreement=1.0, argv=["bench.py"])
    _has_keys(env, KEYS["gpu"])
    assert set(env) == set(KEYS["gpu"])
    assert set(env["workload"]) == set(KEYS["gpu"]["workload"])
    assert set(env["results"]) == set(KEYS["gpu"]["results"])
    ref_gpu = set(KEYS["gpu"]["provenance"]["gpu"])
    assert ref_gpu - CUDA_ONLY <= HIP_GPU
    assert env["schema_version"] == 1
    r = env["results"]
    assert r["gpu_qps"] == pytest.approx(10_000 / 0.025)
    assert r["cpu_mt_qps"] == pytest.approx(10_000 / 12.5)
    assert r["speedup_vs_cpu_mt"] == pytest.approx(500.0)
    assert r["cpu_1t_seconds"] is None and r["speedup_vs_cpu_1t"] is None
    # no device in this container: the gpu block is null rather than an error
    gpu = env["provenance"]["gpu"]
    assert gpu is None or set(gpu) == HIP_GPU
    json.loads(json.dumps(env))


def test_harness_envelope_matches_reference_layout(tmp_path):
    row = envelope.BenchResult(name="flat_gpu", n_base=1000, dim=8, k=10, recall_at_k=1.0,
                               p50_ms=0.1, p99_ms=0.2, mean_ms=0.12, qps_1t=1e4, qps_mt=1e5,
                               memory_mb=0.03)
    env = envelope.results_envelope([row], argv=["x"])
    _has_keys(env, KEYS["sift1m"])
    assert set(env["results"][0]) == set(KEYS["sift1m"]["results"][0])
    assert "gpu" not in env["provenance"]
    prov = env["provenance"]
    assert len(prov["timestamp_utc"]) == 20 and prov["timestamp_utc"].endswith("Z")
    assert prov["argv"] == ["x"]
    path = envelope.write_envelope(tmp_path / "sub" / "r.json", env)
    back = json.loads(path.read_text())
    assert back["results"][0]["name"] == "flat_gpu" and back["schema_version"] == 1
