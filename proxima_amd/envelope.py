"""Benchmark result envelopes in the reference's artefact format (schema_version 1).

The reference writes its benchmark results as JSON envelopes: the Python harness as
``{"schema_version", "provenance", "results": [BenchResult...]}`` (bench/harness.py:19-40,
157-198) and the GPU example as ``{"schema_version", "provenance", "workload", "results"}``
(crates/core/examples/gpu_knn.rs:274-333, e.g. bench/results/gpu.json). This module builds
both shapes so that results from this backend sit beside bench/results/*.json. Provenance
carries the same fields; the GPU block names the HIP device (arch instead of a CUDA compute
capability, HIP runtime/driver versions instead of CUDA's) and adds its compute-unit count.
"""
from __future__ import annotations

import ctypes
import json
import os
import platform
import socket
import subprocess
import sys
from dataclasses import asdict, dataclass
from datetime import datetime, timezone
from pathlib import Path

SCHEMA_VERSION = 1
_REPO = Path(__file__).resolve().parent.parent


@dataclass
class BenchResult:
    """One row of a harness envelope (the fields of bench/harness.py:25-40)."""
    name: str
    n_base: int
    dim: int
    k: int
    recall_at_k: float | None
    p50_ms: float
    p99_ms: float
    mean_ms: float
    qps_1t: float
    qps_mt: float
    memory_mb: float
    latency_samples: int = 0
    build_seconds: float | None = None

    def as_dict(self) -> dict:
        return asdict(self)


def _quiet(fn, default=None):
    try:
        value = fn()
    except Exception:
        return default
    return default if value is None else value


def _cmd(*argv: str) -> str | None:
    try:
        out = subprocess.run(list(argv), cwd=_REPO, capture_output=True, text=True, timeout=20)
    except Exception:
        return None
    return out.stdout.strip() if out.returncode == 0 else None


def _cpu_model() -> str:
    with open("/proc/cpuinfo") as fh:
        for line in fh:
            if line.lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    return platform.processor() or "unknown"


def _physical_cores() -> int | None:
    cores = set()
    package = None
    with open("/proc/cpuinfo") as fh:
        for line in fh:
            if line.startswith("physical id"):
                package = line.split(":", 1)[1].strip()
            elif line.startswith("core id"):
                cores.add((package, line.split(":", 1)[1].strip()))
    return len(cores) or None


def _git() -> dict:
    status = _cmd("git", "status", "--porcelain")
    return {"sha": _cmd("git", "rev-parse", "HEAD"),
            "branch": _cmd("git", "rev-parse", "--abbrev-ref", "HEAD"),
            "dirty": None if status is None else bool(status)}


def gpu_info(device: int = 0) -> dict | None:
    """The HIP device block of the provenance; None without the library or a device."""
    from . import _lib

    try:
        lib = _lib.load()
        count = _lib.device_count()
    except Exception:
        return None
    if count < 1:
        return None
    info = _lib.device_info(device)
    runtime, driver = ctypes.c_int(0), ctypes.c_int(0)
    have = lib.px_hip_versions(ctypes.byref(runtime), ctypes.byref(driver)) == 0
    return {"device_index": device, "device_count": count, "name": info["name"],
            "arch": info["arch"],
            "hip_driver_version": str(driver.value) if have else None,
            "hip_runtime_version": str(runtime.value) if have else None,
            "total_vram_bytes": info["hbm_bytes"], "compute_units": info["cus"]}


def collect_provenance(argv: list[str] | None = None, gpu: bool = True) -> dict:
    """Where and how a result was produced (the keys of bench/harness.py:157-182, plus
    the GPU block of gpu_knn.rs:287-295 when ``gpu``)."""
    import numpy

    from . import __version__

    prov = {
        "timestamp_utc": datetime.now(timezone.utc).strftime("%Y-%m-%dT%H:%M:%SZ"),
        "hostname": _quiet(platform.node) or _quiet(socket.gethostname) or "unknown",
        "argv": list(sys.argv if argv is None else argv),
        "os": {"platform": _quiet(platform.platform), "system": _quiet(platform.system),
               "release": _quiet(platform.release), "machine": _quiet(platform.machine)},
        "cpu": {"model": _quiet(_cpu_model, "unknown"), "cores_physical": _quiet(_physical_cores),
                "cores_logical": _quiet(os.cpu_count)},
    }
    if gpu:
        prov["gpu"] = _quiet(gpu_info)
    prov["git"] = _quiet(_git, {})
    prov["versions"] = {"python": platform.python_version(), "numpy": numpy.__version__,
                        "proxima_amd": __version__,
                        "hipcc": _quiet(lambda: (_cmd("/opt/rocm/bin/hipcc", "--version") or "")
                                        .splitlines()[0] or None)}
    return prov


def results_envelope(results: list[BenchResult], argv: list[str] | None = None) -> dict:
    """The harness envelope (bench/harness.py:185-190)."""
    return {"schema_version": SCHEMA_VERSION, "provenance": collect_provenance(argv, gpu=False),
            "results": [r.as_dict() for r in results]}


def gpu_envelope(*, n_base: int, dim: int, n_queries: int, k: int, metric: str,
                 gpu_seconds: float, reps: int, cpu_mt_seconds: float | None = None,
                 cpu_1t_seconds: float | None = None, topk_agreement: float | None = None,
                 argv: list[str] | None = None) -> dict:
    """The GPU example's envelope (gpu_knn.rs:314-333): seconds are per search of the
    whole n_queries batch; rates and speed-ups follow from them as there."""
    def rate(sec):
        return None if not sec else n_queries / sec

    def ratio(sec):
        return None if not sec or not gpu_seconds else sec / gpu_seconds

    return {
        "schema_version": SCHEMA_VERSION,
        "provenance": collect_provenance(argv, gpu=True),
        "workload": {"n_base": n_base, "dim": dim, "n_queries": n_queries, "k": k,
                     "metric": metric},
        "results": {"cpu_1t_seconds": cpu_1t_seconds, "cpu_1t_qps": rate(cpu_1t_seconds),
                    "cpu_mt_seconds": cpu_mt_seconds, "cpu_mt_qps": rate(cpu_mt_seconds),
                    "gpu_seconds": gpu_seconds, "gpu_qps": rate(gpu_seconds),
                    "speedup_vs_cpu_1t": ratio(cpu_1t_seconds),
                    "speedup_vs_cpu_mt": ratio(cpu_mt_seconds),
                    "reps": reps, "topk_agreement": topk_agreement},
    }


def write_envelope(path, envelope: dict) -> Path:
    """Write an envelope as indented JSON (bench/harness.py:193-197)."""
    out = Path(path)
    out.parent.mkdir(parents=True, exist_ok=True)
    out.write_text(json.dumps(envelope, indent=2) + "\n")
    return out
