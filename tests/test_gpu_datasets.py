"""SIFT1M-format data through the GPU FlatIndex (bench/bench_sift.py:44-60): TEXMEX files
written from synthetic SIFT-like data, ground truth from the oracle, recall from the
reference's definition (bench/harness.py:210-218). SIFT1M itself is not available offline;
`bench.py --sift DIR` runs the same path on it."""
import json
import os
import subprocess
import sys

import numpy as np

import oracle
from proxima_amd import Metric, datagen, datasets

import pytest

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _write_sift(tmp_path, n=20_000, nq=64, k=100):
    base = datagen.sift_like(n, 128, 81)
    q = datagen.sift_like(nq, 128, 82)
    gt, _, _ = oracle.flat_search(base, q, k, oracle.L2)
    datasets.write_fvecs(tmp_path / "sift_base.fvecs", base)
    datasets.write_fvecs(tmp_path / "sift_query.fvecs", q)
    datasets.write_ivecs(tmp_path / "sift_groundtruth.ivecs", gt.astype(np.int32))
    return gt


def test_sift_files_exact_ground_truth(gpu, tmp_path):
    gt = _write_sift(tmp_path)
    ds = datasets.load_sift(tmp_path)
    ids = datasets.exact_ground_truth(ds.base, ds.queries, 100, Metric.L2)
    assert np.array_equal(ids, gt)
    assert datasets.recall_at_k(ids, ds.ground_truth, 100) == 1.0
    assert datasets.recall_at_k(ids[:, :10], ds.ground_truth, 10) == 1.0


def test_bench_sift_mode(gpu, tmp_path):
    _write_sift(tmp_path, n=12_000, nq=300)
    env_path = tmp_path / "env.json"
    out = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--sift", str(tmp_path),
                          "--steps", "2", "--warmup", "1", "--cpu-seconds", "1",
                          "--envelope", str(env_path)],
                         capture_output=True, text=True, timeout=240)
    assert out.returncode == 0, out.stderr[-2000:]
    line = json.loads(out.stdout.strip().splitlines()[-1])
    assert line["recall_at_k"] == 1.0
    assert line["parity_sample"]["id_mismatches"] == 0
    env = json.loads(env_path.read_text())
    assert env["schema_version"] == 1 and env["workload"]["n_base"] == 12_000
    assert env["results"]["topk_agreement"] == 1.0
    assert env["provenance"]["gpu"]["arch"].startswith("gfx950")
