"""Direct oracle parity of every variant of the bounded collect scan on rows of 128 dims.

Batches of at least 256 queries with k + 8 <= 24 over at most 48 corpus splits take the
bounded first round: flat_collect_kernel with the splits' shared bound (DYN), no threshold
sample. Rows of exactly 128 padded dims run it in one of eight forms: L2 or inner product,
unfiltered or with a keep-mask, and multiplying in fp32 or (rows and queries exact in fp16)
in fp16. Each test below names the form it runs, forces it (px_flat_set_scan_f16 off for the
fp32 forms on integer data, whose values are exact in fp16) and asserts the path and the
multiply the search reports, so that a routing change cannot move a case off its kernel.

Workload: 200,000 x 128 rows (32 splits for 2,048 queries) of the SIFT-like integers of the
1M x 128 headline (flat.rs:106-148 restated by the oracle; sums of integer products are
exact in fp32, so ids and distances are bit-identical, ties included), and N(0,1) /
unit-Gaussian rows at the parity rule (ids identical except where two keys differ by less
than 1e-5 relative, distances within 1e-4). Filters keep 50% of 200,000 rows or 10% of
400,000 (the reference applies the mask before the distance, flat.rs:125-129; its tests
tests/test_engine.py:17-41 and tests/test_filter.py:33-42 compare result sets, here every
rank is compared).
"""
import numpy as np
import pytest

import oracle
from conftest import assert_parity
from proxima_amd import FlatIndex, Metric, datagen

pytestmark = pytest.mark.gpu

N, NQ, DIM = 200_000, 2048, 128
KS = (1, 10, 16)


def _key_of(data, queries, metric):
    def key_of(qi, row):
        if metric == oracle.L2:
            return float(oracle.l2_sqr(queries[qi], data[row]))
        return float(-oracle.inner_product(queries[qi], data[row]))
    return key_of


_cache = {}


def _workload(kind, rows, seed):
    key = (kind, rows, seed)
    if key not in _cache:
        gen = {"sift": datagen.sift_like, "gauss": datagen.gaussian,
               "unit": datagen.unit_gaussian}[kind]
        _cache[key] = (gen(rows, DIM, seed), gen(NQ, DIM, seed + 1))
    return _cache[key]


def _run(kind, metric, f16, density=None, rows=N, seed=300):
    data, q = _workload(kind, rows, seed)
    mask = datagen.mask(rows, density, seed + 2) if density is not None else None
    idx = FlatIndex(DIM, Metric.L2 if metric == oracle.L2 else Metric.InnerProduct)
    idx.add(data)
    idx._scan_f16(f16)
    # the oracle's canonical order puts the best k first for every k: one call serves all
    o_ids, o_d, _ = oracle.flat_search(data, q, max(KS), metric, mask=mask)
    exact = kind == "sift"
    for k in KS:
        print(f"case bounded {kind} metric={metric} f16={f16} density={density} rows={rows} "
              f"k={k}", flush=True)
        if mask is None:
            ids, d = idx.search_batch(q, k=k)
        else:
            ids, d = idx.search_batch_filtered(q, mask, k=k)
        t = idx._last_timing()
        assert t["path"] == "collect-bounded", t
        assert t["scan_f16"] == f16, t
        assert t["collect_rounds"] >= 1
        if exact:
            assert np.array_equal(ids, o_ids[:, :k]), k
            assert np.array_equal(d.view(np.uint32), o_d[:, :k].view(np.uint32)), k
        else:
            assert_parity(ids, d, o_ids[:, :k], o_d[:, :k], _key_of(data, q, metric))
    return idx


# ---- fp32 multiplies: the headline kernel's own form and its three siblings ----------

def test_fp32_l2_unfiltered_sift_like(gpu):
    # the headline workload's kernel (flat_collect_kernel<L2, unfiltered, DYN, fp32>) on a
    # fifth of its rows, k = 1 / 10 / 16, bit-exact
    _run("sift", oracle.L2, f16=False)


def test_fp32_l2_unfiltered_gaussian(gpu):
    _run("gauss", oracle.L2, f16=False, seed=310)


def test_fp32_ip_unfiltered_unit_gaussian(gpu):
    _run("unit", oracle.IP, f16=False, seed=320)


def test_fp32_ip_unfiltered_sift_like(gpu):
    _run("sift", oracle.IP, f16=False, seed=330)


@pytest.mark.parametrize("density,rows", [(0.5, N), (0.1, 2 * N)])
def test_fp32_l2_filtered_gaussian(gpu, density, rows):
    _run("gauss", oracle.L2, f16=False, density=density, rows=rows, seed=340)


def test_fp32_l2_filtered_sift_like(gpu):
    _run("sift", oracle.L2, f16=False, density=0.5, seed=350)


def test_fp32_ip_filtered_unit_gaussian(gpu):
    _run("unit", oracle.IP, f16=False, density=0.5, seed=360)


# ---- fp16 multiplies (rows and queries exact in fp16) ---------------------------------

def test_fp16_l2_unfiltered_sift_like(gpu):
    _run("sift", oracle.L2, f16=True, seed=370)


def test_fp16_ip_unfiltered_sift_like(gpu):
    _run("sift", oracle.IP, f16=True, seed=380)


def test_fp16_l2_filtered_sift_like(gpu):
    _run("sift", oracle.L2, f16=True, density=0.5, seed=390)


def test_fp16_ip_filtered_sift_like(gpu):
    _run("sift", oracle.IP, f16=True, density=0.1, rows=2 * N, seed=400)


def test_fp32_and_fp16_agree_bit_for_bit(gpu):
    # the same handle and queries through both multiplies: identical ids and distances
    data, q = _workload("sift", N, 410)
    idx = FlatIndex(DIM, Metric.L2)
    idx.add(data)
    out = {}
    for f16 in (False, True):
        idx._scan_f16(f16)
        out[f16] = idx.search_batch(q, k=10)
        assert idx._last_timing()["scan_f16"] == f16
        assert idx._last_timing()["path"] == "collect-bounded"
    assert np.array_equal(out[False][0], out[True][0])
    assert np.array_equal(out[False][1].view(np.uint32), out[True][1].view(np.uint32))
