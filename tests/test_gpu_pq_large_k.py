"""GPU parity of PqIndex searches with k > 128: the threshold-collect path.

The reference's PqIndex takes any k (pq.rs:299-347 keeps a heap of k). Past the per-wave
candidate lists the library samples a subset of the code rows spread evenly for per-query
thresholds, appends every row at or below them in one collect scan, and finishes each query
whose candidate set is complete and large enough; ADC keys are the reference's own sums
(pq.rs:320-323), so ids and distances are bit-identical to the oracle's with no re-rank.
The last two tests lay the codes out against the sample to force extra rounds.
"""
import ctypes

import numpy as np
import pytest

import oracle
from conftest import sample_positions
from proxima_amd import Metric, PqIndex, datagen

pytestmark = pytest.mark.gpu


def _index(data, m, nbits, metric, iters=4, sample=0):
    pq = PqIndex(data.shape[1], Metric.L2 if metric == oracle.L2 else Metric.InnerProduct,
                 m=m, nbits=nbits, train_iters=iters, train_sample=sample)
    pq.train(data)
    pq.add(data)
    return pq


def _rounds(pq) -> int:
    r = ctypes.c_int(-1)
    assert pq._lib.px_pq_last_rounds(pq._h, ctypes.byref(r)) == 0
    return r.value


def _check(pq, q, k, metric, mask=None):
    print(f"pq case n={len(pq)} nq={q.shape[0]} k={k} metric={metric} "
          f"mask={'yes' if mask is not None else 'no'}", flush=True)
    if mask is None:
        ids, d = pq.search_batch(q, k=k)
    else:
        ids, d = pq.search_batch_filtered(q, mask, k=k)
    o_ids, o_d, _ = oracle.pq_search(pq.codebooks(), pq.codes(), q, k, metric, mask=mask)
    assert np.array_equal(ids, o_ids)
    assert np.array_equal(d, o_d)
    return _rounds(pq)


@pytest.mark.parametrize("metric", [oracle.L2, oracle.IP])
@pytest.mark.parametrize("k", [128, 129, 700, 4096])
def test_pq_large_k_bit_exact(gpu, metric, k):
    data = datagen.gaussian(20_000, 64, 301)
    q = datagen.gaussian(40, 64, 302)
    pq = _index(data, 16, 8, metric)
    rounds = _check(pq, q, k, metric)
    assert (rounds == 0) == (k <= 128)


@pytest.mark.parametrize("m,nbits", [(8, 8), (6, 4)])
def test_pq_large_k_other_shapes_filtered(gpu, m, nbits):
    data = datagen.gaussian(30_000, 48, 303)
    q = datagen.gaussian(33, 48, 304)
    pq = _index(data, m, nbits, oracle.L2)
    mask = datagen.mask(30_000, 0.3, 305)
    _check(pq, q, 500, oracle.L2, mask=mask)
    _check(pq, q, 300, oracle.L2)


def test_pq_k_above_rows_pads(gpu):
    data = datagen.gaussian(700, 32, 306)
    q = datagen.gaussian(10, 32, 307)
    pq = _index(data, 8, 4, oracle.L2)
    _check(pq, q, 1500, oracle.L2)


@pytest.mark.parametrize("metric", [oracle.L2, oracle.IP])
def test_pq_full_sort_past_max_k(gpu, metric):
    # k past PX_MAX_K (the reference's PqIndex takes any k): every ADC key, sorted; bit for
    # bit, filtered or not, k above the rows padded
    data = datagen.gaussian(9000, 32, 308)
    q = datagen.gaussian(12, 32, 309)
    pq = _index(data, 8, 8, metric)
    _check(pq, q, 5000, metric)
    _check(pq, q, 4500, metric, mask=datagen.mask(9000, 0.6, 310))
    _check(pq, q, 9500, metric)


def _laid_out(near_on_sample: bool, seed: int):
    """4 x 16-centroid codebooks; codes near the query on the sampled rows and far from it
    elsewhere (or the other way round)."""
    n, k, m, nbits = 40_000, 992, 4, 4
    data = datagen.gaussian(4000, 32, seed)
    pq = PqIndex(32, Metric.L2, m=m, nbits=nbits, train_iters=4, train_sample=0)
    pq.train(data)
    books = pq.codebooks()                      # [m][16][8]
    q = datagen.gaussian(6, 32, seed + 1)
    # per subspace, the 4 centroids nearest to / farthest from the first query
    d = ((books - q[0].reshape(m, 1, 8)) ** 2).sum(-1)   # [m][16]
    order = np.argsort(d, axis=1, kind="stable")
    near, far = order[:, :4], order[:, -4:]
    rng = np.random.default_rng(seed + 2)
    pick = rng.integers(0, 4, size=(n, m))
    # ADC keys are exact, so the collect path keeps k candidates (no re-rank margin)
    on_sample = np.zeros(n, dtype=bool)
    on_sample[sample_positions(n, k)] = True
    codes = np.where(on_sample[:, None],
                     np.take_along_axis(near if near_on_sample else far, pick.T, 1).T,
                     np.take_along_axis(far if near_on_sample else near, pick.T, 1).T)
    pq.add_codes(codes.astype(np.uint8))
    return pq, q, k


def test_pq_sample_far_overflow_rounds(gpu):
    pq, q, k = _laid_out(near_on_sample=False, seed=310)
    assert _check(pq, q, k, oracle.L2) >= 2


def test_pq_sample_near_underflow_rounds(gpu):
    pq, q, k = _laid_out(near_on_sample=True, seed=320)
    assert _check(pq, q, k, oracle.L2) >= 3
