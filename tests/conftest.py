import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 (MI355X) GPU; runs the HIP path")


def have_gpu() -> bool:
    try:
        from proxima_amd import _lib

        return _lib.device_count() > 0
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    if not have_gpu():
        pytest.fail("GPU test collected without a visible HIP device")
    return True


def sample_positions(n_eff: int, kk: int) -> np.ndarray:
    """Positions of the collect path's threshold sample: S = min(n_eff, 16384,
    80 * n_eff // kk) rows spread evenly, position floor(i * n_eff / S) for i < S. kk is
    the number of candidates the search keeps (k + 8 on the flat path, k for PQ)."""
    s = max(1, min(n_eff, 16384, 80 * n_eff // kk))
    return np.arange(s, dtype=np.int64) * n_eff // s


def rel(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return np.abs(a - b) / np.maximum(np.maximum(np.abs(a), np.abs(b)), 1e-30)


def assert_parity(ids, dists, o_ids, o_dists, key_of, tie_rel=1e-5, dist_rel=1e-4,
                  allow_exempt=True):
    """The parity rule: ids identical at every rank except where the two candidates' keys
    differ by less than tie_rel (relative); distances within dist_rel (relative).
    key_of(query_index, row_id) returns the reference-arithmetic key of a row."""
    ids = np.asarray(ids)
    o_ids = np.asarray(o_ids)
    assert ids.shape == o_ids.shape, (ids.shape, o_ids.shape)
    bad = np.argwhere(ids != o_ids)
    exempt = 0
    for qi, j in bad:
        a, b = int(ids[qi, j]), int(o_ids[qi, j])
        assert a >= 0 and b >= 0, f"padding differs at query {qi} rank {j}: {a} vs {b}"
        assert allow_exempt, f"id differs at query {qi} rank {j}: {a} vs {b}"
        ka, kb = key_of(qi, a), key_of(qi, b)
        assert rel(ka, kb) < tie_rel, (
            f"query {qi} rank {j}: gpu id {a} (key {ka!r}) vs oracle id {b} (key {kb!r})")
        exempt += 1
    pad = o_ids < 0
    assert np.array_equal(dists[pad], o_dists[pad]), "padding distances differ"
    r = rel(dists[~pad], o_dists[~pad])
    assert r.size == 0 or r.max() <= dist_rel, f"max relative distance error {r.max():.3g}"
    return exempt
