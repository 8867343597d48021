"""Writes the golden fixtures under tests/golden/ from the CPU oracle.

The reference ships no golden vectors (its tests regenerate inputs from SplitMix64 seeds),
so these fixtures pin this build's oracle and generators at fixed points: each holds the
SHA-256 of its generated inputs, the oracle's ids and keys in canonical (key, id) order,
and for PQ the SHA-256 of the trained codebooks and codes. Workload slices follow the
benchmark workloads' generators and seeds (corpus 1000c+1, queries 1000c+2, mask 1000c+3).

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from proxima_amd import datagen  # noqa: E402

# name -> (workload number, rows, queries, k values, metric, mask density or None)
FLAT_CASES = {
    "flat_l2_10000x128_gauss_q100": (1, 10_000, 100, (10,), oracle.L2, None),
    "flat_ip_20000x384_unit_q32": (2, 20_000, 32, (10,), oracle.IP, None),
    "flat_l2_100000x128_sift_q32": (3, 100_000, 32, (10, 100), oracle.L2, None),
    "flat_ip_50000x384_unit_q16_mask10": (5, 50_000, 16, (100,), oracle.IP, 0.1),
}
# PQ: workload 4 generators; training on the first 20,000 rows, 10 Lloyd iterations
PQ_CASE = "pq_l2_100000x128_m16_q32"
PQ_TRAIN_ROWS, PQ_ITERS, PQ_SEED, PQ_M, PQ_NBITS = 20_000, 10, 24301, 16, 8


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def flat_inputs(c: int, rows: int, nq: int, p):
    data = datagen.corpus(c, rows=rows)
    q = datagen.queries(c, rows=nq)
    mask = datagen.mask(rows, p, 1000 * c + 3) if p is not None else None
    return data, q, mask


def pq_inputs():
    data = datagen.corpus(4, rows=100_000)
    q = datagen.queries(4, rows=32)
    mask = datagen.mask(100_000, 0.5, 4003)
    return data, q, mask


def pq_model(data):
    books = oracle.pq_train(data[:PQ_TRAIN_ROWS], PQ_M, PQ_NBITS, PQ_ITERS, 0, PQ_SEED)
    codes = oracle.pq_encode(books, data)
    return books, codes


def main() -> None:
    for name, (c, rows, nq, ks, metric, p) in FLAT_CASES.items():
        data, q, mask = flat_inputs(c, rows, nq, p)
        out = {"corpus_sha256": sha(data), "queries_sha256": sha(q),
               "mask_sha256": sha(mask) if mask is not None else ""}
        for k in ks:
            ids, _, keys = oracle.flat_search(data, q, k, metric, mask=mask)
            out[f"ids_k{k}"] = ids.astype(np.int32)
            out[f"keys_k{k}"] = keys
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **out)
        print(name, {kk: (v.shape if hasattr(v, "shape") else v) for kk, v in out.items()})

    data, q, mask = pq_inputs()
    books, codes = pq_model(data)
    out = {"corpus_sha256": sha(data), "queries_sha256": sha(q), "mask_sha256": sha(mask),
           "books_sha256": sha(books), "codes_sha256": sha(codes)}
    for tag, mk in (("", None), ("_mask50", mask)):
        ids, _, keys = oracle.pq_search(books, codes, q, 10, oracle.L2, mask=mk)
        out[f"ids_k10{tag}"] = ids.astype(np.int32)
        out[f"keys_k10{tag}"] = keys
    np.savez_compressed(os.path.join(HERE, PQ_CASE + ".npz"), **out)
    print(PQ_CASE, "written")


if __name__ == "__main__":
    main()
