/*
 * Host-side memory and undefined-behaviour check, built with AddressSanitizer and
 * UndefinedBehaviorSanitizer (tests/c_abi/Makefile, target `sanitize`): the oracle, the
 * host PQ trainer (px_pq_train.cpp) and the host code of libproxima_px.so (px_index.hip,
 * host pass only) are instrumented; GPU code is not.
 *
 * Without a device it drives every host path of the C ABI: FlatIndex storage and reads,
 * argument errors, PQ training and encoding on the host (compared bit for bit with the
 * oracle, including a sample larger than the rows, rows that repeat a few distinct rows so
 * that clusters empty and are re-seeded, and dsub = 1), code ingestion and read-back, and
 * the no-device errors of every search entry point. Any sanitizer report ends the run with
 * a failure.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "proxima_px.h"
#include "px_oracle.h"

static int failures = 0;
#define CHECK(cond, what)                                                   \
    do {                                                                    \
        if (!(cond)) {                                                      \
            fprintf(stderr, "FAIL %s:%d %s (%s)\n", __FILE__, __LINE__, what, \
                    px_last_error());                                       \
            ++failures;                                                     \
        }                                                                   \
    } while (0)

static uint64_t rng_state = 0x9e3779b97f4a7c15ull;
static float uniform(void) {  /* [-1, 1) from the oracle's SplitMix64 */
    return (float)((px_or_splitmix_next(&rng_state) >> 40) * (1.0 / 8388608.0)) - 1.0f;
}
static float* random_rows(int64_t n, int64_t dim) {
    float* x = malloc(sizeof(float) * (size_t)(n * dim));
    for (int64_t i = 0; i < n * dim; ++i) x[i] = uniform();
    return x;
}

static void flat_host_paths(void) {
    const int64_t n = 300, dim = 13;
    float* x = random_rows(n, dim);
    px_flat* f = NULL;
    CHECK(px_flat_create(0, dim, &f) == PX_OK && f, "create");
    CHECK(px_flat_add(f, x, n) == PX_OK, "add (rows wait on the host without a device)");
    CHECK(px_flat_add(f, x, 0) == PX_OK, "add of no rows");
    CHECK(px_flat_size(f) == n && px_flat_dim(f) == dim && px_flat_metric(f) == 0, "sizes");
    CHECK(px_flat_memory_bytes(f) >= n * dim * 4, "memory bytes");
    float* back = malloc(sizeof(float) * (size_t)(n * dim));
    CHECK(px_flat_get_vectors(f, 0, n, back) == PX_OK && !memcmp(back, x, sizeof(float) * n * dim),
          "rows read back bit for bit");
    CHECK(px_flat_get_vectors(f, n - 1, 2, back) == PX_ERR_ARG, "row range past the end");
    float bad[13];
    memcpy(bad, x, sizeof bad);
    bad[7] = NAN;
    CHECK(px_flat_add(f, bad, 1) == PX_ERR_NONFINITE && px_flat_size(f) == n, "NaN row refused");
    int64_t ids[5];
    float d[5];
    CHECK(px_flat_search(f, x, 1, 5, NULL, ids, d) == PX_ERR_DEVICE, "search needs a device");
    CHECK(px_flat_search(f, x, 1, 0, NULL, ids, d) == PX_OK, "k = 0 is a no-op");
    CHECK(px_flat_search(f, x, 1, -1, NULL, ids, d) == PX_ERR_BAD_K, "k < 0");
    CHECK(px_flat_search(f, bad, 1, 5, NULL, ids, d) == PX_ERR_NONFINITE, "NaN query");
    CHECK(px_flat_search_device(f, x, 1, 5, NULL, ids, d) == PX_ERR_DEVICE, "device search");
    CHECK(px_flat_search_device_noalloc(f, x, 1, 5, NULL, ids, d) == PX_ERR_DEVICE,
          "no-allocation search");
    px_flat_destroy(f);
    px_flat_destroy(NULL);
    CHECK(knn_gpu_create(x, (int)n, (int)dim) == NULL, "seam create without a device");
    free(back);
    free(x);
}

/* PQ trained and encoded on the host equals the oracle bit for bit. distinct > 0: the rows
 * repeat `distinct` random rows (empty clusters, re-seeds). */
static void pq_case(int64_t n, int64_t dim, int64_t m, int64_t nbits, int64_t iters,
                    int64_t sample, uint64_t seed, int64_t distinct) {
    const int64_t ks = (int64_t)1 << nbits;
    float* x = random_rows(n, dim);
    for (int64_t i = distinct; distinct > 0 && i < n; ++i)
        memcpy(x + i * dim, x + (i % distinct) * dim, sizeof(float) * (size_t)dim);
    px_pq* p = NULL;
    CHECK(px_pq_create(0, dim, m, nbits, &p) == PX_OK && p, "pq create");
    uint8_t one = 0;
    CHECK(px_pq_add_codes(p, &one, 1) == PX_ERR_UNTRAINED, "codes before training");
    CHECK(px_pq_train(p, x, ks - 1, iters, sample, seed) == PX_ERR_ARG, "fewer rows than centroids");
    CHECK(px_pq_train(p, x, n, iters, sample, seed) == PX_OK, "host training");
    float* books = malloc(sizeof(float) * (size_t)(ks * dim));
    float* obooks = malloc(sizeof(float) * (size_t)(ks * dim));
    CHECK(px_pq_get_codebooks(p, books) == PX_OK, "codebooks");
    CHECK(px_or_pq_train(x, n, dim, m, nbits, iters, sample, seed, obooks, 1) == 0, "oracle");
    CHECK(!memcmp(books, obooks, sizeof(float) * (size_t)(ks * dim)), "codebooks equal the oracle's");
    CHECK(px_pq_add(p, x, n) == PX_OK && px_pq_size(p) == n, "host encode");
    uint8_t* codes = malloc((size_t)(n * m));
    uint8_t* ocodes = malloc((size_t)(n * m));
    CHECK(px_pq_get_codes(p, 0, n, codes) == PX_OK, "codes");
    CHECK(px_or_pq_encode(obooks, dim, m, nbits, x, n, ocodes, 1) == 0, "oracle encode");
    CHECK(!memcmp(codes, ocodes, (size_t)(n * m)), "codes equal the oracle's");
    CHECK(px_pq_set_codebooks(p, obooks) == PX_OK, "set codebooks");
    uint8_t bad_code = (uint8_t)(nbits < 8 ? ks : 0);
    if (nbits < 8) CHECK(px_pq_add_codes(p, &bad_code, 1) == PX_ERR_ARG, "code past 2^nbits");
    int64_t ids[3];
    float d[3];
    CHECK(px_pq_search(p, x, 1, 3, NULL, ids, d) == PX_ERR_DEVICE, "pq search needs a device");
    px_pq_destroy(p);
    free(codes);
    free(ocodes);
    free(books);
    free(obooks);
    free(x);
}

static void oracle_paths(void) {
    const int64_t n = 200, dim = 19, nq = 7, k = 12;
    float* x = random_rows(n, dim);
    float* q = random_rows(nq, dim);
    uint8_t* mask = malloc((size_t)n);
    for (int64_t i = 0; i < n; ++i) mask[i] = (uint8_t)(i % 3 != 0);
    int64_t* ids = malloc(sizeof(int64_t) * (size_t)(nq * k));
    float* d = malloc(sizeof(float) * (size_t)(nq * k));
    float* keys = malloc(sizeof(float) * (size_t)(nq * k));
    for (int metric = 0; metric < 2; ++metric) {
        CHECK(px_or_flat_search(x, n, dim, metric, q, nq, k, NULL, ids, d, keys, 2) == 0, "flat");
        CHECK(px_or_flat_search(x, n, dim, metric, q, nq, k, mask, ids, d, NULL, 1) == 0, "masked");
        /* k past the rows: padding */
        CHECK(px_or_flat_search(x, 5, dim, metric, q, 1, k, NULL, ids, d, keys, 1) == 0 &&
                  ids[5] == -1 && ids[k - 1] == -1, "padding");
    }
    free(keys);
    free(d);
    free(ids);
    free(mask);
    free(q);
    free(x);
}

int main(void) {
    if (px_device_count() > 0) {
        printf("sanitize_check skipped (a device is present; the host paths are checked without one)\n");
        return 0;
    }
    flat_host_paths();
    oracle_paths();
    pq_case(1000, 16, 4, 8, 5, 0, 24301, 0);  /* every row trains */
    pq_case(300, 12, 3, 4, 7, 5000, 7, 0);    /* sample larger than the rows */
    pq_case(500, 8, 4, 3, 6, 200, 11, 0);     /* a sample of the rows */
    pq_case(64, 8, 8, 6, 4, 0, 99, 9);        /* dsub = 1, 9 distinct rows for 64 centroids */
    pq_case(4, 6, 2, 2, 3, 0, 1, 1);          /* one distinct row */
    if (failures) {
        fprintf(stderr, "sanitize_check: %d failure(s)\n", failures);
        return 1;
    }
    printf("sanitize_check ok (AddressSanitizer + UndefinedBehaviorSanitizer, library %s)\n",
           px_version());
    return 0;
}
