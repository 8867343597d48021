/* abi_check.c -- the C ABI of libproxima_px.so exercised from plain C, the way a non-Python
 * host (the reference's Rust crate over gpu.rs:10-15, or any FFI) would bind it.
 *
 * With a gfx950 device: the reference's known answers through both entry families --
 * flat.rs:323-338 (corpus {0^4, 1^4}, query 0^4, k = 5 -> ids [0, 1, -1, -1, -1], distances
 * [0, 2, FLT_MAX x 3]), flat.rs:370-383 (filter keeps row 0 only), the inner-product padding
 * (-FLT_MAX), the raw keys of the CUDA seam for both metrics on one handle (gpu.rs:80-93
 * finishes them), a PQ index built from explicit codebooks and codes -- and the status codes
 * of bad arguments, non-finite host and device queries among them.
 * Without a device: every search fails with PX_ERR_DEVICE and knn_gpu_create returns NULL.
 * Prints "abi_check ok (...)" and exits 0, or names the failed check and exits 1. */
#include <float.h>
#include <math.h>
#include <stdio.h>
#include <string.h>

#include "proxima_px.h"

static int failures = 0;
#define CHECK(cond, what)                                                            \
    do {                                                                             \
        if (!(cond)) {                                                               \
            fprintf(stderr, "abi_check: FAILED %s (line %d): %s\n", what, __LINE__,  \
                    px_last_error());                                                \
            ++failures;                                                              \
        }                                                                            \
    } while (0)

static const float corpus[8] = {0, 0, 0, 0, 1, 1, 1, 1};
static const float query[4] = {0, 0, 0, 0};

static void with_device(void) {
    px_flat* f = NULL;
    CHECK(px_flat_create(0, 4, &f) == PX_OK && f, "px_flat_create L2");
    CHECK(px_flat_add(f, corpus, 2) == PX_OK, "px_flat_add");
    int64_t ids[5];
    float d[5];
    CHECK(px_flat_search(f, query, 1, 5, NULL, ids, d) == PX_OK, "px_flat_search");
    CHECK(ids[0] == 0 && ids[1] == 1 && ids[2] == -1 && ids[3] == -1 && ids[4] == -1,
          "flat.rs:323-338 ids");
    CHECK(d[0] == 0.0f && d[1] == 2.0f && d[2] == FLT_MAX && d[4] == FLT_MAX,
          "flat.rs:323-338 distances");
    const uint8_t keep0[2] = {1, 0};
    CHECK(px_flat_search(f, query, 1, 5, keep0, ids, d) == PX_OK, "filtered search");
    CHECK(ids[0] == 0 && ids[1] == -1 && ids[4] == -1 && d[1] == FLT_MAX,
          "flat.rs:370-383 filtered padding");
    {
        /* any k: past PX_MAX_K every key is sorted (flat.rs:106-148 keeps a heap of k) */
        static long long big_ids[PX_MAX_K + 1];
        static float big_d[PX_MAX_K + 1];
        CHECK(px_flat_search(f, query, 1, PX_MAX_K + 1, NULL, (int64_t*)big_ids, big_d) == PX_OK,
              "k past PX_MAX_K");
        CHECK(big_ids[0] == 0 && big_ids[1] == 1 && big_ids[2] == -1 &&
                  big_ids[PX_MAX_K] == -1 && big_d[1] == 2.0f && big_d[PX_MAX_K] == FLT_MAX,
              "k past PX_MAX_K: rows in order, then padding");
    }
    const float nanq[4] = {0, NAN, 0, 0};
    CHECK(px_flat_search(f, nanq, 1, 5, NULL, ids, d) == PX_ERR_NONFINITE, "non-finite query");
    CHECK(strlen(px_last_error()) > 0, "error text");
    {
        /* the device-pointer form checks its queries on the device before searching */
        void *dq = NULL, *di = NULL, *dd = NULL;
        CHECK(px_dev_alloc(&dq, sizeof nanq) == PX_OK && px_dev_alloc(&di, 5 * 8) == PX_OK &&
                  px_dev_alloc(&dd, 5 * 4) == PX_OK,
              "px_dev_alloc");
        CHECK(px_dev_upload(dq, nanq, sizeof nanq) == PX_OK, "upload NaN query");
        CHECK(px_flat_search_device(f, (const float*)dq, 1, 5, NULL, (int64_t*)di, (float*)dd) ==
                  PX_ERR_NONFINITE,
              "non-finite device query");
        const float infq[4] = {0, 0, -INFINITY, 0};
        CHECK(px_dev_upload(dq, infq, sizeof infq) == PX_OK, "upload infinite query");
        CHECK(px_flat_search_device(f, (const float*)dq, 1, 5, NULL, (int64_t*)di, (float*)dd) ==
                  PX_ERR_NONFINITE,
              "infinite device query");
        CHECK(px_dev_upload(dq, query, sizeof query) == PX_OK, "upload finite query");
        CHECK(px_flat_search_device(f, (const float*)dq, 1, 5, NULL, (int64_t*)di, (float*)dd) ==
                  PX_OK,
              "finite device query after a rejected one");
        CHECK(px_dev_download(ids, di, sizeof ids) == PX_OK && ids[0] == 0 && ids[1] == 1 &&
                  ids[2] == -1,
              "device search results");
        px_dev_free(dq);
        px_dev_free(di);
        px_dev_free(dd);
    }
    px_flat_destroy(f);

    px_flat* g = NULL;
    CHECK(px_flat_create(1, 4, &g) == PX_OK, "px_flat_create IP");
    CHECK(px_flat_add(g, corpus, 2) == PX_OK, "add IP");
    const float q1[4] = {1, 1, 1, 1};
    CHECK(px_flat_search(g, q1, 1, 3, NULL, ids, d) == PX_OK, "IP search");
    CHECK(ids[0] == 1 && d[0] == 4.0f && ids[1] == 0 && d[1] == 0.0f && ids[2] == -1 &&
              d[2] == -FLT_MAX,
          "IP order and padding");
    px_flat_destroy(g);

    /* the reference's CUDA seam: raw keys */
    PxGpuIndex* gi = knn_gpu_create(corpus, 2, 4);
    CHECK(gi != NULL, "knn_gpu_create");
    long long kid[3];
    float kk[3];
    CHECK(knn_gpu_search(gi, query, 1, 3, 0, kid, kk) == 0, "knn_gpu_search");
    CHECK(kid[0] == 0 && kid[1] == 1 && kid[2] == -1 && kk[0] == 0.0f && kk[1] == 4.0f &&
              kk[2] == FLT_MAX,
          "raw squared-L2 keys and padding");
    /* the same handle (one corpus copy) serves the inner product: raw keys are -q.x */
    const float ones[4] = {1, 1, 1, 1};
    CHECK(knn_gpu_search(gi, ones, 1, 3, 1, kid, kk) == 0, "knn_gpu_search IP");
    CHECK(kid[0] == 1 && kid[1] == 0 && kid[2] == -1 && kk[0] == -4.0f && kk[1] == 0.0f &&
              kk[2] == FLT_MAX,
          "raw inner-product keys on the shared corpus copy");
    CHECK(knn_gpu_search(gi, query, 1, 3, 0, kid, kk) == 0 && kk[1] == 4.0f,
          "L2 again after an inner-product search");
    CHECK(knn_gpu_search(gi, query, 1, 0, 0, kid, kk) == -1, "knn.cu:145 k < 1");
    CHECK(knn_gpu_search(gi, query, 1, PX_MAX_K + 1, 0, kid, kk) == -1, "seam k limit");
    knn_gpu_free(gi);
    knn_gpu_free(NULL);

    /* PQ from explicit codebooks and codes: m = 2 subspaces of 2 dims, 2 bits */
    px_pq* p = NULL;
    CHECK(px_pq_create(0, 4, 2, 2, &p) == PX_OK, "px_pq_create");
    float books[2 * 4 * 2];
    for (int s = 0; s < 2; ++s)
        for (int c = 0; c < 4; ++c) {
            books[(s * 4 + c) * 2 + 0] = (float)c;
            books[(s * 4 + c) * 2 + 1] = (float)(s * c);
        }
    CHECK(px_pq_set_codebooks(p, books) == PX_OK, "set codebooks");
    const uint8_t codes[3 * 2] = {3, 3, 0, 0, 1, 2};
    CHECK(px_pq_add_codes(p, codes, 3) == PX_OK, "add codes");
    CHECK(px_pq_search(p, query, 1, 4, NULL, ids, d) == PX_OK, "pq search");
    /* ADC keys: row0 (3,0)+(3,3) -> 9 + 18 = 27; row1 0; row2 (1,0)+(2,2) -> 1 + 8 = 9 */
    CHECK(ids[0] == 1 && ids[1] == 2 && ids[2] == 0 && ids[3] == -1, "pq order");
    CHECK(d[0] == 0.0f && d[1] == 3.0f && fabsf(d[2] - sqrtf(27.0f)) == 0.0f && d[3] == FLT_MAX,
          "pq distances");
    {
        const float nanq[4] = {NAN, 0, 0, 0};
        void *dq = NULL, *di = NULL, *dd = NULL;
        CHECK(px_dev_alloc(&dq, sizeof nanq) == PX_OK && px_dev_alloc(&di, 4 * 8) == PX_OK &&
                  px_dev_alloc(&dd, 4 * 4) == PX_OK,
              "px_dev_alloc (pq)");
        CHECK(px_dev_upload(dq, nanq, sizeof nanq) == PX_OK, "upload NaN query (pq)");
        CHECK(px_pq_search_device(p, (const float*)dq, 1, 4, NULL, (int64_t*)di, (float*)dd) ==
                  PX_ERR_NONFINITE,
              "non-finite device query (pq)");
        px_dev_free(dq);
        px_dev_free(di);
        px_dev_free(dd);
    }
    px_pq_destroy(p);
}

static void without_device(void) {
    px_flat* f = NULL;
    CHECK(px_flat_create(0, 4, &f) == PX_OK, "px_flat_create");
    CHECK(px_flat_add(f, corpus, 2) == PX_OK, "px_flat_add keeps rows on the host");
    int64_t ids[5];
    float d[5];
    CHECK(px_flat_search(f, query, 1, 5, NULL, ids, d) == PX_ERR_DEVICE, "search needs a GPU");
    px_flat_destroy(f);
    CHECK(knn_gpu_create(corpus, 2, 4) == NULL, "knn_gpu_create without a device");
}

int main(void) {
    const int devices = px_device_count();
    if (devices > 0)
        with_device();
    else
        without_device();
    if (failures) return 1;
    printf("abi_check ok (%s, %d device%s, library %s)\n", devices > 0 ? "gfx950 path" : "no-device path",
           devices, devices == 1 ? "" : "s", px_version());
    return 0;
}
