/*
 * px_oracle.c -- CPU restatement of Proxima's exact-search path (TEST INFRASTRUCTURE).
 *
 * The checker for libproxima_px.so; never linked into it. See px_oracle.h for the
 * reference file:line each function follows and for the canonical tie order.
 *
 * Build: gcc -O3 -ffp-contract=off (no -ffast-math) -fopenmp -- see oracle/Makefile.
 * The 8-lane loops below are written so that GCC maps one chunk onto one 8-wide
 * vector add, which is the reference's own order (distance.rs:9-14); the lane sum
 * and the remainder stay sequential because GCC never reassociates without
 * -ffast-math.
 */
#include "px_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define PX_LANES 8

int px_or_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

static int resolve_threads(int nthreads) {
    return nthreads > 0 ? nthreads : px_or_max_threads();
}

/* distance.rs:3-21. acc[l] sums elements l, l+8, ... as acc = acc + d*d (no FMA);
 * then the lanes are summed in order 0..7, then the D mod 8 remainder in order.
 * The start value of Rust's f32 Sum (+0.0 or -0.0, depending on the rustc version)
 * cannot change the result: acc[0] starts at +0.0 and can never become -0.0
 * (+0.0 + -0.0 = +0.0), and start + acc[0] = acc[0] for both starts. */
float px_or_l2_sqr(const float* a, const float* b, int64_t n) {
    float acc[PX_LANES] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int64_t chunks = n / PX_LANES;
    for (int64_t c = 0; c < chunks; ++c) {
        const float* ac = a + c * PX_LANES;
        const float* bc = b + c * PX_LANES;
        for (int l = 0; l < PX_LANES; ++l) {
            float d = ac[l] - bc[l];
            acc[l] = acc[l] + d * d;
        }
    }
    float sum = 0.0f;
    for (int l = 0; l < PX_LANES; ++l) sum = sum + acc[l];
    for (int64_t i = chunks * PX_LANES; i < n; ++i) {
        float d = a[i] - b[i];
        sum = sum + d * d;
    }
    return sum;
}

/* distance.rs:23-39, same lane structure as l2_sqr. */
float px_or_inner_product(const float* a, const float* b, int64_t n) {
    float acc[PX_LANES] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int64_t chunks = n / PX_LANES;
    for (int64_t c = 0; c < chunks; ++c) {
        const float* ac = a + c * PX_LANES;
        const float* bc = b + c * PX_LANES;
        for (int l = 0; l < PX_LANES; ++l) acc[l] = acc[l] + ac[l] * bc[l];
    }
    float sum = 0.0f;
    for (int l = 0; l < PX_LANES; ++l) sum = sum + acc[l];
    for (int64_t i = chunks * PX_LANES; i < n; ++i) sum = sum + a[i] * b[i];
    return sum;
}

/* pq.rs:25-33 */
uint64_t px_or_splitmix_next(uint64_t* state) {
    *state += 0x9E3779B97F4A7C15ull;
    uint64_t z = *state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* pq.rs:34-36 */
static uint64_t splitmix_below(uint64_t* state, uint64_t n) {
    return px_or_splitmix_next(state) % n;
}

/* ---------------------------------------------------------------------------
 * Top-k selection: flat.rs:11-32 (Cand ordered by f32::total_cmp) and
 * flat.rs:123-147 (heap of the k best, into_sorted_vec, finish, pad).
 * The heap is ordered on (total-order key, id); see px_oracle.h.
 * ------------------------------------------------------------------------- */
typedef struct {
    int32_t tk; /* key mapped to a signed integer with the IEEE total order */
    float key;
    int64_t id;
} cand_t;

/* The IEEE-754 totalOrder mapping that f32::total_cmp uses: flip the magnitude
 * bits of negative numbers, then compare as signed 32-bit integers. */
static inline int32_t total_key(float f) {
    int32_t b;
    memcpy(&b, &f, sizeof b);
    b ^= (int32_t)(((uint32_t)(b >> 31)) >> 1);
    return b;
}

static inline int cand_less(const cand_t* a, const cand_t* b) {
    return a->tk < b->tk || (a->tk == b->tk && a->id < b->id);
}

static void heap_sift_down(cand_t* h, int64_t len, int64_t i) {
    for (;;) {
        int64_t l = 2 * i + 1, r = l + 1, m = i;
        if (l < len && cand_less(&h[m], &h[l])) m = l;
        if (r < len && cand_less(&h[m], &h[r])) m = r;
        if (m == i) return;
        cand_t t = h[i];
        h[i] = h[m];
        h[m] = t;
        i = m;
    }
}

static void heap_sift_up(cand_t* h, int64_t i) {
    while (i > 0) {
        int64_t p = (i - 1) / 2;
        if (!cand_less(&h[p], &h[i])) return;
        cand_t t = h[i];
        h[i] = h[p];
        h[p] = t;
        i = p;
    }
}

/* offer (key, id) to a max-heap of capacity k holding *len entries (flat.rs:131-136) */
static inline void heap_offer(cand_t* h, int64_t* len, int64_t k, float key, int64_t id) {
    cand_t c;
    c.tk = total_key(key);
    c.key = key;
    c.id = id;
    if (*len < k) {
        h[*len] = c;
        heap_sift_up(h, *len);
        *len += 1;
    } else if (cand_less(&c, &h[0])) {
        h[0] = c;
        heap_sift_down(h, *len, 0);
    }
}

static int cand_cmp(const void* pa, const void* pb) {
    const cand_t* a = (const cand_t*)pa;
    const cand_t* b = (const cand_t*)pb;
    if (cand_less(a, b)) return -1;
    if (cand_less(b, a)) return 1;
    return 0;
}

/* flat.rs:139-147 / pq.rs:332-346: ascending order, finish, pad */
static void heap_finish(cand_t* h, int64_t len, int64_t k, int l2, int64_t* ids, float* dists,
                        float* keys) {
    qsort(h, (size_t)len, sizeof(cand_t), cand_cmp);
    for (int64_t j = 0; j < len; ++j) {
        ids[j] = h[j].id;
        dists[j] = l2 ? sqrtf(h[j].key) : -h[j].key;
        if (keys) keys[j] = h[j].key;
    }
    for (int64_t j = len; j < k; ++j) {
        ids[j] = -1;
        dists[j] = l2 ? FLT_MAX : -FLT_MAX;
        if (keys) keys[j] = INFINITY;
    }
}

/* flat.rs:106-148 for one query, batch over queries as flat.rs:150-230 */
int px_or_flat_search(const float* data, int64_t n, int64_t dim, int metric,
                      const float* queries, int64_t nq, int64_t k, const uint8_t* mask,
                      int64_t* out_ids, float* out_dists, float* out_keys, int nthreads) {
    if (dim <= 0 || n < 0 || nq < 0 || k < 0 || (metric != 0 && metric != 1)) return -1;
    if (k == 0 || nq == 0) return 0;
    const int l2 = metric == 0;
    int bad = 0;
#pragma omp parallel num_threads(resolve_threads(nthreads)) reduction(| : bad)
    {
        cand_t* heap = (cand_t*)malloc((size_t)k * sizeof(cand_t));
        if (!heap) bad = 1;
#pragma omp for schedule(dynamic, 1)
        for (int64_t qi = 0; qi < nq; ++qi) {
            if (!heap) continue;
            const float* q = queries + qi * dim;
            int64_t len = 0;
            for (int64_t i = 0; i < n; ++i) {
                if (mask && !mask[i]) continue; /* flat.rs:125-129: skip before the distance */
                const float* v = data + i * dim;
                float key = l2 ? px_or_l2_sqr(q, v, dim) : -px_or_inner_product(q, v, dim);
                heap_offer(heap, &len, k, key, i);
            }
            heap_finish(heap, len, k, l2, out_ids + qi * k, out_dists + qi * k,
                        out_keys ? out_keys + qi * k : NULL);
        }
        free(heap);
    }
    return bad ? -1 : 0;
}

/* ---------------------------------------------------------------------------
 * Product quantization
 * ------------------------------------------------------------------------- */

/* pq.rs:139-193 */
static void kmeans(const float* data, int64_t n, int64_t d, int64_t ks, int64_t iters,
                   uint64_t seed, float* centroids, int nthreads) {
    uint64_t rng = seed;
    int64_t* order = (int64_t*)malloc((size_t)n * sizeof(int64_t));
    for (int64_t i = 0; i < n; ++i) order[i] = i;
    /* partial Fisher-Yates pick of ks distinct rows (pq.rs:142-148) */
    for (int64_t c = 0; c < ks; ++c) {
        int64_t j = c + (int64_t)splitmix_below(&rng, (uint64_t)(n - c));
        int64_t t = order[c];
        order[c] = order[j];
        order[j] = t;
        memcpy(centroids + c * d, data + order[c] * d, (size_t)d * sizeof(float));
    }
    free(order);

    uint32_t* assign = (uint32_t*)malloc((size_t)n * sizeof(uint32_t));
    float* sums = (float*)malloc((size_t)(ks * d) * sizeof(float));
    uint32_t* counts = (uint32_t*)malloc((size_t)ks * sizeof(uint32_t));

    for (int64_t it = 0; it < iters; ++it) {
        /* pq.rs:155-167: argmin with strict '<' from f32::MAX */
#pragma omp parallel for schedule(static) num_threads(resolve_threads(nthreads))
        for (int64_t i = 0; i < n; ++i) {
            const float* v = data + i * d;
            uint32_t best = 0;
            float best_d = FLT_MAX;
            for (int64_t c = 0; c < ks; ++c) {
                float dist = px_or_l2_sqr(v, centroids + c * d, d);
                if (dist < best_d) {
                    best_d = dist;
                    best = (uint32_t)c;
                }
            }
            assign[i] = best;
        }
        /* pq.rs:169-179: sequential sums in row order */
        for (int64_t x = 0; x < ks * d; ++x) sums[x] = 0.0f;
        for (int64_t c = 0; c < ks; ++c) counts[c] = 0;
        for (int64_t i = 0; i < n; ++i) {
            int64_t c = assign[i];
            counts[c] += 1;
            const float* v = data + i * d;
            float* s = sums + c * d;
            for (int64_t j = 0; j < d; ++j) s[j] = s[j] + v[j];
        }
        /* pq.rs:180-190: empty clusters re-seeded from the rng; else reciprocal multiply */
        for (int64_t c = 0; c < ks; ++c) {
            if (counts[c] == 0) {
                int64_t idx = (int64_t)splitmix_below(&rng, (uint64_t)n);
                memcpy(centroids + c * d, data + idx * d, (size_t)d * sizeof(float));
            } else {
                float inv = 1.0f / (float)counts[c];
                for (int64_t j = 0; j < d; ++j) centroids[c * d + j] = sums[c * d + j] * inv;
            }
        }
    }
    free(assign);
    free(sums);
    free(counts);
}

static int all_finite(const float* x, int64_t len) {
    for (int64_t i = 0; i < len; ++i)
        if (!isfinite(x[i])) return 0;
    return 1;
}

/* pq.rs:54-105 */
int px_or_pq_train(const float* training, int64_t n_all, int64_t dim, int64_t m, int64_t nbits,
                   int64_t train_iters, int64_t train_sample, uint64_t seed, float* codebooks,
                   int nthreads) {
    if (m < 1 || dim <= 0 || dim % m != 0 || nbits < 1 || nbits > 8) return -1;
    const int64_t dsub = dim / m;
    const int64_t ks = (int64_t)1 << nbits;
    if (n_all < ks || train_iters < 0 || train_sample < 0) return -1;
    if (!all_finite(training, n_all * dim)) return -1;

    uint64_t rng = seed;
    int64_t n = n_all;
    if (train_sample > 0) n = train_sample < ks ? ks : (train_sample > n_all ? n_all : train_sample);
    int64_t* sample = (int64_t*)malloc((size_t)n * sizeof(int64_t));
    if (n == n_all) {
        for (int64_t i = 0; i < n; ++i) sample[i] = i;
    } else {
        for (int64_t i = 0; i < n; ++i) sample[i] = (int64_t)splitmix_below(&rng, (uint64_t)n_all);
    }
    float* sub_data = (float*)malloc((size_t)(n * dsub) * sizeof(float));
    for (int64_t sub = 0; sub < m; ++sub) {
        for (int64_t i = 0; i < n; ++i)
            memcpy(sub_data + i * dsub, training + sample[i] * dim + sub * dsub,
                   (size_t)dsub * sizeof(float));
        kmeans(sub_data, n, dsub, ks, train_iters,
               seed ^ ((uint64_t)sub * 0x9E3779B97F4A7C15ull),
               codebooks + sub * ks * dsub, nthreads);
    }
    free(sub_data);
    free(sample);
    return 0;
}

/* pq.rs:107-121 per row, pq.rs:266-284 over rows */
int px_or_pq_encode(const float* codebooks, int64_t dim, int64_t m, int64_t nbits,
                    const float* vectors, int64_t n, uint8_t* codes, int nthreads) {
    if (m < 1 || dim <= 0 || dim % m != 0 || nbits < 1 || nbits > 8 || n < 0) return -1;
    const int64_t dsub = dim / m;
    const int64_t ks = (int64_t)1 << nbits;
#pragma omp parallel for schedule(static) num_threads(resolve_threads(nthreads))
    for (int64_t i = 0; i < n; ++i) {
        const float* v = vectors + i * dim;
        for (int64_t sub = 0; sub < m; ++sub) {
            uint32_t best = 0;
            float best_d = FLT_MAX;
            for (int64_t c = 0; c < ks; ++c) {
                float d = px_or_l2_sqr(v + sub * dsub, codebooks + (sub * ks + c) * dsub, dsub);
                if (d < best_d) {
                    best_d = d;
                    best = (uint32_t)c;
                }
            }
            codes[i * m + sub] = (uint8_t)best;
        }
    }
    return 0;
}

/* pq.rs:123-136 */
void px_or_pq_adc_table(const float* codebooks, int64_t dim, int64_t m, int64_t nbits,
                        int metric, const float* query, float* table) {
    const int64_t dsub = dim / m;
    const int64_t ks = (int64_t)1 << nbits;
    for (int64_t sub = 0; sub < m; ++sub) {
        const float* qs = query + sub * dsub;
        for (int64_t c = 0; c < ks; ++c) {
            const float* cen = codebooks + (sub * ks + c) * dsub;
            table[sub * ks + c] =
                metric == 0 ? px_or_l2_sqr(qs, cen, dsub) : -px_or_inner_product(qs, cen, dsub);
        }
    }
}

/* pq.rs:299-347 per query, pq.rs:361-396 over queries */
int px_or_pq_search(const float* codebooks, int64_t dim, int64_t m, int64_t nbits, int metric,
                    const uint8_t* codes, int64_t n, const float* queries, int64_t nq,
                    int64_t k, const uint8_t* mask, int64_t* out_ids, float* out_dists,
                    float* out_keys, int nthreads) {
    if (m < 1 || dim <= 0 || dim % m != 0 || nbits < 1 || nbits > 8) return -1;
    if (n < 0 || nq < 0 || k < 0 || (metric != 0 && metric != 1)) return -1;
    if (k == 0 || nq == 0) return 0;
    const int64_t ks = (int64_t)1 << nbits;
    const int l2 = metric == 0;
    int bad = 0;
#pragma omp parallel num_threads(resolve_threads(nthreads)) reduction(| : bad)
    {
        cand_t* heap = (cand_t*)malloc((size_t)k * sizeof(cand_t));
        float* table = (float*)malloc((size_t)(m * ks) * sizeof(float));
        if (!heap || !table) bad = 1;
#pragma omp for schedule(dynamic, 1)
        for (int64_t qi = 0; qi < nq; ++qi) {
            if (!heap || !table) continue;
            px_or_pq_adc_table(codebooks, dim, m, nbits, metric, queries + qi * dim, table);
            int64_t len = 0;
            for (int64_t i = 0; i < n; ++i) {
                if (mask && !mask[i]) continue; /* pq.rs:315-319 */
                const uint8_t* code = codes + i * m;
                float key = 0.0f; /* pq.rs:320-323: sequential from +0.0 */
                for (int64_t sub = 0; sub < m; ++sub) key = key + table[sub * ks + code[sub]];
                heap_offer(heap, &len, k, key, i);
            }
            heap_finish(heap, len, k, l2, out_ids + qi * k, out_dists + qi * k,
                        out_keys ? out_keys + qi * k : NULL);
        }
        free(heap);
        free(table);
    }
    return bad ? -1 : 0;
}
