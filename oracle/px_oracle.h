/*
 * px_oracle.h -- CPU restatement of Proxima's exact-search path (TEST INFRASTRUCTURE).
 *
 * This is the checker, not the product. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it. The product (libproxima_px.so) never
 * links or calls it.
 *
 * Every function restates a reference function (paths relative to the reference
 * repository root):
 *   px_or_l2_sqr            crates/core/src/distance.rs:3-21
 *   px_or_inner_product     crates/core/src/distance.rs:23-39
 *   px_or_flat_search       crates/core/src/flat.rs:106-148 (scan), 150-230 (batch)
 *   px_or_pq_train          crates/core/src/pq.rs:54-105 (train), 139-193 (kmeans)
 *   px_or_pq_encode         crates/core/src/pq.rs:107-121, 266-284
 *   px_or_pq_adc_table      crates/core/src/pq.rs:123-136
 *   px_or_pq_search         crates/core/src/pq.rs:299-347 (scan), 361-396 (batch)
 *
 * Canonical order: the reference keeps the first k rows and then replaces the heap
 * maximum only when a new key is strictly smaller under f32::total_cmp (flat.rs:131-136).
 * Which of several equal maxima Rust's BinaryHeap evicts, and the order
 * into_sorted_vec gives equal keys, are std-library details. The oracle resolves
 * both by ordering candidates on (key total-order, row id): equal keys go to the
 * lower row id. Admission is identical to the reference's (a later row has a larger
 * id, so "(key,id) < max" equals "key < max.key"); only exact ties at the k-boundary
 * can differ, and exact ties are exempt under the parity rule (relative key
 * difference 0 < 1e-5).
 *
 * Compile with -ffp-contract=off and without -ffast-math: Rust never contracts a*b+c.
 */
#ifndef PX_ORACLE_H
#define PX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* metric codes follow the reference enum order (metric.rs:3-7): 0 = L2, 1 = InnerProduct */
float px_or_l2_sqr(const float* a, const float* b, int64_t n);
float px_or_inner_product(const float* a, const float* b, int64_t n);

/* SplitMix64 step (pq.rs:25-37). *state is advanced; returns the mixed value. */
uint64_t px_or_splitmix_next(uint64_t* state);

/*
 * Exact search over row-major data[n][dim]. mask (nullable, length n, nonzero = keep).
 * Outputs per query k entries: ids (-1 padding), finished dists (sqrt(key) for L2,
 * -key for IP; padding FLT_MAX / -FLT_MAX) and, if out_keys != NULL, the raw keys
 * (squared L2 or negated IP; padding +inf). nthreads <= 0 uses all cores.
 * Returns 0, or -1 on invalid arguments (the reference panics there).
 */
int px_or_flat_search(const float* data, int64_t n, int64_t dim, int metric,
                      const float* queries, int64_t nq, int64_t k, const uint8_t* mask,
                      int64_t* out_ids, float* out_dists, float* out_keys, int nthreads);

/*
 * Product-quantizer training: codebooks[m][ks][dim/m] with ks = 1 << nbits.
 * train_sample == 0 means "use all rows". Returns 0 or -1 on invalid arguments.
 */
int px_or_pq_train(const float* training, int64_t n_all, int64_t dim, int64_t m, int64_t nbits,
                   int64_t train_iters, int64_t train_sample, uint64_t seed, float* codebooks,
                   int nthreads);

/* codes[n][m] = argmin_c l2_sqr(sub-vector, centroid) with strict '<' (lower centroid wins) */
int px_or_pq_encode(const float* codebooks, int64_t dim, int64_t m, int64_t nbits,
                    const float* vectors, int64_t n, uint8_t* codes, int nthreads);

/* table[m][ks]: l2_sqr(q_sub, centroid) for L2, -inner_product(q_sub, centroid) for IP */
void px_or_pq_adc_table(const float* codebooks, int64_t dim, int64_t m, int64_t nbits,
                        int metric, const float* query, float* table);

/* ADC search over codes[n][m]; same outputs and padding as px_or_flat_search. */
int px_or_pq_search(const float* codebooks, int64_t dim, int64_t m, int64_t nbits, int metric,
                    const uint8_t* codes, int64_t n, const float* queries, int64_t nq,
                    int64_t k, const uint8_t* mask, int64_t* out_ids, float* out_dists,
                    float* out_keys, int nthreads);

/* number of threads px_or_* uses for nthreads <= 0 */
int px_or_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
