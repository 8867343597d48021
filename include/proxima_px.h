/*
 * proxima_px.h -- C ABI of libproxima_px.so, the MI355X (gfx950) exact-search backend for
 * Proxima's FlatIndex and PqIndex.
 *
 * Plain pointers and sizes only. Every entry point names the reference interface it
 * replaces (paths relative to the reference repository root). Metric codes follow the
 * reference enum order (crates/core/src/metric.rs:3-7): 0 = L2, 1 = InnerProduct.
 *
 * Status codes: 0 = ok; negative = argument error (below); positive = a HIP runtime
 * error code (e.g. 100 = no device, 2 = out of memory). px_last_error() returns a
 * message for the calling thread's last failure.
 *
 * Threading: handles may be shared between threads; searches on one handle are
 * serialised internally. add/train/destroy must not race with other calls on the
 * same handle (the reference takes &mut self there).
 *
 * Results: ids ascending by (key, id) with equal keys going to the lower row id; keys are
 * recomputed for the returned rows in the reference's arithmetic (distance.rs:3-39), so
 * distances are the reference's. Short results are padded with id -1 and FLT_MAX (L2)
 * or -FLT_MAX (IP), as flat.rs:144-147.
 */
#ifndef PROXIMA_PX_H
#define PROXIMA_PX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PX_OK 0
#define PX_ERR_BAD_K (-1)      /* k outside what the kernels support (knn.cu:145) */
#define PX_ERR_SHMEM (-2)      /* reserved: knn.cu:147's shared-memory code; never returned */
#define PX_ERR_DIM (-3)        /* dim == 0, or a length not a multiple of dim (flat.rs:73-78, 162-167) */
#define PX_ERR_NONFINITE (-4)  /* NaN or infinite input (flat.rs:79-82, 114-117) */
#define PX_ERR_ARG (-5)        /* null handle/pointer, negative size, bad metric or params */
#define PX_ERR_UNTRAINED (-6)  /* PQ index used before train (crates/py/src/lib.rs:492-504) */
#define PX_ERR_DEVICE (-7)     /* no usable gfx950 device, or a device-side failure of the search
                                  (a collect or list scan whose workgroup stage sync gave
                                  up: no results, the outputs unwritten; px_last_error
                                  names it) */

/* Largest k of the reference's GPU seam (knn_gpu_search). px_flat_search* and
 * px_pq_search* take any k >= 0, as the reference's FlatIndex and PqIndex do
 * (flat.rs:106-148, pq.rs:299-347): past PX_MAX_K every key is computed and sorted. */
#define PX_MAX_K 4096

/* Message for the calling thread's last non-zero status (empty string if none). */
const char* px_last_error(void);

/* Library version string ("0.1.0", crates/py/src/lib.rs:691). */
const char* px_version(void);

/* ------------------------------------------------------------------------------------
 * The reference's own GPU seam, same signatures: crates/core/src/gpu.rs:10-15 declares
 * these three and crates/core/cuda/knn.cu:123-180 implements them for CUDA. A Rust
 * build links this library in place of knn.cu and CudaKnn works unchanged.
 * Keys are raw (squared L2 or negated inner product); the caller finishes them
 * (gpu.rs:80-93). Padding: id -1, key FLT_MAX. k may be up to PX_MAX_K (the CUDA
 * kernel stopped at 46; the reference's FlatIndex takes any k).
 * ---------------------------------------------------------------------------------- */
typedef struct PxGpuIndex PxGpuIndex;

/* knn.cu:123-141: copy n x dim row-major floats to the device; NULL on failure. One device
 * copy of the rows (and their squared norms) serves both metrics. */
PxGpuIndex* knn_gpu_create(const float* base, int n, int dim);

/* knn.cu:143-174: 0 ok, -1 bad k, >0 HIP error. Synchronous; outputs are host memory. */
int knn_gpu_search(const PxGpuIndex* idx, const float* queries, int nq, int k, int metric,
                   long long* out_ids, float* out_keys);

/* knn.cu:176-180: NULL-safe. */
void knn_gpu_free(PxGpuIndex* idx);

/* ------------------------------------------------------------------------------------
 * FlatIndex (crates/core/src/flat.rs:34-231), the path a `hip` feature of
 * crates/core would bind behind FlatIndex::{new, add, search*, len, dim, metric,
 * memory_bytes}.
 * ---------------------------------------------------------------------------------- */
typedef struct px_flat px_flat;

/* FlatIndex::new, flat.rs:43-46 */
int px_flat_create(int metric, int64_t dim, px_flat** out);
/* Drop */
void px_flat_destroy(px_flat* idx);
/* FlatIndex::add, flat.rs:72-85: append n rows (row-major n x dim). */
int px_flat_add(px_flat* idx, const float* vectors, int64_t n);

/*
 * FlatIndex::search_batch / search_batch_filtered, flat.rs:150-230 (search and
 * search_filtered are nq = 1). Host pointers. mask is NULL or px_flat_size() bytes,
 * nonzero = keep (flat.rs:125-129). Outputs nq * k each. k == 0 or nq == 0 is a no-op.
 */
int px_flat_search(const px_flat* idx, const float* queries, int64_t nq, int64_t k,
                   const uint8_t* mask, int64_t* out_ids, float* out_dists);

/*
 * Same search with every pointer in device memory of the index's GPU (queries nq x dim,
 * mask px_flat_size() bytes or NULL, outputs nq * k). Synchronous. No host copies: the
 * form for callers that keep queries and results resident in HBM. The queries are checked
 * on the device before any search work: NaN or infinite values return PX_ERR_NONFINITE with
 * the outputs unwritten, as the host form (flat.rs:114-117).
 */
int px_flat_search_device(const px_flat* idx, const float* d_queries, int64_t nq, int64_t k,
                          const uint8_t* d_mask, int64_t* d_ids, float* d_dists);

/*
 * No counterpart in the reference: px_flat_search_device for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Same arguments, results and checks as px_flat_search_device, but it calls no
 * hipMalloc, hipFree or other allocating routine: its work buffers (split candidate lists,
 * shared bounds, padded queries, a filter's compacted row ids) live in a fixed 64 MiB
 * device array that the library holds on each GPU it runs on until the process ends.
 * Limits: k <= 120 (every search takes the per-split list path); the buffers for nq queries
 * must fit the array (about nq * (k + 8) * 8 bytes per corpus split, plus nq * 132 bytes,
 * nq * padded dim * 4 when dim is not a multiple of 8, and 4 bytes per row with a mask);
 * larger calls return PX_ERR_ARG or PX_ERR_BAD_K naming the limit. The index's rows must
 * already be on the device (px_flat_add with the GPU present). Every call on one GPU uses
 * that GPU's one array: calls that overlap on the same GPU (from several threads or
 * handles) race and must be serialised by the caller. px_flat_last_timing is not updated.
 */
int px_flat_search_device_noalloc(const px_flat* idx, const float* d_queries, int64_t nq,
                                  int64_t k, const uint8_t* d_mask, int64_t* d_ids,
                                  float* d_dists);

/* Copy rows [first, first + n) out as row-major n x dim floats (FlatIndex::save needs the
 * data, flat.rs:64-66 -> lib.rs:19-30). */
int px_flat_get_vectors(const px_flat* idx, int64_t first, int64_t n, float* out);

int64_t px_flat_size(const px_flat* idx);         /* FlatIndex::len, flat.rs:51-53 */
int64_t px_flat_dim(const px_flat* idx);          /* FlatIndex::dim, flat.rs:48-50 */
int px_flat_metric(const px_flat* idx);           /* FlatIndex::metric, flat.rs:57-59 */
int64_t px_flat_memory_bytes(const px_flat* idx); /* FlatIndex::memory_bytes, flat.rs:60-62 */

/* ------------------------------------------------------------------------------------
 * PqIndex (crates/core/src/pq.rs:217-397).
 * ---------------------------------------------------------------------------------- */
typedef struct px_pq px_pq;

/* PyPq::new validation (crates/py/src/lib.rs:450-470): m >= 1, dim % m == 0, nbits 1..8 */
int px_pq_create(int metric, int64_t dim, int64_t m, int64_t nbits, px_pq** out);
void px_pq_destroy(px_pq* idx);
/* PqIndex::train, pq.rs:226-229 + ProductQuantizer::train pq.rs:54-105 (host k-means) */
int px_pq_train(px_pq* idx, const float* training, int64_t n, int64_t train_iters,
                int64_t train_sample, uint64_t seed);
/* Install trained codebooks [m][2^nbits][dim/m] directly (a loaded index). */
int px_pq_set_codebooks(px_pq* idx, const float* codebooks);
/* Copy the codebooks out ([m][2^nbits][dim/m] floats). */
int px_pq_get_codebooks(const px_pq* idx, float* out);
/* PqIndex::add, pq.rs:266-284: encode n rows (pq.rs:107-121) and append their codes. */
int px_pq_add(px_pq* idx, const float* vectors, int64_t n);
/* Append n pre-encoded code rows ([n][m] bytes). */
int px_pq_add_codes(px_pq* idx, const uint8_t* codes, int64_t n);
/* Copy codes [first, first + n) out ([n][m] bytes). */
int px_pq_get_codes(const px_pq* idx, int64_t first, int64_t n, uint8_t* out);

/* PqIndex::search_batch{,_filtered}, pq.rs:349-396. Same contract as px_flat_search. */
int px_pq_search(const px_pq* idx, const float* queries, int64_t nq, int64_t k,
                 const uint8_t* mask, int64_t* out_ids, float* out_dists);
/* Device-pointer form, as px_flat_search_device (queries checked on the device first). */
int px_pq_search_device(const px_pq* idx, const float* d_queries, int64_t nq, int64_t k,
                        const uint8_t* d_mask, int64_t* d_ids, float* d_dists);

int px_pq_is_trained(const px_pq* idx);
int64_t px_pq_size(const px_pq* idx);
int64_t px_pq_dim(const px_pq* idx);
int64_t px_pq_m(const px_pq* idx);
int64_t px_pq_nbits(const px_pq* idx);
int px_pq_metric(const px_pq* idx);
int64_t px_pq_memory_bytes(const px_pq* idx);     /* pq.rs:250-252 */
int64_t px_pq_raw_bytes(const px_pq* idx);        /* pq.rs:254-256 */

/* ------------------------------------------------------------------------------------
 * Device information and measurement support (no counterpart in the reference; the
 * reference's gpu_knn example queries cudaGetDeviceProperties, gpu_knn.rs:60-150).
 * ---------------------------------------------------------------------------------- */
/* Number of visible HIP devices (0 when there is none; never an error). */
int px_device_count(void);
/* name (NUL-terminated, truncated to name_len), compute units, HBM bytes, peak clock kHz */
int px_device_info(int device, char* name, size_t name_len, int* cu_count, int64_t* hbm_bytes,
                   int* clock_khz, char* arch, size_t arch_len);
/* HIP runtime and driver versions (hipRuntimeGetVersion / hipDriverGetVersion), for the
 * provenance of benchmark envelopes; crates/core/examples/gpu_knn.rs:287-295 records the
 * CUDA runtime and driver versions the same way. */
int px_hip_versions(int* runtime_version, int* driver_version);

/* Per-handle kernel timing with HIP events on the handle's stream (off by default). When
 * enabled, each search records the duration of its scan kernel and of the whole device
 * pipeline; the event markers between its kernels cost a few microseconds a search, so
 * throughput is measured with it off. */
int px_flat_set_timing(px_flat* idx, int enable);
int px_flat_last_timing(const px_flat* idx, float* scan_ms, float* total_ms, int* splits,
                        int* blocks);
/* Collect rounds of the handle's last search: 0 when it used per-split candidate lists,
 * else the rounds of the threshold-collect path (1 when every query finished in the
 * first). Diagnostic; no counterpart in the reference. */
int px_flat_last_rounds(const px_flat* idx, int* rounds);
/* Selection path of the handle's last search: PX_PATH_LISTS (per-split candidate lists),
 * PX_PATH_COLLECT_SAMPLED (threshold-collect whose first round takes its thresholds from a
 * strided row sample), PX_PATH_COLLECT_BOUNDED (threshold-collect whose first round is
 * bounded by the splits' shared bound alone, no sample), PX_PATH_VECTOR (the vector-ALU
 * collect scan of a few queries), PX_PATH_FULL_SORT (k past PX_MAX_K). Diagnostic; no
 * counterpart in the reference. */
#define PX_PATH_LISTS 0
#define PX_PATH_COLLECT_SAMPLED 1
#define PX_PATH_COLLECT_BOUNDED 2
#define PX_PATH_VECTOR 3
#define PX_PATH_FULL_SORT 4 /* k past PX_MAX_K: every key computed and sorted */
int px_flat_last_path(const px_flat* idx, int* path);
/* Use of the fp16 copy of 128-dim rows. The copy (2 bytes a value) is kept from the first
 * px_flat_add while every row added is exactly an fp16 zero or normal number (integer-valued
 * descriptors such as SIFT's are). With it, a batch whose queries are exact too multiplies
 * on the fp16 matrix cores with fp32 accumulation in the collect scan, and in the per-split
 * list scan on at least 65,536 rows (each product is exact in fp16 as in fp32; the
 * candidates are re-ranked in the reference's arithmetic as on fp32), and the vector-ALU
 * scan of batches of at most 16 queries reads the copy and widens it to the same fp32
 * values. enable = 0 keeps both scans on the fp32 rows (default 1). Diagnostic and
 * tuning; no counterpart in the reference. */
int px_flat_set_scan_f16(px_flat* idx, int enable);
/* *used = 1 if the handle's last search read the fp16 copy of the rows (either scan), else
 * 0. */
int px_flat_last_scan_f16(const px_flat* idx, int* used);
/* Polls a stage-sync wait of the barrier-free scans (the collect scans; lists of k + 8 <= 32)
 * makes before it gives up; 0 (the default) keeps the kernels' own, 2^16 polls, about 5 ms.
 * A wait that gives up lets its wave go on (every kernel still ends) and is reported: the
 * merge or select writes nothing and the search fails with PX_ERR_DEVICE, its outputs
 * unwritten. A handle's later searches are unaffected. Test hook (a small limit forces the
 * give-up); no counterpart in the reference. */
int px_flat_set_spin_limit(px_flat* idx, int polls);
/* The same for PqIndex searches (k <= 128: per-wave lists; above: threshold-collect). */
int px_pq_last_rounds(const px_pq* idx, int* rounds);
int px_pq_set_timing(px_pq* idx, int enable);
int px_pq_last_timing(const px_pq* idx, float* scan_ms, float* total_ms, int* splits,
                      int* blocks);

/* Device memory plumbing for callers without their own HIP runtime (benchmarks). */
int px_dev_alloc(void** ptr, size_t bytes);
int px_dev_free(void* ptr);
int px_dev_upload(void* dst, const void* src, size_t bytes);
int px_dev_download(void* dst, const void* src, size_t bytes);
/* Streaming copy kernel of `bytes` (multiple of 16): calibrates HBM traffic counters. */
int px_dev_copy_kernel(void* dst, const void* src, size_t bytes, float* ms);
/* LDS read-rate calibration for the PQ scan's roofline: `blocks` workgroups of 512 threads,
 * each thread `iters` x 16 reads of 16 bytes from a 64 KB LDS table, with no bank conflict
 * (random = 0) or at uniform random slots (random = 1: the ADC scan's gathers). *ms: kernel
 * time; *bytes: bytes read. No counterpart in the reference. */
int px_dev_lds_gather(int random, int blocks, int iters, float* ms, double* bytes);

#ifdef __cplusplus
}
#endif
#endif
