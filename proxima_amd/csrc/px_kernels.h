// px_kernels.h -- host-side launchers for the gfx950 kernels of libproxima_px.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace px {

// Device row layout: row-major [rows][dp] fp32 with dp = round_up(dim, 8) and the pad
// columns zero, so every row starts 32-byte aligned and MFMA K-steps come in groups of 8.
inline int64_t padded_dim(int64_t dim) { return (dim + 7) / 8 * 8; }

// Longest candidate list the fused kernels keep per query (k' = k + margin <= 128).
constexpr int kMaxList = 128;
// Largest split-merge width: splits * k' candidates per query sorted in LDS (128 KB).
constexpr int kMaxMerge = 16384;
// Longest split whose list positions fit 16-bit offsets (0xffff is the empty sentinel).
constexpr int64_t kMaxNarrowSplitRows = 65472;
bool flat_list_narrow_ids(int kp);

struct FlatScanArgs {
    const float* corpus;   // [n][dp] row-major, zero pad columns
    const float* norms;    // [n] squared norms (L2 only)
    const float* queries;  // [nq][dp] row-major, zero pad columns
    const int* rowidx;     // optional: ascending row ids of the rows to scan (filter)
    int64_t n_eff;         // rows to scan (rowidx length when filtered)
    int64_t rows_per_split;
    int dp;
    int nq;
    int kl;                // list length k' (<= kp); collect mode with gbest: rank of the bound
    int splits;
    int metric;            // 0 = L2, 1 = inner product
    float* part_keys;      // [nq][splits][kl]
    int* part_ids;         // compacted positions (row ids when unfiltered)
    int* gtau;             // [nq] shared per-query bound, total-order ints; starts at +inf
    int* gbest;            // [32][gbest_ld] per-split published keys, total-order ints
                           // (slot s of query q at s * gbest_ld + q); +inf. Slot-major:
                           // a wave's atomics and loads for consecutive queries share cache
                           // lines, where a query's 32 slots in one line drew every split's
                           // atomics to it. Collect mode: optional (kl <= min(splits, 32),
                           // one 128-dim chunk); each split publishes its smallest key and
                           // rows above the kl-th smallest published key are not appended
    int64_t gbest_ld;      // >= the queries indexed (nq, or the batch's with a qlist)
    // Collect mode (launch_flat_collect): no lists; every row whose (key, position) is at or
    // below its query's threshold is appended to the region of (query slot, split).
    const int* qlist;      // optional: query index of each of the nq slots
    const int* thr_key;    // [queries] threshold keys as total-order ints (by query index)
    const int* thr_pos;    // [queries] threshold positions (ties: position <= thr_pos passes)
    float* cand_keys;      // [nq slots][splits][2][cap]: one region per lane of the query's pair
    int* cand_pos;         // positions (indices into rowidx when filtered)
    int* cand_count;       // [nq slots][splits][2] rows that passed; more than cap = overflow
    int cap;
    // optional (launch_flat_collect, 128-dim rows), [nq slots][splits][2]: where a region's
    // count passes cap, the smallest key of the rows it dropped as a total-order int (it
    // keeps its first cap rows); without it a full region keeps rewriting its last slot
    int* cand_dmin;
    // dense != 0: no thresholds; every key goes to cand_keys as [slot][dense_ld] by position
    // (keys of rows past a split's end are +inf; dense_ld >= splits * rows_per_split)
    int dense;
    int64_t dense_ld;
    // optional: one device int; equal to abort_seq when the scan starts (a query of this
    // search failed its finiteness check), it makes the whole launch a no-op
    const int* abort;
    int abort_seq;
    // debug build: the launch's debug word (null: no checks) and the corpus rows that row
    // ids must stay below
    int* dbg;
    int64_t rows;
    // rows of several 128-dim chunks over several rounds of workgroups: XCD-major block order
    // (flat_scan_kernel), the grid padded to a multiple of 8
    int xcd_major;
    // optional: set nonzero if a stage-sync wait of the scan gave up (the barrier-free
    // scans: collect mode, the collect scan of 128-dim rows, lists of 32); the results of
    // that launch are not to be used, and the merge or select after it writes nothing
    int* spin_fail;
    // polls before a stage-sync wait gives up; 0: kSpinLimit (about 5 ms). Tests lower it
    // to force a give-up (px_flat_set_spin_limit)
    int spin_limit;
    // optional (launch_flat_collect, 128-dim rows), both or neither: the corpus [n][128] and
    // the queries [nq][128] as fp16 bit patterns, given only when every value of both is
    // exactly representable in fp16; the scan then multiplies in fp16 (exact products,
    // fp32 accumulation): its keys equal the fp32 scan's up to the rounding of the sums
    const unsigned short* corpus_h;
    const unsigned short* queries_h;
};

// Waves per workgroup and list capacity used for a list length kl.
int flat_list_capacity(int kl);
int flat_queries_per_block(int kp);
// Lists of capacity kp over rows of dp padded dims: whether launch_flat_scan takes
// flat_list16q_kernel (lists of 32, 129-384 dims), and the query slots a workgroup holds.
bool list_resident_queries(int kp, int64_t dp);
int flat_list_queries_per_block(int kp, int64_t dp);
hipError_t launch_flat_scan(const FlatScanArgs& a, hipStream_t s);
// Total-order int of +inf: the starting value of FlatScanArgs::gtau.
constexpr int kTotalKeyInf = 0x7f800000;
// Threshold-collect selection for k' past the lists (k' > kMaxList): thresholds from a
// sample of rows spread evenly over the corpus, one collect scan, per-query select; queries whose threshold proved too
// tight or too loose go round again.
hipError_t launch_flat_collect(const FlatScanArgs& a, hipStream_t s);
hipError_t launch_flat_collect_v1(const FlatScanArgs& a, hipStream_t s);
// The collect scan of rows of 129-384 padded dims (not dense, no shared bound): 16 queries a
// wave resident in registers, 128 query slots a workgroup (flat_list16q_kernel's collect mode).
bool collect_resident_queries(int64_t dp);
hipError_t launch_flat_collect16q(const FlatScanArgs& a, hipStream_t s);
// The collect scan of fp16 rows (corpus_h and queries_h given, dp 128, not dense): 64
// queries a wave, flat_collect16_queries_per_block() query slots a workgroup; called by
// launch_flat_collect.
hipError_t launch_flat_collect16(const FlatScanArgs& a, hipStream_t s);
int flat_collect16_queries_per_block();
// The collect scan for a few query slots (nq <= kVecQueries, dp <= kVecMaxDp) on the
// vector ALUs: the MFMA scan's 32-query tiles would be nearly all padding, so this one
// streams the corpus at memory speed instead. One region per (slot, split):
// cand_keys [nq slots][splits][cap], cand_count [nq slots][splits]; dense: every key to
// cand_keys [nq slots][n_eff] (no thresholds, no counts).
// (16 queries: 1M x 128 took 0.31 ms against the lists' 0.39 ms; 24 queries: 0.45 against
// 0.41 ms, the vector ALUs' FMAs growing with the slots)
constexpr int kVecQueries = 16;
constexpr int kVecMaxDp = 1024;
constexpr int kVecMaxQueryFloats = 16384;  // nq * dp: the queries' 64 KB of LDS
static_assert(kVecQueries * kVecMaxDp <= kVecMaxQueryFloats, "query rows past 64 KB of LDS");
hipError_t launch_flat_vcollect(const FlatScanArgs& a, hipStream_t s);
// Threshold ladder rungs taken from the sample, loosest last; past the last rung a query's
// threshold is +inf (every row passes).
constexpr int kRungs = 2;
// Most candidates one query's select holds in LDS (8 bytes each, 128 KB).
constexpr int kMaxCollect = 16384;
// Most candidate regions per query of a collect scan (two per split; the select walks
// their counts).
constexpr int kMaxCollectRegions = 1024;
struct CollectSelectArgs {
    const float* cand_keys;  // FlatScanArgs regions of the collect scan
    const int* cand_pos;
    const int* cand_count;
    // optional: FlatScanArgs::cand_dmin of the scan. A query whose regions overflowed but
    // whose k'-th smallest kept key is below every dropped key finishes (the dropped rows
    // cannot be among its best k'); without it an overflow always goes round again.
    const int* cand_dmin;
    int regions, cap;        // regions per query slot (2 x splits), capacity of each
    int lcap;                // candidates the launch's LDS holds (power of two <= kMaxCollect)
    const int* qlist;        // optional: query index of each slot (one workgroup per slot)
    const int* rowidx;       // optional: position -> row id
    int* thr_key;            // [queries] in/out
    int* thr_pos;
    const int* ladder_key;   // [queries][kRungs]
    const int* ladder_pos;
    int* rung;               // [queries] current rung (kRungs once the threshold is +inf)
    int* status;             // [queries] 0: outputs written; 1: collect again
    int kk;                  // candidates re-ranked exactly (k + margin)
    int k;
    int metric;
    // optional [32][gbest_ld]: the scan's shared-bound slots (FlatScanArgs::gbest). The
    // kk-th smallest slot bounds the best kk, and every row at or below it was collected,
    // so a finishing query sorts only the candidates at or below it.
    const int* gbest;
    int64_t gbest_ld;
    const float* corpus;     // nullptr: keys are exact already (PQ), no re-rank
    const float* queries;
    int dim, dp;
    int64_t* out_ids;
    float* out_dists;
    int raw_keys;
    int* dbg;                // debug build: as FlatScanArgs::dbg
    // optional: the scan's FlatScanArgs::spin_fail; nonzero, the launch writes nothing (no
    // outputs, no status words: the host fails the search)
    const int* spin_fail;
};
hipError_t launch_collect_select(const CollectSelectArgs& a, int slots, hipStream_t s);
// Threshold ladder from the dense keys of a collect scan over a row sample: per query,
// rung i is a key value with at least ranks[i] sampled keys at or below it (the upper end
// of the 2^-24-wide bin, in total order, that holds the ranks[i]-th smallest), position
// limit kIdNone (every row with that key passes); rung 0 also goes to thr, rung = 0.
struct LadderArgs {
    const float* keys;       // row-major [nq][ld]: the sampled keys of each query
    int64_t ld;              // row pitch (>= count)
    int count;               // sampled rows (keys a query)
    int nq;
    int ranks[kRungs];
    int* ladder_key;         // [nq][kRungs]
    int* ladder_pos;
    int* thr_key;            // [nq]
    int* thr_pos;
    int* rung;
};
// Most sampled keys (64 per block) a ladder workgroup holds in registers.
constexpr int kMaxLadderEntries = 24576;
hipError_t launch_ladder(const LadderArgs& a, hipStream_t s);
// Row sample of the collect path, count rows spread evenly over n_eff positions:
// position p_i = floor(i * n_eff / count), row[i] = rowidx ? rowidx[p_i] : p_i.
hipError_t launch_sample_rows(const int* rowidx, int64_t count, int64_t n_eff, int* row,
                              hipStream_t s);
hipError_t launch_fill_int(int* p, int64_t n, int v, hipStream_t s);
// n ints from device memory to host memory that is pinned and mapped for the device
// (hipHostMallocMapped), by a kernel on stream s: the host reads them once the stream has
// drained. A hipMemcpyAsync to the host may instead be given to a copy engine whose queue the
// runtime creates on first use, and creating a queue preempts the kernels running on the
// device; this read-back never does.
hipError_t launch_copy_to_host(const int* src, int* host_dst, int64_t n, hipStream_t s);

struct MergeArgs {
    const float* part_keys;  // [nq][width] candidates (key, id/position)
    const int* part_ids;
    const int* rowidx;       // optional: position -> row id
    int width;               // candidates per query (splits * kl)
    // optional [nq] total-order key bounds (the scan's gtau): a split's full list tail, so
    // every candidate of the best kl has a key at or below it; +inf: no bound
    const int* bound;
    // optional [32][gbest_ld] published split keys (the scan's gbest) and the scan's split
    // count: slot i holds a key with m = ceil(kl / min(splits, 32)) candidates of one split
    // at or below it, so the ceil(kl / m)-th smallest slot bounds the best kl as well
    const int* gbest;
    int64_t gbest_ld;
    int splits;
    // nonzero: the candidates are width / kl lists of kl, each in ascending order (PQ); with
    // no published bounds, the kl-th smallest list head bounds the best kl
    int sorted_lists;
    int nq;
    int kl;                  // candidates kept after the first sort
    int k;                   // outputs per query
    int metric;
    // exact re-rank (flat only); corpus == nullptr keeps the incoming keys (PQ: exact already)
    const float* corpus;     // [n][dp]
    const float* queries;    // [nq][dp]
    int dim;                 // true dimension (reference op order runs over dim, not dp)
    int dp;
    // outputs
    int64_t* out_ids;        // [nq][k], -1 padding
    float* out_dists;        // [nq][k] finished (sqrt / negate) or raw keys when raw_keys
    int raw_keys;            // 1: write raw keys (FLT_MAX padding) instead of distances
    const int* abort;        // optional, as FlatScanArgs::abort: equal to abort_seq, nothing
    int abort_seq;           // is written
    // optional: the scan's FlatScanArgs::spin_fail; nonzero, nothing is written either
    const int* spin_fail;
    // optional: workgroup 0 stores *abort (0 without abort) to verdict[0] and *spin_fail (0
    // without it) to verdict[1] (two mapped host ints' device address), so the host reads
    // the search's finiteness and stage-sync verdicts with no copy of its own
    int* verdict;
    int* dbg;                // debug build: as FlatScanArgs::dbg
};
hipError_t launch_merge(const MergeArgs& a, hipStream_t s);

hipError_t launch_row_norms(const float* x, int64_t rows, int dp, float* out, hipStream_t s);
hipError_t launch_pad_rows(const float* src, int64_t rows, int dim, int dp, float* dst,
                           hipStream_t s);

// *flag = 1 when any of x[0 .. count) is NaN or infinite, else 0 (the flag is cleared first).
hipError_t launch_nonfinite_check(const float* x, int64_t count, int* flag, hipStream_t s);
// out[0 .. count) = x as fp16 bit patterns; atomically ORs bit into *inexact when any value
// is not exactly an fp16 zero or normal number (the caller clears it). count % 4 == 0, x
// 16-byte and out 8-byte aligned.
hipError_t launch_to_f16(const float* x, int64_t count, unsigned short* out, int* inexact,
                         hipStream_t s, int bit = 1);
// The per-split list path's first kernel: *flag = max(*flag, seq) when any of count floats
// of x is NaN or infinite (flag is never cleared: each search takes a larger seq; count 0:
// no check, flag may be null), gtau[0..ngtau) and gbest[0..ngbest) filled with
// kTotalKeyInf, and *zero (optional: the scan's spin_fail word) cleared. One launch where a
// flag fill, the check and three fills took five.
hipError_t launch_list_prologue(const float* x, int64_t count, int* flag, int seq, int* gtau,
                                int64_t ngtau, int* gbest, int64_t ngbest, int* zero,
                                hipStream_t s);

// Ordered compaction of a keep-mask (nonzero = keep) into ascending row ids.
// scratch must hold mask_compact_scratch(n) ints; *d_count receives the kept count.
int64_t mask_compact_scratch(int64_t n);
hipError_t launch_mask_compact(const uint8_t* mask, int64_t n, int* rowidx, int* scratch,
                               int* d_count, hipStream_t s);

struct PqScanArgs {
    const uint8_t* codes;     // [n][m]
    const float* codebooks;   // [m][ks][dsub]
    const float* queries;     // [nq][dim]
    const int* rowidx;        // optional filter positions
    int64_t n_eff;
    int64_t rows_per_split;
    int dim, m, ks, dsub;
    int nq;
    int kl;
    int splits;
    int metric;
    float* part_keys;         // [nq][splits * waves][kl]
    int* part_ids;
    // Collect mode (launch_pq_collect), as FlatScanArgs: thresholds by query index, regions
    // [nq slots][splits][waves][cap] with counts [nq slots][splits][waves]; or, with dense,
    // every key to cand_keys[q][n_eff] (no thresholds, no counts).
    const int* qlist;
    const int* thr_key;
    const int* thr_pos;
    float* cand_keys;
    int* cand_pos;
    int* cand_count;
    int cap;
    int dense;
    int* dbg;                 // debug build: as FlatScanArgs::dbg ...
    int64_t rows;             // ... and the code rows
};
int pq_list_capacity(int kl);
int pq_lists_per_split();
// Rows a PQ workgroup's waves take per step (waves x 64): wave w takes rows 64 w .. 64 w + 63
// of every step, so splits of a multiple of it give every wave the same share.
int pq_rows_per_block_step();
int pq_queries_per_block(int m, int ks);
hipError_t launch_pq_scan(const PqScanArgs& a, hipStream_t s);
hipError_t launch_pq_collect(const PqScanArgs& a, hipStream_t s);

// PQ training and encoding (px_pq_kmeans.hip). One Lloyd iteration over all m subspaces:
// data sub-major [m][n][d], centroids [m][ks][d] updated in place, asg [m][pitch(n)] bytes,
// counts [m][ks], rng [m] SplitMix64 states.
int64_t pq_train_asg_pitch(int64_t n);
hipError_t launch_pq_train_iteration(const float* data, int64_t n, int d, int ks, int m,
                                     float* cents, uint8_t* asg, int* counts, uint64_t* rng,
                                     hipStream_t s);
// codes[i][sub] = nearest of books[sub] to vectors[i][sub*d ..), vectors [n][dim].
hipError_t launch_pq_encode(const float* vectors, int64_t n, int dim, int d, int ks, int m,
                            const float* books, uint8_t* codes, hipStream_t s);

// Exact top-k for k past PX_MAX_K (px_sort.hip): keys[q][i] of a chunk of qc queries in
// the reference's arithmetic (flat; PQ keys come from the dense ADC scan), then one stable
// radix sort by (query, key) with positions as values and the first k of each query
// finished and padded. scratch holds full_sort_scratch_bytes(n_eff, qc).
hipError_t launch_flat_exact_keys(const float* corpus, const float* queries, const int* rowidx,
                                  int64_t n_eff, int qc, int dim, int dp, int metric,
                                  float* keys, hipStream_t s);
size_t full_sort_scratch_bytes(int64_t n_eff, int qc);
hipError_t launch_full_sort(const float* keys, int64_t n_eff, int qc, const int* rowidx,
                            int64_t k, int metric, int raw_keys, void* scratch,
                            size_t scratch_bytes, int64_t* out_ids, float* out_dists,
                            hipStream_t s);
// Plain streaming copy (calibrates HBM traffic counters against known bytes).
hipError_t launch_copy(const float4* src, float4* dst, int64_t n4, hipStream_t s);
// LDS read-rate calibration: blocks x lds_gather_threads() threads, each iters x 16 reads of
// 16 bytes from a 64 KB table (random = 0: no bank conflicts; 1: uniform random slots, the
// ADC scan's gathers); out holds one float per thread.
int lds_gather_threads();
hipError_t launch_lds_gather(int random, int blocks, int iters, float* out, hipStream_t s);

}  // namespace px
