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
    int kl;                // list length k' (<= kp)
    int splits;
    int metric;            // 0 = L2, 1 = inner product
    float* part_keys;      // [nq][splits][kl]
    int* part_ids;         // compacted positions (row ids when unfiltered)
    int* gtau;             // [nq] shared per-query bound, total-order ints; starts at +inf
    int* gbest;            // [nq][32] per-split published list keys, total-order ints; +inf
};

// Waves per workgroup and list capacity used for a list length kl.
int flat_list_capacity(int kl);
int flat_queries_per_block(int kp);
hipError_t launch_flat_scan(const FlatScanArgs& a, hipStream_t s);
// Total-order int of +inf: the starting value of FlatScanArgs::gtau.
constexpr int kTotalKeyInf = 0x7f800000;
hipError_t launch_fill_int(int* p, int64_t n, int v, hipStream_t s);

struct MergeArgs {
    const float* part_keys;  // [nq][width] candidates (key, id/position)
    const int* part_ids;
    const int* rowidx;       // optional: position -> row id
    int width;               // candidates per query (splits * kl)
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
};
hipError_t launch_merge(const MergeArgs& a, hipStream_t s);

hipError_t launch_row_norms(const float* x, int64_t rows, int dp, float* out, hipStream_t s);
hipError_t launch_pad_rows(const float* src, int64_t rows, int dim, int dp, float* dst,
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
};
int pq_list_capacity(int kl);
int pq_lists_per_split();
int pq_queries_per_block(int m, int ks);
hipError_t launch_pq_scan(const PqScanArgs& a, hipStream_t s);

// Plain streaming copy (calibrates HBM traffic counters against known bytes).
hipError_t launch_copy(const float4* src, float4* dst, int64_t n4, hipStream_t s);

}  // namespace px
