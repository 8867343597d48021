// px_sort.hip -- exact top-k for any k, by a full sort of every key.
//
// The reference's FlatIndex and PqIndex take any k (crates/core/src/flat.rs:106-148 and
// pq.rs:299-347 keep a heap of k over every row). The fused scans serve k up to PX_MAX_K;
// past it a chunk of queries has every key computed in the reference's arithmetic
// (flat: distance.rs:3-39 with contraction off; PQ: the ADC sum of pq.rs:320-323 from the
// scan's dense mode), packed as (query, total-order key) 64-bit sort keys with the row
// position as the value, sorted once with a stable LSD radix sort (so equal keys keep the
// lower position first), and the first k of each query are finished (sqrt / negate, or raw
// keys) and padded as flat.rs:229-237 does.
#include <hipcub/hipcub.hpp>

#include <cfloat>

#include "px_device.h"
#include "px_kernels.h"

namespace px {

// keys[q][i] = the reference key of row (rowidx ? rowidx[i] : i) for query q0 + q.
__global__ __launch_bounds__(256) void flat_exact_keys_kernel(const float* corpus,
                                                              const float* queries,
                                                              const int* rowidx, int64_t n_eff,
                                                              int dim, int dp, int l2,
                                                              float* keys) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int q = blockIdx.y;
    if (i >= n_eff) return;
    const int64_t row = rowidx ? rowidx[i] : i;
    const float* qv = queries + (int64_t)q * dp;
    const float* xv = corpus + row * dp;
    keys[(int64_t)q * n_eff + i] = l2 ? ref_key_v(qv, xv, dim, true) : -ref_key_v(qv, xv, dim, false);
}

hipError_t launch_flat_exact_keys(const float* corpus, const float* queries, const int* rowidx,
                                  int64_t n_eff, int qc, int dim, int dp, int metric,
                                  float* keys, hipStream_t s) {
    if (n_eff <= 0 || qc <= 0) return hipSuccess;
    const dim3 grid((unsigned)((n_eff + 255) / 256), (unsigned)qc);
    hipLaunchKernelGGL(flat_exact_keys_kernel, grid, dim3(256), 0, s, corpus, queries, rowidx,
                       n_eff, dim, dp, metric == 0 ? 1 : 0, keys);
    return hipGetLastError();
}

// sort key: query in the high word, the total-order key mapped to unsigned order below;
// value: the position
__global__ void full_sort_pack_kernel(const float* keys, int64_t n_eff, int64_t count,
                                      unsigned long long* skeys, int* spos) {
    const int64_t x = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (x >= count) return;
    const int64_t q = x / n_eff;
    skeys[x] = ((unsigned long long)q << 32) | ((unsigned)total_key(keys[x]) ^ 0x80000000u);
    spos[x] = (int)(x - q * n_eff);
}

// outputs of query q (q < qc): the first k of its sorted keys, then padding
__global__ void full_sort_emit_kernel(const unsigned long long* skeys, const int* spos,
                                      const int* rowidx, int64_t n_eff, int64_t k, int metric,
                                      int raw_keys, int64_t* out_ids, float* out_dists) {
    const int64_t x = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t q = blockIdx.y;
    if (x >= k) return;
    int64_t id = -1;
    float d = raw_keys ? FLT_MAX : (metric == 0 ? FLT_MAX : -FLT_MAX);
    if (x < n_eff) {
        const int64_t at = q * n_eff + x;
        const int tk = (int)((unsigned)(skeys[at] & 0xffffffffull) ^ 0x80000000u);
        const float kv = __int_as_float(tk ^ (int)(((unsigned)(tk >> 31)) >> 1));
        const int pos = spos[at];
        id = rowidx ? rowidx[pos] : pos;
        d = raw_keys ? kv : (metric == 0 ? sqrtf(kv) : -kv);
    }
    out_ids[q * k + x] = id;
    out_dists[q * k + x] = d;
}

size_t full_sort_temp_bytes(int64_t count) {
    size_t bytes = 0;
    (void)hipcub::DeviceRadixSort::SortPairs(nullptr, bytes, (const unsigned long long*)nullptr,
                                             (unsigned long long*)nullptr, (const int*)nullptr,
                                             (int*)nullptr, count, 0, 64);
    return bytes;
}

hipError_t launch_full_sort(const float* keys, int64_t n_eff, int qc, const int* rowidx,
                            int64_t k, int metric, int raw_keys, void* scratch,
                            size_t scratch_bytes, int64_t* out_ids, float* out_dists,
                            hipStream_t s) {
    const int64_t count = n_eff * qc;
    // scratch: two sort-key buffers, two position buffers, then the radix sort's own
    auto align = [](size_t v) { return (v + 255) & ~(size_t)255; };
    char* base = static_cast<char*>(scratch);
    unsigned long long* k0 = reinterpret_cast<unsigned long long*>(base);
    unsigned long long* k1 = reinterpret_cast<unsigned long long*>(base + align(8 * count));
    int* p0 = reinterpret_cast<int*>(base + 2 * align(8 * count));
    int* p1 = reinterpret_cast<int*>(base + 2 * align(8 * count) + align(4 * count));
    void* tmp = base + 2 * align(8 * count) + 2 * align(4 * count);
    const size_t used = 2 * align(8 * count) + 2 * align(4 * count);
    size_t tmp_bytes = full_sort_temp_bytes(count);
    if (used + tmp_bytes > scratch_bytes) return hipErrorInvalidValue;
    if (count > 0) {
        hipLaunchKernelGGL(full_sort_pack_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256),
                           0, s, keys, n_eff, count, k0, p0);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        int qbits = 0;
        while ((1ll << qbits) < qc) ++qbits;
        e = hipcub::DeviceRadixSort::SortPairs(tmp, tmp_bytes, k0, k1, p0, p1, count, 0,
                                               32 + qbits, s);
        if (e != hipSuccess) return e;
    }
    const dim3 grid((unsigned)((k + 255) / 256), (unsigned)qc);
    hipLaunchKernelGGL(full_sort_emit_kernel, grid, dim3(256), 0, s, k1, p1, rowidx, n_eff, k,
                       metric, raw_keys, out_ids, out_dists);
    return hipGetLastError();
}

size_t full_sort_scratch_bytes(int64_t n_eff, int qc) {
    const int64_t count = n_eff * qc;
    auto align = [](size_t v) { return (v + 255) & ~(size_t)255; };
    return 2 * align(8 * count) + 2 * align(4 * count) + full_sort_temp_bytes(count);
}

}  // namespace px
