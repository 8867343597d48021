// px_pq_kmeans.hip -- PQ Lloyd iterations and encoding on gfx950.
//
// The GPU side of PqIndex::train/add (crates/core/src/pq.rs:107-121, 149-193, 266-284),
// bit-identical to the reference's host code: every distance is ref_l2_sqr (the 8-lane
// order of distance.rs:3-21, no FMA), argmins keep the lower centroid on ties (strict '<'
// from FLT_MAX), each centroid coordinate is summed over its rows in row order and scaled by
// the correctly rounded reciprocal of the count, and empty clusters are re-seeded in
// cluster order from each subspace's SplitMix64 stream. The training sample, the initial
// centroids and the generator states come from the host plan (px_pq_train.cpp).
//
// Work per Lloyd iteration at 50,000 sampled rows, m = 16, 256 centroids of 8 dims: the
// assignment is 50,000 x 16 x 256 distances (one thread per (row, subspace)); the update is
// one thread per (subspace, centroid, coordinate), each walking the assignment in row order
// -- sequential by definition, 4,096 walks of 50,000 bytes that all waves read in step.
#include "px_device.h"
#include "px_kernels.h"

#include <float.h>

namespace px {

// argmin over ks centroids of dimension d, strict '<' from FLT_MAX (pq.rs:157-165)
__device__ __forceinline__ int nearest_centroid(const float* v, const float* cents, int ks, int d) {
    int best = 0;
    float best_d = FLT_MAX;
    for (int c = 0; c < ks; ++c) {
        const float dist = ref_l2_sqr(v, cents + (int64_t)c * d, d);
        if (dist < best_d) {
            best_d = dist;
            best = c;
        }
    }
    return best;
}

// asg[sub][i] = nearest centroid of sample row i in subspace sub; data is sub-major
// [m][n][d], cents [m][ks][d], asg [m][n_pad].
__global__ __launch_bounds__(256) void pq_train_assign_kernel(const float* data, int64_t n,
                                                              int64_t n_pad, int d, int ks,
                                                              const float* cents, uint8_t* asg) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int sub = blockIdx.y;
    if (i >= n) return;
    asg[(int64_t)sub * n_pad + i] = (uint8_t)nearest_centroid(
        data + ((int64_t)sub * n + i) * d, cents + (int64_t)sub * ks * d, ks, d);
}

// One thread per (subspace, centroid c, coordinate x): the sum of coordinate x over the
// rows assigned to c, in row order (pq.rs:170-178), then the mean by reciprocal multiply
// (pq.rs:185-188). Empty clusters keep their centroid here; the re-seed kernel follows.
// The assignment (one byte per row, rows of a subspace padded to 16 bytes) streams through
// LDS in 8 KB chunks that every thread of the block walks in step.
constexpr int kAsgChunk = 8192;
__global__ __launch_bounds__(256) void pq_train_update_kernel(const float* data, int64_t n,
                                                              int64_t n_pad, int d, int ks,
                                                              const uint8_t* asg, float* cents,
                                                              int* counts) {
    __shared__ uint4 chunk[kAsgChunk / 16];
    const int t = blockIdx.x * 256 + threadIdx.x;
    const int sub = blockIdx.y;
    const int c = t / d, x = t - c * d;
    const bool live = c < ks;
    const uint4* a = reinterpret_cast<const uint4*>(asg + (int64_t)sub * n_pad);
    const float* rows = data + (int64_t)sub * n * d + (live ? x : 0);
    float s = 0.f;
    int cnt = 0;
    for (int64_t base = 0; base < n; base += kAsgChunk) {
        const int words = (int)((min<int64_t>(kAsgChunk, n_pad - base) + 15) / 16);
        __syncthreads();
        for (int w = threadIdx.x; w < words; w += 256) chunk[w] = a[base / 16 + w];
        __syncthreads();
        if (!live) continue;
        for (int w = 0; w < words; ++w) {
            const uint4 v = chunk[w];
            const unsigned part[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int b = 0; b < 16; ++b) {
                const int64_t i = base + w * 16 + b;
                if ((int)((part[b >> 2] >> (8 * (b & 3))) & 0xffu) == c && i < n) {
                    s = s + rows[i * d];
                    ++cnt;
                }
            }
        }
    }
    if (!live) return;
    if (x == 0) counts[sub * ks + c] = cnt;
    if (cnt > 0) {
        const float inv = 1.0f / (float)cnt;
        cents[((int64_t)sub * ks + c) * d + x] = s * inv;
    }
}

__device__ __forceinline__ uint64_t splitmix_next(uint64_t& s) {  // pq.rs:27-33
    s += 0x9E3779B97F4A7C15ull;
    uint64_t z = s;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// One thread per subspace: empty clusters, in cluster order, take a random sample row
// (pq.rs:180-184), advancing the subspace's generator.
__global__ void pq_train_reseed_kernel(const float* data, int64_t n, int d, int ks, int m,
                                       const int* counts, float* cents, uint64_t* rng) {
    const int sub = blockIdx.x * blockDim.x + threadIdx.x;
    if (sub >= m) return;
    uint64_t s = rng[sub];
    for (int c = 0; c < ks; ++c) {
        if (counts[sub * ks + c] != 0) continue;
        const int64_t idx = (int64_t)(splitmix_next(s) % (uint64_t)n);
        for (int x = 0; x < d; ++x)
            cents[((int64_t)sub * ks + c) * d + x] = data[((int64_t)sub * n + idx) * d + x];
    }
    rng[sub] = s;
}

// codes[i][sub] = nearest centroid of vectors[i][sub*d .. sub*d + d) (pq.rs:107-121)
__global__ __launch_bounds__(256) void pq_encode_kernel(const float* vectors, int64_t n, int dim,
                                                        int d, int ks, int m, const float* books,
                                                        uint8_t* codes) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int sub = blockIdx.y;
    if (i >= n) return;
    codes[i * m + sub] = (uint8_t)nearest_centroid(vectors + i * dim + (int64_t)sub * d,
                                                   books + (int64_t)sub * ks * d, ks, d);
}

int64_t pq_train_asg_pitch(int64_t n) { return (n + 15) / 16 * 16; }

hipError_t launch_pq_train_iteration(const float* data, int64_t n, int d, int ks, int m,
                                     float* cents, uint8_t* asg, int* counts, uint64_t* rng,
                                     hipStream_t s) {
    if (n <= 0 || m <= 0 || m > 65535 || (n + 255) / 256 > 0x7fffffff) return hipErrorInvalidValue;
    const int64_t n_pad = pq_train_asg_pitch(n);
    hipLaunchKernelGGL(pq_train_assign_kernel, dim3((unsigned)((n + 255) / 256), (unsigned)m),
                       dim3(256), 0, s, data, n, n_pad, d, ks, cents, asg);
    hipLaunchKernelGGL(pq_train_update_kernel, dim3((unsigned)((ks * d + 255) / 256), (unsigned)m),
                       dim3(256), 0, s, data, n, n_pad, d, ks, asg, cents, counts);
    hipLaunchKernelGGL(pq_train_reseed_kernel, dim3((unsigned)((m + 63) / 64)), dim3(64), 0, s,
                       data, n, d, ks, m, counts, cents, rng);
    return hipGetLastError();
}

hipError_t launch_pq_encode(const float* vectors, int64_t n, int dim, int d, int ks, int m,
                            const float* books, uint8_t* codes, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(pq_encode_kernel, dim3((unsigned)((n + 255) / 256), (unsigned)m), dim3(256),
                       0, s, vectors, n, dim, d, ks, m, books, codes);
    return hipGetLastError();
}

}  // namespace px
