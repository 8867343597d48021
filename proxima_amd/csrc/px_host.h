// px_host.h -- host-only helpers of libproxima_px.so (no HIP types).
#pragma once

#include <stdint.h>

#include <vector>

namespace px {

float host_l2_sqr(const float* a, const float* b, int64_t n);

// Host-side decisions of PQ training (pq.rs:54-95, 139-148): the training sample, and per
// subspace the initial centroids' sample rows [m][ks] and the generator state after them.
struct PqTrainPlan {
    int64_t n = 0, ks = 0;
    std::vector<int64_t> sample;
    std::vector<int64_t> init_rows;
    std::vector<uint64_t> rng_after_init;
};
void pq_train_plan(int64_t n_all, int64_t m, int64_t nbits, int64_t train_sample, uint64_t seed,
                   PqTrainPlan* plan);
void pq_gather_sample(const float* training, int64_t dim, int64_t m, const PqTrainPlan& plan,
                      float* out);
// SplitMix64 below(n) (pq.rs:34-36) from *state, advancing it.
uint64_t splitmix_below(uint64_t* state, uint64_t n);
int host_threads();
void pq_train_host(const float* training, int64_t n_all, int64_t dim, int64_t m, int64_t nbits,
                   int64_t iters, int64_t train_sample, uint64_t seed, float* codebooks);
void pq_encode_host(const float* codebooks, int64_t dim, int64_t m, int64_t nbits,
                    const float* vectors, int64_t n, uint8_t* codes);

}  // namespace px
