// px_host.h -- host-only helpers of libproxima_px.so (no HIP types).
#pragma once

#include <stdint.h>

namespace px {

float host_l2_sqr(const float* a, const float* b, int64_t n);
int host_threads();
void pq_train_host(const float* training, int64_t n_all, int64_t dim, int64_t m, int64_t nbits,
                   int64_t iters, int64_t train_sample, uint64_t seed, float* codebooks);
void pq_encode_host(const float* codebooks, int64_t dim, int64_t m, int64_t nbits,
                    const float* vectors, int64_t n, uint8_t* codes);

}  // namespace px
