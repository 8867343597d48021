// px_pq_train.cpp -- product-quantizer training plan, and host training and encoding.
//
// The reference trains and encodes on the host (crates/core/src/pq.rs:54-193, 266-284).
// With a gfx950 device the library runs the Lloyd iterations and the encoding on the GPU
// (px_pq_kmeans.hip); without one, here. Both follow the same plan -- SplitMix64 sampling
// and initial-centroid picks, made here on the host -- and the same arithmetic: strict '<'
// argmin ties to the lower centroid, sequential sums in row order and a reciprocal
// multiply, built with -ffp-contract=off so a*b+c is never fused (Rust never fuses). The
// codebooks are therefore bit-identical to the reference's for the same inputs, on either
// side.
#include "px_host.h"

#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

namespace px {

// distance.rs:3-21
float host_l2_sqr(const float* a, const float* b, int64_t n) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const int64_t chunks = n / 8;
    for (int64_t c = 0; c < chunks; ++c) {
        for (int l = 0; l < 8; ++l) {
            const float d = a[c * 8 + l] - b[c * 8 + l];
            acc[l] = acc[l] + d * d;
        }
    }
    float sum = 0.f;
    for (int l = 0; l < 8; ++l) sum = sum + acc[l];
    for (int64_t i = chunks * 8; i < n; ++i) {
        const float d = a[i] - b[i];
        sum = sum + d * d;
    }
    return sum;
}

int host_threads() {
    const unsigned hc = std::thread::hardware_concurrency();
    return hc == 0 ? 1 : (int)std::min(hc, 64u);
}

template <class F>
static void parallel_for(int64_t n, F&& body) {
    const int nt = (int)std::min<int64_t>(host_threads(), std::max<int64_t>(n, 1));
    if (nt <= 1) {
        body(0, n);
        return;
    }
    std::vector<std::thread> th;
    th.reserve(nt);
    const int64_t per = (n + nt - 1) / nt;
    for (int t = 0; t < nt; ++t) {
        const int64_t lo = t * per, hi = std::min(n, lo + per);
        if (lo >= hi) break;
        th.emplace_back([&body, lo, hi] { body(lo, hi); });
    }
    for (auto& x : th) x.join();
}

namespace {
struct SplitMix {
    uint64_t s;
    uint64_t next() {  // pq.rs:27-33
        s += 0x9E3779B97F4A7C15ull;
        uint64_t z = s;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    uint64_t below(uint64_t n) { return next() % n; }  // pq.rs:34-36
};
}  // namespace

// pq.rs:54-95 and 139-148: the training sample, and per subspace the rows of the initial
// centroids (a partial Fisher-Yates shuffle) and the generator state after them.
void pq_train_plan(int64_t n_all, int64_t m, int64_t nbits, int64_t train_sample, uint64_t seed,
                   PqTrainPlan* plan) {
    const int64_t ks = (int64_t)1 << nbits;
    SplitMix rng{seed};
    int64_t n = n_all;
    if (train_sample > 0) n = std::clamp<int64_t>(train_sample, ks, n_all);
    plan->n = n;
    plan->ks = ks;
    plan->sample.resize(n);
    if (n == n_all) {
        for (int64_t i = 0; i < n; ++i) plan->sample[i] = i;
    } else {
        for (int64_t i = 0; i < n; ++i) plan->sample[i] = (int64_t)rng.below((uint64_t)n_all);
    }
    plan->init_rows.resize(m * ks);
    plan->rng_after_init.resize(m);
    std::vector<int64_t> order(n);
    for (int64_t sub = 0; sub < m; ++sub) {
        SplitMix r{seed ^ ((uint64_t)sub * 0x9E3779B97F4A7C15ull)};  // pq.rs:95
        for (int64_t i = 0; i < n; ++i) order[i] = i;
        for (int64_t c = 0; c < ks; ++c) {
            const int64_t j = c + (int64_t)r.below((uint64_t)(n - c));
            std::swap(order[c], order[j]);
            plan->init_rows[sub * ks + c] = order[c];
        }
        plan->rng_after_init[sub] = r.s;
    }
}

uint64_t splitmix_below(uint64_t* state, uint64_t n) {
    SplitMix r{*state};
    const uint64_t v = r.below(n);
    *state = r.s;
    return v;
}

namespace {

// argmin over ks centroids of dimension d with strict '<' from FLT_MAX (pq.rs:157-165)
inline uint32_t nearest(const float* v, const float* cents, int64_t ks, int64_t d) {
    uint32_t best = 0;
    float best_d = FLT_MAX;
    for (int64_t c = 0; c < ks; ++c) {
        const float dist = host_l2_sqr(v, cents + c * d, d);
        if (dist < best_d) {
            best_d = dist;
            best = (uint32_t)c;
        }
    }
    return best;
}

// pq.rs:149-193, from the plan's initial centroids and generator state
void kmeans(const float* data, int64_t n, int64_t d, int64_t ks, int64_t iters,
            const int64_t* init_rows, uint64_t rng_state, float* cents) {
    SplitMix rng{rng_state};
    for (int64_t c = 0; c < ks; ++c)
        std::memcpy(cents + c * d, data + init_rows[c] * d, sizeof(float) * d);
    std::vector<uint32_t> assign(n);
    std::vector<float> sums(ks * d);
    std::vector<uint32_t> counts(ks);
    for (int64_t it = 0; it < iters; ++it) {
        parallel_for(n, [&](int64_t lo, int64_t hi) {
            for (int64_t i = lo; i < hi; ++i) assign[i] = nearest(data + i * d, cents, ks, d);
        });
        std::fill(sums.begin(), sums.end(), 0.f);
        std::fill(counts.begin(), counts.end(), 0u);
        for (int64_t i = 0; i < n; ++i) {
            const int64_t c = assign[i];
            counts[c] += 1;
            const float* v = data + i * d;
            float* s = sums.data() + c * d;
            for (int64_t x = 0; x < d; ++x) s[x] = s[x] + v[x];
        }
        for (int64_t c = 0; c < ks; ++c) {
            if (counts[c] == 0) {
                const int64_t idx = (int64_t)rng.below((uint64_t)n);
                std::memcpy(cents + c * d, data + idx * d, sizeof(float) * d);
            } else {
                const float inv = 1.0f / (float)counts[c];
                for (int64_t x = 0; x < d; ++x) cents[c * d + x] = sums[c * d + x] * inv;
            }
        }
    }
}
}  // namespace

// Sub-major copy of the training sample: out[sub][i][x] = training[sample[i]][sub*dsub + x].
void pq_gather_sample(const float* training, int64_t dim, int64_t m, const PqTrainPlan& plan,
                      float* out) {
    const int64_t dsub = dim / m;
    for (int64_t sub = 0; sub < m; ++sub)
        for (int64_t i = 0; i < plan.n; ++i)
            std::memcpy(out + (sub * plan.n + i) * dsub, training + plan.sample[i] * dim + sub * dsub,
                        sizeof(float) * dsub);
}

// pq.rs:54-105; arguments validated by the caller
void pq_train_host(const float* training, int64_t n_all, int64_t dim, int64_t m, int64_t nbits,
                   int64_t iters, int64_t train_sample, uint64_t seed, float* codebooks) {
    const int64_t dsub = dim / m;
    PqTrainPlan plan;
    pq_train_plan(n_all, m, nbits, train_sample, seed, &plan);
    const int64_t n = plan.n, ks = plan.ks;
    std::vector<float> sub_data(m * n * dsub);
    pq_gather_sample(training, dim, m, plan, sub_data.data());
    for (int64_t sub = 0; sub < m; ++sub)
        kmeans(sub_data.data() + sub * n * dsub, n, dsub, ks, iters, plan.init_rows.data() + sub * ks,
               plan.rng_after_init[sub], codebooks + sub * ks * dsub);
}

// pq.rs:107-121 per row, rows in parallel (pq.rs:275-281)
void pq_encode_host(const float* codebooks, int64_t dim, int64_t m, int64_t nbits,
                    const float* vectors, int64_t n, uint8_t* codes) {
    const int64_t dsub = dim / m;
    const int64_t ks = (int64_t)1 << nbits;
    parallel_for(n, [&](int64_t lo, int64_t hi) {
        for (int64_t i = lo; i < hi; ++i)
            for (int64_t sub = 0; sub < m; ++sub)
                codes[i * m + sub] = (uint8_t)nearest(vectors + i * dim + sub * dsub,
                                                      codebooks + sub * ks * dsub, ks, dsub);
    });
}

}  // namespace px
