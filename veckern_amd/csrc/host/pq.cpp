// Product quantizer training and coding on the host (reference interface: include/veckern/pq.hpp,
// src/cpu/pq.cpp). Training reproduces the reference's k-means exactly (pq.cpp:31-69), so the same (x, n, iters,
// seed) gives the reference's codebook byte for byte: one std::mt19937_64 seeded once and consumed in the
// reference's order (a std::shuffle of the point indices per sub-space, then one draw per empty cluster), float
// sums in point order, and the first minimum of l2sq as the assignment. The assignment step is pluggable
// (gpu::train passes the GPU kernel, which returns the same indices).
//
// Nearest-centroid search on the host keeps a transposed codebook [dsub][256] per sub-space so that the 256
// distances of one sub-vector are computed in a loop over centroids the compiler vectorises; each distance is
// still summed over j in order, the arithmetic of l2sq.
#include <algorithm>
#include <limits>
#include <numeric>
#include <random>
#include <vector>

#include "veckern/pq.hpp"

namespace veckern {
namespace {

void transpose_sub(const float* cent, std::size_t dsub, float* cent_t) {
    for (std::size_t c = 0; c < kSubCentroids; ++c)
        for (std::size_t j = 0; j < dsub; ++j) cent_t[j * kSubCentroids + c] = cent[c * dsub + j];
}

// cent_t: [dsub][256]. Returns the index of the nearest centroid to x: a running minimum from FLT_MAX with a
// strict <, so the first minimum wins (nearest_centroid, pq.cpp:11-22).
std::size_t nearest(const float* x, const float* cent_t, std::size_t dsub, float* dist) {
    for (std::size_t c = 0; c < kSubCentroids; ++c) dist[c] = 0.f;
    for (std::size_t j = 0; j < dsub; ++j) {
        const float xj = x[j];
        const float* row = cent_t + j * kSubCentroids;
        for (std::size_t c = 0; c < kSubCentroids; ++c) {
            const float diff = xj - row[c];
            dist[c] += diff * diff;
        }
    }
    std::size_t best = 0;
    float best_dist = std::numeric_limits<float>::max();
    for (std::size_t c = 0; c < kSubCentroids; ++c)
        if (dist[c] < best_dist) {
            best_dist = dist[c];
            best = c;
        }
    return best;
}

void assign_on_host(const float* sub, std::size_t n, const float* cent, std::size_t dsub, uint32_t* out, void*) {
    std::vector<float> cent_t(dsub * kSubCentroids);
    transpose_sub(cent, dsub, cent_t.data());
#pragma omp parallel
    {
        std::vector<float> dist(kSubCentroids);
#pragma omp for schedule(static)
        for (long long i = 0; i < static_cast<long long>(n); ++i)
            out[i] = static_cast<uint32_t>(nearest(sub + i * dsub, cent_t.data(), dsub, dist.data()));
    }
}


}  // namespace

ProductQuantizer::ProductQuantizer(std::size_t d, std::size_t m) : d_(d), m_(m), dsub_(m ? d / m : 0) {
    check(m > 0 && d > 0 && d % m == 0, "d must be a positive multiple of m");
    centroids_.assign(m_ * kSubCentroids * dsub_, 0.f);
}

void ProductQuantizer::set_centroids(const std::vector<float>& centroids) {
    check(centroids.size() == centroids_.size(), "codebook size does not match m * 256 * dsub");
    centroids_ = centroids;
}

void ProductQuantizer::train(const float* x, std::size_t n, std::size_t iters, uint64_t seed) {
    train(x, n, iters, seed, &assign_on_host, nullptr);
}

void ProductQuantizer::train(const float* x, std::size_t n, std::size_t iters, uint64_t seed, AssignFn assign_fn,
                             void* context) {
    check(n >= kSubCentroids, "PQ training needs at least 256 vectors");
    check(assign_fn != nullptr, "assignment function is null");
    std::mt19937_64 rng(seed);  // one stream for the whole codebook, sub-space after sub-space
    std::vector<float> sub(n * dsub_), sums(kSubCentroids * dsub_);
    std::vector<uint32_t> assign(n);
    std::vector<std::size_t> counts(kSubCentroids), order(n);

    for (std::size_t s = 0; s < m_; ++s) {
        for (std::size_t i = 0; i < n; ++i) std::copy_n(x + i * d_ + s * dsub_, dsub_, sub.data() + i * dsub_);
        float* cent = centroids_.data() + s * kSubCentroids * dsub_;

        // Initial centroids: the points at the first 256 positions of a shuffled index order (distinct points).
        std::iota(order.begin(), order.end(), std::size_t{0});
        std::shuffle(order.begin(), order.end(), rng);
        for (std::size_t c = 0; c < kSubCentroids; ++c)
            std::copy_n(sub.data() + order[c] * dsub_, dsub_, cent + c * dsub_);

        for (std::size_t it = 0; it < iters; ++it) {
            assign_fn(sub.data(), n, cent, dsub_, assign.data(), context);
            // Mean update: float sums accumulated in point order, then one division per coordinate.
            std::fill(sums.begin(), sums.end(), 0.f);
            std::fill(counts.begin(), counts.end(), std::size_t{0});
            for (std::size_t i = 0; i < n; ++i) {
                const std::size_t c = assign[i];
                ++counts[c];
                const float* p = sub.data() + i * dsub_;
                float* acc = sums.data() + c * dsub_;
                for (std::size_t j = 0; j < dsub_; ++j) acc[j] += p[j];
            }
            for (std::size_t c = 0; c < kSubCentroids; ++c) {
                float* dst = cent + c * dsub_;
                if (counts[c] == 0) {  // an empty cluster restarts at a random point (one draw, in cluster order)
                    std::copy_n(sub.data() + (rng() % n) * dsub_, dsub_, dst);
                    continue;
                }
                const float count = static_cast<float>(counts[c]);
                for (std::size_t j = 0; j < dsub_; ++j) dst[j] = sums[c * dsub_ + j] / count;
            }
        }
    }
}

void ProductQuantizer::encode(const float* x, std::size_t n, uint8_t* codes) const {
    std::vector<float> cent_t(m_ * dsub_ * kSubCentroids);
    for (std::size_t s = 0; s < m_; ++s)
        transpose_sub(centroids_.data() + s * kSubCentroids * dsub_, dsub_, cent_t.data() + s * dsub_ * kSubCentroids);
#pragma omp parallel
    {
        std::vector<float> dist(kSubCentroids);
#pragma omp for schedule(static)
        for (long long i = 0; i < static_cast<long long>(n); ++i)
            for (std::size_t s = 0; s < m_; ++s)
                codes[i * m_ + s] = static_cast<uint8_t>(nearest(x + i * d_ + s * dsub_,
                                                                 cent_t.data() + s * dsub_ * kSubCentroids, dsub_,
                                                                 dist.data()));
    }
}

void ProductQuantizer::decode(const uint8_t* codes, std::size_t n, float* x) const {
    for (std::size_t i = 0; i < n; ++i)
        for (std::size_t s = 0; s < m_; ++s) std::copy_n(centroid(s, codes[i * m_ + s]), dsub_, x + i * d_ + s * dsub_);
}

}  // namespace veckern
