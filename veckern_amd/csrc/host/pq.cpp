// Product quantizer training and coding on the host (reference interface: include/veckern/pq.hpp,
// src/cpu/pq.cpp). Same algorithm family as the reference — per sub-space k-means from 256 distinct training
// points, empty clusters re-seeded from a random point, nearest centroid with the lowest index on ties — with
// this library's own seeded generator, so codebooks differ from the reference's for the same seed.
//
// Nearest-centroid search keeps a transposed codebook [dsub][256] per sub-space so that the 256 distances of
// one sub-vector are computed in a loop over centroids the compiler vectorises.
#include <algorithm>
#include <limits>
#include <numeric>
#include <vector>

#include "philox.hpp"
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
    std::vector<float> sub(n * dsub_);
    std::vector<uint32_t> assign(n);
    std::vector<std::size_t> counts(kSubCentroids), order(n);
    std::vector<double> sums(kSubCentroids * dsub_);
    uint64_t reseeds = 0;

    for (std::size_t s = 0; s < m_; ++s) {
        for (std::size_t i = 0; i < n; ++i) std::copy_n(x + i * d_ + s * dsub_, dsub_, sub.data() + i * dsub_);
        float* cent = centroids_.data() + s * kSubCentroids * dsub_;

        // 256 distinct training points: the first 256 positions of a seeded Fisher-Yates shuffle.
        std::iota(order.begin(), order.end(), 0);
        for (std::size_t c = 0; c < kSubCentroids; ++c) {
            const uint64_t r = rng::bits64(seed, rng::kTrainInit, s * kSubCentroids + c);
            std::swap(order[c], order[c + r % (n - c)]);
            std::copy_n(sub.data() + order[c] * dsub_, dsub_, cent + c * dsub_);
        }

        for (std::size_t it = 0; it < iters; ++it) {
            assign_fn(sub.data(), n, cent, dsub_, assign.data(), context);
            std::fill(sums.begin(), sums.end(), 0.0);
            std::fill(counts.begin(), counts.end(), 0);
            for (std::size_t i = 0; i < n; ++i) {
                ++counts[assign[i]];
                for (std::size_t j = 0; j < dsub_; ++j) sums[assign[i] * dsub_ + j] += sub[i * dsub_ + j];
            }
            for (std::size_t c = 0; c < kSubCentroids; ++c) {
                if (counts[c] == 0) {  // re-seed an empty cluster with a random training point
                    const uint64_t r = rng::bits64(seed, rng::kTrainReseed, reseeds++);
                    std::copy_n(sub.data() + (r % n) * dsub_, dsub_, cent + c * dsub_);
                    continue;
                }
                for (std::size_t j = 0; j < dsub_; ++j)
                    cent[c * dsub_ + j] = static_cast<float>(sums[c * dsub_ + j] / static_cast<double>(counts[c]));
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
