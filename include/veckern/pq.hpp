#pragma once
// Product quantizer: d dimensions split into m sub-spaces of 256 centroids each, one byte per sub-code
// (reference: include/veckern/pq.hpp). Training and encoding run on the host; they produce the inputs of the
// GPU search path (centroid layout [m][256][dsub], row-major n x m codes).
#include <cstdint>
#include <vector>

#include "veckern/common.hpp"

namespace veckern {

// Nearest-centroid assignment of one sub-space, the inner step of train(): out[i] = index of the centroid of
// `cent` (256 x dsub) nearest to sub-vector i of `sub` (n x dsub). gpu::train passes the GPU kernel; every
// implementation must return the first minimum of l2sq (nearest_centroid's rule) so that training is identical.
using AssignFn = void (*)(const float* sub, std::size_t n, const float* cent, std::size_t dsub, uint32_t* out,
                          void* context);

class ProductQuantizer {
public:
    // Throws std::runtime_error unless d is a positive multiple of m.
    ProductQuantizer(std::size_t d, std::size_t m);

    // Independent k-means per sub-space on the first n rows of x (row-major n x d), the reference's algorithm and
    // random stream (pq.cpp:31-69): initial centroids are 256 distinct points picked by a std::shuffle driven by
    // std::mt19937_64(seed), then `iters` rounds of nearest-centroid assignment and float mean update; an empty
    // cluster restarts at a random point. The same arguments give the reference's codebook bit for bit.
    void train(const float* x, std::size_t n, std::size_t iters = 20, uint64_t seed = 1);
    // The same training with the assignment step delegated (the update, initialisation and re-seeding stay here).
    void train(const float* x, std::size_t n, std::size_t iters, uint64_t seed, AssignFn assign, void* context);
    // codes: row-major n x m bytes, the nearest centroid of each sub-vector (lowest index on ties).
    void encode(const float* x, std::size_t n, uint8_t* codes) const;
    void decode(const uint8_t* codes, std::size_t n, float* x) const;

    const float* centroid(std::size_t sub, std::size_t c) const {
        return centroids_.data() + (sub * kSubCentroids + c) * dsub_;
    }
    // Layout: [m][256][dsub] floats, the layout the GPU LUT build reads.
    const std::vector<float>& centroids() const { return centroids_; }
    // Replaces the codebook (same layout); throws if the size does not match.
    void set_centroids(const std::vector<float>& centroids);

    std::size_t d() const { return d_; }
    std::size_t m() const { return m_; }
    std::size_t dsub() const { return dsub_; }

private:
    std::size_t d_, m_, dsub_;
    std::vector<float> centroids_;
};

}  // namespace veckern
