#pragma once
// Vector-file readers and seeded synthetic data (reference: include/veckern/io.hpp).
//
// All generators are counter-based (Philox4x32-10): every value depends only on (seed, stream, index), so any
// row range can be produced on its own, in parallel, and identically on every machine.
#include <cstdint>
#include <string>
#include <vector>

namespace veckern {

// .fvecs: per row an int32 dimension followed by d float32 values.
std::vector<float> read_fvecs(const std::string& path, std::size_t& n, std::size_t& d, std::size_t max_n = 0);
// .bvecs: per row an int32 dimension followed by d uint8 values (converted to float).
std::vector<float> read_bvecs(const std::string& path, std::size_t& n, std::size_t& d, std::size_t max_n = 0);
// .ivecs: per row an int32 count followed by that many int32 ids (ground-truth files).
std::vector<int32_t> read_ivecs(const std::string& path, std::size_t& n, std::size_t& d, std::size_t max_n = 0);
// Writes row-major n x d floats as .fvecs.
void write_fvecs(const std::string& path, const float* x, std::size_t n, std::size_t d);

// Gaussian mixture: `components` centres drawn N(0, I), each row x = centre_c + sigma * N(0, I) with c uniform.
// Row i depends only on (seed, i). The benchmark's default data (1000 components, sigma 0.3).
class GaussianMixture {
public:
    GaussianMixture(std::size_t d, std::size_t components, float sigma, uint64_t seed);
    void fill(std::size_t first, std::size_t count, float* out) const;  // rows first .. first+count-1
    std::size_t d() const { return d_; }

private:
    std::size_t d_, components_;
    float sigma_;
    uint64_t seed_;
    std::vector<float> centres_;
};

// Structured data like the reference's benchmark source: x = centre_c + A z + noise, with centres uniform in
// [-1, 1], z ~ latent_scale * N(0, I_latent) and A a fixed random d x latent matrix with N(0, 1/latent) entries.
class SyntheticSource {
public:
    SyntheticSource(std::size_t d, std::size_t clusters, uint64_t seed, std::size_t latent_dim = 16,
                    float latent_scale = 0.5f, float noise = 0.05f);
    void fill(std::size_t first, std::size_t count, float* out) const;
    std::size_t d() const { return d_; }

private:
    std::size_t d_, clusters_, latent_;
    uint64_t seed_;
    float latent_scale_, noise_;
    std::vector<float> centres_, basis_;
};

// Gaussian blobs: centres uniform in [-1, 1], noise N(0, 0.15^2), cluster uniform per row.
std::vector<float> synthetic_clustered(std::size_t n, std::size_t d, std::size_t clusters, uint64_t seed);

// Row-major n x m uniform random bytes, row i depending only on (seed, i). PQ codes drawn directly.
void uniform_codes(std::size_t first, std::size_t n, std::size_t m, uint64_t seed, uint8_t* out);
// count values N(0, 1) from (seed, stream), starting at index first.
void normal_values(uint64_t seed, uint32_t stream, std::size_t first, std::size_t count, float* out);

}  // namespace veckern
