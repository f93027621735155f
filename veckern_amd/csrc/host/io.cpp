// Vector-file readers and seeded synthetic data (reference interface: include/veckern/io.hpp, src/cpu/io.cpp).
#include "veckern/io.hpp"

#include <cmath>
#include <fstream>

#include "philox.hpp"
#include "veckern/common.hpp"

namespace veckern {
namespace {

template <typename T>
std::vector<T> read_rows(const std::string& path, std::size_t& n, std::size_t& d, std::size_t max_n) {
    std::ifstream in(path, std::ios::binary);
    check(in.good(), "cannot open " + path);
    int32_t dim = 0;
    in.read(reinterpret_cast<char*>(&dim), sizeof(dim));
    check(in.good() && dim > 0, "bad header in " + path);
    in.seekg(0, std::ios::end);
    const auto bytes = static_cast<std::size_t>(in.tellg());
    const std::size_t row = sizeof(int32_t) + sizeof(T) * static_cast<std::size_t>(dim);
    check(bytes % row == 0, "file size is not a multiple of the row size: " + path);
    n = bytes / row;
    if (max_n > 0 && max_n < n) n = max_n;
    d = static_cast<std::size_t>(dim);
    std::vector<T> out(n * d);
    in.seekg(0);
    for (std::size_t i = 0; i < n; ++i) {
        int32_t row_dim = 0;
        in.read(reinterpret_cast<char*>(&row_dim), sizeof(row_dim));
        check(row_dim == dim, "inconsistent dimension in " + path);
        in.read(reinterpret_cast<char*>(out.data() + i * d), static_cast<std::streamsize>(sizeof(T) * d));
    }
    check(in.good(), "truncated file " + path);
    return out;
}

}  // namespace

std::vector<float> read_fvecs(const std::string& path, std::size_t& n, std::size_t& d, std::size_t max_n) {
    return read_rows<float>(path, n, d, max_n);
}

std::vector<float> read_bvecs(const std::string& path, std::size_t& n, std::size_t& d, std::size_t max_n) {
    const auto bytes = read_rows<uint8_t>(path, n, d, max_n);
    return std::vector<float>(bytes.begin(), bytes.end());
}

std::vector<int32_t> read_ivecs(const std::string& path, std::size_t& n, std::size_t& d, std::size_t max_n) {
    return read_rows<int32_t>(path, n, d, max_n);
}

void write_fvecs(const std::string& path, const float* x, std::size_t n, std::size_t d) {
    std::ofstream out(path, std::ios::binary);
    check(out.good(), "cannot create " + path);
    const int32_t dim = static_cast<int32_t>(d);
    for (std::size_t i = 0; i < n; ++i) {
        out.write(reinterpret_cast<const char*>(&dim), sizeof(dim));
        out.write(reinterpret_cast<const char*>(x + i * d), static_cast<std::streamsize>(sizeof(float) * d));
    }
    check(out.good(), "write failed: " + path);
}

// ---------------------------------------------------------------- Gaussian mixture

GaussianMixture::GaussianMixture(std::size_t d, std::size_t components, float sigma, uint64_t seed)
    : d_(d), components_(components), sigma_(sigma), seed_(seed), centres_(components * d) {
    check(d > 0 && components > 0, "d and components must be positive");
    rng::normals(seed_, rng::kMixtureCentres, 0, centres_.size(), centres_.data());
}

void GaussianMixture::fill(std::size_t first, std::size_t count, float* out) const {
#pragma omp parallel for schedule(static)
    for (long long r = 0; r < static_cast<long long>(count); ++r) {
        const uint64_t row = first + static_cast<uint64_t>(r);
        const std::size_t c = rng::bits64(seed_, rng::kMixtureComponent, row) % components_;
        float* x = out + static_cast<std::size_t>(r) * d_;
        rng::normals(seed_, rng::kMixtureNoise, row * d_, d_, x);
        const float* centre = centres_.data() + c * d_;
        for (std::size_t j = 0; j < d_; ++j) x[j] = centre[j] + sigma_ * x[j];
    }
}

// ---------------------------------------------------------------- latent-structure source

SyntheticSource::SyntheticSource(std::size_t d, std::size_t clusters, uint64_t seed, std::size_t latent_dim,
                                 float latent_scale, float noise)
    : d_(d), clusters_(clusters), latent_(latent_dim), seed_(seed), latent_scale_(latent_scale), noise_(noise),
      centres_(clusters * d), basis_(d * latent_dim) {
    check(d > 0 && clusters > 0 && latent_dim > 0, "d, clusters and latent_dim must be positive");
    for (std::size_t j = 0; j < centres_.size(); ++j)
        centres_[j] = static_cast<float>(2.0 * rng::unit(rng::philox(j, rng::kLatentCentres, seed_).v[0]) - 1.0);
    rng::normals(seed_, rng::kLatentBasis, 0, basis_.size(), basis_.data());
    const float norm = 1.0f / std::sqrt(static_cast<float>(latent_dim));
    for (auto& v : basis_) v *= norm;
}

void SyntheticSource::fill(std::size_t first, std::size_t count, float* out) const {
#pragma omp parallel for schedule(static)
    for (long long r = 0; r < static_cast<long long>(count); ++r) {
        const uint64_t row = first + static_cast<uint64_t>(r);
        const float* c = centres_.data() + (rng::bits64(seed_, rng::kLatentCluster, row) % clusters_) * d_;
        std::vector<float> z(latent_), e(d_);
        rng::normals(seed_, rng::kLatentZ, row * latent_, latent_, z.data());
        rng::normals(seed_, rng::kLatentNoise, row * d_, d_, e.data());
        float* x = out + static_cast<std::size_t>(r) * d_;
        for (std::size_t j = 0; j < d_; ++j) {
            float acc = c[j] + noise_ * e[j];
            for (std::size_t l = 0; l < latent_; ++l) acc += basis_[j * latent_ + l] * latent_scale_ * z[l];
            x[j] = acc;
        }
    }
}

// ---------------------------------------------------------------- Gaussian blobs

std::vector<float> synthetic_clustered(std::size_t n, std::size_t d, std::size_t clusters, uint64_t seed) {
    check(clusters > 0, "clusters must be positive");
    std::vector<float> centres(clusters * d);
    for (std::size_t j = 0; j < centres.size(); ++j)
        centres[j] = static_cast<float>(2.0 * rng::unit(rng::philox(j, rng::kBlobCentres, seed).v[0]) - 1.0);
    std::vector<float> out(n * d);
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < static_cast<long long>(n); ++i) {
        const float* c = centres.data() + (rng::bits64(seed, rng::kBlobCluster, i) % clusters) * d;
        float* x = out.data() + static_cast<std::size_t>(i) * d;
        rng::normals(seed, rng::kBlobNoise, static_cast<uint64_t>(i) * d, d, x);
        for (std::size_t j = 0; j < d; ++j) x[j] = c[j] + 0.15f * x[j];
    }
    return out;
}

// ---------------------------------------------------------------- direct codes and normal values

void uniform_codes(std::size_t first, std::size_t n, std::size_t m, uint64_t seed, uint8_t* out) {
#pragma omp parallel for schedule(static)
    for (long long r = 0; r < static_cast<long long>(n); ++r) {
        const uint64_t byte0 = (first + static_cast<uint64_t>(r)) * m;  // byte index in the code stream
        uint8_t* row = out + static_cast<std::size_t>(r) * m;
        std::size_t s = 0;
        while (s < m) {
            const uint64_t b = byte0 + s;
            const rng::Block blk = rng::philox(b / 16, rng::kCodes, seed);
            const uint8_t* bytes = reinterpret_cast<const uint8_t*>(blk.v);
            for (uint64_t t = b % 16; t < 16 && s < m; ++t, ++s) row[s] = bytes[t];
        }
    }
}

void normal_values(uint64_t seed, uint32_t stream, std::size_t first, std::size_t count, float* out) {
    constexpr std::size_t kChunk = 1 << 16;
    const long long chunks = static_cast<long long>((count + kChunk - 1) / kChunk);
#pragma omp parallel for schedule(static)
    for (long long c = 0; c < chunks; ++c) {
        const std::size_t a = static_cast<std::size_t>(c) * kChunk;
        const std::size_t len = std::min(kChunk, count - a);
        rng::normals(seed, stream, first + a, len, out + a);
    }
}

}  // namespace veckern
