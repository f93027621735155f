// Vector-file readers and seeded synthetic data (reference interface: include/veckern/io.hpp, src/cpu/io.cpp).
#include "veckern/io.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <stdexcept>

#include "philox.hpp"
#include "veckern/common.hpp"

namespace veckern {
namespace {

// The whole file as one read-only mapping (no stream state, no per-row reads); unmapped when it goes out of scope.
class FileView {
public:
    explicit FileView(const std::string& path) {
        const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
        if (fd < 0) throw std::runtime_error(path + ": " + std::strerror(errno));
        struct stat st {};
        const bool sized = ::fstat(fd, &st) == 0;
        size_ = sized ? static_cast<std::size_t>(st.st_size) : 0;
        if (sized && size_ > 0) {
            void* p = ::mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
            if (p != MAP_FAILED) base_ = static_cast<const unsigned char*>(p);
        }
        ::close(fd);
        if (!sized || (size_ > 0 && !base_)) throw std::runtime_error(path + ": the file cannot be mapped");
    }
    ~FileView() {
        if (base_) ::munmap(const_cast<unsigned char*>(base_), size_);
    }
    FileView(const FileView&) = delete;
    FileView& operator=(const FileView&) = delete;
    const unsigned char* data() const { return base_; }
    std::size_t size() const { return size_; }

private:
    const unsigned char* base_ = nullptr;
    std::size_t size_ = 0;
};

int32_t le_int32(const unsigned char* p) {  // the files are little-endian, like the host
    int32_t v;
    std::memcpy(&v, p, sizeof(v));
    return v;
}

// Rows of the *vecs formats: each row is an int32 count d followed by d values of type T, every row with the same
// d. The row count follows from the file size, which must be a whole number of rows; at most max_n rows (0: all)
// are returned, row-major, and each returned row's own count is checked against the first.
template <typename T>
std::vector<T> load_rows(const std::string& path, std::size_t& n, std::size_t& d, std::size_t max_n) {
    const FileView file(path);
    if (file.size() < sizeof(int32_t)) throw std::runtime_error(path + ": no row header (file too short)");
    const int32_t dim = le_int32(file.data());
    if (dim <= 0) throw std::runtime_error(path + ": row header gives dimension " + std::to_string(dim));
    const std::size_t stride = sizeof(int32_t) + sizeof(T) * static_cast<std::size_t>(dim);
    if (file.size() % stride != 0)
        throw std::runtime_error(path + ": " + std::to_string(file.size()) + " bytes are not whole rows of " +
                                 std::to_string(stride) + " bytes (dimension " + std::to_string(dim) + ")");
    const std::size_t rows = file.size() / stride;
    const std::size_t take = max_n > 0 ? std::min(rows, max_n) : rows;
    std::vector<T> out(take * static_cast<std::size_t>(dim));
    long long bad_row = -1;  // the first row whose count differs, if any
#pragma omp parallel for schedule(static) reduction(max : bad_row)
    for (long long r = 0; r < static_cast<long long>(take); ++r) {
        const unsigned char* row = file.data() + static_cast<std::size_t>(r) * stride;
        if (le_int32(row) != dim) {
            bad_row = std::max(bad_row, r);
            continue;
        }
        std::memcpy(out.data() + static_cast<std::size_t>(r) * dim, row + sizeof(int32_t), stride - sizeof(int32_t));
    }
    if (bad_row >= 0)
        throw std::runtime_error(path + ": row " + std::to_string(bad_row) + " does not have dimension " +
                                 std::to_string(dim));
    n = take;
    d = static_cast<std::size_t>(dim);
    return out;
}

}  // namespace

std::vector<float> read_fvecs(const std::string& path, std::size_t& n, std::size_t& d, std::size_t max_n) {
    return load_rows<float>(path, n, d, max_n);
}

std::vector<float> read_bvecs(const std::string& path, std::size_t& n, std::size_t& d, std::size_t max_n) {
    const std::vector<uint8_t> bytes = load_rows<uint8_t>(path, n, d, max_n);
    std::vector<float> out(bytes.size());
    std::transform(bytes.begin(), bytes.end(), out.begin(), [](uint8_t b) { return static_cast<float>(b); });
    return out;
}

std::vector<int32_t> read_ivecs(const std::string& path, std::size_t& n, std::size_t& d, std::size_t max_n) {
    return load_rows<int32_t>(path, n, d, max_n);
}

// One buffer per file: every row's header and values are laid out in memory, then written with a single call.
void write_fvecs(const std::string& path, const float* x, std::size_t n, std::size_t d) {
    const std::size_t stride = sizeof(int32_t) + sizeof(float) * d;
    std::vector<unsigned char> buf(n * stride);
    const int32_t dim = static_cast<int32_t>(d);
    for (std::size_t i = 0; i < n; ++i) {
        std::memcpy(buf.data() + i * stride, &dim, sizeof(dim));
        std::memcpy(buf.data() + i * stride + sizeof(dim), x + i * d, sizeof(float) * d);
    }
    std::FILE* f = std::fopen(path.c_str(), "wb");
    if (!f) throw std::runtime_error(path + ": " + std::strerror(errno));
    const bool ok = std::fwrite(buf.data(), 1, buf.size(), f) == buf.size();
    if (std::fclose(f) != 0 || !ok) throw std::runtime_error(path + ": write failed");
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
