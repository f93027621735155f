// Philox4x32-10 counter-based generator (Salmon, Moraes, Dror and Shaw, "Parallel random numbers: as easy as
// 1, 2, 3", SC 2011), and the value streams the synthetic data is built from. A value depends only on
// (seed, stream, index), so rows can be generated in any order and in parallel.
#pragma once

#include <cmath>
#include <cstddef>
#include <cstdint>

namespace veckern::rng {

struct Block {
    uint32_t v[4];
};

// The raw 10-round bijection on a 128-bit counter under a 64-bit key.
inline Block philox_raw(const uint32_t ctr[4], const uint32_t key[2]) {
    constexpr uint32_t kMul0 = 0xD2511F53u, kMul1 = 0xCD9E8D57u;  // round multipliers
    constexpr uint32_t kWeyl0 = 0x9E3779B9u, kWeyl1 = 0xBB67AE85u;  // key schedule increments
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int r = 0; r < 10; ++r) {
        const uint64_t p0 = static_cast<uint64_t>(kMul0) * c0, p1 = static_cast<uint64_t>(kMul1) * c2;
        const uint32_t hi0 = static_cast<uint32_t>(p0 >> 32), lo0 = static_cast<uint32_t>(p0);
        const uint32_t hi1 = static_cast<uint32_t>(p1 >> 32), lo1 = static_cast<uint32_t>(p1);
        c0 = hi1 ^ c1 ^ k0;
        c1 = lo1;
        c2 = hi0 ^ c3 ^ k1;
        c3 = lo0;
        k0 += kWeyl0;
        k1 += kWeyl1;
    }
    return Block{{c0, c1, c2, c3}};
}

// Counter = (index, stream), key = seed.
inline Block philox(uint64_t counter, uint32_t stream, uint64_t seed) {
    const uint32_t ctr[4] = {static_cast<uint32_t>(counter), static_cast<uint32_t>(counter >> 32), stream, 0u};
    const uint32_t key[2] = {static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32)};
    return philox_raw(ctr, key);
}

// Uniform in (0, 1) from 32 random bits.
inline double unit(uint32_t x) { return (static_cast<double>(x) + 0.5) * (1.0 / 4294967296.0); }

// Two N(0, 1) values from two uniforms (Box-Muller).
inline void box_muller(uint32_t a, uint32_t b, double* z0, double* z1) {
    const double r = std::sqrt(-2.0 * std::log(unit(a)));
    const double t = 6.283185307179586476925286766559 * unit(b);
    *z0 = r * std::cos(t);
    *z1 = r * std::sin(t);
}

// Value `index` of the N(0, 1) stream (seed, stream); one Philox block yields four values.
inline float normal(uint64_t seed, uint32_t stream, uint64_t index) {
    const Block b = philox(index / 4, stream, seed);
    double z[4];
    box_muller(b.v[0], b.v[1], &z[0], &z[1]);
    box_muller(b.v[2], b.v[3], &z[2], &z[3]);
    return static_cast<float>(z[index % 4]);
}

// Fills out[0..count) with values first .. first+count-1 of the N(0, 1) stream, one block per four values.
inline void normals(uint64_t seed, uint32_t stream, uint64_t first, std::size_t count, float* out) {
    std::size_t j = 0;
    while (j < count) {
        const uint64_t idx = first + j;
        const Block b = philox(idx / 4, stream, seed);
        double z[4];
        box_muller(b.v[0], b.v[1], &z[0], &z[1]);
        box_muller(b.v[2], b.v[3], &z[2], &z[3]);
        for (uint64_t t = idx % 4; t < 4 && j < count; ++t, ++j) out[j] = static_cast<float>(z[t]);
    }
}

// 64 random bits for (seed, stream, index).
inline uint64_t bits64(uint64_t seed, uint32_t stream, uint64_t index) {
    const Block b = philox(index, stream, seed);
    return (static_cast<uint64_t>(b.v[0]) << 32) | b.v[1];
}

// Stream numbers, one per kind of value, so that no two generators share random numbers.
enum Stream : uint32_t {
    kMixtureCentres = 1,
    kMixtureComponent = 2,
    kMixtureNoise = 3,
    kCodes = 4,
    kLatentCentres = 5,
    kLatentBasis = 6,
    kLatentCluster = 7,
    kLatentZ = 8,
    kLatentNoise = 9,
    kBlobCentres = 10,
    kBlobCluster = 11,
    kBlobNoise = 12,
};

}  // namespace veckern::rng
