// Host C++ tools on the CPU: vector files, generators, the PQ codec and the evaluation helpers (reference
// cases: tests/test_cpu.cpp:48-56, 69-82, 96-144).
#include <cmath>
#include <cstdio>
#include <fstream>
#include <vector>

#include "check.hpp"
#include "veckern/eval.hpp"
#include "veckern/io.hpp"
#include "veckern/pq.hpp"

using namespace veckern;

CASE("PQ rejects d not divisible by m") { EXPECT_THROWS(ProductQuantizer(30, 8)); }

CASE("PQ training needs 256 vectors and a codebook of the right size") {
    ProductQuantizer pq(16, 4);
    std::vector<float> x(100 * 16, 0.f);
    EXPECT_THROWS(pq.train(x.data(), 100, 2));
    EXPECT_THROWS(pq.set_centroids(std::vector<float>(10)));
}

CASE("PQ reconstruction error is far below the data spread") {
    const std::size_t n = 4000, d = 32, m = 8;
    const auto base = synthetic_clustered(n, d, 20, 7);
    ProductQuantizer pq(d, m);
    pq.train(base.data(), n, 10);
    std::vector<uint8_t> codes(n * m);
    pq.encode(base.data(), n, codes.data());
    std::vector<float> decoded(n * d), mean(d, 0.f);
    pq.decode(codes.data(), n, decoded.data());
    for (std::size_t i = 0; i < n; ++i)
        for (std::size_t j = 0; j < d; ++j) mean[j] += base[i * d + j] / n;
    double err = 0, spread = 0;
    for (std::size_t i = 0; i < n; ++i) {
        err += l2sq(base.data() + i * d, decoded.data() + i * d, d);
        spread += l2sq(base.data() + i * d, mean.data(), d);
    }
    EXPECT(err < 0.2 * spread);
}

CASE("PQ encode picks the nearest centroid and training is deterministic") {
    const std::size_t n = 3000, d = 16, m = 4;
    GaussianMixture src(d, 30, 0.3f, 5);
    std::vector<float> x(n * d);
    src.fill(0, n, x.data());
    ProductQuantizer a(d, m), b(d, m);
    a.train(x.data(), n, 6, 3);
    b.train(x.data(), n, 6, 3);
    EXPECT(a.centroids() == b.centroids());
    std::vector<uint8_t> codes(n * m);
    a.encode(x.data(), n, codes.data());
    for (std::size_t i = 0; i < n; i += 37)
        for (std::size_t s = 0; s < m; ++s) {
            const float chosen = l2sq(x.data() + i * d + s * a.dsub(), a.centroid(s, codes[i * m + s]), a.dsub());
            for (std::size_t c = 0; c < 256; ++c)
                EXPECT(chosen <= l2sq(x.data() + i * d + s * a.dsub(), a.centroid(s, c), a.dsub()) * (1 + 1e-6f) + 1e-12f);
        }
}

CASE("generator rows depend only on (seed, row)") {
    GaussianMixture mix(16, 10, 0.3f, 3);
    SyntheticSource lat(16, 10, 3);
    for (int which = 0; which < 2; ++which) {
        std::vector<float> all(100 * 16), tail(50 * 16);
        if (which == 0) {
            mix.fill(0, 100, all.data());
            mix.fill(50, 50, tail.data());
        } else {
            lat.fill(0, 100, all.data());
            lat.fill(50, 50, tail.data());
        }
        for (std::size_t j = 0; j < tail.size(); ++j) EXPECT(all[50 * 16 + j] == tail[j]);
        EXPECT(all[0] != all[16]);
    }
    std::vector<uint8_t> codes(100 * 16), part(40 * 16);
    uniform_codes(0, 100, 16, 9, codes.data());
    uniform_codes(60, 40, 16, 9, part.data());
    for (std::size_t j = 0; j < part.size(); ++j) EXPECT(codes[60 * 16 + j] == part[j]);
}

CASE("fvecs round trip") {
    const std::string path = "veckern_host_test.fvecs";
    std::vector<float> rows(3 * 4);
    for (int r = 0; r < 3; ++r)
        for (int j = 0; j < 4; ++j) rows[r * 4 + j] = r * 10.f + j;
    write_fvecs(path, rows.data(), 3, 4);
    std::size_t n = 0, d = 0;
    const auto data = read_fvecs(path, n, d, 2);
    std::remove(path.c_str());
    EXPECT(n == 2 && d == 4);
    EXPECT(data[4] == 10.f && data[7] == 13.f);
}

CASE("ivecs and bvecs readers") {
    const std::string ipath = "veckern_host_test.ivecs", bpath = "veckern_host_test.bvecs";
    {
        std::ofstream out(ipath, std::ios::binary);
        for (int32_t r = 0; r < 2; ++r) {
            const int32_t dim = 3;
            out.write(reinterpret_cast<const char*>(&dim), 4);
            for (int32_t j = 0; j < 3; ++j) {
                const int32_t v = 100 * r + j;
                out.write(reinterpret_cast<const char*>(&v), 4);
            }
        }
        std::ofstream bout(bpath, std::ios::binary);
        const int32_t dim = 2;
        const uint8_t vals[2] = {7, 250};
        bout.write(reinterpret_cast<const char*>(&dim), 4);
        bout.write(reinterpret_cast<const char*>(vals), 2);
    }
    std::size_t n = 0, d = 0;
    const auto ids = read_ivecs(ipath, n, d);
    EXPECT(n == 2 && d == 3 && ids[4] == 101);
    const auto bytes = read_bvecs(bpath, n, d);
    EXPECT(n == 1 && d == 2 && bytes[0] == 7.f && bytes[1] == 250.f);
    std::remove(ipath.c_str());
    std::remove(bpath.c_str());
    EXPECT_THROWS(read_fvecs("does_not_exist.fvecs", n, d));
}

CASE("malformed vector files are rejected") {
    const std::string path = "veckern_host_bad.fvecs";
    auto write_words = [&](const std::vector<int32_t>& words, std::size_t extra_bytes) {
        std::ofstream out(path, std::ios::binary);
        out.write(reinterpret_cast<const char*>(words.data()), static_cast<std::streamsize>(4 * words.size()));
        for (std::size_t i = 0; i < extra_bytes; ++i) out.put('\0');
    };
    std::size_t n = 0, d = 0;
    write_words({}, 0);  // empty: no header
    EXPECT_THROWS(read_fvecs(path, n, d));
    write_words({0}, 0);  // dimension 0
    EXPECT_THROWS(read_fvecs(path, n, d));
    write_words({2, 0, 0, 2, 0, 0}, 2);  // two rows of d=2 and a truncated third
    EXPECT_THROWS(read_fvecs(path, n, d));
    write_words({2, 0, 0, 1, 0, 0}, 0);  // the second row claims d=1 though the size fits two rows of d=2
    EXPECT_THROWS(read_fvecs(path, n, d));
    const auto first = read_fvecs(path, n, d, 1);  // the first row alone is well formed
    EXPECT(n == 1 && d == 2 && first.size() == 2);
    std::remove(path.c_str());
}

CASE("exact search finds itself; the selector pads and orders by (dist, id)") {
    const std::size_t n = 4000, d = 32, k = 10;
    const auto base = synthetic_clustered(n, d, 20, 7);
    std::vector<Neighbor> self(5 * k);
    exact_knn(base.data(), n, base.data(), 5, d, k, self.data());
    for (std::size_t q = 0; q < 5; ++q) EXPECT(self[q * k].id == static_cast<int32_t>(q));
    TopK top(3);
    const float values[] = {5, 1, 4, 1, 3};
    for (int i = 0; i < 5; ++i) top.push(values[i], i);
    Neighbor out[3];
    top.write(out);
    EXPECT(out[0].id == 1 && out[1].id == 3 && out[2].id == 4);
    TopK small(4);
    small.push(2.f, 9);
    Neighbor padded[4];
    small.write(padded);
    EXPECT(padded[0].id == 9 && padded[1].id == -1 && std::isinf(padded[3].dist));
}

CASE("recall_at_k counts found ids present among the first k true ids") {
    Neighbor found[4] = {{0, 1}, {0, 2}, {0, 3}, {0, 4}};
    const int32_t truth[4] = {4, 3, 2, 99};
    EXPECT(recall_at_k(found, 4, truth, 4, 1, 4) == 0.75);
    EXPECT(recall_at_k(found, 4, truth, 4, 1, 1) == 0.0);
    EXPECT_THROWS(recall_at_k(found, 4, truth, 4, 1, 5));
}

int main() { return vktest::run(); }
