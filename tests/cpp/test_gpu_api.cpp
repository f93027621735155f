// The reference's GPU test cases (tests/test_gpu.cpp:62-202) restated against this build's C++ API
// (veckern::gpu::PQSearcher over the C ABI), with the oracle (oracle/vk_oracle.h) as the expected answer and a
// bit-exact bar: identical ids and identical distance bits, where the reference allowed 1e-3 and 99% agreement.
#include <cmath>
#include <cstring>
#include <vector>

#include "check.hpp"
#include "slot_order.hpp"
#include "veckern/veckern.h"
#include "veckern/gpu.hpp"
#include "veckern/io.hpp"
#include "veckern/pq.hpp"
#include "vk_oracle.h"

using namespace veckern;
using gpu::ScanVariant;

namespace {

struct Fixture {
    // n is not a multiple of 64 or of any block size, so tails and padding are exercised; nq is prime.
    std::size_t n = 50'003, d = 64, m = 16, nq = 37;
    std::vector<float> base = synthetic_clustered(n, d, 50, 11);
    std::vector<float> queries = synthetic_clustered(nq, d, 50, 12);
    ProductQuantizer pq{d, m};
    std::vector<uint8_t> codes = std::vector<uint8_t>(n * m);
    Fixture() {
        pq.train(base.data(), 20'000, 8);
        pq.encode(base.data(), n, codes.data());
    }
};

Fixture& fixture() {
    static Fixture f;
    return f;
}

std::vector<vko_neighbor> oracle_search(const ProductQuantizer& pq, const std::vector<uint8_t>& codes, std::size_t n,
                                        const float* queries, std::size_t nq, std::size_t k) {
    std::vector<vko_neighbor> out(nq * k);
    if (vko_adc_search(pq.centroids().data(), pq.d(), pq.m(), codes.data(), n, queries, nq, k, out.data()) != 0)
        throw std::runtime_error("oracle rejected its input");
    return out;
}

void same(const std::vector<Neighbor>& got, const std::vector<vko_neighbor>& expected, const char* what) {
    EXPECT(got.size() == expected.size());
    for (std::size_t j = 0; j < got.size(); ++j) {
        uint32_t a, b;
        std::memcpy(&a, &got[j].dist, 4);
        std::memcpy(&b, &expected[j].dist, 4);
        if (got[j].id != expected[j].id || a != b)
            vktest::fail_at(__FILE__, __LINE__, std::string(what) + ": mismatch at " + std::to_string(j));
    }
}

void check_search(std::size_t k, ScanVariant v, const gpu::Tuning& tuning = {}) {
    auto& f = fixture();
    const auto expected = oracle_search(f.pq, f.codes, f.n, f.queries.data(), f.nq, k);
    gpu::PQSearcher searcher(f.pq, f.codes.data(), f.n);
    searcher.set_tuning(tuning);
    std::vector<Neighbor> got(f.nq * k);
    searcher.search(f.queries.data(), f.nq, k, v, got.data());
    same(got, expected, gpu::variant_name(v));
    for (std::size_t q = 0; q < f.nq; ++q)
        for (std::size_t j = 1; j < k; ++j) EXPECT(!(got[q * k + j] < got[q * k + j - 1]));
}

const ScanVariant kScans[] = {ScanVariant::GlobalLut, ScanVariant::SharedLut, ScanVariant::SharedLutVec,
                              ScanVariant::Interleaved};
// v4 is rejected before launch in this build (see the case "v4 is rejected").
const ScanVariant kFused[] = {ScanVariant::FusedReg, ScanVariant::FusedVec, ScanVariant::FusedVecMQ,
                              ScanVariant::FusedWarp};

}  // namespace

CASE("device info is sane") {
    const auto info = gpu::device_info();
    std::printf("      %s, %d CUs, %.0f GB/s peak, %zu B LDS/block\n", info.name.c_str(), info.sm_count,
                info.peak_bandwidth_gbs, info.max_smem_per_block);
    EXPECT(info.sm_count > 0 && info.peak_bandwidth_gbs > 0 && info.max_smem_per_block > 0);
}

CASE("every scan variant reproduces the CPU ADC distances bit for bit") {
    auto& f = fixture();
    std::vector<float> lut(f.nq * f.m * 256), expected(f.nq * f.n), got(f.nq * f.n);
    vko_compute_lut(f.pq.centroids().data(), f.d, f.m, f.queries.data(), f.nq, lut.data());
    vko_adc_scan(lut.data(), f.nq, f.codes.data(), f.n, f.m, expected.data());
    gpu::PQSearcher searcher(f.pq, f.codes.data(), f.n);
    for (auto v : kScans) {
        searcher.distances(f.queries.data(), f.nq, v, got.data());
        EXPECT(std::memcmp(got.data(), expected.data(), got.size() * sizeof(float)) == 0);
    }
}

CASE("search matches the CPU for every variant, k = 10") {
    for (auto v : kScans) check_search(10, v);
    for (auto v : kFused) check_search(10, v);
}

CASE("search covers every K template (k = 1, 16, 33, 100)") {
    for (std::size_t k : {1, 16, 33, 100}) {
        check_search(k, ScanVariant::SharedLut);
        for (auto v : kFused) check_search(k, v);
    }
}

CASE("v7 and v8 are exact for every queries-per-block, nq not divisible by Q") {
    for (int q : {1, 2, 4, 8}) {
        gpu::Tuning t;
        t.queries_per_block = q;
        for (std::size_t k : {1, 8, 10, 32}) check_search(k, ScanVariant::FusedVecMQ, t);
        for (std::size_t k : {1, 8, 10, 32, 64, 128}) check_search(k, ScanVariant::FusedWarp, t);
    }
}

CASE("tuning overrides keep results exact") {
    for (int threads : {64, 128, 512}) {
        gpu::Tuning t;
        t.scan_threads = threads;
        check_search(10, ScanVariant::SharedLutVec, t);
    }
    for (int bpq : {1, 3, 16}) {
        gpu::Tuning t;
        t.blocks_per_query = bpq;
        check_search(10, ScanVariant::FusedReg, t);
        check_search(10, ScanVariant::FusedVec, t);
        check_search(10, ScanVariant::FusedVecMQ, t);
        check_search(10, ScanVariant::FusedWarp, t);
    }
    for (int ilp : {2, 4})
        for (int bpq : {0, 7}) {
            gpu::Tuning t;
            t.vectors_per_step = ilp;
            t.blocks_per_query = bpq;
            for (std::size_t k : {1, 10, 33}) {
                check_search(k, ScanVariant::FusedVec, t);
                check_search(k, ScanVariant::FusedVecMQ, t);
                check_search(k, ScanVariant::FusedWarp, t);
            }
        }
}

CASE("launch shape is reported and a single query fills the device") {
    auto& f = fixture();
    gpu::PQSearcher searcher(f.pq, f.codes.data(), f.n);
    std::vector<Neighbor> out(f.nq * 10);
    searcher.search(f.queries.data(), f.nq, 10, ScanVariant::FusedVecMQ, out.data());
    const auto shape = searcher.last_launch();
    std::printf("      v7: T=%d blocks_x=%d grid_y=%d Q=%d blocks/CU=%d waves=%.2f\n", shape.threads, shape.blocks_x,
                shape.grid_y, shape.queries_per_block, shape.blocks_per_sm, shape.waves);
    EXPECT(shape.queries_per_block == 2 && shape.grid_y == 19);  // ceil(37 / 2)
    EXPECT(shape.blocks_per_sm > 0 && shape.waves > 0);

    std::vector<Neighbor> one(10);
    searcher.search(f.queries.data(), 1, 10, ScanVariant::FusedWarp, one.data());
    const auto single = searcher.last_launch();
    std::printf("      v8, 1 query: blocks=%d waves=%.2f\n", single.blocks_x, single.waves);
    // One query is spread over ceil(n / (16 vectors x 512 threads)) blocks (the reference's rule, test_gpu.cpp:139-145),
    // at most one per CU.
    const auto info = gpu::device_info();
    const std::size_t expected = std::min<std::size_t>(info.sm_count, (f.n + 8191) / 8192);
    EXPECT(single.blocks_x == static_cast<int>(expected) && single.blocks_x > 1);
}

CASE("word-interleaved variants reject m % 16 != 0; v5 accepts it") {
    auto& f = fixture();
    ProductQuantizer pq8(f.d, 8);
    pq8.train(f.base.data(), 5000, 4);
    std::vector<uint8_t> codes8(f.n * 8);
    pq8.encode(f.base.data(), f.n, codes8.data());
    gpu::PQSearcher searcher(pq8, codes8.data(), f.n);
    std::vector<Neighbor> got(f.nq * 10);
    for (auto v : {ScanVariant::SharedLutVec, ScanVariant::FusedVec, ScanVariant::FusedVecMQ, ScanVariant::FusedWarp})
        EXPECT_THROWS(searcher.search(f.queries.data(), f.nq, 10, v, got.data()));
    searcher.search(f.queries.data(), f.nq, 10, ScanVariant::FusedReg, got.data());
    same(got, oracle_search(pq8, codes8, f.n, f.queries.data(), f.nq, 10), "v5 m=8");
}

CASE("v4 is rejected before launch with std::logic_error") {
    auto& f = fixture();
    gpu::PQSearcher searcher(f.pq, f.codes.data(), f.n);
    std::vector<Neighbor> out(10);
    bool logic = false;
    try {
        searcher.search(f.queries.data(), 1, 10, ScanVariant::Fused, out.data());
    } catch (const std::logic_error&) {
        logic = true;
    }
    EXPECT(logic);
}

CASE("invalid tuning is rejected") {
    auto& f = fixture();
    gpu::PQSearcher searcher(f.pq, f.codes.data(), f.n);
    for (auto bad : {gpu::Tuning{100, 0, 2, 1}, gpu::Tuning{256, -1, 2, 1}, gpu::Tuning{256, 0, 3, 1},
                     gpu::Tuning{256, 0, 2, 3}})
        EXPECT_THROWS(searcher.set_tuning(bad));
}

CASE("invalid configurations are rejected") {
    auto& f = fixture();
    gpu::PQSearcher searcher(f.pq, f.codes.data(), f.n);
    std::vector<Neighbor> out(129);
    EXPECT_THROWS(searcher.search(f.queries.data(), 1, 129, ScanVariant::FusedReg, out.data()));
    EXPECT_THROWS(searcher.search(f.queries.data(), 1, 0, ScanVariant::FusedWarp, out.data()));
    EXPECT_THROWS(searcher.distances(f.queries.data(), 1, ScanVariant::FusedWarp, nullptr));
}

int main() { return vktest::run(); }

CASE("Reranker re-scores search candidates bit for bit like the CPU rerank_exact") {
    auto& f = fixture();
    const std::size_t r = 100, k = 10;
    gpu::PQSearcher searcher(f.pq, f.codes.data(), f.n);
    std::vector<Neighbor> cand(f.nq * r);
    searcher.search(f.queries.data(), f.nq, r, ScanVariant::FusedWarp, cand.data());
    cand[3].id = -1;  // padding is skipped
    std::vector<vko_neighbor> expected(f.nq * k);
    EXPECT(vko_rerank_exact(f.base.data(), f.d, f.queries.data(), f.nq,
                            reinterpret_cast<const vko_neighbor*>(cand.data()), r, k, expected.data()) == 0);
    gpu::Reranker reranker(f.base.data(), f.n, f.d);
    std::vector<Neighbor> got(f.nq * k);
    const gpu::Timings t = reranker.rerank(f.queries.data(), f.nq, cand.data(), r, k, got.data());
    same(got, expected, "rerank");
    EXPECT(t.scan_ms > 0);
    cand[5].id = static_cast<int32_t>(f.n);  // out of range
    EXPECT_THROWS(reranker.rerank(f.queries.data(), f.nq, cand.data(), r, k, got.data()));
}

CASE("gpu::encode and gpu::train give the CPU encoder's codes and the CPU trainer's codebook") {
    auto& f = fixture();
    std::vector<uint8_t> gpu_codes(f.n * f.m);
    gpu::encode(f.pq, f.base.data(), f.n, gpu_codes.data());
    EXPECT(gpu_codes == f.codes);
    ProductQuantizer cpu_pq(f.d, f.m), gpu_pq(f.d, f.m);
    cpu_pq.train(f.base.data(), 20'000, 6, 7);
    gpu::train(gpu_pq, f.base.data(), 20'000, 6, 7);
    EXPECT(cpu_pq.centroids() == gpu_pq.centroids());
}

CASE("IVFSearcher probing every list equals the exhaustive search; fewer lists match the oracle") {
    auto& f = fixture();
    const std::size_t nlist = 32, k = 10;
    std::vector<float> coarse(f.base.begin(), f.base.begin() + nlist * f.d);  // the first vectors as centroids
    std::vector<int32_t> lists(f.n);
    gpu::assign_lists(coarse.data(), nlist, f.d, f.base.data(), f.n, lists.data());
    gpu::IVFSearcher ivf(f.pq, coarse.data(), nlist, f.codes.data(), lists.data(), f.n);
    std::vector<Neighbor> got(f.nq * k);
    ivf.search(f.queries.data(), f.nq, nlist, k, got.data());
    same(got, oracle_search(f.pq, f.codes, f.n, f.queries.data(), f.nq, k), "ivf all lists");
    std::vector<vko_neighbor> expected(f.nq * k);
    EXPECT(vko_ivf_search(coarse.data(), nlist, f.pq.centroids().data(), f.d, f.m, f.codes.data(), lists.data(), f.n,
                          f.queries.data(), f.nq, 5, k, expected.data()) == 0);
    ivf.search(f.queries.data(), f.nq, 5, k, got.data());
    same(got, expected, "ivf nprobe 5");
    EXPECT_THROWS(ivf.search(f.queries.data(), f.nq, nlist + 1, k, got.data()));
}

CASE("the code layout built on the GPU equals the host's (sort, row fit, dealing, tile spread, interleave)") {
    struct Case {
        std::size_t n, m;
        bool uniform;  // uniform random codes (blocks dealt) or the fixture's clustered codes (m = 16)
        int q;         // queries per block of the search that builds the layout (0: none, built for 16 lanes)
    };
    const Case cases[] = {{50'003, 16, true, 0},  {50'003, 16, false, 0}, {20'000, 32, true, 0}, {9'999, 64, true, 0},
                          {100, 16, true, 0},     {768, 16, true, 0},     {70'000, 48, true, 0}, {50'003, 16, false, 2},
                          {20'000, 64, true, 2},  {30'000, 16, false, 1}, {12'345, 32, true, 1}};
    for (const Case& c : cases) {
        std::vector<uint8_t> codes(c.n * c.m);
        if (c.uniform) uniform_codes(0, c.n, c.m, 5 + c.m, codes.data());
        else codes.assign(fixture().codes.begin(), fixture().codes.begin() + c.n * c.m);
        const std::size_t d = c.m * 2, n_pad = (c.n + 255) / 256 * 256;
        const std::vector<float> centroids(c.m * 256 * 2, 0.5f);
        vk_searcher* s = nullptr;
        EXPECT(vk_searcher_create(centroids.data(), d, c.m, codes.data(), c.n, &s) == VK_OK);
        const int lanes_expected = c.q == 0 ? 16 : c.q == 2 ? 32 : 64;
        if (c.q) {
            vk_tuning t{};
            EXPECT(vk_searcher_get_tuning(s, &t) == VK_OK);
            t.queries_per_block = c.q;
            EXPECT(vk_searcher_set_tuning(s, &t) == VK_OK);
            const std::vector<float> q(static_cast<std::size_t>(c.q) * d, 0.25f);
            std::vector<vk_neighbor> out(static_cast<std::size_t>(c.q));
            EXPECT(vk_search(s, q.data(), c.q, 1, VK_V8_FUSED_WARP, out.data(), nullptr) == VK_OK);
        }
        std::vector<uint32_t> gpu_ids(n_pad, 0xdeadbeefu);
        std::vector<uint8_t> gpu_rows(c.m * 256, 0);
        int lanes = 0;
        EXPECT(vk_searcher_layout(s, gpu_ids.data(), n_pad, gpu_rows.data(), gpu_rows.size(), &lanes) == VK_OK);
        EXPECT(lanes == lanes_expected);
        EXPECT(vk_searcher_layout(s, gpu_ids.data(), n_pad + 1, nullptr, 0, nullptr) == VK_ERR_INVALID_ARGUMENT);
        EXPECT(vk_searcher_layout(s, gpu_ids.data(), n_pad, gpu_rows.data(), 5, nullptr) == VK_ERR_INVALID_ARGUMENT);
        vk_searcher_destroy(s);
        const vk::order::SlotOrder host = vk::order::slot_order(codes.data(), c.n, c.m, n_pad, lanes_expected, 4);
        EXPECT(gpu_rows == host.rows);
        EXPECT(gpu_ids == host.ids);
    }
}
