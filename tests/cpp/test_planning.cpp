// Host-side launch planning (veckern_amd/csrc/planning.hpp), on the CPU: list-length dispatch, Q capping, the
// balanced work partition of the wave-list scan, and the blocks_x models of the grid kernels; and the slot order of
// the fused scans' code layout (veckern_amd/csrc/slot_order.hpp). The blocks_x model
// is checked against launch shapes the reference recorded on an A100 (108 SMs, 4 resident blocks per SM).
#include <algorithm>
#include <climits>
#include <cstdint>
#include <cstdio>
#include <random>
#include <utility>
#include <vector>

#include "check.hpp"
#include "planning.hpp"
#include "slot_order.hpp"

using namespace vk::plan;

CASE("dispatched_k picks the smallest of 8, 16, 32, 64, 128 that holds k") {
    EXPECT(dispatched_k(1) == 8 && dispatched_k(8) == 8 && dispatched_k(9) == 16 && dispatched_k(10) == 16);
    EXPECT(dispatched_k(33) == 64 && dispatched_k(64) == 64 && dispatched_k(100) == 128 && dispatched_k(128) == 128);
    EXPECT(dispatched_k(129) == 0);
}

CASE("effective_q halves Q until the tables fit and, for per-thread lists, Q*K <= 64") {
    const std::size_t lds = 160 * 1024;
    EXPECT(effective_q(4, 16, lds, false, 16) == 4);
    EXPECT(effective_q(8, 16, lds, false, 16) == 8);   // 128 KB
    EXPECT(effective_q(8, 32, lds, false, 16) == 4);   // 256 KB -> 128 KB
    EXPECT(effective_q(4, 64, lds, false, 128) == 2);  // 256 KB -> 128 KB
    EXPECT(effective_q(8, 16, lds, true, 16) == 4);    // Q*K = 128 -> 64
    EXPECT(effective_q(2, 16, lds, true, 128) == 1);
    EXPECT(effective_q(8, 160, lds, false, 8) == 1);
}

CASE("cap_q_by_batch keeps no more query slots than the batch needs") {
    EXPECT(cap_q_by_batch(4, 1) == 1);
    EXPECT(cap_q_by_batch(4, 2) == 2);
    EXPECT(cap_q_by_batch(4, 3) == 4);
    EXPECT(cap_q_by_batch(8, 5) == 8);
    EXPECT(cap_q_by_batch(8, 4) == 4);
    EXPECT(cap_q_by_batch(4, 1000) == 4);
    EXPECT(cap_q_by_batch(1, 1) == 1);
}

CASE("blocks_x_waves reproduces the reference's recorded launch shapes") {
    const int64_t wave = 4 * 108;  // A100: 4 resident blocks per SM x 108 SMs
    // tests/test_gpu.cpp fixture, v7 Q=2 T=128: run_all.log:28 "blocks_x=22 grid_y=19 ... waves=0.97"
    WaveChoice c = blocks_x_waves(50'003, 19, 128, wave, 0);
    EXPECT(c.blocks_x == 22);
    EXPECT(c.waves > 0.96 && c.waves < 0.98);
    // 1M headline, v8 Q=2 T=256: results/final/scaling.csv:11 "blocks_x 6, grid_y 500"
    c = blocks_x_waves(1'000'000, 500, 256, wave, 0);
    EXPECT(c.blocks_x == 6);
    // 10M, one query, v8 T=256: results/final/latency.csv:17 "bx=430"
    c = blocks_x_waves(10'000'000, 1, 256, wave, 0);
    EXPECT(c.blocks_x == 430);
    // an explicit blocks_per_query wins
    c = blocks_x_waves(1'000'000, 500, 256, wave, 7);
    EXPECT(c.blocks_x == 7);
}

CASE("blocks_x_fill: ~8 blocks per CU over the grid, >= 16 vectors per thread, override wins") {
    EXPECT(blocks_x_fill(50'003, 37, 256, 256, 0) == 13);      // by work: ceil(50003 / 4096)
    EXPECT(blocks_x_fill(10'000'000, 1000, 256, 256, 0) == 3);  // to fill: ceil(2048 / 1000)
    EXPECT(blocks_x_fill(10, 1, 256, 256, 0) == 1);
    EXPECT(blocks_x_fill(10'000'000, 1000, 256, 256, 5) == 5);
}

CASE("bulk admission is chosen while a block scans few vectors of a slab") {
    // 100k vectors, nq=100, Q=4: 13 blocks per slab, ~7.7k vectors each
    EXPECT(bulk_scan(balanced_partition(100'000, 100, 4, 4, 512, 0, 256), 4));
    // 10M vectors, nq=8, Q=4: 2 slabs of 256 blocks, ~39k vectors each
    EXPECT(bulk_scan(balanced_partition(10'000'000, 8, 4, 4, 512, 0, 256), 4));
    // the 1M headline (2 blocks per slab, 500k vectors each) and 10M at nq=1000 (5M each): one by one
    EXPECT(!bulk_scan(balanced_partition(1'000'000, 1000, 4, 4, 512, 0, 256), 4));
    EXPECT(!bulk_scan(balanced_partition(10'000'000, 1000, 4, 4, 512, 0, 256), 4));
    // the limit: a block's run of one slab, in vectors, against kBulkScanVectors
    for (int64_t per_block : {int64_t{1000}, int64_t{1023}, int64_t{1024}, int64_t{1025}, int64_t{4096}}) {
        const int64_t n = per_block * 256 * 4;  // 4 blocks per slab at ilp 1, granules of 64 vectors
        const Partition p = balanced_partition(n, 8, 4, 1, 8, 4, 0);
        EXPECT(p.grid == 8);
        EXPECT(bulk_scan(p, 1) == (per_block * 256 < kBulkScanVectors));
    }
    EXPECT(!bulk_scan(Partition{}, 4));
}

CASE("balanced_partition covers every item exactly once and bounds the slots per slab") {
    // one slab on 256 CUs with two resident blocks each: one block per CU, not two
    EXPECT(balanced_partition(10'000'000, 1, 1, 4, 512, 0, 256).grid == 256);
    EXPECT(balanced_partition(10'000'000, 2, 1, 4, 512, 0, 256).grid == 512);
    EXPECT(balanced_partition(10'000'000, 1, 1, 4, 512, 0).grid == 512);
    // slabs no more than the slots: floor(slots / slabs) whole blocks per slab (1M x nq=1000 at Q = 4: 2 each)
    const Partition b = balanced_partition(1'000'000, 1000, 4, 4, 512, 0, 256);
    EXPECT(b.grid == 500 && b.max_slots == 2);
    EXPECT(balanced_partition(1'000'000, 1000, 4, 4, 256, 0, 256).grid == 250);  // one block per slab
    EXPECT(balanced_partition(1'000'000, 1000, 2, 4, 256, 0, 256).grid == 256);  // 500 slabs > 256 slots
    // small slabs: at most ceil(n / kMinBlockVectors) blocks each (100k vectors: 13 blocks of ~7.7k vectors)
    EXPECT(balanced_partition(100'000, 100, 4, 4, 512, 0, 256).grid == 25 * 13);
    // one query: spread over ceil(n / (16 x 512)) blocks when the CUs allow (the reference's rule)
    EXPECT(balanced_partition(50'003, 1, 1, 4, 512, 0, 256).grid == 7);
    EXPECT(balanced_partition(1'000, 1, 1, 4, 512, 0, 256).grid == 1);
    std::mt19937_64 rng(7);
    for (int trial = 0; trial < 300; ++trial) {
        const int64_t n = 1 + static_cast<int64_t>(rng() % 200'000);
        const std::size_t nq = 1 + rng() % 700;
        const int q = 1 << (rng() % 4);
        const int ilp = 1 << (rng() % 3);
        const int64_t slots = 1 + static_cast<int64_t>(rng() % 1100);
        const int bpq = (trial % 3 == 0) ? static_cast<int>(1 + rng() % 40) : 0;
        const int64_t cus = (trial % 2 == 0) ? 1 + static_cast<int64_t>(rng() % 300) : 0;
        const Partition p = balanced_partition(n, nq, q, ilp, slots, bpq, cus);
        EXPECT(p.slabs == static_cast<int64_t>((nq + q - 1) / q));
        EXPECT(p.n_gran == ((n + 63) / 64 + ilp - 1) / ilp);
        EXPECT(p.total == p.slabs * p.n_gran && p.grid >= 1 && p.grid <= p.total);
        if (bpq == 0) EXPECT(p.grid <= slots);
        if (bpq == 0 && cus > 0) EXPECT(p.grid <= p.slabs * cus);  // a slab never gets more blocks than CUs
        const bool aligned = bpq > 0 || p.slabs <= slots;  // whole blocks per slab: no block crosses a boundary
        if (aligned) EXPECT(p.grid % p.slabs == 0);
        // block ranges tile [0, total) in order, and every block is non-empty
        int64_t prev_end = 0;
        for (int64_t b = 0; b < p.grid; ++b) {
            const int64_t start = b * p.total / p.grid, end = (b + 1) * p.total / p.grid;
            EXPECT(start == prev_end && end > start);
            prev_end = end;
        }
        EXPECT(prev_end == p.total);
        // the blocks touching each slab are [first(slab start), first(slab end - 1)], at most max_slots of them
        for (int64_t slab = 0; slab < p.slabs; ++slab) {
            const int64_t lo = first_block(slab * p.n_gran, p.grid, p.total);
            const int64_t hi = first_block((slab + 1) * p.n_gran - 1, p.grid, p.total);
            EXPECT(lo * p.total / p.grid <= slab * p.n_gran && slab * p.n_gran < (lo + 1) * p.total / p.grid);
            EXPECT(hi - lo + 1 <= p.max_slots);
            if (aligned) EXPECT(hi - lo + 1 == p.grid / p.slabs && lo == slab * (p.grid / p.slabs));
        }
    }
}

int main() { return vktest::run(); }

namespace {

std::vector<uint8_t> random_codes(size_t n, size_t m, uint64_t seed, int distinct_rows = 0) {
    std::mt19937_64 rng(seed);
    std::vector<uint8_t> c(n * m);
    if (distinct_rows > 0) {  // clustered: every row one of a few prototypes
        std::vector<uint8_t> proto(static_cast<size_t>(distinct_rows) * m);
        for (auto& x : proto) x = static_cast<uint8_t>(rng());
        for (size_t i = 0; i < n; ++i) {
            const size_t r = rng() % distinct_rows;
            std::copy(proto.begin() + r * m, proto.begin() + (r + 1) * m, c.begin() + i * m);
        }
    } else {
        for (auto& x : c) x = static_cast<uint8_t>(rng());
    }
    return c;
}

// Mean over the full 256-slot blocks' (pass, sub-space) pairs of the largest number of distinct table entries in one
// bank group among a pass's `lanes` lanes, the group of code e of sub-space s being rows[s * 256 + e] % lanes
// (rows empty: e % lanes); vec_of(slot) gives the slot's vector. Written out here, independently of
// vk::order::block_stats.
template <typename F>
double bank_load(const std::vector<uint8_t>& codes, size_t n, size_t m, int lanes, const std::vector<uint8_t>& rows,
                 F vec_of) {
    double total = 0;
    size_t count = 0;
    for (size_t p0 = 0; p0 + lanes <= n / 256 * 256; p0 += lanes)
        for (size_t s = 0; s < m; ++s) {
            bool seen[256] = {};
            int groups[64] = {}, mx = 0;
            for (int l = 0; l < lanes; ++l) {
                const int e = codes[vec_of(p0 + l) * m + s];
                if (seen[e]) continue;
                seen[e] = true;
                const int row = rows.empty() ? e : rows[s * 256 + e];
                mx = std::max(mx, ++groups[row % lanes]);
            }
            total += mx;
            ++count;
        }
    return total / count;
}

bool is_permutation_of_rows(const std::vector<uint8_t>& rows, size_t m) {
    for (size_t s = 0; s < m; ++s) {
        std::vector<char> hit(256, 0);
        for (int e = 0; e < 256; ++e) hit[rows[s * 256 + e]] = 1;
        if (std::count(hit.begin(), hit.end(), 1) != 256) return false;
    }
    return true;
}

}  // namespace

CASE("slot order: slots [0, n) hold every vector once, blocks sorted by code bytes, tiles spread; padding holds 0") {
    const std::pair<size_t, size_t> shapes[] = {{1, 16},     {63, 16},         {300, 16},          {4096, 32},
                                                {65536, 16}, {65536 + 700, 16}, {3 * 65536 + 17, 16}};
    for (const auto& [n, m] : shapes)
        for (int clustered : {0, 5})
            for (int lanes : {16, 32, 64}) {
                if (lanes != 16 && n > 70000) continue;  // the wider passes on the smaller shapes
                const std::vector<uint8_t> codes = random_codes(n, m, n * 7 + m + clustered, clustered);
                const size_t n_pad = (n + 255) / 256 * 256;
                const vk::order::SlotOrder o = vk::order::slot_order(codes.data(), n, m, n_pad, lanes, 1);
                const std::vector<uint32_t>& ids = o.ids;
                const vk::order::SlotOrder o3 = vk::order::slot_order(codes.data(), n, m, n_pad, lanes, 3);
                EXPECT(ids == o3.ids && o.rows == o3.rows && o.lanes == lanes);
                EXPECT(ids.size() == n_pad && o.rows.size() == m * 256 && is_permutation_of_rows(o.rows, m));
                std::vector<char> seen(n, 0);
                bool once = true;
                for (size_t slot = 0; slot < n; ++slot) {
                    const size_t v = ids[vk::order::interleaved(slot)];
                    once = once && v < n && !seen[v];
                    if (v < n) seen[v] = 1;
                }
                EXPECT(once);
                // Sorted slot t sits at slot spread_slot(t): tiles of the full blocks spread, the partial block in
                // place. Taken in sorted order unit by unit (pools of pool_blocks full blocks, then single blocks),
                // every vector of a later unit sorts at or after every vector of an earlier one (dealing only
                // permutes within a unit).
                auto key = [&](size_t v) { return (uint32_t(codes[v * m]) << 24) | (uint32_t(codes[v * m + 1]) << 16) |
                                                  (uint32_t(codes[v * m + 2]) << 8) | codes[v * m + 3]; };
                const size_t tiles = n / 256 * 4, stride = vk::order::spread_stride(tiles);
                const vk::order::Units units(n, vk::order::pool_blocks(m, lanes));
                std::vector<char> used(n, 0);
                bool bijective = true, sorted = true;
                uint32_t prev_max = 0;
                for (size_t u = 0; u < units.count; ++u) {
                    const size_t b0 = units.unit_block(u) * 256, b1 = b0 + units.unit_size(u) * 256;
                    uint32_t lo = UINT32_MAX, hi = 0;
                    for (size_t t = b0; t < std::min(n, b1); ++t) {
                        const size_t at = vk::order::spread_slot(t, tiles, stride);
                        bijective = bijective && at < n && !used[at];
                        if (at >= n) continue;
                        used[at] = 1;
                        const uint32_t k = key(ids[vk::order::interleaved(at)]);
                        lo = std::min(lo, k);
                        hi = std::max(hi, k);
                    }
                    sorted = sorted && (u == 0 || prev_max <= lo);
                    prev_max = hi;
                }
                EXPECT(bijective);
                EXPECT(sorted);
                bool pad_zero = true;
                for (size_t slot = n; slot < n_pad; ++slot) pad_zero = pad_zero && ids[vk::order::interleaved(slot)] == 0;
                EXPECT(pad_zero);
            }
}

CASE("slot order: dealing pools fit the GPU builder's LDS budget; units cover every block once") {
    EXPECT(vk::order::pool_blocks(16, 16) == 4 && vk::order::pool_blocks(32, 16) == 2 && vk::order::pool_blocks(64, 16) == 1);
    EXPECT(vk::order::pool_blocks(64, 32) == 2 && vk::order::pool_blocks(32, 32) == 4 && vk::order::pool_blocks(48, 32) == 2);
    for (size_t m : {size_t{16}, size_t{32}, size_t{48}, size_t{64}})
        for (int lanes : {16, 32, 64}) {
            const int pool = vk::order::pool_blocks(m, lanes);
            EXPECT(vk::order::pool_lds_bytes(m, lanes, pool) <= vk::order::kPoolLdsBytes && 256 * pool / lanes <= 64);
        }
    for (size_t n : {size_t{1}, size_t{255}, size_t{256}, size_t{1023}, size_t{1024}, size_t{5 * 256 + 3}, size_t{9 * 256}})
        for (int pool : {1, 2, 4}) {
            const vk::order::Units units(n, pool);
            std::vector<int> hits((n + 255) / 256, 0);
            for (size_t u = 0; u < units.count; ++u)
                for (size_t b = 0; b < units.unit_size(u); ++b) ++hits[units.unit_block(u) + b];
            bool once = true;
            for (int h : hits) once = once && h == 1;
            EXPECT(once);
            for (size_t u = 0; u < units.pools; ++u) EXPECT((units.unit_block(u) + pool) * 256 <= n);  // pools are full
        }
}

CASE("slot order: the spread stride is coprime with the tile count and near its golden section") {
    for (size_t full : {size_t{3}, size_t{4}, size_t{10}, size_t{256}, size_t{3906}, size_t{390625}}) {
        const size_t s = vk::order::spread_stride(full);
        size_t a = s, b = full;
        while (b) { const size_t t = a % b; a = b; b = t; }
        EXPECT(a == 1);
        EXPECT(s >= full * 0.6 && s <= full * 0.65 + 2);
    }
    EXPECT(vk::order::spread_stride(1) == 1 && vk::order::spread_stride(2) == 1);
}

CASE("slot order: an inverted list's members sorted by code key (ties by id), full tiles spread") {
    const size_t n = 30000, m = 16;
    const std::vector<uint8_t> codes = random_codes(n, m, 7, 5);
    for (size_t count : {size_t{0}, size_t{1}, size_t{63}, size_t{64}, size_t{200}, size_t{9999}}) {
        std::vector<int32_t> members;
        for (size_t i = 0; i < count; ++i) members.push_back(static_cast<int32_t>(i * 3));
        std::vector<int32_t> placed = members;
        std::vector<uint64_t> scratch;
        vk::order::order_members(codes.data(), m, placed.data(), placed.size(), scratch);
        std::vector<int32_t> a = members, b = placed;
        std::sort(a.begin(), a.end());
        std::sort(b.begin(), b.end());
        EXPECT(a == b);
        // undo the spread and check the sorted order
        const size_t tiles = count / 64, stride = vk::order::spread_stride(tiles);
        std::vector<int32_t> sorted(count);
        for (size_t j = 0; j < count; ++j) sorted[j] = placed[vk::order::spread_slot(j, tiles, stride)];
        bool ordered = true;
        for (size_t j = 1; j < count; ++j) {
            const uint32_t k0 = vk::order::code_key(&codes[sorted[j - 1] * m], m);
            const uint32_t k1 = vk::order::code_key(&codes[sorted[j] * m], m);
            ordered = ordered && (k0 < k1 || (k0 == k1 && sorted[j - 1] < sorted[j]));
        }
        EXPECT(ordered);
    }
    EXPECT(vk::order::code_key(&codes[0], 2) == ((uint32_t(codes[0]) << 24) | (uint32_t(codes[1]) << 16)));
}

CASE("slot order: the order lowers the LDS bank load of uniform random codes") {
    const size_t n = 2 * 65536, m = 16;
    const std::vector<uint8_t> codes = random_codes(n, m, 99);
    for (int lanes : {16, 32}) {
        const vk::order::SlotOrder o = vk::order::slot_order(codes.data(), n, m, n, lanes, 2);
        const double natural = bank_load(codes, n, m, lanes, {}, [](size_t slot) { return slot; });
        const double ordered = bank_load(codes, n, m, lanes, o.rows,
                                         [&](size_t slot) { return size_t{o.ids[vk::order::interleaved(slot)]}; });
        std::printf("    %d lanes per pass: bank load in vector order %.3f, slot order %.3f\n", lanes, natural, ordered);
        EXPECT(natural > (lanes == 16 ? 2.8 : 3.0) && ordered < natural * 0.8);
    }
}

CASE("slot order: co-occurrence counts are symmetric, the GPU's upper triangle mirrors to them, and match a count") {
    const size_t n = 20 * 256 + 9, m = 16;
    const std::vector<uint8_t> codes = random_codes(n, m, 5, 40);
    const std::vector<uint32_t> sorted = vk::order::sorted_ids(codes.data(), n, m, 1);
    for (int lanes : {16, 64}) {
        const std::vector<uint32_t> w = vk::order::cooccurrence(codes.data(), n, m, sorted.data(), lanes, 3);
        std::vector<uint32_t> upper(w.size(), 0);
        bool symmetric = true, zero_diagonal = true;
        for (size_t s = 0; s < m; ++s)
            for (int a = 0; a < 256; ++a) {
                zero_diagonal = zero_diagonal && w[(s * 256 + a) * 256 + a] == 0;
                for (int b = 0; b < 256; ++b) {
                    symmetric = symmetric && w[(s * 256 + a) * 256 + b] == w[(s * 256 + b) * 256 + a];
                    if (a < b) upper[(s * 256 + a) * 256 + b] = w[(s * 256 + a) * 256 + b];
                }
            }
        EXPECT(symmetric && zero_diagonal);
        vk::order::mirror_counts(upper, m);
        EXPECT(upper == w);
        // Every full block is sampled here (20 < kSampleBlocks): entry pairs counted directly, sub-space 3.
        uint64_t pairs = 0, total = 0;
        for (size_t b0 = 0; b0 + 256 <= n; b0 += 256)
            for (size_t p0 = b0; p0 < b0 + 256; p0 += lanes) {
                std::vector<int> distinct;
                for (int l = 0; l < lanes; ++l) {
                    const int e = codes[sorted[p0 + l] * m + 3];
                    if (std::find(distinct.begin(), distinct.end(), e) == distinct.end()) distinct.push_back(e);
                }
                pairs += distinct.size() * (distinct.size() - 1);
            }
        for (int a = 0; a < 256; ++a)
            for (int b = 0; b < 256; ++b) total += w[(3 * 256 + a) * 256 + b];
        EXPECT(pairs == total);
    }
}

CASE("slot order: fitted table rows put entries that are read together into different bank groups") {
    // 16 cliques of 16 entries, clique c = {c, c + 16, ..., c + 240}: with rows = codes every clique sits in one bank
    // group (entry % 16). Each clique's entries co-occur; a clique's members must end in 16 distinct groups.
    for (int lanes : {16, 32}) {
        std::vector<uint32_t> w(256 * 256, 0);
        for (int a = 0; a < 256; ++a)
            for (int b = 0; b < 256; ++b)
                if (a != b && a % 16 == b % 16) w[a * 256 + b] = 5;
        std::vector<uint8_t> rows(256);
        vk::order::fit_rows(w.data(), lanes, rows.data());
        EXPECT(is_permutation_of_rows(rows, 1));
        bool spread = true;
        for (int c = 0; c < 16; ++c) {
            std::vector<int> groups;
            for (int j = 0; j < 16; ++j) groups.push_back(rows[c + 16 * j] % lanes);
            std::sort(groups.begin(), groups.end());
            spread = spread && std::unique(groups.begin(), groups.end()) == groups.end();
        }
        EXPECT(spread);
    }
    std::vector<uint32_t> none(256 * 256, 0);
    std::vector<uint8_t> rows(256);
    vk::order::fit_rows(none.data(), 16, rows.data());
    bool identity = true;
    for (int e = 0; e < 256; ++e) identity = identity && rows[e] == e;
    EXPECT(identity);  // nothing co-occurs: rows stay the codes
}

CASE("slot order: on clustered codes the fitted rows lower the modelled bank load") {
    // Codes whose vectors draw each sub-space's entry from one of a few per-cluster sets that share a bank group.
    const size_t n = 64 * 256, m = 16;
    std::mt19937_64 rng(17);
    std::vector<uint8_t> codes(n * m);
    for (size_t i = 0; i < n; ++i) {
        const int cluster = static_cast<int>(rng() % 64);
        for (size_t s = 0; s < m; ++s) {
            const int base = (cluster * 7 + static_cast<int>(s) * 3) % 16;  // the cluster's bank group in sub-space s
            codes[i * m + s] = static_cast<uint8_t>(s < 4 ? cluster * 4 + rng() % 4 : base + 16 * (rng() % 16));
        }
    }
    const vk::order::SlotOrder o = vk::order::slot_order(codes.data(), n, m, n, 16, 2);
    auto vec = [&](size_t slot) { return size_t{o.ids[vk::order::interleaved(slot)]}; };
    const double plain = bank_load(codes, n, m, 16, {}, vec), fitted = bank_load(codes, n, m, 16, o.rows, vec);
    std::printf("    clustered codes, slot order: bank load with rows = codes %.3f, fitted rows %.3f\n", plain, fitted);
    EXPECT(fitted < plain * 0.8);
}
