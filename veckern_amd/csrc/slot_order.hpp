// Slot order of the fused scans' code layout (host side, at searcher creation while the codes are at hand).
//
// A wave64 ds_read_b128 is served in four passes of 16 consecutive lanes; within a pass, lanes reading different
// 16-byte table entries of one bank group (entry index mod 16, 64 banks of 4 bytes) queue one behind another, and
// lanes reading the same entry share one broadcast. Measured on MI355X (a pattern microbenchmark): a read costs about
// 4 cycles per CU when every pass has 16 distinct bank groups and about the sum over its passes of the largest
// number of distinct entries in one group otherwise (uniform random entries: ~3 per pass, ~12 cycles).
//
// The order has two levels. Within each run of 65536 slots, the run's vectors are sorted by their first two code
// bytes (a counting sort): vectors that share code bytes then sit in the same passes, where their shared entries
// are broadcasts. Within each full block of 256 slots (16 passes, four tiles), the block's vectors are then dealt
// to passes first-fit: in sorted order, each goes to the pass (with room) where its entries add the fewest distinct
// entries to bank groups already in use; entries already present cost nothing. Only blocks with little sharing are
// dealt (kDealMinDistinct), and only where it lowers the block's bank load. Mean of the largest distinct-entry count
// per (pass, sub-space): uniform random codes 2.92 in vector order, 2.70 sorted, 2.14 sorted and dealt (100M uniform
// codes, nq=1000: 116.4 -> 106.0 ms per search).
//
// The result holds, per slot, its vector's index within its run (16 bits), interleaved by four tiles:
// ids[(tile / 4) * 256 + lane * 4 + tile % 4] for slot = tile * 64 + lane. Slots [0, n) hold every vector exactly
// once, each run's own; padding slots [n, n_pad) hold 0 and are never read as vectors.
#pragma once

#include <algorithm>
#include <climits>
#include <cstddef>
#include <cstdint>
#include <thread>
#include <vector>

namespace vk::order {

constexpr size_t kRun = 65536;   // slots per run: a vector's index within its run fits in 16 bits
constexpr size_t kBlock = 256;   // slots dealt together: 16 passes of 16 lanes, four tiles
constexpr int kPasses = 16;
constexpr int kLanes = 16;

inline size_t interleaved(size_t slot) {
    const size_t tile = slot / 64, lane = slot % 64;
    return (tile / 4) * 256 + lane * 4 + tile % 4;
}

// Deals one full block's vectors (run-relative indices, in sorted order) to its 16 passes; `out` receives them in
// slot order (pass p holds slots 16p .. 16p+15). Scratch: `present[s * 256 + e]`, the passes (bit p) that already
// read entry e of sub-space s, and `groups[(s * 16 + g) * 16 + p]`, pass p's distinct entries in bank group g of
// sub-space s; the costs of all 16 passes are summed side by side (the compiler vectorises the pass loop).
inline void deal_block(const uint8_t* run_codes, size_t m, const uint32_t* vec, uint32_t* out,
                       std::vector<uint16_t>& present, std::vector<uint8_t>& groups) {
    present.assign(m * 256, 0);
    groups.assign(m * 16 * kPasses, 0);
    int fill[kPasses] = {};
    for (size_t i = 0; i < kBlock; ++i) {
        const uint8_t* row = run_codes + static_cast<size_t>(vec[i]) * m;
        uint16_t cost[kPasses] = {};
        for (size_t s = 0; s < m; ++s) {
            const unsigned e = row[s];
            const unsigned mask = present[s * 256 + e];
            const uint8_t* g = &groups[(s * 16 + (e & 15)) * kPasses];
            for (int p = 0; p < kPasses; ++p) cost[p] += ((mask >> p) & 1u) ? 0 : g[p];
        }
        int best = -1;
        unsigned best_cost = UINT_MAX;
        for (int p = 0; p < kPasses; ++p)
            if (fill[p] < kLanes && cost[p] < best_cost) {
                best_cost = cost[p];
                best = p;
            }
        for (size_t s = 0; s < m; ++s) {
            const unsigned e = row[s];
            uint16_t& mask = present[s * 256 + e];
            if ((mask >> best) & 1u) continue;
            mask = static_cast<uint16_t>(mask | (1u << best));
            ++groups[(s * 16 + (e & 15)) * kPasses + best];
        }
        out[best * kLanes + fill[best]++] = vec[i];
    }
}

// A block in slot order, over its 16 passes and the m sub-spaces: `load`, the sum of the largest number of distinct
// entries in one bank group among a pass's 16 lanes (about the LDS cycles of its reads, up to a factor), and
// `distinct`, the sum of the numbers of distinct entries.
struct BlockStats {
    unsigned load = 0, distinct = 0;
};
inline BlockStats block_stats(const uint8_t* run_codes, size_t m, const uint32_t* block) {
    BlockStats st;
    for (int p = 0; p < kPasses; ++p)
        for (size_t s = 0; s < m; ++s) {
            uint64_t seen[4] = {};
            uint8_t groups[16] = {};
            unsigned mx = 0;
            for (int l = 0; l < kLanes; ++l) {
                const unsigned e = run_codes[static_cast<size_t>(block[p * kLanes + l]) * m + s];
                if ((seen[e >> 6] >> (e & 63)) & 1) continue;
                seen[e >> 6] |= uint64_t{1} << (e & 63);
                mx = std::max<unsigned>(mx, ++groups[e & 15]);
                ++st.distinct;
            }
            st.load += mx;
        }
    return st;
}

// Blocks whose sorted passes read at least this many distinct entries per (pass, sub-space) on average are dealt.
// Uniform random codes: 14 (dealing lowers their load 2.70 -> 2.14); 1M Gaussian-mixture codes: 2-6 per block,
// where dealing lowers the modelled load too (1.41 -> 1.31) but measured 2 % slower (their passes' shared entries
// are split up).
constexpr unsigned kDealMinDistinct = 8;

// The slot ids of runs [run_lo, run_hi) into `ids` (sized n_pad). Codes row-major n x m.
inline void order_runs(const uint8_t* codes, size_t n, size_t m, size_t run_lo, size_t run_hi, uint16_t* ids) {
    std::vector<uint32_t> start(kRun + 1), sorted(kRun), dealt(kBlock);
    std::vector<uint16_t> present;
    std::vector<uint8_t> groups;
    for (size_t r = run_lo; r < run_hi; ++r) {
        const size_t r0 = r * kRun, len = std::min(kRun, n - r0);
        const uint8_t* run_codes = codes + r0 * m;
        auto key = [&](size_t i) {
            const uint8_t* row = run_codes + i * m;
            return (static_cast<uint32_t>(row[0]) << 8) | (m > 1 ? row[1] : 0u);
        };
        std::fill(start.begin(), start.end(), 0u);
        for (size_t i = 0; i < len; ++i) ++start[key(i) + 1];
        for (size_t b = 0; b < kRun; ++b) start[b + 1] += start[b];
        for (size_t i = 0; i < len; ++i) sorted[start[key(i)]++] = static_cast<uint32_t>(i);
        for (size_t b0 = 0; b0 < len; b0 += kBlock) {
            const uint32_t* block = sorted.data() + b0;
            if (b0 + kBlock <= len) {
                const BlockStats st = block_stats(run_codes, m, block);
                if (st.distinct >= kDealMinDistinct * kPasses * m) {
                    deal_block(run_codes, m, block, dealt.data(), present, groups);
                    if (block_stats(run_codes, m, dealt.data()).load < st.load) block = dealt.data();
                }
            }
            const size_t cnt = std::min(kBlock, len - b0);
            for (size_t j = 0; j < cnt; ++j) ids[interleaved(r0 + b0 + j)] = static_cast<uint16_t>(block[j]);
        }
    }
}

// Slot ids of the whole layout; runs are ordered on up to `threads` host threads.
inline std::vector<uint16_t> slot_ids(const uint8_t* codes, size_t n, size_t m, size_t n_pad, unsigned threads = 0) {
    std::vector<uint16_t> ids(n_pad, 0);
    const size_t runs = (n + kRun - 1) / kRun;
    if (threads == 0) threads = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    threads = static_cast<unsigned>(std::min<size_t>(threads, runs));
    if (threads <= 1) {
        order_runs(codes, n, m, 0, runs, ids.data());
        return ids;
    }
    std::vector<std::thread> pool;
    for (unsigned t = 0; t < threads; ++t)
        pool.emplace_back(order_runs, codes, n, m, runs * t / threads, runs * (t + 1) / threads, ids.data());
    for (std::thread& th : pool) th.join();
    return ids;
}

}  // namespace vk::order
