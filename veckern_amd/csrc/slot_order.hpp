// Slot order of the fused scans' code layout: the host definition. Searchers build the same order on the GPU
// (slot_order.hip, checked slot for slot against this one) the first time a v8/v9 search needs it; this host
// version orders inverted-list members at index build and the layouts of m > 64.
//
// A wave64 ds_read_b128 is served in four passes of 16 consecutive lanes; within a pass, lanes reading different
// 16-byte table entries of one bank group (entry index mod 16, 64 banks of 4 bytes) queue one behind another, and
// lanes reading the same entry share one broadcast. Measured on MI355X (a pattern microbenchmark): a read costs about
// 4 cycles per CU when every pass has 16 distinct bank groups and about the sum over its passes of the largest
// number of distinct entries in one group otherwise (uniform random entries: ~3 per pass, ~12 cycles).
//
// The order has three levels. All vectors are sorted by their first four code bytes (a radix sort): vectors that
// share code bytes then sit in the same passes, where their shared entries are broadcasts.
// Within each full block of 256 slots (16 passes, four tiles), the block's vectors are then dealt
// to passes first-fit: in sorted order, each goes to the pass (with room) where its entries add the fewest distinct
// entries to bank groups already in use; entries already present cost nothing. Only blocks with little sharing are
// dealt (kDealMinDistinct), and only where it lowers the block's bank load. Mean of the largest distinct-entry count
// per (pass, sub-space): uniform random codes 2.92 in vector order, 2.70 sorted, 2.14 sorted and dealt (100M uniform
// codes, nq=1000: 116.4 -> 106.0 ms per search).
// Last, the tiles of the full blocks are spread over the layout: sorted tile t (64 slots, four passes) goes to tile
// position t * s mod T (T tiles in full blocks, s the integer nearest T / golden ratio that is coprime with T); the
// partial last block stays last. A scan block's range of slots then holds tiles from all over the sorted order, and
// a granule's U consecutive tiles come from far-apart parts of it, as in vector order. Kept in sorted order, a scan
// block covers a narrow range of leading code bytes and a granule a run of near-identical vectors: the wave lists
// admit candidates in bursts, and the blocks nearest the query take many more inserts than the rest. Measured scan
// time (ms) of blocks in sorted order / spread by 256-slot block / by 16-slot pass / by 64-slot tile: 1M x nq=1000
// 0.750 / 0.730 / 0.735 / 0.711, fp16 tables 0.896 / 0.837 / 0.762 / 0.799; 10M x nq=1000 5.91 / 5.91 / 6.28 / 5.88;
// 10M x one query 0.059 / 0.056 / 0.048 / 0.047; 100M x nq=1000 100.3 / 99.9 / 99.7 / 99.8.
//
// The result holds, per slot, its vector's id, interleaved by four tiles: ids[(tile / 4) * 256 + lane * 4 + tile % 4]
// for slot = tile * 64 + lane. Slots [0, n) hold every vector exactly once; padding slots [n, n_pad) hold 0 and are
// never read as vectors. Sorting only within runs of 65536 slots (16-bit ids), with no spread, measured 1M x
// nq=1000 0.767 ms, fp16 tables 0.787, 10M 6.83, 10M x one query 0.048, 100M 105.7: whole clusters line up only in a
// global order.
#pragma once

#include <algorithm>
#include <climits>
#include <cstddef>
#include <cstdint>
#include <thread>
#include <utility>
#include <vector>

namespace vk::order {

constexpr size_t kBlock = 256;   // slots dealt together: 16 passes of 16 lanes, four tiles
constexpr int kPasses = 16;
constexpr int kLanes = 16;

inline size_t interleaved(size_t slot) {
    const size_t tile = slot / 64, lane = slot % 64;
    return (tile / 4) * 256 + lane * 4 + tile % 4;
}

// Deals one full block's vectors (ids, in sorted order) to its 16 passes; `out` receives them in
// slot order (pass p holds slots 16p .. 16p+15). Scratch: `present[s * 256 + e]`, the passes (bit p) that already
// read entry e of sub-space s, and `groups[(s * 16 + g) * 16 + p]`, pass p's distinct entries in bank group g of
// sub-space s; the costs of all 16 passes are summed side by side (the compiler vectorises the pass loop).
inline void deal_block(const uint8_t* codes, size_t m, const uint32_t* vec, uint32_t* out,
                       std::vector<uint16_t>& present, std::vector<uint8_t>& groups) {
    present.assign(m * 256, 0);
    groups.assign(m * 16 * kPasses, 0);
    int fill[kPasses] = {};
    for (size_t i = 0; i < kBlock; ++i) {
        const uint8_t* row = codes + static_cast<size_t>(vec[i]) * m;
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
inline BlockStats block_stats(const uint8_t* codes, size_t m, const uint32_t* block) {
    BlockStats st;
    for (int p = 0; p < kPasses; ++p)
        for (size_t s = 0; s < m; ++s) {
            uint64_t seen[4] = {};
            uint8_t groups[16] = {};
            unsigned mx = 0;
            for (int l = 0; l < kLanes; ++l) {
                const unsigned e = codes[static_cast<size_t>(block[p * kLanes + l]) * m + s];
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

// Runs f(t) for t in [0, threads) on host threads (inline when threads <= 1).
template <typename F>
inline void parallel(unsigned threads, F&& f) {
    if (threads <= 1) {
        f(0u);
        return;
    }
    std::vector<std::thread> pool;
    for (unsigned t = 0; t < threads; ++t) pool.emplace_back(f, t);
    for (std::thread& th : pool) th.join();
}

// Sort key of a code row: its first four bytes, big-endian (missing bytes count as 0).
inline uint32_t code_key(const uint8_t* row, size_t m) {
    uint32_t key = 0;
    for (size_t b = 0; b < 4; ++b) key = (key << 8) | (b < m ? row[b] : 0u);
    return key;
}

// All vector ids sorted by their first four code bytes (missing bytes count as 0): (key << 32 | id) pairs, then an
// LSD radix sort on the key's four bytes (stable, so equal keys keep id order), each pass split over `threads`
// contiguous chunks (per-chunk digit counts give every chunk its own output offsets).
inline std::vector<uint32_t> sorted_ids(const uint8_t* codes, size_t n, size_t m, unsigned threads) {
    std::vector<uint64_t> a(n), t(n);
    auto chunk = [&](unsigned c) { return std::pair<size_t, size_t>{n * c / threads, n * (c + 1) / threads}; };
    parallel(threads, [&](unsigned c) {
        const auto [lo, hi] = chunk(c);
        for (size_t i = lo; i < hi; ++i) {
            a[i] = (static_cast<uint64_t>(code_key(codes + i * m, m)) << 32) | static_cast<uint32_t>(i);
        }
    });
    std::vector<size_t> count(static_cast<size_t>(threads) * 256);
    for (int shift = 32; shift < 64; shift += 8) {
        std::fill(count.begin(), count.end(), size_t{0});
        parallel(threads, [&](unsigned c) {
            const auto [lo, hi] = chunk(c);
            size_t* cnt = count.data() + static_cast<size_t>(c) * 256;
            for (size_t i = lo; i < hi; ++i) ++cnt[(a[i] >> shift) & 0xffu];
        });
        size_t at = 0;  // digit-major, then chunk: chunk c's entries of digit d follow those of chunks < c
        for (int d = 0; d < 256; ++d)
            for (unsigned c = 0; c < threads; ++c) {
                size_t& slot = count[static_cast<size_t>(c) * 256 + d];
                const size_t k = slot;
                slot = at;
                at += k;
            }
        parallel(threads, [&](unsigned c) {
            const auto [lo, hi] = chunk(c);
            size_t* next = count.data() + static_cast<size_t>(c) * 256;
            for (size_t i = lo; i < hi; ++i) t[next[(a[i] >> shift) & 0xffu]++] = a[i];
        });
        a.swap(t);
    }
    std::vector<uint32_t> ids(n);
    for (size_t i = 0; i < n; ++i) ids[i] = static_cast<uint32_t>(a[i]);
    return ids;
}

// Multiplier of the spread over `count` tiles: the integer nearest count / golden ratio, raised until coprime with
// `count` (so that t -> t * stride mod count is a bijection); 1 for fewer than three tiles.
inline size_t spread_stride(size_t count) {
    if (count < 3) return 1;
    auto gcd = [](size_t a, size_t b) {
        while (b) {
            const size_t t = a % b;
            a = b;
            b = t;
        }
        return a;
    };
    size_t s = static_cast<size_t>(static_cast<double>(count) * 0.6180339887498949 + 0.5);
    while (gcd(s, count) != 1) ++s;
    return s;
}

constexpr size_t kTile = 64;  // slots of one wave step

// Slot of sorted slot t: in the full blocks' `tiles` tiles, its tile spread by `stride`; past them, t itself.
inline size_t spread_slot(size_t t, size_t tiles, size_t stride) {
    return t < tiles * kTile ? (t / kTile) * stride % tiles * kTile + t % kTile : t;
}

// Blocks [blk_lo, blk_hi) of the sorted ids: dealt where that pays, then written to `ids` at their spread slots. A
// full block's code rows are first gathered into a local copy, which the statistics and the dealing then read.
inline void order_blocks(const uint8_t* codes, size_t n, size_t m, const uint32_t* sorted, size_t blk_lo,
                         size_t blk_hi, uint32_t* ids) {
    const size_t tiles = n / kBlock * (kBlock / kTile), stride = spread_stride(tiles);
    auto place = [&](size_t t) { return interleaved(spread_slot(t, tiles, stride)); };
    std::vector<uint32_t> local(kBlock), dealt(kBlock);
    std::vector<uint8_t> rows(kBlock * m);
    std::vector<uint16_t> present;
    std::vector<uint8_t> groups;
    for (size_t i = 0; i < kBlock; ++i) local[i] = static_cast<uint32_t>(i);
    for (size_t blk = blk_lo; blk < blk_hi; ++blk) {
        const size_t b0 = blk * kBlock;
        const size_t cnt = std::min(kBlock, n - b0);
        const uint32_t* block = sorted + b0;
        if (cnt == kBlock) {
            for (size_t i = 0; i < kBlock; ++i)
                std::copy(codes + static_cast<size_t>(block[i]) * m, codes + (static_cast<size_t>(block[i]) + 1) * m,
                          rows.begin() + i * m);
            const BlockStats st = block_stats(rows.data(), m, local.data());
            if (st.distinct >= kDealMinDistinct * kPasses * m) {
                deal_block(rows.data(), m, local.data(), dealt.data(), present, groups);
                if (block_stats(rows.data(), m, dealt.data()).load < st.load) {
                    for (size_t j = 0; j < kBlock; ++j) ids[place(b0 + j)] = block[dealt[j]];
                    continue;
                }
            }
        }
        for (size_t j = 0; j < cnt; ++j) ids[place(b0 + j)] = block[j];
    }
}

// Slot ids of the whole layout; blocks are ordered on up to `threads` host threads.
inline std::vector<uint32_t> slot_ids(const uint8_t* codes, size_t n, size_t m, size_t n_pad, unsigned threads = 0) {
    std::vector<uint32_t> ids(n_pad, 0);
    const size_t blocks = (n + kBlock - 1) / kBlock;
    if (threads == 0) threads = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    threads = static_cast<unsigned>(std::max<size_t>(1, std::min<size_t>(threads, (blocks + 63) / 64)));
    const std::vector<uint32_t> sorted = sorted_ids(codes, n, m, threads);
    parallel(threads, [&](unsigned t) {
        order_blocks(codes, n, m, sorted.data(), blocks * t / threads, blocks * (t + 1) / threads, ids.data());
    });
    return ids;
}

// Members of one inverted list (vector ids), reordered: sorted by their code keys, equal keys in id order, then the
// list's full 64-slot tiles spread over its tile positions as in the exhaustive layout (t -> t * s mod T; members of a
// partial last tile stay last). The IVF scan reads one query's table per block (4-byte entries, one per lane):
// members that share code bytes then read shared table entries, which the LDS serves as broadcasts, and the spread
// keeps a wave's successive tiles from being near-identical runs. Not dealt: the dealing models 16-byte reads.
// 1M vectors, 1024 lists, nq=1000: nprobe 32 scan 0.233 ms in id order, 0.218 sorted, 0.214 sorted and spread;
// nprobe 8 0.098, 0.097, 0.092.
inline void order_members(const uint8_t* codes, size_t m, int32_t* members, size_t count,
                          std::vector<uint64_t>& scratch) {
    scratch.resize(count);
    for (size_t j = 0; j < count; ++j)
        scratch[j] = (static_cast<uint64_t>(code_key(codes + static_cast<size_t>(members[j]) * m, m)) << 32) |
                     static_cast<uint32_t>(members[j]);
    std::sort(scratch.begin(), scratch.end());
    const size_t tiles = count / kTile, stride = spread_stride(tiles);
    for (size_t j = 0; j < count; ++j)
        members[spread_slot(j, tiles, stride)] = static_cast<int32_t>(static_cast<uint32_t>(scratch[j]));
}

}  // namespace vk::order
