// Code layout of the fused scans (slot order and table rows): the host definition. Searchers build the same layout
// on the GPU (slot_order.hip, checked slot for slot and row for row against this one) the first time a v8/v9 search
// needs it; this host version orders inverted-list members at index build and the layouts of m > 64.
//
// A wave64 LDS read of E-byte table entries is served in passes of 256 / E lanes (16-byte entries: four passes of
// 16 consecutive lanes; 8-byte: two of 32; 4-byte: one of 64); within a pass, lanes reading different entries of one
// bank group (table row mod the pass's lanes, 64 banks of 4 bytes) queue one behind another, and lanes reading the
// same entry share one broadcast. Measured on MI355X (a pattern microbenchmark): a 16-byte read costs about 4
// cycles per CU when every pass has 16 distinct bank groups and about the sum over its passes of the largest number
// of distinct entries in one group otherwise (uniform random entries: ~3 per pass, ~12 cycles). The same model with
// 32-lane passes matches the counters of 8-byte reads (1M x m=64: 5.68 modelled against 5.62 LDS cycles per read).
//
// The layout has four steps. All vectors are sorted by their first four code bytes (a radix sort): vectors that
// share code bytes then sit in the same passes, where their shared entries are broadcasts. Each sub-space's table
// rows are then fitted (fit_rows) to the co-occurrences of its entries in the sorted passes of a sample of blocks:
// entries that passes often read together get rows in different bank groups, and the layout stores each code's row
// in place of the code (the scan's table build writes the entry of code c at its row, so every sum is unchanged).
// Next, within each full block of 256 slots (four tiles), blocks with little sharing (kDealMinDistinct) have their
// vectors dealt to passes first-fit by the fitted bank groups, kept only where that lowers the block's bank load.
// Mean of the largest distinct-entry count per (pass, sub-space), 16-lane passes: 1M Gaussian-mixture codes
// (m=16) 1.21 sorted, 1.05 with fitted rows; m=32 1.86, 1.51; 100M uniform codes 2.92 in vector order, 2.56 sorted,
// 2.03 dealt (rows change nothing there). Measured per search: 1M x m=16 0.646 -> 0.627 ms, m=32 k=100 1.85 ->
// 1.71, m=64 k=100 (32-lane passes) 4.88 -> 4.34, 10M x m=16 5.30 -> 4.96 (earlier, dealing alone took 100M
// uniform codes from 116.4 to 106.0 ms).
// Last, the tiles of the full blocks are spread over the layout: sorted tile t (64 slots) goes to tile position
// t * s mod T (T tiles in full blocks, s the integer nearest T / golden ratio that is coprime with T); the partial
// last block stays last. A scan block's range of slots then holds tiles from all over the sorted order, and a
// granule's U consecutive tiles come from far-apart parts of it, as in vector order. Kept in sorted order, a scan
// block covers a narrow range of leading code bytes and a granule a run of near-identical vectors: the wave lists
// admit candidates in bursts, and the blocks nearest the query take many more inserts than the rest. Measured scan
// time (ms) of blocks in sorted order / spread by 256-slot block / by 16-slot pass / by 64-slot tile: 1M x nq=1000
// 0.750 / 0.730 / 0.735 / 0.711, fp16 tables 0.896 / 0.837 / 0.762 / 0.799; 10M x nq=1000 5.91 / 5.91 / 6.28 / 5.88;
// 10M x one query 0.059 / 0.056 / 0.048 / 0.047; 100M x nq=1000 100.3 / 99.9 / 99.7 / 99.8.
//
// The ids are kept per slot, interleaved by four tiles: ids[(tile / 4) * 256 + lane * 4 + tile % 4] for
// slot = tile * 64 + lane. Slots [0, n) hold every vector exactly once; padding slots [n, n_pad) hold 0 and are
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

constexpr size_t kBlock = 256;  // slots dealt together: one wave step of four 64-slot tiles
constexpr int kEntries = 256;   // table rows per sub-space

// Lanes served together by one pass of a table read, and the number of bank groups: 64 banks of 4 bytes return
// 256 bytes per clock, so a pass holds 256 / (entry bytes) lanes (16-byte entries: 16 lanes, 8-byte: 32, 4-byte:
// 64) and an entry's bank group is its table row mod that count. 2-byte entries (fp16 tables, one query) are taken
// as 4-byte ones: there two rows share each bank word, which this model does not separate.
inline int pass_lanes(int entry_bytes) { return entry_bytes >= 16 ? 16 : entry_bytes >= 8 ? 32 : 64; }

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

inline size_t interleaved(size_t slot) {
    const size_t tile = slot / 64, lane = slot % 64;
    return (tile / 4) * 256 + lane * 4 + tile % 4;
}

// The fused scans' code layout: per slot, its vector's id (interleaved by four tiles, `interleaved`), and per
// sub-space the LDS table row of each code value (`rows[s * 256 + e]`: the layout stores rows[s * 256 + code]
// in place of the code, and the scan's table build writes entry e of sub-space s at that row).
struct SlotOrder {
    std::vector<uint32_t> ids;
    std::vector<uint8_t> rows;
    int lanes = 16;
};

// The cost of `slots` slots (whole blocks) in the model of the reads: over their slots / lanes passes and the m
// sub-spaces, `load` sums the largest number of distinct entries in one bank group among a pass's lanes (about the
// LDS cycles of its reads, up to a factor; entries read by several lanes of a pass are one broadcast), and
// `distinct` the numbers of distinct entries. `rows` holds the slots' code rows, `order` the local row of each
// slot, `group` the bank group of each (sub-space, code).
struct BlockStats {
    unsigned load = 0, distinct = 0;
};
template <typename Index>
inline BlockStats block_stats(const uint8_t* rows, size_t m, const Index* order, int lanes, const uint8_t* group,
                              size_t slots = kBlock) {
    BlockStats st;
    for (int p = 0; p < static_cast<int>(slots) / lanes; ++p)
        for (size_t s = 0; s < m; ++s) {
            uint64_t seen[4] = {};
            uint8_t count[64] = {};
            unsigned mx = 0;
            for (int l = 0; l < lanes; ++l) {
                const unsigned e = rows[static_cast<size_t>(order[p * lanes + l]) * m + s];
                if ((seen[e >> 6] >> (e & 63)) & 1) continue;
                seen[e >> 6] |= uint64_t{1} << (e & 63);
                mx = std::max<unsigned>(mx, ++count[group[s * kEntries + e]]);
                ++st.distinct;
            }
            st.load += mx;
        }
    return st;
}

// Blocks whose passes (in sorted order) read at least half as many distinct entries as they have lanes, on average
// over passes and sub-spaces, are dealt: kDealMinDistinct * m distinct (pass, sub-space) entries per block.
constexpr unsigned kDealMinDistinct = kBlock / 2;

// Consecutive full blocks dealt together (a pool): their vectors may go to any pass of the pool, which leaves the
// dealing more choice. The pool is the largest of 4, 2, 1 blocks with at most 64 passes whose bookkeeping fits the
// GPU builder's LDS budget (kPoolLdsBytes, sized for m rounded up to 64 when it is not 16, 32 or 64): entry masks
// (one bit per pass), group counts, pass maxima, bank groups, the pool's code rows and its dealt order. Modelled
// bank load (mean largest distinct-entry count per (pass, sub-space)): 100M uniform codes, 16-lane passes, 2.03 per
// block, 1.93 in pools of 4; 1M x m=64, 32-lane passes, 2.60 per block, 2.51 in pools of 2.
constexpr size_t kPoolLdsBytes = 120 * 1024;
constexpr size_t pool_lds_bytes(size_t m, int lanes, int pool) {
    const size_t mm = (m == 16 || m == 32 || m == 64) ? m : 64;
    const size_t passes = kBlock * static_cast<size_t>(pool) / static_cast<size_t>(lanes);
    const size_t mask = passes <= 16 ? 2 : passes <= 32 ? 4 : 8;
    return mm * kEntries * mask + mm * kEntries * pool + mm * passes + mm * kEntries + kBlock * pool * mm +
           2 * kBlock * pool;
}
constexpr int pool_blocks(size_t m, int lanes) {
    for (int pool = 4; pool > 1; pool /= 2)
        if (kBlock * pool / lanes <= 64 && pool_lds_bytes(m, lanes, pool) <= kPoolLdsBytes) return pool;
    return 1;
}

// The dealing's extra cost for an entry that raises a pass's largest bank-group count: 2 for passes of 32 or 64
// lanes, none for 16. Measured on the search kernel: 1M x m=64 (32 lanes) 4.42 -> 4.34 ms with it; 100M uniform
// codes (16 lanes) 99.2 -> 99.8 ms, so 16-lane passes go without.
inline unsigned raise_penalty(int lanes) { return lanes > 16 ? 2u : 0u; }

// Deals the vectors of `slots` slots (whole blocks; local rows 0..slots-1, in sorted order) to their passes; `out`
// receives local rows in slot order (pass p holds slots p * lanes ..). One vector at a time goes to the pass with
// room where it costs least, the lowest pass on ties. Its cost in a pass sums, over the sub-spaces whose entry the
// pass does not read yet, the entries the pass already reads in that entry's bank group, plus raise_penalty(lanes)
// if the entry would raise the pass's largest group count above max(that count, 1). Scratch: `present[s * 256 + e]`,
// the passes (bit p) that read entry e of sub-space s; `count[(s * lanes + g) * passes + p]`, pass p's distinct
// entries in group g of sub-space s; `top[s * passes + p]`, the largest of those over g.
inline void deal_block(const uint8_t* rows, size_t m, int lanes, const uint8_t* group, size_t slots, uint16_t* out,
                       std::vector<uint64_t>& present, std::vector<uint8_t>& count, std::vector<uint8_t>& top) {
    const int passes = static_cast<int>(slots) / lanes;  // at most 64
    present.assign(m * kEntries, 0);
    count.assign(m * lanes * passes, 0);
    top.assign(m * passes, 0);
    const unsigned raise = raise_penalty(lanes);
    int fill[64] = {};
    for (int i = 0; i < static_cast<int>(slots); ++i) {
        const uint8_t* row = rows + static_cast<size_t>(i) * m;
        unsigned cost[64] = {};
        for (size_t s = 0; s < m; ++s) {
            const unsigned e = row[s];
            const uint64_t mask = present[s * kEntries + e];
            const uint8_t* c = &count[(s * lanes + group[s * kEntries + e]) * passes];
            const uint8_t* t = &top[s * passes];
            for (int p = 0; p < passes; ++p)
                if (!((mask >> p) & 1u)) cost[p] += c[p] + (c[p] + 1u > std::max<unsigned>(t[p], 1u) ? raise : 0u);
        }
        int best = -1;
        unsigned best_cost = UINT_MAX;
        for (int p = 0; p < passes; ++p)
            if (fill[p] < lanes && cost[p] < best_cost) {
                best_cost = cost[p];
                best = p;
            }
        for (size_t s = 0; s < m; ++s) {
            const unsigned e = row[s];
            uint64_t& mask = present[s * kEntries + e];
            if ((mask >> best) & 1u) continue;
            mask |= uint64_t{1} << best;
            uint8_t& c = count[(s * lanes + group[s * kEntries + e]) * passes + best];
            uint8_t& t = top[s * passes + best];
            t = std::max<uint8_t>(t, ++c);
        }
        out[best * lanes + fill[best]++] = static_cast<uint16_t>(i);
    }
}

// Sampled blocks of the co-occurrence counts: up to this many full blocks, evenly spaced.
constexpr size_t kSampleBlocks = 4096;
inline size_t sample_count(size_t full_blocks) { return std::min(full_blocks, kSampleBlocks); }
inline size_t sample_block(size_t i, size_t full_blocks) { return i * full_blocks / sample_count(full_blocks); }

// Co-occurrence of code values within passes: `w[(s * 256 + a) * 256 + b]` counts the passes of the sampled
// blocks (in sorted order) whose lanes read both entries a != b of sub-space s. Sub-spaces are split over
// `threads` host threads.
inline std::vector<uint32_t> cooccurrence(const uint8_t* codes, size_t n, size_t m, const uint32_t* sorted, int lanes,
                                          unsigned threads) {
    std::vector<uint32_t> w(m * kEntries * kEntries, 0);
    const size_t full = n / kBlock;
    parallel(threads, [&](unsigned t) {
        for (size_t s = t; s < m; s += threads) {
            uint32_t* ws = &w[s * kEntries * kEntries];
            for (size_t i = 0; i < sample_count(full); ++i) {
                const uint32_t* block = sorted + sample_block(i, full) * kBlock;
                for (size_t p0 = 0; p0 < kBlock; p0 += static_cast<size_t>(lanes)) {
                    uint8_t entry[64];
                    int k = 0;
                    uint64_t seen[4] = {};
                    for (int l = 0; l < lanes; ++l) {
                        const unsigned e = codes[static_cast<size_t>(block[p0 + l]) * m + s];
                        if ((seen[e >> 6] >> (e & 63)) & 1) continue;
                        seen[e >> 6] |= uint64_t{1} << (e & 63);
                        entry[k++] = static_cast<uint8_t>(e);
                    }
                    for (int a = 0; a < k; ++a)
                        for (int b = 0; b < k; ++b)
                            if (a != b) ++ws[entry[a] * kEntries + entry[b]];
                }
            }
        }
    });
    return w;
}

constexpr int kFitSweeps = 64;

// Table rows of one sub-space from its co-occurrence counts `w` (256 x 256, symmetric, zero diagonal): rows start as
// the code values; then, in sweeps over the pairs (a, b), a < b, in order, two entries of different bank groups
// (row mod lanes) swap rows when that lowers the sum of co-occurrences within groups, until a sweep swaps nothing
// (at most kFitSweeps). Entries that pass often read together then sit in different bank groups.
inline void fit_rows(const uint32_t* w, int lanes, uint8_t* rows) {
    int64_t cost[kEntries][64] = {};  // cost[e][g]: co-occurrences of e with the entries of group g
    uint8_t grp[kEntries];
    for (int e = 0; e < kEntries; ++e) {
        rows[e] = static_cast<uint8_t>(e);
        grp[e] = static_cast<uint8_t>(e % lanes);
    }
    for (int e = 0; e < kEntries; ++e)
        for (int f = 0; f < kEntries; ++f) cost[e][grp[f]] += w[e * kEntries + f];
    for (int sweep = 0; sweep < kFitSweeps; ++sweep) {
        bool swapped = false;
        for (int a = 0; a < kEntries; ++a)
            for (int b = a + 1; b < kEntries; ++b) {
                const int ga = grp[a], gb = grp[b];
                if (ga == gb) continue;
                const int64_t wab = w[a * kEntries + b];
                if (cost[a][gb] + cost[b][ga] - 2 * wab >= cost[a][ga] + cost[b][gb]) continue;
                for (int f = 0; f < kEntries; ++f) {
                    const int64_t wa = w[f * kEntries + a], wb = w[f * kEntries + b];
                    cost[f][ga] += wb - wa;
                    cost[f][gb] += wa - wb;
                }
                std::swap(rows[a], rows[b]);
                grp[a] = static_cast<uint8_t>(gb);
                grp[b] = static_cast<uint8_t>(ga);
                swapped = true;
            }
        if (!swapped) break;
    }
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

// Table rows of every sub-space from full co-occurrence counts (cooccurrence), fitted on up to `threads` host
// threads (fit_rows per sub-space).
inline std::vector<uint8_t> fit_all_rows(const std::vector<uint32_t>& w, size_t m, int lanes, unsigned threads) {
    std::vector<uint8_t> rows(m * kEntries);
    threads = static_cast<unsigned>(std::max<size_t>(1, std::min<size_t>(threads, m)));
    parallel(threads, [&](unsigned t) {
        for (size_t s = t; s < m; s += threads) fit_rows(&w[s * kEntries * kEntries], lanes, &rows[s * kEntries]);
    });
    return rows;
}

// Completes counts of which only the entries [s][a][b] with a < b are filled (the GPU's): [s][b][a] = [s][a][b].
inline void mirror_counts(std::vector<uint32_t>& w, size_t m) {
    for (size_t s = 0; s < m; ++s) {
        uint32_t* ws = &w[s * kEntries * kEntries];
        for (int a = 0; a < kEntries; ++a)
            for (int b = a + 1; b < kEntries; ++b) ws[b * kEntries + a] = ws[a * kEntries + b];
    }
}

// Units of the dealing: the first full_blocks / pool * pool full blocks in pools of `pool`, then the remaining
// blocks one at a time (the partial last block, if any, among them). Unit u starts at block unit_block(u) and holds
// unit_size(u) blocks.
struct Units {
    size_t pools = 0, pool = 1, rest_first = 0, count = 0;
    Units(size_t n, int pool_) : pool(static_cast<size_t>(pool_)) {
        const size_t full = n / kBlock, blocks = (n + kBlock - 1) / kBlock;
        pools = pool > 1 ? full / pool : 0;
        rest_first = pools * pool;
        count = pools + (blocks - rest_first);
    }
    size_t unit_block(size_t u) const { return u < pools ? u * pool : rest_first + (u - pools); }
    size_t unit_size(size_t u) const { return u < pools ? pool : 1; }
};

// Units [u_lo, u_hi) of the sorted ids: a unit of full blocks is dealt where that pays (at least kDealMinDistinct * m
// distinct entries per block, and a lower modelled load), then every slot is written to `ids` at its spread slot. A
// unit's code rows are first gathered into a local copy, which the statistics and the dealing then read.
inline void order_units(const uint8_t* codes, size_t n, size_t m, const uint32_t* sorted, int lanes,
                        const uint8_t* group, const Units& units, size_t u_lo, size_t u_hi, uint32_t* ids) {
    const size_t tiles = n / kBlock * (kBlock / kTile), stride = spread_stride(tiles);
    auto place = [&](size_t t) { return interleaved(spread_slot(t, tiles, stride)); };
    const size_t cap = kBlock * units.pool;
    std::vector<uint16_t> local(cap), dealt(cap);
    std::vector<uint8_t> rows(cap * m);
    std::vector<uint64_t> present;
    std::vector<uint8_t> count, top;
    for (size_t i = 0; i < cap; ++i) local[i] = static_cast<uint16_t>(i);
    for (size_t u = u_lo; u < u_hi; ++u) {
        const size_t b0 = units.unit_block(u) * kBlock;
        const size_t slots = units.unit_size(u) * kBlock;
        const size_t cnt = std::min(slots, n - b0);
        const uint32_t* block = sorted + b0;
        if (cnt == slots) {
            for (size_t i = 0; i < slots; ++i)
                std::copy(codes + static_cast<size_t>(block[i]) * m, codes + (static_cast<size_t>(block[i]) + 1) * m,
                          rows.begin() + i * m);
            const BlockStats st = block_stats(rows.data(), m, local.data(), lanes, group, slots);
            if (st.distinct >= kDealMinDistinct * m * (slots / kBlock)) {
                deal_block(rows.data(), m, lanes, group, slots, dealt.data(), present, count, top);
                if (block_stats(rows.data(), m, dealt.data(), lanes, group, slots).load < st.load) {
                    for (size_t j = 0; j < slots; ++j) ids[place(b0 + j)] = block[dealt[j]];
                    continue;
                }
            }
        }
        for (size_t j = 0; j < cnt; ++j) ids[place(b0 + j)] = block[j];
    }
}

// The layout for table reads of `lanes` lanes per pass (pass_lanes): vectors sorted by their first four code bytes;
// table rows fitted per sub-space to the sorted passes' co-occurrences (fit_rows); the full blocks dealt in pools
// (pool_blocks) with the fitted bank groups where that pays; tiles spread and ids interleaved. Work is split over up to `threads` host
// threads.
inline SlotOrder slot_order(const uint8_t* codes, size_t n, size_t m, size_t n_pad, int lanes, unsigned threads = 0) {
    SlotOrder o;
    o.lanes = lanes;
    o.ids.assign(n_pad, 0);
    const size_t blocks = (n + kBlock - 1) / kBlock;
    if (threads == 0) threads = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    threads = static_cast<unsigned>(std::max<size_t>(1, std::min<size_t>(threads, (blocks + 63) / 64)));
    const std::vector<uint32_t> sorted = sorted_ids(codes, n, m, threads);
    const unsigned sub_threads = static_cast<unsigned>(std::min<size_t>(std::max(threads, 1u), m));
    o.rows = fit_all_rows(cooccurrence(codes, n, m, sorted.data(), lanes, sub_threads), m, lanes, sub_threads);
    std::vector<uint8_t> group(m * kEntries);
    for (size_t e = 0; e < group.size(); ++e) group[e] = static_cast<uint8_t>(o.rows[e] % lanes);
    const Units units(n, pool_blocks(m, lanes));
    parallel(threads, [&](unsigned t) {
        order_units(codes, n, m, sorted.data(), lanes, group.data(), units, units.count * t / threads,
                    units.count * (t + 1) / threads, o.ids.data());
    });
    return o;
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
