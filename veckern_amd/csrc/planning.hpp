// Host-side launch planning shared by the C ABI and its CPU tests: list-length dispatch, queries-per-block
// capping, the balanced work partition of the wave-list scan, and the blocks_x model of the grid kernels.
#pragma once

#include <algorithm>
#include <cstddef>
#include <cstdint>

namespace vk::plan {

// Smallest supported list length >= k (searcher.cu:86-90); 0 when k > 128.
inline int dispatched_k(size_t k) {
    for (int K : {8, 16, 32, 64, 128})
        if (k <= static_cast<size_t>(K)) return K;
    return 0;
}

// v3-v5 read the byte-interleaved layout, v6-v7 the 16-byte-word one (searcher.cu:222-241); v8 and v9 read the
// same words with the vectors in a sorted slot order.
inline bool uses_byte_layout(int v) { return v == 3 || v == 4 || v == 5; }
inline bool uses_word_layout(int v) { return v == 6 || v == 7; }
inline bool uses_sorted_layout(int v) { return v == 8 || v == 9; }  // words in the fused scans' slot order

// Queries per block: the requested Q, halved until the Q tables (Q * m * 256 entries) fit in LDS; for per-thread
// lists (v7) also until Q * K <= 64, as searcher.cu:213-220. entry_bytes: 4 for fp32 tables, 2 for fp16.
inline int effective_q(int requested, size_t m, size_t max_lds, bool per_thread_lists, int K,
                       size_t entry_bytes = sizeof(float)) {
    int q = std::max(requested, 1);
    while (q > 1 && ((per_thread_lists && q * K > 64) || static_cast<size_t>(q) * m * 256 * entry_bytes > max_lds))
        q /= 2;
    return q;
}

// A slab never holds more query slots than the batch needs: Q is halved while half of it still covers nq
// (nq = 1 scans with one table per block, whose b32 reads cost half the LDS time of a 4-query b128 read).
inline int cap_q_by_batch(int q, size_t nq) {
    while (q > 1 && static_cast<size_t>(q / 2) >= nq) q /= 2;
    return q;
}

// First block whose range [b*total/grid, (b+1)*total/grid) contains `item`.
inline int64_t first_block(int64_t item, int64_t grid, int64_t total) { return ((item + 1) * grid - 1) / total; }

// Balanced partition of the wave-list scan: slabs of q queries, each cut into granules of 64*ilp vectors;
// the slabs*n_gran items are split evenly over `grid` blocks. blocks_per_query > 0 fixes the blocks per slab.
// Otherwise, when the slabs are no more than the resident blocks (`slots`), each slab gets floor(slots / slabs)
// blocks, at most `cus` (> 0) of them and at most ceil(n / kMinBlockVectors), so that no block crosses a
// slab boundary; with more slabs than slots, grid = slots and blocks span slab boundaries. Measured on MI355X: with
// granules assigned statically to waves, blocks crossing slabs made the two blocks sharing a CU finish ~0.4 ms apart
// at 1M x nq=1000 (the older block's waves get issue priority): 1.43 ms against 1.35 ms slab-aligned (fp16 tables at
// Q = 8: 1.07 -> 0.90 ms). Aligned blocks also sweep the codes in lockstep (the blocks on each part of the codes read
// the same lines at about the same time, so the L2s serve most code reads). An even split over every resident slot
// when the aligned layout leaves slots idle (250 slabs on 512 slots) gained 0.5-1.6 % with codes in vector order,
// but on the sorted code layout, where the scan is faster and leans on the L2s, it lost: 1M x nq=1000 +7.7 %, 10M
// +9.6 %, 100M +1.5 %. A slab's blocks beyond one per CU only lengthen its final merge (nq = 1 at 10M: 73 -> 67 us).
// kMinBlockVectors: 16 vectors per thread of a 512-thread block, the reference's rule for how far a search is spread
// (searcher.cu:196-197; its tests/test_gpu.cpp:139-145 expect a single query over at least ceil(n / (16 * threads))
// blocks). Fewer vectors per block and a block's table build and merges outweigh its scan (100k vectors, nq=100:
// 20 blocks per slab 94 us, 10 blocks 78 us).
constexpr int64_t kMinBlockVectors = 8192;

struct Partition {
    int64_t slabs = 0, n_gran = 0, total = 0, grid = 0;
    int max_slots = 0;  // most blocks touching one slab = partial lists per query
};

inline Partition balanced_partition(int64_t n, size_t nq, int q, int ilp, int64_t slots, int blocks_per_query,
                                    int64_t cus = 0) {
    Partition p;
    p.slabs = static_cast<int64_t>((nq + q - 1) / q);
    const int64_t tiles = (n + 63) / 64;
    p.n_gran = (tiles + ilp - 1) / ilp;
    p.total = p.slabs * p.n_gran;
    slots = std::max<int64_t>(slots, 1);
    int64_t per_slab = blocks_per_query;
    if (per_slab <= 0 && p.slabs <= slots) {
        per_slab = slots / p.slabs;
        if (cus > 0) per_slab = std::min(per_slab, cus);
        per_slab = std::max<int64_t>(1, std::min(per_slab, (n + kMinBlockVectors - 1) / kMinBlockVectors));
    }
    if (per_slab > 0)
        p.grid = p.slabs * std::min<int64_t>(per_slab, p.n_gran);
    else
        p.grid = std::min<int64_t>(slots, p.total);
    // Keep grid * total (the kernel's range arithmetic) and the grid size itself in range.
    const int64_t limit = std::min<int64_t>(int64_t{1} << 31 >> 1, (int64_t{1} << 62) / std::max<int64_t>(p.total, 1));
    p.grid = std::max<int64_t>(1, std::min(p.grid, limit));
    for (int64_t slab = 0; slab < p.slabs; ++slab) {
        const int64_t lo = first_block(slab * p.n_gran, p.grid, p.total);
        const int64_t hi = first_block((slab + 1) * p.n_gran - 1, p.grid, p.total);
        p.max_slots = std::max<int>(p.max_slots, static_cast<int>(hi - lo + 1));
    }
    return p;
}

// Bulk admission into one-register wave lists pays while a block scans few vectors of a slab: it replaces the
// one-by-one inserts into the fresh lists of a block's first steps (several times the cost of a later step),
// and over millions of vectors per block its code in the scan loop costs about 1 %. Measured with 4 queries per
// block: 11k vectors per block -26 %, 39k -11 %, 500k neutral, 5M +1 %.
constexpr int64_t kBulkScanVectors = int64_t{1} << 18;

// Vectors one block scans of one slab (the longest run of a slab's granules in one block) below the bulk limit.
inline bool bulk_scan(const Partition& p, int ilp) {
    if (p.grid <= 0 || p.total <= 0) return false;
    const int64_t per_block = std::min(p.n_gran, (p.total + p.grid - 1) / p.grid);
    return per_block * 64 * ilp < kBulkScanVectors;
}

// blocks_x of the unfused scans (searcher.cu:172-177, where the reference also sizes v4 with it): an override, else
// about 8 blocks per CU over the whole grid, never fewer than 16 vectors per thread.
inline int64_t blocks_x_fill(int64_t n, int64_t grid_y, int threads, int cus, int blocks_per_query) {
    if (blocks_per_query > 0) return blocks_per_query;
    const int64_t by_work = (n + int64_t{threads} * 16 - 1) / (int64_t{threads} * 16);
    const int64_t to_fill = (int64_t{8} * cus + grid_y - 1) / grid_y;
    return std::max<int64_t>(1, std::min(by_work, to_fill));
}

// blocks_x of the per-thread-list fused scans v5-v7 (searcher.cu:184-208): a wave is the number of blocks resident
// at once (occupancy API); run time is taken as proportional to ceil(bx * grid_y / wave) / bx, and a larger bx is
// chosen only when it is at least 2% cheaper. bx is capped at max(64, 4 waves' worth per query row) and at 16
// vectors per thread.
struct WaveChoice {
    int64_t blocks_x = 1;
    double waves = 0.0;
};

inline WaveChoice blocks_x_waves(int64_t n, int64_t grid_y, int threads, int64_t resident, int blocks_per_query) {
    const int64_t wave = std::max<int64_t>(resident, 1);
    WaveChoice c;
    if (blocks_per_query > 0) {
        c.blocks_x = blocks_per_query;
    } else {
        const int64_t cap = std::max<int64_t>(64, 4 * ((wave + grid_y - 1) / grid_y));
        const int64_t useful = (n + int64_t{threads} * 16 - 1) / (int64_t{threads} * 16);
        const int64_t max_bx = std::max<int64_t>(1, std::min(cap, useful));
        double best = static_cast<double>((grid_y + wave - 1) / wave);
        for (int64_t bx = 2; bx <= max_bx; ++bx) {
            const double cost = static_cast<double>((bx * grid_y + wave - 1) / wave) / static_cast<double>(bx);
            if (cost < 0.98 * best) {
                best = cost;
                c.blocks_x = bx;
            }
        }
    }
    c.waves = static_cast<double>(c.blocks_x * grid_y) / static_cast<double>(wave);
    return c;
}

}  // namespace vk::plan
