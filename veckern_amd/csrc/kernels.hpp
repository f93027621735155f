// Internal launch interface between the C-ABI host layer (capi.hip) and the kernel translation units.
// Nothing here is exported from the shared library.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "device.hpp"

namespace vk {

// ---- LUT build (lut.hip). Writes lut[g][s][c][qg] for groups g of qg consecutive queries; query slots past nq
// are written as 0.f so that padded groups hold defined values. groups >= ceil(nq / qg).
hipError_t launch_lut(const float* queries, const float* centroids, int d, int m, int nq, int qg, int groups,
                      float* lut, hipStream_t stream);

// ---- code layouts (layout.hip). n_pad is a multiple of 64; vectors past n are zero codes.
// Word-interleaved: out[(tile * (m/16) + w) * 64 + lane] = 16 sub-codes 16w..16w+15 of vector tile*64+lane.
hipError_t launch_build_words(const uint8_t* codes, int64_t n, int m, int64_t n_pad, uint4* out, hipStream_t stream);
// The word-interleaved layout in the fused scans' slot order: slot j holds vector slot_ids[j's interleaved
// position], each code byte c of sub-space s replaced by rows[s * 256 + c] (rows == nullptr: c itself); slots
// [n, n_pad) are zero.
hipError_t launch_build_sorted_words(const uint8_t* codes, int64_t n, int m, int64_t n_pad, const uint32_t* slot_ids,
                                     const uint8_t* rows, uint4* out, hipStream_t stream);
// Byte-interleaved: out[(tile * m + s) * 64 + lane] = sub-code s of vector tile*64+lane.
hipError_t launch_build_bytes(const uint8_t* codes, int64_t n, int m, int64_t n_pad, uint8_t* out,
                              hipStream_t stream);
// Zeroes count 32-bit words with a kernel (no memset node).
hipError_t launch_zero_words(unsigned* p, int64_t count, hipStream_t stream);
// The fused scans' slot order and table rows on the GPU (slot_order.hip), equal to order::slot_order of
// slot_order.hpp for m <= 64 and lanes 16, 32 or 64, in two launches around the host's fit of the rows:
// launch_slot_sort sorts the vectors and leaves, in scratch, the co-occurrence counts of the sampled blocks' passes
// (`*counts`: [m][256][256] words, entries [s][a][b] with a < b filled, the rest zero); the host fits the rows
// (order::fit_rows on the mirrored counts) and launch_slot_place, with the same scratch, deals the blocks and writes
// the n_pad interleaved slot ids to `out` (padding slots 0). scratch: slot_order_scratch_bytes(n, m) bytes.
hipError_t slot_order_scratch_bytes(int64_t n, int m, size_t* bytes);
hipError_t launch_slot_sort(const uint8_t* codes, int64_t n, int m, int lanes, void* scratch, size_t scratch_bytes,
                            const uint32_t** counts, hipStream_t stream);
hipError_t launch_slot_place(const uint8_t* codes, int64_t n, int m, int64_t n_pad, int lanes, void* scratch,
                             size_t scratch_bytes, const uint8_t* rows, uint32_t* out, hipStream_t stream);

// ---- fused scan with wave-cooperative lists (fused_wave_*.hip)
struct WaveScanArgs {
    const float* queries;    // nq x d; each block builds its slab's tables from these
    const float* centroids;  // [m][256][d / m]
    const uint4* codes;      // word-interleaved, padded to a multiple of 256 vectors (exhaustive scans: the sorted
                             // layout, slot order given by slot_ids)
    const uint32_t* slot_ids;  // exhaustive scans: per slot, its vector's id, interleaved by four tiles
                               // ([tile / 4][lane][tile % 4])
    const uint8_t* table_rows;  // exhaustive scans: [m][256] LDS table row of each code value (the layout stores
                                // rows, not codes); nullptr: row = code
    int64_t n;
    int d;
    int m;
    int nq;
    int K;                   // list length, <= 64 * S
    int k;                   // results per query
    int64_t n_gran;          // granules (64 * ilp vectors) per slab
    int64_t total;           // slabs * n_gran
    int max_slots;           // blocks per slab, upper bound over slabs
    int lists_per_block;     // partial lists a block writes per (slab, query): one per wave, or 1 (merged in LDS)
    Pair* part;              // [slabs][qg * ng][max_slots][lists_per_block][K]
    unsigned* counters;      // [slabs], zero between searches: blocks of a slab that have finished
    Pair* out;               // [nq][k]; empty slots become {+inf, -1}
    // Inverted lists (IVF instances only, one query per slab, the plan of launch_ivf_plan); `n_gran`, `total` and
    // `max_slots` are then unused (the total is query_gran[nq]).
    int64_t n_slabs;
    const int64_t* slab_gran;      // [n_slabs + 1] granule prefix of the slabs
    const int64_t* slab_tile;      // [n_slabs] first tile in `codes` / `ids` of the list each slab scans
    const int32_t* slab_queries;   // [n_slabs] query of each slab; a query's slabs are consecutive
    const int64_t* query_gran;     // [nq + 1] granule prefix of the queries' runs of slabs
    const int64_t* list_tile;      // [lists + 1] first tile of each list in `codes` / `ids`
    const int32_t* ids;            // [tiles * 64] vector id of each padded position, -1 for padding
    const float* lut;              // [nq][m][256] tables computed once per search (a query meets many lists)
};

struct WaveScanKernel {
    const void* fn = nullptr;  // kernel symbol, for occupancy queries
    int threads = 0;
    bool dynamic_lds = false;  // tables in dynamic LDS (m not fixed at compile time) rather than a static array
    hipError_t (*launch)(const WaveScanArgs&, int grid, size_t smem, hipStream_t) = nullptr;
};

// Returns a kernel with fn == nullptr when the combination is not built. f16: binary16 tables (v9). bulk: the
// instance with bulk admission into one-register lists (fp32, more than one query per block only). threads: block
// size, 512 or 1024 (built for four tiles per wave step where two 512-thread blocks' tables fit one CU).
WaveScanKernel fused_wave_kernel(int qg, int ng, int ilp, int m, int segments, bool f16, bool bulk = false,
                                 int threads = 512);
// The inverted-list scan (ivf_m*.hip): fp32 tables, one query per slab, four tiles per wave step.
WaveScanKernel ivf_kernel(int m, int segments);

// ---- IVF plan (ivf.hip): from the probes (nq x nprobe, id -1 = no list), slab q * nprobe + p = query q's p-th
// probed list: slab_tile (the list's first tile) / slab_queries [nq * nprobe], slab_gran [nq * nprobe + 1] (granule
// starts; a probe of no
// list or of an empty list is an empty slab), query_gran [nq + 1] (the granule start of each query's run; the last
// entry is the total).
struct IvfPlanArgs {
    const Pair* probes;
    int nprobe;
    int64_t nq;
    const int64_t* list_tile;
    int64_t* slab_tile;
    int32_t* slab_queries;
    int64_t* slab_gran;
    int64_t* query_gran;
};
hipError_t launch_ivf_plan(const IvfPlanArgs& a, hipStream_t stream);

// ---- IVF probe (probe.hip): out[q][l] = exact squared L2 distance of query q to coarse centroid l (nq x nlist)
hipError_t launch_coarse_distances(const float* queries, int64_t nq, const float* coarse, int64_t nlist, int d,
                                   float* out, hipStream_t stream);
// list_ids[i] = the nearest coarse centroid of vector i by (exact squared L2 distance, centroid index)
hipError_t launch_coarse_assign(const float* x, int64_t n, const float* coarse, int64_t nlist, int d,
                                int32_t* list_ids, hipStream_t stream);

// ---- IVF final merge (ivf.hip): block b of the scan (grid blocks, lists_per_block lists of K pairs each) writes
// its lists for query q at part[(b + q) * lists_per_block * K]; the k results of q go to out[q * k].
struct IvfMergeArgs {
    const Pair* part;
    const int64_t* query_gran;
    int64_t grid;
    int lists_per_block;
    int64_t nq;
    int K;
    int k;
    Pair* out;
};
hipError_t launch_ivf_merge(const IvfMergeArgs& a, hipStream_t stream);

// Blocks covering slab `slab` in the balanced partition of `total` work items over `grid` blocks
// (block b owns items [b*total/grid, (b+1)*total/grid)).
__host__ __device__ inline int64_t first_block_of(int64_t item, int64_t grid, int64_t total) {
    return ((item + 1) * grid - 1) / total;
}

// ---- unfused scans v0-v3 (scan_thread.hip): dists[q][i] for q < nq, grid (blocks_x, nq)
struct ScanArgs {
    const float* lut;         // [nq][m][256]
    const uint8_t* codes;     // row-major n x m (v0-v2)
    const uint8_t* codes_il;  // byte-interleaved (v3)
    int64_t n;
    int m;
    float* dists;             // [nq][n]
};
hipError_t launch_scan(int variant, const ScanArgs& a, int blocks_x, int nq, int threads, hipStream_t stream);

// ---- fused scans with per-thread lists, v5-v7 (scan_thread.hip): grid (blocks_x, ceil(nq / Q)), 256 threads
struct ThreadScanArgs {
    const float* lut;         // [nq padded to a multiple of Q][m][256]; padded tables are zero
    const uint8_t* codes_il;  // v5
    const uint4* codes_v;     // v6, v7
    int64_t n;
    int m;
    int nq;
    Pair* part;               // [nq][blocks_x][K]
};

struct ThreadScanKernel {
    const void* fn = nullptr;
    int threads = 0;
    hipError_t (*launch)(const ThreadScanArgs&, dim3 grid, size_t smem, hipStream_t) = nullptr;
};

// The instance for a variant (5-7), list length K and the effective Q (v7) and ILP (v6, v7).
ThreadScanKernel fused_thread_kernel(int variant, int K, int q, int ilp);

// ---- selection / final merge (select.hip)
struct SelectArgs {
    int mode;              // 0: rows of distances, ids = column index; 1: grid partials
    const float* dists;    // mode 0: [nq][len]
    int64_t len;
    const Pair* part;      // mode 1
    int K;                 // list length of the selection (and of each partial list)
    int64_t bx;            // mode 1: partial lists per query, layout [q][bx][K]
    int k;                 // results written per query
    Pair* out;             // [nq][k]; empty slots become {+inf, -1}
};
hipError_t launch_select(const SelectArgs& a, int nq, hipStream_t stream);

// ---- exact re-ranking (rerank.hip): one wave per query over its r candidates
struct RerankArgs {
    const float* base;        // n x d, row-major
    int64_t n;
    int d;
    const float* queries;     // nq x d
    int64_t nq;
    const Pair* candidates;   // nq x r; ids < 0 are skipped. Null: candidate j of every query is base row j
    int64_t r;
    int K;                    // list length (dispatched k)
    int k;                    // results per query
    Pair* out;                // nq x k; empty slots become {+inf, -1}
    unsigned* error;          // set to non-zero when a candidate id is >= n (that candidate is not read)
};
hipError_t launch_rerank(const RerankArgs& a, hipStream_t stream);

// ---- nearest-centroid assignment (pq_assign.hip): PQ encoding and the k-means assignment step
struct NearestArgs {
    const float* x;           // n vectors; sub-space s of vector i starts at x + i * x_stride + s * dsub
    int64_t n;
    int64_t x_stride;         // floats between consecutive vectors (d for encoding, dsub for training)
    int m;                    // sub-spaces (grid y)
    int dsub;
    const float* centroids;   // [m][256][dsub]
    uint8_t* codes;           // n x m codes, or null
    uint32_t* assign;         // n indices (m == 1), or null
};
hipError_t launch_nearest(const NearestArgs& a, hipStream_t stream);

}  // namespace vk
