#pragma once
// Host-side C++ API of the GPU search (the reference's include/veckern/gpu.hpp, kept name for name). It contains
// no HIP types: veckern::gpu::PQSearcher and the free functions are implemented in libveckern_gpu.so on top of
// the C ABI of libveckern.so (include/veckern/veckern.h), whose status codes become the exception types the
// reference throws (std::invalid_argument, std::logic_error, std::runtime_error).
#include <cstdint>
#include <memory>
#include <string>

#include "veckern/common.hpp"
#include "veckern/pq.hpp"

namespace veckern::gpu {

// Each variant is one step of the reference's optimisation ladder; the values match the C ABI's vk_variant.
enum class ScanVariant {
    GlobalLut,     // v0: LUT read from global memory, row-major codes
    SharedLut,     // v1: LUT staged in LDS
    SharedLutVec,  // v2: + 16-byte row loads (m % 16 == 0)
    Interleaved,   // v3: + wave64-interleaved byte layout
    Fused,         // v4: interleaved scan fused with a per-thread list (rejected before launch in this build)
    FusedReg,      // v5: per-thread list in registers
    FusedVec,      // v6: v5 + 16-byte-word interleaved layout (m % 16 == 0)
    FusedVecMQ,    // v7: v6 + Q queries per block sharing every code load (m % 16 == 0)
    FusedWarp,     // v8: one wave-cooperative list per (wave, query), query-interleaved LDS tables
    FusedWarpF16,  // v9 (not in the reference): v8 with fp16 LDS tables, up to 8 queries per 16-byte read
};

const char* variant_name(ScanVariant v);
bool is_fused(ScanVariant v);

// Launch-shape overrides for parameter sweeps. 0 = use the built-in heuristic.
struct Tuning {
    int scan_threads = 256;      // block size of the v0-v3 scans (multiple of 32, <= 1024)
    int blocks_per_query = 0;    // blocks per query (group) for scans and fused kernels; 0 = auto
    int queries_per_block = 2;   // Q for v7/v8 (1, 2, 4 or 8); v7 also caps Q * K <= 64; LDS caps both
    int vectors_per_step = 4;    // ILP for v6-v8 (1, 2 or 4)
};

struct DeviceInfo {
    std::string name;
    int sm_count = 0;                    // compute units
    double peak_bandwidth_gbs = 0.0;     // theoretical HBM bandwidth
    std::size_t max_smem_per_block = 0;  // LDS bytes per block
};

DeviceInfo device_info(int device = 0);

// Milliseconds per stage, measured with HIP events and summed over query batches.
struct Timings {
    double transfer_ms = 0, lut_ms = 0, scan_ms = 0, select_ms = 0;
    double kernel_ms() const { return lut_ms + scan_ms + select_ms; }
    double total_ms() const { return transfer_ms + kernel_ms(); }
};

class PQSearcher {
public:
    // Copies centroids and codes (row-major n x m) to the device once.
    PQSearcher(const ProductQuantizer& pq, const uint8_t* codes, std::size_t n);
    ~PQSearcher();
    PQSearcher(const PQSearcher&) = delete;
    PQSearcher& operator=(const PQSearcher&) = delete;

    // out: nq x k neighbours, ascending (dist, id). Supports 1 <= k <= min(128, n).
    Timings search(const float* queries, std::size_t nq, std::size_t k, ScanVariant variant, Neighbor* out);
    // out: nq x n ADC distances. Not available for the fused variants.
    Timings distances(const float* queries, std::size_t nq, ScanVariant variant, float* out);

    void set_tuning(const Tuning& tuning);
    const Tuning& tuning() const;
    // The launch shape actually used by the last search (after heuristics and clamping).
    struct LaunchShape {
        int threads = 0, blocks_x = 0, grid_y = 0, queries_per_block = 1, vectors_per_step = 1;
        int blocks_per_sm = 0;  // occupancy-API residency (fused variants)
        double waves = 0.0;     // grid blocks / resident blocks
    };
    LaunchShape last_launch() const;

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

// PQ training and encoding with the nearest-centroid searches on the GPU (not in the reference's gpu.hpp, where
// ProductQuantizer::train / encode run on the CPU). Results are identical to pq.train(x, n, iters, seed) and
// pq.encode(x, n, codes): the kernel keeps nearest_centroid's first-minimum rule and l2sq's arithmetic.
void train(ProductQuantizer& pq, const float* x, std::size_t n, std::size_t iters = 20, uint64_t seed = 1);
void encode(const ProductQuantizer& pq, const float* x, std::size_t n, uint8_t* codes);

// Inverted-file PQ search on the GPU (not in the reference, whose README lists IVF as a next step). coarse: nlist
// x d centroids; codes: n x m PQ codes of the raw vectors (pq's codebook); list_ids[i] in [0, nlist): vector i's
// list (for instance from assign_lists). search() probes each query's nprobe nearest lists (exact distances, lower
// list id on ties) and returns the k best of their vectors by (ADC distance, id), padded {+inf, -1}. Requires
// m % 16 == 0; nprobe in [1, min(128, nlist)]; k in [1, min(128, n)].
class IVFSearcher {
public:
    IVFSearcher(const ProductQuantizer& pq, const float* coarse, std::size_t nlist, const uint8_t* codes,
                const int32_t* list_ids, std::size_t n);
    ~IVFSearcher();
    IVFSearcher(const IVFSearcher&) = delete;
    IVFSearcher& operator=(const IVFSearcher&) = delete;

    Timings search(const float* queries, std::size_t nq, std::size_t nprobe, std::size_t k, Neighbor* out);
    void set_tuning(const Tuning& tuning);  // validated and kept; the scan takes one query per slab

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

// The nearest of nlist coarse centroids (exact, lower index on ties) for each of the n vectors x (n x d).
void assign_lists(const float* coarse, std::size_t nlist, std::size_t d, const float* x, std::size_t n,
                  int32_t* list_ids);

// Exact re-ranking on the GPU (not in the reference's gpu.hpp: its rerank_exact, cpu_ref.hpp:55-56, runs on the
// CPU). The n x d base vectors are copied to the device once; rerank() takes the same arguments as rerank_exact
// minus the base and returns bit-identical results (ids < 0 skipped; ids >= n throw std::invalid_argument).
class Reranker {
public:
    Reranker(const float* base, std::size_t n, std::size_t d);
    ~Reranker();
    Reranker(const Reranker&) = delete;
    Reranker& operator=(const Reranker&) = delete;

    // candidates: nq x r; out: nq x k, ascending (dist, id), padded {+inf, -1}. 1 <= k <= 128.
    Timings rerank(const float* queries, std::size_t nq, const Neighbor* candidates, std::size_t r, std::size_t k,
                   Neighbor* out);

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

}  // namespace veckern::gpu
