/*
 * veckern.h — C ABI of the MI355X (gfx950) PQ search library, libveckern.so.
 *
 * Plain C: pointers, sizes and integer status codes; no HIP, CUDA or C++ types. The C++ API of the reference
 * (include/veckern/gpu.hpp: veckern::gpu::PQSearcher, ScanVariant, Tuning, DeviceInfo, Timings, LaunchShape)
 * is implemented on top of these entry points by libveckern_gpu.so, and other languages bind them directly.
 * Each declaration names the reference interface it replaces (paths relative to the reference checkout).
 *
 * Status: every int-returning call returns VK_OK or an error code; vk_last_error() then holds a message for
 * the calling thread. The C++ layer rethrows VK_ERR_INVALID_ARGUMENT as std::invalid_argument, VK_ERR_LOGIC as
 * std::logic_error and the others as std::runtime_error, the exception types the reference throws.
 *
 * Threading: a searcher owns one HIP stream and device buffers; calls on one searcher must not overlap.
 * Every search call is synchronous. Results are deterministic.
 */
#ifndef VECKERN_H
#define VECKERN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VK_ABI_VERSION 1

enum vk_status {
    VK_OK = 0,
    VK_ERR_INVALID_ARGUMENT = 1, /* std::invalid_argument in the reference (searcher.cu:83, 89) */
    VK_ERR_RUNTIME = 2,          /* std::runtime_error from check() (common.hpp:23-25) */
    VK_ERR_LOGIC = 3,            /* std::logic_error (searcher.cu:281) */
    VK_ERR_DEVICE = 4,           /* a HIP runtime call failed (the reference's VK_CUDA_CHECK, searcher.cu:11-16) */
    VK_ERR_OUT_OF_MEMORY = 5     /* device allocation failed */
};

/* Scan variants: values and order of veckern::gpu::ScanVariant (gpu.hpp:13-23), plus one of this build's own:
 * VK_V9_FUSED_WARP_F16 is v8 with binary16 LDS tables (each query's fp32 entries scaled by a power of two so the
 * largest lies in [2^14, 2^15), rounded to nearest even; sums in fp32 and scaled back exactly). It is the
 * reference's "lower-precision tables" next step (README.md:219): distances differ from v8's by the table rounding
 * (relative error of order 1e-3), so results can differ from the fp32 path where candidates are that close. */
enum vk_variant {
    VK_V0_GLOBAL_LUT = 0,
    VK_V1_SHARED_LUT = 1,
    VK_V2_SHARED_LUT_VEC = 2,
    VK_V3_INTERLEAVED = 3,
    VK_V4_FUSED = 4,
    VK_V5_FUSED_REG = 5,
    VK_V6_FUSED_VEC = 6,
    VK_V7_FUSED_VEC_MQ = 7,
    VK_V8_FUSED_WARP = 8,
    VK_V9_FUSED_WARP_F16 = 9,
    VK_NUM_VARIANTS = 10
};

/* Same layout as veckern::Neighbor (common.hpp:13-16): ascending (dist, id); padding is {+inf, -1}. */
typedef struct vk_neighbor {
    float dist;
    int32_t id;
} vk_neighbor;

/* veckern::gpu::Tuning (gpu.hpp:29-34); defaults {256, 0, 2, 4}. */
typedef struct vk_tuning {
    int scan_threads;      /* block size of the v0-v3 scans: multiple of 32 in [32, 1024] */
    int blocks_per_query;  /* blocks per query (group) for scans and fused kernels; 0 = automatic */
    int queries_per_block; /* Q for v7/v8: 1, 2, 4 or 8, lowered when the tables do not fit in LDS */
    int vectors_per_step;  /* ILP for v6-v8: 1, 2 or 4 */
} vk_tuning;

/* veckern::gpu::Timings (gpu.hpp:46-50): milliseconds per stage from HIP events, summed over batches. */
typedef struct vk_timings {
    double transfer_ms, lut_ms, scan_ms, select_ms;
} vk_timings;

/* veckern::gpu::PQSearcher::LaunchShape (gpu.hpp:67-73): the shape the last search actually used. */
typedef struct vk_launch_shape {
    int threads, blocks_x, grid_y, queries_per_block, vectors_per_step;
    int blocks_per_sm; /* occupancy-API residency (fused variants) */
    double waves;      /* grid blocks / resident blocks */
} vk_launch_shape;

/* veckern::gpu::DeviceInfo (gpu.hpp:36-43), plus fields the MI355X reports need. */
typedef struct vk_device_info {
    char name[256];
    char arch[64];              /* e.g. "gfx950:sramecc+:xnack-" */
    int sm_count;               /* compute units */
    double peak_bandwidth_gbs;  /* theoretical HBM bandwidth from memory clock and bus width */
    size_t max_smem_per_block;  /* LDS bytes a block may use */
    int clock_khz;
    int warp_size;
    size_t l2_bytes;
    size_t total_mem_bytes;
} vk_device_info;

typedef struct vk_searcher vk_searcher;
typedef struct vk_reranker vk_reranker;
typedef struct vk_ivf vk_ivf;

/* Message of the last failed call on this thread ("" if none). */
const char* vk_last_error(void);
int vk_abi_version(void);

/* gpu.hpp:25 variant_name (names as searcher.cu:123-136), e.g. "v8_fused_warp"; "unknown" when out of range. */
const char* vk_variant_name(int variant);
/* gpu.hpp:26 is_fused (searcher.cu:138-141): 1 for v4-v9, 0 otherwise (v4 is rejected before launch). */
int vk_is_fused(int variant);
/* Whether a variant needs m % 16 == 0 (bench_main.cpp:184-187; searcher.cu:243-246). */
int vk_needs_m16(int variant);

/* Host-only helpers (no device needed). */
/* Tuning defaults of gpu.hpp:29-34. */
void vk_tuning_default(vk_tuning* out);
/* PQSearcher::set_tuning validation (searcher.cu:450-460): VK_OK or VK_ERR_RUNTIME with the reason. */
int vk_tuning_validate(const vk_tuning* t);
/* The list length K used for k (searcher.cu:86-90): smallest of 8, 16, 32, 64, 128 that is >= k;
 * 0 with VK_ERR_INVALID_ARGUMENT when k > 128. */
int vk_dispatched_k(size_t k);

/* gpu.hpp:42 device_info(int device) (searcher.cu:143-156). */
int vk_get_device_count(int* count);
int vk_get_device_info(int device, vk_device_info* out);

/* gpu.hpp:55 PQSearcher(pq, codes, n) (searcher.cu:427-444). centroids: [m][256][d/m] floats (pq.hpp:20-24);
 * codes: row-major n x m bytes. Both are copied to the current device once; no host pointer is kept.
 * Errors: d, m invalid or n == 0 or n >= INT32_MAX (VK_ERR_RUNTIME). */
int vk_searcher_create(const float* centroids, size_t d, size_t m, const uint8_t* codes, size_t n,
                       vk_searcher** out);
/* gpu.hpp:56 ~PQSearcher. Accepts NULL. */
void vk_searcher_destroy(vk_searcher* s);
/* gpu.hpp:63-64 set_tuning / tuning. */
int vk_searcher_set_tuning(vk_searcher* s, const vk_tuning* t);
int vk_searcher_get_tuning(const vk_searcher* s, vk_tuning* out);
/* gpu.hpp:74 last_launch. */
int vk_searcher_last_launch(const vk_searcher* s, vk_launch_shape* out);
/* The v8/v9 code layout. ids[ids_count] receives, for each slot of the searcher's n padded to a multiple of 256
 * (ids_count must be that padded size), the id of the vector scanned there, interleaved by four 64-slot tiles
 * (ids[(tile / 4) * 256 + lane * 4 + tile % 4] for slot = tile * 64 + lane; padding slots hold 0). rows[rows_count]
 * (rows_count must be m * 256; rows may be NULL with rows_count 0) receives the LDS table row of each code value
 * (rows[s * 256 + c]): the layout stores rows in place of codes and the scan writes the entry of code c at row
 * rows[s * 256 + c]. *lanes (may be NULL) receives the lanes per table-read pass the layout was built for: the
 * first v8/v9 search builds it for its own reads (16 for 16-byte entries, 32 for 8-byte, 64 for 4-byte), a call
 * before any such search for 16. Built on the GPU. No counterpart in the reference (whose layouts keep vector order
 * and codes); for tests and tools that inspect the layout. Errors: m % 16 != 0 or a count that does not match
 * (VK_ERR_INVALID_ARGUMENT). */
int vk_searcher_layout(vk_searcher* s, uint32_t* ids, size_t ids_count, uint8_t* rows, size_t rows_count, int* lanes);

/* gpu.hpp:61 search (searcher.cu:466-520): out[nq * k] host memory, ascending (dist, id) per query, padded
 * {+inf, -1}. Errors: k not in [1, min(128, n)] (VK_ERR_RUNTIME), m % 16 != 0 for v2/v6/v7/v8 or tables that
 * do not fit in LDS (VK_ERR_RUNTIME). timings may be NULL. nq == 0 is a no-op. */
int vk_search(vk_searcher* s, const float* queries, size_t nq, size_t k, int variant, vk_neighbor* out,
              vk_timings* timings);
/* gpu.hpp:62 distances (searcher.cu:522-547): out[nq * n] host memory of ADC distances; v0-v3 only
 * (VK_ERR_RUNTIME for fused variants, as check() in the reference). */
int vk_distances(vk_searcher* s, const float* queries, size_t nq, int variant, float* out, vk_timings* timings);

/* Device-resident search: same as vk_search, but d_queries (nq x d floats) and d_out (nq x k vk_neighbor) are
 * device pointers on the searcher's device, so no PCIe transfer is made or timed (transfer_ms = 0). This is the
 * entry a caller whose data already lives in HBM uses. No counterpart in the reference, which always copies
 * queries in and results out. */
int vk_search_device(vk_searcher* s, const float* d_queries, size_t nq, size_t k, int variant, vk_neighbor* d_out,
                     vk_timings* timings);

/* Allocation-free device-resident search. No counterpart in the reference: it is for callers that cannot allocate
 * device memory during a search (tight serving loops, harnesses that forbid hipMalloc). It launches on the
 * searcher's own stream and waits for that stream before returning, so it cannot be recorded into a caller's HIP
 * graph.
 * Same arguments, results and errors as vk_search_device for v8_fused_warp and v9_fused_warp_f16 (other variants:
 * VK_ERR_INVALID_ARGUMENT), but the partial lists and slab counters live in a static device array of
 * VK_NOALLOC_SCRATCH_BYTES that the library holds on each device it runs on until the process ends (the first
 * VK_NOALLOC_COUNTER_BYTES for the counters, one 4-byte counter per slab of queries_per_block queries; the rest for
 * the partial lists), so the call makes no device allocation, creates no events and records no timings. A search
 * needing more than that (very large nq x k) is rejected before any launch with VK_ERR_INVALID_ARGUMENT; split it
 * into smaller calls. The searcher's sorted code layout (v8 and v9) must already exist: one vk_search or
 * vk_search_device call with v8 or v9 builds it (that call allocates); otherwise VK_ERR_LOGIC. Calls on one device
 * share its array: the library serialises them within a process (a per-device lock held until the call's stream
 * has finished), and overlapping calls would otherwise race on it. Synchronous, like vk_search_device. */
#define VK_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
#define VK_NOALLOC_COUNTER_BYTES ((size_t)64 << 10)
int vk_search_device_noalloc(vk_searcher* s, const float* d_queries, size_t nq, size_t k, int variant,
                             vk_neighbor* d_out);

/* Exact re-ranking on the GPU: replaces rerank_exact (cpu_ref.hpp:55-56, cpu_ref.cpp:66-77), the step after the
 * search that bench --rerank R runs (bench_main.cpp:145-153). The reference re-ranks on the CPU from host arrays;
 * here the n x d base vectors are copied to the current device once by vk_reranker_create, and each call scores
 * the candidates of nq queries: for every candidate id in [0, n) the squared L2 distance summed in dimension order
 * (bit-identical to the reference's l2sq), then the k smallest by (dist, id), padded {+inf, -1}. Candidate ids < 0
 * are skipped, as in the reference; an id >= n is an error (VK_ERR_INVALID_ARGUMENT; the reference would read out
 * of bounds) and that candidate is never read. k must be in [1, 128]. Timings: transfer_ms (host entry point)
 * and scan_ms (the re-rank kernel). */
int vk_reranker_create(const float* base, size_t n, size_t d, vk_reranker** out);
void vk_reranker_destroy(vk_reranker* r);
/* Host buffers: queries nq x d, candidates nq x r, out nq x k. */
int vk_rerank(vk_reranker* r, const float* queries, size_t nq, const vk_neighbor* candidates, size_t r_per_query,
              size_t k, vk_neighbor* out, vk_timings* timings);
/* Device pointers on the re-ranker's device (for instance the output of vk_search_device). */
int vk_rerank_device(vk_reranker* r, const float* d_queries, size_t nq, const vk_neighbor* d_candidates,
                     size_t r_per_query, size_t k, vk_neighbor* d_out, vk_timings* timings);

/* Inverted-file (IVF) PQ search: the reference's "IVF coarse partitioning" next step (README.md:219), which it
 * does not implement. The index holds nlist coarse centroids (nlist x d), the PQ codebook ([m][256][d/m]) and the
 * PQ codes of the n base vectors (row-major n x m, codes of the raw vectors, not residuals) grouped by
 * list_ids[i] (each in [0, nlist), e.g. the nearest coarse centroid). A search takes, per query, the nprobe lists
 * whose coarse centroids are nearest (exact squared L2, ties to the lower list id) and returns the k best vectors
 * of those lists by (ADC distance, id), padded {+inf, -1}: the exhaustive search (vk_search) restricted to the
 * probed lists, with bit-identical distances. m % 16 == 0; nprobe in [1, min(128, nlist)]; k in [1, min(128, n)].
 * Timings: lut_ms = coarse probe, table and plan kernels, scan_ms = list scan, select_ms = merge, transfer_ms =
 * host copies of queries and results (none for vk_ivf_search_device). */
int vk_ivf_create(const float* coarse, size_t nlist, const float* centroids, size_t d, size_t m, const uint8_t* codes,
                  const int32_t* list_ids, size_t n, vk_ivf** out);
void vk_ivf_destroy(vk_ivf* index);
/* Index building helper: list_ids[i] = the coarse centroid nearest to x_i (exact squared L2, the lower index on
 * ties; 0 if every distance is NaN). coarse: nlist x d, x: n x d host buffers. */
int vk_ivf_assign(const float* coarse, size_t nlist, size_t d, const float* x, size_t n, int32_t* list_ids);
/* The IVF scan takes one query per slab (a query's probed lists are scanned as one run); the tuning is validated
 * and kept, and no field of it changes the launch. */
int vk_ivf_set_tuning(vk_ivf* index, const vk_tuning* t);
int vk_ivf_last_launch(const vk_ivf* index, vk_launch_shape* out);
int vk_ivf_search(vk_ivf* index, const float* queries, size_t nq, size_t nprobe, size_t k, vk_neighbor* out,
                  vk_timings* timings);
/* Device-resident IVF search: d_queries (nq x d floats) and d_out (nq x k vk_neighbor) are device pointers on the
 * index's device; no transfer is made or timed. Like vk_search_device, no counterpart in the reference. */
int vk_ivf_search_device(vk_ivf* index, const float* d_queries, size_t nq, size_t nprobe, size_t k,
                         vk_neighbor* d_out, vk_timings* timings);

/* PQ encoding on the GPU: ProductQuantizer::encode (pq.hpp:36, pq.cpp:70-75). codes[i * m + s] is the first
 * c in 0..255 with the smallest l2sq(x_i's sub-vector s, centroids[s][c]) (nearest_centroid, pq.cpp:11-22: a
 * running minimum from FLT_MAX, strict <, dimension order without FMA), so codes are identical to the CPU's.
 * centroids: [m][256][d/m]; x: n x d. Host buffers (x staged in 512 MiB chunks) or device pointers. */
int vk_pq_encode(const float* centroids, size_t d, size_t m, const float* x, size_t n, uint8_t* codes);
int vk_pq_encode_device(const float* d_centroids, size_t d, size_t m, const float* d_x, size_t n, uint8_t* d_codes);
/* The assignment step of k-means training (ProductQuantizer::train, pq.cpp:52-54) for one sub-space: assign[i] =
 * nearest of the 256 centroids (256 x dsub) to sub-vector i (sub: n x dsub). Host buffers. */
int vk_pq_assign(const float* centroids, size_t dsub, const float* sub, size_t n, uint32_t* assign);

#ifdef __cplusplus
}
#endif

#endif /* VECKERN_H */
