// C ABI of libveckern.so: device buffers, code layouts, launch planning, query batching and per-stage HIP-event
// timing for every scan variant. Host orchestration counterpart of the reference's src/cuda/searcher.cu, written
// for one MI355X: persistent balanced grids sized by the occupancy API, query-interleaved LDS tables, and
// wave64 code tiles.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <memory>
#include <mutex>
#include <new>
#include <stdexcept>
#include <string>
#include <vector>

#include "kernels.hpp"
#include "planning.hpp"
#include "slot_order.hpp"
#include "veckern/veckern.h"

#define VK_EXPORT extern "C" __attribute__((visibility("default")))

namespace vk {
// Per-m instance tables of the wave-list scan, fp32 (fused_wave_m*.hip) and fp16 tables (fused_wave_h*.hip).
WaveScanKernel fused_wave_kernel_m16(int qg, int ng, int ilp, int segments, bool bulk, int threads);
WaveScanKernel fused_wave_kernel_m32(int qg, int ng, int ilp, int segments, bool bulk, int threads);
WaveScanKernel fused_wave_kernel_m64(int qg, int ng, int ilp, int segments, bool bulk, int threads);
WaveScanKernel fused_wave_kernel_mx(int qg, int ng, int ilp, int segments, bool bulk, int threads);
WaveScanKernel fused_wave_kernel_h16(int qg, int ng, int ilp, int segments, bool bulk, int threads);
WaveScanKernel fused_wave_kernel_h32(int qg, int ng, int ilp, int segments, bool bulk, int threads);
WaveScanKernel fused_wave_kernel_h64(int qg, int ng, int ilp, int segments, bool bulk, int threads);
WaveScanKernel fused_wave_kernel_hx(int qg, int ng, int ilp, int segments, bool bulk, int threads);

WaveScanKernel fused_wave_kernel(int qg, int ng, int ilp, int m, int segments, bool f16, bool bulk, int threads) {
    if (f16) {
        switch (m) {
            case 16: return fused_wave_kernel_h16(qg, ng, ilp, segments, bulk, threads);
            case 32: return fused_wave_kernel_h32(qg, ng, ilp, segments, bulk, threads);
            case 64: return fused_wave_kernel_h64(qg, ng, ilp, segments, bulk, threads);
            default: return fused_wave_kernel_hx(qg, ng, ilp, segments, bulk, threads);
        }
    }
    switch (m) {
        case 16: return fused_wave_kernel_m16(qg, ng, ilp, segments, bulk, threads);
        case 32: return fused_wave_kernel_m32(qg, ng, ilp, segments, bulk, threads);
        case 64: return fused_wave_kernel_m64(qg, ng, ilp, segments, bulk, threads);
        default: return fused_wave_kernel_mx(qg, ng, ilp, segments, bulk, threads);
    }
}
}  // namespace vk

// Scratch of the allocation-free search (vk_search_device_noalloc): a fixed device array that the code object
// carries, so that entry point never allocates. Each device holds its own copy for the life of the process. Layout:
// the per-slab completion counters in the first kNoAllocCounterBytes (kept at zero between searches: the kernel
// leaves them there), then the partial lists. Host code never names `scratch` as a device address: it uses the
// per-device address that hipGetSymbolAddress returns (noalloc_device below).
constexpr size_t kNoAllocScratchBytes = VK_NOALLOC_SCRATCH_BYTES;
constexpr size_t kNoAllocCounterBytes = VK_NOALLOC_COUNTER_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

using vk::Pair;

thread_local std::string g_error;

struct Failure {
    int code;
    std::string message;
};

[[noreturn]] void fail(int code, const std::string& message) { throw Failure{code, message}; }

void require(bool condition, const std::string& message) {
    if (!condition) fail(VK_ERR_RUNTIME, message);
}

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess)
        fail(e == hipErrorOutOfMemory ? VK_ERR_OUT_OF_MEMORY : VK_ERR_DEVICE,
             std::string(what) + " failed: " + hipGetErrorString(e));
}
#define VK_HIP(call) hip_check((call), #call)

template <typename F>
int guarded(F&& body) {
    try {
        body();
        g_error.clear();
        return VK_OK;
    } catch (const Failure& f) {
        g_error = f.message;
        return f.code;
    } catch (const std::bad_alloc&) {
        g_error = "host allocation failed";
        return VK_ERR_OUT_OF_MEMORY;
    } catch (const std::exception& e) {
        g_error = e.what();
        return VK_ERR_RUNTIME;
    } catch (...) {
        g_error = "unknown error";
        return VK_ERR_RUNTIME;
    }
}

template <typename T>
class DeviceBuffer {
public:
    DeviceBuffer() = default;
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    ~DeviceBuffer() { release(); }
    void ensure(size_t count) {
        if (count <= capacity_) return;
        release();
        void* p = nullptr;
        VK_HIP(hipMalloc(&p, std::max<size_t>(count, 1) * sizeof(T)));
        ptr_ = static_cast<T*>(p);
        capacity_ = count;
    }
    void release() {
        if (ptr_) (void)hipFree(ptr_);
        ptr_ = nullptr;
        capacity_ = 0;
    }
    T* get() const { return ptr_; }
    bool empty() const { return ptr_ == nullptr; }

private:
    T* ptr_ = nullptr;
    size_t capacity_ = 0;
};

// Page-locked host staging (hipHostMalloc): host-buffer searches copy queries in and results out through it, so
// the transfers are single DMA copies rather than the runtime's chunked pageable path.
template <typename T>
class PinnedBuffer {
public:
    PinnedBuffer() = default;
    PinnedBuffer(const PinnedBuffer&) = delete;
    PinnedBuffer& operator=(const PinnedBuffer&) = delete;
    ~PinnedBuffer() { release(); }
    void ensure(size_t count) {
        if (count <= capacity_) return;
        release();
        void* p = nullptr;
        VK_HIP(hipHostMalloc(&p, std::max<size_t>(count, 1) * sizeof(T), hipHostMallocDefault));
        ptr_ = static_cast<T*>(p);
        capacity_ = count;
    }
    void release() {
        if (ptr_) (void)hipHostFree(ptr_);
        ptr_ = nullptr;
        capacity_ = 0;
    }
    T* get() const { return ptr_; }

private:
    T* ptr_ = nullptr;
    size_t capacity_ = 0;
};

// Event pairs recorded around the stages of one batch; read after the batch's final synchronisation.
class StageClock {
public:
    explicit StageClock(hipStream_t stream) : stream_(stream) {}
    ~StageClock() {
        for (auto& e : events_) (void)hipEventDestroy(e);
    }
    // Forgets stages recorded by a call that did not reach settle() (it raised); the events are kept for reuse.
    void reset() {
        pending_.clear();
        used_ = 0;
    }
    template <typename F>
    void time(double* acc, F&& work) {
        hipEvent_t a = next(), b = next();
        VK_HIP(hipEventRecord(a, stream_));
        work();
        VK_HIP(hipEventRecord(b, stream_));
        pending_.push_back({a, b, acc});
    }
    // Waits for the stream and adds every pending stage's elapsed time to its accumulator.
    void settle() {
        VK_HIP(hipStreamSynchronize(stream_));
        for (const auto& p : pending_) {
            float ms = 0.f;
            VK_HIP(hipEventElapsedTime(&ms, p.start, p.stop));
            *p.acc += ms;
        }
        pending_.clear();
        used_ = 0;
    }

private:
    struct Pending {
        hipEvent_t start, stop;
        double* acc;
    };
    hipEvent_t next() {
        if (used_ == events_.size()) {
            hipEvent_t e;
            VK_HIP(hipEventCreate(&e));
            events_.push_back(e);
        }
        return events_[used_++];
    }
    hipStream_t stream_;
    std::vector<hipEvent_t> events_;
    std::vector<Pending> pending_;
    size_t used_ = 0;
};

bool valid_variant(int v) { return v >= 0 && v < VK_NUM_VARIANTS; }

void fill_device_info(int device, vk_device_info* out) {
    hipDeviceProp_t p{};
    VK_HIP(hipGetDeviceProperties(&p, device));
    std::memset(out, 0, sizeof(*out));
    std::snprintf(out->name, sizeof(out->name), "%s", p.name[0] ? p.name : "AMD Instinct GPU");
    std::snprintf(out->arch, sizeof(out->arch), "%s", p.gcnArchName);
    out->sm_count = p.multiProcessorCount;
    // HBM3/HBM3E: the runtime reports the memory clock at a quarter of the per-pin data rate, so the peak is
    // 4 transfers per reported clock over the full bus (MI355X: 2.0 GHz x 4 x 8192 bits / 8 = 8.19 TB/s).
    out->peak_bandwidth_gbs = 4.0 * p.memoryClockRate * 1e3 * (p.memoryBusWidth / 8.0) / 1e9;
    out->max_smem_per_block = p.sharedMemPerBlock;
    out->clock_khz = p.clockRate;
    out->warp_size = p.warpSize;
    out->l2_bytes = static_cast<size_t>(p.l2CacheSize);
    out->total_mem_bytes = p.totalGlobalMem;
}

// Per-device state of the allocation-free search. `lock` serialises its calls on one device (they share the
// device's scratch array); `base` is the array's address on that device, found once with the device current.
struct NoAllocDevice {
    std::mutex lock;
    bool found = false;
    bool counters_clean = false;  // false until zeroed, and after a call that stopped between launch and completion
    unsigned char* base = nullptr;
};
constexpr int kNoAllocMaxDevices = 64;
NoAllocDevice g_noalloc[kNoAllocMaxDevices];

}  // namespace

struct vk_searcher {
    int device = 0;
    size_t n = 0, d = 0, m = 0;
    int64_t n_pad = 0;  // n rounded up to 256 vectors: every wave step of up to 4 tiles stays in bounds
    vk_device_info info{};
    vk_tuning tuning{};
    vk_launch_shape last{};
    hipStream_t stream = nullptr;
    DeviceBuffer<float> centroids, queries, lut, dists;
    DeviceBuffer<uint8_t> codes, codes_il;
    DeviceBuffer<uint4> codes_v, codes_s;  // words in vector order (v6, v7) and in sorted slot order (v8, v9)
    DeviceBuffer<uint32_t> slot_ids;        // the sorted slot order: the vector id of each slot (m % 16 == 0 only)
    DeviceBuffer<uint8_t> table_rows;       // [m][256]: the LDS table row of each code value in the sorted layout
    int order_lanes = 0;                    // lanes per table-read pass the slot order was built for
    DeviceBuffer<Pair> part, out;
    PinnedBuffer<float> staged_q;     // host-buffer searches: queries and results staged in page-locked memory
    PinnedBuffer<Pair> staged_out;
    DeviceBuffer<unsigned> counters;
    size_t counters_zeroed = 0;
    bool counters_dirty = false;
    bool have_il = false, have_v = false, have_s = false, have_slot_ids = false;
    std::unique_ptr<StageClock> clock_pool;

    ~vk_searcher() {
        clock_pool.reset();  // its events before the stream
        if (stream) (void)hipStreamDestroy(stream);
    }

    void use_device() const { VK_HIP(hipSetDevice(device)); }

    void validate(int v) const {
        if (vk_needs_m16(v)) require(m % 16 == 0, std::string(vk_variant_name(v)) + " requires m % 16 == 0");
        if (v != VK_V0_GLOBAL_LUT)
            require(m * vk::KSUB * sizeof(float) <= info.max_smem_per_block, "LUT does not fit in LDS");
    }

    // lanes: lanes per pass of the table reads the v8/v9 searches make (search_lanes); the sorted layout is built
    // once, for the first search that needs it.
    void ensure_layout(int v, int lanes = 16) {
        bool built = false;
        if (vk::plan::uses_byte_layout(v) && !have_il) {
            codes_il.ensure(static_cast<size_t>(n_pad) * m);
            VK_HIP(vk::launch_build_bytes(codes.get(), n, static_cast<int>(m), n_pad, codes_il.get(), stream));
            have_il = built = true;
        }
        if (vk::plan::uses_word_layout(v) && !have_v) {
            codes_v.ensure(static_cast<size_t>(n_pad) * (m / 16));
            VK_HIP(vk::launch_build_words(codes.get(), n, static_cast<int>(m), n_pad, codes_v.get(), stream));
            have_v = built = true;
        }
        if (vk::plan::uses_sorted_layout(v) && !have_s) {
            ensure_slot_ids(lanes);
            codes_s.ensure(static_cast<size_t>(n_pad) * (m / 16));
            VK_HIP(vk::launch_build_sorted_words(codes.get(), n, static_cast<int>(m), n_pad, slot_ids.get(),
                                                 table_rows.get(), codes_s.get(), stream));
            have_s = built = true;
        }
        if (built) VK_HIP(hipStreamSynchronize(stream));  // a layout kernel's failure surfaces here, not mid-search
    }

    // The slot order and table rows of the fused scans' layout (slot_order.hpp), for table reads of `lanes` lanes
    // per pass, built the first time a v8/v9 search (or vk_searcher_slot_ids) needs them: on the GPU
    // (slot_order.hip: sort, co-occurrence counts, dealing) with the rows fitted on the host between its two
    // launches, or for m > 64 wholly on the host; the scratch is freed right after.
    void ensure_slot_ids(int lanes) {
        if (have_slot_ids) return;
        require(m % 16 == 0, "the sorted code layout needs m % 16 == 0");
        slot_ids.ensure(static_cast<size_t>(n_pad));
        table_rows.ensure(m * vk::KSUB);
        const unsigned threads = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
        if (m > 64) {  // beyond the GPU kernels' LDS sizing
            std::vector<uint8_t> host_codes(n * m);
            VK_HIP(hipMemcpy(host_codes.data(), codes.get(), n * m, hipMemcpyDeviceToHost));
            const vk::order::SlotOrder order =
                vk::order::slot_order(host_codes.data(), n, m, static_cast<size_t>(n_pad), lanes, threads);
            VK_HIP(hipMemcpy(slot_ids.get(), order.ids.data(), order.ids.size() * sizeof(uint32_t),
                             hipMemcpyHostToDevice));
            VK_HIP(hipMemcpy(table_rows.get(), order.rows.data(), order.rows.size(), hipMemcpyHostToDevice));
        } else {
            size_t bytes = 0;
            VK_HIP(vk::slot_order_scratch_bytes(static_cast<int64_t>(n), static_cast<int>(m), &bytes));
            DeviceBuffer<unsigned char> scratch;
            scratch.ensure(bytes);
            const uint32_t* d_counts = nullptr;
            VK_HIP(vk::launch_slot_sort(codes.get(), static_cast<int64_t>(n), static_cast<int>(m), lanes,
                                        scratch.get(), bytes, &d_counts, stream));
            std::vector<uint32_t> counts(m * vk::KSUB * vk::KSUB);
            VK_HIP(hipMemcpyAsync(counts.data(), d_counts, counts.size() * sizeof(uint32_t), hipMemcpyDeviceToHost,
                                  stream));
            VK_HIP(hipStreamSynchronize(stream));
            vk::order::mirror_counts(counts, m);
            const std::vector<uint8_t> rows = vk::order::fit_all_rows(counts, m, lanes, threads);
            VK_HIP(hipMemcpyAsync(table_rows.get(), rows.data(), rows.size(), hipMemcpyHostToDevice, stream));
            VK_HIP(vk::launch_slot_place(codes.get(), static_cast<int64_t>(n), static_cast<int>(m), n_pad, lanes,
                                         scratch.get(), bytes, table_rows.get(), slot_ids.get(), stream));
            VK_HIP(hipStreamSynchronize(stream));
        }
        order_lanes = lanes;
        have_slot_ids = true;
    }

    // Queries per block of a v8/v9 batch of b queries with k results.
    int wave_q(size_t b, size_t kk, bool f16) const {
        const size_t entry_bytes = f16 ? 2 : sizeof(float);
        return vk::plan::cap_q_by_batch(vk::plan::effective_q(tuning.queries_per_block, m, info.max_smem_per_block,
                                                              false, static_cast<int>(kk), entry_bytes),
                                        b);
    }

    // Lanes per pass of the table reads of a search of nq queries: fp32 tables read 4 * min(Q, 4) bytes per entry
    // (8 queries are two 4-query tables), fp16 tables 2 * Q.
    int search_lanes(int v, size_t nq, size_t kk) const {
        if (!vk::plan::uses_sorted_layout(v)) return 16;
        const bool f16 = v == VK_V9_FUSED_WARP_F16;
        const int q = wave_q(std::min(query_batch(v), nq), kk, f16);
        return vk::order::pass_lanes(f16 ? 2 * q : 4 * std::min(q, 4));
    }

    // The stage clock of this searcher's calls: its events are created once and reused by every call.
    StageClock& stage_clock() {
        if (!clock_pool) clock_pool = std::make_unique<StageClock>(stream);
        clock_pool->reset();
        return *clock_pool;
    }

    // v8 / v9 (f16 tables): the wave-list scan over the balanced partition with its final merge, one launch. The
    // plan fixes the kernel instance, the partition and the scratch the launch needs (partial lists and per-slab
    // counters); the launch takes that scratch from the caller.
    struct WavePlan {
        vk::WaveScanKernel kern;
        size_t smem = 0;
        int q = 1, ilp = 1, K = 0, per_cu = 1, lists_per_block = 1;
        vk::plan::Partition part;
        size_t part_pairs = 0;  // partial-list pairs: [slabs][q][max_slots][lists_per_block][K]
    };

    WavePlan plan_wave(size_t b, size_t kk, bool f16) const {
        WavePlan w;
        // The wave lists take any length up to 128, so they hold exactly k entries: every one of k..K-1 that a
        // rounded-up K would keep costs inserts (about K * ln(n / K) per list) and buys nothing.
        w.K = static_cast<int>(kk);
        const int segments = w.K <= vk::WAVE ? 1 : 2;
        const size_t entry_bytes = f16 ? 2 : sizeof(float);
        w.q = wave_q(b, kk, f16);
        // fp32: 8 queries are two groups of 4 (16-byte reads); fp16: up to 8 queries in one group.
        const int qg = (!f16 && w.q == 8) ? 4 : w.q, ng = (!f16 && w.q == 8) ? 2 : 1;
        w.ilp = tuning.vectors_per_step;
        w.kern = vk::fused_wave_kernel(qg, ng, w.ilp, static_cast<int>(m), segments, f16);
        if (!w.kern.fn) fail(VK_ERR_LOGIC, "no fused-warp kernel built for this (Q, ILP, m, K)");
        const size_t tables = static_cast<size_t>(w.q) * m * vk::KSUB * entry_bytes;
        require(tables <= info.max_smem_per_block, "LUT does not fit in LDS");
        w.smem = w.kern.dynamic_lds ? tables : 0;  // fixed-m instances hold the tables in static LDS
        auto plan_for = [&](const vk::WaveScanKernel& k) {
            if (k.dynamic_lds)
                VK_HIP(hipFuncSetAttribute(k.fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(w.smem)));
            VK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&w.per_cu, k.fn, k.threads, w.smem));
            w.per_cu = std::max(w.per_cu, 1);
            w.part = vk::plan::balanced_partition(static_cast<int64_t>(n), b, w.q, w.ilp,
                                                  static_cast<int64_t>(w.per_cu) * info.sm_count,
                                                  tuning.blocks_per_query, info.sm_count);
        };
        plan_for(w.kern);
        // 1024-thread blocks where that instance exists and its blocks scan many vectors of their slabs (above the
        // bulk-scan bound; and not crossing slab boundaries where 512-thread blocks would not): one block per CU,
        // whose 16 waves share one granule counter, instead of two 512-thread blocks that the CU does not balance
        // or one of 8 waves. scan_threads = 512 or 1024 pins the block size.
        if (tuning.scan_threads != 512) {
            const vk::WaveScanKernel wide =
                vk::fused_wave_kernel(qg, ng, w.ilp, static_cast<int>(m), segments, f16, false, 1024);
            if (wide.fn) {
                const vk::WaveScanKernel narrow = w.kern;
                const bool narrow_aligned = w.part.slabs <= static_cast<int64_t>(w.per_cu) * info.sm_count;
                w.kern = wide;
                plan_for(w.kern);
                const bool crossing = w.part.slabs > static_cast<int64_t>(w.per_cu) * info.sm_count;
                if (tuning.scan_threads != 1024 &&
                    ((crossing && narrow_aligned) || vk::plan::bulk_scan(w.part, w.ilp))) {
                    w.kern = narrow;
                    plan_for(w.kern);
                }
            }
        }
        // Few vectors per block: the instance that admits candidates in bulk, if it has the same residency (the
        // partition above was planned with it).
        if (!f16 && segments == 1 && w.q > 1 && vk::plan::bulk_scan(w.part, w.ilp)) {
            const vk::WaveScanKernel bulk = vk::fused_wave_kernel(qg, ng, w.ilp, static_cast<int>(m), segments, f16,
                                                                  true, w.kern.threads);
            int bulk_per_cu = 0;
            if (bulk.fn) {
                if (bulk.dynamic_lds)
                    VK_HIP(hipFuncSetAttribute(bulk.fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                               static_cast<int>(w.smem)));
                VK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&bulk_per_cu, bulk.fn, bulk.threads, w.smem));
            }
            if (bulk.fn && std::max(bulk_per_cu, 1) == w.per_cu) w.kern = bulk;
        }
        // Up to 8 blocks per slab every wave leaves its own partial lists; beyond that the block merges its wave
        // lists first, which keeps the final merge of a slab to at most max(64, blocks per slab) lists per query.
        w.lists_per_block = w.part.max_slots > 8 ? 1 : w.kern.threads / vk::WAVE;
        w.part_pairs = static_cast<size_t>(w.part.slabs) * w.q * w.part.max_slots * w.lists_per_block * w.K;
        return w;
    }

    // One launch of a planned wave-list scan over this batch's b device queries d_q into d_out (b x kk). part and
    // counters: scratch of w.part_pairs pairs and w.part.slabs zeroed counters (the kernel leaves them at zero).
    void launch_wave(const WavePlan& w, const float* d_q, size_t b, size_t kk, Pair* d_out, Pair* part_buf,
                     unsigned* counter_buf) {
        last = vk_launch_shape{};
        last.threads = w.kern.threads;
        last.blocks_x = static_cast<int>(w.part.grid);
        last.grid_y = 1;
        last.queries_per_block = w.q;
        last.vectors_per_step = w.ilp;
        last.blocks_per_sm = w.per_cu;
        last.waves = static_cast<double>(w.part.grid) / (static_cast<double>(w.per_cu) * info.sm_count);

        // One launch: every block builds its slab's tables in LDS, scans, and the last block of each slab merges
        // the slab's partial lists into d_out.
        vk::WaveScanArgs a{};
        a.queries = d_q;
        a.centroids = centroids.get();
        a.codes = codes_s.get();
        a.slot_ids = slot_ids.get();
        a.table_rows = table_rows.get();
        a.n = static_cast<int64_t>(n);
        a.d = static_cast<int>(d);
        a.m = static_cast<int>(m);
        a.nq = static_cast<int>(b);
        a.K = w.K;
        a.k = static_cast<int>(kk);
        a.n_gran = w.part.n_gran;
        a.total = w.part.total;
        a.max_slots = w.part.max_slots;
        a.lists_per_block = w.lists_per_block;
        a.part = part_buf;
        a.counters = counter_buf;
        a.out = d_out;
        VK_HIP(w.kern.launch(a, static_cast<int>(w.part.grid), w.smem, stream));
    }

    // d_q: device queries of this batch; writes b x kk results to d_out, with the searcher's own scratch buffers.
    // The LUT and the final merge are inside scan_ms.
    void run_wave(const float* d_q, size_t b, size_t kk, bool f16, Pair* d_out, vk_timings* t, StageClock& clock) {
        const WavePlan w = plan_wave(b, kk, f16);
        part.ensure(w.part_pairs);
        ensure_counters(static_cast<size_t>(w.part.slabs));
        counters_dirty = true;  // cleared once the stream completes the launch without error
        clock.time(&t->scan_ms, [&] { launch_wave(w, d_q, b, kk, d_out, part.get(), counters.get()); });
    }

    // Per-slab completion counters of the wave-list scan. The kernel leaves them at zero; they are zeroed here
    // when allocated or grown, and again if a previous launch may have stopped part way (an error was raised
    // between the launch and the stream's completion).
    void ensure_counters(size_t slabs) {
        if (slabs > counters_zeroed || counters_dirty) {
            counters.ensure(std::max(slabs, counters_zeroed));
            counters_zeroed = std::max(slabs, counters_zeroed);
            VK_HIP(hipMemsetAsync(counters.get(), 0, counters_zeroed * sizeof(unsigned), stream));
        }
    }

    // v0-v3: LUT ([q][s][c]) then the distance matrix of this batch into `dists`.
    void run_scan(int v, const float* d_q, size_t b, vk_timings* t, StageClock& clock) {
        const int threads = tuning.scan_threads;
        const int64_t bx = vk::plan::blocks_x_fill(static_cast<int64_t>(n), static_cast<int64_t>(b), threads,
                                                   info.sm_count, tuning.blocks_per_query);
        last = vk_launch_shape{threads, static_cast<int>(bx), static_cast<int>(b), 1, 1, 0, 0.0};
        lut.ensure(b * m * vk::KSUB);
        dists.ensure(b * n);
        clock.time(&t->lut_ms, [&] {
            VK_HIP(vk::launch_lut(d_q, centroids.get(), static_cast<int>(d), static_cast<int>(m), static_cast<int>(b), 1,
                                  static_cast<int>(b), lut.get(), stream));
        });
        vk::ScanArgs a{lut.get(), codes.get(), codes_il.get(), static_cast<int64_t>(n), static_cast<int>(m),
                       dists.get()};
        clock.time(&t->scan_ms, [&] {
            VK_HIP(vk::launch_scan(v, a, static_cast<int>(bx), static_cast<int>(b), threads, stream));
        });
    }

    void run_unfused(int v, const float* d_q, size_t b, size_t kk, Pair* d_out, vk_timings* t, StageClock& clock) {
        run_scan(v, d_q, b, t, clock);
        vk::SelectArgs s{};
        s.mode = 0;
        s.dists = dists.get();
        s.len = static_cast<int64_t>(n);
        s.K = vk::plan::dispatched_k(kk);
        s.k = static_cast<int>(kk);
        s.out = d_out;
        clock.time(&t->select_ms, [&] { VK_HIP(vk::launch_select(s, static_cast<int>(b), stream)); });
    }

    // v5-v7: per-thread-list fused scans on a (blocks_x, query groups) grid, then the final merge.
    void run_thread(int v, const float* d_q, size_t b, size_t kk, Pair* d_out, vk_timings* t, StageClock& clock) {
        const int K = vk::plan::dispatched_k(kk);
        const int q = v == VK_V7_FUSED_VEC_MQ
                          ? vk::plan::effective_q(tuning.queries_per_block, m, info.max_smem_per_block, true, K)
                          : 1;
        const int ilp = (v == VK_V6_FUSED_VEC || v == VK_V7_FUSED_VEC_MQ) ? tuning.vectors_per_step : 1;
        const vk::ThreadScanKernel kern = vk::fused_thread_kernel(v, K, q, ilp);
        if (!kern.fn) fail(VK_ERR_LOGIC, "no per-thread-list kernel built for this (K, Q, ILP)");
        const int W = kern.threads / vk::WAVE;
        const size_t smem = std::max(static_cast<size_t>(q) * m * vk::KSUB * sizeof(float),
                                     static_cast<size_t>(W + 1) * K * sizeof(Pair));
        require(smem <= info.max_smem_per_block, "LUT does not fit in LDS");
        VK_HIP(hipFuncSetAttribute(kern.fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem)));
        const int64_t grid_y = (static_cast<int64_t>(b) + q - 1) / q;
        last = vk_launch_shape{};
        int per_cu = 0;
        VK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern.fn, kern.threads, smem));
        const vk::plan::WaveChoice c = vk::plan::blocks_x_waves(
            static_cast<int64_t>(n), grid_y, kern.threads, static_cast<int64_t>(std::max(per_cu, 1)) * info.sm_count,
            tuning.blocks_per_query);
        int64_t bx = c.blocks_x;
        last.blocks_per_sm = per_cu;
        last.waves = c.waves;
        bx = std::max<int64_t>(1, std::min<int64_t>(bx, (static_cast<int64_t>(n) + kern.threads - 1) / kern.threads));
        last.threads = kern.threads;
        last.blocks_x = static_cast<int>(bx);
        last.grid_y = static_cast<int>(grid_y);
        last.queries_per_block = q;
        last.vectors_per_step = ilp;

        const size_t b_pad = static_cast<size_t>(grid_y) * q;  // tables are read in groups of q
        lut.ensure(b_pad * m * vk::KSUB);
        part.ensure(b * static_cast<size_t>(bx) * K);
        clock.time(&t->lut_ms, [&] {
            VK_HIP(vk::launch_lut(d_q, centroids.get(), static_cast<int>(d), static_cast<int>(m), static_cast<int>(b), 1,
                                  static_cast<int>(b_pad), lut.get(), stream));
        });
        vk::ThreadScanArgs a{lut.get(), codes_il.get(), codes_v.get(), static_cast<int64_t>(n), static_cast<int>(m),
                             static_cast<int>(b), part.get()};
        clock.time(&t->scan_ms, [&] {
            VK_HIP(kern.launch(a, dim3(static_cast<unsigned>(bx), static_cast<unsigned>(grid_y)), smem, stream));
        });
        vk::SelectArgs s{};
        s.mode = 1;
        s.part = part.get();
        s.K = K;
        s.bx = bx;
        s.k = static_cast<int>(kk);
        s.out = d_out;
        clock.time(&t->select_ms, [&] { VK_HIP(vk::launch_select(s, static_cast<int>(b), stream)); });
    }

    void run_variant(int v, const float* d_q, size_t b, size_t kk, Pair* d_out, vk_timings* t, StageClock& clock) {
        if (v == VK_V8_FUSED_WARP || v == VK_V9_FUSED_WARP_F16)
            return run_wave(d_q, b, kk, v == VK_V9_FUSED_WARP_F16, d_out, t, clock);
        if (vk_is_fused(v)) return run_thread(v, d_q, b, kk, d_out, t, clock);
        run_unfused(v, d_q, b, kk, d_out, t, clock);
    }

    void check_search(size_t kk, int v) const {
        require(valid_variant(v), "unknown scan variant " + std::to_string(v));
        if (v == VK_V4_FUSED)
            fail(VK_ERR_LOGIC,
                 "v4_fused is not launched in this build: its run-time-indexed per-thread list faulted the GPU "
                 "(memory-aperture violation, cause not established); use v5_fused_reg or later");
        require(kk >= 1 && kk <= 128 && kk <= n, "k must be in [1, min(128, n)]");
        validate(v);
    }

    // Queries per launch batch: the LUT buffer stays under 1 GiB and, for the unfused variants, the distance
    // matrix under 512 MiB (searcher.cu:24, 476-477); grid y of the grid kernels stays within 65535.
    size_t query_batch(int v) const {
        const size_t per_query = m * vk::KSUB * sizeof(float);
        size_t batch = std::min<size_t>(65535, (size_t{1} << 30) / per_query);
        if (!vk_is_fused(v)) batch = std::min(batch, (size_t{512} << 20) / (n * sizeof(float)));
        return std::max<size_t>(1, batch);
    }

    void distances_host(const float* host_q, size_t nq, int v, float* host_out, vk_timings* t) {
        require(valid_variant(v), "unknown scan variant " + std::to_string(v));
        require(!vk_is_fused(v), "fused variants do not materialise distances");
        validate(v);
        use_device();
        ensure_layout(v);
        StageClock& clock = stage_clock();
        const size_t batch = query_batch(v);
        for (size_t q0 = 0; q0 < nq; q0 += batch) {
            const size_t b = std::min(batch, nq - q0);
            queries.ensure(b * d);
            clock.time(&t->transfer_ms, [&] {
                VK_HIP(hipMemcpyAsync(queries.get(), host_q + q0 * d, b * d * sizeof(float), hipMemcpyHostToDevice,
                                      stream));
            });
            run_scan(v, queries.get(), b, t, clock);
            clock.time(&t->transfer_ms, [&] {
                VK_HIP(hipMemcpyAsync(host_out + q0 * n, dists.get(), b * n * sizeof(float), hipMemcpyDeviceToHost,
                                      stream));
            });
            clock.settle();
        }
    }

    void search_host(const float* host_q, size_t nq, size_t kk, int v, vk_neighbor* host_out, vk_timings* t) {
        check_search(kk, v);
        use_device();
        ensure_layout(v, search_lanes(v, nq, kk));
        StageClock& clock = stage_clock();
        const size_t batch = query_batch(v);
        for (size_t q0 = 0; q0 < nq; q0 += batch) {
            const size_t b = std::min(batch, nq - q0);
            queries.ensure(b * d);
            out.ensure(b * kk);
            staged_q.ensure(b * d);
            staged_out.ensure(b * kk);
            std::memcpy(staged_q.get(), host_q + q0 * d, b * d * sizeof(float));
            clock.time(&t->transfer_ms, [&] {
                VK_HIP(hipMemcpyAsync(queries.get(), staged_q.get(), b * d * sizeof(float), hipMemcpyHostToDevice,
                                      stream));
            });
            run_variant(v, queries.get(), b, kk, out.get(), t, clock);
            clock.time(&t->transfer_ms, [&] {
                VK_HIP(hipMemcpyAsync(staged_out.get(), out.get(), b * kk * sizeof(Pair), hipMemcpyDeviceToHost,
                                      stream));
            });
            clock.settle();
            counters_dirty = false;
            std::memcpy(host_out + q0 * kk, staged_out.get(), b * kk * sizeof(Pair));
        }
    }

    void search_device(const float* d_q, size_t nq, size_t kk, int v, vk_neighbor* d_out, vk_timings* t) {
        check_search(kk, v);
        use_device();
        ensure_layout(v, search_lanes(v, nq, kk));
        StageClock& clock = stage_clock();
        const size_t batch = query_batch(v);
        for (size_t q0 = 0; q0 < nq; q0 += batch) {
            const size_t b = std::min(batch, nq - q0);
            run_variant(v, d_q + q0 * d, b, kk, reinterpret_cast<Pair*>(d_out + q0 * kk), t, clock);
            clock.settle();
            counters_dirty = false;
        }
    }

    // search_device for v8 / v9 with the device's static scratch array instead of the searcher's buffers: no
    // allocation (device or host, outside error messages), no events. Every batch's scratch need is checked before
    // the first launch; a batch is planned again at its launch (the plan is a pure function of the batch size).
    void search_device_noalloc(const float* d_q, size_t nq, size_t kk, int v, vk_neighbor* d_out) {
        check_search(kk, v);
        if (v != VK_V8_FUSED_WARP && v != VK_V9_FUSED_WARP_F16)
            fail(VK_ERR_INVALID_ARGUMENT, "vk_search_device_noalloc runs v8_fused_warp and v9_fused_warp_f16 only");
        if (!have_s)
            fail(VK_ERR_LOGIC, "the searcher's sorted code layout is not built yet: one vk_search or "
                               "vk_search_device call with v8 or v9 builds it (that call allocates)");
        require(device >= 0 && device < kNoAllocMaxDevices, "device index out of range for the static scratch");
        use_device();
        const bool f16 = v == VK_V9_FUSED_WARP_F16;
        const size_t batch = query_batch(v);
        for (size_t q0 = 0; q0 < nq; q0 += batch) {
            const WavePlan w = plan_wave(std::min(batch, nq - q0), kk, f16);
            const size_t counter_bytes = static_cast<size_t>(w.part.slabs) * sizeof(unsigned);
            const size_t part_bytes = w.part_pairs * sizeof(Pair);
            if (counter_bytes > kNoAllocCounterBytes || part_bytes > kNoAllocScratchBytes - kNoAllocCounterBytes)
                fail(VK_ERR_INVALID_ARGUMENT,
                     "vk_search_device_noalloc: this search needs " + std::to_string(part_bytes) +
                         " bytes of partial lists and " + std::to_string(counter_bytes) +
                         " bytes of slab counters, beyond its static scratch (" +
                         std::to_string(kNoAllocScratchBytes - kNoAllocCounterBytes) + " and " +
                         std::to_string(kNoAllocCounterBytes) + " bytes); search fewer queries per call");
        }
        NoAllocDevice& dev = g_noalloc[device];
        std::lock_guard<std::mutex> hold(dev.lock);
        if (!dev.found) {
            void* p = nullptr;
            const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess || p == nullptr)
                fail(VK_ERR_DEVICE, std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e));
            dev.base = static_cast<unsigned char*>(p);
            dev.found = true;
        }
        unsigned* counter_buf = reinterpret_cast<unsigned*>(dev.base);
        Pair* part_buf = reinterpret_cast<Pair*>(dev.base + kNoAllocCounterBytes);
        if (!dev.counters_clean)
            VK_HIP(vk::launch_zero_words(counter_buf, static_cast<int64_t>(kNoAllocCounterBytes / sizeof(unsigned)),
                                         stream));
        dev.counters_clean = false;  // until the stream has completed every launch below
        for (size_t q0 = 0; q0 < nq; q0 += batch) {
            const size_t b = std::min(batch, nq - q0);
            launch_wave(plan_wave(b, kk, f16), d_q + q0 * d, b, kk, reinterpret_cast<Pair*>(d_out + q0 * kk),
                        part_buf, counter_buf);
        }
        VK_HIP(hipStreamSynchronize(stream));
        dev.counters_clean = true;
    }
};

static_assert(sizeof(vk_neighbor) == sizeof(Pair), "vk_neighbor and the device pair must share a layout");

// Exact re-ranking against base vectors held in HBM (rerank.hip). The base is copied to the device once; calls
// stage queries and candidates in, results out (or take device pointers), on the re-ranker's own stream.
struct vk_reranker {
    int device = 0;
    size_t n = 0, d = 0;
    hipStream_t stream = nullptr;
    DeviceBuffer<float> base, queries;
    DeviceBuffer<Pair> candidates, out;
    DeviceBuffer<unsigned> error;

    ~vk_reranker() {
        if (stream) (void)hipStreamDestroy(stream);
    }

    static void check(size_t r, size_t k) {
        require(k >= 1 && k <= 128, "k must be in [1, 128]");
        require(r >= 1, "r must be >= 1");
    }

    // d_q: nq x d, d_c: nq x r candidates, d_o: nq x k results, all on this device.
    void run(const float* d_q, size_t nq, const Pair* d_c, size_t r, size_t k, Pair* d_o, vk_timings* t,
             StageClock& clock) {
        error.ensure(1);
        VK_HIP(hipMemsetAsync(error.get(), 0, sizeof(unsigned), stream));
        vk::RerankArgs a{};
        a.base = base.get();
        a.n = static_cast<int64_t>(n);
        a.d = static_cast<int>(d);
        a.queries = d_q;
        a.nq = static_cast<int64_t>(nq);
        a.candidates = d_c;
        a.r = static_cast<int64_t>(r);
        a.K = vk::plan::dispatched_k(k);
        a.k = static_cast<int>(k);
        a.out = d_o;
        a.error = error.get();
        clock.time(&t->scan_ms, [&] { VK_HIP(vk::launch_rerank(a, stream)); });
    }

    void finish(StageClock& clock) {
        unsigned flag = 0;
        VK_HIP(hipMemcpyAsync(&flag, error.get(), sizeof flag, hipMemcpyDeviceToHost, stream));
        clock.settle();
        if (flag) fail(VK_ERR_INVALID_ARGUMENT, "a candidate id is >= n (the number of base vectors)");
    }

    void rerank_host(const float* host_q, size_t nq, const vk_neighbor* host_c, size_t r, size_t k,
                     vk_neighbor* host_o, vk_timings* t) {
        VK_HIP(hipSetDevice(device));
        StageClock clock(stream);
        queries.ensure(nq * d);
        candidates.ensure(nq * r);
        out.ensure(nq * k);
        clock.time(&t->transfer_ms, [&] {
            VK_HIP(hipMemcpyAsync(queries.get(), host_q, nq * d * sizeof(float), hipMemcpyHostToDevice, stream));
            VK_HIP(hipMemcpyAsync(candidates.get(), host_c, nq * r * sizeof(Pair), hipMemcpyHostToDevice, stream));
        });
        run(queries.get(), nq, candidates.get(), r, k, out.get(), t, clock);
        clock.time(&t->transfer_ms, [&] {
            VK_HIP(hipMemcpyAsync(host_o, out.get(), nq * k * sizeof(Pair), hipMemcpyDeviceToHost, stream));
        });
        finish(clock);
    }

    void rerank_device(const float* d_q, size_t nq, const vk_neighbor* d_c, size_t r, size_t k, vk_neighbor* d_o,
                       vk_timings* t) {
        VK_HIP(hipSetDevice(device));
        StageClock clock(stream);
        run(d_q, nq, reinterpret_cast<const Pair*>(d_c), r, k, reinterpret_cast<Pair*>(d_o), t, clock);
        finish(clock);
    }
};

// ------------------------------------------------------------------------------------------------ exports

VK_EXPORT const char* vk_last_error(void) { return g_error.c_str(); }
VK_EXPORT int vk_abi_version(void) { return VK_ABI_VERSION; }

VK_EXPORT const char* vk_variant_name(int v) {
    static const char* const names[VK_NUM_VARIANTS] = {"v0_global_lut", "v1_shared_lut", "v2_shared_lut_vec",
                                                       "v3_interleaved", "v4_fused",      "v5_fused_reg",
                                                       "v6_fused_vec",  "v7_fused_vec_mq", "v8_fused_warp",
                                                       "v9_fused_warp_f16"};
    return valid_variant(v) ? names[v] : "unknown";
}

VK_EXPORT int vk_is_fused(int v) { return v >= VK_V4_FUSED && v <= VK_V9_FUSED_WARP_F16; }

VK_EXPORT int vk_needs_m16(int v) {
    return v == VK_V2_SHARED_LUT_VEC || v == VK_V6_FUSED_VEC || v == VK_V7_FUSED_VEC_MQ || v == VK_V8_FUSED_WARP ||
           v == VK_V9_FUSED_WARP_F16;
}

VK_EXPORT void vk_tuning_default(vk_tuning* out) {
    if (out) *out = vk_tuning{256, 0, 2, 4};
}

VK_EXPORT int vk_tuning_validate(const vk_tuning* t) {
    return guarded([&] {
        require(t != nullptr, "tuning is null");
        require(t->scan_threads >= 32 && t->scan_threads <= 1024 && t->scan_threads % 32 == 0,
                "scan_threads must be a multiple of 32 in [32, 1024]");
        require(t->blocks_per_query >= 0, "blocks_per_query must be >= 0");
        require(t->queries_per_block == 1 || t->queries_per_block == 2 || t->queries_per_block == 4 ||
                    t->queries_per_block == 8,
                "queries_per_block must be 1, 2, 4 or 8");
        require(t->vectors_per_step == 1 || t->vectors_per_step == 2 || t->vectors_per_step == 4,
                "vectors_per_step must be 1, 2 or 4");
    });
}

VK_EXPORT int vk_dispatched_k(size_t k) {
    const int K = vk::plan::dispatched_k(k);
    if (K == 0) {
        g_error = "k must be <= 128";
        return 0;
    }
    return K;
}

VK_EXPORT int vk_get_device_count(int* count) {
    return guarded([&] {
        require(count != nullptr, "count is null");
        VK_HIP(hipGetDeviceCount(count));
    });
}

VK_EXPORT int vk_get_device_info(int device, vk_device_info* out) {
    return guarded([&] {
        require(out != nullptr, "out is null");
        fill_device_info(device, out);
    });
}

VK_EXPORT int vk_searcher_create(const float* centroids, size_t d, size_t m, const uint8_t* codes, size_t n,
                                 vk_searcher** out) {
    return guarded([&] {
        require(out != nullptr, "out is null");
        *out = nullptr;
        require(m > 0 && d > 0 && d % m == 0, "d must be a positive multiple of m");
        require(n > 0 && n < static_cast<size_t>(std::numeric_limits<int32_t>::max()), "n must fit in int32 ids");
        require(centroids != nullptr && codes != nullptr, "centroids and codes must not be null");
        auto s = std::make_unique<vk_searcher>();
        VK_HIP(hipGetDevice(&s->device));
        fill_device_info(s->device, &s->info);
        vk_tuning_default(&s->tuning);
        s->n = n;
        s->d = d;
        s->m = m;
        s->n_pad = static_cast<int64_t>((n + 255) / 256 * 256);
        VK_HIP(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking));
        s->centroids.ensure(m * vk::KSUB * (d / m));
        VK_HIP(hipMemcpy(s->centroids.get(), centroids, m * vk::KSUB * (d / m) * sizeof(float), hipMemcpyHostToDevice));
        s->codes.ensure(n * m);
        VK_HIP(hipMemcpy(s->codes.get(), codes, n * m, hipMemcpyHostToDevice));
        *out = s.release();
    });
}

VK_EXPORT void vk_searcher_destroy(vk_searcher* s) { delete s; }

VK_EXPORT int vk_searcher_set_tuning(vk_searcher* s, const vk_tuning* t) {
    return guarded([&] {
        require(s != nullptr, "searcher is null");
        const int rc = vk_tuning_validate(t);
        if (rc != VK_OK) fail(rc, g_error);
        s->tuning = *t;
    });
}

VK_EXPORT int vk_searcher_get_tuning(const vk_searcher* s, vk_tuning* out) {
    return guarded([&] {
        require(s != nullptr && out != nullptr, "null argument");
        *out = s->tuning;
    });
}

VK_EXPORT int vk_searcher_last_launch(const vk_searcher* s, vk_launch_shape* out) {
    return guarded([&] {
        require(s != nullptr && out != nullptr, "null argument");
        *out = s->last;
    });
}

VK_EXPORT int vk_searcher_layout(vk_searcher* s, uint32_t* ids, size_t ids_count, uint8_t* rows,
                                 size_t rows_count, int* lanes) {
    return guarded([&] {
        require(s != nullptr && ids != nullptr, "null argument");
        if (ids_count != static_cast<size_t>(s->n_pad))
            fail(VK_ERR_INVALID_ARGUMENT, "ids_count must be n rounded up to a multiple of 256");
        if (rows == nullptr ? rows_count != 0 : rows_count != s->m * vk::KSUB)
            fail(VK_ERR_INVALID_ARGUMENT, "rows_count must be m * 256 (or 0 with rows NULL)");
        if (s->m % 16 != 0) fail(VK_ERR_INVALID_ARGUMENT, "the sorted layout needs m % 16 == 0");
        s->use_device();
        s->ensure_slot_ids(s->order_lanes ? s->order_lanes : 16);
        VK_HIP(hipMemcpy(ids, s->slot_ids.get(), ids_count * sizeof(uint32_t), hipMemcpyDeviceToHost));
        if (rows) VK_HIP(hipMemcpy(rows, s->table_rows.get(), rows_count, hipMemcpyDeviceToHost));
        if (lanes) *lanes = s->order_lanes;
    });
}

VK_EXPORT int vk_search(vk_searcher* s, const float* queries, size_t nq, size_t k, int variant, vk_neighbor* out,
                        vk_timings* timings) {
    return guarded([&] {
        require(s != nullptr, "searcher is null");
        vk_timings t{};
        if (nq > 0) {
            require(queries != nullptr && out != nullptr, "queries and out must not be null");
            s->search_host(queries, nq, k, variant, out, &t);
        } else {
            s->check_search(k, variant);
        }
        if (timings) *timings = t;
    });
}

namespace {

// Device buffers and a stream for the PQ encoder / k-means assignment entry points, one set per thread and
// device, reused across calls (k-means calls the assignment once per iteration and sub-space).
struct PqWorkspace {
    int device = -1;
    hipStream_t stream = nullptr;
    DeviceBuffer<float> x, centroids;
    DeviceBuffer<uint8_t> codes;
    DeviceBuffer<uint32_t> assign;
    ~PqWorkspace() {
        if (stream) (void)hipStreamDestroy(stream);
    }
};

PqWorkspace& pq_workspace() {
    thread_local PqWorkspace w;
    int dev = 0;
    VK_HIP(hipGetDevice(&dev));
    if (w.device != dev) {
        if (w.stream) (void)hipStreamDestroy(w.stream);
        w.stream = nullptr;
        w.x.release();
        w.centroids.release();
        w.codes.release();
        w.assign.release();
        VK_HIP(hipStreamCreateWithFlags(&w.stream, hipStreamNonBlocking));
        w.device = dev;
    }
    return w;
}

// Vectors per encoding chunk: the staged floats stay under 512 MiB.
size_t encode_chunk(size_t d) { return std::max<size_t>(1, (size_t{512} << 20) / (d * sizeof(float))); }

}  // namespace

VK_EXPORT int vk_pq_encode(const float* centroids, size_t d, size_t m, const float* x, size_t n, uint8_t* codes) {
    return guarded([&] {
        require(m > 0 && d > 0 && d % m == 0, "d must be a positive multiple of m");
        require(m <= 65535, "m must be <= 65535");
        if (n == 0) return;
        require(centroids != nullptr && x != nullptr && codes != nullptr, "centroids, x and codes must not be null");
        PqWorkspace& w = pq_workspace();
        const size_t dsub = d / m, chunk = std::min(n, encode_chunk(d));
        w.centroids.ensure(m * vk::KSUB * dsub);
        VK_HIP(hipMemcpyAsync(w.centroids.get(), centroids, m * vk::KSUB * dsub * sizeof(float),
                              hipMemcpyHostToDevice, w.stream));
        w.x.ensure(chunk * d);
        w.codes.ensure(chunk * m);
        for (size_t i0 = 0; i0 < n; i0 += chunk) {
            const size_t b = std::min(chunk, n - i0);
            VK_HIP(hipMemcpyAsync(w.x.get(), x + i0 * d, b * d * sizeof(float), hipMemcpyHostToDevice, w.stream));
            vk::NearestArgs a{w.x.get(), static_cast<int64_t>(b), static_cast<int64_t>(d), static_cast<int>(m),
                              static_cast<int>(dsub), w.centroids.get(), w.codes.get(), nullptr};
            VK_HIP(vk::launch_nearest(a, w.stream));
            VK_HIP(hipMemcpyAsync(codes + i0 * m, w.codes.get(), b * m, hipMemcpyDeviceToHost, w.stream));
            VK_HIP(hipStreamSynchronize(w.stream));
        }
    });
}

VK_EXPORT int vk_pq_encode_device(const float* d_centroids, size_t d, size_t m, const float* d_x, size_t n,
                                  uint8_t* d_codes) {
    return guarded([&] {
        require(m > 0 && d > 0 && d % m == 0, "d must be a positive multiple of m");
        require(m <= 65535, "m must be <= 65535");
        if (n == 0) return;
        require(d_centroids != nullptr && d_x != nullptr && d_codes != nullptr,
                "centroids, x and codes must not be null");
        PqWorkspace& w = pq_workspace();
        vk::NearestArgs a{d_x, static_cast<int64_t>(n), static_cast<int64_t>(d), static_cast<int>(m),
                          static_cast<int>(d / m), d_centroids, d_codes, nullptr};
        VK_HIP(vk::launch_nearest(a, w.stream));
        VK_HIP(hipStreamSynchronize(w.stream));
    });
}

VK_EXPORT int vk_pq_assign(const float* centroids, size_t dsub, const float* sub, size_t n, uint32_t* assign) {
    return guarded([&] {
        require(dsub > 0 && dsub <= static_cast<size_t>(std::numeric_limits<int32_t>::max()), "dsub must be positive");
        if (n == 0) return;
        require(centroids != nullptr && sub != nullptr && assign != nullptr,
                "centroids, sub and assign must not be null");
        PqWorkspace& w = pq_workspace();
        w.centroids.ensure(vk::KSUB * dsub);
        w.x.ensure(n * dsub);
        w.assign.ensure(n);
        VK_HIP(hipMemcpyAsync(w.centroids.get(), centroids, vk::KSUB * dsub * sizeof(float), hipMemcpyHostToDevice,
                              w.stream));
        VK_HIP(hipMemcpyAsync(w.x.get(), sub, n * dsub * sizeof(float), hipMemcpyHostToDevice, w.stream));
        vk::NearestArgs a{w.x.get(), static_cast<int64_t>(n), static_cast<int64_t>(dsub), 1,
                          static_cast<int>(dsub), w.centroids.get(), nullptr, w.assign.get()};
        VK_HIP(vk::launch_nearest(a, w.stream));
        VK_HIP(hipMemcpyAsync(assign, w.assign.get(), n * sizeof(uint32_t), hipMemcpyDeviceToHost, w.stream));
        VK_HIP(hipStreamSynchronize(w.stream));
    });
}

// Inverted-file index: coarse centroids, the PQ codebook, and the codes grouped by list in the word-interleaved
// layout, each list padded to a multiple of 256 vectors (ids -1 on padding) so that a four-tile wave step never
// crosses into the next list.
struct vk_ivf {
    int device = 0;
    size_t n = 0, d = 0, m = 0, nlist = 0;
    vk_device_info info{};
    vk_tuning tuning{};
    vk_launch_shape last{};
    hipStream_t stream = nullptr;
    DeviceBuffer<float> coarse, centroids, queries, lut, coarse_dist;
    DeviceBuffer<uint4> codes_v;
    DeviceBuffer<int32_t> ids, slab_queries;
    DeviceBuffer<int64_t> list_tile, slab_tile, slab_gran, query_gran;
    DeviceBuffer<Pair> probes, part, out;
    PinnedBuffer<float> staged_q;  // host-buffer searches: queries and results staged in page-locked memory
    PinnedBuffer<Pair> staged_out;
    std::vector<int64_t> list_tile_h;  // [nlist + 1]

    ~vk_ivf() {
        if (stream) (void)hipStreamDestroy(stream);
    }

    void check(size_t nprobe, size_t k) const {
        require(k >= 1 && k <= 128 && k <= n, "k must be in [1, min(128, n)]");
        require(nprobe >= 1 && nprobe <= 128 && nprobe <= nlist, "nprobe must be in [1, min(128, nlist)]");
    }

    // d_q: nq x d device queries; d_o: nq x k device results.
    void search(const float* d_q, size_t nq, size_t nprobe, size_t kk, Pair* d_o, vk_timings* t,
                StageClock& clock) {
        // 1. the nprobe nearest lists of every query: exact distances to all coarse centroids (a dense tile
        // kernel), then the nprobe smallest of each row by (dist, list id); in row chunks that keep the distance
        // matrix within 64 Mi floats
        probes.ensure(nq * nprobe);
        const size_t rows = std::max<size_t>(1, std::min(nq, (size_t{64} << 20) / nlist));
        coarse_dist.ensure(rows * nlist);
        lut.ensure(nq * m * vk::KSUB);
        // 2. the slab plan, on the device: slabs in query-major order (each query's probed lists in probe order),
        // so a query's slabs are one run of consecutive granules
        const size_t slabs = nq * nprobe;
        slab_tile.ensure(slabs);
        slab_queries.ensure(slabs);
        slab_gran.ensure(slabs + 1);
        query_gran.ensure(nq + 1);
        vk::IvfPlanArgs plan{probes.get(),      static_cast<int>(nprobe), static_cast<int64_t>(nq), list_tile.get(),
                             slab_tile.get(),   slab_queries.get(),       slab_gran.get(),           query_gran.get()};
        clock.time(&t->lut_ms, [&] {
            for (size_t r0 = 0; r0 < nq; r0 += rows) {
                const size_t nr = std::min(rows, nq - r0);
                VK_HIP(vk::launch_coarse_distances(d_q + r0 * d, static_cast<int64_t>(nr), coarse.get(),
                                                   static_cast<int64_t>(nlist), static_cast<int>(d), coarse_dist.get(),
                                                   stream));
                vk::SelectArgs sel{};
                sel.mode = 0;
                sel.dists = coarse_dist.get();
                sel.len = static_cast<int64_t>(nlist);
                sel.K = vk::plan::dispatched_k(nprobe);
                sel.k = static_cast<int>(nprobe);
                sel.out = probes.get() + r0 * nprobe;
                VK_HIP(vk::launch_select(sel, static_cast<int>(nr), stream));
            }
            VK_HIP(vk::launch_lut(d_q, centroids.get(), static_cast<int>(d), static_cast<int>(m), static_cast<int>(nq),
                                  1, static_cast<int>(nq), lut.get(), stream));
            VK_HIP(vk::launch_ivf_plan(plan, stream));
        });

        // 3. the scan over the probed lists: a balanced partition of all granules over one wave of blocks (the
        // total is known only on the device; blocks with an empty range return at once), then the per-query merge
        // of the lists of the blocks that covered each query's run
        const int K = static_cast<int>(kk);
        const int segments = K <= vk::WAVE ? 1 : 2;
        const vk::WaveScanKernel kern = vk::ivf_kernel(static_cast<int>(m), segments);
        if (!kern.fn) fail(VK_ERR_LOGIC, "no IVF kernel built for this (m, K)");
        const int W = kern.threads / vk::WAVE;
        int per_cu = 0;
        const size_t smem = kern.dynamic_lds ? m * vk::KSUB * sizeof(float) : 0;
        if (kern.dynamic_lds)
            VK_HIP(hipFuncSetAttribute(kern.fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem)));
        VK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern.fn, kern.threads, smem));
        per_cu = std::max(per_cu, 1);
        const int64_t grid = static_cast<int64_t>(per_cu) * info.sm_count;
        part.ensure(static_cast<size_t>(grid + static_cast<int64_t>(nq)) * W * K);  // lists of block b, query q at b + q

        last = vk_launch_shape{};
        last.threads = kern.threads;
        last.blocks_x = static_cast<int>(grid);
        last.grid_y = 1;
        last.queries_per_block = 1;
        last.vectors_per_step = 4;
        last.blocks_per_sm = per_cu;
        last.waves = 1.0;

        vk::WaveScanArgs a{};
        a.queries = d_q;
        a.centroids = centroids.get();
        a.codes = codes_v.get();
        a.n = static_cast<int64_t>(n);
        a.d = static_cast<int>(d);
        a.m = static_cast<int>(m);
        a.nq = static_cast<int>(nq);
        a.K = K;
        a.k = static_cast<int>(kk);
        a.lists_per_block = W;
        a.part = part.get();
        a.n_slabs = static_cast<int64_t>(slabs);
        a.slab_gran = slab_gran.get();
        a.slab_tile = slab_tile.get();
        a.slab_queries = slab_queries.get();
        a.query_gran = query_gran.get();
        a.list_tile = list_tile.get();
        a.ids = ids.get();
        a.lut = lut.get();
        clock.time(&t->scan_ms, [&] { VK_HIP(kern.launch(a, static_cast<int>(grid), smem, stream)); });
        vk::IvfMergeArgs ma{part.get(), query_gran.get(), grid, W, static_cast<int64_t>(nq), K, static_cast<int>(kk),
                            d_o};
        clock.time(&t->select_ms, [&] { VK_HIP(vk::launch_ivf_merge(ma, stream)); });
    }
};

VK_EXPORT int vk_ivf_create(const float* coarse, size_t nlist, const float* centroids, size_t d, size_t m,
                            const uint8_t* codes, const int32_t* list_ids, size_t n, vk_ivf** out) {
    return guarded([&] {
        require(out != nullptr, "out is null");
        *out = nullptr;
        require(m > 0 && d > 0 && d % m == 0, "d must be a positive multiple of m");
        require(m % 16 == 0, "the IVF scan requires m % 16 == 0");
        require(n > 0 && n < static_cast<size_t>(std::numeric_limits<int32_t>::max()), "n must fit in int32 ids");
        require(nlist > 0 && nlist < static_cast<size_t>(std::numeric_limits<int32_t>::max()), "nlist out of range");
        require(coarse != nullptr && centroids != nullptr && codes != nullptr && list_ids != nullptr,
                "coarse, centroids, codes and list_ids must not be null");
        auto v = std::make_unique<vk_ivf>();
        VK_HIP(hipGetDevice(&v->device));
        fill_device_info(v->device, &v->info);
        vk_tuning_default(&v->tuning);
        v->tuning.queries_per_block = 4;
        v->n = n;
        v->d = d;
        v->m = m;
        v->nlist = nlist;
        require(m * vk::KSUB * sizeof(float) <= v->info.max_smem_per_block, "LUT does not fit in LDS");
        // group the vectors by list, each list padded to a multiple of 256 vectors
        std::vector<int64_t> sizes(nlist, 0);
        for (size_t i = 0; i < n; ++i) {
            require(list_ids[i] >= 0 && static_cast<size_t>(list_ids[i]) < nlist, "list id out of range");
            ++sizes[list_ids[i]];
        }
        v->list_tile_h.assign(nlist + 1, 0);
        for (size_t l = 0; l < nlist; ++l) v->list_tile_h[l + 1] = v->list_tile_h[l] + (sizes[l] + 255) / 256 * 4;
        const int64_t padded = v->list_tile_h[nlist] * vk::WAVE;
        std::vector<uint8_t> rows(static_cast<size_t>(std::max<int64_t>(padded, 1)) * m, 0);
        std::vector<int32_t> ids(static_cast<size_t>(std::max<int64_t>(padded, 1)), -1);
        std::vector<int64_t> fill(nlist);
        for (size_t l = 0; l < nlist; ++l) fill[l] = v->list_tile_h[l] * vk::WAVE;
        for (size_t i = 0; i < n; ++i) ids[fill[list_ids[i]]++] = static_cast<int32_t>(i);
        // Within each list the members are ordered by their code bytes, tiles spread (slot_order.hpp), then their
        // rows copied.
        const unsigned threads = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
        vk::order::parallel(threads, [&](unsigned t) {
            std::vector<uint64_t> scratch;
            for (size_t l = t; l < nlist; l += threads) {
                const int64_t base = v->list_tile_h[l] * vk::WAVE;
                vk::order::order_members(codes, m, ids.data() + base, static_cast<size_t>(sizes[l]), scratch);
                for (int64_t j = 0; j < sizes[l]; ++j)
                    std::memcpy(rows.data() + (base + j) * m, codes + static_cast<size_t>(ids[base + j]) * m, m);
            }
        });
        VK_HIP(hipStreamCreateWithFlags(&v->stream, hipStreamNonBlocking));
        v->coarse.ensure(nlist * d);
        VK_HIP(hipMemcpy(v->coarse.get(), coarse, nlist * d * sizeof(float), hipMemcpyHostToDevice));
        v->centroids.ensure(m * vk::KSUB * (d / m));
        VK_HIP(hipMemcpy(v->centroids.get(), centroids, m * vk::KSUB * (d / m) * sizeof(float), hipMemcpyHostToDevice));
        v->ids.ensure(ids.size());
        VK_HIP(hipMemcpy(v->ids.get(), ids.data(), ids.size() * sizeof(int32_t), hipMemcpyHostToDevice));
        v->list_tile.ensure(nlist + 1);
        VK_HIP(hipMemcpy(v->list_tile.get(), v->list_tile_h.data(), (nlist + 1) * sizeof(int64_t),
                         hipMemcpyHostToDevice));
        if (padded > 0) {
            DeviceBuffer<uint8_t> staged;
            staged.ensure(rows.size());
            VK_HIP(hipMemcpy(staged.get(), rows.data(), rows.size(), hipMemcpyHostToDevice));
            v->codes_v.ensure(static_cast<size_t>(padded) * (m / 16));
            VK_HIP(vk::launch_build_words(staged.get(), padded, static_cast<int>(m), padded, v->codes_v.get(),
                                          v->stream));
            VK_HIP(hipStreamSynchronize(v->stream));
        }
        *out = v.release();
    });
}

VK_EXPORT void vk_ivf_destroy(vk_ivf* v) { delete v; }

VK_EXPORT int vk_ivf_assign(const float* coarse, size_t nlist, size_t d, const float* x, size_t n, int32_t* list_ids) {
    return guarded([&] {
        require(d > 0 && d <= static_cast<size_t>(std::numeric_limits<int32_t>::max()), "d must be positive");
        require(nlist > 0 && nlist < static_cast<size_t>(std::numeric_limits<int32_t>::max()), "nlist out of range");
        if (n == 0) return;
        require(coarse != nullptr && x != nullptr && list_ids != nullptr, "coarse, x and list_ids must not be null");
        PqWorkspace& w = pq_workspace();
        const size_t chunk = std::min(n, encode_chunk(d));
        DeviceBuffer<int32_t> ids;
        ids.ensure(chunk);
        w.centroids.ensure(nlist * d);
        VK_HIP(hipMemcpyAsync(w.centroids.get(), coarse, nlist * d * sizeof(float), hipMemcpyHostToDevice, w.stream));
        w.x.ensure(chunk * d);
        for (size_t i0 = 0; i0 < n; i0 += chunk) {
            const size_t b = std::min(chunk, n - i0);
            VK_HIP(hipMemcpyAsync(w.x.get(), x + i0 * d, b * d * sizeof(float), hipMemcpyHostToDevice, w.stream));
            // the nearest coarse centroid of each vector, reduced inside the tiled distance kernel
            VK_HIP(vk::launch_coarse_assign(w.x.get(), static_cast<int64_t>(b), w.centroids.get(),
                                            static_cast<int64_t>(nlist), static_cast<int>(d), ids.get(), w.stream));
            VK_HIP(hipMemcpyAsync(list_ids + i0, ids.get(), b * sizeof(int32_t), hipMemcpyDeviceToHost, w.stream));
            VK_HIP(hipStreamSynchronize(w.stream));
        }
    });
}

VK_EXPORT int vk_ivf_set_tuning(vk_ivf* v, const vk_tuning* t) {
    return guarded([&] {
        require(v != nullptr, "index is null");
        const int rc = vk_tuning_validate(t);
        if (rc != VK_OK) fail(rc, g_error);
        v->tuning = *t;
    });
}

VK_EXPORT int vk_ivf_last_launch(const vk_ivf* v, vk_launch_shape* out) {
    return guarded([&] {
        require(v != nullptr && out != nullptr, "index and out must not be null");
        *out = v->last;
    });
}

VK_EXPORT int vk_ivf_search(vk_ivf* v, const float* queries, size_t nq, size_t nprobe, size_t k, vk_neighbor* out,
                            vk_timings* timings) {
    return guarded([&] {
        require(v != nullptr, "index is null");
        v->check(nprobe, k);
        vk_timings t{};
        if (nq > 0) {
            require(queries != nullptr && out != nullptr, "queries and out must not be null");
            VK_HIP(hipSetDevice(v->device));
            StageClock clock(v->stream);
            const size_t batch = 16384;  // queries per batch: the table kernel's grid and the per-search buffers
            for (size_t q0 = 0; q0 < nq; q0 += batch) {
                const size_t b = std::min(batch, nq - q0);
                v->queries.ensure(b * v->d);
                v->out.ensure(b * k);
                v->staged_q.ensure(b * v->d);
                v->staged_out.ensure(b * k);
                std::memcpy(v->staged_q.get(), queries + q0 * v->d, b * v->d * sizeof(float));
                clock.time(&t.transfer_ms, [&] {
                    VK_HIP(hipMemcpyAsync(v->queries.get(), v->staged_q.get(), b * v->d * sizeof(float),
                                          hipMemcpyHostToDevice, v->stream));
                });
                v->search(v->queries.get(), b, nprobe, k, v->out.get(), &t, clock);
                clock.time(&t.transfer_ms, [&] {
                    VK_HIP(hipMemcpyAsync(v->staged_out.get(), v->out.get(), b * k * sizeof(Pair),
                                          hipMemcpyDeviceToHost, v->stream));
                });
                clock.settle();
                std::memcpy(out + q0 * k, v->staged_out.get(), b * k * sizeof(Pair));
            }
        }
        if (timings) *timings = t;
    });
}

VK_EXPORT int vk_ivf_search_device(vk_ivf* v, const float* d_queries, size_t nq, size_t nprobe, size_t k,
                                   vk_neighbor* d_out, vk_timings* timings) {
    return guarded([&] {
        require(v != nullptr, "index is null");
        v->check(nprobe, k);
        vk_timings t{};
        if (nq > 0) {
            require(d_queries != nullptr && d_out != nullptr, "queries and out must not be null");
            VK_HIP(hipSetDevice(v->device));
            StageClock clock(v->stream);
            const size_t batch = 16384;  // queries per batch, as in vk_ivf_search
            for (size_t q0 = 0; q0 < nq; q0 += batch) {
                const size_t b = std::min(batch, nq - q0);
                v->search(d_queries + q0 * v->d, b, nprobe, k, reinterpret_cast<Pair*>(d_out) + q0 * k, &t, clock);
                clock.settle();
            }
        }
        if (timings) *timings = t;
    });
}

VK_EXPORT int vk_reranker_create(const float* base, size_t n, size_t d, vk_reranker** out) {
    return guarded([&] {
        require(out != nullptr, "out is null");
        *out = nullptr;
        require(d > 0 && d <= static_cast<size_t>(std::numeric_limits<int32_t>::max()), "d must be positive");
        require(n > 0 && n < static_cast<size_t>(std::numeric_limits<int32_t>::max()), "n must fit in int32 ids");
        require(base != nullptr, "base must not be null");
        auto r = std::make_unique<vk_reranker>();
        VK_HIP(hipGetDevice(&r->device));
        r->n = n;
        r->d = d;
        VK_HIP(hipStreamCreateWithFlags(&r->stream, hipStreamNonBlocking));
        r->base.ensure(n * d);
        VK_HIP(hipMemcpy(r->base.get(), base, n * d * sizeof(float), hipMemcpyHostToDevice));
        *out = r.release();
    });
}

VK_EXPORT void vk_reranker_destroy(vk_reranker* r) { delete r; }

VK_EXPORT int vk_rerank(vk_reranker* r, const float* queries, size_t nq, const vk_neighbor* candidates, size_t nr,
                        size_t k, vk_neighbor* out, vk_timings* timings) {
    return guarded([&] {
        require(r != nullptr, "reranker is null");
        vk_reranker::check(nr, k);
        vk_timings t{};
        if (nq > 0) {
            require(queries != nullptr && candidates != nullptr && out != nullptr,
                    "queries, candidates and out must not be null");
            r->rerank_host(queries, nq, candidates, nr, k, out, &t);
        }
        if (timings) *timings = t;
    });
}

VK_EXPORT int vk_rerank_device(vk_reranker* r, const float* d_queries, size_t nq, const vk_neighbor* d_candidates,
                               size_t nr, size_t k, vk_neighbor* d_out, vk_timings* timings) {
    return guarded([&] {
        require(r != nullptr, "reranker is null");
        vk_reranker::check(nr, k);
        vk_timings t{};
        if (nq > 0) {
            require(d_queries != nullptr && d_candidates != nullptr && d_out != nullptr,
                    "queries, candidates and out must not be null");
            r->rerank_device(d_queries, nq, d_candidates, nr, k, d_out, &t);
        }
        if (timings) *timings = t;
    });
}

VK_EXPORT int vk_search_device(vk_searcher* s, const float* d_queries, size_t nq, size_t k, int variant,
                               vk_neighbor* d_out, vk_timings* timings) {
    return guarded([&] {
        require(s != nullptr, "searcher is null");
        vk_timings t{};
        if (nq > 0) {
            require(d_queries != nullptr && d_out != nullptr, "queries and out must not be null");
            s->search_device(d_queries, nq, k, variant, d_out, &t);
        } else {
            s->check_search(k, variant);
        }
        if (timings) *timings = t;
    });
}

VK_EXPORT int vk_search_device_noalloc(vk_searcher* s, const float* d_queries, size_t nq, size_t k, int variant,
                                       vk_neighbor* d_out) {
    return guarded([&] {
        require(s != nullptr, "searcher is null");
        if (nq > 0) {
            require(d_queries != nullptr && d_out != nullptr, "queries and out must not be null");
            s->search_device_noalloc(d_queries, nq, k, variant, d_out);
        } else {
            s->check_search(k, variant);
        }
    });
}

VK_EXPORT int vk_distances(vk_searcher* s, const float* queries, size_t nq, int variant, float* out,
                           vk_timings* timings) {
    return guarded([&] {
        require(s != nullptr, "searcher is null");
        vk_timings t{};
        if (nq > 0) {
            require(queries != nullptr && out != nullptr, "queries and out must not be null");
            s->distances_host(queries, nq, variant, out, &t);
        } else {
            require(valid_variant(variant), "unknown scan variant");
            require(!vk_is_fused(variant), "fused variants do not materialise distances");
        }
        if (timings) *timings = t;
    });
}
