// veckern::gpu C++ API (include/veckern/gpu.hpp) over the C ABI of libveckern.so. Every call forwards to a vk_*
// entry point and turns its status into the exception type the reference throws for the same condition
// (reference: src/cuda/searcher.cu — check() -> std::runtime_error, k > 128 dispatch -> std::invalid_argument,
// fused variants in the scan path -> std::logic_error).
#include <stdexcept>
#include <string>

#include "veckern/gpu.hpp"
#include "veckern/veckern.h"

namespace veckern::gpu {
namespace {

void rethrow(int status) {
    if (status == VK_OK) return;
    const std::string message = vk_last_error();
    switch (status) {
        case VK_ERR_INVALID_ARGUMENT: throw std::invalid_argument(message);
        case VK_ERR_LOGIC: throw std::logic_error(message);
        default: throw std::runtime_error(message);
    }
}

vk_tuning to_c(const Tuning& t) { return vk_tuning{t.scan_threads, t.blocks_per_query, t.queries_per_block, t.vectors_per_step}; }

Timings from_c(const vk_timings& t) { return Timings{t.transfer_ms, t.lut_ms, t.scan_ms, t.select_ms}; }

static_assert(sizeof(Neighbor) == sizeof(vk_neighbor), "Neighbor and vk_neighbor must share a layout");
static_assert(static_cast<int>(ScanVariant::FusedWarp) == VK_V8_FUSED_WARP, "variant numbering");
static_assert(static_cast<int>(ScanVariant::FusedWarpF16) == VK_V9_FUSED_WARP_F16, "variant numbering");

}  // namespace

const char* variant_name(ScanVariant v) { return vk_variant_name(static_cast<int>(v)); }

bool is_fused(ScanVariant v) { return vk_is_fused(static_cast<int>(v)) != 0; }

DeviceInfo device_info(int device) {
    vk_device_info c{};
    rethrow(vk_get_device_info(device, &c));
    DeviceInfo info;
    info.name = c.name;
    info.sm_count = c.sm_count;
    info.peak_bandwidth_gbs = c.peak_bandwidth_gbs;
    info.max_smem_per_block = c.max_smem_per_block;
    return info;
}

struct PQSearcher::Impl {
    vk_searcher* handle = nullptr;
    Tuning tuning;
    ~Impl() { vk_searcher_destroy(handle); }
};

PQSearcher::PQSearcher(const ProductQuantizer& pq, const uint8_t* codes, std::size_t n)
    : impl_(std::make_unique<Impl>()) {
    rethrow(vk_searcher_create(pq.centroids().data(), pq.d(), pq.m(), codes, n, &impl_->handle));
}

PQSearcher::~PQSearcher() = default;

Timings PQSearcher::search(const float* queries, std::size_t nq, std::size_t k, ScanVariant variant, Neighbor* out) {
    vk_timings t{};
    rethrow(vk_search(impl_->handle, queries, nq, k, static_cast<int>(variant), reinterpret_cast<vk_neighbor*>(out),
                      &t));
    return from_c(t);
}

Timings PQSearcher::distances(const float* queries, std::size_t nq, ScanVariant variant, float* out) {
    vk_timings t{};
    rethrow(vk_distances(impl_->handle, queries, nq, static_cast<int>(variant), out, &t));
    return from_c(t);
}

void PQSearcher::set_tuning(const Tuning& tuning) {
    const vk_tuning c = to_c(tuning);
    rethrow(vk_searcher_set_tuning(impl_->handle, &c));
    impl_->tuning = tuning;
}

const Tuning& PQSearcher::tuning() const { return impl_->tuning; }

namespace {
void assign_on_gpu(const float* sub, std::size_t n, const float* cent, std::size_t dsub, uint32_t* out, void*) {
    rethrow(vk_pq_assign(cent, dsub, sub, n, out));
}
}  // namespace

void train(ProductQuantizer& pq, const float* x, std::size_t n, std::size_t iters, uint64_t seed) {
    pq.train(x, n, iters, seed, &assign_on_gpu, nullptr);
}

void encode(const ProductQuantizer& pq, const float* x, std::size_t n, uint8_t* codes) {
    rethrow(vk_pq_encode(pq.centroids().data(), pq.d(), pq.m(), x, n, codes));
}

struct IVFSearcher::Impl {
    vk_ivf* handle = nullptr;
    ~Impl() { vk_ivf_destroy(handle); }
};

IVFSearcher::IVFSearcher(const ProductQuantizer& pq, const float* coarse, std::size_t nlist, const uint8_t* codes,
                         const int32_t* list_ids, std::size_t n)
    : impl_(std::make_unique<Impl>()) {
    rethrow(vk_ivf_create(coarse, nlist, pq.centroids().data(), pq.d(), pq.m(), codes, list_ids, n, &impl_->handle));
}

IVFSearcher::~IVFSearcher() = default;

Timings IVFSearcher::search(const float* queries, std::size_t nq, std::size_t nprobe, std::size_t k, Neighbor* out) {
    vk_timings t{};
    rethrow(vk_ivf_search(impl_->handle, queries, nq, nprobe, k, reinterpret_cast<vk_neighbor*>(out), &t));
    return from_c(t);
}

void IVFSearcher::set_tuning(const Tuning& tuning) {
    const vk_tuning c = to_c(tuning);
    rethrow(vk_ivf_set_tuning(impl_->handle, &c));
}

void assign_lists(const float* coarse, std::size_t nlist, std::size_t d, const float* x, std::size_t n,
                  int32_t* list_ids) {
    rethrow(vk_ivf_assign(coarse, nlist, d, x, n, list_ids));
}

struct Reranker::Impl {
    vk_reranker* handle = nullptr;
    ~Impl() { vk_reranker_destroy(handle); }
};

Reranker::Reranker(const float* base, std::size_t n, std::size_t d) : impl_(std::make_unique<Impl>()) {
    rethrow(vk_reranker_create(base, n, d, &impl_->handle));
}

Reranker::~Reranker() = default;

Timings Reranker::rerank(const float* queries, std::size_t nq, const Neighbor* candidates, std::size_t r,
                         std::size_t k, Neighbor* out) {
    vk_timings t{};
    rethrow(vk_rerank(impl_->handle, queries, nq, reinterpret_cast<const vk_neighbor*>(candidates), r, k,
                      reinterpret_cast<vk_neighbor*>(out), &t));
    return from_c(t);
}

PQSearcher::LaunchShape PQSearcher::last_launch() const {
    vk_launch_shape c{};
    rethrow(vk_searcher_last_launch(impl_->handle, &c));
    LaunchShape s;
    s.threads = c.threads;
    s.blocks_x = c.blocks_x;
    s.grid_y = c.grid_y;
    s.queries_per_block = c.queries_per_block;
    s.vectors_per_step = c.vectors_per_step;
    s.blocks_per_sm = c.blocks_per_sm;
    s.waves = c.waves;
    return s;
}

}  // namespace veckern::gpu
