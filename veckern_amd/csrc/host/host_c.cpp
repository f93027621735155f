// C API of libveckern_cpu.so (include/veckern/host.h) over the C++ host tools.
#include "veckern/host.h"

#include <cstring>
#include <exception>
#include <string>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

#include "philox.hpp"
#include "veckern/cpu_ref.hpp"
#include "veckern/eval.hpp"
#include "veckern/io.hpp"
#include "veckern/pq.hpp"

#define VKH_EXPORT extern "C" __attribute__((visibility("default")))

namespace {

thread_local std::string g_error;

template <typename F>
int guarded(F&& body) {
    try {
        body();
        g_error.clear();
        return 0;
    } catch (const std::exception& e) {
        g_error = e.what();
    } catch (...) {
        g_error = "unknown error";
    }
    return 2;
}

veckern::ProductQuantizer make_pq(const float* centroids, size_t d, size_t m) {
    veckern::ProductQuantizer pq(d, m);
    pq.set_centroids(std::vector<float>(centroids, centroids + m * veckern::kSubCentroids * (d / m)));
    return pq;
}

static_assert(sizeof(vk_neighbor) == sizeof(veckern::Neighbor), "vk_neighbor and Neighbor must share a layout");

}  // namespace

VKH_EXPORT const char* vkh_last_error(void) { return g_error.c_str(); }

VKH_EXPORT int vkh_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

VKH_EXPORT void vkh_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    const veckern::rng::Block b = veckern::rng::philox_raw(ctr, key);
    std::memcpy(out, b.v, sizeof(b.v));
}

VKH_EXPORT int vkh_gaussian_mixture(size_t d, size_t components, float sigma, uint64_t seed, size_t first,
                                    size_t count, float* out) {
    return guarded([&] { veckern::GaussianMixture(d, components, sigma, seed).fill(first, count, out); });
}

VKH_EXPORT int vkh_synthetic_source(size_t d, size_t clusters, uint64_t seed, size_t latent_dim, size_t first,
                                    size_t count, float* out) {
    return guarded([&] { veckern::SyntheticSource(d, clusters, seed, latent_dim).fill(first, count, out); });
}

VKH_EXPORT int vkh_synthetic_clustered(size_t n, size_t d, size_t clusters, uint64_t seed, float* out) {
    return guarded([&] {
        const auto v = veckern::synthetic_clustered(n, d, clusters, seed);
        std::memcpy(out, v.data(), v.size() * sizeof(float));
    });
}

VKH_EXPORT int vkh_uniform_codes(size_t first, size_t n, size_t m, uint64_t seed, uint8_t* out) {
    return guarded([&] { veckern::uniform_codes(first, n, m, seed, out); });
}

VKH_EXPORT int vkh_normal_values(uint64_t seed, uint32_t stream, size_t first, size_t count, float* out) {
    return guarded([&] { veckern::normal_values(seed, stream, first, count, out); });
}

VKH_EXPORT int vkh_pq_train(const float* x, size_t n, size_t d, size_t m, size_t iters, uint64_t seed,
                            float* centroids) {
    return guarded([&] {
        veckern::ProductQuantizer pq(d, m);
        pq.train(x, n, iters, seed);
        std::memcpy(centroids, pq.centroids().data(), pq.centroids().size() * sizeof(float));
    });
}

VKH_EXPORT int vkh_pq_encode(const float* centroids, size_t d, size_t m, const float* x, size_t n, uint8_t* codes) {
    return guarded([&] { make_pq(centroids, d, m).encode(x, n, codes); });
}

VKH_EXPORT int vkh_pq_decode(const float* centroids, size_t d, size_t m, const uint8_t* codes, size_t n, float* x) {
    return guarded([&] { make_pq(centroids, d, m).decode(codes, n, x); });
}

VKH_EXPORT int vkh_compute_lut(const float* centroids, size_t d, size_t m, const float* queries, size_t nq,
                               float* lut) {
    return guarded([&] { veckern::compute_lut(make_pq(centroids, d, m), queries, nq, lut); });
}

VKH_EXPORT int vkh_adc_scan(const float* lut, size_t nq, const uint8_t* codes, size_t n, size_t m, float* dists) {
    return guarded([&] { veckern::adc_scan(lut, nq, codes, n, m, dists); });
}

VKH_EXPORT int vkh_select_topk(const float* dists, size_t nq, size_t n, size_t k, vk_neighbor* out) {
    return guarded([&] { veckern::select_topk(dists, nq, n, k, reinterpret_cast<veckern::Neighbor*>(out)); });
}

VKH_EXPORT int vkh_adc_search(const float* centroids, size_t d, size_t m, const uint8_t* codes, size_t n,
                              const float* queries, size_t nq, size_t k, vk_neighbor* out) {
    return guarded([&] {
        veckern::adc_search(make_pq(centroids, d, m), codes, n, queries, nq, k,
                            reinterpret_cast<veckern::Neighbor*>(out));
    });
}

VKH_EXPORT int vkh_exact_knn(const float* base, size_t n, const float* queries, size_t nq, size_t d, size_t k,
                             vk_neighbor* out) {
    return guarded([&] { veckern::exact_knn(base, n, queries, nq, d, k, reinterpret_cast<veckern::Neighbor*>(out)); });
}

VKH_EXPORT int vkh_rerank_exact(const float* base, size_t d, const float* queries, size_t nq,
                                const vk_neighbor* candidates, size_t r, size_t k, vk_neighbor* out) {
    return guarded([&] {
        veckern::rerank_exact(base, d, queries, nq, reinterpret_cast<const veckern::Neighbor*>(candidates), r, k,
                              reinterpret_cast<veckern::Neighbor*>(out));
    });
}

VKH_EXPORT double vkh_recall_at_k(const vk_neighbor* found, size_t found_stride, const int32_t* truth,
                                  size_t truth_stride, size_t nq, size_t k) {
    double r = -1.0;
    const int rc = guarded([&] {
        r = veckern::recall_at_k(reinterpret_cast<const veckern::Neighbor*>(found), found_stride, truth, truth_stride,
                                 nq, k);
    });
    return rc == 0 ? r : -1.0;
}
