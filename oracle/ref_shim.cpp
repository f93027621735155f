// C bindings over the reference's own CPU library (src/cpu/{cpu_ref,pq,io}.cpp, compiled from the reference
// checkout by oracle/Makefile into oracle/_ref/libvkref.so). TEST INFRASTRUCTURE ONLY: the tests use it to pin
// the oracle restatement bit-for-bit against the code it restates, and bench.py may time its adc_search as
// the "reference" CPU baseline. Nothing in the product loads it.
#include <cstring>
#include <exception>
#include <vector>

#include "veckern/cpu_ref.hpp"
#include "veckern/io.hpp"
#include "veckern/pq.hpp"

using veckern::Neighbor;
using veckern::ProductQuantizer;

extern "C" {

struct vkref_pq {
    ProductQuantizer pq;
};

// Returns nullptr when the reference constructor throws (d not a positive multiple of m, pq.cpp:25-28).
vkref_pq* vkref_pq_create(size_t d, size_t m) {
    try {
        return new vkref_pq{ProductQuantizer(d, m)};
    } catch (const std::exception&) {
        return nullptr;
    }
}

void vkref_pq_destroy(vkref_pq* h) { delete h; }

int vkref_pq_train(vkref_pq* h, const float* x, size_t n, size_t iters, uint64_t seed) {
    try {
        h->pq.train(x, n, iters, seed);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

void vkref_pq_encode(const vkref_pq* h, const float* x, size_t n, uint8_t* codes) { h->pq.encode(x, n, codes); }
void vkref_pq_decode(const vkref_pq* h, const uint8_t* codes, size_t n, float* x) { h->pq.decode(codes, n, x); }

void vkref_pq_centroids(const vkref_pq* h, float* out) {
    const auto& c = h->pq.centroids();
    std::memcpy(out, c.data(), c.size() * sizeof(float));
}

void vkref_compute_lut(const vkref_pq* h, const float* queries, size_t nq, float* lut) {
    veckern::compute_lut(h->pq, queries, nq, lut);
}

void vkref_adc_scan(const float* lut, size_t nq, const uint8_t* codes, size_t n, size_t m, float* dists) {
    veckern::adc_scan(lut, nq, codes, n, m, dists);
}

void vkref_select_topk(const float* dists, size_t nq, size_t n, size_t k, Neighbor* out) {
    veckern::select_topk(dists, nq, n, k, out);
}

void vkref_adc_search(const vkref_pq* h, const uint8_t* codes, size_t n, const float* queries, size_t nq, size_t k,
                      Neighbor* out) {
    veckern::adc_search(h->pq, codes, n, queries, nq, k, out);
}

void vkref_exact_knn(const float* base, size_t n, const float* queries, size_t nq, size_t d, size_t k, Neighbor* out) {
    veckern::exact_knn(base, n, queries, nq, d, k, out);
}

void vkref_rerank_exact(const float* base, size_t d, const float* queries, size_t nq, const Neighbor* candidates,
                        size_t r, size_t k, Neighbor* out) {
    veckern::rerank_exact(base, d, queries, nq, candidates, r, k, out);
}

// Returns -1.0 where the reference throws (k larger than a stride).
double vkref_recall_at_k(const Neighbor* found, size_t found_stride, const int32_t* truth, size_t truth_stride,
                         size_t nq, size_t k) {
    try {
        return veckern::recall_at_k(found, found_stride, truth, truth_stride, nq, k);
    } catch (const std::exception&) {
        return -1.0;
    }
}

// Pushes (dists[j], ids[j]) for j < count into a reference TopK(k) and writes its k results.
void vkref_topk_run(const float* dists, const int32_t* ids, size_t count, size_t k, Neighbor* out) {
    veckern::TopK top(k);
    for (size_t j = 0; j < count; ++j) top.push(dists[j], ids[j]);
    top.write(out);
}

void vkref_synthetic_clustered(size_t n, size_t d, size_t clusters, uint64_t seed, float* out) {
    const std::vector<float> v = veckern::synthetic_clustered(n, d, clusters, seed);
    std::memcpy(out, v.data(), v.size() * sizeof(float));
}

}  // extern "C"
