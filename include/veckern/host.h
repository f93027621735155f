/*
 * host.h — C API of libveckern_cpu.so, the host-side tools around the GPU search: seeded synthetic data, the
 * PQ codec (k-means training, encoding), recall evaluation and the CPU search path. They build the search
 * path's inputs, score its outputs and time the CPU beside the GPU (the C++ interfaces are veckern/io.hpp,
 * veckern/pq.hpp, veckern/eval.hpp and veckern/cpu_ref.hpp); the GPU search is veckern.h. Status codes: 0 on success, 2 on error with vkh_last_error() set.
 */
#ifndef VECKERN_HOST_H
#define VECKERN_HOST_H

#include <stddef.h>
#include <stdint.h>

#include "veckern/veckern.h"

#ifdef __cplusplus
extern "C" {
#endif

const char* vkh_last_error(void);
int vkh_max_threads(void);

/* Philox4x32-10 on a raw 128-bit counter and 64-bit key (exposed for known-answer tests). */
void vkh_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);

/* Rows first .. first+count-1 of the Gaussian mixture (veckern::GaussianMixture). out: count x d. */
int vkh_gaussian_mixture(size_t d, size_t components, float sigma, uint64_t seed, size_t first, size_t count,
                         float* out);
/* Rows of the latent-structure source (veckern::SyntheticSource). */
int vkh_synthetic_source(size_t d, size_t clusters, uint64_t seed, size_t latent_dim, size_t first, size_t count,
                         float* out);
/* Gaussian blobs (veckern::synthetic_clustered). out: n x d. */
int vkh_synthetic_clustered(size_t n, size_t d, size_t clusters, uint64_t seed, float* out);
/* Uniform PQ codes, rows first .. first+n-1 (veckern::uniform_codes). out: n x m. */
int vkh_uniform_codes(size_t first, size_t n, size_t m, uint64_t seed, uint8_t* out);
/* N(0, 1) values first .. first+count-1 of stream `stream` (veckern::normal_values). */
int vkh_normal_values(uint64_t seed, uint32_t stream, size_t first, size_t count, float* out);

/* ProductQuantizer(d, m).train(x, n, iters, seed); writes the [m][256][d/m] codebook. */
int vkh_pq_train(const float* x, size_t n, size_t d, size_t m, size_t iters, uint64_t seed, float* centroids);
/* Nearest-centroid codes for x (n x d) under the given codebook. codes: n x m. */
int vkh_pq_encode(const float* centroids, size_t d, size_t m, const float* x, size_t n, uint8_t* codes);
int vkh_pq_decode(const float* centroids, size_t d, size_t m, const uint8_t* codes, size_t n, float* x);

/* The CPU search path (veckern/cpu_ref.hpp) under the given [m][256][d/m] codebook: compute_lut (lut: nq x m x 256),
 * adc_scan (dists: nq x n), select_topk (rows of n distances, out: nq x k), adc_search (out: nq x k). */
int vkh_compute_lut(const float* centroids, size_t d, size_t m, const float* queries, size_t nq, float* lut);
int vkh_adc_scan(const float* lut, size_t nq, const uint8_t* codes, size_t n, size_t m, float* dists);
int vkh_select_topk(const float* dists, size_t nq, size_t n, size_t k, vk_neighbor* out);
int vkh_adc_search(const float* centroids, size_t d, size_t m, const uint8_t* codes, size_t n, const float* queries,
                   size_t nq, size_t k, vk_neighbor* out);

/* veckern::exact_knn / rerank_exact / recall_at_k. recall returns -1 on error. */
int vkh_exact_knn(const float* base, size_t n, const float* queries, size_t nq, size_t d, size_t k,
                  vk_neighbor* out);
int vkh_rerank_exact(const float* base, size_t d, const float* queries, size_t nq, const vk_neighbor* candidates,
                     size_t r, size_t k, vk_neighbor* out);
double vkh_recall_at_k(const vk_neighbor* found, size_t found_stride, const int32_t* truth, size_t truth_stride,
                       size_t nq, size_t k);

#ifdef __cplusplus
}
#endif

#endif /* VECKERN_HOST_H */
