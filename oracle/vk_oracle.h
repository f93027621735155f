/*
 * vk_oracle — CPU restatement of VecKern's product-quantisation search path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker that the GPU path is compared against. Only the
 * test suite, the smoke check and the CPU-baseline leg of bench.py may load it. The product path never
 * calls it and has no CPU fallback.
 *
 * Every function restates one reference function (paths relative to the reference checkout) and keeps its
 * arithmetic order, so that results are bit-identical:
 *   vko_l2sq            include/veckern/common.hpp:27-34   sequential j, acc += diff * diff, no FMA
 *   vko_less            include/veckern/common.hpp:19-21   total order by (dist, id)
 *   vko_topk_*          include/veckern/cpu_ref.hpp:14-40  bounded max-heap; write() sorts ascending and pads
 *   vko_compute_lut     src/cpu/cpu_ref.cpp:7-14           lut[q][s][c] = l2sq(query sub-vector, centroid)
 *   vko_adc_scan        src/cpu/cpu_ref.cpp:16-27          dist = sum over s = 0..m-1, from 0.f, in order
 *   vko_select_topk     src/cpu/cpu_ref.cpp:29-36          ids are column indices
 *   vko_adc_search      src/cpu/cpu_ref.cpp:38-54          LUT + scan + top-k per query, OpenMP over queries
 *   vko_recall_at_k     src/cpu/cpu_ref.cpp:79-91          mean |found[:k] ∩ set(truth[:k])| / k
 *
 * Pinning (how each function is checked, in tests/test_oracle.py):
 *   - against the reference's own CPU sources compiled into oracle/_ref (bit-exact), when that library is built;
 *   - against the committed golden fixtures in tests/golden/ (written from oracle/_ref);
 *   - against the reference's known-answer tests (tests/test_cpu.cpp:33-46) and invariants
 *     (ADC == exact L2 to the decoded vector, tests/test_cpu.cpp:58-67; staged == fused, :84-94);
 *   - against brute force (full sort of all (dist, id) pairs) and numpy float32 on small inputs.
 * No function is left unpinned.
 *
 * Build flags matter for bit-exactness: -O3 -ffp-contract=off, no -march and no -ffast-math, so that no FMA
 * contraction or reassociation changes the rounding (the reference builds with plain -O3 on x86-64).
 */
#ifndef VK_ORACLE_H
#define VK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VKO_KSUB 256 /* centroids per sub-space: one byte per sub-code (common.hpp:11) */

typedef struct {
    float dist;
    int32_t id; /* -1 marks padding when fewer than k results exist */
} vko_neighbor;

/* Bounded top-k: keeps the k smallest (dist, id) pairs. */
typedef struct {
    size_t k;
    size_t size;
    vko_neighbor* heap; /* max-heap of capacity k */
} vko_topk;

int vko_less(float ad, int32_t ai, float bd, int32_t bi);
float vko_l2sq(const float* a, const float* b, size_t d);

int vko_topk_init(vko_topk* t, size_t k);
void vko_topk_free(vko_topk* t);
void vko_topk_push(vko_topk* t, float dist, int32_t id);
/* Writes k results in ascending (dist, id) order, padding with {+inf, -1}; empties the heap. */
void vko_topk_write(vko_topk* t, vko_neighbor* out);

/* centroids: [m][256][dsub] floats, dsub = d / m. queries: nq x d. lut: nq x m x 256. */
void vko_compute_lut(const float* centroids, size_t d, size_t m, const float* queries, size_t nq, float* lut);
/* codes: row-major n x m bytes. dists: nq x n. */
void vko_adc_scan(const float* lut, size_t nq, const uint8_t* codes, size_t n, size_t m, float* dists);
/* Top-k of each row of an nq x n matrix; ids are column indices. out: nq x k. */
void vko_select_topk(const float* dists, size_t nq, size_t n, size_t k, vko_neighbor* out);
/* LUT + scan + selection per query without the nq x n matrix. out: nq x k. Returns 0, or -1 on bad input. */
int vko_adc_search(const float* centroids, size_t d, size_t m, const uint8_t* codes, size_t n, const float* queries,
                   size_t nq, size_t k, vko_neighbor* out);
/* Returns -1.0 when k exceeds either stride (the reference throws there). */
double vko_recall_at_k(const vko_neighbor* found, size_t found_stride, const int32_t* truth, size_t truth_stride,
                       size_t nq, size_t k);
/* Pushes (dists[j], ids[j]) for j < count into a top-k of size k and writes its k results (test helper for the
 * TopK known-answer tests, cpu_ref.hpp:14-40). */
void vko_topk_run(const float* dists, const int32_t* ids, size_t count, size_t k, vko_neighbor* out);
/* Threads the OpenMP loops above will use. */
int vko_max_threads(void);

#ifdef __cplusplus
}
#endif

#endif /* VK_ORACLE_H */
