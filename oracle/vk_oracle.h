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
 *   vko_rerank_exact    src/cpu/cpu_ref.cpp:66-77          exact l2sq of each candidate id >= 0, top-k
 *   vko_ivf_search      (no reference code: README.md:219 lists IVF as a next step) the exhaustive search of
 *                       cpu_ref.cpp:38-54 restricted to the nprobe lists whose coarse centroids are nearest by
 *                       (l2sq, list id)
 *   vko_pq_encode       src/cpu/pq.cpp:11-22, 70-75        nearest centroid per sub-space: running minimum from
 *                                                           FLT_MAX, strict <, so the first minimum wins
 *
 * The fp16-table search (ScanVariant::FusedWarpF16, this build's own variant; the reference lists lower-precision
 * tables as a next step, README.md:219) is restated on top of the same LUT:
 *   vko_f32_to_f16 / vko_f16_to_f32   IEEE 754 binary16 conversion, round to nearest even (from the format's
 *                                     definition: 1 sign, 5 exponent, 10 fraction bits, subnormals kept)
 *   vko_table_shift     per-query power of two bringing the largest LUT entry into [2^14, 2^15)
 *   vko_adc_search_f16  LUT -> scaled and rounded to binary16 -> the fp32 sequential scan of cpu_ref.cpp:46-49
 *                       -> top-k -> distances scaled back by the power of two
 *
 * Pinning (how each function is checked, in tests/test_oracle.py):
 *   - against the reference's own CPU sources compiled into oracle/_ref (bit-exact), when that library is built;
 *   - against the committed golden fixtures in tests/golden/ (written from oracle/_ref);
 *   - against the reference's known-answer tests (tests/test_cpu.cpp:33-46) and invariants
 *     (ADC == exact L2 to the decoded vector, tests/test_cpu.cpp:58-67; staged == fused, :84-94);
 *   - against brute force (full sort of all (dist, id) pairs) and numpy float32 on small inputs;
 *   - fp16: the conversions against numpy's float16 (every binary16 value, every midpoint between neighbours,
 *     random bit patterns); the search against a numpy restatement, and equal to the fp32 search when every
 *     scaled entry is exactly representable.
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
/* IVF search: coarse nlist x d; list_ids[i] in [0, nlist) is vector i's list; out: nq x k. Returns 0, or -1 on bad
 * input or allocation failure. */
int vko_ivf_search(const float* coarse, size_t nlist, const float* centroids, size_t d, size_t m, const uint8_t* codes,
                   const int32_t* list_ids, size_t n, const float* queries, size_t nq, size_t nprobe, size_t k,
                   vko_neighbor* out);
/* PQ encoding: codes[i * m + s] = nearest of the 256 centroids of sub-space s (centroids [m][256][d/m]). */
void vko_pq_encode(const float* centroids, size_t d, size_t m, const float* x, size_t n, uint8_t* codes);
/* Exact re-ranking: for query q, every candidates[q * r + j] with id >= 0 scored by vko_l2sq against
 * base + id * d, then the k smallest by (dist, id). out: nq x k. Returns 0, or -1 on allocation failure. */
int vko_rerank_exact(const float* base, size_t d, const float* queries, size_t nq, const vko_neighbor* candidates,
                     size_t r, size_t k, vko_neighbor* out);
/* IEEE binary16 bits of x, rounded to nearest even; overflow gives infinity, NaN stays NaN (quiet). */
uint16_t vko_f32_to_f16(float x);
/* The float value of binary16 bits h (exact). */
float vko_f16_to_f32(uint16_t h);
/* Element-wise forms of the two conversions over count values. */
void vko_f32_to_f16_array(const float* x, size_t count, uint16_t* out);
void vko_f16_to_f32_array(const uint16_t* h, size_t count, float* out);
/* Exponent e applied to one query's table (entries scaled by 2^-e): with E = floor(log2(largest entry)),
 * e = E - 14; 0 when the largest entry is 0, infinite or NaN. */
int vko_table_shift(const float* table, size_t count);
/* fp16-table search: per query, the fp32 LUT of vko_compute_lut, each entry scaled by 2^-e and rounded to
 * binary16, the sequential fp32 scan, top-k, and the k distances scaled by 2^e. out: nq x k. */
int vko_adc_search_f16(const float* centroids, size_t d, size_t m, const uint8_t* codes, size_t n, const float* queries,
                       size_t nq, size_t k, vko_neighbor* out);
/* Threads the OpenMP loops above will use. */
int vko_max_threads(void);

#ifdef __cplusplus
}
#endif

#endif /* VK_ORACLE_H */
