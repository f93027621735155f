/*
 * vk_oracle — CPU restatement of VecKern's PQ search path. TEST INFRASTRUCTURE ONLY: the checker for the GPU
 * path, never part of it. The reference line each function follows is cited in vk_oracle.h and below.
 */
#include "vk_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* common.hpp:19-21 — strict order by (dist, id), so CPU and GPU break distance ties by id. */
int vko_less(float ad, int32_t ai, float bd, int32_t bi) { return ad < bd || (ad == bd && ai < bi); }

/* common.hpp:27-34 — squared L2 with a single accumulator, terms added in index order. */
float vko_l2sq(const float* a, const float* b, size_t d) {
    float acc = 0.f;
    for (size_t j = 0; j < d; ++j) {
        const float diff = a[j] - b[j];
        acc += diff * diff;
    }
    return acc;
}

/* ---- bounded top-k (cpu_ref.hpp:14-40). A binary max-heap under vko_less holds the k best seen so far;
 * the root is the worst of them, so a new pair enters only if it is strictly better than the root. */

static int nb_less(const vko_neighbor* a, const vko_neighbor* b) { return vko_less(a->dist, a->id, b->dist, b->id); }

static void swap_nb(vko_neighbor* a, vko_neighbor* b) {
    const vko_neighbor t = *a;
    *a = *b;
    *b = t;
}

static void sift_down(vko_neighbor* h, size_t size, size_t i) {
    for (;;) {
        const size_t l = 2 * i + 1, r = l + 1;
        size_t big = i;
        if (l < size && nb_less(&h[big], &h[l])) big = l;
        if (r < size && nb_less(&h[big], &h[r])) big = r;
        if (big == i) return;
        swap_nb(&h[i], &h[big]);
        i = big;
    }
}

static void sift_up(vko_neighbor* h, size_t i) {
    while (i > 0) {
        const size_t p = (i - 1) / 2;
        if (!nb_less(&h[p], &h[i])) return;
        swap_nb(&h[p], &h[i]);
        i = p;
    }
}

int vko_topk_init(vko_topk* t, size_t k) {
    t->k = k;
    t->size = 0;
    t->heap = k ? (vko_neighbor*)malloc(k * sizeof(vko_neighbor)) : NULL;
    return (k == 0 || t->heap) ? 0 : -1;
}

void vko_topk_free(vko_topk* t) {
    free(t->heap);
    t->heap = NULL;
    t->size = t->k = 0;
}

void vko_topk_push(vko_topk* t, float dist, int32_t id) {
    const vko_neighbor cand = {dist, id};
    if (t->size < t->k) {
        t->heap[t->size] = cand;
        sift_up(t->heap, t->size);
        ++t->size;
    } else if (t->k > 0 && nb_less(&cand, &t->heap[0])) {
        t->heap[0] = cand;
        sift_down(t->heap, t->size, 0);
    }
}

void vko_topk_write(vko_topk* t, vko_neighbor* out) {
    /* heapsort in place: the root (largest) goes to the end each round, giving ascending order */
    for (size_t end = t->size; end > 1; --end) {
        swap_nb(&t->heap[0], &t->heap[end - 1]);
        sift_down(t->heap, end - 1, 0);
    }
    for (size_t j = 0; j < t->size; ++j) out[j] = t->heap[j];
    for (size_t j = t->size; j < t->k; ++j) {
        out[j].dist = INFINITY;
        out[j].id = -1;
    }
    t->size = 0;
}

/* ---- cpu_ref.cpp:7-14. Centroid (s, c) starts at centroids + (s * 256 + c) * dsub (pq.hpp:20-24). */
void vko_compute_lut(const float* centroids, size_t d, size_t m, const float* queries, size_t nq, float* lut) {
    const size_t dsub = d / m;
#pragma omp parallel for schedule(static)
    for (long long q = 0; q < (long long)nq; ++q)
        for (size_t s = 0; s < m; ++s)
            for (size_t c = 0; c < VKO_KSUB; ++c)
                lut[((size_t)q * m + s) * VKO_KSUB + c] =
                    vko_l2sq(queries + (size_t)q * d + s * dsub, centroids + (s * VKO_KSUB + c) * dsub, dsub);
}

/* ---- cpu_ref.cpp:16-27: the distance of vector i is summed over s = 0..m-1 starting from 0.f. */
void vko_adc_scan(const float* lut, size_t nq, const uint8_t* codes, size_t n, size_t m, float* dists) {
#pragma omp parallel for schedule(static)
    for (long long q = 0; q < (long long)nq; ++q) {
        const float* table = lut + (size_t)q * m * VKO_KSUB;
        for (size_t i = 0; i < n; ++i) {
            const uint8_t* code = codes + i * m;
            float acc = 0.f;
            for (size_t s = 0; s < m; ++s) acc += table[s * VKO_KSUB + code[s]];
            dists[(size_t)q * n + i] = acc;
        }
    }
}

/* ---- cpu_ref.cpp:29-36 */
void vko_select_topk(const float* dists, size_t nq, size_t n, size_t k, vko_neighbor* out) {
#pragma omp parallel for schedule(static)
    for (long long q = 0; q < (long long)nq; ++q) {
        vko_topk top;
        if (vko_topk_init(&top, k) != 0) continue;
        for (size_t i = 0; i < n; ++i) vko_topk_push(&top, dists[(size_t)q * n + i], (int32_t)i);
        vko_topk_write(&top, out + (size_t)q * k);
        vko_topk_free(&top);
    }
}

/* ---- cpu_ref.cpp:38-54: one query at a time (dynamic schedule), its own LUT, sequential scan, heap. */
int vko_adc_search(const float* centroids, size_t d, size_t m, const uint8_t* codes, size_t n, const float* queries,
                   size_t nq, size_t k, vko_neighbor* out) {
    if (m == 0 || d == 0 || d % m != 0) return -1;
    int failed = 0;
#pragma omp parallel for schedule(dynamic)
    for (long long q = 0; q < (long long)nq; ++q) {
        float* lut = (float*)malloc(m * VKO_KSUB * sizeof(float));
        vko_topk top;
        if (!lut || vko_topk_init(&top, k) != 0) {
            free(lut);
            failed = 1;
            continue;
        }
        const float* x = queries + (size_t)q * d;
        const size_t dsub = d / m;
        for (size_t s = 0; s < m; ++s)
            for (size_t c = 0; c < VKO_KSUB; ++c)
                lut[s * VKO_KSUB + c] = vko_l2sq(x + s * dsub, centroids + (s * VKO_KSUB + c) * dsub, dsub);
        for (size_t i = 0; i < n; ++i) {
            const uint8_t* code = codes + i * m;
            float acc = 0.f;
            for (size_t s = 0; s < m; ++s) acc += lut[s * VKO_KSUB + code[s]];
            vko_topk_push(&top, acc, (int32_t)i);
        }
        vko_topk_write(&top, out + (size_t)q * k);
        vko_topk_free(&top);
        free(lut);
    }
    return failed ? -1 : 0;
}

/* ---- IVF: the probe is a top-nprobe over the coarse centroids by (l2sq, list id); the scan of the probed lists is
 * cpu_ref.cpp:38-54's, in id order. */
int vko_ivf_search(const float* coarse, size_t nlist, const float* centroids, size_t d, size_t m, const uint8_t* codes,
                   const int32_t* list_ids, size_t n, const float* queries, size_t nq, size_t nprobe, size_t k,
                   vko_neighbor* out) {
    if (m == 0 || d == 0 || d % m != 0 || nprobe == 0 || nprobe > nlist) return -1;
    int failed = 0;
#pragma omp parallel for schedule(dynamic)
    for (long long q = 0; q < (long long)nq; ++q) {
        const float* x = queries + (size_t)q * d;
        float* lut = (float*)malloc(m * VKO_KSUB * sizeof(float));
        vko_neighbor* probes = (vko_neighbor*)malloc(nprobe * sizeof(vko_neighbor));
        unsigned char* probed = (unsigned char*)calloc(nlist, 1);
        vko_topk near, top;
        int ok_near = 0, ok_top = 0;
        if (lut && probes && probed) {
            ok_near = vko_topk_init(&near, nprobe) == 0;
            ok_top = ok_near && vko_topk_init(&top, k) == 0;
        }
        if (!ok_top) {
            if (ok_near) vko_topk_free(&near);
            free(lut);
            free(probes);
            free(probed);
            failed = 1;
            continue;
        }
        for (size_t l = 0; l < nlist; ++l) vko_topk_push(&near, vko_l2sq(x, coarse + l * d, d), (int32_t)l);
        vko_topk_write(&near, probes);
        for (size_t p = 0; p < nprobe; ++p)
            if (probes[p].id >= 0) probed[probes[p].id] = 1;
        const size_t dsub = d / m;
        for (size_t s = 0; s < m; ++s)
            for (size_t c = 0; c < VKO_KSUB; ++c)
                lut[s * VKO_KSUB + c] = vko_l2sq(x + s * dsub, centroids + (s * VKO_KSUB + c) * dsub, dsub);
        for (size_t i = 0; i < n; ++i) {
            if (!probed[list_ids[i]]) continue;
            const uint8_t* code = codes + i * m;
            float acc = 0.f;
            for (size_t s = 0; s < m; ++s) acc += lut[s * VKO_KSUB + code[s]];
            vko_topk_push(&top, acc, (int32_t)i);
        }
        vko_topk_write(&top, out + (size_t)q * k);
        vko_topk_free(&near);
        vko_topk_free(&top);
        free(lut);
        free(probes);
        free(probed);
    }
    return failed ? -1 : 0;
}

/* ---- pq.cpp:11-22 (nearest_centroid) and 70-75 (encode) */
void vko_pq_encode(const float* centroids, size_t d, size_t m, const float* x, size_t n, uint8_t* codes) {
    const size_t dsub = d / m;
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; ++i)
        for (size_t s = 0; s < m; ++s) {
            const float* sub = x + (size_t)i * d + s * dsub;
            const float* cent = centroids + s * VKO_KSUB * dsub;
            size_t best = 0;
            float best_dist = FLT_MAX;
            for (size_t c = 0; c < VKO_KSUB; ++c) {
                const float dist = vko_l2sq(sub, cent + c * dsub, dsub);
                if (dist < best_dist) {
                    best_dist = dist;
                    best = c;
                }
            }
            codes[(size_t)i * m + s] = (uint8_t)best;
        }
}

/* ---- cpu_ref.cpp:66-77: candidates with a negative id are skipped; the others are re-scored exactly. */
int vko_rerank_exact(const float* base, size_t d, const float* queries, size_t nq, const vko_neighbor* candidates,
                     size_t r, size_t k, vko_neighbor* out) {
    int failed = 0;
#pragma omp parallel for schedule(static)
    for (long long q = 0; q < (long long)nq; ++q) {
        vko_topk top;
        if (vko_topk_init(&top, k) != 0) {
            failed = 1;
            continue;
        }
        for (size_t j = 0; j < r; ++j) {
            const int32_t id = candidates[(size_t)q * r + j].id;
            if (id >= 0) vko_topk_push(&top, vko_l2sq(queries + (size_t)q * d, base + (size_t)id * d, d), id);
        }
        vko_topk_write(&top, out + (size_t)q * k);
        vko_topk_free(&top);
    }
    return failed ? -1 : 0;
}

/* ---- binary16 (IEEE 754-2008): sign bit 15, exponent bits 14-10 (bias 15), fraction bits 9-0. */
static uint32_t f32_bits(float x) {
    uint32_t b;
    memcpy(&b, &x, sizeof b);
    return b;
}

static float f32_from_bits(uint32_t b) {
    float x;
    memcpy(&x, &b, sizeof x);
    return x;
}

uint16_t vko_f32_to_f16(float x) {
    const uint32_t b = f32_bits(x);
    const uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    const uint32_t a = b & 0x7fffffffu;
    if (a >= 0x7f800000u) /* infinity, or NaN with its top fraction bits kept and the quiet bit set */
        return (uint16_t)(sign | 0x7c00u | (a > 0x7f800000u ? 0x0200u | ((a >> 13) & 0x03ffu) : 0u));
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520: rounds past the largest finite, 65504 */
    if (a >= 0x38800000u) { /* normal binary16 (>= 2^-14): drop 13 fraction bits, round to nearest even */
        uint32_t h = ((a >> 23) - 127u + 15u) << 10 | ((a >> 13) & 0x03ffu);
        const uint32_t rest = a & 0x1fffu;
        if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ++h; /* a carry into the exponent is correct */
        return (uint16_t)(sign | h);
    }
    if (a < 0x33000000u) return sign; /* below 2^-25: rounds to zero (2^-25 itself is handled below, to even 0) */
    { /* subnormal binary16: units of 2^-24; the f32 value is mant * 2^(e - 23), e in [-25, -15] */
        const int e = (int)(a >> 23) - 127;
        const uint32_t mant = (a & 0x007fffffu) | 0x00800000u;
        const int drop = -e - 1; /* 14 .. 24 */
        uint32_t h = mant >> drop;
        const uint32_t rest = mant & ((1u << drop) - 1u), half = 1u << (drop - 1);
        if (rest > half || (rest == half && (h & 1u))) ++h;
        return (uint16_t)(sign | h);
    }
}

float vko_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, frac = h & 0x03ffu;
    if (e == 31u) return f32_from_bits(sign | 0x7f800000u | frac << 13);
    if (e != 0u) return f32_from_bits(sign | (e - 15u + 127u) << 23 | frac << 13);
    if (frac == 0u) return f32_from_bits(sign);
    /* subnormal: frac * 2^-24, normalised for f32 */
    int exp = -14;
    uint32_t f = frac;
    while (!(f & 0x0400u)) {
        f <<= 1;
        --exp;
    }
    return f32_from_bits(sign | (uint32_t)(exp + 127) << 23 | (f & 0x03ffu) << 13);
}

void vko_f32_to_f16_array(const float* x, size_t count, uint16_t* out) {
    for (size_t i = 0; i < count; ++i) out[i] = vko_f32_to_f16(x[i]);
}

void vko_f16_to_f32_array(const uint16_t* h, size_t count, float* out) {
    for (size_t i = 0; i < count; ++i) out[i] = vko_f16_to_f32(h[i]);
}

int vko_table_shift(const float* table, size_t count) {
    uint32_t mx = 0;
    for (size_t i = 0; i < count; ++i) {
        const uint32_t b = f32_bits(table[i]);
        if (b > mx) mx = b; /* entries are >= +0, so the bit order is the value order (NaN above +inf) */
    }
    if (mx == 0u || mx >= 0x7f800000u) return 0;
    int e;
    if (mx >= 0x00800000u) {
        e = (int)(mx >> 23) - 127;
    } else { /* subnormal: the position of the highest set bit */
        e = -150;
        for (uint32_t v = mx; v; v >>= 1) ++e;
    }
    return e - 14;
}

int vko_adc_search_f16(const float* centroids, size_t d, size_t m, const uint8_t* codes, size_t n, const float* queries,
                       size_t nq, size_t k, vko_neighbor* out) {
    if (m == 0 || d == 0 || d % m != 0) return -1;
    int failed = 0;
#pragma omp parallel for schedule(dynamic)
    for (long long q = 0; q < (long long)nq; ++q) {
        float* lut = (float*)malloc(m * VKO_KSUB * sizeof(float));
        vko_topk top;
        if (!lut || vko_topk_init(&top, k) != 0) {
            free(lut);
            failed = 1;
            continue;
        }
        vko_compute_lut(centroids, d, m, queries + (size_t)q * d, 1, lut);
        const int shift = vko_table_shift(lut, m * VKO_KSUB);
        for (size_t j = 0; j < m * VKO_KSUB; ++j) lut[j] = vko_f16_to_f32(vko_f32_to_f16(ldexpf(lut[j], -shift)));
        for (size_t i = 0; i < n; ++i) {
            const uint8_t* code = codes + i * m;
            float acc = 0.f;
            for (size_t s = 0; s < m; ++s) acc += lut[s * VKO_KSUB + code[s]];
            vko_topk_push(&top, acc, (int32_t)i);
        }
        vko_neighbor* res = out + (size_t)q * k;
        vko_topk_write(&top, res);
        for (size_t j = 0; j < k; ++j)
            if (res[j].id >= 0) res[j].dist = ldexpf(res[j].dist, shift);
        vko_topk_free(&top);
        free(lut);
    }
    return failed ? -1 : 0;
}

/* ---- cpu_ref.cpp:79-91: truth[:k] is treated as a set; every found id that is in it counts as a hit. */
double vko_recall_at_k(const vko_neighbor* found, size_t found_stride, const int32_t* truth, size_t truth_stride,
                       size_t nq, size_t k) {
    if (k > found_stride || k > truth_stride) return -1.0;
    if (nq == 0 || k == 0) return 0.0;
    double total = 0.0;
    for (size_t q = 0; q < nq; ++q) {
        const int32_t* t = truth + q * truth_stride;
        size_t hits = 0;
        for (size_t j = 0; j < k; ++j) {
            const int32_t id = found[q * found_stride + j].id;
            for (size_t u = 0; u < k; ++u)
                if (t[u] == id) {
                    ++hits;
                    break;
                }
        }
        total += (double)hits / (double)k;
    }
    return total / (double)nq;
}

void vko_topk_run(const float* dists, const int32_t* ids, size_t count, size_t k, vko_neighbor* out) {
    vko_topk top;
    if (vko_topk_init(&top, k) != 0) return;
    for (size_t j = 0; j < count; ++j) vko_topk_push(&top, dists[j], ids[j]);
    vko_topk_write(&top, out);
    vko_topk_free(&top);
}

int vko_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
