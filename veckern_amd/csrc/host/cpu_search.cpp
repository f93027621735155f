// The CPU search path (include/veckern/cpu_ref.hpp; reference interface cpu_ref.hpp:42-49, behaviour
// cpu_ref.cpp:7-54). It is what veckern_bench times as its "cpu_reference" row, on all host threads.
//
// One query per OpenMP task (dynamic schedule: queries cost the same, but the threads of a shared host do not).
// A task builds its query's table in a thread-local buffer, then scans the codes in chunks: a chunk's distances
// are computed first (each summed over s = 0..m-1 from 0.f, the reference's order, so they are bit-identical),
// and only the ones at or below the current k-th best enter a sorted list of k pairs by insertion. Once the list
// is full almost every candidate is rejected by that one comparison.
#include <algorithm>
#include <limits>
#include <vector>

#include "veckern/cpu_ref.hpp"

namespace veckern {
namespace {

// The k smallest pairs seen so far under the (dist, id) order, ascending; `bound` is the k-th (+inf until full).
class SortedList {
public:
    explicit SortedList(std::size_t k) : k_(k) { items_.reserve(k + 1); }

    float bound() const {
        if (items_.size() < k_) return std::numeric_limits<float>::infinity();
        return k_ == 0 ? -std::numeric_limits<float>::infinity() : items_.back().dist;
    }

    void offer(float dist, int32_t id) {
        const Neighbor cand{dist, id};
        if (items_.size() == k_) {
            if (k_ == 0 || !(cand < items_.back())) return;
            items_.pop_back();
        }
        items_.insert(std::upper_bound(items_.begin(), items_.end(), cand), cand);
    }

    void write(Neighbor* out) const {
        std::copy(items_.begin(), items_.end(), out);
        for (std::size_t j = items_.size(); j < k_; ++j) out[j] = {std::numeric_limits<float>::infinity(), -1};
    }

private:
    std::size_t k_;
    std::vector<Neighbor> items_;
};

// Table of one query: table[s * 256 + c] = l2sq(sub-vector s of x, centroid c of sub-space s).
void query_table(const ProductQuantizer& pq, const float* x, float* table) {
    const std::size_t m = pq.m(), dsub = pq.dsub();
    for (std::size_t s = 0; s < m; ++s)
        for (std::size_t c = 0; c < kSubCentroids; ++c)
            table[s * kSubCentroids + c] = l2sq(x + s * dsub, pq.centroid(s, c), dsub);
}

// dist[i] = sum over s of table[s][code(i)[s]] for `count` consecutive row-major codes, s ascending from 0.f.
void scan_chunk(const float* table, const uint8_t* codes, std::size_t count, std::size_t m, float* dist) {
    for (std::size_t i = 0; i < count; ++i) {
        const uint8_t* code = codes + i * m;
        float acc = 0.f;
        for (std::size_t s = 0; s < m; ++s) acc += table[s * kSubCentroids + code[s]];
        dist[i] = acc;
    }
}

constexpr std::size_t kChunk = 1024;  // vectors per scan chunk: their distances stay in L1

}  // namespace

void compute_lut(const ProductQuantizer& pq, const float* queries, std::size_t nq, float* lut) {
    const std::size_t per_query = pq.m() * kSubCentroids;
#pragma omp parallel for schedule(static)
    for (long long q = 0; q < static_cast<long long>(nq); ++q)
        query_table(pq, queries + static_cast<std::size_t>(q) * pq.d(), lut + static_cast<std::size_t>(q) * per_query);
}

void adc_scan(const float* lut, std::size_t nq, const uint8_t* codes, std::size_t n, std::size_t m, float* dists) {
#pragma omp parallel for schedule(static)
    for (long long q = 0; q < static_cast<long long>(nq); ++q)
        scan_chunk(lut + static_cast<std::size_t>(q) * m * kSubCentroids, codes, n, m,
                   dists + static_cast<std::size_t>(q) * n);
}

void select_topk(const float* dists, std::size_t nq, std::size_t n, std::size_t k, Neighbor* out) {
#pragma omp parallel for schedule(static)
    for (long long q = 0; q < static_cast<long long>(nq); ++q) {
        const float* row = dists + static_cast<std::size_t>(q) * n;
        SortedList list(k);
        for (std::size_t i = 0; i < n; ++i)
            if (row[i] <= list.bound()) list.offer(row[i], static_cast<int32_t>(i));
        list.write(out + static_cast<std::size_t>(q) * k);
    }
}

void adc_search(const ProductQuantizer& pq, const uint8_t* codes, std::size_t n, const float* queries,
                std::size_t nq, std::size_t k, Neighbor* out) {
    const std::size_t m = pq.m();
#pragma omp parallel
    {
        std::vector<float> table(m * kSubCentroids), dist(kChunk);
#pragma omp for schedule(dynamic)
        for (long long q = 0; q < static_cast<long long>(nq); ++q) {
            query_table(pq, queries + static_cast<std::size_t>(q) * pq.d(), table.data());
            SortedList list(k);
            for (std::size_t i0 = 0; i0 < n; i0 += kChunk) {
                const std::size_t count = std::min(kChunk, n - i0);
                scan_chunk(table.data(), codes + i0 * m, count, m, dist.data());
                float bound = list.bound();
                for (std::size_t i = 0; i < count; ++i)
                    if (dist[i] <= bound) {
                        list.offer(dist[i], static_cast<int32_t>(i0 + i));
                        bound = list.bound();
                    }
            }
            list.write(out + static_cast<std::size_t>(q) * k);
        }
    }
}

}  // namespace veckern
