#pragma once
// The CPU search path (reference interface: include/veckern/cpu_ref.hpp:42-59): per-query LUT, ADC scan and top-k
// on the host, in libveckern_cpu. It is the CPU counterpart that veckern_bench times beside the GPU (its
// "cpu_reference" row), with the reference's declarations so the reference's own callers (its bench driver and
// tests) compile against this header unchanged. Results are those of the reference's CPU path bit for bit: LUT
// entries are l2sq of the sub-vectors (terms in index order), distances are summed over sub-spaces s = 0..m-1 from
// 0.f, and the k results are the k smallest (dist, id) pairs in ascending order, padded with {+inf, -1}.
//
// The selector (TopK), exact search, exact re-ranking and recall are declared in eval.hpp, included here.
#include <cstdint>

#include "veckern/common.hpp"
#include "veckern/eval.hpp"
#include "veckern/pq.hpp"

namespace veckern {

// lut: nq x m x 256 squared sub-distances of each query to every centroid (cpu_ref.hpp:42).
void compute_lut(const ProductQuantizer& pq, const float* queries, std::size_t nq, float* lut);
// dists: nq x n ADC distances of every query to every coded vector (cpu_ref.hpp:44).
void adc_scan(const float* lut, std::size_t nq, const uint8_t* codes, std::size_t n, std::size_t m, float* dists);
// The k smallest of each row of an nq x n distance matrix; ids are column indices (cpu_ref.hpp:46).
void select_topk(const float* dists, std::size_t nq, std::size_t n, std::size_t k, Neighbor* out);
// LUT, scan and selection per query without the nq x n matrix; out: nq x k (cpu_ref.hpp:48-49).
void adc_search(const ProductQuantizer& pq, const uint8_t* codes, std::size_t n, const float* queries,
                std::size_t nq, std::size_t k, Neighbor* out);

}  // namespace veckern
