// Exact re-ranking of search candidates on the GPU: the step after the PQ search (reference rerank_exact,
// cpu_ref.cpp:66-77, used by bench --rerank, bench_main.cpp:145-153). For each query, the full-precision squared
// L2 distance to each candidate's base vector, then the k smallest by (dist, id).
//
// One wave per query; lane l takes candidates l, l + 64, ... . A lane computes its candidate's distance alone, in
// dimension order j = 0..d-1 with a separate multiply and add, exactly like l2sq (common.hpp:27-34), so distances
// are bit-identical to the CPU's; the query's values are wave-uniform scalar loads and the candidate's row is read
// with 16-byte loads when d % 4 == 0. The candidates of a wave feed a wave-cooperative sorted list (device.hpp).
// The work is a random gather of r rows of d floats per query: bound by HBM/L2 latency, not by arithmetic.
#include "kernels.hpp"

namespace vk {

namespace {

template <bool VEC4>
__device__ __forceinline__ float l2sq_row(const float* x, const float* row, int d) {
#pragma clang fp contract(off)
    float acc = 0.f;
    if constexpr (VEC4) {
        // Unrolled so that eight 16-byte loads of the row are in flight at once (the row is a random gather).
#pragma unroll 8
        for (int j = 0; j < d; j += 4) {
            const float4 v = *reinterpret_cast<const float4*>(row + j);
            float diff = x[j] - v.x;
            acc += diff * diff;
            diff = x[j + 1] - v.y;
            acc += diff * diff;
            diff = x[j + 2] - v.z;
            acc += diff * diff;
            diff = x[j + 3] - v.w;
            acc += diff * diff;
        }
    } else {
        for (int j = 0; j < d; ++j) {
            const float diff = x[j] - row[j];
            acc += diff * diff;
        }
    }
    return acc;
}

constexpr int kRerankThreads = 256;

template <int S, bool VEC4>
__global__ void __launch_bounds__(kRerankThreads) rerank_kernel(RerankArgs a) {
    const int lane = __lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / WAVE);
    const int64_t q = static_cast<int64_t>(blockIdx.x) * (kRerankThreads / WAVE) + wave;
    if (q >= a.nq) return;  // wave-uniform
    const float* x = a.queries + q * a.d;
    const Pair* cand = a.candidates ? a.candidates + q * a.r : nullptr;
    WaveList<S> list;
    list.init();
    bool bad = false;
    for (int64_t base = 0; base < a.r; base += WAVE) {
        const int64_t j = base + lane;
        const int32_t id = j < a.r ? (cand ? cand[j].i : static_cast<int32_t>(j)) : -1;
        bad |= id >= a.n;  // an id past the base: reported, never read
        const bool use = id >= 0 && id < a.n;
        const float dist = use ? l2sq_row<VEC4>(x, a.base + static_cast<int64_t>(id) * a.d, a.d) : INFINITY;
        list.offer(dist, id, use, a.K);
    }
    if (__builtin_amdgcn_ballot_w64(bad) && lane == 0) atomicOr(a.error, 1u);
    Pair* out = a.out + q * a.k;
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int p = s * WAVE + lane;
        if (p < a.k) out[p] = list.id[s] == kEmptyId ? Pair{INFINITY, -1} : Pair{list.d[s], list.id[s]};
    }
}

}  // namespace

hipError_t launch_rerank(const RerankArgs& a, hipStream_t stream) {
    const int waves_per_block = kRerankThreads / WAVE;
    const dim3 grid(static_cast<unsigned>((a.nq + waves_per_block - 1) / waves_per_block));
    const bool vec4 = a.d % 4 == 0;
    if (a.K <= WAVE) {
        if (vec4) hipLaunchKernelGGL((rerank_kernel<1, true>), grid, dim3(kRerankThreads), 0, stream, a);
        else hipLaunchKernelGGL((rerank_kernel<1, false>), grid, dim3(kRerankThreads), 0, stream, a);
    } else if (a.K <= 2 * WAVE) {
        if (vec4) hipLaunchKernelGGL((rerank_kernel<2, true>), grid, dim3(kRerankThreads), 0, stream, a);
        else hipLaunchKernelGGL((rerank_kernel<2, false>), grid, dim3(kRerankThreads), 0, stream, a);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace vk
