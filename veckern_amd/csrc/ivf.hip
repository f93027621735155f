// Inverted-file (IVF) search, the reference's "coarse partitioning" next step (README.md:219): per query, the
// nprobe nearest coarse centroids (exact distances, the re-rank kernel with every list as a candidate), then the
// fused wave-list scan over only those lists' PQ codes (fused_wave.inl with IVF = true: slabs = (query, probed
// list) in query-major order), then this file's merge of each query's partial lists.
#include "kernels.hpp"

namespace vk {

WaveScanKernel ivf_kernel_m16(int segments);
WaveScanKernel ivf_kernel_m32(int segments);
WaveScanKernel ivf_kernel_m64(int segments);
WaveScanKernel ivf_kernel_mx(int segments);

WaveScanKernel ivf_kernel(int m, int segments) {
    switch (m) {
        case 16: return ivf_kernel_m16(segments);
        case 32: return ivf_kernel_m32(segments);
        case 64: return ivf_kernel_m64(segments);
        default: return ivf_kernel_mx(segments);
    }
}

namespace {

constexpr int kMergeThreads = 256;

// One wave per query streams the pairs of its partial lists through a wave list (four 64-pair chunks in flight
// per round) and writes the k best, empty slots as {+inf, -1}.
template <int S>
__global__ void __launch_bounds__(kMergeThreads) ivf_merge_kernel(IvfMergeArgs a) {
    const int lane = __lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / WAVE);
    const int64_t q = static_cast<int64_t>(blockIdx.x) * (kMergeThreads / WAVE) + wave;
    if (q >= a.nq) return;  // wave-uniform
    WaveList<S> wl;
    wl.init();
    const Pair* first = a.part + a.seg_off[q];
    const int len = a.seg_len[q];
    constexpr int B = 4;
    for (int base = 0; base < len; base += B * WAVE) {
        Pair e[B];
#pragma unroll
        for (int u = 0; u < B; ++u) {
            const int j = base + u * WAVE + lane;
            e[u] = j < len ? first[j] : Pair{INFINITY, kEmptyId};
        }
#pragma unroll
        for (int u = 0; u < B; ++u) wl.offer(e[u].d, e[u].i, e[u].i != kEmptyId, a.K);
    }
    Pair* out = a.out + q * a.k;
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int j = s * WAVE + lane;
        if (j < a.k) out[j] = wl.id[s] == kEmptyId ? Pair{INFINITY, -1} : Pair{wl.d[s], wl.id[s]};
    }
}

}  // namespace

hipError_t launch_ivf_merge(const IvfMergeArgs& a, hipStream_t stream) {
    const int waves_per_block = kMergeThreads / WAVE;
    const dim3 grid(static_cast<unsigned>((a.nq + waves_per_block - 1) / waves_per_block));
    if (a.K <= WAVE) hipLaunchKernelGGL(ivf_merge_kernel<1>, grid, dim3(kMergeThreads), 0, stream, a);
    else if (a.K <= 2 * WAVE) hipLaunchKernelGGL(ivf_merge_kernel<2>, grid, dim3(kMergeThreads), 0, stream, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace vk
