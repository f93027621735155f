// Inverted-file (IVF) search, the reference's "coarse partitioning" next step (README.md:219): per query, the
// nprobe nearest coarse centroids (exact distances in tiles, probe.hip, and the row top-k of select.hip), then the
// fused wave-list scan over only those lists' PQ codes (fused_wave.inl with IVF = true: slabs = (query, probed
// list) in query-major order), then this file's merge of each query's partial lists. The slab plan is built on
// the device from the probes (this file's plan kernels), so a search makes no host round trip before its results.
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
constexpr int kPlanThreads = 256;
constexpr int kScanThreads = 1024;

__device__ __forceinline__ int64_t wave_inclusive_sum(int64_t v) {
    const int lane = __lane_id();
#pragma unroll
    for (int o = 1; o < WAVE; o <<= 1) {
        const int64_t up = __shfl_up(v, o);
        if (lane >= o) v += up;
    }
    return v;
}

// Plan, step 1 (one wave per query): slab q * nprobe + p is query q's p-th probed list; its granule count is the
// list's padded tiles / 4 (0 for a probe of no list). slab_gran receives each slab's start within its query's run
// and query_gran[q] the run's length.
__global__ void __launch_bounds__(kPlanThreads) ivf_plan_runs_kernel(IvfPlanArgs a) {
    const int lane = __lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / WAVE);
    const int64_t q = static_cast<int64_t>(blockIdx.x) * (kPlanThreads / WAVE) + wave;
    if (q >= a.nq) return;  // wave-uniform
    int64_t run = 0;
    for (int base = 0; base < a.nprobe; base += WAVE) {
        const int p = base + lane;
        int64_t tile = 0;
        int64_t gran = 0;
        if (p < a.nprobe) {
            const int32_t l = a.probes[q * a.nprobe + p].i;
            if (l >= 0) {  // a query whose coarse distances are all NaN probes nothing
                tile = a.list_tile[l];
                gran = (a.list_tile[l + 1] - tile) / 4;
            }
        }
        const int64_t incl = wave_inclusive_sum(gran);
        if (p < a.nprobe) {
            const int64_t s = q * a.nprobe + p;
            a.slab_tile[s] = tile;
            a.slab_queries[s] = static_cast<int32_t>(q);
            a.slab_gran[s] = run + incl - gran;
        }
        run += __shfl(incl, WAVE - 1);
    }
    if (lane == 0) a.query_gran[q] = run;
}

// Plan, step 2 (one block): query_gran[0..nq) from run lengths to their exclusive prefix, query_gran[nq] = total.
__global__ void __launch_bounds__(kScanThreads) ivf_plan_scan_kernel(IvfPlanArgs a) {
    __shared__ int64_t wave_sums[kScanThreads / WAVE];
    const int tid = threadIdx.x, lane = __lane_id(), wave = tid / WAVE;
    const int64_t per = (a.nq + kScanThreads - 1) / kScanThreads;
    const int64_t lo = min<int64_t>(a.nq, tid * per), hi = min<int64_t>(a.nq, lo + per);
    int64_t sum = 0;
    for (int64_t i = lo; i < hi; ++i) sum += a.query_gran[i];
    const int64_t incl = wave_inclusive_sum(sum);
    if (lane == WAVE - 1) wave_sums[wave] = incl;
    __syncthreads();
    int64_t before = 0;
    for (int w = 0; w < wave; ++w) before += wave_sums[w];
    int64_t run = before + incl - sum;
    for (int64_t i = lo; i < hi; ++i) {
        const int64_t len = a.query_gran[i];
        a.query_gran[i] = run;
        run += len;
    }
    if (tid == kScanThreads - 1) a.query_gran[a.nq] = run;
}

// Plan, step 3 (one thread per slab): slab starts from run-relative to absolute; slab_gran[n_slabs] = total.
__global__ void __launch_bounds__(kPlanThreads) ivf_plan_offsets_kernel(IvfPlanArgs a) {
    const int64_t s = static_cast<int64_t>(blockIdx.x) * kPlanThreads + threadIdx.x;
    const int64_t slabs = a.nq * a.nprobe;
    if (s < slabs) a.slab_gran[s] += a.query_gran[s / a.nprobe];
    if (s == slabs) a.slab_gran[s] = a.query_gran[a.nq];
}

// One wave per query streams its partial lists through a wave list (device.hpp: whole lists when long, else
// 64-pair chunks) and writes the k best, empty slots as {+inf, -1}. The lists of query q are those of the blocks
// b_lo .. b_hi that cover its run, at (b + q) * W * K (the scan's layout), so one contiguous range; the scan used
// min(grid, total) blocks, each owning at least one granule, so every block of that range wrote its lists.
template <int S>
__global__ void __launch_bounds__(kMergeThreads) ivf_merge_kernel(IvfMergeArgs a) {
    const int lane = __lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / WAVE);
    const int64_t q = static_cast<int64_t>(blockIdx.x) * (kMergeThreads / WAVE) + wave;
    if (q >= a.nq) return;  // wave-uniform
    WaveList<S, true> wl;
    wl.init();
    const int64_t r_first = a.query_gran[q], r_next = a.query_gran[q + 1], total = a.query_gran[a.nq];
    const int64_t grid = min(a.grid, total);  // the blocks that took part in the scan
    if (r_next > r_first) {  // an empty run (no probed vectors) has no lists: all slots stay empty
        const int64_t b_lo = first_block_of(r_first, grid, total), b_hi = first_block_of(r_next - 1, grid, total);
        const Pair* first = a.part + (b_lo + q) * a.lists_per_block * a.K;
        const int lists = static_cast<int>((b_hi - b_lo + 1) * a.lists_per_block);
        stream_partials(wl, first, 0, 1, lists, a.K, lane);
    }
    Pair* out = a.out + q * a.k;
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int j = s * WAVE + lane;
        if (j < a.k) out[j] = wl.id[s] == kEmptyId ? Pair{INFINITY, -1} : Pair{wl.d[s], wl.id[s]};
    }
}

}  // namespace

hipError_t launch_ivf_plan(const IvfPlanArgs& a, hipStream_t stream) {
    if (a.nq <= 0 || a.nprobe <= 0) return hipErrorInvalidValue;
    const int waves = kPlanThreads / WAVE;
    hipLaunchKernelGGL(ivf_plan_runs_kernel, dim3(static_cast<unsigned>((a.nq + waves - 1) / waves)),
                       dim3(kPlanThreads), 0, stream, a);
    hipLaunchKernelGGL(ivf_plan_scan_kernel, dim3(1), dim3(kScanThreads), 0, stream, a);
    const int64_t slabs = a.nq * a.nprobe + 1;
    hipLaunchKernelGGL(ivf_plan_offsets_kernel, dim3(static_cast<unsigned>((slabs + kPlanThreads - 1) / kPlanThreads)),
                       dim3(kPlanThreads), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_ivf_merge(const IvfMergeArgs& a, hipStream_t stream) {
    const int waves_per_block = kMergeThreads / WAVE;
    const dim3 grid(static_cast<unsigned>((a.nq + waves_per_block - 1) / waves_per_block));
    if (a.K <= WAVE) hipLaunchKernelGGL(ivf_merge_kernel<1>, grid, dim3(kMergeThreads), 0, stream, a);
    else if (a.K <= 2 * WAVE) hipLaunchKernelGGL(ivf_merge_kernel<2>, grid, dim3(kMergeThreads), 0, stream, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace vk
