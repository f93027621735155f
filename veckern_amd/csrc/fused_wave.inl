// Fused PQ scan + top-k with one wave-cooperative sorted list per (wave, query): the ScanVariant::FusedWarp
// path (reference: kernels.cuh:392-526, launch searcher.cu:365-415), designed for gfx950.
//
// Work decomposition. Queries are packed into slabs of QG*NG queries whose lookup tables sit together in LDS.
// A slab's work is its n vectors cut into granules of 64*U vectors (one wave step). The slabs * n_gran work
// items are split into `grid` equal contiguous ranges, one per block, with grid = resident blocks on the
// device (occupancy API), so every CU gets the same number of items and no tail wave is left. A block whose
// range spans two slabs reloads its tables in between; each (block, slab) pair emits one partial K-list per
// query, merged afterwards by the select kernel.
//
// LDS tables. A group of QG queries shares one table laid out [s][c][QG] floats, so a single ds_read_b32 /
// b64 / b128 at ((s * 256 + c) * QG) returns the entries of all QG queries for code byte c. Measured on
// MI355X with uniform random bytes, a wave64 ds_read_b128 costs about 12 CU cycles against 6.4 for b32, so
// QG = 4 gives ~2.1x the lookups per cycle of one table per query. NG groups share every code load.
//
// Exactness. Each query's distance is summed in sub-space order s = 0..m-1 from 0.f, exactly like the CPU
// reference (cpu_ref.cpp:46-49), so GPU and CPU distances are bit-identical and ids agree exactly under the
// (dist, id) order.
#pragma once

#include "kernels.hpp"

namespace vk {

template <int QG>
struct LdsVec;
template <>
struct LdsVec<1> {
    using T = float;
    __device__ static void add(float* acc, float v) { acc[0] += v; }
};
template <>
struct LdsVec<2> {
    using T = float2;
    __device__ static void add(float* acc, float2 v) {
        acc[0] += v.x;
        acc[1] += v.y;
    }
};
template <>
struct LdsVec<4> {
    using T = float4;
    __device__ static void add(float* acc, float4 v) {
        acc[0] += v.x;
        acc[1] += v.y;
        acc[2] += v.z;
        acc[3] += v.w;
    }
};

// QG: queries per table (1, 2, 4). NG: tables per block (1, 2). U: 64-vector tiles per wave step.
// M: sub-spaces if fixed at compile time, 0 for any m % 16 == 0. S: list registers per lane (K <= 64 * S).
// Waves per SIMD the block residency allows: blocks per CU are bounded by LDS (tables of QG*NG*M KB) and by
// 2048 threads; the register budget is set so that residency is not cut further by VGPRs (4 waves -> 128).
template <int QG, int NG, int M, int T>
constexpr int wave_kernel_waves_per_simd() {
    if (M == 0) return 1;
    const int by_lds = (160 * 1024) / (QG * NG * M * KSUB * 4);
    const int blocks = by_lds < 2048 / T ? by_lds : 2048 / T;
    const int waves = blocks * (T / WAVE) / 4;
    return waves < 1 ? 1 : (waves > 4 ? 4 : waves);
}

template <int QG, int NG, int U, int M, int S, int T>
__global__ void __launch_bounds__(T)
    __attribute__((amdgpu_waves_per_eu(wave_kernel_waves_per_simd<QG, NG, M, T>())))
    fused_wave_kernel_t(WaveScanArgs a) {
    constexpr int QS = QG * NG;
    constexpr int W = T / WAVE;
    using V = typename LdsVec<QG>::T;
    // With m fixed the tables are a static LDS array at address 0, so a lookup address is one SDWA shift of
    // the code byte plus a compile-time immediate offset; a dynamic (extern) array's base is a link-time
    // symbol that costs two more VALU adds per lookup.
    constexpr int kStaticFloats = M ? QG * NG * M * KSUB : 4;
    __shared__ __align__(16) float lds_static[kStaticFloats];
    extern __shared__ __align__(16) float lds_dynamic[];
    float* const lds_base = M ? lds_static : lds_dynamic;
    unsigned char* const smem = reinterpret_cast<unsigned char*>(lds_base);
    const float* lds = lds_base;
    const int m = M ? M : a.m;
    const int words = m / 16;
    const int table = m * KSUB * QG;  // floats per group table
    const int tid = threadIdx.x, lane = __lane_id(), wave = tid / WAVE;
    const int64_t grid = gridDim.x, b = blockIdx.x;
    const int64_t start = b * a.total / grid, end = (b + 1) * a.total / grid;

    for (int64_t item = start; item < end;) {
        const int64_t slab = item / a.n_gran;
        const int64_t g_lo = item - slab * a.n_gran;
        const int64_t g_hi = min(end - slab * a.n_gran, a.n_gran);

        __syncthreads();  // the previous slab's merge has finished with LDS
        {
            const float4* src = reinterpret_cast<const float4*>(a.lut + slab * NG * (int64_t)table);
            float4* dst = reinterpret_cast<float4*>(smem);
            const int n4 = NG * table / 4;
            for (int j = tid; j < n4; j += T) dst[j] = src[j];
        }
        __syncthreads();

        WaveList<S> lists[QS];
#pragma unroll
        for (int q = 0; q < QS; ++q) lists[q].init();
        const int live = static_cast<int>(min<int64_t>(QS, a.nq - slab * QS));  // padded queries are not offered

        for (int64_t g = g_lo + wave; g < g_hi; g += W) {
            const int64_t tile0 = g * U;
            const uint4* tile_codes = a.codes + tile0 * words * WAVE + lane;  // wave-uniform base + lane
            // All code words of the U tiles are loaded first (the global-load ILP). The lookups then run one
            // tile at a time behind a scheduling fence, and each tile's candidates are offered before the next
            // tile starts: only one tile's LDS results and accumulators are live, which keeps the register
            // count within what the LDS-limited residency allows.
            constexpr int WORDS = M ? M / 16 : 1;
            uint4 cw[U][WORDS];
            if constexpr (M > 0) {
#pragma unroll
                for (int u = 0; u < U; ++u)
#pragma unroll
                    for (int w = 0; w < WORDS; ++w) cw[u][w] = tile_codes[(u * WORDS + w) * WAVE];
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                float acc[QS];
#pragma unroll
                for (int q = 0; q < QS; ++q) acc[q] = 0.f;
                // 16 lookups of one code word, sub-spaces 16w .. 16w+15 in order.
                auto lookup_word = [&](const uint4 word, const int w) {
                    const uint32_t part[4] = {word.x, word.y, word.z, word.w};
#pragma unroll
                    for (int j = 0; j < 16; ++j) {
                        const uint32_t c = (part[j >> 2] >> (8 * (j & 3))) & 0xffu;
                        const int s = w * 16 + j;
#pragma unroll
                        for (int t = 0; t < NG; ++t) {
                            const V v = *reinterpret_cast<const V*>(lds + t * table + (s * KSUB + (int)c) * QG);
                            LdsVec<QG>::add(&acc[t * QG], v);
                        }
                    }
                };
                if constexpr (M > 0) {
#pragma unroll
                    for (int w = 0; w < WORDS; ++w) lookup_word(cw[u][w], w);
                } else {
                    for (int w = 0; w < words; ++w) lookup_word(tile_codes[(u * words + w) * WAVE], w);
                }
                __builtin_amdgcn_sched_barrier(0);
                const int64_t i = (tile0 + u) * WAVE + lane;
                const bool valid = i < a.n;
#pragma unroll
                for (int q = 0; q < QS; ++q)
                    if (q < live) lists[q].offer(acc[q], static_cast<int32_t>(i), valid, a.K);
            }
        }

        // Merge the W wave lists of each query into the block's partial list for this slab.
        const int slot = static_cast<int>(b - first_block_of(slab * a.n_gran, grid, a.total));
        Pair* buf = reinterpret_cast<Pair*>(smem);
        Pair* merged = buf + W * a.K;
#pragma unroll
        for (int q = 0; q < QS; ++q) {
            __syncthreads();
            lists[q].store(buf + wave * a.K, a.K);
            __syncthreads();
            merge_lists(buf, W, a.K, merged, tid, T);
            __syncthreads();
            Pair* dst = a.part + ((slab * a.max_slots + slot) * QS + q) * (int64_t)a.K;
            for (int j = tid; j < a.K; j += T) dst[j] = merged[j];
        }
        item = (slab + 1) * a.n_gran;
    }
}

template <int QG, int NG, int U, int M, int S, int T>
hipError_t launch_fused_wave_t(const WaveScanArgs& a, int grid, size_t smem, hipStream_t stream) {
    hipLaunchKernelGGL((fused_wave_kernel_t<QG, NG, U, M, S, T>), dim3(grid), dim3(T), smem, stream, a);
    return hipGetLastError();
}

template <int QG, int NG, int U, int M, int S>
WaveScanKernel make_wave_kernel() {
    constexpr int T = 512;
    WaveScanKernel k;
    k.fn = reinterpret_cast<const void*>(&fused_wave_kernel_t<QG, NG, U, M, S, T>);
    k.threads = T;
    k.dynamic_lds = M == 0;
    k.launch = &launch_fused_wave_t<QG, NG, U, M, S, T>;
    return k;
}

// Instances for one M: every (QG, NG) whose tables fit in 160 KB of LDS when M is known.
template <int M>
WaveScanKernel select_wave_kernel(int qg, int ng, int ilp, int segments) {
    constexpr int kLds = 160 * 1024;
#define VK_WAVE_CASE(QG_, NG_)                                                                      \
    if (qg == QG_ && ng == NG_) {                                                                   \
        if constexpr (M == 0 || QG_ * NG_ * M * KSUB * 4 <= kLds) {                                 \
            if (segments == 1) {                                                                    \
                if (ilp == 1) return make_wave_kernel<QG_, NG_, 1, M, 1>();                         \
                if (ilp == 2) return make_wave_kernel<QG_, NG_, 2, M, 1>();                         \
                if (ilp == 4) return make_wave_kernel<QG_, NG_, 4, M, 1>();                         \
            } else if (segments == 2) {                                                             \
                if (ilp == 1) return make_wave_kernel<QG_, NG_, 1, M, 2>();                         \
                if (ilp == 2) return make_wave_kernel<QG_, NG_, 2, M, 2>();                         \
                if (ilp == 4) return make_wave_kernel<QG_, NG_, 4, M, 2>();                         \
            }                                                                                       \
        }                                                                                           \
        return WaveScanKernel{};                                                                    \
    }
    VK_WAVE_CASE(1, 1)
    VK_WAVE_CASE(2, 1)
    VK_WAVE_CASE(4, 1)
    VK_WAVE_CASE(4, 2)
#undef VK_WAVE_CASE
    return WaveScanKernel{};
}

}  // namespace vk
