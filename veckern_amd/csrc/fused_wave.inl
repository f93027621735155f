// Fused PQ scan + top-k with one wave-cooperative sorted list per (wave, query): the ScanVariant::FusedWarp
// path (reference: kernels.cuh:392-526, launch searcher.cu:365-415), designed for gfx950.
//
// Work decomposition. Queries are packed into slabs of QG*NG queries whose lookup tables sit together in LDS.
// A slab's work is its n vectors cut into granules of 64*U vectors (one wave step). The slabs * n_gran work
// items are split into `grid` equal contiguous ranges, one per block, with grid = resident blocks on the
// device (occupancy API), so every CU gets the same number of items and no tail wave is left. A block builds
// the tables of each slab its range touches directly in LDS from the queries and the codebook (no LUT in HBM),
// and each (block, slab) pair emits one partial K-list per query. The last block to finish a slab (a per-slab
// counter) merges the slab's partial lists into the final results, so a search is a single launch.
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

#include <algorithm>

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

// Loads n consecutive floats from p (16-byte aligned when n % 4 == 0, 8-byte aligned when n == 2) with the widest
// vector loads the alignment allows.
template <int N>
__device__ __forceinline__ void load_floats(const float* p, float* out) {
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (int j = 0; j < N; j += 4) {
            const float4 v = *reinterpret_cast<const float4*>(p + j);
            out[j] = v.x;
            out[j + 1] = v.y;
            out[j + 2] = v.z;
            out[j + 3] = v.w;
        }
    } else if constexpr (N == 2) {
        const float2 v = *reinterpret_cast<const float2*>(p);
        out[0] = v.x;
        out[1] = v.y;
    } else {
#pragma unroll
        for (int j = 0; j < N; ++j) out[j] = p[j];
    }
}

// Builds the NG query-interleaved tables of a slab in LDS: entry (s, c) of query q is
// sum_j (x_q[s*dsub + j] - C[s][c][j])^2 with j in order and a separate multiply and add, the CPU reference's
// arithmetic (cpu_ref.cpp:7-14, common.hpp:27-34). Wave w takes sub-spaces w, w + W, ..., so the query values it
// reads are wave-uniform (scalar loads); lane l takes centroids l, l + 64, l + 128, l + 192. With the sub-vector
// width DSUB known at compile time, the four centroids' loads of a sub-space are issued together, so a build costs
// about one memory round trip per sub-space a wave handles rather than one per element. DSUB = 0: any width.
// Padded query slots read the last real query; their entries are never used.
template <int QG, int NG, int M, int W, int DSUB>
__device__ __forceinline__ void build_tables_w(const WaveScanArgs& a, int64_t slab, float* lds, int wave, int lane) {
#pragma clang fp contract(off)
    constexpr int QS = QG * NG;
    constexpr int R = KSUB / WAVE;  // centroids per lane and sub-space
    const int m = M ? M : a.m;
    const int dsub = DSUB ? DSUB : a.d / m;
    const int table = m * KSUB * QG;
    const float* qrow[QS];
#pragma unroll
    for (int q = 0; q < QS; ++q) qrow[q] = a.queries + std::min<int64_t>(slab * QS + q, a.nq - 1) * a.d;
    auto store = [&](int s, int c, const float* acc) {
#pragma unroll
        for (int t = 0; t < NG; ++t) {
            float* dst = lds + t * table + (s * KSUB + c) * QG;
            if constexpr (QG == 4) *reinterpret_cast<float4*>(dst) = make_float4(acc[t * 4], acc[t * 4 + 1],
                                                                                 acc[t * 4 + 2], acc[t * 4 + 3]);
            else if constexpr (QG == 2) *reinterpret_cast<float2*>(dst) = make_float2(acc[t * 2], acc[t * 2 + 1]);
            else dst[0] = acc[t];
        }
    };
    for (int s = wave; s < m; s += W) {
        const float* cbase = a.centroids + static_cast<int64_t>(s) * KSUB * dsub;
        if constexpr (DSUB > 0) {
            float cv[R][DSUB];
#pragma unroll
            for (int r = 0; r < R; ++r) load_floats<DSUB>(cbase + (r * WAVE + lane) * DSUB, cv[r]);
            float qv[QS][DSUB];
#pragma unroll
            for (int q = 0; q < QS; ++q)
#pragma unroll
                for (int j = 0; j < DSUB; ++j) qv[q][j] = qrow[q][s * DSUB + j];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float acc[QS];
#pragma unroll
                for (int q = 0; q < QS; ++q) {
                    acc[q] = 0.f;
#pragma unroll
                    for (int j = 0; j < DSUB; ++j) {
                        const float diff = qv[q][j] - cv[r][j];
                        acc[q] += diff * diff;
                    }
                }
                store(s, r * WAVE + lane, acc);
            }
        } else {
            for (int r = 0; r < R; ++r) {
                const int c = r * WAVE + lane;
                const float* cent = cbase + c * dsub;
                float acc[QS];
#pragma unroll
                for (int q = 0; q < QS; ++q) acc[q] = 0.f;
                for (int j = 0; j < dsub; ++j) {
                    const float cj = cent[j];
#pragma unroll
                    for (int q = 0; q < QS; ++q) {
                        const float diff = qrow[q][s * dsub + j] - cj;
                        acc[q] += diff * diff;
                    }
                }
                store(s, c, acc);
            }
        }
    }
}

// Sub-vector widths of d = 128 at m = 16, 32, 64 (and 64 at m = 16) get an unrolled build; others the generic one.
template <int QG, int NG, int M, int W>
__device__ __forceinline__ void build_tables(const WaveScanArgs& a, int64_t slab, float* lds, int wave, int lane) {
    const int dsub = a.d / (M ? M : a.m);
    if (dsub == 8) build_tables_w<QG, NG, M, W, 8>(a, slab, lds, wave, lane);
    else if (dsub == 4) build_tables_w<QG, NG, M, W, 4>(a, slab, lds, wave, lane);
    else if (dsub == 2) build_tables_w<QG, NG, M, W, 2>(a, slab, lds, wave, lane);
    else build_tables_w<QG, NG, M, W, 0>(a, slab, lds, wave, lane);
}

// Streams pairs [begin, all) of consecutive partial lists through a wave list: four 64-pair chunks per round (four
// loads in flight), rounds `step` pairs apart so that several waves can split one range.
template <int S>
__device__ __forceinline__ void stream_pairs(WaveList<S>& wl, const Pair* first, int begin, int step, int all, int K,
                                             int lane) {
    constexpr int B = 4;
    for (int base = begin; base < all; base += step) {
        Pair p[B];
#pragma unroll
        for (int u = 0; u < B; ++u) {
            const int e = base + u * WAVE + lane;
            p[u] = e < all ? first[e] : Pair{INFINITY, kEmptyId};
        }
#pragma unroll
        for (int u = 0; u < B; ++u) wl.offer(p[u].d, p[u].i, p[u].i != kEmptyId, K);
    }
}

// Final merge of one query of a slab by a single wave (few partial lists): no barriers; the wave list's first k
// entries are the results, empty slots written as the reference's {+inf, -1}.
template <int S>
__device__ __forceinline__ void merge_query_wave(const Pair* first, int lists, int K, int k, Pair* out, int lane) {
    WaveList<S> wl;
    wl.init();
    stream_pairs(wl, first, 0, 4 * WAVE, lists * K, K, lane);
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int j = s * WAVE + lane;
        if (j < k) out[j] = wl.id[s] == kEmptyId ? Pair{INFINITY, -1} : Pair{wl.d[s], wl.id[s]};
    }
}

// Final merge of one query of a slab by the last block to finish the slab: the slab's `lists` partial lists for
// the query (K pairs each, `first[l * K + j]`) are split over the W waves, each streaming its share through a wave
// list, four 64-pair chunks per round; the W wave lists are then merged by rank into the query's k results. LDS
// `buf` holds W * K pairs. Called by all threads of the block.
template <int S, int W>
__device__ __forceinline__ void merge_query(const Pair* first, int lists, int K, int k, Pair* out, Pair* buf,
                                            int tid, int wave, int lane) {
    WaveList<S> wl;
    wl.init();
    stream_pairs(wl, first, wave * 4 * WAVE, W * 4 * WAVE, lists * K, K, lane);
    wl.store(buf + wave * K, K);
    __syncthreads();
    merge_lists(buf, W, K, out, tid, W * WAVE, k, true);
    __syncthreads();
}

// QG: queries per table (1, 2, 4). NG: tables per block (1, 2). U: 64-vector tiles per wave step.
// M: sub-spaces if fixed at compile time, 0 for any m % 16 == 0. S: list registers per lane (K <= 64 * S).
// Waves per SIMD the block residency allows: blocks per CU are bounded by LDS (tables of QG*NG*M KB) and by
// 2048 threads; the register budget is set so that residency is not cut further by VGPRs (4 waves -> 128).
template <int QG, int NG, int M, int T>
constexpr int wave_kernel_waves_per_simd() {
    if (M == 0) return 1;
    const int by_lds = (160 * 1024) / (QG * NG * (M ? M : 16) * KSUB * 4);
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
    __shared__ bool last_block;
    float* const lds_base = M ? lds_static : lds_dynamic;
    const float* lds = lds_base;
    const int m = M ? M : a.m;
    const int words = m / 16;
    const int table = m * KSUB * QG;  // floats per group table
    // The wave index is the same in every lane; reading it through a scalar register lets the compiler keep the
    // granule, tile and id arithmetic of the scan loop on the scalar unit.
    const int tid = threadIdx.x, lane = __lane_id(), wave = __builtin_amdgcn_readfirstlane(tid / WAVE);
    const int64_t grid = gridDim.x, b = blockIdx.x;
    const int64_t start = b * a.total / grid, end = (b + 1) * a.total / grid;

    for (int64_t item = start; item < end;) {
        const int64_t slab = item / a.n_gran;
        const int64_t g_lo = item - slab * a.n_gran;
        const int64_t g_hi = min(end - slab * a.n_gran, a.n_gran);

        __syncthreads();  // the previous slab's merge has finished with LDS
        build_tables<QG, NG, M, W>(a, slab, lds_base, wave, lane);
        __syncthreads();

        // A padded query slot (past nq in the last slab) gets the threshold -inf: no distance passes it, so the
        // scan loop offers every slot without a per-query test.
        WaveList<S> lists[QS];
        const int64_t live = a.nq - slab * QS;
#pragma unroll
        for (int q = 0; q < QS; ++q) {
            lists[q].init();
            if (q >= live) lists[q].thr_d = -INFINITY;
        }
        const uint32_t n32 = static_cast<uint32_t>(a.n);  // n < 2^31: ids and tile bounds fit in 32 bits

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
                // Lanes holding a real vector: all of them except in the database's last tile.
                const uint32_t first = static_cast<uint32_t>((tile0 + u) * WAVE);
                const uint32_t id = first + static_cast<uint32_t>(lane);
                const uint64_t valid = first + WAVE <= n32 ? ~uint64_t{0} : __builtin_amdgcn_ballot_w64(id < n32);
#pragma unroll
                for (int q = 0; q < QS; ++q) lists[q].offer_masked(acc[q], static_cast<int32_t>(id), valid, a.K);
            }
        }

        // Partial lists of this (block, slab): part[slab][q][slot][list][K], the lists of one query contiguous.
        // With few blocks per slab every wave writes its own lists; with many, the block first merges its W lists
        // per query in LDS (the tables are dead by then), so the final merge reads W times fewer pairs.
        const int slot = static_cast<int>(b - first_block_of(slab * a.n_gran, grid, a.total));
        const int lpb = a.lists_per_block;
        Pair* const slab_part = a.part + slab * QS * a.max_slots * lpb * static_cast<int64_t>(a.K);
        Pair* const buf = reinterpret_cast<Pair*>(lds_base);  // QS * W * K pairs fit in the tables' space
        if (lpb == 1) {
            __syncthreads();  // every wave has finished reading the tables
#pragma unroll
            for (int q = 0; q < QS; ++q) lists[q].store(buf + (q * W + wave) * a.K, a.K);
            __syncthreads();
#pragma unroll
            for (int q = 0; q < QS; ++q)
                merge_lists(buf + q * W * a.K, W, a.K, slab_part + (q * a.max_slots + slot) * a.K, tid, T);
        } else {
#pragma unroll
            for (int q = 0; q < QS; ++q)
                lists[q].store(slab_part + ((q * a.max_slots + slot) * W + wave) * a.K, a.K);
        }

        // The last of the slab's blocks to get here merges all its partial lists into the final results. The
        // counter is incremented with wrap-around at count - 1, so it is back at zero for the next search. The
        // agent-scope release fence after the barrier publishes the whole block's partial lists before the
        // increment; the last block's acquire fence makes every other block's lists visible to it.
        const int64_t lo = first_block_of(slab * a.n_gran, grid, a.total);
        const int count = static_cast<int>(first_block_of((slab + 1) * a.n_gran - 1, grid, a.total) - lo + 1);
        __syncthreads();
        if (tid == 0) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
            last_block = atomicInc(a.counters + slab, static_cast<unsigned>(count - 1)) == count - 1u;
        }
        __syncthreads();
        if (last_block) {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            if (lpb == W) {  // at most 8 blocks per slab: one wave per query
                for (int q = wave; q < QS && slab * QS + q < a.nq; q += W)
                    merge_query_wave<S>(slab_part + q * a.max_slots * W * a.K, count * W, a.K, a.k,
                                        a.out + (slab * QS + q) * a.k, lane);
            } else {
                for (int q = 0; q < QS && slab * QS + q < a.nq; ++q)
                    merge_query<S, W>(slab_part + q * a.max_slots * a.K, count, a.K, a.k,
                                      a.out + (slab * QS + q) * a.k, buf, tid, wave, lane);
            }
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
