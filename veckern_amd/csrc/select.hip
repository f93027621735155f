// Top-k selection (reference: select_kernel, kernels.cuh:179-202, launched by searcher.cu:285-296).
// One block per query. Each wave streams its share of the candidates into a wave-cooperative sorted list
// (threshold test per candidate, rare inserts), then the four wave lists are merged by rank. Two candidate
// sources share the kernel:
//   mode 0 — a row of n distances, ids are column indices (unfused scans);
//   mode 1 — bx partial K-lists per query laid out [q][bx][K] (per-thread-list fused scans).
// Empty slots ({+inf, INT32_MAX}) are skipped, like the reference skips id < 0, and the output turns any that
// remain into {+inf, -1}.
#include <type_traits>

#include "kernels.hpp"

namespace vk {

template <int S>
__global__ void __launch_bounds__(256) select_kernel(SelectArgs a) {
    constexpr int T = 256, W = T / WAVE;
    __shared__ Pair buf[(W + 1) * WAVE * S];
    const int64_t q = blockIdx.x;
    const int tid = threadIdx.x, lane = __lane_id(), wave = tid / WAVE;
    const int K = a.K;

    WaveList<S, true> list;  // bulk admission: a row's first chunks admit most of their lanes
    list.init();
    if (a.mode == 0) {
        // Long rows (n distances of an unfused scan): each wave reads 4 x 1 KB per round (16-byte loads, four in
        // flight) and offers them as 16 candidates per lane; the threshold test rejects nearly all of them once the
        // list fills. Short rows (an IVF probe's nlist distances): one 16-byte load per lane per round, so that
        // every wave of the block takes a share of the row.
        const float* row = a.dists + q * a.len;
        constexpr int V = 4;
        const bool vec = a.len % V == 0 && reinterpret_cast<uintptr_t>(row) % 16 == 0;
        auto rounds = [&](auto r_tag) -> int64_t {
            constexpr int R = decltype(r_tag)::value, CH = WAVE * V * R;  // floats per wave per round
            const int64_t full = vec ? a.len / CH * CH : 0;  // complete rounds; chunk c goes to wave c % W
            for (int64_t base = static_cast<int64_t>(wave) * CH; base < full; base += W * CH) {
                float4 v[R];
#pragma unroll
                for (int r = 0; r < R; ++r)
                    v[r] = *reinterpret_cast<const float4*>(row + base + (r * WAVE + lane) * V);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const int32_t j = static_cast<int32_t>(base + (r * WAVE + lane) * V);
                    list.offer(v[r].x, j, true, K);
                    list.offer(v[r].y, j + 1, true, K);
                    list.offer(v[r].z, j + 2, true, K);
                    list.offer(v[r].w, j + 3, true, K);
                }
            }
            return full;
        };
        const int64_t full = a.len >= int64_t{W} * WAVE * V * 4 ? rounds(std::integral_constant<int, 4>{})
                                                                 : rounds(std::integral_constant<int, 1>{});
        // The rest of the row (all of it when unaligned): one distance per lane, waves interleaved.
        for (int64_t b0 = full + static_cast<int64_t>(wave) * WAVE; b0 < a.len; b0 += W * WAVE) {
            const int64_t j = b0 + lane;
            const bool valid = j < a.len;
            const float x = valid ? row[j] : INFINITY;
            list.offer(x, static_cast<int32_t>(j), valid, K);
        }
    } else {
        const Pair* first = a.part + q * a.bx * K;
        const int64_t all = a.bx * K;
        for (int64_t base = static_cast<int64_t>(wave) * WAVE; base < all; base += W * WAVE) {
            const int64_t e = base + lane;
            Pair p{INFINITY, kEmptyId};
            if (e < all) p = first[e];
            list.offer(p.d, p.i, p.i != kEmptyId, K);
        }
    }

    Pair* merged = buf + W * K;
    list.store(buf + wave * K, K);
    __syncthreads();
    merge_lists(buf, W, K, merged, tid, T);
    __syncthreads();
    for (int j = tid; j < a.k; j += T) {
        const Pair p = merged[j];
        a.out[q * a.k + j] = p.i == kEmptyId ? Pair{INFINITY, -1} : p;
    }
}

hipError_t launch_select(const SelectArgs& a, int nq, hipStream_t stream) {
    if (a.K <= WAVE) hipLaunchKernelGGL(select_kernel<1>, dim3(nq), dim3(256), 0, stream, a);
    else if (a.K <= 2 * WAVE) hipLaunchKernelGGL(select_kernel<2>, dim3(nq), dim3(256), 0, stream, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace vk
