// Per-query lookup-table build: lut[q][s][c] = sum_j (x_q[s*dsub + j] - C[s][c][j])^2 with j in order
// (reference: cpu_ref.cpp:7-14 with l2sq, common.hpp:27-34; GPU lut_kernel, kernels.cuh:17-30).
//
// Grid (m, groups), block 256: thread c owns centroid c of sub-space s and produces the entries of the QG
// queries of group g, stored contiguously as lut[g][s][c][0..QG): the query-interleaved layout (QG = 2 or 4). The
// plain [q][s][c] layout (QG = 1) has its own kernel below. The query sub-vector is
// block-uniform, so it is read through scalar loads; the centroid row is read once and reused for all QG queries.
#include "kernels.hpp"

namespace vk {

template <int QG>
__global__ void __launch_bounds__(KSUB)
    lut_kernel(const float* __restrict__ queries, const float* __restrict__ centroids, int d, int m, int dsub, int nq,
               float* __restrict__ lut) {
    // Separate multiply and add, no FMA contraction: the CPU reference rounds diff*diff before adding it.
#pragma clang fp contract(off)
    const int s = blockIdx.x, g = blockIdx.y, c = threadIdx.x;
    const float* cent = centroids + (static_cast<size_t>(s) * KSUB + c) * dsub;
    float out[QG];
#pragma unroll
    for (int qq = 0; qq < QG; ++qq) {
        const int q = g * QG + qq;
        float acc = 0.f;
        if (q < nq) {
            const float* x = queries + static_cast<size_t>(q) * d + static_cast<size_t>(s) * dsub;
            for (int j = 0; j < dsub; ++j) {
                const float diff = x[j] - cent[j];
                acc += diff * diff;
            }
        }
        out[qq] = acc;
    }
    float* dst = lut + ((static_cast<size_t>(g) * m + s) * KSUB + c) * QG;
#pragma unroll
    for (int qq = 0; qq < QG; ++qq) dst[qq] = out[qq];
}

// The plain [q][s][c] layout (QG = 1), G queries per block: thread c reads centroid c of sub-space s once (DSUB
// known at compile time: one or two 16-byte loads) and produces its entry for each of the G queries, each store
// coalesced over c. A block per (s, query) would reread the centroid row G times and leave each thread one entry.
constexpr int kLutQueries = 8;

template <int DSUB>
__global__ void __launch_bounds__(KSUB)
    lut_rows_kernel(const float* __restrict__ queries, const float* __restrict__ centroids, int d, int m, int dsub_rt,
                    int nq, float* __restrict__ lut) {
#pragma clang fp contract(off)
    const int dsub = DSUB ? DSUB : dsub_rt;
    const int s = blockIdx.x, c = threadIdx.x;
    const int q0 = blockIdx.y * kLutQueries;
    const float* cent = centroids + (static_cast<size_t>(s) * KSUB + c) * dsub;
    float cv[DSUB ? DSUB : 1];
    if constexpr (DSUB > 0) {
#pragma unroll
        for (int j = 0; j < DSUB; ++j) cv[j] = cent[j];
    }
#pragma unroll
    for (int qq = 0; qq < kLutQueries; ++qq) {
        const int q = q0 + qq;
        if (q >= nq) break;  // block-uniform
        const float* x = queries + static_cast<size_t>(q) * d + static_cast<size_t>(s) * dsub;
        float acc = 0.f;
        if constexpr (DSUB > 0) {
#pragma unroll
            for (int j = 0; j < DSUB; ++j) {
                const float diff = x[j] - cv[j];
                acc += diff * diff;
            }
        } else {
            for (int j = 0; j < dsub; ++j) {
                const float diff = x[j] - cent[j];
                acc += diff * diff;
            }
        }
        lut[(static_cast<size_t>(q) * m + s) * KSUB + c] = acc;
    }
}

hipError_t launch_lut(const float* queries, const float* centroids, int d, int m, int nq, int qg, int groups,
                      float* lut, hipStream_t stream) {
    const int dsub = d / m;
    const dim3 grid(m, groups);
    if (qg == 1) {
        const dim3 rows(m, (nq + kLutQueries - 1) / kLutQueries);
        auto kernel = dsub == 8 ? lut_rows_kernel<8> : dsub == 4 ? lut_rows_kernel<4>
                                                     : dsub == 2 ? lut_rows_kernel<2> : lut_rows_kernel<0>;
        hipLaunchKernelGGL(kernel, rows, dim3(KSUB), 0, stream, queries, centroids, d, m, dsub, nq, lut);
        return hipGetLastError();
    }
    switch (qg) {
        case 2: hipLaunchKernelGGL(lut_kernel<2>, grid, dim3(KSUB), 0, stream, queries, centroids, d, m, dsub, nq, lut); break;
        case 4: hipLaunchKernelGGL(lut_kernel<4>, grid, dim3(KSUB), 0, stream, queries, centroids, d, m, dsub, nq, lut); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace vk
