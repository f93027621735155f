// Per-query lookup-table build: lut[q][s][c] = sum_j (x_q[s*dsub + j] - C[s][c][j])^2 with j in order
// (reference: cpu_ref.cpp:7-14 with l2sq, common.hpp:27-34; GPU lut_kernel, kernels.cuh:17-30).
//
// Grid (m, groups), block 256: thread c owns centroid c of sub-space s and produces the entries of the QG
// queries of group g, stored contiguously as lut[g][s][c][0..QG). QG = 1 is the plain [q][s][c] layout; QG = 2
// or 4 is the query-interleaved layout the fused wave kernel copies straight into LDS. The query sub-vector is
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

hipError_t launch_lut(const float* queries, const float* centroids, int d, int m, int nq, int qg, int groups,
                      float* lut, hipStream_t stream) {
    const int dsub = d / m;
    const dim3 grid(m, groups);
    switch (qg) {
        case 1: hipLaunchKernelGGL(lut_kernel<1>, grid, dim3(KSUB), 0, stream, queries, centroids, d, m, dsub, nq, lut); break;
        case 2: hipLaunchKernelGGL(lut_kernel<2>, grid, dim3(KSUB), 0, stream, queries, centroids, d, m, dsub, nq, lut); break;
        case 4: hipLaunchKernelGGL(lut_kernel<4>, grid, dim3(KSUB), 0, stream, queries, centroids, d, m, dsub, nq, lut); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace vk
