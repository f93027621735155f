// Nearest-centroid assignment on the GPU: the PQ encoder and the assignment step of k-means training (reference
// ProductQuantizer::encode / train, pq.cpp:11-22, 31-76). For sub-vector x of sub-space s it returns the first c
// in 0..255 with the smallest l2sq(x, C[s][c]), scanning c in order from a best distance of FLT_MAX exactly as
// nearest_centroid does, with l2sq's dimension order and separate multiply and add, so codes are identical to the
// CPU's, ties included.
//
// One lane per (vector, sub-space); a block's lanes share one sub-space (grid y), so the centroid being compared
// is the same for every lane: the sub-space's codebook is staged in LDS once per block and each centroid is an LDS
// broadcast (scalar loads of it per wave were latency-bound: 26 ms for 1M vectors at m=16, d=128, against ~2.5 ms
// of VALU work, 256 x dsub x 3 flops per code). A dense MFMA form
// (|x|^2 - 2 x.c + |c|^2) would be faster but rounds differently and can flip near-ties, so it is not used here.
#include <cfloat>

#include "kernels.hpp"

namespace vk {

namespace {

constexpr int kAssignThreads = 256;

template <int DSUB>
__global__ void __launch_bounds__(kAssignThreads) nearest_kernel(NearestArgs a) {
#pragma clang fp contract(off)
    const int s = blockIdx.y;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kAssignThreads + threadIdx.x;
    const int dsub = DSUB ? DSUB : a.dsub;
    const bool live = i < a.n;
    const float* xr = a.x + (live ? i : 0) * a.x_stride + static_cast<int64_t>(s) * dsub;
    const float* cent = a.centroids + static_cast<int64_t>(s) * 256 * dsub;
    int best = 0;
    float best_dist = FLT_MAX;
    if constexpr (DSUB > 0) {
        // The block's sub-space codebook (256 x DSUB floats, <= 16 KB) staged in LDS once; every lane then reads
        // the same centroid at the same time (an LDS broadcast, 16-byte reads when DSUB % 4 == 0).
        __shared__ __align__(16) float cl[256 * DSUB];
        for (int e = threadIdx.x; e < 256 * DSUB; e += kAssignThreads) cl[e] = cent[e];
        __syncthreads();
        float x[DSUB];
#pragma unroll
        for (int j = 0; j < DSUB; ++j) x[j] = xr[j];
        for (int c = 0; c < 256; ++c) {
            float cv[DSUB];
            if constexpr (DSUB % 4 == 0) {
#pragma unroll
                for (int j = 0; j < DSUB; j += 4) {
                    const float4 v = *reinterpret_cast<const float4*>(cl + c * DSUB + j);
                    cv[j] = v.x;
                    cv[j + 1] = v.y;
                    cv[j + 2] = v.z;
                    cv[j + 3] = v.w;
                }
            } else {
#pragma unroll
                for (int j = 0; j < DSUB; ++j) cv[j] = cl[c * DSUB + j];
            }
            float acc = 0.f;
#pragma unroll
            for (int j = 0; j < DSUB; ++j) {
                const float diff = x[j] - cv[j];
                acc += diff * diff;
            }
            if (acc < best_dist) {
                best_dist = acc;
                best = c;
            }
        }
    } else {
        for (int c = 0; c < 256; ++c) {
            float acc = 0.f;
            for (int j = 0; j < dsub; ++j) {
                const float diff = xr[j] - cent[c * dsub + j];
                acc += diff * diff;
            }
            if (acc < best_dist) {
                best_dist = acc;
                best = c;
            }
        }
    }
    if (!live) return;
    if (a.codes) a.codes[i * a.m + s] = static_cast<uint8_t>(best);
    if (a.assign) a.assign[i] = static_cast<uint32_t>(best);
}

}  // namespace

hipError_t launch_nearest(const NearestArgs& a, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((a.n + kAssignThreads - 1) / kAssignThreads), static_cast<unsigned>(a.m));
    switch (a.dsub) {
        case 2: hipLaunchKernelGGL(nearest_kernel<2>, grid, dim3(kAssignThreads), 0, stream, a); break;
        case 4: hipLaunchKernelGGL(nearest_kernel<4>, grid, dim3(kAssignThreads), 0, stream, a); break;
        case 8: hipLaunchKernelGGL(nearest_kernel<8>, grid, dim3(kAssignThreads), 0, stream, a); break;
        case 16: hipLaunchKernelGGL(nearest_kernel<16>, grid, dim3(kAssignThreads), 0, stream, a); break;
        default: hipLaunchKernelGGL(nearest_kernel<0>, grid, dim3(kAssignThreads), 0, stream, a); break;
    }
    return hipGetLastError();
}

}  // namespace vk
