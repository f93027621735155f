// Exact squared L2 distances between every query and every coarse centroid of an inverted-file index: the
// first step of an IVF search (the probe), out[q][l] = sum_j (x_q[j] - coarse_l[j])^2 with j in order from 0.f
// and a separate multiply and add, the arithmetic of the reference's l2sq (common.hpp:27-34), so a following
// top-nprobe selection by (dist, id) picks exactly the lists the CPU would.
//
// The (query, list) matrix is dense, so it is computed in 32 x 64 tiles: the block stages 64-dimension slices of
// its 32 query rows and 64 centroid rows in LDS, and each of the 256 threads keeps a 2 x 4 block of running sums
// in registers, reading one 8-byte and one 16-byte LDS value per dimension for 8 sums. A wave per query over all centroids
// (what the exact re-rank kernel would do) reads each centroid row from L2 once per query and leaves most of the
// GPU idle at a few thousand queries.
#include "kernels.hpp"

namespace vk {

namespace {

constexpr int kTileQ = 32;    // queries per block tile
constexpr int kTileL = 64;    // centroids per block tile
constexpr int kSlice = 64;    // dimensions staged per LDS pass
constexpr int kThreads = 256;

__global__ void __launch_bounds__(kThreads) coarse_distance_kernel(const float* __restrict__ queries, int64_t nq,
                                                                  const float* __restrict__ coarse, int64_t nlist,
                                                                  int d, float* __restrict__ out) {
#pragma clang fp contract(off)
    // Slices stored dimension-major: thread (ty, tx) reads its queries 2ty, 2ty+1 and centroids 4tx..4tx+3 of
    // dimension c as one 8-byte and one 16-byte LDS read (the 16 tx of a wave cover 256 consecutive bytes).
    // Rows padded by 4 floats: the staging writes (consecutive lanes = consecutive dimensions of one row) then
    // spread over 16 banks instead of 1-2, and rows stay 16-byte aligned for the reads.
    __shared__ __align__(16) float xs[kSlice][kTileQ + 4];
    __shared__ __align__(16) float cs[kSlice][kTileL + 4];
    const int tid = threadIdx.x, ty = tid / 16, tx = tid % 16;
    const int64_t q0 = static_cast<int64_t>(blockIdx.y) * kTileQ, l0 = static_cast<int64_t>(blockIdx.x) * kTileL;
    float acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
    for (int j0 = 0; j0 < d; j0 += kSlice) {
        // Stage rows q0.. and l0.. for dimensions j0 .. j0 + kSlice - 1 (zeros past the ends; never summed into a
        // stored result: rows past nq or nlist are not written, dimensions past d are not read below).
        for (int e = tid; e < kTileQ * kSlice; e += kThreads) {
            const int r = e / kSlice, c = e % kSlice, j = j0 + c;
            const int64_t qr = q0 + r;
            xs[c][r] = (qr < nq && j < d) ? queries[qr * d + j] : 0.f;
        }
        for (int e = tid; e < kTileL * kSlice; e += kThreads) {
            const int r = e / kSlice, c = e % kSlice, j = j0 + c;
            const int64_t lr = l0 + r;
            cs[c][r] = (lr < nlist && j < d) ? coarse[lr * d + j] : 0.f;
        }
        __syncthreads();
        const int width = min(kSlice, d - j0);
        for (int c = 0; c < width; ++c) {
            const float2 xv = *reinterpret_cast<const float2*>(&xs[c][2 * ty]);
            const float4 cv = *reinterpret_cast<const float4*>(&cs[c][4 * tx]);
            const float xa[2] = {xv.x, xv.y}, ca[4] = {cv.x, cv.y, cv.z, cv.w};
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float diff = xa[i] - ca[j];
                    acc[i][j] += diff * diff;
                }
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int64_t q = q0 + 2 * ty + i;
        if (q >= nq) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t l = l0 + 4 * tx + j;
            if (l < nlist) out[q * nlist + l] = acc[i][j];
        }
    }
}

}  // namespace

hipError_t launch_coarse_distances(const float* queries, int64_t nq, const float* coarse, int64_t nlist, int d,
                                   float* out, hipStream_t stream) {
    if (nq <= 0 || nlist <= 0 || d <= 0 || (nq + kTileQ - 1) / kTileQ > 65535) return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>((nlist + kTileL - 1) / kTileL),
                    static_cast<unsigned>((nq + kTileQ - 1) / kTileQ));
    hipLaunchKernelGGL(coarse_distance_kernel, grid, dim3(kThreads), 0, stream, queries, nq, coarse, nlist, d, out);
    return hipGetLastError();
}

}  // namespace vk
