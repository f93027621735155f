// Exact squared L2 distances between vectors and the coarse centroids of an inverted-file index, sum_j (x[j] -
// coarse_l[j])^2 with j in order from 0.f and a separate multiply and add: the arithmetic of the reference's l2sq
// (common.hpp:27-34), so a selection by (dist, id) over them picks exactly the lists the CPU would. Two uses:
//  - the probe of a search: the dense (query x list) matrix, followed by the row top-nprobe kernel;
//  - list assignment while building an index: the nearest list of each vector (nprobe = 1), reduced inside the
//    kernel, so the n x nlist matrix is never written.
//
// The matrix is computed in 32 x 64 tiles: the block stages 64-dimension slices of its 32 vector rows and 64
// centroid rows in LDS, and each of the 256 threads keeps a 2 x 4 block of running sums in registers, reading one
// 8-byte and one 16-byte LDS value per dimension for 8 sums. A wave per vector over all centroids (what the exact
// re-rank kernel would do) reads each centroid row from L2 once per vector and leaves most of the GPU idle at a
// few thousand queries.
#include <climits>

#include "kernels.hpp"

namespace vk {

namespace {

constexpr int kTileQ = 32;    // vectors (queries) per block tile
constexpr int kTileL = 64;    // centroids per block tile
constexpr int kSlice = 64;    // dimensions staged per LDS pass
constexpr int kThreads = 256;

// Slices stored dimension-major: thread (ty, tx) reads its rows 2ty, 2ty+1 and centroids 4tx..4tx+3 of dimension c
// as one 8-byte and one 16-byte LDS read (the 16 tx of a wave cover 256 consecutive bytes). Rows padded by 4
// floats: the staging writes (consecutive lanes = consecutive dimensions of one row) then spread over 16 banks
// instead of 1-2, and rows stay 16-byte aligned for the reads.
struct TileSmem {
    float xs[kSlice][kTileQ + 4];
    float cs[kSlice][kTileL + 4];
};

// acc[i][j] = distance of row q0 + 2ty + i to centroid l0 + 4tx + j over all d dimensions. Rows past nq and
// centroids past nlist are staged as zeros and give values the callers never use.
__device__ __forceinline__ void tile_sums(const float* __restrict__ x, int64_t nq, const float* __restrict__ coarse,
                                          int64_t nlist, int d, int64_t q0, int64_t l0, TileSmem& sm,
                                          float (&acc)[2][4]) {
#pragma clang fp contract(off)
    const int tid = threadIdx.x, ty = tid / 16, tx = tid % 16;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
    for (int j0 = 0; j0 < d; j0 += kSlice) {
        for (int e = tid; e < kTileQ * kSlice; e += kThreads) {
            const int r = e / kSlice, c = e % kSlice, j = j0 + c;
            const int64_t qr = q0 + r;
            sm.xs[c][r] = (qr < nq && j < d) ? x[qr * d + j] : 0.f;
        }
        for (int e = tid; e < kTileL * kSlice; e += kThreads) {
            const int r = e / kSlice, c = e % kSlice, j = j0 + c;
            const int64_t lr = l0 + r;
            sm.cs[c][r] = (lr < nlist && j < d) ? coarse[lr * d + j] : 0.f;
        }
        __syncthreads();
        const int width = min(kSlice, d - j0);
        for (int c = 0; c < width; ++c) {
            const float2 xv = *reinterpret_cast<const float2*>(&sm.xs[c][2 * ty]);
            const float4 cv = *reinterpret_cast<const float4*>(&sm.cs[c][4 * tx]);
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
}

__global__ void __launch_bounds__(kThreads) coarse_distance_kernel(const float* __restrict__ queries, int64_t nq,
                                                                  const float* __restrict__ coarse, int64_t nlist,
                                                                  int d, float* __restrict__ out) {
    __shared__ __align__(16) TileSmem sm;
    const int tid = threadIdx.x, ty = tid / 16, tx = tid % 16;
    const int64_t q0 = static_cast<int64_t>(blockIdx.y) * kTileQ, l0 = static_cast<int64_t>(blockIdx.x) * kTileL;
    float acc[2][4];
    tile_sums(queries, nq, coarse, nlist, d, q0, l0, sm, acc);
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

// (dist, id) order of the search's results: the smaller distance, the lower id on equal distances. A NaN distance
// never wins.
__device__ __forceinline__ bool closer(float d, int id, float bd, int bi) { return d < bd || (d == bd && id < bi); }

// One block per 32 vectors, looping over all centroid tiles: the nearest centroid of each vector by (dist, id).
// Each thread keeps the best of the centroids it summed for its two rows; the 16 threads sharing a row (16
// consecutive lanes of one wave) then reduce by lane exchanges. A vector whose every distance is NaN gets list 0.
__global__ void __launch_bounds__(kThreads) coarse_assign_kernel(const float* __restrict__ x, int64_t n,
                                                                const float* __restrict__ coarse, int64_t nlist,
                                                                int d, int32_t* __restrict__ list_ids) {
    __shared__ __align__(16) TileSmem sm;
    const int tid = threadIdx.x, ty = tid / 16, tx = tid % 16;
    const int64_t q0 = static_cast<int64_t>(blockIdx.x) * kTileQ;
    float best_d[2] = {__builtin_inff(), __builtin_inff()};
    int best_i[2] = {INT_MAX, INT_MAX};
    float acc[2][4];
    for (int64_t l0 = 0; l0 < nlist; l0 += kTileL) {
        tile_sums(x, n, coarse, nlist, d, q0, l0, sm, acc);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t l = l0 + 4 * tx + j;
            if (l >= nlist) continue;
#pragma unroll
            for (int i = 0; i < 2; ++i)
                if (closer(acc[i][j], static_cast<int>(l), best_d[i], best_i[i])) {
                    best_d[i] = acc[i][j];
                    best_i[i] = static_cast<int>(l);
                }
        }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int mask = 8; mask >= 1; mask >>= 1) {
            const float od = __shfl_xor(best_d[i], mask);
            const int oi = __shfl_xor(best_i[i], mask);
            if (closer(od, oi, best_d[i], best_i[i])) {
                best_d[i] = od;
                best_i[i] = oi;
            }
        }
        const int64_t q = q0 + 2 * ty + i;
        if (tx == 0 && q < n) list_ids[q] = best_i[i] == INT_MAX ? 0 : best_i[i];
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

hipError_t launch_coarse_assign(const float* x, int64_t n, const float* coarse, int64_t nlist, int d,
                                int32_t* list_ids, hipStream_t stream) {
    if (n <= 0 || nlist <= 0 || nlist >= INT_MAX || d <= 0 || (n + kTileQ - 1) / kTileQ > INT_MAX)
        return hipErrorInvalidValue;
    const unsigned grid = static_cast<unsigned>((n + kTileQ - 1) / kTileQ);
    hipLaunchKernelGGL(coarse_assign_kernel, dim3(grid), dim3(kThreads), 0, stream, x, n, coarse, nlist, d, list_ids);
    return hipGetLastError();
}

}  // namespace vk
