// Exact squared L2 distances between vectors and the coarse centroids of an inverted-file index, sum_j (x[j] -
// coarse_l[j])^2 with j in order from 0.f and a separate multiply and add: the arithmetic of the reference's l2sq
// (common.hpp:27-34), so a selection by (dist, id) over them picks exactly the lists the CPU would. Two uses:
//  - the probe of a search: the dense (query x list) matrix, followed by the row top-nprobe kernel;
//  - list assignment while building an index: the nearest list of each vector (nprobe = 1), reduced inside the
//    kernel, so the n x nlist matrix is never written.
//
// The matrix is computed in tiles: the block stages 64-dimension slices of its vector rows and centroid rows in LDS,
// and each of the 256 threads keeps a block of running sums in registers (assignment: 32 x 64 tiles, 2 x 4 sums per
// thread from one 8-byte and one 16-byte LDS value per dimension; probe: 32 x 32 tiles, 2 x 2 sums). A wave per vector over all centroids (what the exact
// re-rank kernel would do) reads each centroid row from L2 once per vector and leaves most of the GPU idle at a
// few thousand queries.
#include <climits>

#include "kernels.hpp"

namespace vk {

namespace {

constexpr int kSlice = 64;    // dimensions staged per LDS pass
constexpr int kThreads = 256;

// Tiles of 16 RQ vector rows x 16 CJ centroids: thread (ty, tx) of the 16 x 16 grid keeps an RQ x CJ block of running
// sums. Slices stored dimension-major: the thread reads its rows RQ ty .. and centroids CJ tx .. of dimension c as
// one RQ- and one CJ-float LDS read (the 16 tx of a wave cover consecutive bytes). Rows padded by 4 floats: the
// staging writes (consecutive lanes = consecutive dimensions of one row) then spread over 16 banks instead of 1-2,
// and rows stay 16-byte aligned for the reads.
template <int RQ, int CJ>
struct Tile {
    static constexpr int kQ = 16 * RQ, kL = 16 * CJ;
    float xs[kSlice][kQ + 4];
    float cs[kSlice][kL + 4];
};
template <int N>
struct Floats;
template <>
struct Floats<1> {
    using T = float;
    __device__ static void get(const T& v, float (&a)[1]) { a[0] = v; }
};
template <>
struct Floats<2> {
    using T = float2;
    __device__ static void get(const T& v, float (&a)[2]) { a[0] = v.x; a[1] = v.y; }
};
template <>
struct Floats<4> {
    using T = float4;
    __device__ static void get(const T& v, float (&a)[4]) { a[0] = v.x; a[1] = v.y; a[2] = v.z; a[3] = v.w; }
};

// acc[i][j] = distance of row q0 + RQ ty + i to centroid l0 + CJ tx + j over all d dimensions. Rows past nq and
// centroids past nlist are staged as zeros and give values the callers never use.
template <int RQ, int CJ>
__device__ __forceinline__ void tile_sums(const float* __restrict__ x, int64_t nq, const float* __restrict__ coarse,
                                          int64_t nlist, int d, int64_t q0, int64_t l0, Tile<RQ, CJ>& sm,
                                          float (&acc)[RQ][CJ]) {
#pragma clang fp contract(off)
    constexpr int kQ = Tile<RQ, CJ>::kQ, kL = Tile<RQ, CJ>::kL;
    const int tid = threadIdx.x, ty = tid / 16, tx = tid % 16;
#pragma unroll
    for (int i = 0; i < RQ; ++i)
#pragma unroll
        for (int j = 0; j < CJ; ++j) acc[i][j] = 0.f;
    for (int j0 = 0; j0 < d; j0 += kSlice) {
        for (int e = tid; e < kQ * kSlice; e += kThreads) {
            const int r = e / kSlice, c = e % kSlice, j = j0 + c;
            const int64_t qr = q0 + r;
            sm.xs[c][r] = (qr < nq && j < d) ? x[qr * d + j] : 0.f;
        }
        for (int e = tid; e < kL * kSlice; e += kThreads) {
            const int r = e / kSlice, c = e % kSlice, j = j0 + c;
            const int64_t lr = l0 + r;
            sm.cs[c][r] = (lr < nlist && j < d) ? coarse[lr * d + j] : 0.f;
        }
        __syncthreads();
        const int width = min(kSlice, d - j0);
        for (int c = 0; c < width; ++c) {
            float xa[RQ], ca[CJ];
            Floats<RQ>::get(*reinterpret_cast<const typename Floats<RQ>::T*>(&sm.xs[c][RQ * ty]), xa);
            Floats<CJ>::get(*reinterpret_cast<const typename Floats<CJ>::T*>(&sm.cs[c][CJ * tx]), ca);
#pragma unroll
            for (int i = 0; i < RQ; ++i)
#pragma unroll
                for (int j = 0; j < CJ; ++j) {
                    const float diff = xa[i] - ca[j];
                    acc[i][j] += diff * diff;
                }
        }
        __syncthreads();
    }
}

// The probe's tiles: 2 x 2 sums per thread (32 x 32 per block), half the assignment's 2 x 4, so that a search's
// thousand queries give every CU four blocks instead of two (1000 queries x 1024 lists: 1024 blocks; the probe
// stage 0.048 -> 0.044 ms; 1 x 4 per thread gave 0.046).
constexpr int kProbeRQ = 2, kProbeCJ = 2;

__global__ void __launch_bounds__(kThreads) coarse_distance_kernel(const float* __restrict__ queries, int64_t nq,
                                                                  const float* __restrict__ coarse, int64_t nlist,
                                                                  int d, float* __restrict__ out) {
    __shared__ __align__(16) Tile<kProbeRQ, kProbeCJ> sm;
    const int tid = threadIdx.x, ty = tid / 16, tx = tid % 16;
    const int64_t q0 = static_cast<int64_t>(blockIdx.y) * Tile<kProbeRQ, kProbeCJ>::kQ;
    const int64_t l0 = static_cast<int64_t>(blockIdx.x) * Tile<kProbeRQ, kProbeCJ>::kL;
    float acc[kProbeRQ][kProbeCJ];
    tile_sums(queries, nq, coarse, nlist, d, q0, l0, sm, acc);
#pragma unroll
    for (int i = 0; i < kProbeRQ; ++i) {
        const int64_t q = q0 + kProbeRQ * ty + i;
        if (q >= nq) continue;
#pragma unroll
        for (int j = 0; j < kProbeCJ; ++j) {
            const int64_t l = l0 + kProbeCJ * tx + j;
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
    __shared__ __align__(16) Tile<2, 4> sm;
    const int tid = threadIdx.x, ty = tid / 16, tx = tid % 16;
    const int64_t q0 = static_cast<int64_t>(blockIdx.x) * Tile<2, 4>::kQ;
    float best_d[2] = {__builtin_inff(), __builtin_inff()};
    int best_i[2] = {INT_MAX, INT_MAX};
    float acc[2][4];
    for (int64_t l0 = 0; l0 < nlist; l0 += Tile<2, 4>::kL) {
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
    constexpr int kQ = Tile<kProbeRQ, kProbeCJ>::kQ, kL = Tile<kProbeRQ, kProbeCJ>::kL;
    if (nq <= 0 || nlist <= 0 || d <= 0 || (nq + kQ - 1) / kQ > 65535) return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>((nlist + kL - 1) / kL), static_cast<unsigned>((nq + kQ - 1) / kQ));
    hipLaunchKernelGGL(coarse_distance_kernel, grid, dim3(kThreads), 0, stream, queries, nq, coarse, nlist, d, out);
    return hipGetLastError();
}

hipError_t launch_coarse_assign(const float* x, int64_t n, const float* coarse, int64_t nlist, int d,
                                int32_t* list_ids, hipStream_t stream) {
    constexpr int kQ = Tile<2, 4>::kQ;
    if (n <= 0 || nlist <= 0 || nlist >= INT_MAX || d <= 0 || (n + kQ - 1) / kQ > INT_MAX) return hipErrorInvalidValue;
    const unsigned grid = static_cast<unsigned>((n + kQ - 1) / kQ);
    hipLaunchKernelGGL(coarse_assign_kernel, dim3(grid), dim3(kThreads), 0, stream, x, n, coarse, nlist, d, list_ids);
    return hipGetLastError();
}

}  // namespace vk
