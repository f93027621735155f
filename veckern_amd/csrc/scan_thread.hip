// The registry's earlier variants, kept so every ScanVariant of the reference's API runs (reference:
// kernels.cuh:42-109 for v0-v3, :207-382 for v4-v7; launches searcher.cu:258-362), written for gfx950:
//   v0 GlobalLut     LUT read from global memory (cached), row-major byte codes, one thread per vector
//   v1 SharedLut     LUT staged in LDS
//   v2 SharedLutVec  16-byte row loads (m % 16 == 0)
//   v3 Interleaved   byte-interleaved wave64 tiles: code s of 64 consecutive vectors is 64 contiguous bytes
//   v4 Fused         not launched: its run-time-indexed per-thread list faulted the GPU with a memory-aperture
//                    violation whose cause is not established; the host rejects v4 before any launch
//   v5 FusedReg      per-thread list updated with compile-time indices only, so it stays in registers
//   v6 FusedVec      v5 over 16-byte-word-interleaved tiles, ILP vectors per thread per step
//   v7 FusedVecMQ    v6 with Q queries per block sharing each code load (Q * K <= 64)
// v0-v3 write the nq x n distance matrix, reduced by the select kernel; v5-v7 emit one partial K-list per
// (query, block), reduced by the select kernel. Distances are summed in sub-space order s = 0..m-1 from 0.f,
// like the CPU reference, so every variant is bit-exact against it.
#include "kernels.hpp"

namespace vk {

// ---------------------------------------------------------------- v0 - v3

template <int V>
__global__ void __launch_bounds__(1024) scan_kernel(ScanArgs a) {
    extern __shared__ __align__(16) float table_lds[];
    const int m = a.m;
    const float* table = a.lut + static_cast<int64_t>(blockIdx.y) * m * KSUB;
    if constexpr (V != 0) {
        for (int j = threadIdx.x; j < m * KSUB; j += blockDim.x) table_lds[j] = table[j];
        __syncthreads();
        table = table_lds;
    }
    float* out = a.dists + static_cast<int64_t>(blockIdx.y) * a.n;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < a.n; i += stride) {
        float acc = 0.f;
        if constexpr (V == 0 || V == 1) {
            const uint8_t* row = a.codes + i * m;
            for (int s = 0; s < m; ++s) acc += table[s * KSUB + row[s]];
        } else if constexpr (V == 2) {
            const uint4* row = reinterpret_cast<const uint4*>(a.codes + i * m);
            for (int w = 0; w < m / 16; ++w) {
                const uint4 v = row[w];
                const uint32_t part[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int j = 0; j < 16; ++j) acc += table[(w * 16 + j) * KSUB + ((part[j >> 2] >> (8 * (j & 3))) & 0xffu)];
            }
        } else {
            const uint8_t* tile = a.codes_il + (i >> 6) * m * WAVE + (i & 63);
            for (int s = 0; s < m; ++s) acc += table[s * KSUB + tile[s * WAVE]];
        }
        out[i] = acc;
    }
}

hipError_t launch_scan(int variant, const ScanArgs& a, int blocks_x, int nq, int threads, hipStream_t stream) {
    const dim3 grid(blocks_x, nq);
    const size_t smem = variant == 0 ? 0 : static_cast<size_t>(a.m) * KSUB * sizeof(float);
    switch (variant) {
        case 0: hipLaunchKernelGGL(scan_kernel<0>, grid, dim3(threads), smem, stream, a); break;
        case 1:
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&scan_kernel<1>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem));
            hipLaunchKernelGGL(scan_kernel<1>, grid, dim3(threads), smem, stream, a);
            break;
        case 2:
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&scan_kernel<2>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem));
            hipLaunchKernelGGL(scan_kernel<2>, grid, dim3(threads), smem, stream, a);
            break;
        case 3:
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&scan_kernel<3>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem));
            hipLaunchKernelGGL(scan_kernel<3>, grid, dim3(threads), smem, stream, a);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------- v5 - v7: per-thread register lists

// Sorted insertion with compile-time indices only (v5-v7): new[j] is old[j-1] when x precedes old[j-1], else x
// when x precedes old[j], else old[j]; computed from the back so old[j-1] is still unchanged.
template <int K>
__device__ __forceinline__ void insert_registers(float (&d)[K], int32_t (&id)[K], float x, int32_t xi) {
    if (!pair_less(x, xi, d[K - 1], id[K - 1])) return;
#pragma unroll
    for (int j = K - 1; j > 0; --j) {
        const bool moves = pair_less(x, xi, d[j - 1], id[j - 1]);
        const bool here = pair_less(x, xi, d[j], id[j]);
        const float nd = moves ? d[j - 1] : (here ? x : d[j]);
        const int32_t ni = moves ? id[j - 1] : (here ? xi : id[j]);
        d[j] = nd;
        id[j] = ni;
    }
    if (pair_less(x, xi, d[0], id[0])) {
        d[0] = x;
        id[0] = xi;
    }
}

// grid (blocks_x, ceil(nq / Q)), 256 threads. WORDS: word-interleaved codes (else byte-interleaved). U vectors
// per thread per step (i, i + stride, ...). Each thread keeps Q register lists of K entries.
template <int K, int Q, int U, bool WORDS>
__global__ void __launch_bounds__(256) fused_thread_kernel_t(ThreadScanArgs a) {
    constexpr int T = 256, W = T / WAVE, S = K <= WAVE ? 1 : 2;
    extern __shared__ __align__(16) unsigned char smem[];
    float* tables = reinterpret_cast<float*>(smem);
    const int m = a.m, tsize = m * KSUB;
    const int tid = threadIdx.x, wave = tid / WAVE;
    const int64_t q0 = static_cast<int64_t>(blockIdx.y) * Q;
    for (int j = tid; j < Q * tsize; j += T) tables[j] = a.lut[q0 * tsize + j];  // LUT padded to a multiple of Q
    __syncthreads();

    float kd[Q][K];
    int32_t ki[Q][K];
#pragma unroll
    for (int q = 0; q < Q; ++q)
#pragma unroll
        for (int j = 0; j < K; ++j) {
            kd[q][j] = INFINITY;
            ki[q][j] = kEmptyId;
        }

    const int64_t stride = static_cast<int64_t>(gridDim.x) * T;
    for (int64_t i0 = static_cast<int64_t>(blockIdx.x) * T + tid; i0 < a.n; i0 += stride * U) {
        float acc[U][Q];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t i = i0 + u * stride;
#pragma unroll
            for (int q = 0; q < Q; ++q) acc[u][q] = 0.f;
            if (i >= a.n) continue;
            if constexpr (WORDS) {
                const int words = m / 16;
                const uint4* tile = a.codes_v + (i >> 6) * words * WAVE + (i & 63);
                for (int w = 0; w < words; ++w) {
                    const uint4 v = tile[w * WAVE];  // one 16-byte load serves all Q queries
                    const uint32_t part[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int j = 0; j < 16; ++j) {
                        const int c = static_cast<int>((part[j >> 2] >> (8 * (j & 3))) & 0xffu);
#pragma unroll
                        for (int q = 0; q < Q; ++q) acc[u][q] += tables[q * tsize + (w * 16 + j) * KSUB + c];
                    }
                }
            } else {
                const uint8_t* tile = a.codes_il + (i >> 6) * m * WAVE + (i & 63);
                for (int s = 0; s < m; ++s) {
                    const int c = tile[s * WAVE];
#pragma unroll
                    for (int q = 0; q < Q; ++q) acc[u][q] += tables[q * tsize + s * KSUB + c];
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t i = i0 + u * stride;
            if (i >= a.n) continue;
#pragma unroll
            for (int q = 0; q < Q; ++q) {
                insert_registers<K>(kd[q], ki[q], acc[u][q], static_cast<int32_t>(i));
            }
        }
    }

    // Block merge: the 64 lists of a wave go into one wave list (entry j of every lane at a time; each lane's
    // entries ascend and the threshold only falls, so once no lane's entry j is admitted none of its later
    // entries is), then the W wave lists are merged by rank.
    Pair* buf = reinterpret_cast<Pair*>(smem);
    Pair* merged = buf + W * K;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        WaveList<S> wl;
        wl.init();
#pragma unroll
        for (int j = 0; j < K; ++j) {
            const bool valid = ki[q][j] != kEmptyId;
            if (__ballot(valid && kd[q][j] <= wl.thr_d) == 0) break;
            wl.offer(kd[q][j], ki[q][j], valid, K);
        }
        __syncthreads();  // the tables (first query) or the previous query's merge are done with LDS
        wl.store(buf + wave * K, K);
        __syncthreads();
        merge_lists(buf, W, K, merged, tid, T);
        __syncthreads();
        if (q0 + q < a.nq) {
            Pair* dst = a.part + ((q0 + q) * gridDim.x + blockIdx.x) * static_cast<int64_t>(K);
            for (int j = tid; j < K; j += T) dst[j] = merged[j];
        }
    }
}

template <int K, int Q, int U, bool WORDS>
hipError_t launch_fused_thread_t(const ThreadScanArgs& a, dim3 grid, size_t smem, hipStream_t stream) {
    hipLaunchKernelGGL((fused_thread_kernel_t<K, Q, U, WORDS>), grid, dim3(256), smem, stream, a);
    return hipGetLastError();
}

template <int K, int Q, int U, bool WORDS>
ThreadScanKernel make_thread_kernel() {
    ThreadScanKernel k;
    k.fn = reinterpret_cast<const void*>(&fused_thread_kernel_t<K, Q, U, WORDS>);
    k.threads = 256;
    k.launch = &launch_fused_thread_t<K, Q, U, WORDS>;
    return k;
}

template <int K, int Q>
ThreadScanKernel vec_kernel(int ilp) {
    if (ilp == 4) return make_thread_kernel<K, Q, 4, true>();
    if (ilp == 2) return make_thread_kernel<K, Q, 2, true>();
    return make_thread_kernel<K, Q, 1, true>();
}

template <int K>
ThreadScanKernel thread_kernel_for_k(int variant, int q, int ilp) {
    if (variant == 4) return ThreadScanKernel{};  // v4 is not launched (see the header of this file)
    if (variant == 5) return make_thread_kernel<K, 1, 1, false>();
    if (variant == 6 || q <= 1) return vec_kernel<K, 1>(ilp);
    if constexpr (K <= 8) {
        if (q >= 8) return vec_kernel<K, 8>(ilp);
    }
    if constexpr (K <= 16) {
        if (q >= 4) return vec_kernel<K, 4>(ilp);
    }
    if constexpr (K <= 32) {
        if (q >= 2) return vec_kernel<K, 2>(ilp);
    }
    return vec_kernel<K, 1>(ilp);
}

ThreadScanKernel fused_thread_kernel(int variant, int K, int q, int ilp) {
    switch (K) {
        case 8: return thread_kernel_for_k<8>(variant, q, ilp);
        case 16: return thread_kernel_for_k<16>(variant, q, ilp);
        case 32: return thread_kernel_for_k<32>(variant, q, ilp);
        case 64: return thread_kernel_for_k<64>(variant, q, ilp);
        case 128: return thread_kernel_for_k<128>(variant, q, ilp);
        default: return ThreadScanKernel{};
    }
}

}  // namespace vk
