// Roofline microbenchmarks for the PQ scan (lib/libveckern_bench.so, used by bench.py):
//   - vkb_lds_floor: uniform random byte-indexed lookups into query-interleaved LDS tables, the same table
//     layout ([s][c][QG] floats), block size and LDS footprint as the fused scan, codes generated in registers
//     (no global loads). Its lookups/s is the LDS-lookup roofline the scan is measured against.
//   - vkb_lds_peak: the same 16-byte table reads with no bank conflict (each 16-lane pass of a wave64 ds_read_b128
//     touches 16 distinct 16-byte bank groups) and almost no VALU work: the LDS's own read rate, against which the
//     scan's 64-lookups-per-CU-cycle peak (256 B/clk/CU) is checked.
//   - vkb_hbm_read: 16-byte streaming reads of a large buffer (the HBM read roofline).
//   - vkb_copy: a plain copy of known size, run under rocprofv3 to calibrate FETCH_SIZE / WRITE_SIZE.
#include <hip/hip_runtime.h>

#include <cstdint>

#define VKB_EXPORT extern "C" __attribute__((visibility("default")))

namespace {

constexpr int kThreads = 512;
constexpr int kM = 16;

__device__ inline uint32_t mix32(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

template <int QG>
struct Vec;
template <>
struct Vec<1> {
    using T = float;
    __device__ static float sum(float v) { return v; }
};
template <>
struct Vec<2> {
    using T = float2;
    __device__ static float sum(float2 v) { return v.x + v.y; }
};
template <>
struct Vec<4> {
    using T = float4;
    __device__ static float sum(float4 v) { return (v.x + v.y) + (v.z + v.w); }
};

// Each lane holds 16 random code bytes; every iteration does 16 lookups (sub-spaces 0..15) and then rotates
// the bytes so the next iteration reads new random addresses. QG floats per lookup: b32 / b64 / b128 reads.
template <int QG>
__global__ void __launch_bounds__(kThreads) lds_floor_kernel(float* out, int iters) {
    __shared__ __align__(16) float table[kM * 256 * QG];
    for (int j = threadIdx.x; j < kM * 256 * QG; j += kThreads) table[j] = static_cast<float>(j & 1023) * 1e-3f;
    __syncthreads();
    const uint32_t gid = blockIdx.x * kThreads + threadIdx.x;
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) w[k] = mix32(gid * 8u + k);
    float acc = 0.f;
    using V = typename Vec<QG>::T;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int s = 0; s < kM; ++s) {
            const uint32_t c = (w[s >> 2] >> (8 * (s & 3))) & 0xffu;
            acc += Vec<QG>::sum(*reinterpret_cast<const V*>(table + (s * 256 + c) * QG));
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) w[k] = __builtin_amdgcn_alignbit(w[k], w[k], 7) ^ static_cast<uint32_t>(it);
    }
    out[gid] = acc;
}

// Conflict-free 16-byte reads: lane l of every 16-lane pass reads bank group (l + s) % 16 of sub-space s; the
// addresses are held in registers and each read's four floats are kept live by an empty asm (no adds).
__global__ void __launch_bounds__(kThreads) lds_peak_kernel(float* out, int iters) {
    __shared__ __align__(16) float table[kM * 256 * 4];
    for (int j = threadIdx.x; j < kM * 256 * 4; j += kThreads) table[j] = static_cast<float>(j & 1023) * 1e-3f;
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63;
    uint32_t addr[kM];
#pragma unroll
    for (int s = 0; s < kM; ++s) addr[s] = (s * 256u + (((lane + s) & 15u) | ((lane >> 4) << 4))) * 16u;
    float acc = 0.f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int s = 0; s < kM; ++s) {
            uint32_t a = addr[s];
            asm volatile("" : "+v"(a));
            const float4 v = *reinterpret_cast<const float4*>(reinterpret_cast<const char*>(table) + a);
            asm volatile("" ::"v"(v.x), "v"(v.y), "v"(v.z), "v"(v.w));
            if (s == 0) acc += v.x;
        }
    }
    out[blockIdx.x * kThreads + threadIdx.x] = acc;
}

__global__ void __launch_bounds__(256) hbm_read_kernel(const uint4* __restrict__ p, size_t n16, uint32_t* out) {
    uint32_t x = 0;
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n16; i += static_cast<size_t>(gridDim.x) * 256) {
        const uint4 v = p[i];
        x ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (x == 0x9e3779b9u) out[0] = x;  // keeps the loads alive; practically never written
}

__global__ void __launch_bounds__(256) copy_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t n16) {
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n16; i += static_cast<size_t>(gridDim.x) * 256)
        dst[i] = src[i];
}

int cu_count() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    return cus;
}

template <typename F>
int time_best(int reps, float* best_ms, F&& launch) {
    hipEvent_t a, b;
    if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) return 1;
    launch();  // warm-up
    if (hipDeviceSynchronize() != hipSuccess) return 1;
    *best_ms = 1e30f;
    for (int r = 0; r < reps; ++r) {
        (void)hipEventRecord(a, 0);
        launch();
        (void)hipEventRecord(b, 0);
        if (hipEventSynchronize(b) != hipSuccess) return 1;
        float ms = 0.f;
        (void)hipEventElapsedTime(&ms, a, b);
        if (ms < *best_ms) *best_ms = ms;
    }
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

}  // namespace

// Lookups per second (query-lookups: QG per LDS read) for tables of QG = 1, 2 or 4 queries. Returns 0 on success.
VKB_EXPORT int vkb_lds_floor(int qg, int iters, int reps, double* lookups_per_s, double* ms) {
    const int cus = cu_count();
    if (cus <= 0 || iters <= 0 || reps <= 0) return 1;
    void* fn = nullptr;
    if (qg == 1) fn = reinterpret_cast<void*>(&lds_floor_kernel<1>);
    else if (qg == 2) fn = reinterpret_cast<void*>(&lds_floor_kernel<2>);
    else if (qg == 4) fn = reinterpret_cast<void*>(&lds_floor_kernel<4>);
    else return 1;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kThreads, 0) != hipSuccess || per_cu < 1) return 1;
    const int grid = cus * per_cu;  // one full wave of resident blocks
    float* out = nullptr;
    if (hipMalloc(&out, static_cast<size_t>(grid) * kThreads * sizeof(float)) != hipSuccess) return 1;
    float best = 0.f;
    int rc = time_best(reps, &best, [&] {
        if (qg == 1) hipLaunchKernelGGL(lds_floor_kernel<1>, dim3(grid), dim3(kThreads), 0, 0, out, iters);
        else if (qg == 2) hipLaunchKernelGGL(lds_floor_kernel<2>, dim3(grid), dim3(kThreads), 0, 0, out, iters);
        else hipLaunchKernelGGL(lds_floor_kernel<4>, dim3(grid), dim3(kThreads), 0, 0, out, iters);
    });
    (void)hipFree(out);
    if (rc) return rc;
    const double lookups = static_cast<double>(grid) * kThreads * iters * kM * qg;
    *lookups_per_s = lookups / (best * 1e-3);
    *ms = best;
    return 0;
}

// Streaming read bandwidth over `bytes` (a multiple of 16), best of reps, in GB/s.
// Conflict-free LDS read rate in 4-byte table entries per second (four per lane per ds_read_b128). 0 on success.
VKB_EXPORT int vkb_lds_peak(int iters, int reps, double* entries_per_s) {
    const int cus = cu_count();
    if (cus <= 0 || iters <= 0 || reps <= 0) return 1;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(&lds_peak_kernel), kThreads,
                                                     0) != hipSuccess || per_cu < 1)
        return 1;
    const int grid = cus * per_cu;
    float* out = nullptr;
    if (hipMalloc(&out, static_cast<size_t>(grid) * kThreads * sizeof(float)) != hipSuccess) return 1;
    float best = 0.f;
    const int rc = time_best(reps, &best, [&] {
        hipLaunchKernelGGL(lds_peak_kernel, dim3(grid), dim3(kThreads), 0, 0, out, iters);
    });
    (void)hipFree(out);
    if (rc) return rc;
    *entries_per_s = static_cast<double>(grid) * kThreads * iters * kM * 4 / (best * 1e-3);
    return 0;
}

VKB_EXPORT int vkb_hbm_read(size_t bytes, int reps, double* gbs) {
    const int cus = cu_count();
    if (cus <= 0 || bytes < 16 || reps <= 0) return 1;
    void* buf = nullptr;
    uint32_t* out = nullptr;
    if (hipMalloc(&buf, bytes) != hipSuccess) return 1;
    if (hipMalloc(&out, sizeof(uint32_t)) != hipSuccess) {
        (void)hipFree(buf);
        return 1;
    }
    (void)hipMemset(buf, 1, bytes);
    float best = 0.f;
    const int rc = time_best(reps, &best, [&] {
        hipLaunchKernelGGL(hbm_read_kernel, dim3(cus * 4), dim3(256), 0, 0, static_cast<const uint4*>(buf), bytes / 16, out);
    });
    (void)hipFree(buf);
    (void)hipFree(out);
    if (rc) return rc;
    *gbs = static_cast<double>(bytes) / (best * 1e-3) / 1e9;
    return 0;
}

// Copies `bytes` (a multiple of 16) once per rep; reports GB/s of bytes read + written.
VKB_EXPORT int vkb_copy(size_t bytes, int reps, double* gbs) {
    const int cus = cu_count();
    if (cus <= 0 || bytes < 16 || reps <= 0) return 1;
    void *src = nullptr, *dst = nullptr;
    if (hipMalloc(&src, bytes) != hipSuccess) return 1;
    if (hipMalloc(&dst, bytes) != hipSuccess) {
        (void)hipFree(src);
        return 1;
    }
    (void)hipMemset(src, 3, bytes);
    float best = 0.f;
    const int rc = time_best(reps, &best, [&] {
        hipLaunchKernelGGL(copy_kernel, dim3(cus * 4), dim3(256), 0, 0, static_cast<const uint4*>(src),
                           static_cast<uint4*>(dst), bytes / 16);
    });
    (void)hipFree(src);
    (void)hipFree(dst);
    if (rc) return rc;
    *gbs = 2.0 * static_cast<double>(bytes) / (best * 1e-3) / 1e9;
    return 0;
}
