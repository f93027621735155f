// One-time code layout transforms, run on the GPU when a variant first needs them (reference:
// build_interleaved_bytes / build_interleaved_words, searcher.cu:103-119, formulas kernels.cuh:92-94, 238-240).
// Tiles are 64 vectors (one wave64) instead of the reference's 32. Every output element is written once, with
// coalesced stores; the strided row-major reads are a one-off cost.
#include "kernels.hpp"

namespace vk {

__global__ void __launch_bounds__(256)
    build_words_kernel(const uint8_t* __restrict__ codes, int64_t n, int words, int64_t total, uint4* __restrict__ out) {
    for (int64_t o = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; o < total;
         o += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t lane = o % WAVE, w = (o / WAVE) % words, tile = o / (static_cast<int64_t>(WAVE) * words);
        const int64_t i = tile * WAVE + lane;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (i < n) v = *reinterpret_cast<const uint4*>(codes + (i * words + w) * 16);
        out[o] = v;
    }
}

__global__ void __launch_bounds__(256)
    build_bytes_kernel(const uint8_t* __restrict__ codes, int64_t n, int m, int64_t total, uint8_t* __restrict__ out) {
    for (int64_t o = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; o < total;
         o += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t lane = o % WAVE, s = (o / WAVE) % m, tile = o / (static_cast<int64_t>(WAVE) * m);
        const int64_t i = tile * WAVE + lane;
        out[o] = i < n ? codes[i * m + s] : 0;
    }
}

static int layout_grid(int64_t total) {
    const int64_t blocks = (total + 255) / 256;
    return static_cast<int>(blocks < 4096 ? (blocks > 0 ? blocks : 1) : 4096);
}

hipError_t launch_build_words(const uint8_t* codes, int64_t n, int m, int64_t n_pad, uint4* out, hipStream_t stream) {
    const int words = m / 16;
    const int64_t total = n_pad * words;  // uint4 elements
    hipLaunchKernelGGL(build_words_kernel, dim3(layout_grid(total)), dim3(256), 0, stream, codes, n, words, total, out);
    return hipGetLastError();
}

__global__ void __launch_bounds__(256)
    build_sorted_words_kernel(const uint8_t* __restrict__ codes, int64_t n, int words, int64_t total,
                              const uint32_t* __restrict__ slot_ids, const uint8_t* __restrict__ rows,
                              uint4* __restrict__ out) {
    for (int64_t o = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; o < total;
         o += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t lane = o % WAVE, w = (o / WAVE) % words, tile = o / (static_cast<int64_t>(WAVE) * words);
        const int64_t slot = tile * WAVE + lane;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (slot < n) {
            const int64_t i = slot_ids[(tile >> 2) * 256 + lane * 4 + (tile & 3)];
            if (i < n) v = *reinterpret_cast<const uint4*>(codes + (i * words + w) * 16);  // ids are < n
            if (rows) {  // code byte j of the word (sub-space 16 w + j) -> its table row
                const uint8_t* r = rows + w * 16 * 256;
                uint32_t x[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    uint32_t y = 0;
#pragma unroll
                    for (int b = 0; b < 4; ++b)
                        y |= static_cast<uint32_t>(r[(k * 4 + b) * 256 + ((x[k] >> (8 * b)) & 0xffu)]) << (8 * b);
                    x[k] = y;
                }
                v = make_uint4(x[0], x[1], x[2], x[3]);
            }
        }
        out[o] = v;
    }
}

hipError_t launch_build_sorted_words(const uint8_t* codes, int64_t n, int m, int64_t n_pad, const uint32_t* slot_ids,
                                     const uint8_t* rows, uint4* out, hipStream_t stream) {
    const int words = m / 16;
    const int64_t total = n_pad * words;
    hipLaunchKernelGGL(build_sorted_words_kernel, dim3(layout_grid(total)), dim3(256), 0, stream, codes, n, words, total,
                       slot_ids, rows, out);
    return hipGetLastError();
}

hipError_t launch_build_bytes(const uint8_t* codes, int64_t n, int m, int64_t n_pad, uint8_t* out,
                              hipStream_t stream) {
    const int64_t total = n_pad * m;
    hipLaunchKernelGGL(build_bytes_kernel, dim3(layout_grid(total)), dim3(256), 0, stream, codes, n, m, total, out);
    return hipGetLastError();
}

// Sets count words to zero with vector stores (used where a hipMemsetAsync node is unwanted, e.g. in work a
// caller may capture into a graph).
__global__ void __launch_bounds__(256) zero_words_kernel(unsigned* __restrict__ p, int64_t count) {
    for (int64_t o = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; o < count;
         o += static_cast<int64_t>(gridDim.x) * 256)
        p[o] = 0u;
}

hipError_t launch_zero_words(unsigned* p, int64_t count, hipStream_t stream) {
    if (count <= 0) return hipSuccess;
    hipLaunchKernelGGL(zero_words_kernel, dim3(layout_grid(count)), dim3(256), 0, stream, p, count);
    return hipGetLastError();
}

}  // namespace vk
