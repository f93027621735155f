// The fused scans' slot order built on the GPU: the same order as slot_order.hpp (vectors sorted by their first
// four code bytes, little-sharing 256-slot blocks dealt over their 16 passes by bank group, the blocks' 64-slot tiles
// spread over the layout, ids interleaved by four tiles), slot for slot. The sort is a stable radix sort of
// (key, id) pairs; each 256-slot block is then ordered by one wave, with the block's code rows, entry-present masks
// and bank-group counts in LDS.
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>

#include "kernels.hpp"
#include "slot_order.hpp"

namespace vk {
namespace {

constexpr int kBlockSlots = static_cast<int>(order::kBlock);  // 256 slots: 16 passes of 16 lanes
constexpr int kPasses = order::kPasses;
constexpr int kLanes = order::kLanes;

// keys[i]: row i's first four code bytes, big-endian (missing bytes 0); ids[i] = i.
__global__ void __launch_bounds__(256) slot_keys_kernel(const uint8_t* __restrict__ codes, int64_t n, int m,
                                                          uint32_t* __restrict__ keys, uint32_t* __restrict__ ids) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        const uint8_t* row = codes + i * m;
        uint32_t key = 0;
        for (int b = 0; b < 4; ++b) key = (key << 8) | (b < m ? row[b] : 0u);
        keys[i] = key;
        ids[i] = static_cast<uint32_t>(i);
    }
}

// Wave-wide sum of one value per lane.
__device__ __forceinline__ unsigned wave_sum(unsigned v) {
#pragma unroll
    for (int o = WAVE / 2; o > 0; o >>= 1) v += static_cast<unsigned>(__shfl_xor(static_cast<int>(v), o));
    return v;
}

// order::block_stats of the block whose rows (in LDS, [256][m]) are read in `slot_order` (local row per slot): lane l
// takes the (pass, sub-space) pairs l, l + 64, ...; returns {load, distinct} summed over the wave. Per pair, the 16
// entries are compared pairwise in registers: an entry is new when no earlier lane read it, and the largest number
// of new entries in one bank group (entry mod 16) is the running count order::block_stats takes the maximum of.
template <int M>
__device__ order::BlockStats block_stats(const uint8_t* rows, int m, const uint8_t* slot_order, int lane) {
    const int mm = M ? M : m;
    unsigned load = 0, distinct = 0;
    for (int pair = lane; pair < kPasses * mm; pair += WAVE) {
        const int p = pair / mm, s = pair % mm;
        unsigned e[kLanes];
#pragma unroll
        for (int l = 0; l < kLanes; ++l) e[l] = rows[slot_order[p * kLanes + l] * mm + s];
        unsigned fresh = 0, mx = 0;  // fresh: bit l set when lane l's entry is new
#pragma unroll
        for (int l = 0; l < kLanes; ++l) {
            bool seen = false;
            unsigned same_group = 1;
#pragma unroll
            for (int k = 0; k < l; ++k) {
                seen = seen || e[k] == e[l];
                same_group += ((fresh >> k) & 1u) && ((e[k] ^ e[l]) & 15u) == 0 ? 1u : 0u;
            }
            if (!seen) {
                fresh |= 1u << l;
                ++distinct;
                mx = same_group > mx ? same_group : mx;
            }
        }
        load += mx;
    }
    return {wave_sum(load), wave_sum(distinct)};
}

// One full 256-slot block per wave: the block's rows are gathered into LDS; if its sorted passes read at least
// kDealMinDistinct distinct entries per (pass, sub-space) on average, its vectors are dealt over the 16 passes
// first-fit (order::deal_block, one vector at a time: lane (p, s-group) sums pass p's cost over its sub-spaces, the
// wave picks the cheapest pass with room, lowest first on ties) and the dealt order is kept if its load is lower.
// The block's ids are then written at their spread, interleaved slots. Partial last block: ids in sorted order.
template <int M>
__global__ void __launch_bounds__(64) order_blocks_kernel(const uint8_t* __restrict__ codes, int64_t n, int m,
                                                            const uint32_t* __restrict__ sorted, int64_t blocks,
                                                            int64_t tiles, int64_t stride, uint32_t* __restrict__ out) {
    constexpr int MM = M ? M : 64;  // LDS sized for the largest m when m is not fixed (m <= 64)
    __shared__ uint8_t rows[kBlockSlots * MM];
    __shared__ uint16_t present[MM * 256];
    __shared__ uint8_t groups[MM * 16 * kPasses];
    __shared__ uint8_t local[kBlockSlots], dealt[kBlockSlots];
    const int lane = threadIdx.x;
    const int mm = M ? M : m;
    const int64_t blk = blockIdx.x;
    if (blk >= blocks) return;
    const int64_t b0 = blk * kBlockSlots;
    const int cnt = static_cast<int>(min<int64_t>(kBlockSlots, n - b0));
    const uint32_t* block = sorted + b0;
    auto place = [&](int64_t t) {
        const int64_t slot = t < tiles * 64 ? (t / 64) * stride % tiles * 64 + t % 64 : t;
        return (slot / 64 / 4) * 256 + (slot % 64) * 4 + (slot / 64) % 4;
    };
    // Slots in sorted order (every block, the partial last one included), unless the block's dealt order is kept.
    for (int i = lane; i < kBlockSlots; i += WAVE) local[i] = static_cast<uint8_t>(i);
    const uint8_t* order_used = local;
    if (cnt == kBlockSlots) {
        for (int e = lane; e < kBlockSlots * mm; e += WAVE) rows[e] = codes[static_cast<int64_t>(block[e / mm]) * mm + e % mm];
    }
    __syncthreads();
    if (cnt == kBlockSlots) {
        const order::BlockStats st = block_stats<M>(rows, mm, local, lane);
        if (st.distinct >= order::kDealMinDistinct * kPasses * mm) {
            for (int e = lane; e < mm * 256; e += WAVE) present[e] = 0;
            for (int e = lane; e < mm * 16 * kPasses; e += WAVE) groups[e] = 0;
            __syncthreads();
            const int p = lane % kPasses, s0 = lane / kPasses;  // this lane's pass and first sub-space (of 4)
            int fill = 0;                                      // lanes p: vectors dealt to pass p so far
            for (int i = 0; i < kBlockSlots; ++i) {
                const uint8_t* row = rows + i * mm;
                unsigned cost = 0;
                for (int s = s0; s < mm; s += WAVE / kPasses) {
                    const unsigned e = row[s];
                    cost += ((present[s * 256 + e] >> p) & 1u) ? 0u : groups[(s * 16 + (e & 15)) * kPasses + p];
                }
                cost += static_cast<unsigned>(__shfl_xor(static_cast<int>(cost), 16));
                cost += static_cast<unsigned>(__shfl_xor(static_cast<int>(cost), 32));
                // Cheapest pass with room, lowest pass on ties: the minimum of (cost, pass) over passes with room.
                unsigned key = fill < kLanes ? (cost << 4) | static_cast<unsigned>(p) : 0xffffffffu;
#pragma unroll
                for (int o = 1; o < kPasses; o <<= 1) {
                    const unsigned other = static_cast<unsigned>(__shfl_xor(static_cast<int>(key), o));
                    key = other < key ? other : key;
                }
                const int best = static_cast<int>(key & 15u);
                const int at = __shfl(fill, best);  // the best pass's fill before this vector
                __syncthreads();  // every lane has read present / groups for this vector
                for (int s = lane; s < mm; s += WAVE) {
                    const unsigned e = row[s];
                    const uint16_t mask = present[s * 256 + e];
                    if ((mask >> best) & 1u) continue;
                    present[s * 256 + e] = static_cast<uint16_t>(mask | (1u << best));
                    ++groups[(s * 16 + (e & 15)) * kPasses + best];
                }
                if (lane == 0) dealt[best * kLanes + at] = static_cast<uint8_t>(i);
                if (p == best) ++fill;
                __syncthreads();
            }
            if (block_stats<M>(rows, mm, dealt, lane).load < st.load) order_used = dealt;
        }
    }
    for (int j = lane; j < cnt; j += WAVE) out[place(b0 + j)] = block[order_used[j]];
}

template <int M>
hipError_t launch_order_blocks(const uint8_t* codes, int64_t n, int m, const uint32_t* sorted, int64_t blocks,
                               int64_t tiles, int64_t stride, uint32_t* out, hipStream_t stream) {
    hipLaunchKernelGGL(order_blocks_kernel<M>, dim3(static_cast<unsigned>(blocks)), dim3(64), 0, stream, codes, n, m,
                       sorted, blocks, tiles, stride, out);
    return hipGetLastError();
}

}  // namespace

// Scratch of the slot order: the radix sort's temporary storage first (at the allocation's aligned start), then keys,
// ids, sorted keys and sorted ids (n words each).
static size_t sort_temp_bytes(int64_t n, hipError_t* e) {
    size_t sort_bytes = 0;
    *e = hipcub::DeviceRadixSort::SortPairs(nullptr, sort_bytes, static_cast<const uint32_t*>(nullptr),
                                            static_cast<uint32_t*>(nullptr), static_cast<const uint32_t*>(nullptr),
                                            static_cast<uint32_t*>(nullptr), static_cast<int>(n), 0, 32);
    return (sort_bytes + 255) / 256 * 256;
}

hipError_t slot_order_scratch_bytes(int64_t n, size_t* bytes) {
    hipError_t e;
    *bytes = sort_temp_bytes(n, &e) + 4 * static_cast<size_t>(n) * sizeof(uint32_t);
    return e;
}

hipError_t launch_slot_order(const uint8_t* codes, int64_t n, int m, int64_t n_pad, void* scratch,
                             size_t scratch_bytes, uint32_t* out, hipStream_t stream) {
    if (n <= 0 || m <= 0 || m > 64 || n > (int64_t{1} << 31) - 1) return hipErrorInvalidValue;
    hipError_t e;
    size_t temp_bytes = sort_temp_bytes(n, &e);
    if (e != hipSuccess) return e;
    if (scratch_bytes < temp_bytes + 4 * static_cast<size_t>(n) * sizeof(uint32_t)) return hipErrorInvalidValue;
    void* temp = scratch;
    uint32_t* keys = reinterpret_cast<uint32_t*>(static_cast<unsigned char*>(scratch) + temp_bytes);
    uint32_t* ids = keys + n;
    uint32_t* keys_sorted = ids + n;
    uint32_t* sorted = keys_sorted + n;
    e = launch_zero_words(out, n_pad, stream);  // padding slots [n, n_pad) hold 0
    if (e != hipSuccess) return e;
    const int64_t grid = std::min<int64_t>((n + 255) / 256, 65535);
    hipLaunchKernelGGL(slot_keys_kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0, stream, codes, n, m, keys,
                       ids);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    e = hipcub::DeviceRadixSort::SortPairs(temp, temp_bytes, keys, keys_sorted, ids, sorted, static_cast<int>(n), 0,
                                           32, stream);
    if (e != hipSuccess) return e;
    const int64_t blocks = (n + kBlockSlots - 1) / kBlockSlots;
    const int64_t tiles = n / kBlockSlots * (kBlockSlots / 64);
    const int64_t stride = static_cast<int64_t>(order::spread_stride(static_cast<size_t>(tiles)));
    switch (m) {
        case 16: return launch_order_blocks<16>(codes, n, m, sorted, blocks, tiles, stride, out, stream);
        case 32: return launch_order_blocks<32>(codes, n, m, sorted, blocks, tiles, stride, out, stream);
        case 64: return launch_order_blocks<64>(codes, n, m, sorted, blocks, tiles, stride, out, stream);
        default: return launch_order_blocks<0>(codes, n, m, sorted, blocks, tiles, stride, out, stream);
    }
}

}  // namespace vk
