// The fused scans' code layout built on the GPU: the same slot order and table rows as slot_order.hpp (vectors
// sorted by their first four code bytes, table rows fitted to the sorted passes' co-occurrences, full 256-slot
// blocks dealt over their passes by bank group where that pays, tiles spread, ids interleaved), slot for slot.
// The sort is a stable radix sort of (key, id) pairs; the co-occurrence counts of the sampled blocks are
// accumulated with atomics; the fit of the rows (a few milliseconds per sub-space) runs on the host between the two
// launches; each block is then ordered by one wave, with its code rows, entry-present masks and bank-group counts
// in LDS.
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>

#include <type_traits>

#include "kernels.hpp"
#include "slot_order.hpp"

namespace vk {
namespace {

constexpr int kBlockSlots = static_cast<int>(order::kBlock);  // 256 slots: one wave step of four tiles
constexpr int kRows = order::kEntries;                         // 256 table rows per sub-space

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

// Co-occurrence counts of the sampled blocks (order::cooccurrence), upper triangle only: w[(s * 256 + a) * 256 + b]
// for a < b. One workgroup per sampled block; thread t takes the (pass, sub-space) pairs t, t + 256, ...: it gathers
// the pass's entries, keeps the distinct ones in its LDS row and adds one to every pair of them.
template <int L>
__global__ void __launch_bounds__(256) cooccurrence_kernel(const uint8_t* __restrict__ codes, int m,
                                                             const uint32_t* __restrict__ sorted, int64_t full,
                                                             int64_t samples, uint32_t* __restrict__ w) {
    __shared__ uint8_t seen[256][L];
    const int64_t i = blockIdx.x;
    if (i >= samples) return;
    const uint32_t* block = sorted + (i * full / samples) * kBlockSlots;
    uint8_t* list = seen[threadIdx.x];
    constexpr int P = kBlockSlots / L;
    for (int c = threadIdx.x; c < P * m; c += 256) {
        const int p = c / m, s = c % m;
        int k = 0;
        for (int l = 0; l < L; ++l) {
            const uint8_t e = codes[static_cast<int64_t>(block[p * L + l]) * m + s];
            bool found = false;
            for (int j = 0; j < k; ++j) found = found || list[j] == e;
            if (!found) list[k++] = e;
        }
        uint32_t* ws = w + static_cast<int64_t>(s) * kRows * kRows;
        for (int a = 0; a < k; ++a)
            for (int b = a + 1; b < k; ++b) {
                const unsigned x = list[a], y = list[b];
                atomicAdd(ws + (x < y ? x * kRows + y : y * kRows + x), 1u);
            }
    }
}

// Entry masks of a unit's passes: one bit per pass.
template <int PASSES>
using PassMask = std::conditional_t<(PASSES <= 16), uint16_t, std::conditional_t<(PASSES <= 32), uint32_t, uint64_t>>;

// One dealing unit per wave (order::order_units): POOL full blocks, or one block (the units past the pools). The
// unit's code rows are gathered into LDS. Its sorted passes' statistics (order::block_stats: the sum over (pass,
// sub-space) of the largest bank-group count of distinct entries, and the number of distinct entries) are taken by
// filling the passes in slot order with the same bookkeeping the dealing keeps: `present[s * 256 + e]` (bit p: pass p
// reads entry e of sub-space s), `count[(s * L + g) * P + p]` (pass p's distinct entries in group g of sub-space s)
// and `top[s * P + p]` (the largest such count), lane s updating sub-space s. If the unit reads at least
// kDealMinDistinct * m distinct entries per block, its vectors are dealt (order::deal_block: lane (p, s-group) sums
// pass p's cost over its sub-spaces, the wave picks the cheapest pass with room, lowest first on ties), and the dealt
// order is kept if its load is lower. The unit's ids are then written at their spread, interleaved slots. The
// partial last block: ids in sorted order.
template <int M, int L, int POOL>
__global__ void __launch_bounds__(64) order_units_kernel(const uint8_t* __restrict__ codes, int64_t n, int m,
                                                           const uint32_t* __restrict__ sorted,
                                                           const uint8_t* __restrict__ table_rows, int64_t pools,
                                                           int64_t rest_first, int64_t units, int64_t tiles,
                                                           int64_t stride, uint32_t* __restrict__ out) {
    constexpr int MM = M ? M : 64;  // LDS sized for the largest m when m is not fixed (m <= 64)
    constexpr int kMaxSlots = kBlockSlots * POOL;
    constexpr int kMaxPasses = kMaxSlots / L;  // at most 64
    static_assert(kMaxPasses <= 64, "a pass mask holds at most 64 passes");
    using Mask = PassMask<kMaxPasses>;
    constexpr unsigned kRaise = L > 16 ? 2u : 0u;  // order::raise_penalty(L)
    __shared__ uint8_t rows[kMaxSlots * MM];
    __shared__ uint8_t group[MM * kRows];
    __shared__ Mask present[MM * kRows];
    __shared__ uint8_t count[MM * L * kMaxPasses];
    __shared__ uint8_t top[MM * kMaxPasses];
    __shared__ uint16_t dealt[kMaxSlots];
    const int lane = threadIdx.x;
    const int mm = M ? M : m;
    const int64_t u = blockIdx.x;
    if (u >= units) return;
    const int64_t blk = u < pools ? u * POOL : rest_first + (u - pools);
    const int slots = u < pools ? kMaxSlots : kBlockSlots;
    const int P = slots / L;  // passes of this unit
    const int64_t b0 = blk * kBlockSlots;
    const int cnt = static_cast<int>(min<int64_t>(slots, n - b0));
    const uint32_t* block = sorted + b0;
    auto place = [&](int64_t t) {
        const int64_t slot = t < tiles * 64 ? (t / 64) * stride % tiles * 64 + t % 64 : t;
        return (slot / 64 / 4) * 256 + (slot % 64) * 4 + (slot / 64) % 4;
    };
    bool use_dealt = false;
    if (cnt == slots) {
        for (int e = lane; e < slots * mm; e += WAVE) rows[e] = codes[static_cast<int64_t>(block[e / mm]) * mm + e % mm];
        for (int e = lane; e < mm * kRows; e += WAVE) group[e] = static_cast<uint8_t>(table_rows[e] % L);
        auto reset = [&] {
            for (int e = lane; e < mm * kRows; e += WAVE) present[e] = 0;
            for (int e = lane; e < mm * L * P; e += WAVE) count[e] = 0;
            for (int e = lane; e < mm * P; e += WAVE) top[e] = 0;
        };
        // Adds row i to pass p in sub-space s = lane (one sub-space per lane); returns whether its entry is new.
        auto add = [&](int i, int p) {
            if (lane >= mm) return 0u;
            const int s = lane;
            const unsigned e = rows[i * mm + s];
            const Mask mask = present[s * kRows + e];
            if ((mask >> p) & 1u) return 0u;
            present[s * kRows + e] = static_cast<Mask>(mask | (Mask{1} << p));
            const int c = ++count[(s * L + group[s * kRows + e]) * P + p];
            if (c > top[s * P + p]) top[s * P + p] = static_cast<uint8_t>(c);
            return 1u;
        };
        auto load = [&] {  // sum of top over (sub-space, pass)
            unsigned t = 0;
            for (int e = lane; e < mm * P; e += WAVE) t += top[e];
            for (int o = WAVE / 2; o > 0; o >>= 1) t += static_cast<unsigned>(__shfl_xor(static_cast<int>(t), o));
            return t;
        };
        reset();
        __syncthreads();
        unsigned distinct = 0;
        for (int i = 0; i < slots; ++i) distinct += add(i, i / L);  // lane s touches sub-space s only
        __syncthreads();
        for (int o = WAVE / 2; o > 0; o >>= 1) distinct += static_cast<unsigned>(__shfl_xor(static_cast<int>(distinct), o));
        const unsigned sorted_load = load();
        // The dealing, with the unit's pass count PP a compile-time constant (the cost loop then unrolls over a
        // fixed m and keeps its table reads in flight together).
        auto deal = [&](auto pc) {
            constexpr int PP = decltype(pc)::value;
            const int p = lane % PP, s0 = lane / PP;  // this lane's pass and first sub-space
            constexpr int kStep = WAVE / PP;
            int fill = 0;                            // lanes of pass p: vectors dealt to it so far
            for (int i = 0; i < PP * L; ++i) {
                const uint8_t* row = rows + i * mm;
                auto cost_of = [&](int s) {
                    const unsigned e = row[s];
                    const unsigned c = count[(s * L + group[s * kRows + e]) * PP + p];
                    const unsigned t = top[s * PP + p];
                    const bool there = (present[s * kRows + e] >> p) & 1u;
                    return there ? 0u : c + (c + 1u > (t > 1u ? t : 1u) ? kRaise : 0u);
                };
                unsigned cost = 0;
                if constexpr (M > 0) {
#pragma unroll
                    for (int k = 0; k < (M + kStep - 1) / kStep; ++k)
                        if (s0 + k * kStep < M) cost += cost_of(s0 + k * kStep);
                } else {
                    for (int s = s0; s < mm; s += kStep) cost += cost_of(s);
                }
#pragma unroll
                for (int o = PP; o < WAVE; o <<= 1) cost += static_cast<unsigned>(__shfl_xor(static_cast<int>(cost), o));
                // Cheapest pass with room, lowest pass on ties: the minimum of (cost, pass) over passes with room.
                unsigned key = fill < L ? (cost << 6) | static_cast<unsigned>(p) : 0xffffffffu;
#pragma unroll
                for (int o = 1; o < PP; o <<= 1) {
                    const unsigned other = static_cast<unsigned>(__shfl_xor(static_cast<int>(key), o));
                    key = other < key ? other : key;
                }
                const int best = static_cast<int>(key & 63u);
                const int at = __shfl(fill, best);  // the best pass's fill before this vector (lane best: pass best)
                __syncthreads();                    // every lane has read present / count / top for this vector
                add(i, best);
                if (lane == 0) dealt[best * L + at] = static_cast<uint16_t>(i);
                if (p == best) ++fill;
                __syncthreads();
            }
        };
        if (distinct >= order::kDealMinDistinct * static_cast<unsigned>(mm) * static_cast<unsigned>(slots / kBlockSlots)) {
            __syncthreads();
            reset();
            __syncthreads();
            if (slots == kMaxSlots) deal(std::integral_constant<int, kMaxPasses>{});
            else deal(std::integral_constant<int, kBlockSlots / L>{});
            use_dealt = load() < sorted_load;
        }
    }
    __syncthreads();
    for (int j = lane; j < cnt; j += WAVE) out[place(b0 + j)] = block[use_dealt ? dealt[j] : j];
}

template <int M, int L, int POOL>
hipError_t launch_order_units(const uint8_t* codes, int64_t n, int m, const uint32_t* sorted, const uint8_t* rows,
                              const order::Units& un, int64_t tiles, int64_t stride, uint32_t* out,
                              hipStream_t stream) {
    hipLaunchKernelGGL((order_units_kernel<M, L, POOL>), dim3(static_cast<unsigned>(un.count)), dim3(64), 0, stream,
                       codes, n, m, sorted, rows, static_cast<int64_t>(un.pools), static_cast<int64_t>(un.rest_first),
                       static_cast<int64_t>(un.count), tiles, stride, out);
    return hipGetLastError();
}

// The instance of the pool order::pool_blocks gives for this m (fixed, or up to 64) and pass width.
template <int M, int L>
hipError_t launch_order_units_pool(const uint8_t* codes, int64_t n, int m, const uint32_t* sorted,
                                   const uint8_t* rows, const order::Units& un, int64_t tiles, int64_t stride,
                                   uint32_t* out, hipStream_t stream) {
    constexpr int kPool = order::pool_blocks(M ? M : 64, L);  // m not fixed: sized as m = 64, like pool_blocks
    if (static_cast<int>(un.pool) != kPool) return hipErrorInvalidValue;
    return launch_order_units<M, L, kPool>(codes, n, m, sorted, rows, un, tiles, stride, out, stream);
}

template <int L>
hipError_t launch_order_units_m(const uint8_t* codes, int64_t n, int m, const uint32_t* sorted, const uint8_t* rows,
                                const order::Units& un, int64_t tiles, int64_t stride, uint32_t* out,
                                hipStream_t stream) {
    switch (m) {
        case 16: return launch_order_units_pool<16, L>(codes, n, m, sorted, rows, un, tiles, stride, out, stream);
        case 32: return launch_order_units_pool<32, L>(codes, n, m, sorted, rows, un, tiles, stride, out, stream);
        case 64: return launch_order_units_pool<64, L>(codes, n, m, sorted, rows, un, tiles, stride, out, stream);
        default: return launch_order_units_pool<0, L>(codes, n, m, sorted, rows, un, tiles, stride, out, stream);
    }
}

// Scratch of the slot order: the radix sort's temporary storage first (at the allocation's aligned start), then keys,
// ids, sorted keys and sorted ids (n words each), then the co-occurrence counts (m * 256 * 256 words).
size_t sort_temp_bytes(int64_t n, hipError_t* e) {
    size_t sort_bytes = 0;
    *e = hipcub::DeviceRadixSort::SortPairs(nullptr, sort_bytes, static_cast<const uint32_t*>(nullptr),
                                            static_cast<uint32_t*>(nullptr), static_cast<const uint32_t*>(nullptr),
                                            static_cast<uint32_t*>(nullptr), static_cast<int>(n), 0, 32);
    return (sort_bytes + 255) / 256 * 256;
}

struct ScratchParts {
    void* temp;
    size_t temp_bytes;
    uint32_t *keys, *ids, *keys_sorted, *sorted, *counts;
};

hipError_t scratch_parts(void* scratch, size_t scratch_bytes, int64_t n, int m, ScratchParts* sp) {
    hipError_t e;
    sp->temp_bytes = sort_temp_bytes(n, &e);
    if (e != hipSuccess) return e;
    const size_t words = (4 * static_cast<size_t>(n) + 63) / 64 * 64;
    if (scratch_bytes < sp->temp_bytes + (words + static_cast<size_t>(m) * kRows * kRows) * sizeof(uint32_t))
        return hipErrorInvalidValue;
    sp->temp = scratch;
    sp->keys = reinterpret_cast<uint32_t*>(static_cast<unsigned char*>(scratch) + sp->temp_bytes);
    sp->ids = sp->keys + n;
    sp->keys_sorted = sp->ids + n;
    sp->sorted = sp->keys_sorted + n;
    sp->counts = sp->keys + words;
    return hipSuccess;
}

}  // namespace

hipError_t slot_order_scratch_bytes(int64_t n, int m, size_t* bytes) {
    hipError_t e;
    const size_t words = (4 * static_cast<size_t>(n) + 63) / 64 * 64;
    *bytes = sort_temp_bytes(n, &e) + (words + static_cast<size_t>(m) * kRows * kRows) * sizeof(uint32_t);
    return e;
}

hipError_t launch_slot_sort(const uint8_t* codes, int64_t n, int m, int lanes, void* scratch, size_t scratch_bytes,
                            const uint32_t** counts, hipStream_t stream) {
    if (n <= 0 || m <= 0 || m > 64 || n > (int64_t{1} << 31) - 1 || (lanes != 16 && lanes != 32 && lanes != 64))
        return hipErrorInvalidValue;
    ScratchParts sp;
    hipError_t e = scratch_parts(scratch, scratch_bytes, n, m, &sp);
    if (e != hipSuccess) return e;
    const int64_t grid = std::min<int64_t>((n + 255) / 256, 65535);
    hipLaunchKernelGGL(slot_keys_kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0, stream, codes, n, m, sp.keys,
                       sp.ids);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    e = hipcub::DeviceRadixSort::SortPairs(sp.temp, sp.temp_bytes, sp.keys, sp.keys_sorted, sp.ids, sp.sorted,
                                           static_cast<int>(n), 0, 32, stream);
    if (e != hipSuccess) return e;
    e = launch_zero_words(sp.counts, static_cast<int64_t>(m) * kRows * kRows, stream);
    if (e != hipSuccess) return e;
    const int64_t full = n / kBlockSlots;
    const int64_t samples = static_cast<int64_t>(order::sample_count(static_cast<size_t>(full)));
    if (samples > 0) {
        if (lanes == 16)
            hipLaunchKernelGGL(cooccurrence_kernel<16>, dim3(static_cast<unsigned>(samples)), dim3(256), 0, stream,
                               codes, m, sp.sorted, full, samples, sp.counts);
        else if (lanes == 32)
            hipLaunchKernelGGL(cooccurrence_kernel<32>, dim3(static_cast<unsigned>(samples)), dim3(256), 0, stream,
                               codes, m, sp.sorted, full, samples, sp.counts);
        else
            hipLaunchKernelGGL(cooccurrence_kernel<64>, dim3(static_cast<unsigned>(samples)), dim3(256), 0, stream,
                               codes, m, sp.sorted, full, samples, sp.counts);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    *counts = sp.counts;
    return hipSuccess;
}

hipError_t launch_slot_place(const uint8_t* codes, int64_t n, int m, int64_t n_pad, int lanes, void* scratch,
                             size_t scratch_bytes, const uint8_t* rows, uint32_t* out, hipStream_t stream) {
    if (n <= 0 || m <= 0 || m > 64 || n > (int64_t{1} << 31) - 1 || n_pad < n ||
        (lanes != 16 && lanes != 32 && lanes != 64))
        return hipErrorInvalidValue;
    ScratchParts sp;
    hipError_t e = scratch_parts(scratch, scratch_bytes, n, m, &sp);
    if (e != hipSuccess) return e;
    e = launch_zero_words(out, n_pad, stream);  // padding slots [n, n_pad) hold 0
    if (e != hipSuccess) return e;
    const int64_t tiles = n / kBlockSlots * (kBlockSlots / 64);
    const int64_t stride = static_cast<int64_t>(order::spread_stride(static_cast<size_t>(tiles)));
    const order::Units units(static_cast<size_t>(n), order::pool_blocks(static_cast<size_t>(m), lanes));
    if (lanes == 16) return launch_order_units_m<16>(codes, n, m, sp.sorted, rows, units, tiles, stride, out, stream);
    if (lanes == 32) return launch_order_units_m<32>(codes, n, m, sp.sorted, rows, units, tiles, stride, out, stream);
    return launch_order_units_m<64>(codes, n, m, sp.sorted, rows, units, tiles, stride, out, stream);
}

}  // namespace vk
