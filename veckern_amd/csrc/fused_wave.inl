// Fused PQ scan + top-k with one wave-cooperative sorted list per (wave, query): the ScanVariant::FusedWarp
// path (reference: kernels.cuh:392-526, launch searcher.cu:365-415), designed for gfx950, and its fp16-table
// counterpart FusedWarpF16.
//
// Work decomposition. Queries are packed into slabs of QG*NG queries whose lookup tables sit together in LDS.
// A slab's work is its n vectors cut into granules of 64*U vectors (one wave step). The slabs * n_gran work
// items are split into `grid` equal contiguous ranges, one per block, with grid = resident blocks on the
// device (occupancy API), so every CU gets the same number of items and no tail wave is left. A block builds
// the tables of each slab its range touches directly in LDS from the queries and the codebook (no LUT in HBM),
// and each (block, slab) pair emits partial K-lists per query. The last block to finish a slab (a per-slab
// counter) merges the slab's partial lists into the final results, so a search is a single launch.
//
// LDS tables. A group of QG queries shares one table laid out [s][c][QG] entries, so a single ds_read_b32 /
// b64 / b128 at ((s * 256 + c) * QG * entry bytes) returns the entries of all QG queries for code byte c.
// Measured on MI355X with uniform random bytes, a wave64 ds_read_b128 costs about 12 CU cycles against 6.4 for
// b32, so 16-byte entry groups give ~2.1x the lookups per cycle of one fp32 table per query. NG groups share
// every code load. fp16 tables put 8 queries in one 16-byte read. Most of those 12 cycles are bank conflicts within
// the read's four 16-lane passes; the exhaustive scans read codes in a slot order (slot_order.hpp) that puts
// vectors sharing code bytes in the same passes (one broadcast per shared entry) and spreads the rest over the bank
// groups, and the vector ids travel beside the codes (SlotIds).
//
// Exactness. Each query's distance is summed in fp32 in sub-space order s = 0..m-1 from 0.f, exactly like the
// CPU reference (cpu_ref.cpp:46-49), so fp32-table distances are bit-identical to the CPU's and ids agree exactly
// under the (dist, id) order. fp16 tables hold each query's fp32 entries scaled by a power of two (so that the
// largest lies in [2^14, 2^15)) and rounded to nearest-even binary16; the sums stay fp32 and are scaled back
// exactly, which the CPU restatement of the fp16 path reproduces bit for bit.
#pragma once

#include <algorithm>
#include <type_traits>

#include "kernels.hpp"

namespace vk {

// acc + (binary16 in the low / high half of h2) as fma(widened half, one, acc) with `one` a binary16 1.0 the
// compiler cannot see through (opaque_half_one): the product is exact, so the single rounding equals an fp32 add of
// the widened value, and the backend selects one v_fma_mix_f32 (op_sel picks the half) instead of a conversion and
// an add. A literal 1.0 would be folded into an fadd, which has no mixed-precision form.
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float add_half_lo(float acc, uint32_t h2, _Float16 one) {
    return __builtin_fmaf(static_cast<float>(__builtin_bit_cast(half2_t, h2).x), static_cast<float>(one), acc);
}
__device__ __forceinline__ float add_half_hi(float acc, uint32_t h2, _Float16 one) {
    return __builtin_fmaf(static_cast<float>(__builtin_bit_cast(half2_t, h2).y), static_cast<float>(one), acc);
}
__device__ __forceinline__ _Float16 opaque_half_one() {
    uint32_t bits = 0x3c00u;  // binary16 1.0
    asm volatile("" : "+s"(bits));
    return __builtin_bit_cast(_Float16, static_cast<uint16_t>(bits));
}

// s_waitcnt with vmcnt(0) and the other counters at their maxima (expcnt 7, lgkmcnt 15): the gfx9 encoding of
// vmcnt in bits [3:0] and [15:14], expcnt in [6:4], lgkmcnt in [11:8].
constexpr int kWaitVmcnt0 = 0x0f70;

// One LDS read of a table entry group: QG consecutive fp32 or fp16 entries.
template <int QG, bool F16>
struct Entries {
    static constexpr int kBytes = (F16 ? 2 : 4) * QG;
    using T = std::conditional_t<
        F16,
        std::conditional_t<QG == 1, uint16_t,
                           std::conditional_t<QG == 2, uint32_t, std::conditional_t<QG == 4, uint2, uint4>>>,
        std::conditional_t<QG == 1, float, std::conditional_t<QG == 2, float2, float4>>>;
    // The first sub-space's entries: acc = entry equals the reference's 0.f + entry bit for bit, since entries
    // are sums of squares (+0 or above, never -0), and saves the zeroing and one add per query and vector.
    __device__ static void set(float* acc, const T& v) {
        if constexpr (!F16) {
            if constexpr (QG == 1) {
                acc[0] = v;
            } else if constexpr (QG == 2) {
                acc[0] = v.x;
                acc[1] = v.y;
            } else {
                acc[0] = v.x;
                acc[1] = v.y;
                acc[2] = v.z;
                acc[3] = v.w;
            }
        } else {
            auto widen = [&](int i, uint32_t h2) {  // the exact fp32 values of a pair of binary16 entries
                acc[i] = static_cast<float>(__builtin_bit_cast(half2_t, h2).x);
                acc[i + 1] = static_cast<float>(__builtin_bit_cast(half2_t, h2).y);
            };
            if constexpr (QG == 1) {
                acc[0] = static_cast<float>(__builtin_bit_cast(_Float16, v));
            } else if constexpr (QG == 2) {
                widen(0, v);
            } else if constexpr (QG == 4) {
                widen(0, v.x);
                widen(2, v.y);
            } else {
                widen(0, v.x);
                widen(2, v.y);
                widen(4, v.z);
                widen(6, v.w);
            }
        }
    }
    __device__ static void add(float* acc, const T& v, _Float16 one) {
        if constexpr (!F16) {
            if constexpr (QG == 1) {
                acc[0] += v;
            } else if constexpr (QG == 2) {
                acc[0] += v.x;
                acc[1] += v.y;
            } else {
                acc[0] += v.x;
                acc[1] += v.y;
                acc[2] += v.z;
                acc[3] += v.w;
            }
        } else {
            if constexpr (QG == 1) {
                acc[0] = add_half_lo(acc[0], static_cast<uint32_t>(v), one);
            } else if constexpr (QG == 2) {
                acc[0] = add_half_lo(acc[0], v, one);
                acc[1] = add_half_hi(acc[1], v, one);
            } else if constexpr (QG == 4) {
                // One statement per read: the scheduler places a read's accumulations (independent, one per
                // query) together, so no two dependent v_fma_mix_f32 sit back to back needing a wait state.
                // Operands as in add_half_lo/hi: src0 the binary16 half selected by op_sel, src1 fp32 1.0.
                asm("v_fma_mix_f32 %0, %4, 1.0, %0 op_sel_hi:[1,0,0]\n\t"
                    "v_fma_mix_f32 %1, %4, 1.0, %1 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
                    "v_fma_mix_f32 %2, %5, 1.0, %2 op_sel_hi:[1,0,0]\n\t"
                    "v_fma_mix_f32 %3, %5, 1.0, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
                    : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3])
                    : "v"(v.x), "v"(v.y));
            } else {
                asm("v_fma_mix_f32 %0, %8, 1.0, %0 op_sel_hi:[1,0,0]\n\t"
                    "v_fma_mix_f32 %1, %8, 1.0, %1 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
                    "v_fma_mix_f32 %2, %9, 1.0, %2 op_sel_hi:[1,0,0]\n\t"
                    "v_fma_mix_f32 %3, %9, 1.0, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
                    "v_fma_mix_f32 %4, %10, 1.0, %4 op_sel_hi:[1,0,0]\n\t"
                    "v_fma_mix_f32 %5, %10, 1.0, %5 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
                    "v_fma_mix_f32 %6, %11, 1.0, %6 op_sel_hi:[1,0,0]\n\t"
                    "v_fma_mix_f32 %7, %11, 1.0, %7 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
                    : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]), "+v"(acc[4]), "+v"(acc[5]),
                      "+v"(acc[6]), "+v"(acc[7])
                    : "v"(v.x), "v"(v.y), "v"(v.z), "v"(v.w));
            }
        }
    }
};

// Power-of-two exponent applied to one query's fp16 table: the largest fp32 entry (as raw bits; entries are
// >= 0) is brought into [2^14, 2^15), well inside binary16's range. 0 for an all-zero, infinite or NaN table.
__device__ __forceinline__ int table_shift(uint32_t max_bits) {
    if (max_bits == 0u || max_bits >= 0x7f800000u) return 0;
    const int e = max_bits >= 0x00800000u ? static_cast<int>(max_bits >> 23) - 127
                                          : -126 - (static_cast<int>(__clz(max_bits)) - 8);
    return e - 14;
}

__device__ __forceinline__ uint32_t to_half_bits(float x) {  // round to nearest even
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
}

// Byte b of w times 2^SHIFT (a table entry's byte offset) in one VALU op: the compiler selects a shift with an SDWA
// byte select for bytes 1-3 by itself, but turns byte 0 into a shift and a mask; the asm keeps byte 0 to one op as
// well (the shift amount sits in a VGPR, as SDWA requires).
template <int SHIFT>
__device__ __forceinline__ uint32_t scaled_byte(uint32_t w, int b) {
    if (b != 0) return ((w >> (8 * b)) & 0xffu) << SHIFT;
    uint32_t r;
    asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0"
        : "=v"(r)
        : "v"(static_cast<uint32_t>(SHIFT)), "v"(w));
    return r;
}

// Byte B of w times 2^SHIFT written into the low half of r, whose high half is kept (SDWA dst_sel:WORD_0 with
// dst_unused:UNUSED_PRESERVE). A DS instruction's immediate offset reaches 64 KB; with r's high half at 1, r is the
// byte's table offset plus 64 KB in one VALU op, so tables past 64 KB of LDS cost no extra add per lookup. The
// scaled byte (at most 255 << 4) fits the 16-bit half.
template <int SHIFT, int B>
__device__ __forceinline__ void scaled_byte_low_half(uint32_t& r, uint32_t w) {
    static_assert(B >= 0 && B < 4 && (255 << SHIFT) < 65536, "byte select and 16-bit result");
    const uint32_t shift = SHIFT;
    if constexpr (B == 0)
        asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:WORD_0 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:BYTE_0"
            : "+v"(r) : "v"(shift), "v"(w));
    else if constexpr (B == 1)
        asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:WORD_0 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:BYTE_1"
            : "+v"(r) : "v"(shift), "v"(w));
    else if constexpr (B == 2)
        asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:WORD_0 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:BYTE_2"
            : "+v"(r) : "v"(shift), "v"(w));
    else
        asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:WORD_0 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:BYTE_3"
            : "+v"(r) : "v"(shift), "v"(w));
}

constexpr int log2_int(int x) { return x <= 1 ? 0 : 1 + log2_int(x / 2); }

// Compile-time unrolled loop: f(std::integral_constant<int, I>) for I = 0 .. N-1.
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

// Loads n consecutive floats from p (16-byte aligned when n % 4 == 0, 8-byte aligned when n == 2) with the widest
// vector loads the alignment allows.
template <int N>
__device__ __forceinline__ void load_floats(const float* p, float* out) {
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (int j = 0; j < N; j += 4) {
            const float4 v = *reinterpret_cast<const float4*>(p + j);
            out[j] = v.x;
            out[j + 1] = v.y;
            out[j + 2] = v.z;
            out[j + 3] = v.w;
        }
    } else if constexpr (N == 2) {
        const float2 v = *reinterpret_cast<const float2*>(p);
        out[0] = v.x;
        out[1] = v.y;
    } else {
#pragma unroll
        for (int j = 0; j < N; ++j) out[j] = p[j];
    }
}

// Computes the fp32 table entries of a slab's QS queries and hands each (s, c) to sink(s, c, acc[QS]): entry (s, c)
// of query q is sum_j (x_q[s*dsub + j] - C[s][c][j])^2 with j in order and a separate multiply and add, the CPU
// reference's arithmetic (cpu_ref.cpp:7-14, common.hpp:27-34). Wave w takes sub-spaces w, w + W, ..., so the query
// values it reads are wave-uniform (scalar loads); lane l takes centroids l, l + 64, l + 128, l + 192. With the
// sub-vector width DSUB known at compile time, the four centroids' loads of a sub-space are issued together, so a
// pass costs about one memory round trip per sub-space a wave handles rather than one per element. DSUB = 0: any
// width. qrow[q]: query q's row (padded slots repeat a real query; their entries are never used).
template <int QS, int M, int W, int DSUB, typename Sink>
__device__ __forceinline__ void table_entries_w(const WaveScanArgs& a, const float* const (&qrow)[QS], int wave,
                                                int lane, Sink& sink) {
#pragma clang fp contract(off)
    constexpr int R = KSUB / WAVE;  // centroids per lane and sub-space
    const int m = M ? M : a.m;
    const int dsub = DSUB ? DSUB : a.d / m;
    for (int s = wave; s < m; s += W) {
        const float* cbase = a.centroids + static_cast<int64_t>(s) * KSUB * dsub;
        if constexpr (DSUB > 0) {
            float cv[R][DSUB];
#pragma unroll
            for (int r = 0; r < R; ++r) load_floats<DSUB>(cbase + (r * WAVE + lane) * DSUB, cv[r]);
            float qv[QS][DSUB];
#pragma unroll
            for (int q = 0; q < QS; ++q)
#pragma unroll
                for (int j = 0; j < DSUB; ++j) qv[q][j] = qrow[q][s * DSUB + j];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float acc[QS];
#pragma unroll
                for (int q = 0; q < QS; ++q) {
                    acc[q] = 0.f;
#pragma unroll
                    for (int j = 0; j < DSUB; ++j) {
                        const float diff = qv[q][j] - cv[r][j];
                        acc[q] += diff * diff;
                    }
                }
                sink(s, r * WAVE + lane, acc);
            }
        } else {
            for (int r = 0; r < R; ++r) {
                const int c = r * WAVE + lane;
                const float* cent = cbase + c * dsub;
                float acc[QS];
#pragma unroll
                for (int q = 0; q < QS; ++q) acc[q] = 0.f;
                for (int j = 0; j < dsub; ++j) {
                    const float cj = cent[j];
#pragma unroll
                    for (int q = 0; q < QS; ++q) {
                        const float diff = qrow[q][s * dsub + j] - cj;
                        acc[q] += diff * diff;
                    }
                }
                sink(s, c, acc);
            }
        }
    }
}

// Sub-vector widths of d = 128 at m = 16, 32, 64 (and 64 at m = 16) get an unrolled pass; others the generic one.
template <int QS, int M, int W, typename Sink>
__device__ __forceinline__ void table_entries(const WaveScanArgs& a, const float* const (&qrow)[QS], int wave,
                                              int lane, Sink& sink) {
    const int dsub = a.d / (M ? M : a.m);
    if (dsub == 8) table_entries_w<QS, M, W, 8>(a, qrow, wave, lane, sink);
    else if (dsub == 4) table_entries_w<QS, M, W, 4>(a, qrow, wave, lane, sink);
    else if (dsub == 2) table_entries_w<QS, M, W, 2>(a, qrow, wave, lane, sink);
    else table_entries_w<QS, M, W, 0>(a, qrow, wave, lane, sink);
}

// Writes the NG query-interleaved tables of a slab into LDS, interleaved per sub-space: group t's entry for code c
// of sub-space s is at ((s * NG + t) * 256 + row) * entry bytes, row = a.table_rows[s * 256 + c] (the row the code
// layout stores for c) or c, so the NG reads of one code byte lie within 256 * NG entries of each other and share
// one address register (immediate offsets). fp16 tables take each
// query's power-of-two shift from the per-query maxima in `qmax` (raw fp32 bits).
template <int QG, int NG, int M, int W, bool F16>
__device__ __forceinline__ void build_tables(const WaveScanArgs& a, const float* const (&qrow)[QG * NG],
                                             unsigned char* tables, const unsigned* qmax, int wave, int lane) {
    constexpr int QS = QG * NG;
    constexpr int EB = Entries<QG, F16>::kBytes;
    if constexpr (!F16) {
        // One group of QG queries at a time: the unrolled pass holds QG query rows and their sums, not QS.
#pragma unroll 1
        for (int t = 0; t < NG; ++t) {
            const float* group[QG];
#pragma unroll
            for (int q = 0; q < QG; ++q) group[q] = qrow[t * QG + q];
            auto sink = [&](int s, int c, const float* acc) {
                const int row = a.table_rows ? a.table_rows[s * KSUB + c] : c;
                unsigned char* dst = tables + ((s * NG + t) * KSUB + row) * EB;
                if constexpr (QG == 4) *reinterpret_cast<float4*>(dst) = make_float4(acc[0], acc[1], acc[2], acc[3]);
                else if constexpr (QG == 2) *reinterpret_cast<float2*>(dst) = make_float2(acc[0], acc[1]);
                else *reinterpret_cast<float*>(dst) = acc[0];
            };
            table_entries<QG, M, W>(a, group, wave, lane, sink);
        }
    } else {
        int shift[QS];
#pragma unroll
        for (int q = 0; q < QS; ++q) shift[q] = table_shift(qmax[q]);
        auto sink = [&](int s, int c, const float* acc) {
            uint32_t h[QS];
#pragma unroll
            for (int q = 0; q < QS; ++q) h[q] = to_half_bits(ldexpf(acc[q], -shift[q]));
            const int row = a.table_rows ? a.table_rows[s * KSUB + c] : c;
#pragma unroll
            for (int t = 0; t < NG; ++t) {
                unsigned char* dst = tables + ((s * NG + t) * KSUB + row) * EB;
                const uint32_t* g = h + t * QG;
                if constexpr (QG == 8)
                    *reinterpret_cast<uint4*>(dst) = make_uint4(g[0] | g[1] << 16, g[2] | g[3] << 16,
                                                                g[4] | g[5] << 16, g[6] | g[7] << 16);
                else if constexpr (QG == 4)
                    *reinterpret_cast<uint2*>(dst) = make_uint2(g[0] | g[1] << 16, g[2] | g[3] << 16);
                else if constexpr (QG == 2) *reinterpret_cast<uint32_t*>(dst) = g[0] | g[1] << 16;
                else *reinterpret_cast<uint16_t*>(dst) = static_cast<uint16_t>(g[0]);
            }
        };
        table_entries<QS, M, W>(a, qrow, wave, lane, sink);
    }
}

// Inverted lists: a query's table is the same for every list it probes, so the tables are computed once per
// search into HBM ([q][s][c], lut.hip) and each slab only gathers its queries' rows into the interleaved LDS layout
// (coalesced reads of consecutive entries, one 16-byte LDS write per entry group).
template <int QG, int M, int T>
__device__ __forceinline__ void gather_tables(const WaveScanArgs& a, const float* const (&lrow)[QG],
                                              unsigned char* tables, int tid) {
    const int entries = (M ? M : a.m) * KSUB;
    for (int e = tid; e < entries; e += T) {
        float v[QG];
#pragma unroll
        for (int q = 0; q < QG; ++q) v[q] = lrow[q][e];
        unsigned char* dst = tables + e * QG * 4;
        if constexpr (QG == 4) *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
        else if constexpr (QG == 2) *reinterpret_cast<float2*>(dst) = make_float2(v[0], v[1]);
        else *reinterpret_cast<float*>(dst) = v[0];
    }
}

// Per-query maximum of a slab's fp32 table entries, as raw bits (entries are >= 0, so the unsigned order is the
// float order, with NaN above +inf): lane maxima, a wave reduction, one LDS atomicMax per (wave, query). qmax must
// be zero beforehand; the caller synchronises after.
template <int QS, int M, int W>
__device__ __forceinline__ void table_maxima(const WaveScanArgs& a, const float* const (&qrow)[QS], unsigned* qmax,
                                             int wave, int lane) {
    uint32_t mx[QS];
#pragma unroll
    for (int q = 0; q < QS; ++q) mx[q] = 0u;
    auto sink = [&](int, int, const float* acc) {
#pragma unroll
        for (int q = 0; q < QS; ++q) mx[q] = max(mx[q], __float_as_uint(acc[q]));
    };
    table_entries<QS, M, W>(a, qrow, wave, lane, sink);
#pragma unroll
    for (int q = 0; q < QS; ++q) {
#pragma unroll
        for (int o = WAVE / 2; o > 0; o >>= 1)
            mx[q] = max(mx[q], static_cast<uint32_t>(__shfl_xor(static_cast<int>(mx[q]), o)));
        if (lane == 0) atomicMax(qmax + q, mx[q]);
    }
}

// The value a final result carries: fp16-table sums are scaled back by the table's power of two (exact).
__device__ __forceinline__ Pair final_pair(float d, int32_t id, int shift) {
    if (id == kEmptyId) return Pair{INFINITY, -1};
    return Pair{shift ? ldexpf(d, shift) : d, id};
}

// Final merge of one query of a slab by a single wave (few partial lists): no barriers; the wave list's first k
// entries are the results.
template <int S>
__device__ __forceinline__ void merge_query_wave(const Pair* first, int lists, int K, int k, Pair* out, int shift,
                                                 int lane) {
    WaveList<S, true> wl;
    wl.init();
    stream_partials(wl, first, 0, 1, lists, K, lane);
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int j = s * WAVE + lane;
        if (j < k) out[j] = final_pair(wl.d[s], wl.id[s], shift);
    }
}

__device__ __forceinline__ uint64_t lane_read_key(uint64_t v, int lane) {
    const uint32_t lo = static_cast<uint32_t>(lane_read(static_cast<int32_t>(static_cast<uint32_t>(v)), lane));
    const uint32_t hi = static_cast<uint32_t>(lane_read(static_cast<int32_t>(static_cast<uint32_t>(v >> 32)), lane));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

// Final merge of one query over many partial lists of K <= 64 sorted pairs (`first[l * K + j]`) by a bound and a
// filter instead of merge networks over every pair. Wave w sorts the heads (entry 0) of lists 64w .. 64w+63: when
// K of them are real, their K-th smallest key T_w has K entries of distinct lists at or below it, so the query's
// K-th best is at or below it too; T = min over the waves. Every pair above T, and every empty slot, is dropped;
// the survivors (a few dozen for hundreds of lists) are appended to LDS, and wave 0 sorts them in one network (or,
// more than 64, streams them through a wave list). The result is the K smallest pairs by (dist, id), the same as
// a merge of every list. The pair loads are issued before the head sort, so their round trip overlaps it. LDS
// `buf` holds the W bounds, the survivor count and the survivors (`buf_pairs` pairs in all); returns false, for
// every thread, when the survivors do not fit (the caller then merges every list). Called by all threads.
template <int W>
__device__ bool merge_query_filtered(const Pair* first, int lists, int K, int k, Pair* out, int shift, Pair* buf,
                                     int buf_pairs, int wave, int lane) {
    uint64_t* const bounds = reinterpret_cast<uint64_t*>(buf);
    unsigned* const count = reinterpret_cast<unsigned*>(buf + W);
    Pair* const surv = buf + W + 1;
    const int cap = buf_pairs - (W + 1);
    const int64_t total = static_cast<int64_t>(lists) * K;
    constexpr int B = 8;  // rounds of W * 64 pairs per batch, all loads of a batch in flight
    constexpr int64_t kRound = static_cast<int64_t>(W) * WAVE;
    Pair p[B];
    auto load_batch = [&](int64_t base) {
#pragma unroll
        for (int u = 0; u < B; ++u) {
            const int64_t e = base + u * kRound + wave * WAVE + lane;
            p[u] = e < total ? first[e] : Pair{INFINITY, kEmptyId};
        }
    };
    uint64_t head = kEmptyKey;
    const int hl = wave * WAVE + lane;
    if (hl < lists) {
        const Pair h = first[static_cast<int64_t>(hl) * K];
        head = pair_key(h.d, h.i);
    }
    load_batch(0);
    wave_sort<2, false>(head);
    // Read with the whole wave active: inside a lane-0 branch the compiler may sink the sort's last
    // compare-exchange into the branch, which then updates lane 0 only, and lane K-1 would still hold its value from
    // before that step.
    const uint64_t kth = lane_read_key(head, K - 1);
    if (lane == 0) bounds[wave] = kth;
    if (wave == 0 && lane == 0) *count = 0u;
    __syncthreads();
    uint64_t t = bounds[0];
#pragma unroll
    for (int w = 1; w < W; ++w) t = bounds[w] < t ? bounds[w] : t;
    for (int64_t base = 0; base < total; base += B * kRound) {
        if (base > 0) load_batch(base);
        uint64_t keep[B];
        unsigned n = 0;
#pragma unroll
        for (int u = 0; u < B; ++u) {
            keep[u] = __builtin_amdgcn_ballot_w64(p[u].i != kEmptyId && pair_key(p[u].d, p[u].i) <= t);
            n += static_cast<unsigned>(__popcll(keep[u]));
        }
        if (n == 0) continue;  // wave-uniform
        unsigned at = 0;
        if (lane == 0) at = atomicAdd(count, n);
        at = static_cast<unsigned>(__builtin_amdgcn_readfirstlane(static_cast<int>(at)));
#pragma unroll
        for (int u = 0; u < B; ++u) {
            const unsigned pos = at + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(keep[u] >> 32),
                                                                __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(keep[u]), 0u));
            if (((keep[u] >> lane) & 1) && pos < static_cast<unsigned>(cap)) surv[pos] = p[u];
            at += static_cast<unsigned>(__popcll(keep[u]));
        }
    }
    __syncthreads();
    const unsigned survivors = *count;
    // Every thread holds the count before any wave writes `buf` again: the fallback merge stores wave lists over
    // the bounds and the count, and a wave still to read the count would otherwise take the other branch.
    __syncthreads();
    if (survivors > static_cast<unsigned>(cap)) return false;  // block-uniform: every thread read the same count
    if (wave == 0) {
        if (survivors <= static_cast<unsigned>(WAVE)) {
            uint64_t key = kEmptyKey;
            if (static_cast<unsigned>(lane) < survivors) key = pair_key(surv[lane].d, surv[lane].i);
            wave_sort<2, false>(key);
            if (lane < k) out[lane] = final_pair(key_dist(key), key_id(key), shift);
        } else {
            WaveList<1, true> wl;
            wl.init();
            stream_pairs(wl, surv, 0, 4 * WAVE, static_cast<int>(survivors), K, lane);
            if (lane < k) out[lane] = final_pair(wl.d[0], wl.id[0], shift);
        }
    }
    __syncthreads();
    return true;
}

// Final merge of one query of a slab by the last block to finish the slab: the slab's `lists` partial lists for
// the query (K pairs each, `first[l * K + j]`); for K <= 64 by the filter above when its survivors fit in `buf`.
// Otherwise they are split over the W waves, each streaming its share through a wave list; wave 0 then streams the
// W wave lists (LDS `buf`, W * K pairs) into the query's k results. Called by all threads of the block.
template <int S, int W>
__device__ __forceinline__ void merge_query(const Pair* first, int lists, int K, int k, Pair* out, int shift,
                                            Pair* buf, int buf_pairs, int wave, int lane) {
    if constexpr (S == 1) {
        if (merge_query_filtered<W>(first, lists, K, k, out, shift, buf, buf_pairs, wave, lane)) return;
    }
    WaveList<S, true> wl;
    wl.init();
    stream_partials(wl, first, wave, W, lists, K, lane);
    wl.store(buf + wave * K, K);
    __syncthreads();
    if (wave == 0) merge_query_wave<S>(buf, W, K, k, out, shift, lane);
    __syncthreads();
}

// Vector ids of a granule's U tiles in the sorted code layout (exhaustive scans): per slot, its vector's id,
// interleaved by four tiles ([tile / 4][lane][tile % 4]), so one load of 4U bytes gives a lane the ids of its U
// tiles (a granule's tiles start at a multiple of U, and U <= 4).
template <int U>
struct SlotIds {
    static_assert(U == 1 || U == 2 || U == 4, "a granule's tiles lie within one group of four tiles");
    uint32_t w[U];
    __device__ __forceinline__ void load(const uint32_t* slot_ids, int64_t tile0, int lane) {
        const uint32_t* p = slot_ids + (tile0 >> 2) * 256 + lane * 4 + (tile0 & 3);
        if constexpr (U == 4) {
            const uint4 v = *reinterpret_cast<const uint4*>(p);
            w[0] = v.x;
            w[1] = v.y;
            w[2] = v.z;
            w[3] = v.w;
        } else if constexpr (U == 2) {
            const uint2 v = *reinterpret_cast<const uint2*>(p);
            w[0] = v.x;
            w[1] = v.y;
        } else {
            w[0] = *p;
        }
    }
    __device__ __forceinline__ uint32_t get(int u) const { return w[u]; }
};

// QG: queries per table (1, 2, 4; 8 with fp16 entries). NG: tables per block (1, 2). U: 64-vector tiles per wave
// step. M: sub-spaces if fixed at compile time, 0 for any m % 16 == 0. S: list registers per lane (K <= 64 * S).
// F16: binary16 table entries.
// Waves per SIMD the block residency allows: blocks per CU are bounded by LDS (the NG tables) and by 2048
// threads; the register budget is set so that residency is not cut further by VGPRs (4 waves -> 128).
template <int QG, int NG, int M, int T, bool F16>
constexpr int wave_kernel_waves_per_simd() {
    if (M == 0) return 1;
    const int by_lds = (160 * 1024) / (NG * (M ? M : 16) * KSUB * Entries<QG, F16>::kBytes);
    const int blocks = by_lds < 2048 / T ? by_lds : 2048 / T;
    const int waves = blocks * (T / WAVE) / 4;
    return waves < 1 ? 1 : (waves > 4 ? 4 : waves);
}

// First slab whose granule range [slab_gran[s], slab_gran[s + 1]) contains `item` (binary search; inverted lists).
__device__ __forceinline__ int64_t slab_of(const int64_t* slab_gran, int64_t slabs, int64_t item) {
    int64_t lo = 0, hi = slabs - 1;
    while (lo < hi) {
        const int64_t mid = (lo + hi + 1) >> 1;
        if (slab_gran[mid] <= item) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// IVF (one query per slab, QS = 1): the scan runs over inverted lists. Slab s is a list probed by query
// a.slab_queries[s]; slabs are in query-major order, so a query's probed lists form one run of consecutive slabs,
// granules [a.query_gran[q], a.query_gran[q + 1]) of the balanced partition (a.query_gran[nq] = total). Slab s covers
// granules [a.slab_gran[s], a.slab_gran[s + 1]) (possibly none), its list's padded tiles start at a.slab_tile[s] in
// the word-interleaved codes (the plan copies the list's first tile there, one dependent load fewer per slab than
// looking it up by list), and the vector ids come from a.ids (-1 on padding). A block
// gathers a query's tables and starts its lists once per run and writes them once, at the end of the run (or of
// its range); a separate merge kernel combines the partial lists of each query.
template <int QG, int NG, int U, int M, int S, int T, bool F16, bool IVF, bool BULK>
__global__ void __launch_bounds__(T)
    __attribute__((amdgpu_waves_per_eu(wave_kernel_waves_per_simd<QG, NG, M, T, F16>())))
    fused_wave_kernel_t(WaveScanArgs a) {
    constexpr int QS = QG * NG;
    constexpr int W = T / WAVE;
    static_assert(!IVF || (QS == 1 && !F16), "inverted-list scans take one query per slab and fp32 tables");
    using E = Entries<QG, F16>;
    using V = typename E::T;
    // With m fixed the tables are a static LDS array at address 0, so a lookup address is one SDWA shift of
    // the code byte plus a compile-time immediate offset; a dynamic (extern) array's base is a link-time
    // symbol that costs two more VALU adds per lookup.
    constexpr int kStaticVec = M ? NG * M * KSUB * E::kBytes / 16 : 1;
    __shared__ uint4 lds_static[kStaticVec];
    extern __shared__ uint4 lds_dynamic[];
    __shared__ bool last_block;
    // Exhaustive search: granules of the block's range past the first W, handed out one at a time to whichever wave
    // asks next. With static assignment the waves a SIMD favours finish their share first and leave one wave per
    // SIMD to finish the block, too few to keep the LDS pipe busy.
    __shared__ unsigned next_gran;
    __shared__ unsigned qmax[QS];  // fp16 tables: per-query maximum entry of the current slab (raw bits)
    // Long lists (K > 64), and the bulk instances (few vectors per block): per (query, wave), the distance of the
    // wave list's entry ceil(K/W) - 1 for the current slab (raw bits of a distance >= 0, so unsigned order is float
    // order; +inf until the list holds that many). If every wave holds ceil(K/W) entries at or below T, the block
    // holds at least K, so the maximum over the waves bounds the block's K-th best: a candidate beyond it cannot
    // reach the merged top K, and every wave filters by it. At K = 128 this removes ~40 % of the inserts. For
    // one-register lists over many vectors per block the bookkeeping costs more than the inserts it saves
    // (measured with the lane-parallel form below: 1M x nq=1000 +0.5 %, 10M +0.8 %, fp16 tables at 8 queries
    // +4.7 %); with few vectors per block, where a larger share of the candidates enters fresh lists, it pays
    // (100k x nq=100: -2 %).
    constexpr bool kShareBound = S > 1 || (BULK && !IVF);
    // When every (query, wave) slot fits in one wave, a step reads all of them with one LDS read (lane l: slot l)
    // and takes each query's maximum over its W lanes by DPP exchanges; a wave publishes its QS values with one
    // LDS write (lane q: query q), always (they only fall).
    constexpr bool kLaneBound = kShareBound && QS * W <= WAVE && (W == 2 || W == 4 || W == 8 || W == 16);
    __shared__ __align__(16) unsigned rank_bound[QS][W];
    // Admission queue of the wave lists (fp32 tables, static LDS): candidates that pass a list's filter a few at a
    // time are appended to a run of kQueueCap LDS slots of their (query, wave) instead of being inserted one by one
    // (~22 VALU instructions each into a one-register list, ~32 into a two-register one). A full run and the end of
    // the slab go in by one bitonic merge from the upper half-wave (merge_upper_half), a tile that admits a whole
    // run's worth at once by one from all its lanes (merge_wave). A merge keeps the K smallest pairs of the list and
    // of everything offered to it, so the list ends as the one-by-one inserts leave it; the queued candidates were
    // tested against a threshold that has fallen since, which only admits a few more. Measured: 1M x nq=1000 (m=16, k=10) 0.637 -> 0.605 ms per search, m=32 (k=100) VALU per
    // table read 7.18 -> 5.93 (3.5 % faster, the LDS then binding); 10M and 100M unchanged; inverted lists
    // (flushed when a query's run of lists ends) 0.201 -> 0.190 ms at nprobe 32, 0.087 -> 0.080 at nprobe 8. The
    // fp16-table kernels have no registers for it: their 8-query loop then spilled (1M -11 %, 10M -28 %).
    constexpr int kTableBytes = NG * M * KSUB * E::kBytes;
    constexpr int kRunBytes = QS * W * static_cast<int>(sizeof(Pair));  // one slot per (query, wave)
    constexpr int kQueueCap = kTableBytes + 32 * kRunBytes <= 150 * 1024 ? 32
                              : kTableBytes + 16 * kRunBytes <= 150 * 1024 ? 16 : 0;
    constexpr bool kQueue = !F16 && S <= 2 && M > 0 && kQueueCap > 0;
    static_assert(kQueueCap <= WAVE / 2, "a flush merges at most half a wave of queued candidates");
    __shared__ Pair queue[kQueue ? QS * W * kQueueCap : 1];
    unsigned char* const tables = reinterpret_cast<unsigned char*>(M ? lds_static : lds_dynamic);
    const int m = M ? M : a.m;
    const int words = m / 16;
    const int table_bytes = m * KSUB * E::kBytes;  // one group table
    // The wave index is the same in every lane; reading it through a scalar register lets the compiler keep the
    // granule, tile and id arithmetic of the scan loop on the scalar unit.
    const int tid = threadIdx.x, lane = __lane_id(), wave = __builtin_amdgcn_readfirstlane(tid / WAVE);
    // Inverted lists are planned on the device: the total is read here, and with fewer granules than blocks only
    // the first `total` blocks take part, so that every block of the partition owns at least one granule (the
    // merge kernel expects lists from every block between a query's first and last).
    const int64_t total = IVF ? a.query_gran[a.nq] : a.total;
    const int64_t grid = IVF ? min<int64_t>(gridDim.x, total) : gridDim.x, b = blockIdx.x;
    if (IVF && b >= grid) return;  // block-uniform, before any barrier
    const int64_t start = b * total / grid, end = (b + 1) * total / grid;
    const _Float16 one = opaque_half_one();
    // Address registers of the sub-spaces whose tables lie past the first 64 KB of LDS: the high half stays 1, the
    // low half takes each lookup's scaled code byte (scaled_byte_low_half). A few registers in rotation: a read
    // takes its address when it issues, so the register is free for the fourth lookup after it.
    constexpr bool kWindowed = M > 0 && NG * M * KSUB * E::kBytes > 65536;
    constexpr int kHi = kWindowed ? 4 : 1;
    uint32_t hi[kHi];
#pragma unroll
    for (int j = 0; j < kHi; ++j) hi[j] = 0x10000u;

    // Inverted lists: the first slab of the block's range by binary search (the last slab starting at or before
    // `start`, i.e. the non-empty one holding it); every later one is the next non-empty slab, so the search costs
    // one chain of dependent loads per block, not one per slab.
    int64_t next_slab = IVF && start < end ? slab_of(a.slab_gran, a.n_slabs, start) : 0;
    // Bulk admission (device.hpp) for long lists; for inverted lists, whose partial lists cover a few probed lists
    // each, so that many of their candidates arrive while the list is filling; for one query per block; and where
    // the launch asks for it (BULK): a list admits about K ln(n / K) candidates over n, a third of the first 64
    // among them, and one by one those first inserts cost a wave's first step several times a later one. Over a
    // block's first few steps that dominates; over millions of vectors per block the merge's code in the scan loop
    // costs about 1 %. The fp16 kernels (Q = 8) have no registers to spare for it in the loop. Lists that admit
    // one by one still take a wave's first granule step in bulk (kPeel, at the scan loop).
    constexpr bool kBulkOne = QS == 1 && !F16;
    WaveList<S, IVF || (!F16 && S > 1) || kBulkOne || BULK, kShareBound> lists[QS];
    float published[QS];
    unsigned queued[QS];  // admission queue: candidates held in each list's run (wave-uniform)
    const int bound_rank = (a.K + W - 1) / W - 1;  // < 64: the entry lives in the lists' first register
    int32_t run_query = -1;                        // IVF: the query whose tables and lists are current
    // One query per block over 16-byte codes: the next granule's code words and ids are loaded before this
    // granule's lookups (U more registers), so a wave's next memory round trip overlaps its own lookups; a slab's
    // first granule is loaded before the tables are built. With one query per block the codes stream from HBM and the
    // few waves per CU leave that latency open otherwise. The multi-query instances read codes mostly from L2 and
    // need the registers for their accumulators (four queries, sorted codes, slab-aligned blocks: 1M x nq=1000
    // +4.5 % with the prefetch, 10M +3.6 %).
    constexpr bool kPrefetch = !IVF && QS == 1 && M == 16;
    // Several code words per tile, or two tables, in a 1024-thread block (128 VGPRs): loading all U tiles' words at
    // the step's start spilled the later tiles' words to scratch in every step (m=32, k=100: 1 GB of scratch writes
    // per search), so each tile's words are loaded as the tile before it starts.
    constexpr bool kStagedWords = !IVF && T == 1024 && (M >= 32 || NG > 1);
    uint4 next_words[kPrefetch ? U : 1];
    SlotIds<U> next_ids;

    for (int64_t item = start; item < end;) {
        // The slab holding `item` and its granules [slab_first, slab_next) in the balanced partition.
        int64_t slab, slab_first, slab_next;
        if constexpr (IVF) {
            // Probes of no list or of an empty list are empty slabs: skipped (a non-empty slab holds `item`).
            slab = next_slab;
            while (a.slab_gran[slab + 1] == a.slab_gran[slab]) ++slab;
            next_slab = slab + 1;
            slab_first = a.slab_gran[slab];
            slab_next = a.slab_gran[slab + 1];
        } else {
            slab = item / a.n_gran;
            slab_first = slab * a.n_gran;
            slab_next = slab_first + a.n_gran;
        }
        const int64_t g_lo = item - slab_first;
        const int64_t g_hi = min(end, slab_next) - slab_first;
        // Query rows of the slab; live[q] is false for padded slots (which repeat a real query's row). lrow: the
        // query's row of the per-search tables (inverted lists). An inverted-list slab continues the run of its
        // query's slabs (query-major order) unless the query changes: tables and lists carry over.
        const float* qrow[QS];
        const float* lrow[QS];
        bool live[QS];
        bool new_run = true;
        if constexpr (IVF) {
            const int32_t qi = a.slab_queries[slab];
            new_run = qi != run_query;
            run_query = qi;
            qrow[0] = a.queries + static_cast<int64_t>(qi) * a.d;
            lrow[0] = a.lut + static_cast<int64_t>(qi) * (M ? M : a.m) * KSUB;
            live[0] = true;
        } else {
#pragma unroll
            for (int q = 0; q < QS; ++q) {
                int64_t qi = slab * QS + q;
                live[q] = qi < a.nq;
                if (!live[q]) qi = a.nq - 1;
                qrow[q] = a.queries + qi * a.d;
                lrow[q] = nullptr;
            }
        }
        int64_t list_tile0 = 0;  // IVF: first tile of the slab's list
        if constexpr (IVF) list_tile0 = a.slab_tile[slab];
        if constexpr (kPrefetch) {
            if (g_lo + wave < g_hi) {
                const uint4* c = a.codes + (g_lo + wave) * U * WAVE + lane;
#pragma unroll
                for (int u = 0; u < U; ++u) next_words[u] = c[u * WAVE];
                next_ids.load(a.slot_ids, (g_lo + wave) * U, lane);
            }
        }

        if (new_run) {
            __syncthreads();  // the previous slab's merge has finished with LDS
            if constexpr (F16) {
                if (tid < QS) qmax[tid] = 0u;
                __syncthreads();
                table_maxima<QS, M, W>(a, qrow, qmax, wave, lane);
                __syncthreads();
            }
            if constexpr (IVF) gather_tables<QG, M, T>(a, lrow, tables, tid);
            else build_tables<QG, NG, M, W, F16>(a, qrow, tables, qmax, wave, lane);
            if constexpr (kShareBound)
                for (int t = tid; t < QS * W; t += T) (&rank_bound[0][0])[t] = 0x7f800000u;  // +inf
            if (!IVF && tid == 0) next_gran = W;
            __syncthreads();

            // A padded query slot (past nq in the last slab) gets the threshold -inf: no distance passes it, so
            // the scan loop offers every slot without a per-query test.
#pragma unroll
            for (int q = 0; q < QS; ++q) {
                lists[q].init();
                if (!live[q]) lists[q].disable();
                published[q] = INFINITY;
                queued[q] = 0;
            }
        }
        const uint32_t n32 = static_cast<uint32_t>(a.n);  // n < 2^31: ids and tile bounds fit in 32 bits

        // One granule step of this wave (g: the wave's granule, advanced at the end). bulk_step: candidates are
        // admitted in bulk whatever the list type.
        int64_t g = g_lo + wave;
        // Admission queue: merges list q's queued candidates into it. Lanes read slots that other lanes of the wave
        // wrote: the LDS serves one wave's accesses in order, and the wave barriers keep the compiler from moving
        // these reads above those writes, or the next appends above these reads.
        auto flush = [&](int q) __attribute__((always_inline)) {
            const Pair* const run = queue + (q * W + wave) * kQueueCap;
            const bool held = lane >= WAVE / 2 && static_cast<unsigned>(lane - WAVE / 2) < queued[q];
            Pair e{INFINITY, kEmptyId};
            __builtin_amdgcn_wave_barrier();
            if (held) e = run[lane - WAVE / 2];
            __builtin_amdgcn_wave_barrier();
            lists[q].merge_upper_half(e.d, e.i, held, a.K);
            queued[q] = 0;
        };
        // Admission queue: offers this tile's candidates of query q.
        auto queue_offer = [&](int q, float x, int32_t xi, uint64_t valid) __attribute__((always_inline)) {
            uint64_t mask = __builtin_amdgcn_ballot_w64(x <= lists[q].filter) & valid;
            if (!mask) return;
            unsigned n = static_cast<unsigned>(__popcll(mask));
            if (n >= static_cast<unsigned>(kQueueCap)) {
                lists[q].merge_wave(x, xi, (mask >> lane) & 1, a.K);
                return;
            }
            if (queued[q] + n > static_cast<unsigned>(kQueueCap)) {
                flush(q);
                mask = __builtin_amdgcn_ballot_w64(x <= lists[q].filter) & valid;
                if (!mask) return;
                n = static_cast<unsigned>(__popcll(mask));
            }
            const unsigned pos = queued[q] + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u));
            if ((mask >> lane) & 1) queue[(q * W + wave) * kQueueCap + pos] = Pair{x, xi};
            queued[q] += n;
        };
        auto granule = [&](auto bulk_step) __attribute__((always_inline)) {
            // The next granule for this wave, asked for now and used after this one (inverted lists: every W-th).
            unsigned grab = 0;
            if constexpr (!IVF)
                if (lane == 0) grab = atomicAdd(&next_gran, 1u);
            // The block's bound per query (a stale slot only loosens it: published values only fall).
            // Lane-parallel form: the slots are read here and used only after the first tile's lookups (a wait for
            // this read right away would queue behind the CU's random table reads).
            int bound_raw = 0;
            if constexpr (kLaneBound) {
                bound_raw = lane < QS * W ? static_cast<int>((&rank_bound[0][0])[lane]) : 0;
            } else if constexpr (kShareBound) {
#pragma unroll
                for (int q = 0; q < QS; ++q) {
                    unsigned mx = 0u;
#pragma unroll
                    for (int w = 0; w < W; ++w) mx = max(mx, rank_bound[q][w]);
                    lists[q].set_cap(__uint_as_float(mx));
                }
            }
            const int64_t tile0 = g * U;
            const uint4* tile_codes = a.codes + (list_tile0 + tile0) * words * WAVE + lane;  // uniform base + lane
            // All code words of the U tiles are loaded first (the global-load ILP). The lookups then run one
            // tile at a time behind a scheduling fence, and each tile's candidates are offered before the next
            // tile starts: only one tile's LDS results and accumulators are live, which keeps the register
            // count within what the LDS-limited residency allows.
            constexpr int WORDS = M ? M / 16 : 1;
            uint4 cw[U][WORDS];
            SlotIds<U> ids;
            if constexpr (kPrefetch) {
                const int64_t g_next = g_lo + static_cast<int64_t>(__builtin_amdgcn_readfirstlane(grab));
#pragma unroll
                for (int u = 0; u < U; ++u) cw[u][0] = next_words[u];
                ids = next_ids;
                if (g_next < g_hi) {
                    const uint4* c = a.codes + g_next * U * WAVE + lane;
#pragma unroll
                    for (int u = 0; u < U; ++u) next_words[u] = c[u * WAVE];
                    next_ids.load(a.slot_ids, g_next * U, lane);
                }
            } else {
                if constexpr (M > 0) {
#pragma unroll
                    for (int u = 0; u < (kStagedWords ? 1 : U); ++u)
#pragma unroll
                        for (int w = 0; w < WORDS; ++w) cw[u][w] = tile_codes[(u * WORDS + w) * WAVE];
                }
                if constexpr (!IVF) ids.load(a.slot_ids, tile0, lane);
            }
            // Inverted lists: the tiles' vector ids travel with their codes (loaded after a tile's lookups, each
            // would cost its own memory round trip behind the scheduling fence).
            int32_t vids[IVF ? U : 1];
            if constexpr (IVF) {
#pragma unroll
                for (int u = 0; u < U; ++u) vids[u] = a.ids[(list_tile0 + tile0 + u) * WAVE + lane];
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                // Staged words: the next tile's code words are asked for as this tile starts.
                if constexpr (kStagedWords) {
                    if (u + 1 < U) {
#pragma unroll
                        for (int w = 0; w < WORDS; ++w) cw[u + 1][w] = tile_codes[((u + 1) * WORDS + w) * WAVE];
                    }
                }
                float acc[QS];
                if constexpr (M == 0) {
#pragma unroll
                    for (int q = 0; q < QS; ++q) acc[q] = 0.f;
                }
                // 16 lookups of one code word, sub-spaces 16w .. 16w+15 in order; the first sub-space of a vector
                // (w == 0 with m fixed) sets the accumulators instead of adding to zeroed ones.
                constexpr int kShift = log2_int(E::kBytes);
                // Entry group t of code byte j of a word: its LDS address is reg + imm (imm a compile-time
                // immediate offset below 64 KB). With m fixed, sub-space s's groups start at s * NG * 256 entries;
                // those past 64 KB take their byte offset in a register whose high half is 1 (hi[j]), the rest
                // the plain scaled byte. WC: the word index, a compile-time constant when m is fixed.
                auto address = [&](const uint32_t (&part)[4], auto jc, auto wc, uint32_t& reg, int& imm) {
                    constexpr int j = decltype(jc)::value;
                    if constexpr (M > 0) {
                        constexpr int base = (decltype(wc)::value * 16 + j) * NG * KSUB * E::kBytes;
                        static_assert((base >> 16) <= 1 && ((base + NG * KSUB * E::kBytes - 1) >> 16) == (base >> 16),
                                      "a sub-space's entry groups lie in one 64 KB window, the first or the second");
                        if constexpr ((base >> 16) == 0) {
                            reg = scaled_byte<kShift>(part[j >> 2], j & 3);
                            imm = base;
                        } else {
                            scaled_byte_low_half<kShift, j & 3>(hi[j % kHi], part[j >> 2]);
                            reg = hi[j % kHi];
                            imm = base - 65536;
                        }
                    } else {
                        reg = scaled_byte<kShift>(part[j >> 2], j & 3);
                        imm = (static_cast<int>(wc) * 16 + j) * NG * KSUB * E::kBytes;
                    }
                };
                auto lookup_word = [&](const uint4 word, auto wc) {
                    const uint32_t part[4] = {word.x, word.y, word.z, word.w};
                    bool first = false;
                    if constexpr (M > 0) first = decltype(wc)::value == 0;
                    if constexpr (F16 && QG >= 4) {
                        // The word's reads are issued eight at a time before their accumulations: the
                        // one-statement-per-read accumulations would otherwise be scheduled right behind their own
                        // read, one read in flight at a time. Eight, not all sixteen: the sixteen results held 64
                        // VGPRs and made the 8-query loop reload spilled values every step (8 queries: 1M -0.8 %,
                        // 10M -1.4 %).
                        static_for<0, 2>([&](auto hc) {
                            constexpr int h = decltype(hc)::value;
                            V v[8 * NG];
                            static_for<0, 8>([&](auto jjc) {
                                constexpr int jj = decltype(jjc)::value;
                                uint32_t reg;
                                int imm;
                                address(part, std::integral_constant<int, h * 8 + jj>{}, wc, reg, imm);
#pragma unroll
                                for (int t = 0; t < NG; ++t)
                                    v[jj * NG + t] =
                                        *reinterpret_cast<const V*>(tables + reg + imm + t * KSUB * E::kBytes);
                            });
                            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                            for (int jj = 0; jj < 8; ++jj)
#pragma unroll
                                for (int t = 0; t < NG; ++t) {
                                    if (first && h == 0 && jj == 0) E::set(&acc[t * QG], v[jj * NG + t]);
                                    else E::add(&acc[t * QG], v[jj * NG + t], one);
                                }
                        });
                        return;
                    }
                    // The reads are issued in batches of 16 (16 / NG sub-spaces), each batch before its adds: 16
                    // reads in flight per wave, in 64 VGPRs at most (four-query entries). Left to itself the scheduler
                    // either hoists every read of a tile (eight queries: 128 VGPRs, spilled) or, with the sums fenced
                    // before the offers, waits for each read before issuing the next. Two-register lists or two
                    // tables in a 1024-thread block (128 VGPRs) take batches of 8: with 16 the read addresses spilled.
                    constexpr int kBatch = ((S > 1 || NG > 1) && T == 1024 ? 8 : 16) / NG;
                    static_for<0, 16 / kBatch>([&](auto bc) {
                        constexpr int b = decltype(bc)::value;
                        V v[kBatch * NG];
                        static_for<0, kBatch>([&](auto jjc) {
                            constexpr int jj = decltype(jjc)::value;
                            uint32_t reg;
                            int imm;
                            address(part, std::integral_constant<int, b * kBatch + jj>{}, wc, reg, imm);
#pragma unroll
                            for (int t = 0; t < NG; ++t)
                                v[jj * NG + t] =
                                    *reinterpret_cast<const V*>(tables + reg + imm + t * KSUB * E::kBytes);
                        });
                        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                        for (int jj = 0; jj < kBatch; ++jj)
#pragma unroll
                            for (int t = 0; t < NG; ++t) {
                                if (first && b == 0 && jj == 0) E::set(&acc[t * QG], v[jj * NG + t]);
                                else E::add(&acc[t * QG], v[jj * NG + t], one);
                            }
                        __builtin_amdgcn_sched_barrier(0);
                    });
                };
                if constexpr (M > 0) {
                    static_for<0, WORDS>([&](auto wc) { lookup_word(cw[u][decltype(wc)::value], wc); });
                } else {
                    for (int w = 0; w < words; ++w) lookup_word(tile_codes[(u * words + w) * WAVE], w);
                }
                // Every query's sum is complete here, before the first offer: left alone, the compiler sinks each
                // query's adds to just before that query's offer, so the table reads of the later queries stay live
                // across the earlier queries' insert branches (eight queries: spilled to scratch).
#pragma unroll
                for (int q = 0; q < QS; ++q) asm volatile("" : "+v"(acc[q]));
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (kLaneBound) {
                    if (u == 0) {  // raw bits of distances >= 0 or +inf: signed order is float order
                        int mx = max(bound_raw, xor_lane<1>(bound_raw));
                        if constexpr (W > 2) mx = max(mx, xor_lane<2>(mx));
                        if constexpr (W > 4) mx = max(mx, xor_lane<4>(mx));
                        if constexpr (W > 8) mx = max(mx, xor_lane<8>(mx));
#pragma unroll
                        for (int q = 0; q < QS; ++q)
                            lists[q].set_cap(__int_as_float(__builtin_amdgcn_readlane(mx, q * W)));
                    }
                }
                // Lanes holding a real vector: all of them except in the database's last tile (or, for inverted
                // lists, the padding at the end of each list).
                uint32_t id;
                uint64_t valid;
                if constexpr (IVF) {
                    const int32_t vid = vids[u];
                    id = static_cast<uint32_t>(vid);
                    valid = __builtin_amdgcn_ballot_w64(vid >= 0);
                } else {
                    // Slots [0, n) hold the real vectors of the sorted layout, each with its id beside it.
                    const uint32_t first = static_cast<uint32_t>((tile0 + u) * WAVE);
                    id = ids.get(u);
                    valid = first + WAVE <= n32 ? ~uint64_t{0}
                                                : __builtin_amdgcn_ballot_w64(first + static_cast<uint32_t>(lane) < n32);
                }
#pragma unroll
                for (int q = 0; q < QS; ++q) {
                    if constexpr (decltype(bulk_step)::value) lists[q].offer_masked_bulk(acc[q], static_cast<int32_t>(id), valid, a.K);
                    else if constexpr (kQueue) queue_offer(q, acc[q], static_cast<int32_t>(id), valid);
                    else lists[q].offer_masked(acc[q], static_cast<int32_t>(id), valid, a.K);
                }
            }
            // Publish this wave's entry ceil(K/W) - 1 when it has fallen.
            if constexpr (kLaneBound) {
                int pub = 0;
#pragma unroll
                for (int q = 0; q < QS; ++q) {
                    const int v = __float_as_int(lane_read(lists[q].d[0], bound_rank));
                    pub = lane == q ? v : pub;
                }
                if (lane < QS) rank_bound[lane][wave] = static_cast<unsigned>(pub);
            } else if constexpr (kShareBound) {
#pragma unroll
                for (int q = 0; q < QS; ++q) {
                    const float v = lane_read(lists[q].d[0], bound_rank);
                    if (v < published[q]) {
                        published[q] = v;
                        if (lane == 0) rank_bound[q][wave] = __float_as_uint(v);
                    }
                }
            }
            if constexpr (IVF) g += W;
            else g = g_lo + static_cast<int64_t>(__builtin_amdgcn_readfirstlane(grab));
        };
        // Lists that admit one by one take a wave's first step in bulk: the fresh lists admit about a third of the
        // first tile's candidates and, one by one, those inserts made the step several times a later one, with
        // every wave of the CU inserting at once. The step is a separate copy of the body ahead of the loop, so the
        // loop's own code is that of one-by-one admission (1M x nq=1000: -1.2 %; fp16 tables, 8 queries: -5 %).
        constexpr bool kPeel = !(IVF || S > 1 || kBulkOne || BULK);
        if constexpr (kPeel) {
            if (g < g_hi) granule(std::true_type{});
        }
        while (g < g_hi) granule(std::false_type{});
        // Queued candidates go into the lists before they are stored (inverted lists: at the end of a query's run).
        auto flush_all = [&]() __attribute__((always_inline)) {
            if constexpr (kQueue) {
#pragma unroll
                for (int q = 0; q < QS; ++q)
                    if (queued[q]) flush(q);
            }
        };
        if constexpr (!IVF) flush_all();

        // Inverted lists: when the query's run of slabs ends (or the block's range does), every wave writes its
        // list for the query at part[((b + query) * W + wave) * K]. Along the granule order both the block and the
        // query only grow and one of them grows at every new (block, query) pair, so b + query is unique per pair
        // and a query's lists (from consecutive blocks) are contiguous for the merge kernel.
        if constexpr (IVF) {
            item = slab_next;
            if (item >= end || item >= a.query_gran[run_query + 1]) {
                flush_all();
                lists[0].store(a.part + ((b + run_query) * W + wave) * a.K, a.K);
            }
            continue;
        }

        // Partial lists of this (block, slab): part[slab][q][slot][list][K], the lists of one query contiguous.
        // With few blocks per slab every wave writes its own lists; with many, the block first merges its W lists
        // per query in LDS (the tables are dead by then), so the final merge reads W times fewer pairs.
        const int64_t lo = first_block_of(slab_first, grid, total);
        const int count = static_cast<int>(first_block_of(slab_next - 1, grid, total) - lo + 1);
        const int slot = static_cast<int>(b - lo);
        const int lpb = a.lists_per_block;
        const int slots = a.max_slots;  // every slab reserves max_slots blocks
        Pair* const slab_part = a.part + slab * QS * a.max_slots * lpb * static_cast<int64_t>(a.K);
        Pair* const buf = reinterpret_cast<Pair*>(tables);  // QS * W * K pairs fit in the tables' space
        if (count == 1) {
            // The block scanned the whole slab: its wave lists go to LDS and wave q merges query q's W lists
            // straight into the results, with no partial lists in HBM, no fences and no ticket.
            __syncthreads();  // every wave has finished reading the tables
#pragma unroll
            for (int q = 0; q < QS; ++q) lists[q].store(buf + (q * W + wave) * a.K, a.K);
            __syncthreads();
            for (int q = wave; q < QS && slab * QS + q < a.nq; q += W)
                merge_query_wave<S>(buf + q * W * a.K, W, a.K, a.k, a.out + (slab * QS + q) * a.k,
                                    F16 ? table_shift(qmax[q]) : 0, lane);
            item = slab_next;
            continue;
        }
        if (lpb == 1) {
            __syncthreads();  // every wave has finished reading the tables
#pragma unroll
            for (int q = 0; q < QS; ++q) lists[q].store(buf + (q * W + wave) * a.K, a.K);
            __syncthreads();
            // Wave q streams query q's W lists (W * K pairs in LDS) into one list (QS <= W).
            if (wave < QS) {
                WaveList<S, true> wl;
                wl.init();
                stream_partials(wl, buf + wave * W * a.K, 0, 1, W, a.K, lane);
                wl.store(slab_part + (wave * slots + slot) * a.K, a.K);
            }
        } else {
#pragma unroll
            for (int q = 0; q < QS; ++q)
                lists[q].store(slab_part + ((q * slots + slot) * W + wave) * a.K, a.K);
        }

        // The last of the slab's blocks to get here merges all its partial lists into the final results. The
        // counter is incremented with wrap-around at count - 1, so it is back at zero for the next search.
        // Publication: every wave first waits for its own partial-list stores to complete in its XCD's L2
        // (s_waitcnt vmcnt(0); a barrier alone does not wait for another wave's stores), so after the barrier
        // thread 0's agent-scope release (an L2 write-back, then a wait for it) covers the whole block's lists
        // before the increment; the last block's acquire fence (L2 invalidate) then makes every block's lists
        // visible to it. An agent-scope release fence in every wave would do the same with eight L2 write-backs
        // per block (+2.7 % on the 1M x nq=1000 search, against 0.1 % for the wait).
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        __syncthreads();
        if (tid == 0) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
            last_block = atomicInc(a.counters + slab, static_cast<unsigned>(count - 1)) == count - 1u;
        }
        __syncthreads();
        if (last_block) {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            if (lpb == W || QS > 1) {  // one wave per query, the queries in parallel
                const int per_block = lpb == W ? W : 1;
                for (int q = wave; q < QS && slab * QS + q < a.nq; q += W)
                    merge_query_wave<S>(slab_part + q * a.max_slots * per_block * a.K, count * per_block, a.K,
                                        a.k, a.out + (slab * QS + q) * a.k, F16 ? table_shift(qmax[q]) : 0, lane);
            } else if (slab < static_cast<int64_t>(a.nq)) {  // one query (Q = 1) over many blocks: all waves
                merge_query<S, W>(slab_part, count, a.K, a.k, a.out + slab * a.k, F16 ? table_shift(qmax[0]) : 0,
                                  buf, NG * table_bytes / static_cast<int>(sizeof(Pair)), wave, lane);
            }
        }
        item = slab_next;
    }
}

template <int QG, int NG, int U, int M, int S, int T, bool F16, bool IVF, bool BULK>
hipError_t launch_fused_wave_t(const WaveScanArgs& a, int grid, size_t smem, hipStream_t stream) {
    hipLaunchKernelGGL((fused_wave_kernel_t<QG, NG, U, M, S, T, F16, IVF, BULK>), dim3(grid), dim3(T), smem, stream,
                       a);
    return hipGetLastError();
}

template <int QG, int NG, int U, int M, int S, bool F16, bool IVF = false, bool BULK = false, int T = 512>
WaveScanKernel make_wave_kernel() {
    WaveScanKernel k;
    k.fn = reinterpret_cast<const void*>(&fused_wave_kernel_t<QG, NG, U, M, S, T, F16, IVF, BULK>);
    k.threads = T;
    k.dynamic_lds = M == 0;
    k.launch = &launch_fused_wave_t<QG, NG, U, M, S, T, F16, IVF, BULK>;
    return k;
}

// 1024-thread blocks (16 waves, 128 VGPRs each): one block holds all of a CU's waves and its LDS granule counter
// balances them. Where the tables leave room for two 512-thread blocks per CU, those two are not balanced: the older
// block's waves get issue priority, so on every CU one block ended its scan ~30 % before the other, which then ran
// alone at half occupancy (1M x nq=1000: 590 against 770 us; 10M: 4.4 against 5.9 ms). Where the tables take more
// than half the LDS, 512 threads are 8 waves per CU. The block merge of 16 wave lists per query must fit the tables'
// space (QS * 16 * 64S pairs).
template <int QG, int NG, int M, int S, bool F16>
constexpr bool kWideBlock = M > 0 && QG * NG * 16 * WAVE * S * 8 <= NG * M * KSUB * Entries<QG, F16>::kBytes;

// Inverted-list instances for one M: fp32 tables, one query per slab, four tiles per wave step (each list is
// padded to a multiple of 256 vectors).
template <int M>
WaveScanKernel select_ivf_kernel(int segments) {
    if (segments == 1) return make_wave_kernel<1, 1, 4, M, 1, false, true>();
    if (segments == 2) return make_wave_kernel<1, 1, 4, M, 2, false, true>();
    return WaveScanKernel{};
}

// Instances for one M and entry type: every (QG, NG) whose tables fit in 160 KB of LDS when M is known. fp32
// tables: QG 1, 2, 4 and two groups of 4; fp16 tables: QG 1, 2, 4, 8 in one group. `bulk` asks for bulk admission
// into one-register lists: a second instance of the fp32 multi-query kernels (the others admit in bulk already, or,
// fp16, never). threads: 512, or 1024 where kWideBlock holds (four tiles per wave step only). An empty result when
// there is no such instance.
template <int M, bool F16>
WaveScanKernel select_wave_kernel(int qg, int ng, int ilp, int segments, bool bulk, int threads) {
    constexpr int kLds = 160 * 1024;
#define VK_WAVE_ILP(QG_, NG_, S_, BULK_)                                                                    \
    if (threads == 1024) {                                                                                 \
        if constexpr (kWideBlock<QG_, NG_, M, S_, F16>) {                                                  \
            if (ilp == 4) return make_wave_kernel<QG_, NG_, 4, M, S_, F16, false, BULK_, 1024>();          \
        }                                                                                                  \
        return WaveScanKernel{};                                                                           \
    }                                                                                                      \
    if (ilp == 1) return make_wave_kernel<QG_, NG_, 1, M, S_, F16, false, BULK_>();                        \
    if (ilp == 2) return make_wave_kernel<QG_, NG_, 2, M, S_, F16, false, BULK_>();                        \
    if (ilp == 4) return make_wave_kernel<QG_, NG_, 4, M, S_, F16, false, BULK_>();
#define VK_WAVE_CASE(QG_, NG_)                                                                      \
    if (qg == QG_ && ng == NG_) {                                                                   \
        if constexpr (M == 0 || NG_ * M * KSUB * Entries<QG_, F16>::kBytes <= kLds) {               \
            if (segments == 1 && bulk) {                                                            \
                if constexpr (!F16 && QG_ * NG_ > 1) {                                              \
                    VK_WAVE_ILP(QG_, NG_, 1, true)                                                  \
                }                                                                                   \
            } else if (segments == 1) {                                                             \
                VK_WAVE_ILP(QG_, NG_, 1, false)                                                     \
            } else if (segments == 2) {                                                             \
                VK_WAVE_ILP(QG_, NG_, 2, false)                                                     \
            }                                                                                       \
        }                                                                                           \
        return WaveScanKernel{};                                                                    \
    }
    if constexpr (!F16) {
        VK_WAVE_CASE(1, 1)
        VK_WAVE_CASE(2, 1)
        VK_WAVE_CASE(4, 1)
        VK_WAVE_CASE(4, 2)
    } else {
        VK_WAVE_CASE(1, 1)
        VK_WAVE_CASE(2, 1)
        VK_WAVE_CASE(4, 1)
        VK_WAVE_CASE(8, 1)
    }
#undef VK_WAVE_CASE
#undef VK_WAVE_ILP
    return WaveScanKernel{};
}

}  // namespace vk
