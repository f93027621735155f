// Device building blocks shared by the gfx950 kernels: result ordering, the empty-slot sentinel, and the
// wave64-cooperative sorted top-k list.
#pragma once

#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>
#include <cstdint>

namespace vk {

constexpr int KSUB = 256;  // centroids per sub-space: one byte per sub-code
constexpr int WAVE = 64;   // CDNA wavefront width

// An empty list slot is (+inf, INT32_MAX). It sorts after every real candidate, including one whose distance
// overflowed to +inf, so lists stay exact under the total order and the host turns surviving empty slots into
// the reference's {+inf, -1} padding (searcher.cu:514-517).
constexpr int32_t kEmptyId = INT32_MAX;

struct alignas(8) Pair {
    float d;
    int32_t i;
};

// Total order by (distance, id): common.hpp:19-21 / kernels.cuh:116.
__device__ __forceinline__ bool pair_less(float ad, int32_t ai, float bd, int32_t bi) {
    return ad < bd || (ad == bd && ai < bi);
}

__device__ __forceinline__ float lane_read(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ int32_t lane_read(int32_t v, int lane) { return __builtin_amdgcn_readlane(v, lane); }

// DPP wave_shr:1 — lane l receives lane l-1's value; lane 0 receives 0 (bound_ctrl). One VALU op, no LDS traffic and
// no copy of the destination's old value.
__device__ __forceinline__ float wave_shr1(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x138, 0xf, 0xf, true));
}
__device__ __forceinline__ int32_t wave_shr1(int32_t v) { return __builtin_amdgcn_mov_dpp(v, 0x138, 0xf, 0xf, true); }

// The value of lane ^ J. Within a row of 16 lanes by DPP (VALU only): quad_perm for J = 1, 2; for J = 4, 8 a
// row_shl:J into the lanes whose bit J is clear and a row_shr:J into the others, selected by bank (4-lane group)
// masks. J = 16 by ds_swizzle's bit-mask mode (xor within 32 lanes, no address), J = 32 by ds_bpermute.
template <int J>
__device__ __forceinline__ int xor_lane(int v) {
    if constexpr (J == 1) {
        return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xf, 0xf, false);  // quad_perm [1, 0, 3, 2]
    } else if constexpr (J == 2) {
        return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xf, 0xf, false);  // quad_perm [2, 3, 0, 1]
    } else if constexpr (J == 4) {
        const int t = __builtin_amdgcn_update_dpp(v, v, 0x104, 0xf, 0x5, false);  // row_shl:4, banks 0, 2
        return __builtin_amdgcn_update_dpp(t, v, 0x114, 0xf, 0xa, false);         // row_shr:4, banks 1, 3
    } else if constexpr (J == 8) {
        const int t = __builtin_amdgcn_update_dpp(v, v, 0x108, 0xf, 0x3, false);  // row_shl:8, banks 0, 1
        return __builtin_amdgcn_update_dpp(t, v, 0x118, 0xf, 0xc, false);         // row_shr:8, banks 2, 3
    } else if constexpr (J == 16) {
        return __builtin_amdgcn_ds_swizzle(v, (16 << 10) | 0x1f);  // and 0x1f, or 0, xor 16
    } else {
        static_assert(J == 32, "lane distance");
        return __builtin_amdgcn_ds_bpermute((__lane_id() ^ 32) << 2, v);
    }
}

// A pair as one 64-bit key: the distance's bits above, the id below. For the pairs a wave list holds -- distances
// >= +0 or +inf (a NaN distance is never admitted: no comparison with it holds) and ids >= 0 or kEmptyId -- the
// unsigned order of the keys is the (dist, id) order, so the sorting networks below compare pairs with one 64-bit
// compare instead of three 32-bit ones.
__device__ __forceinline__ uint64_t pair_key(float d, int32_t i) {
    return (static_cast<uint64_t>(__float_as_uint(d)) << 32) | static_cast<uint32_t>(i);
}
__device__ __forceinline__ float key_dist(uint64_t k) { return __uint_as_float(static_cast<uint32_t>(k >> 32)); }
__device__ __forceinline__ int32_t key_id(uint64_t k) { return static_cast<int32_t>(static_cast<uint32_t>(k)); }
constexpr uint64_t kEmptyKey = (uint64_t{0x7f800000u} << 32) | static_cast<uint32_t>(kEmptyId);  // (+inf, kEmptyId)

// Compare-exchange of a lane's key with the key of lane ^ J: the lane keeps the smaller of the two when keep_min,
// else the larger. Both lanes of an exchange decide consistently, so the two keys are kept, never duplicated.
template <int J>
__device__ __forceinline__ void exchange_xor(uint64_t& k, bool keep_min) {
    const int lo = xor_lane<J>(static_cast<int>(static_cast<uint32_t>(k)));
    const int hi = xor_lane<J>(static_cast<int>(static_cast<uint32_t>(k >> 32)));
    const uint64_t pk = (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo);
    const bool take = (pk < k) == keep_min;
    k = take ? pk : k;
}

// Bitonic sort of one key per lane, ascending by lane, or descending with DESC (21 compare-exchange steps).
template <int K = 2, bool DESC = false>
__device__ __forceinline__ void wave_sort(uint64_t& k) {
    if constexpr (K <= WAVE) {
        const int lane = __lane_id();
        const bool up = K == WAVE ? !DESC : (lane & K) == 0;
        if constexpr (K >= 64) exchange_xor<32>(k, ((lane & 32) == 0) == up);
        if constexpr (K >= 32) exchange_xor<16>(k, ((lane & 16) == 0) == up);
        if constexpr (K >= 16) exchange_xor<8>(k, ((lane & 8) == 0) == up);
        if constexpr (K >= 8) exchange_xor<4>(k, ((lane & 4) == 0) == up);
        if constexpr (K >= 4) exchange_xor<2>(k, ((lane & 2) == 0) == up);
        exchange_xor<1>(k, ((lane & 1) == 0) == up);
        wave_sort<K * 2, DESC>(k);
    }
}

// Bitonic sort of each half-wave: lanes 0-31 ascending, lanes 32-63 descending (15 compare-exchange steps, none
// across the halves).
template <int K = 2>
__device__ __forceinline__ void wave_sort_halves(uint64_t& k) {
    if constexpr (K <= WAVE / 2) {
        const int lane = __lane_id();
        const bool up = (lane & K) == 0;
        if constexpr (K >= 32) exchange_xor<16>(k, ((lane & 16) == 0) == up);
        if constexpr (K >= 16) exchange_xor<8>(k, ((lane & 8) == 0) == up);
        if constexpr (K >= 8) exchange_xor<4>(k, ((lane & 4) == 0) == up);
        if constexpr (K >= 4) exchange_xor<2>(k, ((lane & 2) == 0) == up);
        exchange_xor<1>(k, ((lane & 1) == 0) == up);
        wave_sort_halves<K * 2>(k);
    }
}

// Sorts a bitonic sequence of one key per lane ascending (6 compare-exchange steps).
__device__ __forceinline__ void wave_clean(uint64_t& k) {
    const int lane = __lane_id();
    exchange_xor<32>(k, (lane & 32) == 0);
    exchange_xor<16>(k, (lane & 16) == 0);
    exchange_xor<8>(k, (lane & 8) == 0);
    exchange_xor<4>(k, (lane & 4) == 0);
    exchange_xor<2>(k, (lane & 2) == 0);
    exchange_xor<1>(k, (lane & 1) == 0);
}

// One sorted list of up to 64*S (dist, id) pairs spread over a wave: entry p lives in lane p % 64, register
// p / 64. The admission threshold (entry K-1) is wave-uniform, so the compiler keeps it in SGPRs. Every
// member must be called by all 64 lanes with wave-uniform arguments (control flow stays uniform).
//
// `cap` is an optional outside bound: the threshold of another list over a disjoint part of the same candidate
// stream (a sibling wave's). A candidate farther than it has K better candidates in that list, so it cannot be in
// the merged top K and is not offered; ties at the cap are still offered, which keeps the (dist, id) order exact.
// CAP = false: the list never takes an outside bound (set_cap is not called), so its filter is its threshold.
template <int S, bool BULK = (S > 1), bool CAP = true>
struct WaveList {
    float d[S];
    int32_t id[S];
    float thr_d;
    int32_t thr_i;
    float cap;     // outside bound, +inf when none
    float filter;  // min(thr_d, cap): the ballot pre-test of offers

    __device__ __forceinline__ void init() {
#pragma unroll
        for (int s = 0; s < S; ++s) {
            d[s] = INFINITY;
            id[s] = kEmptyId;
        }
        thr_d = INFINITY;
        thr_i = kEmptyId;
        cap = INFINITY;
        filter = INFINITY;
    }

    // A list that must admit nothing (a padded query slot).
    __device__ __forceinline__ void disable() {
        thr_d = -INFINITY;
        filter = -INFINITY;
    }

    __device__ __forceinline__ void set_cap(float c) {
        static_assert(CAP, "a list built without an outside bound");
        cap = c;
        filter = fminf(thr_d, cap);
    }

    // Inserts the wave-uniform pair (x, xi) at its sorted position; entries behind it move one place back.
    __device__ __forceinline__ void insert(float x, int32_t xi, int K) {
        const int lane = __lane_id();
        // Entries strictly before (x, xi) form a prefix (the list is sorted): those with a smaller distance, plus,
        // only when some entry has exactly distance x (rare), those equal in distance with a smaller id.
        int pos = 0;
#pragma unroll
        for (int s = 0; s < S; ++s) {
            pos += __popcll(__builtin_amdgcn_ballot_w64(d[s] < x));
            if (__builtin_amdgcn_ballot_w64(d[s] == x)) pos += __popcll(__builtin_amdgcn_ballot_w64(d[s] == x && id[s] < xi));
        }
        float carry_d = 0.f;
        int32_t carry_i = 0;
#pragma unroll
        for (int s = 0; s < S; ++s) {
            float prev_d = wave_shr1(d[s]);
            int32_t prev_i = wave_shr1(id[s]);
            if (s > 0 && lane == 0) {  // lane 0 of a later register takes the last entry of the previous one
                prev_d = carry_d;
                prev_i = carry_i;
            }
            if (s + 1 < S) {
                carry_d = lane_read(d[s], WAVE - 1);
                carry_i = lane_read(id[s], WAVE - 1);
            }
            const bool keep = s * WAVE + lane < pos;
            d[s] = keep ? d[s] : prev_d;
            id[s] = keep ? id[s] : prev_i;
            const int at = pos - s * WAVE;  // wave-uniform: the candidate's lane in this register, if any
            if (at >= 0 && at < WAVE) {
                const bool here = lane == at;
                d[s] = here ? x : d[s];
                id[s] = here ? xi : id[s];
            }
        }
        refresh(K);
    }

    __device__ __forceinline__ void refresh(int K) {
        const int t = K - 1;
        if (S == 1 || t < WAVE) {
            thr_d = lane_read(d[0], t);
            thr_i = lane_read(id[0], t);
        } else {
            thr_d = lane_read(d[S - 1], t - (S - 1) * WAVE);
            thr_i = lane_read(id[S - 1], t - (S - 1) * WAVE);
        }
        filter = CAP ? fminf(thr_d, cap) : thr_d;
    }

    // Each lane offers one candidate. The ballot uses dist <= threshold as a cheap superset test. A few admitted
    // lanes are inserted one at a time, lowest lane first, with the exact (dist, id) test re-done per candidate
    // because the threshold falls as candidates go in; kMergeMin or more go in by one bitonic merge.
    __device__ __forceinline__ void offer(float x, int32_t xi, bool valid, int K) {
        offer_masked(x, xi, __builtin_amdgcn_ballot_w64(valid), K);
    }

    // As offer, with the lanes that hold candidates given as a wave-uniform mask: the common no-candidate case is
    // one compare into a scalar mask and one branch.
    __device__ __forceinline__ void offer_masked(float x, int32_t xi, uint64_t valid, int K) {
        uint64_t mask = __builtin_amdgcn_ballot_w64(x <= filter) & valid;
        if (BULK && __popcll(mask) >= kMergeMin) {
            merge_wave(x, xi, (mask >> __lane_id()) & 1, K);
            return;
        }
        while (mask) {
            const int src = __ffsll(static_cast<unsigned long long>(mask)) - 1;
            mask &= mask - 1;
            const float vx = lane_read(x, src);
            const int32_t vi = lane_read(xi, src);
            if (pair_less(vx, vi, thr_d, thr_i)) insert(vx, vi, K);
        }
    }

    // As offer_masked, with bulk admission whatever BULK is (a list's first candidates).
    __device__ __forceinline__ void offer_masked_bulk(float x, int32_t xi, uint64_t valid, int K) {
        const uint64_t mask = __builtin_amdgcn_ballot_w64(x <= filter) & valid;
        if (__popcll(mask) >= kMergeMin) {
            merge_wave(x, xi, (mask >> __lane_id()) & 1, K);
            return;
        }
        offer_masked(x, xi, valid, K);
    }

    // Admitted lanes from which one bitonic merge of the whole wave costs less than inserting them one by one.
    // BULK = false inserts one by one always: by default for single-register lists (K <= 64), where the merge's
    // code and registers cost the scan loop more than the inserts it replaces.
    static constexpr int kMergeMin = 8;

    // Admits every offered lane's pair at once: the wave's pairs are sorted descending (lanes not offering carry
    // the empty slot) and folded into the list's last register by elementwise minimum, which leaves the list a
    // bitonic sequence holding the 64*S smallest pairs of both; a bitonic clean sorts it. The result is the list
    // the one-by-one inserts would give.
    __device__ __forceinline__ void merge_wave(float x, int32_t xi, bool offered, int K) {
        uint64_t c = offered ? pair_key(x, xi) : kEmptyKey;
        wave_sort<2, true>(c);
        const uint64_t last = pair_key(d[S - 1], id[S - 1]);
        const uint64_t low = c < last ? c : last;
        d[S - 1] = key_dist(low);
        id[S - 1] = key_id(low);
        clean(K);
    }

    // As merge_wave for at most 32 candidates, offered by lanes 32-63 only (lanes 0-31 must not offer): sorting the
    // upper half descending makes the whole wave descending (the lower half holds empty slots), with 15
    // compare-exchange steps instead of 21.
    __device__ __forceinline__ void merge_upper_half(float x, int32_t xi, bool offered, int K) {
        uint64_t c = offered ? pair_key(x, xi) : kEmptyKey;
        wave_sort_halves(c);
        const uint64_t last = pair_key(d[S - 1], id[S - 1]);
        const uint64_t low = c < last ? c : last;
        d[S - 1] = key_dist(low);
        id[S - 1] = key_id(low);
        clean(K);
    }

    // Lists with at least this many admitted entries are merged whole rather than inserted one by one.
    static constexpr int kListMergeMin = 3;

    // Admits a whole sorted list given in descending order over the 64*S positions: position p holds the list's
    // entry 64*S-1-p, or the empty slot where the list has none (a list of K entries fills the last K positions).
    // A few admitted entries go in one by one. More go in by one bitonic merge: the elementwise minimum of the
    // ascending list and the descending one is a bitonic sequence holding the 64*S smallest pairs of both, which
    // the clean sorts; no sort of the incoming list is needed.
    __device__ __forceinline__ void admit_desc(float (&cd)[S], int32_t (&ci)[S], int K) {
        int admitted = 0;
#pragma unroll
        for (int s = 0; s < S; ++s)
            admitted += __popcll(__builtin_amdgcn_ballot_w64((cd[s] <= filter) & (ci[s] != kEmptyId)));
        if (admitted == 0) return;
        if (admitted < kListMergeMin) {
#pragma unroll
            for (int s = 0; s < S; ++s) offer(cd[s], ci[s], ci[s] != kEmptyId, K);
            return;
        }
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const uint64_t c = pair_key(cd[s], ci[s]), own = pair_key(d[s], id[s]);
            const uint64_t low = c < own ? c : own;
            d[s] = key_dist(low);
            id[s] = key_id(low);
        }
        clean(K);
    }

    // Sorts the list after an elementwise minimum left it bitonic, and reads the new threshold.
    __device__ __forceinline__ void clean(int K) {
        uint64_t k[S];
#pragma unroll
        for (int s = 0; s < S; ++s) k[s] = pair_key(d[s], id[s]);
#pragma unroll
        for (int h = S / 2; h > 0; h >>= 1)  // register distances (S is a power of two)
#pragma unroll
            for (int s = 0; s < S; ++s)
                if ((s & h) == 0) {
                    const bool swap = k[s + h] < k[s];
                    const uint64_t lo = swap ? k[s + h] : k[s], hi = swap ? k[s] : k[s + h];
                    k[s] = lo;
                    k[s + h] = hi;
                }
#pragma unroll
        for (int s = 0; s < S; ++s) {
            wave_clean(k[s]);
            d[s] = key_dist(k[s]);
            id[s] = key_id(k[s]);
        }
        refresh(K);
    }

    // Writes entries 0..K-1 to dst (LDS or global).
    __device__ __forceinline__ void store(Pair* dst, int K) const {
        const int lane = __lane_id();
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int p = s * WAVE + lane;
            if (p < K) dst[p] = Pair{d[s], id[s]};
        }
    }
};

// Streams pairs [begin, all) of consecutive partial lists through a wave list: four 64-pair chunks per round (four
// loads in flight), rounds `step` pairs apart so that several waves can split one range. The list takes them with
// bulk admission (merge_wave): a chunk of sorted partial lists admits many pairs at once while the list fills.
template <int S>
__device__ __forceinline__ void stream_pairs(WaveList<S, true>& wl, const Pair* first, int begin, int step, int all,
                                             int K, int lane) {
    constexpr int B = 4;
    for (int base = begin; base < all; base += step) {
        Pair p[B];
#pragma unroll
        for (int u = 0; u < B; ++u) {
            const int e = base + u * WAVE + lane;
            p[u] = e < all ? first[e] : Pair{INFINITY, kEmptyId};
        }
#pragma unroll
        for (int u = 0; u < B; ++u) wl.offer(p[u].d, p[u].i, p[u].i != kEmptyId, K);
    }
}

// Streams whole partial lists [begin, lists), `step` lists apart, through a wave list: each sorted list of K
// pairs is read into the wave list's layout in descending order and admitted by `admit_desc`, with the next four
// lists' loads in flight. For long lists (K > 32): after the first few, a list still admits about K / j of its
// entries at the j-th, which one by one cost far more than one merge network.
template <int S>
__device__ __forceinline__ void stream_lists(WaveList<S, true>& wl, const Pair* first, int begin, int step,
                                             int lists, int K, int lane) {
    constexpr int L = 4;
    float rd[L][S];
    int32_t ri[L][S];
    auto load = [&](int l, float (&dd)[S], int32_t (&ii)[S]) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int j = S * WAVE - 1 - (s * WAVE + lane);  // the list's entry at this position
            const bool have = l < lists && j < K;
            const Pair e = have ? first[static_cast<int64_t>(l) * K + j] : Pair{INFINITY, kEmptyId};
            dd[s] = e.d;
            ii[s] = e.i;
        }
    };
#pragma unroll
    for (int u = 0; u < L; ++u) load(begin + u * step, rd[u], ri[u]);
    for (int l0 = begin; l0 < lists; l0 += L * step) {
#pragma unroll
        for (int u = 0; u < L; ++u) {
            const int l = l0 + u * step;
            if (l >= lists) break;
            float cd[S];
            int32_t ci[S];
#pragma unroll
            for (int s = 0; s < S; ++s) {
                cd[s] = rd[u][s];
                ci[s] = ri[u][s];
            }
            load(l + L * step, rd[u], ri[u]);
            wl.admit_desc(cd, ci, K);
        }
    }
}

// Merges share `part` of `parts` (waves splitting one merge) of `lists` consecutive partial lists of K sorted pairs
// into a wave list: whole lists, every parts-th, when they are long; else rounds of four 64-pair chunks, every
// parts-th round (several short lists per ballot).
template <int S>
__device__ __forceinline__ void stream_partials(WaveList<S, true>& wl, const Pair* first, int part, int parts,
                                                int lists, int K, int lane) {
    if (K > 32) stream_lists(wl, first, part, parts, lists, K, lane);
    else stream_pairs(wl, first, part * 4 * WAVE, parts * 4 * WAVE, lists * K, K, lane);
}

// Number of entries of the sorted list l[0..K) that precede e: strictly less when strict, else less-or-equal.
__device__ __forceinline__ int count_before(const Pair* l, int K, Pair e, bool strict) {
    int lo = 0, hi = K;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        const Pair v = l[mid];
        const bool before = strict ? pair_less(v.d, v.i, e.d, e.i) : !pair_less(e.d, e.i, v.d, v.i);
        if (before) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

// Merges L sorted lists of K pairs (lists[l * K + j], in LDS) into their `limit` (<= K) smallest, written to
// out[0..limit) (LDS or global). Rank of an entry = its index in its own list + entries of earlier lists that are
// <= it + entries of later lists that are < it; ranks are unique even with equal (sentinel) entries. With `pad`
// (final results), empty slots are written as the reference's {+inf, -1} and distances are scaled by 2^shift
// (exact; fp16-table sums). All threads of the block call it; the caller synchronises before (lists written) and,
// for LDS output, after (out read).
__device__ __forceinline__ void merge_lists(const Pair* lists, int L, int K, Pair* out, int tid, int nthreads,
                                            int limit, bool pad, int shift = 0) {
    for (int t = tid; t < L * K; t += nthreads) {
        const int l = t / K, j = t % K;
        const Pair e = lists[t];
        int rank = j;
        for (int o = 0; o < L && rank < limit; ++o)
            if (o != l) rank += count_before(lists + o * K, K, e, o > l);
        if (rank < limit) {
            if (pad && e.i == kEmptyId) out[rank] = Pair{INFINITY, -1};
            else out[rank] = Pair{pad && shift ? ldexpf(e.d, shift) : e.d, e.i};
        }
    }
}
__device__ __forceinline__ void merge_lists(const Pair* lists, int L, int K, Pair* out, int tid, int nthreads) {
    merge_lists(lists, L, K, out, tid, nthreads, K, false);
}

}  // namespace vk
