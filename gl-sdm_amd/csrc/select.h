// Exact top-K selection on rank keys, shared by the route kernels.  Factor keys
// are doubles for fp32 scores (a 48-bit key as a positive normal double) and
// 32-bit integers for bf16 scores; candidate keys are 64-bit integers
// (glsdm_internal.h).  The list primitives are generic over the key type.
//
// A group of G adjacent lanes owns one score row.  Each lane keeps a
// descending top-K list of keys in registers (K a power of two).  Elements
// arrive in chunks of K per lane: a chunk is sorted by a sorting network (the
// 60-comparator network of sortnet16.h for K = 16, bitonic otherwise) and
// merged into the list by a bitonic merge that keeps the K largest.  The G
// lists are finally merged by a butterfly (DPP quad permutes for the two
// innermost levels, __shfl_xor beyond), after which every lane of the group
// holds the row's exact top-K.  Keys are distinct (the index is part of the
// key), so "the K largest keys" is well defined and equals the reference's
// chain of stable argsorts.
//
// Candidate stage: with both factor lists sorted, cell (i, j) of the sum grid
// is dominated by the (i+1)(j+1)-1 cells (i' <= i, j' <= j), whose fp32 sums
// are >= its own (rounding is monotone).  The selection therefore runs on the
// staircase P = {(i, j): (i+1)(j+1) <= width} only, and then *verifies* that
// every cell outside P scores strictly below the width-th pick: per grid row
// the first excluded cell bounds all later ones, so one check per row suffices.
// Ties at the boundary, infinities or NaN among the factor scores send the row
// to the full-grid selection, so the result is exact in every case.
#pragma once

#include "glsdm_internal.h"
#include "sortnet16.h"

namespace glsdm {

// Larger / smaller of two distinct keys: v_max_u32 / v_min_u32 for 32-bit keys,
// v_max_f64 / v_min_f64 for double keys, compare + selects for 64-bit keys.
__device__ __forceinline__ uint32_t kmax(uint32_t a, uint32_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint32_t kmin(uint32_t a, uint32_t b) { return a > b ? b : a; }
__device__ __forceinline__ uint64_t kmax(uint64_t a, uint64_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint64_t kmin(uint64_t a, uint64_t b) { return a > b ? b : a; }
__device__ __forceinline__ double kmax(double a, double b) { return __builtin_fmax(a, b); }
__device__ __forceinline__ double kmin(double a, double b) { return __builtin_fmin(a, b); }

template <int K, bool DESC, typename KT>
__device__ __forceinline__ void bitonic_sort(KT (&v)[K])
{
#pragma unroll
    for (int size = 2; size <= K; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
#pragma unroll
            for (int i = 0; i < K; ++i) {
                const int j = i ^ stride;
                if (j > i) {
                    const bool down = ((i & size) == 0) == DESC;
                    const KT a = v[i], b = v[j];
                    v[i] = down ? kmax(a, b) : kmin(a, b);
                    v[j] = down ? kmin(a, b) : kmax(a, b);
                }
            }
        }
    }
}

// t <- the K largest of t U c; both sorted descending, result sorted descending.
template <int K, typename KT>
__device__ __forceinline__ void merge_top(KT (&t)[K], const KT (&c)[K])
{
#pragma unroll
    for (int i = 0; i < K; ++i) t[i] = kmax(t[i], c[K - 1 - i]);
#pragma unroll
    for (int stride = K >> 1; stride > 0; stride >>= 1) {
#pragma unroll
        for (int i = 0; i < K; ++i) {
            const int j = i ^ stride;
            if (j > i) {
                const KT a = t[i], b = t[j];
                t[i] = kmax(a, b);
                t[j] = kmin(a, b);
            }
        }
    }
}

template <int K, typename KT>
__device__ __forceinline__ void list_clear(KT (&t)[K])
{
#pragma unroll
    for (int i = 0; i < K; ++i) t[i] = 0;
}

// Sort of 16 keys with the 60-comparator network (bitonic needs 80);
// descending unless ASC.
template <bool ASC = false, typename KT>
__device__ __forceinline__ void sort16(KT (&v)[16])
{
#pragma unroll
    for (int c = 0; c < SORTNET16_SIZE; ++c) {
        const int i = SORTNET16[c][0], j = SORTNET16[c][1];
        const KT a = v[i], b = v[j];
        v[i] = ASC ? kmin(a, b) : kmax(a, b);
        v[j] = ASC ? kmax(a, b) : kmin(a, b);
    }
}

template <int K, bool DESC, typename KT>
__device__ __forceinline__ void chunk_sort(KT (&c)[K])
{
    if constexpr (K == 16)
        sort16<!DESC>(c);
    else
        bitonic_sort<K, DESC>(c);
}

// Merge one unsorted chunk of K keys into the lane's running list.
template <int K, typename KT>
__device__ __forceinline__ void list_absorb(KT (&t)[K], KT (&c)[K])
{
    chunk_sort<K, true>(c);
    merge_top<K>(t, c);
}

// A lane's first chunk: sorted, it is the list (no merge with an empty list).
template <int K, typename KT>
__device__ __forceinline__ void list_first(KT (&t)[K], KT (&c)[K])
{
    chunk_sort<K, true>(c);
#pragma unroll
    for (int i = 0; i < K; ++i) t[i] = c[i];
}

// Value of lane (lane ^ S) for S in {1, 2} through a DPP quad permute, else a shuffle.
template <int S>
__device__ __forceinline__ uint32_t lane_xor(uint32_t v)
{
    if constexpr (S == 1)
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
    else if constexpr (S == 2)
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
    else
        return (uint32_t)__shfl_xor((int)v, S);
}

template <int S>
__device__ __forceinline__ uint64_t lane_xor(uint64_t v)
{
    return ((uint64_t)lane_xor<S>((uint32_t)(v >> 32)) << 32) | lane_xor<S>((uint32_t)v);
}

template <int S>
__device__ __forceinline__ double lane_xor(double v)
{
    return __longlong_as_double((long long)lane_xor<S>((uint64_t)__double_as_longlong(v)));
}

template <int K, int S, typename KT>
__device__ __forceinline__ void butterfly_level(KT (&t)[K])
{
    KT p[K];
#pragma unroll
    for (int q = 0; q < K; ++q) p[q] = lane_xor<S>(t[q]);
    merge_top<K>(t, p);
}

// Butterfly merge of the G lane lists of a group (G a power of two <= 64).
template <int K, int G, typename KT>
__device__ __forceinline__ void group_merge(KT (&t)[K])
{
    if constexpr (G > 1) butterfly_level<K, 1>(t);
    if constexpr (G > 2) butterfly_level<K, 2>(t);
    if constexpr (G > 4) butterfly_level<K, 4>(t);
    if constexpr (G > 8) butterfly_level<K, 8>(t);
    if constexpr (G > 16) butterfly_level<K, 16>(t);
    if constexpr (G > 32) butterfly_level<K, 32>(t);
}

// Two independent lists merged level by level (more independent work per level).
template <int K, int G, typename KT>
__device__ __forceinline__ void group_merge2(KT (&t)[K], KT (&u)[K])
{
    if constexpr (G > 1) { butterfly_level<K, 1>(t); butterfly_level<K, 1>(u); }
    if constexpr (G > 2) { butterfly_level<K, 2>(t); butterfly_level<K, 2>(u); }
    if constexpr (G > 4) { butterfly_level<K, 4>(t); butterfly_level<K, 4>(u); }
    if constexpr (G > 8) { butterfly_level<K, 8>(t); butterfly_level<K, 8>(u); }
    if constexpr (G > 16) { butterfly_level<K, 16>(t); butterfly_level<K, 16>(u); }
    if constexpr (G > 32) { butterfly_level<K, 32>(t); butterfly_level<K, 32>(u); }
}

// Exact top-K keys of `n` elements produced by key_of(i), for the G-lane group
// that lane g belongs to (element i is read by lane i % G).
template <int K, int G, typename KeyOf, typename KT>
__device__ __forceinline__ void group_top(int n, int g, KeyOf key_of, KT (&t)[K])
{
    if constexpr (K >= 32) {
        // at most K/2 elements per lane: sort those, the zero sentinels stay below
        if (n <= G * (K / 2)) {
            KT c[K / 2];
#pragma unroll
            for (int q = 0; q < K / 2; ++q) {
                const int i = q * G + g;
                c[q] = i < n ? key_of(i) : 0;
            }
            chunk_sort<K / 2, true>(c);
#pragma unroll
            for (int q = 0; q < K; ++q) t[q] = q < K / 2 ? c[q] : 0;
            group_merge<K, G>(t);
            return;
        }
    }
    if (n <= 0) list_clear<K>(t);
    for (int base = 0; base < n; base += G * K) {
        KT c[K];
#pragma unroll
        for (int q = 0; q < K; ++q) {
            const int i = base + q * G + g;
            c[q] = i < n ? key_of(i) : 0;
        }
        if (base == 0)
            list_first<K>(t, c);
        else
            list_absorb<K>(t, c);
    }
    group_merge<K, G>(t);
}

// ------------------------------------------------------------------ staircase

constexpr int STAIR_MAX = 280;   // |P| for width 64 (sum over n <= 64 of floor(64 / n))

// Builds the staircase cells (i << 8 | j) of P for (kk, width) in LDS;
// every thread of the block calls it, the caller synchronises before use.
// Lane i of each wavefront takes row i's length (kk <= 64); a shuffle scan
// gives the row offsets, and the first wavefront writes the cells.
__device__ __forceinline__ int staircase_build(uint16_t *pairs, int kk, int width)
{
    const int i = threadIdx.x & 63;
    const int len = i < kk ? min(kk, width / (i + 1)) : 0;
    int incl = len;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(incl, off);
        if (i >= off) incl += y;
    }
    const int total = __shfl(incl, 63);
    if (threadIdx.x < 64)
        for (int j = 0; j < len; ++j) pairs[incl - len + j] = (uint16_t)((i << 8) | j);
    return total;
}

// Optional proposal-key outputs of a route (glsdm_score_route_keys): for row
// (request b, position t, head h) the pick of slot s gets the absolute address
// a = (b*H + h)*S + s and the collision key a*chunk*layers + (offset + t)*layers
// + layer, at its output position (the arithmetic of glsdm_proposal_keys).
struct KeyArgs {
    int64_t *addr, *keys;        // [rows, width] each; addr == nullptr: no key outputs
    int64_t T, S, offset, chunk, layers, layer;
};

struct KeyRow {
    int64_t *addr, *keys;
    int64_t base, mul, add;
};

// The key outputs of flattened route row r = (b*T + t)*H + h.
__device__ __forceinline__ KeyRow key_row(const KeyArgs &ka, int64_t r, int64_t H, int width)
{
    const int64_t h = r % H, bt = r / H, t = bt % ka.T, b = bt / ka.T;
    return KeyRow{ka.addr + r * width, ka.keys + r * width, (b * H + h) * ka.S, ka.chunk * ka.layers,
                  (ka.offset + t) * ka.layers + ka.layer};
}

// Keys of the candidate stage (cells of the sum grid): the fp32 sum's order
// bits above the slot's tie bits.  CellKey64 is the plain 64-bit key;
// CellKeyD packs the same order into a positive normal double when the slots
// fit `ib` <= 30 bits (compare-exchange = v_max_f64 + v_min_f64).
struct CellKey64 {
    using KT = uint64_t;
    int tie;
    __device__ __forceinline__ KT make(float s, uint32_t slot) const { return rank_key(s, slot, tie); }
    __device__ __forceinline__ uint32_t order(KT k) const { return (uint32_t)(k >> 32); }
    __device__ __forceinline__ uint32_t slot(KT k) const { return rank_index(k, tie); }
};

struct CellKeyD {
    using KT = double;
    int tie, ib, shift;        // shift = 30 - ib: the 32 + ib key bits end at bit 62
    uint32_t imask;
    __device__ __forceinline__ KT make(float s, uint32_t slot) const
    {
        const uint32_t t = tie == GLSDM_TIE_HIGHEST ? slot : imask - slot;
        const uint64_t k = ((uint64_t)order_bits(s) << ib) | t;
        return __longlong_as_double((long long)((1ull << 52) + (k << shift)));
    }
    __device__ __forceinline__ uint64_t raw(KT k) const
    {
        return ((uint64_t)__double_as_longlong(k) - (1ull << 52)) >> shift;
    }
    __device__ __forceinline__ uint32_t order(KT k) const { return (uint32_t)(raw(k) >> ib); }
    __device__ __forceinline__ uint32_t slot(KT k) const
    {
        const uint32_t t = (uint32_t)raw(k) & imask;
        return tie == GLSDM_TIE_HIGHEST ? t : imask - t;
    }
};

// Best `width` cells (top-K list, descending keys) of the kk x kk sum grid of
// the factor lists i0/v0 and i1/v1 (sorted descending by rank key).
template <int K, int G, typename CK>
__device__ __forceinline__ void candidate_top(const uint32_t *i0, const float *v0, const uint32_t *i1,
                                              const float *v1, int half, int width, const CK &ck, int g,
                                              const uint16_t *pairs, int npairs, bool finite,
                                              typename CK::KT (&t)[K])
{
    const int kk = width < half ? width : half;
    auto cell = [&](int i, int j) {
        const float s = v0[i] + v1[j];
        return ck.make(s, i0[i] * (uint32_t)half + i1[j]);
    };
    bool exact = false;
    if (finite && npairs >= width) {
        group_top<K, G>(npairs, g, [&](int c) {
            const int pr = pairs[c];
            return cell(pr >> 8, pr & 0xFF);
        }, t);
        // verify: the first excluded cell of each grid row scores strictly below the width-th pick
        uint32_t tau = 0;
#pragma unroll
        for (int w = 0; w < K; ++w)
            if (w == width - 1) tau = ck.order(t[w]);
        bool ok = true;
        for (int i = g; i < kk; i += G) {
            const int j = min(kk, width / (i + 1));
            if (j < kk) ok = ok && order_bits(v0[i] + v1[j]) < tau;
        }
        // all G lanes of the group must agree
        uint64_t bad = __ballot(!ok);
        const int lane = threadIdx.x & 63;
        const uint64_t mine = ((G >= 64) ? ~0ull : ((1ull << G) - 1ull)) << (lane & ~(G - 1));
        exact = (bad & mine) == 0;
    }
    if (!exact) {
        group_top<K, G>(kk * kk, g, [&](int c) {
            const int i = c / kk;
            return cell(i, c - i * kk);
        }, t);
    }
}

// Output stage of one route row from its candidate list t (top-K, descending;
// every lane of the group holds it): the chosen slots in ascending order and a
// softmax over their sums.  Lane g of the group handles the picks w with
// w % G == g: a pick's output position is the number of chosen slots below its
// own (slots are distinct), so no sort is needed.  The max runs over the picks
// in list order; the exponentials are summed per lane, then across the group by
// a fixed butterfly, so the result is deterministic.
template <int K, int G, typename CK>
__device__ __forceinline__ void finish_route(const typename CK::KT (&t)[K], const CK &ck, int width, int g,
                                             bool live, int64_t *index_row, float *weight_row,
                                             const KeyRow &kr)
{
    uint32_t slot[K];
    float val[K];
    float m = -INFINITY;
#pragma unroll
    for (int w = 0; w < K; ++w) {
        slot[w] = w < width ? ck.slot(t[w]) : 0xFFFFFFFFu;
        val[w] = order_value(ck.order(t[w]));
        if (w < width) m = (val[w] > m || val[w] != val[w]) ? val[w] : m;
    }
    constexpr int MINE = (K + G - 1) / G;
    // this lane's picks w = u*G + g, selected from the G candidates of each u
    // (register selects: a lane-dependent index would put the lists in scratch)
    float e[MINE];
    uint32_t my_slot[MINE];
    float part = 0.0f;
#pragma unroll
    for (int u = 0; u < MINE; ++u) {
        float x = 0.0f;
        my_slot[u] = 0xFFFFFFFFu;
#pragma unroll
        for (int q = 0; q < G; ++q) {
            if (u * G + q < K && q == g) {
                x = val[u * G + q];
                my_slot[u] = slot[u * G + q];
            }
        }
        const int w = u * G + g;
        e[u] = 0.0f;
        if (w < width && w < K) {
            e[u] = expf(x - m);
            part += e[u];
        }
    }
    float total = part;
#pragma unroll
    for (int x = 1; x < G; x <<= 1) total += __shfl_xor(total, x);
    const float inv = 1.0f / total;
    if (live) {
#pragma unroll
        for (int u = 0; u < MINE; ++u) {
            const int w = u * G + g;
            if (w < width && w < K) {
                int rank = 0;
#pragma unroll
                for (int j = 0; j < K; ++j) rank += slot[j] < my_slot[u] ? 1 : 0;
                index_row[rank] = (int64_t)my_slot[u];
                weight_row[rank] = e[u] * inv;
                if (kr.addr) {
                    const int64_t a = kr.base + (int64_t)my_slot[u];
                    kr.addr[rank] = a;
                    kr.keys[rank] = a * kr.mul + kr.add;
                }
            }
        }
    }
}

// Candidate stage + output stage of one route row from its stashed factor
// lists: double cell keys when the slots fit 30 bits, else 64-bit keys.
template <int K, int G>
__device__ __forceinline__ void route_tail(const uint32_t *i0, const float *v0, const uint32_t *i1, const float *v1,
                                           int half, int width, int tie, int g, const uint16_t *pairs, int npairs,
                                           bool finite, bool live, int64_t *index_row, float *weight_row,
                                           const KeyRow &kr = KeyRow{nullptr, nullptr, 0, 0, 0})
{
    const int64_t slots = (int64_t)half * half;
    if (slots <= (1ll << 30)) {
        int ib = 1;
        while ((1ll << ib) < slots) ++ib;
        const CellKeyD ck{tie, ib, 30 - ib, (uint32_t)((1ull << ib) - 1ull)};
        double t[K];
        candidate_top<K, G>(i0, v0, i1, v1, half, width, ck, g, pairs, npairs, finite, t);
        finish_route<K, G>(t, ck, width, g, live, index_row, weight_row, kr);
    } else {
        const CellKey64 ck{tie};
        uint64_t t[K];
        candidate_top<K, G>(i0, v0, i1, v1, half, width, ck, g, pairs, npairs, finite, t);
        finish_route<K, G>(t, ck, width, g, live, index_row, weight_row, kr);
    }
}

// route_tail for width == 16 with factor lists of 16 (kk = 16) and slots in 30
// bits, G = 4: the staircase of P is fixed (rows of 16, 8, 5, 4, 3, 2, 2, 2
// and eight of 1 cells, 50 in all), so lane g takes a fixed set of at most 15
// cells -- columns j = g (mod 4) of rows 0-7 and column 0 of rows 8+g and 12+g
// -- read from the stashed lists without a pairs table, keyed exactly as
// CellKeyD does (finite factor scores: their sums are never NaN).  The
// verification and the full-grid fallback are candidate_top's.
__device__ __forceinline__ void route_tail16(const uint32_t *i0, const float *v0, const uint32_t *i1, const float *v1,
                                             int half, int tie, int g, const uint16_t *pairs, bool finite, bool live,
                                             int64_t *index_row, float *weight_row, const KeyRow &kr)
{
    constexpr int K = 16, G = 4, W = 16;
    int ib = 1;
    while ((1ll << ib) < (int64_t)half * half) ++ib;
    const CellKeyD ck{tie, ib, 30 - ib, (uint32_t)((1ull << ib) - 1ull)};
    double t[K];
    bool exact = false;
    if (finite) {
        auto cell = [&](float a, uint32_t ia, float b, uint32_t jb) -> double {
            const uint32_t x = __float_as_uint((a + b) + 0.0f);              // -0 folded onto +0
            const uint32_t ob = x ^ (uint32_t)(((int32_t)x >> 31) | (int32_t)0x80000000);
            const uint32_t slot = ia * (uint32_t)half + jb;
            const uint32_t tb = tie == GLSDM_TIE_HIGHEST ? slot : ck.imask - slot;
            return __hiloint2double((int)((ob >> 2) + 0x00100000u), (int)((ob << 30) | (tb << ck.shift)));
        };
        float w1[4];
        uint32_t x1[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            w1[q] = v1[g + 4 * q];
            x1[q] = i1[g + 4 * q];
        }
        const float b0 = v1[0];
        const uint32_t jb0 = i1[0];
        double c[K];
#pragma unroll
        for (int q = 0; q < 4; ++q) c[q] = cell(v0[0], i0[0], w1[q], x1[q]);        // row 0
        c[4] = cell(v0[1], i0[1], w1[0], x1[0]);                                      // row 1: j = g, g + 4
        c[5] = cell(v0[1], i0[1], w1[1], x1[1]);
        c[6] = cell(v0[2], i0[2], w1[0], x1[0]);                                      // row 2: j = g, and 4
        c[7] = g == 0 ? cell(v0[2], i0[2], w1[1], x1[1]) : 0.0;
        c[8] = cell(v0[3], i0[3], w1[0], x1[0]);                                      // row 3
        c[9] = g < 3 ? cell(v0[4], i0[4], w1[0], x1[0]) : 0.0;                        // row 4
        c[10] = g < 2 ? cell(v0[5], i0[5], w1[0], x1[0]) : 0.0;                       // rows 5-7
        c[11] = g < 2 ? cell(v0[6], i0[6], w1[0], x1[0]) : 0.0;
        c[12] = g < 2 ? cell(v0[7], i0[7], w1[0], x1[0]) : 0.0;
        c[13] = cell(v0[8 + g], i0[8 + g], b0, jb0);                                  // rows 8-15: j = 0
        c[14] = cell(v0[12 + g], i0[12 + g], b0, jb0);
        c[15] = 0.0;
        list_first<K>(t, c);
        group_merge<K, G>(t);
        // verify: the first excluded cell of each row (column len_i) scores below the 16th pick
        const uint32_t tau = ck.order(t[W - 1]);
        bool ok = true;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int i = g + 4 * q;
            const int j = i == 0 ? W : i == 1 ? 8 : i == 2 ? 5 : i == 3 ? 4 : i == 4 ? 3 : i < 8 ? 2 : 1;
            if (j < W) ok = ok && order_bits(v0[i] + v1[j]) < tau;
        }
        const uint64_t bad = __ballot(!ok);
        const int lane = threadIdx.x & 63;
        exact = ((bad >> (lane & ~(G - 1))) & 0xFull) == 0;
    }
    if (!exact) candidate_top<K, G>(i0, v0, i1, v1, half, W, ck, g, pairs, 0, false, t);
    finish_route<K, G>(t, ck, W, g, live, index_row, weight_row, kr);
}

// Stashes the top-kk of a factor list (indices and scores) for the candidate
// stage; returns whether all kk scores are finite.
template <int K, int G, typename KT>
__device__ __forceinline__ bool stash_factor(const KT (&t)[K], int kk, int tie, int g, uint32_t *idx,
                                             float *val)
{
    bool finite = true;
#pragma unroll
    for (int i = 0; i < K; ++i) {
        if (i < kk) {
            const float v = key_value(t[i]);
            finite = finite && (fabsf(v) <= 3.402823466e38f);
            if (i % G == g) {
                idx[i] = key_index(t[i], tie);
                val[i] = v;
            }
        }
    }
    return finite;
}

// Second kernel of the split paths (score_part_kernel, route_part_kernel): one
// G-lane group per row merges the row's per-range lists of each factor (64-bit
// keys; each range list holds its range's K best, K >= kk, so the merge is
// exact), then runs the candidate stage and the softmax.
template <int K, int G, int MG = G>
__global__ __launch_bounds__(256) void route_merge_kernel(const uint64_t *__restrict__ parts, int64_t rows,
                                                          int splits, int half, int width, int tie,
                                                          int64_t *__restrict__ index, float *__restrict__ weights,
                                                          KeyArgs ka, int64_t heads)
{
    // MG >= G lanes per row merge the range lists; the candidate and output
    // stages then run in G-lane subgroups (each subgroup computes the same
    // result; the first one writes it), so the softmax sums in the same order
    // as a G-lane kernel and the bits do not depend on MG.
    static_assert(MG >= G && MG % G == 0, "merge group");
    constexpr int RPB = 256 / MG;
    __shared__ uint32_t s_idx[RPB][2][K];
    __shared__ float s_val[RPB][2][K];
    __shared__ uint16_t s_pairs[STAIR_MAX];
    const int lr = threadIdx.x / MG, m = threadIdx.x % MG, g = m % G;
    const int64_t row = (int64_t)blockIdx.x * RPB + lr;
    const bool live = row < rows;
    const int64_t r = live ? row : rows - 1;
    const int kk = width < half ? width : half;
    const int npairs = staircase_build(s_pairs, kk, width);
    bool finite = true;
    // the range lists hold 64-bit factor keys (index < 65536): merged as double keys
#pragma unroll
    for (int f = 0; f < 2; ++f) {
        double t[K];
        if (m < splits) {
            const uint64_t *src = parts + ((r * 2 + f) * splits + m) * K;
#pragma unroll
            for (int w = 0; w < K; ++w) t[w] = narrow_keyd(src[w]);
        } else {
            list_clear<K>(t);
        }
        for (int s = m + MG; s < splits; s += MG) {
            const uint64_t *src = parts + ((r * 2 + f) * splits + s) * K;
            double c[K];
#pragma unroll
            for (int w = 0; w < K; ++w) c[w] = narrow_keyd(src[w]);
            merge_top<K>(t, c);
        }
        group_merge<K, MG>(t);
        bool ok = true;
        if (m < G) ok = stash_factor<K, G>(t, kk, tie, g, s_idx[lr][f], s_val[lr][f]);
        finite = finite && ok;
    }
    __syncthreads();
    const KeyRow kr = ka.addr ? key_row(ka, r, heads, width) : KeyRow{nullptr, nullptr, 0, 0, 0};
    route_tail<K, G>(s_idx[lr][0], s_val[lr][0], s_idx[lr][1], s_val[lr][1], half, width, tie, g, s_pairs, npairs,
                     finite, live && m < G, index + r * width, weights + r * width, kr);
}

// ------------------------------------------------------------ wave-per-row merge
//
// Sorting networks over keys held E per lane, blocked across a wavefront:
// element i lives in lane i / E, register i % E.  Cross-lane steps exchange
// whole registers with lane ^ (stride / E).

// One compare-exchange step over elements i and i ^ STRIDE: the lower index
// keeps the larger key where desc(i) holds, the smaller one elsewhere.
template <int E, int STRIDE, typename KT, typename DescFn>
__device__ __forceinline__ void wave_cx(KT (&v)[E], int lane, DescFn desc)
{
    if constexpr (STRIDE >= E) {
        constexpr int M = STRIDE / E;
        const bool upper = (lane & M) != 0;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const KT x = lane_xor<M>(v[e]);
            v[e] = (desc(lane * E + e) != upper) ? kmax(v[e], x) : kmin(v[e], x);
        }
    } else {
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int f = e ^ STRIDE;
            if (f > e) {
                const KT a = v[e], b = v[f];
                const bool d = desc(lane * E + e);
                v[e] = d ? kmax(a, b) : kmin(a, b);
                v[f] = d ? kmin(a, b) : kmax(a, b);
            }
        }
    }
}

template <int E, int SIZE, int STRIDE, typename KT>
__device__ __forceinline__ void wave_sort_stage(KT (&v)[E], int lane)
{
    wave_cx<E, STRIDE>(v, lane, [](int i) { return (i & SIZE) == 0; });
    if constexpr (STRIDE > 1) wave_sort_stage<E, SIZE, STRIDE / 2>(v, lane);
}

template <int E, int SIZE, typename KT>
__device__ __forceinline__ void wave_sort_from(KT (&v)[E], int lane)
{
    wave_sort_stage<E, SIZE, SIZE / 2>(v, lane);
    if constexpr (SIZE < 64 * E) wave_sort_from<E, SIZE * 2>(v, lane);
}

// Bitonic sort of the wavefront's 64*E keys, descending (element 0 the largest).
template <int E, typename KT>
__device__ __forceinline__ void wave_sort_desc(KT (&v)[E], int lane)
{
    wave_sort_from<E, 2>(v, lane);
}

// Half-cleaner of a bitonic sequence of K keys held E per lane in segments of
// K / E lanes: afterwards each segment's list is sorted descending.
template <int E, int S, typename KT>
__device__ __forceinline__ void seg_clean(KT (&v)[E], int lane)
{
    wave_cx<E, S>(v, lane, [](int) { return true; });
    if constexpr (S > 1) seg_clean<E, S / 2>(v, lane);
}

// Lists of K keys sorted descending, one per segment of P = K / E lanes: each
// segment gets the top K of its own list and that of segment seg ^ M.  The
// partner list is read reversed (lane pl takes lane P-1-pl's registers in
// reverse), so the elementwise maximum is bitonic and holds the top K.
template <int K, int E, int M, typename KT>
__device__ __forceinline__ void seg_merge(KT (&v)[E], int lane)
{
    constexpr int P = K / E;
    KT x[E];
#pragma unroll
    for (int e = 0; e < E; ++e) x[e] = lane_xor<M * P + P - 1>(v[E - 1 - e]);
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = kmax(v[e], x[e]);
    seg_clean<E, K / 2>(v, lane);
}

// Butterfly over the first `used` segments (a power of two) of each half-wave.
template <int K, int E, int M, typename KT>
__device__ __forceinline__ void seg_butterfly(KT (&v)[E], int lane, int used)
{
    constexpr int NSEG = 32 / (K / E);                // segments per half-wave
    if constexpr (M < NSEG) {
        if (M < used) seg_merge<K, E, M>(v, lane);     // wave-uniform
        seg_butterfly<K, E, 2 * M>(v, lane, used);
    }
}

// Wave-per-row variant of route_merge_kernel for the split paths' K = 16 and 32
// with slots in 30 bits: one wavefront per row, so the merge, the candidate
// stage and their selections run on 64 lanes instead of one lane group.
//   merge      half-wave f merges factor f: segment s (P = K / E lanes) loads
//              range lists s, s + NSEG, ... (folded in), then a butterfly of
//              bitonic merges leaves the factor's top K in every segment
//   candidates the staircase cells (E2 per lane) are keyed as CellKeyD and
//              sorted across the wave; the same verification as
//              candidate_top, else the whole kk x kk grid (E3 per lane)
//   output     the sorted top-K through LDS into finish_route's G-lane group,
//              so the slots, the softmax and its summation order are those of
//              route_merge_kernel<K, G> bit for bit.
template <int K, int G, int E>
__global__ __launch_bounds__(256) void route_merge_wave_kernel(const uint64_t *__restrict__ parts, int64_t rows,
                                                               int splits, int half, int width, int tie,
                                                               int64_t *__restrict__ index,
                                                               float *__restrict__ weights, KeyArgs ka,
                                                               int64_t heads)
{
    static_assert(K % E == 0 && (K == 16 || K == 32) && K * K % 64 == 0, "wave merge shape");
    constexpr int P = K / E, NSEG = 32 / P;
    constexpr int E2 = K == 16 ? 1 : 2;               // staircase of width <= K: at most 50 / 119 cells
    constexpr int E3 = K * K / 64;                    // the whole kk x kk grid, kk <= K
    __shared__ uint32_t s_idx[4][2][K];
    __shared__ float s_val[4][2][K];
    __shared__ double s_t[4][K];
    __shared__ uint16_t s_pairs[STAIR_MAX];
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + wv;
    const bool live = row < rows;
    const int64_t r = live ? row : rows - 1;
    const int kk = width < half ? width : half;
    const int npairs = staircase_build(s_pairs, kk, width);

    // 1. factor lists: half-wave f, segment seg, lane pl of the segment
    const int f = lane >> 5, seg = (lane & 31) / P, pl = lane % P;
    double v[E];
    const uint64_t *base = parts + (r * 2 + f) * splits * (int64_t)K;
    if (seg < splits) {
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = narrow_keyd(base[(int64_t)seg * K + pl * E + e]);
    } else {
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = 0.0;
    }
    // more range lists than segments: each segment folds in lists seg + NSEG, ...
    // (read reversed; a segment without one takes empty keys, which keep its
    // list as it is), every lane in every round since the clean crosses lanes
    for (int s0 = NSEG; s0 < splits; s0 += NSEG) {
        const int s = s0 + seg;
        const uint64_t *src = base + (int64_t)s * K;
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = kmax(v[e], s < splits ? narrow_keyd(src[K - 1 - (pl * E + e)]) : 0.0);
        seg_clean<E, K / 2>(v, lane);
    }
    int used = 1;                                     // segments holding lists, to a power of two
    while (used < splits && used < NSEG) used <<= 1;
    seg_butterfly<K, E, 1>(v, lane, used);
    bool ok = true;
    if (seg == 0) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int i = pl * E + e;
            if (i < kk) {
                const float x = key_value(v[e]);
                ok = ok && (fabsf(x) <= 3.402823466e38f);
                s_idx[wv][f][i] = key_index(v[e], tie);
                s_val[wv][f][i] = x;
            }
        }
    }
    const bool finite = __ballot(!ok) == 0;
    __syncthreads();                                  // stashed lists and the staircase cells

    // 2. candidate stage
    const uint32_t *i0 = s_idx[wv][0], *i1 = s_idx[wv][1];
    const float *v0 = s_val[wv][0], *v1 = s_val[wv][1];
    int ib = 1;
    while ((1ll << ib) < (int64_t)half * half) ++ib;
    const CellKeyD ck{tie, ib, 30 - ib, (uint32_t)((1ull << ib) - 1ull)};
    auto cell = [&](int i, int j) { return ck.make(v0[i] + v1[j], i0[i] * (uint32_t)half + i1[j]); };
    bool exact = false;
    if (finite && npairs >= width) {
        double c[E2];
#pragma unroll
        for (int e = 0; e < E2; ++e) {
            const int q = lane * E2 + e;
            c[e] = 0.0;
            if (q < npairs) {
                const int pr = s_pairs[q];
                c[e] = cell(pr >> 8, pr & 0xFF);
            }
        }
        wave_sort_desc<E2>(c, lane);
        // verify: the first excluded cell of each grid row scores strictly below the width-th pick
        double wth = 0.0;
#pragma unroll
        for (int e = 0; e < E2; ++e)
            if (lane * E2 + e == width - 1) wth = c[e];
        wth = __shfl(wth, (width - 1) / E2);
        const uint32_t tau = ck.order(wth);
        bool good = true;
        if (lane < kk) {
            const int j = min(kk, width / (lane + 1));
            if (j < kk) good = order_bits(v0[lane] + v1[j]) < tau;
        }
        exact = __ballot(!good) == 0;
        if (exact) {
#pragma unroll
            for (int e = 0; e < E2; ++e)
                if (lane * E2 + e < K) s_t[wv][lane * E2 + e] = c[e];
        }
    }
    if (!exact) {                                     // wave-uniform
        double c[E3];
#pragma unroll
        for (int e = 0; e < E3; ++e) {
            const int q = lane * E3 + e;
            c[e] = 0.0;
            if (q < kk * kk) {
                const int i = q / kk;
                c[e] = cell(i, q - i * kk);
            }
        }
        wave_sort_desc<E3>(c, lane);
#pragma unroll
        for (int e = 0; e < E3; ++e)
            if (lane * E3 + e < K) s_t[wv][lane * E3 + e] = c[e];
    }
    __syncthreads();

    // 3. output: every lane holds the list; the first G lanes write the row
    double t[K];
#pragma unroll
    for (int w = 0; w < K; ++w) t[w] = s_t[wv][w];
    const KeyRow kr = ka.addr ? key_row(ka, r, heads, width) : KeyRow{nullptr, nullptr, 0, 0, 0};
    finish_route<K, G>(t, ck, width, lane % G, live && lane < G, index + r * width, weights + r * width, kr);
}

}  // namespace glsdm
