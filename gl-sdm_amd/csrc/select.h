// Exact top-K selection on 64-bit rank keys, shared by the route kernels.
//
// A group of G adjacent lanes owns one score row.  Each lane keeps a
// descending top-K list of keys in registers (K a power of two).  Elements
// arrive in chunks of K per lane: a chunk is sorted by a bitonic network and
// merged into the list by a bitonic merge that keeps the K largest.  The G
// lists are finally merged by a butterfly over __shfl_xor, after which every
// lane of the group holds the row's exact top-K.  Keys are distinct (the index
// is part of the key), so "the K largest keys" is well defined and equals the
// reference's chain of stable argsorts.
#pragma once

#include "glsdm_internal.h"

namespace glsdm {

template <int K, bool DESC>
__device__ __forceinline__ void bitonic_sort(uint64_t (&v)[K])
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
                    const uint64_t a = v[i], b = v[j];
                    const bool swap = down ? (a < b) : (a > b);
                    v[i] = swap ? b : a;
                    v[j] = swap ? a : b;
                }
            }
        }
    }
}

// t <- the K largest of t U c; both sorted descending, result sorted descending.
template <int K>
__device__ __forceinline__ void merge_top(uint64_t (&t)[K], const uint64_t (&c)[K])
{
#pragma unroll
    for (int i = 0; i < K; ++i) t[i] = t[i] > c[K - 1 - i] ? t[i] : c[K - 1 - i];
#pragma unroll
    for (int stride = K >> 1; stride > 0; stride >>= 1) {
#pragma unroll
        for (int i = 0; i < K; ++i) {
            const int j = i ^ stride;
            if (j > i) {
                const uint64_t a = t[i], b = t[j];
                t[i] = a > b ? a : b;
                t[j] = a > b ? b : a;
            }
        }
    }
}

template <int K>
__device__ __forceinline__ void list_clear(uint64_t (&t)[K])
{
#pragma unroll
    for (int i = 0; i < K; ++i) t[i] = 0;
}

// Merge one unsorted chunk of K keys into the lane's running list.
template <int K>
__device__ __forceinline__ void list_absorb(uint64_t (&t)[K], uint64_t (&c)[K])
{
    bitonic_sort<K, true>(c);
    merge_top<K>(t, c);
}

// Butterfly merge of the G lane lists of a group (G a power of two <= 64).
template <int K, int G>
__device__ __forceinline__ void group_merge(uint64_t (&t)[K])
{
#pragma unroll
    for (int s = 1; s < G; s <<= 1) {
        uint64_t p[K];
#pragma unroll
        for (int q = 0; q < K; ++q) p[q] = shfl_xor_u64(t[q], s);
        merge_top<K>(t, p);
    }
}

// Exact top-K keys of `n` elements produced by key_of(i), for the G-lane group
// that lane g belongs to (element i is read by lane i % G).
template <int K, int G, typename KeyOf>
__device__ __forceinline__ void group_top(int n, int g, KeyOf key_of, uint64_t (&t)[K])
{
    list_clear<K>(t);
    for (int base = 0; base < n; base += G * K) {
        uint64_t c[K];
#pragma unroll
        for (int q = 0; q < K; ++q) {
            const int i = base + q * G + g;
            c[q] = i < n ? key_of(i) : 0;
        }
        list_absorb<K>(t, c);
    }
    group_merge<K, G>(t);
}

// Candidate stage and output of one route row.  i0/v0 and i1/v1 hold the
// kk = min(width, half) best sub-keys of the two factors (indices and scores);
// all G lanes of the group call this and lane g writes outputs w % G == g.
template <int K, int G>
__device__ __forceinline__ void finish_route(const uint32_t *i0, const float *v0, const uint32_t *i1,
                                             const float *v1, int half, int width, int tie, int g, bool live,
                                             int64_t *index_row, float *weight_row)
{
    const int kk = width < half ? width : half;
    uint64_t t[K];
    group_top<K, G>(kk * kk, g, [&](int c) {
        const int i = c / kk, j = c - i * kk;
        const float s = v0[i] + v1[j];
        return rank_key(s, i0[i] * (uint32_t)half + i1[j], tie);
    }, t);

    // chosen slots in ascending order, softmax over their sums
    uint64_t u[K];
#pragma unroll
    for (int w = 0; w < K; ++w) {
        if (w < width) {
            const uint32_t slot = rank_index(t[w], tie);
            const float s = order_value((uint32_t)(t[w] >> 32));
            u[w] = ((uint64_t)slot << 32) | __float_as_uint(s);
        } else {
            u[w] = ~0ull;
        }
    }
    bitonic_sort<K, false>(u);
    float m = -INFINITY;
#pragma unroll
    for (int w = 0; w < K; ++w) {
        if (w < width) {
            const float s = __uint_as_float((uint32_t)u[w]);
            m = (s > m || s != s) ? s : m;
        }
    }
    float e[K];
    float total = 0.0f;
#pragma unroll
    for (int w = 0; w < K; ++w) {
        if (w < width) {
            e[w] = expf(__uint_as_float((uint32_t)u[w]) - m);
            total += e[w];
        }
    }
    const float inv = 1.0f / total;
    if (live) {
#pragma unroll
        for (int w = 0; w < K; ++w) {
            if (w < width && w % G == g) {
                index_row[w] = (int64_t)(u[w] >> 32);
                weight_row[w] = e[w] * inv;
            }
        }
    }
}

}  // namespace glsdm
