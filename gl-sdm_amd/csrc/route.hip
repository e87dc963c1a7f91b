// Product-key routing of fp32 factor scores on gfx950.
//
// Semantics (S/ = projects/gl-sdm/src/gl_sdm/): S/memory/routing.py:10-26 with
// tie HIGHEST, S/layers/router.py:39-61 with tie LOWEST.  Every element is
// ranked by a distinct 64-bit key (monotone score bits << 32 | tie bits of its
// index), which is the total order the reference's chain of stable argsorts
// induces, so "top-k by key" reproduces the reference's selection exactly,
// including ties and signed zeros.
//
// Work decomposition: a group of G adjacent lanes owns one score row.  Each
// lane keeps a descending top-K list of 64-bit keys in registers (K = width
// rounded up to a power of two).  It streams its strided share of the row in
// chunks of K: a chunk is sorted by a bitonic network and merged into the list
// by a bitonic merge that keeps the K largest.  The G lists of the group are
// then merged by a butterfly over __shfl_xor, after which every lane of the
// group holds the row's exact top-K.  Factor lists go through LDS to the
// candidate stage (kk*kk fp32 sums), which runs the same selection; the chosen
// slots are sorted ascending and weighted by a softmax.
#include "select.h"

namespace glsdm {

template <int K, int G, bool PAIR>
__global__ __launch_bounds__(256) void route_kernel(const float *__restrict__ scores, int64_t rows,
                                                    int half, int width, int tie,
                                                    int64_t *__restrict__ index,
                                                    float *__restrict__ weights)
{
    constexpr int RPB = 256 / G;
    __shared__ uint32_t s_idx[RPB][2][K];
    __shared__ float s_val[RPB][2][K];
    __shared__ uint16_t s_pairs[STAIR_MAX];

    const int lr = threadIdx.x / G;
    const int g = threadIdx.x % G;
    const int64_t row = (int64_t)blockIdx.x * RPB + lr;
    const bool live = row < rows;
    const int64_t r = live ? row : rows - 1;
    const float *f0 = scores + r * 2 * (int64_t)half;
    const float *f1 = f0 + half;
    const int kk = width < half ? width : half;
    const int npairs = staircase_build(s_pairs, kk, width);

    // 1. per-factor top-kk sub-keys (both factors in the same pass unless K = 64)
    bool finite = true;
    if constexpr (PAIR) {
        uint64_t t0[K], t1[K];
        list_clear<K>(t0);
        list_clear<K>(t1);
        for (int base = 0; base < half; base += G * K) {
            uint64_t c0[K], c1[K];
#pragma unroll
            for (int q = 0; q < K; ++q) {
                const int i = base + q * G + g;
                c0[q] = i < half ? rank_key(f0[i], (uint32_t)i, tie) : 0;
                c1[q] = i < half ? rank_key(f1[i], (uint32_t)i, tie) : 0;
            }
            if (base == 0) {
                list_first<K>(t0, c0);
                list_first<K>(t1, c1);
            } else {
                list_absorb<K>(t0, c0);
                list_absorb<K>(t1, c1);
            }
        }
        group_merge2<K, G>(t0, t1);
        const bool fa = stash_factor<K, G>(t0, kk, tie, g, s_idx[lr][0], s_val[lr][0]);
        const bool fb = stash_factor<K, G>(t1, kk, tie, g, s_idx[lr][1], s_val[lr][1]);
        finite = fa && fb;
    } else {
#pragma unroll
        for (int f = 0; f < 2; ++f) {
            const float *fs = f ? f1 : f0;
            uint64_t t0[K];
            group_top<K, G>(half, g, [&](int i) { return rank_key(fs[i], (uint32_t)i, tie); }, t0);
            const bool fa = stash_factor<K, G>(t0, kk, tie, g, s_idx[lr][f], s_val[lr][f]);
            finite = finite && fa;
        }
    }
    __syncthreads();

    // 2. best `width` cells of the kk x kk grid of fp32 sums, ascending slots, softmax
    uint64_t t[K];
    candidate_top<K, G>(s_idx[lr][0], s_val[lr][0], s_idx[lr][1], s_val[lr][1], half, width, tie, g, s_pairs,
                        npairs, finite, t);
    finish_route<K, G>(t, width, tie, g, live, index + row * width, weights + row * width);
}

template <int K, int G, bool PAIR = (K < 64)>
static int launch_route(const float *scores, int64_t rows, int half, int width, int tie,
                        int64_t *index, float *weights, hipStream_t st)
{
    constexpr int RPB = 256 / G;
    const int64_t blocks = ceil_div(rows, RPB);
    hipLaunchKernelGGL((route_kernel<K, G, PAIR>), dim3((unsigned)blocks), dim3(256), 0, st, scores, rows,
                       half, width, tie, index, weights);
    return check_launch("route_kernel");
}

int route_launch(const float *scores, int64_t rows, int half, int width, int tie, int64_t *index,
                 float *weights, hipStream_t st)
{
    if (rows < 0) return fail(GLSDM_ERR_ARG, "route: rows must be >= 0");
    if (half < 1 || half > 65535) return fail(GLSDM_ERR_UNSUPPORTED, "route: half must be in [1, 65535]");
    if (width < 1 || width > 64) return fail(GLSDM_ERR_UNSUPPORTED, "route: width must be in [1, 64]");
    if ((int64_t)width > (int64_t)half * half) return fail(GLSDM_ERR_ARG, "route: width exceeds slots");
    if (tie != GLSDM_TIE_HIGHEST && tie != GLSDM_TIE_LOWEST) return fail(GLSDM_ERR_ARG, "route: bad tie rule");
    if (rows == 0) return GLSDM_OK;
    if (!scores || !index || !weights) return fail(GLSDM_ERR_ARG, "route: null pointer");
    if (rows > (int64_t)0x7FFFFFFF * 8) return fail(GLSDM_ERR_UNSUPPORTED, "route: too many rows");
    switch (pow2_ceil(width)) {
    case 1: return launch_route<1, 4>(scores, rows, half, width, tie, index, weights, st);
    case 2: return launch_route<2, 4>(scores, rows, half, width, tie, index, weights, st);
    case 4: return launch_route<4, 4>(scores, rows, half, width, tie, index, weights, st);
    case 8: return launch_route<8, 4>(scores, rows, half, width, tie, index, weights, st);
    case 16: return launch_route<16, 4>(scores, rows, half, width, tie, index, weights, st);
    case 32: return launch_route<32, 8>(scores, rows, half, width, tie, index, weights, st);
    default: return launch_route<64, 8>(scores, rows, half, width, tie, index, weights, st);
    }
}

}  // namespace glsdm

extern "C" int glsdm_route(const float *scores, int64_t rows, int32_t half, int32_t width, int32_t tie,
                           int64_t *index, float *weights, void *stream)
{
    return glsdm::route_launch(scores, rows, half, width, tie, index, weights, glsdm::as_stream(stream));
}
