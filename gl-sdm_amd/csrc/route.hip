// Product-key routing of fp32 or bf16 factor scores on gfx950.
//
// Semantics (S/ = projects/gl-sdm/src/gl_sdm/): S/memory/routing.py:10-26 with
// tie HIGHEST, S/layers/router.py:39-61 with tie LOWEST.  Every element is
// ranked by a distinct key (monotone score bits above tie bits of its index),
// which is the total order the reference's chain of stable argsorts induces,
// so "top-k by key" reproduces the reference's selection exactly, including
// ties and signed zeros.  fp32 scores use double keys (a 48-bit key as a
// positive normal double: compare-exchange = v_max_f64 + v_min_f64); bf16
// scores (the bf16 router projections of the stack, which the reference widens
// with .float()) use 32-bit keys that order exactly as the widened values'
// keys (v_max_u32 + v_min_u32).
//
// Work decomposition: a group of G adjacent lanes owns one score row.  Each
// lane keeps a descending top-K list of keys in registers (K = width rounded
// up to a power of two) and streams its share of the row in chunks of K
// consecutive elements (16-byte loads where the row layout allows): a chunk is
// sorted by a sorting network and merged into the list by a bitonic merge that
// keeps the K largest.  The G lists of the group are then merged by a
// butterfly, after which every lane of the group holds the row's exact top-K.
// Factor lists go through LDS to the candidate stage (kk*kk fp32 sums), which
// runs the same selection; the chosen slots are sorted ascending and weighted
// by a softmax.
//
// Split path, for launches that would leave most CUs idle (decode: one token
// per stream): route_part_kernel blocks each own one factor and one range of
// its columns for 256/G rows and write the range's exact top-K (as 64-bit keys)
// to a caller workspace; route_merge_kernel (select.h) merges them and runs the
// candidate stage and softmax.  Same results, bit for bit.
#include "select.h"

namespace glsdm {

template <typename TS> struct ScoreKey;
template <> struct ScoreKey<float> {
    using KT = double;
    __device__ __forceinline__ static KT key(float x, uint32_t i, int tie) { return rank_keyd(x, i, tie); }
};
template <> struct ScoreKey<bf16_t> {
    using KT = uint32_t;
    __device__ __forceinline__ static KT key(bf16_t x, uint32_t i, int tie) { return rank_key16(x, i, tie); }
};

// Keys of elements [start, start + K) of a factor row (0 beyond n).  `vec`: the
// row and `start` are 16-byte aligned, so whole 16-byte pieces are loaded.
template <typename TS, int K>
__device__ __forceinline__ void chunk_keys(const TS *__restrict__ f, int start, int n, bool vec, int tie,
                                           typename ScoreKey<TS>::KT (&c)[K])
{
    constexpr int PER = 16 / sizeof(TS);
    if constexpr (K % PER == 0) {
        if (vec && start + K <= n) {
#pragma unroll
            for (int v = 0; v < K / PER; ++v) {
                const uint4 u = *reinterpret_cast<const uint4 *>(f + start + v * PER);
                const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int e = 0; e < PER; ++e) {
                    TS x;
                    if constexpr (sizeof(TS) == 4)
                        x = __uint_as_float(w[e]);
                    else
                        x = (bf16_t)((e & 1) ? (w[e >> 1] >> 16) : (w[e >> 1] & 0xFFFFu));
                    const int i = start + v * PER + e;
                    c[v * PER + e] = ScoreKey<TS>::key(x, (uint32_t)i, tie);
                }
            }
            return;
        }
    }
#pragma unroll
    for (int q = 0; q < K; ++q) {
        const int i = start + q;
        c[q] = i < n ? ScoreKey<TS>::key(f[i], (uint32_t)i, tie) : 0;
    }
}

// Exact top-K keys of factor-row elements [lo, hi) for the G-lane group: lane g
// takes the K-element chunks lo + g*K, lo + (g+G)*K, ...
template <typename TS, int K, int G>
__device__ __forceinline__ void range_top(const TS *__restrict__ f, int lo, int hi, int g, bool vec, int tie,
                                          typename ScoreKey<TS>::KT (&t)[K])
{
    using KT = typename ScoreKey<TS>::KT;
    list_clear<K>(t);
    bool first = true;
    for (int base = lo; base < hi; base += G * K) {
        KT c[K];
        chunk_keys<TS, K>(f, base + g * K, hi, vec, tie, c);
        if (first)
            list_first<K>(t, c);
        else
            list_absorb<K>(t, c);
        first = false;
    }
    group_merge<K, G>(t);
}

template <int K, int G, bool PAIR, typename TS>
__global__ __launch_bounds__(256) void route_kernel(const TS *__restrict__ scores, int64_t rows, int half,
                                                    int width, int tie, bool vec, int64_t *__restrict__ index,
                                                    float *__restrict__ weights)
{
    using KT = typename ScoreKey<TS>::KT;
    constexpr int RPB = 256 / G;
    __shared__ uint32_t s_idx[RPB][2][K];
    __shared__ float s_val[RPB][2][K];
    __shared__ uint16_t s_pairs[STAIR_MAX];

    const int lr = threadIdx.x / G;
    const int g = threadIdx.x % G;
    const int64_t row = (int64_t)blockIdx.x * RPB + lr;
    const bool live = row < rows;
    const int64_t r = live ? row : rows - 1;
    const TS *f0 = scores + r * 2 * (int64_t)half;
    const TS *f1 = f0 + half;
    const int kk = width < half ? width : half;
    const int npairs = staircase_build(s_pairs, kk, width);

    // 1. per-factor top-kk sub-keys (both factors in the same pass unless K = 64)
    bool finite = true;
    if constexpr (PAIR) {
        KT t0[K], t1[K];
        list_clear<K>(t0);
        list_clear<K>(t1);
        for (int base = 0; base < half; base += G * K) {
            KT c0[K], c1[K];
            chunk_keys<TS, K>(f0, base + g * K, half, vec, tie, c0);
            chunk_keys<TS, K>(f1, base + g * K, half, vec, tie, c1);
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
            KT t0[K];
            range_top<TS, K, G>(f ? f1 : f0, 0, half, g, vec, tie, t0);
            const bool fa = stash_factor<K, G>(t0, kk, tie, g, s_idx[lr][f], s_val[lr][f]);
            finite = finite && fa;
        }
    }
    __syncthreads();

    // 2. best `width` cells of the kk x kk grid of fp32 sums, ascending slots, softmax
    route_tail<K, G>(s_idx[lr][0], s_val[lr][0], s_idx[lr][1], s_val[lr][1], half, width, tie, g, s_pairs, npairs,
                     finite, live, index + row * width, weights + row * width);
}

// One block: 256/G rows, factor f, columns [s*span, s*span + span) of that factor.
template <int K, int G, typename TS>
__global__ __launch_bounds__(256) void route_part_kernel(const TS *__restrict__ scores, int64_t rows, int half,
                                                         int tie, bool vec, int splits, int span,
                                                         uint64_t *__restrict__ parts)
{
    using KT = typename ScoreKey<TS>::KT;
    constexpr int RPB = 256 / G;
    // block order: column range fastest, then factor, then row tile
    int64_t bid = blockIdx.x;
    const int s = (int)(bid % splits);
    bid /= splits;
    const int f = (int)(bid % 2);
    const int64_t row = (bid / 2) * RPB + threadIdx.x / G;
    const int g = threadIdx.x % G;
    const int64_t r = row < rows ? row : rows - 1;
    const int lo = s * span, hi = min(half, lo + span);
    KT t[K];
    range_top<TS, K, G>(scores + (r * 2 + f) * (int64_t)half, lo, hi, g, vec, tie, t);
    if (row < rows) {
        uint64_t *out = parts + ((row * 2 + f) * splits + s) * K;
#pragma unroll
        for (int w = 0; w < K; ++w) {
            if (w % G == g) out[w] = widen_key(t[w], tie);
        }
    }
}

// Shape of the split path for (rows, half, width): 0 splits when the single
// kernel already fills the GPU or the factor is too short to split.
struct RouteSplit {
    int splits, span;
    size_t bytes;
};

constexpr int64_t ROUTE_SPLIT_MIN_BLOCKS = 256;   // single-kernel launches below one block per CU split
#ifndef GLSDM_ROUTE_SPLIT_TARGET
#define GLSDM_ROUTE_SPLIT_TARGET 1024
#endif
constexpr int64_t ROUTE_SPLIT_TARGET_BLOCKS = GLSDM_ROUTE_SPLIT_TARGET;

static int route_group(int K) { return K >= 32 ? 8 : 4; }

static RouteSplit route_split(int64_t rows, int half, int width)
{
    RouteSplit p{0, 0, 0};
    const int K = pow2_ceil(width), G = route_group(K);
    if (rows <= 0 || ceil_div(rows, 256 / G) >= ROUTE_SPLIT_MIN_BLOCKS) return p;
    const int piece = G * K;                               // columns one group pass covers
    const int pieces = (int)ceil_div(half, piece);
    if (pieces < 2) return p;
    const int64_t tiles = ceil_div(rows, 256 / G) * 2;
    int splits = 1;
    while (splits < pieces && tiles * splits < ROUTE_SPLIT_TARGET_BLOCKS) splits <<= 1;
    if (splits > pieces) splits = pieces;
    p.span = (int)ceil_div(pieces, splits) * piece;
    p.splits = (int)ceil_div(half, p.span);
    p.bytes = (size_t)rows * 2 * (size_t)p.splits * (size_t)K * sizeof(uint64_t);
    return p;
}

template <int K, typename TS>
static int launch_route(const TS *scores, int64_t rows, int half, int width, int tie, bool vec,
                        const RouteSplit &sp, uint64_t *parts, int64_t *index, float *weights, hipStream_t st)
{
    constexpr int G = K >= 32 ? 8 : 4;
    constexpr int RPB = 256 / G;
    if (parts) {
        const int64_t blocks = ceil_div(rows, RPB) * 2 * sp.splits;
        hipLaunchKernelGGL((route_part_kernel<K, G, TS>), dim3((unsigned)blocks), dim3(256), 0, st, scores, rows,
                           half, tie, vec, sp.splits, sp.span, parts);
        int rc = check_launch("route_part_kernel");
        if (rc) return rc;
        // 16 lanes per row merge the range lists (more blocks for few rows); the
        // candidate and output stages keep the single kernel's G-lane groups, whose
        // softmax summation order fixes the bits
        constexpr int MG = G > 16 ? G : 16;
        if constexpr (K == 16 || K == 32) {
            if ((int64_t)half * half <= (1ll << 30)) {
                // one wavefront per row (the same bits as route_merge_kernel<K, G, MG>)
                hipLaunchKernelGGL((route_merge_wave_kernel<K, G, 8>), dim3((unsigned)ceil_div(rows, 4)), dim3(256),
                                   0, st, parts, rows, sp.splits, half, width, tie, index, weights, KeyArgs{},
                                   (int64_t)1);
                return check_launch("route_merge_wave_kernel");
            }
        }
        hipLaunchKernelGGL((route_merge_kernel<K, G, MG>), dim3((unsigned)ceil_div(rows, 256 / MG)), dim3(256), 0,
                           st, parts, rows, sp.splits, half, width, tie, index, weights, KeyArgs{}, (int64_t)1);
        return check_launch("route_merge_kernel");
    }
    hipLaunchKernelGGL((route_kernel<K, G, (K < 64), TS>), dim3((unsigned)ceil_div(rows, RPB)), dim3(256), 0, st,
                       scores, rows, half, width, tie, vec, index, weights);
    return check_launch("route_kernel");
}

template <typename TS>
static int route_typed(const TS *scores, int64_t rows, int half, int width, int tie, void *workspace,
                       size_t workspace_bytes, int64_t *index, float *weights, hipStream_t st)
{
    const bool vec = ((reinterpret_cast<uintptr_t>(scores) & 15) == 0) && ((half * sizeof(TS)) % 16 == 0);
    const RouteSplit sp = route_split(rows, half, width);
    uint64_t *parts = nullptr;
    if (sp.splits > 0 && workspace && workspace_bytes >= sp.bytes && (reinterpret_cast<uintptr_t>(workspace) & 7) == 0)
        parts = static_cast<uint64_t *>(workspace);
    switch (pow2_ceil(width)) {
    case 1: return launch_route<1>(scores, rows, half, width, tie, vec, sp, parts, index, weights, st);
    case 2: return launch_route<2>(scores, rows, half, width, tie, vec, sp, parts, index, weights, st);
    case 4: return launch_route<4>(scores, rows, half, width, tie, vec, sp, parts, index, weights, st);
    case 8: return launch_route<8>(scores, rows, half, width, tie, vec, sp, parts, index, weights, st);
    case 16: return launch_route<16>(scores, rows, half, width, tie, vec, sp, parts, index, weights, st);
    case 32: return launch_route<32>(scores, rows, half, width, tie, vec, sp, parts, index, weights, st);
    default: return launch_route<64>(scores, rows, half, width, tie, vec, sp, parts, index, weights, st);
    }
}

int route_launch(const void *scores, int32_t scores_dtype, int64_t rows, int half, int width, int tie,
                 void *workspace, size_t workspace_bytes, int64_t *index, float *weights, hipStream_t st)
{
    if (rows < 0) return fail(GLSDM_ERR_ARG, "route: rows must be >= 0");
    if (!dtype_ok(scores_dtype)) return fail(GLSDM_ERR_ARG, "route: scores dtype must be fp32 or bf16");
    if (half < 1 || half > 65535) return fail(GLSDM_ERR_UNSUPPORTED, "route: half must be in [1, 65535]");
    if (width < 1 || width > 64) return fail(GLSDM_ERR_UNSUPPORTED, "route: width must be in [1, 64]");
    if ((int64_t)width > (int64_t)half * half) return fail(GLSDM_ERR_ARG, "route: width exceeds slots");
    if (tie != GLSDM_TIE_HIGHEST && tie != GLSDM_TIE_LOWEST) return fail(GLSDM_ERR_ARG, "route: bad tie rule");
    if (rows == 0) return GLSDM_OK;
    if (!scores || !index || !weights) return fail(GLSDM_ERR_ARG, "route: null pointer");
    if (rows > (int64_t)0x7FFFFFFF * 8) return fail(GLSDM_ERR_UNSUPPORTED, "route: too many rows");
    if (scores_dtype == GLSDM_F32)
        return route_typed(static_cast<const float *>(scores), rows, half, width, tie, workspace, workspace_bytes,
                           index, weights, st);
    return route_typed(static_cast<const bf16_t *>(scores), rows, half, width, tie, workspace, workspace_bytes,
                       index, weights, st);
}

size_t route_workspace(int64_t rows, int half, int width) { return route_split(rows, half, width).bytes; }

}  // namespace glsdm

extern "C" int glsdm_route_workspace_bytes(int64_t rows, int32_t half, int32_t width, size_t *bytes)
{
    if (!bytes) return glsdm::fail(GLSDM_ERR_ARG, "route_workspace_bytes: null output");
    if (rows < 0 || half < 1 || half > 65535 || width < 1 || width > 64)
        return glsdm::fail(GLSDM_ERR_ARG, "route_workspace_bytes: bad shape");
    *bytes = glsdm::route_workspace(rows, half, width);
    return GLSDM_OK;
}

extern "C" int glsdm_route(const void *scores, int32_t scores_dtype, int64_t rows, int32_t half, int32_t width,
                           int32_t tie, int64_t *index, float *weights, void *workspace, size_t workspace_bytes,
                           void *stream)
{
    return glsdm::route_launch(scores, scores_dtype, rows, half, width, tie, workspace, workspace_bytes, index,
                               weights, glsdm::as_stream(stream));
}
