// Fused address scoring + product-key routing on gfx950.
//
// One block owns R = 256/G tokens of one head h.  The sub-key columns of both
// factors (one factor at a time for K = 64, to fit LDS) are streamed in chunks
// of CW: the block stages the chunk's sub-key rows in LDS once (padded rows;
// for K <= 16, the larger lists need the LDS themselves), its four wavefronts
// compute the chunk's R x CW fp32 scores with v_mfma_f32_16x16x32_bf16 (query
// fragments stay in registers for the whole kernel) and drop them in LDS;
// then every G-lane group folds its token's CW scores into
// its exact top-K lists (select.h).  Scores never reach HBM unless the caller
// asks for them (scores_out, used for parity checks).  Blocks are numbered
// head-fastest, so with 8 heads on 8 XCDs each XCD's L2 serves one head's
// sub-key table.
//
// Split path, for launches that would leave most CUs idle (few tokens, one
// head): score_part_kernel blocks each own one factor and one range of its
// sub-key columns for R tokens and write that range's exact top-K keys to a
// caller workspace; route_merge_kernel merges a token's per-range lists into
// the factor lists (exact: each range list holds its range's K best, K >= kk)
// and runs the candidate stage and softmax.  Same results, bit for bit.
//
// Semantics: scores as glsdm_score, routing as glsdm_route (the chosen slots,
// weights and tie rule are identical on identical scores).
#include <type_traits>

#include "select.h"

namespace glsdm {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float floatx4_t;

constexpr int KS_MAX = 8;   // dk <= 256

// score_route16.hip: the filtered kernel for 9-16 picks and the shapes it takes.
bool score_route16_takes(int dk, int half, int width);
int score_route16_launch(const void *q, const void *keys, int64_t N, int64_t H, int dk, int half, int width,
                         int tie, int64_t *index, float *weights, const KeyArgs &ka, hipStream_t st);

// Orders LDS traffic between the lanes that produced a score chunk and the lanes
// that select from it: the wavefront itself when every wavefront owns its own
// 16 tokens end to end, else the whole block.
template <bool WAVE_LOCAL>
__device__ __forceinline__ void chunk_sync()
{
    if constexpr (WAVE_LOCAL) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    } else {
        __syncthreads();
    }
}

template <int K, int G, int CW, bool PAIR, int KSM, bool STAGE>
__global__ __launch_bounds__(256) void score_route_kernel(const bf16_t *__restrict__ q,
                                                          const bf16_t *__restrict__ keys, int64_t N,
                                                          int64_t H, int dk, int half, int width, int tie,
                                                          float *__restrict__ scores_out,
                                                          int64_t *__restrict__ index,
                                                          float *__restrict__ weights, KeyArgs ka)
{
    constexpr int R = 256 / G;       // tokens per block
    constexpr int RT = R / 16;       // 16-row MFMA tiles
    constexpr int WPR = 4 / RT;      // wavefronts per row tile
    constexpr int CT = CW / 16;      // 16-column tiles per chunk and factor
    constexpr int CTW = CT / WPR;    // column tiles per wavefront and factor
    constexpr int SUB = CW / (G * K);
    constexpr int LDW = CW + 4;      // padded LDS score row (keeps 16-byte alignment)
    constexpr int NF = PAIR ? 2 : 1; // factors per pass over the sub-keys
    constexpr int LDK = KSM * 32 + 8;              // padded LDS sub-key row (bf16), breaks bank aliasing
    constexpr int VPR = KSM * 4;                   // 16-byte pieces per sub-key row at the largest dk
    constexpr int PIECES = (NF * CW * VPR + 255) / 256;   // staged pieces per thread and chunk
    constexpr int SKN = STAGE ? NF : 1, SKC = STAGE ? CW : 1, SKL = STAGE ? LDK : 8;
    // With G = 4 the 16-token MFMA tile of wavefront w is exactly the 16 tokens its
    // lanes select for, so no other wavefront touches its score rows.
    constexpr bool WAVE_LOCAL = (RT == 4 && WPR == 1 && G == 4);
    static_assert(RT >= 1 && RT <= 4 && CT % WPR == 0 && CTW >= 1 && SUB >= 1, "tiling");
    // With both factors in one pass the score chunks are dead once the chunk loop
    // ends, so the factor lists of the candidate stage reuse their LDS (a block
    // barrier separates the two); one factor per pass keeps them apart.
    constexpr int SC_WORDS = NF * R * LDW, LIST_WORDS = 2 * R * 2 * K;
    constexpr int LIST_AT = PAIR ? 0 : SC_WORDS;
    constexpr int BUF_WORDS = (LIST_AT + LIST_WORDS > SC_WORDS) ? LIST_AT + LIST_WORDS : SC_WORDS;
    __shared__ __attribute__((aligned(16))) float s_buf[BUF_WORDS];
    __shared__ __attribute__((aligned(16))) bf16_t s_k[SKN][SKC][SKL];
    __shared__ uint16_t s_pairs[STAIR_MAX];
    auto s_sc = reinterpret_cast<float (*)[R][LDW]>(s_buf);
    auto s_idx = reinterpret_cast<uint32_t (*)[2][K]>(s_buf + LIST_AT);
    auto s_val = reinterpret_cast<float (*)[2][K]>(s_buf + LIST_AT + R * 2 * K);

    const int h = (int)(blockIdx.x % H);
    const int64_t n0 = (int64_t)(blockIdx.x / H) * R;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rt = wave % RT, cshare = wave / RT;
    const int li = lane & 15, kq = lane >> 4;
    const int L = 2 * half;
    const int ks = dk / 32;
    const int vpr = dk / 8;          // 16-byte pieces per sub-key row

    const int lr = threadIdx.x / G, g = threadIdx.x % G;
    const int64_t row_n = n0 + lr;
    const bool live = row_n < N;
    const int kk = width < half ? width : half;
    const int npairs = staircase_build(s_pairs, kk, width);

    // query fragments of this wavefront's 16-token tile, for all k-steps
    int64_t qn = n0 + rt * 16 + li;
    if (qn >= N) qn = N - 1;
    const bf16_t *qrow = q + (qn * H + h) * dk + kq * 8;
    bf16x8_t qa[KSM];
#pragma unroll
    for (int s = 0; s < KSM; ++s)
        if (s < ks) qa[s] = *reinterpret_cast<const bf16x8_t *>(qrow + s * 32);

    const bf16_t *hkeys = keys + (int64_t)h * L * dk;
    // cooperative staging of a chunk's sub-key rows in LDS: piece p of this
    // thread is (factor, column, 16-byte slice) = decode(threadIdx.x + 256 * p)
    auto stage_chunk = [&](int fp, int c0) {
        if constexpr (STAGE) {
#pragma unroll
            for (int p = 0; p < PIECES; ++p) {
                const int id = threadIdx.x + 256 * p;
                const int fi = id / (CW * vpr), rem = id - fi * (CW * vpr);
                const int col = rem / vpr, sl = rem - col * vpr;
                if (fi < NF && c0 + col < half)
                    *reinterpret_cast<uint4 *>(&s_k[fi][col][sl * 8]) = *reinterpret_cast<const uint4 *>(
                        hkeys + (int64_t)((fp + fi) * half + c0 + col) * dk + sl * 8);
            }
        }
    };

    bool finite = true;
    for (int fp = 0; fp < 2; fp += NF) {
        double ta[K], tb[K];
        list_clear<K>(ta);
        if constexpr (PAIR) list_clear<K>(tb);
        // one chunk of CW columns: MFMA scores into LDS, then each lane folds its share
        // into its lists (the pass's first chunk becomes the lists: FIRST)
        auto chunk = [&](int c0, auto first_tag) {
            constexpr bool FIRST = decltype(first_tag)::value;
            if constexpr (STAGE) {
                __syncthreads();                  // every wavefront is done with the previous s_k
                stage_chunk(fp, c0);
                __syncthreads();                  // s_k holds this chunk
            }
            // MFMA: the pass's factors' scores of columns [c0, c0 + CW) for the block's R tokens
#pragma unroll
            for (int fi = 0; fi < NF; ++fi) {
                const int f = fp + fi;
#pragma unroll
                for (int j = 0; j < CTW; ++j) {
                    const int ct = cshare * CTW + j;
                    const int col = c0 + ct * 16;
                    if (col >= half) continue;            // wave-uniform: half % 16 == 0
                    const bf16_t *krow = STAGE ? &s_k[fi][ct * 16 + li][kq * 8]
                                               : hkeys + (int64_t)(f * half + col + li) * dk + kq * 8;
                    floatx4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int s = 0; s < KSM; ++s)
                        if (s < ks)
                            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                qa[s], *reinterpret_cast<const bf16x8_t *>(krow + s * 32), acc, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; ++r) s_sc[fi][rt * 16 + 4 * kq + r][ct * 16 + li] = acc[r];
                    if (scores_out) {
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int64_t n = n0 + rt * 16 + 4 * kq + r;
                            if (n < N) scores_out[(n * H + h) * L + f * half + col + li] = acc[r];
                        }
                    }
                }
            }
            chunk_sync<WAVE_LOCAL>();
            // selection: lane g of a token folds K contiguous columns per factor into its lists
#pragma unroll
            for (int sub = 0; sub < SUB; ++sub) {
                const int first = (sub * G + g) * K;
                double a[K], b[K];
#pragma unroll
                for (int qi = 0; qi < K; ++qi) {
                    const int col = c0 + first + qi;
                    const bool in = col < half;
                    a[qi] = in ? rank_keyd(s_sc[0][lr][first + qi], (uint32_t)col, tie) : 0.0;
                    if constexpr (PAIR) b[qi] = in ? rank_keyd(s_sc[NF - 1][lr][first + qi], (uint32_t)col, tie) : 0.0;
                }
                if (FIRST && sub == 0) {
                    list_first<K>(ta, a);
                    if constexpr (PAIR) list_first<K>(tb, b);
                } else {
                    list_absorb<K>(ta, a);
                    if constexpr (PAIR) list_absorb<K>(tb, b);
                }
            }
            chunk_sync<WAVE_LOCAL>();
        };
        chunk(0, std::true_type{});
        for (int c0 = CW; c0 < half; c0 += CW) chunk(c0, std::false_type{});
        __syncthreads();   // the lists overwrite the score chunks of every wavefront
        if constexpr (PAIR) {
            group_merge2<K, G>(ta, tb);
            const bool fa = stash_factor<K, G>(ta, kk, tie, g, s_idx[lr][0], s_val[lr][0]);
            const bool fb = stash_factor<K, G>(tb, kk, tie, g, s_idx[lr][1], s_val[lr][1]);
            finite = fa && fb;
        } else {
            group_merge<K, G>(ta);
            const bool fa = stash_factor<K, G>(ta, kk, tie, g, s_idx[lr][fp], s_val[lr][fp]);
            finite = finite && fa;
        }
    }
    chunk_sync<WAVE_LOCAL>();

    const int64_t out_row = (live ? row_n : 0) * H + h;
    const KeyRow kr = ka.addr ? key_row(ka, out_row, H, width) : KeyRow{nullptr, nullptr, 0, 0, 0};
    route_tail<K, G>(s_idx[lr][0], s_val[lr][0], s_idx[lr][1], s_val[lr][1], half, width, tie, g, s_pairs, npairs,
                     finite, live, index + out_row * width, weights + out_row * width, kr);
}

// One block: R tokens of head h, factor f, sub-key columns [s*span, s*span + span).
template <int K, int G, int CW, int KSM, bool STAGE>
__global__ __launch_bounds__(256) void score_part_kernel(const bf16_t *__restrict__ q,
                                                         const bf16_t *__restrict__ keys, int64_t N, int64_t H,
                                                         int dk, int half, int tie, int splits, int span,
                                                         float *__restrict__ scores_out,
                                                         uint64_t *__restrict__ parts)
{
    constexpr int R = 256 / G;
    constexpr int RT = R / 16;
    constexpr int WPR = 4 / RT;
    constexpr int CT = CW / 16;
    constexpr int CTW = CT / WPR;
    constexpr int SUB = CW / (G * K);
    constexpr int LDW = CW + 4;
    constexpr int LDK = KSM * 32 + 8;
    constexpr int VPR = KSM * 4;
    constexpr int PIECES = (CW * VPR + 255) / 256;
    constexpr int SKC = STAGE ? CW : 1, SKL = STAGE ? LDK : 8;
    constexpr bool WAVE_LOCAL = (RT == 4 && WPR == 1 && G == 4);
    static_assert(RT >= 1 && RT <= 4 && CT % WPR == 0 && CTW >= 1 && SUB >= 1, "tiling");
    __shared__ __attribute__((aligned(16))) float s_sc[R][LDW];
    __shared__ __attribute__((aligned(16))) bf16_t s_k[SKC][SKL];

    // block order: head fastest, then column range, factor, token tile
    int64_t bid = blockIdx.x;
    const int h = (int)(bid % H);
    bid /= H;
    const int s = (int)(bid % splits);
    bid /= splits;
    const int f = (int)(bid % 2);
    const int64_t n0 = (bid / 2) * R;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rt = wave % RT, cshare = wave / RT;
    const int li = lane & 15, kq = lane >> 4;
    const int L = 2 * half;
    const int ks = dk / 32;
    const int vpr = dk / 8;
    const int lr = threadIdx.x / G, g = threadIdx.x % G;
    const int64_t row_n = n0 + lr;
    const int lo = s * span, hi = min(half, lo + span);

    int64_t qn = n0 + rt * 16 + li;
    if (qn >= N) qn = N - 1;
    const bf16_t *qrow = q + (qn * H + h) * dk + kq * 8;
    bf16x8_t qa[KSM];
#pragma unroll
    for (int t = 0; t < KSM; ++t)
        if (t < ks) qa[t] = *reinterpret_cast<const bf16x8_t *>(qrow + t * 32);
    const bf16_t *fkeys = keys + ((int64_t)h * L + (int64_t)f * half) * dk;

    double ta[K];
    list_clear<K>(ta);
    auto chunk = [&](int c0, auto first_tag) {
        constexpr bool FIRST = decltype(first_tag)::value;
        if constexpr (STAGE) {
            __syncthreads();                  // every wavefront is done with the previous s_k
#pragma unroll
            for (int p = 0; p < PIECES; ++p) {
                const int id = threadIdx.x + 256 * p;
                const int col = id / vpr, sl = id - col * vpr;
                if (col < CW && c0 + col < half)
                    *reinterpret_cast<uint4 *>(&s_k[col][sl * 8]) =
                        *reinterpret_cast<const uint4 *>(fkeys + (int64_t)(c0 + col) * dk + sl * 8);
            }
            __syncthreads();                  // s_k holds this chunk
        }
#pragma unroll
        for (int j = 0; j < CTW; ++j) {
            const int ct = cshare * CTW + j;
            const int col = c0 + ct * 16;
            if (col >= half) continue;        // wave-uniform: half % 16 == 0
            const bf16_t *krow = STAGE ? &s_k[ct * 16 + li][kq * 8] : fkeys + (int64_t)(col + li) * dk + kq * 8;
            floatx4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < KSM; ++t)
                if (t < ks)
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        qa[t], *reinterpret_cast<const bf16x8_t *>(krow + t * 32), acc, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) s_sc[rt * 16 + 4 * kq + r][ct * 16 + li] = acc[r];
            if (scores_out) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t n = n0 + rt * 16 + 4 * kq + r;
                    if (n < N) scores_out[(n * H + h) * L + f * half + col + li] = acc[r];
                }
            }
        }
        chunk_sync<WAVE_LOCAL>();
#pragma unroll
        for (int sub = 0; sub < SUB; ++sub) {
            const int first = (sub * G + g) * K;
            double a[K];
#pragma unroll
            for (int qi = 0; qi < K; ++qi) {
                const int col = c0 + first + qi;
                a[qi] = col < hi ? rank_keyd(s_sc[lr][first + qi], (uint32_t)col, tie) : 0.0;
            }
            if (FIRST && sub == 0)
                list_first<K>(ta, a);
            else
                list_absorb<K>(ta, a);
        }
        chunk_sync<WAVE_LOCAL>();
    };
    if (lo < hi) chunk(lo, std::true_type{});
    for (int c0 = lo + CW; c0 < hi; c0 += CW) chunk(c0, std::false_type{});
    group_merge<K, G>(ta);
    if (row_n < N) {
        uint64_t *out = parts + (((row_n * H + h) * 2 + f) * splits + s) * K;
#pragma unroll
        for (int w = 0; w < K; ++w)
            if (w % G == g) out[w] = widen_key(ta[w], tie);
    }
}

// The split path's shape for (N, H, half, width): 0 splits when the single
// kernel already fills the GPU (or the split path would not add blocks).
struct SplitPlan {
    int splits, span, cw, r;
    size_t bytes;
};

constexpr int64_t SPLIT_MIN_BLOCKS = 256;    // single-kernel launches below one block per CU split
constexpr int64_t SPLIT_TARGET_BLOCKS = 512;

static SplitPlan split_plan(int64_t N, int64_t H, int half, int width)
{
    SplitPlan p{0, 0, 0, 0, 0};
    const int K = pow2_ceil(width);
    const int r_single = K >= 32 ? 32 : 64;   // tokens per block of score_route_kernel (G = 8 for K >= 32)
    if (ceil_div(N, r_single) * H >= SPLIT_MIN_BLOCKS) return p;
    p.cw = K <= 16 ? 64 : 4 * K;              // G = 4 lanes per token, K columns per lane and chunk
    p.r = 64;
    const int chunks = (int)ceil_div(half, p.cw);
    const int64_t tiles = ceil_div(N, p.r) * H * 2;
    int splits = 1;
    while (splits < chunks && tiles * splits < SPLIT_TARGET_BLOCKS) splits <<= 1;
    if (splits > chunks) splits = chunks;
    p.splits = splits;
    p.span = (int)ceil_div(chunks, splits) * p.cw;
    p.bytes = (size_t)N * (size_t)H * 2 * (size_t)splits * (size_t)K * sizeof(uint64_t);
    return p;
}

template <int K>
static int launch_split(const void *q, const void *keys, int64_t N, int64_t H, int dk, int half, int width,
                        int tie, const SplitPlan &p, float *scores_out, uint64_t *parts, int64_t *index,
                        float *weights, const KeyArgs &ka, hipStream_t st)
{
    constexpr int G = 4;
    constexpr int CW = K <= 16 ? 64 : 4 * K;
    constexpr bool STAGE = K <= 16;
    const int64_t blocks = ceil_div(N, 256 / G) * H * 2 * p.splits;
    if (blocks > 0x7FFFFFFF) return fail(GLSDM_ERR_UNSUPPORTED, "score_route: grid too large");
    const bf16_t *qq = static_cast<const bf16_t *>(q), *kk = static_cast<const bf16_t *>(keys);
    if (dk <= 128)
        hipLaunchKernelGGL((score_part_kernel<K, G, CW, 4, STAGE>), dim3((unsigned)blocks), dim3(256), 0, st, qq,
                           kk, N, H, dk, half, tie, p.splits, p.span, scores_out, parts);
    else
        hipLaunchKernelGGL((score_part_kernel<K, G, CW, KS_MAX, STAGE>), dim3((unsigned)blocks), dim3(256), 0, st,
                           qq, kk, N, H, dk, half, tie, p.splits, p.span, scores_out, parts);
    int rc = check_launch("score_part_kernel");
    if (rc) return rc;
    constexpr int MG = K >= 32 ? 8 : 4;
    const int64_t rows = N * H;
    if constexpr (K == 16 || K == 32) {
        if ((int64_t)half * half <= (1ll << 30)) {
            // one wavefront per row (the same bits as route_merge_kernel<K, MG>)
            hipLaunchKernelGGL((route_merge_wave_kernel<K, MG, 8>), dim3((unsigned)ceil_div(rows, 4)), dim3(256), 0,
                               st, parts, rows, p.splits, half, width, tie, index, weights, ka, H);
            return check_launch("route_merge_wave_kernel");
        }
    }
    hipLaunchKernelGGL((route_merge_kernel<K, MG>), dim3((unsigned)ceil_div(rows, 256 / MG)), dim3(256), 0, st,
                       parts, rows, p.splits, half, width, tie, index, weights, ka, H);
    return check_launch("route_merge_kernel");
}

template <int K, int G, int CW, bool PAIR>
static int launch_score_route(const void *q, const void *keys, int64_t N, int64_t H, int dk, int half,
                              int width, int tie, float *scores_out, int64_t *index, float *weights,
                              const KeyArgs &ka, hipStream_t st)
{
    constexpr int R = 256 / G;
    const int64_t blocks = ceil_div(N, R) * H;
    if (blocks > 0x7FFFFFFF) return fail(GLSDM_ERR_UNSUPPORTED, "score_route: grid too large");
    const bf16_t *qq = static_cast<const bf16_t *>(q), *kk = static_cast<const bf16_t *>(keys);
    constexpr bool STAGE = K <= 16;   // the larger lists need the LDS for themselves
    if (dk <= 128)
        hipLaunchKernelGGL((score_route_kernel<K, G, CW, PAIR, 4, STAGE>), dim3((unsigned)blocks), dim3(256), 0,
                           st, qq, kk, N, H, dk, half, width, tie, scores_out, index, weights, ka);
    else
        hipLaunchKernelGGL((score_route_kernel<K, G, CW, PAIR, KS_MAX, STAGE>), dim3((unsigned)blocks),
                           dim3(256), 0, st, qq, kk, N, H, dk, half, width, tie, scores_out, index, weights, ka);
    return check_launch("score_route_kernel");
}

}  // namespace glsdm

using namespace glsdm;

extern "C" int glsdm_score_route_workspace_bytes(int64_t B, int64_t T, int64_t H, int32_t half, int32_t width,
                                                 size_t *bytes)
{
    if (!bytes) return fail(GLSDM_ERR_ARG, "score_route_workspace_bytes: null output");
    if (B < 0 || T < 0 || H < 1 || half < 1 || width < 1 || width > 64)
        return fail(GLSDM_ERR_ARG, "score_route_workspace_bytes: bad shape");
    *bytes = B * T == 0 ? 0 : split_plan(B * T, H, half, width).bytes;
    return GLSDM_OK;
}

static int score_route_any(const void *queries, const void *subkeys, int64_t B, int64_t T, int64_t H, int32_t dk,
                           int32_t half, int32_t width, int32_t tie, float *scores_out, int64_t *index,
                           float *weights, const KeyArgs &ka, void *workspace, size_t workspace_bytes,
                           hipStream_t st)
{
    if (B < 0 || T < 0 || H < 1 || dk < 1 || half < 1) return fail(GLSDM_ERR_ARG, "score_route: bad shape");
    if (dk % 32 != 0 || dk > 32 * KS_MAX) return fail(GLSDM_ERR_UNSUPPORTED, "score_route: dk=%d must be a multiple of 32 up to 256", dk);
    if (half % 16 != 0 || half > 65535) return fail(GLSDM_ERR_UNSUPPORTED, "score_route: half=%d must be a multiple of 16", half);
    if (width < 1 || width > 64) return fail(GLSDM_ERR_UNSUPPORTED, "score_route: width must be in [1, 64]");
    if ((int64_t)width > (int64_t)half * half) return fail(GLSDM_ERR_ARG, "score_route: width exceeds slots");
    if (tie != GLSDM_TIE_HIGHEST && tie != GLSDM_TIE_LOWEST) return fail(GLSDM_ERR_ARG, "score_route: bad tie rule");
    const int64_t N = B * T;
    if (N == 0) return GLSDM_OK;
    if (!queries || !subkeys || !index || !weights) return fail(GLSDM_ERR_ARG, "score_route: null pointer");
    if (((reinterpret_cast<uintptr_t>(queries) | reinterpret_cast<uintptr_t>(subkeys)) & 15) != 0)
        return fail(GLSDM_ERR_UNSUPPORTED, "score_route: queries and sub-keys must be 16-byte aligned");
    const SplitPlan plan = split_plan(N, H, half, width);
    if (plan.splits > 0 && workspace && workspace_bytes >= plan.bytes &&
        (reinterpret_cast<uintptr_t>(workspace) & 7) == 0) {
        uint64_t *parts = static_cast<uint64_t *>(workspace);
        switch (pow2_ceil(width)) {
        case 1: return launch_split<1>(queries, subkeys, N, H, dk, half, width, tie, plan, scores_out, parts, index, weights, ka, st);
        case 2: return launch_split<2>(queries, subkeys, N, H, dk, half, width, tie, plan, scores_out, parts, index, weights, ka, st);
        case 4: return launch_split<4>(queries, subkeys, N, H, dk, half, width, tie, plan, scores_out, parts, index, weights, ka, st);
        case 8: return launch_split<8>(queries, subkeys, N, H, dk, half, width, tie, plan, scores_out, parts, index, weights, ka, st);
        case 16: return launch_split<16>(queries, subkeys, N, H, dk, half, width, tie, plan, scores_out, parts, index, weights, ka, st);
        case 32: return launch_split<32>(queries, subkeys, N, H, dk, half, width, tie, plan, scores_out, parts, index, weights, ka, st);
        default: return launch_split<64>(queries, subkeys, N, H, dk, half, width, tie, plan, scores_out, parts, index, weights, ka, st);
        }
    }
    if (!scores_out && score_route16_takes(dk, half, width))
        return score_route16_launch(queries, subkeys, N, H, dk, half, width, tie, index, weights, ka, st);
    switch (pow2_ceil(width)) {
    case 1: return launch_score_route<1, 4, 64, true>(queries, subkeys, N, H, dk, half, width, tie, scores_out, index, weights, ka, st);
    case 2: return launch_score_route<2, 4, 64, true>(queries, subkeys, N, H, dk, half, width, tie, scores_out, index, weights, ka, st);
    case 4: return launch_score_route<4, 4, 64, true>(queries, subkeys, N, H, dk, half, width, tie, scores_out, index, weights, ka, st);
    case 8: return launch_score_route<8, 4, 64, true>(queries, subkeys, N, H, dk, half, width, tie, scores_out, index, weights, ka, st);
    case 16: return launch_score_route<16, 4, 64, true>(queries, subkeys, N, H, dk, half, width, tie, scores_out, index, weights, ka, st);
    case 32: return launch_score_route<32, 8, 256, true>(queries, subkeys, N, H, dk, half, width, tie, scores_out, index, weights, ka, st);
    default: return launch_score_route<64, 8, 512, false>(queries, subkeys, N, H, dk, half, width, tie, scores_out, index, weights, ka, st);
    }
}

extern "C" int glsdm_score_route(const void *queries, const void *subkeys, int64_t B, int64_t T, int64_t H,
                                 int32_t dk, int32_t half, int32_t width, int32_t tie, float *scores_out,
                                 int64_t *index, float *weights, void *workspace, size_t workspace_bytes,
                                 void *stream)
{
    return score_route_any(queries, subkeys, B, T, H, dk, half, width, tie, scores_out, index, weights, KeyArgs{},
                           workspace, workspace_bytes, as_stream(stream));
}

extern "C" int glsdm_score_route_keys(const void *queries, const void *subkeys, int64_t B, int64_t T, int64_t H,
                                      int32_t dk, int32_t half, int32_t width, int32_t tie, int64_t position_offset,
                                      int64_t chunk, int64_t layers, int64_t layer, int64_t *index, float *weights,
                                      int64_t *addresses, int64_t *keys, void *workspace, size_t workspace_bytes,
                                      void *stream)
{
    if (chunk < 1 || layers < 1 || layer < 0 || layer >= layers || position_offset < 0)
        return fail(GLSDM_ERR_ARG, "score_route_keys: bad key arguments");
    if (B * T > 0 && (!addresses || !keys)) return fail(GLSDM_ERR_ARG, "score_route_keys: null pointer");
    const KeyArgs ka{addresses, keys, T, (int64_t)half * half, position_offset, chunk, layers, layer};
    return score_route_any(queries, subkeys, B, T, H, dk, half, width, tie, nullptr, index, weights, ka, workspace,
                           workspace_bytes, as_stream(stream));
}
