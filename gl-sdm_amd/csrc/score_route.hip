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

// ------------------------------------------------------------ filtered K = 16 kernel
//
// score_route16_kernel: the fused kernel for routes of 9 to 16 picks (K = 16)
// with the key dimension and tie rule fixed at compile time.  A block owns 64
// tokens of one head.  The wavefronts split the sub-key columns, not the
// tokens: each keeps the query fragments of all 64 tokens in registers and
// loads only its own 16 columns of every 64-column chunk straight from L2
// (the next chunk's while the current one is multiplied), so sub-keys never
// pass through LDS and no two wavefronts fetch the same rows.  Selection is
// filtered instead of sorting every score:
//   pass 1  the maximum of every group of 4 adjacent columns is formed in
//           registers (two DPP steps across the 4 lanes holding them); the
//           K-th largest of a token's group maxima (exact, in order-bit keys)
//           is tau.  The K groups whose maxima are largest hold K distinct
//           scores >= tau, so tau is at most the factor's K-th best score and
//           every score below it can be dropped without changing the result.
//   pass 2  the scores are computed again (the MFMA work is small) and those
//           not below tau (NaN included: NaN ranks highest) are appended,
//           with their column, to the token's buffer of 32 through an LDS
//           counter (about 18 of 256 survive on random scores; their order in
//           the buffer does not matter, the keys are distinct); the factor's
//           exact top K is sorted from those alone.
// A token whose survivors overflow its buffer (heavy ties, e.g. all-equal
// scores) makes the block select that factor again the unfiltered way, every
// score keyed, sorted and merged: the result is the same list in every case,
// bit for bit.  Candidate stage and output are route_tail's.
constexpr int F16_R = 64;      // tokens per block
constexpr int F16_CW = 64;     // sub-key columns per chunk (one factor at a time), 16 per wavefront
constexpr int F16_MP = 68;     // padded LDS row of a token's 64 group maxima
constexpr int F16_SV = 32;     // survivor capacity per token and factor

// Value of lane (lane ^ S) of the same quad, S in {1, 2} (DPP quad permute).
template <int S>
__device__ __forceinline__ int quad_xor(int v)
{
    constexpr int ctrl = S == 1 ? 0xB1 : 0x4E;   // quad_perm [1,0,3,2] / [2,3,0,1]
    return __builtin_amdgcn_update_dpp(0, v, ctrl, 0xF, 0xF, false);
}

// A signed integer whose order is the fp32 order of x (-0 just below +0, a NaN
// with the sign bit clear above +inf, one with it set below -inf): three
// integer operations, no canonicalisation.
__device__ __forceinline__ int float_order(float x)
{
    const int b = __float_as_int(x);
    return b ^ ((b >> 31) & 0x7FFFFFFF);
}

// The float whose float_order is o.
__device__ __forceinline__ float float_of_order(int o)
{
    return __int_as_float(o ^ ((o >> 31) & 0x7FFFFFFF));
}

// Quad reduce-scatter of a maximum: lane j of each quad holds v[0..3]; on return
// it holds the maximum over the quad's 4 lanes of v[j].
__device__ __forceinline__ int quad_max_scatter(const int (&v)[4], int j)
{
    const bool o1 = j & 1, o2 = j & 2;
    // step 1, lanes j ^ 1: lane j keeps the rows r with r & 1 == j & 1
    const int keep0 = o1 ? v[1] : v[0], send0 = o1 ? v[0] : v[1];
    const int keep1 = o1 ? v[3] : v[2], send1 = o1 ? v[2] : v[3];
    const int w0 = max(keep0, quad_xor<1>(send0));          // row (j & 1)
    const int w1 = max(keep1, quad_xor<1>(send1));          // row 2 + (j & 1)
    // step 2, lanes j ^ 2: lane j keeps row j
    const int keep = o2 ? w1 : w0, send = o2 ? w0 : w1;
    return max(keep, quad_xor<2>(send));
}

template <int DK, int TIE>
__global__ __launch_bounds__(256) void score_route16_kernel(const bf16_t *__restrict__ q,
                                                            const bf16_t *__restrict__ keys, int64_t N, int64_t H,
                                                            int half, int width, int64_t *__restrict__ index,
                                                            float *__restrict__ weights, KeyArgs ka)
{
    constexpr int K = 16, G = 4, R = F16_R, CW = F16_CW, MP = F16_MP, SV = F16_SV;
    constexpr int KS = DK / 32;               // MFMA k-steps
    constexpr int RT = R / 16;                // 16-token row tiles
    static_assert(KS >= 1 && RT * 16 == R && CW == 64, "tiling");
    // region A: pass 1's group maxima [R][MP] (u32 order bits), then the stashed factor lists
    constexpr int A_WORDS = R * MP > R * 2 * K * 2 ? R * MP : R * 2 * K * 2;
    // region B, per factor: pass 2's survivors [R][SV] (score bits, column); the unfiltered
    // fallback's scores [R][CW] of that factor
    constexpr int B_WORDS = R * SV * 2 > R * CW ? R * SV * 2 : R * CW;
    __shared__ __attribute__((aligned(16))) uint32_t s_a[A_WORDS];
    __shared__ __attribute__((aligned(16))) uint32_t s_b[2][B_WORDS];
    __shared__ __attribute__((aligned(16))) float s_tau[2][R];
    __shared__ uint32_t s_cnt[2][R];
    __shared__ uint16_t s_pairs[STAIR_MAX];
    auto s_mx = reinterpret_cast<uint32_t (*)[MP]>(s_a);
    auto s_idx = reinterpret_cast<uint32_t (*)[2][K]>(s_a);
    auto s_val = reinterpret_cast<float (*)[2][K]>(s_a + R * 2 * K);

    const int h = (int)(blockIdx.x % H);
    const int64_t n0 = (int64_t)(blockIdx.x / H) * R;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int li = lane & 15, kq = lane >> 4;
    const int lr = tid / G, g = tid % G;      // selection roles: token lr, lane g of its G
    const int64_t row_n = n0 + lr;
    const bool live = row_n < N;
    const int kk = width < half ? width : half;
    const int npairs = staircase_build(s_pairs, kk, width);
    if (tid < 2 * R) s_cnt[tid / R][tid % R] = 0;

    // query fragments of all 64 tokens (row tile rt: tokens rt*16 + li), every k-step
    struct Queries {
        bf16x8_t a[RT][KS];
    };
    // the block's 64 query rows staged once through LDS (region B is idle until pass 2),
    // padded rows (DK + 8 bf16) so the fragment reads spread over the banks
    constexpr int LDQ = DK + 8;
    constexpr bool STAGE_Q = R * LDQ * 2 <= (int)sizeof(s_b);   // all but DK = 256
    auto stage_queries = [&]() {
        bf16_t *sq = reinterpret_cast<bf16_t *>(&s_b[0][0]);
        constexpr int PER_ROW = DK / 8, PIECES = STAGE_Q ? R * PER_ROW / 256 : 0;
#pragma unroll
        for (int p = 0; p < PIECES; ++p) {
            const int id = tid + 256 * p, row = id / PER_ROW, sl = id % PER_ROW;
            int64_t qn = n0 + row;
            if (qn >= N) qn = N - 1;
            *reinterpret_cast<uint4 *>(sq + row * LDQ + sl * 8) =
                *reinterpret_cast<const uint4 *>(q + (qn * H + h) * DK + sl * 8);
        }
        __syncthreads();
        Queries qs;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int s = 0; s < KS; ++s)
                qs.a[rt][s] = *reinterpret_cast<const bf16x8_t *>(sq + (rt * 16 + li) * LDQ + kq * 8 + s * 32);
        __syncthreads();                      // region B is free again
        return qs;
    };
    auto load_queries = [&]() {
        Queries qs;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            int64_t qn = n0 + rt * 16 + li;
            if (qn >= N) qn = N - 1;
            const bf16_t *qrow = q + (qn * H + h) * DK + kq * 8;
#pragma unroll
            for (int s = 0; s < KS; ++s) qs.a[rt][s] = *reinterpret_cast<const bf16x8_t *>(qrow + s * 32);
        }
        return qs;
    };
    const bf16_t *hk = keys + (int64_t)h * 2 * half * DK;
    const int m = half / CW;                  // chunks per factor
    const int steps = 4 * m;                  // pass 1 of factors 0, 1, then pass 2 of factors 0, 1

    // this wavefront's B fragments of a step: sub-key row (factor, c0 + 16 wave + li)
    struct Frag {
        bf16x8_t b[KS];
    };
    auto load = [&](int step) {
        const int f = (step / m) & 1, c0 = (step % m) * CW;
        const bf16_t *src = hk + (int64_t)(f * half + c0 + 16 * wave + li) * DK + kq * 8;
        Frag fr;
#pragma unroll
        for (int s = 0; s < KS; ++s) fr.b[s] = *reinterpret_cast<const bf16x8_t *>(src + s * 32);
        return fr;
    };
    // acc[rt][r]: score of token rt*16 + 4 kq + r at chunk column 16 wave + li
    struct Scores {
        floatx4_t v[RT];
    };
    auto multiply = [&](const Queries &qs, const Frag &fr) {
        Scores sc;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            sc.v[rt] = floatx4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < KS; ++s)
                sc.v[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qs.a[rt][s], fr.b[s], sc.v[rt], 0, 0, 0);
        }
        return sc;
    };

    uint32_t tl[K];                 // pass 1: running top K of the token's group maxima (lanes lr, g)
    list_clear<K>(tl);
    bool first_group = true;
    float tau[RT][4];               // pass 2: thresholds of the lane's 16 tokens

    {
        Frag nxt = load(0);
        Queries qs;
        if constexpr (STAGE_Q) qs = stage_queries();
        else qs = load_queries();
        for (int step = 0; step < steps; ++step) {
            const bool pass2 = step >= 2 * m;
            const int f = (step / m) & 1, c = step % m, c0 = c * CW;
            const Frag cur = nxt;
            if (step + 1 < steps) nxt = load(step + 1);
            const Scores sc = multiply(qs, cur);
            if (!pass2) {
                // group maxima over the 4 lanes li = 4a .. 4a+3 (columns 16 wave + 4a ..), as
                // float_order keys; lane li & 3 ends with (and stores) token row r = li & 3's
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    int v[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) v[r] = float_order(sc.v[rt][r]);
                    s_mx[rt * 16 + 4 * kq + (li & 3)][(c & 3) * 16 + wave * 4 + (li >> 2)] =
                        (uint32_t)quad_max_scatter(v, li & 3);
                }
                if ((c & 3) == 3 || c == m - 1) {
                    __syncthreads();          // the window's maxima are in LDS
                    const int valid = ((c & 3) + 1) * 16;
                    // signed float_order keys biased to unsigned (0 stays below every key)
                    uint32_t x[K];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int gi = 16 * j + 4 * g + e;
                            x[4 * j + e] = gi < valid ? (s_mx[lr][gi] ^ 0x80000000u) | 1u : 0u;
                        }
                    }
                    if (first_group) list_first<K>(tl, x);
                    else list_absorb<K>(tl, x);
                    first_group = false;
                    if (c == m - 1) {
                        group_merge<K, G>(tl);
                        uint32_t t = 0;
#pragma unroll
                        for (int w = 0; w < K; ++w)
                            if (w == kk - 1) t = tl[w];
                        // the keys carry their low bit set (none is the 0 sentinel); clearing it
                        // gives at most the kk-th largest group maximum.  t == 0 (fewer than kk
                        // groups): tau = NaN keeps every score
                        const float tv = t == 0 ? __int_as_float(0x7FC00000)
                                                : float_of_order((int)((t & ~1u) ^ 0x80000000u));
                        if (g == 0) s_tau[f][lr] = tv;
                        list_clear<K>(tl);
                        first_group = true;
                    }
                    __syncthreads();          // region A is rewritten by the next window; tau published
                }
            } else {
                if (c == 0) {
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt) {
                        const float4 t4 = *reinterpret_cast<const float4 *>(&s_tau[f][rt * 16 + 4 * kq]);
                        tau[rt][0] = t4.x; tau[rt][1] = t4.y; tau[rt][2] = t4.z; tau[rt][3] = t4.w;
                    }
                }
                auto sv = reinterpret_cast<uint32_t (*)[SV][2]>(s_b[f]);
                const uint32_t col = (uint32_t)(c0 + 16 * wave + li);
                // every survivor's slot first (the counter increments are issued back to
                // back), then the stores
                uint32_t pos[RT][4];
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        pos[rt][r] = SV;
                        if (!(sc.v[rt][r] < tau[rt][r]))         // NaN scores are kept
                            pos[rt][r] = atomicAdd(&s_cnt[f][rt * 16 + 4 * kq + r], 1u);
                    }
                }
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        if (pos[rt][r] < (uint32_t)SV) {
                            const int t = rt * 16 + 4 * kq + r;
                            *reinterpret_cast<uint2 *>(&sv[t][pos[rt][r]][0]) =
                                make_uint2(__float_as_uint(sc.v[rt][r]), col);
                        }
                    }
                }
            }
        }
    }
    __syncthreads();                          // every survivor is in LDS

    // each factor's exact top K from its survivors, or unfiltered when some token's overflowed
    bool finite = true;
#pragma unroll 1
    for (int f = 0; f < 2; ++f) {
        const uint32_t cnt = s_cnt[f][lr];
        double t[K];
        if (!__syncthreads_or(cnt > (uint32_t)SV)) {
            auto sv = reinterpret_cast<uint32_t (*)[SV][2]>(s_b[f]);
            double x[8];
#pragma unroll
            for (int qi = 0; qi < 8; ++qi) {
                const uint32_t i = (uint32_t)(qi * G + g);
                x[qi] = i < cnt ? rank_keyd(__uint_as_float(sv[lr][i][0]), sv[lr][i][1], TIE) : 0.0;
            }
            bitonic_sort<8, true>(x);
#pragma unroll
            for (int w = 0; w < K; ++w) t[w] = w < 8 ? x[w] : 0.0;
            group_merge<K, G>(t);
        } else {
            // every score of this factor keyed, sorted and merged, chunk by chunk through LDS
            auto fb = reinterpret_cast<float (*)[CW]>(s_b[f]);
            const Queries qs = load_queries();
#pragma unroll 1
            for (int cc = 0; cc < m; ++cc) {
                const Scores sc = multiply(qs, load(f * m + cc));
                __syncthreads();                         // the previous chunk's scores are consumed
#pragma unroll
                for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                    for (int r = 0; r < 4; ++r) fb[rt * 16 + 4 * kq + r][16 * wave + li] = sc.v[rt][r];
                __syncthreads();
                double a[K];
#pragma unroll
                for (int e = 0; e < K; ++e)
                    a[e] = rank_keyd(fb[lr][16 * g + e], (uint32_t)(cc * CW + 16 * g + e), TIE);
                if (cc == 0) list_first<K>(t, a);
                else list_absorb<K>(t, a);
            }
            group_merge<K, G>(t);
        }
        finite = stash_factor<K, G>(t, kk, TIE, g, s_idx[lr][f], s_val[lr][f]) && finite;
    }
    const int64_t out_row = (live ? row_n : 0) * H + h;
    const KeyRow kr = ka.addr ? key_row(ka, out_row, H, width) : KeyRow{nullptr, nullptr, 0, 0, 0};
    __syncthreads();                          // the stashed lists are read across lanes of the token
    if (width == K && half <= 32768)
        route_tail16(s_idx[lr][0], s_val[lr][0], s_idx[lr][1], s_val[lr][1], half, TIE, g, s_pairs, finite, live,
                     index + out_row * width, weights + out_row * width, kr);
    else
        route_tail<K, G>(s_idx[lr][0], s_val[lr][0], s_idx[lr][1], s_val[lr][1], half, width, TIE, g, s_pairs,
                         npairs, finite, live, index + out_row * width, weights + out_row * width, kr);
}

template <int DK>
static int launch_score_route16(const void *q, const void *keys, int64_t N, int64_t H, int half, int width, int tie,
                                int64_t *index, float *weights, const KeyArgs &ka, hipStream_t st)
{
    const int64_t blocks = ceil_div(N, F16_R) * H;
    if (blocks > 0x7FFFFFFF) return fail(GLSDM_ERR_UNSUPPORTED, "score_route: grid too large");
    const bf16_t *qq = static_cast<const bf16_t *>(q), *kk = static_cast<const bf16_t *>(keys);
    if (tie == GLSDM_TIE_HIGHEST)
        hipLaunchKernelGGL((score_route16_kernel<DK, GLSDM_TIE_HIGHEST>), dim3((unsigned)blocks), dim3(256), 0, st,
                           qq, kk, N, H, half, width, index, weights, ka);
    else
        hipLaunchKernelGGL((score_route16_kernel<DK, GLSDM_TIE_LOWEST>), dim3((unsigned)blocks), dim3(256), 0, st,
                           qq, kk, N, H, half, width, index, weights, ka);
    return check_launch("score_route16_kernel");
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
    if (!scores_out && pow2_ceil(width) == 16 && half % F16_CW == 0 && (dk == 64 || dk == 128 || dk == 256)) {
        if (dk == 64) return launch_score_route16<64>(queries, subkeys, N, H, half, width, tie, index, weights, ka, st);
        if (dk == 128) return launch_score_route16<128>(queries, subkeys, N, H, half, width, tie, index, weights, ka, st);
        return launch_score_route16<256>(queries, subkeys, N, H, half, width, tie, index, weights, ka, st);
    }
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
