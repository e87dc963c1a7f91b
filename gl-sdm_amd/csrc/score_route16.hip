// Fused address scoring + product-key routing for routes of 9 to 16 picks on
// gfx950: the filtered kernel (one launch per route call).  Semantics as
// glsdm_score_route: the chosen slots, weights and tie rule are identical on
// identical scores to glsdm_route's.
#include "select.h"

namespace glsdm {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float floatx4_t;

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
constexpr int RES_CHUNKS = 4;  // resident-score variant: chunks of a factor held in registers

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

template <int DK, int TIE, bool RES>
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

    if constexpr (RES) {
        // Resident scores (half <= RES_CHUNKS * CW): a factor's scores stay in registers
        // from the multiply to the filter, so they are computed once.  Per factor: the
        // chunks' MFMA scores and group maxima, one barrier, tau from the maxima, one
        // barrier, then the filter of the held scores against tau.
        Frag nxt = load(0);
        // The block's query rows live in factor 1's survivor buffer until factor 1's
        // last multiply (its filter writes the buffer only after the barrier that follows
        // every multiply), unpadded: 16-byte piece p of row r is stored at piece p ^ (r & SWZ)
        // so a fragment read (16 rows, one piece each) spreads over the banks.
        constexpr int PER_ROW = DK / 8, SWZ = (PER_ROW < 16 ? PER_ROW : 16) - 1;
        static_assert(R * DK * 2 <= (int)sizeof(s_b[1]), "query rows fit factor 1's buffer");
        uint4 *s_q = reinterpret_cast<uint4 *>(s_b[1]);
        {
            constexpr int PIECES = R * PER_ROW / 256;
            static_assert(PIECES * 256 == R * PER_ROW, "query staging");
#pragma unroll
            for (int p = 0; p < PIECES; ++p) {
                const int id = tid + 256 * p, row = id / PER_ROW, sl = id % PER_ROW;
                int64_t qn = n0 + row;
                if (qn >= N) qn = N - 1;
                s_q[row * PER_ROW + (sl ^ (row & SWZ))] =
                    *reinterpret_cast<const uint4 *>(q + (qn * H + h) * DK + sl * 8);
            }
        }
        __syncthreads();                          // the query rows are in LDS
        // the A fragments come from LDS at every multiply, so no query registers are held
        auto multiply_s = [&](const Frag &fr) {
            Scores sc;
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                sc.v[rt] = floatx4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s = 0; s < KS; ++s)
                    sc.v[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        *reinterpret_cast<const bf16x8_t *>(&s_q[(rt * 16 + li) * PER_ROW + ((kq + 4 * s) ^ (li & SWZ))]),
                        fr.b[s], sc.v[rt], 0, 0, 0);
            }
            return sc;
        };
#pragma unroll 1
        for (int f = 0; f < 2; ++f) {
            Scores held[RES_CHUNKS];
#pragma unroll
            for (int c = 0; c < RES_CHUNKS; ++c) {
                if (c < m) {                      // block-uniform
                    const Frag cur = nxt;
                    if (c + 1 < m) nxt = load(f * m + c + 1);
                    else if (f == 0) nxt = load(m);           // factor 1's first chunk
                    held[c] = multiply_s(cur);
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt) {
                        int v[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) v[r] = float_order(held[c].v[rt][r]);
                        s_mx[rt * 16 + 4 * kq + (li & 3)][c * 16 + wave * 4 + (li >> 2)] =
                            (uint32_t)quad_max_scatter(v, li & 3);
                    }
                }
            }
            __syncthreads();                      // the factor's group maxima are in LDS
            {
                const int valid = m * 16;
                uint32_t x[K];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int gi = 16 * j + 4 * g + e;
                        x[4 * j + e] = gi < valid ? (s_mx[lr][gi] ^ 0x80000000u) | 1u : 0u;
                    }
                }
                list_first<K>(tl, x);
                group_merge<K, G>(tl);
                uint32_t t = 0;
#pragma unroll
                for (int w = 0; w < K; ++w)
                    if (w == kk - 1) t = tl[w];
                const float tv = t == 0 ? __int_as_float(0x7FC00000)
                                        : float_of_order((int)((t & ~1u) ^ 0x80000000u));
                if (g == 0) s_tau[f][lr] = tv;
            }
            __syncthreads();                      // tau published; s_mx is free for the next factor
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const float4 t4 = *reinterpret_cast<const float4 *>(&s_tau[f][rt * 16 + 4 * kq]);
                tau[rt][0] = t4.x; tau[rt][1] = t4.y; tau[rt][2] = t4.z; tau[rt][3] = t4.w;
            }
            auto sv = reinterpret_cast<uint32_t (*)[SV][2]>(s_b[f]);
#pragma unroll
            for (int c = 0; c < RES_CHUNKS; ++c) {
                if (c < m) {
                    const uint32_t col = (uint32_t)(c * CW + 16 * wave + li);
                    uint32_t pos[RT][4];
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            pos[rt][r] = SV;
                            if (!(held[c].v[rt][r] < tau[rt][r]))     // NaN scores are kept
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
                                    make_uint2(__float_as_uint(held[c].v[rt][r]), col);
                            }
                        }
                    }
                }
            }
        }
    } else {
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
    // half <= RES_CHUNKS * F16_CW: every score of a factor is held in registers (one MFMA pass)
    constexpr bool RES_OK = DK <= 128;            // the query rows fit one survivor buffer
    const bool res = RES_OK && half <= RES_CHUNKS * F16_CW;
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3((unsigned)blocks), dim3(256), 0, st, qq, kk, N, H, half, width, index, weights,
                           ka);
    };
    if (tie == GLSDM_TIE_HIGHEST) {
        if (res) go(score_route16_kernel<DK, GLSDM_TIE_HIGHEST, RES_OK>);
        else go(score_route16_kernel<DK, GLSDM_TIE_HIGHEST, false>);
    } else {
        if (res) go(score_route16_kernel<DK, GLSDM_TIE_LOWEST, RES_OK>);
        else go(score_route16_kernel<DK, GLSDM_TIE_LOWEST, false>);
    }
    return check_launch("score_route16_kernel");
}

// Whether the filtered kernel takes a route call of this shape: lists of 16
// (9 to 16 picks), dk in {64, 128, 256}, half a multiple of its chunk width.
bool score_route16_takes(int dk, int half, int width)
{
    return pow2_ceil(width) == 16 && half % F16_CW == 0 && (dk == 64 || dk == 128 || dk == 256);
}

// The filtered kernel's launch for one route call of a shape it takes.
int score_route16_launch(const void *q, const void *keys, int64_t N, int64_t H, int dk, int half, int width,
                         int tie, int64_t *index, float *weights, const KeyArgs &ka, hipStream_t st)
{
    if (dk == 64) return launch_score_route16<64>(q, keys, N, H, half, width, tie, index, weights, ka, st);
    if (dk == 128) return launch_score_route16<128>(q, keys, N, H, half, width, tie, index, weights, ka, st);
    return launch_score_route16<256>(q, keys, N, H, half, width, tie, index, weights, ka, st);
}

}  // namespace glsdm
