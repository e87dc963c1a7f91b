// The stack's bf16 projections for decode-sized inputs (at most 64 rows) on gfx950.
//
// Semantics: torch.nn.functional.linear in bf16 (every nn.Linear of the stack:
// S/layers/attention.py:23-26, S/layers/common.py:22-23, S/layers/router.py:23-28,
// S/model.py:45), out[m, n] = bf16(sum_k x[m, k] * w[n, k] + bias[n]): bf16
// products accumulated in fp32 and rounded once, round-to-nearest-even.  The
// fp32 summation order is this kernel's (the library GEMM's order is its own),
// so results agree with torch's to the rounding of the fp32 sum.
//
// Why: a decode step of the config-5 stack makes over a hundred of these
// projections of 64 rows each, and the library GEMM spends ~20 us of host time
// per call against ~5 us for a launch through this library, so the step is
// bound by the host.  The work itself is small: one block per 16 output columns,
// its four waves split K in four and each runs v_mfma_f32_16x16x32_bf16 over
// up to four 16-row tiles (fragments loaded straight from L2/HBM: x is shared by
// every block, each weight row is read once), then the four partial tiles are
// summed in a fixed order through LDS and the bias is added before the rounding.
// Projections of one input (a layer's q, k and v) can share one launch: the grid
// is their column tiles side by side, each block picks its projection by index.
#include "glsdm_internal.h"

namespace glsdm {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float floatx4_t;

constexpr int LS_MAX_ROWS = 64;

// gate * bf16(relu(u)^2) rounded to bf16, for 8 bf16 pairs packed in 16 bytes
__device__ __forceinline__ bf16x8_t relu2_gate8(uint4 u, uint4 g)
{
#pragma clang fp contract(off)
    const uint32_t uw[4] = {u.x, u.y, u.z, u.w}, gw[4] = {g.x, g.y, g.z, g.w};
    uint32_t ow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t pair = 0;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const float uf = bf16_to_f32((bf16_t)(uw[i] >> (16 * e))), gf = bf16_to_f32((bf16_t)(gw[i] >> (16 * e)));
            const float relu = (uf > 0.0f || uf != uf) ? uf : 0.0f;   // relu keeps NaN
            const float sq = bf16_to_f32(f32_to_bf16(relu * relu));
            pair |= (uint32_t)f32_to_bf16(gf * sq) << (16 * e);
        }
        ow[i] = pair;
    }
    const uint4 o = {ow[0], ow[1], ow[2], ow[3]};
    return __builtin_bit_cast(bf16x8_t, o);
}
constexpr int LS_MAX_GROUP = 8;

// the projections of one launch (passed by value): projection i owns blocks
// [first[i], first[i + 1]) and writes out[i] [M, N[i]]
struct LinearGroup {
    const bf16_t *w[LS_MAX_GROUP];
    const bf16_t *bias[LS_MAX_GROUP];
    bf16_t *out[LS_MAX_GROUP];
    int N[LS_MAX_GROUP];
    int first[LS_MAX_GROUP + 1];
    int count;
    // residual form (one projection): res_out = residual + float(bf16 result)
    const float *residual;
    float *res_out;
};

// CT column tiles of 16 per block: each wave multiplies its x fragments into CT
// weight tiles, so wide projections (2^15 columns) read x from L2 CT times less.
// W waves split K (16 for deep reductions: each wave's chain of dependent k-steps
// stays at 8 for K = 4096).  RES: the residual form, whose rounded bf16 result is
// added in fp32 to an fp32 residual (torch's x + y for fp32 x and bf16 y).
// RELU2: x is the MLP's fc output h [M, 2K] and the operand is formed on load,
// a = bf16(gate * bf16(relu(u)^2)) for u = h[:, :K], gate = h[:, K:] (relu keeps
// NaN), the roundings of the separate activation launch.
template <int CT, int W, bool RES, bool RELU2>
__global__ __launch_bounds__(64 * W) void linear_small_kernel(const bf16_t *__restrict__ x, const LinearGroup g, int M,
                                                           int K)
{
#pragma clang fp contract(off)
    __shared__ float s_part[W][LS_MAX_ROWS][16 * CT + 1];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int li = lane & 15, kq = lane >> 4;
    // this block's projection, chosen with constant indices only (a runtime index
    // into the argument struct would copy it to scratch memory)
    const bf16_t *__restrict__ w = g.w[0];
    const bf16_t *__restrict__ bias = g.bias[0];
    bf16_t *__restrict__ out = g.out[0];
    int N = g.N[0], base = 0;
#pragma unroll
    for (int i = 1; i < LS_MAX_GROUP; ++i)
        if (i < g.count && (int)blockIdx.x >= g.first[i]) {
            w = g.w[i];
            bias = g.bias[i];
            out = g.out[i];
            N = g.N[i];
            base = g.first[i];
        }
    const int n0 = ((int)blockIdx.x - base) * 16 * CT;
    const int kw = K / W;                     // this wave's K range [wave * kw, wave * kw + kw)
    const int RT = (M + 15) / 16;             // row tiles (block-uniform)
    const bf16_t *wrow[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) wrow[ct] = w + (int64_t)(n0 + 16 * ct + li) * K + wave * kw + kq * 8;
    floatx4_t acc[4][CT];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) acc[rt][ct] = floatx4_t{0.f, 0.f, 0.f, 0.f};
    // row li of tile rt; rows past M read row M - 1 and are never stored
    const int64_t xstride = RELU2 ? 2 * (int64_t)K : K;
    const bf16_t *xrow[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
        const int m = rt * 16 + li < M ? rt * 16 + li : M - 1;
        xrow[rt] = x + (int64_t)m * xstride + wave * kw + kq * 8;
    }
    // Every k-step loads its weight fragments and all four row tiles (rows past M
    // read row M - 1, a valid address, and their results are never stored) with no
    // branch between the loads, and two k-steps are loaded before either's MFMAs,
    // so up to 2 * (CT + 4) loads are in flight before the first wait.  The MFMAs
    // of each (row tile, column tile) still run in k order.
    auto load = [&](int k0, bf16x8_t (&b)[CT], bf16x8_t (&a)[4]) {
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) b[ct] = *reinterpret_cast<const bf16x8_t *>(wrow[ct] + k0);
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
            if constexpr (RELU2) {
                const uint4 u = *reinterpret_cast<const uint4 *>(xrow[rt] + k0);
                const uint4 gt = *reinterpret_cast<const uint4 *>(xrow[rt] + K + k0);
                a[rt] = relu2_gate8(u, gt);
            } else {
                a[rt] = *reinterpret_cast<const bf16x8_t *>(xrow[rt] + k0);
            }
        }
    };
    auto multiply = [&](const bf16x8_t (&b)[CT], const bf16x8_t (&a)[4]) {
#pragma unroll
        for (int rt = 0; rt < 4; ++rt)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct)
                acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[rt], b[ct], acc[rt][ct], 0, 0, 0);
    };
    int k0 = 0;
    for (; k0 + 64 <= kw; k0 += 64) {
        bf16x8_t b0[CT], a0[4], b1[CT], a1[4];
        load(k0, b0, a0);
        load(k0 + 32, b1, a1);
        multiply(b0, a0);
        multiply(b1, a1);
    }
    if (k0 < kw) {
        bf16x8_t b0[CT], a0[4];
        load(k0, b0, a0);
        multiply(b0, a0);
    }
    // acc[rt][ct][i]: row rt*16 + 4*kq + i, column n0 + 16 ct + li
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
        if (rt < RT)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct)
#pragma unroll
                for (int i = 0; i < 4; ++i) s_part[wave][rt * 16 + 4 * kq + i][16 * ct + li] = acc[rt][ct][i];
    __syncthreads();
    // the W partial tiles summed in wave order, then the bias, then one rounding
    for (int e = threadIdx.x; e < RT * 16 * 16 * CT; e += 64 * W) {
        const int m = e / (16 * CT), c = e % (16 * CT);
        if (m < M) {
            float s = s_part[0][m][c];
#pragma unroll
            for (int q = 1; q < W; ++q) s = s + s_part[q][m][c];
            if (bias) s = s + bf16_to_f32(bias[n0 + c]);
            const int64_t o = (int64_t)m * N + n0 + c;
            if constexpr (RES)
                g.res_out[o] = g.residual[o] + bf16_to_f32(f32_to_bf16(s));
            else
                out[o] = f32_to_bf16(s);
        }
    }
}

}  // namespace glsdm

using namespace glsdm;

namespace {

// CT = 4 for wide projections (still >= 256 blocks each), 1 otherwise; W = 16 waves
// over K for deep reductions.  W fixes the summation order; CT does not.
template <bool RES, bool RELU2>
int launch_group(const bf16_t *x, LinearGroup &g, int M, int K, bool wide, hipStream_t st)
{
    const int CT = wide ? 4 : 1;
    g.first[0] = 0;
    for (int i = 0; i < g.count; ++i) g.first[i + 1] = g.first[i] + g.N[i] / (16 * CT);
    for (int i = g.count + 1; i <= LS_MAX_GROUP; ++i) g.first[i] = g.first[g.count];
    const dim3 grid((unsigned)g.first[g.count]);
    if (wide)
        hipLaunchKernelGGL((linear_small_kernel<4, 4, RES, RELU2>), grid, dim3(256), 0, st, x, g, M, K);
    else if (K >= 4096 && K % (16 * 32) == 0)
        hipLaunchKernelGGL((linear_small_kernel<1, 16, RES, RELU2>), grid, dim3(1024), 0, st, x, g, M, K);
    else
        hipLaunchKernelGGL((linear_small_kernel<1, 4, RES, RELU2>), grid, dim3(256), 0, st, x, g, M, K);
    return check_launch("linear_small_kernel");
}

int check_shape(const void *x, int64_t M, int64_t K)
{
    if (M < 1 || K < 1) return fail(GLSDM_ERR_ARG, "linear_small: bad shape");
    if (M > LS_MAX_ROWS || K % 128 != 0 || K > 0x7FFFFFFF)
        return fail(GLSDM_ERR_UNSUPPORTED, "linear_small: M <= 64, N a multiple of 16 and K of 128 required");
    if (!x) return fail(GLSDM_ERR_ARG, "linear_small: null pointer");
    if ((reinterpret_cast<uintptr_t>(x) & 15) != 0)
        return fail(GLSDM_ERR_UNSUPPORTED, "linear_small: x and weight must be 16-byte aligned");
    return GLSDM_OK;
}

int check_projection(const void *weight, const void *out, int64_t N)
{
    if (N < 1) return fail(GLSDM_ERR_ARG, "linear_small: bad shape");
    if (N % 16 != 0 || N > 0x7FFFFFF0)
        return fail(GLSDM_ERR_UNSUPPORTED, "linear_small: M <= 64, N a multiple of 16 and K of 128 required");
    if (!weight || !out) return fail(GLSDM_ERR_ARG, "linear_small: null pointer");
    if ((reinterpret_cast<uintptr_t>(weight) & 15) != 0)
        return fail(GLSDM_ERR_UNSUPPORTED, "linear_small: x and weight must be 16-byte aligned");
    return GLSDM_OK;
}

}  // namespace

extern "C" int glsdm_linear_small(const void *x, const void *weight, const void *bias, void *out, int64_t M,
                                  int64_t N, int64_t K, void *stream)
{
    int rc = check_shape(x, M, K);
    if (rc == GLSDM_OK) rc = check_projection(weight, out, N);
    if (rc != GLSDM_OK) return rc;
    LinearGroup g{};
    g.count = 1;
    g.w[0] = static_cast<const bf16_t *>(weight);
    g.bias[0] = static_cast<const bf16_t *>(bias);
    g.out[0] = static_cast<bf16_t *>(out);
    g.N[0] = (int)N;
    return launch_group<false, false>(static_cast<const bf16_t *>(x), g, (int)M, (int)K, N % 64 == 0 && N >= 16384,
                                      as_stream(stream));
}

extern "C" int glsdm_linear_small_residual(const void *x, const void *weight, const void *bias, const float *residual,
                                           float *out, int64_t M, int64_t N, int64_t K, void *stream)
{
    int rc = check_shape(x, M, K);
    if (rc == GLSDM_OK) rc = check_projection(weight, out, N);
    if (rc != GLSDM_OK) return rc;
    if (!residual) return fail(GLSDM_ERR_ARG, "linear_small_residual: null pointer");
    LinearGroup g{};
    g.count = 1;
    g.w[0] = static_cast<const bf16_t *>(weight);
    g.bias[0] = static_cast<const bf16_t *>(bias);
    g.N[0] = (int)N;
    g.residual = residual;
    g.res_out = out;
    return launch_group<true, false>(static_cast<const bf16_t *>(x), g, (int)M, (int)K, N % 64 == 0 && N >= 16384,
                                     as_stream(stream));
}

extern "C" int glsdm_linear_small_relu2(const void *h, const void *weight, const void *bias, const float *residual,
                                        void *out, int64_t M, int64_t N, int64_t K, void *stream)
{
    int rc = check_shape(h, M, K);
    if (rc == GLSDM_OK) rc = check_projection(weight, out, N);
    if (rc != GLSDM_OK) return rc;
    if (K > 0x3FFFFFFF) return fail(GLSDM_ERR_UNSUPPORTED, "linear_small_relu2: inner width too large");
    LinearGroup g{};
    g.count = 1;
    g.w[0] = static_cast<const bf16_t *>(weight);
    g.bias[0] = static_cast<const bf16_t *>(bias);
    g.N[0] = (int)N;
    const bf16_t *hh = static_cast<const bf16_t *>(h);
    const bool wide = N % 64 == 0 && N >= 16384;
    if (!residual) {
        g.out[0] = static_cast<bf16_t *>(out);
        return launch_group<false, true>(hh, g, (int)M, (int)K, wide, as_stream(stream));
    }
    g.residual = residual;
    g.res_out = static_cast<float *>(out);
    return launch_group<true, true>(hh, g, (int)M, (int)K, wide, as_stream(stream));
}

extern "C" int glsdm_linear_small_group(const void *x, int32_t count, const void *const *weights,
                                        const void *const *biases, void *const *outs, const int64_t *N, int64_t M,
                                        int64_t K, void *stream)
{
    int rc = check_shape(x, M, K);
    if (rc != GLSDM_OK) return rc;
    if (count < 1 || count > LS_MAX_GROUP) return fail(GLSDM_ERR_ARG, "linear_small_group: 1 to 8 projections");
    if (!weights || !outs || !N) return fail(GLSDM_ERR_ARG, "linear_small_group: null pointer");
    LinearGroup g{};
    g.count = count;
    bool wide = true;
    int64_t blocks = 0;
    for (int i = 0; i < count; ++i) {
        if ((rc = check_projection(weights[i], outs[i], N[i])) != GLSDM_OK) return rc;
        g.w[i] = static_cast<const bf16_t *>(weights[i]);
        g.bias[i] = biases ? static_cast<const bf16_t *>(biases[i]) : nullptr;
        g.out[i] = static_cast<bf16_t *>(outs[i]);
        g.N[i] = (int)N[i];
        wide = wide && N[i] % 64 == 0 && N[i] >= 16384;
        blocks += N[i] / 16;
    }
    if (blocks > 0x7FFFFFFF) return fail(GLSDM_ERR_UNSUPPORTED, "linear_small_group: too many columns");
    return launch_group<false, false>(static_cast<const bf16_t *>(x), g, (int)M, (int)K, wide, as_stream(stream));
}
