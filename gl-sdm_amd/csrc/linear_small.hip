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
#include "glsdm_internal.h"

namespace glsdm {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float floatx4_t;

constexpr int LS_MAX_ROWS = 64;

// CT column tiles of 16 per block: each wave multiplies its x fragments into CT
// weight tiles, so wide projections (2^15 columns) read x from L2 CT times less.
// W waves split K (16 for deep reductions: each wave's chain of dependent k-steps
// stays at 8 for K = 4096).
template <int CT, int W>
__global__ __launch_bounds__(64 * W) void linear_small_kernel(const bf16_t *__restrict__ x, const bf16_t *__restrict__ w,
                                                           const bf16_t *__restrict__ bias, bf16_t *__restrict__ out,
                                                           int M, int N, int K)
{
#pragma clang fp contract(off)
    __shared__ float s_part[W][LS_MAX_ROWS][16 * CT + 1];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int li = lane & 15, kq = lane >> 4;
    const int n0 = blockIdx.x * 16 * CT;
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
    const bf16_t *xrow[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
        const int m = rt * 16 + li < M ? rt * 16 + li : M - 1;
        xrow[rt] = x + (int64_t)m * K + wave * kw + kq * 8;
    }
    for (int k0 = 0; k0 < kw; k0 += 32) {
        bf16x8_t b[CT];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) b[ct] = *reinterpret_cast<const bf16x8_t *>(wrow[ct] + k0);
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
            if (rt < RT) {
                const bf16x8_t a = *reinterpret_cast<const bf16x8_t *>(xrow[rt] + k0);
#pragma unroll
                for (int ct = 0; ct < CT; ++ct)
                    acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[ct], acc[rt][ct], 0, 0, 0);
            }
        }
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
            out[(int64_t)m * N + n0 + c] = f32_to_bf16(s);
        }
    }
}

}  // namespace glsdm

using namespace glsdm;

extern "C" int glsdm_linear_small(const void *x, const void *weight, const void *bias, void *out, int64_t M,
                                  int64_t N, int64_t K, void *stream)
{
    if (M < 1 || N < 1 || K < 1) return fail(GLSDM_ERR_ARG, "linear_small: bad shape");
    if (M > LS_MAX_ROWS || N % 16 != 0 || K % 128 != 0 || N > (int64_t)16 * 0x7FFFFFFF || K > 0x7FFFFFFF)
        return fail(GLSDM_ERR_UNSUPPORTED, "linear_small: M <= 64, N a multiple of 16 and K of 128 required");
    if (!x || !weight || !out) return fail(GLSDM_ERR_ARG, "linear_small: null pointer");
    if (((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(weight)) & 15) != 0)
        return fail(GLSDM_ERR_UNSUPPORTED, "linear_small: x and weight must be 16-byte aligned");
    const bf16_t *xx = static_cast<const bf16_t *>(x), *ww = static_cast<const bf16_t *>(weight);
    const bf16_t *bb = static_cast<const bf16_t *>(bias);
    bf16_t *oo = static_cast<bf16_t *>(out);
    // four column tiles per block for wide projections (still >= 256 blocks), one otherwise;
    // sixteen waves over K for deep reductions
    hipStream_t st = as_stream(stream);
    if (N % 64 == 0 && N >= 16384)
        hipLaunchKernelGGL((linear_small_kernel<4, 4>), dim3((unsigned)(N / 64)), dim3(256), 0, st, xx, ww, bb, oo,
                           (int)M, (int)N, (int)K);
    else if (K >= 4096 && K % (16 * 32) == 0)
        hipLaunchKernelGGL((linear_small_kernel<1, 16>), dim3((unsigned)(N / 16)), dim3(1024), 0, st, xx, ww, bb, oo,
                           (int)M, (int)N, (int)K);
    else
        hipLaunchKernelGGL((linear_small_kernel<1, 4>), dim3((unsigned)(N / 16)), dim3(256), 0, st, xx, ww, bb, oo,
                           (int)M, (int)N, (int)K);
    return check_launch("linear_small_kernel");
}
