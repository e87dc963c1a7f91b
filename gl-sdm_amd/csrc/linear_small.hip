// The stack's bf16 projections for decode-sized inputs (at most 64 rows) on gfx950.
//
// Semantics: torch.nn.functional.linear in bf16 (S/layers/*.py: every nn.Linear
// of the stack), out[m, n] = bf16(sum_k x[m, k] * w[n, k] + bias[n]): bf16
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

__global__ __launch_bounds__(256) void linear_small_kernel(const bf16_t *__restrict__ x, const bf16_t *__restrict__ w,
                                                           const bf16_t *__restrict__ bias, bf16_t *__restrict__ out,
                                                           int M, int N, int K)
{
#pragma clang fp contract(off)
    __shared__ float s_part[4][LS_MAX_ROWS][17];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int li = lane & 15, kq = lane >> 4;
    const int n0 = blockIdx.x * 16;
    const int kw = K / 4;                     // this wave's K range [wave * kw, wave * kw + kw)
    const int RT = (M + 15) / 16;             // row tiles (block-uniform)
    const bf16_t *wrow = w + (int64_t)(n0 + li) * K + wave * kw + kq * 8;
    floatx4_t acc[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) acc[rt] = floatx4_t{0.f, 0.f, 0.f, 0.f};
    // row li of tile rt; rows past M read row M - 1 and are never stored
    const bf16_t *xrow[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
        const int m = rt * 16 + li < M ? rt * 16 + li : M - 1;
        xrow[rt] = x + (int64_t)m * K + wave * kw + kq * 8;
    }
    for (int k0 = 0; k0 < kw; k0 += 32) {
        const bf16x8_t b = *reinterpret_cast<const bf16x8_t *>(wrow + k0);
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
            if (rt < RT) {
                const bf16x8_t a = *reinterpret_cast<const bf16x8_t *>(xrow[rt] + k0);
                acc[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[rt], 0, 0, 0);
            }
        }
    }
    // acc[rt][i]: row rt*16 + 4*kq + i, column n0 + li
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
        if (rt < RT)
#pragma unroll
            for (int i = 0; i < 4; ++i) s_part[wave][rt * 16 + 4 * kq + i][li] = acc[rt][i];
    __syncthreads();
    for (int e = threadIdx.x; e < RT * 16 * 16; e += 256) {
        const int m = e >> 4, c = e & 15;
        if (m < M) {
            float s = s_part[0][m][c] + s_part[1][m][c];
            s = s + s_part[2][m][c];
            s = s + s_part[3][m][c];
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
    hipLaunchKernelGGL(linear_small_kernel, dim3((unsigned)(N / 16)), dim3(256), 0, as_stream(stream),
                       static_cast<const bf16_t *>(x), static_cast<const bf16_t *>(weight),
                       static_cast<const bf16_t *>(bias), static_cast<bf16_t *>(out), (int)M, (int)N, (int)K);
    return check_launch("linear_small_kernel");
}
