// Address scoring on bf16 MFMA (gfx950 v_mfma_f32_16x16x32_bf16).
//
// scores[(n*H + h), c] = sum_e q[(n*H + h), e] * K[h, c, e], fp32 accumulation,
// n over the B*T tokens, c over the L = 2*half sub-keys of head h.  This is the
// per-head sub-key form of the factor-score projection that feeds routing
// (S/layers/global_layer.py:26,42 with weights S/layers/router.py:23-24).
//
// Tiling: a 256-thread block owns 64 tokens x 64 sub-keys of one head; each
// wavefront computes 16 tokens x 64 sub-keys as four 16x16 MFMA tiles, dk/32
// k-steps each.  Operands are loaded straight from HBM/L2 as 16-byte bf16x8
// fragments (dk = 128 makes a token's query row 256 B); the sub-key fragments
// are shared by the block's four waves through L1.
#include "glsdm_internal.h"

namespace glsdm {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float floatx4_t;

__global__ __launch_bounds__(256) void score_kernel(const bf16_t *__restrict__ q,
                                                    const bf16_t *__restrict__ keys, int64_t N,
                                                    int64_t H, int dk, int L, float *__restrict__ scores)
{
    const int h = blockIdx.z;
    const int lane = threadIdx.x & 63;
    const int i = lane & 15, kq = lane >> 4;
    const int64_t n0 = (int64_t)blockIdx.x * 64 + (threadIdx.x >> 6) * 16;
    const int c0 = blockIdx.y * 64;
    int64_t n = n0 + i;
    if (n >= N) n = N - 1;   // clamp loads; stores below are masked
    const bf16_t *qrow = q + (n * H + h) * dk + kq * 8;
    const bf16_t *krow = keys + ((int64_t)h * L + c0 + i) * dk + kq * 8;

    floatx4_t acc[4];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) acc[ct] = floatx4_t{0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < dk; k0 += 32) {
        const bf16x8_t a = *reinterpret_cast<const bf16x8_t *>(qrow + k0);
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
            const bf16x8_t b = *reinterpret_cast<const bf16x8_t *>(krow + (int64_t)ct * 16 * dk + k0);
            acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[ct], 0, 0, 0);
        }
    }
    // accumulator layout: lane holds rows 4*kq + r (r < 4) of column i
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t nn = n0 + 4 * kq + r;
            if (nn < N) scores[(nn * H + h) * L + c0 + ct * 16 + i] = acc[ct][r];
        }
    }
}

}  // namespace glsdm

using namespace glsdm;

extern "C" int glsdm_score(const void *queries, const void *subkeys, int64_t B, int64_t T, int64_t H,
                           int32_t dk, int32_t half, float *scores, void *stream)
{
    if (B < 0 || T < 0 || H < 1 || dk < 1 || half < 1) return fail(GLSDM_ERR_ARG, "score: bad shape");
    const int L = 2 * half;
    if (dk % 32 != 0) return fail(GLSDM_ERR_UNSUPPORTED, "score: dk=%d is not a multiple of 32", dk);
    if (L % 64 != 0) return fail(GLSDM_ERR_UNSUPPORTED, "score: 2*half=%d is not a multiple of 64", L);
    if (H > 65535) return fail(GLSDM_ERR_UNSUPPORTED, "score: too many heads");
    const int64_t N = B * T;
    if (N == 0) return GLSDM_OK;
    if (!queries || !subkeys || !scores) return fail(GLSDM_ERR_ARG, "score: null pointer");
    if (((reinterpret_cast<uintptr_t>(queries) | reinterpret_cast<uintptr_t>(subkeys)) & 15) != 0)
        return fail(GLSDM_ERR_UNSUPPORTED, "score: queries and sub-keys must be 16-byte aligned");
    if (ceil_div(N, 64) > 0x7FFFFFFF || L / 64 > 65535) return fail(GLSDM_ERR_UNSUPPORTED, "score: grid too large");
    const dim3 grid((unsigned)ceil_div(N, 64), (unsigned)(L / 64), (unsigned)H);
    hipLaunchKernelGGL(score_kernel, grid, dim3(256), 0, as_stream(stream),
                       static_cast<const bf16_t *>(queries), static_cast<const bf16_t *>(subkeys), N, H,
                       dk, L, scores);
    return check_launch("score_kernel");
}
