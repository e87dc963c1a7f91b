// QK normalisation and rotary positions of the stack's local attention, fused.
//
// Semantics (S/ = projects/gl-sdm/src/gl_sdm/): S/layers/attention.py:38-42
// and :51-52.  Per head row x of dk elements (the query half of the
// [query | gate] projection, or a key row):
//   y = x * rsqrt(mean(x^2) + eps), rounded to the row dtype  (F.rms_norm
//       without weight; eps = the fp32 machine epsilon, its default)
//   with a = y[:dk/2], b = y[dk/2:] in fp32 and theta_j = (offset + t) * freq[j]:
//   out = cat(a cos(theta) + b sin(theta), -a sin(theta) + b cos(theta)),
//       rounded to the row dtype,
// every product and sum a separate fp32 operation in that order.  One
// wavefront per row; rows are read through a row stride (the query half is a
// strided view) and written [B, heads, T, dk] contiguous, the layout
// attention and the KV cache take, so the transposes disappear as well.
#include "glsdm_internal.h"

namespace glsdm {

template <typename TX> struct RowIO;
template <> struct RowIO<float> {
    __device__ __forceinline__ static float load(const float *p) { return *p; }
    __device__ __forceinline__ static float round(float v) { return v; }
    __device__ __forceinline__ static void store(float *p, float v) { *p = v; }
};
template <> struct RowIO<bf16_t> {
    __device__ __forceinline__ static float load(const bf16_t *p) { return bf16_to_f32(*p); }
    __device__ __forceinline__ static float round(float v) { return bf16_to_f32(f32_to_bf16(v)); }
    __device__ __forceinline__ static void store(bf16_t *p, float v) { *p = f32_to_bf16(v); }
};

constexpr int QK_MAX_PAIRS = 2;          // dk <= 256: each lane takes up to two (a, b) pairs

template <typename TX>
__global__ __launch_bounds__(256) void qk_norm_rotary_kernel(const TX *__restrict__ x, int64_t row_stride,
                                                             int64_t rows, int64_t T, int64_t heads, int dk,
                                                             const float *__restrict__ freq, int64_t offset,
                                                             TX *__restrict__ out)
{
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int64_t r = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (r >= rows) return;                                  // wave-uniform
    const int half = dk >> 1;
    const TX *src = x + r * row_stride;
    float a[QK_MAX_PAIRS], b[QK_MAX_PAIRS];
    float ss = 0.0f;
#pragma unroll
    for (int p = 0; p < QK_MAX_PAIRS; ++p) {
        const int j = lane + 64 * p;
        a[p] = j < half ? RowIO<TX>::load(src + j) : 0.0f;
        b[p] = j < half ? RowIO<TX>::load(src + half + j) : 0.0f;
        ss += a[p] * a[p];
        ss += b[p] * b[p];
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
    const float scale = rsqrtf(ss / (float)dk + __FLT_EPSILON__);
    // row r = (bt * heads + h) with bt = batch * T + t
    const int64_t h = r % heads, bt = r / heads;
    const int64_t t = bt % T, batch = bt / T;
    TX *dst = out + ((batch * heads + h) * T + t) * dk;
    const float pos = (float)(offset + t);
#pragma unroll
    for (int p = 0; p < QK_MAX_PAIRS; ++p) {
        const int j = lane + 64 * p;
        if (j >= half) continue;
        const float ya = RowIO<TX>::round(a[p] * scale), yb = RowIO<TX>::round(b[p] * scale);
        const float theta = pos * freq[j];
        const float c = cosf(theta), s = sinf(theta);
        const float ac = ya * c, bs = yb * s;
        const float na = -ya;
        const float as = na * s, bc = yb * c;
        RowIO<TX>::store(dst + j, ac + bs);
        RowIO<TX>::store(dst + half + j, as + bc);
    }
}

}  // namespace glsdm

using namespace glsdm;

extern "C" int glsdm_qk_norm_rotary(const void *x, int32_t dtype, int64_t B, int64_t T, int64_t heads, int64_t dk,
                                    int64_t row_stride, const float *freq, int64_t offset, void *out, void *stream)
{
    if (B < 0 || T < 0 || heads < 1 || dk < 4 || dk % 4 != 0 || dk > 64 * 2 * QK_MAX_PAIRS || row_stride < dk ||
        offset < 0)
        return fail(GLSDM_ERR_ARG, "qk_norm_rotary: bad shape B=%lld T=%lld heads=%lld dk=%lld stride=%lld",
                    (long long)B, (long long)T, (long long)heads, (long long)dk, (long long)row_stride);
    if (!dtype_ok(dtype)) return fail(GLSDM_ERR_ARG, "qk_norm_rotary: bad dtype");
    if (offset + T > (int64_t)1 << 24)
        return fail(GLSDM_ERR_UNSUPPORTED, "qk_norm_rotary: positions above 2^24 are not exact in fp32");
    const int64_t rows = B * T * heads;
    if (rows == 0) return GLSDM_OK;
    if (!x || !freq || !out) return fail(GLSDM_ERR_ARG, "qk_norm_rotary: null pointer");
    const hipStream_t st = as_stream(stream);
    const dim3 grid((unsigned)ceil_div(rows, 4)), block(256);
    if (dtype == GLSDM_F32)
        hipLaunchKernelGGL(qk_norm_rotary_kernel<float>, grid, block, 0, st, static_cast<const float *>(x), row_stride,
                           rows, T, heads, (int)dk, freq, offset, static_cast<float *>(out));
    else
        hipLaunchKernelGGL(qk_norm_rotary_kernel<bf16_t>, grid, block, 0, st, static_cast<const bf16_t *>(x),
                           row_stride, rows, T, heads, (int)dk, freq, offset, static_cast<bf16_t *>(out));
    return check_launch("qk_norm_rotary_kernel");
}
