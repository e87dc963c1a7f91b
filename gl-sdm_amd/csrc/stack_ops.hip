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
// every product and sum a separate fp32 operation in that order.  One block
// per token (b, t): its threads first put cos/sin of the token's dk/2 angles
// in LDS (shared by all heads), then take the heads' rows, dk/4 lanes per row,
// each lane two consecutive (a, b) pairs; the row's sum of squares is reduced
// over its lanes with shuffles.  Rows are read through a row stride (the
// query half is a strided view) and written [B, heads, T, dk] contiguous, the
// layout attention and the KV cache take, so the transposes disappear too.
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

constexpr int QK_THREADS = 256;
constexpr int QK_MAX_DK = 256;

// One row of dk = 4L elements, L lanes (lane li owns elements 2li, 2li+1 of each
// half): RMS norm (eps = FLT_EPSILON, rounded to TX), then the rotation by the
// position's angles in s_cos / s_sin.  The roundings of the reference's
// F.rms_norm + rotary in TX.
template <typename TX, int L>
__device__ __forceinline__ void norm_rotary_row(const TX *__restrict__ src, TX *__restrict__ dst, int li,
                                                const float *s_cos, const float *s_sin)
{
#pragma clang fp contract(off)
    constexpr int dk = 4 * L, half = 2 * L;
    const int j = 2 * li;
    float a0 = RowIO<TX>::load(src + j), a1 = RowIO<TX>::load(src + j + 1);
    float b0 = RowIO<TX>::load(src + half + j), b1 = RowIO<TX>::load(src + half + j + 1);
    float ss = a0 * a0;
    ss += a1 * a1;
    ss += b0 * b0;
    ss += b1 * b1;
#pragma unroll
    for (int off = L / 2; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
    const float scale = rsqrtf(ss / (float)dk + __FLT_EPSILON__);
    a0 = RowIO<TX>::round(a0 * scale);
    a1 = RowIO<TX>::round(a1 * scale);
    b0 = RowIO<TX>::round(b0 * scale);
    b1 = RowIO<TX>::round(b1 * scale);
    const float c0 = s_cos[j], c1 = s_cos[j + 1], s0 = s_sin[j], s1 = s_sin[j + 1];
    const float ac0 = a0 * c0, bs0 = b0 * s0, ac1 = a1 * c1, bs1 = b1 * s1;
    const float as0 = (-a0) * s0, bc0 = b0 * c0, as1 = (-a1) * s1, bc1 = b1 * c1;
    RowIO<TX>::store(dst + j, ac0 + bs0);
    RowIO<TX>::store(dst + j + 1, ac1 + bs1);
    RowIO<TX>::store(dst + half + j, as0 + bc0);
    RowIO<TX>::store(dst + half + j + 1, as1 + bc1);
}

// cos and sin of position offset + t for the first half of the frequencies
__device__ __forceinline__ void rotary_angles(const float *__restrict__ freq, int half, int64_t pos, float *s_cos,
                                              float *s_sin)
{
    const int tid = threadIdx.x;
    if (tid < half) {
        const float theta = (float)pos * freq[tid];
        s_cos[tid] = cosf(theta);
        s_sin[tid] = sinf(theta);
    }
    __syncthreads();
}

template <typename TX, int L>   // L = dk / 4 lanes per row, a power of two <= 64
__global__ __launch_bounds__(QK_THREADS) void qk_norm_rotary_kernel(const TX *__restrict__ x, int64_t row_stride,
                                                                    int64_t T, int64_t heads,
                                                                    const float *__restrict__ freq, int64_t offset,
                                                                    TX *__restrict__ out)
{
    constexpr int dk = 4 * L, rows_per_pass = QK_THREADS / L;
    __shared__ float s_cos[QK_MAX_DK / 2], s_sin[QK_MAX_DK / 2];
    const int64_t bt = blockIdx.x;                          // token b*T + t
    const int64_t t = bt % T, batch = bt / T;
    rotary_angles(freq, 2 * L, offset + t, s_cos, s_sin);
    const int tid = threadIdx.x, li = tid % L;
    for (int64_t h = tid / L; h < heads; h += rows_per_pass)      // uniform within a row's lanes
        norm_rotary_row<TX, L>(x + (bt * heads + h) * row_stride, out + ((batch * heads + h) * T + t) * dk, li,
                               s_cos, s_sin);
}

// A decode step's q/k preparation and KV append in one launch: per token, the
// q rows normed and rotated into q_out [B, Hq, T, dk], the k rows normed and
// rotated into the key buffer and the v rows copied into the value buffer, both
// at (b, h, t) through dst strides (the buffers' slices for the new positions).
template <typename TX, int L>
__global__ __launch_bounds__(QK_THREADS) void decode_qkv_kernel(
    const TX *__restrict__ q, int64_t q_stride, int64_t Hq, const TX *__restrict__ k, int64_t k_stride,
    const TX *__restrict__ v, int64_t v_stride, int64_t Hkv, int64_t T, const float *__restrict__ freq,
    int64_t offset, TX *__restrict__ q_out, TX *__restrict__ k_dst, TX *__restrict__ v_dst, int64_t ds0,
    int64_t ds1, int64_t ds2)
{
    constexpr int dk = 4 * L, rows_per_pass = QK_THREADS / L;
    __shared__ float s_cos[QK_MAX_DK / 2], s_sin[QK_MAX_DK / 2];
    const int64_t bt = blockIdx.x;
    const int64_t t = bt % T, batch = bt / T;
    rotary_angles(freq, 2 * L, offset + t, s_cos, s_sin);
    const int tid = threadIdx.x, li = tid % L;
    for (int64_t h = tid / L; h < Hq + Hkv; h += rows_per_pass) {
        if (h < Hq)
            norm_rotary_row<TX, L>(q + (bt * Hq + h) * q_stride, q_out + ((batch * Hq + h) * T + t) * dk, li, s_cos,
                                   s_sin);
        else
            norm_rotary_row<TX, L>(k + (bt * Hkv + h - Hq) * k_stride, k_dst + batch * ds0 + (h - Hq) * ds1 + t * ds2,
                                   li, s_cos, s_sin);
    }
    for (int64_t e = tid; e < Hkv * dk; e += QK_THREADS) {
        const int64_t h = e / dk, d = e % dk;
        v_dst[batch * ds0 + h * ds1 + t * ds2 + d] = v[(bt * Hkv + h) * v_stride + d];
    }
}

template <typename TX>
static void launch_qk(const void *x, int64_t row_stride, int64_t tokens, int64_t T, int64_t heads, int64_t dk,
                      const float *freq, int64_t offset, void *out, hipStream_t st)
{
    const TX *xp = static_cast<const TX *>(x);
    TX *op = static_cast<TX *>(out);
    const dim3 grid((unsigned)tokens), block(QK_THREADS);
#define GLSDM_QK(LANES)                                                                                       \
    hipLaunchKernelGGL((qk_norm_rotary_kernel<TX, LANES>), grid, block, 0, st, xp, row_stride, T, heads, freq, \
                       offset, op)
    switch (dk / 4) {
    case 1: GLSDM_QK(1); break;
    case 2: GLSDM_QK(2); break;
    case 4: GLSDM_QK(4); break;
    case 8: GLSDM_QK(8); break;
    case 16: GLSDM_QK(16); break;
    case 32: GLSDM_QK(32); break;
    default: GLSDM_QK(64); break;
    }
#undef GLSDM_QK
}

// The attention output's gate (S/layers/attention.py:77, before proj):
// out[b, t, h*dk + i] = o[b, h, t, i] * sigmoid(gate[b, t, h, i]), with the
// sigmoid 1 / (1 + exp(-g)) in fp32 rounded to the dtype, then the product
// rounded to the dtype.  o and gate are read through their strides (SDPA's
// output and the gate half of the [query | gate] projection); out is
// [B, T, H*dk] contiguous, the input of proj.  One thread per element.
template <typename TX>
__global__ __launch_bounds__(256) void gate_merge_kernel(const TX *__restrict__ o, int64_t os0, int64_t os1,
                                                         int64_t os2, const TX *__restrict__ gate, int64_t gs0,
                                                         int64_t gs1, int64_t gs2, int64_t T, int64_t H, int64_t dk,
                                                         int64_t n, TX *__restrict__ out)
{
#pragma clang fp contract(off)
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n) return;
    const int64_t i = e % dk, r = e / dk;                   // r = (b*T + t)*H + h
    const int64_t h = r % H, bt = r / H;
    const int64_t t = bt % T, b = bt / T;
    const float g = RowIO<TX>::load(gate + b * gs0 + t * gs1 + h * gs2 + i);
    const float sig = RowIO<TX>::round(1.0f / (1.0f + expf(-g)));
    const float v = RowIO<TX>::load(o + b * os0 + h * os1 + t * os2 + i);
    RowIO<TX>::store(out + e, v * sig);
}

// The MLP's activation (S/layers/common.py:19-27): with u, g the two halves of
// each row of fc(x) [rows, 2*inner], out = g * relu(u)^2, the square rounded
// to the dtype, then the product rounded to the dtype (the tensor ops'
// roundings).  VEC elements (16 bytes) per thread, inner a multiple of VEC.
template <typename TX> struct Vec16;
template <> struct Vec16<float> {
    static constexpr int N = 4;
    typedef float4 Raw;
    __device__ __forceinline__ static void unpack(const Raw &r, float (&v)[N])
    {
        v[0] = r.x;
        v[1] = r.y;
        v[2] = r.z;
        v[3] = r.w;
    }
    __device__ __forceinline__ static Raw pack(const float (&v)[N]) { return make_float4(v[0], v[1], v[2], v[3]); }
};
template <> struct Vec16<bf16_t> {
    static constexpr int N = 8;
    typedef uint4 Raw;
    __device__ __forceinline__ static void unpack(const Raw &r, float (&v)[N])
    {
        const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = bf16_to_f32((bf16_t)(w[i] & 0xFFFFu));
            v[2 * i + 1] = bf16_to_f32((bf16_t)(w[i] >> 16));
        }
    }
    __device__ __forceinline__ static Raw pack(const float (&v)[N])
    {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            w[i] = (uint32_t)f32_to_bf16(v[2 * i]) | ((uint32_t)f32_to_bf16(v[2 * i + 1]) << 16);
        return make_uint4(w[0], w[1], w[2], w[3]);
    }
};

template <typename TX>
__global__ __launch_bounds__(256) void relu2_gate_kernel(const TX *__restrict__ fc, int64_t rows, int64_t inner,
                                                         TX *__restrict__ out)
{
#pragma clang fp contract(off)
    using V = Vec16<TX>;
    const int64_t per_row = inner / V::N;
    const int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (v >= rows * per_row) return;
    const int64_t r = v / per_row, c = (v % per_row) * V::N;
    const TX *row = fc + r * 2 * inner;
    float u[V::N], g[V::N], o[V::N];
    V::unpack(*reinterpret_cast<const typename V::Raw *>(row + c), u);
    V::unpack(*reinterpret_cast<const typename V::Raw *>(row + inner + c), g);
#pragma unroll
    for (int i = 0; i < V::N; ++i) {
        const float relu = (u[i] > 0.0f || u[i] != u[i]) ? u[i] : 0.0f;   // relu keeps NaN
        const float sq = RowIO<TX>::round(relu * relu);
        o[i] = g[i] * sq;
    }
    *reinterpret_cast<typename V::Raw *>(out + r * inner + c) = V::pack(o);
}

// RMSNorm then a cast (S/layers/common.py:7-17 followed by .to(dtype), as
// the blocks apply it, S/baselines/block.py and S/layers/global_layer.py):
// per row x of dim elements, r = rsqrt(mean(x^2) + eps), y = (x * r) * w in
// fp32 (w the weight rounded to the input dtype) rounded once to the input
// dtype, then to the output dtype -- the roundings of PyTorch's fused GPU
// kernel; the mean's summation order differs from it.  One block per row.
template <typename TI, typename TO, typename TW>
__global__ __launch_bounds__(256) void rms_norm_cast_kernel(const TI *__restrict__ x, const TW *__restrict__ w,
                                                            int64_t dim, float eps, TO *__restrict__ out)
{
#pragma clang fp contract(off)
    __shared__ float s_part[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const TI *row = x + (int64_t)blockIdx.x * dim;
    float ss = 0.0f;
    for (int64_t i = tid; i < dim; i += 256) {
        const float v = RowIO<TI>::load(row + i);
        ss += v * v;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
    if (lane == 0) s_part[wave] = ss;
    __syncthreads();
    const float total = (s_part[0] + s_part[1]) + (s_part[2] + s_part[3]);
    const float r = rsqrtf(total / (float)dim + eps);
    TO *dst = out + (int64_t)blockIdx.x * dim;
    for (int64_t i = tid; i < dim; i += 256) {
        const float t = RowIO<TI>::load(row + i) * r;
        const float y = RowIO<TI>::round(t * RowIO<TI>::round(RowIO<TW>::load(w + i)));
        RowIO<TO>::store(dst + i, y);
    }
}

// The write gates of a global layer's proposal (write_gate_values) from the
// bf16 or fp32 outputs of the beta and decay projections, in fp32.  One thread
// per (token, head).
template <typename TX>
__global__ __launch_bounds__(256) void write_gates_kernel(const TX *__restrict__ b, const TX *__restrict__ d,
                                                          int64_t n, float *__restrict__ beta,
                                                          float *__restrict__ log_decay)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float bet, ld;
    write_gate_values(RowIO<TX>::load(b + i), RowIO<TX>::load(d + i), bet, ld);
    beta[i] = bet;
    log_decay[i] = ld;
}

}  // namespace glsdm

using namespace glsdm;

extern "C" int glsdm_write_gates(const void *beta_in, const void *decay_in, int32_t dtype, int64_t n, float *beta,
                                 float *log_decay, void *stream)
{
    if (n < 0) return fail(GLSDM_ERR_ARG, "write_gates: bad shape");
    if (!dtype_ok(dtype)) return fail(GLSDM_ERR_ARG, "write_gates: bad dtype");
    if (n == 0) return GLSDM_OK;
    if (!beta_in || !decay_in || !beta || !log_decay) return fail(GLSDM_ERR_ARG, "write_gates: null pointer");
    if (ceil_div(n, 256) > INT32_MAX) return fail(GLSDM_ERR_UNSUPPORTED, "write_gates: too many elements");
    const hipStream_t st = as_stream(stream);
    const dim3 grid((unsigned)ceil_div(n, 256)), block(256);
    if (dtype == GLSDM_F32)
        hipLaunchKernelGGL(write_gates_kernel<float>, grid, block, 0, st, static_cast<const float *>(beta_in),
                           static_cast<const float *>(decay_in), n, beta, log_decay);
    else
        hipLaunchKernelGGL(write_gates_kernel<bf16_t>, grid, block, 0, st, static_cast<const bf16_t *>(beta_in),
                           static_cast<const bf16_t *>(decay_in), n, beta, log_decay);
    return check_launch("write_gates_kernel");
}

template <typename TW>
static void launch_rms(const void *x, int32_t x_dtype, const void *weight, int64_t rows, int64_t dim, float eps,
                       void *out, int32_t out_dtype, hipStream_t st)
{
    const TW *w = static_cast<const TW *>(weight);
    const dim3 grid((unsigned)rows), block(256);
#define GLSDM_RMS(TI, TO)                                                                                     \
    hipLaunchKernelGGL((rms_norm_cast_kernel<TI, TO, TW>), grid, block, 0, st, static_cast<const TI *>(x), w,  \
                       dim, eps, static_cast<TO *>(out))
    if (x_dtype == GLSDM_F32 && out_dtype == GLSDM_F32) GLSDM_RMS(float, float);
    else if (x_dtype == GLSDM_F32) GLSDM_RMS(float, bf16_t);
    else if (out_dtype == GLSDM_F32) GLSDM_RMS(bf16_t, float);
    else GLSDM_RMS(bf16_t, bf16_t);
#undef GLSDM_RMS
}

extern "C" int glsdm_rms_norm_cast(const void *x, int32_t x_dtype, const void *weight, int32_t w_dtype, int64_t rows,
                                   int64_t dim, float eps, void *out, int32_t out_dtype, void *stream)
{
    if (rows < 0 || dim < 1) return fail(GLSDM_ERR_ARG, "rms_norm_cast: bad shape");
    if (!dtype_ok(x_dtype) || !dtype_ok(out_dtype) || !dtype_ok(w_dtype))
        return fail(GLSDM_ERR_ARG, "rms_norm_cast: bad dtype");
    if (rows == 0) return GLSDM_OK;
    if (rows > INT32_MAX) return fail(GLSDM_ERR_UNSUPPORTED, "rms_norm_cast: more than 2^31-1 rows");
    if (!x || !weight || !out) return fail(GLSDM_ERR_ARG, "rms_norm_cast: null pointer");
    const hipStream_t st = as_stream(stream);
    if (w_dtype == GLSDM_F32)
        launch_rms<float>(x, x_dtype, weight, rows, dim, eps, out, out_dtype, st);
    else
        launch_rms<bf16_t>(x, x_dtype, weight, rows, dim, eps, out, out_dtype, st);
    return check_launch("rms_norm_cast_kernel");
}

extern "C" int glsdm_relu2_gate(const void *fc, int32_t dtype, int64_t rows, int64_t inner, void *out, void *stream)
{
    if (rows < 0 || inner < 1) return fail(GLSDM_ERR_ARG, "relu2_gate: bad shape");
    if (!dtype_ok(dtype)) return fail(GLSDM_ERR_ARG, "relu2_gate: bad dtype");
    const int vec = dtype == GLSDM_F32 ? 4 : 8;
    if (inner % vec != 0) return fail(GLSDM_ERR_UNSUPPORTED, "relu2_gate: inner %lld not a multiple of %d",
                                      (long long)inner, vec);
    if (rows == 0) return GLSDM_OK;
    if (!fc || !out) return fail(GLSDM_ERR_ARG, "relu2_gate: null pointer");
    if ((reinterpret_cast<uintptr_t>(fc) | reinterpret_cast<uintptr_t>(out)) & 15)
        return fail(GLSDM_ERR_UNSUPPORTED, "relu2_gate: pointers must be 16-byte aligned");
    const int64_t threads = rows * (inner / vec);
    if (ceil_div(threads, 256) > INT32_MAX) return fail(GLSDM_ERR_UNSUPPORTED, "relu2_gate: too many elements");
    const hipStream_t st = as_stream(stream);
    const dim3 grid((unsigned)ceil_div(threads, 256)), block(256);
    if (dtype == GLSDM_F32)
        hipLaunchKernelGGL(relu2_gate_kernel<float>, grid, block, 0, st, static_cast<const float *>(fc), rows, inner,
                           static_cast<float *>(out));
    else
        hipLaunchKernelGGL(relu2_gate_kernel<bf16_t>, grid, block, 0, st, static_cast<const bf16_t *>(fc), rows,
                           inner, static_cast<bf16_t *>(out));
    return check_launch("relu2_gate_kernel");
}

extern "C" int glsdm_gate_merge(const void *o, const int64_t *o_strides, const void *gate, const int64_t *gate_strides,
                                int32_t dtype, int64_t B, int64_t T, int64_t H, int64_t dk, void *out, void *stream)
{
    if (B < 0 || T < 0 || H < 1 || dk < 1) return fail(GLSDM_ERR_ARG, "gate_merge: bad shape");
    if (!dtype_ok(dtype)) return fail(GLSDM_ERR_ARG, "gate_merge: bad dtype");
    const int64_t n = B * T * H * dk;
    if (n == 0) return GLSDM_OK;
    if (!o || !o_strides || !gate || !gate_strides || !out) return fail(GLSDM_ERR_ARG, "gate_merge: null pointer");
    if (o_strides[3] != 1 || gate_strides[3] != 1)
        return fail(GLSDM_ERR_UNSUPPORTED, "gate_merge: the last dimension must be contiguous");
    if (ceil_div(n, 256) > INT32_MAX) return fail(GLSDM_ERR_UNSUPPORTED, "gate_merge: too many elements");
    const hipStream_t st = as_stream(stream);
    const dim3 grid((unsigned)ceil_div(n, 256)), block(256);
    if (dtype == GLSDM_F32)
        hipLaunchKernelGGL(gate_merge_kernel<float>, grid, block, 0, st, static_cast<const float *>(o), o_strides[0],
                           o_strides[1], o_strides[2], static_cast<const float *>(gate), gate_strides[0],
                           gate_strides[1], gate_strides[2], T, H, dk, n, static_cast<float *>(out));
    else
        hipLaunchKernelGGL(gate_merge_kernel<bf16_t>, grid, block, 0, st, static_cast<const bf16_t *>(o),
                           o_strides[0], o_strides[1], o_strides[2], static_cast<const bf16_t *>(gate),
                           gate_strides[0], gate_strides[1], gate_strides[2], T, H, dk, n,
                           static_cast<bf16_t *>(out));
    return check_launch("gate_merge_kernel");
}

template <typename TX>
static void launch_decode_qkv(const void *q, int64_t q_stride, int64_t Hq, const void *k, int64_t k_stride,
                              const void *v, int64_t v_stride, int64_t Hkv, int64_t tokens, int64_t T, int64_t dk,
                              const float *freq, int64_t offset, void *q_out, void *k_dst, void *v_dst,
                              const int64_t *ds, hipStream_t st)
{
    const TX *qp = static_cast<const TX *>(q), *kp = static_cast<const TX *>(k), *vp = static_cast<const TX *>(v);
    TX *qo = static_cast<TX *>(q_out), *kd = static_cast<TX *>(k_dst), *vd = static_cast<TX *>(v_dst);
    const dim3 grid((unsigned)tokens), block(QK_THREADS);
#define GLSDM_DQKV(LANES)                                                                                          \
    hipLaunchKernelGGL((decode_qkv_kernel<TX, LANES>), grid, block, 0, st, qp, q_stride, Hq, kp, k_stride, vp,     \
                       v_stride, Hkv, T, freq, offset, qo, kd, vd, ds[0], ds[1], ds[2])
    switch (dk / 4) {
    case 1: GLSDM_DQKV(1); break;
    case 2: GLSDM_DQKV(2); break;
    case 4: GLSDM_DQKV(4); break;
    case 8: GLSDM_DQKV(8); break;
    case 16: GLSDM_DQKV(16); break;
    case 32: GLSDM_DQKV(32); break;
    default: GLSDM_DQKV(64); break;
    }
#undef GLSDM_DQKV
}

extern "C" int glsdm_decode_qkv(const void *q, int64_t q_row_stride, int64_t q_heads, const void *k,
                                int64_t k_row_stride, const void *v, int64_t v_row_stride, int64_t kv_heads,
                                int32_t dtype, int64_t B, int64_t T, int64_t dk, const float *freq, int64_t offset,
                                void *q_out, void *k_dst, void *v_dst, const int64_t *dst_strides, void *stream)
{
    const bool pow2 = dk >= 4 && dk <= QK_MAX_DK && (dk & (dk - 1)) == 0;
    if (B < 0 || T < 0 || q_heads < 1 || kv_heads < 1 || !pow2 || q_row_stride < dk || k_row_stride < dk ||
        v_row_stride < dk || offset < 0)
        return fail(GLSDM_ERR_ARG, "decode_qkv: bad shape (dk a power of two in [4, 256], row strides >= dk)");
    if (!dtype_ok(dtype)) return fail(GLSDM_ERR_ARG, "decode_qkv: bad dtype");
    if (offset + T > (int64_t)1 << 24)
        return fail(GLSDM_ERR_UNSUPPORTED, "decode_qkv: positions above 2^24 are not exact in fp32");
    const int64_t tokens = B * T;
    if (tokens == 0) return GLSDM_OK;
    if (tokens > INT32_MAX) return fail(GLSDM_ERR_UNSUPPORTED, "decode_qkv: more than 2^31-1 tokens");
    if (!q || !k || !v || !freq || !q_out || !k_dst || !v_dst || !dst_strides)
        return fail(GLSDM_ERR_ARG, "decode_qkv: null pointer");
    const hipStream_t st = as_stream(stream);
    if (dtype == GLSDM_F32)
        launch_decode_qkv<float>(q, q_row_stride, q_heads, k, k_row_stride, v, v_row_stride, kv_heads, tokens, T, dk,
                                 freq, offset, q_out, k_dst, v_dst, dst_strides, st);
    else
        launch_decode_qkv<bf16_t>(q, q_row_stride, q_heads, k, k_row_stride, v, v_row_stride, kv_heads, tokens, T,
                                  dk, freq, offset, q_out, k_dst, v_dst, dst_strides, st);
    return check_launch("decode_qkv_kernel");
}

extern "C" int glsdm_qk_norm_rotary(const void *x, int32_t dtype, int64_t B, int64_t T, int64_t heads, int64_t dk,
                                    int64_t row_stride, const float *freq, int64_t offset, void *out, void *stream)
{
    const bool pow2 = dk >= 4 && dk <= QK_MAX_DK && (dk & (dk - 1)) == 0;
    if (B < 0 || T < 0 || heads < 1 || !pow2 || row_stride < dk || offset < 0)
        return fail(GLSDM_ERR_ARG, "qk_norm_rotary: bad shape B=%lld T=%lld heads=%lld dk=%lld stride=%lld "
                    "(dk a power of two in [4, 256])", (long long)B, (long long)T, (long long)heads, (long long)dk,
                    (long long)row_stride);
    if (!dtype_ok(dtype)) return fail(GLSDM_ERR_ARG, "qk_norm_rotary: bad dtype");
    if (offset + T > (int64_t)1 << 24)
        return fail(GLSDM_ERR_UNSUPPORTED, "qk_norm_rotary: positions above 2^24 are not exact in fp32");
    const int64_t tokens = B * T;
    if (tokens == 0) return GLSDM_OK;
    if (tokens > INT32_MAX) return fail(GLSDM_ERR_UNSUPPORTED, "qk_norm_rotary: more than 2^31-1 tokens");
    if (!x || !freq || !out) return fail(GLSDM_ERR_ARG, "qk_norm_rotary: null pointer");
    const hipStream_t st = as_stream(stream);
    if (dtype == GLSDM_F32)
        launch_qk<float>(x, row_stride, tokens, T, heads, dk, freq, offset, out, st);
    else
        launch_qk<bf16_t>(x, row_stride, tokens, T, heads, dk, freq, offset, out, st);
    return check_launch("qk_norm_rotary_kernel");
}
