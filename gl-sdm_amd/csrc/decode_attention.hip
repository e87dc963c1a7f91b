// One-token attention over a local window, for the stack's decode steps, on gfx950.
//
// Semantics: F.scaled_dot_product_attention of S/layers/attention.py:76 for a
// single query row per (request, head) whose keys all lie inside the window
// (so the window mask is all zeros): out = softmax(q . k_j * scale) . v_j over
// the L cached keys, fp32 scores, exponentials and sums, the output rounded
// once to bf16.  The summation order is this kernel's (the library's flash
// kernel has its own), so results agree with SDPA's to rounding.
//
// One block per (request, head), four waves splitting the keys into four
// ranges (flash-decoding): a lane scores one key at a time (the key row is 8
// 16-byte loads, the query sits in registers), the wave reduces its maximum and
// sum with shuffles, stores its probabilities in LDS and then accumulates
// p_j * v_j with lane d owning output dimension d (each value row is one
// coalesced 128-byte read); the four partial results are merged in wave order.
// Keys and values are read through (request, head, key) strides, so the cache's
// window views need no copy.  With a gate, the output row is multiplied by
// bf16(sigmoid(gate)) and rounded again (the local layer's output gate,
// S/layers/attention.py:77, with the roundings of its bf16 tensor ops).
#include "glsdm_internal.h"

namespace glsdm {

constexpr int DA_MAX_KEYS = 1024;

template <int DK>
__global__ __launch_bounds__(256) void decode_attention_kernel(const bf16_t *__restrict__ q,
                                                               const bf16_t *__restrict__ k,
                                                               const bf16_t *__restrict__ v, bf16_t *__restrict__ out,
                                                               int64_t H, int L, int64_t ksb, int64_t ksh,
                                                               int64_t ksl, int64_t vsb, int64_t vsh, int64_t vsl,
                                                               float scale, const bf16_t *__restrict__ gate,
                                                               int64_t gsb, int64_t gsh)
{
#pragma clang fp contract(off)
    __shared__ float s_p[4][DA_MAX_KEYS / 4];
    __shared__ float s_m[4], s_l[4];
    __shared__ float s_acc[4][DK];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t bh = blockIdx.x, b = bh / H, h = bh % H;
    const bf16_t *kb = k + b * ksb + h * ksh, *vb = v + b * vsb + h * vsh;
    // the gate element of output dimension threadIdx.x, loaded before the key loop
    const float gval = gate && threadIdx.x < DK ? bf16_to_f32(gate[b * gsb + h * gsh + threadIdx.x]) : 0.0f;
    // the query row in fp32 registers (every lane holds all of it)
    float qf[DK];
#pragma unroll
    for (int p = 0; p < DK / 8; ++p) {
        const uint4 u = *reinterpret_cast<const uint4 *>(q + bh * DK + p * 8);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            qf[p * 8 + 2 * i] = __uint_as_float(w[i] << 16);
            qf[p * 8 + 2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
        }
    }
    const int per = (L + 3) / 4, j0 = wave * per, j1 = min(L, j0 + per);
    // scores of this wave's keys, one per lane at a time
    float m = -INFINITY;
    for (int j = j0 + lane; j < j1; j += 64) {
        const bf16_t *kr = kb + (int64_t)j * ksl;
        float s = 0.0f;
#pragma unroll
        for (int p = 0; p < DK / 8; ++p) {
            const uint4 u = *reinterpret_cast<const uint4 *>(kr + p * 8);
            const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                s = s + qf[p * 8 + 2 * i] * __uint_as_float(w[i] << 16);
                s = s + qf[p * 8 + 2 * i + 1] * __uint_as_float(w[i] & 0xFFFF0000u);
            }
        }
        s = s * scale;
        s_p[wave][j - j0] = s;
        m = fmaxf(m, s);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float l = 0.0f;
    for (int j = j0 + lane; j < j1; j += 64) {
        const float p = j1 > j0 ? expf(s_p[wave][j - j0] - m) : 0.0f;
        s_p[wave][j - j0] = p;
        l = l + p;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) l = l + __shfl_xor(l, o);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // p_j * v_j: lane d owns output dimension d (DK <= 64) or d and d + 64
    float acc[DK / 64 > 0 ? DK / 64 : 1];
#pragma unroll
    for (int c = 0; c < (DK + 63) / 64; ++c) acc[c] = 0.0f;
#pragma unroll 8
    for (int j = j0; j < j1; ++j) {
        const float p = s_p[wave][j - j0];
        const bf16_t *vr = vb + (int64_t)j * vsl;
#pragma unroll
        for (int c = 0; c < (DK + 63) / 64; ++c) {
            const int d = lane + 64 * c;
            if (d < DK) acc[c] = acc[c] + p * bf16_to_f32(vr[d]);
        }
    }
    if (lane == 0) {
        s_m[wave] = m;
        s_l[wave] = l;
    }
#pragma unroll
    for (int c = 0; c < (DK + 63) / 64; ++c) {
        const int d = lane + 64 * c;
        if (d < DK) s_acc[wave][d] = acc[c];
    }
    __syncthreads();
    // merge the four ranges in wave order (an empty range has m = -inf and adds nothing)
    if (threadIdx.x < DK) {
        const int d = threadIdx.x;
        float M = s_m[0];
#pragma unroll
        for (int w = 1; w < 4; ++w) M = fmaxf(M, s_m[w]);
        float num = 0.0f, den = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float f = s_m[w] == -INFINITY ? 0.0f : expf(s_m[w] - M);
            num = num + f * s_acc[w][d];
            den = den + f * s_l[w];
        }
        if (gate) {
            const float a = bf16_to_f32(f32_to_bf16(num / den));
            const float sig = bf16_to_f32(f32_to_bf16(1.0f / (1.0f + expf(-gval))));
            out[bh * DK + d] = f32_to_bf16(a * sig);
        } else {
            out[bh * DK + d] = f32_to_bf16(num / den);
        }
    }
}

}  // namespace glsdm

using namespace glsdm;

namespace {

int decode_attention(const void *q, const void *k, const void *v, const void *gate, void *out, int64_t B, int64_t H,
                     int64_t L, int64_t dk, const int64_t *k_strides, const int64_t *v_strides,
                     const int64_t *gate_strides, float scale, void *stream)
{
    if (B < 1 || H < 1 || L < 1 || dk < 1) return fail(GLSDM_ERR_ARG, "decode_attention: bad shape");
    if (L > DA_MAX_KEYS || (dk != 64 && dk != 128))
        return fail(GLSDM_ERR_UNSUPPORTED, "decode_attention: at most 1024 keys and dk 64 or 128");
    if (!q || !k || !v || !out || !k_strides || !v_strides || (gate && !gate_strides))
        return fail(GLSDM_ERR_ARG, "decode_attention: null pointer");
    if (((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k)) & 15) != 0 || k_strides[2] % 8 != 0 ||
        k_strides[0] % 8 != 0 || k_strides[1] % 8 != 0)
        return fail(GLSDM_ERR_UNSUPPORTED, "decode_attention: query and key rows must be 16-byte aligned");
    const bf16_t *qq = static_cast<const bf16_t *>(q), *kk = static_cast<const bf16_t *>(k),
                 *vv = static_cast<const bf16_t *>(v), *gg = static_cast<const bf16_t *>(gate);
    bf16_t *oo = static_cast<bf16_t *>(out);
    const int64_t gsb = gate ? gate_strides[0] : 0, gsh = gate ? gate_strides[1] : 0;
    const dim3 grid((unsigned)(B * H)), block(256);
    if (dk == 64)
        hipLaunchKernelGGL((decode_attention_kernel<64>), grid, block, 0, as_stream(stream), qq, kk, vv, oo, H, (int)L,
                           k_strides[0], k_strides[1], k_strides[2], v_strides[0], v_strides[1], v_strides[2], scale,
                           gg, gsb, gsh);
    else
        hipLaunchKernelGGL((decode_attention_kernel<128>), grid, block, 0, as_stream(stream), qq, kk, vv, oo, H, (int)L,
                           k_strides[0], k_strides[1], k_strides[2], v_strides[0], v_strides[1], v_strides[2], scale,
                           gg, gsb, gsh);
    return check_launch("decode_attention_kernel");
}

}  // namespace

extern "C" int glsdm_decode_attention(const void *q, const void *k, const void *v, void *out, int64_t B, int64_t H,
                                      int64_t L, int64_t dk, const int64_t *k_strides, const int64_t *v_strides,
                                      float scale, void *stream)
{
    return decode_attention(q, k, v, nullptr, out, B, H, L, dk, k_strides, v_strides, nullptr, scale, stream);
}

extern "C" int glsdm_decode_attention_gated(const void *q, const void *k, const void *v, const void *gate, void *out,
                                            int64_t B, int64_t H, int64_t L, int64_t dk, const int64_t *k_strides,
                                            const int64_t *v_strides, const int64_t *gate_strides, float scale,
                                            void *stream)
{
    if (!gate) return fail(GLSDM_ERR_ARG, "decode_attention_gated: null gate");
    return decode_attention(q, k, v, gate, out, B, H, L, dk, k_strides, v_strides, gate_strides, scale, stream);
}
