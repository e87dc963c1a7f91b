// Internal helpers shared by the gfx950 kernels of libglsdm.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "glsdm.h"

namespace glsdm {

// ---------------------------------------------------------------- host side
int fail(int status, const char *fmt, ...);   // records glsdm_last_error()
int check_launch(const char *what);           // hipGetLastError -> status

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }
__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline int pow2_ceil(int64_t x)
{
    int p = 1;
    while (p < x) p <<= 1;
    return p;
}
inline size_t dtype_size(int32_t dt) { return dt == GLSDM_BF16 ? 2 : 4; }
inline bool dtype_ok(int32_t dt) { return dt == GLSDM_F32 || dt == GLSDM_BF16; }

// Layout of one bank/value row of D elements over the lanes of a wave:
// `vec` elements per 16-byte (or scalar) access, `nv` accesses per row,
// `lpr` lanes per row (power of two <= 64), `ch` accesses per lane.
struct RowPlan {
    int vec, nv, lpr, ch;
};
inline RowPlan row_plan(int64_t D, size_t elem)
{
    RowPlan p;
    int full = (int)(16 / elem);
    p.vec = (D % full == 0) ? full : 1;
    p.nv = (int)(D / p.vec);
    p.lpr = pow2_ceil(p.nv) < 64 ? pow2_ceil(p.nv) : 64;
    p.ch = (int)ceil_div(p.nv, p.lpr);
    return p;
}

// ---------------------------------------------------------------- device side
typedef uint16_t bf16_t;

__device__ __forceinline__ float bf16_to_f32(bf16_t h)
{
    return __uint_as_float(((uint32_t)h) << 16);
}

// Round-to-nearest-even fp32 -> bf16; NaN becomes the quiet NaN 0x7FC0.
__device__ __forceinline__ bf16_t f32_to_bf16(float f)
{
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (bf16_t)0x7FC0;
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (bf16_t)(u >> 16);
}

// Monotone map of an fp32 score to uint32: a < b  <=>  key(a) < key(b).
// -0 and +0 map to the same key (torch's sorts compare them equal) and every
// NaN maps above +inf (torch sorts NaN as the largest value).
__device__ __forceinline__ uint32_t order_bits(float x)
{
    if (x != x) return 0xFFFFFFFFu;
    uint32_t b = __float_as_uint(x == 0.0f ? 0.0f : x);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Inverse of order_bits (maps the folded keys back to +0 / canonical NaN).
__device__ __forceinline__ float order_value(uint32_t k)
{
    uint32_t b = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
    return __uint_as_float(b);
}

// Composite rank key: score first, then the tie rule on the index.  All keys of
// real elements are > 0, so 0 is a sentinel below every element.
__device__ __forceinline__ uint64_t rank_key(float score, uint32_t index, int tie)
{
    uint32_t t = tie == GLSDM_TIE_HIGHEST ? index : 0xFFFFFFFFu - index;
    return ((uint64_t)order_bits(score) << 32) | t;
}

__device__ __forceinline__ uint32_t rank_index(uint64_t key, int tie)
{
    uint32_t lo = (uint32_t)key;
    return tie == GLSDM_TIE_HIGHEST ? lo : 0xFFFFFFFFu - lo;
}

// 32-bit rank key of a bf16 score: the bf16 order bits (the 16-bit analogue of
// order_bits: -0 folded onto +0, NaN above +inf) above the 16-bit tie bits of
// the index (< 65536).  On bf16 values it orders exactly as rank_key does on
// the same values widened to fp32.
__device__ __forceinline__ uint32_t rank_key16(bf16_t b, uint32_t index, int tie)
{
    uint32_t o;
    if ((b & 0x7FFFu) > 0x7F80u) o = 0xFFFFu;
    else if ((b & 0x7FFFu) == 0) o = 0x8000u;
    else o = (b & 0x8000u) ? (~(uint32_t)b & 0xFFFFu) : ((uint32_t)b | 0x8000u);
    const uint32_t t = tie == GLSDM_TIE_HIGHEST ? index : 0xFFFFu - index;
    return (o << 16) | t;
}

// Score and index of a rank key (64-bit fp32 keys and 32-bit bf16 keys).
__device__ __forceinline__ float key_value(uint64_t k) { return order_value((uint32_t)(k >> 32)); }
__device__ __forceinline__ uint32_t key_index(uint64_t k, int tie) { return rank_index(k, tie); }
__device__ __forceinline__ float key_value(uint32_t k)
{
    const uint32_t o = k >> 16;
    const uint32_t b = (o & 0x8000u) ? (o & 0x7FFFu) : (~o & 0xFFFFu);
    return __uint_as_float(b << 16);
}
__device__ __forceinline__ uint32_t key_index(uint32_t k, int tie)
{
    const uint32_t lo = k & 0xFFFFu;
    return tie == GLSDM_TIE_HIGHEST ? lo : 0xFFFFu - lo;
}
// The 64-bit key of the same element (0, the empty-slot sentinel, stays 0).
__device__ __forceinline__ uint64_t widen_key(uint32_t k, int tie)
{
    return k ? rank_key(key_value(k), key_index(k, tie), tie) : 0;
}

// Factor key of an fp32 score with an index below 65536, as a double: the
// 48-bit key (order_bits(score) << 16 | 16-bit tie bits) placed at bits
// [14, 62) above 2^52, i.e. a positive normal double whose numeric order is the
// key order.  Compare-exchanges of such keys are one v_max_f64 and one
// v_min_f64 (exact on finite values) instead of a 64-bit compare and four
// selects; 0.0 is the empty-slot sentinel below every key.
__device__ __forceinline__ double rank_keyd(float score, uint32_t index, int tie)
{
    const uint32_t t = tie == GLSDM_TIE_HIGHEST ? index : 0xFFFFu - index;
    const uint64_t k48 = ((uint64_t)order_bits(score) << 16) | t;
    return __longlong_as_double((long long)((1ull << 52) + (k48 << 14)));
}
__device__ __forceinline__ uint64_t keyd_bits(double k)
{
    return ((uint64_t)__double_as_longlong(k) - (1ull << 52)) >> 14;
}
__device__ __forceinline__ float key_value(double k) { return order_value((uint32_t)(keyd_bits(k) >> 16)); }
__device__ __forceinline__ uint32_t key_index(double k, int tie)
{
    const uint32_t lo = (uint32_t)keyd_bits(k) & 0xFFFFu;
    return tie == GLSDM_TIE_HIGHEST ? lo : 0xFFFFu - lo;
}
// A 64-bit rank key of a factor element (index < 65536) as its double key
// (the same order: the 16-bit tie bits are the low 16 of the 32-bit ones).
__device__ __forceinline__ double narrow_keyd(uint64_t k)
{
    if (k == 0) return 0.0;
    const uint64_t k48 = ((k >> 32) << 16) | (k & 0xFFFFu);
    return __longlong_as_double((long long)((1ull << 52) + (k48 << 14)));
}
__device__ __forceinline__ uint64_t widen_key(double k, int tie)
{
    return k != 0.0 ? rank_key(key_value(k), key_index(k, tie), tie) : 0;
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int mask)
{
    uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
    lo = (uint32_t)__shfl_xor((int)lo, mask);
    hi = (uint32_t)__shfl_xor((int)hi, mask);
    return ((uint64_t)hi << 32) | lo;
}

// The write gates of a global layer's proposal (S/layers/global_layer.py:48-49)
// from the beta and decay projections' outputs b and d, in fp32:
// beta = sigmoid(b) = 1 / (1 + exp(-b)) and log_decay = -softplus(d - 4) with
// softplus(v) = v above 20, else log1p(exp(v)).
__device__ __forceinline__ void write_gate_values(float b, float d, float &beta, float &log_decay)
{
#pragma clang fp contract(off)
    beta = 1.0f / (1.0f + expf(-b));
    const float v = d - 4.0f;
    const float sp = v > 20.0f ? v : log1pf(expf(v));
    log_decay = -sp;
}

// Load `VEC` consecutive elements of type T starting at p (16-byte aligned when
// VEC*sizeof(T) == 16) and widen them to fp32.
template <typename T, int VEC> struct VecLoad;

template <int VEC> struct VecLoad<float, VEC> {
    __device__ __forceinline__ static void load(const float *p, float (&x)[VEC])
    {
        if constexpr (VEC == 4) {
            float4 v = *reinterpret_cast<const float4 *>(p);
            x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
        } else {
#pragma unroll
            for (int i = 0; i < VEC; ++i) x[i] = p[i];
        }
    }
};

template <int VEC> struct VecLoad<bf16_t, VEC> {
    __device__ __forceinline__ static void load(const bf16_t *p, float (&x)[VEC])
    {
        if constexpr (VEC == 8) {
            uint4 v = *reinterpret_cast<const uint4 *>(p);
            uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                x[2 * i] = __uint_as_float(w[i] << 16);
                x[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
            }
        } else {
#pragma unroll
            for (int i = 0; i < VEC; ++i) x[i] = bf16_to_f32(p[i]);
        }
    }
};

#ifndef GLSDM_NT
#define GLSDM_NT 1
#endif
typedef unsigned int glsdm_u32x4 __attribute__((ext_vector_type(4)));

// A 16-byte load / store with the nontemporal hint (data used once: streamed
// past the caches' replacement), when GLSDM_NT is set.
__device__ __forceinline__ uint4 load16_stream(const void *p)
{
#if GLSDM_NT
    const glsdm_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const glsdm_u32x4 *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
#else
    return *reinterpret_cast<const uint4 *>(p);
#endif
}
__device__ __forceinline__ void store16_stream(void *p, uint4 u)
{
#if GLSDM_NT
    glsdm_u32x4 v = {u.x, u.y, u.z, u.w};
    __builtin_nontemporal_store(v, reinterpret_cast<glsdm_u32x4 *>(p));
#else
    *reinterpret_cast<uint4 *>(p) = u;
#endif
}

template <typename T, int VEC> struct VecStore;

template <int VEC> struct VecStore<float, VEC> {
    __device__ __forceinline__ static void store(float *p, const float (&x)[VEC])
    {
        if constexpr (VEC == 4) {
            *reinterpret_cast<float4 *>(p) = make_float4(x[0], x[1], x[2], x[3]);
        } else {
#pragma unroll
            for (int i = 0; i < VEC; ++i) p[i] = x[i];
        }
    }
};

template <int VEC> struct VecStore<bf16_t, VEC> {
    __device__ __forceinline__ static void store(bf16_t *p, const float (&x)[VEC])
    {
        if constexpr (VEC == 8) {
            uint32_t w[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                w[i] = (uint32_t)f32_to_bf16(x[2 * i]) | ((uint32_t)f32_to_bf16(x[2 * i + 1]) << 16);
            *reinterpret_cast<uint4 *>(p) = make_uint4(w[0], w[1], w[2], w[3]);
        } else {
#pragma unroll
            for (int i = 0; i < VEC; ++i) p[i] = f32_to_bf16(x[i]);
        }
    }
};

}  // namespace glsdm
