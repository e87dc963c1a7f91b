// Overlay snapshots on gfx950: reads and dense materialisation.
//
// An overlay view holds one immutable base bank [H, S, D] shared by all B
// requests, a slot map int32 [B, H, S] (-1: the base row) and a pool of
// touched rows [capacity, D]; glsdm_overlay_commit (commit.hip) writes the pool.
// Row (b, h, slot) of the logical bank is pool[map[b,h,slot]] when mapped, else
// base[h, slot].  This replaces the per-request clones of
// S/memory/state.py:61-62 (snapshot) and the full-bank functional copy of
// S/memory/transactions.py:96 (commit) with storage that grows with the touched
// rows; results equal the dense bank's bit for bit.
//
// Read layout as read.hip: one wavefront per output row, 16-byte row pieces
// over `lpr` lanes, 64/lpr picks in flight, fp32 accumulation without FMA
// contraction; the only difference is the map lookup per pick.
#include "glsdm_internal.h"

namespace glsdm {

template <typename TB, typename TO, int VEC, int CH>
__global__ __launch_bounds__(256) void overlay_read_kernel(const TB *__restrict__ base,
                                                           const int32_t *__restrict__ map,
                                                           const TB *__restrict__ pool, int64_t H, int64_t S,
                                                           int64_t D, int64_t T, int width,
                                                           const int64_t *__restrict__ index,
                                                           const float *__restrict__ weights, TO *__restrict__ out,
                                                           int64_t rows, int nv, int lpr)
{
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;  // wave-uniform
    const int ng = 64 / lpr, grp = lane / lpr, li = lane % lpr;
    const int64_t b = r / (T * H), h = r % H;
    const int32_t *part_map = map + (b * H + h) * S;
    const TB *part_base = base + h * S * D;
    const int64_t *ix = index + r * width;
    const float *wt = weights + r * width;
    float acc[CH][VEC];
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[c][e] = 0.0f;
#pragma unroll 4
    for (int j = grp; j < width; j += ng) {
        const int64_t slot = ix[j];
        const float w = wt[j];
        if (slot < 0 || slot >= S) continue;
        const int32_t m = part_map[slot];
        const TB *row = m >= 0 ? pool + (int64_t)m * D : part_base + slot * D;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int v = li + c * lpr;
            if (v < nv) {
                float x[VEC];
                VecLoad<TB, VEC>::load(row + (int64_t)v * VEC, x);
#pragma unroll
                for (int e = 0; e < VEC; ++e) acc[c][e] += x[e] * w;
            }
        }
    }
    for (int s = lpr; s < 64; s <<= 1) {
#pragma unroll
        for (int c = 0; c < CH; ++c)
#pragma unroll
            for (int e = 0; e < VEC; ++e) acc[c][e] += __shfl_xor(acc[c][e], s);
    }
    if (grp == 0) {
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int v = li + c * lpr;
            if (v < nv) VecStore<TO, VEC>::store(out + r * D + (int64_t)v * VEC, acc[c]);
        }
    }
}

// Dense copy of the logical bank: one thread per element (serving state or checks).
template <typename TB>
__global__ __launch_bounds__(256) void overlay_materialise_kernel(const TB *__restrict__ base,
                                                                  const int32_t *__restrict__ map,
                                                                  const TB *__restrict__ pool, int64_t HS,
                                                                  int64_t D, int64_t total, TB *__restrict__ out)
{
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t a = i / D, d = i - a * D;
        const int32_t m = map[a];
        out[i] = m >= 0 ? pool[(int64_t)m * D + d] : base[(a % HS) * D + d];
    }
}

template <typename TB, typename TO, int VEC>
static int launch_overlay_read(const void *base, const int32_t *map, const void *pool, int64_t H, int64_t S,
                               int64_t D, int64_t T, int width, const int64_t *index, const float *weights,
                               void *out, int64_t rows, const RowPlan &p, hipStream_t st)
{
    const dim3 grid((unsigned)ceil_div(rows, 4)), block(256);
    const TB *bs = static_cast<const TB *>(base), *pl = static_cast<const TB *>(pool);
    TO *o = static_cast<TO *>(out);
#define GLSDM_OVR(C)                                                                                          \
    hipLaunchKernelGGL((overlay_read_kernel<TB, TO, VEC, C>), grid, block, 0, st, bs, map, pl, H, S, D, T, width, \
                       index, weights, o, rows, p.nv, p.lpr)
    switch (p.ch) {
    case 1: GLSDM_OVR(1); break;
    case 2: GLSDM_OVR(2); break;
    case 3:
    case 4: GLSDM_OVR(4); break;
    default: GLSDM_OVR(8); break;
    }
#undef GLSDM_OVR
    return check_launch("overlay_read_kernel");
}

template <typename TB, typename TO>
static int overlay_read_t(const void *base, const int32_t *map, const void *pool, int64_t H, int64_t S, int64_t D,
                          int64_t T, int width, const int64_t *index, const float *weights, void *out,
                          int64_t rows, hipStream_t st)
{
    constexpr int FULL = 16 / sizeof(TB);
    RowPlan p = row_plan(D, sizeof(TB));
    const bool aligned = ((reinterpret_cast<uintptr_t>(base) | reinterpret_cast<uintptr_t>(pool) |
                           reinterpret_cast<uintptr_t>(out)) & 15) == 0;
    if (p.vec == FULL && aligned)
        return launch_overlay_read<TB, TO, FULL>(base, map, pool, H, S, D, T, width, index, weights, out, rows, p,
                                                 st);
    p = RowPlan{1, (int)D, D < 64 ? pow2_ceil(D) : 64, (int)ceil_div(D, 64)};
    return launch_overlay_read<TB, TO, 1>(base, map, pool, H, S, D, T, width, index, weights, out, rows, p, st);
}

}  // namespace glsdm

using namespace glsdm;

extern "C" int glsdm_overlay_read(const void *base, int32_t dtype, const int32_t *map, const void *pool, int64_t B,
                                  int64_t H, int64_t S, int64_t D, int64_t T, int32_t width, const int64_t *index,
                                  const float *weights, void *out, int32_t out_dtype, void *stream)
{
    if (B < 0 || H < 1 || S < 1 || D < 1 || T < 0 || width < 1) return fail(GLSDM_ERR_ARG, "overlay_read: bad shape");
    if (!dtype_ok(dtype) || !dtype_ok(out_dtype)) return fail(GLSDM_ERR_ARG, "overlay_read: bad dtype");
    if (width > 1024) return fail(GLSDM_ERR_UNSUPPORTED, "overlay_read: width > 1024");
    const int64_t rows = B * T * H;
    if (rows == 0) return GLSDM_OK;
    const int64_t max_d = (D % (int64_t)(16 / dtype_size(dtype)) == 0) ? 64 * 8 * (16 / (int64_t)dtype_size(dtype)) : 512;
    if (D > max_d) return fail(GLSDM_ERR_UNSUPPORTED, "overlay_read: D=%lld above %lld", (long long)D, (long long)max_d);
    if (!base || !map || !pool || !index || !weights || !out) return fail(GLSDM_ERR_ARG, "overlay_read: null pointer");
    const hipStream_t st = as_stream(stream);
    if (dtype == GLSDM_F32 && out_dtype == GLSDM_F32)
        return overlay_read_t<float, float>(base, map, pool, H, S, D, T, width, index, weights, out, rows, st);
    if (dtype == GLSDM_BF16 && out_dtype == GLSDM_F32)
        return overlay_read_t<bf16_t, float>(base, map, pool, H, S, D, T, width, index, weights, out, rows, st);
    if (dtype == GLSDM_F32)
        return overlay_read_t<float, bf16_t>(base, map, pool, H, S, D, T, width, index, weights, out, rows, st);
    return overlay_read_t<bf16_t, bf16_t>(base, map, pool, H, S, D, T, width, index, weights, out, rows, st);
}

extern "C" int glsdm_overlay_materialise(const void *base, int32_t dtype, const int32_t *map, const void *pool,
                                         int64_t B, int64_t H, int64_t S, int64_t D, void *out, void *stream)
{
    if (B < 0 || H < 1 || S < 1 || D < 1) return fail(GLSDM_ERR_ARG, "overlay_materialise: bad shape");
    if (!dtype_ok(dtype)) return fail(GLSDM_ERR_ARG, "overlay_materialise: bad dtype");
    const int64_t total = B * H * S * D;
    if (total == 0) return GLSDM_OK;
    if (!base || !map || !pool || !out) return fail(GLSDM_ERR_ARG, "overlay_materialise: null pointer");
    const unsigned blocks = (unsigned)std::min<int64_t>(ceil_div(total, 256), 65536);
    const hipStream_t st = as_stream(stream);
    if (dtype == GLSDM_F32)
        hipLaunchKernelGGL(overlay_materialise_kernel<float>, dim3(blocks), dim3(256), 0, st,
                           static_cast<const float *>(base), map, static_cast<const float *>(pool), H * S, D, total,
                           static_cast<float *>(out));
    else
        hipLaunchKernelGGL(overlay_materialise_kernel<bf16_t>, dim3(blocks), dim3(256), 0, st,
                           static_cast<const bf16_t *>(base), map, static_cast<const bf16_t *>(pool), H * S, D,
                           total, static_cast<bf16_t *>(out));
    return check_launch("overlay_materialise_kernel");
}
