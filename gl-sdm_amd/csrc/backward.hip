// Backward of the route and of the snapshot read on gfx950.
//
// Semantics (S/ = projects/gl-sdm/src/gl_sdm/):
//   route  S/memory/backends/token.py:69-82 (_route_backward) and the autograd
//          of S/memory/routing.py:10-26: per row, the softmax backward
//              g_j = w_j * (gw_j - sum_v w_v gw_v)
//          of the chosen slots' weights, and every pick's g_j credited to the
//          two factor sub-keys its slot is made of (slot / half, slot % half);
//          the factor-score gradient [rows, 2*half] is zero elsewhere.
//   read   the autograd of S/memory/routing.py:27-28 (out = sum_j w_j row_j):
//              grad_w[r, j] = <grad_out[r], row_j>
//          (the rows' own gradient, w_j * grad_out[r] accumulated per bank
//          row, is glsdm_read_backward_rows in commit.hip).
// Sums run in a fixed order (picks in list order; lane partials then a fixed
// butterfly), so results are deterministic; they match the reference within
// fp32 rounding of a different summation order.
#include "glsdm_internal.h"

namespace glsdm {

// Sum over the 64 lanes of a wavefront by a fixed butterfly.
__device__ __forceinline__ float wave_sum(float x)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
    return x;
}

// One wavefront per route row.
template <bool QUAD>
__global__ __launch_bounds__(256) void route_backward_kernel(const int64_t *__restrict__ index,
                                                             const float *__restrict__ weights,
                                                             const float *__restrict__ grad_weights, int64_t rows,
                                                             int half, int width, float *__restrict__ grad_scores)
{
#pragma clang fp contract(off)
    __shared__ int32_t s_sub[4][2][64];   // each pick's sub-key per factor (-1: no pick)
    __shared__ float s_g[4][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t r = (int64_t)blockIdx.x * 4 + wave;
    if (r >= rows) return;   // wave-uniform; no block barrier below
    // lane j < width holds pick j; the dot product sum_v w_v gw_v by butterfly
    float w = 0.0f, gw = 0.0f;
    int32_t i0 = -1, i1 = -1;
    if (lane < width) {
        w = weights[r * width + lane];
        gw = grad_weights[r * width + lane];
        const int64_t slot = index[r * width + lane];
        if (slot >= 0 && slot < (int64_t)half * half) {
            i0 = (int32_t)(slot / half);
            i1 = (int32_t)(slot - (int64_t)i0 * half);
        }
    }
    const float dot = wave_sum(w * gw);
    s_g[wave][lane] = lane < width ? w * (gw - dot) : 0.0f;
    s_sub[wave][0][lane] = i0;
    s_sub[wave][1][lane] = i1;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // column c of factor f gets the picks whose sub-key of factor f is c, in pick order
    float *out = grad_scores + r * 2 * (int64_t)half;
    if (QUAD) {
        // four adjacent columns per lane (one factor: half % 4 == 0), one 16-byte store
        for (int c = 4 * lane; c < 2 * half; c += 256) {
            const int f = c >= half ? 1 : 0, sub = f ? c - half : c;
            float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            for (int j = 0; j < width; ++j) {
                const int d = s_sub[wave][f][j] - sub;
                const float gj = s_g[wave][j];
#pragma unroll
                for (int x = 0; x < 4; ++x)
                    if (d == x) acc[x] += gj;
            }
            *reinterpret_cast<float4 *>(out + c) = make_float4(acc[0], acc[1], acc[2], acc[3]);
        }
    } else {
        for (int c = lane; c < 2 * half; c += 64) {
            const int f = c >= half ? 1 : 0, sub = f ? c - half : c;
            float acc = 0.0f;
            for (int j = 0; j < width; ++j)
                if (s_sub[wave][f][j] == sub) acc += s_g[wave][j];
            out[c] = acc;
        }
    }
}

// One wavefront per read row: grad_w[r, j] = <grad_out[r], bank[addr(r, j)]>.
// Lane groups of `lpr` lanes (16-byte row pieces) take picks j = grp, grp + ng,
// ...; each group reduces its dot product over its own lanes.
template <typename TB, int VEC, int CH>
__global__ __launch_bounds__(256) void read_backward_weights_kernel(const TB *__restrict__ bank, int64_t H,
                                                                    int64_t S, int64_t D, int64_t T, int width,
                                                                    const int64_t *__restrict__ index,
                                                                    const float *__restrict__ grad_out,
                                                                    float *__restrict__ grad_weights, int64_t rows,
                                                                    int nv, int lpr)
{
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);   // (b*T + t)*H + h
    if (r >= rows) return;   // wave-uniform
    const int ng = 64 / lpr, grp = lane / lpr, li = lane % lpr;
    const int64_t h = r % H, b = r / H / T;
    float go[CH][VEC];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int v = li + c * lpr;
        if (v < nv) VecLoad<float, VEC>::load(grad_out + r * D + (int64_t)v * VEC, go[c]);
    }
    const TB *part = bank + (b * H + h) * S * D;
    // every group runs the same number of rounds, so the shuffles see whole groups
    const int rounds = (width + ng - 1) / ng;
    for (int q = 0; q < rounds; ++q) {
        const int j = q * ng + grp;
        const int64_t slot = j < width ? index[r * width + j] : -1;
        float acc = 0.0f;
        if (slot >= 0 && slot < S) {
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                const int v = li + c * lpr;
                if (v < nv) {
                    float x[VEC];
                    VecLoad<TB, VEC>::load(part + slot * D + (int64_t)v * VEC, x);
#pragma unroll
                    for (int y = 0; y < VEC; ++y) {
                        const float p = go[c][y] * x[y];
                        acc += p;
                    }
                }
            }
        }
        for (int off = lpr >> 1; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
        if (li == 0 && j < width) grad_weights[r * width + j] = acc;
    }
}

template <typename TB, int VEC>
static void launch_rbw(const void *bank, int64_t H, int64_t S, int64_t D, int64_t T, int width,
                       const int64_t *index, const float *grad_out, float *grad_weights, int64_t rows,
                       const RowPlan &p, hipStream_t st)
{
    const dim3 grid((unsigned)ceil_div(rows, 4)), block(256);
    const TB *bk = static_cast<const TB *>(bank);
#define GLSDM_RBW(C)                                                                                        \
    hipLaunchKernelGGL((read_backward_weights_kernel<TB, VEC, C>), grid, block, 0, st, bk, H, S, D, T, width, \
                       index, grad_out, grad_weights, rows, p.nv, p.lpr)
    switch (p.ch) {
    case 1: GLSDM_RBW(1); break;
    case 2: GLSDM_RBW(2); break;
    case 3:
    case 4: GLSDM_RBW(4); break;
    default: GLSDM_RBW(8); break;
    }
#undef GLSDM_RBW
}

}  // namespace glsdm

using namespace glsdm;

extern "C" int glsdm_route_backward(const int64_t *index, const float *weights, const float *grad_weights,
                                    int64_t rows, int32_t half, int32_t width, float *grad_scores, void *stream)
{
    if (rows < 0 || half < 1 || width < 1) return fail(GLSDM_ERR_ARG, "route_backward: bad shape");
    if (width > 64) return fail(GLSDM_ERR_UNSUPPORTED, "route_backward: width must be in [1, 64]");
    if (half > 65535) return fail(GLSDM_ERR_UNSUPPORTED, "route_backward: half must be in [1, 65535]");
    if (rows == 0) return GLSDM_OK;
    if (!index || !weights || !grad_weights || !grad_scores) return fail(GLSDM_ERR_ARG, "route_backward: null pointer");
    if (ceil_div(rows, 4) > (int64_t)UINT32_MAX) return fail(GLSDM_ERR_UNSUPPORTED, "route_backward: too many rows");
    const dim3 grid((unsigned)ceil_div(rows, 4)), block(256);
    if (half % 4 == 0 && (reinterpret_cast<uintptr_t>(grad_scores) & 15) == 0)
        hipLaunchKernelGGL(route_backward_kernel<true>, grid, block, 0, as_stream(stream), index, weights,
                           grad_weights, rows, half, width, grad_scores);
    else
        hipLaunchKernelGGL(route_backward_kernel<false>, grid, block, 0, as_stream(stream), index, weights,
                           grad_weights, rows, half, width, grad_scores);
    return check_launch("route_backward_kernel");
}

extern "C" int glsdm_read_backward_weights(const void *bank, int32_t bank_dtype, int64_t B, int64_t H, int64_t S,
                                           int64_t D, int64_t T, int32_t width, const int64_t *index,
                                           const float *grad_out, float *grad_weights, void *stream)
{
    if (B < 0 || H < 1 || S < 1 || D < 1 || T < 0 || width < 1)
        return fail(GLSDM_ERR_ARG, "read_backward_weights: bad shape");
    if (!dtype_ok(bank_dtype)) return fail(GLSDM_ERR_ARG, "read_backward_weights: bad dtype");
    if (D > 2048 || (D % 4 != 0 && D > 512))
        return fail(GLSDM_ERR_UNSUPPORTED, "read_backward_weights: D=%lld", (long long)D);
    const int64_t rows = B * T * H;
    if (rows == 0) return GLSDM_OK;
    if (!bank || !index || !grad_out || !grad_weights) return fail(GLSDM_ERR_ARG, "read_backward_weights: null pointer");
    if (ceil_div(rows, 4) > (int64_t)UINT32_MAX) return fail(GLSDM_ERR_UNSUPPORTED, "read_backward_weights: too many rows");
    const bool aligned = ((reinterpret_cast<uintptr_t>(bank) | reinterpret_cast<uintptr_t>(grad_out)) & 15) == 0;
    const hipStream_t st = as_stream(stream);
    // 16-byte pieces of the bank row (8 bf16 or 4 fp32 per lane), else scalar
    const RowPlan p = row_plan(D, dtype_size(bank_dtype));
    const bool vector = p.vec > 1 && aligned;
    if (!vector && D > 512)
        return fail(GLSDM_ERR_UNSUPPORTED, "read_backward_weights: D=%lld needs 16-byte rows above 512", (long long)D);
    if (bank_dtype == GLSDM_F32) {
        if (vector) launch_rbw<float, 4>(bank, H, S, D, T, width, index, grad_out, grad_weights, rows, p, st);
        else launch_rbw<float, 1>(bank, H, S, D, T, width, index, grad_out, grad_weights, rows, row_plan(D, 16), st);
    } else {
        if (vector) launch_rbw<bf16_t, 8>(bank, H, S, D, T, width, index, grad_out, grad_weights, rows, p, st);
        else launch_rbw<bf16_t, 1>(bank, H, S, D, T, width, index, grad_out, grad_weights, rows, row_plan(D, 16), st);
    }
    return check_launch("read_backward_weights_kernel");
}
