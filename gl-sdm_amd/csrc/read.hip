// Snapshot read, row gather and address arithmetic on gfx950.
//
// Read semantics: S/memory/routing.py:27-28 (out = sum_j w_j * row_j, fp32),
// rows addressed as (b*H + h)*S + slot (S/memory/routing.py:31-34).
//
// Layout: one wavefront per output row (b, t, h).  A bank row of D elements is
// fetched by `lpr` lanes with 16-byte loads (for D = 128 bf16: 16 lanes x 16 B
// = 256 B, two full 128-byte lines), so one wave keeps 64/lpr route entries in
// flight at once; partial sums are combined across those lane groups with
// __shfl_xor and the first group stores the row.  Products are rounded before
// the add (no FMA contraction), as in the reference's rows * w then sum.
#include <type_traits>

#include "glsdm_internal.h"

namespace glsdm {

template <typename TB, typename TO, int VEC, int CH, int U>
__global__ __launch_bounds__(256) void read_kernel(const TB *__restrict__ bank, int64_t H, int64_t S,
                                                   int64_t D, int64_t T, int width,
                                                   const int64_t *__restrict__ index,
                                                   const float *__restrict__ weights,
                                                   TO *__restrict__ out, int64_t rows, int nv, int lpr)
{
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;  // wave-uniform
    const int ng = 64 / lpr;
    const int grp = lane / lpr;
    const int li = lane % lpr;
    const int64_t b = r / (T * H);
    const int64_t h = r % H;
    const TB *base = bank + (b * H + h) * S * D;
    const int64_t *ix = index + r * width;
    const float *wt = weights + r * width;

    float acc[CH][VEC];
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[c][e] = 0.0f;

    // U route entries per lane group at a time: their slots and weights are loaded
    // first, then all U row loads are issued before any is used (an out-of-range
    // slot reads row 0 and adds nothing), so a wave keeps U rows per group in flight
    // instead of waiting on each slot before its row.  The entries are still added in
    // the order j = grp, grp + ng, ...: the same bits for every U.
    for (int j0 = grp; j0 < width; j0 += U * ng) {
        int64_t slot[U];
        float w[U];
        bool ok[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = j0 + u * ng;
            const bool in = j < width;
            const int jj = in ? j : width - 1;             // a valid position: loads stay unconditional
            slot[u] = ix[jj];
            w[u] = wt[jj];
            ok[u] = in && slot[u] >= 0 && slot[u] < S;
        }
        // lanes past the row's last piece load its last piece again (unconditional
        // loads, no branch between them) and never store what they sum
        constexpr bool RAW = VEC * sizeof(TB) == 16 && std::is_same<TB, bf16_t>::value;
        uint4 raw[U][CH];
        float x[RAW ? 1 : U][CH][VEC];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const TB *row = base + (ok[u] ? slot[u] : 0) * D;
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                const int v = li + c * lpr < nv ? li + c * lpr : nv - 1;
                if constexpr (RAW)
                    raw[u][c] = load16_stream(row + (int64_t)v * VEC);    // random rows: little reuse
                else
                    VecLoad<TB, VEC>::load(row + (int64_t)v * VEC, x[u][c]);
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                float y[VEC];
                if constexpr (RAW) {
                    const uint32_t wd[4] = {raw[u][c].x, raw[u][c].y, raw[u][c].z, raw[u][c].w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        y[2 * i] = __uint_as_float(wd[i] << 16);
                        y[2 * i + 1] = __uint_as_float(wd[i] & 0xFFFF0000u);
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < VEC; ++e) y[e] = x[u][c][e];
                }
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    const float sum = acc[c][e] + y[e] * w[u];
                    acc[c][e] = ok[u] ? sum : acc[c][e];
                }
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

template <typename TB, typename TO, int VEC, int CH>
static void launch_read_u(const TB *bk, int64_t H, int64_t S, int64_t D, int64_t T, int width,
                          const int64_t *index, const float *weights, TO *o, int64_t rows, const RowPlan &p,
                          bool narrow, hipStream_t st)
{
    // wide: several route entries per lane group in flight; narrow: one (at most 32
    // VGPRs for 16-byte pieces, so eight of its waves leave a SIMD room for one wave of
    // the 248-VGPR route kernel when both run at once)
    constexpr int U = CH <= 2 ? 4 : (CH <= 4 ? 2 : 1);
    const dim3 grid((unsigned)ceil_div(rows, 4)), block(256);
    if (narrow || U == 1)
        hipLaunchKernelGGL((read_kernel<TB, TO, VEC, CH, 1>), grid, block, 0, st, bk, H, S, D, T, width, index,
                           weights, o, rows, p.nv, p.lpr);
    else
        hipLaunchKernelGGL((read_kernel<TB, TO, VEC, CH, U>), grid, block, 0, st, bk, H, S, D, T, width, index,
                           weights, o, rows, p.nv, p.lpr);
}

template <typename TB, typename TO, int VEC>
static int launch_read_ch(const void *bank, int64_t H, int64_t S, int64_t D, int64_t T, int width,
                          const int64_t *index, const float *weights, void *out, int64_t rows,
                          const RowPlan &p, bool narrow, hipStream_t st)
{
    const TB *bk = static_cast<const TB *>(bank);
    TO *o = static_cast<TO *>(out);
    switch (p.ch) {
    case 1: launch_read_u<TB, TO, VEC, 1>(bk, H, S, D, T, width, index, weights, o, rows, p, narrow, st); break;
    case 2: launch_read_u<TB, TO, VEC, 2>(bk, H, S, D, T, width, index, weights, o, rows, p, narrow, st); break;
    case 3:
    case 4: launch_read_u<TB, TO, VEC, 4>(bk, H, S, D, T, width, index, weights, o, rows, p, narrow, st); break;
    default: launch_read_u<TB, TO, VEC, 8>(bk, H, S, D, T, width, index, weights, o, rows, p, narrow, st); break;
    }
    return check_launch("read_kernel");
}

template <typename TB, typename TO>
static int launch_read_t(const void *bank, int64_t H, int64_t S, int64_t D, int64_t T, int width,
                         const int64_t *index, const float *weights, void *out, int64_t rows,
                         bool narrow, hipStream_t st)
{
    constexpr int FULL = 16 / sizeof(TB);
    RowPlan p = row_plan(D, sizeof(TB));
    // 16-byte accesses need 16-byte aligned base pointers (D % FULL == 0 keeps rows aligned).
    const bool aligned = ((reinterpret_cast<uintptr_t>(bank) | reinterpret_cast<uintptr_t>(out)) & 15) == 0;
    if (p.vec == FULL && aligned)
        return launch_read_ch<TB, TO, FULL>(bank, H, S, D, T, width, index, weights, out, rows, p, narrow, st);
    p = RowPlan{1, (int)D, D < 64 ? pow2_ceil(D) : 64, (int)ceil_div(D, 64)};
    return launch_read_ch<TB, TO, 1>(bank, H, S, D, T, width, index, weights, out, rows, p, narrow, st);
}

int read_launch(const void *bank, int32_t bank_dtype, int64_t B, int64_t H, int64_t S, int64_t D,
                int64_t T, int32_t width, const int64_t *index, const float *weights, void *out,
                int32_t out_dtype, hipStream_t st, bool narrow)
{
    if (B < 0 || H < 1 || S < 1 || D < 1 || T < 0 || width < 1)
        return fail(GLSDM_ERR_ARG, "read: bad shape B=%lld H=%lld S=%lld D=%lld T=%lld width=%d",
                    (long long)B, (long long)H, (long long)S, (long long)D, (long long)T, width);
    if (!dtype_ok(bank_dtype) || !dtype_ok(out_dtype)) return fail(GLSDM_ERR_ARG, "read: bad dtype");
    if (width > 1024) return fail(GLSDM_ERR_UNSUPPORTED, "read: width > 1024");
    const int64_t rows = B * T * H;
    if (rows == 0) return GLSDM_OK;
    const int64_t max_d = (D % (int64_t)(16 / dtype_size(bank_dtype)) == 0) ? 64 * 8 * (16 / (int64_t)dtype_size(bank_dtype)) : 512;
    if (D > max_d) return fail(GLSDM_ERR_UNSUPPORTED, "read: D=%lld above %lld", (long long)D, (long long)max_d);
    if (!bank || !index || !weights || !out) return fail(GLSDM_ERR_ARG, "read: null pointer");
    if (bank_dtype == GLSDM_F32 && out_dtype == GLSDM_F32)
        return launch_read_t<float, float>(bank, H, S, D, T, width, index, weights, out, rows, narrow, st);
    if (bank_dtype == GLSDM_BF16 && out_dtype == GLSDM_F32)
        return launch_read_t<bf16_t, float>(bank, H, S, D, T, width, index, weights, out, rows, narrow, st);
    if (bank_dtype == GLSDM_F32 && out_dtype == GLSDM_BF16)
        return launch_read_t<float, bf16_t>(bank, H, S, D, T, width, index, weights, out, rows, narrow, st);
    return launch_read_t<bf16_t, bf16_t>(bank, H, S, D, T, width, index, weights, out, rows, narrow, st);
}

// ------------------------------------------------------------ gather / addresses

template <typename T>
__global__ __launch_bounds__(256) void gather_kernel(const T *__restrict__ bank, int64_t rows, int64_t D,
                                                     const int64_t *__restrict__ addresses, int64_t n,
                                                     T *__restrict__ out)
{
    const int64_t total = n * D;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t k = i / D, d = i - k * D;
        const int64_t a = addresses[k];
        out[i] = (a >= 0 && a < rows) ? bank[a * D + d] : T(0);
    }
}

__global__ __launch_bounds__(256) void address_kernel(const int64_t *__restrict__ index, int64_t T,
                                                      int64_t H, int width, int64_t S, int64_t n,
                                                      int64_t *__restrict__ out)
{
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / width;         // (b*T + t)*H + h
        const int64_t h = r % H, b = r / (T * H);
        out[i] = (b * H + h) * S + index[i];
    }
}

}  // namespace glsdm

using namespace glsdm;

extern "C" int glsdm_read(const void *bank, int32_t bank_dtype, int64_t B, int64_t H, int64_t S,
                          int64_t D, int64_t T, int32_t width, const int64_t *index,
                          const float *weights, void *out, int32_t out_dtype, void *stream)
{
    return read_launch(bank, bank_dtype, B, H, S, D, T, width, index, weights, out, out_dtype,
                       as_stream(stream), false);
}

extern "C" int glsdm_read_narrow(const void *bank, int32_t bank_dtype, int64_t B, int64_t H, int64_t S,
                                 int64_t D, int64_t T, int32_t width, const int64_t *index,
                                 const float *weights, void *out, int32_t out_dtype, void *stream)
{
    return read_launch(bank, bank_dtype, B, H, S, D, T, width, index, weights, out, out_dtype,
                       as_stream(stream), true);
}

namespace glsdm {
int route_launch(const void *scores, int32_t scores_dtype, int64_t rows, int half, int width, int tie,
                 void *workspace, size_t workspace_bytes, int64_t *index, float *weights, hipStream_t st);
}

extern "C" int glsdm_route_read(const void *bank, int32_t bank_dtype, int64_t B, int64_t H, int64_t S,
                                int64_t D, int64_t T, const void *scores, int32_t scores_dtype, int32_t width,
                                int32_t tie, void *out, int32_t out_dtype, int64_t *index, float *weights,
                                void *workspace, size_t workspace_bytes, void *stream)
{
    if (S < 1) return fail(GLSDM_ERR_ARG, "route_read: S must be >= 1");
    int64_t half = 1;
    while (half * half < S) ++half;
    if (half * half != S) return fail(GLSDM_ERR_ARG, "route_read: slots S=%lld is not a square", (long long)S);
    const hipStream_t st = as_stream(stream);
    int rc = glsdm::route_launch(scores, scores_dtype, B * T * H, (int)half, width, tie, workspace,
                                 workspace_bytes, index, weights, st);
    if (rc != GLSDM_OK) return rc;
    return read_launch(bank, bank_dtype, B, H, S, D, T, width, index, weights, out, out_dtype, st, false);
}

extern "C" int glsdm_gather_rows(const void *bank, int32_t bank_dtype, int64_t rows, int64_t D,
                                 const int64_t *addresses, int64_t n, void *out, void *stream)
{
    if (rows < 1 || D < 1 || n < 0) return fail(GLSDM_ERR_ARG, "gather_rows: bad shape");
    if (!dtype_ok(bank_dtype)) return fail(GLSDM_ERR_ARG, "gather_rows: bad dtype");
    if (n == 0) return GLSDM_OK;
    if (!bank || !addresses || !out) return fail(GLSDM_ERR_ARG, "gather_rows: null pointer");
    const int64_t blocks = std::min<int64_t>(ceil_div(n * D, 256), 65536);
    if (bank_dtype == GLSDM_F32)
        hipLaunchKernelGGL(gather_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                           static_cast<const float *>(bank), rows, D, addresses, n, static_cast<float *>(out));
    else
        hipLaunchKernelGGL(gather_kernel<bf16_t>, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                           static_cast<const bf16_t *>(bank), rows, D, addresses, n, static_cast<bf16_t *>(out));
    return check_launch("gather_kernel");
}

extern "C" int glsdm_absolute_addresses(const int64_t *index, int64_t B, int64_t T, int64_t H,
                                        int32_t width, int64_t S, int64_t *out, void *stream)
{
    if (B < 0 || T < 0 || H < 1 || width < 1 || S < 1) return fail(GLSDM_ERR_ARG, "absolute_addresses: bad shape");
    const int64_t n = B * T * H * width;
    if (n == 0) return GLSDM_OK;
    if (!index || !out) return fail(GLSDM_ERR_ARG, "absolute_addresses: null pointer");
    const int64_t blocks = std::min<int64_t>(ceil_div(n, 256), 65536);
    hipLaunchKernelGGL(address_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), index, T, H,
                       width, S, n, out);
    return check_launch("address_kernel");
}

namespace glsdm {

// addresses = (b*H + h)*S + slot and keys = address*(chunk*layers) + (offset + t)*layers + layer
// for a proposal index [B, T, H, width] (S/layers/global_layer.py:45,52-53).
__global__ __launch_bounds__(256) void proposal_keys_kernel(const int64_t *__restrict__ index, int64_t T,
                                                            int64_t H, int width, int64_t S,
                                                            int64_t offset, int64_t scale, int64_t layers,
                                                            int64_t layer, int64_t n,
                                                            int64_t *__restrict__ addresses,
                                                            int64_t *__restrict__ keys)
{
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / width;         // (b*T + t)*H + h
        const int64_t h = r % H, bt = r / H;
        const int64_t t = bt % T, b = bt / T;
        const int64_t a = (b * H + h) * S + index[i];
        addresses[i] = a;
        keys[i] = a * scale + (offset + t) * layers + layer;
    }
}

}  // namespace glsdm

extern "C" int glsdm_proposal_keys(const int64_t *index, int64_t B, int64_t T, int64_t H, int32_t width,
                                   int64_t S, int64_t position_offset, int64_t chunk, int64_t layers,
                                   int64_t layer, int64_t *addresses, int64_t *keys, void *stream)
{
    if (B < 0 || T < 0 || H < 1 || width < 1 || S < 1 || chunk < 1 || layers < 1 || layer < 0 ||
        layer >= layers || position_offset < 0)
        return fail(GLSDM_ERR_ARG, "proposal_keys: bad arguments");
    const int64_t n = B * T * H * width;
    if (n == 0) return GLSDM_OK;
    if (!index || !addresses || !keys) return fail(GLSDM_ERR_ARG, "proposal_keys: null pointer");
    const int64_t blocks = std::min<int64_t>(ceil_div(n, 256), 65536);
    hipLaunchKernelGGL(proposal_keys_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), index,
                       T, H, width, S, position_offset, chunk * layers, layers, layer, n, addresses, keys);
    return check_launch("proposal_keys_kernel");
}
