// Write-proposal arithmetic on gfx950.
//
// Semantics (S/ = projects/gl-sdm/src/gl_sdm/): S/runtime/dense.py:11-14
//     decay = exp(log_decay)
//     error = beta * (target - decay * prediction)
//     delta = mass * ((decay - 1) * rows + weights * error)
// per proposal row r = (leading index) * heads + h, with rows/weights holding
// `width` selected bank rows per r and mass one value per leading index.
// Every product and sum is a separate fp32 operation in that order (FMA
// contraction is off), so the bits match the reference's eager torch ops for
// the same decay values.
//
// Two kernels, both one wavefront per proposal row with 16-byte accesses:
//   proposal_error_kernel  decay[r] and the error row (the per-row terms the
//                          fused commit consumes; the deltas are never stored)
//   proposal_delta_kernel  the materialised deltas [R, width, D] from given
//                          rows, the drop-in for dense.py's proposal_delta;
//                          the error row is formed once in registers and
//                          reused for the `width` rows.
#include "glsdm_internal.h"

namespace glsdm {

template <typename TT, int VEC, int CH>
__global__ __launch_bounds__(256) void proposal_error_kernel(int64_t R, int64_t D, int nv,
                                                             const float *__restrict__ prediction,
                                                             const TT *__restrict__ target,
                                                             const float *__restrict__ beta,
                                                             const float *__restrict__ log_decay,
                                                             float *__restrict__ error, float *__restrict__ decay)
{
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= R) return;   // wave-uniform
    const float g = expf(log_decay[r]);
    const float bet = beta[r];
    if (lane == 0) decay[r] = g;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int v = lane + c * 64;
        if (v < nv) {
            float tg[VEC], pr[VEC], er[VEC];
            VecLoad<TT, VEC>::load(target + r * D + (int64_t)v * VEC, tg);
            VecLoad<float, VEC>::load(prediction + r * D + (int64_t)v * VEC, pr);
#pragma unroll
            for (int x = 0; x < VEC; ++x) {
                const float gp = g * pr[x];
                const float diff = tg[x] - gp;
                er[x] = bet * diff;
            }
            VecStore<float, VEC>::store(error + r * D + (int64_t)v * VEC, er);
        }
    }
}

// The proposal log's append step, the inference path of a global layer's write
// proposal (S/layers/global_layer.py:33-54 after its write route): one
// wavefront per proposal row r = (b*T + t)*H + h writes, at the log's fill,
//   decay[r] = exp(log_decay), the error row beta * (target - decay * prediction)
// with beta and log_decay the write gates of the beta/decay projections'
// outputs (write_gate_values), and for each of its `width` picks the absolute
// address (b*H + h)*S + slot, the collision key addr*(C*L) + (offset + t)*L +
// layer and the route weight.  Bit for bit what write_gates, proposal_keys and
// proposal_error produce one after another.
template <typename TT, typename TG, int VEC, int CH>
__global__ __launch_bounds__(256) void proposal_append_kernel(
    int64_t R, int64_t T, int64_t H, int width, int64_t S, int64_t D, int nv, int64_t offset, int64_t scale,
    int64_t layers, int64_t layer, const int64_t *__restrict__ index, const float *__restrict__ weights,
    const float *__restrict__ prediction, const TT *__restrict__ target, const TG *__restrict__ b_in,
    const TG *__restrict__ d_in, int64_t *__restrict__ addresses, int64_t *__restrict__ keys,
    float *__restrict__ weights_out, float *__restrict__ error, float *__restrict__ decay)
{
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= R) return;   // wave-uniform
    float bv[1], dv[1], bet, ld;
    VecLoad<TG, 1>::load(b_in + r, bv);
    VecLoad<TG, 1>::load(d_in + r, dv);
    write_gate_values(bv[0], dv[0], bet, ld);
    const float g = expf(ld);
    if (lane == 0) decay[r] = g;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int v = lane + c * 64;
        if (v < nv) {
            float tg[VEC], pr[VEC], er[VEC];
            VecLoad<TT, VEC>::load(target + r * D + (int64_t)v * VEC, tg);
            VecLoad<float, VEC>::load(prediction + r * D + (int64_t)v * VEC, pr);
#pragma unroll
            for (int x = 0; x < VEC; ++x) {
                const float gp = g * pr[x];
                const float diff = tg[x] - gp;
                er[x] = bet * diff;
            }
            VecStore<float, VEC>::store(error + r * D + (int64_t)v * VEC, er);
        }
    }
    const int64_t h = r % H, bt = r / H;
    const int64_t t = bt % T, b = bt / T;
    const int64_t row0 = (b * H + h) * S;
    for (int j = lane; j < width; j += 64) {
        const int64_t i = r * width + j;
        const int64_t a = row0 + index[i];
        addresses[i] = a;
        keys[i] = a * scale + (offset + t) * layers + layer;
        weights_out[i] = weights[i];
    }
}

template <typename TR, typename TT, int VEC, int CH>
__global__ __launch_bounds__(256) void proposal_delta_kernel(
    int64_t R, int width, int64_t D, int nv, const TR *__restrict__ rows, const float *__restrict__ weights,
    const float *__restrict__ prediction, const TT *__restrict__ target, const float *__restrict__ beta,
    const float *__restrict__ log_decay, const float *__restrict__ mass, int64_t heads,
    float *__restrict__ deltas)
{
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= R) return;   // wave-uniform
    const float g = expf(log_decay[r]);
    const float gm1 = g - 1.0f;
    const float bet = beta[r];
    const float m = mass[r / heads];
    float err[CH][VEC];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int v = lane + c * 64;
        if (v < nv) {
            float tg[VEC], pr[VEC];
            VecLoad<TT, VEC>::load(target + r * D + (int64_t)v * VEC, tg);
            VecLoad<float, VEC>::load(prediction + r * D + (int64_t)v * VEC, pr);
#pragma unroll
            for (int x = 0; x < VEC; ++x) {
                const float gp = g * pr[x];
                const float diff = tg[x] - gp;
                err[c][x] = bet * diff;
            }
        }
    }
    for (int j = 0; j < width; ++j) {
        const int64_t e = r * width + j;
        const float w = weights[e];
        const TR *src = rows + e * D;
        float *out = deltas + e * D;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int v = lane + c * 64;
            if (v < nv) {
                float row[VEC], dl[VEC];
                VecLoad<TR, VEC>::load(src + (int64_t)v * VEC, row);
#pragma unroll
                for (int x = 0; x < VEC; ++x) {
                    const float a = gm1 * row[x];
                    const float b = w * err[c][x];
                    const float s = a + b;
                    dl[x] = m * s;
                }
                VecStore<float, VEC>::store(out + (int64_t)v * VEC, dl);
            }
        }
    }
}

// Per-row accesses: 16 bytes of fp32 (VEC = 4) when D and every row pointer
// allow it, else scalar; up to 8 accesses per lane (D <= 2048).
struct ProposalPlan {
    int vec, nv, ch;
};

static ProposalPlan proposal_plan(int64_t D, uintptr_t pointer_bits)
{
    ProposalPlan p;
    p.vec = (D % 4 == 0 && (pointer_bits & 15) == 0) ? 4 : 1;
    p.nv = (int)(D / p.vec);
    p.ch = (int)ceil_div(p.nv, 64);
    if (p.ch > 2) p.ch = p.ch <= 4 ? 4 : 8;
    return p;
}

static uintptr_t bits_of(const void *a, const void *b, const void *c, const void *d = nullptr)
{
    return reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) | reinterpret_cast<uintptr_t>(c) |
           reinterpret_cast<uintptr_t>(d);
}

#define GLSDM_CH_SWITCH(ch, LAUNCH) \
    switch (ch) {                   \
    case 1: LAUNCH(1); break;       \
    case 2: LAUNCH(2); break;       \
    case 4: LAUNCH(4); break;       \
    default: LAUNCH(8); break;      \
    }

template <typename TT, int VEC>
static void launch_error(int64_t R, int64_t D, int nv, int ch, const float *prediction, const void *target,
                         const float *beta, const float *log_decay, float *error, float *decay, hipStream_t st)
{
    const dim3 grid((unsigned)ceil_div(R, 4)), block(256);
    const TT *tg = static_cast<const TT *>(target);
#define GLSDM_ERR_LAUNCH(C)                                                                                  \
    hipLaunchKernelGGL((proposal_error_kernel<TT, VEC, C>), grid, block, 0, st, R, D, nv, prediction, tg, beta, \
                       log_decay, error, decay)
    GLSDM_CH_SWITCH(ch, GLSDM_ERR_LAUNCH)
#undef GLSDM_ERR_LAUNCH
}

struct AppendArgs {
    int64_t R, T, H;
    int width;
    int64_t S, D, offset, scale, layers, layer;
    const int64_t *index;
    const float *weights, *prediction;
    const void *target, *b_in, *d_in;
    int64_t *addresses, *keys;
    float *weights_out, *error, *decay;
};

template <typename TT, typename TG, int VEC>
static void launch_append(const AppendArgs &a, int nv, int ch, hipStream_t st)
{
    const dim3 grid((unsigned)ceil_div(a.R, 4)), block(256);
    const TT *tg = static_cast<const TT *>(a.target);
    const TG *bi = static_cast<const TG *>(a.b_in), *di = static_cast<const TG *>(a.d_in);
#define GLSDM_APPEND_LAUNCH(C)                                                                                 \
    hipLaunchKernelGGL((proposal_append_kernel<TT, TG, VEC, C>), grid, block, 0, st, a.R, a.T, a.H, a.width, a.S, \
                       a.D, nv, a.offset, a.scale, a.layers, a.layer, a.index, a.weights, a.prediction, tg, bi, di,  \
                       a.addresses, a.keys, a.weights_out, a.error, a.decay)
    GLSDM_CH_SWITCH(ch, GLSDM_APPEND_LAUNCH)
#undef GLSDM_APPEND_LAUNCH
}

template <typename TT, typename TG>
static void launch_append_t(const AppendArgs &a, const ProposalPlan &p, hipStream_t st)
{
    if (p.vec == 4) launch_append<TT, TG, 4>(a, p.nv, p.ch, st);
    else launch_append<TT, TG, 1>(a, p.nv, p.ch, st);
}

template <typename TR, typename TT, int VEC>
static void launch_delta(int64_t R, int width, int64_t D, int nv, int ch, const void *rows, const float *weights,
                         const float *prediction, const void *target, const float *beta, const float *log_decay,
                         const float *mass, int64_t heads, float *deltas, hipStream_t st)
{
    const dim3 grid((unsigned)ceil_div(R, 4)), block(256);
    const TR *rw = static_cast<const TR *>(rows);
    const TT *tg = static_cast<const TT *>(target);
#define GLSDM_DELTA_LAUNCH(C)                                                                                  \
    hipLaunchKernelGGL((proposal_delta_kernel<TR, TT, VEC, C>), grid, block, 0, st, R, width, D, nv, rw, weights, \
                       prediction, tg, beta, log_decay, mass, heads, deltas)
    GLSDM_CH_SWITCH(ch, GLSDM_DELTA_LAUNCH)
#undef GLSDM_DELTA_LAUNCH
}

template <typename TR, typename TT>
static void launch_delta_t(const ProposalPlan &p, int64_t R, int width, int64_t D, const void *rows,
                           const float *weights, const float *prediction, const void *target, const float *beta,
                           const float *log_decay, const float *mass, int64_t heads, float *deltas, hipStream_t st)
{
    if (p.vec == 4)
        launch_delta<TR, TT, 4>(R, width, D, p.nv, p.ch, rows, weights, prediction, target, beta, log_decay, mass,
                                heads, deltas, st);
    else
        launch_delta<TR, TT, 1>(R, width, D, p.nv, p.ch, rows, weights, prediction, target, beta, log_decay, mass,
                                heads, deltas, st);
}

static int check_proposal_shape(const char *what, int64_t R, int64_t D)
{
    if (R < 0 || D < 1) return fail(GLSDM_ERR_ARG, "%s: bad shape R=%lld D=%lld", what, (long long)R, (long long)D);
    if (D > 2048) return fail(GLSDM_ERR_UNSUPPORTED, "%s: D=%lld above 2048", what, (long long)D);
    if (D % 4 != 0 && D > 512)
        return fail(GLSDM_ERR_UNSUPPORTED, "%s: D=%lld not a multiple of 4 above 512", what, (long long)D);
    if (ceil_div(R, 4) > (int64_t)UINT32_MAX) return fail(GLSDM_ERR_UNSUPPORTED, "%s: too many proposal rows", what);
    return GLSDM_OK;
}

}  // namespace glsdm

using namespace glsdm;

extern "C" int glsdm_proposal_error(int64_t R, int64_t D, const float *prediction, const void *target,
                                    int32_t target_dtype, const float *beta, const float *log_decay,
                                    float *error, float *decay, void *stream)
{
    int rc = check_proposal_shape("proposal_error", R, D);
    if (rc) return rc;
    if (!dtype_ok(target_dtype)) return fail(GLSDM_ERR_ARG, "proposal_error: bad dtype");
    if (R == 0) return GLSDM_OK;
    if (!prediction || !target || !beta || !log_decay || !error || !decay)
        return fail(GLSDM_ERR_ARG, "proposal_error: null pointer");
    const ProposalPlan p = proposal_plan(D, bits_of(prediction, target, error));
    const hipStream_t st = as_stream(stream);
    if (target_dtype == GLSDM_F32) {
        if (p.vec == 4) launch_error<float, 4>(R, D, p.nv, p.ch, prediction, target, beta, log_decay, error, decay, st);
        else launch_error<float, 1>(R, D, p.nv, p.ch, prediction, target, beta, log_decay, error, decay, st);
    } else {
        if (p.vec == 4) launch_error<bf16_t, 4>(R, D, p.nv, p.ch, prediction, target, beta, log_decay, error, decay, st);
        else launch_error<bf16_t, 1>(R, D, p.nv, p.ch, prediction, target, beta, log_decay, error, decay, st);
    }
    return check_launch("proposal_error_kernel");
}

extern "C" int glsdm_proposal_append(const int64_t *index, const float *weights, const float *prediction,
                                     const void *target, int32_t target_dtype, const void *beta_in,
                                     const void *decay_in, int32_t gate_dtype, int64_t B, int64_t T, int64_t H,
                                     int32_t width, int64_t S, int64_t D, int64_t position_offset, int64_t chunk,
                                     int64_t layers, int64_t layer, int64_t *addresses, int64_t *keys,
                                     float *weights_out, float *error, float *decay, void *stream)
{
    if (B < 0 || T < 0 || H < 1 || width < 1 || S < 1 || chunk < 1 || layers < 1 || layer < 0 ||
        layer >= layers || position_offset < 0)
        return fail(GLSDM_ERR_ARG, "proposal_append: bad arguments");
    const int64_t R = B * T * H;
    int rc = check_proposal_shape("proposal_append", R, D);
    if (rc) return rc;
    if (!dtype_ok(target_dtype) || !dtype_ok(gate_dtype)) return fail(GLSDM_ERR_ARG, "proposal_append: bad dtype");
    if (R == 0) return GLSDM_OK;
    if (!index || !weights || !prediction || !target || !beta_in || !decay_in || !addresses || !keys ||
        !weights_out || !error || !decay)
        return fail(GLSDM_ERR_ARG, "proposal_append: null pointer");
    const AppendArgs a{R, T, H, width, S, D, position_offset, chunk * layers, layers, layer, index, weights,
                       prediction, target, beta_in, decay_in, addresses, keys, weights_out, error, decay};
    const ProposalPlan p = proposal_plan(D, bits_of(prediction, target, error));
    const hipStream_t st = as_stream(stream);
    if (target_dtype == GLSDM_F32 && gate_dtype == GLSDM_F32) launch_append_t<float, float>(a, p, st);
    else if (target_dtype == GLSDM_F32) launch_append_t<float, bf16_t>(a, p, st);
    else if (gate_dtype == GLSDM_F32) launch_append_t<bf16_t, float>(a, p, st);
    else launch_append_t<bf16_t, bf16_t>(a, p, st);
    return check_launch("proposal_append_kernel");
}

extern "C" int glsdm_proposal_delta(const void *rows, int32_t rows_dtype, int64_t R, int32_t width, int64_t D,
                                    const float *weights, const float *prediction, const void *target,
                                    int32_t target_dtype, const float *beta, const float *log_decay,
                                    const float *mass, int64_t heads, float *deltas, void *stream)
{
    int rc = check_proposal_shape("proposal_delta", R, D);
    if (rc) return rc;
    if (width < 1 || heads < 1 || R % heads != 0)
        return fail(GLSDM_ERR_ARG, "proposal_delta: bad width=%d or heads=%lld", (int)width, (long long)heads);
    if (!dtype_ok(rows_dtype) || !dtype_ok(target_dtype)) return fail(GLSDM_ERR_ARG, "proposal_delta: bad dtype");
    if (R == 0) return GLSDM_OK;
    if (!rows || !weights || !prediction || !target || !beta || !log_decay || !mass || !deltas)
        return fail(GLSDM_ERR_ARG, "proposal_delta: null pointer");
    const ProposalPlan p = proposal_plan(D, bits_of(rows, prediction, target, deltas));
    const hipStream_t st = as_stream(stream);
    if (rows_dtype == GLSDM_F32 && target_dtype == GLSDM_F32)
        launch_delta_t<float, float>(p, R, width, D, rows, weights, prediction, target, beta, log_decay, mass, heads,
                                     deltas, st);
    else if (rows_dtype == GLSDM_F32)
        launch_delta_t<float, bf16_t>(p, R, width, D, rows, weights, prediction, target, beta, log_decay, mass,
                                      heads, deltas, st);
    else if (target_dtype == GLSDM_F32)
        launch_delta_t<bf16_t, float>(p, R, width, D, rows, weights, prediction, target, beta, log_decay, mass,
                                      heads, deltas, st);
    else
        launch_delta_t<bf16_t, bf16_t>(p, R, width, D, rows, weights, prediction, target, beta, log_decay, mass,
                                       heads, deltas, st);
    return check_launch("proposal_delta_kernel");
}
