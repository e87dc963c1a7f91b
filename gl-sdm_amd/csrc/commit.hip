// Deterministic buffered commit on gfx950.
//
// Semantics (S/ = projects/gl-sdm/src/gl_sdm/): S/memory/transactions.py:89-96
// and S/memory/backends/commit.py:22-33 -- stable sort of the entries by key,
// then, for each run of equal addresses, an fp32 sum from 0 in sorted order,
// then old + sum.  No float atomics anywhere, so the result is bitwise
// reproducible.
//
// Pipeline (all stream-ordered, no host sync):
//   1. pack:    v[e] = (key[e] - key_min) << ebits | e, ebits = bits of E-1.
//               Ordering the packed words orders by (key, entry) -- a stable
//               key sort -- and the entry id rides along for free.
//   2. radix:   LSD radix sort of the packed words over bits [ebits, ebits +
//               key_bits) in 8-bit digits.  Each pass is histogram -> one-block
//               exclusive scan -> stable scatter.  The entry bits below ebits
//               are never sorted: they start in ascending order and every pass
//               is stable.  Stable in-tile ranking uses wavefront ballots
//               (match-any over the 8 digit bits) and per-wave LDS counters.
//   3. segment: one lane group per sorted position; the first position of each
//               address run walks the run in order, accumulating the deltas in
//               fp32 registers, then read-modify-writes the bank row once.
//               Exactly one group writes each touched row.
#include "glsdm_internal.h"

namespace glsdm {

constexpr int RADIX_BITS = 8;
constexpr int RADIX = 1 << RADIX_BITS;
constexpr int SORT_THREADS = 256;
constexpr int SORT_ITEMS = 8;                           // per thread
constexpr int SORT_TILE = SORT_THREADS * SORT_ITEMS;    // 2048 entries
constexpr int SORT_WAVES = SORT_THREADS / 64;
constexpr int WAVE_ITEMS = SORT_TILE / SORT_WAVES;      // 512 consecutive entries per wave
constexpr int SCAN_THREADS = 1024;

static inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct CommitWorkspace {
    uint64_t *a, *b;
    uint32_t *hist;
    int64_t tiles;
    size_t bytes;
};

static CommitWorkspace plan_workspace(void *base, int64_t entries)
{
    CommitWorkspace w;
    w.tiles = ceil_div(entries, SORT_TILE);
    const size_t words = align256(sizeof(uint64_t) * (size_t)entries);
    const size_t hist = align256(sizeof(uint32_t) * (size_t)RADIX * (size_t)w.tiles);
    char *p = static_cast<char *>(base);
    w.a = reinterpret_cast<uint64_t *>(p);
    w.b = reinterpret_cast<uint64_t *>(p + words);
    w.hist = reinterpret_cast<uint32_t *>(p + 2 * words);
    w.bytes = 2 * words + hist;
    return w;
}

static int entry_bits(int64_t entries)
{
    int b = 1;
    while (b < 63 && ((int64_t)1 << b) < entries) ++b;
    return b;
}

__global__ __launch_bounds__(256) void pack_kernel(const int64_t *__restrict__ keys,
                                                   const int64_t *__restrict__ addresses,
                                                   int64_t key_min, int ebits, int64_t n,
                                                   uint64_t *__restrict__ out)
{
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t k = (keys ? keys[i] : addresses[i]) - key_min;
        out[i] = ((uint64_t)k << ebits) | (uint64_t)i;
    }
}

__global__ __launch_bounds__(SORT_THREADS) void radix_hist_kernel(const uint64_t *__restrict__ in, int64_t n,
                                                                  int shift, uint32_t *__restrict__ hist,
                                                                  int64_t tiles)
{
    __shared__ uint32_t h[RADIX];
    h[threadIdx.x] = 0;
    __syncthreads();
    const int64_t base = (int64_t)blockIdx.x * SORT_TILE;
#pragma unroll
    for (int k = 0; k < SORT_ITEMS; ++k) {
        const int64_t i = base + k * SORT_THREADS + threadIdx.x;
        if (i < n) atomicAdd(&h[(uint32_t)(in[i] >> shift) & (RADIX - 1)], 1u);
    }
    __syncthreads();
    hist[(int64_t)threadIdx.x * tiles + blockIdx.x] = h[threadIdx.x];
}

// Exclusive scan of n counters in place, by one block.
__global__ __launch_bounds__(SCAN_THREADS) void radix_scan_kernel(uint32_t *__restrict__ hist, int64_t n)
{
    __shared__ uint32_t part[SCAN_THREADS];
    const int64_t per = ceil_div(n, SCAN_THREADS);
    const int64_t lo = threadIdx.x * per;
    const int64_t hi = lo + per < n ? lo + per : n;
    uint32_t s = 0;
    for (int64_t i = lo; i < hi; ++i) s += hist[i];
    part[threadIdx.x] = s;
    __syncthreads();
    for (int off = 1; off < SCAN_THREADS; off <<= 1) {   // Hillis-Steele inclusive scan
        const uint32_t x = threadIdx.x >= (unsigned)off ? part[threadIdx.x - off] : 0u;
        __syncthreads();
        part[threadIdx.x] += x;
        __syncthreads();
    }
    uint32_t run = part[threadIdx.x] - s;
    for (int64_t i = lo; i < hi; ++i) {
        const uint32_t c = hist[i];
        hist[i] = run;
        run += c;
    }
}

__global__ __launch_bounds__(SORT_THREADS) void radix_scatter_kernel(const uint64_t *__restrict__ in,
                                                                     uint64_t *__restrict__ out, int64_t n,
                                                                     int shift,
                                                                     const uint32_t *__restrict__ offsets,
                                                                     int64_t tiles)
{
    __shared__ uint32_t cnt[SORT_WAVES][RADIX];
    __shared__ uint32_t tile_base[RADIX];
    const int tid = threadIdx.x;
#pragma unroll
    for (int w = 0; w < SORT_WAVES; ++w) cnt[w][tid] = 0;
    tile_base[tid] = offsets[(int64_t)tid * tiles + blockIdx.x];
    __syncthreads();

    const int wave = tid >> 6, lane = tid & 63;
    const uint64_t lt = (1ull << lane) - 1ull;
    const int64_t start = (int64_t)blockIdx.x * SORT_TILE + (int64_t)wave * WAVE_ITEMS;
    uint64_t v[SORT_ITEMS];
    uint32_t dig[SORT_ITEMS], pos[SORT_ITEMS];
#pragma unroll
    for (int k = 0; k < SORT_ITEMS; ++k) {
        const int64_t i = start + k * 64 + lane;
        const bool valid = i < n;
        v[k] = valid ? in[i] : 0ull;
        const uint32_t d = (uint32_t)(v[k] >> shift) & (RADIX - 1);
        dig[k] = d;
        // lanes of this wave holding the same digit, restricted to valid lanes
        uint64_t peers = __ballot(valid);
#pragma unroll
        for (int bit = 0; bit < RADIX_BITS; ++bit) {
            const bool on = (d >> bit) & 1u;
            const uint64_t m = __ballot(on);
            peers &= on ? m : ~m;
        }
        const uint32_t before = (uint32_t)__popcll(peers & lt);
        uint32_t c = 0;
        if (valid) c = cnt[wave][d];
        pos[k] = c + before;
        if (valid && before == 0) cnt[wave][d] = c + (uint32_t)__popcll(peers);
    }
    __syncthreads();
    {   // exclusive prefix of the per-wave counts, per digit
        uint32_t run = 0;
#pragma unroll
        for (int w = 0; w < SORT_WAVES; ++w) {
            const uint32_t x = cnt[w][tid];
            cnt[w][tid] = run;
            run += x;
        }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < SORT_ITEMS; ++k) {
        const int64_t i = start + k * 64 + lane;
        const int64_t dst = (int64_t)tile_base[dig[k]] + cnt[wave][dig[k]] + pos[k];
        if (i < n && dst < n) out[dst] = v[k];   // dst < n always holds; the guard keeps a bug from faulting
    }
}

template <typename TB, typename TD, int VEC, int CH>
__global__ __launch_bounds__(256) void segment_kernel(TB *__restrict__ bank, int64_t rows, int64_t D,
                                                      const int64_t *__restrict__ addresses,
                                                      const TD *__restrict__ deltas,
                                                      const uint64_t *__restrict__ sorted, int64_t n,
                                                      uint64_t emask, int nv, int lpr,
                                                      int64_t *__restrict__ unique_out)
{
    const int lane = threadIdx.x & 63;
    const int ng = 64 / lpr;
    const int grp = lane / lpr, li = lane % lpr;
    const int64_t p = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * ng + grp;
    if (p >= n) return;
    // entry id -> address; an id outside [0, n) (impossible after a correct sort) reads as -1
    auto addr_at = [&](int64_t q) -> int64_t {
        const int64_t e = (int64_t)(sorted[q] & emask);
        return e < n ? addresses[e] : -1;
    };
    const int64_t a = addr_at(p);
    if (p > 0 && addr_at(p - 1) == a) return;   // not the first of its run
    const bool in_range = a >= 0 && a < rows;

    float acc[CH][VEC];
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[c][e] = 0.0f;
    int64_t q = p;
    do {
        const int64_t ent = (int64_t)(sorted[q] & emask);
        if (in_range && ent < n) {
            const TD *src = deltas + ent * D;
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                const int v = li + c * lpr;
                if (v < nv) {
                    float x[VEC];
                    VecLoad<TD, VEC>::load(src + (int64_t)v * VEC, x);
#pragma unroll
                    for (int e = 0; e < VEC; ++e) acc[c][e] += x[e];
                }
            }
        }
        ++q;
    } while (q < n && addr_at(q) == a);
    if (!in_range) return;

    TB *row = bank + a * D;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int v = li + c * lpr;
        if (v < nv) {
            float old[VEC];
            VecLoad<TB, VEC>::load(row + (int64_t)v * VEC, old);
#pragma unroll
            for (int e = 0; e < VEC; ++e) old[e] = old[e] + acc[c][e];
            VecStore<TB, VEC>::store(row + (int64_t)v * VEC, old);
        }
    }
    if (unique_out && li == 0) atomicAdd(reinterpret_cast<unsigned long long *>(unique_out), 1ull);
}

template <typename TB, typename TD, int VEC>
static int launch_segment_ch(void *bank, int64_t rows, int64_t D, const int64_t *addresses,
                             const void *deltas, const uint64_t *sorted, int64_t n, uint64_t emask,
                             const RowPlan &p, int64_t *unique_out, hipStream_t st)
{
    const int64_t per_block = 4 * (64 / p.lpr);
    const dim3 grid((unsigned)ceil_div(n, per_block)), block(256);
    TB *bk = static_cast<TB *>(bank);
    const TD *dl = static_cast<const TD *>(deltas);
    switch (p.ch) {
    case 1: hipLaunchKernelGGL((segment_kernel<TB, TD, VEC, 1>), grid, block, 0, st, bk, rows, D, addresses, dl, sorted, n, emask, p.nv, p.lpr, unique_out); break;
    case 2: hipLaunchKernelGGL((segment_kernel<TB, TD, VEC, 2>), grid, block, 0, st, bk, rows, D, addresses, dl, sorted, n, emask, p.nv, p.lpr, unique_out); break;
    case 3:
    case 4: hipLaunchKernelGGL((segment_kernel<TB, TD, VEC, 4>), grid, block, 0, st, bk, rows, D, addresses, dl, sorted, n, emask, p.nv, p.lpr, unique_out); break;
    default: hipLaunchKernelGGL((segment_kernel<TB, TD, VEC, 8>), grid, block, 0, st, bk, rows, D, addresses, dl, sorted, n, emask, p.nv, p.lpr, unique_out); break;
    }
    return check_launch("segment_kernel");
}

template <typename TB, typename TD>
static int launch_segment_t(void *bank, int64_t rows, int64_t D, const int64_t *addresses,
                            const void *deltas, const uint64_t *sorted, int64_t n, uint64_t emask,
                            int64_t *unique_out, hipStream_t st)
{
    // One vector width for both operands: the narrower type's 16-byte vector.
    constexpr int VEC = 16 / (sizeof(TB) > sizeof(TD) ? sizeof(TB) : sizeof(TD));
    const bool aligned = ((reinterpret_cast<uintptr_t>(bank) | reinterpret_cast<uintptr_t>(deltas)) & 15) == 0;
    if (D % VEC == 0 && aligned) {
        RowPlan p{VEC, (int)(D / VEC), 0, 0};
        p.lpr = pow2_ceil(p.nv) < 64 ? pow2_ceil(p.nv) : 64;
        p.ch = (int)ceil_div(p.nv, p.lpr);
        return launch_segment_ch<TB, TD, VEC>(bank, rows, D, addresses, deltas, sorted, n, emask, p, unique_out, st);
    }
    RowPlan p{1, (int)D, D < 64 ? pow2_ceil(D) : 64, (int)ceil_div(D, 64)};
    return launch_segment_ch<TB, TD, 1>(bank, rows, D, addresses, deltas, sorted, n, emask, p, unique_out, st);
}

}  // namespace glsdm

using namespace glsdm;

extern "C" int glsdm_commit_workspace_bytes(int64_t entries, int32_t key_bits, size_t *bytes)
{
    if (!bytes) return fail(GLSDM_ERR_ARG, "commit_workspace_bytes: null output");
    if (entries < 0 || key_bits < 0 || key_bits > 63) return fail(GLSDM_ERR_ARG, "commit_workspace_bytes: bad arguments");
    if (entries > 0 && key_bits + entry_bits(entries) > 64)
        return fail(GLSDM_ERR_UNSUPPORTED, "commit: key_bits %d + entry bits %d exceed 64", key_bits, entry_bits(entries));
    *bytes = entries == 0 ? 0 : plan_workspace(nullptr, entries).bytes;
    return GLSDM_OK;
}

extern "C" int glsdm_commit(void *bank, int32_t bank_dtype, int64_t rows, int64_t D,
                            const int64_t *addresses, const void *deltas, int32_t delta_dtype,
                            const int64_t *keys, int64_t key_min, int32_t key_bits, int64_t entries,
                            void *workspace, size_t workspace_bytes, int64_t *unique_out, void *stream)
{
    if (rows < 1 || D < 1 || entries < 0) return fail(GLSDM_ERR_ARG, "commit: bad shape rows=%lld D=%lld entries=%lld", (long long)rows, (long long)D, (long long)entries);
    if (!dtype_ok(bank_dtype) || !dtype_ok(delta_dtype)) return fail(GLSDM_ERR_ARG, "commit: bad dtype");
    if (key_bits < 0 || key_bits > 63) return fail(GLSDM_ERR_ARG, "commit: key_bits must be in [0, 63]");
    if (entries == 0) return GLSDM_OK;
    if (!bank || !addresses || !deltas) return fail(GLSDM_ERR_ARG, "commit: null pointer");
    if (D > 512 && D % 8 != 0) return fail(GLSDM_ERR_UNSUPPORTED, "commit: D=%lld not a multiple of 8 above 512", (long long)D);
    if (D > 64 * 8 * 4) return fail(GLSDM_ERR_UNSUPPORTED, "commit: D=%lld above 2048", (long long)D);
    const int ebits = entry_bits(entries);
    if (key_bits + ebits > 64)
        return fail(GLSDM_ERR_UNSUPPORTED, "commit: key_bits %d + entry bits %d exceed 64", key_bits, ebits);
    CommitWorkspace ws = plan_workspace(workspace, entries);
    if (!workspace || workspace_bytes < ws.bytes)
        return fail(GLSDM_ERR_WORKSPACE, "commit: workspace of %zu bytes needed, %zu given", ws.bytes, workspace_bytes);
    const hipStream_t st = as_stream(stream);

    const unsigned pack_blocks = (unsigned)std::min<int64_t>(ceil_div(entries, 256), 65536);
    hipLaunchKernelGGL(pack_kernel, dim3(pack_blocks), dim3(256), 0, st, keys, addresses, key_min, ebits, entries, ws.a);
    int rc = check_launch("pack_kernel");
    if (rc) return rc;

    uint64_t *src = ws.a, *dst = ws.b;
    for (int shift = ebits; shift < ebits + key_bits; shift += RADIX_BITS) {
        hipLaunchKernelGGL(radix_hist_kernel, dim3((unsigned)ws.tiles), dim3(SORT_THREADS), 0, st, src, entries, shift, ws.hist, ws.tiles);
        hipLaunchKernelGGL(radix_scan_kernel, dim3(1), dim3(SCAN_THREADS), 0, st, ws.hist, (int64_t)RADIX * ws.tiles);
        hipLaunchKernelGGL(radix_scatter_kernel, dim3((unsigned)ws.tiles), dim3(SORT_THREADS), 0, st, src, dst, entries, shift, ws.hist, ws.tiles);
        if ((rc = check_launch("radix pass"))) return rc;
        uint64_t *t = src; src = dst; dst = t;
    }

    const uint64_t emask = (ebits >= 64) ? ~0ull : ((1ull << ebits) - 1ull);
    if (bank_dtype == GLSDM_F32 && delta_dtype == GLSDM_F32)
        return launch_segment_t<float, float>(bank, rows, D, addresses, deltas, src, entries, emask, unique_out, st);
    if (bank_dtype == GLSDM_F32 && delta_dtype == GLSDM_BF16)
        return launch_segment_t<float, bf16_t>(bank, rows, D, addresses, deltas, src, entries, emask, unique_out, st);
    if (bank_dtype == GLSDM_BF16 && delta_dtype == GLSDM_F32)
        return launch_segment_t<bf16_t, float>(bank, rows, D, addresses, deltas, src, entries, emask, unique_out, st);
    return launch_segment_t<bf16_t, bf16_t>(bank, rows, D, addresses, deltas, src, entries, emask, unique_out, st);
}
