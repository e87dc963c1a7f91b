// Deterministic buffered commit on gfx950.
//
// Semantics (S/ = projects/gl-sdm/src/gl_sdm/): S/memory/transactions.py:89-96
// and S/memory/backends/commit.py:22-33 -- stable sort of the entries by key,
// then, for each run of equal addresses, an fp32 sum from 0 in sorted order,
// then old + sum.  No float atomics anywhere, so the result is bitwise
// reproducible.
//
// Pipeline (stream-ordered, no host sync, 3 + passes launches):
//   1. prep:      zero the per-pass digit histograms, look-back words and tile
//                 counters of the workspace (a fill kernel, safe under capture).
//   2. pack+hist: v[e] = a(e) << ebits | e with a(e) the row address (rows for an
//                 out-of-range address) and ebits = bits of E-1, plus the digit
//                 histograms of every radix pass in one read.
//   3. passes:    LSD radix sort of the packed words over the address bits, 8-bit
//                 digits, one kernel per pass: tiles take ids in launch order,
//                 rank their items stably (wavefront ballots: match-any over the
//                 8 digit bits, per-wave LDS counters), publish per-digit counts
//                 and resolve their global offsets by decoupled look-back over
//                 earlier tiles' published counts.  The entry bits below ebits
//                 are never sorted: they start ascending and every pass is
//                 stable, so each address's entries end up in arrival order.
//      Addresses of three or more digits (2^16 rows or more) take the bucket path
//      instead of steps 1-3, two launches: each tile packs its words and orders
//      them stably by the top address digit in LDS, recording where each
//      digit's piece lies; then a block per top digit gathers its pieces from
//      every tile, in tile order, and sorts them by the remaining digits.
//   4. segment:   a wavefront per 64 sorted positions reads the addresses from
//                 the sorted words, finds run heads with a ballot, and its lane
//                 groups each walk one run, summing the deltas in fp32 registers
//                 in (key, entry) order, then read-modify-write that bank row
//                 once.  Exactly one lane group writes each touched row.
//                 A run's arrival order already is its key order when its keys
//                 rise with the entry index (one proposal: keys grow with the
//                 token position); this is checked while walking, and a run
//                 that is not in key order is summed in (key, entry) order by a
//                 selection loop over the run instead.
// Grouping by address and ordering each address's deltas by (key, entry) is
// the reference's stable key sort followed by grouping of equal consecutive
// addresses whenever its keys keep equal addresses together (keys = addresses,
// and the stack's addr*(C*L) + pos*L + layer).
#include <atomic>
#include <mutex>

#include <type_traits>

#include "glsdm_internal.h"

namespace glsdm {

constexpr int RADIX_BITS = 8;
constexpr int RADIX = 1 << RADIX_BITS;
#ifndef GLSDM_BUCKET_SORT
#define GLSDM_BUCKET_SORT 1                              // tile-local top digit + per-bucket sort
#endif
#ifndef GLSDM_SORT_THREADS
#define GLSDM_SORT_THREADS 512
#endif
constexpr int SORT_THREADS = GLSDM_SORT_THREADS;       // >= RADIX: threads below RADIX own one digit each
#ifndef GLSDM_SORT_ITEMS
#define GLSDM_SORT_ITEMS 8
#endif
#ifndef GLSDM_PACK_BLOCKS
#define GLSDM_PACK_BLOCKS 1024
#endif
constexpr int SORT_ITEMS = GLSDM_SORT_ITEMS;            // per thread
constexpr int SORT_TILE = SORT_THREADS * SORT_ITEMS;    // entries per tile
constexpr int SORT_WAVES = SORT_THREADS / 64;
constexpr int WAVE_ITEMS = SORT_TILE / SORT_WAVES;      // consecutive entries per wave
#ifndef GLSDM_BT_THREADS
#define GLSDM_BT_THREADS 512
#endif
#ifndef GLSDM_BT_ITEMS
#define GLSDM_BT_ITEMS 4
#endif
constexpr int BT_THREADS = GLSDM_BT_THREADS;           // bucket path, step 1: threads per tile (>= RADIX)
constexpr int BT_ITEMS = GLSDM_BT_ITEMS;
constexpr int BT_TILE = BT_THREADS * BT_ITEMS;
constexpr int BT_WAVES = BT_THREADS / 64;
constexpr int BT_WAVE_ITEMS = BT_TILE / BT_WAVES;
constexpr int MAX_PASSES = 8;
constexpr int64_t MAX_ENTRIES = (int64_t)1 << 30;       // look-back words hold 30-bit counts
#ifndef GLSDM_SEG_WAVES
#define GLSDM_SEG_WAVES 8192                             // segment waves wanted before windows shrink
#endif

constexpr uint32_t LB_AGGREGATE = 1u << 30;             // tile's own count published
constexpr uint32_t LB_PREFIX = 2u << 30;                // inclusive prefix published
constexpr uint32_t LB_VALUE = LB_AGGREGATE - 1;
constexpr uint32_t LB_SPIN_LIMIT = 1u << 22;            // bounded wait; exceeded only by a bug

// Workspace words after the per-pass tile counters: the sort's error flags
// (bit 0: a look-back wait gave up, bit 1: a bucket's pieces were
// inconsistent; either way the segment step writes nothing), the deferred-run
// count, and the number of entries dropped for an out-of-range address.
constexpr int CW_ERROR = MAX_PASSES, CW_LONG = MAX_PASSES + 1, CW_DROPPED = MAX_PASSES + 2;
constexpr int CW_WORDS = MAX_PASSES + 3;

// Polls of an unpublished predecessor before a look-back wait gives up;
// glsdm_debug_force_lookback_timeout sets it to 0 (give up at once) so a test
// can drive the error path from the host.
static std::atomic<uint32_t> g_spin_limit{LB_SPIN_LIMIT};

static inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct CommitWorkspace {
    uint64_t *a, *b, *c;
    uint32_t *ghist;    // [MAX_PASSES][RADIX] global digit counts
    uint32_t *status;   // [passes][tiles][RADIX] look-back words
    uint32_t *counter;  // [MAX_PASSES] tile-id counters, then the CW_* words
    int64_t tiles, bucket_tiles;
    size_t status_words;
    size_t bytes;
};

static CommitWorkspace plan_workspace(void *base, int64_t entries, int passes)
{
    CommitWorkspace w;
    w.tiles = ceil_div(entries, SORT_TILE);
    w.bucket_tiles = ceil_div(entries, BT_TILE);
    // look-back words of the LSD passes, or the bucket path's piece words
    w.status_words = std::max((size_t)passes * (size_t)w.tiles, (size_t)w.bucket_tiles) * RADIX;
    const size_t words = align256(sizeof(uint64_t) * (size_t)entries);
    const size_t ghist = align256(sizeof(uint32_t) * MAX_PASSES * RADIX);
    const size_t status = align256(sizeof(uint32_t) * w.status_words);
    const size_t counter = align256(sizeof(uint32_t) * CW_WORDS);
    char *p = static_cast<char *>(base);
    w.a = reinterpret_cast<uint64_t *>(p);
    w.b = reinterpret_cast<uint64_t *>(p + words);
    w.c = reinterpret_cast<uint64_t *>(p + 2 * words);
    w.ghist = reinterpret_cast<uint32_t *>(p + 3 * words);
    w.status = reinterpret_cast<uint32_t *>(p + 3 * words + ghist);
    w.counter = reinterpret_cast<uint32_t *>(p + 3 * words + ghist + status);
    w.bytes = 3 * words + ghist + status + counter;
    return w;
}

static int entry_bits(int64_t entries)
{
    int b = 1;
    while (b < 63 && ((int64_t)1 << b) < entries) ++b;
    return b;
}

static int pass_count(int key_bits) { return (key_bits + RADIX_BITS - 1) / RADIX_BITS; }

__global__ __launch_bounds__(256) void commit_prep_kernel(uint32_t *__restrict__ ghist, uint32_t *__restrict__ status,
                                                          int64_t status_words, uint32_t *__restrict__ counter)
{
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (int64_t i = tid; i < status_words; i += stride) status[i] = 0;
    if (tid < MAX_PASSES * RADIX) ghist[tid] = 0;
    if (tid < CW_WORDS) counter[tid] = 0;
}

// The commit's status words for the caller: [0] the sort's error flags, [1]
// the entries dropped for an out-of-range address (no workspace: zeros).
__global__ __launch_bounds__(64) void commit_status_kernel(const uint32_t *__restrict__ counter,
                                                           int64_t *__restrict__ out)
{
    if (threadIdx.x == 0) {
        out[0] = counter ? (int64_t)counter[CW_ERROR] : 0;
        out[1] = counter ? (int64_t)counter[CW_DROPPED] : 0;
    }
}

__global__ __launch_bounds__(256) void pack_hist_kernel(const int64_t *__restrict__ addresses, int64_t rows,
                                                        int ebits, int first_shift, int passes, int64_t n,
                                                        uint64_t *__restrict__ out, uint32_t *__restrict__ ghist)
{
    __shared__ uint32_t h[MAX_PASSES][RADIX];
    for (int p = 0; p < passes; ++p) h[p][threadIdx.x] = 0;
    __syncthreads();
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t a = addresses[i];
        const uint64_t row = (a >= 0 && a < rows) ? (uint64_t)a : (uint64_t)rows;   // out of range: one run, dropped
        const uint64_t v = (row << ebits) | (uint64_t)i;
        out[i] = v;
        for (int p = 0; p < passes; ++p)
            atomicAdd(&h[p][(uint32_t)(v >> (first_shift + p * RADIX_BITS)) & (RADIX - 1)], 1u);
    }
    __syncthreads();
    for (int p = 0; p < passes; ++p) {
        const uint32_t c = h[p][threadIdx.x];
        if (c) atomicAdd(&ghist[p * RADIX + threadIdx.x], c);
    }
}

// Inclusive prefix sum of one value per digit over the digit-owner threads
// (tid < RADIX, whole wavefronts): shuffle scans within wavefronts, one block
// barrier, then the earlier wavefronts' totals.  Every thread of the block
// calls it (non-owners pass 0).
__device__ __forceinline__ uint32_t digit_scan(uint32_t x, uint32_t *s_wave)
{
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(x, off);
        if (lane >= off) x += y;
    }
    if (tid < RADIX && lane == 63) s_wave[wave] = x;
    __syncthreads();
    uint32_t add = 0;
    if (tid < RADIX)
        for (int w = 0; w < wave; ++w) add += s_wave[w];
    return x + add;
}

__global__ __launch_bounds__(SORT_THREADS) void onesweep_kernel(const uint64_t *__restrict__ in,
                                                                uint64_t *__restrict__ out, int64_t n, int shift,
                                                                const uint32_t *__restrict__ ghist,
                                                                uint32_t *__restrict__ status,
                                                                uint32_t *__restrict__ counter,
                                                                uint32_t *__restrict__ error, uint32_t spin_limit)
{
    static_assert(SORT_THREADS >= RADIX && SORT_THREADS % 64 == 0, "one thread per digit");
    __shared__ uint32_t cnt[SORT_WAVES][RADIX];
    __shared__ int32_t base[RADIX];           // global position of the tile's first item of each digit, minus
                                              // that item's position in the tile's digit-ordered LDS copy
    __shared__ uint32_t s_wsum[2][RADIX / 64];
    __shared__ uint32_t lstart[RADIX];        // first LDS position of each digit in the tile
    __shared__ uint64_t s_items[SORT_TILE];   // the tile's items in (digit, rank) order
    __shared__ uint32_t s_tile;
    const int tid = threadIdx.x;
    const bool owner = tid < RADIX;           // thread `tid` owns digit `tid`
    if (tid == 0) s_tile = atomicAdd(counter, 1u);     // tile ids in the order tiles start
    for (int x = tid; x < SORT_WAVES * RADIX; x += SORT_THREADS) (&cnt[0][0])[x] = 0;
    // exclusive prefix over digits of the global histogram
    const uint32_t own = owner ? ghist[tid] : 0u;
    const uint32_t digit_base = digit_scan(own, s_wsum[0]) - own;   // its barrier also publishes cnt, s_tile
    const int64_t tile = s_tile;

    // stable rank of each item within its wave's WAVE_ITEMS consecutive entries
    const int wave = tid >> 6, lane = tid & 63;
    const uint64_t lt = (1ull << lane) - 1ull;
    const int64_t start = tile * SORT_TILE + (int64_t)wave * WAVE_ITEMS;
    uint64_t v[SORT_ITEMS];
    uint32_t dig[SORT_ITEMS], pos[SORT_ITEMS];
#pragma unroll
    for (int k = 0; k < SORT_ITEMS; ++k) {
        const int64_t i = start + k * 64 + lane;
        const bool valid = i < n;
        v[k] = valid ? in[i] : 0ull;
        const uint32_t d = (uint32_t)(v[k] >> shift) & (RADIX - 1);
        dig[k] = d;
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

    // digit owners: wave prefix and tile total, published at once
    uint32_t total = 0;
    uint32_t *word = status + tile * RADIX + tid;
    if (owner) {
#pragma unroll
        for (int w = 0; w < SORT_WAVES; ++w) {
            const uint32_t x = cnt[w][tid];
            cnt[w][tid] = total;
            total += x;
        }
        __hip_atomic_store(word, (tile == 0 ? LB_PREFIX : LB_AGGREGATE) | total, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }

    // the tile's items in digit order in LDS: exclusive prefix of the tile totals
    const uint32_t first = digit_scan(total, s_wsum[1]) - total;
    if (owner) lstart[tid] = first;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < SORT_ITEMS; ++k) {
        const int64_t i = start + k * 64 + lane;
        const uint32_t at = lstart[dig[k]] + cnt[wave][dig[k]] + pos[k];
        if (i < n && at < (uint32_t)SORT_TILE) s_items[at] = v[k];
    }

    // digit owners: decoupled look-back over earlier tiles' counts of their digit
    if (owner) {
        uint32_t prefix = 0;
        if (tile > 0) {
            const uint32_t *look = word - RADIX;
            uint32_t spins = 0;
            for (;;) {
                const uint32_t s = __hip_atomic_load(look, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                // predecessor not published yet (a zero limit never waits: the host-forced failure)
                if ((s & ~LB_VALUE) == 0 || spin_limit == 0) {
                    if (spins++ >= spin_limit) { atomicOr(error, 1u); break; }
                    continue;
                }
                prefix += s & LB_VALUE;
                if (s & LB_PREFIX) break;
                look -= RADIX;                         // aggregate only: keep walking back
            }
            __hip_atomic_store(word, LB_PREFIX | (prefix + total), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        base[tid] = (int32_t)(digit_base + prefix) - (int32_t)first;
    }
    __syncthreads();

    // write-out in LDS order: consecutive threads write a digit's consecutive positions
    const int64_t tile_n = n - tile * SORT_TILE;
    const int valid_items = tile_n < SORT_TILE ? (int)tile_n : SORT_TILE;
#pragma unroll
    for (int k = 0; k < SORT_ITEMS; ++k) {
        const int j = k * SORT_THREADS + tid;
        if (j < valid_items) {
            const uint64_t x = s_items[j];
            const int64_t dst = (int64_t)base[(uint32_t)(x >> shift) & (RADIX - 1)] + j;
            if (dst >= 0 && dst < n) out[dst] = x;   // always in range; the guard keeps a bug from faulting
        }
    }
}

// The address sort when the address needs three or more 8-bit digits (the
// bucket path, two launches): the words are grouped by their top address digit
// (256 buckets, stable) and one block per bucket sorts its words by the
// remaining address digits, least significant first, each pass stable, so the
// result equals the full LSD sort.  The top digit is taken from the bits of the
// largest real row (rows - 1), so real rows spread over all 256 buckets; the
// out-of-range value `rows` clamps to the last bucket when rows is a power of
// two, and that bucket's sort then also covers the sentinel's bit (one more
// pass), which orders it after every real row.  A bucket of up to BK_CAP words is sorted
// in LDS; a larger one (skewed addresses) in chunks of BK_CAP through global
// scratch, with a counting pass per digit.
#ifndef GLSDM_BK_THREADS
#define GLSDM_BK_THREADS 1024
#endif
constexpr int BK_THREADS = GLSDM_BK_THREADS;
#ifndef GLSDM_BK_CAP
// 4096 words (two 32 KiB LDS buffers): twice the ~2048 words a bucket holds when
// 2^19 entries spread over 256 buckets; larger buckets take the global path.
// Measured against 8192 and 3072 with the route stream beside it (config 2 commit
// 110 -> 108 us, the overlapped step ~0.5 % faster, config 3 unchanged)
#define GLSDM_BK_CAP 4096
#endif
constexpr int BK_ITEMS = GLSDM_BK_CAP / BK_THREADS;
constexpr int BK_CAP = BK_THREADS * BK_ITEMS;          // words a bucket may hold to be sorted in LDS
constexpr int BK_WAVES = BK_THREADS / 64;

// Stable ranks of one chunk's items (held BK_ITEMS per thread at wave-major
// positions): on return (after a block barrier) cnt[w][d] is the number of
// digit-d items in waves before w, total the chunk's count of digit `tid`
// (owners), pos[k] the rank of item k among its wave's digit-d items.
__device__ __forceinline__ void bk_rank(const uint64_t (&v)[BK_ITEMS], const bool (&valid)[BK_ITEMS], int wi,
                                        int shift, uint32_t (&dig)[BK_ITEMS], uint32_t (&pos)[BK_ITEMS],
                                        uint32_t (*cnt)[RADIX], uint32_t &total)
{
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint64_t lt = (1ull << lane) - 1ull;
    for (int x = tid; x < BK_WAVES * RADIX; x += BK_THREADS) (&cnt[0][0])[x] = 0;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < BK_ITEMS; ++k) {
        dig[k] = 0;
        pos[k] = 0;
        if (k >= wi) continue;                            // block-uniform: this item slot is empty everywhere
        const uint32_t d = (uint32_t)(v[k] >> shift) & (RADIX - 1);
        dig[k] = d;
        uint64_t peers = __ballot(valid[k]);
#pragma unroll
        for (int bit = 0; bit < RADIX_BITS; ++bit) {
            const bool on = (d >> bit) & 1u;
            const uint64_t m = __ballot(on);
            peers &= on ? m : ~m;
        }
        const uint32_t before = (uint32_t)__popcll(peers & lt);
        uint32_t c = 0;
        if (valid[k]) c = cnt[wave][d];
        pos[k] = c + before;
        if (valid[k] && before == 0) cnt[wave][d] = c + (uint32_t)__popcll(peers);
    }
    __syncthreads();
    total = 0;
    if (tid < RADIX) {
#pragma unroll
        for (int w = 0; w < BK_WAVES; ++w) {
            const uint32_t x = cnt[w][tid];
            cnt[w][tid] = total;
            total += x;
        }
    }
    __syncthreads();                                      // the wave prefixes are read by every thread
}

// Bucket path, step 1: each tile of BT_TILE consecutive entries packs its
// words, orders them stably by the top address digit in LDS and stores them in
// that order at the tile's own position, with one word per (digit, tile) -- the tile's first position of
// the digit << 16 | the digit's count in the tile -- stored digit-major, so the
// block that sorts a bucket reads its pieces of every tile in one coalesced
// load.  Block 0 also clears the workspace's counter words.
static_assert(BT_TILE < 65536 && BT_THREADS >= RADIX && BT_THREADS % 64 == 0,
              "tile positions and counts are 16-bit; one thread per digit");

__global__ __launch_bounds__(BT_THREADS) void tile_bucket_kernel(const int64_t *__restrict__ addresses,
                                                                   int64_t rows, int ebits, int shift, int64_t n,
                                                                   uint64_t *__restrict__ out,
                                                                   uint32_t *__restrict__ pieces, int64_t tiles,
                                                                   uint32_t *__restrict__ counter)
{
    __shared__ uint32_t cnt[BT_WAVES][RADIX];
    __shared__ uint32_t s_wsum[RADIX / 64];
    __shared__ uint32_t lstart[RADIX];
    __shared__ uint64_t s_items[BT_TILE];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const bool owner = tid < RADIX;
    const int64_t tile = blockIdx.x;
    if (tile == 0 && tid < CW_WORDS) counter[tid] = 0;
    for (int x = tid; x < BT_WAVES * RADIX; x += BT_THREADS) (&cnt[0][0])[x] = 0;
    __syncthreads();

    // stable rank of each item among its wave's items of the same digit
    const uint64_t lt = (1ull << lane) - 1ull;
    const int64_t start = tile * BT_TILE + (int64_t)wave * BT_WAVE_ITEMS;
    uint64_t v[BT_ITEMS];
    uint32_t dig[BT_ITEMS], pos[BT_ITEMS];
#pragma unroll
    for (int k = 0; k < BT_ITEMS; ++k) {
        const int64_t i = start + k * 64 + lane;
        const bool valid = i < n;
        const int64_t a = valid ? addresses[i] : 0;
        const uint64_t row = (a >= 0 && a < rows) ? (uint64_t)a : (uint64_t)rows;   // out of range: one run, dropped
        v[k] = (row << ebits) | (uint64_t)i;
        const uint64_t top = v[k] >> shift;                        // <= RADIX: the clamped sentinel
        const uint32_t d = top < (uint64_t)RADIX ? (uint32_t)top : (uint32_t)(RADIX - 1);
        dig[k] = d;
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

    // digit owners: per-wave prefixes and the tile's count of their digit
    uint32_t total = 0;
    if (owner) {
#pragma unroll
        for (int w = 0; w < BT_WAVES; ++w) {
            const uint32_t x = cnt[w][tid];
            cnt[w][tid] = total;
            total += x;
        }
    }
    const uint32_t first = digit_scan(total, s_wsum) - total;    // its barrier publishes the wave prefixes
    if (owner) {
        lstart[tid] = first;
        pieces[(int64_t)tid * tiles + tile] = first << 16 | total;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < BT_ITEMS; ++k) {
        const int64_t i = start + k * 64 + lane;
        const uint32_t at = lstart[dig[k]] + cnt[wave][dig[k]] + pos[k];
        if (i < n && at < (uint32_t)BT_TILE) s_items[at] = v[k];
    }
    __syncthreads();
    const int64_t tile_n = n - tile * BT_TILE;
    const int valid_items = tile_n < BT_TILE ? (int)tile_n : BT_TILE;
#pragma unroll
    for (int k = 0; k < BT_ITEMS; ++k) {
        const int j = k * BT_THREADS + tid;
        if (j < valid_items) out[tile * BT_TILE + j] = s_items[j];
    }
}

// Inclusive prefix sum over the BK_THREADS threads of a block (every thread
// calls it); *total gets the block's sum.
__device__ __forceinline__ uint32_t block_scan(uint32_t x, uint32_t *s_w, uint32_t *total)
{
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(x, off);
        if (lane >= off) x += y;
    }
    if (lane == 63) s_w[wave] = x;
    __syncthreads();
    uint32_t add = 0, sum = 0;
#pragma unroll
    for (int w = 0; w < BK_WAVES; ++w) {
        const uint32_t y = s_w[w];
        add += w < wave ? y : 0u;
        sum += y;
    }
    __syncthreads();                                      // s_w is free again
    *total = sum;
    return x + add;
}

// Bucket path, step 2: one block per top digit gathers its pieces in tile
// order (tiles hold increasing entry ranges, so the gathered bucket is in entry
// order within each address) and sorts them by the remaining address digits,
// in LDS up to BK_CAP words, else in global memory; the words of bucket d end
// at positions [start_d, start_d + size_d) of out, start_d the count of words
// with a smaller top digit.
__global__ __launch_bounds__(BK_THREADS) void bucket_sort_kernel(const uint64_t *__restrict__ in,
                                                                      const uint32_t *__restrict__ pieces,
                                                                      int64_t tiles, int64_t n,
                                                                      uint64_t *__restrict__ scratch,
                                                                      uint64_t *__restrict__ out, int ebits,
                                                                      int lpasses_all, int lpasses_last,
                                                                      uint32_t *__restrict__ error)
{
    const int lpasses = blockIdx.x == RADIX - 1 ? lpasses_last : lpasses_all;
    __shared__ uint64_t s_x[BK_CAP];
    __shared__ uint64_t s_y[BK_CAP];
    __shared__ uint32_t cnt[BK_WAVES][RADIX];
    __shared__ uint32_t lstart[RADIX];
    __shared__ uint32_t s_wsum[2][RADIX / 64];
    __shared__ uint32_t s_scan[BK_WAVES];
    __shared__ int64_t s_base[RADIX];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t *mine = pieces + (int64_t)blockIdx.x * tiles;
    // the bucket's size and start: sums over the tiles of its piece counts and first positions
    uint32_t my_cnt = 0, my_first = 0;
    for (int64_t t = tid; t < tiles; t += BK_THREADS) {
        const uint32_t w = mine[t];
        my_cnt += w & 0xffffu;
        my_first += w >> 16;
    }
    uint32_t size32, start32;
    block_scan(my_cnt, s_scan, &size32);
    block_scan(my_first, s_scan, &start32);
    const int64_t size = size32, start = start32;
    if (start + size > n) {                                 // block-uniform; never holds after step 1
        if (tid == 0) atomicOr(error, 2u);
        return;
    }
    if (size == 0) return;
    const bool in_lds = size <= BK_CAP;
    // global path: gather into X, then passes X -> Y -> X ..., the last one into out
    uint64_t *X = ((lpasses % 2 == 0) ? out : scratch) + start;
    uint64_t *Y = ((lpasses % 2 == 0) ? scratch : out) + start;
    // up to BK_THREADS tiles at a time: the pieces' inclusive prefix and source
    // positions in LDS (in cnt, which the ranking clears before use), then every
    // thread copies words j, j + BK_THREADS, ..., finding each one's tile by
    // binary search, so consecutive threads copy consecutive words
    static_assert(2 * BK_THREADS <= BK_WAVES * RADIX, "gather tables fit in cnt");
    uint32_t *s_pref = &cnt[0][0], *s_from = &cnt[0][0] + BK_THREADS;
    uint32_t carry = 0;
    for (int64_t c0 = 0; c0 < tiles; c0 += BK_THREADS) {   // block-uniform trip count
        const int64_t t = c0 + tid;
        const uint32_t w = t < tiles ? mine[t] : 0u;
        uint32_t chunk;
        const uint32_t incl = block_scan(w & 0xffffu, s_scan, &chunk);   // its barriers end the last round's reads
        s_pref[tid] = incl;
        s_from[tid] = (uint32_t)(t * BT_TILE + (w >> 16));              // < n <= 2^30
        __syncthreads();
        const int last = (int)(tiles - c0 < BK_THREADS ? tiles - c0 : BK_THREADS) - 1;
        for (uint32_t j = tid; j < chunk; j += BK_THREADS) {
            int lo = 0, hi = last;                                     // first tile whose prefix exceeds j
            while (lo < hi) {
                const int mid = (lo + hi) >> 1;
                if (s_pref[mid] > j) hi = mid;
                else lo = mid + 1;
            }
            const int64_t from = (int64_t)s_from[lo] + (j - (lo ? s_pref[lo - 1] : 0u));
            const uint32_t at = carry + j;
            const uint64_t x = from < n ? in[from] : 0ull;
            if (in_lds) {
                if (at < (uint32_t)BK_CAP) s_x[at] = x;
            } else if (at < (uint32_t)size) {
                X[at] = x;
            }
        }
        carry += chunk;
        __syncthreads();
    }
    if (in_lds) {
        const int wi = (int)ceil_div(size, 64 * BK_WAVES);
        const int base_at = wave * wi * 64 + lane;         // item k of this thread: base_at + 64 k
        uint64_t *src = s_x, *dst = s_y;
        for (int p = 0; p < lpasses; ++p) {
            uint64_t v[BK_ITEMS];
            bool valid[BK_ITEMS];
            uint32_t dig[BK_ITEMS], pos[BK_ITEMS], total;
#pragma unroll
            for (int k = 0; k < BK_ITEMS; ++k) {
                const int i = base_at + 64 * k;
                valid[k] = k < wi && i < size;
                v[k] = valid[k] ? src[i] : 0ull;
            }
            bk_rank(v, valid, wi, ebits + p * RADIX_BITS, dig, pos, cnt, total);
            const uint32_t first = digit_scan(total, s_wsum[p & 1]) - total;
            if (tid < RADIX) lstart[tid] = first;
            __syncthreads();
#pragma unroll
            for (int k = 0; k < BK_ITEMS; ++k) {
                const uint32_t at = lstart[dig[k]] + cnt[wave][dig[k]] + pos[k];
                if (valid[k] && at < (uint32_t)BK_CAP) dst[at] = v[k];
            }
            __syncthreads();
            uint64_t *t = src; src = dst; dst = t;
        }
#pragma unroll
        for (int k = 0; k < BK_ITEMS; ++k) {
            const int i = k * BK_THREADS + tid;
            if (i < size) out[start + i] = src[i];
        }
        return;
    }
    uint64_t *src = X;
    for (int p = 0; p < lpasses; ++p) {
        uint64_t *dst = (p % 2 == 0) ? Y : X;
        const int shift = ebits + p * RADIX_BITS;
        for (int x = tid; x < RADIX; x += BK_THREADS) lstart[x] = 0;
        __syncthreads();
        for (int64_t i = tid; i < size; i += BK_THREADS)
            atomicAdd(&lstart[(uint32_t)(src[i] >> shift) & (RADIX - 1)], 1u);
        __syncthreads();
        const uint32_t cnt_d = tid < RADIX ? lstart[tid] : 0u;
        const uint32_t first = digit_scan(cnt_d, s_wsum[p & 1]) - cnt_d;
        if (tid < RADIX) s_base[tid] = first;
        __syncthreads();
        for (int64_t c0 = 0; c0 < size; c0 += BK_CAP) {
            uint64_t v[BK_ITEMS];
            bool valid[BK_ITEMS];
            uint32_t dig[BK_ITEMS], pos[BK_ITEMS], total;
            const int64_t left = size - c0;
            const int wi = left < BK_CAP ? (int)ceil_div(left, 64 * BK_WAVES) : BK_ITEMS;
            const int base_at = wave * wi * 64 + lane;
#pragma unroll
            for (int k = 0; k < BK_ITEMS; ++k) {
                const int64_t i = c0 + base_at + 64 * k;
                valid[k] = k < wi && i < size;
                v[k] = valid[k] ? src[i] : 0ull;
            }
            bk_rank(v, valid, wi, shift, dig, pos, cnt, total);
#pragma unroll
            for (int k = 0; k < BK_ITEMS; ++k) {
                const int64_t at = s_base[dig[k]] + cnt[wave][dig[k]] + pos[k];
                if (valid[k] && at < size) dst[at] = v[k];
            }
            __syncthreads();
            if (tid < RADIX) s_base[tid] += total;
            __syncthreads();
        }
        src = dst;
    }
}

// Where the segment kernel takes each entry's delta row from.
//
// StoredDeltas: the materialised deltas [E, D] (fp32 or bf16).
template <typename TD> struct StoredDeltas {
    const TD *deltas;
    int64_t D;
    struct Entry {
        const TD *src;
    };
    __device__ __forceinline__ Entry entry(int64_t ent) const { return {deltas + ent * D}; }
    template <int VEC>
    __device__ __forceinline__ void get(const Entry &e, int v, const float (&)[VEC], float (&x)[VEC]) const
    {
        if constexpr (VEC * sizeof(TD) == 16 && std::is_same<TD, bf16_t>::value) {
            const uint4 u = load16_stream(e.src + (int64_t)v * VEC);   // each delta is read once
            const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                x[2 * i] = __uint_as_float(w[i] << 16);
                x[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
            }
        } else {
            VecLoad<TD, VEC>::load(e.src + (int64_t)v * VEC, x);
        }
    }
};

// ProposalTerms: the write-proposal delta of S/runtime/dense.py:11-14,
//     mass * ((decay - 1) * row + weight * error),
// evaluated from the row's value before the commit, which is the snapshot row
// the proposal gathered (S/layers/global_layer.py:44): entry e belongs to
// proposal row r = e / width, whose error row and decay were computed once,
// and to mass group r / heads.  Separate fp32 operations in that order.
struct ProposalTerms {
    const float *error, *decay, *weights, *mass;
    int64_t D;
    uint32_t width, heads;
    struct Entry {
        const float *err;
        float a, w, m;
    };
    __device__ __forceinline__ Entry entry(int64_t ent) const
    {
#pragma clang fp contract(off)
        const uint32_t r = (uint32_t)ent / width;
        return {error + (int64_t)r * D, decay[r] - 1.0f, weights[ent], mass[r / heads]};
    }
    template <int VEC>
    __device__ __forceinline__ void get(const Entry &e, int v, const float (&old)[VEC], float (&x)[VEC]) const
    {
#pragma clang fp contract(off)
        float er[VEC];
        VecLoad<float, VEC>::load(e.err + (int64_t)v * VEC, er);
#pragma unroll
        for (int y = 0; y < VEC; ++y) {
            const float p = e.a * old[y];
            const float q = e.w * er[y];
            const float s = p + q;
            x[y] = e.m * s;
        }
    }
};

// ReadGradTerms: the gathered rows' gradient in the read's backward,
//     weights[e] * grad_out[e / width]
// (the autograd of out = sum_j w_j row_j, S/memory/routing.py:27-28), added
// onto a gradient bank in entry order: the result of the reference's
// accumulating index backward of flat[address] (S/memory/routing.py:42).
struct ReadGradTerms {
    const float *weights, *grad_out;
    int64_t D;
    uint32_t width;
    struct Entry {
        const float *g;
        float w;
    };
    __device__ __forceinline__ Entry entry(int64_t ent) const
    {
        const uint32_t r = (uint32_t)ent / width;
        return {grad_out + (int64_t)r * D, weights[ent]};
    }
    template <int VEC>
    __device__ __forceinline__ void get(const Entry &e, int v, const float (&)[VEC], float (&x)[VEC]) const
    {
#pragma clang fp contract(off)
        float g[VEC];
        VecLoad<float, VEC>::load(e.g + (int64_t)v * VEC, g);
#pragma unroll
        for (int y = 0; y < VEC; ++y) x[y] = g[y] * e.w;
    }
};

// Where the segment kernel reads each touched row's old value and writes its
// new one.
//
// DenseRows: the bank [rows, D] itself, in place.
template <typename TB> struct DenseRows {
    TB *bank;
    int64_t D;
    __device__ __forceinline__ const TB *old_row(int64_t a) const { return bank + a * D; }
    __device__ __forceinline__ TB *new_row(int64_t a, int, int64_t) const { return bank + a * D; }
};

// OverlayRows: a shared base [H*S, D] and, per request, a slot map [B*H*S]
// (-1: the base row) into a pool of rows.  Address a = (b*H + h)*S + slot reads
// pool row map[a] or base row a % (H*S); a row written for the first time gets
// pool row offset + p, with p the sorted position of its run's head (distinct
// per run, < entries), so allocation needs no atomics and the pool layout is
// the same on every run.  The caller advances offset by entries per commit.
template <typename TB> struct OverlayRows {
    const TB *base;
    int32_t *map;
    TB *pool;
    int64_t D, hs, offset;
    __device__ __forceinline__ const TB *old_row(int64_t a) const
    {
        const int32_t m = map[a];
        return m >= 0 ? pool + (int64_t)m * D : base + (a % hs) * D;
    }
    // every lane of the run's group calls it; `li` is the lane within the group
    __device__ __forceinline__ TB *new_row(int64_t a, int li, int64_t head) const
    {
        int32_t m = map[a];
        if (m < 0) {
            m = (int32_t)(offset + head);
            if (li == 0) map[a] = m;
        }
        return pool + (int64_t)m * D;
    }
};

// The segment step's side words in the workspace: where runs that continue
// past their window are left (a word buffer the sorted words are not in, and
// its counter), and the sort's status words (CW_ERROR .. CW_DROPPED).
struct SegAux {
    int64_t *long_list;
    uint32_t *long_count;
    uint32_t *status;
};

// One wavefront per window of `win` (a power of two <= 64) consecutive sorted
// positions; lane groups of `lpr` lanes (one bank row each) walk the address
// runs that start in the window, continuing past its end when a run does.
template <typename TB, typename SRC, typename ROWS, int VEC, int CH, bool DEFER>
__global__ __launch_bounds__(256) void segment_kernel(const ROWS store, int64_t rows, int64_t D,
                                                      const int64_t *__restrict__ keys, const SRC src,
                                                      const uint64_t *__restrict__ sorted, int64_t n, int ebits,
                                                      int nv, int lpr, int win,
                                                      unsigned long long *__restrict__ unique_out, SegAux aux)
{
#pragma clang fp contract(off)
    if (aux.status[0] != 0) return;                     // the sort failed: leave every row untouched
    __shared__ uint64_t s_w[4][64];
    __shared__ int s_head[4][64];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t p0 = ((int64_t)blockIdx.x * 4 + wave) * win;
    const int64_t p = p0 + lane;
    const bool valid = lane < win && p < n;
    const uint64_t emask = (1ull << ebits) - 1ull;
    const uint64_t w = valid ? sorted[p] : ~0ull;
    const int64_t a = valid ? (int64_t)(w >> ebits) : -1;
    int64_t prev = __shfl_up(a, 1);
    if (lane == 0) prev = (p0 > 0 && p0 - 1 < n) ? (int64_t)(sorted[p0 - 1] >> ebits) : -2;
    const bool head = valid && a != prev;
    const uint64_t heads = __ballot(head);
    s_w[wave][lane] = w;
    if (head) s_head[wave][__popcll(heads & ((1ull << lane) - 1ull))] = lane;
    const int nheads = __popcll(heads);
    // rows this window will write: heads whose address is in range (one atomic per wave)
    const uint64_t live = __ballot(head && a < rows);
    if (unique_out && lane == 0 && live) atomicAdd(unique_out, (unsigned long long)__popcll(live));
    __syncthreads();

    const int ng = 64 / lpr;
    const int grp = lane / lpr, li = lane % lpr;
    // whether the window's last run continues past it (wave-uniform)
    bool crosses = false;
    if constexpr (DEFER) crosses = p0 + win < n && (sorted[p0 + win] >> ebits) == (s_w[wave][win - 1] >> ebits);
    auto word_at = [&](int q) -> uint64_t { return q < win ? s_w[wave][q] : sorted[p0 + q]; };
    auto add_delta = [&](int64_t ent, const float (&old)[CH][VEC], float (&acc)[CH][VEC]) {
        if (ent >= n) return;                           // impossible after a correct sort; never read out of bounds
        const typename SRC::Entry e = src.entry(ent);
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int v = li + c * lpr;
            if (v < nv) {
                float x[VEC];
                src.template get<VEC>(e, v, old[c], x);
#pragma unroll
                for (int y = 0; y < VEC; ++y) acc[c][y] += x[y];
            }
        }
    };
    for (int r = grp; r < nheads; r += ng) {
        const int h = s_head[wave][r];
        const uint64_t hw = s_w[wave][h];
        const int64_t row_addr = (int64_t)(hw >> ebits);
        if (row_addr >= rows) {                         // out-of-range entries: dropped, and counted
            if (li == 0) aux.status[CW_DROPPED - CW_ERROR] = (uint32_t)(n - (p0 + h));   // they sort last
            continue;
        }
        // run length: positions after the head with the same address.  DEFER
        // (small windows, which long runs cross many of): a run that continues
        // past the window is left to long_run_kernel
        int len = 1;
        if constexpr (DEFER) {
            while (h + len < win && p0 + h + len < n && (int64_t)(s_w[wave][h + len] >> ebits) == row_addr) ++len;
            if (h + len == win && crosses) {
                if (li == 0) aux.long_list[atomicAdd(aux.long_count, 1u)] = p0 + h;
                continue;
            }
        } else {
            while (p0 + h + len < n && (int64_t)(word_at(h + len) >> ebits) == row_addr) ++len;
        }
        const TB *row = store.old_row(row_addr);
        float old[CH][VEC], acc[CH][VEC];
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int v = li + c * lpr;
#pragma unroll
            for (int x = 0; x < VEC; ++x) {
                acc[c][x] = 0.0f;                               // sums start from +0
                old[c][x] = 0.0f;
            }
            if (v < nv) VecLoad<TB, VEC>::load(row + (int64_t)v * VEC, old[c]);
        }
        // arrival order is key order unless a later entry has a smaller key; the
        // group's lanes compare the run's neighbouring pairs in parallel
        bool in_order = true;
        auto key_of = [&](uint64_t word) -> int64_t {
            const int64_t e = (int64_t)(word & emask);
            return e < n ? keys[e] : INT64_MAX;
        };
        if (keys && len > 1) {
            bool ok = true;
            for (int q = 1 + li; q < len; q += lpr) {
                const int64_t k0 = key_of(word_at(h + q - 1)), k1 = key_of(word_at(h + q));
                ok &= k1 >= k0;
            }
            const uint64_t bad = __ballot(!ok);
            const uint64_t mine = (lpr >= 64 ? ~0ull : ((1ull << lpr) - 1ull)) << (grp * lpr);
            in_order = (bad & mine) == 0;
        }
        if (in_order) {
            for (int q = 0; q < len; ++q) add_delta((int64_t)(word_at(h + q) & emask), old, acc);
        } else {
            // exact (key, entry) order by repeated selection of the next smallest pair
            int64_t last_k = INT64_MIN, last_e = -1;
            for (int r2 = 0; r2 < len; ++r2) {
                int64_t best_k = INT64_MAX, best_e = INT64_MAX;
                for (int q = 0; q < len; ++q) {
                    const uint64_t wq = word_at(h + q);
                    const int64_t e = (int64_t)(wq & emask);
                    const int64_t k = key_of(wq);
                    const bool after = k > last_k || (k == last_k && e > last_e);
                    const bool before = k < best_k || (k == best_k && e < best_e);
                    if (after && before) { best_k = k; best_e = e; }
                }
                add_delta(best_e, old, acc);
                last_k = best_k;
                last_e = best_e;
            }
        }
        TB *dst = store.new_row(row_addr, li, p0 + h);
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int v = li + c * lpr;
            if (v < nv) {
#pragma unroll
                for (int x = 0; x < VEC; ++x) old[c][x] = old[c][x] + acc[c][x];
                if constexpr (VEC * sizeof(TB) == 16 && std::is_same<TB, bf16_t>::value) {
                    uint32_t w[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        w[i] = (uint32_t)f32_to_bf16(old[c][2 * i]) | ((uint32_t)f32_to_bf16(old[c][2 * i + 1]) << 16);
                    store16_stream(dst + (int64_t)v * VEC, make_uint4(w[0], w[1], w[2], w[3]));
                } else {
                    VecStore<TB, VEC>::store(dst + (int64_t)v * VEC, old[c]);
                }
            }
        }
    }
}

// The runs segment_kernel left because they continue past their window (long
// collision runs under skewed routes, or runs that straddle a window's end):
// one lane group per run finds the run's end lpr positions at a time, fetches
// lpr entry indices at a time, and sums the deltas in the same (key, entry)
// order as segment_kernel, so the result is the same bit for bit.
template <typename TB, typename SRC, typename ROWS, int VEC, int CH>
__global__ __launch_bounds__(256) void long_run_kernel(const ROWS store, int64_t D, const int64_t *__restrict__ keys,
                                                       const SRC src, const uint64_t *__restrict__ sorted, int64_t n,
                                                       int ebits, int nv, int lpr,
                                                       const SegAux aux)
{
#pragma clang fp contract(off)
    if (aux.status[0] != 0) return;
    const int lane = threadIdx.x & 63;
    const int ng = 64 / lpr, grp = lane / lpr, li = lane % lpr;
    const uint64_t mine = (lpr >= 64 ? ~0ull : ((1ull << lpr) - 1ull)) << (grp * lpr);
    const uint64_t emask = (1ull << ebits) - 1ull;
    const int64_t count = *aux.long_count;
    const int64_t groups = (int64_t)gridDim.x * 4 * ng;
    auto key_of = [&](uint64_t word) -> int64_t {
        const int64_t e = (int64_t)(word & emask);
        return e < n ? keys[e] : INT64_MAX;
    };
    auto add_delta = [&](int64_t ent, const float (&old)[CH][VEC], float (&acc)[CH][VEC]) {
        if (ent >= n) return;
        const typename SRC::Entry e = src.entry(ent);
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int v = li + c * lpr;
            if (v < nv) {
                float x[VEC];
                src.template get<VEC>(e, v, old[c], x);
#pragma unroll
                for (int y = 0; y < VEC; ++y) acc[c][y] += x[y];
            }
        }
    };
    // every lane of a group runs the same iterations (group-uniform control flow)
    for (int64_t i = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * ng + grp; i < count; i += groups) {
        const int64_t hp = aux.long_list[i];
        const int64_t row_addr = (int64_t)(sorted[hp] >> ebits);
        const TB *row = store.old_row(row_addr);
        float old[CH][VEC], acc[CH][VEC];
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int v = li + c * lpr;
#pragma unroll
            for (int x = 0; x < VEC; ++x) {
                acc[c][x] = 0.0f;
                old[c][x] = 0.0f;
            }
            if (v < nv) VecLoad<TB, VEC>::load(row + (int64_t)v * VEC, old[c]);
        }
        // one pass over the run, lpr positions at a time: each lane fetches one word
        // (the run's end is the first position of another address), its entry's key
        // (the run's keys must not fall: checked against the lane before) and, PF
        // entries at a time, the delta pieces, added in position order.  The sum
        // assumes arrival order is key order; a run whose keys fall is summed again
        // below in exact (key, entry) order
        constexpr int PF = CH * VEC >= 64 ? 1 : (CH * VEC >= 32 ? 2 : 128 / (CH * VEC));
        int len = 0;
        bool ok = true;
        int64_t carry = INT64_MIN;                      // the key before this chunk's first position
        for (;;) {
            const int64_t at = hp + len + li;
            const uint64_t w = at < n ? sorted[at] : ~0ull;
            const bool same = at < n && (int64_t)(w >> ebits) == row_addr;
            const uint64_t stop = __ballot(!same) & mine;
            const int cnt = stop ? __ffsll((unsigned long long)(stop >> (grp * lpr))) - 1 : lpr;
            const int my_ent = li < cnt ? (int)(w & emask) : (int)n;
            if (keys) {
                const int64_t k = li < cnt ? key_of(w) : INT64_MAX;
                int64_t before = __shfl_up(k, 1, lpr);
                if (li == 0) before = carry;
                ok &= li >= cnt || k >= before;
                carry = __shfl(k, grp * lpr + (cnt > 0 ? cnt - 1 : 0));
            }
            for (int j0 = 0; j0 < cnt; j0 += PF) {
                float x[PF][CH][VEC];
                bool have[PF];
#pragma unroll
                for (int u = 0; u < PF; ++u) {
                    const int j = j0 + u;
                    const int ent = __shfl(my_ent, grp * lpr + (j < cnt ? j : 0));
                    have[u] = j < cnt && ent < n;
                    if (have[u]) {
                        const typename SRC::Entry e = src.entry(ent);
#pragma unroll
                        for (int c = 0; c < CH; ++c) {
                            const int v = li + c * lpr;
                            if (v < nv) src.template get<VEC>(e, v, old[c], x[u][c]);
                        }
                    }
                }
#pragma unroll
                for (int u = 0; u < PF; ++u) {
                    if (have[u]) {
#pragma unroll
                        for (int c = 0; c < CH; ++c) {
                            const int v = li + c * lpr;
                            if (v < nv) {
#pragma unroll
                                for (int y = 0; y < VEC; ++y) acc[c][y] += x[u][c][y];
                            }
                        }
                    }
                }
            }
            len += cnt;
            if (stop) break;
        }
        const bool in_order = (__ballot(!ok) & mine) == 0;
        if (!in_order) {
#pragma unroll
            for (int c = 0; c < CH; ++c)
#pragma unroll
                for (int x = 0; x < VEC; ++x) acc[c][x] = 0.0f;   // the run again, in (key, entry) order
            int64_t last_k = INT64_MIN, last_e = -1;
            for (int r2 = 0; r2 < len; ++r2) {
                int64_t best_k = INT64_MAX, best_e = INT64_MAX;
                for (int q = 0; q < len; ++q) {
                    const uint64_t wq = sorted[hp + q];
                    const int64_t e = (int64_t)(wq & emask);
                    const int64_t k = key_of(wq);
                    const bool after = k > last_k || (k == last_k && e > last_e);
                    const bool before = k < best_k || (k == best_k && e < best_e);
                    if (after && before) { best_k = k; best_e = e; }
                }
                add_delta(best_e, old, acc);
                last_k = best_k;
                last_e = best_e;
            }
        }
        TB *dst = store.new_row(row_addr, li, hp);
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int v = li + c * lpr;
            if (v < nv) {
#pragma unroll
                for (int x = 0; x < VEC; ++x) old[c][x] = old[c][x] + acc[c][x];
                VecStore<TB, VEC>::store(dst + (int64_t)v * VEC, old[c]);
            }
        }
    }
}

template <typename TB, int VEC, typename SRC, typename ROWS>
static int launch_segment_ch(const ROWS &store, int64_t rows, int64_t D, const int64_t *keys, const SRC &src,
                             const uint64_t *sorted, int64_t n, int ebits, const RowPlan &p,
                             int64_t *unique_out, const SegAux &lr, hipStream_t st)
{
    // window: 64 positions per wave when that still makes GLSDM_SEG_WAVES waves,
    // shorter for small commits (so they fill the chip), never below one
    // position per lane group
    const int groups = 64 / p.lpr;
    int win = 64;
    while (win > groups && ceil_div(n, win) < GLSDM_SEG_WAVES) win >>= 1;
    const dim3 grid((unsigned)ceil_div(n, 4 * win)), block(256);
    auto *u = reinterpret_cast<unsigned long long *>(unique_out);
    // mid-sized windows (commits of a few 10^4 entries, where skewed runs cross many
    // windows): runs that cross a window go to long_run_kernel, at most one per
    // window.  Full windows see few, short crossings; in tiny windows (tiny
    // commits) nearly every repeated address crosses, and the second launch costs
    // more than it saves (measured)
    const bool defer = win >= 8 && win < 64;
    const int64_t windows = ceil_div(n, win);
    const dim3 lgrid((unsigned)std::max<int64_t>(1, std::min<int64_t>(ceil_div(windows, 4 * groups), 4096)));
#define GLSDM_SEG_LAUNCH(C)                                                                                 \
    if (defer) {                                                                                              \
        hipLaunchKernelGGL((segment_kernel<TB, SRC, ROWS, VEC, C, true>), grid, block, 0, st, store, rows, D,  \
                           keys, src, sorted, n, ebits, p.nv, p.lpr, win, u, lr);                             \
        if ((rc = check_launch("segment_kernel"))) return rc;                                                 \
        hipLaunchKernelGGL((long_run_kernel<TB, SRC, ROWS, VEC, C>), lgrid, block, 0, st, store, D, keys, src, \
                           sorted, n, ebits, p.nv, p.lpr, lr);                                                \
    } else {                                                                                                  \
        hipLaunchKernelGGL((segment_kernel<TB, SRC, ROWS, VEC, C, false>), grid, block, 0, st, store, rows, D, \
                           keys, src, sorted, n, ebits, p.nv, p.lpr, win, u, lr);                             \
    }
    int rc;
    switch (p.ch) {
    case 1: GLSDM_SEG_LAUNCH(1); break;
    case 2: GLSDM_SEG_LAUNCH(2); break;
    case 3:
    case 4: GLSDM_SEG_LAUNCH(4); break;
    default: GLSDM_SEG_LAUNCH(8); break;
    }
#undef GLSDM_SEG_LAUNCH
    return check_launch("long_run_kernel");
}

// One vector width for bank and delta rows: the wider element type's 16-byte
// vector when D and the row pointers allow it, else scalar accesses.
template <typename TB, typename TD, typename SRC, typename ROWS>
static int launch_segment_rows(const ROWS &store, uintptr_t row_bits, int64_t rows, int64_t D, const int64_t *keys,
                               const SRC &src, const void *delta_rows, const uint64_t *sorted, int64_t n,
                               int ebits, int64_t *unique_out, const SegAux &lr, hipStream_t st)
{
    constexpr int VEC = 16 / (sizeof(TB) > sizeof(TD) ? sizeof(TB) : sizeof(TD));
    const bool aligned = ((row_bits | reinterpret_cast<uintptr_t>(delta_rows)) & 15) == 0;
    if (D % VEC == 0 && aligned) {
        RowPlan p{VEC, (int)(D / VEC), 0, 0};
        p.lpr = pow2_ceil(p.nv) < 64 ? pow2_ceil(p.nv) : 64;
        p.ch = (int)ceil_div(p.nv, p.lpr);
        return launch_segment_ch<TB, VEC>(store, rows, D, keys, src, sorted, n, ebits, p, unique_out, lr, st);
    }
    RowPlan p{1, (int)D, D < 64 ? pow2_ceil(D) : 64, (int)ceil_div(D, 64)};
    return launch_segment_ch<TB, 1>(store, rows, D, keys, src, sorted, n, ebits, p, unique_out, lr, st);
}

// The bank itself as the row store.
template <typename TB, typename TD, typename SRC>
static int launch_segment_t(void *bank, int64_t rows, int64_t D, const int64_t *keys, const SRC &src,
                            const void *delta_rows, const uint64_t *sorted, int64_t n, int ebits,
                            int64_t *unique_out, const SegAux &lr, hipStream_t st)
{
    return launch_segment_rows<TB, TD>(DenseRows<TB>{static_cast<TB *>(bank), D}, reinterpret_cast<uintptr_t>(bank),
                                       rows, D, keys, src, delta_rows, sorted, n, ebits, unique_out, lr, st);
}

}  // namespace glsdm

using namespace glsdm;

static int address_bits(int64_t rows)
{
    int b = 0;                         // bits for the values 0 .. rows (rows = "out of range")
    while (((int64_t)1 << b) <= rows) ++b;
    return b;
}

extern "C" int glsdm_commit_workspace_bytes(int64_t entries, int64_t rows, size_t *bytes)
{
    if (!bytes) return fail(GLSDM_ERR_ARG, "commit_workspace_bytes: null output");
    if (entries < 0 || rows < 1) return fail(GLSDM_ERR_ARG, "commit_workspace_bytes: bad arguments");
    if (entries > MAX_ENTRIES) return fail(GLSDM_ERR_UNSUPPORTED, "commit: more than 2^30 entries");
    if (entries > 0 && address_bits(rows) + entry_bits(entries) > 64)
        return fail(GLSDM_ERR_UNSUPPORTED, "commit: address bits %d + entry bits %d exceed 64", address_bits(rows),
                    entry_bits(entries));
    *bytes = entries == 0 ? 0 : plan_workspace(nullptr, entries, pass_count(address_bits(rows))).bytes;
    return GLSDM_OK;
}

// Shape checks shared by both commit entry points; entries > 0.
static int check_commit(const char *what, int64_t rows, int64_t D, int64_t entries)
{
    if (entries > MAX_ENTRIES) return fail(GLSDM_ERR_UNSUPPORTED, "%s: more than 2^30 entries", what);
    if (D > 512 && D % 8 != 0)
        return fail(GLSDM_ERR_UNSUPPORTED, "%s: D=%lld not a multiple of 8 above 512", what, (long long)D);
    if (D > 64 * 8 * 4) return fail(GLSDM_ERR_UNSUPPORTED, "%s: D=%lld above 2048", what, (long long)D);
    if (address_bits(rows) + entry_bits(entries) > 64)
        return fail(GLSDM_ERR_UNSUPPORTED, "%s: address bits %d + entry bits %d exceed 64", what,
                    address_bits(rows), entry_bits(entries));
    return GLSDM_OK;
}

// Steps 1-3 of the pipeline: the packed (address, entry) words sorted by
// address, in *sorted (one of the workspace word buffers); *long_runs is
// another, free one, for the segment step's deferred runs.
// Where commit_sort leaves the sorted words and the deferred-run list for
// (rows, entries): a function of the shape alone, so a later call (the apply
// step) finds them without state.
static void sort_result(const CommitWorkspace &ws, int passes, const uint64_t **sorted, SegAux *aux)
{
#if GLSDM_BUCKET_SORT
    if (passes >= 3) {
        *sorted = ws.c;
        *aux = SegAux{reinterpret_cast<int64_t *>(ws.a), ws.counter + CW_LONG, ws.counter + CW_ERROR};
        return;
    }
#endif
    // LSD passes ping-pong a -> b -> a ...; c is free for the deferred runs
    *sorted = passes % 2 == 0 ? ws.a : ws.b;
    *aux = SegAux{reinterpret_cast<int64_t *>(ws.c), ws.counter + CW_LONG, ws.counter + CW_ERROR};
}

static int commit_sort(int64_t rows, const int64_t *addresses, int64_t entries, void *workspace,
                       size_t workspace_bytes, const char *what, const uint64_t **sorted, int *ebits_out,
                       SegAux *long_runs, hipStream_t st)
{
    const int ebits = entry_bits(entries), abits = address_bits(rows);
    const int passes = pass_count(abits);
    CommitWorkspace ws = plan_workspace(workspace, entries, passes);
    if (!workspace || workspace_bytes < ws.bytes)
        return fail(GLSDM_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, %zu given", what, ws.bytes,
                    workspace_bytes);
    int rc;
#if GLSDM_BUCKET_SORT
    if (passes >= 3) {
        // each tile orders its words by the top address digit (-> b, pieces in the
        // look-back words' space), then each bucket gathers its pieces and sorts them (-> c)
        // top digit: bits [real - 8, real) of the address, real = the bits of rows - 1
        const int real = address_bits(rows - 1);
        const int msd = ebits + real - RADIX_BITS;
        const int lpasses = (real - RADIX_BITS + RADIX_BITS - 1) / RADIX_BITS;
        const bool pow2 = (rows & (rows - 1)) == 0;      // the sentinel `rows` clamps into the last bucket
        const int last = pow2 ? (real + 1 + RADIX_BITS - 1) / RADIX_BITS : lpasses;
        hipLaunchKernelGGL(tile_bucket_kernel, dim3((unsigned)ws.bucket_tiles), dim3(BT_THREADS), 0, st, addresses,
                           rows, ebits, msd, entries, ws.b, ws.status, ws.bucket_tiles, ws.counter);
        if ((rc = check_launch("tile_bucket_kernel"))) return rc;
        hipLaunchKernelGGL(bucket_sort_kernel, dim3(RADIX), dim3(BK_THREADS), 0, st, ws.b, ws.status, ws.bucket_tiles,
                           entries, ws.a, ws.c, ebits, lpasses, last, ws.counter + CW_ERROR);
        if ((rc = check_launch("bucket_sort_kernel"))) return rc;
        sort_result(ws, passes, sorted, long_runs);
        *ebits_out = ebits;
        return GLSDM_OK;
    }
#endif
    const unsigned prep_blocks = (unsigned)std::max<int64_t>(
        std::min<int64_t>(ceil_div((int64_t)ws.status_words, 256), 4096), (MAX_PASSES * RADIX) / 256);
    hipLaunchKernelGGL(commit_prep_kernel, dim3(prep_blocks), dim3(256), 0, st, ws.ghist, ws.status,
                       (int64_t)ws.status_words, ws.counter);
    const unsigned pack_blocks = (unsigned)std::min<int64_t>(ceil_div(entries, 256), GLSDM_PACK_BLOCKS);
    hipLaunchKernelGGL(pack_hist_kernel, dim3(pack_blocks), dim3(256), 0, st, addresses, rows, ebits, ebits, passes,
                       entries, ws.a, ws.ghist);
    if ((rc = check_launch("commit pack"))) return rc;

    uint64_t *src = ws.a, *dst = ws.b;
    for (int p = 0; p < passes; ++p) {
        hipLaunchKernelGGL(onesweep_kernel, dim3((unsigned)ws.tiles), dim3(SORT_THREADS), 0, st, src, dst, entries,
                           ebits + p * RADIX_BITS, ws.ghist + p * RADIX,
                           ws.status + (size_t)p * ws.tiles * RADIX, ws.counter + p, ws.counter + CW_ERROR,
                           g_spin_limit.load(std::memory_order_relaxed));
        if ((rc = check_launch("onesweep_kernel"))) return rc;
        uint64_t *t = src; src = dst; dst = t;
    }
    sort_result(ws, passes, sorted, long_runs);
    if (*sorted != src) return fail(GLSDM_ERR_ARG, "%s: internal sort buffer mismatch", what);
    *ebits_out = ebits;
    return GLSDM_OK;
}

template <typename TB, typename TD>
static int segment_stored(void *bank, int64_t rows, int64_t D, const int64_t *keys, const void *deltas,
                          const uint64_t *sorted, int64_t n, int ebits, int64_t *unique_out, const SegAux &lr,
                          hipStream_t st)
{
    const StoredDeltas<TD> src{static_cast<const TD *>(deltas), D};
    return launch_segment_t<TB, TD>(bank, rows, D, keys, src, deltas, sorted, n, ebits, unique_out, lr, st);
}

static int commit_apply(void *bank, int32_t bank_dtype, int64_t rows, int64_t D, const void *deltas,
                        int32_t delta_dtype, const int64_t *keys, int64_t entries, const uint64_t *sorted, int ebits,
                        int64_t *unique_out, const SegAux &lr, hipStream_t st)
{
    if (bank_dtype == GLSDM_F32 && delta_dtype == GLSDM_F32)
        return segment_stored<float, float>(bank, rows, D, keys, deltas, sorted, entries, ebits, unique_out, lr, st);
    if (bank_dtype == GLSDM_F32 && delta_dtype == GLSDM_BF16)
        return segment_stored<float, bf16_t>(bank, rows, D, keys, deltas, sorted, entries, ebits, unique_out, lr, st);
    if (bank_dtype == GLSDM_BF16 && delta_dtype == GLSDM_F32)
        return segment_stored<bf16_t, float>(bank, rows, D, keys, deltas, sorted, entries, ebits, unique_out, lr, st);
    return segment_stored<bf16_t, bf16_t>(bank, rows, D, keys, deltas, sorted, entries, ebits, unique_out, lr, st);
}

extern "C" int glsdm_commit(void *bank, int32_t bank_dtype, int64_t rows, int64_t D,
                            const int64_t *addresses, const void *deltas, int32_t delta_dtype,
                            const int64_t *keys, int64_t entries, void *workspace, size_t workspace_bytes,
                            int64_t *unique_out, void *stream)
{
    if (rows < 1 || D < 1 || entries < 0) return fail(GLSDM_ERR_ARG, "commit: bad shape rows=%lld D=%lld entries=%lld", (long long)rows, (long long)D, (long long)entries);
    if (!dtype_ok(bank_dtype) || !dtype_ok(delta_dtype)) return fail(GLSDM_ERR_ARG, "commit: bad dtype");
    if (entries == 0) return GLSDM_OK;
    int rc = check_commit("commit", rows, D, entries);
    if (rc) return rc;
    if (!bank || !addresses || !deltas) return fail(GLSDM_ERR_ARG, "commit: null pointer");
    const hipStream_t st = as_stream(stream);
    const uint64_t *sorted = nullptr;
    int ebits = 0;
    SegAux lr{nullptr, nullptr, nullptr};
    if ((rc = commit_sort(rows, addresses, entries, workspace, workspace_bytes, "commit", &sorted, &ebits, &lr, st)))
        return rc;
    return commit_apply(bank, bank_dtype, rows, D, deltas, delta_dtype, keys, entries, sorted, ebits, unique_out,
                        lr, st);
}

extern "C" int glsdm_commit_prepare(int64_t rows, const int64_t *addresses, int64_t entries, void *workspace,
                                    size_t workspace_bytes, void *stream)
{
    if (rows < 1 || entries < 0) return fail(GLSDM_ERR_ARG, "commit_prepare: bad shape");
    if (entries == 0) return GLSDM_OK;
    int rc = check_commit("commit_prepare", rows, 1, entries);
    if (rc) return rc;
    if (!addresses) return fail(GLSDM_ERR_ARG, "commit_prepare: null pointer");
    const uint64_t *sorted = nullptr;
    int ebits = 0;
    SegAux lr{nullptr, nullptr, nullptr};
    return commit_sort(rows, addresses, entries, workspace, workspace_bytes, "commit_prepare", &sorted, &ebits, &lr,
                       as_stream(stream));
}

extern "C" int glsdm_commit_apply(void *bank, int32_t bank_dtype, int64_t rows, int64_t D, const void *deltas,
                                  int32_t delta_dtype, const int64_t *keys, int64_t entries, void *workspace,
                                  size_t workspace_bytes, int64_t *unique_out, void *stream)
{
    if (rows < 1 || D < 1 || entries < 0) return fail(GLSDM_ERR_ARG, "commit_apply: bad shape");
    if (!dtype_ok(bank_dtype) || !dtype_ok(delta_dtype)) return fail(GLSDM_ERR_ARG, "commit_apply: bad dtype");
    if (entries == 0) return GLSDM_OK;
    int rc = check_commit("commit_apply", rows, D, entries);
    if (rc) return rc;
    if (!bank || !deltas) return fail(GLSDM_ERR_ARG, "commit_apply: null pointer");
    const int passes = pass_count(address_bits(rows));
    const CommitWorkspace ws = plan_workspace(workspace, entries, passes);
    if (!workspace || workspace_bytes < ws.bytes)
        return fail(GLSDM_ERR_WORKSPACE, "commit_apply: workspace of %zu bytes needed, %zu given", ws.bytes,
                    workspace_bytes);
    const uint64_t *sorted = nullptr;
    SegAux lr{nullptr, nullptr, nullptr};
    sort_result(ws, passes, &sorted, &lr);
    return commit_apply(bank, bank_dtype, rows, D, deltas, delta_dtype, keys, entries, sorted, entry_bits(entries),
                        unique_out, lr, as_stream(stream));
}

extern "C" int glsdm_commit_proposals(void *bank, int32_t bank_dtype, int64_t rows, int64_t D,
                                      const int64_t *addresses, const int64_t *keys, int64_t entries, int32_t width,
                                      const float *weights, const float *error, const float *decay,
                                      const float *mass, int64_t heads, void *workspace, size_t workspace_bytes,
                                      int64_t *unique_out, void *stream)
{
    if (rows < 1 || D < 1 || entries < 0 || width < 1 || heads < 1)
        return fail(GLSDM_ERR_ARG, "commit_proposals: bad shape rows=%lld D=%lld entries=%lld width=%d heads=%lld",
                    (long long)rows, (long long)D, (long long)entries, (int)width, (long long)heads);
    if (!dtype_ok(bank_dtype)) return fail(GLSDM_ERR_ARG, "commit_proposals: bad dtype");
    if (entries % width != 0 || (entries / width) % heads != 0)
        return fail(GLSDM_ERR_ARG, "commit_proposals: %lld entries are not whole rows of width %d and %lld heads",
                    (long long)entries, (int)width, (long long)heads);
    if (entries == 0) return GLSDM_OK;
    int rc = check_commit("commit_proposals", rows, D, entries);
    if (rc) return rc;
    if (!bank || !addresses || !weights || !error || !decay || !mass)
        return fail(GLSDM_ERR_ARG, "commit_proposals: null pointer");
    const hipStream_t st = as_stream(stream);
    const uint64_t *sorted = nullptr;
    int ebits = 0;
    SegAux lr{nullptr, nullptr, nullptr};
    if ((rc = commit_sort(rows, addresses, entries, workspace, workspace_bytes, "commit_proposals", &sorted,
                          &ebits, &lr, st)))
        return rc;
    const ProposalTerms src{error, decay, weights, mass, D, (uint32_t)width, (uint32_t)heads};
    if (bank_dtype == GLSDM_F32)
        return launch_segment_t<float, float>(bank, rows, D, keys, src, error, sorted, entries, ebits,
                                              unique_out, lr, st);
    return launch_segment_t<bf16_t, float>(bank, rows, D, keys, src, error, sorted, entries, ebits, unique_out,
                                           lr, st);
}

extern "C" int glsdm_read_backward_rows(float *grad_bank, int64_t rows, int64_t D, const int64_t *addresses,
                                        int64_t entries, int32_t width, const float *weights,
                                        const float *grad_out, void *workspace, size_t workspace_bytes,
                                        void *stream)
{
    if (rows < 1 || D < 1 || entries < 0 || width < 1)
        return fail(GLSDM_ERR_ARG, "read_backward_rows: bad shape rows=%lld D=%lld entries=%lld width=%d",
                    (long long)rows, (long long)D, (long long)entries, (int)width);
    if (entries % width != 0)
        return fail(GLSDM_ERR_ARG, "read_backward_rows: %lld entries are not whole rows of width %d",
                    (long long)entries, (int)width);
    if (entries == 0) return GLSDM_OK;
    int rc = check_commit("read_backward_rows", rows, D, entries);
    if (rc) return rc;
    if (!grad_bank || !addresses || !weights || !grad_out) return fail(GLSDM_ERR_ARG, "read_backward_rows: null pointer");
    const hipStream_t st = as_stream(stream);
    const uint64_t *sorted = nullptr;
    int ebits = 0;
    SegAux lr{nullptr, nullptr, nullptr};
    if ((rc = commit_sort(rows, addresses, entries, workspace, workspace_bytes, "read_backward_rows", &sorted,
                          &ebits, &lr, st)))
        return rc;
    const ReadGradTerms src{weights, grad_out, D, (uint32_t)width};
    return launch_segment_t<float, float>(grad_bank, rows, D, nullptr, src, grad_out, sorted, entries, ebits,
                                          nullptr, lr, st);
}

extern "C" int glsdm_overlay_commit(const void *base, int32_t dtype, int64_t B, int64_t H, int64_t S, int64_t D,
                                    int32_t *map, void *pool, int64_t capacity, int64_t pool_offset,
                                    const int64_t *addresses, const void *deltas, int32_t delta_dtype,
                                    const int64_t *keys, int64_t entries, void *workspace, size_t workspace_bytes,
                                    int64_t *unique_out, void *stream)
{
    if (B < 1 || H < 1 || S < 1 || D < 1 || entries < 0 || capacity < 0 || pool_offset < 0)
        return fail(GLSDM_ERR_ARG, "overlay_commit: bad shape");
    if (!dtype_ok(dtype) || !dtype_ok(delta_dtype)) return fail(GLSDM_ERR_ARG, "overlay_commit: bad dtype");
    if (capacity > INT32_MAX) return fail(GLSDM_ERR_UNSUPPORTED, "overlay_commit: capacity above 2^31-1 rows");
    if (entries == 0) return GLSDM_OK;
    if (pool_offset + entries > capacity)
        return fail(GLSDM_ERR_ARG, "overlay_commit: pool rows [%lld, %lld) exceed capacity %lld",
                    (long long)pool_offset, (long long)(pool_offset + entries), (long long)capacity);
    const int64_t rows = B * H * S;
    int rc = check_commit("overlay_commit", rows, D, entries);
    if (rc) return rc;
    if (!base || !map || !pool || !addresses || !deltas) return fail(GLSDM_ERR_ARG, "overlay_commit: null pointer");
    const hipStream_t st = as_stream(stream);
    const uint64_t *sorted = nullptr;
    int ebits = 0;
    SegAux lr{nullptr, nullptr, nullptr};
    if ((rc = commit_sort(rows, addresses, entries, workspace, workspace_bytes, "overlay_commit", &sorted, &ebits,
                          &lr, st)))
        return rc;
    const uintptr_t row_bits = reinterpret_cast<uintptr_t>(base) | reinterpret_cast<uintptr_t>(pool);
#define GLSDM_OVERLAY(TB, TD)                                                                                  \
    {                                                                                                         \
        const OverlayRows<TB> ov{static_cast<const TB *>(base), map, static_cast<TB *>(pool), D, H * S,       \
                                 pool_offset};                                                                \
        const StoredDeltas<TD> src{static_cast<const TD *>(deltas), D};                                       \
        return launch_segment_rows<TB, TD>(ov, row_bits, rows, D, keys, src, deltas, sorted, entries, ebits,  \
                                           unique_out, lr, st);                                               \
    }
    if (dtype == GLSDM_F32 && delta_dtype == GLSDM_F32) GLSDM_OVERLAY(float, float)
    if (dtype == GLSDM_F32) GLSDM_OVERLAY(float, bf16_t)
    if (delta_dtype == GLSDM_F32) GLSDM_OVERLAY(bf16_t, float)
    GLSDM_OVERLAY(bf16_t, bf16_t)
#undef GLSDM_OVERLAY
}

// ------------------------------------------------------------ allocation-free commit
//
// glsdm_commit_noalloc runs glsdm_commit's kernels with their workspace in a
// file-scope device array instead of a caller buffer, for callers that cannot
// allocate.  Each GPU holds its own copy of the array from module load until
// the process ends; host code addresses it only through the per-device pointer
// that hipGetSymbolAddress returns (the array's name on the host is not a
// device address).  Calls on one GPU share the array, so calls that overlap
// on one GPU race; every call clears the words it needs before use.
constexpr int64_t NOALLOC_MAX_ENTRIES = (int64_t)1 << 19;      // the workspace then fits in 13 MiB, any rows
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)16 << 20;

__device__ __attribute__((aligned(256))) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

constexpr int NOALLOC_MAX_DEVICES = 64;
static std::mutex g_scratch_mutex;
static void *g_scratch_ptr[NOALLOC_MAX_DEVICES];

// The current device's copy of the scratch array (looked up once per device).
static int scratch_address(void **out)
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(GLSDM_ERR_HIP, "commit_noalloc: hipGetDevice failed");
    if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) return fail(GLSDM_ERR_UNSUPPORTED, "commit_noalloc: device %d", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(GLSDM_ERR_HIP, "commit_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return GLSDM_OK;
}

extern "C" int glsdm_commit_noalloc(void *bank, int32_t bank_dtype, int64_t rows, int64_t D,
                                    const int64_t *addresses, const void *deltas, int32_t delta_dtype,
                                    const int64_t *keys, int64_t entries, int64_t *unique_out, void *stream)
{
    if (rows < 1 || D < 1 || entries < 0)
        return fail(GLSDM_ERR_ARG, "commit_noalloc: bad shape rows=%lld D=%lld entries=%lld", (long long)rows,
                    (long long)D, (long long)entries);
    if (entries > NOALLOC_MAX_ENTRIES)
        return fail(GLSDM_ERR_UNSUPPORTED, "commit_noalloc: %lld entries exceed the static scratch's limit of %lld",
                    (long long)entries, (long long)NOALLOC_MAX_ENTRIES);
    if (entries == 0) return GLSDM_OK;
    int rc = check_commit("commit_noalloc", rows, D, entries);
    if (rc) return rc;
    const size_t need = plan_workspace(nullptr, entries, pass_count(address_bits(rows))).bytes;
    if (need > NOALLOC_SCRATCH_BYTES)
        return fail(GLSDM_ERR_UNSUPPORTED, "commit_noalloc: %zu scratch bytes needed, %zu available", need,
                    NOALLOC_SCRATCH_BYTES);
    void *ws = nullptr;
    if ((rc = scratch_address(&ws))) return rc;
    return glsdm_commit(bank, bank_dtype, rows, D, addresses, deltas, delta_dtype, keys, entries, ws,
                        NOALLOC_SCRATCH_BYTES, unique_out, stream);
}

extern "C" int glsdm_commit_status(const void *workspace, size_t workspace_bytes, int64_t entries, int64_t rows,
                                   int64_t *status, void *stream)
{
    if (!status) return fail(GLSDM_ERR_ARG, "commit_status: null output");
    if (rows < 1 || entries < 0) return fail(GLSDM_ERR_ARG, "commit_status: bad shape");
    const uint32_t *counter = nullptr;
    if (entries > 0) {
        int rc = check_commit("commit_status", rows, 1, entries);
        if (rc) return rc;
        if (!workspace) {                    // the status of glsdm_commit_noalloc on this device
            void *ws = nullptr;
            if ((rc = scratch_address(&ws))) return rc;
            workspace = ws;
            workspace_bytes = NOALLOC_SCRATCH_BYTES;
        }
        const CommitWorkspace ws = plan_workspace(const_cast<void *>(workspace), entries,
                                                  pass_count(address_bits(rows)));
        if (!workspace || workspace_bytes < ws.bytes)
            return fail(GLSDM_ERR_WORKSPACE, "commit_status: workspace of %zu bytes needed, %zu given", ws.bytes,
                        workspace_bytes);
        counter = ws.counter;
    }
    hipLaunchKernelGGL(commit_status_kernel, dim3(1), dim3(64), 0, as_stream(stream), counter, status);
    return check_launch("commit_status_kernel");
}

extern "C" int glsdm_debug_force_lookback_timeout(int32_t on)
{
    g_spin_limit.store(on ? 0u : LB_SPIN_LIMIT, std::memory_order_relaxed);
    return GLSDM_OK;
}
