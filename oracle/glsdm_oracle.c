/*
 * Scalar C restatement of the GL-SDM memory operator -- CPU oracle.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py through oracle/c_oracle.py.  The product library
 * (libglsdm.so) never links or calls it.
 *
 * The algorithm is the reference's, restated with explicit loops instead of
 * torch ops (S/ = projects/gl-sdm/src/gl_sdm/):
 *   oracle_route   S/memory/routing.py:10-26 (tie 0 = highest slot wins)
 *                  S/layers/router.py:39-61  (tie 1 = lowest slot wins)
 *                  An element's rank is the composite key
 *                  (monotone fp32 score bits) << 32 | tie bits of its index,
 *                  which is exactly the order the reference's chain of stable
 *                  argsorts produces; -0 is folded onto +0 (torch compares them
 *                  equal) and every NaN ranks above +inf (torch's sort order).
 *   oracle_read    S/memory/routing.py:27-28  sum_j w_j * row_j, fp32, j ascending
 *   oracle_commit  S/memory/transactions.py:89-96 and
 *                  S/memory/backends/commit.py:22-33: stable sort by key, then
 *                  per run of equal addresses an fp32 sum from 0 in sorted
 *                  order, then old + sum.
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no FMA contraction).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static uint32_t order_bits(float x)
{
    uint32_t b;
    if (x != x) return 0xFFFFFFFFu;   /* NaN: above +inf, all NaNs tie */
    if (x == 0.0f) x = 0.0f;          /* fold -0 onto +0 */
    memcpy(&b, &x, 4);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

static uint64_t rank_key(float score, uint32_t index, int tie)
{
    uint32_t t = tie == 0 ? index : 0xFFFFFFFFu - index;
    return ((uint64_t)order_bits(score) << 32) | t;
}

static int desc_u64(const void *a, const void *b)
{
    uint64_t x = *(const uint64_t *)a, y = *(const uint64_t *)b;
    return x < y ? 1 : (x > y ? -1 : 0);
}

static int asc_u32(const void *a, const void *b)
{
    uint32_t x = *(const uint32_t *)a, y = *(const uint32_t *)b;
    return x < y ? -1 : (x > y ? 1 : 0);
}

/* scores [rows, 2*half] fp32 -> index [rows, width] int64 ascending, weights fp32. */
int oracle_route(const float *scores, int64_t rows, int half, int width, int tie,
                 int64_t *index, float *weights)
{
    if (half < 1 || width < 1 || (int64_t)width > (int64_t)half * half || (tie != 0 && tie != 1))
        return -1;
    int k = width < half ? width : half;
    uint64_t *fk = malloc(sizeof(uint64_t) * (size_t)half);
    uint64_t *ck = malloc(sizeof(uint64_t) * (size_t)k * k);
    uint32_t *pick = malloc(sizeof(uint32_t) * 2 * (size_t)k);
    float *best = malloc(sizeof(float) * 2 * (size_t)k);
    uint32_t *slot = malloc(sizeof(uint32_t) * (size_t)width);
    float *logit = malloc(sizeof(float) * (size_t)width);
    if (!fk || !ck || !pick || !best || !slot || !logit) return -2;
    for (int64_t r = 0; r < rows; ++r) {
        const float *row = scores + r * 2 * (int64_t)half;
        for (int f = 0; f < 2; ++f) {
            for (int i = 0; i < half; ++i) fk[i] = rank_key(row[f * half + i], (uint32_t)i, tie);
            qsort(fk, (size_t)half, sizeof(uint64_t), desc_u64);
            for (int i = 0; i < k; ++i) {
                uint32_t lo = (uint32_t)fk[i];
                uint32_t idx = tie == 0 ? lo : 0xFFFFFFFFu - lo;
                pick[f * k + i] = idx;
                best[f * k + i] = row[f * half + idx];
            }
        }
        for (int i = 0; i < k; ++i)
            for (int j = 0; j < k; ++j) {
                float s = best[i] + best[k + j];
                uint32_t a = pick[i] * (uint32_t)half + pick[k + j];
                ck[i * k + j] = rank_key(s, a, tie);
            }
        qsort(ck, (size_t)k * k, sizeof(uint64_t), desc_u64);
        for (int w = 0; w < width; ++w) {
            uint32_t lo = (uint32_t)ck[w];
            slot[w] = tie == 0 ? lo : 0xFFFFFFFFu - lo;
        }
        qsort(slot, (size_t)width, sizeof(uint32_t), asc_u32);
        float m = -INFINITY;
        for (int w = 0; w < width; ++w) {
            uint32_t i = slot[w] / (uint32_t)half, j = slot[w] % (uint32_t)half;
            logit[w] = row[i] + row[half + j];
            if (logit[w] > m || logit[w] != logit[w]) m = logit[w];
        }
        float total = 0.0f;
        for (int w = 0; w < width; ++w) { logit[w] = expf(logit[w] - m); total += logit[w]; }
        for (int w = 0; w < width; ++w) {
            index[r * width + w] = slot[w];
            weights[r * width + w] = logit[w] / total;
        }
    }
    free(fk); free(ck); free(pick); free(best); free(slot); free(logit);
    return 0;
}

/* bank [B,H,S,D] fp32; index/weights [B,T,H,width]; out [B,T,H,D] fp32. */
int oracle_read(const float *bank, int64_t B, int64_t H, int64_t S, int64_t D, int64_t T,
                int width, const int64_t *index, const float *weights, float *out)
{
    for (int64_t b = 0; b < B; ++b)
        for (int64_t t = 0; t < T; ++t)
            for (int64_t h = 0; h < H; ++h) {
                int64_t r = (b * T + t) * H + h;
                float *o = out + r * D;
                for (int64_t d = 0; d < D; ++d) o[d] = 0.0f;
                for (int w = 0; w < width; ++w) {
                    int64_t slot = index[r * width + w];
                    if (slot < 0 || slot >= S) return -1;
                    const float *row = bank + ((b * H + h) * S + slot) * D;
                    float wt = weights[r * width + w];
                    for (int64_t d = 0; d < D; ++d) o[d] += row[d] * wt;
                }
            }
    return 0;
}

static void merge_sort_by_key(int64_t *ord, int64_t *tmp, const int64_t *key, int64_t n)
{
    /* bottom-up stable merge sort of entry ids by key */
    for (int64_t i = 0; i < n; ++i) ord[i] = i;
    for (int64_t width = 1; width < n; width *= 2) {
        for (int64_t lo = 0; lo < n; lo += 2 * width) {
            int64_t mid = lo + width < n ? lo + width : n;
            int64_t hi = lo + 2 * width < n ? lo + 2 * width : n;
            int64_t a = lo, b = mid, o = lo;
            while (a < mid && b < hi) tmp[o++] = key[ord[b]] < key[ord[a]] ? ord[b++] : ord[a++];
            while (a < mid) tmp[o++] = ord[a++];
            while (b < hi) tmp[o++] = ord[b++];
        }
        memcpy(ord, tmp, sizeof(int64_t) * (size_t)n);
    }
}

/* In-place commit of E deltas [E,D] fp32 into bank [rows,D] fp32.
 * keys == NULL means keys = addresses.  Returns the number of touched rows. */
int64_t oracle_commit(float *bank, int64_t rows, int64_t D, const int64_t *addr,
                      const float *deltas, const int64_t *keys, int64_t E)
{
    if (E < 1) return 0;
    const int64_t *k = keys ? keys : addr;
    int64_t *ord = malloc(sizeof(int64_t) * (size_t)E);
    int64_t *tmp = malloc(sizeof(int64_t) * (size_t)E);
    float *acc = malloc(sizeof(float) * (size_t)D);
    if (!ord || !tmp || !acc) return -2;
    for (int64_t e = 0; e < E; ++e)
        if (addr[e] < 0 || addr[e] >= rows) { free(ord); free(tmp); free(acc); return -1; }
    merge_sort_by_key(ord, tmp, k, E);
    int64_t unique = 0;
    for (int64_t p = 0; p < E;) {
        int64_t a = addr[ord[p]];
        for (int64_t d = 0; d < D; ++d) acc[d] = 0.0f;
        while (p < E && addr[ord[p]] == a) {
            const float *x = deltas + ord[p] * D;
            for (int64_t d = 0; d < D; ++d) acc[d] += x[d];
            ++p;
        }
        float *row = bank + a * D;
        for (int64_t d = 0; d < D; ++d) row[d] = row[d] + acc[d];
        ++unique;
    }
    free(ord); free(tmp); free(acc);
    return unique;
}

/* Factor scores of the per-head sub-key form: scores[(n*H + h)*L + c] =
 * sum_e q[(n*H + h)*dk + e] * keys[(h*L + c)*dk + e], fp32, e ascending.
 * (The contraction S/layers/global_layer.py:26,42 computes with router.q/k.) */
void oracle_score(const float *q, const float *keys, int64_t N, int64_t H, int64_t dk, int64_t L,
                  float *scores)
{
    for (int64_t n = 0; n < N; ++n)
        for (int64_t h = 0; h < H; ++h) {
            const float *x = q + (n * H + h) * dk;
            float *out = scores + (n * H + h) * L;
            for (int64_t c = 0; c < L; ++c) {
                const float *k = keys + (h * L + c) * dk;
                float s = 0.0f;
                for (int64_t e = 0; e < dk; ++e) s += x[e] * k[e];
                out[c] = s;
            }
        }
}
