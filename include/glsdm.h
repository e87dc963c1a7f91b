/*
 * glsdm.h -- C ABI of libglsdm.so, the MI355X (gfx950) implementation of
 * GL-SDM's transactional sparse-memory operator: product-key routing, snapshot
 * read and the deterministic buffered commit.
 *
 * Reference citations use S/ = projects/gl-sdm/src/gl_sdm/ in kreasof-ai/GL-SDM.
 *
 * Conventions (every entry point):
 *   - Plain pointers to device memory and sizes; no C++ or framework types.
 *   - Returns GLSDM_OK (0) or a negative status; glsdm_last_error() then holds
 *     a message (thread-local).
 *   - Asynchronous on the given HIP stream (hipStream_t passed as void*; NULL is
 *     the null stream).  No host synchronisation, no device allocation: the
 *     caller owns every buffer, including the commit workspace.
 *   - Bank / value rows are row-major [rows, D] of dtype GLSDM_F32 or
 *     GLSDM_BF16.  Index tensors are int64, weights and scores fp32.
 *   - Out-of-range slots or addresses never fault: such route entries
 *     contribute nothing to a read and such commit entries are dropped (and
 *     counted: glsdm_commit_status).  The reference's torch indexing raises on
 *     them instead; a caller that wants that checks ranges or the count.
 */
#ifndef GLSDM_H
#define GLSDM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GLSDM_OK 0
#define GLSDM_ERR_ARG (-1)         /* invalid argument or shape */
#define GLSDM_ERR_UNSUPPORTED (-2) /* valid but outside the supported envelope */
#define GLSDM_ERR_WORKSPACE (-3)   /* workspace missing or too small */
#define GLSDM_ERR_HIP (-4)         /* a HIP runtime call failed */

#define GLSDM_F32 0
#define GLSDM_BF16 1

/* Tie rule for equal scores.  HIGHEST: the larger sub-key / slot index wins
 * (the chunk path, S/memory/routing.py:4,15-17,21-23).  LOWEST: the smaller
 * index wins (the token path, S/layers/router.py:45-55). */
#define GLSDM_TIE_HIGHEST 0
#define GLSDM_TIE_LOWEST 1

/* Library version string. */
const char *glsdm_version(void);

/* Message for the last non-zero status returned on this thread. */
const char *glsdm_last_error(void);

/*
 * Product-key route of fp32 or bf16 factor scores.
 *   scores  [rows, 2*half] of scores_dtype (GLSDM_F32 or GLSDM_BF16): factor 0 in
 *           columns [0, half), factor 1 in [half, 2*half).  bf16 scores route exactly
 *           as the same values widened to fp32 (the reference's .float() of the bf16
 *           router projection, S/layers/global_layer.py:26,42).
 *   index   [rows, width] int64 out: chosen slots i*half + j, ascending
 *   weights [rows, width] fp32 out: softmax of the chosen slots' summed scores
 *   workspace (optional, may be NULL): glsdm_route_workspace_bytes() bytes, 8-byte
 *           aligned; with it, launches of few rows (decode) split each factor's
 *           columns over more blocks.  Results are identical either way.
 * Per row: per factor the min(width, half) best sub-keys, their grid of fp32
 * sums, the best `width` grid cells, ascending slot order, softmax.
 * Envelope: 1 <= half <= 65535, 1 <= width <= 64, width <= half*half.
 * Replaces: the route half of S/memory/routing.py:10-26 (torch_routed_read) and
 * of S/memory/backends/urm.py:109-122 (routed_snapshot_read), with tie HIGHEST;
 * S/memory/backends/token.py:85-114 (_Route / route) and S/layers/router.py:39-61, with
 * tie LOWEST.
 */
int glsdm_route(const void *scores, int32_t scores_dtype, int64_t rows, int32_t half, int32_t width,
                int32_t tie, int64_t *index, float *weights, void *workspace, size_t workspace_bytes,
                void *stream);

/*
 * Workspace bytes for glsdm_route / glsdm_route_read on `rows` rows (0 when the
 * single-kernel path already fills the GPU).  No counterpart in the reference
 * (its routes allocate internally); sized on the host, no device work.
 */
int glsdm_route_workspace_bytes(int64_t rows, int32_t half, int32_t width, size_t *bytes);

/*
 * Snapshot read from supplied routes.
 *   bank    [B, H, S, D] of bank_dtype (flattened rows (b*H + h)*S + slot)
 *   index   [B, T, H, width] int64 local slots in [0, S); weights same shape fp32
 *   out     [B, T, H, D] of out_dtype: sum_j weights[j] * bank_row[j], fp32 accumulation
 * Envelope: D <= 64 * 8 * (16 / sizeof(bank element)) when D is a multiple of the
 * 16-byte vector, D <= 512 otherwise; width <= 1024.
 * Replaces: S/memory/routing.py:27-28 (weighted gather of torch_routed_read),
 * S/memory/backends/urm.py:64-82 (snapshot_read) and the native branch of
 * S/memory/transactions.py:28-35 (read).
 */
int glsdm_read(const void *bank, int32_t bank_dtype, int64_t B, int64_t H, int64_t S, int64_t D,
               int64_t T, int32_t width, const int64_t *index, const float *weights,
               void *out, int32_t out_dtype, void *stream);

/*
 * glsdm_read with one route entry per lane group in flight (glsdm_read keeps up to
 * four): the same arguments and the same bits, slower alone (config 2: 38 vs 32 us)
 * but small enough (at most 32 VGPRs for 16-byte row pieces) that its waves leave
 * each SIMD room for a wave of the fused route kernel, for a read that runs while
 * another stream routes.  No counterpart in the reference (its read is one torch
 * gather); for callers that overlap reading with routing on two streams.
 */
int glsdm_read_narrow(const void *bank, int32_t bank_dtype, int64_t B, int64_t H, int64_t S, int64_t D,
                      int64_t T, int32_t width, const int64_t *index, const float *weights,
                      void *out, int32_t out_dtype, void *stream);

/*
 * Route then read (glsdm_route followed by glsdm_read on the same stream).
 *   scores [B, T, H, 2*half] of scores_dtype (fp32 or bf16) with half*half == S;
 *   workspace as glsdm_route, for rows = B*T*H.
 * Replaces: S/memory/backends/urm.py:109-122 (routed_snapshot_read) and
 * S/memory/routing.py:10-28 (torch_routed_read).
 */
int glsdm_route_read(const void *bank, int32_t bank_dtype, int64_t B, int64_t H, int64_t S,
                     int64_t D, int64_t T, const void *scores, int32_t scores_dtype, int32_t width,
                     int32_t tie, void *out, int32_t out_dtype, int64_t *index, float *weights,
                     void *workspace, size_t workspace_bytes, void *stream);

/*
 * Address scoring on bf16 MFMA: scores[b,t,h,c] = sum_e queries[b,t,h,e] * subkeys[h,c,e]
 * with fp32 accumulation, c in [0, 2*half).  queries [B,T,H,dk] bf16,
 * subkeys [H, 2*half, dk] bf16, scores [B,T,H,2*half] fp32 out.
 * Envelope: dk a multiple of 32, 2*half a multiple of 64.
 * Replaces: the factor-score projection feeding routed_read,
 * S/layers/global_layer.py:26 (router.q) and :42 (router.k), in its per-head
 * sub-key form.
 */
int glsdm_score(const void *queries, const void *subkeys, int64_t B, int64_t T, int64_t H,
                int32_t dk, int32_t half, float *scores, void *stream);

/*
 * Fused scoring + route: the factor scores of glsdm_score are produced on MFMA
 * and fed to the glsdm_route selection through LDS, without an HBM round trip.
 *   queries [B,T,H,dk] bf16, subkeys [H, 2*half, dk] bf16 (16-byte aligned)
 *   index [B,T,H,width] int64 out (ascending slots), weights fp32 out
 *   scores_out: NULL, or [B,T,H,2*half] fp32 to also export the scores
 *   workspace: NULL, or glsdm_score_route_workspace_bytes() bytes (8-byte
 *             aligned).  Launches with fewer token tiles than CUs (few
 *             tokens, one head) then split every factor's sub-key columns
 *             over more blocks and merge their exact partial top-k lists; the
 *             results are the same, bit for bit, with or without it.
 * Results equal glsdm_route applied to the exported scores, bit for bit.
 * Envelope: dk a multiple of 32 up to 256, half a multiple of 16, width <= 64.
 * Replaces: S/layers/global_layer.py:26-27 and :42-43 (router.q/k projection
 * followed by routing.routed_read's route, S/memory/routing.py:10-26).
 */
int glsdm_score_route(const void *queries, const void *subkeys, int64_t B, int64_t T, int64_t H,
                      int32_t dk, int32_t half, int32_t width, int32_t tie, float *scores_out,
                      int64_t *index, float *weights, void *workspace, size_t workspace_bytes,
                      void *stream);

/*
 * Fused scoring + route that also emits the route's proposal addresses and
 * collision keys: glsdm_score_route followed by glsdm_proposal_keys with the
 * same (position_offset, chunk, layers, layer), in one launch.
 *   addresses [B,T,H,width] int64 out: (b*H + h)*half*half + slot
 *   keys      [B,T,H,width] int64 out: address*chunk*layers + (position_offset + t)*layers + layer
 * Replaces: the write route of S/layers/global_layer.py:42-43 followed by the
 * address/key construction of :45,52-53.
 */
int glsdm_score_route_keys(const void *queries, const void *subkeys, int64_t B, int64_t T, int64_t H,
                           int32_t dk, int32_t half, int32_t width, int32_t tie, int64_t position_offset,
                           int64_t chunk, int64_t layers, int64_t layer, int64_t *index, float *weights,
                           int64_t *addresses, int64_t *keys, void *workspace, size_t workspace_bytes,
                           void *stream);

/*
 * Workspace bytes glsdm_score_route can use for this shape (0: the shape
 * already fills the GPU and no workspace is used).  No counterpart in the
 * reference (which materialises the [B,T,H,2*half] scores instead).
 */
int glsdm_score_route_workspace_bytes(int64_t B, int64_t T, int64_t H, int32_t half, int32_t width,
                                      size_t *bytes);

/*
 * Bytes of workspace glsdm_commit needs for `entries` deltas into a bank of
 * `rows` rows.
 */
int glsdm_commit_workspace_bytes(int64_t entries, int64_t rows, size_t *bytes);

/*
 * Deterministic buffered commit, in place on `bank`.
 *   bank      [rows, D] of bank_dtype, updated in place
 *   addresses [entries] int64 absolute rows; entries outside [0, rows) are dropped
 *   deltas    [entries, D] of delta_dtype
 *   keys      [entries] int64 collision order, or NULL for arrival order
 *   unique_out: optional int64 device counter; the number of touched rows is
 *             added to it (NULL to skip)
 * Result: for every address a, bank[a] = round(bank[a] + s_a) where s_a is the
 * fp32 sum, starting from +0, of a's deltas in ascending (key, entry index)
 * order; round is identity for fp32 and round-to-nearest-even for bf16.  This
 * equals the reference's stable key sort followed by grouping of equal
 * consecutive addresses whenever the keys keep equal addresses together (keys =
 * addresses, or the stack's addr*(C*L) + pos*L + layer).  No floating point
 * atomics: the result is bitwise reproducible.  The keys are only read for
 * addresses with several entries.
 * Replaces: S/memory/transactions.py:69-97 (commit; torch branch order) and
 * S/memory/backends/commit.py:36-58 (_Commit.forward), without the full-bank
 * clone (callers that need the old bank copy it first).
 */
int glsdm_commit(void *bank, int32_t bank_dtype, int64_t rows, int64_t D,
                 const int64_t *addresses, const void *deltas, int32_t delta_dtype,
                 const int64_t *keys, int64_t entries, void *workspace, size_t workspace_bytes,
                 int64_t *unique_out, void *stream);

/*
 * glsdm_commit without a workspace argument, allocating nothing: its workspace
 * is a static device array of the library (16 MiB, held on every GPU the
 * library runs on until the process ends), addressed through the pointer
 * hipGetSymbolAddress returns for the calling thread's current device, which
 * must be the stream's device.  Same arguments and results as glsdm_commit,
 * bit for bit, for entries <= 2^19 (524,288, one config-2 epoch); larger
 * commits return GLSDM_ERR_UNSUPPORTED before any launch.  It calls no
 * hipMalloc or hipFree.  Calls on one GPU share the array: calls that overlap
 * on one GPU (several streams or threads) race and must be serialised by the
 * caller.  Status: glsdm_commit_status with a NULL workspace.
 * No counterpart in the reference; it is for callers that cannot allocate
 * (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc).
 */
int glsdm_commit_noalloc(void *bank, int32_t bank_dtype, int64_t rows, int64_t D,
                         const int64_t *addresses, const void *deltas, int32_t delta_dtype,
                         const int64_t *keys, int64_t entries, int64_t *unique_out, void *stream);

/*
 * glsdm_commit in two steps: glsdm_commit_prepare groups the entries by address
 * (the sort; it reads only the addresses, never the bank) into the workspace,
 * and glsdm_commit_apply, later on any stream ordered after it, runs the
 * segmented sums and the read-modify-write of the touched rows from that
 * workspace.  The pair with the same (rows, entries, workspace) equals
 * glsdm_commit bit for bit; the workspace must not be reused in between.  A
 * pipelined caller can sort epoch e+1's entries while epoch e's commit updates
 * the bank (the sort does not depend on the bank).
 * Replaces: the stable key sort + unique_consecutive of
 * S/memory/transactions.py:89-91 (prepare) and the segment_reduce + index_copy
 * of :92-96 (apply).
 */
int glsdm_commit_prepare(int64_t rows, const int64_t *addresses, int64_t entries, void *workspace,
                         size_t workspace_bytes, void *stream);
int glsdm_commit_apply(void *bank, int32_t bank_dtype, int64_t rows, int64_t D, const void *deltas,
                       int32_t delta_dtype, const int64_t *keys, int64_t entries, void *workspace,
                       size_t workspace_bytes, int64_t *unique_out, void *stream);

/*
 * Status of the last commit-family call (glsdm_commit, glsdm_commit_apply,
 * glsdm_commit_proposals, glsdm_read_backward_rows, glsdm_overlay_commit) made
 * with this workspace and these (entries, rows), written to status (int64[2],
 * device memory) on the stream after it, without a host synchronisation:
 *   status[0]: the sort's error flags -- 0, or bit 0 (a bounded look-back wait
 *              gave up) / bit 1 (inconsistent bucket pieces); when non-zero the
 *              call wrote no bank row;
 *   status[1]: the number of entries dropped for an address outside [0, rows).
 * entries == 0 reports zeros (no workspace needed).  workspace NULL: the status
 * of the last glsdm_commit_noalloc on the calling thread's current device.
 * No counterpart in the reference: its sort cannot fail and its torch indexing
 * raises on an out-of-range address (flat[unique] and index_copy of
 * S/memory/transactions.py:96); a caller that wants that behaviour raises on
 * status[1] != 0, or checks the addresses first.
 */
int glsdm_commit_status(const void *workspace, size_t workspace_bytes, int64_t entries, int64_t rows,
                        int64_t *status, void *stream);

/*
 * Test hook: on != 0 makes every look-back wait of the commit sort give up at
 * once (commits into fewer than 65536 rows, whose sort uses look-back passes),
 * so that a test can drive the failure path from the host and check that it
 * leaves the bank untouched and is reported by glsdm_commit_status; 0 restores
 * the normal bounded wait.  Process-wide.  No counterpart in the reference.
 */
int glsdm_debug_force_lookback_timeout(int32_t on);

/*
 * Absolute addresses (b*H + h)*S + index[b,t,h,j] for index [B,T,H,width].
 * Replaces: S/memory/routing.py:31-34 (absolute_addresses) and
 * S/memory/transactions.py:13-16 (addresses, with requests = arange(B)).
 */
int glsdm_absolute_addresses(const int64_t *index, int64_t B, int64_t T, int64_t H,
                             int32_t width, int64_t S, int64_t *out, void *stream);

/*
 * Write addresses and collision keys of one proposal, index [B,T,H,width]:
 *   addresses = (b*H + h)*S + index[b,t,h,j]
 *   keys      = addresses*(chunk*layers) + (position_offset + t)*layers + layer
 * so collisions order by (address, position in the chunk, layer).
 * Replaces: S/layers/global_layer.py:45 (absolute_addresses) and :52-53
 * (keys = addresses * (chunk_size * num_layers) + positions * num_layers + layer_idx).
 */
int glsdm_proposal_keys(const int64_t *index, int64_t B, int64_t T, int64_t H, int32_t width,
                        int64_t S, int64_t position_offset, int64_t chunk, int64_t layers,
                        int64_t layer, int64_t *addresses, int64_t *keys, void *stream);

/*
 * Row gather out[i] = bank[addresses[i]] for n addresses; out has bank_dtype.
 * Replaces: S/memory/routing.py:37-42 (gather_rows) and
 * S/memory/backends/primitives.py:15-20 (_gather).
 */
int glsdm_gather_rows(const void *bank, int32_t bank_dtype, int64_t rows, int64_t D,
                      const int64_t *addresses, int64_t n, void *out, void *stream);

/*
 * Per-row terms of a write proposal, for R proposal rows (r = token*H + h):
 *   decay[r]    = exp(log_decay[r])
 *   error[r, :] = beta[r] * (target[r, :] - decay[r] * prediction[r, :])
 * prediction [R, D] fp32 (the routed read of the write route), target [R, D]
 * of target_dtype, beta/log_decay [R] fp32; outputs error [R, D] fp32 and
 * decay [R] fp32.  Separate fp32 operations in the reference's order.
 * Replaces: the decay and error lines of S/runtime/dense.py:12-13
 * (proposal_delta), whose operands S/layers/global_layer.py:42-50 builds.
 */
int glsdm_proposal_error(int64_t R, int64_t D, const float *prediction, const void *target,
                         int32_t target_dtype, const float *beta, const float *log_decay,
                         float *error, float *decay, void *stream);

/*
 * One write proposal appended to a proposal log (preallocated per-chunk
 * buffers that the fused commit later reads as one proposal), for the
 * B*T*H proposal rows r = (b*T + t)*H + h of a [B, T, H, width] write route:
 *   error [R, D] fp32, decay [R] fp32:   glsdm_proposal_error of the row, with
 *       beta = sigmoid(b) = 1 / (1 + exp(-b)) and log_decay = -softplus(d - 4)
 *       (softplus(v) = v above 20, else log1p(exp(v))) from beta_in / decay_in
 *       [R] (the beta and decay projections' outputs, of gate_dtype);
 *   addresses, keys [R*width] int64:    glsdm_proposal_keys of index;
 *   weights_out [R*width] fp32:         a copy of the route weights.
 * The output pointers are the log's buffers at its current fill; index
 * [B,T,H,width] int64, weights the same shape fp32, prediction [R, D] fp32,
 * target [R, D] of target_dtype.  Bitwise equal to write gates +
 * glsdm_proposal_keys + glsdm_proposal_error.
 * Replaces: the proposal construction of S/layers/global_layer.py:45-54 (gates
 * :48-49, keys :52-53) and the per-row terms of S/runtime/dense.py:12-13; the
 * list of proposals the reference concatenates at its commit
 * (S/memory/transactions.py:73-79) becomes the log's buffers.
 */
int glsdm_proposal_append(const int64_t *index, const float *weights, const float *prediction,
                          const void *target, int32_t target_dtype, const void *beta_in, const void *decay_in,
                          int32_t gate_dtype, int64_t B, int64_t T, int64_t H, int32_t width, int64_t S,
                          int64_t D, int64_t position_offset, int64_t chunk, int64_t layers, int64_t layer,
                          int64_t *addresses, int64_t *keys, float *weights_out, float *error, float *decay,
                          void *stream);

/*
 * Materialised write-proposal deltas, for R proposal rows of `width` entries:
 *   deltas[r, j, :] = mass[r / heads] * ((decay[r] - 1) * rows[r, j, :]
 *                                        + weights[r, j] * error[r, :])
 * with decay and error as in glsdm_proposal_error.  rows [R, width, D] of
 * rows_dtype (the gathered snapshot rows), weights [R, width] fp32, mass
 * [R / heads] fp32 (one value per token), deltas [R, width, D] fp32.
 * Replaces: S/runtime/dense.py:11-14 (proposal_delta), with rows, weights,
 * prediction, target, beta, log_decay and mass of shapes [..., H, k, D],
 * [..., H, k], [..., H, D], [..., H, D], [..., H, 1], [..., H, 1], [...].
 */
int glsdm_proposal_delta(const void *rows, int32_t rows_dtype, int64_t R, int32_t width, int64_t D,
                         const float *weights, const float *prediction, const void *target,
                         int32_t target_dtype, const float *beta, const float *log_decay,
                         const float *mass, int64_t heads, float *deltas, void *stream);

/*
 * Fused proposal -> commit, in place on `bank`: glsdm_commit of the deltas
 *   delta[e, :] = mass[r / heads] * ((decay[r] - 1) * bank[addresses[e], :]
 *                                    + weights[e] * error[r, :]),  r = e / width,
 * evaluated inside the commit from each touched row's value before the
 * commit, so the deltas [entries, D] are never stored.  error/decay come from
 * glsdm_proposal_error; weights [entries] fp32, mass [entries / width / heads].
 * entries must be a multiple of width * heads.  The result is bitwise that of
 * glsdm_proposal_delta on the gathered rows followed by glsdm_commit, when the
 * bank is the snapshot the proposal gathered its rows from (the reference
 * commits only against that version: S/memory/transactions.py:72-73).
 * Several proposals (layers) of equal width and heads are committed together
 * by concatenating their entries, rows of error/decay, and mass.
 * Workspace: glsdm_commit_workspace_bytes(entries, rows).
 * Replaces: S/runtime/dense.py:11-14 (proposal_delta) with
 * S/layers/global_layer.py:44 (gather_rows) feeding
 * S/memory/transactions.py:69-97 (commit) through S/layers/stack.py:65.
 */
int glsdm_commit_proposals(void *bank, int32_t bank_dtype, int64_t rows, int64_t D,
                           const int64_t *addresses, const int64_t *keys, int64_t entries, int32_t width,
                           const float *weights, const float *error, const float *decay,
                           const float *mass, int64_t heads, void *workspace, size_t workspace_bytes,
                           int64_t *unique_out, void *stream);

/*
 * Backward of the route: the factor-score gradient of a route's weights.
 *   index [rows, width] int64 (slots), weights [rows, width] fp32 (the route's
 *   softmax), grad_weights [rows, width] fp32 in; grad_scores [rows, 2*half]
 *   fp32 out: with g_j = w_j * (gw_j - sum_v w_v gw_v), column c < half is the
 *   sum of g_j over the picks with slot / half == c, column half + c the sum
 *   over the picks with slot % half == c (in pick order), 0 elsewhere.
 * Replaces: S/memory/backends/token.py:69-82 (_route_backward) and the autograd
 * of S/memory/routing.py:10-26 (torch_routed_read's route).
 */
int glsdm_route_backward(const int64_t *index, const float *weights, const float *grad_weights,
                         int64_t rows, int32_t half, int32_t width, float *grad_scores, void *stream);

/*
 * Backward of the snapshot read w.r.t. its weights:
 *   grad_weights[b,t,h,j] = sum_d grad_out[b,t,h,d] * bank[b,h,index[b,t,h,j],d]
 * (fp32; bank [B,H,S,D] of bank_dtype; out-of-range slots give 0).
 * Replaces: the weights' gradient in the autograd of S/memory/routing.py:27-28
 * ((rows * weights).sum(-2)) and URM's read backward (S/memory/backends/urm.py).
 */
int glsdm_read_backward_weights(const void *bank, int32_t bank_dtype, int64_t B, int64_t H, int64_t S,
                                int64_t D, int64_t T, int32_t width, const int64_t *index,
                                const float *grad_out, float *grad_weights, void *stream);

/*
 * Backward of the snapshot read w.r.t. the bank rows, accumulated in place:
 *   grad_bank[addresses[e]] += weights[e] * grad_out[e / width]
 * for every in-range entry, each address's terms summed from +0 in entry order
 * and then added once (no float atomics; deterministic).  grad_bank [rows, D]
 * fp32; addresses [entries] int64 absolute rows of grad_bank (e.g. those of
 * glsdm_absolute_addresses, or h*S + slot to fold the requests' replicas into
 * one [H,S,D] gradient); weights [entries]; grad_out [entries / width, D].
 * Workspace: glsdm_commit_workspace_bytes(entries, rows).
 * Replaces: the accumulating index backward of S/memory/routing.py:42
 * (flat[address]) in the autograd of the read, without the dense full-bank
 * gradient the reference's read backward materialises per call.
 */
int glsdm_read_backward_rows(float *grad_bank, int64_t rows, int64_t D, const int64_t *addresses,
                             int64_t entries, int32_t width, const float *weights, const float *grad_out,
                             void *workspace, size_t workspace_bytes, void *stream);

/*
 * Overlay snapshots: B requests' banks as one immutable base [H, S, D] (dtype)
 * plus, per request, an int32 slot map [B, H, S] (-1: the base row) into a pool
 * of touched rows [capacity, D] (dtype).  Logical row (b, h, slot) is
 * pool[map[b,h,slot]] when mapped, else base[h, slot].  Storage grows with the
 * touched rows instead of B full replicas, and a commit writes only its touched
 * rows; every result equals that of the dense [B, H, S, D] bank bit for bit.
 * Replaces: the per-request clones of S/memory/state.py:61-62 (snapshot) and the
 * full-bank functional copy of S/memory/transactions.py:96 (commit), following
 * the overlay plan of P/OPTIMIZATION_PLAN.md:114-120 (P/ = projects/gl-sdm/).
 */

/* glsdm_read on the logical bank of an overlay. */
int glsdm_overlay_read(const void *base, int32_t dtype, const int32_t *map, const void *pool, int64_t B,
                       int64_t H, int64_t S, int64_t D, int64_t T, int32_t width, const int64_t *index,
                       const float *weights, void *out, int32_t out_dtype, void *stream);

/*
 * glsdm_commit on the logical bank of an overlay, in place: a touched row's old
 * value comes from its pool row or the base, its new value goes to its pool
 * row.  A row written for the first time takes pool row pool_offset + p, with p
 * its address run's position among the sorted entries (no atomics; the pool
 * layout is deterministic), so each commit uses pool rows
 * [pool_offset, pool_offset + entries): the caller passes the previous
 * commit's pool_offset + entries and sizes the pool accordingly
 * (pool_offset + entries <= capacity, checked).  addresses are absolute rows
 * (b*H + h)*S + slot; keys as glsdm_commit.
 * Workspace: glsdm_commit_workspace_bytes(entries, B*H*S).
 */
int glsdm_overlay_commit(const void *base, int32_t dtype, int64_t B, int64_t H, int64_t S, int64_t D,
                         int32_t *map, void *pool, int64_t capacity, int64_t pool_offset,
                         const int64_t *addresses, const void *deltas, int32_t delta_dtype,
                         const int64_t *keys, int64_t entries, void *workspace, size_t workspace_bytes,
                         int64_t *unique_out, void *stream);

/* The logical bank [B, H, S, D] of an overlay, written densely to out. */
int glsdm_overlay_materialise(const void *base, int32_t dtype, const int32_t *map, const void *pool,
                              int64_t B, int64_t H, int64_t S, int64_t D, void *out, void *stream);

/*
 * QK normalisation and rotary positions of a local attention layer, fused:
 * per head row x (dk elements at x + r*row_stride, r = (b*T + t)*heads + h),
 * y = x*rsqrt(mean(x^2) + FLT_EPSILON) rounded to dtype, then with
 * a = y[:dk/2], b = y[dk/2:], theta_j = (offset + t)*freq[j] (fp32, freq has
 * dk/2 entries): cat(a cos + b sin, -a sin + b cos) rounded to dtype, written
 * to out [B, heads, T, dk] contiguous.  dk a power of two in [4, 256];
 * offset + T <= 2^24.
 * Replaces: F.rms_norm(q|k, (head_dim,)) and Transformer.rotary, then
 * .transpose(1, 2), of S/layers/attention.py:38-42,51-52.
 */
int glsdm_qk_norm_rotary(const void *x, int32_t dtype, int64_t B, int64_t T, int64_t heads, int64_t dk,
                         int64_t row_stride, const float *freq, int64_t offset, void *out, void *stream);

/*
 * A local layer's decode-step preparation in one launch: glsdm_qk_norm_rotary of
 * the q rows (q + ((b*T + t)*q_heads + h)*q_row_stride) into q_out [B, q_heads,
 * T, dk] contiguous, of the k rows (same addressing with kv_heads, k_row_stride)
 * into k_dst, and a copy of the v rows (v_row_stride) into v_dst, where element
 * d of (b, h, t) of k_dst / v_dst is at b*s[0] + h*s[1] + t*s[2] + d for
 * s = dst_strides (the KV window buffers' slices for the new positions).
 * Bit-identical to two glsdm_qk_norm_rotary calls and the two copies; limits
 * as glsdm_qk_norm_rotary.
 * Replaces: S/layers/attention.py:38-42,51-52 (q/k norm and rotary) and the
 * cache concatenation of S/layers/attention.py:55 for a decode step.
 */
int glsdm_decode_qkv(const void *q, int64_t q_row_stride, int64_t q_heads, const void *k, int64_t k_row_stride,
                     const void *v, int64_t v_row_stride, int64_t kv_heads, int32_t dtype, int64_t B, int64_t T,
                     int64_t dk, const float *freq, int64_t offset, void *q_out, void *k_dst, void *v_dst,
                     const int64_t *dst_strides, void *stream);

/*
 * The gated attention output: out[b, t, h*dk + i] = o[b, h, t, i] *
 * sigmoid(gate[b, t, h, i]) (sigmoid in fp32 rounded to dtype, then the
 * product rounded to dtype), o [B, H, T, dk] and gate [B, T, H, dk] read
 * through their element strides (4 each, last one 1), out [B, T, H*dk]
 * contiguous.
 * Replaces: out.transpose(1, 2).reshape(B, T, D) * gate.reshape(B, T, D).sigmoid()
 * of S/layers/attention.py:77.
 */
int glsdm_gate_merge(const void *o, const int64_t *o_strides, const void *gate, const int64_t *gate_strides,
                     int32_t dtype, int64_t B, int64_t T, int64_t H, int64_t dk, void *out, void *stream);

/*
 * The MLP activation: with u, g the halves of each row of fc [rows, 2*inner],
 * out [rows, inner] = g * relu(u)^2 (the square rounded to dtype, then the
 * product rounded to dtype).  inner a multiple of 16 bytes' worth of
 * elements; fc and out 16-byte aligned.
 * Replaces: u, gate = fc(x).chunk(2, -1); gate * u.relu().square() of
 * S/layers/common.py:26-27.
 */
int glsdm_relu2_gate(const void *fc, int32_t dtype, int64_t rows, int64_t inner, void *out, void *stream);

/*
 * A bf16 projection of at most 64 rows (decode):
 *   out [M, N] = bf16(sum_k x[m, k] * weight[n, k] + bias[n]), fp32 accumulation
 *   rounded once (round-to-nearest-even); bias may be NULL.
 * M <= 64, N a multiple of 16, K a multiple of 128; x and weight 16-byte aligned
 * (GLSDM_ERR_UNSUPPORTED otherwise, nothing launched).  The fp32 summation order
 * is the kernel's own: results agree with torch's bf16 linear to the rounding of
 * the fp32 sum.
 * Replaces: the nn.Linear projections of S/layers/attention.py:23-26,
 * S/layers/common.py:22-23, S/layers/router.py:23-28 and the head of
 * S/model.py:45 for decode-sized inputs (torch.nn.functional.linear).
 */
int glsdm_linear_small(const void *x, const void *weight, const void *bias, void *out, int64_t M, int64_t N,
                       int64_t K, void *stream);

/*
 * glsdm_linear_small followed by the residual add, in one launch:
 *   out [M, N] = residual [M, N] + float(bf16(x . weight^T + bias)), fp32, the
 * bits of torch's x + linear(h) for an fp32 x and a bf16 projection; out may be
 * residual itself.  Requirements as glsdm_linear_small.
 * Replaces: the residual adds after the mixer and MLP projections,
 * S/baselines/block.py:25-26 and S/layers/global_layer.py:29-30, for
 * decode-sized inputs.
 */
int glsdm_linear_small_residual(const void *x, const void *weight, const void *bias, const float *residual,
                                float *out, int64_t M, int64_t N, int64_t K, void *stream);

/*
 * The MLP's down projection with its activation formed as the operand is loaded:
 * for h [M, 2K] bf16 (the fc output; u = h[:, :K], gate = h[:, K:]) the operand is
 * a = bf16(gate * bf16(relu(u)^2)) (glsdm_relu2_gate's roundings), then
 *   residual NULL: out [M, N] bf16 = glsdm_linear_small of a;
 *   otherwise:     out [M, N] fp32 = residual + float(that), as glsdm_linear_small_residual.
 * Bit-identical to glsdm_relu2_gate followed by that call.  Requirements as
 * glsdm_linear_small with K the inner width (h 16-byte aligned).
 * Replaces: gate * x.relu().square() and self.proj of S/layers/common.py:26-27
 * (and the residual add after the MLP, S/baselines/block.py:26,
 * S/layers/global_layer.py:30) for decode-sized inputs.
 */
int glsdm_linear_small_relu2(const void *h, const void *weight, const void *bias, const float *residual, void *out,
                             int64_t M, int64_t N, int64_t K, void *stream);

/*
 * glsdm_linear_small for up to 8 projections of one input in one launch:
 *   outs[i] [M, N[i]] = bf16(x . weights[i]^T + biases[i]), i < count,
 * each with glsdm_linear_small's requirements and bit-identical to it (biases may
 * be NULL, or any biases[i] NULL).
 * Replaces: the projections of one input, S/layers/attention.py:23-25 (q, k, v of
 * a local layer) and S/layers/router.py:25-27 (v, beta, decay of a global layer's
 * write), for decode-sized inputs.
 */
int glsdm_linear_small_group(const void *x, int32_t count, const void *const *weights, const void *const *biases,
                             void *const *outs, const int64_t *N, int64_t M, int64_t K, void *stream);

/*
 * One-token attention of the local layer's decode step, bf16:
 *   out [B, H, 1, dk] = softmax(q . k_j * scale) . v_j over the L keys of each
 *   (b, h), q [B, H, 1, dk] contiguous, k/v [B, H, L, dk] read through
 *   k_strides/v_strides (elements, for the b, h and key dimensions; unit stride
 *   within a row).  fp32 scores, exponentials and sums, the output rounded once.
 * No mask: for one query whose keys all lie inside its window.  L <= 1024,
 * dk 64 or 128, q and key rows 16-byte aligned (GLSDM_ERR_UNSUPPORTED otherwise).
 * Replaces: F.scaled_dot_product_attention of S/layers/attention.py:76 for a
 * decode step (T = 1).
 */
int glsdm_decode_attention(const void *q, const void *k, const void *v, void *out, int64_t B, int64_t H, int64_t L,
                           int64_t dk, const int64_t *k_strides, const int64_t *v_strides, float scale, void *stream);

/*
 * glsdm_decode_attention with the local layer's output gate applied to each
 * output row: out[b, h, d] = bf16(bf16(attention) * bf16(sigmoid(g))) for
 * g = gate[b*gate_strides[0] + h*gate_strides[1] + d] (bf16; sigmoid = 1/(1 +
 * exp(-g)) in fp32), written as [B, H*dk] -- the input of proj for one token.
 * Bit-identical to glsdm_decode_attention followed by glsdm_gate_merge.
 * Replaces: S/layers/attention.py:76-77 (attention and the gate before proj)
 * for a decode step.
 */
int glsdm_decode_attention_gated(const void *q, const void *k, const void *v, const void *gate, void *out,
                                 int64_t B, int64_t H, int64_t L, int64_t dk, const int64_t *k_strides,
                                 const int64_t *v_strides, const int64_t *gate_strides, float scale, void *stream);

/*
 * RMSNorm then a cast: per row of x [rows, dim] (x_dtype), r =
 * rsqrt(mean(x^2) + eps), y = (x*r)*w in fp32 rounded to x_dtype (w [dim] of
 * w_dtype, rounded to x_dtype first), y written as out_dtype to out [rows, dim].
 * Replaces: RMSNorm.forward (S/layers/common.py:7-17) followed by .to(dtype)
 * in the blocks (S/baselines/block.py, S/layers/global_layer.py:23-31).
 */
int glsdm_rms_norm_cast(const void *x, int32_t x_dtype, const void *weight, int32_t w_dtype, int64_t rows,
                        int64_t dim, float eps, void *out, int32_t out_dtype, void *stream);

/*
 * The write gates of a proposal from the beta and decay projections' outputs
 * (n values each, dtype): beta = sigmoid(b), log_decay = -softplus(d - 4)
 * (softplus(v) = v above 20, else log1p(exp(v))), fp32 [n] each.
 * Replaces: router.beta(dense).float().sigmoid() and
 * -F.softplus(router.decay(dense).float() - 4) of S/layers/global_layer.py:48-49.
 */
int glsdm_write_gates(const void *beta_in, const void *decay_in, int32_t dtype, int64_t n, float *beta,
                      float *log_decay, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* GLSDM_H */
