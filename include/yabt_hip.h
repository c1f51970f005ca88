/*
 * yabt_hip.h -- C ABI of the gfx950 tree-growing library (libyabt_hip.so).
 *
 * Drop-in for the native boundary of YABT's C grower: the reference loads
 * yabt/_cgrow/grow.c through ctypes (yabt/grow_c.py:154-200, 412-426) and calls
 * `cgrow` / `capply`.  This library exports the same operations on device
 * memory (HIP), plus the per-stage kernels so each can be tested alone.
 *
 * Conventions
 *   - every pointer is device memory unless stated; sizes are plain integers;
 *   - calls are asynchronous on `stream` (hipStream_t, 0 = null stream);
 *   - return 0 on success, < 0 on a rejected argument or launch failure; the
 *     message is available from yabt_last_error() (per calling thread);
 *   - histograms are exact int64 fixed point: the caller's grad/hess are
 *     quantised as q = rint(x * 2^s) with one shift per channel and call,
 *     under one of two contracts (k = ceil(log2(n)), max|x| < 2^e, s = 0 if
 *     max|x| = 0):
 *       narrow: s = 30 - min(k, 11) - e; q keeps 19 bits of the largest |x|
 *         (more for n <= 2048) and any 2048 values sum below 2^31 in
 *         magnitude (the streaming root histogram packs q(g) and q(h) into
 *         one 64-bit word per update);
 *       wide: s = 61 - max(k, 21) - e; q keeps 37 bits of the largest |x| at
 *         10M rows (40 at <= 2M rows), g and h a 64-bit word each;
 *     calls that choose the shifts themselves take narrow only when its
 *     quantisation residual sum |x - q 2^-s| is at most 2^-17 of sum |x|
 *     for both g and h (exact integer sums, so the choice is deterministic),
 *     else wide; every sum over <= n rows is exact either way;
 *   - bin counts: the count plane of a root histogram depends only on the
 *     bins, so callers that keep them for a whole fit pass the table
 *     yabt_bin_counts made for these bins and this n as `bin_counts`
 *     (yabt_bin_counts_words(n, F) uint32: the (F, 256) counts, then the
 *     per-segment maxima that let the root skip its packed cells' epochs);
 *     NULL makes the call count them itself (one more pass over the
 *     feature-major bins);
 *   - bins: feature-major (F, ld_fm) uint8 with ld_fm >= n, ld_fm % 16 == 0,
 *     and a row-major copy (n, ld_rm) uint8 with ld_rm >= F, ld_rm % 16 == 0
 *     (yabt_transpose_bins builds it); bins, grad, hess 16-byte aligned.
 */
#ifndef YABT_HIP_H
#define YABT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t *yabt_stream_t; /* == hipStream_t */

/* Last error message of the calling thread ("" if none).
 * Replaces: the RuntimeError text of yabt/grow_c.py:236-238. */
const char *yabt_last_error(void);

/* Bytes of device workspace yabt_grow needs for (n, F, max_leaves). */
size_t yabt_grow_workspace_bytes(int64_t n, int F, int max_leaves);

/* Grow one best-first tree.  Replaces `int cgrow(...)` (yabt/_cgrow/grow.c:243-250,
 * ctypes signature yabt/grow_c.py:168-200; caller yabt/grow_c.py:412-426).
 * Same parameters and the same node-array outputs (each of length
 * 2*max_leaves+1, device memory); differences:
 *   - bins come in both layouts (bins_fm, bins_rm) instead of `binned` (F,n);
 *   - the sparse CSR arguments of cgrow are replaced by `default_bin` (F int32,
 *     may be NULL): rows in a feature's default bin are not accumulated and
 *     that bin is restored as node total minus the other bins, which with
 *     exact integer sums gives the dense histogram bit for bit (the sparse
 *     builder's default-bin fill, grow.c:68-107, made exact).  Any bin is a
 *     correct choice; the most frequent one saves the most work;
 *   - B (always 256) and n_threads are dropped;
 *   - `bin_counts` (may be NULL): the per-fit counts of the bins (above);
 *   - `workspace` (>= yabt_grow_workspace_bytes) replaces cgrow's mallocs;
 *   - the node count is written to out_status[0] on the device (cgrow's return
 *     value); out_status[0] = -1 if grad or hess holds a non-finite value.
 * Requires 0 <= n < 2^32, F >= 1, 1 <= max_leaves <= 32767. */
int yabt_grow(const uint8_t *bins_fm, int64_t ld_fm, const uint8_t *bins_rm, int64_t ld_rm,
              const float *grad, const float *hess, const uint8_t *fmask, const float *imat,
              float ib, int use_imat, const int32_t *nbins, const int32_t *default_bin,
              const uint32_t *bin_counts, int64_t n, int F, float lam, float gamma, float mcw, int msl,
              float lr, int max_leaves,
              int max_depth, void *workspace, size_t workspace_bytes, int64_t *out_feature,
              int64_t *out_thr_bin, int64_t *out_left, int64_t *out_right, float *out_value,
              int64_t *out_depth, int32_t *out_status, yabt_stream_t stream);

/* Per-row leaf node id (int64, n) of the tree the previous yabt_grow call on
 * `workspace` grew, read from the final partition (the membership cgrow's
 * rows[] holds at grow.c:410; what yabt/boosting.py:492 recomputes with
 * Tree.apply).  feature/depth/status are that call's outputs. */
int yabt_grow_leaf_ids(void *workspace, int64_t n, int F, int max_leaves, const int64_t *feature,
                       const int64_t *depth, const int32_t *status, int64_t *out,
                       yabt_stream_t stream);

/* Row-major copy of the feature-major bins; padding columns are zero.
 * Replaces the host-side transpose of yabt/grow_c.py:364-367 (its inverse). */
int yabt_transpose_bins(const uint8_t *bins_fm, int64_t ld_fm, int64_t n, int F,
                        uint8_t *bins_rm, int64_t ld_rm, yabt_stream_t stream);

/* Route raw X (n, ldx) row-major to leaves: x[f] <= threshold goes left.
 * Replaces `void capply(...)` (yabt/_cgrow/grow.c:223-225, caller
 * yabt/grow_c.py:305-333); n_threads is dropped, n_nodes bounds the walk. */
int yabt_apply(const float *X, int64_t ldx, int64_t n, int F, const int64_t *feature,
               const float *threshold, const int64_t *left, const int64_t *right, int n_nodes,
               int64_t *out_node, yabt_stream_t stream);

/* Workspace bytes of yabt_hist. */
size_t yabt_hist_workspace_bytes(void);

/* Exact node histogram out[3][F][256] int64 = (sum q(g), sum q(h), count) over
 * the rows rows[0:m] (row-major gather; every id < n), or over all n rows when
 * rows == NULL (feature-major stream).  out_shifts[0..2] (device int32) receive
 * the shifts (sg, sh) and the contract (0 narrow, 1 wide) chosen from grad/hess.
 * Replaces `build_hist` (yabt/_cgrow/grow.c:37-62) and the CUDA `hist_build`
 * K==1 path (yabt/_cuda/hist.cu:101-125, yabt/cuda_hist.py:79-89). */
int yabt_hist(const uint8_t *bins_fm, int64_t ld_fm, const uint8_t *bins_rm, int64_t ld_rm,
              const float *grad, const float *hess, int64_t n, int F, const uint32_t *rows,
              int64_t m, void *workspace, int64_t *out, int32_t *out_shifts,
              yabt_stream_t stream);

/* yabt_hist with caller-given shifts (sg, sh) and contract (wide 0: narrow,
 * the shifts keep |x * 2^s| within the narrow bound; 1: wide, within the wide
 * bound), adding into `out` without clearing it (rows == NULL: two launches,
 * the bin counts and the streaming root histogram).  workspace: >=
 * yabt_hist_workspace_bytes() when rows != NULL, else unused.
 * Replaces `build_hist` (yabt/_cgrow/grow.c:37-62) for callers that manage
 * the quantisation themselves. */
int yabt_hist_accumulate(const uint8_t *bins_fm, int64_t ld_fm, const uint8_t *bins_rm,
                         int64_t ld_rm, const float *grad, const float *hess, int64_t n, int F,
                         const uint32_t *rows, int64_t m, int sg, int sh, int wide, void *workspace,
                         int64_t *out, yabt_stream_t stream);

/* Per-fit count table of the bins (uint32, yabt_bin_counts_words(n, F)
 * words): out_counts[f * 256 + b] = number of rows r < n with
 * bins_fm[f * ld_fm + r] == b, the count plane of every root histogram over
 * these bins; then out_counts[F * 256 + f * S + s], S = ceil(n / 65536) =
 * the largest count of any bin of feature f among rows
 * [65536 s, 65536 (s + 1)), which bounds the rows any cell of a root chunk
 * takes.  yabt_grow* and yabt_hist_root take the table as `bin_counts`.
 * Replaces nothing in the reference (cgrow counts every node's rows itself,
 * grow.c:55-60); it is the setup of the packed root histogram. */
size_t yabt_bin_counts_words(int64_t n, int F);
int yabt_bin_counts(const uint8_t *bins_fm, int64_t ld_fm, int64_t n, int F, uint32_t *out_counts,
                    yabt_stream_t stream);

/* The streaming root histogram alone: adds sum q(g) and sum q(h) over all n
 * rows (shifts sg, sh and contract `wide` given, as in yabt_hist_accumulate)
 * into planes 0 and 1 of out (3, F, 256) int64,
 * and bin_counts (may be NULL: plane 2 untouched) into plane 2 -- exactly
 * one kernel launch, which is what a timing harness brackets.  Replaces the
 * root call of `build_hist` (yabt/_cgrow/grow.c:37-62, grow.c:296-300). */
int yabt_hist_root(const uint8_t *bins_fm, int64_t ld_fm, const float *grad, const float *hess,
                   int64_t n, int F, const uint32_t *bin_counts, int sg, int sh, int wide,
                   int64_t *out, yabt_stream_t stream);

/* yabt_hist without a workspace argument, for callers that cannot allocate
 * device memory: code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc.  No counterpart in the reference (whose
 * grower mallocs its scratch per call, grow.c:271-287).  Same arguments,
 * outputs and errors as yabt_hist minus `workspace`; the call allocates
 * nothing (no hipMalloc, hipFree or allocating library routine).  Its
 * scratch (the quantisation record and the gather job) is a static device
 * array of 512 bytes per device, whatever n and F, held until the process
 * ends; the device is the current one, and `stream` must belong to it.
 * Every call on a device shares that device's array, and each call clears
 * what must start at zero with kernels (no memset nodes under capture), so
 * calls that overlap on one device -- on two streams or from two host
 * threads -- race and must be serialised by the caller. */
int yabt_hist_noalloc(const uint8_t *bins_fm, int64_t ld_fm, const uint8_t *bins_rm, int64_t ld_rm,
                      const float *grad, const float *hess, int64_t n, int F, const uint32_t *rows,
                      int64_t m, int64_t *out, int32_t *out_shifts, yabt_stream_t stream);

/* Workspace bytes of yabt_best_split for F features. */
size_t yabt_best_split_workspace_bytes(int F);

/* Best split of one exact histogram; out_gain[0] (device double) = true gain
 * or -inf, out_fb[0..1] (device int32) = (feature, bin), -1 if none.
 * boost may be NULL (all 1).  Replaces `best_split` (yabt/_cgrow/grow.c:129-197). */
int yabt_best_split(const int64_t *hist, int F, const int32_t *nbins, const uint8_t *fmask,
                    const float *boost, int sg, int sh, double lam, double gamma, double mcw,
                    int msl, void *workspace, double *out_gain, int32_t *out_fb,
                    yabt_stream_t stream);

/* Workspace bytes of yabt_partition. */
size_t yabt_partition_workspace_bytes(void);

/* Stable partition of rows_in[0:m] (NULL: the positions 0..m-1) by
 * bins_fm[f*ld_fm + row] <= b into rows_out (lefts first, each side in input
 * order); out_mid[0] (device int64) = number of left rows.  Same membership as
 * `partition_rows` (yabt/_cgrow/grow.c:201-217), whose order is unstable.
 * The caller guarantees f < F and every row id < n. */
int yabt_partition(const uint8_t *bins_fm, int64_t ld_fm, int64_t n, int f, int b,
                   const uint32_t *rows_in, int64_t m, uint32_t *rows_out, void *workspace,
                   int64_t *out_mid, yabt_stream_t stream);

/* Workspace bytes of yabt_leaf_fit for n rows, n_nodes nodes, K inputs. */
size_t yabt_leaf_fit_workspace_bytes(int64_t n, int n_nodes, int K);

/* Linear leaf models of one tree: for every leaf (feature[node] == -1) with at
 * least min_samples rows, theta = solve(M + diag(lam,..,lam,1e-8), b) with
 * x1 = [(x - mu) / sd (fp32), 1], M = sum h x1 x1^T, b = -sum g x1 over the
 * leaf's rows.  gram_mode 0: each product of the reference's fp64 factors
 * rounded once to int64 fixed point and summed exactly (order-free); 1: the same sums in
 * fp64 on the matrix cores (v_mfma_f64_16x16x4_f64, a fixed order).
 * Replaces `_fit_linear` (yabt/neural_leaves.py:42-90) and the counts and
 * envelopes of `fit_leaf_networks` (yabt/neural_leaves.py:157-176).
 *   x_kind 0: X is fp32 row-major (n, ldx), input j of row i = X[i*ldx + feats[j]];
 *   x_kind 1: X is uint8 feature-major (F, ldx >= n), input = (float)X[feats[j]*ldx + i];
 *   x_kind 2: X is fp32 feature-major (F, ldx >= n), input = X[feats[j]*ldx + i]
 *     (the same results as x_kind 0 on the transposed matrix; the row passes
 *     read four rows of a column with one 16-byte load when X is 16-byte
 *     aligned and ldx % 4 == 0);
 *   leaf_of_row (n) node ids in [0, n_nodes); mu, sd (K) fp32; 1 <= K <= 8.
 * Outputs (device): out_W (n_nodes, K) and out_b (n_nodes) in the standardised
 * inputs (zero where not fitted); out_lo/out_hi (n_nodes, K) per-node min/max of
 * the raw inputs (+inf/-inf for empty nodes); out_count (n_nodes) rows per node;
 * out_status[0] = 0, -1 (a leaf id out of range or a non-finite input) or -2
 * (a singular system, where the reference's torch.linalg.solve raises);
 * out_status[1] = the number of leaves fitted. */
int yabt_leaf_fit(int x_kind, const void *X, int64_t ldx, int64_t n, const int32_t *feats, int K,
                  const float *mu, const float *sd, const float *grad, const float *hess,
                  const int64_t *leaf_of_row, const int64_t *feature, int n_nodes, int min_samples,
                  double lam, int gram_mode, void *workspace, size_t workspace_bytes, float *out_W,
                  float *out_b, float *out_lo, float *out_hi, int64_t *out_count,
                  int32_t *out_status, yabt_stream_t stream);

/* The fold of the leaf models into raw space, in the fp32 order of the
 * reference's torch expressions: per node, acc = sum_j W[j] * (mu[j] / sd[j])
 * left to right, out_value = value_in + lr * (b - acc), out_linear[j] =
 * (lr * W[j]) / sd[j].  W (n_nodes, K) and b (n_nodes) as yabt_leaf_fit
 * writes them.  Replaces the fold of `fit_leaf_networks`
 * (yabt/neural_leaves.py:178-184). */
int yabt_leaf_fold(int n_nodes, int K, const float *W, const float *b, const float *mu,
                   const float *sd, float lr, const float *value_in, float *out_value,
                   float *out_linear, yabt_stream_t stream);

/* The leaf models' inputs: the internal nodes' features (feature[i] >= 0 of
 * n_nodes entries, 1 <= F <= 4096), most used first, equal counts in the
 * order torch's CPU argsort gives them (libstdc++'s introsort over the
 * ascending unique features), the first k (1..8) written to out_feats
 * (int64) and out_feats32; positions past the used features get 0.
 * *out_m (device) = the number of used features, -1 if a node names a
 * feature >= F.  One block on `stream`, nothing read back: a caller may
 * launch yabt_leaf_moments / yabt_leaf_fit on out_feats32 before reading
 * *out_m, and falls back when *out_m < k.  Replaces the ranking of
 * `_used_features` (yabt/neural_leaves.py:27-31). */
int yabt_leaf_rank_features(const int64_t *feature, int n_nodes, int F, int k, int64_t *out_feats,
                            int32_t *out_feats32, int32_t *out_m, yabt_stream_t stream);

/* One tree's leaf models in one call: yabt_leaf_rank_features (the first K
 * of the tree's split features, F = the features of X), yabt_leaf_moments on
 * them, yabt_leaf_fit and yabt_leaf_fold, launched back to back on `stream`
 * with nothing read back, so that the device runs the step without waiting
 * for the host between the calls (the same kernels and results as the four
 * calls).  ws_moments and ws_fit: the workspaces of yabt_leaf_moments and
 * yabt_leaf_fit; out_feats, out_feats32 as yabt_leaf_rank_features; out_mu,
 * out_sd as yabt_leaf_moments; out_W .. out_count as yabt_leaf_fit;
 * out_value, out_linear as yabt_leaf_fold; out_status (3): [0] and [1] as
 * yabt_leaf_fit, [2] the number of used features (yabt_leaf_rank_features'
 * out_m: the results hold only when it is >= K).  Replaces the sequence of
 * `fit_leaf_networks` (yabt/neural_leaves.py:131-184) for one tree. */
int yabt_leaf_step(int x_kind, const void *X, int64_t ldx, int64_t n, int F, int K, const float *grad,
                   const float *hess, const int64_t *leaf_of_row, const int64_t *feature,
                   const float *value_in, int n_nodes, int min_samples, double lam, float lr,
                   int gram_mode, void *ws_moments, size_t ws_moments_bytes, void *ws_fit,
                   size_t ws_fit_bytes, int64_t *out_feats, int32_t *out_feats32, float *out_mu,
                   float *out_sd, float *out_W, float *out_b, float *out_lo, float *out_hi,
                   int64_t *out_count, float *out_value, float *out_linear, int32_t *out_status,
                   yabt_stream_t stream);

/* Workspace bytes of yabt_leaf_moments for n rows. */
size_t yabt_leaf_moments_workspace_bytes(int64_t n);

/* Standardisation of the leaf-model inputs: out_mu[j] = mean, out_sd[j] =
 * max(unbiased std, 1e-6) of input j over the n rows (fp32 results of fp64
 * sums reduced in a fixed order).  Same inputs as yabt_leaf_fit.  Replaces
 * `Xs.mean(dim=0)`, `Xs.std(dim=0).clamp_min(1e-6)` (yabt/neural_leaves.py:152-154). */
int yabt_leaf_moments(int x_kind, const void *X, int64_t ldx, int64_t n, const int32_t *feats, int K,
                      void *workspace, size_t workspace_bytes, float *out_mu, float *out_sd,
                      yabt_stream_t stream);

/* Workspace bytes of yabt_hist_slots. */
size_t yabt_hist_slots_workspace_bytes(int64_t n, int F, int K);

/* K-slot histogram of the level-wise grower: out (3, K, F, 256) fp32,
 * out[0][s][f][b] = sum g, out[1] = sum h, out[2] = sum w over the rows i with
 * slot[i] == s and binned[i*ldb + f] == b; rows with slot outside [0, K) are
 * skipped.  g, h, w are each quantised to int64 fixed point (one shift per
 * channel from max|.| and n), summed exactly and rounded to fp32.
 * out_status (device int32 x 4): status (0, or -1 for a non-finite input) and
 * the three shifts.  Replaces `hist_build` (yabt/_cuda/hist.cu:101-133) behind
 * `cuda_hist.build_hist` (yabt/cuda_hist.py:79-89), B fixed at 256. */
int yabt_hist_slots(const uint8_t *binned, int64_t ldb, const int64_t *slot, const float *g,
                    const float *h, const float *w, int64_t n, int F, int K, void *workspace,
                    size_t workspace_bytes, float *out, int32_t *out_status, yabt_stream_t stream);

/* Bytes of device workspace yabt_grow_batched needs for (n, F, max_leaves);
 * 0 when the sizes are out of range (max_leaves above 1024). */
size_t yabt_grow_batched_workspace_bytes(int64_t n, int F, int max_leaves);

/* yabt_grow in rounds: several splits are computed per round (one
 * partition, one histogram and one scan launch for all of them), and cgrow's
 * best-first leaf table (yabt/_cgrow/grow.c:321-408) is replayed over the
 * computed splits to commit them in cgrow's order and numbering.  The next
 * round is planned by running the table further ahead -- a leaf with a
 * computed split gives way to its children -- and taking up to 16 leaves
 * without one, at most 2 uncomputed levels below a committed leaf, while the
 * leaves committed and taken fit in the leaf budget.  A leaf's split depends
 * only on its rows, so the node arrays, values and per-row leaf ids are
 * yabt_grow's bit for bit.  Same arguments and outputs as yabt_grow, plus
 * out_leaf_of_row (n int64, may be NULL): each row's leaf; out_status holds
 * 3 int32: the node count (or -1 for a non-finite input), the rounds run and
 * the splits computed (committed or not).  Requires max_leaves <= 1024.  The
 * host keeps three rounds in flight (it watches a round counter in mapped
 * host memory), so the call returns when the tree is grown; it synchronises
 * `stream`. */
int yabt_grow_batched(const uint8_t *bins_fm, int64_t ld_fm, const uint8_t *bins_rm, int64_t ld_rm,
                      const float *grad, const float *hess, const uint8_t *fmask, const float *imat,
                      float ib, int use_imat, const int32_t *nbins, const int32_t *default_bin,
                      const uint32_t *bin_counts, int64_t n, int F, float lam, float gamma, float mcw,
                      int msl, float lr,
                      int max_leaves, int max_depth, void *workspace, size_t workspace_bytes,
                      int64_t *out_feature, int64_t *out_thr_bin, int64_t *out_left,
                      int64_t *out_right, float *out_value, int64_t *out_depth,
                      int64_t *out_leaf_of_row, int32_t *out_status, yabt_stream_t stream);

/* Bytes of device workspace yabt_grow_levelwise needs; 0 when the sizes are
 * out of range or max_leaves < 2^max_depth. */
size_t yabt_grow_levelwise_workspace_bytes(int64_t n, int F, int max_leaves, int max_depth);

/* yabt_grow for trees whose leaf budget cannot bind (max_leaves >= 2^max_depth,
 * max_depth <= 16): every node of one depth is grown in one batch (routing
 * pass, histograms of all built children, sibling subtraction, one scan
 * launch), and the nodes are then numbered by replaying cgrow's best-first
 * leaf table (yabt/_cgrow/grow.c:321-408) over the computed gains.  Same
 * arguments and outputs as yabt_grow (no default_bin) -- bit-identical node
 * arrays -- plus out_leaf_of_row (n int64, may be NULL): each row's leaf.
 * Returns -3 if the budget could bind.  One device round trip per depth;
 * the call synchronises `stream`. */
int yabt_grow_levelwise(const uint8_t *bins_fm, int64_t ld_fm, const uint8_t *bins_rm, int64_t ld_rm,
                        const float *grad, const float *hess, const uint8_t *fmask, const float *imat,
                        float ib, int use_imat, const int32_t *nbins, const uint32_t *bin_counts,
                        int64_t n, int F, float lam, float gamma, float mcw, int msl, float lr,
                        int max_leaves, int max_depth,
                        void *workspace, size_t workspace_bytes, int64_t *out_feature,
                        int64_t *out_thr_bin, int64_t *out_left, int64_t *out_right, float *out_value,
                        int64_t *out_depth, int64_t *out_leaf_of_row, int32_t *out_status,
                        yabt_stream_t stream);

/* Bytes of device workspace yabt_grow_ref is meant to get for (n, F,
 * max_leaves), with sparse != 0 when it is called with default bins (the
 * sparse builder): the per-tile bucket lists of every feature at once, about
 * n * F * (2 + 2 * sparse) bytes, while those stay within 8 GiB (else of as
 * many features as fit), plus the (2L+1, 3, F, 256) fp32 histograms. */
size_t yabt_grow_ref_workspace_bytes(int64_t n, int F, int max_leaves, int sparse);

/* The smallest workspace yabt_grow_ref accepts: bucket lists of one feature
 * at a time.  Any size from this one up works; yabt_grow_ref buckets as many
 * features per pass as the workspace it is given holds (the result does not
 * depend on it). */
size_t yabt_grow_ref_workspace_min_bytes(int64_t n, int F, int max_leaves, int sparse);

/* Grow one best-first tree with the reference's own arithmetic: the same
 * trees as `cgrow` (yabt/_cgrow/grow.c:243-427) bit for bit -- fp32
 * histograms summed per (feature, bin) in cgrow's row order, cgrow's
 * in-place two-pointer partition order (grow.c:201-217), fp32 sibling
 * subtraction, the double-precision scan and node values, fp32 leaf gains.
 * Arguments as yabt_grow, except that default_bin selects the histogram
 * builder rather than a shortcut: NULL is cgrow's dense builder
 * (use_sparse = 0, grow.c:37-62); a device (F,) int32 array, entries in
 * [0, 255], is cgrow's sparse builder (use_sparse = 1, grow.c:68-107) for a
 * CSR layout of the same bins whose implicit bins are these (the layout of
 * yabt/grow_numba.py:341-367; only its default bins are read, the entries
 * are the bins outside them): each node's default-bin cell is
 * (float)(double row-order sum over the node - double row-order sum over the
 * node's rows outside the default bin).  out_status is replaced by
 * out_n_nodes (device int32, cgrow's return value).  Optional outputs (NULL
 * to skip): out_leaf_of_row (n int64) per-row leaf node ids; out_rows (n
 * int64) cgrow's final rows[] array.  cgrow's leaf table runs on the host,
 * which computes up to 16 splits per round (planned by running the table
 * ahead through the splits already computed) and commits them in cgrow's
 * order: one device round trip per round.  root_order (NULL: the root is
 * bucketed in the call): the rank table yabt_ref_root_order made for these
 * bins_fm, n and F, which the dense builder's root then reads instead of
 * bucketing its rows again (the sparse builder ignores it).  The call returns
 * after the stream has finished (it synchronises `stream`).  Requires
 * n < 2^32, F >= 1, 1 <= max_leaves <= 32767. */
int yabt_grow_ref(const uint8_t *bins_fm, int64_t ld_fm, const uint8_t *bins_rm, int64_t ld_rm,
                  const float *grad, const float *hess, const uint8_t *fmask, const float *imat,
                  float ib, int use_imat, const int32_t *nbins, const int32_t *default_bin,
                  int64_t n, int F, float lam, float gamma, float mcw, int msl, float lr,
                  int max_leaves, int max_depth, void *workspace, size_t workspace_bytes,
                  const void *root_order, int64_t *out_feature, int64_t *out_thr_bin, int64_t *out_left, int64_t *out_right,
                  float *out_value, int64_t *out_depth, int64_t *out_leaf_of_row, int64_t *out_rows,
                  int32_t *out_n_nodes, yabt_stream_t stream);

/* Bytes of the root rank table of yabt_ref_root_order for n rows, F features
 * (0: bad sizes). */
size_t yabt_ref_root_order_bytes(int64_t n, int F);

/* The root rank table of yabt_grow_ref's dense builder, once per fit: for
 * every feature and every 4096-row tile of rows 0 .. n - 1, each row's rank
 * among the tile's rows in its bin (row order), the tile's bin starts, its
 * longest run and its largest bin --
 * the bucketing of cgrow's row-order histogram chains (yabt/_cgrow/grow.c:
 * 37-62) of the root, which is the same for every tree grown on these bins.
 * out: device memory of at least yabt_ref_root_order_bytes(n, F) bytes.
 * Replaces nothing in the reference (cgrow sums the root's rows directly);
 * it is set-up that the device's root histogram reuses across trees. */
int yabt_ref_root_order(const uint8_t *bins_fm, int64_t ld_fm, int64_t n, int F, void *out, size_t out_bytes,
                        yabt_stream_t stream);

/* The reference-arithmetic root histogram alone: out (3, F, 256) float32 =
 * cgrow's dense build_hist over rows 0 .. n - 1 (yabt/_cgrow/grow.c:37-62):
 * per (feature, bin) the fp32 sums of g, of h and of 1.0f in row order, from
 * the rank table yabt_ref_root_order made for these bins (root_order_bytes:
 * its size).  Replaces build_hist for the root node. */
int yabt_ref_root_hist(const uint8_t *bins_fm, int64_t ld_fm, const float *grad, const float *hess, int64_t n,
                       int F, const void *root_order, size_t root_order_bytes, float *out, yabt_stream_t stream);

/* Bytes of device workspace yabt_bin_fit needs for an m-row sample of F features. */
size_t yabt_bin_fit_workspace_bytes(int64_t m, int F);

/* Fit the quantile binner (yabt/binning.py:29-69, the numpy path) on X
 * (fp32 row-major (n, ldx)).  The sample is rows sample_rows[0:m] in that
 * order (NULL: all rows, m == n; the reference draws 200 000 rows with
 * default_rng(0).choice when n > 200 000).  Per feature f, over the sample's
 * non-NaN values (or [0.0] if none):
 *   out_edges[f*ld_edges + 0 : out_nedges[f]] = np.unique of the fp32-rounded
 *     numpy linear quantiles at linspace(0, 1, max_bins + 1)[1:-1];
 *   out_scales[f] = q75 - q25 (double, numpy linear quantiles), or numpy's
 *     float32 std of the sample column when that is 0, or 1;
 * and over all n rows: out_medians[f] = np.nanmedian (0 where all NaN).
 * 2 <= max_bins <= 256, ld_edges >= max_bins - 1. */
int yabt_bin_fit(const float *X, int64_t ldx, int64_t n, int F, const int64_t *sample_rows, int64_t m,
                 int max_bins, void *workspace, size_t workspace_bytes, float *out_edges,
                 int64_t ld_edges, int32_t *out_nedges, float *out_scales, float *out_medians,
                 yabt_stream_t stream);

/* Transform with a fitted binner (yabt/binning.py:71-112): x := medians[f] where
 * NaN, bin = #{edges_f < x} (torch.searchsorted, left).  Any of the outputs may
 * be NULL: out_fm (F, ld_fm >= n) feature-major bins (the grower's layout),
 * out_rm (n, ld_rm >= F) row-major bins, out_imputed (n, ld_imputed >= F) fp32
 * imputed X (binning.py:114-118). */
int yabt_bin_transform(const float *X, int64_t ldx, int64_t n, int F, const float *edges,
                       int64_t ld_edges, const int32_t *nedges, const float *medians,
                       uint8_t *out_fm, int64_t ld_fm, uint8_t *out_rm, int64_t ld_rm,
                       float *out_imputed, int64_t ld_imputed, yabt_stream_t stream);

/* Gradients and hessians of the boosting losses, fp32 (n rows):
 *   loss 0, MSELoss:  g = m - y, h = 1            (yabt/boosting.py:52-54)
 *   loss 1, LogLoss:  p = 1 / (1 + exp(-m)), g = p - y, h = max(p (1 - p), 1e-6)
 *                                                 (yabt/boosting.py:35-38)
 * with m = margin[i], or m = margin[i] + value[leaf_of_row[i]] when both
 * leaf_of_row and value (n_nodes entries) are given (the leaf-model targets of
 * yabt/neural_leaves.py:147); a leaf id outside [0, n_nodes) reads nothing
 * and leaves m = margin[i].  Replaces `self.loss.grad_hess(margin, yt)`
 * (yabt/boosting.py:362). */
int yabt_grad_hess(int loss, const float *margin, const int64_t *leaf_of_row, const float *value,
                   int64_t n_nodes, const float *y, int64_t n, float *out_g, float *out_h,
                   yabt_stream_t stream);

/* Margin update of one boosting round, in place (n rows):
 *   margin[i] += value[l] + sum_{j<K} linear[l*K+j] * clamp(x_ij, lo[l*K+j], hi[l*K+j]),
 *   l = leaf_of_row[i] in [0, n_nodes) (rows with other ids are left unchanged);
 *   K = 0 adds value[l] only (no leaf models);
 * inputs x_ij as in yabt_leaf_fit (x_kind 0: fp32 row-major X[i*ldx + feats[j]];
 * x_kind 1: uint8 feature-major X[feats[j]*ldx + i]; x_kind 2: fp32
 * feature-major X[feats[j]*ldx + i]); 0 <= K <= 8.
 * Replaces `contrib = tree.value[leaf_idx] + tree.net_contribution(Xraw,
 * leaf_idx); margin = margin + contrib` (yabt/boosting.py:508-511,
 * yabt/tree.py:118-128). */
int yabt_margin_update(float *margin, int64_t n, const int64_t *leaf_of_row, const float *value,
                       int64_t n_nodes, int K, const int32_t *feats, const float *linear,
                       const float *lo, const float *hi, int x_kind, const void *X, int64_t ldx,
                       yabt_stream_t stream);

/* Forest prediction: out[i] = (accumulate ? out[i] : base) + sum over trees
 * t = 0..T-1, in order, of value[node] + the node's linear-leaf contribution,
 * where node is the leaf that row i of X (fp32 row-major, ldx >= F) reaches in
 * tree t.  The trees are concatenated: tree t owns global nodes
 * [node_off[t], node_off[t+1]) (node_off (T+1) int64 on the device,
 * node_off[T] <= n_total) and its left/right ids are local to the tree.
 * Linear leaves (optional, net_k == NULL for none): tree t has net_k[t] <= K
 * inputs net_feats[t*K + j]; linear, lo, hi are (n_total, K) (lo/hi NULL:
 * unclamped).  Replaces `Booster._margin` / `Tree.predict`
 * (yabt/boosting.py:536-545, yabt/tree.py:82-135) and `capply`
 * (yabt/_cgrow/grow.c:223-239) for whole forests. */
int yabt_predict(const float *X, int64_t ldx, int64_t n, int F, int T, const int64_t *node_off,
                 int64_t n_total, const int64_t *feature, const float *threshold, const int64_t *left,
                 const int64_t *right, const float *value, int K, const int32_t *net_k,
                 const int32_t *net_feats, const float *linear, const float *lo, const float *hi,
                 float base, int accumulate, float *out, yabt_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* YABT_HIP_H */
