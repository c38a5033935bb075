/*
 * bsscl_hip.h -- C ABI of the MI355X engine for BSSCL-GBM's histogram path.
 *
 * Plain C types only.  Every entry point returns BSSCL_OK (0) or an error
 * code; bsscl_last_error() gives the calling thread's message for the last
 * failure.  An engine owns device memory and one HIP stream on one GPU; use
 * one engine per thread (or serialise calls), and create engines after any
 * fork(), never before.
 *
 * Each entry point names the reference function it replaces
 * (src/bsscl_gbm/estimator_v1_0_1.py, "est:" below).  The reference has no
 * FFI: its seam is the Numba functions the estimator calls, with NumPy
 * arrays.  The arrays here carry the same meaning, shapes and dtypes.
 */
#ifndef BSSCL_HIP_H
#define BSSCL_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BSSCL_OK 0
#define BSSCL_EINVAL 1   /* bad argument (ValueError in the Python layer) */
#define BSSCL_ENOMEM 2   /* host or device allocation failed */
#define BSSCL_EDEVICE 3  /* no GPU, or a HIP runtime call failed */
#define BSSCL_EINTERNAL 4

typedef struct bsscl_engine bsscl_engine;
typedef struct bsscl_sampler bsscl_sampler;

/* Message of the calling thread's last failing call ("" if none). */
const char *bsscl_last_error(void);

/* Number of visible HIP devices (0 without a GPU). */
int bsscl_device_count(int32_t *out);

/* Engine lifecycle.  No reference counterpart: the reference runs in-process
 * Numba code with no device state. */
int bsscl_engine_create(int32_t device, bsscl_engine **out);
void bsscl_engine_destroy(bsscl_engine *eng);

/*
 * Binning.  Replaces bin_all_features_hybrid_numba / _standard_numba
 * (est:155-226) together with the NaN handling of _bin_features
 * (est:2144-2189): codes are the largest k in [0, nb-1] with e[k] <= v
 * (0 below e[0], nb-1 at or above e[nb]); when any feature had NaN in
 * training (nan_bin_id[j] >= 0 for some j), NaN inputs are binned as 0.0 and
 * NaN-feature codes are shifted by +1 with NaN -> 0.
 *   X          row-major n x F, float32 (x_is_f64 = 0) or float64
 *   edges_2d   row-major F x edge_stride float64 (the reference's bin_edges)
 *   bin_counts int32[F], nan_bin_id int32[F]
 * X may be NULL to bin the matrix staged by bsscl_stage_features (below).
 * The codes stay on the device as matrix `slot` (0 = training, 1 = scoring),
 * stored feature-major as uint8 tiers: T tiers when the largest bin count nb
 * needs them (T = 1 up to 256 bins, else (nb - 2) / 255 + 1), tier t of a
 * code holding clamp(code - 255 t, 0, 255).  Bin counts go up to 65536: the
 * reference keeps codes as uint16 above 255 bins (est:2163-2166), and
 * n_bins = 256, its 'auto' value for p >= 28 (est:1963-1964), already gives
 * 257.  Every split and prediction sees the reference's codes; a code above
 * 255 T (a scoring value above the training range of a NaN feature) is held
 * as 255 T, which every threshold (<= nb - 2) treats identically.  When
 * codes_out is not NULL the codes are also copied back row-major (n x F
 * uint8, min(code, 255)).  More than 65536 bins fail with BSSCL_EINVAL.
 */
int bsscl_bin_features(bsscl_engine *eng, int32_t slot, const void *X,
                       int32_t x_is_f64, int64_t n, int32_t F,
                       const double *edges_2d, int32_t edge_stride,
                       const int32_t *bin_counts, const int32_t *nan_bin_id,
                       uint8_t *codes_out);

/* Upload an already binned matrix: the reference's X_bin, row-major n x F of
 * uint8 (codes_u16 = 0) or uint16 (codes_u16 = 1). */
int bsscl_load_codes(bsscl_engine *eng, int32_t slot, const void *codes,
                     int32_t codes_u16, int64_t n, int32_t F);

/* Copy matrix `slot` back row-major: n x F uint8 min(code, 255), or (_u16)
 * n x F uint16 codes as the reference stores them when _max_bins > 255
 * (est:2163-2166).  A code above 255 T (T tiers, bsscl_bin_features) reads
 * back as 255 T. */
int bsscl_get_codes(bsscl_engine *eng, int32_t slot, uint8_t *codes_out);
int bsscl_get_codes_u16(bsscl_engine *eng, int32_t slot, uint16_t *codes_out);

/*
 * Bin edges on the device.  Replace the data passes of _build_bin_edges
 * (est:2073-2141): np.isnan (est:2092-2093), np.unique (est:2107, 2111) and
 * the partition inside np.percentile (est:2126).  The caller keeps the
 * reference's host arithmetic: the branch on the number of distinct values,
 * np.linspace, the percentile interpolation between the order statistics
 * returned here, np.unique of the result and the appended last edge.
 *
 * bsscl_stage_features copies X (row-major n x F, float32 or float64) to the
 * device, where it stays until bsscl_release_staged or the next staging.
 * bsscl_release_staged ends the staged matrix; its memory, with the sorted
 * columns', stays allocated for the next staging while the three buffers
 * hold at most 1 GiB together (freed by bsscl_engine_destroy), and is freed
 * otherwise.
 * bsscl_bin_features with X = NULL then bins the staged matrix (same n, F
 * and dtype) without a second upload.
 *
 * bsscl_sort_columns sorts every staged column on the device with its NaNs
 * removed and returns, per column, the number of NaNs and the number of
 * distinct non-NaN values (np.unique semantics: -0.0 and +0.0 are one value,
 * and it is returned as +0.0).  The sorted columns stay on the device.
 *
 * bsscl_sorted_gather returns out[k] = the value of rank pos[k] (0-based,
 * ascending, NaNs excluded) of column col[k], as float64 (exact for float32
 * columns); every pos[k] must be below the column's non-NaN count.
 *
 * bsscl_sorted_uniques returns the distinct values of column col in
 * ascending order (the reference's np.unique(col_clean)); fails when there
 * are more than max_out.
 */
int bsscl_stage_features(bsscl_engine *eng, const void *X, int32_t x_is_f64,
                         int64_t n, int32_t F);
int bsscl_sort_columns(bsscl_engine *eng, int64_t *nan_count, int64_t *n_unique);
int bsscl_sorted_gather(bsscl_engine *eng, int64_t count, const int32_t *col,
                        const int64_t *pos, double *out);
int bsscl_sorted_uniques(bsscl_engine *eng, int32_t col, int32_t max_out,
                         double *out, int32_t *count);
int bsscl_release_staged(bsscl_engine *eng);

/*
 * Tree builder.  Replaces _build_tree_leafwise (est:517-823) and the no-op
 * post-prune that follows it (est:827-841, est:2452): same arguments, same
 * 7-tuple.  Runs on training matrix 0.
 *   grad, hess        float64[n] indexed by row id (n = rows of matrix 0)
 *   sample_indices    int64[n_samples] row ids of the in-bag rows
 *   feature_indices   int32[n_selected], ascending
 *   out_*             arrays of length 2*max_leaves+2 (est:528-537);
 *                     out_node_count receives node_count
 * Gradient and hessian sums are accumulated in 64-bit fixed point, so the
 * tree does not depend on the order of sample_indices.
 */
int bsscl_build_tree(bsscl_engine *eng, const double *grad, const double *hess,
                     const int64_t *sample_indices, int64_t n_samples,
                     const int32_t *feature_indices, int32_t n_selected,
                     int32_t max_leaves, int32_t max_depth,
                     int32_t min_samples_leaf, double min_child_weight,
                     const int32_t *bin_counts, int32_t max_bins,
                     double reg_lambda, double gamma, int32_t *out_features,
                     int64_t *out_thresholds, double *out_values,
                     int32_t *out_left, int32_t *out_right,
                     int32_t *out_node_count, double *out_split_gains);

/*
 * Binary boosting loop state on matrix 0.  Replaces the set-up of
 * _fit_binary (est:2825-2848): y int64[n] in {0,1}, per-class weights w0/w1
 * (est:2570-2603), F initialised to base_score (est:2831-2834).
 */
int bsscl_boost_begin(bsscl_engine *eng, const int64_t *y, int64_t n,
                      double w0, double w1, double base_score);

/*
 * One boosting round of _fit_binary (est:2849-2906): gradients and hessians
 * from F (est:2861, est:2873-2874), the round's rows and features from the
 * sampler (est:2886, est:2502-2517), the tree (est:2891), F += lr * tree(X)
 * over all rows (est:2896-2897) and the training log-loss (est:2905,
 * est:2320-2325).  Outputs as for bsscl_build_tree, plus out_train_loss.
 */
int bsscl_boost_round(bsscl_engine *eng, bsscl_sampler *sampler,
                      int32_t max_leaves, int32_t max_depth,
                      int32_t min_samples_leaf, double min_child_weight,
                      const int32_t *bin_counts, int32_t max_bins,
                      double reg_lambda, double gamma, double learning_rate,
                      int32_t *out_features, int64_t *out_thresholds,
                      double *out_values, int32_t *out_left,
                      int32_t *out_right, int32_t *out_node_count,
                      double *out_split_gains, double *out_train_loss);

/* Pipelined rounds (no reference counterpart; the reference's loop is
 * synchronous, est:2825-2906): with `on`, bsscl_boost_round enqueues the
 * sampler's next round, with the same arguments, before it returns the
 * current one, so the GPU never waits for the caller.  Every later call
 * must pass the same arguments until pipelining is turned off; turning it
 * off (or bsscl_boost_begin) waits for and drops a round enqueued ahead,
 * whose F update then stays applied.  Trees deeper than 9 levels or with
 * more than 1022 leaves are not enqueued ahead.  The sampler must outlive a
 * round enqueued ahead: turn pipelining off before destroying it. */
int bsscl_boost_set_pipeline(bsscl_engine *eng, int32_t on);

/* F of the boosting run (float64[n]). */
int bsscl_boost_get_F(bsscl_engine *eng, double *F_out);

/* Gradients and hessians of the current F (float64[n] each). */
int bsscl_boost_grad_hess(bsscl_engine *eng, double *grad_out,
                          double *hess_out);

/* The largest |g| and h over all rows of the current F (out[0], out[1]),
 * as the device holds them for the next round's fixed-point scale (no
 * reference counterpart: the reference sums float64 gradients, est:581-596).
 * A round on the device path scales its tree's int64 gradients by
 * 2^(62 - ceil(log2 m) - e) with max |g| < 2^e (hessians likewise), so any
 * sum over its m rows fits in int64.  Waits for the engine's stream. */
int bsscl_boost_grad_hess_max(bsscl_engine *eng, double *out);

/*
 * Multiclass rounds with the scores on the device.  Replace the NumPy
 * arithmetic of the reference's multiclass loop (est:2949-3065): the (n, K)
 * score matrix starting at 0 (est:2958), each round's softmax gradients and
 * hessians from the scores at the round's start (est:2996, 3013-3014, hessians
 * floored at 1e-8), each class's tree (the _build_tree_leafwise seam on those
 * gradients, est:3016-3026) and its score update F[:, k] += lr * tree (est:3029),
 * and the round's multiclass log-loss (est:3035).  Runs on training matrix 0.
 *   mc_begin       y int64[n] in [0, n_classes), sample_weight float64[n] > 0,
 *                  2 <= n_classes <= 16
 *   mc_round       the round's in-bag rows (int64[n_samples], shared by its
 *                  K trees); computes every class's gradients and hessians
 *   mc_round_sampled  as mc_round with the sampler's next round (est:2502-2517
 *                  at est:2996): with BSSCL_SAMPLER_DEVICE_ROWS the rows are
 *                  permuted on the GPU as bsscl_boost_round does; the round's
 *                  ascending feature subset goes to feats_out (int32[f_sub],
 *                  may be NULL)
 *   mc_build_tree  class k's tree from the round's rows and the features
 *                  (arguments and outputs as bsscl_build_tree), then adds
 *                  learning_rate * tree to class k's scores
 *   mc_build_trees the round's K trees at once, classes 0..K-1, with the
 *                  arguments of mc_build_tree but no k: the same trees and
 *                  score updates, enqueued back to back and read back once.
 *                  Outputs hold K blocks of M = 2 * max_leaves + 2 entries
 *                  (class k's tree at k * M) and out_node_count K entries.
 *                  Replaces the loop over k of est:3016-3029
 *   mc_round_trees one whole round: mc_round_sampled, mc_build_trees and
 *                  mc_loss in one call.  It also takes the sampler's next
 *                  round and makes its rows on a second stream while this
 *                  round's trees are built; the next call uses them.
 *                  bsscl_boost_set_pipeline(eng, 0), mc_begin, mc_round and
 *                  mc_round_sampled hand such a round back; the sampler
 *                  must outlive it
 *   mc_loss        -mean log(clip(softmax(F)[y], 1e-15, 1 - 1e-15))
 *   mc_get_scores  F as float64[n_classes * n], class by class (row i of
 *                  class k at k * n + i)
 *   mc_get_grad_hess  the last mc_round's gradients and hessians (est:3013-3014,
 *                  hessians after the 1e-8 floor of est:3019), float64[n_classes * n]
 *                  each, laid out as mc_get_scores
 */
int bsscl_mc_begin(bsscl_engine *eng, const int64_t *y, int64_t n, int32_t n_classes,
                   const double *sample_weight);
int bsscl_mc_round(bsscl_engine *eng, const int64_t *sample_indices, int64_t n_samples);
int bsscl_mc_round_sampled(bsscl_engine *eng, bsscl_sampler *sampler, int32_t *feats_out);
int bsscl_mc_build_tree(bsscl_engine *eng, int32_t k, const int32_t *feature_indices,
                        int32_t n_selected, int32_t max_leaves, int32_t max_depth,
                        int32_t min_samples_leaf, double min_child_weight,
                        const int32_t *bin_counts, int32_t max_bins, double reg_lambda,
                        double gamma, double learning_rate, int32_t *out_features,
                        int64_t *out_thresholds, double *out_values, int32_t *out_left,
                        int32_t *out_right, int32_t *out_node_count, double *out_split_gains);
int bsscl_mc_build_trees(bsscl_engine *eng, const int32_t *feature_indices, int32_t n_selected,
                         int32_t max_leaves, int32_t max_depth, int32_t min_samples_leaf,
                         double min_child_weight, const int32_t *bin_counts, int32_t max_bins,
                         double reg_lambda, double gamma, double learning_rate,
                         int32_t *out_features, int64_t *out_thresholds, double *out_values,
                         int32_t *out_left, int32_t *out_right, int32_t *out_node_count,
                         double *out_split_gains);
int bsscl_mc_round_trees(bsscl_engine *eng, bsscl_sampler *sampler, int32_t *feats_out,
                         int32_t max_leaves, int32_t max_depth, int32_t min_samples_leaf,
                         double min_child_weight, const int32_t *bin_counts, int32_t max_bins,
                         double reg_lambda, double gamma, double learning_rate,
                         int32_t *out_features, int64_t *out_thresholds, double *out_values,
                         int32_t *out_left, int32_t *out_right, int32_t *out_node_count,
                         double *out_split_gains, double *out_loss);
int bsscl_mc_loss(bsscl_engine *eng, double *out_loss);
int bsscl_mc_get_scores(bsscl_engine *eng, double *out);
int bsscl_mc_get_grad_hess(bsscl_engine *eng, double *grad_out, double *hess_out);

/*
 * Ensemble prediction.  Replaces predict_all_trees_jit (est:863-884):
 * out_F[i] = sum over trees t of learning_rate * value_t(leaf of row i),
 * accumulated tree by tree from 0.0, on the rows of matrix `slot`.  The tree
 * arrays are the packed arrays of _pack_tree_list (est:2192-2216).
 */
int bsscl_predict(bsscl_engine *eng, int32_t slot, const int16_t *features,
                  const int64_t *thresholds, const double *values,
                  const int32_t *left, const int32_t *right,
                  const int32_t *offsets, int32_t n_trees,
                  double learning_rate, double *out_F);
/*
 * predict_proba of a binary model (est:3318-3336) from the same arrays:
 * F as bsscl_predict, plus base_score, then p = 1 / (1 + exp(-clip(F, -500,
 * 500))); out_proba float64[2 * n] holds (1 - p, p) row by row.  The device's
 * exp may differ from NumPy's in the last bit.
 */
int bsscl_predict_proba(bsscl_engine *eng, int32_t slot, const int16_t *features,
                        const int64_t *thresholds, const double *values,
                        const int32_t *left, const int32_t *right,
                        const int32_t *offsets, int32_t n_trees, double learning_rate,
                        double base_score, double *out_proba);
/*
 * The whole of a binary model's predict_proba from host rows: binning X
 * (est:3289, as bsscl_bin_features with the same edges, bin counts and NaN
 * bins), the walk and the probabilities (est:3318-3336, as
 * bsscl_predict_proba), with identical results.  X streams through the
 * device in row chunks of about 256 MB: a chunk's upload runs while the
 * device bins and walks the chunk before it.  Leaves matrix slots 0 and 1
 * as they were.
 */
int bsscl_predict_proba_rows(bsscl_engine *eng, const void *X, int32_t x_is_f64, int64_t n,
                             int32_t F, const double *edges_2d, int32_t edge_stride,
                             const int32_t *bin_counts, const int32_t *nan_bin_id,
                             const int16_t *features, const int64_t *thresholds,
                             const double *values, const int32_t *left, const int32_t *right,
                             const int32_t *offsets, int32_t n_trees, double learning_rate,
                             double base_score, double *out_proba);
/*
 * predict_proba of a multiclass model (est:3293-3315): per class k, F[:, k]
 * accumulated tree by tree from 0.0 over the rows of matrix `slot` (class
 * k's packed arrays, n_trees[k] of them, possibly none), then each row's
 * softmax (est:2327-2332, in the arithmetic of the training rounds: the
 * class sum in NumPy's pairwise order); out_proba float64[n * K], row by
 * row.  2 <= K <= 16.  The device's exp may differ from NumPy's in the last
 * bit.
 */
int bsscl_predict_proba_mc(bsscl_engine *eng, int32_t slot, int32_t K,
                           const int16_t *const *features, const int64_t *const *thresholds,
                           const double *const *values, const int32_t *const *left,
                           const int32_t *const *right, const int32_t *const *offsets,
                           const int32_t *n_trees, double learning_rate, double *out_proba);

/*
 * Ensemble prediction that allocates nothing.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (serving
 * loops, code under HIP graph capture, harnesses that forbid hipMalloc).
 * Same trees, arithmetic and result as bsscl_predict, but out_F_dev is a
 * float64[n] buffer in the device memory of the engine's GPU (n = rows of
 * matrix `slot`), written before the call returns.  The packed trees are
 * copied into a fixed per-GPU scratch area of at most 131072 nodes and 16384
 * trees; larger ensembles fail with BSSCL_EINVAL.  No hipMalloc, hipFree or
 * other allocating call is made.  Calls on one GPU share that area (it keeps
 * the last call's trees): calls that overlap on one GPU race.
 */
int bsscl_predict_noalloc(bsscl_engine *eng, int32_t slot, const int16_t *features,
                          const int64_t *thresholds, const double *values,
                          const int32_t *left, const int32_t *right,
                          const int32_t *offsets, int32_t n_trees,
                          double learning_rate, double *out_F_dev);

/* One tree over the rows of matrix `slot`: predict_batch_jit (est:843-861). */
int bsscl_predict_tree(bsscl_engine *eng, int32_t slot,
                       const int32_t *features, const int64_t *thresholds,
                       const double *values, const int32_t *left,
                       const int32_t *right, int32_t node_count, double *out);

/*
 * One node's histogram and best split on matrix 0: the root histogram
 * (est:581-596) and root split scan (est:598-621) for the given rows.
 * out_G/out_H: float64[n_selected * 256] (feature-position major, bins past
 * bin_counts are 0); bin counts up to 256.  out_gain/out_feature/out_bin receive the best split
 * (out_feature = -1 when none qualifies).  Any output may be NULL.
 */
int bsscl_node_split(bsscl_engine *eng, const double *grad, const double *hess,
                     const int64_t *rows, int64_t m,
                     const int32_t *feature_indices, int32_t n_selected,
                     const int32_t *bin_counts, double min_child_weight,
                     double reg_lambda, double *out_G, double *out_H,
                     double *out_gain, int32_t *out_feature, int32_t *out_bin);

/*
 * Partition of a row set by one split on matrix 0: the reference's in-place
 * two-pointer loop (est:662-674) moves rows with code <= bin to the front.
 * Here the order is stable: out_rows[0:*out_n_left] are the left rows in
 * input order, then the right rows in input order.
 */
int bsscl_partition(bsscl_engine *eng, const int64_t *rows, int64_t m,
                    int32_t feature, int32_t bin, int64_t *out_rows,
                    int64_t *out_n_left);

/* Row/column bagging stream, bit-identical to NumPy RandomState
 * (est:2502-2517).  key[624]/pos come from RandomState.get_state() and are
 * updated in place.  rs_shuffle_*: RandomState.shuffle of data[n]. */
int bsscl_rs_shuffle_i64(uint32_t *key, int32_t *pos, int64_t *data,
                         int64_t n);
int bsscl_rs_shuffle_i32(uint32_t *key, int32_t *pos, int32_t *data,
                         int64_t n);
/* The random half of RandomState.shuffle of n items (est:2506): the bounded
 * draws j(i) of the steps i = n-1 .. 1, draws_out[n-1-i] = j(i). */
int bsscl_rs_draws(uint32_t *key, int32_t *pos, uint32_t *draws_out, int64_t n);
/* The swap half of RandomState.shuffle on the GPU (est:2506): data[n] is
 * permuted in place by the steps i = n-1 .. 1 (swap data[i], data[j(i)])
 * with draws[n-1-i] = j(i) <= i.  No reference counterpart as a separate
 * call; bsscl_boost_round uses the same kernels. */
int bsscl_fisher_yates_apply(bsscl_engine *eng, const uint32_t *draws,
                             int64_t n, int32_t *data);

/* Sampler flag: the rows are permuted on GPU `device` by bsscl_boost_round
 * (the sampler copies each round's draws there on a stream of its own, ahead
 * of use); bsscl_sampler_next then refuses row bagging.  `device` is
 * ignored without the flag. */
#define BSSCL_SAMPLER_DEVICE_ROWS 1
int bsscl_sampler_create(const uint32_t *key, int32_t pos, int64_t n,
                         int64_t n_sub, int32_t do_rows, int32_t n_features,
                         int32_t f_sub, int32_t do_feats, int32_t n_rounds,
                         int32_t lookahead, int32_t flags, int32_t device,
                         bsscl_sampler **out);
/* Next round: the reference's sample_idx (int32[n_sub], in its order) and
 * the ascending feature subset (int32[f_sub]); either output may be NULL. */
int bsscl_sampler_next(bsscl_sampler *s, int32_t *rows_out,
                       int32_t *feats_out);
int bsscl_sampler_state(bsscl_sampler *s, uint32_t *key_out,
                        int32_t *pos_out);
/* Host time of the sampler's stages (no reference counterpart): [0] rounds
 * produced, [1] ms drawing bounded integers, [2] ms applying swaps on the
 * host, [3] ms generating MT19937 words (twisting, in the parallel form),
 * [4] chunks of words mapped through a transfer function and [5] chunks
 * counted word by word (parallel form; 0 otherwise). */
int bsscl_sampler_stats(bsscl_sampler *s, double *out, int32_t cap,
                        int32_t *n_out);
void bsscl_sampler_destroy(bsscl_sampler *s);

/*
 * Timing of the engine's own kernels while profiling is on: level 1 times
 * the histogram and prediction kernels only, level 2 also the partition and
 * split groups (0 turns it off).  No reference counterpart (the reference
 * records only wall times, est:1904).  bsscl_engine_stats fills up to `cap`
 * doubles in this order:
 *   [0] histogram launches   [1] histogram ms (sum of launch durations)
 *   [2] histogram rows x features  [3] histogram algorithmic bytes
 *   [4] partition launches   [5] partition ms
 *   [6] split launches       [7] split ms
 *   [8] trees built          [9] nodes expanded
 *   [10] host ms waiting for the bagging sample in bsscl_boost_round
 *   [11] host ms in bsscl_boost_round (whole rounds)
 *   [12] histogram-reduction launches  [13] histogram-reduction ms
 *   [14] host ms enqueueing rounds     [15] host ms waiting for a round's results
 *   [16] prediction launches (bsscl_predict)  [17] prediction ms
 *   [18] boosting rounds whose rows-stream kernels (bagging, in-bag sort,
 *        root gather) ran as a captured HIP graph
 *   [19] boosting rounds whose tree kernels ran as a captured HIP graph
 *   [20] graphs captured
 * and returns the number written in *n_out.  A histogram launch's time runs
 * from its first block's start to its last block's end, stamped by the
 * kernel on the device's constant-rate clock; prediction times come from
 * events recorded by the kernel's own dispatch; the other groups are
 * bracketed by event pairs on the stream.  The host times [10], [11], [14],
 * [15] and the counters [18]-[20] are kept at every level (0 included);
 * set_profiling with a level of 1 or 2 clears every entry.  The rows-stream
 * sequence runs as a graph by default, the tree sequence with
 * BSSCL_GRAPHS=1 in the environment and only while profiling is off (its
 * stamps and event pairs take per-round addresses); BSSCL_GRAPHS=0 launches
 * every kernel one by one.
 */
int bsscl_engine_set_profiling(bsscl_engine *eng, int32_t on);
int bsscl_engine_stats(bsscl_engine *eng, double *out, int32_t cap,
                       int32_t *n_out);

#ifdef __cplusplus
}
#endif

#endif /* BSSCL_HIP_H */
