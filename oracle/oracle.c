/*
 * oracle.c -- CPU restatement of the reference's histogram-GBM hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP engine and
 * the timed CPU baseline in bench.py (kind "port").  Nothing in the product
 * (bsscl-gbm_amd/) links, loads or calls it.
 *
 * Every function follows the cited lines of the reference module
 * src/bsscl_gbm/estimator_v1_0_1.py (abbreviated "est:" below) step by step,
 * including its summation order (serial fp64 sums in the order of the row
 * index array), its unstable two-pointer partition and its candidate-slot
 * bookkeeping, so that it produces the trees the reference would produce.
 *
 * The histogram loops are parallel over features with OpenMP, as the
 * reference's `prange` over features is (est:581-596, 722-745): each feature's
 * bins are summed by one thread in row order, so the thread count does not
 * change any result.
 *
 * Build: oracle/Makefile -> oracle/_build/liboracle.so
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORACLE_OK 0
#define ORACLE_EALLOC 1
#define ORACLE_EFORCE 2

/* ------------------------------------------------------------------------ */
/* Binning kernels                                                           */
/* ------------------------------------------------------------------------ */

/* Standard strategy, est:204-226: bounds test, then binary search for the
 * largest k in [0, nb-1] with e[k] <= v. */
static int32_t code_standard(double v, const double *e, int32_t nb)
{
    int32_t lo = 0, hi = nb - 1;
    if (v < e[0]) return 0;
    if (v >= e[nb]) return nb - 1;
    while (lo < hi) {
        int32_t mid = (lo + hi) >> 1;
        if (e[mid + 1] <= v) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

/* Hybrid strategy, est:155-202: interpolation guess, then a +-4 window
 * search, then a full binary search.  The guess of a NaN input is taken as 0
 * (the reference converts NaN with LLVM fptosi; on x86 that yields INT64_MIN,
 * which its own `if g < 0: g = 0` clamps to 0). */
static int32_t code_hybrid(double v, const double *e, int32_t nb)
{
    int32_t last = nb - 1;
    double b_first = e[0], b_end = e[nb];
    double scale = (b_end > b_first) ? (double)last / (b_end - b_first) : 1.0;
    int64_t g;
    int32_t lo, hi;
    if (v < b_first) return 0;
    if (v >= b_end) return last;
    {
        double t = (v - b_first) * scale;
        g = isnan(t) ? 0 : (int64_t)t;
    }
    if (g < 0) g = 0;
    else if (g > last) g = last;
    if (e[g] <= v && (g == last || v < e[g + 1])) return (int32_t)g;
    lo = (int32_t)g - 4;
    hi = (int32_t)g + 4;
    if (lo < 0) lo = 0;
    if (hi > last) hi = last;
    if (!(v >= e[lo] && (hi == last || v < e[hi + 1]))) {
        lo = 0;
        hi = last;
    }
    while (lo < hi) {
        int32_t mid = (lo + hi) >> 1;
        if (e[mid + 1] <= v) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

/* bin_all_features_{standard,hybrid}_numba (est:155-226) over a row-major
 * (n, p) matrix of float32 (x_is_f64 == 0) or float64 values.  Codes are
 * written as uint16 (the caller narrows, as est:2163-2166 chooses the dtype). */
int oracle_bin_features(const void *X, int x_is_f64, int64_t n, int32_t p,
                        const double *edges, int32_t edge_stride,
                        const int32_t *bin_counts, int hybrid, uint16_t *out)
{
    int64_t i;
#pragma omp parallel for schedule(static)
    for (i = 0; i < n; ++i) {
        int32_t j;
        for (j = 0; j < p; ++j) {
            double v = x_is_f64 ? ((const double *)X)[i * p + j]
                                : (double)((const float *)X)[i * p + j];
            const double *e = edges + (int64_t)j * edge_stride;
            int32_t nb = bin_counts[j];
            out[i * p + j] = (uint16_t)(hybrid ? code_hybrid(v, e, nb)
                                               : code_standard(v, e, nb));
        }
    }
    return ORACLE_OK;
}

/* ------------------------------------------------------------------------ */
/* Leaf-wise tree builder, est:517-823                                       */
/* ------------------------------------------------------------------------ */

static inline int32_t xbin_at(const void *xb, int u16, int64_t row, int32_t p,
                              int32_t j)
{
    return u16 ? (int32_t)((const uint16_t *)xb)[row * p + j]
               : (int32_t)((const uint8_t *)xb)[row * p + j];
}

/* Wall time spent in build_hist and the (row, feature) updates it made,
 * since the last oracle_hist_stats(..., reset=1): the CPU baseline's
 * histogram rows x features per second.  Updated by the calling thread
 * only (build_hist parallelises inside). */
static double g_hist_seconds = 0.0;
static int64_t g_hist_row_features = 0;

void oracle_hist_stats(double *seconds, int64_t *row_features, int reset)
{
    if (seconds) *seconds = g_hist_seconds;
    if (row_features) *row_features = g_hist_row_features;
    if (reset) {
        g_hist_seconds = 0.0;
        g_hist_row_features = 0;
    }
}

/* Histogram of rows indices[start:end) for the selected features into slot
 * `slot` (est:581-596 root, est:722-737 smaller child). */
static void build_hist(const void *xb, int u16, int32_t p, const double *grad,
                       const double *hess, const int64_t *indices,
                       int64_t start, int64_t end, const int32_t *feats,
                       int32_t n_sel, const int32_t *bin_counts,
                       double *hG, double *hH, int64_t slot_stride,
                       int32_t max_bins, int32_t slot)
{
    int32_t jj;
    const double t0 = omp_get_wtime();
#pragma omp parallel for schedule(dynamic, 1)
    for (jj = 0; jj < n_sel; ++jj) {
        int32_t j = feats[jj];
        int32_t nb = bin_counts[j];
        double *G = hG + slot * slot_stride + (int64_t)j * max_bins;
        double *H = hH + slot * slot_stride + (int64_t)j * max_bins;
        int64_t k;
        int32_t b;
        for (b = 0; b < nb; ++b) {
            G[b] = 0.0;
            H[b] = 0.0;
        }
        for (k = start; k < end; ++k) {
            int64_t ii = indices[k];
            int32_t bv = xbin_at(xb, u16, ii, p, j);
            if (bv >= nb) bv = nb - 1;
            G[bv] += grad[ii];
            H[bv] += hess[ii];
        }
    }
    g_hist_seconds += omp_get_wtime() - t0;
    g_hist_row_features += (end - start) * (int64_t)n_sel;
}

/* Best split scan over the selected features of one slot (est:598-621 root,
 * est:779-801 child): strict '>' keeps the first feature in `feats` order and
 * then the lowest bin among equal gains. */
static void best_split(const double *hG, const double *hH, int64_t slot_stride,
                       int32_t max_bins, int32_t slot, const int32_t *feats,
                       int32_t n_sel, const int32_t *bin_counts, double mcw,
                       double lam, int32_t force_feat, int32_t force_bin,
                       double *out_gain, int32_t *out_feat, int32_t *out_bin)
{
    double best_gain = -1e9;
    int32_t best_feat = -1, best_bin = 0;
    int32_t jj;
    int forced_found = 0;
    for (jj = 0; jj < n_sel; ++jj) {
        int32_t j = feats[jj];
        int32_t nb = bin_counts[j];
        const double *G = hG + slot * slot_stride + (int64_t)j * max_bins;
        const double *H = hH + slot * slot_stride + (int64_t)j * max_bins;
        double Gt = 0.0, Ht = 0.0, GL = 0.0, HL = 0.0;
        int32_t b;
        if (nb < 2) continue;
        for (b = 0; b < nb; ++b) {
            Gt += G[b];
            Ht += H[b];
        }
        for (b = 0; b < nb - 1; ++b) {
            double GR, HR, gain;
            GL += G[b];
            HL += H[b];
            GR = Gt - GL;
            HR = Ht - HL;
            if (HL < mcw || HR < mcw) continue;
            gain = (GL * GL / (HL + lam) + GR * GR / (HR + lam)) -
                   Gt * Gt / (Ht + lam);
            if (force_feat >= 0) {
                if (j == force_feat && b == force_bin) {
                    best_gain = gain;
                    best_feat = j;
                    best_bin = b;
                    forced_found = 1;
                }
            } else if (gain > best_gain) {
                best_gain = gain;
                best_feat = j;
                best_bin = b;
            }
        }
    }
    if (force_feat >= 0 && !forced_found) {
        /* The forced split is not a candidate of this node (feature not
         * selected, bin out of range or a min_child_weight violation). */
        best_gain = -1e9;
        best_feat = -2;
        best_bin = 0;
    }
    *out_gain = best_gain;
    *out_feat = best_feat;
    *out_bin = best_bin;
}

/*
 * Returns the reference's 7-tuple through the out arrays (each of length
 * 2*max_leaves+2, est:528-537) and node_count.
 *
 * Optional trace (may be NULL): for each successful split in order, the
 * partition counts (n_left, n_right) are appended to trace_counts[2*s..] and
 * the number of splits attempted (including min_samples_leaf rejections) is
 * written to *trace_pops.  Tests use it to check partitions.
 *
 * Optional forced splits (may be NULL; arrays of 2*max_leaves+2 indexed by
 * node id, -1 = not forced): the split search of node v returns
 * (force_feat[v], force_bin[v]) with the gain this builder computes for it,
 * in place of the argmax.  Tests use it to follow the other builder's choice
 * at a certified gain tie, so comparison can go on below that node.  A
 * forced split that is not a candidate of its node fails the call with
 * ORACLE_EFORCE.
 *
 * Optional forced pops (may be NULL; max_leaves entries indexed by the
 * number of splits done, -1 = not forced): the pop that would make split s
 * takes the active candidate of node force_pop[s] in place of the max-gain
 * one (est:645-653), once.  Tests use it to follow the other builder's order
 * where two nodes' gains tie.  A forced node that is not an active candidate
 * with a split fails the call with ORACLE_EFORCE.
 */
int oracle_build_tree_leafwise(
    const void *X_bin, int xbin_u16, int64_t n_rows, int32_t p,
    const double *grad, const double *hess, const int64_t *sample_indices,
    int64_t n_samples, const int32_t *feats, int32_t n_sel,
    int32_t max_leaves, int32_t max_depth, int32_t min_samples_leaf,
    double mcw, const int32_t *bin_counts, int32_t max_bins, double lam,
    double gamma, int32_t *tf, int64_t *tt, double *tv, int32_t *tl,
    int32_t *tr, int32_t *node_count_out, double *sg,
    int64_t *trace_counts, int32_t *trace_pops,
    const int32_t *force_feat, const int32_t *force_bin,
    const int32_t *force_pop)
{
    const int32_t max_nodes = max_leaves * 2 + 2;
    const int32_t MAX_C = max_leaves + 2;
    const int64_t slot_stride = (int64_t)p * max_bins;
    int32_t node_count = 0;
    int32_t n_splits_done = 0, n_pops = 0;
    int64_t *indices = NULL;
    double *hG = NULL, *hH = NULL;
    int32_t *c_node = NULL, *c_depth = NULL, *c_feat = NULL, *c_bin = NULL;
    int64_t *c_start = NULL, *c_end = NULL;
    double *c_gain = NULL, *c_val = NULL;
    int8_t *c_active = NULL;
    int32_t i, root_id;
    int64_t k;
    double g_root = 0.0, h_root = 0.0, root_val;
    double r_gain;
    int32_t r_feat, r_bin;
    int rc = ORACLE_OK;
    int32_t pop_forced_at = -1;
    (void)n_rows;

    for (i = 0; i < max_nodes; ++i) {
        tf[i] = -1;
        tt[i] = 0;
        tv[i] = 0.0;
        tl[i] = -1;
        tr[i] = -1;
        sg[i] = 0.0;
    }

    indices = (int64_t *)malloc(sizeof(int64_t) * (size_t)(n_samples > 0 ? n_samples : 1));
    hG = (double *)calloc((size_t)MAX_C * (size_t)slot_stride, sizeof(double));
    hH = (double *)calloc((size_t)MAX_C * (size_t)slot_stride, sizeof(double));
    c_node = (int32_t *)calloc(MAX_C, sizeof(int32_t));
    c_depth = (int32_t *)calloc(MAX_C, sizeof(int32_t));
    c_feat = (int32_t *)calloc(MAX_C, sizeof(int32_t));
    c_bin = (int32_t *)calloc(MAX_C, sizeof(int32_t));
    c_start = (int64_t *)calloc(MAX_C, sizeof(int64_t));
    c_end = (int64_t *)calloc(MAX_C, sizeof(int64_t));
    c_gain = (double *)calloc(MAX_C, sizeof(double));
    c_val = (double *)calloc(MAX_C, sizeof(double));
    c_active = (int8_t *)calloc(MAX_C, sizeof(int8_t));
    if (!indices || !hG || !hH || !c_node || !c_depth || !c_feat || !c_bin ||
        !c_start || !c_end || !c_gain || !c_val || !c_active) {
        free(indices); free(hG); free(hH); free(c_node); free(c_depth);
        free(c_feat); free(c_bin); free(c_start); free(c_end); free(c_gain);
        free(c_val); free(c_active);
        return ORACLE_EALLOC;
    }
    for (i = 0; i < MAX_C; ++i) {
        c_gain[i] = -1.0;
        c_feat[i] = -1;
    }
    memcpy(indices, sample_indices, sizeof(int64_t) * (size_t)n_samples);

    /* Root (est:563-639). */
    root_id = node_count++;
    for (k = 0; k < n_samples; ++k) {
        int64_t ii = indices[k];
        g_root += grad[ii];
        h_root += hess[ii];
    }
    root_val = -g_root / (h_root + lam);
    if (n_samples < min_samples_leaf || h_root < mcw) {
        tf[root_id] = -1;
        tv[root_id] = root_val;
        goto done;
    }
    build_hist(X_bin, xbin_u16, p, grad, hess, indices, 0, n_samples, feats,
               n_sel, bin_counts, hG, hH, slot_stride, max_bins, 0);
    best_split(hG, hH, slot_stride, max_bins, 0, feats, n_sel, bin_counts, mcw,
               lam, force_feat ? force_feat[root_id] : -1,
               force_bin ? force_bin[root_id] : 0, &r_gain, &r_feat, &r_bin);
    if (r_feat == -2) {
        rc = ORACLE_EFORCE;
        goto done;
    }
    c_node[0] = root_id;
    c_start[0] = 0;
    c_end[0] = n_samples;
    c_depth[0] = 0;
    c_gain[0] = (r_feat >= 0) ? r_gain : -1.0;
    c_feat[0] = r_feat;
    c_bin[0] = r_bin;
    c_val[0] = root_val;
    c_active[0] = 1;
    if (r_feat < 0) {
        tf[root_id] = -1;
        tv[root_id] = root_val;
        goto done;
    }

    /* Main loop (est:641-813). */
    while (n_splits_done < max_leaves - 1) {
        int32_t best_ci = -1, ci, cur, depth, bf, bb, new_depth;
        double best_gain = gamma;
        int64_t start, end, lp, rp, split_pos, n_left, n_right;
        int64_t s_start, s_end, l_start, l_end;
        int32_t small_id, large_id, left_id, right_id;
        int32_t slot_small = -1, slot_large = -1, si, pass;

        if (force_pop && force_pop[n_splits_done] >= 0 &&
            pop_forced_at != n_splits_done) {
            pop_forced_at = n_splits_done;
            for (ci = 0; ci < MAX_C; ++ci) {
                if (c_active[ci] && c_node[ci] == force_pop[n_splits_done]) break;
            }
            if (ci == MAX_C || c_feat[ci] < 0 || !(c_gain[ci] > gamma)) {
                rc = ORACLE_EFORCE;
                goto done;
            }
            best_ci = ci;
        } else {
            for (ci = 0; ci < MAX_C; ++ci) {
                if (c_active[ci] && c_feat[ci] >= 0 && c_gain[ci] > best_gain) {
                    best_gain = c_gain[ci];
                    best_ci = ci;
                }
            }
        }
        if (best_ci < 0) break;
        ci = best_ci;
        cur = c_node[ci];
        start = c_start[ci];
        end = c_end[ci];
        depth = c_depth[ci];
        bf = c_feat[ci];
        bb = c_bin[ci];
        ++n_pops;

        /* Two-pointer in-place partition (est:662-674). */
        lp = start;
        rp = end - 1;
        while (lp <= rp) {
            int64_t ii = indices[lp];
            if (xbin_at(X_bin, xbin_u16, ii, p, bf) <= bb) {
                ++lp;
            } else {
                indices[lp] = indices[rp];
                indices[rp] = ii;
                --rp;
            }
        }
        split_pos = lp;
        n_left = split_pos - start;
        n_right = end - split_pos;
        if (n_left < min_samples_leaf || n_right < min_samples_leaf) {
            tf[cur] = -1;
            tv[cur] = c_val[ci];
            c_active[ci] = 0;
            continue;
        }
        if (trace_counts) {
            trace_counts[2 * n_splits_done] = n_left;
            trace_counts[2 * n_splits_done + 1] = n_right;
        }

        left_id = node_count++;
        right_id = node_count++;
        tf[cur] = bf;
        tt[cur] = bb;
        tl[cur] = left_id;
        tr[cur] = right_id;
        tv[cur] = c_val[ci];
        sg[cur] = c_gain[ci];
        ++n_splits_done;
        new_depth = depth + 1;

        /* Smaller child gets the built histogram (est:701-709). */
        if (n_left <= n_right) {
            s_start = start; s_end = split_pos;
            l_start = split_pos; l_end = end;
            small_id = left_id; large_id = right_id;
        } else {
            s_start = split_pos; s_end = end;
            l_start = start; l_end = split_pos;
            small_id = right_id; large_id = left_id;
        }
        /* First two inactive slots other than ci (est:711-720). */
        for (si = 0; si < MAX_C; ++si) {
            if (si != ci && !c_active[si]) {
                if (slot_small < 0) slot_small = si;
                else if (slot_large < 0) {
                    slot_large = si;
                    break;
                }
            }
        }
        build_hist(X_bin, xbin_u16, p, grad, hess, indices, s_start, s_end,
                   feats, n_sel, bin_counts, hG, hH, slot_stride, max_bins,
                   slot_small);
        /* Larger child by subtraction (est:739-745). */
        {
            int32_t jj;
            for (jj = 0; jj < n_sel; ++jj) {
                int32_t j = feats[jj], nb = bin_counts[j], b;
                double *Gp = hG + ci * slot_stride + (int64_t)j * max_bins;
                double *Hp = hH + ci * slot_stride + (int64_t)j * max_bins;
                double *Gs = hG + slot_small * slot_stride + (int64_t)j * max_bins;
                double *Hs = hH + slot_small * slot_stride + (int64_t)j * max_bins;
                double *Gl = hG + slot_large * slot_stride + (int64_t)j * max_bins;
                double *Hl = hH + slot_large * slot_stride + (int64_t)j * max_bins;
                for (b = 0; b < nb; ++b) {
                    Gl[b] = Gp[b] - Gs[b];
                    Hl[b] = Hp[b] - Hs[b];
                }
            }
        }
        c_active[ci] = 0;

        /* Both children, smaller first (est:751-813). */
        for (pass = 0; pass < 2; ++pass) {
            int64_t cs = pass == 0 ? s_start : l_start;
            int64_t ce = pass == 0 ? s_end : l_end;
            int32_t cid = pass == 0 ? small_id : large_id;
            int32_t slot = pass == 0 ? slot_small : slot_large;
            int64_t cn = ce - cs;
            double gc = 0.0, hc = 0.0, cval;
            double cb_gain = -1e9;
            int32_t cb_feat = -1, cb_bin = 0;
            int can_split;
            for (k = cs; k < ce; ++k) {
                int64_t ii = indices[k];
                gc += grad[ii];
                hc += hess[ii];
            }
            cval = -gc / (hc + lam);
            can_split = (cn >= min_samples_leaf && hc >= mcw && new_depth < max_depth);
            if (can_split) {
                best_split(hG, hH, slot_stride, max_bins, slot, feats, n_sel,
                           bin_counts, mcw, lam,
                           force_feat ? force_feat[cid] : -1,
                           force_bin ? force_bin[cid] : 0,
                           &cb_gain, &cb_feat, &cb_bin);
                if (cb_feat == -2) {
                    rc = ORACLE_EFORCE;
                    goto done;
                }
            }
            c_node[slot] = cid;
            c_start[slot] = cs;
            c_end[slot] = ce;
            c_depth[slot] = new_depth;
            c_gain[slot] = (cb_feat >= 0) ? cb_gain : -1.0;
            c_feat[slot] = cb_feat;
            c_bin[slot] = cb_bin;
            c_val[slot] = cval;
            c_active[slot] = 1;
        }
    }

    /* Remaining candidates become leaves (est:815-820). */
    for (i = 0; i < MAX_C; ++i) {
        if (c_active[i]) {
            tf[c_node[i]] = -1;
            tv[c_node[i]] = c_val[i];
        }
    }

done:
    *node_count_out = node_count;
    if (trace_pops) *trace_pops = n_pops;
    free(indices); free(hG); free(hH); free(c_node); free(c_depth);
    free(c_feat); free(c_bin); free(c_start); free(c_end); free(c_gain);
    free(c_val); free(c_active);
    return rc;
}

/* Post-prune (est:827-841), restated for completeness; after leaf-wise growth
 * it changes nothing because a split needs gain > gamma and pruning needs
 * gain < gamma. */
void oracle_post_prune(int32_t *features, int32_t *left, int32_t *right,
                       const double *split_gains, double gamma,
                       int32_t node_count)
{
    int32_t node;
    for (node = node_count - 1; node >= 0; --node) {
        if (features[node] != -1) {
            int32_t l = left[node], r = right[node];
            if (features[l] == -1 && features[r] == -1 && split_gains[node] < gamma) {
                features[node] = -1;
                left[node] = -1;
                right[node] = -1;
            }
        }
    }
}

/* predict_batch_jit (est:843-861) for numeric features: one tree, all rows. */
int oracle_predict_tree(const void *X_bin, int xbin_u16, int64_t n, int32_t p,
                        const int32_t *features, const int64_t *thresholds,
                        const double *values, const int32_t *left,
                        const int32_t *right, double *out)
{
    int64_t i;
#pragma omp parallel for schedule(static)
    for (i = 0; i < n; ++i) {
        int32_t node = 0;
        while (features[node] >= 0) {
            int32_t f = features[node];
            int64_t v = xbin_at(X_bin, xbin_u16, i, p, f);
            node = (v <= thresholds[node]) ? left[node] : right[node];
        }
        out[i] = values[node];
    }
    return ORACLE_OK;
}

/* predict_all_trees_jit (est:863-884) for numeric features: F starts at 0.0
 * and adds lr * leaf value tree by tree. */
int oracle_predict_all_trees(const void *X_bin, int xbin_u16, int64_t n,
                             int32_t p, const int16_t *features,
                             const int64_t *thresholds, const double *values,
                             const int32_t *left, const int32_t *right,
                             const int32_t *offsets, int32_t n_trees,
                             double lr, double *out)
{
    int64_t i;
#pragma omp parallel for schedule(static)
    for (i = 0; i < n; ++i) {
        double F = 0.0;
        int32_t t;
        for (t = 0; t < n_trees; ++t) {
            int32_t off = offsets[t], node = 0;
            while (features[off + node] >= 0) {
                int32_t f = features[off + node];
                int64_t v = xbin_at(X_bin, xbin_u16, i, p, f);
                node = (v <= thresholds[off + node]) ? left[off + node]
                                                     : right[off + node];
            }
            F += lr * values[off + node];
        }
        out[i] = F;
    }
    return ORACLE_OK;
}
