// Device data structures and kernel launchers of the tree engine.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace bsscl {

constexpr int kBins = 256;          // histogram bins per feature (uint8 codes)
constexpr int kHistPerFeat = 512;   // int64 words per feature: [bin][g,h]

// A node's row segment in the compact buffers of its depth (buffer = depth%2).
struct NodeSeg {
  int64_t start;
  int64_t count;
  int32_t valid;     // 1 when the node exists (its parent's split was kept)
  int32_t is_small;  // 1 when its histogram is built, 0 when subtracted
};

// Parent split of one level (host -> device).
struct PartParent {
  int64_t start;
  int64_t count;
  int32_t fpos;      // split feature, position in the selected-feature list
  int32_t bin;       // rows with code <= bin go left
  int32_t left_id;   // internal node ids of the children
  int32_t right_id;
};

// One partition tile of a parent (host -> device).
struct PartTile {
  int64_t row0;
  int32_t rows;
  int32_t parent;    // index into the level's PartParent array
};

// One histogram work item: `tile`-th block of rows of node hist_node[ref].
struct HistTask {
  int32_t ref;
  int32_t tile;
};

// One node whose split is searched.  parent < 0: its own histogram is read;
// otherwise a non-small node's histogram is parent minus sibling.
struct SplitTask {
  int32_t node;
  int32_t parent;
  int32_t sibling;
  int32_t depth;
};

// Best split of one (node, feature): bin < 0 when no bin qualifies.
struct SplitCand {
  double gain;
  int32_t bin;
  int32_t pad;
};

struct SplitParams {
  double min_child_weight;
  double reg_lambda;
  double g_scale;      // 2^-sg: fixed point -> gradient
  double h_scale;      // 2^-sh: fixed point -> hessian
  int32_t min_samples_leaf;
  int32_t max_depth;
};

// A tree in device form for traversal (node_count entries).
struct TreeNodeDev {
  int32_t feature;     // -1 for a leaf
  int32_t threshold;   // go left when code <= threshold
  int32_t left;
  int32_t right;
  double value;
};

// A run of kPartTile rows starting at a 4-row boundary (tiles of one parent
// are consecutive; rows outside the parent's segment are masked).
constexpr int kPartTile = 1024;

// A node's result after its split search, packed for readback.
struct NodeOut {
  int64_t start;
  int64_t count;
  long long Gq;
  long long Hq;
  double gain;     // best gain (-1e9 when fpos < 0)
  int32_t fpos;    // best feature position, -1 when none qualifies
  int32_t bin;
  int32_t valid;
  int32_t pad;
};

// Launchers (kernels.hip).  All are asynchronous on `st`.
hipError_t launch_bin(hipStream_t st, const void *X, int is_f64, int64_t n,
                      int32_t F, const double *edges, int32_t stride,
                      const int32_t *nb, const int32_t *nan_id,
                      int32_t has_any_nan, uint8_t *codes, int64_t ld);
hipError_t launch_load_codes(hipStream_t st, const void *src, int is_u16,
                             int64_t n, int32_t F, uint8_t *codes, int64_t ld);
hipError_t launch_get_codes(hipStream_t st, const uint8_t *codes, int64_t ld,
                            int64_t n, int32_t F, uint8_t *dst);
hipError_t launch_quantize(hipStream_t st, const double *g, const double *h,
                           int64_t n, double g_mul, double h_mul, int2 *ghq);
hipError_t launch_grad_hess(hipStream_t st, const double *F, const uint8_t *y,
                            int64_t n, double w0, double w1, double g_mul,
                            double h_mul, int2 *ghq);
hipError_t launch_grad_hess_f64(hipStream_t st, const double *F,
                                const uint8_t *y, int64_t n, double w0,
                                double w1, double *g, double *h);
hipError_t launch_sort_rows(hipStream_t st, const int32_t *rows, int64_t m,
                            uint8_t *flags, int64_t n_pad, int32_t *block_tmp,
                            int32_t *out);
int64_t sort_rows_flag_bytes(int64_t n);
hipError_t launch_gather_root(hipStream_t st, const uint8_t *codes, int64_t ld,
                              const int32_t *feat, int32_t F_sel,
                              const int32_t *rows32, const int64_t *rows64,
                              int64_t m, const int2 *ghq, uint8_t *codes_c,
                              int64_t ld_c, int2 *gh_c, int32_t *rid_c,
                              int64_t pad_to, NodeSeg *segs, int32_t *hist_node,
                              unsigned long long *root_hist, int64_t hist_words);
hipError_t launch_hist(hipStream_t st, const uint8_t *codes_c, int64_t ld_c,
                       const int2 *gh_c, const HistTask *tasks,
                       int32_t n_tasks, const int32_t *hist_node,
                       const NodeSeg *segs, const int32_t *nb_sel,
                       const int32_t *hot_sel, int32_t F_sel, int32_t fchunk,
                       int32_t tile_rows, unsigned long long *pool,
                       int64_t node_stride);
int hist_blocks(int32_t n_tasks, int32_t nchunks);
hipError_t launch_part_count(hipStream_t st, const uint8_t *codes_c,
                             int64_t ld_c, const PartParent *parents,
                             const PartTile *tiles, int32_t n_tiles,
                             int32_t *tile_left);
hipError_t launch_part_scan(hipStream_t st, const PartParent *parents,
                            int32_t n_parents, const int32_t *tile_begin,
                            const int32_t *tile_left, int64_t *tile_left_off,
                            int64_t *parent_nleft, NodeSeg *segs,
                            int32_t *hist_node, int32_t min_samples_leaf,
                            unsigned long long *pool, int64_t node_stride);
hipError_t launch_part_scatter(hipStream_t st, const uint8_t *codes_src,
                               uint8_t *codes_dst, int64_t ld_c,
                               const int2 *gh_src, int2 *gh_dst,
                               const int32_t *rid_src, int32_t *rid_dst,
                               const PartParent *parents,
                               const PartTile *tiles, int32_t n_tiles,
                               const int64_t *tile_left_off,
                               const int64_t *parent_nleft, int32_t F_sel);
hipError_t launch_split(hipStream_t st, const SplitTask *tasks, int32_t n_tasks,
                        const NodeSeg *segs, unsigned long long *pool,
                        int64_t node_stride, const int32_t *nb_sel,
                        int32_t F_sel, SplitParams p, SplitCand *cand,
                        long long *totals);
hipError_t launch_node_best(hipStream_t st, const NodeSeg *segs,
                            const long long *totals, const SplitCand *cand,
                            int32_t F_sel, int32_t first, int32_t count,
                            int32_t no_split, NodeOut *out);
hipError_t launch_child_totals(hipStream_t st, const PartParent *parents,
                               int32_t n_parents, const int32_t *parent_ids,
                               const NodeSeg *segs, const unsigned long long *pool,
                               int64_t node_stride, long long *totals);
hipError_t launch_code_counts(hipStream_t st, const uint8_t *codes, int64_t ld,
                              int64_t n, int32_t F, unsigned int *counts);
hipError_t launch_update_F(hipStream_t st, const uint8_t *codes, int64_t ld,
                           int64_t n, const TreeNodeDev *tree,
                           int32_t node_count, double lr, double *F,
                           const uint8_t *y, double *loss_partials,
                           int32_t n_blocks);
hipError_t launch_sum_partials(hipStream_t st, const double *partials,
                               int32_t count, double *out);
hipError_t launch_predict_tree(hipStream_t st, const uint8_t *codes,
                               int64_t ld, int64_t n, const TreeNodeDev *tree,
                               int32_t node_count, double *out);
hipError_t launch_predict(hipStream_t st, const uint8_t *codes, int64_t ld,
                          int64_t n, const TreeNodeDev *nodes,
                          const int32_t *offsets, int32_t n_trees, double lr,
                          double *out);

int update_F_blocks(int64_t n);

}  // namespace bsscl
