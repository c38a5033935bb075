// Device data structures and kernel launchers of the tree engine.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace bsscl {

constexpr int kBins = 256;          // histogram bins per feature (uint8 codes)
constexpr int kHistPerFeat = 512;   // int64 words per feature: [bin][g,h]

// Codes above 255 (the reference keeps uint16 codes when a feature has more
// than 255 bins, est:2163-2166) are held in tiers of uint8 columns: column
// t * F + j of feature j holds clamp(code - 255 t, 0, 255), so tier 0 is
// min(code, 255).  The reference's split "code <= 255 t + b" (0 <= b <= 254)
// is "tier t <= b", tier t's cumulative histogram up to bin b is the
// feature's up to 255 t + b, and the tiers of a row add up to its code (up to
// 255 T for T tiers).
constexpr int32_t kMaxBinCount = 65536;  // uint16 codes
constexpr int32_t kMaxTiers = 257;       // tiers_for_bins(kMaxBinCount)
// Tiers a feature of nb bins splits on (thresholds 0 .. nb - 2).
inline int32_t tiers_for_bins(int32_t nb) { return nb <= kBins ? 1 : (nb - 2) / 255 + 1; }
// Tiers that hold code c exactly.
inline int32_t tiers_for_code(int32_t c) { return c <= 255 ? 1 : (c + 254) / 255; }

// Fixed-point gradient and hessian of one row: (g * 2^sg, h * 2^sh) as
// int64, with the exponents chosen so that a sum over all rows of a tree
// fits in int64.
using GH = longlong2;

// A node's row segment in the compact buffers of its depth (buffer = depth%2).
struct NodeSeg {
  int64_t start;
  int64_t count;
  int32_t valid;     // 1 when the node exists (its parent's split was kept)
  int32_t is_small;  // 1 when its histogram is built, 0 when subtracted
};

// Parent split of one level.
struct PartParent {
  int64_t start;
  int64_t count;
  int32_t fpos;      // split feature, position in the selected-feature list
  int32_t bin;       // rows with code <= bin go left
  int32_t left_id;   // internal node ids of the children
  int32_t right_id;
  int32_t node;      // the parent's own id
  int32_t gslot;     // 2 * its PartGroup + its side (levels with groups only)
  // The partition tiles [tile0, tile1) that count this parent's rows (runs
  // 2 * side and 2 * side + 1 of each, side = gslot & 1 with groups, else 0).
  int32_t tile0, tile1;
};

// A partition group: the rows [start, start + count) of the source set,
// sent first by an optional split (fpos >= 0: code <= bin is side 0, else
// side 1; fpos < 0: every row is on side 0) to the parent par[side], then
// by that parent's own split to its left or right child.  The rows of a
// side whose par is -1 are not moved.  A level whose parents' rows lie in
// their own segments has no groups: group i is parent i.  A level whose
// parents are the children of the previous level's parents, still in their
// parent's segment, has one group per such grandparent.  Each tile counts
// its rows of the four runs 2 * side + (right child ? 1 : 0).
struct PartGroup {
  int64_t start;
  int64_t count;
  int32_t fpos;
  int32_t bin;
  int32_t par[2];
};

// Work counts of one level, written by the planner kernel (or uploaded for
// the root) and read by every kernel of the level, whose grids are upper
// bounds.
struct LevelPlan {
  int32_t n_parents;    // PartParent entries
  int32_t n_tiles;      // PartTile entries
  int32_t n_hist;       // HistTask entries
  int32_t n_split;      // nodes created at this level (the next level's candidates)
  int32_t first_child;  // id of the first node created at this level
  int32_t tile_rows;    // rows per HistTask tile
  int32_t n_nodes;      // nodes in the tree after this level
  int32_t overflow;     // nodes needed when the node table is too small, else 0
};

// Planner inputs that do not change within a tree.
struct PlanArgs {
  double gamma;
  int32_t level;          // depth of the nodes that become parents
  int32_t max_leaves;
  int32_t last;           // their children are at max_depth
  int32_t node_cap;       // node table capacity
  int32_t tile_cap;       // PartTile capacity
  int32_t hist_cap;       // HistTask capacity
  int32_t hist_target;    // histogram row tiles wanted per level
  int32_t rows_per_flush; // fewest rows per histogram tile flush
  int32_t part_tile;      // rows per partition tile
  int32_t mode;           // kLevelMove, kLevelInPlace or kLevelGrouped
  // Every split a candidate can take is kept when popped: a split needs
  // H >= min_child_weight on both sides and no row's hessian exceeds
  // min_child_weight / min_samples_leaf, so both children have at least
  // min_samples_leaf rows (est:614-615, 678-683).  Then the level's other
  // candidates with a split count as kept splits ranked above a candidate.
  int32_t all_kept;
  int32_t part_rows;      // rows per thread of a partition tile (4, 8 or 16)
  // In place and grouped levels: blocks 1.. of the planner launch count the
  // level's partition tiles (plan_count_role) while block 0 plans.
  int32_t fused_count;
};

// How a level treats its rows:
//   kLevelMove: the parents' rows move to their children's segments in the
//     other set (one group per parent), and the smaller children's
//     histograms read them there;
//   kLevelInPlace: the rows stay in the parents' segments; the children get
//     the segments the move would give them, and the smaller child's
//     histogram reads its parent's segment, taking the rows that go its way;
//   kLevelGrouped: the parents are the children of an in-place level; their
//     rows move from the grandparents' segments (one group per grandparent)
//     straight to their children's segments in the other set.
constexpr int32_t kLevelMove = 0;
constexpr int32_t kLevelInPlace = 1;
constexpr int32_t kLevelGrouped = 2;

// One partition tile of a group (host -> device).
struct PartTile {
  int64_t row0;
  int32_t rows;
  int32_t parent;    // its PartGroup (the PartParent of that index without groups)
};

// One histogram work item: `tile`-th block of rows of node hist_node[ref].
struct HistTask {
  int32_t ref;
  int32_t tile;
};

// One node whose split is searched.  parent < 0: its own histogram is read;
// otherwise a non-small node's histogram is parent minus sibling.
// Best split of one (node, feature): bin < 0 when no bin qualifies.
struct SplitCand {
  double gain;
  int32_t bin;
  int32_t pad;
};

// The largest |g| and h of a boosting round's rows, held on the device as
// the bit patterns of non-negative doubles (which order as unsigned
// integers), and the bits a row's fixed-point value may use
// (62 - ceil(log2(rows summed))).  A kernel given `max` takes its scales
// from them (dev_fixed_mul); with max == nullptr it uses the host's.
struct DevScale {
  const unsigned long long *max;  // [max |g|, max h] or nullptr
  int32_t bits;
  int32_t pad;
};

struct SplitParams {
  double min_child_weight;
  double reg_lambda;
  double g_scale;      // 2^-sg: fixed point -> gradient
  double h_scale;      // 2^-sh: fixed point -> hessian
  int32_t min_samples_leaf;
  int32_t max_depth;
  DevScale dev;
};

// A tree in device form for traversal (node_count entries).
struct TreeNodeDev {
  int32_t feature;     // -1 for a leaf
  int32_t threshold;   // go left when code <= threshold
  int32_t left;
  int32_t right;
  double value;
};

// Partition tiles are runs of 256 * R rows (R = 4, 8 or 16 rows per thread,
// chosen per tree) starting at a 16-row boundary (tiles of one parent are
// consecutive; rows outside the parent's segment are masked).
constexpr int kPartThreads = 256;

// The node table of a tree: a node's split search result (k_node_best),
// its frontier rank and children (k_plan).  Read back once per tree.
struct NodeOut {
  int64_t start;
  int64_t count;
  long long Gq;
  long long Hq;
  double gain;     // best gain (-1e9 when fpos < 0)
  double e;        // smallest best gain on the path from the root
  int32_t fpos;    // best feature position, -1 when none qualifies
  int32_t bin;
  int32_t valid;   // the parent's split was kept
  int32_t left;    // id of the left child (right = left + 1), -1 if not expanded
};

// Result header of one boosting round on the device, read back with the
// tree arrays in one copy.
struct RoundHeader {
  int32_t node_count;  // nodes of the replayed tree, 0 when status != 0
  int32_t status;      // 0 ok; 1 node table too small (needed nodes in
                       // `needed`); 2 a popped node was not expanded;
                       // 3 no free candidate slot; 4 too many leaves for the
                       // device replay; 5 level lists overflowed
  int32_t needed;
  // Profiling counts of the node table, from the in-LDS replay
  // (k_replay_tree): nodes with children, and the rows of the smaller child
  // of every kept split whose children are above max_depth (the rows the
  // level loop histogrammed besides the root's).  expanded is -1 when the
  // replay did not count them (k_replay).
  int32_t expanded;
  double loss_sum;     // sum over rows of y log p + (1-y) log(1-p)
  int64_t hist_rows;
  double pad2[4];
};

struct ReplayArgs {
  double gamma;
  double reg_lambda;
  double g_scale;
  double h_scale;
  DevScale dev;        // device-held scales (SplitParams::dev)
  int32_t max_leaves;
  int32_t out_len;     // 2 * max_leaves + 2 entries per output array
  int32_t stage_limit; // node records are staged in LDS up to this many nodes
  int32_t node_cap;    // node table capacity of the tree
  int32_t max_depth;   // for the profiling counts in RoundHeader
  int32_t pad;
};

// Output arrays of the replayed tree (the reference's 7-tuple layout).
struct TreeArrays {
  int32_t *features;
  int64_t *thresholds;
  double *values;
  int32_t *left;
  int32_t *right;
  double *gains;
};

constexpr int kReplaySlots = 1024;  // candidate slots the device replay holds

// Launchers (kernels.hip).  All are asynchronous on `st`.
hipError_t launch_bin(hipStream_t st, const void *X, int is_f64, int64_t n,
                      int32_t F, const double *edges, int32_t stride,
                      const int32_t *nb, const int32_t *nan_id,
                      int32_t has_any_nan, uint8_t *codes, int64_t ld, int32_t tiers);
hipError_t launch_load_codes(hipStream_t st, const void *src, int is_u16,
                             int64_t n, int32_t F, uint8_t *codes, int64_t ld, int32_t tiers);
hipError_t launch_get_codes(hipStream_t st, const uint8_t *codes, int64_t ld,
                            int64_t n, int32_t F, int32_t tiers, void *dst, int as_u16);
// ghq = (g, h) in fixed point, multiplied by g_mul and h_mul, or by the
// multipliers of the maxima dev holds (dev.max set).
hipError_t launch_quantize(hipStream_t st, const double *g, const double *h,
                           int64_t n, double g_mul, double h_mul, GH *ghq,
                           DevScale dev = DevScale{nullptr, 0, 0});
hipError_t launch_grad_hess(hipStream_t st, const double *F, const uint8_t *y,
                            int64_t n, double w0, double w1, double g_mul,
                            double h_mul, GH *ghq);
hipError_t launch_grad_hess_f64(hipStream_t st, const double *F,
                                const uint8_t *y, int64_t n, double w0,
                                double w1, double *g, double *h);
hipError_t launch_sort_rows(hipStream_t st, const int32_t *rows, int64_t m,
                            uint8_t *flags, int64_t n_pad, int32_t *block_tmp,
                            int32_t *out, bool marked = false);
int64_t sort_rows_flag_bytes(int64_t n);
hipError_t launch_iota(hipStream_t st, int32_t *a, int64_t n);
// a[0, n) = v.
hipError_t launch_fill_f64(hipStream_t st, double *a, int64_t n, double v);
// Work arrays of the device Fisher-Yates (fisher_yates.hip): int32[n] each.
struct FyWork {
  int32_t *head, *next, *v;
  // Sorted form (used when keys is set): (position, step) keys, their sort
  // buffer and counts (sort_u64_ld(n) keys, sort_u64_count_words(n) and
  // 256 words).
  uint64_t *keys = nullptr, *keys_tmp = nullptr;
  uint32_t *counts = nullptr, *totals = nullptr;
  // When set, the kernels read the draws' address from this device word
  // instead of taking `draws`, so that one captured launch sequence serves
  // every round's draws buffer (the word is uploaded with the round's root
  // pack).
  const uint32_t *const *draws_ref = nullptr;
};
// a_new = a_old after the Fisher-Yates steps i = n-1 .. 1 with draws[t] =
// j(n-1-t) <= n-1-t.  With flags (sorted form only), flags[a_new[i]] is also
// set to 1 for every i < m (the in-bag rows of launch_sort_rows).
hipError_t launch_fisher_yates(hipStream_t st, const uint32_t *draws, int64_t n,
                               const int32_t *a_old, int32_t *a_new, const FyWork &w,
                               uint8_t *flags = nullptr, int64_t m = 0);

hipError_t launch_gather_root(hipStream_t st, const uint8_t *codes, int64_t ld,
                              const int32_t *feat, int32_t F_sel,
                              const int32_t *rows32, const int64_t *rows64,
                              int64_t m, const GH *ghq, uint8_t *codes_c,
                              int64_t ld_c, GH *gh_c, int32_t *rid_c,
                              int64_t pad_to, NodeSeg *segs, int32_t *hist_node);
// Root gather in two parts for a boosting round: the codes (when the rows are
// known) and the fixed-point (g, h) with the root segment (when F is).
hipError_t launch_gather_codes(hipStream_t st, const uint8_t *codes, int64_t ld,
                               const int32_t *feat, int32_t F_sel, const int32_t *rows32,
                               int64_t m, uint8_t *codes_c, int64_t ld_c, int64_t pad_to);
hipError_t launch_gather_gh(hipStream_t st, const double *F, const uint8_t *y,
                            const int32_t *rows32, int64_t m, double w0, double w1,
                            double g_mul, double h_mul, DevScale dev, GH *gh_c,
                            int64_t pad_to, NodeSeg *segs, int32_t *hist_node,
                            const LevelPlan *plan_src = nullptr,
                            LevelPlan *plan_dst = nullptr);
// Level kernels take their work counts from a device LevelPlan; the grid
// argument (blocks, tasks or parents) is an upper bound, and blocks loop
// over the work with a grid stride, so any bound >= 1 gives the same result.
// An in-place level's histogram inputs (see launch_hist).
struct SpanLevel {
  const PartParent *parents;  // the level's parents; task.ref indexes them
  const int32_t *tile_cnt;    // their tiles' run counts (PartParent::tile0, tile1)
  int64_t *parent_nleft;      // written: each parent's left rows
  int32_t min_samples_leaf;
};
// With `span` (an in-place level), a task's rows are a tile of its parent's
// segment: the task finds the children's sizes from the tile counts, its
// parent's first task writes the children's segments, whether the split is
// kept and the smaller child (segs, hist_node, parent_nleft), and only the
// rows the split sends to the smaller child are added.
hipError_t launch_hist(hipStream_t st, const uint8_t *codes_c, int64_t ld_c,
                       const GH *gh_c, const HistTask *tasks,
                       const LevelPlan *plan, int32_t max_tasks,
                       int32_t *hist_node, const int32_t *hist_begin,
                       NodeSeg *segs,
                       const int32_t *nb_sel, const int32_t *hot_sel,
                       int32_t F_sel, int32_t fchunk, int32_t copies,
                       unsigned long long *part, unsigned long long *pool,
                       int64_t node_stride, const SpanLevel *span = nullptr,
                       unsigned long long *ktime = nullptr);
int hist_blocks(int32_t n_tasks, int32_t nchunks);
// Per tile, its rows of each of the four runs (tile_cnt[4 * tile + run]).
// groups == nullptr: group i is parent i.
hipError_t launch_part_count(hipStream_t st, const uint8_t *codes_c,
                             int64_t ld_c, const PartParent *parents, const PartGroup *groups,
                             const PartTile *tiles, const LevelPlan *plan,
                             int32_t max_tiles, int32_t part_rows, int32_t *tile_cnt);
// Moves the rows of every group to its parents' children's segments in the
// other set; each group's first tile writes the children's segments.
hipError_t launch_part_scatter(hipStream_t st, const uint8_t *codes_src,
                               uint8_t *codes_dst, int64_t ld_c,
                               const GH *gh_src, GH *gh_dst,
                               const int32_t *rid_src, int32_t *rid_dst,
                               const PartParent *parents, const PartGroup *groups,
                               const PartTile *tiles, const LevelPlan *plan,
                               int32_t max_tiles, int32_t part_rows,
                               const int32_t *tile_begin, const int32_t *tile_cnt,
                               int64_t *parent_nleft, NodeSeg *segs, int32_t *hist_node,
                               int32_t min_samples_leaf, int32_t F_sel);
// Histogram reduction and split search of one level (parents == nullptr:
// the root, node 0, whose tasks hist_begin[0] .. hist_begin[1] built it).
// span_parents: the tasks of parent p tiled its own segment (an in-place
// level), not its smaller child's.
hipError_t launch_reduce_split(hipStream_t st, const LevelPlan *plan, int32_t max_parents,
                               const PartParent *parents, const int32_t *hist_begin,
                               const int32_t *hist_node, const NodeSeg *segs,
                               const unsigned long long *part, unsigned long long *pool,
                               int64_t node_stride, const int32_t *nb_sel, int32_t F_sel,
                               int32_t child_depth, SplitParams p, SplitCand *cand,
                               long long *totals, int32_t span_parents = 0);
hipError_t launch_node_best(hipStream_t st, const NodeSeg *segs,
                            const long long *totals, const SplitCand *cand,
                            int32_t F_sel, const LevelPlan *plan,
                            int32_t max_nodes, int32_t no_split, NodeOut *nodes);
// The last level after its partition count: each parent's scan, its
// children's totals and table records, one wave per parent (grouped: the
// parent's counts are its side's runs in its group's tiles).
hipError_t launch_last_level(hipStream_t st, const PartParent *parents, int32_t grouped,
                             const LevelPlan *plan,
                             int32_t max_parents, const int32_t *tile_begin,
                             const int32_t *tile_cnt, int64_t *parent_nleft, NodeSeg *segs,
                             int32_t *hist_node, int32_t min_samples_leaf,
                             const unsigned long long *pool, int64_t node_stride,
                             long long *totals, NodeOut *nodes);
// One workgroup: picks the level's parents among the nodes created by the
// previous level and writes their PartParent, PartTile and HistTask lists
// and the LevelPlan (see k_plan).
hipError_t launch_plan(hipStream_t st, NodeOut *nodes, LevelPlan *plan,
                       const PartParent *prev_parents, PartParent *parents,
                       int32_t *tile_begin, int32_t *hist_begin,
                       PartTile *tiles, HistTask *hist_tasks,
                       int32_t *work_flag,
                       double *work_e, const NodeSeg *segs, const long long *totals,
                       const SplitCand *cand, int32_t F_sel, PlanArgs a);
// k_plan with its intermediates in LDS, for trees of at most 513 nodes; keeps
// kept_e (node ranks of kept splits, per node) and parent_e (ranks of a
// level's parents, by level parity) for the levels after it.  Plans any
// level mode (a.mode); a grouped level also writes its PartGroup list.
// (k_plan plans kLevelMove levels only.)  With a.fused_count (in-place and
// grouped levels) the launch has 1 + count_blocks blocks: blocks 1.. count
// the level's partition tiles into tile_cnt (codes of set codes_c), as
// k_part_count would for every candidate, while block 0 plans.  level_in
// holds {first candidate, candidates} of this level (written by the
// previous level's planner; unused at level 0, whose only candidate is the
// root) and the planner writes the next level's into level_out.
hipError_t launch_plan_lds(hipStream_t st, NodeOut *nodes, LevelPlan *plan,
                           const PartParent *prev_parents, PartParent *parents,
                           PartGroup *groups,
                           int32_t *tile_begin, int32_t *hist_begin, PartTile *tiles,
                           HistTask *hist_tasks, const NodeSeg *segs,
                           const long long *totals, const SplitCand *cand, double *kept_e,
                           const double *prev_parent_e, double *parent_e, int32_t F_sel,
                           PlanArgs a, const uint8_t *codes_c, int64_t ld_c,
                           int32_t *tile_cnt, const int32_t *level_in, int32_t *level_out,
                           int32_t count_blocks);
// Partition tiles of a level's count: each of `items` rows segments (in
// place: the candidates; grouped: the previous level's parents), from its
// start rounded down to 16, in tiles of part_tile rows, at least one.
constexpr int kCountTilesPerBlock = 4;  // tiles a counting block of the planner launch takes
constexpr int32_t kPlanLdsMaxNodes = 513;
hipError_t launch_code_counts(hipStream_t st, const uint8_t *codes, int64_t ld,
                              int64_t n, int32_t F, unsigned int *counts);
// F += lr * tree(row) for every row unless *node_count_d == 0 (then F is
// left alone); per-block partial sums of the training log-likelihood.
// gh_max_out (optional): raised to the largest |g| and h (logistic_gh with
// weights w0, w1) of the updated F over all rows, one atomic max per block
// that exceeds it; gh_max_clear (optional) is set to zero by block 0.
// tree_len == 0 leaves F unchanged.
hipError_t launch_update_F(hipStream_t st, const uint8_t *codes, int64_t ld,
                           int64_t n, const TreeNodeDev *tree, int32_t tree_len,
                           const int32_t *node_count_d, double lr, double *F,
                           const uint8_t *y, double *loss_partials,
                           int32_t n_blocks, double w0 = 1.0, double w1 = 1.0,
                           unsigned long long *gh_max_out = nullptr,
                           unsigned long long *gh_max_clear = nullptr);
// The reference's best-first candidate loop (est:641-820) over the node
// table, one wave: writes the tree arrays, its TreeNodeDev form and
// hdr->node_count / status.
hipError_t launch_replay(hipStream_t st, const NodeOut *nodes, const LevelPlan *plan,
                         const int32_t *feats, ReplayArgs a, TreeArrays out,
                         TreeNodeDev *tree, RoundHeader *hdr);
// Whether launch_replay takes the in-LDS form, which also fills
// hdr->expanded and hdr->hist_rows.
bool replay_counts_nodes(const ReplayArgs &a);
hipError_t launch_sum_partials(hipStream_t st, const double *partials,
                               int32_t count, double *out);
// Multiclass rounds: scores, gradients and hessians as [K][n] float64, for
// 2 <= K <= kMcMaxK classes.
constexpr int kMcMaxK = 16;
hipError_t launch_mc_grad_hess(hipStream_t st, const double *F, const int32_t *y, const double *w,
                               int64_t n, int32_t K, double *G, double *H,
                               unsigned long long *mx);
// F[:, k] += lr * tree(X); nothing when node_count_d is given and holds 0
// (a device replay that failed).
hipError_t launch_mc_apply(hipStream_t st, const uint8_t *codes, int64_t ld, int64_t n,
                           const TreeNodeDev *tree, const int32_t *node_count_d, double lr,
                           double *Fk);
int64_t mc_loss_blocks(int64_t n);
hipError_t launch_mc_loss(hipStream_t st, const double *F, const int32_t *y, int64_t n,
                          int32_t K, double *partials);
// P[i][k] = softmax over the classes of F[k][i] (row-major n x K output).
hipError_t launch_mc_softmax(hipStream_t st, const double *F, int64_t n, int32_t K, double *P);
hipError_t launch_predict_tree(hipStream_t st, const uint8_t *codes,
                               int64_t ld, int64_t n, const TreeNodeDev *tree,
                               int32_t node_count, double *out);
hipError_t launch_pack_trees(hipStream_t st, const int16_t *features, const int64_t *thresholds,
                             const double *values, const int32_t *left, const int32_t *right,
                             int32_t total, int32_t F, int32_t tiers, TreeNodeDev *nodes);
// Ensemble prediction.  With `chunks` (predict_chunks' list of n_chunks
// runs of whole trees; only when predict_staged_ok) the rows' codes and the
// trees are staged in LDS; otherwise each row walks the trees in HBM.
int32_t predict_chunk_nodes();
// (right_follows_left: every split node's right child is its left child + 1.)
bool predict_staged_ok(int32_t n_cols, int32_t max_tree_nodes, bool right_follows_left);
// Greedy runs of whole trees of at most predict_chunk_nodes() nodes: writes
// the first tree of each run and n_trees after the last (n_trees + 1 entries
// at most); returns the number of runs.
int32_t predict_chunks(const int32_t *offsets, int32_t n_trees, int32_t *chunks);
// out[2i], out[2i + 1] = 1 - p, p with p = 1 / (1 + exp(-clip(F[i] + base,
// -500, 500))); out 16-byte aligned.
hipError_t launch_binary_proba(hipStream_t st, const double *F, int64_t n, double base,
                               double *out);
hipError_t launch_predict(hipStream_t st, const uint8_t *codes, int64_t ld,
                          int64_t n, int32_t n_cols, const TreeNodeDev *nodes,
                          const int32_t *offsets, int32_t n_trees, const int32_t *chunks,
                          int32_t n_chunks, double lr, double *out,
                          hipEvent_t ev_start = nullptr, hipEvent_t ev_stop = nullptr);

int update_F_blocks(int64_t n);

// Column sort for the bin edges (colsort.hip).  Keys are stored
// feature-major [F][ld] with ld = col_sort_ld(n, is_f64); counts holds
// col_sort_count_words(...) words and totals F * 256 words; keys and tmp
// hold F * ld keys of 4 (float32) or 8 (float64) bytes.  Afterwards keys
// holds every column sorted (NaNs last) and m[col] its non-NaN count.
int64_t col_sort_ld(int64_t n, int is_f64);
int64_t col_sort_count_words(int64_t n, int32_t F, int is_f64);
hipError_t launch_col_sort(hipStream_t st, const void *X, int is_f64, int64_t n, int32_t F,
                           void *keys, void *tmp, int64_t ld, uint32_t *counts,
                           uint32_t *totals, int64_t *m);
// out[col] += number of adjacent unequal pairs in the first m[col] keys.
hipError_t launch_col_changes(hipStream_t st, const void *keys, int is_f64, int64_t ld, int32_t F,
                              const int64_t *m, int64_t max_m, unsigned long long *out);
// First position of every run of equal keys among the first m keys of
// column col (unordered, at most max_out stored); *count = number of runs.
hipError_t launch_col_run_starts(hipStream_t st, const void *keys, int is_f64, int64_t ld,
                                 int32_t col, int64_t m, int32_t max_out, int64_t *pos,
                                 unsigned int *count);
// out[k] = value at position pos[k] of sorted column col[k], as float64.
// Stable LSD sort of one padded column of ld 64-bit keys by bits
// [lo_bit, hi_bit) (8-bit digits); *result is the buffer holding it.
int64_t sort_u64_ld(int64_t n);
int64_t sort_u64_count_words(int64_t n);
hipError_t launch_sort_u64(hipStream_t st, uint64_t *keys, uint64_t *tmp, int64_t ld,
                           int lo_bit, int hi_bit, uint32_t *counts, uint32_t *totals,
                           uint64_t **result);
// Key s of the Fisher-Yates sort (s < n): (j(s) << 32) | s for every step
// s >= 1 (self steps included) and (0 << 32) | 0 for position 0; the
// largest key from n on.  draws[t] = j(n - 1 - t).
struct FyKeysIn {
  const uint32_t *draws;
  const uint32_t *const *draws_ref;  // where the draws' address is, or null
  int64_t n;
  __device__ void prepare() {
    if (draws_ref) draws = *draws_ref;
  }
  __device__ uint64_t operator()(int32_t, int64_t s) const {
    if (s >= n) return ~0ull;
    const uint64_t p = s > 0 ? (uint64_t)draws[n - 1 - s] : 0ull;
    return (p << 32) | (uint64_t)s;
  }
};
// The same sort with the first pass reading FyKeysIn (no key array), its
// output in `keys`, later passes alternating with `tmp`.
hipError_t launch_sort_fy_keys(hipStream_t st, FyKeysIn first, uint64_t *keys, uint64_t *tmp,
                               int64_t ld, int lo_bit, int hi_bit, uint32_t *counts,
                               uint32_t *totals, uint64_t **result);
hipError_t launch_col_gather(hipStream_t st, const void *keys, int is_f64, int64_t ld,
                             int64_t count, const int32_t *col, const int64_t *pos, double *out);

}  // namespace bsscl
