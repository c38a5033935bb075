// Engine: device memory, the tree builder's host driver and the C ABI.
//
// Tree building (replaces est:517-823; "est:" is
// src/bsscl_gbm/estimator_v1_0_1.py).
//
// The reference grows a tree best-first: it repeatedly splits the candidate
// leaf with the largest gain, builds the smaller child's histogram, derives
// the larger one by subtraction and scans both for their best splits.  A
// node's histogram and best split depend only on its rows, never on the
// order of the splits, so this engine computes them level by level -- one
// batch of kernels per depth for all nodes of that depth -- and afterwards
// replays the reference's candidate loop (slot table, tie-breaks, rejected
// splits, node numbering) on the host with the computed values.
//
// Which nodes must be expanded: best-first search pops nodes in
// non-increasing order of e(v) = min of the gains on the path from the root
// to v (the node with the largest gain in the frontier always has the
// largest e there).  A node v cannot be split if at least max_leaves-1 kept
// splits u have e(u) > e(v), because all of those come first.  Each level
// expands every frontier node not excluded by that count; the replay
// checks that every node it splits was expanded.
//
// The levels run without host round trips: a one-workgroup planner kernel
// (k_plan) applies that rule on the device and writes the next level's
// work lists, every level kernel reads its counts from the device plan and
// is launched with an upper-bound grid, and the node table comes back to
// the host once per tree for the replay.
#include <hip/hip_runtime.h>

#include <unistd.h>

#include <algorithm>
#include <array>
#include <atomic>
#include <chrono>
#include <cmath>
#include <condition_variable>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "bsscl_internal.h"
#include "kernels.h"

namespace bsscl {

namespace {
thread_local std::string g_last_error;
}

int set_error(int code, const std::string &msg) {
  g_last_error = msg;
  return code;
}

namespace {

#define HIPCHK(expr)                                                          \
  do {                                                                        \
    hipError_t e_ = (expr);                                                   \
    if (e_ != hipSuccess)                                                     \
      return set_error(BSSCL_EDEVICE,                                         \
                       std::string(#expr) + ": " + hipGetErrorString(e_));    \
  } while (0)

#define CHK(expr)                 \
  do {                            \
    int rc_ = (expr);             \
    if (rc_ != BSSCL_OK) return rc_; \
  } while (0)

// Counts device allocations and frees made through DevBuf.  A captured
// round (RoundGraph) holds the addresses of the buffers it uses, so it is
// replayed only while this count is the one it was captured at.
std::atomic<uint64_t> g_alloc_gen{0};

template <typename T>
struct DevBuf {
  T *p = nullptr;
  size_t cap = 0;
  bool tracked = true;  // counted in g_alloc_gen (false: never used by a captured round)
  DevBuf() = default;
  explicit DevBuf(bool counted) : tracked(counted) {}
  int ensure(size_t count) {
    if (count <= cap && p) return BSSCL_OK;
    if (tracked) g_alloc_gen.fetch_add(1, std::memory_order_relaxed);
    if (p) (void)hipFree(p);
    p = nullptr;
    cap = 0;
    const size_t c = std::max<size_t>(count, 1);
    hipError_t e = hipMalloc(reinterpret_cast<void **>(&p), c * sizeof(T));
    if (e != hipSuccess)
      return set_error(BSSCL_ENOMEM, std::string("hipMalloc of ") +
                                         std::to_string(c * sizeof(T)) +
                                         " bytes: " + hipGetErrorString(e));
    cap = c;
    return BSSCL_OK;
  }
  void release() {
    if (p) {
      if (tracked) g_alloc_gen.fetch_add(1, std::memory_order_relaxed);
      (void)hipFree(p);
    }
    p = nullptr;
    cap = 0;
  }
};

// A buffer of the binning and staging calls: no captured round uses it, so
// allocating or freeing it leaves the captured rounds valid.
template <typename T>
struct TempBuf : DevBuf<T> {
  TempBuf() : DevBuf<T>(false) {}
};

// A TempBuf local to one call: freed when the call returns, on every path.
template <typename T>
struct ScopedBuf : TempBuf<T> {
  ScopedBuf() = default;
  ScopedBuf(const ScopedBuf &) = delete;
  ScopedBuf &operator=(const ScopedBuf &) = delete;
  ~ScopedBuf() { this->release(); }
};

// Pinned host staging for the small per-level uploads and readbacks.  Reset
// only after a stream synchronisation, when no copy still reads from it.
struct PinnedArena {
  char *base = nullptr;
  size_t cap = 0, off = 0;
  int reserve(size_t bytes) {
    if (bytes <= cap) return BSSCL_OK;
    if (base) (void)hipHostFree(base);
    base = nullptr;
    cap = 0;
    hipError_t e = hipHostMalloc(reinterpret_cast<void **>(&base), bytes, hipHostMallocDefault);
    if (e != hipSuccess)
      return set_error(BSSCL_ENOMEM, std::string("hipHostMalloc: ") + hipGetErrorString(e));
    cap = bytes;
    off = 0;
    return BSSCL_OK;
  }
  template <typename T>
  T *take(size_t count) {
    size_t o = (off + 255) & ~size_t(255);
    size_t bytes = count * sizeof(T);
    if (o + bytes > cap) return nullptr;
    off = o + bytes;
    return reinterpret_cast<T *>(base + o);
  }
  void reset() { off = 0; }
  void release() {
    if (base) (void)hipHostFree(base);
    base = nullptr;
    cap = off = 0;
  }
};

struct Matrix {
  DevBuf<uint8_t> codes;
  int64_t n = 0, ld = 0;
  int32_t F = 0;
  // Code tiers (kernels.h): column t * F + j holds clamp(code - 255 t, 0,
  // 255) of feature j.  More than one when some feature has more than 256
  // bins (n_bins = 256 with 257 bins is the reference's 'auto' value from 28
  // features on, est:1963-1964), whose codes the reference keeps as uint16
  // (est:2163-2166, 2179-2182).
  int32_t tiers = 1;
  int32_t cols() const { return tiers * F; }
};

struct HNode {
  int32_t parent = -1, depth = 0, left = -1, right = -1;
  int64_t start = 0, count = 0;
  bool valid = true;
  long long Gq = 0, Hq = 0;
  int32_t fpos = -1, bin = 0;
  double gain = -1.0;
  bool expanded = false, split_ok = false;
  int64_t nl = 0, nr = 0;
  double e = 0.0;
};

struct TreeParams {
  int32_t max_leaves, max_depth, min_samples_leaf;
  double mcw, lam, gamma;
};

struct TreeOut {
  int32_t *features;
  int64_t *thresholds;
  double *values;
  int32_t *left, *right;
  int32_t *node_count;
  double *gains;
};

inline int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

// Arguments of bsscl_boost_round that a speculatively enqueued round reuses.
struct RoundArgs {
  int32_t max_leaves = 0, max_depth = 0, min_samples_leaf = 0;
  double min_child_weight = 0.0, reg_lambda = 0.0, gamma = 0.0, learning_rate = 0.0;
  const int32_t *bin_counts = nullptr;
  bool operator==(const RoundArgs &o) const {
    return max_leaves == o.max_leaves && max_depth == o.max_depth &&
           min_samples_leaf == o.min_samples_leaf && min_child_weight == o.min_child_weight &&
           reg_lambda == o.reg_lambda && gamma == o.gamma && learning_rate == o.learning_rate &&
           bin_counts == o.bin_counts;
  }
};

// A boosting round enqueued on the stream and not yet read back.  Its
// readback goes to buffer `buf` (two rounds can be in flight).
struct RoundSlot {
  bool active = false;
  bool device_replay = true;
  bool table_readback = false;  // the node table comes back for tree_stats
  bsscl_sampler *sampler = nullptr;
  void *token = nullptr;
  RoundArgs args;
  int32_t M = 0, run = 0, buf = 0;
  int64_t m = 0;
  std::vector<int32_t> feats, nb_sel;
  hipEvent_t done = nullptr;  // after the round's readback copies
  uint64_t seq = 0;           // tags the round's profiling events
};

// A captured launch sequence of one stream of a boosting round (a HIP
// graph), replayed for every later round whose key matches: the key holds
// every host value the launches take (sizes, parameters, slot, device
// addresses through the allocation count).  Rows graphs: Fisher-Yates, the
// in-bag sort and the root's code gather.  Tree graphs: gradients, root,
// levels, replay and F update, while profiling is off (the histogram
// launches' timing stamps and the event pairs take per-round addresses).
struct RoundGraph {
  std::vector<uint64_t> key;
  hipGraphExec_t exec = nullptr;
  int32_t run = 0;  // tree graphs: levels enqueued
};

}  // namespace
}  // namespace bsscl

using namespace bsscl;

// ---------------------------------------------------------------------------
// Fixed device scratch of bsscl_predict_noalloc: one call's packed tree
// arrays and their traversal form, so that call allocates nothing.  Each GPU
// holds its own copy of the array at its own address, looked up once per
// device with that device current (scratch_for_device) and kept; host code
// passes only those addresses to copies and kernels, never the symbol.
// Calls on one GPU share its copy: overlapping calls race.
// ---------------------------------------------------------------------------
namespace {
constexpr int32_t kNoAllocMaxNodes = 1 << 17;   // nodes of all trees of a call
constexpr int32_t kNoAllocMaxTrees = 1 << 14;
constexpr size_t align256(size_t b) { return (b + 255) & ~size_t(255); }
constexpr size_t kScrNodes = 0;
constexpr size_t kScrFeat = kScrNodes + align256(sizeof(TreeNodeDev) * kNoAllocMaxNodes);
constexpr size_t kScrThr = kScrFeat + align256(sizeof(int16_t) * kNoAllocMaxNodes);
constexpr size_t kScrVal = kScrThr + align256(sizeof(int64_t) * kNoAllocMaxNodes);
constexpr size_t kScrLeft = kScrVal + align256(sizeof(double) * kNoAllocMaxNodes);
constexpr size_t kScrRight = kScrLeft + align256(sizeof(int32_t) * kNoAllocMaxNodes);
constexpr size_t kScrOffs = kScrRight + align256(sizeof(int32_t) * kNoAllocMaxNodes);
constexpr size_t kScrChunks = kScrOffs + align256(sizeof(int32_t) * (kNoAllocMaxTrees + 1));
constexpr size_t kScratchBytes = kScrChunks + align256(sizeof(int32_t) * (kNoAllocMaxTrees + 1));
static_assert(kScratchBytes <= (7u << 20), "noalloc scratch stays under 7 MiB");
constexpr int kMaxDevices = 64;
}  // namespace

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
std::mutex g_scratch_mu;
unsigned char *g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on `device`, which must be current.
int scratch_for_device(int device, unsigned char **out) {
  if (device < 0 || device >= kMaxDevices)
    return set_error(BSSCL_EDEVICE, "device index beyond the scratch table");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(BSSCL_EDEVICE, std::string("hipGetSymbolAddress(scratch): ") +
                                          hipGetErrorString(e));
    g_scratch_ptr[device] = static_cast<unsigned char *>(p);
  }
  *out = g_scratch_ptr[device];
  return BSSCL_OK;
}
}  // namespace

struct bsscl_engine {
  int32_t device = 0;
  hipStream_t st = nullptr;
  unsigned char *scratch_p = nullptr;  // this device's copy of `scratch`
  // A boosting round's in-bag rows (Fisher-Yates, sort) are made on their
  // own stream, so the next round's rows are ready while this round's tree
  // is built; the tree stream waits on rows_ready of its slot.
  hipStream_t st_rows = nullptr;
  hipEvent_t rows_ready[2] = {nullptr, nullptr};
  int32_t n_cu = 256;
  size_t max_lds = 64 * 1024;
  Matrix mat[2];

  // Boosting run on matrix 0.
  bool boosting = false;
  DevBuf<double> F;
  DevBuf<uint8_t> y;
  double w0 = 1.0, w1 = 1.0;
  DevBuf<GH> ghq;
  DevBuf<double> g64, h64;
  double g_scale = 1.0, h_scale = 1.0;  // fixed point -> value
  double h_bound = 0.0;  // no hessian of the current tree's rows exceeds this
  // The largest |g| and h over all rows of the current F, as k_update_F
  // leaves them: two slots of [max |g|, max h].  gh_slot holds the current
  // F's; the update that makes the next F raises the other slot and clears
  // this one.  A boosting round on the device path scales its tree's fixed
  // point from them (gh_ok; BSSCL_TEST_BOUND_SCALE=1 keeps the bound
  // max(w0, w1) instead).
  DevBuf<unsigned long long> ghmax_d;
  int32_t gh_slot = 0;
  bool gh_ok = false;
  DevScale round_dev{nullptr, 0, 0};  // the tree being enqueued (split_params)

  // Multiclass run on matrix 0: scores, gradients and hessians [K][n], the
  // rows' class and weight, each class's largest |g| and h of the round.
  int32_t mc_K = 0;
  int64_t mc_m = 0;  // the round's in-bag rows: mc_rows32 (int32) or, when null, rows64
  const int32_t *mc_rows32 = nullptr;
  // A round enqueued ahead by bsscl_mc_round_trees: its rows in
  // round_rows[mc_next_slot], made on the rows stream (complete at
  // mc_next_ev), its sampler round held until the next call.
  bool mc_next = false;
  int mc_next_slot = 0;
  void *mc_next_token = nullptr;
  bsscl_sampler *mc_next_sampler = nullptr;
  std::vector<int32_t> mc_next_feats;
  hipEvent_t mc_next_ev = nullptr;
  int mc_slot = 0;  // round_rows slot of the next round taken directly
  DevBuf<double> mc_F, mc_G, mc_H, mc_w, mc_part;
  DevBuf<int32_t> mc_y;
  DevBuf<unsigned long long> mc_max;
  std::vector<double> mc_gm, mc_hm;  // fixed-point multipliers per class
  std::vector<double> mc_hmax;       // largest hessian per class
  // Whether mc_gm, mc_hm and mc_hmax hold this round's values; a round of
  // bsscl_mc_round_trees leaves its maxima on the device (mc_max) and its
  // trees take their scales there.
  bool mc_scales_host = false;
  double mc_hbound = 0.0;  // no multiclass hessian exceeds this (max weight / 4)
  DevBuf<int32_t> mc_feat_d;  // the round's engine columns (its root codes' gather)
  // A multiclass round's K trees as the device replayed them: K blocks of
  // round_out_bytes(2 * max_leaves + 2), and their pinned readback.
  DevBuf<char> mc_out_d;
  char *mc_out_pin = nullptr;
  size_t mc_out_pin_bytes = 0;

  // Tree workspace.
  // Compact row sets: a tree uses sets set_base and set_base + 1 (levels
  // alternate); a boosting round in slot s uses base 2s, so the next round's
  // root codes are gathered while this round's tree still reads its own.
  DevBuf<uint8_t> codes_c[4];
  DevBuf<GH> gh_c[4];
  DevBuf<int32_t> rid_c[2];  // with set_base 0 only
  int32_t set_base = 0;
  // A tree's root rows in another set than set_base (-1: set_base).  Its
  // levels then never write it, so the root codes of a multiclass round,
  // gathered once, serve all its classes (root_codes_ready: the root's
  // gather brings the (g,h) alone).
  int32_t root_set = -1;
  bool root_codes_ready = false;
  // A boosting round's root inputs (RootPack), uploaded by the rows stream
  // into the slot's own arena.
  DevBuf<char> root_d[2];
  char *root_pin[2] = {nullptr, nullptr};
  size_t root_pin_n[2] = {0, 0};
  bool track_rid = false;  // carry row ids through the partition (bsscl_partition)
  int64_t ld_c = 0;
  DevBuf<int32_t> round_rows[2];  // in-bag rows of round slot s, ascending
  DevBuf<int64_t> rows64;
  DevBuf<int32_t> rows_in, sort_tmp;
  // Row permutation of a device-rows sampler (cumulative over its rounds)
  // and the Fisher-Yates work arrays.
  DevBuf<int32_t> perm[2];
  int perm_cur = 0;
  const void *perm_sampler = nullptr;
  int32_t perm_next_round = 0;
  DevBuf<int32_t> fy_head, fy_next, fy_v;
  DevBuf<uint64_t> fy_keys[2];       // sorted Fisher-Yates form (long shuffles)
  DevBuf<uint32_t> fy_counts, fy_totals;
  DevBuf<uint8_t> row_flags;  // all zero between rounds
  int64_t row_flags_n = 0;
  // Node-indexed buffers (node_cap nodes) and the level lists the planner
  // writes (see ensure_nodes / prepare_tree_buffers for their sizes).
  DevBuf<unsigned long long> pool;
  DevBuf<unsigned long long> part_d;  // per-task partial histograms [task][F_sel][bin][g,h]
  int32_t node_alloc = 0;      // nodes the node-indexed buffers were sized for
  int32_t node_cap = 0;        // nodes the planner may create in this tree
  int32_t node_cap_floor = 0;  // raised when a tree needed more nodes
  int64_t node_stride = 0;     // int64 words per node histogram
  DevBuf<NodeSeg> segs;
  DevBuf<SplitCand> cand;
  DevBuf<long long> totals;
  DevBuf<char> table_d;               // [LevelPlan, padded to 64 B][NodeOut x node_cap]
  char *table_pin = nullptr;          // pinned readback of table_d
  size_t table_pin_bytes = 0;
  LevelPlan *plan_d = nullptr;
  NodeOut *nodes_d = nullptr;
  DevBuf<PartParent> parents_d[2];    // by level parity
  DevBuf<PartGroup> groups_d;         // a grouped level's partition groups
  // Rows move every second level (in-place and grouped levels alternate;
  // with the LDS planner) instead of at every level.
  bool pair_levels = false;
  DevBuf<int32_t> tile_begin_d, hist_begin_d, work_flag_d, hist_node_d;
  DevBuf<double> work_e_d;
  // Planner in LDS (trees of at most kPlanLdsMaxNodes nodes): ranks of kept
  // splits per node and of each level's parents (by level parity).
  bool plan_lds = false;
  DevBuf<double> kept_e_d, parent_e_d[2];
  DevBuf<int64_t> nleft_d;
  int32_t tile_cap = 0, hist_cap = 0;
  DevBuf<PartTile> tiles_d;
  DevBuf<int32_t> tile_cnt_d;         // per partition tile: its rows of the four runs
  // {first candidate, candidates} of the next level, by level parity: the
  // planner of level d writes slot (d + 1) & 1 for level d + 1's counting
  // blocks (which cannot read the plan that level's planner rewrites).
  DevBuf<int32_t> level_args_d;
  DevBuf<HistTask> hist_tasks_d;
  DevBuf<char> lvl_d;                 // packed inputs of the root (one upload per tree)
  const int32_t *feat_d = nullptr;    // selected feature indices
  const int32_t *nb_sel_d = nullptr;  // bin counts of the selected features
  const int32_t *hot_sel_d = nullptr; // most frequent bin of each selected feature
  std::vector<int32_t> hot_bin;       // most frequent code per feature of matrix 0
  DevBuf<TreeNodeDev> tree_d;
  DevBuf<char> round_d[2];            // RoundHeader + tree arrays of a round
  char *round_pin[2] = {nullptr, nullptr};   // pinned readbacks of round_d
  size_t round_pin_bytes[2] = {0, 0};
  char *rtable_pin[2] = {nullptr, nullptr};  // node-table readbacks (profiling)
  size_t rtable_pin_bytes[2] = {0, 0};
  RoundSlot rslot[2];
  int32_t rslot_next = 0;
  // Captured rounds by slot (off with BSSCL_GRAPHS=0, and after a capture
  // that failed); the first boosting round of an engine runs uncaptured.
  RoundGraph rows_graph[2], tree_graph[2];
  bool graphs = true;
  bool launched_round = false;
  bool pipeline = false;   // enqueue the next round before returning one
  int32_t ahead = -1;      // slot of a round enqueued ahead, or -1
  uint64_t round_seq = 0;
  DevBuf<int32_t> offsets_d;
  DevBuf<double> partials_d, loss_d, out_d, proba_d;
  PinnedArena pin;
  // Large host transfers go through these pinned chunks (host_upload,
  // host_download), and binning of a host matrix through xchunk.
  char *xfer_pin[3] = {nullptr, nullptr, nullptr};
  hipEvent_t xfer_ev[3] = {nullptr, nullptr, nullptr};
  int xfer_next = 0;  // the pinned chunk the next piece goes through
  TempBuf<unsigned char> xchunk;
  // bsscl_predict_proba_rows: the second row chunk of X, one chunk's codes,
  // and its events (chunk uploaded, chunk binned; two of each).
  TempBuf<unsigned char> xchunk2;
  TempBuf<uint8_t> pcodes;
  hipEvent_t pipe_ev[4] = {nullptr, nullptr, nullptr, nullptr};
  // The bin edges, bin counts and NaN bins of the last binning call.
  TempBuf<double> edges_d;
  TempBuf<int32_t> nbins_d, nanid_d;

  // Feature matrix staged by bsscl_stage_features (row-major, as given) and
  // its columns sorted by bsscl_sort_columns (keys [F][col_ld]).
  TempBuf<unsigned char> xstage;
  int64_t xs_n = 0;
  int32_t xs_F = 0, xs_f64 = 0;
  TempBuf<unsigned char> col_keys;
  int64_t col_ld = 0;
  bool cols_sorted = false;
  std::vector<int64_t> col_m;  // non-NaN values per sorted column
  // The column sort's work buffers: the keys' other half of each pass,
  // digit counts and totals, per-column counts.
  TempBuf<unsigned char> col_tmp;
  TempBuf<uint32_t> col_counts, col_totals;
  TempBuf<int64_t> col_m_d;
  TempBuf<unsigned long long> col_changes_d;
  // bsscl_sorted_gather's columns, ranks and values.
  TempBuf<int32_t> gather_c;
  TempBuf<int64_t> gather_p;
  TempBuf<double> gather_o;

  // Histogram launch shape of the current tree (see read_hist_tuning,
  // hist_fchunk, hist_tile_rows); tunable with BSSCL_HIST_FC,
  // BSSCL_HIST_BLOCKS_PER_CU and BSSCL_HIST_ROWS_PER_FLUSH.
  int32_t hist_fc = 1;
  int32_t hist_copies = 4;
  // The same for the in-place levels' histograms (BSSCL_HIST_SPAN_FC,
  // BSSCL_HIST_SPAN_COPIES).
  int32_t hist_fc_span = 1;
  int32_t hist_copies_span = 1;
  // Partition tile of the current tree: 256 threads x part_rows rows.
  int32_t part_rows = 4;
  int32_t part_tile = 1024;
  int32_t hist_blocks_per_cu = 8;
  int32_t hist_rows_per_flush = 10240;       // the root's tiles
  int32_t hist_rows_per_flush_level = 2560;  // the planned levels' tiles

  // Profiling.
  int prof = 0;  // 0 off, 1 histogram kernel timed, 2 every kernel group timed
  std::vector<hipEvent_t> ev_pool;  // every timing event (destroyed with the engine)
  std::vector<hipEvent_t> ev_free;
  struct Pending {
    hipEvent_t a, b;
    int kind;      // 0 hist, 1 partition, 2 split
    uint64_t seq;  // boosting round that recorded them
  };
  std::vector<Pending> pending;
  // Histogram launches timed by the kernel itself: slot k holds the first
  // block's start and the last block's end on the device's constant-rate
  // clock (no event packets between the tree's kernels, which would each
  // hold the queue for several microseconds).
  DevBuf<unsigned long long> ktime_d;
  size_t ktime_used = 0;                                   // words
  std::vector<std::pair<size_t, size_t>> ktime_launches;  // (first word, blocks)
  double wall_khz = 0.0;
  double stats[21] = {0};
};

namespace bsscl {
namespace {

// Two timing events from the free list (created when it is empty).
int ev_pair(bsscl_engine *E, hipEvent_t &a, hipEvent_t &b) {
  while (E->ev_free.size() < 2) {
    hipEvent_t ev;
    HIPCHK(hipEventCreate(&ev));
    E->ev_pool.push_back(ev);
    E->ev_free.push_back(ev);
  }
  a = E->ev_free.back();
  E->ev_free.pop_back();
  b = E->ev_free.back();
  E->ev_free.pop_back();
  return BSSCL_OK;
}

// Starts a timed region of `kind` when profiling; returns the stop event.
int prof_begin(bsscl_engine *E, int kind, hipEvent_t *stop) {
  *stop = nullptr;
  // Level 1 times the histogram kernel only; level 2 every kernel group
  // (each event pair costs a few microseconds of queue time).
  if (E->prof < (kind == 0 ? 1 : 2)) return BSSCL_OK;
  hipEvent_t a, b;
  CHK(ev_pair(E, a, b));
  HIPCHK(hipEventRecord(a, E->st));
  E->pending.push_back({a, b, kind, E->round_seq});
  *stop = b;
  return BSSCL_OK;
}

// The start/stop events of one timed kernel of `kind` (4 prediction),
// recorded by that kernel's own dispatch (hipExtLaunchKernelGGL), so the
// time is the kernel's execution alone; null events when not profiling.
// (Histogram launches are timed by the kernel itself: prof_slot.)
int prof_kernel(bsscl_engine *E, int kind, hipEvent_t *start, hipEvent_t *stop) {
  *start = *stop = nullptr;
  if (E->prof < 1) return BSSCL_OK;
  if (kind == 0) return BSSCL_OK;  // histograms: prof_slot
  hipEvent_t a, b;
  CHK(ev_pair(E, a, b));
  E->pending.push_back({a, b, kind, E->round_seq});
  *start = a;
  *stop = b;
  return BSSCL_OK;
}

// Per-block (start, end) pairs of one histogram launch of `blocks` blocks
// when profiling (null otherwise, or when this profiling run's space is
// used up).
constexpr size_t kTimeWords = (size_t)1 << 22;  // 32 MB of pairs

unsigned long long *prof_slot(bsscl_engine *E, int64_t blocks) {
  if (E->prof < 1 || blocks <= 0) return nullptr;
  if (!E->ktime_d.p && E->ktime_d.ensure(kTimeWords) != BSSCL_OK) return nullptr;
  if (E->ktime_used + 2 * (size_t)blocks > kTimeWords) return nullptr;
  unsigned long long *p = E->ktime_d.p + E->ktime_used;
  E->ktime_launches.push_back({E->ktime_used, (size_t)blocks});
  E->ktime_used += 2 * (size_t)blocks;
  return p;
}

// Folds the recorded launches into the histogram timings (after a
// synchronisation): each launch from its first block's start to its last
// block's end.
int prof_slots_collect(bsscl_engine *E) {
  if (E->ktime_launches.empty()) return BSSCL_OK;
  std::vector<unsigned long long> t(E->ktime_used);
  HIPCHK(hipMemcpy(t.data(), E->ktime_d.p, t.size() * 8, hipMemcpyDeviceToHost));
  for (const auto &L : E->ktime_launches) {
    unsigned long long a = ~0ull, b = 0ull;
    for (size_t k = 0; k < L.second; ++k) {
      a = std::min(a, t[L.first + 2 * k]);
      b = std::max(b, t[L.first + 2 * k + 1]);
    }
    if (b < a) continue;
    E->stats[0] += 1.0;
    E->stats[1] += (double)(b - a) / E->wall_khz;  // ms
  }
  E->ktime_launches.clear();
  E->ktime_used = 0;
  return BSSCL_OK;
}

int prof_end(bsscl_engine *E, hipEvent_t stop) {
  if (stop) HIPCHK(hipEventRecord(stop, E->st));
  return BSSCL_OK;
}

// Folds finished timings into stats: every pending pair after a stream
// synchronisation, or those of rounds up to `upto` once they are done.
int prof_collect(bsscl_engine *E, uint64_t upto = UINT64_MAX) {
  std::vector<bsscl_engine::Pending> keep;
  for (const auto &p : E->pending) {
    if (p.seq > upto) {
      keep.push_back(p);
      continue;
    }
    float ms = 0.f;
    HIPCHK(hipEventElapsedTime(&ms, p.a, p.b));
    const int slot = p.kind == 0 ? 0 : p.kind == 1 ? 4 : p.kind == 2 ? 6 : p.kind == 4 ? 16 : 12;
    E->stats[slot] += 1.0;
    E->stats[slot + 1] += (double)ms;
    E->ev_free.push_back(p.a);
    E->ev_free.push_back(p.b);
  }
  E->pending.swap(keep);
  return BSSCL_OK;
}

int sync(bsscl_engine *E) {
  HIPCHK(hipStreamSynchronize(E->st_rows));
  HIPCHK(hipStreamSynchronize(E->st));
  CHK(prof_collect(E));
  E->pin.reset();
  return BSSCL_OK;
}

template <typename T>
int upload(bsscl_engine *E, DevBuf<T> &dst, const T *src, size_t count) {
  CHK(dst.ensure(count));
  if (count == 0) return BSSCL_OK;
  T *stage = E->pin.take<T>(count);
  if (stage) {
    std::memcpy(stage, src, count * sizeof(T));
    HIPCHK(hipMemcpyAsync(dst.p, stage, count * sizeof(T), hipMemcpyHostToDevice, E->st));
  } else {
    HIPCHK(hipMemcpyAsync(dst.p, src, count * sizeof(T), hipMemcpyHostToDevice, E->st));
    HIPCHK(hipStreamSynchronize(E->st));
  }
  return BSSCL_OK;
}

// ---------------------------------------------------------------------------
// Large host <-> device transfers.  A copy from pageable memory makes HIP
// stage it through its own pinned buffers, one after the other (about
// 19 GB/s for a 112 MB matrix, 27-29 GB/s for 2 GB).  Here host threads
// copy chunks into three pinned buffers while the DMA engine moves the
// chunk before, so both run at once, and the DMA engine sets the rate.
// ---------------------------------------------------------------------------

// A few host threads that split a memcpy with the caller.  One pool per
// process: a child made by fork() has none of its parent's threads, so it
// starts its own.  The threads live until the process ends.
class CopyPool {
 public:
  static CopyPool &get() {
    static std::mutex mu;
    static CopyPool *pool = nullptr;
    static pid_t owner = 0;
    std::lock_guard<std::mutex> lk(mu);
    if (!pool || owner != getpid()) {  // (the parent's pool is left as it is)
      pool = new CopyPool();
      owner = getpid();
    }
    return *pool;
  }

  void copy(void *dst, const void *src, size_t bytes) {
    if (bytes < (1u << 20) || threads_.empty()) {
      std::memcpy(dst, src, bytes);
      return;
    }
    std::lock_guard<std::mutex> call(call_mu_);  // one copy at a time
    {
      std::lock_guard<std::mutex> lk(mu_);
      dst_ = static_cast<char *>(dst);
      src_ = static_cast<const char *>(src);
      bytes_ = bytes;
      pending_ = (int)threads_.size();
      ++gen_;
    }
    cv_.notify_all();
    part(0, dst_, src_, bytes);
    std::unique_lock<std::mutex> lk(mu_);
    done_.wait(lk, [&] { return pending_ == 0; });
  }

 private:
  CopyPool() {
    const unsigned hw = std::thread::hardware_concurrency();
    const int n = (int)std::min<unsigned>(3, hw > 2 ? hw / 2 - 1 : 0);
    for (int t = 0; t < n; ++t) {
      try {
        threads_.emplace_back([this, t] { run(t + 1); });
      } catch (...) {
        break;  // fewer threads
      }
    }
    for (auto &th : threads_) th.detach();
  }

  // Part i of parts() pieces, cut at 64-byte boundaries.
  void part(int i, char *d, const char *s, size_t b) const {
    const size_t parts = threads_.size() + 1;
    const size_t per = ((b + parts - 1) / parts + 63) & ~size_t(63);
    const size_t off = per * (size_t)i;
    if (off < b) std::memcpy(d + off, s + off, std::min(per, b - off));
  }

  void run(int i) {
    uint64_t seen = 0;
    std::unique_lock<std::mutex> lk(mu_);
    for (;;) {
      cv_.wait(lk, [&] { return gen_ != seen; });
      seen = gen_;
      char *d = dst_;
      const char *s = src_;
      const size_t b = bytes_;
      lk.unlock();
      part(i, d, s, b);
      lk.lock();
      if (--pending_ == 0) done_.notify_one();
    }
  }

  std::mutex call_mu_, mu_;
  std::condition_variable cv_, done_;
  std::vector<std::thread> threads_;
  uint64_t gen_ = 0;
  int pending_ = 0;
  char *dst_ = nullptr;
  const char *src_ = nullptr;
  size_t bytes_ = 0;
};

// Chunks of 8 MB keep small transfers pipelined; from 512 MB on, 32 MB
// chunks reach 55 GB/s host to device against 52 (10M x 50 float32: 36 ms;
// HIP's own pageable copy 69-73 ms).
constexpr size_t kXferChunkMax = 32u << 20;
size_t xfer_chunk(size_t bytes) { return bytes >= (512u << 20) ? kXferChunkMax : 8u << 20; }

int ensure_xfer(bsscl_engine *E) {
  for (int b = 0; b < 3; ++b) {
    if (!E->xfer_pin[b])
      HIPCHK(hipHostMalloc(reinterpret_cast<void **>(&E->xfer_pin[b]), kXferChunkMax,
                           hipHostMallocDefault));
    if (!E->xfer_ev[b]) HIPCHK(hipEventCreateWithFlags(&E->xfer_ev[b], hipEventDisableTiming));
  }
  return BSSCL_OK;
}

// Enqueues dst (device) = src (host, pageable) on stream `st` in pieces of
// `piece` bytes through the pinned chunks, and returns once the last piece
// has been copied into its pinned chunk; the copies complete on `st`.  A
// pinned chunk is refilled only after the copy that last read it, whichever
// call or stream enqueued that one.
int host_upload_async(bsscl_engine *E, hipStream_t st, void *dst, const void *src, size_t bytes,
                      size_t piece) {
  if (bytes < 2 * piece) {
    HIPCHK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, st));
    return BSSCL_OK;
  }
  CHK(ensure_xfer(E));
  CopyPool &pool = CopyPool::get();
  for (size_t off = 0; off < bytes; off += piece) {
    const int b = E->xfer_next;
    E->xfer_next = (b + 1) % 3;
    const size_t len = std::min(piece, bytes - off);
    HIPCHK(hipEventSynchronize(E->xfer_ev[b]));  // its previous piece has gone
    pool.copy(E->xfer_pin[b], static_cast<const char *>(src) + off, len);
    HIPCHK(hipMemcpyAsync(static_cast<char *>(dst) + off, E->xfer_pin[b], len,
                          hipMemcpyHostToDevice, st));
    HIPCHK(hipEventRecord(E->xfer_ev[b], st));
  }
  return BSSCL_OK;
}

// dst (device) = src (host, pageable) on E->st; returns once the copy is
// complete.
int host_upload(bsscl_engine *E, void *dst, const void *src, size_t bytes) {
  CHK(host_upload_async(E, E->st, dst, src, bytes, xfer_chunk(bytes)));
  HIPCHK(hipStreamSynchronize(E->st));
  return BSSCL_OK;
}

// dst (host, pageable) = src (device) after the work already on stream
// `st`; returns once dst holds it.
int host_download_on(bsscl_engine *E, hipStream_t st, void *dst, const void *src, size_t bytes) {
  const size_t chunk = xfer_chunk(bytes);
  if (bytes < 2 * chunk) {
    HIPCHK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, st));
    HIPCHK(hipStreamSynchronize(st));
    return BSSCL_OK;
  }
  CHK(ensure_xfer(E));
  CopyPool &pool = CopyPool::get();
  const size_t n_chunks = (bytes + chunk - 1) / chunk;
  auto enqueue = [&](size_t c) -> int {
    const int b = (int)(c % 3);
    const size_t off = c * chunk;
    HIPCHK(hipEventSynchronize(E->xfer_ev[b]));  // no upload still reads the chunk
    HIPCHK(hipMemcpyAsync(E->xfer_pin[b], static_cast<const char *>(src) + off,
                          std::min(chunk, bytes - off), hipMemcpyDeviceToHost, st));
    HIPCHK(hipEventRecord(E->xfer_ev[b], st));
    return BSSCL_OK;
  };
  // Two chunks in flight ahead of the one being copied out.
  for (size_t c = 0; c < std::min<size_t>(2, n_chunks); ++c) CHK(enqueue(c));
  for (size_t c = 0; c < n_chunks; ++c) {
    if (c + 2 < n_chunks) CHK(enqueue(c + 2));
    const int b = (int)(c % 3);
    HIPCHK(hipEventSynchronize(E->xfer_ev[b]));
    const size_t off = c * chunk;
    pool.copy(static_cast<char *>(dst) + off, E->xfer_pin[b], std::min(chunk, bytes - off));
  }
  return BSSCL_OK;
}

// dst (host, pageable) = src (device) after the work already on E->st.
int host_download(bsscl_engine *E, void *dst, const void *src, size_t bytes) {
  return host_download_on(E, E->st, dst, src, bytes);
}

// Code tiers and NaN presence of binning with these bin counts (checked).
int bin_layout(int32_t F, int32_t edge_stride, const int32_t *bin_counts,
               const int32_t *nan_bin_id, int32_t *tiers, int32_t *has_any_nan) {
  *tiers = 1;
  *has_any_nan = 0;
  for (int32_t j = 0; j < F; ++j) {
    if (bin_counts[j] < 1 || bin_counts[j] >= edge_stride)
      return set_error(BSSCL_EINVAL, "bin_features: bin_counts must be in [1, edge_stride)");
    if (bin_counts[j] > kMaxBinCount)
      return set_error(BSSCL_EINVAL, "bin_features: more than 65536 bins");
    // Training codes are at most nb - 1, which these tiers hold exactly.
    *tiers = std::max(*tiers, tiers_for_bins(bin_counts[j]));
    if (nan_bin_id[j] >= 0) *has_any_nan = 1;
  }
  return BSSCL_OK;
}

// A binning call's edges [F][edge_stride], bin counts and NaN bins into
// E->edges_d, nbins_d and nanid_d (on E->st).
int upload_edges(bsscl_engine *E, int32_t F, const double *edges_2d, int32_t edge_stride,
                 const int32_t *bin_counts, const int32_t *nan_bin_id) {
  CHK(E->edges_d.ensure((size_t)F * edge_stride));
  CHK(E->nbins_d.ensure((size_t)F));
  CHK(E->nanid_d.ensure((size_t)F));
  HIPCHK(hipMemcpyAsync(E->edges_d.p, edges_2d, (size_t)F * edge_stride * 8,
                        hipMemcpyHostToDevice, E->st));
  HIPCHK(hipMemcpyAsync(E->nbins_d.p, bin_counts, (size_t)F * 4, hipMemcpyHostToDevice, E->st));
  HIPCHK(hipMemcpyAsync(E->nanid_d.p, nan_bin_id, (size_t)F * 4, hipMemcpyHostToDevice, E->st));
  return BSSCL_OK;
}

// The staged matrix, its sorted columns and the sort's work buffers.
void release_staging(bsscl_engine *E) {
  E->xstage.release();
  E->col_keys.release();
  E->col_tmp.release();
  E->col_counts.release();
  E->col_totals.release();
  E->col_m_d.release();
  E->col_changes_d.release();
  E->gather_c.release();
  E->gather_p.release();
  E->gather_o.release();
  E->xs_n = 0;
  E->cols_sorted = false;
  E->col_m.clear();
}

// Staging memory up to this size stays allocated for the next fit's
// staging (1M x 28 float32: 0.75 ms of hipFree and the allocations again,
// in a 47 ms fit); larger staging is freed when the edges are done.
constexpr size_t kStagingKeptBytes = size_t(1) << 30;

int check_matrix(bsscl_engine *E, int32_t slot) {
  if (slot < 0 || slot > 1) return set_error(BSSCL_EINVAL, "matrix slot must be 0 or 1");
  if (!E->mat[slot].codes.p || E->mat[slot].n <= 0)
    return set_error(BSSCL_EINVAL, "matrix slot " + std::to_string(slot) + " is empty");
  return BSSCL_OK;
}

int alloc_matrix(bsscl_engine *E, int32_t slot, int64_t n, int32_t F, int32_t tiers = 1) {
  Matrix &M = E->mat[slot];
  const int64_t ld = round_up(n + 8, 256);
  const size_t bytes = (size_t)ld * (size_t)F * (size_t)tiers;
  CHK(M.codes.ensure(bytes));
  HIPCHK(hipMemsetAsync(M.codes.p, 0, bytes, E->st));
  M.n = n;
  M.ld = ld;
  M.F = F;
  M.tiers = tiers;
  return BSSCL_OK;
}

// Gives matrix `slot` at least `tiers` code tiers.  Its codes are held
// exactly by the tiers it has (codes <= 255 * M.tiers), so the added tiers
// are zero.
int ensure_tiers(bsscl_engine *E, int32_t slot, int32_t tiers) {
  Matrix &M = E->mat[slot];
  if (M.tiers >= tiers) return BSSCL_OK;
  const size_t have = (size_t)M.ld * (size_t)M.F * (size_t)M.tiers;
  const size_t want = (size_t)M.ld * (size_t)M.F * (size_t)tiers;
  DevBuf<uint8_t> wide;
  CHK(wide.ensure(want));
  HIPCHK(hipMemcpyAsync(wide.p, M.codes.p, have, hipMemcpyDeviceToDevice, E->st));
  HIPCHK(hipMemsetAsync(wide.p + have, 0, want - have, E->st));
  HIPCHK(hipStreamSynchronize(E->st));
  std::swap(M.codes, wide);
  wide.release();
  M.tiers = tiers;
  return BSSCL_OK;
}

// Engine columns of a tree's selected features (ascending feature ids, each
// with bin count nb in [1, kMaxBinCount]): the feature's tier-0 column and,
// right after it for a feature of more than 256 bins, its tiers 1 .. k - 1
// (k = tiers_for_bins(nb)), tier t with min(256, nb - 255 t) bins.  The
// reference's candidates (j, 255 t + b) are tier t's candidates (t F + j, b),
// listed in the reference's order (est:611-621), so the argmax and its
// strict-'>' tie-breaks pick the same split.
int expand_features(const Matrix &X, const std::vector<int32_t> &feats,
                    const std::vector<int32_t> &nb, std::vector<int32_t> &cols,
                    std::vector<int32_t> &nb_cols) {
  cols.clear();
  nb_cols.clear();
  for (size_t i = 0; i < feats.size(); ++i) {
    const int32_t k = tiers_for_bins(nb[i]);
    if (k > X.tiers)
      return set_error(BSSCL_EINVAL, "feature " + std::to_string(feats[i]) + " has " +
                                         std::to_string(nb[i]) +
                                         " bins but the matrix holds smaller codes");
    for (int32_t t = 0; t < k; ++t) {
      cols.push_back(t * X.F + feats[i]);
      nb_cols.push_back(std::min(kBins, nb[i] - 255 * t));
    }
  }
  return BSSCL_OK;
}

// Scale 2^s of the 64-bit fixed-point values of a tree whose sums run over at
// most `rows` rows: every row's |v| * 2^s < 2^B with B = 62 - ceil(log2(rows)),
// so any such sum (and the difference of two nested ones) fits in int64.
// The widest exponent the sums allow: a bin of many tiny, equal hessians
// (confident rows late in a fit) then keeps its relative precision.
int32_t fixed_bits(int64_t rows) {
  int lg = 1;
  while (lg < 62 && (int64_t(1) << lg) < rows) ++lg;
  return 62 - lg;
}

double fixed_mul(double max_abs, int64_t rows) {
  const int B = fixed_bits(rows);
  if (!(max_abs > 0.0) || !std::isfinite(max_abs)) return std::ldexp(1.0, B);
  int e;
  std::frexp(max_abs, &e);  // max_abs < 2^e
  return std::ldexp(1.0, B - e);
}

// Nodes a tree of `levels` levels can hold: the full binary tree when it is
// small, else room for about 8 * max_leaves (the node table grows if a tree
// needs more).
int32_t initial_node_cap(int32_t levels, int32_t max_leaves) {
  const int64_t full = levels >= 20 ? (int64_t)1 << 21 : ((int64_t)2 << levels) - 1;
  if (full <= 1023) return (int32_t)full;
  return (int32_t)std::min<int64_t>(full, std::max<int64_t>(1023, 8 * (int64_t)max_leaves + 3));
}

// Node-indexed buffers for `cap` nodes of F_sel features.  Contents do not
// survive a reallocation (a tree is rebuilt from its root after one).
int ensure_nodes(bsscl_engine *E, int32_t cap, int32_t F_sel) {
  const int64_t stride = (int64_t)F_sel * kHistPerFeat;
  if (cap <= E->node_alloc && (size_t)cap * stride <= E->pool.cap &&
      (size_t)cap * F_sel <= E->cand.cap) {
    // Exactly the requested capacity: the level lists are sized from it.
    E->node_cap = cap;
    E->node_stride = stride;
    return BSSCL_OK;
  }
  CHK(sync(E));
  const int32_t pcap = cap / 2 + 2;
  CHK(E->pool.ensure((size_t)cap * stride));
  CHK(E->segs.ensure((size_t)cap));
  CHK(E->cand.ensure((size_t)cap * F_sel));
  CHK(E->totals.ensure((size_t)cap * 2));
  const size_t tbytes = 64 + (size_t)cap * sizeof(NodeOut);
  CHK(E->table_d.ensure(tbytes));
  if (E->table_pin_bytes < tbytes) {
    if (E->table_pin) (void)hipHostFree(E->table_pin);
    E->table_pin = nullptr;
    E->table_pin_bytes = 0;
    HIPCHK(hipHostMalloc(reinterpret_cast<void **>(&E->table_pin), tbytes, hipHostMallocDefault));
    E->table_pin_bytes = tbytes;
  }
  E->plan_d = reinterpret_cast<LevelPlan *>(E->table_d.p);
  E->nodes_d = reinterpret_cast<NodeOut *>(E->table_d.p + 64);
  for (int s = 0; s < 2; ++s) CHK(E->parents_d[s].ensure((size_t)pcap));
  CHK(E->groups_d.ensure((size_t)pcap));
  CHK(E->tile_begin_d.ensure((size_t)pcap + 1));
  CHK(E->hist_begin_d.ensure((size_t)pcap + 1));
  CHK(E->hist_node_d.ensure((size_t)pcap));
  CHK(E->nleft_d.ensure((size_t)pcap));
  CHK(E->work_flag_d.ensure((size_t)cap));
  CHK(E->work_e_d.ensure((size_t)cap));
  CHK(E->kept_e_d.ensure((size_t)cap));
  for (int s = 0; s < 2; ++s) CHK(E->parent_e_d[s].ensure((size_t)pcap));
  E->node_alloc = cap;
  E->node_cap = cap;
  E->node_stride = stride;
  return BSSCL_OK;
}

// Feature chunk of a histogram block (hist_fc, or hist_fc_span for an
// in-place level, at most F_sel).
int32_t hist_fchunk(bsscl_engine *E, int32_t F_sel, bool span = false) {
  int32_t fc = span ? E->hist_fc_span : E->hist_fc;
  while (fc > 1 && fc > F_sel) fc >>= 1;
  return fc;
}

// Blocks of a histogram launch for up to max_tasks tasks.
int64_t hist_grid(bsscl_engine *E, int32_t max_tasks, int32_t F_sel, bool span = false) {
  const int32_t fc = hist_fchunk(E, F_sel, span);
  return max_tasks > 0 ? hist_blocks(max_tasks, (F_sel + fc - 1) / fc) : 0;
}

// Histogram row tiles wanted per level: about hist_blocks_per_cu blocks per
// CU over all feature chunks.
int32_t hist_target(bsscl_engine *E, int32_t F_sel, bool span = false) {
  const int32_t fc = hist_fchunk(E, F_sel, span);
  const int32_t nchunks = (F_sel + fc - 1) / fc;
  return std::max<int32_t>(1, (E->hist_blocks_per_cu * E->n_cu + nchunks - 1) / nchunks);
}

// Rows per histogram tile for S rows: enough tiles for about
// hist_blocks_per_cu blocks per CU, but never so many that flushed bins
// (tiles * F_sel * 512 atomics) exceed ~5% of the LDS adds (S * F_sel * 2),
// i.e. at most S/hist_rows_per_flush tiles.
// (plan_tile_rows computes the same on the device for the planned levels,
// with hist_rows_per_flush_level.)
int32_t hist_tile_rows(bsscl_engine *E, int64_t S, int32_t F_sel) {
  int64_t tiles = hist_target(E, F_sel);
  tiles = std::min<int64_t>(tiles, std::max<int64_t>(1, S / E->hist_rows_per_flush));
  int64_t t = round_up((S + tiles - 1) / tiles, 4096);
  return (int32_t)std::min<int64_t>(std::max<int64_t>(t, 4096), 1 << 24);
}

// Packs host arrays into the pinned arena and uploads them with one copy
// into E->lvl_d; returns device pointers through `offs`.
struct Pack {
  std::vector<std::pair<const void *, size_t>> parts;
  size_t add(const void *p, size_t bytes) {
    parts.emplace_back(p, bytes);
    return parts.size() - 1;
  }
};

// Byte offsets of the pack's parts (256-byte aligned); returns the total.
size_t pack_layout(const Pack &pk, std::vector<size_t> &off) {
  size_t total = 0;
  off.resize(pk.parts.size());
  for (size_t i = 0; i < pk.parts.size(); ++i) {
    off[i] = total;
    total = (total + pk.parts[i].second + 255) & ~size_t(255);
  }
  return total;
}

void pack_copy(const Pack &pk, const std::vector<size_t> &off, char *stage) {
  for (size_t i = 0; i < pk.parts.size(); ++i)
    if (pk.parts[i].second) std::memcpy(stage + off[i], pk.parts[i].first, pk.parts[i].second);
}

int upload_pack(bsscl_engine *E, const Pack &pk, std::vector<char *> &dev) {
  std::vector<size_t> off;
  const size_t total = pack_layout(pk, off);
  CHK(E->lvl_d.ensure(std::max<size_t>(total, 256)));
  char *stage = E->pin.take<char>(total);
  if (!stage) {
    // Arena too small: synchronise (nothing may still read it) and grow.
    HIPCHK(hipStreamSynchronize(E->st));
    E->pin.reset();
    CHK(E->pin.reserve(2 * total + (1u << 20)));
    stage = E->pin.take<char>(total);
    if (!stage) return set_error(BSSCL_EINTERNAL, "pinned staging");
  }
  pack_copy(pk, off, stage);
  HIPCHK(hipMemcpyAsync(E->lvl_d.p, stage, total, hipMemcpyHostToDevice, E->st));
  dev.resize(pk.parts.size());
  for (size_t i = 0; i < pk.parts.size(); ++i) dev[i] = E->lvl_d.p + off[i];
  return BSSCL_OK;
}

// Replays est:641-820 on the computed nodes.
int replay(bsscl_engine *E, const std::vector<HNode> &nodes,
           const std::vector<int32_t> &feats, const TreeParams &tp,
           TreeOut &out) {
  const int32_t M = 2 * tp.max_leaves + 2;
  const int32_t MAX_C = tp.max_leaves + 2;
  for (int32_t i = 0; i < M; ++i) {
    out.features[i] = -1;
    out.thresholds[i] = 0;
    out.values[i] = 0.0;
    out.left[i] = -1;
    out.right[i] = -1;
    out.gains[i] = 0.0;
  }
  auto value = [&](const HNode &nd) {
    const double G = (double)nd.Gq * E->g_scale;
    const double H = (double)nd.Hq * E->h_scale;
    return -G / (H + tp.lam);
  };
  int32_t node_count = 0;
  const HNode &root = nodes[0];
  const int32_t root_id = node_count++;
  if (root.fpos < 0) {  // est:575-579 and est:632-637
    out.features[root_id] = -1;
    out.values[root_id] = value(root);
    *out.node_count = node_count;
    return BSSCL_OK;
  }
  std::vector<int32_t> c_node(MAX_C, 0), c_int(MAX_C, -1), c_feat(MAX_C, -1);
  std::vector<double> c_gain(MAX_C, -1.0), c_val(MAX_C, 0.0);
  std::vector<char> c_active(MAX_C, 0);
  c_node[0] = root_id;
  c_int[0] = 0;
  c_gain[0] = root.gain;
  c_feat[0] = root.fpos;
  c_val[0] = value(root);
  c_active[0] = 1;
  int32_t n_splits = 0;
  while (n_splits < tp.max_leaves - 1) {
    int32_t best_ci = -1;
    double best_gain = tp.gamma;
    for (int32_t ci = 0; ci < MAX_C; ++ci)
      if (c_active[ci] && c_feat[ci] >= 0 && c_gain[ci] > best_gain) {
        best_gain = c_gain[ci];
        best_ci = ci;
      }
    if (best_ci < 0) break;
    const int32_t ci = best_ci;
    const HNode &nd = nodes[(size_t)c_int[ci]];
    const int32_t cur = c_node[ci];
    if (!nd.expanded)
      return set_error(BSSCL_EINTERNAL, "tree builder: node popped without expansion");
    if (!nd.split_ok) {  // est:678-683
      out.features[cur] = -1;
      out.values[cur] = c_val[ci];
      c_active[ci] = 0;
      continue;
    }
    const int32_t left_id = node_count++;
    const int32_t right_id = node_count++;
    out.features[cur] = feats[(size_t)nd.fpos];
    out.thresholds[cur] = nd.bin;
    out.left[cur] = left_id;
    out.right[cur] = right_id;
    out.values[cur] = c_val[ci];
    out.gains[cur] = c_gain[ci];
    ++n_splits;
    const bool left_small = nd.nl <= nd.nr;
    const int32_t small_int = left_small ? nd.left : nd.right;
    const int32_t large_int = left_small ? nd.right : nd.left;
    const int32_t small_id = left_small ? left_id : right_id;
    const int32_t large_id = left_small ? right_id : left_id;
    int32_t slot_small = -1, slot_large = -1;
    for (int32_t si = 0; si < MAX_C; ++si)
      if (si != ci && !c_active[si]) {
        if (slot_small < 0) slot_small = si;
        else if (slot_large < 0) {
          slot_large = si;
          break;
        }
      }
    if (slot_small < 0 || slot_large < 0)
      return set_error(BSSCL_EINTERNAL, "tree builder: no free candidate slot");
    c_active[ci] = 0;
    for (int pass = 0; pass < 2; ++pass) {
      const int32_t slot = pass == 0 ? slot_small : slot_large;
      const int32_t ch = pass == 0 ? small_int : large_int;
      const HNode &cn = nodes[(size_t)ch];
      c_node[slot] = pass == 0 ? small_id : large_id;
      c_int[slot] = ch;
      c_feat[slot] = cn.fpos;
      c_gain[slot] = cn.fpos >= 0 ? cn.gain : -1.0;
      c_val[slot] = value(cn);
      c_active[slot] = 1;
    }
  }
  for (int32_t ci = 0; ci < MAX_C; ++ci)
    if (c_active[ci]) {
      out.features[c_node[ci]] = -1;
      out.values[c_node[ci]] = c_val[ci];
    }
  *out.node_count = node_count;
  return BSSCL_OK;
}

void add_part_tiles(const bsscl_engine *E, const PartParent &P, int32_t parent_index,
                    std::vector<PartTile> &tiles) {
  const int64_t a = P.start & ~int64_t(15);
  for (int64_t r = a; r < P.start + P.count; r += E->part_tile)
    tiles.push_back({r, E->part_tile, parent_index});
}

// Histogram launch shape of a tree over m rows of F_sel features.  A block
// reads its rows' 16-byte (g,h) once per feature chunk, so wider
// chunks read them less often but hold more LDS.  Measured on MI355X (whole
// rounds): 1M x 22, two features per block 2080 trees/s against 2009 with
// one and 1939 with four; 5M x 35, four features per block 336 trees/s
// against 324 with two.  The environment overrides the defaults (read per
// tree, for tuning sweeps).
void read_hist_tuning(bsscl_engine *E, int64_t m, int32_t F_sel) {
  auto env_int = [](const char *name, int32_t lo, int32_t hi, int32_t dflt) {
    const char *e = std::getenv(name);
    if (!e) return dflt;
    const long x = std::strtol(e, nullptr, 10);
    return (x >= lo && x <= hi) ? (int32_t)x : dflt;
  };
  const int32_t fc0 = (double)m * F_sel >= 64e6 ? 4 : 2;
  E->hist_fc = env_int("BSSCL_HIST_FC", 1, 8, fc0);
  if (E->hist_fc != 1 && E->hist_fc != 2 && E->hist_fc != 4 && E->hist_fc != 8) E->hist_fc = fc0;
  // Four lane-owned copies of each histogram in LDS (see k_hist): 18.6
  // instead of 21.7 us per launch at 1M x 28, 72 instead of 85 at 10M x 50.
  E->hist_copies = env_int("BSSCL_HIST_COPIES", 1, 8, 4);
  if (E->hist_copies != 1 && E->hist_copies != 4 && E->hist_copies != 8) E->hist_copies = 1;
  if (E->hist_fc * E->hist_copies > 8) E->hist_copies = 8 / E->hist_fc;
  if (E->hist_copies == 2) E->hist_copies = 1;
  E->hist_fc_span = env_int("BSSCL_HIST_SPAN_FC", 1, 8, E->hist_fc);
  if (E->hist_fc_span != 1 && E->hist_fc_span != 2 && E->hist_fc_span != 4 &&
      E->hist_fc_span != 8)
    E->hist_fc_span = E->hist_fc;
  // In place one copy: the listed rows' LDS adds come from scattered lanes,
  // and the smaller block leaves room for more waves (1M x 28: 2330 trees/s
  // against 1780-2180 with four copies; 10M x 50: 364 with four features).
  E->hist_copies_span = env_int("BSSCL_HIST_SPAN_COPIES", 1, 8, 1);
  if (E->hist_copies_span != 1 && E->hist_copies_span != 4 && E->hist_copies_span != 8)
    E->hist_copies_span = 1;
  if (E->hist_fc_span * E->hist_copies_span > 8) E->hist_copies_span = 8 / E->hist_fc_span;
  if (E->hist_copies_span == 2) E->hist_copies_span = 1;
  E->hist_blocks_per_cu = env_int("BSSCL_HIST_BLOCKS_PER_CU", 1, 64, 8);
  // The root: at least 10240 rows per tile (1M x 28, 73 tiles and half the
  // partials of 5120-row tiles: 2440 -> 2480 trees/s; at 10M x 50 the block
  // target decides, 227 tiles either way).
  E->hist_rows_per_flush = env_int("BSSCL_HIST_ROWS_PER_FLUSH", 256, 1 << 22, 10240);
  // Below the root, smaller tiles (more blocks for the smaller levels, more
  // partials to sum): 1M x 28, 2560 rows took the five planned levels'
  // histograms and reductions from 120 to 114 us per round.
  E->hist_rows_per_flush_level =
      env_int("BSSCL_HIST_ROWS_PER_FLUSH_LEVEL", 256, 1 << 22, 2560);
}

// Buffers of a tree over m rows: the compact sets, the node table for the
// tree's levels and the level lists, whose capacities bound what the
// planner may write (PartTile: m/kPartTile + 2 per parent; HistTask: the target
// plus 2 per parent).
int prepare_tree_buffers(bsscl_engine *E, int64_t m, int32_t F_sel, int32_t levels,
                         int32_t max_leaves) {
  read_hist_tuning(E, m, F_sel);
  const int64_t ld_c = round_up(m + 32, 256);
  bool grow = false;
  const int b = E->set_base;
  for (int s = 0; s < 2; ++s)
    grow = grow || E->codes_c[b + s].cap < (size_t)ld_c * F_sel ||
           E->gh_c[b + s].cap < (size_t)ld_c || (b == 0 && E->rid_c[s].cap < (size_t)ld_c);
  const int r = E->root_set;
  if (r >= 0)
    grow = grow || E->codes_c[r].cap < (size_t)ld_c * F_sel || E->gh_c[r].cap < (size_t)ld_c;
  int32_t cap = std::max(initial_node_cap(levels, max_leaves), E->node_cap_floor);
  // Test hook: a small starting node table, to exercise the regrowth path.
  if (const char *t = std::getenv("BSSCL_TEST_NODE_CAP")) {
    const long v = std::strtol(t, nullptr, 10);
    if (v >= 3) cap = std::max<int32_t>((int32_t)std::min<long>(v, cap), E->node_cap_floor);
  }
  // Partition tiles: the most rows per thread that still gives about 512
  // tiles for the root (16-byte loads at 10M rows; 4-byte loads and more
  // blocks at 1M, where 4096-row tiles left CUs idle).
  E->part_rows = 16;
  while (E->part_rows > 4 && m / ((int64_t)kPartThreads * E->part_rows) < 512) E->part_rows >>= 1;
  E->part_tile = kPartThreads * E->part_rows;
  // (A level counts the tiles of every candidate or previous parent: at most
  // m / part_tile plus two partial tiles per candidate.)
  const int64_t tcap = m / E->part_tile + 2 * (int64_t)cap + 4;
  const int64_t hcap =
      (int64_t)std::max(hist_target(E, F_sel), hist_target(E, F_sel, true)) + cap + 4;
  if (tcap > INT32_MAX / 2 || hcap > INT32_MAX / 2)
    return set_error(BSSCL_EINVAL, "tree too large for the level lists");
  grow = grow || E->tiles_d.cap < (size_t)tcap || E->hist_tasks_d.cap < (size_t)hcap ||
         E->part_d.cap < (size_t)hcap * F_sel * kHistPerFeat;
  if (grow) CHK(sync(E));
  E->ld_c = ld_c;
  for (int s = 0; s < 2; ++s) {
    CHK(E->codes_c[b + s].ensure((size_t)ld_c * F_sel));
    CHK(E->gh_c[b + s].ensure((size_t)ld_c));
    if (b == 0) CHK(E->rid_c[s].ensure((size_t)ld_c));
  }
  if (r >= 0) {
    CHK(E->codes_c[r].ensure((size_t)ld_c * F_sel));
    CHK(E->gh_c[r].ensure((size_t)ld_c));
  }
  CHK(E->tiles_d.ensure((size_t)tcap));
  CHK(E->tile_cnt_d.ensure(4 * (size_t)tcap + 8));  // a 16-byte read past the last tile
  CHK(E->level_args_d.ensure(4));
  CHK(E->hist_tasks_d.ensure((size_t)hcap));
  CHK(E->part_d.ensure((size_t)hcap * F_sel * kHistPerFeat));
  E->tile_cap = (int32_t)tcap;
  E->hist_cap = (int32_t)hcap;
  CHK(E->pin.reserve(std::max<size_t>(E->pin.cap, 16u << 20)));
  CHK(ensure_nodes(E, cap, F_sel));
  // One planner for the whole tree (the LDS planner's per-node ranks are
  // written by its own earlier levels).  Test hook: BSSCL_TEST_PLAN_GLOBAL=1
  // keeps the general planner.
  const char *pg = std::getenv("BSSCL_TEST_PLAN_GLOBAL");
  E->plan_lds = E->node_cap <= kPlanLdsMaxNodes && !(pg && pg[0] == '1');
  return BSSCL_OK;
}

SplitParams split_params(bsscl_engine *E, const TreeParams &tp) {
  SplitParams sp;
  sp.min_child_weight = tp.mcw;
  sp.reg_lambda = tp.lam;
  sp.g_scale = E->g_scale;
  sp.h_scale = E->h_scale;
  sp.min_samples_leaf = tp.min_samples_leaf;
  sp.max_depth = tp.max_depth;
  sp.dev = E->round_dev;
  return sp;
}

// The root's inputs as one upload: the selected features, their bin counts
// followed by their most frequent bins, the root's histogram tasks, its
// LevelPlan, its task range and, for a boosting round, the address of the
// round's bagging draws, which the Fisher-Yates kernels read from there
// (parts kPack*, in order).
enum { kPackFeat = 0, kPackNbHot, kPackHist, kPackPlan, kPackTasks, kPackDraws };
struct RootPack {
  std::vector<HistTask> ht;
  std::vector<int32_t> nb_hot;
  LevelPlan rp = {};
  int32_t root_tasks[2] = {0, 0};
  const void *draws = nullptr;
  Pack pk;  // points into the members above: a RootPack is not copied
  RootPack() = default;
  RootPack(const RootPack &) = delete;
  RootPack &operator=(const RootPack &) = delete;
};

void build_root_pack(bsscl_engine *E, int64_t m, const std::vector<int32_t> &feats,
                     const std::vector<int32_t> &nb_sel, RootPack &R) {
  const int32_t F_sel = (int32_t)feats.size();
  const int32_t th = hist_tile_rows(E, m, F_sel);
  R.ht.clear();
  for (int64_t t = 0; t * th < m; ++t) R.ht.push_back({0, (int32_t)t});
  R.rp = LevelPlan{};
  R.rp.n_parents = 1;  // the root's histogram reference, for the reduction
  R.rp.n_hist = (int32_t)R.ht.size();
  R.rp.n_split = 1;
  R.rp.first_child = 0;
  R.rp.tile_rows = th;
  R.rp.n_nodes = 1;
  R.nb_hot.assign(2 * (size_t)F_sel, 0);
  for (int32_t i = 0; i < F_sel; ++i) {
    R.nb_hot[(size_t)i] = nb_sel[(size_t)i];
    const int32_t f = feats[(size_t)i];
    const int32_t hb = (size_t)f < E->hot_bin.size() ? E->hot_bin[(size_t)f] : -1;
    R.nb_hot[(size_t)(F_sel + i)] = hb < 0 ? -1 : std::min(hb, nb_sel[(size_t)i] - 1);
  }
  R.root_tasks[0] = 0;
  R.root_tasks[1] = R.rp.n_hist;
  R.pk = Pack{};
  R.pk.add(feats.data(), feats.size() * 4);
  R.pk.add(R.nb_hot.data(), R.nb_hot.size() * 4);
  R.pk.add(R.ht.data(), R.ht.size() * sizeof(HistTask));
  R.pk.add(&R.rp, sizeof(LevelPlan));
  R.pk.add(R.root_tasks, sizeof(R.root_tasks));
  R.pk.add(&R.draws, sizeof(R.draws));
}

// A root pack already on the device (a boosting round's, uploaded by the
// rows stream; its plan installed by k_gather_gh).
struct PreRoot {
  int32_t n_hist = 0;
  std::vector<char *> dev;
};

// Root: gather the in-bag rows into set 0, its histogram and split search.
// The root's pack goes up in one copy, unless `pre` holds it already.
int launch_root(bsscl_engine *E, const int32_t *rows32, int64_t m,
                const std::vector<int32_t> &feats,
                const std::vector<int32_t> &nb_sel, const TreeParams &tp, bool gathered,
                const PreRoot *pre = nullptr) {
  const int b = E->root_set >= 0 ? E->root_set : E->set_base;
  const Matrix &X = E->mat[0];
  const int32_t F_sel = (int32_t)feats.size();
  std::vector<char *> dv;
  int32_t n_hist = 0;
  if (pre) {
    dv = pre->dev;
    n_hist = pre->n_hist;
  } else {
    RootPack R;
    build_root_pack(E, m, feats, nb_sel, R);
    CHK(upload_pack(E, R.pk, dv));
    HIPCHK(hipMemcpyAsync(E->plan_d, dv[kPackPlan], sizeof(LevelPlan), hipMemcpyDeviceToDevice,
                          E->st));
    n_hist = R.rp.n_hist;
  }
  const int32_t *feat_d = reinterpret_cast<const int32_t *>(dv[kPackFeat]);
  // The root's arena stays untouched until the next tree's upload (a
  // round's: until its slot's next round).
  E->feat_d = feat_d;
  E->nb_sel_d = reinterpret_cast<const int32_t *>(dv[kPackNbHot]);
  E->hot_sel_d = E->nb_sel_d + F_sel;
  // (A boosting round's root rows are already in set b: launch_gather_codes
  // and launch_gather_gh.)
  // (With the root's codes already in place, the gather brings the (g,h)
  // alone: no feature columns.)
  if (!gathered)
    HIPCHK(launch_gather_root(E->st, X.codes.p, X.ld, feat_d, E->root_codes_ready ? 0 : F_sel,
                              rows32, rows32 ? nullptr : E->rows64.p, m, E->ghq.p,
                              E->codes_c[b].p, E->ld_c, E->gh_c[b].p,
                              E->track_rid && b == 0 ? E->rid_c[0].p : nullptr,
                              E->ld_c, E->segs.p, E->hist_node_d.p));
  hipEvent_t stop;
  HIPCHK(launch_hist(E->st, E->codes_c[b].p, E->ld_c, E->gh_c[b].p,
                     reinterpret_cast<const HistTask *>(dv[kPackHist]), E->plan_d, n_hist,
                     E->hist_node_d.p, reinterpret_cast<const int32_t *>(dv[kPackTasks]), E->segs.p,
                     E->nb_sel_d, E->hot_sel_d, F_sel, hist_fchunk(E, F_sel), E->hist_copies,
                     E->part_d.p, E->pool.p, E->node_stride, nullptr,
                     prof_slot(E, hist_grid(E, n_hist, F_sel))));
  CHK(prof_begin(E, 2, &stop));
  HIPCHK(launch_reduce_split(E->st, E->plan_d, 1, nullptr,
                             reinterpret_cast<const int32_t *>(dv[kPackTasks]), E->hist_node_d.p,
                             E->segs.p, E->part_d.p, E->pool.p, E->node_stride, E->nb_sel_d,
                             F_sel, 0, split_params(E, tp), E->cand.p, E->totals.p));
  // The root's table record is written by the level-0 planner.
  CHK(prof_end(E, stop));
  return BSSCL_OK;
}

// Largest number of parents level `level` can have.
int32_t level_parents_bound(bsscl_engine *E, int32_t level) {
  const int64_t full = level >= 30 ? INT32_MAX : (int64_t)1 << level;
  return (int32_t)std::max<int64_t>(1, std::min<int64_t>(full, (E->node_cap - 1) / 2));
}

// How level `level` (parents at that depth) treats its rows: with paired
// levels, in place at even depths and grouped at odd ones, so that rows
// move once every two levels; otherwise every level moves them.
int32_t level_mode(const bsscl_engine *E, int32_t level) {
  if (!E->pair_levels) return kLevelMove;
  return (level & 1) ? kLevelGrouped : kLevelInPlace;
}

// The set holding the rows of level `level`'s parents (their own segments;
// a grouped level's: its grandparents'); a moving level writes the other
// set of the tree's pair.
int level_src(const bsscl_engine *E, int32_t level) {
  const int32_t q = E->pair_levels ? (level >> 1) : level;  // moves made before the level
  if (q == 0 && E->root_set >= 0) return E->root_set;
  return E->set_base + (q & 1);
}

// Whether every split a node can take is kept when popped (est:678-683):
// a split has H >= min_child_weight on each side (est:614-615), so with no
// row's hessian above h_bound each side holds at least mcw / h_bound rows.
// The margin covers the rounding of the hessians (a few ulps of w p (1 - p))
// and of their fixed-point values (below 2^-30 of h_bound).
// (Test hook: BSSCL_TEST_ALL_KEPT=0 plans as if a split could be refused.)
bool splits_always_kept(const bsscl_engine *E, const TreeParams &tp) {
  const char *t = std::getenv("BSSCL_TEST_ALL_KEPT");
  if (t && t[0] == '0') return false;
  if (tp.min_samples_leaf <= 0) return true;
  if (!(tp.mcw > 0.0) || !(E->h_bound > 0.0) || !std::isfinite(E->h_bound)) return false;
  return tp.mcw >= (double)tp.min_samples_leaf * E->h_bound * (1.0 + 1e-9);
}

// Whether level `level`'s partition tiles are counted by its planner
// launch (in-place and grouped levels, with the LDS planner) rather than by
// k_part_count after it.
bool count_fused(const bsscl_engine *E, int32_t level) {
  return E->plan_lds && level_mode(E, level) != kLevelMove;
}

// Most partition tiles level `level` can count over m rows: m / part_tile
// plus two partial tiles per candidate (at most 2^level of them).
int64_t count_tiles_bound(const bsscl_engine *E, int32_t level, int64_t m) {
  const int64_t items = std::min<int64_t>(level >= 30 ? INT32_MAX : (int64_t)1 << level,
                                          (int64_t)E->node_cap);
  return std::min<int64_t>(E->tile_cap, m / E->part_tile + 2 * items + 2);
}

// The planner of level `level`.
int launch_level_plan(bsscl_engine *E, int32_t level, bool last, const TreeParams &tp,
                      int32_t F_sel, int64_t m) {
  PlanArgs pa;
  pa.gamma = tp.gamma;
  pa.level = level;
  pa.max_leaves = tp.max_leaves;
  pa.last = last ? 1 : 0;
  pa.node_cap = E->node_cap;
  pa.tile_cap = E->tile_cap;
  pa.hist_cap = E->hist_cap;
  pa.hist_target = hist_target(E, F_sel, level_mode(E, level) == kLevelInPlace);
  pa.rows_per_flush = E->hist_rows_per_flush_level;
  pa.part_tile = E->part_tile;
  pa.mode = level_mode(E, level);
  pa.all_kept = splits_always_kept(E, tp) ? 1 : 0;
  pa.part_rows = E->part_rows;
  pa.fused_count = count_fused(E, level) ? 1 : 0;
  hipEvent_t stop;
  CHK(prof_begin(E, 2, &stop));
  if (E->plan_lds) {
    // The counting blocks read the level's rows where its parents hold them.
    const int src = level_src(E, level);
    const int64_t tiles = count_tiles_bound(E, level, m);
    const int32_t cblocks =
        (int32_t)std::max<int64_t>(1, (tiles + kCountTilesPerBlock - 1) / kCountTilesPerBlock);
    HIPCHK(launch_plan_lds(E->st, E->nodes_d, E->plan_d, E->parents_d[(level + 1) & 1].p,
                           E->parents_d[level & 1].p, E->groups_d.p, E->tile_begin_d.p,
                           E->hist_begin_d.p, E->tiles_d.p, E->hist_tasks_d.p, E->segs.p,
                           E->totals.p, E->cand.p, E->kept_e_d.p,
                           E->parent_e_d[(level + 1) & 1].p, E->parent_e_d[level & 1].p,
                           F_sel, pa, E->codes_c[src].p, E->ld_c, E->tile_cnt_d.p,
                           E->level_args_d.p + 2 * (level & 1),
                           E->level_args_d.p + 2 * ((level + 1) & 1), cblocks));
  }
  else if (pa.mode == kLevelMove)
    HIPCHK(launch_plan(E->st, E->nodes_d, E->plan_d, E->parents_d[(level + 1) & 1].p,
                       E->parents_d[level & 1].p, E->tile_begin_d.p, E->hist_begin_d.p,
                       E->tiles_d.p, E->hist_tasks_d.p,
                       E->work_flag_d.p, E->work_e_d.p, E->segs.p, E->totals.p, E->cand.p,
                       F_sel, pa));
  else
    return set_error(BSSCL_EINTERNAL, "paired levels need the LDS planner");
  CHK(prof_end(E, stop));
  return BSSCL_OK;
}

// Count of one level's groups (groups == nullptr: one per parent), then
// the scatter of their rows from set src to their children's segments in
// set dst (move_rows).  (A level that moves nothing takes the children's
// sizes from the counts in its next kernel: the in-place histogram, or
// k_last_level.)
int launch_partition(bsscl_engine *E, int src, int dst, const PartParent *parents,
                     const PartGroup *groups, const int32_t *tile_begin, const PartTile *tiles,
                     const LevelPlan *plan, int32_t max_tiles, int32_t F_sel,
                     int32_t min_samples_leaf, bool move_rows, bool counted = false) {
  if (counted && !move_rows) return BSSCL_OK;
  hipEvent_t stop;
  CHK(prof_begin(E, 1, &stop));
  if (!counted)  // (counted: the planner launch has counted the tiles)
    HIPCHK(launch_part_count(E->st, E->codes_c[src].p, E->ld_c, parents, groups, tiles, plan,
                             max_tiles, E->part_rows, E->tile_cnt_d.p));
  if (move_rows)  // the scatter does each group's scan itself
    HIPCHK(launch_part_scatter(E->st, E->codes_c[src].p, E->codes_c[dst].p, E->ld_c,
                               E->gh_c[src].p, E->gh_c[dst].p,
                               E->track_rid ? E->rid_c[src & 1].p : nullptr,
                               E->track_rid ? E->rid_c[dst & 1].p : nullptr, parents, groups,
                               tiles, plan, max_tiles, E->part_rows, tile_begin,
                               E->tile_cnt_d.p, E->nleft_d.p, E->segs.p, E->hist_node_d.p,
                               min_samples_leaf, F_sel));
  CHK(prof_end(E, stop));
  return BSSCL_OK;
}

// The kernels of level `level` after its planner.  Grids are upper bounds
// from the level's depth; the kernels read the planned counts.  Children at
// max_depth can never be split (est:775-777): they need their sizes and
// totals only, so their rows are not moved and their histograms not built.
int launch_level(bsscl_engine *E, int32_t level, bool last, int64_t m,
                 const TreeParams &tp, int32_t F_sel) {
  const int32_t mode = level_mode(E, level);
  const int src = level_src(E, level);
  const int dst = level_src(E, level + 1);  // where a moving level writes its rows
  const PartParent *par = E->parents_d[level & 1].p;
  const PartGroup *grp = mode == kLevelGrouped ? E->groups_d.p : nullptr;
  const bool in_place = mode == kLevelInPlace;
  const int32_t P = level_parents_bound(E, level);
  const int32_t T = (int32_t)std::min<int64_t>(E->tile_cap, m / E->part_tile + 2 * (int64_t)P + 1);
  CHK(launch_partition(E, src, dst, par, grp, E->tile_begin_d.p, E->tiles_d.p, E->plan_d, T,
                       F_sel, tp.min_samples_leaf, !last && !in_place, count_fused(E, level)));
  hipEvent_t stop;
  if (last) {
    CHK(prof_begin(E, 2, &stop));
    HIPCHK(launch_last_level(E->st, par, grp ? 1 : 0, E->plan_d, std::min(P, 4096),
                             E->tile_begin_d.p, E->tile_cnt_d.p, E->nleft_d.p, E->segs.p,
                             E->hist_node_d.p, tp.min_samples_leaf, E->pool.p, E->node_stride,
                             E->totals.p, E->nodes_d));
    CHK(prof_end(E, stop));
    return BSSCL_OK;
  }
  const int32_t H = (int32_t)std::min<int64_t>(
      E->hist_cap, (int64_t)hist_target(E, F_sel, in_place) + 2 * (int64_t)P + 2);
  // In place, the smaller children's rows are read from their parents'
  // segments in src, and the histogram launch takes the children's sizes.
  const int hs = in_place ? src : dst;
  const SpanLevel span{par, E->tile_cnt_d.p, E->nleft_d.p, tp.min_samples_leaf};
  HIPCHK(launch_hist(E->st, E->codes_c[hs].p, E->ld_c, E->gh_c[hs].p, E->hist_tasks_d.p,
                     E->plan_d, H, E->hist_node_d.p, E->hist_begin_d.p, E->segs.p,
                     E->nb_sel_d, E->hot_sel_d, F_sel, hist_fchunk(E, F_sel, in_place),
                     in_place ? E->hist_copies_span : E->hist_copies, E->part_d.p, E->pool.p,
                     E->node_stride, in_place ? &span : nullptr,
                     prof_slot(E, hist_grid(E, H, F_sel, in_place))));
  CHK(prof_begin(E, 2, &stop));
  HIPCHK(launch_reduce_split(E->st, E->plan_d, P, par, E->hist_begin_d.p, E->hist_node_d.p,
                             E->segs.p, E->part_d.p, E->pool.p, E->node_stride, E->nb_sel_d,
                             F_sel, level + 1, split_params(E, tp), E->cand.p, E->totals.p,
                             in_place ? 1 : 0));
  // The new nodes' table records are written by the next level's planner.
  CHK(prof_end(E, stop));
  return BSSCL_OK;
}

// Copies the plan and the first `n` nodes of the node table to the host.
int read_table(bsscl_engine *E, int32_t n, LevelPlan &plan) {
  const size_t bytes = 64 + (size_t)std::max(0, std::min(n, E->node_cap)) * sizeof(NodeOut);
  HIPCHK(hipMemcpyAsync(E->table_pin, E->table_d.p, bytes, hipMemcpyDeviceToHost, E->st));
  CHK(sync(E));
  std::memcpy(&plan, E->table_pin, sizeof(LevelPlan));
  return BSSCL_OK;
}

// One boosting round's readback: RoundHeader, then the tree arrays of M
// entries (features i32, thresholds i64, values f64, left i32, right i32,
// gains f64), each 8-byte aligned.
size_t round_out_bytes(int32_t M) {
  const size_t a4 = ((size_t)M * 4 + 7) & ~size_t(7);
  return sizeof(RoundHeader) + 3 * a4 + 3 * (size_t)M * 8;
}

TreeArrays round_arrays(char *base, int32_t M) {
  const size_t a4 = ((size_t)M * 4 + 7) & ~size_t(7);
  char *p = base + sizeof(RoundHeader);
  TreeArrays t;
  t.features = reinterpret_cast<int32_t *>(p);
  p += a4;
  t.thresholds = reinterpret_cast<int64_t *>(p);
  p += (size_t)M * 8;
  t.values = reinterpret_cast<double *>(p);
  p += (size_t)M * 8;
  t.left = reinterpret_cast<int32_t *>(p);
  p += a4;
  t.right = reinterpret_cast<int32_t *>(p);
  p += a4;
  t.gains = reinterpret_cast<double *>(p);
  return t;
}

int ensure_host_pinned(bsscl_engine *E, char *&p, size_t &have, size_t bytes) {
  if (have >= bytes) return BSSCL_OK;
  CHK(sync(E));
  if (p) (void)hipHostFree(p);
  p = nullptr;
  have = 0;
  HIPCHK(hipHostMalloc(reinterpret_cast<void **>(&p), bytes, hipHostMallocDefault));
  have = bytes;
  return BSSCL_OK;
}

// Readback buffers of round buffer b: the round's header and tree, and the
// node table (for profiling counters).
// The sum k_sum_partials forms, in its order: 256 strided sums, each wave's
// xor butterfly, then the four waves' sums pairwise (so a round summed here
// gives the bits of one summed on the device).
double sum_partials_host(const double *p, int32_t count) {
  double lane[256];
  for (int t = 0; t < 256; ++t) {
    double acc = 0.0;
    for (int32_t i = t; i < count; i += 256) acc += p[i];
    lane[t] = acc;
  }
  double red[4];
  for (int w = 0; w < 4; ++w) {
    double a[64], b[64];
    for (int l = 0; l < 64; ++l) a[l] = lane[64 * w + l];
    for (int o = 32; o >= 1; o >>= 1) {
      for (int l = 0; l < 64; ++l) b[l] = a[l] + a[l ^ o];
      std::memcpy(a, b, sizeof(a));
    }
    red[w] = a[0];
  }
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// A round's readback: the round_out_bytes(M) of the tree, then the F
// update's per-block losses (`partials` doubles).
int ensure_round_out(bsscl_engine *E, int b, int32_t M, int32_t partials) {
  const size_t bytes = round_out_bytes(M) + (size_t)partials * 8;
  if (E->round_d[b].cap < bytes) CHK(sync(E));
  CHK(E->round_d[b].ensure(bytes));
  CHK(ensure_host_pinned(E, E->round_pin[b], E->round_pin_bytes[b], bytes));
  CHK(ensure_host_pinned(E, E->rtable_pin[b], E->rtable_pin_bytes[b],
                         64 + (size_t)E->node_alloc * sizeof(NodeOut)));
  return BSSCL_OK;
}

// Device Fisher-Yates work arrays for n items.
// Shuffles of at least this many positions build their step lists by
// sorting (position, step) keys; shorter ones use per-position linked
// lists.  (Test hook: BSSCL_FY_SORTED=1 or 0 forces one form.)
constexpr int64_t kFySortedMin = 1 << 18;

int ensure_fy_work(bsscl_engine *E, int64_t n, FyWork &w) {
  for (DevBuf<int32_t> *x : {&E->fy_head, &E->fy_next, &E->fy_v}) CHK(x->ensure((size_t)n));
  w.head = E->fy_head.p;
  w.next = E->fy_next.p;
  w.v = E->fy_v.p;
  const char *force = std::getenv("BSSCL_FY_SORTED");
  const bool sorted = force && (force[0] == '0' || force[0] == '1') ? force[0] == '1'
                                                                    : n >= kFySortedMin;
  w.keys = w.keys_tmp = nullptr;
  w.counts = w.totals = nullptr;
  if (sorted && n > 1) {
    const size_t ld = (size_t)sort_u64_ld(n);
    for (auto &k : E->fy_keys) CHK(k.ensure(ld));
    CHK(E->fy_counts.ensure((size_t)sort_u64_count_words(n)));
    CHK(E->fy_totals.ensure(256));
    w.keys = E->fy_keys[0].p;
    w.keys_tmp = E->fy_keys[1].p;
    w.counts = E->fy_counts.p;
    w.totals = E->fy_totals.p;
  }
  return BSSCL_OK;
}

constexpr int32_t kLevelsPerCheck = 8;  // levels enqueued between host checks

// Whether a tree moves its rows every second level (with the LDS planner).
// (Test hook: BSSCL_TEST_PAIR_LEVELS=0 moves the rows at every level.)
bool want_pair_levels(const bsscl_engine *E) {
  const char *pl = std::getenv("BSSCL_TEST_PAIR_LEVELS");
  return E->plan_lds && !(pl && pl[0] == '0');
}

// Enqueues the root and every level of one tree (after
// prepare_tree_buffers).  All levels are enqueued without host round trips:
// the planner kernel chooses each level's parents on the device; every
// kLevelsPerCheck levels the host reads the plan and stops enqueueing once
// the tree has ended (unless `checks` is false: then every level is
// enqueued).  *run = levels enqueued.
int launch_tree(bsscl_engine *E, const int32_t *rows32, int64_t m,
                const std::vector<int32_t> &feats,
                const std::vector<int32_t> &nb_sel, const TreeParams &tp, int32_t *run,
                bool checks = true, bool gathered = false, const PreRoot *pre = nullptr) {
  const int32_t F_sel = (int32_t)feats.size();
  const int32_t levels = std::max(1, tp.max_depth);
  E->pair_levels = want_pair_levels(E);
  CHK(launch_root(E, rows32, m, feats, nb_sel, tp, gathered, pre));
  *run = 0;
  for (int32_t d = 0; d < levels; ++d) {
    const bool last = d + 1 >= tp.max_depth;
    CHK(launch_level_plan(E, d, last, tp, F_sel, m));
    if (checks && d > 0 && d % kLevelsPerCheck == 0) {
      LevelPlan plan;
      CHK(read_table(E, 0, plan));
      if (plan.n_parents == 0 || plan.overflow != 0) break;
    }
    CHK(launch_level(E, d, last, m, tp, F_sel));
    *run = d + 1;
  }
  return BSSCL_OK;
}

// Nodes a tree of `run` enqueued levels can have (bounds the readback).
int32_t table_bound(bsscl_engine *E, int32_t run) {
  const int64_t most = run >= 30 ? INT32_MAX : ((int64_t)2 << run) - 1;
  return (int32_t)std::min<int64_t>(most, E->node_cap);
}

// Arguments of the device replay of the tree just enqueued, with the
// engine's current scales.
ReplayArgs replay_args(bsscl_engine *E, const TreeParams &tp, int32_t M) {
  ReplayArgs ra;
  ra.gamma = tp.gamma;
  ra.reg_lambda = tp.lam;
  ra.g_scale = E->g_scale;
  ra.h_scale = E->h_scale;
  ra.dev = DevScale{nullptr, 0, 0};
  ra.max_leaves = tp.max_leaves;
  ra.out_len = M;
  // (Test hook BSSCL_TEST_REPLAY_GLOBAL: 1 reads the node table from HBM,
  // 2 keeps the candidate slots in LDS instead of registers.)
  const char *rg = std::getenv("BSSCL_TEST_REPLAY_GLOBAL");
  ra.stage_limit = !rg ? (1 << 30) : rg[0] == '1' ? 0 : rg[0] == '2' ? 1023 : (1 << 30);
  ra.node_cap = E->node_cap;
  ra.max_depth = tp.max_depth;
  ra.pad = 0;
  return ra;
}

// Whether trees of `max_leaves` go through the device replay (the
// candidate slots hold max_leaves + 2 entries).  Test hook:
// BSSCL_TEST_HOST_REPLAY=1 forces the host path.
bool device_replay_fits(int32_t max_leaves) {
  const char *force_host = std::getenv("BSSCL_TEST_HOST_REPLAY");
  return max_leaves + 2 <= kReplaySlots && !(force_host && force_host[0] == '1');
}

// Profiling counters of one built tree from its node table: histogram
// rows x features and algorithmic bytes (the root and the smaller child of
// every kept split above the last level), nodes expanded, trees.
// `small_rows` sums the smaller child's rows over those splits, `expanded`
// counts the nodes with children.
void tree_stats_add(bsscl_engine *E, int64_t m, int32_t F_sel, int64_t small_rows,
                    int32_t expanded) {
  E->stats[2] += (double)(m + small_rows) * F_sel;
  E->stats[3] += (double)(m + small_rows) * (F_sel + 8);
  E->stats[9] += (double)expanded;
  E->stats[8] += 1.0;
}

void tree_stats(bsscl_engine *E, const NodeOut *t, int32_t n, int64_t m, int32_t F_sel,
                const TreeParams &tp) {
  std::vector<int32_t> depth((size_t)n, 0);
  int64_t small_rows = 0;
  int32_t expanded = 0;
  for (int32_t i = 0; i < n; ++i) {
    const int32_t l = t[i].left;
    if (l < 0 || l + 1 >= n) continue;
    depth[(size_t)l] = depth[(size_t)l + 1] = depth[(size_t)i] + 1;
    ++expanded;
    if (t[l].valid && depth[(size_t)i] + 1 < tp.max_depth)
      small_rows += std::min(t[l].count, t[l + 1].count);
  }
  tree_stats_add(E, m, F_sel, small_rows, expanded);
}

// Builds one tree from the rows already in rows32 (device, int32) or, when
// rows32 is null, E->rows64,
// with quantized gradients in E->ghq, and replays the reference's candidate
// loop on the host.  The node table comes back once (twice when it had to
// grow).
int build_tree_core(bsscl_engine *E, const int32_t *rows32, int64_t m,
                    const std::vector<int32_t> &feats,
                    const std::vector<int32_t> &nb_sel, const TreeParams &tp,
                    TreeOut &out, HNode *root_out = nullptr) {
  const int32_t F_sel = (int32_t)feats.size();
  const int32_t levels = std::max(1, tp.max_depth);
  LevelPlan plan = {};
  for (;;) {
    CHK(prepare_tree_buffers(E, m, F_sel, levels, tp.max_leaves));
    int32_t run = 0;
    CHK(launch_tree(E, rows32, m, feats, nb_sel, tp, &run));
    CHK(read_table(E, table_bound(E, run), plan));
    if (plan.overflow < 0) return set_error(BSSCL_EINTERNAL, "tree builder: level list overflow");
    if (plan.overflow == 0) break;
    // The node table was too small: grow it and build the tree again.
    E->node_cap_floor = std::max(plan.overflow, 2 * E->node_cap);
  }
  const int32_t n = plan.n_nodes;
  if (n < 1 || n > E->node_cap) return set_error(BSSCL_EINTERNAL, "tree builder: bad node count");
  const NodeOut *t = reinterpret_cast<const NodeOut *>(E->table_pin + 64);
  std::vector<HNode> nodes((size_t)n);
  for (int32_t i = 0; i < n; ++i) {
    HNode &nd = nodes[(size_t)i];
    const NodeOut &o = t[i];
    nd.start = o.start;
    nd.count = o.count;
    nd.valid = o.valid != 0;
    nd.Gq = o.Gq;
    nd.Hq = o.Hq;
    nd.fpos = o.fpos;
    nd.bin = o.bin;
    nd.gain = o.gain;
    nd.e = o.e;
    if (o.left >= 0) {
      if (o.left <= i || o.left + 1 >= n)
        return set_error(BSSCL_EINTERNAL, "tree builder: bad child link");
      nd.expanded = true;
      nd.left = o.left;
      nd.right = o.left + 1;
      nd.nl = t[o.left].count;
      nd.nr = t[o.left + 1].count;
      nd.split_ok = t[o.left].valid != 0;
      nodes[(size_t)o.left].parent = nodes[(size_t)o.left + 1].parent = i;
    }
  }
  if (root_out) *root_out = nodes[0];
  if (E->prof) tree_stats(E, t, n, m, F_sel, tp);
  return replay(E, nodes, feats, tp, out);
}

int validate_tree_args(bsscl_engine *E, const int32_t *feature_indices,
                       int32_t n_selected, int32_t max_leaves,
                       int32_t min_samples_leaf, const int32_t *bin_counts,
                       const TreeOut &out, std::vector<int32_t> &feats,
                       std::vector<int32_t> &nb_sel) {
  const Matrix &X = E->mat[0];
  if (!feature_indices || n_selected <= 0 || !bin_counts)
    return set_error(BSSCL_EINVAL, "feature_indices/bin_counts missing");
  if (max_leaves < 1) return set_error(BSSCL_EINVAL, "max_leaves must be >= 1");
  if (!out.features || !out.thresholds || !out.values || !out.left ||
      !out.right || !out.node_count || !out.gains)
    return set_error(BSSCL_EINVAL, "output arrays missing");
  (void)min_samples_leaf;
  feats.assign(feature_indices, feature_indices + n_selected);
  nb_sel.resize((size_t)n_selected);
  for (int32_t i = 0; i < n_selected; ++i) {
    const int32_t f = feats[(size_t)i];
    if (f < 0 || f >= X.F) return set_error(BSSCL_EINVAL, "feature index out of range");
    if (i > 0 && f <= feats[(size_t)i - 1])
      return set_error(BSSCL_EINVAL, "feature_indices must be strictly ascending");
    const int32_t nb = bin_counts[f];
    if (nb < 1 || nb > kMaxBinCount)
      return set_error(BSSCL_EINVAL, "bin_counts must be in [1, 65536]");
    nb_sel[(size_t)i] = nb;
    CHK(ensure_tiers(E, 0, tiers_for_bins(nb)));
  }
  std::vector<int32_t> cols, nb_cols;
  CHK(expand_features(X, feats, nb_sel, cols, nb_cols));
  feats.swap(cols);
  nb_sel.swap(nb_cols);
  return BSSCL_OK;
}

// Tree arrays from engine columns to the reference's features: a split on
// tier t, (t F + j, b), is the split (j, 255 t + b).
void tree_to_reference(const Matrix &X, const TreeOut &out) {
  const int32_t n = *out.node_count;
  for (int32_t i = 0; i < n; ++i) {
    if (out.features[i] >= X.F) {
      const int32_t t = out.features[i] / X.F;
      out.features[i] -= t * X.F;
      out.thresholds[i] += 255 * (int64_t)t;
    }
  }
}

// A reference split (j, c) as the engine traverses it on matrix X: tier
// t = c / 255 at b = c - 255 t (a threshold above the last tier's range
// sends every row left, as b = 255 does).
inline void split_to_engine(const Matrix &X, int32_t &feature, int64_t &threshold) {
  if (X.tiers > 1 && feature >= 0 && threshold >= 255) {
    const int32_t t = (int32_t)std::min<int64_t>(threshold / 255, X.tiers - 1);
    feature += t * X.F;
    threshold = std::min<int64_t>(threshold - 255 * (int64_t)t, 255);
  }
}

// Uploads host gradients/hessians and quantizes them with scales from their
// largest magnitudes.
int load_grad_hess(bsscl_engine *E, const double *grad, const double *hess,
                   int64_t n, int64_t rows_summed) {
  double gmax = 0.0, hmax = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    const double a = std::fabs(grad[i]), b = std::fabs(hess[i]);
    if (!std::isfinite(a) || !std::isfinite(b))
      return set_error(BSSCL_EINVAL, "grad/hess must be finite");
    gmax = std::max(gmax, a);
    hmax = std::max(hmax, b);
  }
  const double gm = fixed_mul(gmax, rows_summed), hm = fixed_mul(hmax, rows_summed);
  E->g_scale = 1.0 / gm;
  E->h_scale = 1.0 / hm;
  E->h_bound = hmax;
  CHK(E->g64.ensure((size_t)n));
  CHK(E->h64.ensure((size_t)n));
  CHK(E->ghq.ensure((size_t)n));
  HIPCHK(hipMemcpyAsync(E->g64.p, grad, (size_t)n * 8, hipMemcpyHostToDevice, E->st));
  HIPCHK(hipMemcpyAsync(E->h64.p, hess, (size_t)n * 8, hipMemcpyHostToDevice, E->st));
  HIPCHK(launch_quantize(E->st, E->g64.p, E->h64.p, n, gm, hm, E->ghq.p));
  return BSSCL_OK;
}

// Most frequent code of each feature of matrix 0: the histogram kernel sums
// that bin in registers instead of LDS atomics.
int find_hot_bins(bsscl_engine *E) {
  const Matrix &M = E->mat[0];
  const int32_t C = M.cols();
  TempBuf<unsigned int> cnt;
  CHK(cnt.ensure((size_t)C * 256));
  std::vector<unsigned int> h((size_t)C * 256);
  hipError_t e = hipMemsetAsync(cnt.p, 0, (size_t)C * 256 * 4, E->st);
  if (e == hipSuccess) e = launch_code_counts(E->st, M.codes.p, M.ld, M.n, C, cnt.p);
  if (e == hipSuccess) e = hipMemcpyAsync(h.data(), cnt.p, h.size() * 4, hipMemcpyDeviceToHost, E->st);
  if (e == hipSuccess) e = hipStreamSynchronize(E->st);
  cnt.release();
  if (e != hipSuccess) return set_error(BSSCL_EDEVICE, std::string("code counts: ") + hipGetErrorString(e));
  // Only a bin holding at least 10% of the rows is worth the divergent
  // register path; -1 (no bin) otherwise.
  E->hot_bin.assign((size_t)C, -1);
  for (int32_t f = 0; f < C; ++f) {
    const unsigned int *c = h.data() + (size_t)f * 256;
    const int32_t b = (int32_t)(std::max_element(c, c + 256) - c);
    if ((double)c[b] >= 0.10 * (double)M.n) E->hot_bin[(size_t)f] = b;
  }
  return BSSCL_OK;
}

int upload_tree(bsscl_engine *E, const int32_t *features,
                const int64_t *thresholds, const double *values,
                const int32_t *left, const int32_t *right, int32_t node_count,
                int32_t F) {
  if (node_count <= 0) return set_error(BSSCL_EINVAL, "empty tree");
  std::vector<TreeNodeDev> t((size_t)node_count);
  for (int32_t i = 0; i < node_count; ++i) {
    TreeNodeDev &d = t[(size_t)i];
    d.feature = features[i];
    d.value = values[i];
    if (d.feature >= 0) {
      if (d.feature >= F || left[i] <= i || right[i] <= i || left[i] >= node_count ||
          right[i] >= node_count)
        return set_error(BSSCL_EINVAL, "malformed tree node " + std::to_string(i));
      d.threshold = (int32_t)std::max<int64_t>(-1, std::min<int64_t>(thresholds[i], 1 << 20));
      d.left = left[i];
      d.right = right[i];
    } else {
      d.feature = -1;
      d.threshold = 0;
      d.left = d.right = 0;
    }
  }
  CHK(E->pin.reserve(std::max<size_t>(E->pin.cap, 8u << 20)));
  CHK(upload(E, E->tree_d, t.data(), t.size()));
  return BSSCL_OK;
}

}  // namespace
}  // namespace bsscl

namespace bsscl {
namespace {

// Speculative rounds need a device path that cannot fall back: the node
// table holds the full tree (max_depth <= 9) and the replay's slots hold
// every candidate.
bool pipeline_safe(bsscl_engine *E, const RoundArgs &a, bsscl_sampler *sampler) {
  (void)E;
  (void)sampler;
  if (a.max_depth > 9 || a.max_leaves + 2 > kReplaySlots) return false;
  for (const char *k : {"BSSCL_TEST_HOST_REPLAY", "BSSCL_TEST_NODE_CAP", "BSSCL_TEST_REPLAY_GLOBAL"})
    if (std::getenv(k)) return false;
  return true;
}

// Waits for the round in slot s and returns its sampler buffers; its
// results are dropped.
int drain_rounds(bsscl_engine *E, int s) {
  RoundSlot &r = E->rslot[s];
  if (!r.active) return BSSCL_OK;
  hipError_t e = hipStreamSynchronize(E->st_rows);
  const hipError_t e2 = hipStreamSynchronize(E->st);
  if (e == hipSuccess) e = e2;
  sampler_give_back(r.sampler, r.token);
  r.active = false;
  r.token = nullptr;
  (void)prof_collect(E);
  if (e != hipSuccess) return set_error(BSSCL_EDEVICE, std::string("boost_round: ") + hipGetErrorString(e));
  return BSSCL_OK;
}

void release_graph(RoundGraph &g) {
  if (g.exec) (void)hipGraphExecDestroy(g.exec);
  g = RoundGraph{};
}

template <typename T>
void key_add(std::vector<uint64_t> &k, T v) {
  static_assert(sizeof(T) <= 8, "scalar");
  uint64_t u = 0;
  std::memcpy(&u, &v, sizeof(T));
  k.push_back(u);
}

// Which of a round's launch sequences run as captured graphs: the rows
// stream's by default; BSSCL_GRAPHS=1 adds the tree stream's, =0 turns both
// off.  On one MI355X at 1M x 28 rows graphs left the GPU time per round as
// it was and took 0.05-0.09 ms of host time off each round's enqueue; tree
// graphs took another 0.07-0.1 ms off but made the GPU round about 2%
// longer (the same kernels, dispatched from a graph), so they are for hosts
// whose enqueue paces the rounds.
bool graphs_wanted(bool tree) {
  const char *v = std::getenv("BSSCL_GRAPHS");
  if (v && v[0] == '0') return false;
  return !tree || (v && v[0] == '1');
}

// Enqueues `launches` (a function returning an engine status) on stream st:
// through g's graph when its key is `key`, else captured into a new graph
// for `key` and launched, or run directly while the engine has not yet run
// a round, or graphs are off.  A capture that fails turns graphs off and
// runs the launches directly.  Sets *replayed when the launches ran as a
// graph.
template <typename F>
int run_graph(bsscl_engine *E, RoundGraph &g, const std::vector<uint64_t> &key, hipStream_t st,
              bool tree, F &&launches, bool *replayed) {
  *replayed = false;
  if (!E->graphs || !E->launched_round || !graphs_wanted(tree)) return launches();
  if (g.exec && g.key == key) {
    HIPCHK(hipGraphLaunch(g.exec, st));
    *replayed = true;
    return BSSCL_OK;
  }
  // (The slot's previous round has finished: its graph is idle.)
  release_graph(g);
  hipGraph_t graph = nullptr;
  hipError_t e = hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal);
  int rc = BSSCL_OK;
  if (e == hipSuccess) {
    rc = launches();
    const hipError_t e2 = hipStreamEndCapture(st, &graph);
    if (e2 != hipSuccess) e = e2;
  }
  if (rc == BSSCL_OK && e == hipSuccess && graph)
    e = hipGraphInstantiate(&g.exec, graph, nullptr, nullptr, 0);
  if (graph) (void)hipGraphDestroy(graph);
  if (rc != BSSCL_OK || e != hipSuccess || !g.exec) {
    (void)hipGetLastError();
    release_graph(g);
    E->graphs = false;
    return launches();  // captured, not run: run them now
  }
  g.key = key;
  E->stats[20] += 1.0;
  HIPCHK(hipGraphLaunch(g.exec, st));
  *replayed = true;
  return BSSCL_OK;
}

// The fixed-point multipliers of a boosting tree over m rows on the
// host-driven path, from the largest |g| and h of the current F as the
// device holds them (read back; the host-driven path waits for the stream
// anyway), so the path quantises as the device path does; from the bound
// max(w0, w1) when the device holds none or BSSCL_TEST_BOUND_SCALE=1.  Sets
// the engine's scales to match.
int host_round_scales(bsscl_engine *E, int64_t m, double &gm, double &hm) {
  const double wmax = std::max(E->w0, E->w1);
  double gmax = wmax, hmax = 0.25 * wmax;
  const char *bound_env = std::getenv("BSSCL_TEST_BOUND_SCALE");
  if (E->gh_ok && !(bound_env && bound_env[0] == '1')) {
    unsigned long long bits[2];
    HIPCHK(hipMemcpyAsync(bits, E->ghmax_d.p + 2 * E->gh_slot, sizeof(bits),
                          hipMemcpyDeviceToHost, E->st));
    HIPCHK(hipStreamSynchronize(E->st));
    std::memcpy(&gmax, &bits[0], 8);
    std::memcpy(&hmax, &bits[1], 8);
  }
  gm = fixed_mul(gmax, m);
  hm = fixed_mul(hmax, m);
  E->g_scale = 1.0 / gm;
  E->h_scale = 1.0 / hm;
  return BSSCL_OK;
}

// Enqueues one boosting round: gradients from the current F (est:2868),
// the sampler's round (est:2886, est:2502-2517), the tree, its replay
// (est:641-820), F += lr * tree(X) and the training log-loss, and the
// readback of the tree and the loss into round buffer s.  A tree that needs
// the host-driven path (a larger node table, more candidate slots than the
// device replay holds) is finished by finish_round.
int enqueue_round(bsscl_engine *E, bsscl_sampler *sampler, const RoundArgs &a, int s) {
  const Matrix &X = E->mat[0];
  RoundSlot &R = E->rslot[s];
  const SamplerShape sh = sampler_shape(sampler);
  const int64_t m = sh.n_sub;
  if (sh.n != X.n) return set_error(BSSCL_EINVAL, "boost_round: sampler rows differ from matrix rows");
  ++E->round_seq;
  // Gradients from the current F: |g| <= max(w0, w1), h <= max(w0, w1)/4.
  // (The device path scales from the maxima themselves, see dev_scale; the
  // host-driven path reads them back, host_round_scales.)
  const double wmax = std::max(E->w0, E->w1);
  double gm = fixed_mul(wmax, m), hm = fixed_mul(0.25 * wmax, m);
  E->g_scale = 1.0 / gm;
  E->h_scale = 1.0 / hm;
  E->h_bound = 0.25 * wmax;
  SamplerRound sr;
  void *token = nullptr;
  const auto t_wait0 = std::chrono::steady_clock::now();
  CHK(sampler_take(sampler, &sr, &token));
  E->stats[10] += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t_wait0).count();
  R.active = true;
  R.sampler = sampler;
  R.token = token;
  R.args = a;
  R.m = m;
  R.buf = s;
  R.seq = E->round_seq;
  R.M = 2 * a.max_leaves + 2;
  R.run = 0;
  auto fail = [&](int rc) {
    (void)hipStreamSynchronize(E->st_rows);
    (void)hipStreamSynchronize(E->st);
    E->gh_ok = false;  // the device maxima may be out of step with gh_slot
    E->round_dev = DevScale{nullptr, 0, 0};
    sampler_give_back(sampler, token);
    R.active = false;
    R.token = nullptr;
    return rc;
  };
  TreeOut none{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
  (void)none;
  int rc = BSSCL_OK;
  {
    // Feature subset and bin counts (validate_tree_args without outputs).
    const int32_t f_sub = sh.f_sub;
    if (a.max_leaves < 1) rc = set_error(BSSCL_EINVAL, "max_leaves must be >= 1");
    if (rc == BSSCL_OK && !a.bin_counts) rc = set_error(BSSCL_EINVAL, "bin_counts missing");
    std::vector<int32_t> feats(sr.feats, sr.feats + f_sub), nb((size_t)f_sub);
    for (int32_t i = 0; rc == BSSCL_OK && i < f_sub; ++i) {
      const int32_t f = feats[(size_t)i];
      if (f < 0 || f >= X.F) rc = set_error(BSSCL_EINVAL, "feature index out of range");
      else if (a.bin_counts[f] < 1 || a.bin_counts[f] > kMaxBinCount)
        rc = set_error(BSSCL_EINVAL, "bin_counts must be in [1, 65536]");
      else nb[(size_t)i] = a.bin_counts[f];
    }
    // Engine columns: a feature of more than 256 bins adds its code tiers.
    if (rc == BSSCL_OK) rc = expand_features(X, feats, nb, R.feats, R.nb_sel);
  }
  const TreeParams tp{a.max_leaves, a.max_depth, a.min_samples_leaf, a.min_child_weight,
                      a.reg_lambda, a.gamma};
  const int32_t F_sel = (int32_t)R.feats.size();
  const int nb = update_F_blocks(X.n);
  // More candidate slots than the device replay holds: host replay only.
  R.device_replay = device_replay_fits(a.max_leaves);
  R.table_readback = false;
  // The tree's compact row sets: 2s and 2s + 1.
  E->set_base = 2 * s;
  if (rc == BSSCL_OK && R.device_replay)
    rc = prepare_tree_buffers(E, m, F_sel, std::max(1, a.max_depth), a.max_leaves);
  // The root's pack, for the rows stream to upload into the slot's arena
  // (root_pin[s] and root_d[s] were last used by the round before the
  // previous one, which finish_round has waited for).
  RootPack rpk;
  std::vector<size_t> rpk_off;
  size_t total = 0;
  PreRoot pre;
  if (rc == BSSCL_OK && R.device_replay) {
    build_root_pack(E, m, R.feats, R.nb_sel, rpk);
    total = pack_layout(rpk.pk, rpk_off);
    if (E->root_pin_n[s] < total) {
      if (E->root_pin[s]) (void)hipHostFree(E->root_pin[s]);
      E->root_pin[s] = nullptr;
      E->root_pin_n[s] = 0;
      hipError_t e = hipHostMalloc(reinterpret_cast<void **>(&E->root_pin[s]), 2 * total,
                                   hipHostMallocDefault);
      if (e != hipSuccess) rc = set_error(BSSCL_EDEVICE, std::string("root pack: ") + hipGetErrorString(e));
      else E->root_pin_n[s] = 2 * total;
    }
    if (rc == BSSCL_OK) rc = E->root_d[s].ensure(total);
    if (rc == BSSCL_OK) {
      pre.n_hist = rpk.rp.n_hist;
      pre.dev.resize(rpk_off.size());
      for (size_t i = 0; i < rpk_off.size(); ++i) pre.dev[i] = E->root_d[s].p + rpk_off[i];
    }
  }
  // The round's in-bag rows on the device, ascending: the reference's
  // sample_idx (a prefix of the cumulative permutation) sorted.  Made on
  // the rows stream; only that stream touches the permutation, the
  // Fisher-Yates arrays, the row flags and round_rows[s] until rows_ready[s].
  // (round_rows[s] was last read by the tree of the round before the
  // previous one, which finish_round has waited for.)
  const int64_t n_pad = sort_rows_flag_bytes(X.n);
  hipStream_t rs = E->st_rows;
  if (rc == BSSCL_OK) rc = E->round_rows[s].ensure((size_t)m);
  if (rc == BSSCL_OK) rc = E->sort_tmp.ensure((size_t)(n_pad / 4096 + 1));
  if (rc == BSSCL_OK && E->row_flags_n != n_pad) {
    rc = E->row_flags.ensure((size_t)n_pad);
    if (rc == BSSCL_OK) {
      hipError_t e = hipMemsetAsync(E->row_flags.p, 0, (size_t)n_pad, rs);
      if (e != hipSuccess) rc = set_error(BSSCL_EDEVICE, std::string("flags: ") + hipGetErrorString(e));
      else E->row_flags_n = n_pad;
    }
  }
  if (rc == BSSCL_OK) {
    hipError_t e = hipSuccess;
    const int32_t *rows_d = nullptr;
    FyWork w;
    bool fy = false;  // this round's Fisher-Yates steps run on the device
    if (!sh.do_rows) {
      e = launch_iota(rs, E->round_rows[s].p, m);  // every row, in order
    } else if (sh.device_rows) {
      if (sh.device != E->device)
        rc = set_error(BSSCL_EINVAL, "boost_round: the sampler copies its draws to another GPU");
      // Cumulative permutation: identity before the sampler's first round.
      if (rc != BSSCL_OK) {
      } else if (sr.round == 0) {
        rc = E->perm[0].ensure((size_t)X.n);
        if (rc == BSSCL_OK) rc = E->perm[1].ensure((size_t)X.n);
        if (rc == BSSCL_OK) {
          E->perm_cur = 0;
          E->perm_sampler = sampler;
          E->perm_next_round = 0;
          e = launch_iota(rs, E->perm[0].p, X.n);
        }
      } else if (E->perm_sampler != sampler || E->perm_next_round != sr.round) {
        rc = set_error(BSSCL_EINVAL, "boost_round: the sampler's earlier rounds did not run on this engine");
      }
      if (rc == BSSCL_OK) rc = ensure_fy_work(E, X.n, w);
      // The sampler copied the draws on its own stream.
      if (rc == BSSCL_OK && e == hipSuccess) e = hipStreamWaitEvent(rs, sr.draws_copied, 0);
      if (rc == BSSCL_OK && e == hipSuccess) {
        fy = true;
        rows_d = E->perm[E->perm_cur ^ 1].p;
      }
    } else {
      rc = E->rows_in.ensure((size_t)m);
      if (rc == BSSCL_OK) e = hipMemcpyAsync(E->rows_in.p, sr.rows, (size_t)m * 4, hipMemcpyHostToDevice, rs);
      rows_d = E->rows_in.p;
    }
    // The root's pack (root_d[s], like sets 2s and 2s + 1, was last read by
    // the tree of the round before the previous one).
    if (rc == BSSCL_OK && e == hipSuccess && R.device_replay) {
      rpk.draws = fy ? static_cast<const void *>(sr.draws_dev) : nullptr;
      pack_copy(rpk.pk, rpk_off, E->root_pin[s]);
      e = hipMemcpyAsync(E->root_d[s].p, E->root_pin[s], total, hipMemcpyHostToDevice, rs);
    }
    // Device rows after the sampler's first round go through the slot's
    // rows graph; the draws' address reaches it in the root's pack.
    const bool rows_graph = fy && sr.round > 0 && R.device_replay && E->prof <= 1;
    if (rows_graph)
      w.draws_ref = reinterpret_cast<const uint32_t *const *>(pre.dev[kPackDraws]);
    const int cur = E->perm_cur;
    auto rows_launches = [&]() -> int {
      hipError_t e2 = hipSuccess;
      // The sorted Fisher-Yates form flags the in-bag rows as it writes them.
      const bool marked = fy && w.keys;
      if (fy)
        e2 = launch_fisher_yates(rs, w.draws_ref ? nullptr : sr.draws_dev, X.n, E->perm[cur].p,
                                 E->perm[cur ^ 1].p, w, marked ? E->row_flags.p : nullptr, m);
      if (e2 == hipSuccess && rows_d)
        e2 = launch_sort_rows(rs, rows_d, m, E->row_flags.p, n_pad, E->sort_tmp.p,
                              E->round_rows[s].p, marked);
      if (e2 == hipSuccess && R.device_replay)
        e2 = launch_gather_codes(rs, X.codes.p, X.ld,
                                 reinterpret_cast<const int32_t *>(pre.dev[kPackFeat]), F_sel,
                                 E->round_rows[s].p, m, E->codes_c[2 * s].p, E->ld_c, E->ld_c);
      if (e2 != hipSuccess) return set_error(BSSCL_EDEVICE, std::string("rows: ") + hipGetErrorString(e2));
      return BSSCL_OK;
    };
    if (rc == BSSCL_OK && e == hipSuccess) {
      if (rows_graph) {
        std::vector<uint64_t> key;
        key_add(key, g_alloc_gen.load(std::memory_order_relaxed));
        for (int64_t v : {(int64_t)s, X.n, X.ld, m, (int64_t)cur, n_pad, (int64_t)F_sel, E->ld_c})
          key_add(key, v);
        for (const void *ptr : {(const void *)X.codes.p, (const void *)pre.dev[kPackFeat],
                                (const void *)pre.dev[kPackDraws], (const void *)w.keys,
                                (const void *)rows_d})
          key_add(key, ptr);
        bool replayed = false;
        rc = run_graph(E, E->rows_graph[s], key, rs, false, rows_launches, &replayed);
        if (rc == BSSCL_OK && replayed) E->stats[18] += 1.0;
      } else {
        rc = rows_launches();
      }
    }
    if (rc == BSSCL_OK && e == hipSuccess && fy) {
      E->perm_cur = cur ^ 1;
      E->perm_next_round = sr.round + 1;
    }
    if (rc == BSSCL_OK && e == hipSuccess && !E->rows_ready[s])
      e = hipEventCreateWithFlags(&E->rows_ready[s], hipEventDisableTiming);
    if (rc == BSSCL_OK && e == hipSuccess) e = hipEventRecord(E->rows_ready[s], rs);
    if (rc == BSSCL_OK && e == hipSuccess) e = hipStreamWaitEvent(E->st, E->rows_ready[s], 0);
    if (rc == BSSCL_OK && e != hipSuccess) rc = set_error(BSSCL_EDEVICE, std::string("rows: ") + hipGetErrorString(e));
  }
  if (rc != BSSCL_OK) return fail(rc);
  if (rc == BSSCL_OK) rc = E->partials_d.ensure((size_t)nb);
  if (rc == BSSCL_OK) rc = E->tree_d.ensure((size_t)R.M);
  if (rc == BSSCL_OK) rc = ensure_round_out(E, s, R.M, nb);
  // Gradients from the current F (est:2868): for every row on the
  // host-driven path, which gathers them itself.
  if (rc == BSSCL_OK && !R.device_replay) rc = host_round_scales(E, m, gm, hm);
  if (rc == BSSCL_OK && !R.device_replay) {
    const hipError_t e = launch_grad_hess(E->st, E->F.p, E->y.p, X.n, E->w0, E->w1, gm, hm,
                                          E->ghq.p);
    if (e != hipSuccess) rc = set_error(BSSCL_EDEVICE, std::string("gradients: ") + hipGetErrorString(e));
  }
  if (rc == BSSCL_OK && R.device_replay) {
    RoundHeader *hdr = reinterpret_cast<RoundHeader *>(E->round_d[s].p);
    ReplayArgs ra = replay_args(E, tp, R.M);
    // The tree's fixed point from the largest |g| and h of the current F
    // (every row's; the in-bag rows are among them), which the previous
    // F update or boost_begin left on the device.
    const char *bound_env = std::getenv("BSSCL_TEST_BOUND_SCALE");
    const bool dev_scale = E->gh_ok && !(bound_env && bound_env[0] == '1');
    DevScale dv{nullptr, 0, 0};
    unsigned long long *gh_next = nullptr, *gh_cur = nullptr;
    if (E->gh_ok) {
      gh_cur = E->ghmax_d.p + 2 * E->gh_slot;
      gh_next = E->ghmax_d.p + 2 * (E->gh_slot ^ 1);
    }
    if (dev_scale) dv = DevScale{gh_cur, fixed_bits(m), 0};
    ra.dev = dv;
    R.table_readback = E->prof && !replay_counts_nodes(ra);
    char *const partials = E->round_d[s].p + round_out_bytes(R.M);
    const bool checks = !E->pipeline;
    // Gradients of the in-bag rows straight into the root's set, the tree,
    // its replay, then F += lr * tree(X) with the per-block losses, which the
    // host sums (sum_partials_host).
    auto tree_launches = [&]() -> int {
      hipError_t e = launch_gather_gh(E->st, E->F.p, E->y.p, E->round_rows[s].p, m, E->w0,
                                      E->w1, gm, hm, dv, E->gh_c[2 * s].p, E->ld_c, E->segs.p,
                                      E->hist_node_d.p,
                                      reinterpret_cast<const LevelPlan *>(pre.dev[kPackPlan]),
                                      E->plan_d);
      if (e != hipSuccess) return set_error(BSSCL_EDEVICE, std::string("gradients: ") + hipGetErrorString(e));
      E->round_dev = dv;
      const int trc = launch_tree(E, E->round_rows[s].p, m, R.feats, R.nb_sel, tp, &R.run,
                                  checks, true, &pre);
      E->round_dev = DevScale{nullptr, 0, 0};
      CHK(trc);
      e = launch_replay(E->st, E->nodes_d, E->plan_d, E->feat_d, ra,
                        round_arrays(E->round_d[s].p, R.M), E->tree_d.p, hdr);
      if (e == hipSuccess)
        e = launch_update_F(E->st, X.codes.p, X.ld, X.n, E->tree_d.p, R.M, &hdr->node_count,
                            a.learning_rate, E->F.p, E->y.p, reinterpret_cast<double *>(partials),
                            nb, E->w0, E->w1, gh_next, gh_cur);
      // The round's readback (tree arrays and losses) into pinned memory,
      // inside the graph: an operation enqueued after a graph waits for
      // the graph's completion, which costs microseconds per round.
      if (e == hipSuccess)
        e = hipMemcpyAsync(E->round_pin[s], E->round_d[s].p, round_out_bytes(R.M) + (size_t)nb * 8,
                           hipMemcpyDeviceToHost, E->st);
      if (e != hipSuccess) return set_error(BSSCL_EDEVICE, std::string("round: ") + hipGetErrorString(e));
      return BSSCL_OK;
    };
    // A tree graph needs every level enqueued without a host check, and
    // profiling off.
    const bool tree_graph =
        E->prof == 0 && (!checks || std::max(1, a.max_depth) <= kLevelsPerCheck);
    if (tree_graph) {
      const bool pair = want_pair_levels(E);
      std::vector<uint64_t> key;
      key_add(key, g_alloc_gen.load(std::memory_order_relaxed));
      for (int64_t v : {(int64_t)s, X.n, X.ld, m, (int64_t)F_sel, (int64_t)R.M, (int64_t)nb,
                        (int64_t)E->prof, (int64_t)checks, (int64_t)pair, (int64_t)E->plan_lds,
                        (int64_t)E->track_rid, (int64_t)E->node_cap, (int64_t)E->tile_cap,
                        (int64_t)E->hist_cap, E->ld_c, E->node_stride, (int64_t)E->part_rows,
                        (int64_t)pre.n_hist, (int64_t)ra.stage_limit,
                        (int64_t)E->hist_fc, (int64_t)E->hist_copies, (int64_t)E->hist_fc_span,
                        (int64_t)E->hist_copies_span, (int64_t)E->hist_blocks_per_cu,
                        (int64_t)E->hist_rows_per_flush, (int64_t)E->hist_rows_per_flush_level,
                        (int64_t)tp.max_leaves, (int64_t)tp.max_depth,
                        (int64_t)tp.min_samples_leaf})
        key_add(key, v);
      for (double v : {tp.mcw, tp.lam, tp.gamma, a.learning_rate, gm, hm, E->w0, E->w1})
        key_add(key, v);
      for (int64_t v : {(int64_t)E->gh_ok, (int64_t)dev_scale, (int64_t)E->gh_slot})
        key_add(key, v);
      // (round_pin is host memory: its address is not covered by the
      // allocation count.)
      for (const void *ptr : {(const void *)X.codes.p, (const void *)pre.dev[kPackFeat],
                              (const void *)pre.dev[kPackNbHot], (const void *)pre.dev[kPackHist],
                              (const void *)pre.dev[kPackPlan], (const void *)pre.dev[kPackTasks],
                              (const void *)E->round_pin[s]})
        key_add(key, ptr);
      bool replayed = false;
      RoundGraph &g = E->tree_graph[s];
      rc = run_graph(E, g, key, E->st, true, tree_launches, &replayed);
      if (rc == BSSCL_OK && replayed) {
        E->stats[19] += 1.0;
        if (R.run > 0) g.run = R.run;  // captured in this round
        else R.run = g.run;
      }
    } else {
      rc = tree_launches();
    }
    hipError_t e = rc == BSSCL_OK ? hipSuccess : hipErrorUnknown;
    if (e == hipSuccess && R.table_readback)
      e = hipMemcpyAsync(E->rtable_pin[s], E->table_d.p,
                         64 + (size_t)table_bound(E, R.run) * sizeof(NodeOut),
                         hipMemcpyDeviceToHost, E->st);
    if (e == hipSuccess && !R.done) e = hipEventCreateWithFlags(&R.done, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventRecord(R.done, E->st);
    if (rc == BSSCL_OK && e != hipSuccess) rc = set_error(BSSCL_EDEVICE, std::string("round: ") + hipGetErrorString(e));
    // The F update raised the other slot.
    if (rc == BSSCL_OK && E->gh_ok) E->gh_slot ^= 1;
  }
  if (rc != BSSCL_OK) return fail(rc);
  E->launched_round = true;
  return BSSCL_OK;
}

// Waits for the round in slot s, returns its sampler buffers and hands its
// tree and loss to the caller (finishing it on the host-driven path when
// the device path could not).
int finish_round(bsscl_engine *E, int s, TreeOut &out, double *out_train_loss) {
  const Matrix &X = E->mat[0];
  RoundSlot &R = E->rslot[s];
  if (!R.active) return set_error(BSSCL_EINTERNAL, "boost_round: no round in flight");
  const TreeParams tp{R.args.max_leaves, R.args.max_depth, R.args.min_samples_leaf,
                      R.args.min_child_weight, R.args.reg_lambda, R.args.gamma};
  hipError_t e = hipSuccess;
  if (R.device_replay) {
    e = hipEventSynchronize(R.done);
  } else {
    e = hipStreamSynchronize(E->st);  // the sampler's buffers must be read first
  }
  if (e == hipSuccess && E->prof) {
    const int rc = prof_collect(E, R.seq);
    if (rc != BSSCL_OK) e = hipErrorUnknown;
  }
  sampler_give_back(R.sampler, R.token);
  R.active = false;
  R.token = nullptr;
  if (e != hipSuccess) return set_error(BSSCL_EDEVICE, std::string("boost_round: ") + hipGetErrorString(e));
  const int32_t M = R.M;
  RoundHeader h;
  if (R.device_replay) {
    h = *reinterpret_cast<const RoundHeader *>(E->round_pin[s]);
  } else {
    h = RoundHeader{};
    h.status = 4;
  }
  if (h.status == 0) {
    if (E->prof && h.expanded >= 0) {
      tree_stats_add(E, R.m, (int32_t)R.feats.size(), h.hist_rows, h.expanded);
    } else if (R.table_readback) {
      const LevelPlan *pl = reinterpret_cast<const LevelPlan *>(E->rtable_pin[s]);
      const int32_t tb = table_bound(E, R.run);
      if (pl->overflow == 0 && pl->n_nodes >= 1 && pl->n_nodes <= tb)
        tree_stats(E, reinterpret_cast<const NodeOut *>(E->rtable_pin[s] + 64), pl->n_nodes, R.m,
                   (int32_t)R.feats.size(), tp);
    }
    const TreeArrays ha = round_arrays(E->round_pin[s], M);
    std::memcpy(out.features, ha.features, (size_t)M * 4);
    std::memcpy(out.thresholds, ha.thresholds, (size_t)M * 8);
    std::memcpy(out.values, ha.values, (size_t)M * 8);
    std::memcpy(out.left, ha.left, (size_t)M * 4);
    std::memcpy(out.right, ha.right, (size_t)M * 4);
    std::memcpy(out.gains, ha.gains, (size_t)M * 8);
    *out.node_count = h.node_count;
    tree_to_reference(X, out);
    if (out_train_loss) {
      const double *parts =
          reinterpret_cast<const double *>(E->round_pin[s] + round_out_bytes(R.M));
      *out_train_loss = -sum_partials_host(parts, update_F_blocks(X.n)) / (double)X.n;
    }
    return BSSCL_OK;
  }
  if (h.status != 1 && h.status != 4)
    return set_error(BSSCL_EINTERNAL, "tree builder: device replay failed (status " +
                                          std::to_string(h.status) + ")");
  // F was left alone: build the tree on the host-driven path and apply it.
  // (Never with a round enqueued behind this one: see pipeline_safe.)
  if (h.status == 1) E->node_cap_floor = std::max(h.needed, 2 * E->node_cap);
  {
    // Gradients of every row from the unchanged F (the device path gathered
    // only the in-bag rows'), with the scales the device path used.
    double gm = 0.0, hm = 0.0;
    CHK(host_round_scales(E, R.m, gm, hm));
    HIPCHK(launch_grad_hess(E->st, E->F.p, E->y.p, X.n, E->w0, E->w1, gm, hm, E->ghq.p));
  }
  E->set_base = 2 * s;
  CHK(build_tree_core(E, E->round_rows[s].p, R.m, R.feats, R.nb_sel, tp, out));
  CHK(upload_tree(E, out.features, out.thresholds, out.values, out.left, out.right,
                  *out.node_count, X.cols()));
  tree_to_reference(X, out);
  const int nb = update_F_blocks(X.n);
  CHK(E->loss_d.ensure(1));
  {
    unsigned long long *gh_cur = E->gh_ok ? E->ghmax_d.p + 2 * E->gh_slot : nullptr;
    unsigned long long *gh_next = E->gh_ok ? E->ghmax_d.p + 2 * (E->gh_slot ^ 1) : nullptr;
    const hipError_t e2 = launch_update_F(E->st, X.codes.p, X.ld, X.n, E->tree_d.p,
                                          *out.node_count, nullptr, R.args.learning_rate,
                                          E->F.p, E->y.p, E->partials_d.p, nb, E->w0, E->w1,
                                          gh_next, gh_cur);
    if (e2 != hipSuccess) {
      E->gh_ok = false;
      return set_error(BSSCL_EDEVICE, std::string("F update: ") + hipGetErrorString(e2));
    }
    if (E->gh_ok) E->gh_slot ^= 1;
  }
  HIPCHK(launch_sum_partials(E->st, E->partials_d.p, nb, E->loss_d.p));
  double sum = 0.0;
  HIPCHK(hipMemcpyAsync(&sum, E->loss_d.p, 8, hipMemcpyDeviceToHost, E->st));
  CHK(sync(E));
  if (out_train_loss) *out_train_loss = -sum / (double)X.n;
  return BSSCL_OK;
}

// Every class's gradients and hessians from the scores at the round's start
// (est:2996, 3013-3019) and each class's fixed point from its largest |g|
// and h, read back; the round's m in-bag rows are already on the device.
int mc_read_scales(bsscl_engine *E);

int mc_gradients(bsscl_engine *E, int64_t m, bool read_back = true) {
  const int64_t n = E->mat[0].n;
  const int32_t K = E->mc_K;
  HIPCHK(hipMemsetAsync(E->mc_max.p, 0, 2 * (size_t)K * 8, E->st));
  HIPCHK(launch_mc_grad_hess(E->st, E->mc_F.p, E->mc_y.p, E->mc_w.p, n, K, E->mc_G.p, E->mc_H.p,
                             E->mc_max.p));
  E->mc_m = m;
  E->mc_scales_host = false;
  return read_back ? mc_read_scales(E) : BSSCL_OK;
}

// Each class's fixed point from its largest |g| and h of the round, read
// back from the device (mc_max) after the gradient kernel.
int mc_read_scales(bsscl_engine *E) {
  const int32_t K = E->mc_K;
  const int64_t m = E->mc_m;
  unsigned long long mx[2 * kMcMaxK];
  HIPCHK(hipMemcpyAsync(mx, E->mc_max.p, 2 * (size_t)K * 8, hipMemcpyDeviceToHost, E->st));
  HIPCHK(hipStreamSynchronize(E->st));
  E->mc_gm.assign((size_t)K, 0.0);
  E->mc_hm.assign((size_t)K, 0.0);
  E->mc_hmax.assign((size_t)K, 0.0);
  for (int32_t k = 0; k < K; ++k) {
    double gmax, hmax;
    std::memcpy(&gmax, &mx[2 * k], 8);
    std::memcpy(&hmax, &mx[2 * k + 1], 8);
    if (!std::isfinite(gmax) || !std::isfinite(hmax)) {
      E->mc_m = 0;
      return set_error(BSSCL_EINVAL, "mc_round: gradients are not finite");
    }
    // The scale load_grad_hess would take from the same arrays.
    E->mc_gm[(size_t)k] = fixed_mul(gmax, m);
    E->mc_hm[(size_t)k] = fixed_mul(hmax, m);
    E->mc_hmax[(size_t)k] = hmax;
  }
  E->mc_scales_host = true;
  return BSSCL_OK;
}

// The in-bag rows of a sampler's round on the device, into round_rows[slot]
// on stream `st`: every row in order without row bagging; with device rows,
// the round's steps of the reference's shuffle (est:2506) applied to the
// cumulative permutation and its first n_sub entries sorted ascending, as a
// boosting round makes them; otherwise the sampler's rows, in the
// reference's order.  (A tree's histograms are exact integer sums and its
// partitions stable, so the order of its rows does not enter it.)  The
// sampler's round must stay taken until the work on `st` is done.
int mc_rows_from_sampler(bsscl_engine *E, bsscl_sampler *sampler, const SamplerShape &sh,
                         const SamplerRound &sr, int slot, hipStream_t st) {
  const Matrix &X = E->mat[0];
  const int64_t m = sh.n_sub;
  if (m <= 0) return set_error(BSSCL_EINVAL, "mc round: no samples");
  CHK(E->round_rows[slot].ensure((size_t)m));
  int32_t *out = E->round_rows[slot].p;
  if (!sh.do_rows) {
    HIPCHK(launch_iota(st, out, m));
    return BSSCL_OK;
  }
  if (!sh.device_rows) {
    HIPCHK(hipMemcpyAsync(out, sr.rows, (size_t)m * 4, hipMemcpyHostToDevice, st));
    return BSSCL_OK;
  }
  if (sh.device != E->device)
    return set_error(BSSCL_EINVAL, "mc round: the sampler copies its draws to another GPU");
  // The cumulative permutation: identity before the sampler's first round.
  if (sr.round == 0) {
    CHK(E->perm[0].ensure((size_t)X.n));
    CHK(E->perm[1].ensure((size_t)X.n));
    E->perm_cur = 0;
    E->perm_sampler = sampler;
    E->perm_next_round = 0;
    HIPCHK(launch_iota(st, E->perm[0].p, X.n));
  } else if (E->perm_sampler != sampler || E->perm_next_round != sr.round) {
    return set_error(BSSCL_EINVAL, "mc round: the sampler's earlier rounds did not run on this engine");
  }
  const int64_t n_pad = sort_rows_flag_bytes(X.n);
  CHK(E->sort_tmp.ensure((size_t)(n_pad / 4096 + 1)));
  if (E->row_flags_n != n_pad) {
    CHK(E->row_flags.ensure((size_t)n_pad));
    HIPCHK(hipMemsetAsync(E->row_flags.p, 0, (size_t)n_pad, st));
    E->row_flags_n = n_pad;
  }
  FyWork w;
  CHK(ensure_fy_work(E, X.n, w));
  HIPCHK(hipStreamWaitEvent(st, sr.draws_copied, 0));  // the sampler copied the draws
  const int cur = E->perm_cur;
  // The sorted Fisher-Yates form flags the in-bag rows as it writes them.
  const bool marked = w.keys != nullptr;
  HIPCHK(launch_fisher_yates(st, sr.draws_dev, X.n, E->perm[cur].p, E->perm[cur ^ 1].p, w,
                             marked ? E->row_flags.p : nullptr, m));
  HIPCHK(launch_sort_rows(st, E->perm[cur ^ 1].p, m, E->row_flags.p, n_pad, E->sort_tmp.p, out,
                          marked));
  E->perm_cur = cur ^ 1;
  E->perm_next_round = sr.round + 1;
  return BSSCL_OK;
}

// Hands back a multiclass round enqueued ahead (bsscl_mc_round_trees), once
// the rows stream has finished with its draws.
void mc_drop_next(bsscl_engine *E) {
  if (!E->mc_next) return;
  (void)hipStreamSynchronize(E->st_rows);
  sampler_give_back(E->mc_next_sampler, E->mc_next_token);
  E->mc_next = false;
  E->mc_next_token = nullptr;
  E->mc_next_sampler = nullptr;
}

// Multiclass class k's fixed point: the round's largest |g| and h of the
// class (bsscl_mc_round).
int mc_class_scales(bsscl_engine *E, int32_t k) {
  if (!E->mc_scales_host) CHK(mc_read_scales(E));
  E->g_scale = 1.0 / E->mc_gm[(size_t)k];
  E->h_scale = 1.0 / E->mc_hm[(size_t)k];
  E->h_bound = E->mc_hmax[(size_t)k];
  return BSSCL_OK;
}

// Class k's tree of the multiclass round on the host-driven path (its node
// table comes back and the host replays est:641-820), then
// F[:, k] += lr * tree(X) (est:3029).
int mc_tree_host(bsscl_engine *E, int32_t k, const std::vector<int32_t> &feats,
                 const std::vector<int32_t> &nb_sel, const TreeParams &tp, double lr,
                 TreeOut &out) {
  const Matrix &X = E->mat[0];
  const int64_t n = X.n;
  CHK(mc_class_scales(E, k));
  HIPCHK(launch_quantize(E->st, E->mc_G.p + (size_t)k * n, E->mc_H.p + (size_t)k * n, n,
                         E->mc_gm[(size_t)k], E->mc_hm[(size_t)k], E->ghq.p));
  E->set_base = 0;
  CHK(build_tree_core(E, E->mc_rows32, E->mc_m, feats, nb_sel, tp, out));
  // (upload_tree takes the tree in the engine's columns.)
  CHK(upload_tree(E, out.features, out.thresholds, out.values, out.left, out.right,
                  *out.node_count, X.cols()));
  HIPCHK(launch_mc_apply(E->st, X.codes.p, X.ld, n, E->tree_d.p, nullptr, lr,
                         E->mc_F.p + (size_t)k * n));
  tree_to_reference(X, out);
  return BSSCL_OK;
}

// The round's K trees back to back with no host wait between them: per
// class its quantized gradients, the tree, the tree's replay on the device
// and F[:, k] += lr * tree(X) (k_mc_apply skips it when the replay failed);
// then one readback of the K trees.  The classes' gradients all come from
// the scores before the round (est:3013-3019), so the order of the K
// updates does not enter any tree, and a class whose device replay failed
// is built again on the host-driven path from its unchanged gradients.
// `out(k)` gives class k's output arrays.
template <typename OutFn>
int mc_trees_device(bsscl_engine *E, const std::vector<int32_t> &feats,
                    const std::vector<int32_t> &nb_sel, const TreeParams &tp, double lr,
                    OutFn out) {
  const Matrix &X = E->mat[0];
  const int64_t n = X.n, m = E->mc_m;
  const int32_t K = E->mc_K, M = 2 * tp.max_leaves + 2;
  const int32_t F_sel = (int32_t)feats.size();
  const size_t per = round_out_bytes(M);
  // (mc_out_d is released only when no copy reads it: the previous call
  // ended with a synchronisation.)
  CHK(E->tree_d.ensure((size_t)M));
  CHK(E->mc_out_d.ensure(per * (size_t)K));
  CHK(ensure_host_pinned(E, E->mc_out_pin, E->mc_out_pin_bytes, per * (size_t)K));
  // The K trees share their rows and features: the round's root codes are
  // gathered once into set 2, which the trees' levels never write (they
  // alternate between sets 0 and 1), and each class's root gathers its
  // (g,h) alone.
  // (Rows given as int64 by bsscl_mc_round have no int32 list for that
  // gather: each class then gathers its root itself.)
  const bool shared_root = E->mc_rows32 != nullptr;
  E->set_base = 0;
  E->root_set = shared_root ? 2 : -1;
  struct RootReset {
    bsscl_engine *e;
    ~RootReset() {
      e->root_set = -1;
      e->root_codes_ready = false;
    }
  } root_reset{E};
  CHK(prepare_tree_buffers(E, m, F_sel, std::max(1, tp.max_depth), tp.max_leaves));
  if (shared_root) {
    CHK(upload(E, E->mc_feat_d, feats.data(), feats.size()));
    HIPCHK(launch_gather_codes(E->st, X.codes.p, X.ld, E->mc_feat_d.p, F_sel, E->mc_rows32, m,
                               E->codes_c[2].p, E->ld_c, E->ld_c));
    E->root_codes_ready = true;
  }
  for (int32_t k = 0; k < K; ++k) {
    // The class's fixed point: from the maxima the host read back, or from
    // those on the device (the same multipliers, dev_fixed_mul), with the
    // hessian bound max weight / 4 for the planner's kept-split rule.
    DevScale dv{nullptr, 0, 0};
    if (E->mc_scales_host) {
      CHK(mc_class_scales(E, k));
    } else {
      dv = DevScale{E->mc_max.p + 2 * k, fixed_bits(m), 0};
      E->g_scale = E->h_scale = 1.0;  // (the kernels take dv's)
      E->h_bound = E->mc_hbound;
    }
    HIPCHK(launch_quantize(E->st, E->mc_G.p + (size_t)k * n, E->mc_H.p + (size_t)k * n, n,
                           dv.max ? 1.0 : E->mc_gm[(size_t)k], dv.max ? 1.0 : E->mc_hm[(size_t)k],
                           E->ghq.p, dv));
    int32_t run = 0;
    E->round_dev = dv;
    const int trc = launch_tree(E, E->mc_rows32, m, feats, nb_sel, tp, &run);
    E->round_dev = DevScale{nullptr, 0, 0};
    CHK(trc);
    char *base = E->mc_out_d.p + (size_t)k * per;
    RoundHeader *hdr = reinterpret_cast<RoundHeader *>(base);
    ReplayArgs ra = replay_args(E, tp, M);
    ra.dev = dv;
    HIPCHK(launch_replay(E->st, E->nodes_d, E->plan_d, E->feat_d, ra, round_arrays(base, M),
                         E->tree_d.p, hdr));
    HIPCHK(launch_mc_apply(E->st, X.codes.p, X.ld, n, E->tree_d.p, &hdr->node_count, lr,
                           E->mc_F.p + (size_t)k * n));
  }
  HIPCHK(hipMemcpyAsync(E->mc_out_pin, E->mc_out_d.p, per * (size_t)K, hipMemcpyDeviceToHost,
                        E->st));
  CHK(sync(E));
  // (A class rebuilt on the host-driven path below gathers its own root.)
  E->root_set = -1;
  E->root_codes_ready = false;
  for (int32_t k = 0; k < K; ++k) {
    TreeOut o = out(k);
    const char *base = E->mc_out_pin + (size_t)k * per;
    RoundHeader h;
    std::memcpy(&h, base, sizeof(h));
    if (h.status == 0) {
      if (E->prof && h.expanded >= 0) tree_stats_add(E, m, F_sel, h.hist_rows, h.expanded);
      const TreeArrays ha = round_arrays(const_cast<char *>(base), M);
      std::memcpy(o.features, ha.features, (size_t)M * 4);
      std::memcpy(o.thresholds, ha.thresholds, (size_t)M * 8);
      std::memcpy(o.values, ha.values, (size_t)M * 8);
      std::memcpy(o.left, ha.left, (size_t)M * 4);
      std::memcpy(o.right, ha.right, (size_t)M * 4);
      std::memcpy(o.gains, ha.gains, (size_t)M * 8);
      *o.node_count = h.node_count;
      tree_to_reference(X, o);
      continue;
    }
    if (h.status != 1 && h.status != 4)
      return set_error(BSSCL_EINTERNAL, "tree builder: device replay failed (status " +
                                            std::to_string(h.status) + ")");
    // The node table was too small, or the replay could not finish: F[:, k]
    // was left alone.
    if (h.status == 1) E->node_cap_floor = std::max(h.needed, 2 * E->node_cap);
    CHK(mc_tree_host(E, k, feats, nb_sel, tp, lr, o));
  }
  return BSSCL_OK;
}

}  // namespace
}  // namespace bsscl

// ===========================================================================
// C ABI
// ===========================================================================
namespace bsscl {

hipStream_t copy_stream(int device) {
  static std::mutex mu;
  static std::vector<hipStream_t> streams;
  std::lock_guard<std::mutex> lk(mu);
  if (device < 0) return nullptr;
  if ((size_t)device >= streams.size()) streams.resize((size_t)device + 1, nullptr);
  hipStream_t &s = streams[(size_t)device];
  if (!s) {
    int cur = 0;
    (void)hipGetDevice(&cur);
    if (hipSetDevice(device) != hipSuccess ||
        hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess)
      s = nullptr;
    (void)hipSetDevice(cur);
  }
  return s;
}

}  // namespace bsscl

namespace bsscl {
namespace {

// The ensemble's F of matrix `slot` into E->out_d (est:863-884).
// The packed trees (est:2192-2216) on the device in the engine's columns of
// matrices with M's features and tiers: tree_d, and offsets_d with, for the
// LDS-staged walk (*staged), its *n_chunks runs of whole trees after them.
int upload_trees(bsscl_engine *E, const Matrix &M, const int16_t *features,
                 const int64_t *thresholds, const double *values, const int32_t *left,
                 const int32_t *right, const int32_t *offsets, int32_t n_trees, bool *staged_out,
                 int32_t *n_chunks_out) {
  const int32_t total = n_trees > 0 ? offsets[n_trees] : 0;
  std::vector<TreeNodeDev> nodes((size_t)std::max(total, 1));
  bool adjacent = true;  // every right child is its left child + 1
  for (int32_t t = 0; t < n_trees; ++t) {
    const int32_t a = offsets[t], b = offsets[t + 1];
    if (a < 0 || b <= a || b > total) return set_error(BSSCL_EINVAL, "predict: bad offsets");
    for (int32_t i = a; i < b; ++i) {
      TreeNodeDev &d = nodes[(size_t)i];
      d.value = values[i];
      d.feature = features[i];
      if (d.feature >= 0) {
        const int32_t l = left[i], r = right[i];
        if (d.feature >= M.F || l < 0 || r < 0 || l >= b - a || r >= b - a || l <= i - a || r <= i - a)
          return set_error(BSSCL_EINVAL, "predict: malformed tree " + std::to_string(t));
        adjacent = adjacent && r == l + 1;
        int64_t thr = thresholds[i];
        split_to_engine(M, d.feature, thr);
        d.threshold = (int32_t)std::max<int64_t>(-1, std::min<int64_t>(thr, 1 << 20));
        d.left = l;
        d.right = r;
      } else {
        d.feature = -1;
        d.threshold = 0;
        d.left = d.right = 0;
      }
    }
  }
  CHK(E->pin.reserve(std::max<size_t>(E->pin.cap, 8u << 20)));
  // The offsets, then (for the LDS-staged kernel) the runs of whole trees it
  // stages at a time.
  int32_t max_nodes = 0;
  for (int32_t t = 0; t < n_trees; ++t) max_nodes = std::max(max_nodes, offsets[t + 1] - offsets[t]);
  // (Test hook BSSCL_TEST_PREDICT_GLOBAL=1: every row walks the trees in HBM.)
  const bool staged = n_trees > 0 && predict_staged_ok(M.cols(), max_nodes, adjacent) &&
                      !std::getenv("BSSCL_TEST_PREDICT_GLOBAL");
  // (A model without trees may pass no arrays at all: offsets is read only
  // when there are trees.)
  std::vector<int32_t> offs((size_t)n_trees + 1, 0);
  if (n_trees > 0) std::copy(offsets, offsets + n_trees + 1, offs.begin());
  int32_t n_chunks = 0;
  if (staged) {
    offs.resize(2 * ((size_t)n_trees + 1));
    n_chunks = predict_chunks(offsets, n_trees, offs.data() + n_trees + 1);
  }
  CHK(upload(E, E->tree_d, nodes.data(), nodes.size()));
  CHK(upload(E, E->offsets_d, offs.data(), offs.size()));
  *staged_out = staged;
  *n_chunks_out = n_chunks;
  return BSSCL_OK;
}

int predict_to_device(bsscl_engine *E, int32_t slot, const int16_t *features,
                      const int64_t *thresholds, const double *values,
                      const int32_t *left, const int32_t *right,
                      const int32_t *offsets, int32_t n_trees, double learning_rate) {
  if (!E || (n_trees > 0 && (!features || !thresholds || !values || !left || !right || !offsets)))
    return set_error(BSSCL_EINVAL, "predict: null argument");
  CHK(check_matrix(E, slot));
  if (n_trees < 0) return set_error(BSSCL_EINVAL, "predict: negative tree count");
  HIPCHK(hipSetDevice(E->device));
  const Matrix &M = E->mat[slot];
  bool staged = false;
  int32_t n_chunks = 0;
  CHK(upload_trees(E, M, features, thresholds, values, left, right, offsets, n_trees, &staged,
                   &n_chunks));
  CHK(E->out_d.ensure((size_t)M.n));
  hipEvent_t start, stop;
  CHK(prof_kernel(E, 4, &start, &stop));
  HIPCHK(launch_predict(E->st, M.codes.p, M.ld, M.n, M.cols(), E->tree_d.p, E->offsets_d.p,
                        n_trees, staged ? E->offsets_d.p + n_trees + 1 : nullptr, n_chunks,
                        learning_rate, E->out_d.p, start, stop));
  return BSSCL_OK;
}

}  // namespace
}  // namespace bsscl

extern "C" {

const char *bsscl_last_error(void) { return g_last_error.c_str(); }

int bsscl_device_count(int32_t *out) {
  if (!out) return set_error(BSSCL_EINVAL, "null output");
  int c = 0;
  hipError_t e = hipGetDeviceCount(&c);
  *out = (e == hipSuccess) ? c : 0;
  return BSSCL_OK;
}

int bsscl_engine_create(int32_t device, bsscl_engine **out) {
  if (!out) return set_error(BSSCL_EINVAL, "null output");
  *out = nullptr;
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= 0)
    return set_error(BSSCL_EDEVICE, "no HIP device is visible");
  if (device < 0 || device >= count)
    return set_error(BSSCL_EINVAL, "device index out of range");
  HIPCHK(hipSetDevice(device));
  bsscl_engine *E = new (std::nothrow) bsscl_engine();
  if (!E) return set_error(BSSCL_ENOMEM, "engine allocation failed");
  E->device = device;
  hipError_t e = hipStreamCreateWithFlags(&E->st, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&E->st_rows, hipStreamNonBlocking);
  if (e != hipSuccess) {
    if (E->st_rows) (void)hipStreamDestroy(E->st_rows);
    if (E->st) (void)hipStreamDestroy(E->st);
    delete E;
    return set_error(BSSCL_EDEVICE, std::string("hipStreamCreate: ") + hipGetErrorString(e));
  }
  if (!copy_stream(device)) {
    (void)hipStreamDestroy(E->st_rows);
    (void)hipStreamDestroy(E->st);
    delete E;
    return set_error(BSSCL_EDEVICE, "hipStreamCreate of the draws' copy stream failed");
  }
  int v = 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && v > 0)
    E->n_cu = v;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, device) == hipSuccess && v > 0)
    E->max_lds = (size_t)v;
  // The rate of the clock kernels read with wall_clock64 (kHz).
  E->wall_khz = 100000.0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeWallClockRate, device) == hipSuccess && v > 0)
    E->wall_khz = (double)v;
  if (scratch_for_device(device, &E->scratch_p) != BSSCL_OK) {
    const std::string msg = bsscl_last_error();
    bsscl_engine_destroy(E);
    return set_error(BSSCL_EDEVICE, msg);
  }

  *out = E;
  return BSSCL_OK;
}

void bsscl_engine_destroy(bsscl_engine *E) {
  if (!E) return;
  (void)hipSetDevice(E->device);
  if (E->st_rows) (void)hipStreamSynchronize(E->st_rows);
  if (E->st) (void)hipStreamSynchronize(E->st);
  // A round enqueued ahead hands its sampler buffers back (the sampler
  // outlives the rounds it feeds).
  if (E->ahead >= 0 && E->rslot[E->ahead].active)
    sampler_give_back(E->rslot[E->ahead].sampler, E->rslot[E->ahead].token);
  E->ahead = -1;
  mc_drop_next(E);
  if (E->mc_next_ev) (void)hipEventDestroy(E->mc_next_ev);
  for (int b = 0; b < 2; ++b) {
    release_graph(E->rows_graph[b]);
    release_graph(E->tree_graph[b]);
  }
  for (auto &m : E->mat) m.codes.release();
  E->F.release();
  E->ghmax_d.release();
  E->y.release();
  E->ghq.release();
  E->g64.release();
  E->h64.release();
  for (int s = 0; s < 4; ++s) {
    E->codes_c[s].release();
    E->gh_c[s].release();
  }
  for (int s = 0; s < 2; ++s) {
    E->rid_c[s].release();
    E->root_d[s].release();
    if (E->root_pin[s]) (void)hipHostFree(E->root_pin[s]);
  }
  for (auto &r : E->round_rows) r.release();
  E->rows64.release();
  E->rows_in.release();
  E->sort_tmp.release();
  for (int s = 0; s < 2; ++s) E->perm[s].release();
  E->fy_head.release();
  E->fy_next.release();
  E->fy_v.release();
  for (auto &k : E->fy_keys) k.release();
  E->fy_counts.release();
  E->fy_totals.release();

  E->row_flags.release();
  for (DevBuf<double> *b : {&E->mc_F, &E->mc_G, &E->mc_H, &E->mc_w, &E->mc_part}) b->release();
  E->mc_y.release();
  E->mc_max.release();
  E->mc_out_d.release();
  E->mc_feat_d.release();
  if (E->mc_out_pin) (void)hipHostFree(E->mc_out_pin);
  E->level_args_d.release();
  E->lvl_d.release();
  E->table_d.release();
  if (E->table_pin) (void)hipHostFree(E->table_pin);
  E->pool.release();
  E->part_d.release();
  E->segs.release();
  E->cand.release();
  E->totals.release();
  for (int s = 0; s < 2; ++s) E->parents_d[s].release();
  E->groups_d.release();
  E->tile_begin_d.release();
  E->hist_begin_d.release();
  E->work_flag_d.release();
  E->kept_e_d.release();
  for (auto &b : E->parent_e_d) b.release();
  E->hist_node_d.release();
  E->work_e_d.release();
  E->nleft_d.release();
  E->tiles_d.release();
  E->tile_cnt_d.release();
  E->hist_tasks_d.release();
  E->tree_d.release();
  for (int b = 0; b < 2; ++b) {
    E->round_d[b].release();
    if (E->round_pin[b]) (void)hipHostFree(E->round_pin[b]);
    if (E->rtable_pin[b]) (void)hipHostFree(E->rtable_pin[b]);
    if (E->rslot[b].done) (void)hipEventDestroy(E->rslot[b].done);
  }
  E->offsets_d.release();
  E->partials_d.release();
  E->ktime_d.release();
  E->loss_d.release();
  E->out_d.release();
  E->proba_d.release();
  E->pin.release();
  for (int b = 0; b < 3; ++b) {
    if (E->xfer_pin[b]) (void)hipHostFree(E->xfer_pin[b]);
    if (E->xfer_ev[b]) (void)hipEventDestroy(E->xfer_ev[b]);
  }
  E->xchunk.release();
  E->xchunk2.release();
  E->pcodes.release();
  E->edges_d.release();
  E->nbins_d.release();
  E->nanid_d.release();
  for (hipEvent_t ev : E->pipe_ev)
    if (ev) (void)hipEventDestroy(ev);
  release_staging(E);
  for (hipEvent_t ev : E->ev_pool) (void)hipEventDestroy(ev);
  for (hipEvent_t ev : E->rows_ready)
    if (ev) (void)hipEventDestroy(ev);
  if (E->st_rows) (void)hipStreamDestroy(E->st_rows);
  if (E->st) (void)hipStreamDestroy(E->st);
  delete E;
}

int bsscl_bin_features(bsscl_engine *E, int32_t slot, const void *X,
                       int32_t x_is_f64, int64_t n, int32_t F,
                       const double *edges_2d, int32_t edge_stride,
                       const int32_t *bin_counts, const int32_t *nan_bin_id,
                       uint8_t *codes_out) {
  if (!E || !edges_2d || !bin_counts || !nan_bin_id)
    return set_error(BSSCL_EINVAL, "bin_features: null argument");
  if (slot < 0 || slot > 1) return set_error(BSSCL_EINVAL, "matrix slot must be 0 or 1");
  if (n <= 0 || n > INT32_MAX || F <= 0)
    return set_error(BSSCL_EINVAL, "bin_features: bad shape");
  const bool staged = (X == nullptr);
  if (staged && (!E->xstage.p || E->xs_n != n || E->xs_F != F || E->xs_f64 != (x_is_f64 ? 1 : 0)))
    return set_error(BSSCL_EINVAL,
                     "bin_features: X is NULL but no staged matrix of this shape and dtype");
  int32_t has_any_nan = 0, tiers = 1;
  CHK(bin_layout(F, edge_stride, bin_counts, nan_bin_id, &tiers, &has_any_nan));
  HIPCHK(hipSetDevice(E->device));
  CHK(alloc_matrix(E, slot, n, F, tiers));
  CHK(upload_edges(E, F, edges_2d, edge_stride, bin_counts, nan_bin_id));
  const double *ed = E->edges_d.p;
  const int32_t *nb = E->nbins_d.p, *nid = E->nanid_d.p;
  Matrix &M = E->mat[slot];
  const size_t esz = x_is_f64 ? 8 : 4;
  if (staged) {
    hipError_t e = launch_bin(E->st, E->xstage.p, x_is_f64, n, F, ed, edge_stride, nb, nid,
                              has_any_nan, M.codes.p, M.ld, tiers);
    if (e == hipSuccess) e = hipStreamSynchronize(E->st);
    if (e != hipSuccess)
      return set_error(BSSCL_EDEVICE, std::string("binning: ") + hipGetErrorString(e));
  } else {
    // Stream X through the device in row chunks of at most 512 MB (each
    // chunk's upload then takes the 32 MB pieces of host_upload).
    int64_t chunk = std::max<int64_t>(64, (int64_t)((512u << 20) / (esz * (size_t)F)) / 64 * 64);
    chunk = std::min<int64_t>(chunk, round_up(n, 64));
    // (The chunk buffer stays allocated for the next host matrix.)
    TempBuf<unsigned char> &xd = E->xchunk;
    CHK(xd.ensure((size_t)chunk * F * esz));
    for (int64_t r0 = 0; r0 < n; r0 += chunk) {
      const int64_t rows = std::min(chunk, n - r0);
      CHK(host_upload(E, xd.p, (const unsigned char *)X + (size_t)r0 * F * esz,
                      (size_t)rows * F * esz));
      hipError_t e = launch_bin(E->st, xd.p, x_is_f64, rows, F, ed, edge_stride, nb, nid,
                                has_any_nan, M.codes.p + r0, M.ld, tiers);
      if (e == hipSuccess) e = hipStreamSynchronize(E->st);
      if (e != hipSuccess)
        return set_error(BSSCL_EDEVICE, std::string("binning: ") + hipGetErrorString(e));
    }
  }
  if (slot == 0) CHK(find_hot_bins(E));
  if (codes_out) return bsscl_get_codes(E, slot, codes_out);
  return BSSCL_OK;
}

int bsscl_stage_features(bsscl_engine *E, const void *X, int32_t x_is_f64, int64_t n,
                         int32_t F) {
  if (!E || !X) return set_error(BSSCL_EINVAL, "stage_features: null argument");
  if (n <= 0 || n > INT32_MAX || F <= 0)
    return set_error(BSSCL_EINVAL, "stage_features: bad shape");
  HIPCHK(hipSetDevice(E->device));
  E->cols_sorted = false;
  E->col_m.clear();
  const size_t bytes = (size_t)n * F * (x_is_f64 ? 8 : 4);
  CHK(E->xstage.ensure(bytes));
  E->xs_n = 0;
  CHK(host_upload(E, E->xstage.p, X, bytes));
  E->xs_n = n;
  E->xs_F = F;
  E->xs_f64 = x_is_f64 ? 1 : 0;
  return BSSCL_OK;
}

int bsscl_sort_columns(bsscl_engine *E, int64_t *nan_count, int64_t *n_unique) {
  if (!E || !nan_count || !n_unique) return set_error(BSSCL_EINVAL, "sort_columns: null argument");
  if (!E->xstage.p || E->xs_n <= 0)
    return set_error(BSSCL_EINVAL, "sort_columns: no staged matrix (call bsscl_stage_features)");
  HIPCHK(hipSetDevice(E->device));
  const int64_t n = E->xs_n;
  const int32_t F = E->xs_F;
  const int f64 = E->xs_f64;
  const int64_t ld = col_sort_ld(n, f64);
  const size_t ksz = f64 ? 8 : 4;
  E->cols_sorted = false;
  CHK(E->col_keys.ensure((size_t)F * ld * ksz));
  CHK(E->col_tmp.ensure((size_t)F * ld * ksz));
  CHK(E->col_counts.ensure((size_t)col_sort_count_words(n, F, f64)));
  CHK(E->col_totals.ensure((size_t)F * 256));
  CHK(E->col_m_d.ensure((size_t)F));
  CHK(E->col_changes_d.ensure((size_t)F));
  std::vector<int64_t> m(F);
  std::vector<unsigned long long> changes(F);
  hipError_t e = launch_col_sort(E->st, E->xstage.p, f64, n, F, E->col_keys.p, E->col_tmp.p, ld,
                                 E->col_counts.p, E->col_totals.p, E->col_m_d.p);
  if (e == hipSuccess) e = hipMemsetAsync(E->col_changes_d.p, 0, (size_t)F * 8, E->st);
  if (e == hipSuccess)
    e = launch_col_changes(E->st, E->col_keys.p, f64, ld, F, E->col_m_d.p, n,
                           E->col_changes_d.p);
  if (e == hipSuccess)
    e = hipMemcpyAsync(m.data(), E->col_m_d.p, (size_t)F * 8, hipMemcpyDeviceToHost, E->st);
  if (e == hipSuccess)
    e = hipMemcpyAsync(changes.data(), E->col_changes_d.p, (size_t)F * 8,
                       hipMemcpyDeviceToHost, E->st);
  if (e == hipSuccess) e = hipStreamSynchronize(E->st);
  if (e != hipSuccess)
    return set_error(BSSCL_EDEVICE, std::string("sort_columns: ") + hipGetErrorString(e));
  for (int32_t j = 0; j < F; ++j) {
    if (m[j] < 0 || m[j] > n) return set_error(BSSCL_EINTERNAL, "sort_columns: bad count");
    nan_count[j] = n - m[j];
    n_unique[j] = m[j] > 0 ? 1 + (int64_t)changes[j] : 0;
  }
  E->col_ld = ld;
  E->col_m = m;
  E->cols_sorted = true;
  return BSSCL_OK;
}

int bsscl_sorted_gather(bsscl_engine *E, int64_t count, const int32_t *col, const int64_t *pos,
                        double *out) {
  if (!E || (count > 0 && (!col || !pos || !out)))
    return set_error(BSSCL_EINVAL, "sorted_gather: null argument");
  if (!E->cols_sorted) return set_error(BSSCL_EINVAL, "sorted_gather: columns are not sorted");
  if (count <= 0) return BSSCL_OK;
  for (int64_t k = 0; k < count; ++k) {
    if (col[k] < 0 || col[k] >= E->xs_F || pos[k] < 0 || pos[k] >= E->col_m[col[k]])
      return set_error(BSSCL_EINVAL, "sorted_gather: position outside the column's values");
  }
  HIPCHK(hipSetDevice(E->device));
  CHK(E->gather_c.ensure((size_t)count));
  CHK(E->gather_p.ensure((size_t)count));
  CHK(E->gather_o.ensure((size_t)count));
  hipError_t e =
      hipMemcpyAsync(E->gather_c.p, col, (size_t)count * 4, hipMemcpyHostToDevice, E->st);
  if (e == hipSuccess)
    e = hipMemcpyAsync(E->gather_p.p, pos, (size_t)count * 8, hipMemcpyHostToDevice, E->st);
  if (e == hipSuccess)
    e = launch_col_gather(E->st, E->col_keys.p, E->xs_f64, E->col_ld, count, E->gather_c.p,
                          E->gather_p.p, E->gather_o.p);
  if (e == hipSuccess)
    e = hipMemcpyAsync(out, E->gather_o.p, (size_t)count * 8, hipMemcpyDeviceToHost, E->st);
  if (e == hipSuccess) e = hipStreamSynchronize(E->st);
  if (e != hipSuccess)
    return set_error(BSSCL_EDEVICE, std::string("sorted_gather: ") + hipGetErrorString(e));
  return BSSCL_OK;
}

int bsscl_sorted_uniques(bsscl_engine *E, int32_t col, int32_t max_out, double *out,
                         int32_t *count) {
  if (!E || !count || (max_out > 0 && !out))
    return set_error(BSSCL_EINVAL, "sorted_uniques: null argument");
  if (!E->cols_sorted) return set_error(BSSCL_EINVAL, "sorted_uniques: columns are not sorted");
  if (col < 0 || col >= E->xs_F) return set_error(BSSCL_EINVAL, "sorted_uniques: bad column");
  if (max_out < 0) return set_error(BSSCL_EINVAL, "sorted_uniques: max_out < 0");
  const int64_t m = E->col_m[col];
  *count = 0;
  if (m == 0) return BSSCL_OK;
  HIPCHK(hipSetDevice(E->device));
  ScopedBuf<int64_t> p_d;
  ScopedBuf<unsigned int> cnt_d;
  CHK(p_d.ensure((size_t)std::max(max_out, 1)));
  CHK(cnt_d.ensure(1));
  unsigned int cnt = 0;
  hipError_t e = hipMemsetAsync(cnt_d.p, 0, 4, E->st);
  if (e == hipSuccess)
    e = launch_col_run_starts(E->st, E->col_keys.p, E->xs_f64, E->col_ld, col, m, max_out,
                              p_d.p, cnt_d.p);
  if (e == hipSuccess) e = hipMemcpyAsync(&cnt, cnt_d.p, 4, hipMemcpyDeviceToHost, E->st);
  if (e == hipSuccess) e = hipStreamSynchronize(E->st);
  if (e != hipSuccess)
    return set_error(BSSCL_EDEVICE, std::string("sorted_uniques: ") + hipGetErrorString(e));
  if ((int64_t)cnt > (int64_t)max_out)
    return set_error(BSSCL_EINVAL, "sorted_uniques: the column has more than max_out values");
  std::vector<int64_t> pos(cnt);
  if (cnt) {
    HIPCHK(hipMemcpy(pos.data(), p_d.p, (size_t)cnt * 8, hipMemcpyDeviceToHost));
    std::sort(pos.begin(), pos.end());
    std::vector<int32_t> cols(cnt, col);
    CHK(bsscl_sorted_gather(E, cnt, cols.data(), pos.data(), out));
  }
  *count = (int32_t)cnt;
  return BSSCL_OK;
}

int bsscl_release_staged(bsscl_engine *E) {
  if (!E) return set_error(BSSCL_EINVAL, "release_staged: null engine");
  HIPCHK(hipSetDevice(E->device));
  E->xs_n = 0;
  E->cols_sorted = false;
  E->col_m.clear();
  // (Kept buffers are next written by work on E->st, after what reads them.)
  const size_t held = E->xstage.cap + E->col_keys.cap + E->col_tmp.cap;
  if (held > kStagingKeptBytes) {
    HIPCHK(hipStreamSynchronize(E->st));
    release_staging(E);
  }
  return BSSCL_OK;
}

int bsscl_load_codes(bsscl_engine *E, int32_t slot, const void *codes,
                     int32_t codes_u16, int64_t n, int32_t F) {
  if (!E || !codes) return set_error(BSSCL_EINVAL, "load_codes: null argument");
  if (slot < 0 || slot > 1) return set_error(BSSCL_EINVAL, "matrix slot must be 0 or 1");
  if (n <= 0 || n > INT32_MAX || F <= 0) return set_error(BSSCL_EINVAL, "load_codes: bad shape");
  HIPCHK(hipSetDevice(E->device));
  int32_t tiers = 1;
  if (codes_u16) {
    const uint16_t *c16 = static_cast<const uint16_t *>(codes);
    uint16_t cmax = 0;
    for (int64_t k = 0; k < n * F; ++k) cmax = std::max(cmax, c16[k]);
    tiers = tiers_for_code(cmax);
  }
  CHK(alloc_matrix(E, slot, n, F, tiers));
  const size_t bytes = (size_t)n * F * (codes_u16 ? 2 : 1);
  TempBuf<unsigned char> tmp;
  CHK(tmp.ensure(bytes));
  {
    const int rc = host_upload(E, tmp.p, codes, bytes);
    if (rc != BSSCL_OK) {
      tmp.release();
      return rc;
    }
  }
  hipError_t e = launch_load_codes(E->st, tmp.p, codes_u16, n, F, E->mat[slot].codes.p, E->mat[slot].ld,
                          tiers);
  if (e == hipSuccess) e = hipStreamSynchronize(E->st);
  tmp.release();
  if (e != hipSuccess) return set_error(BSSCL_EDEVICE, std::string("load_codes: ") + hipGetErrorString(e));
  if (slot == 0) CHK(find_hot_bins(E));
  return BSSCL_OK;
}

namespace {
int get_codes(bsscl_engine *E, int32_t slot, void *codes_out, int as_u16) {
  if (!E || !codes_out) return set_error(BSSCL_EINVAL, "get_codes: null argument");
  CHK(check_matrix(E, slot));
  HIPCHK(hipSetDevice(E->device));
  const Matrix &M = E->mat[slot];
  const size_t bytes = (size_t)M.n * M.F * (as_u16 ? 2 : 1);
  TempBuf<uint8_t> tmp;
  CHK(tmp.ensure(bytes));
  hipError_t e = launch_get_codes(E->st, M.codes.p, M.ld, M.n, M.F, M.tiers, tmp.p, as_u16);
  if (e == hipSuccess) e = hipMemcpyAsync(codes_out, tmp.p, bytes, hipMemcpyDeviceToHost, E->st);
  if (e == hipSuccess) e = hipStreamSynchronize(E->st);
  tmp.release();
  if (e != hipSuccess) return set_error(BSSCL_EDEVICE, std::string("get_codes: ") + hipGetErrorString(e));
  return BSSCL_OK;
}
}  // namespace

int bsscl_get_codes(bsscl_engine *E, int32_t slot, uint8_t *codes_out) {
  return get_codes(E, slot, codes_out, 0);
}

int bsscl_get_codes_u16(bsscl_engine *E, int32_t slot, uint16_t *codes_out) {
  return get_codes(E, slot, codes_out, 1);
}

int bsscl_build_tree(bsscl_engine *E, const double *grad, const double *hess,
                     const int64_t *sample_indices, int64_t n_samples,
                     const int32_t *feature_indices, int32_t n_selected,
                     int32_t max_leaves, int32_t max_depth,
                     int32_t min_samples_leaf, double min_child_weight,
                     const int32_t *bin_counts, int32_t max_bins,
                     double reg_lambda, double gamma, int32_t *out_features,
                     int64_t *out_thresholds, double *out_values,
                     int32_t *out_left, int32_t *out_right,
                     int32_t *out_node_count, double *out_split_gains) {
  if (!E || !grad || !hess || !sample_indices)
    return set_error(BSSCL_EINVAL, "build_tree: null argument");
  CHK(check_matrix(E, 0));
  (void)max_bins;
  const Matrix &X = E->mat[0];
  if (n_samples <= 0) return set_error(BSSCL_EINVAL, "build_tree: no samples");
  for (int64_t k = 0; k < n_samples; ++k)
    if (sample_indices[k] < 0 || sample_indices[k] >= X.n)
      return set_error(BSSCL_EINVAL, "build_tree: sample index out of range");
  TreeOut out{out_features, out_thresholds, out_values, out_left, out_right,
              out_node_count, out_split_gains};
  std::vector<int32_t> feats, nb_sel;
  HIPCHK(hipSetDevice(E->device));
  CHK(validate_tree_args(E, feature_indices, n_selected, max_leaves,
                         min_samples_leaf, bin_counts, out, feats, nb_sel));
  CHK(load_grad_hess(E, grad, hess, X.n, n_samples));
  CHK(E->rows64.ensure((size_t)n_samples));
  HIPCHK(hipMemcpyAsync(E->rows64.p, sample_indices, (size_t)n_samples * 8,
                        hipMemcpyHostToDevice, E->st));
  TreeParams tp{max_leaves, max_depth, min_samples_leaf, min_child_weight,
                reg_lambda, gamma};
  E->set_base = 0;
  CHK(build_tree_core(E, nullptr, n_samples, feats, nb_sel, tp, out));
  tree_to_reference(X, out);
  return BSSCL_OK;
}

int bsscl_boost_begin(bsscl_engine *E, const int64_t *y, int64_t n, double w0,
                      double w1, double base_score) {
  if (!E || !y) return set_error(BSSCL_EINVAL, "boost_begin: null argument");
  if (E->ahead >= 0) {
    const int p = E->ahead;
    E->ahead = -1;
    CHK(drain_rounds(E, p));
  }
  CHK(check_matrix(E, 0));
  if (n != E->mat[0].n) return set_error(BSSCL_EINVAL, "boost_begin: y length differs from matrix rows");
  if (!(w0 > 0.0) || !(w1 > 0.0) || !std::isfinite(w0) || !std::isfinite(w1))
    return set_error(BSSCL_EINVAL, "boost_begin: class weights must be positive");
  HIPCHK(hipSetDevice(E->device));
  std::vector<uint8_t> yb((size_t)n);
  uint64_t bad = 0;  // any label outside {0, 1} (one branch-free pass)
  for (int64_t i = 0; i < n; ++i) {
    bad |= (uint64_t)y[i] >> 1;
    yb[(size_t)i] = (uint8_t)y[i];
  }
  if (bad) return set_error(BSSCL_EINVAL, "boost_begin: labels must be 0 or 1");
  CHK(E->y.ensure((size_t)n));
  CHK(E->F.ensure((size_t)n));
  CHK(E->ghq.ensure((size_t)n));
  HIPCHK(hipMemcpyAsync(E->y.p, yb.data(), (size_t)n, hipMemcpyHostToDevice, E->st));
  HIPCHK(launch_fill_f64(E->st, E->F.p, n, base_score));  // F starts at base_score (est:2834)
  // The largest |g| and h of the starting F into slot 0 (an F update with
  // no tree).
  E->gh_ok = false;
  const int nb = update_F_blocks(n);
  CHK(E->ghmax_d.ensure(4));
  CHK(E->partials_d.ensure((size_t)nb));
  HIPCHK(hipMemsetAsync(E->ghmax_d.p, 0, 4 * sizeof(unsigned long long), E->st));
  HIPCHK(launch_update_F(E->st, E->mat[0].codes.p, E->mat[0].ld, n, nullptr, 0, nullptr, 0.0,
                         E->F.p, E->y.p, E->partials_d.p, nb, w0, w1, E->ghmax_d.p, nullptr));
  HIPCHK(hipStreamSynchronize(E->st));
  E->gh_slot = 0;
  E->gh_ok = true;
  E->w0 = w0;
  E->w1 = w1;
  E->boosting = true;
  E->node_cap_floor = 0;  // a new fit starts from the node table its trees' shape asks for
  return BSSCL_OK;
}

int bsscl_boost_round(bsscl_engine *E, bsscl_sampler *sampler,
                      int32_t max_leaves, int32_t max_depth,
                      int32_t min_samples_leaf, double min_child_weight,
                      const int32_t *bin_counts, int32_t max_bins,
                      double reg_lambda, double gamma, double learning_rate,
                      int32_t *out_features, int64_t *out_thresholds,
                      double *out_values, int32_t *out_left,
                      int32_t *out_right, int32_t *out_node_count,
                      double *out_split_gains, double *out_train_loss) {
  if (!E || !sampler) return set_error(BSSCL_EINVAL, "boost_round: null argument");
  if (!E->boosting) return set_error(BSSCL_EINVAL, "boost_round: call boost_begin first");
  (void)max_bins;
  HIPCHK(hipSetDevice(E->device));
  const auto t0 = std::chrono::steady_clock::now();
  RoundArgs a;
  a.max_leaves = max_leaves;
  a.max_depth = max_depth;
  a.min_samples_leaf = min_samples_leaf;
  a.min_child_weight = min_child_weight;
  a.reg_lambda = reg_lambda;
  a.gamma = gamma;
  a.learning_rate = learning_rate;
  a.bin_counts = bin_counts;
  TreeOut out{out_features, out_thresholds, out_values, out_left, out_right,
              out_node_count, out_split_gains};
  if (!out.features || !out.thresholds || !out.values || !out.left || !out.right ||
      !out.node_count || !out.gains)
    return set_error(BSSCL_EINVAL, "boost_round: output arrays missing");
  int cur = E->ahead;
  E->ahead = -1;
  if (cur >= 0) {
    const RoundSlot &p = E->rslot[cur];
    if (p.sampler != sampler || !(p.args == a)) {
      (void)drain_rounds(E, cur);
      return set_error(BSSCL_EINVAL,
                       "boost_round: arguments differ from the round enqueued ahead "
                       "(turn pipelining off to change them between rounds)");
    }
  } else {
    cur = E->rslot_next;
    E->rslot_next ^= 1;
    CHK(enqueue_round(E, sampler, a, cur));
  }
  // Enqueue the next round now, so the GPU works on it while this one is
  // read back and handed to the caller.
  if (E->pipeline && pipeline_safe(E, a, sampler) && sampler_remaining(sampler) > 0) {
    const int nxt = E->rslot_next;
    E->rslot_next ^= 1;
    const auto te = std::chrono::steady_clock::now();
    const int rc = enqueue_round(E, sampler, a, nxt);
    E->stats[14] += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - te).count();
    if (rc != BSSCL_OK) {
      (void)drain_rounds(E, cur);
      return rc;
    }
    E->ahead = nxt;
  }
  const auto tf = std::chrono::steady_clock::now();
  const int rc = finish_round(E, cur, out, out_train_loss);
  E->stats[15] += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - tf).count();
  if (rc != BSSCL_OK) {
    if (E->ahead >= 0) (void)drain_rounds(E, E->ahead);
    E->ahead = -1;
    return rc;
  }
  E->stats[11] += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
  return BSSCL_OK;
}

int bsscl_boost_set_pipeline(bsscl_engine *E, int32_t on) {
  if (!E) return set_error(BSSCL_EINVAL, "null engine");
  HIPCHK(hipSetDevice(E->device));
  if (!on && E->ahead >= 0) {
    const int p = E->ahead;
    E->ahead = -1;
    CHK(drain_rounds(E, p));
  }
  if (!on) mc_drop_next(E);
  E->pipeline = on != 0;
  return BSSCL_OK;
}

// ---------------------------------------------------------------------------
// Multiclass rounds (est:2949-3065) with the scores on the device.
// ---------------------------------------------------------------------------
int bsscl_mc_begin(bsscl_engine *E, const int64_t *y, int64_t n, int32_t n_classes,
                   const double *sample_weight) {
  if (!E || !y || !sample_weight) return set_error(BSSCL_EINVAL, "mc_begin: null argument");
  CHK(check_matrix(E, 0));
  if (n != E->mat[0].n) return set_error(BSSCL_EINVAL, "mc_begin: y length differs from matrix rows");
  if (n_classes < 2 || n_classes > kMcMaxK)
    return set_error(BSSCL_EINVAL, "mc_begin: between 2 and " + std::to_string(kMcMaxK) + " classes");
  if (E->ahead >= 0) {  // a boosting round enqueued ahead shares the row buffers
    const int p = E->ahead;
    E->ahead = -1;
    CHK(drain_rounds(E, p));
  }
  mc_drop_next(E);
  std::vector<int32_t> yi((size_t)n);
  double wmax = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    if (y[i] < 0 || y[i] >= n_classes) return set_error(BSSCL_EINVAL, "mc_begin: label out of range");
    if (!(sample_weight[i] > 0.0) || !std::isfinite(sample_weight[i]))
      return set_error(BSSCL_EINVAL, "mc_begin: sample weights must be positive");
    yi[(size_t)i] = (int32_t)y[i];
    wmax = std::max(wmax, sample_weight[i]);
  }
  HIPCHK(hipSetDevice(E->device));
  const size_t nk = (size_t)n * (size_t)n_classes;
  CHK(E->mc_F.ensure(nk));
  CHK(E->mc_G.ensure(nk));
  CHK(E->mc_H.ensure(nk));
  CHK(E->mc_w.ensure((size_t)n));
  CHK(E->mc_y.ensure((size_t)n));
  CHK(E->mc_max.ensure(2 * (size_t)kMcMaxK));
  CHK(E->mc_part.ensure((size_t)mc_loss_blocks(n)));
  CHK(E->ghq.ensure((size_t)n));
  HIPCHK(hipMemcpyAsync(E->mc_y.p, yi.data(), (size_t)n * 4, hipMemcpyHostToDevice, E->st));
  HIPCHK(hipMemcpyAsync(E->mc_w.p, sample_weight, (size_t)n * 8, hipMemcpyHostToDevice, E->st));
  HIPCHK(hipMemsetAsync(E->mc_F.p, 0, nk * 8, E->st));  // the reference starts from 0 (est:2958)
  HIPCHK(hipStreamSynchronize(E->st));
  E->mc_K = n_classes;
  E->mc_m = 0;
  E->mc_rows32 = nullptr;
  // h = w p (1 - p) <= w / 4, floored at 1e-8 (est:3019).
  E->mc_hbound = std::max(0.25 * wmax, 1e-8);
  E->node_cap_floor = 0;  // a new fit starts from the node table its trees' shape asks for
  return BSSCL_OK;
}

int bsscl_mc_round(bsscl_engine *E, const int64_t *sample_indices, int64_t n_samples) {
  if (!E || !sample_indices) return set_error(BSSCL_EINVAL, "mc_round: null argument");
  if (E->mc_K < 2) return set_error(BSSCL_EINVAL, "mc_round: no multiclass run");
  CHK(check_matrix(E, 0));
  const int64_t n = E->mat[0].n;
  if (n_samples <= 0) return set_error(BSSCL_EINVAL, "mc_round: no samples");
  for (int64_t k = 0; k < n_samples; ++k)
    if (sample_indices[k] < 0 || sample_indices[k] >= n)
      return set_error(BSSCL_EINVAL, "mc_round: sample index out of range");
  HIPCHK(hipSetDevice(E->device));
  mc_drop_next(E);
  E->mc_m = 0;
  CHK(E->rows64.ensure((size_t)n_samples));
  HIPCHK(hipMemcpyAsync(E->rows64.p, sample_indices, (size_t)n_samples * 8,
                        hipMemcpyHostToDevice, E->st));
  E->mc_rows32 = nullptr;
  return mc_gradients(E, n_samples);
}

int bsscl_mc_round_sampled(bsscl_engine *E, bsscl_sampler *sampler, int32_t *feats_out) {
  if (!E || !sampler) return set_error(BSSCL_EINVAL, "mc_round_sampled: null argument");
  if (E->mc_K < 2) return set_error(BSSCL_EINVAL, "mc_round_sampled: no multiclass run");
  CHK(check_matrix(E, 0));
  const SamplerShape sh = sampler_shape(sampler);
  if (sh.n != E->mat[0].n)
    return set_error(BSSCL_EINVAL, "mc_round_sampled: sampler rows differ from matrix rows");
  HIPCHK(hipSetDevice(E->device));
  E->mc_m = 0;
  mc_drop_next(E);  // (a round taken ahead by bsscl_mc_round_trees goes back)
  SamplerRound sr;
  void *token = nullptr;
  CHK(sampler_take(sampler, &sr, &token));
  int rc = mc_rows_from_sampler(E, sampler, sh, sr, 0, E->st);
  if (rc == BSSCL_OK) E->mc_rows32 = E->round_rows[0].p;
  if (rc == BSSCL_OK && feats_out) std::memcpy(feats_out, sr.feats, (size_t)sh.f_sub * 4);
  if (rc == BSSCL_OK) rc = mc_gradients(E, sh.n_sub);  // (ends with a synchronisation)
  if (rc != BSSCL_OK) {
    (void)hipStreamSynchronize(E->st);
    E->mc_m = 0;
  }
  sampler_give_back(sampler, token);
  return rc;
}

int bsscl_mc_build_tree(bsscl_engine *E, int32_t k, const int32_t *feature_indices,
                        int32_t n_selected, int32_t max_leaves, int32_t max_depth,
                        int32_t min_samples_leaf, double min_child_weight,
                        const int32_t *bin_counts, int32_t max_bins, double reg_lambda,
                        double gamma, double learning_rate, int32_t *out_features,
                        int64_t *out_thresholds, double *out_values, int32_t *out_left,
                        int32_t *out_right, int32_t *out_node_count, double *out_split_gains) {
  if (!E) return set_error(BSSCL_EINVAL, "mc_build_tree: null argument");
  if (E->mc_K < 2 || E->mc_m <= 0) return set_error(BSSCL_EINVAL, "mc_build_tree: no round");
  if (k < 0 || k >= E->mc_K) return set_error(BSSCL_EINVAL, "mc_build_tree: class out of range");
  CHK(check_matrix(E, 0));
  (void)max_bins;
  TreeOut out{out_features, out_thresholds, out_values, out_left, out_right,
              out_node_count, out_split_gains};
  std::vector<int32_t> feats, nb_sel;
  HIPCHK(hipSetDevice(E->device));
  CHK(validate_tree_args(E, feature_indices, n_selected, max_leaves,
                         min_samples_leaf, bin_counts, out, feats, nb_sel));
  const TreeParams tp{max_leaves, max_depth, min_samples_leaf, min_child_weight, reg_lambda,
                      gamma};
  return mc_tree_host(E, k, feats, nb_sel, tp, learning_rate, out);
}

int bsscl_mc_build_trees(bsscl_engine *E, const int32_t *feature_indices, int32_t n_selected,
                         int32_t max_leaves, int32_t max_depth, int32_t min_samples_leaf,
                         double min_child_weight, const int32_t *bin_counts, int32_t max_bins,
                         double reg_lambda, double gamma, double learning_rate,
                         int32_t *out_features, int64_t *out_thresholds, double *out_values,
                         int32_t *out_left, int32_t *out_right, int32_t *out_node_count,
                         double *out_split_gains) {
  if (!E) return set_error(BSSCL_EINVAL, "mc_build_trees: null argument");
  if (E->mc_K < 2 || E->mc_m <= 0) return set_error(BSSCL_EINVAL, "mc_build_trees: no round");
  CHK(check_matrix(E, 0));
  (void)max_bins;
  TreeOut out0{out_features, out_thresholds, out_values, out_left, out_right,
               out_node_count, out_split_gains};
  std::vector<int32_t> feats, nb_sel;
  HIPCHK(hipSetDevice(E->device));
  CHK(validate_tree_args(E, feature_indices, n_selected, max_leaves,
                         min_samples_leaf, bin_counts, out0, feats, nb_sel));
  const TreeParams tp{max_leaves, max_depth, min_samples_leaf, min_child_weight, reg_lambda,
                      gamma};
  const size_t M = 2 * (size_t)max_leaves + 2;
  auto out = [&](int32_t k) {
    const size_t o = (size_t)k * M;
    return TreeOut{out_features + o, out_thresholds + o, out_values + o, out_left + o,
                   out_right + o, out_node_count + k, out_split_gains + o};
  };
  if (device_replay_fits(max_leaves))
    return mc_trees_device(E, feats, nb_sel, tp, learning_rate, out);
  for (int32_t k = 0; k < E->mc_K; ++k) {
    TreeOut o = out(k);
    CHK(mc_tree_host(E, k, feats, nb_sel, tp, learning_rate, o));
  }
  return BSSCL_OK;
}

int bsscl_mc_round_trees(bsscl_engine *E, bsscl_sampler *sampler, int32_t *feats_out,
                         int32_t max_leaves, int32_t max_depth, int32_t min_samples_leaf,
                         double min_child_weight, const int32_t *bin_counts, int32_t max_bins,
                         double reg_lambda, double gamma, double learning_rate,
                         int32_t *out_features, int64_t *out_thresholds, double *out_values,
                         int32_t *out_left, int32_t *out_right, int32_t *out_node_count,
                         double *out_split_gains, double *out_loss) {
  if (!E || !sampler || !out_loss) return set_error(BSSCL_EINVAL, "mc_round_trees: null argument");
  if (E->mc_K < 2) return set_error(BSSCL_EINVAL, "mc_round_trees: no multiclass run");
  CHK(check_matrix(E, 0));
  const SamplerShape sh = sampler_shape(sampler);
  if (sh.n != E->mat[0].n)
    return set_error(BSSCL_EINVAL, "mc_round_trees: sampler rows differ from matrix rows");
  HIPCHK(hipSetDevice(E->device));
  if (E->mc_next && E->mc_next_sampler != sampler) mc_drop_next(E);
  E->mc_m = 0;
  // This round's rows: made on the rows stream by the previous call, or now.
  int slot = E->mc_slot;
  void *token = nullptr;
  std::vector<int32_t> feats_sel;
  int rc = BSSCL_OK;
  if (!E->mc_next_ev) HIPCHK(hipEventCreateWithFlags(&E->mc_next_ev, hipEventDisableTiming));
  if (E->mc_next) {
    slot = E->mc_next_slot;
    token = E->mc_next_token;
    feats_sel.swap(E->mc_next_feats);
    E->mc_next = false;
    E->mc_next_token = nullptr;
  } else {
    SamplerRound sr;
    CHK(sampler_take(sampler, &sr, &token));
    feats_sel.assign(sr.feats, sr.feats + sh.f_sub);
    rc = mc_rows_from_sampler(E, sampler, sh, sr, slot, E->st_rows);
    if (rc == BSSCL_OK && hipEventRecord(E->mc_next_ev, E->st_rows) != hipSuccess)
      rc = set_error(BSSCL_EDEVICE, "mc_round_trees: event record failed");
  }
  auto release = [&](int code) {
    (void)hipStreamSynchronize(E->st_rows);
    (void)hipStreamSynchronize(E->st);
    if (token) sampler_give_back(sampler, token);
    E->mc_m = 0;
    return code;
  };
  if (rc != BSSCL_OK) return release(rc);
  // The trees read the round's rows after the rows stream has made them.
  if (hipStreamWaitEvent(E->st, E->mc_next_ev, 0) != hipSuccess)
    return release(set_error(BSSCL_EDEVICE, "mc_round_trees: stream wait failed"));
  E->mc_rows32 = E->round_rows[slot].p;
  E->mc_slot = slot ^ 1;
  // The next round's rows on the rows stream, beside this round's
  // gradients and trees (they touch the permutation, the row flags and the
  // other slot's rows only).
  if (sampler_remaining(sampler) > 0) {
    SamplerRound sr2;
    void *token2 = nullptr;
    rc = sampler_take(sampler, &sr2, &token2);
    if (rc == BSSCL_OK) {
      rc = mc_rows_from_sampler(E, sampler, sh, sr2, slot ^ 1, E->st_rows);
      if (rc == BSSCL_OK && hipEventRecord(E->mc_next_ev, E->st_rows) != hipSuccess)
        rc = set_error(BSSCL_EDEVICE, "mc_round_trees: event record failed");
      if (rc == BSSCL_OK) {
        E->mc_next = true;
        E->mc_next_slot = slot ^ 1;
        E->mc_next_token = token2;
        E->mc_next_sampler = sampler;
        E->mc_next_feats.assign(sr2.feats, sr2.feats + sh.f_sub);
      } else {
        (void)hipStreamSynchronize(E->st_rows);
        sampler_give_back(sampler, token2);
      }
    }
    if (rc != BSSCL_OK) return release(rc);
  }
  // Gradients from the scores at the round's start (after the last round's
  // updates on the same stream), their maxima left on the device for the
  // trees' scales; then the trees, read back once.
  rc = mc_gradients(E, sh.n_sub, false);
  if (rc != BSSCL_OK) return release(rc);
  if (feats_out) std::memcpy(feats_out, feats_sel.data(), feats_sel.size() * 4);
  rc = bsscl_mc_build_trees(E, feats_sel.data(), (int32_t)feats_sel.size(), max_leaves, max_depth,
                            min_samples_leaf, min_child_weight, bin_counts, max_bins, reg_lambda,
                            gamma, learning_rate, out_features, out_thresholds, out_values,
                            out_left, out_right, out_node_count, out_split_gains);
  if (rc != BSSCL_OK) return release(rc);
  // (The readback waited for the trees, which waited for this round's rows:
  // its sampler round goes back.)
  sampler_give_back(sampler, token);
  token = nullptr;
  rc = bsscl_mc_loss(E, out_loss);
  if (rc != BSSCL_OK) return release(rc);
  return BSSCL_OK;
}

int bsscl_mc_loss(bsscl_engine *E, double *out_loss) {
  if (!E || !out_loss) return set_error(BSSCL_EINVAL, "mc_loss: null argument");
  if (E->mc_K < 2) return set_error(BSSCL_EINVAL, "mc_loss: no multiclass run");
  HIPCHK(hipSetDevice(E->device));
  const int64_t n = E->mat[0].n, nb = mc_loss_blocks(n);
  HIPCHK(launch_mc_loss(E->st, E->mc_F.p, E->mc_y.p, n, E->mc_K, E->mc_part.p));
  std::vector<double> part((size_t)nb);
  HIPCHK(hipMemcpyAsync(part.data(), E->mc_part.p, (size_t)nb * 8, hipMemcpyDeviceToHost, E->st));
  HIPCHK(hipStreamSynchronize(E->st));
  double acc = 0.0;
  for (double v : part) acc += v;
  *out_loss = -(acc / (double)n);
  return BSSCL_OK;
}

int bsscl_mc_get_scores(bsscl_engine *E, double *out) {
  if (!E || !out) return set_error(BSSCL_EINVAL, "mc_get_scores: null argument");
  if (E->mc_K < 2) return set_error(BSSCL_EINVAL, "mc_get_scores: no multiclass run");
  HIPCHK(hipSetDevice(E->device));
  const size_t nk = (size_t)E->mat[0].n * (size_t)E->mc_K;
  HIPCHK(hipMemcpyAsync(out, E->mc_F.p, nk * 8, hipMemcpyDeviceToHost, E->st));
  HIPCHK(hipStreamSynchronize(E->st));
  return BSSCL_OK;
}

int bsscl_mc_get_grad_hess(bsscl_engine *E, double *grad_out, double *hess_out) {
  if (!E || !grad_out || !hess_out) return set_error(BSSCL_EINVAL, "mc_get_grad_hess: null argument");
  if (E->mc_K < 2 || E->mc_m <= 0) return set_error(BSSCL_EINVAL, "mc_get_grad_hess: no round");
  HIPCHK(hipSetDevice(E->device));
  const size_t nk = (size_t)E->mat[0].n * (size_t)E->mc_K;
  HIPCHK(hipMemcpyAsync(grad_out, E->mc_G.p, nk * 8, hipMemcpyDeviceToHost, E->st));
  HIPCHK(hipMemcpyAsync(hess_out, E->mc_H.p, nk * 8, hipMemcpyDeviceToHost, E->st));
  HIPCHK(hipStreamSynchronize(E->st));
  return BSSCL_OK;
}

int bsscl_boost_get_F(bsscl_engine *E, double *F_out) {
  if (!E || !F_out) return set_error(BSSCL_EINVAL, "boost_get_F: null argument");
  if (!E->boosting) return set_error(BSSCL_EINVAL, "boost_get_F: no boosting run");
  HIPCHK(hipSetDevice(E->device));
  HIPCHK(hipMemcpyAsync(F_out, E->F.p, (size_t)E->mat[0].n * 8, hipMemcpyDeviceToHost, E->st));
  HIPCHK(hipStreamSynchronize(E->st));
  return BSSCL_OK;
}

int bsscl_boost_grad_hess_max(bsscl_engine *E, double *out) {
  if (!E || !out) return set_error(BSSCL_EINVAL, "boost_grad_hess_max: null argument");
  if (!E->boosting) return set_error(BSSCL_EINVAL, "boost_grad_hess_max: no boosting run");
  if (!E->gh_ok) return set_error(BSSCL_EINVAL, "boost_grad_hess_max: no maxima on the device");
  HIPCHK(hipSetDevice(E->device));
  unsigned long long bits[2];
  HIPCHK(hipMemcpyAsync(bits, E->ghmax_d.p + 2 * E->gh_slot, sizeof(bits), hipMemcpyDeviceToHost,
                        E->st));
  HIPCHK(hipStreamSynchronize(E->st));
  std::memcpy(out, bits, sizeof(bits));
  return BSSCL_OK;
}

int bsscl_boost_grad_hess(bsscl_engine *E, double *grad_out, double *hess_out) {
  if (!E || !grad_out || !hess_out) return set_error(BSSCL_EINVAL, "boost_grad_hess: null argument");
  if (!E->boosting) return set_error(BSSCL_EINVAL, "boost_grad_hess: no boosting run");
  HIPCHK(hipSetDevice(E->device));
  const int64_t n = E->mat[0].n;
  CHK(E->g64.ensure((size_t)n));
  CHK(E->h64.ensure((size_t)n));
  HIPCHK(launch_grad_hess_f64(E->st, E->F.p, E->y.p, n, E->w0, E->w1, E->g64.p, E->h64.p));
  HIPCHK(hipMemcpyAsync(grad_out, E->g64.p, (size_t)n * 8, hipMemcpyDeviceToHost, E->st));
  HIPCHK(hipMemcpyAsync(hess_out, E->h64.p, (size_t)n * 8, hipMemcpyDeviceToHost, E->st));
  HIPCHK(hipStreamSynchronize(E->st));
  return BSSCL_OK;
}

int bsscl_predict(bsscl_engine *E, int32_t slot, const int16_t *features,
                  const int64_t *thresholds, const double *values,
                  const int32_t *left, const int32_t *right,
                  const int32_t *offsets, int32_t n_trees,
                  double learning_rate, double *out_F) {
  if (!out_F) return set_error(BSSCL_EINVAL, "predict: null argument");
  CHK(predict_to_device(E, slot, features, thresholds, values, left, right, offsets, n_trees,
                        learning_rate));
  CHK(host_download(E, out_F, E->out_d.p, (size_t)E->mat[slot].n * 8));
  CHK(sync(E));
  return BSSCL_OK;
}

int bsscl_predict_proba(bsscl_engine *E, int32_t slot, const int16_t *features,
                        const int64_t *thresholds, const double *values,
                        const int32_t *left, const int32_t *right,
                        const int32_t *offsets, int32_t n_trees, double learning_rate,
                        double base_score, double *out_proba) {
  if (!out_proba) return set_error(BSSCL_EINVAL, "predict_proba: null argument");
  CHK(predict_to_device(E, slot, features, thresholds, values, left, right, offsets, n_trees,
                        learning_rate));
  const int64_t n = E->mat[slot].n;
  CHK(E->proba_d.ensure(2 * (size_t)n));
  HIPCHK(launch_binary_proba(E->st, E->out_d.p, n, base_score, E->proba_d.p));
  CHK(host_download(E, out_proba, E->proba_d.p, (size_t)n * 16));
  CHK(sync(E));
  return BSSCL_OK;
}

int bsscl_predict_proba_rows(bsscl_engine *E, const void *X, int32_t x_is_f64, int64_t n,
                             int32_t F, const double *edges_2d, int32_t edge_stride,
                             const int32_t *bin_counts, const int32_t *nan_bin_id,
                             const int16_t *features, const int64_t *thresholds,
                             const double *values, const int32_t *left, const int32_t *right,
                             const int32_t *offsets, int32_t n_trees, double learning_rate,
                             double base_score, double *out_proba) {
  if (!E || !X || !edges_2d || !bin_counts || !nan_bin_id || !out_proba ||
      (n_trees > 0 && (!features || !thresholds || !values || !left || !right || !offsets)))
    return set_error(BSSCL_EINVAL, "predict_proba_rows: null argument");
  if (n <= 0 || n > INT32_MAX || F <= 0)
    return set_error(BSSCL_EINVAL, "predict_proba_rows: bad shape");
  if (n_trees < 0) return set_error(BSSCL_EINVAL, "predict_proba_rows: negative tree count");
  int32_t tiers = 1, has_any_nan = 0;
  CHK(bin_layout(F, edge_stride, bin_counts, nan_bin_id, &tiers, &has_any_nan));
  HIPCHK(hipSetDevice(E->device));
  const size_t esz = x_is_f64 ? 8 : 4;
  // Rows per chunk: about 256 MB of X, in whole blocks of the walk (512
  // rows).  The walk hides its LDS latency only with many blocks per CU:
  // 1M x 28 in eighths took 1.46 ms of walk against 0.36 ms in one launch,
  // and 10M x 50 in 9 chunks 33 ms against 30 ms in 8.  (Test hook
  // BSSCL_TEST_PREDICT_CHUNK_ROWS: another count.)
  int64_t rows_c = (int64_t)((256u << 20) / (esz * (size_t)F));
  if (const char *t = std::getenv("BSSCL_TEST_PREDICT_CHUNK_ROWS"))
    rows_c = std::strtoll(t, nullptr, 10);
  rows_c = std::min<int64_t>(std::max<int64_t>(512, rows_c / 512 * 512), round_up(n, 512));
  // One chunk's codes, in the layout of a matrix of rows_c rows.
  Matrix view;
  view.n = rows_c;
  view.ld = round_up(rows_c + 8, 256);
  view.F = F;
  view.tiers = tiers;
  CHK(E->pcodes.ensure((size_t)view.ld * view.cols()));
  bool staged = false;
  int32_t n_chunks = 0;
  CHK(upload_trees(E, view, features, thresholds, values, left, right, offsets, n_trees, &staged,
                   &n_chunks));
  CHK(upload_edges(E, F, edges_2d, edge_stride, bin_counts, nan_bin_id));
  CHK(E->out_d.ensure((size_t)n));
  CHK(E->proba_d.ensure(2 * (size_t)n));
  const bool one_chunk = n <= rows_c;
  const size_t xbytes = (size_t)rows_c * F * esz;
  CHK(E->xchunk.ensure(xbytes));
  if (!one_chunk) CHK(E->xchunk2.ensure(xbytes));
  for (hipEvent_t &ev : E->pipe_ev)
    if (!ev) HIPCHK(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
  // Chunk c goes up on the rows stream into buffer c % 2 (after the binning
  // of chunk c - 2 has read it); the engine's stream bins it, walks it and
  // turns its F into probabilities, while chunk c + 1 goes up.  (A single
  // chunk goes up on the engine's stream, with nothing to overlap.)
  hipStream_t up = one_chunk ? E->st : E->st_rows;
  const size_t piece = xfer_chunk((size_t)n * F * esz);
  const unsigned char *xs = static_cast<const unsigned char *>(X);
  std::vector<hipEvent_t> done;  // chunk c's probabilities are written
  int rc = BSSCL_OK;
  int c = 0;
  for (int64_t r0 = 0; r0 < n && rc == BSSCL_OK; r0 += rows_c, ++c) {
    const int64_t rows = std::min(rows_c, n - r0);
    const int b = c & 1;
    unsigned char *xb = b ? E->xchunk2.p : E->xchunk.p;
    hipError_t e = hipSuccess;
    if (c >= 2) e = hipStreamWaitEvent(up, E->pipe_ev[2 + b], 0);
    if (e == hipSuccess) {
      rc = host_upload_async(E, up, xb, xs + (size_t)r0 * F * esz, (size_t)rows * F * esz, piece);
      if (rc != BSSCL_OK) break;
      if (!one_chunk) e = hipEventRecord(E->pipe_ev[b], up);
    }
    if (e == hipSuccess && !one_chunk) e = hipStreamWaitEvent(E->st, E->pipe_ev[b], 0);
    if (e == hipSuccess)
      e = launch_bin(E->st, xb, x_is_f64, rows, F, E->edges_d.p, edge_stride, E->nbins_d.p,
                     E->nanid_d.p, has_any_nan, E->pcodes.p, view.ld, tiers);
    if (e == hipSuccess && !one_chunk) e = hipEventRecord(E->pipe_ev[2 + b], E->st);
    hipEvent_t start = nullptr, stop = nullptr;
    if (e == hipSuccess) {
      rc = prof_kernel(E, 4, &start, &stop);
      if (rc != BSSCL_OK) break;
    }
    if (e == hipSuccess)
      e = launch_predict(E->st, E->pcodes.p, view.ld, rows, view.cols(), E->tree_d.p,
                         E->offsets_d.p, n_trees, staged ? E->offsets_d.p + n_trees + 1 : nullptr,
                         n_chunks, learning_rate, E->out_d.p + r0, start, stop);
    if (e == hipSuccess)
      e = launch_binary_proba(E->st, E->out_d.p + r0, rows, base_score, E->proba_d.p + 2 * r0);
    if (e == hipSuccess && !one_chunk) {
      hipEvent_t ev = nullptr;
      e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
      if (e == hipSuccess) {
        done.push_back(ev);
        e = hipEventRecord(ev, E->st);
      }
    }
    if (e != hipSuccess)
      rc = set_error(BSSCL_EDEVICE, std::string("predict_proba_rows: ") + hipGetErrorString(e));
  }
  // The probabilities come back chunk by chunk on the rows stream, each as
  // soon as its chunk is done, while the device works on the later chunks.
  if (rc == BSSCL_OK && one_chunk) rc = host_download(E, out_proba, E->proba_d.p, (size_t)n * 16);
  for (size_t k = 0; rc == BSSCL_OK && k < done.size(); ++k) {
    const int64_t r0 = (int64_t)k * rows_c, rows = std::min(rows_c, n - r0);
    if (hipStreamWaitEvent(E->st_rows, done[k], 0) != hipSuccess) {
      rc = set_error(BSSCL_EDEVICE, "predict_proba_rows: stream wait failed");
      break;
    }
    rc = host_download_on(E, E->st_rows, out_proba + 2 * r0, E->proba_d.p + 2 * r0,
                          (size_t)rows * 16);
  }
  // (Both streams drain before the buffers can be used again, on every path.)
  (void)hipStreamSynchronize(E->st_rows);
  (void)hipStreamSynchronize(E->st);
  for (hipEvent_t ev : done) (void)hipEventDestroy(ev);
  if (rc != BSSCL_OK) return rc;
  CHK(sync(E));
  return BSSCL_OK;
}

int bsscl_predict_proba_mc(bsscl_engine *E, int32_t slot, int32_t K,
                           const int16_t *const *features, const int64_t *const *thresholds,
                           const double *const *values, const int32_t *const *left,
                           const int32_t *const *right, const int32_t *const *offsets,
                           const int32_t *n_trees, double learning_rate, double *out_proba) {
  if (!E || !out_proba || !n_trees || !features || !thresholds || !values || !left || !right ||
      !offsets)
    return set_error(BSSCL_EINVAL, "predict_proba_mc: null argument");
  if (K < 2 || K > kMcMaxK)
    return set_error(BSSCL_EINVAL, "predict_proba_mc: K must be in [2, " +
                                       std::to_string(kMcMaxK) + "]");
  CHK(check_matrix(E, slot));
  int32_t max_total = 1, max_trees = 0;
  for (int32_t k = 0; k < K; ++k) {
    if (n_trees[k] < 0) return set_error(BSSCL_EINVAL, "predict_proba_mc: negative tree count");
    if (n_trees[k] > 0 && (!features[k] || !thresholds[k] || !values[k] || !left[k] ||
                           !right[k] || !offsets[k]))
      return set_error(BSSCL_EINVAL, "predict_proba_mc: null tree array");
    if (n_trees[k] > 0) max_total = std::max(max_total, offsets[k][n_trees[k]]);
    max_trees = std::max(max_trees, n_trees[k]);
  }
  HIPCHK(hipSetDevice(E->device));
  const Matrix &M = E->mat[slot];
  const int64_t n = M.n;
  // Every class's trees fit the tree buffers, so that no class's upload
  // reallocates them under the walk of the class before.
  CHK(E->tree_d.ensure((size_t)max_total));
  CHK(E->offsets_d.ensure(2 * ((size_t)max_trees + 1)));
  CHK(E->out_d.ensure((size_t)K * n));
  CHK(E->proba_d.ensure((size_t)K * n));
  // F[k] accumulated tree by tree from 0.0 (est:3293-3315), one walk per
  // class, then the softmax of each row and one readback.
  for (int32_t k = 0; k < K; ++k) {
    bool staged = false;
    int32_t n_chunks = 0;
    CHK(upload_trees(E, M, features[k], thresholds[k], values[k], left[k], right[k], offsets[k],
                     n_trees[k], &staged, &n_chunks));
    hipEvent_t start, stop;
    CHK(prof_kernel(E, 4, &start, &stop));
    HIPCHK(launch_predict(E->st, M.codes.p, M.ld, n, M.cols(), E->tree_d.p, E->offsets_d.p,
                          n_trees[k], staged ? E->offsets_d.p + n_trees[k] + 1 : nullptr,
                          n_chunks, learning_rate, E->out_d.p + (size_t)k * n, start, stop));
  }
  HIPCHK(launch_mc_softmax(E->st, E->out_d.p, n, K, E->proba_d.p));
  CHK(host_download(E, out_proba, E->proba_d.p, (size_t)n * K * 8));
  CHK(sync(E));
  return BSSCL_OK;
}

int bsscl_predict_noalloc(bsscl_engine *E, int32_t slot, const int16_t *features,
                          const int64_t *thresholds, const double *values,
                          const int32_t *left, const int32_t *right,
                          const int32_t *offsets, int32_t n_trees,
                          double learning_rate, double *out_F_dev) {
  if (!E || !out_F_dev ||
      (n_trees > 0 && (!features || !thresholds || !values || !left || !right || !offsets)))
    return set_error(BSSCL_EINVAL, "predict_noalloc: null argument");
  CHK(check_matrix(E, slot));
  if (n_trees < 0) return set_error(BSSCL_EINVAL, "predict_noalloc: negative tree count");
  if (n_trees > kNoAllocMaxTrees)
    return set_error(BSSCL_EINVAL, "predict_noalloc: " + std::to_string(n_trees) +
                                       " trees exceed the fixed scratch (at most " +
                                       std::to_string(kNoAllocMaxTrees) + ")");
  const Matrix &M = E->mat[slot];
  const int32_t total = n_trees > 0 ? offsets[n_trees] : 0;
  if (n_trees > 0 && offsets[0] != 0) return set_error(BSSCL_EINVAL, "predict_noalloc: bad offsets");
  if (total > kNoAllocMaxNodes)
    return set_error(BSSCL_EINVAL, "predict_noalloc: " + std::to_string(total) +
                                       " nodes exceed the fixed scratch (at most " +
                                       std::to_string(kNoAllocMaxNodes) + ")");
  // The same checks as bsscl_predict: every traversal stays in its tree.
  bool adjacent = true;  // every right child is its left child + 1
  for (int32_t t = 0; t < n_trees; ++t) {
    const int32_t a = offsets[t], b = offsets[t + 1];
    if (a < 0 || b <= a || b > total) return set_error(BSSCL_EINVAL, "predict_noalloc: bad offsets");
    for (int32_t i = a; i < b; ++i) {
      if (features[i] < 0) continue;
      const int32_t l = left[i], r = right[i];
      if (features[i] >= M.F || l < 0 || r < 0 || l >= b - a || r >= b - a || l <= i - a ||
          r <= i - a)
        return set_error(BSSCL_EINVAL, "predict_noalloc: malformed tree " + std::to_string(t));
      adjacent = adjacent && r == l + 1;
    }
  }
  HIPCHK(hipSetDevice(E->device));
  hipPointerAttribute_t attr;
  if (hipPointerGetAttributes(&attr, out_F_dev) != hipSuccess ||
      attr.type != hipMemoryTypeDevice || attr.device != E->device) {
    (void)hipGetLastError();
    return set_error(BSSCL_EINVAL, "predict_noalloc: out_F_dev is not device memory of GPU " +
                                       std::to_string(E->device));
  }
  unsigned char *S = E->scratch_p;
  if (!S) return set_error(BSSCL_EINTERNAL, "predict_noalloc: scratch address missing");
  TreeNodeDev *nodes = reinterpret_cast<TreeNodeDev *>(S + kScrNodes);
  int32_t *offs = reinterpret_cast<int32_t *>(S + kScrOffs);
  if (total > 0) {
    const size_t nt = (size_t)total;
    HIPCHK(hipMemcpyAsync(S + kScrFeat, features, nt * 2, hipMemcpyHostToDevice, E->st));
    HIPCHK(hipMemcpyAsync(S + kScrThr, thresholds, nt * 8, hipMemcpyHostToDevice, E->st));
    HIPCHK(hipMemcpyAsync(S + kScrVal, values, nt * 8, hipMemcpyHostToDevice, E->st));
    HIPCHK(hipMemcpyAsync(S + kScrLeft, left, nt * 4, hipMemcpyHostToDevice, E->st));
    HIPCHK(hipMemcpyAsync(S + kScrRight, right, nt * 4, hipMemcpyHostToDevice, E->st));
    HIPCHK(hipMemcpyAsync(offs, offsets, ((size_t)n_trees + 1) * 4, hipMemcpyHostToDevice,
                          E->st));
    HIPCHK(launch_pack_trees(E->st, reinterpret_cast<const int16_t *>(S + kScrFeat),
                             reinterpret_cast<const int64_t *>(S + kScrThr),
                             reinterpret_cast<const double *>(S + kScrVal),
                             reinterpret_cast<const int32_t *>(S + kScrLeft),
                             reinterpret_cast<const int32_t *>(S + kScrRight), total,
                             M.F, M.tiers, nodes));
  }
  // The LDS-staged kernel's runs of whole trees (host list on the stack; the
  // copy has finished when the call returns).
  int32_t max_nodes = 0;
  for (int32_t t = 0; t < n_trees; ++t) max_nodes = std::max(max_nodes, offsets[t + 1] - offsets[t]);
  const bool staged = n_trees > 0 && predict_staged_ok(M.cols(), max_nodes, adjacent) &&
                      !std::getenv("BSSCL_TEST_PREDICT_GLOBAL");
  int32_t n_chunks = 0;
  int32_t *chunks_d = reinterpret_cast<int32_t *>(S + kScrChunks);
  if (staged) {
    std::array<int32_t, kNoAllocMaxTrees + 1> chunks;
    n_chunks = predict_chunks(offsets, n_trees, chunks.data());
    HIPCHK(hipMemcpyAsync(chunks_d, chunks.data(), ((size_t)n_chunks + 1) * 4,
                          hipMemcpyHostToDevice, E->st));
    HIPCHK(launch_predict(E->st, M.codes.p, M.ld, M.n, M.cols(), nodes, offs, n_trees, chunks_d,
                          n_chunks, learning_rate, out_F_dev));
    HIPCHK(hipStreamSynchronize(E->st));
    return BSSCL_OK;
  }
  HIPCHK(launch_predict(E->st, M.codes.p, M.ld, M.n, M.cols(), nodes, offs, n_trees, nullptr, 0,
                        learning_rate, out_F_dev));
  HIPCHK(hipStreamSynchronize(E->st));
  return BSSCL_OK;
}

int bsscl_predict_tree(bsscl_engine *E, int32_t slot, const int32_t *features,
                       const int64_t *thresholds, const double *values,
                       const int32_t *left, const int32_t *right,
                       int32_t node_count, double *out) {
  if (!E || !features || !thresholds || !values || !left || !right || !out)
    return set_error(BSSCL_EINVAL, "predict_tree: null argument");
  CHK(check_matrix(E, slot));
  HIPCHK(hipSetDevice(E->device));
  const Matrix &M = E->mat[slot];
  if (node_count <= 0) return set_error(BSSCL_EINVAL, "empty tree");
  std::vector<int32_t> f(features, features + node_count);
  std::vector<int64_t> t(thresholds, thresholds + node_count);
  for (int32_t i = 0; i < node_count; ++i) {
    if (f[(size_t)i] >= M.F) return set_error(BSSCL_EINVAL, "malformed tree node " + std::to_string(i));
    split_to_engine(M, f[(size_t)i], t[(size_t)i]);
  }
  CHK(upload_tree(E, f.data(), t.data(), values, left, right, node_count, M.cols()));
  CHK(E->out_d.ensure((size_t)M.n));
  HIPCHK(launch_predict_tree(E->st, M.codes.p, M.ld, M.n, E->tree_d.p, node_count, E->out_d.p));
  CHK(host_download(E, out, E->out_d.p, (size_t)M.n * 8));
  CHK(sync(E));
  return BSSCL_OK;
}

int bsscl_node_split(bsscl_engine *E, const double *grad, const double *hess,
                     const int64_t *rows, int64_t m,
                     const int32_t *feature_indices, int32_t n_selected,
                     const int32_t *bin_counts, double min_child_weight,
                     double reg_lambda, double *out_G, double *out_H,
                     double *out_gain, int32_t *out_feature, int32_t *out_bin) {
  if (!E || !grad || !hess || !rows || !feature_indices || !bin_counts)
    return set_error(BSSCL_EINVAL, "node_split: null argument");
  CHK(check_matrix(E, 0));
  const Matrix &X = E->mat[0];
  if (m <= 0) return set_error(BSSCL_EINVAL, "node_split: no rows");
  for (int64_t k = 0; k < m; ++k)
    if (rows[k] < 0 || rows[k] >= X.n) return set_error(BSSCL_EINVAL, "node_split: row out of range");
  if (n_selected <= 0) return set_error(BSSCL_EINVAL, "node_split: no features");
  std::vector<int32_t> feats(feature_indices, feature_indices + n_selected), nb_sel((size_t)n_selected);
  for (int32_t i = 0; i < n_selected; ++i) {
    if (feats[(size_t)i] < 0 || feats[(size_t)i] >= X.F) return set_error(BSSCL_EINVAL, "node_split: feature out of range");
    nb_sel[(size_t)i] = bin_counts[feats[(size_t)i]];
    if (nb_sel[(size_t)i] < 1 || nb_sel[(size_t)i] > kBins) return set_error(BSSCL_EINVAL, "node_split: bad bin count");
  }
  HIPCHK(hipSetDevice(E->device));
  CHK(load_grad_hess(E, grad, hess, X.n, m));
  CHK(E->rows64.ensure((size_t)m));
  HIPCHK(hipMemcpyAsync(E->rows64.p, rows, (size_t)m * 8, hipMemcpyHostToDevice, E->st));
  // The root of a tree build: histogram and split search of these rows.
  const int32_t F_sel = n_selected;
  TreeParams tp{1, 1, 0, min_child_weight, reg_lambda, 0.0};
  E->set_base = 0;
  CHK(prepare_tree_buffers(E, m, F_sel, 1, 2));
  CHK(launch_root(E, nullptr, m, feats, nb_sel, tp, false));
  // No planner follows this root: write its table record here.
  HIPCHK(launch_node_best(E->st, E->segs.p, E->totals.p, E->cand.p, F_sel, E->plan_d, 1, 0,
                          E->nodes_d));
  LevelPlan plan;
  CHK(read_table(E, 1, plan));
  const NodeOut root = *reinterpret_cast<const NodeOut *>(E->table_pin + 64);
  if (root.fpos >= F_sel) return set_error(BSSCL_EINTERNAL, "node_split: bad split record");
  if (out_G || out_H) {
    std::vector<long long> h((size_t)E->node_stride);
    HIPCHK(hipMemcpyAsync(h.data(), E->pool.p, (size_t)E->node_stride * 8, hipMemcpyDeviceToHost, E->st));
    HIPCHK(hipStreamSynchronize(E->st));
    for (int64_t i = 0; i < (int64_t)F_sel * kBins; ++i) {
      if (out_G) out_G[i] = (double)h[(size_t)(2 * i)] * E->g_scale;
      if (out_H) out_H[i] = (double)h[(size_t)(2 * i + 1)] * E->h_scale;
    }
  }
  if (out_gain) *out_gain = root.fpos >= 0 ? root.gain : -1e9;
  if (out_feature) *out_feature = root.fpos >= 0 ? feats[(size_t)root.fpos] : -1;
  if (out_bin) *out_bin = root.fpos >= 0 ? root.bin : 0;
  return BSSCL_OK;
}

int bsscl_partition(bsscl_engine *E, const int64_t *rows, int64_t m,
                    int32_t feature, int32_t bin, int64_t *out_rows,
                    int64_t *out_n_left) {
  if (!E || !rows || !out_rows || !out_n_left)
    return set_error(BSSCL_EINVAL, "partition: null argument");
  CHK(check_matrix(E, 0));
  const Matrix &X = E->mat[0];
  if (m <= 0) return set_error(BSSCL_EINVAL, "partition: no rows");
  if (feature < 0 || feature >= X.F) return set_error(BSSCL_EINVAL, "partition: feature out of range");
  int64_t bin64 = bin;
  split_to_engine(X, feature, bin64);
  bin = (int32_t)bin64;
  for (int64_t k = 0; k < m; ++k)
    if (rows[k] < 0 || rows[k] >= X.n) return set_error(BSSCL_EINVAL, "partition: row out of range");
  HIPCHK(hipSetDevice(E->device));
  if (!E->ghq.p || E->ghq.cap < (size_t)X.n) {
    CHK(E->ghq.ensure((size_t)X.n));
    HIPCHK(hipMemsetAsync(E->ghq.p, 0, (size_t)X.n * sizeof(GH), E->st));
  }
  CHK(E->rows64.ensure((size_t)m));
  HIPCHK(hipMemcpyAsync(E->rows64.p, rows, (size_t)m * 8, hipMemcpyHostToDevice, E->st));
  E->set_base = 0;
  CHK(prepare_tree_buffers(E, m, 1, 1, 2));
  const int32_t f1 = feature;
  Pack pk;
  pk.add(&f1, 4);
  std::vector<char *> dv;
  CHK(upload_pack(E, pk, dv));
  HIPCHK(launch_gather_root(E->st, X.codes.p, X.ld, reinterpret_cast<const int32_t *>(dv[0]), 1,
                            nullptr, E->rows64.p, m, E->ghq.p, E->codes_c[0].p, E->ld_c,
                            E->gh_c[0].p, E->rid_c[0].p, E->ld_c, E->segs.p,
                            E->hist_node_d.p));
  E->track_rid = true;  // this call reads the moved row ids back
  PartParent P{0, m, 0, bin, 1, 2, 0, 0, 0, 0};
  std::vector<PartTile> tiles;
  add_part_tiles(E, P, 0, tiles);
  P.tile1 = (int32_t)tiles.size();
  const int32_t tb[2] = {0, (int32_t)tiles.size()};
  LevelPlan lp = {};
  lp.n_parents = 1;
  lp.n_tiles = (int32_t)tiles.size();
  Pack pk2;
  pk2.add(&P, sizeof(P));
  pk2.add(tb, sizeof(tb));
  pk2.add(tiles.data(), tiles.size() * sizeof(PartTile));
  pk2.add(&lp, sizeof(lp));
  CHK(sync(E));  // the gather has read dv[0]: the arena may be reused
  CHK(upload_pack(E, pk2, dv));
  CHK(launch_partition(E, 0, 1, reinterpret_cast<const PartParent *>(dv[0]), nullptr,
                       reinterpret_cast<const int32_t *>(dv[1]),
                       reinterpret_cast<const PartTile *>(dv[2]),
                       reinterpret_cast<const LevelPlan *>(dv[3]), (int32_t)tiles.size(),
                       1, 0, true));
  E->track_rid = false;
  std::vector<int32_t> r32((size_t)m);
  int64_t nl = 0;
  HIPCHK(hipMemcpyAsync(r32.data(), E->rid_c[1].p, (size_t)m * 4, hipMemcpyDeviceToHost, E->st));
  HIPCHK(hipMemcpyAsync(&nl, E->nleft_d.p, 8, hipMemcpyDeviceToHost, E->st));
  CHK(sync(E));
  for (int64_t k = 0; k < m; ++k) out_rows[k] = r32[(size_t)k];
  *out_n_left = nl;
  return BSSCL_OK;
}

int bsscl_fisher_yates_apply(bsscl_engine *E, const uint32_t *draws, int64_t n,
                             int32_t *data) {
  if (!E || n < 0 || n > INT32_MAX || (n > 0 && !data) || (n > 1 && !draws))
    return set_error(BSSCL_EINVAL, "fisher_yates_apply: bad arguments");
  for (int64_t t = 0; t + 1 < n; ++t)
    if ((int64_t)draws[t] > n - 1 - t)
      return set_error(BSSCL_EINVAL, "fisher_yates_apply: draw " + std::to_string(t) +
                                         " exceeds its step " + std::to_string(n - 1 - t));
  if (n <= 1) return BSSCL_OK;
  HIPCHK(hipSetDevice(E->device));
  HIPCHK(hipStreamSynchronize(E->st_rows));  // the work arrays are shared with the rounds
  TempBuf<int32_t> a, b;
  TempBuf<uint32_t> d;
  FyWork w;
  int rc = BSSCL_OK;
  for (DevBuf<int32_t> *x : {&a, &b})
    if (rc == BSSCL_OK) rc = x->ensure((size_t)n);
  if (rc == BSSCL_OK) rc = d.ensure((size_t)n);
  if (rc == BSSCL_OK) rc = ensure_fy_work(E, n, w);
  hipError_t e = hipSuccess;
  if (rc == BSSCL_OK) {
    e = hipMemcpyAsync(a.p, data, (size_t)n * 4, hipMemcpyHostToDevice, E->st);
    if (e == hipSuccess) e = hipMemcpyAsync(d.p, draws, (size_t)(n - 1) * 4, hipMemcpyHostToDevice, E->st);
    if (e == hipSuccess) e = launch_fisher_yates(E->st, d.p, n, a.p, b.p, w);
    if (e == hipSuccess) e = hipMemcpyAsync(data, b.p, (size_t)n * 4, hipMemcpyDeviceToHost, E->st);
    if (e == hipSuccess) e = hipStreamSynchronize(E->st);
    if (e != hipSuccess) rc = set_error(BSSCL_EDEVICE, std::string("fisher_yates_apply: ") + hipGetErrorString(e));
  }
  (void)hipStreamSynchronize(E->st);
  for (DevBuf<int32_t> *x : {&a, &b}) x->release();
  d.release();
  return rc;
}

int bsscl_engine_set_profiling(bsscl_engine *E, int32_t on) {
  if (!E) return set_error(BSSCL_EINVAL, "null engine");
  HIPCHK(hipSetDevice(E->device));
  HIPCHK(hipStreamSynchronize(E->st));
  CHK(prof_collect(E));
  if (on) {
    std::memset(E->stats, 0, sizeof(E->stats));
    E->ktime_launches.clear();
    E->ktime_used = 0;
  }
  E->prof = std::max(0, std::min(2, (int)on));
  return BSSCL_OK;
}

int bsscl_engine_stats(bsscl_engine *E, double *out, int32_t cap, int32_t *n_out) {
  if (!E || !out || !n_out) return set_error(BSSCL_EINVAL, "null argument");
  if (!E->ktime_launches.empty()) {
    HIPCHK(hipSetDevice(E->device));
    HIPCHK(hipStreamSynchronize(E->st));
    CHK(prof_slots_collect(E));
  }
  const int32_t n = std::min<int32_t>(cap, 21);
  for (int32_t i = 0; i < n; ++i) out[i] = E->stats[i];
  *n_out = n;
  return BSSCL_OK;
}

}  // extern "C"
