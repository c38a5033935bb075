// Column sort for the bin edges of _build_bin_edges (est:2073-2141; "est:"
// is src/bsscl_gbm/estimator_v1_0_1.py).
//
// The reference finds each feature's edges on the host: np.isnan, then
// np.unique (a full sort) and np.percentile (a partition) of the non-NaN
// values.  Everything those calls need from the data is order statistics:
// the number of NaNs, the number of distinct values, the distinct values
// themselves when there are few, and the values at the ranks np.percentile
// interpolates between.  This file sorts every column on the device so the
// host can read exactly those values; the interpolation stays on the host in
// NumPy's own arithmetic.
//
// Keys.  A value becomes an unsigned integer whose order is the float order:
// non-negative floats get the sign bit set, negative floats are inverted.
// Every NaN maps to the largest key, so NaNs sort last, and -0.0 maps to the
// key of +0.0, so the two zeros count as one value (np.unique treats them
// as equal).  The columns are stored feature-major, padded to whole tiles
// with the largest key.
//
// Sort.  Least-significant-digit radix sort with 8-bit digits: 4 passes for
// float32 columns, 8 for float64.  Each pass is
//   k_rs_count   per tile (4096 keys of one column): digit counts, stored
//                tile-major (one coalesced 1 KB row per tile),
//   k_rs_scan_tiles  per group of 32 tiles: each tile's exclusive prefix
//                within the group (in place) and the group's totals,
//   k_rs_scan_groups per column: each group's exclusive prefix and each
//                digit's start,
//   k_rs_scatter per tile: each key's stable rank among the tile's keys of
//                its digit, the tile regrouped by digit in LDS, then written
//                out run by run (consecutive threads, consecutive addresses).
// Ranks within a wave come from a match of the 8 digit bits over ballots,
// so equal digits never meet in an LDS atomic.  Keys keep their order
// within a digit (round-major order inside a tile, tiles in order), which
// is what makes the passes compose into a sort.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "kernels.h"

namespace bsscl {

namespace {

constexpr int kSortThreads = 256;
constexpr int kSortWaves = kSortThreads / 64;
constexpr int kRadix = 256;

template <typename KT> struct SortTile;
template <> struct SortTile<uint32_t> { static constexpr int kItems = 16; };
template <> struct SortTile<uint64_t> { static constexpr int kItems = 8; };

template <typename KT>
constexpr int tile_keys() { return kSortThreads * SortTile<KT>::kItems; }

__device__ __forceinline__ uint32_t sort_key(float v) {
  if (v != v) return 0xffffffffu;
  uint32_t u = __float_as_uint(v);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ uint64_t sort_key(double v) {
  if (v != v) return ~0ull;
  uint64_t u = (uint64_t)__double_as_longlong(v);
  if (u == 0x8000000000000000ull) u = 0ull;
  return (u >> 63) ? ~u : (u | 0x8000000000000000ull);
}

__device__ __forceinline__ double key_value(uint32_t k) {
  const uint32_t u = (k & 0x80000000u) ? (k ^ 0x80000000u) : ~k;
  return (double)__uint_as_float(u);
}

__device__ __forceinline__ double key_value(uint64_t k) {
  const uint64_t u = (k >> 63) ? (k ^ 0x8000000000000000ull) : ~k;
  return __longlong_as_double((long long)u);
}

// Lanes of the wave whose 8-bit digit equals this lane's (all lanes active).
__device__ __forceinline__ uint64_t match_digit(uint32_t d) {
  uint64_t m = ~0ull;
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    const bool bit = (d >> b) & 1u;
    const uint64_t bal = __ballot(bit);
    m &= bit ? bal : ~bal;
  }
  return m;
}

__device__ __forceinline__ uint32_t lanes_below(uint64_t m) {
  const uint32_t lane = threadIdx.x & 63u;
  return (uint32_t)__popcll(m & ((1ull << lane) - 1ull));
}

// Exclusive prefix over the 256 values held one per thread (block of 256).
__device__ __forceinline__ uint32_t block_excl_256(uint32_t v, uint32_t *tmp) {
  const int t = (int)threadIdx.x, lane = t & 63, w = t >> 6;
  uint32_t x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) tmp[w] = x;
  __syncthreads();
  uint32_t base = 0;
  for (int k = 0; k < w; ++k) base += tmp[k];
  __syncthreads();
  return base + x - v;
}

// Row-major X (n x F) -> feature-major keys [F][ld], 64 rows per block
// staged through LDS (as the binning kernel).
constexpr int kKeyRows = 64;

template <typename T, typename KT>
__global__ __launch_bounds__(256) void k_col_keys(const T *__restrict__ X, int64_t n,
                                                  int32_t F, KT *__restrict__ keys,
                                                  int64_t ld) {
  extern __shared__ unsigned char smem[];
  T *xs = reinterpret_cast<T *>(smem);  // [64][F]
  const int64_t r0 = (int64_t)blockIdx.x * kKeyRows;
  const int rows = (int)min<int64_t>(kKeyRows, n - r0);
  for (int i = threadIdx.x; i < rows * F; i += blockDim.x) xs[i] = X[r0 * F + i];
  __syncthreads();
  for (int i = threadIdx.x; i < kKeyRows * F; i += blockDim.x) {
    const int f = i / kKeyRows, r = i % kKeyRows;
    if (r < rows) keys[(int64_t)f * ld + r0 + r] = sort_key(xs[r * F + f]);
  }
}

// Same, one thread per (row, feature), for matrices too wide for LDS.
template <typename T, typename KT>
__global__ __launch_bounds__(256) void k_col_keys_wide(const T *__restrict__ X, int64_t n,
                                                       int32_t F, KT *__restrict__ keys,
                                                       int64_t ld) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int32_t f = (int32_t)blockIdx.y;
  if (i < n) keys[(int64_t)f * ld + i] = sort_key(X[i * F + f]);
}

// Pads every column's keys [n, ld) with the largest key.
template <typename KT>
__global__ __launch_bounds__(256) void k_col_pad(KT *__restrict__ keys, int64_t n, int64_t ld) {
  const int64_t i = n + (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < ld) keys[(int64_t)blockIdx.y * ld + i] = (KT)~(KT)0;
}

// Key sources of a pass: the keys of the previous pass in memory, or (the
// first pass of the Fisher-Yates sort) keys made from the draws.  in(col, s)
// is key s of column col.
template <typename KT>
struct KeysIn {
  const KT *keys;
  int64_t ld;
  __device__ void prepare() {}
  __device__ KT operator()(int32_t col, int64_t s) const { return keys[(int64_t)col * ld + s]; }
};

}  // namespace

namespace {

// Digit counts of one tile: counts[(col * n_tiles + tile) * 256 + d].
template <typename KT, typename In>
__global__ __launch_bounds__(kSortThreads) void k_rs_count(In in, int32_t n_tiles, int32_t shift,
                                                           uint32_t *__restrict__ counts) {
  constexpr int kItems = SortTile<KT>::kItems;
  __shared__ uint32_t cnt[kSortWaves][kRadix];
  const int t = (int)threadIdx.x, w = t >> 6;
  const int32_t tile = (int32_t)blockIdx.x, col = (int32_t)blockIdx.y;
  for (int k = 0; k < kSortWaves; ++k) cnt[k][t] = 0;
  __syncthreads();
  in.prepare();
  const int64_t s0 = (int64_t)tile * tile_keys<KT>();
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const uint32_t d = (uint32_t)(in(col, s0 + i * kSortThreads + t) >> shift) & 255u;
    const uint64_t m = match_digit(d);
    if (lanes_below(m) == 0) cnt[w][d] += (uint32_t)__popcll(m);
  }
  __syncthreads();
  uint32_t s = 0;
#pragma unroll
  for (int k = 0; k < kSortWaves; ++k) s += cnt[k][t];
  counts[((int64_t)col * n_tiles + tile) * kRadix + t] = s;
}

// Tiles per group of the two-level prefix over the tiles.
constexpr int kScanGroup = 32;

__host__ __device__ constexpr int32_t scan_groups(int32_t n_tiles) {
  return (n_tiles + kScanGroup - 1) / kScanGroup;
}

// One group of kScanGroup tiles of one column, one thread per digit: each
// tile's count becomes the exclusive prefix of the group's earlier tiles (in
// place), and the group's total goes to gsum[(col * n_groups + g) * 256 + d].
__global__ __launch_bounds__(256) void k_rs_scan_tiles(uint32_t *__restrict__ counts,
                                                       int32_t n_tiles, int32_t n_groups,
                                                       uint32_t *__restrict__ gsum) {
  const int d = (int)threadIdx.x;
  const int32_t g = (int32_t)blockIdx.x, col = (int32_t)blockIdx.y;
  const int32_t t0 = g * kScanGroup;
  uint32_t *c = counts + ((int64_t)col * n_tiles + t0) * kRadix + d;
  uint32_t v[kScanGroup];
#pragma unroll
  for (int i = 0; i < kScanGroup; ++i) v[i] = t0 + i < n_tiles ? c[(int64_t)i * kRadix] : 0u;
  uint32_t run = 0;
#pragma unroll
  for (int i = 0; i < kScanGroup; ++i) {
    if (t0 + i < n_tiles) c[(int64_t)i * kRadix] = run;
    run += v[i];
  }
  gsum[((int64_t)col * n_groups + g) * kRadix + d] = run;
}

// One column, one thread per digit: each group's total becomes the
// exclusive prefix of the earlier groups (in place), and each digit's start
// in the output (the keys of all smaller digits) goes to starts[col * 256 + d].
__global__ __launch_bounds__(256) void k_rs_scan_groups(uint32_t *__restrict__ gsum,
                                                        int32_t n_groups,
                                                        uint32_t *__restrict__ starts) {
  __shared__ uint32_t tmp[4];
  const int d = (int)threadIdx.x;
  const int32_t col = (int32_t)blockIdx.x;
  uint32_t *gs = gsum + (int64_t)col * n_groups * kRadix + d;
  uint32_t run = 0;
  for (int32_t g0 = 0; g0 < n_groups; g0 += 8) {
    uint32_t v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = g0 + e < n_groups ? gs[(int64_t)(g0 + e) * kRadix] : 0u;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (g0 + e < n_groups) gs[(int64_t)(g0 + e) * kRadix] = run;
      run += v[e];
    }
  }
  starts[(int64_t)col * kRadix + d] = block_excl_256(run, tmp);
}

// One stable counting-sort pass of one tile by the digit at `shift`.
template <typename KT, typename In>
__global__ __launch_bounds__(kSortThreads) void k_rs_scatter(In in, KT *__restrict__ out,
                                                             int64_t ld, int32_t n_tiles,
                                                             int32_t shift,
                                                             const uint32_t *__restrict__ offs,
                                                             const uint32_t *__restrict__ gpre,
                                                             const uint32_t *__restrict__ starts) {
  constexpr int kItems = SortTile<KT>::kItems;
  constexpr int kTile = tile_keys<KT>();
  __shared__ KT tk[kTile];
  __shared__ uint32_t wcnt[kSortWaves][kRadix];
  __shared__ uint32_t running[kRadix], local_off[kRadix], gbase[kRadix];
  __shared__ uint32_t tmp[4];
  const int t = (int)threadIdx.x, w = t >> 6;
  const int32_t tile = (int32_t)blockIdx.x, col = (int32_t)blockIdx.y;
  in.prepare();
  const int64_t s0 = (int64_t)tile * kTile;
  KT key[kItems];
#pragma unroll
  for (int i = 0; i < kItems; ++i) key[i] = in(col, s0 + i * kSortThreads + t);
  // Start of digit t's run for this tile in the output column: the digit's
  // start, its keys in the earlier groups and in the group's earlier tiles.
  const int32_t n_groups = scan_groups(n_tiles);
  gbase[t] = starts[(int64_t)col * kRadix + t] +
             gpre[((int64_t)col * n_groups + tile / kScanGroup) * kRadix + t] +
             offs[((int64_t)col * n_tiles + tile) * kRadix + t];
  running[t] = 0;
  for (int k = 0; k < kSortWaves; ++k) wcnt[k][t] = 0;
  __syncthreads();
  uint32_t pos[kItems];
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const uint32_t d = (uint32_t)(key[i] >> shift) & 255u;
    const uint64_t m = match_digit(d);
    const uint32_t r = lanes_below(m);
    if (r == 0) wcnt[w][d] = (uint32_t)__popcll(m);
    __syncthreads();
    uint32_t p = running[d] + r;
    for (int k = 0; k < w; ++k) p += wcnt[k][d];
    pos[i] = p;
    __syncthreads();
    uint32_t s = 0;
#pragma unroll
    for (int k = 0; k < kSortWaves; ++k) {
      s += wcnt[k][t];
      wcnt[k][t] = 0;
    }
    running[t] += s;
    __syncthreads();
  }
  const uint32_t lo = block_excl_256(running[t], tmp);
  local_off[t] = lo;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const uint32_t d = (uint32_t)(key[i] >> shift) & 255u;
    tk[local_off[d] + pos[i]] = key[i];
  }
  __syncthreads();
  KT *dst = out + (int64_t)col * ld;
  for (int j = t; j < kTile; j += kSortThreads) {
    const KT k = tk[j];
    const uint32_t d = (uint32_t)(k >> shift) & 255u;
    dst[gbase[d] + (uint32_t)j - local_off[d]] = k;
  }
}

// m[col] = number of non-NaN values of a sorted column: the position of
// the first largest key (NaNs and padding), found by binary search.
template <typename KT>
__global__ __launch_bounds__(64) void k_col_valid(const KT *__restrict__ keys, int64_t ld,
                                                  int32_t F, int64_t *__restrict__ m) {
  const int32_t col = (int32_t)(blockIdx.x * blockDim.x + threadIdx.x);
  if (col >= F) return;
  const KT *k = keys + (int64_t)col * ld;
  const KT top = (KT)~(KT)0;
  int64_t lo = 0, hi = ld;  // first position in [lo, hi] holding top
  while (lo < hi) {
    const int64_t mid = lo + (hi - lo) / 2;
    if (k[mid] == top) hi = mid;
    else lo = mid + 1;
  }
  m[col] = lo;
}

// Number of i in [1, m_col) with key[i] != key[i-1], added to out[col]:
// one atomic per block (a few dozen blocks per column).
template <typename KT>
__global__ __launch_bounds__(256) void k_col_changes(const KT *__restrict__ keys, int64_t ld,
                                                     const int64_t *__restrict__ m,
                                                     unsigned long long *__restrict__ out) {
  __shared__ unsigned long long wsum[4];
  const int32_t col = (int32_t)blockIdx.y;
  const int64_t mc = m[col];
  const KT *k = keys + (int64_t)col * ld;
  unsigned long long c = 0;
  for (int64_t i = 1 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < mc;
       i += (int64_t)gridDim.x * blockDim.x)
    c += (k[i] != k[i - 1]) ? 1ull : 0ull;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) c += __shfl_xor(c, o, 64);
  if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned long long t = wsum[0] + wsum[1] + wsum[2] + wsum[3];
    if (t) atomicAdd(out + col, t);
  }
}

// Positions of the first key of every run of equal keys in [0, m); at most
// max_out positions are stored (in no particular order), all are counted.
template <typename KT>
__global__ __launch_bounds__(256) void k_col_run_starts(const KT *__restrict__ keys, int64_t m,
                                                        int32_t max_out,
                                                        int64_t *__restrict__ pos,
                                                        unsigned int *__restrict__ count) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < m;
       i += (int64_t)gridDim.x * blockDim.x) {
    if (i == 0 || keys[i] != keys[i - 1]) {
      const unsigned int s = atomicAdd(count, 1u);
      if ((int32_t)s < max_out) pos[s] = i;
    }
  }
}

// out[k] = value at position pos[k] of sorted column col[k].
template <typename KT>
__global__ __launch_bounds__(256) void k_col_gather(const KT *__restrict__ keys, int64_t ld,
                                                    int64_t count, const int32_t *__restrict__ col,
                                                    const int64_t *__restrict__ pos,
                                                    double *__restrict__ out) {
  const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (k < count) out[k] = key_value(keys[(int64_t)col[k] * ld + pos[k]]);
}

unsigned grid_1d(int64_t n, int64_t cap) {
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>((n + 255) / 256, cap));
}

template <typename T, typename KT>
hipError_t col_sort_impl(hipStream_t st, const void *Xv, int64_t n, int32_t F, void *keys_v,
                         void *tmp_v, int64_t ld, uint32_t *counts, uint32_t *totals,
                         int64_t *m) {
  const T *X = static_cast<const T *>(Xv);
  KT *keys = static_cast<KT *>(keys_v);
  KT *tmp = static_cast<KT *>(tmp_v);
  const size_t lds = sizeof(T) * (size_t)kKeyRows * F;
  if (lds <= 48 * 1024) {
    hipLaunchKernelGGL((k_col_keys<T, KT>), dim3((unsigned)((n + kKeyRows - 1) / kKeyRows)),
                       dim3(256), lds, st, X, n, F, keys, ld);
  } else {
    hipLaunchKernelGGL((k_col_keys_wide<T, KT>), dim3((unsigned)((n + 255) / 256), (unsigned)F),
                       dim3(256), 0, st, X, n, F, keys, ld);
  }
  if (ld > n)
    hipLaunchKernelGGL((k_col_pad<KT>), dim3((unsigned)((ld - n + 255) / 256), (unsigned)F),
                       dim3(256), 0, st, keys, n, ld);
  const int32_t n_tiles = (int32_t)(ld / tile_keys<KT>());
  const int32_t n_groups = scan_groups(n_tiles);
  uint32_t *gsum = counts + (int64_t)F * n_tiles * kRadix;  // after the counts
  const dim3 tiles((unsigned)n_tiles, (unsigned)F);
  for (int shift = 0; shift < (int)(8 * sizeof(KT)); shift += 8) {
    hipLaunchKernelGGL((k_rs_count<KT, KeysIn<KT>>), tiles, dim3(kSortThreads), 0, st,
                       KeysIn<KT>{keys, ld}, n_tiles, shift, counts);
    hipLaunchKernelGGL(k_rs_scan_tiles, dim3((unsigned)n_groups, (unsigned)F), dim3(256), 0, st,
                       counts, n_tiles, n_groups, gsum);
    hipLaunchKernelGGL(k_rs_scan_groups, dim3((unsigned)F), dim3(256), 0, st, gsum, n_groups,
                       totals);
    hipLaunchKernelGGL((k_rs_scatter<KT, KeysIn<KT>>), tiles, dim3(kSortThreads), 0, st,
                       KeysIn<KT>{keys, ld}, tmp, ld, n_tiles, shift, counts, gsum, totals);
    std::swap(keys, tmp);
  }
  // An even number of passes leaves the sorted keys in keys_v.
  hipLaunchKernelGGL((k_col_valid<KT>), dim3((unsigned)((F + 63) / 64)), dim3(64), 0, st,
                     static_cast<const KT *>(keys_v), ld, F, m);
  return hipGetLastError();
}

}  // namespace

int64_t col_sort_ld(int64_t n, int is_f64) {
  const int64_t tile = is_f64 ? tile_keys<uint64_t>() : tile_keys<uint32_t>();
  return (n + tile - 1) / tile * tile;
}

int64_t col_sort_count_words(int64_t n, int32_t F, int is_f64) {
  const int64_t tile = is_f64 ? tile_keys<uint64_t>() : tile_keys<uint32_t>();
  const int64_t n_tiles = col_sort_ld(n, is_f64) / tile;
  // The tiles' counts, then the groups' prefixes.
  return (int64_t)F * kRadix * (n_tiles + scan_groups((int32_t)n_tiles));
}

hipError_t launch_col_sort(hipStream_t st, const void *X, int is_f64, int64_t n, int32_t F,
                           void *keys, void *tmp, int64_t ld, uint32_t *counts,
                           uint32_t *totals, int64_t *m) {
  if (n <= 0 || F <= 0) return hipSuccess;
  if (is_f64)
    return col_sort_impl<double, uint64_t>(st, X, n, F, keys, tmp, ld, counts, totals, m);
  return col_sort_impl<float, uint32_t>(st, X, n, F, keys, tmp, ld, counts, totals, m);
}

int64_t sort_u64_ld(int64_t n) { return col_sort_ld(n, 1); }

int64_t sort_u64_count_words(int64_t n) { return col_sort_count_words(n, 1, 1); }

namespace {

// Passes over bits [lo_bit, hi_bit) in 8-bit digits, the first one reading
// its keys from `first` (the keys buffer, or keys made on the fly), the
// others from the previous pass's output; `keys` and `tmp` alternate as
// outputs, starting with `keys`.
template <typename In>
hipError_t sort_u64_passes(hipStream_t st, In first, uint64_t *keys, uint64_t *tmp, int64_t ld,
                           int lo_bit, int hi_bit, uint32_t *counts, uint32_t *totals,
                           uint64_t **result) {
  const int32_t n_tiles = (int32_t)(ld / tile_keys<uint64_t>());
  const int32_t n_groups = scan_groups(n_tiles);
  uint32_t *gsum = counts + (int64_t)n_tiles * kRadix;  // after the counts
  const dim3 tiles((unsigned)n_tiles, 1u);
  const uint64_t *src = nullptr;
  uint64_t *dst = keys, *other = tmp;
  for (int shift = lo_bit; shift < hi_bit; shift += 8) {
    if (!src) {
      hipLaunchKernelGGL((k_rs_count<uint64_t, In>), tiles, dim3(kSortThreads), 0, st, first,
                         n_tiles, shift, counts);
    } else {
      hipLaunchKernelGGL((k_rs_count<uint64_t, KeysIn<uint64_t>>), tiles, dim3(kSortThreads), 0,
                         st, KeysIn<uint64_t>{src, ld}, n_tiles, shift, counts);
    }
    hipLaunchKernelGGL(k_rs_scan_tiles, dim3((unsigned)n_groups, 1u), dim3(256), 0, st, counts,
                       n_tiles, n_groups, gsum);
    hipLaunchKernelGGL(k_rs_scan_groups, dim3(1u), dim3(256), 0, st, gsum, n_groups, totals);
    if (!src) {
      hipLaunchKernelGGL((k_rs_scatter<uint64_t, In>), tiles, dim3(kSortThreads), 0, st, first,
                         dst, ld, n_tiles, shift, counts, gsum, totals);
    } else {
      hipLaunchKernelGGL((k_rs_scatter<uint64_t, KeysIn<uint64_t>>), tiles, dim3(kSortThreads),
                         0, st, KeysIn<uint64_t>{src, ld}, dst, ld, n_tiles, shift, counts, gsum,
                         totals);
    }
    src = dst;
    std::swap(dst, other);
  }
  *result = const_cast<uint64_t *>(src);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_sort_u64(hipStream_t st, uint64_t *keys, uint64_t *tmp, int64_t ld,
                           int lo_bit, int hi_bit, uint32_t *counts, uint32_t *totals,
                           uint64_t **result) {
  // The first pass reads `keys` and writes `tmp`.
  if (lo_bit >= hi_bit) {
    *result = keys;
    return hipSuccess;
  }
  return sort_u64_passes(st, KeysIn<uint64_t>{keys, ld}, tmp, keys, ld, lo_bit, hi_bit, counts,
                         totals, result);
}

hipError_t launch_sort_fy_keys(hipStream_t st, FyKeysIn first, uint64_t *keys, uint64_t *tmp,
                               int64_t ld, int lo_bit, int hi_bit, uint32_t *counts,
                               uint32_t *totals, uint64_t **result) {
  return sort_u64_passes(st, first, keys, tmp, ld, lo_bit, hi_bit, counts, totals, result);
}

hipError_t launch_col_changes(hipStream_t st, const void *keys, int is_f64, int64_t ld, int32_t F,
                              const int64_t *m, int64_t max_m, unsigned long long *out) {
  if (F <= 0 || max_m <= 1) return hipSuccess;
  const dim3 grid(grid_1d(max_m, 64), (unsigned)F);
  if (is_f64)
    hipLaunchKernelGGL(k_col_changes<uint64_t>, grid, dim3(256), 0, st,
                       static_cast<const uint64_t *>(keys), ld, m, out);
  else
    hipLaunchKernelGGL(k_col_changes<uint32_t>, grid, dim3(256), 0, st,
                       static_cast<const uint32_t *>(keys), ld, m, out);
  return hipGetLastError();
}

hipError_t launch_col_run_starts(hipStream_t st, const void *keys, int is_f64, int64_t ld,
                                 int32_t col, int64_t m, int32_t max_out, int64_t *pos,
                                 unsigned int *count) {
  if (m <= 0) return hipSuccess;
  if (is_f64)
    hipLaunchKernelGGL(k_col_run_starts<uint64_t>, dim3(grid_1d(m, 4096)), dim3(256), 0, st,
                       static_cast<const uint64_t *>(keys) + (int64_t)col * ld, m, max_out, pos,
                       count);
  else
    hipLaunchKernelGGL(k_col_run_starts<uint32_t>, dim3(grid_1d(m, 4096)), dim3(256), 0, st,
                       static_cast<const uint32_t *>(keys) + (int64_t)col * ld, m, max_out, pos,
                       count);
  return hipGetLastError();
}

hipError_t launch_col_gather(hipStream_t st, const void *keys, int is_f64, int64_t ld,
                             int64_t count, const int32_t *col, const int64_t *pos, double *out) {
  if (count <= 0) return hipSuccess;
  const dim3 grid((unsigned)((count + 255) / 256));
  if (is_f64)
    hipLaunchKernelGGL(k_col_gather<uint64_t>, grid, dim3(256), 0, st,
                       static_cast<const uint64_t *>(keys), ld, count, col, pos, out);
  else
    hipLaunchKernelGGL(k_col_gather<uint32_t>, grid, dim3(256), 0, st,
                       static_cast<const uint32_t *>(keys), ld, count, col, pos, out);
  return hipGetLastError();
}

}  // namespace bsscl
