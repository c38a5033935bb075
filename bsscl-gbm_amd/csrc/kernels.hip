// HIP kernels of the tree engine, written for gfx950 (wave64, 160 KB LDS).
//
// Layouts in HBM
//   codes     feature-major uint8 [F][ld], ld a multiple of 256, zero padded
//   ghq       GH [n]: gradient and hessian of each row in 64-bit fixed
//             point (g*2^sg, h*2^sh), rebuilt every boosting round
//   compact   per tree, two ping-pong sets of (codes_c [F_sel][ld_c] uint8,
//             gh_c GH [ld_c], rid_c int32 [ld_c]); every node's rows are a
//             contiguous segment of the set of its depth's parity
//   pool      per node [F_sel][256 bins][g,h] int64 fixed-point sums
//
// Fixed-point sums are exact integer additions, so histograms, splits and
// trees do not depend on atomic order or on the order of rows.
#include "kernels.h"
#include "wave.h"

#include <hip/hip_ext.h>

#include <algorithm>

namespace bsscl {

namespace {

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & 63); }

// a / b for a >= 0, b > 0 in 32-bit arithmetic when both fit (row counts
// do); the 64-bit division is a long software sequence.
__device__ __forceinline__ int64_t div_pos(int64_t a, int64_t b) {
  if ((((uint64_t)a | (uint64_t)b) >> 32) == 0) return (int64_t)((uint32_t)a / (uint32_t)b);
  return a / b;
}

// Exclusive scan over a block of BLOCK threads; `tmp` holds BLOCK/64 words.
template <int BLOCK, typename T>
__device__ __forceinline__ T block_excl_scan(T v, T *tmp, T &total) {
  const int wid = (int)(threadIdx.x >> 6);
  const T incl = wave_incl_scan<T>(v);
  if (lane_id() == 63) tmp[wid] = incl;
  __syncthreads();
  T pre = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < BLOCK / 64; ++w) {
    T s = tmp[w];
    pre += (w < wid) ? s : T(0);
    tot += s;
  }
  __syncthreads();
  total = tot;
  return pre + incl - v;
}

}  // namespace

// ---------------------------------------------------------------------------
// Binning: est:155-226 codes plus est:2144-2189 NaN handling.  A block bins
// 64 rows x all features: the rows are read row-major (coalesced) into LDS,
// each code is found by the binary search of the standard strategy (the
// hybrid strategy returns the same code), and each feature's 64 codes are
// written as one contiguous run of the feature-major matrix.
// ---------------------------------------------------------------------------
constexpr int kBinRows = 64;

// Code of one value: the largest k in [0, nb-1] with e[k] <= v, 0 below
// e[0], nb-1 at or above e[nb] (est:204-226); NaN handling of est:2159-2177.
// The matrix stores the code's tiers (tier_code) in columns t * F + f.
__device__ __forceinline__ int32_t bin_one(double v, const double *__restrict__ e,
                                           int32_t nbf, bool nan_feat,
                                           int32_t has_any_nan) {
  if (v != v) {
    if (nan_feat) return 0;
    if (has_any_nan) v = 0.0;  // placeholder value of est:2160
  }
  int32_t c;
  if (v < e[0]) {
    c = 0;
  } else if (v >= e[nbf]) {
    c = nbf - 1;
  } else {
    int32_t lo = 0, hi = nbf - 1;
    while (lo < hi) {
      const int32_t mid = (lo + hi) >> 1;
      if (e[mid + 1] <= v) lo = mid + 1;
      else hi = mid;
    }
    c = lo;
  }
  if (nan_feat) c += 1;  // est:2176
  return c;
}

// Tier t of a code (t = 0: min(code, 255); kernels.h).
__device__ __forceinline__ uint8_t tier_code(int32_t code, int32_t t) {
  return (uint8_t)min(max(code - 255 * t, 0), 255);
}

template <typename T>
__global__ __launch_bounds__(256) void k_bin(
    const T *__restrict__ X, int64_t n, int32_t F,
    const double *__restrict__ edges, int32_t stride,
    const int32_t *__restrict__ nb, const int32_t *__restrict__ nan_id,
    int32_t has_any_nan, uint8_t *__restrict__ codes, int64_t ld, int32_t tiers) {
  extern __shared__ unsigned char smem[];
  T *xs = reinterpret_cast<T *>(smem);                        // [64][F]
  uint8_t *cs = smem + sizeof(T) * (size_t)kBinRows * F;     // [tiers * F][64]
  const int64_t r0 = (int64_t)blockIdx.x * kBinRows;
  const int rows = (int)min<int64_t>(kBinRows, n - r0);
  const int tot = rows * F;
  const int cols = tiers * F;
  for (int i = threadIdx.x; i < tot; i += blockDim.x)
    xs[i] = X[r0 * F + i];
  __syncthreads();
  for (int i = threadIdx.x; i < kBinRows * F; i += blockDim.x) {
    const int f = i / kBinRows, r = i % kBinRows;
    int32_t code = 0;
    if (r < rows)
      code = bin_one((double)xs[r * F + f], edges + (int64_t)f * stride, nb[f],
                     nan_id[f] >= 0, has_any_nan);
    for (int32_t t = 0; t < tiers; ++t) cs[(t * F + f) * kBinRows + r] = tier_code(code, t);
  }
  __syncthreads();
  // 16 dwords per column.
  for (int i = threadIdx.x; i < cols * (kBinRows / 4); i += blockDim.x) {
    const int f = i / (kBinRows / 4), w = i % (kBinRows / 4);
    const uint32_t v = *reinterpret_cast<const uint32_t *>(cs + f * kBinRows + 4 * w);
    *reinterpret_cast<uint32_t *>(codes + (int64_t)f * ld + r0 + 4 * w) = v;
  }
}

// One thread per (row, feature) for matrices too wide to stage 64 rows in LDS.
template <typename T>
__global__ __launch_bounds__(256) void k_bin_wide(
    const T *__restrict__ X, int64_t n, int32_t F,
    const double *__restrict__ edges, int32_t stride,
    const int32_t *__restrict__ nb, const int32_t *__restrict__ nan_id,
    int32_t has_any_nan, uint8_t *__restrict__ codes, int64_t ld, int32_t tiers) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int32_t f = (int32_t)blockIdx.y;
  if (i >= n) return;
  const int32_t code = bin_one((double)X[i * F + f], edges + (int64_t)f * stride, nb[f],
                               nan_id[f] >= 0, has_any_nan);
  for (int32_t t = 0; t < tiers; ++t) codes[(int64_t)(t * F + f) * ld + i] = tier_code(code, t);
}

hipError_t launch_bin(hipStream_t st, const void *X, int is_f64, int64_t n,
                      int32_t F, const double *edges, int32_t stride,
                      const int32_t *nb, const int32_t *nan_id,
                      int32_t has_any_nan, uint8_t *codes, int64_t ld, int32_t tiers) {
  if (n <= 0) return hipSuccess;
  const size_t lds = (is_f64 ? 8 : 4) * (size_t)kBinRows * F +
                     (size_t)kBinRows * F * (size_t)tiers;
  if (lds > 48 * 1024) {
    const dim3 grid((unsigned)((n + 255) / 256), (unsigned)F);
    if (is_f64)
      hipLaunchKernelGGL(k_bin_wide<double>, grid, dim3(256), 0, st,
                         (const double *)X, n, F, edges, stride, nb, nan_id,
                         has_any_nan, codes, ld, tiers);
    else
      hipLaunchKernelGGL(k_bin_wide<float>, grid, dim3(256), 0, st,
                         (const float *)X, n, F, edges, stride, nb, nan_id,
                         has_any_nan, codes, ld, tiers);
    return hipGetLastError();
  }
  const unsigned blocks = (unsigned)((n + kBinRows - 1) / kBinRows);
  if (is_f64)
    hipLaunchKernelGGL(k_bin<double>, dim3(blocks), dim3(256), lds, st,
                       (const double *)X, n, F, edges, stride, nb, nan_id,
                       has_any_nan, codes, ld, tiers);
  else
    hipLaunchKernelGGL(k_bin<float>, dim3(blocks), dim3(256), lds, st,
                       (const float *)X, n, F, edges, stride, nb, nan_id,
                       has_any_nan, codes, ld, tiers);
  return hipGetLastError();
}

// Per-feature code counts of a matrix (for each feature's most frequent
// bin).  Block (x, f) counts 64K rows of feature f in LDS.
constexpr int kCountRows = 1 << 16;

__global__ __launch_bounds__(256) void k_code_counts(const uint8_t *__restrict__ codes,
                                                     int64_t ld, int64_t n,
                                                     unsigned int *__restrict__ counts) {
  __shared__ unsigned int c[256];
  const int f = (int)blockIdx.y;
  c[threadIdx.x] = 0;
  __syncthreads();
  const int64_t r0 = (int64_t)blockIdx.x * kCountRows;
  const int64_t r1 = min(n, r0 + kCountRows);
  const uint8_t *col = codes + (int64_t)f * ld;
  for (int64_t r = r0 + threadIdx.x; r < r1; r += 256) atomicAdd(&c[col[r]], 1u);
  __syncthreads();
  if (c[threadIdx.x]) atomicAdd(&counts[f * 256 + threadIdx.x], c[threadIdx.x]);
}

hipError_t launch_code_counts(hipStream_t st, const uint8_t *codes, int64_t ld,
                              int64_t n, int32_t F, unsigned int *counts) {
  if (n <= 0) return hipSuccess;
  const dim3 grid((unsigned)((n + kCountRows - 1) / kCountRows), (unsigned)F);
  hipLaunchKernelGGL(k_code_counts, grid, dim3(256), 0, st, codes, ld, n, counts);
  return hipGetLastError();
}

// Row-major uint8/uint16 codes -> feature-major tiers (tier_code).
template <typename T>
__global__ __launch_bounds__(256) void k_load_codes(const T *__restrict__ src,
                                                    int64_t n, int32_t F,
                                                    uint8_t *__restrict__ codes,
                                                    int64_t ld, int32_t tiers) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  for (int32_t f = 0; f < F; ++f) {
    const int32_t v = (int32_t)src[i * F + f];
    for (int32_t t = 0; t < tiers; ++t) codes[(int64_t)(t * F + f) * ld + i] = tier_code(v, t);
  }
}

hipError_t launch_load_codes(hipStream_t st, const void *src, int is_u16,
                             int64_t n, int32_t F, uint8_t *codes, int64_t ld, int32_t tiers) {
  if (n <= 0) return hipSuccess;
  const unsigned blocks = (unsigned)((n + 255) / 256);
  if (is_u16)
    hipLaunchKernelGGL(k_load_codes<uint16_t>, dim3(blocks), dim3(256), 0, st,
                       (const uint16_t *)src, n, F, codes, ld, tiers);
  else
    hipLaunchKernelGGL(k_load_codes<uint8_t>, dim3(blocks), dim3(256), 0, st,
                       (const uint8_t *)src, n, F, codes, ld, tiers);
  return hipGetLastError();
}

// Feature-major matrix -> row-major codes: uint8 min(code, 255) (tier 0), or
// uint16 the sum of the tiers (the code, up to 255 * tiers).
template <typename T>
__global__ __launch_bounds__(256) void k_get_codes(const uint8_t *__restrict__ codes,
                                                   int64_t ld, int64_t n, int32_t F,
                                                   int32_t tiers, T *__restrict__ dst) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  for (int32_t f = 0; f < F; ++f) {
    uint32_t v = 0;
    for (int32_t t = 0; t < tiers; ++t) v += codes[(int64_t)(t * F + f) * ld + i];
    dst[i * F + f] = (T)v;
  }
}

hipError_t launch_get_codes(hipStream_t st, const uint8_t *codes, int64_t ld,
                            int64_t n, int32_t F, int32_t tiers, void *dst, int as_u16) {
  if (n <= 0) return hipSuccess;
  const dim3 grid((unsigned)((n + 255) / 256));
  if (as_u16)
    hipLaunchKernelGGL(k_get_codes<uint16_t>, grid, dim3(256), 0, st, codes, ld, n, F, tiers,
                       (uint16_t *)dst);
  else
    hipLaunchKernelGGL(k_get_codes<uint8_t>, grid, dim3(256), 0, st, codes, ld, n, F, 1,
                       (uint8_t *)dst);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Gradients / hessians.
// ---------------------------------------------------------------------------
__device__ __forceinline__ double dev_fixed_mul(unsigned long long max_bits, int32_t bits);

// With dev.max set, the multipliers come from the maxima on the device
// (dev_fixed_mul) instead of g_mul and h_mul.
__global__ __launch_bounds__(256) void k_quantize(const double *__restrict__ g,
                                                  const double *__restrict__ h,
                                                  int64_t n, double g_mul,
                                                  double h_mul, DevScale dev,
                                                  GH *__restrict__ ghq) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  if (dev.max) {
    g_mul = dev_fixed_mul(dev.max[0], dev.bits);
    h_mul = dev_fixed_mul(dev.max[1], dev.bits);
  }
  ghq[i] = make_longlong2(__double2ll_rn(g[i] * g_mul), __double2ll_rn(h[i] * h_mul));
}

hipError_t launch_quantize(hipStream_t st, const double *g, const double *h,
                           int64_t n, double g_mul, double h_mul, GH *ghq, DevScale dev) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_quantize, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     st, g, h, n, g_mul, h_mul, dev, ghq);
  return hipGetLastError();
}

// est:2861 and est:2873-2874: p = 1/(1+exp(-clip(F,-500,500))),
// g = w*(p-y), h = (w*p)*(1-p), each product rounded separately.
__device__ __forceinline__ void logistic_gh(double F, double y, double w,
                                            double &g, double &h) {
  const double Fc = fmin(fmax(F, -500.0), 500.0);
  const double p = 1.0 / (1.0 + exp(-Fc));
  g = __dmul_rn(w, __dsub_rn(p, y));
  h = __dmul_rn(__dmul_rn(w, p), __dsub_rn(1.0, p));
}

// engine.hip::fixed_mul from a maximum held on the device (DevScale):
// 2^(bits - e) with max < 2^e, or 2^bits when the maximum is not positive.
// frexp and ldexp are exact, so the result equals the host's for the same
// maximum.
__device__ __forceinline__ double dev_fixed_mul(unsigned long long max_bits, int32_t bits) {
  const double mx = __longlong_as_double((long long)max_bits);
  if (!(mx > 0.0) || !isfinite(mx)) return ldexp(1.0, bits);
  int e;
  (void)frexp(mx, &e);
  return ldexp(1.0, bits - e);
}

// The fixed point -> value scales 1 / dev_fixed_mul of both maxima.
__device__ __forceinline__ void dev_scales(const DevScale &d, double &g_scale, double &h_scale) {
  g_scale = 1.0 / dev_fixed_mul(d.max[0], d.bits);
  h_scale = 1.0 / dev_fixed_mul(d.max[1], d.bits);
}

__global__ __launch_bounds__(256) void k_grad_hess(const double *__restrict__ F,
                                                   const uint8_t *__restrict__ y,
                                                   int64_t n, double w0, double w1,
                                                   double g_mul, double h_mul,
                                                   GH *__restrict__ ghq) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int yi = y[i];
  double g, h;
  logistic_gh(F[i], (double)yi, yi ? w1 : w0, g, h);
  ghq[i] = make_longlong2(__double2ll_rn(g * g_mul), __double2ll_rn(h * h_mul));
}

hipError_t launch_grad_hess(hipStream_t st, const double *F, const uint8_t *y,
                            int64_t n, double w0, double w1, double g_mul,
                            double h_mul, GH *ghq) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_grad_hess, dim3((unsigned)((n + 255) / 256)), dim3(256),
                     0, st, F, y, n, w0, w1, g_mul, h_mul, ghq);
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void k_grad_hess_f64(const double *__restrict__ F,
                                                       const uint8_t *__restrict__ y,
                                                       int64_t n, double w0,
                                                       double w1, double *__restrict__ g,
                                                       double *__restrict__ h) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int yi = y[i];
  logistic_gh(F[i], (double)yi, yi ? w1 : w0, g[i], h[i]);
}

hipError_t launch_grad_hess_f64(hipStream_t st, const double *F,
                                const uint8_t *y, int64_t n, double w0,
                                double w1, double *g, double *h) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_grad_hess_f64, dim3((unsigned)((n + 255) / 256)),
                     dim3(256), 0, st, F, y, n, w0, w1, g, h);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// In-bag rows in ascending order.  The sampler hands over the reference's
// sample_idx (distinct row ids in shuffled order); a byte flag per row and a
// stream compaction give the same set in ascending order, so the root gather
// streams through each feature column.  The write pass clears the flags for
// the next round.
// ---------------------------------------------------------------------------
constexpr int kFlagBlock = 256;
constexpr int kFlagTile = kFlagBlock * 16;  // flag bytes per block

__global__ __launch_bounds__(256) void k_mark(const int32_t *__restrict__ rows,
                                              int64_t m, uint8_t *__restrict__ flags) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < m) flags[rows[i]] = 1;
}

__device__ __forceinline__ uint32_t byte_sum(uint4 v) {
  // Each byte is 0 or 1: a multiply-by-0x01010101 sums the four bytes of a
  // word into its top byte.
  return ((v.x * 0x01010101u) >> 24) + ((v.y * 0x01010101u) >> 24) +
         ((v.z * 0x01010101u) >> 24) + ((v.w * 0x01010101u) >> 24);
}

__global__ __launch_bounds__(kFlagBlock) void k_flag_count(const uint8_t *__restrict__ flags,
                                                           int32_t *__restrict__ block_cnt) {
  __shared__ uint32_t tmp[kFlagBlock / 64];
  const uint4 v = reinterpret_cast<const uint4 *>(flags)[(int64_t)blockIdx.x * kFlagBlock + threadIdx.x];
  uint32_t total;
  block_excl_scan<kFlagBlock>(byte_sum(v), tmp, total);
  if (threadIdx.x == 0) block_cnt[blockIdx.x] = (int32_t)total;
}

__global__ __launch_bounds__(kFlagBlock) void k_block_scan(int32_t *__restrict__ cnt_to_off,
                                                           int32_t nb) {
  __shared__ uint32_t tmp[kFlagBlock / 64];
  uint32_t carry = 0;
  for (int base = 0; base < nb; base += kFlagBlock) {
    const int b = base + (int)threadIdx.x;
    const uint32_t v = b < nb ? (uint32_t)cnt_to_off[b] : 0u;
    uint32_t total;
    const uint32_t pre = block_excl_scan<kFlagBlock>(v, tmp, total);
    if (b < nb) cnt_to_off[b] = (int32_t)(carry + pre);
    carry += total;
  }
}

__global__ __launch_bounds__(kFlagBlock) void k_flag_write(uint8_t *__restrict__ flags,
                                                           const int32_t *__restrict__ block_off,
                                                           int32_t *__restrict__ out) {
  __shared__ uint32_t tmp[kFlagBlock / 64];
  uint4 *fp = reinterpret_cast<uint4 *>(flags) + (int64_t)blockIdx.x * kFlagBlock + threadIdx.x;
  const uint4 v = *fp;
  uint32_t total;
  uint32_t o = (uint32_t)block_off[blockIdx.x] +
               block_excl_scan<kFlagBlock>(byte_sum(v), tmp, total);
  const int64_t base = ((int64_t)blockIdx.x * kFlagBlock + threadIdx.x) * 16;
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int b = 0; b < 4; ++b)
      if ((w[q] >> (8 * b)) & 1u) out[o++] = (int32_t)(base + 4 * q + b);
  if (v.x | v.y | v.z | v.w) *fp = make_uint4(0, 0, 0, 0);
}

// flags: n_pad bytes (multiple of kFlagTile), zero on entry and on exit.
// `marked`: the rows' flags are already set (launch_fisher_yates did it).
hipError_t launch_sort_rows(hipStream_t st, const int32_t *rows, int64_t m,
                            uint8_t *flags, int64_t n_pad, int32_t *block_tmp,
                            int32_t *out, bool marked) {
  if (m <= 0) return hipSuccess;
  const unsigned nb = (unsigned)(n_pad / kFlagTile);
  if (!marked)
    hipLaunchKernelGGL(k_mark, dim3((unsigned)((m + 255) / 256)), dim3(256), 0, st, rows, m,
                       flags);
  hipLaunchKernelGGL(k_flag_count, dim3(nb), dim3(kFlagBlock), 0, st, flags, block_tmp);
  hipLaunchKernelGGL(k_block_scan, dim3(1), dim3(kFlagBlock), 0, st, block_tmp, (int32_t)nb);
  hipLaunchKernelGGL(k_flag_write, dim3(nb), dim3(kFlagBlock), 0, st, flags, block_tmp, out);
  return hipGetLastError();
}

int64_t sort_rows_flag_bytes(int64_t n) {
  return (n + kFlagTile - 1) / kFlagTile * kFlagTile;
}

// ---------------------------------------------------------------------------
// Root gather: the tree's in-bag rows (ascending ids from the sampler, or the
// caller's order) -> compact feature-major set 0.  One thread fills 4
// consecutive compact rows, so every store is a dword.  Row ids are kept
// (rid_c) only when a caller reads the partition back.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_gather_root(
    const uint8_t *__restrict__ codes, int64_t ld, const int32_t *__restrict__ feat,
    int32_t F_sel, const int32_t *__restrict__ rows32,
    const int64_t *__restrict__ rows64, int64_t m, const GH *__restrict__ ghq,
    uint8_t *__restrict__ codes_c, int64_t ld_c, GH *__restrict__ gh_c,
    int32_t *__restrict__ rid_c, int64_t pad_to, NodeSeg *__restrict__ segs,
    int32_t *__restrict__ hist_node) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  // The root's segment and histogram slot.
  if (t == 0) {
    NodeSeg r;
    r.start = 0;
    r.count = m;
    r.valid = 1;
    r.is_small = 1;
    segs[0] = r;
    hist_node[0] = 0;
  }
  const int64_t k0 = t * 4;
  if (k0 >= pad_to) return;
  int32_t r[4];
  bool ok[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    ok[k] = (k0 + k) < m;
    r[k] = ok[k] ? (rows32 ? rows32[k0 + k] : (int32_t)rows64[k0 + k]) : 0;
    gh_c[k0 + k] = ok[k] ? ghq[r[k]] : make_longlong2(0, 0);
    if (rid_c) rid_c[k0 + k] = ok[k] ? r[k] : -1;
  }
  for (int32_t f = 0; f < F_sel; ++f) {
    const uint8_t *col = codes + (int64_t)feat[f] * ld;
    uint32_t w = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      w |= (ok[k] ? (uint32_t)col[r[k]] : 0u) << (8 * k);
    *reinterpret_cast<uint32_t *>(codes_c + (int64_t)f * ld_c + k0) = w;
  }
}

// The in-bag rows' codes alone, for a round whose rows are known before its
// gradients (the codes are gathered while the previous tree is built).
__global__ __launch_bounds__(256) void k_gather_codes(
    const uint8_t *__restrict__ codes, int64_t ld, const int32_t *__restrict__ feat,
    int32_t F_sel, const int32_t *__restrict__ rows32, int64_t m,
    uint8_t *__restrict__ codes_c, int64_t ld_c, int64_t pad_to) {
  const int64_t k0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (k0 >= pad_to) return;
  int32_t r[4];
  bool ok[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    ok[k] = (k0 + k) < m;
    r[k] = ok[k] ? rows32[k0 + k] : 0;
  }
  for (int32_t f = 0; f < F_sel; ++f) {
    const uint8_t *col = codes + (int64_t)feat[f] * ld;
    uint32_t w = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      w |= (ok[k] ? (uint32_t)col[r[k]] : 0u) << (8 * k);
    *reinterpret_cast<uint32_t *>(codes_c + (int64_t)f * ld_c + k0) = w;
  }
}

// The in-bag rows' fixed-point (g, h) straight from F and y (k_grad_hess's
// arithmetic, for these rows only), the root's segment and, when plan_src is
// given, the root's LevelPlan (copied to plan_dst).
__global__ __launch_bounds__(256) void k_gather_gh(
    const double *__restrict__ F, const uint8_t *__restrict__ y,
    const int32_t *__restrict__ rows32, int64_t m, double w0, double w1, double g_mul,
    double h_mul, DevScale dev, GH *__restrict__ gh_c, int64_t pad_to,
    NodeSeg *__restrict__ segs, int32_t *__restrict__ hist_node,
    const LevelPlan *__restrict__ plan_src, LevelPlan *__restrict__ plan_dst) {
  const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (dev.max) {
    g_mul = dev_fixed_mul(dev.max[0], dev.bits);
    h_mul = dev_fixed_mul(dev.max[1], dev.bits);
  }
  if (k == 0) {
    if (plan_src) *plan_dst = *plan_src;
    NodeSeg r;
    r.start = 0;
    r.count = m;
    r.valid = 1;
    r.is_small = 1;
    segs[0] = r;
    hist_node[0] = 0;
  }
  if (k >= pad_to) return;
  GH q = make_longlong2(0, 0);
  if (k < m) {
    const int32_t i = rows32[k];
    const int yi = y[i];
    double g, h;
    logistic_gh(F[i], (double)yi, yi ? w1 : w0, g, h);
    q = make_longlong2(__double2ll_rn(g * g_mul), __double2ll_rn(h * h_mul));
  }
  gh_c[k] = q;
}

hipError_t launch_gather_codes(hipStream_t st, const uint8_t *codes, int64_t ld,
                               const int32_t *feat, int32_t F_sel, const int32_t *rows32,
                               int64_t m, uint8_t *codes_c, int64_t ld_c, int64_t pad_to) {
  const int64_t threads = (pad_to + 3) / 4;
  if (threads <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_gather_codes, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     st, codes, ld, feat, F_sel, rows32, m, codes_c, ld_c, pad_to);
  return hipGetLastError();
}

hipError_t launch_gather_gh(hipStream_t st, const double *F, const uint8_t *y,
                            const int32_t *rows32, int64_t m, double w0, double w1,
                            double g_mul, double h_mul, DevScale dev, GH *gh_c,
                            int64_t pad_to, NodeSeg *segs, int32_t *hist_node,
                            const LevelPlan *plan_src, LevelPlan *plan_dst) {
  if (pad_to <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_gather_gh, dim3((unsigned)((pad_to + 255) / 256)), dim3(256), 0, st,
                     F, y, rows32, m, w0, w1, g_mul, h_mul, dev, gh_c, pad_to, segs,
                     hist_node, plan_src, plan_dst);
  return hipGetLastError();
}

hipError_t launch_gather_root(hipStream_t st, const uint8_t *codes, int64_t ld,
                              const int32_t *feat, int32_t F_sel,
                              const int32_t *rows32, const int64_t *rows64,
                              int64_t m, const GH *ghq, uint8_t *codes_c,
                              int64_t ld_c, GH *gh_c, int32_t *rid_c,
                              int64_t pad_to, NodeSeg *segs, int32_t *hist_node) {
  const int64_t threads = (pad_to + 3) / 4;
  if (threads <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_gather_root, dim3((unsigned)((threads + 255) / 256)),
                     dim3(256), 0, st, codes, ld, feat, F_sel, rows32, rows64, m,
                     ghq, codes_c, ld_c, gh_c, rid_c, pad_to, segs, hist_node);
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void k_iota(int32_t *__restrict__ a, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    a[i] = (int32_t)i;
}

static unsigned elementwise_blocks(int64_t n) {
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>((n + 255) / 256, 65536));
}

hipError_t launch_iota(hipStream_t st, int32_t *a, int64_t n) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_iota, dim3(elementwise_blocks(n)), dim3(256), 0, st, a, n);
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void k_fill_f64(double *__restrict__ a, int64_t n, double v) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    a[i] = v;
}

hipError_t launch_fill_f64(hipStream_t st, double *a, int64_t n, double v) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_fill_f64, dim3(elementwise_blocks(n)), dim3(256), 0, st, a, n, v);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Histogram build (est:581-596, est:722-737).
//
// A work item is one row tile of a node and one chunk of FC selected
// features.  Its private histogram [FC][g[256], h[256]] int64 lives in LDS
// (4 KB per feature, so several blocks share a CU).  Keeping the g and h
// sums in separate arrays spreads a wave's 64 adds over all LDS banks
// (interleaved [bin][g,h] pairs use half of them): 2.17 instead of 1.70
// (g,h) updates per clock per CU on MI355X with uniform random bins.
//
// The block stores its histogram, as [bin][g,h], into the task's slot of
// the partial buffer with plain coalesced stores; k_reduce_split then sums a
// node's partials into its histogram.  (Adding every block's bins into the
// node's histogram with device-scope atomics made one memory-side atomic
// per bin per block: as many bytes as the codes at 1M rows.)  A thread takes 16
// consecutive rows: 128 bytes of (g,h), then per feature one 16-byte load of
// packed codes and 32 64-bit LDS adds.  Rows outside the tile add zero.  The
// block then adds its non-zero bins into the node's histogram in HBM.
//
// Blocks are numbered so that all feature chunks of one row tile get the
// same blockIdx modulo 8: blocks are dealt to the 8 XCDs round-robin, so
// the tile's (g,h) rows are fetched from HBM once and then hit that XCD's L2.
// Splitting features across blocks (rather than rows) keeps the number of
// flushed bins, rows/tile_rows * F_sel * 512, small.
// ---------------------------------------------------------------------------
constexpr int kHistBlock = 256;
constexpr int kHistRows = 16;  // rows per thread per step

// With C > 1 copies, lane l adds into copy l % C, stored at bin * C + c:
// the copies of one bin sit in C consecutive words, so lanes of different
// copies never meet in an LDS bank whatever their bins (3.13 instead of 2.18
// (g,h) updates per clock per CU for C = 8 on MI355X).
// Sums over tiles t = t_first, t_first + stride, ... < t1 of the two
// adjacent counts cnt[4t], cnt[4t + 1], eight loads in flight per pass.
__device__ __forceinline__ void strided_side_counts(const int32_t *__restrict__ cnt,
                                                    int32_t t_first, int32_t t1, int32_t stride,
                                                    long long &a, long long &b) {
  a = 0;
  b = 0;
  for (int32_t t = t_first; t < t1; t += 8 * stride) {
    int2 v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int32_t te = t + e * stride;
      v[e] = te < t1 ? *reinterpret_cast<const int2 *>(cnt + 4 * (int64_t)te) : make_int2(0, 0);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      a += v[e].x;
      b += v[e].y;
    }
  }
}

// The children of parent p, whose split sends nl of its rows left and nr
// right: their segments (left first, from the parent's start), whether the
// split is kept (est:678-683) and which child is the smaller one
// (est:701-709), whose histogram is built.
__device__ __forceinline__ void write_children(const PartParent &P, int32_t p, int64_t nl,
                                               int64_t nr, int32_t min_samples_leaf,
                                               int64_t *__restrict__ parent_nleft,
                                               NodeSeg *__restrict__ segs,
                                               int32_t *__restrict__ hist_node) {
  const bool ok = nl >= min_samples_leaf && nr >= min_samples_leaf;
  const bool left_small = nl <= nr;
  parent_nleft[p] = nl;
  NodeSeg Ls, Rs;
  Ls.start = P.start;
  Ls.count = nl;
  Ls.valid = ok ? 1 : 0;
  Ls.is_small = left_small ? 1 : 0;
  Rs.start = P.start + nl;
  Rs.count = nr;
  Rs.valid = ok ? 1 : 0;
  Rs.is_small = left_small ? 0 : 1;
  segs[P.left_id] = Ls;
  segs[P.right_id] = Rs;
  hist_node[p] = ok ? (left_small ? P.left_id : P.right_id) : -1;
}

// Tasks of histogram reference p that hold rows: at most the planned tasks,
// and none past the node's last row.
__device__ __forceinline__ int32_t hist_tasks_with_rows(const int32_t *__restrict__ hist_begin,
                                                        int32_t p, int64_t count,
                                                        int32_t tile_rows) {
  const int64_t with_rows = div_pos(count + tile_rows - 1, tile_rows);
  return (int32_t)min((int64_t)(hist_begin[p + 1] - hist_begin[p]), with_rows);
}

// In place (an in-place level's task: a tile of its parent's segment, of
// which only the rows going to the smaller child are added).  Each wave
// takes 64 x kSpanRows rows at a time: every lane loads its rows' codes of
// the split feature and of the block's features (one load per feature, as
// the compact path), stores each row's codes as one word per four features
// in the wave's part of LDS, and the wave lists the rows to add (a prefix
// sum over its lanes).  The lanes then take the listed rows in turn, with
// one (g,h) load each, so that every LDS add has all lanes active whatever
// share of the rows is added.  A wave reads only what it wrote itself, and
// a wave's LDS operations complete in issue order, so no barrier is needed
// between its steps.
constexpr int kSpanRows = 8;
constexpr int kSpanWave = 64 * kSpanRows;        // rows per wave and step
constexpr int kSpanStep = kHistBlock * kSpanRows;  // rows per block and step

// A lane's codes of one step: the split feature's and the block's features'
// for its kSpanRows rows (group g of the tile's groups g < g1).
template <int FC>
struct SpanCodes {
  uint2 sv;
  uint2 cv[FC];
};

template <int FC>
__device__ __forceinline__ void span_load(SpanCodes<FC> &L, const uint8_t *__restrict__ codes_c,
                                          int64_t ld_c, const uint8_t *__restrict__ scol, int f0,
                                          int nf, int64_t g, int64_t g1) {
  if (g < g1) {
    const int64_t row = g * kSpanRows;
    L.sv = *reinterpret_cast<const uint2 *>(scol + row);
#pragma unroll
    for (int u = 0; u < FC; ++u)
      L.cv[u] = u < nf ? *reinterpret_cast<const uint2 *>(codes_c + (int64_t)(f0 + u) * ld_c + row)
                       : make_uint2(0u, 0u);
  }
}

// The wave's groups of kSpanRows rows are every fourth run of 64 groups of
// the tile, from group r0 / kSpanRows + 64 * wave, whose codes the caller
// has loaded into L; the codes of the wave's next step are loaded before
// this step's listed rows are added.
template <int FC, int C>
__device__ __forceinline__ void hist_rows_span(
    unsigned long long *lh, uint32_t *stage, uint16_t *mlist,
    const uint8_t *__restrict__ codes_c, int64_t ld_c, const GH *__restrict__ gh_c, int f0,
    int nf, const uint32_t (&lim)[FC], const uint32_t (&hb)[FC], long long (&ag)[FC],
    long long (&ah)[FC], int64_t r0, int64_t r1, const uint8_t *__restrict__ scol,
    uint32_t sbin, bool sright, SpanCodes<FC> &L) {
  constexpr int kW = (FC + 3) / 4;  // LDS words per row
  const int lane = lane_id(), wave = (int)(threadIdx.x >> 6);
  const int copy = lane & (C - 1);
  uint32_t *wst = stage + wave * kSpanWave;  // this wave's rows: word q at q * kSpanStep
  uint16_t *wl = mlist + wave * kSpanWave;
  const int64_t g0 = r0 / kSpanRows, g1 = (r1 + kSpanRows - 1) / kSpanRows;
  for (int64_t gb = g0 + (int64_t)wave * 64; gb < g1; gb += (int64_t)kHistBlock) {
    const int64_t g = gb + lane;
    const int64_t row = g * kSpanRows;
    uint32_t mem = 0u;
    if (g < g1) {
      const uint2 sv = L.sv;
      uint2 cv[FC];
#pragma unroll
      for (int u = 0; u < FC; ++u) cv[u] = L.cv[u];
      const uint32_t sw[2] = {sv.x, sv.y};
#pragma unroll
      for (int k = 0; k < kSpanRows; ++k) {
        const bool right = ((sw[k >> 2] >> (8 * (k & 3))) & 255u) > sbin;
        const bool in = row + k >= r0 && row + k < r1;
        mem |= ((in && right == sright) ? 1u : 0u) << k;
      }
#pragma unroll
      for (int q = 0; q < kW; ++q) {
        uint32_t w[kSpanRows];
#pragma unroll
        for (int k = 0; k < kSpanRows; ++k) {
          w[k] = 0u;
#pragma unroll
          for (int u = 4 * q; u < FC && u < 4 * q + 4; ++u) {
            const uint32_t cw = (k < 4) ? cv[u].x : cv[u].y;
            w[k] |= ((cw >> (8 * (k & 3))) & 255u) << (8 * (u - 4 * q));
          }
        }
        uint4 *sp = reinterpret_cast<uint4 *>(wst + q * kSpanStep + kSpanRows * lane);
        sp[0] = make_uint4(w[0], w[1], w[2], w[3]);
        sp[1] = make_uint4(w[4], w[5], w[6], w[7]);
      }
    }
    if (gb + kHistBlock < g1) span_load<FC>(L, codes_c, ld_c, scol, f0, nf, gb + kHistBlock + lane, g1);
    const uint32_t cnt = (uint32_t)__builtin_popcount(mem);
    const uint32_t incl = wave_incl_scan<uint32_t>(cnt);
    const int nm = (int)wave_lane(incl, 63);
    uint32_t at = incl - cnt;
#pragma unroll
    for (int k = 0; k < kSpanRows; ++k)
      if ((mem >> k) & 1u) wl[at++] = (uint16_t)(kSpanRows * lane + k);
    __builtin_amdgcn_wave_barrier();
    // The listed rows, four per lane in flight.
    const int64_t base = gb * kSpanRows;
    for (int j0 = lane; j0 < nm; j0 += 4 * 64) {
      long long gq[4], hq[4];
      uint32_t ww[4][kW];
      bool ok[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int j = j0 + e * 64;
        ok[e] = j < nm;
        const int rl = ok[e] ? (int)wl[j] : 0;
        const GH v = ok[e] ? gh_c[base + rl] : GH{0, 0};
        gq[e] = v.x;
        hq[e] = v.y;
#pragma unroll
        for (int q = 0; q < kW; ++q) ww[e][q] = wst[q * kSpanStep + rl];
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (!ok[e]) continue;
#pragma unroll
        for (int u = 0; u < FC; ++u) {
          if (u >= nf) break;
          unsigned long long *hf = lh + u * kHistPerFeat * C + copy;
          const uint32_t bin = min((ww[e][u >> 2] >> (8 * (u & 3))) & 255u, lim[u]);
          // The feature's most frequent bin is summed in registers.
          if (bin == hb[u]) {
            ag[u] += gq[e];
            ah[u] += hq[e];
          } else {
            __hip_atomic_fetch_add(hf + bin * C, (unsigned long long)gq[e], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_WORKGROUP);
            __hip_atomic_fetch_add(hf + (kBins + bin) * C, (unsigned long long)hq[e],
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
          }
        }
      }
    }
    __builtin_amdgcn_wave_barrier();  // (the next step's stores follow these reads)
  }
}

// SPAN: the task tiles the segment of parent span[task.ref] and adds the
// rows whose code of the parent's split feature sends them to the smaller
// child hist_node[task.ref] (hist_rows_span).
template <int FC, int C, bool SPAN>
__device__ __forceinline__ void hist_item(
    unsigned long long *lh, uint32_t *stage, uint16_t *mlist,
    const uint8_t *__restrict__ codes_c, int64_t ld_c,
    const GH *__restrict__ gh_c, const HistTask task, int32_t ti, int chunk,
    int32_t *__restrict__ hist_node, const int32_t *__restrict__ hist_begin,
    NodeSeg *__restrict__ segs, const SpanLevel &span, long long (*sred)[kHistBlock / 64],
    const int32_t *__restrict__ nb_sel, const int32_t *__restrict__ hot_sel,
    int32_t F_sel, int32_t tile_rows, unsigned long long *__restrict__ part,
    unsigned long long *__restrict__ pool, int64_t node_stride) {
  int32_t node = -1;
  int64_t s0, sn;  // the rows the tasks of this reference tile
  const uint8_t *scol = nullptr;
  uint32_t sbin = 0u;
  PartParent P;
  if constexpr (SPAN) {
    P = span.parents[task.ref];
    s0 = P.start;
    sn = P.count;
    scol = codes_c + (int64_t)P.fpos * ld_c;
    sbin = (uint32_t)P.bin;
  } else {
    node = hist_node[task.ref];
    if (node < 0) return;
    const NodeSeg seg = segs[node];
    if (!seg.valid) return;
    s0 = seg.start;
    sn = seg.count;
  }
  const int64_t r0 = s0 + (int64_t)task.tile * tile_rows;
  const int64_t rend = s0 + sn;
  if (r0 >= rend) return;  // (never a parent's first task: it writes the children)
  const int64_t r1 = min(rend, r0 + (int64_t)tile_rows);
  const int f0 = chunk * FC;
  const int nf = min(FC, F_sel - f0);
  // In place: the first step's codes, then the children's sizes (the
  // parent's tiles' counts of runs 0, left, and 1, right), both in flight
  // together; every block of the parent sums them.
  SpanCodes<FC> L;
  if constexpr (SPAN) {
    span_load<FC>(L, codes_c, ld_c, scol, f0, nf,
                  r0 / kSpanRows + 64 * (int64_t)(threadIdx.x >> 6) + lane_id(),
                  (r1 + kSpanRows - 1) / kSpanRows);
    const int32_t t0 = P.tile0, t1 = P.tile1;
    long long nl, nr;
    strided_side_counts(span.tile_cnt, t0 + (int32_t)threadIdx.x, t1, kHistBlock, nl, nr);
    nl = wave_sum(nl);
    nr = wave_sum(nr);
    if (lane_id() == 0) {
      sred[0][threadIdx.x >> 6] = nl;
      sred[1][threadIdx.x >> 6] = nr;
    }
  }
  uint32_t lim[FC], hb[FC];
  long long ag[FC], ah[FC];
#pragma unroll
  for (int u = 0; u < FC; ++u) {
    lim[u] = (u < nf) ? (uint32_t)(nb_sel[f0 + u] - 1) : 0u;
    // hot_sel < 0 (no frequent bin) becomes 0xffffffff: never matches.
    hb[u] = (u < nf) ? (uint32_t)hot_sel[f0 + u] : 0xffffffffu;
    ag[u] = 0;
    ah[u] = 0;
  }
  for (int i = threadIdx.x; i < FC * kHistPerFeat * C; i += kHistBlock) lh[i] = 0ull;
  __syncthreads();
  bool sright = false;
  if constexpr (SPAN) {
    long long nl = 0, nr = 0;
#pragma unroll
    for (int w = 0; w < kHistBlock / 64; ++w) {
      nl += sred[0][w];
      nr += sred[1][w];
    }
    // The parent's first block writes the children's segments, whether the
    // split is kept and the smaller child (as k_last_level does).
    if (task.tile == 0 && chunk == 0 && threadIdx.x == 0)
      write_children(P, task.ref, nl, nr, span.min_samples_leaf, span.parent_nleft, segs,
                     hist_node);
    if (nl < span.min_samples_leaf || nr < span.min_samples_leaf) {  // split not kept
      __syncthreads();  // sred is rewritten by the block's next item
      return;
    }
    node = nl <= nr ? P.left_id : P.right_id;
    sright = node != P.left_id;
  }
  const int copy = lane_id() & (C - 1);

  if constexpr (SPAN) {
    hist_rows_span<FC, C>(lh, stage, mlist, codes_c, ld_c, gh_c, f0, nf, lim, hb, ag, ah, r0, r1,
                          scol, sbin, sright, L);
  } else {
  const int64_t g0 = r0 >> 4, g1 = (r1 + 15) >> 4;
  for (int64_t g = g0 + threadIdx.x; g < g1; g += kHistBlock) {
    const int64_t row = g << 4;
    // Every load of the step first: (g,h) of the 16 rows, then each
    // feature's 16 codes.
    long long gq[kHistRows], hq[kHistRows];
#pragma unroll
    for (int q = 0; q < kHistRows; ++q) {
      const GH v = gh_c[row + q];
      gq[q] = v.x;
      hq[q] = v.y;
    }
    uint4 cv[FC];
#pragma unroll
    for (int u = 0; u < FC; ++u)
      if (u < nf) cv[u] = *reinterpret_cast<const uint4 *>(codes_c + (int64_t)(f0 + u) * ld_c + row);
    // Rows [klo, khi) of the group lie in the tile: all 16 except at a
    // node's first and last groups.  Rows outside add zero.
    const int klo = (int)max((int64_t)0, min((int64_t)kHistRows, r0 - row));
    const int khi = (int)max((int64_t)0, min((int64_t)kHistRows, r1 - row));
    if (klo != 0 || khi != kHistRows) {
#pragma unroll
      for (int k = 0; k < kHistRows; ++k) {
        const bool in = k >= klo && k < khi;
        gq[k] = in ? gq[k] : 0;
        hq[k] = in ? hq[k] : 0;
      }
    }
#pragma unroll
    for (int u = 0; u < FC; ++u) {
      if (u < nf) {
        const uint32_t cw[4] = {cv[u].x, cv[u].y, cv[u].z, cv[u].w};
        unsigned long long *hf = lh + u * kHistPerFeat * C + copy;
        if (hb[u] == 0xffffffffu) {
          // No frequent bin (the same for the whole block): every row is
          // one pair of LDS adds, without a branch.
#pragma unroll
          for (int k = 0; k < kHistRows; ++k) {
            const uint32_t bin = min((cw[k >> 2] >> (8 * (k & 3))) & 255u, lim[u]);
            __hip_atomic_fetch_add(hf + bin * C, (unsigned long long)gq[k],
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            __hip_atomic_fetch_add(hf + (kBins + bin) * C, (unsigned long long)hq[k],
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
          }
        } else {
#pragma unroll
          for (int k = 0; k < kHistRows; ++k) {
            const uint32_t bin = min((cw[k >> 2] >> (8 * (k & 3))) & 255u, lim[u]);
            // The feature's most frequent bin (NaN, zeros) is summed in
            // registers: same-address LDS atomics within a wave serialise.
            if (bin == hb[u]) {
              ag[u] += gq[k];
              ah[u] += hq[k];
            } else {
              __hip_atomic_fetch_add(hf + bin * C, (unsigned long long)gq[k],
                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
              __hip_atomic_fetch_add(hf + (kBins + bin) * C, (unsigned long long)hq[k],
                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
          }
        }
      }
    }
  }
  }
  // Hot-bin sums: wave reduction, then one LDS add per wave.
#pragma unroll
  for (int u = 0; u < FC; ++u) {
    const long long a = wave_sum(ag[u]), c = wave_sum(ah[u]);
    if (u < nf && hb[u] != 0xffffffffu && lane_id() == 0 && (a | c)) {
      __hip_atomic_fetch_add(lh + u * kHistPerFeat * C + hb[u] * C, (unsigned long long)a,
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      __hip_atomic_fetch_add(lh + u * kHistPerFeat * C + (kBins + hb[u]) * C,
                             (unsigned long long)c, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  }
  __syncthreads();
  // Partial of task ti, features f0 .. f0+nf-1, as [bin][g,h]; a node built
  // by this one task gets it as its histogram directly (k_reduce_split reads
  // such nodes).
  unsigned long long *dst =
      hist_tasks_with_rows(hist_begin, task.ref, sn, tile_rows) == 1
          ? pool + (int64_t)node * node_stride + (int64_t)f0 * kHistPerFeat
          : part + ((int64_t)ti * F_sel + f0) * kHistPerFeat;
  for (int i = threadIdx.x; i < nf * kHistPerFeat; i += kHistBlock) {
    const int j = i & (kHistPerFeat - 1);
    const unsigned long long *src = lh + ((i - j) + (j & 1) * kBins + (j >> 1)) * C;
    unsigned long long v = 0ull;
#pragma unroll
    for (int c = 0; c < C; ++c) v += src[c];
    dst[i] = v;
  }
  __syncthreads();  // lh is cleared again by the block's next item
}

// (In place, five waves per SIMD: the listed rows' loads need the waves.)
template <int FC, int C, bool SPAN>
__global__ __launch_bounds__(kHistBlock) __attribute__((amdgpu_waves_per_eu(SPAN ? 5 : 1)))
void k_hist(
    const uint8_t *__restrict__ codes_c, int64_t ld_c,
    const GH *__restrict__ gh_c, const HistTask *__restrict__ tasks,
    const LevelPlan *__restrict__ plan, int32_t *__restrict__ hist_node,
    const int32_t *__restrict__ hist_begin, NodeSeg *__restrict__ segs, SpanLevel span,
    const int32_t *__restrict__ nb_sel,
    const int32_t *__restrict__ hot_sel, int32_t F_sel, int32_t nchunks,
    unsigned long long *__restrict__ part, unsigned long long *__restrict__ pool,
    int64_t node_stride, unsigned long long *__restrict__ ktime) {
  __shared__ unsigned long long lh[FC * kHistPerFeat * C];
  // In place: each step's codes (one word per four features and row) and
  // listed rows.
  __shared__ __align__(16) uint32_t stage[SPAN ? (FC + 3) / 4 : 1][SPAN ? kSpanStep : 1];
  __shared__ uint16_t mlist[SPAN ? kSpanStep : 1];
  __shared__ long long sred[2][kHistBlock / 64];
  const int32_t n_tasks = plan->n_hist;
  const int32_t tile_rows = plan->tile_rows;
  // Optional timing: each block's start and end on the constant-rate clock,
  // one plain store each into its own pair (the launch's time is the first
  // start to the last end).
  if (ktime && threadIdx.x == 0) ktime[2 * blockIdx.x] = (unsigned long long)wall_clock64();
  // The grid is a multiple of 8 * nchunks, so every block keeps its XCD
  // (b & 7) and feature chunk as it strides.
  for (int b = (int)blockIdx.x;; b += (int)gridDim.x) {
    const int j = b >> 3;
    const int ti = (j / nchunks) * 8 + (b & 7);
    if ((j / nchunks) * 8 >= n_tasks) break;
    if (ti >= n_tasks) continue;
    hist_item<FC, C, SPAN>(lh, &stage[0][0], mlist, codes_c, ld_c, gh_c, tasks[ti], ti,
                           j % nchunks, hist_node, hist_begin, segs, span, sred, nb_sel, hot_sel,
                           F_sel, tile_rows, part, pool, node_stride);
  }
  if (ktime) {
    __syncthreads();  // every wave's stores issued
    if (threadIdx.x == 0) ktime[2 * blockIdx.x + 1] = (unsigned long long)wall_clock64();
  }
}

int hist_blocks(int32_t n_tasks, int32_t nchunks) {
  return ((n_tasks + 7) / 8) * 8 * nchunks;
}

hipError_t launch_hist(hipStream_t st, const uint8_t *codes_c, int64_t ld_c,
                       const GH *gh_c, const HistTask *tasks,
                       const LevelPlan *plan, int32_t max_tasks,
                       int32_t *hist_node, const int32_t *hist_begin,
                       NodeSeg *segs,
                       const int32_t *nb_sel, const int32_t *hot_sel,
                       int32_t F_sel, int32_t fchunk, int32_t copies,
                       unsigned long long *part, unsigned long long *pool,
                       int64_t node_stride, const SpanLevel *span,
                       unsigned long long *ktime) {
  if (max_tasks <= 0) return hipSuccess;
  const SpanLevel sp = span ? *span : SpanLevel{};
  const int32_t nchunks = (F_sel + fchunk - 1) / fchunk;
  const dim3 grid((unsigned)hist_blocks(max_tasks, nchunks));
#define BSSCL_HIST(FC, C)                                                                    \
  if (span)                                                                                  \
    hipLaunchKernelGGL((k_hist<FC, C, true>), grid, dim3(kHistBlock), 0, st, codes_c, ld_c, gh_c, \
                       tasks, plan, hist_node, hist_begin, segs, sp, nb_sel, hot_sel, F_sel,    \
                       nchunks, part, pool, node_stride, ktime);                              \
  else                                                                                       \
    hipLaunchKernelGGL((k_hist<FC, C, false>), grid, dim3(kHistBlock), 0, st, codes_c, ld_c,   \
                       gh_c, tasks, plan, hist_node, hist_begin, segs, sp, nb_sel, hot_sel,    \
                       F_sel, nchunks, part, pool, node_stride, ktime)
  // LDS per block: fchunk * copies * 8 KB (at most 32 KB).
  switch (fchunk * 16 + copies) {
    case 1 * 16 + 1: BSSCL_HIST(1, 1); break;
    case 1 * 16 + 4: BSSCL_HIST(1, 4); break;
    case 1 * 16 + 8: BSSCL_HIST(1, 8); break;
    case 2 * 16 + 1: BSSCL_HIST(2, 1); break;
    case 2 * 16 + 4: BSSCL_HIST(2, 4); break;
    case 4 * 16 + 1: BSSCL_HIST(4, 1); break;
    case 8 * 16 + 1: BSSCL_HIST(8, 1); break;
    default: return hipErrorInvalidValue;
  }
#undef BSSCL_HIST
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Partition (est:662-674, made stable): count, scan, scatter.  A tile is 256
// threads x R rows (R = 4, 8 or 16, chosen per tree: 1024 to 4096 rows)
// starting at a 16-row boundary; rows of the tile outside its group's
// segment are masked.  A thread reads its R rows' codes of a feature as one
// R-byte load.  A group (PartGroup) sends each row by up to two splits to
// one of four runs, 2 * side + (right child ? 1 : 0), so one pass can move
// rows down two tree levels; each run keeps the input order.
// ---------------------------------------------------------------------------
constexpr int kPartBlock = 256;

template <int R> struct CodesR;  // R consecutive codes as one load
template <> struct CodesR<4> { using T = uint32_t; };
template <> struct CodesR<8> { using T = uint2; };
template <> struct CodesR<16> { using T = uint4; };

template <int R>
union CodeWords {
  typename CodesR<R>::T v;
  uint32_t w[R / 4];
};

template <int R>
__device__ __forceinline__ CodeWords<R> zero_codes() {
  CodeWords<R> c;
#pragma unroll
  for (int k = 0; k < R / 4; ++k) c.w[k] = 0u;
  return c;
}

// The R codes of rows row .. row+R-1 of one feature column; a group wholly
// outside [lo, hi) is not read (it may lie past the buffer).
template <int R>
__device__ __forceinline__ CodeWords<R> load_codes(const uint8_t *__restrict__ col, int64_t row,
                                                   int64_t lo, int64_t hi) {
  CodeWords<R> c;
  if (row < hi && row + R > lo) {
    c.v = *reinterpret_cast<const typename CodesR<R>::T *>(col + row);
  } else {
    c = zero_codes<R>();
  }
  return c;
}

// Tile t's group: groups[g], or (without groups) parent g as the only side.
__device__ __forceinline__ PartGroup tile_group(const PartGroup *__restrict__ groups,
                                                const PartParent *__restrict__ parents,
                                                int32_t g) {
  if (groups) return groups[g];
  const PartParent P = parents[g];
  PartGroup G;
  G.start = P.start;
  G.count = P.count;
  G.fpos = -1;
  G.bin = 0;
  G.par[0] = g;
  G.par[1] = -1;
  return G;
}

// A tile's routing: its group's rows of the tile [lo, hi), the side
// parents' splits and the codes each split reads for this thread's rows.
template <int R>
struct Route {
  int64_t lo, hi;
  CodeWords<R> c0, ca, cb;  // the group's split, side 0's and side 1's
  uint32_t bin_a, bin_b;
};

template <int R>
__device__ __forceinline__ Route<R> route_load(const uint8_t *__restrict__ codes_c, int64_t ld_c,
                                               const PartTile &t, const PartGroup &G,
                                               const PartParent &Pa, const PartParent &Pb,
                                               int64_t row) {
  Route<R> q;
  q.lo = max(t.row0, G.start);
  q.hi = min(t.row0 + (int64_t)t.rows, G.start + G.count);
  q.bin_a = (uint32_t)Pa.bin;
  q.bin_b = (uint32_t)Pb.bin;
  q.c0 = G.fpos >= 0 ? load_codes<R>(codes_c + (int64_t)G.fpos * ld_c, row, q.lo, q.hi)
                     : zero_codes<R>();
  q.ca = G.par[0] >= 0 ? load_codes<R>(codes_c + (int64_t)Pa.fpos * ld_c, row, q.lo, q.hi)
                       : zero_codes<R>();
  q.cb = G.par[1] >= 0 ? load_codes<R>(codes_c + (int64_t)Pb.fpos * ld_c, row, q.lo, q.hi)
                       : zero_codes<R>();
  return q;
}

// Bit k of run[r]: row row+k lies in the tile's part of the group and goes
// to run r (side 1 when the group's split sends it right, then right when
// its side's parent's split does: code > bin).  Rows of a side without a
// parent are in no run.
template <int R>
__device__ __forceinline__ void route_masks(const Route<R> &q, const PartGroup &G, int64_t row,
                                            uint32_t (&run)[4]) {
  const bool has_a = G.par[0] >= 0, has_b = G.par[1] >= 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) run[r] = 0u;
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const int sh = 8 * (k & 3);
    const bool in = (row + k >= q.lo) && (row + k < q.hi);
    const bool side = G.fpos >= 0 && ((q.c0.w[k >> 2] >> sh) & 255u) > (uint32_t)G.bin;
    const bool right = side ? ((q.cb.w[k >> 2] >> sh) & 255u) > q.bin_b
                            : ((q.ca.w[k >> 2] >> sh) & 255u) > q.bin_a;
    const uint32_t bit = ((in && (side ? has_b : has_a)) ? 1u : 0u) << k;
    run[0] |= (!side && !right) ? bit : 0u;
    run[1] |= (!side && right) ? bit : 0u;
    run[2] |= (side && !right) ? bit : 0u;
    run[3] |= (side && right) ? bit : 0u;
  }
}

// The side parents of a group (start 0 and no split when a side has none).
__device__ __forceinline__ void group_parents(const PartGroup &G,
                                              const PartParent *__restrict__ parents,
                                              PartParent &Pa, PartParent &Pb) {
  const PartParent none{0, 0, 0, 0, -1, -1, -1, 0, 0, 0};
  Pa = G.par[0] >= 0 ? parents[G.par[0]] : none;
  Pb = G.par[1] >= 0 ? parents[G.par[1]] : none;
}

template <int R>
__global__ __launch_bounds__(kPartBlock) void k_part_count(
    const uint8_t *__restrict__ codes_c, int64_t ld_c,
    const PartParent *__restrict__ parents, const PartGroup *__restrict__ groups,
    const PartTile *__restrict__ tiles, const LevelPlan *__restrict__ plan,
    int32_t *__restrict__ tile_cnt) {
  __shared__ uint2 red[kPartBlock / 64];
  const int32_t n_tiles = plan->n_tiles;
  for (int32_t ti = (int32_t)blockIdx.x; ti < n_tiles; ti += (int32_t)gridDim.x) {
    const PartTile t = tiles[ti];
    const PartGroup G = tile_group(groups, parents, t.parent);
    PartParent Pa, Pb;
    group_parents(G, parents, Pa, Pb);
    const int64_t row = t.row0 + (int64_t)R * threadIdx.x;
    const Route<R> rt = route_load<R>(codes_c, ld_c, t, G, Pa, Pb, row);
    uint32_t run[4];
    route_masks<R>(rt, G, row, run);
    // Four counts as 16-bit fields (a tile has at most 4096 rows).
    const uint32_t a = wave_sum((uint32_t)__builtin_popcount(run[0]) |
                                ((uint32_t)__builtin_popcount(run[1]) << 16));
    const uint32_t b = wave_sum((uint32_t)__builtin_popcount(run[2]) |
                                ((uint32_t)__builtin_popcount(run[3]) << 16));
    if (lane_id() == 0) red[threadIdx.x >> 6] = make_uint2(a, b);
    __syncthreads();
    if (threadIdx.x == 0) {
      uint32_t sa = 0u, sb = 0u;
#pragma unroll
      for (int w = 0; w < kPartBlock / 64; ++w) {
        sa += red[w].x;
        sb += red[w].y;
      }
      *reinterpret_cast<uint4 *>(tile_cnt + 4 * (int64_t)ti) =
          make_uint4(sa & 0xffffu, sa >> 16, sb & 0xffffu, sb >> 16);
    }
    __syncthreads();  // red is rewritten by the block's next tile
  }
}

hipError_t launch_part_count(hipStream_t st, const uint8_t *codes_c,
                             int64_t ld_c, const PartParent *parents, const PartGroup *groups,
                             const PartTile *tiles, const LevelPlan *plan,
                             int32_t max_tiles, int32_t part_rows, int32_t *tile_cnt) {
  if (max_tiles <= 0) return hipSuccess;
#define BSSCL_COUNT(R)                                                                 \
  hipLaunchKernelGGL(k_part_count<R>, dim3((unsigned)max_tiles), dim3(kPartBlock), 0, st, \
                     codes_c, ld_c, parents, groups, tiles, plan, tile_cnt)
  switch (part_rows) {
    case 4: BSSCL_COUNT(4); break;
    case 8: BSSCL_COUNT(8); break;
    case 16: BSSCL_COUNT(16); break;
    default: return hipErrorInvalidValue;
  }
#undef BSSCL_COUNT
  return hipGetLastError();
}

// A side's rows over its group's tiles [t0, t1): runs 2*side (left) and
// 2*side + 1 (right), summed by one wave (every lane gets the sums).
__device__ __forceinline__ void wave_side_counts(const int32_t *__restrict__ tile_cnt, int32_t t0,
                                                 int32_t t1, int side, long long &nl,
                                                 long long &nr) {
  strided_side_counts(tile_cnt + 2 * side, t0 + lane_id(), t1, 64, nl, nr);
  nl = wave_sum(nl);
  nr = wave_sum(nr);
}

// Moves a tile's rows to their runs' segments in the other buffer set,
// keeping the input order within each run.  A row's slot (the tile's rows
// of run 0, then run 1, 2, 3) is a block-wide exclusive scan of per-thread
// counts plus its rank among the thread's R rows; inv[slot] is the row it
// came from.  The output is cut into R-byte chunks aligned in the
// destination.  Features move four at a time: each tile row's four codes go
// to LDS as one 32-bit word (a 4x4 byte transpose of the thread's loads),
// and each output chunk reads its R source rows' words and transposes them
// back into one R-byte store per feature (byte stores only for the chunks
// at the ends of a run, which it shares with the neighbouring tiles).
// (g,h) and row ids are gathered through inv and stored as consecutive
// elements.
constexpr int kChunkSlots = 2;  // output chunks a thread may own (<= 264 per tile)
constexpr int kQuad = 4;        // features per LDS pass (one 32-bit word per row)

// 4x4 byte transpose: byte j of r_i is byte i of w_j.
__device__ __forceinline__ void transpose4(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3,
                                           uint32_t &r0, uint32_t &r1, uint32_t &r2,
                                           uint32_t &r3) {
  const uint32_t lo01 = (w0 & 0x00ff00ffu) | ((w1 & 0x00ff00ffu) << 8);  // w0.0 w1.0 w0.2 w1.2
  const uint32_t hi01 = ((w0 >> 8) & 0x00ff00ffu) | (w1 & 0xff00ff00u);  // w0.1 w1.1 w0.3 w1.3
  const uint32_t lo23 = (w2 & 0x00ff00ffu) | ((w3 & 0x00ff00ffu) << 8);
  const uint32_t hi23 = ((w2 >> 8) & 0x00ff00ffu) | (w3 & 0xff00ff00u);
  r0 = (lo01 & 0xffffu) | (lo23 << 16);
  r1 = (hi01 & 0xffffu) | (hi23 << 16);
  r2 = (lo01 >> 16) | (lo23 & 0xffff0000u);
  r3 = (hi01 >> 16) | (hi23 & 0xffff0000u);
}
// Waves per SIMD the register budget must allow (4: 128 VGPRs, which the
// four-run routing needs without spilling).  16-row tiles move one feature
// per barrier through LDS bytes instead of four through words: the word
// transposes of 16 rows need more registers than that.
template <int R> struct ScatterWaves { static constexpr int value = 4; };
// Features a 16-row tile stages per barrier: each thread's next Q codes
// loads are in flight while it gathers the current ones.  At 10M x 50
// (35 features) one feature per barrier kept about 16 KB of loads in flight
// per CU and moved 2.9 TB/s; Q = 2, 4 and 8 ran the round in 2.49, 2.46 and
// 2.56 ms against 2.54 (Q = 8: 74 KB of LDS, two blocks per CU).
template <int R> struct ScatterQ { static constexpr int value = 1; };
template <> struct ScatterQ<16> { static constexpr int value = 4; };

// One of four values by a run index r in 0..3, as selects of values (an
// array indexed by r would live in scratch memory).
template <typename T>
__device__ __forceinline__ T sel4(int r, T a, T b, T c, T d) {
  return r == 0 ? a : r == 1 ? b : r == 2 ? c : d;
}

template <int R, int Q = ScatterQ<R>::value>
__global__ __launch_bounds__(kPartBlock) __attribute__((amdgpu_waves_per_eu(ScatterWaves<R>::value)))
void k_part_scatter(
    const uint8_t *__restrict__ codes_src, uint8_t *__restrict__ codes_dst,
    int64_t ld_c, const GH *__restrict__ gh_src, GH *__restrict__ gh_dst,
    const int32_t *__restrict__ rid_src, int32_t *__restrict__ rid_dst,
    const PartParent *__restrict__ parents, const PartGroup *__restrict__ groups,
    const PartTile *__restrict__ tiles,
    const LevelPlan *__restrict__ plan, const int32_t *__restrict__ tile_begin,
    const int32_t *__restrict__ tile_cnt, int64_t *__restrict__ parent_nleft,
    NodeSeg *__restrict__ segs, int32_t *__restrict__ hist_node, int32_t min_samples_leaf,
    int32_t F_sel) {
  __shared__ unsigned long long tmp[kPartBlock / 64];
  __shared__ unsigned long long red[kPartBlock / 64][4];
  constexpr int kTile = kPartBlock * R;
  __shared__ uint16_t inv[kTile];
  constexpr bool kQuads = R < 16;
  // Four features' codes per tile row (16-row tiles: Q features' codes per
  // thread), double buffered.
  __shared__ __align__(16) uint32_t rows4[2][kQuads ? kTile : 1];
  __shared__ typename CodesR<R>::T cs[2][kQuads ? 1 : Q * kPartBlock];
  const int32_t n_tiles = plan->n_tiles;
  const int tid = (int)threadIdx.x;
  for (int32_t ti = (int32_t)blockIdx.x; ti < n_tiles; ti += (int32_t)gridDim.x) {
    const PartTile t = tiles[ti];
    const PartGroup G = tile_group(groups, parents, t.parent);
    if (G.par[0] < 0 && G.par[1] < 0) continue;  // a group with no expanded side: rows stay
    PartParent Pa, Pb;
    group_parents(G, parents, Pa, Pb);
    const int64_t row = t.row0 + (int64_t)R * tid;
    const Route<R> rt = route_load<R>(codes_src, ld_c, t, G, Pa, Pb, row);
    const int64_t lo = rt.lo, hi = rt.hi;
    // (The masks first: the routing codes are not held through the scan.)
    uint32_t run[4];
    route_masks<R>(rt, G, row, run);
    // The group's scan of its tiles' run counts, done by each of its tiles:
    // per run, the rows of the tiles before this one (high word) and of all
    // of them (low word).  (One 16-byte load per tile, two per thread in
    // flight.)
    const int32_t tb0 = tile_begin[t.parent], tb1 = tile_begin[t.parent + 1];
    unsigned long long acc[4] = {0ull, 0ull, 0ull, 0ull};
    for (int k0 = tb0 + tid; k0 < tb1; k0 += 2 * kPartBlock) {
      const int k1 = k0 + kPartBlock;
      const uint4 a = *reinterpret_cast<const uint4 *>(tile_cnt + 4 * (int64_t)k0);
      const uint4 b = k1 < tb1 ? *reinterpret_cast<const uint4 *>(tile_cnt + 4 * (int64_t)k1)
                               : make_uint4(0u, 0u, 0u, 0u);
      const uint32_t va[4] = {a.x, a.y, a.z, a.w}, vb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const unsigned long long x = va[r], y = vb[r];
        acc[r] += x + y + (k0 < ti ? x << 32 : 0ull) + (k1 < ti ? y << 32 : 0ull);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = wave_sum(acc[r]);
    if (lane_id() == 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) red[tid >> 6][r] = acc[r];
    }
    // This thread's counts as four 16-bit fields (a tile has at most 4096 rows).
    const unsigned long long packed = (unsigned long long)__builtin_popcount(run[0]) |
                                      ((unsigned long long)__builtin_popcount(run[1]) << 16) |
                                      ((unsigned long long)__builtin_popcount(run[2]) << 32) |
                                      ((unsigned long long)__builtin_popcount(run[3]) << 48);
    unsigned long long tot;
    const unsigned long long pre =
        block_excl_scan<kPartBlock>(packed, tmp, tot);  // (its barriers publish red)
    int64_t gpre[4], gtot[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      unsigned long long s = 0ull;
#pragma unroll
      for (int w = 0; w < kPartBlock / 64; ++w) s += red[w][r];
      gpre[r] = (int64_t)(s >> 32);
      gtot[r] = (int64_t)(s & 0xffffffffull);
    }
    // Destination of each run's first row of this tile: side 0's parent's
    // left child, its right child, then side 1's.
    const int64_t base[4] = {Pa.start + gpre[0], Pa.start + gtot[0] + gpre[1],
                             Pb.start + gpre[2], Pb.start + gtot[2] + gpre[3]};
    if (ti == tb0 && tid == 0) {
      if (G.par[0] >= 0)
        write_children(Pa, G.par[0], gtot[0], gtot[1], min_samples_leaf, parent_nleft, segs,
                       hist_node);
      if (G.par[1] >= 0)
        write_children(Pb, G.par[1], gtot[2], gtot[3], min_samples_leaf, parent_nleft, segs,
                       hist_node);
    }
    int len[4], off[4], tpre[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      len[r] = (int)((tot >> (16 * r)) & 0xffffull);
      tpre[r] = (int)((pre >> (16 * r)) & 0xffffull);
    }
    off[0] = 0;
    off[1] = len[0];
    off[2] = off[1] + len[1];
    off[3] = off[2] + len[2];
    const int vtot = off[3] + len[3];
    {
      int rk[4] = {0, 0, 0, 0};
#pragma unroll
      for (int k = 0; k < R; ++k) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if ((run[r] >> k) & 1u) {
            inv[off[r] + tpre[r] + rk[r]] = (uint16_t)(R * tid + k);
            ++rk[r];
          }
        }
      }
    }
    __syncthreads();
    // (g,h) and row ids: slot s -> its destination row.  (An empty run's
    // offset equals the next one's, so the count below skips it.)
    for (int sl = tid; sl < vtot; sl += kPartBlock) {
      const int r = (sl >= off[1] ? 1 : 0) + (sl >= off[2] ? 1 : 0) + (sl >= off[3] ? 1 : 0);
      const int64_t d = sel4(r, base[0], base[1], base[2], base[3]) +
                        (sl - sel4(r, off[0], off[1], off[2], off[3]));
      const int64_t src = t.row0 + inv[sl];
      gh_dst[d] = gh_src[src];
      if (rid_dst) rid_dst[d] = rid_src[src];
    }
    // Output chunks: each run's aligned R-byte chunks, runs in order.
    int cum[4], n_chunks = 0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      cum[r] = n_chunks;
      n_chunks += len[r] ? (int)((base[r] + len[r] + R - 1) / R - base[r] / R) : 0;
    }
    if constexpr (!kQuads) {
      // 16-row tiles.  Per owned chunk: its destination row, the slot (inv
      // index) of its first byte and the bytes [klo, khi) that lie in its
      // run (all 16 for a full chunk); each batch of Q features reads the
      // chunk's 16 tile rows from inv once.
      int64_t cdst[kChunkSlots];
      int32_t cinv[kChunkSlots], kr[kChunkSlots];
      bool cown[kChunkSlots];
#pragma unroll
      for (int q = 0; q < kChunkSlots; ++q) {
        const int c = tid + q * kPartBlock;
        cown[q] = c < n_chunks;
        const int r = (c >= cum[1] ? 1 : 0) + (c >= cum[2] ? 1 : 0) + (c >= cum[3] ? 1 : 0);
        const int64_t D = sel4(r, base[0], base[1], base[2], base[3]);
        const int L = sel4(r, len[0], len[1], len[2], len[3]);
        const int S = sel4(r, off[0], off[1], off[2], off[3]);
        const int64_t c0 =
            (D & ~int64_t(R - 1)) + R * (int64_t)(c - sel4(r, cum[0], cum[1], cum[2], cum[3]));
        cdst[q] = c0;
        cinv[q] = S + (int)(c0 - D);
        const int klo = (int)max<int64_t>(0, D - c0);
        const int khi = (int)min<int64_t>(R, D + L - c0);
        kr[q] = klo | (khi << 8);
      }
      CodeWords<R> nxt[Q];
#pragma unroll
      for (int u = 0; u < Q; ++u)
        nxt[u] = u < F_sel ? load_codes<R>(codes_src + (int64_t)u * ld_c, row, lo, hi)
                           : zero_codes<R>();
      for (int f0 = 0, b = 0; f0 < F_sel; f0 += Q, b ^= 1) {
#pragma unroll
        for (int u = 0; u < Q; ++u) cs[b][u * kPartBlock + tid] = nxt[u].v;
#pragma unroll
        for (int u = 0; u < Q; ++u)
          if (f0 + Q + u < F_sel)
            nxt[u] = load_codes<R>(codes_src + (int64_t)(f0 + Q + u) * ld_c, row, lo, hi);
        __syncthreads();
        const int nf = min(Q, F_sel - f0);
#pragma unroll
        for (int q = 0; q < kChunkSlots; ++q) {
          if (!cown[q]) continue;
          const int klo = kr[q] & 255, khi = kr[q] >> 8;
          if (klo == 0 && khi == R) {
            uint32_t src[R];
#pragma unroll
            for (int k = 0; k < R; ++k) src[k] = inv[cinv[q] + k];
#pragma unroll
            for (int u = 0; u < Q; ++u) {
              if (u >= nf) break;
              const uint8_t *tb = reinterpret_cast<const uint8_t *>(cs[b] + u * kPartBlock);
              CodeWords<R> o;
#pragma unroll
              for (int k = 0; k < R / 4; ++k)
                o.w[k] = (uint32_t)tb[src[4 * k]] | ((uint32_t)tb[src[4 * k + 1]] << 8) |
                         ((uint32_t)tb[src[4 * k + 2]] << 16) |
                         ((uint32_t)tb[src[4 * k + 3]] << 24);
              *reinterpret_cast<typename CodesR<R>::T *>(codes_dst + (int64_t)(f0 + u) * ld_c +
                                                         cdst[q]) = o.v;
            }
          } else {
            for (int u = 0; u < nf; ++u) {
              const uint8_t *tb = reinterpret_cast<const uint8_t *>(cs[b] + u * kPartBlock);
              uint8_t *dcol = codes_dst + (int64_t)(f0 + u) * ld_c;
              for (int k = klo; k < khi; ++k) dcol[cdst[q] + k] = tb[inv[cinv[q] + k]];
            }
          }
        }
      }
    } else {
      // Per owned chunk: its destination row and, per byte, the tile row it
      // copies (0xffff: outside the run, not written).
      int64_t cdst[kChunkSlots];
      uint32_t csrc[kChunkSlots][R / 2];  // R x u16 tile rows
      bool cfull[kChunkSlots], cown[kChunkSlots];
#pragma unroll
      for (int q = 0; q < kChunkSlots; ++q) {
        const int c = tid + q * kPartBlock;
        cown[q] = c < n_chunks;
        const int r = (c >= cum[1] ? 1 : 0) + (c >= cum[2] ? 1 : 0) + (c >= cum[3] ? 1 : 0);
        const int64_t D = sel4(r, base[0], base[1], base[2], base[3]);
        const int L = sel4(r, len[0], len[1], len[2], len[3]);
        const int S = sel4(r, off[0], off[1], off[2], off[3]);
        const int64_t c0 =
            (D & ~int64_t(R - 1)) + R * (int64_t)(c - sel4(r, cum[0], cum[1], cum[2], cum[3]));
        cdst[q] = c0;
        bool full = true;
#pragma unroll
        for (int k = 0; k < R; k += 2) {
          uint32_t pairv = 0u;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int64_t dr = c0 + k + h;
            const bool in = cown[q] && dr >= D && dr < D + L;
            full = full && in;
            const uint32_t src = in ? (uint32_t)inv[S + (int)(dr - D)] : 0xffffu;
            pairv |= src << (16 * h);
          }
          csrc[q][k >> 1] = pairv;
        }
        cfull[q] = full;
      }
      // Four features per batch, as one word of four codes per tile row,
      // double buffered in LDS (one barrier per batch, the next batch's
      // loads in flight meanwhile), then the owned chunks gathered and stored.
      CodeWords<R> cur[kQuad];
#pragma unroll
      for (int u = 0; u < kQuad; ++u) {
        if (u < F_sel) {
          cur[u] = load_codes<R>(codes_src + (int64_t)u * ld_c, row, lo, hi);
        } else {
#pragma unroll
          for (int k = 0; k < R / 4; ++k) cur[u].w[k] = 0u;
        }
      }
      for (int f0 = 0, b = 0; f0 < F_sel; f0 += kQuad, b ^= 1) {
#pragma unroll
        for (int g = 0; g < R / 4; ++g) {
          uint4 r;
          transpose4(cur[0].w[g], cur[1].w[g], cur[2].w[g], cur[3].w[g], r.x, r.y, r.z, r.w);
          *reinterpret_cast<uint4 *>(&rows4[b][R * tid + 4 * g]) = r;
        }
#pragma unroll
        for (int u = 0; u < kQuad; ++u) {
          if (f0 + kQuad + u < F_sel) {
            cur[u] = load_codes<R>(codes_src + (int64_t)(f0 + kQuad + u) * ld_c, row, lo, hi);
          } else {
#pragma unroll
            for (int k = 0; k < R / 4; ++k) cur[u].w[k] = 0u;
          }
        }
        __syncthreads();
        const int nf = min(kQuad, F_sel - f0);
#pragma unroll
        for (int q = 0; q < kChunkSlots; ++q) {
          if (!cown[q]) continue;
          CodeWords<R> o[kQuad];
#pragma unroll
          for (int g = 0; g < R / 4; ++g) {
            uint32_t sw[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const uint32_t sv = (csrc[q][(4 * g + j) >> 1] >> (16 * ((4 * g + j) & 1))) & 0xffffu;
              sw[j] = rows4[b][sv < (uint32_t)kTile ? sv : 0u];
            }
            transpose4(sw[0], sw[1], sw[2], sw[3], o[0].w[g], o[1].w[g], o[2].w[g], o[3].w[g]);
          }
#pragma unroll
          for (int u = 0; u < kQuad; ++u) {
            if (u >= nf) break;
            uint8_t *dcol = codes_dst + (int64_t)(f0 + u) * ld_c;
            if (cfull[q]) {
              *reinterpret_cast<typename CodesR<R>::T *>(dcol + cdst[q]) = o[u].v;
            } else {
#pragma unroll
              for (int k = 0; k < R; ++k) {
                const uint32_t sv = (csrc[q][k >> 1] >> (16 * (k & 1))) & 0xffffu;
                if (sv != 0xffffu) dcol[cdst[q] + k] = (uint8_t)(o[u].w[k >> 2] >> (8 * (k & 3)));
              }
            }
          }
        }
      }
    }
    __syncthreads();  // inv and rows4 are rewritten by the block's next tile
  }
}

hipError_t launch_part_scatter(hipStream_t st, const uint8_t *codes_src,
                               uint8_t *codes_dst, int64_t ld_c,
                               const GH *gh_src, GH *gh_dst,
                               const int32_t *rid_src, int32_t *rid_dst,
                               const PartParent *parents, const PartGroup *groups,
                               const PartTile *tiles, const LevelPlan *plan,
                               int32_t max_tiles, int32_t part_rows,
                               const int32_t *tile_begin, const int32_t *tile_cnt,
                               int64_t *parent_nleft, NodeSeg *segs, int32_t *hist_node,
                               int32_t min_samples_leaf, int32_t F_sel) {
  if (max_tiles <= 0) return hipSuccess;
#define BSSCL_SCATTER(R, Q)                                                                   \
  hipLaunchKernelGGL((k_part_scatter<R, Q>), dim3((unsigned)max_tiles), dim3(kPartBlock), 0, st, \
                     codes_src, codes_dst, ld_c, gh_src, gh_dst, rid_src, rid_dst, parents,      \
                     groups, tiles, plan, tile_begin, tile_cnt, parent_nleft, segs,            \
                     hist_node,                                                                \
                     min_samples_leaf, F_sel)
  switch (part_rows) {
    case 4: BSSCL_SCATTER(4, ScatterQ<4>::value); break;
    case 8: BSSCL_SCATTER(8, ScatterQ<8>::value); break;
    case 16: BSSCL_SCATTER(16, ScatterQ<16>::value); break;
    default: return hipErrorInvalidValue;
  }
#undef BSSCL_SCATTER
  return hipGetLastError();
}


// ---------------------------------------------------------------------------
// Split search (est:598-621, est:775-801).  One wave per (node, feature):
// lane l holds bins 4l..4l+3; an exact int64 prefix scan gives GL, HL for
// every bin; the gain is the reference's expression in fp64 without
// contraction; the wave keeps the largest gain, the lowest bin on ties.
// ---------------------------------------------------------------------------
#pragma clang fp contract(off)
// Histogram reduction and split search of one level in one launch.  A block
// of eight waves owns one (parent, feature): the waves sum every eighth of the
// small child's per-task partials (or read its histogram from the pool when
// one task wrote it there), the eight sums meet in LDS, then wave 0 stores
// the small child's histogram and searches it, and wave 1 stores the larger
// child's (parent minus small) and searches that.  The root is a level of
// one parent-less node.
__device__ __forceinline__ void split_search(const long long (&g)[4], const long long (&h)[4],
                                             int32_t node, const NodeSeg &s, bool depth_ok,
                                             int32_t fpos, int32_t nb, const SplitParams &P,
                                             int32_t F_sel, SplitCand *__restrict__ cand,
                                             long long *__restrict__ totals) {
  const int lane = lane_id();
  const long long lg = g[0] + g[1] + g[2] + g[3];
  const long long lhs = h[0] + h[1] + h[2] + h[3];
  const long long ig = wave_incl_scan<long long>(lg);
  const long long ih = wave_incl_scan<long long>(lhs);
  const long long Gt = wave_lane(ig, 63);
  const long long Ht = wave_lane(ih, 63);
  if (fpos == 0 && lane == 0) {
    totals[2 * (int64_t)node] = Gt;
    totals[2 * (int64_t)node + 1] = Ht;
  }
  const double Gtd = (double)Gt * P.g_scale;
  const double Htd = (double)Ht * P.h_scale;
  const bool can = s.count >= P.min_samples_leaf && Htd >= P.min_child_weight && depth_ok;
  double best = -1e9;
  int32_t bb = -1;
  if (can && nb >= 2) {
    const double lam = P.reg_lambda, mcw = P.min_child_weight;
    const double parent_term = Gtd * Gtd / (Htd + lam);
    long long GLq = ig - lg, HLq = ih - lhs;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      GLq += g[k];
      HLq += h[k];
      const int32_t b = lane * 4 + k;
      if (b <= nb - 2) {
        const double GL = (double)GLq * P.g_scale;
        const double HL = (double)HLq * P.h_scale;
        const double GR = (double)(Gt - GLq) * P.g_scale;
        const double HR = (double)(Ht - HLq) * P.h_scale;
        if (!(HL < mcw || HR < mcw)) {
          const double gain = (GL * GL / (HL + lam) + GR * GR / (HR + lam)) - parent_term;
          if (gain > best) {
            best = gain;
            bb = b;
          }
        }
      }
    }
  }
  int32_t unused = 0;
  wave_argmax(best, bb, unused);
  if (lane == 0) {
    SplitCand c;
    c.gain = best;
    c.bin = bb;
    c.pad = 0;
    cand[(int64_t)node * F_sel + fpos] = c;
  }
}

constexpr int kRsWaves = 8;  // waves of a reduce-split block

__global__ __launch_bounds__(64 * kRsWaves) void k_reduce_split(
    const LevelPlan *__restrict__ plan, const PartParent *__restrict__ parents,
    const int32_t *__restrict__ hist_begin, const int32_t *__restrict__ hist_node,
    const NodeSeg *__restrict__ segs, const unsigned long long *__restrict__ part,
    unsigned long long *__restrict__ pool, int64_t node_stride,
    const int32_t *__restrict__ nb_sel, int32_t F_sel, int32_t child_depth, SplitParams P,
    SplitCand *__restrict__ cand, long long *__restrict__ totals, int32_t span_parents) {
  __shared__ long long red[kRsWaves][kHistPerFeat];
  const int lane = lane_id(), wave = (int)(threadIdx.x >> 6);
  if (P.dev.max) dev_scales(P.dev, P.g_scale, P.h_scale);
  // An item's records: its parent's split, smaller child and task range.
  // The first item's are loaded with the plan (its parent index is below
  // the launch's parent bound, so the reads stay in the level lists even
  // when the level has fewer parents); the root's block (parents ==
  // nullptr) has one node and no sibling.
  struct Item {
    int32_t small, hb0, hb1;
    PartParent pp;
  };
  const auto records = [&](int32_t p) {
    Item r;
    r.small = parents ? hist_node[p] : 0;
    r.pp = parents ? parents[p] : PartParent{0, 0, 0, 0, -1, -1, -1, 0, 0, 0};
    r.hb0 = hist_begin[p];
    r.hb1 = hist_begin[p + 1];
    return r;
  };
  const int64_t it0 = blockIdx.x;
  Item cur = records((int32_t)div_pos(it0, F_sel));
  const int32_t n_par = parents ? plan->n_parents : 1;
  const int32_t tile_rows = plan->tile_rows;
  const int64_t n_items = (int64_t)n_par * F_sel;
  for (int64_t it = it0; it < n_items; it += gridDim.x) {
    const int32_t p = (int32_t)div_pos(it, F_sel), fpos = (int32_t)(it - (int64_t)p * F_sel);
    if (it != it0) cur = records(p);
    const int32_t small = cur.small;
    if (small < 0) continue;  // split not kept: no children (uniform)
    const PartParent &pp = cur.pp;
    const int32_t large = parents ? (pp.left_id == small ? pp.right_id : pp.left_id) : small;
    // Both children's segments and (wave 1) the parent's histogram, in
    // flight with the partials below.
    const NodeSeg ss = segs[small];
    const NodeSeg sl = segs[large];
    const int64_t woff = (int64_t)fpos * kHistPerFeat + lane * 8;
    long long pg[4] = {0, 0, 0, 0}, ph[4] = {0, 0, 0, 0};
    if (wave == 1 && parents) {
      const unsigned long long *hp = pool + (int64_t)pp.node * node_stride + woff;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        pg[k] = (long long)hp[2 * k];
        ph[k] = (long long)hp[2 * k + 1];
      }
    }
    // (An in-place level's tasks tiled the parent's segment.)
    const int64_t rows_tiled = span_parents ? pp.count : ss.count;
    const int32_t nt = (int32_t)min((int64_t)(cur.hb1 - cur.hb0),
                                    div_pos(rows_tiled + tile_rows - 1, tile_rows));
    unsigned long long *hs = pool + (int64_t)small * node_stride + woff;
    long long g[4] = {0, 0, 0, 0}, h[4] = {0, 0, 0, 0};
    if (nt == 1) {
      if (wave == 0) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          g[k] = (long long)hs[2 * k];
          h[k] = (long long)hs[2 * k + 1];
        }
      }
    } else {
      const unsigned long long *src =
          part + ((int64_t)cur.hb0 * F_sel) * kHistPerFeat + woff;
      const int64_t tstride = (int64_t)F_sel * kHistPerFeat;
      int32_t t = wave;
      for (; t + kRsWaves < nt; t += 2 * kRsWaves) {
        const longlong2 *a = reinterpret_cast<const longlong2 *>(src + (int64_t)t * tstride);
        const longlong2 *b =
            reinterpret_cast<const longlong2 *>(src + (int64_t)(t + kRsWaves) * tstride);
        longlong2 va[4], vb[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          va[k] = a[k];
          vb[k] = b[k];
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          g[k] += va[k].x + vb[k].x;
          h[k] += va[k].y + vb[k].y;
        }
      }
      if (t < nt) {
        const longlong2 *a = reinterpret_cast<const longlong2 *>(src + (int64_t)t * tstride);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const longlong2 v = a[k];
          g[k] += v.x;
          h[k] += v.y;
        }
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      red[wave][lane * 8 + 2 * k] = g[k];
      red[wave][lane * 8 + 2 * k + 1] = h[k];
    }
    __syncthreads();
    if (wave < 2 && (wave == 0 || parents)) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        g[k] = 0;
        h[k] = 0;
#pragma unroll
        for (int w = 0; w < kRsWaves; ++w) {
          g[k] += red[w][lane * 8 + 2 * k];
          h[k] += red[w][lane * 8 + 2 * k + 1];
        }
      }
      int32_t node = small;
      NodeSeg s = ss;
      if (wave == 0) {
        if (nt != 1) {
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            hs[2 * k] = (unsigned long long)g[k];
            hs[2 * k + 1] = (unsigned long long)h[k];
          }
        }
      } else {
        // The larger child: parent minus small.
        node = large;
        s = sl;
        unsigned long long *hl = pool + (int64_t)node * node_stride + woff;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          g[k] = pg[k] - g[k];
          h[k] = ph[k] - h[k];
          hl[2 * k] = (unsigned long long)g[k];
          hl[2 * k + 1] = (unsigned long long)h[k];
        }
      }
      split_search(g, h, node, s, !parents || child_depth < P.max_depth, fpos, nb_sel[fpos], P,
                   F_sel, cand, totals);
    }
    __syncthreads();  // red is rewritten by the block's next item
  }
}

#pragma clang fp contract(on)

hipError_t launch_reduce_split(hipStream_t st, const LevelPlan *plan, int32_t max_parents,
                               const PartParent *parents, const int32_t *hist_begin,
                               const int32_t *hist_node, const NodeSeg *segs,
                               const unsigned long long *part, unsigned long long *pool,
                               int64_t node_stride, const int32_t *nb_sel, int32_t F_sel,
                               int32_t child_depth, SplitParams p, SplitCand *cand,
                               long long *totals, int32_t span_parents) {
  const int64_t items = (int64_t)max_parents * F_sel;
  if (items <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_reduce_split, dim3((unsigned)std::min<int64_t>(items, 16384)),
                     dim3(64 * kRsWaves), 0, st, plan, parents, hist_begin, hist_node, segs, part, pool, node_stride,
                     nb_sel, F_sel, child_depth, p, cand, totals, span_parents);
  return hipGetLastError();
}

// The last level (its children are at max_depth, est:775-777): one wave per
// parent sums its side's runs over its group's tiles (the children's
// segments, whether the split is kept, est:678-683), the children's totals
// from the parent's histogram of the split feature, and the children's
// table records (no split).  Replaces scan, child totals and record kernels.
__global__ __launch_bounds__(256) void k_last_level(
    const PartParent *__restrict__ parents, int32_t grouped, const LevelPlan *__restrict__ plan,
    const int32_t *__restrict__ tile_begin, const int32_t *__restrict__ tile_cnt,
    int64_t *__restrict__ parent_nleft, NodeSeg *__restrict__ segs,
    int32_t *__restrict__ hist_node, int32_t min_samples_leaf,
    const unsigned long long *__restrict__ pool, int64_t node_stride,
    long long *__restrict__ totals, NodeOut *__restrict__ nodes) {
  const int lane = lane_id();
  const int32_t n_parents = plan->n_parents;
  for (int w = (int)(blockIdx.x * 4 + (threadIdx.x >> 6)); w < n_parents;
       w += (int)gridDim.x * 4) {
    const PartParent P = parents[w];
    long long nl, nr;
    wave_side_counts(tile_cnt, P.tile0, P.tile1, grouped ? (P.gslot & 1) : 0, nl, nr);
    // The parent's histogram of its split feature: totals of bins <= bin.
    const long long *h = reinterpret_cast<const long long *>(pool) +
                         (int64_t)P.node * node_stride + (int64_t)P.fpos * kHistPerFeat;
    long long gl = 0, hl = 0, gt = 0, ht = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int b = lane * 4 + k;
      const long long g = h[2 * b], hh = h[2 * b + 1];
      gt += g;
      ht += hh;
      if (b <= P.bin) {
        gl += g;
        hl += hh;
      }
    }
    gl = wave_sum(gl);
    hl = wave_sum(hl);
    gt = wave_sum(gt);
    ht = wave_sum(ht);
    if (lane == 0) {
      write_children(P, w, nl, nr, min_samples_leaf, parent_nleft, segs, hist_node);
      const bool ok = nl >= min_samples_leaf && nr >= min_samples_leaf;
      if (ok) {
        totals[2 * (int64_t)P.left_id] = gl;
        totals[2 * (int64_t)P.left_id + 1] = hl;
        totals[2 * (int64_t)P.right_id] = gt - gl;
        totals[2 * (int64_t)P.right_id + 1] = ht - hl;
      }
      NodeOut o;
      o.gain = -1e9;
      o.e = 0.0;
      o.fpos = -1;
      o.bin = 0;
      o.valid = ok ? 1 : 0;
      o.left = -1;
      o.start = P.start;
      o.count = nl;
      o.Gq = ok ? gl : 0;
      o.Hq = ok ? hl : 0;
      nodes[P.left_id] = o;
      o.start = P.start + nl;
      o.count = nr;
      o.Gq = ok ? gt - gl : 0;
      o.Hq = ok ? ht - hl : 0;
      nodes[P.right_id] = o;
    }
  }
}

hipError_t launch_last_level(hipStream_t st, const PartParent *parents, int32_t grouped,
                             const LevelPlan *plan,
                             int32_t max_parents, const int32_t *tile_begin,
                             const int32_t *tile_cnt, int64_t *parent_nleft, NodeSeg *segs,
                             int32_t *hist_node, int32_t min_samples_leaf,
                             const unsigned long long *pool, int64_t node_stride,
                             long long *totals, NodeOut *nodes) {
  if (max_parents <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_last_level, dim3((unsigned)((max_parents + 3) / 4)), dim3(256), 0, st,
                     parents, grouped, plan, tile_begin, tile_cnt, parent_nleft, segs, hist_node,
                     min_samples_leaf, pool, node_stride, totals, nodes);
  return hipGetLastError();
}


// A node's table record: its segment, fixed-point totals and best split
// over the features -- the largest gain, the lowest feature position on
// ties (est:618-621) -- not yet expanded (left = -1).  One thread.
__device__ __forceinline__ NodeOut node_record(int32_t node, const NodeSeg *__restrict__ segs,
                                               const long long *__restrict__ totals,
                                               const SplitCand *__restrict__ cand,
                                               int32_t F_sel) {
  const NodeSeg s = segs[node];
  double best = 0.0;
  int32_t bf = -1, bb = 0;
  if (s.valid) {
    for (int32_t f = 0; f < F_sel; ++f) {
      const SplitCand c = cand[(int64_t)node * F_sel + f];
      if (c.bin >= 0 && (bf < 0 || c.gain > best)) {
        best = c.gain;
        bf = f;
        bb = c.bin;
      }
    }
  }
  NodeOut o;
  o.start = s.start;
  o.count = s.count;
  o.valid = s.valid;
  o.Gq = s.valid ? totals[2 * (int64_t)node] : 0;
  o.Hq = s.valid ? totals[2 * (int64_t)node + 1] : 0;
  o.gain = bf >= 0 ? best : -1e9;
  o.e = 0.0;
  o.fpos = bf;
  o.bin = bf >= 0 ? bb : 0;
  o.left = -1;
  return o;
}

// Per node: node_record with one wave over the features (the last level,
// whose children have no planner after them).
__global__ __launch_bounds__(256) void k_node_best(
    const NodeSeg *__restrict__ segs, const long long *__restrict__ totals,
    const SplitCand *__restrict__ cand, int32_t F_sel,
    const LevelPlan *__restrict__ plan, int32_t no_split,
    NodeOut *__restrict__ nodes) {
  const int lane = lane_id();
  const int32_t first = plan->first_child, count = plan->n_split;
  for (int w = (int)(blockIdx.x * 4 + (threadIdx.x >> 6)); w < count;
       w += (int)gridDim.x * 4) {
    const int node = first + w;
    const NodeSeg s = segs[node];
    double best = 0.0;
    int32_t bf = -1, bb = 0;
    if (s.valid && !no_split) {
      for (int f = lane; f < F_sel; f += 64) {
        const SplitCand c = cand[(int64_t)node * F_sel + f];
        if (c.bin >= 0 && (bf < 0 || c.gain > best)) {
          best = c.gain;
          bf = f;
          bb = c.bin;
        }
      }
    }
    wave_argmax(best, bf, bb);
    if (lane == 0) {
      NodeOut o;
      o.start = s.start;
      o.count = s.count;
      o.valid = s.valid;
      o.Gq = s.valid ? totals[2 * (int64_t)node] : 0;
      o.Hq = s.valid ? totals[2 * (int64_t)node + 1] : 0;
      o.gain = bf >= 0 ? best : -1e9;
      o.e = 0.0;
      o.fpos = bf;
      o.bin = bf >= 0 ? bb : 0;
      o.left = -1;
      nodes[node] = o;
    }
  }
}

hipError_t launch_node_best(hipStream_t st, const NodeSeg *segs,
                            const long long *totals, const SplitCand *cand,
                            int32_t F_sel, const LevelPlan *plan,
                            int32_t max_nodes, int32_t no_split, NodeOut *nodes) {
  if (max_nodes <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_node_best, dim3((unsigned)((max_nodes + 3) / 4)), dim3(256), 0,
                     st, segs, totals, cand, F_sel, plan, no_split, nodes);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Level planner: est:641-820 grown one depth at a time.  One workgroup.
//
// The candidates of level `a.level` are the nodes the previous level created
// (the root at level 0).  A candidate is expanded when it is valid, has a
// split whose gain exceeds gamma (est:649-652), and fewer than max_leaves - 1
// splits kept at earlier levels rank above it.  A node's rank e is the
// smallest best gain on its root path; the best-first loop pops nodes in
// non-increasing e order and stops after max_leaves - 1 kept splits, so a
// node with that many kept splits strictly above it is never popped and its
// subtree is never needed.  Expanded nodes get consecutive child ids, and the
// kernel writes the level's PartParent, PartTile and HistTask lists and its
// LevelPlan.  When the node table is too small the plan
// records the nodes needed in `overflow` and every later kernel does nothing.
// ---------------------------------------------------------------------------
constexpr int kPlanBlock = 1024;
constexpr int kPlanChunk = 2048;  // ranks of earlier nodes staged in LDS at a time

// Rows per histogram tile for S rows: about hist_target tiles, but no fewer
// than rows_per_flush rows per tile, a multiple of 4096 rows.
__device__ __forceinline__ int32_t plan_tile_rows(int64_t S, const PlanArgs &a) {
  int64_t tiles = max((int64_t)1, (int64_t)a.hist_target);
  tiles = min(tiles, max((int64_t)1, div_pos(S, a.rows_per_flush)));
  const int64_t t = (div_pos(S + tiles - 1, tiles) + 4095) / 4096 * 4096;
  return (int32_t)min(max(t, (int64_t)4096), (int64_t)1 << 24);
}

__global__ __launch_bounds__(kPlanBlock) void k_plan(
    NodeOut *__restrict__ nodes, LevelPlan *__restrict__ plan,
    const PartParent *__restrict__ prev_parents, PartParent *__restrict__ parents,
    int32_t *__restrict__ tile_begin, int32_t *__restrict__ hist_begin,
    PartTile *__restrict__ tiles, HistTask *__restrict__ hist_tasks,
    int32_t *__restrict__ work_flag,
    double *__restrict__ work_e, const NodeSeg *__restrict__ segs,
    const long long *__restrict__ totals, const SplitCand *__restrict__ cand, int32_t F_sel,
    PlanArgs a) {
  __shared__ uint32_t stmp[kPlanBlock / 64];
  __shared__ double ke[kPlanChunk];
  __shared__ unsigned long long s_rows;
  const int tid = (int)threadIdx.x;
  const LevelPlan prev = *plan;
  if (prev.overflow) return;  // an earlier level ran out of nodes
  const int32_t first = prev.first_child, nc = prev.n_split, n_prev = prev.n_nodes;
  if (tid == 0) s_rows = 0ull;

  // Candidates: their table records (best split over the features), rank
  // and whether they may be split (est:649-652, 762-801).
  for (int j = tid; j < nc; j += kPlanBlock) {
    const int c = first + j;
    NodeOut N = node_record(c, segs, totals, cand, F_sel);
    double e = 0.0;
    int32_t f = 0;
    if (N.valid) {
      const double pe = a.level == 0 ? N.gain : nodes[prev_parents[j >> 1].node].e;
      e = pe < N.gain ? pe : N.gain;
      f = (N.fpos >= 0 && N.gain > a.gamma) ? 1 : 0;
    }
    N.e = e;
    nodes[c] = N;
    work_e[j] = e;
    work_flag[j] = f;
  }
  __syncthreads();

  // Kept splits of earlier levels (expanded, children valid) ranked above.
  for (int jb = 0; jb < nc; jb += kPlanBlock) {
    const int j = jb + tid;
    const bool act = j < nc && work_flag[j] != 0;
    const double ev = act ? work_e[j] : 0.0;
    int32_t above = 0;
    for (int kb = 0; kb < first; kb += kPlanChunk) {
      const int kn = min(kPlanChunk, first - kb);
      for (int i = tid; i < kn; i += kPlanBlock) {
        const int32_t l = nodes[kb + i].left;
        const bool kept = l >= 0 && nodes[l].valid != 0;
        ke[i] = kept ? nodes[kb + i].e : -INFINITY;
      }
      __syncthreads();
      if (act)
        for (int i = 0; i < kn; ++i) above += ke[i] > ev ? 1 : 0;
      __syncthreads();
    }
    if (j < nc) work_flag[j] = (act && above < a.max_leaves - 1) ? 1 : 0;
  }
  __syncthreads();

  // Expanded candidates in candidate order: work_flag becomes the parent
  // index, -1 when not expanded.
  uint32_t carry = 0;
  for (int jb = 0; jb < nc; jb += kPlanBlock) {
    const int j = jb + tid;
    const uint32_t f = (j < nc) ? (uint32_t)work_flag[j] : 0u;
    uint32_t tot;
    const uint32_t pre = block_excl_scan<kPlanBlock>(f, stmp, tot);
    if (j < nc) work_flag[j] = f ? (int32_t)(carry + pre) : -1;
    carry += tot;
  }
  const int32_t n_exp = (int32_t)carry;
  const int64_t n_new = (int64_t)n_prev + 2 * (int64_t)n_exp;
  if (n_new > a.node_cap) {
    if (tid == 0) {
      LevelPlan q = {};
      q.first_child = n_prev;
      q.tile_rows = 4096;
      q.n_nodes = n_prev;
      q.overflow = (int32_t)min(n_new, (int64_t)INT32_MAX);
      *plan = q;
    }
    return;
  }

  // Parents and child links; tiles per parent; rows to histogram.
  unsigned long long rows = 0;
  for (int j = tid; j < nc; j += kPlanBlock) {
    const int32_t i = work_flag[j];
    if (i < 0) continue;
    const int32_t v = first + j;
    const int32_t L = n_prev + 2 * i;
    const NodeOut N = nodes[v];
    nodes[v].left = L;
    PartParent P;
    P.start = N.start;
    P.count = N.count;
    P.fpos = N.fpos;
    P.bin = N.bin;
    P.left_id = L;
    P.right_id = L + 1;
    P.node = v;
    P.gslot = 2 * i;
    parents[i] = P;
    const int64_t a0 = N.start & ~int64_t(15);
    // At least one tile: a parent's first tile writes its children's segments.
    tile_begin[i] = (int32_t)max((int64_t)1, div_pos(N.start + N.count - a0 + a.part_tile - 1, a.part_tile));
    rows += (unsigned long long)(N.count / 2);
  }
  rows = wave_sum(rows);
  if (lane_id() == 0 && rows) atomicAdd(&s_rows, rows);
  __syncthreads();
  const int32_t th = plan_tile_rows((int64_t)s_rows, a);

  // Exclusive offsets of each parent's tiles and histogram tasks.
  uint32_t tcar = 0, hcar = 0;
  for (int ib = 0; ib < n_exp; ib += kPlanBlock) {
    const int i = ib + tid;
    uint32_t nt = 0, nh = 0;
    if (i < n_exp) {
      nt = (uint32_t)tile_begin[i];
      nh = a.last ? 0u : (uint32_t)div_pos(parents[i].count / 2 + th, th);
    }
    uint32_t tt, ht;
    const uint32_t tp = block_excl_scan<kPlanBlock>(nt, stmp, tt);
    const uint32_t hp = block_excl_scan<kPlanBlock>(nh, stmp, ht);
    if (i < n_exp) {
      tile_begin[i] = (int32_t)(tcar + tp);
      hist_begin[i] = (int32_t)(hcar + hp);
    }
    tcar += tt;
    hcar += ht;
  }
  if (tcar > (uint32_t)a.tile_cap || hcar > (uint32_t)a.hist_cap) {
    // Capacities are sized from proven bounds; reaching this is a bug.
    if (tid == 0) {
      LevelPlan q = {};
      q.first_child = n_prev;
      q.tile_rows = 4096;
      q.n_nodes = n_prev;
      q.overflow = -1;
      *plan = q;
    }
    return;
  }
  if (tid == 0) {
    tile_begin[n_exp] = (int32_t)tcar;
    hist_begin[n_exp] = (int32_t)hcar;
  }
  __syncthreads();
  for (int i = tid; i < n_exp; i += kPlanBlock) {  // each parent's own tiles
    parents[i].tile0 = tile_begin[i];
    parents[i].tile1 = tile_begin[i + 1];
  }

  // Tile and histogram-task lists: item -> its parent by binary search.
  for (int t = tid; t < (int)tcar; t += kPlanBlock) {
    int lo = 0, hi = n_exp - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (tile_begin[mid] <= t) lo = mid;
      else hi = mid - 1;
    }
    PartTile T;
    T.row0 = (parents[lo].start & ~int64_t(15)) + (int64_t)(t - tile_begin[lo]) * a.part_tile;
    T.rows = a.part_tile;
    T.parent = lo;
    tiles[t] = T;
  }
  for (int q = tid; q < (int)hcar; q += kPlanBlock) {
    int lo = 0, hi = n_exp - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (hist_begin[mid] <= q) lo = mid;
      else hi = mid - 1;
    }
    hist_tasks[q] = HistTask{lo, q - hist_begin[lo]};
  }
  if (tid == 0) {
    LevelPlan q;
    q.n_parents = n_exp;
    q.n_tiles = (int32_t)tcar;
    q.n_hist = (int32_t)hcar;
    q.n_split = 2 * n_exp;
    q.first_child = n_prev;
    q.tile_rows = th;
    q.n_nodes = (int32_t)n_new;
    q.overflow = 0;
    *plan = q;
  }
}

// The same planner with every intermediate in LDS, for trees of at most
// kPlanLdsC + 1 nodes.  The reference's rule and outputs are those of
// k_plan; what changes is where the inputs come from, so that the kernel
// waits on global memory twice (the plan, then all its inputs at once)
// instead of once per phase:
//   * kept_e[u] is the rank e(u) of node u when u is a kept split (expanded,
//     children valid), -inf otherwise.  A level writes it for its candidates
//     that are not expanded and for the previous level's parents, whose
//     children are this level's candidates;
//   * parent_e[i] is the rank of this level's parent i, read by the next
//     level as prev_parent_e;
//   * the best split of a candidate over its features is a wave reduction,
//     four candidates per wave at a time.
constexpr int kPlanLdsC = 512;

// A candidate's planner record in LDS (est:649-652, 762-801): its best
// split over the features (bf < 0: none), its rank e (the smaller of its
// parent's rank `ppe` and its gain; the root's is its gain) and whether it
// may be split.
__device__ __forceinline__ void plan_record(
    int j, const NodeSeg &sg, long long gq, long long hq, double ppe, double best, int32_t bf,
    int32_t bb, const PlanArgs &a, int64_t *s_start, int64_t *s_count, long long *s_gq,
    long long *s_hq, double *s_gain, double *s_e, int32_t *s_fpos, int32_t *s_bin,
    int32_t *s_valid, int32_t *s_flag) {
  const bool valid = sg.valid != 0;
  if (!valid) bf = -1;
  const double gain = bf >= 0 ? best : -1e9;
  double e = 0.0;
  int32_t fl = 0;
  if (valid) {
    const double pv = a.level == 0 ? gain : ppe;
    e = pv < gain ? pv : gain;
    fl = (bf >= 0 && gain > a.gamma) ? 1 : 0;
  }
  s_start[j] = sg.start;
  s_count[j] = sg.count;
  s_gq[j] = valid ? gq : 0;
  s_hq[j] = valid ? hq : 0;
  s_gain[j] = gain;
  s_e[j] = e;
  s_fpos[j] = bf;
  s_bin[j] = bf >= 0 ? bb : 0;
  s_valid[j] = sg.valid;
  s_flag[j] = fl;
}

// Candidates x features staged in LDS by k_plan_lds (levels of up to 64
// candidates over up to 64 features; larger ones use a wave per candidate).
constexpr int kStageC = 64, kStageF = 64;
// Its fast path also needs at most this many nodes before the level's
// candidates (every level of a tree of up to 63 leaves).
constexpr int kFastFirst = 128;

// The next level's {first candidate, candidates}, for its counting blocks.
__device__ __forceinline__ void plan_next_level(int32_t *level_out, int32_t first, int32_t nc) {
  if (level_out) {
    level_out[0] = first;
    level_out[1] = nc;
  }
}

// Tiles of one item of a level's count: its rows [start, start + count)
// from start rounded down to 16, part_tile rows a tile, at least one (a
// parent's first tile writes its children's segments); none when off.
__device__ __forceinline__ uint32_t count_item_tiles(int64_t start, int64_t count, bool on,
                                                     int32_t part_tile) {
  if (!on) return 0u;
  const int64_t a0 = start & ~int64_t(15);
  return (uint32_t)max((int64_t)1, div_pos(start + count - a0 + part_tile - 1, part_tile));
}

// A candidate's best split over its features, as the planner takes it
// (est:618-621: the largest gain, the first position of equal gains), by
// one wave (wave-uniform `exists`); fpos -1 when there is none.
__device__ __forceinline__ void wave_best_split(const SplitCand *__restrict__ cand, int64_t c,
                                                int32_t F_sel, bool exists, int32_t &fpos,
                                                int32_t &bin) {
  double best = 0.0;
  int32_t bf = -1, bb = 0;
  if (exists) {
    for (int32_t f = lane_id(); f < F_sel; f += 64) {
      const SplitCand x = cand[c * F_sel + f];
      if (x.bin >= 0 && (bf < 0 || x.gain > best)) {
        best = x.gain;
        bf = f;
        bb = x.bin;
      }
    }
  }
  wave_argmax(best, bf, bb);
  fpos = bf;
  bin = bb;
}

// The counting role of an in-place or grouped level's planner launch
// (blocks 1..): the level's partition tiles over every candidate (in place)
// or every previous parent (grouped), from count_item_tiles in item order as
// block 0 lays them out, each routed by its candidates' best splits whether
// or not block 0 expands them, and each tile's four run counts written as
// k_part_count writes them.  The level's kernels read the counts of the
// expanded parents' tiles only (PartParent::tile0, tile1).  Each quarter of
// the block (256 threads, R rows each) takes one tile at a time.
template <int R>
__device__ void plan_count_role(const uint8_t *__restrict__ codes_c, int64_t ld_c,
                                const NodeSeg *__restrict__ segs,
                                const SplitCand *__restrict__ cand, int32_t F_sel,
                                const PartParent *__restrict__ prev_parents, int32_t first,
                                int32_t nc, bool grouped, const PlanArgs &a,
                                int32_t *__restrict__ tile_cnt, uint32_t *stmp, uint32_t *s_ctb,
                                int32_t (*s_cbest)[2][2], uint2 (*s_cred)[4]) {
  static_assert(kPlanBlock == kCountTilesPerBlock * kPartBlock, "a quarter per tile");
  const int tid = (int)threadIdx.x;
  const int n_items = grouped ? nc / 2 : nc;
  uint32_t nt = 0u;
  if (tid < n_items) {
    if (grouped) {
      const PartParent pp = prev_parents[tid];
      nt = count_item_tiles(pp.start, pp.count, true, a.part_tile);
    } else {
      const NodeSeg sg = segs[first + tid];
      nt = count_item_tiles(sg.start, sg.count, sg.valid != 0, a.part_tile);
    }
  }
  uint32_t total;
  const uint32_t pre = block_excl_scan<kPlanBlock>(nt, stmp, total);
  if (tid < kPlanLdsC) s_ctb[tid] = pre;
  if (tid == 0) s_ctb[kPlanLdsC] = total;
  __syncthreads();
  if (total > (uint32_t)a.tile_cap) return;  // block 0 reports the level as broken
  const int q = tid / kPartBlock, r = tid % kPartBlock, w = (tid >> 6) & 3;
  const int64_t stride = (int64_t)(gridDim.x - 1) * kCountTilesPerBlock;
  for (int64_t base = (int64_t)(blockIdx.x - 1) * kCountTilesPerBlock; base < (int64_t)total;
       base += stride) {
    const int64_t t = base + q;
    const bool act = t < (int64_t)total;
    int item = 0;
    if (act) {
      int lo = 0, hi = n_items - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if ((int64_t)s_ctb[mid] <= t) lo = mid;
        else hi = mid - 1;
      }
      item = lo;
    }
    // The best split of each side's candidate: wave 0 of the quarter for
    // side 0 (in place: the candidate itself), wave 1 for side 1.
    if (act && (w == 0 || (grouped && w == 1))) {
      const int32_t j = grouped ? 2 * item + w : item;
      const bool exists = segs[first + j].valid != 0;
      int32_t fp, bn;
      wave_best_split(cand, (int64_t)first + j, F_sel, exists, fp, bn);
      if (lane_id() == 0) {
        s_cbest[q][w][0] = fp;
        s_cbest[q][w][1] = bn;
      }
    }
    __syncthreads();
    uint32_t run[4] = {0u, 0u, 0u, 0u};
    if (act) {
      PartGroup G;
      if (grouped) {
        const PartParent pp = prev_parents[item];
        G.start = pp.start;
        G.count = pp.count;
        G.fpos = pp.fpos;
        G.bin = pp.bin;
      } else {
        const NodeSeg sg = segs[first + item];
        G.start = sg.start;
        G.count = sg.count;
        G.fpos = -1;
        G.bin = 0;
      }
      const int32_t fa = s_cbest[q][0][0], fb = grouped ? s_cbest[q][1][0] : -1;
      G.par[0] = fa >= 0 ? 0 : -1;
      G.par[1] = fb >= 0 ? 1 : -1;
      PartParent Pa{0, 0, fa, s_cbest[q][0][1], -1, -1, -1, 0, 0, 0};
      PartParent Pb{0, 0, fb, grouped ? s_cbest[q][1][1] : 0, -1, -1, -1, 0, 0, 0};
      PartTile T;
      T.row0 = (G.start & ~int64_t(15)) + (t - (int64_t)s_ctb[item]) * a.part_tile;
      T.rows = a.part_tile;
      T.parent = item;
      const int64_t row = T.row0 + (int64_t)R * r;
      const Route<R> rt = route_load<R>(codes_c, ld_c, T, G, Pa, Pb, row);
      route_masks<R>(rt, G, row, run);
    }
    // Four counts as 16-bit fields (a tile has at most 4096 rows).
    const uint32_t ca = wave_sum((uint32_t)__builtin_popcount(run[0]) |
                                 ((uint32_t)__builtin_popcount(run[1]) << 16));
    const uint32_t cb = wave_sum((uint32_t)__builtin_popcount(run[2]) |
                                 ((uint32_t)__builtin_popcount(run[3]) << 16));
    if (lane_id() == 0) s_cred[q][w] = make_uint2(ca, cb);
    __syncthreads();
    if (act && r == 0) {
      uint32_t sa = 0u, sb = 0u;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        sa += s_cred[q][k].x;
        sb += s_cred[q][k].y;
      }
      *reinterpret_cast<uint4 *>(tile_cnt + 4 * t) =
          make_uint4(sa & 0xffffu, sa >> 16, sb & 0xffffu, sb >> 16);
    }
    __syncthreads();  // s_cbest and s_cred are rewritten by the next tiles
  }
}

__global__ __launch_bounds__(kPlanBlock) void k_plan_lds(
    NodeOut *__restrict__ nodes, LevelPlan *__restrict__ plan,
    const PartParent *__restrict__ prev_parents, PartParent *__restrict__ parents,
    PartGroup *__restrict__ groups,
    int32_t *__restrict__ tile_begin, int32_t *__restrict__ hist_begin,
    PartTile *__restrict__ tiles, HistTask *__restrict__ hist_tasks,
    const NodeSeg *__restrict__ segs,
    const long long *__restrict__ totals, const SplitCand *__restrict__ cand,
    double *__restrict__ kept_e, const double *__restrict__ prev_parent_e,
    double *__restrict__ parent_e, int32_t F_sel, PlanArgs a,
    const uint8_t *__restrict__ codes_c, int64_t ld_c, int32_t *__restrict__ tile_cnt,
    const int32_t *__restrict__ level_in, int32_t *__restrict__ level_out) {
  __shared__ uint32_t stmp[kPlanBlock / 64];
  __shared__ uint32_t s_ctb[kPlanLdsC + 1];  // each count item's first tile (and the total)
  __shared__ double s_ke[kPlanLdsC + 1];
  __shared__ int64_t s_start[kPlanLdsC], s_count[kPlanLdsC];
  __shared__ long long s_gq[kPlanLdsC], s_hq[kPlanLdsC];
  __shared__ double s_gain[kPlanLdsC], s_e[kPlanLdsC];
  __shared__ int32_t s_fpos[kPlanLdsC], s_bin[kPlanLdsC], s_valid[kPlanLdsC];
  __shared__ int32_t s_flag[kPlanLdsC];
  __shared__ int32_t s_pj[kPlanLdsC / 2 + 1];  // candidate of each parent
  __shared__ int32_t s_tb[kPlanLdsC / 2 + 1], s_hb[kPlanLdsC / 2 + 1];
  // Grouped levels: each candidate's parent index (-1: not expanded); each
  // group's (parent's) first tile row.
  __shared__ int32_t s_pidx[kPlanLdsC];
  __shared__ int64_t s_gs[kPlanLdsC / 2 + 1];
  __shared__ uint32_t s_tcar;
  __shared__ unsigned long long s_rows;
  __shared__ double s_cg[kStageF * kStageC];   // staged gains [feature][candidate]
  __shared__ int16_t s_cb[kStageF * kStageC];  // staged bins (-1: no split)
  __shared__ int32_t s_fast[8];                // fast path: wave 0's results
  __shared__ int32_t s_cpf[(kPlanBlock / 64) * kStageC];  // fast path: each wave's best feature
  // Counting blocks: each tile's candidates' best splits and its waves' counts.
  __shared__ int32_t s_cbest[kCountTilesPerBlock][2][2];
  __shared__ uint2 s_cred[kCountTilesPerBlock][4];
  const int tid = (int)threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  if (blockIdx.x > 0) {
    // Counting blocks (a.fused_count): this level's candidates come from the
    // previous level's planner (the root alone at level 0), not from *plan,
    // which block 0 rewrites meanwhile.
    const int32_t c_first = a.level == 0 ? 0 : level_in[0];
    const int32_t c_nc = a.level == 0 ? 1 : level_in[1];
    if (a.fused_count && c_nc > 0 && c_nc <= kPlanLdsC) {
      const bool g = a.mode == kLevelGrouped;
      switch (a.part_rows) {
        case 4:
          plan_count_role<4>(codes_c, ld_c, segs, cand, F_sel, prev_parents, c_first, c_nc, g, a,
                             tile_cnt, stmp, s_ctb, s_cbest, s_cred);
          break;
        case 8:
          plan_count_role<8>(codes_c, ld_c, segs, cand, F_sel, prev_parents, c_first, c_nc, g, a,
                             tile_cnt, stmp, s_ctb, s_cbest, s_cred);
          break;
        default:
          plan_count_role<16>(codes_c, ld_c, segs, cand, F_sel, prev_parents, c_first, c_nc, g,
                              a, tile_cnt, stmp, s_ctb, s_cbest, s_cred);
          break;
      }
    }
    return;
  }
  const LevelPlan prev = *plan;
  if (prev.overflow) {
    if (tid == 0) plan_next_level(level_out, prev.n_nodes, 0);
    return;
  }
  const int32_t first = prev.first_child, nc = prev.n_split, n_prev = prev.n_nodes;
  const int32_t n_pp = a.level == 0 ? 0 : nc / 2;  // the previous level's parents
  if (nc > kPlanLdsC || first > kPlanLdsC + 1) {
    // The host selects this kernel only for trees that fit; reaching this is a bug.
    if (tid == 0) {
      LevelPlan q = {};
      q.first_child = n_prev;
      q.tile_rows = 4096;
      q.n_nodes = n_prev;
      q.overflow = -1;
      *plan = q;
      plan_next_level(level_out, n_prev, 0);
    }
    return;
  }
  const bool grouped = a.mode == kLevelGrouped;
  if (nc <= kStageC && first <= kFastFirst && F_sel <= kStageF) {
    // Fast path: one candidate per lane of wave 0, which takes every
    // decision below with wave operations and no block barrier; the other
    // waves stage the split candidates and write the tile and task lists.
    // Wave w takes features 4w .. 4w + 3 of candidate `lane` (F_sel <= 64).
    constexpr int kFw = kStageF / (kPlanBlock / 64);
    SplitCand cv[kFw];
#pragma unroll
    for (int u = 0; u < kFw; ++u) {
      const int32_t f = wave * kFw + u;
      cv[u] = (lane < nc && f < F_sel) ? cand[(int64_t)(first + lane) * F_sel + f]
                                       : SplitCand{0.0, -1, 0};
    }
    const int j = lane;  // wave 0: candidate j, previous parent j, earlier nodes j, j + 64
    NodeSeg sg{0, 0, 0, 0};
    long long gq = 0, hq = 0;
    double ppe = 0.0, pe = 0.0, ke_a = 0.0, ke_b = 0.0;
    PartParent pq{0, 0, 0, 0, -1, -1, -1, 0, 0, 0};
    if (wave == 0) {
      if (j < nc) {
        const int64_t c = first + j;
        sg = segs[c];
        gq = totals[2 * c];
        hq = totals[2 * c + 1];
        ppe = a.level == 0 ? 0.0 : prev_parent_e[j >> 1];
      }
      if (j < n_pp) {
        pq = prev_parents[j];
        pe = prev_parent_e[j];
      }
      if (j < first) ke_a = kept_e[j];
      if (j + 64 < first) ke_b = kept_e[j + 64];
    }
    {
      // This wave's best over its features (largest gain, first position of
      // equal gains), for the merge below.
      double pb = 0.0;
      int32_t pf = -1, pbin = 0;
#pragma unroll
      for (int u = 0; u < kFw; ++u) {
        if (cv[u].bin >= 0 && (pf < 0 || cv[u].gain > pb)) {
          pb = cv[u].gain;
          pf = wave * kFw + u;
          pbin = cv[u].bin;
        }
      }
      s_cg[wave * kStageC + lane] = pb;
      s_cpf[wave * kStageC + lane] = pf;
      s_cb[wave * kStageC + lane] = (int16_t)pbin;
    }
    if (wave == 0) {
      if (j < first) s_ke[j] = ke_a;
      if (j + 64 < first) s_ke[j + 64] = ke_b;
    }
    __syncthreads();
    if (wave == 0) {
      // Best split over the features: the waves' bests in feature order
      // (largest gain, first position of equal gains), then the candidate's
      // rank and whether it may be split (est:649-652, 762-801).
      const bool is_cand = j < nc;
      double best = 0.0;
      int32_t bf = -1, bb = 0;
      if (is_cand) {
        double g[kPlanBlock / 64];
        int32_t f[kPlanBlock / 64], b[kPlanBlock / 64];
#pragma unroll
        for (int w = 0; w < kPlanBlock / 64; ++w) {
          g[w] = s_cg[w * kStageC + j];
          f[w] = s_cpf[w * kStageC + j];
          b[w] = s_cb[w * kStageC + j];
        }
#pragma unroll
        for (int w = 0; w < kPlanBlock / 64; ++w) {
          if (f[w] >= 0 && (bf < 0 || g[w] > best)) {
            best = g[w];
            bf = f[w];
            bb = b[w];
          }
        }
      }
      const bool valid = is_cand && sg.valid != 0;
      if (!valid) bf = -1;
      const double gain = bf >= 0 ? best : -1e9;
      double e = 0.0;
      int32_t cand_ok = 0;
      if (valid) {
        const double pv = a.level == 0 ? gain : ppe;
        e = pv < gain ? pv : gain;
        cand_ok = (bf >= 0 && gain > a.gamma) ? 1 : 0;
      }
      // The previous level's parents are kept splits when their children
      // (this level's candidates 2j, 2j + 1) are valid.
      const int32_t v2 = __shfl(valid ? 1 : 0, min(2 * j, 63), 64);
      if (j < n_pp) {
        const double kv = v2 ? pe : -INFINITY;
        s_ke[pq.node] = kv;
        kept_e[pq.node] = kv;
      }
      // With every split kept (a.all_kept), the level's candidates with a
      // split are kept splits too: their ranks, for the count below.
      if (a.all_kept && is_cand) s_e[j] = cand_ok ? e : -INFINITY;
      __builtin_amdgcn_wave_barrier();
      // Expanded: fewer than max_leaves - 1 kept splits ranked above.
      int32_t fl = 0;
      if (cand_ok) {
        int32_t above = 0;
        for (int32_t u0 = 0; u0 < first; u0 += 8) {
          double k8[8];
#pragma unroll
          for (int q = 0; q < 8; ++q) k8[q] = s_ke[u0 + q];
#pragma unroll
          for (int q = 0; q < 8; ++q) above += (u0 + q < first && k8[q] > e) ? 1 : 0;
        }
        if (a.all_kept)
          for (int32_t q = 0; q < nc; ++q) above += (q != j && s_e[q] > e) ? 1 : 0;
        fl = above < a.max_leaves - 1 ? 1 : 0;
      }
      const uint32_t fincl = wave_incl_scan<uint32_t>((uint32_t)fl);
      const uint32_t pidx = fincl - (uint32_t)fl;
      const int32_t n_exp = (int32_t)wave_lane(fincl, 63);
      const int64_t n_new = (int64_t)n_prev + 2 * (int64_t)n_exp;
      int32_t status = n_new > a.node_cap ? 1 : 0;
      int32_t n_groups = n_exp;
      uint32_t tcar = 0, hcar = 0;
      int32_t th = 0;
      if (status == 0) {
        // Partition tiles, each lane's item in order: in place every
        // candidate and grouped every previous parent (counted by the
        // launch's other blocks, plan_count_role, whether or not a side is
        // expanded); moving, the expanded parents (k_part_count).
        uint32_t ntc = 0u;
        if (a.mode == kLevelInPlace)
          ntc = is_cand ? count_item_tiles(sg.start, sg.count, sg.valid != 0, a.part_tile) : 0u;
        else if (grouped)
          ntc = j < n_pp ? count_item_tiles(pq.start, pq.count, true, a.part_tile) : 0u;
        else
          ntc = fl ? count_item_tiles(sg.start, sg.count, true, a.part_tile) : 0u;
        const uint32_t cincl = wave_incl_scan<uint32_t>(ntc);
        const uint32_t cpre = cincl - ntc;
        tcar = wave_lane(cincl, 63);
        // A grouped level's groups: every previous parent, par -1 for a side
        // that is not expanded (its rows stay), tiles over its segment.
        if (grouped) {
          const int32_t pid_or = fl ? (int32_t)pidx : -1;
          const int32_t pl = __shfl(pid_or, min(2 * j, 63), 64);
          const int32_t pr = __shfl(pid_or, min(2 * j + 1, 63), 64);
          if (j < n_pp) {
            PartGroup G;
            G.start = pq.start;
            G.count = pq.count;
            G.fpos = pq.fpos;
            G.bin = pq.bin;
            G.par[0] = pl;
            G.par[1] = pr;
            groups[j] = G;
            s_tb[j] = (int32_t)cpre;
            s_gs[j] = pq.start & ~int64_t(15);
            tile_begin[j] = (int32_t)cpre;
          }
          if (j == 0) {
            s_tb[n_pp] = (int32_t)tcar;
            tile_begin[n_pp] = (int32_t)tcar;
          }
          n_groups = n_pp;
        }
        // The tiles that count a candidate's rows: its own, or grouped its
        // previous parent's (j >> 1).
        const uint32_t g0 = __shfl(cpre, j >> 1, 64), g1 = __shfl(cpre + ntc, j >> 1, 64);
        const uint32_t t0 = grouped ? g0 : cpre, t1 = grouped ? g1 : cpre + ntc;
        // Records, parents, ranks; rows to build.
        unsigned long long rows = 0;
        if (is_cand) {
          const int32_t v = first + j;
          const int32_t L = fl ? n_prev + 2 * (int32_t)pidx : -1;
          NodeOut N;
          N.start = sg.start;
          N.count = sg.count;
          N.Gq = valid ? gq : 0;
          N.Hq = valid ? hq : 0;
          N.gain = gain;
          N.e = e;
          N.fpos = bf;
          N.bin = bf >= 0 ? bb : 0;
          N.valid = sg.valid;
          N.left = L;
          nodes[v] = N;
          if (!fl) {
            kept_e[v] = -INFINITY;
          } else {
            const int32_t i = (int32_t)pidx;
            PartParent P;
            P.start = N.start;
            P.count = N.count;
            P.fpos = N.fpos;
            P.bin = N.bin;
            P.left_id = L;
            P.right_id = L + 1;
            P.node = v;
            P.gslot = grouped ? j : 2 * i;  // grouped: 2 * group (j >> 1) + side
            P.tile0 = (int32_t)t0;
            P.tile1 = (int32_t)t1;
            parents[i] = P;
            parent_e[i] = N.e;
            if (a.mode == kLevelMove) {
              s_tb[i] = (int32_t)cpre;
              s_gs[i] = N.start & ~int64_t(15);
              tile_begin[i] = (int32_t)cpre;
            }
            s_count[i] = N.count;
            rows = (unsigned long long)(N.count / 2);  // at most the smaller child's
          }
        }
        if (a.mode == kLevelMove && j == 0) {
          s_tb[n_exp] = (int32_t)tcar;
          tile_begin[n_exp] = (int32_t)tcar;
        }
        rows = wave_sum(rows);
        __builtin_amdgcn_wave_barrier();
        // Rows per histogram task: sized for the smaller children's rows;
        // in place a task tiles twice as many of its parent's rows, of which
        // it adds those of the smaller child (at most half).
        th = plan_tile_rows((int64_t)rows, a) * (a.mode == kLevelInPlace ? 2 : 1);
        uint32_t nh = 0;
        if (j < n_exp) {
          const int64_t cnt = s_count[j];
          nh = a.last ? 0u
                      : a.mode == kLevelInPlace ? (uint32_t)max((int64_t)1, div_pos(cnt + th - 1, th))
                                                : (uint32_t)div_pos(cnt / 2 + th, th);
        }
        const uint32_t hincl = wave_incl_scan<uint32_t>(nh);
        const uint32_t hpre = hincl - nh;
        hcar = wave_lane(hincl, 63);
        if (tcar > (uint32_t)a.tile_cap || hcar > (uint32_t)a.hist_cap) {
          status = 2;  // capacities are sized from proven bounds; reaching this is a bug
        } else {
          if (j < n_exp) {
            s_hb[j] = (int32_t)hpre;
            hist_begin[j] = (int32_t)hpre;
          }
          if (j == 0) {
            s_hb[n_exp] = (int32_t)hcar;
            hist_begin[n_exp] = (int32_t)hcar;
          }
        }
      }
      if (j == 0) {
        s_fast[0] = status;
        s_fast[1] = n_exp;
        s_fast[2] = n_groups;
        s_fast[3] = (int32_t)tcar;
        s_fast[4] = (int32_t)hcar;
        s_fast[5] = th;
        s_fast[6] = (int32_t)min(n_new, (int64_t)INT32_MAX);
      }
    }
    __syncthreads();
    const int32_t status = s_fast[0], n_exp = s_fast[1], n_groups = s_fast[2];
    const int32_t tcar = s_fast[3], hcar = s_fast[4];
    if (status != 0) {
      if (tid == 0) {
        LevelPlan q = {};
        q.first_child = n_prev;
        q.tile_rows = 4096;
        q.n_nodes = n_prev;
        q.overflow = status == 1 ? s_fast[6] : -1;
        *plan = q;
        plan_next_level(level_out, n_prev, 0);
      }
      return;
    }
    // Tile and histogram-task lists: item -> its group (parent) by binary
    // search.  (In place the counting blocks tile the candidates themselves:
    // no tile list.)
    const int32_t listed = a.mode == kLevelInPlace ? 0 : tcar;
    for (int t = tid; t < listed; t += kPlanBlock) {
      int lo = 0, hi = n_groups - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_tb[mid] <= t) lo = mid;
        else hi = mid - 1;
      }
      PartTile T;
      T.row0 = s_gs[lo] + (int64_t)(t - s_tb[lo]) * a.part_tile;
      T.rows = a.part_tile;
      T.parent = lo;
      tiles[t] = T;
    }
    for (int q = tid; q < hcar; q += kPlanBlock) {
      int lo = 0, hi = n_exp - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_hb[mid] <= q) lo = mid;
        else hi = mid - 1;
      }
      hist_tasks[q] = HistTask{lo, q - s_hb[lo]};
    }
    if (tid == 0) {
      LevelPlan q;
      q.n_parents = n_exp;
      q.n_tiles = tcar;
      q.n_hist = hcar;
      q.n_split = 2 * n_exp;
      q.first_child = n_prev;
      q.tile_rows = s_fast[5];
      q.n_nodes = (int32_t)((int64_t)n_prev + 2 * (int64_t)n_exp);
      q.overflow = 0;
      *plan = q;
      plan_next_level(level_out, n_prev, 2 * n_exp);
    }
    return;
  }
  if (tid == 0) s_rows = 0ull;

  // Every input at once: earlier ranks, the previous parents' ids and ranks,
  // and the candidates' segments, totals and split candidates.  The earlier
  // ranks go through registers so that their LDS stores wait after every
  // load is issued.  (first <= kPlanLdsC + 1 <= kPlanBlock: one per thread.)
  const double ke0 = tid < first ? kept_e[tid] : 0.0;
  PartParent pq{0, 0, 0, 0, -1, -1, -1, 0, 0, 0};  // previous parent tid (a grouped level's grandparent)
  double pe = 0.0;
  if (tid < n_pp) {
    pq = prev_parents[tid];
    pe = prev_parent_e[tid];
  }
  const int32_t pnode = pq.node;
  if (nc <= kStageC && F_sel <= kStageF) {
    // Staged: the level's split candidates (nc x F_sel consecutive records)
    // in one coalesced pass of the whole block, transposed into LDS; then
    // one lane per candidate takes the best over its features in order
    // (largest gain, lowest position on ties: the first of equal gains).
    const int32_t E = nc * F_sel;
    SplitCand cv[kStageC * kStageF / kPlanBlock];
#pragma unroll
    for (int k = 0; k < kStageC * kStageF / kPlanBlock; ++k) {
      const int32_t e = tid + k * kPlanBlock;
      cv[k] = e < E ? cand[(int64_t)first * F_sel + e] : SplitCand{0.0, -1, 0};
    }
    NodeSeg sg{0, 0, 0, 0};
    long long gq = 0, hq = 0;
    double ppe = 0.0;
    if (tid < nc) {
      const int64_t c = first + tid;
      sg = segs[c];
      gq = totals[2 * c];
      hq = totals[2 * c + 1];
      ppe = a.level == 0 ? 0.0 : prev_parent_e[tid >> 1];
    }
    if (tid < first) s_ke[tid] = ke0;
#pragma unroll
    for (int k = 0; k < kStageC * kStageF / kPlanBlock; ++k) {
      const int32_t e = tid + k * kPlanBlock;
      if (e < E) {
        const int32_t j = e / F_sel, f = e - j * F_sel;
        s_cg[f * kStageC + j] = cv[k].gain;
        s_cb[f * kStageC + j] = (int16_t)cv[k].bin;
      }
    }
    __syncthreads();
    if (tid < nc) {
      double best = 0.0;
      int32_t bf = -1, bb = 0;
      // Eight features' reads in flight, then their comparisons in order.
      for (int32_t f0 = 0; f0 < F_sel; f0 += 8) {
        double g[8];
        int32_t b[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int32_t f = min(f0 + u, kStageF - 1);
          g[u] = s_cg[f * kStageC + tid];
          b[u] = s_cb[f * kStageC + tid];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          if (f0 + u < F_sel && b[u] >= 0 && (bf < 0 || g[u] > best)) {
            best = g[u];
            bf = f0 + u;
            bb = b[u];
          }
        }
      }
      plan_record(tid, sg, gq, hq, ppe, best, bf, bb, a, s_start, s_count, s_gq, s_hq, s_gain,
                  s_e, s_fpos, s_bin, s_valid, s_flag);
    }
  } else {
    // Four candidates per wave and pass, one lane per feature (one pass for
    // up to 64 candidates).
    constexpr int kPer = 4;
    for (int jb = wave * kPer; jb < nc; jb += (kPlanBlock / 64) * kPer) {
      NodeSeg sg[kPer];
      long long gq[kPer], hq[kPer];
      double ppe[kPer];
      SplitCand cf[kPer];
#pragma unroll
      for (int q = 0; q < kPer; ++q) {
        const int j = min(jb + q, nc - 1);
        const int64_t c = first + j;
        sg[q] = segs[c];
        gq[q] = totals[2 * c];
        hq[q] = totals[2 * c + 1];
        ppe[q] = a.level == 0 ? 0.0 : prev_parent_e[j >> 1];
        cf[q] = lane < F_sel ? cand[c * F_sel + lane] : SplitCand{0.0, -1, 0};
      }
      if (jb == wave * kPer && tid < first) s_ke[tid] = ke0;
#pragma unroll
      for (int q = 0; q < kPer; ++q) {
        const int j = jb + q;
        const int64_t c = first + min(j, nc - 1);
        // Best over the features: largest gain, lowest position on ties.
        double best = 0.0;
        int32_t bf = -1, bb = 0;
        if (cf[q].bin >= 0) {
          best = cf[q].gain;
          bf = lane;
          bb = cf[q].bin;
        }
        for (int f = lane + 64; f < F_sel; f += 64) {
          const SplitCand x = cand[c * F_sel + f];
          if (x.bin >= 0 && (bf < 0 || x.gain > best)) {
            best = x.gain;
            bf = f;
            bb = x.bin;
          }
        }
        wave_argmax(best, bf, bb);
        if (lane == 0 && j < nc)
          plan_record(j, sg[q], gq[q], hq[q], ppe[q], best, bf, bb, a, s_start, s_count, s_gq,
                      s_hq, s_gain, s_e, s_fpos, s_bin, s_valid, s_flag);
      }
    }
    // (Waves that took no candidate store their earlier ranks here.)
    if (wave * kPer >= nc && tid < first) s_ke[tid] = ke0;
  }
  __syncthreads();

  // The previous level's parents are kept splits when their children (this
  // level's candidates 2i, 2i+1) are valid.
  if (tid < n_pp) {
    const double kv = s_valid[2 * tid] ? pe : -INFINITY;
    s_ke[pnode] = kv;
    kept_e[pnode] = kv;
  }
  __syncthreads();

  // Expanded: valid, a split above gamma, and fewer than max_leaves - 1 kept
  // splits ranked above it.
  // With every split kept (a.all_kept), the level's other candidates with a
  // split count as well.
  int32_t fl = 0;
  if (tid < nc && s_flag[tid]) {
    const double ev = s_e[tid];
    int32_t above = 0;
    for (int u = 0; u < first; ++u) above += s_ke[u] > ev ? 1 : 0;
    if (a.all_kept)
      for (int u = 0; u < nc; ++u) above += (u != tid && s_flag[u] && s_e[u] > ev) ? 1 : 0;
    fl = above < a.max_leaves - 1 ? 1 : 0;
  }
  uint32_t n_exp_u;
  const uint32_t pidx = block_excl_scan<kPlanBlock>((uint32_t)fl, stmp, n_exp_u);
  const int32_t n_exp = (int32_t)n_exp_u;
  const int64_t n_new = (int64_t)n_prev + 2 * (int64_t)n_exp;
  if (n_new > a.node_cap) {
    if (tid == 0) {
      LevelPlan q = {};
      q.first_child = n_prev;
      q.tile_rows = 4096;
      q.n_nodes = n_prev;
      q.overflow = (int32_t)min(n_new, (int64_t)INT32_MAX);
      *plan = q;
      plan_next_level(level_out, n_prev, 0);
    }
    return;
  }

  // Partition tiles, one item per thread in order (as the fast path): in
  // place every candidate and grouped every previous parent (counted by the
  // launch's other blocks, plan_count_role), moving the expanded parents
  // (k_part_count).  Item i's tiles are [s_ctb[i], s_ctb[i + 1]).
  {
    uint32_t ntc = 0u;
    if (a.mode == kLevelInPlace) {
      if (tid < nc) ntc = count_item_tiles(s_start[tid], s_count[tid], s_valid[tid] != 0, a.part_tile);
    } else if (grouped) {
      if (tid < n_pp) ntc = count_item_tiles(pq.start, pq.count, true, a.part_tile);
    } else if (fl) {
      ntc = count_item_tiles(s_start[tid], s_count[tid], true, a.part_tile);
    }
    uint32_t ctot;
    const uint32_t cpre = block_excl_scan<kPlanBlock>(ntc, stmp, ctot);
    if (tid < kPlanLdsC) s_ctb[tid] = cpre;
    if (tid == 0) {
      s_ctb[kPlanLdsC] = ctot;
      s_tcar = ctot;
    }
    __syncthreads();
  }

  // A grouped level's groups: every previous parent, par -1 for a side
  // that is not expanded (its rows stay), tiles over its segment.
  if (grouped) {
    if (tid < nc) s_pidx[tid] = fl ? (int32_t)pidx : -1;
    __syncthreads();
    if (tid < n_pp) {
      PartGroup G;
      G.start = pq.start;
      G.count = pq.count;
      G.fpos = pq.fpos;
      G.bin = pq.bin;
      G.par[0] = s_pidx[2 * tid];
      G.par[1] = s_pidx[2 * tid + 1];
      groups[tid] = G;
      s_tb[tid] = (int32_t)s_ctb[tid];
      s_gs[tid] = pq.start & ~int64_t(15);
      tile_begin[tid] = (int32_t)s_ctb[tid];
    }
    if (tid == 0) {
      s_tb[n_pp] = (int32_t)s_ctb[n_pp];
      tile_begin[n_pp] = (int32_t)s_ctb[n_pp];
    }
  }

  // Records, parents, ranks; rows to build.
  unsigned long long rows = 0;
  if (tid < nc) {
    const int32_t v = first + tid;
    const int32_t L = fl ? n_prev + 2 * (int32_t)pidx : -1;
    NodeOut N;
    N.start = s_start[tid];
    N.count = s_count[tid];
    N.Gq = s_gq[tid];
    N.Hq = s_hq[tid];
    N.gain = s_gain[tid];
    N.e = s_e[tid];
    N.fpos = s_fpos[tid];
    N.bin = s_bin[tid];
    N.valid = s_valid[tid];
    N.left = L;
    nodes[v] = N;
    if (!fl) {
      kept_e[v] = -INFINITY;
    } else {
      const int32_t i = (int32_t)pidx;
      PartParent P;
      P.start = N.start;
      P.count = N.count;
      P.fpos = N.fpos;
      P.bin = N.bin;
      P.left_id = L;
      P.right_id = L + 1;
      P.node = v;
      P.gslot = grouped ? tid : 2 * i;  // grouped: 2 * group (tid >> 1) + side
      const int32_t it = grouped ? (tid >> 1) : tid;  // the item counting its rows
      P.tile0 = (int32_t)s_ctb[it];
      P.tile1 = (int32_t)s_ctb[it + 1];
      parents[i] = P;
      parent_e[i] = N.e;
      if (a.mode == kLevelMove) {
        s_tb[i] = (int32_t)s_ctb[tid];
        s_gs[i] = N.start & ~int64_t(15);
        tile_begin[i] = (int32_t)s_ctb[tid];
      }
      s_pj[i] = tid;
      rows = (unsigned long long)(N.count / 2);  // at most the smaller child's
    }
  }
  if (a.mode == kLevelMove && tid == 0) {
    s_tb[n_exp] = (int32_t)s_tcar;
    tile_begin[n_exp] = (int32_t)s_tcar;
  }
  rows = wave_sum(rows);
  if (lane == 0 && rows) atomicAdd(&s_rows, rows);
  __syncthreads();
  // Rows per histogram task: sized for the smaller children's rows; in
  // place a task tiles twice as many of its parent's rows, of which it adds
  // those of the smaller child (at most half).
  const int32_t th = plan_tile_rows((int64_t)s_rows, a) * (a.mode == kLevelInPlace ? 2 : 1);

  // Exclusive offsets of each parent's histogram tasks.
  uint32_t nh = 0;
  if (tid < n_exp) {
    const int64_t cnt = s_count[s_pj[tid]];
    nh = a.last ? 0u
                : a.mode == kLevelInPlace ? (uint32_t)max((int64_t)1, div_pos(cnt + th - 1, th))
                                          : (uint32_t)div_pos(cnt / 2 + th, th);
  }
  uint32_t hcar;
  const uint32_t hp = block_excl_scan<kPlanBlock>(nh, stmp, hcar);
  const uint32_t tcar = s_tcar;
  if (tcar > (uint32_t)a.tile_cap || hcar > (uint32_t)a.hist_cap) {
    // Capacities are sized from proven bounds; reaching this is a bug.
    if (tid == 0) {
      LevelPlan q = {};
      q.first_child = n_prev;
      q.tile_rows = 4096;
      q.n_nodes = n_prev;
      q.overflow = -1;
      *plan = q;
      plan_next_level(level_out, n_prev, 0);
    }
    return;
  }
  if (tid < n_exp) {
    s_hb[tid] = (int32_t)hp;
    hist_begin[tid] = (int32_t)hp;
  }
  if (tid == 0) {
    s_hb[n_exp] = (int32_t)hcar;
    hist_begin[n_exp] = (int32_t)hcar;
  }
  __syncthreads();

  // Tile and histogram-task lists: item -> its group (parent) by binary
  // search.  (In place the counting blocks tile the candidates themselves:
  // no tile list.)
  const int32_t n_groups = grouped ? n_pp : n_exp;
  const int32_t listed = a.mode == kLevelInPlace ? 0 : (int32_t)tcar;
  for (int t = tid; t < listed; t += kPlanBlock) {
    int lo = 0, hi = n_groups - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_tb[mid] <= t) lo = mid;
      else hi = mid - 1;
    }
    PartTile T;
    T.row0 = s_gs[lo] + (int64_t)(t - s_tb[lo]) * a.part_tile;
    T.rows = a.part_tile;
    T.parent = lo;
    tiles[t] = T;
  }
  for (int q = tid; q < (int)hcar; q += kPlanBlock) {
    int lo = 0, hi = n_exp - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_hb[mid] <= q) lo = mid;
      else hi = mid - 1;
    }
    hist_tasks[q] = HistTask{lo, q - s_hb[lo]};
  }
  if (tid == 0) {
    LevelPlan q;
    q.n_parents = n_exp;
    q.n_tiles = (int32_t)tcar;
    q.n_hist = (int32_t)hcar;
    q.n_split = 2 * n_exp;
    q.first_child = n_prev;
    q.tile_rows = th;
    q.n_nodes = (int32_t)n_new;
    q.overflow = 0;
    *plan = q;
    plan_next_level(level_out, n_prev, 2 * n_exp);
  }
}

hipError_t launch_plan_lds(hipStream_t st, NodeOut *nodes, LevelPlan *plan,
                           const PartParent *prev_parents, PartParent *parents,
                           PartGroup *groups,
                           int32_t *tile_begin, int32_t *hist_begin, PartTile *tiles,
                           HistTask *hist_tasks, const NodeSeg *segs,
                           const long long *totals, const SplitCand *cand, double *kept_e,
                           const double *prev_parent_e, double *parent_e, int32_t F_sel,
                           PlanArgs a, const uint8_t *codes_c, int64_t ld_c,
                           int32_t *tile_cnt, const int32_t *level_in, int32_t *level_out,
                           int32_t count_blocks) {
  if (a.fused_count && (a.part_rows != 4 && a.part_rows != 8 && a.part_rows != 16))
    return hipErrorInvalidValue;
  const unsigned grid = 1u + (a.fused_count ? (unsigned)std::max(1, count_blocks) : 0u);
  hipLaunchKernelGGL(k_plan_lds, dim3(grid), dim3(kPlanBlock), 0, st, nodes, plan, prev_parents,
                     parents, groups, tile_begin, hist_begin, tiles, hist_tasks, segs,
                     totals, cand, kept_e, prev_parent_e, parent_e, F_sel, a, codes_c, ld_c,
                     tile_cnt, level_in, level_out);
  return hipGetLastError();
}

hipError_t launch_plan(hipStream_t st, NodeOut *nodes, LevelPlan *plan,
                       const PartParent *prev_parents, PartParent *parents,
                       int32_t *tile_begin, int32_t *hist_begin,
                       PartTile *tiles, HistTask *hist_tasks,
                       int32_t *work_flag,
                       double *work_e, const NodeSeg *segs, const long long *totals,
                       const SplitCand *cand, int32_t F_sel, PlanArgs a) {
  hipLaunchKernelGGL(k_plan, dim3(1), dim3(kPlanBlock), 0, st, nodes, plan,
                     prev_parents, parents, tile_begin, hist_begin, tiles,
                     hist_tasks, work_flag, work_e, segs, totals, cand, F_sel,
                     a);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// F update and training loss (est:2896-2897, est:2905 -> est:2320-2325).
// ---------------------------------------------------------------------------
constexpr int kUpdBlock = 256;
constexpr int kUpdRows = 4;  // rows a thread walks at once

// One pass of kUpdRows rows per thread where the grid allows (every row's
// chain of code loads in flight at once), at most 8192 blocks.
int update_F_blocks(int64_t n) {
  int64_t b = (n + kUpdBlock * kUpdRows - 1) / (kUpdBlock * kUpdRows);
  if (b < 1) b = 1;
  if (b > 8192) b = 8192;
  return (int)b;
}

__device__ __forceinline__ int32_t traverse(const TreeNodeDev *__restrict__ tree,
                                            const uint8_t *__restrict__ codes,
                                            int64_t ld, int64_t i) {
  int32_t node = 0;
  TreeNodeDev nd = tree[0];
  while (nd.feature >= 0) {
    const int32_t c = codes[(int64_t)nd.feature * ld + i];
    node = (c <= nd.threshold) ? nd.left : nd.right;
    nd = tree[node];
  }
  return node;
}

// F += lr * tree(x) for every row (est:2896-2897) and the log-loss of the
// new F (est:2320-2325, est:2905), partial sums per block.  The tree sits in
// LDS (up to kUpdTreeLds nodes) and each thread walks four rows at once, so
// four chains of dependent code loads are in flight per thread.
constexpr int kUpdTreeLds = 1024;

#pragma clang fp contract(off)
__device__ __forceinline__ double row_loss(double f, uint8_t yi) {
  const double fc = fmin(fmax(f, -500.0), 500.0);
  double p = 1.0 / (1.0 + exp(-fc));
  p = fmin(fmax(p, 1e-15), 1.0 - 1e-15);
  return yi ? log(p) : log(1.0 - p);
}

// row_loss, and the row's gradient and hessian of the next round from the
// same p (logistic_gh's expressions: the next round's k_gather_gh computes
// the same values from the same F).
__device__ __forceinline__ double row_loss_gh(double f, uint8_t yi, double w, double &g,
                                              double &h) {
  const double fc = fmin(fmax(f, -500.0), 500.0);
  const double p = 1.0 / (1.0 + exp(-fc));
  g = __dmul_rn(w, __dsub_rn(p, (double)yi));
  h = __dmul_rn(__dmul_rn(w, p), __dsub_rn(1.0, p));
  const double pc = fmin(fmax(p, 1e-15), 1.0 - 1e-15);
  return yi ? log(pc) : log(1.0 - pc);
}

// Raises out[0], out[1] to the block's largest |g| and h (bit patterns of
// non-negative doubles order as unsigned integers).  A block whose maxima
// do not exceed what it reads issues no atomic.
__device__ __forceinline__ void block_gh_max(double gm, double hm, unsigned long long *out) {
  __shared__ double s_mx[kUpdBlock / 64][2];
  for (int o = 32; o >= 1; o >>= 1) {
    gm = fmax(gm, __shfl_xor(gm, o, 64));
    hm = fmax(hm, __shfl_xor(hm, o, 64));
  }
  if (lane_id() == 0) {
    s_mx[threadIdx.x >> 6][0] = gm;
    s_mx[threadIdx.x >> 6][1] = hm;
  }
  __syncthreads();
  if (threadIdx.x < 2) {
    double v = 0.0;
    for (int w = 0; w < kUpdBlock / 64; ++w) v = fmax(v, s_mx[w][threadIdx.x]);
    const unsigned long long bits = (unsigned long long)__double_as_longlong(v);
    unsigned long long *dst = out + threadIdx.x;
    if (bits > __hip_atomic_load(dst, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
      (void)__hip_atomic_fetch_max(dst, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

__global__ __launch_bounds__(kUpdBlock) void k_update_F(
    const uint8_t *__restrict__ codes, int64_t ld, int64_t n,
    const TreeNodeDev *__restrict__ tree, int32_t tree_len,
    const int32_t *__restrict__ node_count_d, double lr, double *__restrict__ F,
    const uint8_t *__restrict__ y, double *__restrict__ partials, double w0, double w1,
    unsigned long long *__restrict__ gh_max_out, unsigned long long *__restrict__ gh_max_clear) {
  __shared__ double red[kUpdBlock / 64];
  __shared__ TreeNodeDev st[kUpdTreeLds];
  if (gh_max_clear && blockIdx.x == 0 && threadIdx.x < 2) gh_max_clear[threadIdx.x] = 0ull;
  const bool apply = tree_len > 0 && (!node_count_d || *node_count_d > 0);
  const bool lds = tree_len <= kUpdTreeLds;
  if (apply && lds)
    for (int32_t k = (int32_t)threadIdx.x; k < tree_len; k += kUpdBlock) st[k] = tree[k];
  __syncthreads();
  const TreeNodeDev *tr = lds ? st : tree;
  double acc = 0.0, gm = 0.0, hm = 0.0;
  const int64_t step = (int64_t)gridDim.x * kUpdBlock * kUpdRows;
  for (int64_t base = (int64_t)blockIdx.x * kUpdBlock * kUpdRows + threadIdx.x; base < n;
       base += step) {
    int64_t i[kUpdRows];
    bool in[kUpdRows];
    double f[kUpdRows];
#pragma unroll
    for (int r = 0; r < kUpdRows; ++r) {
      i[r] = base + (int64_t)r * kUpdBlock;
      in[r] = i[r] < n;
      f[r] = in[r] ? F[i[r]] : 0.0;
    }
    if (apply) {
      TreeNodeDev nd[kUpdRows];
      int32_t node[kUpdRows];
#pragma unroll
      for (int r = 0; r < kUpdRows; ++r) {
        node[r] = 0;
        nd[r] = tr[0];
      }
      bool more = true;
      while (more) {
        int32_t c[kUpdRows];
#pragma unroll
        for (int r = 0; r < kUpdRows; ++r)
          c[r] = (in[r] && nd[r].feature >= 0) ? codes[(int64_t)nd[r].feature * ld + i[r]] : 0;
        more = false;
#pragma unroll
        for (int r = 0; r < kUpdRows; ++r) {
          if (in[r] && nd[r].feature >= 0) {
            node[r] = (c[r] <= nd[r].threshold) ? nd[r].left : nd[r].right;
            nd[r] = tr[node[r]];
            more = more || nd[r].feature >= 0;
          }
        }
      }
#pragma unroll
      for (int r = 0; r < kUpdRows; ++r)
        if (in[r]) {
          f[r] = __dadd_rn(f[r], __dmul_rn(lr, nd[r].value));
          F[i[r]] = f[r];
        }
    }
    if (gh_max_out) {
#pragma unroll
      for (int r = 0; r < kUpdRows; ++r)
        if (in[r]) {
          const uint8_t yi = y[i[r]];
          double g, h;
          acc += row_loss_gh(f[r], yi, yi ? w1 : w0, g, h);
          gm = fmax(gm, fabs(g));
          hm = fmax(hm, h);
        }
    } else {
#pragma unroll
      for (int r = 0; r < kUpdRows; ++r)
        if (in[r]) acc += row_loss(f[r], y[i[r]]);
    }
  }
  for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, 64);
  if (lane_id() == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    double s = 0.0;
    for (int w = 0; w < kUpdBlock / 64; ++w) s += red[w];
    partials[blockIdx.x] = s;
  }
  if (gh_max_out) block_gh_max(gm, hm, gh_max_out);
}
#pragma clang fp contract(on)

hipError_t launch_update_F(hipStream_t st, const uint8_t *codes, int64_t ld,
                           int64_t n, const TreeNodeDev *tree, int32_t tree_len,
                           const int32_t *node_count_d, double lr, double *F,
                           const uint8_t *y, double *loss_partials,
                           int32_t n_blocks, double w0, double w1,
                           unsigned long long *gh_max_out,
                           unsigned long long *gh_max_clear) {
  hipLaunchKernelGGL(k_update_F, dim3((unsigned)n_blocks), dim3(kUpdBlock), 0, st,
                     codes, ld, n, tree, tree_len, node_count_d, lr, F, y, loss_partials,
                     w0, w1, gh_max_out, gh_max_clear);
  return hipGetLastError();
}

// Fixed-order sum of the per-block partials (deterministic).
__global__ __launch_bounds__(256) void k_sum_partials(const double *__restrict__ p,
                                                      int32_t count,
                                                      double *__restrict__ out) {
  __shared__ double red[4];
  double acc = 0.0;
  for (int i = threadIdx.x; i < count; i += 256) acc += p[i];
  for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, 64);
  if (lane_id() == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) *out = (red[0] + red[1]) + (red[2] + red[3]);
}

hipError_t launch_sum_partials(hipStream_t st, const double *partials,
                               int32_t count, double *out) {
  hipLaunchKernelGGL(k_sum_partials, dim3(1), dim3(256), 0, st, partials, count,
                     out);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Best-first replay (est:641-820) on the device, so a boosting round needs
// no host round trip between the tree and the F update.  One wave; the
// candidate slots (max_leaves + 2 of them) live in LDS.  Same steps as the
// host replay in engine.hip: pop the active slot with the largest gain
// above gamma (the lowest slot on ties); a node whose split was rejected
// becomes a leaf; a kept split numbers its children left then right, puts
// the smaller child in the first free slot and the larger in the next.
// ---------------------------------------------------------------------------
__device__ __forceinline__ double leaf_value(const NodeOut &nd, const ReplayArgs &a) {
  const double G = (double)nd.Gq * a.g_scale;
  const double H = (double)nd.Hq * a.h_scale;
  return -G / (H + a.reg_lambda);
}

constexpr int kReplayNodes = 1024;            // node records staged in LDS
constexpr int kReplayOut = 2 * kReplaySlots + 2;  // output nodes of the largest tree

// LDS of k_replay (one wave): node records (gain, leaf value, size, split,
// first child, kept flag); candidate slots (output id, internal id, gain or
// -inf when the candidate cannot be split, active flag); the output tree as
// (internal node, left child or -1) per output node.
__shared__ double rp_gain[kReplayNodes], rp_val[kReplayNodes];
__shared__ int32_t rp_count[kReplayNodes], rp_fpos[kReplayNodes], rp_left[kReplayNodes];
__shared__ uint8_t rp_valid[kReplayNodes], rp_bin[kReplayNodes];
__shared__ int32_t rs_node[kReplaySlots], rs_int[kReplaySlots];
__shared__ double rs_gain[kReplaySlots];
__shared__ uint8_t rs_active[kReplaySlots];
__shared__ int32_t ro_int[kReplayOut], ro_left[kReplayOut];

// Node fields from the LDS records (kStaged) or from the table in HBM.
template <bool kStaged> struct ReplayNodes {
  const NodeOut *nodes;
  ReplayArgs a;
  __device__ double gain(int32_t i) const { return kStaged ? rp_gain[i] : nodes[i].gain; }
  __device__ double val(int32_t i) const { return kStaged ? rp_val[i] : leaf_value(nodes[i], a); }
  __device__ int64_t count(int32_t i) const { return kStaged ? (int64_t)rp_count[i] : nodes[i].count; }
  __device__ int32_t fpos(int32_t i) const { return kStaged ? rp_fpos[i] : nodes[i].fpos; }
  __device__ int32_t bin(int32_t i) const { return kStaged ? (int32_t)rp_bin[i] : nodes[i].bin; }
  __device__ int32_t left(int32_t i) const { return kStaged ? rp_left[i] : nodes[i].left; }
  __device__ int32_t valid(int32_t i) const { return kStaged ? (int32_t)rp_valid[i] : nodes[i].valid; }
};

// Largest value over the wave, returned to every lane: DPP shifts within
// rows of 16 lanes, then row broadcasts (lane 63 ends with the maximum),
// then a read of lane 63.  Lanes without a source keep their own value.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ double dpp_max_step(double x) {
  const int hi = __builtin_amdgcn_update_dpp(__double2hiint(x), __double2hiint(x), kCtrl, kRowMask, 0xf, false);
  const int lo = __builtin_amdgcn_update_dpp(__double2loint(x), __double2loint(x), kCtrl, kRowMask, 0xf, false);
  return fmax(x, __hiloint2double(hi, lo));
}

__device__ __forceinline__ double wave_max_f64(double x) {
  x = dpp_max_step<0x111, 0xf>(x);  // row_shr:1
  x = dpp_max_step<0x112, 0xf>(x);  // row_shr:2
  x = dpp_max_step<0x114, 0xf>(x);  // row_shr:4
  x = dpp_max_step<0x118, 0xf>(x);  // row_shr:8
  x = dpp_max_step<0x142, 0xa>(x);  // row_bcast:15 into rows 1 and 3
  x = dpp_max_step<0x143, 0xc>(x);  // row_bcast:31 into rows 2 and 3
  const int hi = __builtin_amdgcn_readlane(__double2hiint(x), 63);
  const int lo = __builtin_amdgcn_readlane(__double2loint(x), 63);
  return __hiloint2double(hi, lo);
}

// Puts internal node v in slot k as output node `id`.
template <bool kStaged>
__device__ __forceinline__ void replay_set_slot(const ReplayNodes<kStaged> &N, int32_t k,
                                                int32_t id, int32_t v) {
  rs_node[k] = id;
  rs_int[k] = v;
  rs_gain[k] = N.fpos(v) >= 0 ? N.gain(v) : -INFINITY;
  rs_active[k] = 1;
}

// The candidate loop; returns the node count (0 with *status set on error).
template <bool kStaged>
__device__ int32_t replay_loop(const ReplayNodes<kStaged> &N, int32_t C, int32_t *status) {
  const int lane = (int)threadIdx.x;
  const ReplayArgs &a = N.a;
  for (int32_t i = lane; i < C; i += 64) {
    rs_active[i] = 0;
    rs_gain[i] = -INFINITY;
  }
  __syncthreads();
  int32_t node_count = 1;
  if (lane == 0) {
    ro_int[0] = 0;
    ro_left[0] = -1;
  }
  if (N.fpos(0) < 0) return 1;  // the root is the only leaf (est:575-579, 632-637)
  if (lane == 0) replay_set_slot(N, 0, 0, 0);
  __syncthreads();
  int32_t n_splits = 0;
  while (n_splits < a.max_leaves - 1) {
    // The largest gain above gamma, at the lowest slot holding it.
    double lmax = -INFINITY;
    for (int32_t i = lane; i < C; i += 64) lmax = fmax(lmax, rs_gain[i]);  // -inf: not a candidate
    const double best = wave_max_f64(lmax);
    if (!(best > a.gamma)) break;
    int32_t ci = -1;
    for (int32_t base = 0; base < C && ci < 0; base += 64) {
      const int32_t i = base + lane;
      const unsigned long long m = __ballot(i < C && rs_gain[i] == best);
      if (m) ci = base + __builtin_ctzll(m);
    }
    const int32_t v = rs_int[ci];
    const int32_t cur = rs_node[ci];
    const int32_t l = N.left(v);
    if (l < 0) {
      *status = 2;
      return 0;
    }
    if (!N.valid(l)) {  // est:678-683: the node stays a leaf
      __syncthreads();
      if (lane == 0) {
        ro_int[cur] = v;
        ro_left[cur] = -1;
        rs_active[ci] = 0;
        rs_gain[ci] = -INFINITY;
      }
      __syncthreads();
      continue;
    }
    const int32_t left_id = node_count, right_id = node_count + 1;
    node_count += 2;
    ++n_splits;
    const bool left_small = N.count(l) <= N.count(l + 1);
    // The first two free slots other than ci, in slot order.
    int32_t slot_small = -1, slot_large = -1;
    for (int32_t base = 0; base < C && slot_large < 0; base += 64) {
      const int32_t i = base + lane;
      unsigned long long m = __ballot(i < C && i != ci && !rs_active[i]);
      while (m && slot_large < 0) {
        const int32_t k = base + __builtin_ctzll(m);
        m &= m - 1;
        if (slot_small < 0) slot_small = k;
        else slot_large = k;
      }
    }
    if (slot_large < 0) {
      *status = 3;
      return 0;
    }
    __syncthreads();
    if (lane == 0) {
      ro_int[cur] = v;
      ro_left[cur] = left_id;
      rs_active[ci] = 0;
      rs_gain[ci] = -INFINITY;
      replay_set_slot(N, slot_small, left_small ? left_id : right_id, left_small ? l : l + 1);
      replay_set_slot(N, slot_large, left_small ? right_id : left_id, left_small ? l + 1 : l);
    }
    __syncthreads();
  }
  // Candidates left in the slots are leaves.
  for (int32_t i = lane; i < C; i += 64)
    if (rs_active[i]) {
      ro_int[rs_node[i]] = rs_int[i];
      ro_left[rs_node[i]] = -1;
    }
  return node_count;
}

template <bool kStaged>
__device__ void replay_write(const ReplayNodes<kStaged> &N, const int32_t *__restrict__ feats,
                             int32_t node_count, int32_t M, TreeArrays out,
                             TreeNodeDev *__restrict__ tree, const int32_t *o_int = ro_int,
                             const int32_t *o_left = ro_left, int32_t stride = 64) {
  for (int32_t i = (int32_t)threadIdx.x; i < M; i += stride) {
    int32_t f = -1, lc = -1, rc = -1;
    int64_t th = 0;
    double val = 0.0, g = 0.0;
    if (i < node_count) {
      const int32_t v = o_int[i];
      val = N.val(v);
      if (o_left[i] >= 0) {
        f = feats[N.fpos(v)];
        th = N.bin(v);
        lc = o_left[i];
        rc = lc + 1;
        g = N.gain(v);
      }
      TreeNodeDev d;
      d.feature = f;
      d.threshold = f >= 0 ? (int32_t)th : 0;
      d.left = f >= 0 ? lc : 0;
      d.right = f >= 0 ? rc : 0;
      d.value = val;
      tree[i] = d;
    }
    out.features[i] = f;
    out.thresholds[i] = th;
    out.values[i] = val;
    out.left[i] = lc;
    out.right[i] = rc;
    out.gains[i] = g;
  }
}

__global__ __launch_bounds__(64) void k_replay(
    const NodeOut *__restrict__ nodes, const LevelPlan *__restrict__ plan,
    const int32_t *__restrict__ feats, ReplayArgs a, TreeArrays out,
    TreeNodeDev *__restrict__ tree, RoundHeader *__restrict__ hdr) {
  const int lane = (int)threadIdx.x;
  if (a.dev.max) dev_scales(a.dev, a.g_scale, a.h_scale);
  const int32_t M = a.out_len;
  const int32_t C = a.max_leaves + 2;
  int32_t status = 0, needed = 0;
  const LevelPlan pl = *plan;
  if (pl.overflow > 0) {
    status = 1;
    needed = pl.overflow;
  } else if (pl.overflow < 0) {
    status = 5;
  } else if (C > kReplaySlots || M > kReplayOut) {
    status = 4;
  }
  int32_t node_count = 0;
  if (status == 0) {
    const int32_t n_nodes = pl.n_nodes;
    if (n_nodes <= min(kReplayNodes, a.stage_limit)) {
      for (int32_t i = lane; i < n_nodes; i += 64) {
        const NodeOut nd = nodes[i];
        rp_gain[i] = nd.gain;
        rp_val[i] = leaf_value(nd, a);
        rp_count[i] = (int32_t)nd.count;
        rp_fpos[i] = nd.fpos;
        rp_bin[i] = (uint8_t)nd.bin;
        rp_left[i] = nd.left;
        rp_valid[i] = (uint8_t)nd.valid;
      }
      __syncthreads();
      const ReplayNodes<true> N{nodes, a};
      node_count = replay_loop(N, C, &status);
      __syncthreads();
      replay_write(N, feats, status == 0 ? node_count : 0, M, out, tree);
    } else {
      const ReplayNodes<false> N{nodes, a};
      node_count = replay_loop(N, C, &status);
      __syncthreads();
      replay_write(N, feats, status == 0 ? node_count : 0, M, out, tree);
    }
  }
  if (lane == 0) {
    hdr->node_count = status == 0 ? node_count : 0;
    hdr->status = status;
    hdr->needed = needed;
    hdr->expanded = -1;
    hdr->hist_rows = 0;
  }
}

// Trees of up to kRegSlots candidate slots and kReplayNodes nodes: one
// workgroup.  Best-first search with distinct keys pops nodes in a fixed
// order.  Let a candidate be a node whose ancestors are all kept splits with
// key > gamma and whose own key G (best gain, -inf without a split) is
// > gamma; give each candidate the vector whose component d is the smallest
// key on its path below depth d (+inf past its depth).  For two candidates,
// the node on the other's path comes first (its vector is larger at the
// ancestor's depth); otherwise the paths below their deepest common
// ancestor hold distinct keys, the one whose smallest such key is larger is
// popped first (every node of the other path that is popped first had the
// largest key of the frontier while an unpopped node of this path waited
// there with a larger one -- impossible), and the vectors first differ
// exactly there.  So the kernel ranks the candidates by their vectors (keys
// replaced by their ranks, 11 bits per depth), and the loop's stop rules
// become a cut of that order: after max_leaves - 1 kept splits; every
// candidate before it is popped (a candidate whose level loop did not expand
// it is the replay's failure, status 2).  Output ids follow from the number
// of kept splits before each one.  Candidates with equal keys (the slot
// order breaks those ties) or deeper trees run the slot loop below in
// wave 0.
constexpr int kRegSlotsPerLane = 2;
constexpr int kRegSlots = 64 * kRegSlotsPerLane;
constexpr int kTreeBlock = 1024;
constexpr int kTreeMaxDepth = 10;  // components of a node's vector (11 bits each)
constexpr uint32_t kCodeInf = 2047;
constexpr int32_t kKept = 1 << 30, kLeftSmall = 1 << 29, kChildMask = (1 << 29) - 1;

__shared__ int32_t rq_child[kReplayNodes];  // first child | kept | left smaller, or -1
__shared__ double rt_G[kReplayNodes];
__shared__ int16_t rt_parent[kReplayNodes], rt_code[kReplayNodes], rt_at[kReplayNodes];
__shared__ int16_t rt_kk[kReplayNodes];  // kept splits popped before a popped kept split, else -1
__shared__ uint8_t rt_pc[kReplayNodes], rt_depth[kReplayNodes];
// Staging of the child facts, then the candidates' keys, then their vectors.
__shared__ __align__(16) unsigned long long rt_raw[2 * kReplayNodes];
__shared__ int32_t rt_int[2 * kRegSlots + 2], rt_left[2 * kRegSlots + 2];
__shared__ int32_t rt_flags[4];  // [0] slot loop needed, [1] candidates, [2] status, [3] nodes

// The slot loop (one wave): candidate slot k in lane k % 64, register
// k / 64; a pop is a DPP maximum, a ballot and two lane reads.
__device__ int32_t replay_slot_loop(int32_t C, const ReplayArgs &a, int32_t &status) {
  const int lane = lane_id();
  double g[kRegSlotsPerLane];
  int32_t sid[kRegSlotsPerLane], sint[kRegSlotsPerLane];
  bool act[kRegSlotsPerLane];
#pragma unroll
  for (int q = 0; q < kRegSlotsPerLane; ++q) {
    g[q] = -INFINITY;
    sid[q] = 0;
    sint[q] = 0;
    act[q] = false;
  }
  int32_t node_count = 1;
  if (lane == 0) {
    rt_int[0] = 0;
    rt_left[0] = -1;
  }
  if (rp_fpos[0] < 0) return node_count;
  if (lane == 0) {
    g[0] = rp_gain[0];
    act[0] = true;
  }
  int32_t n_splits = 0;
  while (n_splits < a.max_leaves - 1) {
    double lmax = g[0];
#pragma unroll
    for (int q = 1; q < kRegSlotsPerLane; ++q) lmax = fmax(lmax, g[q]);
    const double best = wave_max_f64(lmax);
    if (!(best > a.gamma)) break;
    int32_t ci = -1;
#pragma unroll
    for (int q = 0; q < kRegSlotsPerLane; ++q) {
      const unsigned long long m = __ballot(g[q] == best);
      if (ci < 0 && m) ci = 64 * q + __builtin_ctzll(m);
    }
    const int cq = ci >> 6, cl = ci & 63;
    int32_t v = 0, cur = 0;
#pragma unroll
    for (int q = 0; q < kRegSlotsPerLane; ++q)
      if (q == cq) {
        v = __builtin_amdgcn_readlane(sint[q], cl);
        cur = __builtin_amdgcn_readlane(sid[q], cl);
      }
    const int32_t c = rq_child[v];
    if (c < 0) {
      status = 2;
      break;
    }
    // The popped slot is free again.
#pragma unroll
    for (int q = 0; q < kRegSlotsPerLane; ++q)
      if (q == cq && lane == cl) {
        act[q] = false;
        g[q] = -INFINITY;
      }
    if (!(c & kKept)) {  // est:678-683: the node stays a leaf
      if (lane == 0) {
        rt_int[cur] = v;
        rt_left[cur] = -1;
      }
      continue;
    }
    const int32_t l = c & kChildMask;
    const bool left_small = (c & kLeftSmall) != 0;
    const int32_t left_id = node_count, right_id = node_count + 1;
    node_count += 2;
    ++n_splits;
    // The first two free slots other than ci, in slot order.
    int32_t slot_small = -1, slot_large = -1;
#pragma unroll
    for (int q = 0; q < kRegSlotsPerLane; ++q) {
      const int32_t k = 64 * q + lane;
      unsigned long long m = __ballot(k < C && k != ci && !act[q]);
      while (m && slot_large < 0) {
        const int32_t kk = 64 * q + __builtin_ctzll(m);
        m &= m - 1;
        if (slot_small < 0) slot_small = kk;
        else slot_large = kk;
      }
    }
    if (slot_large < 0) {
      status = 3;
      break;
    }
    const double gl = rt_G[l], gr = rt_G[l + 1];
#pragma unroll
    for (int q = 0; q < kRegSlotsPerLane; ++q) {
      const int32_t k = 64 * q + lane;
      if (k == slot_small || k == slot_large) {
        const bool is_left = (k == slot_small) == left_small;
        act[q] = true;
        sid[q] = is_left ? left_id : right_id;
        sint[q] = is_left ? l : l + 1;
        g[q] = is_left ? gl : gr;
      }
    }
    if (lane == 0) {
      rt_int[cur] = v;
      rt_left[cur] = left_id;
    }
  }
  if (status == 0) {
#pragma unroll
    for (int q = 0; q < kRegSlotsPerLane; ++q)
      if (act[q]) {
        rt_int[sid[q]] = sint[q];
        rt_left[sid[q]] = -1;
      }
  }
  return node_count;
}

__global__ __launch_bounds__(kTreeBlock) void k_replay_tree(
    const NodeOut *__restrict__ nodes, const LevelPlan *__restrict__ plan,
    const int32_t *__restrict__ feats, ReplayArgs a, TreeArrays out,
    TreeNodeDev *__restrict__ tree, RoundHeader *__restrict__ hdr) {
  __shared__ uint32_t stmp[kTreeBlock / 64];
  __shared__ long long s_hist_rows[kTreeBlock / 64];
  __shared__ int32_t s_expanded[kTreeBlock / 64];
  static_assert(kReplayNodes <= kTreeBlock, "one node per thread");
  const int tid = (int)threadIdx.x, wave = tid >> 6;
  if (a.dev.max) dev_scales(a.dev, a.g_scale, a.h_scale);
  const int32_t M = a.out_len;
  const int32_t C = a.max_leaves + 2;
  int32_t status = 0, needed = 0;
  const LevelPlan pl = *plan;
  const int32_t n = pl.n_nodes;
  if (pl.overflow > 0) {
    status = 1;
    needed = pl.overflow;
  } else if (pl.overflow < 0) {
    status = 5;
  } else if (C > kRegSlots || M > 2 * kRegSlots + 2 || n > kReplayNodes || n < 1) {
    status = 4;
  }
  int32_t node_count = 0;
  if (status == 0) {  // (uniform)
    int32_t *cnt = reinterpret_cast<int32_t *>(rt_raw);
    int32_t *lft = cnt + kReplayNodes;
    uint8_t *vld = reinterpret_cast<uint8_t *>(lft + kReplayNodes);
    for (int32_t i = tid; i < n; i += kTreeBlock) {
      const NodeOut nd = nodes[i];
      rp_gain[i] = nd.gain;
      rp_val[i] = leaf_value(nd, a);
      rp_fpos[i] = nd.fpos;
      rp_bin[i] = (uint8_t)nd.bin;
      rt_G[i] = nd.fpos >= 0 ? nd.gain : -INFINITY;
      cnt[i] = (int32_t)nd.count;
      lft[i] = nd.left;
      vld[i] = (uint8_t)nd.valid;
      rt_parent[i] = -1;
      rt_kk[i] = -1;
    }
    if (tid < 4) rt_flags[tid] = 0;
    __syncthreads();
    // Profiling counts (one node per thread): the smaller child's rows of a
    // kept split, added below when the children are above max_depth.
    long long small_rows = -1;
    int32_t expanded = 0;
    for (int32_t v = tid; v < n; v += kTreeBlock) {
      const int32_t l = lft[v];
      int32_t c = -1;
      if (l >= 0) {
        expanded = 1;
        if (vld[l]) small_rows = min(cnt[l], cnt[l + 1]);
        c = l | (vld[l] ? kKept : 0) | (cnt[l] <= cnt[l + 1] ? kLeftSmall : 0);
        rt_parent[l] = (int16_t)v;
        rt_parent[l + 1] = (int16_t)v;
      }
      rq_child[v] = c;
    }
    __syncthreads();
    // Candidates and depths (each node walks to the root).
    double *gc = reinterpret_cast<double *>(rt_raw);  // key of a candidate, NaN otherwise
    for (int32_t v = tid; v < n; v += kTreeBlock) {
      bool pc = rt_G[v] > a.gamma;
      int32_t d = 0, u = v;
      while (u != 0 && d <= kTreeMaxDepth) {
        const int32_t p = rt_parent[u];
        if (p < 0) {
          pc = false;
          break;
        }
        pc = pc && (rq_child[p] & kKept) && rt_G[p] > a.gamma;
        u = p;
        ++d;
      }
      if (d > kTreeMaxDepth) rt_flags[0] = 1;
      rt_pc[v] = pc ? 1 : 0;
      rt_depth[v] = (uint8_t)min(d, 255);
      gc[v] = pc ? rt_G[v] : __longlong_as_double(0x7ff8000000000000ll);
      // The full depth for the counts (parents have lower ids: the walk ends).
      int32_t depth = d;
      while (depth > kTreeMaxDepth && u != 0 && rt_parent[u] >= 0) {
        u = rt_parent[u];
        ++depth;
      }
      if (depth + 1 >= a.max_depth) small_rows = -1;
    }
    {
      const long long hr = wave_sum(small_rows > 0 ? small_rows : 0ll);
      const int32_t ex = wave_sum(expanded);
      if ((tid & 63) == 0) {
        s_hist_rows[wave] = hr;
        s_expanded[wave] = ex;
      }
    }
    __syncthreads();
    // Key ranks among the candidates; equal keys need the slot loop.
    for (int32_t v = tid; v < n; v += kTreeBlock) {
      if (!rt_pc[v]) continue;
      const double gv = gc[v];
      int32_t lt = 0, eq = 0;
      int32_t u = 0;
      // Eight keys per step in four 16-byte LDS reads, all in flight at once.
      const double2 *gc2 = reinterpret_cast<const double2 *>(gc);
      for (; u + 8 <= n; u += 8) {
        double2 q[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) q[j] = gc2[(u >> 1) + j];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          lt += (q[j].x < gv) + (q[j].y < gv);
          eq += (q[j].x == gv) + (q[j].y == gv);
        }
      }
      for (; u < n; ++u) {
        lt += gc[u] < gv;
        eq += gc[u] == gv;
      }
      rt_code[v] = (int16_t)lt;
      if (eq > 1) rt_flags[0] = 1;
      atomicAdd(&rt_flags[1], 1);
    }
    __syncthreads();
    const bool slots = rt_flags[0] != 0;
    if (!slots) {
      // Vectors: component d (depth d + 1 and below) in 11 bits, d = 0 in
      // the top bits of hi; 0 for nodes that are not candidates.
      unsigned long long *key = rt_raw;
      for (int32_t v = tid; v < n; v += kTreeBlock) {
        unsigned long long hi = 0, lo = 0;
        if (rt_pc[v]) {
          uint32_t comp[kTreeMaxDepth];
#pragma unroll
          for (int d = 0; d < kTreeMaxDepth; ++d) comp[d] = kCodeInf;
          uint32_t mn = kCodeInf;
          int32_t u = v;
          for (int d = (int)rt_depth[v] - 1; d >= 0; --d) {
            mn = min(mn, (uint32_t)rt_code[u]);
#pragma unroll
            for (int q = 0; q < kTreeMaxDepth; ++q)
              if (q == d) comp[q] = mn;
            u = rt_parent[u];
          }
#pragma unroll
          for (int d = 0; d < 5; ++d) {
            hi |= (unsigned long long)comp[d] << (44 - 11 * d);
            lo |= (unsigned long long)comp[d + 5] << (44 - 11 * d);
          }
        }
        key[2 * v] = hi;
        key[2 * v + 1] = lo;
      }
      __syncthreads();
      for (int32_t v = tid; v < n; v += kTreeBlock) {
        if (!rt_pc[v]) continue;
        const unsigned long long kh = key[2 * v], kl = key[2 * v + 1];
        int32_t r = 0;
        int32_t u = 0;
        // Eight (hi, lo) vectors per step, one 16-byte LDS read each, all in
        // flight at once.
        const ulonglong2 *key2 = reinterpret_cast<const ulonglong2 *>(key);
        for (; u + 8 <= n; u += 8) {
          ulonglong2 q[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) q[j] = key2[u + j];
#pragma unroll
          for (int j = 0; j < 8; ++j) r += (q[j].x > kh || (q[j].x == kh && q[j].y > kl)) ? 1 : 0;
        }
        for (; u < n; ++u) {
          const unsigned long long uh = key[2 * u], ul = key[2 * u + 1];
          r += (uh > kh || (uh == kh && ul > kl)) ? 1 : 0;
        }
        rt_at[r] = (int16_t)v;
      }
      __syncthreads();
      // The cut: a candidate is popped while fewer than max_leaves - 1
      // kept splits came before it.
      const int32_t npc = rt_flags[1];
      int32_t v = -1, c = -1;
      if (tid < npc) {
        v = rt_at[tid];
        c = rq_child[v];
      }
      const uint32_t ks = (v >= 0 && c >= 0 && (c & kKept)) ? 1u : 0u;
      uint32_t ktot;
      const uint32_t kb = block_excl_scan<kTreeBlock>(ks, stmp, ktot);
      const bool popped = v >= 0 && (int32_t)kb < a.max_leaves - 1;
      if (popped && c < 0) rt_flags[2] = 2;
      if (popped && ks) rt_kk[v] = (int16_t)kb;
      __syncthreads();
      const int32_t K = min((int32_t)ktot, a.max_leaves - 1);
      node_count = 1 + 2 * K;
      if (rt_flags[2] == 0) {
        if (tid == 0) {
          rt_int[0] = 0;
          rt_left[0] = rt_kk[0] >= 0 ? 1 + 2 * rt_kk[0] : -1;
        }
        for (int32_t u = tid; u < n; u += kTreeBlock) {
          const int32_t k = rt_kk[u];
          if (k < 0) continue;
          const int32_t l = rq_child[u] & kChildMask, lid = 1 + 2 * k;
          rt_int[lid] = l;
          rt_left[lid] = rt_kk[l] >= 0 ? 1 + 2 * rt_kk[l] : -1;
          rt_int[lid + 1] = l + 1;
          rt_left[lid + 1] = rt_kk[l + 1] >= 0 ? 1 + 2 * rt_kk[l + 1] : -1;
        }
      }
      status = rt_flags[2];
    } else {
      if (wave == 0) {
        int32_t st = 0;
        const int32_t nc = replay_slot_loop(C, a, st);
        if (lane_id() == 0) {
          rt_flags[2] = st;
          rt_flags[3] = nc;
        }
      }
      __syncthreads();
      status = rt_flags[2];
      node_count = rt_flags[3];
    }
    __syncthreads();
    const ReplayNodes<true> N{nodes, a};
    replay_write(N, feats, status == 0 ? node_count : 0, M, out, tree, rt_int, rt_left,
                 kTreeBlock);
  }
  if (tid == 0) {
    hdr->node_count = status == 0 ? node_count : 0;
    hdr->status = status;
    hdr->needed = needed;
    long long hr = 0;
    int32_t ex = 0;
    if (status == 0) {
      for (int w = 0; w < kTreeBlock / 64; ++w) {
        hr += s_hist_rows[w];
        ex += s_expanded[w];
      }
    }
    hdr->expanded = status == 0 ? ex : -1;
    hdr->hist_rows = hr;
  }
}

bool replay_counts_nodes(const ReplayArgs &a) {
  return a.max_leaves + 2 <= kRegSlots && a.stage_limit >= kReplayNodes &&
         a.node_cap <= kReplayNodes;
}

hipError_t launch_replay(hipStream_t st, const NodeOut *nodes, const LevelPlan *plan,
                         const int32_t *feats, ReplayArgs a, TreeArrays out,
                         TreeNodeDev *tree, RoundHeader *hdr) {
  // Up to 128 candidate slots when every node fits in LDS: the order form.
  if (replay_counts_nodes(a))
    hipLaunchKernelGGL(k_replay_tree, dim3(1), dim3(kTreeBlock), 0, st, nodes, plan, feats, a,
                       out, tree, hdr);
  else
    hipLaunchKernelGGL(k_replay, dim3(1), dim3(64), 0, st, nodes, plan, feats, a, out, tree, hdr);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Prediction (est:843-861 one tree; est:863-884 ensemble).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_predict_tree(
    const uint8_t *__restrict__ codes, int64_t ld, int64_t n,
    const TreeNodeDev *__restrict__ tree, double *__restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = tree[traverse(tree, codes, ld, i)].value;
}

hipError_t launch_predict_tree(hipStream_t st, const uint8_t *codes,
                               int64_t ld, int64_t n, const TreeNodeDev *tree,
                               int32_t node_count, double *out) {
  (void)node_count;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_predict_tree, dim3((unsigned)((n + 255) / 256)), dim3(256),
                     0, st, codes, ld, n, tree, out);
  return hipGetLastError();
}

#pragma clang fp contract(off)
__global__ __launch_bounds__(256) void k_predict(
    const uint8_t *__restrict__ codes, int64_t ld, int64_t n,
    const TreeNodeDev *__restrict__ nodes, const int32_t *__restrict__ offsets,
    int32_t n_trees, double lr, double *__restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  double F = 0.0;
  for (int32_t t = 0; t < n_trees; ++t) {
    const TreeNodeDev *tree = nodes + offsets[t];
    F = __dadd_rn(F, __dmul_rn(lr, tree[traverse(tree, codes, ld, i)].value));
  }
  out[i] = F;
}
#pragma clang fp contract(on)

// predict_proba of a binary model (est:3318-3324, 3335-3336): F + base_score,
// p = 1 / (1 + exp(-clip(F, -500, 500))) and the columns (1 - p, p), each
// operation rounded separately as NumPy's are (clip keeps a NaN).
#pragma clang fp contract(off)
__global__ __launch_bounds__(256) void k_binary_proba(const double *__restrict__ F, int64_t n,
                                                      double base, double2 *__restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const double f = __dadd_rn(F[i], base);
  const double fc = isnan(f) ? f : fmin(fmax(f, -500.0), 500.0);
  const double p = __ddiv_rn(1.0, __dadd_rn(1.0, exp(-fc)));
  out[i] = make_double2(__dsub_rn(1.0, p), p);
}
#pragma clang fp contract(on)

hipError_t launch_binary_proba(hipStream_t st, const double *F, int64_t n, double base,
                               double *out) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_binary_proba, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, F, n,
                     base, reinterpret_cast<double2 *>(out));
  return hipGetLastError();
}

// Packed trees of _pack_tree_list (est:2192-2216) -> traversal nodes: the
// host has checked every feature and child index.
__global__ __launch_bounds__(256) void k_pack_trees(
    const int16_t *__restrict__ features, const int64_t *__restrict__ thresholds,
    const double *__restrict__ values, const int32_t *__restrict__ left,
    const int32_t *__restrict__ right, int32_t total, int32_t F, int32_t tiers,
    TreeNodeDev *__restrict__ nodes) {
  const int32_t i = (int32_t)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= total) return;
  TreeNodeDev d;
  d.value = values[i];
  d.feature = features[i];
  if (d.feature >= 0) {
    const int64_t t = thresholds[i];
    d.threshold = (int32_t)(t < -1 ? -1 : (t > (1 << 20) ? (1 << 20) : t));
    if (tiers > 1 && d.threshold >= 255) {
      // "code <= 255 k + b" is "tier k <= b" (kernels.h); a threshold above
      // the last tier's range sends every row left, as b = 255 does.
      const int32_t k = min(d.threshold / 255, tiers - 1);
      d.feature += k * F;
      d.threshold = min(d.threshold - 255 * k, 255);
    }
    d.left = left[i];
    d.right = right[i];
  } else {
    d.feature = -1;
    d.threshold = 0;
    d.left = 0;
    d.right = 0;
  }
  nodes[i] = d;
}

hipError_t launch_pack_trees(hipStream_t st, const int16_t *features, const int64_t *thresholds,
                             const double *values, const int32_t *left, const int32_t *right,
                             int32_t total, int32_t F, int32_t tiers, TreeNodeDev *nodes) {
  if (total <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_pack_trees, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st,
                     features, thresholds, values, left, right, total, F, tiers, nodes);
  return hipGetLastError();
}

// Ensemble prediction with the rows' codes and the trees staged in LDS.
// A block takes kPredRows rows (two per thread, two independent walks in
// flight): it loads their codes of every column once (16-byte loads, all
// independent), then walks the trees a chunk at a time.  A chunk is a run of
// whole trees of at most kPredChunk nodes (the host's list, predict_chunks),
// copied into LDS as one 32-bit word per node plus the values.  Per row the
// trees are added in order from 0.0, lr * value and the add rounded
// separately, so the result is bit-identical to k_predict's.
//
// Node word: bits 0-8 threshold + 1 (go left when code < it; thresholds
// clamped to [-1, 255]), bits 9-15 column (127 for a leaf), bits 16-31 the
// left child's index in the chunk; the right child is the next node, as the
// builder numbers them (est:686-687; the host checks every tree).
constexpr int kPredRows = 512;
constexpr int kPredChunk = 1024;
constexpr int kPredMaxCols = 64;   // staged columns (7 bits, 127 marks a leaf)
constexpr uint32_t kPredLeaf = 127u;

int32_t predict_chunk_nodes() { return kPredChunk; }

bool predict_staged_ok(int32_t n_cols, int32_t max_tree_nodes, bool right_follows_left) {
  return right_follows_left && n_cols > 0 && n_cols <= kPredMaxCols &&
         max_tree_nodes <= kPredChunk;
}

int32_t predict_chunks(const int32_t *offsets, int32_t n_trees, int32_t *chunks) {
  int32_t nc = 0;
  int32_t t0 = 0;
  while (t0 < n_trees) {
    int32_t t1 = t0 + 1;
    while (t1 < n_trees && offsets[t1 + 1] - offsets[t0] <= kPredChunk) ++t1;
    chunks[nc++] = t0;
    t0 = t1;
  }
  chunks[nc] = n_trees;
  return nc;
}

#pragma clang fp contract(off)
__global__ __launch_bounds__(256) void k_predict_staged(
    const uint8_t *__restrict__ codes, int64_t ld, int64_t n, int32_t n_cols,
    const TreeNodeDev *__restrict__ nodes, const int32_t *__restrict__ offsets,
    const int32_t *__restrict__ chunks, int32_t n_chunks, double lr, double *__restrict__ out) {
  extern __shared__ uint4 sc4[];  // codes [n_cols][kPredRows]
  __shared__ uint32_t wn[kPredChunk];
  __shared__ double wv[kPredChunk];
  __shared__ int32_t wt[kPredChunk];  // each staged tree's first node
  const int tid = (int)threadIdx.x;
  const int64_t row0 = (int64_t)blockIdx.x * kPredRows;
  constexpr int kChunksPerCol = kPredRows / 16;
  // Chunks past ld (the last column's padding) are never read: rows there
  // are >= n.
  for (int k = tid; k < n_cols * kChunksPerCol; k += 256) {
    const int c = k / kChunksPerCol, ch = k % kChunksPerCol;
    const int64_t r = row0 + 16 * ch;
    if (r < ld) sc4[k] = *reinterpret_cast<const uint4 *>(codes + (int64_t)c * ld + r);
  }
  const uint8_t *sc0 = reinterpret_cast<const uint8_t *>(sc4) + tid;
  const uint8_t *sc1 = sc0 + 256;
  const bool in0 = row0 + tid < n, in1 = row0 + tid + 256 < n;
  double F0 = 0.0, F1 = 0.0;
  // Chunk c + 1's nodes and tree starts are loaded into registers while
  // chunk c is walked (kPredChunk / 256 nodes and tree starts per thread).
  constexpr int kPer = kPredChunk / 256;
  TreeNodeDev pn[kPer];
  int32_t pt[kPer];
  int32_t t0 = 0, t1 = 0, base = 0, cnt = 0;
  auto prefetch = [&](int32_t c) {
    t0 = chunks[c];
    t1 = chunks[c + 1];
    base = offsets[t0];
    cnt = offsets[t1] - base;
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const int k = tid + 256 * q;
      if (k < cnt) pn[q] = nodes[base + k];
      if (k < t1 - t0) pt[q] = offsets[t0 + k] - base;
    }
  };
  if (n_chunks > 0) prefetch(0);
  for (int32_t c = 0; c < n_chunks; ++c) {
    const int32_t nt = t1 - t0, nn = cnt;
    __syncthreads();  // the previous chunk's walks are done
#pragma unroll
    for (int q = 0; q < kPer; ++q)
      if (tid + 256 * q < nt) wt[tid + 256 * q] = pt[q];
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const int k = tid + 256 * q;
      if (k >= nn) continue;
      const TreeNodeDev d = pn[q];
      // The node's tree starts at the last wt <= k (binary search).
      int lo = 0, hi = nt - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (wt[mid] <= k) lo = mid;
        else hi = mid - 1;
      }
      const uint32_t col = d.feature >= 0 ? (uint32_t)d.feature : kPredLeaf;
      const uint32_t thr1 = (uint32_t)(min(max(d.threshold, -1), 255) + 1);
      const uint32_t left = d.feature >= 0 ? (uint32_t)(wt[lo] + d.left) : 0u;
      wn[k] = thr1 | (col << 9) | (left << 16);
      wv[k] = d.value;
    }
    __syncthreads();
    if (c + 1 < n_chunks) prefetch(c + 1);
    for (int32_t t = 0; t < nt; ++t) {
      int32_t n0 = wt[t], n1 = n0;
      uint32_t w0 = wn[n0], w1 = w0;
      bool a0 = in0 && ((w0 >> 9) & 127u) != kPredLeaf;
      bool a1 = in1 && ((w1 >> 9) & 127u) != kPredLeaf;
      while (a0 || a1) {
        if (a0) {
          const uint32_t code = sc0[((w0 >> 9) & 127u) * kPredRows];
          n0 = (int32_t)(w0 >> 16) + (code < (w0 & 511u) ? 0 : 1);
          w0 = wn[n0];
          a0 = ((w0 >> 9) & 127u) != kPredLeaf;
        }
        if (a1) {
          const uint32_t code = sc1[((w1 >> 9) & 127u) * kPredRows];
          n1 = (int32_t)(w1 >> 16) + (code < (w1 & 511u) ? 0 : 1);
          w1 = wn[n1];
          a1 = ((w1 >> 9) & 127u) != kPredLeaf;
        }
      }
      F0 = __dadd_rn(F0, __dmul_rn(lr, wv[n0]));
      F1 = __dadd_rn(F1, __dmul_rn(lr, wv[n1]));
    }
  }
  if (in0) out[row0 + tid] = F0;
  if (in1) out[row0 + tid + 256] = F1;
}
#pragma clang fp contract(on)

hipError_t launch_predict(hipStream_t st, const uint8_t *codes, int64_t ld,
                          int64_t n, int32_t n_cols, const TreeNodeDev *nodes,
                          const int32_t *offsets, int32_t n_trees, const int32_t *chunks,
                          int32_t n_chunks, double lr, double *out, hipEvent_t ev_start,
                          hipEvent_t ev_stop) {
  if (n <= 0) return hipSuccess;
  if (chunks) {
    const size_t lds = (size_t)n_cols * kPredRows;
    hipExtLaunchKernelGGL(k_predict_staged, dim3((unsigned)((n + kPredRows - 1) / kPredRows)),
                          dim3(256), lds, st, ev_start, ev_stop, 0, codes, ld, n, n_cols, nodes,
                          offsets, chunks, n_chunks, lr, out);
  } else {
    hipExtLaunchKernelGGL(k_predict, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                          ev_start, ev_stop, 0, codes, ld, n, nodes, offsets, n_trees, lr, out);
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Multiclass rounds (est:2949-3065).  Scores F are [K][n] float64, class k's
// gradients G[k][i] and hessians H[k][i] likewise.  A row's softmax follows
// the reference's NumPy order: F - max over the classes, exp, the sum over
// the classes in the order NumPy's sum(axis=1) adds a contiguous row (below),
// then one division per class.
// ---------------------------------------------------------------------------
#pragma clang fp contract(off)
namespace {

// Sum of e[0..K-1] in the order of NumPy's pairwise summation of a
// contiguous run of K <= 16 doubles: below 8 terms one running sum in index
// order; from 8 on, eight partial sums r[j] = e[j] (+ e[j + 8] when a second
// whole block of eight exists, K = 16), combined as
// ((r0 + r1) + (r2 + r3)) + ((r4 + r5) + (r6 + r7)), then the terms left
// after the whole blocks added one by one in index order.
__device__ __forceinline__ double numpy_row_sum(const double (&e)[kMcMaxK], int K) {
  static_assert(kMcMaxK == 16, "the block structure below covers at most two blocks of eight");
  if (K < 8) {
    double s = e[0];
#pragma unroll
    for (int k = 1; k < 8; ++k)
      if (k < K) s = __dadd_rn(s, e[k]);
    return s;
  }
  double r[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = K == 16 ? __dadd_rn(e[j], e[j + 8]) : e[j];
  double s = __dadd_rn(__dadd_rn(__dadd_rn(r[0], r[1]), __dadd_rn(r[2], r[3])),
                       __dadd_rn(__dadd_rn(r[4], r[5]), __dadd_rn(r[6], r[7])));
  if (K < 16) {
#pragma unroll
    for (int k = 8; k < 16; ++k)
      if (k < K) s = __dadd_rn(s, e[k]);
  }
  return s;
}

// Order-preserving bits of a non-negative double.
__device__ __forceinline__ unsigned long long nonneg_bits(double v) {
  return (unsigned long long)__double_as_longlong(v);
}

__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const unsigned long long t = __shfl_xor(v, o, 64);
    v = t > v ? t : v;
  }
  return v;
}

}  // namespace

// grad_all = w * (p - onehot), hess_all = w * p * (1 - p) floored at 1e-8
// (softmax est:2327-2332 called at est:2996, gradients est:3013-3014, floor
// est:3019); mx[2k], mx[2k + 1] collect the largest |g| and h of class
// k over the rows (the fixed-point scale of its tree).
__global__ __launch_bounds__(256) void k_mc_grad_hess(
    const double *__restrict__ F, const int32_t *__restrict__ y, const double *__restrict__ w,
    int64_t n, int32_t K, double *__restrict__ G, double *__restrict__ H,
    unsigned long long *__restrict__ mx) {
  __shared__ unsigned long long red[2 * kMcMaxK][256 / 64];
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const bool in = i < n;
  double e[kMcMaxK];
  double fmaxv = -INFINITY;
#pragma unroll
  for (int k = 0; k < kMcMaxK; ++k) {
    e[k] = (in && k < K) ? F[(int64_t)k * n + i] : 0.0;
    if (k < K) fmaxv = fmax(fmaxv, e[k]);
  }
#pragma unroll
  for (int k = 0; k < kMcMaxK; ++k)
    if (k < K) e[k] = exp(__dsub_rn(e[k], fmaxv));
  const double sum = numpy_row_sum(e, K);
  const double wi = in ? w[i] : 0.0;
  const int32_t yi = in ? y[i] : -1;
#pragma unroll
  for (int k = 0; k < kMcMaxK; ++k) {
    if (k >= K) continue;  // (uniform)
    const double p = __ddiv_rn(e[k], sum);
    const double g = __dmul_rn(wi, __dsub_rn(p, yi == k ? 1.0 : 0.0));
    const double h = fmax(__dmul_rn(__dmul_rn(wi, p), __dsub_rn(1.0, p)), 1e-8);
    if (in) {
      G[(int64_t)k * n + i] = g;
      H[(int64_t)k * n + i] = h;
    }
    const unsigned long long gm = wave_max_u64(in ? nonneg_bits(fabs(g)) : 0ull);
    const unsigned long long hm = wave_max_u64(in ? nonneg_bits(h) : 0ull);
    if ((threadIdx.x & 63) == 0) {
      red[2 * k][threadIdx.x >> 6] = gm;
      red[2 * k + 1][threadIdx.x >> 6] = hm;
    }
  }
  __syncthreads();
  if ((int)threadIdx.x < 2 * K) {
    unsigned long long m = 0ull;
#pragma unroll
    for (int q = 0; q < 256 / 64; ++q) m = red[threadIdx.x][q] > m ? red[threadIdx.x][q] : m;
    atomicMax(mx + threadIdx.x, m);
  }
}

// F[i] += lr * tree(x_i) for one class's scores (est:3029).
__global__ __launch_bounds__(256) void k_mc_apply(const uint8_t *__restrict__ codes, int64_t ld,
                                                  int64_t n, const TreeNodeDev *__restrict__ tree,
                                                  const int32_t *__restrict__ node_count_d,
                                                  double lr, double *__restrict__ Fk) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  // A device replay that failed left node_count at 0: F stays as it is.
  if (i >= n || (node_count_d && *node_count_d <= 0)) return;
  Fk[i] = __dadd_rn(Fk[i], __dmul_rn(lr, tree[traverse(tree, codes, ld, i)].value));
}

// Per block: the sum of log(clip(softmax(F_i))[y_i], 1e-15, 1 - 1e-15)
// over its rows (est:2335-2341, called at est:3035).
__global__ __launch_bounds__(256) void k_mc_loss(const double *__restrict__ F,
                                                 const int32_t *__restrict__ y, int64_t n,
                                                 int32_t K, double *__restrict__ partials) {
  __shared__ double red[256 / 64];
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  double v = 0.0;
  if (i < n) {
    double e[kMcMaxK];
    double fmaxv = -INFINITY;
#pragma unroll
    for (int k = 0; k < kMcMaxK; ++k) {
      e[k] = k < K ? F[(int64_t)k * n + i] : 0.0;
      if (k < K) fmaxv = fmax(fmaxv, e[k]);
    }
    double ey = 0.0;
    const int32_t yi = y[i];
#pragma unroll
    for (int k = 0; k < kMcMaxK; ++k) {
      if (k < K) {
        e[k] = exp(__dsub_rn(e[k], fmaxv));
        if (k == yi) ey = e[k];
      }
    }
    const double sum = numpy_row_sum(e, K);
    const double p = fmin(fmax(__ddiv_rn(ey, sum), 1e-15), 1.0 - 1e-15);
    v = log(p);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  if (threadIdx.x == 0) partials[blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
}

// predict_proba of a multiclass model (est:3315 with est:2327-2332): row
// i's softmax over its scores F[k][i] in the arithmetic of k_mc_grad_hess,
// written row by row, P[i][k].
__global__ __launch_bounds__(256) void k_mc_softmax(const double *__restrict__ F, int64_t n,
                                                    int32_t K, double *__restrict__ P) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  double e[kMcMaxK];
  double fmaxv = -INFINITY;
#pragma unroll
  for (int k = 0; k < kMcMaxK; ++k) {
    e[k] = k < K ? F[(int64_t)k * n + i] : 0.0;
    if (k < K) fmaxv = fmax(fmaxv, e[k]);
  }
#pragma unroll
  for (int k = 0; k < kMcMaxK; ++k)
    if (k < K) e[k] = exp(__dsub_rn(e[k], fmaxv));
  const double sum = numpy_row_sum(e, K);
#pragma unroll
  for (int k = 0; k < kMcMaxK; ++k)
    if (k < K) P[i * K + k] = __ddiv_rn(e[k], sum);
}
#pragma clang fp contract(on)

hipError_t launch_mc_grad_hess(hipStream_t st, const double *F, const int32_t *y, const double *w,
                               int64_t n, int32_t K, double *G, double *H,
                               unsigned long long *mx) {
  if (n <= 0) return hipSuccess;
  if (K < 2 || K > kMcMaxK) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_mc_grad_hess, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, F, y,
                     w, n, K, G, H, mx);
  return hipGetLastError();
}

hipError_t launch_mc_apply(hipStream_t st, const uint8_t *codes, int64_t ld, int64_t n,
                           const TreeNodeDev *tree, const int32_t *node_count_d, double lr,
                           double *Fk) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_mc_apply, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, codes, ld,
                     n, tree, node_count_d, lr, Fk);
  return hipGetLastError();
}

hipError_t launch_mc_softmax(hipStream_t st, const double *F, int64_t n, int32_t K, double *P) {
  if (n <= 0) return hipSuccess;
  if (K < 2 || K > kMcMaxK) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_mc_softmax, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, F, n, K,
                     P);
  return hipGetLastError();
}

int64_t mc_loss_blocks(int64_t n) { return (n + 255) / 256; }

hipError_t launch_mc_loss(hipStream_t st, const double *F, const int32_t *y, int64_t n,
                          int32_t K, double *partials) {
  if (n <= 0) return hipSuccess;
  if (K < 2 || K > kMcMaxK) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_mc_loss, dim3((unsigned)mc_loss_blocks(n)), dim3(256), 0, st, F, y, n, K,
                     partials);
  return hipGetLastError();
}

}  // namespace bsscl
