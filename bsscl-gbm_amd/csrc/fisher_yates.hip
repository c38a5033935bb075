// Fisher-Yates on the device: the swap half of the reference's bagging
// shuffle (src/bsscl_gbm/estimator_v1_0_1.py:2506), given the draws j(i)
// made on the host (sampler.cpp).
//
// Step i (i = n-1 .. 1, in that order) swaps positions i and j(i) <= i, and
// position i never changes after step i.  Let the steps that choose
// position p (j(k) = p, k > p) be s_1 < ... < s_L; they run s_L first.  Then
// position p holds a_old[p] until step s_L, and after step s_m it holds the
// value that step s_m brought from position s_m, v(s_m), where
//   v(k) = the value at position k just before step k
//        = v(s_1(k)) if any step chose k before, else a_old[k].
// So a_new[s_m] = v(s_{m+1}) for m < L, a_new[s_L] = a_old[p],
// a_new[i] = v(i) when j(i) = i, and a_new[0] = v(0).
//
// Each step k with j(k) != k pushes itself on position j(k)'s list (atomic
// exchange); each list is then sorted ascending (head = s_1, links
// s_m -> s_{m+1}, the last link holding -2 - p): lists of up to 8 steps in
// registers with a sorting network, longer ones by a linked-list merge sort
// (O(L log L) for any draws).  The chains k -> s_1(k) -> ... strictly
// increase and are short for random draws (about ln(n/k) links); any draws
// give the sequential result.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "kernels.h"

namespace bsscl {

namespace {

// These kernels run on the rows stream beside a tree, and most of their
// accesses are random 4-byte ones: they take at most one block per CU of the
// MI355X (grid-stride loops), so that fewer of their loads are in flight at
// once.  10M x 50: 372 -> 392 trees/s against 65536-block grids (128 blocks:
// 311, the tree then waits for the rows; 512: 387); 1M x 28: 2380 -> 2450.
constexpr int64_t kRowsStreamBlocks = 256;

unsigned blocks_for(int64_t n) {
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>((n + 255) / 256, kRowsStreamBlocks));
}

__global__ __launch_bounds__(256) void k_fy_push(const uint32_t *__restrict__ draws,
                                                 const uint32_t *const *draws_ref, int64_t n,
                                                 int32_t *__restrict__ head,
                                                 int32_t *__restrict__ next) {
  if (draws_ref) draws = *draws_ref;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < n - 1;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int32_t k = (int32_t)(n - 1 - t);
    const int32_t p = (int32_t)draws[t];
    if (p != k) next[k] = atomicExch(head + p, k);
  }
}

// a[0, n) = -1 with 16-byte stores (a is 16-byte aligned).
__global__ __launch_bounds__(256) void k_fill_neg(int32_t *__restrict__ a, int64_t n) {
  const int64_t n4 = n >> 2;
  int4 *a4 = reinterpret_cast<int4 *>(a);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4;
       i += (int64_t)gridDim.x * blockDim.x)
    a4[i] = make_int4(-1, -1, -1, -1);
  if (blockIdx.x == 0 && (int64_t)threadIdx.x < (n & 3)) a[(n4 << 2) + threadIdx.x] = -1;
}

// Ascending merge sort of the list starting at `h` (links in next[], -1
// ends it); O(L log L).
__device__ int32_t fy_merge_sort(int32_t h, int32_t *__restrict__ next) {
  int64_t L = 0;
  for (int32_t x = h; x >= 0; x = next[x]) ++L;
  for (int64_t width = 1; width < L; width *= 2) {
    int32_t cur = h, new_head = -1, tail = -1;
    while (cur >= 0) {
      int32_t a = cur, at = cur;
      for (int64_t k = 1; k < width && next[at] >= 0; ++k) at = next[at];
      int32_t b = next[at];
      next[at] = -1;
      int32_t rest = -1;
      if (b >= 0) {
        int32_t bt = b;
        for (int64_t k = 1; k < width && next[bt] >= 0; ++k) bt = next[bt];
        rest = next[bt];
        next[bt] = -1;
      }
      while (a >= 0 || b >= 0) {
        int32_t take;
        if (b < 0 || (a >= 0 && a < b)) {
          take = a;
          a = next[a];
        } else {
          take = b;
          b = next[b];
        }
        if (tail < 0) new_head = take;
        else next[tail] = take;
        tail = take;
      }
      next[tail] = -1;
      cur = rest;
    }
    h = new_head;
  }
  return h;
}

__device__ __forceinline__ void cswap(int32_t &a, int32_t &b) {
  const int32_t lo = min(a, b), hi = max(a, b);
  a = lo;
  b = hi;
}

// Batcher's odd-even merge sort network (K. Batcher, 1968) on registers:
// every index is a compile-time constant once the templates unroll.
template <int LO, int N, int R, int K>
__device__ __forceinline__ void oe_merge(int32_t (&e)[K]) {
  constexpr int STEP = R * 2;
  if constexpr (STEP < N) {
    oe_merge<LO, N, STEP>(e);
    oe_merge<LO + R, N, STEP>(e);
#pragma unroll
    for (int i = LO + R; i < LO + N - R; i += STEP) cswap(e[i], e[i + R]);
  } else {
    cswap(e[LO], e[LO + R]);
  }
}

template <int LO, int N, int K>
__device__ __forceinline__ void oe_sort(int32_t (&e)[K]) {
  if constexpr (N > 1) {
    oe_sort<LO, N / 2>(e);
    oe_sort<LO + N / 2, N / 2>(e);
    oe_merge<LO, N, 1>(e);
  }
}

// Lists of up to kFyRegs steps are sorted in registers (for random draws
// position p's list holds about ln(n/p) steps, position 0's about ln n).
constexpr int kFyRegs = 32;

__global__ __launch_bounds__(256) void k_fy_sort(int32_t *__restrict__ head,
                                                 int32_t *__restrict__ next, int64_t n) {
  for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < n;
       p += (int64_t)gridDim.x * blockDim.x) {
    const int32_t h = head[p];
    if (h < 0) continue;
    int32_t e[kFyRegs];
    int L = 0;
    int32_t x = h;
#pragma unroll
    for (int q = 0; q < kFyRegs; ++q) {
      e[q] = INT32_MAX;
      if (x >= 0) {
        e[q] = x;
        x = next[x];
        L = q + 1;
      }
    }
    if (x >= 0) {  // longer: merge sort in place
      const int32_t s = fy_merge_sort(h, next);
      head[p] = s;
      int32_t y = s;
      while (next[y] >= 0) y = next[y];
      next[y] = -2 - (int32_t)p;
      continue;
    }
    if (L > 1) oe_sort<0, kFyRegs>(e);
    head[p] = e[0];
#pragma unroll
    for (int q = 0; q < kFyRegs; ++q)
      if (q < L) next[e[q]] = (q + 1 < L) ? e[q + 1] : -2 - (int32_t)p;
  }
}

__global__ __launch_bounds__(256) void k_fy_resolve(const int32_t *__restrict__ head,
                                                    const int32_t *__restrict__ a_old,
                                                    int32_t *__restrict__ v, int64_t n) {
  for (int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; k < n;
       k += (int64_t)gridDim.x * blockDim.x) {
    int32_t x = (int32_t)k;
    for (int32_t h = head[x]; h >= 0; h = head[x]) x = h;
    v[k] = a_old[x];
  }
}

__global__ __launch_bounds__(256) void k_fy_final(const uint32_t *__restrict__ draws,
                                                  const uint32_t *const *draws_ref, int64_t n,
                                                  const int32_t *__restrict__ next,
                                                  const int32_t *__restrict__ v,
                                                  const int32_t *__restrict__ a_old,
                                                  int32_t *__restrict__ a_new) {
  if (draws_ref) draws = *draws_ref;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    int32_t out;
    if (i == 0 || (int64_t)draws[n - 1 - i] == i) {
      out = v[i];
    } else {
      const int32_t g = next[i];
      out = g >= 0 ? v[g] : a_old[-2 - g];
    }
    a_new[i] = out;
  }
}

// ---------------------------------------------------------------------------
// Sorted form of the same lists.  Key s (s < n) is (j(s) << 32) | s for
// every step s >= 1, self steps (j(s) = s) included, and (0 << 32) | 0 for
// position 0 (FyKeysIn); the radix sort's first pass makes them from the
// draws.  A stable sort by the high word puts each position's steps
// together in ascending order.  A self step s, or position 0, is the first
// key of position s's run (every other step choosing s is larger), and its
// successor in the run is head[s] of the list form, so
//   a_new[s] = v(successor) or a_old[s] without one
// is the same rule as for the other steps (v(s) = v(head[s]) or a_old[s]);
// head[p] itself skips it.
// ---------------------------------------------------------------------------
constexpr uint64_t kFyNoKey = ~0ull;

// head[p] of every position with steps: the run's first step (the second
// when the first is p itself).  (head is -1 everywhere on entry: positions
// without steps keep it.  Writing those here instead, from each run start
// over the positions before it, made the 10M round 10% longer: near the
// top positions are chosen rarely, so single lanes looped over long gaps.)
__global__ __launch_bounds__(256) void k_fy_links(const uint64_t *__restrict__ keys, int64_t ld,
                                                  int32_t *__restrict__ head) {
  for (int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; s < ld;
       s += (int64_t)gridDim.x * blockDim.x) {
    const uint64_t key = keys[s];
    if (key == kFyNoKey) continue;
    const uint32_t p = (uint32_t)(key >> 32);
    if (s > 0 && (uint32_t)(keys[s - 1] >> 32) == p) continue;  // not a run start
    const int32_t k = (int32_t)(key & 0xffffffffu);
    const uint64_t nk = s + 1 < ld ? keys[s + 1] : kFyNoKey;
    const bool next_same = nk != kFyNoKey && (uint32_t)(nk >> 32) == p;
    head[p] = k != (int32_t)p ? k : (next_same ? (int32_t)(nk & 0xffffffffu) : -1);
  }
}

// v(x) = a_old at the end of x's chain x -> head[x] -> ... (the value at
// position x just before step x).
__device__ __forceinline__ int32_t fy_value(const int32_t *__restrict__ head,
                                            const int32_t *__restrict__ a_old, int32_t x) {
  for (int32_t h = head[x]; h >= 0; h = head[x]) x = h;
  return a_old[x];
}

// a_new[k] for every key, in sorted order: v of the next step of k's run
// (resolved here, for the about 37% of the keys that have one), or a_old[p]
// for the last key of position p's run.  With flags, flags[a_new[k]] = 1
// for k < m.
__global__ __launch_bounds__(256) void k_fy_final_sorted(const uint64_t *__restrict__ keys,
                                                         int64_t ld,
                                                         const int32_t *__restrict__ head,
                                                         const int32_t *__restrict__ a_old,
                                                         int32_t *__restrict__ a_new,
                                                         uint8_t *__restrict__ flags, int64_t m) {
  for (int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; s < ld;
       s += (int64_t)gridDim.x * blockDim.x) {
    const uint64_t key = keys[s];
    if (key == kFyNoKey) continue;
    const uint32_t p = (uint32_t)(key >> 32);
    const int32_t k = (int32_t)(key & 0xffffffffu);
    const uint64_t nk = s + 1 < ld ? keys[s + 1] : kFyNoKey;
    const bool has_next = nk != kFyNoKey && (uint32_t)(nk >> 32) == p;
    const int32_t v = has_next ? fy_value(head, a_old, (int32_t)(nk & 0xffffffffu)) : a_old[p];
    a_new[k] = v;
    if (flags && k < m) flags[v] = 1;
  }
}

}  // namespace

hipError_t launch_fisher_yates(hipStream_t st, const uint32_t *draws, int64_t n,
                               const int32_t *a_old, int32_t *a_new, const FyWork &w,
                               uint8_t *flags, int64_t m) {
  if (n <= 0) return hipSuccess;
  const dim3 g(blocks_for(n)), b(256);
  if (w.keys) {
    const int64_t ld = sort_u64_ld(n);
    int bits = 8;  // at least one pass, which makes the keys
    while (bits < 32 && ((uint64_t)(n - 1) >> bits) != 0) bits += 8;  // positions < 2^bits
    const dim3 gk(blocks_for(ld));
    uint64_t *sorted = nullptr;
    hipLaunchKernelGGL(k_fill_neg, dim3(blocks_for((n + 3) / 4)), b, 0, st, w.head, n);
    hipError_t e = launch_sort_fy_keys(st, FyKeysIn{draws, w.draws_ref, n}, w.keys, w.keys_tmp,
                                       ld, 32, 32 + bits, w.counts, w.totals, &sorted);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_fy_links, gk, b, 0, st, sorted, ld, w.head);
    hipLaunchKernelGGL(k_fy_final_sorted, gk, b, 0, st, sorted, ld, w.head, a_old, a_new, flags,
                       m);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(k_fill_neg, dim3(blocks_for((n + 3) / 4)), b, 0, st, w.head, n);
  if (n > 1) hipLaunchKernelGGL(k_fy_push, g, b, 0, st, draws, w.draws_ref, n, w.head, w.next);
  hipLaunchKernelGGL(k_fy_sort, g, b, 0, st, w.head, w.next, n);
  hipLaunchKernelGGL(k_fy_resolve, g, b, 0, st, w.head, a_old, w.v, n);
  hipLaunchKernelGGL(k_fy_final, g, b, 0, st, draws, w.draws_ref, n, w.next, w.v, a_old, a_new);
  return hipGetLastError();
}

}  // namespace bsscl
