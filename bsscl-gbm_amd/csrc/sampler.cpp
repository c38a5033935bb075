// Row/column bagging stream of the boosting loop, native and bit-identical to
// NumPy's legacy RandomState.
//
// The reference draws each round's in-bag rows with
//   rng.shuffle(all_sample_indices); sample_idx = all_sample_indices[:n_sub]
// and its feature subset with
//   rng.shuffle(all_feature_indices); feat_idx = sort(all_feature_indices[:k])
// (src/bsscl_gbm/estimator_v1_0_1.py:2502-2517, rng created at :3159).  The
// shuffle is cumulative across rounds and single-threaded in NumPy (44 ms for
// 1M rows on an 8-core Xeon), which would cap the engine's trees/s on the
// host.  This file restates the same stream:
//
//   * MT19937 (Matsumoto & Nishimura 1998): 624-word state, twist with
//     matrix 0x9908b0df, tempering shifts 11/7/15/18 with masks
//     0x9d2c5680/0xefc60000.  The state and position come from
//     RandomState.get_state(), so no seeding code is needed here.
//   * NumPy's bounded integer for the legacy shuffle: smallest all-ones mask
//     >= max, draw 32-bit words (64-bit when max > 2^32-1, high word first)
//     until (word & mask) <= max.
//   * Fisher-Yates from the end: for i = n-1 .. 1, swap a[i] with a[j(i)].
//
// The random numbers never depend on the data, which allows three changes
// that leave the sequence of swaps unchanged:
//   * each 624-word block is twisted and tempered at once, and the bounded
//     draws for a whole range of mask-constant steps run in one branch-free
//     loop (a rejected word is overwritten by the next one);
//   * the draws of round r+1 are made on one thread while another thread
//     applies the swaps of round r;
//   * the swap loop prefetches a[j] a fixed distance ahead.
//
// Each round is delivered as the reference's sample_idx (the first n_sub
// entries of the permuted array, in that order) and the sorted feature
// subset, up to `lookahead` rounds ahead of the consumer.
#include "bsscl_internal.h"

#include <hip/hip_runtime.h>

#include <sys/mman.h>

#include <algorithm>
#include <chrono>
#include <condition_variable>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <mutex>
#include <thread>
#include <vector>

namespace bsscl {

namespace {

constexpr int kN = 624;
constexpr int kM = 397;
constexpr uint32_t kMatrixA = 0x9908b0dfu;
constexpr uint32_t kUpper = 0x80000000u;
constexpr uint32_t kLower = 0x7fffffffu;

inline uint32_t temper(uint32_t y) {
  y ^= y >> 11;
  y ^= (y << 7) & 0x9d2c5680u;
  y ^= (y << 15) & 0xefc60000u;
  y ^= y >> 18;
  return y;
}

struct MT {
  uint32_t key[kN];
  uint32_t out[kN];  // tempered key[] of the current block
  int pos;           // next word of the block (NumPy's state position)

  void load(const uint32_t *k, int p) {
    std::memcpy(key, k, sizeof(key));
    pos = p;
    for (int i = 0; i < kN; ++i) out[i] = temper(key[i]);
  }

  void twist() {
    int i = 0;
    for (; i < kN - kM; ++i) {
      uint32_t y = (key[i] & kUpper) | (key[i + 1] & kLower);
      key[i] = key[i + kM] ^ (y >> 1) ^ ((0u - (y & 1u)) & kMatrixA);
    }
    for (; i < kN - 1; ++i) {
      uint32_t y = (key[i] & kUpper) | (key[i + 1] & kLower);
      key[i] = key[i + kM - kN] ^ (y >> 1) ^ ((0u - (y & 1u)) & kMatrixA);
    }
    uint32_t y = (key[kN - 1] & kUpper) | (key[0] & kLower);
    key[kN - 1] = key[kM - 1] ^ (y >> 1) ^ ((0u - (y & 1u)) & kMatrixA);
    for (int k = 0; k < kN; ++k) out[k] = temper(key[k]);
    pos = 0;
  }

  inline uint32_t next32() {
    if (pos >= kN) twist();
    return out[pos++];
  }

  // Masked rejection for one bounded draw (any max).
  inline uint64_t interval(uint64_t max) {
    if (max == 0) return 0;
    uint64_t mask = max;
    mask |= mask >> 1;
    mask |= mask >> 2;
    mask |= mask >> 4;
    mask |= mask >> 8;
    mask |= mask >> 16;
    mask |= mask >> 32;
    uint64_t v;
    if (max <= 0xffffffffull) {
      while ((v = (next32() & mask)) > max) {
      }
    } else {
      do {
        const uint64_t hi = next32();
        const uint64_t lo = next32();
        v = ((hi << 32) | lo) & mask;
      } while (v > max);
    }
    return v;
  }

  // Draws for steps i = hi .. 1 of a shuffle (j[i] in [0, i]); hi < 2^32.
  // Within [2^k, 2^(k+1)-1] the mask is constant; the loop writes every word
  // to j[i] and moves to the next step only when the word is accepted.
  void draws(uint64_t hi, uint32_t *j) {
    uint64_t i = hi;
    while (i >= 1) {
      const int k = 63 - __builtin_clzll(i);
      const uint64_t lo = 1ull << k;
      const uint32_t mask = (uint32_t)((lo << 1) - 1);
      while (i >= lo) {
        if (pos >= kN) twist();
        const uint32_t *w = out + pos;
        const int avail = kN - pos;
        int used = 0;
        while (used < avail && i >= lo) {
          const uint32_t v = w[used++] & mask;
          j[i] = v;
          i -= (v <= i) ? 1u : 0u;
        }
        pos += used;
      }
    }
  }
};

template <typename T>
void shuffle_inplace(MT &mt, T *a, int64_t n) {
  if (n <= 1) return;
  if ((uint64_t)(n - 1) > 0xffffffffull) {
    for (int64_t i = n - 1; i >= 1; --i) {
      const uint64_t j = mt.interval((uint64_t)i);
      T t = a[j];
      a[j] = a[i];
      a[i] = t;
    }
    return;
  }
  std::vector<uint32_t> j((size_t)n);
  mt.draws((uint64_t)(n - 1), j.data());
  constexpr int64_t kAhead = 32;
  for (int64_t i = n - 1; i >= 1; --i) {
    if (i > kAhead) __builtin_prefetch(a + j[(size_t)(i - kAhead)], 1, 1);
    const uint32_t ji = j[(size_t)i];
    T t = a[ji];
    a[ji] = a[i];
    a[i] = t;
  }
}

// Host buffer for a round's rows: pinned when a HIP device is present (the
// engine copies it to the GPU asynchronously), plain memory otherwise.
struct HostBuf {
  int32_t *p = nullptr;
  size_t n = 0;
  bool pinned = false;
  void alloc(size_t count) {
    if (count <= n && p) return;
    release();
    void *q = nullptr;
    if (hipHostMalloc(&q, count * sizeof(int32_t), hipHostMallocDefault) == hipSuccess) {
      pinned = true;
    } else {
      (void)hipGetLastError();
      q = std::malloc(count * sizeof(int32_t));
      pinned = false;
    }
    if (!q) throw std::bad_alloc();
    p = static_cast<int32_t *>(q);
    n = count;
  }
  void release() {
    if (p) {
      if (pinned) (void)hipHostFree(p);
      else std::free(p);
    }
    p = nullptr;
    n = 0;
  }
};

// Array backed by 2 MB pages where the kernel allows it: the swap loop makes
// one random access per step into an array of up to 40 MB, and 4 KB pages
// would add a TLB miss to most of them.
template <typename T>
struct BigArray {
  T *p = nullptr;
  size_t n = 0;
  void alloc(size_t count) {
    const size_t huge = size_t(2) << 20;
    const size_t bytes = (count * sizeof(T) + huge - 1) / huge * huge;
    void *q = std::aligned_alloc(huge, bytes);
    if (!q) throw std::bad_alloc();
    (void)madvise(q, bytes, MADV_HUGEPAGE);
    p = static_cast<T *>(q);
    n = count;
  }
  ~BigArray() { std::free(p); }
  T &operator[](size_t i) { return p[i]; }
  T *data() { return p; }
};

}  // namespace

struct Sampler {
  MT mt;  // owned by the draw thread once started
  int64_t n = 0, n_sub = 0;
  int32_t F = 0, f_sub = 0;
  bool do_rows = false, do_feats = false;
  int32_t n_rounds = 0, lookahead = 2;

  struct Draws {  // one round's bounded draws
    std::vector<uint32_t> rows, feats;
  };
  struct Round {
    HostBuf rows;                // sample_idx, reference order
    std::vector<int32_t> feats;  // ascending selected features
  };

  std::deque<Draws> drawn;       // draw thread -> swap thread
  std::vector<Draws> draw_pool;
  std::deque<Round> ready;       // swap thread -> consumer
  std::vector<Round> pool;
  int32_t n_drawn = 0, produced = 0, consumed = 0;
  bool stop = false;
  uint32_t final_key[kN];
  int final_pos = 0;
  std::mutex mu;
  std::condition_variable cv;
  std::thread draw_thread, swap_thread;
  std::string error;

  // Cumulative permutations (swap thread only).
  BigArray<int32_t> rows;
  std::vector<int32_t> feats;
  double draw_ms = 0.0, swap_ms = 0.0;  // time spent in each stage

  void run_draws() {
    try {
      for (;;) {
        Draws d;
        {
          std::unique_lock<std::mutex> lk(mu);
          cv.wait(lk, [&] { return stop || (n_drawn < n_rounds && (int32_t)drawn.size() < 2); });
          if (stop || n_drawn >= n_rounds) return;
          if (!draw_pool.empty()) {
            d = std::move(draw_pool.back());
            draw_pool.pop_back();
          }
        }
        const auto t0 = std::chrono::steady_clock::now();
        if (do_rows) {
          d.rows.resize((size_t)n);
          mt.draws((uint64_t)(n - 1), d.rows.data());
        }
        if (do_feats && F > 1) {
          d.feats.resize((size_t)F);
          mt.draws((uint64_t)(F - 1), d.feats.data());
        }
        const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        {
          std::lock_guard<std::mutex> lk(mu);
          draw_ms += ms;
          drawn.push_back(std::move(d));
          ++n_drawn;
          if (n_drawn == n_rounds) {
            std::memcpy(final_key, mt.key, sizeof(final_key));
            final_pos = mt.pos;
          }
        }
        cv.notify_all();
      }
    } catch (...) {
      std::lock_guard<std::mutex> lk(mu);
      error = "sampler: draw thread failed";
      stop = true;
      cv.notify_all();
    }
  }

  // Applies one round's swaps and fills r; returns the milliseconds spent in
  // the swap loops (the round buffer's first allocation is not counted).
  double apply(const Draws &d, Round &r) {
    const auto t0 = std::chrono::steady_clock::now();
    if (do_rows) {
      const uint32_t *j = d.rows.data();
      int32_t *a = rows.data();
      constexpr int64_t kAhead = 32;
      for (int64_t i = n - 1; i >= 1; --i) {
        if (i > kAhead) __builtin_prefetch(a + j[i - kAhead], 1, 1);
        const uint32_t ji = j[i];
        const int32_t t = a[ji];
        a[ji] = a[i];
        a[i] = t;
      }
    }
    if (do_feats && F > 1) {
      const uint32_t *j = d.feats.data();
      for (int32_t i = F - 1; i >= 1; --i) std::swap(feats[(size_t)i], feats[j[i]]);
    }
    const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    r.rows.alloc((size_t)n_sub);
    std::memcpy(r.rows.p, rows.data(), (size_t)n_sub * sizeof(int32_t));
    r.feats.assign(feats.begin(), feats.begin() + f_sub);
    std::sort(r.feats.begin(), r.feats.end());
    return ms;
  }

  void run_swaps() {
    try {
      for (;;) {
        Draws d;
        Round r;
        {
          std::unique_lock<std::mutex> lk(mu);
          cv.wait(lk, [&] {
            return stop || produced >= n_rounds ||
                   (!drawn.empty() && (int32_t)ready.size() < lookahead);
          });
          if (stop || produced >= n_rounds) return;
          d = std::move(drawn.front());
          drawn.pop_front();
          if (!pool.empty()) {
            r = std::move(pool.back());
            pool.pop_back();
          }
        }
        cv.notify_all();
        const double ms = apply(d, r);
        {
          std::lock_guard<std::mutex> lk(mu);
          swap_ms += ms;
          ready.push_back(std::move(r));
          ++produced;
          draw_pool.push_back(std::move(d));
        }
        cv.notify_all();
      }
    } catch (...) {
      std::lock_guard<std::mutex> lk(mu);
      error = "sampler: swap thread failed (out of memory?)";
      stop = true;
      cv.notify_all();
    }
  }

  // Blocks until the next round is ready; the caller returns it with give().
  Round *take() {
    std::unique_lock<std::mutex> lk(mu);
    if (consumed >= n_rounds) return nullptr;
    cv.wait(lk, [&] { return stop || !ready.empty(); });
    if (ready.empty()) return nullptr;
    Round *r = new Round(std::move(ready.front()));
    ready.pop_front();
    ++consumed;
    lk.unlock();
    cv.notify_all();
    return r;
  }

  void give(Round *r) {
    {
      std::lock_guard<std::mutex> lk(mu);
      pool.push_back(std::move(*r));
    }
    delete r;
    cv.notify_all();
  }

  ~Sampler() {
    {
      std::lock_guard<std::mutex> lk(mu);
      stop = true;
    }
    cv.notify_all();
    if (draw_thread.joinable()) draw_thread.join();
    if (swap_thread.joinable()) swap_thread.join();
    for (auto &r : ready) r.rows.release();
    for (auto &r : pool) r.rows.release();
  }
};

int sampler_take(bsscl_sampler *hs, const int32_t **rows, const int32_t **feats,
                 void **token) {
  Sampler *s = reinterpret_cast<Sampler *>(hs);
  if (!s) return set_error(BSSCL_EINVAL, "sampler: null sampler");
  Sampler::Round *r = s->take();
  if (!r) {
    std::lock_guard<std::mutex> lk(s->mu);
    return set_error(BSSCL_EINVAL, s->error.empty() ? "sampler: all rounds consumed" : s->error);
  }
  *rows = r->rows.p;
  *feats = r->feats.data();
  *token = r;
  return BSSCL_OK;
}

void sampler_give_back(bsscl_sampler *hs, void *token) {
  Sampler *s = reinterpret_cast<Sampler *>(hs);
  auto *r = static_cast<Sampler::Round *>(token);
  if (!s || !r) return;
  s->give(r);
}

int64_t sampler_n_sub(bsscl_sampler *hs) {
  return reinterpret_cast<Sampler *>(hs)->n_sub;
}
int32_t sampler_f_sub(bsscl_sampler *hs) {
  return reinterpret_cast<Sampler *>(hs)->f_sub;
}

}  // namespace bsscl

using bsscl::Sampler;

extern "C" {

int bsscl_rs_shuffle_i64(uint32_t *key, int32_t *pos, int64_t *data,
                         int64_t n) {
  if (!key || !pos || (n > 0 && !data) || *pos < 0 || *pos > 624)
    return bsscl::set_error(BSSCL_EINVAL, "rs_shuffle: bad state or buffer");
  bsscl::MT mt;
  mt.load(key, *pos);
  bsscl::shuffle_inplace(mt, data, n);
  std::memcpy(key, mt.key, sizeof(mt.key));
  *pos = mt.pos;
  return BSSCL_OK;
}

int bsscl_rs_shuffle_i32(uint32_t *key, int32_t *pos, int32_t *data,
                         int64_t n) {
  if (!key || !pos || (n > 0 && !data) || *pos < 0 || *pos > 624)
    return bsscl::set_error(BSSCL_EINVAL, "rs_shuffle: bad state or buffer");
  bsscl::MT mt;
  mt.load(key, *pos);
  bsscl::shuffle_inplace(mt, data, n);
  std::memcpy(key, mt.key, sizeof(mt.key));
  *pos = mt.pos;
  return BSSCL_OK;
}

int bsscl_sampler_create(const uint32_t *key, int32_t pos, int64_t n,
                         int64_t n_sub, int32_t do_rows, int32_t n_features,
                         int32_t f_sub, int32_t do_feats, int32_t n_rounds,
                         int32_t lookahead, bsscl_sampler **out) {
  if (!key || !out || pos < 0 || pos > 624 || n <= 0 || n > INT32_MAX ||
      n_sub <= 0 || n_sub > n || n_features <= 0 || f_sub <= 0 ||
      f_sub > n_features || n_rounds < 0 || lookahead < 1)
    return bsscl::set_error(BSSCL_EINVAL, "sampler_create: bad arguments");
  if (!do_rows && n_sub != n)
    return bsscl::set_error(BSSCL_EINVAL,
                            "sampler_create: n_sub must equal n without row bagging");
  if (!do_feats && f_sub != n_features)
    return bsscl::set_error(BSSCL_EINVAL,
                            "sampler_create: f_sub must equal F without column bagging");
  Sampler *s = new (std::nothrow) Sampler();
  if (!s) return bsscl::set_error(BSSCL_ENOMEM, "sampler_create: out of memory");
  s->mt.load(key, pos);
  s->n = n;
  s->n_sub = n_sub;
  s->F = n_features;
  s->f_sub = f_sub;
  s->do_rows = do_rows != 0;
  s->do_feats = do_feats != 0;
  s->n_rounds = n_rounds;
  s->lookahead = lookahead;
  std::memcpy(s->final_key, key, sizeof(s->final_key));
  s->final_pos = pos;
  try {
    s->rows.alloc((size_t)n);
    for (int64_t i = 0; i < n; ++i) s->rows[(size_t)i] = (int32_t)i;
    s->feats.resize((size_t)n_features);
    for (int32_t j = 0; j < n_features; ++j) s->feats[(size_t)j] = j;
    s->draw_thread = std::thread([s] { s->run_draws(); });
    s->swap_thread = std::thread([s] { s->run_swaps(); });
  } catch (...) {
    delete s;
    return bsscl::set_error(BSSCL_ENOMEM, "sampler_create: allocation failed");
  }
  *out = reinterpret_cast<bsscl_sampler *>(s);
  return BSSCL_OK;
}

int bsscl_sampler_next(bsscl_sampler *hs, int32_t *rows_out,
                       int32_t *feats_out) {
  const int32_t *rows = nullptr, *feats = nullptr;
  void *token = nullptr;
  int rc = bsscl::sampler_take(hs, &rows, &feats, &token);
  if (rc != BSSCL_OK) return rc;
  Sampler *s = reinterpret_cast<Sampler *>(hs);
  if (rows_out) std::memcpy(rows_out, rows, (size_t)s->n_sub * sizeof(int32_t));
  if (feats_out) std::memcpy(feats_out, feats, (size_t)s->f_sub * sizeof(int32_t));
  bsscl::sampler_give_back(hs, token);
  return BSSCL_OK;
}

int bsscl_sampler_state(bsscl_sampler *hs, uint32_t *key_out,
                        int32_t *pos_out) {
  Sampler *s = reinterpret_cast<Sampler *>(hs);
  if (!s || !key_out || !pos_out)
    return bsscl::set_error(BSSCL_EINVAL, "sampler_state: bad arguments");
  std::unique_lock<std::mutex> lk(s->mu);
  s->cv.wait(lk, [&] { return s->stop || s->n_drawn >= s->n_rounds; });
  if (s->n_drawn < s->n_rounds)
    return bsscl::set_error(BSSCL_EINVAL, "sampler_state: sampler stopped early");
  std::memcpy(key_out, s->final_key, sizeof(s->final_key));
  *pos_out = s->final_pos;
  return BSSCL_OK;
}

int bsscl_sampler_stats(bsscl_sampler *hs, double *out, int32_t cap,
                        int32_t *n_out) {
  Sampler *s = reinterpret_cast<Sampler *>(hs);
  if (!s || !out || !n_out) return bsscl::set_error(BSSCL_EINVAL, "sampler_stats: bad arguments");
  std::lock_guard<std::mutex> lk(s->mu);
  const double v[3] = {(double)s->produced, s->draw_ms, s->swap_ms};
  const int32_t k = std::min<int32_t>(cap, 3);
  for (int32_t i = 0; i < k; ++i) out[i] = v[i];
  *n_out = k;
  return BSSCL_OK;
}

void bsscl_sampler_destroy(bsscl_sampler *hs) {
  delete reinterpret_cast<Sampler *>(hs);
}

}  // extern "C"
