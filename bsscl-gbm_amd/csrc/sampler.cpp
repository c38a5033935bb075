// Row/column bagging stream of the boosting loop, native and bit-identical to
// NumPy's legacy RandomState.
//
// The reference draws each round's in-bag rows with
//   rng.shuffle(all_sample_indices); sample_idx = all_sample_indices[:n_sub]
// and its feature subset with
//   rng.shuffle(all_feature_indices); feat_idx = sort(all_feature_indices[:k])
// (src/bsscl_gbm/estimator_v1_0_1.py:2502-2517, rng created at :3159).  The
// shuffle is cumulative across rounds and single-threaded in NumPy (44 ms for
// 1M rows, 0.63 s for 10M on an 8-core Xeon), which would cap the engine's
// trees/s on the host.  This file restates the same stream:
//
//   * MT19937 (Matsumoto & Nishimura 1998): 624-word state, twist with
//     matrix 0x9908b0df, tempering shifts 11/7/15/18 with masks
//     0x9d2c5680/0xefc60000; the state and position come from
//     RandomState.get_state(), so no seeding code is needed here.
//   * NumPy's bounded integer for the legacy shuffle: smallest all-ones mask
//     >= max, draw 32-bit words (64-bit when max > 2^32-1, high word first)
//     until (word & mask) <= max.
//   * Fisher-Yates from the end: for i = n-1 .. 1, swap a[i] with a[j(i)].
//
// The random numbers do not depend on the data, so the swap loop draws them
// a fixed distance ahead and prefetches a[j] -- the only change from the
// plain loop, and it leaves the sequence of swaps unchanged.
//
// Rounds are produced by a worker thread up to `lookahead` rounds ahead of
// the consumer; each round is delivered as the in-bag row ids in ascending
// order (the tree builder's fixed-point sums do not depend on row order) and
// the sorted feature subset.
#include "bsscl_internal.h"

#include <algorithm>
#include <condition_variable>
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

struct MT {
  uint32_t key[kN];
  int pos;

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
    pos = 0;
  }

  inline uint32_t next32() {
    if (pos >= kN) twist();
    uint32_t y = key[pos++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
  }

  inline uint64_t next64() {
    uint64_t hi = next32();
    uint64_t lo = next32();
    return (hi << 32) | lo;
  }

  // Uniform integer in [0, max] by masked rejection.
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
      while ((v = (next64() & mask)) > max) {
      }
    }
    return v;
  }
};

template <typename T>
void shuffle_inplace(MT &mt, T *a, int64_t n) {
  if (n <= 1) return;
  constexpr int kAhead = 32;  // power of two
  uint64_t ring[kAhead];
  const int64_t first = n - 1;  // steps i = n-1 down to 1
  const int64_t steps = n - 1;
  const int64_t pre = std::min<int64_t>(kAhead, steps);
  for (int64_t s = 0; s < pre; ++s) {
    uint64_t j = mt.interval((uint64_t)(first - s));
    ring[s & (kAhead - 1)] = j;
    __builtin_prefetch(a + j, 1, 1);
  }
  for (int64_t s = 0; s < steps; ++s) {
    const int64_t i = first - s;
    const uint64_t j = ring[s & (kAhead - 1)];
    T t = a[j];
    a[j] = a[i];
    a[i] = t;
    const int64_t s2 = s + kAhead;
    if (s2 < steps) {
      uint64_t j2 = mt.interval((uint64_t)(first - s2));
      ring[s2 & (kAhead - 1)] = j2;
      __builtin_prefetch(a + j2, 1, 1);
    }
  }
}

}  // namespace

struct Sampler {
  MT mt;
  int64_t n = 0, n_sub = 0;
  int32_t F = 0, f_sub = 0;
  bool do_rows = false, do_feats = false;
  int32_t n_rounds = 0, lookahead = 2;
  std::vector<int32_t> rows;   // cumulative permutation of 0..n-1
  std::vector<int32_t> feats;  // cumulative permutation of 0..F-1
  std::vector<uint64_t> bitmap;

  struct Round {
    std::vector<int32_t> rows;   // ascending in-bag row ids (n_sub)
    std::vector<int32_t> feats;  // ascending selected features (f_sub)
  };
  std::deque<Round> ready;
  std::vector<Round> pool;
  int32_t produced = 0, consumed = 0;
  bool stop = false;
  std::mutex mu;
  std::condition_variable cv_prod, cv_cons;
  std::thread worker;

  void produce_one(Round &r) {
    if (do_rows) shuffle_inplace(mt, rows.data(), n);
    if (do_feats) shuffle_inplace(mt, feats.data(), (int64_t)F);
    r.rows.resize((size_t)n_sub);
    r.feats.resize((size_t)f_sub);
    if (do_rows) {
      // Ascending order of rows[0:n_sub] through a bitmap: O(n) and sequential
      // in memory, cheaper than a sort.
      std::fill(bitmap.begin(), bitmap.end(), 0ull);
      for (int64_t k = 0; k < n_sub; ++k) {
        uint32_t v = (uint32_t)rows[(size_t)k];
        bitmap[v >> 6] |= 1ull << (v & 63);
      }
      int64_t o = 0;
      for (size_t w = 0; w < bitmap.size(); ++w) {
        uint64_t b = bitmap[w];
        while (b) {
          int t = __builtin_ctzll(b);
          r.rows[(size_t)o++] = (int32_t)(w * 64 + (size_t)t);
          b &= b - 1;
        }
      }
    } else {
      for (int64_t k = 0; k < n_sub; ++k) r.rows[(size_t)k] = (int32_t)k;
    }
    std::copy(feats.begin(), feats.begin() + f_sub, r.feats.begin());
    std::sort(r.feats.begin(), r.feats.end());
  }

  void run() {
    for (;;) {
      Round r;
      {
        std::unique_lock<std::mutex> lk(mu);
        cv_prod.wait(lk, [&] {
          return stop || (produced < n_rounds &&
                          (int32_t)ready.size() < lookahead);
        });
        if (stop || produced >= n_rounds) return;
        if (!pool.empty()) {
          r = std::move(pool.back());
          pool.pop_back();
        }
      }
      produce_one(r);
      {
        std::lock_guard<std::mutex> lk(mu);
        ready.push_back(std::move(r));
        ++produced;
      }
      cv_cons.notify_all();
    }
  }
};

}  // namespace bsscl

// Internal: hand the next round to the engine without an extra copy.
namespace bsscl {
int sampler_take(bsscl_sampler *hs, const int32_t **rows, const int32_t **feats,
                 void **token) {
  Sampler *s = reinterpret_cast<Sampler *>(hs);
  if (!s) return set_error(BSSCL_EINVAL, "sampler: null sampler");
  std::unique_lock<std::mutex> lk(s->mu);
  if (s->consumed >= s->n_rounds)
    return set_error(BSSCL_EINVAL, "sampler: all rounds consumed");
  s->cv_cons.wait(lk, [&] { return !s->ready.empty(); });
  auto *r = new Sampler::Round(std::move(s->ready.front()));
  s->ready.pop_front();
  ++s->consumed;
  lk.unlock();
  s->cv_prod.notify_all();
  *rows = r->rows.data();
  *feats = r->feats.data();
  *token = r;
  return BSSCL_OK;
}

void sampler_give_back(bsscl_sampler *hs, void *token) {
  Sampler *s = reinterpret_cast<Sampler *>(hs);
  auto *r = static_cast<Sampler::Round *>(token);
  if (!s || !r) return;
  {
    std::lock_guard<std::mutex> lk(s->mu);
    s->pool.push_back(std::move(*r));
  }
  delete r;
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
  std::memcpy(mt.key, key, sizeof(mt.key));
  mt.pos = *pos;
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
  std::memcpy(mt.key, key, sizeof(mt.key));
  mt.pos = *pos;
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
  std::memcpy(s->mt.key, key, sizeof(s->mt.key));
  s->mt.pos = pos;
  s->n = n;
  s->n_sub = n_sub;
  s->F = n_features;
  s->f_sub = f_sub;
  s->do_rows = do_rows != 0;
  s->do_feats = do_feats != 0;
  s->n_rounds = n_rounds;
  s->lookahead = lookahead;
  try {
    s->rows.resize((size_t)n);
    for (int64_t i = 0; i < n; ++i) s->rows[(size_t)i] = (int32_t)i;
    s->feats.resize((size_t)n_features);
    for (int32_t j = 0; j < n_features; ++j) s->feats[(size_t)j] = j;
    s->bitmap.resize((size_t)((n + 63) / 64));
    s->worker = std::thread([s] { s->run(); });
  } catch (...) {
    delete s;
    return bsscl::set_error(BSSCL_ENOMEM, "sampler_create: allocation failed");
  }
  *out = reinterpret_cast<bsscl_sampler *>(s);
  return BSSCL_OK;
}

int bsscl_sampler_next(bsscl_sampler *hs, int32_t *rows_out,
                       int32_t *feats_out) {
  Sampler *s = reinterpret_cast<Sampler *>(hs);
  if (!s) return bsscl::set_error(BSSCL_EINVAL, "sampler_next: null sampler");
  Sampler::Round r;
  {
    std::unique_lock<std::mutex> lk(s->mu);
    if (s->consumed >= s->n_rounds)
      return bsscl::set_error(BSSCL_EINVAL, "sampler_next: all rounds consumed");
    s->cv_cons.wait(lk, [&] { return !s->ready.empty(); });
    r = std::move(s->ready.front());
    s->ready.pop_front();
    ++s->consumed;
  }
  s->cv_prod.notify_all();
  if (rows_out) std::memcpy(rows_out, r.rows.data(), r.rows.size() * sizeof(int32_t));
  if (feats_out) std::memcpy(feats_out, r.feats.data(), r.feats.size() * sizeof(int32_t));
  {
    std::lock_guard<std::mutex> lk(s->mu);
    s->pool.push_back(std::move(r));
  }
  return BSSCL_OK;
}

int bsscl_sampler_state(bsscl_sampler *hs, uint32_t *key_out,
                        int32_t *pos_out) {
  // State after every produced round (the worker may be ahead of the
  // consumer); only meaningful once all rounds are produced.
  Sampler *s = reinterpret_cast<Sampler *>(hs);
  if (!s || !key_out || !pos_out)
    return bsscl::set_error(BSSCL_EINVAL, "sampler_state: bad arguments");
  std::unique_lock<std::mutex> lk(s->mu);
  if (s->produced < s->n_rounds)
    return bsscl::set_error(BSSCL_EINVAL, "sampler_state: rounds still pending");
  std::memcpy(key_out, s->mt.key, sizeof(s->mt.key));
  *pos_out = s->mt.pos;
  return BSSCL_OK;
}

void bsscl_sampler_destroy(bsscl_sampler *hs) {
  Sampler *s = reinterpret_cast<Sampler *>(hs);
  if (!s) return;
  {
    std::lock_guard<std::mutex> lk(s->mu);
    s->stop = true;
  }
  s->cv_prod.notify_all();
  if (s->worker.joinable()) s->worker.join();
  delete s;
}

}  // extern "C"
