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
// The random numbers never depend on the data, so the work is split into
// stages that run on their own threads without changing the sequence:
//   * a draw thread twists and tempers whole 624-word blocks (AVX-512 when
//     the CPU has it), a chunk at a time, and turns the words into the
//     bounded draws j(i) of every round.  Within a run of steps with a
//     constant mask, W = 64 (then 16) words are classified at once: a word
//     <= i - (W-1) is accepted whatever happened to the words before it
//     (each acceptance lowers i by one), a word > i is rejected whatever
//     happened, and only a block holding a word in between is decided with
//     a narrower window or one word at a time;
//   * long shuffles are counted in parallel instead: a twister thread makes
//     each chunk's first-block state ahead of time, worker threads compute
//     every chunk's transfer function (entry step -> exit step) over a
//     window of likely entry steps, the draw thread maps the true entry
//     step through the chunks in order, and worker threads regenerate each
//     chunk and write its draws (see "Parallel draws" below);
//   * the swaps: in device-rows mode the draws are handed to the engine,
//     which applies them on the GPU (bsscl_fisher_yates_apply); otherwise a
//     swap thread applies them on the host and delivers sample_idx.
//
// Each round is delivered up to `lookahead` rounds ahead of the consumer.
#include "bsscl_internal.h"

#include <hip/hip_runtime.h>

#include <immintrin.h>
#include <pthread.h>
#include <sys/mman.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <condition_variable>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <memory>
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

inline uint32_t twist_word(uint32_t a, uint32_t b, uint32_t m) {
  const uint32_t y = (a & kUpper) | (b & kLower);
  return m ^ (y >> 1) ^ ((0u - (y & 1u)) & kMatrixA);
}

// One MT19937 state transition in place (scalar).
void twist_scalar(uint32_t *key) {
  int i = 0;
  for (; i < kN - kM; ++i) key[i] = twist_word(key[i], key[i + 1], key[i + kM]);
  for (; i < kN - 1; ++i) key[i] = twist_word(key[i], key[i + 1], key[i + kM - kN]);
  key[kN - 1] = twist_word(key[kN - 1], key[0], key[kM - 1]);
}

// key[i .. i+15] = twist of (key[i+k], key[i+k+1]) xor key[m+k].
__attribute__((target("avx512f"))) inline void twist16(uint32_t *key, int i, int m) {
  const __m512i a = _mm512_loadu_si512(key + i);
  const __m512i b = _mm512_loadu_si512(key + i + 1);
  const __m512i c = _mm512_loadu_si512(key + m);
  const __m512i y = _mm512_or_si512(_mm512_and_si512(a, _mm512_set1_epi32((int)kUpper)),
                                    _mm512_and_si512(b, _mm512_set1_epi32((int)kLower)));
  const __mmask16 odd = _mm512_test_epi32_mask(y, _mm512_set1_epi32(1));
  __m512i r = _mm512_xor_si512(c, _mm512_srli_epi32(y, 1));
  r = _mm512_mask_xor_epi32(r, odd, r, _mm512_set1_epi32((int)kMatrixA));
  _mm512_storeu_si512(key + i, r);
}

// The same transition 16 words at a time.  Words [0, 227) read only old
// words (i + 1 and i + 397); words [227, 623) read i + 1 (old) and i - 227,
// which an earlier step of this pass has already written.
__attribute__((target("avx512f"))) void twist_avx512(uint32_t *key) {
  int i = 0;
  for (; i + 16 <= kN - kM; i += 16) twist16(key, i, i + kM);
  for (; i < kN - kM; ++i) key[i] = twist_word(key[i], key[i + 1], key[i + kM]);
  for (; i + 16 <= kN - 1; i += 16) twist16(key, i, i + kM - kN);
  for (; i < kN - 1; ++i) key[i] = twist_word(key[i], key[i + 1], key[i + kM - kN]);
  key[kN - 1] = twist_word(key[kN - 1], key[0], key[kM - 1]);
}

__attribute__((target("avx512f"))) void temper_avx512(const uint32_t *key, uint32_t *out) {
  const __m512i b = _mm512_set1_epi32((int)0x9d2c5680u);
  const __m512i c = _mm512_set1_epi32((int)0xefc60000u);
  for (int i = 0; i < kN; i += 16) {  // 624 = 39 * 16
    __m512i y = _mm512_loadu_si512(key + i);
    y = _mm512_xor_si512(y, _mm512_srli_epi32(y, 11));
    y = _mm512_xor_si512(y, _mm512_and_si512(_mm512_slli_epi32(y, 7), b));
    y = _mm512_xor_si512(y, _mm512_and_si512(_mm512_slli_epi32(y, 15), c));
    y = _mm512_xor_si512(y, _mm512_srli_epi32(y, 18));
    _mm512_storeu_si512(out + i, y);
  }
}

// AVX-512 paths unless the CPU lacks them or BSSCL_SAMPLER_SCALAR=1.
bool use_avx512() {
  static const bool ok = [] {
    const char *e = std::getenv("BSSCL_SAMPLER_SCALAR");
    if (e && e[0] == '1') return false;
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512vl") &&
           __builtin_cpu_supports("avx512bw");
  }();
  return ok;
}

// Scalar MT19937 with NumPy's position convention, for one-shot shuffles
// and draws (bsscl_rs_*).
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
    twist_scalar(key);
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
};

template <typename T>
void shuffle_inplace(MT &mt, T *a, int64_t n) {
  for (int64_t i = n - 1; i >= 1; --i) {
    const uint64_t j = mt.interval((uint64_t)i);
    T t = a[j];
    a[j] = a[i];
    a[i] = t;
  }
}

// Pinned host blocks outlive the sampler that allocated them: the
// process's next sampler takes them.  A fit makes one sampler, and pinning
// a round's draws buffer (4 bytes per row) when the round is first drawn
// held up its first rounds by up to 1.3 ms each at 1M rows.  One list per
// process (a child made by fork() starts an empty one).
struct PinnedBlock {
  void *p;
  size_t bytes;
};
// (Never destroyed: a sampler released during the process's exit still
// finds them.)
std::mutex &g_pinned_mu = *new std::mutex;
std::vector<PinnedBlock> &g_pinned = *new std::vector<PinnedBlock>;
pid_t g_pinned_pid = 0;
constexpr size_t kPinnedKept = 24;

void pinned_list_for_this_process() {
  if (g_pinned_pid != getpid()) {  // (the parent's blocks are not pinned here)
    g_pinned.clear();
    g_pinned_pid = getpid();
  }
}

// The smallest kept block of at least `bytes` (and at most four times
// that); null if none.
void *take_pinned(size_t bytes, size_t *got) {
  std::lock_guard<std::mutex> lk(g_pinned_mu);
  pinned_list_for_this_process();
  size_t best = g_pinned.size();
  for (size_t i = 0; i < g_pinned.size(); ++i)
    if (g_pinned[i].bytes >= bytes && g_pinned[i].bytes / 4 <= bytes &&
        (best == g_pinned.size() || g_pinned[i].bytes < g_pinned[best].bytes))
      best = i;
  if (best == g_pinned.size()) return nullptr;
  void *p = g_pinned[best].p;
  *got = g_pinned[best].bytes;
  g_pinned.erase(g_pinned.begin() + (std::ptrdiff_t)best);
  return p;
}

void keep_pinned(void *p, size_t bytes) {
  {
    std::lock_guard<std::mutex> lk(g_pinned_mu);
    pinned_list_for_this_process();
    if (g_pinned.size() < kPinnedKept) {
      g_pinned.push_back(PinnedBlock{p, bytes});
      return;
    }
  }
  (void)hipHostFree(p);
}

// Host buffer the engine copies from: pinned when a HIP device is present,
// plain memory otherwise.  (A pinned block is kept for later buffers when
// this one is released: no copy reads it by then.)
template <typename T>
struct HostBuf {
  T *p = nullptr;
  size_t n = 0;
  bool pinned = false;
  void alloc(size_t count) {
    if (count <= n && p) return;
    release();
    size_t got = 0;
    void *q = take_pinned(count * sizeof(T), &got);
    if (q) {
      pinned = true;
      count = got / sizeof(T);
    } else if (hipHostMalloc(&q, count * sizeof(T), hipHostMallocDefault) == hipSuccess) {
      pinned = true;
    } else {
      (void)hipGetLastError();
      q = std::malloc(count * sizeof(T));
      pinned = false;
    }
    if (!q) throw std::bad_alloc();
    p = static_cast<T *>(q);
    n = count;
  }
  void release() {
    if (p) {
      if (pinned) keep_pinned(p, n * sizeof(T));
      else std::free(p);
    }
    p = nullptr;
    n = 0;
  }
  HostBuf() = default;
  HostBuf(const HostBuf &) = delete;
  HostBuf &operator=(const HostBuf &) = delete;
  ~HostBuf() { release(); }
};

// Array backed by 2 MB pages where the kernel allows it: the host swap loop
// makes one random access per step into an array of up to 40 MB.
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
  BigArray() = default;
  BigArray(const BigArray &) = delete;
  BigArray &operator=(const BigArray &) = delete;
  ~BigArray() { std::free(p); }
  T &operator[](size_t i) { return p[i]; }
  T *data() { return p; }
};

// ---------------------------------------------------------------------------
// Word stream.  Block b of the stream is the given state (b = 0) or the
// state after b twists, tempered; chunk c holds blocks [c*B, (c+1)*B).  The
// thread that reads the words generates each chunk just before reading it,
// so the words come from its own L2.  (A generator thread feeding a ring of
// chunks to the reader ran at either 0.08 or 0.6 ns per word on the same
// host, from run to run; generating in place costs 0.08 ns per word.)
// ---------------------------------------------------------------------------
constexpr int kChunkBlocks = 32;
constexpr int64_t kChunkWords = (int64_t)kChunkBlocks * kN;

struct Stream {
  const uint32_t *p = nullptr, *end = nullptr, *base = nullptr;
  int64_t chunk = -1;
  uint32_t key[kN];                    // state of the last generated block
  uint32_t cur_key[kN], prev_key[kN];  // first block of the current / previous chunk
  std::vector<uint32_t> buf;           // tempered words of the current chunk
  const std::atomic<bool> *halt = nullptr;
  std::atomic<double> *gen_ms = nullptr;  // time spent generating
  bool vec = false;
  bool key_is_next = true;  // key[] is the next chunk's first block (else: its predecessor)

  // Positions the stream at word pos0 of the state key0.
  bool start(const uint32_t *key0, int pos0, const std::atomic<bool> *h, std::atomic<double> *ms) {
    std::memcpy(key, key0, sizeof(key));
    buf.resize((size_t)kChunkWords);
    halt = h;
    gen_ms = ms;
    vec = use_avx512();
    key_is_next = true;
    if (!next_chunk()) return false;
    p = base + pos0;  // block 0 starts at the given position
    return true;
  }

  // Positions the stream at word `off` of chunk c, whose first block has
  // state key_c.
  bool seek(int64_t c, int64_t off, const uint32_t *key_c, const std::atomic<bool> *h) {
    std::memcpy(key, key_c, sizeof(key));
    buf.resize((size_t)kChunkWords);
    halt = h;
    gen_ms = nullptr;
    vec = use_avx512();
    chunk = c - 1;
    key_is_next = true;
    if (!next_chunk()) return false;
    p = base + off;
    return true;
  }

  // Generates and moves to chunk `chunk + 1`; false if the sampler stops.
  bool next_chunk() {
    if (halt && halt->load(std::memory_order_relaxed)) return false;
    if (chunk >= 0) std::memcpy(prev_key, cur_key, sizeof(cur_key));
    ++chunk;
    const auto t0 = std::chrono::steady_clock::now();
    uint32_t *o = buf.data();
    for (int b = 0; b < kChunkBlocks; ++b, o += kN) {
      if (b > 0 || !key_is_next) {
        if (vec) twist_avx512(key);
        else twist_scalar(key);
      }
      if (b == 0) std::memcpy(cur_key, key, sizeof(key));
      if (vec) {
        temper_avx512(key, o);
      } else {
        for (int k = 0; k < kN; ++k) o[k] = temper(key[k]);
      }
    }
    key_is_next = false;
    if (gen_ms)
      gen_ms->store(gen_ms->load(std::memory_order_relaxed) +
                        std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count(),
                    std::memory_order_relaxed);
    base = buf.data();
    p = base;
    end = base + kChunkWords;
    return true;
  }

  int64_t position() const { return chunk * kChunkWords + (p - base); }

  // NumPy state (key, pos) after the words consumed so far, given the
  // initial state (key0, pos0): the key of the block holding the last
  // consumed word and the offset just past it (pos = 624 at a block's end).
  void state(const uint32_t *key0, int pos0, uint32_t *key_out, int *pos_out) const {
    const int64_t G = position();
    if (G <= pos0) {
      std::memcpy(key_out, key0, sizeof(uint32_t) * kN);
      *pos_out = pos0;
      return;
    }
    const int64_t b = (G - 1) / kN;
    const int64_t c = b / kChunkBlocks;  // chunk, or chunk - 1 when nothing was read from it
    uint32_t k[kN];
    std::memcpy(k, c == chunk ? cur_key : prev_key, sizeof(k));
    for (int64_t t = c * kChunkBlocks; t < b; ++t) twist_scalar(k);
    std::memcpy(key_out, k, sizeof(k));
    *pos_out = (int)(G - b * kN);
  }
};

// Bounded draws of the shuffle steps i = hi .. 1: out[hi - i] = j(i).
// `out` needs 16 words of room past its last entry.  False if stopped.
bool draw_steps_scalar(Stream &s, uint32_t hi, uint32_t *out) {
  uint32_t i = hi;
  while (i >= 1) {
    const uint32_t lo = 1u << (31 - __builtin_clz(i));
    const uint32_t mask = lo | (lo - 1);
    while (i >= lo) {
      if (s.p == s.end && !s.next_chunk()) return false;
      const uint32_t *p = s.p, *e = s.end;
      while (p < e && i >= lo) {
        const uint32_t v = *p++ & mask;
        *out = v;  // kept only when accepted
        const uint32_t a = v <= i ? 1u : 0u;
        out += a;
        i -= a;
      }
      s.p = p;
    }
  }
  return true;
}

// Draws of a long shuffle go through a staging buffer that stays in L1:
// whole 4 KB blocks of it are written to the destination with
// non-temporal stores, which need no read-for-ownership of the
// destination's lines (the destination is read next by the copy engine).
// Ordinary stores made the draw thread store-bound at 10M rows.
constexpr int kStageWords = 1024;

struct Staged {
  alignas(64) uint32_t buf[kStageWords + 128];
  uint32_t *dst = nullptr;

  __attribute__((target("avx512f"))) uint32_t *flush(uint32_t *o) {
    for (int k = 0; k < kStageWords; k += 16)
      _mm512_stream_si512(reinterpret_cast<__m512i *>(dst + k), _mm512_load_si512(buf + k));
    dst += kStageWords;
    const ptrdiff_t rest = (o - buf) - kStageWords;
    std::memmove(buf, buf + kStageWords, (size_t)rest * sizeof(uint32_t));
    return buf + rest;
  }
  void finish(uint32_t *o) {
    std::memcpy(dst, buf, (size_t)(o - buf) * sizeof(uint32_t));
    _mm_sfence();
  }
};

__attribute__((target("avx512f,avx512vl,avx512bw,popcnt")))
bool draw_steps_avx512(Stream &s, uint32_t hi, uint32_t *out) {
  uint32_t i = hi;
  std::unique_ptr<Staged> st;
  uint32_t *const out0 = out;
  const bool staged = hi >= 4 * kStageWords && (reinterpret_cast<uintptr_t>(out) & 63) == 0;
  if (staged) {
    st.reset(new Staged());
    st->dst = out0;
    out = st->buf;
  }
  while (i >= 1) {
    const uint32_t lo = 1u << (31 - __builtin_clz(i));
    const uint32_t mask = lo | (lo - 1);
    const __m512i vm = _mm512_set1_epi32((int)mask);
    while (i >= lo) {
      if (s.p == s.end && !s.next_chunk()) return false;
      const uint32_t *p = s.p, *e = s.end;
      // 64 words at a time: word t's threshold is i - (words accepted
      // before it) >= i - 63, so no word in [i - 62, i] means acceptance is
      // exactly (word <= i).  The mask stays the same for all of them.
      while (i - lo >= 64 && e - p >= 64) {
        const __m512i v0 = _mm512_and_si512(_mm512_loadu_si512(p), vm);
        const __m512i v1 = _mm512_and_si512(_mm512_loadu_si512(p + 16), vm);
        const __m512i v2 = _mm512_and_si512(_mm512_loadu_si512(p + 32), vm);
        const __m512i v3 = _mm512_and_si512(_mm512_loadu_si512(p + 48), vm);
        const __m512i si = _mm512_set1_epi32((int)i);
        const __m512i sb = _mm512_set1_epi32((int)(i - 62));
        const __mmask16 a0 = _mm512_cmple_epu32_mask(v0, si);
        const __mmask16 a1 = _mm512_cmple_epu32_mask(v1, si);
        const __mmask16 a2 = _mm512_cmple_epu32_mask(v2, si);
        const __mmask16 a3 = _mm512_cmple_epu32_mask(v3, si);
        const __mmask16 amb = _mm512_mask_cmpge_epu32_mask(a0, v0, sb) |
                              _mm512_mask_cmpge_epu32_mask(a1, v1, sb) |
                              _mm512_mask_cmpge_epu32_mask(a2, v2, sb) |
                              _mm512_mask_cmpge_epu32_mask(a3, v3, sb);
        if (amb) break;
        const uint32_t c0 = (uint32_t)__builtin_popcount((unsigned)a0);
        const uint32_t c1 = (uint32_t)__builtin_popcount((unsigned)a1);
        const uint32_t c2 = (uint32_t)__builtin_popcount((unsigned)a2);
        const uint32_t c3 = (uint32_t)__builtin_popcount((unsigned)a3);
        _mm512_storeu_si512(out, _mm512_maskz_compress_epi32(a0, v0));
        _mm512_storeu_si512(out + c0, _mm512_maskz_compress_epi32(a1, v1));
        _mm512_storeu_si512(out + c0 + c1, _mm512_maskz_compress_epi32(a2, v2));
        _mm512_storeu_si512(out + c0 + c1 + c2, _mm512_maskz_compress_epi32(a3, v3));
        out += c0 + c1 + c2 + c3;
        i -= c0 + c1 + c2 + c3;
        p += 64;
        if (staged && out - st->buf >= kStageWords) out = st->flush(out);
      }
      // 16 at a time (band [i - 14, i]).
      while (i - lo >= 16 && e - p >= 16) {
        const __m512i v = _mm512_and_si512(_mm512_loadu_si512(p), vm);
        const __mmask16 acc = _mm512_cmple_epu32_mask(v, _mm512_set1_epi32((int)i));
        const __mmask16 amb = _mm512_mask_cmpge_epu32_mask(acc, v, _mm512_set1_epi32((int)(i - 14)));
        if (amb) break;
        _mm512_storeu_si512(out, _mm512_maskz_compress_epi32(acc, v));
        const uint32_t c = (uint32_t)__builtin_popcount((unsigned)acc);
        out += c;
        i -= c;
        p += 16;
        if (staged && out - st->buf >= kStageWords) out = st->flush(out);
      }
      // One word: a block with an order-dependent word, the end of a mask
      // range or the end of a chunk.
      if (p < e) {
        const uint32_t v = *p++ & mask;
        *out = v;
        const uint32_t a = v <= i ? 1u : 0u;
        out += a;
        i -= a;
        if (staged && out - st->buf >= kStageWords) out = st->flush(out);
      }
      s.p = p;
    }
  }
  if (staged) st->finish(out);
  (void)out0;
  return true;
}

// ---------------------------------------------------------------------------
// Parallel draws.  Which words a shuffle accepts is a sequential question
// (word t is tested against the step i, which counts the words accepted
// before it), but its dependence on the step a chunk of words starts at is
// simple.  Run two copies of the test from entry steps e and e + 1 over the
// same words: a word v <= e is accepted by both, v > e + 1 by neither, and
// v = e + 1 is accepted by the upper one only, after which both sit at e
// and stay together.  So the trajectories of a whole window of entries
// [lo, hi] (one mask range) always occupy an interval [a, b] of steps: a word
// v <= a moves it down by one, v > b leaves it, and a < v <= b merges the
// trajectories at v - 1 and v (b drops by one).  A chunk's transfer function
// over its window is therefore the exit of the lowest entry plus the list of
// merges, which worker threads compute for every chunk of a round at once,
// each around the step the chunk is expected to start at.  The draw thread
// then walks the chunks in order with the true entry step, which maps
// through a chunk in O(merges); a chunk whose entry falls outside its window,
// whose window crosses a mask range, or that holds the round's last steps is
// counted word by word.  Each chunk becomes a segment (the chunk's first-
// block state, the first word, the entry step) whose draws, out[hi - i],
// worker threads write with masked stores, so segments never touch each
// other's entries.  The chunks' first-block states come from a twister
// thread that runs ahead of the stream.
// ---------------------------------------------------------------------------
struct Segment {
  uint32_t key[kN];  // state of the chunk's first block (before tempering)
  int32_t w0;        // first word of the segment, offset in the chunk
  uint32_t i0;       // the step that word is tested for
  void *round;       // the round whose draws it writes
};

// The tempered words of the chunk whose first block has state key0.
__attribute__((target("avx512f"))) void gen_chunk(const uint32_t *key0, uint32_t *out) {
  alignas(64) uint32_t k[kN];
  std::memcpy(k, key0, sizeof(k));
  for (int b = 0; b < kChunkBlocks; ++b, out += kN) {
    if (b > 0) twist_avx512(k);
    temper_avx512(k, out);
  }
}

// Windows never reach below this step (a transfer function must not hold
// the round's end, where the words go on to the feature shuffle).
constexpr uint32_t kSpecMin = 4096;
constexpr int32_t kMaxMerges = 4096;

// Transfer function of one chunk over the entry window [lo, hi]: entry e
// leaves the chunk at a_exit + g(e), g(e) = (e - lo) lowered by one for
// every merge m (in order) below it.
struct ChunkFn {
  std::atomic<int32_t> state{0};  // 0 pending, 1 ready, 2 not available (count word by word)
  uint32_t lo = 0, hi = 0, a_exit = 0;
  int32_t nm = 0;
  std::vector<uint32_t> m;  // lower group of each merge, in order
};

inline uint32_t chunk_exit(const ChunkFn &f, uint32_t e) {
  uint32_t g = e - f.lo;
  for (int32_t t = 0; t < f.nm; ++t) g -= g > f.m[t] ? 1u : 0u;
  return f.a_exit + g;
}

// The transfer function of a whole chunk of words over [lo, hi]; false if
// the window crosses a mask range, comes within kSpecMin of the round's end
// or merges more than kMaxMerges times.
__attribute__((target("avx512f,avx512vl,avx512bw,popcnt")))
bool spec_chunk_avx512(const uint32_t *words, uint32_t lo, uint32_t hi, ChunkFn &f) {
  uint32_t a = lo, b = hi;
  int32_t nm = 0;
  f.m.clear();
  const uint32_t *p = words, *const e = words + kChunkWords;
  while (p < e) {
    if (a < kSpecMin) return false;
    const int k = 31 - __builtin_clz(a);
    if (31 - __builtin_clz(b) != k) return false;
    const uint32_t lo_pow = 1u << k;
    const uint32_t mask = lo_pow | (lo_pow - 1);
    const __m512i vm = _mm512_set1_epi32((int)mask);
    // 64 words with none in (a - 63, b]: each is accepted by every
    // trajectory (v <= a - 63 <= the lowest one's step) or by none (v > b).
    while (a - lo_pow >= 64 && e - p >= 64) {
      const __m512i sa = _mm512_set1_epi32((int)(a - 63));
      const __m512i sb = _mm512_set1_epi32((int)b);
      const __m512i v0 = _mm512_and_si512(_mm512_loadu_si512(p), vm);
      const __m512i v1 = _mm512_and_si512(_mm512_loadu_si512(p + 16), vm);
      const __m512i v2 = _mm512_and_si512(_mm512_loadu_si512(p + 32), vm);
      const __m512i v3 = _mm512_and_si512(_mm512_loadu_si512(p + 48), vm);
      const __mmask16 amb =
          _mm512_mask_cmple_epu32_mask(_mm512_cmpgt_epu32_mask(v0, sa), v0, sb) |
          _mm512_mask_cmple_epu32_mask(_mm512_cmpgt_epu32_mask(v1, sa), v1, sb) |
          _mm512_mask_cmple_epu32_mask(_mm512_cmpgt_epu32_mask(v2, sa), v2, sb) |
          _mm512_mask_cmple_epu32_mask(_mm512_cmpgt_epu32_mask(v3, sa), v3, sb);
      if (amb) break;
      const uint64_t all = (uint64_t)_mm512_cmple_epu32_mask(v0, sa) |
                           ((uint64_t)_mm512_cmple_epu32_mask(v1, sa) << 16) |
                           ((uint64_t)_mm512_cmple_epu32_mask(v2, sa) << 32) |
                           ((uint64_t)_mm512_cmple_epu32_mask(v3, sa) << 48);
      const uint32_t c = (uint32_t)__builtin_popcountll(all);
      a -= c;
      b -= c;
      p += 64;
    }
    while (a - lo_pow >= 16 && e - p >= 16) {
      const __m512i sa = _mm512_set1_epi32((int)(a - 15));
      const __m512i v = _mm512_and_si512(_mm512_loadu_si512(p), vm);
      const __mmask16 amb = _mm512_mask_cmple_epu32_mask(_mm512_cmpgt_epu32_mask(v, sa), v,
                                                         _mm512_set1_epi32((int)b));
      if (amb) break;
      const uint32_t c = (uint32_t)__builtin_popcount((unsigned)_mm512_cmple_epu32_mask(v, sa));
      a -= c;
      b -= c;
      p += 16;
    }
    if (p < e) {
      const uint32_t v = *p++ & mask;
      if (v <= a) {
        --a;
        --b;
      } else if (v <= b) {
        if (nm == kMaxMerges) return false;
        f.m.push_back(v - 1 - a);
        ++nm;
        --b;
      }
    }
  }
  f.lo = lo;
  f.hi = hi;
  f.a_exit = a;
  f.nm = nm;
  return true;
}

// Expected step after o words of a shuffle that starts at step n - 1: step
// s takes (mask + 1) / (s + 1) words on average, so within one mask range
// (all-ones mask M - 1) the step after w words from step i is about
// (i + 1) exp(-w / M) - 1, and the range is left after M ln((i + 1) / lo)
// words (lo = M / 2).  at() takes increasing offsets, so a round's chunks
// walk the mask ranges once.
struct ExpectedSteps {
  double i, o0 = 0.0, M = 0.0, wr = 0.0;  // range entered at offset o0 with step i
  explicit ExpectedSteps(int64_t n) : i((double)(n - 1)) { enter(); }
  void enter() {
    if (i < 1.0) return;
    const int k = 63 - __builtin_clzll((uint64_t)i);
    const double lo = std::ldexp(1.0, k);
    M = 2.0 * lo;
    wr = M * std::log((i + 1.0) / lo);
  }
  double at(double o) {  // o must not decrease between calls
    while (i >= 1.0) {
      if (o - o0 <= wr) return (i + 1.0) * std::exp(-(o - o0) / M) - 1.0;
      o0 += wr;
      i = std::ldexp(1.0, 63 - __builtin_clzll((uint64_t)i)) - 1.0;
      enter();
    }
    return 0.0;
  }
};

// Expected words of a shuffle of n entries (steps n - 1 .. 1).
double expected_words(int64_t n) {
  double i = (double)(n - 1), w = 0.0;
  while (i >= 1.0) {
    const int k = 63 - __builtin_clzll((uint64_t)i);
    const double lo = std::ldexp(1.0, k);
    w += 2.0 * lo * std::log((i + 1.0) / lo);
    i = lo - 1.0;
  }
  return w;
}

// Counting form of write_segment_avx512: from word w0 at step i0 to the
// chunk's end or the round's last step; returns the offset just past the
// last word read and the step reached (0 when the round ended).
__attribute__((target("avx512f,avx512vl,avx512bw,popcnt")))
int64_t count_segment_avx512(const uint32_t *words, int64_t w0, uint32_t i0, uint32_t &i_out) {
  const uint32_t *p = words + w0, *const e = words + kChunkWords;
  uint32_t i = i0;
  while (i >= 1 && p < e) {
    const uint32_t lo = 1u << (31 - __builtin_clz(i));
    const uint32_t mask = lo | (lo - 1);
    const __m512i vm = _mm512_set1_epi32((int)mask);
    while (i >= lo && p < e) {
      while (i - lo >= 64 && e - p >= 64) {
        const __m512i si = _mm512_set1_epi32((int)i);
        const __m512i sb = _mm512_set1_epi32((int)(i - 62));
        const __m512i v0 = _mm512_and_si512(_mm512_loadu_si512(p), vm);
        const __m512i v1 = _mm512_and_si512(_mm512_loadu_si512(p + 16), vm);
        const __m512i v2 = _mm512_and_si512(_mm512_loadu_si512(p + 32), vm);
        const __m512i v3 = _mm512_and_si512(_mm512_loadu_si512(p + 48), vm);
        const __mmask16 a0 = _mm512_cmple_epu32_mask(v0, si);
        const __mmask16 a1 = _mm512_cmple_epu32_mask(v1, si);
        const __mmask16 a2 = _mm512_cmple_epu32_mask(v2, si);
        const __mmask16 a3 = _mm512_cmple_epu32_mask(v3, si);
        const __mmask16 amb = _mm512_mask_cmpge_epu32_mask(a0, v0, sb) |
                              _mm512_mask_cmpge_epu32_mask(a1, v1, sb) |
                              _mm512_mask_cmpge_epu32_mask(a2, v2, sb) |
                              _mm512_mask_cmpge_epu32_mask(a3, v3, sb);
        if (amb) break;
        const uint64_t all = (uint64_t)a0 | ((uint64_t)a1 << 16) | ((uint64_t)a2 << 32) |
                             ((uint64_t)a3 << 48);
        i -= (uint32_t)__builtin_popcountll(all);
        p += 64;
      }
      while (i - lo >= 16 && e - p >= 16) {
        const __m512i v = _mm512_and_si512(_mm512_loadu_si512(p), vm);
        const __mmask16 acc = _mm512_cmple_epu32_mask(v, _mm512_set1_epi32((int)i));
        const __mmask16 amb = _mm512_mask_cmpge_epu32_mask(acc, v, _mm512_set1_epi32((int)(i - 14)));
        if (amb) break;
        i -= (uint32_t)__builtin_popcount((unsigned)acc);
        p += 16;
      }
      if (p < e) {
        const uint32_t v = *p++ & mask;
        i -= v <= i ? 1u : 0u;
      }
    }
  }
  i_out = i;
  return p - words;
}

// A segment's draws: from word w0 of the chunk `words` at step i0 to the
// chunk's end or step 1, written to out[hi - i].  Same tests as the
// counting pass; only accepted lanes are stored.
__attribute__((target("avx512f,avx512vl,avx512bw,popcnt")))
void write_segment_avx512(const uint32_t *words, int32_t w0, uint32_t i0, uint32_t hi,
                          uint32_t *draws) {
  const uint32_t *p = words + w0, *const e = words + kChunkWords;
  uint32_t i = i0;
  uint32_t *out = draws + (hi - i0);
  while (i >= 1 && p < e) {
    const uint32_t lo = 1u << (31 - __builtin_clz(i));
    const uint32_t mask = lo | (lo - 1);
    const __m512i vm = _mm512_set1_epi32((int)mask);
    while (i >= lo && p < e) {
      while (i - lo >= 64 && e - p >= 64) {
        const __m512i si = _mm512_set1_epi32((int)i);
        const __m512i sb = _mm512_set1_epi32((int)(i - 62));
        const __m512i v0 = _mm512_and_si512(_mm512_loadu_si512(p), vm);
        const __m512i v1 = _mm512_and_si512(_mm512_loadu_si512(p + 16), vm);
        const __m512i v2 = _mm512_and_si512(_mm512_loadu_si512(p + 32), vm);
        const __m512i v3 = _mm512_and_si512(_mm512_loadu_si512(p + 48), vm);
        const __mmask16 a0 = _mm512_cmple_epu32_mask(v0, si);
        const __mmask16 a1 = _mm512_cmple_epu32_mask(v1, si);
        const __mmask16 a2 = _mm512_cmple_epu32_mask(v2, si);
        const __mmask16 a3 = _mm512_cmple_epu32_mask(v3, si);
        const __mmask16 amb = _mm512_mask_cmpge_epu32_mask(a0, v0, sb) |
                              _mm512_mask_cmpge_epu32_mask(a1, v1, sb) |
                              _mm512_mask_cmpge_epu32_mask(a2, v2, sb) |
                              _mm512_mask_cmpge_epu32_mask(a3, v3, sb);
        if (amb) break;
        const uint32_t c0 = (uint32_t)__builtin_popcount((unsigned)a0);
        const uint32_t c1 = (uint32_t)__builtin_popcount((unsigned)a1);
        const uint32_t c2 = (uint32_t)__builtin_popcount((unsigned)a2);
        const uint32_t c3 = (uint32_t)__builtin_popcount((unsigned)a3);
        _mm512_mask_storeu_epi32(out, (__mmask16)((1u << c0) - 1u), _mm512_maskz_compress_epi32(a0, v0));
        out += c0;
        _mm512_mask_storeu_epi32(out, (__mmask16)((1u << c1) - 1u), _mm512_maskz_compress_epi32(a1, v1));
        out += c1;
        _mm512_mask_storeu_epi32(out, (__mmask16)((1u << c2) - 1u), _mm512_maskz_compress_epi32(a2, v2));
        out += c2;
        _mm512_mask_storeu_epi32(out, (__mmask16)((1u << c3) - 1u), _mm512_maskz_compress_epi32(a3, v3));
        out += c3;
        i -= c0 + c1 + c2 + c3;
        p += 64;
      }
      while (i - lo >= 16 && e - p >= 16) {
        const __m512i v = _mm512_and_si512(_mm512_loadu_si512(p), vm);
        const __mmask16 acc = _mm512_cmple_epu32_mask(v, _mm512_set1_epi32((int)i));
        const __mmask16 amb = _mm512_mask_cmpge_epu32_mask(acc, v, _mm512_set1_epi32((int)(i - 14)));
        if (amb) break;
        const uint32_t c = (uint32_t)__builtin_popcount((unsigned)acc);
        _mm512_mask_storeu_epi32(out, (__mmask16)((1u << c) - 1u), _mm512_maskz_compress_epi32(acc, v));
        out += c;
        i -= c;
        p += 16;
      }
      if (p < e) {
        const uint32_t v = *p++ & mask;
        if (v <= i) {
          *out++ = v;
          --i;
        }
      }
    }
  }
}

bool draw_steps(Stream &s, uint32_t hi, uint32_t *out) {
  if (hi == 0) return true;
  return use_avx512() ? draw_steps_avx512(s, hi, out) : draw_steps_scalar(s, hi, out);
}

// Device copies of the draws outlive their sampler: the process's next
// sampler on the same GPU takes them.  A fit makes one sampler, and a
// hipMalloc and hipEventCreate per round buffer, with their frees at the
// end, cost its first rounds about a millisecond each.  One list per
// process (a child made by fork() starts an empty one).
struct DrawsBuf {
  int device;
  size_t bytes;
  uint32_t *p;
  hipEvent_t ev;
};
std::mutex &g_draws_mu = *new std::mutex;  // (never destroyed, as g_pinned)
std::vector<DrawsBuf> &g_draws = *new std::vector<DrawsBuf>;
pid_t g_draws_pid = 0;
constexpr size_t kDrawsKept = 16;

// The smallest kept buffer of `device` holding `bytes`; false if none.
bool take_kept_draws(int device, size_t bytes, DrawsBuf *out) {
  std::lock_guard<std::mutex> lk(g_draws_mu);
  if (g_draws_pid != getpid()) {  // (the parent's buffers are not this process's)
    g_draws.clear();
    g_draws_pid = getpid();
  }
  size_t best = g_draws.size();
  for (size_t i = 0; i < g_draws.size(); ++i)
    if (g_draws[i].device == device && g_draws[i].bytes >= bytes &&
        (best == g_draws.size() || g_draws[i].bytes < g_draws[best].bytes))
      best = i;
  if (best == g_draws.size()) return false;
  *out = g_draws[best];
  g_draws.erase(g_draws.begin() + (std::ptrdiff_t)best);
  return true;
}

// Keeps an idle buffer (no copy or kernel uses it any more) for a later
// sampler, or frees it when enough are kept.
void keep_draws(const DrawsBuf &b) {
  {
    std::lock_guard<std::mutex> lk(g_draws_mu);
    if (g_draws_pid != getpid()) {
      g_draws.clear();
      g_draws_pid = getpid();
    }
    if (g_draws.size() < kDrawsKept) {
      g_draws.push_back(b);
      return;
    }
  }
  if (b.p) (void)hipFree(b.p);
  if (b.ev) (void)hipEventDestroy(b.ev);
}

}  // namespace

struct Sampler {
  int64_t n = 0, n_sub = 0;
  int32_t F = 0, f_sub = 0;
  bool do_rows = false, do_feats = false, device_rows = false;
  int32_t n_rounds = 0, lookahead = 2;
  uint32_t key0[kN];
  int pos0 = 0;

  struct Round {
    HostBuf<uint32_t> draws;     // j(i) of steps n-1 .. 1
    uint32_t *draws_d = nullptr; // device copy (device-rows mode)
    size_t draws_d_bytes = 0;
    hipEvent_t copied = nullptr; // recorded after the copy on copy_st
    HostBuf<int32_t> rows;       // sample_idx (host mode)
    std::vector<int32_t> feats;  // ascending selected features
    int32_t index = 0;
    std::atomic<int32_t> pending{0};  // segments still being written, +1 while counting
    bool done = false;                // draws complete (and copied): deliverable
    bool on_device = false;           // draws_d holds this round's draws
  };
  int32_t device = -1;                // GPU of the device copies
  hipStream_t copy_st = nullptr;      // the process's copy stream (copy_stream)
  // Device-rows mode: rounds finished before the first take keep their
  // draws on the host, and the first take copies them; later rounds are
  // copied as soon as they are drawn.  A sampler made before its fit bins X
  // then draws its first rounds meanwhile, and allocates its device buffers
  // after the engine's.
  std::atomic<bool> device_go{false};

  std::atomic<bool> halt{false};     // makes the draw thread's stream stop
  std::atomic<double> gen_ms{0.0};   // word generation (inside draw_ms)
  std::deque<std::unique_ptr<Round>> inflight;  // counted, draws being written (in order)
  std::deque<std::unique_ptr<Round>> drawn;  // draw thread -> swap thread
  std::deque<std::unique_ptr<Round>> ready;  // -> consumer
  // Parallel draws (rounds of at least four chunks of steps, AVX-512):
  // chunk transfer functions and segments, both done by the worker threads.
  struct CountTask {
    int64_t chunk;
    uint32_t lo, hi;
    ChunkFn *out;
  };
  std::deque<CountTask> ctasks;
  int32_t count_running = 0;  // count tasks being worked on
  std::deque<Segment> segs;
  std::condition_variable seg_cv;
  int32_t idle_workers = 0;  // workers asleep on seg_cv
  std::vector<std::thread> workers;
  bool parallel = false;
  double window_scale = 1.0;  // entry windows: scale * (2.5 sqrt(words) + 64)
  std::unique_ptr<ChunkFn[]> fns;
  int64_t fns_cap = 0;
  // First-block states of the chunks [produced - cap, produced), made by the
  // twister thread, which stays fewer than ring_lead <= cap chunks ahead of
  // ring_floor (the draw thread's chunk).
  static constexpr int64_t kRingChunks = 4096;
  int64_t ring_lead = kRingChunks;
  std::vector<uint32_t> ring;
  std::atomic<int64_t> ring_produced{0};
  std::atomic<int64_t> ring_floor{0};
  std::mutex ring_mu;
  std::condition_variable ring_cv;
  std::thread twister;
  std::vector<std::unique_ptr<Round>> pool;
  int32_t n_drawn = 0, produced = 0, consumed = 0;
  bool stop = false;
  uint32_t final_key[kN];
  int final_pos = 0;
  std::mutex mu;
  std::condition_variable cv;
  std::thread draw_thread, swap_thread;
  std::string error;

  BigArray<int32_t> rows;      // cumulative row permutation (host mode)
  std::vector<int32_t> feats;  // cumulative feature permutation (draw thread)
  double draw_ms = 0.0, swap_ms = 0.0;
  int64_t spec_chunks = 0, seq_chunks = 0;  // parallel form: chunks by transfer function / word by word

  void fail(const char *msg) {
    {
      std::lock_guard<std::mutex> lk(mu);
      if (error.empty()) error = msg;
      stop = true;
    }
    set_halt();
    cv.notify_all();
    seg_cv.notify_all();
  }

  // halt and ring_floor change under ring_mu, so the twister cannot miss
  // the wake-up between its predicate check and its wait.
  void set_halt() {
    {
      std::lock_guard<std::mutex> lk(ring_mu);
      halt.store(true);
    }
    ring_cv.notify_all();
  }

  // Device-rows mode: the round's draws go to the GPU on the sampler's own
  // stream, so the copy overlaps the engine's work on the previous round.
  bool copy_to_device(Round &R) {
    if (!copy_st || hipSetDevice(device) != hipSuccess) {
      fail("sampler: no copy stream");
      return false;
    }
    if (!R.draws_d) {
      DrawsBuf kept;
      if (take_kept_draws(device, (size_t)n * 4, &kept)) {
        R.draws_d = kept.p;
        R.draws_d_bytes = kept.bytes;
        R.copied = kept.ev;
      } else if (hipMalloc(reinterpret_cast<void **>(&R.draws_d), (size_t)n * 4) != hipSuccess) {
        R.draws_d = nullptr;
        fail("sampler: hipMalloc of the draws failed");
        return false;
      } else {
        R.draws_d_bytes = (size_t)n * 4;
      }
    }
    if (!R.copied && hipEventCreateWithFlags(&R.copied, hipEventDisableTiming) != hipSuccess) {
      R.copied = nullptr;
      fail("sampler: hipEventCreate failed");
      return false;
    }
    if (n > 1 && hipMemcpyAsync(R.draws_d, R.draws.p, (size_t)(n - 1) * 4, hipMemcpyHostToDevice,
                                copy_st) != hipSuccess) {
      fail("sampler: draws copy failed");
      return false;
    }
    if (hipEventRecord(R.copied, copy_st) != hipSuccess) {
      fail("sampler: hipEventRecord failed");
      return false;
    }
    R.on_device = true;
    return true;
  }

  // (Called after copy_st is drained, when no round of this sampler is in
  // use on the device.)
  void free_device(Round &R) {
    if (R.draws_d)
      keep_draws(DrawsBuf{device, R.draws_d_bytes, R.draws_d, R.copied});
    else if (R.copied)
      (void)hipEventDestroy(R.copied);
    R.draws_d = nullptr;
    R.draws_d_bytes = 0;
    R.copied = nullptr;
  }

  // The round's draws are complete: copy them to the device (device-rows
  // mode), then hand every complete round at the head of `inflight` on, in
  // round order.
  void finalize(Round *R) {
    if (device_rows && do_rows && device_go.load(std::memory_order_acquire) &&
        !copy_to_device(*R))
      return;
    {
      std::lock_guard<std::mutex> lk(mu);
      R->done = true;
      while (!inflight.empty() && inflight.front()->done) {
        std::unique_ptr<Round> q = std::move(inflight.front());
        inflight.pop_front();
        if (device_rows || !do_rows) {
          ready.push_back(std::move(q));
          ++produced;
        } else {
          drawn.push_back(std::move(q));
        }
      }
    }
    cv.notify_all();
  }

  void release(Round *R) {
    if (R->pending.fetch_sub(1, std::memory_order_acq_rel) == 1) finalize(R);
  }

  void run_worker() {
    (void)pthread_setname_np(pthread_self(), "bsscl-drawseg");
    try {
      if (device_rows && do_rows && hipSetDevice(device) != hipSuccess) {
        fail("sampler: hipSetDevice failed");
        return;
      }
      std::vector<uint32_t> words((size_t)kChunkWords + 16);
      for (;;) {
        Segment sg;
        CountTask ct{-1, 0, 0, nullptr};
        {
          std::unique_lock<std::mutex> lk(mu);
          if (!stop && segs.empty() && ctasks.empty()) {
            ++idle_workers;
            seg_cv.wait(lk, [&] { return stop || !segs.empty() || !ctasks.empty(); });
            --idle_workers;
          }
          if (stop) return;
          if (!ctasks.empty()) {  // transfer functions first: the draw thread waits on them
            ct = ctasks.front();
            ctasks.pop_front();
            ++count_running;
          } else {
            sg = segs.front();
            segs.pop_front();
          }
        }
        if (ct.out) {
          bool ok = wait_key(ct.chunk);
          if (ok) {
            gen_chunk(ring_key(ct.chunk), words.data());
            ok = spec_chunk_avx512(words.data(), ct.lo, ct.hi, *ct.out);
          }
          ct.out->state.store(ok ? 1 : 2, std::memory_order_release);
          std::lock_guard<std::mutex> lk(mu);
          --count_running;
          continue;
        }
        Round *R = static_cast<Round *>(sg.round);
        gen_chunk(sg.key, words.data());
        write_segment_avx512(words.data(), sg.w0, sg.i0, (uint32_t)(n - 1), R->draws.p);
        release(R);
      }
    } catch (...) {
      fail("sampler: draw worker failed (out of memory?)");
    }
  }

  const uint32_t *ring_key(int64_t c) const {
    return ring.data() + (size_t)(c % kRingChunks) * kN;
  }

  // Waits until chunk c's first-block state exists; false if stopping.
  bool wait_key(int64_t c) {
    for (int spin = 0; ring_produced.load(std::memory_order_acquire) <= c; ++spin) {
      if (halt.load(std::memory_order_relaxed)) return false;
      if (spin < 4096) {
        _mm_pause();
      } else {
        std::unique_lock<std::mutex> lk(ring_mu);
        ring_cv.wait_for(lk, std::chrono::microseconds(200), [&] {
          return halt.load(std::memory_order_relaxed) ||
                 ring_produced.load(std::memory_order_acquire) > c;
        });
      }
    }
    return true;
  }

  // The floor moves in steps of kFloorStep chunks: each move takes ring_mu
  // and wakes the twister, and a floor that lags only holds the twister
  // back (ring_lead is at least 64 chunks).
  static constexpr int64_t kFloorStep = 16;
  void set_floor(int64_t c) {
    if (ring_floor.load(std::memory_order_relaxed) + kFloorStep > c) return;
    {
      std::lock_guard<std::mutex> lk(ring_mu);
      ring_floor.store(c, std::memory_order_release);
    }
    ring_cv.notify_all();
  }

  // Twists the stream ahead of its readers, chunk after chunk (the states
  // do not depend on how the words are used).
  void run_twister() {
    (void)pthread_setname_np(pthread_self(), "bsscl-twist");
    alignas(64) uint32_t k[kN];
    std::memcpy(k, key0, sizeof(k));
    for (int64_t c = 0;; ++c) {
      if (c > 0) {
        const auto t0 = std::chrono::steady_clock::now();
        for (int b = 0; b < kChunkBlocks; ++b) twist_avx512(k);
        gen_ms.store(gen_ms.load(std::memory_order_relaxed) +
                         std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count(),
                     std::memory_order_relaxed);
      }
      if (c >= ring_floor.load(std::memory_order_acquire) + ring_lead) {
        std::unique_lock<std::mutex> lk(ring_mu);
        ring_cv.wait(lk, [&] {
          return halt.load(std::memory_order_relaxed) ||
                 c < ring_floor.load(std::memory_order_acquire) + ring_lead;
        });
      }
      if (halt.load(std::memory_order_relaxed)) return;
      std::memcpy(ring.data() + (size_t)(c % kRingChunks) * kN, k, sizeof(k));
      ring_produced.store(c + 1, std::memory_order_release);
      ring_cv.notify_all();
    }
  }

  static constexpr size_t kSegBatch = 16;
  // Waits for a transfer function; 0 if the sampler stops.
  int32_t wait_fn(const ChunkFn &f) {
    for (int spin = 0;; ++spin) {
      const int32_t st = f.state.load(std::memory_order_acquire);
      if (st != 0) return st;
      if (halt.load(std::memory_order_relaxed)) return 0;
      if (spin < 4096) _mm_pause();
      else std::this_thread::yield();
    }
  }

  // The row steps of one round from global word G, as segments for the
  // workers (emit); returns the global word after the round's last step, or
  // -1 if the sampler stops.
  template <class Emit>
  int64_t resolve_round(int64_t G, Emit &&emit, std::vector<uint32_t> &words) {
    const int64_t c0 = G / kChunkWords;
    // Transfer functions of the chunks after the first, each around its
    // expected entry step, while the window stays above kSpecMin.
    int64_t nt = 0;
    {
      std::vector<CountTask> tl;
      ExpectedSteps es(n);
      for (int64_t c = c0 + 1;; ++c) {
        const double o = (double)(c * kChunkWords - G);
        const double e = es.at(o);
        const double h = window_scale * (2.5 * std::sqrt(o) + 64.0);
        if (e - h < (double)kSpecMin) break;
        const double hi = std::min(e + h, (double)(n - 1));
        tl.push_back({c, (uint32_t)(e - h), (uint32_t)hi, nullptr});
      }
      nt = (int64_t)tl.size();
      if (nt > fns_cap) {
        fns.reset(new ChunkFn[(size_t)nt]);
        fns_cap = nt;
      }
      for (int64_t t = 0; t < nt; ++t) {
        fns[(size_t)t].state.store(0, std::memory_order_relaxed);
        tl[(size_t)t].out = &fns[(size_t)t];
      }
      if (nt) {
        {
          std::lock_guard<std::mutex> lk(mu);
          for (const CountTask &t : tl) ctasks.push_back(t);
        }
        seg_cv.notify_all();
      }
    }
    uint32_t i = (uint32_t)(n - 1);
    int64_t c = c0, w = G - c0 * kChunkWords, end = -1, n_spec = 0, n_seq = 0;
    while (end < 0) {
      set_floor(c - 1);  // (the state of the word before a chunk's first stays readable)
      if (!wait_key(c)) break;
      const int64_t t = c - c0 - 1;
      if (t >= 0 && t < nt) {
        const ChunkFn &f = fns[(size_t)t];
        const int32_t st = wait_fn(f);
        if (st == 0) break;
        if (st == 1 && f.lo <= i && i <= f.hi) {
          ++n_spec;
          emit(ring_key(c), 0, i);
          i = chunk_exit(f, i);
          ++c;
          w = 0;
          continue;
        }
      }
      // Word by word: the round's first and last chunks, and any chunk
      // whose transfer function does not cover the entry step.
      ++n_seq;
      gen_chunk(ring_key(c), words.data());
      emit(ring_key(c), (int32_t)w, i);
      uint32_t i2 = 0;
      const int64_t pe = count_segment_avx512(words.data(), w, i, i2);
      i = i2;
      if (i == 0) end = c * kChunkWords + pe;
      ++c;
      w = 0;
    }
    // Transfer functions past the round's end are not needed.
    {
      std::unique_lock<std::mutex> lk(mu);
      spec_chunks += n_spec;
      seq_chunks += n_seq;
      ctasks.clear();
      while (count_running > 0 && !stop) {
        lk.unlock();
        std::this_thread::yield();
        lk.lock();
      }
    }
    return end;
  }

  // NumPy state after the words before global position G.
  void state_at(int64_t G, uint32_t *key_out, int *pos_out) {
    if (G <= pos0) {
      std::memcpy(key_out, key0, sizeof(uint32_t) * kN);
      *pos_out = pos0;
      return;
    }
    const int64_t b = (G - 1) / kN;
    const int64_t c = b / kChunkBlocks;
    alignas(64) uint32_t k[kN];
    if (!wait_key(c)) return;
    std::memcpy(k, ring_key(c), sizeof(k));
    for (int64_t t = c * kChunkBlocks; t < b; ++t) twist_scalar(k);
    std::memcpy(key_out, k, sizeof(k));
    *pos_out = (int)(G - b * kN);
  }

  // Draw loop of the parallel form.
  void run_draws_parallel() {
    std::vector<uint32_t> jf((size_t)F + 16);
    std::vector<Segment> sbatch;
    sbatch.reserve(kSegBatch);
    std::vector<uint32_t> words((size_t)kChunkWords + 16);
    int64_t G = pos0;  // global position of the next word
    for (int32_t r = 0; r < n_rounds; ++r) {
      std::unique_ptr<Round> R;
      {
        std::unique_lock<std::mutex> lk(mu);
        cv.wait(lk, [&] {
          return stop || (int32_t)(inflight.size() + drawn.size() + ready.size()) < lookahead;
        });
        if (stop) return;
        if (!pool.empty()) {
          R = std::move(pool.back());
          pool.pop_back();
        }
      }
      if (!R) R.reset(new Round());
      R->draws.alloc((size_t)n + 16);
      R->done = false;
      R->on_device = false;
      R->pending.store(1, std::memory_order_relaxed);  // this thread's share
      Round *Rp = R.get();
      {
        std::lock_guard<std::mutex> lk(mu);
        inflight.push_back(std::move(R));
      }
      const auto t0 = std::chrono::steady_clock::now();
      // Segments go to the workers kSegBatch at a time: one lock and at
      // most one wake-up (a system call) per batch.
      auto publish = [&] {
        if (sbatch.empty()) return;
        bool wake;
        {
          std::lock_guard<std::mutex> lk(mu);
          for (const Segment &sg : sbatch) segs.push_back(sg);
          wake = idle_workers > 0;
        }
        sbatch.clear();
        if (wake) seg_cv.notify_all();
      };
      auto emit = [&](const uint32_t *key, int32_t w0, uint32_t i) {
        sbatch.emplace_back();
        Segment &sg = sbatch.back();
        std::memcpy(sg.key, key, sizeof(sg.key));
        sg.w0 = w0;
        sg.i0 = i;
        sg.round = Rp;
        Rp->pending.fetch_add(1, std::memory_order_relaxed);
        if (sbatch.size() >= kSegBatch) publish();
      };
      const int64_t end = resolve_round(G, emit, words);
      publish();  // the round's last segments
      seg_cv.notify_all();
      if (end < 0) return;
      G = end;
      if (do_feats && F > 1) {
        Stream fs;
        const int64_t c = G / kChunkWords;
        if (!wait_key(c) || !fs.seek(c, G - c * kChunkWords, ring_key(c), &halt)) return;
        if (!draw_steps(fs, (uint32_t)(F - 1), jf.data())) return;
        for (int32_t t = 0; t < F - 1; ++t) std::swap(feats[(size_t)(F - 1 - t)], feats[jf[(size_t)t]]);
        G = fs.position();
      }
      Rp->feats.assign(feats.begin(), feats.begin() + f_sub);
      std::sort(Rp->feats.begin(), Rp->feats.end());
      Rp->index = r;
      const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
      uint32_t fk[kN];
      std::memcpy(fk, key0, sizeof(fk));
      int fp = pos0;
      const bool last = r + 1 == n_rounds;
      if (last) state_at(G, fk, &fp);
      {
        std::lock_guard<std::mutex> lk(mu);
        draw_ms += ms;
        ++n_drawn;
        if (last) {
          std::memcpy(final_key, fk, sizeof(fk));
          final_pos = fp;
        }
      }
      cv.notify_all();
      release(Rp);
    }
  }

  void run_draws() {
    (void)pthread_setname_np(pthread_self(), "bsscl-draw");
    try {
      if (device_rows && do_rows && hipSetDevice(device) != hipSuccess) {
        fail("sampler: hipSetDevice failed");
        return;
      }
      if (do_rows && parallel) {
        run_draws_parallel();
        return;
      }
      Stream st;
      if (!st.start(key0, pos0, &halt, &gen_ms)) return;
      std::vector<uint32_t> jf((size_t)F + 16);
      for (int32_t r = 0; r < n_rounds; ++r) {
        std::unique_ptr<Round> R;
        {
          std::unique_lock<std::mutex> lk(mu);
          cv.wait(lk, [&] {
            return stop ||
                   (int32_t)(inflight.size() + drawn.size() + ready.size()) < lookahead;
          });
          if (stop) return;
          if (!pool.empty()) {
            R = std::move(pool.back());
            pool.pop_back();
          }
        }
        if (!R) R.reset(new Round());
        if (do_rows) R->draws.alloc((size_t)n + 16);
        R->done = false;
        R->on_device = false;
        R->pending.store(1, std::memory_order_relaxed);  // this thread's share
        Round *Rp = R.get();
        {
          std::lock_guard<std::mutex> lk(mu);
          inflight.push_back(std::move(R));
        }
        const auto t0 = std::chrono::steady_clock::now();
        if (do_rows && !draw_steps(st, (uint32_t)(n - 1), Rp->draws.p)) {
          return;
        }
        if (do_feats && F > 1) {
          if (!draw_steps(st, (uint32_t)(F - 1), jf.data())) return;
          for (int32_t t = 0; t < F - 1; ++t) std::swap(feats[(size_t)(F - 1 - t)], feats[jf[(size_t)t]]);
        }
        Rp->feats.assign(feats.begin(), feats.begin() + f_sub);
        std::sort(Rp->feats.begin(), Rp->feats.end());
        Rp->index = r;
        const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        {
          std::lock_guard<std::mutex> lk(mu);
          draw_ms += ms;
          ++n_drawn;
          if (n_drawn == n_rounds) st.state(key0, pos0, final_key, &final_pos);
        }
        cv.notify_all();
        release(Rp);
      }
    } catch (...) {
      fail("sampler: draw thread failed (out of memory?)");
    }
  }

  // Host mode: Fisher-Yates swaps of each round on the row permutation.
  void run_swaps() {
    try {
      for (;;) {
        std::unique_ptr<Round> R;
        {
          std::unique_lock<std::mutex> lk(mu);
          cv.wait(lk, [&] { return stop || produced >= n_rounds || !drawn.empty(); });
          if (stop || produced >= n_rounds) return;
          R = std::move(drawn.front());
          drawn.pop_front();
        }
        const auto t0 = std::chrono::steady_clock::now();
        const uint32_t *j = R->draws.p;
        int32_t *a = rows.data();
        constexpr int64_t kAhead = 32;
        for (int64_t t = 0; t < n - 1; ++t) {
          if (t + kAhead < n - 1) __builtin_prefetch(a + j[t + kAhead], 1, 1);
          const int64_t i = n - 1 - t;
          const uint32_t ji = j[t];
          const int32_t v = a[ji];
          a[ji] = a[i];
          a[i] = v;
        }
        const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        R->rows.alloc((size_t)n_sub);
        std::memcpy(R->rows.p, a, (size_t)n_sub * sizeof(int32_t));
        {
          std::lock_guard<std::mutex> lk(mu);
          swap_ms += ms;
          ready.push_back(std::move(R));
          ++produced;
        }
        cv.notify_all();
      }
    } catch (...) {
      fail("sampler: swap thread failed (out of memory?)");
    }
  }

  // Blocks until the next round is ready; the caller returns it with give().
  Round *take() {
    std::unique_lock<std::mutex> lk(mu);
    if (consumed >= n_rounds) return nullptr;
    cv.wait(lk, [&] { return stop || !ready.empty(); });
    if (ready.empty()) return nullptr;
    Round *r = ready.front().release();
    ready.pop_front();
    ++consumed;
    lk.unlock();
    cv.notify_all();
    return r;
  }

  void give(Round *r) {
    {
      std::lock_guard<std::mutex> lk(mu);
      pool.emplace_back(r);
    }
    cv.notify_all();
  }

  ~Sampler() {
    {
      std::lock_guard<std::mutex> lk(mu);
      stop = true;
    }
    cv.notify_all();
    seg_cv.notify_all();
    set_halt();
    if (draw_thread.joinable()) draw_thread.join();
    if (twister.joinable()) twister.join();
    for (auto &w : workers)
      if (w.joinable()) w.join();
    if (swap_thread.joinable()) swap_thread.join();
    if (copy_st) {
      (void)hipSetDevice(device);
      (void)hipStreamSynchronize(copy_st);
      for (auto &r : ready) free_device(*r);
      for (auto &r : pool) free_device(*r);
      for (auto &r : inflight) free_device(*r);
      // (copy_st is the process's copy stream: it stays.)
    }
  }
};

int sampler_take(bsscl_sampler *hs, SamplerRound *out, void **token) {
  Sampler *s = reinterpret_cast<Sampler *>(hs);
  if (!s || !out || !token) return set_error(BSSCL_EINVAL, "sampler: null argument");
  if (s->device_rows && s->do_rows) s->device_go.store(true, std::memory_order_release);
  Sampler::Round *r = s->take();
  if (!r) {
    std::lock_guard<std::mutex> lk(s->mu);
    return set_error(BSSCL_EINVAL, s->error.empty() ? "sampler: all rounds consumed" : s->error);
  }
  // A round drawn before the first take is copied by the taker.
  if (s->device_rows && s->do_rows && !r->on_device && !s->copy_to_device(*r)) {
    s->give(r);
    std::lock_guard<std::mutex> lk(s->mu);
    return set_error(BSSCL_EDEVICE, s->error.empty() ? "sampler: draws copy failed" : s->error);
  }
  out->draws = s->do_rows ? r->draws.p : nullptr;
  out->draws_dev = (s->do_rows && s->device_rows) ? r->draws_d : nullptr;
  out->draws_copied = (s->do_rows && s->device_rows) ? r->copied : nullptr;
  out->rows = (s->do_rows && !s->device_rows) ? r->rows.p : nullptr;
  out->feats = r->feats.data();
  out->round = r->index;
  *token = r;
  return BSSCL_OK;
}

void sampler_give_back(bsscl_sampler *hs, void *token) {
  Sampler *s = reinterpret_cast<Sampler *>(hs);
  auto *r = static_cast<Sampler::Round *>(token);
  if (!s || !r) return;
  s->give(r);
}

int32_t sampler_remaining(bsscl_sampler *hs) {
  Sampler *s = reinterpret_cast<Sampler *>(hs);
  std::lock_guard<std::mutex> lk(s->mu);
  return s->n_rounds - s->consumed;
}

SamplerShape sampler_shape(bsscl_sampler *hs) {
  const Sampler *s = reinterpret_cast<const Sampler *>(hs);
  SamplerShape sh;
  sh.n = s->n;
  sh.n_sub = s->n_sub;
  sh.f_sub = s->f_sub;
  sh.do_rows = s->do_rows;
  sh.device_rows = s->device_rows;
  sh.device = s->device;
  return sh;
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

int bsscl_rs_draws(uint32_t *key, int32_t *pos, uint32_t *draws_out, int64_t n) {
  if (!key || !pos || (n > 1 && !draws_out) || *pos < 0 || *pos > 624 || n < 0 ||
      n > INT32_MAX)
    return bsscl::set_error(BSSCL_EINVAL, "rs_draws: bad state, buffer or length");
  bsscl::MT mt;
  mt.load(key, *pos);
  for (int64_t i = n - 1; i >= 1; --i) draws_out[n - 1 - i] = (uint32_t)mt.interval((uint64_t)i);
  std::memcpy(key, mt.key, sizeof(mt.key));
  *pos = mt.pos;
  return BSSCL_OK;
}

int bsscl_sampler_create(const uint32_t *key, int32_t pos, int64_t n,
                         int64_t n_sub, int32_t do_rows, int32_t n_features,
                         int32_t f_sub, int32_t do_feats, int32_t n_rounds,
                         int32_t lookahead, int32_t flags, int32_t device,
                         bsscl_sampler **out) {
  if (!key || !out || pos < 0 || pos > 624 || n <= 0 || n > INT32_MAX ||
      n_sub <= 0 || n_sub > n || n_features <= 0 || f_sub <= 0 ||
      f_sub > n_features || n_rounds < 0 || lookahead < 1 ||
      (flags & ~BSSCL_SAMPLER_DEVICE_ROWS) != 0)
    return bsscl::set_error(BSSCL_EINVAL, "sampler_create: bad arguments");
  if (!do_rows && n_sub != n)
    return bsscl::set_error(BSSCL_EINVAL,
                            "sampler_create: n_sub must equal n without row bagging");
  if (!do_feats && f_sub != n_features)
    return bsscl::set_error(BSSCL_EINVAL,
                            "sampler_create: f_sub must equal F without column bagging");
  Sampler *s = new (std::nothrow) Sampler();
  if (!s) return bsscl::set_error(BSSCL_ENOMEM, "sampler_create: out of memory");
  std::memcpy(s->key0, key, sizeof(s->key0));
  s->pos0 = pos;
  s->n = n;
  s->n_sub = n_sub;
  s->F = n_features;
  s->f_sub = f_sub;
  s->do_rows = do_rows != 0;
  s->do_feats = do_feats != 0;
  s->device_rows = (flags & BSSCL_SAMPLER_DEVICE_ROWS) != 0;
  s->device = device;
  if (s->device_rows && s->do_rows) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count) {
      delete s;
      return bsscl::set_error(BSSCL_EINVAL, "sampler_create: device-rows mode needs a valid HIP device");
    }
    s->copy_st = bsscl::copy_stream(device);
    if (!s->copy_st) {
      delete s;
      return bsscl::set_error(BSSCL_EDEVICE, "sampler_create: no copy stream");
    }
  }
  s->n_rounds = n_rounds;
  s->lookahead = lookahead;
  std::memcpy(s->final_key, key, sizeof(s->final_key));
  s->final_pos = pos;
  try {
    if (s->do_rows && !s->device_rows) {
      s->rows.alloc((size_t)n);
      for (int64_t i = 0; i < n; ++i) s->rows[(size_t)i] = (int32_t)i;
    }
    s->feats.resize((size_t)n_features);
    for (int32_t j = 0; j < n_features; ++j) s->feats[(size_t)j] = j;
    // Rounds of at least four chunks of steps split their draws over
    // worker threads (AVX-512 only; the scalar path stays sequential).
    s->parallel = s->do_rows && bsscl::use_avx512() && n - 1 >= 4 * bsscl::kChunkWords;
    if (s->parallel) {
      // (Test hook: BSSCL_SAMPLER_WINDOW scales the entry windows; 0 makes
      // almost every chunk miss its window and be counted word by word.)
      const char *ws = std::getenv("BSSCL_SAMPLER_WINDOW");
      if (ws && ws[0]) s->window_scale = std::max(0.0, std::atof(ws));
      s->ring.resize((size_t)Sampler::kRingChunks * bsscl::kN);
      // The twister stays about three rounds of words ahead.
      const double rc = bsscl::expected_words(n) / (double)bsscl::kChunkWords;
      s->ring_lead = std::min<int64_t>(Sampler::kRingChunks, (int64_t)(3.0 * rc) + 64);
      const unsigned hw = std::max(2u, std::thread::hardware_concurrency());
      int nw = (int)std::max(2u, std::min(8u, hw / 2));
      // (Test hook: BSSCL_SAMPLER_WORKERS sets the worker count, 1-32.)
      if (const char *wv = std::getenv("BSSCL_SAMPLER_WORKERS"))
        nw = std::max(1, std::min(32, std::atoi(wv)));
      for (int w = 0; w < nw; ++w) s->workers.emplace_back([s] { s->run_worker(); });
      s->twister = std::thread([s] { s->run_twister(); });
    }
    s->draw_thread = std::thread([s] { s->run_draws(); });
    if (s->do_rows && !s->device_rows) s->swap_thread = std::thread([s] { s->run_swaps(); });
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
  if (s->device_rows && s->do_rows)
    return bsscl::set_error(BSSCL_EINVAL,
                            "sampler_next: a device-rows sampler's rows exist only on the GPU");
  bsscl::SamplerRound r;
  void *token = nullptr;
  int rc = bsscl::sampler_take(hs, &r, &token);
  if (rc != BSSCL_OK) return rc;
  if (rows_out) {
    if (r.rows) {
      std::memcpy(rows_out, r.rows, (size_t)s->n_sub * sizeof(int32_t));
    } else {
      for (int64_t i = 0; i < s->n_sub; ++i) rows_out[i] = (int32_t)i;
    }
  }
  if (feats_out) std::memcpy(feats_out, r.feats, (size_t)s->f_sub * sizeof(int32_t));
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
  const double v[6] = {(double)s->produced, s->draw_ms, s->swap_ms,
                       s->gen_ms.load(std::memory_order_relaxed), (double)s->spec_chunks,
                       (double)s->seq_chunks};
  const int32_t k = std::max<int32_t>(0, std::min<int32_t>(cap, 6));
  for (int32_t i = 0; i < k; ++i) out[i] = v[i];
  *n_out = k;
  return BSSCL_OK;
}

void bsscl_sampler_destroy(bsscl_sampler *hs) {
  delete reinterpret_cast<Sampler *>(hs);
}

}  // extern "C"
