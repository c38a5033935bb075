// Wave-level scans and reductions for gfx950 (wave64) built on DPP row
// operations and v_readlane instead of ds_bpermute.  A DPP move stays in the
// VALU (a few cycles); a bpermute is an LDS round trip (about a hundred
// cycles), and a scan or reduction chains six of them.
//
// Every function here must be called by all 64 lanes of the wave (full EXEC,
// wave-uniform control flow).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace bsscl {

// DPP controls (GFX9 encoding).
constexpr int kDppQuadXor1 = 0xB1;      // quad_perm [1,0,3,2]: lane ^ 1
constexpr int kDppQuadXor2 = 0x4E;      // quad_perm [2,3,0,1]: lane ^ 2
constexpr int kDppRowShr = 0x110;       // + k: row_shr:k (lane - k within a row of 16)
constexpr int kDppRowMirror = 0x140;    // lane 15 - i within a row of 16
constexpr int kDppRowHalfMirror = 0x141;  // lane 7 - i within a half row of 8

// The value of lane (CTRL) as a 32-bit word; a source lane outside the row
// reads 0.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, true);
}

template <int CTRL, typename T>
__device__ __forceinline__ T dpp(T v) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit values");
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, dpp32<CTRL>(__builtin_bit_cast(uint32_t, v)));
  } else {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint64_t lo = dpp32<CTRL>((uint32_t)u);
    const uint64_t hi = dpp32<CTRL>((uint32_t)(u >> 32));
    return __builtin_bit_cast(T, lo | (hi << 32));
  }
}

// Lane `l` of v (l wave-uniform); the result is uniform.
template <typename T>
__device__ __forceinline__ T wave_lane(T v, int l) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit values");
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(
        T, (uint32_t)__builtin_amdgcn_readlane((int)__builtin_bit_cast(uint32_t, v), l));
  } else {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint64_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, l);
    const uint64_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), l);
    return __builtin_bit_cast(T, lo | (hi << 32));
  }
}

// Inclusive prefix sum over the wave's 64 lanes (integers: exact in any
// order).  Within each row of 16 lanes a Hillis-Steele scan of row shifts
// 1, 2, 4, 8; then each row adds the totals of the rows before it, read from
// lanes 15, 31 and 47.
template <typename T>
__device__ __forceinline__ T wave_incl_scan(T v) {
  static_assert(std::is_integral<T>::value, "integer scan");
  v += dpp<kDppRowShr + 1>(v);
  v += dpp<kDppRowShr + 2>(v);
  v += dpp<kDppRowShr + 4>(v);
  v += dpp<kDppRowShr + 8>(v);
  const T r0 = wave_lane(v, 15), r1 = wave_lane(v, 31), r2 = wave_lane(v, 47);
  const int row = (int)(threadIdx.x & 63) >> 4;
  const T add = (row >= 1 ? r0 : T(0)) + (row >= 2 ? r1 : T(0)) + (row >= 3 ? r2 : T(0));
  return v + add;
}

// Sum over the wave's 64 lanes, in every lane (integers).  The four steps
// leave each row of 16 lanes with its row's sum; the rows meet through
// lanes 0, 16, 32 and 48.
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
  static_assert(std::is_integral<T>::value, "integer sum");
  v += dpp<kDppQuadXor1>(v);
  v += dpp<kDppQuadXor2>(v);
  v += dpp<kDppRowHalfMirror>(v);
  v += dpp<kDppRowMirror>(v);
  return (wave_lane(v, 0) + wave_lane(v, 16)) + (wave_lane(v, 32) + wave_lane(v, 48));
}

// Best (value, index, aux) over the wave, in every lane: a candidate with
// index >= 0 beats one with index < 0, then the larger value wins, then the
// lower index.  Valid indices are distinct across lanes and every invalid
// lane holds the same triple, so the order of comparisons cannot change the
// result.
__device__ __forceinline__ void argmax_take(double &best, int32_t &idx, int32_t &aux, double ov,
                                            int32_t oi, int32_t oa) {
  const bool take = oi >= 0 && (idx < 0 || ov > best || (ov == best && oi < idx));
  best = take ? ov : best;
  idx = take ? oi : idx;
  aux = take ? oa : aux;
}

template <int CTRL>
__device__ __forceinline__ void argmax_step(double &best, int32_t &idx, int32_t &aux) {
  const double ov = dpp<CTRL>(best);
  const int32_t oi = dpp<CTRL>(idx);
  const int32_t oa = dpp<CTRL>(aux);
  argmax_take(best, idx, aux, ov, oi, oa);
}

__device__ __forceinline__ void wave_argmax(double &best, int32_t &idx, int32_t &aux) {
  argmax_step<kDppQuadXor1>(best, idx, aux);
  argmax_step<kDppQuadXor2>(best, idx, aux);
  argmax_step<kDppRowHalfMirror>(best, idx, aux);
  argmax_step<kDppRowMirror>(best, idx, aux);
  double b = wave_lane(best, 0);
  int32_t i = wave_lane(idx, 0), a = wave_lane(aux, 0);
#pragma unroll
  for (int r = 1; r < 4; ++r)
    argmax_take(b, i, a, wave_lane(best, 16 * r), wave_lane(idx, 16 * r), wave_lane(aux, 16 * r));
  best = b;
  idx = i;
  aux = a;
}

}  // namespace bsscl
