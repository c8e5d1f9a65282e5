// Wave64 reductions and scans over DPP lane moves (no LDS traffic), and
// ballot-based counting, for gfx950.
//
// DPP controls used: quad_perm [1,0,3,2] (0xB1) and [2,3,0,1] (0x4E),
// row_half_mirror (0x141), row_mirror (0x140), row_shr:n (0x110 + n),
// row_bcast:15 (0x142) and row_bcast:31 (0x143).  Full reductions combine the
// four 16-lane rows with readlane and return a wave-uniform value.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lps {

template <int CTRL, int ROWMASK = 0xF, bool BC = false>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t old, uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROWMASK, 0xF, BC);
}
template <int CTRL, int ROWMASK = 0xF, bool BC = false>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t old, uint64_t v) {
  const uint32_t lo = dpp_u32<CTRL, ROWMASK, BC>((uint32_t)old, (uint32_t)v);
  const uint32_t hi = dpp_u32<CTRL, ROWMASK, BC>((uint32_t)(old >> 32), (uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint32_t rdlane_u32(uint32_t v, int l) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, l);
}
__device__ __forceinline__ uint64_t rdlane_u64(uint64_t v, int l) {
  return ((uint64_t)rdlane_u32((uint32_t)(v >> 32), l) << 32) | rdlane_u32((uint32_t)v, l);
}

// XCD id of the executing wave: hardware register HW_REG_XCC_ID (20), bits 0-3.
__device__ __forceinline__ uint32_t xcc_id() {
  return (uint32_t)__builtin_amdgcn_s_getreg(20 | (0 << 6) | ((4 - 1) << 11)) & 0xFu;
}

struct OpAdd {
  template <typename T> __device__ __forceinline__ T operator()(T a, T b) const { return a + b; }
};
struct OpMax {
  template <typename T> __device__ __forceinline__ T operator()(T a, T b) const { return a > b ? a : b; }
};
struct OpMin {
  template <typename T> __device__ __forceinline__ T operator()(T a, T b) const { return a < b ? a : b; }
};
struct OpOr {
  template <typename T> __device__ __forceinline__ T operator()(T a, T b) const { return a | b; }
};

// Lane moves of any 4- or 8-byte type, bit for bit.
template <int CTRL, int ROWMASK = 0xF, bool BC = false, typename T>
__device__ __forceinline__ T dpp_t(T old, T v) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "4- or 8-byte lane values");
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, dpp_u32<CTRL, ROWMASK, BC>(__builtin_bit_cast(uint32_t, old),
                                                            __builtin_bit_cast(uint32_t, v)));
  } else {
    return __builtin_bit_cast(T, dpp_u64<CTRL, ROWMASK, BC>(__builtin_bit_cast(uint64_t, old),
                                                            __builtin_bit_cast(uint64_t, v)));
  }
}
template <typename T>
__device__ __forceinline__ T rdlane(T v, int l) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "4- or 8-byte lane values");
  if constexpr (sizeof(T) == 4) return __builtin_bit_cast(T, rdlane_u32(__builtin_bit_cast(uint32_t, v), l));
  else return __builtin_bit_cast(T, rdlane_u64(__builtin_bit_cast(uint64_t, v), l));
}

// Reduction over the 64 lanes; every lane gets the (wave-uniform) result.
template <typename T, typename Op>
__device__ __forceinline__ T wreduce(T v, Op op) {
  v = op(v, dpp_t<0xB1>(v, v));   // quad_perm [1,0,3,2]
  v = op(v, dpp_t<0x4E>(v, v));   // quad_perm [2,3,0,1]
  v = op(v, dpp_t<0x141>(v, v));  // row_half_mirror
  v = op(v, dpp_t<0x140>(v, v));  // row_mirror
  return op(op(rdlane(v, 0), rdlane(v, 16)), op(rdlane(v, 32), rdlane(v, 48)));
}
template <typename T> __device__ __forceinline__ T wsum(T v) { return wreduce(v, OpAdd{}); }
template <typename T> __device__ __forceinline__ T wmax(T v) { return wreduce(v, OpMax{}); }
template <typename T> __device__ __forceinline__ T wmin(T v) { return wreduce(v, OpMin{}); }

// Inclusive prefix sum over the 64 lanes (lane order): row_shr 1, 2, 4, 8 with
// zero fill, then row_bcast:15 into rows 1 and 3 and row_bcast:31 into rows 2, 3.
template <typename T>
__device__ __forceinline__ T wscan_incl(T v) {
  const T z = (T)0;
  v += dpp_t<0x111, 0xF, true>(z, v);
  v += dpp_t<0x112, 0xF, true>(z, v);
  v += dpp_t<0x114, 0xF, true>(z, v);
  v += dpp_t<0x118, 0xF, true>(z, v);
  v += dpp_t<0x142, 0xA, false>(z, v);
  v += dpp_t<0x143, 0xC, false>(z, v);
  return v;
}

// Reduction over lanes 0-15 (the first row; the other rows' values do not
// enter), in every lane.  With the other rows holding the identity it equals
// wreduce bit for bit (the same steps, then exact combines with the identity).
template <typename T, typename Op>
__device__ __forceinline__ T rreduce16(T v, Op op) {
  v = op(v, dpp_t<0xB1>(v, v));
  v = op(v, dpp_t<0x4E>(v, v));
  v = op(v, dpp_t<0x141>(v, v));
  v = op(v, dpp_t<0x140>(v, v));
  return rdlane(v, 0);
}
// Inclusive prefix sum within each row of 16 lanes.
template <typename T>
__device__ __forceinline__ T rscan16(T v) {
  const T z = (T)0;
  v += dpp_t<0x111, 0xF, true>(z, v);
  v += dpp_t<0x112, 0xF, true>(z, v);
  v += dpp_t<0x114, 0xF, true>(z, v);
  v += dpp_t<0x118, 0xF, true>(z, v);
  return v;
}

__device__ __forceinline__ uint64_t wballot(bool p) { return __ballot(p); }
// Set lanes of m below this lane.
__device__ __forceinline__ uint32_t lanes_below(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Largest t with #{values >= t} >= m over the wave (M values per lane,
// m >= 1, at least m values present): the m-th largest value of the wave.
// For m <= 16, by taking the wave's largest remaining value and its copies
// out until m are counted (at most m rounds); else a 32-step bit search.
template <int M>
__device__ __forceinline__ uint32_t wave_kth_largest(const uint32_t (&v)[M], uint32_t m) {
  if (m <= 16u) {
    uint32_t w[M];
#pragma unroll
    for (int i = 0; i < M; i++) w[i] = v[i];
    uint32_t need = m, t = 0;
#pragma unroll 1
    for (int it = 0; it < 16; it++) {
      uint32_t lm = w[0];
#pragma unroll
      for (int i = 1; i < M; i++) lm = w[i] > lm ? w[i] : lm;
      t = wreduce(lm, OpMax{});
      uint32_t n = 0;
#pragma unroll
      for (int i = 0; i < M; i++) n += (uint32_t)__builtin_popcountll(wballot(w[i] == t));
      if (n >= need || t == 0u) break;
      need -= n;
#pragma unroll
      for (int i = 0; i < M; i++) w[i] = w[i] == t ? 0u : w[i];
    }
    return t;
  }
  uint32_t t = 0;
#pragma unroll 1
  for (int b = 31; b >= 0; b--) {
    const uint32_t c = t | (1u << b);
    uint32_t n = 0;
#pragma unroll
    for (int i = 0; i < M; i++) n += (uint32_t)__builtin_popcountll(wballot(v[i] >= c));
    if (n >= m) t = c;
  }
  return t;
}

}  // namespace lps
