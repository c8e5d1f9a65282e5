// Shared device helpers for the lps sampler kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lps.h"

// Keeps x in a vector register, opaque to the optimiser (an empty asm with a
// VGPR operand).  A host build of the kernels for the bounds-checking test
// harness defines its own before this header.
#ifndef LPS_KEEP_VGPR
#define LPS_KEEP_VGPR(x) __asm__ volatile("" : "+v"(x))
#endif

namespace lps {

constexpr float kLog2e = 1.4426950408889634f;
// Softmax masses e = exp(z - z_max) lie in (0, 1]; they are accumulated as
// unsigned fixed point with this many fraction bits, so sums are exact and
// independent of the order of accumulation (V * 2^44 < 2^63 for V < 2^19).
constexpr int kMassBits = 44;
constexpr float kMassScale = 17592186044416.0f;  // 2^44
constexpr uint32_t kNoTie = 0xFFFFFFFFu;

// ---------------------------------------------------------------------------
// Element loads: bf16 / fp16 / fp32 -> fp32 (exact conversions).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)h);
}

// NTL: nontemporal (streamed once, not kept in the caches); false for data
// that is read again soon (the row softmax's second and third passes).
template <typename T, bool NTL>
__device__ __forceinline__ T ldg(const T* p) {
  if constexpr (NTL) return __builtin_nontemporal_load(p);
  else return *p;
}

template <int DT, bool NTL = true>
__device__ __forceinline__ float load1(const void* row, int64_t i) {
  if constexpr (DT == LPS_DTYPE_F32) {
    return ldg<float, NTL>(reinterpret_cast<const float*>(row) + i);
  } else {
    uint32_t h = ldg<unsigned short, NTL>(reinterpret_cast<const unsigned short*>(row) + i);
    return DT == LPS_DTYPE_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
  }
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Loads VEC consecutive elements starting at element i0 (i0 % VEC == 0) with
// one 16-byte load when VEC covers 16 bytes, else element loads.
template <int DT, int VEC, bool NTL = true>
__device__ __forceinline__ void loadv(const void* row, int64_t i0, float (&x)[VEC]) {
  if constexpr ((DT == LPS_DTYPE_F32 && VEC == 4) || (DT != LPS_DTYPE_F32 && VEC == 8)) {
    const u32x4* p = reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(row) +
                                                     i0 * (DT == LPS_DTYPE_F32 ? 4 : 2));
    u32x4 v = ldg<u32x4, NTL>(p);
    if constexpr (DT == LPS_DTYPE_F32) {
      x[0] = __uint_as_float(v.x); x[1] = __uint_as_float(v.y);
      x[2] = __uint_as_float(v.z); x[3] = __uint_as_float(v.w);
    } else {
      uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        if constexpr (DT == LPS_DTYPE_BF16) {
          x[2 * j] = bf16_to_f32(w[j] & 0xFFFFu);
          x[2 * j + 1] = bf16_to_f32(w[j] >> 16);
        } else {
          x[2 * j] = f16_to_f32(w[j] & 0xFFFFu);
          x[2 * j + 1] = f16_to_f32(w[j] >> 16);
        }
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < VEC; j++) x[j] = load1<DT, NTL>(row, i0 + j);
  }
}

// ---------------------------------------------------------------------------
// Order-preserving float keys.  Larger key = larger value; -0.0 and +0.0 share
// a key (they compare equal in torch); NaN ranks above +inf, as torch.argmax
// and torch.topk rank it.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t f2key(float f) {
  uint32_t b = __float_as_uint(f);
  if (b == 0x80000000u) b = 0u;
  uint32_t k = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return (f != f) ? 0xFFFFFFFFu : k;
}
__device__ __forceinline__ float key2f(uint32_t k) {
  uint32_t b = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
  return __uint_as_float(b);
}

// Penalised logit: CTRL repetition penalty (x > 0 ? x / r : x * r, once per
// distinct id), then the frequency and presence penalties, every step a
// correctly rounded fp32 operation (no FMA contraction).
__device__ __forceinline__ float penalize(float x, int cnt, float rep, float pres, float freq) {
  if (rep != 1.0f) x = x > 0.0f ? __fdiv_rn(x, rep) : __fmul_rn(x, rep);
  if (freq != 0.0f) x = __fsub_rn(x, __fmul_rn((float)cnt, freq));
  if (pres != 0.0f) x = __fsub_rn(x, pres);
  return x;
}

// Softmax mass of a scaled logit relative to the row maximum, in fixed point.
__device__ __forceinline__ float mass_f(float z, float zmax) {
  return exp2f(__fmul_rn(__fsub_rn(z, zmax), kLog2e));
}
__device__ __forceinline__ uint64_t mass_fixed(float e) {
  return (uint64_t)__float2ull_rn(__fmul_rn(e, kMassScale));
}

// ---------------------------------------------------------------------------
// Wave / block reductions and scans (wave64).
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
template <typename T>
__device__ __forceinline__ T wave_max(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    T w = __shfl_xor(v, o, 64);
    v = w > v ? w : v;
  }
  return v;
}
template <typename T>
__device__ __forceinline__ T wave_min(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    T w = __shfl_xor(v, o, 64);
    v = w < v ? w : v;
  }
  return v;
}
// Inclusive scan within a wave.
template <typename T>
__device__ __forceinline__ T wave_incl_scan(T v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    T w = __shfl_up(v, o, 64);
    if (lane >= o) v += w;
  }
  return v;
}

}  // namespace lps
