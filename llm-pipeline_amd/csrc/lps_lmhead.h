// LM-head projection with a softmax-statistics epilogue: the logits producer
// of the sampling path (reference: models/qwen3/custom_builder.py:415 and
// models/qwen3_5/model.py:263, logits = lm_head(hidden), an nn.Linear without
// bias), fused with the per-row statistics a softmax of those logits needs.
//
//   out[m, n] = sum_k x[m, k] * w[n, k]          (fp32 accumulation, MFMA)
//   stats[m, b] = (max, sum exp(v - max))  over the 128 columns of block b,
//                 v = out[m, n] as stored (rounded to the output dtype)
//
// One 256-thread workgroup computes a 64-row x 128-column tile: each wave a
// 64 x 32 slice as two 32x32 accumulators of v_mfma_f32_32x32x16_{bf16,f16}.
// Operand layout of that instruction (checked on gfx950): lane l holds A row
// l % 32 and B column l % 32, k = 8 (l / 32) .. +7; accumulator element i of
// lane l is row 8 (i / 4) + 4 (l / 32) + i % 4, column l % 32.  The weight,
// read once, is the HBM traffic; X (a few hundred KB) is served by the caches.
// The epilogue moves the rounded tile through LDS (row stride 33 words), so
// that each quad of threads owns one row's 128 columns: it stores them in
// 16-byte vectors, 64 contiguous bytes per store instruction, and reduces the
// row's (max, sum) for the block.
#pragma once

#include "lps_common.h"
#include "lps_wave.h"

namespace lps {

constexpr int LMH_BN = 128;   // columns per workgroup (and per statistics block)
constexpr int LMH_BM = 64;    // rows per workgroup

struct LmHeadParams {
  const void* x;       // [M, H], row stride x_stride elements
  const void* w;       // [V, H], row stride w_stride elements
  void* out;           // [M, V], row stride out_stride elements
  float* stats;        // [M, G] pairs (max, sum), G = ceil(V / 128), or null
  int M, V, H;
  int64_t x_stride, w_stride, out_stride;
  int G;
};

template <int DT> struct MfmaOps;
template <> struct MfmaOps<LPS_DTYPE_BF16> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  typedef float acc __attribute__((ext_vector_type(16)));
  __device__ __forceinline__ static acc mma(u32x4 a, u32x4 b, acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0, 0);
  }
};
template <> struct MfmaOps<LPS_DTYPE_F16> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  typedef float acc __attribute__((ext_vector_type(16)));
  __device__ __forceinline__ static acc mma(u32x4 a, u32x4 b, acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0, 0);
  }
};

// fp32 -> the output dtype and back (the value the output holds), RNE.
template <int ODT>
__device__ __forceinline__ float round_to(float v) {
  if constexpr (ODT == LPS_DTYPE_F32) {
    return v;
  } else if constexpr (ODT == LPS_DTYPE_BF16) {
    return __uint_as_float((uint32_t)__builtin_bit_cast(unsigned short, (__bf16)v) << 16);
  } else {
    return (float)(_Float16)v;
  }
}

// K-chunks of KC columns are staged through LDS (one or two buffers): the W tile
// (128 rows) and the X tile (64 rows) of a chunk are read with fully
// coalesced 16-byte loads (CPR threads per row), written to LDS rows padded to
// KC * 2 + 16 bytes (so that the MFMA fragment reads, 16 bytes from each of 32
// rows, are bank-conflict free), and the loads of chunk s + 1 are in flight
// (in registers) while chunk s is multiplied.  Columns past H (the last chunk when H is not a
// multiple of KC) are zero-filled, not read.
template <int KC>
struct LmStage {
  static constexpr int RS = KC * 2 + 16;          // LDS row stride (bytes)
  static constexpr int CPR = KC / 8;               // 16-byte chunks per row
  static constexpr int WL = LMH_BN * CPR / 256;    // W chunks per thread
  static constexpr int XL = LMH_BM * CPR / 256;    // X chunks per thread
  static constexpr int WB = LMH_BN * RS, XB = LMH_BM * RS;
  static constexpr int BYTES = WB + XB;            // one stage
};
// Stage shape, measured on 64 x 4096 -> 151936 bf16 with the variants timed
// in turn in one process (medians of 9): KC = 256 with one buffer, 269.6 us;
// KC = 128 with one buffer (three workgroups per CU), 273.5 us; persistent
// grids walking the tiles with the next tile's loads under the epilogue
// (KC = 128 / 256, one to three workgroups per CU), 288-293 us; two buffers
// (one workgroup per CU at KC = 128) and KC <= 64 slower still.
#ifndef LMH_KC
#define LMH_KC 256
#endif
#ifndef LMH_NB
#define LMH_NB 1
#endif
constexpr int LMH_TILE_BYTES = 4 * LMH_BM * 33 * 4;   // the epilogue's tile
template <int KC, int NB>
constexpr int lmh_lds_bytes() {
  return NB * LmStage<KC>::BYTES > LMH_TILE_BYTES ? NB * LmStage<KC>::BYTES : LMH_TILE_BYTES;
}

// A thread's share of one stage: global sources (rows clamped into range;
// their results are dropped) and LDS destinations of its 16-byte chunks, and
// the chunks themselves while in flight.
template <int KC>
struct LmLoader {
  using St = LmStage<KC>;
  static_assert(St::XL >= 1 && (KC % 16) == 0 && 256 % St::CPR == 0, "stage shape: whole rows per thread group");
  const char* wsrc[St::WL];
  const char* xsrc[St::XL];
  u32x4 gw[St::WL], gx[St::XL];

  __device__ __forceinline__ static int row_of(int i) { return (int)threadIdx.x / St::CPR + i * (256 / St::CPR); }
  __device__ __forceinline__ static int col_of() { return ((int)threadIdx.x % St::CPR) * 8; }

  __device__ __forceinline__ void setup(const LmHeadParams& P, int n0, int m0) {
#pragma unroll
    for (int i = 0; i < St::WL; i++) {
      const int n = n0 + row_of(i);
      wsrc[i] = reinterpret_cast<const char*>(P.w) + ((int64_t)(n < P.V ? n : P.V - 1) * P.w_stride + col_of()) * 2;
    }
#pragma unroll
    for (int i = 0; i < St::XL; i++) {
      const int m = m0 + row_of(i);
      xsrc[i] = reinterpret_cast<const char*>(P.x) + ((int64_t)(m < P.M ? m : P.M - 1) * P.x_stride + col_of()) * 2;
    }
  }
  // columns past H are zero-filled, not read
  __device__ __forceinline__ void gload(const LmHeadParams& P, int kb) {
    const u32x4 zero = {0u, 0u, 0u, 0u};
    const bool in = kb + col_of() < P.H;
#pragma unroll
    for (int i = 0; i < St::WL; i++)
      gw[i] = in ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wsrc[i] + kb * 2)) : zero;
#pragma unroll
    for (int i = 0; i < St::XL; i++) gx[i] = in ? *reinterpret_cast<const u32x4*>(xsrc[i] + kb * 2) : zero;
  }
  __device__ __forceinline__ void lstore(char* buf) const {
    const int c = col_of() * 2;
#pragma unroll
    for (int i = 0; i < St::WL; i++) *reinterpret_cast<u32x4*>(buf + row_of(i) * St::RS + c) = gw[i];
#pragma unroll
    for (int i = 0; i < St::XL; i++) *reinterpret_cast<u32x4*>(buf + St::WB + row_of(i) * St::RS + c) = gx[i];
  }
};

// The MFMAs of one stage: B row wv * 32 + (l & 31), A rows (l & 31) and
// 32 + (l & 31), k = 16 ks + 8 (l >> 5) within the stage.
template <int DT, int KC>
__device__ __forceinline__ void lmh_stage_mma(const char* cur, typename MfmaOps<DT>::acc& c0,
                                              typename MfmaOps<DT>::acc& c1) {
  using St = LmStage<KC>;
  const int wv = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int boff = (wv * 32 + (l & 31)) * St::RS + (l >> 5) * 16;
  const int aoff0 = St::WB + (l & 31) * St::RS + (l >> 5) * 16;
  const int aoff1 = aoff0 + 32 * St::RS;
#pragma unroll
  for (int ks = 0; ks < KC / 16; ks++) {
    const u32x4 b = *reinterpret_cast<const u32x4*>(cur + boff + ks * 32);
    const u32x4 a0 = *reinterpret_cast<const u32x4*>(cur + aoff0 + ks * 32);
    const u32x4 a1 = *reinterpret_cast<const u32x4*>(cur + aoff1 + ks * 32);
    c0 = MfmaOps<DT>::mma(a0, b, c0);
    c1 = MfmaOps<DT>::mma(a1, b, c1);
  }
}

// The tile's rounded values through LDS (the stages are free by then), the
// block statistics and the 16-byte stores of the output.
template <int DT, int ODT>
__device__ __forceinline__ void lmh_epilogue(const LmHeadParams& P, char* lds, const typename MfmaOps<DT>::acc& c0,
                                             const typename MfmaOps<DT>::acc& c1, int n0, int m0) {
  float(*tile)[LMH_BM][33] = reinterpret_cast<float(*)[LMH_BM][33]>(lds);
  const int wv = threadIdx.x >> 6, l = threadIdx.x & 63;
  // rounded tile into LDS: wave wv's 32 columns of the 64 rows
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const int row = 8 * (i >> 2) + 4 * (l >> 5) + (i & 3);
    tile[wv][row][l & 31] = round_to<ODT>(c0[i]);
    tile[wv][row + 32][l & 31] = round_to<ODT>(c1[i]);
  }
  __syncthreads();
  // thread (row r, part p) of row m0 + r: the four 8-column pieces
  // n0 + 32 q + 8 p .. +7, q < 4, so that the quad's q-th stores are 64
  // contiguous bytes (whole lines reach the memory, not 16-byte pieces)
  const int r = threadIdx.x >> 2, p = threadIdx.x & 3;
  const int m = m0 + r;
  float v[32];
#pragma unroll
  for (int q = 0; q < 4; q++)
#pragma unroll
    for (int e = 0; e < 8; e++) v[8 * q + e] = n0 + 32 * q + 8 * p + e < P.V ? tile[q][r][8 * p + e] : -INFINITY;
  if (P.stats) {
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 32; j++) mx = fmaxf(mx, v[j]);
    mx = fmaxf(mx, dpp_t<0xB1>(mx, mx));   // quad_perm [1,0,3,2]
    mx = fmaxf(mx, dpp_t<0x4E>(mx, mx));   // quad_perm [2,3,0,1]
    // sum of exp2(v c - M c), c = log2 e (every block holds a valid column;
    // a NaN or +inf value makes the sum NaN)
    const float mc = __fmul_rn(mx, 1.44269504088896340736f);
    float t = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; j++) t += __builtin_amdgcn_exp2f(__builtin_fmaf(v[j], 1.44269504088896340736f, -mc));
    double s = (double)t;
    s += dpp_t<0xB1>(s, s);
    s += dpp_t<0x4E>(s, s);
    if (p == 0 && m < P.M) {
      float* o = P.stats + ((int64_t)m * P.G + n0 / LMH_BN) * 2;
      o[0] = mx;
      o[1] = (float)s;
    }
  }
  if (m < P.M) {
    constexpr int ES = ODT == LPS_DTYPE_F32 ? 4 : 2;
    char* orow = reinterpret_cast<char*>(P.out) + (int64_t)m * P.out_stride * ES;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int c0 = n0 + 32 * q + 8 * p;     // first column of the piece
      const float* pv = v + 8 * q;
      char* dst = orow + (int64_t)c0 * ES;
      if (c0 + 8 <= P.V && (reinterpret_cast<uintptr_t>(dst) & 15) == 0) {
        if constexpr (ODT == LPS_DTYPE_F32) {
          u32x4 w0, w1;
          w0.x = __float_as_uint(pv[0]); w0.y = __float_as_uint(pv[1]); w0.z = __float_as_uint(pv[2]); w0.w = __float_as_uint(pv[3]);
          w1.x = __float_as_uint(pv[4]); w1.y = __float_as_uint(pv[5]); w1.z = __float_as_uint(pv[6]); w1.w = __float_as_uint(pv[7]);
          reinterpret_cast<u32x4*>(dst)[0] = w0;
          reinterpret_cast<u32x4*>(dst)[1] = w1;
        } else {
          uint32_t h[4];
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const float a = pv[2 * e], b = pv[2 * e + 1];
            // the values already hold the output dtype's rounding: exact
            const uint32_t ha = ODT == LPS_DTYPE_BF16 ? (__float_as_uint(a) >> 16)
                                                      : (uint32_t)__builtin_bit_cast(unsigned short, (_Float16)a);
            const uint32_t hb = ODT == LPS_DTYPE_BF16 ? (__float_as_uint(b) >> 16)
                                                      : (uint32_t)__builtin_bit_cast(unsigned short, (_Float16)b);
            h[e] = ha | (hb << 16);
          }
          u32x4 wq;
          wq.x = h[0]; wq.y = h[1]; wq.z = h[2]; wq.w = h[3];
          *reinterpret_cast<u32x4*>(dst) = wq;
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; e++) {
          if (c0 + e < P.V) {
            if constexpr (ODT == LPS_DTYPE_F32) {
              reinterpret_cast<float*>(dst)[e] = pv[e];
            } else if constexpr (ODT == LPS_DTYPE_BF16) {
              reinterpret_cast<unsigned short*>(dst)[e] = (unsigned short)(__float_as_uint(pv[e]) >> 16);
            } else {
              reinterpret_cast<unsigned short*>(dst)[e] = __builtin_bit_cast(unsigned short, (_Float16)pv[e]);
            }
          }
        }
      }
    }
  }
}

// One tile per workgroup.  KC: K columns per stage; NB: LDS stage buffers
// (2: the next stage is written while the current one is read; 1: written
// after a barrier, for half the LDS and more workgroups per CU).
template <int DT, int ODT, int KC, int NB>
__global__ __launch_bounds__(256) void lmhead_kernel(LmHeadParams P) {
  using St = LmStage<KC>;
  __shared__ __attribute__((aligned(16))) char lds[lmh_lds_bytes<KC, NB>()];
  const int n0 = blockIdx.x * LMH_BN, m0 = blockIdx.y * LMH_BM;
  LmLoader<KC> L;
  L.setup(P, n0, m0);
  typename MfmaOps<DT>::acc c0 = {}, c1 = {};
  const int ns = (P.H + KC - 1) / KC;
  L.gload(P, 0);
  L.lstore(lds);
  __syncthreads();
  for (int s = 0; s < ns; s++) {
    const char* cur = lds + (NB == 2 ? (s & 1) * St::BYTES : 0);
    if (s + 1 < ns) L.gload(P, (s + 1) * KC);
    lmh_stage_mma<DT, KC>(cur, c0, c1);
    if (NB == 1) __syncthreads();   // every wave is done reading the buffer
    if (s + 1 < ns) L.lstore(lds + (NB == 2 ? ((s + 1) & 1) * St::BYTES : 0));
    __syncthreads();
  }
  lmh_epilogue<DT, ODT>(P, lds, c0, c1, n0, m0);
}

}  // namespace lps
