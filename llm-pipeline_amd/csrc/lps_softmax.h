// Row softmax with an optional causal mask: the LM-head / attention softmax
// producer (reference: quantization/kernels/triton_softmax.py:65-102,
// fused_softmax_triton; reference semantics at :105-113:
// softmax(masked_fill(col > row + offset, -inf)) in fp32, out in the input dtype).
//
// Three kernels, chosen per call by the host:
//  * softmax_wave_kernel: one wave per row (rows of up to 64 x 32 words: 2048
//    fp32 / 4096 16-bit columns).  The row is read once into registers, the
//    max and the sum are wave reductions, the output is written from the
//    registers: one HBM read, one write, no LDS, no barrier.
//  * softmax_chunk_kernel: G workgroups per row, each holding a chunk of up
//    to 256 x 32 words (8192 fp32 / 16384 16-bit columns) in registers.  With
//    G > 1 each chunk publishes its (max, sum) record, one 64-bit atomic word
//    in the workspace, and polls the row's other records; after its stores,
//    the row's last workgroup zeroes them, so every launch leaves the
//    workspace zeroed for the next (graph replays included).  A row's chunk
//    workgroups are placed on one XCD (workgroup b runs on XCD b % 8) and are
//    dispatched in order, so they are resident together; the wait is bounded,
//    and a workgroup that times out computes every chunk's record itself
//    from the row (the same arithmetic, so the same result).
//  * softmax_kernel: one workgroup per row in three passes (max; sum; output),
//    for rows that are not 16-byte aligned, longer rows, calls without a
//    workspace and in-place calls of split rows.
//
// Arithmetic of the register kernels, per lane: m = the lane's max, then
// e = exp2(fma(x, c, -m c)) (c = log2 e) replaces x in the registers, summed in
// fp32 over each 16-byte vector and in fp64 across vectors.  (max, sum) pairs
// combine as s_a exp2(m_a c - M c) + s_b exp2(m_b c - M c), over lanes, waves,
// then chunk records (sums rounded to fp32); the output is e times the lane's
// scale exp2(m c - M c) / S.  Every workgroup of a row combines the same
// records in the same order, so the row's (M, S) is the same in all of them.
// Non-finite rows come out as torch's do: a NaN or +inf anywhere, or an all
// -inf row, gives a NaN row.  Output conversions round to nearest even
// (v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32 for 16-byte vectors).
#pragma once

#include "lps_common.h"
#include "lps_wave.h"

namespace lps {

struct SoftmaxParams {
  const void* x;
  void* out;
  int64_t x_stride, out_stride;  // elements between rows
  int rows, cols;
  int causal, seq_len, row_offset;  // causal: col > (row % seq_len) + row_offset is -inf
  float* row_lse;                   // optional: log(sum(exp(x))) per row, natural log
  int G;                            // chunk kernel: workgroups per row
  void* records;                    // chunk kernel, G > 1: rows x G 8-byte records, zero between launches
  uint32_t* done;                   // chunk kernel, G > 1: rows counters, zero between launches
  const float* row_stats;           // apply kernel: per row, nstats (max, sum) block pairs
  int64_t stats_stride;             // floats between rows of row_stats
  int nstats;
};

// Per-chunk record of the split softmax, 0 while absent (see pack_record);
// only accessed with device-scope atomics.
typedef unsigned long long SmRecord;

constexpr int SM_NT = 256;          // threads of the chunk / wave kernels' workgroups
constexpr int SM_MAXG = 64;         // chunks per row (one wave combines the records)
constexpr float SM_LOG2E = 1.44269504088896340736f;
constexpr double SM_LN2 = 0.69314718055994530942;

// fp32 -> bf16 / fp16 with round to nearest even (NaN kept NaN).
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ uint32_t f32_to_f16_rne(float f) {
  return (uint32_t)__builtin_bit_cast(unsigned short, (_Float16)f);  // v_cvt_f16_f32: round to nearest even
}

template <int DT>
__device__ __forceinline__ void store1(void* row, int64_t i, float v) {
  if constexpr (DT == LPS_DTYPE_F32) {
    reinterpret_cast<float*>(row)[i] = v;
  } else {
    reinterpret_cast<unsigned short*>(row)[i] =
        (unsigned short)(DT == LPS_DTYPE_BF16 ? f32_to_bf16_rne(v) : f32_to_f16_rne(v));
  }
}

// 16 bytes of output (4 fp32 or 8 16-bit values) at element i0, streamed.
template <int DT>
__device__ __forceinline__ void store16(void* row, int64_t i0, const float* v) {
  constexpr int ES = DT == LPS_DTYPE_F32 ? 4 : 2;
  u32x4 w;
  if constexpr (DT == LPS_DTYPE_F32) {
    w.x = __float_as_uint(v[0]); w.y = __float_as_uint(v[1]);
    w.z = __float_as_uint(v[2]); w.w = __float_as_uint(v[3]);
  } else {
    typedef float f2 __attribute__((ext_vector_type(2)));
    uint32_t h[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const f2 f = {v[2 * e], v[2 * e + 1]};
      if constexpr (DT == LPS_DTYPE_BF16) {
        typedef __bf16 b2 __attribute__((ext_vector_type(2)));
        h[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, b2));
      } else {
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        h[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, h2));
      }
    }
    w.x = h[0]; w.y = h[1]; w.z = h[2]; w.w = h[3];
  }
  __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(reinterpret_cast<char*>(row) + i0 * ES));
}

// Block reduction over NT threads (NT / 64 waves; slot holds NT / 64 values).
template <int NT, typename T, typename Op, typename ST>
__device__ __forceinline__ T block_reduce(T v, ST* slot_raw, Op op) {
  T* slot = reinterpret_cast<T*>(slot_raw);
  v = wreduce(v, op);
  if ((threadIdx.x & 63) == 0) slot[threadIdx.x >> 6] = v;
  __syncthreads();
  T r = slot[0];
#pragma unroll
  for (int w = 1; w < NT / 64; w++) r = op(r, slot[w]);
  __syncthreads();
  return r;
}

// Columns [lim, cols) of row r are -inf (the causal mask).
__device__ __forceinline__ int causal_limit(const SoftmaxParams& S, int r) {
  if (!S.causal) return S.cols;
  const int64_t last = (int64_t)(r % S.seq_len) + S.row_offset;  // last visible column
  return last < 0 ? 0 : (last + 1 < S.cols ? (int)(last + 1) : S.cols);
}

// ---------------------------------------------------------------------------
// Register-resident rows / chunks.
// ---------------------------------------------------------------------------
// (max, sum) pair of a lane, a chunk or a row: s = sum of exp2(x c - m c),
// c = log2(e), with m c the fp32 product.  An all -inf set is (-inf, 0); a set
// holding a NaN has s = NaN.
struct MS {
  float m;
  double s;
};

// Combines two pairs (exactly commutative: the same result either way round).
__device__ __forceinline__ MS ms_combine(MS a, MS b) {
  const float M = fmaxf(a.m, b.m);   // m is never NaN
  const float Mc = __fmul_rn(M, SM_LOG2E);
  const double ta = a.m == -INFINITY ? a.s : a.s * (double)__builtin_amdgcn_exp2f(__fsub_rn(__fmul_rn(a.m, SM_LOG2E), Mc));
  const double tb = b.m == -INFINITY ? b.s : b.s * (double)__builtin_amdgcn_exp2f(__fsub_rn(__fmul_rn(b.m, SM_LOG2E), Mc));
  return MS{M, ta + tb};
}

template <int CTRL>
__device__ __forceinline__ MS ms_dpp_step(MS v) {
  return ms_combine(v, MS{dpp_t<CTRL>(v.m, v.m), dpp_t<CTRL>(v.s, v.s)});
}

// Over the 64 lanes of a wave; every lane gets the same pair.  Each step pairs
// lanes symmetrically, so every lane of a 16-lane row holds the same value
// before the rows are combined in a fixed order.
__device__ __forceinline__ MS wreduce_ms(MS v) {
  v = ms_dpp_step<0xB1>(v);    // quad_perm [1,0,3,2]
  v = ms_dpp_step<0x4E>(v);    // quad_perm [2,3,0,1]
  v = ms_dpp_step<0x141>(v);   // row_half_mirror
  v = ms_dpp_step<0x140>(v);   // row_mirror
  const MS r0{rdlane(v.m, 0), rdlane(v.s, 0)}, r1{rdlane(v.m, 16), rdlane(v.s, 16)};
  const MS r2{rdlane(v.m, 32), rdlane(v.s, 32)}, r3{rdlane(v.m, 48), rdlane(v.s, 48)};
  return ms_combine(ms_combine(r0, r1), ms_combine(r2, r3));
}

struct SmShared {
  float m[SM_NT / 64];
  double s[SM_NT / 64];
  double S;
  float M;
  int flag;
};

// Over the 256 threads of a workgroup; every thread gets the same pair.
__device__ __forceinline__ MS block_reduce_ms(MS v, SmShared& sh) {
  v = wreduce_ms(v);
  if ((threadIdx.x & 63) == 0) {
    sh.m[threadIdx.x >> 6] = v.m;
    sh.s[threadIdx.x >> 6] = v.s;
  }
  __syncthreads();
  const MS r = ms_combine(ms_combine(MS{sh.m[0], sh.s[0]}, MS{sh.m[1], sh.s[1]}),
                          ms_combine(MS{sh.m[2], sh.s[2]}, MS{sh.m[3], sh.s[3]}));
  __syncthreads();
  return r;
}

// A lane's share of a chunk: NV 16-byte vectors at elements
// base + (k * LANES + lane) * VPL, k < NV, in groups of GV vectors.  load()
// reads the values (-inf past lim; vector rows wholly past it are not read);
// exps() turns each group's values into e = exp2(x c - mc_g), mc_g = the
// group's max times c, and returns the lane's pair; store() writes e times its
// group's scale.  A group depends only on its own loads, so its exponentials
// run while the loads of later groups are in flight.  FULL: the whole chunk
// lies before lim and inside the row (no bounds checks).
template <int DT, int NV, int LANES>
struct RegChunk {
  static constexpr int VPL = DT == LPS_DTYPE_F32 ? 4 : 8;   // elements per 16 bytes
  static constexpr int GV = NV < 2 ? NV : 2;                // vectors per group (the last may hold 1)
  static constexpr int NGRP = (NV + GV - 1) / GV;
  __device__ __forceinline__ static constexpr int gend(int g) { return (g + 1) * GV < NV ? (g + 1) * GV : NV; }
  float v[NV][VPL];
  float mc[NGRP];

  __device__ __forceinline__ static int at(int base, int k, int lane) { return base + (k * LANES + lane) * VPL; }
  __device__ __forceinline__ static int row0(int base, int k) { return base + k * LANES * VPL; }   // uniform

  template <bool FULL>
  __device__ __forceinline__ void load(const void* row, int base, int lane, int lim) {
#pragma unroll
    for (int k = 0; k < NV; k++) {
      const int i0 = at(base, k, lane);
      if (FULL) {
        loadv<DT, VPL>(row, i0, v[k]);
        continue;
      }
      if (row0(base, k) >= lim) {
#pragma unroll
        for (int e = 0; e < VPL; e++) v[k][e] = -INFINITY;
      } else if (i0 + VPL <= lim) {
        loadv<DT, VPL>(row, i0, v[k]);
      } else {
#pragma unroll
        for (int e = 0; e < VPL; e++) v[k][e] = i0 + e < lim ? load1<DT>(row, i0 + e) : -INFINITY;
      }
    }
  }

  template <bool FULL>
  __device__ __forceinline__ MS exps(int base, int lim) {
    float mg[NGRP];
    double sg[NGRP];
#pragma unroll
    for (int g = 0; g < NGRP; g++) {
      float m = -INFINITY;
#pragma unroll
      for (int k = g * GV; k < gend(g); k++)
#pragma unroll
        for (int e = 0; e < VPL; e++) m = fmaxf(m, v[k][e]);   // NaN ignored
      mg[g] = m;
      if (m == -INFINITY) {
        // every value -inf or NaN: nothing to exponentiate
        bool nan = false;
#pragma unroll
        for (int k = g * GV; k < gend(g); k++)
#pragma unroll
          for (int e = 0; e < VPL; e++) {
            nan |= v[k][e] != v[k][e];
            v[k][e] = 0.0f;
          }
        mc[g] = -INFINITY;
        sg[g] = nan ? __builtin_nan("") : 0.0;
        continue;
      }
      mc[g] = __fmul_rn(m, SM_LOG2E);
      double s = 0.0;
#pragma unroll
      for (int k = g * GV; k < gend(g); k++) {
        if (!FULL && row0(base, k) >= lim) {   // wholly masked (uniform): e = 0
#pragma unroll
          for (int e = 0; e < VPL; e++) v[k][e] = 0.0f;
          continue;
        }
        float t = 0.0f;
#pragma unroll
        for (int e = 0; e < VPL; e++) {
          v[k][e] = __builtin_amdgcn_exp2f(__builtin_fmaf(v[k][e], SM_LOG2E, -mc[g]));
          t += v[k][e];
        }
        s += (double)t;   // fp32 within a vector, fp64 across vectors
      }
      sg[g] = s;
    }
    // the lane's pair: groups rescaled to the lane max, in group order
    float m = mg[0];
#pragma unroll
    for (int g = 1; g < NGRP; g++) m = fmaxf(m, mg[g]);
    if (NGRP == 1 || m == -INFINITY) {
      double s = 0.0;
#pragma unroll
      for (int g = 0; g < NGRP; g++) s += sg[g];
      return MS{m, s};
    }
    const float lmc = __fmul_rn(m, SM_LOG2E);
    double s = 0.0;
#pragma unroll
    for (int g = 0; g < NGRP; g++)
      s += mg[g] == -INFINITY ? sg[g] : sg[g] * (double)__builtin_amdgcn_exp2f(__fsub_rn(mc[g], lmc));
    return MS{m, s};
  }

  // writes e times exp2(mc_g - M c) / S for the row pair (M, S)
  template <bool FULL>
  __device__ __forceinline__ void store(void* orow, int base, int lane, int n, MS row) const {
    const float Mc = __fmul_rn(row.m, SM_LOG2E);
    const double inv = 1.0 / row.s;
#pragma unroll
    for (int g = 0; g < NGRP; g++) {
      const float sc = (float)((double)__builtin_amdgcn_exp2f(__fsub_rn(mc[g], Mc)) * inv);
#pragma unroll
      for (int k = g * GV; k < gend(g); k++) {
        const int i0 = at(base, k, lane);
        float p[VPL];
#pragma unroll
        for (int e = 0; e < VPL; e++) p[e] = __fmul_rn(v[k][e], sc);
        if (FULL || i0 + VPL <= n) {
          store16<DT>(orow, i0, p);
        } else {
#pragma unroll
          for (int e = 0; e < VPL; e++)
            if (i0 + e < n) store1<DT>(orow, i0 + e, p[e]);
        }
      }
    }
  }
};

// log(sum(exp(x))) of a row from its pair: -inf for an all -inf row, NaN for a
// row holding a NaN or +inf.
__device__ __forceinline__ float row_lse_value(MS row) {
  if (row.m == -INFINITY && row.s == 0.0) return -INFINITY;
  return (float)((double)__fmul_rn(row.m, SM_LOG2E) * SM_LN2 + log(row.s));
}

template <int DT, int NV, bool FULL>
__device__ __forceinline__ void wave_row(const SoftmaxParams& S, const void* row, void* orow, int r, int lane, int lim) {
  RegChunk<DT, NV, 64> C;
  C.template load<FULL>(row, 0, lane, lim);
  const MS rs = wreduce_ms(C.template exps<FULL>(0, lim));
  if (S.row_lse && lane == 0) S.row_lse[r] = row_lse_value(rs);
  C.template store<FULL>(orow, 0, lane, S.cols, rs);
}

// One wave per row.
template <int DT, int NV>
__global__ __launch_bounds__(SM_NT) void softmax_wave_kernel(SoftmaxParams S) {
  const int r = blockIdx.x * (SM_NT / 64) + (threadIdx.x >> 6);
  if (r >= S.rows) return;   // whole waves leave; no block barrier follows
  constexpr int ES = DT == LPS_DTYPE_F32 ? 4 : 2;
  constexpr int CH = 64 * NV * RegChunk<DT, NV, 64>::VPL;
  const int lane = threadIdx.x & 63;
  const void* row = reinterpret_cast<const char*>(S.x) + (int64_t)ES * r * S.x_stride;
  void* orow = reinterpret_cast<char*>(S.out) + (int64_t)ES * r * S.out_stride;
  const int lim = causal_limit(S, r);
  if (lim == CH && S.cols == CH) wave_row<DT, NV, true>(S, row, orow, r, lane, lim);
  else wave_row<DT, NV, false>(S, row, orow, r, lane, lim);
}

__device__ __forceinline__ uint32_t l2_add_u32(uint32_t* p, uint32_t v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A chunk record: the chunk max (low word) and its sum rounded to fp32 (high
// word).  Never 0: a chunk's sum is >= 1 unless its max is -inf.
__device__ __forceinline__ unsigned long long pack_record(MS c) {
  return (unsigned long long)__float_as_uint(c.m) | ((unsigned long long)__float_as_uint((float)c.s) << 32);
}
__device__ __forceinline__ MS unpack_record(unsigned long long w) {
  return MS{__uint_as_float((uint32_t)w), (double)__uint_as_float((uint32_t)(w >> 32))};
}

// Chunk j of row r.  With G > 1: publish the chunk's record, wait for the
// row's others (or fall back to the row), store, then count this workgroup
// out of the row's records.
template <int DT, int NV, bool FULL>
__device__ __forceinline__ void chunk_row(const SoftmaxParams& S, SmShared& sh, const void* row, void* orow, int r,
                                          int j, int lim) {
  using RC = RegChunk<DT, NV, SM_NT>;
  constexpr int CH = SM_NT * NV * RC::VPL;
  const int G = S.G;
  const int tid = threadIdx.x;
  const int base = j * CH;
  RC C;
  C.template load<FULL>(row, base, tid, lim);
  const MS ch = block_reduce_ms(C.template exps<FULL>(base, lim), sh);
  MS rs = ch;
  unsigned long long* rec = reinterpret_cast<unsigned long long*>(S.records) + (int64_t)r * G;
  if (G > 1) {
    const unsigned long long mine = pack_record(ch);
    if (tid == 0) __hip_atomic_exchange(&rec[j], mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid < 64) {
      // wave 0, lane t < G: wait for record t (a few microseconds).  The bound
      // (about 2^16 polls) only guards a launch whose chunk workgroups are not
      // resident together; then the workgroup falls back to the row itself.
      const int lane = tid;
      unsigned long long w = lane == j ? mine : 0ull;
      bool have = lane >= G || lane == j;
      int spins = 0;
      while (!__all(have)) {
        if (!have) {
          w = atomicCAS(&rec[lane], ~0ull, ~0ull);   // read at the L2 (a record is never ~0)
          have = w != 0ull;
        }
        if (++spins > (1 << 16)) break;
      }
      const bool fallback = !__all(have);
      const MS row_pair = wreduce_ms(lane < G && !fallback ? unpack_record(w) : MS{-INFINITY, 0.0});
      if (lane == 0) {
        sh.flag = fallback ? 1 : 0;
        sh.M = row_pair.m;
        sh.S = row_pair.s;
      }
    }
    __syncthreads();
    if (sh.flag) {
      // every chunk's record from the row itself, in the same arithmetic (the
      // chunk registers are reused, then reloaded with this workgroup's chunk;
      // the host never splits an in-place call)
      unsigned long long w = 0ull;
      for (int t = 0; t < G; t++) {
        C.template load<false>(row, t * CH, tid, lim);
        const MS ct = block_reduce_ms(C.template exps<false>(t * CH, lim), sh);
        if (tid == t) w = pack_record(ct);
      }
      if (tid < 64) {
        const MS row_pair = wreduce_ms(tid < G ? unpack_record(w) : MS{-INFINITY, 0.0});
        if (tid == 0) {
          sh.M = row_pair.m;
          sh.S = row_pair.s;
        }
      }
      C.template load<FULL>(row, base, tid, lim);
      C.template exps<FULL>(base, lim);
      __syncthreads();
    }
    rs = MS{sh.M, sh.S};
  }
  if (S.row_lse && j == 0 && tid == 0) S.row_lse[r] = row_lse_value(rs);
  C.template store<FULL>(orow, base, tid, S.cols, rs);
  if (G > 1 && tid < 64) {
    // this workgroup reads no record any more; the row's last one zeroes the
    // row's records and counter for the next launch
    uint32_t last = 0;
    if (tid == 0) last = l2_add_u32(&S.done[r], 1u) + 1u == (uint32_t)G ? 1u : 0u;
    if (rdlane_u32(last, 0)) {
      if (tid < G) __hip_atomic_exchange(&rec[tid], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (tid == 0) __hip_atomic_exchange(&S.done[r], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// G workgroups per row (workgroup b: XCD b % 8, row (b / 8) / G * 8 + b % 8,
// chunk (b / 8) % G), each holding CH = 256 * NV * VPL columns in registers.
template <int DT, int NV>
__global__ __launch_bounds__(SM_NT) void softmax_chunk_kernel(SoftmaxParams S) {
  __shared__ SmShared sh;
  constexpr int ES = DT == LPS_DTYPE_F32 ? 4 : 2;
  constexpr int CH = SM_NT * NV * RegChunk<DT, NV, SM_NT>::VPL;
  const int G = S.G;
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  const int r = (slot / G) * 8 + xcd, j = slot % G;
  if (r >= S.rows) return;   // uniform over the workgroup
  const void* row = reinterpret_cast<const char*>(S.x) + (int64_t)ES * r * S.x_stride;
  void* orow = reinterpret_cast<char*>(S.out) + (int64_t)ES * r * S.out_stride;
  const int lim = causal_limit(S, r);
  if ((j + 1) * CH <= lim) chunk_row<DT, NV, true>(S, sh, row, orow, r, j, lim);   // lim <= cols
  else chunk_row<DT, NV, false>(S, sh, row, orow, r, j, lim);
}

// Single pass from block statistics (the LM-head epilogue's): every
// workgroup of a row combines the row's nstats (max, sum) pairs in the same
// order (thread t takes pairs t, t + 256, ...; then the block reduction), so
// all of them hold the same (M, S); then its chunk is streamed as
// exp2(x c - M c) / S.  Mapping as the chunk kernel's.
template <int DT, int NV>
__global__ __launch_bounds__(SM_NT) void softmax_apply_kernel(SoftmaxParams S) {
  __shared__ SmShared sh;
  constexpr int ES = DT == LPS_DTYPE_F32 ? 4 : 2;
  constexpr int VPL = DT == LPS_DTYPE_F32 ? 4 : 8;
  constexpr int CH = SM_NT * NV * VPL;
  const int G = S.G;
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  const int r = (slot / G) * 8 + xcd, j = slot % G;
  if (r >= S.rows) return;   // uniform over the workgroup
  const int tid = threadIdx.x;
  const void* row = reinterpret_cast<const char*>(S.x) + (int64_t)ES * r * S.x_stride;
  void* orow = reinterpret_cast<char*>(S.out) + (int64_t)ES * r * S.out_stride;
  const int n = S.cols;
  // the chunk's loads first: they are in flight while the statistics combine
  float v[NV][VPL];
#pragma unroll
  for (int k = 0; k < NV; k++) {
    const int i0 = j * CH + (k * SM_NT + tid) * VPL;
    if (i0 + VPL <= n) {
      loadv<DT, VPL>(row, i0, v[k]);
    } else {
#pragma unroll
      for (int e = 0; e < VPL; e++) v[k][e] = i0 + e < n ? load1<DT>(row, i0 + e) : -INFINITY;
    }
  }
  const float* st = S.row_stats + (int64_t)r * S.stats_stride;
  MS acc{-INFINITY, 0.0};
  for (int b = tid; b < S.nstats; b += SM_NT) acc = ms_combine(acc, MS{st[2 * b], (double)st[2 * b + 1]});
  const MS rs = block_reduce_ms(acc, sh);
  if (S.row_lse && j == 0 && tid == 0) S.row_lse[r] = row_lse_value(rs);
  const float Mc = __fmul_rn(rs.m, SM_LOG2E);
  const float inv = rs.m == -INFINITY ? __builtin_nanf("") : (float)(1.0 / rs.s);
#pragma unroll
  for (int k = 0; k < NV; k++) {
    const int i0 = j * CH + (k * SM_NT + tid) * VPL;
    if (i0 >= n) continue;
    float p[VPL];
#pragma unroll
    for (int e = 0; e < VPL; e++) p[e] = __fmul_rn(__builtin_amdgcn_exp2f(__builtin_fmaf(v[k][e], SM_LOG2E, -Mc)), inv);
    if (i0 + VPL <= n) {
      store16<DT>(orow, i0, p);
    } else {
#pragma unroll
      for (int e = 0; e < VPL; e++)
        if (i0 + e < n) store1<DT>(orow, i0 + e, p[e]);
    }
  }
}

// ---------------------------------------------------------------------------
// One workgroup per row, three passes: pass 1 reads the row from HBM (max);
// passes 2 and 3 re-read it, from the caches where it fits (sum of exp(x - max)
// accumulated in fp64; then exp(x - max) / sum).  torch's formula.
// ---------------------------------------------------------------------------
template <int DT, int VEC, int NT>
__global__ __launch_bounds__(NT) void softmax_kernel(SoftmaxParams S) {
  __shared__ double slot[NT / 64];
  constexpr int ES = DT == LPS_DTYPE_F32 ? 4 : 2;
  const int r = blockIdx.x;
  const int tid = threadIdx.x;
  const int n = S.cols;
  const void* row = reinterpret_cast<const char*>(S.x) + (int64_t)ES * r * S.x_stride;
  void* orow = reinterpret_cast<char*>(S.out) + (int64_t)ES * r * S.out_stride;
  const int lim = causal_limit(S, r);
  // passes 1 and 2 keep the row in the caches; pass 3 streams it
  auto get_kept = [&](int64_t i0, float (&v)[VEC]) {
    if (i0 + VEC <= lim) {
      loadv<DT, VEC, false>(row, i0, v);
    } else {
#pragma unroll
      for (int j = 0; j < VEC; j++) v[j] = i0 + j < lim ? load1<DT, false>(row, i0 + j) : -INFINITY;
    }
  };
  auto get_last = [&](int64_t i0, float (&v)[VEC]) {
    if (i0 + VEC <= lim) {
      loadv<DT, VEC, true>(row, i0, v);
    } else {
#pragma unroll
      for (int j = 0; j < VEC; j++) v[j] = i0 + j < lim ? load1<DT, true>(row, i0 + j) : -INFINITY;
    }
  };
  // pass 1: max (NaN propagates into the sum of pass 2)
  float m = -INFINITY;
  uint32_t nan = 0;
  for (int64_t i0 = (int64_t)tid * VEC; i0 < n; i0 += (int64_t)NT * VEC) {
    float v[VEC];
    get_kept(i0, v);
#pragma unroll
    for (int j = 0; j < VEC; j++) {
      m = fmaxf(m, v[j]);
      nan |= v[j] != v[j] ? 1u : 0u;
    }
  }
  m = block_reduce<NT>(m, slot, OpMax{});
  nan = block_reduce<NT>(nan, slot, OpOr{});
  // pass 2: sum of exp(x - max)
  double sd = 0.0;
  for (int64_t i0 = (int64_t)tid * VEC; i0 < n; i0 += (int64_t)NT * VEC) {
    float v[VEC];
    get_kept(i0, v);
#pragma unroll
    for (int j = 0; j < VEC; j++) sd += (double)expf(__fsub_rn(v[j], m));
  }
  sd = block_reduce<NT>(sd, slot, OpAdd{});
  if (S.row_lse && tid == 0) S.row_lse[r] = !nan && m == -INFINITY ? -INFINITY : (float)((double)m + log(sd));
  // pass 3: exp(x - max) / sum
  const float inv = (float)(1.0 / sd);
  for (int64_t i0 = (int64_t)tid * VEC; i0 < n; i0 += (int64_t)NT * VEC) {
    float v[VEC];
    get_last(i0, v);
#pragma unroll
    for (int j = 0; j < VEC; j++) store1<DT>(orow, i0 + j, __fmul_rn(expf(__fsub_rn(v[j], m)), inv));
  }
}

}  // namespace lps
