// Row-group sampling kernel: the fast path of lps_sample on gfx950.
//
// Shape.  Every row is split into G chunks of 16-byte vectors; one workgroup
// of 512 threads holds one chunk in registers (NE logits per thread, read
// once from HBM with non-temporal 16-byte loads).  Workgroup b serves row
// ((b >> 3) / G) * 8 + (b & 7), chunk (b >> 3) % G: ids are dispatched
// round-robin over the 8 XCDs, so the G workgroups of a row run on one XCD,
// dispatched one after another, and exchange data through its L2.  With one
// workgroup per CU (512 threads, up to 256 VGPRs each) a c2 batch (64 rows x 4
// chunks of 40960 logits) is 256 workgroups: one resident wave on 256 CUs.
//
// Per chunk workgroup, by row mode (row_cfg):
//   all      penalties from an 8-bit count table of the chunk's history ids
//            (LDS), legality bits, thread max, workgroup max.
//   GREEDY   first argmax; with logprobs the chunk mass and top-N candidates.
//   TOPK     a threshold below the chunk's k'-th largest logit (from the
//            wave-level k'/8-th largest thread maxima), lowered to the start
//            of its division-collision group; every logit at or above it is
//            published as a candidate.
//   NUCLEUS  (and PURE, top_p = 1): an exact mass histogram of the chunk in
//            LDS: e = exp2(fma(x, c, -ref)), ref = ceil(max * c), binned by
//            e's exponent and top 7 mantissa bits (the top 32 octaves, 128
//            bins each), accumulating count << 48 | the low 16 mantissa bits,
//            so each bin's mass is exact; smaller masses are summed in
//            registers, and the chunk's total mass Z is exact to fp64.
//            The bins are published; after one barrier among the
//            row's workgroups every workgroup merges them (rescaled to the
//            row's reference) and locates two regions: the bins holding the
//            top-p cut (cumulative mass p * Z from the top) and the bins
//            holding the draw (u times the kept mass).  Elements in either
//            region are published as candidates, with the exact mass above
//            each region.
// The last workgroup of a row to finish (an arrival count) finalises it: a
// radix select over the candidates for top-k; for the nucleus, the two region
// lists rank-sorted in LDS with exact fixed-point prefix masses (radix mass
// selects when the lists exceed the sort's capacity); then the outputs.  The
// draw is an inverse CDF in sorted order: kept ids by scaled logit
// descending, ties lower index first.
//
// A row the kernel cannot finish exactly (e.g. a flat row whose regions hold
// more candidates than the finaliser's capacity, min-p / typical-p without
// top-k, entropy requested) is marked LPS_ROW_DEFERRED in the workspace status
// and sampled by the general kernel, launched after this one with that status
// as its filter.
//
// Cross-workgroup handoffs (the histogram barrier and the arrival count):
// every thread of the publishing workgroup stores, then an agent-scope
// release fence; one thread then adds to the row's counter.  The reader spins
// on relaxed agent-scope loads and then takes an agent-scope acquire fence
// before reading the published data.
#pragma once

#include <cstddef>

#include "lps_fast_kernel.h"

// Phase stamps of a timing build (LPS_RG_STAMPS): thread 0 of every
// workgroup records the 100 MHz real-time counter at phase marks into
// rg_stamps (read back with lps_debug_stamps); empty otherwise.
#ifdef LPS_RG_STAMPS
#define RG_STAMP(i)                                                                              \
  do {                                                                                            \
    if (threadIdx.x == 0 && blockIdx.x < 8192)                                                    \
      ::lps::rg::rg_stamps[blockIdx.x * 32 + (i)] = __builtin_amdgcn_s_memrealtime();             \
  } while (0)
#else
#define RG_STAMP(i) ((void)0)
#endif

namespace lps {
namespace rg {
#ifdef LPS_RG_STAMPS
__device__ uint64_t rg_stamps[8192 * 32];
#endif

constexpr int NT = 512;            // threads per workgroup (8 waves: up to 256 VGPRs each)
constexpr int NW = NT / 64;        // waves per workgroup
constexpr int HB = 4096;           // mass histogram bins: the top 32 octaves x 128 sub-bins
constexpr int HOCT = 128;          // bins per octave
constexpr int HB_NAN = HB - 1;     // bin of NaN masses (no real mass reaches it)
constexpr int HPUB = HB;           // published bins
constexpr uint32_t BELOW = 0xFFFFu;  // "bin" of masses under the histogram (summed apart)
constexpr int HE0 = 96;            // float exponent of bin 0: masses from 2^-31
constexpr int MAXG = 16;           // chunks per row
constexpr int CAPR = 4096;         // candidates per row (the finaliser holds 4 per thread)
constexpr int FPT = CAPR / NT;     // finaliser candidates per thread
constexpr int KEPT = 512;          // top-k kept list
constexpr int SELB = 2048;         // radix-select digit bins (11 bits)
constexpr int SELD = 11;
constexpr int HPT = HPUB / NT;     // published histogram bins per thread
constexpr int HLT = HB / NT;       // LDS histogram bins per thread
constexpr int SPT = SELB / NT;     // select bins per thread
constexpr double kFix = 17592186044416.0;  // 2^44: fixed-point masses (relative to the row reference)

// Chunk flags (RgSum.flags); any of them defers the row.
enum {
  RF_OVERFLOW = 1,    // more candidates than the workgroup's slots
  RF_HISTORY = 2,     // a history count does not fit 8 bits
  RF_SPLIT = 4,       // the row's workgroups ran on more than one XCD
  RF_REGION = 8,      // no usable cut / draw region, or the barrier timed out
};

// Per-chunk summary, one 64-byte record (published for the finaliser).
struct RgSum {
  uint32_t mkey;      // max key of the penalised logits (0xFFFFFFFF: NaN present)
  int32_t amax;       // first index of that key (greedy rows)
  float ref;          // mass reference (an integer, log2 units; -inf: no finite logit)
  uint32_t spare;
  uint32_t flags;     // RF_*
  uint32_t xcc;       // XCD that ran the chunk
  uint32_t nab1;      // nucleus: elements above region 1
  uint32_t nanbin;    // nucleus: NaN / +inf masses seen
  double zsum;        // chunk mass: sum of exp2(fma(x, c, -ref))
  double ab1;         // nucleus: exact mass above region 1 (chunk reference)
  double ab2;         // nucleus: exact mass above region 2
  int32_t reg[4];     // nucleus: the regions lo1, hi1, lo2, hi2 (row bins; the same in every chunk)
  uint16_t wc[NW];    // candidates published by each wave (WC_OVER: its segment overflowed);
                      // stored by the waves themselves, the rest by thread 0 (store_sum)
};
constexpr uint16_t WC_OVER = 0xFFFF;
// Thread 0's part of a chunk summary: every field but the wave counts.
__device__ __forceinline__ void store_sum(RgSum* d, const RgSum& a) {
  d->mkey = a.mkey; d->amax = a.amax; d->ref = a.ref; d->spare = a.spare;
  d->flags = a.flags; d->xcc = a.xcc; d->nab1 = a.nab1; d->nanbin = a.nanbin;
  d->zsum = a.zsum; d->ab1 = a.ab1; d->ab2 = a.ab2;
  d->reg[0] = a.reg[0]; d->reg[1] = a.reg[1]; d->reg[2] = a.reg[2]; d->reg[3] = a.reg[3];
}

struct RgParams {
  KParams k;
  // sums: row r holds 2 * MAXG records: [0, G) published before the histogram
  // barrier (max, reference, mass), [MAXG, MAXG + G) at the chunk's end
  int G;               // chunks per row
  int cv;              // vectors per chunk (the last chunk may hold fewer)
  int nvec;            // vectors per row
  int heavy_first;     // dispatch rows without top-k first
  uint32_t* counters;  // [R * 32]: [0] arrivals, [2] histogram barrier; zero between launches
  int32_t* status;     // [R]
  RgSum* sums;         // row r at sums + r * 2 * MAXG
  float* hist;         // row r at hist + r * G * HPUB
  uint2* cands;        // row r at cands + r * CAPR: chunk j owns [j * capw, (j + 1) * capw),
                       // its wave w the segment [w * capw / NW, (w + 1) * capw / NW) of that
  int capw;            // candidate slots per chunk (a multiple of NW)
};

// ---------------------------------------------------------------------------
// Shared memory.
// ---------------------------------------------------------------------------
struct RgX {  // cross-wave exchange slots, each reused only after a barrier
  float f[NW];
  uint32_t u[NW], u2[NW], u3[NW];
  int32_t i1[NW], i2[NW], i3[NW];
  uint64_t q[NW];
  double d[NW], d2[NW], d3[NW], d4[NW], d5[NW];
  uint32_t u4[NW];
  int32_t mi[32];
  double md[16];
  uint64_t mq[8];
  float mf[8];
  int32_t wpre[MAXG * NW];           // finaliser: candidates of each wave segment
  int32_t opre[MAXG * NW];           // finaliser: prefix of the segments' overflow entries
  float rf[MAXG];                    // the row's chunk references
  float rm[MAXG];                    // the row's chunk maxima (NaN chunk: +inf)
};
template <int NE>
struct RgChunkS : RgX {
  uint32_t hc[NT * NE / 4];            // 8-bit history counts of the chunk's ids
  unsigned long long hist[HB + 64];     // count << 48 | sum of low 16 mantissa bits (+ spare slots)
};
struct RgFinalS : RgX {
  uint32_t cnt[SELB];                   // select histograms: counts
  unsigned long long mass[SELB];        // select histograms: fixed-point masses
  int32_t cidx[CAPR];                   // candidate e * NT + t: vocabulary index | region flags
  float cx[CAPR];                       // candidate logit
  uint64_t kkey[KEPT];                  // kept list: (z key << 32) | ~index
  unsigned long long kmass[KEPT];
  int32_t kord[KEPT];                   // sorted position -> slot
  unsigned long long kcum[KEPT];        // inclusive prefix in sorted order
  int32_t lslot[KEPT];                  // nucleus lists: candidate slot of each entry
};
template <int NE>
union RgShared {
  RgChunkS<NE> c;
  RgFinalS f;
};

// ---------------------------------------------------------------------------
// Block helpers (NT threads).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

// Block reduction of a per-thread value; every thread gets the result.  The
// slot array is free again after the next barrier.
template <typename T, typename Op>
__device__ __forceinline__ T bred(T v, T* slot, Op op) {
  v = wreduce(v, op);
  if (lane_id() == 0) slot[wave_id()] = v;
  __syncthreads();
  T r = slot[0];
#pragma unroll
  for (int i = 1; i < NW; i++) r = op(r, slot[i]);
  return r;
}
// Exclusive prefix over the block in thread order; *total gets the sum.
template <typename T>
__device__ __forceinline__ T bscan(T v, T* total, T* slot) {
  const T inc = wscan_incl(v);
  if (lane_id() == 63) slot[wave_id()] = inc;
  __syncthreads();
  T off = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < NW; i++) {
    const T s = slot[i];
    off += (i < wave_id()) ? s : (T)0;
    tot += s;
  }
  *total = tot;
  return off + inc - v;
}

// ---------------------------------------------------------------------------
// Cross-workgroup handoff.
// ---------------------------------------------------------------------------
// Publish protocol (LPS_RG_FENCE): a workgroup publishes data with plain
// stores, then one of its threads adds to a row counter; a reader spins on the
// counter, then reads the data with agent-scope (L1-bypassing) loads.
//   0  every thread waits for its stores to complete (they are then in the
//      XCD's L2, which the row's workgroups share) before the count
//   3  as 0, and the counting thread's add is an agent-scope release, the
//      spinning thread's last load an agent-scope acquire (one L2 writeback
//      and one invalidate per handoff)
//   1  every thread: agent-scope release fence; readers: agent-scope acquire
//      fence (a writeback / invalidate per wave)
#ifndef LPS_RG_FENCE
#define LPS_RG_FENCE 0
#endif
// every thread of the publishing workgroup, before the barrier that precedes the count
__device__ __forceinline__ void release_agent() {
#if LPS_RG_FENCE == 1
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
#else
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
#endif
}
// the counting thread, after that barrier
__device__ __forceinline__ void release_count() {
#if LPS_RG_FENCE == 3
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
#endif
}
// the spinning thread, after the count reached its target
__device__ __forceinline__ void acquire_one() {
#if LPS_RG_FENCE == 3
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
#endif
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// every thread of the reading workgroup, after the barrier that follows the spin
__device__ __forceinline__ void acquire_agent() {
#if LPS_RG_FENCE == 1
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
#endif
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// Loads of published data: agent-scope relaxed atomic loads, which read the
// L2 (never a line this CU's L1 may hold from before the publish).
template <typename T>
__device__ __forceinline__ T ld_pub(const T* p) {
  static_assert(sizeof(T) % 8 == 0 || sizeof(T) == 4, "whole words");
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, __hip_atomic_load(reinterpret_cast<const uint32_t*>(p), __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT));
  } else {
    constexpr int N = sizeof(T) / 8;
    struct W { uint64_t w[N]; } a;
    const uint64_t* s = reinterpret_cast<const uint64_t*>(p);
#pragma unroll
    for (int i = 0; i < N; i++) a.w[i] = __hip_atomic_load(s + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return __builtin_bit_cast(T, a);
  }
}
__device__ __forceinline__ uint32_t ld_agent(uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t add_agent(uint32_t* p, uint32_t v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Masses and bins.
// ---------------------------------------------------------------------------
// Mass of logit x against the integer reference ref: exp2(fma(x, c, -ref)),
// in (0, 1] for x <= the chunk max; 0 for x = -inf.
__device__ __forceinline__ float emass(float x, float c, float ref) {
  return __builtin_amdgcn_exp2f(__builtin_fmaf(x, c, -ref));
}
// Histogram bin of a mass: its exponent and top 7 mantissa bits, 32 octaves
// below 2 (bin 3968 holds [1, 1 + 1/128)); smaller masses (and 0) BELOW,
// NaN / inf in bin HB_NAN.
__device__ __forceinline__ uint32_t ebin(float e) {
  const uint32_t q = __float_as_uint(e) >> 16;
  if (q < (uint32_t)(HE0 << 7)) return BELOW;
  const uint32_t b = q - (uint32_t)(HE0 << 7);
  return b < (uint32_t)HB_NAN ? b : (uint32_t)HB_NAN;
}
// Exact mass of a bin from its accumulator (count << 48 | sum of the low 16
// mantissa bits): 2^(E - 150) * (count * (2^23 + t * 2^16) + low).
__device__ __forceinline__ double bin_mass(uint32_t b, unsigned long long acc) {
  const double cnt = (double)(acc >> 48);
  const double low = (double)(acc & 0xFFFFFFFFFFFFull);
  const int E = (int)(b >> 7) + HE0;
  const double m = cnt * (8388608.0 + (double)(b & 127u) * 65536.0) + low;
  return ldexp(m, E - 150);
}
// Fixed-point mass (2^44 units) of a scaled logit z against the row
// reference R: exp2(fma(z, log2 e, -R)), a function of z alone.
__device__ __forceinline__ uint64_t zmass_fix(float z, float R) {
  return (uint64_t)__float2ull_rn(ldexpf(__builtin_amdgcn_exp2f(__builtin_fmaf(z, kLog2e, -R)), 44));
}
// bin_mass for an accumulator whose low-bit sum fits 32 bits (a chunk bin
// holds at most NT * 80 < 2^16 masses): 2^(E - 150) (count (128 + t) 2^16 + low).
__device__ __forceinline__ double bin_mass_u(int b, unsigned long long acc) {
  const uint32_t cnt = (uint32_t)(acc >> 48), low = (uint32_t)acc;
  const double m = __builtin_fma((double)(cnt * (128u + (uint32_t)(b & 127))), 65536.0, (double)low);
  return ldexp(m, (b >> 7) + HE0 - 150);
}
// The smallest mass of bin b.
__device__ __forceinline__ double bin_base(int b) {
  return ldexp(8388608.0 + (double)(b & 127) * 65536.0, (b >> 7) + HE0 - 150);
}

// ---------------------------------------------------------------------------
// The chunk: NE logits per thread, as NV vectors of VPE logits (VPE = 1 for
// rows read element by element).  Slot s = i * VPE + e of thread t is logit
// (v0 + t + i * NT) * VPE + e of the row.
// ---------------------------------------------------------------------------
template <int DT, int VPE, int NE>
struct Chk {
  static constexpr int NV = NE / VPE;
  static constexpr int ES = DT == LPS_DTYPE_F32 ? 4 : 2;
  static_assert(NE % VPE == 0, "whole vectors");
  static_assert(VPE == 1 || VPE * ES == 16, "16-byte vectors");
  float x[NE];

  // Issues every load before any use; vectors past the chunk end read the
  // chunk's last vector and become -inf.
  __device__ __forceinline__ void load(const char* row, int v0, int nv) {
    const int t = threadIdx.x;
    if constexpr (VPE == 1) {
      float raw[NE];
#pragma unroll
      for (int i = 0; i < NE; i++) raw[i] = load1<DT>(row, (int64_t)v0 + min(t + i * NT, nv - 1));
#pragma unroll
      for (int i = 0; i < NE; i++) x[i] = (t + i * NT) < nv ? raw[i] : -INFINITY;
    } else {
      u32x4 raw[NV];
#pragma unroll
      for (int i = 0; i < NV; i++)
        raw[i] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4*>(row + (int64_t)(v0 + min(t + i * NT, nv - 1)) * 16));
#pragma unroll
      for (int i = 0; i < NV; i++) {
        const bool ok = (t + i * NT) < nv;
        const uint32_t w[4] = {raw[i].x, raw[i].y, raw[i].z, raw[i].w};
        if constexpr (DT == LPS_DTYPE_F32) {
#pragma unroll
          for (int e = 0; e < 4; e++) x[i * 4 + e] = ok ? __uint_as_float(w[e]) : -INFINITY;
        } else {
#pragma unroll
          for (int e = 0; e < 8; e++) {
            const uint32_t h = (w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
            const float f = DT == LPS_DTYPE_BF16 ? __uint_as_float(h << 16) : f16_to_f32(h);
            x[i * 8 + e] = ok ? f : -INFINITY;
          }
        }
      }
    }
  }
  // Vocabulary index of slot s.
  __device__ static __forceinline__ int index(int v0, int s) {
    return (v0 + (int)threadIdx.x + (s / VPE) * NT) * VPE + (s % VPE);
  }
  // Illegal ids to -inf from the row's legality bits (one byte per vector).
  __device__ __forceinline__ void mask(const uint8_t* am, int v0, int nv) {
    if (!am) return;
    const int t = threadIdx.x;
    uint32_t b[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) {
      const int id0 = (v0 + min(t + i * NT, nv - 1)) * VPE;
      b[i] = (uint32_t)am[id0 >> 3] >> (id0 & 7);
    }
#pragma unroll
    for (int i = 0; i < NV; i++)
#pragma unroll
      for (int e = 0; e < VPE; e++)
        if (!((b[i] >> e) & 1u)) x[i * VPE + e] = -INFINITY;
  }
};

// Publishes the slots s < NS for which sel(s) holds into this wave's segment
// (cap entries at seg), in slot order with lane order inside a slot: one
// ballot per slot gives every lane its position, so no block scan is needed.
// Returns the wave's count (the same in every lane; > cap: overflowed).
template <int NS, class Sel, class Emit>
__device__ __forceinline__ uint32_t wave_emit(Sel sel, Emit emit, uint2* seg, uint32_t cap) {
  uint32_t n = 0;
#pragma unroll
  for (int s = 0; s < NS; s++) {
    const bool on = sel(s);
    const uint64_t m = __builtin_amdgcn_ballot_w64(on);
    if (m) {
      if (on) {
        const uint32_t p =
            n + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
        if (p < cap) seg[p] = emit(s);
      }
      n += (uint32_t)__popcll(m);
    }
  }
  return n;
}
// Region bounds [lo, hi] of chunk bins as u16 pairs for the packed test in
// emit_regions: L = lo | lo << 16, C = count | count << 16 (0: empty region).
__device__ __forceinline__ void region_pair(int lo, int hi, uint32_t& L, uint32_t& C) {
  hi = min(hi, HB_NAN - 1);
  const bool empty = lo > hi;
  const uint32_t l = empty ? 0u : (uint32_t)lo, n = empty ? 0u : (uint32_t)(hi - lo + 1);
  L = l | (l << 16);
  C = n | (n << 16);
}
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
// Nonzero halves where the pair of bins w lies in [L, L + C): one wrapping
// and one saturating packed subtraction.
__device__ __forceinline__ uint32_t in_region2(uint32_t w, uint32_t L, uint32_t C) {
  const u16x2 d = __builtin_bit_cast(u16x2, w) - __builtin_bit_cast(u16x2, L);
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_sub_sat(__builtin_bit_cast(u16x2, C), d));
}
// A wave's count into the chunk summary (lane 0 of the wave).
__device__ __forceinline__ void store_wave_count(RgSum* d, uint32_t n, uint32_t cap) {
  if ((threadIdx.x & 63) == 0) d->wc[threadIdx.x >> 6] = n > cap ? WC_OVER : (uint16_t)n;
}

// History ids of the row: the first NT are read before the chunk, so the count
// table is built while the chunk's loads are in flight.
__device__ __forceinline__ int prefetch_hist(const int32_t* hrow, int hlen) {
  const int j = threadIdx.x;
  return (hrow && j < hlen) ? hrow[j] : -1;
}
// 8-bit counts of the history ids that fall in the chunk's ids [lo, lo + n).
// Returns false when a count reaches 255.  Ends with a barrier.
template <int NE>
__device__ __forceinline__ bool build_counts(RgChunkS<NE>& S, const int32_t* hrow, int hlen, int id0, int lo, int n) {
  constexpr int WORDS = NT * NE / 4;
  static_assert(WORDS % 4 == 0, "whole 16-byte stores");
  u32x4* h4 = reinterpret_cast<u32x4*>(S.hc);
#pragma unroll
  for (int i = threadIdx.x; i < WORDS / 4; i += NT) h4[i] = u32x4{0u, 0u, 0u, 0u};
  if (threadIdx.x == 0) S.mi[30] = 0;
  __syncthreads();
  bool sat = false;
  auto add = [&](int id) {
    if (id >= lo && id < lo + n) {
      const int l = id - lo;
      const int sh = 8 * (l & 3);
      const uint32_t old = atomicAdd(&S.hc[l >> 2], 1u << sh);
      if (((old >> sh) & 0xFFu) >= 254u) sat = true;
    }
  };
  add(id0);
  for (int j = NT + (int)threadIdx.x; j < hlen; j += NT) add(hrow[j]);
  if (sat) S.mi[30] = 1;
  __syncthreads();
  return S.mi[30] == 0;
}
// Penalties of the counted ids, applied in place (a vector whose counts are
// all zero costs one LDS read and a branch).
template <int DT, int VPE, int NE>
__device__ __forceinline__ void apply_counts(Chk<DT, VPE, NE>& C, const uint32_t* hc, int nv, float rep, float pres,
                                             float freq) {
  constexpr int NV = Chk<DT, VPE, NE>::NV;
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < NV; i++) {
    const int vl = t + i * NT;
    if (vl >= nv) continue;
    const int l0 = vl * VPE;  // chunk-local id of the vector's first logit
    uint64_t cw;
    if constexpr (VPE == 8) {
      const uint2 q = *reinterpret_cast<const uint2*>(hc + (l0 >> 2));
      cw = ((uint64_t)q.y << 32) | q.x;
    } else if constexpr (VPE == 4) {
      cw = hc[l0 >> 2];
    } else {
      cw = (hc[l0 >> 2] >> (8 * (l0 & 3))) & 0xFFu;
    }
    if (!cw) continue;
#pragma unroll
    for (int e = 0; e < VPE; e++) {
      const uint32_t cnt = (uint32_t)(cw >> (8 * e)) & 0xFFu;
      if (cnt) C.x[i * VPE + e] = penalize(C.x[i * VPE + e], (int)cnt, rep, pres, freq);
    }
  }
}

// ---------------------------------------------------------------------------
// Radix selects of the finaliser over register-resident candidates: thread t
// holds candidate e * NT + t in ck[e], present when e < np.  MSB-first over
// key - kmin with 11-bit digits; each level: one histogram pass, one scan.
// ---------------------------------------------------------------------------
struct Range {
  uint32_t base;
  int bits;
};
template <typename PF>
__device__ __forceinline__ Range key_range(const uint32_t (&ck)[FPT], PF present, RgFinalS& S) {
  uint32_t mn = 0xFFFFFFFFu, mx = 0u;
#pragma unroll
  for (int e = 0; e < FPT; e++)
    if (present(e)) { mn = min(mn, ck[e]); mx = max(mx, ck[e]); }
  mn = bred(mn, S.u, OpMin{});
  mx = bred(mx, S.u2, OpMax{});
  Range R;
  R.base = mn;
  R.bits = mx > mn ? 32 - __clz(mx - mn) : 0;
  return R;
}
// Clears the select histograms (counts, and masses when asked); caller barriers.
__device__ __forceinline__ void clear_sel(RgFinalS& S, bool masses) {
  for (int i = threadIdx.x; i < SELB; i += NT) {
    S.cnt[i] = 0u;
    if (masses) S.mass[i] = 0ull;
  }
}

// kk-th largest present key (1 <= kk <= number present).
template <typename PF>
__device__ uint32_t sel_count(const uint32_t (&ck)[FPT], PF present, uint32_t kk, RgFinalS& S) {
  const Range R = key_range(ck, present, S);
  if (R.bits == 0) { __syncthreads(); return R.base; }
  uint32_t hi = 0, need = kk;
  int top = R.bits;
  while (top > 0) {
    const int sh = top > SELD ? top - SELD : 0;
    const int dw = top - sh;
    clear_sel(S, false);
    __syncthreads();
#pragma unroll
    for (int e = 0; e < FPT; e++) {
      if (present(e)) {
        const uint32_t d = ck[e] - R.base;
        const uint32_t up = top >= 32 ? 0u : (d >> top);
        if (up == hi) atomicAdd(&S.cnt[(d >> sh) & ((1u << dw) - 1u)], 1u);
      }
    }
    __syncthreads();
    // bins from the top: thread t owns descending bins SPT t .. SPT t + SPT - 1
    const int nb = 1 << dw;
    uint32_t cc[SPT], loc = 0;
#pragma unroll
    for (int i = 0; i < SPT; i++) {
      const int b = nb - 1 - SPT * (int)threadIdx.x - i;
      cc[i] = b >= 0 ? S.cnt[b] : 0u;
      loc += cc[i];
    }
    uint32_t tot;
    uint32_t ex = bscan<uint32_t>(loc, &tot, S.u);
#pragma unroll
    for (int i = 0; i < SPT; i++) {
      const int b = nb - 1 - SPT * (int)threadIdx.x - i;
      if (b >= 0 && ex < need && need <= ex + cc[i]) { S.mi[0] = b; S.mi[1] = (int)ex; }
      ex += cc[i];
    }
    __syncthreads();
    hi = (hi << dw) | (uint32_t)S.mi[0];
    need -= (uint32_t)S.mi[1];
    top = sh;
    __syncthreads();
  }
  return R.base + hi;
}

// Mass-weighted select: the largest present key v with A + mass(key >= v) > P
// (requires A <= P < A + total present mass; ok = 0 otherwise).  above =
// A + mass(key > v); ceq / meq = count and mass of key == v.
struct MassSel {
  uint32_t key;
  uint64_t above;
  uint32_t ceq;
  uint64_t meq;
  int ok;
};
template <typename PF>
__device__ MassSel sel_mass(const uint32_t (&ck)[FPT], const uint64_t (&cm)[FPT], PF present, uint64_t A, uint64_t P,
                            RgFinalS& S) {
  MassSel ms{0u, A, 0u, 0ull, 0};
  const Range R = key_range(ck, present, S);
  uint32_t hi = 0;
  int top = R.bits;
  for (;;) {
    const int sh = top > SELD ? top - SELD : 0;
    const int dw = top - sh;
    clear_sel(S, true);
    if (threadIdx.x == 0) S.mi[0] = -1;
    __syncthreads();
#pragma unroll
    for (int e = 0; e < FPT; e++) {
      if (present(e)) {
        const uint32_t d = ck[e] - R.base;
        const uint32_t up = top >= 32 ? 0u : (d >> top);
        if (up == hi) {
          const uint32_t b = dw > 0 ? ((d >> sh) & ((1u << dw) - 1u)) : 0u;
          atomicAdd(&S.cnt[b], 1u);
          if (cm[e]) atomicAdd(&S.mass[b], (unsigned long long)cm[e]);
        }
      }
    }
    __syncthreads();
    const int nb = 1 << dw;
    uint64_t mm[SPT], loc = 0;
#pragma unroll
    for (int i = 0; i < SPT; i++) {
      const int b = nb - 1 - SPT * (int)threadIdx.x - i;
      mm[i] = b >= 0 ? S.mass[b] : 0ull;
      loc += mm[i];
    }
    uint64_t tot;
    uint64_t ex = ms.above + bscan<uint64_t>(loc, &tot, S.q);
#pragma unroll
    for (int i = 0; i < SPT; i++) {
      const int b = nb - 1 - SPT * (int)threadIdx.x - i;
      if (b >= 0 && ex <= P && P < ex + mm[i]) { S.mi[0] = b; S.mi[1] = (int)S.cnt[b]; S.mq[0] = ex; S.mq[1] = mm[i]; }
      ex += mm[i];
    }
    __syncthreads();
    if (S.mi[0] < 0) { __syncthreads(); return ms; }
    hi = (hi << dw) | (uint32_t)S.mi[0];
    ms.above = S.mq[0];
    ms.ceq = (uint32_t)S.mi[1];
    ms.meq = S.mq[1];
    top = sh;
    __syncthreads();
    if (top == 0) break;
  }
  ms.key = R.base + hi;
  ms.ok = 1;
  return ms;
}

// The division-collision group of z = fl(x0 / T): [lo, hi] of every x with
// fl(x / T) == z, searched up to 64 keys each way by one wave (lane l tests the
// step l -> l + 1).  ok = 0 when a side did not end within 64 keys.
struct Group {
  float lo, hi;
  int ok;
};
__device__ __forceinline__ Group collision_group(float x0, float T) {
  const float z = __fdiv_rn(x0, T);
  const uint32_t k0 = f2key(x0);
  const uint32_t l = (uint32_t)lane_id();
  const uint32_t kd = k0 - l, ku = k0 + l;
  const uint64_t fd = wballot(!(kd > kNegInfKey + 1u && __fdiv_rn(key2f(kd - 1u), T) == z));
  const uint64_t fu = wballot(!(ku < 0xFFFFFFFEu && __fdiv_rn(key2f(ku + 1u), T) == z));
  Group g;
  g.lo = key2f(k0 - (fd ? (uint32_t)__builtin_ctzll(fd) : 64u));
  g.hi = key2f(k0 + (fu ? (uint32_t)__builtin_ctzll(fu) : 64u));
  g.ok = (fd != 0ull && fu != 0ull) ? 1 : 0;
  return g;
}

// Row pointer of row r.
template <int DT>
__device__ __forceinline__ const char* row_ptr(const KParams& P, int r) {
  constexpr int ES = DT == LPS_DTYPE_F32 ? 4 : 2;
  return reinterpret_cast<const char*>(P.logits) +
         ES * ((int64_t)(r / P.rows_inner) * P.stride_outer + (int64_t)(r % P.rows_inner) * P.stride_inner);
}

}  // namespace rg
}  // namespace lps

#include "lps_rowgroup_kernel.h"
