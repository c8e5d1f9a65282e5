// Fast row sampler in two kernels.
//
// chunk_kernel: every row is split into G chunks of 8192 logits, one
// 256-thread workgroup per chunk, the chunk held in registers (the logits are
// read from HBM once; only the chunk that holds the draw of a nucleus / pure
// row is read a second time, by the row's finaliser, normally from the L2).
// Each chunk publishes a summary (max, mass, histogram top bin) and, depending
// on the row's mode, candidates.  Workgroup ids are dispatched round-robin over
// the XCDs, and chunk workgroups of a row are given ids congruent modulo 8, so
// a row's chunks share one L2: nucleus rows pass one intra-row barrier there.
//
// final_kernel: one workgroup per row reads the row's chunk summaries and
// candidates (published by the previous kernel, so visible to every XCD) and
// finishes the row.
//
// Row modes (decided per row from its parameters):
//   GREEDY  T <= 0: first argmax (plus logprobs).
//   TOPK    0 < top_k <= FAST_KMAX: each chunk publishes a small superset of
//           its local top-k' (k' = max(k, n_top)), found with per-wave ballot
//           selection; the finaliser selects the global k-th value among the
//           published candidates, applies top-p / min-p / typical-p on the
//           small kept set and draws from it.
//   PURE    top_k off and no other filter: no cut; the finaliser picks the
//           chunk holding the draw from per-chunk masses and rescans it.
//   NUCLEUS top_k off, top_p < 1: chunks publish a fine mass histogram, pass
//           one intra-row barrier, all derive the same cut region (the bins
//           whose cumulative mass meets top_p within a tolerance band), and
//           publish the candidates inside it plus their exact mass above it;
//           the finaliser makes the exact cut by a mass-weighted radix select
//           and rescans the chunk holding the draw.
// A row the fast path cannot finish exactly (e.g. a flat row whose cut region
// holds more candidates than fit, min-p / typical-p without top-k, top_k above
// FAST_KMAX) is flagged LPS_ROW_DEFERRED in the workspace status and sampled by
// the general kernel, launched after the finaliser with that status as filter.
#pragma once

#include "lps_generic.h"
#include "lps_wave.h"

// Phase marks inside the chunk and finaliser code (LPS_FSTAMP refers to the
// finalised row r of its scope); empty unless a timing build defines them.
#ifndef LPS_STAMP
#define LPS_STAMP(i) ((void)0)
#endif
#ifndef LPS_FSTAMP
#define LPS_FSTAMP(i) ((void)0)
#endif

namespace lps {

constexpr int FT = 256;                 // threads per workgroup
constexpr int FW = FT / 64;             // waves per workgroup
constexpr int FCH_MIN = FT * 32;        // smallest chunk (fp32 and element-read rows): sizes the workspace
constexpr int FAST_KMAX = 256;          // largest top_k / top-N handled by the fast path
constexpr int FCPT = 16;                // finaliser candidates per thread (registers)
constexpr int FCAP = FT * FCPT;         // finaliser candidate capacity (4096)
constexpr int KEPTCAP = 512;            // finaliser kept list
constexpr int HB = 256;                 // histogram bins per chunk (1/8 log2 unit each)
constexpr int HS = 8;                   // bins per log2 unit
constexpr int FB = 256;                 // nucleus level-2 fine bins (one per thread)
constexpr int FSUB_MAX = 5;             // fine bins per coarse bin: at most 2^5
#ifndef LPS_FINE_MIN
#define LPS_FINE_MIN 2048               // level 2 runs when the coarse region may hold more elements
#endif
#ifndef LPS_SELD
#define LPS_SELD 11
#endif
#ifndef LPS_SELDM
#define LPS_SELDM 9
#endif
constexpr int SELD = LPS_SELD;          // count-select digit bits
constexpr int SELB = 1 << SELD;         // count-select histogram bins
constexpr int SELDM = LPS_SELDM;        // mass-select digit bits
constexpr int SELBM = 1 << SELDM;       // mass-select histogram bins
constexpr int HPF = 4;                  // history ids prefetched per thread
constexpr int MAXG = 64;                // chunks per row (V <= 524287)

enum { MODE_GREEDY = 0, MODE_TOPK = 1, MODE_PURE = 2, MODE_NUCLEUS = 3, MODE_DEFER = 4 };
enum { CF_OVERFLOW = 1, CF_HISTORY = 2, CF_SPLIT = 4, CF_REGION = 8 };

struct ChunkSum1 {   // per chunk, for the finaliser
  uint32_t mkey;     // max key of the penalised logits of the chunk (NaN -> 0xFFFFFFFF)
  int32_t amax;      // greedy rows: first index of that key
  double zsum;       // sum over the chunk of exp2(x c - xmax_chunk c), c = log2(e) / T
  int32_t btop;      // histogram top bin (absolute) of the chunk
  uint32_t ninf;     // -inf logits in the chunk (when counted)
  uint32_t flags;    // CF_*
  uint32_t xcc;      // XCD that ran the chunk
};
struct ChunkSum2 {   // published at the end of phase 1
  uint32_t ncand;    // candidates published
  uint32_t flags;    // CF_*
  uint64_t above;    // nucleus: fixed-point mass above the cut region (chunk reference)
  uint32_t nabove;   // nucleus: count above the cut region
  int32_t blo, bhi;  // nucleus: the cut region (absolute bins of 2^-(3 + sub) log2 units), the same in every chunk
  uint32_t sub;
};

struct FParams {
  KParams k;           // per-row parameters and outputs (shared with the general kernel)
  int G;               // chunks per row
  int heavy_first;     // fused kernel, R <= 128: dispatch rows without top-k first
  uint32_t* counters;  // [R * 32]: fused handoff arrivals at [0], nucleus barrier arrivals at [2] and [4]; zero between launches
  int32_t* status;     // [R]
  ChunkSum1* sum1;     // row r at sum1 + r * s_stride
  ChunkSum2* sum2;
  float* hist;         // row r at hist + r * h_stride: G x HB masses (chunk reference), then G x FB fine masses
  uint2* cands;        // row r at cands + r * c_stride: G x PUB (x key, idx), PUB of the chunk variant
  int64_t s_stride, h_stride, c_stride;
};

// LDS.  The chunk phase and the finaliser never overlap in one workgroup.
// Cross-wave exchange slots (each slot is reused only after an intervening barrier).
struct XShared {
  uint64_t xa[FW], xb[FW];
  double xd[FW], xe[FW];
  uint32_t xc[FW], xf[FW], xg[FW], xh[FW];
  double xv[FW][8];
  int32_t mi[32];
  uint64_t m64[8];
  double md[8];
  float mf[4];
};
// Shared block of the chunk phase (NR: logit registers per thread).
template <int NR>
struct CSharedT : XShared {
  uint32_t hc[NR * 128];                  // history counts: 16-bit (fp32 chunks) or 8-bit (packed chunks)
  unsigned long long hm[HB];              // chunk mass histogram, fixed point
  unsigned long long gm[HB];              // nucleus region: merged row histogram, fixed point
  unsigned long long fm[FB];              // nucleus region level 2: chunk fine histogram, fixed point
  double scale[MAXG];                     // nucleus region: chunk -> row reference
  int32_t btop[MAXG];
};
// Shared block of the finaliser.
template <int NR>
struct FSharedT : XShared {
  union {
    uint32_t cnt[2][SELB];                // count select, double-buffered digit histograms
    struct {
      uint32_t cnt[2][SELBM];
      unsigned long long mass[2][SELBM];
    } selm;                               // mass select
    struct {
      uint64_t skey[KEPTCAP];             // (z key << 32) | ~index: larger = earlier in sorted order
      unsigned long long km[KEPTCAP];
      int32_t kidx[KEPTCAP];
      int32_t kord[KEPTCAP];              // sorted position -> slot
      int32_t iord[KEPTCAP];              // index-order position -> slot
      unsigned long long cum[KEPTCAP];
    } k;                                  // kept list
    uint32_t hc[NR * 128];                // rescan history counts
  } x;
  int32_t cidx[FCAP];                     // vocabulary index of candidate slot e of thread t, at e * FT + t
  uint32_t pre[MAXG + 1];                 // candidate prefix over chunks
  double scale[MAXG];                     // chunk -> row reference
  float wm[MAXG];                         // chunk max * c (the chunk's mass reference)
  double keptm[MAXG];                     // kept mass per chunk
  double abvm[MAXG];                      // nucleus: mass above the region per chunk
  unsigned long long keptf[MAXG];         // nucleus: kept candidate mass per chunk, fixed point
};

// ---------------------------------------------------------------------------
// L2-level communication primitives.
// ---------------------------------------------------------------------------
// Counter reads: a compare-and-swap whose compare value a counter never holds,
// so it always fails and returns the current value; it executes at the L2
// (never in a possibly stale L1) and cannot be turned into a plain load.
__device__ __forceinline__ uint32_t ld_l2_u32(uint32_t* p) {
  return atomicCAS(p, 0xFFFFFFFFu, 0xFFFFFFFFu);
}
// Atomic add that returns the old value.
__device__ __forceinline__ uint32_t l2_fetch_add(uint32_t* p, uint32_t v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_stores() { __builtin_amdgcn_s_waitcnt(0); }

// ---------------------------------------------------------------------------
// 256-thread block helpers: wave results meet in one exchange slot, one barrier.
// ---------------------------------------------------------------------------
template <typename T, typename Op>
__device__ __forceinline__ T bcombine(T v, T* slot, Op op) {  // v wave-uniform
  if ((threadIdx.x & 63) == 0) slot[threadIdx.x >> 6] = v;
  __syncthreads();
  return op(op(slot[0], slot[1]), op(slot[2], slot[3]));
}
// Exclusive prefix over the block (thread order) of v; *total gets the sum.
template <typename T>
__device__ __forceinline__ T bscan_excl(T v, T* total, T* slot) {
  const T inc = wscan_incl(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 63) slot[w] = inc;
  __syncthreads();
  T off = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < FW; i++) {
    const T s = slot[i];
    off += (i < w) ? s : (T)0;
    tot += s;
  }
  *total = tot;
  return off + inc - v;
}

// Absolute histogram bin of a logit: floor(x c 8), c = log2(e) / T.
__device__ __forceinline__ int wbin(float x, float c) { return (int)floorf(__fmul_rn(__fmul_rn(x, c), (float)HS)); }

// The chunk-reference mass exp2(w - wm), w <= wm: the hardware exp2 alone.
// Results below 2^-126 flush to zero; they are far below the 2^-44 resolution
// of the fixed-point masses.  The chunk pass and the finaliser's rescan use
// this same function, so their per-chunk sums agree.
__device__ __forceinline__ float chunk_mass(float w, float wm) { return __builtin_amdgcn_exp2f(__fsub_rn(w, wm)); }

// ---------------------------------------------------------------------------
// A thread's share of a chunk, held in 32 registers r[].
//   fp32 in 16-byte vectors of 4, and every dtype read element by element
//   (unaligned rows): 32 logits as fp32 bits; penalties applied in place.
//   bf16 / fp16 in 16-byte vectors of 8 (PACKED): 64 logits, two per register
//   in the input format; slots whose id has a history count are flagged in
//   pmask and penalised (exactly, in fp32) whenever they are read.
// Slot s of thread t is chunk-local index ((s / VEC) * FT + t) * VEC + s % VEC;
// slots at or beyond the chunk end hold -inf.
// ---------------------------------------------------------------------------
template <bool B> struct BoolT { static constexpr bool value = B; };

struct PenArgs {        // penalties of the row, and the chunk's count table in LDS
  const uint32_t* hc;   // 16-bit counts (fp32 chunks) or 8-bit counts (packed chunks)
  float rep, pres, freq;
};

// Packed 16-bit chunks (64 logits per thread, 16384 per chunk) halve the
// workgroup count but add an unpack per pass; measured slower on MI355X, so off.
#ifndef LPS_PACK16
#define LPS_PACK16 0
#endif
template <int DT, int VEC, int NR = 32>
struct Chunk {
  static_assert(NR == 32 || NR == 64, "32 or 64 logit registers per thread");
  static constexpr bool PACKED = LPS_PACK16 && DT != LPS_DTYPE_F32 && VEC == 8 && NR == 32;
  static constexpr int NE = PACKED ? 64 : NR;   // logits per thread (one per fp32 register)
  static constexpr int CH = FT * NE;            // logits per chunk
  static constexpr int NV = NE / VEC;           // vectors per thread
  static constexpr int ES = DT == LPS_DTYPE_F32 ? 4 : 2;
  static constexpr uint32_t NEG16 = DT == LPS_DTYPE_BF16 ? 0xFF80u : 0xFC00u;  // -inf, 16-bit
  uint32_t r[NR];
  static constexpr int PUB = 16 * NR;          // published candidates per chunk
  uint64_t pmask;

  __device__ static __forceinline__ int local(int s) {
    return ((s / VEC) * FT + (int)threadIdx.x) * VEC + (s % VEC);
  }
  __device__ static __forceinline__ float h2f(uint32_t h) {
    return DT == LPS_DTYPE_BF16 ? __uint_as_float(h << 16) : f16_to_f32(h);
  }
  // Logit of slot s (penalised when PEN and the slot is flagged).
  template <bool PEN>
  __device__ __forceinline__ float val(int s, const PenArgs& pa) const {
    if constexpr (!PACKED) {
      return __uint_as_float(r[s]);
    } else {
      const uint32_t w = r[s >> 1];
      float f;
      if constexpr (DT == LPS_DTYPE_BF16) f = __uint_as_float((s & 1) ? (w & 0xFFFF0000u) : (w << 16));
      else f = f16_to_f32((s & 1) ? (w >> 16) : (w & 0xFFFFu));
      if constexpr (PEN) {
        if ((pmask >> s) & 1ull) {
          // this thread's 8-bit counts: one base, a constant offset per slot
          const uint8_t* hb = reinterpret_cast<const uint8_t*>(pa.hc) + threadIdx.x * VEC;
          const uint32_t cnt = hb[(s / VEC) * (FT * VEC) + (s % VEC)];
          f = penalize(f, (int)cnt, pa.rep, pa.pres, pa.freq);
        }
      }
      return f;
    }
  }

  // Every full 16-byte vector load is issued before any value is used
  // (positions clamped to the chunk's last full vector, no branch between the
  // loads); the at most one partial vector of a chunk is read element by element.
  __device__ __forceinline__ void load(const void* row, int lo, int n) {
    pmask = 0ull;
    const char* base = reinterpret_cast<const char*>(row);
    if constexpr (VEC == 1) {
      float raw[NR];
#pragma unroll
      for (int s = 0; s < NR; s++) raw[s] = load1<DT>(row, (int64_t)(lo + min(s * FT + (int)threadIdx.x, n - 1)));
#pragma unroll
      for (int s = 0; s < NR; s++) r[s] = __float_as_uint((s * FT + (int)threadIdx.x) < n ? raw[s] : -INFINITY);
    } else {
      static_assert(VEC * ES == 16, "vector slots are 16 bytes");
      const int lastv = (n / VEC - 1) * VEC;  // start of the last full vector; < 0 when none
      u32x4 raw[NV];
      if (lastv >= 0) {
#pragma unroll
        for (int v = 0; v < NV; v++) {
          const int lv = min((v * FT + (int)threadIdx.x) * VEC, lastv);
          raw[v] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + (int64_t)(lo + lv) * ES));
        }
      }
#pragma unroll
      for (int v = 0; v < NV; v++) {
        const int l0 = (v * FT + (int)threadIdx.x) * VEC;
        uint32_t w[4] = {raw[v].x, raw[v].y, raw[v].z, raw[v].w};
        if (l0 + VEC > n) {  // partial or empty vector
#pragma unroll
          for (int q = 0; q < 4; q++) {
            if constexpr (DT == LPS_DTYPE_F32) {
              w[q] = __float_as_uint(l0 + q < n ? load1<DT>(row, (int64_t)(lo + l0 + q)) : -INFINITY);
            } else {
              const int a = l0 + 2 * q, b = a + 1;
              const uint32_t ha = a < n ? (uint32_t)__builtin_nontemporal_load(
                                              reinterpret_cast<const unsigned short*>(base) + lo + a) : NEG16;
              const uint32_t hb = b < n ? (uint32_t)__builtin_nontemporal_load(
                                              reinterpret_cast<const unsigned short*>(base) + lo + b) : NEG16;
              w[q] = ha | (hb << 16);
            }
          }
        }
        if constexpr (PACKED || DT == LPS_DTYPE_F32) {
#pragma unroll
          for (int q = 0; q < 4; q++) r[v * 4 + q] = w[q];
        } else {  // 16-bit logits kept as fp32 registers
#pragma unroll
          for (int e = 0; e < 8; e++) r[v * 8 + e] = __float_as_uint(h2f((w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu));
        }
      }
    }
  }
  // Slot s to -inf.
  __device__ __forceinline__ void kill(int s) {
    if constexpr (!PACKED) {
      r[s] = __float_as_uint(-INFINITY);
    } else {
      const uint32_t sh = 16u * (uint32_t)(s & 1);
      r[s >> 1] = (r[s >> 1] & ~(0xFFFFu << sh)) | (NEG16 << sh);
    }
  }
  // Illegal ids of [lo, lo + n) to -inf, from the row's legality bits am (one
  // byte read per vector, clamped inside the row; nullptr: every id legal).
  __device__ __forceinline__ void mask(const uint8_t* am, int lo, int n) {
    if (!am) return;
    constexpr int NVS = VEC == 1 ? NR : NV;  // reads per thread
    uint32_t b[NVS];
#pragma unroll
    for (int v = 0; v < NVS; v++) {
      const int l0 = VEC == 1 ? v * FT + (int)threadIdx.x : (v * FT + (int)threadIdx.x) * VEC;
      b[v] = (uint32_t)am[(lo + min(l0, n - 1)) >> 3] >> ((lo + min(l0, n - 1)) & 7);
    }
#pragma unroll
    for (int v = 0; v < NVS; v++) {
#pragma unroll
      for (int e = 0; e < VEC; e++)
        if (!((b[v] >> e) & 1u)) kill(v * VEC + e);
    }
  }
};

// History ids of the row, the first HPF * FT of them, read before the chunk so
// that the table can be built while the chunk loads are in flight (reads stay
// inside the row's history_stride).
struct HistPrefetch {
  int32_t id[HPF];
};
__device__ __forceinline__ void prefetch_history(const int32_t* hrow, int64_t stride, HistPrefetch& hp) {
#pragma unroll
  for (int i = 0; i < HPF; i++) {
    const int jj = i * FT + (int)threadIdx.x;
    hp.id[i] = (hrow && jj < stride) ? hrow[jj] : -1;
  }
}
// Counts of the history ids inside [lo, lo + n), BITS (16 or 8) bits per id in
// hc (WORDS words: WORDS * 32 / BITS ids, at least n).  Returns false when a
// count does not fit (16-bit: hlen > 65535 is refused by the caller; 8-bit: a
// count reached 255).  Ends with a barrier.
template <int BITS, int WORDS>
__device__ __forceinline__ bool build_counts(uint32_t (&hc)[WORDS], const int32_t* hrow, int hlen, const HistPrefetch& hp,
                                             int lo, int n, XShared& S) {
  constexpr int PER = 32 / BITS;  // ids per word
  static_assert(WORDS % (4 * FT) == 0, "whole 16-byte stores per thread");
  u32x4* h4 = reinterpret_cast<u32x4*>(hc);
#pragma unroll
  for (int i = 0; i < WORDS / 4 / FT; i++) h4[i * FT + threadIdx.x] = u32x4{0u, 0u, 0u, 0u};
  if (threadIdx.x == 0) S.mi[30] = 0;
  __syncthreads();
  bool sat = false;
  auto add = [&](int id) {
    if (id >= lo && id < lo + n) {
      const int l = id - lo;
      const int sh = BITS * (l % PER);
      const uint32_t old = atomicAdd(&hc[l / PER], 1u << sh);
      if (BITS == 8 && ((old >> sh) & 0xFFu) >= 254u) sat = true;
    }
  };
#pragma unroll
  for (int i = 0; i < HPF; i++)
    if (i * FT + (int)threadIdx.x < hlen) add(hp.id[i]);
  for (int jj = HPF * FT + (int)threadIdx.x; jj < hlen; jj += FT) add(hrow[jj]);
  if (sat) S.mi[30] = 1;
  __syncthreads();
  return S.mi[30] == 0;
}
// fp32 chunks: apply the 16-bit count table in place.
template <int DT, int VEC, int NR>
__device__ __forceinline__ void apply_counts(Chunk<DT, VEC, NR>& C, int n, const PenArgs& pa) {
  static_assert(!Chunk<DT, VEC, NR>::PACKED, "in-place penalties are for fp32 registers");
  constexpr int NV = Chunk<DT, VEC, NR>::NV;
#pragma unroll
  for (int v = 0; v < NV; v++) {
    const int l0 = (v * FT + (int)threadIdx.x) * VEC;
    if (l0 >= n) continue;
    uint32_t w[(VEC + 1) / 2];
    if constexpr (VEC == 8) {
      const u32x4 q = *reinterpret_cast<const u32x4*>(pa.hc + (l0 >> 1));
      w[0] = q.x; w[1] = q.y; w[2] = q.z; w[3] = q.w;
    } else if constexpr (VEC == 4) {
      const uint2 q = *reinterpret_cast<const uint2*>(pa.hc + (l0 >> 1));
      w[0] = q.x; w[1] = q.y;
    } else {
      w[0] = (pa.hc[l0 >> 1] >> (16 * (l0 & 1))) & 0xFFFFu;
    }
    uint32_t any = 0;
#pragma unroll
    for (int i = 0; i < (VEC + 1) / 2; i++) any |= w[i];
    if (!any) continue;
#pragma unroll
    for (int e = 0; e < VEC; e++) {
      const uint32_t cnt = VEC == 1 ? w[0] : ((w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
      const int s = v * VEC + e;
      if (cnt) C.r[s] = __float_as_uint(penalize(__uint_as_float(C.r[s]), (int)cnt, pa.rep, pa.pres, pa.freq));
    }
  }
}
// Packed chunks: flag the slots with an 8-bit count.
template <int DT, int VEC, int NR>
__device__ __forceinline__ void mark_counts(Chunk<DT, VEC, NR>& C, int n, const PenArgs& pa) {
  static_assert(Chunk<DT, VEC, NR>::PACKED, "flags are for packed registers");
  constexpr int NV = Chunk<DT, VEC, NR>::NV;
  uint64_t m = 0;
#pragma unroll
  for (int v = 0; v < NV; v++) {
    const int l0 = (v * FT + (int)threadIdx.x) * VEC;  // 8 ids = 2 words
    const uint2 q = *reinterpret_cast<const uint2*>(pa.hc + (l0 >> 2));
    const uint64_t c = ((uint64_t)q.y << 32) | q.x;
#pragma unroll
    for (int e = 0; e < 8; e++) m |= ((c >> (8 * e)) & 0xFFull) ? (1ull << (v * 8 + e)) : 0ull;
  }
  (void)n;
  C.pmask = m;
}

// Smallest x whose fl(x / T) equals fl(x0 / T) (x0 finite, T > 0): the lower end
// of the division-collision group of x0, so that "z >= fl(x0 / T)" is
// "x >= result" for every x.  The group is searched at most 64 keys down, all
// at once: lane l of the wave tests the step from l to l + 1 keys below x0,
// and the group ends at the first failing lane.  x0 is wave-uniform and every
// lane of the wave calls this.
__device__ __forceinline__ float collision_lo(float x0, float T) {
  const float q = __fdiv_rn(x0, T);
  const uint32_t k0 = f2key(x0);
  const uint32_t k = k0 - (threadIdx.x & 63u);
  const uint64_t fail = wballot(!(k > kNegInfKey + 1u && __fdiv_rn(key2f(k - 1u), T) == q));
  return key2f(k0 - (fail ? (uint32_t)__builtin_ctzll(fail) : 64u));
}

// ---------------------------------------------------------------------------
// Selections over register-resident candidates: thread t holds candidate
// e * FT + t in slot e, present when e < np.  MSB-first radix over
// key - kmin; the digit histograms are double-buffered so that one level costs
// three barriers (histogram, scan, result).  Each thread scans SELB / FT (or
// SELBM / FT) consecutive bins, highest digit first.
// ---------------------------------------------------------------------------
struct SelLevel {
  uint32_t base;   // kmin
  int bits;        // bit length of kmax - kmin
};
// Key range of the present candidates; clears histogram buffer 0 (nb bins of
// cnt0, and of m0 when given) before its barrier.
template <class FS>
__device__ __forceinline__ SelLevel sel_range(const uint32_t (&ck)[FCPT], int np, uint32_t* cnt0, int nb,
                                              unsigned long long* m0, FS& S) {
  uint32_t mn = 0xFFFFFFFFu, mx = 0;
#pragma unroll
  for (int e = 0; e < FCPT; e++)
    if (e < np) { mn = ck[e] < mn ? ck[e] : mn; mx = ck[e] > mx ? ck[e] : mx; }
  mn = wmin(mn);
  mx = wmax(mx);
  if ((threadIdx.x & 63) == 0) { S.xc[threadIdx.x >> 6] = mn; S.xf[threadIdx.x >> 6] = mx; }
  for (int i = threadIdx.x; i < nb; i += FT) {
    cnt0[i] = 0u;
    if (m0) m0[i] = 0ull;
  }
  __syncthreads();
  mn = min(min(S.xc[0], S.xc[1]), min(S.xc[2], S.xc[3]));
  mx = max(max(S.xf[0], S.xf[1]), max(S.xf[2], S.xf[3]));
  SelLevel L;
  L.base = mn;
  L.bits = mx > mn ? 32 - __clz(mx - mn) : 0;
  return L;
}

// kk-th largest present key (1 <= kk <= number present).
template <class FS>
__device__ __forceinline__ uint32_t sel_count(const uint32_t (&ck)[FCPT], int np, uint32_t kk, FS& S) {
  auto& H = S.x.cnt;
  const SelLevel L = sel_range(ck, np, H[0], SELB, nullptr, S);
  if (L.bits == 0) return L.base;
  constexpr int PER = SELB / FT;
  uint32_t hi = 0;      // digits matched so far
  int top = L.bits;     // bits not yet resolved: [0, top)
  uint32_t need = kk;
  int buf = 0;
  while (top > 0) {
    const int sh = top > SELD ? top - SELD : 0;
    const int dw = top - sh;
#pragma unroll
    for (int e = 0; e < FCPT; e++) {
      if (e < np) {
        const uint32_t d = ck[e] - L.base;
        const uint32_t up = top >= 32 ? 0u : (d >> top);
        if (up == hi) atomicAdd(&H[buf][(d >> sh) & ((1u << dw) - 1u)], 1u);
      }
    }
    for (int i = threadIdx.x; i < SELB; i += FT) H[buf ^ 1][i] = 0u;  // next level's buffer
    __syncthreads();
    uint32_t c[PER], loc = 0;
#pragma unroll
    for (int i = 0; i < PER; i++) { c[i] = H[buf][SELB - 1 - (PER * (int)threadIdx.x + i)]; loc += c[i]; }
    uint32_t tot;
    uint32_t ex = bscan_excl<uint32_t>(loc, &tot, S.xg);
#pragma unroll
    for (int i = 0; i < PER; i++) {
      if (ex < need && need <= ex + c[i]) { S.mi[0] = SELB - 1 - (PER * (int)threadIdx.x + i); S.mi[1] = (int)ex; }
      ex += c[i];
    }
    __syncthreads();
    hi = (hi << dw) | (uint32_t)S.mi[0];
    need -= (uint32_t)S.mi[1];
    top = sh;
    buf ^= 1;
  }
  __syncthreads();
  return L.base + hi;
}

// Mass-weighted select: the largest present key v with A + mass(key >= v) > P,
// requiring A <= P < A + total (ok = 0 otherwise).  above = A + mass(key > v);
// ceq / meq = count and mass of key == v.  mass(e) gives a candidate's mass.
struct MassSel {
  uint32_t key;
  uint64_t above;
  uint32_t ceq;
  uint64_t meq;
  int ok;
};
template <typename MF, class FS>
__device__ __forceinline__ MassSel sel_mass(const uint32_t (&ck)[FCPT], int np, MF mass, uint64_t A, uint64_t P,
                                            FS& S) {
  MassSel ms{0, A, 0, 0, 0};
  auto& H = S.x.selm;
  const SelLevel L = sel_range(ck, np, H.cnt[0], SELBM, H.mass[0], S);
  constexpr int PER = SELBM / FT;
  uint32_t hi = 0;
  int top = L.bits;
  int buf = 0;
  for (;;) {
    const int sh = top > SELDM ? top - SELDM : 0;
    const int dw = top - sh;
    if (threadIdx.x == 0) S.mi[0] = -1;
#pragma unroll
    for (int e = 0; e < FCPT; e++) {
      if (e < np) {
        const uint32_t d = ck[e] - L.base;
        const uint32_t up = top >= 32 ? 0u : (d >> top);
        if (up == hi) {
          const uint32_t b = dw > 0 ? ((d >> sh) & ((1u << dw) - 1u)) : 0u;
          atomicAdd(&H.cnt[buf][b], 1u);
          // the mass is recomputed at every level: hoisted out of the level
          // loop, the 16 64-bit masses would hold 32 more registers for the
          // whole select and cost the fused kernel a workgroup per CU
          uint32_t kv = ck[e];
          asm volatile("" : "+v"(kv));
          const uint64_t m = mass(kv);
          if (m) atomicAdd(&H.mass[buf][b], (unsigned long long)m);
        }
      }
    }
    for (int i = threadIdx.x; i < SELBM; i += FT) { H.cnt[buf ^ 1][i] = 0u; H.mass[buf ^ 1][i] = 0ull; }
    __syncthreads();
    uint32_t c[PER];
    uint64_t m[PER], loc = 0;
#pragma unroll
    for (int i = 0; i < PER; i++) {
      const int b = SELBM - 1 - (PER * (int)threadIdx.x + i);
      c[i] = H.cnt[buf][b];
      m[i] = H.mass[buf][b];
      loc += m[i];
    }
    uint64_t tot;
    uint64_t ex = ms.above + bscan_excl<uint64_t>(loc, &tot, S.xa);
#pragma unroll
    for (int i = 0; i < PER; i++) {
      if (ex <= P && P < ex + m[i]) {
        S.mi[0] = SELBM - 1 - (PER * (int)threadIdx.x + i);
        S.mi[1] = (int)c[i];
        S.m64[0] = ex;
        S.m64[1] = m[i];
      }
      ex += m[i];
    }
    __syncthreads();
    if (S.mi[0] < 0) { __syncthreads(); return ms; }
    hi = (hi << dw) | (uint32_t)S.mi[0];
    ms.above = S.m64[0];
    ms.ceq = (uint32_t)S.mi[1];
    ms.meq = S.m64[1];
    top = sh;
    buf ^= 1;
    __syncthreads();  // S.mi[0] is reset by the next level
    if (top == 0) break;
  }
  ms.key = L.base + hi;
  ms.ok = 1;
  return ms;
}

}  // namespace lps
