// Fast row sampler: every row is split into G chunks of 8192 logits, one
// 256-thread workgroup per chunk, the chunk held in registers for the whole
// kernel (the logits are read from HBM exactly once).
//
// Placement: workgroup ids are dispatched round-robin over the XCDs, so chunk
// workgroups of a row are given ids congruent modulo 8.  They then share one
// L2, and their partial results meet there: a workgroup publishes with plain
// stores (write-through L1 -> L2), waits for them, and counts its arrival with
// a global atomic; the last arrival of a row finalises it, reading the
// partials with L1-bypassing loads.  No agent-scope release fence (an L2
// write-back) is ever issued.
//
// Row modes (decided per row from its parameters):
//   GREEDY  T <= 0: first argmax (plus logprobs).
//   TOPK    0 < top_k <= FAST_KMAX: each chunk publishes its exact local
//           top-k' (k' = max(k, n_top)) candidates; the finaliser selects the
//           global k-th value, applies top-p / min-p / typical-p on the small
//           kept set and draws from it.
//   PURE    top_k off and no other filter: no cut; the finaliser picks the
//           chunk holding the draw from per-chunk masses and rescans it.
//   NUCLEUS top_k off, top_p < 1: chunks publish a fine mass histogram, pass
//           one intra-XCD barrier, derive the same global cut region, publish
//           the candidates inside it plus their exact mass above it; the
//           finaliser makes the exact cut and rescans the chunk holding the
//           draw.
// A row the fast path cannot finish exactly (e.g. a flat row whose cut region
// holds more candidates than fit, min-p / typical-p without top-k, top_k above
// FAST_KMAX) is flagged LPS_ROW_DEFERRED and finished by the general kernel.
#pragma once

#include "lps_generic.h"

namespace lps {

constexpr int FT = 256;                 // threads per workgroup
constexpr int FW = FT / 64;             // waves per workgroup
constexpr int FE = 32;                  // elements per thread
constexpr int FCH = FT * FE;            // chunk size (8192)
constexpr int FAST_KMAX = 256;          // largest top_k / top-N handled by the fast path
constexpr int LCAP = 1024;              // local candidate list (per workgroup)
constexpr int PUBCAP = 512;             // published candidates per chunk
constexpr int KEPTCAP = 512;            // finaliser kept list
constexpr int HB = 256;                 // histogram bins per chunk (1/8 log2 unit each)
constexpr int HS = 8;                   // bins per log2 unit
constexpr int HU = HB / HS;             // histogram units (1 log2 unit each)
constexpr int FHASH = 1024;             // per-chunk history hash slots
constexpr int FHASH_MAX = 768;          // distinct ids a chunk table holds
constexpr int FBITS = FCH / 32;         // per-chunk history bitmap words
constexpr int MAXG = 64;                // chunks per row (V <= 524287)

enum { MODE_GREEDY = 0, MODE_TOPK = 1, MODE_PURE = 2, MODE_NUCLEUS = 3, MODE_DEFER = 4 };
enum { CF_OVERFLOW = 1, CF_HISTORY = 2, CF_SPLIT = 4, CF_REGION = 8 };
constexpr int32_t LPS_ROW_DEFERRED = 8;  // internal: finished by the general kernel

struct ChunkSum1 {   // published before the barrier / handoff
  uint32_t mkey;     // max key of the penalised logits of the chunk
  int32_t amax;      // its first index
  float zsum;        // sum over the chunk of exp2((x - xmax_chunk) * c)
  int32_t btop;      // histogram top bin (absolute) of the chunk
  uint32_t ninf;     // -inf logits in the chunk
  uint32_t flags;    // CF_*
  uint32_t xcc;      // XCD the chunk ran on
  uint32_t pad;
};
struct ChunkSum2 {   // published at the handoff
  uint32_t ncand;    // candidates published
  uint32_t flags;    // CF_*
  uint64_t above;    // nucleus: fixed-point mass above the cut region (chunk reference)
  uint32_t nabove;   // nucleus: count above the cut region
  uint32_t pad[3];
};

struct FParams {
  KParams k;           // per-row parameters and outputs (shared with the general kernel)
  int G;               // chunks per row
  uint32_t* counters;  // [R * 32]: u64 handoff word at [0..1], barrier arrivals at [2]
  int32_t* status;     // [R]
  ChunkSum1* sum1;     // row r at sum1 + r * s_stride
  ChunkSum2* sum2;
  float* hist;         // row r at hist + r * h_stride: G x (HB fine + HU unit) masses
  uint2* cands;        // row r at cands + r * c_stride: G x PUBCAP (key, idx)
  int64_t s_stride, h_stride, c_stride;
};

struct FShared {
  int32_t hkey[FHASH];
  uint32_t hcnt[FHASH / 2];  // two 16-bit counts per word
  uint32_t bits[FBITS];
  uint32_t rh[256];          // radix digit histogram
  union {
    struct {                 // chunk phase
      uint64_t hm[HB];       // fixed-point histogram masses (chunk reference)
      uint32_t tmax[FT];
      union {
        struct {
          uint32_t lkey[LCAP];
          int32_t lidx[LCAP];
        } l;
        struct {             // nucleus region search
          double scale[MAXG];
          int32_t btop[MAXG];
          double zs[MAXG];
          double um[HU + 2];
          double bm[HS];
        } n;
      } v;
    } c;
    struct {                 // finaliser
      uint32_t kkey[KEPTCAP];  // z keys
      uint32_t kx[KEPTCAP];    // x keys
      int32_t kidx[KEPTCAP];
      uint64_t km[KEPTCAP];
      int32_t kord[KEPTCAP];
      int32_t iord[KEPTCAP];
      uint64_t cum[KEPTCAP];
      uint32_t cmk[MAXG];      // per-chunk max key
      int32_t cam[MAXG];       // per-chunk argmax
      float czs[MAXG];         // per-chunk zsum
      uint32_t cnc[MAXG];      // per-chunk published candidates
      uint32_t pre[MAXG];      // candidate prefix
      uint32_t cfl[MAXG];
      uint32_t cninf[MAXG];
      uint32_t ctie[MAXG];     // kept ties in chunks before q
      double scale[MAXG];      // chunk reference -> row reference
      double keptm[MAXG];      // kept mass per chunk
      double abv[MAXG];
      uint32_t nab[MAXG];
      unsigned long long keptf[MAXG];  // kept candidate mass per chunk (fixed point)
      uint32_t keptc[MAXG];            // kept candidate count per chunk
    } f;
  } u;
  uint64_t r64[FW];
  double rd[FW];
  uint32_t r32[FW];
  int32_t mi[16];
  uint64_t m64[8];
  float mf[8];
  double md[8];
};

// ---------------------------------------------------------------------------
// L2-level communication primitives.
// ---------------------------------------------------------------------------
// XCD id of the executing wave: hardware register HW_REG_XCC_ID (20), bits 0-3.
__device__ __forceinline__ uint32_t xcc_id() {
  return (uint32_t)__builtin_amdgcn_s_getreg(20 | (0 << 6) | ((4 - 1) << 11)) & 0xFu;
}
// Counter reads: a compare-and-swap whose compare value a counter never holds,
// so it always fails and returns the current value; it executes at the L2
// (never in a possibly stale L1) and cannot be turned into a plain load.
__device__ __forceinline__ uint32_t ld_l2_u32(uint32_t* p) {
  return atomicCAS(p, 0xFFFFFFFFu, 0xFFFFFFFFu);
}
// Atomic adds that return the old value.
__device__ __forceinline__ uint64_t l2_fetch_add64(uint64_t* p, uint64_t v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t l2_fetch_add(uint32_t* p, uint32_t v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_stores() { __builtin_amdgcn_s_waitcnt(0); }

// ---------------------------------------------------------------------------
// 256-thread block helpers.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t fmax_u64(uint64_t v, FShared& S) {
  v = wave_max(v);
  if ((threadIdx.x & 63) == 0) S.r64[threadIdx.x >> 6] = v;
  __syncthreads();
  uint64_t r = S.r64[0];
#pragma unroll
  for (int i = 1; i < FW; i++) r = S.r64[i] > r ? S.r64[i] : r;
  __syncthreads();
  return r;
}
__device__ __forceinline__ uint64_t fsum_u64(uint64_t v, FShared& S) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) S.r64[threadIdx.x >> 6] = v;
  __syncthreads();
  uint64_t r = 0;
#pragma unroll
  for (int i = 0; i < FW; i++) r += S.r64[i];
  __syncthreads();
  return r;
}
__device__ __forceinline__ uint32_t fsum_u32(uint32_t v, FShared& S) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) S.r32[threadIdx.x >> 6] = v;
  __syncthreads();
  uint32_t r = 0;
#pragma unroll
  for (int i = 0; i < FW; i++) r += S.r32[i];
  __syncthreads();
  return r;
}
__device__ __forceinline__ double fsum_f64(double v, FShared& S) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) S.rd[threadIdx.x >> 6] = v;
  __syncthreads();
  double r = 0;
#pragma unroll
  for (int i = 0; i < FW; i++) r += S.rd[i];
  __syncthreads();
  return r;
}
template <typename T>
__device__ __forceinline__ T fexcl_scan(T v, T* total, T* scratch) {
  T inc = wave_incl_scan(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 63) scratch[w] = inc;
  __syncthreads();
  T off = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < FW; i++) {
    T s = scratch[i];
    off += (i < w) ? s : (T)0;
    tot += s;
  }
  __syncthreads();
  *total = tot;
  return off + inc - v;
}

// ---------------------------------------------------------------------------
// Per-chunk history table (counts of distinct in-range ids).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t fhash(int id) { return ((uint32_t)id * 2654435761u) >> (32 - 10); }

struct FPen {
  bool active;
  float rep, pres, freq;
  int lo;
  const FShared* S;
  __device__ __forceinline__ int count(int id) const {
    uint32_t s = fhash(id);
    for (int p = 0; p < FHASH; p++) {
      const int k = S->hkey[s];
      if (k == id) return (int)((S->hcnt[s >> 1] >> ((s & 1) * 16)) & 0xFFFFu);
      if (k < 0) return 0;
      s = (s + 1) & (FHASH - 1);
    }
    return 0;
  }
  // x holds VEC consecutive logits starting at absolute id i0 (inside the chunk).
  template <int VEC>
  __device__ __forceinline__ void apply(int i0, float (&x)[VEC]) const {
    if (!active) return;
    const int l = i0 - lo;
    uint32_t w = S->bits[l >> 5] >> (l & 31);
    if (VEC < 32) w &= (1u << VEC) - 1u;
    if (!w) return;
#pragma unroll
    for (int e = 0; e < VEC; e++)
      if ((w >> e) & 1u) {
        const int c = count(i0 + e);
        if (c) x[e] = penalize(x[e], c, rep, pres, freq);
      }
  }
};

// Builds the table for ids in [lo, lo + n); returns false on overflow.
__device__ bool build_pen(FShared& S, const int32_t* h, int hlen, int lo, int n) {
  for (int i = threadIdx.x; i < FHASH; i += FT) S.hkey[i] = -1;
  for (int i = threadIdx.x; i < FHASH / 2; i += FT) S.hcnt[i] = 0u;
  for (int i = threadIdx.x; i < FBITS; i += FT) S.bits[i] = 0u;
  __syncthreads();
  uint32_t fail = 0;
  for (int j = threadIdx.x; j < hlen; j += FT) {
    const int id = h[j];
    if (id < lo || id >= lo + n) continue;
    uint32_t s = fhash(id);
    bool done = false;
    for (int p = 0; p < FHASH && !done; p++) {
      const int old = atomicCAS(&S.hkey[s], -1, id);
      if (old == -1 || old == id) {
        atomicAdd(&S.hcnt[s >> 1], 1u << ((s & 1) * 16));
        done = true;
      } else {
        s = (s + 1) & (FHASH - 1);
      }
    }
    if (!done) fail = 1;
    atomicOr(&S.bits[(id - lo) >> 5], 1u << ((id - lo) & 31));
  }
  __syncthreads();
  uint32_t used = 0;
  for (int i = threadIdx.x; i < FHASH; i += FT) used += S.hkey[i] >= 0 ? 1u : 0u;
  used = fsum_u32(used, S);
  fail = fsum_u32(fail, S);
  return fail == 0 && used <= FHASH_MAX;
}

// Chunk load: element slot (v, e) of thread t is chunk-local index
// (v * FT + t) * VEC + e.
template <int DT, int VEC>
__device__ __forceinline__ void load_chunk(const void* row, int lo, int n, const FPen& pen, float (&x)[FE]) {
  constexpr int NV = FE / VEC;
#pragma unroll
  for (int v = 0; v < NV; v++) {
    const int l0 = (v * FT + (int)threadIdx.x) * VEC;
    float t[VEC];
    if (l0 + VEC <= n) {
      loadv<DT, VEC>(row, (int64_t)(lo + l0), t);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; e++) t[e] = (l0 + e < n) ? load1<DT>(row, (int64_t)(lo + l0 + e)) : -INFINITY;
    }
    if (l0 < n) pen.apply<VEC>(lo + l0, t);
#pragma unroll
    for (int e = 0; e < VEC; e++) x[v * VEC + e] = t[e];
  }
}
template <int VEC>
__device__ __forceinline__ int slot_local(int s) {  // register slot -> chunk-local index
  return ((s / VEC) * FT + (int)threadIdx.x) * VEC + (s % VEC);
}

// Smallest x whose fl(x / T) equals fl(x0 / T) (x0 finite, T > 0): the lower end
// of the division-collision group of x0, so that "z >= fl(x0 / T)" is
// "x >= result" for every x.
__device__ __forceinline__ float collision_lo(float x0, float T) {
  const float q = __fdiv_rn(x0, T);
  float x = x0;
  for (int i = 0; i < 64; i++) {
    const uint32_t k = f2key(x);
    if (k <= kNegInfKey + 1u) break;
    const float y = key2f(k - 1u);
    if (__fdiv_rn(y, T) != q) break;
    x = y;
  }
  return x;
}

// kk-th largest (1-based, counting multiplicity, kk <= n) of n keys produced by
// key_at(i), i in [0, n), by MSB-first 8-bit radix select with S.rh.
template <typename KA>
__device__ uint32_t block_select_kth(int n, uint32_t kk, KA key_at, FShared& S) {
  uint32_t prefix = 0, hmask = 0;
  for (int l = 0; l < 4; l++) {
    const int sh = 24 - 8 * l;
    S.rh[threadIdx.x] = 0;
    if (threadIdx.x == 0) { S.mi[0] = 0; S.mi[1] = 0; }
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += FT) {
      const uint32_t k = key_at(i);
      if ((k & hmask) == prefix) atomicAdd(&S.rh[(k >> sh) & 255u], 1u);
    }
    __syncthreads();
    // descending: thread t owns bin 255 - t
    const uint32_t c = S.rh[255 - threadIdx.x];
    uint32_t tot;
    const uint32_t ex = fexcl_scan<uint32_t>(c, &tot, S.r32);
    if (ex < kk && kk <= ex + c) { S.mi[0] = 255 - (int)threadIdx.x; S.mi[1] = (int)ex; }
    __syncthreads();
    prefix |= (uint32_t)S.mi[0] << sh;
    kk -= (uint32_t)S.mi[1];
    hmask |= 255u << sh;
    __syncthreads();
  }
  return prefix;
}

// Mass-weighted MSB-first radix select over n candidates produced by cand(i)
// -> (key, mass): the largest key v with A + mass(key >= v) > P.  Requires
// A <= P < A + total mass (ok = 0 otherwise).  above = A + mass(key > v).
struct MassSel {
  uint32_t key;
  uint64_t above;
  uint32_t ceq;
  uint64_t meq;
  int ok;
};
template <typename CA>
__device__ MassSel block_mass_select(int n, uint64_t A, uint64_t P, CA cand, uint64_t* mh, FShared& S) {
  MassSel ms{0, A, 0, 0, 1};
  uint32_t prefix = 0, hmask = 0;
  for (int l = 0; l < 4; l++) {
    const int sh = 24 - 8 * l;
    S.rh[threadIdx.x] = 0;
    mh[threadIdx.x] = 0;
    if (threadIdx.x == 0) S.mi[0] = -1;
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += FT) {
      uint32_t k;
      uint64_t m;
      cand(i, &k, &m);
      if ((k & hmask) == prefix) {
        atomicAdd(&S.rh[(k >> sh) & 255u], 1u);
        if (m) atomicAdd((unsigned long long*)&mh[(k >> sh) & 255u], (unsigned long long)m);
      }
    }
    __syncthreads();
    const int b = 255 - (int)threadIdx.x;
    const uint32_t c = S.rh[b];
    const uint64_t m = mh[b];
    uint64_t tot;
    const uint64_t ex = fexcl_scan<uint64_t>(m, &tot, S.r64);
    if (ms.above + ex <= P && P < ms.above + ex + m) {
      S.mi[0] = b;
      S.mi[1] = (int)c;
      S.m64[0] = ex;
      S.m64[1] = m;
    }
    __syncthreads();
    if (S.mi[0] < 0) { ms.ok = 0; return ms; }
    prefix |= (uint32_t)S.mi[0] << sh;
    ms.above += S.m64[0];
    ms.ceq = (uint32_t)S.mi[1];
    ms.meq = S.m64[1];
    hmask |= 255u << sh;
    __syncthreads();
  }
  ms.key = prefix;
  return ms;
}

}  // namespace lps
