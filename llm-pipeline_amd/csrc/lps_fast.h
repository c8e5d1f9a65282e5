// Fast row sampler: every row is split into G chunks of 8192 logits, one
// 256-thread workgroup per chunk, the chunk held in registers (the logits are
// read from HBM once; only the chunk that holds the draw of a nucleus / pure
// row is read a second time, by the row's finaliser, normally from the L2).
//
// Placement: workgroup ids are dispatched round-robin over the XCDs, so chunk
// workgroups of a row are given ids congruent modulo 8.  They then share one
// L2, and their partial results meet there: a workgroup publishes with plain
// stores (write-through L1 -> L2), waits for them, and counts its arrival with
// a global atomic; the last arrival of a row finalises it.  No agent-scope
// release fence (an L2 write-back) is ever issued.  A row whose chunks were
// not all seen on one XCD is finished by the general algorithm instead.
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
//           one intra-XCD barrier, all derive the same cut region (the bins
//           whose cumulative mass meets top_p within a tolerance band), and
//           publish the candidates inside it plus their exact mass above it;
//           the finaliser makes the exact cut by a mass-weighted radix select
//           and rescans the chunk holding the draw.
// A row the fast path cannot finish exactly (e.g. a flat row whose cut region
// holds more candidates than fit, min-p / typical-p without top-k, top_k above
// FAST_KMAX) is flagged LPS_ROW_DEFERRED and runs the general algorithm in the
// same workgroup.
#pragma once

#include "lps_generic.h"
#include "lps_wave.h"

// Phase marks inside the fast kernel; empty unless a timing build defines it.
#ifndef LPS_STAMP
#define LPS_STAMP(i) ((void)0)
#endif

namespace lps {

constexpr int FT = 256;                 // threads per workgroup
constexpr int FW = FT / 64;             // waves per workgroup
constexpr int FE = 32;                  // elements per thread
constexpr int FCH = FT * FE;            // chunk size (8192)
constexpr int FAST_KMAX = 256;          // largest top_k / top-N handled by the fast path
constexpr int PUBCAP = 512;             // published candidates per chunk
constexpr int FCPT = 16;                // finaliser candidates per thread (registers)
constexpr int FCAP = FT * FCPT;         // finaliser candidate capacity (4096)
constexpr int KEPTCAP = 512;            // finaliser kept list
constexpr int HB = 256;                 // histogram bins per chunk (1/8 log2 unit each)
constexpr int HS = 8;                   // bins per log2 unit
constexpr int SELD = 11;                // select digit bits
constexpr int SELB = 1 << SELD;         // select histogram bins
constexpr int HPF = 4;                  // history ids prefetched per thread
constexpr int MAXG = 64;                // chunks per row (V <= 524287)

enum { MODE_GREEDY = 0, MODE_TOPK = 1, MODE_PURE = 2, MODE_NUCLEUS = 3, MODE_DEFER = 4 };
enum { CF_OVERFLOW = 1, CF_HISTORY = 2, CF_SPLIT = 4, CF_REGION = 8 };
constexpr int32_t LPS_ROW_DEFERRED = 8;  // internal: finished by the general algorithm

struct ChunkSum1 {   // published before the barrier / handoff
  uint32_t mkey;     // max key of the penalised logits of the chunk (NaN -> 0xFFFFFFFF)
  int32_t amax;      // greedy rows: first index of that key
  float zsum;        // sum over the chunk of exp2(x c - xmax_chunk c), c = log2(e) / T
  int32_t btop;      // histogram top bin (absolute) of the chunk
  uint32_t ninf;     // -inf logits in the chunk (when counted)
  uint32_t flags;    // CF_*
  uint32_t pad[2];
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
  float* hist;         // row r at hist + r * h_stride: G x HB masses (chunk reference)
  uint2* cands;        // row r at cands + r * c_stride: G x PUBCAP (x key, idx)
  int64_t s_stride, h_stride, c_stride;
};

// LDS.  The chunk phase and the finaliser never overlap in one workgroup.
struct FShared {
  union {
    struct {                              // chunk phase
      uint32_t hc[FCH / 2];               // history counts, two 16-bit counts per word
      unsigned long long hm[HB];          // chunk mass histogram, fixed point
      double scale[MAXG];                 // nucleus region: chunk -> row reference
      int32_t btop[MAXG];
    } c;
    struct {                              // finaliser
      union {
        struct {
          uint32_t cnt[SELB];
          unsigned long long mass[SELB];
        } sel;                            // select histograms
        struct {
          uint32_t kkey[KEPTCAP];         // z keys
          uint32_t kx[KEPTCAP];           // x keys
          int32_t kidx[KEPTCAP];
          unsigned long long km[KEPTCAP];
          int32_t kord[KEPTCAP];          // sorted position -> slot
          int32_t iord[KEPTCAP];          // index-order position -> slot
          unsigned long long cum[KEPTCAP];
        } k;                              // kept list
        uint32_t hc[FCH / 2];             // rescan history counts
      } x;
      uint32_t pre[MAXG + 1];             // candidate prefix over chunks
      double scale[MAXG];                 // chunk -> row reference
      double keptm[MAXG];                 // kept mass per chunk
      double abvm[MAXG];                  // nucleus: mass above the region per chunk
      unsigned long long epre[MAXG];      // nucleus: kept candidate mass prefix at chunk starts
      unsigned long long eend[MAXG];      // ... and after each chunk's last candidate
    } f;
  } u;
  // cross-wave exchange slots (each slot is reused only after an intervening barrier)
  uint64_t xa[FW], xb[FW];
  double xd[FW], xe[FW];
  uint32_t xc[FW], xf[FW], xg[FW], xh[FW];
  double xv[FW][8];
  int32_t mi[32];
  uint64_t m64[8];
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

// ---------------------------------------------------------------------------
// Chunk loads and the per-chunk history count table.
// ---------------------------------------------------------------------------
// Element slot (v, e) of thread t is chunk-local index (v * FT + t) * VEC + e;
// slots at or beyond n hold -inf.
template <int DT, int VEC>
__device__ __forceinline__ void load_chunk(const void* row, int lo, int n, float (&x)[FE]) {
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
#pragma unroll
    for (int e = 0; e < VEC; e++) x[v * VEC + e] = t[e];
  }
}
template <int VEC>
__device__ __forceinline__ int slot_local(int s) {  // register slot -> chunk-local index
  return ((s / VEC) * FT + (int)threadIdx.x) * VEC + (s % VEC);
}

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
// Counts of the history ids inside [lo, lo + n) (hlen <= 65535).  Ends with a barrier.
__device__ __forceinline__ void build_counts(uint32_t* hc, const int32_t* hrow, int hlen, const HistPrefetch& hp,
                                             int lo, int n) {
  u32x4* h4 = reinterpret_cast<u32x4*>(hc);
#pragma unroll
  for (int i = 0; i < FCH / 8 / FT; i++) h4[i * FT + threadIdx.x] = u32x4{0u, 0u, 0u, 0u};
  __syncthreads();
#pragma unroll
  for (int i = 0; i < HPF; i++) {
    const int jj = i * FT + (int)threadIdx.x;
    const int id = hp.id[i];
    if (jj < hlen && id >= lo && id < lo + n) atomicAdd(&hc[(id - lo) >> 1], 1u << (16 * ((id - lo) & 1)));
  }
  for (int jj = HPF * FT + (int)threadIdx.x; jj < hlen; jj += FT) {
    const int id = hrow[jj];
    if (id >= lo && id < lo + n) atomicAdd(&hc[(id - lo) >> 1], 1u << (16 * ((id - lo) & 1)));
  }
  __syncthreads();
}
// Applies the penalties of the count table to the chunk in registers.
template <int VEC>
__device__ __forceinline__ void apply_counts(const uint32_t* hc, int n, float rep, float pres, float freq,
                                             float (&x)[FE]) {
  constexpr int NV = FE / VEC;
#pragma unroll
  for (int v = 0; v < NV; v++) {
    const int l0 = (v * FT + (int)threadIdx.x) * VEC;
    if (l0 >= n) continue;
    uint32_t w[(VEC + 1) / 2];
    if constexpr (VEC == 8) {
      const u32x4 q = *reinterpret_cast<const u32x4*>(hc + (l0 >> 1));
      w[0] = q.x; w[1] = q.y; w[2] = q.z; w[3] = q.w;
    } else if constexpr (VEC == 4) {
      const uint2 q = *reinterpret_cast<const uint2*>(hc + (l0 >> 1));
      w[0] = q.x; w[1] = q.y;
    } else {
      w[0] = hc[l0 >> 1] >> (16 * (l0 & 1));
    }
    uint32_t any = 0;
#pragma unroll
    for (int i = 0; i < (VEC + 1) / 2; i++) any |= w[i];
    if (VEC == 1) any &= 0xFFFFu;
    if (!any) continue;
#pragma unroll
    for (int e = 0; e < VEC; e++) {
      const uint32_t cnt = VEC == 1 ? (w[0] & 0xFFFFu) : ((w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
      if (cnt) x[v * VEC + e] = penalize(x[v * VEC + e], (int)cnt, rep, pres, freq);
    }
  }
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

// ---------------------------------------------------------------------------
// Selections over register-resident candidates (FCPT per thread; slot e of a
// thread is present when e < np).  MSB-first radix over key - kmin with
// SELD-bit digits; the histogram scan gives each thread SELB / FT bins.
// ---------------------------------------------------------------------------
struct SelLevel {
  uint32_t base;   // kmin
  int bits;        // bit length of kmax - kmin
};
__device__ __forceinline__ SelLevel sel_range(const uint32_t (&ck)[FCPT], int np, FShared& S) {
  uint32_t mn = 0xFFFFFFFFu, mx = 0;
#pragma unroll
  for (int e = 0; e < FCPT; e++)
    if (e < np) { mn = ck[e] < mn ? ck[e] : mn; mx = ck[e] > mx ? ck[e] : mx; }
  mn = wmin(mn);
  mx = wmax(mx);
  if ((threadIdx.x & 63) == 0) { S.xc[threadIdx.x >> 6] = mn; S.xf[threadIdx.x >> 6] = mx; }
  __syncthreads();
  mn = min(min(S.xc[0], S.xc[1]), min(S.xc[2], S.xc[3]));
  mx = max(max(S.xf[0], S.xf[1]), max(S.xf[2], S.xf[3]));
  SelLevel L;
  L.base = mn;
  L.bits = mx > mn ? 32 - __clz(mx - mn) : 0;
  return L;
}

// kk-th largest present key (1 <= kk <= number present).
__device__ __forceinline__ uint32_t sel_count(const uint32_t (&ck)[FCPT], int np, uint32_t kk, FShared& S) {
  const SelLevel L = sel_range(ck, np, S);
  if (L.bits == 0) return L.base;
  constexpr int PER = SELB / FT;
  uint32_t hi = 0;      // digits matched so far
  int top = L.bits;     // bits not yet resolved: [0, top)
  uint32_t need = kk;
  while (top > 0) {
    const int sh = top > SELD ? top - SELD : 0;
    const int dw = top - sh;
    for (int i = threadIdx.x; i < SELB; i += FT) S.u.f.x.sel.cnt[i] = 0;
    __syncthreads();
#pragma unroll
    for (int e = 0; e < FCPT; e++) {
      if (e < np) {
        const uint32_t d = ck[e] - L.base;
        const uint32_t up = top >= 32 ? 0u : (d >> top);
        if (up == hi) atomicAdd(&S.u.f.x.sel.cnt[(d >> sh) & ((1u << dw) - 1u)], 1u);
      }
    }
    __syncthreads();
    // descending digits: thread t owns digits SELB-1-PER*t ... SELB-PER-PER*t
    uint32_t c[PER], loc = 0;
#pragma unroll
    for (int i = 0; i < PER; i++) { c[i] = S.u.f.x.sel.cnt[SELB - 1 - (PER * (int)threadIdx.x + i)]; loc += c[i]; }
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
    __syncthreads();
  }
  return L.base + hi;
}

// Mass-weighted select: the largest present key v with A + mass(key >= v) > P,
// requiring A <= P < A + total (ok = 0 otherwise).  above = A + mass(key > v);
// ceq / meq = count and mass of key == v.
struct MassSel {
  uint32_t key;
  uint64_t above;
  uint32_t ceq;
  uint64_t meq;
  int ok;
};
// Candidate masses are mass_fixed(mass_f(z, zmax)) of their z keys, recomputed per level.
__device__ __forceinline__ MassSel sel_mass(const uint32_t (&ck)[FCPT], int np, float zmax, uint64_t A, uint64_t P,
                                            FShared& S) {
  MassSel ms{0, A, 0, 0, 0};
  const SelLevel L = sel_range(ck, np, S);
  constexpr int PER = SELB / FT;
  uint32_t hi = 0;
  int top = L.bits;
  for (;;) {
    const int sh = top > SELD ? top - SELD : 0;
    const int dw = top - sh;
    for (int i = threadIdx.x; i < SELB; i += FT) { S.u.f.x.sel.cnt[i] = 0; S.u.f.x.sel.mass[i] = 0ull; }
    if (threadIdx.x == 0) S.mi[0] = -1;
    __syncthreads();
#pragma unroll
    for (int e = 0; e < FCPT; e++) {
      if (e < np) {
        const uint32_t d = ck[e] - L.base;
        const uint32_t up = top >= 32 ? 0u : (d >> top);
        if (up == hi) {
          const uint32_t b = dw > 0 ? ((d >> sh) & ((1u << dw) - 1u)) : 0u;
          atomicAdd(&S.u.f.x.sel.cnt[b], 1u);
          const uint64_t m = mass_fixed(mass_f(key2f(ck[e]), zmax));
          if (m) atomicAdd(&S.u.f.x.sel.mass[b], (unsigned long long)m);
        }
      }
    }
    __syncthreads();
    uint32_t c[PER];
    uint64_t m[PER], loc = 0;
#pragma unroll
    for (int i = 0; i < PER; i++) {
      const int b = SELB - 1 - (PER * (int)threadIdx.x + i);
      c[i] = S.u.f.x.sel.cnt[b];
      m[i] = S.u.f.x.sel.mass[b];
      loc += m[i];
    }
    uint64_t tot;
    uint64_t ex = ms.above + bscan_excl<uint64_t>(loc, &tot, S.xa);
#pragma unroll
    for (int i = 0; i < PER; i++) {
      if (ex <= P && P < ex + m[i]) {
        S.mi[0] = SELB - 1 - (PER * (int)threadIdx.x + i);
        S.mi[1] = (int)c[i];
        S.m64[0] = ex;
        S.m64[1] = m[i];
      }
      ex += m[i];
    }
    __syncthreads();
    if (S.mi[0] < 0) return ms;
    hi = (hi << dw) | (uint32_t)S.mi[0];
    ms.above = S.m64[0];
    ms.ceq = (uint32_t)S.mi[1];
    ms.meq = S.m64[1];
    top = sh;
    __syncthreads();
    if (top == 0) break;
  }
  ms.key = L.base + hi;
  ms.ok = 1;
  return ms;
}

}  // namespace lps
