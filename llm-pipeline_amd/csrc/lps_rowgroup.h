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
//   all      penalties from a 16-bit count table of the chunk's history ids
//            (LDS; any number of distinct ids, a count of 65535 or more
//            defers the row), legality bits, thread max, workgroup max.
//   GREEDY   first argmax; with logprobs the chunk mass and top-N candidates.
//   TOPK     a threshold below the chunk's k'-th largest logit (from the
//            wave-level k'/8-th largest thread maxima), lowered to the start
//            of its division-collision group; every logit at or above it is
//            a candidate.
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
//            region are candidates (one list per region), with the exact mass
//            above each region.  Regions too crowded for the lists (flat
//            rows: thousands of logits in one bin) take a second level: each
//            chunk bins its elements of the (at most RW) region bins by the
//            next 8 mantissa bits, exactly as above; after a second barrier
//            the fine bins are merged and the regions located among them.
// Candidates are gathered in LDS (per-wave segments filled by ballots), sorted
// in the chunk by (z = fl(x / T) descending, index ascending) with a rank sort,
// and published sorted; a top-k list stops after its k'-th entry and the
// entries tied with it.
// The last workgroup of a row to finish (an arrival count) finalises it: it
// loads the G sorted lists of each kind; a top-k row keeps the entries at or
// above a bound on its k'-th largest (from the lists' m-th entries) and
// rank-sorts them, a nucleus row merges its lists (the rank of an entry is its
// position in its own list plus a binary search in each other list); then it
// finds the top-k set, the top-p cut and the draw by binary searches over
// exact fixed-point prefix masses in sorted order.  The draw is an inverse
// CDF in sorted order: kept ids by scaled logit descending, ties lower index
// first.
//
// With the entropy output (an instantiation of its own), nucleus and pure rows
// also sum e * log2(e) per chunk, and the finaliser gives H = ln Z - sum(e ln e) / Z.
// The same instantiation takes min-p rows without top-k as nucleus rows (region
// 1 also covers the bins that can hold the min-p boundary, and the finaliser
// applies the exact test to the sorted candidates), typical-p rows that top-p or
// min-p cut (only the argmax is kept), and typical-p rows without other filters
// (the cut from the row's entropy: the argmax, every logit, a threshold cut
// like min-p's, or a cut under the histogram that the chunks count), and rows
// with top_k past the lists and no top-p / min-p (the chunks also publish a
// count byte per bin; the merged counts locate the k-th largest's bin).
// A row the kernel cannot finish exactly (e.g. a region wider than RW bins
// holding more candidates than the lists take, typical-p after a top-p / min-p
// that removed nothing, entropy with top-k or greedy) is marked LPS_ROW_DEFERRED in the workspace status and
// sampled by the general kernel, launched after this one with that status as
// its filter.  (Sampling such rows in the same launch, in one tail workgroup
// per row, was measured: the tail code in the kernel made every launch slower,
// also those that never ran a tail.)
//
// Cross-workgroup handoffs (the histogram barrier and the arrival count):
// every thread of the publishing workgroup stores, then waits for its stores
// to complete (they are then in the XCD's L2, which the row's workgroups
// share); one thread then adds to the row's counter.  The reader spins on the
// counter with agent-scope loads and reads the published data with
// agent-scope loads, which are served by that L2 (never by a CU's L1).  A
// row whose workgroups did not all run on one XCD is deferred.
#pragma once

#include <cstddef>

#include "lps_generic.h"
#include "lps_wave.h"

// Phase stamps of a timing build (LPS_RG_STAMPS): thread 0 of every
// workgroup records the 100 MHz real-time counter at phase marks into
// rg_stamps (read back with lps_debug_stamps); empty otherwise.
#ifdef LPS_RG_STAMPS
#define RG_STAMP(i)                                                                              \
  do {                                                                                            \
    if (threadIdx.x == 0 && blockIdx.x < 8192)                                                    \
      ::lps::rg::rg_stamps[blockIdx.x * 32 + (i)] = __builtin_amdgcn_s_memrealtime();             \
  } while (0)
// a stamp taken once value v is available
#define RG_STAMP_DEP(i, v)                                                                       \
  do {                                                                                            \
    if (threadIdx.x == 0 && blockIdx.x < 8192) {                                                  \
      __asm__ volatile("" ::"v"(v));                                                              \
      ::lps::rg::rg_stamps[blockIdx.x * 32 + (i)] = __builtin_amdgcn_s_memrealtime();             \
    }                                                                                             \
  } while (0)
#else
#define RG_STAMP(i) ((void)0)
#define RG_STAMP_DEP(i, v) ((void)0)
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
constexpr int RW = 2;              // second level: bins of one region it refines
constexpr int FSUB = 256;          // second level: fine bins per bin (8 more mantissa bits)
constexpr int FHN = 2 * RW * FSUB; // second level: fine bins of a chunk (region 1, then region 2)
constexpr int CAPR = 2048;         // published list entries per row (all chunks, both lists)
constexpr int FT = 256;            // finaliser threads (waves 0-3, one per SIMD; the others leave)
constexpr int FW = FT / 64;        // finaliser waves
constexpr int FPT = CAPR / FT;     // finaliser: loaded entries per thread
constexpr int FP1 = 4;             // finaliser: first-pass slots (loaded before the list lengths are known)
constexpr int SEGCAP = 128;        // chunk: entries of one list per wave segment
constexpr int CLMAX = NW * SEGCAP; // chunk: entries of one list
constexpr int LKM = CAPR;          // finaliser: loaded entries of one list (all chunks)
constexpr int KM = 1024;           // finaliser: merged (sorted) entries of one list
constexpr int KPT = KM / FT;       // merged entries per thread in the prefix scans
constexpr int HPT = HPUB / NT;     // published histogram bins per thread
constexpr int HLT = HB / NT;       // LDS histogram bins per thread
constexpr double kFix = 17592186044416.0;  // 2^44: fixed-point masses (relative to the row reference)
constexpr int FAST_KMAX = 256;     // largest top_k / top-N of the row-group kernel
constexpr int STREAM_KMAX = 128;   // largest top_k / top-N of the streaming kernel
constexpr int STREAM_VMAX = 163840;  // largest vocabulary of the streaming kernel

// Row modes, decided per row from its parameters (row_cfg).
enum { MODE_GREEDY = 0, MODE_TOPK = 1, MODE_PURE = 2, MODE_NUCLEUS = 3, MODE_DEFER = 4 };

// Chunk flags (RgSum.flags); any of them defers the row.
enum {
  RF_OVERFLOW = 1,    // more candidates than the lists take
  RF_HISTORY = 2,     // a history count does not fit 16 bits
  RF_SPLIT = 4,       // a chunk summary is not this launch's, or its chunk ran on another XCD
  RF_REGION = 8,      // no usable cut / draw region, or the barrier timed out
  RF_WIDE = 16,       // a crowded region wider than the second level takes (RW bins)
};

// Per-chunk summary (published for the finaliser).
struct RgSum {
  uint64_t tag;       // rg_tag(epoch, row, XCD): which launch, row and XCD wrote it (one 8-byte word,
                      // read by one load: a current tag vouches for the XCD it names)
  uint32_t mkey;      // max key of the penalised logits (0xFFFFFFFF: NaN present)
  int32_t amax;       // first index of that key (greedy rows)
  float ref;          // mass reference (an integer, log2 units; -inf: no finite logit)
  uint16_t n1, n2;    // published entries of list 1 (top-k / region 1) and list 2 (region 2)
  uint32_t flags;     // RF_*
  uint32_t nab1;      // nucleus: elements above region 1
  uint32_t nanbin;    // nucleus: NaN / +inf masses seen
  double zsum;        // chunk mass: sum of exp2(fma(x, c, -ref))
  double ab1;         // nucleus: exact mass above region 1 (chunk reference).  Typical-p rows
                      // without other filters (tw_pack): at the barrier, the chunk's -inf
                      // logits and its least logit's key; at arrival, for a cut under the
                      // histogram (no region 1), the logits it drops and the least kept key
  double ab2;         // nucleus: exact mass above region 2
  double zent;        // entropy rows: sum of e * log2(e), e = exp2(fma(x, c, -ref)) (chunk reference)
  int32_t reg[4];     // nucleus: the regions lo1, hi1, lo2, hi2 (row fine bins, efine scale; the same
                      // in every chunk)
};
static_assert(sizeof(RgSum) % 8 == 0 && offsetof(RgSum, tag) == 0, "8-byte words, the tag first");
__device__ __forceinline__ void store_sum(RgSum* d, const RgSum& a) { *d = a; }
__device__ __forceinline__ double tw_pack(uint32_t n, uint32_t key) {
  return __builtin_bit_cast(double, ((uint64_t)key << 32) | n);
}
__device__ __forceinline__ uint32_t tw_n(double v) { return (uint32_t)__builtin_bit_cast(uint64_t, v); }
__device__ __forceinline__ uint32_t tw_key(double v) { return (uint32_t)(__builtin_bit_cast(uint64_t, v) >> 32); }
// Summary tag: the row's launch epoch (a per-row count in the workspace that
// each launch's finaliser advances, so a record left by an earlier launch
// carries an older one; zero-filled memory never matches, the epochs start at
// 1), the row (records of another row or workspace layout never match) and
// the XCD that ran the chunk.
__device__ __forceinline__ uint64_t rg_tag(uint32_t epoch, int r, uint32_t xcc) {
  return ((uint64_t)(epoch + 1u) << 32) | ((uint64_t)(uint32_t)r << 8) | (uint64_t)(xcc & 0xFFu);
}
constexpr int CTR_ARRIVE = 0;  // counter words of a row (32 per row): arrivals,
constexpr int CTR_HIST = 2;    // the histogram barrier,
constexpr int CTR_EPOCH = 4;   // the row's launch epoch (never reset),
constexpr int CTR_FINE = 6;    // and the second-level barrier

struct RgParams {
  KParams k;
  // sums: row r holds 2 * MAXG records: [0, G) published before the histogram
  // barrier (max, reference, mass), [MAXG, MAXG + G) at the chunk's end
  int G;               // chunks per row
  int cv;              // vectors per chunk (the last chunk may hold fewer)
  int nvec;            // vectors per row
  int heavy_first;     // dispatch rows without top-k first
  int skip_topk;       // the streaming kernel's rows (stream_takes) ran there: skip them
  int stream_only;     // the row-group kernel is not launched: the streaming kernel defers the others
  uint32_t* counters;  // [R * 32]: arrivals and the histogram barrier (zero between launches), the
                       // row's launch epoch (CTR_*)
  int32_t* status;     // [R]
  RgSum* sums;         // row r at sums + r * 2 * MAXG
  float* hist;         // row r at hist + r * G * HPUB
  float* fine;         // second-level bins: row r at fine + r * G * FHN (large top-k rows: one
                       // count byte per published bin instead)
  uint4* cands;        // row r at cands + r * CAPR: chunk j owns [j * capw, (j + 1) * capw): its
                       // sorted list 1, then its sorted list 2, entries {z key, index, x bits, 0}
  int capw;            // list entries per chunk
};

// ---------------------------------------------------------------------------
// Row configuration.
// ---------------------------------------------------------------------------
struct RowCfg {
  float T, c, topp, minp, typp, rep, pres, freq, u;  // c = log2(e) / T (1 / T -> log2(e) for greedy rows)
  int topk, ntop, mode, kprime, hlen;
  int64_t qtok;
  bool greedy, pen;
  bool bigk;  // FAST_KMAX < top_k < V, no top-p / min-p: a nucleus row with a count cut
  const int32_t* hrow;
};
// Parameters and mode of row r (sampling.py:66-82 filter order; the row-group
// kernel takes greedy rows, top-k rows with k <= FAST_KMAX, nucleus and pure
// rows, and defers the rest to the general kernel).
// A per-row parameter, or its default for a NULL array.  The load is issued
// unconditionally (a NULL array reads a dummy word, then its value is
// dropped), so every parameter load of a row is in flight at once instead of
// one dependent round trip each.
__device__ int32_t rg_dummy_word[2];
template <typename T>
__device__ __forceinline__ T param_or(const T* p, int64_t i, T def) {
  const T* q = p ? p + i : reinterpret_cast<const T*>(rg_dummy_word);
  const T v = *q;
  return p ? v : def;
}
// MT: the kernel takes min-p and typical-p rows without top-k (else they are
// deferred).
template <bool MT = true>
__device__ __forceinline__ RowCfg row_cfg(const KParams& P, int r) {
  RowCfg g;
  g.bigk = false;
  g.T = param_or(P.temperature, r, P.temperature_def);
  g.topk = param_or(P.top_k, r, P.top_k_def);
  // top_k >= V keeps every id (sampling.py:152 clamps k to V; nothing is under
  // the V-th value): the row samples as one without top-k
  if (g.topk >= P.V) g.topk = 0;
  g.topp = param_or(P.top_p, r, P.top_p_def);
  g.minp = param_or(P.min_p, r, P.min_p_def);
  g.typp = param_or(P.typical_p, r, P.typical_p_def);
  g.rep = param_or(P.rep, r, P.rep_def);
  g.pres = param_or(P.pres, r, P.pres_def);
  g.freq = param_or(P.freq, r, P.freq_def);
  g.u = param_or(row_uniforms(P, r), r, 0.5f);
  const int64_t qi = row_query_index(P, r);
  g.qtok = param_or(qi >= 0 ? P.query_tokens : (const int64_t*)nullptr, qi >= 0 ? qi : 0, (int64_t)-1);
  // a query id outside the vocabulary has probability 0 (as verify_drafts_kernel
  // treats it); no logit is read for it
  if (g.qtok >= (int64_t)P.V) g.qtok = -1;
  if (g.topp != g.topp) g.topp = 1.0f;
  g.greedy = !(g.T > 0.0f);
  g.c = __fdiv_rn(kLog2e, g.greedy ? 1.0f : g.T);
  g.ntop = (P.n_top > 0 && P.top_logprobs) ? P.n_top : 0;
  int mode;
  if (g.greedy) mode = MODE_GREEDY;
  else if (!(g.T >= 1e-4f)) mode = MODE_DEFER;
  else if (g.topk > 0) {
    mode = g.topk <= FAST_KMAX ? MODE_TOPK : MODE_DEFER;
    // (past the lists: the k-th largest located by counts in the histogram,
    // when neither top-p nor min-p follows; typical-p then keeps the argmax)
    if (MT && mode == MODE_DEFER && !(g.topp < 1.0f) && !(g.minp > 0.0f) && g.ntop == 0) {
      mode = MODE_NUCLEUS;
      g.bigk = true;
    }
  }
  else if (!MT) {
    if (g.minp > 0.0f || g.typp < 1.0f || g.ntop > 0) mode = MODE_DEFER;
    else mode = g.topp < 1.0f ? MODE_NUCLEUS : MODE_PURE;
  } else if (g.ntop > 0 || g.minp > 1.0f) mode = MODE_DEFER;
  // (typical-p after a filter that removed ids keeps the argmax; on a full row
  // it is a threshold cut like min-p's)
  else mode = (g.topp < 1.0f || g.minp > 0.0f || g.typp < 1.0f) ? MODE_NUCLEUS : MODE_PURE;
  if (P.entropy && mode != MODE_NUCLEUS && mode != MODE_PURE) mode = MODE_DEFER;
  g.kprime = mode == MODE_TOPK ? (g.topk > g.ntop ? g.topk : g.ntop) : (mode == MODE_GREEDY ? g.ntop : 0);
  if (g.kprime > FAST_KMAX) mode = MODE_DEFER;
  g.mode = mode;
  g.hrow = P.history ? P.history + (int64_t)r * P.history_stride : nullptr;
  int hlen = param_or(g.hrow ? P.history_len : (const int32_t*)nullptr, r, 0);
  if (P.history_stride > 0 && hlen > P.history_stride) hlen = (int)P.history_stride;
  g.hlen = hlen;
  g.pen = hlen > 0 && (g.rep != 1.0f || g.pres != 0.0f || g.freq != 0.0f);
  return g;
}

// Rows the streaming kernel (one workgroup per row) takes when it runs:
// greedy and top-k rows with k' <= STREAM_KMAX.
__device__ __forceinline__ bool stream_takes(const RowCfg& g) {
  return (g.mode == MODE_GREEDY || g.mode == MODE_TOPK) && g.kprime <= STREAM_KMAX;
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

// Row order with rows that sample without top-k (nucleus / pure: the longest
// finalisers) first: virtual row vr -> row, a bijection on [0, R) (R <= 128),
// the same in every workgroup.
__device__ __forceinline__ int heavy_first_row(const KParams& P, const int vr) {
  const int lane = threadIdx.x & 63;
  auto heavy = [&](int r) -> bool {
    if (r >= P.R) return false;
    const float T = P.temperature ? P.temperature[r] : P.temperature_def;
    const int k = P.top_k ? P.top_k[r] : P.top_k_def;
    return T > 0.0f && k <= 0;
  };
  const uint64_t m1 = wballot(heavy(lane)), m2 = wballot(heavy(lane + 64));
  const uint64_t v1 = wballot(lane < P.R), v2 = wballot(lane + 64 < P.R);
  const int nh = __popcll(m1) + __popcll(m2);
  const bool hv = vr < nh;
  const uint64_t a = hv ? m1 : (v1 & ~m1), b = hv ? m2 : (v2 & ~m2);
  const int k = hv ? vr : vr - nh;
  const int pa = __popcll(a);
  const uint64_t sel = k < pa ? a : b;
  const int kk = k < pa ? k : k - pa;
  const uint64_t w = wballot(((sel >> lane) & 1ull) && (int)lanes_below(sel) == kk);
  return (k < pa ? 0 : 64) + (int)__builtin_ctzll(w);
}

// ---------------------------------------------------------------------------
// Shared memory.
// ---------------------------------------------------------------------------
struct RgX {  // cross-wave exchange slots, each reused only after a barrier
  float f[NW];
  uint32_t u[NW], u2[NW], u3[NW];
  int32_t i1[NW], i2[NW], i3[NW];
  uint64_t q[NW], q2[NW];
  double d[NW], d2[NW], d3[NW], d4[NW], d5[NW];
  uint32_t u4[NW];
  int32_t mi[32];
  double md[16];
  uint64_t mq[8];
  float mf[8];
  int32_t cn[2][MAXG];               // finaliser: entries of each chunk's lists
  int32_t cb[2][MAXG + 1];           // finaliser: list prefixes over chunks
  int32_t opre[MAXG + 1];            // finaliser: prefix of the chunks' entries past the first pass
  float rf[MAXG];                    // the row's chunk references
  float rm[MAXG];                    // the row's chunk maxima (NaN chunk: +inf)
};
// Chunk candidate lists: per-wave segments filled by ballots, then compacted.
struct RgLists {
  int32_t si[2][NW][SEGCAP];         // segment entries: vocabulary index
  uint32_t sx[2][NW][SEGCAP];        // their logits (bits)
  uint64_t ck[2][CLMAX];             // compacted
  uint32_t cx[2][CLMAX];
  int32_t scnt[2][NW];               // segment counts (SEGCAP + 1: overflowed)
};
// Words of the count table region: the chunk's 16-bit counts, and at least
// the lists' size, so that the lists (which overlay it) end before the
// histogram, which is read while the lists fill.
template <int NE>
constexpr int hc_words() {
  static_assert(sizeof(unsigned long long) * FHN <= sizeof(RgLists), "the fine bins end before the histogram");
  return NT * NE / 2 > (int)(sizeof(RgLists) + 3) / 4 ? NT * NE / 2 : (int)((sizeof(RgLists) + 15) / 16 * 4);
}
template <int NE>
struct RgChunkS : RgX {
  union {
    struct {
      uint32_t hc[hc_words<NE>()];          // 16-bit history counts of the chunk's ids
      unsigned long long hist[HB + 64];     // count << 48 | sum of low 16 mantissa bits (+ spare slots)
    } a;
    RgLists l;                               // after the counts are used
    // second level (nucleus rows, after the counts are used and before the
    // lists fill): count << 48 | sum of low 8 mantissa bits
    unsigned long long fh[FHN];
  };
};
struct RgFinalS : RgX {
  uint64_t lk[2][LKM];                  // loaded lists, chunk by chunk (sorted within a chunk)
  uint32_t lx[2][LKM];                  // their logits (bits)
  uint64_t sk[2][KM];                   // merged lists: keys in sorted order
  uint32_t sx[2][KM];                   // logits (bits)
  uint64_t sm[2][KM];                   // fixed-point masses
  uint64_t sc[2][KM];                   // inclusive prefix of the masses
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

// Block reduction of a per-thread value over W waves; every thread gets the
// result.  The slot array is free again after the next barrier.
template <int W = NW, typename T, typename Op>
__device__ __forceinline__ T bred(T v, T* slot, Op op) {
  v = wreduce(v, op);
  if (lane_id() == 0) slot[wave_id()] = v;
  __syncthreads();
  T r = slot[0];
#pragma unroll
  for (int i = 1; i < W; i++) r = op(r, slot[i]);
  return r;
}
// Exclusive prefix over the block (W waves) in thread order; *total gets the sum.
template <int W = NW, typename T>
__device__ __forceinline__ T bscan(T v, T* total, T* slot) {
  const T inc = wscan_incl(v);
  if (lane_id() == 63) slot[wave_id()] = inc;
  __syncthreads();
  T off = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < W; i++) {
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
  // (log2(e) as kLog2e + kLog2eLo: for |z| in the hundreds the rounding of
  // kLog2e alone moves the exponent by ~3e-6)
  constexpr float kLog2eLo = 1.925963e-08f;
  const float t = __builtin_fmaf(z, kLog2eLo, __builtin_fmaf(z, kLog2e, -R));
  return (uint64_t)__float2ull_rn(ldexpf(__builtin_amdgcn_exp2f(t), 44));
}
// bin_mass for an accumulator whose low-bit sum fits 32 bits (a chunk bin
// holds at most NT * 80 < 2^16 masses): 2^(E - 150) (count (128 + t) 2^16 + low).
__device__ __forceinline__ double bin_mass_u(int b, unsigned long long acc) {
  const uint32_t cnt = (uint32_t)(acc >> 48), low = (uint32_t)acc;
  const double m = __builtin_fma((double)(cnt * (128u + (uint32_t)(b & 127))), 65536.0, (double)low);
  return ldexp(m, (b >> 7) + HE0 - 150);
}
// Fine bin of a mass on the second level's scale: its exponent and top 15
// mantissa bits, bin ebin(e) << 8 | the next 8 bits (negative under the
// histogram; from HB_NAN << 8 for NaN / inf).
__device__ __forceinline__ int efine(float e) { return (int)(__float_as_uint(e) >> 8) - (HE0 << 15); }
// Exact mass of fine bin f from its accumulator (count << 48 | sum of the low
// 8 mantissa bits; at most NT * 80 < 2^16 masses): 2^(E - 150) (count (2^15 +
// top 15 bits) 2^8 + low).  0 for an empty bin, whatever f.
__device__ __forceinline__ double fine_mass(int f, unsigned long long acc) {
  const uint32_t cnt = (uint32_t)(acc >> 48), low = (uint32_t)acc;
  const double m = __builtin_fma((double)(cnt * (uint32_t)(0x8000 + (f & 0x7FFF))), 256.0, (double)low);
  return cnt ? ldexp(m, (f >> 15) + HE0 - 150) : 0.0;
}
// First float key k (in f2key order, over the non-NaN keys, from -inf's
// exclusive to +inf's) where a predicate of the logit, false then true over
// the keys, holds.  One wave searches 64 keys per round (6 rounds); every lane
// of the wave calls it with the same arguments.
// first_key_reaching: the first whose logit reaches fine bin thr,
// efine(emass(key2f(k), c, ref)) >= thr.  The hardware exp2 is non-decreasing
// over every fp32 input (lps_selftest_exp2_monotone) and fma(x, c, -ref) is
// non-decreasing in x for c > 0; +inf's key satisfies it for thr < 2^22.
template <class Pr>
__device__ __forceinline__ uint32_t first_key_where(Pr pred) {
  constexpr uint32_t kNegInfK = 0x007FFFFFu, kPosInfK = 0xFF800000u;
  const uint64_t l1 = (uint64_t)(threadIdx.x & 63) + 1u;
  uint32_t lo = kNegInfK, hi = kPosInfK;  // the predicate is taken to fail at lo and to hold at hi
  while (hi - lo > 1u) {
    const uint64_t span = hi - lo, step = (span + 63u) >> 6;
    const uint32_t k = lo + (uint32_t)(l1 * step < span ? l1 * step : span);
    const uint64_t m = __builtin_amdgcn_ballot_w64(pred(key2f(k)));
    const uint64_t j = m ? (uint64_t)__builtin_ctzll(m) : 63u;
    hi = lo + (uint32_t)((j + 1u) * step < span ? (j + 1u) * step : span);
    lo = lo + (uint32_t)(j * step);
  }
  return hi;
}
__device__ __forceinline__ uint32_t first_key_reaching(int thr, float c, float ref) {
  return first_key_where([&](float x) { return efine(emass(x, c, ref)) >= thr; });
}
// The smallest mass of bin b.
__device__ __forceinline__ double bin_base(int b) {
  return ldexp(8388608.0 + (double)(b & 127) * 65536.0, (b >> 7) + HE0 - 150);
}
// Row bins [lo, hi] that can hold a threshold cut "mass relative to the row
// maximum >= ratio": the general kernel's min-p rule (keep z iff mass_f(z,
// zmax) >= min_p, ratio = min_p, 0 < min_p <= 1; sampling.py:187-205) and its
// typical-p rule on a full row (keep z iff z - zmax >= dmin, ratio =
// exp(dmin); sampling.py:207-238).  The boundary's mass against the row
// reference R is ratio times the row maximum's; every id the rule keeps has its
// binned mass (emass against its chunk's reference, rescaled) above that mass
// times 2^-E and every id it drops has it under that mass times 2^E.  E bounds
// the rounding of both computations, in log2 units: each step rounds a value of
// magnitude at most W = |xmax c| + |log2 ratio| + 4 (the scaled logits near
// the boundary, the references, their differences) by 2^-24 relative, and the
// two exp2 add a few ulps; 2^-19 W is several times their sum.  False when the
// range leaves the histogram (a ratio under about 2^-30, or 0).
__device__ __forceinline__ bool cut_bins(float ratio, float xmax, float c, float R, int& lo, int& hi) {
  const float W = fabsf(__fmul_rn(xmax, c)) + fabsf(log2f(ratio)) + 4.0f;
  const float E = ldexpf(W, -19);
  const float tm = __fmul_rn(emass(xmax, c, R), ratio);
  const uint32_t bl = ebin(__fmul_rn(tm, __builtin_amdgcn_exp2f(-E)));
  const uint32_t bh = ebin(__fmul_rn(tm, __builtin_amdgcn_exp2f(E)));
  lo = (int)bl;
  hi = (int)bh;
  return bl != BELOW && bh < (uint32_t)HB_NAN && !(xmax != xmax);
}
// Typical-p rows without other filters, by what their cut keeps (decided
// alike in every chunk and in the finaliser, from the same summaries):
enum {
  TYP_ARGMAX = 0,  // the row holds -inf (NaN entropy) or the cut keeps nothing: only the argmax
  TYP_ALL = 1,     // the cut keeps the least logit, so every logit: a pure row
  TYP_CUT = 2,     // the boundary lies in the histogram, in bins [lo, hi]: a threshold cut
  TYP_LOW = 3,     // the boundary lies under the histogram: every binned logit is kept, a pure
                   // draw; the chunks count the few logits it drops
  TYP_WIDE = 4     // the boundary's range straddles the histogram's bottom: deferred
};
__device__ __forceinline__ int typical_case(uint32_t ninf, double dmin, float xmin, float xmax, float T, float c,
                                            float R, int& lo, int& hi) {
  if (ninf > 0u || !(dmin <= 0.0)) return TYP_ARGMAX;
  if ((double)__fsub_rn(__fdiv_rn(xmin, T), __fdiv_rn(xmax, T)) >= dmin) return TYP_ALL;
  const float ratio = (float)exp(dmin);
  if (!(ratio > 0.0f)) return TYP_LOW;
  if (cut_bins(ratio, xmax, c, R, lo, hi)) return TYP_CUT;
  return (uint32_t)hi == BELOW ? TYP_LOW : TYP_WIDE;
}
// Typical-p on a full row in the general kernel's terms (no id removed, no
// -inf): lnZ = ln sum exp(z - zmax), H = lnZ - sum e (z - zmax) / Z, tau =
// fl(exp(H)) typical_p, and z is kept iff z - zmax >= dmin = lnZ - tau.  From
// the row mass Z and AH = sum e log2 e, both against 2^R (e = exp2(fma(x, c,
// -R))): sum exp(z - zmax) is Z over the maximum's mass exp2(fma(xmax, c, -R)),
// and H is invariant to the reference.
__device__ __forceinline__ double typical_dmin(double Z, double AH, float R, float xmax, float c, float typp) {
  const double lZ = log(Z);
  const double lnZ = lZ - 0.6931471805599453 * (double)__builtin_fmaf(xmax, c, -R);
  const double H = lZ - 0.6931471805599453 * AH / Z;
  const float tau = __fmul_rn((float)exp(H), typp);
  return lnZ - (double)tau;
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
// History ids of the row: the first NT are read before the chunk, so the count
// table is built while the chunk's loads are in flight.
__device__ __forceinline__ int prefetch_hist(const int32_t* hrow, int hlen) {
  const int j = threadIdx.x;
  return (hrow && j < hlen) ? hrow[j] : -1;
}
// 16-bit counts of the history ids that fall in the chunk's ids [lo, lo + n)
// (two per word).  Returns false when a count reaches 65534 (the row is then
// deferred: an increment past 65535 would carry into the next id's count).
// Ends with a barrier.
template <int NE>
__device__ __forceinline__ bool build_counts(RgChunkS<NE>& S, const int32_t* hrow, int hlen, int id0, int lo, int n) {
  constexpr int WORDS = NT * NE / 2;
  static_assert(WORDS % 4 == 0, "whole 16-byte stores");
  u32x4* h4 = reinterpret_cast<u32x4*>(S.a.hc);
#pragma unroll
  for (int i = threadIdx.x; i < WORDS / 4; i += NT) h4[i] = u32x4{0u, 0u, 0u, 0u};
  if (threadIdx.x == 0) S.mi[30] = 0;
  __syncthreads();
  bool sat = false;
  auto add = [&](int id) {
    if (id >= lo && id < lo + n) {
      const int l = id - lo;
      const int sh = 16 * (l & 1);
      const uint32_t old = atomicAdd(&S.a.hc[l >> 1], 1u << sh);
      if (((old >> sh) & 0xFFFFu) >= 65533u) sat = true;
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
    uint32_t cw[(VPE + 1) / 2];  // the vector's counts, two per word
    if constexpr (VPE == 8) {
      const uint4 q = *reinterpret_cast<const uint4*>(hc + (l0 >> 1));
      cw[0] = q.x; cw[1] = q.y; cw[2] = q.z; cw[3] = q.w;
    } else if constexpr (VPE == 4) {
      const uint2 q = *reinterpret_cast<const uint2*>(hc + (l0 >> 1));
      cw[0] = q.x; cw[1] = q.y;
    } else {
      cw[0] = (hc[l0 >> 1] >> (16 * (l0 & 1))) & 0xFFFFu;
    }
    uint32_t any = 0;
#pragma unroll
    for (int q = 0; q < (VPE + 1) / 2; q++) any |= cw[q];
    if (!any) continue;
#pragma unroll
    for (int e = 0; e < VPE; e++) {
      const uint32_t cnt = VPE == 1 ? cw[0] : (cw[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
      if (cnt) C.x[i * VPE + e] = penalize(C.x[i * VPE + e], (int)cnt, rep, pres, freq);
    }
  }
}

// ---------------------------------------------------------------------------
// Chunk candidate lists.
// ---------------------------------------------------------------------------
// Sort key of a candidate: (z key << 32) | ~index, z = fl(x / T) (x for greedy
// rows).  Keys are distinct within a row; descending key order is z
// descending, ties lower index first (the order of the reference's sort).
__device__ __forceinline__ uint64_t cand_key(float x, int idx, bool greedy, float T) {
  const float z = greedy ? x : __fdiv_rn(x, T);
  return ((uint64_t)f2key(z) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)idx);
}
__device__ __forceinline__ int key_index(uint64_t k) { return (int)(0xFFFFFFFFu - (uint32_t)k); }
__device__ __forceinline__ uint32_t key_z(uint64_t k) { return (uint32_t)(k >> 32); }

// Appends this lane's (x, index) to this wave's segment of list l when on:
// one ballot per slot gives every lane its position (slot order, then lane
// order).  n is the wave's running count (wave-uniform).
__device__ __forceinline__ void seg_put(RgLists& L, int l, bool on, uint32_t& n, float x, int idx) {
  const uint64_t m = __builtin_amdgcn_ballot_w64(on);
  if (m) {
    if (on) {
      const uint32_t p = n + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
      if (p < (uint32_t)SEGCAP) {
        L.si[l][threadIdx.x >> 6][p] = idx;
        L.sx[l][threadIdx.x >> 6][p] = __float_as_uint(x);
      }
    }
    n += (uint32_t)__popcll(m);
  }
}
// A wave's segment count (lane 0 of the wave); SEGCAP + 1 marks an overflow.
__device__ __forceinline__ void seg_done(RgLists& L, int l, uint32_t n) {
  if ((threadIdx.x & 63) == 0) L.scnt[l][threadIdx.x >> 6] = n > (uint32_t)SEGCAP ? SEGCAP + 1 : (int)n;
}

// Sorts the chunk's lists l < nl (their wave segments complete; the caller
// barriers after seg_done) by key, descending, and writes them to dst: list 0
// at [0, np0), list 1 at [np0, np0 + np1), entries {z key, index, x bits, 0}.  List 0
// stops after rank lim0 - 1 and the entries whose z equals that entry's z
// (lim0 = 0: no limit).  np[l] receives the counts; returns false when a
// segment overflowed or the lists, list 0 after its limit, exceed cap
// (nothing written then).  Every thread calls it; it ends with a barrier.
__device__ __forceinline__ bool sort_publish(RgLists& L, RgX& X, int nl, int lim0, bool greedy, float T, uint4* dst, int cap,
                                             int (&np)[2]) {
  const int tid = threadIdx.x;
  int n[2] = {0, 0}, pre[2][NW];
  bool over = false;
#pragma unroll
  for (int l = 0; l < 2; l++)
#pragma unroll
    for (int w = 0; w < NW; w++) {
      const int c = l < nl ? L.scnt[l][w] : 0;
      over |= c > SEGCAP;
      pre[l][w] = n[l];
      n[l] += c > SEGCAP ? SEGCAP : c;
    }
  if (over || (lim0 <= 0 && n[0] + n[1] > cap) || (lim0 > 0 && min(n[0], lim0) + n[1] > cap)) {
    // (list 0 keeps at least min(n0, lim0) entries: past cap in any case)
    np[0] = np[1] = 0;
    __syncthreads();
    return false;
  }
  // compact the segments (entry f of list l: the segment whose prefix holds it)
#pragma unroll
  for (int l = 0; l < 2; l++) {
    for (int f = tid; f < n[l]; f += NT) {
      int w = 0, b = 0;
#pragma unroll
      for (int q = 1; q < NW; q++) {
        const bool in = f >= pre[l][q];
        w = in ? q : w;
        b = in ? pre[l][q] : b;
      }
      const uint32_t xb = L.sx[l][w][f - b];
      L.ck[l][f] = cand_key(__uint_as_float(xb), L.si[l][w][f - b], greedy, T);
      L.cx[l][f] = xb;
    }
  }
  if (tid == 0) X.mi[8] = 0x7FFFFFFF;
  __syncthreads();
  // ranks: 2^lg adjacent lanes share an entry, each counting the keys above it
  // in one slice of its list; list 1 (when present) follows list 0 in the
  // entry numbering
  const int N = n[0] + n[1];
  const int lg = N <= 64 ? 3 : N <= 128 ? 2 : N <= 256 ? 1 : 0;
  const int per = NT >> lg, part = tid & ((1 << lg) - 1);
  int rk[CLMAX * 2 / NT];
  int np0 = n[0];
#pragma unroll
  for (int it = 0; it < CLMAX * 2 / NT; it++) {
    rk[it] = -1;
    const int e = (tid >> lg) + it * per;
    if (it * per >= N) continue;
    int rank = 0;
    if (e < N) {
      const int l = e < n[0] ? 0 : 1;
      const int f = l ? e - n[0] : e;
      const int nl_ = l ? n[1] : n[0];
      const uint64_t* ck = L.ck[l];
      const uint64_t key = ck[f];
      const int len = (nl_ + (1 << lg) - 1) >> lg;
      const int q1 = min(nl_, part * len + len);
      int q = part * len;
      for (; q + 4 <= q1; q += 4) {
        const uint64_t a0 = ck[q], a1 = ck[q + 1], a2 = ck[q + 2], a3 = ck[q + 3];
        rank += (a0 > key ? 1 : 0) + (a1 > key ? 1 : 0) + (a2 > key ? 1 : 0) + (a3 > key ? 1 : 0);
      }
      for (; q < q1; q++) rank += ck[q] > key ? 1 : 0;
    }
    for (int o = 1; o < (1 << lg); o <<= 1) rank += __shfl_xor(rank, o);
    rk[it] = e < N ? rank : -1;
    // list 0's limit: the z key of the entry ranked lim0 - 1
    if (e < n[0] && part == 0 && lim0 > 0 && rank == lim0 - 1) X.mi[9] = (int)key_z(L.ck[0][e]);
  }
  if (lim0 > 0 && lim0 < n[0]) {
    __syncthreads();
    // entries ranked from lim0 on stay when tied in z with the entry ranked lim0 - 1:
    // their ranks are contiguous, so the count is the first rank of a lower z
    const uint32_t zl = (uint32_t)X.mi[9];
    int first_out = 0x7FFFFFFF;
#pragma unroll
    for (int it = 0; it < CLMAX * 2 / NT; it++) {
      const int e = (tid >> lg) + it * per;
      if (part == 0 && rk[it] >= lim0 && e < n[0] && key_z(L.ck[0][e]) != zl) first_out = min(first_out, rk[it]);
    }
    if (first_out != 0x7FFFFFFF) atomicMin(&X.mi[8], first_out);
    __syncthreads();
    np0 = min(n[0], X.mi[8]);
  }
  if (np0 + n[1] > cap) {  // the entries tied with list 0's last kept one pass cap
    np[0] = np[1] = 0;
    __syncthreads();
    return false;
  }
  // write in sorted order
#pragma unroll
  for (int it = 0; it < CLMAX * 2 / NT; it++) {
    const int e = (tid >> lg) + it * per;
    if (part != 0 || rk[it] < 0 || e >= N) continue;
    const int l = e < n[0] ? 0 : 1;
    const int f = l ? e - n[0] : e;
    if (l == 0 && rk[it] >= np0) continue;
    const uint64_t key = L.ck[l][f];
    dst[(l ? np0 : 0) + rk[it]] = make_uint4(key_z(key), (uint32_t)key_index(key), L.cx[l][f], 0u);
  }
  np[0] = np0;
  np[1] = n[1];
  __syncthreads();
  return true;
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
  return seg_row_ptr<ES>(P, r);
}

}  // namespace rg
}  // namespace lps

#include "lps_rowgroup_kernel.h"
