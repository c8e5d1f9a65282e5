// General row sampler: one 1024-thread workgroup per row.
//
// Exact for every parameter combination the ABI accepts.  The row is streamed
// from memory once per pass (the first pass from HBM, later ones mostly from
// L2 / MALL); selections are sort-free MSB-first radix selects over
// order-preserving keys of the temperature-scaled logits with LDS histograms
// (11 + 11 + 10 bits), masses are fixed-point so every decision is
// deterministic and independent of accumulation order.
//
// History counts (penalties) are held for one window of GEN_WIN ids at a
// time: each pass walks the row window by window, and a window's counts are
// rebuilt from the row's whole history when the pass enters it.  A history of
// any length, with any number of distinct ids, is therefore counted exactly
// (counts are 32-bit).
//
// Semantics follow Sampler.sample_token (src/llm_pipeline/inference/
// sampling.py:51-85): penalties (:108-137 plus presence/frequency), greedy
// argmax for T <= 0 (:72-75), x / T, top-k with all ties at the k-th value kept
// (:139-156), top-p "keep sorted position j iff j == 0 or cum[j-1] <= p" with
// ties ordered lower index first (:158-185), min-p (:187-205), typical-p
// (:207-238, including its NaN fallback to the argmax when the row holds
// -inf), then an inverse-CDF draw from the caller's uniform over the kept ids
// in sorted order (z descending, ties lower index first).
#pragma once

#include "lps_common.h"

namespace lps {

constexpr int GEN_NT = 1024;            // threads of the general kernel (the code runs with any multiple of 64 up to it)
constexpr int GEN_NW = GEN_NT / 64;     // scratch sized for the largest block
constexpr int GEN_WIN = 8192;           // ids per history-count window: a multiple of every pass's tile
                                        // (threads x vector: at most 1024 x 8)
constexpr int NBINS = 2048;        // radix digit bins (11 bits)
constexpr uint32_t kNegInfKey = 0x007FFFFFu;  // f2key(-inf)

struct RowPlan {
  float zmax;        // max scaled logit
  float T;           // effective temperature (1 for greedy)
  uint32_t key_lo;   // kept: key > key_lo, or key == key_lo and tie rank < n_tie
  uint32_t n_tie;    // kNoTie = all ties at key_lo kept
  uint64_t Zf;       // fixed-point mass of the kept set
  int32_t greedy;
  int32_t argmax;
};

struct KParams {
  const void* logits;
  int V, R, rows_inner;
  int64_t stride_outer, stride_inner;
  // an optional second row segment (rows R1 .. R - 1 when logits2 is set: the
  // speculative draft rows beside the target rows): its own logits and row
  // layout, its own skip_draw, no uniforms
  int R1;
  const void* logits2;
  int rows_inner2;
  int64_t stride_outer2, stride_inner2;
  int skip_draw2;
  const float* temperature; float temperature_def;
  const int32_t* top_k; int top_k_def;
  const float* top_p; float top_p_def;
  const float* min_p; float min_p_def;
  const float* typical_p; float typical_p_def;
  const float* rep; float rep_def;
  const float* pres; float pres_def;
  const float* freq; float freq_def;
  const int32_t* history; int64_t history_stride; const int32_t* history_len;
  const float* uniforms;
  const int64_t* query_tokens; int query_inner; float* query_prob;
  int64_t* tokens;
  float* chosen_logprob;
  float* top_logprobs; int64_t* top_ids; int n_top;
  float* entropy;
  int32_t* row_status;
  int skip_draw;
  float* kept_cut;
  int32_t* kept_ties;
  int32_t* kept_count;
  RowPlan* plans;
  const int32_t* only_status;  // non-null: process only rows whose entry has LPS_ROW_DEFERRED (8) set
  int32_t* row_path;           // optional: 0 fast kernel, 1 general kernel
  const uint32_t* allowed;     // optional legality bits, row r at allowed + r * allowed_stride
  int64_t allowed_stride;      // 32-bit words
  int append_history;          // write each sampled token into the row's history
};

// Row r's segment: its logits base, row within the segment and row layout.
struct RowSeg {
  const void* base;
  int rl, ri;
  int64_t so, si;
  bool second;
};
__device__ __forceinline__ RowSeg row_seg(const KParams& P, int r) {
  const bool s2 = P.logits2 != nullptr && r >= P.R1;
  return RowSeg{s2 ? P.logits2 : P.logits, s2 ? r - P.R1 : r, s2 ? P.rows_inner2 : P.rows_inner,
                s2 ? P.stride_outer2 : P.stride_outer, s2 ? P.stride_inner2 : P.stride_inner, s2};
}
// Row r's logits (ES bytes per element).
template <int ES>
__device__ __forceinline__ const char* seg_row_ptr(const KParams& P, int r) {
  const RowSeg q = row_seg(P, r);
  return reinterpret_cast<const char*>(q.base) + ES * ((int64_t)(q.rl / q.ri) * q.so + (int64_t)(q.rl % q.ri) * q.si);
}
// Row r's draw is skipped.
__device__ __forceinline__ bool row_skips_draw(const KParams& P, int r) {
  return (P.logits2 != nullptr && r >= P.R1) ? P.skip_draw2 != 0 : P.skip_draw != 0;
}
// Row r's uniform array (the second segment has none).
__device__ __forceinline__ const float* row_uniforms(const KParams& P, int r) {
  return (P.logits2 != nullptr && r >= P.R1) ? nullptr : P.uniforms;
}
// Index of row r's query token in query_tokens, or -1 when it has none.
__device__ __forceinline__ int64_t row_query_index(const KParams& P, int r) {
  const RowSeg q = row_seg(P, r);
  if (!P.query_tokens || (q.rl % q.ri) >= P.query_inner) return -1;
  return (int64_t)(q.rl / q.ri) * P.query_inner + (q.rl % q.ri);
}
// With append_history: row r's sampled token joins its history for the next
// step (when the row has room, history_len[r] < history_stride).  One thread.
__device__ __forceinline__ void append_token(const KParams& P, int r, int64_t token) {
  if (!P.append_history || token < 0 || !P.history || !P.history_len) return;
  int32_t* len = const_cast<int32_t*>(P.history_len) + r;
  const int l = *len;
  if (l < 0 || (int64_t)l >= P.history_stride) return;
  const_cast<int32_t*>(P.history)[(int64_t)r * P.history_stride + l] = (int32_t)token;
  *len = l + 1;
}
// Row r's legality bits (nullptr: every id legal).
__device__ __forceinline__ const uint8_t* row_allowed(const KParams& P, int r) {
  return P.allowed ? reinterpret_cast<const uint8_t*>(P.allowed + (int64_t)r * P.allowed_stride) : nullptr;
}
// Whether id i is legal under the row's legality bits.
__device__ __forceinline__ bool id_allowed(const uint8_t* am, int64_t i) {
  return !am || ((am[i >> 3] >> (i & 7)) & 1u);
}
// Workspace row status bit (beside the LPS_ROW_* bits): the fast kernels
// deferred the row to the general kernel (the reason code in bits 8 and up).
constexpr int32_t LPS_ROW_DEFERRED = 8;

struct GenShared {
  alignas(16) uint32_t wcnt[GEN_WIN];  // history counts of the ids [w0, w0 + GEN_WIN) of the loaded window
  union {
    struct {
      uint32_t cnt[NBINS];
      uint64_t mass[NBINS];
    } h;
    struct {
      uint32_t key[LPS_MAX_TOP_LOGPROBS];
      int32_t idx[LPS_MAX_TOP_LOGPROBS];
      int32_t n;
    } lst;
  } u;
  uint64_t red64[GEN_NW];
  double redd[GEN_NW];
  uint32_t red32[GEN_NW];
  int32_t misc[8];
  uint64_t misc64[4];
  int32_t nth;  // threads running the general algorithm: 0 .. nth - 1 (a multiple of 64, at most GEN_NT;
                // the block may hold more, which have left)
};
// Threads running the general algorithm (set by its entry points).
__device__ __forceinline__ int gnt(const GenShared& S) { return S.nth; }

// The row's legality bits and penalties.  The history counts are those of one
// window of ids (pen_window loads it); apply() takes logits of that window.
struct PenCtx {
  bool active;          // penalties apply (a non-empty history and a non-neutral penalty)
  float rep, pres, freq;
  const uint32_t* wcnt; // counts of the loaded window's ids
  int64_t w0;           // first id of the window the pass is in
  int64_t loaded;       // first id of the window whose counts wcnt holds (-1: none)
  const int32_t* hist;  // the row's history ids (any value; ids outside [0, V) count for nothing)
  int hlen;
  int V;
  const uint8_t* am;    // the row's legality bits, or nullptr

  // Illegal ids to -inf, then the penalties, on the VEC logits of ids
  // [i0, i0 + VEC) (i0 a multiple of VEC inside the current window, VEC in
  // {1, 4, 8}).
  template <int VEC>
  __device__ __forceinline__ void apply(int64_t i0, float (&x)[VEC]) const {
    if (am) {
      const uint32_t b = (uint32_t)am[i0 >> 3] >> (i0 & 7);
#pragma unroll
      for (int j = 0; j < VEC; j++)
        if (!((b >> j) & 1u)) x[j] = -INFINITY;
    }
    if (!active) return;
    const uint32_t* c = wcnt + (i0 - w0);
    uint32_t cw[VEC];
    if constexpr (VEC % 4 == 0) {
#pragma unroll
      for (int q = 0; q < VEC / 4; q++) {
        const uint4 a = reinterpret_cast<const uint4*>(c)[q];
        cw[4 * q] = a.x; cw[4 * q + 1] = a.y; cw[4 * q + 2] = a.z; cw[4 * q + 3] = a.w;
      }
    } else {
#pragma unroll
      for (int j = 0; j < VEC; j++) cw[j] = c[j];
    }
    uint32_t any = 0;
#pragma unroll
    for (int j = 0; j < VEC; j++) any |= cw[j];
    if (!any) return;
#pragma unroll
    for (int j = 0; j < VEC; j++)
      if (cw[j]) x[j] = penalize(x[j], (int)cw[j], rep, pres, freq);
  }
};

// Ids per window of a pass: GEN_WIN with penalties, else the whole row.
__device__ __forceinline__ int64_t win_size(const PenCtx& pc) { return pc.active ? (int64_t)GEN_WIN : (int64_t)pc.V; }

// Enters the window starting at id w0: its history counts are counted from the
// row's whole history unless they are loaded already.  Every thread calls it
// (block-uniform arguments); it ends with a barrier when it loads.
__device__ __forceinline__ void pen_window(PenCtx& pc, GenShared& S, int64_t w0) {
  pc.w0 = w0;
  if (!pc.active || pc.loaded == w0) return;
  const int nt = gnt(S);
  __syncthreads();  // every reader of the previous window is done with it
  uint4* c4 = reinterpret_cast<uint4*>(S.wcnt);
  for (int i = threadIdx.x; i < GEN_WIN / 4; i += nt) c4[i] = make_uint4(0u, 0u, 0u, 0u);
  __syncthreads();
  const int64_t w1 = w0 + GEN_WIN < (int64_t)pc.V ? w0 + GEN_WIN : (int64_t)pc.V;
  for (int j = threadIdx.x; j < pc.hlen; j += nt) {
    const int64_t id = pc.hist[j];
    if (id >= w0 && id < w1) atomicAdd(&S.wcnt[id - w0], 1u);
  }
  __syncthreads();
  pc.loaded = w0;
}

// ---------------------------------------------------------------------------
// Block helpers (gnt(S) threads, a multiple of 64, at most GEN_NT).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t gblock_max_u64(uint64_t v, GenShared& S) {
  v = wave_max(v);
  if ((threadIdx.x & 63) == 0) S.red64[threadIdx.x >> 6] = v;
  __syncthreads();
  uint64_t r = S.red64[0];
  for (int i = 1; i < (gnt(S) >> 6); i++) r = S.red64[i] > r ? S.red64[i] : r;
  __syncthreads();
  return r;
}
__device__ __forceinline__ uint64_t gblock_sum_u64(uint64_t v, GenShared& S) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) S.red64[threadIdx.x >> 6] = v;
  __syncthreads();
  uint64_t r = 0;
  for (int i = 0; i < (gnt(S) >> 6); i++) r += S.red64[i];
  __syncthreads();
  return r;
}
__device__ __forceinline__ uint32_t gblock_min_u32(uint32_t v, GenShared& S) {
  v = wave_min(v);
  if ((threadIdx.x & 63) == 0) S.red32[threadIdx.x >> 6] = v;
  __syncthreads();
  uint32_t r = S.red32[0];
  for (int i = 1; i < (gnt(S) >> 6); i++) r = S.red32[i] < r ? S.red32[i] : r;
  __syncthreads();
  return r;
}
__device__ __forceinline__ uint32_t gblock_sum_u32(uint32_t v, GenShared& S) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) S.red32[threadIdx.x >> 6] = v;
  __syncthreads();
  uint32_t r = 0;
  for (int i = 0; i < (gnt(S) >> 6); i++) r += S.red32[i];
  __syncthreads();
  return r;
}
__device__ __forceinline__ double gblock_sum_f64(double v, GenShared& S) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) S.redd[threadIdx.x >> 6] = v;
  __syncthreads();
  double r = 0;
  for (int i = 0; i < (gnt(S) >> 6); i++) r += S.redd[i];
  __syncthreads();
  return r;
}
// Exclusive scan over the nt threads in thread order; *total = their sum.
template <typename T>
__device__ __forceinline__ T gblock_excl_scan(T v, T* total, T* scratch, int nt) {
  T inc = wave_incl_scan(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 63) scratch[w] = inc;
  __syncthreads();
  T off = 0, tot = 0;
  for (int i = 0; i < (nt >> 6); i++) {
    T s = scratch[i];
    off += (i < w) ? s : (T)0;
    tot += s;
  }
  __syncthreads();
  *total = tot;
  return off + inc - v;
}

// ---------------------------------------------------------------------------
// Row passes.
// ---------------------------------------------------------------------------
// One pass over the row, window by window (every thread calls it).
template <int DT, int VEC, typename F>
__device__ __forceinline__ void row_pass(const void* row, int V, PenCtx& pc, GenShared& S, F&& f) {
  const int64_t W = win_size(pc);
  for (int64_t w0 = 0; w0 < V; w0 += W) {
    pen_window(pc, S, w0);
    const int64_t w1 = w0 + W < (int64_t)V ? w0 + W : (int64_t)V;
    for (int64_t i0 = w0 + (int64_t)threadIdx.x * VEC; i0 < w1; i0 += (int64_t)gnt(S) * VEC) {
      float x[VEC];
      loadv<DT, VEC>(row, i0, x);
      pc.apply<VEC>(i0, x);
#pragma unroll
      for (int j = 0; j < VEC; j++) f((int)(i0 + j), x[j]);
    }
  }
}

// Digit layout of the 32-bit key: 11 + 11 + 10 bits.
__device__ __forceinline__ int lvl_shift(int l) { return l == 0 ? 21 : (l == 1 ? 10 : 0); }
__device__ __forceinline__ int lvl_bins(int l) { return l == 2 ? 1024 : 2048; }
__device__ __forceinline__ uint32_t lvl_himask(int l) { return l == 0 ? 0u : (l == 1 ? 0xFFE00000u : 0xFFFFFC00u); }

// Scan the current histogram from the top bin down.  For counts: the bin b
// where (count above b) < target <= (count above b) + cnt[b].  For masses:
// the bin where base + (mass above b) <= limit < base + (mass above b) + mass[b].
// Writes the bin to S.misc[0] and the "above" amounts to S.misc64[0..1].
__device__ void find_bin(GenShared& S, int nb, bool by_mass, uint64_t target_or_limit, uint64_t base) {
  if (threadIdx.x == 0) { S.misc[0] = -1; S.misc64[0] = 0; S.misc64[1] = 0; }
  // thread t owns descending positions r = t*per .. t*per+per-1 (bin = nb-1-r)
  const int per = nb / gnt(S) > 0 ? nb / gnt(S) : 1;
  const int r0 = threadIdx.x * per;
  uint64_t v = 0;
  for (int q = 0; q < per; q++) {
    const int rr = r0 + q;
    if (rr < nb) v += by_mass ? S.u.h.mass[nb - 1 - rr] : (uint64_t)S.u.h.cnt[nb - 1 - rr];
  }
  uint64_t tot;
  uint64_t a = gblock_excl_scan<uint64_t>(v, &tot, S.red64, gnt(S));
  for (int q = 0; q < per; q++) {
    const int rr = r0 + q;
    if (rr >= nb) break;
    const uint64_t c = by_mass ? S.u.h.mass[nb - 1 - rr] : (uint64_t)S.u.h.cnt[nb - 1 - rr];
    if (by_mass) {
      if (base + a <= target_or_limit && target_or_limit < base + a + c) { S.misc[0] = nb - 1 - rr; S.misc64[0] = a; }
    } else {
      if (a < target_or_limit && target_or_limit <= a + c) { S.misc[0] = nb - 1 - rr; S.misc64[0] = a; }
    }
    a += c;
  }
  __syncthreads();
}

template <int DT, int VEC>
__device__ void clear_hist(GenShared& S) {
  for (int i = threadIdx.x; i < NBINS; i += gnt(S)) { S.u.h.cnt[i] = 0; S.u.h.mass[i] = 0; }
  __syncthreads();
}

// kk-th largest key (1-based, counting multiplicity) of keyf over the row.
// Returns the key; *n_above = number of elements with a strictly larger key.
template <int DT, int VEC, typename KF>
__device__ __forceinline__ uint32_t select_kth(const void* row, int V, PenCtx& pc, GenShared& S, uint32_t kk, KF keyf,
                               uint32_t* n_above) {
  uint32_t prefix = 0;
  uint32_t above = 0;
  for (int l = 0; l < 3; l++) {
    const int sh = lvl_shift(l), nb = lvl_bins(l);
    const uint32_t hm = lvl_himask(l);
    clear_hist<DT, VEC>(S);
    row_pass<DT, VEC>(row, V, pc, S, [&](int i, float x) {
      uint32_t k = keyf(x);
      if ((k & hm) == prefix) atomicAdd(&S.u.h.cnt[(k >> sh) & (nb - 1)], 1u);
    });
    __syncthreads();
    find_bin(S, nb, false, kk, 0);
    int b = S.misc[0];
    uint32_t ex = (uint32_t)S.misc64[0];
    __syncthreads();
    if (b < 0) b = 0;  // unreachable when kk <= V
    prefix |= (uint32_t)b << sh;
    kk -= ex;
    above += ex;
  }
  *n_above = above;
  return prefix;
}

struct MassCut {
  uint32_t key;    // v*
  uint64_t above;  // mass strictly above v*
  uint32_t c_eq;   // elements at v*
  uint64_t m_eq;   // their total mass
};

// Largest key v with mass(active, key >= v) > limit (limit < total active mass).
template <int DT, int VEC, typename KF, typename AF>
__device__ __forceinline__ MassCut select_mass(const void* row, int V, PenCtx& pc, GenShared& S, uint64_t limit, KF keyf,
                               AF massf) {
  uint32_t prefix = 0;
  uint64_t A = 0;
  MassCut mc{};
  for (int l = 0; l < 3; l++) {
    const int sh = lvl_shift(l), nb = lvl_bins(l);
    const uint32_t hm = lvl_himask(l);
    clear_hist<DT, VEC>(S);
    row_pass<DT, VEC>(row, V, pc, S, [&](int i, float x) {
      uint32_t k;
      uint64_t m;
      if (massf(x, &k, &m) && (k & hm) == prefix) {
        const int b = (k >> sh) & (nb - 1);
        atomicAdd(&S.u.h.cnt[b], 1u);
        if (m) atomicAdd((unsigned long long*)&S.u.h.mass[b], (unsigned long long)m);
      }
    });
    __syncthreads();
    find_bin(S, nb, true, limit, A);
    int b = S.misc[0];
    uint64_t ex = S.misc64[0];
    if (b < 0) b = 0;  // unreachable while limit < total active mass
    const uint32_t c_b = S.u.h.cnt[b];
    const uint64_t m_b = S.u.h.mass[b];
    __syncthreads();
    prefix |= (uint32_t)b << sh;
    A += ex;
    mc.c_eq = c_b;
    mc.m_eq = m_b;
  }
  mc.key = prefix;
  mc.above = A;
  return mc;
}

// ---------------------------------------------------------------------------
// The kernel.
// ---------------------------------------------------------------------------
// Samples row r with threads 0 .. nth - 1 of the block (nth a multiple of 64,
// at most GEN_NT; threads of the block past nth must have left it, and every
// thread below nth must call this).
template <int DT, int VEC>
__device__ __forceinline__ void gen_row(const KParams& P, const int r, GenShared& S, const int nth) {
  const int tid = threadIdx.x;
  S.nth = nth;  // (every thread stores the same value before its first use)
  constexpr int ES = DT == LPS_DTYPE_F32 ? 4 : 2;
  const void* row = seg_row_ptr<ES>(P, r);
  const int V = P.V;

  const float T = P.temperature ? P.temperature[r] : P.temperature_def;
  const int topk = P.top_k ? P.top_k[r] : P.top_k_def;
  float topp = P.top_p ? P.top_p[r] : P.top_p_def;
  const float minp = P.min_p ? P.min_p[r] : P.min_p_def;
  const float typp = P.typical_p ? P.typical_p[r] : P.typical_p_def;
  const float rep = P.rep ? P.rep[r] : P.rep_def;
  const float pres = P.pres ? P.pres[r] : P.pres_def;
  const float freq = P.freq ? P.freq[r] : P.freq_def;
  if (topp != topp) topp = 1.0f;  // NaN top_p removes nothing in the reference
  const bool greedy = !(T > 0.0f);
  const bool want_lp = P.chosen_logprob || (P.n_top > 0 && P.top_logprobs);
  const bool want_H = P.entropy != nullptr;
  int status = 0;

  // ---- history: its counts are loaded one window of ids at a time by the passes ----
  int hlen = (P.history && P.history_len) ? P.history_len[r] : 0;
  if (P.history_stride > 0 && hlen > P.history_stride) hlen = (int)P.history_stride;  // never past the row
  if (hlen < 0) hlen = 0;
  const bool pen = hlen > 0 && (rep != 1.0f || pres != 0.0f || freq != 0.0f);
  PenCtx pc{pen, rep, pres, freq, S.wcnt, 0, -1, pen ? P.history + (int64_t)r * P.history_stride : nullptr,
            hlen, V, row_allowed(P, r)};

  // ---- pass 1: max and first argmax of the penalised logits ----
  uint64_t best = 0;
  row_pass<DT, VEC>(row, V, pc, S, [&](int i, float x) {
    const uint64_t pk = ((uint64_t)f2key(x) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)i);
    best = pk > best ? pk : best;
  });
  best = gblock_max_u64(best, S);
  const uint32_t mkey = (uint32_t)(best >> 32);
  const int argmax = (int)(0xFFFFFFFFu - (uint32_t)best);
  const float Mx = key2f(mkey);
  const bool has_nan = mkey == 0xFFFFFFFFu;

  const float Te = greedy ? 1.0f : T;
  const float zmax = greedy ? Mx : __fdiv_rn(Mx, T);
  auto zval = [&](float x) -> float { return greedy ? x : __fdiv_rn(x, T); };
  auto zkey = [&](float x) -> uint32_t { return f2key(zval(x)); };

  int64_t token = -1;
  if (!greedy) {
    if (has_nan || Mx == INFINITY || zmax == INFINITY) status |= LPS_ROW_NONFINITE;
    else if (Mx == -INFINITY) status |= LPS_ROW_EMPTY;
  } else {
    token = argmax;
  }

  // ---- full-row statistics: Z over all tokens, sum of e * (z - zmax) ----
  const bool stats_ok = !has_nan && Mx != INFINITY && Mx != -INFINITY && zmax != INFINITY;
  uint64_t Zfull = 0;
  double Sed = 0.0;
  const bool need_full = stats_ok &&
                         (want_lp || want_H || (!greedy && status == 0 && topk <= 0 && topp < 1.0f) ||
                          (!greedy && typp < 1.0f));
  if (need_full) {
    uint64_t zs = 0;
    double sd = 0.0;
    row_pass<DT, VEC>(row, V, pc, S, [&](int i, float x) {
      const float z = zval(x);
      const float e = mass_f(z, zmax);
      zs += mass_fixed(e);
      if (e > 0.0f) sd += (double)e * (double)__fsub_rn(z, zmax);
    });
    Zfull = gblock_sum_u64(zs, S);
    Sed = gblock_sum_f64(sd, S);
  }
  const double Zf_d = (double)Zfull / (double)kMassScale;
  const double lnZ = need_full ? log(Zf_d) : 0.0;
  if (want_H && tid == 0) P.entropy[r] = need_full ? (float)(lnZ - Sed / (double)Zfull * (double)kMassScale) : NAN;

  // ---- sampling-row selection ----
  uint32_t key_lo = 0, n_tie = kNoTie;
  uint64_t Zk = 0;
  float qprob = 0.0f;
  const int64_t qi = row_query_index(P, r);
  const int64_t qtok = qi >= 0 ? P.query_tokens[qi] : -1;
  if (greedy) {
    key_lo = mkey;
    n_tie = 1;
    qprob = (qtok >= 0 && qtok == argmax) ? 1.0f : 0.0f;
  } else if (status == 0) {
    // top-k threshold (all ties at the k-th value kept)
    uint32_t thk = 0;
    if (topk > 0) {
      const uint32_t kk = (uint32_t)(topk < V ? topk : V);
      uint32_t na;
      thk = select_kth<DT, VEC>(row, V, pc, S, kk, zkey, &na);
    }
    key_lo = thk;
    // top-p cut on the mass of the top-k kept set
    if (topp < 1.0f) {
      if (topk <= 0) {
        Zk = Zfull;
      } else {
        uint64_t zs = 0;
        row_pass<DT, VEC>(row, V, pc, S, [&](int i, float x) {
          const float z = zval(x);
          if (f2key(z) >= thk) zs += mass_fixed(mass_f(z, zmax));
        });
        Zk = gblock_sum_u64(zs, S);
      }
      const double pl = topp > 0.0f ? (double)topp * (double)Zk : 0.0;
      uint64_t limit = (uint64_t)pl;
      if (limit >= Zk) limit = Zk - 1;
      MassCut mc = select_mass<DT, VEC>(row, V, pc, S, limit, zkey, [&](float x, uint32_t* k, uint64_t* m) {
        const float z = zval(x);
        *k = f2key(z);
        if (*k < thk) return false;
        *m = mass_fixed(mass_f(z, zmax));
        return true;
      });
      key_lo = mc.key;
      const uint64_t e1 = mc.c_eq ? mc.m_eq / mc.c_eq : 0;
      uint64_t nt = e1 ? (limit - mc.above) / e1 + 1 : (uint64_t)mc.c_eq;
      n_tie = nt >= mc.c_eq ? kNoTie : (uint32_t)nt;
    }
    // min-p: keep e >= min_p (the max has e == 1)
    if (minp > 0.0f) {
      uint32_t mk = 0xFFFFFFFFu;
      row_pass<DT, VEC>(row, V, pc, S, [&](int i, float x) {
        const float z = zval(x);
        const uint32_t k = f2key(z);
        if (k >= key_lo && mass_f(z, zmax) >= minp) mk = k < mk ? k : mk;
      });
      mk = gblock_min_u32(mk, S);
      if (mk == 0xFFFFFFFFu) status |= LPS_ROW_EMPTY;
      else if (mk > key_lo) { key_lo = mk; n_tie = kNoTie; }
    }
    // typical-p
    if (status == 0 && typp < 1.0f) {
      uint32_t ngt = 0, neq = 0, ninf = 0;
      const uint32_t kinf = f2key(-INFINITY);
      row_pass<DT, VEC>(row, V, pc, S, [&](int i, float x) {
        const uint32_t k = zkey(x);
        ngt += k > key_lo ? 1u : 0u;
        neq += k == key_lo ? 1u : 0u;
        ninf += k == kinf ? 1u : 0u;
      });
      ngt = gblock_sum_u32(ngt, S);
      neq = gblock_sum_u32(neq, S);
      ninf = gblock_sum_u32(ninf, S);
      const uint32_t nk = ngt + (n_tie == kNoTie ? neq : (n_tie < neq ? n_tie : neq));
      const uint32_t zmkey = f2key(zmax);
      if (nk < (uint32_t)V || ninf > 0) {
        key_lo = zmkey;
        n_tie = 1;
      } else {
        // information = ln Z - d <= exp(H) * typical_p  <=>  d >= ln Z - tau
        const double H = lnZ - Sed / (double)Zfull * (double)kMassScale;
        const float tau = __fmul_rn((float)exp(H), typp);
        const double dmin = lnZ - (double)tau;
        uint32_t mk = 0xFFFFFFFFu;
        row_pass<DT, VEC>(row, V, pc, S, [&](int i, float x) {
          const float z = zval(x);
          if ((double)__fsub_rn(z, zmax) >= dmin) { const uint32_t k = f2key(z); mk = k < mk ? k : mk; }
        });
        mk = gblock_min_u32(mk, S);
        if (mk == 0xFFFFFFFFu) { key_lo = zmkey; n_tie = 1; }
        else { key_lo = mk; n_tie = kNoTie; }
      }
    }
  }

  // ---- kept mass (tie ranks in vocabulary order) and the query probability ----
  uint64_t Zf = 0;
  uint32_t kept_n = greedy ? 1u : 0u;
  if (!greedy && status == 0) {
    uint64_t acc = 0;
    uint32_t tie_run = 0, nkept = 0;
    uint64_t qm = 0;
    int qk = 0;
    // (windows of ids, tiles in vocabulary order within each: tie ranks run in vocabulary order)
    const int64_t W = win_size(pc);
    for (int64_t w0 = 0; w0 < V; w0 += W) {
    pen_window(pc, S, w0);
    const int64_t w1 = w0 + W < (int64_t)V ? w0 + W : (int64_t)V;
    for (int64_t tile = w0; tile < w1; tile += (int64_t)gnt(S) * VEC) {
      const int64_t i0 = tile + (int64_t)tid * VEC;
      float x[VEC];
      uint32_t k[VEC];
      uint32_t nt_loc = 0;
      if (i0 < w1) {
        loadv<DT, VEC>(row, i0, x);
        pc.apply<VEC>(i0, x);
#pragma unroll
        for (int j = 0; j < VEC; j++) { k[j] = zkey(x[j]); nt_loc += k[j] == key_lo ? 1u : 0u; }
      }
      uint32_t tot = 0, ex = 0;
      if (n_tie != kNoTie) ex = gblock_excl_scan<uint32_t>(nt_loc, &tot, S.red32, gnt(S));
      if (i0 < w1) {
        uint32_t rk = tie_run + ex;
#pragma unroll
        for (int j = 0; j < VEC; j++) {
          bool kept = k[j] > key_lo || (k[j] == key_lo && (n_tie == kNoTie || rk < n_tie));
          if (k[j] == key_lo) rk++;
          if (kept) {
            const uint64_t m = mass_fixed(mass_f(zval(x[j]), zmax));
            acc += m;
            nkept += k[j] != kNegInfKey ? 1u : 0u;
            if (i0 + j == qtok) { qm = m; qk = 1; }
          }
        }
      }
      tie_run += tot;
    }
    }
    Zf = gblock_sum_u64(acc, S);
    kept_n = gblock_sum_u32(nkept, S);
    const uint64_t qmr = gblock_sum_u64(qm, S);
    const uint32_t qkr = gblock_sum_u32((uint32_t)qk, S);
    qprob = qkr ? (float)((double)qmr / (double)Zf) : 0.0f;
  }

  // ---- inverse-CDF draw in sorted order: z descending, ties lower index first ----
  if (!greedy && status == 0 && !row_skips_draw(P, r)) {
    const float* ur = row_uniforms(P, r);
    float u = ur ? ur[r] : 0.5f;
    if (!(u >= 0.0f)) u = 0.0f;
    if (u >= 1.0f) u = 0.99999994f;
    uint64_t target = (uint64_t)((double)u * (double)Zf);
    if (target >= Zf) target = Zf - 1;
    // the key holding the target: the largest v with mass(kept, key > v) <= target
    // (elements of key_lo past the kept ties weigh after every kept one)
    const MassCut dc = select_mass<DT, VEC>(row, V, pc, S, target, zkey, [&](float x, uint32_t* k, uint64_t* m) {
      const float z = zval(x);
      *k = f2key(z);
      if (*k < key_lo) return false;
      *m = mass_fixed(mass_f(z, zmax));
      return true;
    });
    // every element of that key has the same mass: the tie holding the target,
    // counted in vocabulary order
    const uint64_t e1 = dc.c_eq ? dc.m_eq / dc.c_eq : 0;
    uint32_t jt = e1 ? (uint32_t)((target - dc.above) / e1) : 0u;
    if (jt >= dc.c_eq && dc.c_eq) jt = dc.c_eq - 1;
    const uint32_t vkey = dc.key;
    uint32_t run = 0;
    if (tid == 0) S.misc[1] = -1;
    __syncthreads();
    const int64_t W = win_size(pc);
    bool done = false;
    for (int64_t w0 = 0; w0 < V && !done; w0 += W) {
    pen_window(pc, S, w0);
    const int64_t w1 = w0 + W < (int64_t)V ? w0 + W : (int64_t)V;
    for (int64_t tile = w0; tile < w1; tile += (int64_t)gnt(S) * VEC) {
      const int64_t i0 = tile + (int64_t)tid * VEC;
      uint32_t k[VEC];
      uint32_t nt_loc = 0;
      if (i0 < w1) {
        float x[VEC];
        loadv<DT, VEC>(row, i0, x);
        pc.apply<VEC>(i0, x);
#pragma unroll
        for (int j = 0; j < VEC; j++) { k[j] = zkey(x[j]); nt_loc += k[j] == vkey ? 1u : 0u; }
      }
      uint32_t ttot;
      const uint32_t tex = gblock_excl_scan<uint32_t>(nt_loc, &ttot, S.red32, gnt(S));
      if (i0 < w1 && run + tex <= jt && jt < run + tex + nt_loc) {
        uint32_t rk = run + tex;
#pragma unroll
        for (int j = 0; j < VEC; j++) {
          if (k[j] == vkey) {
            if (rk == jt) S.misc[1] = (int)(i0 + j);
            rk++;
          }
        }
      }
      __syncthreads();
      const int found = S.misc[1];
      __syncthreads();
      if (found >= 0) { token = found; done = true; break; }
      run += ttot;
    }
    }
  } else if (!greedy) {
    token = -1;
  }

  // ---- logprobs: chosen id and top-N of log_softmax(penalised z) ----
  if (want_lp) {
    if (P.chosen_logprob) {
      // the drawn id's history count (the whole block counts it)
      uint32_t tc = 0;
      if (pen && token >= 0)
        for (int j = tid; j < hlen; j += gnt(S)) tc += pc.hist[j] == token ? 1u : 0u;
      tc = gblock_sum_u32(tc, S);
      if (tid == 0) {
        float lp = NAN;
        if (token >= 0 && need_full) {
          float xv = load1<DT>(row, token);
          if (!id_allowed(pc.am, token)) xv = -INFINITY;
          if (tc) xv = penalize(xv, (int)tc, rep, pres, freq);
          lp = (float)((double)__fsub_rn(zval(xv), zmax) - lnZ);
        }
        P.chosen_logprob[r] = lp;
      }
    }
    if (P.n_top > 0 && P.top_logprobs) {
      const int N = P.n_top < V ? P.n_top : V;
      uint32_t nabove;
      const uint32_t thn = select_kth<DT, VEC>(row, V, pc, S, (uint32_t)N, zkey, &nabove);
      const uint32_t ties_take = (uint32_t)N - nabove;
      if (tid == 0) S.u.lst.n = 0;
      __syncthreads();
      uint32_t tie_run = 0;
      const int64_t W = win_size(pc);
      for (int64_t w0 = 0; w0 < V; w0 += W) {
      pen_window(pc, S, w0);
      const int64_t w1 = w0 + W < (int64_t)V ? w0 + W : (int64_t)V;
      for (int64_t tile = w0; tile < w1; tile += (int64_t)gnt(S) * VEC) {
        const int64_t i0 = tile + (int64_t)tid * VEC;
        float x[VEC];
        uint32_t k[VEC];
        uint32_t nt_loc = 0;
        if (i0 < w1) {
          loadv<DT, VEC>(row, i0, x);
          pc.apply<VEC>(i0, x);
#pragma unroll
          for (int j = 0; j < VEC; j++) { k[j] = zkey(x[j]); nt_loc += k[j] == thn ? 1u : 0u; }
        }
        uint32_t ttot, tex = gblock_excl_scan<uint32_t>(nt_loc, &ttot, S.red32, gnt(S));
        if (i0 < w1) {
          uint32_t rk = tie_run + tex;
#pragma unroll
          for (int j = 0; j < VEC; j++) {
            bool take = k[j] > thn || (k[j] == thn && rk < ties_take);
            if (k[j] == thn) rk++;
            if (take) {
              int slot = atomicAdd(&S.u.lst.n, 1);
              if (slot < LPS_MAX_TOP_LOGPROBS) { S.u.lst.key[slot] = k[j]; S.u.lst.idx[slot] = (int)(i0 + j); }
            }
          }
        }
        tie_run += ttot;
      }
      }
      __syncthreads();
      const int n = S.u.lst.n < N ? S.u.lst.n : N;
      if (tid < n) {
        const uint32_t ki = S.u.lst.key[tid];
        const int ii = S.u.lst.idx[tid];
        int rank = 0;
        for (int j = 0; j < n; j++) {
          const uint32_t kj = S.u.lst.key[j];
          const int ij = S.u.lst.idx[j];
          rank += (kj > ki || (kj == ki && ij < ii)) ? 1 : 0;
        }
        const float z = key2f(ki);
        P.top_logprobs[(int64_t)r * P.n_top + rank] = need_full ? (float)((double)__fsub_rn(z, zmax) - lnZ) : NAN;
        if (P.top_ids) P.top_ids[(int64_t)r * P.n_top + rank] = ii;
      }
      for (int j = n + tid; j < P.n_top; j += gnt(S)) {
        P.top_logprobs[(int64_t)r * P.n_top + j] = -INFINITY;
        if (P.top_ids) P.top_ids[(int64_t)r * P.n_top + j] = -1;
      }
      __syncthreads();
    }
  }

  if (tid == 0) {
    const bool failed = !greedy && status != 0;
    P.tokens[r] = failed ? -1 : token;
    append_token(P, r, failed ? -1 : token);
    if (P.row_status) P.row_status[r] = status;
    if (P.query_prob) P.query_prob[r] = qprob;
    if (P.kept_cut) P.kept_cut[r] = key_lo <= kNegInfKey ? -INFINITY : key2f(key_lo);  // key 0: nothing cut
    if (P.kept_ties) P.kept_ties[r] = n_tie == kNoTie ? -1 : (int32_t)n_tie;
    if (P.kept_count) P.kept_count[r] = (int32_t)kept_n;
    if (P.row_path) P.row_path[r] = 1;
    if (P.plans) {
      RowPlan pl;
      pl.zmax = zmax; pl.T = Te; pl.key_lo = key_lo; pl.n_tie = n_tie; pl.Zf = Zf;
      pl.greedy = greedy ? 1 : 0; pl.argmax = argmax;
      P.plans[r] = pl;
    }
  }
}

template <int DT, int VEC>
__global__ __launch_bounds__(GEN_NT) void gen_row_kernel(KParams P) {
  __shared__ GenShared S;
  const int r = blockIdx.x;
  if (P.only_status && !(P.only_status[r] & LPS_ROW_DEFERRED)) return;
  // a copy local to the rows that run: the general path takes the parameters
  // by reference, and a skipped row then never copies them to scratch memory
  KParams Pl = P;
  gen_row<DT, VEC>(Pl, r, S, GEN_NT);
}

}  // namespace lps
