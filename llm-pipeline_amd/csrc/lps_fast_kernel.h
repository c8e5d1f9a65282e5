// The fast row-sampling kernels (layout, modes and protocol: lps_fast.h).
//
// Visibility of published data: within a kernel, a row's histograms (and, in
// the fused kernel, its summaries and candidates) are written once, followed
// by a wait for the stores, and read by the row's other workgroups only after
// the barrier or handoff atomic that counts every chunk's arrival.  All of a
// row's chunks run on one XCD (checked: the finaliser defers the row
// otherwise), so the data meet in its L2; the L1 is invalidated at every
// kernel start and no workgroup reads those lines before the count completes.
// final_kernel reads what chunk_kernel wrote after the kernel boundary.
// Counters are only touched with atomics, which execute at the L2, except
// their reset to zero, plain stores by the row's finaliser.
//
// Cross-wave exchange slots of XShared (xa ... xh, xv, mi, m64, md, mf) are each
// rewritten only after a barrier that follows every read of their previous
// value; the comments name the slot each step uses.
#pragma once

#include "lps_fast.h"

namespace lps {

// Block-wide penalised logit of one id (history scanned by all threads).
template <int DT>
__device__ float penalized_logit(const void* row, const uint8_t* am, int id, const int32_t* h, int hlen, bool pen,
                                 float rep, float pres, float freq, XShared& S) {
  uint32_t c = 0;
  if (pen)
    for (int j = threadIdx.x; j < hlen; j += FT) c += h[j] == id ? 1u : 0u;
  __syncthreads();
  c = bcombine(wsum(c), S.xh, OpAdd{});
  __syncthreads();
  float x = load1<DT>(row, id);
  if (!id_allowed(am, id)) x = -INFINITY;
  if (pen && c) x = penalize(x, (int)c, rep, pres, freq);
  return x;
}

// Rank sort of the kept list by (z desc, idx asc), i.e. by skey desc:
// kord[rank] = slot.  LDS reads are batched 8 at a time (independent loads).
template <class FS>
__device__ void rank_sort_kept(int K, FS& S) {
  auto& k = S.x.k;
  for (int i = threadIdx.x; i < K; i += FT) {
    const uint64_t ki = k.skey[i];
    int rank = 0;
    int q = 0;
    for (; q + 8 <= K; q += 8) {
      uint64_t t[8];
#pragma unroll
      for (int u = 0; u < 8; u++) t[u] = k.skey[q + u];
#pragma unroll
      for (int u = 0; u < 8; u++) rank += t[u] > ki ? 1 : 0;
    }
    for (; q < K; q++) rank += k.skey[q] > ki ? 1 : 0;
    k.kord[rank] = i;
  }
  __syncthreads();
}

// Number of entries of a[0, n) below v (batched LDS reads).
__device__ __forceinline__ int count_below(const int32_t* a, int n, int v) {
  int c = 0, q = 0;
  for (; q + 8 <= n; q += 8) {
    int32_t t[8];
#pragma unroll
    for (int u = 0; u < 8; u++) t[u] = a[q + u];
#pragma unroll
    for (int u = 0; u < 8; u++) c += t[u] < v ? 1 : 0;
  }
  for (; q < n; q++) c += a[q] < v ? 1 : 0;
  return c;
}

// Inclusive prefix of km over the sorted order into cum, K <= KEPTCAP (slot xb).
template <class FS>
__device__ void sorted_prefix(int K, FS& S) {
  auto& k = S.x.k;
  constexpr int PER = KEPTCAP / FT;
  uint64_t loc[PER];
  uint64_t t = 0;
#pragma unroll
  for (int q = 0; q < PER; q++) {
    const int pz = threadIdx.x * PER + q;
    loc[q] = pz < K ? k.km[k.kord[pz]] : 0;
    t += loc[q];
  }
  uint64_t tot;
  uint64_t a = bscan_excl<uint64_t>(t, &tot, S.xb);
#pragma unroll
  for (int q = 0; q < PER; q++) {
    const int pz = threadIdx.x * PER + q;
    a += loc[q];
    if (pz < K) k.cum[pz] = a;
  }
  __syncthreads();
}

// Runs fn(BoolT<true>) when the wave holds penalised packed slots, else
// fn(BoolT<false>) (fp32 chunks carry their penalties in place).
template <bool PK, typename Fn>
__device__ __forceinline__ void with_pen(bool wpen, Fn&& fn) {
  if constexpr (PK) {
    if (wpen) fn(BoolT<true>{});
    else fn(BoolT<false>{});
  } else {
    fn(BoolT<false>{});
  }
}

// Per-row parameters and the row's mode, as both kernels derive them.
struct RowCfg {
  float T, topp, minp, typp, rep, pres, freq, u;
  int topk, ntop, mode, kprime, hlen;
  int64_t qtok;
  bool greedy, pen;
  const int32_t* hrow;
};
__device__ __forceinline__ RowCfg row_cfg(const KParams& P, int r) {
  RowCfg g;
  g.T = P.temperature ? P.temperature[r] : P.temperature_def;
  g.topk = P.top_k ? P.top_k[r] : P.top_k_def;
  g.topp = P.top_p ? P.top_p[r] : P.top_p_def;
  g.minp = P.min_p ? P.min_p[r] : P.min_p_def;
  g.typp = P.typical_p ? P.typical_p[r] : P.typical_p_def;
  g.rep = P.rep ? P.rep[r] : P.rep_def;
  g.pres = P.pres ? P.pres[r] : P.pres_def;
  g.freq = P.freq ? P.freq[r] : P.freq_def;
  g.u = P.uniforms ? P.uniforms[r] : 0.5f;
  g.qtok = (P.query_tokens && (r % P.rows_inner) < P.query_inner)
               ? P.query_tokens[(int64_t)(r / P.rows_inner) * P.query_inner + (r % P.rows_inner)]
               : -1;
  // a query id outside the vocabulary has probability 0 (as verify_drafts_kernel
  // treats it); no logit is read for it
  if (g.qtok >= (int64_t)P.V) g.qtok = -1;
  if (g.topp != g.topp) g.topp = 1.0f;
  g.greedy = !(g.T > 0.0f);
  g.ntop = (P.n_top > 0 && P.top_logprobs) ? P.n_top : 0;
  int mode;
  if (g.greedy) mode = MODE_GREEDY;
  else if (!(g.T >= 1e-4f)) mode = MODE_DEFER;
  else if (g.topk > 0) mode = g.topk <= FAST_KMAX ? MODE_TOPK : MODE_DEFER;
  else if (g.minp > 0.0f || g.typp < 1.0f || g.ntop > 0) mode = MODE_DEFER;
  else mode = g.topp < 1.0f ? MODE_NUCLEUS : MODE_PURE;
  if (P.entropy) mode = MODE_DEFER;
  if (mode == MODE_TOPK && g.typp < 1.0f && g.topk >= P.V) mode = MODE_DEFER;
  g.kprime = mode == MODE_TOPK ? (g.topk > g.ntop ? g.topk : g.ntop) : (mode == MODE_GREEDY ? g.ntop : 0);
  if (g.kprime > FAST_KMAX) mode = MODE_DEFER;
  g.mode = mode;
  g.hrow = P.history ? P.history + (int64_t)r * P.history_stride : nullptr;
  int hlen = (g.hrow && P.history_len) ? P.history_len[r] : 0;
  if (P.history_stride > 0 && hlen > P.history_stride) hlen = (int)P.history_stride;
  g.hlen = hlen;
  g.pen = hlen > 0 && (g.rep != 1.0f || g.pres != 0.0f || g.freq != 0.0f);
  return g;
}

// Workgroup id -> (row, chunk): ids are dispatched round-robin over the 8
// XCDs, so the chunks of a row (ids congruent modulo 8) share one XCD.
struct ChunkId {
  int r, j;
};
__device__ __forceinline__ ChunkId chunk_id(int G) {
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  return ChunkId{(slot / G) * 8 + xcd, slot % G};
}

// Fused kernel row order (R <= 128): rows that sample without top-k (nucleus /
// pure: the longest finalisers) are dispatched first, so that their
// finalisers overlap the chunk work of the rows dispatched after them.
// Virtual row vr -> row; a bijection on [0, R), the same in every workgroup.
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

// Phase 1: chunk j of row r (r < R).  Returns the row's mode; a deferred row
// (MODE_DEFER) publishes nothing.
template <int DT, int VEC, int NR>
__device__ __forceinline__ int chunk_body(const FParams& F, CSharedT<NR>& S, const int r, const int j) {
  using CK = Chunk<DT, VEC, NR>;
  constexpr int PUB = CK::PUB;
  constexpr int NE = CK::NE, CH = CK::CH;
  constexpr bool PK = CK::PACKED;
  const KParams& P = F.k;
  const int G = F.G;
  LPS_STAMP(0);
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int V = P.V;
  const int lo = j * CH;
  const int n = (V - lo) < CH ? (V - lo) : CH;
  constexpr int ES = CK::ES;
  const void* row = reinterpret_cast<const char*>(P.logits) +
                    ES * ((int64_t)(r / P.rows_inner) * P.stride_outer + (int64_t)(r % P.rows_inner) * P.stride_inner);
  ChunkSum1* s1 = F.sum1 + (int64_t)r * F.s_stride;
  ChunkSum2* s2 = F.sum2 + (int64_t)r * F.s_stride;
  float* hist = F.hist + (int64_t)r * F.h_stride;
  uint2* cands = F.cands + (int64_t)r * F.c_stride;
  uint32_t* ctr = F.counters + (int64_t)r * 32;

  // ---- history ids, then the chunk: both in flight together ----
  HistPrefetch hp;
  prefetch_history(P.history ? P.history + (int64_t)r * P.history_stride : nullptr, P.history_stride, hp);
  CK C;
  C.load(row, lo, n);
  const uint8_t* am = row_allowed(P, r);
  C.mask(am, lo, n);

  const RowCfg g = row_cfg(P, r);
  const float T = g.T, topp = g.topp, rep = g.rep, pres = g.pres, freq = g.freq;
  const bool greedy = g.greedy, pen = g.pen;
  const int ntop = g.ntop, mode = g.mode, kprime = g.kprime, hlen = g.hlen;
  const int32_t* hrow = g.hrow;
  if (mode == MODE_DEFER) return mode;  // the general algorithm samples the row

  // ---- penalties from a per-chunk count table ----
  uint32_t cflags = 0;
  const PenArgs pa{S.hc, rep, pres, freq};
  if (pen) {
    if (hlen > 65535) cflags |= CF_HISTORY;  // counts are at most 16-bit: such rows take the general path
    if constexpr (PK) {
      if (!build_counts<8>(S.hc, hrow, hlen, hp, lo, n, S)) cflags |= CF_HISTORY;
      mark_counts(C, n, pa);
    } else {
      build_counts<16>(S.hc, hrow, hlen, hp, lo, n, S);
      apply_counts(C, n, pa);
    }
  }
  const bool wpen = PK && pen && wballot(C.pmask != 0ull) != 0ull;  // this wave holds penalised slots
  LPS_STAMP(1);

  // ---- chunk max (NaN aside), NaN flag, greedy argmax, -inf count (slots xd xc xa xf) ----
  float tm = -INFINITY, tm2 = -INFINITY;  // thread max and (top-k' > 64) second max
  uint32_t tnan = 0, ninf = 0;
  uint64_t gbest = 0;
  const bool want_ninf = mode == MODE_PURE && P.kept_count;
  const bool want_top2 = kprime > 64;
  with_pen<PK>(wpen, [&](auto PT) {
    constexpr bool PEN = decltype(PT)::value;
    // one loop per case: no per-element branch on a row-uniform condition
    if (want_top2) {
#pragma unroll
      for (int s = 0; s < NE; s++) {
        const float v = C.template val<PEN>(s, pa);
        tnan |= v != v ? 1u : 0u;
        // branch-free top two (NaN counts as -inf here; the flag reports it)
        const float w = v != v ? -INFINITY : v;
        tm2 = fmaxf(tm2, fminf(tm, w));
        tm = fmaxf(tm, w);
      }
    } else {
#pragma unroll
      for (int s = 0; s < NE; s++) {
        const float v = C.template val<PEN>(s, pa);
        tnan |= v != v ? 1u : 0u;
        tm = fmaxf(tm, v);
      }
    }
    if (greedy) {
#pragma unroll
      for (int s = 0; s < NE; s++) {
        const int l = CK::local(s);
        if (l < n) {
          const uint64_t pk = ((uint64_t)f2key(C.template val<PEN>(s, pa)) << 32) |
                              (uint64_t)(0xFFFFFFFFu - (uint32_t)(lo + l));
          gbest = pk > gbest ? pk : gbest;
        }
      }
    }
    if (want_ninf) {
#pragma unroll
      for (int s = 0; s < NE; s++) ninf += (CK::local(s) < n && C.template val<PEN>(s, pa) == -INFINITY) ? 1u : 0u;
    }
  });
  const float tm_thread = tm;
  {
    const float wmx = wmax(tm);
    const uint32_t wnan = wreduce(tnan, OpOr{});
    const uint64_t wg = greedy ? wmax(gbest) : 0ull;
    const uint32_t wni = wsum(ninf);
    if (lane == 0) { S.xd[wv] = (double)wmx; S.xc[wv] = wnan; S.xa[wv] = wg; S.xf[wv] = wni; }
  }
  if (mode == MODE_NUCLEUS) S.hm[tid] = 0ull;  // HB == FT
  __syncthreads();
  const float cmax = (float)fmax(fmax(S.xd[0], S.xd[1]), fmax(S.xd[2], S.xd[3]));
  const bool anynan = (S.xc[0] | S.xc[1] | S.xc[2] | S.xc[3]) != 0u;
  if (greedy) {
    uint64_t b = S.xa[0];
    for (int i = 1; i < FW; i++) b = S.xa[i] > b ? S.xa[i] : b;
    gbest = b;
  }
  ninf = S.xf[0] + S.xf[1] + S.xf[2] + S.xf[3];
  const uint32_t mkey = greedy ? (uint32_t)(gbest >> 32) : (anynan ? 0xFFFFFFFFu : f2key(cmax));
  const int amax = greedy ? (int)(0xFFFFFFFFu - (uint32_t)gbest) : 0;
  const float xm = key2f(mkey);
  const bool xm_finite = mkey != 0xFFFFFFFFu && xm != INFINITY && xm != -INFINITY;
  const float Te = greedy ? 1.0f : T;
  const float c = __fdiv_rn(kLog2e, Te);
  if (greedy && anynan && kprime > 0) cflags |= CF_OVERFLOW;  // NaN ranking: general path
  LPS_STAMP(2);

  // ---- chunk mass and the nucleus histogram ----
  const bool need_sum = mode == MODE_PURE || mode == MODE_NUCLEUS || P.chosen_logprob || ntop > 0;
  double acc = 0.0;
  int btop = 0;
  if (need_sum && xm_finite) {
    const float wm = __fmul_rn(xm, c);
    btop = (int)floorf(__fmul_rn(wm, (float)HS));
    with_pen<PK>(wpen, [&](auto PT) {
      constexpr bool PEN = decltype(PT)::value;
      if (mode == MODE_NUCLEUS) {
#pragma unroll
        for (int s = 0; s < NE; s++) {
          const float w = __fmul_rn(C.template val<PEN>(s, pa), c);
          const float e = chunk_mass(w, wm);
          acc += (double)e;
          if (e > 0.0f) {
            const int hb = btop - (int)floorf(__fmul_rn(w, (float)HS));
            if (hb < HB) atomicAdd(&S.hm[hb], (unsigned long long)mass_fixed(e));
          }
        }
      } else {
#pragma unroll
        for (int s = 0; s < NE; s++) acc += (double)chunk_mass(__fmul_rn(C.template val<PEN>(s, pa), c), wm);
      }
    });
  }
  LPS_STAMP(3);

  // ---- local top-k' threshold per wave, by ballot selection (slots xe xg) ----
  {
    const double wacc = wsum(acc);
    if (lane == 0) S.xe[wv] = wacc;
  }
  if (kprime > 0) {
    const uint32_t m = (uint32_t)((kprime + FW - 1) / FW);
    uint32_t th;
    if (!want_top2) {
      const uint32_t v1[1] = {f2key(tm_thread)};
      th = wave_kth_largest<1>(v1, m);
    } else {
      const uint32_t v2[2] = {f2key(tm_thread), f2key(tm2)};
      th = wave_kth_largest<2>(v2, m);
    }
    if (lane == 0) S.xg[wv] = th;
  }
  LPS_STAMP(25);
  __syncthreads();
  const double zsum = S.xe[0] + S.xe[1] + S.xe[2] + S.xe[3];

  // ---- local candidates: every element >= the weakest wave threshold (slot xh) ----
  uint32_t ncand = 0;
  if (kprime > 0) {
    uint32_t th = min(min(S.xg[0], S.xg[1]), min(S.xg[2], S.xg[3]));
    if (!greedy && th > kNegInfKey + 1u && th != 0xFFFFFFFFu) th = f2key(collision_lo(key2f(th), T));
    const float xth = key2f(th);
    LPS_STAMP(26);
    uint32_t cnt = 0;
    with_pen<PK>(wpen, [&](auto PT) {
      constexpr bool PEN = decltype(PT)::value;
#pragma unroll
      for (int s = 0; s < NE; s++) cnt += (CK::local(s) < n && C.template val<PEN>(s, pa) >= xth) ? 1u : 0u;
    });
    uint32_t tot;
    uint32_t p = bscan_excl<uint32_t>(cnt, &tot, S.xh);
    LPS_STAMP(27);
    uint2* out = cands + (int64_t)j * PUB;
    if (cnt) {
      with_pen<PK>(wpen, [&](auto PT) {
        constexpr bool PEN = decltype(PT)::value;
#pragma unroll
        for (int s = 0; s < NE; s++) {
          const float v = C.template val<PEN>(s, pa);
          const int l = CK::local(s);
          if (l < n && v >= xth) {
            if (p < (uint32_t)PUB) out[p] = make_uint2(f2key(v), (uint32_t)(lo + l));
            p++;
          }
        }
      });
    }
    ncand = tot > (uint32_t)PUB ? (uint32_t)PUB : tot;
    if (tot > (uint32_t)PUB) cflags |= CF_OVERFLOW;
  }
  LPS_STAMP(4);

  // ---- phase-1 summary ----
  if (tid == 0) {
    ChunkSum1 a;
    a.mkey = mkey; a.amax = amax; a.zsum = zsum; a.btop = btop; a.ninf = ninf; a.flags = cflags;
    a.xcc = xcc_id();
    s1[j] = a;
  }

  // ---- nucleus: histograms, one intra-XCD barrier, the common cut region ----
  uint64_t above = 0;
  uint32_t nabove = 0;
  int blo = 0, bhi = -1, rsub = 0;
  if (mode == MODE_NUCLEUS) {
    hist[(int64_t)j * HB + tid] = (float)((double)S.hm[tid] / (double)kMassScale);
    wait_stores();
    __syncthreads();
    if (tid == 0) {
      S.mi[9] = 0;
      l2_fetch_add(ctr + 2, 1u);
      // the row's chunk workgroups share one XCD and are dispatched in order, so
      // all of them are resident: the wait ends.  The bound only guards a broken launch.
      int spins = 0;
      while (ld_l2_u32(ctr + 2) < (uint32_t)G) {
        if (++spins > (1 << 20)) { S.mi[9] = 1; break; }
        __builtin_amdgcn_s_sleep(2);
      }
    }
    __syncthreads();
    LPS_STAMP(5);
    // Every chunk's relative bin tid (up to 32 chunks per round) is loaded together
    // with the chunk summaries; the bins are then merged in absolute position,
    // rescaled to the row maximum, in fixed point (order-independent sums).
    float hv[32];
    const int g0 = G < 32 ? G : 32;
#pragma unroll
    for (int k = 0; k < 32; k++)
      if (k < g0) hv[k] = hist[(int64_t)k * HB + tid];
    if (wv == 0) {
      ChunkSum1 a{};
      if (lane < G) a = s1[lane];
      const uint32_t gk = wmax(lane < G ? a.mkey : 0u);
      const float xg = key2f(gk);
      const bool rfin = gk != 0xFFFFFFFFu && xg != INFINITY && xg != -INFINITY;
      const float wg = rfin ? __fmul_rn(xg, c) : 0.0f;
      const float xq = key2f(a.mkey);
      const bool qfin = lane < G && a.mkey != 0xFFFFFFFFu && xq != INFINITY && xq != -INFINITY;
      const double sc = (rfin && qfin) ? exp2((double)__fmul_rn(xq, c) - (double)wg) : 0.0;
      const double Z = wsum(a.zsum * sc);
      if (lane < G) { S.scale[lane] = sc; S.btop[lane] = a.btop; }
      if (lane == 0) { S.md[0] = Z; S.mi[10] = rfin ? (int)floorf(__fmul_rn(wg, (float)HS)) : 0; S.mi[11] = rfin ? 1 : 0; }
    }
    S.gm[tid] = 0ull;
    __syncthreads();
    const bool rfin = S.mi[11] != 0;
    const int btg = S.mi[10];
    const double Z = S.md[0];
    const double Pm = (double)topp * Z;
    constexpr double kGm = 1099511627776.0;  // 2^40
    if (rfin) {
#pragma unroll
      for (int k = 0; k < 32; k++) {
        if (k < g0) {
          const int a = tid + (btg - S.btop[k]);
          const double sc = S.scale[k];
          if (sc > 0.0 && a < HB && hv[k] > 0.0f) atomicAdd(&S.gm[a], (unsigned long long)((double)hv[k] * sc * kGm));
        }
      }
      for (int q = 32; q < G; q++) {  // rows of more than 32 chunks
        const int a = tid + (btg - S.btop[q]);
        const double sc = S.scale[q];
        const float h = hist[(int64_t)q * HB + tid];
        if (sc > 0.0 && a < HB && h > 0.0f) atomicAdd(&S.gm[a], (unsigned long long)((double)h * sc * kGm));
      }
    }
    __syncthreads();
    // merged mass of absolute bin btg - tid (slot xd)
    const double m = (double)S.gm[tid] / kGm;
    double mtot;
    const double ex = bscan_excl<double>(m, &mtot, S.xd);
    // bins whose cumulative interval meets [Pm - eps, Pm + eps] (slots xg xh)
    const double eps = 1e-5 * Z;
    const bool meets = rfin && m > 0.0 && ex + m >= Pm - eps && ex <= Pm + eps;
    {
      const int tl = wmin(meets ? tid : (1 << 30));
      const int th = wmax(meets ? tid : -1);
      if (lane == 0) { S.xg[wv] = (uint32_t)tl; S.xh[wv] = (uint32_t)th; }
    }
    __syncthreads();
    const int tmin = min(min((int)S.xg[0], (int)S.xg[1]), min((int)S.xg[2], (int)S.xg[3]));
    const int tmax = max(max((int)S.xh[0], (int)S.xh[1]), max((int)S.xh[2], (int)S.xh[3]));
    LPS_STAMP(19);
    if (S.mi[9] == 1 || (rfin && tmax < 0)) {
      cflags |= CF_REGION;
    } else if (rfin) {
      bhi = btg - tmin;
      blo = btg - tmax;
      // ---- level 2: a coarse region holding many elements is split into 2^sub
      // fine bins per bin; the fine bins are merged over the row after a second
      // barrier, and the fine bins meeting the interval become the region ----
      // The region's element count is bounded from its merged masses (an element
      // of absolute bin btg - t has mass >= 2^-(t + 1) / 8 of the row maximum).
      const bool inr = tid >= tmin && tid <= tmax;
      const double cest = inr ? m * exp2((double)(tid + 1) * 0.125) : 0.0;
      const double nest = bcombine(wsum(cest), S.xe, OpAdd{});
      const int nreg = bhi - blo + 1;
      int sub = 0;
      if (nest > (double)LPS_FINE_MIN)
        while (sub < FSUB_MAX && (nreg << (sub + 1)) <= FB) sub++;
      int flo = blo << sub, fhi = ((bhi + 1) << sub) - 1;  // the region in fine bins (absolute)
      const float wmc = __fmul_rn(xm, c);
      auto fbin_of = [&](float v) -> int { return (int)floorf(__fmul_rn(__fmul_rn(v, c), (float)(HS << sub))); };
      uint64_t afm = 0ull;  // exact mass of this chunk's fine bins above the fine region (thread tid: fine bin tid)
      if (sub > 0) {
        const int nf = nreg << sub;  // fine bins of the coarse region, <= FB
        const int fb0 = flo;
        S.fm[tid] = 0ull;  // FB == FT
        if (tid == tmin) S.md[1] = ex;  // merged mass above the coarse region
        __syncthreads();
        with_pen<PK>(wpen, [&](auto PT) {
          constexpr bool PEN = decltype(PT)::value;
#pragma unroll
          for (int s = 0; s < NE; s++) {
            const float v = C.template val<PEN>(s, pa);
            const bool fin = v != -INFINITY;
            const float w = fin ? __fmul_rn(v, c) : 0.0f;
            const int fi = (int)floorf(__fmul_rn(w, (float)(HS << sub))) - fb0;
            if (fin && fi >= 0 && fi < nf) atomicAdd(&S.fm[fi], (unsigned long long)mass_fixed(chunk_mass(w, wmc)));
          }
        });
        __syncthreads();
        float* hfine = hist + (int64_t)G * HB;  // G x FB fine masses (chunk reference), after the G x HB bins
        hfine[(int64_t)j * FB + tid] = (float)((double)S.fm[tid] / (double)kMassScale);
        wait_stores();
        __syncthreads();
        if (tid == 0) {
          l2_fetch_add(ctr + 4, 1u);
          int spins = 0;
          while (ld_l2_u32(ctr + 4) < (uint32_t)G) {
            if (++spins > (1 << 20)) { S.mi[9] = 1; break; }
            __builtin_amdgcn_s_sleep(2);
          }
        }
        __syncthreads();
        // fine bin nf - 1 - tid (top first) of every chunk, rescaled to the row
        // maximum, summed in fixed point in one register per bin
        const int fi = nf - 1 - tid;
        uint64_t mf = 0ull;
        if (fi >= 0) {
          for (int q = 0; q < G; q++) {
            const float h = hfine[(int64_t)q * FB + fi];
            const double sc = S.scale[q];
            if (sc > 0.0 && h > 0.0f) mf += (unsigned long long)((double)h * sc * kGm);
          }
        }
        const double m2 = (double)mf / kGm;
        double mtot2;
        const double ex2 = S.md[1] + bscan_excl<double>(m2, &mtot2, S.xd);
        const bool meets2 = m2 > 0.0 && ex2 + m2 >= Pm - eps && ex2 <= Pm + eps;
        const int f1 = (int)bcombine(wmin(meets2 ? (uint32_t)tid : (1u << 30)), S.xg, OpMin{});
        const int f2 = (int)bcombine(wmax(meets2 ? (uint32_t)tid + 1u : 0u), S.xh, OpMax{}) - 1;
        if (f2 >= 0) {  // else the coarse region stays (its fine bins all)
          fhi = fb0 + (nf - 1 - f1);
          flo = fb0 + (nf - 1 - f2);
        }
        if (S.mi[9] == 1) cflags |= CF_REGION;
        if (tid < nf && fb0 + tid > fhi) afm = (uint64_t)S.fm[tid];
      }
      // this chunk: mass and count above the region, candidates inside (slots xa xb xc)
      const int hbt = btop - (bhi + 1);  // chunk histogram bins 0..hbt lie above the coarse region
      uint64_t am = ((xm_finite && tid <= hbt) ? (uint64_t)S.hm[tid] : 0ull) + afm;
      uint32_t na = 0, nc = 0;
      uint64_t inreg = 0;
      with_pen<PK>(wpen, [&](auto PT) {
        constexpr bool PEN = decltype(PT)::value;
#pragma unroll
        for (int s = 0; s < NE; s++) {
          const float v = C.template val<PEN>(s, pa);
          if (v != -INFINITY) {
            const int b = fbin_of(v);
            na += b > fhi ? 1u : 0u;
            const bool in = b >= flo && b <= fhi;
            nc += in ? 1u : 0u;
            if (NE <= 64) inreg |= in ? (1ull << (s & 63)) : 0ull;
          }
        }
      });
      am = wsum(am);
      na = wsum(na);
      if (lane == 0) { S.xa[wv] = am; S.xb[wv] = na; }
      uint32_t ctot;
      uint32_t p = bscan_excl<uint32_t>(nc, &ctot, S.xc);
      above = S.xa[0] + S.xa[1] + S.xa[2] + S.xa[3];
      nabove = (uint32_t)(S.xb[0] + S.xb[1] + S.xb[2] + S.xb[3]);
      uint2* out = cands + (int64_t)j * PUB;
      if (nc) {
        with_pen<PK>(wpen, [&](auto PT) {
          constexpr bool PEN = decltype(PT)::value;
#pragma unroll
          for (int s = 0; s < NE; s++) {
            bool in;
            float v;
            if constexpr (NE <= 64) {
              in = (inreg >> s) & 1ull;
              v = in ? C.template val<PEN>(s, pa) : 0.0f;
            } else {
              v = C.template val<PEN>(s, pa);
              const int b = v != -INFINITY ? fbin_of(v) : (flo - 1);
              in = b >= flo && b <= fhi;
            }
            if (in) {
              if (p < (uint32_t)PUB) out[p] = make_uint2(f2key(v), (uint32_t)(lo + CK::local(s)));
              p++;
            }
          }
        });
      }
      ncand = ctot > (uint32_t)PUB ? (uint32_t)PUB : ctot;
      if (ctot > (uint32_t)PUB) cflags |= CF_OVERFLOW;
      blo = flo;  // the summary carries the region in fine bins, and sub
      bhi = fhi;
      rsub = sub;
    }
    LPS_STAMP(20);
  }

  // ---- the chunk's summary for the row's finaliser (next kernel) ----
  LPS_STAMP(6);
  if (tid == 0) {
    ChunkSum2 a;
    a.ncand = ncand; a.flags = cflags; a.above = above; a.nabove = nabove; a.blo = blo; a.bhi = bhi; a.sub = (uint32_t)rsub;
    s2[j] = a;
  }
  return mode;
}

// The finaliser of row r, after every chunk of the row has published.  fused:
// it runs in the row's last chunk workgroup, in the chunks' kernel, and reads
// their data through the XCD's L2.  Returns 0 when the row is done, or a
// positive reason code when the general algorithm must sample it.
template <int DT, int VEC, int NR>
__device__ __forceinline__ int final_body(const FParams& F, FSharedT<NR>& S, const int r, const bool fused) {
  using CK = Chunk<DT, VEC, NR>;
  constexpr int PUB = CK::PUB;
  constexpr int CH = CK::CH, NV = CK::NV;
  constexpr bool PK = CK::PACKED;
  const KParams& P = F.k;
  const int G = F.G;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int V = P.V;
  constexpr int ES = CK::ES;
  const void* row = reinterpret_cast<const char*>(P.logits) +
                    ES * ((int64_t)(r / P.rows_inner) * P.stride_outer + (int64_t)(r % P.rows_inner) * P.stride_inner);
  ChunkSum1* s1 = F.sum1 + (int64_t)r * F.s_stride;
  ChunkSum2* s2 = F.sum2 + (int64_t)r * F.s_stride;
  uint2* cands = F.cands + (int64_t)r * F.c_stride;
  if (tid == 0) {  // the row's counters back to zero for the next launch
    F.counters[(int64_t)r * 32] = 0u;
    F.counters[(int64_t)r * 32 + 2] = 0u;
    F.counters[(int64_t)r * 32 + 4] = 0u;
  }
  const RowCfg g = row_cfg(P, r);
  if (g.mode == MODE_DEFER) return 1;
  const float T = g.T, topp = g.topp, minp = g.minp, typp = g.typp, rep = g.rep, pres = g.pres, freq = g.freq;
  const bool greedy = g.greedy, pen = g.pen;
  const int topk = g.topk, ntop = g.ntop, mode = g.mode, kprime = g.kprime, hlen = g.hlen;
  const int64_t qtok = g.qtok;
  const int32_t* hrow = g.hrow;
  const float c = __fdiv_rn(kLog2e, greedy ? 1.0f : T);
  LPS_FSTAMP(7);

  // =========================== finaliser ===========================
  // F1: wave 0 gathers the per-chunk summaries.
  if (wv == 0) {
    ChunkSum1 a{};
    ChunkSum2 b{};
    if (lane < G) { a = s1[lane]; b = s2[lane]; }
    // chunks that exchanged data through one L2 must have run on one XCD
    const uint32_t xm = wreduce(lane < G ? (1u << a.xcc) : 0u, OpOr{});
    const bool split = __builtin_popcount(xm) > 1 && (fused || g.mode == MODE_NUCLEUS);
    const uint32_t fl = wreduce(lane < G ? (a.flags | b.flags) : 0u, OpOr{}) | (split ? (uint32_t)CF_SPLIT : 0u);
    const uint32_t ninf_all = wsum(lane < G ? a.ninf : 0u);
    const uint32_t nc = lane < G ? b.ncand : 0u;
    const uint32_t ncinc = wscan_incl(nc);
    const uint32_t NC = rdlane(ncinc, 63);
    const uint32_t nab = wsum(lane < G ? b.nabove : 0u);
    const uint64_t pk = wmax(lane < G ? (((uint64_t)a.mkey << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)a.amax)) : 0ull);
    const uint32_t gkey = (uint32_t)(pk >> 32);
    const float xg = key2f(gkey);
    const bool rfin = gkey != 0xFFFFFFFFu && xg != INFINITY && xg != -INFINITY;
    const double wgd = rfin ? (double)__fmul_rn(xg, c) : 0.0;
    const float xq = key2f(a.mkey);
    const bool qfin = lane < G && a.mkey != 0xFFFFFFFFu && xq != INFINITY && xq != -INFINITY;
    const float wq = (rfin && qfin) ? __fmul_rn(xq, c) : 0.0f;
    const double sc = (rfin && qfin) ? exp2((double)wq - wgd) : 0.0;
    const double Zfull = wsum(a.zsum * sc);
    const double abv = (double)b.above / (double)kMassScale * sc;
    const double A = wsum(abv);
    if (lane < G) {
      S.pre[lane] = ncinc - nc;
      S.scale[lane] = sc;
      S.wm[lane] = wq;
      S.abvm[lane] = abv;
      S.keptm[lane] = a.zsum * sc;
      S.keptf[lane] = 0ull;
    }
    if (lane == 0) {
      S.pre[G] = NC;
      S.mi[18] = b.blo;  // every chunk derived the same cut region (fine bins of 2^-(3 + sub) log2 units)
      S.mi[19] = b.bhi;
      S.mi[31] = (int)b.sub;
      S.mi[12] = (int)fl;
      S.mi[13] = (int)NC;
      S.mi[14] = (int)ninf_all;
      S.mi[15] = (int)nab;
      S.mi[16] = (int)gkey;
      S.mi[17] = (int)(0xFFFFFFFFu - (uint32_t)pk);
      S.md[1] = Zfull;
      S.md[2] = A;
    }
  }
  __syncthreads();
  const uint32_t fl = (uint32_t)S.mi[12];
  const int blo = S.mi[18], bhi = S.mi[19], rsub = S.mi[31];
  auto rbin = [&](float x) -> int { return (int)floorf(__fmul_rn(__fmul_rn(x, c), (float)(HS << rsub))); };
  if (fl & (CF_OVERFLOW | CF_HISTORY | CF_SPLIT | CF_REGION)) return (int)fl;
  const int NC = S.mi[13];
  const uint32_t ninf_all = (uint32_t)S.mi[14];
  const uint32_t nab_all = (uint32_t)S.mi[15];
  const uint32_t gkey = (uint32_t)S.mi[16];
  const int gam = S.mi[17];
  const double Zfull = S.md[1];
  const double Aabove = S.md[2];
  LPS_FSTAMP(8);

  const float xmax = key2f(gkey);
  const bool has_nan = gkey == 0xFFFFFFFFu;
  const float zmax = greedy ? xmax : __fdiv_rn(xmax, T);
  int status = 0;
  if (!greedy) {
    if (has_nan || xmax == INFINITY || zmax == INFINITY) status |= LPS_ROW_NONFINITE;
    else if (xmax == -INFINITY) status |= LPS_ROW_EMPTY;
  }
  const double lnZ = Zfull > 0.0 ? log(Zfull) : 0.0;
  float u = g.u;
  if (!(u >= 0.0f)) u = 0.0f;
  if (u >= 1.0f) u = 0.99999994f;

  int64_t token = -1;
  float cut = -INFINITY, qprob = 0.0f, chosen_z = NAN;
  int32_t ties = -1, kept_n = 0;
  int ntop_out = 0;  // entries of the sorted kept list that are top logprobs

  // Candidate i (concatenated over chunks in chunk order) sits in slot
  // i - pre[q] of chunk q, the last chunk with pre[q] <= i.
  auto cand_at = [&](int i) -> uint2 {
    int q = 0;
#pragma unroll
    for (int step = MAXG / 2; step > 0; step >>= 1)
      if (q + step < G && (int)S.pre[q + step] <= i) q += step;
    return cands[(int64_t)q * PUB + (i - (int)S.pre[q])];
  };
  // Candidates: thread t holds candidate e * FT + t in slot e, its z key in
  // register ck[e] and its vocabulary index in S.cidx[e * FT + t] (LDS, read
  // only by that thread: the index is needed for few candidates, and 16 more
  // registers would cost the fused kernel a workgroup per CU).
  uint32_t ck[FCPT];
  auto ci = [&](int e) -> int32_t { return S.cidx[e * FT + tid]; };
  const int np = NC > tid ? min((NC - tid + FT - 1) / FT, FCPT) : 0;
  // The chunk of every slot's candidate by one binary search over pre[], its
  // steps interleaved over the slots (one LDS round trip per step), then all
  // loads (clamped to a valid candidate, no branch between them), then the keys.
  auto load_cands = [&]() {
    const int npmax = min((NC + FT - 1) / FT, FCPT);  // slots any thread uses
    auto idx = [&](int e) { return min(e * FT + tid, NC - 1); };
    int q[FCPT];
#pragma unroll
    for (int e = 0; e < FCPT; e++) q[e] = 0;
#pragma unroll
    for (int step = MAXG / 2; step > 0; step >>= 1) {
      int pv[FCPT];
#pragma unroll
      for (int e = 0; e < FCPT; e++) pv[e] = (int)S.pre[min(q[e] + step, G)];  // pre[G] = NC > any index
#pragma unroll
      for (int e = 0; e < FCPT; e++) q[e] += (q[e] + step < G && pv[e] <= idx(e)) ? step : 0;
    }
#pragma unroll
    for (int e = 0; e < FCPT; e++) q[e] = q[e] * PUB + (idx(e) - (int)S.pre[q[e]]);  // slot in cands
    uint2 cv[FCPT];
#pragma unroll
    for (int e = 0; e < FCPT; e++)
      if (e < npmax) cv[e] = cands[q[e]];
#pragma unroll
    for (int e = 0; e < FCPT; e++) {
      const bool pr = e < np;
      const float xv = key2f(pr ? cv[e].x : 0u);
      ck[e] = pr ? f2key(greedy ? xv : __fdiv_rn(xv, T)) : 0u;
      if (pr) S.cidx[e * FT + tid] = (int32_t)cv[e].y;
    }
  };

  if (status == 0 && kprime > 0) {
    // ---------------- top-k (and top-N logprobs) ----------------
    if (NC > FCAP) return 512;
    load_cands();
    LPS_FSTAMP(22);
    const int keff = mode == MODE_TOPK ? (topk < V ? topk : V) : 0;
    int kc = keff > ntop ? keff : ntop;
    if (kc > NC) kc = NC;
    if (kc <= 0) return 16;
    const uint32_t zc = sel_count(ck, np, (uint32_t)kc, S);
    LPS_FSTAMP(23);
    // collect z >= zc into the kept list (slot xh)
    uint32_t cnt = 0;
#pragma unroll
    for (int e = 0; e < FCPT; e++) cnt += (e < np && ck[e] >= zc) ? 1u : 0u;
    uint32_t Kall;
    uint32_t p = bscan_excl<uint32_t>(cnt, &Kall, S.xh);
    if (Kall > (uint32_t)KEPTCAP) return 32;
    auto& kl = S.x.k;
#pragma unroll
    for (int e = 0; e < FCPT; e++) {
      if (e < np && ck[e] >= zc) {
        const int32_t ix = ci(e);
        kl.skey[p] = ((uint64_t)ck[e] << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)ix);
        kl.kidx[p] = ix;
        kl.km[p] = mass_fixed(mass_f(key2f(ck[e]), zmax));
        p++;
      }
    }
    __syncthreads();
    LPS_FSTAMP(24);
    const int K = (int)Kall;
    rank_sort_kept(K, S);
    auto kz = [&](int slot) -> uint32_t { return (uint32_t)(kl.skey[slot] >> 32); };
    ntop_out = ntop < K ? ntop : K;
    LPS_FSTAMP(16);
    if (mode == MODE_GREEDY) {
      token = gam;
      cut = xmax;
      ties = 1;
      kept_n = 1;
      qprob = (qtok >= 0 && qtok == gam) ? 1.0f : 0.0f;
      chosen_z = xmax;
    } else {
      // the top-k set: sorted positions whose key reaches the keff-th largest
      if (keff > K) return 16;
      const uint32_t kth = kz(kl.kord[keff - 1]);
      if (tid == 0) S.mi[20] = K;
      __syncthreads();
      for (int pz = tid; pz < K; pz += FT)
        if (kz(kl.kord[pz]) >= kth && (pz == K - 1 || kz(kl.kord[pz + 1]) < kth)) S.mi[20] = pz + 1;
      __syncthreads();
      const int nk = S.mi[20];
      sorted_prefix(nk, S);
      const uint64_t Zk = kl.cum[nk - 1];
      int nf = nk;
      if (topp < 1.0f) {  // keep sorted position p iff p == 0 or cum[p-1] <= p * Zk
        const double pl = topp > 0.0f ? (double)topp * (double)Zk : 0.0;
        uint64_t limit = (uint64_t)pl;
        if (limit >= Zk) limit = Zk - 1;
        if (tid == 0) S.mi[21] = nk;
        __syncthreads();
        for (int pz = tid; pz < nk; pz += FT)
          if (kl.cum[pz] > limit && (pz == 0 || kl.cum[pz - 1] <= limit)) S.mi[21] = pz + 1;
        __syncthreads();
        nf = S.mi[21];
      }
      if (minp > 0.0f) {  // keep e >= min_p (the maximum has e == 1)
        if (tid == 0) S.mi[22] = nf;
        __syncthreads();
        for (int pz = tid; pz < nf; pz += FT) {
          const bool ok = mass_f(key2f(kz(kl.kord[pz])), zmax) >= minp;
          const bool okp = pz == 0 || mass_f(key2f(kz(kl.kord[pz - 1])), zmax) >= minp;
          if (!ok && okp) S.mi[22] = pz;
        }
        __syncthreads();
        nf = S.mi[22];
        if (nf == 0) status |= LPS_ROW_EMPTY;
      }
      // typical-p with top-k active: the row holds -inf, the reference keeps only the argmax
      if (status == 0 && typp < 1.0f) nf = 1;
      if (status == 0) {
        const uint64_t Zf = kl.cum[nf - 1];
        const uint32_t ckey = kz(kl.kord[nf - 1]);
        cut = key2f(ckey);
        if (P.kept_ties || P.kept_count) {  // (slots xc xf xg)
          uint32_t ea = 0, ek = 0, nfin = 0;
          for (int q = tid; q < K; q += FT) {
            const uint32_t kq = kz(kl.kord[q]);
            ea += kq == ckey ? 1u : 0u;
            ek += (kq == ckey && q < nf) ? 1u : 0u;
            nfin += (q < nf && kq != kNegInfKey) ? 1u : 0u;
          }
          ea = wsum(ea); ek = wsum(ek); nfin = wsum(nfin);
          if (lane == 0) { S.xc[wv] = ea; S.xf[wv] = ek; S.xg[wv] = nfin; }
          __syncthreads();
          ea = S.xc[0] + S.xc[1] + S.xc[2] + S.xc[3];
          ek = S.xf[0] + S.xf[1] + S.xf[2] + S.xf[3];
          nfin = S.xg[0] + S.xg[1] + S.xg[2] + S.xg[3];
          ties = ek == ea ? -1 : (int32_t)ek;
          kept_n = (int32_t)nfin;
        }
        // vocabulary order over the kept prefix: the kept indices in sorted order
        // (in iord), then each one's rank among them
        for (int pz = tid; pz < nf; pz += FT) kl.iord[pz] = kl.kidx[kl.kord[pz]];
        __syncthreads();
        int rk0 = -1, rk1 = -1;
        for (int pz = tid; pz < nf; pz += FT) {
          const int rk = count_below(kl.iord, nf, kl.iord[pz]);
          if (pz == tid) rk0 = rk; else rk1 = rk;
        }
        __syncthreads();
        if (tid < nf) kl.iord[rk0] = kl.kord[tid];
        if (tid + FT < nf) kl.iord[rk1] = kl.kord[tid + FT];
        if (tid == 0) { S.mi[23] = -1; S.mi[24] = -1; }
        __syncthreads();
        // inverse CDF in vocabulary order: thread t holds positions 2t, 2t+1 (slot xb)
        const int p0 = 2 * tid, p1 = 2 * tid + 1;
        const uint64_t m0 = p0 < nf ? (uint64_t)kl.km[kl.iord[p0]] : 0ull;
        const uint64_t m1 = p1 < nf ? (uint64_t)kl.km[kl.iord[p1]] : 0ull;
        uint64_t mt;
        const uint64_t e0 = bscan_excl<uint64_t>(m0 + m1, &mt, S.xb);
        uint64_t target = (uint64_t)((double)u * (double)Zf);
        if (target >= Zf) target = Zf - 1;
        if (m0 && e0 <= target && target < e0 + m0) S.mi[23] = kl.iord[p0];
        if (m1 && e0 + m0 <= target && target < e0 + m0 + m1) S.mi[23] = kl.iord[p1];
        if (qtok >= 0) {
          if (p0 < nf && kl.kidx[kl.iord[p0]] == qtok) S.mi[24] = kl.iord[p0];
          if (p1 < nf && kl.kidx[kl.iord[p1]] == qtok) S.mi[24] = kl.iord[p1];
        }
        __syncthreads();
        const int ps = S.mi[23] >= 0 ? S.mi[23] : kl.iord[nf - 1];
        token = kl.kidx[ps];
        chosen_z = key2f(kz(ps));
        if (S.mi[24] >= 0) qprob = (float)((double)kl.km[S.mi[24]] / (double)Zf);
      }
    }
  } else if (status == 0 && mode == MODE_GREEDY) {
    token = gam;
    cut = xmax;
    ties = 1;
    kept_n = 1;
    qprob = (qtok >= 0 && qtok == gam) ? 1.0f : 0.0f;
    chosen_z = xmax;
  } else if (status == 0 && (mode == MODE_PURE || mode == MODE_NUCLEUS)) {
    // ---------------- pure / nucleus ----------------
    uint32_t vkey = 0, n_tie = kNoTie;
    int tie_lim = 0x7FFFFFFF;
    double qmass = -1.0;
    if (mode == MODE_PURE) {
      kept_n = V - (int)ninf_all;
    } else {
      // exact cut among the region candidates, above-region masses rescaled to the row
      if (NC > FCAP) return 64;
      load_cands();
      LPS_FSTAMP(25);
      auto cmass = [&](uint32_t key) -> uint64_t { return mass_fixed(mass_f(key2f(key), zmax)); };
      const uint64_t Af = (uint64_t)(Aabove * (double)kMassScale);
      const uint64_t Pf = (uint64_t)((double)topp * Zfull * (double)kMassScale);
      LPS_FSTAMP(16);
      const MassSel ms = sel_mass(ck, np, cmass, Af, Pf, S);
      LPS_FSTAMP(17);
      if (!ms.ok || ms.ceq == 0) return 64;
      vkey = ms.key;
      const uint64_t e1 = ms.meq / ms.ceq;
      const uint64_t nt = e1 ? (Pf - ms.above) / e1 + 1 : (uint64_t)ms.ceq;
      n_tie = nt >= ms.ceq ? kNoTie : (uint32_t)nt;
      // ties at the cut: the kept ones are the n_tie lowest indices (slot xh)
      auto& kl = S.x.k;
      if (tid == 0) { S.mi[25] = 0x7FFFFFFF; S.mi[26] = 0; S.md[6] = -1.0; }
      __syncthreads();
      if (n_tie != kNoTie) {
        uint32_t tc = 0;
#pragma unroll
        for (int e = 0; e < FCPT; e++) tc += (e < np && ck[e] == vkey) ? 1u : 0u;
        uint32_t ttot;
        uint32_t p = bscan_excl<uint32_t>(tc, &ttot, S.xh);
        if (ttot > (uint32_t)KEPTCAP) return 32;
#pragma unroll
        for (int e = 0; e < FCPT; e++)
          if (e < np && ck[e] == vkey) kl.kidx[p++] = ci(e);
        __syncthreads();
        LPS_FSTAMP(29);
        for (int i = tid; i < (int)ttot; i += FT) {
          const int ii = kl.kidx[i];
          if (count_below(kl.kidx, (int)ttot, ii) == (int)n_tie - 1) S.mi[25] = ii;
        }
      }
      // one candidate of the cut key (any: its x is reloaded by one thread)
#pragma unroll
      for (int e = 0; e < FCPT; e++)
        if (e < np && ck[e] == vkey) S.mi[26] = e * FT + tid;
      __syncthreads();
      tie_lim = S.mi[25];
      LPS_FSTAMP(18);
      if (wv == 0) {
        // the cut's division-collision group [xl, xh] = {x : fl(x / T) == cut},
        // which must lie inside the region.  Lane l tests the step from l to
        // l + 1 keys below (above) a candidate of the cut key; the group ends
        // at the first failing lane, after at most 64 steps each way.
        const float xv = key2f(cand_at(S.mi[26]).x);
        const float zc = key2f(vkey);
        const uint32_t k0 = f2key(xv);
        const uint32_t kd = k0 - (uint32_t)lane;
        const uint64_t fd = wballot(!(kd > kNegInfKey + 1u && __fdiv_rn(key2f(kd - 1u), T) == zc));
        const uint32_t ku = k0 + (uint32_t)lane;
        const uint64_t fu = wballot(!(ku < 0xFFFFFFFEu && __fdiv_rn(key2f(ku + 1u), T) == zc));
        if (lane == 0) {
          const bool ended = fd != 0ull, ended2 = fu != 0ull;
          const float xl = key2f(k0 - (ended ? (uint32_t)__builtin_ctzll(fd) : 64u));
          const float xh = key2f(k0 + (ended2 ? (uint32_t)__builtin_ctzll(fu) : 64u));
          const int bl = rbin(xl), bh = rbin(xh);
          S.mi[27] = (ended && ended2 && bl >= blo && bh <= bhi) ? 1 : 0;
          S.mf[0] = xl;
          S.mf[1] = xh;
        }
      }
      LPS_FSTAMP(14);
      // kept candidate mass per chunk and count (slot xg)
      uint32_t lc = 0;
#pragma unroll
      for (int e = 0; e < FCPT; e++) {
        const bool kept = e < np && (ck[e] > vkey || (ck[e] == vkey && ci(e) <= tie_lim));
        if (kept) {
          const int32_t ix = ci(e);
          const uint64_t m = cmass(ck[e]);
          atomicAdd(&S.keptf[ix / CH], (unsigned long long)m);
          if ((int64_t)ix == qtok) S.md[6] = (double)m / (double)kMassScale;
          lc++;
        }
      }
      LPS_FSTAMP(12);
      lc = wsum(lc);
      if (lane == 0) S.xg[wv] = lc;
      __syncthreads();
      if (!S.mi[27]) return 128;
      kept_n = (int32_t)(nab_all + S.xg[0] + S.xg[1] + S.xg[2] + S.xg[3]);
      qmass = S.md[6];
      if (wv == 0 && lane < G)
        S.keptm[lane] = S.abvm[lane] + (double)S.keptf[lane] / (double)kMassScale;
      __syncthreads();
      ties = n_tie == kNoTie ? -1 : (int32_t)n_tie;
      cut = key2f(vkey);
    }
    LPS_FSTAMP(9);
    // the chunk holding u * Zf (wave 0), then its exact scan in vocabulary order
    if (wv == 0) {
      const double km = lane < G ? S.keptm[lane] : 0.0;
      const double inc = wscan_incl(km);
      const double Zf = rdlane(inc, 63);
      const double target = (double)u * Zf;
      const uint64_t hit = wballot(km > 0.0 && target < inc);
      const uint64_t pos = wballot(km > 0.0);
      const int js = hit ? __builtin_ctzll(hit) : (pos ? 63 - __builtin_clzll(pos) : G - 1);
      const double start = rdlane(inc - km, js);
      if (lane == 0) { S.mi[28] = js; S.md[3] = start; S.md[4] = Zf; S.md[5] = target; }
    }
    __syncthreads();
    const int js = S.mi[28];
    const double start = S.md[3], Zf = S.md[4], target = S.md[5];
    if (!P.skip_draw) {
      const int lo2 = js * CH;
      const int n2 = (V - lo2) < CH ? (V - lo2) : CH;
      const float wmj = S.wm[js];
      const double scj = S.scale[js];
      HistPrefetch hp2;
      prefetch_history(hrow, P.history_stride, hp2);
      CK Y;
      Y.load(row, lo2, n2);
      Y.mask(row_allowed(P, r), lo2, n2);
      const PenArgs pa2{S.x.hc, rep, pres, freq};
      if (pen) {  // (a row whose counts did not fit never reaches the finaliser)
        if constexpr (PK) {
          build_counts<8>(S.x.hc, hrow, hlen, hp2, lo2, n2, S);
          mark_counts(Y, n2, pa2);
        } else {
          build_counts<16>(S.x.hc, hrow, hlen, hp2, lo2, n2, S);
          apply_counts(Y, n2, pa2);
        }
      }
      LPS_FSTAMP(21);
      // Kept mass of slot (v, e) with the formulas that built the chunk's kept
      // mass: exp2(x c - wm) * scale outside the cut region (as the chunk pass
      // summed it), the finaliser's exp(z - zmax) for region candidates.
      // Region candidates are kept when z = fl(x / T) is above the cut, i.e.
      // x > xh, or in the cut's collision group [xl, xh] with index <= tie_lim.
      const float cxl = S.mf[0], cxh = S.mf[1];
      auto kept_m = [&](int v, int e) -> double {
        const float yv = Y.template val<true>(v * VEC + e, pa2);
        if (yv == -INFINITY || yv != yv) return 0.0;
        const float w = __fmul_rn(yv, c);
        if (mode == MODE_NUCLEUS) {
          const int b = (int)floorf(__fmul_rn(w, (float)(HS << rsub)));
          if (b < blo) return 0.0;
          if (b <= bhi) {
            if (yv < cxl || (yv <= cxh && lo2 + (v * FT + tid) * VEC + e > tie_lim)) return 0.0;
            return (double)mass_fixed(mass_f(__fdiv_rn(yv, T), zmax)) / (double)kMassScale;
          }
        }
        return (double)chunk_mass(w, wmj) * scj;
      };
      // kept_m with its per-element branches turned into selects and one
      // wave-uniform branch around the region formula (every lane calls it):
      // the same values, without divergent control flow per element.
      auto kept_m_all = [&](int v, int e) -> double {
        const float yv = Y.template val<true>(v * VEC + e, pa2);
        const bool live = yv != -INFINITY && yv == yv;
        const float yl = live ? yv : 0.0f;
        const float w = __fmul_rn(yl, c);
        double m = (double)chunk_mass(w, wmj) * scj;
        if (mode == MODE_NUCLEUS) {
          const int b = (int)floorf(__fmul_rn(w, (float)(HS << rsub)));
          const bool inr = b >= blo && b <= bhi;
          m = b < blo ? 0.0 : m;
          if (wballot(live && inr)) {
            const bool kept = !(yl < cxl || (yl <= cxh && lo2 + (v * FT + tid) * VEC + e > tie_lim));
            const double mr = (double)mass_fixed(mass_f(__fdiv_rn(yl, T), zmax)) / (double)kMassScale;
            m = inr ? (kept ? mr : 0.0) : m;
          }
        }
        return live ? m : 0.0;
      };
      // Vocabulary order is (v, thread, e).  Groups are scanned in batches of NB;
      // each thread keeps its first group whose cumulative end passes the target
      // (slots xv, then xc xf).
      constexpr int NB = NV < 8 ? NV : 8;
      int myfirst = 0x7FFFFFFF, mylast = -1;
      double myoff = 0.0, base = start;
#pragma unroll
      for (int vb = 0; vb < NV; vb += NB) {
        double sv[NB], incv[NB];
#pragma unroll
        for (int b = 0; b < NB; b++) {
          double a = 0.0;
#pragma unroll
          for (int e = 0; e < VEC; e++) a += kept_m_all(vb + b, e);
          sv[b] = a;
          incv[b] = wscan_incl(a);
        }
        if (lane == 63) {
#pragma unroll
          for (int b = 0; b < NB; b++) S.xv[wv][b] = incv[b];
        }
        __syncthreads();
#pragma unroll
        for (int b = 0; b < NB; b++) {
          double wpre = 0.0, wtot = 0.0;
#pragma unroll
          for (int w = 0; w < FW; w++) {
            const double t = S.xv[w][b];
            wtot += t;
            wpre += w < wv ? t : 0.0;
          }
          const double off = base + wpre + incv[b] - sv[b];
          if (sv[b] > 0.0) {
            const int pos = (vb + b) * FT + tid;
            if (myfirst == 0x7FFFFFFF && off + sv[b] > target) { myfirst = pos; myoff = off; }
            mylast = pos;
          }
          base += wtot;
        }
        __syncthreads();
      }
      LPS_FSTAMP(26);
      {
        const int f = wmin(myfirst), l = wmax(mylast);
        if (lane == 0) { S.xc[wv] = (uint32_t)f; S.xf[wv] = (uint32_t)l; }
      }
      if (tid == 0) S.mi[29] = -1;
      __syncthreads();
      const int gf = min(min((int)S.xc[0], (int)S.xc[1]), min((int)S.xc[2], (int)S.xc[3]));
      const int gl = max(max((int)S.xf[0], (int)S.xf[1]), max((int)S.xf[2], (int)S.xf[3]));
      const bool found = gf != 0x7FFFFFFF;
      const int pick = found ? gf : gl;
      LPS_FSTAMP(27);
      if (pick >= 0 && (pick % FT) == tid) {
        // walk the group: the first kept element whose cumulative end passes the
        // target, or (no group passed it: rounding at the top end) the last kept one
        const int v = pick / FT;
        double a = myoff;
        int lp = -1;
        float lz = NAN;
        bool done = false;
#pragma unroll
        for (int vv = 0; vv < NV; vv++) {
          if (vv != v) continue;
#pragma unroll
          for (int e = 0; e < VEC; e++) {
            if (done) continue;
            const double m = kept_m(vv, e);
            if (m > 0.0) {
              lp = lo2 + (vv * FT + tid) * VEC + e;
              lz = __fdiv_rn(Y.template val<true>(vv * VEC + e, pa2), T);
              if (found && target < a + m) done = true;
              a += m;
            }
          }
        }
        S.mi[29] = lp;
        S.md[7] = (double)lz;
      }
      __syncthreads();
      token = S.mi[29];
      chosen_z = (float)S.md[7];
    }
    if (P.query_prob && qtok >= 0) {
      const float xq = penalized_logit<DT>(row, row_allowed(P, r), (int)qtok, hrow, hlen, pen, rep, pres, freq, S);
      const float zq = __fdiv_rn(xq, T);
      if (mode == MODE_PURE) {
        qprob = zq != -INFINITY ? (float)((double)mass_f(zq, zmax) / Zf) : 0.0f;
      } else {
        const int bq = rbin(xq);
        if (bq > bhi && zq != -INFINITY) qprob = (float)((double)mass_f(zq, zmax) / Zf);
        else if (qmass >= 0.0) qprob = (float)(qmass / Zf);
      }
    }
  }
  if (P.skip_draw && !greedy) token = -1;
  LPS_FSTAMP(10);

  // ---- outputs ----
  if (P.chosen_logprob && tid == 0) {
    float lp = NAN;
    if (token >= 0 && Zfull > 0.0 && chosen_z == chosen_z)
      lp = (float)((double)__fsub_rn(chosen_z, zmax) - lnZ);
    P.chosen_logprob[r] = lp;
  }
  if (ntop > 0 && status == 0) {
    auto& kl = S.x.k;
    for (int q = tid; q < P.n_top; q += FT) {
      if (q < ntop_out) {
        const int si = kl.kord[q];
        P.top_logprobs[(int64_t)r * P.n_top + q] =
            (float)((double)__fsub_rn(key2f((uint32_t)(kl.skey[si] >> 32)), zmax) - lnZ);
        if (P.top_ids) P.top_ids[(int64_t)r * P.n_top + q] = kl.kidx[si];
      } else {
        P.top_logprobs[(int64_t)r * P.n_top + q] = -INFINITY;
        if (P.top_ids) P.top_ids[(int64_t)r * P.n_top + q] = -1;
      }
    }
  }
  if (tid == 0) {
    P.tokens[r] = status ? -1 : token;
    append_token(P, r, status ? -1 : token);
    F.status[r] = status;
    if (P.row_status) P.row_status[r] = status;
    if (P.query_prob) P.query_prob[r] = qprob;
    if (P.kept_cut) P.kept_cut[r] = cut;
    if (P.kept_ties) P.kept_ties[r] = ties;
    if (P.kept_count) P.kept_count[r] = kept_n;
    if (P.row_path) P.row_path[r] = 0;
  }
  LPS_FSTAMP(11);
  return 0;
}

// Split path, phase 1: grid of ceil(R / 8) * 8 * G workgroups.
template <int DT, int VEC>
__global__ __launch_bounds__(FT) __attribute__((amdgpu_waves_per_eu(DT != LPS_DTYPE_F32 && VEC == 8 ? 5 : 4, 8))) void chunk_kernel(FParams F) {
  __shared__ CSharedT<32> S;
  const ChunkId c = chunk_id(F.G);
  if (c.r >= F.k.R) return;
  chunk_body<DT, VEC, 32>(F, S, c.r, c.j);
}

// Split path, phase 2: one workgroup per row.  A row the fast path cannot
// finish exactly is marked deferred in the workspace status (reason code in
// bits 8 and up); the general kernel, launched next with that status as its
// filter, samples it.
template <int DT, int VEC>
__global__ __launch_bounds__(FT) void final_kernel(FParams F) {
  __shared__ FSharedT<32> S;
  const int r = blockIdx.x;
  const int reason = final_body<DT, VEC, 32>(F, S, r, false);
  if (reason > 0 && threadIdx.x == 0) F.status[r] = LPS_ROW_DEFERRED | (reason << 8);
}

// Fused path (grids that fit on the GPU at once): the chunk kernel whose last
// workgroup of each row to finish, counted by an L2 atomic, finalises the row
// while other rows are still in their chunk phase.
// Waves per SIMD the fused kernel is built for: four workgroups per CU for
// 16-bit logits (<= 128 VGPRs, 37 KB LDS), three for fp32.
#ifndef LPS_FUSED_WPE
#define LPS_FUSED_WPE(DT) ((DT) == LPS_DTYPE_F32 ? 3 : 4)
#endif
#ifndef LPS_FUSED_NR16
#define LPS_FUSED_NR16 32
#endif
// Logit registers per thread of the fused kernel: 32, i.e. 8192-logit chunks
// for every dtype (16-bit logits are read 8 per 16-byte load and held as fp32).
template <int DT>
constexpr int fused_nr() { return DT == LPS_DTYPE_F32 ? 32 : LPS_FUSED_NR16; }
template <int DT, int VEC>
__global__ __launch_bounds__(FT) __attribute__((amdgpu_waves_per_eu(LPS_FUSED_WPE(DT), 8))) void fused_kernel(FParams F) {
  __shared__ union {
    CSharedT<fused_nr<DT>()> c;
    FSharedT<fused_nr<DT>()> f;
  } SU;
  ChunkId c = chunk_id(F.G);
  if (c.r >= F.k.R) return;
  if (F.heavy_first) c.r = heavy_first_row(F.k, c.r);
  const int mode = chunk_body<DT, VEC, fused_nr<DT>()>(F, SU.c, c.r, c.j);
  if (mode == MODE_DEFER) {
    if (c.j == 0 && threadIdx.x == 0) F.status[c.r] = LPS_ROW_DEFERRED | (1 << 8);
    return;
  }
  // handoff: every thread's stores have reached the L2 before the arrival is counted
  wait_stores();
  __syncthreads();
  if (threadIdx.x == 0) SU.c.mi[5] = l2_fetch_add(F.counters + (int64_t)c.r * 32, 1u) + 1u == (uint32_t)F.G ? 1 : 0;
  __syncthreads();
  if (!SU.c.mi[5]) return;
  const int reason = final_body<DT, VEC, fused_nr<DT>()>(F, SU.f, c.r, true);
  if (reason > 0 && threadIdx.x == 0) F.status[c.r] = LPS_ROW_DEFERRED | (reason << 8);
}

}  // namespace lps
