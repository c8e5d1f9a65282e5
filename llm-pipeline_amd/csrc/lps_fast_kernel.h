// The fast row-sampling kernel (layout, modes and protocol: lps_fast.h).
//
// Visibility of published data: a row's summaries, histograms and candidates
// live in per-row regions padded to whole 128-byte lines.  Each item is
// written once per launch and read only after its writer has waited for its
// stores and then passed the barrier or the handoff atomic.  A workgroup never
// reads a line before its final value is in the L2, so plain loads cannot hit
// a stale L1 line (the L1 is invalidated at every kernel start).  Counters are
// only touched with atomics, which execute at the L2.
//
// Cross-wave exchange slots of FShared (xa ... xh, xv, mi, m64, md) are each
// rewritten only after a barrier that follows every read of their previous
// value; the comments name the slot each step uses.
#pragma once

#include "lps_fast.h"

namespace lps {

// Block-wide penalised logit of one id (history scanned by all threads).
template <int DT>
__device__ float penalized_logit(const void* row, int id, const int32_t* h, int hlen, bool pen, float rep,
                                 float pres, float freq, FShared& S) {
  uint32_t c = 0;
  if (pen)
    for (int j = threadIdx.x; j < hlen; j += FT) c += h[j] == id ? 1u : 0u;
  __syncthreads();
  c = bcombine(wsum(c), S.xh, OpAdd{});
  __syncthreads();
  float x = load1<DT>(row, id);
  if (pen && c) x = penalize(x, (int)c, rep, pres, freq);
  return x;
}

// Rank sort of the kept list by (z desc, idx asc): kord[rank] = slot.
__device__ void rank_sort_kept(int K, FShared& S) {
  auto& k = S.u.f.x.k;
  for (int i = threadIdx.x; i < K; i += FT) {
    const uint32_t ki = k.kkey[i];
    const int ii = k.kidx[i];
    int rank = 0;
    for (int q = 0; q < K; q++) {
      const uint32_t kq = k.kkey[q];
      rank += (kq > ki || (kq == ki && k.kidx[q] < ii)) ? 1 : 0;
    }
    k.kord[rank] = i;
  }
  __syncthreads();
}

// Inclusive prefix of km over the sorted order into cum, K <= KEPTCAP (slot xb).
__device__ void sorted_prefix(int K, FShared& S) {
  auto& k = S.u.f.x.k;
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

__device__ __forceinline__ int floor_div(int a, int b) { return a >= 0 ? a / b : -((-a + b - 1) / b); }

// The fast path for the row / chunk of this workgroup.  Returns 0 when the
// workgroup is done, or a positive reason code when it must run the general
// algorithm on its row (the condition is workgroup-uniform).
template <int DT, int VEC>
__device__ __forceinline__ int fast_body(const FParams& F, FShared& S) {
  const KParams& P = F.k;
  const int G = F.G;
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  const int r = (slot / G) * 8 + xcd, j = slot % G;
  if (r >= P.R) return 0;
  LPS_STAMP(0);
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int V = P.V;
  const int lo = j * FCH;
  const int n = (V - lo) < FCH ? (V - lo) : FCH;
  constexpr int ES = DT == LPS_DTYPE_F32 ? 4 : 2;
  constexpr int NV = FE / VEC;
  const void* row = reinterpret_cast<const char*>(P.logits) +
                    ES * ((int64_t)(r / P.rows_inner) * P.stride_outer + (int64_t)(r % P.rows_inner) * P.stride_inner);
  ChunkSum1* s1 = F.sum1 + (int64_t)r * F.s_stride;
  ChunkSum2* s2 = F.sum2 + (int64_t)r * F.s_stride;
  float* hist = F.hist + (int64_t)r * F.h_stride;
  uint2* cands = F.cands + (int64_t)r * F.c_stride;
  uint32_t* ctr = F.counters + (int64_t)r * 32;

  // ---- history ids, then the chunk: both in flight together ----
  const int32_t* hrow = P.history ? P.history + (int64_t)r * P.history_stride : nullptr;
  HistPrefetch hp;
  prefetch_history(hrow, P.history_stride, hp);
  float x[FE];
  load_chunk<DT, VEC>(row, lo, n, x);

  const float T = P.temperature ? P.temperature[r] : P.temperature_def;
  const int topk = P.top_k ? P.top_k[r] : P.top_k_def;
  float topp = P.top_p ? P.top_p[r] : P.top_p_def;
  const float minp = P.min_p ? P.min_p[r] : P.min_p_def;
  const float typp = P.typical_p ? P.typical_p[r] : P.typical_p_def;
  const float rep = P.rep ? P.rep[r] : P.rep_def;
  const float pres = P.pres ? P.pres[r] : P.pres_def;
  const float freq = P.freq ? P.freq[r] : P.freq_def;
  if (topp != topp) topp = 1.0f;
  const bool greedy = !(T > 0.0f);
  const int ntop = (P.n_top > 0 && P.top_logprobs) ? P.n_top : 0;

  int mode;
  if (greedy) mode = MODE_GREEDY;
  else if (!(T >= 1e-4f)) mode = MODE_DEFER;
  else if (topk > 0) mode = topk <= FAST_KMAX ? MODE_TOPK : MODE_DEFER;
  else if (minp > 0.0f || typp < 1.0f || ntop > 0) mode = MODE_DEFER;
  else mode = topp < 1.0f ? MODE_NUCLEUS : MODE_PURE;
  if (P.entropy) mode = MODE_DEFER;
  if (mode == MODE_TOPK && typp < 1.0f && topk >= V) mode = MODE_DEFER;
  const int kprime = mode == MODE_TOPK ? (topk > ntop ? topk : ntop) : (mode == MODE_GREEDY ? ntop : 0);
  if (kprime > FAST_KMAX) mode = MODE_DEFER;
  if (mode == MODE_DEFER) return j == 0 ? 1 : 0;

  // ---- penalties from a per-chunk count table ----
  int hlen = (hrow && P.history_len) ? P.history_len[r] : 0;
  if (P.history_stride > 0 && hlen > P.history_stride) hlen = (int)P.history_stride;
  const bool pen = hlen > 0 && (rep != 1.0f || pres != 0.0f || freq != 0.0f);
  uint32_t cflags = 0;
  if (pen) {
    if (hlen > 65535) cflags |= CF_HISTORY;  // 16-bit counts: such rows take the general path
    build_counts(S.u.c.hc, hrow, hlen, hp, lo, n);
    apply_counts<VEC>(S.u.c.hc, n, rep, pres, freq, x);
  }
  LPS_STAMP(1);

  // ---- chunk max (NaN aside), NaN flag, greedy argmax, -inf count (slots xd xc xa xf) ----
  float tm = -INFINITY;
  uint32_t tnan = 0;
#pragma unroll
  for (int s = 0; s < FE; s++) {
    tm = fmaxf(tm, x[s]);
    tnan |= x[s] != x[s] ? 1u : 0u;
  }
  const float tm_thread = tm;
  uint64_t gbest = 0;
  if (greedy) {
#pragma unroll
    for (int s = 0; s < FE; s++) {
      const int l = slot_local<VEC>(s);
      if (l < n) {
        const uint64_t pk = ((uint64_t)f2key(x[s]) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)(lo + l));
        gbest = pk > gbest ? pk : gbest;
      }
    }
  }
  uint32_t ninf = 0;
  if (mode == MODE_PURE && P.kept_count) {
#pragma unroll
    for (int s = 0; s < FE; s++) ninf += (slot_local<VEC>(s) < n && x[s] == -INFINITY) ? 1u : 0u;
  }
  {
    const float wmx = wmax(tm);
    const uint32_t wnan = wreduce(tnan, OpOr{});
    const uint64_t wg = greedy ? wmax(gbest) : 0ull;
    const uint32_t wni = wsum(ninf);
    if (lane == 0) { S.xd[wv] = (double)wmx; S.xc[wv] = wnan; S.xa[wv] = wg; S.xf[wv] = wni; }
  }
  if (mode == MODE_NUCLEUS) S.u.c.hm[tid] = 0ull;  // HB == FT
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
    if (mode == MODE_NUCLEUS) {
#pragma unroll
      for (int s = 0; s < FE; s++) {
        const float w = __fmul_rn(x[s], c);
        const float e = exp2f(__fsub_rn(w, wm));
        acc += (double)e;
        if (e > 0.0f) {
          const int hb = btop - (int)floorf(__fmul_rn(w, (float)HS));
          if (hb < HB) atomicAdd(&S.u.c.hm[hb], (unsigned long long)mass_fixed(e));
        }
      }
    } else {
#pragma unroll
      for (int s = 0; s < FE; s++) acc += (double)exp2f(__fsub_rn(__fmul_rn(x[s], c), wm));
    }
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
    if (kprime <= 64) {
      const uint32_t v1[1] = {f2key(tm_thread)};
      th = wave_kth_largest<1>(v1, m);
    } else {
      float m1 = -INFINITY, m2 = -INFINITY;
#pragma unroll
      for (int s = 0; s < FE; s++) {
        const float xv = x[s];
        if (xv > m1) { m2 = m1; m1 = xv; }
        else if (xv > m2) m2 = xv;
      }
      const uint32_t v2[2] = {f2key(m1), f2key(m2)};
      th = wave_kth_largest<2>(v2, m);
    }
    if (lane == 0) S.xg[wv] = th;
  }
  __syncthreads();
  const float zsum = (float)(S.xe[0] + S.xe[1] + S.xe[2] + S.xe[3]);

  // ---- local candidates: every element >= the weakest wave threshold (slot xh) ----
  uint32_t ncand = 0;
  if (kprime > 0) {
    uint32_t th = min(min(S.xg[0], S.xg[1]), min(S.xg[2], S.xg[3]));
    if (!greedy && th > kNegInfKey + 1u && th != 0xFFFFFFFFu) th = f2key(collision_lo(key2f(th), T));
    const float xth = key2f(th);
    uint32_t cnt = 0;
#pragma unroll
    for (int s = 0; s < FE; s++) cnt += (slot_local<VEC>(s) < n && x[s] >= xth) ? 1u : 0u;
    uint32_t tot;
    uint32_t p = bscan_excl<uint32_t>(cnt, &tot, S.xh);
    uint2* out = cands + (int64_t)j * PUBCAP;
#pragma unroll
    for (int s = 0; s < FE; s++) {
      const int l = slot_local<VEC>(s);
      if (l < n && x[s] >= xth) {
        if (p < (uint32_t)PUBCAP) out[p] = make_uint2(f2key(x[s]), (uint32_t)(lo + l));
        p++;
      }
    }
    ncand = tot > (uint32_t)PUBCAP ? (uint32_t)PUBCAP : tot;
    if (tot > (uint32_t)PUBCAP) cflags |= CF_OVERFLOW;
  }
  LPS_STAMP(4);

  // ---- phase-1 summary ----
  if (tid == 0) {
    ChunkSum1 a;
    a.mkey = mkey; a.amax = amax; a.zsum = zsum; a.btop = btop; a.ninf = ninf; a.flags = cflags;
    a.pad[0] = a.pad[1] = 0;
    s1[j] = a;
  }

  // ---- nucleus: histograms, one intra-XCD barrier, the common cut region ----
  uint64_t above = 0;
  uint32_t nabove = 0;
  int blo = 0, bhi = -1;
  if (mode == MODE_NUCLEUS) {
    hist[(int64_t)j * HB + tid] = (float)((double)S.u.c.hm[tid] / (double)kMassScale);
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
    // wave 0: chunk reference -> row reference factors, the row mass Z
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
      const double Z = wsum((double)a.zsum * sc);
      if (lane < G) { S.u.c.scale[lane] = sc; S.u.c.btop[lane] = a.btop; }
      if (lane == 0) { S.md[0] = Z; S.mi[10] = rfin ? (int)floorf(__fmul_rn(wg, (float)HS)) : 0; S.mi[11] = rfin ? 1 : 0; }
    }
    __syncthreads();
    const bool rfin = S.mi[11] != 0;
    const int btg = S.mi[10];
    const double Z = S.md[0];
    const double Pm = (double)topp * Z;
    // merged mass of absolute bin btg - tid (slot xd)
    double m = 0.0;
    if (rfin) {
#pragma unroll 8
      for (int q = 0; q < G; q++) {
        const int idx = tid - (btg - S.u.c.btop[q]);
        const double sc = S.u.c.scale[q];
        if (sc > 0.0 && idx >= 0 && idx < HB) m += (double)hist[(int64_t)q * HB + idx] * sc;
      }
    }
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
      // this chunk: mass and count above the region, candidates inside (slots xa xb xc)
      const int hbt = btop - (bhi + 1);  // chunk histogram bins 0..hbt lie above the region
      uint64_t am = (xm_finite && tid <= hbt) ? (uint64_t)S.u.c.hm[tid] : 0ull;
      uint32_t na = 0, nc = 0, inreg = 0;
#pragma unroll
      for (int s = 0; s < FE; s++) {
        if (x[s] != -INFINITY) {
          const int b = wbin(x[s], c);
          na += b > bhi ? 1u : 0u;
          const bool in = b >= blo && b <= bhi;
          nc += in ? 1u : 0u;
          inreg |= in ? (1u << s) : 0u;
        }
      }
      am = wsum(am);
      na = wsum(na);
      if (lane == 0) { S.xa[wv] = am; S.xb[wv] = na; }
      uint32_t ctot;
      uint32_t p = bscan_excl<uint32_t>(nc, &ctot, S.xc);
      above = S.xa[0] + S.xa[1] + S.xa[2] + S.xa[3];
      nabove = (uint32_t)(S.xb[0] + S.xb[1] + S.xb[2] + S.xb[3]);
      uint2* out = cands + (int64_t)j * PUBCAP;
#pragma unroll
      for (int s = 0; s < FE; s++) {
        if ((inreg >> s) & 1u) {
          if (p < (uint32_t)PUBCAP) out[p] = make_uint2(f2key(x[s]), (uint32_t)(lo + slot_local<VEC>(s)));
          p++;
        }
      }
      ncand = ctot > (uint32_t)PUBCAP ? (uint32_t)PUBCAP : ctot;
      if (ctot > (uint32_t)PUBCAP) cflags |= CF_OVERFLOW;
    }
    LPS_STAMP(20);
  }

  // ---- handoff: the last chunk workgroup of the row finalises it ----
  LPS_STAMP(6);
  wait_stores();
  __syncthreads();
  if (tid == 0) {
    ChunkSum2 a;
    a.ncand = ncand; a.flags = cflags; a.above = above; a.nabove = nabove;
    a.pad[0] = a.pad[1] = a.pad[2] = 0;
    s2[j] = a;
    wait_stores();
    // handoff word: arrivals in bits 0-7, arrivals per XCD in 7-bit fields from bit 8
    const uint64_t add = 1ull + (1ull << (8 + 7 * (xcc_id() & 7u)));
    const uint64_t now = l2_fetch_add64(reinterpret_cast<uint64_t*>(ctr), add) + add;
    int xcds = 0;
    for (int q = 0; q < 8; q++) xcds += ((now >> (8 + 7 * q)) & 0x7Full) ? 1 : 0;
    S.mi[5] = (now & 0xFFull) == (uint64_t)G ? 1 : 0;
    S.mi[6] = xcds;  // more than one XCD: the L2-local exchange cannot be trusted
  }
  __syncthreads();
  LPS_STAMP(7);
  if (!S.mi[5]) return 0;

  // =========================== finaliser ===========================
  // F1: wave 0 gathers the per-chunk summaries.
  const bool split = S.mi[6] > 1;
  if (wv == 0) {
    ChunkSum1 a{};
    ChunkSum2 b{};
    if (lane < G) { a = s1[lane]; b = s2[lane]; }
    const uint32_t fl = wreduce(lane < G ? (a.flags | b.flags) : 0u, OpOr{});
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
    const double sc = (rfin && qfin) ? exp2((double)__fmul_rn(xq, c) - wgd) : 0.0;
    const double Zfull = wsum((double)a.zsum * sc);
    const double abv = (double)b.above / (double)kMassScale * sc;
    const double A = wsum(abv);
    if (lane < G) {
      S.u.f.pre[lane] = ncinc - nc;
      S.u.f.scale[lane] = sc;
      S.u.f.abvm[lane] = abv;
      S.u.f.keptm[lane] = (double)a.zsum * sc;
    }
    if (lane == 0) {
      S.u.f.pre[G] = NC;
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
  if (tid == 0) {
    // counters back to zero for the next launch (stream-ordered)
    atomicExch(reinterpret_cast<unsigned long long*>(ctr), 0ull);
    atomicExch(ctr + 2, 0u);
  }
  __syncthreads();
  const uint32_t fl = (uint32_t)S.mi[12] | (split ? (uint32_t)CF_SPLIT : 0u);
  if (fl & (CF_OVERFLOW | CF_HISTORY | CF_SPLIT | CF_REGION)) return (int)fl;
  const int NC = S.mi[13];
  const uint32_t ninf_all = (uint32_t)S.mi[14];
  const uint32_t nab_all = (uint32_t)S.mi[15];
  const uint32_t gkey = (uint32_t)S.mi[16];
  const int gam = S.mi[17];
  const double Zfull = S.md[1];
  const double Aabove = S.md[2];
  LPS_STAMP(8);

  const float xmax = key2f(gkey);
  const bool has_nan = gkey == 0xFFFFFFFFu;
  const float zmax = greedy ? xmax : __fdiv_rn(xmax, T);
  int status = 0;
  if (!greedy) {
    if (has_nan || xmax == INFINITY || zmax == INFINITY) status |= LPS_ROW_NONFINITE;
    else if (xmax == -INFINITY) status |= LPS_ROW_EMPTY;
  }
  const double lnZ = Zfull > 0.0 ? log(Zfull) : 0.0;
  const int64_t qtok = (P.query_tokens && (r % P.rows_inner) < P.query_inner)
                           ? P.query_tokens[(int64_t)(r / P.rows_inner) * P.query_inner + (r % P.rows_inner)]
                           : -1;
  float u = P.uniforms ? P.uniforms[r] : 0.5f;
  if (!(u >= 0.0f)) u = 0.0f;
  if (u >= 1.0f) u = 0.99999994f;

  int64_t token = -1;
  float cut = -INFINITY, qprob = 0.0f, chosen_z = NAN;
  int32_t ties = -1, kept_n = 0;
  int ntop_out = 0;  // entries of the sorted kept list that are top logprobs

  // Candidates in registers: thread t holds concatenated positions [t*FCPT, t*FCPT + np).
  uint32_t ck[FCPT], cx[FCPT];
  int32_t ci[FCPT];
  int np = 0;
  auto load_cands = [&]() {
    const int i0 = tid * FCPT;
    np = NC - i0;
    np = np < 0 ? 0 : (np > FCPT ? FCPT : np);
    int q = 0;
    if (np > 0) {
      int a = 0, b = G - 1;  // last chunk with pre <= i0
      while (a < b) {
        const int mid = (a + b + 1) >> 1;
        if ((int)S.u.f.pre[mid] <= i0) a = mid; else b = mid - 1;
      }
      q = a;
    }
    int nb = np > 0 ? (int)S.u.f.pre[q + 1] : 0;
#pragma unroll
    for (int e = 0; e < FCPT; e++) {
      cx[e] = 0u;
      ci[e] = -1;
      if (e < np) {
        while (i0 + e >= nb) { q++; nb = (int)S.u.f.pre[q + 1]; }
        const uint2 cv = cands[(int64_t)q * PUBCAP + (i0 + e - (int)S.u.f.pre[q])];
        cx[e] = cv.x;
        ci[e] = (int32_t)cv.y;
      }
    }
  };

  if (status == 0 && kprime > 0) {
    // ---------------- top-k (and top-N logprobs) ----------------
    if (NC > FCAP) return 512;
    load_cands();
#pragma unroll
    for (int e = 0; e < FCPT; e++) {
      const float xv = key2f(cx[e]);
      ck[e] = e < np ? f2key(greedy ? xv : __fdiv_rn(xv, T)) : 0u;
    }
    const int keff = mode == MODE_TOPK ? (topk < V ? topk : V) : 0;
    int kc = keff > ntop ? keff : ntop;
    if (kc > NC) kc = NC;
    if (kc <= 0) return 16;
    const uint32_t zc = sel_count(ck, np, (uint32_t)kc, S);
    // collect z >= zc into the kept list (slot xh)
    uint32_t cnt = 0;
#pragma unroll
    for (int e = 0; e < FCPT; e++) cnt += (e < np && ck[e] >= zc) ? 1u : 0u;
    uint32_t Kall;
    uint32_t p = bscan_excl<uint32_t>(cnt, &Kall, S.xh);
    if (Kall > (uint32_t)KEPTCAP) return 32;
    auto& kl = S.u.f.x.k;
#pragma unroll
    for (int e = 0; e < FCPT; e++) {
      if (e < np && ck[e] >= zc) {
        kl.kkey[p] = ck[e];
        kl.kx[p] = cx[e];
        kl.kidx[p] = ci[e];
        kl.km[p] = mass_fixed(mass_f(key2f(ck[e]), zmax));
        p++;
      }
    }
    __syncthreads();
    const int K = (int)Kall;
    rank_sort_kept(K, S);
    ntop_out = ntop < K ? ntop : K;
    LPS_STAMP(16);
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
      const uint32_t kth = kl.kkey[kl.kord[keff - 1]];
      if (tid == 0) S.mi[20] = K;
      __syncthreads();
      for (int pz = tid; pz < K; pz += FT)
        if (kl.kkey[kl.kord[pz]] >= kth && (pz == K - 1 || kl.kkey[kl.kord[pz + 1]] < kth)) S.mi[20] = pz + 1;
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
          const bool ok = mass_f(key2f(kl.kkey[kl.kord[pz]]), zmax) >= minp;
          const bool okp = pz == 0 || mass_f(key2f(kl.kkey[kl.kord[pz - 1]]), zmax) >= minp;
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
        const uint32_t ckey = kl.kkey[kl.kord[nf - 1]];
        cut = key2f(ckey);
        if (P.kept_ties || P.kept_count) {  // (slots xc xf xg)
          uint32_t ea = 0, ek = 0, nfin = 0;
          for (int q = tid; q < K; q += FT) {
            const uint32_t kq = kl.kkey[kl.kord[q]];
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
        // vocabulary order over the kept prefix
        for (int pz = tid; pz < nf; pz += FT) {
          const int si = kl.kord[pz];
          const int ii = kl.kidx[si];
          int rk = 0;
          for (int q = 0; q < nf; q++) rk += kl.kidx[kl.kord[q]] < ii ? 1 : 0;
          kl.iord[rk] = si;
        }
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
        chosen_z = key2f(kl.kkey[ps]);
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
#pragma unroll
      for (int e = 0; e < FCPT; e++) ck[e] = e < np ? f2key(__fdiv_rn(key2f(cx[e]), T)) : 0u;
      auto cmass = [&](int e) -> uint64_t { return mass_fixed(mass_f(key2f(ck[e]), zmax)); };
      const uint64_t Af = (uint64_t)(Aabove * (double)kMassScale);
      const uint64_t Pf = (uint64_t)((double)topp * Zfull * (double)kMassScale);
      LPS_STAMP(16);
      const MassSel ms = sel_mass(ck, np, zmax, Af, Pf, S);
      LPS_STAMP(17);
      if (!ms.ok || ms.ceq == 0) return 64;
      vkey = ms.key;
      const uint64_t e1 = ms.meq / ms.ceq;
      const uint64_t nt = e1 ? (Pf - ms.above) / e1 + 1 : (uint64_t)ms.ceq;
      n_tie = nt >= ms.ceq ? kNoTie : (uint32_t)nt;
      // ties at the cut: the kept ones are the n_tie lowest indices (slot xh)
      auto& kl = S.u.f.x.k;
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
          if (e < np && ck[e] == vkey) kl.kidx[p++] = ci[e];
        __syncthreads();
        for (int i = tid; i < (int)ttot; i += FT) {
          const int ii = kl.kidx[i];
          int rk = 0;
          for (int q = 0; q < (int)ttot; q++) rk += kl.kidx[q] < ii ? 1 : 0;
          if (rk == (int)n_tie - 1) S.mi[25] = ii;
        }
      }
      // any x of the cut's collision group
#pragma unroll
      for (int e = 0; e < FCPT; e++)
        if (e < np && ck[e] == vkey) S.mi[26] = (int)cx[e];
      __syncthreads();
      tie_lim = S.mi[25];
      LPS_STAMP(18);
      if (tid == 0) {
        // the cut's whole division-collision group must lie inside the region
        const float xv = key2f((uint32_t)S.mi[26]);
        const float xl = collision_lo(xv, T);
        float xh = xv;
        for (int it = 0; it < 64; it++) {
          const uint32_t k = f2key(xh);
          if (k >= 0xFFFFFFFEu) break;
          const float y = key2f(k + 1u);
          if (__fdiv_rn(y, T) != key2f(vkey)) break;
          xh = y;
        }
        const int bl = wbin(xl, c), bh = wbin(xh, c);
        S.mi[27] = (bl >= blo && bh <= bhi) ? 1 : 0;
      }
      // kept candidate mass and count; prefix at chunk boundaries (slots xa xg)
      uint64_t lm = 0;
      uint32_t lc = 0;
#pragma unroll
      for (int e = 0; e < FCPT; e++) {
        const bool kept = e < np && (ck[e] > vkey || (ck[e] == vkey && ci[e] <= tie_lim));
        const uint64_t m = kept ? cmass(e) : 0ull;
        lm += m;
        lc += kept ? 1u : 0u;
        if (kept && (int64_t)ci[e] == qtok) S.md[6] = (double)m / (double)kMassScale;
      }
      {
        const uint32_t wl = wsum(lc);
        if (lane == 0) S.xg[wv] = wl;
      }
      uint64_t mtot;
      uint64_t run = bscan_excl<uint64_t>(lm, &mtot, S.xa);
      const int i0 = tid * FCPT;
#pragma unroll
      for (int e = 0; e < FCPT; e++) {
        if (e < np) {
          const int q = ci[e] / FCH;
          if (i0 + e == (int)S.u.f.pre[q]) S.u.f.epre[q] = run;
          const bool kept = ck[e] > vkey || (ck[e] == vkey && ci[e] <= tie_lim);
          run += kept ? cmass(e) : 0ull;
          if (i0 + e == (int)S.u.f.pre[q + 1] - 1) S.u.f.eend[q] = run;
        }
      }
      __syncthreads();
      if (!S.mi[27]) return 128;
      kept_n = (int32_t)(nab_all + S.xg[0] + S.xg[1] + S.xg[2] + S.xg[3]);
      qmass = S.md[6];
      if (wv == 0 && lane < G) {
        const uint32_t ncq = S.u.f.pre[lane + 1] - S.u.f.pre[lane];
        const double cmq = ncq ? (double)(S.u.f.eend[lane] - S.u.f.epre[lane]) / (double)kMassScale : 0.0;
        S.u.f.keptm[lane] = S.u.f.abvm[lane] + cmq;
      }
      __syncthreads();
      ties = n_tie == kNoTie ? -1 : (int32_t)n_tie;
      cut = key2f(vkey);
    }
    LPS_STAMP(9);
    // the chunk holding u * Zf (wave 0), then its exact scan in vocabulary order
    if (wv == 0) {
      const double km = lane < G ? S.u.f.keptm[lane] : 0.0;
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
      const int lo2 = js * FCH;
      const int n2 = (V - lo2) < FCH ? (V - lo2) : FCH;
      HistPrefetch hp2;
      prefetch_history(hrow, P.history_stride, hp2);
      float y[FE];
      load_chunk<DT, VEC>(row, lo2, n2, y);
      if (pen) {
        build_counts(S.u.f.x.hc, hrow, hlen, hp2, lo2, n2);
        apply_counts<VEC>(S.u.f.x.hc, n2, rep, pres, freq, y);
      }
      LPS_STAMP(21);
      auto kept_of = [&](float yv, float z) -> bool {
        if (z == -INFINITY || yv != yv) return false;
        if (mode == MODE_PURE) return true;
        const int b = wbin(yv, c);
        if (b > bhi) return true;
        if (b < blo) return false;
        const uint32_t kz = f2key(z);
        return kz > vkey;  // ties at the cut handled by index below
      };
      auto kept_m = [&](int v, int e) -> double {  // kept mass of slot (v, e), 0 if not kept
        const float yv = y[v * VEC + e];
        const float z = __fdiv_rn(yv, T);
        const int gi = lo2 + (v * FT + tid) * VEC + e;
        const bool kept = kept_of(yv, z) ||
                          (mode == MODE_NUCLEUS && z != -INFINITY && f2key(z) == vkey && gi <= tie_lim &&
                           wbin(yv, c) >= blo && wbin(yv, c) <= bhi);
        return kept ? (double)mass_f(z, zmax) : 0.0;
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
          for (int e = 0; e < VEC; e++) a += kept_m(vb + b, e);
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
              lz = __fdiv_rn(y[vv * VEC + e], T);
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
      const float xq = penalized_logit<DT>(row, (int)qtok, hrow, hlen, pen, rep, pres, freq, S);
      const float zq = __fdiv_rn(xq, T);
      if (mode == MODE_PURE) {
        qprob = zq != -INFINITY ? (float)((double)mass_f(zq, zmax) / Zf) : 0.0f;
      } else {
        const int bq = wbin(xq, c);
        if (bq > bhi && zq != -INFINITY) qprob = (float)((double)mass_f(zq, zmax) / Zf);
        else if (qmass >= 0.0) qprob = (float)(qmass / Zf);
      }
    }
  }
  if (P.skip_draw && !greedy) token = -1;
  LPS_STAMP(10);

  // ---- outputs ----
  if (P.chosen_logprob && tid == 0) {
    float lp = NAN;
    if (token >= 0 && Zfull > 0.0 && chosen_z == chosen_z)
      lp = (float)((double)__fsub_rn(chosen_z, zmax) - lnZ);
    P.chosen_logprob[r] = lp;
  }
  if (ntop > 0 && status == 0) {
    auto& kl = S.u.f.x.k;
    for (int q = tid; q < P.n_top; q += FT) {
      if (q < ntop_out) {
        const int si = kl.kord[q];
        P.top_logprobs[(int64_t)r * P.n_top + q] = (float)((double)__fsub_rn(key2f(kl.kkey[si]), zmax) - lnZ);
        if (P.top_ids) P.top_ids[(int64_t)r * P.n_top + q] = kl.kidx[si];
      } else {
        P.top_logprobs[(int64_t)r * P.n_top + q] = -INFINITY;
        if (P.top_ids) P.top_ids[(int64_t)r * P.n_top + q] = -1;
      }
    }
  }
  if (tid == 0) {
    P.tokens[r] = status ? -1 : token;
    F.status[r] = status;
    if (P.row_status) P.row_status[r] = status;
    if (P.query_prob) P.query_prob[r] = qprob;
    if (P.kept_cut) P.kept_cut[r] = cut;
    if (P.kept_ties) P.kept_ties[r] = ties;
    if (P.kept_count) P.kept_count[r] = kept_n;
    if (P.row_path) P.row_path[r] = 0;
  }
  LPS_STAMP(11);
  return 0;
}

template <int DT, int VEC>
__global__ __launch_bounds__(FT) __attribute__((amdgpu_waves_per_eu(3, 8))) void fast_kernel(FParams F) {
  // the fast path's LDS, or the general path's when a row falls back to it
  __shared__ union {
    FShared f;
    GenShared g;
  } SU;
  const int reason = fast_body<DT, VEC>(F, SU.f);
  if (reason > 0) {
    // a row the fast path cannot finish exactly: this whole workgroup runs the
    // general algorithm on it (no fast-path value is live here)
    const int slot = blockIdx.x >> 3;
    const int r = (slot / F.G) * 8 + (blockIdx.x & 7);
    if (threadIdx.x == 0) F.status[r] = LPS_ROW_DEFERRED | (reason << 8);
    __syncthreads();
    // a copy local to this branch: the general path's uses of its parameters
    // then cost nothing on the fast path (no private copy of the kernel arguments)
    KParams Pk = F.k;
    Pk.plans = nullptr;        // plans serve speculative verification, which uses the general kernel
    Pk.only_status = nullptr;  // the general kernel's own launch filter
    gen_row<DT, 1>(Pk, r, SU.g);  // element loads: the lean variant of the general path
    LPS_STAMP(12);
  }
}

}  // namespace lps
