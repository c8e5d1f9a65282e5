// The fast row-sampling kernel (layout, modes and protocol: lps_fast.h).
//
// Visibility of published data: a row's summaries, histograms and candidates
// live in per-row regions padded to whole 128-byte lines.  Each item is
// written once per launch and read only after its writer has waited for its
// stores and then passed the barrier or the handoff atomic.  A workgroup never
// reads a line before its final value is in the L2, so plain loads cannot hit
// a stale L1 line (the L1 is invalidated at every kernel start).  Counters are
// only touched with atomics, which execute at the L2.
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
  c = fsum_u32(c, S);
  float x = load1<DT>(row, id);
  if (pen && c) x = penalize(x, (int)c, rep, pres, freq);
  return x;
}

// Rank sort of the kept list by (z desc, idx asc): kord[rank] = slot.
__device__ void rank_sort_kept(int K, FShared& S) {
  for (int i = threadIdx.x; i < K; i += FT) {
    const uint32_t ki = S.u.f.kkey[i];
    const int ii = S.u.f.kidx[i];
    int rank = 0;
    for (int q = 0; q < K; q++) {
      const uint32_t kq = S.u.f.kkey[q];
      rank += (kq > ki || (kq == ki && S.u.f.kidx[q] < ii)) ? 1 : 0;
    }
    S.u.f.kord[rank] = i;
  }
  __syncthreads();
}

// Inclusive prefix of km over the sorted order into cum (base added), K <= KEPTCAP.
__device__ void sorted_prefix(int K, uint64_t base, FShared& S) {
  constexpr int PER = KEPTCAP / FT;
  uint64_t loc[PER];
  uint64_t t = 0;
#pragma unroll
  for (int q = 0; q < PER; q++) {
    const int pz = threadIdx.x * PER + q;
    loc[q] = pz < K ? S.u.f.km[S.u.f.kord[pz]] : 0;
    t += loc[q];
  }
  uint64_t tot;
  uint64_t a = base + fexcl_scan<uint64_t>(t, &tot, S.r64);
#pragma unroll
  for (int q = 0; q < PER; q++) {
    const int pz = threadIdx.x * PER + q;
    a += loc[q];
    if (pz < K) S.u.f.cum[pz] = a;
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
  const int tid = threadIdx.x;
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
  if (mode == MODE_DEFER) {
    if (j != 0) return 0;
    return 1;
  }

  // ---- per-chunk history table ----
  int hlen = (P.history && P.history_len) ? P.history_len[r] : 0;
  if (P.history_stride > 0 && hlen > P.history_stride) hlen = (int)P.history_stride;
  const bool pen = hlen > 0 && (rep != 1.0f || pres != 0.0f || freq != 0.0f);
  const int32_t* hrow = pen ? P.history + (int64_t)r * P.history_stride : nullptr;
  uint32_t cflags = 0;
  if (pen && !build_pen(S, hrow, hlen, lo, n)) cflags |= CF_HISTORY;
  const FPen fp{pen, rep, pres, freq, lo, &S};

  // ---- the chunk, in registers ----
  float x[FE];
  load_chunk<DT, VEC>(row, lo, n, fp, x);

  // ---- chunk max (first index) and -inf count ----
  uint64_t best = 0;
  uint32_t ninf = 0;
#pragma unroll
  for (int s = 0; s < FE; s++) {
    const int l = slot_local<VEC>(s);
    if (l < n) {
      const uint64_t pk = ((uint64_t)f2key(x[s]) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)(lo + l));
      best = pk > best ? pk : best;
      ninf += x[s] == -INFINITY ? 1u : 0u;
    }
  }
  best = fmax_u64(best, S);
  ninf = fsum_u32(ninf, S);
  const uint32_t mkey = (uint32_t)(best >> 32);
  const int amax = (int)(0xFFFFFFFFu - (uint32_t)best);
  const float xm = key2f(mkey);
  const bool xm_finite = mkey != 0xFFFFFFFFu && xm != INFINITY && xm != -INFINITY;
  const float Te = greedy ? 1.0f : T;
  const float c = __fdiv_rn(kLog2e, Te);

  // ---- chunk mass and the nucleus histogram ----
  const bool need_sum = mode == MODE_PURE || mode == MODE_NUCLEUS || P.chosen_logprob || ntop > 0;
  float zsum = 0.0f;
  int btop = 0;
  if (mode == MODE_NUCLEUS) {
    for (int i = tid; i < HB; i += FT) S.u.c.hm[i] = 0;
    __syncthreads();
  }
  if (need_sum && xm_finite) {
    const float wm = __fmul_rn(xm, c);
    btop = (int)floorf(__fmul_rn(wm, (float)HS));
    double acc = 0.0;
#pragma unroll
    for (int s = 0; s < FE; s++) {
      const int l = slot_local<VEC>(s);
      if (l < n) {
        const float w = __fmul_rn(x[s], c);
        const float e = exp2f(__fsub_rn(w, wm));
        acc += (double)e;
        if (mode == MODE_NUCLEUS && e > 0.0f) {
          const int hb = btop - (int)floorf(__fmul_rn(w, (float)HS));
          if (hb < HB) atomicAdd((unsigned long long*)&S.u.c.hm[hb], (unsigned long long)mass_fixed(e));
        }
      }
    }
    zsum = (float)fsum_f64(acc, S);
  }

  // ---- local top-k' candidates: exact local k'-th value with a division-collision margin ----
  uint32_t ncand = 0;
  if (kprime > 0) {
    uint32_t tk = 0;
#pragma unroll
    for (int s = 0; s < FE; s++)
      if (slot_local<VEC>(s) < n) { const uint32_t k = f2key(x[s]); tk = k > tk ? k : tk; }
    S.u.c.tmax[tid] = tk;
    if (tid == 0) { S.mi[2] = 0; S.mi[3] = 0; }
    __syncthreads();
    // lower bound: the k'-th largest per-thread maximum (at least k' elements reach it)
    uint32_t th0 = 0;
    if (n > LCAP) th0 = block_select_kth(FT, (uint32_t)kprime, [&](int i) { return S.u.c.tmax[i]; }, S);
    if (!greedy && th0 > kNegInfKey + 1u && th0 != 0xFFFFFFFFu) th0 = f2key(collision_lo(key2f(th0), T));
#pragma unroll
    for (int s = 0; s < FE; s++) {
      const int l = slot_local<VEC>(s);
      if (l < n) {
        const uint32_t k = f2key(x[s]);
        if (k >= th0) {
          const int q = atomicAdd(&S.mi[2], 1);
          if (q < LCAP) { S.u.c.v.l.lkey[q] = k; S.u.c.v.l.lidx[q] = lo + l; }
        }
      }
    }
    __syncthreads();
    const int cnt = S.mi[2];
    const int nl = cnt < LCAP ? cnt : LCAP;
    if (cnt > LCAP) cflags |= CF_OVERFLOW;
    uint32_t thk = 0;
    if (nl > kprime) thk = block_select_kth(nl, (uint32_t)kprime, [&](int i) { return S.u.c.v.l.lkey[i]; }, S);
    if (!greedy && thk > kNegInfKey + 1u && thk != 0xFFFFFFFFu) thk = f2key(collision_lo(key2f(thk), T));
    uint2* out = cands + (int64_t)j * PUBCAP;
    for (int i = tid; i < nl; i += FT) {
      if (S.u.c.v.l.lkey[i] >= thk) {
        const int q = atomicAdd(&S.mi[3], 1);
        if (q < PUBCAP) out[q] = make_uint2(S.u.c.v.l.lkey[i], (uint32_t)S.u.c.v.l.lidx[i]);
      }
    }
    __syncthreads();
    ncand = (uint32_t)S.mi[3];
    if (ncand > PUBCAP) { cflags |= CF_OVERFLOW; ncand = PUBCAP; }
  }

  // ---- phase-1 summary ----
  if (tid == 0) {
    ChunkSum1 a;
    a.mkey = mkey; a.amax = amax; a.zsum = zsum; a.btop = btop; a.ninf = ninf; a.flags = cflags;
    a.xcc = xcc_id(); a.pad = 0;
    s1[j] = a;
  }

  // ---- nucleus: histograms, one intra-XCD barrier, the common cut region ----
  uint64_t above = 0;
  uint32_t nabove = 0;
  int blo = 0, bhi = -1;
  if (mode == MODE_NUCLEUS) {
    // fine masses (chunk reference) and sums over absolute units
    float* hj = hist + (int64_t)j * (HB + HU + 2);
    for (int i = tid; i < HB; i += FT) hj[i] = (float)((double)S.u.c.hm[i] / (double)kMassScale);
    const int ut = floor_div(btop, HS);
    if (tid < HU + 2) {
      double u = 0.0;
      for (int b = 0; b < HS; b++) {
        const int hb = btop - ((ut - tid) * HS + b);
        if (hb >= 0 && hb < HB) u += (double)S.u.c.hm[hb] / (double)kMassScale;
      }
      hj[HB + tid] = (float)u;
    }
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
    auto& N = S.u.c.v.n;
    if (tid < G) {
      const ChunkSum1 q = s1[tid];
      const float xq = key2f(q.mkey);
      S.u.c.tmax[tid] = q.mkey;
      N.btop[tid] = q.btop;
      N.zs[tid] = (double)q.zsum;
      N.scale[tid] = (q.mkey != 0xFFFFFFFFu && xq != -INFINITY && xq != INFINITY) ? (double)__fmul_rn(xq, c) : -1e300;
    }
    __syncthreads();
    uint32_t gk = 0;
    for (int q = 0; q < G; q++) gk = S.u.c.tmax[q] > gk ? S.u.c.tmax[q] : gk;
    const double wg = (double)__fmul_rn(key2f(gk), c);
    const int btg = (int)floorf(__fmul_rn(__fmul_rn(key2f(gk), c), (float)HS));
    const int utg = floor_div(btg, HS);
    __syncthreads();
    if (tid < G) N.scale[tid] = N.scale[tid] > -1e299 ? exp2(N.scale[tid] - wg) : 0.0;
    __syncthreads();
    double Z = 0.0;
    for (int q = 0; q < G; q++) Z += N.zs[q] * N.scale[q];
    const double Pm = (double)topp * Z;
    // global mass of absolute unit utg - t
    if (tid < HU + 2) {
      const int U = utg - tid;
      double m = 0.0;
      for (int q = 0; q < G; q++) {
        if (N.scale[q] == 0.0) continue;
        const int t = floor_div(N.btop[q], HS) - U;
        if (t >= 0 && t < HU + 2) m += (double)hist[(int64_t)q * (HB + HU + 2) + HB + t] * N.scale[q];
      }
      N.um[tid] = m;
    }
    __syncthreads();
    if (tid == 0) {
      double cum = 0.0;
      int uc = -1;
      for (int q = 0; q < HU + 2; q++) {
        if (cum + N.um[q] > Pm) { uc = q; break; }
        cum += N.um[q];
      }
      S.mi[6] = uc;
      S.md[1] = cum;
    }
    __syncthreads();
    const int uc = S.mi[6];
    if (uc >= 0 && tid < HS) {
      // fine bins of the crossing unit, top first
      const int b = (utg - uc) * HS + (HS - 1 - tid);
      double m = 0.0;
      for (int q = 0; q < G; q++) {
        if (N.scale[q] == 0.0) continue;
        const int hb = N.btop[q] - b;
        if (hb >= 0 && hb < HB) m += (double)hist[(int64_t)q * (HB + HU + 2) + hb] * N.scale[q];
      }
      N.bm[tid] = m;
    }
    __syncthreads();
    if (tid == 0) {
      int lb = 0, hb = -1;
      if (uc >= 0) {
        // bins whose cumulative interval meets [Pm - eps Z, Pm + eps Z], plus one bin either side
        const double eps = 1e-5 * Z;
        double cc = S.md[1];
        int first = -1, last = -1;
        for (int t = 0; t < HS; t++) {
          if (cc + N.bm[t] >= Pm - eps && cc <= Pm + eps) { if (first < 0) first = t; last = t; }
          cc += N.bm[t];
        }
        if (first < 0) { first = 0; last = HS - 1; }
        hb = (utg - uc) * HS + (HS - 1 - first) + 1;
        lb = (utg - uc) * HS + (HS - 1 - last) - 1;
      }
      S.mi[7] = lb;
      S.mi[8] = hb;
    }
    __syncthreads();
    blo = S.mi[7];
    bhi = S.mi[8];
    // this chunk: mass above the region (fixed point, chunk reference), count above, candidates inside
    const int hbt = btop - (bhi + 1);
    uint64_t am = 0;
    for (int i = tid; i < HB; i += FT)
      if (i <= hbt) am += S.u.c.hm[i];
    above = fsum_u64(am, S);
    if (tid == 0) S.mi[3] = 0;
    __syncthreads();
    uint32_t na = 0;
    uint2* out = cands + (int64_t)j * PUBCAP;
#pragma unroll
    for (int s = 0; s < FE; s++) {
      const int l = slot_local<VEC>(s);
      if (l < n && x[s] != -INFINITY) {
        const int b = (int)floorf(__fmul_rn(__fmul_rn(x[s], c), (float)HS));
        if (b > bhi) na++;
        else if (b >= blo) {
          const int q = atomicAdd(&S.mi[3], 1);
          if (q < PUBCAP) out[q] = make_uint2(f2key(x[s]), (uint32_t)(lo + l));
        }
      }
    }
    nabove = fsum_u32(na, S);
    ncand = (uint32_t)S.mi[3];
    if (ncand > PUBCAP) { cflags |= CF_OVERFLOW; ncand = PUBCAP; }
    if (S.mi[9] == 1 || uc < 0) cflags |= CF_REGION;
  }

  // ---- handoff: the last chunk workgroup of the row finalises it ----
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
  if (!S.mi[5]) return 0;

  // =========================== finaliser ===========================
  const bool split = S.mi[6] > 1;
  if (tid < G) {
    const ChunkSum1 a = s1[tid];
    const ChunkSum2 b = s2[tid];
    S.u.f.cmk[tid] = a.mkey;
    S.u.f.cam[tid] = a.amax;
    S.u.f.czs[tid] = a.zsum;
    S.u.f.cninf[tid] = a.ninf;
    S.u.f.cfl[tid] = a.flags | b.flags | (split ? (uint32_t)CF_SPLIT : 0u);
    S.u.f.cnc[tid] = b.ncand;
    S.u.f.abv[tid] = (double)b.above / (double)kMassScale;
    S.u.f.nab[tid] = b.nabove;
  }
  if (tid == 0) {
    // counters back to zero for the next launch (stream-ordered)
    atomicExch(reinterpret_cast<unsigned long long*>(ctr), 0ull);
    atomicExch(ctr + 2, 0u);
    uint32_t a = 0;
    for (int q = 0; q < G; q++) { S.u.f.pre[q] = a; a += S.u.f.cnc[q]; }
    S.mi[10] = (int)a;
  }
  __syncthreads();
  uint32_t gkey = 0, fl = 0, ninf_all = 0;
  int gam = 0x7FFFFFFF;
  for (int q = 0; q < G; q++) {
    const uint32_t k = S.u.f.cmk[q];
    if (k > gkey || (k == gkey && S.u.f.cam[q] < gam)) { gkey = k; gam = S.u.f.cam[q]; }
    fl |= S.u.f.cfl[q];
    ninf_all += S.u.f.cninf[q];
  }
  const int NC = S.mi[10];
  if (fl & (CF_OVERFLOW | CF_HISTORY | CF_SPLIT | CF_REGION)) {
    return ((int32_t)fl);
  }
  const float xmax = key2f(gkey);
  const bool has_nan = gkey == 0xFFFFFFFFu;
  const float zmax = greedy ? xmax : __fdiv_rn(xmax, T);
  int status = 0;
  if (!greedy) {
    if (has_nan || xmax == INFINITY || zmax == INFINITY) status |= LPS_ROW_NONFINITE;
    else if (xmax == -INFINITY) status |= LPS_ROW_EMPTY;
  }
  const bool row_finite = !has_nan && xmax != INFINITY && xmax != -INFINITY;
  // chunk reference -> row reference factors, and the full-vocabulary mass
  const double wg = row_finite ? (double)__fmul_rn(xmax, c) : 0.0;
  if (tid < G) {
    const float xq = key2f(S.u.f.cmk[tid]);
    S.u.f.scale[tid] = (row_finite && xq != -INFINITY) ? exp2((double)__fmul_rn(xq, c) - wg) : 0.0;
  }
  __syncthreads();
  double Zfull = 0.0;
  for (int q = 0; q < G; q++) Zfull += (double)S.u.f.czs[q] * S.u.f.scale[q];
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

  auto zval = [&](float xv) -> float { return greedy ? xv : __fdiv_rn(xv, T); };
  auto cand = [&](int i) -> uint2 {
    int q = 0;
    while (q + 1 < G && (int)S.u.f.pre[q + 1] <= i) q++;
    return cands[(int64_t)q * PUBCAP + (i - (int)S.u.f.pre[q])];
  };
  // candidates with z >= the kk-th largest z -> sorted kept list; K, or -1 on overflow
  auto collect = [&](int kk) -> int {
    const int kke = kk < NC ? kk : NC;
    const uint32_t kx = kke > 0 ? block_select_kth(NC, (uint32_t)kke, [&](int i) { return cand(i).x; }, S) : 0u;
    const float zk = zval(key2f(kx));
    if (tid == 0) S.mi[11] = 0;
    __syncthreads();
    for (int i = tid; i < NC; i += FT) {
      const uint2 cv = cand(i);
      const float z = zval(key2f(cv.x));
      if (kke == 0 || z >= zk) {
        const int q = atomicAdd(&S.mi[11], 1);
        if (q < KEPTCAP) {
          S.u.f.kkey[q] = f2key(z);
          S.u.f.kx[q] = cv.x;
          S.u.f.kidx[q] = (int32_t)cv.y;
          S.u.f.km[q] = mass_fixed(mass_f(z, zmax));
        }
      }
    }
    __syncthreads();
    const int K = S.mi[11];
    __syncthreads();
    if (K > KEPTCAP) return -1;
    rank_sort_kept(K, S);
    return K;
  };

  if (status == 0 && mode == MODE_GREEDY) {
    token = gam;
    cut = xmax;
    ties = 1;
    kept_n = 1;
    qprob = (qtok >= 0 && qtok == gam) ? 1.0f : 0.0f;
    chosen_z = xmax;
  } else if (status == 0 && mode == MODE_TOPK) {
    const int K = collect(topk < V ? topk : V);
    if (K <= 0) return (16);
    sorted_prefix(K, 0, S);
    const uint64_t Zk = S.u.f.cum[K - 1];
    int nf = K;
    if (topp < 1.0f) {  // keep sorted position p iff p == 0 or cum[p-1] <= p * Zk
      const double pl = topp > 0.0f ? (double)topp * (double)Zk : 0.0;
      uint64_t limit = (uint64_t)pl;
      if (limit >= Zk) limit = Zk - 1;
      if (tid == 0) S.mi[12] = K;
      __syncthreads();
      for (int pz = tid; pz < K; pz += FT)
        if (S.u.f.cum[pz] > limit && (pz == 0 || S.u.f.cum[pz - 1] <= limit)) S.mi[12] = pz + 1;
      __syncthreads();
      nf = S.mi[12];
    }
    if (minp > 0.0f) {  // keep e >= min_p (the maximum has e == 1)
      if (tid == 0) S.mi[13] = nf;
      __syncthreads();
      for (int pz = tid; pz < nf; pz += FT) {
        const bool ok = mass_f(key2f(S.u.f.kkey[S.u.f.kord[pz]]), zmax) >= minp;
        const bool okp = pz == 0 || mass_f(key2f(S.u.f.kkey[S.u.f.kord[pz - 1]]), zmax) >= minp;
        if (!ok && okp) S.mi[13] = pz;
      }
      __syncthreads();
      nf = S.mi[13];
      if (nf == 0) status |= LPS_ROW_EMPTY;
    }
    // typical-p with top-k active: the row holds -inf, the reference keeps only the argmax
    if (status == 0 && typp < 1.0f) nf = 1;
    if (status == 0) {
      const uint64_t Zf = S.u.f.cum[nf - 1];
      const uint32_t ck = S.u.f.kkey[S.u.f.kord[nf - 1]];
      cut = key2f(ck);
      int eq_all = 0, eq_kept = 0, nfin = 0;
      for (int q = 0; q < K; q++) {
        const uint32_t kq = S.u.f.kkey[S.u.f.kord[q]];
        eq_all += kq == ck ? 1 : 0;
        eq_kept += (kq == ck && q < nf) ? 1 : 0;
        nfin += (q < nf && kq != kNegInfKey) ? 1 : 0;
      }
      ties = eq_kept == eq_all ? -1 : eq_kept;
      kept_n = nfin;
      // draw in vocabulary order over the kept prefix
      for (int pz = tid; pz < nf; pz += FT) {
        const int si = S.u.f.kord[pz];
        const int ii = S.u.f.kidx[si];
        int rk = 0;
        for (int q = 0; q < nf; q++) rk += S.u.f.kidx[S.u.f.kord[q]] < ii ? 1 : 0;
        S.u.f.iord[rk] = si;
      }
      __syncthreads();
      uint64_t target = (uint64_t)((double)u * (double)Zf);
      if (target >= Zf) target = Zf - 1;
      if (tid == 0) {
        uint64_t a = 0;
        int pick = S.u.f.iord[nf - 1];
        for (int q = 0; q < nf; q++) {
          const uint64_t m = S.u.f.km[S.u.f.iord[q]];
          if (m && a <= target && target < a + m) { pick = S.u.f.iord[q]; break; }
          a += m;
        }
        S.mi[14] = pick;
        int qs = -1;
        if (qtok >= 0)
          for (int q = 0; q < nf; q++)
            if (S.u.f.kidx[S.u.f.kord[q]] == qtok) qs = S.u.f.kord[q];
        S.mi[15] = qs;
      }
      __syncthreads();
      const int ps = S.mi[14];
      token = S.u.f.kidx[ps];
      chosen_z = key2f(S.u.f.kkey[ps]);
      if (S.mi[15] >= 0) qprob = (float)((double)S.u.f.km[S.mi[15]] / (double)Zf);
    }
  } else if (status == 0 && (mode == MODE_PURE || mode == MODE_NUCLEUS)) {
    uint32_t vkey = 0, n_tie = kNoTie;
    double qmass = -1.0;
    if (mode == MODE_PURE) {
      if (tid < G) S.u.f.keptm[tid] = (double)S.u.f.czs[tid] * S.u.f.scale[tid];
      if (tid < G) S.u.f.ctie[tid] = 0;
      __syncthreads();
      kept_n = V - (int)ninf_all;
    } else {
      // exact cut among the region candidates (streamed from L2), above-region masses rescaled to the row
      double A = 0.0;
      for (int q = 0; q < G; q++) A += S.u.f.abv[q] * S.u.f.scale[q];
      const uint64_t Af = (uint64_t)(A * (double)kMassScale);
      const uint64_t Pf = (uint64_t)((double)topp * Zfull * (double)kMassScale);
      auto cz = [&](int i, uint32_t* k, uint64_t* m) {
        const uint2 cv = cand(i);
        const float z = __fdiv_rn(key2f(cv.x), T);
        *k = f2key(z);
        *m = mass_fixed(mass_f(z, zmax));
      };
      const MassSel ms = block_mass_select(NC, Af, Pf, cz, S.u.f.cum, S);
      if (!ms.ok || ms.ceq == 0) return (64);
      vkey = ms.key;
      const uint64_t e1 = ms.meq / ms.ceq;
      const uint64_t nt = e1 ? (Pf - ms.above) / e1 + 1 : (uint64_t)ms.ceq;
      n_tie = nt >= ms.ceq ? kNoTie : (uint32_t)nt;
      // kept candidate mass per chunk; ties at the cut listed for their index order
      if (tid < G) { S.u.f.keptf[tid] = 0; S.u.f.keptc[tid] = 0; }
      if (tid == 0) { S.mi[11] = 0; S.md[2] = -1.0; }
      __syncthreads();
      for (int i = tid; i < NC; i += FT) {
        const uint2 cv = cand(i);
        const float z = __fdiv_rn(key2f(cv.x), T);
        const uint32_t k = f2key(z);
        const uint64_t m = mass_fixed(mass_f(z, zmax));
        const int q = (int)cv.y / FCH;
        if (k > vkey) {
          atomicAdd(&S.u.f.keptf[q], (unsigned long long)m);
          atomicAdd(&S.u.f.keptc[q], 1u);
          if ((int64_t)cv.y == qtok) S.md[2] = (double)m / (double)kMassScale;
        } else if (k == vkey) {
          const int t = atomicAdd(&S.mi[11], 1);
          if (t < KEPTCAP) { S.u.f.kidx[t] = (int32_t)cv.y; S.u.f.km[t] = m; S.u.f.kx[t] = cv.x; S.u.f.kkey[t] = k; }
        }
      }
      __syncthreads();
      const int nties = S.mi[11];
      if (nties > KEPTCAP) return (32);
      rank_sort_kept(nties, S);  // equal keys: lowest index first
      if (tid == 0) {
        const int keep = n_tie == kNoTie ? nties : (int)n_tie;
        for (int pz = 0; pz < nties; pz++) {
          const int si = S.u.f.kord[pz];
          const int q = S.u.f.kidx[si] / FCH;
          if (pz < keep) {
            S.u.f.keptf[q] += S.u.f.km[si];
            S.u.f.keptc[q] += 1u;
            if (S.u.f.kidx[si] == qtok) S.md[2] = (double)S.u.f.km[si] / (double)kMassScale;
          }
        }
        uint32_t tb = 0;
        int nk = 0;
        for (int q = 0; q < G; q++) {
          S.u.f.ctie[q] = tb;
          for (int pz = 0; pz < keep; pz++) tb += (S.u.f.kidx[S.u.f.kord[pz]] / FCH == q) ? 1u : 0u;
          S.u.f.keptm[q] = S.u.f.abv[q] * S.u.f.scale[q] + (double)S.u.f.keptf[q] / (double)kMassScale;
          nk += (int)S.u.f.nab[q] + (int)S.u.f.keptc[q];
        }
        S.mi[15] = nk;
        // the cut's whole division-collision group must lie inside the region
        const float xv = key2f(S.u.f.kx[S.u.f.kord[0]]);
        const float xl = collision_lo(xv, T);
        float xh = xv;
        for (int it = 0; it < 64; it++) {
          const uint32_t k = f2key(xh);
          if (k >= 0xFFFFFFFEu) break;
          const float y = key2f(k + 1u);
          if (__fdiv_rn(y, T) != key2f(vkey)) break;
          xh = y;
        }
        const int bl = (int)floorf(__fmul_rn(__fmul_rn(xl, c), (float)HS));
        const int bh = (int)floorf(__fmul_rn(__fmul_rn(xh, c), (float)HS));
        S.mi[14] = (bl >= blo && bh <= bhi) ? 1 : 0;
      }
      __syncthreads();
      if (!S.mi[14]) return (128);
      ties = n_tie == kNoTie ? -1 : (int32_t)n_tie;
      cut = key2f(vkey);
      kept_n = S.mi[15];
      qmass = S.md[2];
    }
    // the chunk holding u * Zf, then its exact scan in vocabulary order
    double Zf = 0.0;
    for (int q = 0; q < G; q++) Zf += S.u.f.keptm[q];
    const double target = (double)u * Zf;
    int js = G - 1;
    double start = 0.0;
    {
      double a = 0.0;
      int last_pos = -1;
      for (int q = 0; q < G; q++) {
        if (S.u.f.keptm[q] > 0.0) last_pos = q;
        if (S.u.f.keptm[q] > 0.0 && target < a + S.u.f.keptm[q]) { js = q; break; }
        a += S.u.f.keptm[q];
        js = last_pos >= 0 ? last_pos : js;
      }
      for (int q = 0; q < js; q++) start += S.u.f.keptm[q];
    }
    if (!P.skip_draw) {
      const int lo2 = js * FCH;
      const int n2 = (V - lo2) < FCH ? (V - lo2) : FCH;
      if (pen) build_pen(S, hrow, hlen, lo2, n2);
      const FPen fp2{pen, rep, pres, freq, lo2, &S};
      float y[FE];
      load_chunk<DT, VEC>(row, lo2, n2, fp2, y);
      const uint32_t tie0 = S.u.f.ctie[js];
      uint32_t trun = 0;
      double run = start;
      if (tid == 0) { S.mi[8] = -1; S.mi[4] = -1; }
      __syncthreads();
      for (int v = 0; v < NV; v++) {
        double mm[VEC];
        float zz[VEC];
        uint32_t tloc = 0;
#pragma unroll
        for (int e = 0; e < VEC; e++) {
          const int l = (v * FT + tid) * VEC + e;
          zz[e] = l < n2 ? __fdiv_rn(y[v * VEC + e], T) : -INFINITY;
          tloc += (mode == MODE_NUCLEUS && zz[e] != -INFINITY && f2key(zz[e]) == vkey) ? 1u : 0u;
        }
        uint32_t ttot = 0;
        const uint32_t tex = fexcl_scan<uint32_t>(tloc, &ttot, S.r32);
        uint32_t rk = tie0 + trun + tex;
        double msum = 0.0;
#pragma unroll
        for (int e = 0; e < VEC; e++) {
          bool kept = zz[e] != -INFINITY;
          if (mode == MODE_NUCLEUS && kept) {
            const int b = (int)floorf(__fmul_rn(__fmul_rn(y[v * VEC + e], c), (float)HS));
            const uint32_t kz = f2key(zz[e]);
            if (b > bhi) kept = true;
            else if (b < blo) kept = false;
            else kept = kz > vkey || (kz == vkey && (n_tie == kNoTie || rk < n_tie));
            if (kz == vkey) rk++;
          }
          mm[e] = kept ? (double)mass_f(zz[e], zmax) : 0.0;
          msum += mm[e];
        }
        double btot;
        const double bex = fexcl_scan<double>(msum, &btot, S.rd);
        if (msum > 0.0 && run + bex <= target && target < run + bex + msum) {
          double a = run + bex;
#pragma unroll
          for (int e = 0; e < VEC; e++) {
            if (mm[e] > 0.0 && a <= target && target < a + mm[e]) S.mi[8] = (v * FT + tid) * VEC + e;
            a += mm[e];
          }
        }
#pragma unroll
        for (int e = 0; e < VEC; e++)
          if (mm[e] > 0.0) atomicMax(&S.mi[4], (v * FT + tid) * VEC + e);
        __syncthreads();
        const bool found = S.mi[8] >= 0;
        __syncthreads();
        if (found) break;
        run += btot;
        trun += ttot;
      }
      const int lp = S.mi[8] >= 0 ? S.mi[8] : S.mi[4];
      token = lp >= 0 ? (int64_t)(lo2 + lp) : -1;
      if (token >= 0 && P.chosen_logprob)
        chosen_z = __fdiv_rn(penalized_logit<DT>(row, (int)token, hrow, hlen, pen, rep, pres, freq, S), T);
    }
    if (P.query_prob && qtok >= 0) {
      const float xq = penalized_logit<DT>(row, (int)qtok, hrow, hlen, pen, rep, pres, freq, S);
      const float zq = __fdiv_rn(xq, T);
      if (mode == MODE_PURE) {
        qprob = zq != -INFINITY ? (float)((double)mass_f(zq, zmax) / Zf) : 0.0f;
      } else {
        const int bq = (int)floorf(__fmul_rn(__fmul_rn(xq, c), (float)HS));
        if (bq > bhi && zq != -INFINITY) qprob = (float)((double)mass_f(zq, zmax) / Zf);
        else if (qmass >= 0.0) qprob = (float)(qmass / Zf);
      }
    }
  }
  if (P.skip_draw && !greedy) token = -1;

  // ---- outputs ----
  if (P.chosen_logprob && tid == 0) {
    float lp = NAN;
    if (token >= 0 && Zfull > 0.0 && chosen_z == chosen_z)
      lp = (float)((double)__fsub_rn(chosen_z, zmax) - lnZ);
    P.chosen_logprob[r] = lp;
  }
  if (ntop > 0 && status == 0) {
    const int K = collect(ntop < V ? ntop : V);
    if (K < 0) return (256);
    const int nt = ntop < K ? ntop : K;
    for (int q = tid; q < P.n_top; q += FT) {
      if (q < nt) {
        const int si = S.u.f.kord[q];
        P.top_logprobs[(int64_t)r * P.n_top + q] = (float)((double)__fsub_rn(key2f(S.u.f.kkey[si]), zmax) - lnZ);
        if (P.top_ids) P.top_ids[(int64_t)r * P.n_top + q] = S.u.f.kidx[si];
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
    gen_row<DT, 1>(F.k, r, SU.g);  // element loads: the lean variant of the general path
  }
}

}  // namespace lps
