// The row-group sampling kernel (layout and protocol: lps_rowgroup.h).
#pragma once

namespace lps {
namespace rg {

// Bounded spin of one thread on a row counter; false when the bound was hit.
__device__ __forceinline__ bool wait_count(uint32_t* p, uint32_t n) {
  for (int spins = 0; spins < (1 << 22); spins++) {
    if (ld_agent(p) >= n) return true;
    __builtin_amdgcn_s_sleep(1);
  }
  return false;
}

// ===========================================================================
// Chunk phase.  Returns the row's mode (MODE_DEFER: nothing published).
// ===========================================================================
template <int DT, int VPE, int NE>
__device__ __forceinline__ int chunk_phase(const RgParams& F, RgChunkS<NE>& S, const int r, const int j) {
  using CK = Chk<DT, VPE, NE>;
  const KParams& P = F.k;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int G = F.G;
  const int v0 = j * F.cv;
  const int nv = min(F.cv, F.nvec - v0);
  const char* row = row_ptr<DT>(P, r);
  RgSum* sums = F.sums + (int64_t)r * 2 * MAXG;
  uint32_t* ctr = F.counters + (int64_t)r * 32;

  // ---- the row's parameters and first history ids, then the chunk's loads ----
  // (issued first so that they are not queued behind the chunk's 16-byte loads)
  RG_STAMP(0);
  const RowCfg g = row_cfg(P, r);
  const int32_t* hrow0 = P.history ? P.history + (int64_t)r * P.history_stride : nullptr;
  const int hid = (hrow0 && (int64_t)tid < P.history_stride) ? hrow0[tid] : -1;
  CK C;
  C.load(row, v0, nv);
  C.mask(row_allowed(P, r), v0, nv);
  if (g.mode == MODE_DEFER) return MODE_DEFER;
  const int mode = g.mode;
  const bool greedy = g.greedy;
  const float T = g.T;
  const float c = __fdiv_rn(kLog2e, greedy ? 1.0f : T);
  uint32_t flags = 0;

  // ---- penalties ----
  if (g.pen) {
    if (!build_counts<NE>(S, g.hrow, g.hlen, tid < g.hlen ? hid : -1, v0 * VPE, nv * VPE)) flags |= RF_HISTORY;
    apply_counts(C, S.hc, nv, g.rep, g.pres, g.freq);
  }

  RG_STAMP(1);
  // ---- thread and chunk max (NaN ignored here; each mode finds NaN its own way) ----
  float tm = -INFINITY;
#pragma unroll
  for (int s = 0; s < NE; s++) tm = fmaxf(tm, C.x[s]);
  const bool hist_mode = mode == MODE_NUCLEUS || mode == MODE_PURE;
  if (hist_mode) {  // clear the histogram before the barrier of the max
    u32x4* h4 = reinterpret_cast<u32x4*>(S.hist);
#pragma unroll
    for (int i = 0; i < HB * 8 / 16 / NT; i++) h4[i * NT + tid] = u32x4{0u, 0u, 0u, 0u};
  }
  const float M = bred(tm, S.f, OpMax{});
  const bool Mfin = M != INFINITY && M != -INFINITY;
  const float ref = Mfin ? ceilf(__fmul_rn(M, c)) : (M == INFINITY ? INFINITY : -INFINITY);

  RG_STAMP(2);
  RgSum sm{};
  sm.mkey = f2key(M);
  sm.amax = 0x7FFFFFFF;
  sm.ref = ref;
  sm.xcc = xcc_id();
  sm.reg[0] = sm.reg[1] = sm.reg[2] = sm.reg[3] = 1 << 30;
  // this wave's candidate segment
  const uint32_t wcap = (uint32_t)(F.capw / NW);
  uint2* wseg = F.cands + (int64_t)r * CAPR + (int64_t)j * F.capw + (int64_t)wv * wcap;
  uint32_t wn = 0;
  const bool want_lp = P.chosen_logprob || g.ntop > 0;
  RG_STAMP(14);

  if (mode == MODE_GREEDY) {
    // ---- first argmax (torch.argmax: the first NaN if any) ----
    uint32_t tn = 0;
#pragma unroll
    for (int s = 0; s < NE; s++) tn |= C.x[s] != C.x[s] ? 1u : 0u;
    int best = 0x7FFFFFFF;
    if (tn) {
#pragma unroll
      for (int s = 0; s < NE; s++)
        if (C.x[s] != C.x[s]) best = min(best, CK::index(v0, s));
    }
    const int bnan = bred(best, S.i1, OpMin{});
    __syncthreads();
    if (bnan != 0x7FFFFFFF) {
      sm.mkey = 0xFFFFFFFFu;
      sm.amax = bnan;
    } else {
      best = 0x7FFFFFFF;
      if (tm == M) {
#pragma unroll
        for (int s = 0; s < NE; s++)
          if (C.x[s] == M) best = min(best, CK::index(v0, s));
      }
      sm.amax = bred(best, S.i2, OpMin{});
    }
  }

  RG_STAMP(15);
  if ((mode == MODE_TOPK || mode == MODE_GREEDY) && (want_lp || mode == MODE_TOPK)) {
    // ---- chunk mass (logprob rows): exp2(fma(x, c, -ref)), fp32 per vector, fp64 across ----
    if (want_lp && Mfin) {
      double zs = 0.0;
#pragma unroll
      for (int i = 0; i < CK::NV; i++) {
        float a = 0.0f;
#pragma unroll
        for (int e = 0; e < VPE; e++) a += emass(C.x[i * VPE + e], c, ref);
        zs += (double)a;
      }
      sm.zsum = bred(zs, S.d, OpAdd{});
    }
    RG_STAMP(3);
    if (g.kprime > 0) {
      // ---- candidates: every logit at or above the chunk threshold ----
      const uint32_t m = (uint32_t)((g.kprime + NW - 1) / NW);
      const uint32_t v1[1] = {f2key(tm)};
      const uint32_t wth = wave_kth_largest<1>(v1, m);
      uint32_t th = bred(wth, S.u, OpMin{});
      if (!greedy && th > kNegInfKey + 1u && th != 0xFFFFFFFFu) th = f2key(collision_lo(key2f(th), T));
      // -inf is never a candidate (it has no mass); NaN always is (!(x < t))
      const float xth = fmaxf(key2f(th), -3.40282347e38f);
      wn = wave_emit<NE>([&](int s) { return !(C.x[s] < xth); },
                         [&](int s) { return make_uint2(__float_as_uint(C.x[s]), (uint32_t)CK::index(v0, s)); },
                         wseg, wcap);
    }
  }

  if (hist_mode) {
    // ---- exact mass histogram of the chunk ----
    uint32_t bins[NE / 2 + 1];
#pragma unroll
    for (int i = 0; i < NE / 2 + 1; i++) bins[i] = 0u;  // (read only when the chunk max is finite)
    // masses under the histogram (each < 2^-31, at most NE of them: an fp32
    // sum is within 2^-40 of the chunk's largest mass)
    float zlow = 0.0f;
    if (Mfin) {
#pragma unroll
      for (int s = 0; s < NE; s++) {
        const float e = emass(C.x[s], c, ref);
        const uint32_t b = ebin(e);
        // masses under the histogram go to a per-lane spare slot (no branch, no conflicts)
        atomicAdd(&S.hist[b != BELOW ? b : (uint32_t)(HB + lane)],
                  (1ull << 48) | (unsigned long long)(__float_as_uint(e) & 0xFFFFu));
        zlow += b == BELOW ? e : 0.0f;
        bins[s >> 1] |= b << (16 * (s & 1));
      }
    }
    RG_STAMP(8);
    __syncthreads();
    RG_STAMP(3);
    // exact chunk mass, NaN count, and the bins as fp32 masses for the merge
    // (thread t: bins t + NT i, so the LDS reads and the stores are unit-stride)
    float* hout = F.hist + ((int64_t)r * G + j) * HPUB;
    {
      double zs = 0.0;
      uint32_t nanc = 0;
#pragma unroll
      for (int i = 0; i < HLT; i++) {
        const int b = tid + NT * i;
        const unsigned long long a = S.hist[b];
        double m = bin_mass_u(b, a);
        if (b == HB_NAN) { nanc = (uint32_t)(a >> 48); m = 0.0; }
        zs += m;
        hout[b] = (float)m;
      }
      zs = wreduce(zs + (double)zlow, OpAdd{});
      nanc = wreduce(nanc, OpAdd{});
      if (lane == 0) { S.d[wv] = zs; S.u[wv] = nanc; }
      __syncthreads();
      zs = 0.0;
      nanc = 0;
#pragma unroll
      for (int i = 0; i < NW; i++) { zs += S.d[i]; nanc += S.u[i]; }
      sm.zsum = zs;
      sm.nanbin = nanc;
    }
    // ---- publish the summary and the bins, one barrier among the row's chunks ----
    if (tid == 0) store_sum(sums + j, sm);
    RG_STAMP(4);
    release_agent();
    __syncthreads();
    if (tid == 0) {
      release_count();
      add_agent(ctr + 2, 1u);
      S.mi[6] = wait_count(ctr + 2, (uint32_t)G) ? 0 : 1;
      acquire_one();
    }
    __syncthreads();
    acquire_agent();
    RG_STAMP(5);
    if (S.mi[6]) flags |= RF_REGION;

    // ---- row reference, row mass ----
    if (wv == 0) {
      RgSum a{};
      if (lane < G) a = ld_pub(sums + lane);
      const bool af = lane < G && a.ref != INFINITY && a.ref != -INFINITY;
      const float R = wmax(af ? a.ref : -INFINITY);
      const double sc = af ? ldexp(1.0, (int)(a.ref - R)) : 0.0;
      const double Z = wsum(af ? a.zsum * sc : 0.0);
      if (lane < G) { S.rf[lane] = af ? a.ref : -INFINITY; }
      if (lane == 0) { S.md[0] = Z; S.mf[0] = R; }
    }
    __syncthreads();
    const float R = S.mf[0];
    const double Z = S.md[0];
    const bool rfin = R != INFINITY && R != -INFINITY;
    RG_STAMP(9);
    // ---- merged histogram: thread t owns row bins 4095 - HPT t - i, i < HPT (descending) ----
    double mrg[HPT];
#pragma unroll
    for (int i = 0; i < HPT; i++) mrg[i] = 0.0;
    if (rfin) {
      // two chunks' bins in flight at a time, summed in chunk order
      for (int w0 = 0; w0 < G; w0 += 2) {
        float hw[2][HPT];
        double sc[2];
#pragma unroll
        for (int q = 0; q < 2; q++) {
          const int w = w0 + q;
          const float rw = w < G ? S.rf[w] : -INFINITY;
          const int dl = (rw != -INFINITY) ? (int)(R - rw) : 4096;
          // the chunk's published index of my lowest row bin
          const int src = HPUB - HPT - HPT * tid + HOCT * dl;
          sc[q] = dl < 1024 ? ldexp(1.0, -dl) : 0.0;
          const float* hsrc = F.hist + ((int64_t)r * G + w) * HPUB + src;
#pragma unroll
          for (int i = 0; i < HPT; i += 2) {
            const float2 v = src <= HPUB - HPT ? ld_pub(reinterpret_cast<const float2*>(hsrc + i)) : make_float2(0.f, 0.f);
            hw[q][i] = v.x; hw[q][i + 1] = v.y;
          }
          if (src == HPUB - HPT) hw[q][HPT - 1] = 0.0f;  // the chunk's NaN bin
        }
#pragma unroll
        for (int q = 0; q < 2; q++)
#pragma unroll
          for (int i = 0; i < HPT; i++) mrg[i] += (double)hw[q][HPT - 1 - i] * sc[q];
      }
      if (tid == 0) mrg[0] = 0.0;  // row bin HB - 1: NaN only
    }
    RG_STAMP(10);
    double msum = 0.0;
#pragma unroll
    for (int i = 0; i < HPT; i++) msum += mrg[i];
    double stot;
    const double sx = bscan<double>(msum, &stot, S.d2);
    // ---- regions: bins whose cumulative interval meets the targets ----
    const double eps = 1e-6 * Z;
    const bool nuc = mode == MODE_NUCLEUS;
    const double Pm = nuc ? (g.topp > 0.0f ? (double)g.topp * Z : 0.0) : Z;
    int lo = 1 << 30, hi = -1;
    {
      double a = sx;
#pragma unroll
      for (int i = 0; i < HPT; i++) {
        const int b = HB - 1 - HPT * tid - i;
        if (nuc && mrg[i] > 0.0 && a <= Pm + eps && a + mrg[i] >= Pm - eps) { lo = min(lo, b); hi = max(hi, b); }
        a += mrg[i];
      }
    }
    const int lo1 = nuc ? bred(lo, S.i1, OpMin{}) : (1 << 30);
    const int hi1 = nuc ? bred(hi, S.i2, OpMax{}) : (1 << 30);
    // cumulative mass at the top of region 1 and at its bottom: the kept mass
    // lies between them, and the draw at u times it
    if (nuc && hi1 >= 0) {
      double a = sx;
#pragma unroll
      for (int i = 0; i < HPT; i++) {
        const int b = HB - 1 - HPT * tid - i;
        if (b == hi1) S.md[1] = a;
        if (b == lo1) S.md[2] = a + mrg[i];
        a += mrg[i];
      }
    }
    __syncthreads();
    if (nuc && hi1 < 0) flags |= RF_REGION;
    const float u = fminf(fmaxf(g.u == g.u ? g.u : 0.0f, 0.0f), 0.99999994f);
    const double t_lo = (nuc ? (double)u * S.md[1] : (double)u * Z) - eps;
    const double t_hi = (nuc ? (double)u * S.md[2] : (double)u * Z) + eps;
    lo = 1 << 30;
    hi = -1;
    double nest = 0.0;
    {
      double a = sx;
#pragma unroll
      for (int i = 0; i < HPT; i++) {
        const int b = HB - 1 - HPT * tid - i;
        const bool in2 = mrg[i] > 0.0 && a <= t_hi && a + mrg[i] >= t_lo;
        if (in2) { lo = min(lo, b); hi = max(hi, b); }
        if (in2 || (b >= lo1 && b <= hi1)) nest += mrg[i] / bin_base(b);
        a += mrg[i];
      }
    }
    const int lo2 = bred(lo, S.i3, OpMin{});
    const int hi2 = bred(hi, S.i1, OpMax{});
    nest = bred(nest, S.d3, OpAdd{});
    if (hi2 < 0 || !rfin) flags |= RF_REGION;
    if (nest > (double)CAPR) flags |= RF_OVERFLOW;
    sm.reg[0] = nuc ? lo1 : (1 << 30);
    sm.reg[1] = nuc ? hi1 : (1 << 30);
    sm.reg[2] = hi2 >= 0 ? lo2 : (1 << 30);
    sm.reg[3] = hi2 >= 0 ? hi2 : (1 << 30);

    RG_STAMP(6);
    // ---- this chunk: candidates in either region, exact masses above them ----
    const int dl = Mfin && rfin ? (int)(R - ref) : 0;
    auto own = [&](int b) { return b >= (1 << 30) ? b : b + HOCT * dl; };
    const int l1 = own(sm.reg[0]), h1 = own(sm.reg[1]), l2 = own(sm.reg[2]), h2 = own(sm.reg[3]);
    double ab1 = 0.0, ab2 = 0.0;
    uint32_t nab = 0;
#pragma unroll
    for (int i = 0; i < HLT; i++) {
      const int b = tid + NT * i;
      const unsigned long long a = S.hist[b];
      const double m = b == HB_NAN ? 0.0 : bin_mass_u(b, a);
      if (b > h1 && b != HB_NAN) { ab1 += m; nab += (uint32_t)(a >> 48); }
      if (b > h2) ab2 += m;
    }
    RG_STAMP(11);
    ab1 = wreduce(ab1, OpAdd{});
    ab2 = wreduce(ab2, OpAdd{});
    nab = wreduce(nab, OpAdd{});
    if (lane == 0) { S.d4[wv] = ab1; S.d5[wv] = ab2; S.u4[wv] = nab; }
    __syncthreads();
    sm.ab1 = 0.0; sm.ab2 = 0.0; sm.nab1 = 0;
#pragma unroll
    for (int i = 0; i < NW; i++) { sm.ab1 += S.d4[i]; sm.ab2 += S.d5[i]; sm.nab1 += S.u4[i]; }
    if (Mfin) {
      // the elements of either region, published by wave ballots (bins in pairs)
      static_assert(NE % 2 == 0, "bin pairs");
      uint32_t L1, C1, L2, C2;
      region_pair(l1, h1, L1, C1);
      region_pair(l2, h2, L2, C2);
      uint32_t n = 0;
#pragma unroll
      for (int k = 0; k < NE / 2; k++) {
        const uint32_t t1 = in_region2(bins[k], L1, C1), t2 = in_region2(bins[k], L2, C2);
        const uint32_t sl = t1 | t2;
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const bool on = (sl >> (16 * h) & 0xFFFFu) != 0u;
          const uint64_t m = __builtin_amdgcn_ballot_w64(on);
          if (m) {
            if (on) {
              const uint32_t p =
                  n + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
              const int s2 = 2 * k + h;
              const uint32_t f = ((t1 >> (16 * h) & 0xFFFFu) ? (1u << 30) : 0u) |
                                 ((t2 >> (16 * h) & 0xFFFFu) ? (1u << 31) : 0u);
              if (p < wcap) wseg[p] = make_uint2(__float_as_uint(C.x[s2]), (uint32_t)CK::index(v0, s2) | f);
            }
            n += (uint32_t)__popcll(m);
          }
        }
      }
      wn = n;
    }
  }

  // ---- the chunk's summary, then the arrival count ----
  RG_STAMP(7);
  sm.flags = flags;
  if (tid == 0) store_sum(sums + MAXG + j, sm);
  store_wave_count(sums + MAXG + j, wn, wcap);
  return mode;
}

// Block-wide penalised logit of one id (legality bit, history count).
template <int DT>
__device__ float penal_logit(const KParams& P, const RowCfg& g, const char* row, int r, int id, RgX& S) {
  uint32_t c = 0;
  if (g.pen)
    for (int k = threadIdx.x; k < g.hlen; k += NT) c += g.hrow[k] == id ? 1u : 0u;
  c = bred(c, S.u2, OpAdd{});
  float x = load1<DT>(row, id);
  if (!id_allowed(row_allowed(P, r), id)) x = -INFINITY;
  if (g.pen && c) x = penalize(x, (int)c, g.rep, g.pres, g.freq);
  __syncthreads();
  return x;
}

// ===========================================================================
// Finaliser: the last chunk workgroup of row r.  Returns 0 when the row is
// done, else a reason code (the row is then sampled by the general kernel).
// ===========================================================================
template <int DT, int VPE>
__device__ __forceinline__ int final_phase(const RgParams& F, RgFinalS& S, const int r) {
  const KParams& P = F.k;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int G = F.G;
  const int V = P.V;
  const char* row = row_ptr<DT>(P, r);
  const RgSum* sums = F.sums + (int64_t)r * 2 * MAXG + MAXG;
  const uint2* cands = F.cands + (int64_t)r * CAPR;
  if (tid == 0) {  // the row's counters back to zero for the next launch
    F.counters[(int64_t)r * 32] = 0u;
    F.counters[(int64_t)r * 32 + 2] = 0u;
  }
  const RowCfg g = row_cfg(P, r);
  const int mode = g.mode;
  const bool greedy = g.greedy;
  const float T = g.T;
  const float c = __fdiv_rn(kLog2e, greedy ? 1.0f : T);

  // ---- candidates, first pass: entry k0 of wave segment s0, loaded before the
  // counts are known (in flight with the summaries); the rest after them ----
  const int capw = F.capw;
  const int nseg = G * NW;
  const int lgK = 31 - __builtin_clz(NT / nseg);  // entries per segment in the first pass
  const int s0 = tid >> lgK, k0 = tid & ((1 << lgK) - 1);
  auto seg_slot = [&](int sg, int k) -> int { return (sg / NW) * capw + (sg % NW) * (capw / NW) + k; };
  uint2 cv0 = make_uint2(0u, 0u);
  if (s0 < nseg) cv0 = ld_pub(cands + seg_slot(s0, k0));

  // ---- F1: the chunk summaries (wave 0) ----
  if (wv == 0) {
    RgSum a{};
    if (lane < G) a = ld_pub(sums + lane);
    const uint32_t xm = wreduce(lane < G ? (1u << a.xcc) : 0u, OpOr{});
    uint32_t fl = wreduce(lane < G ? a.flags : 0u, OpOr{});
    if (__builtin_popcount(xm) > 1) fl |= RF_SPLIT;
    const uint32_t mk = wmax(lane < G ? a.mkey : 0u);
    const int am = wmin(lane < G && a.mkey == mk ? a.amax : 0x7FFFFFFF);
    const bool af = lane < G && a.ref != INFINITY && a.ref != -INFINITY;
    const float R = wmax(af ? a.ref : -INFINITY);
    const double sc = af ? ldexp(1.0, (int)(a.ref - R)) : 0.0;
    const double Z = wsum(af ? a.zsum * sc : 0.0);
    const double A1 = wsum(af ? a.ab1 * sc : 0.0);
    const double A2 = wsum(af ? a.ab2 * sc : 0.0);
    const uint32_t nab = wsum(lane < G ? a.nab1 : 0u);
    const uint32_t nanb = wmax(lane < G ? a.nanbin : 0u);
    // segment counts; overflow beyond the first pass, prefixed over segments
    uint32_t ntot = 0, nover = 0, over = 0;
    if (lane < G) {
#pragma unroll
      for (int q = 0; q < NW; q++) {
        const uint32_t n = a.wc[q];
        over |= n == WC_OVER ? 1u : 0u;
        const uint32_t nn = n == WC_OVER ? 0u : n;
        S.wpre[lane * NW + q] = (int)nn;
        ntot += nn;
        nover += nn > (1u << lgK) ? nn - (1u << lgK) : 0u;
      }
    }
    if (wreduce(over, OpOr{})) fl |= RF_OVERFLOW;
    const uint32_t ncand = wsum(ntot);
    const uint32_t oinc = wscan_incl(nover);
    if (lane < G) {
      uint32_t o = oinc - nover;
#pragma unroll
      for (int q = 0; q < NW; q++) {
        const uint32_t nn = (uint32_t)S.wpre[lane * NW + q];
        S.opre[lane * NW + q] = (int)o;
        o += nn > (1u << lgK) ? nn - (1u << lgK) : 0u;
      }
      S.rf[lane] = af ? a.ref : -INFINITY;
      S.rm[lane] = a.mkey == 0xFFFFFFFFu ? INFINITY : key2f(a.mkey);
    }
    if (lane == 0) {
      S.mi[16] = (int)fl;
      S.mi[17] = (int)mk;
      S.mi[18] = am;
      S.mi[19] = (int)nab;
      S.mi[20] = (int)nanb;
      S.mi[21] = a.reg[0]; S.mi[22] = a.reg[1]; S.mi[23] = a.reg[2]; S.mi[24] = a.reg[3];
      S.mi[25] = (int)ncand;
      S.md[0] = Z; S.md[1] = A1; S.md[2] = A2;
      S.mf[0] = R;
    }
    if (lane == 63) S.mi[26] = (int)oinc;  // overflow entries of the row
  }
  __syncthreads();
  RG_STAMP(25);
  const uint32_t fl = (uint32_t)S.mi[16];
  if (fl) return 2 + (int)(fl << 4);
  const uint32_t mkey = (uint32_t)S.mi[17];
  const int gam = S.mi[18];
  const float xmax = key2f(mkey);
  const bool has_nan = mkey == 0xFFFFFFFFu || S.mi[20] != 0;
  int status = 0;
  if (!greedy) {
    if (has_nan || xmax == INFINITY || __fdiv_rn(xmax, T) == INFINITY) status |= LPS_ROW_NONFINITE;
    else if (xmax == -INFINITY) status |= LPS_ROW_EMPTY;
  }
  const float zmax = greedy ? xmax : __fdiv_rn(xmax, T);
  // the row's mass reference (logprob, nucleus and pure rows published theirs)
  const float Rref = (mode == MODE_NUCLEUS || mode == MODE_PURE || S.mf[0] != -INFINITY)
                         ? S.mf[0]
                         : (xmax != INFINITY && xmax != -INFINITY ? ceilf(__fmul_rn(xmax, c)) : 0.0f);
  const double Zfull = S.md[0];
  // ln of sum exp(z) over the row: Z is in units of 2^Rref of exp2(x c)
  const double lnZ = Zfull > 0.0 ? log(Zfull) + (double)Rref * 0.6931471805599453 : 0.0;
  float u = g.u;
  if (!(u >= 0.0f)) u = 0.0f;
  if (u >= 1.0f) u = 0.99999994f;

  // ---- candidates in register slots e * NT + t: e = 0 the first pass, e >= 1
  // the overflow entries (o = (e - 1) * NT + t of the row's overflow list) ----
  uint32_t ck[FPT];
  uint64_t cm[FPT];
  uint32_t cf[FPT];  // region flags (nucleus)
  const int NC = __builtin_amdgcn_readfirstlane(S.mi[25]);
  const int NO = __builtin_amdgcn_readfirstlane(S.mi[26]);
  if (NO > (FPT - 1) * NT) return 13;
  const bool p0 = s0 < nseg && k0 < S.wpre[min(s0, nseg - 1)];
  auto present = [&](int e) -> bool { return e == 0 ? p0 : (e - 1) * NT + tid < NO; };
  // slot of overflow entry o: the last segment whose overflow prefix is <= o
  auto over_slot = [&](int o) -> int {
    int lo = 0, hi = nseg - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (S.opre[mid] <= o) lo = mid; else hi = mid - 1;
    }
    return seg_slot(lo, (1 << lgK) + o - S.opre[lo]);
  };
  {
    uint2 cv[FPT];
    cv[0] = cv0;
#pragma unroll
    for (int e = 1; e < FPT; e++) {
      cv[e] = make_uint2(0u, 0u);
      if ((e - 1) * NT < NO && present(e)) cv[e] = ld_pub(cands + over_slot((e - 1) * NT + tid));
    }
#pragma unroll
    for (int e = 0; e < FPT; e++) {
      ck[e] = 0u;
      cf[e] = 0u;
      cm[e] = 0ull;
      if (e > 0 && (e - 1) * NT >= NO) continue;
      const int sl = e * NT + tid;
      const bool pr = present(e);
      const float xv = __uint_as_float(cv[e].x);
      const float zv = greedy ? xv : __fdiv_rn(xv, T);
      ck[e] = pr ? f2key(zv) : 0u;
      cf[e] = pr ? (cv[e].y >> 30) : 0u;
      S.cidx[sl] = (int32_t)(cv[e].y & 0x3FFFFFFFu);
      S.cx[sl] = xv;
      // a candidate's mass is a function of its scaled logit z alone, so ids
      // tied at one z weigh the same (the chunks' histograms used x; the two
      // differ by a rounding or two)
      cm[e] = (pr && (mode == MODE_NUCLEUS || mode == MODE_PURE)) ? zmass_fix(zv, Rref) : 0ull;
      if (pr && xv != xv) status |= LPS_ROW_NONFINITE;
    }
  }
  status = bred(status, S.i1, OpOr{});
  __syncthreads();
  RG_STAMP(26);
  if (greedy) status = 0;
  auto cidx = [&](int e) -> int { return S.cidx[e * NT + tid]; };

  int64_t token = -1;
  float cut = -INFINITY, qprob = 0.0f, chosen_z = NAN;
  int32_t ties = -1, kept_n = 0;
  int ntop_out = 0;
  const int64_t qtok = g.qtok;

  if (status == 0 && g.kprime > 0) {
    // ======================= top-k (and top-N logprobs) =======================
    const int keff = mode == MODE_TOPK ? (g.topk < V ? g.topk : V) : 0;
    int kc = keff > g.ntop ? keff : g.ntop;
    if (kc > NC) kc = NC;
    if (kc <= 0) return 3;
    const uint32_t kth = sel_count(ck, present, (uint32_t)kc, S);
    RG_STAMP(27);
    // the kept list: keys >= kth
    uint32_t cnt = 0;
#pragma unroll
    for (int e = 0; e < FPT; e++) cnt += (present(e) && ck[e] >= kth) ? 1u : 0u;
    uint32_t K;
    uint32_t p = bscan<uint32_t>(cnt, &K, S.u);
    if (K > (uint32_t)KEPT) return 4;
    const float Rt = xmax != INFINITY && xmax != -INFINITY ? ceilf(__fmul_rn(xmax, c)) : 0.0f;
#pragma unroll
    for (int e = 0; e < FPT; e++) {
      if (present(e) && ck[e] >= kth) {
        const int ix = cidx(e);
        S.kkey[p] = ((uint64_t)ck[e] << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)ix);
        S.kmass[p] = zmass_fix(key2f(ck[e]), Rt);
        p++;
      }
    }
    __syncthreads();
    // rank sort (keys are distinct: the index is part of the key)
    for (int i = tid; i < (int)K; i += NT) {
      const uint64_t ki = S.kkey[i];
      int rank = 0;
      int q = 0;
      for (; q + 4 <= (int)K; q += 4) {
        const uint64_t t0 = S.kkey[q], t1 = S.kkey[q + 1], t2 = S.kkey[q + 2], t3 = S.kkey[q + 3];
        rank += (t0 > ki ? 1 : 0) + (t1 > ki ? 1 : 0) + (t2 > ki ? 1 : 0) + (t3 > ki ? 1 : 0);
      }
      for (; q < (int)K; q++) rank += S.kkey[q] > ki ? 1 : 0;
      S.kord[rank] = i;
    }
    __syncthreads();
    RG_STAMP(28);
    auto kz = [&](int pos) -> uint32_t { return (uint32_t)(S.kkey[S.kord[pos]] >> 32); };
    auto kix = [&](int pos) -> int { return (int)(0xFFFFFFFFu - (uint32_t)S.kkey[S.kord[pos]]); };
    ntop_out = g.ntop < (int)K ? g.ntop : (int)K;
    if (mode == MODE_GREEDY) {
      token = gam;
      cut = xmax;
      ties = 1;
      kept_n = 1;
      qprob = (qtok >= 0 && qtok == gam) ? 1.0f : 0.0f;
      chosen_z = xmax;
    } else {
      // the top-k set: sorted positions whose key reaches the keff-th
      if (keff > (int)K || keff <= 0) return 5;
      const uint32_t kk = kz(keff - 1);
      int nk = (int)K;
      {
        int lastk = -1;
        for (int pz = tid; pz < (int)K; pz += NT)
          if (kz(pz) >= kk) lastk = max(lastk, pz);
        nk = bred(lastk, S.i2, OpMax{}) + 1;
      }
      // inclusive prefix of the kept masses in sorted order
      {
        const uint64_t mv = tid < nk ? (uint64_t)S.kmass[S.kord[tid]] : 0ull;
        uint64_t tot;
        const uint64_t ex = bscan<uint64_t>(mv, &tot, S.q);
        if (tid < nk) S.kcum[tid] = ex + mv;
        __syncthreads();
      }
      const uint64_t Zk = S.kcum[nk - 1];
      int nf = nk;
      if (g.topp < 1.0f) {  // keep sorted position p iff p == 0 or cum[p-1] <= top_p * Zk
        const double pl = g.topp > 0.0f ? (double)g.topp * (double)Zk : 0.0;
        uint64_t limit = (uint64_t)pl;
        if (limit >= Zk) limit = Zk - 1;
        int first = 0x7FFFFFFF;
        if (tid >= 1 && tid < nk && S.kcum[tid - 1] > limit) first = tid;
        nf = min(nf, bred(first, S.i3, OpMin{}));
        __syncthreads();
      }
      if (g.minp > 0.0f) {  // keep mass >= min_p * (the top mass)
        const float e0 = (float)((double)S.kmass[S.kord[0]] / kFix);
        int first = 0x7FFFFFFF;
        if (tid < nf && (float)((double)S.kmass[S.kord[tid]] / kFix) < __fmul_rn(g.minp, e0)) first = tid;
        const int f = bred(first, S.i1, OpMin{});
        __syncthreads();
        if (f < nf) nf = f;
        if (nf == 0) status |= LPS_ROW_EMPTY;
      }
      // typical-p with top-k active: the row then holds -inf, and the reference keeps only the argmax
      if (status == 0 && g.typp < 1.0f) nf = 1;
      if (status == 0) {
        const uint64_t Zf = S.kcum[nf - 1];
        const uint32_t ckey = kz(nf - 1);
        cut = key2f(ckey);
        if (P.kept_ties || P.kept_count) {
          uint32_t ea = 0, ek = 0, nfin = 0;
          if (tid < (int)K) {
            const uint32_t kq = kz(tid);
            ea = kq == ckey ? 1u : 0u;
            ek = (kq == ckey && tid < nf) ? 1u : 0u;
            nfin = (tid < nf && kq != kNegInfKey) ? 1u : 0u;
          }
          ea = bred(ea, S.u, OpAdd{});
          ek = bred(ek, S.u2, OpAdd{});
          nfin = bred(nfin, S.u3, OpAdd{});
          __syncthreads();
          ties = ek == ea ? -1 : (int32_t)ek;
          kept_n = (int32_t)nfin;
        }
        // inverse CDF in sorted order
        uint64_t target = (uint64_t)((double)u * (double)Zf);
        if (target >= Zf) target = Zf - 1;
        if (tid == 0) { S.mi[4] = nf - 1; S.mi[5] = -1; }
        __syncthreads();
        if (tid < nf) {
          const uint64_t hi_ = S.kcum[tid], lo_ = tid > 0 ? S.kcum[tid - 1] : 0ull;
          if (lo_ <= target && target < hi_) S.mi[4] = tid;
          if (qtok >= 0 && kix(tid) == qtok) S.mi[5] = tid;
        }
        __syncthreads();
        const int ps = S.mi[4];
        token = kix(ps);
        chosen_z = key2f(kz(ps));
        if (S.mi[5] >= 0) qprob = (float)((double)S.kmass[S.kord[S.mi[5]]] / (double)Zf);
      }
    }
  } else if (status == 0 && mode == MODE_GREEDY) {
    token = gam;
    cut = xmax;
    ties = 1;
    kept_n = 1;
    qprob = (qtok >= 0 && qtok == gam) ? 1.0f : 0.0f;
    chosen_z = xmax;
  } else if (status == 0 && (mode == MODE_NUCLEUS || mode == MODE_PURE)) {
    // ======================= nucleus / pure =======================
    const bool nuc = mode == MODE_NUCLEUS;
    const int lo1 = S.mi[21], hi1 = S.mi[22], lo2 = S.mi[23], hi2 = S.mi[24];
    const double Z = S.md[0];
    const uint64_t Zfx = (uint64_t)(Z * kFix);
    uint32_t vkey = 0, n_tie = kNoTie;
    uint64_t Zkept = Zfx;
    // whether every id whose z equals fl(x / T) lies inside row bins [lo, hi]
    // under the binning of each chunk that can hold it (one wave)
    // (one wave; lane w checks chunk w)
    auto group_inside = [&](float x, int lo, int hi) -> bool {
      const Group gr = collision_group(x, T);
      bool bad = false;
      if (lane < G) {
        const float rw = S.rf[lane], mw = S.rm[lane];
        if (rw != -INFINITY && !(gr.lo > mw)) {  // some id of this chunk may reach the group
          const int sh = HOCT * (int)(Rref - rw);
          const uint32_t el = ebin(emass(gr.lo, c, rw)), eh = ebin(emass(fminf(gr.hi, mw), c, rw));
          const int bl = (el == BELOW ? -(1 << 20) : (int)el) - sh;
          const int bh = (eh == BELOW ? -(1 << 20) : (int)min(eh, (uint32_t)HB_NAN - 1u)) - sh;
          bad = !(bl >= lo && bh <= hi);
        }
      }
      return gr.ok != 0 && __builtin_amdgcn_ballot_w64(bad) == 0ull;
    };
    // the kk-th lowest index among the candidates of key v selected by sel
    auto kth_index = [&](auto sel, uint32_t v, uint32_t kk) -> int {
      uint32_t ik[FPT];
#pragma unroll
      for (int e = 0; e < FPT; e++) ik[e] = (sel(e) && ck[e] == v) ? 0xFFFFFFFFu - (uint32_t)cidx(e) : 0u;
      auto has = [&](int e) -> bool { return sel(e) && ck[e] == v; };
      return (int)(0xFFFFFFFFu - sel_count(ik, has, kk, S));
    };
    int tie_lim = 0x7FFFFFFF;  // kept ids at the cut key: index <= tie_lim
    const bool want2 = !P.skip_draw;
    // ---- region lists: region 1 at kkey[0, N1), region 2 at kkey[N1, N1 + N2) ----
    uint32_t c12 = 0;
#pragma unroll
    for (int e = 0; e < FPT; e++)
      if (present(e)) c12 += ((nuc && (cf[e] & 1u)) ? 1u : 0u) + ((want2 && (cf[e] & 2u)) ? 0x10000u : 0u);
    uint32_t t12;
    const uint32_t p12 = bscan<uint32_t>(c12, &t12, S.u);
    const int N1 = (int)(t12 & 0xFFFFu), N2 = (int)(t12 >> 16), NL = N1 + N2;
    if (NL <= KEPT) {
      // ======== lists: rank sort, exact prefix masses in sorted order ========
      uint32_t q1 = p12 & 0xFFFFu, q2 = (uint32_t)N1 + (p12 >> 16);
#pragma unroll
      for (int e = 0; e < FPT; e++) {
        if (!present(e)) continue;
        const uint64_t key = ((uint64_t)ck[e] << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)cidx(e));
        if (nuc && (cf[e] & 1u)) { S.kkey[q1] = key; S.kmass[q1] = cm[e]; S.lslot[q1] = e * NT + tid; q1++; }
        if (want2 && (cf[e] & 2u)) { S.kkey[q2] = key; S.kmass[q2] = cm[e]; S.lslot[q2] = e * NT + tid; q2++; }
      }
      if (tid == 0) S.mi[13] = -1;
      __syncthreads();
      RG_STAMP(16);
      {  // rank sort: keys are distinct within a list (the index is part of the key);
         // 2^lg adjacent lanes share an entry, each comparing one slice of its list
        const int lg = NL <= 64 ? 3 : NL <= 128 ? 2 : NL <= 256 ? 1 : 0;
        const int ie = tid >> lg, part = tid & ((1 << lg) - 1);
        const int b = ie < N1 ? 0 : N1, n = ie < N1 ? N1 : N2;
        int rank = 0;
        if (ie < NL) {
          const uint64_t ki = S.kkey[ie];
          const int len = (n + (1 << lg) - 1) >> lg;
          const int q1 = min(b + n, b + part * len + len);
          int q = b + part * len;
          for (; q + 8 <= q1; q += 8) {
            uint64_t kq[8];
#pragma unroll
            for (int i = 0; i < 8; i++) kq[i] = S.kkey[q + i];
#pragma unroll
            for (int i = 0; i < 8; i++) rank += kq[i] > ki ? 1 : 0;
          }
          for (; q < q1; q++) rank += S.kkey[q] > ki ? 1 : 0;
        }
        for (int o = 1; o < (1 << lg); o <<= 1) rank += __shfl_xor(rank, o);
        if (ie < NL && part == 0) S.kord[b + rank] = ie;
      }
      __syncthreads();
      RG_STAMP(17);
      {  // inclusive prefix of the masses in sorted order (list 2's from kcum[N1 - 1])
        const uint64_t mv = tid < NL ? (uint64_t)S.kmass[S.kord[tid]] : 0ull;
        uint64_t tot;
        const uint64_t ex = bscan<uint64_t>(mv, &tot, S.q);
        if (tid < NL) S.kcum[tid] = ex + mv;
        __syncthreads();
      }
      RG_STAMP(27);
      // every thread finds the cut and the draw by binary search over the
      // prefixes; the two collision-group checks run on two waves at once
      auto zkey_at = [&](int pos) -> uint32_t { return (uint32_t)(S.kkey[S.kord[pos]] >> 32); };
      uint64_t ckey = 0;  // the last kept id's sort key
      int qc = -1, pd = -1;
      if (nuc) {
        // sorted position p of the row is kept iff its exclusive prefix <= limit
        const uint64_t A1 = (uint64_t)(S.md[1] * kFix);
        const double pl = g.topp > 0.0f ? (double)g.topp * (double)Zfx : 0.0;
        uint64_t limit = (uint64_t)pl;
        if (limit >= Zfx) limit = Zfx - 1;
        int lo = 0, hi = N1;  // the first dropped position
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (A1 + (mid > 0 ? S.kcum[mid - 1] : 0ull) <= limit) lo = mid + 1; else hi = mid;
        }
        // the cut must fall inside the list: something kept, something dropped
        if (lo == 0 || A1 + S.kcum[N1 - 1] <= limit) return 6;
        qc = lo - 1;
        ckey = S.kkey[S.kord[qc]];
        vkey = (uint32_t)(ckey >> 32);
        // the ids at the cut's z are contiguous around qc
        int f0 = 0, f1 = qc;  // the first position with z key <= vkey
        while (f0 < f1) {
          const int mid = (f0 + f1) >> 1;
          if (zkey_at(mid) <= vkey) f1 = mid; else f0 = mid + 1;
        }
        int l0 = qc + 1, l1 = N1;  // the first position with z key < vkey
        while (l0 < l1) {
          const int mid = (l0 + l1) >> 1;
          if (zkey_at(mid) < vkey) l1 = mid; else l0 = mid + 1;
        }
        const uint32_t ea = (uint32_t)(l0 - f0), ek = (uint32_t)(qc + 1 - f0);
        n_tie = ek == ea ? kNoTie : ek;
        if (n_tie != kNoTie) tie_lim = (int)(0xFFFFFFFFu - (uint32_t)ckey);
        Zkept = A1 + S.kcum[qc];
        kept_n = (int32_t)((uint32_t)S.mi[19] + (uint32_t)lo);
        ties = n_tie == kNoTie ? -1 : (int32_t)n_tie;
        cut = key2f(vkey);
      } else {
        kept_n = -1;  // filled below when asked
      }
      if (want2) {
        const uint64_t A2 = (uint64_t)(S.md[2] * kFix);
        uint64_t target = (uint64_t)((double)u * (double)Zkept);
        if (target >= Zkept) target = Zkept - 1;
        const uint64_t b2 = N1 > 0 ? S.kcum[N1 - 1] : 0ull;
        int lo = 0, hi = N2;  // the first position whose inclusive prefix passes the target
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (A2 + (S.kcum[N1 + mid] - b2) <= target) lo = mid + 1; else hi = mid;
        }
        if (lo == N2 || target < A2) return 9;
        pd = lo;
      }
      if (wv == 0 && nuc) {  // the cut's collision group lies inside region 1 in every chunk
        const bool ok = group_inside(S.cx[S.lslot[S.kord[qc]]], lo1, hi1);
        if (lane == 0) S.mi[12] = ok ? 1 : 0;
      }
      if (wv == 1 && want2) {  // the drawn id's group inside region 2
        const bool ok = group_inside(S.cx[S.lslot[S.kord[N1 + pd]]], lo2, hi2);
        if (lane == 0) S.mi[14] = ok ? 1 : 0;
      }
      __syncthreads();
      if (nuc && !S.mi[12]) return 8;
      if (want2) {
        if (!S.mi[14]) return 11;
        const uint64_t dkey = S.kkey[S.kord[N1 + pd]];
        token = (int64_t)(0xFFFFFFFFu - (uint32_t)dkey);
        chosen_z = key2f((uint32_t)(dkey >> 32));
        // the drawn id must be kept
        if (nuc && dkey < ckey) return 12;
      }
      RG_STAMP(29);
    } else if (nuc) {
      // ---- the cut: exact mass select over the region-1 candidates ----
      const uint64_t A1 = (uint64_t)(S.md[1] * kFix);
      const double pl = g.topp > 0.0f ? (double)g.topp * (double)Zfx : 0.0;
      uint64_t limit = (uint64_t)pl;
      if (limit >= Zfx) limit = Zfx - 1;
      auto in1 = [&](int e) -> bool { return present(e) && (cf[e] & 1u); };
      const MassSel ms = sel_mass(ck, cm, in1, A1, limit, S);
      RG_STAMP(27);
      if (!ms.ok || ms.ceq == 0) return 6;
      vkey = ms.key;
      // ids tied at the cut key weigh the same: the kept ones are the lowest
      // indices while their exclusive prefix stays <= limit
      const uint64_t m1 = ms.meq / ms.ceq;
      uint64_t nt = m1 ? (limit - ms.above) / m1 + 1 : (uint64_t)ms.ceq;
      if (nt > ms.ceq) nt = ms.ceq;
      n_tie = nt >= ms.ceq ? kNoTie : (uint32_t)nt;
      if (n_tie != kNoTie) tie_lim = kth_index(in1, vkey, n_tie);
      Zkept = ms.above + (uint64_t)nt * m1;
      // the cut's collision group must lie inside region 1 in every chunk
      if (tid == 0) S.mi[11] = -1;
      __syncthreads();
#pragma unroll
      for (int e = 0; e < FPT; e++)
        if (in1(e) && ck[e] == vkey) S.mi[11] = e * NT + tid;
      __syncthreads();
      if (wv == 0) {
        const bool ok = S.mi[11] >= 0 && group_inside(S.cx[S.mi[11]], lo1, hi1);
        if (lane == 0) S.mi[12] = ok ? 1 : 0;
      }
      uint32_t ngt = 0;
#pragma unroll
      for (int e = 0; e < FPT; e++) ngt += (in1(e) && ck[e] > vkey) ? 1u : 0u;
      ngt = bred(ngt, S.u, OpAdd{});
      if (!S.mi[12]) return 8;
      kept_n = (int32_t)((uint32_t)S.mi[19] + ngt + (uint32_t)nt);
      ties = n_tie == kNoTie ? -1 : (int32_t)n_tie;
      cut = key2f(vkey);
      __syncthreads();
    } else {
      kept_n = -1;  // filled below when asked
    }
    // ---- the draw: exact mass select over the region-2 candidates ----
    if (NL > KEPT && want2) {
      const uint64_t A2 = (uint64_t)(S.md[2] * kFix);
      uint64_t target = (uint64_t)((double)u * (double)Zkept);
      if (target >= Zkept) target = Zkept - 1;
      auto in2 = [&](int e) -> bool { return present(e) && (cf[e] & 2u); };
      RG_STAMP(28);
      const MassSel ds = sel_mass(ck, cm, in2, A2, target, S);
      RG_STAMP(29);
      if (!ds.ok || ds.ceq == 0) return 9;
      // the tie holding the target, lowest index first (ties weigh the same)
      const uint64_t m2 = ds.meq / ds.ceq;
      uint64_t jt = m2 ? (target - ds.above) / m2 : 0;
      if (jt >= ds.ceq) jt = ds.ceq - 1;
      token = kth_index(in2, ds.key, (uint32_t)jt + 1u);
      // one candidate of the drawn key, for its logit and collision group
      if (tid == 0) S.mi[13] = -1;
      __syncthreads();
#pragma unroll
      for (int e = 0; e < FPT; e++)
        if (in2(e) && ck[e] == ds.key) S.mi[13] = e * NT + tid;
      __syncthreads();
      if (wv == 0) {
        const bool ok = S.mi[13] >= 0 && group_inside(S.cx[S.mi[13]], lo2, hi2);
        if (lane == 0) S.mi[14] = ok ? 1 : 0;
      }
      __syncthreads();
      if (!S.mi[14]) return 11;
      chosen_z = key2f(ds.key);
      // the drawn id must be kept
      if (nuc && (ds.key < vkey || (ds.key == vkey && n_tie != kNoTie && token > tie_lim))) return 12;
    }
    if (!nuc && P.kept_count) {
      // every finite logit is kept: count the -inf ones (a pass over the row)
      uint32_t ninf = 0;
      const int nvec = F.nvec;
      for (int v = tid; v < nvec; v += NT) {
        float xx[VPE > 1 ? VPE : 1];
        loadv<DT, VPE>(row, (int64_t)v * VPE, xx);
        const uint8_t* am = row_allowed(P, r);
#pragma unroll
        for (int e = 0; e < VPE; e++) ninf += (xx[e] == -INFINITY || !id_allowed(am, (int64_t)v * VPE + e)) ? 1u : 0u;
      }
      ninf = bred(ninf, S.u2, OpAdd{});
      kept_n = V - (int)ninf;
      __syncthreads();
    }
    if (P.query_prob && qtok >= 0) {
      const float xq = penal_logit<DT>(P, g, row, r, (int)qtok, S);
      const float zq = __fdiv_rn(xq, T);
      const uint32_t kq = f2key(zq);
      const bool kept = zq != -INFINITY && (!nuc || kq > vkey || (kq == vkey && (n_tie == kNoTie || qtok <= tie_lim)));
      if (kept) qprob = (float)((double)zmass_fix(zq, Rref) / (double)Zkept);
    }
  }
  if (P.skip_draw && !greedy) token = -1;

  // ---- outputs ----
  if (P.chosen_logprob && tid == 0) {
    float lp = NAN;
    if (token >= 0 && Zfull > 0.0 && chosen_z == chosen_z) lp = (float)((double)chosen_z - lnZ);
    P.chosen_logprob[r] = lp;
  }
  if (g.ntop > 0 && status == 0) {
    for (int q = tid; q < P.n_top; q += NT) {
      if (q < ntop_out) {
        const uint64_t kk = S.kkey[S.kord[q]];
        P.top_logprobs[(int64_t)r * P.n_top + q] = (float)((double)key2f((uint32_t)(kk >> 32)) - lnZ);
        if (P.top_ids) P.top_ids[(int64_t)r * P.n_top + q] = (int64_t)(0xFFFFFFFFu - (uint32_t)kk);
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
  (void)zmax;
  return 0;
}

// ===========================================================================
// The kernel: grid of ceil(R / 8) * 8 * G workgroups of NT threads.
// ===========================================================================
template <int DT, int VPE, int NE>
__global__ __launch_bounds__(NT) void rowgroup_kernel(RgParams F) {
  __shared__ RgShared<NE> SU;
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  int r = (slot / F.G) * 8 + xcd;
  const int j = slot % F.G;
  if (r >= F.k.R) return;
  if (F.heavy_first) r = heavy_first_row(F.k, r);
  const int mode = chunk_phase<DT, VPE, NE>(F, SU.c, r, j);
  if (mode == MODE_DEFER) {
    if (j == 0 && threadIdx.x == 0) F.status[r] = LPS_ROW_DEFERRED | (1 << 8);
    return;
  }
  // arrival: the chunk's stores are visible at agent scope before it is counted
  release_agent();
  __syncthreads();
  if (threadIdx.x == 0) {
    release_count();
    SU.c.mi[7] = add_agent(F.counters + (int64_t)r * 32, 1u) + 1u == (uint32_t)F.G ? 1 : 0;
    if (SU.c.mi[7]) acquire_one();
  }
  __syncthreads();
  if (!SU.c.mi[7]) return;
  acquire_agent();
  RG_STAMP(24);
  const int reason = final_phase<DT, VPE>(F, SU.f, r);
  RG_STAMP(31);
  if (reason > 0 && threadIdx.x == 0) F.status[r] = LPS_ROW_DEFERRED | (reason << 8);
}

}  // namespace rg
}  // namespace lps
