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
template <int DT, int VPE, int NE, bool XF>
__device__ __forceinline__ int chunk_phase(const RgParams& F, RgChunkS<NE>& S, const int r, const int j,
                                           const RowCfg& g, const uint32_t epoch, int& tcase) {
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
  const int32_t* hrow0 = P.history ? P.history + (int64_t)r * P.history_stride : nullptr;
  const int hid = (hrow0 && (int64_t)tid < P.history_stride) ? hrow0[tid] : -1;
  CK C;
  C.load(row, v0, nv);
  C.mask(row_allowed(P, r), v0, nv);
  if (g.mode == MODE_DEFER) return MODE_DEFER;
  const int mode = g.mode;
  const bool greedy = g.greedy;
  const float T = g.T;
  const float c = g.c;
  uint32_t flags = 0;

  // ---- penalties ----
  if (g.pen) {
    if (!build_counts<NE>(S, g.hrow, g.hlen, tid < g.hlen ? hid : -1, v0 * VPE, nv * VPE)) flags |= RF_HISTORY;
    apply_counts(C, S.a.hc, nv, g.rep, g.pres, g.freq);
  }

  RG_STAMP(1);
  // ---- thread and chunk max (NaN ignored here; each mode finds NaN its own way) ----
  float tm = -INFINITY;
#pragma unroll
  for (int s = 0; s < NE; s++) tm = fmaxf(tm, C.x[s]);
  // pure rows without a draw (query probabilities, entropy) need only the
  // row mass: no histogram, barrier or candidates
  const bool zonly = XF && mode == MODE_PURE && row_skips_draw(P, r);
  const bool hist_mode = (mode == MODE_NUCLEUS || mode == MODE_PURE) && !zonly;
  if (hist_mode) {  // clear the histogram before the barrier of the max
    u32x4* h4 = reinterpret_cast<u32x4*>(S.a.hist);
#pragma unroll
    for (int i = 0; i < HB * 8 / 16 / NT; i++) h4[i * NT + tid] = u32x4{0u, 0u, 0u, 0u};
  }
  const float M = bred(tm, S.f, OpMax{});
  if (hist_mode) {  // the second level's bins (over the counts, read until that barrier)
    static_assert(FHN * 8 / 16 == NT, "one store per thread");
    reinterpret_cast<u32x4*>(S.fh)[tid] = u32x4{0u, 0u, 0u, 0u};
  }
  const bool Mfin = M != INFINITY && M != -INFINITY;
  const float ref = Mfin ? ceilf(__fmul_rn(M, c)) : (M == INFINITY ? INFINITY : -INFINITY);

  RG_STAMP(2);
  RgSum sm{};
  sm.mkey = f2key(M);
  sm.amax = 0x7FFFFFFF;
  sm.ref = ref;
  sm.tag = rg_tag(epoch, r, xcc_id());
  sm.reg[0] = sm.reg[1] = sm.reg[2] = sm.reg[3] = 1 << 30;
  // this chunk's published lists
  uint4* cbase = F.cands + (int64_t)r * CAPR + (int64_t)j * F.capw;
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
      RG_STAMP(12);
      if (!greedy && th > kNegInfKey + 1u && th != 0xFFFFFFFFu) th = f2key(collision_lo(key2f(th), T));
      // -inf is never a candidate (it has no mass); NaN always is (!(x < t))
      const float xth = fmaxf(key2f(th), -3.40282347e38f);
      uint32_t n = 0;
#pragma unroll
      for (int s = 0; s < NE; s++) seg_put(S.l, 0, !(C.x[s] < xth), n, C.x[s], CK::index(v0, s));
      seg_done(S.l, 0, n);
      __syncthreads();
      RG_STAMP(13);
      int np[2];
      if (!sort_publish(S.l, S, 1, g.kprime, greedy, T, cbase, F.capw, np)) flags |= RF_OVERFLOW;
      sm.n1 = (uint16_t)np[0];
    }
  }

  if (zonly) {
    // ---- the chunk mass: exp2(fma(x, c, -ref)), fp32 per vector, fp64 across;
    // a NaN logit is counted as the histogram's NaN bin would ----
    double zs = 0.0, zh = 0.0;
    uint32_t nanc = 0;
    if (Mfin) {
#pragma unroll
      for (int i = 0; i < CK::NV; i++) {
        float a = 0.0f, ah = 0.0f;
#pragma unroll
        for (int e = 0; e < VPE; e++) {
          const float x = C.x[i * VPE + e];
          const float t = __builtin_fmaf(x, c, -ref);
          const float m = __builtin_amdgcn_exp2f(t);
          nanc += x != x ? 1u : 0u;
          a += x != x ? 0.0f : m;
          if constexpr (XF) ah += m > 0.0f && x == x ? m * t : 0.0f;
        }
        zs += (double)a;
        zh += (double)ah;
      }
    } else {
#pragma unroll
      for (int s = 0; s < NE; s++) nanc += C.x[s] != C.x[s] ? 1u : 0u;
    }
    sm.zsum = bred(zs, S.d, OpAdd{});
    sm.nanbin = bred(nanc, S.u, OpAdd{});
    if constexpr (XF) sm.zent = bred(zh, S.d3, OpAdd{});
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
        atomicAdd(&S.a.hist[b != BELOW ? b : (uint32_t)(HB + lane)],
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
        const unsigned long long a = S.a.hist[b];
        double m = bin_mass_u(b, a);
        if (b == HB_NAN) { nanc = (uint32_t)(a >> 48); m = 0.0; }
        zs += m;
        hout[b] = (float)m;
      }
      if (XF && g.bigk) {
        // large top-k rows: the bins' counts too, one byte each (255: 255 or
        // more), in the second level's area, which these rows do not use
        static_assert(FHN * 4 == HPUB, "one byte per published bin");
        uint8_t* cout = reinterpret_cast<uint8_t*>(F.fine + ((int64_t)r * G + j) * FHN);
#pragma unroll
        for (int i = 0; i < HLT; i++) {
          const int b = tid + NT * i;
          cout[b] = (uint8_t)min((uint32_t)(S.a.hist[b] >> 48), 255u);
        }
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
    // typical-p without top-p / min-p: the typical filter proper (a threshold
    // cut from the row's entropy), unless the row holds -inf
    const bool tpl = XF && g.typp < 1.0f && !(g.topp < 1.0f) && !(g.minp > 0.0f) && !g.bigk;
    if (XF && (P.entropy || tpl)) {
      // the chunk's sum of e * log2(e), fp32 per vector, fp64 across
      double zh = 0.0;
      if (Mfin) {
#pragma unroll
        for (int i = 0; i < CK::NV; i++) {
          float a = 0.0f;
#pragma unroll
          for (int e = 0; e < VPE; e++) {
            const float t = __builtin_fmaf(C.x[i * VPE + e], c, -ref);
            const float m = __builtin_amdgcn_exp2f(t);
            a += m > 0.0f ? m * t : 0.0f;
          }
          zh += (double)a;
        }
      }
      sm.zent = bred(zh, S.d3, OpAdd{});
    }
    if (XF && __builtin_expect(g.typp < 1.0f, 0) && Mfin) {
      // typical-p rows (kept: the argmax, when a filter removed ids): the
      // chunk's first id whose z equals its maximum's, fl(x / T) == fl(M / T)
      const float xlo = collision_lo(M, T);
      int best = 0x7FFFFFFF;
      if (tm >= xlo) {
#pragma unroll
        for (int s = 0; s < NE; s++)
          if (C.x[s] >= xlo) best = min(best, CK::index(v0, s));
      }
      sm.amax = bred(best, S.i1, OpMin{});
    }
    if (__builtin_expect(tpl, 0)) {
      // (over the chunk's nv vectors: its slots past them hold -inf too)
      uint32_t ni = 0;
      float mn = INFINITY;
#pragma unroll
      for (int q = 0; q < NE / VPE; q++) {
        uint32_t nq = 0;
        float mq = INFINITY;
#pragma unroll
        for (int e = 0; e < VPE; e++) {
          nq += C.x[q * VPE + e] == -INFINITY ? 1u : 0u;
          mq = fminf(mq, C.x[q * VPE + e]);
        }
        const bool inr = tid + q * NT < nv;  // (vector q of this thread)
        ni += inr ? nq : 0u;
        mn = inr ? fminf(mn, mq) : mn;
      }
      const uint32_t nis = bred(ni, S.u2, OpAdd{});
      sm.ab1 = tw_pack(nis, f2key(bred(mn, S.f, OpMin{})));
    }
    // ---- publish the summary and the bins, one barrier among the row's chunks ----
    if (tid == 0) store_sum(sums + j, sm);
    RG_STAMP(4);
    release_agent();
    __syncthreads();
    if (tid == 0) {
      release_count();
      add_agent(ctr + CTR_HIST, 1u);
      S.mi[6] = wait_count(ctr + CTR_HIST, (uint32_t)G) ? 0 : 1;
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
      const uint32_t mk = XF ? wmax(lane < G ? a.mkey : 0u) : 0u;
      // (typical rows: sum e log2 e against R, summed as the finaliser does; -inf count)
      const double ah = tpl ? wsum(af ? sc * (a.zent - (double)(R - a.ref) * a.zsum) : 0.0) : 0.0;
      const uint32_t ni = tpl ? wsum(lane < G ? tw_n(a.ab1) : 0u) : 0u;
      const uint32_t mn = tpl ? wmin(lane < G ? tw_key(a.ab1) : 0xFFFFFFFFu) : 0u;
      if (lane < G) { S.rf[lane] = af ? a.ref : -INFINITY; }
      if (lane == 0) {
        S.md[0] = Z;
        S.mf[0] = R;
        if constexpr (XF) {
          S.mi[8] = (int)mk;
          S.md[1] = ah;
          S.mi[9] = (int)ni;
          S.mi[4] = (int)mn;
        }
      }
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
          const int dl = (rw != -INFINITY) ? (int)fminf(R - rw, 4096.0f) : 4096;
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
    // region bounds, and the cumulative mass at each end of region 1, are
    // collected with LDS atomics by the few threads whose bins meet a target
    // (cleared here, before the scan's barrier); the masses are non-negative
    // doubles, whose bit patterns order as they do
    if (tid == 0) {
      S.mi[0] = 1 << 30; S.mi[1] = -1; S.mi[2] = 1 << 30; S.mi[3] = -1;
      S.u3[0] = 0u;
      S.mq[0] = ~0ull;
      S.mq[1] = 0ull;
      S.mq[2] = ~0ull;
    }
    double stot;
    const double sx = bscan<NW, double>(msum, &stot, S.d2);
    // ---- regions: bins whose cumulative interval meets the targets ----
    const double eps = 1e-6 * Z;
    // large top-k rows: the row bin of the k-th largest logit (kb), from the
    // chunks' byte counts merged like the masses; a count of 255 at or above
    // it (inexact), or a k past the binned logits, defers the row
    int kb = -1;
    if (XF && __builtin_expect(g.bigk, 0)) {
      if (tid == 0) S.mi[7] = -1;
      uint32_t cnt[HPT];
      uint32_t satm = 0u;  // bit i: bin i's count saturated in some chunk
#pragma unroll
      for (int i = 0; i < HPT; i++) cnt[i] = 0u;
      if (rfin) {
        for (int w = 0; w < G; w++) {
          const float rw = S.rf[w];
          if (rw == -INFINITY) continue;
          const int dw = (int)fminf(R - rw, 4096.0f);
          const int src = HPUB - HPT - HPT * tid + HOCT * dw;
          if (src > HPUB - HPT) continue;
          const uint64_t v = ld_pub(reinterpret_cast<const uint64_t*>(
              reinterpret_cast<const uint8_t*>(F.fine + ((int64_t)r * G + w) * FHN) + src));
#pragma unroll
          for (int i = 0; i < HPT; i++) {
            // (byte HPT - 1 - i is row bin HB - 1 - HPT tid - i; the chunk's NaN bin is left out)
            const uint32_t cc = (i == 0 && src == HPUB - HPT) ? 0u : (uint32_t)(v >> (8 * (HPT - 1 - i))) & 0xFFu;
            cnt[i] += cc;
            satm |= cc == 255u ? 1u << i : 0u;
          }
        }
      }
      if (tid == 0) cnt[0] = 0u;  // row bin HB - 1: NaN only
      uint32_t cs = 0u;
#pragma unroll
      for (int i = 0; i < HPT; i++) cs += cnt[i];
      uint32_t ctot;
      uint32_t ca = bscan<NW, uint32_t>(cs, &ctot, S.u2);
      const uint32_t kk = (uint32_t)g.topk;
      int hs = -1;  // this thread's highest saturated bin
#pragma unroll
      for (int i = 0; i < HPT; i++) {
        const int b = HB - 1 - HPT * tid - i;
        if (ca < kk && ca + cnt[i] >= kk) S.mi[7] = b;
        if ((satm >> i) & 1u) hs = max(hs, b);
        ca += cnt[i];
      }
      hs = bred(hs, S.i2, OpMax{});
      kb = S.mi[7];
      if (kb < 0 || hs >= kb) flags |= RF_REGION;
    }
    // threshold cuts (min-p; typical-p on a full row): the bins that can hold
    // the boundary [lom, him], and up to the lowest non-empty bin above them
    // (which holds the least kept id when every id of [lom, him] is dropped):
    // hm.  A typical row holding -inf, or whose cut keeps nothing, keeps only
    // the argmax (targ: no regions, no candidates); one whose cut keeps its
    // least logit keeps every logit, a pure row (tall)
    bool tc = XF && mode == MODE_NUCLEUS && (g.minp > 0.0f || g.bigk) && rfin;
    bool targ = false, tall = false;
    int lom = 0, him = -1, hm = -1;
    double lowtw = 0.0;  // (a typical cut under the histogram: the chunk's dropped logits, least kept key)
    if (XF && __builtin_expect(tpl && rfin, 0)) {
      const float xmx = key2f((uint32_t)S.mi[8]);
      const double dmin = typical_dmin(Z, S.md[1], R, xmx, c, g.typp);
      tcase = typical_case((uint32_t)S.mi[9], dmin, key2f((uint32_t)S.mi[4]), xmx, T, c, R, lom, him);
      targ = tcase == TYP_ARGMAX;
      tall = tcase == TYP_ALL || tcase == TYP_LOW;
      tc = tcase == TYP_CUT;
      if (tcase == TYP_WIDE) flags |= RF_REGION;
      if (tcase == TYP_LOW) {
        // the least logit the cut keeps (first_key_where: z - zmax >= dmin is
        // non-decreasing in x), then this chunk's dropped logits and least kept one
        const float zmx = __fdiv_rn(xmx, T);
        const float xt = key2f(first_key_where([&](float x) { return (double)__fsub_rn(__fdiv_rn(x, T), zmx) >= dmin; }));
        uint32_t nd = 0;
        float mk = INFINITY;
#pragma unroll
        for (int s = 0; s < NE; s++) {
          const bool inr = tid + (s / VPE) * NT < nv;
          nd += inr && C.x[s] < xt ? 1u : 0u;
          mk = inr && C.x[s] >= xt ? fminf(mk, C.x[s]) : mk;
        }
        const uint32_t nds = bred(nd, S.u2, OpAdd{});
        lowtw = tw_pack(nds, f2key(bred(mk, S.f, OpMin{})));
      }
    }
    const bool nuc = mode == MODE_NUCLEUS && !tall;
    const bool topp_on = nuc && (!XF || g.topp < 1.0f);  // (without XF every nucleus row has top-p)
    const double Pm = topp_on ? (g.topp > 0.0f ? (double)g.topp * Z : 0.0) : Z;
    if (XF && g.bigk) {
      lom = him = hm = kb;  // (the k-th largest lies in bin kb)
    } else if (__builtin_expect(tc, 0)) {
      if (!tpl && !cut_bins(g.minp, key2f((uint32_t)S.mi[8]), c, R, lom, him)) flags |= RF_REGION;
      int bp = 1 << 30;
#pragma unroll
      for (int i = 0; i < HPT; i++) {
        const int b = HB - 1 - HPT * tid - i;
        if (b > him && b < HB_NAN && mrg[i] > 0.0) bp = min(bp, b);
      }
      bp = bred(bp, S.i2, OpMin{});
      hm = bp < (1 << 30) ? bp : him;
    }
    if (nuc) {
      // region 1: its highest bin holds the least prefix a, its lowest the
      // largest end a + m (cumulative mass at its top and bottom: the kept
      // mass lies between them, and the draw at u times it)
      int lo = 1 << 30, hi = -1;
      uint64_t atop = ~0ull, abot = 0ull;
      double a = sx;
#pragma unroll
      for (int i = 0; i < HPT; i++) {
        const int b = HB - 1 - HPT * tid - i;
        if (topp_on && mrg[i] > 0.0 && a <= Pm + eps && a + mrg[i] >= Pm - eps) {
          lo = min(lo, b);
          hi = max(hi, b);
          atop = min(atop, __builtin_bit_cast(uint64_t, a));
          abot = max(abot, __builtin_bit_cast(uint64_t, a + mrg[i]));
        }
        // (threshold cuts: the cumulative mass at the top of bin hm and the bottom of bin lom)
        if (tc && b == hm) S.mq[5] = __builtin_bit_cast(uint64_t, a);
        if (tc && b == lom) S.mq[6] = __builtin_bit_cast(uint64_t, a + mrg[i]);
        a += mrg[i];
      }
      if (hi >= 0) {
        atomicMin(&S.mi[0], lo);
        atomicMax(&S.mi[1], hi);
        atomicMin(reinterpret_cast<unsigned long long*>(&S.mq[0]), (unsigned long long)atop);
        atomicMax(reinterpret_cast<unsigned long long*>(&S.mq[1]), (unsigned long long)abot);
      }
    }
    __syncthreads();
    int lo1 = nuc ? S.mi[0] : (1 << 30);
    int hi1 = nuc ? S.mi[1] : (1 << 30);
    uint64_t q1t = S.mq[0], q1b = S.mq[1];
    if (topp_on && hi1 < 0) flags |= RF_REGION;
    if (__builtin_expect(tc, 0)) {
      // the top-p cut entirely above [lom, hm]: top-p alone decides (every id
      // it keeps passes min-p); entirely under it (or no top-p): the threshold
      // alone; else region 1 covers both
      const double mt = __builtin_bit_cast(double, S.mq[5]), mb = __builtin_bit_cast(double, S.mq[6]);
      if (!topp_on || mb < Pm - eps) {
        lo1 = lom; hi1 = hm; q1t = S.mq[5]; q1b = S.mq[6];
      } else if (!(mt > Pm + eps) && hi1 >= 0) {
        lo1 = min(lo1, lom); hi1 = max(hi1, hm);
        q1t = min(q1t, S.mq[5]); q1b = max(q1b, S.mq[6]);
      }
    }
    if (XF && targ) lo1 = hi1 = 1 << 30;
    const float u = fminf(fmaxf(g.u == g.u ? g.u : 0.0f, 0.0f), 0.99999994f);
    double t_lo = (nuc ? (double)u * __builtin_bit_cast(double, q1t) : (double)u * Z) - eps;
    double t_hi = (nuc ? (double)u * __builtin_bit_cast(double, q1b) : (double)u * Z) + eps;
    if (XF && targ) { t_lo = -1.0; t_hi = -2.0; }  // (no draw region)
    {
      int lo = 1 << 30, hi = -1;
      uint32_t nest = 0;  // elements in either region (an upper estimate: bin mass / the bin's least mass)
      uint64_t a2 = ~0ull;  // cumulative mass at region 2's top
      double a = sx;
#pragma unroll
      for (int i = 0; i < HPT; i++) {
        const int b = HB - 1 - HPT * tid - i;
        const bool in2 = mrg[i] > 0.0 && a <= t_hi && a + mrg[i] >= t_lo;
        if (in2) {
          lo = min(lo, b);
          hi = max(hi, b);
          a2 = min(a2, __builtin_bit_cast(uint64_t, a));
        }
        if (in2 || (b >= lo1 && b <= hi1))
          nest += (uint32_t)ceilf(__fmul_rn((float)mrg[i], ldexpf(1.0f, 134 - ((b >> 7) + HE0))) /
                                  (float)(128 + (b & 127)));
        a += mrg[i];
      }
      if (hi >= 0) {
        atomicMin(&S.mi[2], lo);
        atomicMax(&S.mi[3], hi);
        atomicMin(reinterpret_cast<unsigned long long*>(&S.mq[2]), (unsigned long long)a2);
      }
      if (nest) atomicAdd(&S.u3[0], nest);
    }
    __syncthreads();
    const int lo2 = S.mi[2];
    const int hi2 = S.mi[3];
    const uint32_t nest = S.u3[0];
    if (!(XF && targ) && (hi2 < 0 || !rfin)) flags |= RF_REGION;
    const bool need2 = !row_skips_draw(P, r);
    // ---- crowded regions take the second level (a row-uniform decision: every
    // chunk merged the same bins; a chunk whose first barrier timed out is
    // deferred, and counts itself at the second barrier without waiting) ----
    // (past 3/4 of the row's lists, so that no chunk's share passes its own
    // list, or half of what the chunks' wave segments take)
    const bool crowded = __builtin_expect(nest > (uint32_t)min(CAPR * 3 / 4, G * CLMAX / 2), 0);
    const bool refine = crowded && !tc && !S.mi[6] && rfin && (!nuc || (hi1 >= 0 && hi1 - lo1 < RW)) &&
                        (!need2 || (hi2 >= 0 && hi2 - lo2 < RW));
    if (crowded && !refine) flags |= RF_WIDE;
    if (S.mi[6] && tid == 0) add_agent(ctr + CTR_FINE, 1u);
    // the regions in row bins (empty: 1 << 30), and in this chunk's bins
    // (its reference is dl octaves under the row's)
    constexpr int NOB = 1 << 30;
    const int cr[4] = {nuc ? lo1 : NOB, nuc ? hi1 : NOB, hi2 >= 0 ? lo2 : NOB, hi2 >= 0 ? hi2 : NOB};
    const int dl = Mfin && rfin ? (int)fminf(R - ref, 4096.0f) : 0;
    auto own = [&](int b) { return b >= NOB ? b : b + HOCT * dl; };
    const int l1 = own(cr[0]), h1 = own(cr[1]), l2 = own(cr[2]), h2 = own(cr[3]);
    uint32_t L1, C1, L2, C2;
    region_pair(l1, h1, L1, C1);
    region_pair(l2, h2, L2, C2);
    if (!Mfin) C1 = 0u;
    if (!Mfin || !need2) C2 = 0u;
    // published regions: row fine bins (whole bins unless refined)
    int fr[4];
#pragma unroll
    for (int q = 0; q < 4; q++) fr[q] = cr[q] >= NOB ? NOB : cr[q] * FSUB + ((q & 1) ? FSUB - 1 : 0);
    // refined rows: this chunk's fine bounds of each region (for the candidate
    // test) and the exact masses above them inside the region bins
    int cf[4] = {0, -1, 0, -1};
    float xr[4] = {0.0f, -1.0f, 0.0f, -1.0f};  // refined rows: the fine regions as ranges of logits
    double fab1 = 0.0, fab2 = 0.0;
    uint32_t fnab = 0;
    if (__builtin_expect(refine, 0)) {
      // slot p of region q holds the fine bin F0 - p of its top bin (mass descending)
      const int F0a = cr[1] < NOB ? (h1 + 1) * FSUB - 1 : -1, F0b = need2 ? (h2 + 1) * FSUB - 1 : -1;
      // (1) this chunk's fine bins of the region bins (the masses recomputed as binned)
#pragma unroll
      for (int k = 0; k < NE / 2; k++) {
        const uint32_t t1 = in_region2(bins[k], L1, C1), t2 = in_region2(bins[k], L2, C2);
        if (__builtin_amdgcn_ballot_w64((t1 | t2) != 0u) == 0ull) continue;
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const bool o1 = (t1 >> (16 * h) & 0xFFFFu) != 0u, o2 = (t2 >> (16 * h) & 0xFFFFu) != 0u;
          if (o1 || o2) {
            const float e = emass(C.x[2 * k + h], c, ref);
            const int f = efine(e);
            const unsigned long long add = (1ull << 48) | (unsigned long long)(__float_as_uint(e) & 0xFFu);
            if (o1) atomicAdd(&S.fh[F0a - f], add);
            if (o2) atomicAdd(&S.fh[RW * FSUB + F0b - f], add);
          }
        }
      }
      __syncthreads();
      RG_STAMP(17);
      // (2) publish them as fp32 masses (thread t: slots 2t, 2t + 1), one
      // barrier among the row's chunks, merge (rescaled, in chunk order)
      static_assert(FHN == 2 * NT, "two fine bins per thread");
      const bool q2 = tid >= NT / 2;
      const int p0 = 2 * (tid & (NT / 2 - 1));
      const int f0 = q2 ? F0b : F0a;
      const unsigned long long acc0 = S.fh[2 * tid], acc1 = S.fh[2 * tid + 1];
      *reinterpret_cast<float2*>(F.fine + ((int64_t)r * G + j) * FHN + 2 * tid) =
          make_float2((float)fine_mass(f0 - p0, acc0), (float)fine_mass(f0 - p0 - 1, acc1));
      release_agent();
      __syncthreads();
      if (tid == 0) {
        release_count();
        add_agent(ctr + CTR_FINE, 1u);
        S.mi[6] = wait_count(ctr + CTR_FINE, (uint32_t)G) ? 0 : 1;
        acquire_one();
      }
      __syncthreads();
      acquire_agent();
      RG_STAMP(18);
      if (S.mi[6]) flags |= RF_REGION;
      double fm[2] = {0.0, 0.0};
      for (int w0 = 0; w0 < G; w0 += 4) {
        float2 v[4];
        double sw[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int w = w0 + q;
          const float rw = w < G ? S.rf[w] : -INFINITY;
          const int dw = rw != -INFINITY ? (int)fminf(R - rw, 4096.0f) : 4096;
          sw[q] = dw < 1024 ? ldexp(1.0, -dw) : 0.0;
          v[q] = w < G ? ld_pub(reinterpret_cast<const float2*>(F.fine + ((int64_t)r * G + w) * FHN + 2 * tid))
                       : make_float2(0.0f, 0.0f);
        }
#pragma unroll
        for (int q = 0; q < 4; q++) {
          fm[0] += (double)v[q].x * sw[q];
          fm[1] += (double)v[q].y * sw[q];
        }
      }
      // (3) the fine regions: region 1's fine bins meeting the cut, then region
      // 2's meeting the draw (u times the kept mass, bounded by region 1's);
      // cumulative masses from each region's top (exclusive scan per half)
      const double ms = fm[0] + fm[1];
      const double inc = wscan_incl(ms);
      if (lane == 63) S.d3[wv] = inc;
      if (tid == 0) {
        S.mi[10] = NOB; S.mi[11] = -1; S.mi[13] = NOB; S.mi[15] = -1;
        S.mq[3] = ~0ull;
        S.mq[4] = 0ull;
      }
      __syncthreads();
      double a = inc - ms;
#pragma unroll
      for (int i = 0; i < NW; i++) a += (i < wv && (i >= NW / 2) == q2) ? S.d3[i] : 0.0;
      if (!q2 && nuc) {
        a += __builtin_bit_cast(double, S.mq[0]);
        int lo = NOB, hi = -1;
        uint64_t at = ~0ull, ab = 0ull;
#pragma unroll
        for (int i = 0; i < 2; i++) {
          if (fm[i] > 0.0 && a <= Pm + eps && a + fm[i] >= Pm - eps) {
            lo = min(lo, p0 + i);
            hi = max(hi, p0 + i);
            at = min(at, __builtin_bit_cast(uint64_t, a));
            ab = max(ab, __builtin_bit_cast(uint64_t, a + fm[i]));
          }
          a += fm[i];
        }
        if (hi >= 0) {
          atomicMin(&S.mi[10], lo);
          atomicMax(&S.mi[11], hi);
          atomicMin(reinterpret_cast<unsigned long long*>(&S.mq[3]), (unsigned long long)at);
          atomicMax(reinterpret_cast<unsigned long long*>(&S.mq[4]), (unsigned long long)ab);
        }
      }
      __syncthreads();
      if (q2 && need2) {
        a += __builtin_bit_cast(double, S.mq[2]);
        const double tl = (nuc ? (double)u * __builtin_bit_cast(double, S.mq[3]) : (double)u * Z) - eps;
        const double th = (nuc ? (double)u * __builtin_bit_cast(double, S.mq[4]) : (double)u * Z) + eps;
        int lo = NOB, hi = -1;
#pragma unroll
        for (int i = 0; i < 2; i++) {
          if (fm[i] > 0.0 && a <= th && a + fm[i] >= tl) {
            lo = min(lo, p0 + i);
            hi = max(hi, p0 + i);
          }
          a += fm[i];
        }
        if (hi >= 0) {
          atomicMin(&S.mi[13], lo);
          atomicMax(&S.mi[15], hi);
        }
      }
      __syncthreads();
      RG_STAMP(21);
      const int fp[4] = {S.mi[10], S.mi[11], S.mi[13], S.mi[15]};
      if ((nuc && fp[1] < 0) || (need2 && fp[3] < 0)) flags |= RF_REGION;
      if (nuc) {
        cf[0] = F0a - fp[1]; cf[1] = F0a - fp[0];
        fr[0] = (cr[1] + 1) * FSUB - 1 - fp[1]; fr[1] = (cr[1] + 1) * FSUB - 1 - fp[0];
      }
      if (need2) {
        cf[2] = F0b - fp[3]; cf[3] = F0b - fp[2];
        fr[2] = (cr[3] + 1) * FSUB - 1 - fp[3]; fr[3] = (cr[3] + 1) * FSUB - 1 - fp[2];
      }
      // (4) this chunk's exact mass (and count) above each fine region inside its region bins
      const unsigned long long acc[2] = {acc0, acc1};
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const int p = p0 + i;
        if (!q2 && nuc && p < fp[0]) { fab1 += fine_mass(F0a - p, acc[i]); fnab += (uint32_t)(acc[i] >> 48); }
        if (q2 && need2 && p < fp[2]) fab2 += fine_mass(F0b - p, acc[i]);
      }
      // (5) the fine regions as ranges of logits [first key reaching the low
      // bound, first key past the high bound - 1]: wave w < 4 finds bound w
      if (wv < 4) {
        const int thr = wv == 0 ? cf[0] : wv == 1 ? cf[1] + 1 : wv == 2 ? cf[2] : cf[3] + 1;
        const uint32_t k = first_key_reaching(thr, c, ref);
        if (lane == 0) S.i3[wv] = (int32_t)k;
      }
      __syncthreads();
      xr[0] = key2f((uint32_t)S.i3[0]);
      xr[1] = key2f((uint32_t)S.i3[1] - 1u);
      xr[2] = key2f((uint32_t)S.i3[2]);
      xr[3] = key2f((uint32_t)S.i3[3] - 1u);
      if (!nuc || !Mfin) { xr[0] = 0.0f; xr[1] = -1.0f; }
      if (!need2 || !Mfin) { xr[2] = 0.0f; xr[3] = -1.0f; }
    }
    sm.reg[0] = fr[0];
    sm.reg[1] = fr[1];
    sm.reg[2] = fr[2];
    sm.reg[3] = fr[3];

    RG_STAMP(6);
    // ---- this chunk: candidates in either region, exact masses above them ----
    {
      // (per-wave sums, added up by the publishing thread after the barriers
      // of the candidate lists; the lists do not overlap the histogram)
      double ab1 = fab1, ab2 = fab2;
      uint32_t nab = fnab;
#pragma unroll
      for (int i = 0; i < HLT; i++) {
        const int b = tid + NT * i;
        const unsigned long long a = S.a.hist[b];
        const double m = b == HB_NAN ? 0.0 : bin_mass_u(b, a);
        if (b > h1 && b != HB_NAN) { ab1 += m; nab += (uint32_t)(a >> 48); }
        if (b > h2) ab2 += m;
      }
      RG_STAMP(11);
      ab1 = wreduce(ab1, OpAdd{});
      ab2 = wreduce(ab2, OpAdd{});
      nab = wreduce(nab, OpAdd{});
      if (lane == 0) { S.d4[wv] = ab1; S.d5[wv] = ab2; S.u4[wv] = nab; }
    }
    // the elements of either region: list 0 (region 1, nucleus rows) and
    // list 1 (region 2, unless the draw is skipped), tested on bin pairs
    // (refined rows: on their ranges of logits)
    static_assert(NE % 2 == 0, "bin pairs");
    uint32_t n1 = 0, n2 = 0;
    if (__builtin_expect(refine, 0)) {
#pragma unroll
      for (int k = 0; k < NE / 2; k++) {
        bool o[2][2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const float x = C.x[2 * k + h];
          o[h][0] = x >= xr[0] && x <= xr[1];
          o[h][1] = x >= xr[2] && x <= xr[3];
        }
        if (__builtin_amdgcn_ballot_w64(o[0][0] || o[0][1] || o[1][0] || o[1][1]) == 0ull) continue;
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const int s2 = 2 * k + h;
          seg_put(S.l, 0, o[h][0], n1, C.x[s2], CK::index(v0, s2));
          seg_put(S.l, 1, o[h][1], n2, C.x[s2], CK::index(v0, s2));
        }
      }
    } else {
#pragma unroll
      for (int k = 0; k < NE / 2; k++) {
        const uint32_t t1 = in_region2(bins[k], L1, C1), t2 = in_region2(bins[k], L2, C2);
        if (__builtin_amdgcn_ballot_w64((t1 | t2) != 0u) == 0ull) continue;
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const int s2 = 2 * k + h;
          seg_put(S.l, 0, (t1 >> (16 * h) & 0xFFFFu) != 0u, n1, C.x[s2], CK::index(v0, s2));
          seg_put(S.l, 1, (t2 >> (16 * h) & 0xFFFFu) != 0u, n2, C.x[s2], CK::index(v0, s2));
        }
      }
    }
    seg_done(S.l, 0, n1);
    seg_done(S.l, 1, n2);
    __syncthreads();
    RG_STAMP(13);
    int np[2];
    if (!sort_publish(S.l, S, 2, 0, false, T, cbase, F.capw, np)) flags |= RF_OVERFLOW;
    sm.n1 = (uint16_t)np[0];
    sm.n2 = (uint16_t)np[1];
    sm.ab1 = 0.0; sm.ab2 = 0.0; sm.nab1 = 0;
#pragma unroll
    for (int i = 0; i < NW; i++) { sm.ab1 += S.d4[i]; sm.ab2 += S.d5[i]; sm.nab1 += S.u4[i]; }
    if (XF && tcase == TYP_LOW) sm.ab1 = lowtw;  // (no region 1)
  }

  // ---- the chunk's summary, then the arrival count ----
  RG_STAMP(7);
  sm.flags = flags;
  if (tid == 0) store_sum(sums + MAXG + j, sm);
  return mode;
}

// Penalised logit of one id (legality bit, history count), computed by the
// finaliser's FT threads.
template <int DT>
__device__ __forceinline__ float penal_logit(const KParams& P, const RowCfg& g, const char* row, int r, int id, RgX& S) {
  uint32_t c = 0;
  if (g.pen)
    for (int k = threadIdx.x; k < g.hlen; k += FT) c += g.hrow[k] == id ? 1u : 0u;
  c = bred<FW>(c, S.u2, OpAdd{});
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
// First position in [lo, hi) where pred holds, for a predicate that is false
// then true over the range (hi when it never holds), found by one wave with
// ballots: 64 blocks per level, two levels for ranges up to 4096.  Every lane
// of the wave calls it with the same arguments; no barrier.
template <class Pr>
__device__ __forceinline__ int wave_first_true(int lo, int hi, Pr pred) {
  const int lane = threadIdx.x & 63;
  int n = hi - lo;
  if (n <= 0) return hi;
  if (n > 64) {
    // lane i tests the last position of block i (blocks of bs)
    const int bs = (n + 63) >> 6;
    const int q = min(lo + (lane + 1) * bs, hi) - 1;
    const uint64_t m = __builtin_amdgcn_ballot_w64(pred(q));
    if (!m) return hi;
    const int b = (int)__builtin_ctzll(m);
    const int nlo = lo + b * bs;
    hi = min(lo + (b + 1) * bs, hi);  // pred(hi - 1) holds
    lo = nlo;
    n = hi - lo;
  }
  const uint64_t m = __builtin_amdgcn_ballot_w64(lane < n && pred(lo + lane));
  return m ? lo + (int)__builtin_ctzll(m) : hi;
}
// Exclusive prefix over the finaliser's FT threads in thread order of two
// values at once (one barrier); t0 / t1 get the totals.
__device__ __forceinline__ void bscan2(uint64_t v0, uint64_t v1, uint64_t& e0, uint64_t& e1, uint64_t& t0, uint64_t& t1,
                                       uint64_t* s0, uint64_t* s1) {
  const uint64_t i0 = wscan_incl(v0), i1 = wscan_incl(v1);
  if (lane_id() == 63) { s0[wave_id()] = i0; s1[wave_id()] = i1; }
  __syncthreads();
  uint64_t o0 = 0, o1 = 0, a0 = 0, a1 = 0;
#pragma unroll
  for (int i = 0; i < FW; i++) {
    const uint64_t x0 = s0[i], x1 = s1[i];
    o0 += (i < wave_id()) ? x0 : 0ull;
    o1 += (i < wave_id()) ? x1 : 0ull;
    a0 += x0;
    a1 += x1;
  }
  e0 = o0 + i0 - v0;
  e1 = o1 + i1 - v1;
  t0 = a0;
  t1 = a1;
}
// Inclusive prefixes of the masses of merged lists 0 and 1 over positions
// [0, n0) and [0, n1): thread t holds positions KPT t .. KPT t + KPT - 1.
// Ends with a barrier.
__device__ __forceinline__ void scan_lists(RgFinalS& S, int n0, int n1) {
  uint64_t m0[KPT], m1[KPT], l0 = 0, l1 = 0;
#pragma unroll
  for (int i = 0; i < KPT; i++) {
    const int p = KPT * (int)threadIdx.x + i;
    m0[i] = p < n0 ? S.sm[0][p] : 0ull;
    m1[i] = p < n1 ? S.sm[1][p] : 0ull;
    l0 += m0[i];
    l1 += m1[i];
  }
  uint64_t e0, e1, t0, t1;
  bscan2(l0, l1, e0, e1, t0, t1, S.q, S.q2);
#pragma unroll
  for (int i = 0; i < KPT; i++) {
    const int p = KPT * (int)threadIdx.x + i;
    e0 += m0[i];
    e1 += m1[i];
    if (p < n0) S.sc[0][p] = e0;
    if (p < n1) S.sc[1][p] = e1;
  }
  __syncthreads();
}
// Merges the loaded lists (S.lk[l], chunk q's sorted list at [cb[q], cb[q] +
// cn[q])) into sorted order: entry f of list l (chunk c, position p) has rank
// p plus the entries above it in every other chunk's list, found by a
// binary search there (2^D bounds the lists' lengths).  The FT threads take
// the entries of both lists densely; the searches of one entry in the other
// chunks run in one loop, so their reads are issued together.  Each entry is
// written to its rank (ranks >= KM are dropped) with its logit and mass.
template <int MG>
__device__ __forceinline__ void merge_lists(RgFinalS& S, int G, int D, int N0, int N1, float Rm) {
  int cn[2][MG], cb[2][MG];
#pragma unroll
  for (int q = 0; q < MG; q++) {
    cn[0][q] = q < G ? S.cn[0][q] : 0;
    cn[1][q] = q < G ? S.cn[1][q] : 0;
    cb[0][q] = q < G ? S.cb[0][q] : 0;
    cb[1][q] = q < G ? S.cb[1][q] : 0;
  }
  for (int f = threadIdx.x; f < N0 + N1; f += FT) {
    const int l = f < N0 ? 0 : 1;
    const int fl = l ? f - N0 : f;
    // the entry's chunk: the last with cb <= fl
    int c = 0;
#pragma unroll
    for (int q = 1; q < MG; q++) c = (q < G && (l ? cb[1][q] : cb[0][q]) <= fl) ? q : c;
    const uint64_t key = S.lk[l][fl];
    int ps[MG];
#pragma unroll
    for (int q = 0; q < MG; q++) ps[q] = 0;
    for (int sb = D - 1; sb >= 0; sb--) {
      const int step = 1 << sb;
      uint64_t v[MG];
#pragma unroll
      for (int q = 0; q < MG; q++) {
        const int n = l ? cn[1][q] : cn[0][q], bq = l ? cb[1][q] : cb[0][q];
        v[q] = S.lk[l][bq + min(ps[q] + step, max(n, 1)) - 1];
      }
#pragma unroll
      for (int q = 0; q < MG; q++) {
        const int n = l ? cn[1][q] : cn[0][q];
        const int t = ps[q] + step;
        ps[q] = (q != c && t <= n && v[q] > key) ? t : ps[q];
      }
    }
    int rank = fl - (l ? cb[1][0] : cb[0][0]);
#pragma unroll
    for (int q = 1; q < MG; q++) rank = q == c ? fl - (l ? cb[1][q] : cb[0][q]) : rank;
#pragma unroll
    for (int q = 0; q < MG; q++) rank += ps[q];
    if (rank < KM) {
      S.sk[l][rank] = key;
      S.sx[l][rank] = S.lx[l][fl];
      S.sm[l][rank] = zmass_fix(key2f(key_z(key)), Rm);
    }
  }
}
__device__ __forceinline__ void merge_lists_g(RgFinalS& S, int G, int D, int N0, int N1, float Rm) {
  if (G <= 2) merge_lists<2>(S, G, D, N0, N1, Rm);
  else if (G <= 4) merge_lists<4>(S, G, D, N0, N1, Rm);
  else if (G <= 8) merge_lists<8>(S, G, D, N0, N1, Rm);
  else merge_lists<MAXG>(S, G, D, N0, N1, Rm);
}

// Counts, over the other 15 lanes of this lane's row of 16, the values greater
// than v (gt) and at least v (ge): row rotations by 1 .. 15, in either direction
// every other lane once.
template <int D>
__device__ __forceinline__ void row_rank16(uint32_t v, uint32_t& gt, uint32_t& ge) {
  const uint32_t o = dpp_t<0x120 + D>(v, v);  // row_ror:D
  gt += o > v ? 1u : 0u;
  ge += o >= v ? 1u : 0u;
  if constexpr (D < 15) row_rank16<D + 1>(v, gt, ge);
}

// Top-k rows: the merged list 0 without the merge.  Every chunk's list holds
// its logits from the top down.  If j chunks each hold m entries at or above
// z = t, and j m >= kc, the row's kc-th largest z is at least t: so for m =
// kc, kc/2, kc/4, kc/8 (rounded up) the j = ceil(kc / m)-th largest of the
// chunks' m-th entries bounds it from below, and the largest of the four
// bounds is kept.  The entries whose z reaches it (all the top-kc set, ties
// included: typically 1.2-2 kc entries) are compacted into list 1's storage,
// unused by top-k rows, then rank-sorted into sk[0] / sx[0] / sm[0].
// Returns their count, or -1 when more than KM are left (the caller merges
// instead).  FT threads; ends with a barrier.
__device__ __forceinline__ int select_topk_lists(RgFinalS& S, int G, int kc, int N1, float Rm) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  if (wv == 0) {
    // lanes 16 i + q: chunk q's m_i-th entry (0 when chunk q holds fewer than
    // m_i entries); the j_i-th largest of each row of 16 lanes is the value of
    // the lanes with fewer than j_i values above theirs and at least j_i at or
    // above
    const int grp = lane >> 4, q = lane & 15;
    const int m = (kc + (1 << grp) - 1) >> grp;
    const uint32_t jn = (uint32_t)((kc + m - 1) / m);
    uint32_t v = 0u;
    if (q < G && S.cn[0][q] >= m) v = key_z(S.lk[0][S.cb[0][q] + m - 1]);
    uint32_t gt = 0u, ge = 1u;
    row_rank16<1>(v, gt, ge);
    uint32_t t = (gt < jn && jn <= ge) ? v : 0u;
    t = wreduce(t, OpMax{});
    if (lane == 0) S.mi[26] = (int)t;
  }
  __syncthreads();
  RG_STAMP(22);
  const uint32_t zt = (uint32_t)S.mi[26];
  // compaction (in any order: the rank sort below fixes it)
  constexpr int EPT = LKM / FT;
  uint64_t kk[EPT];
  uint32_t xx[EPT];
  uint32_t keep = 0;
#pragma unroll
  for (int i = 0; i < EPT; i++) {
    const int f = i * FT + tid;
    kk[i] = f < N1 ? S.lk[0][f] : 0ull;
    xx[i] = f < N1 ? S.lx[0][f] : 0u;
    keep += (f < N1 && key_z(kk[i]) >= zt) ? 1u : 0u;
  }
  uint32_t tot;
  uint32_t pos = bscan<FW>(keep, &tot, S.u3);
  const int n = (int)tot;
  if (n > KM) {
    __syncthreads();
    return -1;
  }
#pragma unroll
  for (int i = 0; i < EPT; i++) {
    const int f = i * FT + tid;
    if (f < N1 && key_z(kk[i]) >= zt) {
      S.sk[1][pos] = kk[i];
      S.sx[1][pos] = xx[i];
      pos++;
    }
  }
  __syncthreads();
  RG_STAMP(23);
  // rank sort (keys are distinct: the index is in the low word): each wave
  // ranks 64 entries at a time, against 64 keys per register load, read back
  // lane by lane
  for (int e0 = wv * 64; e0 < n; e0 += FT) {
    const int e = e0 + lane;
    const uint64_t key = e < n ? S.sk[1][e] : 0ull;
    uint32_t rank = 0;
    for (int j0 = 0; j0 < n; j0 += 64) {
      const uint64_t kj = j0 + lane < n ? S.sk[1][j0 + lane] : 0ull;  // 0 ranks below every key
      const uint32_t hi = (uint32_t)(kj >> 32), lo = (uint32_t)kj;
#pragma unroll
      for (int l = 0; l < 64; l++) {
        const uint64_t a = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(hi, l) << 32) |
                           (uint64_t)(uint32_t)__builtin_amdgcn_readlane(lo, l);
        rank += a > key ? 1u : 0u;
      }
    }
    if (e < n) {
      S.sk[0][rank] = key;
      S.sx[0][rank] = S.sx[1][e];
      S.sm[0][rank] = zmass_fix(key2f(key_z(key)), Rm);
    }
  }
  __syncthreads();
  return n;
}

// Inclusive prefix of masses m[0, n) into c[0, n) over FT threads (KPT
// positions per thread, n <= KM).  Ends with a barrier.
__device__ __forceinline__ void scan_one(const uint64_t* m, uint64_t* c, int n, uint64_t* slot) {
  uint64_t v[KPT], loc = 0;
#pragma unroll
  for (int i = 0; i < KPT; i++) {
    const int p = KPT * (int)threadIdx.x + i;
    v[i] = p < n ? m[p] : 0ull;
    loc += v[i];
  }
  uint64_t tot;
  uint64_t ex = bscan<FW>(loc, &tot, slot);
#pragma unroll
  for (int i = 0; i < KPT; i++) {
    const int p = KPT * (int)threadIdx.x + i;
    ex += v[i];
    if (p < n) c[p] = ex;
  }
  __syncthreads();
}

// Outcome of a sampling row decided on its sorted candidates.
struct Decision {
  int64_t token = -1;
  float cut = -INFINITY, qprob = 0.0f, chosen_z = NAN;
  int32_t pos = -1;  // sorted position of the drawn candidate (-1: greedy)
  int32_t ties = -1, kept_n = 0;
  int ntop_out = 0;
  int status = 0;
};

// The top-k row's filters and draw (sampling.py:66-85, 149-238) on its
// sorted candidates: sk[0, K) in sorted order (z descending, ties lower index
// first), sm their fixed-point masses, sc scratch for the prefix; K < Ntot
// when candidates past capacity exist.  Greedy rows take the argmax gam.
// Runs on the FT threads; returns 0, or a reason code to defer the row.
__device__ __forceinline__ int topk_decide(const RowCfg& g, int V, const uint64_t* sk, const uint64_t* sm, uint64_t* sc,
                                           int K, int Ntot, float u, int gam, float xmax, RgX& X, Decision& d) {
  const int tid = threadIdx.x;
  const int64_t qtok = g.qtok;
  d.ntop_out = g.ntop < K ? g.ntop : K;
  if (g.mode == MODE_GREEDY) {
    d.token = gam;
    d.cut = xmax;
    d.ties = 1;
    d.kept_n = 1;
    d.qprob = (qtok >= 0 && qtok == gam) ? 1.0f : 0.0f;
    d.chosen_z = xmax;
    return 0;
  }
  const int keff = g.topk < V ? g.topk : V;
  if (keff > K || keff <= 0) return 5;
  // the top-k set: every position whose z reaches the keff-th (ties kept)
  const uint32_t kk = key_z(sk[keff - 1]);
  const int nk = wave_first_true(keff, K, [&](int p) { return key_z(sk[p]) < kk; });
  if (nk == K && K < Ntot) return 4;  // ties past the capacity
  scan_one(sm, sc, nk, X.q);
  const uint64_t Zk = sc[nk - 1];
  int nf = nk;
  if (g.topp < 1.0f) {  // keep sorted position p iff p == 0 or cum[p-1] <= top_p * Zk
    const double pl = g.topp > 0.0f ? (double)g.topp * (double)Zk : 0.0;
    uint64_t limit = (uint64_t)pl;
    if (limit >= Zk) limit = Zk - 1;
    nf = wave_first_true(1, nk, [&](int p) { return sc[p - 1] > limit; });
  }
  if (g.minp > 0.0f) {  // keep mass >= min_p * (the top mass)
    const float e0 = (float)((double)sm[0] / kFix);
    int first = 0x7FFFFFFF;
#pragma unroll
    for (int i = 0; i < KPT; i++) {
      const int p = KPT * tid + i;
      if (p < nf && (float)((double)sm[p] / kFix) < __fmul_rn(g.minp, e0)) first = min(first, p);
    }
    const int f = bred<FW>(first, X.i2, OpMin{});
    if (f < nf) nf = f;
    if (nf == 0) d.status |= LPS_ROW_EMPTY;
  }
  // typical-p with top-k active: the row then holds -inf, and the reference keeps only the argmax
  if (d.status == 0 && g.typp < 1.0f) nf = 1;
  if (d.status != 0) return 0;
  const uint64_t Zf = sc[nf - 1];
  const uint32_t ckey = key_z(sk[nf - 1]);
  d.cut = key2f(ckey);
  // ids tied with the last kept one: contiguous around it
  const int f0 = wave_first_true(0, nf, [&](int p) { return key_z(sk[p]) <= ckey; });
  const int l0 = wave_first_true(nf, K, [&](int p) { return key_z(sk[p]) < ckey; });
  if (l0 == K && K < Ntot) return 4;
  d.ties = (l0 - f0) == (nf - f0) ? -1 : (int32_t)(nf - f0);
  d.kept_n = nf;
  // inverse CDF in sorted order
  uint64_t target = (uint64_t)((double)u * (double)Zf);
  if (target >= Zf) target = Zf - 1;
  const int ps = wave_first_true(0, nf, [&](int p) { return sc[p] > target; });
  d.token = key_index(sk[ps]);
  d.chosen_z = key2f(key_z(sk[ps]));
  d.pos = ps;
  if (qtok >= 0) {
    if (tid == 0) X.mi[5] = -1;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < KPT; i++) {
      const int p = KPT * tid + i;
      if (p < nf && key_index(sk[p]) == qtok) X.mi[5] = p;
    }
    __syncthreads();
    if (X.mi[5] >= 0) d.qprob = (float)((double)sm[X.mi[5]] / (double)Zf);
  }
  return 0;
}

template <int DT, int VPE, bool XF>
__device__ __forceinline__ int final_phase(const RgParams& F, RgFinalS& S, const int r, const RowCfg& g,
                                           const uint32_t epoch, const int tcase) {
  const KParams& P = F.k;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int G = F.G;
  const int V = P.V;
  const char* row = row_ptr<DT>(P, r);
  const RgSum* sums = F.sums + (int64_t)r * 2 * MAXG + MAXG;
  const uint4* cands = F.cands + (int64_t)r * CAPR;
  if (tid == 0) {  // the row's counters back to zero for the next launch, which has the next epoch
    F.counters[(int64_t)r * 32 + CTR_ARRIVE] = 0u;
    F.counters[(int64_t)r * 32 + CTR_HIST] = 0u;
    F.counters[(int64_t)r * 32 + CTR_FINE] = 0u;
    F.counters[(int64_t)r * 32 + CTR_EPOCH] = epoch + 1u;
  }
  const int mode = g.mode;
  const bool greedy = g.greedy;
  const float T = g.T;
  const float c = g.c;
  const int capw = F.capw;

  // ---- first pass of the lists, loaded before their lengths are known (in
  // flight with the summaries): entry i < K0 of chunk c is flat entry
  // f = c K0 + i, held by thread f % FT in slot f / FT (slots < FP1) ----
  const int lgK = 31 - __builtin_clz((FP1 * FT) / G);
  const int K0 = 1 << lgK;
  uint4 cv[FPT];
#pragma unroll
  for (int e = 0; e < FP1; e++) {
    const int f = e * FT + tid, c0 = f >> lgK;
    cv[e] = c0 < G ? ld_pub(cands + c0 * capw + (f & (K0 - 1))) : make_uint4(0u, 0u, 0u, 0u);
  }
#pragma unroll
  for (int e = FP1; e < FPT; e++) cv[e] = make_uint4(0u, 0u, 0u, 0u);

  // ---- F1: the chunk summaries (wave 0; lane q < G holds chunk q's).  The
  // chunks are combined with reductions and prefix sums over the first 16
  // lanes (G <= 16), all independent of each other; the row mass is summed in
  // the same order as the chunks' own (wsum) ----
  if (wv == 0) {
    RgSum a{};
    if (lane < G) a = ld_pub(sums + lane);
    RG_STAMP_DEP(19, a.mkey);
    const bool in = lane < G;
    const bool rfin = in && a.ref != INFINITY && a.ref != -INFINITY;
    const int c1 = in ? (int)a.n1 : 0, c2 = in ? (int)a.n2 : 0;
    const int co = c1 + c2 > K0 ? c1 + c2 - K0 : 0;
    uint32_t fl = rreduce16(in ? a.flags : 0u, OpOr{});
    // every summary is this launch's and was written on this XCD (whose L2
    // then holds everything the chunk published), else the row is deferred
    const uint32_t stale = rreduce16((in && a.tag != rg_tag(epoch, r, xcc_id())) ? 1u : 0u, OpOr{});
    const uint32_t mk = rreduce16(in ? a.mkey : 0u, OpMax{});
    const float R = rreduce16(rfin ? a.ref : -INFINITY, OpMax{});
    const uint32_t nab = rreduce16(in ? a.nab1 : 0u, OpAdd{});
    const uint32_t nanb = rreduce16(in ? a.nanbin : 0u, OpMax{});
    const int nmax = rreduce16(max(c1, c2), OpMax{});
    const int i1 = rscan16(c1), i2 = rscan16(c2), io = rscan16(co);
    // this lane's prefixes (chunks before it) and the totals (lanes >= G add 0)
    const int n1b = i1 - c1, n2b = i2 - c2, ob = io - co;
    const int n1t = rdlane(i1, 15), n2t = rdlane(i2, 15), ot = rdlane(io, 15);
    if (stale) fl |= RF_SPLIT;
    RG_STAMP_DEP(20, fl);
    // (typical-p nucleus rows: the first id at the row's maximum z, over the
    // chunks whose maximum has that z)
    const bool tz = XF && mode == MODE_NUCLEUS && g.typp < 1.0f;
    const float zr = tz ? __fdiv_rn(key2f(mk), T) : 0.0f;
    const bool amc = tz ? __fdiv_rn(key2f(a.mkey), T) == zr : a.mkey == mk;
    const int am = rreduce16(in && amc ? (int)a.amax : 0x7FFFFFFF, OpMin{});
    const double sc = rfin ? ldexp(1.0, (int)(a.ref - R)) : 0.0;
    const double Z = rreduce16(rfin ? a.zsum * sc : 0.0, OpAdd{});
    const double A1 = rreduce16(rfin ? a.ab1 * sc : 0.0, OpAdd{});
    const double A2 = rreduce16(rfin ? a.ab2 * sc : 0.0, OpAdd{});
    // entropy rows: sum of e ln e over the row, against the row reference
    // (a chunk dl octaves under it: e 2^-dl, log2 e - dl), in log2 units
    // (and typical rows without top-p / min-p, with their -inf count)
    const bool tpl = XF && mode == MODE_NUCLEUS && g.typp < 1.0f && !(g.topp < 1.0f) && !(g.minp > 0.0f) && !g.bigk;
    const double AH = (XF && (P.entropy || tpl)) ? rreduce16(rfin ? sc * (a.zent - (double)(R - a.ref) * a.zsum) : 0.0, OpAdd{}) : 0.0;
    // (a typical cut under the histogram: the dropped logits and the least kept key)
    const bool low = tcase == TYP_LOW;
    const uint32_t ndr = low ? rreduce16(in ? tw_n(a.ab1) : 0u, OpAdd{}) : 0u;
    const uint32_t mkp = low ? rreduce16(in ? tw_key(a.ab1) : 0xFFFFFFFFu, OpMin{}) : 0u;
    if (lane < G) {
      S.cn[0][lane] = (int)a.n1;
      S.cn[1][lane] = (int)a.n2;
      S.cb[0][lane] = n1b;
      S.cb[1][lane] = n2b;
      S.opre[lane] = ob;
      S.rf[lane] = (a.ref != INFINITY && a.ref != -INFINITY) ? a.ref : -INFINITY;
      S.rm[lane] = a.mkey == 0xFFFFFFFFu ? INFINITY : key2f(a.mkey);
    }
    if (lane == 0) {
      S.cb[0][G] = n1t;
      S.cb[1][G] = n2t;
      S.opre[G] = ot;
      S.mi[16] = (int)fl;
      S.mi[17] = (int)mk;
      S.mi[18] = am;
      S.mi[19] = (int)nab;
      S.mi[20] = (int)nanb;
      S.mi[21] = a.reg[0]; S.mi[22] = a.reg[1]; S.mi[23] = a.reg[2]; S.mi[24] = a.reg[3];
      S.mi[25] = nmax;
      S.md[0] = Z; S.md[1] = A1; S.md[2] = A2; S.md[3] = AH;
      S.mi[29] = (int)ndr;
      S.mi[31] = (int)mkp;
      S.mf[0] = R;
    }
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
  const bool hmode = mode == MODE_NUCLEUS || mode == MODE_PURE;
  // the row's mass reference (logprob, nucleus and pure rows published theirs)
  const float Rref = (hmode || S.mf[0] != -INFINITY)
                         ? S.mf[0]
                         : (xmax != INFINITY && xmax != -INFINITY ? ceilf(__fmul_rn(xmax, c)) : 0.0f);
  // masses of merged entries: against the row reference (nucleus, pure) or the
  // row maximum (top-k)
  const float Rm = hmode ? Rref : (xmax != INFINITY && xmax != -INFINITY ? ceilf(__fmul_rn(xmax, c)) : 0.0f);
  const double Zfull = S.md[0];
  float u = g.u;
  if (!(u >= 0.0f)) u = 0.0f;
  if (u >= 1.0f) u = 0.99999994f;
  const int N1 = S.cb[0][G], N2 = S.cb[1][G], NO = S.opre[G];
  if (N1 > LKM || N2 > LKM || NO > (FPT - FP1) * FT) return 13;
  const int D = 32 - __builtin_clz((uint32_t)max(S.mi[25], 1));

  // ---- the entries: slots e < FP1 the first pass, slots e >= FP1 the rest
  // (entry o = (e - FP1) FT + tid of the row's overflow: chunk c with
  // opre[c] <= o < opre[c + 1], index K0 + o - opre[c]) ----
  {
    int ci[FPT], ii[FPT];
#pragma unroll
    for (int e = 0; e < FPT; e++) {
      ci[e] = -1;
      ii[e] = 0;
    }
#pragma unroll
    for (int e = 0; e < FP1; e++) {
      const int f = e * FT + tid;
      const int cc = f >> lgK, i = f & (K0 - 1);
      const int ccc = min(cc, G - 1);
      const bool pr = cc < G && i < S.cn[0][ccc] + S.cn[1][ccc];
      ci[e] = pr ? cc : -1;
      ii[e] = i;
    }
    if (NO > 0) {
#pragma unroll
      for (int e = FP1; e < FPT; e++) {
        const int o = (e - FP1) * FT + tid;
        if (o < NO) {
          int cc = 0;
          for (int q = 1; q < G; q++) cc = S.opre[q] <= o ? q : cc;
          ci[e] = cc;
          ii[e] = K0 + o - S.opre[cc];
          cv[e] = ld_pub(cands + cc * capw + ii[e]);
        }
      }
    }
#pragma unroll
    for (int e = 0; e < FPT; e++) {
      if (ci[e] < 0) continue;
      const int cc = ci[e], i = ii[e];
      const int n1c = S.cn[0][cc];
      const int l = i < n1c ? 0 : 1;
      const int p = l ? i - n1c : i;
      const uint64_t key = ((uint64_t)cv[e].x << 32) | (uint64_t)(0xFFFFFFFFu - cv[e].y);
      S.lk[l][S.cb[l][cc] + p] = key;
      S.lx[l][S.cb[l][cc] + p] = cv[e].z;
      const float xv = __uint_as_float(cv[e].z);
      if (xv != xv) status |= LPS_ROW_NONFINITE;
    }
  }
  status = bred<FW>(status, S.i1, OpOr{});
  RG_STAMP(26);
  if (greedy) status = 0;

  // ---- merge the chunks' sorted lists (top-k rows: select, then sort) ----
  RG_STAMP(16);
  int K = min(N1, KM);  // merged positions of list 0 present
  int Ntot = N1;
  const int nsel = (g.kprime > 0 && N2 == 0) ? select_topk_lists(S, G, g.kprime, N1, Rm) : -1;
  if (nsel >= 0) {
    K = Ntot = nsel;
  } else {
    merge_lists_g(S, G, D, N1, N2, Rm);
    __syncthreads();
  }
  RG_STAMP(27);

  int64_t token = -1;
  float cut = -INFINITY, qprob = 0.0f, chosen_z = NAN;
  float chosen_x = NAN;  // the drawn logit (regions' draws): its mass in Z's arithmetic
  int32_t ties = -1, kept_n = 0;
  int ntop_out = 0;
  const int64_t qtok = g.qtok;

  if (status == 0 && g.kprime > 0) {
    // ======================= top-k (and top-N logprobs) =======================
    Decision d;
    const int rc = topk_decide(g, V, S.sk[0], S.sm[0], S.sc[0], K, Ntot, u, gam, xmax, S, d);
    if (rc) return rc;
    token = d.token; cut = d.cut; qprob = d.qprob; chosen_z = d.chosen_z;
    chosen_x = greedy ? xmax : (d.pos >= 0 ? __uint_as_float(S.sx[0][d.pos]) : NAN);
    ties = d.ties; kept_n = d.kept_n; ntop_out = d.ntop_out; status |= d.status;
  } else if (status == 0 && mode == MODE_GREEDY) {
    token = gam;
    cut = xmax;
    ties = 1;
    kept_n = 1;
    qprob = (qtok >= 0 && qtok == gam) ? 1.0f : 0.0f;
    chosen_z = xmax;
  } else if (status == 0 && hmode) {
    // ======================= nucleus / pure =======================
    const double Z = S.md[0];
    // typical-p without top-p / min-p (sampling.py:207-238): the threshold
    // z - zmax >= dmin from the row's entropy; a row holding -inf (NaN
    // entropy) or whose threshold keeps nothing keeps only the argmax (targ),
    // one whose threshold keeps its least logit keeps every logit (tall: a
    // pure row); the chunks decided the same
    const bool tpl = XF && mode == MODE_NUCLEUS && g.typp < 1.0f && !(g.topp < 1.0f) && !(g.minp > 0.0f) && !g.bigk;
    // (the case every chunk decided from the same summaries: this workgroup's own)
    const double dmin = tpl ? typical_dmin(Z, S.md[3], Rref, xmax, c, g.typp) : 0.0;
    if (tpl && (tcase < TYP_ARGMAX || tcase > TYP_LOW)) return 6;
    bool targ = tcase == TYP_ARGMAX;  // typical-p row keeping only its argmax
    const bool tall = tcase == TYP_ALL || tcase == TYP_LOW;
    const bool nuc = mode == MODE_NUCLEUS && !tall;
    const bool want2 = !row_skips_draw(P, r);
    const int lo1 = S.mi[21], hi1 = S.mi[22], lo2 = S.mi[23], hi2 = S.mi[24];
    const uint64_t Zfx = (uint64_t)(Z * kFix);
    if ((nuc && N1 > KM) || (want2 && N2 > KM)) return 7;
    uint32_t vkey = 0, n_tie = kNoTie;
    uint64_t Zkept = Zfx;
    int tie_lim = 0x7FFFFFFF;  // kept ids at the cut key: index <= tie_lim
    // whether every id whose z equals fl(x / T) lies inside the row's fine
    // bins [lo, hi] (a region) under the binning of each chunk that can hold
    // it (one wave; lane w checks chunk w)
    auto group_inside = [&](float x, int lo, int hi) -> bool {
      const Group gr = collision_group(x, T);
      bool bad = false;
      if (lane < G) {
        const float rw = S.rf[lane], mw = S.rm[lane];
        if (rw != -INFINITY && !(gr.lo > mw)) {  // some id of this chunk may reach the group
          const int sh = HOCT * FSUB * (int)fminf(Rref - rw, 4096.0f);
          const int el = efine(emass(gr.lo, c, rw)), eh = efine(emass(fminf(gr.hi, mw), c, rw));
          const int bl = (el < 0 ? -(1 << 28) : el) - sh;
          const int bh = (eh < 0 ? -(1 << 28) : min(eh, HB_NAN * FSUB - 1)) - sh;
          bad = !(bl >= lo && bh <= hi);
        }
      }
      return gr.ok != 0 && __builtin_amdgcn_ballot_w64(bad) == 0ull;
    };
    scan_lists(S, nuc ? N1 : 0, want2 ? N2 : 0);
    RG_STAMP(28);
    uint64_t ckey = 0;  // the last kept id's sort key
    int qc = -1, pd = -1;
    if (nuc && !targ) {
      // sorted position p of the row is kept iff its exclusive prefix <= limit
      const uint64_t A1 = (uint64_t)(S.md[1] * kFix);
      const double pl = g.topp > 0.0f ? (double)g.topp * (double)Zfx : 0.0;
      uint64_t limit = (uint64_t)pl;
      if (limit >= Zfx) limit = Zfx - 1;
      // the first dropped position
      const bool tp = !XF || g.topp < 1.0f;
      int lo = tp ? wave_first_true(0, N1, [&](int p) { return A1 + (p > 0 ? S.sc[0][p - 1] : 0ull) > limit; }) : N1;
      bool mcut = false;  // region 1 holds the whole boundary range of a threshold cut
      if (XF && __builtin_expect(g.bigk, 0)) {
        // top-k past the lists (sampling.py:139-156): every z at or above the
        // k-th largest, which is list 0's entry k - (ids above region 1)
        const int kk = g.topk - S.mi[19];
        if (kk < 1 || kk > N1) return 6;
        const uint32_t zk = key_z(S.sk[0][kk - 1]);
        lo = wave_first_true(kk, N1, [&](int p) { return key_z(S.sk[0][p]) < zk; });
        mcut = true;  // (every id under region 1 is under the k-th largest)
      } else if (XF && __builtin_expect(g.minp > 0.0f || tpl, 0)) {
        // min-p after top-p (sampling.py:187-205): keep z with mass_f(z, zmax)
        // >= min_p; typical-p: keep z - zmax >= dmin.  Each a prefix of the
        // sorted order (exp2 is non-decreasing)
        const float zmax = __fdiv_rn(xmax, T);
        const int lm = wave_first_true(0, N1, [&](int p) {
          const float z = key2f(key_z(S.sk[0][p]));
          return tpl ? !((double)__fsub_rn(z, zmax) >= dmin) : !(mass_f(z, zmax) >= g.minp);
        });
        int bl, bh;
        mcut = cut_bins(tpl ? (float)exp(dmin) : g.minp, xmax, c, Rref, bl, bh) && lo1 <= bl * FSUB &&
               hi1 >= bh * FSUB + FSUB - 1;
        lo = min(lo, lm);
      }
      // the cut must fall inside the list: something kept, and the id after
      // the list dropped (min-p drops every id under region 1 when it holds
      // the boundary range)
      if (XF ? (lo == 0 || (lo == N1 && !mcut && (!tp || A1 + S.sc[0][N1 - 1] <= limit)))
             : (lo == 0 || A1 + S.sc[0][N1 - 1] <= limit))
        return 6;
      qc = lo - 1;
      ckey = S.sk[0][qc];
      vkey = key_z(ckey);
      // the ids at the cut's z are contiguous around qc
      const int f0 = wave_first_true(0, qc, [&](int p) { return key_z(S.sk[0][p]) <= vkey; });
      const int l0 = wave_first_true(qc + 1, N1, [&](int p) { return key_z(S.sk[0][p]) < vkey; });
      const uint32_t ea = (uint32_t)(l0 - f0), ekk = (uint32_t)(qc + 1 - f0);
      n_tie = ekk == ea ? kNoTie : ekk;
      if (n_tie != kNoTie) tie_lim = key_index(ckey);
      Zkept = A1 + S.sc[0][qc];
      kept_n = (int32_t)((uint32_t)S.mi[19] + (uint32_t)lo);
      ties = n_tie == kNoTie ? -1 : (int32_t)n_tie;
      cut = key2f(vkey);
      if (XF && __builtin_expect(g.typp < 1.0f && !tpl, 0)) {
        // typical-p after top-p / min-p (sampling.py:207-238): a row that lost
        // ids holds -inf, its entropy is NaN and only the argmax is kept; a
        // row that kept every id takes the typical filter proper
        if (kept_n >= V) return 14;
        targ = true;
      }
    } else if (XF && tall) {
      // every logit kept but those a cut under the histogram drops (the row holds no -inf)
      kept_n = V - (tcase == TYP_LOW ? S.mi[29] : 0);
      if (tcase == TYP_LOW) {
        const float zc = __fdiv_rn(key2f((uint32_t)S.mi[31]), T);
        vkey = f2key(zc);
        cut = zc;
      }
    } else {
      kept_n = -1;  // filled below when asked
    }
    if (want2 && !targ) {
      const uint64_t A2 = (uint64_t)(S.md[2] * kFix);
      uint64_t target = (uint64_t)((double)u * (double)Zkept);
      if (target >= Zkept) target = Zkept - 1;
      // the first position whose inclusive prefix passes the target
      const int lo = wave_first_true(0, N2, [&](int p) { return A2 + S.sc[1][p] > target; });
      if (lo == N2 || target < A2) return 9;
      pd = lo;
    }
    const bool cutd = nuc && (!XF || qc >= 0);  // (a typical row without a cut keeps its argmax)
    if (wv == 0 && cutd) {  // the cut's collision group lies inside region 1 in every chunk
      const bool ok = group_inside(__uint_as_float(S.sx[0][qc]), lo1, hi1);
      if (lane == 0) S.mi[12] = ok ? 1 : 0;
    }
    if (wv == 1 && want2 && !targ) {  // the drawn id's group inside region 2
      const bool ok = group_inside(__uint_as_float(S.sx[1][pd]), lo2, hi2);
      if (lane == 0) S.mi[14] = ok ? 1 : 0;
    }
    __syncthreads();
    if (cutd && !S.mi[12]) return 8;
    if (XF && __builtin_expect(targ, 0)) {
      // the argmax: the first id at the row's maximum z
      if (gam == 0x7FFFFFFF) return 14;
      const float zr = __fdiv_rn(xmax, T);
      vkey = f2key(zr);
      n_tie = 1;
      tie_lim = gam;
      Zkept = zmass_fix(zr, Rref);
      cut = zr;
      ties = 1;
      kept_n = 1;
      if (want2) {
        token = gam;
        chosen_z = zr;
        chosen_x = P.chosen_logprob ? penal_logit<DT>(P, g, row, r, gam, S) : NAN;
      }
    } else if (want2) {
      if (!S.mi[14]) return 11;
      const uint64_t dkey = S.sk[1][pd];
      token = (int64_t)key_index(dkey);
      chosen_z = key2f(key_z(dkey));
      chosen_x = __uint_as_float(S.sx[1][pd]);
      // the drawn id must be kept
      if (nuc && dkey < ckey) return 12;
    }
    RG_STAMP(29);
    if (!nuc && !(XF && tall) && P.kept_count) {
      // every finite logit is kept: count the -inf ones (a pass over the row)
      uint32_t ninf = 0;
      const int nvec = F.nvec;
      for (int v = tid; v < nvec; v += FT) {
        float xx[VPE > 1 ? VPE : 1];
        loadv<DT, VPE>(row, (int64_t)v * VPE, xx);
        const uint8_t* am = row_allowed(P, r);
#pragma unroll
        for (int e = 0; e < VPE; e++) ninf += (xx[e] == -INFINITY || !id_allowed(am, (int64_t)v * VPE + e)) ? 1u : 0u;
      }
      ninf = bred<FW>(ninf, S.u2, OpAdd{});
      kept_n = V - (int)ninf;
      __syncthreads();
    }
    if (P.query_prob && qtok >= 0) {
      const float xq = penal_logit<DT>(P, g, row, r, (int)qtok, S);
      const float zq = __fdiv_rn(xq, T);
      const uint32_t kq = f2key(zq);
      const bool kept = zq != -INFINITY && ((!nuc && tcase != TYP_LOW) || kq > vkey ||
                                            (kq == vkey && (n_tie == kNoTie || qtok <= tie_lim)));
      if (kept) qprob = (float)((double)zmass_fix(zq, Rref) / (double)Zkept);
    }
  }
  if (row_skips_draw(P, r) && !greedy) token = -1;

  // ---- outputs ----
  // ln of sum exp(z) over the row: Z is in units of 2^Rref of exp2(x c)
  double lnZ = 0.0;
  if ((P.chosen_logprob || g.ntop > 0) && wv == 0 && Zfull > 0.0) lnZ = log(Zfull) + (double)Rref * 0.6931471805599453;
  const double lZ = lnZ - (double)Rref * 0.6931471805599453;  // ln Zfull
  if (XF && P.entropy && tid == 0) {
    // H = ln Z - sum(e ln e) / Z (the general kernel's NaN for rows without finite statistics)
    const bool fin = !has_nan && xmax != INFINITY && xmax != -INFINITY && __fdiv_rn(xmax, T) != INFINITY && Zfull > 0.0;
    P.entropy[r] = fin ? (float)(log(Zfull) - 0.6931471805599453 * S.md[3] / Zfull) : NAN;
  }
  if (P.chosen_logprob && tid == 0) {
    float lp = NAN;
    if (token >= 0 && Zfull > 0.0 && chosen_x == chosen_x && chosen_x != INFINITY && chosen_x != -INFINITY) {
      // the drawn logit's mass computed as Z's are (exp2(x c) against Rref):
      // the ratio is then exact to rounding even when x c is large, where
      // z - lnZ is not (the rounding of c moves x c by ~1e-7 of it)
      lp = (float)((double)__builtin_fmaf(chosen_x, c, -Rref) * 0.6931471805599453 - lZ);
    } else if (token >= 0 && Zfull > 0.0 && chosen_z == chosen_z) {
      lp = (float)((double)chosen_z - lnZ);
    }
    P.chosen_logprob[r] = lp;
  }
  if (g.ntop > 0 && status == 0) {
    // (n_top <= 64: wave 0 writes them)
    for (int q = tid; q < P.n_top; q += 64) {
      if (q < ntop_out) {
        const uint64_t kk = S.sk[0][q];
        const float xq = __uint_as_float(S.sx[0][q]);
        // (as the chosen logprob: the logit's mass in the row mass's arithmetic)
        P.top_logprobs[(int64_t)r * P.n_top + q] =
            xq == xq && xq != INFINITY && xq != -INFINITY
                ? (float)((double)__builtin_fmaf(xq, c, -Rref) * 0.6931471805599453 - lZ)
                : (float)((double)key2f(key_z(kk)) - lnZ);
        if (P.top_ids) P.top_ids[(int64_t)r * P.n_top + q] = (int64_t)key_index(kk);
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
  return 0;
}

// ===========================================================================
// The kernel: grid of ceil(R / 8) * 8 * G workgroups of NT threads.
// ===========================================================================
// XF: the launch asks for the entropy output, may hold pure rows without a
// draw (the mass-only path), or may hold min-p / typical-p rows without top-k
// or rows with top_k past FAST_KMAX; that code is absent otherwise (such rows
// are then deferred).
template <int DT, int VPE, int NE, bool XF>
__global__ __launch_bounds__(NT) void rowgroup_kernel(RgParams F) {
  __shared__ RgShared<NE> SU;
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  int r = (slot / F.G) * 8 + xcd;
  const int j = slot % F.G;
  if (r >= F.k.R) return;
  if (F.heavy_first) r = heavy_first_row(F.k, r);
  const RowCfg g = row_cfg<XF>(F.k, r);
  if (F.skip_topk && stream_takes(g)) return;
  // the row's launch epoch: written only by the finalisers of earlier
  // launches (stream-ordered before this one), read by every chunk of the row
  // before any of them arrives
  const uint32_t epoch = ld_agent(F.counters + (int64_t)r * 32 + CTR_EPOCH);
  int tcase = -1;  // typical-p rows without other filters: TYP_*
  const int mode = chunk_phase<DT, VPE, NE, XF>(F, SU.c, r, j, g, epoch, tcase);
  if (mode == MODE_DEFER) {
    if (j == 0 && threadIdx.x == 0) F.status[r] = LPS_ROW_DEFERRED | (1 << 8);
    return;
  }
  // arrival: the chunk's stores are visible at agent scope before it is counted
  release_agent();
  __syncthreads();
  if (threadIdx.x == 0) {
    release_count();
    SU.c.mi[7] = add_agent(F.counters + (int64_t)r * 32 + CTR_ARRIVE, 1u) + 1u == (uint32_t)F.G ? 1 : 0;
    if (SU.c.mi[7]) acquire_one();
  }
  __syncthreads();
  // the finaliser runs on waves 0 .. FW - 1 (one per SIMD); the others leave
  if (!SU.c.mi[7] || threadIdx.x >= FT) return;
  acquire_agent();
  RG_STAMP(24);
  const int reason = final_phase<DT, VPE, XF>(F, SU.f, r, g, epoch, tcase);
  RG_STAMP(31);
  if (reason > 0 && threadIdx.x == 0) F.status[r] = LPS_ROW_DEFERRED | (reason << 8);
}

}  // namespace rg
}  // namespace lps
