// Streaming sampling kernel: one workgroup per row, for batches of greedy and
// top-k rows too large for one resident round of the row-group kernel.
//
// Reference path: Sampler.sample_token (sampling.py:51-85) with top-k
// (:139-156), top-p on the top-k set (:158-185), min-p (:187-205), the
// typical-p argmax fallback with top-k active (:207-238), greedy argmax
// (:72-75), the repetition penalty (:108-137) plus presence / frequency
// penalties, and the logprob outputs.
//
// Shape.  Workgroup r (512 threads, 8 waves) streams row r once from HBM in
// tiles of SVT 16-byte vectors per thread (consecutive threads read
// consecutive vectors), with the next tile's loads in flight while the current
// one is processed.  Two workgroups share a CU (<= 128 VGPRs, <= 80 KB LDS),
// so one row's loads overlap the other row's arithmetic.
//
// Per element, in registers:
//   - ids of the row's history and illegal ids are set to -inf (the history
//     ids are restored below; illegal ids are -inf in every output);
//   - maximum (greedy rows: first argmax), NaN flag;
//   - logprob rows: sum of exp2(fma(x, c, -ref)) against a per-thread integer
//     reference ref = ceil(max * c), rescaled by an exact power of two when it
//     rises;
//   - candidates: every logit at or above the wave's threshold is appended to
//     the wave's LDS segment (a ballot gives each lane its slot).  The wave's
//     threshold starts at the k'-th largest of the wave's first-tile lane
//     maxima (k' = max(top_k, top-N logprobs)), lowered to the start of its
//     division-collision group, and is raised the same way over the segment
//     when it fills past half.  Each wave thus keeps at least k' of its own
//     logits at or above its threshold, so the row's k'-th largest scaled
//     logit lies at or above the largest wave threshold theta*, and every
//     logit of the row's top-k' set (ties included) is a candidate of its
//     wave.  No barrier is taken inside the stream.
// After the stream:
//   - history ids: each distinct id's logit is read, masked, penalised
//     (penalize: repetition once per distinct id, then frequency and presence)
//     and folded into the maximum, the argmax, the logprob sum and the
//     candidates (when at or above theta*);
//   - candidates at or above theta* form the pool; a pool larger than KM / 2
//     is cut again by the largest per-wave k'-th key of its slices;
//   - the pool is keyed by (z = fl(x / T) descending, index ascending),
//     rank-sorted, given exact fixed-point masses against ceil(max * c), and
//     decided by the row-group finaliser's top-k code (topk_decide): the same
//     kept set, cut, draw and outputs as the row-group kernel.
// Rows the kernel cannot finish exactly (a wave segment overflow, a pool past
// capacity, more distinct history ids than the table holds) are marked
// LPS_ROW_DEFERRED for the general kernel.  Nucleus, pure and deferred-mode
// rows are left to the row-group kernel, or deferred when it is not launched.
#pragma once

#include "lps_rowgroup.h"

namespace lps {
namespace st {

using namespace rg;

constexpr int SNT = 512;          // threads per workgroup (8 waves)
constexpr int SNW = SNT / 64;     // waves
constexpr int SVT = 4;            // 16-byte vectors per thread per tile
constexpr int SEG = 256;          // candidate entries per wave segment
constexpr int BMW = STREAM_VMAX / 32;  // history bitmap words
constexpr int POOL = 2048;        // pool entries (wave candidates and history ids)
static_assert(POOL == SNW * SEG, "the pool reuses the segments' storage");
static_assert(KM == 4 * FT && FT == 256, "topk_decide runs on waves 0-3");
static_assert(STREAM_KMAX <= 128, "first threshold from the lanes' top two");

struct StShared : RgX {
  union {
    uint32_t bm[BMW];                   // history-id bitmap (bit i & 31 of word i >> 5)
    struct {
      uint64_t sk[KM];                  // sorted keys
      uint64_t sm[KM];                  // their fixed-point masses
    } s;
  } a;
  uint64_t sc[KM];                      // prefix of the masses (topk_decide)
  int32_t hkey[HASH_CAP];               // distinct history ids (open addressing)
  int32_t hcnt[HASH_CAP];               // their counts
  union {
    struct {
      uint32_t x[SNW][SEG];             // candidate logits (bits)
      int32_t i[SNW][SEG];              // candidate indices
    } seg;
    uint64_t ck[POOL];                  // pool keys
  } b;
  int32_t segn[SNW];                    // segment counts (SEG + 1: overflowed)
  float segth[SNW];                     // wave thresholds
  int32_t pn;                           // pool count
};
static_assert(sizeof(StShared) <= 80 * 1024, "two workgroups per CU");

// Raises the wave's threshold over its segment (every lane of the wave calls
// it): the kc-th largest buffered logit, lowered to the start of its
// collision group, then keeps the entries at or above it, in order.
__device__ __forceinline__ void wave_refine(StShared& S, int w, uint32_t& n, int kc, bool greedy, float T, float& theta) {
  const int lane = threadIdx.x & 63;
  const int nn = (int)min(n, (uint32_t)SEG);
  uint32_t xb[SEG / 64];
  int ib[SEG / 64];
  uint32_t kv[SEG / 64];
#pragma unroll
  for (int q = 0; q < SEG / 64; q++) {
    const int e = lane + 64 * q;
    xb[q] = e < nn ? S.b.seg.x[w][e] : 0u;
    ib[q] = e < nn ? S.b.seg.i[w][e] : 0;
    kv[q] = e < nn ? f2key(__uint_as_float(xb[q])) : 0u;
  }
  uint32_t th = wave_kth_largest<SEG / 64>(kv, (uint32_t)kc);
  if (!greedy && th > kNegInfKey + 1u && th != 0xFFFFFFFFu) th = f2key(collision_lo(key2f(th), T));
  theta = fmaxf(theta, fmaxf(key2f(th), -3.40282347e38f));
  uint32_t m = 0;
#pragma unroll
  for (int q = 0; q < SEG / 64; q++) {
    const int e = lane + 64 * q;
    const bool keep = e < nn && !(__uint_as_float(xb[q]) < theta);
    const uint64_t bm = __builtin_amdgcn_ballot_w64(keep);
    if (keep) {
      const uint32_t p = m + lanes_below(bm);
      S.b.seg.x[w][p] = xb[q];
      S.b.seg.i[w][p] = ib[q];
    }
    m += (uint32_t)__popcll(bm);
  }
  n = m;
}

template <int DT, int VPE>
__global__ __launch_bounds__(SNT, 4) void stream_kernel(RgParams F) {
  __shared__ StShared S;
  const KParams& P = F.k;
  const int r = blockIdx.x;
  if (r >= P.R) return;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const RowCfg g = row_cfg(P, r);
  if (!stream_takes(g)) {
    // the row-group kernel's rows; deferred when it is not launched
    if (F.stream_only && tid == 0) F.status[r] = LPS_ROW_DEFERRED | (16 << 8);
    return;
  }
  const bool greedy = g.greedy;
  const float T = g.T, c = g.c;
  const int V = P.V;
  const int kc = g.kprime;
  const bool want_lp = P.chosen_logprob || g.ntop > 0;
  const char* row = row_ptr<DT>(P, r);
  const uint8_t* am = row_allowed(P, r);
  const bool pen = g.pen;

  // ---- the history: bitmap of the distinct in-range ids, and their counts ----
  if (pen) {
    const int nw = (V + 31) >> 5;
    for (int i = tid; i < nw; i += SNT) S.a.bm[i] = 0u;
    for (int i = tid; i < HASH_CAP; i += SNT) {
      S.hkey[i] = -1;
      S.hcnt[i] = 0;
    }
  }
  if (tid == 0) {
    S.mi[0] = 0;
    S.pn = 0;
  }
  __syncthreads();
  if (pen) {
    bool full = false;
    for (int j = tid; j < g.hlen; j += SNT) {
      const int id = g.hrow[j];
      if (id < 0 || id >= V) continue;
      atomicOr(&S.a.bm[id >> 5], 1u << (id & 31));
      uint32_t sl = hash_id(id);
      int p = 0;
      for (; p < HASH_CAP; p++) {
        const int old = atomicCAS(&S.hkey[sl], -1, id);
        if (old == -1 || old == id) {
          atomicAdd(&S.hcnt[sl], 1);
          break;
        }
        sl = (sl + 1) & (HASH_CAP - 1);
      }
      if (p == HASH_CAP) full = true;
    }
    if (full) S.mi[0] = 1;
  }
  __syncthreads();
  bool defer_hist = false;
  if (pen) {
    uint32_t used = 0;
    for (int i = tid; i < HASH_CAP; i += SNT) used += S.hkey[i] >= 0 ? 1u : 0u;
    used = bred<SNW>(used, S.u, OpAdd{});
    defer_hist = S.mi[0] != 0 || used > (uint32_t)LPS_MAX_HISTORY_DISTINCT;
  }

  // ---- the stream ----
  const int nvec = F.nvec;
  constexpr int TV = SNT * SVT;     // vectors per tile
  constexpr int NE = SVT * VPE;     // logits per thread per tile
  const int ntiles = (nvec + TV - 1) / TV;
  const uint8_t* bmb = reinterpret_cast<const uint8_t*>(S.a.bm);
  const bool kill = pen || am;
  constexpr uint32_t VMASK = (1u << VPE) - 1u;
  // legality / history bits of vector v (VPE bits: 8 ids per byte, or a nibble)
  auto bits_of = [&](const uint8_t* base, int v) -> uint32_t {
    if constexpr (VPE == 8) return base[v];
    else return ((uint32_t)base[v >> 1] >> ((v & 1) * 4)) & VMASK;
  };
  auto vid = [&](int t, int s) { return (t * TV + (s / VPE) * SNT + tid) * VPE + (s % VPE); };

  float bx = -INFINITY;             // thread maximum (greedy rows: with its first index)
  int bi = 0x7FFFFFFF;
  int nanidx = 0x7FFFFFFF;          // first NaN id seen by this thread
  float ref = -INFINITY;            // logprob mass reference of this thread
  double zs = 0.0;
  float theta = 3.40282347e38f;     // wave threshold (set after the first tile)
  uint32_t nseg = 0;                // wave segment count (wave-uniform)
  bool over = false;

  u32x4 cur[SVT], nxt[SVT];
  uint32_t acur[SVT], anxt[SVT];
  auto load_tile = [&](u32x4 (&d)[SVT], uint32_t (&ab)[SVT], int t) {
#pragma unroll
    for (int i = 0; i < SVT; i++) {
      const int v = min(t * TV + i * SNT + tid, nvec - 1);
      d[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(row + (int64_t)v * 16));
    }
#pragma unroll
    for (int i = 0; i < SVT; i++) ab[i] = am ? bits_of(am, min(t * TV + i * SNT + tid, nvec - 1)) : VMASK;
  };
  load_tile(cur, acur, 0);
  for (int t = 0; t < ntiles; t++) {
    if (t + 1 < ntiles) load_tile(nxt, anxt, t + 1);
    float x[NE];
#pragma unroll
    for (int i = 0; i < SVT; i++) {
      const int v = t * TV + i * SNT + tid;
      const bool ok = v < nvec;
      const uint32_t w[4] = {cur[i].x, cur[i].y, cur[i].z, cur[i].w};
      if constexpr (DT == LPS_DTYPE_F32) {
#pragma unroll
        for (int e = 0; e < 4; e++) x[i * 4 + e] = ok ? __uint_as_float(w[e]) : -INFINITY;
      } else {
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const uint32_t h = (w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
          x[i * 8 + e] = ok ? (DT == LPS_DTYPE_BF16 ? __uint_as_float(h << 16) : f16_to_f32(h)) : -INFINITY;
        }
      }
      if (kill) {
        const uint32_t kb = (~acur[i] & VMASK) | ((pen && ok) ? bits_of(bmb, v) : 0u);
        if (__builtin_amdgcn_ballot_w64(kb != 0u)) {
#pragma unroll
          for (int e = 0; e < VPE; e++) x[i * VPE + e] = ((kb >> e) & 1u) ? -INFINITY : x[i * VPE + e];
        }
      }
    }
    // tile maximum and NaN
    float m = -INFINITY;
    bool tn = false;
#pragma unroll
    for (int s = 0; s < NE; s++) {
      m = fmaxf(m, x[s]);
      tn |= x[s] != x[s];
    }
    if (tn) {
#pragma unroll
      for (int s = 0; s < NE; s++)
        if (x[s] != x[s]) nanidx = min(nanidx, vid(t, s));
    }
    if (greedy) {
      if (m > bx) {  // first index of the new maximum (ids rise with s)
        int f = 0x7FFFFFFF;
#pragma unroll
        for (int s = NE - 1; s >= 0; s--)
          if (x[s] == m) f = vid(t, s);
        bx = m;
        bi = f;
      }
    } else {
      bx = fmaxf(bx, m);
    }
    // logprob mass against this thread's reference
    if (want_lp && m != -INFINITY && m != INFINITY) {
      const float nref = ceilf(__fmul_rn(m, c));
      if (nref > ref) {
        zs = ref == -INFINITY ? 0.0 : ldexp(zs, (int)(ref - nref));
        ref = nref;
      }
#pragma unroll
      for (int i = 0; i < SVT; i++) {
        float a = 0.0f;
#pragma unroll
        for (int e = 0; e < VPE; e++) a += __builtin_amdgcn_exp2f(__builtin_fmaf(x[i * VPE + e], c, -ref));
        zs += (double)a;
      }
    }
    // candidates
    if (kc > 0) {
      if (t == 0) {
        // the wave's first threshold: at least kc logits of its first tile lie at or above it
        uint32_t th;
        if (kc <= 64) {
          const uint32_t v1[1] = {f2key(m)};
          th = wave_kth_largest<1>(v1, (uint32_t)kc);
        } else {
          float m2 = -INFINITY;  // the thread's second largest of the tile
          bool seen = false;
#pragma unroll
          for (int s = 0; s < NE; s++) {
            const bool first = !seen && x[s] == m;
            seen |= first;
            m2 = first ? m2 : fmaxf(m2, x[s]);
          }
          const uint32_t v2[2] = {f2key(m), f2key(m2)};
          th = wave_kth_largest<2>(v2, (uint32_t)kc);
        }
        if (!greedy && th > kNegInfKey + 1u && th != 0xFFFFFFFFu) th = f2key(collision_lo(key2f(th), T));
        theta = fmaxf(key2f(th), -3.40282347e38f);
        // a first tile whose candidates would fill half the segment (short
        // rows, large k'): the exact kc-th largest of the wave's tile instead
        uint32_t cnt = 0;
#pragma unroll
        for (int s = 0; s < NE; s++) cnt += (uint32_t)__popcll(__builtin_amdgcn_ballot_w64(x[s] >= theta));
        if (cnt > (uint32_t)(SEG / 2)) {
          uint32_t kv[NE];
#pragma unroll
          for (int s = 0; s < NE; s++) kv[s] = x[s] == x[s] ? f2key(x[s]) : 0u;
          th = wave_kth_largest<NE>(kv, (uint32_t)kc);
          if (!greedy && th > kNegInfKey + 1u && th != 0xFFFFFFFFu) th = f2key(collision_lo(key2f(th), T));
          theta = fmaxf(theta, fmaxf(key2f(th), -3.40282347e38f));
        }
      }
#pragma unroll
      for (int s = 0; s < NE; s++) {
        const bool on = x[s] >= theta;
        const uint64_t bm = __builtin_amdgcn_ballot_w64(on);
        if (bm) {
          if (on) {
            const uint32_t p = nseg + lanes_below(bm);
            if (p < (uint32_t)SEG) {
              S.b.seg.x[wv][p] = __float_as_uint(x[s]);
              S.b.seg.i[wv][p] = vid(t, s);
            }
          }
          nseg += (uint32_t)__popcll(bm);
        }
      }
      if (nseg > (uint32_t)SEG) {
        over = true;
        break;
      }
      if (nseg > (uint32_t)(SEG / 2)) wave_refine(S, wv, nseg, kc, greedy, T, theta);
    }
#pragma unroll
    for (int i = 0; i < SVT; i++) {
      cur[i] = nxt[i];
      acur[i] = anxt[i];
    }
  }
  if (lane == 0) {
    S.segn[wv] = over ? SEG + 1 : (int)nseg;
    S.segth[wv] = kc > 0 ? theta : 3.40282347e38f;
  }
  __syncthreads();
  float ths = -3.40282347e38f;  // theta*: the largest wave threshold
  bool seg_over = false;
#pragma unroll
  for (int w = 0; w < SNW; w++) {
    ths = fmaxf(ths, S.segth[w]);
    seg_over |= S.segn[w] > SEG;
  }

  // ---- pool, part 1: the wave candidates at or above theta*, read into
  // registers (the pool keys overwrite the segments after the barriers below) ----
  constexpr int PPT = POOL / SNT;
  uint32_t px[PPT];
  int pi[PPT];
  bool pk[PPT];
#pragma unroll
  for (int q = 0; q < PPT; q++) {
    const int e = tid + q * SNT, w = e / SEG, p = e % SEG;
    pk[q] = kc > 0 && !seg_over && p < S.segn[w];
    px[q] = pk[q] ? S.b.seg.x[w][p] : 0u;
    pi[q] = pk[q] ? S.b.seg.i[w][p] : 0;
    pk[q] = pk[q] && !(__uint_as_float(px[q]) < ths);
  }

  // ---- history ids: read, mask, penalise, fold in ----
  constexpr int HPT_ = HASH_CAP / SNT;
  uint32_t hx[HPT_];
  int hid[HPT_];
  bool hk[HPT_];
#pragma unroll
  for (int q = 0; q < HPT_; q++) {
    const int s = tid + q * SNT;
    const int id = pen ? S.hkey[s] : -1;
    hk[q] = false;
    hid[q] = id;
    hx[q] = 0u;
    if (id >= 0) {
      float xv = load1<DT, false>(row, id);
      if (!id_allowed(am, id)) xv = -INFINITY;
      xv = penalize(xv, S.hcnt[s], g.rep, g.pres, g.freq);
      hx[q] = __float_as_uint(xv);
      if (xv != xv) nanidx = min(nanidx, id);
      if (greedy) {
        if (xv > bx || (xv == bx && id < bi)) {
          bx = xv;
          bi = id;
        }
      } else {
        bx = fmaxf(bx, xv);
      }
      if (want_lp && xv != -INFINITY && xv != INFINITY && xv == xv) {
        const float nref = ceilf(__fmul_rn(xv, c));
        if (nref > ref) {
          zs = ref == -INFINITY ? 0.0 : ldexp(zs, (int)(ref - nref));
          ref = nref;
        }
        zs += (double)__builtin_amdgcn_exp2f(__builtin_fmaf(xv, c, -ref));
      }
      hk[q] = kc > 0 && !seg_over && xv >= ths;
    }
  }

  // ---- the row: maximum, first argmax, NaN, log-sum-exp ----
  const uint64_t bk = ((uint64_t)f2key(bx) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)bi);
  const uint64_t rk = bred<SNW>(bk, S.q, OpMax{});
  const int nanr = bred<SNW>(nanidx, S.i1, OpMin{});
  float xmax = key2f((uint32_t)(rk >> 32));
  int gam = key_index(rk);
  if (nanr != 0x7FFFFFFF) {
    xmax = __uint_as_float(0x7FC00000u);
    gam = nanr;
  }
  const bool xfin = xmax == xmax && xmax != INFINITY && xmax != -INFINITY;
  double Z = 0.0;
  float R = -INFINITY;
  if (want_lp) {
    R = bred<SNW>(ref, S.rf, OpMax{});
    const double zsc = (ref != -INFINITY && R != -INFINITY) ? ldexp(zs, (int)(ref - R)) : 0.0;
    Z = bred<SNW>(zsc, S.d, OpAdd{});
    if (!xfin) Z = 0.0;
  }
  int status = 0;
  if (!greedy) {
    if (!(xmax == xmax) || xmax == INFINITY || __fdiv_rn(xmax, T) == INFINITY) status |= LPS_ROW_NONFINITE;
    else if (xmax == -INFINITY) status |= LPS_ROW_EMPTY;
  }
  int reason = defer_hist ? 14 : (seg_over ? 15 : 0);

  // ---- pool, part 2: keys (z descending, index ascending); every segment
  // entry was read before the barriers of the reductions above ----
  const float Rm = xfin ? ceilf(__fmul_rn(xmax, c)) : 0.0f;
  int n = 0;
  if (reason == 0 && kc > 0) {
#pragma unroll
    for (int q = 0; q < PPT; q++)
      if (pk[q]) S.b.ck[atomicAdd(&S.pn, 1)] = cand_key(__uint_as_float(px[q]), pi[q], greedy, T);
#pragma unroll
    for (int q = 0; q < HPT_; q++)
      if (hk[q]) {
        const int p = atomicAdd(&S.pn, 1);
        if (p < POOL) S.b.ck[p] = cand_key(__uint_as_float(hx[q]), hid[q], greedy, T);
      }
    __syncthreads();
    n = S.pn;
    if (n > POOL) reason = 16;
  }
  if (reason == 0 && kc > 0 && n > KM / 2) {
    // cut the pool again: every wave's slice keeps its kc-th largest z and
    // above, so the largest slice threshold bounds the row's kc-th largest
    uint64_t kk[PPT];
    uint32_t kz[PPT];
#pragma unroll
    for (int q = 0; q < PPT; q++) {
      const int e = wv * 64 * PPT + q * 64 + lane;
      kk[q] = e < n ? S.b.ck[e] : 0ull;
      kz[q] = e < n ? key_z(kk[q]) : 0u;
    }
    const uint32_t sth = wave_kth_largest<PPT>(kz, (uint32_t)kc);
    const uint32_t zth = bred<SNW>(sth, S.u2, OpMax{});
    uint32_t keep = 0;
#pragma unroll
    for (int q = 0; q < PPT; q++) {
      const int e = wv * 64 * PPT + q * 64 + lane;
      keep += (e < n && kz[q] >= zth) ? 1u : 0u;
    }
    uint32_t tot;
    uint32_t pos = bscan<SNW>(keep, &tot, S.u3);
    __syncthreads();
#pragma unroll
    for (int q = 0; q < PPT; q++) {
      const int e = wv * 64 * PPT + q * 64 + lane;
      if (e < n && kz[q] >= zth) S.b.ck[pos++] = kk[q];
    }
    __syncthreads();
    n = (int)tot;
  }
  if (reason == 0 && kc > 0 && n > KM) reason = 16;

  // ---- rank sort: each wave ranks 64 entries at a time against every key ----
  if (reason == 0 && kc > 0) {
    for (int e0 = wv * 64; e0 < n; e0 += SNT) {
      const int e = e0 + lane;
      const uint64_t key = e < n ? S.b.ck[e] : 0ull;
      int rank = 0;
      int q = 0;
      for (; q + 2 <= n; q += 2) {
        const uint64_t a0 = S.b.ck[q], a1 = S.b.ck[q + 1];
        rank += (a0 > key ? 1 : 0) + (a1 > key ? 1 : 0);
      }
      if (q < n) rank += S.b.ck[q] > key ? 1 : 0;
      if (e < n) {
        S.a.s.sk[rank] = key;
        S.a.s.sm[rank] = zmass_fix(key2f(key_z(key)), Rm);
      }
    }
  }
  __syncthreads();
  if (reason) {
    if (tid == 0) F.status[r] = LPS_ROW_DEFERRED | (reason << 8);
    return;
  }
  // ---- the decision (waves 0-3; the others leave) and the outputs ----
  if (tid >= FT) return;
  Decision d;
  if (kc > 0 && (status == 0 || greedy)) {
    float u = g.u;
    if (!(u >= 0.0f)) u = 0.0f;
    if (u >= 1.0f) u = 0.99999994f;
    const int rc = topk_decide(g, V, S.a.s.sk, S.a.s.sm, S.sc, n, n, u, gam, xmax, S, d);
    if (rc) {
      if (tid == 0) F.status[r] = LPS_ROW_DEFERRED | (rc << 8);
      return;
    }
    status |= d.status;
  } else if (greedy) {
    d.token = gam;
    d.cut = xmax;
    d.ties = 1;
    d.kept_n = 1;
    d.qprob = (g.qtok >= 0 && g.qtok == gam) ? 1.0f : 0.0f;
    d.chosen_z = xmax;
  }
  if (greedy) status = 0;
  int64_t token = status ? -1 : d.token;
  if (P.skip_draw && !greedy) token = -1;
  double lnZ = 0.0;
  if (want_lp && Z > 0.0) lnZ = log(Z) + (double)R * 0.6931471805599453;
  if (P.chosen_logprob && tid == 0) {
    float lp = NAN;
    if (token >= 0 && Z > 0.0 && d.chosen_z == d.chosen_z) lp = (float)((double)d.chosen_z - lnZ);
    P.chosen_logprob[r] = lp;
  }
  if (g.ntop > 0 && status == 0) {
    for (int q = tid; q < P.n_top; q += 64) {  // n_top <= 64: wave 0
      if (q < d.ntop_out) {
        const uint64_t kk = S.a.s.sk[q];
        P.top_logprobs[(int64_t)r * P.n_top + q] = (float)((double)key2f(key_z(kk)) - lnZ);
        if (P.top_ids) P.top_ids[(int64_t)r * P.n_top + q] = (int64_t)key_index(kk);
      } else {
        P.top_logprobs[(int64_t)r * P.n_top + q] = -INFINITY;
        if (P.top_ids) P.top_ids[(int64_t)r * P.n_top + q] = -1;
      }
    }
  }
  if (tid == 0) {
    P.tokens[r] = token;
    append_token(P, r, token);
    F.status[r] = status;
    if (P.row_status) P.row_status[r] = status;
    if (P.query_prob) P.query_prob[r] = d.qprob;
    if (P.kept_cut) P.kept_cut[r] = d.cut;
    if (P.kept_ties) P.kept_ties[r] = d.ties;
    if (P.kept_count) P.kept_count[r] = d.kept_n;
    if (P.row_path) P.row_path[r] = 0;
  }
}

}  // namespace st
}  // namespace lps
