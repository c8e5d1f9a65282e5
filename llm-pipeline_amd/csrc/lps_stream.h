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
//     logits at or above its threshold.  Every wave also publishes (LDS) a
//     share: its ceil(k'/8)-th largest logit so far, lowered the same way;
//     the eight waves hold at least k' logits at or above the smallest share.
//     So the row's k'-th largest scaled logit lies at or above theta*, the
//     larger of the largest own threshold and the smallest share, and every
//     logit of the row's top-k' set (ties included) is at or above the
//     emission threshold max(own, smallest share) of its wave at any time.
//     No barrier is taken inside the stream.
// History ids.  Before the stream the row's in-range history ids set bits of
// a vocabulary bitmap, and the set bits become a sorted list of the distinct
// ids (a block scan of the threads' bit counts over their words gives each id
// its rank); with a
// frequency penalty every history id then adds to its entry's count (found by
// binary search).  An entry is id | count << 18 (ids < 2^18).
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
// capacity, more than HLIST distinct history ids or a count past HCMAX) are
// marked LPS_ROW_DEFERRED for the general kernel, which counts histories of
// any size.  (Calling the general algorithm from this kernel, even as a
// separate function, costs the stream ~110 spilled VGPRs under its 128-VGPR
// budget.)  Nucleus, pure and deferred-mode rows are left to the row-group
// kernel, or deferred when it is not launched.
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
constexpr int HLIST = 4096;       // distinct history ids of a row (sorted list)
constexpr uint32_t HCMAX = (1u << 14) - 2;  // largest history count of an entry
constexpr int HPT_ = HLIST / SNT; // list entries per thread after the stream
constexpr int BMT = BMW / SNT;    // bitmap words per thread (words BMT t .. BMT t + BMT - 1)
static_assert(BMW % SNT == 0, "whole bitmap words per thread");
static_assert(STREAM_VMAX <= (1 << 18), "18-bit ids in the list entries");
static_assert(POOL == SNW * SEG, "the pool reuses the segments' storage");
static_assert(KM == 4 * FT && FT == 256, "topk_decide runs on waves 0-3");
static_assert(STREAM_KMAX <= 128, "first threshold from the lanes' top two");

struct StShared : RgX {
  union {
    uint32_t bm[BMW];                   // history-id bitmap (bit i & 31 of word i >> 5)
    struct {
      uint64_t sk[KM];                  // sorted keys
      uint64_t sm[KM];                  // their fixed-point masses
      uint32_t sx[KM];                  // their logits (bits)
    } s;
  } a;
  uint64_t sc[KM];                      // prefix of the masses (topk_decide)
  uint32_t hl[HLIST];                   // distinct history ids, ascending: id | count << 18
  uint32_t hwb[SNW];                    // the waves' bitmap bit counts (list ranks)
  union {
    struct {
      uint32_t x[SNW][SEG];             // candidate logits (bits)
      int32_t i[SNW][SEG];              // candidate indices
    } seg;
    uint64_t ck[POOL];                  // pool keys
  } b;
  uint4 km[256];                        // kill masks: the words' -inf positions of a VPE-bit kill pattern
  int32_t segn[SNW];                    // segment counts (SEG + 1: overflowed)
  float segth[SNW];                     // wave thresholds (each wave: >= k' own logits at or above)
  float segjt[SNW];                     // joint shares (each wave: >= ceil(k'/8) own logits at or above)
  int32_t pn;                           // pool count
  uint32_t cx[POOL];                    // pool logits (bits), beside the pool keys
  RowCfg cfg;                           // the row's parameters (loaded by wave 0)
};
static_assert(sizeof(StShared) <= 80 * 1024, "two workgroups per CU");

// Raises the wave's threshold over its segment (every lane of the wave calls
// it): the kc-th largest buffered logit, lowered to the start of its
// collision group, then keeps the entries at or above it, in order.
// The joint threshold: the smallest published share.  Every wave has at least
// ceil(k'/8) of its own logits at or above its share, so the eight waves hold
// at least k' logits at or above the smallest (a wave that has not published
// yet counts as -inf).  Every lane of the wave calls it.
__device__ __forceinline__ float joint_threshold(const StShared& S) {
  float t = S.segjt[0];
#pragma unroll
  for (int v = 1; v < SNW; v++) t = fminf(t, S.segjt[v]);
  return t;
}
// Lower end of the collision group of the key th (greedy rows: th itself), as
// a threshold float no lower than -FLT_MAX.
__device__ __forceinline__ float key_threshold(uint32_t th, bool greedy, float T) {
  if (!greedy && th > kNegInfKey + 1u && th != 0xFFFFFFFFu) th = f2key(collision_lo(key2f(th), T));
  return fmaxf(key2f(th), -3.40282347e38f);
}
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
  // own threshold (k'-th) and joint share (ceil(k'/8)-th): the segment holds
  // every own logit at or above the current emission threshold, which is at
  // most the share, so both are exact over the wave's own logits seen so far
  theta = fmaxf(theta, key_threshold(wave_kth_largest<SEG / 64>(kv, (uint32_t)kc), greedy, T));
  const float share = key_threshold(wave_kth_largest<SEG / 64>(kv, (uint32_t)((kc + SNW - 1) / SNW)), greedy, T);
  if (lane == 0) S.segjt[w] = fmaxf(S.segjt[w], share);
  const float te = fmaxf(theta, joint_threshold(S));
  uint32_t m = 0;
#pragma unroll
  for (int q = 0; q < SEG / 64; q++) {
    const int e = lane + 64 * q;
    const bool keep = e < nn && !(__uint_as_float(xb[q]) < te);
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

// The key of the m-th largest non-NaN value of x over the wave (M values per
// lane; every lane calls it): a 32-step search over keys, each step one float
// comparison per value against the step's key.
template <int M>
__device__ __forceinline__ uint32_t wave_kth_largest_x(const float (&x)[M], uint32_t m) {
  uint32_t t = 0;
#pragma unroll 1
  for (int b = 31; b >= 0; b--) {
    const uint32_t c = t | (1u << b);
    const float th = key2f(c);
    uint32_t n = 0;
#pragma unroll
    for (int i = 0; i < M; i++) n += (uint32_t)__popcll(__builtin_amdgcn_ballot_w64(x[i] >= th));
    if (n >= m) t = c;
  }
  return t;
}

// AM: the launch carries legality masks (P.allowed non-null).
template <int DT, int VPE, bool AM>
__global__ __launch_bounds__(SNT, 4) void stream_kernel(RgParams F) {
  __shared__ StShared S;
  const KParams& P = F.k;
  // rows skewed over the XCDs (workgroup b runs on XCD b % 8): group k of 8
  // workgroups puts row 8k + ((x + k) mod 8) on XCD x, so rows that alternate
  // in kind (greedy / sampled, or any period dividing 8) spread over every
  // XCD instead of one kind per XCD; a last partial group keeps b
  const int wgi = blockIdx.x, wgk = wgi >> 3;
  const int r = (wgk * 8 + 8 <= P.R) ? wgk * 8 + (((wgi & 7) + wgk) & 7) : wgi;
  if (r >= P.R) return;
  // (the wave index through readfirstlane: the compiler then knows it is
  // wave-uniform, and the chunk loop below is a scalar loop)
  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  RG_STAMP(0);
  // ---- the stream's constants; the first three tiles and the first history
  // ids are loaded before anything else (the row's parameters decide below
  // whether this kernel takes the row; the loads of a row it does not take
  // are dropped) ----
  const int V = P.V;
  const char* row = row_ptr<DT>(P, r);
  const uint8_t* am = AM ? row_allowed(P, r) : nullptr;
  const int nvec = F.nvec;
  constexpr int CV = 64 * SVT;      // vectors per chunk (one wave's unit of work)
  constexpr int NE = SVT * VPE;     // logits per thread per tile
  const int nch = (nvec + CV - 1) / CV;
  const uint8_t* bmb = reinterpret_cast<const uint8_t*>(S.a.bm);
  constexpr uint32_t VMASK = (1u << VPE) - 1u;
  // -inf in every element of a 32-bit word of the row
  constexpr uint32_t NEGW = DT == LPS_DTYPE_F32 ? 0xFF800000u : (DT == LPS_DTYPE_BF16 ? 0xFF80FF80u : 0xFC00FC00u);
  // legality / history bits of vector v (VPE bits: 8 ids per byte, or a nibble)
  auto bits_of = [&](const uint8_t* base, int v) -> uint32_t {
    if constexpr (VPE == 8) return base[v];
    else return ((uint32_t)base[v >> 1] >> ((v & 1) * 4)) & VMASK;
  };
  // id of slot s of chunk h (the lane's id base is laundered per use, so the
  // per-slot constants are not hoisted into registers for the whole loop)
  auto vid = [&](int h, int s) {
    int b = lane * VPE;
    LPS_KEEP_VGPR(b);
    return b + h * CV * VPE + (s / VPE) * 64 * VPE + (s % VPE);
  };

  // Chunk h's loads (every call issues the same loads, so the compiler's load
  // counters stay exact): four 16-byte vectors per lane, and with masks their
  // legality bytes.
  // (a tile past the row's end, loaded so that every step issues the same
  // loads, reads the row's last vector on every lane: one line, not a tile)
  auto load_tile = [&](u32x4 (&d)[SVT], uint32_t (&ab)[SVT], int h) {
#pragma unroll
    for (int i = 0; i < SVT; i++) {
      const int v = min(h * CV + i * 64 + lane, nvec - 1);
      d[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(row + (int64_t)v * 16));
    }
#pragma unroll
    for (int i = 0; i < SVT; i++) {
      const int v = min(h * CV + i * 64 + lane, nvec - 1);
      if constexpr (AM) ab[i] = VPE == 8 ? (uint32_t)am[v] : (uint32_t)am[v >> 1];
      else ab[i] = 0xFFu;
    }
  };
  // (the history ids first, then the row's parameters, then the chunks: loads
  // issued behind the whole GPU's first chunks would wait for them)
  const int32_t* hrow0 = P.history ? P.history + (int64_t)r * P.history_stride : nullptr;
  // (a row without history reads nothing; a history_stride of 0 shares one
  // history between the rows, whose first ids are then read at their own offsets)
  const int64_t hs = P.history_stride > 0 ? P.history_stride : ((int64_t)1 << 31);
  const int hraw0 = (hrow0 && tid < hs) ? hrow0[tid] : -1;
  const int hraw1 = (hrow0 && tid + SNT < hs) ? hrow0[tid + SNT] : -1;
  // (wave 0 alone loads the parameters, ahead of its chunks; the other waves'
  // would queue behind the chunks the first waves issued)
  __asm__ volatile("" ::: "memory");
  RowCfg g0;
  if (wv == 0) g0 = row_cfg<false>(P, r);  // (the rows it takes: greedy and top-k)
  __asm__ volatile("" ::: "memory");
  // chunks: each wave takes chunks wv, wv + 8, wv + 16, then the next free one
  // (a counter in LDS), so waves that run faster take more of the row
  int c0 = wv, c1 = wv + SNW, c2 = wv + 2 * SNW;
  u32x4 b0[SVT], b1[SVT], b2[SVT];
  uint32_t a0[SVT], a1[SVT], a2[SVT];
  __asm__ volatile("" ::: "memory");
  const int hid0 = hraw0, hid1 = hraw1;

  if (wv == 0 && lane == 0) S.cfg = g0;

  // ---- kill-mask table: pattern p (bit e = element e of a vector) -> the
  // bits of the vector's four words that belong to killed elements ----
  if (tid < 256) {
    uint32_t mk[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      if constexpr (VPE == 8)
        mk[j] = (((tid >> (2 * j)) & 1) ? 0x0000FFFFu : 0u) | (((tid >> (2 * j + 1)) & 1) ? 0xFFFF0000u : 0u);
      else
        mk[j] = ((tid >> j) & 1) ? 0xFFFFFFFFu : 0u;
    }
    S.km[tid] = make_uint4(mk[0], mk[1], mk[2], mk[3]);
  }
  // ---- the history: bitmap of the distinct in-range ids (cleared before
  // the parameters are known: one barrier for both) ----
  {
    const int nw = (V + 31) >> 5;
    for (int i = tid; i < nw; i += SNT) S.a.bm[i] = 0u;
  }
  if (lane == 0) S.segjt[wv] = -3.40282347e38f;
  if (tid == 0) {
    S.mi[0] = 0;
    S.mi[1] = 0;
    S.mi[2] = 0;  // chunks taken past the first three of every wave
    S.mi[3] = 0;  // distinct history ids
    S.pn = 0;
  }
  __syncthreads();
  const RowCfg g = S.cfg;
  RG_STAMP_DEP(9, g.T);
  if (!stream_takes(g)) {
    // the row-group kernel's rows; deferred when it is not launched
    if (F.stream_only && tid == 0) F.status[r] = LPS_ROW_DEFERRED | (16 << 8);
    return;
  }
  const bool greedy = g.greedy;
  const float T = g.T, c = g.c;
  const int kc = g.kprime;
  const bool want_lp = P.chosen_logprob || g.ntop > 0;
  const bool pen = g.pen;
  const bool kill = pen || am;
  RG_STAMP(11);
  // (without a frequency penalty an id's count does not matter: the list
  // entries keep count 0)
  const bool counts = g.freq != 0.0f;
  if (pen) {
    auto mark = [&](int id) {
      if (id >= 0 && id < V) atomicOr(&S.a.bm[id >> 5], 1u << (id & 31));
    };
    if (tid < g.hlen) mark(hid0);
    if (tid + SNT < g.hlen) mark(hid1);
    for (int j = tid + 2 * SNT; j < g.hlen; j += SNT) mark(g.hrow[j]);
  }
  __syncthreads();
  RG_STAMP(12);
  if (pen) {
    // ranks: thread t holds the words [BMT t, BMT t + BMT), so one scan of
    // the threads' bit counts over the block (per wave by DPP, then across
    // the waves) ranks every id, in ascending order
    const int nw = (V + 31) >> 5;
    uint32_t wd[BMT];
    uint32_t pc = 0;
#pragma unroll
    for (int i = 0; i < BMT; i++) {
      const int w = BMT * tid + i;
      wd[i] = w < nw ? S.a.bm[w] : 0u;
      pc += (uint32_t)__builtin_popcount(wd[i]);
    }
    const uint32_t inc = wscan_incl(pc);
    if (lane == 63) S.hwb[wv] = inc;
    __syncthreads();
    uint32_t before = 0, total = 0;
#pragma unroll
    for (int v = 0; v < SNW; v++) {
      const uint32_t cv = S.hwb[v];
      before += v < wv ? cv : 0u;
      total += cv;
    }
    uint32_t rk = before + inc - pc;
#pragma unroll
    for (int i = 0; i < BMT; i++) {
      const int w0 = (BMT * tid + i) << 5;
      for (uint32_t b = wd[i]; b; b &= b - 1u) {
        if (rk < (uint32_t)HLIST) S.hl[rk] = (uint32_t)(w0 + __builtin_ctz(b));
        rk++;
      }
    }
    if (tid == 0) S.mi[3] = (int)total;
    __syncthreads();
    RG_STAMP(13);
    const int D = S.mi[3];
    if (counts && D <= HLIST) {
      // every history id adds one to its entry (binary search over the sorted ids)
      int lg = 0;
      while ((1 << lg) < D) lg++;
      bool sat = false;
      auto add = [&](int id) {
        if (id < 0 || id >= V) return;
        int p = 0;
        for (int st = 1 << lg; st > 0; st >>= 1)
          if (p + st < D && (int)(S.hl[p + st] & 0x3FFFFu) <= id) p += st;
        const uint32_t old = atomicAdd(&S.hl[p], 1u << 18);
        if ((old >> 18) >= HCMAX) sat = true;
      };
      if (tid < g.hlen) add(hid0);
      if (tid + SNT < g.hlen) add(hid1);
      for (int j = tid + 2 * SNT; j < g.hlen; j += SNT) add(g.hrow[j]);
      if (sat) S.mi[0] = 1;
    }
  }
  __syncthreads();
  RG_STAMP(10);
  const bool defer_hist = pen && (S.mi[0] != 0 || S.mi[3] > HLIST);
  // (the chunks only now, in this order: the loop's waits count on b0, b1 and
  // b2's loads in turn; a first flood of every wave's chunks would hold the
  // parameters and history ids above back behind it)
  __asm__ volatile("" ::: "memory");
  load_tile(b0, a0, c0);
  __asm__ volatile("" ::: "memory");
  load_tile(b1, a1, c1);
  __asm__ volatile("" ::: "memory");
  load_tile(b2, a2, c2);
  __asm__ volatile("" ::: "memory");

  RG_STAMP(1);
  float bx = -INFINITY;             // thread maximum
  int bt = -1;                      // greedy rows: first chunk holding it (its index is found after the stream)
  bool first = true;                // the wave's first chunk (sets the threshold)
  int bi = 0x7FFFFFFF;
  int nanidx = 0x7FFFFFFF;          // first NaN id seen by this thread
  float ref = -INFINITY;            // logprob mass reference of this thread
  double zs = 0.0;
  float theta = -3.40282347e38f;    // wave threshold (set on the wave's first chunk; a wave
                                    // without chunks claims nothing)
  uint32_t nseg = 0;                // wave segment count (wave-uniform)
  bool over = false;

  // Tile t's logits of this thread: history ids, illegal ids and vectors past
  // the row set to -inf on the packed words (one LDS mask lookup per vector),
  // then unpacked.
  auto unpack_tile = [&](u32x4 (&raw)[SVT], const uint32_t (&ab)[SVT], int t, float (&x)[NE]) {
    const bool part = (t + 1) * CV > nvec;
    if (kill || part) {
      uint32_t kb[SVT], any = 0;
#pragma unroll
      for (int i = 0; i < SVT; i++) {
        const int v = t * CV + i * 64 + lane;
        const uint32_t legal = AM ? (VPE == 8 ? ab[i] : ab[i] >> ((v & 1) * 4)) : VMASK;
        kb[i] = v < nvec ? ((~legal & VMASK) | (pen ? bits_of(bmb, v) : 0u)) : VMASK;
        any |= kb[i];
      }
      if (__builtin_amdgcn_ballot_w64(any != 0u)) {
#pragma unroll
        for (int i = 0; i < SVT; i++) {
          const uint4 m = S.km[kb[i]];
          raw[i].x = (m.x & NEGW) | (~m.x & raw[i].x);
          raw[i].y = (m.y & NEGW) | (~m.y & raw[i].y);
          raw[i].z = (m.z & NEGW) | (~m.z & raw[i].z);
          raw[i].w = (m.w & NEGW) | (~m.w & raw[i].w);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < SVT; i++) {
      const uint32_t w[4] = {raw[i].x, raw[i].y, raw[i].z, raw[i].w};
      if constexpr (DT == LPS_DTYPE_F32) {
#pragma unroll
        for (int e = 0; e < 4; e++) x[i * 4 + e] = __uint_as_float(w[e]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const uint32_t h = (w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
          x[i * 8 + e] = DT == LPS_DTYPE_BF16 ? __uint_as_float(h << 16) : f16_to_f32(h);
        }
      }
    }
  };
  // One tile: maxima (NaN-propagating), logprob mass, candidates.  Returns
  // true when the wave's segment overflowed.
  auto process_tile = [&](u32x4 (&raw)[SVT], const uint32_t (&ab)[SVT], int t) -> bool {
    float x[NE];
    unpack_tile(raw, ab, t, x);
    float vm[SVT];  // vector maxima (NaN when the vector holds one)
#pragma unroll
    for (int i = 0; i < SVT; i++) {
      float a = x[i * VPE];
#pragma unroll
      for (int e = 1; e < VPE; e++) a = __builtin_elementwise_maximum(a, x[i * VPE + e]);
      vm[i] = a;
    }
    float m = vm[0];
#pragma unroll
    for (int i = 1; i < SVT; i++) m = __builtin_elementwise_maximum(m, vm[i]);
    if (m != m) {  // a NaN: its first id
#pragma unroll
      for (int s = 0; s < NE; s++)
        if (x[s] != x[s]) nanidx = min(nanidx, vid(t, s));
    } else if (m > bx) {
      bx = m;
      bt = t;
    }
    // logprob mass against this thread's reference
    if (want_lp && m == m && m != -INFINITY && m != INFINITY) {
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
    if (kc <= 0) return false;
    if (first) {
      first = false;
      // the wave's first threshold: at least kc logits of its first tile lie at or above it
      const float mt = m == m ? m : -INFINITY;
      uint32_t th;
      if (kc <= 64) {
        const uint32_t v1[1] = {f2key(mt)};
        th = wave_kth_largest<1>(v1, (uint32_t)kc);
      } else {
        float m2 = -INFINITY;  // the thread's second largest of the tile
        bool seen = false;
#pragma unroll
        for (int s = 0; s < NE; s++) {
          const bool first = !seen && x[s] == mt;
          seen |= first;
          m2 = first ? m2 : fmaxf(m2, x[s]);
        }
        const uint32_t v2[2] = {f2key(mt), f2key(m2)};
        th = wave_kth_largest<2>(v2, (uint32_t)kc);
      }
      theta = key_threshold(th, greedy, T);
      {  // the wave's first joint share: ceil(k'/8) lane maxima at or above it
        const uint32_t v1[1] = {f2key(mt)};
        const float share = key_threshold(wave_kth_largest<1>(v1, (uint32_t)((kc + SNW - 1) / SNW)), greedy, T);
        if (lane == 0) S.segjt[wv] = share;
      }
      // a first tile whose candidates would fill half the segment (short
      // rows, large k'): the exact kc-th largest of the wave's tile instead
      uint32_t cnt = 0;
#pragma unroll
      for (int s = 0; s < NE; s++) cnt += (uint32_t)__popcll(__builtin_amdgcn_ballot_w64(x[s] >= theta));
      if (cnt > (uint32_t)(SEG / 2)) {
        th = wave_kth_largest_x<NE>(x, (uint32_t)kc);
        if (!greedy && th > kNegInfKey + 1u && th != 0xFFFFFFFFu) th = f2key(collision_lo(key2f(th), T));
        theta = fmaxf(theta, fmaxf(key2f(th), -3.40282347e38f));
      }
    }
    // candidates (at or above the wave's own threshold and the joint one):
    // vectors whose maximum reaches it in any lane, then their elements
    const float te = fmaxf(theta, joint_threshold(S));
#pragma unroll
    for (int i = 0; i < SVT; i++) {
      if (!__builtin_amdgcn_ballot_w64(vm[i] >= te)) continue;
#pragma unroll
      for (int e = 0; e < VPE; e++) {
        const int s = i * VPE + e;
        const bool on = x[s] >= te;
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
    }
    if (nseg > (uint32_t)SEG) return true;
    if (nseg > (uint32_t)(SEG / 2)) wave_refine(S, wv, nseg, kc, greedy, T, theta);
    return false;
  };
  // three chunk buffers: once a chunk is processed its buffer loads the wave's
  // next chunk, so two chunks of loads are in flight behind the one processed;
  // the chunks a wave takes rise, so its ids rise with them
  auto take = [&]() -> int {
    int h = 0;
    if (lane == 0) h = atomicAdd(&S.mi[2], 1);
    return __builtin_amdgcn_readfirstlane(h) + 3 * SNW;
  };
  // Every step issues its buffer's next load (the last chunk again once the
  // row is done), so every path into the loop's head has issued the same loads
  // in the same order and the compiler's load-count waits stay two chunks deep.
  auto step = [&](u32x4 (&d)[SVT], uint32_t (&ab)[SVT], int& h) {
    const bool live = h < nch && !over;
    if (live) over = process_tile(d, ab, h);
    h = (live && !over) ? take() : nch;
    load_tile(d, ab, h);
  };
  do {
    step(b0, a0, c0);
    step(b1, a1, c1);
    step(b2, a2, c2);
  } while (c0 < nch && !over);
  RG_STAMP(2);
  // the history ids' logits (id 0 for empty slots: no divergent loads),
  // loaded before the barrier below
  constexpr int ES = DT == LPS_DTYPE_F32 ? 4 : 2;
  uint32_t hraw[HPT_];
  int hid[HPT_];
  uint32_t hct[HPT_];
  const int nhl = (pen && !defer_hist) ? S.mi[3] : 0;
#pragma unroll
  for (int q = 0; q < HPT_; q++) {
    const int e = tid + q * SNT;
    const uint32_t ent = e < nhl ? S.hl[e] : 0u;
    hid[q] = e < nhl ? (int)(ent & 0x3FFFFu) : -1;
    hct[q] = ent >> 18;
    const int64_t o = (int64_t)max(hid[q], 0) * ES;
    if constexpr (ES == 4) hraw[q] = *reinterpret_cast<const uint32_t*>(row + o);
    else hraw[q] = *reinterpret_cast<const unsigned short*>(row + o);
  }
  // the wave's final share: its ceil(k'/8)-th largest buffered logit (the
  // wave has at least that many own logits at or above it, whatever its
  // threshold was), which raises the joint threshold and so cuts the pool;
  // computed while the other waves finish their chunks
  if (kc > 0 && !over) {
    const int nn = (int)min(nseg, (uint32_t)SEG);
    uint32_t kv[SEG / 64];
#pragma unroll
    for (int q = 0; q < SEG / 64; q++) {
      const int e = lane + 64 * q;
      kv[q] = e < nn ? f2key(__uint_as_float(S.b.seg.x[wv][e])) : 0u;
    }
    const float share = key_threshold(wave_kth_largest<SEG / 64>(kv, (uint32_t)((kc + SNW - 1) / SNW)), greedy, T);
    if (lane == 0) S.segjt[wv] = fmaxf(S.segjt[wv], share);
  }
  // greedy rows: the first index of the thread's maximum, from its first tile holding it
  if (greedy && bt >= 0) {
    load_tile(b0, a0, bt);
    float x[NE];
    unpack_tile(b0, a0, bt, x);
#pragma unroll
    for (int s = NE - 1; s >= 0; s--)
      if (x[s] == bx) bi = vid(bt, s);
  }
  if (lane == 0) {
    S.segn[wv] = over ? SEG + 1 : (int)nseg;
    S.segth[wv] = theta;
  }
  __syncthreads();
  // theta*: the largest own threshold, or the joint one when larger
  float ths = joint_threshold(S);
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

  RG_STAMP(3);
  // ---- history ids: mask, penalise, fold in ----
  uint32_t hx[HPT_];
  bool hk[HPT_];
#pragma unroll
  for (int q = 0; q < HPT_; q++) {
    const int id = hid[q];
    hk[q] = false;
    hx[q] = 0u;
    if (id >= 0) {
      float xv = ES == 4 ? __uint_as_float(hraw[q])
                         : (DT == LPS_DTYPE_BF16 ? __uint_as_float(hraw[q] << 16) : f16_to_f32(hraw[q]));
      if (!id_allowed(am, id)) xv = -INFINITY;
      xv = penalize(xv, (int)hct[q], g.rep, g.pres, g.freq);
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
  // maximum and first argmax, first NaN, logprob reference: one barrier
  const uint64_t bk = ((uint64_t)f2key(bx) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)bi);
  {
    const uint64_t wk = wreduce(bk, OpMax{});
    const int wn = wreduce(nanidx, OpMin{});
    const float wr = wreduce(ref, OpMax{});
    if (lane == 0) {
      S.q[wv] = wk;
      S.i1[wv] = wn;
      S.rf[wv] = wr;
    }
  }
  __syncthreads();
  uint64_t rk = S.q[0];
  int nanr = S.i1[0];
  float R = S.rf[0];
#pragma unroll
  for (int w = 1; w < SNW; w++) {
    rk = max(rk, S.q[w]);
    nanr = min(nanr, S.i1[w]);
    R = fmaxf(R, S.rf[w]);
  }
  float xmax = key2f((uint32_t)(rk >> 32));
  int gam = key_index(rk);
  if (nanr != 0x7FFFFFFF) {
    xmax = __uint_as_float(0x7FC00000u);
    gam = nanr;
  }
  const bool xfin = xmax == xmax && xmax != INFINITY && xmax != -INFINITY;
  double Z = 0.0;
  if (want_lp) {
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

  RG_STAMP(4);
  // ---- pool, part 2: keys (z descending, index ascending); every segment
  // entry was read before the barriers of the reductions above ----
  const float Rm = xfin ? ceilf(__fmul_rn(xmax, c)) : 0.0f;
  int n = 0;
  if (reason == 0 && kc > 0) {
#pragma unroll
    for (int q = 0; q < PPT; q++)
      if (pk[q]) {
        const int p = atomicAdd(&S.pn, 1);
        S.b.ck[p] = cand_key(__uint_as_float(px[q]), pi[q], greedy, T);
        S.cx[p] = px[q];
      }
#pragma unroll
    for (int q = 0; q < HPT_; q++)
      if (hk[q]) {
        const int p = atomicAdd(&S.pn, 1);
        if (p < POOL) {
          S.b.ck[p] = cand_key(__uint_as_float(hx[q]), hid[q], greedy, T);
          S.cx[p] = hx[q];
        }
      }
    __syncthreads();
    n = S.pn;
    if (n > POOL) reason = 16;
  }
  if (reason == 0 && kc > 0 && n > KM / 2) {
    // cut the pool again: every wave's slice keeps its kc-th largest z and
    // above, so the largest slice threshold bounds the row's kc-th largest
    uint64_t kk[PPT];
    uint32_t kz[PPT], kx[PPT];
#pragma unroll
    for (int q = 0; q < PPT; q++) {
      const int e = wv * 64 * PPT + q * 64 + lane;
      kk[q] = e < n ? S.b.ck[e] : 0ull;
      kz[q] = e < n ? key_z(kk[q]) : 0u;
      kx[q] = e < n ? S.cx[e] : 0u;
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
      if (e < n && kz[q] >= zth) {
        S.cx[pos] = kx[q];
        S.b.ck[pos++] = kk[q];
      }
    }
    __syncthreads();
    n = (int)tot;
  }
  if (reason == 0 && kc > 0 && n > KM) reason = 16;

  RG_STAMP(5);
  // ---- rank sort: each wave ranks 64 entries at a time against every key ----
  if (reason == 0 && kc > 0) {
    if (tid < 8 && n + tid < ((n + 7) & ~7)) S.b.ck[n + tid] = 0ull;  // (n <= KM < POOL)
    __syncthreads();
    for (int e0 = wv * 64; e0 < n; e0 += SNT) {
      const int e = e0 + lane;
      const uint64_t key = e < n ? S.b.ck[e] : 0ull;
      // (eight keys per step, read as four 16-byte broadcasts issued together;
      // the pool is padded with zero keys up to a multiple of 8, none of which
      // ranks above an entry)
      int rank = 0;
      const uint4* k4 = reinterpret_cast<const uint4*>(S.b.ck);
      for (int q = 0; q < n; q += 8) {
        uint4 w[4];
#pragma unroll
        for (int j = 0; j < 4; j++) w[j] = k4[(q >> 1) + j];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const uint64_t a0 = ((uint64_t)w[j].y << 32) | w[j].x, a1 = ((uint64_t)w[j].w << 32) | w[j].z;
          rank += (a0 > key ? 1 : 0) + (a1 > key ? 1 : 0);
        }
      }
      if (e < n) {
        S.a.s.sk[rank] = key;
        S.a.s.sm[rank] = zmass_fix(key2f(key_z(key)), Rm);
        S.a.s.sx[rank] = S.cx[e];
      }
    }
  }
  __syncthreads();
  if (reason) {
    if (tid == 0) F.status[r] = LPS_ROW_DEFERRED | (reason << 8);
    return;
  }
  RG_STAMP(6);
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
  RG_STAMP(7);
  int64_t token = status ? -1 : d.token;
  if (row_skips_draw(P, r) && !greedy) token = -1;
  double lnZ = 0.0;
  if (want_lp && Z > 0.0) lnZ = log(Z) + (double)R * 0.6931471805599453;
  // logprobs from the logits' masses in the row mass's own arithmetic
  // (exp2(x c) against R): exact to rounding also where x c is large, which
  // z - lnZ is not (the rounding of c moves x c by ~1e-7 of it)
  auto lprob = [&](float xv, float zv) -> float {
    if (xv == xv && xv != INFINITY && xv != -INFINITY)
      return (float)((double)__builtin_fmaf(xv, c, -R) * 0.6931471805599453 - (lnZ - (double)R * 0.6931471805599453));
    return (float)((double)zv - lnZ);
  };
  if (P.chosen_logprob && tid == 0) {
    float lp = NAN;
    const float cx = greedy ? xmax : (d.pos >= 0 ? __uint_as_float(S.a.s.sx[d.pos]) : NAN);
    if (token >= 0 && Z > 0.0 && d.chosen_z == d.chosen_z) lp = lprob(cx, d.chosen_z);
    P.chosen_logprob[r] = lp;
  }
  if (g.ntop > 0 && status == 0) {
    for (int q = tid; q < P.n_top; q += 64) {  // n_top <= 64: wave 0
      if (q < d.ntop_out) {
        const uint64_t kk = S.a.s.sk[q];
        P.top_logprobs[(int64_t)r * P.n_top + q] = lprob(__uint_as_float(S.a.s.sx[q]), key2f(key_z(kk)));
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
  RG_STAMP(8);
}

}  // namespace st
}  // namespace lps
