// Speculative-decoding kernels: the batched accept test of
// verify_drafts_batched (src/llm_pipeline/inference/speculative_kernel.py:24-87)
// and the per-request epilogue of the accept / reject / resample block
// (src/llm_pipeline/inference/speculative.py:119-174).
#pragma once

#include "lps_generic.h"

namespace lps {

// torch.clamp semantics: NaN propagates (fminf / fmaxf would drop it).
__device__ __forceinline__ float spec_ratio(float p, float q) {
  const float qc = q < 1e-9f ? 1e-9f : q;
  const float r = __fdiv_rn(p, qc);
  return r > 1.0f ? 1.0f : r;
}

// accept[i] = u[i] < min(p[i, tok[i]] / max(q[i], 1e-9), 1)   (speculative_kernel.py:61-87)
template <int DT>
__global__ __launch_bounds__(256) void verify_drafts_kernel(const void* tp, int64_t K, int64_t V, int64_t sk,
                                                            int64_t sv, const float* q, const int64_t* tok,
                                                            const float* u, int8_t* out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= K) return;
  const int64_t t = tok[i];
  const float p = (t >= 0 && t < V) ? load1<DT>(tp, i * sk + t * sv) : 0.0f;
  out[i] = (int8_t)(u[i] < spec_ratio(p, q[i]) ? 1 : 0);
}

// One thread per request: accept bits for every position (as
// verify_drafts_batched computes them), the first rejection j, the accepted
// drafts, then the replacement (target draw at j) or the bonus (target draw at
// k); greedy (T <= 0) accepts iff the target one-hot is 1 at the draft token
// (speculative.py:130-132).
__global__ __launch_bounds__(256) void spec_epilogue_kernel(int B, int k, float T, const float* p_t, const float* q_d,
                                                            const int64_t* draws_t, const int64_t* draft_tokens,
                                                            const float* u_acc, int32_t* n_acc, int64_t* tokens,
                                                            int8_t* accept, float* p_out, float* q_out, int leviathan,
                                                            int32_t* first_rej) {
  const int b = blockIdx.x * 256 + threadIdx.x;
  if (b >= B) return;
  (void)leviathan;
  int j = k;
  for (int i = 0; i < k; i++) {
    const float p = p_t[(int64_t)b * (k + 1) + i];
    const float q = q_d[(int64_t)b * k + i];
    bool acc;
    if (!(T > 0.0f)) acc = p == 1.0f;
    else acc = u_acc[(int64_t)b * k + i] < spec_ratio(p, q);
    if (accept) accept[(int64_t)b * k + i] = acc ? 1 : 0;
    if (p_out) p_out[(int64_t)b * k + i] = p;
    if (q_out) q_out[(int64_t)b * k + i] = q;
    if (!acc && j == k) j = i;
  }
  n_acc[b] = j;
  first_rej[b] = j;
  for (int i = 0; i <= k; i++) {
    int64_t t = -1;
    if (i < j) t = draft_tokens[(int64_t)b * k + i];
    else if (i == j) t = draws_t[(int64_t)b * (k + 1) + i];
    tokens[(int64_t)b * (k + 1) + i] = t;
  }
}

// Kept-set membership of one element under a row plan, given its tie rank.
__device__ __forceinline__ bool plan_kept(const RowPlan& pl, uint32_t key, uint32_t rank) {
  return key > pl.key_lo || (key == pl.key_lo && (pl.n_tie == kNoTie || rank < pl.n_tie));
}

// Leviathan residual: one workgroup per request whose first rejection j < k;
// draws from norm(max(p_j - q_j, 0)) with the position's resample uniform.
// p and q are the kept distributions the row kernel planned (same keys, tie
// ranks and fixed-point masses).  A zero residual keeps the target draw the
// epilogue already wrote.
template <int DT, int VEC>
__global__ __launch_bounds__(GEN_NT) void residual_kernel(const void* tl, int64_t tsb, int64_t tsk, const void* dl,
                                                          int64_t dsb, int64_t dsk, int B, int k, int V,
                                                          const RowPlan* plans, const int32_t* first_rej,
                                                          const float* u_res, int64_t* tokens) {
  __shared__ GenShared S;
  const int b = blockIdx.x;
  const int j = first_rej[b];
  if (j >= k) return;
  S.nth = GEN_NT;  // (every thread stores the same value before its first use)
  constexpr int ES = DT == LPS_DTYPE_F32 ? 4 : 2;
  const void* trow = reinterpret_cast<const char*>(tl) + ES * ((int64_t)b * tsb + (int64_t)j * tsk);
  const void* drow = reinterpret_cast<const char*>(dl) + ES * ((int64_t)b * dsb + (int64_t)j * dsk);
  const RowPlan pt = plans[(int64_t)b * (k + 1) + j];
  const RowPlan pd = plans[(int64_t)B * (k + 1) + (int64_t)b * k + j];
  const int tid = threadIdx.x;
  const double it = 1.0 / (double)pt.Zf, id = 1.0 / (double)pd.Zf;

  // per-thread residual masses of one tile; returns the thread's sum
  auto tile_res = [&](int64_t i0, uint32_t trank, uint32_t drank, double (&rr)[VEC]) {
    double s = 0.0;
    float xt[VEC], xd[VEC];
    loadv<DT, VEC>(trow, i0, xt);
    loadv<DT, VEC>(drow, i0, xd);
#pragma unroll
    for (int e = 0; e < VEC; e++) {
      const float zt = __fdiv_rn(xt[e], pt.T), zd = __fdiv_rn(xd[e], pd.T);
      const uint32_t kt = f2key(zt), kd = f2key(zd);
      const bool ktk = plan_kept(pt, kt, trank), kdk = plan_kept(pd, kd, drank);
      trank += kt == pt.key_lo ? 1u : 0u;
      drank += kd == pd.key_lo ? 1u : 0u;
      const double p = ktk ? (double)mass_fixed(mass_f(zt, pt.zmax)) * it : 0.0;
      const double q = kdk ? (double)mass_fixed(mass_f(zd, pd.zmax)) * id : 0.0;
      rr[e] = p > q ? p - q : 0.0;
      s += rr[e];
    }
    return s;
  };
  auto ties = [&](int64_t i0, const void* row, const RowPlan& pl) {
    uint32_t n = 0;
    float x[VEC];
    loadv<DT, VEC>(row, i0, x);
#pragma unroll
    for (int e = 0; e < VEC; e++) n += f2key(__fdiv_rn(x[e], pl.T)) == pl.key_lo ? 1u : 0u;
    return n;
  };

  // pass 1: total residual mass
  double tot = 0.0;
  uint32_t trun = 0, drun = 0;
  for (int64_t tile = 0; tile < V; tile += (int64_t)GEN_NT * VEC) {
    const int64_t i0 = tile + (int64_t)tid * VEC;
    uint32_t nt = 0, nd = 0;
    if (i0 < V) { nt = ties(i0, trow, pt); nd = ties(i0, drow, pd); }
    uint32_t tt, td;
    const uint32_t et = gblock_excl_scan<uint32_t>(nt, &tt, S.red32, GEN_NT);
    const uint32_t ed = gblock_excl_scan<uint32_t>(nd, &td, S.red32, GEN_NT);
    if (i0 < V) {
      double rr[VEC];
      tot += tile_res(i0, trun + et, drun + ed, rr);
    }
    trun += tt;
    drun += td;
  }
  const double R = gblock_sum_f64(tot, S);
  if (!(R > 0.0)) return;
  float u = u_res[(int64_t)b * (k + 1) + j];
  if (!(u >= 0.0f)) u = 0.0f;
  if (u >= 1.0f) u = 0.99999994f;
  const double target = (double)u * R;

  // pass 2: first index whose cumulative residual exceeds u * R
  if (tid == 0) S.misc[1] = -1;
  __syncthreads();
  double run = 0.0;
  trun = drun = 0;
  int last_pos = -1;
  for (int64_t tile = 0; tile < V; tile += (int64_t)GEN_NT * VEC) {
    const int64_t i0 = tile + (int64_t)tid * VEC;
    uint32_t nt = 0, nd = 0;
    if (i0 < V) { nt = ties(i0, trow, pt); nd = ties(i0, drow, pd); }
    uint32_t tt, td;
    const uint32_t et = gblock_excl_scan<uint32_t>(nt, &tt, S.red32, GEN_NT);
    const uint32_t ed = gblock_excl_scan<uint32_t>(nd, &td, S.red32, GEN_NT);
    double rr[VEC];
    double s = 0.0;
    if (i0 < V) s = tile_res(i0, trun + et, drun + ed, rr);
    double btot;
    const double bex = gblock_excl_scan<double>(s, &btot, S.redd, GEN_NT);
    if (i0 < V && s > 0.0 && run + bex <= target && target < run + bex + s) {
      double a = run + bex;
#pragma unroll
      for (int e = 0; e < VEC; e++) {
        if (rr[e] > 0.0 && a <= target && target < a + rr[e]) S.misc[1] = (int)(i0 + e);
        a += rr[e];
      }
    }
    if (i0 < V) {
#pragma unroll
      for (int e = 0; e < VEC; e++) last_pos = rr[e] > 0.0 ? (int)(i0 + e) : last_pos;
    }
    __syncthreads();
    const int found = S.misc[1];
    __syncthreads();
    if (found >= 0) {
      if (tid == 0) tokens[(int64_t)b * (k + 1) + j] = found;
      return;
    }
    run += btot;
    trun += tt;
    drun += td;
  }
  // u * R rounded past the last positive residual: take the last one
  const uint64_t lp = gblock_max_u64((uint64_t)(uint32_t)(last_pos + 1), S);
  if (tid == 0 && lp > 0) tokens[(int64_t)b * (k + 1) + j] = (int64_t)lp - 1;
}

inline hipError_t launch_residual(int dtype, bool vec, const void* tl, int64_t tsb, int64_t tsk, const void* dl,
                                  int64_t dsb, int64_t dsk, int B, int k, int V, const RowPlan* plans,
                                  const int32_t* first_rej, const float* u_res, int64_t* tokens, hipStream_t s) {
#define LPS_RES(DT, VEC)                                                                                        \
  hipLaunchKernelGGL((residual_kernel<DT, VEC>), dim3(B), dim3(GEN_NT), 0, s, tl, tsb, tsk, dl, dsb, dsk, B, k, V, \
                     plans, first_rej, u_res, tokens)
  switch (dtype) {
    case LPS_DTYPE_F32: if (vec) LPS_RES(LPS_DTYPE_F32, 4); else LPS_RES(LPS_DTYPE_F32, 1); break;
    case LPS_DTYPE_BF16: if (vec) LPS_RES(LPS_DTYPE_BF16, 8); else LPS_RES(LPS_DTYPE_BF16, 1); break;
    default: if (vec) LPS_RES(LPS_DTYPE_F16, 8); else LPS_RES(LPS_DTYPE_F16, 1); break;
  }
#undef LPS_RES
  return hipGetLastError();
}

}  // namespace lps
