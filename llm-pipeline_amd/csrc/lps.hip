// C ABI of the lps token sampler (declarations and reference citations are in
// include/lps.h).  Launches only; no allocation, no synchronisation.  The only
// process-wide state is per-device and write-once: the CU count of each device
// (atomic entries) and the no-allocation entry point's workspace address
// (std::call_once per device).
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

#include "lps_rowgroup.h"
#include "lps_stream.h"
#include "lps_generic.h"
#include "lps_lmhead.h"
#include "lps_softmax.h"
#include "lps_spec.h"

using namespace lps;

namespace {

constexpr int kMaxVocab = (1 << 19) - 1;  // fixed-point masses: V * 2^44 < 2^63

template <int DT, int VEC>
hipError_t launch_gen(const KParams& P, hipStream_t s) {
  hipLaunchKernelGGL((gen_row_kernel<DT, VEC>), dim3(P.R), dim3(GEN_NT), 0, s, P);
  return hipGetLastError();
}

hipError_t dispatch_gen(int dtype, bool vec, const KParams& P, hipStream_t s) {
  switch (dtype) {
    case LPS_DTYPE_F32: return vec ? launch_gen<LPS_DTYPE_F32, 4>(P, s) : launch_gen<LPS_DTYPE_F32, 1>(P, s);
    case LPS_DTYPE_BF16: return vec ? launch_gen<LPS_DTYPE_BF16, 8>(P, s) : launch_gen<LPS_DTYPE_BF16, 1>(P, s);
    default: return vec ? launch_gen<LPS_DTYPE_F16, 8>(P, s) : launch_gen<LPS_DTYPE_F16, 1>(P, s);
  }
}

// 16-byte vector loads are legal when every row start is 16-byte aligned and V
// is a whole number of vectors.
bool vec_ok(const void* base, int dtype, int V, int rows_inner, int64_t so, int64_t si) {
  const int vec = dtype == LPS_DTYPE_F32 ? 4 : 8;
  if (reinterpret_cast<uintptr_t>(base) % 16) return false;
  if (V % vec) return false;
  if (so % vec) return false;
  if (rows_inner > 1 && si % vec) return false;
  return true;
}

bool dtype_ok(int d) { return d == LPS_DTYPE_F32 || d == LPS_DTYPE_BF16 || d == LPS_DTYPE_F16; }

size_t round_up(size_t x, size_t m) { return (x + m - 1) / m * m; }

// Row-group workspace: per-row counters (a fixed region at offset 0, so a
// workspace reused for any (rows, vocab) keeps them apart from the data: the
// arrival and barrier counts are zero between launches, every launch leaves
// them zero; the row's launch epoch only grows), row status, chunk summaries,
// histogram exchange and candidates.
struct RgWs {
  uint32_t* counters;
  int32_t* status;
  rg::RgSum* sums;
  float* hist;
  float* fine;
  uint4* cands;
  size_t bytes;
};

// Rows per row-group launch; larger batches are split into launches.
constexpr int RG_MAX_ROWS = 1024;

// CUs of the current device (cached per device): one resident round of
// row-group workgroups.
// (threads that race on a device's first call each store the same value)
std::atomic<int> g_cus[64];
int device_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int c = g_cus[dev].load(std::memory_order_relaxed);
  if (!c) {
    int n = 0;
    c = (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0) ? n : 256;
    g_cus[dev].store(c, std::memory_order_relaxed);
  }
  return c;
}

// Whether a launch needs the row-group kernel's build with the extra features:
// the entropy output, the mass-only path for pure rows without a draw (top_p
// >= 1 by default or per row), min-p / typical-p rows without top-k and rows
// with top_k past FAST_KMAX (unless no row can have them: per-row arrays
// absent and the defaults off, or the caller's hint).
bool rg_wants_xf(const KParams& k, int flags) {
  const bool mt = !(flags & LPS_FLAG_ROWS_BASIC_FILTERS) &&
                  (k.min_p != nullptr || k.min_p_def > 0.0f || k.typical_p != nullptr || k.typical_p_def < 1.0f ||
                   k.top_k != nullptr || k.top_k_def > rg::FAST_KMAX);
  return k.entropy || mt || ((k.skip_draw || (k.logits2 && k.skip_draw2)) && (k.top_p != nullptr || !(k.top_p_def < 1.0f)));
}

// Launch shape of the row-group kernel for a batch: logits per thread (NE) of
// the instantiated variants, chunks per row (G <= MAXG), vectors per chunk.
struct RgPlan {
  int vpe, ne, G, cv, nvec, capw;
  bool ok;
};
RgPlan rg_plan(int dtype, bool vec, int R, int V, bool lean = false) {
  RgPlan p{};
  p.vpe = !vec ? 1 : (dtype == LPS_DTYPE_F32 ? 4 : 8);
  p.nvec = V / p.vpe;
  auto chunks = [&](int ne) { return (p.nvec + rg::NT * (ne / p.vpe) - 1) / (rg::NT * (ne / p.vpe)); };
  // rows of small batches (fp32: up to 16 rows, 16-bit: up to 12): 24
  // logits per thread, so a row spreads over more workgroups (latency; a
  // 16-bit Qwen3 row: 13 chunks instead of 4); rows read element by element:
  // 40; otherwise 80
  p.ne = p.vpe == 1 ? 40 : ((R <= (p.vpe == 4 ? 16 : 12) && chunks(24) <= rg::MAXG) ? 24 : 80);
  // up to 32 rows: 40 per thread while every chunk still fits one resident
  // round (a Qwen3 row: 8 chunks instead of 4)
  if (p.ne == 80 && R <= 32 && (long)((R + 7) / 8 * 8) * chunks(40) <= (long)device_cus()) p.ne = 40;
  // batches of more than one resident round of workgroups (one per CU), in the
  // build without the extra features: 100 (fp32) or 104 (16-bit) logits per
  // thread when that takes fewer chunks per row (fewer rounds, each a little
  // longer; the other build would spill registers at that size)
  if (lean && p.ne == 80) {
    const int wide = p.vpe == 4 ? 100 : 104;
    if (chunks(wide) < chunks(80) && (long)((R + 7) / 8 * 8) * chunks(80) > (long)device_cus()) p.ne = wide;
  }
  p.G = chunks(p.ne);
  p.ok = p.G >= 1 && p.G <= rg::MAXG && V >= 1;
  p.cv = p.ok ? (p.nvec + p.G - 1) / p.G : 1;
  p.capw = p.ok ? (rg::CAPR / p.G) / rg::NW * rg::NW : 0;
  return p;
}
// The most chunks any dtype's plan uses for (R, V): sizes the workspace.
int rg_max_chunks(int R, int V) {
  int g = 1;
  for (int d = 0; d < 2; d++)
    for (int v = 0; v < 2; v++) {
      const RgPlan p = rg_plan(d == 0 ? LPS_DTYPE_F32 : LPS_DTYPE_BF16, v == 1, R, V);
      if (p.ok && p.G > g) g = p.G;
    }
  return g;
}

// Bytes of the per-row counter region at the workspace's start.
size_t rg_counter_bytes() { return (size_t)RG_MAX_ROWS * 128; }

// Region `off` of the workspace at base (nullptr when only sizes are wanted).
template <typename T>
T* ws_at(void* base, size_t off) {
  return base ? reinterpret_cast<T*>(reinterpret_cast<char*>(base) + off) : nullptr;
}

RgWs rg_layout(void* base, int R, int V) {
  RgWs w{};
  if (R > RG_MAX_ROWS) R = RG_MAX_ROWS;
  const int G = rg_max_chunks(R, V);
  size_t off = 0;
  w.counters = ws_at<uint32_t>(base, off); off = rg_counter_bytes();
  w.status = ws_at<int32_t>(base, off); off = round_up(off + (size_t)R * 4, 256);
  w.sums = ws_at<rg::RgSum>(base, off); off = round_up(off + (size_t)R * 2 * rg::MAXG * sizeof(rg::RgSum), 256);
  w.hist = ws_at<float>(base, off); off = round_up(off + (size_t)R * G * rg::HPUB * 4, 256);
  w.fine = ws_at<float>(base, off); off = round_up(off + (size_t)R * G * rg::FHN * 4, 256);
  w.cands = ws_at<uint4>(base, off); off = round_up(off + (size_t)R * rg::CAPR * 16, 256);
  w.bytes = off;
  return w;
}

template <int DT, int VPE, int NE>
hipError_t launch_rg(rg::RgParams F, int flags, hipStream_t s) {
  const unsigned grid = (unsigned)((F.k.R + 7) / 8 * 8 * F.G);
  // batches of more than one resident round of chunk workgroups: greedy and
  // top-k rows stream through one workgroup each (stream_kernel), the
  // row-group kernel takes the others; the row-kind hints skip a kernel no row
  // needs (a row the hint misjudges is deferred to the general kernel)
  // (with nucleus rows possible the batch may run both kernels, one after
  // the other: the streaming kernel then pays only past 8 rounds; c2's mixed
  // rows at 96 to 640 rows take 54-199 us on the row-group kernel alone,
  // 113-692 us on both)
  bool big = false;
  const unsigned cus = (unsigned)device_cus();
  const unsigned lim = (flags & LPS_FLAG_ROWS_TOPK) ? cus : cus * 8u;
  if constexpr (VPE > 1) big = grid > lim && F.k.V <= rg::STREAM_VMAX;
  const bool run_stream = big && !(flags & LPS_FLAG_ROWS_NUCLEUS);
  const bool run_rg = !(run_stream && (flags & LPS_FLAG_ROWS_TOPK));
  if constexpr (VPE > 1) {
    if (run_stream) {
      F.stream_only = run_rg ? 0 : 1;
      if (F.k.allowed) hipLaunchKernelGGL((st::stream_kernel<DT, VPE, true>), dim3(F.k.R), dim3(st::SNT), 0, s, F);
      else hipLaunchKernelGGL((st::stream_kernel<DT, VPE, false>), dim3(F.k.R), dim3(st::SNT), 0, s, F);
      hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
      F.skip_topk = 1;
    }
  }
  if (run_rg) {
    // the build with the extra features when the launch may need them (the
    // plans of more than 80 logits per thread are made only for the other)
    if (rg_wants_xf(F.k, flags)) {
      if constexpr (NE <= 80) hipLaunchKernelGGL((rg::rowgroup_kernel<DT, VPE, NE, true>), dim3(grid), dim3(rg::NT), 0, s, F);
      else return hipErrorInvalidValue;
    } else {
      hipLaunchKernelGGL((rg::rowgroup_kernel<DT, VPE, NE, false>), dim3(grid), dim3(rg::NT), 0, s, F);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  // the rows the fast kernels deferred: the general algorithm, one
  // 1024-thread workgroup per row (the others return at once)
  KParams G = F.k;
  G.only_status = F.status;
  G.plans = nullptr;
  return launch_gen<DT, VPE == 1 ? 1 : (DT == LPS_DTYPE_F32 ? 4 : 8)>(G, s);
}

template <int DT>
hipError_t dispatch_rg_dt(const rg::RgParams& F, const RgPlan& p, int flags, hipStream_t s) {
  if (p.vpe == 1) return launch_rg<DT, 1, 40>(F, flags, s);
  if constexpr (DT == LPS_DTYPE_F32) {
    if (p.ne == 24) return launch_rg<DT, 4, 24>(F, flags, s);
    if (p.ne == 40) return launch_rg<DT, 4, 40>(F, flags, s);
    if (p.ne == 100) return launch_rg<DT, 4, 100>(F, flags, s);
    return launch_rg<DT, 4, 80>(F, flags, s);
  } else {
    if (p.ne == 24) return launch_rg<DT, 8, 24>(F, flags, s);
    if (p.ne == 40) return launch_rg<DT, 8, 40>(F, flags, s);
    if (p.ne == 104) return launch_rg<DT, 8, 104>(F, flags, s);
    return launch_rg<DT, 8, 80>(F, flags, s);
  }
}

// Per-row pointers of a row block starting at row r0 (a multiple of rows_inner).
KParams row_block(const KParams& P, int r0, int nr, int es) {
  KParams B = P;
  const int64_t g0 = r0 / P.rows_inner;
  B.logits = reinterpret_cast<const char*>(P.logits) + es * g0 * P.stride_outer;
  B.R = nr;
  auto f = [&](const float* p) { return p ? p + r0 : p; };
  B.temperature = f(P.temperature); B.top_p = f(P.top_p); B.min_p = f(P.min_p); B.typical_p = f(P.typical_p);
  B.rep = f(P.rep); B.pres = f(P.pres); B.freq = f(P.freq); B.uniforms = f(P.uniforms);
  B.top_k = P.top_k ? P.top_k + r0 : nullptr;
  B.history = P.history ? P.history + (int64_t)r0 * P.history_stride : nullptr;
  B.history_len = P.history_len ? P.history_len + r0 : nullptr;
  B.query_tokens = P.query_tokens ? P.query_tokens + g0 * P.query_inner : nullptr;
  B.query_prob = P.query_prob ? P.query_prob + r0 : nullptr;
  B.tokens = P.tokens + r0;
  B.chosen_logprob = P.chosen_logprob ? P.chosen_logprob + r0 : nullptr;
  B.top_logprobs = P.top_logprobs ? P.top_logprobs + (int64_t)r0 * P.n_top : nullptr;
  B.top_ids = P.top_ids ? P.top_ids + (int64_t)r0 * P.n_top : nullptr;
  B.entropy = P.entropy ? P.entropy + r0 : nullptr;
  B.row_status = P.row_status ? P.row_status + r0 : nullptr;
  B.kept_cut = P.kept_cut ? P.kept_cut + r0 : nullptr;
  B.kept_ties = P.kept_ties ? P.kept_ties + r0 : nullptr;
  B.kept_count = P.kept_count ? P.kept_count + r0 : nullptr;
  B.row_path = P.row_path ? P.row_path + r0 : nullptr;
  B.plans = P.plans ? P.plans + r0 : nullptr;
  B.allowed = P.allowed ? P.allowed + (int64_t)r0 * P.allowed_stride : nullptr;
  return B;
}

// Runs the row-group kernel (rows it cannot finish exactly go to the general
// kernel launched after it), or only the general kernel when asked or without
// workspace.
// plan_rows: the batch size the launch shape is planned for (the whole batch,
// also for its blocks when it is split, so that every block fits the
// workspace sized for it); 0 = P.R.
hipError_t run_sample(const KParams& P, int dtype, bool vec, void* ws, size_t ws_bytes, int flags, hipStream_t s,
                      int plan_rows = 0) {
  if (plan_rows <= 0) plan_rows = P.R;
  const RgWs need = rg_layout(nullptr, plan_rows, P.V);
  if ((flags & LPS_FLAG_GENERIC) || !ws || ws_bytes < need.bytes) return dispatch_gen(dtype, vec, P, s);
  if (P.R > RG_MAX_ROWS) {
    const int blk = RG_MAX_ROWS / P.rows_inner * P.rows_inner;
    if (blk < 1) return dispatch_gen(dtype, vec, P, s);
    const int es = dtype == LPS_DTYPE_F32 ? 4 : 2;
    for (int r0 = 0; r0 < P.R; r0 += blk) {
      const int nr = P.R - r0 < blk ? P.R - r0 : blk;
      hipError_t e = run_sample(row_block(P, r0, nr, es), dtype, vec, ws, ws_bytes, flags, s, plan_rows);
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  }
  const RgPlan p = rg_plan(dtype, vec, plan_rows, P.V, !rg_wants_xf(P, flags));
  if (!p.ok) return dispatch_gen(dtype, vec, P, s);
  const RgWs w = rg_layout(ws, plan_rows, P.V);
  rg::RgParams F{};
  F.k = P;
  F.G = p.G;
  F.cv = p.cv;
  F.nvec = p.nvec;
  F.heavy_first = 0;
  F.skip_topk = 0;
  F.stream_only = 0;
  F.counters = w.counters;
  F.status = w.status;
  F.sums = w.sums;
  F.hist = w.hist;
  F.fine = w.fine;
  F.cands = w.cands;
  F.capw = p.capw;
  switch (dtype) {
    case LPS_DTYPE_F32: return dispatch_rg_dt<LPS_DTYPE_F32>(F, p, flags, s);
    case LPS_DTYPE_BF16: return dispatch_rg_dt<LPS_DTYPE_BF16>(F, p, flags, s);
    default: return dispatch_rg_dt<LPS_DTYPE_F16>(F, p, flags, s);
  }
}

KParams neutral_params() {
  KParams P{};
  P.rows_inner = 1;
  P.temperature_def = 1.0f;
  P.top_k_def = 0;
  P.top_p_def = 1.0f;
  P.min_p_def = 0.0f;
  P.typical_p_def = 1.0f;
  P.rep_def = 1.0f;
  P.pres_def = 0.0f;
  P.freq_def = 0.0f;
  return P;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct SpecWs {
  void* fast;         // the fast path's workspace (first, so its counters never move)
  size_t fast_bytes;
  int64_t* draws_t;   // [B*(k+1)], then draws_d
  int64_t* draws_d;   // [B*k]
  float* p_t;         // [B*(k+1)], then q_d
  float* q_d;         // [B*k]
  int32_t* first_rej; // [B]
  RowPlan* plans;     // [B*(k+1) + B*k]
  size_t bytes;
};

SpecWs spec_layout(void* base, int B, int k, int V) {
  SpecWs w{};
  const size_t Rt = (size_t)B * (k + 1), Rd = (size_t)B * k;
  w.fast = base;
  w.fast_bytes = rg_layout(nullptr, (int)(Rt + Rd), V).bytes;
  size_t off = align256(w.fast_bytes);
  // (target then draft entries, contiguous: one launch may write both)
  w.draws_t = ws_at<int64_t>(base, off);
  w.draws_d = ws_at<int64_t>(base, off + Rt * 8); off = align256(off + (Rt + Rd) * 8);
  w.p_t = ws_at<float>(base, off);
  w.q_d = ws_at<float>(base, off + Rt * 4); off = align256(off + (Rt + Rd) * 4);
  w.first_rej = ws_at<int32_t>(base, off); off = align256(off + (size_t)B * 4);
  w.plans = ws_at<RowPlan>(base, off); off = align256(off + (Rt + Rd) * sizeof(RowPlan));
  w.bytes = off;
  return w;
}

template <int DT, int VEC>
hipError_t launch_softmax(const SoftmaxParams& S, hipStream_t s) {
  if (S.cols >= 16384) hipLaunchKernelGGL((softmax_kernel<DT, VEC, 1024>), dim3(S.rows), dim3(1024), 0, s, S);
  else hipLaunchKernelGGL((softmax_kernel<DT, VEC, 256>), dim3(S.rows), dim3(256), 0, s, S);
  return hipGetLastError();
}

// Softmax kernel choice for rows whose starts are 16-byte aligned: one wave per
// row (kind 0), G register-resident chunks per row (kind 1), or the three-pass
// kernel (kind 2).  nv = 16-byte vectors per lane.
struct SmPlan {
  int kind, nv, G;
};
SmPlan softmax_plan(int dtype, int rows, int cols) {
  const int vpl = dtype == LPS_DTYPE_F32 ? 4 : 8;
  const int64_t vecs = ((int64_t)cols + vpl - 1) / vpl;  // 16-byte vectors per row
  for (int nv = 1; nv <= 8; nv *= 2)
    if (vecs <= 64 * nv) return {0, nv, 1};
  if (vecs <= SM_NT * 4) return {1, 4, 1};
  if (vecs <= SM_NT * 8) return {1, 8, 1};
  auto chunks = [&](int nv) { return (int)((vecs + (int64_t)SM_NT * nv - 1) / ((int64_t)SM_NT * nv)); };
  if (chunks(8) > SM_MAXG) return {2, 0, 1};
  // 8 vectors per lane (16 KB of 16-bit / 32 KB of fp32 columns per chunk):
  // measured fastest on 64 x 151936 bf16 (4 to 19 vectors swept); smaller
  // chunks only for short grids, down to 4 (more chunks per row cost more in
  // the record exchange than they add in parallelism)
  const int nv = (int64_t)rows * chunks(8) < 256 && chunks(4) <= SM_MAXG ? 4 : 8;
  return {1, nv, chunks(nv)};
}
size_t softmax_records_bytes(int rows, int G) {
  return G > 1 ? (size_t)rows * G * sizeof(SmRecord) + ((size_t)rows * 4 + 255) / 256 * 256 : 0;
}

template <int DT>
hipError_t launch_softmax_reg(const SoftmaxParams& S, const SmPlan& p, hipStream_t s) {
  if (p.kind == 0) {
    const dim3 grid((S.rows + SM_NT / 64 - 1) / (SM_NT / 64));
    switch (p.nv) {
      case 1: hipLaunchKernelGGL((softmax_wave_kernel<DT, 1>), grid, dim3(SM_NT), 0, s, S); break;
      case 2: hipLaunchKernelGGL((softmax_wave_kernel<DT, 2>), grid, dim3(SM_NT), 0, s, S); break;
      case 4: hipLaunchKernelGGL((softmax_wave_kernel<DT, 4>), grid, dim3(SM_NT), 0, s, S); break;
      default: hipLaunchKernelGGL((softmax_wave_kernel<DT, 8>), grid, dim3(SM_NT), 0, s, S); break;
    }
  } else {
    const dim3 grid((unsigned)(((int64_t)S.rows + 7) / 8 * S.G * 8));
    if (p.nv == 4) hipLaunchKernelGGL((softmax_chunk_kernel<DT, 4>), grid, dim3(SM_NT), 0, s, S);
    else hipLaunchKernelGGL((softmax_chunk_kernel<DT, 8>), grid, dim3(SM_NT), 0, s, S);
  }
  return hipGetLastError();
}

// Monotonicity of the hardware exp2 (v_exp_f32) over every non-NaN input:
// thread t checks keys [k0 + 1024 t - 1, k0 + 1024 t + 1024) in float-key
// order (each step against the one before it), counting the steps where the
// result decreases.
constexpr uint32_t kKeyNegInf = 0x007FFFFFu, kKeyPosInf = 0xFF800000u;
__global__ __launch_bounds__(256) void exp2_monotone_kernel(unsigned long long* bad) {
  const uint64_t t = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  const uint64_t k0 = kKeyNegInf + t * 1024u;
  if (k0 > kKeyPosInf) return;
  const uint64_t k1 = k0 + 1024u < (uint64_t)kKeyPosInf + 1u ? k0 + 1024u : (uint64_t)kKeyPosInf + 1u;
  uint32_t n = 0;
  float prev = __builtin_amdgcn_exp2f(key2f((uint32_t)(k0 > kKeyNegInf ? k0 - 1u : k0)));
  for (uint64_t k = k0; k < k1; k++) {
    const float r = __builtin_amdgcn_exp2f(key2f((uint32_t)k));
    n += r < prev ? 1u : 0u;
    prev = r;
  }
  if (n) atomicAdd(bad, (unsigned long long)n);
}

}  // namespace

extern "C" {

int lps_selftest_exp2_monotone(unsigned long long* violations) {
  if (!violations) return LPS_EINVAL;
  unsigned long long* d = nullptr;
  if (hipMalloc(&d, sizeof(*d)) != hipSuccess) return LPS_ELAUNCH;
  hipError_t e = hipMemset(d, 0, sizeof(*d));
  const uint64_t nkeys = (uint64_t)kKeyPosInf - kKeyNegInf + 1u;
  const uint32_t blocks = (uint32_t)((nkeys + 256u * 1024u - 1u) / (256u * 1024u));
  if (e == hipSuccess) {
    hipLaunchKernelGGL(exp2_monotone_kernel, dim3(blocks), dim3(256), 0, 0, d);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipMemcpy(violations, d, sizeof(*d), hipMemcpyDeviceToHost);
  (void)hipFree(d);
  return e == hipSuccess ? LPS_OK : LPS_ELAUNCH;
}

#ifdef LPS_RG_STAMPS
// Timing builds only: copies the phase stamps of the last launches (8192 x 32
// uint64 on the host).
int lps_debug_stamps(uint64_t* host) {
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(rg::rg_stamps), sizeof(uint64_t) * 8192 * 32, 0,
                             hipMemcpyDeviceToHost) == hipSuccess ? 0 : 1;
}
#endif

int lps_version(void) { return LPS_ABI_VERSION; }

const char* lps_status_string(int code) {
  switch (code) {
    case LPS_OK: return "ok";
    case LPS_EINVAL: return "invalid argument";
    case LPS_EUNSUPPORTED_DTYPE: return "unsupported logits dtype";
    case LPS_ELAUNCH: return "kernel launch failed";
    case LPS_EWORKSPACE: return "workspace missing or too small";
    case LPS_ENOALLOC_CAPACITY: return "batch needs more workspace than lps_sample_noalloc holds (LPS_NOALLOC_WORKSPACE_BYTES)";
    default: return "unknown status";
  }
}

size_t lps_workspace_bytes(int num_rows, int vocab, int flags) {
  if (num_rows <= 0 || vocab < 1 || vocab > kMaxVocab || (flags & LPS_FLAG_GENERIC)) return 0;
  return rg_layout(nullptr, num_rows, vocab).bytes;
}

size_t lps_spec_workspace_bytes(int batch, int k, int vocab) {
  if (batch <= 0 || k <= 0 || vocab < 1 || vocab > kMaxVocab) return 0;
  return spec_layout(nullptr, batch, k, vocab).bytes;
}

}  // extern "C"

namespace {

// lps_sample's launches with the workspace ws (the caller's, or the
// no-allocation variant's static one).
int sample_impl(const lps_sample_args* a, void* ws, size_t ws_bytes, void* stream) {
  if (!a) return LPS_EINVAL;
  if (!dtype_ok(a->dtype)) return LPS_EUNSUPPORTED_DTYPE;
  if (a->num_rows < 0 || a->vocab < 1 || a->vocab > kMaxVocab || a->rows_inner < 1) return LPS_EINVAL;
  if (a->num_rows == 0) return LPS_OK;
  if (!a->logits || !a->tokens) return LPS_EINVAL;
  if (a->stride_outer < 0 || a->stride_inner < 0) return LPS_EINVAL;
  if (a->n_top < 0 || a->n_top > LPS_MAX_TOP_LOGPROBS || (a->n_top > 0 && !a->top_logprobs)) return LPS_EINVAL;
  if (!a->uniforms && !a->skip_draw) return LPS_EINVAL;
  if (a->history && (!a->history_len || a->history_stride < 0)) return LPS_EINVAL;
  if (a->query_tokens && (a->query_inner < 0 || a->query_inner > a->rows_inner)) return LPS_EINVAL;
  if (a->allowed && a->allowed_stride < (int64_t)((a->vocab + 31) / 32)) return LPS_EINVAL;
  if ((a->flags & LPS_FLAG_APPEND_HISTORY) && (!a->history || !a->history_len)) return LPS_EINVAL;
  KParams P = neutral_params();
  P.logits = a->logits;
  P.V = a->vocab;
  P.R = a->num_rows;
  P.rows_inner = a->rows_inner;
  P.stride_outer = a->stride_outer;
  P.stride_inner = a->stride_inner;
  P.temperature = a->temperature;
  P.top_k = a->top_k;
  P.top_p = a->top_p;
  P.min_p = a->min_p;
  P.typical_p = a->typical_p;
  P.rep = a->repetition_penalty;
  P.pres = a->presence_penalty;
  P.freq = a->frequency_penalty;
  P.history = a->history;
  P.history_stride = a->history_stride;
  P.history_len = a->history_len;
  P.uniforms = a->uniforms;
  P.query_tokens = a->query_tokens;
  P.query_inner = a->query_tokens ? a->query_inner : 0;
  P.query_prob = a->query_prob;
  P.tokens = a->tokens;
  P.chosen_logprob = a->chosen_logprob;
  P.top_logprobs = a->top_logprobs;
  P.top_ids = a->top_ids;
  P.n_top = a->n_top;
  P.entropy = a->entropy;
  P.row_status = a->row_status;
  P.skip_draw = a->skip_draw;
  P.kept_cut = a->kept_cut;
  P.kept_ties = a->kept_ties;
  P.kept_count = a->kept_count;
  P.plans = nullptr;
  P.only_status = nullptr;
  P.row_path = a->row_path;
  P.allowed = a->allowed;
  P.allowed_stride = a->allowed_stride;
  P.append_history = (a->flags & LPS_FLAG_APPEND_HISTORY) ? 1 : 0;
  if (ws && ws_bytes < lps_workspace_bytes(a->num_rows, a->vocab, a->flags)) return LPS_EWORKSPACE;
  const bool vec = vec_ok(a->logits, a->dtype, a->vocab, a->rows_inner, a->stride_outer, a->stride_inner);
  hipError_t e = run_sample(P, a->dtype, vec, ws, ws_bytes, a->flags, reinterpret_cast<hipStream_t>(stream));
  return e == hipSuccess ? LPS_OK : LPS_ELAUNCH;
}

// ---------------------------------------------------------------------------
// The no-allocation variant's workspace: one array per GPU, for the lifetime
// of the process.  Host code never passes the array's name to a kernel or a
// copy (on the host it is only a stand-in); it uses the device address that
// hipGetSymbolAddress returns for the current device.
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[LPS_NOALLOC_WORKSPACE_BYTES];

constexpr int kMaxDevices = 64;
struct ScratchSlot {
  std::once_flag once;
  void* ptr = nullptr;
  hipError_t err = hipErrorNotInitialized;
};
ScratchSlot g_scratch[kMaxDevices];

// Zeroes n 32-bit words (a kernel rather than hipMemsetAsync, so that a
// first call made under graph capture records no memset node).
__global__ void zero_words_kernel(uint32_t* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// The current device's scratch address (set up on the device's first call:
// the address lookup, then the row counters cleared on `s`, the one region
// the kernels need zero at launch; every launch leaves it zero again).
void* scratch_for_current_device(hipStream_t s, int* rc) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    *rc = LPS_ELAUNCH;
    return nullptr;
  }
  ScratchSlot& slot = g_scratch[dev];
  std::call_once(slot.once, [&] {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e == hipSuccess) {
      const int words = (int)(rg_counter_bytes() / 4);
      hipLaunchKernelGGL(zero_words_kernel, dim3((words + 255) / 256), dim3(256), 0, s, static_cast<uint32_t*>(p),
                         words);
      e = hipGetLastError();
    }
    slot.ptr = e == hipSuccess ? p : nullptr;
    slot.err = e;
  });
  if (slot.err != hipSuccess || !slot.ptr) {
    *rc = LPS_ELAUNCH;
    return nullptr;
  }
  *rc = LPS_OK;
  return slot.ptr;
}

}  // namespace

extern "C" {

int lps_sample(const lps_sample_args* a, void* stream) {
  if (!a) return LPS_EINVAL;
  return sample_impl(a, a->workspace, a->workspace_bytes, stream);
}

int lps_sample_noalloc(const lps_sample_args* a, void* stream) {
  if (!a) return LPS_EINVAL;
  const size_t need = lps_workspace_bytes(a->num_rows, a->vocab, a->flags);
  if (need > (size_t)LPS_NOALLOC_WORKSPACE_BYTES) return LPS_ENOALLOC_CAPACITY;
  if (need == 0) return sample_impl(a, nullptr, 0, stream);  // the general kernel (or nothing) needs no workspace
  int rc = LPS_OK;
  void* ws = scratch_for_current_device(reinterpret_cast<hipStream_t>(stream), &rc);
  if (!ws) return rc;
  return sample_impl(a, ws, LPS_NOALLOC_WORKSPACE_BYTES, stream);
}

int lps_spec_verify(const lps_spec_args* a, void* stream) {
  if (!a) return LPS_EINVAL;
  if (!dtype_ok(a->dtype)) return LPS_EUNSUPPORTED_DTYPE;
  if (a->batch < 0 || a->k < 1 || a->vocab < 1 || a->vocab > kMaxVocab) return LPS_EINVAL;
  if (a->batch == 0) return LPS_OK;
  if (!a->target_logits || !a->draft_logits || !a->draft_tokens || !a->u_accept || !a->u_resample ||
      !a->n_accepted || !a->tokens)
    return LPS_EINVAL;
  if (a->residual != LPS_RESIDUAL_TARGET && a->residual != LPS_RESIDUAL_LEVIATHAN) return LPS_EINVAL;
  const int B = a->batch, k = a->k, V = a->vocab;
  const SpecWs need = spec_layout(nullptr, B, k, V);
  if (!a->workspace || a->workspace_bytes < need.bytes) return LPS_EWORKSPACE;
  const SpecWs w = spec_layout(a->workspace, B, k, V);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool lev = a->residual == LPS_RESIDUAL_LEVIATHAN && a->temperature > 0.0f;

  // target rows: probability of each draft token, and a draw per position
  KParams P = neutral_params();
  P.logits = a->target_logits;
  P.V = V;
  P.R = B * (k + 1);
  P.rows_inner = k + 1;
  P.stride_outer = a->target_stride_b;
  P.stride_inner = a->target_stride_k;
  P.temperature_def = a->temperature;
  P.top_p_def = a->top_p;
  P.uniforms = a->u_resample;
  P.query_tokens = a->draft_tokens;
  P.query_inner = k;
  P.query_prob = w.p_t;
  P.tokens = w.draws_t;
  P.row_status = a->row_status;
  P.plans = w.plans;
  // The Leviathan residual reads the general kernel's per-row plans; otherwise
  // both row sets take the fast kernels (rows they cannot finish exactly go
  // to the general kernel after them), with the same results.
  // Every row shares the temperature and top-p: the row-kind hint that skips
  // the kernel no row needs (T > 0: nucleus or pure rows; else greedy).
  const int hint = a->temperature > 0.0f ? LPS_FLAG_ROWS_NUCLEUS : LPS_FLAG_ROWS_TOPK;
  const int Rt = B * (k + 1), Rd = B * k;
  bool vec = vec_ok(a->target_logits, a->dtype, V, k + 1, a->target_stride_b, a->target_stride_k);
  const bool vec_d = vec_ok(a->draft_logits, a->dtype, V, k, a->draft_stride_b, a->draft_stride_k);
  if (!lev && Rt + Rd <= RG_MAX_ROWS) {
    // both row sets in one launch: the target rows, then the draft rows as
    // the second row segment (their own logits and layout, draws skipped);
    // the outputs of the two sets are contiguous in the workspace
    KParams J = P;
    J.R = Rt + Rd;
    J.R1 = Rt;
    J.logits2 = a->draft_logits;
    J.rows_inner2 = k;
    J.stride_outer2 = a->draft_stride_b;
    J.stride_inner2 = a->draft_stride_k;
    J.skip_draw2 = 1;
    if (run_sample(J, a->dtype, vec && vec_d, w.fast, w.fast_bytes, hint, s) != hipSuccess) return LPS_ELAUNCH;
  } else {
  if ((lev ? dispatch_gen(a->dtype, vec, P, s) : run_sample(P, a->dtype, vec, w.fast, w.fast_bytes, hint, s)) !=
      hipSuccess)
    return LPS_ELAUNCH;

  // draft rows: probability of each draft token only
  KParams D = P;
  D.logits = a->draft_logits;
  D.R = B * k;
  D.rows_inner = k;
  D.stride_outer = a->draft_stride_b;
  D.stride_inner = a->draft_stride_k;
  D.uniforms = nullptr;
  D.query_inner = k;
  D.query_prob = w.q_d;
  D.tokens = w.draws_d;
  D.row_status = a->row_status ? a->row_status + (size_t)B * (k + 1) : nullptr;
  D.skip_draw = 1;
  D.plans = w.plans + (size_t)B * (k + 1);
  // (planned for both row sets' count, for which the workspace is sized)
  if ((lev ? dispatch_gen(a->dtype, vec_d, D, s) : run_sample(D, a->dtype, vec_d, w.fast, w.fast_bytes, hint, s, Rt + Rd)) !=
      hipSuccess)
    return LPS_ELAUNCH;
  }

  hipLaunchKernelGGL(spec_epilogue_kernel, dim3((B + 255) / 256), dim3(256), 0, s, B, k, a->temperature, w.p_t,
                     w.q_d, w.draws_t, a->draft_tokens, a->u_accept, a->n_accepted, a->tokens, a->accept,
                     a->p_target, a->q_draft, lev ? 1 : 0, w.first_rej);
  if (hipGetLastError() != hipSuccess) return LPS_ELAUNCH;
  if (lev) {
    const bool vt = vec_ok(a->target_logits, a->dtype, V, k + 1, a->target_stride_b, a->target_stride_k) &&
                    vec_ok(a->draft_logits, a->dtype, V, k, a->draft_stride_b, a->draft_stride_k);
    if (launch_residual(a->dtype, vt, a->target_logits, a->target_stride_b, a->target_stride_k, a->draft_logits,
                        a->draft_stride_b, a->draft_stride_k, B, k, V, w.plans, w.first_rej, a->u_resample,
                        a->tokens, s) != hipSuccess)
      return LPS_ELAUNCH;
  }
  return LPS_OK;
}

int lps_verify_drafts(const void* target_probs, int32_t dtype, int64_t K, int64_t V, int64_t stride_k,
                      int64_t stride_v, const float* draft_probs, const int64_t* draft_tokens,
                      const float* rand_uniform, int8_t* accept, void* stream) {
  if (!dtype_ok(dtype)) return LPS_EUNSUPPORTED_DTYPE;
  if (K < 0 || V < 1) return LPS_EINVAL;
  if (K == 0) return LPS_OK;
  if (!target_probs || !draft_probs || !draft_tokens || !rand_uniform || !accept) return LPS_EINVAL;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((K + 255) / 256));
  switch (dtype) {
    case LPS_DTYPE_F32:
      hipLaunchKernelGGL((verify_drafts_kernel<LPS_DTYPE_F32>), grid, dim3(256), 0, s, target_probs, K, V, stride_k,
                         stride_v, draft_probs, draft_tokens, rand_uniform, accept);
      break;
    case LPS_DTYPE_BF16:
      hipLaunchKernelGGL((verify_drafts_kernel<LPS_DTYPE_BF16>), grid, dim3(256), 0, s, target_probs, K, V, stride_k,
                         stride_v, draft_probs, draft_tokens, rand_uniform, accept);
      break;
    default:
      hipLaunchKernelGGL((verify_drafts_kernel<LPS_DTYPE_F16>), grid, dim3(256), 0, s, target_probs, K, V, stride_k,
                         stride_v, draft_probs, draft_tokens, rand_uniform, accept);
      break;
  }
  return hipGetLastError() == hipSuccess ? LPS_OK : LPS_ELAUNCH;
}

size_t lps_softmax_workspace_bytes(int rows, int cols, int dtype) {
  if (rows <= 0 || cols < 1 || !dtype_ok(dtype)) return 0;
  const SmPlan p = softmax_plan(dtype, rows, cols);
  return p.kind == 1 ? softmax_records_bytes(rows, p.G) : 0;
}

int lps_lm_head(const lps_lm_head_args* a, void* stream) {
  if (!a) return LPS_EINVAL;
  if (a->dtype != LPS_DTYPE_BF16 && a->dtype != LPS_DTYPE_F16) return LPS_EUNSUPPORTED_DTYPE;
  if (!dtype_ok(a->out_dtype)) return LPS_EUNSUPPORTED_DTYPE;
  if (a->rows < 0 || a->vocab < 1 || a->hidden < 16 || a->hidden % 16) return LPS_EINVAL;
  if (a->rows == 0) return LPS_OK;
  if (!a->x || !a->w || !a->out) return LPS_EINVAL;
  if (a->x_stride < a->hidden || a->w_stride < a->hidden || (a->rows > 1 && a->out_stride < a->vocab)) return LPS_EINVAL;
  // 16-byte operand loads: x and w rows start 16-byte aligned
  if (reinterpret_cast<uintptr_t>(a->x) % 16 || reinterpret_cast<uintptr_t>(a->w) % 16 || a->x_stride % 8 ||
      a->w_stride % 8)
    return LPS_EINVAL;
  if ((a->rows + LMH_BM - 1) / LMH_BM > 65535) return LPS_EINVAL;   // grid y
  LmHeadParams P{};
  P.x = a->x;
  P.w = a->w;
  P.out = a->out;
  P.stats = a->stats;
  P.M = a->rows;
  P.V = a->vocab;
  P.H = a->hidden;
  P.x_stride = a->x_stride;
  P.w_stride = a->w_stride;
  P.out_stride = a->rows > 1 ? a->out_stride : a->vocab;
  P.G = (a->vocab + LMH_BN - 1) / LMH_BN;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)P.G, (unsigned)((a->rows + LMH_BM - 1) / LMH_BM));
#define LMH_LAUNCH(DT, ODT) hipLaunchKernelGGL((lmhead_kernel<DT, ODT, LMH_KC, LMH_NB>), grid, dim3(256), 0, s, P)
  if (a->dtype == LPS_DTYPE_BF16) {
    if (a->out_dtype == LPS_DTYPE_BF16) LMH_LAUNCH(LPS_DTYPE_BF16, LPS_DTYPE_BF16);
    else if (a->out_dtype == LPS_DTYPE_F16) LMH_LAUNCH(LPS_DTYPE_BF16, LPS_DTYPE_F16);
    else LMH_LAUNCH(LPS_DTYPE_BF16, LPS_DTYPE_F32);
  } else {
    if (a->out_dtype == LPS_DTYPE_BF16) LMH_LAUNCH(LPS_DTYPE_F16, LPS_DTYPE_BF16);
    else if (a->out_dtype == LPS_DTYPE_F16) LMH_LAUNCH(LPS_DTYPE_F16, LPS_DTYPE_F16);
    else LMH_LAUNCH(LPS_DTYPE_F16, LPS_DTYPE_F32);
  }
#undef LMH_LAUNCH
  return hipGetLastError() == hipSuccess ? LPS_OK : LPS_ELAUNCH;
}

int lps_softmax(const lps_softmax_args* a, void* stream) {
  if (!a) return LPS_EINVAL;
  if (!dtype_ok(a->dtype)) return LPS_EUNSUPPORTED_DTYPE;
  if (a->rows < 0 || a->cols < 1) return LPS_EINVAL;
  if (a->rows == 0) return LPS_OK;
  if (!a->x || !a->out) return LPS_EINVAL;
  if (a->rows > 1 && (a->x_stride < a->cols || a->out_stride < a->cols)) return LPS_EINVAL;
  if (a->causal && a->seq_len < 1) return LPS_EINVAL;
  SoftmaxParams S{};
  S.x = a->x;
  S.out = a->out;
  S.x_stride = a->x_stride;
  S.out_stride = a->out_stride;
  S.rows = a->rows;
  S.cols = a->cols;
  S.causal = a->causal ? 1 : 0;
  S.seq_len = a->causal ? a->seq_len : 1;
  S.row_offset = a->row_offset;
  S.row_lse = a->row_lse;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t e;
  // register-resident kernels: every row of x and out starts 16-byte aligned
  const int vpl = a->dtype == LPS_DTYPE_F32 ? 4 : 8;
  auto aligned = [&](const void* p, int64_t stride) {
    return reinterpret_cast<uintptr_t>(p) % 16 == 0 && (a->rows <= 1 || stride % vpl == 0);
  };
  if (a->row_stats) {
    // one streaming pass from the producer's block statistics
    const int nstats = a->stats_cols > 0 ? (int)(((int64_t)a->cols + a->stats_cols - 1) / a->stats_cols) : 0;
    if (a->causal || a->stats_cols < 1 || (a->rows > 1 && a->stats_stride < 2 * (int64_t)nstats)) return LPS_EINVAL;
    if (aligned(a->x, a->x_stride) && aligned(a->out, a->out_stride)) {
      const int64_t vecs = ((int64_t)a->cols + vpl - 1) / vpl;
      const int nv = vecs > (int64_t)SM_NT * 2 ? 8 : 2;
      S.G = (int)((vecs + (int64_t)SM_NT * nv - 1) / ((int64_t)SM_NT * nv));
      S.row_stats = a->row_stats;
      S.stats_stride = a->rows > 1 ? a->stats_stride : 2 * (int64_t)nstats;
      S.nstats = nstats;
      const dim3 grid((unsigned)(((int64_t)S.rows + 7) / 8 * S.G * 8));
#define SMA_LAUNCH(DT)                                                                       \
  do {                                                                                       \
    if (nv == 8) hipLaunchKernelGGL((softmax_apply_kernel<DT, 8>), grid, dim3(SM_NT), 0, s, S); \
    else hipLaunchKernelGGL((softmax_apply_kernel<DT, 2>), grid, dim3(SM_NT), 0, s, S);         \
  } while (0)
      switch (a->dtype) {
        case LPS_DTYPE_F32: SMA_LAUNCH(LPS_DTYPE_F32); break;
        case LPS_DTYPE_BF16: SMA_LAUNCH(LPS_DTYPE_BF16); break;
        default: SMA_LAUNCH(LPS_DTYPE_F16); break;
      }
#undef SMA_LAUNCH
      e = hipGetLastError();
      return e == hipSuccess ? LPS_OK : LPS_ELAUNCH;
    }
  }
  if (aligned(a->x, a->x_stride) && aligned(a->out, a->out_stride)) {
    SmPlan p = softmax_plan(a->dtype, a->rows, a->cols);
    if (p.kind == 1 && p.G > 1) {
      // split rows need the workspace, and distinct input and output (a
      // workgroup that falls back re-reads its whole row)
      const int es = a->dtype == LPS_DTYPE_F32 ? 4 : 2;
      const char* x0 = static_cast<const char*>(a->x);
      const char* o0 = static_cast<const char*>(a->out);
      const int64_t xs = a->rows > 1 ? a->x_stride : a->cols, os = a->rows > 1 ? a->out_stride : a->cols;
      const char* x1 = x0 + ((int64_t)(a->rows - 1) * xs + a->cols) * es;
      const char* o1 = o0 + ((int64_t)(a->rows - 1) * os + a->cols) * es;
      const bool overlap = x0 < o1 && o0 < x1;
      const size_t need = softmax_records_bytes(a->rows, p.G);
      if (overlap || !a->workspace || a->workspace_bytes < need) {
        p.kind = 2;
      } else {
        S.G = p.G;
        S.records = a->workspace;
        S.done = reinterpret_cast<uint32_t*>(static_cast<char*>(a->workspace) + (size_t)a->rows * p.G * sizeof(SmRecord));
      }
    } else {
      S.G = 1;
    }
    if (p.kind != 2) {
      switch (a->dtype) {
        case LPS_DTYPE_F32: e = launch_softmax_reg<LPS_DTYPE_F32>(S, p, s); break;
        case LPS_DTYPE_BF16: e = launch_softmax_reg<LPS_DTYPE_BF16>(S, p, s); break;
        default: e = launch_softmax_reg<LPS_DTYPE_F16>(S, p, s); break;
      }
      return e == hipSuccess ? LPS_OK : LPS_ELAUNCH;
    }
  }
  // three passes; 16-byte vectors when both rows start 16-byte aligned and cols fill whole vectors
  const bool vec = vec_ok(a->x, a->dtype, a->cols, 1, a->rows > 1 ? a->x_stride : 0, 0) &&
                   vec_ok(a->out, a->dtype, a->cols, 1, a->rows > 1 ? a->out_stride : 0, 0);
  switch (a->dtype) {
    case LPS_DTYPE_F32: e = vec ? launch_softmax<LPS_DTYPE_F32, 4>(S, s) : launch_softmax<LPS_DTYPE_F32, 1>(S, s); break;
    case LPS_DTYPE_BF16: e = vec ? launch_softmax<LPS_DTYPE_BF16, 8>(S, s) : launch_softmax<LPS_DTYPE_BF16, 1>(S, s); break;
    default: e = vec ? launch_softmax<LPS_DTYPE_F16, 8>(S, s) : launch_softmax<LPS_DTYPE_F16, 1>(S, s); break;
  }
  return e == hipSuccess ? LPS_OK : LPS_ELAUNCH;
}

}  // extern "C"
