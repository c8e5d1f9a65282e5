// Host build of the lps C ABI (llm-pipeline_amd/csrc/lps.hip, unchanged) over
// the HIP emulation in shim/hip/hip_runtime.h, under AddressSanitizer and
// UndefinedBehaviorSanitizer (array bounds included): test infrastructure for
// tests/test_hostemu.py.
//
//   run_case IN OUT
//
// IN holds one lps_sample call's inputs, OUT receives its outputs (layouts
// below, little-endian).  The workspace is calloc'd at its exact size, so an
// access past it, past any input or output array, or past an LDS array of a
// kernel, stops the run with the sanitizer's report.
#include "../../llm-pipeline_amd/csrc/lps.hip"

#include <vector>

namespace {

// IN: int32 header[16] = {magic 0x4C505345, dtype, R, V, H, n_top, flags,
//     use_workspace, logprobs, entropy, skip_draw, 0...}, then
//     logits [R * V] (dtype), temperature f32[R], top_k i32[R], top_p f32[R],
//     min_p f32[R], typical_p f32[R], rep f32[R], pres f32[R], freq f32[R],
//     history i32[R * H], history_len i32[R] (both when H > 0), uniforms f32[R].
// OUT: tokens i64[R], status i32[R], kept_cut f32[R], kept_ties i32[R],
//     kept_count i32[R], row_path i32[R], chosen_logprob f32[R] (logprobs),
//     top_logprobs f32[R * n_top], top_ids i64[R * n_top], entropy f32[R] (when
//     asked), then the workspace's
//     row status words i32[R] (LPS_ROW_DEFERRED | reason << 8 for rows the
//     fast kernels deferred; zeros without a workspace).
template <typename T>
std::vector<T> rd(FILE* f, size_t n) {
  std::vector<T> v(n);
  if (n && fread(v.data(), sizeof(T), n, f) != n) {
    fprintf(stderr, "run_case: short input\n");
    exit(2);
  }
  return v;
}
template <typename T>
void wr(FILE* f, const std::vector<T>& v) {
  if (!v.empty()) fwrite(v.data(), sizeof(T), v.size(), f);
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 3) {
    fprintf(stderr, "usage: run_case IN OUT\n");
    return 2;
  }
  FILE* f = fopen(argv[1], "rb");
  if (!f) return 2;
  const std::vector<int32_t> h = rd<int32_t>(f, 16);
  if (h[0] != 0x4C505345) return 2;
  const int dtype = h[1], R = h[2], V = h[3], H = h[4], n_top = h[5], flags = h[6], use_ws = h[7], lp = h[8];
  const int want_h = h[9], skip_draw = h[10];
  const size_t es = dtype == LPS_DTYPE_F32 ? 4 : 2;
  // the logits exactly sized (an access past the last row is caught)
  std::vector<uint8_t> logits_v = rd<uint8_t>(f, (size_t)R * V * es);
  void* logits = malloc(logits_v.size());
  memcpy(logits, logits_v.data(), logits_v.size());
  auto T = rd<float>(f, R);
  auto K = rd<int32_t>(f, R);
  auto P = rd<float>(f, R), MP = rd<float>(f, R), TP = rd<float>(f, R);
  auto REP = rd<float>(f, R), PRES = rd<float>(f, R), FREQ = rd<float>(f, R);
  std::vector<int32_t> hist, hlen;
  if (H > 0) {
    hist = rd<int32_t>(f, (size_t)R * H);
    hlen = rd<int32_t>(f, R);
  }
  auto U = rd<float>(f, R);
  fclose(f);

  std::vector<int64_t> tokens(R, -7);
  std::vector<int32_t> status(R, -7), ties(R, -7), count(R, -7), path(R, -7);
  std::vector<float> cut(R, -7.0f), clp(lp ? R : 0, -7.0f), tlp((size_t)R * n_top, -7.0f);
  std::vector<int64_t> tids((size_t)R * n_top, -7);
  std::vector<float> ent(want_h ? R : 0, -7.0f);

  lps_sample_args a{};
  a.logits = logits;
  a.dtype = dtype;
  a.num_rows = R;
  a.vocab = V;
  a.rows_inner = 1;
  a.stride_outer = V;
  a.stride_inner = 0;
  a.temperature = T.data();
  a.top_k = K.data();
  a.top_p = P.data();
  a.min_p = MP.data();
  a.typical_p = TP.data();
  a.repetition_penalty = REP.data();
  a.presence_penalty = PRES.data();
  a.frequency_penalty = FREQ.data();
  if (H > 0) {
    a.history = hist.data();
    a.history_stride = H;
    a.history_len = hlen.data();
  }
  a.uniforms = U.data();
  a.tokens = tokens.data();
  a.chosen_logprob = lp ? clp.data() : nullptr;
  a.top_logprobs = n_top ? tlp.data() : nullptr;
  a.top_ids = n_top ? tids.data() : nullptr;
  a.n_top = n_top;
  a.row_status = status.data();
  a.kept_cut = cut.data();
  a.kept_ties = ties.data();
  a.kept_count = count.data();
  a.row_path = path.data();
  a.entropy = want_h ? ent.data() : nullptr;
  a.skip_draw = skip_draw;
  a.flags = flags;
  void* ws = nullptr;
  if (use_ws) {
    a.workspace_bytes = lps_workspace_bytes(R, V, flags);
    ws = a.workspace_bytes ? calloc(1, a.workspace_bytes) : nullptr;
    a.workspace = ws;
  }
  const int rc = lps_sample(&a, nullptr);
  if (rc != LPS_OK) {
    fprintf(stderr, "run_case: lps_sample returned %d\n", rc);
    return 3;
  }
  FILE* o = fopen(argv[2], "wb");
  if (!o) return 2;
  wr(o, tokens);
  wr(o, status);
  wr(o, cut);
  wr(o, ties);
  wr(o, count);
  wr(o, path);
  wr(o, clp);
  wr(o, tlp);
  wr(o, tids);
  wr(o, ent);
  std::vector<int32_t> wst(R, 0);
  if (ws) memcpy(wst.data(), static_cast<char*>(ws) + rg_counter_bytes(), (size_t)R * 4);
  wr(o, wst);
  fclose(o);
  free(ws);
  free(logits);
  return 0;
}
