/*
 * lps.h -- C ABI of the MI355X (gfx950) token sampler.
 *
 * Plain C: pointers, sizes and enums only, no torch or HIP types.  The stream
 * argument is a hipStream_t passed as void* (NULL = the null stream).  Every
 * pointer in an args struct is a device pointer unless stated otherwise.  All
 * entry points are stream-ordered and never synchronise.  All are safe to
 * call from several host threads at once: the library's only process-wide
 * state is per-device and written once (the device's CU count, and the
 * address of lps_sample_noalloc's workspace); lps_sample_noalloc shares that
 * one workspace per GPU between its calls (see its declaration).
 *
 * The entry points replace the logits->token path of DavidAkinpelu/llm-pipeline:
 *
 *   lps_sample         Sampler.sample_token
 *                        src/llm_pipeline/inference/sampling.py:51-85
 *                      with its filters (:108-238), per-row parameters as the
 *                      continuous batcher applies them row by row
 *                        src/llm_pipeline/inference/continuous_batching.py:394-401
 *                      and the entropy used by sample_mirostat_v2 (:240-279).
 *   lps_spec_verify    the accept / reject / resample block of speculative_decode
 *                        src/llm_pipeline/inference/speculative.py:119-174
 *                      (and the MTP variant :264-276), batched over requests.
 *   lps_verify_drafts  verify_drafts_batched
 *                        src/llm_pipeline/inference/speculative_kernel.py:24-58
 *                      and its torch fallback :84-87.
 */
#ifndef LPS_H
#define LPS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Version 2: the draw is an inverse CDF over the kept ids in sorted order
 * (scaled logit descending, ties lower index first); version 1 drew in
 * vocabulary order, so the same uniforms gave other tokens.  Histories of any
 * length and any number of distinct ids (LPS_ROW_HISTORY_OVERFLOW is no
 * longer set). */
#define LPS_ABI_VERSION 2

/* Return codes.  The reference raises TypeError / ValueError / RuntimeError
 * (sampling.py:106, speculative.py:90-91, torch.multinomial); the Python
 * host maps these codes back onto the same exception types. */
enum {
  LPS_OK = 0,
  LPS_EINVAL = 1,              /* bad shape, stride, pointer or parameter     */
  LPS_EUNSUPPORTED_DTYPE = 2,  /* logits dtype not one of lps_dtype            */
  LPS_ELAUNCH = 3,             /* the HIP launch failed                         */
  LPS_EWORKSPACE = 4,          /* workspace missing or smaller than required   */
  LPS_ENOALLOC_CAPACITY = 5    /* lps_sample_noalloc: the batch needs more workspace than
                                * LPS_NOALLOC_WORKSPACE_BYTES                    */
};

/* Logits element types. */
enum { LPS_DTYPE_F32 = 0, LPS_DTYPE_BF16 = 1, LPS_DTYPE_F16 = 2 };

/* Per-row status bits written to row_status[] by the kernels.  A set bit on a
 * sampling row corresponds to the RuntimeError torch.multinomial raises for an
 * invalid distribution (NaN / +inf / all -inf after temperature). */
enum {
  LPS_ROW_OK = 0,
  LPS_ROW_NONFINITE = 1,       /* NaN or +inf in the scaled logits of a sampling row */
  LPS_ROW_EMPTY = 2,           /* every logit is -inf on a sampling row               */
  LPS_ROW_HISTORY_OVERFLOW = 4 /* never set since ABI version 2 (kept for callers that test it) */
};

/* Largest top-N logprob count per row. */
#define LPS_MAX_TOP_LOGPROBS 64

/* lps_sample_args.flags */
enum {
  LPS_FLAG_GENERIC = 1,        /* use the general one-workgroup-per-row kernel only */
  LPS_FLAG_APPEND_HISTORY = 2, /* also append each row's sampled token (when >= 0) to its history:
                                * history[r, history_len[r]] = token, history_len[r] += 1, when
                                * history_len[r] < history_stride (a full row is left as is).
                                * The history arrays are then written, so the next step's
                                * penalties see the token without a host round trip (the
                                * reference appends on the host, continuous_batching.py:404,
                                * and passes the list back, sampling.py:125).  Requires history
                                * and history_len. */
  /* Row-kind hints (performance only: a row that breaks a hint is still sampled
   * exactly, by the general kernel).  Large batches run greedy and top-k rows
   * one workgroup per row and the other rows on the row-group kernel; a hint
   * lets the launch skip the kernel no row needs. */
  LPS_FLAG_ROWS_TOPK = 4,      /* every row is greedy (temperature <= 0) or has top_k > 0 */
  LPS_FLAG_ROWS_NUCLEUS = 8,   /* no row is greedy or has top_k > 0 */
  /* No row has min_p > 0, typical_p < 1 or top_k > 256: the row-group kernel
   * then runs without the code for those filters (rows that have them take
   * the general kernel when the hint is wrong).  Without the hint that code is
   * left out only when min_p, typical_p and top_k are NULL and their defaults
   * need none of it. */
  LPS_FLAG_ROWS_BASIC_FILTERS = 16
};

/* Residual used by lps_spec_verify on the first rejected position. */
enum {
  LPS_RESIDUAL_TARGET = 0,     /* reference: resample the target distribution (speculative.py:150-157) */
  LPS_RESIDUAL_LEVIATHAN = 1   /* textbook: norm(max(p - q, 0))                                         */
};

/*
 * Logits addressing: row r of R rows starts at element
 *     (r / rows_inner) * stride_outer + (r % rows_inner) * stride_inner
 * of `logits`; elements of a row are contiguous.  A plain [B, V] tensor has
 * rows_inner = 1, stride_outer = row stride.  The engine's strided view
 * logits[:, -1, :] (qwen3_engine.py:528) is the same with stride_outer = T*V.
 */
typedef struct lps_sample_args {
  /* input logits (read only, never modified) */
  const void* logits;
  int32_t dtype;                  /* lps_dtype */
  int32_t num_rows;               /* R */
  int32_t vocab;                  /* V */
  int32_t rows_inner;             /* >= 1 */
  int64_t stride_outer;           /* elements */
  int64_t stride_inner;           /* elements */

  /* per-row parameters, float32/int32 [R]; NULL = the neutral value
   * (temperature 1, top_k 0, top_p 1, min_p 0, typical_p 1,
   *  repetition 1, presence 0, frequency 0).  temperature <= 0 = greedy. */
  const float* temperature;
  const int32_t* top_k;
  const float* top_p;
  const float* min_p;
  const float* typical_p;
  const float* repetition_penalty;
  const float* presence_penalty;
  const float* frequency_penalty;

  /* per-row token histories: int32 [R, history_stride], row r holds
   * history_len[r] ids; ids outside [0, V) are ignored (sampling.py:126).
   * Any length, any number of distinct ids.  history_stride 0: every row
   * reads the same history.  history == NULL: no penalties. */
  const int32_t* history;
  int64_t history_stride;
  const int32_t* history_len;

  /* uniforms in [0, 1), float32 [R]: the inverse-CDF draw of sampling rows,
   * over the kept ids in sorted order (scaled logit descending, ties lower
   * index first): the token is the first id whose cumulative kept mass
   * exceeds u times the total.  Required when any row samples
   * (temperature > 0). */
  const float* uniforms;

  /* optional query tokens: query_prob[r] = probability of the query token
   * under row r's kept distribution.  Row r's query is
   * query_tokens[(r / rows_inner) * query_inner + (r % rows_inner)] when
   * r % rows_inner < query_inner, else none (query_prob[r] = 0). */
  const int64_t* query_tokens;
  int32_t query_inner;
  float* query_prob;              /* float32 [R] or NULL */

  /* outputs */
  int64_t* tokens;                /* int64 [R], required (-1 on a failed row) */
  float* chosen_logprob;          /* float32 [R] or NULL */
  float* top_logprobs;            /* float32 [R, n_top] or NULL */
  int64_t* top_ids;               /* int64 [R, n_top] or NULL */
  int32_t n_top;                  /* 0 .. LPS_MAX_TOP_LOGPROBS */
  float* entropy;                 /* float32 [R] or NULL: H of softmax(scaled logits), nats */
  int32_t* row_status;            /* int32 [R] or NULL: LPS_ROW_* bits */
  int32_t skip_draw;              /* 1: compute query_prob / logprobs only, tokens[r] = -1 for sampling rows */

  /* optional kept-set descriptor of each row after every filter: the kept set
   * is {z > kept_cut} plus the first kept_ties ids (vocabulary order) with
   * z == kept_cut, where z is the penalised, temperature-scaled logit. */
  float* kept_cut;                /* float32 [R] or NULL */
  int32_t* kept_ties;             /* int32 [R] or NULL (-1 = every id at the cut) */
  int32_t* kept_count;            /* int32 [R] or NULL */

  /* optional: which path finished each row (0 = multi-workgroup fast path,
   * 1 = general one-workgroup-per-row algorithm), int32 [R] or NULL */
  int32_t* row_path;

  /* LPS_FLAG_* */
  int32_t flags;

  /* caller-owned scratch of lps_workspace_bytes() bytes, zero-filled before
   * its first use and then reused as is (every launch leaves it ready for
   * the next); NULL selects the general one-workgroup-per-row kernel.  Calls
   * that overlap in time must not share a workspace. */
  void* workspace;
  size_t workspace_bytes;

  /* optional legality mask, the packed form of the reference's logit
   * constraints (constraints.py:53-80, LogitConstraint.apply_to_logits sets
   * illegal ids to -inf before sampling): id i is legal for row r when bit
   * (i & 31) of allowed[r * allowed_stride + (i >> 5)] is set.  Illegal ids
   * count as -inf logits in every step and every output (logprobs included).
   * NULL = every id legal. */
  const uint32_t* allowed;
  int64_t allowed_stride;         /* 32-bit words per row, >= ceil(V / 32) */
} lps_sample_args;

typedef struct lps_spec_args {
  /* target logits [B, k+1, V], draft logits [B, k, V]; rows contiguous,
   * strides in elements */
  const void* target_logits;
  int64_t target_stride_b, target_stride_k;
  const void* draft_logits;
  int64_t draft_stride_b, draft_stride_k;
  int32_t dtype;                  /* lps_dtype, shared by target and draft */
  int32_t batch;                  /* B */
  int32_t k;                      /* draft length, >= 1 */
  int32_t vocab;                  /* V */
  float temperature;              /* shared; <= 0 = greedy */
  float top_p;                    /* shared; >= 1 = off */
  int32_t residual;               /* LPS_RESIDUAL_* */
  const int64_t* draft_tokens;    /* int64 [B, k] */
  const float* u_accept;          /* float32 [B, k] */
  const float* u_resample;        /* float32 [B, k+1] */
  /* outputs */
  int32_t* n_accepted;            /* int32 [B] */
  int64_t* tokens;                /* int64 [B, k+1]: accepted drafts, then the
                                     replacement / bonus token, then -1 */
  int8_t* accept;                 /* int8 [B, k] or NULL: per-position accept bit */
  float* p_target;                /* float32 [B, k] or NULL */
  float* q_draft;                 /* float32 [B, k] or NULL */
  int32_t* row_status;            /* int32 [B*(2k+1)] or NULL */
  /* caller-owned scratch of lps_spec_workspace_bytes() bytes, zero-filled
   * before its first use and then reused as is (every launch leaves it ready
   * for the next); calls that overlap in time must not share it */
  void* workspace;
  size_t workspace_bytes;
} lps_spec_args;

/* ABI version (LPS_ABI_VERSION). */
int lps_version(void);

/* Human-readable name of a return code. */
const char* lps_status_string(int code);

/* Device self-test (no counterpart in the reference): counts the steps over
 * every non-NaN fp32 input, in increasing order, where the GPU's hardware
 * exp2 (v_exp_f32) decreases.  The row-group kernel locates a histogram
 * region's logits by a search over x that assumes exp2 is non-decreasing
 * (exp2(fma(x, c, -ref)) is then non-decreasing in x), so *violations must be
 * 0 on the device it runs on.  Synchronous on the current device (allocates
 * 8 bytes); a few milliseconds. */
int lps_selftest_exp2_monotone(unsigned long long* violations);

/* Scratch bytes lps_sample needs for num_rows rows of vocab V. */
size_t lps_workspace_bytes(int num_rows, int vocab, int flags);

/* Scratch bytes lps_spec_verify needs. */
size_t lps_spec_workspace_bytes(int batch, int k, int vocab);

/* Sampler.sample_token (sampling.py:51-85), batched with per-row parameters. */
int lps_sample(const lps_sample_args* args, void* stream);

/* lps_sample without a caller workspace and without any allocation.
 *
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  args->workspace / workspace_bytes are ignored; the
 * kernels use the library's own workspace, a device array of
 * LPS_NOALLOC_WORKSPACE_BYTES per GPU that each GPU the library runs on holds
 * until the process ends.  The call itself allocates nothing (no hipMalloc,
 * no allocating library routine); the first call on a device looks the
 * array's address up once and clears its counters with a small kernel on
 * `stream`.  Batches whose lps_workspace_bytes(num_rows, vocab, flags)
 * exceeds LPS_NOALLOC_WORKSPACE_BYTES return LPS_ENOALLOC_CAPACITY (for
 * V = 151936: up to 83 rows per call).  Every call on one GPU shares that GPU's
 * array: calls that overlap in time on one GPU (other streams, other host
 * threads) race and must be ordered by the caller.  Results equal
 * lps_sample's on the same inputs. */
#define LPS_NOALLOC_WORKSPACE_BYTES ((size_t)16 << 20)
int lps_sample_noalloc(const lps_sample_args* args, void* stream);

/* speculative.py:119-174, batched: accept / reject, then the replacement or
 * bonus token. */
int lps_spec_verify(const lps_spec_args* args, void* stream);

/* verify_drafts_batched (speculative_kernel.py:24-58):
 *   accept[i] = rand_uniform[i] < min(target_probs[i, draft_tokens[i]] / max(draft_probs[i], 1e-9), 1)
 * target_probs is [K, V] of `dtype` with element strides (stride_k, stride_v);
 * draft_probs and rand_uniform are float32 [K]; draft_tokens int64 [K];
 * accept int8 [K]. */
int lps_verify_drafts(const void* target_probs, int32_t dtype, int64_t K, int64_t V, int64_t stride_k,
                      int64_t stride_v, const float* draft_probs, const int64_t* draft_tokens,
                      const float* rand_uniform, int8_t* accept, void* stream);

/* Row softmax with an optional causal mask, the softmax producer of the
 * reference's fused_softmax_triton (quantization/kernels/triton_softmax.py:65-102):
 *   out[r, j] = softmax(masked)[j], masked[j] = -inf when causal and
 *   j > (r % seq_len) + row_offset, else x[r, j];
 * computed in fp32, written in `dtype` (round to nearest even).  Rows are
 * contiguous; row r of x / out starts at element r * x_stride / r * out_stride.
 * out may be x itself (in place).  row_lse, when given, gets log(sum(exp))
 * of each row's masked values (natural log; -inf for an all -inf row).
 *
 * workspace: caller-owned scratch of lps_softmax_workspace_bytes() bytes,
 * zero-filled before its first use and then reused as is (every launch leaves
 * it zeroed).  It lets long rows (more than 16384 16-bit / 8192 fp32 columns)
 * be split over several workgroups; NULL (or an in-place call) keeps one
 * workgroup per row.  Calls that overlap in time must not share a workspace. */
typedef struct lps_softmax_args {
  const void* x;
  void* out;
  int32_t dtype;                  /* lps_dtype, x and out */
  int32_t rows;
  int32_t cols;
  int64_t x_stride;               /* elements */
  int64_t out_stride;             /* elements */
  int32_t causal;                 /* 0 / 1 */
  int32_t seq_len;                /* causal: rows per sequence (>= 1) */
  int32_t row_offset;             /* causal: first row's position */
  float* row_lse;                 /* float32 [rows] or NULL */
  void* workspace;                /* or NULL */
  size_t workspace_bytes;
  /* optional block statistics of x from its producer (lps_lm_head's stats):
   * per row, ceil(cols / stats_cols) pairs { max, sum(exp(v - max)) } over
   * consecutive blocks of stats_cols columns; rows stats_stride floats apart.
   * With them the softmax is one streaming pass (not with causal). */
  const float* row_stats;
  int64_t stats_stride;
  int32_t stats_cols;
} lps_softmax_args;

/* LM-head projection with the softmax statistics epilogue, the logits
 * producer of the path (models/qwen3/custom_builder.py:415,
 * models/qwen3_5/model.py:263: logits = lm_head(hidden), nn.Linear without
 * bias):
 *   out[m, n] = sum_k x[m, k] * w[n, k]   (fp32 accumulation, in out_dtype)
 *   stats[m, b] = { max, sum(exp(v - max)) } over columns [128 b, 128 b + 128)
 *                 of the stored (rounded) row, b < ceil(vocab / 128).
 * x, w: bf16 or fp16 (same dtype), rows 16-byte aligned (strides multiples of
 * 8 elements), hidden a multiple of 16.  stats may be NULL. */
#define LPS_LMHEAD_BLOCK_COLS 128
typedef struct lps_lm_head_args {
  const void* x;                  /* [rows, hidden] */
  const void* w;                  /* [vocab, hidden] */
  void* out;                      /* [rows, vocab] in out_dtype */
  float* stats;                   /* float32 [rows, ceil(vocab / 128), 2] or NULL */
  int32_t dtype;                  /* lps_dtype of x and w: BF16 or F16 */
  int32_t out_dtype;              /* lps_dtype of out */
  int32_t rows;
  int32_t vocab;
  int32_t hidden;
  int64_t x_stride;               /* elements */
  int64_t w_stride;               /* elements */
  int64_t out_stride;             /* elements */
} lps_lm_head_args;

int lps_lm_head(const lps_lm_head_args* args, void* stream);

/* Bytes of workspace lps_softmax uses for rows x cols of dtype (0: none). */
size_t lps_softmax_workspace_bytes(int rows, int cols, int dtype);

int lps_softmax(const lps_softmax_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LPS_H */
