/* MI355X token sampler: raw C-ABI core (libd3sampler.so).
 *
 * Replaces the device work behind the sampler of SeungheonOh/drama3-mlx:
 *   - sample_kernel_call / drama3_sample (src/sampling.c:53-177): fused k <= 64;
 *   - the compiled op graph sample_fn (src/sampling.c:22-51): any k, any V;
 *   - the routing of sample_with_noise (src/sampling.c:194-203);
 *   - m_uniform on the GPU stream inside sample_top_k_top_p (src/sampling.c:208,
 *     src/mlxu.c:771-774), as d3s_uniform_fill.
 * Plain pointers and sizes only; every pointer argument is device memory (or
 * memory the device can read); `stream` is a hipStream_t (NULL: the null stream).
 * Calls enqueue work and return.
 *
 * Workspace.  Some routes keep state in device memory between their launches
 * (the arrival counters and records of rows spread over several CUs, the rows
 * the nucleus kernel files for its second launch, the sorting kernels' keys).
 * The *_ws entry points take that workspace from the caller and never
 * allocate: size it with the matching *_workspace_bytes query, allocate it
 * once, clear it once with d3s_workspace_init, and pass it to every call.
 * One workspace serves any sequence of calls on one stream (calls that run
 * at the same time, on several streams, need one workspace each).  Its first
 * 256 KiB are counters that every launch leaves zero again; the rest is
 * scratch.  The calls without _ws (d3s_sample, d3s_sample_ras,
 * d3s_linear_sample_bf16) are a convenience that takes the workspace from a
 * block the library keeps per (device, stream), allocated on the stream's
 * first call that needs one (the NULL stream is one such stream for every
 * thread); d3s_stream_workspace_release frees a stream's block.  Such calls
 * on one stream from several host threads each enqueue all their launches
 * before the next one starts (a lock per (device, stream)): their launches
 * never interleave on the block.
 * d3s_sample_noalloc never allocates either: its workspace is one fixed block
 * of static device memory per GPU.
 */
#ifndef D3S_SAMPLER_H
#define D3S_SAMPLER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define D3S_DTYPE_F32 0  /* fp32 logits */
#define D3S_DTYPE_BF16 1 /* bf16 logits (uint16 bit patterns) */

/* status codes */
#define D3S_OK 0
#define D3S_ERR_ARG -1         /* shape, pointer or parameter out of range */
#define D3S_ERR_UNSUPPORTED -2 /* vocab (and so k) beyond D3S_MAX_VOCAB; d3s_sample_seeded: rows the one-wave kernel does not hold */
#define D3S_ERR_LAUNCH -3      /* the HIP launch failed */
#define D3S_ERR_DTYPE -4       /* unknown logits dtype */
#define D3S_ERR_NOMEM -5       /* the library's workspace could not be allocated */
#define D3S_ERR_SCRATCH -6     /* d3s_sample_noalloc: the call needs more than D3S_SCRATCH_BYTES */
#define D3S_ERR_WORKSPACE -7   /* *_ws: the caller's workspace is smaller than the call needs */

/* The widest row the sampler takes: 2^24 - 1 elements.  The exact row sum
 * adds terms of up to 2^40 (units of 2^-40) in 64 bits, so 2^24 - 1 terms
 * never wrap; wider rows return D3S_ERR_UNSUPPORTED. */
#define D3S_MAX_VOCAB 16777215

/* the fixed device scratch of d3s_sample_noalloc, per GPU */
#define D3S_SCRATCH_BYTES (4u << 20)

/* flags for d3s_sample */
#define D3S_FLAG_GENERIC 1u      /* always the streaming kernel (the same results) */
#define D3S_FLAG_EXACT_LSE 2u    /* register kernels: always compute the exact row
                                    sum (by default only rows whose top-p cut it
                                    could change); the nucleus kernel's ids-only
                                    form: every row by its exact retry (the same
                                    results) */
#define D3S_FLAG_EXACT_SELECT 4u /* register kernels: always the radix select */
#define D3S_FLAG_OP_GRAPH 8u     /* every row in the op graph's order, as the
                                    reference computes it with D3_NO_FUSED_SAMPLER
                                    set (src/sampling.c:197); the environment
                                    variable has the same effect */
#define D3S_FLAG_ONE_LAUNCH 16u  /* d3s_linear_sample_bf16 only: the gemv and the
                                    sample in one launch where it fits */

/* counters[] slots, when a counters array is given (atomic per-row increments) */
#define D3S_COUNTER_REFUSED 0      /* rows with a NaN / +inf x: id -1 */
#define D3S_COUNTER_ALL_MASKED 1   /* rows whose x are all -inf: id 0 */
#define D3S_COUNTER_EXACT_SELECT 2 /* rows that took the radix select */
#define D3S_COUNTER_EXACT_LSE 3    /* rows that took the exact row sum */
#define D3S_NUM_COUNTERS 4

/* One sampled index per row of logits [n_rows, vocab] (row r at
 * logits + r * row_stride elements), with the uniform draws u [n_rows, k]
 * (k = min(top_k, vocab), as the reference derives it, src/sampling.c:186,207).
 *
 * Per row (src/sampling.c:1-3,:22-49,:53-140): T = max(temperature, 1e-5);
 * x = logit / T; ranks by (x desc, index asc); c_r = sum_{j<=r} exp(x_j - lse);
 * ranks r > 0 with c_r > top_p are dropped; p_r = softmax over the kept ranks;
 * ids[row] = index of argmax_r p_r / -log(1 - u_r) (first maximum).
 * The sums take the reference kernel's order (sequential fp32) when the
 * reference would run its kernel (k <= 64, k < vocab, vocab <= 65536, and
 * neither D3S_FLAG_OP_GRAPH nor the environment variable D3_NO_FUSED_SAMPLER,
 * read at every call as src/sampling.c:197 does), else the op graph's order
 * (exact prefix sums, rounded once).
 *
 * temperature, top_p: per-row device arrays [n_rows], or NULL to use the
 * scalars.  banned: per-row index set to -inf first (any value outside
 * [0, vocab) = none), or NULL.  probs, cand: optional [n_rows, k] outputs, the
 * post-filter probability and the index of each rank.  counters: optional
 * [D3S_NUM_COUNTERS] uint32 device array that the call increments.
 * A row with a NaN or +inf x is refused: ids = -1, cand = -1, probs = NaN.
 * A row whose x are all -inf gets ids = 0 (the reference kernel's answer).
 * The result is identical for every flag combination.
 * The workspace comes from the block the library keeps for `stream` (see
 * Workspace above); d3s_sample_ws takes the caller's.
 * Replaces: sample_with_noise (src/sampling.c:194-203, declared src/model.h:175-176). */
int d3s_sample(const void *logits, int dtype, int64_t n_rows, int64_t vocab, int64_t row_stride,
               const float *u, int k, const float *temperature, const float *top_p,
               float temperature_scalar, float top_p_scalar, const int32_t *banned,
               int32_t *ids, float *probs, int32_t *cand, uint32_t *counters, unsigned flags,
               void *stream);

/* Bytes of workspace d3s_sample_ws needs for a call with these arguments (0:
 * the call's route keeps no state in device memory), or a negative status for
 * arguments d3s_sample rejects.  The need depends on dtype, n_rows, vocab, k
 * and flags (and on D3_NO_FUSED_SAMPLER only through the route, not the size).
 * Replaces the one-time set-up of sample_kernel_call (src/sampling.c:142-157). */
int64_t d3s_sample_workspace_bytes(int dtype, int64_t n_rows, int64_t vocab, int k, unsigned flags);

/* d3s_sample with the workspace given: never allocates, so it may be captured
 * in a HIP graph.  workspace: device memory of workspace_bytes (256-byte
 * aligned, cleared once by d3s_workspace_init; it may be NULL when
 * d3s_sample_workspace_bytes is 0).  A workspace smaller than the call needs
 * returns D3S_ERR_WORKSPACE before anything is launched.  Calls that share a
 * workspace must run one after another (one stream).  Same results as
 * d3s_sample. */
int d3s_sample_ws(const void *logits, int dtype, int64_t n_rows, int64_t vocab, int64_t row_stride,
                  const float *u, int k, const float *temperature, const float *top_p,
                  float temperature_scalar, float top_p_scalar, const int32_t *banned,
                  int32_t *ids, float *probs, int32_t *cand, uint32_t *counters, unsigned flags,
                  void *workspace, int64_t workspace_bytes, void *stream);

/* Clears a workspace on `stream` with the library's own fill kernel (no
 * memset node, no allocation).  Call it once after allocating the workspace,
 * before the first call that uses it (every launch leaves it ready for the
 * next).  workspace 256-byte aligned, bytes a multiple of 4. */
int d3s_workspace_init(void *workspace, int64_t bytes, void *stream);

/* Frees the block the library keeps for `stream` on the current device
 * (d3s_sample, d3s_sample_ras and d3s_linear_sample_bf16 without _ws), after
 * waiting for the stream.  For a stream about to be destroyed, or to give the
 * memory back; the next call on the stream that needs a block allocates a new
 * one.  No call may use the stream meanwhile. */
int d3s_stream_workspace_release(void *stream);

/* d3s_sample without any allocation, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid it).  No counterpart in the reference.  Same arguments, results and
 * status codes as d3s_sample; the scratch that d3s_sample takes from a
 * per-stream workspace (allocated on a stream's first call that needs it:
 * the records and arrival counters of the kernel that spreads a wide row over
 * several CUs) comes instead from one fixed block of D3S_SCRATCH_BYTES per GPU,
 * in the library's static device memory, held until the process ends.  Every
 * call the segmented kernel takes fits (it takes at most 4096 segments per
 * launch: 256 KiB of counters and at most 2.1 MiB of records); a call that
 * would not returns D3S_ERR_SCRATCH.
 * All calls on one GPU share that block: calls that overlap on one GPU
 * (several streams or threads at once) race and must not be issued. */
int d3s_sample_noalloc(const void *logits, int dtype, int64_t n_rows, int64_t vocab, int64_t row_stride,
                       const float *u, int k, const float *temperature, const float *top_p,
                       float temperature_scalar, float top_p_scalar, const int32_t *banned,
                       int32_t *ids, float *probs, int32_t *cand, uint32_t *counters, unsigned flags,
                       void *stream);

/* Parameters of d3s_sample_ras: the first draw (SamplingParams, src/model.h:146-149),
 * the retry (RAS_TEMPERATURE / RAS_TOP_K / RAS_TOP_P, src/tower.c:13-16: 1.0, 30,
 * 0.95) and the candidate-to-token map of the backbone head (src/tower.c:405-409,
 * :429-432: eos_id, semantic_start, semantic_end, code_vocab of the Config). */
typedef struct {
  float temperature, top_p;
  int top_k;
  float retry_temperature, retry_top_p;
  int retry_top_k;
  int32_t eos_id, semantic_start, semantic_end, code_vocab;
} d3s_ras_params;

/* Repetition-aware sampling of the main token, both draws in one launch that
 * reads each row of logits once from HBM.  Per row (src/tower.c:425-433):
 *   first = the sampled index with (temperature, top_p, top_k) and u [n_rows, k],
 *   retry = the sampled index with the retry's parameters and u_retry [n_rows, k2]
 *   (k = min(top_k, vocab), k2 = min(retry_top_k, vocab), as d3s_sample);
 *   token(i) = i == 0 ? eos_id : semantic_start + i - 1;
 *   main_tok = token(retry) if token(first) is in [semantic_start, semantic_end]
 *              and equals one of the row's history [n_rows, history_len] (the last
 *              RAS_WINDOW_FRAMES = 16 main tokens, src/generate.h:11,
 *              src/generate.c:83-91), else token(first);
 *   code0 = clip(main_tok - semantic_start, 0, code_vocab - 1).
 * history may be NULL with history_len 0; history_len <= 64.  code0, first_idx,
 * retry_idx (the two draws' indices) are optional.  counters count both draws.
 * A row either of whose draws is refused (its logits give a NaN or +inf x)
 * gets main_tok = code0 = -1: the caller checks for it where the reference's
 * generation loop dies on non-finite logits (src/generate.c:92,130).
 * Rows within one wave's reach (k and k2 <= 64, vocab within d3s_sample's
 * one-wave rows) take one launch that reads each row once; any other k and
 * vocab d3s_sample takes run as two d3s_sample launches and a third that picks
 * (the retry's indices go to retry_idx, else to code0, else to the
 * workspace).  The workspace, when the draws' routes or the retry's indices
 * need one, comes from the block the library keeps for `stream` (see
 * Workspace above; D3S_ERR_NOMEM if it cannot be allocated).
 * Replaces: the two sample_with_noise calls, candidate_token and the repeat test of
 * tower_decode_step (src/tower.c:420-433). */
int d3s_sample_ras(const void *logits, int dtype, int64_t n_rows, int64_t vocab, int64_t row_stride,
                   const float *u, const float *u_retry, const int32_t *history, int history_len,
                   const d3s_ras_params *params, int32_t *main_tok, int32_t *code0,
                   int32_t *first_idx, int32_t *retry_idx, uint32_t *counters, void *stream);

/* Bytes of workspace d3s_sample_ras_ws needs (0: none), or a negative status.
 * has_retry_out: nonzero when the call will pass retry_idx or code0. */
int64_t d3s_sample_ras_workspace_bytes(int dtype, int64_t n_rows, int64_t vocab, const d3s_ras_params *params,
                                       int has_retry_out);

/* d3s_sample_ras with the workspace given (never allocates); the workspace
 * contract of d3s_sample_ws. */
int d3s_sample_ras_ws(const void *logits, int dtype, int64_t n_rows, int64_t vocab, int64_t row_stride,
                      const float *u, const float *u_retry, const int32_t *history, int history_len,
                      const d3s_ras_params *params, int32_t *main_tok, int32_t *code0,
                      int32_t *first_idx, int32_t *retry_idx, uint32_t *counters, void *workspace,
                      int64_t workspace_bytes, void *stream);

/* The backbone head's logits (src/backbone.c:1213-1215: m_linear of the last
 * hidden row with lm_head_audio): y[n, r] = bf16 of x[n, :] . w[r, :], in the
 * order of the reference's single-row gemv (src/mlxu.c:365-400,:492-495): 32
 * lanes, lane l accumulating in fp32 the products of elements c*128 + 4l + t
 * (blocks c in order), fused; a shuffle-down tree over 16, 8, 4, 2, 1 lanes;
 * the sum rounded to nearest-even bf16.  x [n_rows, K], w [V, K], y [n_rows, V]
 * bf16 device arrays (8-byte aligned), K a multiple of 128.  (The reference
 * takes this arithmetic for one row; for more rows MLX's matmul order is not
 * reproduced.)  The head's sample is a d3s_sample on y: the two launches can be
 * captured together in a HIP graph.
 * Replaces: backbone_audio_logits (src/backbone.c:1213-1215) through m_linear's
 * gemv_row (src/mlxu.c:454-496). */
int d3s_linear_bf16(const uint16_t *x, const uint16_t *w, int64_t n_rows, int64_t K, int64_t V,
                    uint16_t *y, void *stream);

/* A head's logits and their sample: y = d3s_linear_bf16(x, w) (the
 * reference's single-row gemv order, bit for bit), then ids = d3s_sample on y
 * as bf16 logits [n_rows, V] with u [n_rows, k], the same temperature / top_p
 * / flags / outputs and the same result bits, including the choice of the
 * reference kernel's or the op graph's order.  y [n_rows, V] receives the
 * logits, or may be NULL when the caller does not keep them (they then go to
 * the workspace).  No banned index.
 * By default the gemv and the sample are two launches on the stream, the
 * faster form.  With D3S_FLAG_ONE_LAUNCH, calls with k <= 64, V <= 8192 and
 * at most 62 rows take one launch instead: each workgroup computes 16 logits
 * and files its part of the sample (max, fast sum, the logits) in the
 * workspace, and the last to arrive samples the row (one kernel node
 * instead of two, about 2 us slower on [1, 2048] x [4097, 2048]); other
 * calls take the two launches.  A workspace, when the call needs one, comes
 * from the block the library keeps for `stream` (see Workspace above;
 * D3S_ERR_NOMEM if it cannot be allocated).
 * Replaces: m_linear through gemv_row (src/mlxu.c:454-496) followed by
 * sample_with_noise on its logits: the backbone head (src/backbone.c:1213-1215)
 * and the tower's codebook heads (src/tower.c:228-232,:264,:440-443). */
int d3s_linear_sample_bf16(const uint16_t *x, const uint16_t *w, int64_t n_rows, int64_t K, int64_t V,
                           uint16_t *y, const float *u, int k, const float *temperature, const float *top_p,
                           float temperature_scalar, float top_p_scalar, int32_t *ids, float *probs,
                           int32_t *cand, uint32_t *counters, unsigned flags, void *stream);

/* Bytes of workspace d3s_linear_sample_bf16_ws needs (0: none), or a negative
 * status.  keeps_logits: nonzero when the call will pass y. */
int64_t d3s_linear_sample_workspace_bytes(int64_t n_rows, int64_t K, int64_t V, int k, unsigned flags,
                                          int keeps_logits);

/* d3s_linear_sample_bf16 with the workspace given (never allocates); the
 * workspace contract of d3s_sample_ws. */
int d3s_linear_sample_bf16_ws(const uint16_t *x, const uint16_t *w, int64_t n_rows, int64_t K, int64_t V,
                              uint16_t *y, const float *u, int k, const float *temperature, const float *top_p,
                              float temperature_scalar, float top_p_scalar, int32_t *ids, float *probs,
                              int32_t *cand, uint32_t *counters, unsigned flags, void *workspace,
                              int64_t workspace_bytes, void *stream);

/* u[i] = the i-th uniform of draw `draw` under `seed` (Philox4x32-10, counter
 * (i/4, draw), key seed, 24-bit values in [0, 1)), for i < n.
 * Replaces: m_uniform (src/mlxu.c:771-774) as used by sample_top_k_top_p
 * (src/sampling.c:208); the MLX generator itself is not reproduced. */
int d3s_uniform_fill(float *u, int64_t n, uint64_t seed, uint64_t draw, void *stream);

/* d3s_uniform_fill(u, n_rows * k, seed, draw) then d3s_sample with that u,
 * in one launch: the one-wave kernel draws each rank's uniform itself (the
 * same bits), so no u is written or read.  Same arguments, checks and
 * results as that pair, with (seed, draw) in u's place.  Only the one-wave
 * kernel's one-row-a-workgroup form draws them: launches of more than 1024
 * rows, rows it does not hold (k above 64; rows longer than 6144 fp32 / 8192
 * bf16 elements, or 6141 / 8185 where the base or the stride leaves a row
 * start off 16 bytes) and D3S_FLAG_GENERIC return D3S_ERR_UNSUPPORTED with
 * nothing launched; take the pair there.  Never allocates.
 * Replaces: sample_top_k_top_p's draw and kernel call together
 * (src/sampling.c:205-209: m_uniform at :208, the call at :209); no single
 * reference function does both. */
int d3s_sample_seeded(const void *logits, int dtype, int64_t n_rows, int64_t vocab, int64_t row_stride,
                      uint64_t seed, uint64_t draw, int k, const float *temperature, const float *top_p,
                      float temperature_scalar, float top_p_scalar, const int32_t *banned, int32_t *ids,
                      float *probs, int32_t *cand, uint32_t *counters, unsigned flags, void *stream);

/* The largest k d3s_sample accepts (D3S_MAX_VOCAB: any k up to the row's
 * vocab), and the largest vocab the fused kernel takes for a dtype (wider
 * rows use the other kernels). */
int d3s_max_k(void);
int d3s_fused_max_vocab(int dtype);

/* Diagnostic, no counterpart in the reference: the device versions of the
 * shared fp32 functions (exp, log, division by `divisor`, 2^-40 fixed-point
 * image), elementwise over in[0..n), for bit-exact comparison with the CPU. */
int d3s_math_selftest(const float *in, float *out_exp, float *out_log, float *out_div,
                      uint64_t *out_fix, int64_t n, float divisor, void *stream);

/* Diagnostic, no counterpart in the reference: out[i] = the hardware 2^in[i]
 * (v_exp_f32) behind the fast row sum, whose error bound the kernel's top-p
 * margin relies on (checked by the tests). */
int d3s_exp2_selftest(const float *in, float *out, int64_t n, void *stream);

/* Diagnostic, no counterpart in the reference: out[i] = the hardware log2(in[i])
 * (v_log_f32) behind the fast row sum's log-sum-exp, whose error bound the
 * kernel's top-p margin relies on (checked by the tests). */
int d3s_log2_selftest(const float *in, float *out, int64_t n, void *stream);

/* "d3sampler <version> gfx950" */
const char *d3s_version(void);

#ifdef __cplusplus
}
#endif

#endif
