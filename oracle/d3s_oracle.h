/* CPU oracle for the token sampler of SeungheonOh/drama3-mlx (src/sampling.c).
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * or as the timed CPU baseline.  The product (the HIP library under
 * drama3-mlx_amd/) never links, loads or falls back to it.
 *
 * Semantics restated (per row; k = number of uniform columns = min(top_k, V)):
 *   T <- max(T, 1e-5)                                  src/sampling.c:16,195
 *   x_i = f32(logit_i) / T                             src/sampling.c:25,70
 *   m = max x; lse = m + log(sum_i exp(x_i - m))       src/sampling.c:37-38,67-89
 *   rank by (x desc, index asc), keep the first k      src/sampling.c:27-36,90-121
 *   c_r = cumulative of exp(v_r - lse) in rank order   src/sampling.c:39,126-127
 *   drop_r = r > 0 and c_r > top_p                     src/sampling.c:40-42,128
 *   p_r = kept ? exp(v_r - v_0) / sum_kept : 0         src/sampling.c:43-44,129-134
 *   noise_r = -log(1 - u_r); score_r = p_r / noise_r   src/sampling.c:45-47,135-136
 *   choice = first r with the greatest score (> -1)    src/sampling.c:132-138
 *   id = index of rank `choice`                         src/sampling.c:48,139
 *
 * Floating-point order (the parts the reference leaves to its hardware):
 *   - exp and log are d3s_expf / d3s_logf (drama3-mlx_amd/csrc/d3s_math.h);
 *   - the row sum inside lse is the exact fixed-point sum (2^-40 units) of the
 *     fp32 terms exp(x_i - m), rounded once to fp32: order independent;
 *   - calls the reference sends to its kernel (k <= 64, k < V, V <= 65536 and
 *     D3_NO_FUSED_SAMPLER unset, src/sampling.c:197): c_r and sum_kept are
 *     sequential fp32 sums in rank order and p_r = e_r * (1/sum_kept), the
 *     operation order of the reference kernel (src/sampling.c:123-139);
 *   - every other call (the reference's op graph, src/sampling.c:22-49, whose
 *     MLX scan and softmax order is unpublished): c_r and sum_kept are exact
 *     fixed-point prefix sums rounded to fp32, p_r = e_r * (1/sum_kept).
 * Rows whose logits (after the optional banned index) give a NaN or +inf x are
 * refused: id -1 (the reference's caller refuses them, src/generate.c:92,130).
 * A row whose x are all -inf returns index 0, as the reference kernel does.
 */
#ifndef D3S_ORACLE_H
#define D3S_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define D3S_ORACLE_DTYPE_F32 0
#define D3S_ORACLE_DTYPE_BF16 1

/* The widest row: the exact row sum adds up to vocab terms of at most 2^40
 * (units of 2^-40) in 64 bits, which 2^24 - 1 terms never wrap. */
#define D3S_ORACLE_MAX_VOCAB 16777215

/* flags per row */
#define D3S_ORACLE_BAD 1          /* non-finite x: refused, id -1 */
#define D3S_ORACLE_TOPP_EDGE 2    /* some r in [1,k) has |c64_r - top_p| < 1e-6 */
#define D3S_ORACLE_RACE_EDGE 4    /* top two race scores within 1e-6 relative */
#define D3S_ORACLE_ALL_MASKED 8   /* every x is -inf */

/* logits: [n_rows, row_stride] of fp32 or bf16 (uint16 bits); u: [n_rows, k].
 * temperature / top_p: per-row arrays, or NULL to use the scalars.
 * banned: per-row index set to -inf before sampling (<0 or >= vocab: none), or NULL.
 * Outputs (each may be NULL except ids): ids [n_rows]; probs, cand [n_rows, k]
 * (post-filter probability and index by rank); lse [n_rows]; flags [n_rows];
 * gaps [n_rows, 2] = (min_r |c64_r - top_p|, relative gap of the top two scores).
 * op_graph: nonzero takes the op graph's order for every call, as the
 * reference does when D3_NO_FUSED_SAMPLER is set (src/sampling.c:197).
 * Returns 0, or -1 for bad arguments (vocab above D3S_ORACLE_MAX_VOCAB included). */
int d3s_oracle_sample(const void *logits, int dtype, int64_t n_rows, int64_t vocab,
                      int64_t row_stride, const float *u, int k, const float *temperature,
                      const float *top_p, float temperature_scalar, float top_p_scalar,
                      const int32_t *banned, int32_t *ids, float *probs, int32_t *cand,
                      float *lse, uint8_t *flags, double *gaps, int op_graph, int n_threads);

/* elementwise d3s_expf / d3s_logf / true division, for the math tests */
/* Repetition-aware selection of the main token (src/tower.c:405-409,:425-433),
 * given the two draws' sampled indices per row (first: the caller's
 * parameters, retry: RAS_TEMPERATURE / RAS_TOP_K / RAS_TOP_P, :13-16):
 *   token(i) = i == 0 ? eos_id : semantic_start + i - 1            (:405-409)
 *   main = token(retry) if semantic_start <= token(first) <= semantic_end
 *          and token(first) is one of the row's history_len recent main
 *          tokens (:429-431), else token(first)                     (:432)
 *   code0 = clip(main - semantic_start, 0, code_vocab - 1)          (:433-434)
 * A row either of whose draws was refused (index -1: a NaN or +inf x) gets
 * main = code0 = -1, the signal a caller checks where the reference's
 * generation loop dies on non-finite logits (src/generate.c:92,130). */
void d3s_oracle_ras_select(const int32_t *first, const int32_t *retry, int64_t n_rows,
                           const int32_t *history, int history_len, int32_t eos_id,
                           int32_t semantic_start, int32_t semantic_end, int32_t code_vocab,
                           int32_t *main_tok, int32_t *code0);
/* The backbone head's logits (src/backbone.c:1213-1215, m_linear of one row,
 * src/mlxu.c:365-400,:492-495): y[n, r] = bf16 of x[n, :] . w[r, :] in the
 * order of the reference's gemv: 32 lanes, lane l accumulating in fp32 the
 * products of elements c*128 + 4l + t (blocks c in order, t = 0..3), then a
 * shuffle-down tree over 16, 8, 4, 2, 1 lanes; lane 0's sum rounded to bf16.
 * The products are fused into the accumulation (fma): the Metal compiler's
 * fast-math contraction, which the reference does not pin.  K % 128 == 0. */
void d3s_oracle_linear_bf16(const uint16_t *x, const uint16_t *w, int64_t n_rows, int64_t K,
                            int64_t V, uint16_t *y);
void d3s_oracle_expf(const float *in, float *out, int64_t n);
void d3s_oracle_logf(const float *in, float *out, int64_t n);
void d3s_oracle_fix40(const float *in, uint64_t *out, int64_t n);
/* out[i] = d3s_fix40_unit(e[i]), the kernels' fix40 for e in [0, 1] */
void d3s_oracle_fix40_unit(const float *e, uint64_t *out, int64_t n);
/* out[i] = d3s_expf_nonpos(a[i]), the kernels' expf for a <= 0 */
void d3s_oracle_expf_nonpos(const float *a, float *out, int64_t n);
/* out[i] = d3s_fix40_exp(z[i]), the kernels' fused form of fix40(expf(z)), z <= 0 */
void d3s_oracle_fix40_exp(const float *z, uint64_t *out, int64_t n);
/* out[i] = the smallest s with fixsum_to_f32(s) > c[i] (the kernels' cut test) */
void d3s_oracle_fixsum_gt_threshold(const float *c, uint64_t *out, int64_t n);
/* out[i] = d3s_div_rn(a[i], b, RN(1/b)), the kernels' division */
void d3s_oracle_div_rn(const float *a, float b, float *out, int64_t n);
float d3s_oracle_u64_to_f32(uint64_t v);
void d3s_oracle_philox(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
/* u[r, j] = d3s_uniform(seed, stream0 + r, j) for r < rows, j < k */
void d3s_oracle_uniform(uint64_t seed, uint64_t stream0, int64_t rows, int64_t k, float *u);

#ifdef __cplusplus
}
#endif

#endif
