/* CPU oracle for the drama3-mlx token sampler.  TEST INFRASTRUCTURE ONLY (see
 * d3s_oracle.h): a plain-C restatement of src/sampling.c used as the parity
 * checker and as the CPU baseline, never by the product path. */
#include "d3s_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "../drama3-mlx_amd/csrc/d3s_math.h"

#define KERNEL_MAX_K 64       /* src/sampling.c:17 */
#define KERNEL_MAX_V (1024 * 64) /* src/sampling.c:197 */
#define MIN_TEMPERATURE 1e-5f /* src/sampling.c:16 */

/* The reference takes its kernel's operation order iff k <= 64, k < V,
 * V <= 65536 and D3_NO_FUSED_SAMPLER is unset (src/sampling.c:197); every other
 * call takes the op graph (src/sampling.c:22-49, :199-201). */
static int kernel_order(int64_t V, int k, int op_graph) {
  return !op_graph && k <= KERNEL_MAX_K && (int64_t)k < V && V <= KERNEL_MAX_V;
}

typedef struct {
  float x;
  int32_t i;
} Cand;

/* a ranks before b: larger x first, then the lower index (src/sampling.c:7-8) */
static inline int beats(float xa, int32_t ia, float xb, int32_t ib) {
  return xa > xb || (xa == xb && ia < ib);
}

static int cmp_rank(const void *pa, const void *pb) {
  const Cand *a = pa, *b = pb;
  if (beats(a->x, a->i, b->x, b->i)) return -1;
  if (beats(b->x, b->i, a->x, a->i)) return 1;
  return 0;
}

/* min-heap on rank order: the root is the worst kept candidate */
static void heap_sift_down(Cand *h, int n, int at) {
  for (;;) {
    int l = 2 * at + 1, r = l + 1, w = at;
    if (l < n && beats(h[w].x, h[w].i, h[l].x, h[l].i)) w = l;
    if (r < n && beats(h[w].x, h[w].i, h[r].x, h[r].i)) w = r;
    if (w == at) return;
    Cand t = h[w];
    h[w] = h[at];
    h[at] = t;
    at = w;
  }
}

/* top k of x[0..V) in rank order (x desc, index asc), src/sampling.c:27-36 / :90-121 */
static void top_k_ranked(const float *x, int64_t V, int k, Cand *out, Cand *scratch) {
  if ((int64_t)k * 8 >= V) {
    for (int64_t i = 0; i < V; i++) {
      scratch[i].x = x[i];
      scratch[i].i = (int32_t)i;
    }
    qsort(scratch, (size_t)V, sizeof(Cand), cmp_rank);
    memcpy(out, scratch, (size_t)k * sizeof(Cand));
    return;
  }
  Cand *h = scratch;
  int n = 0;
  for (int64_t i = 0; i < V; i++) {
    const float xi = x[i];
    if (n < k) {
      h[n].x = xi;
      h[n].i = (int32_t)i;
      n++;
      if (n == k)
        for (int a = k / 2 - 1; a >= 0; a--) heap_sift_down(h, k, a);
    } else if (xi > h[0].x) { /* an equal x with a larger index never wins */
      h[0].x = xi;
      h[0].i = (int32_t)i;
      heap_sift_down(h, k, 0);
    }
  }
  memcpy(out, h, (size_t)k * sizeof(Cand));
  qsort(out, (size_t)k, sizeof(Cand), cmp_rank);
}

static void sample_row(const float *L, int64_t V, int k, int kernel, const float *u, float T,
                       float top_p, int32_t *id_out, float *probs, int32_t *cand, float *lse_out,
                       uint8_t *flags_out, double *gaps, float *x, Cand *top, Cand *scratch,
                       int *drop, float *score) {
  uint8_t flags = 0;
  if (T < MIN_TEMPERATURE) T = MIN_TEMPERATURE; /* src/sampling.c:195 */
  float m = -D3S_INF;
  int bad = 0;
  for (int64_t i = 0; i < V; i++) {
    const float xi = L[i] / T; /* src/sampling.c:25 / :70 */
    x[i] = xi;
    if (d3s_isnan(xi) || xi == D3S_INF) bad = 1;
    if (xi > m) m = xi;
  }
  if (gaps) gaps[0] = gaps[1] = INFINITY;
  if (bad) {
    *id_out = -1;
    if (probs)
      for (int r = 0; r < k; r++) probs[r] = D3S_NAN;
    if (cand)
      for (int r = 0; r < k; r++) cand[r] = -1;
    if (lse_out) *lse_out = D3S_NAN;
    if (flags_out) *flags_out = D3S_ORACLE_BAD;
    return;
  }
  if (m == -D3S_INF) {
    /* every x is -inf: the reference kernel ranks the lowest ids first, every
     * later quantity is NaN and the argmax keeps its initial choice 0 */
    *id_out = 0;
    if (probs)
      for (int r = 0; r < k; r++) probs[r] = D3S_NAN;
    if (cand)
      for (int r = 0; r < k; r++) cand[r] = r;
    if (lse_out) *lse_out = D3S_NAN;
    if (flags_out) *flags_out = D3S_ORACLE_ALL_MASKED;
    return;
  }
  /* lse: exact fixed-point sum of the fp32 terms, src/sampling.c:37-38 / :81-89 */
  uint64_t S = 0;
  for (int64_t i = 0; i < V; i++) S += d3s_fix40(d3s_expf(x[i] - m));
  const float lse = m + d3s_logf(d3s_fixsum_to_f32(S));

  top_k_ranked(x, V, k, top, scratch);

  const float v0 = top[0].x;
  int cut = k;
  float inv;
  if (kernel) {
    /* the reference kernel's order, src/sampling.c:123-131 */
    float cum = 0.0f, sum = 0.0f;
    for (int r = 0; r < k; r++) {
      cum = cum + d3s_expf(top[r].x - lse);
      drop[r] = r > 0 && cum > top_p;
      if (!drop[r]) sum = sum + d3s_expf(top[r].x - v0);
    }
    inv = 1.0f / sum;
  } else {
    /* op graph (src/sampling.c:39-44): exact prefix sums, rounded once */
    uint64_t P = 0, Ssum = 0;
    for (int r = 0; r < k; r++) {
      P += d3s_fix40(d3s_expf(top[r].x - lse));
      drop[r] = r > 0 && d3s_fixsum_to_f32(P) > top_p;
      if (!drop[r]) Ssum += d3s_fix40(d3s_expf(top[r].x - v0));
    }
    inv = 1.0f / d3s_fixsum_to_f32(Ssum);
  }
  for (int r = 0; r < k; r++)
    if (drop[r]) {
      cut = r;
      break;
    }
  /* exponential race, src/sampling.c:132-139 / :45-48 */
  float best = -1.0f;
  int choice = 0;
  for (int r = 0; r < k; r++) {
    const float p = drop[r] ? 0.0f : d3s_expf(top[r].x - v0) * inv;
    const float noise = -d3s_logf(1.0f - u[r]);
    const float s = p / noise;
    score[r] = s;
    if (probs) probs[r] = p;
    if (cand) cand[r] = top[r].i;
    if (s > best) {
      best = s;
      choice = r;
    }
  }
  *id_out = top[choice].i;
  if (lse_out) *lse_out = lse;

  if (!flags_out && !gaps) return; /* no classification asked for */
  /* float64 shadow, for classifying rows where accumulation order could matter */
  double s64 = 0.0;
  for (int64_t i = 0; i < V; i++) s64 += exp((double)x[i] - (double)m);
  const double lse64 = (double)m + log(s64);
  double c64 = 0.0, min_gap = INFINITY;
  for (int r = 0; r < k; r++) {
    c64 += exp((double)top[r].x - lse64);
    if (r >= 1) {
      const double g = fabs(c64 - (double)top_p);
      if (g < min_gap) min_gap = g;
    }
  }
  if (min_gap < 1e-6) flags |= D3S_ORACLE_TOPP_EDGE;
  double kept64 = 0.0;
  for (int r = 0; r < cut; r++) kept64 += exp((double)top[r].x - (double)v0);
  double b1 = -1.0, b2 = -1.0;
  for (int r = 0; r < k; r++) {
    const float noise32 = -d3s_logf(1.0f - u[r]);
    if (!(noise32 > 0.0f)) continue; /* -0 or NaN noise: no race score */
    const double p64 = r < cut ? exp((double)top[r].x - (double)v0) / kept64 : 0.0;
    const double s = p64 / -log1p(-(double)u[r]);
    if (s > b1) {
      b2 = b1;
      b1 = s;
    } else if (s > b2) {
      b2 = s;
    }
  }
  const double race_gap = (b1 > 0.0 && b2 >= 0.0) ? (b1 - b2) / b1 : INFINITY;
  if (race_gap < 1e-6) flags |= D3S_ORACLE_RACE_EDGE;
  if (gaps) {
    gaps[0] = min_gap;
    gaps[1] = race_gap;
  }
  if (flags_out) *flags_out = flags;
}

int d3s_oracle_sample(const void *logits, int dtype, int64_t n_rows, int64_t vocab,
                      int64_t row_stride, const float *u, int k, const float *temperature,
                      const float *top_p, float temperature_scalar, float top_p_scalar,
                      const int32_t *banned, int32_t *ids, float *probs, int32_t *cand,
                      float *lse, uint8_t *flags, double *gaps, int op_graph, int n_threads) {
  if (n_rows < 0 || vocab < 1 || vocab > D3S_ORACLE_MAX_VOCAB || row_stride < vocab || k < 1 || k > vocab ||
      !ids || (n_rows > 0 && (!logits || !u)) ||
      (dtype != D3S_ORACLE_DTYPE_F32 && dtype != D3S_ORACLE_DTYPE_BF16))
    return -1;
  if (n_threads < 1) n_threads = 1;
  const int kernel = kernel_order(vocab, k, op_graph);
  int failed = 0;
#pragma omp parallel num_threads(n_threads)
  {
    float *L = malloc((size_t)vocab * sizeof(float));
    float *x = malloc((size_t)vocab * sizeof(float));
    Cand *top = malloc((size_t)k * sizeof(Cand));
    Cand *scratch = malloc((size_t)vocab * sizeof(Cand));
    int *drop = malloc((size_t)k * sizeof(int));
    float *score = malloc((size_t)k * sizeof(float));
    if (!L || !x || !top || !scratch || !drop || !score) {
#pragma omp atomic write
      failed = 1;
    } else {
#pragma omp for schedule(dynamic, 4)
      for (int64_t row = 0; row < n_rows; row++) {
        if (dtype == D3S_ORACLE_DTYPE_F32) {
          memcpy(L, (const float *)logits + row * row_stride, (size_t)vocab * sizeof(float));
        } else {
          const uint16_t *b = (const uint16_t *)logits + row * row_stride;
          for (int64_t i = 0; i < vocab; i++) L[i] = d3s_bf16_to_f32(b[i]);
        }
        if (banned && banned[row] >= 0 && banned[row] < vocab) L[banned[row]] = -D3S_INF;
        sample_row(L, vocab, k, kernel, u + row * (int64_t)k, temperature ? temperature[row] : temperature_scalar,
                   top_p ? top_p[row] : top_p_scalar, ids + row, probs ? probs + row * (int64_t)k : NULL,
                   cand ? cand + row * (int64_t)k : NULL, lse ? lse + row : NULL,
                   flags ? flags + row : NULL, gaps ? gaps + 2 * row : NULL, x, top, scratch, drop, score);
      }
    }
    free(L);
    free(x);
    free(top);
    free(scratch);
    free(drop);
    free(score);
  }
  return failed ? -1 : 0;
}

void d3s_oracle_ras_select(const int32_t *first, const int32_t *retry, int64_t n_rows,
                           const int32_t *history, int history_len, int32_t eos_id,
                           int32_t semantic_start, int32_t semantic_end, int32_t code_vocab,
                           int32_t *main_tok, int32_t *code0) {
  for (int64_t r = 0; r < n_rows; r++) {
    if (first[r] < 0 || retry[r] < 0) { /* a refused draw: the row's logits are not finite */
      main_tok[r] = -1;
      if (code0) code0[r] = -1;
      continue;
    }
    const int32_t t1 = first[r] == 0 ? eos_id : first[r] + semantic_start - 1;
    const int32_t t2 = retry[r] == 0 ? eos_id : retry[r] + semantic_start - 1;
    int seen = 0;
    for (int h = 0; h < history_len; h++) seen |= history[r * history_len + h] == t1;
    const int32_t t = (seen && t1 >= semantic_start && t1 <= semantic_end) ? t2 : t1;
    main_tok[r] = t;
    if (code0) {
      int32_t c = t - semantic_start;
      code0[r] = c < 0 ? 0 : c > code_vocab - 1 ? code_vocab - 1 : c;
    }
  }
}

void d3s_oracle_linear_bf16(const uint16_t *x, const uint16_t *w, int64_t n_rows, int64_t K,
                            int64_t V, uint16_t *y) {
  for (int64_t n = 0; n < n_rows; n++)
#pragma omp parallel for
    for (int64_t r = 0; r < V; r++) {
      float acc[32];
      for (int l = 0; l < 32; l++) {
        acc[l] = 0.0f;
        for (int64_t c = 0; c < K / 128; c++)
          for (int t = 0; t < 4; t++) {
            const int64_t i = c * 128 + 4 * l + t;
            acc[l] = fmaf(d3s_bf16_to_f32(w[r * K + i]), d3s_bf16_to_f32(x[n * K + i]), acc[l]);
          }
      }
      for (int sn = 16; sn >= 1; sn >>= 1)
        for (int l = 0; l < sn; l++) acc[l] = acc[l] + acc[l + sn];
      y[n * V + r] = d3s_f32_to_bf16_rn(acc[0]);
    }
}

void d3s_oracle_expf(const float *in, float *out, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = d3s_expf(in[i]);
}

void d3s_oracle_logf(const float *in, float *out, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = d3s_logf(in[i]);
}

void d3s_oracle_fix40(const float *in, uint64_t *out, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = d3s_fix40(in[i]);
}

void d3s_oracle_fix40_unit(const float *e, uint64_t *out, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = d3s_fix40_unit(e[i]);
}

void d3s_oracle_expf_nonpos(const float *a, float *out, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = d3s_expf_nonpos(a[i]);
}

void d3s_oracle_fix40_exp(const float *z, uint64_t *out, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = d3s_fix40_exp(z[i]);
}

void d3s_oracle_fixsum_gt_threshold(const float *c, uint64_t *out, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = d3s_fixsum_gt_threshold(c[i]);
}

void d3s_oracle_div_rn(const float *a, float b, float *out, int64_t n) {
  const float y = 1.0f / b;
  for (int64_t i = 0; i < n; i++) out[i] = d3s_div_rn(a[i], b, y);
}

float d3s_oracle_u64_to_f32(uint64_t v) { return d3s_u64_to_f32(v); }

void d3s_oracle_philox(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
  d3s_u32x4 c = {{ctr[0], ctr[1], ctr[2], ctr[3]}};
  d3s_u32x4 o = d3s_philox4x32_10(c, key[0], key[1]);
  memcpy(out, o.v, sizeof(o.v));
}

void d3s_oracle_uniform(uint64_t seed, uint64_t stream0, int64_t rows, int64_t k, float *u) {
  for (int64_t r = 0; r < rows; r++)
    for (int64_t j = 0; j < k; j++) u[r * k + j] = d3s_uniform(seed, stream0 + (uint64_t)r, (uint64_t)j);
}
