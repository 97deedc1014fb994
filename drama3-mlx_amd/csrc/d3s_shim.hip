/* Drop-in sampler interface (include/d3s_model_sampling.h) over the raw core.
 *
 * Mirrors src/sampling.c:179-209 (sample_noise, sample_with_noise,
 * sample_top_k_top_p), src/mlxu.c:769-774 (m_seed, m_uniform), the arena of
 * src/mlxu.c:52-89 and the test export d3_sample of src/testapi.c:155-166.
 * Work goes to the null stream, the counterpart of the reference's default
 * GPU stream (src/mlxu.c:20-26).  This layer allocates device memory for the
 * arrays it returns, as MLX does for the reference's; its sampling calls take
 * the raw core's workspace from the block the library keeps for the null
 * stream (allocated on the first call whose route needs one, then reused). */
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <vector>

#include "../../include/d3s_model_sampling.h"
#include "../../include/d3s_sampler.h"
#include "d3s_math.h"

struct d3s_array_s {
  void *data;
  int dtype, rows, cols; /* storage: rows x cols elements, row_stride apart */
  int64_t row_stride;
  int ndim;     /* 2, or 1 for sampled ids (shape [rows], as src/sampling.c:48,161) */
  bool owns;    /* hipFree on release */
  bool sampled; /* ids from the sampler: -1 marks a refused row */
};

namespace {

uint64_t g_seed = 0;
uint64_t g_draw = 0; /* draws made since the last m_seed */
std::vector<d3s_array> g_arena;

[[noreturn]] void die(const char *fmt, ...) {
  va_list args;
  va_start(args, fmt);
  fprintf(stderr, "error: ");
  vfprintf(stderr, fmt, args);
  fprintf(stderr, "\n");
  va_end(args);
  exit(1);
}

void check(hipError_t e, const char *what) {
  if (e != hipSuccess) die("%s: %s", what, hipGetErrorString(e));
}

size_t elem_size(int dtype) { return dtype == D3S_ARRAY_BF16 ? 2 : 4; }

d3s_array track(d3s_array a) {
  g_arena.push_back(a);
  return a;
}

d3s_array new_device(int dtype, int rows, int cols) {
  d3s_array a = (d3s_array)calloc(1, sizeof(d3s_array_s));
  if (!a) die("out of memory");
  a->dtype = dtype;
  a->rows = rows;
  a->cols = cols;
  a->row_stride = cols;
  a->ndim = 2;
  a->owns = true;
  const size_t bytes = (size_t)rows * cols * elem_size(dtype);
  if (bytes) check(hipMalloc(&a->data, bytes), "hipMalloc");
  return track(a);
}

void release_one(d3s_array a) {
  if (!a) return;
  if (a->owns && a->data) (void)hipFree(a->data);
  free(a);
}

}  // namespace

extern "C" {

void m_seed(uint64_t seed) {
  g_seed = seed;
  g_draw = 0;
}

d3s_array sample_noise(int rows, int V, int top_k) {
  if (rows < 0 || V < 1) die("sample_noise: bad shape [%d, %d]", rows, V);
  const int k = top_k < V ? top_k : V; /* src/sampling.c:186 */
  if (k < 1) die("sample_noise: top_k must be at least 1");
  const uint64_t draw = g_draw++;
  const size_t n = (size_t)rows * k;
  std::vector<float> host(n);
  for (size_t i = 0; i < n; i++) host[i] = d3s_uniform(g_seed, draw, i);
  d3s_array u = new_device(D3S_ARRAY_F32, rows, k);
  if (n) check(hipMemcpy(u->data, host.data(), n * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy");
  return u;
}

d3s_array sample_with_noise(d3s_array logits, d3s_array u, float temperature, float top_p) {
  if (!logits || !u) die("sample_with_noise: null array");
  if (logits->dtype != D3S_ARRAY_F32 && logits->dtype != D3S_ARRAY_BF16)
    die("sample_with_noise: logits must be fp32 or bf16");
  if (u->dtype != D3S_ARRAY_F32 || u->rows != logits->rows || u->row_stride != u->cols)
    die("sample_with_noise: u must be contiguous fp32 [%d, k]", logits->rows);
  d3s_array ids = new_device(D3S_ARRAY_I32, logits->rows, 1);
  ids->ndim = 1; /* int32 [N] */
  ids->sampled = true;
  const int rc = d3s_sample(logits->data, logits->dtype == D3S_ARRAY_F32 ? D3S_DTYPE_F32 : D3S_DTYPE_BF16,
                            logits->rows, logits->cols, logits->row_stride, (const float *)u->data,
                            u->cols, nullptr, nullptr, temperature, top_p, nullptr,
                            (int32_t *)ids->data, nullptr, nullptr, nullptr, 0u, nullptr);
  if (rc != D3S_OK) die("sampling kernel failed (status %d)", rc); /* src/sampling.c:169-170 */
  return ids;
}

d3s_array sample_top_k_top_p(d3s_array logits, float temperature, int top_k, float top_p) {
  if (!logits) die("sample_top_k_top_p: null array");
  const int V = logits->cols, N = logits->rows;
  const int k = top_k < V ? top_k : V; /* src/sampling.c:207 */
  if (k < 1) die("sample_top_k_top_p: top_k must be at least 1");
  if (logits->dtype != D3S_ARRAY_F32 && logits->dtype != D3S_ARRAY_BF16)
    die("sample_top_k_top_p: logits must be fp32 or bf16");
  /* the draw and the kernel in one launch where the one-wave kernel holds
   * the rows (it draws the uniforms itself: the same bits), else the draw
   * into u and the kernel on it */
  d3s_array ids = new_device(D3S_ARRAY_I32, N, 1);
  ids->ndim = 1; /* int32 [N] */
  ids->sampled = true;
  const int rc = d3s_sample_seeded(logits->data, logits->dtype == D3S_ARRAY_F32 ? D3S_DTYPE_F32 : D3S_DTYPE_BF16,
                                   N, V, logits->row_stride, g_seed, g_draw, k, nullptr, nullptr, temperature,
                                   top_p, nullptr, (int32_t *)ids->data, nullptr, nullptr, nullptr, 0u, nullptr);
  if (rc == D3S_OK) {
    g_draw++;
    return ids;
  }
  if (rc != D3S_ERR_UNSUPPORTED) die("sampling kernel failed (status %d)", rc); /* src/sampling.c:169-170 */
  d3s_array u = new_device(D3S_ARRAY_F32, N, k);
  if (d3s_uniform_fill((float *)u->data, (int64_t)N * k, g_seed, g_draw++, nullptr) != D3S_OK)
    die("uniform draw failed");
  return sample_with_noise(logits, u, temperature, top_p);
}

d3s_array d3s_array_from_host(const void *data, int dtype, int rows, int cols) {
  if (rows < 0 || cols < 1 || dtype < D3S_ARRAY_F32 || dtype > D3S_ARRAY_I32)
    die("d3s_array_from_host: bad shape or dtype");
  d3s_array a = new_device(dtype, rows, cols);
  const size_t bytes = (size_t)rows * cols * elem_size(dtype);
  if (bytes) check(hipMemcpy(a->data, data, bytes, hipMemcpyHostToDevice), "hipMemcpy");
  return a;
}

d3s_array d3s_array_from_device(void *ptr, int dtype, int rows, int cols, int64_t row_stride) {
  if (rows < 0 || cols < 1 || row_stride < cols || dtype < D3S_ARRAY_F32 || dtype > D3S_ARRAY_I32)
    die("d3s_array_from_device: bad shape or dtype");
  d3s_array a = (d3s_array)calloc(1, sizeof(d3s_array_s));
  if (!a) die("out of memory");
  a->data = ptr;
  a->dtype = dtype;
  a->rows = rows;
  a->cols = cols;
  a->row_stride = row_stride;
  a->ndim = 2;
  return track(a);
}

int d3s_array_rows(d3s_array a) { return a->rows; }
int d3s_array_cols(d3s_array a) { return a->cols; }
int d3s_array_ndim(d3s_array a) { return a->ndim; }

int d3s_array_dim(d3s_array a, int axis) {
  if (axis < 0) axis += a->ndim; /* src/mlxu.c:848-851 */
  if (axis < 0 || axis >= a->ndim) die("d3s_array_dim: axis out of range");
  if (a->ndim == 1) return a->rows * a->cols;
  return axis == 0 ? a->rows : a->cols;
}
int d3s_array_dtype(d3s_array a) { return a->dtype; }
void *d3s_array_data(d3s_array a) { return a->data; }

void d3s_array_copy_to_host(d3s_array a, void *dst) {
  const size_t es = elem_size(a->dtype);
  check(hipStreamSynchronize(nullptr), "hipStreamSynchronize");
  check(hipMemcpy2D(dst, a->cols * es, a->data, a->row_stride * es, a->cols * es, a->rows,
                    hipMemcpyDeviceToHost),
        "hipMemcpy2D");
}

int32_t *d3s_array_to_host_int32(d3s_array a, size_t *count) {
  if (a->dtype != D3S_ARRAY_I32) die("d3s_array_to_host_int32: not an int32 array");
  const size_t n = (size_t)a->rows * a->cols;
  int32_t *out = (int32_t *)malloc((n ? n : 1) * sizeof(int32_t));
  if (!out) die("out of memory");
  if (n) d3s_array_copy_to_host(a, out);
  if (a->sampled)
    for (size_t i = 0; i < n; i++)
      if (out[i] < 0) die("non-finite logits; refusing to sample invalid audio");
  if (count) *count = n;
  return out;
}

d3s_array d3s_array_own(d3s_array a) {
  for (size_t i = g_arena.size(); i-- > 0;)
    if (g_arena[i] == a) {
      g_arena.erase(g_arena.begin() + (long)i);
      break;
    }
  return a;
}

void d3s_array_free(d3s_array a) {
  d3s_array_own(a);
  release_one(a);
}

size_t d3s_arena_mark(void) { return g_arena.size(); }

void d3s_arena_release(size_t mark) {
  while (g_arena.size() > mark) {
    d3s_array a = g_arena.back();
    g_arena.pop_back();
    release_one(a);
  }
}

void d3_sample(const float *logits, int N, int V, float temperature, int top_k, float top_p,
               unsigned long long seed, int *out) {
  const size_t mark = d3s_arena_mark();
  m_seed(seed);
  d3s_array l = d3s_array_from_host(logits, D3S_ARRAY_F32, N, V);
  size_t n;
  int32_t *ids = d3s_array_to_host_int32(sample_top_k_top_p(l, temperature, top_k, top_p), &n);
  memcpy(out, ids, n * sizeof(int32_t));
  free(ids);
  d3s_arena_release(mark);
}

void d3_sample_with_noise(const float *logits, const float *u, int N, int V, int k,
                          float temperature, float top_p, int *out) {
  const size_t mark = d3s_arena_mark();
  d3s_array l = d3s_array_from_host(logits, D3S_ARRAY_F32, N, V);
  d3s_array uu = d3s_array_from_host(u, D3S_ARRAY_F32, N, k);
  size_t n;
  int32_t *ids = d3s_array_to_host_int32(sample_with_noise(l, uu, temperature, top_p), &n);
  memcpy(out, ids, n * sizeof(int32_t));
  free(ids);
  d3s_arena_release(mark);
}

}  // extern "C"
