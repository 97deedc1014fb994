/* Drop-in sampler interface of SeungheonOh/drama3-mlx on the MI355X sampler.
 *
 * The reference's sampler API (src/model.h:146-149, :169-176) and its global
 * seed (src/mlxu.h:168, src/mlxu.c:769) keep their names and parameter lists;
 * an opaque device-array handle, d3s_array, takes the place of mlx_array.
 * Errors keep the reference's die() behaviour (message on stderr, exit(1),
 * src/mlxu.c:28-36, src/sampling.c:169-170).  Like the reference, the calls
 * are single-threaded: the seed and the draw counter are process-global.
 *
 * Arrays returned by these functions are registered in an arena, as the
 * reference's are (src/mlxu.h:1-6, :24-34): d3s_arena_release(mark) frees every
 * array created since d3s_arena_mark(); d3s_array_own() removes one from the
 * arena so the caller frees it with d3s_array_free().
 */
#ifndef D3S_MODEL_SAMPLING_H
#define D3S_MODEL_SAMPLING_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* src/model.h:146-149 */
typedef struct {
  float temperature, top_p;
  int top_k;
} SamplingParams;

typedef struct d3s_array_s *d3s_array;

#define D3S_ARRAY_F32 0   /* fp32 */
#define D3S_ARRAY_BF16 1  /* bf16 (uint16 bit patterns) */
#define D3S_ARRAY_I32 2   /* int32 */

/* ---- sampling (src/model.h:169-176) ---- */
/* One id per row of logits [N, V] (positions into the last axis), int32 [N]
 * (a 1-D array, as the reference's ids are: src/sampling.c:48,161).
 * Replaces sample_top_k_top_p, src/sampling.c:205-209: draws u [N, min(top_k, V)]
 * on the device from the global seed, then samples. */
d3s_array sample_top_k_top_p(d3s_array logits, float temperature, int top_k, float top_p);
/* The uniform draws sample_top_k_top_p makes for logits [rows, V]: fp32
 * [rows, min(top_k, V)], drawn on the host and copied to the device.
 * Replaces sample_noise, src/sampling.c:179-192. */
d3s_array sample_noise(int rows, int V, int top_k);
/* sample_top_k_top_p with its uniform draws u [rows, k] given.
 * Replaces sample_with_noise, src/sampling.c:194-203. */
d3s_array sample_with_noise(d3s_array logits, d3s_array u, float temperature, float top_p);
/* Global seed of every later draw; restarts the draw counter.
 * Replaces m_seed, src/mlxu.c:769. */
void m_seed(uint64_t seed);

/* ---- arrays (the parts of mlx_array the sampler's callers use) ---- */
/* device copy of host data [rows, cols] */
d3s_array d3s_array_from_host(const void *data, int dtype, int rows, int cols);
/* borrow caller-owned device memory [rows, cols] (row_stride elements apart) */
d3s_array d3s_array_from_device(void *ptr, int dtype, int rows, int cols, int64_t row_stride);
/* the 2-D storage: rows x cols elements (ids [N]: N x 1) */
int d3s_array_rows(d3s_array a);
int d3s_array_cols(d3s_array a);
/* the logical shape: 1 for sampled ids [N], 2 otherwise; the size of an axis
 * (negative axes count from the end).  Replace m_ndim / m_dim, src/mlxu.c:848-851. */
int d3s_array_ndim(d3s_array a);
int d3s_array_dim(d3s_array a, int axis);
int d3s_array_dtype(d3s_array a);
void *d3s_array_data(d3s_array a);
/* Waits for the device and copies an int32 array to a malloc'd buffer (the
 * caller frees it); *count receives the element count.  Dies if a sampled row
 * was refused (non-finite logits), as the reference's generation loop does
 * (src/generate.c:92,130).  Replaces m_to_int32, src/mlxu.c:857-867. */
int32_t *d3s_array_to_host_int32(d3s_array a, size_t *count);
/* copies to host memory the caller provides (rows * cols elements) */
void d3s_array_copy_to_host(d3s_array a, void *dst);
/* take an array out of the arena (src/mlxu.h:30, own) */
d3s_array d3s_array_own(d3s_array a);
void d3s_array_free(d3s_array a);
size_t d3s_arena_mark(void);
void d3s_arena_release(size_t mark);

/* ---- test exports (src/testapi.c:155-166) ---- */
/* Sampling: ids for each row of host logits [N, V] (fp32) under `seed`. */
void d3_sample(const float *logits, int N, int V, float temperature, int top_k, float top_p,
               unsigned long long seed, int *out);
/* The same with host uniform draws u [N, k] given (k = min(top_k, V)). */
void d3_sample_with_noise(const float *logits, const float *u, int N, int V, int k,
                          float temperature, float top_p, int *out);

#ifdef __cplusplus
}
#endif

#endif
