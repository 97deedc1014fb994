/* Internal launch interface between the C-ABI layer (d3s_api.hip) and the
 * kernels (d3s_kernels.hip).  Not installed; the public ABI is include/. */
#ifndef D3S_INTERNAL_H
#define D3S_INTERNAL_H

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace d3s {

/* every row-independent input of one sampling launch; pointers are device
 * pointers (or host memory the device can read) */
struct SampleArgs {
  const void *logits;       /* [n_rows, row_stride] fp32 or bf16 */
  int64_t row_stride;       /* in elements */
  int vocab;                /* V */
  int k;                    /* uniform columns per row, 1 <= k <= V */
  int n_rows;
  const float *u;           /* [n_rows, k]; null: the one-wave kernels draw u[r, j] =
                               d3s_uniform(u_seed, u_stream, r k + j) themselves */
  uint64_t u_seed, u_stream;
  const float *temperature; /* [n_rows] or null -> temperature_scalar */
  const float *top_p;       /* [n_rows] or null -> top_p_scalar */
  float temperature_scalar;
  float top_p_scalar;
  const int32_t *banned;    /* [n_rows] index forced to -inf, or null */
  int32_t *ids;             /* [n_rows] */
  float *probs;             /* [n_rows, k] or null */
  int32_t *cand;            /* [n_rows, k] or null */
  uint32_t *counters;       /* [D3S_NUM_COUNTERS] or null */
  unsigned flags;
  /* the op graph's order for the cumulative and the kept sum (exact prefix
   * sums, src/sampling.c:22-49) instead of the reference kernel's sequential
   * fp32 sums (:123-131): every call the reference does not send to its
   * kernel (src/sampling.c:197) */
  bool opgraph;
};

/* Repetition-aware sampling of the main token (src/tower.c:13-16,:405-433):
 * two draws from each row, one with the caller's parameters and a retry; the
 * retry's id replaces the first's when the first's token is a semantic token
 * among the row's recent main tokens. */
struct RasArgs {
  SampleArgs first, retry;  /* the same logits and rows; their own u, k, T, top_p, ids */
  const int32_t *history;   /* [n_rows, history_len] recent main tokens, or null */
  int history_len;          /* 0 .. 64 */
  int32_t eos_id, semantic_start, semantic_end, code_vocab;
  int32_t *main_tok;        /* [n_rows] */
  int32_t *code0;           /* [n_rows] or null: clip(main - semantic_start, 0, code_vocab - 1) */
};

/* The backbone head's logits (src/backbone.c:1213-1215; src/mlxu.c:365-400,:492-495). */
struct LinearArgs {
  const uint16_t *x; /* [n_rows, K] bf16 */
  const uint16_t *w; /* [V, K] bf16 */
  int K, V, n_rows;
  uint16_t *y;       /* [n_rows, V] bf16 logits */
};

/* counters[] slots (atomic increments per row) */
enum {
  CNT_REFUSED = 0,      /* non-finite x: id -1 */
  CNT_ALL_MASKED = 1,   /* every x -inf */
  CNT_EXACT_SELECT = 2, /* fell back to the radix select */
  CNT_EXACT_LSE = 3,    /* the wave kernel recomputed the row sum exactly */
  CNT_NUM = 4
};

/* flags (same values as the public D3S_FLAG_*) */
enum : unsigned {
  FLAG_GENERIC = 1u,
  FLAG_EXACT_LSE = 2u,
  FLAG_EXACT_SELECT = 4u,
  FLAG_OP_GRAPH = 8u,
};

/* The reference sends a call to its one-kernel sampler iff k <= 64, k < V,
 * V <= 65536 and D3_NO_FUSED_SAMPLER is unset (src/sampling.c:17,197); every
 * other call takes its op graph.  Returns true for the op graph. */
inline bool op_graph_order(int vocab, int k, bool forced) {
  return forced || !(k <= 64 && k < vocab && vocab <= 1024 * 64);
}

enum Dtype { DT_F32 = 0, DT_BF16 = 1 };

/* Launch the one-wave-per-row kernel (k <= 64, V <= wave_max_vocab(dt)).
 * Returns false if no instantiation fits. */
bool launch_wave(const SampleArgs &a, Dtype dt, hipStream_t s);
int wave_max_vocab(Dtype dt);
/* Launch the fused RAS kernel (both draws k <= 64, V within the wave kernel's
 * reach).  Returns false if no instantiation fits. */
bool launch_ras(const RasArgs &r, Dtype dt, hipStream_t s);
/* The pick of the main token alone, from the two draws' indices already in
 * device memory (one wave per row). */
void launch_ras_select(const RasArgs &r, const int32_t *first, const int32_t *retry, hipStream_t s);
/* Device memory the library keeps for one stream of the current device, at
 * least `bytes`, zero when first allocated (kernels that count in it leave it
 * zero again).  The first call on a stream, or one that needs more, allocates
 * (hipMalloc); later calls return the same block.  A block the stream
 * outgrows is kept (a call on another thread may still be enqueueing on it)
 * until release_stream_workspace.  Null when the allocation fails. */
void *stream_workspace(hipStream_t s, size_t bytes);
/* Waits for the stream, then frees its block and the blocks it outgrew. */
int release_stream_workspace(hipStream_t s);
/* Launch the head's gemv. */
void launch_linear(const LinearArgs &la, hipStream_t s);
/* Launch the fused head: the gemv's logits and their sample in one launch
 * (k <= 64, V <= head_max_vocab(), at most head_max_rows() rows).  ws: device memory of
 * ws_bytes (at least head_workspace_bytes) whose first split_counter_bytes()
 * are the arrival counters (zero on entry; the kernel leaves them zero).
 * a: the sample's arguments (vocab = la.V).  Returns false (nothing
 * launched) when the call does not fit. */
bool launch_head(const LinearArgs &la, const SampleArgs &a, void *ws, size_t ws_bytes, hipStream_t s);
int head_max_vocab();
int head_max_rows();
size_t head_workspace_bytes(const LinearArgs &la);
/* out[i] = the hardware 2^in[i] (v_exp_f32) the wave kernel's fast row sum uses */
void launch_exp2_selftest(const float *in, float *out, int64_t n, hipStream_t s);
/* out[i] = the hardware log2(in[i]) (v_log_f32) the fast row sum's log uses */
void launch_log2_selftest(const float *in, float *out, int64_t n, hipStream_t s);
/* Launch the wide kernel: one 1024-thread workgroup per row, the row in the
 * registers of its 16 waves (k <= 64, V <= wide_max_vocab(dt)). */
bool launch_wide(const SampleArgs &a, Dtype dt, hipStream_t s);
int wide_max_vocab(Dtype dt);
/* Launch the segmented kernel: rows cut into segments of 4 waves, every
 * segment one workgroup, the last to arrive merging the row (k <= 64, rows of
 * 2 to 16 segments, at most 4096 segments a launch).  ws: device memory of ws_bytes for the records and the
 * arrival counters (counters zero on entry; the kernel leaves them zero).
 * Returns false (nothing launched) when the row does not fit or ws is too
 * small. */
bool launch_split(const SampleArgs &a, Dtype dt, void *ws, size_t ws_bytes, hipStream_t s);
/* segments per row of launch_split for these rows (0: the kernel does not
 * take them), and the workspace it needs */
int split_segments(const SampleArgs &a, Dtype dt);
size_t split_workspace_bytes(const SampleArgs &a, Dtype dt);
/* the workspace's first bytes: the segmented kernel's arrival counters, which
 * must stay zero between launches (nothing else may be placed there) */
size_t split_counter_bytes();
/* Launch the fused one-workgroup-per-row kernel (k <= 64, V within the
 * register-resident limit).  Returns false if no instantiation fits. */
bool launch_fused(const SampleArgs &a, Dtype dt, hipStream_t s);
/* Largest V the fused kernel accepts for this dtype. */
int fused_max_vocab(Dtype dt);
/* Launch the ranked-nucleus kernel (k > 64, V <= topp_max_vocab()).  Calls
 * that ask for ids only with k = V take the ids-only kernel and a second
 * launch for the rows it leaves to the full path, with ws (at least
 * topp_workspace_bytes: the counter block, whose first two lines hold its
 * counts, then a row list); without ws, the full path for every row. */
bool launch_topp(const SampleArgs &a, Dtype dt, void *ws, size_t ws_bytes, hipStream_t s);
int topp_max_vocab();
size_t topp_workspace_bytes(const SampleArgs &a);
/* Launch the streaming generic kernel (any V, k <= generic_max_k()). */
bool launch_generic(const SampleArgs &a, Dtype dt, hipStream_t s);
int generic_max_k();
/* Launch the sorting kernels for k beyond generic_max_k() (any V, any
 * k <= V): each row cut into up to 16 segments, its keys radix-sorted in ws
 * and the tail taken over the segments (bigk_row_bytes per row: keys, count
 * tables, records, tile sums; rows go in launches of as many as ws holds).
 * Returns false when ws does not hold one row. */
bool launch_bigk(const SampleArgs &a, Dtype dt, void *ws, size_t ws_bytes, hipStream_t s);
size_t bigk_row_bytes(const SampleArgs &a);
/* w[i] = 0 for i < n_words (w 16-byte aligned), by a kernel */
void launch_zero_fill(uint32_t *w, size_t n_words, hipStream_t s);
/* u[i] = d3s_uniform(seed, stream_id, i), i < n */
void launch_uniform(float *u, int64_t n, uint64_t seed, uint64_t stream_id, hipStream_t s);
/* elementwise d3s_expf / d3s_logf / x / divisor / d3s_fix40 for the math self-test */
void launch_math_selftest(const float *in, float *out_exp, float *out_log, float *out_div,
                          uint64_t *out_fix, int64_t n, float divisor, hipStream_t s);

}  // namespace d3s

#endif
