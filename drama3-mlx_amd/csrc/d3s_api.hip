/* C-ABI of the MI355X token sampler (include/d3s_sampler.h): argument checks,
 * the choice of definition and the routing between kernels.
 *
 * The definition mirrors sample_with_noise (src/sampling.c:194-203): the
 * reference kernel's sequential sums when k <= 64, k < V, V <= 65536 and
 * D3_NO_FUSED_SAMPLER is unset (the environment is read at every call, as the
 * reference's getenv is), else the op graph's exact prefix sums.  Either
 * definition runs on whichever kernel holds the row; every kernel computes
 * both bit for bit. */
#include <stdlib.h>
#include <string.h>

#include <map>
#include <mutex>
#include <utility>

#include "../../include/d3s_sampler.h"
#include "d3s_internal.h"

/* The allocation-free entry point's scratch: one block per GPU the library
 * runs on, held until the process ends.  Host code never uses this name as
 * an address (it is a host-side stand-in): each device's address comes from
 * hipGetSymbolAddress, taken once per device with that device current.  It
 * starts zero (the segmented kernel's arrival counters must) and every
 * segmented launch leaves its counters zero again. */
static __device__ __align__(256) unsigned char scratch[D3S_SCRATCH_BYTES];

namespace d3s {

namespace {
struct Block {
  void *ptr = nullptr;
  size_t bytes = 0;
};
std::mutex g_ws_mutex;
std::map<std::pair<int, uintptr_t>, Block> g_ws; /* (device, stream) -> block */
}  // namespace

void *stream_workspace(hipStream_t s, size_t bytes) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> lock(g_ws_mutex);
  Block &b = g_ws[{dev, (uintptr_t)s}];
  if (b.bytes >= bytes) return b.ptr;
  const size_t want = (bytes + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1); /* whole MiB */
  if (b.ptr) {
    (void)hipFree(b.ptr); /* waits for the device: no kernel still uses the block */
    b = Block{};
  }
  void *p = nullptr;
  if (hipMalloc(&p, want) != hipSuccess) return nullptr;
  if (hipMemset(p, 0, want) != hipSuccess) {
    (void)hipFree(p);
    return nullptr;
  }
  b.ptr = p;
  b.bytes = want;
  return p;
}

}  // namespace d3s

namespace {

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mutex;
void *g_scratch_ptr[MAX_DEVICES]; /* each device's address of `scratch`, null until taken */

/* the current device's address of the scratch array (null on failure) */
void *device_scratch() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

/* set, with any value, as src/sampling.c:197 tests it */
bool env_no_fused() { return getenv("D3_NO_FUSED_SAMPLER") != nullptr; }

int launched() { return hipGetLastError() == hipSuccess ? D3S_OK : D3S_ERR_LAUNCH; }

/* the sorting kernels' keys per launch from the stream's workspace: every
 * row, up to 256 MiB (then launches of fewer rows), at least one row */
constexpr size_t BIGK_WS_CAP = (size_t)256 << 20;

/* the workspace sample_routed takes from a stream for these rows: the
 * segmented kernel's (counters and records), or the counters' block and the
 * sorting kernels' keys after it; 0 when no kernel needs one */
size_t routed_workspace_bytes(const d3s::SampleArgs &a, d3s::Dtype dt) {
  const bool generic = (a.flags & D3S_FLAG_GENERIC) != 0u;
  if (!generic && d3s::split_segments(a, dt) > 0) return d3s::split_workspace_bytes(a, dt);
  /* the nucleus kernel takes k > 64 on rows up to topp_max_vocab() (its
   * ids-only form files the rows it leaves in the workspace) */
  const bool topp = !generic && a.k > 64 && a.vocab <= d3s::topp_max_vocab();
  if (topp) return d3s::topp_workspace_bytes(a);
  if (a.k > d3s::generic_max_k() && !topp) {
    const size_t row = d3s::bigk_row_bytes(a);
    size_t keys = row * (size_t)a.n_rows;
    if (keys > BIGK_WS_CAP) keys = BIGK_WS_CAP > row ? BIGK_WS_CAP : row;
    return d3s::split_counter_bytes() + keys;
  }
  return 0;
}

/* the first kernel that holds the row: one wave, the rows cut into segments
 * over many CUs (with a workspace), the fused workgroup (kernel order only),
 * the wide workgroup, the nucleus kernel, else the streaming one.  ws: the
 * workspace for the segmented kernel, or null to take the stream's (allocated
 * on first use); ws_bytes its size. */
int sample_routed(const d3s::SampleArgs &a, d3s::Dtype dt, hipStream_t s, void *ws = nullptr,
                  size_t ws_bytes = 0, bool stream_ws = true) {
  const bool generic = (a.flags & D3S_FLAG_GENERIC) != 0u;
  if (!generic && d3s::launch_wave(a, dt, s)) return launched();
  if (!generic && d3s::split_segments(a, dt) > 0) {
    const size_t need = d3s::split_workspace_bytes(a, dt);
    if (!ws && stream_ws) {
      ws = d3s::stream_workspace(s, need);
      ws_bytes = ws ? need : 0;
    }
    if (ws && d3s::launch_split(a, dt, ws, ws_bytes, s)) return launched();
  }
  if (!generic && !a.opgraph && d3s::launch_fused(a, dt, s)) return launched();
  if (!generic && d3s::launch_wide(a, dt, s)) return launched();
  if (!generic && a.k > 64 && a.vocab <= d3s::topp_max_vocab()) {
    const size_t need = d3s::topp_workspace_bytes(a);
    if (need > 0 && !ws && stream_ws) {
      ws = d3s::stream_workspace(s, need);
      ws_bytes = ws ? need : 0; /* without one: the full path for every row */
    }
    if (d3s::launch_topp(a, dt, ws, ws_bytes, s)) return launched();
  }
  if (a.k > d3s::generic_max_k()) { /* the sorting kernels, their keys after the counters' block */
    const size_t off = d3s::split_counter_bytes();
    if (!ws && stream_ws) {
      const size_t need = routed_workspace_bytes(a, dt);
      ws = d3s::stream_workspace(s, need);
      if (!ws) return D3S_ERR_NOMEM;
      ws_bytes = need;
    }
    if (!ws || ws_bytes < off + d3s::bigk_row_bytes(a)) return stream_ws ? D3S_ERR_NOMEM : D3S_ERR_SCRATCH;
    if (!d3s::launch_bigk(a, dt, (char *)ws + off, ws_bytes - off, s)) return D3S_ERR_SCRATCH;
    return launched();
  }
  if (!d3s::launch_generic(a, dt, s)) return D3S_ERR_UNSUPPORTED;
  return launched();
}

/* d3s_sample's checks and routing; no_alloc: the segmented kernel's records
 * go to the fixed per-device scratch instead of the stream's workspace */
int sample_call(const void *logits, int dtype, int64_t n_rows, int64_t vocab, int64_t row_stride,
                const float *u, int k, const float *temperature, const float *top_p, float temperature_scalar,
                float top_p_scalar, const int32_t *banned, int32_t *ids, float *probs, int32_t *cand,
                uint32_t *counters, unsigned flags, void *stream, bool no_alloc) {
  if (dtype != D3S_DTYPE_F32 && dtype != D3S_DTYPE_BF16) return D3S_ERR_DTYPE;
  if (n_rows < 0 || n_rows > 0x7fffffff || vocab < 1 || vocab > (1 << 26) ||
      row_stride < vocab || k < 1 || k > vocab)
    return D3S_ERR_ARG;
  if (n_rows == 0) return D3S_OK;
  if (!logits || !u || !ids) return D3S_ERR_ARG;
  /* rows are addressed in whole elements */
  if ((uintptr_t)logits % (dtype == D3S_DTYPE_F32 ? 4u : 2u) != 0u) return D3S_ERR_ARG;
  if ((flags & ~(D3S_FLAG_GENERIC | D3S_FLAG_EXACT_LSE | D3S_FLAG_EXACT_SELECT | D3S_FLAG_OP_GRAPH)) != 0u)
    return D3S_ERR_ARG;
  d3s::SampleArgs a;
  a.logits = logits;
  a.row_stride = row_stride;
  a.vocab = (int)vocab;
  a.k = k;
  a.n_rows = (int)n_rows;
  a.u = u;
  a.temperature = temperature;
  a.top_p = top_p;
  a.temperature_scalar = temperature_scalar;
  a.top_p_scalar = top_p_scalar;
  a.banned = banned;
  a.ids = ids;
  a.probs = probs;
  a.cand = cand;
  a.counters = counters;
  a.flags = flags;
  a.opgraph = d3s::op_graph_order(a.vocab, k, (flags & D3S_FLAG_OP_GRAPH) || env_no_fused());
  const d3s::Dtype dt = dtype == D3S_DTYPE_F32 ? d3s::DT_F32 : d3s::DT_BF16;
  if (!no_alloc) return sample_routed(a, dt, (hipStream_t)stream);
  void *ws = nullptr;
  const size_t need = routed_workspace_bytes(a, dt);
  if (need > 0) { /* the segmented kernel, the sorting kernels one row at a time, or the nucleus
                     ids path's filed rows (more rows than the scratch lists: the full path) */
    if (d3s::split_segments(a, dt) > 0 && need > D3S_SCRATCH_BYTES) return D3S_ERR_SCRATCH;
    ws = device_scratch();
    if (!ws) return D3S_ERR_LAUNCH;
  }
  return sample_routed(a, dt, (hipStream_t)stream, ws, D3S_SCRATCH_BYTES, false);
}

}  // namespace

extern "C" {

int d3s_sample(const void *logits, int dtype, int64_t n_rows, int64_t vocab, int64_t row_stride,
               const float *u, int k, const float *temperature, const float *top_p,
               float temperature_scalar, float top_p_scalar, const int32_t *banned,
               int32_t *ids, float *probs, int32_t *cand, uint32_t *counters, unsigned flags,
               void *stream) {
  return sample_call(logits, dtype, n_rows, vocab, row_stride, u, k, temperature, top_p, temperature_scalar,
                     top_p_scalar, banned, ids, probs, cand, counters, flags, stream, false);
}

int d3s_sample_noalloc(const void *logits, int dtype, int64_t n_rows, int64_t vocab, int64_t row_stride,
                       const float *u, int k, const float *temperature, const float *top_p,
                       float temperature_scalar, float top_p_scalar, const int32_t *banned,
                       int32_t *ids, float *probs, int32_t *cand, uint32_t *counters, unsigned flags,
                       void *stream) {
  return sample_call(logits, dtype, n_rows, vocab, row_stride, u, k, temperature, top_p, temperature_scalar,
                     top_p_scalar, banned, ids, probs, cand, counters, flags, stream, true);
}

int d3s_sample_ras(const void *logits, int dtype, int64_t n_rows, int64_t vocab, int64_t row_stride,
                   const float *u, const float *u_retry, const int32_t *history, int history_len,
                   const d3s_ras_params *params, int32_t *main_tok, int32_t *code0,
                   int32_t *first_idx, int32_t *retry_idx, uint32_t *counters, void *stream) {
  if (dtype != D3S_DTYPE_F32 && dtype != D3S_DTYPE_BF16) return D3S_ERR_DTYPE;
  if (!params || n_rows < 0 || n_rows > 0x7fffffff || vocab < 1 || vocab > (1 << 26) ||
      row_stride < vocab || params->top_k < 1 || params->retry_top_k < 1 || history_len < 0 ||
      history_len > 64 || (history_len > 0 && !history) || params->code_vocab < 1)
    return D3S_ERR_ARG;
  if (n_rows == 0) return D3S_OK;
  if (!logits || !u || !u_retry || !main_tok) return D3S_ERR_ARG;
  if ((uintptr_t)logits % (dtype == D3S_DTYPE_F32 ? 4u : 2u) != 0u) return D3S_ERR_ARG;
  d3s::RasArgs r;
  d3s::SampleArgs &a = r.first;
  a.logits = logits;
  a.row_stride = row_stride;
  a.vocab = (int)vocab;
  a.k = params->top_k < vocab ? params->top_k : (int)vocab; /* src/sampling.c:186,207 */
  a.n_rows = (int)n_rows;
  a.u = u;
  a.temperature = nullptr;
  a.top_p = nullptr;
  a.temperature_scalar = params->temperature;
  a.top_p_scalar = params->top_p;
  a.banned = nullptr;
  a.ids = first_idx;
  a.probs = nullptr;
  a.cand = nullptr;
  a.counters = counters;
  a.flags = 0u;
  const bool no_fused = env_no_fused();
  a.opgraph = d3s::op_graph_order(a.vocab, a.k, no_fused);
  r.retry = a;
  r.retry.k = params->retry_top_k < vocab ? params->retry_top_k : (int)vocab;
  r.retry.opgraph = d3s::op_graph_order(a.vocab, r.retry.k, no_fused);
  r.retry.u = u_retry;
  r.retry.temperature_scalar = params->retry_temperature;
  r.retry.top_p_scalar = params->retry_top_p;
  r.retry.ids = retry_idx;
  r.history = history;
  r.history_len = history_len;
  r.eos_id = params->eos_id;
  r.semantic_start = params->semantic_start;
  r.semantic_end = params->semantic_end;
  r.code_vocab = params->code_vocab;
  r.main_tok = main_tok;
  r.code0 = code0;
  const d3s::Dtype dt = dtype == D3S_DTYPE_F32 ? d3s::DT_F32 : d3s::DT_BF16;
  hipStream_t s = (hipStream_t)stream;
  if (d3s::launch_ras(r, dt, s)) return launched();
  /* rows the fused kernel does not hold (k above 64, or wider than one wave's
   * registers): the two draws as routed launches, then the pick.  The first
   * draw's indices go to first_idx or else main_tok (the pick reads each row's
   * before it writes it); the retry's to retry_idx or else the workspace. */
  /* one workspace block: the segmented kernel's counters and records, or the
   * sorting kernels' keys, first (both draws use them in turn), then the
   * retry's indices, never on the counters (which must stay zero for later
   * launches on this stream) */
  size_t split_bytes = routed_workspace_bytes(r.first, dt);
  const size_t split_retry = routed_workspace_bytes(r.retry, dt);
  if (split_retry > split_bytes) split_bytes = split_retry;
  if (split_bytes < d3s::split_counter_bytes()) split_bytes = d3s::split_counter_bytes();
  split_bytes = (split_bytes + 255) & ~(size_t)255;
  const size_t total = split_bytes + (retry_idx ? 0 : (size_t)n_rows * sizeof(int32_t));
  void *ws = d3s::stream_workspace(s, total);
  if (!ws) return D3S_ERR_NOMEM;
  int32_t *fi = first_idx ? first_idx : main_tok;
  int32_t *ri = retry_idx ? retry_idx : (int32_t *)((char *)ws + split_bytes);
  r.first.ids = fi;
  r.retry.ids = ri;
  void *split_ws = ws;
  int rc = sample_routed(r.first, dt, s, split_ws, split_bytes, false);
  if (rc == D3S_OK) rc = sample_routed(r.retry, dt, s, split_ws, split_bytes, false);
  if (rc != D3S_OK) return rc;
  d3s::launch_ras_select(r, fi, ri, s);
  return launched();
}

int d3s_linear_bf16(const uint16_t *x, const uint16_t *w, int64_t n_rows, int64_t K, int64_t V,
                    uint16_t *y, void *stream) {
  if (n_rows < 0 || n_rows > 65535 || K < 128 || K % 128 != 0 || K > (1 << 20) || V < 1 || V > (1 << 24))
    return D3S_ERR_ARG;
  if (n_rows == 0) return D3S_OK;
  if (!x || !w || !y) return D3S_ERR_ARG;
  if ((uintptr_t)x % 8u != 0u || (uintptr_t)w % 8u != 0u || (uintptr_t)y % 2u != 0u) return D3S_ERR_ARG;
  d3s::LinearArgs la;
  la.x = x;
  la.w = w;
  la.K = (int)K;
  la.V = (int)V;
  la.n_rows = (int)n_rows;
  la.y = y;
  d3s::launch_linear(la, (hipStream_t)stream);
  return launched();
}

int d3s_linear_sample_bf16(const uint16_t *x, const uint16_t *w, int64_t n_rows, int64_t K, int64_t V,
                           uint16_t *y, const float *u, int k, const float *temperature, const float *top_p,
                           float temperature_scalar, float top_p_scalar, int32_t *ids, float *probs,
                           int32_t *cand, uint32_t *counters, unsigned flags, void *stream) {
  if (n_rows < 0 || n_rows > 65535 || K < 128 || K % 128 != 0 || K > (1 << 20) || V < 1 || V > (1 << 24) ||
      k < 1 || k > V)
    return D3S_ERR_ARG;
  if (n_rows == 0) return D3S_OK;
  if (!x || !w || !u || !ids) return D3S_ERR_ARG;
  if ((uintptr_t)x % 8u != 0u || (uintptr_t)w % 8u != 0u || (uintptr_t)y % 2u != 0u) return D3S_ERR_ARG;
  if ((flags & ~(D3S_FLAG_GENERIC | D3S_FLAG_EXACT_LSE | D3S_FLAG_EXACT_SELECT | D3S_FLAG_OP_GRAPH |
                 D3S_FLAG_ONE_LAUNCH)) != 0u)
    return D3S_ERR_ARG;
  const bool one_launch = (flags & D3S_FLAG_ONE_LAUNCH) != 0u;
  flags &= ~D3S_FLAG_ONE_LAUNCH;
  d3s::LinearArgs la;
  la.x = x;
  la.w = w;
  la.K = (int)K;
  la.V = (int)V;
  la.n_rows = (int)n_rows;
  la.y = y;
  d3s::SampleArgs a;
  a.logits = y;
  a.row_stride = V;
  a.vocab = (int)V;
  a.k = k;
  a.n_rows = (int)n_rows;
  a.u = u;
  a.temperature = temperature;
  a.top_p = top_p;
  a.temperature_scalar = temperature_scalar;
  a.top_p_scalar = top_p_scalar;
  a.banned = nullptr;
  a.ids = ids;
  a.probs = probs;
  a.cand = cand;
  a.counters = counters;
  a.flags = flags;
  a.opgraph = d3s::op_graph_order(a.vocab, k, (flags & D3S_FLAG_OP_GRAPH) || env_no_fused());
  hipStream_t s = (hipStream_t)stream;
  if (one_launch && !(flags & D3S_FLAG_GENERIC) && k <= 64 && V <= d3s::head_max_vocab() &&
      n_rows <= d3s::head_max_rows()) {
    const size_t need = d3s::head_workspace_bytes(la);
    void *ws = d3s::stream_workspace(s, need);
    if (!ws) return D3S_ERR_NOMEM;
    if (d3s::launch_head(la, a, ws, need, s)) return launched();
  }
  /* the gemv, then the routed sample on its logits (into y, or else the
   * stream's workspace after the segmented kernel's counters and records) */
  size_t split_bytes = routed_workspace_bytes(a, d3s::DT_BF16);
  if (split_bytes < d3s::split_counter_bytes()) split_bytes = d3s::split_counter_bytes();
  split_bytes = (split_bytes + 255) & ~(size_t)255;
  const size_t total = split_bytes + (y ? 0 : (size_t)n_rows * (size_t)V * 2);
  void *ws = d3s::stream_workspace(s, total);
  if (!ws) return D3S_ERR_NOMEM;
  if (!y) {
    la.y = (uint16_t *)((char *)ws + split_bytes);
    a.logits = la.y;
  }
  d3s::launch_linear(la, s);
  const int rc = launched();
  if (rc != D3S_OK) return rc;
  return sample_routed(a, d3s::DT_BF16, s, ws, split_bytes, false);
}

int d3s_uniform_fill(float *u, int64_t n, uint64_t seed, uint64_t draw, void *stream) {
  if (n < 0 || (n > 0 && !u)) return D3S_ERR_ARG;
  d3s::launch_uniform(u, n, seed, draw, (hipStream_t)stream);
  return n > 0 ? launched() : D3S_OK;
}

int d3s_max_k(void) { return 1 << 26; }

int d3s_fused_max_vocab(int dtype) {
  if (dtype != D3S_DTYPE_F32 && dtype != D3S_DTYPE_BF16) return D3S_ERR_DTYPE;
  return d3s::fused_max_vocab(dtype == D3S_DTYPE_F32 ? d3s::DT_F32 : d3s::DT_BF16);
}

int d3s_math_selftest(const float *in, float *out_exp, float *out_log, float *out_div,
                      uint64_t *out_fix, int64_t n, float divisor, void *stream) {
  if (n < 0 || (n > 0 && (!in || !out_exp || !out_log || !out_div || !out_fix))) return D3S_ERR_ARG;
  d3s::launch_math_selftest(in, out_exp, out_log, out_div, out_fix, n, divisor, (hipStream_t)stream);
  return n > 0 ? launched() : D3S_OK;
}

int d3s_exp2_selftest(const float *in, float *out, int64_t n, void *stream) {
  if (n < 0 || (n > 0 && (!in || !out))) return D3S_ERR_ARG;
  d3s::launch_exp2_selftest(in, out, n, (hipStream_t)stream);
  return n > 0 ? launched() : D3S_OK;
}

int d3s_log2_selftest(const float *in, float *out, int64_t n, void *stream) {
  if (n < 0 || (n > 0 && (!in || !out))) return D3S_ERR_ARG;
  d3s::launch_log2_selftest(in, out, n, (hipStream_t)stream);
  return n > 0 ? launched() : D3S_OK;
}

const char *d3s_version(void) { return "d3sampler 0.2 gfx950"; }

}  // extern "C"
