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
#include <memory>
#include <mutex>
#include <utility>
#include <vector>

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
using Key = std::pair<int, uintptr_t>; /* (device, stream) */
std::mutex g_ws_mutex;
std::map<Key, Block> g_ws;
/* blocks a stream has outgrown: a call on another thread may have taken one
 * before it grew and still be enqueueing on it, so they are kept until the
 * stream's block is released */
std::map<Key, std::vector<void *>> g_retired;
/* one lock per key, never freed (a stream handle reused later takes it again) */
std::map<Key, std::unique_ptr<std::recursive_mutex>> g_call_locks;
}  // namespace

/* Held by a call that uses the stream's workspace block while it enqueues:
 * a call is several launches that keep their state in the block (the
 * sorting kernels' keys, the segmented kernel's records), so the launches
 * of two calls on one stream from different host threads must not
 * interleave.  (Recursive: a call may make another through the C-ABI.) */
std::unique_lock<std::recursive_mutex> stream_call_lock(hipStream_t s) {
  int dev = 0;
  (void)hipGetDevice(&dev);
  std::recursive_mutex *m = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    std::unique_ptr<std::recursive_mutex> &p = g_call_locks[Key{dev, (uintptr_t)s}];
    if (!p) p = std::make_unique<std::recursive_mutex>();
    m = p.get();
  }
  return std::unique_lock<std::recursive_mutex>(*m);
}

void *stream_workspace(hipStream_t s, size_t bytes) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> lock(g_ws_mutex);
  const Key key{dev, (uintptr_t)s};
  Block &b = g_ws[key];
  if (b.bytes >= bytes) return b.ptr;
  const size_t want = (bytes + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1); /* whole MiB */
  void *p = nullptr;
  if (hipMalloc(&p, want) != hipSuccess) return nullptr;
  if (hipMemset(p, 0, want) != hipSuccess) {
    (void)hipFree(p);
    return nullptr;
  }
  if (b.ptr) g_retired[key].push_back(b.ptr);
  b.ptr = p;
  b.bytes = want;
  return p;
}

int release_stream_workspace(hipStream_t s) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return D3S_ERR_LAUNCH;
  if (hipStreamSynchronize(s) != hipSuccess) return D3S_ERR_LAUNCH;
  std::lock_guard<std::mutex> lock(g_ws_mutex);
  const Key key{dev, (uintptr_t)s};
  auto it = g_ws.find(key);
  if (it != g_ws.end()) {
    if (it->second.ptr) (void)hipFree(it->second.ptr);
    g_ws.erase(it);
  }
  auto rt = g_retired.find(key);
  if (rt != g_retired.end()) {
    for (void *p : rt->second) (void)hipFree(p);
    g_retired.erase(rt);
  }
  return D3S_OK;
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

/* Where a call's workspace comes from: the block the library keeps for the
 * stream (allocated on the first call that needs one), the allocation-free
 * entry point's static scratch, or the caller's memory. */
struct Ws {
  void *ptr = nullptr;
  size_t bytes = 0;
  bool lazy = true; /* take the stream's block when a route needs one */
  int short_rc = D3S_ERR_NOMEM; /* status when a route needs more than `bytes` */
};

Ws stream_ws() { return Ws{}; }
Ws fixed_ws(void *ptr, size_t bytes, int short_rc) {
  Ws w;
  w.ptr = ptr;
  w.bytes = ptr ? bytes : 0;
  w.lazy = false;
  w.short_rc = short_rc;
  return w;
}

/* the first kernel that holds the row: one wave, the rows cut into segments
 * over many CUs (with a workspace), the fused workgroup (kernel order only),
 * the wide workgroup, the nucleus kernel, the streaming one, else the sorting
 * kernels (with a workspace) */
int sample_routed(const d3s::SampleArgs &a, d3s::Dtype dt, hipStream_t s, Ws w) {
  const bool generic = (a.flags & D3S_FLAG_GENERIC) != 0u;
  if (!generic && d3s::launch_wave(a, dt, s)) return launched();
  if (!generic && d3s::split_segments(a, dt) > 0) {
    const size_t need = d3s::split_workspace_bytes(a, dt);
    if (!w.ptr && w.lazy) {
      w.ptr = d3s::stream_workspace(s, need);
      w.bytes = w.ptr ? need : 0;
    }
    if (w.ptr && d3s::launch_split(a, dt, w.ptr, w.bytes, s)) return launched();
  }
  if (!generic && !a.opgraph && d3s::launch_fused(a, dt, s)) return launched();
  if (!generic && d3s::launch_wide(a, dt, s)) return launched();
  if (!generic && a.k > 64 && a.vocab <= d3s::topp_max_vocab()) {
    const size_t need = d3s::topp_workspace_bytes(a);
    if (need > 0 && !w.ptr && w.lazy) {
      w.ptr = d3s::stream_workspace(s, need);
      w.bytes = w.ptr ? need : 0; /* without one: the full path for every row */
    }
    if (d3s::launch_topp(a, dt, w.ptr, w.bytes, s)) return launched();
  }
  if (a.k > d3s::generic_max_k()) { /* the sorting kernels, their keys after the counters' block */
    const size_t off = d3s::split_counter_bytes();
    if (!w.ptr && w.lazy) {
      const size_t need = routed_workspace_bytes(a, dt);
      w.ptr = d3s::stream_workspace(s, need);
      if (!w.ptr) return D3S_ERR_NOMEM;
      w.bytes = need;
    }
    if (!w.ptr || w.bytes < off + d3s::bigk_row_bytes(a)) return w.short_rc;
    if (!d3s::launch_bigk(a, dt, (char *)w.ptr + off, w.bytes - off, s)) return w.short_rc;
    return launched();
  }
  if (!d3s::launch_generic(a, dt, s)) return D3S_ERR_UNSUPPORTED;
  return launched();
}

/* the size checks every sampling entry point shares; D3S_OK when the row
 * shape is taken */
int check_shape(int64_t n_rows, int64_t vocab, int64_t row_stride, int64_t k) {
  if (n_rows < 0 || n_rows > 0x7fffffff || vocab < 1 || row_stride < vocab || k < 1 || k > vocab)
    return D3S_ERR_ARG;
  if (vocab > D3S_MAX_VOCAB) return D3S_ERR_UNSUPPORTED;
  return D3S_OK;
}

constexpr unsigned SAMPLE_FLAGS = D3S_FLAG_GENERIC | D3S_FLAG_EXACT_LSE | D3S_FLAG_EXACT_SELECT | D3S_FLAG_OP_GRAPH;

size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }

/* a caller's workspace: the call's need must fit, and a workspace that is
 * used must be 256-byte aligned */
int check_caller_ws(const void *ws, int64_t bytes, size_t need) {
  if (bytes < 0) return D3S_ERR_ARG;
  if (need == 0) return D3S_OK;
  if ((size_t)bytes < need || !ws) return D3S_ERR_WORKSPACE;
  if ((uintptr_t)ws % 256u != 0u) return D3S_ERR_ARG;
  return D3S_OK;
}

enum class WsMode { Stream, Scratch, Caller };

/* the checks every d3s_sample form shares and its arguments, all but the
 * uniforms; D3S_OK (and n_rows 0: nothing to launch) or the status */
int sample_args(d3s::SampleArgs &a, const void *logits, int dtype, int64_t n_rows, int64_t vocab,
                int64_t row_stride, int k, const float *temperature, const float *top_p,
                float temperature_scalar, float top_p_scalar, const int32_t *banned, int32_t *ids, float *probs,
                int32_t *cand, uint32_t *counters, unsigned flags) {
  if (dtype != D3S_DTYPE_F32 && dtype != D3S_DTYPE_BF16) return D3S_ERR_DTYPE;
  const int shape = check_shape(n_rows, vocab, row_stride, k);
  if (shape != D3S_OK) return shape;
  if ((flags & ~SAMPLE_FLAGS) != 0u) return D3S_ERR_ARG;
  if (n_rows == 0) return D3S_OK;
  if (!logits || !ids) return D3S_ERR_ARG;
  /* rows are addressed in whole elements */
  if ((uintptr_t)logits % (dtype == D3S_DTYPE_F32 ? 4u : 2u) != 0u) return D3S_ERR_ARG;
  a.logits = logits;
  a.row_stride = row_stride;
  a.vocab = (int)vocab;
  a.k = k;
  a.n_rows = (int)n_rows;
  a.u = nullptr;
  a.u_seed = 0;
  a.u_stream = 0;
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
  return D3S_OK;
}

/* d3s_sample's checks and routing, with the workspace from the stream's
 * block, the static scratch or the caller */
int sample_call(const void *logits, int dtype, int64_t n_rows, int64_t vocab, int64_t row_stride,
                const float *u, int k, const float *temperature, const float *top_p, float temperature_scalar,
                float top_p_scalar, const int32_t *banned, int32_t *ids, float *probs, int32_t *cand,
                uint32_t *counters, unsigned flags, void *stream, WsMode mode, void *ws = nullptr,
                int64_t ws_bytes = 0) {
  d3s::SampleArgs a;
  const int arc = sample_args(a, logits, dtype, n_rows, vocab, row_stride, k, temperature, top_p,
                              temperature_scalar, top_p_scalar, banned, ids, probs, cand, counters, flags);
  if (arc != D3S_OK || n_rows == 0) return arc;
  if (!u) return D3S_ERR_ARG;
  a.u = u;
  const d3s::Dtype dt = dtype == D3S_DTYPE_F32 ? d3s::DT_F32 : d3s::DT_BF16;
  hipStream_t s = (hipStream_t)stream;
  const size_t need = routed_workspace_bytes(a, dt);
  if (mode == WsMode::Stream) return sample_routed(a, dt, s, stream_ws());
  if (mode == WsMode::Caller) {
    const int rc = check_caller_ws(ws, ws_bytes, need);
    if (rc != D3S_OK) return rc;
    return sample_routed(a, dt, s, fixed_ws(need ? ws : nullptr, (size_t)ws_bytes, D3S_ERR_WORKSPACE));
  }
  void *p = nullptr;
  if (need > 0) { /* the segmented kernel, the sorting kernels one row at a time, or the nucleus
                     ids path's filed rows (more rows than the scratch lists: the full path) */
    if (d3s::split_segments(a, dt) > 0 && need > D3S_SCRATCH_BYTES) return D3S_ERR_SCRATCH;
    p = device_scratch();
    if (!p) return D3S_ERR_LAUNCH;
  }
  return sample_routed(a, dt, s, fixed_ws(p, D3S_SCRATCH_BYTES, D3S_ERR_SCRATCH));
}

/* the repetition-aware draw's arguments, shared by its entry points and its
 * size query (logits and outputs may be null for the query) */
int ras_args(d3s::RasArgs &r, const void *logits, int dtype, int64_t n_rows, int64_t vocab,
             int64_t row_stride, const float *u, const float *u_retry, const int32_t *history,
             int history_len, const d3s_ras_params *params, int32_t *main_tok, int32_t *code0,
             int32_t *first_idx, int32_t *retry_idx, uint32_t *counters) {
  if (dtype != D3S_DTYPE_F32 && dtype != D3S_DTYPE_BF16) return D3S_ERR_DTYPE;
  if (!params || params->top_k < 1 || params->retry_top_k < 1 || history_len < 0 || history_len > 64 ||
      (history_len > 0 && !history) || params->code_vocab < 1)
    return D3S_ERR_ARG;
  const int shape = check_shape(n_rows, vocab, row_stride, 1);
  if (shape != D3S_OK) return shape;
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
  return D3S_OK;
}

/* The repetition-aware draw's workspace when it runs as two routed draws and
 * the pick: the routes' (both draws use it in turn), then the retry's indices
 * when the caller keeps neither retry_idx nor code0, placed past the
 * counters' block (which must stay zero for later launches).  *idx_off: where
 * the indices go. */
size_t ras_workspace_need(const d3s::RasArgs &r, d3s::Dtype dt, bool has_retry_out, size_t *idx_off) {
  size_t split_bytes = routed_workspace_bytes(r.first, dt);
  const size_t split_retry = routed_workspace_bytes(r.retry, dt);
  if (split_retry > split_bytes) split_bytes = split_retry;
  split_bytes = round256(split_bytes);
  if (has_retry_out) return split_bytes;
  const size_t off = split_bytes > d3s::split_counter_bytes() ? split_bytes : d3s::split_counter_bytes();
  if (idx_off) *idx_off = off;
  return off + round256((size_t)r.first.n_rows * sizeof(int32_t));
}

int ras_call(const void *logits, int dtype, int64_t n_rows, int64_t vocab, int64_t row_stride, const float *u,
             const float *u_retry, const int32_t *history, int history_len, const d3s_ras_params *params,
             int32_t *main_tok, int32_t *code0, int32_t *first_idx, int32_t *retry_idx, uint32_t *counters,
             void *stream, WsMode mode, void *ws = nullptr, int64_t ws_bytes = 0) {
  d3s::RasArgs r;
  const int arc = ras_args(r, logits, dtype, n_rows, vocab, row_stride, u, u_retry, history, history_len, params,
                           main_tok, code0, first_idx, retry_idx, counters);
  if (arc != D3S_OK) return arc;
  if (n_rows == 0) return D3S_OK;
  if (!logits || !u || !u_retry || !main_tok) return D3S_ERR_ARG;
  if ((uintptr_t)logits % (dtype == D3S_DTYPE_F32 ? 4u : 2u) != 0u) return D3S_ERR_ARG;
  const d3s::Dtype dt = dtype == D3S_DTYPE_F32 ? d3s::DT_F32 : d3s::DT_BF16;
  hipStream_t s = (hipStream_t)stream;
  if (d3s::launch_ras(r, dt, s)) return launched();
  /* rows the fused kernel does not hold (k above 64, or wider than one wave's
   * registers): the two draws as routed launches, then the pick.  The first
   * draw's indices go to first_idx or else main_tok, the retry's to retry_idx,
   * else code0, else the workspace (the pick reads each row's indices before
   * it writes that row's outputs). */
  int32_t *retry_out = retry_idx ? retry_idx : code0;
  size_t idx_off = 0;
  const size_t need = ras_workspace_need(r, dt, retry_out != nullptr, &idx_off);
  void *p = nullptr;
  if (mode == WsMode::Caller) {
    const int rc = check_caller_ws(ws, ws_bytes, need);
    if (rc != D3S_OK) return rc;
    p = need ? ws : nullptr;
  } else if (need > 0) {
    p = d3s::stream_workspace(s, need);
    if (!p) return D3S_ERR_NOMEM;
  }
  int32_t *fi = first_idx ? first_idx : main_tok;
  int32_t *ri = retry_out ? retry_out : (int32_t *)((char *)p + idx_off);
  r.first.ids = fi;
  r.retry.ids = ri;
  const Ws w = fixed_ws(p, need, mode == WsMode::Caller ? D3S_ERR_WORKSPACE : D3S_ERR_NOMEM);
  int rc = sample_routed(r.first, dt, s, w);
  if (rc == D3S_OK) rc = sample_routed(r.retry, dt, s, w);
  if (rc != D3S_OK) return rc;
  d3s::launch_ras_select(r, fi, ri, s);
  return launched();
}

constexpr unsigned LINEAR_FLAGS = SAMPLE_FLAGS | D3S_FLAG_ONE_LAUNCH;

int check_linear_shape(int64_t n_rows, int64_t K, int64_t V) {
  if (n_rows < 0 || n_rows > 65535 || K < 128 || K % 128 != 0 || K > (1 << 20) || V < 1 || V > (1 << 24))
    return D3S_ERR_ARG;
  return D3S_OK;
}

/* the head's gemv and sample: arguments of both, shared by the entry points
 * and the size query */
int linear_sample_args(d3s::LinearArgs &la, d3s::SampleArgs &a, const uint16_t *x, const uint16_t *w,
                       int64_t n_rows, int64_t K, int64_t V, uint16_t *y, const float *u, int k,
                       const float *temperature, const float *top_p, float temperature_scalar,
                       float top_p_scalar, int32_t *ids, float *probs, int32_t *cand, uint32_t *counters,
                       unsigned flags) {
  if (check_linear_shape(n_rows, K, V) != D3S_OK || k < 1 || k > V) return D3S_ERR_ARG;
  if (V > D3S_MAX_VOCAB) return D3S_ERR_UNSUPPORTED;
  if ((flags & ~LINEAR_FLAGS) != 0u) return D3S_ERR_ARG;
  la.x = x;
  la.w = w;
  la.K = (int)K;
  la.V = (int)V;
  la.n_rows = (int)n_rows;
  la.y = y;
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
  a.flags = flags & ~D3S_FLAG_ONE_LAUNCH;
  a.opgraph = d3s::op_graph_order(a.vocab, k, (flags & D3S_FLAG_OP_GRAPH) || env_no_fused());
  return D3S_OK;
}

bool head_one_launch(const d3s::SampleArgs &a, unsigned flags, int64_t n_rows, int64_t V, int k) {
  return (flags & D3S_FLAG_ONE_LAUNCH) && !(flags & D3S_FLAG_GENERIC) && k <= 64 && V <= d3s::head_max_vocab() &&
         n_rows <= d3s::head_max_rows();
}

/* the two launches' workspace: the routed sample's, then the logits when the
 * caller keeps none (past the counters' block); *y_off: where they go */
size_t linear_two_need(const d3s::SampleArgs &a, bool keeps_logits, size_t *y_off) {
  const size_t split_bytes = round256(routed_workspace_bytes(a, d3s::DT_BF16));
  if (keeps_logits) return split_bytes;
  const size_t off = split_bytes > d3s::split_counter_bytes() ? split_bytes : d3s::split_counter_bytes();
  if (y_off) *y_off = off;
  return off + round256((size_t)a.n_rows * (size_t)a.vocab * 2);
}

int linear_sample_call(const uint16_t *x, const uint16_t *w, int64_t n_rows, int64_t K, int64_t V, uint16_t *y,
                       const float *u, int k, const float *temperature, const float *top_p,
                       float temperature_scalar, float top_p_scalar, int32_t *ids, float *probs, int32_t *cand,
                       uint32_t *counters, unsigned flags, void *stream, WsMode mode, void *ws = nullptr,
                       int64_t ws_bytes = 0) {
  d3s::LinearArgs la;
  d3s::SampleArgs a;
  const int arc = linear_sample_args(la, a, x, w, n_rows, K, V, y, u, k, temperature, top_p, temperature_scalar,
                                     top_p_scalar, ids, probs, cand, counters, flags);
  if (arc != D3S_OK) return arc;
  if (n_rows == 0) return D3S_OK;
  if (!x || !w || !u || !ids) return D3S_ERR_ARG;
  if ((uintptr_t)x % 8u != 0u || (uintptr_t)w % 8u != 0u || (uintptr_t)y % 2u != 0u) return D3S_ERR_ARG;
  hipStream_t s = (hipStream_t)stream;
  if (head_one_launch(a, flags, n_rows, V, k)) {
    const size_t need = d3s::head_workspace_bytes(la);
    void *p = nullptr;
    if (mode == WsMode::Caller) {
      const int rc = check_caller_ws(ws, ws_bytes, need);
      if (rc != D3S_OK) return rc;
      p = ws;
    } else {
      p = d3s::stream_workspace(s, need);
      if (!p) return D3S_ERR_NOMEM;
    }
    if (d3s::launch_head(la, a, p, need, s)) return launched();
  }
  /* the gemv, then the routed sample on its logits (into y, or else the
   * workspace after the counters' block) */
  size_t y_off = 0;
  const size_t need = linear_two_need(a, y != nullptr, &y_off);
  void *p = nullptr;
  if (mode == WsMode::Caller) {
    const int rc = check_caller_ws(ws, ws_bytes, need);
    if (rc != D3S_OK) return rc;
    p = need ? ws : nullptr;
  } else if (need > 0) {
    p = d3s::stream_workspace(s, need);
    if (!p) return D3S_ERR_NOMEM;
  }
  if (!y) {
    la.y = (uint16_t *)((char *)p + y_off);
    a.logits = la.y;
  }
  d3s::launch_linear(la, s);
  const int rc = launched();
  if (rc != D3S_OK) return rc;
  return sample_routed(a, d3s::DT_BF16, s,
                       fixed_ws(p, need, mode == WsMode::Caller ? D3S_ERR_WORKSPACE : D3S_ERR_NOMEM));
}

}  // namespace

extern "C" {

int d3s_sample(const void *logits, int dtype, int64_t n_rows, int64_t vocab, int64_t row_stride,
               const float *u, int k, const float *temperature, const float *top_p,
               float temperature_scalar, float top_p_scalar, const int32_t *banned,
               int32_t *ids, float *probs, int32_t *cand, uint32_t *counters, unsigned flags,
               void *stream) {
  const auto lock = d3s::stream_call_lock((hipStream_t)stream);
  return sample_call(logits, dtype, n_rows, vocab, row_stride, u, k, temperature, top_p, temperature_scalar,
                     top_p_scalar, banned, ids, probs, cand, counters, flags, stream, WsMode::Stream);
}

int d3s_sample_ws(const void *logits, int dtype, int64_t n_rows, int64_t vocab, int64_t row_stride,
                  const float *u, int k, const float *temperature, const float *top_p,
                  float temperature_scalar, float top_p_scalar, const int32_t *banned,
                  int32_t *ids, float *probs, int32_t *cand, uint32_t *counters, unsigned flags,
                  void *workspace, int64_t workspace_bytes, void *stream) {
  return sample_call(logits, dtype, n_rows, vocab, row_stride, u, k, temperature, top_p, temperature_scalar,
                     top_p_scalar, banned, ids, probs, cand, counters, flags, stream, WsMode::Caller, workspace,
                     workspace_bytes);
}

int d3s_sample_seeded(const void *logits, int dtype, int64_t n_rows, int64_t vocab, int64_t row_stride,
                      uint64_t seed, uint64_t stream_id, int k, const float *temperature, const float *top_p,
                      float temperature_scalar, float top_p_scalar, const int32_t *banned, int32_t *ids,
                      float *probs, int32_t *cand, uint32_t *counters, unsigned flags, void *stream) {
  d3s::SampleArgs a;
  const int arc = sample_args(a, logits, dtype, n_rows, vocab, row_stride, k, temperature, top_p,
                              temperature_scalar, top_p_scalar, banned, ids, probs, cand, counters, flags);
  if (arc != D3S_OK || n_rows == 0) return arc;
  a.u_seed = seed;
  a.u_stream = stream_id;
  /* the one-wave kernels draw the uniforms themselves; no other route does */
  if ((flags & D3S_FLAG_GENERIC) != 0u) return D3S_ERR_UNSUPPORTED;
  const d3s::Dtype dt = dtype == D3S_DTYPE_F32 ? d3s::DT_F32 : d3s::DT_BF16;
  if (!d3s::launch_wave(a, dt, (hipStream_t)stream)) return D3S_ERR_UNSUPPORTED;
  return launched();
}

int64_t d3s_sample_workspace_bytes(int dtype, int64_t n_rows, int64_t vocab, int k, unsigned flags) {
  if (dtype != D3S_DTYPE_F32 && dtype != D3S_DTYPE_BF16) return D3S_ERR_DTYPE;
  const int shape = check_shape(n_rows, vocab, vocab, k);
  if (shape != D3S_OK) return shape;
  if ((flags & ~SAMPLE_FLAGS) != 0u) return D3S_ERR_ARG;
  if (n_rows == 0) return 0;
  d3s::SampleArgs a{};
  a.vocab = (int)vocab;
  a.row_stride = vocab;
  a.k = k;
  a.n_rows = (int)n_rows;
  a.flags = flags;
  /* probs and cand absent: the ids-only routes, which need the most */
  return (int64_t)round256(routed_workspace_bytes(a, dtype == D3S_DTYPE_F32 ? d3s::DT_F32 : d3s::DT_BF16));
}

int d3s_workspace_init(void *workspace, int64_t bytes, void *stream) {
  if (bytes < 0 || bytes % 4 != 0 || (bytes > 0 && (!workspace || (uintptr_t)workspace % 256u != 0u)))
    return D3S_ERR_ARG;
  if (bytes == 0) return D3S_OK;
  d3s::launch_zero_fill((uint32_t *)workspace, (size_t)bytes / 4, (hipStream_t)stream);
  return launched();
}

int d3s_stream_workspace_release(void *stream) {
  const auto lock = d3s::stream_call_lock((hipStream_t)stream); /* no call mid-enqueue on the block */
  return d3s::release_stream_workspace((hipStream_t)stream);
}

int d3s_sample_noalloc(const void *logits, int dtype, int64_t n_rows, int64_t vocab, int64_t row_stride,
                       const float *u, int k, const float *temperature, const float *top_p,
                       float temperature_scalar, float top_p_scalar, const int32_t *banned,
                       int32_t *ids, float *probs, int32_t *cand, uint32_t *counters, unsigned flags,
                       void *stream) {
  return sample_call(logits, dtype, n_rows, vocab, row_stride, u, k, temperature, top_p, temperature_scalar,
                     top_p_scalar, banned, ids, probs, cand, counters, flags, stream, WsMode::Scratch);
}

int d3s_sample_ras(const void *logits, int dtype, int64_t n_rows, int64_t vocab, int64_t row_stride,
                   const float *u, const float *u_retry, const int32_t *history, int history_len,
                   const d3s_ras_params *params, int32_t *main_tok, int32_t *code0,
                   int32_t *first_idx, int32_t *retry_idx, uint32_t *counters, void *stream) {
  const auto lock = d3s::stream_call_lock((hipStream_t)stream);
  return ras_call(logits, dtype, n_rows, vocab, row_stride, u, u_retry, history, history_len, params, main_tok,
                  code0, first_idx, retry_idx, counters, stream, WsMode::Stream);
}

int d3s_sample_ras_ws(const void *logits, int dtype, int64_t n_rows, int64_t vocab, int64_t row_stride,
                      const float *u, const float *u_retry, const int32_t *history, int history_len,
                      const d3s_ras_params *params, int32_t *main_tok, int32_t *code0,
                      int32_t *first_idx, int32_t *retry_idx, uint32_t *counters, void *workspace,
                      int64_t workspace_bytes, void *stream) {
  return ras_call(logits, dtype, n_rows, vocab, row_stride, u, u_retry, history, history_len, params, main_tok,
                  code0, first_idx, retry_idx, counters, stream, WsMode::Caller, workspace, workspace_bytes);
}

int64_t d3s_sample_ras_workspace_bytes(int dtype, int64_t n_rows, int64_t vocab, const d3s_ras_params *params,
                                       int has_retry_out) {
  d3s::RasArgs r;
  const int arc = ras_args(r, nullptr, dtype, n_rows, vocab, vocab, nullptr, nullptr, nullptr, 0, params,
                           nullptr, nullptr, nullptr, nullptr, nullptr);
  if (arc != D3S_OK) return arc;
  if (n_rows == 0) return 0;
  const d3s::Dtype dt = dtype == D3S_DTYPE_F32 ? d3s::DT_F32 : d3s::DT_BF16;
  /* the one-launch kernel takes the rows at any start offset: no workspace */
  if (r.first.k <= 64 && r.retry.k <= 64 && r.first.vocab <= d3s::wave_max_vocab(dt)) return 0;
  return (int64_t)ras_workspace_need(r, dt, has_retry_out != 0, nullptr);
}

int d3s_linear_bf16(const uint16_t *x, const uint16_t *w, int64_t n_rows, int64_t K, int64_t V,
                    uint16_t *y, void *stream) {
  if (check_linear_shape(n_rows, K, V) != D3S_OK) return D3S_ERR_ARG;
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
  const auto lock = d3s::stream_call_lock((hipStream_t)stream);
  return linear_sample_call(x, w, n_rows, K, V, y, u, k, temperature, top_p, temperature_scalar, top_p_scalar, ids,
                            probs, cand, counters, flags, stream, WsMode::Stream);
}

int d3s_linear_sample_bf16_ws(const uint16_t *x, const uint16_t *w, int64_t n_rows, int64_t K, int64_t V,
                              uint16_t *y, const float *u, int k, const float *temperature, const float *top_p,
                              float temperature_scalar, float top_p_scalar, int32_t *ids, float *probs,
                              int32_t *cand, uint32_t *counters, unsigned flags, void *workspace,
                              int64_t workspace_bytes, void *stream) {
  return linear_sample_call(x, w, n_rows, K, V, y, u, k, temperature, top_p, temperature_scalar, top_p_scalar, ids,
                            probs, cand, counters, flags, stream, WsMode::Caller, workspace, workspace_bytes);
}

int64_t d3s_linear_sample_workspace_bytes(int64_t n_rows, int64_t K, int64_t V, int k, unsigned flags,
                                          int keeps_logits) {
  d3s::LinearArgs la;
  d3s::SampleArgs a;
  const int arc = linear_sample_args(la, a, nullptr, nullptr, n_rows, K, V, nullptr, nullptr, k, nullptr, nullptr,
                                     1.0f, 1.0f, nullptr, nullptr, nullptr, nullptr, flags);
  if (arc != D3S_OK) return arc;
  if (n_rows == 0) return 0;
  size_t need = linear_two_need(a, keeps_logits != 0, nullptr);
  if (head_one_launch(a, flags, n_rows, V, k)) {
    const size_t head = d3s::head_workspace_bytes(la);
    if (head > need) need = head;
  }
  return (int64_t)round256(need);
}

int d3s_uniform_fill(float *u, int64_t n, uint64_t seed, uint64_t draw, void *stream) {
  if (n < 0 || (n > 0 && !u)) return D3S_ERR_ARG;
  d3s::launch_uniform(u, n, seed, draw, (hipStream_t)stream);
  return n > 0 ? launched() : D3S_OK;
}

int d3s_max_k(void) { return D3S_MAX_VOCAB; }

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
