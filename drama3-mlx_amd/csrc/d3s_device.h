/* Wave64 building blocks shared by the sampler kernels (gfx950): DPP scans and
 * reductions, order-preserving composite keys, per-row parameters, the
 * reference kernel's sequential sums and its race (src/sampling.c:123-139).
 * Device code only; every translation unit gets its own copy. */
#ifndef D3S_DEVICE_H
#define D3S_DEVICE_H

#include "d3s_internal.h"
#include "d3s_math.h"

#include <type_traits>

namespace d3s {
namespace {

constexpr int WAVE = 64;
constexpr int KF = 64;                      /* fused kernel's largest k */
constexpr int NB = 256;                     /* histogram bins */

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & (WAVE - 1)); }

/* ---- wave64 primitives on DPP (gfx9 row_shr / row_bcast lane movement) ----
 * A Kogge-Stone scan within each row of 16 lanes (row_shr 1, 2, 4, 8), then
 * row_bcast:15 / row_bcast:31 carry row totals forward: lane i ends with the
 * combination of lanes 0..i, lane 63 with the whole wave.  Lanes without a
 * source keep the identity passed as `old`. */
constexpr int DPP_SHR1 = 0x111, DPP_SHR2 = 0x112, DPP_SHR4 = 0x114, DPP_SHR8 = 0x118;
constexpr int DPP_BCAST15 = 0x142, DPP_BCAST31 = 0x143;

template <int CTRL, int ROWM>
__device__ __forceinline__ uint32_t dpp_u(uint32_t old, uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROWM, 0xf, false);
}
template <int CTRL, int ROWM>
__device__ __forceinline__ float dpp_f(float old, float v) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, ROWM, 0xf, false));
}

__device__ __forceinline__ float readlane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ uint32_t readlane_u(uint32_t v, int l) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, l);
}

/* inclusive prefix sum over the wave */
__device__ __forceinline__ uint32_t wave_scan_add_u32(uint32_t v) {
  v += dpp_u<DPP_SHR1, 0xf>(0u, v);
  v += dpp_u<DPP_SHR2, 0xf>(0u, v);
  v += dpp_u<DPP_SHR4, 0xf>(0u, v);
  v += dpp_u<DPP_SHR8, 0xf>(0u, v);
  v += dpp_u<DPP_BCAST15, 0xa>(0u, v);
  v += dpp_u<DPP_BCAST31, 0xc>(0u, v);
  return v;
}

/* wave-uniform results (lane 63's scan value, read into a scalar) */
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) { return readlane_u(wave_scan_add_u32(v), 63); }

/* the maximum over the wave of values that are never NaN (callers screen
 * NaN first).  v_maximum3_f32 (IEEE maximum) needs no quieting of its
 * operands, where fmaxf's minNum semantics make the compiler canonicalise
 * both at every step. */
__device__ __forceinline__ float wave_max_f(float v) {
  const float ninf = -__builtin_inff();
  v = __builtin_elementwise_maximum(v, dpp_f<DPP_SHR1, 0xf>(ninf, v));
  v = __builtin_elementwise_maximum(v, dpp_f<DPP_SHR2, 0xf>(ninf, v));
  v = __builtin_elementwise_maximum(v, dpp_f<DPP_SHR4, 0xf>(ninf, v));
  v = __builtin_elementwise_maximum(v, dpp_f<DPP_SHR8, 0xf>(ninf, v));
  v = __builtin_elementwise_maximum(v, dpp_f<DPP_BCAST15, 0xa>(ninf, v));
  v = __builtin_elementwise_maximum(v, dpp_f<DPP_BCAST31, 0xc>(ninf, v));
  return readlane_f(v, 63);
}

/* sum of per-lane values below 2^45 (fixed-point partial sums): two 32-bit
 * scans of the high and low parts, recombined */
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
  const uint32_t lo = wave_sum_u32((uint32_t)(v & 0xffffffu));
  const uint32_t hi = wave_sum_u32((uint32_t)(v >> 24));
  return ((uint64_t)hi << 24) + lo;
}

/* inclusive prefix sum over the wave of per-lane values below 2^40 (lane i
 * gets lanes 0..i), exact: the low 24 bits and the rest scanned apart */
__device__ __forceinline__ uint64_t wave_scan_u64(uint64_t v) {
  const uint32_t lo = wave_scan_add_u32((uint32_t)(v & 0xffffffu));
  const uint32_t hi = wave_scan_add_u32((uint32_t)(v >> 24));
  return ((uint64_t)hi << 24) + lo;
}

/* inclusive prefix sum over the wave in fp32 (a fixed tree order; its
 * rounding is within the usual (n - 1) 2^-24 bound of any order for
 * non-negative terms) */
__device__ __forceinline__ float wave_scan_add_f32(float v) {
  v = v + dpp_f<DPP_SHR1, 0xf>(0.0f, v);
  v = v + dpp_f<DPP_SHR2, 0xf>(0.0f, v);
  v = v + dpp_f<DPP_SHR4, 0xf>(0.0f, v);
  v = v + dpp_f<DPP_SHR8, 0xf>(0.0f, v);
  v = v + dpp_f<DPP_BCAST15, 0xa>(0.0f, v);
  v = v + dpp_f<DPP_BCAST31, 0xc>(0.0f, v);
  return v;
}

/* The best (score, rank) over the wave: the greatest score, ties to the
 * smaller rank (the reference's first maximum).  Wave-uniform result. */
__device__ __forceinline__ void wave_argmax(float &s, int &r) {
#define D3S_ARGMAX_STEP(CTRL, ROWM)                                        \
  {                                                                        \
    const float os = dpp_f<CTRL, ROWM>(-2.0f, s);                          \
    const int orr = (int)dpp_u<CTRL, ROWM>(0x7fffffffu, (uint32_t)r);      \
    if (os > s || (os == s && orr < r)) {                                  \
      s = os;                                                              \
      r = orr;                                                             \
    }                                                                      \
  }
  D3S_ARGMAX_STEP(DPP_SHR1, 0xf)
  D3S_ARGMAX_STEP(DPP_SHR2, 0xf)
  D3S_ARGMAX_STEP(DPP_SHR4, 0xf)
  D3S_ARGMAX_STEP(DPP_SHR8, 0xf)
  D3S_ARGMAX_STEP(DPP_BCAST15, 0xa)
  D3S_ARGMAX_STEP(DPP_BCAST31, 0xc)
#undef D3S_ARGMAX_STEP
  s = readlane_f(s, 63);
  r = (int)readlane_u((uint32_t)r, 63);
}

/* The lane of the first maximum of the wave's scores (never NaN): the
 * greatest score by a DPP maximum, then the lowest lane holding it.  The
 * same lane as wave_argmax(s, lane) gives, with half its steps. */
__device__ __forceinline__ int wave_first_max_lane(float s) {
  const float m = wave_max_f(s);
  return (int)__builtin_ctzll(__ballot(s == m));
}

__device__ __forceinline__ uint64_t composite_key(float x, int idx) {
  /* larger key = earlier rank: larger x, then the smaller index */
  return ((uint64_t)d3s_ordkey(x) << 32) | (uint64_t)(uint32_t)(~(uint32_t)idx);
}
__device__ __forceinline__ float key_x(uint64_t key) { return d3s_from_ordkey((uint32_t)(key >> 32)); }
__device__ __forceinline__ int key_idx(uint64_t key) { return (int)(~(uint32_t)key); }

/* The SampleArgs fields a row's first instructions need (its address and
 * width, the banned index, the temperature, the uniforms, k and the flags),
 * passed again as leading scalar kernel arguments ahead of the SampleArgs
 * block.  gfx950
 * preloads leading non-aggregate kernel arguments into SGPRs at wave launch
 * (kernarg preloading, 14 SGPRs here: -amdgpu-kernarg-preload-count in the
 * Makefile), so the row's loads issue at once instead of after the
 * kernarg segment's round trip (~2.6k cycles measured at batch 1); the
 * block's other fields arrive by s_load meanwhile.  56 bytes, no padding. */
#define D3S_HOT_PARAMS                                                                                    \
  const void *hot_logits, int64_t hot_stride, const int32_t *hot_banned, const float *hot_temperature,    \
      const float *hot_u, float hot_T, int hot_vocab, int hot_k, unsigned hot_flags
#define D3S_HOT_ARGS(a)                                                                                   \
  (a).logits, (a).row_stride, (a).banned, (a).temperature, (a).u, (a).temperature_scalar, (a).vocab,     \
      (a).k, (a).flags
/* a's copies of the leading arguments replaced by them (the same values) */
#define D3S_HOT_APPLY(a)                                                                                  \
  do {                                                                                                    \
    (a).logits = hot_logits;                                                                              \
    (a).row_stride = hot_stride;                                                                          \
    (a).banned = hot_banned;                                                                              \
    (a).temperature = hot_temperature;                                                                    \
    (a).u = hot_u;                                                                                        \
    (a).temperature_scalar = hot_T;                                                                       \
    (a).vocab = hot_vocab;                                                                                \
    (a).k = hot_k;                                                                                        \
    (a).flags = hot_flags;                                                                                \
  } while (0)

/* The same for kernels that draw their uniforms (u null), in the same slots
 * with other types: the seed in u's, the width, k and the flags in one word
 * (vocab | k << 16 | flags << 24: vocab < 2^16, k and flags < 2^8, checked
 * before launch) and the draw's stream in the room of k and the flags, so
 * that the draw needs no kernarg read either.  D3S_HOT_PARAMS_T(DRAW) names
 * the one list or the other for a kernel templated on DRAW. */
#define D3S_HOT_PARAMS_T(DRAW)                                                                            \
  const void *hot_logits, int64_t hot_stride, const int32_t *hot_banned, const float *hot_temperature,    \
      std::conditional_t<DRAW, uint64_t, const float *> hot_u, float hot_T,                               \
      std::conditional_t<DRAW, uint32_t, int> hot_vocab, std::conditional_t<DRAW, uint32_t, int> hot_k,   \
      unsigned hot_flags
#define D3S_DRAW_ARGS(a)                                                                                  \
  (a).logits, (a).row_stride, (a).banned, (a).temperature, (a).u_seed, (a).temperature_scalar,           \
      (uint32_t)(a).vocab | (uint32_t)(a).k << 16 | (a).flags << 24, (uint32_t)(a).u_stream,              \
      (unsigned)((a).u_stream >> 32)
#define D3S_DRAW_FITS(a) ((a).vocab < 0x10000 && (a).k < 0x100 && (a).flags < 0x100u)
#define D3S_DRAW_APPLY(a)                                                                                 \
  do {                                                                                                    \
    (a).logits = hot_logits;                                                                              \
    (a).row_stride = hot_stride;                                                                          \
    (a).banned = hot_banned;                                                                              \
    (a).temperature = hot_temperature;                                                                    \
    (a).u = nullptr;                                                                                      \
    (a).u_seed = (uint64_t)hot_u;                                                                         \
    (a).temperature_scalar = hot_T;                                                                       \
    (a).vocab = (int)(hot_vocab & 0xffffu);                                                               \
    (a).k = (int)((hot_vocab >> 16) & 0xffu);                                                             \
    (a).flags = hot_vocab >> 24;                                                                          \
    (a).u_stream = (uint64_t)hot_k | (uint64_t)hot_flags << 32;                                           \
  } while (0)

struct RowP {
  float T, top_p;
  int banned;
};

/* the row's top_p alone: kernels whose first steps must not wait on the
 * kernarg segment read it after them (the other fields of row_params are
 * leading kernel arguments) */
__device__ __forceinline__ float row_top_p(const SampleArgs &a, int row) {
  return a.top_p ? a.top_p[row] : a.top_p_scalar;
}

__device__ __forceinline__ RowP row_params(const SampleArgs &a, int row) {
  RowP p;
  float T = a.temperature ? a.temperature[row] : a.temperature_scalar;
  if (T < 1e-5f) T = 1e-5f; /* src/sampling.c:16,195 */
  p.T = T;
  p.top_p = a.top_p ? a.top_p[row] : a.top_p_scalar;
  p.banned = a.banned ? a.banned[row] : -1;
  return p;
}

/* x = logit / T, correctly rounded (y = RN(1/T)); T = +inf takes the division */
__device__ __forceinline__ float scale_logit(float L, float T, float y, bool t_finite) {
  return t_finite ? d3s_div_rn(L, T, y) : L / T;
}

/* bit 0: NaN or +inf (refused), bit 1: -inf present */
__device__ __forceinline__ uint32_t classify(float v) {
  const uint32_t b = d3s_f2u(v);
  if ((b & 0x7fffffffu) > 0x7f800000u || b == 0x7f800000u) return 1u;
  return b == 0xff800000u ? 2u : 0u;
}

/* A refused row (id -1) or an all -inf row (id 0, ranks 0..k-1); whole block. */
__device__ __forceinline__ void write_special(const SampleArgs &a, int row, bool masked) {
  const int k = a.k;
  if (threadIdx.x == 0) {
    a.ids[row] = masked ? 0 : -1;
    if (a.counters) atomicAdd(&a.counters[masked ? CNT_ALL_MASKED : CNT_REFUSED], 1u);
  }
  for (int r = threadIdx.x; r < k; r += blockDim.x) {
    if (a.probs) a.probs[(size_t)row * k + r] = __builtin_nanf("");
    if (a.cand) a.cand[(size_t)row * k + r] = masked ? r : -1;
  }
}

/* Wave-aggregated append: the lanes with `pred` get consecutive slots from
 * *counter with one atomic per wave.  Called by every lane of the wave. */
__device__ __forceinline__ int wave_append(bool pred, int *counter) {
  const uint64_t m = __ballot(pred);
  if (m == 0ull) return -1;
  int base = 0;
  if (lane_id() == 0) base = atomicAdd(counter, (int)__popcll(m));
  base = __builtin_amdgcn_readfirstlane(base);
  const int below = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                   __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
  return pred ? base + below : -1;
}

/* Make a wave's LDS writes visible to its own later LDS reads (other lanes). */
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

/* Lane r (< k) gets e_0 + e_1 + ... + e_r added left to right in fp32: the
 * reference kernel's sequential cumulative (src/sampling.c:126-127).  The
 * terms go through LDS (`buf`, 64 floats private to the wave, 16-byte
 * aligned) and every lane runs the same chain of additions on broadcast
 * reads of four terms at a time: no cross-lane round trip per step. */
__device__ __forceinline__ float wave_seq_cumsum(float e, int k, float *buf) {
  const int lane = lane_id();
  buf[lane] = lane < k ? e : 0.0f;
  wave_lds_sync();
  const float4 *b4 = (const float4 *)buf;
  float c = 0.0f, mine = 0.0f;
  for (int r4 = 0; r4 < (k + 3) / 4; r4++) {
    const float4 q = b4[r4];
    const int r = 4 * r4;
    c = c + q.x;
    mine = lane == r ? c : mine;
    c = c + q.y;
    mine = lane == r + 1 ? c : mine;
    c = c + q.z;
    mine = lane == r + 2 ? c : mine;
    c = c + q.w;
    mine = lane == r + 3 ? c : mine;
  }
  wave_lds_sync();
  return mine;
}

/* the fp32 sum e_0 + ... + e_{n-1}, left to right, in every lane (n <= 64) */
__device__ __forceinline__ float wave_seq_sum(float e, int n, float *buf) {
  const int lane = lane_id();
  buf[lane] = lane < n ? e : 0.0f;
  wave_lds_sync();
  const float4 *b4 = (const float4 *)buf;
  float s = 0.0f;
  for (int r4 = 0; r4 < n / 4; r4++) {
    const float4 q = b4[r4];
    s = s + q.x;
    s = s + q.y;
    s = s + q.z;
    s = s + q.w;
  }
  for (int r = n & ~3; r < n; r++) s = s + buf[r];
  wave_lds_sync();
  return s;
}

/* One wave; lane r < k holds rank r's x (v), index, c_r and noise -log(1 - u_r).  The
 * exclusive top-p cut, the kept sum, the probabilities and the race, in the
 * reference kernel's order (src/sampling.c:128-139); writes ids/probs/cand. */
__device__ __forceinline__ void wave_tail_finish(const SampleArgs &a, int row, float v, int idx, float c,
                                 float noise, float top_p, float *buf) {
  const int lane = lane_id();
  const int k = a.k;
  const bool act = lane < k;
  const bool drop = act && lane > 0 && c > top_p;
  const uint64_t dm = __ballot(drop);
  const int cut = dm ? __builtin_ctzll(dm) : k; /* c_r is non-decreasing: drops are a suffix */
  const float v0 = readlane_f(v, 0);
  const float ep = act ? d3s_expf(v - v0) : 0.0f;
  const float s = wave_seq_sum(ep, cut, buf);
  const float inv = 1.0f / s;
  const float p = (act && lane < cut) ? ep * inv : 0.0f;
  float sc = -1.0f;
  if (act) {
    const float score = p / noise;
    sc = score > -1.0f ? score : -1.0f; /* NaN, -inf and <= -1 never beat best = -1 */
  }
  const int best = wave_first_max_lane(sc);
  const int id = (int)readlane_u((uint32_t)idx, best);
  if (lane == 0) a.ids[row] = id;
  if (act) {
    if (a.probs) a.probs[(size_t)row * k + lane] = p;
    if (a.cand) a.cand[(size_t)row * k + lane] = idx;
  }
}

/* A wave scans a 256-bin histogram for the bin holding the `need`-th element,
 * counting from bin 0 upward (ASC) or from bin 255 downward (!ASC).  The
 * result (the bin, the count before it, its count) is wave-uniform; ok is
 * false when the histogram holds fewer than `need`. */
struct BinSel {
  bool ok;
  uint32_t bin, above, count;
};

template <bool ASC>
__device__ __forceinline__ BinSel wave_find_bin(const uint32_t *hist, uint32_t need) {
  const int lane = lane_id();
  uint32_t h[4];
#pragma unroll
  for (int q = 0; q < 4; q++) h[q] = hist[ASC ? 4 * lane + q : NB - 1 - 4 * lane - q];
  const uint32_t ls = h[0] + h[1] + h[2] + h[3];
  const uint32_t incl = wave_scan_add_u32(ls);
  const uint32_t total = readlane_u(incl, 63);
  BinSel r;
  r.ok = total >= need;
  r.bin = r.above = r.count = 0u;
  if (!r.ok) return r;
  const int L0 = __builtin_ctzll(__ballot(incl >= need));
  /* every lane walks its own four bins as if it were the selecting lane */
  uint32_t cum = incl - ls, bin = 0u, above = 0u, cnt = 0u;
  bool found = false;
#pragma unroll
  for (int q = 0; q < 4; q++) {
    if (!found && cum + h[q] >= need) {
      found = true;
      bin = (uint32_t)(ASC ? 4 * lane + q : NB - 1 - 4 * lane - q);
      above = cum;
      cnt = h[q];
    } else if (!found) {
      cum += h[q];
    }
  }
  r.bin = readlane_u(bin, L0);
  r.above = readlane_u(above, L0);
  r.count = readlane_u(cnt, L0);
  return r;
}

/* ------------------------------------------------------------------------ */
/* fused kernel                                                              */
/* ------------------------------------------------------------------------ */

/* Wave 0: the exclusive top-p cut over c_r, the kept sum of ep_r (= exp(x_r - x_0)),
 * the probabilities and the race (src/sampling.c:128-139); lane r < k holds
 * rank r's index, c_r, ep_r and noise -log(1 - u_r).  Writes ids/probs/cand. */
__device__ __forceinline__ void wave_race(const SampleArgs &a, int row, int idx, float c, float ep, float noise,
                          float top_p, float *buf) {
  const int lane = lane_id();
  const int k = a.k;
  const bool act = lane < k;
  const bool drop = act && lane > 0 && c > top_p;
  const uint64_t dm = __ballot(drop);
  const int cut = dm ? __builtin_ctzll(dm) : k; /* c_r is non-decreasing: drops are a suffix */
  const float s = wave_seq_sum(ep, cut, buf);
  const float inv = 1.0f / s;
  const float p = (act && lane < cut) ? ep * inv : 0.0f;
  float sc = -1.0f;
  if (act) {
    const float score = p / noise;
    sc = score > -1.0f ? score : -1.0f; /* NaN, -inf and <= -1 never beat best = -1 */
  }
  const int best = wave_first_max_lane(sc);
  const int id = (int)readlane_u((uint32_t)idx, best);
  if (lane == 0) a.ids[row] = id;
  if (act) {
    if (a.probs) a.probs[(size_t)row * k + lane] = p;
    if (a.cand) a.cand[(size_t)row * k + lane] = idx;
  }
}

}  // namespace
}  // namespace d3s

#endif
