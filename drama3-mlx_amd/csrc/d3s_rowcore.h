/* One-wave building blocks of the register-resident sampler kernels (gfx950,
 * wave64), shared by the one-wave kernel (d3s_wave.hip) and the segmented
 * kernel (d3s_split.hip): a row's 16-byte chunks in registers, NaN-propagating
 * wave maxima, the reference kernel's tail (src/sampling.c:123-139, or the op
 * graph's order :39-48) with the fast lse's margin test, and the race.
 * Device code only; every translation unit gets its own copy. */
#ifndef D3S_ROWCORE_H
#define D3S_ROWCORE_H

#include "d3s_generic.h"

#pragma clang fp contract(off)

namespace d3s {
namespace {

constexpr int LCAP = 8;  /* candidates a lane files before the exact select takes over */
/* relative error bound of v_exp_f32 (2^x) for every input with a normal
 * result; the GPU tests check it over dense samples of [-126, 1] */
constexpr float EPS_EXP2 = 0x1p-21f;
constexpr float LOG2E_F = 1.44269504f;
/* dword 3 of a gfx9 buffer resource: 32-bit data format, raw addressing */
constexpr int BUFFER_FLAGS = 0x00020000;
constexpr float LN2_F = 0.693147182f;

__device__ __forceinline__ float fmaximum(float a, float b) { return __builtin_elementwise_maximum(a, b); }

/* wave max that propagates NaN (v_maximum), wave-uniform */
__device__ __forceinline__ float wave_maximum_f(float v) {
  const float ninf = -__builtin_inff();
  v = fmaximum(v, dpp_f<DPP_SHR1, 0xf>(ninf, v));
  v = fmaximum(v, dpp_f<DPP_SHR2, 0xf>(ninf, v));
  v = fmaximum(v, dpp_f<DPP_SHR4, 0xf>(ninf, v));
  v = fmaximum(v, dpp_f<DPP_SHR8, 0xf>(ninf, v));
  v = fmaximum(v, dpp_f<DPP_BCAST15, 0xa>(ninf, v));
  v = fmaximum(v, dpp_f<DPP_BCAST31, 0xc>(ninf, v));
  return readlane_f(v, 63);
}

__device__ __forceinline__ float wave_sum_f(float v) {
  v = v + dpp_f<DPP_SHR1, 0xf>(0.0f, v);
  v = v + dpp_f<DPP_SHR2, 0xf>(0.0f, v);
  v = v + dpp_f<DPP_SHR4, 0xf>(0.0f, v);
  v = v + dpp_f<DPP_SHR8, 0xf>(0.0f, v);
  v = v + dpp_f<DPP_BCAST15, 0xa>(0.0f, v);
  v = v + dpp_f<DPP_BCAST31, 0xc>(0.0f, v);
  return readlane_f(v, 63);
}

/* The k-th largest of the wave's 64 lane keys to 20 bits: the largest p
 * (low 12 bits zero) that at least k lanes' keys reach, 0 when no such p
 * (fewer than k lanes reach 2^12).  A ballot search, one bit a step (faster
 * here than three counts a step).  Wave-uniform. */
__device__ __forceinline__ uint32_t wave_kth_prefix(uint32_t key, uint32_t k) {
  uint32_t pre = 0u;
#pragma unroll
  for (int bit = 31; bit >= 12; bit--) {
    const uint32_t cnd = pre | (1u << bit);
    if ((uint32_t)__popcll(__ballot(key >= cnd)) >= k) pre = cnd;
  }
  return pre;
}

__device__ __forceinline__ int mbcnt64(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

/* e_0 + e_1 + ... + e_{n-1} added left to right in fp32 (lane r holds e_r,
 * n <= 64 wave-uniform), the same value in every lane: the reference kernel's
 * kept sum (src/sampling.c:129-131).  Each term comes from its lane by
 * readlane (a scalar broadcast), so the chain is one add per term. */
__device__ __forceinline__ float wave_seq_sum_rl(float e, int n) {
  float s = 0.0f;
#pragma unroll
  for (int r = 0; r < WAVE; r++) {
    if (r >= n) break;
    s = s + readlane_f(e, r);
  }
  return s;
}

/* The race (src/sampling.c:132-139): lane r < k holds rank r's index, its
 * post-filter probability p_r and noise -log(1 - u_r); the first maximum of
 * p / noise wins (initial best -1).  Writes ids / probs / cand; returns the id. */
__device__ __forceinline__ int wave_race_p(const SampleArgs &a, int row, int idx, float p, float noise) {
  const int lane = lane_id();
  const int k = a.k;
  const bool act = lane < k;
  float sc = -1.0f;
  if (act) {
    const float score = p / noise;
    sc = score > -1.0f ? score : -1.0f; /* NaN, -inf and <= -1 never beat best = -1 */
  }
  const int best = wave_first_max_lane(sc);
  const int id = (int)readlane_u((uint32_t)idx, best);
  if (lane == 0 && a.ids) a.ids[row] = id;
  if (act) {
    if (a.probs) a.probs[(size_t)row * k + lane] = p;
    if (a.cand) a.cand[(size_t)row * k + lane] = idx;
  }
  return id;
}

/* wave_tail's answer when the cut needs the exact lse and the wave cannot
 * compute it (the caller samples the row again by an exact procedure) */
constexpr int NEED_EXACT = (int)0x80000000;

/* The tail of one row on one wave (src/sampling.c:123-139, or in the op
 * graph's order :39-48): lane r < k holds rank r's key (composite_key of x_r
 * and its index), M = x_0 = max x, noise = -log(1 - u_r).  lse is exact when
 * `exact`, else the fast one with relative error bound eps_s.
 *
 * The cut only depends on lse through c_r; the probabilities use exp(x - x_0).
 * With the fast lse the cumulative c'_r is a parallel fp32 scan of hardware
 * 2^x terms, and |c'_r - c_r| <= c'_r (eps_e + (2k + 2) 2^-24) (+ (k + 2)
 * 2^-40 in the op graph's order, whose exact prefixes truncate each term to
 * 2^-40), whichever order the two sums add in; eps_e bounds the relative
 * change of a term exp(v - lse) between the two lse values.  When no c'_r lies
 * that close to top_p, the cut from c' is the cut from c; otherwise
 * exact_lse() gives the exact lse (NaN: the wave cannot, and NEED_EXACT is
 * returned before anything is written) and c is computed in its own order.
 *  - kernel order: c_r and the kept sum are left-to-right fp32 sums in rank
 *    order, p_r = e_r (1 / sum_{r < cut} e_r);
 *  - op graph order: c_r = RN(sum_{j<=r} fix40(exp(x_j - lse)) 2^-40), the
 *    kept sum the same of exp(x_j - x_0) over the kept ranks. */
template <class ExactLse>
__device__ __forceinline__ int wave_tail(const SampleArgs &a, int row, uint64_t key, float M, float lse,
                                         bool exact, float eps_s, float noise, float top_p, float *buf,
                                         ExactLse &&exact_lse) {
  const int lane = lane_id();
  const int k = a.k;
  const bool act = lane < k;
  const float v = key_x(key);
  const int idx = key_idx(key);
  const float ep = act ? d3s_expf_nonpos(v - M) : 0.0f; /* exp(x - x_0), x_0 = m */
  float cc = 0.0f;
  if (!exact) {
    const float D = lse - readlane_f(v, k - 1); /* ranks have non-increasing x */
    const float dl = eps_s + 0x1p-18f + 0x1p-23f * (fabsf(lse) + 1.0f);
    /* a term's relative change: lse's, the rounding of v - lse on either
     * side, of its product with log2(e) and of log2(e) itself (|v - lse| <=
     * D), v_exp_f32's error and d3s_expf's */
    const float eps_e = dl + 0x1p-22f * (D + 1.0f) + 0x1p-20f;
    const float B = 1.01f * (eps_e + (float)(2 * k + 2) * 0x1p-24f);
    const float slack = a.opgraph ? (float)(k + 2) * 0x1p-40f : 0x1p-60f;
    cc = wave_scan_add_f32(act ? __builtin_amdgcn_exp2f((v - lse) * LOG2E_F) : 0.0f);
    exact = __ballot(act && lane > 0 && fabsf(cc - top_p) <= B * cc + slack) != 0ull ||
            (a.flags & FLAG_EXACT_LSE) != 0;
    if (exact) {
      if (lane == 0 && a.counters) atomicAdd(&a.counters[CNT_EXACT_LSE], 1u);
      lse = exact_lse();
      if (d3s_isnan(lse)) return NEED_EXACT;
    }
  }
  if (exact) {
    if (!a.opgraph)
      cc = wave_seq_cumsum(act ? d3s_expf_nonpos(v - lse) : 0.0f, k, buf);
    else
      cc = d3s_fixsum_to_f32(wave_scan_u64(act ? d3s_fix40_exp(v - lse) : 0ull));
  }
  const uint64_t dm = __ballot(act && lane > 0 && cc > top_p);
  const int cut = dm ? __builtin_ctzll(dm) : k; /* c_r is non-decreasing: drops are a suffix */
  const float kept = !a.opgraph ? wave_seq_sum_rl(ep, cut)
                                : d3s_fixsum_to_f32(wave_sum_u64(act && lane < cut ? d3s_fix40_unit(ep) : 0ull));
  const float inv = 1.0f / kept;
  const float p = (act && lane < cut) ? ep * inv : 0.0f;
  return wave_race_p(a, row, idx, p, noise);
}

/* A refused row (id -1) or an all -inf row (id 0, ranks 0..k-1); one wave.
 * Returns the id. */
__device__ __forceinline__ int wave_write_special(const SampleArgs &a, int row, bool masked) {
  const int lane = lane_id(), k = a.k;
  if (lane == 0) {
    if (a.ids) a.ids[row] = masked ? 0 : -1;
    if (a.counters) atomicAdd(&a.counters[masked ? CNT_ALL_MASKED : CNT_REFUSED], 1u);
  }
  if (lane < k) {
    if (a.probs) a.probs[(size_t)row * k + lane] = __builtin_nanf("");
    if (a.cand) a.cand[(size_t)row * k + lane] = masked ? lane : -1;
  }
  return masked ? 0 : -1;
}

/* relaxed agent-scope stores and loads (global_store / global_load with sc1):
 * coherent across the XCDs' L2s without a whole-cache write-back.
 * The cross-workgroup hand-offs (k_split's and k_head's records, the nucleus
 * redo kernel's counts) publish with these stores, retire them with
 * s_waitcnt vmcnt(0) in every wave, meet at a workgroup barrier, and only then
 * count the arrival with a relaxed agent-scope atomic; the last arrival reads
 * with ld_agent.  Under the LLVM AMDGPU memory model's GFX942 code sequences,
 * which gfx950 follows, monotonic agent-scope loads, stores and atomics are
 * single sc1 instructions coherent at agent scope, so a retired record store
 * is visible before the count that follows it.  (A release on the count and
 * an acquire in the reader, which order them in the C++ model, add
 * buffer_wbl2 / buffer_inv sc1, an L2 write-back and invalidate: C4 took
 * 24.4 us per launch that way against 15.4 us.) */
__device__ __forceinline__ void st_agent(uint64_t *p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_agent(const uint64_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* rank the n keys of list (n + 2 entries of room): every key counts the keys
 * above its own; those below k land in ranked by rank (PUBLISH: in global
 * memory, by agent-coherent stores and with no closing barrier: the caller
 * retires the stores before publishing).  Keys are distinct.
 * G adjacent lanes share a key (G = 4 when n <= NT / 4, 2 when n <=
 * NT / 2), each counting a share of the list; quad DPP adds the shares.
 * Called by every thread of an NT-thread workgroup. */
template <int NT, bool PUBLISH = false>
__device__ __forceinline__ void rank_by_count(uint64_t *list, uint32_t n, int k, uint64_t *ranked) {
  if (threadIdx.x == 0) {
    list[n] = 0ull; /* pads below every key */
    list[n + 1] = 0ull;
  }
  __syncthreads();
  const ulonglong2 *k2 = (const ulonglong2 *)list;
  const uint32_t lg = n <= NT / 4 ? 2u : n <= NT / 2 ? 1u : 0u; /* log2 G */
  const uint32_t np = (n + 1) / 2;                                         /* pairs */
  const uint32_t share = (np + (1u << lg) - 1) >> lg;
  const uint32_t part = threadIdx.x & ((1u << lg) - 1);
  const uint32_t p0 = min(np, part * share), p1 = min(np, p0 + share);
  for (uint32_t base = 0; base < n; base += NT >> lg) {
    const uint32_t t = base + (threadIdx.x >> lg);
    const uint64_t my = t < n ? list[t] : ~0ull;
    uint32_t rank = 0u;
#pragma unroll 4
    for (uint32_t j2 = p0; j2 < p1; j2++) {
      const ulonglong2 q = k2[j2];
      rank += (q.x > my ? 1u : 0u) + (q.y > my ? 1u : 0u);
    }
    if (lg >= 1) rank += dpp_u<0xb1, 0xf>(0u, rank); /* quad_perm [1,0,3,2] */
    if (lg >= 2) rank += dpp_u<0x4e, 0xf>(0u, rank); /* quad_perm [2,3,0,1] */
    if (part == 0 && t < n && rank < (uint32_t)k) {
      if (PUBLISH)
        st_agent(ranked + rank, my);
      else
        ranked[rank] = my;
    }
  }
  if (!PUBLISH) __syncthreads();
}

/* A row in registers: CPT 16-byte chunks per lane (chunk j * 64 + lane, from
 * the aligned address at or below the row start), 4 words each: fp32 bits or
 * two bf16 halves.  Element i of a lane is chunk row i / EPC, lane-in-chunk
 * i % EPC; index order is (chunk row, lane, lane-in-chunk). */
template <int CPT, bool BF16>
struct Chunks {
  static constexpr int EPC = BF16 ? 8 : 4; /* elements per 16-byte chunk */
  static constexpr int NV = CPT * EPC;
  uint32_t w[CPT * 4];

  /* through a buffer resource spanning the row's chunks: a chunk past the
   * row's last reads as zeros (masked by the caller), and no per-chunk
   * address arithmetic is needed */
  /* AUX: the loads' cache policy (2: nontemporal, for rows read once) */
  template <int AUX = 0>
  __device__ __forceinline__ void load(const uint4 *src, int nchunks, int lane) {
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void *)src, (short)0, nchunks * 16, BUFFER_FLAGS);
#pragma unroll
    for (int j = 0; j < CPT; j++) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, lane * 16, j * WAVE * 16, AUX);
      const uint4 q = make_uint4(v[0], v[1], v[2], v[3]);
      w[4 * j] = q.x;
      w[4 * j + 1] = q.y;
      w[4 * j + 2] = q.z;
      w[4 * j + 3] = q.w;
    }
  }
  __device__ __forceinline__ float val(int i) const {
    if (BF16) {
      const uint32_t word = w[(i / EPC) * 4 + (i % EPC) / 2];
      return d3s_u2f((i & 1) ? (word & 0xffff0000u) : (word << 16));
    }
    return d3s_u2f(w[i]);
  }
  /* element i becomes -inf when `on` */
  __device__ __forceinline__ void mask(int i, bool on) {
    uint32_t &word = w[BF16 ? (i / EPC) * 4 + (i % EPC) / 2 : i];
    if (BF16)
      word = on ? ((i & 1) ? ((word & 0x0000ffffu) | 0xff800000u) : ((word & 0xffff0000u) | 0x0000ff80u)) : word;
    else
      word = on ? 0xff800000u : word;
  }
  __device__ __forceinline__ static int pos(int pos0, int i) { return pos0 + (i / EPC) * WAVE * EPC + (i % EPC); }
  /* opaque to the compiler: a pass after this unpacks the words again
   * instead of holding every unpacked element from the pass before */
  __device__ __forceinline__ void launder() {
#pragma unroll
    for (int j = 0; j < CPT * 4; j++) asm volatile("" : "+v"(w[j]));
  }
};

}  // namespace
}  // namespace d3s

#endif
