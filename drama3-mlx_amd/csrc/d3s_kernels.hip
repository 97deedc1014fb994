/* HIP kernels of the MI355X token sampler (gfx950, wave64).
 *
 * Semantics: the sampler of SeungheonOh/drama3-mlx, src/sampling.c (temperature
 * :195,:25,:70; row log-sum-exp :37-38,:67-89; top-k ranked by (x desc, index
 * asc) :27-36,:90-121; exclusive top-p :39-42,:126-128; renormalised softmax
 * :43-44,:129-134; exponential race over caller uniforms :45-48,:132-139).
 *
 * Two kernels, one workgroup per row:
 *  - k_fused (k <= 64, row held in registers): one pass over the row computes
 *    the row max, then a second pass over the registers accumulates a fast
 *    sum of exp (hardware exp2) and a 256-bin histogram of the distance to the
 *    max; the bin holding the k-th value bounds a small candidate set that is
 *    ranked exactly.  Rows the histogram cannot settle (too many candidates,
 *    or a candidate tie across the cut) take an exact 8-bit radix select over
 *    order-preserving keys.  The fast sum of exp decides the top-p cut unless
 *    some c_r lies within the fast sum's error bound of top_p; such rows
 *    recompute the exact, order-independent log-sum-exp.  Every row therefore
 *    gets the same bits as the exact definition.
 *  - k_generic (any V, k <= 16384): streams the row from global memory for
 *    every pass; exact log-sum-exp, radix select, LDS bitonic sort of the k
 *    selected, exact-sum top-p for k > 64.  Rows wider than the fused kernel
 *    takes, k > 64 (the reference's op-graph cases), and the
 *    D3S_FLAG_GENERIC switch use it.
 */
#include <mutex>

#include "d3s_internal.h"
#include "d3s_math.h"

#pragma clang fp contract(off)

namespace d3s {
namespace {

constexpr int WAVE = 64;
constexpr int KF = 64;                      /* fused kernel's largest k */
constexpr int NB = 256;                     /* histogram bins */
constexpr float BINS_PER_NAT = 8.0f;        /* 256 bins over 32 units of x below the max */
constexpr int GCAP = 256;                   /* candidate capacity of the fused kernel */
constexpr float LOG2E = 1.44269504088896341f;

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & (WAVE - 1)); }

__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
  for (int o = WAVE / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
  for (int o = WAVE / 2; o > 0; o >>= 1) v = v + __shfl_xor(v, o);
  return v;
}

__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
  for (int o = WAVE / 2; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v) {
  const int lane = lane_id();
#pragma unroll
  for (int o = 1; o < WAVE; o <<= 1) {
    const uint32_t t = __shfl_up(v, (unsigned)o);
    if (lane >= o) v += t;
  }
  return v;
}

__device__ __forceinline__ uint64_t wave_incl_scan_u64(uint64_t v) {
  const int lane = lane_id();
#pragma unroll
  for (int o = 1; o < WAVE; o <<= 1) {
    const uint64_t t = __shfl_up(v, (unsigned)o);
    if (lane >= o) v += t;
  }
  return v;
}

__device__ __forceinline__ float readlane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

__device__ __forceinline__ uint64_t composite_key(float x, int idx) {
  /* larger key = earlier rank: larger x, then the smaller index */
  return ((uint64_t)d3s_ordkey(x) << 32) | (uint64_t)(uint32_t)(~(uint32_t)idx);
}
__device__ __forceinline__ float key_x(uint64_t key) { return d3s_from_ordkey((uint32_t)(key >> 32)); }
__device__ __forceinline__ int key_idx(uint64_t key) { return (int)(~(uint32_t)key); }

struct RowP {
  float T, top_p;
  int banned;
};

__device__ __forceinline__ RowP row_params(const SampleArgs &a, int row) {
  RowP p;
  float T = a.temperature ? a.temperature[row] : a.temperature_scalar;
  if (T < 1e-5f) T = 1e-5f; /* src/sampling.c:16,195 */
  p.T = T;
  p.top_p = a.top_p ? a.top_p[row] : a.top_p_scalar;
  p.banned = a.banned ? a.banned[row] : -1;
  return p;
}

/* bit 0: NaN or +inf (refused), bit 1: -inf present */
__device__ __forceinline__ uint32_t classify(float v) {
  const uint32_t b = d3s_f2u(v);
  if ((b & 0x7fffffffu) > 0x7f800000u || b == 0x7f800000u) return 1u;
  return b == 0xff800000u ? 2u : 0u;
}

/* A refused row (id -1) or an all -inf row (id 0, ranks 0..k-1); whole block. */
__device__ void write_special(const SampleArgs &a, int row, bool masked) {
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

/* Lane r (< k) gets e_0 + e_1 + ... + e_r added left to right in fp32: the
 * reference kernel's sequential cumulative (src/sampling.c:126-127). */
__device__ __forceinline__ float wave_seq_cumsum(float e, int k) {
  const int lane = lane_id();
  float c = 0.0f, mine = 0.0f;
  for (int r = 0; r < k; r++) {
    c = c + readlane_f(e, r);
    if (lane == r) mine = c;
  }
  return mine;
}

/* One wave; lane r < k holds rank r's x and index, and c_r.  The exclusive
 * top-p cut, the kept sum, the probabilities and the race, in the reference
 * kernel's order (src/sampling.c:128-139); writes ids/probs/cand. */
__device__ void wave_tail_finish(const SampleArgs &a, int row, float v, int idx, float c,
                                 float top_p) {
  const int lane = lane_id();
  const int k = a.k;
  const bool act = lane < k;
  const bool drop = act && lane > 0 && c > top_p;
  const uint64_t dm = __ballot(drop);
  const int cut = dm ? __builtin_ctzll(dm) : k; /* c_r is non-decreasing: drops are a suffix */
  const float v0 = readlane_f(v, 0);
  const float ep = act ? d3s_expf(v - v0) : 0.0f;
  float s = 0.0f;
  for (int r = 0; r < cut; r++) s = s + readlane_f(ep, r);
  const float inv = 1.0f / s;
  const float p = (act && lane < cut) ? ep * inv : 0.0f;
  float sc = -1.0f;
  if (act) {
    const float noise = -d3s_logf(1.0f - a.u[(size_t)row * k + lane]);
    const float score = p / noise;
    sc = score > -1.0f ? score : -1.0f; /* NaN, -inf and <= -1 never beat best = -1 */
  }
  int best = lane;
#pragma unroll
  for (int o = WAVE / 2; o > 0; o >>= 1) {
    const float os = __shfl_xor(sc, o);
    const int ob = __shfl_xor(best, o);
    if (os > sc || (os == sc && ob < best)) {
      sc = os;
      best = ob;
    }
  }
  const int id = __shfl(idx, best);
  if (lane == 0) a.ids[row] = id;
  if (act) {
    if (a.probs) a.probs[(size_t)row * k + lane] = p;
    if (a.cand) a.cand[(size_t)row * k + lane] = idx;
  }
}

/* Wave 0 scans a 256-bin histogram for the bin holding the `need`-th element,
 * counting from bin 0 upward (ASC) or from bin 255 downward (!ASC).  The
 * result (the bin, the count before it, its count) is the same in every lane;
 * ok is false when the histogram holds fewer than `need`. */
struct BinSel {
  bool ok;
  uint32_t bin, above, count;
};

template <bool ASC>
__device__ BinSel wave_find_bin(const uint32_t *hist, uint32_t need) {
  const int lane = lane_id();
  uint32_t h[4];
#pragma unroll
  for (int q = 0; q < 4; q++) h[q] = hist[ASC ? 4 * lane + q : NB - 1 - 4 * lane - q];
  const uint32_t ls = h[0] + h[1] + h[2] + h[3];
  const uint32_t incl = wave_incl_scan_u32(ls);
  const uint32_t total = __shfl(incl, WAVE - 1);
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
  r.bin = __shfl(bin, L0);
  r.above = __shfl(above, L0);
  r.count = __shfl(cnt, L0);
  return r;
}

/* ------------------------------------------------------------------------ */
/* fused kernel                                                              */
/* ------------------------------------------------------------------------ */

template <int BLOCK, int CPT, bool BF16>
__global__ __launch_bounds__(BLOCK) void k_fused(SampleArgs a) {
  constexpr int ES = BF16 ? 2 : 4;
  constexpr int EPC = 16 / ES; /* elements per 16-byte chunk */
  constexpr int NV = CPT * EPC;
  constexpr int NW = BLOCK / WAVE;
  static_assert(BLOCK >= GCAP, "one thread per candidate");

  __shared__ uint32_t hist[NB];
  __shared__ float sh_max[NW], sh_sum[NW], sh_out[NW];
  __shared__ uint32_t sh_flag[NW], sh_scan[NW];
  __shared__ uint64_t sh_q[NW];
  __shared__ uint64_t gK[GCAP];
  __shared__ float gX[GCAP];
  __shared__ int gI[GCAP];
  __shared__ float sv[KF];
  __shared__ int si[KF];
  __shared__ uint32_t sel[4];
  __shared__ int n_gather, need_exact_sh, ambiguous_sh;

  const int row = blockIdx.x;
  const int tid = threadIdx.x, lane = lane_id(), wid = tid / WAVE;
  const int V = a.vocab, k = a.k;
  const RowP rp = row_params(a, row);
  const float T = rp.T;

  /* ---- the row, in 16-byte chunks from the aligned address below its start */
  const char *rowp = (const char *)a.logits + (size_t)row * (size_t)a.row_stride * ES;
  const uintptr_t a0 = (uintptr_t)rowp & ~(uintptr_t)15;
  const int off = (int)(((uintptr_t)rowp - a0) / ES);
  const int nchunks = (off + V + EPC - 1) / EPC;
  float L[NV];
#pragma unroll
  for (int j = 0; j < CPT; j++) {
    const int c = j * BLOCK + tid;
    uint4 q = make_uint4(0u, 0u, 0u, 0u);
    if (c < nchunks) q = *(const uint4 *)(a0 + (size_t)c * 16);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int e = 0; e < EPC; e++) {
      if (BF16)
        L[j * EPC + e] = d3s_u2f((e & 1) ? (w[e / 2] & 0xffff0000u) : (w[e / 2] << 16));
      else
        L[j * EPC + e] = d3s_u2f(w[e]);
    }
  }
  auto pos = [&](int j, int e) { return (j * BLOCK + tid) * EPC + e - off; };
  auto valid = [&](int j, int e) { return (unsigned)pos(j, e) < (unsigned)V; };
  if (rp.banned >= 0 && rp.banned < V) {
#pragma unroll
    for (int j = 0; j < CPT; j++)
#pragma unroll
      for (int e = 0; e < EPC; e++)
        if (pos(j, e) == rp.banned) L[j * EPC + e] = -__builtin_inff();
  }

  /* ---- row max and input classification */
  float lmax = -__builtin_inff();
  uint32_t fl = 0;
#pragma unroll
  for (int j = 0; j < CPT; j++)
#pragma unroll
    for (int e = 0; e < EPC; e++)
      if (valid(j, e)) {
        const float v = L[j * EPC + e];
        const uint32_t c = classify(v);
        fl |= c;
        if (!(c & 1u)) lmax = fmaxf(lmax, v);
      }
  for (int i = tid; i < NB; i += BLOCK) hist[i] = 0u;
  if (tid == 0) {
    n_gather = 0;
    need_exact_sh = 0;
    ambiguous_sh = 0;
  }
  lmax = wave_max_f(lmax);
  fl = (__ballot(fl & 1u) ? 1u : 0u) | (__ballot(fl & 2u) ? 2u : 0u);
  if (lane == 0) {
    sh_max[wid] = lmax;
    sh_flag[wid] = fl;
  }
  __syncthreads();
  float M = sh_max[0];
  uint32_t F = sh_flag[0];
#pragma unroll
  for (int w = 1; w < NW; w++) {
    M = fmaxf(M, sh_max[w]);
    F |= sh_flag[w];
  }
  const float xmax = M / T; /* = max x: correctly rounded division is monotone */
  if ((F & 1u) || d3s_isnan(xmax) || xmax == __builtin_inff() ||
      (T == __builtin_inff() && (F & 2u))) {
    write_special(a, row, false);
    return;
  }
  if (M == -__builtin_inff()) {
    write_special(a, row, true);
    return;
  }

  /* ---- fast sum of exp and the distance histogram, one pass over registers */
  const float c2 = LOG2E / T;
  const float hs = BINS_PER_NAT / T;
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < CPT; j++)
#pragma unroll
    for (int e = 0; e < EPC; e++)
      if (valid(j, e)) {
        const float d = M - L[j * EPC + e];
        s = s + __builtin_amdgcn_exp2f(-d * c2);
        const float b = d * hs;
        if (b < (float)NB) atomicAdd(&hist[(int)b], 1u);
      }
  s = wave_sum_f(s);
  if (lane == 0) sh_sum[wid] = s;
  __syncthreads();
  float S_f = 0.0f;
#pragma unroll
  for (int w = 0; w < NW; w++) S_f = S_f + sh_sum[w];
  if (wid == 0) {
    const BinSel b = wave_find_bin<true>(hist, (uint32_t)k);
    if (lane == 0) {
      sel[0] = b.bin;
      sel[1] = b.above;
      sel[2] = b.count;
      if (!b.ok) need_exact_sh = 1;
    }
  }
  __syncthreads();
  bool need_exact = need_exact_sh || (a.flags & FLAG_EXACT_SELECT);
  if (!need_exact && sel[1] + sel[2] > (uint32_t)GCAP) need_exact = true;

  /* ---- candidates: every element in a bin up to the k-th element's bin */
  if (!need_exact) {
    const int bstar = (int)sel[0];
    float lout = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < CPT; j++)
#pragma unroll
      for (int e = 0; e < EPC; e++)
        if (valid(j, e)) {
          const float v = L[j * EPC + e];
          const float b = (M - v) * hs;
          if (b < (float)NB && (int)b <= bstar) {
            const int slot = atomicAdd(&n_gather, 1);
            if (slot < GCAP) {
              gX[slot] = v; /* the logit for now; x below */
              gI[slot] = pos(j, e);
            }
          } else {
            lout = fmaxf(lout, v);
          }
        }
    lout = wave_max_f(lout);
    if (lane == 0) sh_out[wid] = lout;
    __syncthreads();
    const int G = min(n_gather, GCAP);
    float Lo = sh_out[0];
#pragma unroll
    for (int w = 1; w < NW; w++) Lo = fmaxf(Lo, sh_out[w]);
    if (tid < G) {
      const float x = gX[tid] / T;
      gX[tid] = x;
      gK[tid] = composite_key(x, gI[tid]);
    }
    __syncthreads();
    if (tid < G) {
      const uint64_t my = gK[tid];
      int rank = 0;
      for (int j = 0; j < G; j++) rank += gK[j] > my;
      if (rank < k) {
        sv[rank] = gX[tid];
        si[rank] = gI[tid];
      }
    }
    __syncthreads();
    /* an element left out must rank below the k-th: it has a smaller logit, so
     * its x is <= x_k; equality (a tie made by the division) is settled exactly */
    if (Lo / T == sv[k - 1]) need_exact = true;
  }

  /* ---- exact radix select over order-preserving keys of x */
  if (need_exact) {
    if (tid == 0 && a.counters) atomicAdd(&a.counters[CNT_EXACT_SELECT], 1u);
#pragma unroll
    for (int i = 0; i < NV; i++) L[i] = L[i] / T; /* L now holds x */
    uint32_t prefix = 0u, pmask = 0u, need = (uint32_t)k, done = 0u;
    for (int pass = 0; pass < 4 && !done; pass++) {
      const int shift = 24 - 8 * pass;
      __syncthreads();
      for (int i = tid; i < NB; i += BLOCK) hist[i] = 0u;
      __syncthreads();
#pragma unroll
      for (int j = 0; j < CPT; j++)
#pragma unroll
        for (int e = 0; e < EPC; e++)
          if (valid(j, e)) {
            const uint32_t key = d3s_ordkey(L[j * EPC + e]);
            if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
          }
      __syncthreads();
      if (wid == 0) {
        const BinSel b = wave_find_bin<false>(hist, need); /* always holds >= need */
        if (lane == 0) {
          sel[0] = prefix | (b.bin << shift);
          sel[1] = pmask | (0xffu << shift);
          sel[2] = need - b.above;
          sel[3] = (b.count == need - b.above) ? 1u : 0u;
        }
      }
      __syncthreads();
      prefix = sel[0];
      pmask = sel[1];
      need = sel[2];
      done = sel[3];
    }
    /* gather: everything above the group, then the group (all of it when it
     * holds exactly `need`, else its lowest-index `need`: exact ties) */
    if (tid == 0) n_gather = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < CPT; j++)
#pragma unroll
      for (int e = 0; e < EPC; e++)
        if (valid(j, e)) {
          const uint32_t key = d3s_ordkey(L[j * EPC + e]) & pmask;
          if (key > prefix || (done && key == prefix)) {
            const int slot = atomicAdd(&n_gather, 1);
            if (slot < GCAP) {
              gX[slot] = L[j * EPC + e];
              gI[slot] = pos(j, e);
            }
          }
        }
    if (!done) {
      /* index order is (j, tid, e): one block scan per chunk row j */
      uint32_t base = 0u;
      for (int j = 0; j < CPT; j++) {
        uint32_t cnt = 0u;
#pragma unroll
        for (int e = 0; e < EPC; e++)
          if (valid(j, e) && d3s_ordkey(L[j * EPC + e]) == prefix) cnt++;
        const uint32_t incl = wave_incl_scan_u32(cnt);
        if (lane == WAVE - 1) sh_scan[wid] = incl;
        __syncthreads();
        uint32_t wbase = 0u, tot = 0u;
        for (int w = 0; w < NW; w++) {
          const uint32_t t = sh_scan[w];
          if (w < wid) wbase += t;
          tot += t;
        }
        uint32_t ord = base + wbase + incl - cnt;
#pragma unroll
        for (int e = 0; e < EPC; e++)
          if (valid(j, e) && d3s_ordkey(L[j * EPC + e]) == prefix) {
            if (ord < need) {
              const int slot = atomicAdd(&n_gather, 1);
              if (slot < GCAP) {
                gX[slot] = L[j * EPC + e];
                gI[slot] = pos(j, e);
              }
            }
            ord++;
          }
        base += tot;
        __syncthreads();
        if (base >= need) break;
      }
    }
    __syncthreads();
    const int G = min(n_gather, GCAP); /* == k */
    if (tid < G) gK[tid] = composite_key(gX[tid], gI[tid]);
    __syncthreads();
    if (tid < G) {
      const uint64_t my = gK[tid];
      int rank = 0;
      for (int j = 0; j < G; j++) rank += gK[j] > my;
      if (rank < k) {
        sv[rank] = gX[tid];
        si[rank] = gI[tid];
      }
    }
    __syncthreads();
  }

  /* ---- log-sum-exp and the top-p cut */
  const bool have_x = need_exact;
  auto exact_lse = [&]() -> float {
    /* exact fixed-point sum of exp(x_i - m): independent of the order */
    uint64_t acc = 0;
#pragma unroll
    for (int j = 0; j < CPT; j++)
#pragma unroll
      for (int e = 0; e < EPC; e++)
        if (valid(j, e)) {
          const float x = have_x ? L[j * EPC + e] : L[j * EPC + e] / T;
          acc += d3s_fix40(d3s_expf(x - xmax));
        }
    acc = wave_sum_u64(acc);
    if (lane == 0) sh_q[wid] = acc;
    __syncthreads();
    uint64_t S = 0;
#pragma unroll
    for (int w = 0; w < NW; w++) S += sh_q[w];
    if (tid == 0 && a.counters) atomicAdd(&a.counters[CNT_EXACT_LSE], 1u);
    return xmax + d3s_logf(d3s_fixsum_to_f32(S));
  };

  const float v = (wid == 0 && lane < k) ? sv[lane] : 0.0f;
  const int idx = (wid == 0 && lane < k) ? si[lane] : 0;
  const float top_p = rp.top_p;
  if (need_exact || (a.flags & FLAG_EXACT_LSE)) {
    const float lse = exact_lse();
    if (wid == 0) {
      const float c = wave_seq_cumsum(lane < k ? d3s_expf(v - lse) : 0.0f, k);
      wave_tail_finish(a, row, v, idx, c, top_p);
    }
    return;
  }
  float c = 0.0f;
  if (wid == 0) {
    const float lse_f = xmax + d3s_logf(S_f);
    c = wave_seq_cumsum(lane < k ? d3s_expf(v - lse_f) : 0.0f, k);
    /* |lse_f - lse| is below 4*2^-23*(|m|+64) + 1e-5 (input rounding of x,
     * hardware exp2, fp32 summation); a c_r moves by at most that plus 1.2e-5
     * of exp / addition rounding.  Twice that bound is the margin. */
    const float eps = 8.0f * 0x1.0p-23f * (fabsf(xmax) + 64.0f) + 5e-5f;
    const bool amb = lane >= 1 && lane < k && fabsf(c - top_p) <= eps;
    const bool any_amb = __ballot(amb) != 0ull;
    if (lane == 0 && any_amb) ambiguous_sh = 1;
  }
  __syncthreads();
  if (ambiguous_sh) {
    const float lse = exact_lse();
    if (wid == 0) c = wave_seq_cumsum(lane < k ? d3s_expf(v - lse) : 0.0f, k);
  }
  if (wid == 0) wave_tail_finish(a, row, v, idx, c, top_p);
}

/* ------------------------------------------------------------------------ */
/* generic kernel                                                            */
/* ------------------------------------------------------------------------ */

constexpr int GBLOCK = 1024;
constexpr int GNW = GBLOCK / WAVE;

template <bool BF16>
__device__ __forceinline__ float load_logit(const void *rowp, int i, int banned) {
  float v;
  if (BF16)
    v = d3s_bf16_to_f32(((const uint16_t *)rowp)[i]);
  else
    v = ((const float *)rowp)[i];
  return i == banned ? -__builtin_inff() : v;
}

/* exclusive block scan in thread order; `tot` receives the block total */
template <typename U>
__device__ __forceinline__ U block_excl_scan(U v, U *sh, U &tot) {
  const int lane = lane_id(), wid = threadIdx.x / WAVE;
  U incl;
  if constexpr (sizeof(U) == 8)
    incl = wave_incl_scan_u64(v);
  else
    incl = wave_incl_scan_u32(v);
  if (lane == WAVE - 1) sh[wid] = incl;
  __syncthreads();
  U wbase = 0, t = 0;
  for (int w = 0; w < GNW; w++) {
    const U x = sh[w];
    if (w < wid) wbase += x;
    t += x;
  }
  __syncthreads();
  tot = t;
  return wbase + incl - v;
}

template <bool BF16>
__global__ __launch_bounds__(GBLOCK) void k_generic(SampleArgs a, int kpow) {
  extern __shared__ uint64_t glist[]; /* [kpow] composite keys, sorted in place */
  __shared__ uint32_t hist[NB];
  __shared__ float sh_max[GNW];
  __shared__ uint32_t sh_flag[GNW], sh_u32[GNW];
  __shared__ uint64_t sh_q[GNW];
  __shared__ uint32_t sel[4];
  __shared__ int n_gather;
  __shared__ float sh_best[GNW];
  __shared__ int sh_bestr[GNW];

  const int row = blockIdx.x;
  const int tid = threadIdx.x, lane = lane_id(), wid = tid / WAVE;
  const int V = a.vocab, k = a.k;
  const RowP rp = row_params(a, row);
  const float T = rp.T;
  const char *rowp = (const char *)a.logits + (size_t)row * (size_t)a.row_stride * (BF16 ? 2 : 4);

  /* ---- pass 1: max and classification */
  float lmax = -__builtin_inff();
  uint32_t fl = 0;
  for (int i = tid; i < V; i += GBLOCK) {
    const float v = load_logit<BF16>(rowp, i, rp.banned);
    const uint32_t c = classify(v);
    fl |= c;
    if (!(c & 1u)) lmax = fmaxf(lmax, v);
  }
  lmax = wave_max_f(lmax);
  fl = (__ballot(fl & 1u) ? 1u : 0u) | (__ballot(fl & 2u) ? 2u : 0u);
  if (lane == 0) {
    sh_max[wid] = lmax;
    sh_flag[wid] = fl;
  }
  __syncthreads();
  float M = sh_max[0];
  uint32_t F = sh_flag[0];
  for (int w = 1; w < GNW; w++) {
    M = fmaxf(M, sh_max[w]);
    F |= sh_flag[w];
  }
  const float xmax = M / T;
  if ((F & 1u) || d3s_isnan(xmax) || xmax == __builtin_inff() ||
      (T == __builtin_inff() && (F & 2u))) {
    write_special(a, row, false);
    return;
  }
  if (M == -__builtin_inff()) {
    write_special(a, row, true);
    return;
  }

  /* ---- pass 2: exact log-sum-exp */
  uint64_t acc = 0;
  for (int i = tid; i < V; i += GBLOCK)
    acc += d3s_fix40(d3s_expf(load_logit<BF16>(rowp, i, rp.banned) / T - xmax));
  acc = wave_sum_u64(acc);
  if (lane == 0) sh_q[wid] = acc;
  __syncthreads();
  uint64_t S = 0;
  for (int w = 0; w < GNW; w++) S += sh_q[w];
  const float lse = xmax + d3s_logf(d3s_fixsum_to_f32(S));

  /* ---- radix select of the k-th composite rank over keys of x */
  uint32_t prefix = 0u, pmask = 0u, need = (uint32_t)k, done = 0u;
  for (int pass = 0; pass < 4 && !done; pass++) {
    const int shift = 24 - 8 * pass;
    __syncthreads();
    for (int i = tid; i < NB; i += GBLOCK) hist[i] = 0u;
    __syncthreads();
    for (int i = tid; i < V; i += GBLOCK) {
      const uint32_t key = d3s_ordkey(load_logit<BF16>(rowp, i, rp.banned) / T);
      if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (wid == 0) {
      const BinSel b = wave_find_bin<false>(hist, need);
      if (lane == 0) {
        sel[0] = prefix | (b.bin << shift);
        sel[1] = pmask | (0xffu << shift);
        sel[2] = need - b.above;
        sel[3] = (b.count == need - b.above) ? 1u : 0u;
      }
    }
    __syncthreads();
    prefix = sel[0];
    pmask = sel[1];
    need = sel[2];
    done = sel[3];
  }
  if (tid == 0) n_gather = 0;
  __syncthreads();
  for (int i = tid; i < V; i += GBLOCK) {
    const float x = load_logit<BF16>(rowp, i, rp.banned) / T;
    const uint32_t key = d3s_ordkey(x) & pmask;
    if (key > prefix || (done && key == prefix)) {
      const int slot = atomicAdd(&n_gather, 1);
      if (slot < kpow) glist[slot] = composite_key(x, i);
    }
  }
  if (!done) {
    /* exact ties: the lowest-index `need`, one block-wide tile at a time */
    uint32_t base = 0u;
    for (int t0 = 0; t0 < V && base < need; t0 += GBLOCK) {
      const int i = t0 + tid;
      float x = 0.0f;
      uint32_t tie = 0u;
      if (i < V) {
        x = load_logit<BF16>(rowp, i, rp.banned) / T;
        tie = d3s_ordkey(x) == prefix;
      }
      uint32_t tot;
      const uint32_t ord = base + block_excl_scan<uint32_t>(tie, sh_u32, tot);
      if (tie && ord < need) {
        const int slot = atomicAdd(&n_gather, 1);
        if (slot < kpow) glist[slot] = composite_key(x, i);
      }
      base += tot;
    }
  }
  __syncthreads();
  for (int i = k + tid; i < kpow; i += GBLOCK) glist[i] = 0ull; /* sorts last */
  __syncthreads();
  /* ---- bitonic sort, descending */
  for (int size = 2; size <= kpow; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = tid; i < kpow / 2; i += GBLOCK) {
        const int lo = 2 * i - (i & (stride - 1));
        const int hi = lo + stride;
        const uint64_t A = glist[lo], B = glist[hi];
        const bool desc = (lo & size) == 0;
        if (desc ? (A < B) : (A > B)) {
          glist[lo] = B;
          glist[hi] = A;
        }
      }
      __syncthreads();
    }
  }

  const float top_p = rp.top_p;
  if (k <= KF) {
    if (wid == 0) {
      const uint64_t key = lane < k ? glist[lane] : 0ull;
      const float v = key_x(key);
      const int idx = key_idx(key);
      const float c = wave_seq_cumsum(lane < k ? d3s_expf(v - lse) : 0.0f, k);
      wave_tail_finish(a, row, v, idx, c, top_p);
    }
    return;
  }

  /* ---- k > 64: exact prefix sums over ranks (the op graph's cumsum and
   * softmax, src/sampling.c:39-44), each thread owning R consecutive ranks */
  const int R = (k + GBLOCK - 1) / GBLOCK;
  const int r0 = tid * R;
  const float v0 = key_x(glist[0]);
  uint64_t loc = 0;
  for (int q = 0; q < R; q++) {
    const int r = r0 + q;
    if (r < k) loc += d3s_fix40(d3s_expf(key_x(glist[r]) - lse));
  }
  uint64_t tot;
  uint64_t P = block_excl_scan<uint64_t>(loc, sh_q, tot);
  int cut_local = k;
  for (int q = 0; q < R; q++) {
    const int r = r0 + q;
    if (r < k) {
      P += d3s_fix40(d3s_expf(key_x(glist[r]) - lse));
      if (r > 0 && cut_local == k && d3s_fixsum_to_f32(P) > top_p) cut_local = r;
    }
  }
  /* min over the block */
  int cm = cut_local;
#pragma unroll
  for (int o = WAVE / 2; o > 0; o >>= 1) cm = min(cm, __shfl_xor(cm, o));
  if (lane == 0) sh_u32[wid] = (uint32_t)cm;
  __syncthreads();
  int cut = k;
  for (int w = 0; w < GNW; w++) cut = min(cut, (int)sh_u32[w]);
  uint64_t ks = 0;
  for (int q = 0; q < R; q++) {
    const int r = r0 + q;
    if (r < k && r < cut) ks += d3s_fix40(d3s_expf(key_x(glist[r]) - v0));
  }
  ks = wave_sum_u64(ks);
  __syncthreads();
  if (lane == 0) sh_q[wid] = ks;
  __syncthreads();
  uint64_t KS = 0;
  for (int w = 0; w < GNW; w++) KS += sh_q[w];
  const float inv = 1.0f / d3s_fixsum_to_f32(KS);
  float bs = -1.0f;
  int br = 0x7fffffff;
  for (int q = 0; q < R; q++) {
    const int r = r0 + q;
    if (r < k) {
      const uint64_t key = glist[r];
      const float p = r < cut ? d3s_expf(key_x(key) - v0) * inv : 0.0f;
      const float noise = -d3s_logf(1.0f - a.u[(size_t)row * k + r]);
      const float score = p / noise;
      const float sc = score > -1.0f ? score : -1.0f;
      if (sc > bs || br == 0x7fffffff) { /* first maximum within the thread's ranks */
        bs = sc;
        br = r;
      }
      if (a.probs) a.probs[(size_t)row * k + r] = p;
      if (a.cand) a.cand[(size_t)row * k + r] = key_idx(key);
    }
  }
#pragma unroll
  for (int o = WAVE / 2; o > 0; o >>= 1) {
    const float os = __shfl_xor(bs, o);
    const int ob = __shfl_xor(br, o);
    if (os > bs || (os == bs && ob < br)) {
      bs = os;
      br = ob;
    }
  }
  if (lane == 0) {
    sh_best[wid] = bs;
    sh_bestr[wid] = br;
  }
  __syncthreads();
  if (tid == 0) {
    float b = sh_best[0];
    int r = sh_bestr[0];
    for (int w = 1; w < GNW; w++)
      if (sh_best[w] > b || (sh_best[w] == b && sh_bestr[w] < r)) {
        b = sh_best[w];
        r = sh_bestr[w];
      }
    a.ids[row] = key_idx(glist[r]);
  }
}

__global__ void k_uniform(float *u, int64_t n, uint64_t seed, uint64_t stream_id) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) u[i] = d3s_uniform(seed, stream_id, (uint64_t)i);
}

__global__ void k_math(const float *in, float *oe, float *ol, float *od, uint64_t *of, int64_t n,
                       float divisor) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    const float x = in[i];
    oe[i] = d3s_expf(x);
    ol[i] = d3s_logf(x);
    od[i] = x / divisor;
    of[i] = d3s_fix40(x);
  }
}

template <int BLOCK, int CPT, bool BF16>
constexpr int fused_vmax() {
  return BLOCK * CPT * (16 / (BF16 ? 2 : 4)) - (16 / (BF16 ? 2 : 4) - 1);
}

template <int BLOCK, int CPT, bool BF16>
bool try_fused(const SampleArgs &a, hipStream_t s) {
  if (a.vocab > fused_vmax<BLOCK, CPT, BF16>()) return false;
  hipLaunchKernelGGL((k_fused<BLOCK, CPT, BF16>), dim3(a.n_rows), dim3(BLOCK), 0, s, a);
  return true;
}

}  // namespace

int fused_max_vocab(Dtype dt) {
  return dt == DT_F32 ? fused_vmax<1024, 4, false>() : fused_vmax<1024, 4, true>();
}

bool launch_fused(const SampleArgs &a, Dtype dt, hipStream_t s) {
  if (a.k > KF) return false;
  const bool wide = a.n_rows < 64; /* few rows: more waves per row for latency */
  if (dt == DT_F32) {
    if (!wide && try_fused<256, 5, false>(a, s)) return true;
    return try_fused<1024, 2, false>(a, s) || try_fused<1024, 4, false>(a, s);
  }
  if (!wide && try_fused<256, 3, true>(a, s)) return true;
  return try_fused<1024, 1, true>(a, s) || try_fused<1024, 2, true>(a, s) ||
         try_fused<1024, 4, true>(a, s);
}

int generic_max_k() { return 16384; }

bool launch_generic(const SampleArgs &a, Dtype dt, hipStream_t s) {
  if (a.k > generic_max_k()) return false;
  int kpow = 2;
  while (kpow < a.k) kpow <<= 1;
  const size_t lds = (size_t)kpow * sizeof(uint64_t);
  /* dynamic LDS beyond 64 KB must be allowed once per kernel (gfx950: 160 KB) */
  static std::once_flag once;
  std::call_once(once, [] {
    const int most = (int)(generic_max_k() * sizeof(uint64_t));
    (void)hipFuncSetAttribute((const void *)k_generic<false>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, most);
    (void)hipFuncSetAttribute((const void *)k_generic<true>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, most);
  });
  if (dt == DT_F32)
    hipLaunchKernelGGL(k_generic<false>, dim3(a.n_rows), dim3(GBLOCK), lds, s, a, kpow);
  else
    hipLaunchKernelGGL(k_generic<true>, dim3(a.n_rows), dim3(GBLOCK), lds, s, a, kpow);
  return true;
}

void launch_uniform(float *u, int64_t n, uint64_t seed, uint64_t stream_id, hipStream_t s) {
  if (n <= 0) return;
  const int B = 256;
  hipLaunchKernelGGL(k_uniform, dim3((unsigned)((n + B - 1) / B)), dim3(B), 0, s, u, n, seed,
                     stream_id);
}

void launch_math_selftest(const float *in, float *out_exp, float *out_log, float *out_div,
                          uint64_t *out_fix, int64_t n, float divisor, hipStream_t s) {
  if (n <= 0) return;
  const int B = 256;
  hipLaunchKernelGGL(k_math, dim3((unsigned)((n + B - 1) / B)), dim3(B), 0, s, in, out_exp,
                     out_log, out_div, out_fix, n, divisor);
}

}  // namespace d3s
