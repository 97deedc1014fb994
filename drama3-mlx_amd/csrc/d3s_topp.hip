/* The ranked-nucleus kernel of the MI355X token sampler (gfx950, wave64):
 * k_topp, for k > 64 (the reference's op-graph case, src/sampling.c:22-49,
 * with k up to V: "top-k disabled") on rows of at most 1024 * EPT elements.
 *
 * One workgroup per row (512 threads for rows up to 4608 elements, 1024
 * above), EPT elements per thread in registers (element j * TBLOCK + t of
 * thread t).  Every element needs its exact rank:
 * the race draws u[rank] for every kept rank (src/sampling.c:45-47).
 *
 *  1. x = L / T exactly, classification, max m and the smallest finite x.
 *  2. The exact row sum: 2^-40 fixed-point images of d3s_expf(x - m)
 *     (lse = m + log S, src/sampling.c:37-38).
 *  3. Ranks by (x desc, index asc) (:27-36): a counting sort over 4096 or
 *     8192 buckets of m - x, scaled to the row's range (a non-decreasing
 *     function of -x, so buckets are ordered), then each element counts the larger
 *     keys of its own bucket.  The keys end in LDS in rank order, and from
 *     here on each thread owns consecutive ranks.
 *  4. The cut: exact fixed-point prefix sums of d3s_expf(x_r - lse) over
 *     ranks (the op graph's cumsum, :39-42, rounded once), first r > 0 whose
 *     prefix exceeds top_p.
 *  5. Only the kept ranks (x_0 = m): the exact sum of e_r = d3s_expf(x_r -
 *     m), the probabilities e_r * inv and the race p / -log(1 - u[rank]),
 *     first maximum (:43-48).  Dropped ranks race only when no kept score
 *     is positive.
 * The definition is the generic kernel's for k > 64, bit for bit.  A row
 * whose x fall in few buckets (heavy ties) is still exact, only slower. */
#include "d3s_generic.h"

#pragma clang fp contract(off)

namespace d3s {
namespace {

/* workgroups of 512 or 1024 threads; the reductions' LDS rows hold one
 * entry per wave, 16 at most */
constexpr int TNW = 16;
/* buckets of finite x (bucket NBK holds -inf): 8192 for 1024-thread rows of
 * up to 5120 elements, whose LDS (keys and bucket bounds) then still fits
 * twice per CU; 4096 otherwise (512-thread rows of up to 4608 elements fit
 * three times) */
constexpr int topp_buckets(int max_v, int tb) { return max_v <= 5120 && tb == 1024 ? 8192 : 4096; }
/* waves per SIMD that the LDS allows, which sets the register budget:
 * three 512-thread rows of up to 4608 elements per CU (6), two 1024-thread
 * rows of up to 5120 (8), one of up to 8192 (4) */
constexpr int topp_waves(int ept, int tb) { return tb == 512 ? 6 : (ept * tb <= 5120 ? 8 : 4); }

/* Workgroup reductions.  Each wave reduces on DPP and files its value in
 * LDS; after the barrier every lane reads entry lane % 16 and the sixteen
 * entries combine by a butterfly inside each DPP row of 16 lanes (quad_perm
 * 1,0,3,2; quad_perm 2,3,0,1; row_half_mirror; row_mirror), so every lane
 * holds the result.  Each call opens with a barrier: the previous call's
 * entries may still be being read. */
static_assert(TNW == 16, "one LDS entry per lane of a DPP row");
/* (a workgroup of fewer than 16 waves fills the other entries with each
 * reduction's identity once, at its start) */
constexpr int DPP_X1 = 0xb1, DPP_X2 = 0x4e, DPP_HMIR = 0x141, DPP_MIR = 0x140;

struct TRed {
  float f[TNW], g[TNW], h[TNW];
  uint64_t s[TNW];
  uint64_t kept; /* the kept ranks' fixed-point sum */
  uint64_t row_q[3]; /* the ids path's Tq and cut bands (wave 0's) */
  float row_lse;
  uint32_t a[TNW];
  int r[TNW];
};

template <int C>
__device__ __forceinline__ float xch_f(float v) {
  return dpp_f<C, 0xf>(v, v);
}
template <int C>
__device__ __forceinline__ uint32_t xch_u(uint32_t v) {
  return dpp_u<C, 0xf>(v, v);
}
template <int C>
__device__ __forceinline__ uint64_t xch_u64(uint64_t v) {
  return ((uint64_t)xch_u<C>((uint32_t)(v >> 32)) << 32) | xch_u<C>((uint32_t)v);
}

/* (never NaN, as in wave_max_f) */
__device__ __forceinline__ float row16_max_f(float v) {
  v = __builtin_elementwise_maximum(v, xch_f<DPP_X1>(v));
  v = __builtin_elementwise_maximum(v, xch_f<DPP_X2>(v));
  v = __builtin_elementwise_maximum(v, xch_f<DPP_HMIR>(v));
  return __builtin_elementwise_maximum(v, xch_f<DPP_MIR>(v));
}
__device__ __forceinline__ int row16_min_i32(int v) {
  v = min(v, (int)xch_u<DPP_X1>((uint32_t)v));
  v = min(v, (int)xch_u<DPP_X2>((uint32_t)v));
  v = min(v, (int)xch_u<DPP_HMIR>((uint32_t)v));
  return min(v, (int)xch_u<DPP_MIR>((uint32_t)v));
}
__device__ __forceinline__ uint32_t row16_sum_u32(uint32_t v) {
  v += xch_u<DPP_X1>(v);
  v += xch_u<DPP_X2>(v);
  v += xch_u<DPP_HMIR>(v);
  return v + xch_u<DPP_MIR>(v);
}
__device__ __forceinline__ uint64_t row16_sum_u64(uint64_t v) {
  v += xch_u64<DPP_X1>(v);
  v += xch_u64<DPP_X2>(v);
  v += xch_u64<DPP_HMIR>(v);
  return v + xch_u64<DPP_MIR>(v);
}

/* A workgroup reduction leaves the same value in every lane: taken from the
 * first lane it is known to be wave-uniform, so the arithmetic that follows
 * on it (the same in every wave) runs on the scalar unit where it can. */
__device__ __forceinline__ float uni_f(float v) {
  return d3s_u2f((uint32_t)__builtin_amdgcn_readfirstlane((int)d3s_f2u(v)));
}
__device__ __forceinline__ uint32_t uni_u32(uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); }
__device__ __forceinline__ uint64_t uni_u64(uint64_t v) {
  return ((uint64_t)uni_u32((uint32_t)(v >> 32)) << 32) | uni_u32((uint32_t)v);
}

__device__ __forceinline__ float block_max_f(float v, TRed &R) {
  v = wave_max_f(v);
  const int wid = threadIdx.x / WAVE;
  __syncthreads();
  if (lane_id() == 0) R.f[wid] = v;
  __syncthreads();
  return uni_f(row16_max_f(R.f[lane_id() & 15]));
}

/* the maxima of two values in one round (IEEE maximum at every step: a NaN
 * in any lane gives NaN, +inf is kept) */
__device__ __forceinline__ void block_max2_f(float &u, float &v, TRed &R) {
  u = wave_max_f(u);
  v = wave_max_f(v);
  const int wid = threadIdx.x / WAVE, l16 = lane_id() & 15;
  __syncthreads();
  if (lane_id() == 0) {
    R.f[wid] = u;
    R.g[wid] = v;
  }
  __syncthreads();
  u = uni_f(row16_max_f(R.f[l16]));
  v = uni_f(row16_max_f(R.g[l16]));
}

__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, TRed &R) {
  const uint64_t w = wave_sum_u64(v);
  const int wid = threadIdx.x / WAVE;
  __syncthreads();
  if (lane_id() == 0) R.s[wid] = w;
  __syncthreads();
  return uni_u64(row16_sum_u64(R.s[lane_id() & 15]));
}

__device__ __forceinline__ int block_min_i32(int v, TRed &R) {
  v = wave_min_i32(v);
  const int wid = threadIdx.x / WAVE;
  __syncthreads();
  if (lane_id() == 0) R.r[wid] = v;
  __syncthreads();
  return (int)uni_u32((uint32_t)row16_min_i32(R.r[lane_id() & 15]));
}

/* exclusive scan of per-thread counts in thread order; `tot` = the total */
__device__ __forceinline__ uint32_t block_excl_scan_u32(uint32_t v, TRed &R, uint32_t &tot) {
  const int lane = lane_id(), wid = threadIdx.x / WAVE;
  const uint32_t incl = wave_scan_add_u32(v);
  __syncthreads();
  if (lane == WAVE - 1) R.a[wid] = incl;
  __syncthreads();
  const uint32_t x = R.a[lane & 15];
  tot = uni_u32(row16_sum_u32(x));
  return row16_sum_u32((lane & 15) < wid ? x : 0u) + incl - v;
}

/* the same for per-thread fixed-point sums below 2^45 (the wave scan in
 * 24-bit parts) */
__device__ __forceinline__ uint64_t block_excl_scan_u64(uint64_t v, TRed &R) {
  const int lane = lane_id(), wid = threadIdx.x / WAVE;
  const uint32_t lo = wave_scan_add_u32((uint32_t)(v & 0xffffffu));
  const uint32_t hi = wave_scan_add_u32((uint32_t)(v >> 24));
  const uint64_t incl = ((uint64_t)hi << 24) + lo;
  __syncthreads();
  if (lane == WAVE - 1) R.s[wid] = incl;
  __syncthreads();
  const uint64_t x = R.s[lane & 15];
  return row16_sum_u64((lane & 15) < wid ? x : 0ull) + incl - v;
}

/* the race's score of one rank, clamped: NaN, -inf and scores <= -1 never
 * beat the initial -1 (src/sampling.c:45-48) */
__device__ __forceinline__ float topp_score(float p, float u) {
  const float score = p / -d3s_logf(1.0f - u);
  return score > -1.0f ? score : -1.0f;
}

/* the first maximum over the workgroup: the greatest score, ties to the
 * lower rank; every thread gets it */
__device__ __forceinline__ void block_argmax(float &s, int &r, TRed &R) {
  wave_argmax(s, r);
  const int wid = threadIdx.x / WAVE, l16 = lane_id() & 15;
  __syncthreads();
  if (lane_id() == 0) {
    R.f[wid] = s;
    R.r[wid] = r;
  }
  __syncthreads();
  s = R.f[l16];
  r = R.r[l16];
#define D3S_ROW16_ARGMAX_STEP(C)                          \
  {                                                       \
    const float os = xch_f<C>(s);                         \
    const int orr = (int)xch_u<C>((uint32_t)r);           \
    if (os > s || (os == s && orr < r)) {                 \
      s = os;                                             \
      r = orr;                                            \
    }                                                     \
  }
  D3S_ROW16_ARGMAX_STEP(DPP_X1)
  D3S_ROW16_ARGMAX_STEP(DPP_X2)
  D3S_ROW16_ARGMAX_STEP(DPP_HMIR)
  D3S_ROW16_ARGMAX_STEP(DPP_MIR)
#undef D3S_ROW16_ARGMAX_STEP
  s = uni_f(s);
  r = (int)uni_u32((uint32_t)r);
}

/* The cut's certain bands (phase 4 below): ranks whose prefix Q_r of the terms
 * fix40(e_r) reaches tdrop certainly drop, those below tkeep certainly stay.
 * With G = exp(m - lse) and G' = 2^40 / S, |P_r - Q_r G'| <= eps' (Q_r + k) G'
 * + k, P_r the exact prefix of the terms fix40(expf(x_r - lse)).  eps' is each
 * term's relative error, its two argument roundings (2^-24 z on either side,
 * z = lse - x_r <= min(lse - xmin, 30): terms with larger z are below one unit
 * on both sides) and two expf ulps, plus G's against G' (the roundings of
 * S 2^-40, of m + log S, and the log's ulp).  Tq: the smallest prefix that
 * passes top_p; 0 < Tq <= k 2^41. */
struct CutBands {
  uint64_t tdrop, tkeep;
};
__device__ __forceinline__ CutBands topp_cut_bands(uint64_t Tq, uint64_t S, float lse, float lnS, float xmin, int k) {
  /* in fp32: S' = RN(S 2^-40) = 1 / G' within 2^-24; every product and
   * conversion below is within a relative 2^-23, inside the extra 2^-20 */
  const float Sf = d3s_fixsum_to_f32(S);
  const float zf = lse - xmin;
  const float z = zf < 30.0f ? zf : 30.0f; /* NaN and inf too */
  const float et = 0x1p-24f * 1.01f * 2.0f * z + 0x1p-22f;
  const float ulp_ln = lnS > 0x1p-126f ? ldexpf(1.0f, ilogbf(lnS) - 23) : 0x1p-126f;
  const float eg = 0x1p-24f * 1.01f * (fabsf(lse) + 1.0f) + 1.01f * ulp_ln;
  const float ep = (et * 1.0001f + 1.01f * eg) * (1.0f + 1.01f * eg);
  const float slack = ep * (float)k / Sf + (float)k;
  const float Tqf = (float)Tq;
  /* 1 / (1 - ep) <= 1 + 1.13 ep and 1 / (1 + ep) >= 1 - ep for ep < 1/16 */
  const float dd = (Tqf + slack) * Sf * (1.0f + 1.13f * ep + 0x1p-20f);
  const float dk = (Tqf - slack) * Sf * (1.0f - ep - 0x1p-20f);
  /* (an lse so large that the band is wide leaves every rank to the exact
   * prefixes: no rank certainly drops, none certainly stays) */
  const bool wide = !(ep < 0x1p-4f);
  CutBands c;
  c.tdrop = wide || !(dd < 0x1p62f) ? ~0ull : (uint64_t)dd + 2ull;
  c.tkeep = wide || !(dk > 2.0f) ? 0ull : (dk < 0x1p62f ? (uint64_t)dk - 1ull : (1ull << 62));
  return c;
}

/* ---- The ids-only path (k_topp_ids: no probabilities or candidates asked
 * for, k = V).  The race reads every kept rank's uniform u[r], but a rank's
 * bucket bounds its probability (the bucket bounds m - x), and only the few
 * ranks whose score's upper bound reaches the largest lower bound need their
 * element.  So no element is ranked but those of the group of buckets that
 * holds the cut and those of the buckets such ranks fall in:
 *  2'. with the row sum, each element's bucket count and its group's sum of
 *      fix40(e) (a group: the PER buckets one thread scans); one scan gives
 *      each bucket's first rank and each group's prefix Q at its start.
 *  4'. the first group whose end reaches the certain drop band (phase 4's
 *      bands) holds the first certain drop, so the cut lies in [klo, khi]:
 *      the ranks before the group are kept, those after it dropped.
 *  5'. scores are bounded in units of inv = 1 / (kept sum), which cancels
 *      from every comparison: per rank, e <= 1 for the ranks that may be kept
 *      and e >= emin (a bucket bound) for those certainly kept give the first
 *      bounds and their largest lower bound LB1; the ranks whose upper bound
 *      reaches LB1 (a handful) take their bucket's bounds on e (bucket found
 *      by binary search over the starts), whose largest lower bound LB2 picks
 *      the candidates.  One gather brings one wave the cut group's elements
 *      and the candidates' buckets' elements; it ranks them, sums the cut
 *      group's prefixes (the cut, and the kept sum), and takes the candidates'
 *      exact scores: their first maximum is the row's (every rank whose exact
 *      score reaches it is a candidate).
 * A row takes the full path (phases 3-5) when its cut is within the bands'
 * uncertainty, when more elements than a wave holds would go to that wave, or
 * when no kept score is positive. */
constexpr int TOPP_FULL = -2;
constexpr int TOPP_RETRY = -3; /* the ids path's exact retry (internal) */
constexpr int TOPP_REDO_WG = 64; /* k_topp_redo's workgroups (at most) */
constexpr int TF_CAP = WAVE; /* the elements (and refined ranks) one wave takes */

/* byte offsets in the dynamic LDS region: the gathered elements' keys and
 * buckets; the refined ranks and their uniforms; counters; candidate bucket
 * and rank bitmaps (the group sums, one per thread and one past them for
 * the -inf bucket, are a static array of the kernels: their address folds
 * into the atomics' offsets) */
__host__ __device__ constexpr size_t tf_lkey(int) { return 0; }
__host__ __device__ constexpr size_t tf_lval(int tb) { return tf_lkey(tb) + 8 * TF_CAP; }
__host__ __device__ constexpr size_t tf_rr(int tb) { return tf_lval(tb) + 8 * TF_CAP; }
__host__ __device__ constexpr size_t tf_ru(int tb) { return tf_rr(tb) + 4 * TF_CAP; }
__host__ __device__ constexpr size_t tf_misc(int tb) { return tf_ru(tb) + 4 * TF_CAP; }
__host__ __device__ constexpr size_t tf_cbits(int tb) { return tf_misc(tb) + 64; }
__host__ __device__ constexpr size_t tf_rbits(int tb, int nbk) { return tf_cbits(tb) + 4 * (size_t)(nbk / 32 + 4); }
__host__ __device__ constexpr size_t tf_bytes(int tb, int nbk, int V) {
  return tf_rbits(tb, nbk) + 16 * (size_t)((V + 127) / 128);
}

/* uint64 -> fp32 within a relative 2^-22 (two conversions and a sum) */
__device__ __forceinline__ float u64_to_f32_near(uint64_t v) {
  return __builtin_fmaf((float)(uint32_t)(v >> 32), 0x1p32f, (float)(uint32_t)v);
}
/* floor(v) for 0 <= v < 2^56 (v's bits split exactly at 2^32) */
__device__ __forceinline__ uint64_t f32_to_u64_small(float v) {
  const uint32_t hi = (uint32_t)(v * 0x1p-32f);
  const uint32_t lo = (uint32_t)(v - (float)hi * 0x1p32f);
  return ((uint64_t)hi << 32) | lo;
}

/* topp_cut_bands with cheaper conversions: every conversion within 2^-22
 * (inside the extra 2^-20), the log's ulp rounded up to a power of two at
 * least 2^-126, and the band ends capped at 2^56 (wider bands: safe) */
__device__ __forceinline__ CutBands topp_cut_bands_lean(uint64_t Tq, uint64_t S, float lse, float lnS, float xmin,
                                                        int k) {
  const float Sf = u64_to_f32_near(S) * 0x1p-40f;
  const float zf = lse - xmin;
  const float z = zf < 30.0f ? zf : 30.0f;
  const float et = 0x1p-24f * 1.01f * 2.0f * z + 0x1p-22f;
  const float ulp_ln = lnS >= 0x1p-103f ? d3s_u2f((d3s_f2u(lnS) & 0x7f800000u) - (23u << 23)) : 0x1p-126f;
  const float eg = 0x1p-24f * 1.01f * (fabsf(lse) + 1.0f) + 1.01f * ulp_ln;
  const float ep = (et * 1.0001f + 1.01f * eg) * (1.0f + 1.01f * eg);
  const float slack = ep * (float)k / Sf + (float)k;
  const float Tqf = u64_to_f32_near(Tq);
  const float dd = (Tqf + slack) * Sf * (1.0f + 1.13f * ep + 0x1p-20f);
  const float dk = (Tqf - slack) * Sf * (1.0f - ep - 0x1p-20f);
  const bool wide = !(ep < 0x1p-4f);
  CutBands c;
  c.tdrop = wide || !(dd < 0x1p56f) ? ~0ull : f32_to_u64_small(dd) + 2ull;
  c.tkeep = wide || !(dk > 2.0f) ? 0ull : (dk < 0x1p56f ? f32_to_u64_small(dk) - 1ull : (1ull << 56));
  return c;
}

/* Bounds on e = expf(x - m) over bucket b's elements (b < NBK finite; the
 * -inf bucket's e is 0).  Elements of bucket b < NBK - 1 have t =
 * RN(RN(m - x) scale) in [b, b + 1), so x's distance d' = RN(m - x) lies in
 * [b (1 - 2^-24), (b + 1) (1 + 2^-24)] / scale (the last finite bucket: up to
 * dmax = RN(m - xmin)); z_lo and z_hi below lie outside that with the
 * roundings of rs = RN(1 / scale) and of the products.  e = expf(-d') is
 * within an ulp; the hardware 2^(-z log2 e) is within 2^-21 and the
 * exponent's rounding within 2^-16 for z <= 104 (beyond, e is 0 or
 * subnormal): all inside the 2^-12 margins; e_hi is at least 2^-126 (above
 * every subnormal), e_lo 0 far out. */
template <int NBK>
__device__ __forceinline__ void topp_ebounds(int b, float rs, float dmax, float &elo, float &ehi) {
  elo = 0.0f;
  ehi = 0.0f;
  if (b < NBK) {
    const float zlo = (float)b * rs * (1.0f - 0x1p-18f);
    const float zhi = (b < NBK - 1 ? (float)(b + 1) * rs : dmax) * (1.0f + 0x1p-18f);
    ehi = fmaxf(__builtin_amdgcn_exp2f(-zlo * 1.44269504f) * (1.0f + 0x1p-12f), 0x1p-126f);
    elo = zhi < 87.0f ? __builtin_amdgcn_exp2f(-zhi * 1.44269504f) * (1.0f - 0x1p-12f) : 0.0f;
  }
}

/* Score bounds in units of inv from bounds on e, as phase 5's for exact p:
 * p = RN(e inv) lies in [e_lo inv (1 - 2^-24), e_hi inv (1 + 2^-24)], inside
 * the extra 2^-20 margins.  lb: -1 when u gives no bound (every score is at
 * least -1); h: +inf likewise, 0 for u >= 1 (noise +inf or NaN: score 0 or
 * -1). */
__device__ __forceinline__ void topp_sbounds(float elo, float ehi, float uu, float &lb, float &h) {
  lb = -1.0f;
  h = __builtin_inff();
  if (uu >= 0x1p-24f && uu < 1.0f) {
    lb = elo * __builtin_amdgcn_rcpf(uu * __builtin_amdgcn_rcpf(1.0f - uu) + 0x1p-22f) * ((1.0f - 0x1p-18f) * (1.0f - 0x1p-20f));
    if (uu > 0x1p-24f) h = ehi * __builtin_amdgcn_rcpf(uu - 0x1p-24f) * ((1.0f + 0x1p-18f) * (1.0f + 0x1p-20f));
  } else if (uu >= 1.0f) {
    h = 0.0f;
  }
}

/* exclusive scans, in thread order, of a count and a fixed-point sum (below
 * 2^56 in total), and their totals, in one round */
__device__ __forceinline__ void block_excl_scan2(uint32_t c, uint64_t v, TRed &R, uint32_t &cx, uint32_t &ctot,
                                                 uint64_t &vx, uint64_t &vtot) {
  const int lane = lane_id(), wid = threadIdx.x / WAVE;
  const uint32_t ic = wave_scan_add_u32(c);
  const uint32_t lo = wave_scan_add_u32((uint32_t)(v & 0xffffffu));
  const uint32_t hi = wave_scan_add_u32((uint32_t)(v >> 24));
  const uint64_t iv = ((uint64_t)hi << 24) + lo;
  __syncthreads();
  if (lane == WAVE - 1) {
    R.a[wid] = ic;
    R.s[wid] = iv;
  }
  __syncthreads();
  const uint32_t xc = R.a[lane & 15];
  const uint64_t xv = R.s[lane & 15];
  ctot = uni_u32(row16_sum_u32(xc));
  vtot = uni_u64(row16_sum_u64(xv));
  cx = row16_sum_u32((lane & 15) < wid ? xc : 0u) + ic - c;
  vx = row16_sum_u64((lane & 15) < wid ? xv : 0ull) + iv - v;
}

/* a wave's append of popc(mask) items per lane with one atomic: this lane's
 * first slot (every lane of the wave calls it) */
__device__ __forceinline__ int wave_append_mask(uint32_t mask, int *counter) {
  const uint32_t cnt = (uint32_t)__popc(mask);
  const uint32_t incl = wave_scan_add_u32(cnt);
  const uint32_t total = readlane_u(incl, WAVE - 1);
  int base = 0;
  if (total != 0u) {
    if (lane_id() == WAVE - 1) base = atomicAdd(counter, (int)total);
    base = (int)readlane_u((uint32_t)base, WAVE - 1);
  }
  return base + (int)(incl - cnt);
}

/* x's bucket: t = RN(m - x) scale, t <= RN(dmax scale) < NBK for finite x,
 * +inf for -inf (bucket NBK) */
template <int NBK>
__device__ __forceinline__ int topp_bucket_of(float x, float m, float scale) {
  return (int)fminf((m - x) * scale, (float)NBK);
}

/* the largest bucket b with start(b) <= r (bucket of rank r < V) */
template <int NBK>
__device__ __forceinline__ int topp_bucket_of_rank(const uint32_t *bstart, int r) {
  int lo = 0, hi = NBK + 1;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (bstart[mid] <= (uint32_t)r)
      lo = mid;
    else
      hi = mid;
  }
  return lo;
}

/* 4'-5' once the bucket counts and group sums are in LDS.  Returns the id,
 * TOPP_FULL, or (the first try: the exact prefix puts the cut outside the
 * range the bands chose) TOPP_RETRY, after which the row is run again as the
 * exact retry (exact_grp): exact group sums of fix40(expf(x - lse)) then give
 * the group holding the cut and the exact prefix before it.  Every thread
 * calls it and every return follows a barrier. */
template <int EPT, int TBLOCK, int NBK>
__device__ __forceinline__ int topp_ids_fast(const SampleArgs &a, int row, const float (&x)[EPT],
                                             float m, float xmin, float scale, float top_p,
                                             uint32_t *bstart, uint64_t *gsum, char *dyn, TRed &R,
                                             const bool exact_grp) {
  constexpr int PER = NBK / TBLOCK;
  static_assert(PER % 4 == 0, "whole 16-byte groups of buckets per thread");
  const int V = a.vocab, k = a.k;
  const int tid = (int)threadIdx.x, lane = lane_id();
  uint64_t *lkey = (uint64_t *)(dyn + tf_lkey(TBLOCK));
  uint64_t *lval = (uint64_t *)(dyn + tf_lval(TBLOCK)); /* bucket */
  int *rr = (int *)(dyn + tf_rr(TBLOCK));
  float *ru = (float *)(dyn + tf_ru(TBLOCK));
  /* [0] elements, [1] flag, [2] id, [3] refined ranks, [4] the cut group,
   * [5] (the first try) the group holding the certain keep band's end */
  uint32_t *misc = (uint32_t *)(dyn + tf_misc(TBLOCK));
  /* [0] the cut group's prefix Q; [1] the first try: group [5]'s Q, the retry: the
   * exact prefix before the cut group */
  uint64_t *misc64 = (uint64_t *)(dyn + tf_misc(TBLOCK) + 32);
  uint32_t *cbits = (uint32_t *)(dyn + tf_cbits(TBLOCK));
  uint32_t *rbits = (uint32_t *)(dyn + tf_rbits(TBLOCK, NBK));
  /* thread t takes the uniforms of ranks q TBLOCK + t (q < EPT): read
   * coalesced */

  /* this thread's ranks' uniforms, issued before the scan (not with the row:
   * fewer registers live through the counting); the scan and the bands
   * cover their wait */
  float uv[EPT];
#pragma unroll
  for (int q = 0; q < EPT; q++) {
    const int r = q * TBLOCK + tid;
    uv[q] = a.u[(size_t)row * k + (r < k ? r : k - 1)]; /* (r >= k: unused) */
  }

  /* ---- bucket starts, group prefixes and the row sum S, one scan */
  uint64_t gst, gs, S;
  {
    uint4 c[PER / 4];
    uint32_t loc = 0u;
#pragma unroll
    for (int q = 0; q < PER / 4; q++) {
      c[q] = *(const uint4 *)&bstart[tid * PER + 4 * q];
      loc += c[q].x + c[q].y + c[q].z + c[q].w;
    }
    gs = gsum[tid];
    if (exact_grp) gsum[tid] = 0ull; /* (only this thread reads entry tid; the scan's barriers follow) */
    uint32_t run, tot;
    block_excl_scan2(loc, gs, R, run, tot, gst, S);
#pragma unroll
    for (int q = 0; q < PER / 4; q++) {
      const uint32_t cc[4] = {c[q].x, c[q].y, c[q].z, c[q].w};
      uint32_t st[4];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        st[e] = run;
        run += cc[e];
      }
      *(uint4 *)&bstart[tid * PER + 4 * q] = make_uint4(st[0], st[1], st[2], st[3]);
    }
    if (tid == 0) bstart[NBK] = tot;
  }
  /* ---- 4'. the row's lse, the least prefix above top_p (Tq) and the
   * certain drop and keep bands: the same in every thread, so wave 0 alone
   * computes them and files them in LDS while the other waves pass to the
   * barrier; then the cut's range [klo, khi]: the group whose prefix crosses
   * the certain drop band (one thread's: the prefixes only grow) */
  if (tid < WAVE) {
    const float lnS = d3s_logf(d3s_fixsum_to_f32(S));
    const float lse0 = m + lnS;
    const uint64_t Tq0 = d3s_fixsum_gt_threshold(top_p);
    uint64_t td = ~0ull, tk = 0ull;
    if (!exact_grp && Tq0 != 0ull && !(Tq0 > ((uint64_t)k << 41))) {
      const CutBands cb = topp_cut_bands_lean(Tq0, S, lse0, lnS, xmin, k);
      td = cb.tdrop;
      tk = cb.tkeep;
    }
    if (tid == 0) {
      R.row_q[0] = Tq0;
      R.row_q[1] = td;
      R.row_q[2] = tk;
      R.row_lse = lse0;
    }
  }
  __syncthreads();
  const float lse = R.row_lse;
  const uint64_t Tq = R.row_q[0];
  const bool settled1 = Tq == 0ull;                     /* every prefix passes: cut 1 */
  const bool settledk = Tq > ((uint64_t)k << 41);      /* none reaches it: cut k */
  uint64_t tdrop = ~0ull, tkeep = 0ull;
  uint64_t pg0 = 0ull; /* the retry: the exact prefix before the group */
  if (!exact_grp) {
    if (!settled1 && !settledk) {
      tdrop = R.row_q[1];
      tkeep = R.row_q[2];
      if (gst < tdrop && tdrop <= gst + gs) {
        misc[4] = (uint32_t)tid;
        misc64[0] = gst;
      }
      if (gst < tkeep && tkeep <= gst + gs) {
        misc[5] = (uint32_t)tid;
        misc64[1] = gst;
      }
    }
  } else {
    /* the retry: exact group sums (the scan's barriers ordered the clearing
     * before these), their prefixes, the first group reaching Tq */
#pragma unroll
    for (int j = 0; j < EPT; j++) { /* (-inf and past the row: 0, into a slot past the groups') */
      const int b = topp_bucket_of<NBK>(x[j], m, scale);
      atomicAdd((unsigned long long *)&gsum[(uint32_t)b / PER], (unsigned long long)d3s_fix40_exp(x[j] - lse));
    }
    __syncthreads();
    const uint64_t E = gsum[tid];
    uint32_t cx, ctot;
    uint64_t Ex, Etot;
    block_excl_scan2(0u, E, R, cx, ctot, Ex, Etot);
    if (!settled1 && Ex < Tq && Tq <= Ex + E) {
      misc[4] = (uint32_t)tid;
      misc64[0] = gst;
      misc64[1] = Ex;
    }
  }
  __syncthreads(); /* the starts, the map, the cut group */
  const int g = settled1 || (settledk && !exact_grp) ? -1 : (int)misc[4]; /* -1: no group (cleared to ~0) */
  /* the cut lies in groups [gl, g]: the first try widens the range back to the
   * group where the bands' keep end falls when the elements fit one wave
   * (the bands straddling a group boundary would otherwise leave a cut
   * before the group to the retry) */
  int gl = g;
  if (g >= 0) {
    if (exact_grp) {
      pg0 = misc64[1];
    } else {
      const uint32_t l = misc[5]; /* (~0: tkeep 0, no group) */
      if (l < (uint32_t)g && bstart[g * PER + PER] - bstart[l * PER] <= (uint32_t)TF_CAP) gl = (int)l;
    }
  }
  const uint64_t qg = gl < g ? misc64[1] : misc64[0]; /* Q before the range */
  uint32_t s0 = 0u;
  int klo, khi;
  if (settled1) {
    klo = khi = 1;
  } else if (g < 0) {
    klo = khi = k; /* no rank certainly drops (when not settled: the last must certainly stay) */
  } else {
    s0 = bstart[gl * PER];
    const uint32_t n = bstart[g * PER + PER] - s0;
    if (n > (uint32_t)TF_CAP) return TOPP_FULL; /* (after the barrier above) */
    klo = max((int)s0, 1); /* cut = max(r1, 1), r1 the group's first rank reaching tdrop */
    khi = max((int)(s0 + n) - 1, 1);
  }

  /* ---- 5'. first bounds, in units of inv: e <= 1 on every rank that may
   * be kept (r < khi); e >= emin on those certainly kept (r < klo) */
  const float rs = 1.0f / scale, dmax = m - xmin;
  float emin = 1.0f; /* klo = 1: rank 0 alone, e_0 = 1 */
  if (klo > 1) {
    float eh;
    if (g >= 0)
      topp_ebounds<NBK>(gl * PER - 1, rs, dmax, emin, eh); /* the ranks before the range */
    else
      topp_ebounds<NBK>(bstart[NBK] < (uint32_t)V ? NBK : NBK - 1, rs, dmax, emin, eh); /* every rank */
  }
  /* LB1, the largest first lower bound over the certainly kept ranks: lb
   * decreases in u where it is defined (2^-24 <= u < 1; -1 elsewhere), so a
   * thread's is the lb of its least such u (one evaluation, not one a rank) */
  /* this thread's ranks q TBLOCK + tid below klo (khi) are those of q < qlo (qhi) */
  const int qlo = klo > tid ? min((klo - tid + TBLOCK - 1) / TBLOCK, EPT) : 0;
  const int qhi = khi > tid ? min((khi - tid + TBLOCK - 1) / TBLOCK, EPT) : 0;
  float umin = 1.0f;
#pragma unroll
  for (int q = 0; q < EPT; q++)
    if (q < qlo && uv[q] >= 0x1p-24f) umin = fminf(umin, uv[q]);
  float lbm = -1.0f;
  if (umin < 1.0f) {
    float h_unused;
    topp_sbounds(emin, 1.0f, umin, lbm, h_unused);
  }
  const float LB1 = block_max_f(lbm, R);
  /* the ranks whose first upper bound (h = +inf for u <= 2^-24, rcp(u - 2^-24)
   * (1 + 2^-18)(1 + 2^-20) below 1, 0 from 1 on) reaches LB1, to one wave.
   * For LB1 > 0 that is u <= 2^-24 + C / LB1 with C within 1.0000004 (the
   * rcp's ulp included): the test u <= uthr with 1.01 in C's place takes a
   * superset, which the refinement below settles.  For LB1 <= 0 every rank
   * that may be kept. */
  {
    uint32_t pm = 0u;
    const uint32_t qmask = (1u << qhi) - 1u;
    if (LB1 > 0.0f) {
      /* (u < 1 folded in: the threshold is capped below 1) */
      const float uthr = fminf(0x1p-24f + (1.0f / LB1) * 1.01f, 0x1.fffffep-1f);
#pragma unroll
      for (int q = 0; q < EPT; q++) pm |= (uv[q] <= uthr ? 1u : 0u) << q;
      pm &= qmask;
    } else {
      pm = qmask;
    }
    /* (most waves file none: the append is skipped wave by wave) */
    if (__ballot(pm != 0u)) {
      int slot = wave_append_mask(pm, (int *)&misc[3]);
#pragma unroll
      for (int q = 0; q < EPT; q++)
        if ((pm >> q) & 1u) {
          if (slot < TF_CAP) {
            rr[slot] = q * TBLOCK + tid;
            ru[slot] = uv[q];
          }
          slot++;
        }
    }
  }
  __syncthreads();
  const uint32_t nref = misc[3];
  if (nref > (uint32_t)TF_CAP) return TOPP_FULL; /* (after the barrier above) */
  /* wave 0 keeps the refined ranks in registers (lane t: rank t) */
  int my_rr = 0;
  float my_ru = 0.0f;
  if (tid < WAVE) {
    /* their buckets' bounds; LB2 and the candidates */
    const bool mine = lane < (int)nref;
    my_rr = mine ? rr[lane] : 0x7fffffff;
    my_ru = mine ? ru[lane] : 0.0f;
    int b = 0;
    /* the bucket holding rank r: the last whose start is at or below r
     * (a binary search over the starts, for these few ranks) */
    if (mine) b = topp_bucket_of_rank<NBK>(bstart, my_rr);
    float lb = -1.0f, h = -__builtin_inff();
    if (mine) {
      float elo, ehi, l2;
      topp_ebounds<NBK>(b, rs, dmax, elo, ehi);
      topp_sbounds(elo, ehi, my_ru, l2, h);
      if (my_rr < klo) lb = l2;
    }
    const float LB2 = fmaxf(LB1, wave_max_f(lb));
    if (mine && h >= LB2) {
      atomicOr(&rbits[my_rr >> 5], 1u << (my_rr & 31));
      atomicOr(&cbits[b >> 5], 1u << (b & 31));
    }
  }
  __syncthreads();
  /* ---- one gather: the cut group's elements and the candidates' buckets' */
  {
    uint32_t gm = 0u;
    /* the range's buckets [b_lo, b_hi); element j of this thread lies in the row for j < nj */
    const int b_lo = gl * PER, b_hi = g * PER + PER;
    const int nj = V > tid ? min((V - tid + TBLOCK - 1) / TBLOCK, EPT) : 0;
#pragma unroll
    for (int j = 0; j < EPT; j++) {
      const int bb = topp_bucket_of<NBK>(x[j], m, scale);
      const bool in = j < nj && ((bb >= b_lo && bb < b_hi) || ((cbits[bb >> 5] >> (bb & 31)) & 1u) != 0u);
      gm |= (in ? 1u : 0u) << j;
    }
    if (__ballot(gm != 0u)) {
      int slot = wave_append_mask(gm, (int *)&misc[0]);
#pragma unroll
      for (int j = 0; j < EPT; j++)
        if ((gm >> j) & 1u) {
          if (slot < TF_CAP) {
            lkey[slot] = composite_key(x[j], j * TBLOCK + tid);
            lval[slot] = (uint64_t)(uint32_t)topp_bucket_of<NBK>(x[j], m, scale);
          }
          slot++;
        }
    }
  }
  __syncthreads();
  const uint32_t n2 = misc[0];
  if (n2 > (uint32_t)TF_CAP) return TOPP_FULL; /* (after the barrier above) */
  /* ---- wave 0: rank the gathered elements; the cut from the group's
   * prefixes (lane t: element t; the others' keys by readlane) */
  bool mine = false, ing = false;
  uint64_t mk = 0ull, qr = 0ull;
  int r = 0x7fffffff, cut = 0;
  uint64_t qlast = 0ull;
  if (tid < WAVE) {
    mine = lane < (int)n2;
    mk = mine ? lkey[lane] : 0ull;
    const uint32_t mb = mine ? (uint32_t)lval[lane] : 0xffffffffu;
    ing = mine && (int)(mb / PER) >= gl && (int)(mb / PER) <= g; /* (mb / PER < 2^28) */
    const uint64_t f = ing ? d3s_fix40_exp(key_x(mk) - m) : 0ull;
    int rho = 0;
    uint64_t inc = 0ull;
    for (int t = 0; t < (int)n2; t++) {
      const uint64_t kt = ((uint64_t)readlane_u((uint32_t)(mk >> 32), t) << 32) | readlane_u((uint32_t)mk, t);
      const uint32_t bt = readlane_u(mb, t);
      const uint64_t ft = ((uint64_t)readlane_u((uint32_t)(f >> 32), t) << 32) | readlane_u((uint32_t)f, t);
      rho += (bt == mb && kt > mk) ? 1 : 0;
      inc += kt >= mk ? ft : 0ull; /* (0 outside the group) */
    }
    r = mine ? (int)bstart[mb] + rho : 0x7fffffff;
    bool certain;
    if (g >= 0) {
      const uint64_t q0 = qg;
      qr = q0 + inc;
      /* the first rank reaching tdrop (the group's last does); rank 0 never drops */
      const int r1 = wave_min_i32(ing && qr >= tdrop ? r : 0x7fffffff);
      cut = min(max(r1, 1), k);
      qlast = q0; /* cut - 1 = s0 - 1: the prefix before the group */
      if (cut - 1 >= (int)s0) {
        const uint64_t at = __ballot(ing && r == cut - 1);
        const int src = (int)__builtin_ctzll(at | (1ull << 63));
        qlast = ((uint64_t)readlane_u((uint32_t)(qr >> 32), src) << 32) | readlane_u((uint32_t)qr, src);
      }
      /* (the retry: the cut from the group's exact prefixes below) */
      certain = !exact_grp && (cut <= 1 || qlast < tkeep);
    } else {
      cut = klo;
      qlast = cut == 1 ? (1ull << 40) : S; /* rank 0's term, or every term */
      certain = exact_grp || cut <= 1 || settledk || qlast < tkeep;
    }
    if (lane == 0) misc[1] = certain ? 0u : (g >= 0 ? 1u : 2u);
  }
  __syncthreads();
  const uint32_t how = misc[1];
  if (how == 2u) return TOPP_FULL; /* an uncertain last rank: the full path */
  if (how == 1u) {
    /* the cut within the bands' uncertainty: the exact prefix P before the
     * group (block sum of fix40(expf(x - lse)) over the elements of the
     * buckets before it), then the group's exact prefixes */
    uint64_t p0 = pg0;
    if (!exact_grp) {
      uint64_t part = 0ull;
#pragma unroll
      for (int j = 0; j < EPT; j++) {
        const int i = j * TBLOCK + tid;
        const int bb = topp_bucket_of<NBK>(x[j], m, scale);
        if (i < V && bb < gl * PER) part += d3s_fix40_exp(x[j] - lse);
      }
      p0 = block_sum_u64(part, R);
    }
    if (tid < WAVE) {
      const uint64_t pt = ing ? d3s_fix40_exp(key_x(mk) - lse) : 0ull;
      uint64_t pinc = 0ull;
      for (int t = 0; t < (int)n2; t++) {
        const uint64_t kt = ((uint64_t)readlane_u((uint32_t)(mk >> 32), t) << 32) | readlane_u((uint32_t)mk, t);
        const uint64_t ftt = ((uint64_t)readlane_u((uint32_t)(pt >> 32), t) << 32) | readlane_u((uint32_t)pt, t);
        pinc += kt >= mk ? ftt : 0ull;
      }
      /* the first rank whose exact prefix reaches Tq; before the group when
       * p0 does already (then the full path) */
      const int re = wave_min_i32(ing && p0 + pinc >= Tq ? r : 0x7fffffff);
      cut = min(max(re, 1), k);
      qlast = qg;
      if (cut - 1 >= (int)s0) {
        const uint64_t at = __ballot(ing && r == cut - 1);
        const int src = (int)__builtin_ctzll(at | (1ull << 63));
        qlast = ((uint64_t)readlane_u((uint32_t)(qr >> 32), src) << 32) | readlane_u((uint32_t)qr, src);
      }
      /* the cut outside the group: the retry (after the first try), the full path */
      if (lane == 0 && (p0 >= Tq || re == 0x7fffffff)) misc[2] = (uint32_t)(exact_grp ? TOPP_FULL : TOPP_RETRY);
    }
    __syncthreads();
    const uint32_t m2 = misc[2];
    if (m2 == (uint32_t)TOPP_FULL || m2 == (uint32_t)TOPP_RETRY) return (int)m2; /* (after the barrier above) */
  }
  /* ---- the candidates' exact scores and their first maximum */
  if (tid < WAVE) {
    float bs = -2.0f;
    int br = 0x7fffffff;
    const float inv = 1.0f / d3s_fixsum_to_f32(qlast);
    const bool cand = mine && r < cut && ((rbits[r >> 5] >> (r & 31)) & 1u) != 0u;
    /* (every candidate is a refined rank: its uniform is in wave 0's lanes) */
    float uu = 0.0f;
    for (int t = 0; t < (int)nref; t++) {
      const int rt = (int)readlane_u((uint32_t)my_rr, t);
      const float ut = d3s_u2f(readlane_u(d3s_f2u(my_ru), t));
      uu = rt == r ? ut : uu;
    }
    if (cand) {
      bs = topp_score(d3s_expf_nonpos(key_x(mk) - m) * inv, uu);
      br = r;
    }
    const int myr = br;
    wave_argmax(bs, br);
    const uint64_t at = __ballot(cand && myr == br);
    const int src = (int)__builtin_ctzll(at | (1ull << 63));
    const int id = key_idx(((uint64_t)readlane_u((uint32_t)(mk >> 32), src) << 32) | readlane_u((uint32_t)mk, src));
    if (lane == 0) misc[2] = bs > 0.0f ? (uint32_t)id : (uint32_t)TOPP_FULL;
  }
  __syncthreads();
  return (int)misc[2];
}

/* Phases 3-5 (the full path) from x and e = expf(x - m). */
template <int EPT, bool BF16, int TBLOCK>
__device__ __forceinline__ void topp_full(const SampleArgs &a, int row, const RowP &rp, const char *rowp,
                                          const float (&x)[EPT], const float (&ev)[EPT], float m, float xmin,
                                          float scale, uint64_t S, float lnS, float lse, uint32_t *bstart,
                                          uint64_t *keys, TRed &R) {
  constexpr int NBK = topp_buckets(EPT * TBLOCK, TBLOCK);
  const int V = a.vocab, k = a.k;
  const int tid = (int)threadIdx.x;
  const float T = rp.T;
  const bool t_finite = T < __builtin_inff();
  const float y = 1.0f / T;

  /* ---- 3. ranks: counting sort over buckets of m - x, exact within buckets */
#pragma unroll
  for (int b = 4 * tid; b < NBK; b += 4 * TBLOCK) *(uint4 *)&bstart[b] = make_uint4(0u, 0u, 0u, 0u);
  if (tid == 0) bstart[NBK] = 0u;
  __syncthreads();
  int bk[EPT];
#pragma unroll
  for (int j = 0; j < EPT; j++) {
    const int i = j * TBLOCK + tid;
    int b = NBK;
    if (x[j] != -__builtin_inff()) b = scale > 0.0f ? min((int)((m - x[j]) * scale), NBK - 1) : 0;
    bk[j] = b;
    if (i < V) atomicAdd(&bstart[b], 1u);
  }
  __syncthreads();
  {
    /* exclusive scan of the counts of the NBK finite buckets: thread t owns
     * PER consecutive ones, read and written 4 at a time; the -inf bucket
     * starts after them all */
    constexpr int PER = NBK / TBLOCK;
    uint4 c[PER / 4];
    uint32_t loc = 0u;
#pragma unroll
    for (int q = 0; q < PER / 4; q++) {
      c[q] = *(const uint4 *)&bstart[tid * PER + 4 * q];
      loc += c[q].x + c[q].y + c[q].z + c[q].w;
    }
    uint32_t tot;
    uint32_t run = block_excl_scan_u32(loc, R, tot);
#pragma unroll
    for (int q = 0; q < PER / 4; q++) {
      uint4 o;
      o.x = run;
      o.y = o.x + c[q].x;
      o.z = o.y + c[q].y;
      o.w = o.z + c[q].z;
      run = o.w + c[q].w;
      *(uint4 *)&bstart[tid * PER + 4 * q] = o;
    }
    if (tid == 0) bstart[NBK] = tot;
  }
  __syncthreads();
  uint64_t key[EPT];
#pragma unroll
  for (int j = 0; j < EPT; j++) {
    const int i = j * TBLOCK + tid;
    key[j] = composite_key(x[j], i);
    if (i < V) keys[atomicAdd(&bstart[bk[j]], 1u)] = key[j];
  }
  __syncthreads();
  /* now bstart[b] is the end of bucket b, the start of bucket b + 1 */
  /* the elements' buckets side by side, two members of each per step */
  int rank[EPT];
  uint32_t b0[EPT], bn[EPT], most = 0u;
#pragma unroll
  for (int j = 0; j < EPT; j++) {
    const bool in = j * TBLOCK + tid < V;
    b0[j] = in && bk[j] > 0 ? bstart[bk[j] - 1] : 0u;
    bn[j] = in ? bstart[bk[j]] - b0[j] : 0u;
    rank[j] = in ? (int)b0[j] : 0x7fffffff;
    most = max(most, bn[j]);
  }
  for (uint32_t q = 0; q < most; q += 2u) {
#pragma unroll
    for (int j = 0; j < EPT; j++)
      if (q < bn[j]) {
        const uint64_t k0 = keys[b0[j] + q];
        const uint64_t k1 = keys[min(b0[j] + q + 1u, (uint32_t)V - 1u)];
        rank[j] += (k0 > key[j] ? 1 : 0) + (q + 1u < bn[j] && k1 > key[j] ? 1 : 0);
      }
  }
  /* From here on thread t owns the ranks [t RPT, t RPT + RPT): the uniforms
   * are read in rank order (the race needs them last), and LDS holds by rank
   * each element's e (high word) and ~index (low word). */
  const int RPT = (k + TBLOCK - 1) / TBLOCK; /* <= EPT */
  const int r0 = tid * RPT;
  float uv[EPT];
#pragma unroll
  for (int q = 0; q < EPT; q++) uv[q] = (q < RPT && r0 + q < k) ? a.u[(size_t)row * k + r0 + q] : 0.0f;
  __syncthreads();
#pragma unroll
  for (int j = 0; j < EPT; j++)
    if (rank[j] < k) keys[rank[j]] = ((uint64_t)d3s_f2u(ev[j]) << 32) | (uint32_t)key[j];
  __syncthreads();

  /* ---- 4. the cut: the first r > 0 whose exact prefix P_r of the terms
   * fix40(expf(x_r - lse)) passes top_p (fixsum_to_f32(P) > top_p is P >=
   * Tq).  First from the prefixes Q_r of fix40(e_r) and the certain bands
   * (topp_cut_bands): if the rank before the first certain drop does not
   * certainly stay, the exact prefixes decide. */
  const uint64_t Tq = d3s_fixsum_gt_threshold(rp.top_p);
  uint64_t qt[EPT];
  uint64_t qloc = 0;
#pragma unroll
  for (int q = 0; q < EPT; q++) {
    const int r = r0 + q;
    qt[q] = (q < RPT && r < k) ? d3s_fix40_unit(d3s_u2f((uint32_t)(keys[r] >> 32))) : 0ull;
    qloc += qt[q];
  }
  uint64_t Qp = block_excl_scan_u64(qloc, R);
  int cut;
  bool exact_cut = false;
  if (Tq == 0ull) {
    cut = 1; /* every prefix passes; rank 0 never drops */
  } else if (Tq > ((uint64_t)k << 41)) {
    cut = k; /* no prefix of at most k terms below 1 reaches it */
  } else {
    const CutBands cb = topp_cut_bands(Tq, S, lse, lnS, xmin, k);
    const uint64_t Tdrop = cb.tdrop, Tkeep = cb.tkeep;
    int drop = k;
    uint64_t Q = Qp;
#pragma unroll
    for (int q = 0; q < EPT; q++) {
      const int r = r0 + q;
      Q += qt[q];
      if (q < RPT && r < k && r > 0 && drop == k && Q >= Tdrop) drop = r;
    }
    cut = block_min_i32(drop, R);
    /* the rank before it (or the last rank) must certainly stay */
    const int last = cut - 1;
    if (threadIdx.x == 0) R.a[0] = 0u;
    __syncthreads();
    if (last > 0 && last >= r0 && last < r0 + RPT) {
      Q = Qp;
#pragma unroll
      for (int q = 0; q < EPT; q++)
        if (r0 + q <= last) Q += qt[q];
      if (!(Q < Tkeep)) R.a[0] = 1u;
    }
    __syncthreads();
    exact_cut = R.a[0] != 0u || (a.flags & FLAG_EXACT_LSE) != 0;
  }
  if (exact_cut) {
    if (threadIdx.x == 0 && a.counters) atomicAdd(&a.counters[CNT_EXACT_LSE], 1u);
    /* x_r again from the row (the banned index stays -inf), then the exact
     * prefixes */
    uint64_t term[EPT];
    uint64_t loc = 0;
#pragma unroll
    for (int q = 0; q < EPT; q++) {
      const int r = r0 + q;
      term[q] = 0ull;
      if (q < RPT && r < k) {
        const int idx = key_idx(keys[r]);
        const float xr = scale_logit(load_logit<BF16>(rowp, idx, rp.banned), T, y, t_finite);
        term[q] = d3s_fix40_exp(xr - lse); /* x_r <= m <= lse */
      }
      loc += term[q];
    }
    uint64_t P = block_excl_scan_u64(loc, R);
    int cut_local = k;
    /* prefix sums only grow: the cut lies among this thread's ranks only if
     * their last prefix passes the threshold */
    if (P + loc >= Tq) {
#pragma unroll
      for (int q = 0; q < EPT; q++) {
        const int r = r0 + q;
        P += term[q];
        if (q < RPT && r < k && r > 0 && cut_local == k && P >= Tq) cut_local = r;
      }
    }
    cut = block_min_i32(cut_local, R);
  }

  /* ---- 5. the kept ranks r < cut (x_0 = m): their exact sum, probabilities
   * and the race.  Threads whose ranks all lie at or past the cut skip. */
  /* Their exact sum is the prefix at the cut of the terms fix40(e_r) that
   * the cut started from: the thread holding rank cut - 1 files it. */
  {
    const int last = cut - 1;
    if (last >= r0 && last < r0 + RPT) {
      uint64_t Q = Qp;
#pragma unroll
      for (int q = 0; q < EPT; q++)
        if (r0 + q <= last) Q += d3s_fix40_unit(d3s_u2f((uint32_t)(keys[r0 + q] >> 32)));
      R.kept = Q;
    }
  }
  float e[EPT];
#pragma unroll
  for (int q = 0; q < EPT; q++) {
    const int r = r0 + q;
    e[q] = 0.0f;
    if (q < RPT && r < cut) e[q] = d3s_u2f((uint32_t)(keys[r] >> 32)); /* exp(x_r - m), in [0, 1] */
  }
  __syncthreads();
  const float inv = 1.0f / d3s_fixsum_to_f32(uni_u64(R.kept));
  /* Proven bounds of each score sc = max(p / noise, -1), noise = -log(1 - u):
   * RN(1 - u) lies within a relative 2^-24 of 1 - u and d3s_logf within one
   * ulp, so for u in [2^-24, 1)  u - 2^-24 <= noise <= (u / (1 - u) +
   * 2^-24) (1 + 2^-23); the margins 2^-18 also cover the bounds' own
   * rounding.  No score below the largest lower bound can be the first
   * maximum: only the others take the exact logarithm and division. */
  float ub[EPT];
  float lbm = -1.0f;
#pragma unroll
  for (int q = 0; q < EPT; q++) {
    const int r = r0 + q;
    ub[q] = -__builtin_inff();
    if (q < RPT && r < cut) {
      const float p = e[q] * inv;
      const float uu = uv[q];
      float lb = -1.0f, hb = __builtin_inff();
      if (uu >= 0x1p-24f && uu < 1.0f) {
        /* v_rcp_f32 is within one ulp: inside the margins */
        lb = p * __builtin_amdgcn_rcpf(uu * __builtin_amdgcn_rcpf(1.0f - uu) + 0x1p-22f) * (1.0f - 0x1p-18f);
        if (uu > 0x1p-24f) hb = p * __builtin_amdgcn_rcpf(uu - 0x1p-24f) * (1.0f + 0x1p-18f);
      } else if (uu >= 1.0f) {
        hb = 0.0f; /* noise +inf (score 0) or NaN (score -1) */
      }
      ub[q] = hb;
      lbm = fmaxf(lbm, lb);
    }
  }
  const float LB = block_max_f(lbm, R);
  float bs = -1.0f;
  int br = 0x7fffffff;
#pragma unroll
  for (int q = 0; q < EPT; q++) {
    const int r = r0 + q;
    if (ub[q] >= LB) { /* only kept ranks: the others hold -inf */
      const float sc = topp_score(e[q] * inv, uv[q]);
      if (sc > bs || (sc == bs && r < br)) {
        bs = sc;
        br = r;
      }
    }
  }
  /* A dropped rank has p = 0: its score is 0 or NaN.  With a positive kept
   * maximum it cannot win; otherwise (u at or near 0 or 1 on every kept
   * rank) every rank below k races, as in the reference. */
  block_argmax(bs, br, R);
  if (!(bs > 0.0f)) {
    bs = -1.0f;
    br = 0x7fffffff;
#pragma unroll
    for (int q = 0; q < EPT; q++) {
      const int r = r0 + q;
      if (q < RPT && r < k) {
        const float sc = topp_score(r < cut ? e[q] * inv : 0.0f, uv[q]);
        if (sc > bs || (sc == bs && r < br)) {
          bs = sc;
          br = r;
        }
      }
    }
    block_argmax(bs, br, R);
  }
  if (tid == 0) a.ids[row] = key_idx(keys[br]);
  if (a.probs || a.cand) {
#pragma unroll
    for (int q = 0; q < EPT; q++) {
      const int r = r0 + q;
      if (q < RPT && r < k) {
        if (a.probs) a.probs[(size_t)row * k + r] = r < cut ? e[q] * inv : 0.0f;
        if (a.cand) a.cand[(size_t)row * k + r] = key_idx(keys[r]);
      }
    }
  }
}

/* the block's shared arrays and the reduction entries of absent waves */
#define D3S_TOPP_SHARED                                                                         \
  constexpr int NBK = topp_buckets(EPT * TBLOCK, TBLOCK);                                       \
  constexpr int NW = TBLOCK / WAVE;                                                             \
  static_assert(NW <= TNW, "one reduction entry per wave");                                     \
  extern __shared__ uint64_t keys[]; /* V slots: by bucket, then by rank (or the ids path's) */ \
  static_assert(NBK % (4 * TBLOCK) == 0, "whole 16-byte groups of buckets per thread");         \
  __shared__ __align__(16) uint32_t bstart[NBK + 4]; /* bucket counts, first slots, then ends */ \
  __shared__ TRed R;                                                                            \
  const int tid = (int)threadIdx.x;                                                             \
  if (NW < TNW && tid >= NW && tid < TNW) {                                                     \
    /* the reduction entries of absent waves: identities, never overwritten */                  \
    R.f[tid] = R.g[tid] = R.h[tid] = -__builtin_inff();                                         \
    R.s[tid] = 0ull;                                                                            \
    R.a[tid] = 0u;                                                                              \
    R.r[tid] = 0x7fffffff;                                                                      \
  }

/* phase 1's ending: the row's max m (NaN or +inf: refused) and least finite
 * x; false when the row was written as a special case */
template <int EPT>
__device__ __forceinline__ bool topp_max_min(const SampleArgs &a, int row, float xm, float xl, float &m, float &xmin,
                                             TRed &R) {
  /* xm: the thread's maximum with NaN propagated and +inf kept, so the
   * row's is NaN or +inf exactly when some x is (refused) */
  float M = xm, nxl = -xl;
  block_max2_f(M, nxl, R);
  m = M;
  if (!(M < __builtin_inff())) {
    write_special(a, row, false);
    return false;
  }
  if (m == -__builtin_inff()) {
    write_special(a, row, true);
    return false;
  }
  xmin = -nxl;
  return true;
}

/* The full path for row `row` (every output: ids, probabilities,
 * candidates), by the whole workgroup; keys: V slots of LDS. */
template <int EPT, bool BF16, int TBLOCK, int NBK>
__device__ __forceinline__ void topp_full_row(const SampleArgs &a, const int row, uint64_t *keys, uint32_t *bstart,
                                              TRed &R) {
  const int tid = (int)threadIdx.x;
  const int V = a.vocab;
  const RowP rp = row_params(a, row);
  const float T = rp.T;
  const bool t_finite = T < __builtin_inff();
  const float y = 1.0f / T;
  const char *rowp = (const char *)a.logits + (size_t)row * (size_t)a.row_stride * (BF16 ? 2 : 4);

  /* ---- 1. x, classification, max and smallest finite x */
  float x[EPT];
  float xm = -__builtin_inff(), xl = __builtin_inff();
  /* every load in flight before the first use (past the row's end, the last
   * element is read again and ignored) */
#pragma unroll
  for (int j = 0; j < EPT; j++) {
    const int i = j * TBLOCK + tid;
    x[j] = load_logit<BF16>(rowp, i < V ? i : V - 1, rp.banned);
  }
  /* xm: the maximum with NaN propagated, so NaN or +inf anywhere shows in it;
   * xl: the least x above -inf */
#pragma unroll
  for (int j = 0; j < EPT; j++) {
    const int i = j * TBLOCK + tid;
    const float xi = i < V ? scale_logit(x[j], T, y, t_finite) : -__builtin_inff();
    x[j] = xi;
    xm = __builtin_elementwise_maximum(xm, xi);
    xl = fminf(xl, xi > -__builtin_inff() ? xi : __builtin_inff());
  }
  float m, xmin;
  if (!topp_max_min<EPT>(a, row, xm, xl, m, xmin, R)) return;
  const float dmax = m - xmin;
  const float scale = (dmax > 0.0f && dmax < __builtin_inff()) ? (float)(NBK - 1) / dmax : 0.0f;

  /* ---- 2. e = exp(x - m) and the exact row sum and lse (x = -inf, and
   * i >= V, add 0); e is also each element's softmax term (x_0 = m) */
  float ev[EPT];
  uint64_t acc = 0;
#pragma unroll
  for (int j = 0; j < EPT; j++) {
    ev[j] = d3s_expf_nonpos(x[j] - m); /* in [0, 1] */
    acc += d3s_fix40_unit(ev[j]);
  }
  const uint64_t S = block_sum_u64(acc, R);
  const float lnS = d3s_logf(d3s_fixsum_to_f32(S));
  const float lse = m + lnS;
  topp_full<EPT, BF16, TBLOCK>(a, row, rp, rowp, x, ev, m, xmin, scale, S, lnS, lse, bstart, keys, R);
}

/* k_topp: every output (ids, probabilities, candidates) by the full path */
template <int EPT, bool BF16, int TBLOCK>
__global__ __launch_bounds__(TBLOCK) __attribute__((amdgpu_waves_per_eu(topp_waves(EPT, TBLOCK)))) void k_topp(
    SampleArgs a) {
  D3S_TOPP_SHARED
  topp_full_row<EPT, BF16, TBLOCK, NBK>(a, (int)blockIdx.x, keys, bstart, R);
}

/* The rows the ids-only path leaves to the full path: a count and the rows,
 * filed by k_topp_ids and taken by k_topp_redo, which leaves the count (and
 * its own arrival count) zero again.  The counts sit in the first two
 * 128-byte lines of the stream workspace's counter block (every kernel that
 * counts there leaves its counters zero); the rows after the block. */
struct ToppRedo {
  uint32_t *count; /* rows filed */
  uint32_t *done;  /* k_topp_redo's workgroups finished */
  int32_t *rows;   /* [n_rows] */
};

/* waves per SIMD of the ids-only kernel: its LDS (the bucket bounds and the
 * ids path's arrays, without the full path's keys) fits four 512-thread
 * workgroups per CU */
constexpr int topp_ids_waves(int ept, int tb) { return tb == 512 ? 8 : topp_waves(ept, tb); }

/* The ids-only path for row `row` (ids only, k = V), by the whole workgroup;
 * dyn: its LDS arrays.  Returns true when the row's id is written, false when
 * the row needs another pass (the retry, exact_grp, or after it the full path). */
template <int EPT, bool BF16, int TBLOCK, int NBK>
__device__ __forceinline__ bool topp_ids_row(const SampleArgs &a, const int row, char *dyn, uint32_t *bstart,
                                             uint64_t *gsum, TRed &R, const bool exact_grp) {
  constexpr int PER = NBK / TBLOCK;
  const int tid = (int)threadIdx.x;
  const int V = a.vocab;
  const RowP rp = row_params(a, row);
  const float T = rp.T;
  const bool t_finite = T < __builtin_inff();
  const float y = 1.0f / T;
  const char *rowp = (const char *)a.logits + (size_t)row * (size_t)a.row_stride * (BF16 ? 2 : 4);
  {
    /* bucket counts, group sums, counters and bitmaps cleared (phase 1's
     * barriers order this before the counting) */
#pragma unroll
    for (int b = 4 * tid; b < NBK; b += 4 * TBLOCK) *(uint4 *)&bstart[b] = make_uint4(0u, 0u, 0u, 0u);
    if (tid < 4) bstart[NBK + tid] = 0u;
    if (tid < 16) ((uint32_t *)(dyn + tf_misc(TBLOCK)))[tid] = tid == 4 || tid == 5 ? ~0u : 0u;
    gsum[tid] = 0ull;
    uint32_t *cbits = (uint32_t *)(dyn + tf_cbits(TBLOCK));
    uint32_t *rbits = (uint32_t *)(dyn + tf_rbits(TBLOCK, NBK));
    for (int w = tid; w < NBK / 32 + 4; w += TBLOCK) cbits[w] = 0u;
    for (int w = tid; w < 4 * ((V + 127) / 128); w += TBLOCK) rbits[w] = 0u;
  }

  /* ---- 1. x (with T = 1, x = L: RN(L / 1) = L), max and least finite x */
  float x[EPT];
  float xm = -__builtin_inff(), xl = __builtin_inff();
  /* element j of this thread lies in the row for j < nj; reads through a
   * buffer resource spanning the row (past its end they return 0, masked
   * below), and the banned element is masked by the one thread holding it */
  const int nj = V > tid ? min((V - tid + TBLOCK - 1) / TBLOCK, EPT) : 0;
  {
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void *)rowp, (short)0, V * (BF16 ? 2 : 4), 0x00020000);
#pragma unroll
    for (int j = 0; j < EPT; j++) {
      const int i = j * TBLOCK + tid;
      if (BF16)
        x[j] = d3s_u2f((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, i * 2, 0, 0) << 16);
      else
        x[j] = d3s_u2f(__builtin_amdgcn_raw_buffer_load_b32(rs, i * 4, 0, 0));
    }
    if ((unsigned)rp.banned < (unsigned)V && tid == rp.banned % TBLOCK) {
      const int jb = rp.banned / TBLOCK;
#pragma unroll
      for (int j = 0; j < EPT; j++)
        if (j == jb) x[j] = -__builtin_inff();
    }
  }
  if (T == 1.0f) {
#pragma unroll
    for (int j = 0; j < EPT; j++) {
      const float xi = j < nj ? x[j] : -__builtin_inff();
      x[j] = xi;
      xm = __builtin_elementwise_maximum(xm, xi);
      xl = fminf(xl, xi > -__builtin_inff() ? xi : __builtin_inff());
    }
  } else {
#pragma unroll
    for (int j = 0; j < EPT; j++) {
      const float xi = j < nj ? scale_logit(x[j], T, y, t_finite) : -__builtin_inff();
      x[j] = xi;
      xm = __builtin_elementwise_maximum(xm, xi);
      xl = fminf(xl, xi > -__builtin_inff() ? xi : __builtin_inff());
    }
  }
  float m, xmin;
  if (!topp_max_min<EPT>(a, row, xm, xl, m, xmin, R)) return true; /* (id written) */
  const float dmax = m - xmin;
  const float scale = (dmax > 0.0f && dmax < __builtin_inff()) ? (float)(NBK - 1) / dmax : 0.0f;

  /* ---- 2'. each element's bucket count and its group's sum of fix40(e).
   * Elements past the row hold x = -inf: they count in the -inf bucket NBK,
   * whose count nothing reads (its start is the finite total and it runs to
   * the row's end), and add 0 to a sum past the groups'.  The bucket comes
   * from d = x - m, as (m - x) scale = d (-scale) exactly. */
  if (scale > 0.0f) {
    const float nscale = -scale;
#pragma unroll
    for (int j = 0; j < EPT; j++) {
      const float d = x[j] - m;
      const uint64_t f = d3s_fix40_exp(d); /* fix40(expf(x - m)), 0 for -inf */
      const int b = (int)fminf(d * nscale, (float)NBK);
      atomicAdd(&bstart[b], 1u);
      atomicAdd((unsigned long long *)&gsum[(uint32_t)b / PER], (unsigned long long)f);
    }
    __syncthreads(); /* the counts and sums in (the row sum S is their total) */
    const int id = topp_ids_fast<EPT, TBLOCK, NBK>(a, row, x, m, xmin, scale, rp.top_p, bstart, gsum, dyn, R, exact_grp);
    if (id >= 0) {
      if (tid == 0) a.ids[row] = id;
      return true;
    }
  }
  return false; /* TOPP_FULL, TOPP_RETRY, or scale 0 (a single finite x, or a row of equal ones) */
}

/* k_topp_ids: ids only, k = V; the ids-only path, the rows it leaves (the retry
 * or the full path) filed for k_topp_redo */
template <int EPT, bool BF16, int TBLOCK>
__global__ __launch_bounds__(TBLOCK) __attribute__((amdgpu_waves_per_eu(topp_ids_waves(EPT, TBLOCK)))) void k_topp_ids(
    D3S_HOT_PARAMS, SampleArgs a, ToppRedo rd) {
  D3S_HOT_APPLY(a);
  D3S_TOPP_SHARED
  __shared__ uint64_t gsum_s[TBLOCK + 2]; /* the group sums (entry TBLOCK: the -inf bucket's group) */
  const int row = (int)blockIdx.x;
  /* (FLAG_EXACT_LSE: every row straight to the exact retry) */
  const bool filed =
      (a.flags & FLAG_EXACT_LSE) != 0u ||
      !topp_ids_row<EPT, BF16, TBLOCK, NBK>(a, row, (char *)keys, bstart, gsum_s, R, false);
  if (filed && tid == 0) rd.rows[atomicAdd(rd.count, 1u)] = row;
}

/* k_topp_redo: each filed row again, the ids-only path's exact retry and, where
 * that leaves it, the full path (TOPP_REDO_WG workgroups take the rows in
 * turn; a few rows per launch, so registers are given room: the loop around
 * the row must not spill); the last workgroup to finish clears the counts.
 * No waiting: a workgroup that finds no row left ends.  LDS: the larger of
 * the two paths' arrays. */
template <int EPT, bool BF16, int TBLOCK>
__global__ __launch_bounds__(TBLOCK) __attribute__((amdgpu_waves_per_eu(2))) void k_topp_redo(
    uint32_t *hot_count, SampleArgs a, ToppRedo rd) {
  D3S_TOPP_SHARED
  __shared__ uint64_t gsum_s[TBLOCK + 2]; /* the group sums (entry TBLOCK: the -inf bucket's group) */
  /* rd.count again as a leading (preloaded) argument: the count's load
   * issues without waiting for the kernarg segment */
  rd.count = hot_count;
  const uint32_t n = __hip_atomic_load(rd.count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  /* every workgroup reads the same count (nothing changes it before the
   * last arrival below); none filed: the counts are zero already, and no
   * workgroup arrives */
  if (n == 0u) return;
#pragma unroll 1
  for (uint32_t i = blockIdx.x; i < n; i += gridDim.x) {
    const int row = rd.rows[i];
    __syncthreads(); /* the previous row's LDS reads done */
    /* (1024-thread workgroups: the full path alone; with the retry beside it
     * the loop would need scratch at four waves per SIMD) */
    if (TBLOCK > 512 || !topp_ids_row<EPT, BF16, TBLOCK, NBK>(a, row, (char *)keys, bstart, gsum_s, R, true)) {
      __syncthreads();
      topp_full_row<EPT, BF16, TBLOCK, NBK>(a, row, keys, bstart, R);
    }
  }
  __syncthreads();
  if (tid == 0) {
    const uint32_t old = __hip_atomic_fetch_add(rd.done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == gridDim.x - 1u) { /* every workgroup has read the count */
      __hip_atomic_store(rd.count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(rd.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

#undef D3S_TOPP_SHARED

/* the ids-only path takes calls with k = V and neither probabilities nor
 * candidates (with FLAG_EXACT_LSE, every row by its exact retry) */
bool topp_ids_call(const SampleArgs &a) { return !a.probs && !a.cand && a.k == a.vocab; }

template <int EPT, bool BF16, int TBLOCK>
bool try_topp(const SampleArgs &a, void *ws, size_t ws_bytes, hipStream_t s) {
  if (a.vocab > EPT * TBLOCK) return false;
  const size_t ranked = (size_t)a.vocab * sizeof(uint64_t); /* the full path's keys */
  /* (rows past 5120 elements: the redo kernel's loop would need scratch at
   * 1024 threads a workgroup, so those take the full path) */
  if constexpr (EPT * TBLOCK <= 5120) {
    if (topp_ids_call(a) && ws && ws_bytes >= topp_workspace_bytes(a)) {
      /* ids only, k = V (top-k disabled): the ids-only path with its own LDS,
       * then the full path for the rows it files */
      const size_t arrays = tf_bytes(TBLOCK, topp_buckets(EPT * TBLOCK, TBLOCK), a.vocab);
      ToppRedo rd;
      rd.count = (uint32_t *)ws;
      rd.done = (uint32_t *)((char *)ws + 128);
      rd.rows = (int32_t *)((char *)ws + split_counter_bytes());
      hipLaunchKernelGGL((k_topp_ids<EPT, BF16, TBLOCK>), dim3(a.n_rows), dim3(TBLOCK), arrays, s,
                         D3S_HOT_ARGS(a), a, rd);
      /* (every row filed under FLAG_EXACT_LSE: a workgroup each) */
      const int grid = a.n_rows < TOPP_REDO_WG || (a.flags & FLAG_EXACT_LSE) ? a.n_rows : TOPP_REDO_WG;
      hipLaunchKernelGGL((k_topp_redo<EPT, BF16, TBLOCK>), dim3(grid), dim3(TBLOCK), ranked > arrays ? ranked : arrays,
                         s, rd.count, a, rd);
      return true;
    }
  }
  hipLaunchKernelGGL((k_topp<EPT, BF16, TBLOCK>), dim3(a.n_rows), dim3(TBLOCK), ranked, s, a);
  return true;
}

}  // namespace

int topp_max_vocab() { return 8 * 1024; }

size_t topp_workspace_bytes(const SampleArgs &a) {
  return a.k > KF && a.vocab <= 5120 && topp_ids_call(a)
             ? split_counter_bytes() + (size_t)a.n_rows * sizeof(int32_t)
             : 0;
}

bool launch_topp(const SampleArgs &a, Dtype dt, void *ws, size_t ws_bytes, hipStream_t s) {
  if (a.k <= KF) return false;
  /* rows up to 4608 elements: 512 threads, three workgroups per CU (the
   * per-wave share of the reductions and the row's scalar arithmetic is
   * paid by 8 waves instead of 16); longer rows: 1024 threads */
  if (dt == DT_F32)
    return try_topp<9, false, 512>(a, ws, ws_bytes, s) || try_topp<5, false, 1024>(a, ws, ws_bytes, s) ||
           try_topp<8, false, 1024>(a, ws, ws_bytes, s);
  return try_topp<9, true, 512>(a, ws, ws_bytes, s) || try_topp<5, true, 1024>(a, ws, ws_bytes, s) ||
         try_topp<8, true, 1024>(a, ws, ws_bytes, s);
}

}  // namespace d3s
