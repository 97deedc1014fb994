/* The generic row procedure of the sampler (gfx950, wave64), shared by the
 * kernels: one 1024-thread workgroup samples one row, streaming it from
 * global memory for every pass (any V, k <= 16384): exact log-sum-exp
 * (src/sampling.c:81-89), an 8-bit radix select of the k-th rank over
 * order-preserving keys of x (:90-121), an LDS bitonic sort of the k selected,
 * then the reference kernel's tail (:123-139) or, in the op graph's order,
 * exact prefix sums over ranks (its cumsum and softmax, :39-44).
 * Device code only; every translation unit gets its own copy. */
#ifndef D3S_GENERIC_H
#define D3S_GENERIC_H

#include "d3s_device.h"

namespace d3s {
namespace {

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

/* exclusive block scan of per-thread counts in thread order (NW waves);
 * `tot` = total */
template <int NW>
__device__ __forceinline__ uint32_t block_excl_scan_u32(uint32_t v, uint32_t *sh, uint32_t &tot) {
  const int lane = lane_id(), wid = threadIdx.x / WAVE;
  const uint32_t incl = wave_scan_add_u32(v);
  if (lane == WAVE - 1) sh[wid] = incl;
  __syncthreads();
  uint32_t wbase = 0u, t = 0u;
  for (int w = 0; w < NW; w++) {
    const uint32_t x = sh[w];
    if (w < wid) wbase += x;
    t += x;
  }
  __syncthreads();
  tot = t;
  return wbase + incl - v;
}

/* the same for per-thread fixed-point sums below 2^45 (split in 24-bit parts) */
template <int NW>
__device__ __forceinline__ uint64_t block_excl_scan_u64(uint64_t v, uint32_t *sh_lo, uint32_t *sh_hi) {
  const int lane = lane_id(), wid = threadIdx.x / WAVE;
  const uint32_t lo = wave_scan_add_u32((uint32_t)(v & 0xffffffu));
  const uint32_t hi = wave_scan_add_u32((uint32_t)(v >> 24));
  if (lane == WAVE - 1) {
    sh_lo[wid] = lo;
    sh_hi[wid] = hi;
  }
  __syncthreads();
  uint64_t wbase = 0;
  for (int w = 0; w < wid; w++) wbase += ((uint64_t)sh_hi[w] << 24) + sh_lo[w];
  __syncthreads();
  return wbase + ((uint64_t)hi << 24) + lo - v;
}

__device__ __forceinline__ int wave_min_i32(int v) {
  const int big = 0x7fffffff;
  v = min(v, (int)dpp_u<DPP_SHR1, 0xf>((uint32_t)big, (uint32_t)v));
  v = min(v, (int)dpp_u<DPP_SHR2, 0xf>((uint32_t)big, (uint32_t)v));
  v = min(v, (int)dpp_u<DPP_SHR4, 0xf>((uint32_t)big, (uint32_t)v));
  v = min(v, (int)dpp_u<DPP_SHR8, 0xf>((uint32_t)big, (uint32_t)v));
  v = min(v, (int)dpp_u<DPP_BCAST15, 0xa>((uint32_t)big, (uint32_t)v));
  v = min(v, (int)dpp_u<DPP_BCAST31, 0xc>((uint32_t)big, (uint32_t)v));
  return (int)readlane_u((uint32_t)v, 63);
}

/* The op graph's order over the k ranked keys of glist (composite keys, rank
 * order; LDS or global memory): exact prefix sums of fix40(d3s_expf(x_r -
 * lse)) over ranks (its cumsum, rounded once, src/sampling.c:39-42), the cut
 * (the first r > 0 whose prefix exceeds top_p), the kept sum of
 * fix40(d3s_expf(x_r - x_0)), the probabilities and the race over every rank
 * (:43-48), each thread owning R consecutive ranks.  Every thread of the
 * BLOCK-thread workgroup calls it. */
template <int BLOCK>
__device__ __forceinline__ void generic_tail_opgraph(const SampleArgs &a, const int row, const float lse,
                                                     const float top_p, const uint64_t *glist) {
  constexpr int GBLOCK = BLOCK, GNW = BLOCK / WAVE;
  __shared__ uint32_t sh_u32[GNW], sh_lo[GNW], sh_hi[GNW];
  __shared__ float sh_best[GNW];
  __shared__ int sh_bestr[GNW];
  const int tid = threadIdx.x, lane = lane_id(), wid = tid / WAVE;
  const int k = a.k;
  const int R = (k + GBLOCK - 1) / GBLOCK;
  const int r0 = tid * R;
  const float v0 = key_x(glist[0]);
  uint64_t loc = 0;
  for (int q = 0; q < R; q++) {
    const int r = r0 + q;
    if (r < k) loc += d3s_fix40(d3s_expf(key_x(glist[r]) - lse));
  }
  uint64_t P = block_excl_scan_u64<GNW>(loc, sh_lo, sh_hi);
  int cut_local = k;
  for (int q = 0; q < R; q++) {
    const int r = r0 + q;
    if (r < k) {
      P += d3s_fix40(d3s_expf(key_x(glist[r]) - lse));
      if (r > 0 && cut_local == k && d3s_fixsum_to_f32(P) > top_p) cut_local = r;
    }
  }
  const int cm = wave_min_i32(cut_local);
  if (lane == 0) sh_u32[wid] = (uint32_t)cm;
  __syncthreads();
  int cut = k;
  for (int w = 0; w < GNW; w++) cut = min(cut, (int)sh_u32[w]);
  uint64_t ks = 0;
  for (int q = 0; q < R; q++) {
    const int r = r0 + q;
    if (r < k && r < cut) ks += d3s_fix40(d3s_expf(key_x(glist[r]) - v0));
  }
  {
    const uint64_t w = wave_sum_u64(ks);
    __syncthreads();
    if (lane == 0) {
      sh_lo[wid] = (uint32_t)w;
      sh_hi[wid] = (uint32_t)(w >> 32);
    }
  }
  __syncthreads();
  uint64_t KS = 0;
  for (int w = 0; w < GNW; w++) KS += ((uint64_t)sh_hi[w] << 32) | sh_lo[w];
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
  wave_argmax(bs, br);
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

/* Row `row` by the whole BLOCK-thread workgroup (BLOCK a multiple of 256);
 * glist: LDS for kpow >= k composite keys (kpow a power of two); src(i): the
 * row's logit i as fp32, -inf at the banned index.  Every thread of the
 * workgroup calls it and returns from it. */
template <int BLOCK, class Src>
__device__ __forceinline__ void generic_row_src(const SampleArgs &a, const int row, const int kpow,
                                                uint64_t *glist, Src &&src) {
  constexpr int GBLOCK = BLOCK, GNW = BLOCK / WAVE;
  __shared__ uint32_t hist[NB];
  __shared__ float sh_max[GNW];
  __shared__ uint32_t sh_flag[GNW], sh_u32[GNW], sh_lo[GNW], sh_hi[GNW];
  __shared__ int n_gather;
  __shared__ __align__(16) float wbuf[WAVE];

  const int tid = threadIdx.x, lane = lane_id(), wid = tid / WAVE;
  const int V = a.vocab, k = a.k;
  const RowP rp = row_params(a, row);
  const float T = rp.T;
  const bool t_finite = T < __builtin_inff();
  const float y = 1.0f / T;
  auto xat = [&](int i) { return scale_logit(src(i), T, y, t_finite); };

  /* ---- pass 1: max and classification */
  float xm = -__builtin_inff();
  uint32_t fl = 0;
  for (int i = tid; i < V; i += GBLOCK) {
    const float xi = xat(i);
    const uint32_t c = classify(xi);
    fl |= c;
    if (!(c & 1u)) xm = fmaxf(xm, xi);
  }
  xm = wave_max_f(xm);
  const uint32_t wf = (__ballot(fl & 1u) ? 1u : 0u) | (__ballot(fl & 2u) ? 2u : 0u);
  if (lane == 0) {
    sh_max[wid] = xm;
    sh_flag[wid] = wf;
  }
  if (tid == 0) n_gather = 0;
  __syncthreads();
  float M = sh_max[0];
  uint32_t F = sh_flag[0];
  for (int w = 1; w < GNW; w++) {
    M = fmaxf(M, sh_max[w]);
    F |= sh_flag[w];
  }
  if (F & 1u) {
    write_special(a, row, false);
    return;
  }
  if (M == -__builtin_inff()) {
    write_special(a, row, true);
    return;
  }

  /* ---- pass 2: exact log-sum-exp */
  uint64_t acc = 0;
  for (int i = tid; i < V; i += GBLOCK) acc += d3s_fix40(d3s_expf(xat(i) - M));
  {
    const uint64_t w = wave_sum_u64(acc);
    if (lane == 0) {
      sh_lo[wid] = (uint32_t)w;
      sh_hi[wid] = (uint32_t)(w >> 32);
    }
  }
  __syncthreads();
  uint64_t S = 0;
  for (int w = 0; w < GNW; w++) S += ((uint64_t)sh_hi[w] << 32) | sh_lo[w];
  const float lse = M + d3s_logf(d3s_fixsum_to_f32(S));

  /* ---- radix select of the k-th rank over order-preserving keys of x */
  uint32_t prefix = 0u, pmask = 0u, need = (uint32_t)k, done = 0u;
  for (int pass = 0; pass < 4 && !done; pass++) {
    const int shift = 24 - 8 * pass;
    __syncthreads();
    for (int i = tid; i < NB; i += GBLOCK) hist[i] = 0u;
    __syncthreads();
    for (int i = tid; i < V; i += GBLOCK) {
      const uint32_t key = d3s_ordkey(xat(i));
      if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    const BinSel b = wave_find_bin<false>(hist, need);
    prefix |= b.bin << shift;
    pmask |= 0xffu << shift;
    done = b.count == need - b.above;
    need -= b.above;
  }
  for (int i = tid; i < V; i += GBLOCK) {
    const float xi = xat(i);
    const uint32_t key = d3s_ordkey(xi) & pmask;
    if (key > prefix || (done && key == prefix)) {
      const int slot = atomicAdd(&n_gather, 1);
      if (slot < kpow) glist[slot] = composite_key(xi, i);
    }
  }
  if (!done) {
    /* exact ties: the lowest-index `need`, one block-wide tile at a time */
    uint32_t base = 0u;
    for (int t0 = 0; t0 < V && base < need; t0 += GBLOCK) {
      const int i = t0 + tid;
      float xi = 0.0f;
      uint32_t tie = 0u;
      if (i < V) {
        xi = xat(i);
        tie = d3s_ordkey(xi) == prefix;
      }
      uint32_t tot;
      const uint32_t ord = base + block_excl_scan_u32<GNW>(tie, sh_u32, tot);
      if (tie && ord < need) {
        const int slot = atomicAdd(&n_gather, 1);
        if (slot < kpow) glist[slot] = composite_key(xi, i);
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
  if (!a.opgraph) { /* the reference kernel's order (k <= 64 then) */
    if (wid == 0) {
      const uint64_t key = lane < k ? glist[lane] : 0ull;
      const float v = key_x(key);
      const int idx = key_idx(key);
      const float uval = lane < k ? a.u[(size_t)row * k + lane] : 0.0f;
      const float c = wave_seq_cumsum(lane < k ? d3s_expf(v - lse) : 0.0f, k, wbuf);
      wave_tail_finish(a, row, v, idx, c, -d3s_logf(1.0f - uval), top_p, wbuf);
    }
    return;
  }

  generic_tail_opgraph<BLOCK>(a, row, lse, top_p, glist);
}

/* generic_row_src over row `row` of a.logits */
template <bool BF16, int BLOCK = GBLOCK>
__device__ __forceinline__ void generic_row(const SampleArgs &a, const int row, const int kpow,
                                            uint64_t *glist) {
  const int banned = row_params(a, row).banned;
  const char *rowp = (const char *)a.logits + (size_t)row * (size_t)a.row_stride * (BF16 ? 2 : 4);
  generic_row_src<BLOCK>(a, row, kpow, glist, [&](int i) { return load_logit<BF16>(rowp, i, banned); });
}

}  // namespace
}  // namespace d3s

#endif
