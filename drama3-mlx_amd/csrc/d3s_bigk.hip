/* The sorting path: the op graph's sampler for k beyond the generic
 * kernel's LDS sort (k > 16384, on rows longer than the nucleus kernel
 * takes), gfx950 wave64.
 *
 * The reference's op graph (src/sampling.c:22-49) takes any k up to V: with
 * top-k disabled it argsorts the whole row (:33-35).  Each row is cut into
 * up to 16 segments of whole 1024-key tiles, so a launch of few rows still
 * spreads over the CUs; six launches, 1024 threads a workgroup:
 *  k_bk_keys (a workgroup per segment): x = L / T, classification and the
 *     segment's max; the composite keys (ordkey(x), ~index) written to the
 *     workspace in index order, with the segment's digit counts for the first
 *     radix pass;
 *  k_bk_pass, four times (a workgroup per segment): one pass of a stable LSD
 *     radix sort by ordkey(x) descending (8-bit digits, between two buffers).
 *     The segment's first place for digit d is the row's keys of smaller
 *     digits plus the earlier segments' keys of digit d (every segment's
 *     counts, from the pass before); within the segment, tiles of 1024 keys
 *     in order: a wave's peers of a digit by eight ballots, per-wave digit
 *     counts in LDS turned into places by one thread per digit, two barriers
 *     a tile (ordering LDS only; each tile's keys load during the tile
 *     before).  Each key's place gives the segment it lands in for the next
 *     pass: the next pass's counts per (segment, digit), gathered in LDS and
 *     added to the workspace's table once per workgroup.  A row whose x all
 *     have zero low 16 bits (bf16 logits at T = 1) skips the first two passes
 *     (bk_row_max says why that is exact).  The row's first pass also takes
 *     the segment's exact sum (2^-40 fixed point of d3s_expf(x - m), m the
 *     row's max from every segment's).  Stability keeps equal x in index
 *     order, so the result is the order (x desc, index asc) of every kernel;
 *  the tail, over the first k ranks cut into the same segments (k_bk_sums,
 *     k_bk_cut, k_bk_race, k_bk_pick below): refused and all -inf rows as
 *     every kernel treats them; else the generic kernel's definition: the
 *     exact prefix sums to the cut, the kept sum, probabilities and the race.
 * The same definition as the generic and nucleus kernels, bit for bit.  The
 * workspace holds, per row, two buffers of the row's keys (16 bytes per
 * element), the passes' count tables and the segments' records. */
#include "d3s_generic.h"

#pragma clang fp contract(off)

namespace d3s {
namespace {

constexpr int BK_T = 1024;
constexpr int BK_NW = BK_T / WAVE;

/* a workgroup barrier that orders LDS only: global loads and stores stay in
 * flight across it (a pass's global writes are ordered before the next pass
 * by the launch boundary between them) */
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

/* the sort digit of a composite key in a pass: byte `pass` of ~ordkey(x)
 * (ascending ~ordkey is descending x) */
__device__ __forceinline__ uint32_t bk_digit(uint64_t key, int pass) {
  return (uint32_t)((~key) >> (32 + 8 * pass)) & 0xffu;
}

/* the wave's lanes whose d has the same low `bits` bits as this lane's
 * (among the lanes in `live`), by one ballot per bit */
template <int BITS>
__device__ __forceinline__ uint64_t wave_peers(uint32_t d, uint64_t live) {
  uint64_t peers = live;
#pragma unroll
  for (int b = 0; b < BITS; b++) {
    const uint64_t bb = __ballot((d >> b) & 1u);
    peers &= ((d >> b) & 1u) ? bb : ~bb;
  }
  return peers;
}

__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int l) {
  return ((uint64_t)readlane_u((uint32_t)(v >> 32), l) << 32) | readlane_u((uint32_t)v, l);
}

/* sum over the wave of per-lane 64-bit values, exact modulo 2^64 (three
 * 24-bit parts, each summed in 32 bits): a thread's partial sum over a long
 * segment of terms near 2^40 can pass the shared wave sum's 2^45 */
__device__ __forceinline__ uint64_t bk_wave_sum(uint64_t v) {
  const uint32_t p0 = wave_sum_u32((uint32_t)(v & 0xffffffu));
  const uint32_t p1 = wave_sum_u32((uint32_t)((v >> 24) & 0xffffffu));
  const uint32_t p2 = wave_sum_u32((uint32_t)(v >> 48));
  return (uint64_t)p0 + ((uint64_t)p1 << 24) + ((uint64_t)p2 << 48);
}

/* inclusive prefix sum over the wave of per-lane 64-bit values, exact
 * modulo 2^64 (three 24-bit parts) */
__device__ __forceinline__ uint64_t bk_wave_scan(uint64_t v) {
  const uint32_t p0 = wave_scan_add_u32((uint32_t)(v & 0xffffffu));
  const uint32_t p1 = wave_scan_add_u32((uint32_t)((v >> 24) & 0xffffffu));
  const uint32_t p2 = wave_scan_add_u32((uint32_t)(v >> 48));
  return (uint64_t)p0 + ((uint64_t)p1 << 24) + ((uint64_t)p2 << 48);
}

/* block sum of per-thread fixed-point values, exact modulo 2^64 (the
 * oracle's integer sums); opens with a barrier (the scratch may still be
 * being read) */
__device__ __forceinline__ uint64_t bk_block_sum(uint64_t v, uint32_t *lo, uint32_t *hi) {
  const uint64_t w = bk_wave_sum(v);
  __syncthreads();
  if (lane_id() == 0) {
    lo[threadIdx.x / WAVE] = (uint32_t)w;
    hi[threadIdx.x / WAVE] = (uint32_t)(w >> 32);
  }
  __syncthreads();
  uint64_t t = 0;
#pragma unroll
  for (int w2 = 0; w2 < BK_NW; w2++) t += ((uint64_t)hi[w2] << 32) | lo[w2];
  return t;
}

constexpr int BK_SMAX = 16; /* segments per row (at most) */
constexpr int BK_B = 8;     /* loads a thread keeps in flight in the streaming loops */
constexpr int BK_PF = 4;    /* tiles of keys a pass keeps in flight (even) */
constexpr int BK_WGS = 512; /* workgroups a launch aims at: two per CU */

/* a segment's record: its max and refusal flag (k_bk_keys), its exact sum
 * (the row's first pass); then, for the segment's ranks [s L, s L + L) after the
 * sort, the sums of their terms fix40(d3s_expf(x_r - lse)) and
 * fix40(d3s_expf(x_r - x_0)) (k_bk_sums) and their race's first maximum
 * (k_bk_race); segment 0's record also holds the row's cut and 1 / kept sum
 * (k_bk_cut) */
struct __align__(16) BkMeta {
  float max;
  uint32_t flags;
  uint64_t sum;
  uint32_t kor, kand; /* OR and AND of the segment's digit words (k_bk_keys) */
  uint32_t klow;      /* OR of the low 16 bits of its x (k_bk_keys) */
  uint64_t psum, ksum;
  float best;
  int bestr;
  int cut;
  float inv;
};

/* a launch's rows in the workspace (the tile sums after the records): the rows' key buffers, their count
 * tables ([row][pass][segment][digit]: filled by the pass before each), the
 * segments' counts of digits 0 and 2 in index order ([row][2][segment][digit]:
 * the first pass's, k_bk_keys'), then their segments' records */
struct BkLayout {
  uint64_t *keys; /* [n][2][vstride] */
  uint32_t *hist; /* [n][4][BK_SMAX][NB] */
  uint32_t *hidx; /* [n][2][BK_SMAX][NB] */
  BkMeta *meta;   /* [n][BK_SMAX] */
  uint64_t *tsum; /* [n][ntiles][2]: each tile's exact prefix and kept-sum terms' sums (k_bk_sums) */
  int ntiles;     /* tiles of BK_T ranks a row */
  int64_t vstride;
  int nseg, tps;  /* segments per row, tiles per segment */
  int pass0;      /* the first pass launched: 2 when every row's x is known to
                     have zero low 16 bits (bf16 logits at a scalar T of 1),
                     else 0 */
  float inv_sl;   /* 1 / (tps BK_T), rounded */
};

/* the segment holding position pos: pos / (tps BK_T), from a float
 * estimate within one of it (pos < 2^26 and the segment length are exact
 * in fp32; the product's relative error is below 2^-23) */
__device__ __forceinline__ uint32_t bk_seg_of(uint32_t pos, const BkLayout &L) {
  const uint32_t sl = (uint32_t)(L.tps * BK_T);
  uint32_t q = (uint32_t)((float)pos * L.inv_sl);
  q = q * sl > pos ? q - 1u : q;
  q = (q + 1u) * sl <= pos ? q + 1u : q;
  return q;
}

/* the row's max and refusal flag from its segments' records (every wave
 * alike: lane s reads segment s, all in one round of loads); with S, also
 * the row's exact sum (the first pass's); with fp, the first radix pass the
 * row runs: 4 when every key's x is the same (no pass reorders anything:
 * the keys stay in index order), 2 when every x has its low 16 bits zero
 * (bf16 logits at T = 1), else 0.  In the second case digits 0 and 1 are
 * 0x0000 or 0xffff by x's sign, which digit 3 holds: keys equal in digits 2
 * and 3 are equal in x, so passes 2 and 3 alone, from index order, give the
 * same stable order as all four.  Skipping two keeps the result in the
 * first buffer. */
__device__ __forceinline__ void bk_row_max(const BkLayout &L, int row, float &M, uint32_t &F, uint64_t *S = nullptr,
                                           int *fp = nullptr) {
  const int lane = lane_id();
  const BkMeta *mt = L.meta + (size_t)row * BK_SMAX;
  float m = -__builtin_inff();
  uint32_t f = 0u, o = 0u, n = ~0u, lw = 0u;
  uint64_t sm = 0ull;
  if (lane < L.nseg) {
    m = mt[lane].max;
    f = mt[lane].flags;
    if (S) sm = mt[lane].sum;
    if (fp) {
      o = mt[lane].kor;
      n = mt[lane].kand;
      lw = mt[lane].klow;
    }
  }
  M = wave_max_f(m);
  F = __ballot(f & 1u) ? 1u : 0u;
  if (S) {
    uint64_t t = 0ull;
    for (int s2 = 0; s2 < L.nseg; s2++) t += readlane_u64(sm, s2);
    *S = t;
  }
  if (fp) {
    uint32_t ro = 0u, rn = ~0u;
    for (int s2 = 0; s2 < L.nseg; s2++) {
      ro |= readlane_u(o, s2);
      rn &= readlane_u(n, s2);
    }
    *fp = ro == rn ? 4 : (__ballot(lw != 0u) == 0ull ? 2 : 0);
  }
}

/* k_bk_keys: a segment's keys in index order, its max and flags, its counts
 * of digits 0 and 2 in index order (the first pass's, whichever it is) and
 * the OR and AND of its digit words; the later passes' counts of the
 * segment zeroed (they are added to by the pass before each) */
template <bool BF16>
__global__ __launch_bounds__(BK_T) void k_bk_keys(SampleArgs a, BkLayout L) {
  __shared__ uint32_t hist[2][NB];
  __shared__ float sh_max[BK_NW];
  __shared__ uint32_t sh_flag[BK_NW], sh_or[BK_NW], sh_and[BK_NW], sh_low[BK_NW];
  const int seg = (int)blockIdx.x, row = (int)blockIdx.y;
  const int tid = (int)threadIdx.x, lane = lane_id(), wid = tid / WAVE;
  const int V = a.vocab;
  const int lo = seg * L.tps * BK_T, hi = min(V, lo + L.tps * BK_T);
  const RowP rp = row_params(a, row);
  const float T = rp.T;
  const bool t_finite = T < __builtin_inff();
  const float y = 1.0f / T;
  const char *rowp = (const char *)a.logits + (size_t)row * (size_t)a.row_stride * (BF16 ? 2 : 4);
  uint64_t *buf0 = L.keys + (size_t)row * 2 * (size_t)L.vstride;
  if (tid < 2 * NB) (&hist[0][0])[tid] = 0u;
  __syncthreads();
  float xm = -__builtin_inff();
  uint32_t fl = 0u, wo = 0u, wn = ~0u, wl = 0u;
#pragma unroll 1
  for (int i0 = lo + tid; i0 < hi; i0 += BK_B * BK_T) { /* BK_B loads in flight, then their work */
    float v[BK_B];
#pragma unroll
    for (int q = 0; q < BK_B; q++) {
      const int i = i0 + q * BK_T;
      v[q] = i < hi ? load_logit<BF16>(rowp, i, rp.banned) : 0.0f;
    }
#pragma unroll
    for (int q = 0; q < BK_B; q++) {
      const int i = i0 + q * BK_T;
      if (i < hi) {
        const float xi = scale_logit(v[q], T, y, t_finite);
        const uint32_t c = classify(xi);
        fl |= c;
        if (!(c & 1u)) xm = fmaxf(xm, xi);
        const uint64_t key = composite_key(xi, i);
        buf0[i] = key;
        /* (with pass 0 not launched its counts are not read; its digit is
         * then one of two values by the sign: 1024 atomics on two words) */
        if (L.pass0 == 0) atomicAdd(&hist[0][bk_digit(key, 0)], 1u);
        atomicAdd(&hist[1][bk_digit(key, 2)], 1u);
        const uint32_t dw = (uint32_t)((~key) >> 32); /* the digit word */
        wo |= dw;
        wn &= dw;
        wl |= d3s_f2u(xi) & 0xffffu;
      }
    }
  }
  xm = wave_max_f(xm);
  const uint32_t wf = __ballot(fl & 1u) ? 1u : 0u;
#pragma unroll
  for (int sh = 1; sh < WAVE; sh <<= 1) {
    wo |= (uint32_t)__shfl_xor((int)wo, sh);
    wn &= (uint32_t)__shfl_xor((int)wn, sh);
    wl |= (uint32_t)__shfl_xor((int)wl, sh);
  }
  if (lane == 0) {
    sh_max[wid] = xm;
    sh_flag[wid] = wf;
    sh_or[wid] = wo;
    sh_and[wid] = wn;
    sh_low[wid] = wl;
  }
  __syncthreads();
  uint32_t *gh = L.hist + (size_t)row * 4 * BK_SMAX * NB;
  uint32_t *hx = L.hidx + (size_t)row * 2 * BK_SMAX * NB;
  if (tid < NB) {
    hx[seg * NB + tid] = hist[0][tid];
    hx[(BK_SMAX + seg) * NB + tid] = hist[1][tid];
#pragma unroll
    for (int p = 1; p < 4; p++) gh[(p * BK_SMAX + seg) * NB + tid] = 0u;
  }
  if (tid == 0) {
    float M = sh_max[0];
    uint32_t F = sh_flag[0], O = sh_or[0], N = sh_and[0], W = sh_low[0];
    for (int w = 1; w < BK_NW; w++) {
      M = fmaxf(M, sh_max[w]);
      F |= sh_flag[w];
      O |= sh_or[w];
      N &= sh_and[w];
      W |= sh_low[w];
    }
    BkMeta m;
    m.max = M;
    m.flags = F;
    m.sum = 0ull;
    m.kor = O;
    m.kand = N;
    m.klow = W;
    L.meta[(size_t)row * BK_SMAX + seg] = m;
  }
}

/* k_bk_pass: one radix pass of a segment (the layout above); refused and all
 * -inf rows are left to the tail */
__global__ __launch_bounds__(BK_T) void k_bk_pass(SampleArgs a, BkLayout L, int pass) {
  __shared__ uint32_t base[NB];            /* a digit's next place */
  __shared__ uint32_t tot[NB];             /* the row's keys of each digit */
  __shared__ uint32_t wcnt[2][BK_NW][NB];  /* a tile's count of each digit in each wave, then its place */
  __shared__ uint32_t nxt[BK_SMAX * NB];   /* the next pass's counts by (segment, digit) */
  __shared__ uint32_t sh_lo[BK_NW], sh_hi[BK_NW];
  const int seg = (int)blockIdx.x, row = (int)blockIdx.y;
  const int tid = (int)threadIdx.x, lane = lane_id(), wid = tid / WAVE;
  const int V = a.vocab;
  const int lo = seg * L.tps * BK_T, hi = min(V, lo + L.tps * BK_T);
  float M;
  uint32_t F;
  int fp;
  bk_row_max(L, row, M, F, nullptr, &fp);
  if ((F & 1u) || M == -__builtin_inff()) return; /* (every workgroup of the row alike) */
  uint64_t *buf = L.keys + (size_t)row * 2 * (size_t)L.vstride;
  if (pass < fp) { /* a pass the row skips; with no pass to run, the first launched takes the sum */
    if (fp == 4 && pass == L.pass0) {
      uint64_t acc = 0ull;
#pragma unroll 1
      for (int r0 = lo + tid; r0 < hi; r0 += BK_B * BK_T) {
        uint64_t kv[BK_B];
#pragma unroll
        for (int q = 0; q < BK_B; q++) kv[q] = r0 + q * BK_T < hi ? buf[r0 + q * BK_T] : 0ull;
#pragma unroll
        for (int q = 0; q < BK_B; q++)
          if (r0 + q * BK_T < hi) acc += d3s_fix40_exp(key_x(kv[q]) - M); /* (x <= m) */
      }
      const uint64_t S = bk_block_sum(acc, sh_lo, sh_hi);
      if (tid == 0) L.meta[(size_t)row * BK_SMAX + seg].sum = S;
    }
    return;
  }
  const int e = pass - fp; /* the passes run before this one */
  const uint64_t *src = buf + (e & 1) * L.vstride;
  uint64_t *dst = buf + ((e & 1) ^ 1) * L.vstride;
  uint32_t *gh = L.hist + (size_t)row * 4 * BK_SMAX * NB;
  /* the segments' counts: the index order's for the row's first pass, else
   * the pass before's */
  const uint32_t *cnt = pass == fp ? L.hidx + (size_t)row * 2 * BK_SMAX * NB + (fp == 2 ? BK_SMAX * NB : 0)
                                   : gh + (size_t)pass * BK_SMAX * NB;

  /* the segment's first place of each digit: the row's keys of smaller
   * digits plus the earlier segments' of this digit */
  if (tid < NB) {
    uint32_t c[BK_SMAX];
#pragma unroll
    for (int s2 = 0; s2 < BK_SMAX; s2++) c[s2] = s2 < L.nseg ? cnt[s2 * NB + tid] : 0u; /* one round of loads */
    uint32_t t = 0u, pre = 0u;
#pragma unroll
    for (int s2 = 0; s2 < BK_SMAX; s2++) {
      pre += s2 < seg ? c[s2] : 0u;
      t += c[s2];
    }
    tot[tid] = t;
    base[tid] = pre;
  }
  for (int j = tid; j < 2 * BK_NW * NB; j += BK_T) (&wcnt[0][0][0])[j] = 0u;
  if (pass < 3)
    for (int j = tid; j < L.nseg * NB; j += BK_T) nxt[j] = 0u;
  __syncthreads();
  if (wid == 0) { /* the digits' starts, four per lane */
    uint32_t h[4];
#pragma unroll
    for (int q = 0; q < 4; q++) h[q] = tot[4 * lane + q];
    const uint32_t ls = h[0] + h[1] + h[2] + h[3];
    uint32_t run = wave_scan_add_u32(ls) - ls;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      base[4 * lane + q] += run;
      run += h[q];
    }
  }
  __syncthreads();

  /* the segment's tiles in order: two count buffers alternate between
   * tiles, each cleared a tile after its last read; each thread's keys of
   * the next BK_PF tiles in flight (a workgroup keeps BK_PF tiles of reads
   * outstanding: the pass is bound by that latency, not by its work) */
  const uint64_t lt = (1ull << lane) - 1ull;
  uint64_t acc = 0ull; /* the row's first pass: the segment's exact sum */
  uint64_t pf[BK_PF];
#pragma unroll
  for (int q = 0; q < BK_PF; q++) pf[q] = lo + q * BK_T + tid < hi ? src[lo + q * BK_T + tid] : 0ull;
#pragma unroll 1
  for (int g0 = lo; g0 < hi; g0 += BK_PF * BK_T) {
#pragma unroll
    for (int q = 0; q < BK_PF; q++) {
      const int t0 = g0 + q * BK_T;
      if (t0 >= hi) break; /* (uniform) */
      const int par = q & 1; /* (BK_PF even: tiles alternate) */
      const int i = t0 + tid;
      const bool valid = i < hi;
      const uint64_t key = pf[q];
      const int ip = i + BK_PF * BK_T;
      pf[q] = ip < hi ? src[ip] : 0ull;
      const uint64_t live = __ballot(valid);
      const uint32_t d = bk_digit(key, pass);
      const uint64_t peers = wave_peers<8>(d, live);
      const uint32_t below = (uint32_t)__popcll(peers & lt);
      if (valid && below == 0u) wcnt[par][wid][d] = (uint32_t)__popcll(peers);
      if (pass == fp && valid) acc += d3s_fix40_exp(key_x(key) - M); /* (the row's first pass; x <= m) */
      lds_barrier();
      if (tid < NB) {
        uint32_t run = base[tid];
#pragma unroll
        for (int w = 0; w < BK_NW; w++) {
          const uint32_t c = wcnt[par][w][tid];
          wcnt[par][w][tid] = run;
          wcnt[par ^ 1][w][tid] = 0u; /* last read a tile ago */
          run += c;
        }
        base[tid] = run;
      }
      lds_barrier();
      if (valid) {
        const uint32_t pos = wcnt[par][wid][d] + below;
        dst[pos] = key;
        if (pass < 3) { /* the segment the key lands in, for the next pass */
          const uint32_t ds = bk_seg_of(pos, L);
          atomicAdd(&nxt[ds * NB + bk_digit(key, pass + 1)], 1u);
        }
      }
    }
  }
  __syncthreads();
  if (pass < 3) {
    uint32_t *gn = gh + (size_t)(pass + 1) * BK_SMAX * NB;
    for (int j = tid; j < L.nseg * NB; j += BK_T) {
      const uint32_t c = nxt[j];
      if (c) atomicAdd(&gn[j], c);
    }
  }
  if (pass == fp) {
    const uint64_t S = bk_block_sum(acc, sh_lo, sh_hi);
    if (tid == 0) L.meta[(size_t)row * BK_SMAX + seg].sum = S;
  }
}

/* the row's lse (and the refusal or all -inf decision) from its segments'
 * records; false for a row the tail leaves to k_bk_cut's special result */
__device__ __forceinline__ bool bk_row_lse(const BkLayout &L, int row, float &lse) {
  float M;
  uint32_t F;
  uint64_t S;
  bk_row_max(L, row, M, F, &S);
  if ((F & 1u) || M == -__builtin_inff()) return false;
  lse = M + d3s_logf(d3s_fixsum_to_f32(S));
  return true;
}

/* The op graph's tail (generic_tail_opgraph's definition, bit for bit) over
 * the first k ranks, the ranks cut into the sort's segments:
 *  k_bk_sums (a workgroup per segment): the segment's sums of the exact
 *    prefix terms fix40(d3s_expf(x_r - lse)) and of the kept-sum terms
 *    fix40(d3s_expf(x_r - x_0)) (integers: any order);
 *  k_bk_cut (a workgroup per row): the cut, the first r > 0 whose exact
 *    prefix passes top_p: the first segment whose end passes it, then that
 *    segment chunk by chunk and the passing chunk rank by rank; the kept sum
 *    (the earlier segments' sums plus the cut segment's ranks below the cut);
 *  k_bk_race (a workgroup per segment): probabilities, candidates and each
 *    segment's race (the first maximum: the largest score, ties to the
 *    smaller rank);
 *  k_bk_pick (a wave per row): the segments' maxima, the first one. */
__global__ __launch_bounds__(BK_T) void k_bk_sums(SampleArgs a, BkLayout L) {
  __shared__ uint32_t sh_lo[BK_NW], sh_hi[BK_NW];
  const int seg = (int)blockIdx.x, row = (int)blockIdx.y, tid = (int)threadIdx.x;
  const int lane = lane_id(), wid = tid / WAVE;
  float lse;
  if (!bk_row_lse(L, row, lse)) return;
  const uint64_t *glist = L.keys + (size_t)row * 2 * (size_t)L.vstride;
  uint64_t *ts = L.tsum + (size_t)row * 2 * (size_t)L.ntiles;
  const float v0 = key_x(glist[0]);
  const int lo = seg * L.tps * BK_T, hi = min(a.k, lo + L.tps * BK_T);
  /* wave w: the segment's tiles w, w + 16, ...; lane l the tile's ranks
   * l + 64 q; each tile's two sums filed, the wave's totals kept */
  uint64_t wp = 0ull, wk = 0ull;
  for (int t = lo / BK_T + wid; t * BK_T < hi; t += BK_NW) {
    const int r0 = t * BK_T + lane;
    uint64_t kv[BK_T / WAVE];
#pragma unroll
    for (int q = 0; q < BK_T / WAVE; q++) kv[q] = r0 + q * WAVE < hi ? glist[r0 + q * WAVE] : 0ull;
    uint64_t ps = 0ull, ks = 0ull;
#pragma unroll
    for (int q = 0; q < BK_T / WAVE; q++)
      if (r0 + q * WAVE < hi) {
        const float x = key_x(kv[q]);
        ps += d3s_fix40_exp(x - lse); /* (x <= x_0 <= lse) */
        ks += d3s_fix40_exp(x - v0);
      }
    ps = bk_wave_sum(ps);
    ks = bk_wave_sum(ks);
    if (lane == 0) {
      ts[2 * t] = ps;
      ts[2 * t + 1] = ks;
    }
    wp += ps;
    wk += ks;
  }
  const uint64_t sp = bk_block_sum(lane == 0 ? wp : 0ull, sh_lo, sh_hi);
  const uint64_t sk = bk_block_sum(lane == 0 ? wk : 0ull, sh_lo, sh_hi);
  if (tid == 0) {
    L.meta[(size_t)row * BK_SMAX + seg].psum = sp;
    L.meta[(size_t)row * BK_SMAX + seg].ksum = sk;
  }
}

__global__ __launch_bounds__(BK_T) void k_bk_cut(SampleArgs a, BkLayout L) {
  __shared__ uint32_t sh_lo[BK_NW], sh_hi[BK_NW], sh_u32[BK_NW];
  __shared__ uint64_t sh_pk[2];
  const int row = (int)blockIdx.x, tid = (int)threadIdx.x, lane = lane_id(), wid = tid / WAVE;
  const int k = a.k;
  float lse;
  if (!bk_row_lse(L, row, lse)) {
    float M;
    uint32_t F;
    bk_row_max(L, row, M, F);
    write_special(a, row, !(F & 1u));
    return;
  }
  const RowP rp = row_params(a, row);
  const float top_p = rp.top_p;
  const uint64_t *glist = L.keys + (size_t)row * 2 * (size_t)L.vstride;
  BkMeta *mt = L.meta + (size_t)row * BK_SMAX;
  const float v0 = key_x(glist[0]);
  const int SL = L.tps * BK_T;
  const int nrs = (k + SL - 1) / SL; /* segments holding ranks below k */
  /* the first segment whose end passes top_p (its prefix before: base);
   * lane s holds segment s's sums */
  uint64_t lp = 0ull, lk = 0ull;
  if (lane < nrs) {
    lp = mt[lane].psum;
    lk = mt[lane].ksum;
  }
  uint64_t base = 0ull, kept = 0ull;
  int c = nrs;
  for (int s2 = 0; s2 < nrs; s2++) {
    const uint64_t P = base + readlane_u64(lp, s2);
    if (d3s_fixsum_to_f32(P) > top_p) {
      c = s2;
      break;
    }
    base = P;
    kept += readlane_u64(lk, s2);
  }
  int cut = k;
  if (c < nrs) {
    /* the cut lies in segment c: wave 0 finds the first of its tiles whose
     * end passes top_p (with the prefix and the kept sum before it) from
     * the tile sums; then that tile rank by rank, one rank a thread (a pass
     * at rank 0 alone is no cut: the tile's later ranks pass too, and the
     * first of them is) */
    const int lo = c * SL, hi = min(k, lo + SL);
    const uint64_t *ts = L.tsum + (size_t)row * 2 * (size_t)L.ntiles;
    if (wid == 0) {
      const int t_hi = (hi + BK_T - 1) / BK_T;
      int ct = t_hi - 1;
      uint64_t b = base, kk = kept;
      for (int t0 = lo / BK_T; t0 < t_hi; t0 += WAVE) {
        const int t = t0 + lane;
        const uint64_t pt = t < t_hi ? ts[2 * t] : 0ull, kt = t < t_hi ? ts[2 * t + 1] : 0ull;
        const uint64_t pin = bk_wave_scan(pt), kin = bk_wave_scan(kt);
        const uint64_t m = __ballot(t < t_hi && d3s_fixsum_to_f32(b + pin) > top_p);
        if (m) {
          const int j = (int)__builtin_ctzll(m);
          ct = t0 + j;
          b += readlane_u64(pin - pt, j);
          kk += readlane_u64(kin - kt, j);
          break;
        }
        b += readlane_u64(pin, WAVE - 1);
        kk += readlane_u64(kin, WAVE - 1);
      }
      if (lane == 0) {
        sh_u32[0] = (uint32_t)ct;
        sh_pk[0] = b;
        sh_pk[1] = kk;
      }
    }
    __syncthreads();
    const int ct = (int)sh_u32[0];
    base = sh_pk[0];
    kept = sh_pk[1];
    const int r = ct * BK_T + tid;
    const bool in = r < hi;
    const float x = in ? key_x(glist[r]) : 0.0f;
    const uint64_t f = in ? d3s_fix40_exp(x - lse) : 0ull;
    const uint64_t P = base + block_excl_scan_u64<BK_NW>(f, sh_lo, sh_hi) + f;
    const int cm = wave_min_i32(in && r > 0 && d3s_fixsum_to_f32(P) > top_p ? r : k);
    __syncthreads(); /* (sh_u32 read above) */
    if (lane == 0) sh_u32[wid] = (uint32_t)cm;
    __syncthreads();
    for (int w = 0; w < BK_NW; w++) cut = min(cut, (int)sh_u32[w]);
    /* the kept sum: what came before the tile and its ranks below the cut */
    kept += bk_block_sum(in && r < cut ? d3s_fix40_exp(x - v0) : 0ull, sh_lo, sh_hi);
  }
  if (tid == 0) {
    mt[0].cut = cut;
    mt[0].inv = 1.0f / d3s_fixsum_to_f32(kept);
  }
}

__global__ __launch_bounds__(BK_T) void k_bk_race(SampleArgs a, BkLayout L) {
  __shared__ float sh_best[BK_NW];
  __shared__ int sh_bestr[BK_NW];
  const int seg = (int)blockIdx.x, row = (int)blockIdx.y;
  const int tid = (int)threadIdx.x, lane = lane_id(), wid = tid / WAVE;
  const int k = a.k;
  float lse;
  if (!bk_row_lse(L, row, lse)) return;
  const uint64_t *glist = L.keys + (size_t)row * 2 * (size_t)L.vstride;
  BkMeta *mt = L.meta + (size_t)row * BK_SMAX;
  const int lo = seg * L.tps * BK_T, hi = min(k, lo + L.tps * BK_T);
  if (lo >= hi) return;
  const int cut = mt[0].cut;
  const float inv = mt[0].inv;
  const float v0 = key_x(glist[0]);
  float bs = -1.0f;
  int br = 0x7fffffff;
  const float *urow = a.u + (size_t)row * k;
#pragma unroll 1
  for (int r0 = lo + tid; r0 < hi; r0 += BK_B * BK_T) {
    uint64_t kv[BK_B];
    float uu[BK_B];
#pragma unroll
    for (int q = 0; q < BK_B; q++) {
      const int r = r0 + q * BK_T;
      kv[q] = r < hi ? glist[r] : 0ull;
      uu[q] = r < hi ? urow[r] : 0.0f;
    }
#pragma unroll
    for (int q = 0; q < BK_B; q++) {
      const int r = r0 + q * BK_T;
      if (r < hi) {
        const uint64_t key = kv[q];
        const float p = r < cut ? d3s_expf_nonpos(key_x(key) - v0) * inv : 0.0f;
        const float noise = -d3s_logf(1.0f - uu[q]);
        const float score = p / noise;
        const float sc = score > -1.0f ? score : -1.0f;
        if (sc > bs || br == 0x7fffffff) { /* this thread's ranks increase: its first maximum */
          bs = sc;
          br = r;
        }
        if (a.probs) a.probs[(size_t)row * k + r] = p;
        if (a.cand) a.cand[(size_t)row * k + r] = key_idx(key);
      }
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
    for (int w = 1; w < BK_NW; w++)
      if (sh_best[w] > b || (sh_best[w] == b && sh_bestr[w] < r)) {
        b = sh_best[w];
        r = sh_bestr[w];
      }
    mt[seg].best = b;
    mt[seg].bestr = r;
  }
}

__global__ __launch_bounds__(WAVE) void k_bk_pick(SampleArgs a, BkLayout L) {
  const int row = (int)blockIdx.x, lane = lane_id();
  float lse;
  if (!bk_row_lse(L, row, lse)) return;
  const BkMeta *mt = L.meta + (size_t)row * BK_SMAX;
  const int SL = L.tps * BK_T;
  const int nrs = (a.k + SL - 1) / SL;
  float b = -2.0f;
  int r = 0x7fffffff;
  if (lane < nrs) {
    b = mt[lane].best;
    r = mt[lane].bestr;
  }
  wave_argmax(b, r);
  if (lane == 0) a.ids[row] = key_idx(L.keys[(size_t)row * 2 * (size_t)L.vstride + r]);
}

}  // namespace

/* elements of a row's key buffer (whole 512-byte blocks) */
static int64_t bigk_vstride(int vocab) { return ((int64_t)vocab + 63) & ~(int64_t)63; }

/* per row: two key buffers, six count tables, the segments' records, the
 * tile sums */
size_t bigk_row_bytes(const SampleArgs &a) {
  return 2 * (size_t)bigk_vstride(a.vocab) * sizeof(uint64_t) + 6 * (size_t)BK_SMAX * NB * sizeof(uint32_t) +
         (size_t)BK_SMAX * sizeof(BkMeta) + 2 * (size_t)((a.vocab + BK_T - 1) / BK_T) * sizeof(uint64_t);
}

bool launch_bigk(const SampleArgs &a, Dtype dt, void *ws, size_t ws_bytes, hipStream_t s) {
  const size_t per_row = bigk_row_bytes(a);
  if (!ws || ws_bytes < per_row || a.vocab < 1) return false;
  const int64_t chunk = (int64_t)(ws_bytes / per_row);
  const int es = dt == DT_F32 ? 4 : 2;
  const int64_t vstride = bigk_vstride(a.vocab);
  const int tiles = (a.vocab + BK_T - 1) / BK_T;
  for (int64_t r0 = 0; r0 < a.n_rows; r0 += chunk) {
    SampleArgs c = a;
    const int64_t n = a.n_rows - r0 < chunk ? a.n_rows - r0 : chunk;
    c.n_rows = (int)n;
    c.logits = (const char *)a.logits + (size_t)r0 * (size_t)a.row_stride * es;
    c.u = a.u + (size_t)r0 * a.k;
    if (a.temperature) c.temperature = a.temperature + r0;
    if (a.top_p) c.top_p = a.top_p + r0;
    if (a.banned) c.banned = a.banned + r0;
    c.ids = a.ids + r0;
    if (a.probs) c.probs = a.probs + (size_t)r0 * a.k;
    if (a.cand) c.cand = a.cand + (size_t)r0 * a.k;
    /* segments: enough workgroups for the CUs, whole tiles each */
    int want = (int)((BK_WGS + n - 1) / n);
    want = want < 1 ? 1 : (want > BK_SMAX ? BK_SMAX : want);
    BkLayout L{};
    L.tps = (tiles + want - 1) / want;
    L.nseg = (tiles + L.tps - 1) / L.tps;
    L.inv_sl = 1.0f / (float)(L.tps * BK_T);
    /* bf16 logits at T = 1 (after the clamp to 1e-5 either way): x = L, whose
     * low 16 bits are zero, so every row skips passes 0 and 1 (bk_row_max) */
    L.pass0 = dt == DT_BF16 && !a.temperature && a.temperature_scalar == 1.0f ? 2 : 0;
    L.vstride = vstride;
    L.keys = (uint64_t *)ws;
    L.hist = (uint32_t *)((char *)ws + (size_t)n * 2 * (size_t)vstride * sizeof(uint64_t));
    L.hidx = L.hist + (size_t)n * 4 * BK_SMAX * NB;
    L.meta = (BkMeta *)(L.hidx + (size_t)n * 2 * BK_SMAX * NB);
    L.ntiles = tiles;
    L.tsum = (uint64_t *)(L.meta + (size_t)n * BK_SMAX);
    const dim3 grid((unsigned)L.nseg, (unsigned)n);
    if (dt == DT_F32)
      hipLaunchKernelGGL(k_bk_keys<false>, grid, dim3(BK_T), 0, s, c, L);
    else
      hipLaunchKernelGGL(k_bk_keys<true>, grid, dim3(BK_T), 0, s, c, L);
    for (int pass = L.pass0; pass < 4; pass++) hipLaunchKernelGGL(k_bk_pass, grid, dim3(BK_T), 0, s, c, L, pass);
    hipLaunchKernelGGL(k_bk_sums, grid, dim3(BK_T), 0, s, c, L);
    hipLaunchKernelGGL(k_bk_cut, dim3((unsigned)n), dim3(BK_T), 0, s, c, L);
    hipLaunchKernelGGL(k_bk_race, grid, dim3(BK_T), 0, s, c, L);
    hipLaunchKernelGGL(k_bk_pick, dim3((unsigned)n), dim3(WAVE), 0, s, c, L);
  }
  return true;
}

}  // namespace d3s
