/* k_bigk: the op graph's sampler for k beyond the generic kernel's LDS sort
 * (k > 16384, on rows longer than the nucleus kernel takes), gfx950 wave64.
 *
 * The reference's op graph (src/sampling.c:22-49) takes any k up to V: with
 * top-k disabled it argsorts the whole row (:33-35).  One 1024-thread
 * workgroup per row:
 *  1. x = L / T, classification and max (refused / all -inf rows as every
 *     kernel treats them);
 *  2. the exact row sum (2^-40 fixed point of d3s_expf(x - m)), and the row's
 *     composite keys (ordkey(x), ~index) written to the workspace in index
 *     order, with the first pass's digit counts;
 *  3. a stable LSD radix sort of the keys by ordkey(x) descending, four 8-bit
 *     passes between two workspace buffers, in tiles of 1024 keys in index
 *     order: a wave's peers of a digit by eight ballots, per-wave digit counts
 *     in LDS turned into places by one thread per digit, two barriers a tile
 *     (ordering LDS only; each tile's keys load during the tile before), and
 *     the next pass's digit counts taken on the way.  Stability keeps equal x
 *     in index order, so the result is the order (x desc, index asc) of every
 *     kernel;
 *  4. the op graph's tail over the first k ranks (bigk_tail: the generic
 *     kernel's definition with coalesced reads: exact prefix sums chunk by
 *     chunk to the cut, the kept sum, probabilities and the race).
 * The same definition as the generic and nucleus kernels, bit for bit.  The
 * workspace holds two buffers of the row's keys (16 bytes per element). */
#include "d3s_generic.h"

#pragma clang fp contract(off)

namespace d3s {
namespace {

constexpr int BK_T = 1024;
constexpr int BK_NW = BK_T / WAVE;

/* a workgroup barrier that orders LDS only: global loads and stores stay in
 * flight across it (the sort's global writes are ordered by the full barrier
 * at the start of the next pass) */
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

constexpr int BK_CH = 4096; /* ranks of the cut's exact scan, staged in LDS */

/* block sum of per-thread fixed-point values (below 2^56 in total); opens
 * with a barrier (the scratch may still be being read) */
__device__ __forceinline__ uint64_t bk_block_sum(uint64_t v, uint32_t *lo, uint32_t *hi) {
  const uint64_t w = wave_sum_u64(v);
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

/* The op graph's tail (generic_tail_opgraph's definition, bit for bit) over
 * the k ranked keys in global memory, with coalesced reads: the exact prefix
 * sums of fix40(d3s_expf(x_r - lse)) are taken chunk by chunk (interleaved
 * per-thread sums: integers, so the order does not matter) until a chunk's
 * end passes top_p; that chunk is staged in LDS and scanned rank by rank for
 * the cut.  The kept sum, the probabilities and the race run over the ranks
 * interleaved across the threads (the race's first maximum: the largest
 * score, ties to the smaller rank). */
__device__ __forceinline__ void bigk_tail(const SampleArgs &a, const int row, const float lse, const float top_p,
                                          const uint64_t *glist, uint64_t *lch, uint32_t *sh_lo, uint32_t *sh_hi,
                                          uint32_t *sh_u32, float *sh_best, int *sh_bestr) {
  const int tid = (int)threadIdx.x, lane = lane_id(), wid = tid / WAVE;
  const int k = a.k;
  const float v0 = key_x(glist[0]);
  /* ---- the cut: the first r > 0 whose exact prefix passes top_p */
  int cut = k;
  uint64_t base = 0;
#pragma unroll 1
  for (int r_lo = 0; r_lo < k; r_lo += BK_CH) {
    const int r_hi = min(k, r_lo + BK_CH);
    uint64_t loc = 0;
#pragma unroll 4
    for (int r = r_lo + tid; r < r_hi; r += BK_T) loc += d3s_fix40(d3s_expf(key_x(glist[r]) - lse));
    const uint64_t tot = bk_block_sum(loc, sh_lo, sh_hi);
    if (!(r_hi > 1 && d3s_fixsum_to_f32(base + tot) > top_p)) {
      base += tot;
      continue;
    }
    /* the cut lies in this chunk: its keys to LDS, each thread a run of
     * BK_CH / BK_T consecutive ranks */
    for (int r = r_lo + tid; r < r_hi; r += BK_T) lch[r - r_lo] = glist[r];
    __syncthreads();
    constexpr int RUN = BK_CH / BK_T;
    uint64_t f[RUN];
    uint64_t part = 0;
#pragma unroll
    for (int q = 0; q < RUN; q++) {
      const int r = r_lo + tid * RUN + q;
      f[q] = r < r_hi ? d3s_fix40(d3s_expf(key_x(lch[tid * RUN + q]) - lse)) : 0ull;
      part += f[q];
    }
    uint64_t P = base + block_excl_scan_u64<BK_NW>(part, sh_lo, sh_hi);
    int cl = k;
#pragma unroll
    for (int q = 0; q < RUN; q++) {
      const int r = r_lo + tid * RUN + q;
      P += f[q];
      if (r < r_hi && r > 0 && cl == k && d3s_fixsum_to_f32(P) > top_p) cl = r;
    }
    const int cm = wave_min_i32(cl);
    if (lane == 0) sh_u32[wid] = (uint32_t)cm;
    __syncthreads();
    for (int w = 0; w < BK_NW; w++) cut = min(cut, (int)sh_u32[w]);
    break;
  }
  /* ---- the kept sum of fix40(d3s_expf(x_r - x_0)) over r < cut */
  uint64_t ks = 0;
#pragma unroll 4
  for (int r = tid; r < cut; r += BK_T) ks += d3s_fix40(d3s_expf(key_x(glist[r]) - v0));
  const float inv = 1.0f / d3s_fixsum_to_f32(bk_block_sum(ks, sh_lo, sh_hi));
  /* ---- probabilities, candidates and the race over every rank */
  float bs = -1.0f;
  int br = 0x7fffffff;
  const float *urow = a.u + (size_t)row * k;
#pragma unroll 2
  for (int r = tid; r < k; r += BK_T) {
    const uint64_t key = glist[r];
    const float p = r < cut ? d3s_expf(key_x(key) - v0) * inv : 0.0f;
    const float noise = -d3s_logf(1.0f - urow[r]);
    const float score = p / noise;
    const float sc = score > -1.0f ? score : -1.0f;
    if (sc > bs || br == 0x7fffffff) { /* this thread's ranks increase: its first maximum */
      bs = sc;
      br = r;
    }
    if (a.probs) a.probs[(size_t)row * k + r] = p;
    if (a.cand) a.cand[(size_t)row * k + r] = key_idx(key);
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
    a.ids[row] = key_idx(glist[r]);
  }
}

template <bool BF16>
__global__ __launch_bounds__(BK_T) void k_bigk(SampleArgs a, uint64_t *ws, int64_t vstride) {
  __shared__ uint32_t base[NB];            /* a digit's next place */
  __shared__ uint32_t hist[NB];            /* the next pass's digit counts */
  __shared__ uint32_t wcnt[2][BK_NW][NB];  /* a tile's count of each digit in each wave, then its place */
  __shared__ float sh_max[BK_NW];
  __shared__ uint32_t sh_flag[BK_NW], sh_lo[BK_NW], sh_hi[BK_NW];
  const int row = (int)blockIdx.x, tid = (int)threadIdx.x, lane = lane_id(), wid = tid / WAVE;
  const int V = a.vocab;
  const RowP rp = row_params(a, row);
  const float T = rp.T;
  const bool t_finite = T < __builtin_inff();
  const float y = 1.0f / T;
  const char *rowp = (const char *)a.logits + (size_t)row * (size_t)a.row_stride * (BF16 ? 2 : 4);
  auto xat = [&](int i) { return scale_logit(load_logit<BF16>(rowp, i, rp.banned), T, y, t_finite); };

  /* ---- 1. max and classification */
  float xm = -__builtin_inff();
  uint32_t fl = 0u;
  for (int i = tid; i < V; i += BK_T) {
    const float xi = xat(i);
    const uint32_t c = classify(xi);
    fl |= c;
    if (!(c & 1u)) xm = fmaxf(xm, xi);
  }
  xm = wave_max_f(xm);
  const uint32_t wf = __ballot(fl & 1u) ? 1u : 0u;
  if (lane == 0) {
    sh_max[wid] = xm;
    sh_flag[wid] = wf;
  }
  if (tid < NB) hist[tid] = 0u;
  __syncthreads();
  float M = sh_max[0];
  uint32_t F = sh_flag[0];
  for (int w = 1; w < BK_NW; w++) {
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

  /* ---- 2. the exact row sum, the keys in index order and the first pass's
   * digit counts */
  uint64_t *buf[2] = {ws + (size_t)row * 2 * (size_t)vstride, ws + (size_t)row * 2 * (size_t)vstride + vstride};
  uint64_t acc = 0;
  for (int i = tid; i < V; i += BK_T) {
    const float xi = xat(i);
    acc += d3s_fix40(d3s_expf(xi - M));
    const uint64_t key = composite_key(xi, i);
    buf[0][i] = key;
    atomicAdd(&hist[bk_digit(key, 0)], 1u);
  }
  {
    const uint64_t w = wave_sum_u64(acc);
    if (lane == 0) {
      sh_lo[wid] = (uint32_t)w;
      sh_hi[wid] = (uint32_t)(w >> 32);
    }
  }
  __syncthreads();
  uint64_t S = 0;
  for (int w = 0; w < BK_NW; w++) S += ((uint64_t)sh_hi[w] << 32) | sh_lo[w];
  const float lse = M + d3s_logf(d3s_fixsum_to_f32(S));

  /* ---- 3. stable LSD radix sort by ordkey(x) descending.  Per tile of
   * 1024 keys (index order within the pass): each wave counts its keys of
   * each digit (the first lane of a digit's peers files the count); thread t
   * < 256 turns digit t's counts into places (the running base plus the
   * earlier waves'); each key goes to its wave's place plus its peers below
   * it.  Two count buffers alternate between tiles, so each is cleared a tile
   * after its last read.  The next pass's digit counts are taken on the way. */
  const uint64_t lt = (1ull << lane) - 1ull; /* lanes below this one */
#pragma unroll 1
  for (int pass = 0; pass < 4; pass++) {
    const uint64_t *src = buf[pass & 1];
    uint64_t *dst = buf[(pass & 1) ^ 1];
    /* both count buffers zero for the pass's first two tiles (the last
     * tile of the pass before left its places in one of them) */
    for (int j = tid; j < 2 * BK_NW * NB; j += BK_T) (&wcnt[0][0][0])[j] = 0u;
    if (wid == 0) { /* the pass's digit counts -> starts, four per lane */
      uint32_t h[4];
#pragma unroll
      for (int q = 0; q < 4; q++) h[q] = hist[4 * lane + q];
      const uint32_t ls = h[0] + h[1] + h[2] + h[3];
      uint32_t run = wave_scan_add_u32(ls) - ls;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        base[4 * lane + q] = run;
        hist[4 * lane + q] = 0u;
        run += h[q];
      }
    }
    __syncthreads();
    /* each tile's key is loaded one tile ahead, its latency behind the
     * previous tile's barriers (which order LDS only) */
    uint64_t next = tid < V ? src[tid] : 0ull;
    int par = 0;
#pragma unroll 1
    for (int t0 = 0; t0 < V; t0 += BK_T, par ^= 1) {
      const int i = t0 + tid;
      const bool valid = i < V;
      const uint64_t key = next;
      next = i + BK_T < V ? src[i + BK_T] : 0ull;
      const uint64_t live = __ballot(valid);
      const uint32_t d = bk_digit(key, pass);
      const uint64_t peers = wave_peers<8>(d, live);
      const uint32_t below = (uint32_t)__popcll(peers & lt);
      if (valid && below == 0u) wcnt[par][wid][d] = (uint32_t)__popcll(peers);
      if (pass < 3) {
        const uint32_t d2 = bk_digit(key, pass + 1);
        const uint64_t p2 = wave_peers<8>(d2, live);
        if (valid && (p2 & lt) == 0ull) atomicAdd(&hist[d2], (uint32_t)__popcll(p2));
      }
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
      if (valid) dst[wcnt[par][wid][d] + below] = key;
    }
    __syncthreads(); /* the pass's keys and the next pass's counts, for every thread */
  }

  /* ---- 4. the op graph's tail over the first k ranks (four passes end in
   * buf[0]) */
  {
    __shared__ uint32_t sh_u32[BK_NW];
    __shared__ float sh_best[BK_NW];
    __shared__ int sh_bestr[BK_NW];
    static_assert(sizeof(wcnt) >= BK_CH * sizeof(uint64_t), "the chunk fits in the count buffers");
    bigk_tail(a, row, lse, rp.top_p, buf[0], (uint64_t *)&wcnt[0][0][0], sh_lo, sh_hi, sh_u32, sh_best, sh_bestr);
  }
}

}  // namespace

/* elements of a row's key buffer (whole 512-byte blocks) */
static int64_t bigk_vstride(int vocab) { return ((int64_t)vocab + 63) & ~(int64_t)63; }

size_t bigk_row_bytes(const SampleArgs &a) { return 2 * (size_t)bigk_vstride(a.vocab) * sizeof(uint64_t); }

bool launch_bigk(const SampleArgs &a, Dtype dt, void *ws, size_t ws_bytes, hipStream_t s) {
  const size_t per_row = bigk_row_bytes(a);
  if (!ws || ws_bytes < per_row) return false;
  const int64_t chunk = (int64_t)(ws_bytes / per_row);
  const int es = dt == DT_F32 ? 4 : 2;
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
    if (dt == DT_F32)
      hipLaunchKernelGGL(k_bigk<false>, dim3((unsigned)n), dim3(BK_T), 0, s, c, (uint64_t *)ws,
                         bigk_vstride(a.vocab));
    else
      hipLaunchKernelGGL(k_bigk<true>, dim3((unsigned)n), dim3(BK_T), 0, s, c, (uint64_t *)ws,
                         bigk_vstride(a.vocab));
  }
  return true;
}

}  // namespace d3s
