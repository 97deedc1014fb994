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
 *     order;
 *  3. a stable LSD radix sort of the keys by ordkey(x) descending, four 8-bit
 *     passes between two workspace buffers: per pass a digit histogram and
 *     its scan, then tiles of 1024 keys in index order, each key placed at
 *     its digit's running base plus the keys of its digit before it in the
 *     tile (a wave's peers by eight ballots, earlier waves' counts in LDS).
 *     Stability keeps equal x in index order, so the result is the order
 *     (x desc, index asc) of every kernel;
 *  4. the op graph's tail over the first k ranks (generic_tail_opgraph: exact
 *     prefix sums, the cut, the kept sum, probabilities and the race).
 * The same definition as the generic and nucleus kernels, bit for bit.  The
 * workspace holds two buffers of the row's keys (16 bytes per element). */
#include "d3s_generic.h"

#pragma clang fp contract(off)

namespace d3s {
namespace {

constexpr int BK_T = 1024;
constexpr int BK_NW = BK_T / WAVE;

/* the sort digit of a composite key in a pass: byte `pass` of ~ordkey(x)
 * (ascending ~ordkey is descending x) */
__device__ __forceinline__ uint32_t bk_digit(uint64_t key, int pass) {
  return (uint32_t)((~key) >> (32 + 8 * pass)) & 0xffu;
}

template <bool BF16>
__global__ __launch_bounds__(BK_T) void k_bigk(SampleArgs a, uint64_t *ws, int64_t vstride) {
  __shared__ uint32_t base[NB];         /* a digit's next place */
  __shared__ uint32_t wcnt[BK_NW][NB];  /* a tile's count of each digit in each wave */
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

  /* ---- 2. the exact row sum, and the keys in index order */
  uint64_t *buf[2] = {ws + (size_t)row * 2 * (size_t)vstride, ws + (size_t)row * 2 * (size_t)vstride + vstride};
  uint64_t acc = 0;
  for (int i = tid; i < V; i += BK_T) {
    const float xi = xat(i);
    acc += d3s_fix40(d3s_expf(xi - M));
    buf[0][i] = composite_key(xi, i);
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

  /* ---- 3. stable LSD radix sort by ordkey(x) descending */
  const uint64_t lt = (1ull << lane) - 1ull; /* lanes below this one */
#pragma unroll 1
  for (int pass = 0; pass < 4; pass++) {
    const uint64_t *src = buf[pass & 1];
    uint64_t *dst = buf[(pass & 1) ^ 1];
    if (tid < NB) base[tid] = 0u;
    for (int j = tid; j < BK_NW * NB; j += BK_T) (&wcnt[0][0])[j] = 0u;
    __syncthreads();
    for (int i = tid; i < V; i += BK_T) atomicAdd(&base[bk_digit(src[i], pass)], 1u);
    __syncthreads();
    if (wid == 0) { /* exclusive scan of the 256 counts, four per lane */
      uint32_t h[4];
#pragma unroll
      for (int q = 0; q < 4; q++) h[q] = base[4 * lane + q];
      const uint32_t ls = h[0] + h[1] + h[2] + h[3];
      uint32_t run = wave_scan_add_u32(ls) - ls;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        base[4 * lane + q] = run;
        run += h[q];
      }
    }
    __syncthreads();
#pragma unroll 1
    for (int t0 = 0; t0 < V; t0 += BK_T) {
      const int i = t0 + tid;
      const bool valid = i < V;
      const uint64_t key = valid ? src[i] : 0ull;
      const uint32_t d = bk_digit(key, pass);
      uint64_t peers = __ballot(valid); /* the wave's keys of digit d */
#pragma unroll
      for (int b = 0; b < 8; b++) {
        const uint64_t bb = __ballot((d >> b) & 1u);
        peers &= ((d >> b) & 1u) ? bb : ~bb;
      }
      const uint32_t below = (uint32_t)__popcll(peers & lt);
      if (valid && below == 0u) wcnt[wid][d] = (uint32_t)__popcll(peers);
      __syncthreads();
      if (valid) {
        uint32_t off = base[d] + below;
        for (int w = 0; w < wid; w++) off += wcnt[w][d];
        dst[off] = key;
      }
      __syncthreads();
      if (tid < NB) {
        uint32_t tot = 0u;
#pragma unroll
        for (int w = 0; w < BK_NW; w++) {
          tot += wcnt[w][tid];
          wcnt[w][tid] = 0u;
        }
        base[tid] += tot;
      }
      __syncthreads();
    }
  }

  /* ---- 4. the op graph's tail over the first k ranks (four passes end in
   * buf[0]) */
  generic_tail_opgraph<BK_T>(a, row, lse, rp.top_p, buf[0]);
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
