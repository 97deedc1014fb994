/* HIP kernels of the MI355X token sampler (gfx950, wave64).
 *
 * Semantics: the sampler of SeungheonOh/drama3-mlx, src/sampling.c (temperature
 * :195,:25,:70; row log-sum-exp :37-38,:67-89; top-k ranked by (x desc, index
 * asc) :27-36,:90-121; exclusive top-p :39-42,:126-128; renormalised softmax
 * :43-44,:129-134; exponential race over caller uniforms :45-48,:132-139).
 *
 * Two kernels, one workgroup per row:
 *  - k_fused (k <= 64, row held in registers, 1024 threads): pass 1 divides
 *    the row by T exactly (FMA division) and takes its max; pass 2 sums
 *    exp(x - m) exactly in 2^-40 fixed point (order independent) and builds a
 *    256-bin histogram of the distance below the max; the bin holding the k-th
 *    value bounds a small candidate set, each candidate finds its own rank and
 *    files its rank-independent terms, and wave 0 runs the reference kernel's
 *    sequential cumulative, the cut and the race.  Rows the histogram cannot
 *    settle take an exact 8-bit radix select over order-preserving keys.
 *  - k_generic (any V, k <= 16384): streams the row from global memory for
 *    every pass; exact log-sum-exp, radix select, LDS bitonic sort of the k
 *    selected, exact-sum top-p for k > 64.  Rows wider than the fused kernel
 *    takes, k > 64 (the reference's op-graph cases), and the
 *    D3S_FLAG_GENERIC switch use it.
 * Both compute the same definition bit for bit (the oracle's).
 */
#include <mutex>

#include "d3s_generic.h"

#pragma clang fp contract(off)

namespace d3s {
namespace {

constexpr float BINS_PER_NAT = 8.0f;        /* 256 bins over 32 units of x below the max */
constexpr int GCAP = 256;                   /* candidate capacity of the fused kernel */

template <int BLOCK, int CPT, bool BF16>
__global__ __launch_bounds__(BLOCK) void k_fused(SampleArgs a) {
  constexpr int ES = BF16 ? 2 : 4;
  constexpr int EPC = 16 / ES; /* elements per 16-byte chunk */
  constexpr int NV = CPT * EPC;
  constexpr int NW = BLOCK / WAVE;
  static_assert(BLOCK >= GCAP, "one thread per candidate");

  /* bins, then one overflow bin per lane: skipped elements still add (no branch) */
  __shared__ uint32_t hist[NB + WAVE];
  __shared__ float sh_max[NW];
  __shared__ uint32_t sh_flag[NW], sh_scan[NW], sh_lo[NW], sh_hi[NW];
  /* candidates, zero past them, then one write-off slot per lane */
  __shared__ __align__(16) uint64_t gK[GCAP + 2 + WAVE];
  /* by rank: index, exp(x - lse), exp(x - x_0) */
  __shared__ int si[KF];
  __shared__ float se[KF], sp[KF];
  __shared__ __align__(16) float wbuf[WAVE];
  __shared__ int n_gather;

  const int row = blockIdx.x;
  const int tid = threadIdx.x, lane = lane_id(), wid = tid / WAVE;
  const int V = a.vocab, k = a.k;
  const RowP rp = row_params(a, row);
  const float T = rp.T;
  const bool t_finite = T < __builtin_inff();
  const float y = 1.0f / T;
  float uval = 0.0f; /* this row's uniforms, fetched early: the race reads them last */
  if (wid == 0 && lane < k) uval = a.u[(size_t)row * k + lane];

  /* ---- the row, in 16-byte chunks from the aligned address at or below its
   * start (a chunk never crosses a page, so the bytes outside the row that it
   * covers are readable; they are masked out below) */
  const char *rowp = (const char *)a.logits + (size_t)row * (size_t)a.row_stride * ES;
  const int off = (int)(((uintptr_t)rowp & 15u) / ES);
  const uint4 *src = (const uint4 *)(rowp - off * ES);
  const int nchunks = (off + V + EPC - 1) / EPC;
  float x[NV];
#pragma unroll
  for (int j = 0; j < CPT; j++) {
    const int c = j * BLOCK + tid;
    uint4 q = make_uint4(0u, 0u, 0u, 0u);
    if (c < nchunks) q = src[c];
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int e = 0; e < EPC; e++) {
      if (BF16)
        x[j * EPC + e] = d3s_u2f((e & 1) ? (w[e / 2] & 0xffff0000u) : (w[e / 2] << 16));
      else
        x[j * EPC + e] = d3s_u2f(w[e]);
    }
  }
  /* element i of this thread: chunk row i/EPC, lane-in-chunk i%EPC; index order
   * is (chunk row, thread, lane-in-chunk) */
  auto pos = [&](int i) { return ((i / EPC) * BLOCK + tid) * EPC + (i % EPC) - off; };
  auto valid = [&](int i) { return (unsigned)pos(i) < (unsigned)V; };
  /* does any lane of this wave hold a chunk of row j (wave-uniform) */
  auto wave_has_row = [&](int j) {
    return __builtin_amdgcn_readfirstlane(j * BLOCK + wid * WAVE) < nchunks;
  };

  /* ---- pass 1: x = logit / T exactly, classification, row max.  A wave whose
   * logits all lie where the FMA division is exact takes it without branches;
   * otherwise each element picks its own way (d3s_div_rn). */
  bool in_range = true;
#pragma unroll
  for (int i = 0; i < NV; i++) {
    const uint32_t ea = (d3s_f2u(x[i]) >> 23) & 0xffu;
    const bool ok = ea - 67u <= 160u && pos(i) != rp.banned; /* 2^-60 <= |L| < 2^101 */
    in_range = in_range && (ok || !valid(i));
  }
  float xm = -__builtin_inff();
  uint32_t fl = 0u;
  if (t_finite && __all(in_range)) {
#pragma unroll
    for (int i = 0; i < NV; i++) {
      const float q = x[i] * y;
      const float r = __builtin_fmaf(-q, T, x[i]);
      const float xi = __builtin_fmaf(r, y, q);
      x[i] = xi;
      const bool vld = valid(i);
      fl |= vld ? classify(xi) : 0u;
      xm = vld ? fmaxf(xm, xi) : xm;
    }
  } else {
#pragma unroll
    for (int i = 0; i < NV; i++)
      if (valid(i)) {
        const float L = pos(i) == rp.banned ? -__builtin_inff() : x[i];
        const float xi = scale_logit(L, T, y, t_finite);
        x[i] = xi;
        const uint32_t c = classify(xi);
        fl |= c;
        if (!(c & 1u)) xm = fmaxf(xm, xi);
      }
  }
  for (int i = tid; i < NB + WAVE; i += BLOCK) hist[i] = 0u;
  for (int i = tid; i < GCAP + 2; i += BLOCK) gK[i] = 0ull;
  if (tid == 0) n_gather = 0;
  /* the race's noise -log(1 - u) only needs u: wave 0 computes it while the
   * other waves finish the first pass */
  const float noise = wid == 0 ? -d3s_logf(1.0f - uval) : 0.0f;
  xm = wave_max_f(xm);
  const uint32_t wf = (__ballot(fl & 1u) ? 1u : 0u) | (__ballot(fl & 2u) ? 2u : 0u);
  if (lane == 0) {
    sh_max[wid] = xm;
    sh_flag[wid] = wf;
  }
  __syncthreads();
  float M = sh_max[0];
  uint32_t F = sh_flag[0];
#pragma unroll
  for (int w = 1; w < NW; w++) {
    M = fmaxf(M, sh_max[w]);
    F |= sh_flag[w];
  }
  if (F & 1u) { /* a NaN or +inf x */
    write_special(a, row, false);
    return;
  }
  if (M == -__builtin_inff()) {
    write_special(a, row, true);
    return;
  }

  /* ---- pass 2: the exact row sum of exp(x - m) in 2^-40 fixed point (order
   * independent, src/sampling.c:81-89) and a histogram of the distance below
   * the max, 8 bins per unit of x over 32 units */
  uint64_t acc = 0;
  const int overflow_bin = NB + lane;
#pragma unroll
  for (int j = 0; j < CPT; j++)
    if (wave_has_row(j)) {
#pragma unroll
      for (int e = 0; e < EPC; e++) {
        const int i = j * EPC + e;
        const bool vld = valid(i);
        const float z = x[i] - M;
        const uint64_t f = d3s_fix40_exp(z);
        acc += vld ? f : 0ull;
        const float b = -z * BINS_PER_NAT;
        atomicAdd(&hist[(vld && b < (float)NB) ? (int)b : overflow_bin], 1u);
      }
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
#pragma unroll
  for (int w = 0; w < NW; w++) S += ((uint64_t)sh_hi[w] << 32) | sh_lo[w];
  const float lse = M + d3s_logf(d3s_fixsum_to_f32(S)); /* src/sampling.c:89 */
  /* every wave finds the k-th element's bin: same answer, no extra barrier */
  const BinSel bs = wave_find_bin<true>(hist, (uint32_t)k);
  const bool need_exact = !bs.ok || bs.above + bs.count > (uint32_t)GCAP || (a.flags & FLAG_EXACT_SELECT);

  int G;
  if (!need_exact) {
    /* candidates: every element in a bin up to the k-th element's.  The bin is
     * a non-increasing function of x, so an element left out has a smaller x
     * than every candidate and ranks below all of them. */
    const float blim = (float)(bs.bin + 1u); /* b < bin + 1  <=>  (int)b <= bin */
    uint32_t mine = 0u;
#pragma unroll
    for (int i = 0; i < NV; i++) mine += (valid(i) && -(x[i] - M) * BINS_PER_NAT < blim) ? 1u : 0u;
    /* slots: one atomic per wave, then each lane's exclusive prefix */
    const uint32_t incl = wave_scan_add_u32(mine);
    const uint32_t wtot = readlane_u(incl, 63);
    int base = 0;
    if (wtot != 0u) {
      if (lane == 0) base = atomicAdd(&n_gather, (int)wtot);
      base = __builtin_amdgcn_readfirstlane(base);
    }
    uint32_t slot = (uint32_t)base + incl - mine;
    const uint32_t write_off = GCAP + 2 + lane;
#pragma unroll
    for (int j = 0; j < CPT; j++)
      if (wave_has_row(j)) {
#pragma unroll
        for (int e = 0; e < EPC; e++) {
          const int i = j * EPC + e;
          const bool cnd = valid(i) && -(x[i] - M) * BINS_PER_NAT < blim;
          gK[(cnd && slot < (uint32_t)GCAP) ? slot : write_off] = composite_key(x[i], pos(i));
          slot += cnd ? 1u : 0u;
        }
      }
    __syncthreads();
    G = min(n_gather, GCAP); /* = above + count >= k */
  } else {
    /* ---- exact radix select of the k-th (x desc, index asc) rank over
     * order-preserving keys of x, 8 bits per pass */
    if (tid == 0 && a.counters) atomicAdd(&a.counters[CNT_EXACT_SELECT], 1u);
    uint32_t prefix = 0u, pmask = 0u, need = (uint32_t)k, done = 0u;
#pragma unroll
    for (int pass = 0; pass < 4; pass++) {
      if (!done) {
        const int shift = 24 - 8 * pass;
        __syncthreads(); /* every wave has read the previous histogram */
        for (int i = tid; i < NB; i += BLOCK) hist[i] = 0u;
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NV; i++) {
          const uint32_t key = d3s_ordkey(x[i]);
          if (valid(i) && (key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
        }
        __syncthreads();
        const BinSel b = wave_find_bin<false>(hist, need); /* holds >= need */
        prefix |= b.bin << shift;
        pmask |= 0xffu << shift;
        done = b.count == need - b.above;
        need -= b.above;
      }
    }
    /* everything above the group, then the group: all of it when it holds
     * exactly `need`, else (exact ties) its lowest-index `need` */
#pragma unroll
    for (int i = 0; i < NV; i++) {
      const uint32_t key = d3s_ordkey(x[i]) & pmask;
      const int slot = wave_append(valid(i) && (key > prefix || (done && key == prefix)), &n_gather);
      if (slot >= 0 && slot < GCAP) gK[slot] = composite_key(x[i], pos(i));
    }
    if (!done) {
      uint32_t base = 0u;
#pragma unroll
      for (int j = 0; j < CPT; j++) {
        uint32_t cnt = 0u;
#pragma unroll
        for (int e = 0; e < EPC; e++) {
          const int i = j * EPC + e;
          cnt += (valid(i) && d3s_ordkey(x[i]) == prefix) ? 1u : 0u;
        }
        const uint32_t incl = wave_scan_add_u32(cnt);
        if (lane == WAVE - 1) sh_scan[wid] = incl;
        __syncthreads();
        uint32_t wbase = 0u, tot = 0u;
#pragma unroll
        for (int w = 0; w < NW; w++) {
          const uint32_t t = sh_scan[w];
          if (w < wid) wbase += t;
          tot += t;
        }
        uint32_t ord = base + wbase + incl - cnt;
#pragma unroll
        for (int e = 0; e < EPC; e++) {
          const int i = j * EPC + e;
          const bool tie = valid(i) && d3s_ordkey(x[i]) == prefix;
          const int slot = wave_append(tie && ord < need, &n_gather);
          if (slot >= 0 && slot < GCAP) gK[slot] = composite_key(x[i], pos(i));
          ord += tie ? 1u : 0u;
        }
        base += tot;
        __syncthreads();
      }
    }
    __syncthreads();
    G = min(n_gather, GCAP); /* == k */
  }

  /* ---- each candidate finds its rank (keys above its own, broadcast reads of
   * two keys at a time) and, if it is among the top k, files its index and
   * its rank-independent terms exp(x - lse) (src/sampling.c:127) and
   * exp(x - x_0) (x_0 = m; src/sampling.c:129,134) at its rank */
  if (tid < G) {
    const uint64_t my = gK[tid];
    const ulonglong2 *k2 = (const ulonglong2 *)gK;
    int rank = 0;
#pragma unroll 4
    for (int j2 = 0; j2 < (G + 1) / 2; j2++) {
      const ulonglong2 q = k2[j2];
      rank += (q.x > my ? 1 : 0) + (q.y > my ? 1 : 0);
    }
    if (rank < k) {
      const float xr = key_x(my);
      si[rank] = key_idx(my);
      se[rank] = d3s_expf(xr - lse);
      sp[rank] = d3s_expf(xr - M);
    }
  }
  if (G > WAVE)
    __syncthreads();
  if (wid != 0) return;
  wave_lds_sync();
  const bool act = lane < k;
  const int idx = act ? si[lane] : 0;
  const float e = act ? se[lane] : 0.0f;
  const float ep = act ? sp[lane] : 0.0f;
  /* ---- the reference kernel's sequential cumulative (src/sampling.c:126-128) */
  const float c = wave_seq_cumsum(e, k, wbuf);
  wave_race(a, row, idx, c, ep, noise, rp.top_p, wbuf);
}

/* ------------------------------------------------------------------------ */
/* generic kernel                                                            */
/* ------------------------------------------------------------------------ */

template <bool BF16>
__global__ __launch_bounds__(GBLOCK) void k_generic(SampleArgs a, int kpow) {
  extern __shared__ uint64_t glist[]; /* [kpow] composite keys, sorted in place */
  generic_row<BF16>(a, (int)blockIdx.x, kpow, glist);
}

__global__ void k_uniform(float *u, int64_t n, uint64_t seed, uint64_t stream_id) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) u[i] = d3s_uniform(seed, stream_id, (uint64_t)i);
}

/* w[i] = 0 for i < n, 16 bytes per thread where whole vectors fit (the
 * workspace clear: a kernel node, never a memset node, in a captured graph) */
__global__ void k_zero_fill(uint32_t *w, int64_t n) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i + 4 <= n) {
    *(uint4 *)(w + i) = make_uint4(0u, 0u, 0u, 0u);
  } else {
    for (int64_t j = i; j < n; j++) w[j] = 0u;
  }
}

__global__ void k_math(const float *in, float *oe, float *ol, float *od, uint64_t *of, int64_t n,
                       float divisor) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    const float x = in[i];
    oe[i] = d3s_expf(x);
    ol[i] = d3s_logf(x);
    od[i] = d3s_div_rn(x, divisor, 1.0f / divisor);
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
  /* 1024 threads per row: a few elements per thread keeps the row's passes short */
  if (dt == DT_F32) return try_fused<1024, 2, false>(a, s) || try_fused<1024, 4, false>(a, s);
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

void launch_zero_fill(uint32_t *w, size_t n_words, hipStream_t s) {
  if (n_words == 0) return;
  const int B = 256;
  const size_t threads = (n_words + 3) / 4;
  hipLaunchKernelGGL(k_zero_fill, dim3((unsigned)((threads + B - 1) / B)), dim3(B), 0, s, w, (int64_t)n_words);
}

void launch_math_selftest(const float *in, float *out_exp, float *out_log, float *out_div,
                          uint64_t *out_fix, int64_t n, float divisor, hipStream_t s) {
  if (n <= 0) return;
  const int B = 256;
  hipLaunchKernelGGL(k_math, dim3((unsigned)((n + B - 1) / B)), dim3(B), 0, s, in, out_exp,
                     out_log, out_div, out_fix, n, divisor);
}

}  // namespace d3s
