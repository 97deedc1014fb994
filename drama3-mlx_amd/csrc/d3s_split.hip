/* k_split: rows too wide for one wave (k <= 64) cut into segments, every
 * segment of every row in one launch (gfx950, wave64).
 *
 * A segment is SPLIT_NW waves x 64 lanes x CPT 16-byte chunks of the row, one
 * workgroup.  It runs the one-wave kernel's passes on its part (registers,
 * NaN-propagating max, a threshold from an 8-bit histogram of its 256 lane
 * maxima, candidate bits, the fast sum 2^(L c - h_s) relative to its own max)
 * and ranks its candidates: its top min(k, candidates) keys hold every key of
 * the row's top k that lies in the segment.  It publishes a record (max, fast
 * sum, flags, keys by rank) with agent-coherent stores, waits for them to
 * complete, and counts its arrival on the row's counter (one counter per
 * 128-byte line: rows do not contend).  The workgroup that arrives last merges
 * the records: the row max, the fast sums rescaled to the row's offset, the
 * top k of the segments' keys, and runs the reference kernel's tail
 * (src/sampling.c:123-139, or the op graph's order :39-48) with the fast lse's
 * margin test.  A cut within the margin takes the exact lse (the whole
 * workgroup streams the row once); T not finite, logits too large for the fast
 * sum, more candidates than a segment files or fewer finite keys than k
 * sample the row by the generic procedure.  Every result is the oracle's bits.
 * No spin-waits: a workgroup that is not last ends; the counter wraps to 0 for
 * the next launch. */
#include "d3s_rowcore.h"

namespace d3s {
namespace {

constexpr int SPLIT_NW = 4;              /* waves per segment */
constexpr int SPLIT_CPT = 8;             /* 16-byte chunks per lane */
constexpr int SPLIT_T = SPLIT_NW * WAVE; /* threads per segment */
constexpr int SCAP = SPLIT_T;            /* candidates a segment ranks (one per thread) */
constexpr int SPLIT_MAX_SEG = 16;        /* segments per row */
constexpr int MCAP = SPLIT_MAX_SEG * KF; /* keys the merger ranks */

/* record flags */
constexpr uint32_t SEG_GENERIC = 1u;  /* T not finite or logits too large: the generic procedure */
constexpr uint32_t SEG_OVERFLOW = 2u; /* more candidates than the segment files (or forced) */

struct __align__(16) SplitLds {
  uint64_t keys[MCAP + 2]; /* a segment's candidates; the merger's keys (+ zero pads) */
  uint64_t ranked[KF];
  uint32_t hist[NB];
  float buf[WAVE];
  float wmax[SPLIT_NW], wsum[SPLIT_NW];
  uint32_t wcnt[SPLIT_NW];
  float smax[SPLIT_MAX_SEG], ssum[SPLIT_MAX_SEG];
  uint32_t sflags[SPLIT_MAX_SEG], sn[SPLIT_MAX_SEG];
  uint32_t last, exact;
  uint32_t slo[SPLIT_NW], shi[SPLIT_NW];
};

__device__ __forceinline__ void st_agent(uint64_t *p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_agent(const uint64_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* The exact lse of the row (the oracle's: 2^-40 fixed point of d3s_expf(x -
 * M)), by the whole workgroup streaming the row once. */
template <bool BF16>
__device__ __forceinline__ float split_exact_lse(const SampleArgs &a, int row, float M, SplitLds &S) {
  const RowP rp = row_params(a, row);
  const float y = 1.0f / rp.T;
  const char *rowp = (const char *)a.logits + (size_t)row * (size_t)a.row_stride * (BF16 ? 2 : 4);
  uint64_t acc = 0;
  for (int i = threadIdx.x; i < a.vocab; i += SPLIT_T)
    acc += d3s_fix40_exp(scale_logit(load_logit<BF16>(rowp, i, rp.banned), rp.T, y, true) - M);
  const uint64_t w = wave_sum_u64(acc);
  const int wid = threadIdx.x / WAVE;
  if (lane_id() == 0) {
    S.slo[wid] = (uint32_t)w;
    S.shi[wid] = (uint32_t)(w >> 32);
  }
  __syncthreads();
  uint64_t tot = 0;
#pragma unroll
  for (int q = 0; q < SPLIT_NW; q++) tot += ((uint64_t)S.shi[q] << 32) | S.slo[q];
  return M + d3s_logf(d3s_fixsum_to_f32(tot));
}

/* rank the n keys in S.keys (n <= cap): every key counts the keys above its
 * own; those below k land in S.ranked by rank.  Called by every thread. */
__device__ __forceinline__ void split_rank(SplitLds &S, uint32_t n, int k) {
  if (threadIdx.x == 0) {
    S.keys[n] = 0ull; /* pads below every key */
    S.keys[n + 1] = 0ull;
  }
  __syncthreads();
  const ulonglong2 *k2 = (const ulonglong2 *)S.keys;
  for (uint32_t t = threadIdx.x; t < n; t += SPLIT_T) {
    const uint64_t my = S.keys[t];
    int rank = 0;
#pragma unroll 4
    for (int j2 = 0; j2 < (int)(n + 1) / 2; j2++) {
      const ulonglong2 q = k2[j2];
      rank += (q.x > my ? 1 : 0) + (q.y > my ? 1 : 0);
    }
    if (rank < k) S.ranked[rank] = my;
  }
  __syncthreads();
}

template <int CPT, bool BF16>
__global__ __launch_bounds__(SPLIT_T) void k_split(SampleArgs a, uint32_t *counters_ws, uint64_t *records,
                                                   int nseg, int rec_words) {
  using C = Chunks<CPT, BF16>;
  constexpr int ES = BF16 ? 2 : 4, EPC = C::EPC, NV = C::NV;
  constexpr int CAP = SPLIT_NW * CPT * WAVE; /* chunks per segment */
  constexpr int EARLY = 3;
  __shared__ SplitLds S;
  __shared__ uint64_t glist[KF]; /* the generic procedure's sort list */
  const int row = (int)blockIdx.x / nseg, seg = (int)blockIdx.x % nseg;
  const int wid = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / WAVE));
  const int lane = lane_id();
  const int V = a.vocab, k = a.k;
  int kpow = 2;
  while (kpow < k) kpow <<= 1;
  const RowP rp = row_params(a, row);
  const float T = rp.T, top_p = rp.top_p;
  const int banned = rp.banned;
  const bool t_finite = T < __builtin_inff(); /* false for +inf and NaN */
  const float y = 1.0f / T;
  const char *rowp = (const char *)a.logits + (size_t)row * (size_t)a.row_stride * ES;
  const int off = (int)(((uintptr_t)rowp & 15u) / ES);
  const uint4 *src = (const uint4 *)(rowp - off * ES);
  const int nchunks = (off + V + EPC - 1) / EPC;
  const int cbase = seg * CAP + wid * CPT * WAVE; /* this wave's first chunk */
  C c;
  c.load(src + cbase, min(max(nchunks - cbase, 0), CPT * WAVE), lane);
  const int pos0 = (cbase + lane) * EPC - off;
  auto valid = [&](int i) { return (unsigned)C::pos(pos0, i) < (unsigned)V; };
#pragma unroll
  for (int j = 0; j < CPT; j++) {
    const int p_lo = (cbase + j * WAVE) * EPC - off; /* wave-uniform */
    if (p_lo < 0 || p_lo + WAVE * EPC > V) {
#pragma unroll
      for (int e = 0; e < EPC; e++) c.mask(j * EPC + e, !valid(j * EPC + e));
    }
  }
  if ((unsigned)banned < (unsigned)V) {
    const int bc = (banned + off) / EPC, eb = (banned + off) % EPC;
    if (bc >= cbase && bc < cbase + CPT * WAVE) {
      const int jb = (bc - cbase) / WAVE, lb = (bc - cbase) % WAVE;
#pragma unroll
      for (int j = 0; j < CPT; j++)
        if (j == jb) {
#pragma unroll
          for (int e = 0; e < EPC; e++) c.mask(j * EPC + e, lane == lb && e == eb);
        }
    }
  }

  /* ---- the segment's max of the logits; NaN propagates */
  const float ninf = -__builtin_inff();
  float lm = ninf;
#pragma unroll
  for (int i = 0; i < NV; i++) lm = fmaximum(lm, c.val(i));
  {
    const float wm = wave_maximum_f(lm);
    if (lane == 0) S.wmax[wid] = wm;
  }
  __syncthreads();
  float Ls = S.wmax[0];
#pragma unroll
  for (int w = 1; w < SPLIT_NW; w++) Ls = fmaximum(Ls, S.wmax[w]);
  uint32_t flags = 0u, nfiled = 0u;
  float ssum = 0.0f;
  const float cf = LOG2E_F / T;
  /* a segment with a NaN or +inf, or with no finite logit, files no keys */
  const bool live = !d3s_isnan(Ls) && Ls != __builtin_inff() && Ls != ninf;
  if (live) {
    if (!t_finite || !(fabsf(Ls * cf) < 0x1p24f)) flags |= SEG_GENERIC;
  }
  if (live && flags == 0u) {
    const float b = -(Ls * cf);
    /* ---- tau: the k-th largest of the segment's lane maxima to 16 bits of
     * its order key (a lower bound: at least k elements reach it) */
    const uint32_t lkey = d3s_ordkey(lm);
    uint32_t prefix = 0u, pmask = 0u, need = (uint32_t)k;
#pragma unroll
    for (int pass = 0; pass < 2; pass++) {
      const int shift = 24 - 8 * pass;
      S.hist[threadIdx.x] = 0u; /* SPLIT_T == NB */
      __syncthreads();
      if ((lkey & pmask) == prefix) atomicAdd(&S.hist[(lkey >> shift) & 255u], 1u);
      __syncthreads();
      const BinSel bs = wave_find_bin<false>(S.hist, need); /* 256 keys >= need */
      prefix |= bs.bin << shift;
      pmask |= 0xffu << shift;
      need -= bs.above;
      __syncthreads(); /* every wave has read the histogram */
    }
    bool over = (a.flags & FLAG_EXACT_SELECT) != 0;
    /* below every logit whose x ties with tau's (as in the one-wave kernel);
     * when the k-th lane max is -inf, every finite logit is a candidate (a
     * row that needs x = -inf keys is sampled by the generic procedure) */
    const float tau = d3s_from_ordkey(prefix);
    const float tau_lo = prefix < d3s_ordkey(-0x1.fffffep127f) ? -0x1.fffffep127f
                                                              : tau - (fabsf(tau) * 0x1p-21f + T * 0x1p-120f);
    /* a threshold at -inf would take masked padding for candidates */
    if (!(tau_lo >= -0x1.fffffep127f)) over = true;

    /* ---- the candidates as a bit per element, no branches */
    if (BF16) c.launder();
    constexpr int NWORD = (NV + 31) / 32;
    uint32_t bits[NWORD];
#pragma unroll
    for (int w = 0; w < NWORD; w++) bits[w] = 0u;
#pragma unroll
    for (int i = 0; i < NV; i++) {
      asm("v_cmp_ge_f32 vcc, %1, %2\n\ts_nop 1\n\tv_addc_co_u32 %0, vcc, %0, %0, vcc"
          : "+v"(bits[i / 32])
          : "v"(c.val(i)), "v"(tau_lo)
          : "vcc");
    }
    if (NV % 32) bits[NWORD - 1] <<= 32 - NV % 32;
    int cnt = 0;
#pragma unroll
    for (int w = 0; w < NWORD; w++) cnt += __popc(bits[w]);
    const uint32_t wtot = wave_sum_u32((uint32_t)cnt);
    over = over || __ballot(cnt > LCAP) != 0ull;
    auto next_cand = [&]() {
      int i = 0;
      bool found = false;
#pragma unroll
      for (int w = 0; w < NWORD; w++) {
        const int e = __builtin_clz(bits[w] | 1u); /* bits[w] != 0 below */
        const bool here = !found && bits[w] != 0u;
        i = here ? 32 * w + e : i;
        bits[w] = here ? bits[w] & ~(0x80000000u >> e) : bits[w];
        found = found || here;
      }
      return C::pos(pos0, i);
    };
    auto read_logit = [&](int p) {
      return BF16 ? d3s_bf16_to_f32(((const uint16_t *)rowp)[p]) : ((const float *)rowp)[p];
    };
    /* the first candidates read again now, while the segment is in L2 */
    int cpos[EARLY];
    float cl[EARLY];
#pragma unroll
    for (int q = 0; q < EARLY; q++) {
      cpos[q] = 0;
      cl[q] = 0.0f;
    }
    if (!over) {
#pragma unroll
      for (int q = 0; q < EARLY; q++) {
        if (q > 0 && !__ballot(q < cnt)) break;
        cpos[q] = next_cand();
        if (q < cnt) cl[q] = read_logit(cpos[q]);
      }
    }

    /* ---- the segment's fast sum, relative to its own max */
    if (BF16) c.launder();
    float acc[EPC];
#pragma unroll
    for (int e = 0; e < EPC; e++) acc[e] = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; i++) acc[i % EPC] += __builtin_amdgcn_exp2f(__builtin_fmaf(c.val(i), cf, b));
#pragma unroll
    for (int w = EPC / 2; w >= 1; w /= 2)
#pragma unroll
      for (int e = 0; e < w; e++) acc[e] = acc[e] + acc[e + w];
    {
      const float ws = wave_sum_f(acc[0]);
      if (lane == 0) {
        S.wsum[wid] = ws;
        S.wcnt[wid] = over ? 0xffffffffu : wtot;
      }
    }
    __syncthreads();
    uint32_t tot = 0u, base = 0u;
    ssum = S.wsum[0];
#pragma unroll
    for (int w = 0; w < SPLIT_NW; w++) {
      const uint32_t t = S.wcnt[w];
      over = over || t == 0xffffffffu;
      base += w < wid ? t : 0u;
      tot += t;
      if (w > 0) ssum = ssum + S.wsum[w]; /* the same order in every wave */
    }
    over = over || tot > (uint32_t)SCAP;
    if (over) {
      flags |= SEG_OVERFLOW;
    } else {
      /* ---- file the keys, rank them, keep the top k */
      const uint32_t excl = base + wave_scan_add_u32((uint32_t)cnt) - (uint32_t)cnt;
#pragma unroll
      for (int q = 0; q < EARLY; q++)
        if (q < cnt) S.keys[excl + q] = composite_key(scale_logit(cl[q], T, y, true), cpos[q]);
#pragma unroll 1
      for (int q = EARLY; q < LCAP; q++) {
        if (!__ballot(q < cnt)) break;
        const int p = next_cand();
        if (q < cnt) S.keys[excl + q] = composite_key(scale_logit(read_logit(p), T, y, true), p);
      }
      split_rank(S, tot, k);
      nfiled = min(tot, (uint32_t)k);
    }
  }

  /* ---- publish the record: agent-coherent stores, completed before the
   * arrival is counted */
  uint64_t *rec = records + ((size_t)row * nseg + seg) * rec_words;
  if (threadIdx.x < nfiled) st_agent(rec + 2 + threadIdx.x, S.ranked[threadIdx.x]);
  if (threadIdx.x == 0) {
    st_agent(rec, (uint64_t)d3s_f2u(Ls) | ((uint64_t)d3s_f2u(ssum) << 32));
    st_agent(rec + 1, (uint64_t)flags | ((uint64_t)nfiled << 32));
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t *cnt_row = counters_ws + (size_t)row * 32; /* one counter per 128 bytes */
    const uint32_t old = __hip_atomic_fetch_add(cnt_row, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    S.last = old == (uint32_t)(nseg - 1);
    if (S.last) __hip_atomic_store(cnt_row, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    S.exact = 0u;
  }
  __syncthreads();
  if (!S.last) return;

  /* ---- the last arrival merges the row's records */
  const uint64_t *rrow = records + (size_t)row * nseg * rec_words;
  if (threadIdx.x < (unsigned)nseg) {
    const uint64_t h0 = ld_agent(rrow + (size_t)threadIdx.x * rec_words);
    const uint64_t h1 = ld_agent(rrow + (size_t)threadIdx.x * rec_words + 1);
    S.smax[threadIdx.x] = d3s_u2f((uint32_t)h0);
    S.ssum[threadIdx.x] = d3s_u2f((uint32_t)(h0 >> 32));
    S.sflags[threadIdx.x] = (uint32_t)h1;
    S.sn[threadIdx.x] = (uint32_t)(h1 >> 32);
  }
  __syncthreads();
  float Lmax = S.smax[0];
  uint32_t F = S.sflags[0], total = S.sn[0];
  for (int s = 1; s < nseg; s++) {
    Lmax = fmaximum(Lmax, S.smax[s]);
    F |= S.sflags[s];
    total += S.sn[s];
  }
  if (d3s_isnan(Lmax) || Lmax == __builtin_inff()) {
    if (wid == 0) wave_write_special(a, row, false);
    return;
  }
  if (Lmax == ninf) {
    if (wid == 0) wave_write_special(a, row, true);
    return;
  }
  const float M = t_finite ? scale_logit(Lmax, T, y, true) : 0.0f; /* = max x */
  if (t_finite && (M == __builtin_inff() || M == ninf)) {
    if (wid == 0) wave_write_special(a, row, M == ninf);
    return;
  }
  if ((F & SEG_GENERIC) || (F & SEG_OVERFLOW) || total < (uint32_t)k) {
    if ((F & SEG_OVERFLOW) && !(F & SEG_GENERIC) && threadIdx.x == 0 && a.counters)
      atomicAdd(&a.counters[CNT_EXACT_SELECT], 1u);
    generic_row<BF16, SPLIT_T>(a, row, kpow, glist);
    return;
  }
  /* the segments' keys, at offsets in segment order */
  for (int i = threadIdx.x; i < nseg * KF; i += SPLIT_T) {
    const int s = i / KF, j = i % KF;
    if ((uint32_t)j < S.sn[s]) {
      uint32_t o = 0u;
      for (int q = 0; q < s; q++) o += S.sn[q];
      S.keys[o + j] = ld_agent(rrow + (size_t)s * rec_words + 2 + j);
    }
  }
  /* the rescaled fast sum and its error bound: the segment holding the max
   * contributes 2^delta (about 1); segment s's terms were taken relative to
   * h_s = RN(Ls cf) and are scaled by 2^(h_s - h) (hardware 2^x of the rounded
   * difference).  Weighted by its share (at most CAP * EPC 2^(h_s - h), capped
   * at 1), each segment adds its own term-rounding bound and the rescale's. */
  const float cfr = LOG2E_F / T;
  const float h = Lmax * cfr;
  const float delta = __builtin_fmaf(Lmax, cfr, -h); /* Lmax * cf - h exactly */
  float sp = 0.0f, eps_seg = 0.0f;
  for (int s = 0; s < nseg; s++) {
    const float Lm = S.smax[s];
    if (Lm == ninf) continue;
    const float d = Lm * cfr - h; /* <= 0 */
    const float f = __builtin_amdgcn_exp2f(d);
    sp = sp + S.ssum[s] * f;
    const float w = fminf(1.0f, (float)(CAP * EPC) * f);
    eps_seg = eps_seg + w * (0x1p-24f * (2.0f * fabsf(Lm) * y + 160.0f) + 0x1p-24f * fabsf(d) + EPS_EXP2);
  }
  const float l2 = __builtin_amdgcn_logf(sp); /* within 2^-23 |log2 sp| + 2^-24 */
  const float lse = M + (l2 * LN2_F - delta * LN2_F);
  /* the one-wave kernel's bound (its term for the max's rounding is in
   * eps_seg), with each segment's SPLIT_NW additions, the nseg products and
   * additions of the rescale, and eps_seg */
  const float eps_s = EPS_EXP2 + 0x1p-23f + (float)(CPT + 11 + SPLIT_NW + 2 * nseg) * 0x1p-24f +
                      (float)V * 0x1p-40f + 0x1p-22f * fabsf(l2) + 0x1p-23f + eps_seg;
  split_rank(S, total, k);
  if (key_x(S.ranked[k - 1]) == ninf) { /* the top k reach x = -inf: ties the segments did not file */
    generic_row<BF16, SPLIT_T>(a, row, kpow, glist);
    return;
  }
  /* ---- the tail on wave 0; a cut within the margin takes the exact lse */
  const float uval = (wid == 0 && lane < k) ? a.u[(size_t)row * k + lane] : 0.0f;
  const float noise = -d3s_logf(1.0f - uval);
  const uint64_t key = lane < k ? S.ranked[lane] : 0ull;
  if (wid == 0) {
    const int id = wave_tail(a, row, key, M, lse, false, eps_s, noise, top_p, S.buf,
                             []() { return __builtin_nanf(""); });
    if (id == NEED_EXACT && lane == 0) S.exact = 1u;
  }
  __syncthreads();
  if (!S.exact) return;
  const float lx = split_exact_lse<BF16>(a, row, M, S);
  if (wid == 0) (void)wave_tail(a, row, key, M, lx, true, 0.0f, noise, top_p, S.buf, []() { return 0.0f; });
}

template <int CPT, bool BF16>
bool try_split(const SampleArgs &a, int nseg, void *ws, size_t ws_bytes, hipStream_t s) {
  if (nseg < 2 || nseg > SPLIT_MAX_SEG) return false;
  const size_t cnt_bytes = ((size_t)a.n_rows * 128 + 255) & ~(size_t)255;
  const int rec_words = 2 + KF;
  const size_t need = cnt_bytes + (size_t)a.n_rows * nseg * rec_words * 8;
  if (!ws || need > ws_bytes) return false;
  hipLaunchKernelGGL((k_split<CPT, BF16>), dim3((unsigned)(a.n_rows * nseg)), dim3(SPLIT_T), 0, s, a,
                     (uint32_t *)ws, (uint64_t *)((char *)ws + cnt_bytes), nseg, rec_words);
  return true;
}

}  // namespace

int split_segments(const SampleArgs &a, Dtype dt) {
  const int EPC = dt == DT_F32 ? 4 : 8;
  const int cap = SPLIT_NW * SPLIT_CPT * WAVE;
  const int nchunks = (EPC - 1 + a.vocab + EPC - 1) / EPC; /* any start offset */
  const int nseg = (nchunks + cap - 1) / cap;
  return (a.k > KF || nseg < 2 || nseg > SPLIT_MAX_SEG) ? 0 : nseg;
}

size_t split_workspace_bytes(const SampleArgs &a, Dtype dt) {
  const int nseg = split_segments(a, dt);
  if (!nseg) return 0;
  return (((size_t)a.n_rows * 128 + 255) & ~(size_t)255) + (size_t)a.n_rows * nseg * (2 + KF) * 8;
}

bool launch_split(const SampleArgs &a, Dtype dt, void *ws, size_t ws_bytes, hipStream_t s) {
  const int nseg = split_segments(a, dt);
  if (!nseg) return false;
  return dt == DT_F32 ? try_split<SPLIT_CPT, false>(a, nseg, ws, ws_bytes, s)
                      : try_split<SPLIT_CPT, true>(a, nseg, ws, ws_bytes, s);
}

}  // namespace d3s
