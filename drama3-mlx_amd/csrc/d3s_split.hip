/* k_split: rows too wide for one wave (k <= 64) cut into segments, every
 * segment of every row in one launch (gfx950, wave64).
 *
 * A segment is SPLIT_NW waves x 64 lanes x CPT 16-byte chunks of the row, one
 * workgroup.  It runs the one-wave kernel's passes on its part (registers,
 * NaN-propagating max, a threshold that at least k of its lane maxima reach:
 * the least of its waves' ceil(k / SPLIT_NW)-th largest, candidate chunks,
 * the fast sum 2^(L c - h_s) relative to its own max)
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

constexpr int SPLIT_NW = 8;              /* waves per segment (two per SIMD) */
constexpr int SPLIT_CPT = 8;             /* 16-byte chunks per lane */
constexpr int SPLIT_CPT_WIDE = 10;       /* the wider form, when it fills the CUs more evenly */
constexpr int SPLIT_CPT_LONG = 19;       /* the longest form */
constexpr int SPLIT_T = SPLIT_NW * WAVE; /* threads per segment */
constexpr int SCAP = SPLIT_T;            /* candidates a segment ranks (one per thread) */
constexpr int SPLIT_MAX_SEG = 16;        /* segments per row */
constexpr int SPLIT_MAX_BLOCKS = 4096;   /* segments per launch */
/* The workspace: arrival counters (one per 128 bytes) for the most rows a
 * launch can have, then the records.  The counters' place never depends on
 * the launch, so records of one launch never land on another's counters. */
constexpr size_t SPLIT_CNT_BYTES = (size_t)(SPLIT_MAX_BLOCKS / 2) * 128;
constexpr int MCAP = SPLIT_MAX_SEG * KF; /* keys the merger ranks */

/* record flags */
constexpr uint32_t SEG_GENERIC = 1u;  /* T not finite or logits too large: the generic procedure */
constexpr uint32_t SEG_OVERFLOW = 2u; /* more candidates than the segment files (or forced) */

struct __align__(16) SplitLds {
  uint64_t keys[MCAP + 2]; /* a segment's candidates; the merger's keys at or above its cut (+ zero pads) */
  uint64_t kth[SPLIT_MAX_SEG]; /* the merger's k-th key of each segment */
  uint64_t kc[SPLIT_MAX_SEG];  /* the merger's ceil(k / nseg)-th key of each segment */
  uint64_t ranked[KF];
  uint32_t lk[SPLIT_T];        /* order keys of the lane maxima */
  float buf[WAVE];
  float wmax[SPLIT_NW], wsum[SPLIT_NW];
  uint32_t wpre[SPLIT_NW];
  uint32_t wcnt[SPLIT_NW];         /* pairs each wave filed (all ones: more than its region) */
  uint4 stage[SPLIT_NW * WAVE];    /* each wave's candidate chunks */
  uint32_t spos[SPLIT_NW * WAVE];  /* their first positions */
  uint64_t raw[SPLIT_NW * WAVE];   /* each wave's (logit bits, position) pairs */
  float smax[SPLIT_MAX_SEG], ssum[SPLIT_MAX_SEG];
  uint32_t sflags[SPLIT_MAX_SEG], sn[SPLIT_MAX_SEG];
  uint32_t last, exact, mcount;
  uint32_t slo[SPLIT_NW], shi[SPLIT_NW];
};

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

/* wave_kth_prefix over the SPLIT_T keys of a workgroup held in LDS, by
 * every wave */
__device__ __forceinline__ uint32_t group_kth_prefix(const uint32_t *keys, uint32_t k) {
  const int lane = lane_id();
  uint32_t kk[SPLIT_NW];
#pragma unroll
  for (int w = 0; w < SPLIT_NW; w++) kk[w] = keys[w * WAVE + lane];
  uint32_t pre = 0u;
#pragma unroll
  for (int bit = 31; bit >= 12; bit--) {
    const uint32_t cnd = pre | (1u << bit);
    uint32_t c = 0u;
#pragma unroll
    for (int w = 0; w < SPLIT_NW; w++) c += (uint32_t)__popcll(__ballot(kk[w] >= cnd));
    if (c >= k) pre = cnd;
  }
  return pre;
}

/* wave maximum of 64-bit values (the high words, then the low words of the
 * lanes that hold the highest); wave-uniform */
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  auto wmax = [](uint32_t x) {
    x = max(x, dpp_u<DPP_SHR1, 0xf>(0u, x));
    x = max(x, dpp_u<DPP_SHR2, 0xf>(0u, x));
    x = max(x, dpp_u<DPP_SHR4, 0xf>(0u, x));
    x = max(x, dpp_u<DPP_SHR8, 0xf>(0u, x));
    x = max(x, dpp_u<DPP_BCAST15, 0xa>(0u, x));
    x = max(x, dpp_u<DPP_BCAST31, 0xc>(0u, x));
    return readlane_u(x, 63);
  };
  const uint32_t hi = wmax((uint32_t)(v >> 32));
  const uint32_t lo = wmax((uint32_t)(v >> 32) == hi ? (uint32_t)v : 0u);
  return ((uint64_t)hi << 32) | lo;
}

/* The leading scalar arguments (preloaded into SGPRs at wave launch): the
 * fields a segment's loads and first steps need, and nseg, which places the
 * segment; 48 bytes.  The SampleArgs block's copies are replaced by them. */
template <int CPT, bool BF16>
__global__ __launch_bounds__(SPLIT_T) void k_split(const void *hot_logits, int64_t hot_stride,
                                                   const int32_t *hot_banned, const float *hot_temperature,
                                                   float hot_T, int hot_vocab, int hot_k, int nseg, SampleArgs a,
                                                   uint32_t *counters_ws, uint64_t *records, int rec_words) {
  a.logits = hot_logits;
  a.row_stride = hot_stride;
  a.banned = hot_banned;
  a.temperature = hot_temperature;
  a.temperature_scalar = hot_T;
  a.vocab = hot_vocab;
  a.k = hot_k;
  using C = Chunks<CPT, BF16>;
  constexpr int ES = BF16 ? 2 : 4, EPC = C::EPC, NV = C::NV;
  constexpr int CAP = SPLIT_NW * CPT * WAVE; /* chunks per segment */
  __shared__ SplitLds S;
  __shared__ uint64_t glist[KF]; /* the generic procedure's sort list */
  const int row = (int)blockIdx.x / nseg, seg = (int)blockIdx.x % nseg;
  const int wid = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / WAVE));
  const int lane = lane_id();
  const int V = a.vocab, k = a.k;
  int kpow = 2;
  while (kpow < k) kpow <<= 1;
  const char *rowp = (const char *)a.logits + (size_t)row * (size_t)a.row_stride * ES;
  const int off = (int)(((uintptr_t)rowp & 15u) / ES);
  const uint4 *src = (const uint4 *)(rowp - off * ES);
  const int nchunks = (off + V + EPC - 1) / EPC;
  /* the row's chunks in nseg equal parts (at most CAP each), each part in
   * SPLIT_NW equal runs, one per wave: every wave holds as many logits as the
   * others (the per-wave thresholds below assume it) */
  const int segc = (nchunks + nseg - 1) / nseg;
  const int wch = (segc + SPLIT_NW - 1) / SPLIT_NW;                  /* chunks per wave */
  const int cend = min(nchunks, (seg + 1) * segc);                   /* past the segment's last chunk */
  const int cbase = seg * segc + wid * wch;                          /* this wave's first chunk */
  const int wend = min(cend, cbase + wch);                           /* past its last */
  const int vend = min(V, wend * EPC - off);                         /* past its last position */
  C c;
  c.load(src + cbase, min(max(wend - cbase, 0), CPT * WAVE), lane);
  /* the row's parameters after its loads are issued (these may wait on the
   * kernarg segment) */
  const RowP rp = row_params(a, row);
  const float T = rp.T, top_p = rp.top_p;
  const int banned = rp.banned;
  const bool t_finite = T < __builtin_inff(); /* false for +inf and NaN */
  const float y = 1.0f / T;
  const int pos0 = (cbase + lane) * EPC - off;
  auto valid = [&](int i) { return (unsigned)C::pos(pos0, i) < (unsigned)vend; };
#pragma unroll
  for (int j = 0; j < CPT; j++) {
    const int p_lo = (cbase + j * WAVE) * EPC - off; /* wave-uniform */
    if (p_lo < 0 || p_lo + WAVE * EPC > vend) {
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

  /* ---- each chunk's max, the segment's max (NaN propagates) and, per wave,
   * the ceil(k / SPLIT_NW)-th largest of its lane maxima */
  const float ninf = -__builtin_inff();
  float cm[CPT];
  float lm = ninf;
#pragma unroll
  for (int j = 0; j < CPT; j++) {
    float m = c.val(j * EPC);
#pragma unroll
    for (int e = 1; e < EPC; e++) m = fmaximum(m, c.val(j * EPC + e));
    cm[j] = m;
    lm = fmaximum(lm, m);
  }
  const uint32_t lkey = d3s_ordkey(lm);
  {
    const float wm = wave_maximum_f(lm);
    const uint32_t wp = wave_kth_prefix(lkey, (uint32_t)(k + SPLIT_NW - 1) / SPLIT_NW);
    if (lane == 0) {
      S.wmax[wid] = wm;
      S.wpre[wid] = wp;
    }
    S.lk[threadIdx.x] = lkey;
  }
  __syncthreads();
  float Ls = S.wmax[0];
  uint32_t prefix = S.wpre[0];
#pragma unroll
  for (int w = 1; w < SPLIT_NW; w++) {
    Ls = fmaximum(Ls, S.wmax[w]);
    prefix = min(prefix, S.wpre[w]);
  }
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
    /* ---- tau, a lower bound with at least k elements reaching it: the least
     * of the waves' prefixes (SPLIT_NW ceil(k / SPLIT_NW) >= k lane maxima
     * reach it).  When a wave holds fewer finite lane maxima than its share
     * (a segment past the row's end, or -inf logits), the k-th largest of all
     * the segment's lane maxima instead. */
    if (prefix < d3s_ordkey(-0x1.fffffep127f)) prefix = group_kth_prefix(S.lk, (uint32_t)k);
    bool over = (a.flags & FLAG_EXACT_SELECT) != 0;
    /* below every logit whose x ties with tau's (as in the one-wave kernel);
     * when the k-th lane max is -inf, every finite logit is a candidate (a
     * row that needs x = -inf keys is sampled by the generic procedure) */
    const float tau = d3s_from_ordkey(prefix);
    const float tau_lo = prefix < d3s_ordkey(-0x1.fffffep127f) ? -0x1.fffffep127f
                                                              : tau - (fabsf(tau) * 0x1p-21f + T * 0x1p-120f);
    /* a threshold at -inf would take masked padding for candidates */
    if (!(tau_lo >= -0x1.fffffep127f)) over = true;

    /* ---- the candidate chunks (their max reaches tau_lo), one bit each */
    uint32_t cb = 0u;
#pragma unroll
    for (int j = 0; j < CPT; j++) cb |= (cm[j] >= tau_lo ? 1u : 0u) << j;
    if (over) cb = 0u;

    /* ---- the segment's fast sum, relative to its own max */
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
      if (lane == 0) S.wsum[wid] = ws;
    }

    /* ---- file the candidates in one pass: each wave stages its candidate
     * chunks in LDS (slots by a wave scan), lane t takes staged chunk t and
     * files its valid elements that reach tau_lo as (logit bits, position)
     * pairs in the wave's region; the keys are made after the barrier, one
     * per thread.  A wave with more than 64 chunks or pairs overflows. */
    {
      const uint32_t nc = (uint32_t)__popc(cb);
      const uint32_t cinc = wave_scan_add_u32(nc);
      const uint32_t wchunks = readlane_u(cinc, 63);
      uint32_t slot = cinc - nc;
      uint4 *stg = S.stage + wid * WAVE;
      uint32_t *sps = S.spos + wid * WAVE;
#pragma unroll
      for (int j = 0; j < CPT; j++)
        if ((cb >> j) & 1u) {
          if (slot < (uint32_t)WAVE) {
            stg[slot] = make_uint4(c.w[4 * j], c.w[4 * j + 1], c.w[4 * j + 2], c.w[4 * j + 3]);
            sps[slot] = (uint32_t)C::pos(pos0, j * EPC);
          }
          slot++;
        }
      wave_lds_sync();
      float v[EPC];
      uint32_t vm = 0u, pb = 0u;
      if ((uint32_t)lane < min(wchunks, (uint32_t)WAVE)) {
        const uint4 q = stg[lane];
        const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
        pb = sps[lane];
#pragma unroll
        for (int e = 0; e < EPC; e++) {
          v[e] = BF16 ? d3s_u2f((e & 1) ? (qw[e / 2] & 0xffff0000u) : (qw[e / 2] << 16)) : d3s_u2f(qw[e]);
          vm |= (v[e] >= tau_lo ? 1u : 0u) << e; /* masked elements hold -inf */
        }
      }
      const uint32_t ne = (uint32_t)__popc(vm);
      const uint32_t einc = wave_scan_add_u32(ne);
      const uint32_t wpairs = readlane_u(einc, 63);
      uint32_t at = einc - ne;
      uint64_t *rw = S.raw + wid * WAVE;
#pragma unroll
      for (int e = 0; e < EPC; e++)
        if ((vm >> e) & 1u) {
          if (at < (uint32_t)WAVE) rw[at] = ((uint64_t)d3s_f2u(v[e]) << 32) | (pb + (uint32_t)e);
          at++;
        }
      if (lane == 0) S.wcnt[wid] = wchunks > (uint32_t)WAVE || wpairs > (uint32_t)WAVE ? 0xffffffffu : wpairs;
    }
    __syncthreads();
    ssum = S.wsum[0];
#pragma unroll
    for (int w = 1; w < SPLIT_NW; w++) ssum = ssum + S.wsum[w]; /* the same order in every wave */
    uint32_t tot = 0u;
#pragma unroll
    for (int w = 0; w < SPLIT_NW; w++) {
      const uint32_t t = S.wcnt[w];
      over = over || t == 0xffffffffu;
      tot += t == 0xffffffffu ? 0u : t;
    }
    if (over || tot > (uint32_t)SCAP) {
      flags |= SEG_OVERFLOW;
    } else {
      /* ---- the keys, one per thread (from the waves' regions in wave
       * order); rank them, keep the top k */
      if (threadIdx.x < tot) {
        uint32_t t = threadIdx.x;
        int w = 0;
#pragma unroll
        for (int q = 0; q < SPLIT_NW - 1; q++)
          if (w == q && t >= S.wcnt[q]) {
            t -= S.wcnt[q];
            w = q + 1;
          }
        const uint64_t lp = S.raw[w * WAVE + t];
        S.keys[threadIdx.x] = composite_key(scale_logit(d3s_u2f((uint32_t)(lp >> 32)), T, y, true), (int)(uint32_t)lp);
      }
      /* ranked straight into the record's key slots */
      rank_by_count<SPLIT_T, true>(S.keys, tot, k, records + ((size_t)row * nseg + seg) * rec_words + 2);
      nfiled = min(tot, (uint32_t)k);
    }
  }

  /* ---- publish the record: agent-coherent stores, completed before the
   * arrival is counted (the ordering argument is at st_agent) */
  uint64_t *rec = records + ((size_t)row * nseg + seg) * rec_words;
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
    S.mcount = 0u;
  }
  __syncthreads();
  if (!S.last) return;

  /* ---- the last arrival merges the row's records: every word of them read
   * at once (one round trip), the key of rank r of segment s in slot q of
   * thread t (t + q SPLIT_T = r SPLIT_MAX_SEG + s), the headers by the first
   * 2 nseg threads; the uniforms of wave 0 as well */
  const uint64_t *rrow = records + (size_t)row * nseg * rec_words;
  const int kc = (k + nseg - 1) / nseg;
  constexpr int PK = (KF * SPLIT_MAX_SEG + SPLIT_T - 1) / SPLIT_T;
  uint64_t kv[PK];
#pragma unroll
  for (int q = 0; q < PK; q++) {
    const int i = (int)threadIdx.x + q * SPLIT_T, r = i / SPLIT_MAX_SEG, sg = i % SPLIT_MAX_SEG;
    kv[q] = sg < nseg && r < k ? ld_agent(rrow + sg * rec_words + 2 + r) : 0ull;
  }
  const int ht = (int)threadIdx.x;
  const uint64_t hv = ht < 2 * nseg ? ld_agent(rrow + (ht >> 1) * rec_words + (ht & 1)) : 0ull;
  const float uval = (wid == 0 && lane < k) ? a.u[(size_t)row * k + lane] : 0.0f;
  const float noise = -d3s_logf(1.0f - uval); /* off the tail's path */
#pragma unroll
  for (int q = 0; q < PK; q++) {
    const int i = (int)threadIdx.x + q * SPLIT_T, r = i / SPLIT_MAX_SEG, sg = i % SPLIT_MAX_SEG;
    if (sg < nseg && r == k - 1) S.kth[sg] = kv[q];
    if (sg < nseg && r == kc - 1) S.kc[sg] = kv[q];
  }
  if (ht < 2 * nseg) {
    if (ht & 1) {
      S.sflags[ht >> 1] = (uint32_t)hv;
      S.sn[ht >> 1] = (uint32_t)(hv >> 32);
    } else {
      S.smax[ht >> 1] = d3s_u2f((uint32_t)hv);
      S.ssum[ht >> 1] = d3s_u2f((uint32_t)(hv >> 32));
    }
  }
  __syncthreads();
  /* every wave reduces the headers, lane s holding segment s: the row max,
   * the flags, the keys filed, and a cut the row's k-th key reaches: T0, the
   * largest k-th key of a segment that filed k (that segment alone has k keys
   * at or above it), and T1, the least kc-th key, kc = ceil(k / nseg), when
   * the segments that filed kc or more hold k keys at or above it */
  const bool ls = lane < nseg;
  const int sl = ls ? lane : 0;
  const float lm_s = ls ? S.smax[sl] : ninf;
  const uint32_t fl_s = ls ? S.sflags[sl] : 0u, n_s = ls ? S.sn[sl] : 0u;
  const float Lmax = wave_maximum_f(lm_s);
  const uint32_t F = (__ballot(fl_s & SEG_GENERIC) ? SEG_GENERIC : 0u) | (__ballot(fl_s & SEG_OVERFLOW) ? SEG_OVERFLOW : 0u);
  const uint32_t total = wave_sum_u32(n_s);
  const uint64_t T0 = wave_max_u64(ls && n_s == (uint32_t)k ? S.kth[sl] : 0ull);
  const bool has_c = ls && n_s >= (uint32_t)kc;
  const uint64_t T1 = ~wave_max_u64(has_c ? ~S.kc[sl] : 0ull); /* the least */
  const uint64_t cut = (uint32_t)__popcll(__ballot(has_c)) * (uint32_t)kc >= (uint32_t)k ? max(T0, T1) : T0;
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
  bool generic = (F & SEG_GENERIC) || (F & SEG_OVERFLOW) || total < (uint32_t)k;
  if ((F & SEG_OVERFLOW) && !(F & SEG_GENERIC) && threadIdx.x == 0 && a.counters)
    atomicAdd(&a.counters[CNT_EXACT_SELECT], 1u);
  float lse = 0.0f, eps_s = 0.0f;
  if (!generic) {
    /* the rescaled fast sum and its error bound: the segment holding the max
     * contributes 2^delta (about 1); segment s's terms were taken relative to
     * h_s = RN(Ls cf) and are scaled by 2^(h_s - h) (hardware 2^x of the
     * rounded difference).  Weighted by its share (at most CAP * EPC
     * 2^(h_s - h), capped at 1), each segment adds its own term-rounding bound
     * and the rescale's.  Lane s takes segment s; the wave sums them
     * (non-negative terms: within the bound of nseg - 1 additions in any
     * order). */
    const float cfr = LOG2E_F / T;
    const float h = Lmax * cfr;
    const float delta = __builtin_fmaf(Lmax, cfr, -h); /* Lmax * cf - h exactly */
    float term = 0.0f, eterm = 0.0f;
    if (ls && lm_s != ninf) {
      const float d = lm_s * cfr - h; /* <= 0 */
      const float f = __builtin_amdgcn_exp2f(d);
      term = S.ssum[sl] * f;
      const float w = fminf(1.0f, (float)(CAP * EPC) * f);
      eterm = w * (0x1p-24f * (2.0f * fabsf(lm_s) * y + 160.0f) + 0x1p-24f * fabsf(d) + EPS_EXP2);
    }
    const float sp = wave_sum_f(term);
    const float eps_seg = wave_sum_f(eterm) * (1.0f + 0x1p-20f); /* the bound's own rounding */
    const float l2 = __builtin_amdgcn_logf(sp); /* within 2^-23 |log2 sp| + 2^-24 */
    lse = M + (l2 * LN2_F - delta * LN2_F);
    /* the one-wave kernel's bound (its term for the max's rounding is in
     * eps_seg), with each segment's SPLIT_NW additions, the nseg products and
     * additions of the rescale, and eps_seg */
    eps_s = EPS_EXP2 + 0x1p-23f + (float)(CPT + 11 + SPLIT_NW + 2 * nseg) * 0x1p-24f + (float)V * 0x1p-40f +
            0x1p-22f * fabsf(l2) + 0x1p-23f + eps_seg;
    /* ---- the row's top k: the filed keys at or above the cut (at most nseg
     * k of them; k or more by the cut's choice), ranked by counting */
#pragma unroll
    for (int q = 0; q < PK; q++) {
      const int i = (int)threadIdx.x + q * SPLIT_T, r = i / SPLIT_MAX_SEG, sg = i % SPLIT_MAX_SEG;
      const bool take = sg < nseg && (uint32_t)r < S.sn[sg < nseg ? sg : 0] && kv[q] >= cut;
      const int at = wave_append(take, (int *)&S.mcount);
      if (take) S.keys[at] = kv[q];
    }
    __syncthreads();
    rank_by_count<SPLIT_T>(S.keys, S.mcount, k, S.ranked);
    /* the top k reach x = -inf: ties the segments did not file */
    generic = key_x(S.ranked[k - 1]) == ninf;
  }
  if (generic) {
    generic_row<BF16, SPLIT_T>(a, row, kpow, glist);
    return;
  }
  /* ---- the tail on wave 0; a cut within the margin takes the exact lse (by
   * the whole workgroup) and the tail again */
  const uint64_t key = lane < k ? S.ranked[lane] : 0ull;
  bool exact = false;
#pragma unroll 1
  for (;;) {
    if (wid == 0) {
      const int id = wave_tail(a, row, key, M, lse, exact, eps_s, noise, top_p, S.buf,
                               []() { return __builtin_nanf(""); });
      if (id == NEED_EXACT && lane == 0) S.exact = 1u;
    }
    __syncthreads();
    if (exact || !S.exact) return;
    lse = split_exact_lse<BF16>(a, row, M, S);
    exact = true;
  }
}

template <int CPT, bool BF16>
bool try_split(const SampleArgs &a, int nseg, void *ws, size_t ws_bytes, hipStream_t s) {
  if (nseg < 2 || nseg > SPLIT_MAX_SEG || (int64_t)a.n_rows * nseg > SPLIT_MAX_BLOCKS) return false;
  const int rec_words = 2 + a.k; /* header, then the keys by rank */
  const size_t need = SPLIT_CNT_BYTES + (size_t)a.n_rows * nseg * rec_words * 8;
  if (!ws || need > ws_bytes) return false;
  hipLaunchKernelGGL((k_split<CPT, BF16>), dim3((unsigned)(a.n_rows * nseg)), dim3(SPLIT_T), 0, s, a.logits,
                     a.row_stride, a.banned, a.temperature, a.temperature_scalar, a.vocab, a.k, nseg, a,
                     (uint32_t *)ws, (uint64_t *)((char *)ws + SPLIT_CNT_BYTES), rec_words);
  return true;
}

}  // namespace

size_t split_counter_bytes() { return SPLIT_CNT_BYTES; }

namespace {

/* compute units of the current device (queried once per device) */
int device_cus() {
  static int cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cus[dev]) {
    int n = 0;
    cus[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
  }
  return cus[dev];
}

struct SplitShape {
  int cpt, nseg; /* nseg 0: the segmented kernel does not take the rows */
};

/* The segments' form for these rows: SPLIT_CPT chunks per lane, or a longer
 * form (SPLIT_CPT_WIDE, SPLIT_CPT_LONG: fewer, longer segments) when its
 * launch fits in one round and fills whole rounds of the CUs at least as
 * evenly; of equal fills the fewest segments (the merge has fewer records).
 * Workgroups per CU by registers (eight-wave workgroups): bf16 two and one
 * for 8 and 10 chunks (19 bf16 chunks, 152 elements a lane, measured slower
 * than more segments: not taken); fp32 three, three and two.  A row's merge
 * waits for its slowest segment, and a CU holding one workgroup more than
 * the others makes that segment slow. */
SplitShape split_shape(const SampleArgs &a, Dtype dt) {
  const int EPC = dt == DT_F32 ? 4 : 8;
  const int nchunks = (EPC - 1 + a.vocab + EPC - 1) / EPC; /* any start offset */
  const int cus = device_cus();
  SplitShape best{SPLIT_CPT, 0};
  double best_fill = -1.0;
  int64_t best_blocks = 0;
  for (const int cpt : {SPLIT_CPT, SPLIT_CPT_WIDE, SPLIT_CPT_LONG}) {
    const int cap = SPLIT_NW * cpt * WAVE;
    const int nseg = (nchunks + cap - 1) / cap;
    const int64_t blocks = (int64_t)a.n_rows * nseg;
    if (a.k > KF || nseg < 2 || nseg > SPLIT_MAX_SEG || blocks > SPLIT_MAX_BLOCKS) continue;
    const int per_cu = dt == DT_BF16 ? (cpt == SPLIT_CPT ? 2 : cpt == SPLIT_CPT_WIDE ? 1 : 0)
                                     : (cpt == SPLIT_CPT_LONG ? 2 : 3);
    if (cpt != SPLIT_CPT && blocks > (int64_t)cus * per_cu) continue;
    const int64_t rounds = (blocks + cus - 1) / cus;
    const double fill = (double)blocks / (double)(rounds * cus);
    if (fill > best_fill + 1e-9 || (fill > best_fill - 1e-9 && blocks < best_blocks)) {
      best = SplitShape{cpt, nseg};
      best_fill = fill;
      best_blocks = blocks;
    }
  }
  return best;
}

}  // namespace

int split_segments(const SampleArgs &a, Dtype dt) { return split_shape(a, dt).nseg; }

size_t split_workspace_bytes(const SampleArgs &a, Dtype dt) {
  const int nseg = split_segments(a, dt);
  if (!nseg) return 0;
  return SPLIT_CNT_BYTES + (size_t)a.n_rows * nseg * (2 + KF) * 8;
}

bool launch_split(const SampleArgs &a, Dtype dt, void *ws, size_t ws_bytes, hipStream_t s) {
  const SplitShape sh = split_shape(a, dt);
  if (!sh.nseg) return false;
  if (sh.cpt == SPLIT_CPT_LONG) /* (fp32 only) */
    return dt == DT_F32 && try_split<SPLIT_CPT_LONG, false>(a, sh.nseg, ws, ws_bytes, s);
  if (sh.cpt == SPLIT_CPT_WIDE)
    return dt == DT_F32 ? try_split<SPLIT_CPT_WIDE, false>(a, sh.nseg, ws, ws_bytes, s)
                        : try_split<SPLIT_CPT_WIDE, true>(a, sh.nseg, ws, ws_bytes, s);
  return dt == DT_F32 ? try_split<SPLIT_CPT, false>(a, sh.nseg, ws, ws_bytes, s)
                      : try_split<SPLIT_CPT, true>(a, sh.nseg, ws, ws_bytes, s);
}

}  // namespace d3s
