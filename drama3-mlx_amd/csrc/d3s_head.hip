/* k_head: a head's logits and their sample in one launch (gfx950, wave64),
 * d3s_linear_sample_bf16's D3S_FLAG_ONE_LAUNCH form.
 *
 * The backbone head (src/backbone.c:1213-1215) and the tower's codebook heads
 * (src/tower.c:228-232,:264) are single-row gemvs, m_linear through gemv_row
 * (src/mlxu.c:454-496), whose bf16 logits the sampler takes next
 * (src/tower.c:426-443).  Here each workgroup computes one segment of a row's
 * logits (HEAD_NL per half-wave, in the reference gemv's order:
 * gemv_half_wave_n) and, on the same data, the sampler's front end for its
 * segment: the NaN-propagating max and the fast sum 2^(L c - h_s) relative to
 * its own max.  It publishes a record (max, fast sum, flags, its logits as
 * bf16) with agent-coherent stores, waits for them, and counts its arrival
 * (on its group's counter; the last of a group on the row's).  The last
 * arrival merges: it takes every record in one round of coherent loads (the
 * row's logits land in its LDS), the row max, a threshold from the segment
 * maxima (the k-th largest, exactly, by two 8-bit histogram passes: bf16
 * values have 16-bit order keys), the candidates of the segments that reach it, their
 * ranks, the fast sums rescaled to the row's offset, and runs the reference
 * kernel's tail (src/sampling.c:123-139, or the op graph's order :39-48) with
 * the fast lse's margin test.  A cut within the margin takes the exact lse
 * from the LDS row; T not finite, logits too large for the fast sum, too many
 * candidates or a top k reaching x = -inf sample the row by the generic
 * procedure over the LDS row.  Every result is the oracle's bits for the
 * logits the gemv wrote.  No spin-waits: a workgroup that is not last ends;
 * the last resets the counters for the next launch.
 *
 * Measured on [1, 2048] x [4097, 2048]: the segments are all counted about
 * 8.4 us after the first starts (gemv 3.4 us median per workgroup, publishing
 * 0.8 us, counting 0.4-0.9 us), and the merge takes 5 us as one workgroup's
 * dependent chain, much of it instruction fetch of code the CU has not run
 * (loads 1.2, threshold and candidates 2.5, ranking 0.7, sum 0.3, tail 1.5):
 * 1.4-2.2 us slower per call than the gemv and the one-wave sample as two
 * launches, whose second dispatch overlaps the first.  So the two launches
 * stay the default. */
#include "d3s_rowcore.h"
#include "d3s_gemv.h"

namespace d3s {
namespace {

/* The form: NW waves a workgroup, each half-wave computing NL logits, so a
 * segment holds HEAD_SEG = 2 NW NL logits.  Fewer, fuller workgroups start
 * sooner (a launch's workgroups are dispatched over microseconds) and leave
 * fewer records to merge. */
constexpr int HEAD_NW = 8;
constexpr int HEAD_NL = 1;
constexpr int HEAD_T = HEAD_NW * WAVE;                  /* threads per workgroup */
constexpr int HEAD_SEG = 2 * HEAD_NW * HEAD_NL;         /* logits per segment */
constexpr int HEAD_LW = HEAD_SEG / 4;                   /* record words of logits (bf16, four a word) */
constexpr int HEAD_RW = (2 + HEAD_LW + 7) / 8 * 8;      /* record words per segment (whole 64 bytes) */
constexpr int HEAD_MAX_SEG = HEAD_T;                    /* segments per row: one per merging thread */
constexpr int HEAD_MAX_V = 8192;                        /* the merger's LDS row */
static_assert(HEAD_MAX_V <= HEAD_MAX_SEG * HEAD_SEG, "a row's segments exceed the merging threads");
static_assert(HEAD_SEG <= WAVE, "a segment's front end runs on one wave");
constexpr int HEAD_MCAP = HEAD_T;                       /* candidates the merger ranks */
/* Arrivals are counted in two levels: a segment counts on its group's
 * counter (HEAD_GRP segments a group), the last of a group on the row's.
 * Atomics on one address serialise across the device.  Every counter has its
 * own 128-byte line: the row's, then its groups', HEAD_CLINES lines a row,
 * inside the segmented kernel's 256 KiB counter block (both kernels leave
 * every counter zero). */
constexpr int HEAD_GRP = 16;
constexpr int HEAD_CLINES = 1 + (HEAD_MAX_V / HEAD_SEG + HEAD_GRP - 1) / HEAD_GRP;
constexpr size_t HEAD_CNT_BYTES = (size_t)2048 * 128;
constexpr int HEAD_MAX_ROWS = (int)(HEAD_CNT_BYTES / 128) / HEAD_CLINES;

constexpr uint32_t HSEG_GENERIC = 1u; /* T not finite or logits too large for the fast sum */

struct __align__(16) HeadLds {
  uint64_t row[HEAD_MAX_V / 4];   /* the merger's copy of the row: bf16, four per word */
  uint64_t keys[HEAD_MCAP + 2];   /* candidates (+ pads); the generic procedure's sort list */
  uint64_t ranked[KF];
  uint64_t seg[HEAD_LW];          /* a segment's logits, bf16 */
  uint32_t mk[HEAD_MAX_SEG];      /* order keys of the segment maxima */
  uint32_t hist[2][NB];           /* the threshold's two histogram passes */
  uint32_t sel[3];
  float buf[WAVE];
  float wmax[HEAD_NW], wsum[HEAD_NW], weps[HEAD_NW];
  uint32_t wflag[HEAD_NW], slo[HEAD_NW], shi[HEAD_NW];
  uint32_t last, exact, mcount;
};

/* logit i of the merger's LDS row */
__device__ __forceinline__ float head_logit(const HeadLds &S, int i) {
  return d3s_bf16_to_f32(((const uint16_t *)S.row)[i]);
}

/* logit e of a segment's record words */
__device__ __forceinline__ float seg_logit(const uint64_t *lw, int e) {
  return d3s_u2f(((uint32_t)(lw[e / 4] >> (16 * (e % 4))) & 0xffffu) << 16);
}

/* The exact lse of the row (the oracle's: 2^-40 fixed point of d3s_expf(x -
 * M)) from the LDS row, by the whole workgroup. */
__device__ __forceinline__ float head_exact_lse(HeadLds &S, int V, float T, float M) {
  const float y = 1.0f / T;
  uint64_t acc = 0;
  for (int i = threadIdx.x; i < V; i += HEAD_T) acc += d3s_fix40_exp(scale_logit(head_logit(S, i), T, y, true) - M);
  const uint64_t w = wave_sum_u64(acc);
  const int wid = threadIdx.x / WAVE;
  if (lane_id() == 0) {
    S.slo[wid] = (uint32_t)w;
    S.shi[wid] = (uint32_t)(w >> 32);
  }
  __syncthreads();
  uint64_t tot = 0;
#pragma unroll
  for (int q = 0; q < HEAD_NW; q++) tot += ((uint64_t)S.shi[q] << 32) | S.slo[q];
  return M + d3s_logf(d3s_fixsum_to_f32(tot));
}

/* grid (nseg, n_rows); a: the sample's arguments (vocab = la.V; logits,
 * row_stride and banned unused).  The merger runs once per launch on one
 * workgroup, so its code is cold in the instruction cache: its loops stay
 * rolled. */
__global__ __launch_bounds__(HEAD_T) void k_head(LinearArgs la, SampleArgs a, uint32_t *counters_ws,
                                                 uint64_t *records, int nseg) {
  __shared__ HeadLds S;
  const int row = (int)blockIdx.y, seg = (int)blockIdx.x;
  const int wid = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / WAVE));
  const int lane = lane_id(), hl = lane & 31;
  const int V = la.V, k = a.k;
  const float ninf = -__builtin_inff();

  /* ---- the segment's logits: HEAD_NL per half-wave */
  {
    const int h = wid * 2 + (lane >> 5);
    const int r0 = seg * HEAD_SEG + h * HEAD_NL;
    float acc[HEAD_NL];
    gemv_half_wave_n<HEAD_NL>(la, row, r0, hl, acc);
    if (hl == 0) {
#pragma unroll
      for (int j = 0; j < HEAD_NL; j++) {
        const int r = r0 + j;
        const uint16_t yb = d3s_f32_to_bf16_rn(acc[j]);
        if (r < V && la.y) la.y[(size_t)row * V + r] = yb;
        ((uint16_t *)S.seg)[h * HEAD_NL + j] = r < V ? yb : (uint16_t)0xff80u; /* past V: -inf */
      }
    }
  }
  __syncthreads();

  const RowP rp = row_params(a, row);
  const float T = rp.T, top_p = rp.top_p;
  const bool t_finite = T < __builtin_inff(); /* false for +inf and NaN */
  const float y = 1.0f / T;
  const float cf = LOG2E_F / T;

  /* ---- the segment's max and fast sum (wave 0, lane i < HEAD_SEG holding
   * logit i), its record, its arrival */
  if (wid == 0) {
    const float L = lane < HEAD_SEG ? d3s_bf16_to_f32(((const uint16_t *)S.seg)[lane]) : ninf;
    const float Ls = wave_maximum_f(L);
    const bool live = !d3s_isnan(Ls) && Ls != __builtin_inff() && Ls != ninf;
    uint32_t flags = 0u;
    float ssum = 0.0f;
    if (live && (!t_finite || !(fabsf(Ls * cf) < 0x1p24f))) flags |= HSEG_GENERIC;
    if (live && flags == 0u) {
      const float b = -(Ls * cf);
      ssum = wave_sum_f(lane < HEAD_SEG ? __builtin_amdgcn_exp2f(__builtin_fmaf(L, cf, b)) : 0.0f);
    }
    uint64_t *rec = records + ((size_t)row * nseg + seg) * HEAD_RW;
    if (lane < HEAD_LW) st_agent(rec + 2 + lane, S.seg[lane]);
    if (lane == 0) {
      st_agent(rec, (uint64_t)d3s_f2u(Ls) | ((uint64_t)d3s_f2u(ssum) << 32));
      st_agent(rec + 1, (uint64_t)flags);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); /* the records retired before the count (see st_agent) */
    if (lane == 0) {
      uint32_t *cnt_row = counters_ws + (size_t)row * HEAD_CLINES * 32; /* 32 words = 128 bytes */
      const int g = seg / HEAD_GRP, ng = (nseg + HEAD_GRP - 1) / HEAD_GRP;
      uint32_t *cnt_grp = cnt_row + (size_t)(1 + g) * 32;
      const uint32_t gsize = (uint32_t)min(HEAD_GRP, nseg - g * HEAD_GRP);
      bool last = false;
      const uint32_t og = __hip_atomic_fetch_add(cnt_grp, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (og == gsize - 1u) {
        __hip_atomic_store(cnt_grp, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t orow = __hip_atomic_fetch_add(cnt_row, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = orow == (uint32_t)(ng - 1);
        if (last) __hip_atomic_store(cnt_row, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      S.last = last;
      S.exact = 0u;
      S.mcount = 0u;
    }
  }
  __syncthreads();
  if (!S.last) return;

  /* ---- the last arrival merges.  Every record word in one round of coherent
   * loads: thread t takes segment t's header and logits; wave 0 its uniforms */
  const int t = (int)threadIdx.x;
  const uint64_t *rrow = records + (size_t)row * nseg * HEAD_RW;
  uint64_t h0 = 0ull, h1 = 0ull, lw[HEAD_LW];
#pragma unroll
  for (int q = 0; q < HEAD_LW; q++) lw[q] = 0xff80ff80ff80ff80ull; /* -inf */
  if (t < nseg) {
    const uint64_t *rec = rrow + (size_t)t * HEAD_RW;
    h0 = ld_agent(rec);
    h1 = ld_agent(rec + 1);
#pragma unroll
    for (int q = 0; q < HEAD_LW; q++) lw[q] = ld_agent(rec + 2 + q);
  }
  const float uval = (wid == 0 && lane < k) ? a.u[(size_t)row * k + lane] : 0.0f;
  const float noise = -d3s_logf(1.0f - uval); /* off the tail's path */
  if (t < nseg) {
#pragma unroll
    for (int q = 0; q < HEAD_LW; q++) S.row[t * HEAD_LW + q] = lw[q];
  }
  const float Ls_t = t < nseg ? d3s_u2f((uint32_t)h0) : ninf;
  const float ss_t = d3s_u2f((uint32_t)(h0 >> 32));
  S.mk[t] = t < nseg ? d3s_ordkey(Ls_t) : 0u;
  {
    const float wm = wave_maximum_f(Ls_t);
    const uint32_t wf = __ballot(((uint32_t)h1 & HSEG_GENERIC) != 0u) ? HSEG_GENERIC : 0u;
    if (lane == 0) {
      S.wmax[wid] = wm;
      S.wflag[wid] = wf;
    }
  }
  __syncthreads();
  float Lmax = S.wmax[0];
  uint32_t F = S.wflag[0];
#pragma unroll
  for (int w = 1; w < HEAD_NW; w++) {
    Lmax = fmaximum(Lmax, S.wmax[w]);
    F |= S.wflag[w];
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
  int kpow = 2;
  while (kpow < k) kpow <<= 1;
  bool generic = !t_finite || F != 0u || (a.flags & FLAG_EXACT_SELECT) != 0u;
  if ((a.flags & FLAG_EXACT_SELECT) && t_finite && F == 0u && t == 0 && a.counters)
    atomicAdd(&a.counters[CNT_EXACT_SELECT], 1u);
  if (!generic) {
    /* ---- tau: the k-th largest segment maximum, exactly: the order key of
     * a bf16 value has its low 16 bits all equal, so two 8-bit histogram
     * passes over the top 16 bits decide it (0 when fewer than k segments);
     * at least k logits reach it */
    const uint32_t key16 = S.mk[t] >> 16;
    if (t < NB) {
      S.hist[0][t] = 0u;
      S.hist[1][t] = 0u;
    }
    __syncthreads();
    if (t < nseg) atomicAdd(&S.hist[0][key16 >> 8], 1u);
    __syncthreads();
    if (wid == 0) {
      const BinSel b = wave_find_bin<false>(S.hist[0], (uint32_t)k);
      if (lane == 0) {
        S.sel[0] = b.ok ? b.bin : 0xffffffffu;
        S.sel[1] = (uint32_t)k - b.above;
      }
    }
    __syncthreads();
    const uint32_t b1 = S.sel[0];
    if (t < nseg && (key16 >> 8) == b1) atomicAdd(&S.hist[1][key16 & 0xffu], 1u);
    __syncthreads();
    if (wid == 0 && b1 != 0xffffffffu) {
      const BinSel b = wave_find_bin<false>(S.hist[1], S.sel[1]);
      if (lane == 0) S.sel[2] = b.bin;
    }
    __syncthreads();
    const uint32_t pre = b1 == 0xffffffffu ? 0u : (b1 << 24) | (S.sel[2] << 16);
    /* below every logit whose x ties with tau's (as in the one-wave kernel);
     * when the k-th segment max is -inf, every finite logit is a candidate
     * (and fewer than k of them send the row to the generic procedure) */
    const float tau = d3s_from_ordkey(pre);
    const float tau_lo = pre < d3s_ordkey(-0x1.fffffep127f) ? -0x1.fffffep127f
                                                           : tau - (fabsf(tau) * 0x1p-21f + T * 0x1p-120f);
    /* ---- the candidates: the logits that reach tau_lo, from the segments
     * whose max does; filed with one LDS atomic per wave */
    uint64_t cm = 0ull;
    if (t < nseg && Ls_t >= tau_lo) {
#pragma unroll
      for (int e = 0; e < HEAD_SEG; e++) cm |= (uint64_t)(seg_logit(lw, e) >= tau_lo ? 1u : 0u) << e;
    }
    const uint32_t c = (uint32_t)__popcll(cm);
    const uint32_t incl = wave_scan_add_u32(c);
    const uint32_t wtot = readlane_u(incl, 63);
    uint32_t base = 0u;
    if (lane == 0 && wtot) base = atomicAdd(&S.mcount, wtot);
    base = readlane_u(base, 0);
    uint32_t at = base + incl - c;
#pragma unroll 1
    while (cm) {
      const int e = __builtin_ctzll(cm);
      cm &= cm - 1ull;
      if (at < (uint32_t)HEAD_MCAP) {
        const uint32_t hw = (uint32_t)(S.row[t * HEAD_LW + e / 4] >> (16 * (e % 4))) & 0xffffu;
        S.keys[at] = composite_key(scale_logit(d3s_u2f(hw << 16), T, y, true), t * HEAD_SEG + e);
      }
      at++;
    }
    __syncthreads();
    const uint32_t n = S.mcount;
    generic = n > (uint32_t)HEAD_MCAP || n < (uint32_t)k;
    if (!generic) {
      rank_by_count<HEAD_T>(S.keys, n, k, S.ranked);
      /* the top k reach x = -inf (a logit / T overflowing): ties the
       * candidates may not hold */
      generic = key_x(S.ranked[k - 1]) == ninf;
    }
  }
  if (generic) {
    generic_row_src<HEAD_T>(a, row, kpow, S.keys, [&](int i) { return head_logit(S, i); });
    return;
  }

  /* ---- the rescaled fast sum and its error bound.  Segment s's terms were
   * taken relative to h_s = RN(Ls cf) and are scaled by 2^(h_s - h), h =
   * RN(Lmax cf) (hardware 2^x of the rounded difference); weighted by its share
   * (at most HEAD_SEG 2^(h_s - h), capped at 1), each segment adds its own
   * terms' rounding bound and the rescale's.  Thread t takes segment t. */
  const float h = Lmax * cf;
  const float delta = __builtin_fmaf(Lmax, cf, -h); /* Lmax * cf - h exactly */
  float term = 0.0f, eterm = 0.0f;
  if (t < nseg && Ls_t != ninf) {
    const float d = Ls_t * cf - h; /* <= 0 */
    const float f = __builtin_amdgcn_exp2f(d);
    term = ss_t * f;
    const float w = fminf(1.0f, (float)HEAD_SEG * f);
    eterm = w * (0x1p-24f * (2.0f * fabsf(Ls_t) * y + 160.0f) + 0x1p-24f * fabsf(d) + EPS_EXP2);
  }
  {
    const float ws = wave_sum_f(term), we = wave_sum_f(eterm);
    if (lane == 0) {
      S.wsum[wid] = ws;
      S.weps[wid] = we;
    }
  }
  __syncthreads();
  float sp = S.wsum[0], eps_seg = S.weps[0];
#pragma unroll
  for (int w = 1; w < HEAD_NW; w++) { /* the same order in every wave */
    sp = sp + S.wsum[w];
    eps_seg = eps_seg + S.weps[w];
  }
  eps_seg = eps_seg * (1.0f + 0x1p-20f); /* the bound's own rounding */
  const float l2 = __builtin_amdgcn_logf(sp); /* within 2^-23 |log2 sp| + 2^-24 */
  float lse = M + (l2 * LN2_F - delta * LN2_F);
  /* the one-wave kernel's bound (its term for the max's rounding is in
   * eps_seg; one term per lane in a segment), the rescale's products and the
   * merger's sum (a 6-step DPP tree and HEAD_NW - 1 additions: every term
   * passes at most 6 + HEAD_NW roundings), doubled, and eps_seg */
  const float eps_s = EPS_EXP2 + 0x1p-23f + (float)(1 + 11 + 2 * (1 + 6 + HEAD_NW)) * 0x1p-24f +
                      (float)V * 0x1p-40f + 0x1p-22f * fabsf(l2) + 0x1p-23f + eps_seg;

  /* ---- the tail on wave 0; a cut within the margin takes the exact lse (by
   * the whole workgroup, from the LDS row) and the tail again */
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
    lse = head_exact_lse(S, V, T, M);
    exact = true;
  }
}

}  // namespace

int head_max_vocab() { return HEAD_MAX_V; }

int head_max_rows() { return HEAD_MAX_ROWS; }

size_t head_workspace_bytes(const LinearArgs &la) {
  const int nseg = (la.V + HEAD_SEG - 1) / HEAD_SEG;
  return HEAD_CNT_BYTES + (size_t)la.n_rows * nseg * HEAD_RW * 8;
}

bool launch_head(const LinearArgs &la, const SampleArgs &a, void *ws, size_t ws_bytes, hipStream_t s) {
  if (a.k > KF || la.V > HEAD_MAX_V || la.n_rows > HEAD_MAX_ROWS || la.n_rows > 65535) return false;
  const int nseg = (la.V + HEAD_SEG - 1) / HEAD_SEG;
  if (!ws || head_workspace_bytes(la) > ws_bytes) return false;
  hipLaunchKernelGGL(k_head, dim3((unsigned)nseg, (unsigned)la.n_rows), dim3(HEAD_T), 0, s, la, a,
                     (uint32_t *)ws, (uint64_t *)((char *)ws + HEAD_CNT_BYTES), nseg);
  return true;
}

}  // namespace d3s
