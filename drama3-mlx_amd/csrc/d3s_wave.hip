/* The one-wave-per-row sampler kernel (gfx950, wave64): k_wave.
 *
 * Each wave samples one row held in its registers (up to 96 fp32 or 128 bf16
 * elements per lane); a 256-thread workgroup carries four independent rows (a
 * launch of at most 1024 rows takes one per workgroup) and has no
 * workgroup barrier, so a launch of many rows streams at HBM rate while a
 * launch of one row runs on a single wave.  Semantics are the oracle's
 * (src/sampling.c:1-3,:22-49,:53-140), bit for bit:
 *
 *  1. load the row (16-byte chunks), NaN-propagating max per lane and row:
 *     refused / all -inf rows as the reference kernel (src/sampling.c:54-79);
 *     m = max x = RN(max logit / T) (division is monotone).
 *  2. tau = the k-th largest of the 64 lane maxima (a ballot radix search):
 *     at least k elements reach it.  tau_lo steps tau down past logits whose
 *     x ties with tau's x, so {logit >= tau_lo} holds every element whose x
 *     reaches the k-th largest x: the top k (src/sampling.c:90-121) lie in it.
 *  3. passes over the registers: the candidates {logit >= tau_lo} as a bit
 *     per element, then the fast row sum S' = sum 2^(logit*c - h)
 *     (c = log2(e)/T, v_exp_f32) while the first candidates are read again.
 *  4. candidates take their exact x, rank by (x desc, index asc) and the top k
 *     run the reference kernel's tail (src/sampling.c:123-139) with
 *     lse' = m + ln S'.  lse only decides the top-p cut (the probabilities use
 *     exp(x - x_0)), so when every c'_r is farther from top_p than the proven
 *     bound on |c'_r - c_r| the cut equals the one under the exact lse.
 *     Otherwise the wave computes the exact row sum (2^-40 fixed point of
 *     d3s_expf(x - m), as the oracle) and redoes the cumulative.
 *  Exact fallbacks: more candidates than a wave holds -> 8-bit radix select
 *  over order-preserving keys of x; T not finite or |m| beyond 2^24 -> every
 *  quantity per element from x exactly (slow_row).
 * k_wide (below) runs the same passes on rows spread over a workgroup.
 */
#include "d3s_rowcore.h"
#include "d3s_gemv.h"

#pragma clang fp contract(off)

namespace d3s {
namespace {

constexpr int WR = 4;   /* rows (waves) per 256-thread workgroup */
constexpr int WR_SPREAD_ROWS = 1024; /* up to this many rows, one row per workgroup */

struct __align__(16) WaveLds {
  float buf[WAVE];         /* sequential sums (16-byte aligned float4 reads) */
  uint64_t keys[WAVE + 2]; /* dense candidate keys (+ a zero pad for pair reads) */
  uint64_t ranked[WAVE];   /* keys by rank */
  uint32_t hist[NB];       /* radix-select histogram */
};

/* What a row's rare exact paths need.  They read the row again (from L2), a
 * group of chunk rows at a time (every load of a group in flight at once), so
 * their registers stay few next to the fast path's. */
struct RowRef {
  uint32_t *counters;
  WaveLds *Sp;
  const uint4 *src;
  int nchunks, pos0, V, k, lane, banned;
  float T, y;
  bool t_finite;
};

/* chunk rows the rare paths read at once (the most that leaves the kernel's
 * register count where the fast path puts it) */
template <int CPT, bool BF16>
constexpr int rare_group() {
  return BF16 ? 4 : 6;
}

/* f(i, x, in) for every element of chunk rows j0 .. j0 + GROUP - 1 (in: the
 * position lies in the row; x = L / T, -inf at the banned index) */
template <int CPT, bool BF16, class F>
__device__ __forceinline__ void for_group(const RowRef &R, int j0, F &&f) {
  constexpr int GROUP = rare_group<CPT, BF16>();
  using C = Chunks<1, BF16>;
  constexpr int EPC = C::EPC;
  const uint4 *src = R.src;
  asm volatile("" : "+s"(src)); /* a second read: not to be matched with the first */
  uint4 q[GROUP];
#pragma unroll
  for (int g = 0; g < GROUP; g++)
    if (j0 + g < CPT) q[g] = src[min((j0 + g) * WAVE + R.lane, R.nchunks - 1)];
#pragma unroll
  for (int g = 0; g < GROUP; g++)
    if (j0 + g < CPT) {
      C c;
      c.w[0] = q[g].x;
      c.w[1] = q[g].y;
      c.w[2] = q[g].z;
      c.w[3] = q[g].w;
#pragma unroll
      for (int e = 0; e < EPC; e++) {
        const int i = (j0 + g) * EPC + e;
        const int p = R.pos0 + (j0 + g) * WAVE * EPC + e;
        const bool in = (unsigned)p < (unsigned)R.V;
        f(i, scale_logit(p == R.banned ? -__builtin_inff() : c.val(e), R.T, R.y, R.t_finite), in);
      }
      __builtin_amdgcn_sched_barrier(0); /* one chunk at a time */
    }
}

/* ---- exact 8-bit radix select of the top k by (x desc, index asc); writes
 * exactly k keys to S.keys and returns k */
template <int CPT, bool BF16>
__device__ __forceinline__ int exact_select(const RowRef &R) {
  constexpr int GROUP = rare_group<CPT, BF16>();
  constexpr int EPC = Chunks<1, BF16>::EPC;
  if (R.lane == 0 && R.counters) atomicAdd(&R.counters[CNT_EXACT_SELECT], 1u);
  WaveLds &S = *R.Sp;
  uint32_t prefix = 0u, pmask = 0u, need = (uint32_t)R.k;
  bool done = false;
#pragma unroll 1
  for (int pass = 0; pass < 4 && !done; pass++) {
    const int shift = 24 - 8 * pass;
    wave_lds_sync();
    for (int i = R.lane; i < NB; i += WAVE) S.hist[i] = 0u;
    wave_lds_sync();
#pragma unroll 1
    for (int j0 = 0; j0 < CPT; j0 += GROUP)
      for_group<CPT, BF16>(R, j0, [&](int, float x, bool in) {
        const uint32_t key = d3s_ordkey(x);
        if (in && (key & pmask) == prefix) atomicAdd(&S.hist[(key >> shift) & 255u], 1u);
      });
    wave_lds_sync();
    const BinSel b = wave_find_bin<false>(S.hist, need); /* holds >= need */
    prefix |= b.bin << shift;
    pmask |= 0xffu << shift;
    done = b.count == need - b.above;
    need -= b.above;
  }
  /* everything above the group, then the group (all of it when it holds
   * exactly `need`, else its lowest-index `need`, in index order) */
  uint32_t base = 0u;
#pragma unroll 1
  for (int j0 = 0; j0 < CPT; j0 += GROUP)
    for_group<CPT, BF16>(R, j0, [&](int i, float x, bool in) {
      const uint32_t km = d3s_ordkey(x) & pmask;
      const bool sel = in && (km > prefix || (done && km == prefix));
      const uint64_t m = __ballot(sel);
      if (sel) S.keys[base + (uint32_t)mbcnt64(m)] = composite_key(x, Chunks<1, BF16>::pos(R.pos0, i));
      base += (uint32_t)__popcll(m);
    });
  if (!done) {
    /* chunk row by chunk row: each lane's tie count, an exclusive scan for
     * the ties' ordinals in index order, and the first `need` ties written */
    uint32_t ord0 = 0u;
#pragma unroll 1
    for (int j0 = 0; j0 < CPT; j0 += GROUP) {
      uint32_t cnts[GROUP * EPC];
      for_group<CPT, BF16>(R, j0, [&](int i, float x, bool in) {
        cnts[(i - j0 * EPC)] = (in && d3s_ordkey(x) == prefix) ? 1u : 0u;
      });
#pragma unroll
      for (int g = 0; g < GROUP; g++)
        if (j0 + g < CPT) {
          uint32_t c = 0u;
#pragma unroll
          for (int e = 0; e < EPC; e++) c += cnts[g * EPC + e];
          const uint32_t incl = wave_scan_add_u32(c);
          uint32_t o = ord0 + incl - c;
          ord0 += readlane_u(incl, 63);
#pragma unroll
          for (int e = 0; e < EPC; e++) {
            if (cnts[g * EPC + e] && o < need) {
              const int i = (j0 + g) * EPC + e;
              const int p = Chunks<1, BF16>::pos(R.pos0, i);
              S.keys[base + o] = ((uint64_t)prefix << 32) | (uint64_t)(uint32_t)(~(uint32_t)p);
            }
            o += cnts[g * EPC + e];
          }
        }
    }
  }
  return R.k;
}

/* the exact row sum of the oracle: 2^-40 fixed point of d3s_expf(x - m) */
template <int CPT, bool BF16>
__device__ __forceinline__ float exact_lse(const RowRef &R, float M) {
  constexpr int GROUP = rare_group<CPT, BF16>();
  uint64_t acc = 0;
#pragma unroll 1
  for (int j0 = 0; j0 < CPT; j0 += GROUP)
    for_group<CPT, BF16>(R, j0, [&](int, float x, bool in) { acc += in ? d3s_fix40_exp(x - M) : 0ull; });
  return M + d3s_logf(d3s_fixsum_to_f32(wave_sum_u64(acc)));
}

/* refusal and max of x = L / T element by element (T not finite, or logits
 * too large for the fast row sum): the max, or NaN when some x is NaN or +inf */
template <int CPT, bool BF16>
__device__ __forceinline__ float slow_max(const RowRef &R) {
  constexpr int GROUP = rare_group<CPT, BF16>();
  float xm = -__builtin_inff();
  bool bad = false;
#pragma unroll 1
  for (int j0 = 0; j0 < CPT; j0 += GROUP)
    for_group<CPT, BF16>(R, j0, [&](int, float x, bool in) {
      bad = bad || (in && (classify(x) & 1u));
      xm = (in && !d3s_isnan(x)) ? fmaxf(xm, x) : xm;
    });
  return __ballot(bad) ? __builtin_nanf("") : wave_max_f(xm);
}

/* The candidates as a bit per element, no branches: element i of word i / 32
 * at bit 31 - i % 32, set when v(i) >= t.  For t finite or +inf and v(i)
 * finite or -inf, v - t is negative exactly when v < t (a difference is zero
 * only between equal values, +0 then; a flushed one keeps its sign; -inf
 * gives -inf), so its sign bit is the element's bit inverted: each word
 * takes (w << 1) | sign(v - t) (one v_alignbit after the subtraction; the
 * words' chains are independent), then is inverted; the last word's padding
 * shifts out. */
template <int NV, class F>
__device__ __forceinline__ void cand_bits(uint32_t (&bits)[(NV + 31) / 32], F &&v, float t) {
  constexpr int NWORD = (NV + 31) / 32;
  uint32_t below[NWORD];
#pragma unroll
  for (int w = 0; w < NWORD; w++) below[w] = 0u;
#pragma unroll
  for (int i = 0; i < NV; i++) below[i / 32] = (below[i / 32] << 1) | (d3s_f2u(v(i) - t) >> 31);
#pragma unroll
  for (int w = 0; w < NWORD; w++) bits[w] = ~below[w];
  if (NV % 32) bits[NWORD - 1] <<= 32 - NV % 32;
}

/* DRAW: the call gives no u; the row's uniforms are drawn here (only the
 * one-row kernel is built so: the other forms keep no trace of it) */
template <int CPT, bool BF16, bool DRAW = false>
struct WaveRow {
  /* candidates per lane read again while the row is still in L2 */
  static constexpr int EARLY = 3;
  using C = Chunks<CPT, BF16>;
  static constexpr int ES = BF16 ? 2 : 4;
  static constexpr int EPC = C::EPC;
  static constexpr int NV = C::NV;

  const SampleArgs a;
  WaveLds &S;
  int row, V, k, lane, pos0, off, nchunks, banned;
  const uint4 *src;
  const char *rowp;
  float T, y, uval, top_p;
  bool t_finite;
  /* a cut that needs the exact lse returns NEED_EXACT instead of the wave
   * computing it alone (k_wave_row sets it beside ex_in, whose shares answer
   * first: it keeps the one-wave exact pass out of that kernel's code) */
  bool defer_exact = false;
  float fin_M = 0.0f, fin_noise = 0.0f; /* the tail's max x and noise */
  /* the candidates from the registers (staged in LDS) instead of read again
   * from L2: long launches, whose rows leave L2 before a second read */
  bool reg_cands = false;
  /* k_wave_row: the fast lse' and its bound come from the workgroup's helper
   * wave (lse_in: the two floats it files), read after a workgroup barrier
   * that wave 0 passes on the way to the tail; `synced` says whether it did
   * (the rows that end earlier pass it in the kernel) */
  const float *lse_in = nullptr;
  bool synced = false;
  /* k_wave_row: the exact row sum's three shares (2^-40 fixed point), filed
   * by the helper waves before that same barrier; a cut within the fast lse's
   * margin takes the exact lse from them */
  const uint64_t *ex_in = nullptr;
  /* DRAW, k_wave_row: the race's noise per lane, filed by helper wave 2
   * before that same barrier (its ten Philox rounds and the logarithm then
   * stay off wave 0's path) */
  const float *noise_in = nullptr;
  float *noise_out = nullptr; /* set on the helper that files it */
  C c; /* -inf outside the row and at the banned index */

  __device__ WaveRow(const SampleArgs &a_, WaveLds &S_, int row_) : a(a_), S(S_), row(row_) {}

  __device__ __forceinline__ bool valid(int i) const { return (unsigned)C::pos(pos0, i) < (unsigned)V; }
  /* chunk row j holds part of the row in some lane (wave-uniform) */
  __device__ __forceinline__ bool live(int j) const { return j * WAVE < nchunks; }
  __device__ __forceinline__ RowRef ref() const {
    return RowRef{a.counters, &S, src, nchunks, pos0, V, k, lane, banned, T, y, t_finite};
  }

  /* where the row's chunks lie (from the row's address and width alone) */
  __device__ __forceinline__ void setup() {
    /* a chunk never crosses a page, so the bytes outside the row it covers
     * are readable; they become -inf below */
    rowp = (const char *)a.logits + (size_t)row * (size_t)a.row_stride * ES;
    off = (int)(((uintptr_t)rowp & 15u) / ES);
    src = (const uint4 *)(rowp - off * ES);
    nchunks = (off + V + EPC - 1) / EPC;
    pos0 = lane * EPC - off;
  }

  /* one dword of a row-indexed array by a vector load (a VGPR, read into a
   * scalar only where it is used): waiting for it counts vector loads only
   * (issued in order), never the kernarg segment's scalar loads in flight */
  __device__ __forceinline__ uint32_t row_word(const void *base) const {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (row + 1) * 4, BUFFER_FLAGS);
    return __builtin_amdgcn_raw_buffer_load_b32(r, 0, row * 4, 0);
  }

  /* the row's temperature, banned index and uniform (top_p, which only the
   * tail needs, later), loaded before the row so that waiting for them does
   * not wait for it; params_done() takes them once the row's loads are out
   * (DRAW: no u; draw_noise() draws it) */
  uint32_t t_word, b_word;
  __device__ __forceinline__ void params() {
    t_word = a.temperature ? row_word(a.temperature) : d3s_f2u(a.temperature_scalar);
    b_word = a.banned ? row_word(a.banned) : 0xffffffffu;
    if constexpr (!DRAW) uval = lane < k ? a.u[(size_t)row * k + lane] : 0.0f;
  }
  __device__ __forceinline__ void params_done() {
    const float t = d3s_u2f((uint32_t)__builtin_amdgcn_readfirstlane((int)t_word));
    T = t < 1e-5f ? 1e-5f : t; /* src/sampling.c:16,195 */
    banned = __builtin_amdgcn_readfirstlane((int)b_word);
    t_finite = T < __builtin_inff(); /* false for +inf and NaN */
    y = 1.0f / T;
  }

  __device__ __forceinline__ void load() {
    /* every operand these loads need is a leading kernel argument (preloaded
     * into SGPRs): nothing here waits on the kernarg segment */
    setup();
    params();
    /* rows taken once (candidates from the registers) stream past the caches */
    if (reg_cands)
      c.template load<2>(src, nchunks, lane);
    else
      c.load(src, nchunks, lane);
    params_done();
    /* DRAW: the helper that files the race's noise draws it here, while the
     * row's loads are in flight (the masking below waits for them) */
    if constexpr (DRAW)
      if (noise_out) noise_out[lane] = draw_noise();
    /* the partial chunk at the row start and every chunk row from the one
     * holding the row end on */
    const int jlast = (nchunks - 1) / WAVE;
#pragma unroll
    for (int j = 0; j < CPT; j++)
      if ((j == 0 && off != 0) || j >= jlast) {
#pragma unroll
        for (int e = 0; e < EPC; e++) c.mask(j * EPC + e, !valid(j * EPC + e));
      }
    if ((unsigned)banned < (unsigned)V) {
      const int bp = banned + off;
      const int jb = bp / (WAVE * EPC), lb = (bp / EPC) % WAVE, eb = bp % EPC;
#pragma unroll
      for (int j = 0; j < CPT; j++)
        if (j == jb) {
#pragma unroll
          for (int e = 0; e < EPC; e++) c.mask(j * EPC + e, lane == lb && e == eb);
        }
    }
  }

  /* rank the n >= k keys in S.keys: the top k land in S.ranked by rank */
  __device__ __forceinline__ void rank_keys(int n) {
    if (lane == 0) S.keys[n] = 0ull; /* pad for the pair reads; below every key */
    wave_lds_sync();
    const uint64_t my = lane < n ? S.keys[lane] : 0ull;
    int rank = 0;
    const ulonglong2 *k2 = (const ulonglong2 *)S.keys;
#pragma unroll 4
    for (int j2 = 0; j2 < (n + 1) / 2; j2++) {
      const ulonglong2 q = k2[j2];
      rank += (q.x > my ? 1 : 0) + (q.y > my ? 1 : 0);
    }
    if (lane < n && rank < k) S.ranked[rank] = my;
    wave_lds_sync();
  }

  /* Rank the n >= k candidates in S.keys by key and run the tail (the
   * reference kernel's cumulative, cut, softmax and race, src/sampling.c:
   * 123-139, or the op graph's, :39-48); the exact row sum is computed when
   * the fast lse cannot settle the cut.  selected: S.keys holds exactly the
   * top k (the exact select's). */
  __device__ __forceinline__ int finish(int n, float M, float lse, bool exact, float eps_s, float noise,
                                        bool selected) {
    rank_keys(n);
    if (!selected && key_x(S.ranked[k - 1]) == -__builtin_inff()) {
      /* the top k reach x = -inf: the candidates need not hold the -inf
       * ties of lowest index; the exact select files exactly the top k */
      rank_keys(exact_select<CPT, BF16>(ref()));
    }
    const uint64_t key = lane < k ? S.ranked[lane] : 0ull;
    fin_M = M;
    fin_noise = noise;
    return wave_tail(a, row, key, M, lse, exact, eps_s, noise, top_p, S.buf, [&]() {
      if (ex_in) return M + d3s_logf(d3s_fixsum_to_f32(ex_in[0] + ex_in[1] + ex_in[2]));
      return defer_exact ? __builtin_nanf("") : exact_lse<CPT, BF16>(ref(), M);
    });
  }

  /* the tail again with the exact lse lx, after finish() returned NEED_EXACT */
  __device__ __forceinline__ int exact_tail(float lx) {
    const uint64_t key = lane < k ? S.ranked[lane] : 0ull;
    return wave_tail(a, row, key, fin_M, lx, true, 0.0f, fin_noise, top_p, S.buf, []() { return 0.0f; });
  }

  /* every quantity per element from x = L / T, as the oracle (T not finite,
   * or logits too large for the fast row sum) */
  __device__ __forceinline__ int slow_row() {
    top_p = row_top_p(a, row);
    const RowRef R = ref();
    const float M = slow_max<CPT, BF16>(R);
    if (d3s_isnan(M) || M == -__builtin_inff()) return wave_write_special(a, row, !d3s_isnan(M));
    const int n = exact_select<CPT, BF16>(R);
    return finish(n, M, exact_lse<CPT, BF16>(R, M), true, 0.0f, own_noise(), true);
  }

  /* The fast row sum S' = sum 2^(L c + b) over the row (b = -RN(Lmax c)),
   * lse' = M + ln 2 (log2 S' - delta) (delta = Lmax c + b exactly) and eps_s,
   * the bound on |lse' - lse| less the final roundings: the relative error of
   * 2^-delta S' against the exact row sum (the rounding of x, m, x - m and
   * log2(e)/T, the fast exponent's error, d3s_expf's, the terms below e^-40,
   * the fixed-point truncation, the accumulation's CPT + 3 + 6 roundings and
   * the final one), then the log: twice its bound, times ln 2, with the
   * product's rounding. */
  __device__ __forceinline__ void fast_lse(float M, float cf, float b, float delta, float &lse, float &eps_s) {
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
    const float sp = wave_sum_f(acc[0]); /* >= 2^delta, about 1 */
    /* the hardware log2, within 2^-23 |log2 sp| + 2^-24 (checked by the tests) */
    const float l2 = __builtin_amdgcn_logf(sp);
    lse = M + (l2 * LN2_F - delta * LN2_F);
    eps_s = 0x1p-24f * (2.0f * fabsf(M) + 160.0f) + EPS_EXP2 + 0x1p-23f + (float)(CPT + 11) * 0x1p-24f +
            (float)V * 0x1p-40f + 0x1p-22f * fabsf(l2) + 0x1p-23f;
  }

  /* k_wave_row's helper wave: the row's max as compute() takes it, then
   * fast_lse, filed at out[0..1] for wave 0.  Rows that compute() ends
   * before its tail (refused, all -inf, T not finite, logits too large for
   * the fast sum: the same tests on the same values) file nothing. */
  __device__ __forceinline__ void helper_lse(float *out, uint64_t *ex_out = nullptr) {
    if (!t_finite) return;
    const float ninf = -__builtin_inff();
    const float cf = LOG2E_F / T;
    float lm = ninf;
#pragma unroll
    for (int i = 0; i < NV; i++) lm = fmaximum(lm, c.val(i));
    const float Lmax = wave_maximum_f(lm);
    if (d3s_isnan(Lmax) || Lmax == __builtin_inff()) return;
    const float M = scale_logit(Lmax, T, y, true);
    if (M == __builtin_inff() || M == ninf) return;
    const float h = Lmax * cf;
    if (!(fabsf(h) < 0x1p24f)) return;
    const float b = -h;
    const float delta = __builtin_fmaf(Lmax, cf, b);
    float lse, eps_s;
    fast_lse(M, cf, b, delta, lse, eps_s);
    if (lane == 0) {
      out[0] = lse;
      out[1] = eps_s;
    }
    if (ex_out) { /* k_wave_row: the first share of the exact row sum */
      if (BF16) c.launder();
      const uint64_t w = exact_part<0, EX1>(M);
      if (lane == 0) ex_out[0] = w;
    }
  }

  /* k_wave_row's three shares of the exact row sum, by element of each lane:
   * wave 1 (after its fast sum) [0, EX1), waves 2 and 3 [EX1, EX2) and
   * [EX2, NV) (about a fifth and two halves of the rest: each files before
   * wave 0 reaches its tail) */
  static constexpr int EX1 = (NV / 5) & ~1;
  /* (DRAW: wave 2 also draws the race's noise, ten Philox rounds and a log:
   * it takes 3/8 of the rest, wave 3 the other 5/8, so the two file about
   * together) */
  static constexpr int EX2 = EX1 + (DRAW ? ((NV - EX1) * 3 / 8) & ~1 : (NV - EX1) / 2);

  /* the terms fix40(d3s_expf(x - M)) of elements [LO, HI) of every lane,
   * summed over the wave (masked elements hold -inf, whose term is 0).  An
   * integer sum, the same in any order: the shares add to the oracle's row
   * sum.
   * x = L / T: d3s_div_rn is q = L y and two fmas wherever T lies in
   * [2^-20, 2^21) and |L| in [2^-60, 2^100].  Smaller |L| give |x| < 2^-43,
   * below half an ulp of M when |M| >= 2^-15, so x - M rounds to -M from
   * either quotient; -inf (masked) and L < -2^100 give the term 0 from either
   * (-inf, a huge x or NaN all clamp to -43); L > 2^100 sends wave 0 to the
   * slow path, which does not read this sum.  Otherwise (rare) the chunks are
   * read again, one at a time, and every term takes d3s_div_rn. */
  template <int LO, int HI>
  __device__ __forceinline__ uint64_t exact_part(float M) {
    const uint32_t eb = (d3s_f2u(T) >> 23) & 0xffu;
    const bool quick = eb >= 127u - 20u && eb <= 127u + 20u && fabsf(M) >= 0x1p-15f;
    uint64_t acc = 0;
    if (quick) {
      /* two terms at a time (few live registers) */
#pragma unroll
      for (int i = LO; i < HI; i++) {
        const float L = c.val(i);
        const float q = L * y;
        acc += d3s_fix40_exp(__builtin_fmaf(__builtin_fmaf(-q, T, L), y, q) - M);
        if ((i - LO) & 1) __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      using C1 = Chunks<1, BF16>;
      const uint4 *s1 = src;
      asm volatile("" : "+s"(s1)); /* a second read: not to be matched with the first */
#pragma unroll 1
      for (int j = LO / EPC; j < (HI + EPC - 1) / EPC; j++) {
        const uint4 q = s1[min(j * WAVE + lane, nchunks - 1)];
        C1 one;
        one.w[0] = q.x;
        one.w[1] = q.y;
        one.w[2] = q.z;
        one.w[3] = q.w;
#pragma unroll
        for (int e = 0; e < EPC; e++) {
          const int i = j * EPC + e;
          const int pe = C::pos(pos0, i);
          const float L = pe == banned ? -__builtin_inff() : one.val(e);
          const bool take = i >= LO && i < HI && (unsigned)pe < (unsigned)V;
          acc += take ? d3s_fix40_exp(scale_logit(L, T, y, true) - M) : 0ull;
        }
      }
    }
    return wave_sum_u64(acc);
  }

  /* waves 2 and 3 of k_wave_row: the row's max as compute() takes it (the
   * same M), then their share of the exact row sum, filed at out[0].  Rows
   * that compute() ends at the max (refused, all -inf, T not finite: the same
   * tests on the same values) file nothing; every other row files, whichever
   * path wave 0 then takes. */
  __device__ __forceinline__ void helper_exact(uint64_t *out, int part) {
    if (!t_finite) return;
    const float ninf = -__builtin_inff();
    float lm = ninf;
#pragma unroll
    for (int i = 0; i < NV; i++) lm = fmaximum(lm, c.val(i));
    const float Lmax = wave_maximum_f(lm);
    if (d3s_isnan(Lmax) || Lmax == __builtin_inff()) return;
    const float M = scale_logit(Lmax, T, y, true);
    if (M == __builtin_inff() || M == ninf) return;
    if (BF16) c.launder();
    const uint64_t w = part == 0 ? exact_part<EX1, EX2>(M) : exact_part<EX2, NV>(M);
    if (lane == 0) out[0] = w;
  }

  /* DRAW: the race's noise -log(1 - u) from this lane's uniform, drawn here
   * (the same bits as d3s_uniform_fill's element r k + lane; u = 0 on lanes
   * past k, as the regular kernels' uval) */
  __device__ __forceinline__ float draw_noise() const {
    const float u =
        lane < k ? d3s_uniform(a.u_seed, a.u_stream, (uint64_t)row * (uint64_t)k + (uint64_t)lane) : 0.0f;
    return -d3s_logf(1.0f - u);
  }
  __device__ __forceinline__ float own_noise() const {
    if constexpr (DRAW)
      return draw_noise();
    else
      return -d3s_logf(1.0f - uval);
  }

  /* the row, once loaded (and masked), to its id */
  __device__ __forceinline__ int compute() {
    const float ninf = -__builtin_inff();
    /* the race's noise needs only u (DRAW: taken after the barrier below) */
    float noise = DRAW ? 0.0f : own_noise();
    bool slow = !t_finite;
    const float cf = slow ? 0.0f : LOG2E_F / T; /* needs only T: off the max's path */
    float M = 0.0f, b = 0.0f, delta = 0.0f, lm = ninf;
    if (!slow) {
      /* ---- row max of the logits; NaN propagates */
#pragma unroll
      for (int i = 0; i < NV; i++) lm = fmaximum(lm, c.val(i));
      const float Lmax = wave_maximum_f(lm);
      if (d3s_isnan(Lmax) || Lmax == __builtin_inff()) return wave_write_special(a, row, false);
      M = scale_logit(Lmax, T, y, true); /* = max x */
      if (M == __builtin_inff() || M == ninf) return wave_write_special(a, row, M == ninf);
      const float h = Lmax * cf;
      slow = !(fabsf(h) < 0x1p24f);
      b = -h;
      delta = __builtin_fmaf(Lmax, cf, b); /* Lmax * cf + b exactly */
    }
    if (slow) return slow_row();

    /* ---- tau: the k-th largest lane max, to 20 bits of its order key (a
     * lower bound: at least k elements reach it), by ballot radix search */
    bool need_sel = (a.flags & FLAG_EXACT_SELECT) != 0;
    const uint32_t pre = wave_kth_prefix(d3s_ordkey(lm), (uint32_t)k);
    /* top_p now (the kernarg segment has arrived by this step); the fence
     * keeps its load from moving up to where a wait for it would stall the
     * row's first steps */
    asm volatile("" ::: "memory");
    top_p = row_top_p(a, row);
    /* keys below -FLT_MAX's: the k-th lane max is -inf */
    if (pre < d3s_ordkey(-0x1.fffffep127f)) need_sel = true;
    const float tau = d3s_from_ordkey(pre);
    /* tau_lo: below every logit whose x ties with tau's (|L - tau| <=
     * T ulp(x_tau) <= 2^-22 |tau|, or T 2^-149 for a subnormal x_tau), so
     * {L >= tau_lo} holds every element whose x reaches the k-th largest */
    float tau_lo = need_sel ? __builtin_inff() : tau - (fabsf(tau) * 0x1p-21f + T * 0x1p-120f);
    /* a threshold at -inf would take masked padding for candidates */
    if (!(tau_lo >= -0x1.fffffep127f)) {
      need_sel = true;
      tau_lo = __builtin_inff();
    }

    /* ---- the candidates as a bit per element (element i of word i / 32
     * at bit 31 - i % 32), no branches */
    constexpr int NWORD = (NV + 31) / 32;
    uint32_t bits[NWORD];
    cand_bits<NV>(bits, [&](int i) { return c.val(i); }, tau_lo);
    int cnt = 0;
#pragma unroll
    for (int w = 0; w < NWORD; w++) cnt += __popc(bits[w]);
    const uint32_t tot = wave_sum_u32((uint32_t)cnt);
    if (__ballot(cnt > LCAP) || tot > (uint32_t)WAVE) need_sel = true;
    /* each lane takes its candidates in element order: the first EARLY are
     * read again now, while the row is still in L2 (the reads land during the
     * row sum below), the rest, rarely, after it */
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
      return pos0 + (i / EPC) * WAVE * EPC + (i % EPC);
    };
    auto read_logit = [&](int p) {
      return BF16 ? d3s_bf16_to_f32(((const uint16_t *)rowp)[p]) : ((const float *)rowp)[p];
    };
    int cpos[EARLY];
    float cl[EARLY];
#pragma unroll
    for (int q = 0; q < EARLY; q++) {
      cpos[q] = 0;
      cl[q] = 0.0f;
    }
    if (!need_sel && !reg_cands) {
#pragma unroll
      for (int q = 0; q < EARLY; q++) {
        if (q > 0 && !__ballot(q < cnt)) break;
        cpos[q] = next_cand();
        if (q < cnt) cl[q] = read_logit(cpos[q]);
      }
    }

    /* ---- the fast row sum (here, or on the helper wave) */
    float lse = 0.0f, eps_s = 0.0f;
    if (!lse_in) fast_lse(M, cf, b, delta, lse, eps_s);

    int n;
    if (need_sel) {
      n = exact_select<CPT, BF16>(ref());
    } else if (reg_cands) {
      /* each lane's chunks that hold a candidate are staged in LDS (the
       * histogram's and buf's room, idle here; slots by a wave scan), then
       * lane t files staged chunk t's elements that reach tau_lo (at most
       * tot <= 64 chunks) */
      uint32_t cm = 0u;
#pragma unroll
      for (int j = 0; j < CPT; j++) {
        const int i0 = j * EPC; /* a chunk's elements lie in one word */
        const uint32_t part = (bits[i0 / 32] >> (32 - EPC - i0 % 32)) & ((1u << EPC) - 1u);
        cm |= (part != 0u ? 1u : 0u) << j;
      }
      const uint32_t nc = (uint32_t)__popc(cm);
      const uint32_t cinc = wave_scan_add_u32(nc);
      uint32_t slot = cinc - nc;
      uint4 *stg = (uint4 *)S.hist;
      uint32_t *sps = (uint32_t *)S.buf;
#pragma unroll
      for (int j = 0; j < CPT; j++)
        if ((cm >> j) & 1u) {
          stg[slot] = make_uint4(c.w[4 * j], c.w[4 * j + 1], c.w[4 * j + 2], c.w[4 * j + 3]);
          sps[slot] = (uint32_t)C::pos(pos0, j * EPC);
          slot++;
        }
      wave_lds_sync();
      float v[EPC];
      uint32_t vm = 0u, pb = 0u;
      if ((uint32_t)lane < readlane_u(cinc, 63)) {
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
      uint32_t at = wave_scan_add_u32(ne) - ne;
#pragma unroll
      for (int e = 0; e < EPC; e++)
        if ((vm >> e) & 1u) {
          S.keys[at] = composite_key(scale_logit(v[e], T, y, true), (int)pb + e);
          at++;
        }
      n = (int)tot;
    } else {
      const uint32_t excl = wave_scan_add_u32((uint32_t)cnt) - (uint32_t)cnt;
#pragma unroll
      for (int q = 0; q < EARLY; q++)
        if (q < cnt) S.keys[excl + q] = composite_key(scale_logit(cl[q], T, y, true), cpos[q]);
#pragma unroll 1
      for (int q = EARLY; q < LCAP; q++) {
        if (!__ballot(q < cnt)) break;
        const int p = next_cand();
        if (q < cnt) S.keys[excl + q] = composite_key(scale_logit(read_logit(p), T, y, true), p);
      }
      n = (int)tot;
    }
    if (lse_in) {
      __syncthreads(); /* the helper wave files lse' before it arrives */
      synced = true;
      lse = lse_in[0];
      eps_s = lse_in[1];
    }
    if constexpr (DRAW) noise = (noise_in && synced) ? noise_in[lane] : draw_noise();
    return finish(n, M, lse, false, eps_s, noise, need_sel);
  }

  __device__ __forceinline__ void run() {
    load();
    (void)compute();
  }
};

/* waves per SIMD the register budget is set for (the row's 4 * CPT
 * registers plus the rest; checked for spills at build time) */
template <int CPT, bool BF16>
constexpr int wave_occupancy() {
  return BF16 ? (CPT <= 8 ? 5 : 4) : (CPT <= 17 ? 5 : 3);
}
/* k_wave_row: at most WR_SPREAD_ROWS one-row workgroups over the CUs, so
 * four waves per SIMD at most; the exact-sum helpers' terms get the room
 * (bf16 rows past 5120 elements: three, the room their 64 words need) */
template <int CPT, bool BF16>
constexpr int row_occupancy() {
  return (BF16 && CPT > 10) ? 3 : wave_occupancy<CPT, BF16>() < 4 ? wave_occupancy<CPT, BF16>() : 4;
}

/* k_linear: the backbone head's logits (src/backbone.c:1213-1215).  Each
 * half-wave takes one logit r and follows the reference's single-row gemv
 * (gemv_half_wave); the sum is rounded to bf16.  k_head (d3s_head.hip) runs
 * the same gemv and samples its logits in the same launch. */
constexpr int LIN_WAVES = 4;
constexpr int LIN_PER_WG = 2 * LIN_WAVES; /* logits per workgroup */

/* LinearArgs's fields as scalar arguments, so all of them are preloaded into
 * SGPRs (9) and the gemv's first loads wait on no kernarg read */
__global__ __launch_bounds__(WAVE *LIN_WAVES) void k_linear(const uint16_t *x, const uint16_t *w, int K, int V,
                                                           int n_rows, uint16_t *y) {
  const LinearArgs la{x, w, K, V, n_rows, y};
  const int n = (int)blockIdx.y;
  const int wid = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / WAVE));
  const int lane = lane_id(), hl = lane & 31;
  const int r = ((int)blockIdx.x * LIN_WAVES + wid) * 2 + (lane >> 5);
  const float acc = gemv_half_wave(la, n, r, hl);
  if (hl == 0 && r < la.V) la.y[(size_t)n * la.V + r] = d3s_f32_to_bf16_rn(acc);
}

/* ------------------------------------------------------------------------
 * k_wide: one 1024-thread workgroup per row too wide for one wave (k <= 64).
 * Wave w holds chunks [w * CPT * 64, (w + 1) * CPT * 64) of the row in its
 * registers and runs the wave kernel's passes over them; the workgroup
 * combines in LDS the maxima, the threshold (the k-th largest of its 1024
 * lane maxima, by 8-bit histogram passes), the candidates and the fast row
 * sums, and wave 0 runs the tail.  A row that needs an exact path (T not
 * finite, logits too large for the fast sum, more candidates than the
 * workgroup files, or a top-p cut within the fast sum's margin) is sampled
 * again by the generic row procedure: the same definition, bit for bit. */
constexpr int WIDE_NW = 16;  /* waves per row */
constexpr int WCAP = 512;    /* candidates the workgroup files */

struct __align__(16) WideLds {
  uint64_t keys[WCAP + 2]; /* candidates, then zero pads for the pair reads */
  uint64_t ranked[WAVE];
  uint32_t hist[NB];
  float buf[WAVE];
  float wmax[WIDE_NW], wsum[WIDE_NW];
  uint32_t wcnt[WIDE_NW];
  uint32_t exact;
};

/* The workgroup's tail once its `tot` candidates (every key that can rank
 * below k) are in S.keys: ranks by counting (thread t < tot counts the keys
 * above its own), then wave 0 runs the wave kernel's cumulative, margin test
 * and race; a cut within the fast sum's margin samples the row again by the
 * generic procedure.  Every thread of the 1024 calls it. */
template <bool BF16>
__device__ __forceinline__ void wide_finish(const SampleArgs &a, int row, WideLds &S, uint64_t *glist,
                                            uint32_t tot, float M, float lse, float eps_s, float noise,
                                            float top_p, int kpow) {
  const int wid = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / WAVE));
  const int lane = lane_id();
  const int k = a.k;
  if (threadIdx.x == 0) {
    S.keys[tot] = 0ull; /* pads below every key */
    S.keys[tot + 1] = 0ull;
  }
  __syncthreads();
  /* ---- ranks: candidate t counts the keys above its own */
  if (threadIdx.x < tot) {
    const uint64_t my = S.keys[threadIdx.x];
    const ulonglong2 *k2 = (const ulonglong2 *)S.keys;
    int rank = 0;
#pragma unroll 4
    for (int j2 = 0; j2 < (int)(tot + 1) / 2; j2++) {
      const ulonglong2 q = k2[j2];
      rank += (q.x > my ? 1 : 0) + (q.y > my ? 1 : 0);
    }
    if (rank < k) S.ranked[rank] = my;
  }
  __syncthreads();
  /* the top k reach x = -inf: the candidates need not hold the -inf ties of
   * lowest index */
  if (key_x(S.ranked[k - 1]) == -__builtin_inff()) {
    generic_row<BF16>(a, row, kpow, glist);
    return;
  }
  /* ---- the tail on wave 0 (the wave kernel's, with its margin test); a cut
   * the fast lse cannot settle samples the row again by the generic procedure */
  if (wid == 0) {
    const uint64_t key = lane < k ? S.ranked[lane] : 0ull;
    const int id = wave_tail(a, row, key, M, lse, false, eps_s, noise, top_p, S.buf,
                             []() { return __builtin_nanf(""); });
    if (id == NEED_EXACT && lane == 0) S.exact = 1u;
  }
  __syncthreads();
  if (S.exact) generic_row<BF16>(a, row, kpow, glist);
}

template <int CPT, bool BF16>
__global__ __launch_bounds__(WAVE *WIDE_NW) __attribute__((amdgpu_waves_per_eu(4)))
void k_wide(SampleArgs a) {
  using C = Chunks<CPT, BF16>;
  constexpr int ES = BF16 ? 2 : 4, EPC = C::EPC, NV = C::NV, NW = WIDE_NW;
  constexpr int EARLY = 3;
  __shared__ WideLds S;
  __shared__ uint64_t glist[KF]; /* the generic procedure's sort list */
  const int row = (int)blockIdx.x;
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
  const float uval = (wid == 0 && lane < k) ? a.u[(size_t)row * k + lane] : 0.0f;
  /* a chunk never crosses a page, so the bytes outside the row it covers are
   * readable; they become -inf below */
  const char *rowp = (const char *)a.logits + (size_t)row * (size_t)a.row_stride * ES;
  const int off = (int)(((uintptr_t)rowp & 15u) / ES);
  const uint4 *src = (const uint4 *)(rowp - off * ES);
  const int nchunks = (off + V + EPC - 1) / EPC;
  const int cbase = wid * CPT * WAVE; /* this wave's first chunk */
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
    if (bc / (CPT * WAVE) == wid) {
      const int jb = (bc % (CPT * WAVE)) / WAVE, lb = bc % WAVE;
#pragma unroll
      for (int j = 0; j < CPT; j++)
        if (j == jb) {
#pragma unroll
          for (int e = 0; e < EPC; e++) c.mask(j * EPC + e, lane == lb && e == eb);
        }
    }
  }

  /* ---- row max of the logits; NaN propagates */
  const float ninf = -__builtin_inff();
  float lm = ninf;
#pragma unroll
  for (int i = 0; i < NV; i++) lm = fmaximum(lm, c.val(i));
  {
    const float wm = wave_maximum_f(lm);
    if (lane == 0) S.wmax[wid] = wm;
  }
  if (threadIdx.x == 0) S.exact = 0u;
  const float noise = wid == 0 ? -d3s_logf(1.0f - uval) : 0.0f; /* the race's noise needs only u */
  __syncthreads();
  bool slow = !t_finite;
  float M = 0.0f, cf = 0.0f, b = 0.0f, delta = 0.0f;
  if (!slow) {
    float Lmax = S.wmax[0];
#pragma unroll
    for (int w = 1; w < NW; w++) Lmax = fmaximum(Lmax, S.wmax[w]);
    if (d3s_isnan(Lmax) || Lmax == __builtin_inff()) {
      if (wid == 0) wave_write_special(a, row, false);
      return;
    }
    M = scale_logit(Lmax, T, y, true); /* = max x */
    if (M == __builtin_inff() || M == ninf) {
      if (wid == 0) wave_write_special(a, row, M == ninf);
      return;
    }
    cf = LOG2E_F / T;
    const float h = Lmax * cf;
    slow = !(fabsf(h) < 0x1p24f);
    b = -h;
    delta = __builtin_fmaf(Lmax, cf, b); /* Lmax * cf + b exactly */
  }
  if (slow) {
    generic_row<BF16>(a, row, kpow, glist);
    return;
  }

  /* ---- tau: the k-th largest of the 1024 lane maxima to 16 bits of its
   * order key (a lower bound: at least k elements reach it; the candidates
   * are ranked exactly after, so a coarser bound only admits a few more) */
  const uint32_t lkey = d3s_ordkey(lm);
  uint32_t prefix = 0u, pmask = 0u, need = (uint32_t)k;
#pragma unroll
  for (int pass = 0; pass < 2; pass++) {
    const int shift = 24 - 8 * pass;
    if (threadIdx.x < NB) S.hist[threadIdx.x] = 0u;
    __syncthreads();
    if ((lkey & pmask) == prefix) atomicAdd(&S.hist[(lkey >> shift) & 255u], 1u);
    __syncthreads();
    const BinSel bs = wave_find_bin<false>(S.hist, need); /* 1024 keys >= need */
    prefix |= bs.bin << shift;
    pmask |= 0xffu << shift;
    need -= bs.above;
    __syncthreads(); /* every wave has read the histogram */
  }
  /* keys below -FLT_MAX's: the k-th lane max is -inf */
  bool need_sel = (a.flags & FLAG_EXACT_SELECT) != 0 || prefix < d3s_ordkey(-0x1.fffffep127f);
  const float tau = d3s_from_ordkey(prefix);
  /* below every logit whose x ties with tau's (as in the wave kernel); a
   * threshold at -inf would take masked padding for candidates */
  float tau_lo = need_sel ? __builtin_inff() : tau - (fabsf(tau) * 0x1p-21f + T * 0x1p-120f);
  if (!(tau_lo >= -0x1.fffffep127f)) {
    need_sel = true;
    tau_lo = __builtin_inff();
  }

  /* ---- the candidates as a bit per element, no branches */
  if (BF16) c.launder();
  constexpr int NWORD = (NV + 31) / 32;
  uint32_t bits[NWORD];
  cand_bits<NV>(bits, [&](int i) { return c.val(i); }, tau_lo);
  int cnt = 0;
#pragma unroll
  for (int w = 0; w < NWORD; w++) cnt += __popc(bits[w]);
  const uint32_t wtot = wave_sum_u32((uint32_t)cnt);
  const bool over = __ballot(cnt > LCAP) != 0ull;
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
  /* the first candidates read again now, while the row is in L2 */
  int cpos[EARLY];
  float cl[EARLY];
#pragma unroll
  for (int q = 0; q < EARLY; q++) {
    cpos[q] = 0;
    cl[q] = 0.0f;
  }
  if (!need_sel && !over) {
#pragma unroll
    for (int q = 0; q < EARLY; q++) {
      if (q > 0 && !__ballot(q < cnt)) break;
      cpos[q] = next_cand();
      if (q < cnt) cl[q] = read_logit(cpos[q]);
    }
  }

  /* ---- the fast row sum */
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
  float sp = S.wsum[0];
#pragma unroll
  for (int w = 0; w < NW; w++) {
    const uint32_t t = S.wcnt[w];
    need_sel = need_sel || t == 0xffffffffu;
    base += w < wid ? t : 0u;
    tot += t;
    if (w > 0) sp = sp + S.wsum[w]; /* the same order in every wave */
  }
  need_sel = need_sel || tot > (uint32_t)WCAP;
  if (need_sel) {
    if (threadIdx.x == 0 && a.counters) atomicAdd(&a.counters[CNT_EXACT_SELECT], 1u);
    generic_row<BF16>(a, row, kpow, glist);
    return;
  }
  const float l2 = __builtin_amdgcn_logf(sp); /* within 2^-23 |log2 sp| + 2^-24 */
  const float lse = M + (l2 * LN2_F - delta * LN2_F);
  /* the wave kernel's bound, with NW - 1 more roundings for the sum over the waves */
  const float eps_s = 0x1p-24f * (2.0f * fabsf(M) + 160.0f) + EPS_EXP2 + 0x1p-23f +
                      (float)(CPT + 11 + NW) * 0x1p-24f + (float)V * 0x1p-40f + 0x1p-22f * fabsf(l2) + 0x1p-23f;

  /* ---- file the keys: this wave's slots from base on, lane by lane */
  {
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
  }
  wide_finish<BF16>(a, row, S, glist, tot, M, lse, eps_s, noise, top_p, kpow);
}


/* The main token of one row from its two draws' indices, on one wave (lane
 * h checks history entry h): candidate index i -> token (0 -> eos, i ->
 * semantic_start + i - 1, src/tower.c:405-409); the retry's token replaces the
 * first's when the first is a semantic token found among the row's history
 * (:429-433); code0 = clip(main - semantic_start, 0, code_vocab - 1) (:434-435).
 * A refused draw (-1: the row's logits give a NaN or +inf x) writes -1 to
 * main_tok and code0, the signal a caller checks where the reference's
 * generation loop dies on non-finite logits (src/generate.c:92,130). */
__device__ __forceinline__ void ras_pick(const RasArgs &ra, int row, int id1, int id2) {
  const int lane = lane_id();
  const int32_t first_tok = id1 == 0 ? ra.eos_id : id1 + ra.semantic_start - 1;
  const int32_t retry_tok = id2 == 0 ? ra.eos_id : id2 + ra.semantic_start - 1;
  const bool seen = lane < ra.history_len && ra.history[(size_t)row * ra.history_len + lane] == first_tok;
  const bool repeated = __ballot(seen) != 0ull && first_tok >= ra.semantic_start && first_tok <= ra.semantic_end;
  const bool refused = id1 < 0 || id2 < 0;
  const int32_t tok = refused ? -1 : repeated ? retry_tok : first_tok;
  if (lane == 0) {
    ra.main_tok[row] = tok;
    if (ra.code0) ra.code0[row] = refused ? -1 : min(max(tok - ra.semantic_start, 0), ra.code_vocab - 1);
  }
}

/* k_ras: the main token's two draws (src/tower.c:425-433) in one launch.  Two
 * waves of a workgroup take one row: the first samples it with the caller's
 * parameters, the second with the retry's, side by side (the second's loads
 * of the row meet the first's in L2, so HBM reads it once).  Then the first
 * wave picks the main token (ras_pick).  helpers (launches of one row per
 * workgroup): waves 2 and 3 take the fast row sums of waves 0 and 1 (the
 * draws' temperatures differ), as k_wave_row's wave 1 does; every wave then
 * passes one barrier before the draws' tails.  Otherwise a workgroup of four
 * waves takes two rows. */
/* k_ras's leading arguments, preloaded into SGPRs as D3S_HOT_PARAMS are for
 * the other one-wave kernels: what both draws' waves need before their row
 * loads (the shared logits, stride, width and row count, each draw's
 * uniforms and temperature, and kk = k | retry k << 8 | helpers << 16).  The
 * draws' per-row temperature and banned arrays are never set on this route
 * and their flags are 0 (checked before launch): the waves take them so.
 * 52 bytes, no padding. */
#define D3S_RAS_HOT_PARAMS                                                                                \
  const void *hot_logits, int64_t hot_stride, const float *hot_u, const float *hot_u_retry, float hot_T,  \
      float hot_T_retry, int hot_vocab, int hot_rows, uint32_t hot_kk
#define D3S_RAS_HOT_ARGS(r, helpers)                                                                      \
  (r).first.logits, (r).first.row_stride, (r).first.u, (r).retry.u, (r).first.temperature_scalar,        \
      (r).retry.temperature_scalar, (r).first.vocab, (r).first.n_rows,                                    \
      (uint32_t)(r).first.k | (uint32_t)(r).retry.k << 8 | (uint32_t)(helpers) << 16

template <int CPT, bool BF16>
__global__ __launch_bounds__(WAVE *WR) __attribute__((amdgpu_waves_per_eu(wave_occupancy<CPT, BF16>())))
void k_ras(D3S_RAS_HOT_PARAMS, RasArgs ra) {
  __shared__ WaveLds lds_all[WR];
  __shared__ int drawn[WR];
  __shared__ float lse_sh[2][2];
  const int helpers = (int)(hot_kk >> 16);
  const int n_rows = hot_rows;
  const int wid = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / WAVE));
  /* (blocks of WAVE * WR threads, as launched) */
  const int row = helpers ? (int)blockIdx.x : (int)(blockIdx.x * (WR / 2)) + wid / 2;
  const bool retry = (wid & 1) != 0;
  const int lane = lane_id();
  SampleArgs a = retry ? ra.retry : ra.first; /* the fields the tail needs, later */
  a.logits = hot_logits;
  a.row_stride = hot_stride;
  a.vocab = hot_vocab;
  a.n_rows = n_rows;
  a.u = retry ? hot_u_retry : hot_u;
  a.temperature = nullptr;
  a.temperature_scalar = retry ? hot_T_retry : hot_T;
  a.banned = nullptr;
  a.k = (int)((hot_kk >> (retry ? 8 : 0)) & 0xffu);
  a.flags = 0u;
  WaveRow<CPT, BF16> r(a, lds_all[wid], row);
  r.V = a.vocab;
  r.k = a.k;
  r.lane = lane;
  if (helpers && wid >= 2) {
    r.load();
    r.helper_lse(lse_sh[wid & 1]);
    __syncthreads();
  } else if (row < n_rows) {
    if (helpers) r.lse_in = lse_sh[wid & 1];
    r.load();
    const int id = r.compute();
    if (lane == 0) drawn[wid] = id;
    if (helpers && !r.synced) __syncthreads();
  }
  __syncthreads();
  if (retry || (helpers && wid >= 2) || row >= n_rows) return;
  ras_pick(ra, row, drawn[wid], drawn[wid + 1]);
}

/* k_wave for small launches: one row per 4-wave workgroup.  Wave 0 samples
 * the row as k_wave's waves do, except for the row sums: wave 1 loads the row
 * too (its loads meet wave 0's in L2) and takes the max, the fast sum and a
 * fifth of the exact row sum (the 2^-40 fixed-point sum of d3s_expf(x - M)),
 * waves 2 and 3 the rest of the exact sum, while wave 0 runs the threshold,
 * the candidates and their filing.  Wave 0 reads lse' after the workgroup's
 * one barrier, just before its tail (or passes it here, on rows that end
 * earlier); a cut within the fast lse's margin takes the exact lse from the
 * helpers' shares and the tail goes on in the exact order, with no second
 * pass over the row. */
template <int CPT, bool BF16, bool DRAW = false>
__global__ __launch_bounds__(WAVE *WR) __attribute__((amdgpu_waves_per_eu(row_occupancy<CPT, BF16>())))
void k_wave_row(D3S_HOT_PARAMS_T(DRAW), SampleArgs a) {
  if constexpr (DRAW)
    D3S_DRAW_APPLY(a);
  else
    D3S_HOT_APPLY(a);
  __shared__ WaveLds lds;
  __shared__ float lse_sh[2];
  __shared__ uint64_t ex_sh[3];
  __shared__ float noise_sh[DRAW ? WAVE : 1];
  const int wid = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / WAVE));
  const int lane = lane_id();
  const int row = (int)blockIdx.x;
  WaveRow<CPT, BF16, DRAW> r(a, lds, row);
  r.V = a.vocab;
  r.k = a.k;
  r.lane = lane;
  /* the exact-sum helpers' loads wait ~512 cycles: issued with wave 0's,
   * they share the CU's load path with them (C1 0.2 us slower); a little
   * later they read L2 after wave 0's row is in, and still finish before
   * wave 0 reaches its tail (2048 cycles: too late) */
  if (wid >= 2) __builtin_amdgcn_s_sleep(8);
  if constexpr (DRAW)
    if (wid == 2) r.noise_out = noise_sh;
  r.load();
  if (wid == 0) {
    r.lse_in = lse_sh;
    r.ex_in = ex_sh;
    r.defer_exact = true; /* (never reached: ex_in answers first) */
    if constexpr (DRAW) r.noise_in = noise_sh;
    (void)r.compute();
    if (!r.synced) __syncthreads();
  } else {
    if (wid == 1)
      r.helper_lse(lse_sh, &ex_sh[0]);
    else
      r.helper_exact(&ex_sh[wid - 1], wid - 2);
    __syncthreads();
  }
}

/* The pick alone, one wave per row, after the two draws ran as separate
 * launches that wrote their indices to `first` and `retry` (rows the fused
 * kernel does not hold: k above 64, or rows wider than one wave's registers). */
__global__ __launch_bounds__(WAVE *WR) void k_ras_select(RasArgs ra, const int32_t *first, const int32_t *retry) {
  const int wid = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / WAVE));
  const int row = (int)(blockIdx.x * WR) + wid;
  if (row >= ra.first.n_rows) return;
  ras_pick(ra, row, first[row], retry[row]);
}

template <int CPT, bool BF16>
__global__ __launch_bounds__(WAVE *WR) __attribute__((amdgpu_waves_per_eu(wave_occupancy<CPT, BF16>())))
void k_wave(D3S_HOT_PARAMS, SampleArgs a) {
  D3S_HOT_APPLY(a);
  __shared__ WaveLds lds_all[WR];
  /* wave-uniform (the compiler cannot see it): row and all that follows stay scalar */
  const int wid = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / WAVE));
  const int row = (int)(blockIdx.x * (blockDim.x / WAVE)) + wid;
  if (row >= a.n_rows) return;
  WaveRow<CPT, BF16> r(a, lds_all[wid], row);
  r.V = a.vocab;
  r.k = a.k;
  r.lane = lane_id();
  r.reg_cands = true;
  r.run();
}

__global__ void k_log2(const float *in, float *out, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = __builtin_amdgcn_logf(in[i]);
}

__global__ void k_exp2(const float *in, float *out, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = __builtin_amdgcn_exp2f(in[i]);
}

/* the widest row k_wave<CPT, BF16> holds: rows starting off elements past a
 * 16-byte boundary need off more slots */
template <int CPT, bool BF16>
constexpr int wave_vmax(int off) {
  return WAVE * CPT * (16 / (BF16 ? 2 : 4)) - off;
}

template <int CPT, bool BF16>
bool try_wave(const SampleArgs &a, int max_off, hipStream_t s) {
  if (a.vocab > wave_vmax<CPT, BF16>(max_off)) return false;
  /* a launch too small to fill the chip spreads its rows one per workgroup
   * over more CUs, with three helper waves for the exact lse; larger ones
   * pack WR rows, which keeps the CUs fuller */
  if (!a.u) { /* the call's draw in the kernel: one-row launches only */
    if (a.n_rows > WR_SPREAD_ROWS || !D3S_DRAW_FITS(a)) return false;
    hipLaunchKernelGGL((k_wave_row<CPT, BF16, true>), dim3((unsigned)a.n_rows), dim3(WAVE * WR), 0, s,
                       D3S_DRAW_ARGS(a), a);
  } else if (a.n_rows <= WR_SPREAD_ROWS)
    hipLaunchKernelGGL((k_wave_row<CPT, BF16>), dim3((unsigned)a.n_rows), dim3(WAVE * WR), 0, s, D3S_HOT_ARGS(a), a);
  else
    hipLaunchKernelGGL((k_wave<CPT, BF16>), dim3((unsigned)((a.n_rows + WR - 1) / WR)), dim3(WAVE * WR), 0, s,
                       D3S_HOT_ARGS(a), a);
  return true;
}

/* the widest row k_wide<CPT, BF16> holds, at any start offset */
template <int CPT, bool BF16>
constexpr int wide_vmax() {
  return WIDE_NW * WAVE * CPT * (16 / (BF16 ? 2 : 4)) - (16 / (BF16 ? 2 : 4) - 1);
}

template <int CPT, bool BF16>
bool try_wide(const SampleArgs &a, hipStream_t s) {
  if (a.vocab > wide_vmax<CPT, BF16>()) return false;
  hipLaunchKernelGGL((k_wide<CPT, BF16>), dim3(a.n_rows), dim3(WAVE * WIDE_NW), 0, s, a);
  return true;
}

}  // namespace

void launch_log2_selftest(const float *in, float *out, int64_t n, hipStream_t s) {
  if (n <= 0) return;
  const int B = 256;
  hipLaunchKernelGGL(k_log2, dim3((unsigned)((n + B - 1) / B)), dim3(B), 0, s, in, out, n);
}

void launch_exp2_selftest(const float *in, float *out, int64_t n, hipStream_t s) {
  if (n <= 0) return;
  const int B = 256;
  hipLaunchKernelGGL(k_exp2, dim3((unsigned)((n + B - 1) / B)), dim3(B), 0, s, in, out, n);
}

template <int CPT, bool BF16>
bool try_ras(const RasArgs &r, int max_off, hipStream_t s) {
  if (r.first.vocab > wave_vmax<CPT, BF16>(max_off)) return false;
  /* two waves per row: for small launches one row per workgroup with two
   * helper waves, otherwise two rows per workgroup */
  const int n = r.first.n_rows;
  const int rpw = n <= WR_SPREAD_ROWS ? 1 : WR / 2;
  hipLaunchKernelGGL((k_ras<CPT, BF16>), dim3((unsigned)((n + rpw - 1) / rpw)), dim3(WAVE * WR), 0, s,
                     D3S_RAS_HOT_ARGS(r, rpw == 1 ? 1 : 0), r);
  return true;
}

bool launch_ras(const RasArgs &r, Dtype dt, hipStream_t s) {
  if (r.first.k > KF || r.retry.k > KF) return false;
  /* what k_ras takes as given (its leading arguments carry the rest) */
  if (r.first.temperature || r.retry.temperature || r.first.banned || r.retry.banned || r.first.flags ||
      r.retry.flags || r.first.logits != r.retry.logits || r.first.row_stride != r.retry.row_stride ||
      r.first.vocab != r.retry.vocab || r.first.n_rows != r.retry.n_rows)
    return false;
  const SampleArgs &a = r.first;
  const int es = dt == DT_F32 ? 4 : 2;
  const bool aligned = ((uintptr_t)a.logits % 16u) == 0u && (a.row_stride * es) % 16 == 0;
  const int max_off = aligned ? 0 : 16 / es - 1;
  if (dt == DT_F32)
    return try_ras<4, false>(r, max_off, s) || try_ras<8, false>(r, max_off, s) ||
           try_ras<17, false>(r, max_off, s) || try_ras<24, false>(r, max_off, s);
  return try_ras<4, true>(r, max_off, s) || try_ras<8, true>(r, max_off, s) ||
         try_ras<10, true>(r, max_off, s) || try_ras<16, true>(r, max_off, s);
}

void launch_ras_select(const RasArgs &r, const int32_t *first, const int32_t *retry, hipStream_t s) {
  const unsigned blocks = (unsigned)((r.first.n_rows + WR - 1) / WR);
  hipLaunchKernelGGL(k_ras_select, dim3(blocks), dim3(WAVE * WR), 0, s, r, first, retry);
}

void launch_linear(const LinearArgs &la, hipStream_t s) {
  const unsigned groups = (unsigned)((la.V + LIN_PER_WG - 1) / LIN_PER_WG);
  hipLaunchKernelGGL(k_linear, dim3(groups, (unsigned)la.n_rows), dim3(WAVE * LIN_WAVES), 0, s, la.x, la.w, la.K,
                     la.V, la.n_rows, la.y);
}

int wide_max_vocab(Dtype dt) { return dt == DT_F32 ? wide_vmax<19, false>() : wide_vmax<19, true>(); }

bool launch_wide(const SampleArgs &a, Dtype dt, hipStream_t s) {
  if (a.k > KF) return false;
  return dt == DT_F32 ? try_wide<19, false>(a, s) : try_wide<19, true>(a, s);
}

int wave_max_vocab(Dtype dt) { return dt == DT_F32 ? wave_vmax<24, false>(3) : wave_vmax<16, true>(7); }

bool launch_wave(const SampleArgs &a, Dtype dt, hipStream_t s) {
  if (a.k > KF) return false;
  /* the largest start offset of a row within its 16-byte chunk: 0 when the
   * base and the stride are both 16-byte multiples */
  const int es = dt == DT_F32 ? 4 : 2;
  const bool aligned = ((uintptr_t)a.logits % 16u) == 0u && (a.row_stride * es) % 16 == 0;
  const int max_off = aligned ? 0 : 16 / es - 1;
  if (dt == DT_F32)
    return try_wave<4, false>(a, max_off, s) || try_wave<8, false>(a, max_off, s) ||
           try_wave<16, false>(a, max_off, s) || try_wave<17, false>(a, max_off, s) ||
           try_wave<24, false>(a, max_off, s);
  /* (9 chunk rows per lane is left out: it allocates registers badly) */
  return try_wave<4, true>(a, max_off, s) || try_wave<8, true>(a, max_off, s) ||
         try_wave<10, true>(a, max_off, s) || try_wave<16, true>(a, max_off, s);
}

}  // namespace d3s
