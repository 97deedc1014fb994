/* Deterministic fp32 arithmetic shared, as the same source, by the HIP kernels and
 * by the CPU build (the C oracle, the host side of the library).
 *
 * Every function here is a fixed sequence of IEEE-754 binary32 operations that
 * are correctly rounded on both targets (add, sub, mul, true division, fused
 * multiply-add) plus integer work, so a CPU and a gfx950 GPU produce the same
 * bits.  Callers must compile with floating-point contraction off
 * (-ffp-contract=off): a fused a*b+c where the source says two operations
 * would change the rounding.
 *
 * The sampler of SeungheonOh/drama3-mlx (src/sampling.c:123-139) uses Apple's
 * metal::precise::exp, metal::fast::exp and metal::precise::log; their bit
 * patterns are unpublished, so exp and log are written here from published
 * methods instead:
 *   - d3s_expf: Cody & Waite argument reduction a = n*ln2 + r (Cody & Waite,
 *     "Software Manual for the Elementary Functions", 1980) with a two-part ln2,
 *     then the degree-7 Taylor polynomial of e^r on |r| <= ln2/2 (truncation
 *     error < 6e-9 relative), then exact scaling by 2^n.
 *   - d3s_logf: y = 2^e * m with m in [sqrt(2)/2, sqrt(2)), f = m - 1,
 *     s = f/(2+f), log(m) = 2*atanh(s) evaluated as f - s*(f - R) with
 *     R = s*z*(2/3 + 2z/5 + 2z^2/7 + 2z^3/9), z = s^2 (|s| <= 0.1716, truncation
 *     error < 3e-9 relative), log(y) = e*ln2 + log(m) with the two-part ln2.
 * Both are checked against double-precision libm over dense sweeps by the
 * tests (error below 1 ulp), on the CPU and, bit for bit, on the GPU.
 */
#ifndef D3S_MATH_H
#define D3S_MATH_H

#include <stdint.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define D3S_HD __host__ __device__ __forceinline__
#define D3S_FMAF __builtin_fmaf
#else
#include <math.h>
#include <string.h>
#define D3S_HD static inline
#define D3S_FMAF fmaf
#endif

#ifdef __cplusplus
#define D3S_INF (__builtin_inff())
#define D3S_NAN (__builtin_nanf(""))
#else
#define D3S_INF (__builtin_inff())
#define D3S_NAN (__builtin_nanf(""))
#endif

D3S_HD uint32_t d3s_f2u(float f) {
#if defined(__HIPCC__)
  return __builtin_bit_cast(uint32_t, f);
#else
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
#endif
}

D3S_HD float d3s_u2f(uint32_t u) {
#if defined(__HIPCC__)
  return __builtin_bit_cast(float, u);
#else
  float f;
  memcpy(&f, &u, 4);
  return f;
#endif
}

/* bf16 -> fp32 is exact: the bf16 bits are the top half of the fp32 bits. */
D3S_HD float d3s_bf16_to_f32(uint16_t b) { return d3s_u2f((uint32_t)b << 16); }

/* fp32 -> bf16, rounded to nearest even; NaN -> a quiet NaN of the same sign
 * (MLX's bfloat16 conversion, used when the reference's gemv stores its result) */
D3S_HD uint16_t d3s_f32_to_bf16_rn(float f) {
  const uint32_t b = d3s_f2u(f);
  if ((b & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((b >> 16) | 0x0040u);
  return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

/* Order-preserving key: a > b (as floats, NaN excluded) iff key(a) > key(b).
 * -0 and +0 compare equal, so -0 is mapped to the key of +0. */
D3S_HD uint32_t d3s_ordkey(float f) {
  uint32_t b = d3s_f2u(f);
  if (b == 0x80000000u) b = 0u;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

D3S_HD float d3s_from_ordkey(uint32_t k) {
  return d3s_u2f((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

D3S_HD int d3s_isnan(float f) { return (d3s_f2u(f) & 0x7fffffffu) > 0x7f800000u; }

/* The shared core of the exponentials below: for ac in [-104, 89], n =
 * round(ac log2 e) (ties to even, exact for |t| < 2^22) and exp's polynomial
 * value p in [2^-1/2, 2^1/2] at r = ac - n ln 2 (Cody-Waite, ln 2 in two
 * parts, the first product exact); e^ac = p 2^n. */
D3S_HD float d3s_exp_core(float ac, float *n_out) {
#if defined(__clang__)
#pragma clang fp contract(off)
#endif
  const float t = ac * 0x1.715476p+0f;                        /* a * log2(e) */
#if defined(__HIP_DEVICE_COMPILE__)
  const float n = __builtin_rintf(t); /* the same: |t| < 2^22, ties to even (v_rndne_f32) */
#else
  const float n = (t + 0x1.8p+23f) - 0x1.8p+23f;
#endif
  float r = D3S_FMAF(n, -0x1.62e400p-1f, ac); /* a - n*ln2_hi (exact) */
  r = D3S_FMAF(n, -0x1.7f7d1cp-20f, r);       /* - n*ln2_lo */
  float p = 0x1.a01a02p-13f;                  /* 1/7! */
  p = D3S_FMAF(p, r, 0x1.6c16c2p-10f);        /* 1/6! */
  p = D3S_FMAF(p, r, 0x1.111112p-7f);         /* 1/5! */
  p = D3S_FMAF(p, r, 0x1.555556p-5f);         /* 1/4! */
  p = D3S_FMAF(p, r, 0x1.555556p-3f);         /* 1/3! */
  p = D3S_FMAF(p, r, 0x1.0p-1f);              /* 1/2! */
  p = D3S_FMAF(p, r, 1.0f);
  p = D3S_FMAF(p, r, 1.0f);
  *n_out = n;
  return p;
}

/* e^a, correctly handling NaN, +-inf, overflow and subnormal results.
 * Branch-free: the main path runs on a clamped argument and the special cases
 * are selected at the end (divergent branches are costly on a GPU wave). */
D3S_HD float d3s_expf(float a) {
#if defined(__clang__)
#pragma clang fp contract(off)
#endif
  const float ac = fminf(fmaxf(a, -0x1.a0p+6f), 0x1.64p+6f); /* [-104, 89]; NaN -> -104 */
  float n;
  const float p = d3s_exp_core(ac, &n);
  const int ni = (int)n; /* -150 <= ni <= 128 */
  /* p * 2^ni with one rounding: the first product is exact, the second rounds
   * into the subnormal range (or overflows) when it has to. */
  const int lo = ni < -126, hi = ni > 127;
  const int ns = lo ? ni + 127 : (hi ? ni - 1 : ni);
  const float s2 = lo ? 0x1.0p-127f : (hi ? 2.0f : 1.0f);
  float res = (p * d3s_u2f((uint32_t)(ns + 127) << 23)) * s2;
  res = a > 0x1.62e430p+6f ? D3S_INF : res; /* > 88.7228394: overflows */
  res = a < -0x1.a0p+6f ? 0.0f : res;       /* < -104: below half the least subnormal */
  return d3s_isnan(a) ? a : res;
}

/* d3s_expf(a) for a <= 88 or -inf (not NaN): the same bits without the
 * overflow and NaN cases (up to 88, n <= 127). */
D3S_HD float d3s_expf_nonpos(float a) {
#if defined(__clang__)
#pragma clang fp contract(off)
#endif
  const float ac = fmaxf(a, -0x1.a0p+6f); /* [-104, 88] */
  float n;
  const float p = d3s_exp_core(ac, &n);
  const int ni = (int)n; /* -150 <= ni <= 127 */
  const int lo = ni < -126;
  const float s2 = lo ? 0x1.0p-127f : 1.0f;
  const float res = (p * d3s_u2f((uint32_t)((lo ? ni + 127 : ni) + 127) << 23)) * s2;
  return a < -0x1.a0p+6f ? 0.0f : res;
}

/* natural log, correctly handling NaN, negative, zero, subnormal and +inf;
 * branch-free like d3s_expf. */
D3S_HD float d3s_logf(float y) {
#if defined(__clang__)
#pragma clang fp contract(off)
#endif
  const uint32_t b0 = d3s_f2u(y);
  const int sub = b0 < 0x00800000u; /* +0 or a positive subnormal: scale into the normal range */
  const uint32_t b = sub ? d3s_f2u(y * 0x1.0p+23f) : b0;
  int e = (sub ? -23 : 0) + (int)((b >> 23) & 0xffu) - 127;
  float m = d3s_u2f((b & 0x007fffffu) | 0x3f800000u); /* [1, 2) */
  const int big = m > 0x1.6a09e6p+0f;                 /* > sqrt(2) */
  m = big ? m * 0.5f : m;
  e += big;
  const float f = m - 1.0f; /* exact */
  const float s = f / (2.0f + f);
  const float z = s * s;
  /* 2*atanh(s) = 2s + s*z*(2/3 + 2z/5 + ...), and 2s = f - s*f exactly in
   * real arithmetic, so log(1+f) = f - s*(f - R) with R = z*(2/3 + 2z/5 + ...):
   * the exact f carries the result and the rounding of s only touches the
   * small correction term. */
  float q = 0x1.c71c72p-3f;          /* 2/9 */
  q = D3S_FMAF(q, z, 0x1.24924ap-2f); /* 2/7 */
  q = D3S_FMAF(q, z, 0x1.99999ap-2f); /* 2/5 */
  q = D3S_FMAF(q, z, 0x1.555556p-1f); /* 2/3 */
  const float R = z * q;
  const float lm = D3S_FMAF(-s, f - R, f);
  const float ef = (float)e;
  float res = D3S_FMAF(ef, 0x1.7f7d1cp-20f, lm); /* + e*ln2_lo */
  res = D3S_FMAF(ef, 0x1.62e400p-1f, res);       /* + e*ln2_hi */
  res = y == D3S_INF ? D3S_INF : res;
  res = y == 0.0f ? -D3S_INF : res;
  res = y < 0.0f ? D3S_NAN : res;
  return d3s_isnan(y) ? y : res;
}

/* a / b correctly rounded, given y = RN(1/b) (b finite, nonzero, 2^-126 < |b| < 2^126):
 * q = RN(a*y) is within one ulp of a/b, the remainder r = a - b*q is exact in
 * one fused multiply-add, and RN(q + r*y) is RN(a/b) (Markstein, "Computation
 * of elementary functions on the IBM RISC System/6000 processor", IBM J. Res.
 * Dev. 34(1), 1990; Muller et al., Handbook of Floating-Point Arithmetic, 2nd
 * ed., section 5.3).  Operands whose remainder or quotient could leave the
 * normal range (|a| below 2^-60 or above 2^100, b outside [2^-20, 2^21),
 * infinities, NaN) take the division instead; zero is exact either way up to
 * the sign of a zero result. */
D3S_HD float d3s_div_rn(float a, float b, float y) {
#if defined(__clang__)
#pragma clang fp contract(off)
#endif
  const uint32_t ea = (d3s_f2u(a) >> 23) & 0xffu; /* biased exponent of a */
  const uint32_t eb = (d3s_f2u(b) >> 23) & 0xffu; /* of b (b > 0) */
  if (ea < 127u - 60u || ea > 127u + 100u || eb < 127u - 20u || eb > 127u + 20u) return a / b;
  const float q = a * y;
  const float r = D3S_FMAF(-q, b, a);
  return D3S_FMAF(r, y, q);
}

/* Fixed-point image of a probability-like term e in [0, 1]: floor(e * 2^40).
 * Sums of these are exact in uint64 (up to 2^23 terms), so a sum does not
 * depend on the order the terms are added in. */
#define D3S_FIX_BITS 40
D3S_HD uint64_t d3s_fix40(float e) {
  const uint32_t b = d3s_f2u(e);
  const uint32_t E = (b >> 23) & 0xffu;
  const uint64_t m = (uint64_t)((b & 0x007fffffu) | (E ? 0x00800000u : 0u));
  /* e = m * 2^(max(E,1) - 150), so e * 2^40 = m * 2^(max(E,1) - 110); the
   * shifts are clamped so every lane computes both cases without overflow */
  const int sh = 110 - (int)(E ? E : 1u);
  const uint64_t left = m << (sh < 0 ? (-sh > 16 ? 16 : -sh) : 0); /* e in [2^-17, 1) */
  const uint64_t right = m >> (sh > 63 ? 63 : (sh > 0 ? sh : 0));
  uint64_t r = sh <= 0 ? left : right;
  r = e >= 1.0f ? ((uint64_t)1 << D3S_FIX_BITS) : r;
  return e > 0.0f ? r : 0; /* 0, -0, negative, NaN */
}

/* d3s_fix40(e) for e in [0, 1] (not NaN), in float operations: F = e 2^40 is
 * exact and below 2^40 + 1; its integer part is hi 2^32 + lo with hi =
 * trunc(F 2^-32) and lo = trunc(F - hi 2^32), the subtraction exact (both
 * terms are multiples of F's ulp and the difference is below 2^32). */
D3S_HD uint64_t d3s_fix40_unit(float e) {
#if defined(__clang__)
#pragma clang fp contract(off)
#endif
  const float F = e * 0x1.0p+40f;
  const uint32_t hi = (uint32_t)(F * 0x1.0p-32f);
  const uint32_t lo = (uint32_t)(F - (float)hi * 0x1.0p+32f);
  return ((uint64_t)hi << 32) | lo;
}

/* d3s_fix40(d3s_expf(z)) for z <= 0 (or -0, or -inf), without forming the
 * fp32 result: exp's polynomial value p lies in [2^-1/2, 2^1/2], so p * 2^24
 * is an integer P below 2^25 and floor(p * 2^n * 2^40) = floor(P * 2^(n + 16))
 * = (P * 2^16) >> -n (n <= 0): one 64-bit shift.  Arguments below -43 give 0
 * (e^-43 2^40 < 2^-22), as the clamp to -43 does (n >= -62, so the shift
 * stays below 64, and P 2^16 < 2^41 shifted by 62 is 0).  Same bits as the
 * two-step form; fewer instructions for the per-element row sum. */
D3S_HD uint64_t d3s_fix40_exp(float z) {
  const float zc = fmaxf(z, -43.0f); /* [-43, 0]; -inf -> -43 */
  float n;
  const float p = d3s_exp_core(zc, &n);
  const uint64_t P16 = (uint64_t)(uint32_t)(p * 0x1.0p+24f) << 16; /* below 2^41 */
  return P16 >> (int)(-n);                                          /* 0 <= -n <= 62 */
}

/* uint64 -> fp32, round to nearest, ties to even (integer steps only). */
D3S_HD float d3s_u64_to_f32(uint64_t v) {
  if (v == 0) return 0.0f;
  int lz = 0;
  {
    uint64_t t = v;
    if (!(t >> 32)) { lz += 32; t <<= 32; }
    if (!(t >> 48)) { lz += 16; t <<= 16; }
    if (!(t >> 56)) { lz += 8; t <<= 8; }
    if (!(t >> 60)) { lz += 4; t <<= 4; }
    if (!(t >> 62)) { lz += 2; t <<= 2; }
    if (!(t >> 63)) { lz += 1; }
  }
  const int msb = 63 - lz;
  if (msb < 24) return d3s_u2f(((uint32_t)(127 + msb) << 23) | (((uint32_t)v << (23 - msb)) & 0x7fffffu));
  const int sh = msb - 23;
  uint64_t mant = v >> sh;
  const uint64_t rem = v & ((((uint64_t)1) << sh) - 1);
  const uint64_t half = ((uint64_t)1) << (sh - 1);
  int ex = msb;
  if (rem > half || (rem == half && (mant & 1))) {
    mant += 1;
    if (mant >> 24) {
      mant >>= 1;
      ex += 1;
    }
  }
  return d3s_u2f(((uint32_t)(127 + ex) << 23) | ((uint32_t)mant & 0x7fffffu));
}

/* fixed-point sum (scale 2^40) -> fp32, round to nearest */
D3S_HD float d3s_fixsum_to_f32(uint64_t s) { return d3s_u64_to_f32(s) * 0x1.0p-40f; }

/* The smallest s with d3s_fixsum_to_f32(s) > c (UINT64_MAX when none, c NaN
 * or at least 2^23), so that the test is one integer comparison.  With
 * t = c * 2^40 (exact): below 2^24 every integer converts exactly, so s =
 * floor(t) + 1; from 2^24 on t is an integer with half-ulp h = 2^(e - 24),
 * s = t + h rounds to the even neighbour, which is above t when t's last
 * mantissa bit is 1, and to t otherwise (then s = t + h + 1). */
D3S_HD uint64_t d3s_fixsum_gt_threshold(float c) {
  const float t = c * 0x1.0p+40f;
  if (!(t >= 0.0f)) return t < 0.0f ? 0ull : ~0ull;
  if (t >= 0x1.0p+63f) return ~0ull;
  if (t < 0x1.0p+24f) return (uint64_t)t + 1ull;
  const uint32_t b = d3s_f2u(t);
  const int e = (int)((b >> 23) & 0xffu) - 127;
  return (uint64_t)t + (1ull << (e - 24)) + ((b & 1u) ? 0ull : 1ull);
}

/* ---- Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11) ---- */
typedef struct {
  uint32_t v[4];
} d3s_u32x4;

D3S_HD void d3s_mulhilo(uint32_t a, uint32_t b, uint32_t *hi, uint32_t *lo) {
  const uint64_t p = (uint64_t)a * (uint64_t)b;
  *hi = (uint32_t)(p >> 32);
  *lo = (uint32_t)p;
}

D3S_HD d3s_u32x4 d3s_philox4x32_10(d3s_u32x4 c, uint32_t k0, uint32_t k1) {
  for (int i = 0; i < 10; i++) {
    uint32_t hi0, lo0, hi1, lo1;
    d3s_mulhilo(0xD2511F53u, c.v[0], &hi0, &lo0);
    d3s_mulhilo(0xCD9E8D57u, c.v[2], &hi1, &lo1);
    d3s_u32x4 n;
    n.v[0] = hi1 ^ c.v[1] ^ k0;
    n.v[1] = lo1;
    n.v[2] = hi0 ^ c.v[3] ^ k1;
    n.v[3] = lo0;
    c = n;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return c;
}

/* The uniform draw number `index` of draw call `stream` under `seed`:
 * counter (index/4, stream), key seed, word index%4, 24 random bits.
 * Values are multiples of 2^-24 in [0, 1), exact in fp32. */
D3S_HD float d3s_uniform(uint64_t seed, uint64_t stream, uint64_t index) {
  d3s_u32x4 c;
  const uint64_t q = index >> 2;
  c.v[0] = (uint32_t)q;
  c.v[1] = (uint32_t)(q >> 32);
  c.v[2] = (uint32_t)stream;
  c.v[3] = (uint32_t)(stream >> 32);
  const d3s_u32x4 o = d3s_philox4x32_10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
  /* selects, not o.v[index & 3]: a run-time index into the array makes the
   * device compiler move it to LDS, which needs the dispatch packet and so
   * costs the kernel two preloaded argument registers */
  const uint32_t j = (uint32_t)index & 3u;
  const uint32_t w = j == 0 ? o.v[0] : j == 1 ? o.v[1] : j == 2 ? o.v[2] : o.v[3];
  return (float)(w >> 8) * 0x1.0p-24f;
}

#endif /* D3S_MATH_H */
