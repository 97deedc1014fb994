/* The head's single-row gemv (gfx950, wave64), shared by k_linear (logits
 * only) and k_head (logits and their sample in one launch).  Device code only;
 * every translation unit gets its own copy. */
#ifndef D3S_GEMV_H
#define D3S_GEMV_H

#include "d3s_device.h"

namespace d3s {
namespace {

/* Logit r of row n (src/mlxu.c:365-400): the calling half-wave's 32 lanes
 * (hl = lane within the half) accumulate in fp32, lane hl the products of
 * elements c*128 + 4 hl + t in block order, fused (fma); a shuffle-down tree
 * over 16, 8, 4, 2, 1 lanes adds them.  Lane hl = 0 returns the sum (the caller
 * rounds it to bf16); a half-wave with r >= V returns 0.  Every lane of the
 * wave calls it (the tree's shuffles). */
__device__ __forceinline__ float gemv_half_wave(const LinearArgs &la, int n, int r, int hl) {
  const int KB = la.K / 128;
  float acc = 0.0f;
  if (r < la.V) {
    const uint2 *wp = (const uint2 *)(la.w + (size_t)r * la.K) + hl;
    const uint2 *xp = (const uint2 *)(la.x + (size_t)n * la.K) + hl;
    for (int c0 = 0; c0 < KB; c0 += 16) {
      uint2 wv[16], xv[16];
#pragma unroll
      for (int c = 0; c < 16; c++)
        if (c0 + c < KB) {
          wv[c] = wp[(c0 + c) * 32];
          xv[c] = xp[(c0 + c) * 32];
        }
#pragma unroll
      for (int c = 0; c < 16; c++)
        if (c0 + c < KB) {
          const uint32_t wq[2] = {wv[c].x, wv[c].y}, xq[2] = {xv[c].x, xv[c].y};
#pragma unroll
          for (int t = 0; t < 4; t++) {
            const float wf = d3s_u2f(t & 1 ? wq[t / 2] & 0xffff0000u : wq[t / 2] << 16);
            const float xf = d3s_u2f(t & 1 ? xq[t / 2] & 0xffff0000u : xq[t / 2] << 16);
            acc = __builtin_fmaf(wf, xf, acc);
          }
        }
    }
  }
#pragma unroll
  for (int sn = 16; sn >= 1; sn >>= 1) acc = acc + __shfl_down(acc, sn, 32);
  return acc;
}

/* gemv_half_wave for NL logits r0 .. r0 + NL - 1 of row n at once (those
 * below V; acc[j] of lane hl = 0 holds logit r0 + j, 0 past V): the shared
 * x values are loaded once, and NL independent chains keep more loads in
 * flight.  Each logit's arithmetic is gemv_half_wave's, in the same order. */
template <int NL>
__device__ __forceinline__ void gemv_half_wave_n(const LinearArgs &la, int n, int r0, int hl, float (&acc)[NL]) {
  constexpr int CH = NL <= 2 ? 16 : 8; /* blocks whose loads are in flight together */
  const int KB = la.K / 128;
  const uint2 *xp = (const uint2 *)(la.x + (size_t)n * la.K) + hl;
  const uint2 *wp[NL];
  bool live[NL];
#pragma unroll
  for (int j = 0; j < NL; j++) {
    acc[j] = 0.0f;
    live[j] = r0 + j < la.V;
    wp[j] = (const uint2 *)(la.w + (size_t)(live[j] ? r0 + j : 0) * la.K) + hl;
  }
  for (int c0 = 0; c0 < KB; c0 += CH) {
    uint2 xv[CH], wv[NL][CH];
#pragma unroll
    for (int c = 0; c < CH; c++)
      if (c0 + c < KB) {
        xv[c] = xp[(c0 + c) * 32];
#pragma unroll
        for (int j = 0; j < NL; j++)
          if (live[j]) wv[j][c] = wp[j][(c0 + c) * 32];
      }
#pragma unroll
    for (int c = 0; c < CH; c++)
      if (c0 + c < KB) {
        const uint32_t xq[2] = {xv[c].x, xv[c].y};
#pragma unroll
        for (int j = 0; j < NL; j++)
          if (live[j]) {
            const uint32_t wq[2] = {wv[j][c].x, wv[j][c].y};
#pragma unroll
            for (int t = 0; t < 4; t++) {
              const float wf = d3s_u2f(t & 1 ? wq[t / 2] & 0xffff0000u : wq[t / 2] << 16);
              const float xf = d3s_u2f(t & 1 ? xq[t / 2] & 0xffff0000u : xq[t / 2] << 16);
              acc[j] = __builtin_fmaf(wf, xf, acc[j]);
            }
          }
      }
  }
#pragma unroll
  for (int j = 0; j < NL; j++)
#pragma unroll
    for (int sn = 16; sn >= 1; sn >>= 1) acc[j] = acc[j] + __shfl_down(acc[j], sn, 32);
}

}  // namespace
}  // namespace d3s

#endif
