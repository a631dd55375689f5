// kl_sums.h — the paired logits GEMM's per-tile KL sums and how they are
// re-expressed against other maxima when tiles (or half tiles) merge.
// Device code shared by gemm.hip (the epilogue's two column halves) and
// rowpass.hip (the tiles of a row).
//
// For a range of columns j of one (student s, teacher t) row pair with the
// rows' own maxima ms, mt over the range, the sums are
//   x = Σ e^((t_j - mt)/T) · ((t_j - mt) - (s_j - ms))·log2(e)
//   y = Σ (e^((s_j - ms)/T) - e^((t_j - mt)/T))
// next to the rows' statistics Σ e^((s_j - ms)/T) and Σ e^((t_j - mt)/T).
// Each element's terms are relative to the two maxima, so a constant offset
// between the rows cancels element by element, and y's differences are
// rounded before they are summed. Over a whole row,
//   KL = x·ln2/(T·Σe^((t-mt)/T)) + log1p(y / Σe^((t-mt)/T))
// (the mean of (t - s)/T under p_t^T plus lse_s^T - lse_t^T, both shifted by
// (mt - ms)/T in opposite directions).
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>

namespace orda {

// 2^(-q) - 1 for |q| < 1/4 from its Taylor series in x = -q·ln2 (the
// remainder x^7/5040 is below 1e-9 of the result there), so that a factor
// near 1 keeps its small difference from 1 exactly.
__device__ __forceinline__ float exp2m1_small(float q) {
  const float x = -q * 0.6931471805599453f;
  float p = fmaf(x, 1.f / 720.f, 1.f / 120.f);
  p = fmaf(x, p, 1.f / 24.f);
  p = fmaf(x, p, 1.f / 6.f);
  p = fmaf(x, p, 0.5f);
  p = fmaf(x, p, 1.f);
  return x * p;
}

// The sums c of a range with maxima ms, mt and statistics sdT = Σe^((s-ms)/T),
// tdT = Σe^((t-mt)/T), re-expressed relative to maxima Ms >= ms, Mt >= mt.
// With ft = e^((mt - Mt)/T), fs = e^((ms - Ms)/T), D = ((mt - Mt) - (ms - Ms))·
// log2(e):
//   x -> ft·(x + D·tdT)
//   y -> ft·y + (fs - ft)·sdT, with fs - ft = ft·(2^(-D/T) - 1) from the
//        series when |D/T| < 1/4, so nearly equal shifts (rows that differ
//        by little more than a constant) lose nothing; beyond, the two
//        factors' difference (the rows then differ well beyond rounding).
// A range without columns (a maximum of -inf) contributes nothing.
__device__ __forceinline__ float2 kl_rebase(float2 c, float ms, float mt, float sdT, float tdT,
                                            float Ms, float Mt, float inv_t) {
  constexpr float kLog2eK = 1.4426950408889634f;
  if (mt == -INFINITY || ms == -INFINITY) return make_float2(0.f, 0.f);
  const float it2 = inv_t * kLog2eK;
  const float ft = __builtin_amdgcn_exp2f((mt - Mt) * it2);
  const float d = ((mt - Mt) - (ms - Ms)) * kLog2eK;
  const float q = d * inv_t;
  const float fd = fabsf(q) < 0.25f ? ft * exp2m1_small(q)
                                    : __builtin_amdgcn_exp2f((ms - Ms) * it2) - ft;
  return make_float2(ft * fmaf(d, tdT, c.x), fmaf(fd, sdT, ft * c.y));
}

}  // namespace orda
