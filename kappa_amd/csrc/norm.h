// rms_norm's reduction (kappa/qwen3/norms.py:10-16), shared by the stand-alone
// norm kernel and the split router that normalises its own input.
#pragma once

#include "common.h"

namespace kmoe {

constexpr int kNormBatch = 32;  // row elements per lane in flight (a 2048-wide row in one batch)

// LDS floats one wave needs to stage a row of D elements: [slice][65].
__host__ __device__ inline int norm_row_floats(int D) { return ((D + kRouterSlice - 1) / kRouterSlice) * (kRouterSlice + 1); }

// One wave: stage the row src[0..D) in LDS as f32 row[slice][65] (the pad puts
// the 64 lanes' slice chains in distinct banks) and return
//   r = 1 / sqrt(S / D + eps),  S = sum_d src[d]^2
// in the canonical order: each square rounded to float, lane s adds the
// squares of slice s (64 indices) in a sequential chain from +0.0f, and the
// slice sums are combined by the zero-padded pairwise tree p[l] += p[l + st]
// (the router's order); IEEE division and square root. The row stays in LDS
// for the caller; every lane of the wave must call it, and gets r.
template <typename A>
__device__ __forceinline__ float wave_rms_factor(const A* __restrict__ src, int D, float eps, float* row) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int NS = (D + kRouterSlice - 1) / kRouterSlice;
  int P = 1;
  while (P < NS) P <<= 1;
  // loads in batches of kNormBatch per lane, all issued before their LDS
  // writes (addresses clamped into the row, so no load sits behind a branch)
  for (int base = 0; base < D; base += 64 * kNormBatch) {
    float v[kNormBatch];
#pragma unroll
    for (int j = 0; j < kNormBatch; ++j) v[j] = Act<A>::load(src, min(base + 64 * j + lane, D - 1));
#pragma unroll
    for (int j = 0; j < kNormBatch; ++j) {
      const int d = base + 64 * j + lane;
      if (d < D) row[(d >> 6) * (kRouterSlice + 1) + (d & 63)] = v[j];
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float acc = 0.0f;
  if (lane < NS) {
    const float* sl = row + lane * (kRouterSlice + 1);
    const int n = min(kRouterSlice, D - lane * kRouterSlice);
    for (int i = 0; i < n; ++i) {
      const float sq = sl[i] * sl[i];
      acc = acc + sq;
    }
  }
  for (int st = 1; st < P; st <<= 1) {
    const float o = __shfl_down(acc, st, 64);
    if ((lane & (2 * st - 1)) == 0) acc = acc + o;
  }
  const float total = __shfl(acc, 0, 64);
  const float var = total / (float)D;
  return 1.0f / sqrtf(var + eps);
}

// One normalised element: round_act((x * r) * scale), each product rounded.
template <typename A>
__device__ __forceinline__ float rms_apply(float x, float r, float s) {
#pragma clang fp contract(off)
  const float n = x * r;
  return Act<A>::round(n * s);
}

}  // namespace kmoe
