// The steps on either side of the MoE block in a Qwen3 MoE layer
// (kappa/qwen3/block.py:196-207): the pre-FFN RMSNorm that produces the
// block's input, and (in the combine kernels of expert.hip) the residual add
// of its output.
//
// rms_norm (kappa/qwen3/norms.py:10-16) in a canonical order shared with the
// oracle: the squares f32(h)*f32(h), each rounded to float, are summed per
// 64-wide slice in a sequential chain from +0.0f, and the slice sums are
// combined by the same zero-padded pairwise tree as the router logits;
// var = S / D, r = 1 / sqrt(var + eps) with IEEE division and square root, and
// h2 = round_act((f32(h) * r) * f32(scale)).
#include "common.h"
#include "launch.h"
#include "norm.h"

namespace kmoe {

constexpr int kNormWaves = 4;  // tokens per block, one wave each

// One wave per token: wave_rms_factor stages the row in LDS and reduces it,
// then the wave writes round_act((x * r) * scale).
template <typename A, typename S>
__global__ __launch_bounds__(256) void k_rms_norm(int T, int D, float eps, const A* __restrict__ h,
                                                   const S* __restrict__ scale, A* __restrict__ out) {
  extern __shared__ float rows[];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int t = blockIdx.x * kNormWaves + w;
  if (t >= T) return;  // per wave: this kernel has no block-wide barrier
  float* row = rows + (size_t)w * norm_row_floats(D);
  // the first batch of the scale is loaded with the row
  float sc[kNormBatch];
#pragma unroll
  for (int j = 0; j < kNormBatch; ++j) sc[j] = Act<S>::load(scale, min(64 * j + lane, D - 1));
  const float r = wave_rms_factor(h + (int64_t)t * D, D, eps, row);
  A* dst = out + (int64_t)t * D;
  for (int base = 0; base < D; base += 64 * kNormBatch) {
    if (base) {
#pragma unroll
      for (int j = 0; j < kNormBatch; ++j) sc[j] = Act<S>::load(scale, min(base + 64 * j + lane, D - 1));
    }
#pragma unroll
    for (int j = 0; j < kNormBatch; ++j) {
      const int d = base + 64 * j + lane;
      if (d < D) Act<A>::store(dst, d, rms_apply<A>(row[(d >> 6) * (kRouterSlice + 1) + (d & 63)], r, sc[j]));
    }
  }
}

}  // namespace kmoe

namespace kmoe_host {

using namespace kmoe;

size_t rms_norm_lds_bytes(int64_t D) { return (size_t)kNormWaves * norm_row_floats((int)D) * sizeof(float); }

hipError_t launch_rms_norm(const kmoe_desc& d, const void* h, const void* scale, kmoe_dtype scale_dtype, float eps,
                           void* out, hipStream_t st) {
  const int T = (int)d.tokens, D = (int)d.hidden;
  if (T == 0) return hipSuccess;
  const dim3 grid((T + kNormWaves - 1) / kNormWaves);
  const size_t lds = rms_norm_lds_bytes(D);
  const bool act_bf16 = d.act_dtype == KMOE_DTYPE_BF16, s_bf16 = scale_dtype == KMOE_DTYPE_BF16;
  if (act_bf16 && s_bf16)
    hipLaunchKernelGGL((k_rms_norm<uint16_t, uint16_t>), grid, dim3(64 * kNormWaves), lds, st, T, D, eps,
                       reinterpret_cast<const uint16_t*>(h), reinterpret_cast<const uint16_t*>(scale),
                       reinterpret_cast<uint16_t*>(out));
  else if (act_bf16)
    hipLaunchKernelGGL((k_rms_norm<uint16_t, float>), grid, dim3(64 * kNormWaves), lds, st, T, D, eps,
                       reinterpret_cast<const uint16_t*>(h), reinterpret_cast<const float*>(scale),
                       reinterpret_cast<uint16_t*>(out));
  else if (s_bf16)
    hipLaunchKernelGGL((k_rms_norm<float, uint16_t>), grid, dim3(64 * kNormWaves), lds, st, T, D, eps,
                       reinterpret_cast<const float*>(h), reinterpret_cast<const uint16_t*>(scale),
                       reinterpret_cast<float*>(out));
  else
    hipLaunchKernelGGL((k_rms_norm<float, float>), grid, dim3(64 * kNormWaves), lds, st, T, D, eps,
                       reinterpret_cast<const float*>(h), reinterpret_cast<const float*>(scale),
                       reinterpret_cast<float*>(out));
  return hipGetLastError();
}

}  // namespace kmoe_host
