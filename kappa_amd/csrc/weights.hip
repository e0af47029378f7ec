// Weight-side kernels: the one-time relayout of W8 experts for the gfx950
// kernels, to_compute_dtype (kappa/qwen3/quant.py:34-38) and the per-channel
// int8 quantiser (kappa/qwen3/quant.py:41-48 with a per-channel max-abs).
#include <float.h>

#include "common.h"
#include "launch.h"

namespace kmoe {

__device__ __forceinline__ float scale_at(const void* s, int s_bf16, size_t i) {
  return s_bf16 ? bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(s)[i]) : reinterpret_cast<const float*>(s)[i];
}

// One thread per 16-byte cell of w13 [E][I/16][2][D/16][16 col][16 k]:
// cell (e, ig, which, kg, col) holds src[e][kg*16 + kk][ig*16 + col], kk = 0..15.
__global__ __launch_bounds__(256) void k_pack_w13(int64_t ncell, int D, int I, const int8_t* __restrict__ gate,
                                                  const int8_t* __restrict__ up, int8_t* __restrict__ w13) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= ncell) return;
  const int col = (int)(c & 15);
  int64_t r = c >> 4;
  const int KG = D >> 4, IG = I >> 4;
  const int kg = (int)(r % KG);
  r /= KG;
  const int which = (int)(r & 1);
  r >>= 1;
  const int ig = (int)(r % IG);
  const int64_t e = r / IG;
  const int8_t* src = (which ? up : gate) + (e * D + (int64_t)kg * 16) * I + ig * 16 + col;
  uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
  for (int kk = 0; kk < 16; ++kk) w[kk >> 2] |= (uint32_t)(uint8_t)src[(int64_t)kk * I] << (8 * (kk & 3));
  *reinterpret_cast<uint4*>(w13 + c * 16) = uint4{w[0], w[1], w[2], w[3]};
}

// w2 [E][D/16][I/16][16 col][16 k]: cell (e, dg, kg, col) holds down[e][kg*16 + kk][dg*16 + col].
__global__ __launch_bounds__(256) void k_pack_w2(int64_t ncell, int D, int I, const int8_t* __restrict__ down,
                                                 int8_t* __restrict__ w2) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= ncell) return;
  const int col = (int)(c & 15);
  int64_t r = c >> 4;
  const int KG = I >> 4, DG = D >> 4;
  const int kg = (int)(r % KG);
  r /= KG;
  const int dg = (int)(r % DG);
  const int64_t e = r / DG;
  const int8_t* src = down + (e * I + (int64_t)kg * 16) * D + dg * 16 + col;
  uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
  for (int kk = 0; kk < 16; ++kk) w[kk >> 2] |= (uint32_t)(uint8_t)src[(int64_t)kk * D] << (8 * (kk & 3));
  *reinterpret_cast<uint4*>(w2 + c * 16) = uint4{w[0], w[1], w[2], w[3]};
}

// s13 [E][I/16][2][16] and s2 [E][D]: the scales as given, in f32 (the kernels
// cast them to bf16 for the gather and fixed_capacity programs,
// kappa/qwen3/quant.py:37, and use them as they are for the ragged program's
// f32 dequantisation, kappa/qwen3/ffn_moe.py:203-205).
__global__ __launch_bounds__(256) void k_pack_scales(int E, int D, int I, const void* __restrict__ gs, int g_bf16,
                                                     int g_pc, const void* __restrict__ us, int u_bf16, int u_pc,
                                                     const void* __restrict__ ds, int d_bf16, int d_pc,
                                                     float* __restrict__ s13, float* __restrict__ s2) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t n13 = (int64_t)E * I * 2;
  if (i < n13) {
    const int col = (int)(i & 15);
    const int which = (int)((i >> 4) & 1);
    const int64_t r = i >> 5;
    const int ig = (int)(r % (I >> 4));
    const int64_t e = r / (I >> 4);
    const int64_t ch = e * I + ig * 16 + col;
    const float v = which ? scale_at(us, u_bf16, u_pc ? ch : 0) : scale_at(gs, g_bf16, g_pc ? ch : 0);
    s13[i] = v;
  } else if (i < n13 + (int64_t)E * D) {
    const int64_t j = i - n13;
    s2[j] = scale_at(ds, d_bf16, d_pc ? j : 0);
  }
}

// out[o, c] = to_compute_dtype(w)[o, c]; for int8 the scale of (o / rows_per_block, c).
template <typename O>
__global__ __launch_bounds__(256) void k_to_compute(int64_t outer, int64_t channels, int64_t rows_per_block,
                                                    const void* __restrict__ v, int wt, const void* __restrict__ s,
                                                    int s_bf16, int per_channel, O* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= outer * channels) return;
  float r;
  if (wt == 0) {
    r = Act<O>::round(reinterpret_cast<const float*>(v)[i]);
  } else if (wt == 1) {
    r = bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(v)[i]);
  } else {
    const int64_t o = i / channels, c = i - o * channels;
    const float sv = scale_at(s, s_bf16, per_channel ? (size_t)((o / rows_per_block) * channels + c) : 0);
    const float q = (float)reinterpret_cast<const int8_t*>(v)[i];
    r = Act<O>::kBf16 ? round_bf16(q * round_bf16(sv)) : q * sv;
  }
  Act<O>::store(out, i, r);
}

// Per-output-channel quantiser over [E, Kd, N]: one thread per (e, n).
template <typename W>
__global__ __launch_bounds__(256) void k_quantize_pc(int64_t E, int64_t Kd, int64_t N, const W* __restrict__ w,
                                                     int8_t* __restrict__ q, float* __restrict__ s) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t e = blockIdx.y;
  if (n >= N) return;
  const W* we = w + e * Kd * N + n;
  float amax = 0.0f;
  for (int64_t k = 0; k < Kd; ++k) amax = fmaxf(amax, fabsf(Act<W>::load(we, k * N)));
  float sc = amax / 127.0f;
  sc = sc > FLT_MIN ? sc : FLT_MIN;
  s[e * N + n] = sc;
  int8_t* qe = q + e * Kd * N + n;
  for (int64_t k = 0; k < Kd; ++k) {
    float r = rintf(Act<W>::load(we, k * N) / sc);
    r = fminf(fmaxf(r, -128.0f), 127.0f);
    qe[k * N] = (int8_t)r;
  }
}

}  // namespace kmoe

namespace kmoe_host {

using namespace kmoe;

hipError_t launch_prepack(const kmoe_desc& d, const kmoe_weight& gate, const kmoe_weight& up, const kmoe_weight& down,
                          const kmoe_packed_experts& p, hipStream_t st) {
  const int E = (int)d.num_experts, D = (int)d.hidden, I = (int)d.intermediate;
  const int64_t nc13 = (int64_t)E * (I / 16) * 2 * (D / 16) * 16;
  const int64_t nc2 = (int64_t)E * (D / 16) * (I / 16) * 16;
  hipLaunchKernelGGL(k_pack_w13, dim3((unsigned)((nc13 + 255) / 256)), dim3(256), 0, st, nc13, D, I,
                     reinterpret_cast<const int8_t*>(gate.values), reinterpret_cast<const int8_t*>(up.values),
                     reinterpret_cast<int8_t*>(p.w13));
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(k_pack_w2, dim3((unsigned)((nc2 + 255) / 256)), dim3(256), 0, st, nc2, D, I,
                     reinterpret_cast<const int8_t*>(down.values), reinterpret_cast<int8_t*>(p.w2));
  err = hipGetLastError();
  if (err != hipSuccess) return err;
  const int64_t ns = (int64_t)E * I * 2 + (int64_t)E * D;
  auto bf = [](const kmoe_weight& w) { return w.scale_dtype == KMOE_DTYPE_BF16 ? 1 : 0; };
  auto pc = [](const kmoe_weight& w) { return w.scale_kind == KMOE_SCALE_CHANNEL ? 1 : 0; };
  hipLaunchKernelGGL(k_pack_scales, dim3((unsigned)((ns + 255) / 256)), dim3(256), 0, st, E, D, I, gate.scale,
                     bf(gate), pc(gate), up.scale, bf(up), pc(up), down.scale, bf(down), pc(down),
                     reinterpret_cast<float*>(p.s13), reinterpret_cast<float*>(p.s2));
  return hipGetLastError();
}

hipError_t launch_to_compute_dtype(const kmoe_weight& w, int64_t outer, int64_t channels, int64_t rows_per_block,
                                   kmoe_dtype out_dtype, void* out, hipStream_t st) {
  const int64_t n = outer * channels;
  const unsigned blocks = (unsigned)((n + 255) / 256);
  const int wt = w.dtype == KMOE_DTYPE_F32 ? 0 : (w.dtype == KMOE_DTYPE_BF16 ? 1 : 2);
  const int s_bf16 = (wt == 2 && w.scale_dtype == KMOE_DTYPE_BF16) ? 1 : 0;
  const int pc = (wt == 2 && w.scale_kind == KMOE_SCALE_CHANNEL) ? 1 : 0;
  if (out_dtype == KMOE_DTYPE_BF16)
    hipLaunchKernelGGL((k_to_compute<uint16_t>), dim3(blocks), dim3(256), 0, st, outer, channels, rows_per_block,
                       w.values, wt, w.scale, s_bf16, pc, reinterpret_cast<uint16_t*>(out));
  else
    hipLaunchKernelGGL((k_to_compute<float>), dim3(blocks), dim3(256), 0, st, outer, channels, rows_per_block,
                       w.values, wt, w.scale, s_bf16, pc, reinterpret_cast<float*>(out));
  return hipGetLastError();
}

hipError_t launch_quantize_per_channel(int64_t E, int64_t Kd, int64_t N, const void* w, kmoe_dtype w_dtype, int8_t* q,
                                       float* s, hipStream_t st) {
  dim3 grid((unsigned)((N + 255) / 256), (unsigned)E);
  if (w_dtype == KMOE_DTYPE_BF16)
    hipLaunchKernelGGL((k_quantize_pc<uint16_t>), grid, dim3(256), 0, st, E, Kd, N,
                       reinterpret_cast<const uint16_t*>(w), q, s);
  else
    hipLaunchKernelGGL((k_quantize_pc<float>), grid, dim3(256), 0, st, E, Kd, N, reinterpret_cast<const float*>(w), q,
                       s);
  return hipGetLastError();
}

}  // namespace kmoe_host
