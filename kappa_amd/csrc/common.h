// Shared device helpers for the gfx950 MoE kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "host.h"
#include "kmoe.h"

namespace kmoe {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef int int32x4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// Round-to-nearest-even float -> bf16 bits (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  __bf16 h = (__bf16)f;
  return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

// Activation element access, templated on storage type (uint16_t = bf16 bits, float = f32).
template <typename A>
struct Act;
template <>
struct Act<float> {
  static constexpr bool kBf16 = false;
  __device__ __forceinline__ static float load(const float* p, int64_t i) { return p[i]; }
  __device__ __forceinline__ static float round(float v) { return v; }
  __device__ __forceinline__ static void store(float* p, int64_t i, float v) { p[i] = v; }
};
template <>
struct Act<uint16_t> {
  static constexpr bool kBf16 = true;
  __device__ __forceinline__ static float load(const uint16_t* p, int64_t i) { return bf16_bits_to_f32(p[i]); }
  __device__ __forceinline__ static float round(float v) { return round_bf16(v); }
  __device__ __forceinline__ static void store(uint16_t* p, int64_t i, float v) { p[i] = f32_to_bf16_bits(v); }
};

// sigmoid(g) = 1 / (1 + exp(-g)) in f32 (jax.nn.sigmoid) with the hardware exp2
// and reciprocal: within a few f32 ulps of the correctly rounded value, far
// below the bf16 rounding that follows (kChainAct) or the output tolerance
// (kChainF32); exp overflow gives 0 and underflow 1, as the exact form does.
__device__ __forceinline__ float sigmoid_f32(float g) { return __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }

// jax.nn.silu(g) * u (kappa/qwen3/ffn_moe.py:101, 151, 209) with silu(g) = g * sigmoid(g):
// each product rounded to the activation dtype when R rounds (bf16), else f32.
template <bool BF16>
__device__ __forceinline__ float swiglu(float g, float u) {
  if (BF16) {
    const float sg = round_bf16(__fmul_rn(g, round_bf16(sigmoid_f32(g))));
    return round_bf16(__fmul_rn(sg, u));
  }
  return __fmul_rn(__fmul_rn(g, sigmoid_f32(g)), u);
}

// h = hi + lo with hi = bf16(h), lo = bf16(h - hi) (h - hi is exact in f32)
__device__ __forceinline__ void split_bf16(float h, uint16_t& hi, uint16_t& lo) {
  hi = f32_to_bf16_bits(h);
  lo = f32_to_bf16_bits(__fsub_rn(h, bf16_bits_to_f32(hi)));
}

__device__ __forceinline__ int ceil_div(int a, int b) { return (a + b - 1) / b; }

}  // namespace kmoe
