// Shared device helpers for the gfx950 MoE kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kmoe.h"

namespace kmoe {

// Slice length of the canonical router summation order: each slice of 64
// consecutive hidden indices is a sequential fmaf chain from +0.0f, and the
// slice partials are combined by a pairwise tree.
constexpr int kRouterSlice = 64;
// Tokens per dispatch block (per-block expert histograms).
constexpr int kDispatchBlock = 64;
// Largest expert count / top-k the routing kernels hold in registers and LDS.
constexpr int kMaxExperts = 1024;
constexpr int kMaxTopK = 64;
constexpr int kMaxRouterSlices = 64;  // D <= 4096
// Decode kernels keep up to this many 16-row blocks of one expert in registers.
constexpr int kDecodeMaxRowBlocks = 4;  // T <= 64 tokens
constexpr int kRowsPathMaxTokens = 128;  // above the decode sizes, the row-group kernels up to this T
constexpr int kDownCombineMaxRows = 8;          // assignments per block of the fused decode down + combine
constexpr int kDownCombineMaxAssignments = 32;  // T * K it takes

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
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

// Rounding chain of the expert products (which array program runs):
//   kChainAct: _moe_gather_einsum / _moe_fixed_capacity (kappa/qwen3/ffn_moe.py:99-102,
//     146-152): weights bf16(q * bf16(s)), g, u, every step of silu(g) * u and y
//     rounded to the activation dtype;
//   kChainF32: _moe_ragged (:202-213): weights q * s in f32 (the scale applied to the
//     f32 sum, a per-output-channel factor), g, u, h and the down sum in f32, only y
//     rounded. With bf16 activations h is stored as two bf16 planes per row, hi =
//     bf16(h) and lo = bf16(h - hi) ([M][2I]), which the MFMA down products take as
//     two operands (hi + lo carries h to ~2^-17 relative).
constexpr int kChainAct = 0;
constexpr int kChainF32 = 1;

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

// Host-side helpers shared by the launch wrappers.
namespace kmoe_host {

// Rows an expert keeps: the fixed_capacity slot limit, or no limit.
inline int capacity_of(const kmoe_desc& d) {
  return d.expert_capacity > 0 && d.expert_capacity < 0x7fffffff ? (int)d.expert_capacity : 0x7fffffff;
}

inline size_t dtype_size(kmoe_dtype t) {
  switch (t) {
    case KMOE_DTYPE_F32:
      return 4;
    case KMOE_DTYPE_BF16:
      return 2;
    case KMOE_DTYPE_I8:
      return 1;
  }
  return 0;
}

}  // namespace kmoe_host
