// Router logits, top-k with renormalised weights, and the stable dispatch sort.
//
// Reference: _route (kappa/qwen3/ffn_moe.py:38-56) and the ordering part of
// _moe_ragged (kappa/qwen3/ffn_moe.py:189-200, 212).
#include <float.h>

#include "common.h"
#include "launch.h"

namespace kmoe {

// ---------------------------------------------------------------------------
// Router logits in the canonical order.
//
// logits[t,e] = tree_s( fmaf-chain_{d in slice s}( x[t,d] * r[d,e] ) ),
// slices of 64 hidden indices; the tree is p[i] += p[i+st] for st = 1,2,4,..
// over the slices zero-padded to GW = next power of two.
//
// A group of GW lanes owns one slice each and TB tokens x 8 experts of output;
// the slice tree is a shuffle-down reduction inside the group. x for the TB
// tokens is staged in LDS as f32 with each 64-slice padded to 65 floats so the
// lanes of a group (one slice each) hit distinct banks.
// ---------------------------------------------------------------------------
template <int RT>
struct RouterRow;

// f32 router
template <>
struct RouterRow<0> {
  __device__ __forceinline__ static void load8(const void* rw, int64_t off, float* r, const float*) {
    const float* p = reinterpret_cast<const float*>(rw) + off;
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = p[j];
  }
  __device__ __forceinline__ static float load1(const void* rw, int64_t off, float) {
    return reinterpret_cast<const float*>(rw)[off];
  }
};
// bf16 router
template <>
struct RouterRow<1> {
  __device__ __forceinline__ static void load8(const void* rw, int64_t off, float* r, const float*) {
    const uint4 v = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(rw) + off);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      r[2 * j] = __uint_as_float(w[j] << 16);
      r[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
    }
  }
  __device__ __forceinline__ static float load1(const void* rw, int64_t off, float) {
    return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(rw)[off]);
  }
};
// int8 router: f32(q) * f32(scale[e])  (to_compute_dtype(router_w, f32))
template <>
struct RouterRow<2> {
  __device__ __forceinline__ static void load8(const void* rw, int64_t off, float* r, const float* s) {
    const uint2 v = *reinterpret_cast<const uint2*>(reinterpret_cast<const int8_t*>(rw) + off);
    const uint32_t w[2] = {v.x, v.y};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      int8_t q = (int8_t)((w[j >> 2] >> (8 * (j & 3))) & 0xffu);
      r[j] = (float)q * s[j];
    }
  }
  __device__ __forceinline__ static float load1(const void* rw, int64_t off, float s) {
    return (float)reinterpret_cast<const int8_t*>(rw)[off] * s;
  }
};

__device__ __forceinline__ float load_scale(const void* scale, int scale_bf16, int64_t i) {
  return scale_bf16 ? bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(scale)[i])
                    : reinterpret_cast<const float*>(scale)[i];
}

template <typename A, int RT, int TB, bool VEC>
__global__ __launch_bounds__(256) void k_router_logits(int T, int D, int E, const A* __restrict__ x,
                                                        const void* __restrict__ rw, const void* __restrict__ rscale,
                                                        int scale_bf16, int scale_per_channel,
                                                        float* __restrict__ logits, int gw_log2) {
  extern __shared__ float xs[];  // [TB][S][65]
  const int S = (D + kRouterSlice - 1) / kRouterSlice;
  const int GW = 1 << gw_log2;
  const int t0 = blockIdx.x * TB;
  const int xstride = S * 65;
  for (int i = threadIdx.x; i < TB * D; i += blockDim.x) {
    const int tt = i / D, d = i - tt * D;
    const float v = (t0 + tt < T) ? Act<A>::load(x, (int64_t)(t0 + tt) * D + d) : 0.0f;
    xs[tt * xstride + (d >> 6) * 65 + (d & 63)] = v;
  }
  __syncthreads();

  const int ls = threadIdx.x & (GW - 1);
  const int g = threadIdx.x >> gw_log2;
  const int NG = (int)blockDim.x >> gw_log2;
  const int e0 = (blockIdx.y * NG + g) * 8;

  float sc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    sc[j] = 0.0f;
    if (RT == 2 && e0 + j < E) sc[j] = load_scale(rscale, scale_bf16, scale_per_channel ? e0 + j : 0);
  }

  float acc[TB][8];
#pragma unroll
  for (int tt = 0; tt < TB; ++tt)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[tt][j] = 0.0f;

  if (ls < S && e0 < E) {
    const int d0 = ls * kRouterSlice;
    const int d1 = min(D, d0 + kRouterSlice);
    const float* xl = xs + ls * 65;
    for (int d = d0; d < d1; ++d) {
      float r[8];
      if (VEC) {
        RouterRow<RT>::load8(rw, (int64_t)d * E + e0, r, sc);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = (e0 + j < E) ? RouterRow<RT>::load1(rw, (int64_t)d * E + e0 + j, sc[j]) : 0.0f;
      }
#pragma unroll
      for (int tt = 0; tt < TB; ++tt) {
        const float xv = xl[tt * xstride + (d - d0)];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[tt][j] = __builtin_fmaf(xv, r[j], acc[tt][j]);
      }
    }
  }
  // pairwise tree over the slices held by the GW lanes of this group
  for (int st = 1; st < GW; st <<= 1) {
#pragma unroll
    for (int tt = 0; tt < TB; ++tt)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[tt][j] = acc[tt][j] + __shfl_down(acc[tt][j], st, GW);
  }
  if (ls == 0 && e0 < E) {
#pragma unroll
    for (int tt = 0; tt < TB; ++tt) {
      if (t0 + tt >= T) break;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (e0 + j < E) logits[(int64_t)(t0 + tt) * E + e0 + j] = acc[tt][j];
    }
  }
}

// ---------------------------------------------------------------------------
// Top-k (value descending, ties to the lower expert index) and softmax over the
// selected logits, rounded to the activation dtype; per 64-token block expert
// histogram for the dispatch. One wave per token; 16 waves per block.
// ---------------------------------------------------------------------------
template <bool BF16W>
__global__ __launch_bounds__(1024) void k_topk(int T, int E, int K, const float* __restrict__ logits,
                                                int32_t* __restrict__ topk_idx, float* __restrict__ topk_w,
                                                int32_t* __restrict__ hist) {
  __shared__ int h[kMaxExperts];
  __shared__ float sv[16][kMaxTopK];
  __shared__ int si[16][kMaxTopK];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int tb0 = blockIdx.x * kDispatchBlock;
  for (int e = threadIdx.x; e < E; e += blockDim.x) h[e] = 0;
  __syncthreads();
  const int nper = (E + 63) / 64;
  for (int tl = wv; tl < kDispatchBlock; tl += 16) {
    const int t = tb0 + tl;
    if (t >= T) break;
    const float* lt = logits + (int64_t)t * E;
    float v[kMaxExperts / 64];
    uint32_t taken = 0;
#pragma unroll
    for (int i = 0; i < kMaxExperts / 64; ++i) {
      const int e = lane + 64 * i;
      const float lv = (i < nper && e < E) ? lt[e] : -INFINITY;
      v[i] = (lv != lv) ? -INFINITY : lv;  // NaN ranks lowest, so a winner always exists
    }
    for (int j = 0; j < K; ++j) {
      float bv = -INFINITY;
      int bi = 0x7fffffff;
#pragma unroll
      for (int i = 0; i < kMaxExperts / 64; ++i) {
        const int e = lane + 64 * i;
        if (i < nper && e < E && !((taken >> i) & 1u)) {
          if (v[i] > bv || (v[i] == bv && e < bi)) {
            bv = v[i];
            bi = e;
          }
        }
      }
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        if (ov > bv || (ov == bv && oi < bi)) {
          bv = ov;
          bi = oi;
        }
      }
      if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
      if (lane == 0) {
        sv[wv][j] = bv;
        si[wv][j] = bi;
      }
    }
    __builtin_amdgcn_wave_barrier();
    if (lane == 0) {
      const float m = sv[wv][0];
      float s = 0.0f;
      for (int j = 0; j < K; ++j) s = s + expf(sv[wv][j] - m);
      for (int j = 0; j < K; ++j) {
        const float p = expf(sv[wv][j] - m) / s;
        topk_w[(int64_t)t * K + j] = BF16W ? round_bf16(p) : p;
        topk_idx[(int64_t)t * K + j] = si[wv][j];
        atomicAdd(&h[si[wv][j]], 1);
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x) hist[(int64_t)blockIdx.x * E + e] = h[e];
}

// ---------------------------------------------------------------------------
// Dispatch: stable counting sort of the row-major (t, j) assignments by
// expert. Block b owns tokens [64b, 64b+64); its write cursor for expert e is
// offsets[e] + sum_{b' < b} hist[b'][e]; within the block tokens are taken in
// increasing order, which keeps the sort stable (jnp.argsort(stable=True)).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_dispatch(int T, int E, int K, int nblk, const int32_t* __restrict__ topk_idx,
                                                   const int32_t* __restrict__ hist, int32_t* __restrict__ group_sizes,
                                                   int32_t* __restrict__ offsets, int32_t* __restrict__ active,
                                                   int32_t* __restrict__ sorted_token,
                                                   int32_t* __restrict__ sorted_expert, int32_t* __restrict__ inv) {
  __shared__ int tot[kMaxExperts];
  __shared__ int cur[kMaxExperts];
  const int b = blockIdx.x;
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    int before = 0, after = 0;
    for (int bb = 0; bb < b; ++bb) before += hist[(int64_t)bb * E + e];
    for (int bb = b; bb < nblk; ++bb) after += hist[(int64_t)bb * E + e];
    tot[e] = before + after;
    cur[e] = before;
  }
  __syncthreads();
  int pre_reg[kMaxExperts / 256];
  int act_reg[kMaxExperts / 256];
#pragma unroll
  for (int i = 0; i < kMaxExperts / 256; ++i) {
    const int e = threadIdx.x + 256 * i;
    int s = 0, a = 0;
    if (e < E)
      for (int ee = 0; ee < e; ++ee) {
        s += tot[ee];
        a += tot[ee] > 0;
      }
    pre_reg[i] = s;
    act_reg[i] = a;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kMaxExperts / 256; ++i) {
    const int e = threadIdx.x + 256 * i;
    if (e < E) {
      if (b == 0) {
        group_sizes[e] = tot[e];
        offsets[e] = pre_reg[i];
        if (tot[e] > 0) active[act_reg[i]] = e;
        if (e == E - 1) {
          offsets[E] = pre_reg[i] + tot[e];
          active[E] = act_reg[i] + (tot[e] > 0);
        }
      }
      cur[e] += pre_reg[i];
    }
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const int t1 = min(T, (b + 1) * kDispatchBlock);
    for (int t = b * kDispatchBlock; t < t1; ++t) {
      if (lane < K) {
        const int m = t * K + lane;
        const int e = topk_idx[m];
        // indices outside [0, E) or a histogram that disagrees with them are
        // caller errors; they are skipped rather than written out of bounds
        if ((unsigned)e < (unsigned)E) {
          const int p = cur[e];
          cur[e] = p + 1;
          if ((unsigned)p < (unsigned)(T * K)) {
            sorted_token[p] = t;
            sorted_expert[p] = e;
            inv[m] = p;
          }
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
  }
}

}  // namespace kmoe

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
namespace kmoe_host {

using namespace kmoe;

template <typename A, int RT, int TB>
static hipError_t launch_router_tb(const kmoe_desc& d, const void* x, const kmoe_weight& r, float* logits,
                                   hipStream_t st) {
  const int T = (int)d.tokens, D = (int)d.hidden, E = (int)d.num_experts;
  const int S = (D + kRouterSlice - 1) / kRouterSlice;
  int gw_log2 = 0;
  while ((1 << gw_log2) < S) ++gw_log2;
  const int NG = 256 >> gw_log2;
  const int EB = NG * 8;
  dim3 grid((T + TB - 1) / TB, (E + EB - 1) / EB);
  const size_t lds = sizeof(float) * (size_t)TB * S * 65;
  const int scale_bf16 = (r.dtype == KMOE_DTYPE_I8 && r.scale_dtype == KMOE_DTYPE_BF16) ? 1 : 0;
  const int per_channel = (r.dtype == KMOE_DTYPE_I8 && r.scale_kind == KMOE_SCALE_CHANNEL) ? 1 : 0;
  const bool vec = (E % 8) == 0;
  if (vec)
    hipLaunchKernelGGL((k_router_logits<A, RT, TB, true>), grid, dim3(256), lds, st, T, D, E,
                       reinterpret_cast<const A*>(x), r.values, r.scale, scale_bf16, per_channel, logits, gw_log2);
  else
    hipLaunchKernelGGL((k_router_logits<A, RT, TB, false>), grid, dim3(256), lds, st, T, D, E,
                       reinterpret_cast<const A*>(x), r.values, r.scale, scale_bf16, per_channel, logits, gw_log2);
  return hipGetLastError();
}

template <typename A, int RT>
static hipError_t launch_router_rt(const kmoe_desc& d, const void* x, const kmoe_weight& r, float* logits,
                                   hipStream_t st) {
  const int S = (int)((d.hidden + kRouterSlice - 1) / kRouterSlice);
  // tokens per block: as many as the 64 KB x stage allows, fewer for small T
  int tb = 8;
  while (tb > 1 && (size_t)tb * S * 65 * sizeof(float) > 65536) tb >>= 1;
  while (tb > 1 && d.tokens < (int64_t)tb * 16) tb >>= 1;
  switch (tb) {
    case 8:
      return launch_router_tb<A, RT, 8>(d, x, r, logits, st);
    case 4:
      return launch_router_tb<A, RT, 4>(d, x, r, logits, st);
    case 2:
      return launch_router_tb<A, RT, 2>(d, x, r, logits, st);
    default:
      return launch_router_tb<A, RT, 1>(d, x, r, logits, st);
  }
}

hipError_t launch_route(const kmoe_desc& d, const void* x, const kmoe_weight& r, float* logits, int32_t* topk_idx,
                        float* topk_w, int32_t* hist, hipStream_t st) {
  hipError_t err;
  const bool bf16 = d.act_dtype == KMOE_DTYPE_BF16;
  const int rt = r.dtype == KMOE_DTYPE_F32 ? 0 : (r.dtype == KMOE_DTYPE_BF16 ? 1 : 2);
  if (bf16) {
    err = rt == 0 ? launch_router_rt<uint16_t, 0>(d, x, r, logits, st)
                  : (rt == 1 ? launch_router_rt<uint16_t, 1>(d, x, r, logits, st)
                             : launch_router_rt<uint16_t, 2>(d, x, r, logits, st));
  } else {
    err = rt == 0 ? launch_router_rt<float, 0>(d, x, r, logits, st)
                  : (rt == 1 ? launch_router_rt<float, 1>(d, x, r, logits, st)
                             : launch_router_rt<float, 2>(d, x, r, logits, st));
  }
  if (err != hipSuccess) return err;
  const int T = (int)d.tokens, E = (int)d.num_experts, K = (int)d.top_k;
  const int nblk = (T + kDispatchBlock - 1) / kDispatchBlock;
  if (bf16)
    hipLaunchKernelGGL((k_topk<true>), dim3(nblk), dim3(1024), 0, st, T, E, K, logits, topk_idx, topk_w, hist);
  else
    hipLaunchKernelGGL((k_topk<false>), dim3(nblk), dim3(1024), 0, st, T, E, K, logits, topk_idx, topk_w, hist);
  return hipGetLastError();
}

hipError_t launch_dispatch(const kmoe_desc& d, const int32_t* topk_idx, const int32_t* hist, int32_t* group_sizes,
                           int32_t* offsets, int32_t* active, int32_t* sorted_token, int32_t* sorted_expert,
                           int32_t* inv, hipStream_t st) {
  const int T = (int)d.tokens, E = (int)d.num_experts, K = (int)d.top_k;
  const int nblk = (T + kDispatchBlock - 1) / kDispatchBlock;
  hipLaunchKernelGGL(k_dispatch, dim3(nblk), dim3(256), 0, st, T, E, K, nblk, topk_idx, hist, group_sizes, offsets,
                     active, sorted_token, sorted_expert, inv);
  return hipGetLastError();
}

}  // namespace kmoe_host
