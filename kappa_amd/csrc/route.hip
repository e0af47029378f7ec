// Router logits, top-k with renormalised weights, and the stable dispatch sort.
//
// Reference: _route (kappa/qwen3/ffn_moe.py:38-56) and the ordering part of
// _moe_ragged (kappa/qwen3/ffn_moe.py:189-200, 212).
#include <float.h>

#include <algorithm>
#include <cmath>

#include "common.h"
#include "launch.h"
#include "norm.h"
#include "route_dev.h"

namespace kmoe {

// ---------------------------------------------------------------------------
// Router weight rows. A lane owns EPL consecutive experts of one hidden row
// and loads them with 16-byte loads, or one 8- or 4-byte load when the EPL
// experts take 8 or 4 bytes; LPR = E / EPL lanes cover a row contiguously.
// ---------------------------------------------------------------------------
template <int RT, int EPL>
struct RouterRow {
  static constexpr int kBytes = EPL * (RT == 0 ? 4 : (RT == 1 ? 2 : 1));
  static constexpr int kWords = kBytes / 4;
  struct Raw {
    uint32_t w[kWords];
  };
  __device__ __forceinline__ static void load(const void* rw, int64_t elem, Raw& r) {
    load_at(reinterpret_cast<const char*>(rw) + elem * (kBytes / EPL), 0, r);
  }
  // row pointer (uniform across the wave) plus a per-lane byte offset
  __device__ __forceinline__ static void load_at(const char* row, int off, Raw& r) {
    const char* p = row + off;
    if constexpr (kWords % 4 == 0) {
#pragma unroll
      for (int q = 0; q < kWords / 4; ++q) {
        const uint4 v = reinterpret_cast<const uint4*>(p)[q];
        r.w[4 * q] = v.x, r.w[4 * q + 1] = v.y, r.w[4 * q + 2] = v.z, r.w[4 * q + 3] = v.w;
      }
    } else if constexpr (kWords == 2) {
      const uint2 v = *reinterpret_cast<const uint2*>(p);
      r.w[0] = v.x, r.w[1] = v.y;
    } else {
      static_assert(kWords == 1, "router rows of 4, 8 or 16k bytes per lane");
      r.w[0] = *reinterpret_cast<const uint32_t*>(p);
    }
  }
  // to_compute_dtype(router_w, f32) (kappa/qwen3/quant.py:34-38): int8 is f32(q) * f32(scale)
  __device__ __forceinline__ static void convert(const Raw& r, const float* sc, float* out) {
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      if constexpr (RT == 0) {
        out[i] = __uint_as_float(r.w[i]);
      } else if constexpr (RT == 1) {
        const uint32_t v = r.w[i >> 1];
        out[i] = __uint_as_float((i & 1) ? (v & 0xffff0000u) : (v << 16));
      } else {
        const int8_t q = (int8_t)((r.w[i >> 2] >> (8 * (i & 3))) & 0xffu);
        out[i] = (float)q * sc[i];
      }
    }
  }
  __device__ __forceinline__ static float load1(const void* rw, int64_t elem, float sc) {
    if constexpr (RT == 0) return reinterpret_cast<const float*>(rw)[elem];
    if constexpr (RT == 1) return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(rw)[elem]);
    return (float)reinterpret_cast<const int8_t*>(rw)[elem] * sc;
  }
};

__device__ __forceinline__ float load_scale(const void* scale, int scale_bf16, int64_t i) {
  return scale_bf16 ? bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(scale)[i])
                    : reinterpret_cast<const float*>(scale)[i];
}

// ---------------------------------------------------------------------------
// Fused router: logits in the canonical order, top-k, softmax.
//
// logits[t,e] = tree_s( fmaf-chain_{d in slice s}( x[t,d] * r[d,e] ) ) with
// slices of 64 hidden indices and the pairwise tree p[i] += p[i+st],
// st = 1, 2, 4, ... over the slices zero-padded to P = next power of two.
//
// Slice s is owned by lane group lg = s % SPW of wave-group s / SPW (a lane
// group is LPR lanes covering all experts; SPW groups per wave). A wave runs
// G wave-groups one after the other; the tree levels st < SPW are shuffles
// between lane groups, the levels SPW <= st < SPW*G combine the G wave-groups
// in registers, and the remaining levels combine the waves' partials through
// LDS, one element's partials per thread. x for the TB tokens of the block
// is staged in LDS as f32 [slice][64][TB] (slice pitch padded by 4 floats:
// the lane groups of a wave read different slices in distinct banks); the
// same LDS then holds the wave partials [wave][TB][E].
//
// Then one wave per token selects the top K (value descending, ties to the
// lower expert index; NaN ranks as -inf) with K wave-wide arg-max rounds, and
// lane j < K writes selection j and its softmax weight
//   w_j = expf(l_j - l_0) / sum_{i<K} expf(l_i - l_0)   (sum in i order),
// rounded to the activation dtype when out_bf16.
// ---------------------------------------------------------------------------
template <int TB, int EPL>
struct Acc {
  float v[TB][EPL];
};

template <typename A, int RT, int EPL, int TB, int G>
__global__ __launch_bounds__(1024) void k_route(int T, int D, int E, int K, int LPR, int SPW, int P,
                                                 const A* __restrict__ x, const void* __restrict__ rw,
                                                 const void* __restrict__ rscale, int scale_bf16, int scale_pc,
                                                 float* __restrict__ logits, int32_t* __restrict__ topk_idx,
                                                 float* __restrict__ topk_w, int out_bf16) {
  using Row = RouterRow<RT, EPL>;
  // rows per prefetch stage: a stage of raw rows is 32 registers for one
  // token per block (latency-bound: a 64-row slice of a bf16 router takes 8
  // dependent memory round trips), 16 registers otherwise (two stages and the
  // accumulators fit the 128 registers of a 1024-thread block)
  constexpr int RW = TB == 1 && G == 1 ? 32 : 16;
  constexpr int U0 = RW / Row::kWords < 1 ? 1 : RW / Row::kWords;
  constexpr int U = U0 < 16 / TB ? U0 : 16 / TB;
  extern __shared__ float lds[];
  const int NWB = blockDim.x >> 6;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int S = (D + kRouterSlice - 1) / kRouterSlice;
  const int XP = kRouterSlice * TB + 4;
  const int t0 = blockIdx.x * TB;
#pragma unroll
  for (int tt = 0; tt < TB; ++tt)
    for (int d = threadIdx.x; d < D; d += blockDim.x)
      lds[(d >> 6) * XP + (d & 63) * TB + tt] = (t0 + tt < T) ? Act<A>::load(x, (int64_t)(t0 + tt) * D + d) : 0.0f;
  __syncthreads();

  const int lg = lane / LPR, le = lane - lg * LPR;
  const int e0 = le * EPL;
  const bool lane_on = lg < SPW && e0 < E;
  const bool vec = (E % 8) == 0 && e0 + EPL <= E;
  float sc[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    sc[i] = 0.0f;
    if (RT == 2 && e0 + i < E) sc[i] = load_scale(rscale, scale_bf16, scale_pc ? e0 + i : 0);
  }

  Acc<TB, EPL> p0, p1;
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
    Acc<TB, EPL> c;
#pragma unroll
    for (int tt = 0; tt < TB; ++tt)
#pragma unroll
      for (int i = 0; i < EPL; ++i) c.v[tt][i] = 0.0f;
    const int s = (w * G + gi) * SPW + lg;
    if (lane_on && s < S) {
      const int d0 = s * kRouterSlice;
      const int d1 = min(D, d0 + kRouterSlice);
      const float* xs = lds + s * XP - d0 * TB;
      if (vec && d1 - d0 == kRouterSlice) {
        // two register stages used in turn (the loop body covers 2U rows, and
        // 2U divides the 64 rows of a slice), so no stage is copied
        static_assert(kRouterSlice % (2 * U) == 0, "two stages per step");
        typename Row::Raw b0[U], b1[U];
        auto rows = [&](const typename Row::Raw* raw, int db) {
#pragma unroll
          for (int u = 0; u < U; ++u) {
            float r[EPL], xv[TB];
            Row::convert(raw[u], sc, r);
            // the x stage is 16-byte aligned for TB >= 4 (slice stride
            // 64*TB + 4 floats, row stride TB floats)
            if constexpr (TB % 4 == 0) {
#pragma unroll
              for (int q = 0; q < TB / 4; ++q) {
                const float4 v4 = *reinterpret_cast<const float4*>(xs + (db + u) * TB + 4 * q);
                xv[4 * q] = v4.x, xv[4 * q + 1] = v4.y, xv[4 * q + 2] = v4.z, xv[4 * q + 3] = v4.w;
              }
            } else {
#pragma unroll
              for (int tt = 0; tt < TB; ++tt) xv[tt] = xs[(db + u) * TB + tt];
            }
#pragma unroll
            for (int tt = 0; tt < TB; ++tt)
#pragma unroll
              for (int i = 0; i < EPL; ++i) c.v[tt][i] = __builtin_fmaf(xv[tt], r[i], c.v[tt][i]);
          }
        };
#pragma unroll
        for (int u = 0; u < U; ++u) Row::load(rw, (int64_t)(d0 + u) * E + e0, b0[u]);
        for (int db = d0; db < d1; db += 2 * U) {
#pragma unroll
          for (int u = 0; u < U; ++u) Row::load(rw, (int64_t)(db + U + u) * E + e0, b1[u]);
          rows(b0, db);
          if (db + 2 * U < d1) {
#pragma unroll
            for (int u = 0; u < U; ++u) Row::load(rw, (int64_t)(db + 2 * U + u) * E + e0, b0[u]);
          }
          rows(b1, db + U);
        }
      } else {
        for (int d = d0; d < d1; ++d) {
          float r[EPL];
#pragma unroll
          for (int i = 0; i < EPL; ++i) r[i] = (e0 + i < E) ? Row::load1(rw, (int64_t)d * E + e0 + i, sc[i]) : 0.0f;
#pragma unroll
          for (int tt = 0; tt < TB; ++tt) {
            const float xv = xs[d * TB + tt];
#pragma unroll
            for (int i = 0; i < EPL; ++i) c.v[tt][i] = __builtin_fmaf(xv, r[i], c.v[tt][i]);
          }
        }
      }
    }
    // tree levels st < SPW: lane group lg += lane group lg + st
    for (int st = 1; st < SPW && st < P; st <<= 1) {
#pragma unroll
      for (int tt = 0; tt < TB; ++tt)
#pragma unroll
        for (int i = 0; i < EPL; ++i) c.v[tt][i] = c.v[tt][i] + __shfl_down(c.v[tt][i], st * LPR, 64);
    }
    // tree levels over the wave's G wave-groups (G <= 4)
#pragma unroll
    for (int tt = 0; tt < TB; ++tt)
#pragma unroll
      for (int i = 0; i < EPL; ++i) {
        if (G == 1 || gi == 0) {
          p0.v[tt][i] = c.v[tt][i];
        } else if (gi == 1) {
          p0.v[tt][i] = p0.v[tt][i] + c.v[tt][i];
        } else if (gi == 2) {
          p1.v[tt][i] = c.v[tt][i];
        } else {
          p1.v[tt][i] = p1.v[tt][i] + c.v[tt][i];
          p0.v[tt][i] = p0.v[tt][i] + p1.v[tt][i];
        }
      }
  }
  __syncthreads();  // x no longer needed: the LDS now holds the wave partials
  float* part = lds;
  const int TE = TB * E;
  if (lg == 0) {
#pragma unroll
    for (int tt = 0; tt < TB; ++tt)
#pragma unroll
      for (int i = 0; i < EPL; ++i)
        if (e0 + i < E) part[(size_t)w * TE + tt * E + e0 + i] = p0.v[tt][i];
  }
  __syncthreads();
  // the tree levels across the NWB waves (a power of two, at most 16): a
  // thread takes an element's NWB partials and applies the levels
  // p[g] += p[g + st], st = 1, 2, 4, 8, in registers
  for (int rem = threadIdx.x; rem < TE; rem += blockDim.x) {
    float v[16];
#pragma unroll
    for (int g = 0; g < 16; ++g) v[g] = g < NWB ? part[(size_t)g * TE + rem] : 0.0f;
#pragma unroll
    for (int st = 1; st < 16; st <<= 1)
#pragma unroll
      for (int g = 0; g + st < 16; g += 2 * st)
        if (g + st < NWB) v[g] = v[g] + v[g + st];
    part[rem] = v[0];
  }
  __syncthreads();

  // top-k: lane owns experts lane + 64*i, i < EPL (E <= 64 * EPL); the
  // per-wave selection scratch sits after the partials
  TopkLds* tk = reinterpret_cast<TopkLds*>(lds + (size_t)NWB * TE);
  for (int tt = w; tt < TB; tt += NWB) {
    const int t = t0 + tt;
    if (t >= T) break;
    float v[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int e = lane + 64 * i;
      const float q = e < E ? part[tt * E + e] : 0.0f;
      v[i] = (e < E && q == q) ? q : -INFINITY;
      if (logits && e < E) logits[(int64_t)t * E + e] = q;
    }
    if (E <= 128 || EPL < 4)
      wave_topk<(EPL < 2 ? EPL : 2)>(t, E, K, v, topk_idx, topk_w, out_bf16, nullptr, tk[w]);
    else if (E <= 256 || EPL < 8)
      wave_topk<(EPL < 4 ? EPL : 4)>(t, E, K, v, topk_idx, topk_w, out_bf16, nullptr, tk[w]);
    else if (E <= 512 || EPL < 16)
      wave_topk<(EPL < 8 ? EPL : 8)>(t, E, K, v, topk_idx, topk_w, out_bf16, nullptr, tk[w]);
    else
      wave_topk<EPL>(t, E, K, v, topk_idx, topk_w, out_bf16, nullptr, tk[w]);
  }
}

// ---------------------------------------------------------------------------
// Split router for small token counts (decode): the same canonical logits as
// k_route, computed by many blocks per token instead of one.
//
// k_route_slices, block (g, tb): wave w runs the fmaf chain of slice
// s = 4g + w for the TB tokens tb*TB .. tb*TB+TB-1 (with a SliceNorm, x is
// the residual stream and the block first normalises its tokens' rows -
// rms_norm of kappa/qwen3/norms.py:10-16 - writing its four slices of the
// normalised rows for the expert kernels), a lane owning EPL
// consecutive experts (all 64 rows of the slice in flight at once when they
// fit in 64 registers). The block then applies tree levels st = 1 and 2 to its
// four slices (the zero-padded tree's aligned group of four) and writes the
// group partial part[t][g][e], g < Q = max(1, P / 4).
// k_route_finish, one wave per token: tree levels st = 4, 8, ... over the Q
// group partials (the levels st >= 4 of the same tree), then the top-k and
// softmax of k_route.
// ---------------------------------------------------------------------------
template <typename A, int RT, int EPL, int TB>
__global__ __launch_bounds__(256) void k_route_slices(int T, int D, int E, int P, int Q, const A* __restrict__ x,
                                                       const void* __restrict__ rw, const void* __restrict__ rscale,
                                                       int scale_bf16, int scale_pc, float* __restrict__ part,
                                                       const kmoe_host::SliceNorm nm) {
  using Row = RouterRow<RT, EPL>;
  constexpr int U = Row::kWords <= 1 ? 64 : 64 / Row::kWords;  // rows per load stage
  __shared__ float xs[4][kRouterSlice][TB];
  __shared__ float red[2][TB * EPL][64];
  __shared__ float rfac[TB];
  extern __shared__ float nrow[];  // with nm.scale: TB staged rows, norm_row_floats(D) each
  const int g = blockIdx.x, t0 = blockIdx.y * TB;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int s = 4 * g + w;
  const int d0 = s * kRouterSlice;
  const int NRF = norm_row_floats(D);
  if (nm.scale) {
    // x is the residual stream h: wave tt reduces row t0 + tt (the canonical
    // rms_norm order); the slices are normalised below
    if (w < TB && t0 + w < T) {
      const float r = wave_rms_factor(x + (int64_t)(t0 + w) * D, D, nm.eps, nrow + w * NRF);
      if (lane == 0) rfac[w] = r;
    }
    __syncthreads();
  }
  for (int i = threadIdx.x; i < 4 * kRouterSlice * TB; i += blockDim.x) {
    const int tt = i % TB, r = (i / TB) % kRouterSlice, ws = i / (TB * kRouterSlice);
    const int d = (4 * g + ws) * kRouterSlice + r;
    float v = 0.0f;
    if (t0 + tt < T && d < D) {
      if (nm.scale) {
        // the block's input h2 = round_act((h * r) * scale): staged here and
        // written out for the expert kernels (each block writes its slices)
        const float sc = load_scale(nm.scale, nm.scale_bf16, d);
        v = rms_apply<A>(nrow[tt * NRF + (d >> 6) * (kRouterSlice + 1) + (d & 63)], rfac[tt], sc);
        Act<A>::store(reinterpret_cast<A*>(nm.h2), (int64_t)(t0 + tt) * D + d, v);
      } else {
        v = Act<A>::load(x, (int64_t)(t0 + tt) * D + d);
      }
    }
    xs[ws][r][tt] = v;
  }
  const int LPR = (E + EPL - 1) / EPL;
  const int e0 = lane * EPL;
  float sc[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    sc[i] = 0.0f;
    if (RT == 2 && e0 + i < E) sc[i] = load_scale(rscale, scale_bf16, scale_pc ? e0 + i : 0);
  }
  float acc[TB][EPL];
#pragma unroll
  for (int tt = 0; tt < TB; ++tt)
#pragma unroll
    for (int i = 0; i < EPL; ++i) acc[tt][i] = 0.0f;
  __syncthreads();
  if (lane < LPR && d0 < D) {
    const int n = min(kRouterSlice, D - d0);
    if (E % EPL == 0 && n == kRouterSlice) {
      // row pointers are uniform (scalar registers), the lane offset is e0
      constexpr int kBpe = Row::kBytes / EPL;
      const char* row0 = reinterpret_cast<const char*>(rw) + (int64_t)d0 * E * kBpe;
      const int64_t pitch = (int64_t)E * kBpe;
      const int loff = e0 * kBpe;
      for (int db = 0; db < kRouterSlice; db += U) {
        typename Row::Raw raw[U];
#pragma unroll
        for (int u = 0; u < U; ++u) Row::load_at(row0 + (db + u) * pitch, loff, raw[u]);
#pragma unroll
        for (int u = 0; u < U; ++u) {
          float r[EPL];
          Row::convert(raw[u], sc, r);
#pragma unroll
          for (int tt = 0; tt < TB; ++tt) {
            const float xv = xs[w][db + u][tt];
#pragma unroll
            for (int i = 0; i < EPL; ++i) acc[tt][i] = __builtin_fmaf(xv, r[i], acc[tt][i]);
          }
        }
      }
    } else {
      for (int r0 = 0; r0 < n; ++r0) {
        float r[EPL];
#pragma unroll
        for (int i = 0; i < EPL; ++i)
          r[i] = (e0 + i < E) ? Row::load1(rw, (int64_t)(d0 + r0) * E + e0 + i, sc[i]) : 0.0f;
#pragma unroll
        for (int tt = 0; tt < TB; ++tt) {
          const float xv = xs[w][r0][tt];
#pragma unroll
          for (int i = 0; i < EPL; ++i) acc[tt][i] = __builtin_fmaf(xv, r[i], acc[tt][i]);
        }
      }
    }
  }
  // tree levels st = 1 (slices 0+1, 2+3) and st = 2 (0+2) of the group
  if (w & 1) {
#pragma unroll
    for (int tt = 0; tt < TB; ++tt)
#pragma unroll
      for (int i = 0; i < EPL; ++i) red[w >> 1][tt * EPL + i][lane] = acc[tt][i];
  }
  __syncthreads();
  if (!(w & 1) && 1 < P) {
#pragma unroll
    for (int tt = 0; tt < TB; ++tt)
#pragma unroll
      for (int i = 0; i < EPL; ++i) acc[tt][i] = acc[tt][i] + red[w >> 1][tt * EPL + i][lane];
  }
  __syncthreads();
  if (w == 2) {
#pragma unroll
    for (int tt = 0; tt < TB; ++tt)
#pragma unroll
      for (int i = 0; i < EPL; ++i) red[0][tt * EPL + i][lane] = acc[tt][i];
  }
  __syncthreads();
  if (w != 0 || lane >= LPR) return;
#pragma unroll
  for (int tt = 0; tt < TB; ++tt) {
    if (t0 + tt >= T) break;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const float v = 2 < P ? acc[tt][i] + red[0][tt * EPL + i][lane] : acc[tt][i];
      if (e0 + i < E) part[((int64_t)(t0 + tt) * Q + g) * E + e0 + i] = v;
    }
  }
}

template <int EPL>
__global__ __launch_bounds__(256) void k_route_finish(int T, int E, int K, int Q, const float* __restrict__ part,
                                                       float* __restrict__ logits, int32_t* __restrict__ topk_idx,
                                                       float* __restrict__ topk_w, int out_bf16) {
  __shared__ TopkLds tk[4];
  const int w = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + w;
  if (t >= T) return;  // per wave: this kernel has no block-wide barrier
  finish_token<EPL>(t, E, K, Q, part, logits, topk_idx, topk_w, out_bf16, nullptr, tk[w]);
}

__global__ __launch_bounds__(256) void k_dispatch_count(int T, int E, int K, const int32_t* __restrict__ topk_idx,
                                                         int32_t* __restrict__ hist) {
  __shared__ unsigned long long mask[kMaxExperts];
  chunk_masks(T, E, K, blockIdx.x, topk_idx, mask);
  for (int e = threadIdx.x; e < E; e += blockDim.x) hist[(int64_t)blockIdx.x * E + e] = __popcll(mask[e]);
}

// T <= NW <= 16: the finish is one block of NW waves, one token each, so it
// also runs the dispatch sort of the tokens (the selections pass through LDS;
// no second kernel). At larger T a single block's serial top-ks and sort
// cost more than the separate dispatch kernel.
template <int EPL, int NW>
__global__ __launch_bounds__(64 * NW) void k_route_finish_dispatch(
    int T, int E, int K, int Q, const float* __restrict__ part, float* __restrict__ logits,
    int32_t* __restrict__ topk_idx, float* __restrict__ topk_w, int out_bf16, int32_t* __restrict__ group_sizes,
    int32_t* __restrict__ offsets, int32_t* __restrict__ active, int32_t* __restrict__ sorted_token,
    int32_t* __restrict__ sorted_expert, int32_t* __restrict__ inv, int cap) {
  static_assert(NW >= 4 && NW <= 16, "dispatch_chunk needs 256 threads; one wave per token");
  __shared__ TopkLds tk[NW];
  __shared__ DispatchLds L;
  __shared__ int32_t idx_lds[NW * kMaxTopK];
  const int w = threadIdx.x >> 6;
  if (w < T) finish_token<EPL>(w, E, K, Q, part, logits, topk_idx, topk_w, out_bf16, idx_lds, tk[w]);
  __syncthreads();
  if (dispatch_fits_wave(T * K, E))
    dispatch_wave(T, E, K, idx_lds, group_sizes, offsets, active, sorted_token, sorted_expert, inv, cap);
  else
    dispatch_chunk(T, E, K, 0, 1, idx_lds, nullptr, group_sizes, offsets, active, sorted_token, sorted_expert, inv,
                   cap, L);
}

__global__ __launch_bounds__(256) void k_dispatch_scatter(int T, int E, int K, int nblk,
                                                           const int32_t* __restrict__ topk_idx,
                                                           const int32_t* __restrict__ hist,
                                                           int32_t* __restrict__ group_sizes,
                                                           int32_t* __restrict__ offsets, int32_t* __restrict__ active,
                                                           int32_t* __restrict__ sorted_token,
                                                           int32_t* __restrict__ sorted_expert,
                                                           int32_t* __restrict__ inv, int cap) {
  __shared__ DispatchLds L;
  dispatch_chunk(T, E, K, blockIdx.x, nblk, topk_idx, hist, group_sizes, offsets, active, sorted_token, sorted_expert,
                 inv, cap, L);
}


// ---------------------------------------------------------------------------
// Two-phase router: bf16 activations and router, D = 64 S with S a power of
// two from 8 to 64, E % 16 == 0, E <= 256.
//
// Bit-exact top-k needs the canonical logits (k_route's order) only where the
// ranking is in doubt. Phase 1 computes every logit on the matrix cores
// (v_mfma_f32_16x16x32_bf16: exact products, f32 sums in the hardware's order):
// L~[t,e]. The exact sum, the canonical L and L~ differ by at most
// c * sum_d |x_d r_de| <= c * ||x_t|| * ||r_e|| (Cauchy-Schwarz), where c covers
// the MFMA's accumulation (taken as up to 2D roundings of up to 2u each,
// u = 2^-24), the canonical chains and tree (64 + log2 P roundings), the
// rounding of the norms and of L~ -/+ delta (the host passes c). So L lies in
// [lo, hi] = [L~ - delta, L~ + delta], delta = c * ||x_t|| * ||r_e|| + 1e-30.
// Let tau be the K-th largest lo (the search stops at 16 key bits, which can
// only lower it). An expert whose hi is below tau has K experts strictly above
// it and cannot be selected, ties included; the top K are among the
// candidates {e : hi_e >= tau}. Phase 2 recomputes the candidates' logits in
// the canonical order, ranks them (value descending, ties to the lower index)
// and takes the softmax of the first K, as wave_topk does. A token with a
// non-finite L~ or bound takes every expert as a candidate.
//
// The router is transposed once per call into rTq [E][8][S][8] bf16: element
// (e, d = 64 s + 8 i + j) at ((e * 8 + i) * S + s) * 8 + j. Eight consecutive
// hidden indices of one expert (an MFMA B fragment, or eight steps of a slice
// chain) are one 16-byte load, and the 8-element pieces i of the S slices of
// one expert are contiguous, so the slice lanes of a chain read 16 S
// consecutive bytes per step.
// ---------------------------------------------------------------------------
constexpr int kRouteSliceBytes = 144;  // a 64-element bf16 slice of x in LDS, padded by 16 bytes

// Block (e, p): experts 16e .. 16e+15, hidden rows 256p .. 256p+255 (slices
// 4p .. 4p+3) of the router: rTq (exact; through LDS, so the stores are the
// 64-byte runs of four slices of one eighth), the partial sums of squares of
// the 16 columns npart[p][e], and the histograms zeroed. D % 256 == 0.
__global__ __launch_bounds__(256) void k_router_prep(int D, int E, const uint16_t* __restrict__ r,
                                                      uint16_t* __restrict__ rtq, float* __restrict__ npart,
                                                      int32_t* __restrict__ hist, int nhist) {
  __shared__ float red[4][16];
  __shared__ __attribute__((aligned(16))) uint16_t tile[16 * 8 * 4 * 8];  // [e][eighth][slice][8]
  const int e0 = blockIdx.x * 16, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int nb = gridDim.x * gridDim.y, b = blockIdx.y * gridDim.x + blockIdx.x;
  for (int i = b * 256 + tid; i < nhist; i += nb * 256) hist[i] = 0;
  const int d = blockIdx.y * 256 + tid, S = D >> 6;
  const uint4* row = reinterpret_cast<const uint4*>(r + (int64_t)d * E + e0);
  const uint4 a = row[0], c = row[1];
  const uint32_t wd[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
  const int sl = tid >> 6, i8 = (tid >> 3) & 7, j = tid & 7;
  float sq[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t bits = (i & 1) ? (wd[i >> 1] >> 16) : (wd[i >> 1] & 0xffffu);
    const float v = __uint_as_float(bits << 16);
    tile[((i * 8 + i8) * 4 + sl) * 8 + j] = (uint16_t)bits;
    sq[i] = v * v;
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sq[i] += __shfl_xor(sq[i], off, 64);
  }
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) red[w][i] = sq[i];
  }
  __syncthreads();
  if (tid < 16) npart[(int64_t)blockIdx.y * E + e0 + tid] = ((red[0][tid] + red[1][tid]) + red[2][tid]) + red[3][tid];
  // 512 pieces of 16 bytes: piece q = (expert q / 32, eighth (q / 4) % 8, slice q % 4)
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int q = tid + 256 * k;
    const int e = q >> 5, ei = (q >> 2) & 7, s4 = q & 3;
    *reinterpret_cast<uint4*>(rtq + ((int64_t)((e0 + e) * 8 + ei) * S + 4 * blockIdx.y + s4) * 8) =
        reinterpret_cast<const uint4*>(tile)[q];
  }
}

// Order-preserving key of a float (-0.0 keyed as +0.0), as wave_topk.
__device__ __forceinline__ uint32_t float_key(float v) {
  const uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
  return (u >> 31) ? ~u : (u | 0x80000000u);
}

// Block: TB tokens, one wave each. The token rows are staged in LDS first
// (slice-padded: slice s of row r at r * XRS + s * 144). Phase 1: the
// 16-token x 16-expert logit tiles over waves (tile = w % NT, and with more
// waves than tiles the reduction split KS ways, ks = w / NT), A from LDS, B
// from rTq in batches of 16 steps; partial sums to LDS, and the waves of tile
// 0 also sum the squares of their rows for ||x||. Phase 2: wave w finishes
// token w: P lanes per candidate chain (the zero-padded slice count), 64 / P
// chains side by side.
template <int EPL, int P, int TB>
__global__ __launch_bounds__(64 * TB) void k_route_mfma(int T, int D, int E, int K, const uint16_t* __restrict__ x,
                                                         const uint16_t* __restrict__ rtq,
                                                         const float* __restrict__ npart, float cbound,
                                                         int32_t* __restrict__ topk_idx, float* __restrict__ topk_w,
                                                         int32_t* __restrict__ hist, int out_bf16) {
  static_assert(EPL <= 4, "experts per lane");
  constexpr int CP = 64 / P;  // chains side by side in a wave
  extern __shared__ __attribute__((aligned(16))) uint8_t lds8[];
  __shared__ TopkLds tk[TB];
  __shared__ float nxp[16][16];  // [ks][row] partial sums of squares
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int t0 = blockIdx.x * TB;
  const int S = D >> 6;
  const int XRS = S * kRouteSliceBytes + 16;
  const int NT = E >> 4;
  const int KS = TB >= NT ? TB / NT : 1;
  uint8_t* xs = lds8;
  float* lgp = reinterpret_cast<float*>(lds8 + TB * XRS);
  const int lgp_floats = TB * 256 > 16 * E ? TB * 256 : 16 * E;
  int32_t* cand = reinterpret_cast<int32_t*>(lgp + lgp_floats) + w * E;
  float* cval = reinterpret_cast<float*>(reinterpret_cast<int32_t*>(lgp + lgp_floats) + TB * E) + w * E;
  // the router columns' partial sums of squares, [D / 256][E], staged with the token rows
  const int NPD = (D + 255) >> 8;
  float* npl = reinterpret_cast<float*>(lds8 + TB * XRS) + lgp_floats + 2 * TB * E;

  // ---- phase 1 assignment: tiles tile0, tile0 + tstep, ... over steps [s0, s1) ----
  // Step st, k-lane kq takes the 8 hidden indices of piece p = 4 st + kq, with
  // piece p = slice p % S, eighth p / S (any one-to-one map of the reduction
  // works when A and B follow it): the four k-lanes of an expert then read 64
  // consecutive bytes of rTq.
  const int m = lane & 15, kq = lane >> 4;
  const int nsteps = D >> 5;
  const int spk = (nsteps + KS - 1) / KS;
  const bool split = TB >= NT;
  // with more waves than tiles, waves past KS * NT (NT not dividing TB) sit out
  const int tile0 = split ? (w < KS * NT ? w % NT : NT) : w;
  const int tstep = split ? NT : TB;
  const int ks = split ? w / NT : 0;
  const int s0 = ks * spk, s1 = min(nsteps, s0 + spk);
  static_assert((P & (P - 1)) == 0 && P >= 8, "slices: a power of two");
  constexpr int LP = P == 8 ? 3 : (P == 16 ? 4 : (P == 32 ? 5 : 6));  // log2 S (S == P)
  auto bload = [&](int tile, int st) {
    const int p = 4 * st + kq;
    return *reinterpret_cast<const uint4*>(rtq + ((int64_t)((16 * tile + m) * 8 + (p >> LP)) * P + (p & (P - 1))) * 8);
  };
  // router fragments in batches of kRouteBatch steps per wave
  constexpr int kRouteBatch = 8;
  uint4 b[kRouteBatch];
  const bool pre = tile0 < NT && s1 - s0 >= kRouteBatch;

  // ---- the token rows into LDS (rows past T as zeros), the norm partials,
  // and the first batch of router fragments requested behind them ----
  {
    const int cpr = D >> 3;  // 16-byte pieces per row
    const int per = (TB * cpr) / (64 * TB);  // per thread (D / 512, exact)
    constexpr int PMAX = TB >= 16 ? 4 : 8;    // the host runs 16 tokens per block up to D = 2048
    uint4 v[PMAX];
#pragma unroll
    for (int k = 0; k < PMAX; ++k) {
      if (k < per) {
        const int i = threadIdx.x + k * 64 * TB;
        const int r = i / cpr, c = i - r * cpr;
        v[k] = t0 + r < T ? reinterpret_cast<const uint4*>(x + (int64_t)(t0 + r) * D)[c] : uint4{0u, 0u, 0u, 0u};
      }
    }
    if (pre) {
#pragma unroll
      for (int j = 0; j < kRouteBatch; ++j) b[j] = bload(tile0, s0 + j);
    }
    for (int i = threadIdx.x; i < NPD * E; i += 64 * TB) npl[i] = npart[i];
#pragma unroll
    for (int k = 0; k < PMAX; ++k) {
      if (k < per) {
        const int i = threadIdx.x + k * 64 * TB;
        const int r = i / cpr, c = i - r * cpr;
        *reinterpret_cast<uint4*>(xs + r * XRS + (c >> 3) * kRouteSliceBytes + (c & 7) * 16) = v[k];
      }
    }
  }
  __syncthreads();

  // ---- phase 1 ----
  {
    const uint8_t* xa = xs + (m % TB) * XRS;
    for (int tile = tile0; tile < NT; tile += tstep) {
      const int e = 16 * tile + m;
      floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
      float ss = 0.0f;
      auto step = [&](int st, const uint4 bb) {
        const int p = 4 * st + kq;
        const uint4 a = *reinterpret_cast<const uint4*>(xa + (p & (P - 1)) * kRouteSliceBytes + (p >> LP) * 16);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, bb),
                                                      acc, 0, 0, 0);
        if (tile == 0) {
          const uint32_t av[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float lo = __uint_as_float(av[i] << 16), hi = __uint_as_float(av[i] & 0xffff0000u);
            ss = __builtin_fmaf(lo, lo, ss);
            ss = __builtin_fmaf(hi, hi, ss);
          }
        }
      };
      int st = s0;
      bool have = tile == tile0 && pre;  // b holds steps s0 .. s0 + kRouteBatch - 1
      for (; st + kRouteBatch <= s1; st += kRouteBatch) {
        if (!have) {
#pragma unroll
          for (int j = 0; j < kRouteBatch; ++j) b[j] = bload(tile, st + j);
        }
        have = false;
#pragma unroll
        for (int j = 0; j < kRouteBatch; ++j) step(st + j, b[j]);
      }
      for (; st < s1; ++st) step(st, bload(tile, st));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = 4 * kq + j;
        if (row < TB) lgp[(ks * 16 + row) * E + e] = acc[j];
      }
      if (tile == 0) {
        // row m's squares over this wave's reduction range: the four k-lanes of the row
        ss += __shfl_xor(ss, 16, 64);
        ss += __shfl_xor(ss, 32, 64);
        if (kq == 0) nxp[ks][m] = ss;
      }
    }
  }
  __syncthreads();

  // ---- phase 2: wave w, token t0 + w ----
  const int t = t0 + w;
  if (t >= T) return;
  const int s = lane % P, g = lane / P;
  float ss = 0.0f;
  for (int k2 = 0; k2 < KS; ++k2) ss += nxp[k2][w];
  const float nxv = sqrtf(ss);
  float lo[EPL], hi[EPL];
  bool bad = !(nxv <= 3.0e38f);
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane + 64 * i;
    lo[i] = -INFINITY;
    hi[i] = -INFINITY;
    if (e < E) {
      float v = lgp[w * E + e];
      for (int k2 = 1; k2 < KS; ++k2) v += lgp[(k2 * 16 + w) * E + e];
      float n2 = 0.0f;
      for (int p = 0; p < NPD; ++p) n2 += npl[p * E + e];
      const float dl = __builtin_fmaf(cbound * nxv, sqrtf(n2), 1e-30f);
      lo[i] = v - dl;
      hi[i] = v + dl;
      bad = bad || !(lo[i] >= -3.0e38f && hi[i] <= 3.0e38f);
    }
  }
  const bool all = __ballot(bad) != 0ull;
  // tau: a lower bound of the K-th largest lo, to 16 key bits
  uint32_t lk[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) lk[i] = lane + 64 * i < E ? float_key(lo[i]) : 0u;
  uint32_t thr = 0;
  if (!all) {
    for (int b = 31; b >= 16; --b) {
      const uint32_t c = thr | (1u << b);
      int cnt = 0;
#pragma unroll
      for (int i = 0; i < EPL; ++i) cnt += __popcll(__ballot(lk[i] >= c));
      if (cnt >= K) thr = c;
    }
  }
  // the candidates, in expert order
  const unsigned long long below = (1ull << lane) - 1ull;
  int nc = 0;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane + 64 * i;
    const bool c = e < E && (all || float_key(hi[i]) >= thr);
    const unsigned long long mk = __ballot(c);
    if (c) cand[nc + __popcll(mk & below)] = e;
    nc += __popcll(mk);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // canonical logits of the candidates: lane s of a group of P runs slice s of
  // candidates g, g + CP, ... (x[64 s ..] times r[64 s ..][e], one fmaf chain
  // from +0), then the pairwise tree over the P slices
  float xf[64];
  if (s < S) {
    const uint8_t* xrow = xs + w * XRS + s * kRouteSliceBytes;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const uint4 v = *reinterpret_cast<const uint4*>(xrow + 16 * q);
      const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        xf[8 * q + 2 * i] = __uint_as_float(wd[i] << 16);
        xf[8 * q + 2 * i + 1] = __uint_as_float(wd[i] & 0xffff0000u);
      }
    }
  }
  for (int c = g; c < ((nc + CP - 1) / CP) * CP; c += CP) {
    float acc = 0.0f;
    if (s < S && c < nc) {
      // chains past the candidates do no loads and are not stored
      const uint4* rp = reinterpret_cast<const uint4*>(rtq + ((int64_t)cand[c] * 8 * S + s) * 8);
      uint4 rv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) rv[i] = rp[(int64_t)i * S];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t wd[4] = {rv[i].x, rv[i].y, rv[i].z, rv[i].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc = __builtin_fmaf(xf[8 * i + 2 * j], __uint_as_float(wd[j] << 16), acc);
          acc = __builtin_fmaf(xf[8 * i + 2 * j + 1], __uint_as_float(wd[j] & 0xffff0000u), acc);
        }
      }
    }
#pragma unroll
    for (int st = 1; st < P; st <<= 1) acc = acc + __shfl_down(acc, st, P);
    if (s == 0 && c < nc) cval[c] = acc;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (nc <= 64) {
    // rank the candidates (value descending, ties to the lower expert; NaN as
    // -inf), then the softmax of the first K in rank order (the sum in rank
    // order, as wave_topk)
    float mv = -INFINITY;
    int me = 0x7fffffff, rank = 0;
    if (lane < nc) {
      const float q = cval[lane];
      mv = q == q ? q : -INFINITY;
      me = cand[lane];
      for (int c = 0; c < nc; ++c) {
        const float qc0 = cval[c];
        const float qc = qc0 == qc0 ? qc0 : -INFINITY;
        rank += (qc > mv) || (qc == mv && cand[c] < me);
      }
    }
    if (lane < nc && rank < K) {
      tk[w].sidx[rank] = me;
      tk[w].key[rank] = __float_as_uint(mv);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const float l0 = __uint_as_float(tk[w].key[0]);
    const float ej = lane < K ? expf(__uint_as_float(tk[w].key[lane]) - l0) : 0.0f;
    float ssum = 0.0f;
    for (int j = 0; j < K; ++j) ssum = ssum + __shfl(ej, j, 64);
    if (lane < K) {
      const int e = tk[w].sidx[lane];
      const float p = ej / ssum;
      topk_w[(int64_t)t * K + lane] = out_bf16 ? round_bf16(p) : p;
      topk_idx[(int64_t)t * K + lane] = e;
      atomicAdd(&hist[(int64_t)(t / kDispatchBlock) * E + e], 1);
    }
  } else {
    // more than 64 candidates (a token taking every expert): wave_topk over the
    // canonical logits by expert; the candidate list is increasing in expert
    float v[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int e = lane + 64 * i;
      v[i] = -INFINITY;
      if (e < E) {
        int a = 0, z = nc - 1;
        while (a < z) {
          const int mid = (a + z) >> 1;
          if (cand[mid] < e)
            a = mid + 1;
          else
            z = mid;
        }
        if (cand[a] == e) {
          const float q = cval[a];
          v[i] = q == q ? q : -INFINITY;
        }
      }
    }
    wave_topk<EPL>(t, E, K, v, topk_idx, topk_w, out_bf16, nullptr, tk[w]);
    if (lane < K) atomicAdd(&hist[(int64_t)(t / kDispatchBlock) * E + topk_idx[(int64_t)t * K + lane]], 1);
  }
}

}  // namespace kmoe

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
namespace kmoe_host {

using namespace kmoe;

struct RouteShape {
  int S, P, EPL, LPR, SPW, G, NWB, TB;
  size_t lds;
};

static RouteShape route_shape(const kmoe_desc& d) {
  RouteShape r;
  const int D = (int)d.hidden, E = (int)d.num_experts;
  const int T = (int)d.tokens;
  r.S = (D + kRouterSlice - 1) / kRouterSlice;
  r.P = 1;
  while (r.P < r.S) r.P <<= 1;
  r.EPL = E <= 512 ? 8 : 16;
  r.LPR = (E + r.EPL - 1) / r.EPL;
  r.SPW = 1;
  while (2 * r.SPW * r.LPR <= 64) r.SPW <<= 1;
  const int NG = r.P > r.SPW ? r.P / r.SPW : 1;
  r.G = NG > 16 ? NG / 16 : 1;
  r.NWB = NG / r.G;
  // tokens per block: accumulators within the register budget, x stage <= 80 KB
  // (two blocks per CU), partials <= 64 KB, and enough blocks to cover the chip
  int tb = 8;
  const int acc_cap = r.G > 1 ? 2 * r.EPL : 64;
  auto x_bytes = [&](int t) { return (size_t)4 * r.S * (kRouterSlice * t + 4); };
  auto part_bytes = [&](int t) { return (size_t)4 * r.NWB * t * E + r.NWB * sizeof(TopkLds); };
  while (tb > 1 && (tb * r.EPL > acc_cap || x_bytes(tb) > 81920 || part_bytes(tb) > 65536)) tb >>= 1;
  // two blocks per CU where four tokens per block still give them (T = 2048:
  // 35.9 -> 32.3 us); fewer tokens per block re-read the router too often
  while (tb > 4 && (T + tb - 1) / tb < 512) tb >>= 1;
  while (tb > 1 && (T + tb - 1) / tb < 256) tb >>= 1;
  r.TB = tb;
  r.lds = std::max(x_bytes(tb), part_bytes(tb));
  return r;
}

template <typename A, int RT, int EPL, int TB, int G>
static void launch_route_k(const kmoe_desc& d, const RouteShape& rs, const void* x, const kmoe_weight& r,
                           float* logits, int32_t* topk_idx, float* topk_w, hipStream_t st) {
  const int T = (int)d.tokens, D = (int)d.hidden, E = (int)d.num_experts, K = (int)d.top_k;
  const int scale_bf16 = (r.dtype == KMOE_DTYPE_I8 && r.scale_dtype == KMOE_DTYPE_BF16) ? 1 : 0;
  const int scale_pc = (r.dtype == KMOE_DTYPE_I8 && r.scale_kind == KMOE_SCALE_CHANNEL) ? 1 : 0;
  const int out_bf16 = d.act_dtype == KMOE_DTYPE_BF16 ? 1 : 0;
  hipLaunchKernelGGL((k_route<A, RT, EPL, TB, G>), dim3((T + TB - 1) / TB), dim3(64 * rs.NWB), rs.lds, st, T, D, E,
                     K, rs.LPR, rs.SPW, rs.P, reinterpret_cast<const A*>(x), r.values, r.scale, scale_bf16,
                     scale_pc, logits, topk_idx, topk_w, out_bf16);
}

template <typename A, int RT, int EPL>
static void route_tb(const kmoe_desc& d, const RouteShape& rs, const void* x, const kmoe_weight& r, float* logits,
                     int32_t* idx, float* w, hipStream_t st) {
  if (rs.G == 4) {
    if (rs.TB == 2) return launch_route_k<A, RT, EPL, 2, 4>(d, rs, x, r, logits, idx, w, st);
    return launch_route_k<A, RT, EPL, 1, 4>(d, rs, x, r, logits, idx, w, st);
  }
  if (rs.G == 2) {
    if (rs.TB == 2) return launch_route_k<A, RT, EPL, 2, 2>(d, rs, x, r, logits, idx, w, st);
    return launch_route_k<A, RT, EPL, 1, 2>(d, rs, x, r, logits, idx, w, st);
  }
  switch (rs.TB) {
    case 8:
      if constexpr (EPL == 8) return launch_route_k<A, RT, EPL, 8, 1>(d, rs, x, r, logits, idx, w, st);
      [[fallthrough]];
    case 4:
      if constexpr (EPL == 8) return launch_route_k<A, RT, EPL, 4, 1>(d, rs, x, r, logits, idx, w, st);
      [[fallthrough]];
    case 2:
      return launch_route_k<A, RT, EPL, 2, 1>(d, rs, x, r, logits, idx, w, st);
    default:
      return launch_route_k<A, RT, EPL, 1, 1>(d, rs, x, r, logits, idx, w, st);
  }
}

template <typename A, int RT>
static void route_epl(const kmoe_desc& d, const RouteShape& rs, const void* x, const kmoe_weight& r, float* logits,
                      int32_t* idx, float* w, hipStream_t st) {
  if (rs.EPL == 8) return route_tb<A, RT, 8>(d, rs, x, r, logits, idx, w, st);
  return route_tb<A, RT, 16>(d, rs, x, r, logits, idx, w, st);
}

template <typename A>
static void route_rt(const kmoe_desc& d, const RouteShape& rs, const void* x, const kmoe_weight& r, float* logits,
                     int32_t* idx, float* w, hipStream_t st) {
  if (r.dtype == KMOE_DTYPE_F32) return route_epl<A, 0>(d, rs, x, r, logits, idx, w, st);
  if (r.dtype == KMOE_DTYPE_BF16) return route_epl<A, 1>(d, rs, x, r, logits, idx, w, st);
  return route_epl<A, 2>(d, rs, x, r, logits, idx, w, st);
}

hipError_t launch_route(const kmoe_desc& d, const void* x, const kmoe_weight& r, float* logits, int32_t* topk_idx,
                        float* topk_w, int32_t* hist, hipStream_t st) {
  const RouteShape rs = route_shape(d);
  if (d.act_dtype == KMOE_DTYPE_BF16)
    route_rt<uint16_t>(d, rs, x, r, logits, topk_idx, topk_w, st);
  else
    route_rt<float>(d, rs, x, r, logits, topk_idx, topk_w, st);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || !hist) return err;
  return launch_dispatch_count(d, topk_idx, hist, st);
}

hipError_t launch_dispatch_count(const kmoe_desc& d, const int32_t* topk_idx, int32_t* hist, hipStream_t st) {
  const int T = (int)d.tokens, E = (int)d.num_experts, K = (int)d.top_k;
  const int nblk = (T + kDispatchBlock - 1) / kDispatchBlock;
  hipLaunchKernelGGL(k_dispatch_count, dim3(nblk), dim3(256), 0, st, T, E, K, topk_idx, hist);
  return hipGetLastError();
}

// Split router: experts per lane for the slice kernel (>= 4 bytes of weights
// per row and lane, at most 64 lanes per row), tokens per block, group count.
struct SplitShape {
  int EPL, TB, P, Q;
};

static SplitShape split_shape(const kmoe_desc& d, const kmoe_weight& r) {
  SplitShape sh;
  const int E = (int)d.num_experts, T = (int)d.tokens;
  const int S = (int)((d.hidden + kRouterSlice - 1) / kRouterSlice);
  const int min_epl = r.dtype == KMOE_DTYPE_F32 ? 1 : (r.dtype == KMOE_DTYPE_BF16 ? 2 : 4);
  sh.EPL = min_epl;
  while (sh.EPL * 64 < E) sh.EPL <<= 1;
  sh.TB = T <= 16 ? 1 : (T <= 64 ? 2 : 4);
  sh.P = 1;
  while (sh.P < S) sh.P <<= 1;
  sh.Q = route_split_groups(d);
  return sh;
}

template <typename A, int RT, int EPL, int TB>
static void launch_slices(const kmoe_desc& d, const SplitShape& sh, const void* x, const kmoe_weight& r, float* part,
                          const SliceNorm& nm, hipStream_t st) {
  const int T = (int)d.tokens, D = (int)d.hidden, E = (int)d.num_experts;
  const int scale_bf16 = (r.dtype == KMOE_DTYPE_I8 && r.scale_dtype == KMOE_DTYPE_BF16) ? 1 : 0;
  const int scale_pc = (r.dtype == KMOE_DTYPE_I8 && r.scale_kind == KMOE_SCALE_CHANNEL) ? 1 : 0;
  const size_t lds = nm.scale ? (size_t)TB * norm_row_floats(D) * sizeof(float) : 0;
  hipLaunchKernelGGL((k_route_slices<A, RT, EPL, TB>), dim3(sh.Q, (T + TB - 1) / TB), dim3(256), lds, st, T, D, E,
                     sh.P, sh.Q, reinterpret_cast<const A*>(x), r.values, r.scale, scale_bf16, scale_pc, part, nm);
}

template <typename A, int RT, int EPL>
static void slices_tb(const kmoe_desc& d, const SplitShape& sh, const void* x, const kmoe_weight& r, float* part,
                      const SliceNorm& nm, hipStream_t st) {
  if (sh.TB == 1) return launch_slices<A, RT, EPL, 1>(d, sh, x, r, part, nm, st);
  if (sh.TB == 2) return launch_slices<A, RT, EPL, 2>(d, sh, x, r, part, nm, st);
  return launch_slices<A, RT, EPL, 4>(d, sh, x, r, part, nm, st);
}

template <typename A, int RT>
static void slices_epl(const kmoe_desc& d, const SplitShape& sh, const void* x, const kmoe_weight& r, float* part,
                       const SliceNorm& nm, hipStream_t st) {
  switch (sh.EPL) {
    case 1:
      if constexpr (RT == 0) return slices_tb<A, RT, 1>(d, sh, x, r, part, nm, st);
      [[fallthrough]];
    case 2:
      if constexpr (RT != 2) return slices_tb<A, RT, 2>(d, sh, x, r, part, nm, st);
      [[fallthrough]];
    case 4:
      return slices_tb<A, RT, 4>(d, sh, x, r, part, nm, st);
    case 8:
      return slices_tb<A, RT, 8>(d, sh, x, r, part, nm, st);
    default:
      return slices_tb<A, RT, 16>(d, sh, x, r, part, nm, st);
  }
}

template <typename A>
static void slices_rt(const kmoe_desc& d, const SplitShape& sh, const void* x, const kmoe_weight& r, float* part,
                      const SliceNorm& nm, hipStream_t st) {
  if (r.dtype == KMOE_DTYPE_F32) return slices_epl<A, 0>(d, sh, x, r, part, nm, st);
  if (r.dtype == KMOE_DTYPE_BF16) return slices_epl<A, 1>(d, sh, x, r, part, nm, st);
  return slices_epl<A, 2>(d, sh, x, r, part, nm, st);
}

template <int EPL>
static void launch_finish(const kmoe_desc& d, const SplitShape& sh, const float* part, float* logits,
                          int32_t* topk_idx, float* topk_w, const DispatchOut* ds, hipStream_t st) {
  const int T = (int)d.tokens, E = (int)d.num_experts, K = (int)d.top_k;
  const int out_bf16 = d.act_dtype == KMOE_DTYPE_BF16 ? 1 : 0;
  if (ds && T <= 4)
    hipLaunchKernelGGL((k_route_finish_dispatch<EPL, 4>), dim3(1), dim3(256), 0, st, T, E, K, sh.Q, part, logits,
                       topk_idx, topk_w, out_bf16, ds->group_sizes, ds->offsets, ds->active, ds->sorted_token,
                       ds->sorted_expert, ds->inv, capacity_of(d));
  else if (ds)
    hipLaunchKernelGGL((k_route_finish_dispatch<EPL, 16>), dim3(1), dim3(1024), 0, st, T, E, K, sh.Q, part, logits,
                       topk_idx, topk_w, out_bf16, ds->group_sizes, ds->offsets, ds->active, ds->sorted_token,
                       ds->sorted_expert, ds->inv, capacity_of(d));
  else
    hipLaunchKernelGGL((k_route_finish<EPL>), dim3((T + 3) / 4), dim3(256), 0, st, T, E, K, sh.Q, part, logits,
                       topk_idx, topk_w, out_bf16);
}

hipError_t launch_route_slices(const kmoe_desc& d, const void* x, const kmoe_weight& r, float* part, hipStream_t st,
                               const SliceNorm* norm) {
  const SplitShape sh = split_shape(d, r);
  const SliceNorm nm = norm ? *norm : SliceNorm{nullptr, 0, 0.0f, nullptr};
  if (d.act_dtype == KMOE_DTYPE_BF16)
    slices_rt<uint16_t>(d, sh, x, r, part, nm, st);
  else
    slices_rt<float>(d, sh, x, r, part, nm, st);
  return hipGetLastError();
}

hipError_t launch_route_split(const kmoe_desc& d, const void* x, const kmoe_weight& r, float* part, float* logits,
                              int32_t* topk_idx, float* topk_w, hipStream_t st, const SliceNorm* norm,
                              const DispatchOut* dispatch) {
  // the dispatch rides along when the finish is a single block
  const DispatchOut* ds = dispatch && split_router_dispatches(d) ? dispatch : nullptr;
  const SplitShape sh = split_shape(d, r);
  const SliceNorm nm = norm ? *norm : SliceNorm{nullptr, 0, 0.0f, nullptr};
  if (d.act_dtype == KMOE_DTYPE_BF16)
    slices_rt<uint16_t>(d, sh, x, r, part, nm, st);
  else
    slices_rt<float>(d, sh, x, r, part, nm, st);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  const int E = (int)d.num_experts;
  if (E <= 64)
    launch_finish<1>(d, sh, part, logits, topk_idx, topk_w, ds, st);
  else if (E <= 128)
    launch_finish<2>(d, sh, part, logits, topk_idx, topk_w, ds, st);
  else if (E <= 256)
    launch_finish<4>(d, sh, part, logits, topk_idx, topk_w, ds, st);
  else if (E <= 512)
    launch_finish<8>(d, sh, part, logits, topk_idx, topk_w, ds, st);
  else
    launch_finish<16>(d, sh, part, logits, topk_idx, topk_w, ds, st);
  return hipGetLastError();
}

hipError_t launch_dispatch(const kmoe_desc& d, const int32_t* topk_idx, const int32_t* hist, int32_t* group_sizes,
                           int32_t* offsets, int32_t* active, int32_t* sorted_token, int32_t* sorted_expert,
                           int32_t* inv, hipStream_t st) {
  const int T = (int)d.tokens, E = (int)d.num_experts, K = (int)d.top_k;
  const int nblk = (T + kDispatchBlock - 1) / kDispatchBlock;
  if (!hist && nblk > 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_dispatch_scatter, dim3(nblk), dim3(256), 0, st, T, E, K, nblk, topk_idx, hist, group_sizes,
                     offsets, active, sorted_token, sorted_expert, inv, capacity_of(d));
  return hipGetLastError();
}

// Two-phase router: the prep kernel (router transposed to rTq, column-norm
// partials, histograms zeroed), then the MFMA logits, the candidates'
// canonical logits, top-k, softmax and the per-64-token expert counts
// (launch_dispatch reads them as it reads k_dispatch_count's).
template <int EPL, int P, int TB>
static void launch_route_mfma_k(const kmoe_desc& d, const uint16_t* x, const uint16_t* rtq, const float* npart,
                                float cb, int32_t* topk_idx, float* topk_w, int32_t* hist, hipStream_t st) {
  const int T = (int)d.tokens, D = (int)d.hidden, E = (int)d.num_experts, K = (int)d.top_k;
  const int XRS = (D / 64) * kRouteSliceBytes + 16;
  const int lgp = TB * 256 > 16 * E ? TB * 256 : 16 * E;
  const size_t lds = (size_t)TB * XRS + 4 * ((size_t)lgp + 2 * (size_t)TB * E + (size_t)((D + 255) / 256) * E);
  hipLaunchKernelGGL((k_route_mfma<EPL, P, TB>), dim3((T + TB - 1) / TB), dim3(64 * TB), lds, st, T, D, E, K, x, rtq,
                     npart, cb, topk_idx, topk_w, hist, d.act_dtype == KMOE_DTYPE_BF16 ? 1 : 0);
}

// P lanes per candidate chain (the slice count rounded up to a power of two);
// 16 tokens per block up to D = 2048, 8 above (the staged rows fit LDS).
template <int EPL>
static void route_mfma_p(const kmoe_desc& d, const uint16_t* x, const uint16_t* rtq, const float* npart, float cb,
                         int32_t* topk_idx, float* topk_w, int32_t* hist, hipStream_t st) {
  const int S = (int)(d.hidden / 64);
  if (S <= 8) return launch_route_mfma_k<EPL, 8, 16>(d, x, rtq, npart, cb, topk_idx, topk_w, hist, st);
  if (S <= 16) return launch_route_mfma_k<EPL, 16, 16>(d, x, rtq, npart, cb, topk_idx, topk_w, hist, st);
  if (S <= 32) return launch_route_mfma_k<EPL, 32, 16>(d, x, rtq, npart, cb, topk_idx, topk_w, hist, st);
  return launch_route_mfma_k<EPL, 64, 8>(d, x, rtq, npart, cb, topk_idx, topk_w, hist, st);
}

hipError_t launch_route_mfma(const kmoe_desc& d, const void* x, const kmoe_weight& r, void* scratch,
                             int32_t* topk_idx, float* topk_w, int32_t* hist, hipStream_t st) {
  const int T = (int)d.tokens, D = (int)d.hidden, E = (int)d.num_experts;
  char* base = reinterpret_cast<char*>(scratch);
  uint16_t* rtq = reinterpret_cast<uint16_t*>(base);
  float* npart = reinterpret_cast<float*>(base + route_mfma_scratch_offsets(d, 1));
  const int nhist = ((T + kDispatchBlock - 1) / kDispatchBlock) * E;
  hipLaunchKernelGGL(k_router_prep, dim3(E / 16, (D + 255) / 256), dim3(256), 0, st, D, E,
                     reinterpret_cast<const uint16_t*>(r.values), rtq, npart, hist, nhist);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  // the error bound's constant, relative to ||x|| ||r_e||: the MFMA sums as up
  // to 2D roundings of up to 2u, the canonical chains and tree, the norms and
  // lo / hi, with room to spare
  const float cb = (float)std::ldexp(4.0 * D + 512.0, -24);
  const uint16_t* xb = reinterpret_cast<const uint16_t*>(x);
  if (E <= 64)
    route_mfma_p<1>(d, xb, rtq, npart, cb, topk_idx, topk_w, hist, st);
  else if (E <= 128)
    route_mfma_p<2>(d, xb, rtq, npart, cb, topk_idx, topk_w, hist, st);
  else
    route_mfma_p<4>(d, xb, rtq, npart, cb, topk_idx, topk_w, hist, st);
  return hipGetLastError();
}

}  // namespace kmoe_host
