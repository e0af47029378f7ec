// Routing device code shared by the router kernels and the fused decode
// kernels: the top-k of one token by one wave, the finish of a token from the
// split router's group partials, and the dispatch sort of a chunk of tokens.
#pragma once

#include <hip/hip_runtime.h>

#include "common.h"

namespace kmoe {

// Top-k of one token held by a wave (value descending, ties to the lower
// expert index, as jax.lax.top_k), then w_j = expf(l_j - l_0) / sum_{i<K}
// expf(l_i - l_0) (sum in j order). Lane owns experts lane + 64*i, i < EPL;
// v[i] is the logit, -inf for NaN; entries past E are ignored.
//
// A radix select over order-preserving 32-bit keys (one ballot per bit and
// experts-per-lane) finds the K-th largest key; the selected experts (keys
// above it, then the lowest-index ties at it) are compacted into per-wave
// LDS, each of the first K lanes ranks one of them against the others, and
// the sorted list gives the outputs. -0.0 is keyed as +0.0 (they compare
// equal). No wave-wide shuffles: ballots and scalar popcounts only.
struct TopkLds {
  uint32_t key[kMaxTopK];
  int32_t idx[kMaxTopK];
  float val[kMaxTopK];
  int32_t sidx[kMaxTopK];
};

template <int EPL>
__device__ __forceinline__ void wave_topk(int t, int E, int K, const float* v, int32_t* __restrict__ topk_idx,
                                          float* __restrict__ topk_w, int out_bf16, int32_t* idx_lds, TopkLds& S) {
  const int lane = threadIdx.x & 63;
  const unsigned long long below = (1ull << lane) - 1ull;
  uint32_t key[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const float f = v[i] == 0.0f ? 0.0f : v[i];
    const uint32_t u = __float_as_uint(f);
    key[i] = (lane + 64 * i < E) ? ((u >> 31) ? ~u : (u | 0x80000000u)) : 0u;
  }
  uint32_t thr = 0;
  for (int b = 31; b >= 0; --b) {
    const uint32_t cand = thr | (1u << b);
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < EPL; ++i) cnt += __popcll(__ballot(key[i] >= cand));
    if (cnt >= K) thr = cand;
  }
  int gt = 0;
#pragma unroll
  for (int i = 0; i < EPL; ++i) gt += __popcll(__ballot(key[i] > thr));
  const int need = K - gt;
  int base_sel = 0, base_tie = 0;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const bool tie = key[i] == thr;
    const unsigned long long mt = __ballot(tie);
    const bool sel = key[i] > thr || (tie && base_tie + __popcll(mt & below) < need);
    const unsigned long long ms = __ballot(sel);
    if (sel) {
      const int pos = base_sel + __popcll(ms & below);
      S.key[pos] = key[i];
      S.idx[pos] = lane + 64 * i;
      S.val[pos] = v[i];
    }
    base_sel += __popcll(ms);
    base_tie += __popcll(mt);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float my_v = 0.0f;
  int my_i = 0, rank = 0;
  if (lane < K) {
    const uint32_t kj = S.key[lane];
    my_i = S.idx[lane];
    my_v = S.val[lane];
    for (int m = 0; m < K; ++m) {
      const uint32_t km = S.key[m];
      rank += (km > kj) || (km == kj && S.idx[m] < my_i);
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (lane < K) {
    S.sidx[rank] = my_i;
    S.key[rank] = __float_as_uint(my_v);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (lane < K) {
    const float l0 = __uint_as_float(S.key[0]);
    float ssum = 0.0f;
    for (int j = 0; j < K; ++j) ssum = ssum + expf(__uint_as_float(S.key[j]) - l0);
    const float p = expf(__uint_as_float(S.key[lane]) - l0) / ssum;
    const int e = S.sidx[lane];
    topk_w[(int64_t)t * K + lane] = out_bf16 ? round_bf16(p) : p;
    topk_idx[(int64_t)t * K + lane] = e;
    if (idx_lds) idx_lds[t * K + lane] = e;
  }
  // the LDS scratch is reused by this wave's next token
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Finish of token t by one wave: the remaining tree levels and the top-k;
// idx_lds (may be NULL) also receives the selections.
template <int EPL>
__device__ __forceinline__ void finish_token(int t, int E, int K, int Q, const float* __restrict__ part,
                                             float* __restrict__ logits, int32_t* __restrict__ topk_idx,
                                             float* __restrict__ topk_w, int out_bf16, int32_t* idx_lds,
                                             TopkLds& tk) {
  const int lane = threadIdx.x & 63;
  const float* const pt = part + (int64_t)t * Q * E;  // [Q][E] partials of token t
  float v[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane + 64 * i;
    float p[kMaxRouterSlices / 4];
    const float* pq = pt + e;
#pragma unroll
    for (int q = 0; q < kMaxRouterSlices / 4; ++q, pq += E) p[q] = (q < Q && e < E) ? *pq : 0.0f;
#pragma unroll
    for (int st = 1; st < kMaxRouterSlices / 4; st <<= 1)
      if (st < Q)
#pragma unroll
        for (int q = 0; q + st < kMaxRouterSlices / 4; q += 2 * st) p[q] = p[q] + p[q + st];
    const float l = p[0];
    v[i] = (e < E && l == l) ? l : -INFINITY;
    if (logits && e < E) logits[(int64_t)t * E + e] = l;
  }
  wave_topk<EPL>(t, E, K, v, topk_idx, topk_w, out_bf16, idx_lds, tk);
}

// ---------------------------------------------------------------------------
// Dispatch: stable counting sort of the row-major (t, j) assignments by expert
// (jnp.argsort(stable=True) over the flattened top-k indices).
//
// Tokens are cut into chunks of 64. Within a chunk, the assignments of expert
// e form a 64-bit token mask (a token picks an expert at most once), so the
// stable rank of token tl among them is popcount(mask[e] & ((1 << tl) - 1)).
// The position of an assignment is
//   offsets[e] + (assignments of e in earlier chunks) + rank,
// with the per-chunk counts from k_dispatch_count.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void chunk_masks(int T, int E, int K, int b, const int32_t* __restrict__ topk_idx,
                                            unsigned long long* mask) {
  for (int e = threadIdx.x; e < E; e += blockDim.x) mask[e] = 0ull;
  __syncthreads();
  const int t0 = b * kDispatchBlock;
  const int n = min(kDispatchBlock, T - t0) * K;
  for (int m = threadIdx.x; m < n; m += blockDim.x) {
    const int tl = m / K;
    const int e = topk_idx[(int64_t)t0 * K + m];
    if ((unsigned)e < (unsigned)E) atomicOr(&mask[e], 1ull << tl);
  }
  __syncthreads();
}

// The scatter for token chunk b. hist == nullptr: the counts come from this
// chunk's masks (valid when T <= 64). idx may point to global memory or LDS.
// An assignment whose slot within its expert (sorted position - the expert's
// offset) is >= cap is dropped: inv = -1 (fixed_capacity).
// Threads 0..255 do the work (blockDim.x >= 256, a multiple of 64); every
// thread of the block must call it.
struct DispatchLds {
  unsigned long long mask[kMaxExperts];
  int base[kMaxExperts];
  int start[kMaxExperts];
  int wsum[4], wact[4];
  int red_tot[4 * 256], red_bef[4 * 256];
};

static __device__ void dispatch_chunk(int T, int E, int K, int b, int nblk, const int32_t* idx,
                               const int32_t* __restrict__ hist, int32_t* __restrict__ group_sizes,
                               int32_t* __restrict__ offsets, int32_t* __restrict__ active,
                               int32_t* __restrict__ sorted_token, int32_t* __restrict__ sorted_expert,
                               int32_t* __restrict__ inv, int cap, DispatchLds& L) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const bool wk = tid < 256;
  chunk_masks(T, E, K, b, idx, L.mask);

  // this thread's experts: 4*tid .. 4*tid+3
  int tot[4], bef[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    tot[i] = 0;
    bef[i] = 0;
  }
  if (hist) {
    // Chunk totals: the Q = ceil(E/4) expert quads are summed over the chunks
    // by G = 256/Q thread groups (group g takes chunks g, g+G, ...), then the
    // quad owner adds the groups' partials from LDS. Integer sums: any order.
    const int Q = (E + 3) >> 2, G = 256 / Q;
    const int q = tid % Q, gi = tid / Q;
    int pt[4] = {0, 0, 0, 0}, pb[4] = {0, 0, 0, 0};
    if (wk && gi < G) {
      const bool vec4 = (E & 3) == 0;
#pragma unroll 4
      for (int bb = gi; bb < nblk; bb += G) {
        const int32_t* hp = hist + (int64_t)bb * E + 4 * q;
        int h[4];
        if (vec4) {
          const int4 v = *reinterpret_cast<const int4*>(hp);
          h[0] = v.x, h[1] = v.y, h[2] = v.z, h[3] = v.w;
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) h[i] = 4 * q + i < E ? hp[i] : 0;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pt[i] += h[i];
          pb[i] += bb < b ? h[i] : 0;
        }
      }
    }
    if (wk) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        L.red_tot[i * 256 + tid] = pt[i];
        L.red_bef[i * 256 + tid] = pb[i];
      }
    }
    __syncthreads();
    if (tid < Q) {
      for (int g = 0; g < G; ++g) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          tot[i] += L.red_tot[i * 256 + g * Q + tid];
          bef[i] += L.red_bef[i * 256 + g * Q + tid];
        }
      }
    }
  } else if (wk) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (4 * tid + i < E) tot[i] = __popcll(L.mask[4 * tid + i]);
  }
  int lsum = 0, lact = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (4 * tid + i >= E) tot[i] = bef[i] = 0;
    lsum += tot[i];
    lact += tot[i] > 0;
  }
  int isum = lsum, iact = lact;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int vs = __shfl_up(isum, off, 64);
    const int va = __shfl_up(iact, off, 64);
    if (lane >= off) {
      isum += vs;
      iact += va;
    }
  }
  if (wk && lane == 63) {
    L.wsum[wv] = isum;
    L.wact[wv] = iact;
  }
  __syncthreads();
  if (wk) {
    int run = isum - lsum, arun = iact - lact;
    for (int q = 0; q < wv; ++q) {
      run += L.wsum[q];
      arun += L.wact[q];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = 4 * tid + i;
      if (e < E) {
        if (b == 0) {
          group_sizes[e] = tot[i];
          offsets[e] = run;
          if (tot[i] > 0) active[arun] = e;
        }
        L.base[e] = run + bef[i];
        L.start[e] = run;
      }
      run += tot[i];
      arun += tot[i] > 0;
    }
    if (b == 0 && tid == 255) {
      offsets[E] = run;
      active[E] = arun;
    }
  }
  __syncthreads();

  const int t0 = b * kDispatchBlock;
  const int n = min(kDispatchBlock, T - t0) * K;
  const int M = T * K;
  for (int m = tid; m < n; m += blockDim.x) {
    const int tl = m / K;
    const int e = idx[(int64_t)t0 * K + m];
    // indices outside [0, E) or counts that disagree with them are caller errors
    // of the stage entry point; they are skipped rather than written out of bounds
    if ((unsigned)e < (unsigned)E) {
      const int p = L.base[e] + __popcll(L.mask[e] & ((1ull << tl) - 1ull));
      if ((unsigned)p < (unsigned)M) {
        sorted_token[p] = t0 + tl;
        sorted_expert[p] = e;
        inv[(int64_t)t0 * K + m] = p - L.start[e] < cap ? p : -1;
      }
    }
  }
}

// The same dispatch by one wave with no barrier, for a call with at most 8
// assignments (one token) and 256 experts (every thread may call it; wave 0
// works). sel holds the T*K row-major selections (LDS or global, read by all
// lanes at once). Assignment m = lane: its position is the number of
// assignments with a smaller expert plus the earlier ones with the same expert
// (the stable sort); an expert's count and offset come from one pass over the
// selections. It is correct up to 64 assignments, but its serial passes cost
// more than dispatch_chunk's barriers from 16 assignments on (T=1 decode
// layer 24.4 -> 23.7 us; T=4 and T=8 2 and 5 us slower).
__device__ __forceinline__ bool dispatch_fits_wave(int M, int E) { return M <= 8 && E <= 256; }

static __device__ void dispatch_wave(int T, int E, int K, const int32_t* sel, int32_t* __restrict__ group_sizes,
                                     int32_t* __restrict__ offsets, int32_t* __restrict__ active,
                                     int32_t* __restrict__ sorted_token, int32_t* __restrict__ sorted_expert,
                                     int32_t* __restrict__ inv, int cap) {
  if ((threadIdx.x >> 6) != 0) return;
  const int lane = threadIdx.x & 63;
  const int M = T * K;
  const int em = lane < M ? sel[lane] : -1;
  int below = 0, before = 0;
  for (int i = 0; i < M; ++i) {
    const int ei = sel[i];
    below += ei < em;
    before += ei == em && i < lane;
  }
  // an assignment that is its expert's first: its index among the active experts
  const bool first = lane < M && before == 0;
  const unsigned long long firsts = __ballot(first);
  int rank = 0;
  for (int i = 0; i < M; ++i)
    if ((firsts >> i) & 1ull) rank += sel[i] < em;
  if (lane < M) {
    const int p = below + before;
    sorted_token[p] = lane / K;
    sorted_expert[p] = em;
    inv[lane] = before < cap ? p : -1;
    if (first) active[rank] = em;
  }
  for (int e = lane; e < E; e += 64) {
    int cnt = 0, less = 0;
    for (int i = 0; i < M; ++i) {
      const int ei = sel[i];
      cnt += ei == e;
      less += ei < e;
    }
    group_sizes[e] = cnt;
    offsets[e] = less;
  }
  if (lane == 0) {
    offsets[E] = M;
    active[E] = __popcll(firsts);
  }
}

}  // namespace kmoe
