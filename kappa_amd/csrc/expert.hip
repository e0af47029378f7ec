// SwiGLU experts over the dispatch-sorted rows, and the weighted combine.
//
// Reference: the rounding points of the array program that runs
// (_moe_gather_einsum kappa/qwen3/ffn_moe.py:74-104 and _moe_fixed_capacity
// :107-158 on the kChainAct chain, _moe_ragged :174-216 on the kChainF32
// chain), in the grouped form of _moe_ragged: every expert's weights are read
// once per row tile instead of once per assignment.
//
// Packed int8 experts (bf16 activations) run on bf16 MFMA
// (v_mfma_f32_16x16x32_bf16); int8 is converted in registers right after a
// coalesced 16-byte load, to bf16(q * bf16(scale)) for kChainAct and to the
// exact integers for kChainF32, whose f32 per-column scale multiplies the f32
// sum in the epilogue (q * s summed over k equals s * sum(q) up to f32
// rounding, since the scale is constant along the reduction). The MFMA k order
// inside a 64-wide chunk is permuted: lane l supplies k = 16*(l/16) + 8*s + 0..7
// in sub-step s, for both operands, which matches the packed layout
// [.., k/16, col, 16 k] where each lane's 16 bytes are one column's 16 k.
#include <algorithm>
#include <atomic>

#include "common.h"
#include "launch.h"
#include "route_dev.h"

namespace kmoe {

// ---------------------------------------------------------------------------
// helpers
// ---------------------------------------------------------------------------
// two floats -> one dword of bf16 (RNE), a in the low half: one v_cvt_pk_bf16_f32
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
}

// 16 int8 -> bf16(q * s) (s already rounded to bf16), one packed pair at a time.
// Each byte is biased to u = q + 128 (one XOR per four bytes) and converted by
// v_cvt_f32_ubyteN; fma(u, s, -128 s) is then q * s exactly (both terms are
// exact and q * s has at most 16 significant bits), so the only rounding is the
// bf16 conversion: two instructions and a half per weight.
__device__ __forceinline__ void dequant16(const uint4 q, const float s, bf16x8& lo, bf16x8& hi) {
  const uint32_t w[4] = {q.x ^ 0x80808080u, q.y ^ 0x80808080u, q.z ^ 0x80808080u, q.w ^ 0x80808080u};
  const float nb = -128.0f * s;
  uint32_t o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t v = w[j >> 1];
    const int sh = 16 * (j & 1);
    const float a = (float)((v >> sh) & 0xffu);
    const float b = (float)((v >> (sh + 8)) & 0xffu);
    o[j] = pack_bf16x2(__builtin_fmaf(a, s, nb), __builtin_fmaf(b, s, nb));
  }
  lo = __builtin_bit_cast(bf16x8, uint4{o[0], o[1], o[2], o[3]});
  hi = __builtin_bit_cast(bf16x8, uint4{o[4], o[5], o[6], o[7]});
}

// 16 int8 -> the same 16 integers in bf16 (exact: |q| <= 128 needs 8 bits), for the
// f32 chain, which applies its f32 scale to the sum
__device__ __forceinline__ void cvt16(const uint4 q, bf16x8& lo, bf16x8& hi) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
  uint32_t o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t v = w[j >> 1];
    const int sh = 16 * (j & 1);
    o[j] = pack_bf16x2((float)(int8_t)((v >> sh) & 0xffu), (float)(int8_t)((v >> (sh + 8)) & 0xffu));
  }
  lo = __builtin_bit_cast(bf16x8, uint4{o[0], o[1], o[2], o[3]});
  hi = __builtin_bit_cast(bf16x8, uint4{o[4], o[5], o[6], o[7]});
}

// The B operand of a 16-byte int8 load for chain CH: bf16(q * s) with s already
// rounded to bf16 (kChainAct), or the exact integers (kChainF32).
template <int CH>
__device__ __forceinline__ void weights16(const uint4 q, const float s, bf16x8& lo, bf16x8& hi) {
  if (CH == kChainAct)
    dequant16(q, s, lo, hi);
  else
    cvt16(q, lo, hi);
}

// The packed scales are stored as given (f32); kChainAct casts them to bf16
// first (kappa/qwen3/quant.py:37, 74).
template <int CH>
__device__ __forceinline__ float chain_scale(float s) {
  return CH == kChainAct ? round_bf16(s) : s;
}

__device__ __forceinline__ bf16x8 as_bf16x8(const uint4 v) { return __builtin_bit_cast(bf16x8, v); }

// 16 bytes with a nontemporal load: for data a kernel reads exactly once, such
// as the decode weights (streaming reads this way sustain ~7.1 TB/s on MI355X
// against ~6.3 TB/s for ordinary loads, which also allocate in the caches)
__device__ __forceinline__ uint4 load_stream16(const int8_t* p) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return uint4{v.x, v.y, v.z, v.w};
}

__device__ __forceinline__ floatx4 mfma16(const bf16x8 a, const bf16x8 b, const floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Block-wide tile prefix over experts: mtp[e] = sum_{e' < e} ceil(min(group_size[e'], cap) / BM), mtp[E] = total.
// The first 256 threads compute it (E <= 1024); blockDim.x must be a multiple of 64, at least 256.
// wsum: 4 ints of LDS scratch. offs (optional, E + 1 ints of LDS): a copy of offsets, so
// the caller's later lookups of its expert's row range are LDS reads, not another global
// round trip.
template <int BM>
__device__ void tile_prefix(const int32_t* __restrict__ offsets, int E, int cap, int* mtp, int* wsum,
                            int* offs = nullptr) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  int c[4];
  int local = 0, incl = 0;
  if (tid < 256) {
    // offsets[4 tid .. 4 tid + 4], clamped to the array: five loads in flight
    // together (guarded loads would each wait a round trip of their own)
    int o[5];
#pragma unroll
    for (int i = 0; i < 5; ++i) o[i] = offsets[min(tid * 4 + i, E)];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid * 4 + i;
      c[i] = e < E ? (min(o[i + 1] - o[i], cap) + BM - 1) / BM : 0;
      if (offs != nullptr && e <= E) offs[e] = o[i];
      local += c[i];
    }
    if (offs != nullptr && tid * 4 + 4 == E) offs[E] = o[4];
    incl = local;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int v = __shfl_up(incl, off, 64);
      if (lane >= off) incl += v;
    }
    if (lane == 63) wsum[wv] = incl;
  }
  __syncthreads();
  if (tid < 256) {
    int base = 0;
    for (int w = 0; w < wv; ++w) base += wsum[w];
    int run = base + incl - local;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid * 4 + i;
      if (e < E) mtp[e] = run;
      run += c[i];
    }
    if (tid == 255) mtp[E] = base + incl;
  }
  __syncthreads();
}

// largest e in [0, E) with mtp[e] <= v (mtp non-decreasing, mtp[0] = 0)
__device__ __forceinline__ int tile_expert(const int* mtp, int E, int v) {
  int lo = 0, hi = E - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (mtp[mid] <= v)
      lo = mid;
    else
      hi = mid - 1;
  }
  return lo;
}

// ---------------------------------------------------------------------------
// Decode (T <= 64): one block per (active expert, 16-column group); the WPB
// waves split the reduction axis. The reduction is cut into eight fixed parts
// (chunks [KC*k/8, KC*(k+1)/8), one MFMA chain each) summed as
// (((p0 + p1) + (p2 + p3)) + (p4 + p5)) + (p6 + p7) whatever the wave count
// (eight waves: one part each; four: two parts each, added in the wave), so
// every shape of this kernel - and with it a token's h - is the same for any
// batch of up to 128 tokens.
// Each weight byte is read exactly once per call. A wave issues the weight
// loads of a batch of NB 64-deep chunks (NB x 1 KB per operand in flight)
// before anything else - they depend only on the expert - then finds its rows
// and loads the activation fragments, dequantises and runs the MFMAs; the raw
// int8 stays in registers across 16-row blocks. GUARD handles a chunk count
// per wave that NB does not divide.
//
// DENSE (T <= 16): the 16-row tile is the T tokens themselves, in token
// order, instead of the expert's gathered rows; it pays while T is small,
// since every block reads all T activation rows. A row's products do not
// depend on the other rows of the tile, so each stored row is the value the
// gathered tile gives; only the rows of the tokens routed to the expert are
// stored. The first load batch's activation fragments depend on nothing and
// are issued first, ahead of the expert lookup; later batches load theirs in
// the loop.
// ---------------------------------------------------------------------------
template <int WPB, int NB, bool GUARD, int MRB, bool DENSE, bool ALLROWS, int CH>
__device__ __forceinline__ void gateup_decode_body(int ig, int slot, int rg, int T, int D, int I, int E,
                                                   const uint16_t* __restrict__ x,
                                                   const int32_t* __restrict__ offsets,
                                                   const int32_t* __restrict__ active,
                                                   const int32_t* __restrict__ sorted_token,
                                                   const int8_t* __restrict__ w13, const float* __restrict__ s13,
                                                   uint16_t* __restrict__ h_sorted, int cap) {
  static_assert(!DENSE || (MRB == 1 && !GUARD), "dense tiles: one row block, whole load batches");
  static_assert(!ALLROWS || (!DENSE && !GUARD), "row groups: gathered rows, one batch per wave");
  static_assert(WPB == 8 || WPB == 4, "eight reduction parts over eight or four waves");
  constexpr int PPW = 8 / WPB;  // reduction parts per wave
  const int pslot = (threadIdx.x >> 6) == 0 ? WPB - 1 : (threadIdx.x >> 6) - 1;
  // red[w - 1]: wave w's sum for the cross-wave reduction; with two parts per
  // wave, slot pslot also holds the wave's first part while it runs the second
  __shared__ floatx4 red[8 / WPB == 2 ? WPB : WPB - 1][MRB][2][64];
  __shared__ int srt[16];  // DENSE: the tokens of the expert's rows
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int IG = I >> 4, KC = D >> 6;
  const int c0 = (KC * wv) / WPB, c1 = (KC * (wv + 1)) / WPB;
  const int csplit = (KC * (PPW * wv + 1)) / 8;  // PPW = 2: the wave's second part starts here
  const int koff = 16 * (lane >> 4);
  uint4 da0[DENSE ? NB : 1], da1[DENSE ? NB : 1];
  if (DENSE) {
    const int t = lane & 15;
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      da0[i] = uint4{0, 0, 0, 0};
      da1[i] = uint4{0, 0, 0, 0};
      if (t < T) {
        const uint4* ap = reinterpret_cast<const uint4*>(x + (size_t)t * D + koff + (c0 + i) * 64);
        da0[i] = ap[0];
        da1[i] = ap[1];
      }
    }
  }
  const int n_active = active[E];
  const int e = active[slot < E ? slot : 0];
  if (slot >= n_active) return;
  // row group rg > 0 (rows from 16 * MRB * rg on): nothing to do, and no load
  // issued, when the expert has fewer rows
  if (rg > 0 && 16 * MRB * rg >= min(offsets[e + 1] - offsets[e], cap)) return;
  const size_t cell = (size_t)(D >> 4) * 256;
  const int8_t* bg = w13 + (((size_t)e * IG + ig) * 2 + 0) * cell + lane * 16;
  const int8_t* bu = bg + cell;
  uint4 qg[NB], qu[NB];
  auto load_w = [&](int cb) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      if (!GUARD || cb + i < c1) {
        qg[i] = load_stream16(bg + (size_t)(cb + i) * 1024);
        qu[i] = load_stream16(bu + (size_t)(cb + i) * 1024);
      }
    }
  };
  load_w(c0);
  const float sg = chain_scale<CH>(s13[(((size_t)e * IG + ig) * 2 + 0) * 16 + (lane & 15)]);
  const float su = chain_scale<CH>(s13[(((size_t)e * IG + ig) * 2 + 1) * 16 + (lane & 15)]);
  const int r0 = offsets[e];
  const int nrows = min(offsets[e + 1] - r0, cap);
  if (DENSE && wv == 0 && lane < nrows) srt[lane] = sorted_token[r0 + lane];
  // ALLROWS: the expert's rows in groups of MRB 16-row blocks, the weights of
  // the wave's single load batch kept in registers across the groups
  const int ngroups = ALLROWS ? (nrows + 16 * MRB - 1) / (16 * MRB) : 1;
  for (int grp = 0; grp < ngroups; ++grp) {
    const int rbase = (rg + grp) * 16 * MRB;
    const int nrb = DENSE ? 1 : min((nrows - rbase + 15) >> 4, MRB);
    const uint16_t* xr[MRB];
    if (!DENSE) {
#pragma unroll
      for (int rb = 0; rb < MRB; ++rb) {
        const int row = rbase + rb * 16 + (lane & 15);
        const int tok = sorted_token[r0 + min(row, nrows - 1)];
        xr[rb] = row < nrows ? x + (size_t)tok * D + koff : nullptr;
      }
    }
    // ag/au: the current reduction part; with two parts per wave (PPW = 2) the
    // first is set aside in the wave's LDS slot when the second starts and
    // added to it at the end, p(2w) + p(2w+1)
    floatx4 ag[MRB], au[MRB];
#pragma unroll
    for (int rb = 0; rb < MRB; ++rb) {
      ag[rb] = floatx4{0.f, 0.f, 0.f, 0.f};
      au[rb] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
    bool parked = false;  // a first part is in the slot (wave-uniform)
    auto set_aside = [&](int rb) {
      parked = true;
      red[pslot][rb][0][lane] = ag[rb];
      red[pslot][rb][1][lane] = au[rb];
      ag[rb] = floatx4{0.f, 0.f, 0.f, 0.f};
      au[rb] = floatx4{0.f, 0.f, 0.f, 0.f};
    };
    auto next_part = [&]() {
#pragma unroll
      for (int rb = 0; rb < MRB; ++rb)
        if (rb < nrb) set_aside(rb);
    };
    // Two parts start on load-batch boundaries when NB divides KC / 8 (D = 2048,
    // 4096), or (a row-group kernel's single batch) in its middle.
    constexpr bool SPLIT_IN_BATCH = ALLROWS && PPW == 2;
    for (int cb = c0; cb < c1; cb += NB) {
      if (cb != c0) load_w(cb);
      if (PPW == 2 && !SPLIT_IN_BATCH && cb == csplit) next_part();
#pragma unroll
      for (int rb = 0; rb < MRB; ++rb) {
        if (rb < nrb) {
          uint4 a0[NB], a1[NB];
#pragma unroll
          for (int i = 0; i < NB; ++i) {
            if (DENSE) {
              if (cb == c0) {
                a0[i] = da0[i];
                a1[i] = da1[i];
              } else {
                // a later batch: the T token rows at its chunks
                const int t = lane & 15;
                a0[i] = uint4{0, 0, 0, 0};
                a1[i] = uint4{0, 0, 0, 0};
                if (t < T) {
                  const uint4* ap = reinterpret_cast<const uint4*>(x + (size_t)t * D + koff + (cb + i) * 64);
                  a0[i] = ap[0];
                  a1[i] = ap[1];
                }
              }
              continue;
            }
            a0[i] = uint4{0, 0, 0, 0};
            a1[i] = uint4{0, 0, 0, 0};
            if (xr[rb] && (!GUARD || cb + i < c1)) {
              const uint4* ap = reinterpret_cast<const uint4*>(xr[rb] + (cb + i) * 64);
              a0[i] = ap[0];
              a1[i] = ap[1];
            }
          }
#pragma unroll
          for (int i = 0; i < NB; ++i) {
            if (SPLIT_IN_BATCH && i == NB / 2) set_aside(rb);
            if (!GUARD || cb + i < c1) {
              bf16x8 bg0, bg1, bu0, bu1;
              weights16<CH>(qg[i], sg, bg0, bg1);
              weights16<CH>(qu[i], su, bu0, bu1);
              ag[rb] = mfma16(as_bf16x8(a0[i]), bg0, ag[rb]);
              ag[rb] = mfma16(as_bf16x8(a1[i]), bg1, ag[rb]);
              au[rb] = mfma16(as_bf16x8(a0[i]), bu0, au[rb]);
              au[rb] = mfma16(as_bf16x8(a1[i]), bu1, au[rb]);
            }
          }
        }
      }
    }
    // PPW = 2: the wave's pair sum p(2w) + p(2w+1) (its own slot, read back by
    // the lanes that wrote it)
    if (PPW == 2 && parked) {
#pragma unroll
      for (int rb = 0; rb < MRB; ++rb) {
        if (rb < nrb) {
          ag[rb] = red[pslot][rb][0][lane] + ag[rb];
          au[rb] = red[pslot][rb][1][lane] + au[rb];
        }
      }
    }
    if (wv > 0) {
#pragma unroll
      for (int rb = 0; rb < MRB; ++rb) {
        if (rb < nrb) {
          red[wv - 1][rb][0][lane] = ag[rb];
          red[wv - 1][rb][1][lane] = au[rb];
        }
      }
    }
    __syncthreads();
    if (wv == 0) {
#pragma unroll
      for (int rb = 0; rb < MRB; ++rb) {
        if (rb >= nrb) break;
        floatx4 g = ag[rb], u = au[rb];
        if (PPW == 1) {
          // (((p0 + p1) + (p2 + p3)) + (p4 + p5)) + (p6 + p7), red[w - 1] = p(w)
          g += red[0][rb][0][lane];
          u += red[0][rb][1][lane];
#pragma unroll
          for (int w = 1; w < WPB - 1; w += 2) {
            g += red[w][rb][0][lane] + red[w + 1][rb][0][lane];
            u += red[w][rb][1][lane] + red[w + 1][rb][1][lane];
          }
        } else {
          // ((q0 + q1) + q2) + q3 with q(w) = p(2w) + p(2w+1), red[w - 1] = q(w)
#pragma unroll
          for (int w = 0; w < WPB - 1; ++w) {
            g += red[w][rb][0][lane];
            u += red[w][rb][1][lane];
          }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int row = rbase + rb * 16 + 4 * (lane >> 4) + j;
          // DENSE: tile row = token; find its position among the expert's rows
          int pos = row < nrows ? r0 + row : -1;
          if (DENSE) {
            pos = -1;
            for (int r = 0; r < nrows; ++r)
              if (srt[r] == row) pos = r0 + r;
          }
          if (pos >= 0) {
            if (CH == kChainAct) {
              const float gv = round_bf16(g[j]), uv = round_bf16(u[j]);
              h_sorted[(size_t)pos * I + ig * 16 + (lane & 15)] = f32_to_bf16_bits(swiglu<true>(gv, uv));
            } else {
              // f32 g, u, h; h as its hi and lo planes (row stride 2I)
              const float hv = swiglu<false>(__fmul_rn(g[j], sg), __fmul_rn(u[j], su));
              uint16_t hi, lo;
              split_bf16(hv, hi, lo);
              uint16_t* hr = h_sorted + (size_t)pos * 2 * I + ig * 16 + (lane & 15);
              hr[0] = hi;
              hr[I] = lo;
            }
          }
        }
      }
    }
    // the reduction stage is reused by the next group
    if (ALLROWS) __syncthreads();
  }
}

template <int WPB, int NB, bool GUARD, int MRB, bool DENSE, bool ALLROWS, int CH>
__global__ __launch_bounds__(512) void k_gateup_decode(int T, int D, int I, int E, const uint16_t* __restrict__ x,
                                                        const int32_t* __restrict__ offsets,
                                                        const int32_t* __restrict__ active,
                                                        const int32_t* __restrict__ sorted_token,
                                                        const int8_t* __restrict__ w13, const float* __restrict__ s13,
                                                        uint16_t* __restrict__ h_sorted, int cap) {
  gateup_decode_body<WPB, NB, GUARD, MRB, DENSE, ALLROWS, CH>(blockIdx.x, blockIdx.y, blockIdx.z, T, D, I, E, x,
                                                              offsets, active, sorted_token, w13, s13, h_sorted, cap);
}

// Decode with at most four tokens, whole-block call: the router's finish and
// the dispatch sort run at the start of every gate/up block (each block
// finishes the T tokens from the split router's group partials and sorts
// their assignments into LDS, all blocks alike), so no kernel sits between
// the router's slices and the expert products. Block 0 also writes the
// selections, weights and dispatch arrays for the down + combine kernel.
// The grid is at most one resident round of blocks; each block then runs the
// (16-column group, active expert) items blockIdx.x, + gridDim.x, ..., so the
// routing is paid once per block. The products are those of
// k_gateup_decode's dense form.
template <int EPL, int NB, int CH>
__global__ __launch_bounds__(512) void k_gateup_routed(int T, int D, int I, int E, int K, int Q,
                                                        const float* __restrict__ part, int out_bf16,
                                                        const uint16_t* __restrict__ x,
                                                        const int8_t* __restrict__ w13, const float* __restrict__ s13,
                                                        uint16_t* __restrict__ h_sorted, int cap,
                                                        int32_t* __restrict__ topk_idx, float* __restrict__ topk_w,
                                                        int32_t* __restrict__ group_sizes, int32_t* __restrict__ offsets,
                                                        int32_t* __restrict__ active,
                                                        int32_t* __restrict__ sorted_token,
                                                        int32_t* __restrict__ sorted_expert,
                                                        int32_t* __restrict__ inv) {
  constexpr int MT = 4 * kMaxTopK;  // T <= 4
  __shared__ TopkLds tk[4];
  __shared__ DispatchLds L;
  __shared__ int32_t sel[MT], l_tidx[MT], l_stok[MT], l_sexp[MT], l_inv[MT];
  __shared__ float l_tw[MT];
  __shared__ int32_t l_gs[kMaxExperts], l_off[kMaxExperts + 1], l_act[kMaxExperts + 1];
  const int w = threadIdx.x >> 6;
  if (w < T) finish_token<EPL>(w, E, K, Q, part, nullptr, l_tidx, l_tw, out_bf16, sel, tk[w]);
  __syncthreads();
  if (dispatch_fits_wave(T * K, E))
    dispatch_wave(T, E, K, sel, l_gs, l_off, l_act, l_stok, l_sexp, l_inv, cap);
  else
    dispatch_chunk(T, E, K, 0, 1, sel, nullptr, l_gs, l_off, l_act, l_stok, l_sexp, l_inv, cap, L);
  __syncthreads();
  if (blockIdx.x == 0) {
    const int M = T * K;
    for (int i = threadIdx.x; i < M; i += blockDim.x) {
      topk_idx[i] = l_tidx[i];
      topk_w[i] = l_tw[i];
      sorted_token[i] = l_stok[i];
      sorted_expert[i] = l_sexp[i];
      inv[i] = l_inv[i];
    }
    for (int e = threadIdx.x; e <= E; e += blockDim.x) {
      offsets[e] = l_off[e];
      active[e] = l_act[e];
      if (e < E) group_sizes[e] = l_gs[e];
    }
  }
  const int IG = I >> 4;
  const int n_items = IG * l_act[E];
  for (int it = blockIdx.x; it < n_items; it += gridDim.x) {
    gateup_decode_body<8, NB, false, 1, true, false, CH>(it % IG, it / IG, 0, T, D, I, E, x, l_off, l_act, l_stok,
                                                         w13, s13, h_sorted, cap);
    // the body's LDS reduction stage is reused by the next item
    __syncthreads();
  }
}

// Down projection for decode: one block per (active expert, NCG*16 output
// columns), the reduction axis (I) split over the four waves; same load order
// as the gate/up kernel.
template <int WPB, int NCG, int NB, bool GUARD, bool ALLROWS, int CH>
__global__ __launch_bounds__(512) void k_down_decode(int D, int I, int E, const uint16_t* __restrict__ h_sorted,
                                                      const int32_t* __restrict__ offsets,
                                                      const int32_t* __restrict__ active,
                                                      const int8_t* __restrict__ w2, const float* __restrict__ s2,
                                                      uint16_t* __restrict__ y_sorted, int cap) {
  static_assert(!ALLROWS || !GUARD, "row groups: one batch per wave");
  // Rows per 16-row MFMA tile: 16, or 8 for kChainF32, whose tile rows 0..7 carry
  // the hi plane of 8 rows of h and tile rows 8..15 their lo plane; the two
  // halves of the product are added at the end. A decode expert has a few rows,
  // so the lo plane rides in tile rows that would otherwise be empty.
  constexpr int RPT = CH == kChainF32 ? 8 : 16;
  constexpr int RPG = RPT * kDecodeMaxRowBlocks;  // rows per group
  __shared__ floatx4 red[WPB > 1 ? WPB - 1 : 1][kDecodeMaxRowBlocks][NCG][64];
  const int dt = blockIdx.x;  // NCG*16 output columns
  const int slot = blockIdx.y;
  const int n_active = active[E];
  const int e = active[slot < E ? slot : 0];
  if (slot >= n_active) return;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int DG = D >> 4, KC = I >> 6;
  const size_t cell = (size_t)(I >> 4) * 256;
  const int8_t* bp = w2 + ((size_t)e * DG + dt * NCG) * cell + lane * 16;
  const int c0 = (KC * wv) / WPB, c1 = (KC * (wv + 1)) / WPB;
  uint4 q[NB][NCG];
  auto load_w = [&](int cb) {
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg)
        if (!GUARD || cb + i < c1) q[i][cg] = load_stream16(bp + cg * cell + (size_t)(cb + i) * 1024);
  };
  load_w(c0);
  float sc[NCG];
#pragma unroll
  for (int cg = 0; cg < NCG; ++cg) sc[cg] = chain_scale<CH>(s2[(size_t)e * D + (dt * NCG + cg) * 16 + (lane & 15)]);
  const int r0 = offsets[e];
  const int nrows = min(offsets[e + 1] - r0, cap);
  const int koff = 16 * (lane >> 4);
  // Groups of RPG rows: ALLROWS (one load batch per wave, kept in registers) and
  // kChainF32 (32 rows per group) loop over them; a wave with several load
  // batches loads its weights again for each group.
  const bool multi = c1 - c0 > NB;
  const int ngroups = (ALLROWS || CH == kChainF32) ? (nrows + RPG - 1) / RPG : 1;
  for (int grp = 0; grp < ngroups; ++grp) {
    const int rbase = grp * RPG;
    const int nrb = min((nrows - rbase + RPT - 1) / RPT, kDecodeMaxRowBlocks);
    const uint16_t* hr[kDecodeMaxRowBlocks];
#pragma unroll
    for (int rb = 0; rb < kDecodeMaxRowBlocks; ++rb) {
      if (CH == kChainF32) {
        const int row = rbase + rb * 8 + (lane & 7);
        hr[rb] = row < nrows ? h_sorted + (size_t)(r0 + row) * 2 * I + ((lane >> 3) & 1) * I + koff : nullptr;
      } else {
        const int row = rbase + rb * 16 + (lane & 15);
        hr[rb] = row < nrows ? h_sorted + (size_t)(r0 + row) * I + koff : nullptr;
      }
    }
    floatx4 acc[kDecodeMaxRowBlocks][NCG];
#pragma unroll
    for (int rb = 0; rb < kDecodeMaxRowBlocks; ++rb)
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) acc[rb][cg] = floatx4{0.f, 0.f, 0.f, 0.f};
    for (int cb = c0; cb < c1; cb += NB) {
      if (cb != c0 || (grp > 0 && multi)) load_w(cb);
#pragma unroll
      for (int rb = 0; rb < kDecodeMaxRowBlocks; ++rb) {
        if (rb < nrb) {
          uint4 a0[NB], a1[NB];
#pragma unroll
          for (int i = 0; i < NB; ++i) {
            a0[i] = uint4{0, 0, 0, 0};
            a1[i] = uint4{0, 0, 0, 0};
            if (hr[rb] && (!GUARD || cb + i < c1)) {
              const uint4* ap = reinterpret_cast<const uint4*>(hr[rb] + (cb + i) * 64);
              a0[i] = ap[0];
              a1[i] = ap[1];
            }
          }
#pragma unroll
          for (int i = 0; i < NB; ++i) {
            if (!GUARD || cb + i < c1) {
#pragma unroll
              for (int cg = 0; cg < NCG; ++cg) {
                bf16x8 b0, b1;
                weights16<CH>(q[i][cg], sc[cg], b0, b1);
                acc[rb][cg] = mfma16(as_bf16x8(a0[i]), b0, acc[rb][cg]);
                acc[rb][cg] = mfma16(as_bf16x8(a1[i]), b1, acc[rb][cg]);
              }
            }
          }
        }
      }
    }
    if (wv > 0) {
#pragma unroll
      for (int rb = 0; rb < kDecodeMaxRowBlocks; ++rb)
        if (rb < nrb)
#pragma unroll
          for (int cg = 0; cg < NCG; ++cg) red[wv - 1][rb][cg][lane] = acc[rb][cg];
    }
    __syncthreads();
    if (wv == 0) {
#pragma unroll
      for (int rb = 0; rb < kDecodeMaxRowBlocks; ++rb) {
        if (rb >= nrb) break;
#pragma unroll
        for (int cg = 0; cg < NCG; ++cg) {
          floatx4 v = acc[rb][cg];
#pragma unroll
          for (int w = 0; w < WPB - 1; ++w) v += red[w][rb][cg][lane];
          if (CH == kChainF32) {
            // tile row r (lanes 0..31) is the hi half of row r, tile row r + 8
            // (lanes 32..63) its lo half: y = (hi + lo) * s
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const float lo = __shfl_down(v[j], 32, 64);
              const int row = rbase + rb * 8 + 4 * (lane >> 4) + j;
              if (lane < 32 && row < nrows)
                y_sorted[(size_t)(r0 + row) * D + (dt * NCG + cg) * 16 + (lane & 15)] =
                    f32_to_bf16_bits(__fmul_rn(v[j] + lo, sc[cg]));
            }
          } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int row = rbase + rb * 16 + 4 * (lane >> 4) + j;
              if (row < nrows)
                y_sorted[(size_t)(r0 + row) * D + (dt * NCG + cg) * 16 + (lane & 15)] = f32_to_bf16_bits(v[j]);
            }
          }
        }
      }
    }
    // the reduction stage is reused by the next group
    if (ngroups > 1) __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Prefill: grouped GEMM over (expert, 128-row tile, column tile) work items.
// 4 waves as 2 (rows) x 2 (columns); each wave owns 64 rows. A (activation
// rows) and B (dequantised weights) are staged in double-buffered LDS in
// 64-deep k chunks; one barrier per chunk. Work items are laid out so that all
// column tiles of one (expert, row tile) run on the same XCD (its L2).
// ---------------------------------------------------------------------------
constexpr int kBM = 128;
constexpr int kAStride = 72;  // bf16 elements per LDS row (64 + 8 pad: conflict-free fragment reads)

struct PrefillLds {
  alignas(16) uint16_t a[2][kBM][kAStride];
  alignas(16) uint16_t b[2][2][8][64][8];  // [buf][sub-step][col group][lane][8 bf16]
  int mtp[kMaxExperts + 1];
  int tok[kBM];
  int wsum[4];
};

__device__ __forceinline__ bool prefill_tile(const int32_t* __restrict__ offsets, int E, int NT, int cap, PrefillLds& s,
                                             int& e, int& row0, int& rows, int& nt) {
  tile_prefix<kBM>(offsets, E, cap, s.mtp, s.wsum);
  const int ntiles = s.mtp[E] * NT;
  const int per = (ntiles + 7) >> 3;
  const int q = blockIdx.x >> 3;
  if (q >= per) return false;
  const int L = (blockIdx.x & 7) * per + q;
  if (L >= ntiles) return false;
  const int mt_glob = L / NT;
  nt = L - mt_glob * NT;
  e = tile_expert(s.mtp, E, mt_glob);
  const int mt = mt_glob - s.mtp[e];
  row0 = offsets[e] + mt * kBM;
  rows = min(kBM, offsets[e] + min(offsets[e + 1] - offsets[e], cap) - row0);
  return true;
}

// GATEUP = true: A rows gathered from x by token, B = gate|up column groups,
// epilogue SwiGLU -> h_sorted. GATEUP = false: A = h_sorted rows, B = down,
// epilogue -> y_sorted.
template <bool GATEUP, int CH>
__global__ __launch_bounds__(256, 2) void k_prefill(int D, int I, int E, const uint16_t* __restrict__ src,
                                                     const int32_t* __restrict__ offsets,
                                                     const int32_t* __restrict__ sorted_token,
                                                     const int8_t* __restrict__ wp, const float* __restrict__ sp,
                                                     uint16_t* __restrict__ dst, int cap) {
  __shared__ PrefillLds s;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  // kChainF32 down: the A rows are h's hi and lo planes (2I wide), both against the
  // same weight chunks
  const int Kdim = GATEUP ? D : (CH == kChainF32 ? 2 * I : I);
  const int KCW = (GATEUP ? D : I) >> 6;  // weight chunks along the reduction
  const int Ndim = GATEUP ? I : D;
  const int NT = GATEUP ? (I >> 6) : (D >> 7);
  int e, row0, rows, nt;
  if (!prefill_tile(offsets, E, NT, cap, s, e, row0, rows, nt)) return;
  if (tid < kBM) s.tok[tid] = (tid < rows) ? (GATEUP ? sorted_token[row0 + tid] : row0 + tid) : -1;
  __syncthreads();

  // global -> LDS mapping
  const int ar = tid >> 1, ah = tid & 1;
  const int arow = s.tok[ar];
  const uint16_t* ap = arow >= 0 ? src + (size_t)arow * Kdim + ah * 32 : nullptr;
  const int cg = tid >> 5;
  const int l0 = (tid & 31) << 1;
  const int8_t* bp;
  float sc0, sc1;
  if (GATEUP) {
    const int which = cg >> 2;
    const int igl = nt * 4 + (cg & 3);
    const size_t cid = ((size_t)e * (I >> 4) + igl) * 2 + which;
    bp = wp + cid * (size_t)(D >> 4) * 256;
    sc0 = chain_scale<CH>(sp[cid * 16 + (l0 & 15)]);
    sc1 = chain_scale<CH>(sp[cid * 16 + ((l0 + 1) & 15)]);
  } else {
    const int dg = nt * 8 + cg;
    bp = wp + ((size_t)e * (D >> 4) + dg) * (size_t)(I >> 4) * 256;
    sc0 = chain_scale<CH>(sp[(size_t)e * D + dg * 16 + (l0 & 15)]);
    sc1 = chain_scale<CH>(sp[(size_t)e * D + dg * 16 + ((l0 + 1) & 15)]);
  }

  uint4 ra[4], rq[2];
  auto gload = [&](int c) {
#pragma unroll
    for (int j = 0; j < 4; ++j) ra[j] = ap ? reinterpret_cast<const uint4*>(ap + c * 64)[j] : uint4{0, 0, 0, 0};
    const int cw = c % KCW;
    rq[0] = *reinterpret_cast<const uint4*>(bp + (size_t)cw * 1024 + l0 * 16);
    rq[1] = *reinterpret_cast<const uint4*>(bp + (size_t)cw * 1024 + (l0 + 1) * 16);
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<uint4*>(&s.a[buf][ar][ah * 32 + 8 * j]) = ra[j];
    bf16x8 lo, hi;
    weights16<CH>(rq[0], sc0, lo, hi);
    *reinterpret_cast<bf16x8*>(&s.b[buf][0][cg][l0][0]) = lo;
    *reinterpret_cast<bf16x8*>(&s.b[buf][1][cg][l0][0]) = hi;
    weights16<CH>(rq[1], sc1, lo, hi);
    *reinterpret_cast<bf16x8*>(&s.b[buf][0][cg][l0 + 1][0]) = lo;
    *reinterpret_cast<bf16x8*>(&s.b[buf][1][cg][l0 + 1][0]) = hi;
  };

  const int wm = wv & 1, wn = wv >> 1;
  // accumulators: GATEUP: [mi][ni 0..1][gate/up]; down: [mi][ni 0..3]
  floatx4 acc[4][4];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[mi][n] = floatx4{0.f, 0.f, 0.f, 0.f};
  // column groups of this wave, in acc order
  int wcg[4];
#pragma unroll
  for (int n = 0; n < 4; ++n) wcg[n] = GATEUP ? ((n & 1) ? 4 : 0) + wn * 2 + (n >> 1) : wn * 4 + n;
  int mlim = 0;
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
    if (wm * 64 + mi * 16 < rows) mlim = mi + 1;

  const int KC = Kdim >> 6;
  gload(0);
  lstore(0);
  __syncthreads();
  for (int c = 0; c < KC; ++c) {
    const int buf = c & 1;
    if (c + 1 < KC) gload(c + 1);
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      bf16x8 a[4], b[4];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
        a[mi] = *reinterpret_cast<const bf16x8*>(&s.a[buf][wm * 64 + mi * 16 + (lane & 15)][16 * (lane >> 4) + 8 * st]);
#pragma unroll
      for (int n = 0; n < 4; ++n) b[n] = *reinterpret_cast<const bf16x8*>(&s.b[buf][st][wcg[n]][lane][0]);
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
        if (mi < mlim) {
#pragma unroll
          for (int n = 0; n < 4; ++n) acc[mi][n] = mfma16(a[mi], b[n], acc[mi][n]);
        }
      }
    }
    if (c + 1 < KC) lstore(buf ^ 1);
    __syncthreads();
  }

  // epilogue: lane holds rows 4*(lane/16)+j of each 16x16 tile, column lane%16
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = wm * 64 + mi * 16 + 4 * (lane >> 4) + j;
      if (row >= rows) continue;
      uint16_t* drow = dst + (size_t)(row0 + row) * (GATEUP && CH == kChainF32 ? 2 * Ndim : Ndim);
      if (GATEUP) {
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
          const int col = nt * 64 + wn * 32 + ni * 16 + (lane & 15);
          if (CH == kChainAct) {
            const float g = round_bf16(acc[mi][2 * ni][j]);
            const float u = round_bf16(acc[mi][2 * ni + 1][j]);
            drow[col] = f32_to_bf16_bits(swiglu<true>(g, u));
          } else {
            const size_t cid = ((size_t)e * (I >> 4) + (col >> 4)) * 2;
            const float g = __fmul_rn(acc[mi][2 * ni][j], sp[cid * 16 + (lane & 15)]);
            const float u = __fmul_rn(acc[mi][2 * ni + 1][j], sp[(cid + 1) * 16 + (lane & 15)]);
            split_bf16(swiglu<false>(g, u), drow[col], drow[I + col]);
          }
        }
      } else {
#pragma unroll
        for (int n = 0; n < 4; ++n) {
          const int col = nt * 128 + wn * 64 + n * 16 + (lane & 15);
          drow[col] = f32_to_bf16_bits(CH == kChainF32 ? __fmul_rn(acc[mi][n][j], sp[(size_t)e * D + col]) : acc[mi][n][j]);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Prefill grouped GEMM over (expert, row tile, column tile) work items.
//
// A block of four waves computes up to 128 (or 160) rows x 256 B columns
// (gate/up: 128 gate + 128 up columns, i.e. 128 columns of h; down: 256 output
// columns); two blocks share a CU. Wave w owns the 16-column cells 4w .. 4w+3
// (gate/up: two gate cells and the matching two up cells, so the SwiGLU epilogue pairs
// registers of one lane) for all rows, in accumulator tiles of
// v_mfma_f32_16x16x32_bf16, and dequantises its cells to bf16(q * bf16(s)) in
// registers once per 64-deep k chunk.
//
// Both operands reach LDS by direct global->LDS loads (global_load_lds_dwordx4):
// A (activation rows, gathered by token for gate/up) in a 2-stage ring as
// [row][8 x 16 B] with the 16-byte pieces XOR-swizzled by row, B (the packed
// cells, whose 16 bytes per lane are exactly one lane's MFMA fragment of one
// column) in a 3-stage ring, so the weights, which come from HBM, are
// requested two chunks ahead and the activation rows, mostly L2 hits, one
// chunk ahead. 80 KB per block: two blocks fill the CU's LDS. The 160-row form
// (for experts with 96 rows or more on average) has a 20 KB A stage and a
// 2-stage weight ring (72 KB): the gate/up weights then come one chunk ahead,
// the down weights (read for two chunks of h planes) still two. The loads are
// inline asm, so the compiler's wait-count pass does not see them: every wave
// issues the same loads in the same order and the chunk loop waits for them
// itself (vmcnt is in-order), then a barrier publishes the stage and frees
// the ones read last.
//
// Rows past the expert's end are loaded from a clamped copy of row 0 and never
// stored; the loop body is instantiated for 1 to 8 (10) active 16-row tiles.
// Work items are ordered (expert, column tile, row tile) and consecutive items
// go to the same XCD, so the row tiles of one expert share
// its weights, and the column tiles its rows, in that XCD's L2.
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(const lds_void*)p; }

// 16 bytes per lane from global memory (sbase + voff) into LDS at lds + 16 * lane.
// sbase and lds must be wave-uniform. The LDS address goes through M0: the
// asm keeps the caller's M0 (saved and restored, so no clobber of a register
// the compiler reserves) and puts one wait state between the SALU write of M0
// and the LDS-DMA load that reads it (a gfx9 hazard the compiler does not see
// inside inline asm).
__device__ __forceinline__ void dma16(uint32_t voff, const void* sbase, uint32_t lds) {
  uint32_t m0save;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
      : "=&s"(m0save)
      : "v"(voff), "s"(sbase), "s"(lds)
      : "memory");
}
// The same with the nontemporal hint, for weights no other tile re-reads.
__device__ __forceinline__ void dma16_stream(uint32_t voff, const void* sbase, uint32_t lds) {
  uint32_t m0save;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 nt\n\ts_mov_b32 m0, %0"
      : "=&s"(m0save)
      : "v"(voff), "s"(sbase), "s"(lds)
      : "memory");
}

// Wait until at most N of this wave's vector-memory loads are outstanding and
// its LDS reads are done, then a workgroup barrier. The "memory" clobber keeps
// every LDS access on its side.
template <int N>
__device__ __forceinline__ void vm_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// Element offset of 16-byte piece p of row r in an A stage: [row][8 x 16 B],
// pieces XOR-swizzled by (r >> 1) & 7. A row is half the 256-byte bank width,
// so this puts the 16 rows one fragment read touches on 16 distinct 16-byte
// bank groups.
__device__ __forceinline__ int a_piece(int r, int p) { return p ^ (r & 7); }
__device__ __forceinline__ int a_swz(int r, int p) { return r * 64 + (a_piece(r, p) << 3); }

constexpr int kGemmRows = 128;                // rows per tile (the 128-row form)
constexpr int kGemmB = 16 * 1024;             // B stage: 16 cells x 64 k x 16 columns int8
constexpr int kGemmBJ = 4;                    // B loads per wave per chunk (one cell each)
// ring depths of the int8-plane down product (A and weights alike): two chunks
// (48 KB, three blocks per CU). Three, both issued two chunks ahead (72 KB, two
// blocks per CU), ran 30B-A3B T = 2048 / 4096 296 / 470 -> 301 / 480 us and
// 235B-A22B T = 2048 791 -> 803 us per layer; a three-deep weight ring with the
// activation rows one chunk ahead, 476 -> 492 us at T = 4096.
constexpr int kI8Ring = 2;

// Tile shapes: 128 rows with a weight ring three chunks deep (80 KB), or 160
// rows with a ring two chunks deep (72 KB; an expert with up to 160 rows is
// one tile): either way two blocks fill a CU's LDS. 64 rows with a ring two
// chunks deep (48 KB): three blocks per CU.
template <int RW, int NB = 0, int NA = 2>
struct GemmShape {
  static_assert(RW == 64 || RW == 128 || RW == 160, "tile rows");
  static constexpr int kRows = RW;
  static constexpr int kA = RW * 128;          // A stage: RW rows x 64 bf16
  static constexpr int kAJ = RW / 32;          // A loads per wave per chunk (8 rows each)
  static constexpr int kNA = NA;               // A ring depth
  static constexpr int kNB = NB ? NB : (RW == 128 ? 3 : 2);  // B ring depth
  static constexpr int kLds = kNA * kA + kNB * kGemmB;
};

// Per-wave load descriptors of one tile.
template <int AJ>
struct GemmLoads {
  uint32_t avoff[AJ];       // byte offsets (per lane) of this wave's A loads in src
  const int8_t* bsrc[4];    // this wave's four B cells, at chunk 0
  float sc[4];              // their scales (column lane % 16)
};

// KCW weight chunks of 64 along the reduction. PL = 1: A chunk c meets weight
// chunk c. PL = 2 (the kChainF32 down product): an A row is h's hi plane then
// its lo plane (2 * KCW chunks); A chunk c is plane c & 1 of weight chunk
// c >> 1, so each weight chunk is loaded and converted once and meets both
// planes in two consecutive iterations.
template <bool GATEUP, int MT, bool NTB, int CH, int PL, int RW>
__device__ __forceinline__ void gemm_tile(uint8_t* smem, const GemmLoads<GemmShape<RW>::kAJ>& gl, int KCW, int wv,
                                          int rows, int row0, int nt, const uint16_t* __restrict__ src,
                                          uint16_t* __restrict__ dst, int Ndim) {
  using Sh = GemmShape<RW>;
  constexpr int kGemmA = Sh::kA, kGemmAJ = Sh::kAJ, kGemmNA = Sh::kNA, kGemmNB = Sh::kNB;
  const int lane = threadIdx.x & 63;
  const uint32_t lds0 = lds_addr(smem);
  const uint8_t* const bring = smem + kGemmNA * kGemmA;
  const int KC = PL * KCW;  // A chunks
  floatx4 acc[MT][4];
#pragma unroll
  for (int mi = 0; mi < MT; ++mi)
#pragma unroll
    for (int g = 0; g < 4; ++g) acc[mi][g] = floatx4{0.f, 0.f, 0.f, 0.f};

  auto issue_a = [&](int c) {
    const uint32_t st = lds0 + (uint32_t)((c & 1) * kGemmA + wv * kGemmAJ * 1024);
    const uint16_t* abase = src + (PL == 2 ? (c & 1) * (KCW * 64) + (c >> 1) * 64 : c * 64);
#pragma unroll
    for (int j = 0; j < kGemmAJ; ++j) dma16(gl.avoff[j], abase, st + j * 1024);
  };
  auto issue_b = [&](int b) {
    const uint32_t st = lds0 + (uint32_t)(kGemmNA * kGemmA + (b % kGemmNB) * kGemmB + wv * 4096);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      if (NTB)
        dma16_stream(lane * 16, gl.bsrc[g] + b * 1024, st + g * 1024);
      else
        dma16(lane * 16, gl.bsrc[g] + b * 1024, st + g * 1024);
    }
  };

  // PL = 1, three B stages. Issue order: B(0), A(0), B(1); then iteration c
  // issues A(c+1), B(c+2) and at its end waits for A(c+1) and B(c+1) (only
  // B(c+2) may be outstanding).
  // PL = 1, two B stages: B(0), A(0); iteration c issues A(c+1) and B(c+1)
  // (into the stage B(c-1) left) and at its end waits for both.
  // PL = 2 (two stages suffice). Issue order: B(0), A(0); iteration c issues
  // A(c+1) and, when c is even, B(c/2 + 1); at its end it waits for A(c+1)
  // (c even: B(c/2 + 1) may stay outstanding) or for everything (c odd:
  // B((c+1)/2) is read next).
  constexpr int kAhead = PL == 1 && kGemmNB == 3 ? 2 : 1;  // weight chunks issued ahead (PL = 1)
  issue_b(0);
  issue_a(0);
  if (PL == 1 && kAhead == 2 && 1 < KC) {
    issue_b(1);
    vm_barrier<kGemmBJ>();
  } else {
    vm_barrier<0>();
  }
  bf16x8 lo[4], hi[4];
  for (int c = 0; c < KC; ++c) {
    const int b = PL == 2 ? c >> 1 : c;
    bool b_ahead = false;  // a weight chunk issued this iteration
    if (c + 1 < KC) issue_a(c + 1);
    if (PL == 1 && c + kAhead < KC) {
      issue_b(c + kAhead);
      b_ahead = kAhead == 2;
    }
    if (PL == 2 && (c & 1) == 0 && b + 1 < KCW) {
      issue_b(b + 1);
      b_ahead = true;
    }
    if (PL == 1 || (c & 1) == 0) {
      uint4 raw[4];
      const uint8_t* bp = bring + (b % kGemmNB) * kGemmB + wv * 4096 + lane * 16;
#pragma unroll
      for (int g = 0; g < 4; ++g) raw[g] = *reinterpret_cast<const uint4*>(bp + g * 1024);
#pragma unroll
      for (int g = 0; g < 4; ++g) weights16<CH>(raw[g], gl.sc[g], lo[g], hi[g]);
    }
    const uint16_t* As = reinterpret_cast<const uint16_t*>(smem + (c & 1) * kGemmA);
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const int p = 2 * (lane >> 4) + st;
#pragma unroll
      for (int mi = 0; mi < MT; ++mi) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(As + a_swz(mi * 16 + (lane & 15), p));
        // weights as the first operand: the accumulator tile is the output
        // transposed, so a lane holds four consecutive columns of one row
#pragma unroll
        for (int g = 0; g < 4; ++g) acc[mi][g] = mfma16(st ? hi[g] : lo[g], a, acc[mi][g]);
      }
    }
    if (c + 1 < KC) {
      if (b_ahead)
        vm_barrier<kGemmBJ>();
      else
        vm_barrier<0>();
    }
  }

  // epilogue: lane holds row mi*16 + lane%16 and columns 4*(lane/16) + j of
  // cell g, stored as 8-byte runs. kChainF32 scales each column: lane c holds
  // column c's scale, shuffled to the lanes that hold the column (every lane
  // takes part, before the lanes past the tile's rows drop out).
  float scq[4][4];
  if (CH == kChainF32) {
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int j = 0; j < 4; ++j) scq[g][j] = __shfl(gl.sc[g], 4 * (lane >> 4) + j, 64);
  }
#pragma unroll
  for (int mi = 0; mi < MT; ++mi) {
    const int row = mi * 16 + (lane & 15);
    if (row >= rows) continue;
    uint16_t* drow = dst + (size_t)(row0 + row) * (GATEUP && CH == kChainF32 ? 2 * Ndim : Ndim);
    if (GATEUP) {
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const int col = nt * 128 + wv * 32 + g * 16 + 4 * (lane >> 4);
        float hv[4], lv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (CH == kChainAct) {
            const float gv = round_bf16(acc[mi][g][j]);
            const float uv = round_bf16(acc[mi][g + 2][j]);
            hv[j] = swiglu<true>(gv, uv);
          } else {
            const float gv = __fmul_rn(acc[mi][g][j], scq[g][j]);
            const float uv = __fmul_rn(acc[mi][g + 2][j], scq[g + 2][j]);
            const float h = swiglu<false>(gv, uv);
            hv[j] = round_bf16(h);
            lv[j] = __fsub_rn(h, hv[j]);
          }
        }
        *reinterpret_cast<uint2*>(drow + col) = uint2{pack_bf16x2(hv[0], hv[1]), pack_bf16x2(hv[2], hv[3])};
        if (CH == kChainF32)
          *reinterpret_cast<uint2*>(drow + Ndim + col) = uint2{pack_bf16x2(lv[0], lv[1]), pack_bf16x2(lv[2], lv[3])};
      }
    } else {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = CH == kChainF32 ? __fmul_rn(acc[mi][g][j], scq[g][j]) : acc[mi][g][j];
        *reinterpret_cast<uint2*>(drow + nt * 256 + wv * 64 + g * 16 + 4 * (lane >> 4)) =
            uint2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
      }
    }
  }
}

// The kChainF32 down product on integer planes (k_gemm with I8): A rows are h's
// two int8 digit planes (k_h_planes), B the packed int8 weights as they are, on
// v_mfma_i32_16x16x64_i8 (lane l: row / column l % 16, k = 16 (l / 16) .. + 15,
// the layout of a packed 16-byte piece). A chunk is 64 k of both planes: a row's
// 128 bytes at chunk offset c * 128 (plane 0 in pieces 0..3, plane 1 in 4..7),
// the bytes of a bf16 chunk, so the A ring, its swizzle and its loads are the
// PL = 1 ones. The planes accumulate exactly in i32 (|sum| <= I * 127 * 128);
// the epilogue forms 256 a1 + a2 in f32 and applies the row's scale (a power of
// two) and the column's.
template <int MT, bool NTB, int RW>
__device__ __forceinline__ void gemm_tile_i8(uint8_t* smem, const GemmLoads<GemmShape<RW>::kAJ>& gl, int KC, int wv,
                                             int rows, int row0, int nt, const uint16_t* __restrict__ src,
                                             const float* __restrict__ hs, uint16_t* __restrict__ dst, int Ndim) {
  using Sh = GemmShape<RW, kI8Ring, kI8Ring>;
  constexpr int kGemmA = Sh::kA, kGemmAJ = Sh::kAJ, kGemmNA = Sh::kNA, kGemmNB = Sh::kNB;
  static_assert(kGemmNA == kGemmNB && (kGemmNA == 2 || kGemmNA == 3), "rings of two or three chunks");
  const int lane = threadIdx.x & 63;
  const uint32_t lds0 = lds_addr(smem);
  const uint8_t* const bring = smem + kGemmNA * kGemmA;
  int32x4 a1c[MT][4], a2c[MT][4];
#pragma unroll
  for (int mi = 0; mi < MT; ++mi)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      a1c[mi][g] = int32x4{0, 0, 0, 0};
      a2c[mi][g] = int32x4{0, 0, 0, 0};
    }
  // chunk c's A and weights both in stage c % depth
  auto issue = [&](int c) {
    const uint32_t sa = lds0 + (uint32_t)((c % kGemmNA) * kGemmA + wv * kGemmAJ * 1024);
    const uint16_t* abase = src + c * 64;
#pragma unroll
    for (int j = 0; j < kGemmAJ; ++j) dma16(gl.avoff[j], abase, sa + j * 1024);
    const uint32_t sb = lds0 + (uint32_t)(kGemmNA * kGemmA + (c % kGemmNB) * kGemmB + wv * 4096);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      if (NTB)
        dma16_stream(lane * 16, gl.bsrc[g] + c * 1024, sb + g * 1024);
      else
        dma16(lane * 16, gl.bsrc[g] + c * 1024, sb + g * 1024);
    }
  };
  // chunks issued ahead: depth - 1. Iteration c issues chunk c + depth - 1 (into
  // the stage chunk c - 1 used, free after the previous iteration's barrier)
  // and at its end waits for chunk c + 1: the only loads left outstanding are
  // those of the chunks issued after it, kGemmAJ + 4 each.
  constexpr int kAhead = kGemmNA - 1;
  constexpr int kPer = kGemmAJ + kGemmBJ;
  static_assert(RW <= 64, "one row scale per lane");
  // the rows' scales, requested before the chunks (lane r holds row r's; the
  // epilogue shuffles them out), so the epilogue does not wait a round trip
  const float hsv = lane < rows ? hs[row0 + lane] : 0.0f;
#pragma unroll
  for (int c = 0; c < kAhead + 1; ++c)
    if (c < KC) issue(c);
  // chunk 0 before the first iteration: the chunks issued after it may stay outstanding
  const int after0 = min(KC - 1, kAhead);
  if (after0 == 2)
    vm_barrier<2 * kPer>();
  else if (after0 == 1)
    vm_barrier<kPer>();
  else
    vm_barrier<0>();
  for (int c = 0; c < KC; ++c) {
    if (c + kAhead < KC && c > 0) issue(c + kAhead);
    int32x4 q[4];
    const uint8_t* bp = bring + (c % kGemmNB) * kGemmB + wv * 4096 + lane * 16;
#pragma unroll
    for (int g = 0; g < 4; ++g) q[g] = *reinterpret_cast<const int32x4*>(bp + g * 1024);
    const uint16_t* As = reinterpret_cast<const uint16_t*>(smem + (c % kGemmNA) * kGemmA);
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) {
      const int r = mi * 16 + (lane & 15);
      const int32x4 p1 = *reinterpret_cast<const int32x4*>(As + a_swz(r, lane >> 4));
      const int32x4 p2 = *reinterpret_cast<const int32x4*>(As + a_swz(r, 4 + (lane >> 4)));
      // weights as the first operand: the accumulator tile is the output
      // transposed, so a lane holds four consecutive columns of one row
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        a1c[mi][g] = __builtin_amdgcn_mfma_i32_16x16x64_i8(q[g], p1, a1c[mi][g], 0, 0, 0);
        a2c[mi][g] = __builtin_amdgcn_mfma_i32_16x16x64_i8(q[g], p2, a2c[mi][g], 0, 0, 0);
      }
    }
    if (c + 1 < KC) {
      // outstanding after chunk c + 1: the chunks issued after it
      const int after = min(KC - 1, c + kAhead) - (c + 1);
      if (kAhead == 2 && after > 0)
        vm_barrier<kPer>();
      else
        vm_barrier<0>();
    }
  }
  // epilogue: lane holds row mi*16 + lane%16 and columns 4*(lane/16) + j of
  // cell g, stored as one 8-byte run. The column scales move to those lanes
  // (lane c holds column c's) and the row scales likewise, with every lane
  // taking part in the shuffles (an exec-masked source lane gives no data)
  // before the lanes past the tile's rows drop out.
  float scq[4][4];
#pragma unroll
  for (int g = 0; g < 4; ++g)
#pragma unroll
    for (int j = 0; j < 4; ++j) scq[g][j] = __shfl(gl.sc[g], 4 * (lane >> 4) + j, 64);
#pragma unroll
  for (int mi = 0; mi < MT; ++mi) {
    const int row = mi * 16 + (lane & 15);
    const float rs = __shfl(hsv, row, 64);
    if (row >= rows) continue;
    uint16_t* drow = dst + (size_t)(row0 + row) * Ndim + nt * 256 + wv * 64 + 4 * (lane >> 4);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float v = __fadd_rn(__fmul_rn((float)a1c[mi][g][j], 256.0f), (float)a2c[mi][g][j]);
        o[j] = __fmul_rn(__fmul_rn(v, rs), scq[g][j]);
      }
      *reinterpret_cast<uint2*>(drow + g * 16) = uint2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
    }
  }
}

// GATEUP = true: A rows gathered from x by token, B = gate|up cells, epilogue
// SwiGLU -> h_sorted. GATEUP = false: A = h_sorted rows, B = down, epilogue ->
// y_sorted. src must span fewer than 2^32 bytes (32-bit load offsets).
// NTB: the weights are loaded with the nontemporal hint (few rows per expert,
// so no second row tile would find them in L2).
template <bool GATEUP, bool NTB, int CH, int RW, bool I8 = false>
__global__ __launch_bounds__(256, 2) void k_gemm(int D, int I, int E, const uint16_t* __restrict__ src,
                                                  const int32_t* __restrict__ offsets,
                                                  const int32_t* __restrict__ sorted_token,
                                                  const int8_t* __restrict__ wp, const float* __restrict__ sp,
                                                  uint16_t* __restrict__ dst, int cap, const float* __restrict__ hs) {
  static_assert(!I8 || (!GATEUP && CH == kChainF32 && RW == 64), "int8 planes: the f32 chain's down product");
  using Sh = GemmShape<RW, I8 ? kI8Ring : 0, I8 ? kI8Ring : 2>;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[Sh::kLds];
  // set-up scratch inside the ring (no loads are in flight yet)
  int* const mtp = reinterpret_cast<int*>(smem);
  int* const offs = mtp + kMaxExperts + 1;
  int* const wsum = offs + kMaxExperts + 1;
  int* const tok = wsum + 4;
  const int tid = threadIdx.x, lane = tid & 63;
  const int NT = GATEUP ? I / 128 : D / 256;
  tile_prefix<RW>(offsets, E, cap, mtp, wsum, offs);
  const int ntiles = mtp[E] * NT;
  const int per = (ntiles + 7) >> 3;
  const int q = blockIdx.x >> 3;
  if (q >= per) return;
  const int L = (blockIdx.x & 7) * per + q;
  if (L >= ntiles) return;
  // L -> (expert, column tile, row tile), row tile fastest
  const int e = __builtin_amdgcn_readfirstlane(tile_expert(mtp, E, L / NT));
  const int nmt_e = mtp[e + 1] - mtp[e];
  const int rem = L - mtp[e] * NT;
  const int nt = __builtin_amdgcn_readfirstlane(rem / nmt_e);
  const int mt = rem - nt * nmt_e;
  // the expert's rows split evenly over its nmt_e row tiles (multiples of 16
  // rows; every tile gets at least one row): tiles of one column block then run
  // at the same pace and meet each other's weight chunks in L2, where a full
  // tile and a nearly empty one would each fetch them
  const int ne = min(offs[e + 1] - offs[e], cap);
  const int tr = (((ne + nmt_e - 1) / nmt_e) + 15) & ~15;
  const int row0 = __builtin_amdgcn_readfirstlane(offs[e] + mt * tr);
  const int rows = __builtin_amdgcn_readfirstlane(min(tr, ne - mt * tr));
  if (tid < RW) tok[tid] = (tid < rows) ? (GATEUP ? sorted_token[row0 + tid] : row0 + tid) : -1;
  __syncthreads();

  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  // kChainF32 down: A rows are h's hi and lo planes (2I wide)
  const int Kdim = GATEUP ? D : (CH == kChainF32 ? 2 * I : I);
  const int KCW = (GATEUP ? D : I) >> 6;
  const int Ndim = GATEUP ? I : D;
  GemmLoads<Sh::kAJ> gl;
  // A load j of wave wv covers tile rows 8q .. 8q+7, q = wv * AJ + j: lane -> (row, LDS piece lane % 8)
#pragma unroll
  for (int j = 0; j < Sh::kAJ; ++j) {
    const int r = 8 * (wv * Sh::kAJ + j) + (lane >> 3);
    const int t = tok[r] >= 0 ? tok[r] : tok[0];
    gl.avoff[j] = ((uint32_t)t * (uint32_t)Kdim + (uint32_t)(a_piece(r, lane & 7) << 3)) * 2u;
  }
  // this wave's cells: gate/up -> (which = g >> 1, h group nt*8 + 2*wv + (g & 1)); down -> column group nt*16 + 4*wv + g
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    if (GATEUP) {
      const size_t cid = ((size_t)e * (I >> 4) + nt * 8 + 2 * wv + (g & 1)) * 2 + (g >> 1);
      gl.bsrc[g] = wp + cid * (size_t)(D >> 4) * 256;
      gl.sc[g] = chain_scale<CH>(sp[cid * 16 + (lane & 15)]);
    } else {
      const size_t dg = (size_t)e * (D >> 4) + nt * 16 + 4 * wv + g;
      gl.bsrc[g] = wp + dg * (size_t)(I >> 4) * 256;
      gl.sc[g] = chain_scale<CH>(sp[dg * 16 + (lane & 15)]);
    }
  }
  // kChainAct dequantises with the scales in the chunk loop: consume the scale
  // loads here, so the compiler's waits for them sit before the loop (inside
  // it they would also drain the ring's loads). kChainF32 applies them in the
  // epilogue only, where the loads have long landed: leaving them in flight
  // takes a global round trip off every tile's start. And no wave may start
  // loading into the ring while another still reads tok.
  if constexpr (CH != kChainF32) asm volatile("" ::"v"(gl.sc[0]), "v"(gl.sc[1]), "v"(gl.sc[2]), "v"(gl.sc[3]));
  __syncthreads();
  constexpr int PL = !GATEUP && CH == kChainF32 && !I8 ? 2 : 1;  // h planes of the down product
  if constexpr (I8) {
    switch ((rows + 15) >> 4) {
      case 4:
        gemm_tile_i8<4, NTB, RW>(smem, gl, KCW, wv, rows, row0, nt, src, hs, dst, Ndim);
        break;
      case 3:
        gemm_tile_i8<3, NTB, RW>(smem, gl, KCW, wv, rows, row0, nt, src, hs, dst, Ndim);
        break;
      case 2:
        gemm_tile_i8<2, NTB, RW>(smem, gl, KCW, wv, rows, row0, nt, src, hs, dst, Ndim);
        break;
      default:
        gemm_tile_i8<1, NTB, RW>(smem, gl, KCW, wv, rows, row0, nt, src, hs, dst, Ndim);
        break;
    }
    return;
  }
  // as many 16-row MFMA tiles as the rows need
  switch ((rows + 15) >> 4) {
    case 10:
      if constexpr (RW >= 160)
        gemm_tile<GATEUP, 10, NTB, CH, PL, RW>(smem, gl, KCW, wv, rows, row0, nt, src, dst, Ndim);
      break;
    case 9:
      if constexpr (RW >= 144)
        gemm_tile<GATEUP, 9, NTB, CH, PL, RW>(smem, gl, KCW, wv, rows, row0, nt, src, dst, Ndim);
      break;
    case 8:
      if constexpr (RW >= 128)
        gemm_tile<GATEUP, 8, NTB, CH, PL, RW>(smem, gl, KCW, wv, rows, row0, nt, src, dst, Ndim);
      break;
    case 7:
      if constexpr (RW >= 112)
        gemm_tile<GATEUP, 7, NTB, CH, PL, RW>(smem, gl, KCW, wv, rows, row0, nt, src, dst, Ndim);
      break;
    case 6:
      if constexpr (RW >= 96)
        gemm_tile<GATEUP, 6, NTB, CH, PL, RW>(smem, gl, KCW, wv, rows, row0, nt, src, dst, Ndim);
      break;
    case 5:
      if constexpr (RW >= 80)
        gemm_tile<GATEUP, 5, NTB, CH, PL, RW>(smem, gl, KCW, wv, rows, row0, nt, src, dst, Ndim);
      break;
    case 4:
      gemm_tile<GATEUP, 4, NTB, CH, PL, RW>(smem, gl, KCW, wv, rows, row0, nt, src, dst, Ndim);
      break;
    case 3:
      gemm_tile<GATEUP, 3, NTB, CH, PL, RW>(smem, gl, KCW, wv, rows, row0, nt, src, dst, Ndim);
      break;
    case 2:
      gemm_tile<GATEUP, 2, NTB, CH, PL, RW>(smem, gl, KCW, wv, rows, row0, nt, src, dst, Ndim);
      break;
    default:
      gemm_tile<GATEUP, 1, NTB, CH, PL, RW>(smem, gl, KCW, wv, rows, row0, nt, src, dst, Ndim);
      break;
  }
}

// The f32 chain's h for the integer down product: row m's hi and lo planes
// (h = hi + lo, exact in f32) become two int8 digit planes of the integer
// H = rint(h * 2^k), H = 256 p1 + p2 with p2 in [-128, 127] and p1 in
// [-127, 127]; k is the largest power of two with max |h| * 2^k <= 32639, so H
// keeps 15 bits relative to the row's largest |h|. In place: the planes take
// the first 2I bytes of the row (chunk c: p1 at c * 128, p2 at c * 128 + 64)
// once the wave holds the whole row; hs[m] = 2^-k. A row with a non-finite h
// gets hs[m] = NaN, so its whole y row is NaN. One wave per row, I <= 2048.
__global__ __launch_bounds__(256) void k_h_planes(int M, int I, uint16_t* __restrict__ h, float* __restrict__ hs) {
  const int lane = threadIdx.x & 63;
  const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (m >= M) return;
  uint16_t* row = h + (size_t)m * 2 * I;
  // lane L, step s: the eight elements from 8 (L + 64 s) on (16-byte loads of
  // each bf16 plane, 8-byte stores of each int8 plane)
  constexpr int kSteps = kPlanesMaxChunks / 8;
  float v[kSteps][8];
  // the largest |h| as f32 bits: above 0x7f7fffff for an inf or a NaN (which
  // fmaxf would pass over)
  uint32_t mb = 0;
#pragma unroll
  for (int st = 0; st < kSteps; ++st) {
    const int e = 8 * (lane + 64 * st);
    if (e < I) {
      const uint4 hi = *reinterpret_cast<const uint4*>(row + e);
      const uint4 lo = *reinterpret_cast<const uint4*>(row + I + e);
      const uint32_t hw[4] = {hi.x, hi.y, hi.z, hi.w}, lw[4] = {lo.x, lo.y, lo.z, lo.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[st][2 * i] = __uint_as_float(hw[i] << 16) + __uint_as_float(lw[i] << 16);
        v[st][2 * i + 1] = __uint_as_float(hw[i] & 0xffff0000u) + __uint_as_float(lw[i] & 0xffff0000u);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) mb = max(mb, __float_as_uint(v[st][i]) & 0x7fffffffu);
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mb = max(mb, (uint32_t)__shfl_xor((int)mb, o, 64));
  const bool bad = mb > 0x7f7fffffu;
  const float mx = __uint_as_float(mb);
  int k = 0;
  if (!bad && mx > 0.0f) {
    int ex;
    (void)frexpf(mx, &ex);  // mx < 2^ex
    k = ldexpf(mx, 15 - ex) <= 32639.0f ? 15 - ex : 14 - ex;
  }
  uint8_t* out = reinterpret_cast<uint8_t*>(row);
#pragma unroll
  for (int st = 0; st < kSteps; ++st) {
    const int e = 8 * (lane + 64 * st);
    if (e < I) {
      uint32_t w1[2] = {0, 0}, w2[2] = {0, 0};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int H = bad ? 0 : (int)rintf(ldexpf(v[st][i], k));
        const int p2 = ((H + 128) & 255) - 128;
        w1[i >> 2] |= (uint32_t)(((H - p2) >> 8) & 255) << (8 * (i & 3));
        w2[i >> 2] |= (uint32_t)(p2 & 255) << (8 * (i & 3));
      }
      const int c = e >> 6, o = e & 63;
      *reinterpret_cast<uint2*>(out + c * 128 + o) = uint2{w1[0], w1[1]};
      *reinterpret_cast<uint2*>(out + c * 128 + 64 + o) = uint2{w2[0], w2[1]};
    }
  }
  if (lane == 0) hs[m] = bad ? __builtin_nanf("") : ldexpf(1.0f, -k);
}

// ---------------------------------------------------------------------------
// Layout-native experts: one thread per output element, a sequential fmaf
// chain over the reduction axis from +0.0f (the oracle's order). Serves the
// f32 configuration, plain-weight layers and unpacked int8 weights.
// ---------------------------------------------------------------------------
struct WView {
  const void* v;
  const void* s;
  int wt;  // 0 f32, 1 bf16, 2 int8
  int s_bf16;
  int per_channel;
};

template <bool BF16>
__device__ __forceinline__ float w_at(const WView& w, size_t idx, size_t sidx) {
  if (w.wt == 0) {
    const float v = reinterpret_cast<const float*>(w.v)[idx];
    return BF16 ? round_bf16(v) : v;
  }
  if (w.wt == 1) return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(w.v)[idx]);
  const float q = (float)reinterpret_cast<const int8_t*>(w.v)[idx];
  const size_t si = w.per_channel ? sidx : 0;
  const float sv = w.s_bf16 ? bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(w.s)[si])
                            : reinterpret_cast<const float*>(w.s)[si];
  return BF16 ? round_bf16(q * round_bf16(sv)) : q * sv;
}

// kChainAct with bf16 activations rounds the weights and g, u, every silu step
// and y to bf16; kChainF32 (and any chain with f32 activations) keeps weights
// and intermediates in f32, h of bf16 activations as its hi and lo planes.
template <typename A, int CH>
struct GenericChain {
  static constexpr bool kRound = Act<A>::kBf16 && CH == kChainAct;
  static constexpr bool kSplitH = Act<A>::kBf16 && CH == kChainF32;
};

template <typename A, int CH>
__global__ __launch_bounds__(256) void k_gateup_generic(int D, int I, const A* __restrict__ x,
                                                         const int32_t* __restrict__ sorted_token,
                                                         const int32_t* __restrict__ sorted_expert, WView wg, WView wu,
                                                         A* __restrict__ h_sorted) {
  using C = GenericChain<A, CH>;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  const int m = blockIdx.y;
  if (i >= I) return;
  const int t = sorted_token[m], e = sorted_expert[m];
  float g = 0.0f, u = 0.0f;
  for (int d = 0; d < D; ++d) {
    const float xv = Act<A>::load(x, (int64_t)t * D + d);
    const size_t idx = ((size_t)e * D + d) * I + i;
    g = __builtin_fmaf(xv, w_at<C::kRound>(wg, idx, (size_t)e * I + i), g);
    u = __builtin_fmaf(xv, w_at<C::kRound>(wu, idx, (size_t)e * I + i), u);
  }
  if (C::kRound) {
    g = round_bf16(g);
    u = round_bf16(u);
  }
  const float h = swiglu<C::kRound>(g, u);
  if (C::kSplitH) {
    uint16_t* hr = reinterpret_cast<uint16_t*>(h_sorted) + (int64_t)m * 2 * I + i;
    split_bf16(h, hr[0], hr[I]);
  } else {
    Act<A>::store(h_sorted, (int64_t)m * I + i, h);
  }
}

template <typename A, int CH>
__global__ __launch_bounds__(256) void k_down_generic(int D, int I, const A* __restrict__ h_sorted,
                                                       const int32_t* __restrict__ sorted_expert, WView wd,
                                                       A* __restrict__ y_sorted) {
  using C = GenericChain<A, CH>;
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  const int m = blockIdx.y;
  if (n >= D) return;
  const int e = sorted_expert[m];
  float acc = 0.0f;
  for (int i = 0; i < I; ++i) {
    float hv;
    if (C::kSplitH) {
      const uint16_t* hr = reinterpret_cast<const uint16_t*>(h_sorted) + (int64_t)m * 2 * I + i;
      hv = bf16_bits_to_f32(hr[0]) + bf16_bits_to_f32(hr[I]);  // exact in f32
    } else {
      hv = Act<A>::load(h_sorted, (int64_t)m * I + i);
    }
    acc = __builtin_fmaf(hv, w_at<C::kRound>(wd, ((size_t)e * I + i) * D + n, (size_t)e * D + n), acc);
  }
  Act<A>::store(y_sorted, (int64_t)m * D + n, acc);
}

// ---------------------------------------------------------------------------
// Combine: out[t, n] from the terms p_j = round(w[t,j] * y_sorted[inv[t*K+j], n])
// in j order: SCATTER = false sums them in f32 from +0.0f and rounds once
// (jnp.sum of y_k * w, kappa/qwen3/ffn_moe.py:103); SCATTER = true rounds the
// running sum after every add (out.at[token].add(y * w) into a zero buffer of
// x.dtype, :157, :215). No atomics, one writer per element.
// A thread owns 8 consecutive columns (one 16-byte bf16 load per row); the
// row indices and weights of a token are read first and the K row loads are
// issued in batches of 8 before the FMAs. With res (the residual stream h of
// kappa/qwen3/block.py:207) the rounded sum is added to res[t, n] in f32 and
// rounded again.
// ---------------------------------------------------------------------------
template <typename A>
struct Vec8;
template <>
struct Vec8<uint16_t> {
  // the combine reads each y row and residual once: nontemporal loads
  __device__ __forceinline__ static void load(const uint16_t* p, float* v) {
    const uint4 q = load_stream16(reinterpret_cast<const int8_t*>(p));
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = __uint_as_float(w[j] << 16);
      v[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
    }
  }
  __device__ __forceinline__ static void store(uint16_t* p, const float* v) {
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      w[j] = (uint32_t)f32_to_bf16_bits(v[2 * j]) | ((uint32_t)f32_to_bf16_bits(v[2 * j + 1]) << 16);
    *reinterpret_cast<uint4*>(p) = uint4{w[0], w[1], w[2], w[3]};
  }
};
template <>
struct Vec8<float> {
  __device__ __forceinline__ static void load(const float* p, float* v) {
    const uint4 a = load_stream16(reinterpret_cast<const int8_t*>(p));
    const uint4 b = load_stream16(reinterpret_cast<const int8_t*>(p + 4));
    v[0] = __uint_as_float(a.x), v[1] = __uint_as_float(a.y), v[2] = __uint_as_float(a.z);
    v[3] = __uint_as_float(a.w), v[4] = __uint_as_float(b.x), v[5] = __uint_as_float(b.y);
    v[6] = __uint_as_float(b.z), v[7] = __uint_as_float(b.w);
  }
  __device__ __forceinline__ static void store(float* p, const float* v) {
    reinterpret_cast<float4*>(p)[0] = float4{v[0], v[1], v[2], v[3]};
    reinterpret_cast<float4*>(p)[1] = float4{v[4], v[5], v[6], v[7]};
  }
};

// acc + round(w * y), the sum rounded again when SCATTER
template <typename A, bool SCATTER>
__device__ __forceinline__ float combine_term(float acc, float w, float y) {
  const float s = __fadd_rn(acc, Act<A>::round(__fmul_rn(w, y)));
  return SCATTER ? Act<A>::round(s) : s;
}

template <typename A, bool SCATTER>
__global__ __launch_bounds__(256) void k_combine8(int T, int K, int D, const A* __restrict__ y,
                                                   const int32_t* __restrict__ inv, const float* __restrict__ w,
                                                   A* __restrict__ out, const A* __restrict__ res) {
  const int t = blockIdx.y;
  const int n0 = (blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (n0 >= D) return;
  float acc[8];
#pragma unroll
  for (int v = 0; v < 8; ++v) acc[v] = 0.0f;
  for (int jb = 0; jb < K; jb += 8) {
    const int nj = min(8, K - jb);
    float wj[8], yv[8][8];
    bool on[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      // a dropped assignment (inv < 0, fixed_capacity) adds nothing
      const int p = j < nj ? inv[(int64_t)t * K + jb + j] : -1;
      on[j] = p >= 0;
      if (on[j]) {
        wj[j] = w[(int64_t)t * K + jb + j];
        Vec8<A>::load(y + (int64_t)p * D + n0, yv[j]);
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (on[j])
#pragma unroll
        for (int v = 0; v < 8; ++v) acc[v] = combine_term<A, SCATTER>(acc[v], wj[j], yv[j][v]);
  }
  if (res) {
    // the block's output is rounded to the activation dtype, then added to h
    float r[8];
    Vec8<A>::load(res + (int64_t)t * D + n0, r);
#pragma unroll
    for (int v = 0; v < 8; ++v) acc[v] = r[v] + Act<A>::round(acc[v]);
  }
  Vec8<A>::store(out + (int64_t)t * D + n0, acc);
}

// Any D: one column per thread.
template <typename A, bool SCATTER>
__global__ __launch_bounds__(256) void k_combine1(int T, int K, int D, const A* __restrict__ y,
                                                   const int32_t* __restrict__ inv, const float* __restrict__ w,
                                                   A* __restrict__ out, const A* __restrict__ res) {
  const int t = blockIdx.y;
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= D) return;
  float acc = 0.0f;
  for (int j = 0; j < K; ++j) {
    const int p = inv[(int64_t)t * K + j];
    if (p >= 0) acc = combine_term<A, SCATTER>(acc, w[(int64_t)t * K + j], Act<A>::load(y, (int64_t)p * D + n));
  }
  if (res) acc = Act<A>::load(res, (int64_t)t * D + n) + Act<A>::round(acc);
  Act<A>::store(out, (int64_t)t * D + n, acc);
}


// ---------------------------------------------------------------------------
// Decode with few assignments (T * K <= 32, K <= 8): the down projection and
// the weighted combine in one kernel, so y never leaves the CU. Block
// (dt, tb) owns output columns 16*dt .. 16*dt+15 of the TPB = 8 / K tokens
// tb*TPB ...; waves 2m and 2m+1 compute the block's assignment m (row inv of
// h_sorted against expert topk_idx, global index tb*TPB*K + m) as row 0 of a
// 16-row MFMA tile. The reduction axis keeps the four partial chains of
// k_down_decode's wave split (chunks [KC*r/4, KC*(r+1)/4)): wave 2m runs
// chains 0 and 1, wave 2m+1 chains 2 and 3, and the combine adds them in
// k_down_decode's order, so each y is the value k_down_decode stores; the
// sum over j then follows k_combine8's order. A wave issues all its weight
// loads first, its chunks of the h row go through LDS, and the combine's
// selections and weights are loaded at the start. An expert picked by tokens
// of several blocks is read by each of them, which is why the fused form stops
// at 32 assignments (at 64 it was slower than the two kernels).
// ---------------------------------------------------------------------------
template <int KCMAX, int CH, bool SCATTER>
__global__ __launch_bounds__(1024) void k_down_combine(int T, int K, int TPB, int D, int I,
                                                        const uint16_t* __restrict__ h_sorted,
                                                        const int32_t* __restrict__ topk_idx,
                                                        const int32_t* __restrict__ inv,
                                                        const float* __restrict__ topk_w,
                                                        const int8_t* __restrict__ w2, const float* __restrict__ s2,
                                                        uint16_t* __restrict__ out, const uint16_t* __restrict__ res) {
  // kChainF32: an h row is its hi and lo planes (2I)
  constexpr int NP = CH == kChainF32 ? 2 : 1;
  extern __shared__ __attribute__((aligned(16))) uint16_t hrows[];  // [TPB*K][NP*I]
  __shared__ float part[2][3][kDownCombineMaxRows][16];  // [hi, lo] x chains 0+1, 2, 3 of row 0
  __shared__ float scl[kDownCombineMaxRows][16];                    // kChainF32: the column scales
  const int dt = blockIdx.x, tid = threadIdx.x;
  const int lane = tid & 63, wv = tid >> 6;  // blockDim.x = 128 * TPB * K
  const int m = wv >> 1, half = wv & 1;
  const int t0 = blockIdx.y * TPB, nt = min(TPB, T - t0);  // this block's tokens
  const int64_t a0 = (int64_t)t0 * K;                      // its first assignment
  const int KC = I >> 6;
  // the combine thread (token t0 + tid / 16, column tid % 16) fetches its row
  // of selections now
  const bool comb = tid < nt * 16;
  int cinv[kDownCombineMaxRows];
  float cw[kDownCombineMaxRows];
#pragma unroll
  for (int j = 0; j < kDownCombineMaxRows; ++j) {
    cinv[j] = -1;
    cw[j] = 0.0f;
    if (comb && j < K) {
      cinv[j] = inv[a0 + (tid >> 4) * K + j];
      cw[j] = topk_w[a0 + (tid >> 4) * K + j];
    }
  }
  const int p = m < nt * K ? inv[a0 + m] : -1;
  if (p >= 0) {
    const int e = topk_idx[a0 + m];
    const int cl = (KC * 2 * half) >> 2, ch = (KC * 2 * (half + 1)) >> 2;  // chains 2h and 2h+1
    const size_t cell = (size_t)(I >> 4) * 256;
    const int8_t* bp = w2 + ((size_t)e * (D >> 4) + dt) * cell + lane * 16;
    uint4 q[KCMAX];
#pragma unroll
    for (int c = 0; c < KCMAX; ++c)
      if (cl + c < ch) q[c] = load_stream16(bp + (size_t)(cl + c) * 1024);
    const float sc = chain_scale<CH>(s2[(size_t)e * D + dt * 16 + (lane & 15)]);
    if (CH == kChainF32 && half == 0 && lane < 16) scl[m][lane] = sc;
    // this wave's chunks of the h row (8 pieces of 16 bytes per chunk, per plane)
    uint16_t* hr = hrows + (size_t)m * NP * I;
    const uint4* src = reinterpret_cast<const uint4*>(h_sorted + (size_t)p * NP * I);
#pragma unroll
    for (int pl = 0; pl < NP; ++pl)
      for (int i = cl * 8 + lane; i < ch * 8; i += 64)
        reinterpret_cast<uint4*>(hr)[pl * (I >> 3) + i] = src[pl * (I >> 3) + i];
    // the pieces are read back by other lanes of this wave only
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // the assignment's row is tile row 0; kChainF32 puts its lo plane in tile
    // row 8, as k_down_decode does
    const bool rowhi = (lane & 15) == 0, rowlo = CH == kChainF32 && (lane & 15) == 8;
    const int koff = 16 * (lane >> 4) + (rowlo ? I : 0);
    floatx4 acc[2];
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const int r = 2 * half + rr;
      const int c0 = (KC * r) >> 2, c1 = (KC * (r + 1)) >> 2;
      acc[rr] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < KCMAX; ++c) {
        if (cl + c >= c0 && cl + c < c1) {
          uint4 a0v = uint4{0, 0, 0, 0}, a1v = uint4{0, 0, 0, 0};
          if (rowhi || rowlo) {
            const uint4* ap = reinterpret_cast<const uint4*>(hr + (cl + c) * 64 + koff);
            a0v = ap[0];
            a1v = ap[1];
          }
          bf16x8 b0, b1;
          weights16<CH>(q[c], sc, b0, b1);
          acc[rr] = mfma16(as_bf16x8(a0v), b0, acc[rr]);
          acc[rr] = mfma16(as_bf16x8(a1v), b1, acc[rr]);
        }
      }
    }
    // lanes 0..15 hold tile row 0 (columns 0..15), lanes 32..47 tile row 8
    const int pl = lane >> 5;
    if ((lane & 31) < 16 && (pl == 0 || CH == kChainF32)) {
      if (half == 0) {
        part[pl][0][m][lane & 15] = acc[0][0] + acc[1][0];
      } else {
        part[pl][1][m][lane & 15] = acc[0][0];
        part[pl][2][m][lane & 15] = acc[1][0];
      }
    }
  }
  __syncthreads();
  if (comb) {
    const int t = tid >> 4, col = tid & 15;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < kDownCombineMaxRows; ++j) {
      // a dropped assignment (inv < 0, fixed_capacity) adds nothing
      if (j < K && cinv[j] >= 0) {
        const int mj = t * K + j;
        float v = (part[0][0][mj][col] + part[0][1][mj][col]) + part[0][2][mj][col];
        if (CH == kChainF32)
          v = __fmul_rn(v + ((part[1][0][mj][col] + part[1][1][mj][col]) + part[1][2][mj][col]), scl[mj][col]);
        acc = combine_term<uint16_t, SCATTER>(acc, cw[j], round_bf16(v));
      }
    }
    const int64_t o = (int64_t)(t0 + t) * D + dt * 16 + col;
    if (res) acc = bf16_bits_to_f32(res[o]) + round_bf16(acc);
    out[o] = f32_to_bf16_bits(acc);
  }
}

template <typename A>
__global__ __launch_bounds__(256) void k_cast_from_f32(int64_t n, const float* __restrict__ in, A* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) Act<A>::store(out, i, in[i]);
}

}  // namespace kmoe

namespace kmoe_host {

using namespace kmoe;

namespace {

// The packed-weight kernels of one rounding chain.
template <int CH>
hipError_t packed_stages(const kmoe_desc& d, int family, int stages, const uint16_t* xb, const int32_t* offsets,
                         const int32_t* active, const int32_t* sorted_token, const int8_t* w13, const float* s13,
                         const int8_t* w2, const float* s2, uint16_t* hb, uint16_t* yb, float* hs, hipStream_t st) {
  const int T = (int)d.tokens, D = (int)d.hidden, E = (int)d.num_experts, K = (int)d.top_k,
            I = (int)d.intermediate;
  const int M = T * K;
  const int slots = M < E ? M : E;
  const int cap = capacity_of(d);
  if (family == kFamilyDecode) {
    // shapes from a sweep on MI355X (30B-A3B layer, T = 1..64): four waves split
    // the reduction, batches of 4 (gate/up) or 3 (down) chunks per load stage
    if (stages & kStageGateUp) {
      if ((T <= 4 && D / 64 == 32) || (T <= 16 && D / 64 == 64)) {
        // eight waves of load batches of four chunks (one batch at D = 2048,
        // two at D = 4096), at most one 16-row block per expert; up to four
        // tokens the tile is the T tokens themselves (DENSE), beyond it the
        // expert's gathered rows. At D = 4096 this beats the four-wave form
        // below up to 16 tokens (235B-A22B T=16 241 against 258 us per layer).
        const dim3 grid(I / 16, slots);
        if (T <= 4)
          hipLaunchKernelGGL((k_gateup_decode<8, 4, false, 1, true, false, CH>), grid, dim3(512), 0, st, T, D, I, E,
                             xb, offsets, active, sorted_token, w13, s13, hb, cap);
        else
          hipLaunchKernelGGL((k_gateup_decode<8, 4, false, 1, false, false, CH>), grid, dim3(512), 0, st, T, D, I, E,
                             xb, offsets, active, sorted_token, w13, s13, hb, cap);
      } else {
        // one 16-row block per block, the expert's rows spread over grid z
        // (ceil(T/16) groups; an expert has at most T rows); four waves of two
        // reduction parts each. Against one block holding all of an expert's
        // rows (up to four 16-row blocks): decode T=64 gate/up 70 -> 64 us,
        // from the smaller register and LDS footprint. At D = 2048 it also
        // beats the eight-wave form from five tokens on (30B-A3B T=16 gate/up
        // 45.4 -> 42.9 us, T=8 29.8 -> 28.9 us).
        const dim3 grid(I / 16, slots, (T + 15) / 16);
        if ((D / 64) % 16 == 0)
          hipLaunchKernelGGL((k_gateup_decode<4, 4, false, 1, false, false, CH>), grid, dim3(256), 0, st, T, D, I, E,
                             xb, offsets, active, sorted_token, w13, s13, hb, cap);
        else
          hipLaunchKernelGGL((k_gateup_decode<4, 4, true, 1, false, false, CH>), grid, dim3(256), 0, st, T, D, I, E,
                             xb, offsets, active, sorted_token, w13, s13, hb, cap);
      }
      hipError_t err = hipGetLastError();
      if (err != hipSuccess) return err;
    }
    if (stages & kStageDown) {
      const int cpw = (I / 64) / 4;
      const dim3 grid(D / 32, slots);
      if ((I / 64) % 4 == 0 && cpw % 3 == 0)
        hipLaunchKernelGGL((k_down_decode<4, 2, 3, false, false, CH>), grid, dim3(256), 0, st, D, I, E, hb, offsets,
                           active, w2, s2, yb, cap);
      else
        hipLaunchKernelGGL((k_down_decode<4, 2, 4, true, false, CH>), grid, dim3(256), 0, st, D, I, E, hb, offsets,
                           active, w2, s2, yb, cap);
      return hipGetLastError();
    }
    return hipSuccess;
  }
  if (family == kFamilyRows && T <= kRowsPathMaxTokens && (D / 64 == 32 || D / 64 == 64) &&
      (I / 64 == 12 || I / 64 == 24)) {
    // just above the decode sizes: the decode kernels over all of an expert's
    // rows in groups of 64, each wave's weights loaded once and kept in
    // registers (65 and 128 tokens: 158 -> 143 and 161 -> 155 us per layer
    // against the grouped GEMMs; from 256 tokens on the GEMMs are faster)
    if (stages & kStageGateUp) {
      const dim3 grid(I / 16, slots);
      if (D / 64 == 32)
        hipLaunchKernelGGL((k_gateup_decode<4, 8, false, kDecodeMaxRowBlocks, false, true, CH>), grid, dim3(256), 0,
                           st, T, D, I, E, xb, offsets, active, sorted_token, w13, s13, hb, cap);
      else
        hipLaunchKernelGGL((k_gateup_decode<8, 8, false, kDecodeMaxRowBlocks, false, true, CH>), grid, dim3(512), 0,
                           st, T, D, I, E, xb, offsets, active, sorted_token, w13, s13, hb, cap);
      hipError_t err = hipGetLastError();
      if (err != hipSuccess) return err;
    }
    if (stages & kStageDown) {
      const dim3 grid(D / 32, slots);
      if (I / 64 == 12)
        hipLaunchKernelGGL((k_down_decode<4, 2, 3, false, true, CH>), grid, dim3(256), 0, st, D, I, E, hb, offsets,
                           active, w2, s2, yb, cap);
      else
        hipLaunchKernelGGL((k_down_decode<4, 2, 6, false, true, CH>), grid, dim3(256), 0, st, D, I, E, hb, offsets,
                           active, w2, s2, yb, cap);
      return hipGetLastError();
    }
    return hipSuccess;
  }
  // 32-bit load offsets: the gathered source must span fewer than 2^32 bytes
  const uint64_t hrow = CH == kChainF32 ? 2ull * I : (uint64_t)I;
  const bool small_src = (uint64_t)T * D * 2 < (1ull << 32) && (uint64_t)M * hrow * 2 < (1ull << 32);
  if (I % 128 == 0 && D % 256 == 0 && small_src) {
    // weights that only one row tile per expert reads (up to 64 rows per
    // expert on average) stream past the caches: T = 256 / 512 / 1024 gain
    // 14 / 9 / 6 us per layer; at 128 rows per expert (T = 2048) the second
    // tiles of the busier experts lose their L2 hits (+8 us)
    const bool ntb = M <= E * kGemmRows / 2;
    // 160-row tiles from 96 rows per expert on average: an expert's rows take
    // fewer tiles, each converting the same weight chunks (T = 1536 / 2048 /
    // 4096: 308 -> 294, 339 -> 328, 550 -> 509 us per layer; 235B-A22B at
    // T = 2048 1051 -> 937 us); below that the three-deep weight ring of the
    // 128-row form hides more of the weight stream's latency
    const bool big = M >= E * 96;
    // with up to 128 rows per expert on average a 160-row tile is mostly the
    // expert's only one: its weights stream past the caches as well
    const bool ntb160 = big && M <= E * 128;
    // 64-row tiles up to 44 rows per expert on average (48 KB of LDS, three
    // blocks per CU, so the grid's tiles are all resident at once and stream
    // their weights together): T = 256 / 512 / 576 / 640 / 704 159 -> 151,
    // 169 -> 156, 179 -> 168, 181 -> 169, 187 -> 174 us per layer; at 48 and
    // 64 rows per expert (T = 768 / 1024) they lose 9 / 18 us
    const bool s64 = M <= E * 44;
    const int rw = big ? 160 : (s64 ? 64 : kGemmRows);
    const int upper_mt = (M + rw - 1) / rw + slots;
    auto grid_for = [&](int NT) { return ((upper_mt * NT + 7) / 8) * 8; };
    if (stages & kStageGateUp) {
      if (s64)
        hipLaunchKernelGGL((k_gemm<true, true, CH, 64>), dim3(grid_for(I / 128)), dim3(256), 0, st, D, I, E, xb,
                           offsets, sorted_token, w13, s13, hb, cap, nullptr);
      else if (ntb)
        hipLaunchKernelGGL((k_gemm<true, true, CH, 128>), dim3(grid_for(I / 128)), dim3(256), 0, st, D, I, E, xb,
                           offsets, sorted_token, w13, s13, hb, cap, nullptr);
      else if (ntb160)
        hipLaunchKernelGGL((k_gemm<true, true, CH, 160>), dim3(grid_for(I / 128)), dim3(256), 0, st, D, I, E, xb,
                           offsets, sorted_token, w13, s13, hb, cap, nullptr);
      else if (big)
        hipLaunchKernelGGL((k_gemm<true, false, CH, 160>), dim3(grid_for(I / 128)), dim3(256), 0, st, D, I, E, xb,
                           offsets, sorted_token, w13, s13, hb, cap, nullptr);
      else
        hipLaunchKernelGGL((k_gemm<true, false, CH, 128>), dim3(grid_for(I / 128)), dim3(256), 0, st, D, I, E, xb,
                           offsets, sorted_token, w13, s13, hb, cap, nullptr);
      hipError_t err = hipGetLastError();
      if (err != hipSuccess) return err;
    }
    if (stages & kStageDown) {
      if (CH == kChainF32 && hs != nullptr && down_planes_fits(d)) {
        // h as two int8 planes with a per-row scale (in place), then the
        // integer down product on 64-row tiles
        hipLaunchKernelGGL(k_h_planes, dim3((M + 3) / 4), dim3(256), 0, st, M, I, hb, hs);
        hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
        const int mt64 = (M + 63) / 64 + slots;
        hipLaunchKernelGGL((k_gemm<false, false, kChainF32, 64, true>), dim3(((mt64 * (D / 256) + 7) / 8) * 8),
                           dim3(256), 0, st, D, I, E, hb, offsets, sorted_token, w2, s2, yb, cap, hs);
        return hipGetLastError();
      }
      if (s64)
        hipLaunchKernelGGL((k_gemm<false, true, CH, 64>), dim3(grid_for(D / 256)), dim3(256), 0, st, D, I, E, hb,
                           offsets, sorted_token, w2, s2, yb, cap, nullptr);
      else if (ntb)
        hipLaunchKernelGGL((k_gemm<false, true, CH, 128>), dim3(grid_for(D / 256)), dim3(256), 0, st, D, I, E, hb,
                           offsets, sorted_token, w2, s2, yb, cap, nullptr);
      else if (ntb160)
        hipLaunchKernelGGL((k_gemm<false, true, CH, 160>), dim3(grid_for(D / 256)), dim3(256), 0, st, D, I, E, hb,
                           offsets, sorted_token, w2, s2, yb, cap, nullptr);
      else if (big)
        hipLaunchKernelGGL((k_gemm<false, false, CH, 160>), dim3(grid_for(D / 256)), dim3(256), 0, st, D, I, E, hb,
                           offsets, sorted_token, w2, s2, yb, cap, nullptr);
      else
        hipLaunchKernelGGL((k_gemm<false, false, CH, 128>), dim3(grid_for(D / 256)), dim3(256), 0, st, D, I, E, hb,
                           offsets, sorted_token, w2, s2, yb, cap, nullptr);
      return hipGetLastError();
    }
    return hipSuccess;
  }
  const int upper_mt = (M + kBM - 1) / kBM + slots;
  auto grid_for = [&](int NT) {
    int g = upper_mt * NT;
    return ((g + 7) / 8) * 8;
  };
  if (stages & kStageGateUp) {
    hipLaunchKernelGGL((k_prefill<true, CH>), dim3(grid_for(I / 64)), dim3(256), 0, st, D, I, E, xb, offsets,
                       sorted_token, w13, s13, hb, cap);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  if (stages & kStageDown) {
    hipLaunchKernelGGL((k_prefill<false, CH>), dim3(grid_for(D / 128)), dim3(256), 0, st, D, I, E, hb, offsets,
                       sorted_token, w2, s2, yb, cap);
    return hipGetLastError();
  }
  return hipSuccess;
}

}  // namespace

hipError_t launch_expert_packed(const kmoe_desc& d, int chain, int family, int stages, const void* x,
                                const int32_t* offsets, const int32_t* active, const int32_t* sorted_token,
                                const kmoe_packed_experts& p, void* h_sorted, void* y_sorted, hipStream_t st,
                                float* h_scale) {
  const uint16_t* xb = reinterpret_cast<const uint16_t*>(x);
  uint16_t* hb = reinterpret_cast<uint16_t*>(h_sorted);
  uint16_t* yb = reinterpret_cast<uint16_t*>(y_sorted);
  const int8_t* w13 = reinterpret_cast<const int8_t*>(p.w13);
  const int8_t* w2 = reinterpret_cast<const int8_t*>(p.w2);
  const float* s13 = reinterpret_cast<const float*>(p.s13);
  const float* s2 = reinterpret_cast<const float*>(p.s2);
  if (chain == kChainF32)
    return packed_stages<kChainF32>(d, family, stages, xb, offsets, active, sorted_token, w13, s13, w2, s2, hb, yb,
                                    h_scale, st);
  return packed_stages<kChainAct>(d, family, stages, xb, offsets, active, sorted_token, w13, s13, w2, s2, hb, yb,
                                  nullptr, st);
}

static WView make_view(const kmoe_weight& w) {
  WView v;
  v.v = w.values;
  v.s = w.scale;
  v.wt = w.dtype == KMOE_DTYPE_F32 ? 0 : (w.dtype == KMOE_DTYPE_BF16 ? 1 : 2);
  v.s_bf16 = (w.dtype == KMOE_DTYPE_I8 && w.scale_dtype == KMOE_DTYPE_BF16) ? 1 : 0;
  v.per_channel = (w.dtype == KMOE_DTYPE_I8 && w.scale_kind == KMOE_SCALE_CHANNEL) ? 1 : 0;
  return v;
}

template <typename A, int CH>
static hipError_t generic_stages(int stages, int D, int I, int M, const void* x, const int32_t* sorted_token,
                                 const int32_t* sorted_expert, const WView& wg, const WView& wu, const WView& wd,
                                 void* h_sorted, void* y_sorted, hipStream_t st) {
  if (stages & kStageGateUp) {
    hipLaunchKernelGGL((k_gateup_generic<A, CH>), dim3((I + 255) / 256, M), dim3(256), 0, st, D, I,
                       reinterpret_cast<const A*>(x), sorted_token, sorted_expert, wg, wu,
                       reinterpret_cast<A*>(h_sorted));
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  if (stages & kStageDown) {
    hipLaunchKernelGGL((k_down_generic<A, CH>), dim3((D + 255) / 256, M), dim3(256), 0, st, D, I,
                       reinterpret_cast<const A*>(h_sorted), sorted_expert, wd, reinterpret_cast<A*>(y_sorted));
    return hipGetLastError();
  }
  return hipSuccess;
}

hipError_t launch_expert_generic(const kmoe_desc& d, int chain, int stages, const void* x, const int32_t* sorted_token,
                                 const int32_t* sorted_expert, const kmoe_weight* gate, const kmoe_weight* up,
                                 const kmoe_weight* down, void* h_sorted, void* y_sorted, hipStream_t st) {
  const int T = (int)d.tokens, D = (int)d.hidden, K = (int)d.top_k, I = (int)d.intermediate;
  const int M = T * K;
  const WView none = {nullptr, nullptr, 0, 0, 0};
  const WView wg = gate ? make_view(*gate) : none, wu = up ? make_view(*up) : none,
              wd = down ? make_view(*down) : none;
  if (d.act_dtype == KMOE_DTYPE_BF16) {
    if (chain == kChainF32)
      return generic_stages<uint16_t, kChainF32>(stages, D, I, M, x, sorted_token, sorted_expert, wg, wu, wd,
                                                 h_sorted, y_sorted, st);
    return generic_stages<uint16_t, kChainAct>(stages, D, I, M, x, sorted_token, sorted_expert, wg, wu, wd, h_sorted,
                                               y_sorted, st);
  }
  // f32 activations: every chain computes in f32
  return generic_stages<float, kChainF32>(stages, D, I, M, x, sorted_token, sorted_expert, wg, wu, wd, h_sorted,
                                          y_sorted, st);
}

template <typename A, bool SCATTER>
static void combine_launch(const kmoe_desc& d, const void* y_sorted, const int32_t* inv, const float* topk_w,
                           void* out, hipStream_t st, const void* res) {
  const int T = (int)d.tokens, D = (int)d.hidden, K = (int)d.top_k;
  const A* y = reinterpret_cast<const A*>(y_sorted);
  A* o = reinterpret_cast<A*>(out);
  const A* r = reinterpret_cast<const A*>(res);
  if (D % 8 == 0)
    hipLaunchKernelGGL((k_combine8<A, SCATTER>), dim3((D / 8 + 255) / 256, T), dim3(256), 0, st, T, K, D, y, inv,
                       topk_w, o, r);
  else
    hipLaunchKernelGGL((k_combine1<A, SCATTER>), dim3((D + 255) / 256, T), dim3(256), 0, st, T, K, D, y, inv, topk_w,
                       o, r);
}

hipError_t launch_combine(const kmoe_desc& d, bool scatter, const void* y_sorted, const int32_t* inv,
                          const float* topk_w, void* out, hipStream_t st, const void* res) {
  if (d.act_dtype == KMOE_DTYPE_BF16) {
    if (scatter)
      combine_launch<uint16_t, true>(d, y_sorted, inv, topk_w, out, st, res);
    else
      combine_launch<uint16_t, false>(d, y_sorted, inv, topk_w, out, st, res);
  } else {
    // f32: a rounded running sum is the f32 sum
    combine_launch<float, false>(d, y_sorted, inv, topk_w, out, st, res);
  }
  return hipGetLastError();
}

// the weights of a wave's chunks (half the reduction) stay in registers: at
// most 12 chunks of 64; a block holds the 8 / K tokens of up to 8 assignments
// and their h rows (both planes for kChainF32) in LDS
bool down_combine_fits(const kmoe_desc& d, int chain) {
  const int64_t M = d.tokens * d.top_k, KC = d.intermediate / 64;
  const int64_t planes = chain == kChainF32 ? 2 : 1;
  return d.top_k >= 1 && d.top_k <= kDownCombineMaxRows && M <= kDownCombineMaxAssignments && KC <= 24 &&
         (int64_t)kDownCombineMaxRows * planes * d.intermediate * 2 <= 65536;
}

template <int KCMAX, int CH, bool SCATTER>
static void down_combine_launch(dim3 grid, dim3 block, size_t lds, hipStream_t st, int T, int K, int TPB, int D,
                                int I, const uint16_t* hb, const int32_t* topk_idx, const int32_t* inv,
                                const float* topk_w, const int8_t* w2, const float* s2, uint16_t* ob,
                                const uint16_t* rb) {
  hipLaunchKernelGGL((k_down_combine<KCMAX, CH, SCATTER>), grid, block, lds, st, T, K, TPB, D, I, hb, topk_idx, inv,
                     topk_w, w2, s2, ob, rb);
}

template <int KCMAX>
static void down_combine_modes(int chain, bool scatter, dim3 grid, dim3 block, size_t lds, hipStream_t st, int T,
                               int K, int TPB, int D, int I, const uint16_t* hb, const int32_t* topk_idx,
                               const int32_t* inv, const float* topk_w, const int8_t* w2, const float* s2,
                               uint16_t* ob, const uint16_t* rb) {
  if (chain == kChainF32) {
    if (scatter)
      down_combine_launch<KCMAX, kChainF32, true>(grid, block, lds, st, T, K, TPB, D, I, hb, topk_idx, inv, topk_w,
                                                  w2, s2, ob, rb);
    else
      down_combine_launch<KCMAX, kChainF32, false>(grid, block, lds, st, T, K, TPB, D, I, hb, topk_idx, inv, topk_w,
                                                   w2, s2, ob, rb);
  } else {
    if (scatter)
      down_combine_launch<KCMAX, kChainAct, true>(grid, block, lds, st, T, K, TPB, D, I, hb, topk_idx, inv, topk_w,
                                                  w2, s2, ob, rb);
    else
      down_combine_launch<KCMAX, kChainAct, false>(grid, block, lds, st, T, K, TPB, D, I, hb, topk_idx, inv, topk_w,
                                                   w2, s2, ob, rb);
  }
}

hipError_t launch_down_combine(const kmoe_desc& d, int chain, bool scatter, const void* h_sorted,
                               const int32_t* topk_idx, const int32_t* inv, const float* topk_w,
                               const kmoe_packed_experts& p, void* out, hipStream_t st, const void* res) {
  const int T = (int)d.tokens, K = (int)d.top_k, D = (int)d.hidden, I = (int)d.intermediate;
  if (!down_combine_fits(d, chain)) return hipErrorInvalidValue;
  const int TPB = std::min(T, kDownCombineMaxRows / K);
  const dim3 grid(D / 16, (T + TPB - 1) / TPB), block(128 * TPB * K);
  const size_t lds = (size_t)TPB * K * I * 2 * (chain == kChainF32 ? 2 : 1);
  const uint16_t* hb = reinterpret_cast<const uint16_t*>(h_sorted);
  const int8_t* w2 = reinterpret_cast<const int8_t*>(p.w2);
  const float* s2 = reinterpret_cast<const float*>(p.s2);
  uint16_t* ob = reinterpret_cast<uint16_t*>(out);
  const uint16_t* rb = reinterpret_cast<const uint16_t*>(res);
  if (I / 64 <= 12)
    down_combine_modes<6>(chain, scatter, grid, block, lds, st, T, K, TPB, D, I, hb, topk_idx, inv, topk_w, w2, s2,
                          ob, rb);
  else
    down_combine_modes<12>(chain, scatter, grid, block, lds, st, T, K, TPB, D, I, hb, topk_idx, inv, topk_w, w2, s2,
                           ob, rb);
  return hipGetLastError();
}

// Compute units of the current device (cached per device).
static int cu_count() {
  constexpr int kDevices = 64;
  static std::atomic<int> cache[kDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kDevices) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

bool gateup_routed_fits(const kmoe_desc& d) {
  return d.tokens >= 1 && d.tokens <= 4 && d.act_dtype == KMOE_DTYPE_BF16 &&
         (d.hidden == 32 * 64 || d.hidden == 64 * 64) && d.intermediate % 16 == 0 && d.top_k >= 1 &&
         d.top_k <= kmoe::kMaxTopK && d.num_experts <= kmoe::kMaxExperts;
}

template <int EPL, int CH>
static void routed_launch(const kmoe_desc& d, int Q, const float* part, const uint16_t* xb, const int8_t* w13,
                          const float* s13, uint16_t* hb, int32_t* tidx, float* tw, const DispatchOut& o,
                          hipStream_t st) {
  const int T = (int)d.tokens, D = (int)d.hidden, E = (int)d.num_experts, K = (int)d.top_k,
            I = (int)d.intermediate;
  // at most min(T*K, E) active experts; two blocks per CU are resident
  const int items = (I / 16) * std::min(T * K, E);
  const dim3 grid(std::min(items, 2 * cu_count()));
  // load batches of four chunks at both hidden sizes (two per wave at D = 4096)
  hipLaunchKernelGGL((k_gateup_routed<EPL, 4, CH>), grid, dim3(512), 0, st, T, D, I, E, K, Q, part, 1, xb, w13, s13,
                     hb, capacity_of(d), tidx, tw, o.group_sizes, o.offsets, o.active, o.sorted_token,
                     o.sorted_expert, o.inv);
}

template <int CH>
static void routed_epl(const kmoe_desc& d, int Q, const float* part, const uint16_t* xb, const int8_t* w13,
                       const float* s13, uint16_t* hb, int32_t* tidx, float* tw, const DispatchOut& o,
                       hipStream_t st) {
  const int E = (int)d.num_experts;
  if (E <= 64)
    routed_launch<1, CH>(d, Q, part, xb, w13, s13, hb, tidx, tw, o, st);
  else if (E <= 128)
    routed_launch<2, CH>(d, Q, part, xb, w13, s13, hb, tidx, tw, o, st);
  else if (E <= 256)
    routed_launch<4, CH>(d, Q, part, xb, w13, s13, hb, tidx, tw, o, st);
  else if (E <= 512)
    routed_launch<8, CH>(d, Q, part, xb, w13, s13, hb, tidx, tw, o, st);
  else
    routed_launch<16, CH>(d, Q, part, xb, w13, s13, hb, tidx, tw, o, st);
}

hipError_t launch_gateup_routed(const kmoe_desc& d, int chain, const float* part, const void* x,
                                const kmoe_packed_experts& p, void* h_sorted, int32_t* topk_idx, float* topk_w,
                                const DispatchOut& dout, hipStream_t st) {
  if (!gateup_routed_fits(d)) return hipErrorInvalidValue;
  const int Q = route_split_groups(d);
  const uint16_t* xb = reinterpret_cast<const uint16_t*>(x);
  const int8_t* w13 = reinterpret_cast<const int8_t*>(p.w13);
  const float* s13 = reinterpret_cast<const float*>(p.s13);
  uint16_t* hb = reinterpret_cast<uint16_t*>(h_sorted);
  if (chain == kChainF32)
    routed_epl<kChainF32>(d, Q, part, xb, w13, s13, hb, topk_idx, topk_w, dout, st);
  else
    routed_epl<kChainAct>(d, Q, part, xb, w13, s13, hb, topk_idx, topk_w, dout, st);
  return hipGetLastError();
}

hipError_t launch_topk_w_cast(const kmoe_desc& d, const float* topk_w, void* out, hipStream_t st) {
  const int64_t n = d.tokens * d.top_k;
  const int blocks = (int)((n + 255) / 256);
  if (d.act_dtype == KMOE_DTYPE_BF16)
    hipLaunchKernelGGL((k_cast_from_f32<uint16_t>), dim3(blocks), dim3(256), 0, st, n, topk_w,
                       reinterpret_cast<uint16_t*>(out));
  else
    hipLaunchKernelGGL((k_cast_from_f32<float>), dim3(blocks), dim3(256), 0, st, n, topk_w,
                       reinterpret_cast<float*>(out));
  return hipGetLastError();
}

}  // namespace kmoe_host
