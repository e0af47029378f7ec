/*
 * CPU oracle for the Qwen3 MoE feed-forward block.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker that the HIP library in
 * kappa_amd/ is compared against; it is never part of the product path. Only
 * tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py load it.
 *
 * It restates, in plain C, the arithmetic of the reference layer
 *   moe_swiglu_ffn(x, router_w, ffn_gate, ffn_up, ffn_down, *, cfg)
 *   (kappa/qwen3/ffn_moe.py:226-299)
 * following the rounding points each implementation of the reference writes
 * down (kappa/qwen3/ffn_moe.py): the router is shared, the expert products and
 * the combine depend on the MoEImpl that runs (after the decode switch of
 * _effective_moe_impl, :219-223).
 *
 * Router (_route, :38-56), every impl:
 *  N0 logits[t,e] = sum_d f32(x[t,d]) * r[d,e]   (:50)
 *     in a canonical order: D is cut into slices of 64; each slice is a
 *     sequential fmaf chain starting from +0.0f; slice partials are combined
 *     by a pairwise tree (p[i] += p[i+s], s = 1,2,4,...), zero-padded to a
 *     power of two.  r = to_compute_dtype(router_w, f32)
 *     (:46, kappa/qwen3/quant.py:34-38).
 *  N1 top-k by value, descending, ties to the lower expert index
 *     (jax.lax.top_k, :51).
 *  N2 w = act(softmax_f32(top_logits)) (:52):
 *     e_j = expf(l_j - l_0), s = sum_j e_j in j order, w_j = e_j / s.
 *  N3 dispatch = stable sort of the row-major (t, j) assignment list by expert
 *     (jnp.argsort(stable=True), :196-200, 212; jnp.lexsort((token, expert)),
 *     :130, gives the same order).
 *
 * act(v) rounds to the activation dtype: the identity for f32 activations,
 * round-to-nearest-even to bfloat16 for bf16 activations. Every bf16 value is
 * carried in a float. Each jnp operation of the written program rounds its
 * result to its array dtype; XLA may legally keep more precision inside a
 * fusion, which no file of the reference pins.
 *
 * Expert products, ORC_CHAIN_ACT (gather_einsum :74-104 through
 * moe_take_dequant, kappa/qwen3/quant.py:60-76; fixed_capacity :146-152
 * through to_compute_dtype(., x.dtype)):
 *  W = act(f32(q) * act(s))  (the scale cast to x.dtype first, quant.py:37,74)
 *  g = act(sum_d x*W), u likewise (sequential fmaf over d from +0.0f)
 *  h = act(act(g * act(sigmoid(g))) * u)   (jax.nn.silu(g) * u, :101, :151:
 *      silu(g) = g * sigmoid(g), each op in x.dtype)
 *  y = act(sum_i h*Wd)
 * Expert products, ORC_CHAIN_F32 (_moe_ragged :202-213):
 *  W = f32(q) * f32(s) in f32 (to_compute_dtype(., f32), :203-205)
 *  g, u = sum_d f32(x)*W in f32; h = (g * sigmoid(g)) * u in f32 (:209)
 *  y = act(sum_i h*Wd) (the f32 ragged_dot, then y.astype(x.dtype), :210-213)
 * sigmoid(g) = 1 / (1 + expf(-g)) in f32.
 *
 * Combine, ORC_COMBINE_SUM (gather_einsum, :103):
 *  p_j = act(y_j * w_j); out = act(sum_j f32(p_j)) summed in j order from
 *  +0.0f (jnp.sum of a bf16 array accumulates in f32 and rounds once).
 * Combine, ORC_COMBINE_SCATTER (_moe_ragged :214-215, fixed_capacity :156-157):
 *  p_j = act(y_j * w_j); o = 0; o = act(o + p_j) for j = 0..K-1
 *  (out_flat.at[token_flat].add in x.dtype: each update rounds; the updates
 *  of token t arrive in j order). A dropped assignment (fixed_capacity,
 *  y_pick = 0, :153) contributes act(0 * w) = 0 and is skipped.
 *
 * Around the block (the steps on either side of it in a Qwen3 MoE layer,
 * kappa/qwen3/block.py:196-207):
 *  R1 h2 = rms_norm(h, scale, eps) (kappa/qwen3/norms.py:10-16):
 *     S = sum_d f32(h_d)*f32(h_d) with every square rounded to float and the
 *     sum in the N0 order (slices of 64, each a sequential chain of adds from
 *     +0.0f, slice sums combined by the zero-padded pairwise tree);
 *     var = S / D; r = 1 / sqrtf(var + eps) (IEEE division and square root);
 *     h2_d = round_act((f32(h_d) * r) * f32(scale_d)).
 *  R2 out = round_act(f32(h) + f32(moe_out)), moe_out already round_act.
 *
 * Each output element is produced by exactly one thread in a fixed order, so
 * results do not depend on the OpenMP thread count.
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_SLICE 64

/* Round-to-nearest-even float -> bfloat16, returned widened to float. */
static inline float bf16r(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u) {
    if (u & 0x007fffffu) u |= 0x00400000u;
    u &= 0xffff0000u;
  } else {
    u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
  }
  memcpy(&f, &u, 4);
  return f;
}

float orc_bf16_round(float f) { return bf16r(f); }

void orc_bf16_round_array(int64_t n, const float* in, float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = bf16r(in[i]);
}

void orc_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

int orc_get_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* Expert-product chains and combines (see the header). */
#define ORC_CHAIN_ACT 0
#define ORC_CHAIN_F32 1
#define ORC_COMBINE_SUM 0
#define ORC_COMBINE_SCATTER 1

/* One weight tensor [E][Kd][N]: either plain floats (wf != NULL) or int8
 * values wq with one f32 scale per (expert, output channel) ws[e*N + n].
 * A per-tensor scale is passed as a per-channel array with equal entries
 * (kappa/qwen3/quant.py:15-19 stores one scalar; broadcasting it is exact).
 * act_w: dequantise to the activation dtype (ORC_CHAIN_ACT with bf16
 * activations, values.astype(bf16) * scale.astype(bf16)); otherwise to f32. */
static inline float deq(const float* wf, const int8_t* wq, const float* ws, int64_t idx, int64_t sidx,
                        int act_w) {
  if (wf) return act_w ? bf16r(wf[idx]) : wf[idx];
  float q = (float)wq[idx];
  if (act_w) return bf16r(q * bf16r(ws[sidx]));
  return q * ws[sidx];
}

/* N0: router logits in the canonical slice/tree order.
 * Router weight [D][E]: plain floats rf, or int8 rq with per-expert scale rs[e]
 * (a per-tensor scale is passed expanded). Dequant is f32(q) * f32(s). */
void orc_router_logits(int64_t T, int64_t D, int64_t E, const float* x, const float* rf, const int8_t* rq,
                       const float* rs, float* logits) {
  int64_t S = (D + ORC_SLICE - 1) / ORC_SLICE;
  int64_t P = 1;
  while (P < S) P <<= 1;
#pragma omp parallel
  {
    float* part = (float*)malloc(sizeof(float) * (size_t)(P * E));
    float* rrow = (float*)malloc(sizeof(float) * (size_t)E);
#pragma omp for schedule(static)
    for (int64_t t = 0; t < T; ++t) {
      for (int64_t i = 0; i < P * E; ++i) part[i] = 0.0f;
      for (int64_t s = 0; s < S; ++s) {
        float* acc = part + s * E;
        int64_t d1 = (s + 1) * ORC_SLICE < D ? (s + 1) * ORC_SLICE : D;
        for (int64_t d = s * ORC_SLICE; d < d1; ++d) {
          float xv = x[t * D + d];
          if (rf) {
            const float* r = rf + d * E;
            for (int64_t e = 0; e < E; ++e) acc[e] = fmaf(xv, r[e], acc[e]);
          } else {
            const int8_t* r = rq + d * E;
            for (int64_t e = 0; e < E; ++e) rrow[e] = (float)r[e] * rs[e];
            for (int64_t e = 0; e < E; ++e) acc[e] = fmaf(xv, rrow[e], acc[e]);
          }
        }
      }
      for (int64_t st = 1; st < P; st <<= 1)
        for (int64_t i = 0; i + st < P; i += 2 * st)
          for (int64_t e = 0; e < E; ++e) part[i * E + e] = part[i * E + e] + part[(i + st) * E + e];
      memcpy(logits + t * E, part, sizeof(float) * (size_t)E);
    }
    free(part);
    free(rrow);
  }
}

/* N1 + N2: top-k selection (ties to the lower index) and renormalised weights. */
void orc_topk_softmax(int64_t T, int64_t E, int64_t K, int round_bf16, const float* logits, int32_t* idx,
                      float* w) {
#pragma omp parallel
  {
    unsigned char* taken = (unsigned char*)malloc((size_t)E);
    float* top = (float*)malloc(sizeof(float) * (size_t)K);
#pragma omp for schedule(static)
    for (int64_t t = 0; t < T; ++t) {
      const float* l = logits + t * E;
      memset(taken, 0, (size_t)E);
      for (int64_t j = 0; j < K; ++j) {
        int64_t best = -1;
        for (int64_t e = 0; e < E; ++e) {
          if (taken[e]) continue;
          if (best < 0 || l[e] > l[best]) best = e;
        }
        taken[best] = 1;
        idx[t * K + j] = (int32_t)best;
        top[j] = l[best];
      }
      float m = top[0];
      float s = 0.0f;
      for (int64_t j = 0; j < K; ++j) {
        top[j] = expf(top[j] - m);
        s = s + top[j];
      }
      for (int64_t j = 0; j < K; ++j) {
        float v = top[j] / s;
        w[t * K + j] = round_bf16 ? bf16r(v) : v;
      }
    }
    free(taken);
    free(top);
  }
}

/* N3: stable counting sort of assignments m = t*K + j by expert.
 * group_sizes[e]  = number of assignments to expert e (jnp.bincount)
 * offsets[e]      = exclusive prefix sum, offsets[E] = T*K
 * order[p]        = assignment index m at sorted position p (the argsort)
 * sorted_token[p] = order[p] / K,  inv[m] = p (kappa/qwen3/ffn_moe.py:212). */
void orc_dispatch(int64_t T, int64_t K, int64_t E, const int32_t* idx, int32_t* group_sizes, int32_t* offsets,
                  int32_t* order, int32_t* sorted_token, int32_t* inv) {
  int64_t M = T * K;
  for (int64_t e = 0; e < E; ++e) group_sizes[e] = 0;
  for (int64_t m = 0; m < M; ++m) group_sizes[idx[m]]++;
  offsets[0] = 0;
  for (int64_t e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + group_sizes[e];
  int32_t* fill = (int32_t*)malloc(sizeof(int32_t) * (size_t)(E > 0 ? E : 1));
  for (int64_t e = 0; e < E; ++e) fill[e] = offsets[e];
  for (int64_t m = 0; m < M; ++m) {
    int32_t p = fill[idx[m]]++;
    order[p] = (int32_t)m;
    sorted_token[p] = (int32_t)(m / K);
    inv[m] = p;
  }
  free(fill);
}

static inline float sigmoid_f32(float g) { return 1.0f / (1.0f + expf(-g)); }

/* h from g and u (jax.nn.silu(g) * u, kappa/qwen3/ffn_moe.py:101, 151, 209):
 * silu(g) = g * sigmoid(g); every product rounded to act (ORC_CHAIN_ACT with
 * bf16 activations) or to f32. */
static inline float swiglu(float g, float u, int act) {
  if (act) {
    const float sg = bf16r(g * bf16r(sigmoid_f32(g)));
    return bf16r(sg * u);
  }
  const float sg = g * sigmoid_f32(g);
  return sg * u;
}

/* Expert products over the sorted rows: h_sorted [M][I], y_sorted [M][D].
 * Weights: gate/up [E][D][I], down [E][I][D] (kappa/qwen3/weights.py:58-62,
 * kappa/checkpoint/qwen_hf_convert.py:212-218); each is plain (f) or int8
 * values (q) with per-(expert, output channel) scales (s).
 * chain ORC_CHAIN_ACT: _moe_gather_einsum / _moe_fixed_capacity rounding
 * points (kappa/qwen3/ffn_moe.py:99-102, 149-152); ORC_CHAIN_F32:
 * _moe_ragged (:202-213). h_sorted holds f32 values under ORC_CHAIN_F32. */
#define ORC_ROWS 4
void orc_expert_ffn(int64_t T, int64_t D, int64_t E, int64_t K, int64_t I, int round_bf16, int chain,
                    const float* x, const int32_t* offsets, const int32_t* sorted_token, const float* gf,
                    const int8_t* gq, const float* gs, const float* uf, const int8_t* uq, const float* us,
                    const float* df, const int8_t* dq, const float* ds, float* h_sorted, float* y_sorted) {
  (void)T;
  (void)K;
  /* the arrays that carry x.dtype in the written program */
  const int act = round_bf16 && chain == ORC_CHAIN_ACT;
  int64_t nblocks_total = 0;
  for (int64_t e = 0; e < E; ++e) nblocks_total += (offsets[e + 1] - offsets[e] + ORC_ROWS - 1) / ORC_ROWS;
  /* flatten (expert, row block) pairs so that OpenMP balances skewed groups */
  int64_t* blk_e = (int64_t*)malloc(sizeof(int64_t) * (size_t)(nblocks_total > 0 ? nblocks_total : 1));
  int64_t* blk_m = (int64_t*)malloc(sizeof(int64_t) * (size_t)(nblocks_total > 0 ? nblocks_total : 1));
  int64_t nb = 0;
  for (int64_t e = 0; e < E; ++e)
    for (int64_t m = offsets[e]; m < offsets[e + 1]; m += ORC_ROWS) {
      blk_e[nb] = e;
      blk_m[nb] = m;
      ++nb;
    }
#pragma omp parallel
  {
    float* wrow = (float*)malloc(sizeof(float) * (size_t)(2 * I > D ? 2 * I : D));
    float* accg = (float*)malloc(sizeof(float) * (size_t)(ORC_ROWS * I));
    float* accu = (float*)malloc(sizeof(float) * (size_t)(ORC_ROWS * I));
    float* accy = (float*)malloc(sizeof(float) * (size_t)(ORC_ROWS * D));
#pragma omp for schedule(dynamic, 1)
    for (int64_t b = 0; b < nb; ++b) {
      int64_t e = blk_e[b], m0 = blk_m[b];
      int64_t nr = offsets[e + 1] - m0;
      if (nr > ORC_ROWS) nr = ORC_ROWS;
      for (int64_t i = 0; i < ORC_ROWS * I; ++i) accg[i] = accu[i] = 0.0f;
      for (int64_t d = 0; d < D; ++d) {
        int64_t base = (e * D + d) * I;
        float* wg = wrow;
        float* wu = wrow + I;
        for (int64_t i = 0; i < I; ++i) {
          wg[i] = deq(gf, gq, gs, base + i, e * I + i, act);
          wu[i] = deq(uf, uq, us, base + i, e * I + i, act);
        }
        for (int64_t r = 0; r < nr; ++r) {
          float xv = x[(int64_t)sorted_token[m0 + r] * D + d];
          float* ag = accg + r * I;
          float* au = accu + r * I;
          for (int64_t i = 0; i < I; ++i) {
            ag[i] = fmaf(xv, wg[i], ag[i]);
            au[i] = fmaf(xv, wu[i], au[i]);
          }
        }
      }
      for (int64_t r = 0; r < nr; ++r) {
        float* hr = h_sorted + (m0 + r) * I;
        for (int64_t i = 0; i < I; ++i) {
          float g = accg[r * I + i], u = accu[r * I + i];
          if (act) {
            g = bf16r(g);
            u = bf16r(u);
          }
          hr[i] = swiglu(g, u, act);
        }
      }
      for (int64_t i = 0; i < ORC_ROWS * D; ++i) accy[i] = 0.0f;
      for (int64_t i = 0; i < I; ++i) {
        int64_t base = (e * I + i) * D;
        for (int64_t n = 0; n < D; ++n) wrow[n] = deq(df, dq, ds, base + n, e * D + n, act);
        for (int64_t r = 0; r < nr; ++r) {
          float hv = h_sorted[(m0 + r) * I + i];
          float* ay = accy + r * D;
          for (int64_t n = 0; n < D; ++n) ay[n] = fmaf(hv, wrow[n], ay[n]);
        }
      }
      for (int64_t r = 0; r < nr; ++r) {
        float* yr = y_sorted + (m0 + r) * D;
        for (int64_t n = 0; n < D; ++n) yr[n] = round_bf16 ? bf16r(accy[r * D + n]) : accy[r * D + n];
      }
    }
    free(wrow);
    free(accg);
    free(accu);
    free(accy);
  }
  free(blk_e);
  free(blk_m);
}

/* Weighted combine back to token order (kappa/qwen3/ffn_moe.py:103 with
 * ORC_COMBINE_SUM, :156-157 / :214-215 with ORC_COMBINE_SCATTER). inv < 0
 * marks an assignment dropped by fixed_capacity (y_pick = 0, :153): its
 * product is zero and it is skipped. */
void orc_combine(int64_t T, int64_t K, int64_t D, int round_bf16, int mode, const float* y_sorted, const int32_t* inv,
                 const float* w, float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < T; ++t) {
    for (int64_t n = 0; n < D; ++n) {
      float acc = 0.0f;
      for (int64_t j = 0; j < K; ++j) {
        if (inv[t * K + j] < 0) continue;
        float p = y_sorted[(int64_t)inv[t * K + j] * D + n] * w[t * K + j];
        if (round_bf16) p = bf16r(p);
        acc = acc + p;
        if (mode == ORC_COMBINE_SCATTER && round_bf16) acc = bf16r(acc);
      }
      out[t * D + n] = round_bf16 ? bf16r(acc) : acc;
    }
  }
}

/* R1: rms_norm of each row of h [T][D] (kappa/qwen3/norms.py:10-16). */
void orc_rms_norm(int64_t T, int64_t D, int round_bf16, const float* h, const float* scale, float eps, float* out) {
  const int64_t S = (D + ORC_SLICE - 1) / ORC_SLICE;
  int64_t P = 1;
  while (P < S) P <<= 1;
#pragma omp parallel
  {
    float* part = (float*)calloc((size_t)P, sizeof(float));
#pragma omp for schedule(static)
    for (int64_t t = 0; t < T; ++t) {
      const float* row = h + t * D;
      for (int64_t s = 0; s < P; ++s) {
        float acc = 0.0f;
        if (s < S) {
          const int64_t d1 = (s + 1) * ORC_SLICE < D ? (s + 1) * ORC_SLICE : D;
          for (int64_t d = s * ORC_SLICE; d < d1; ++d) {
            const float sq = row[d] * row[d];
            acc = acc + sq;
          }
        }
        part[s] = acc;
      }
      for (int64_t st = 1; st < P; st <<= 1)
        for (int64_t i = 0; i + st < P; i += 2 * st) part[i] = part[i] + part[i + st];
      const float var = part[0] / (float)D;
      const float r = 1.0f / sqrtf(var + eps);
      for (int64_t d = 0; d < D; ++d) {
        const float n = row[d] * r;
        const float v = n * scale[d];
        out[t * D + d] = round_bf16 ? bf16r(v) : v;
      }
    }
    free(part);
  }
}

/* A7 quantiser, per output channel: amax over the input axis of [E][Kd][N],
 * s = max(amax / 127, FLT_MIN), q = clip(rint(w / s), -128, 127)
 * (kappa/qwen3/quant.py:41-48 with the reduction restricted to one channel). */
void orc_quantize_per_channel(int64_t E, int64_t Kd, int64_t N, const float* w, int8_t* q, float* s) {
#pragma omp parallel for schedule(static)
  for (int64_t e = 0; e < E; ++e) {
    float* se = s + e * N;
    for (int64_t n = 0; n < N; ++n) se[n] = 0.0f;
    for (int64_t k = 0; k < Kd; ++k)
      for (int64_t n = 0; n < N; ++n) {
        float a = fabsf(w[(e * Kd + k) * N + n]);
        if (a > se[n]) se[n] = a;
      }
    for (int64_t n = 0; n < N; ++n) {
      float v = se[n] / 127.0f;
      se[n] = v > FLT_MIN ? v : FLT_MIN;
    }
    for (int64_t k = 0; k < Kd; ++k)
      for (int64_t n = 0; n < N; ++n) {
        float r = rintf(w[(e * Kd + k) * N + n] / se[n]);
        if (r < -128.0f) r = -128.0f;
        if (r > 127.0f) r = 127.0f;
        q[(e * Kd + k) * N + n] = (int8_t)r;
      }
  }
}

/* A7 quantiser as written in the reference: one scale for the whole tensor. */
float orc_quantize_per_tensor(int64_t n, const float* w, int8_t* q) {
  float amax = 0.0f;
  for (int64_t i = 0; i < n; ++i) {
    float a = fabsf(w[i]);
    if (a > amax) amax = a;
  }
  float s = amax / 127.0f;
  if (!(s > FLT_MIN)) s = FLT_MIN;
  for (int64_t i = 0; i < n; ++i) {
    float r = rintf(w[i] / s);
    if (r < -128.0f) r = -128.0f;
    if (r > 127.0f) r = 127.0f;
    q[i] = (int8_t)r;
  }
  return s;
}
