/*
 * kmoe.h -- C ABI of the MI355X (gfx950) Qwen3 MoE feed-forward block.
 *
 * The library replaces the array program behind the reference layer
 *   moe_swiglu_ffn(x, router_w, ffn_gate, ffn_up, ffn_down, *, cfg)
 *   (kappa/qwen3/ffn_moe.py:226-299)
 * with hand-written HIP kernels. Every pointer argument that names a tensor is
 * a device pointer; sizes are element counts. No torch, JAX or HIP types appear
 * in the signatures: a stream is passed as an opaque `void*` (a hipStream_t,
 * NULL for the default stream), so ctypes / cgo / JNI can bind this header
 * without HIP headers.
 *
 * Layouts (kappa/qwen3/weights.py:58-62, kappa/checkpoint/qwen_hf_convert.py:212-218):
 *   x        [T, D]      activations, bf16 or f32 (T = B*L flattened tokens)
 *   router   [D, E]      f32 / bf16, or int8 + scale (Q8Weight, kappa/qwen3/quant.py:15-19)
 *   gate, up [E, D, I]  f32 / bf16, or int8 + scale (per tensor or per output channel)
 *   down     [E, I, D]
 *   out      [T, D]      same dtype as x
 *
 * Ownership: the caller owns every buffer (inputs, outputs, workspace, packed
 * weights). The library never allocates device memory and keeps no per-call
 * state; calls are stream-ordered and asynchronous. Distinct streams with
 * distinct workspaces may be used from several threads at once.
 *
 * Errors: every entry point validates its arguments on the host before any HIP
 * call and returns a status; kmoe_last_error() gives the message of the last
 * failure on the calling thread. Nothing aborts and nothing is swallowed.
 */
#ifndef KMOE_H_
#define KMOE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KMOE_ABI_VERSION 4

typedef enum kmoe_status {
  KMOE_OK = 0,
  KMOE_ERR_INVALID_ARG = 1,          /* shapes, dtypes or pointers are inconsistent */
  KMOE_ERR_UNSUPPORTED = 2,          /* valid request this build does not implement */
  KMOE_ERR_WORKSPACE_TOO_SMALL = 3,  /* workspace_bytes < kmoe_workspace_bytes()    */
  KMOE_ERR_NO_DEVICE = 4,            /* no HIP device is visible                    */
  KMOE_ERR_HIP = 5                   /* a HIP runtime call or kernel launch failed  */
} kmoe_status;

typedef enum kmoe_dtype {
  KMOE_DTYPE_F32 = 0,
  KMOE_DTYPE_BF16 = 1,
  KMOE_DTYPE_I8 = 2
} kmoe_dtype;

typedef enum kmoe_scale_kind {
  KMOE_SCALE_NONE = 0,     /* plain f32 / bf16 weight                        */
  KMOE_SCALE_TENSOR = 1,   /* one scale for the whole tensor (the reference)  */
  KMOE_SCALE_CHANNEL = 2   /* one scale per (expert, output channel): [E, 1, N] */
} kmoe_scale_kind;

/* The array program of the layer, cfg.moe_impl (MoEImpl, kappa/qwen3/architecture.py:14).
 * Each has its own rounding points, which the kernels follow:
 *   GATHER_EINSUM   _moe_gather_einsum (kappa/qwen3/ffn_moe.py:74-104): weights
 *                   bf16(q * bf16(s)); g, u, every step of silu(g) * u and y in x.dtype;
 *                   out = round(sum_k f32(round(y_k * w_k))). Takes plain weights or one
 *                   scale per tensor (moe_take_dequant, kappa/qwen3/quant.py:71-74, does not
 *                   broadcast [E, 1, N] scales against the gathered [T, K, D, I] values).
 *   RAGGED          _moe_ragged (:174-216; ragged_jax and ragged_tokamax): weights
 *                   q * s and g, u, h, y in f32; y rounded to x.dtype; the products
 *                   round(y * w) added into a zero buffer of x.dtype in j order, each add
 *                   rounded. With T <= decode_token_threshold the layer runs
 *                   GATHER_EINSUM instead (_effective_moe_impl, :219-223).
 *   FIXED_CAPACITY  _moe_fixed_capacity (:107-158): the GATHER_EINSUM expert chain on
 *                   each expert's first expert_capacity assignments, the RAGGED combine. */
typedef enum kmoe_impl {
  KMOE_IMPL_GATHER_EINSUM = 0,
  KMOE_IMPL_RAGGED = 1,
  KMOE_IMPL_FIXED_CAPACITY = 2
} kmoe_impl;

/* Kernel family of the expert products. Every family follows the impl's rounding
 * points; they add the same products in different f32 orders, so results agree to
 * rounding but are not bit-identical across families. */
typedef enum kmoe_kernels {
  KMOE_KERNELS_AUTO = 0,     /* by token count: GEMV-style up to 64 tokens, grouped GEMMs above */
  KMOE_KERNELS_DECODE = 1,   /* the GEMV-style kernels (at most 128 tokens; row groups above 64) */
  KMOE_KERNELS_GROUPED = 2   /* the grouped GEMMs at any token count                  */
} kmoe_kernels;

/* A weight operand: `Weight = Array | Q8Weight(values, scale)`
 * (kappa/qwen3/quant.py:15-22). For int8 values the dequantised weight is
 * values * scale with the scale first cast to the compute dtype
 * (kappa/qwen3/quant.py:34-38). */
typedef struct kmoe_weight {
  const void* values;
  kmoe_dtype dtype;            /* F32, BF16 or I8 */
  const void* scale;           /* NULL unless dtype == I8 */
  kmoe_dtype scale_dtype;      /* F32 or BF16 */
  kmoe_scale_kind scale_kind;  /* NONE for F32/BF16 values */
} kmoe_weight;

/* Problem description: the MoE fields of Qwen3Config
 * (kappa/qwen3/architecture.py:36-49) plus the flattened token count. */
typedef struct kmoe_desc {
  int64_t tokens;                 /* T = B*L                                   */
  int64_t hidden;                 /* D = model_dim                             */
  int64_t num_experts;            /* E                                         */
  int64_t top_k;                  /* K = num_experts_per_tok                   */
  int64_t intermediate;           /* I = moe intermediate size                 */
  kmoe_dtype act_dtype;           /* F32 or BF16 (x.dtype)                     */
  kmoe_impl impl;                 /* cfg.moe_impl                              */
  int64_t decode_token_threshold; /* moe_ragged_decode_token_threshold (:49):
                                     impl RAGGED with T <= this runs GATHER_EINSUM */
  int64_t expert_capacity;        /* impl FIXED_CAPACITY: the slot limit
                                     min(c_dyn, c_buf) >= 1 (:136-141); an assignment
                                     whose slot within its expert's stable order is
                                     >= this is dropped and adds nothing to its
                                     token's output. 0 for the other impls. */
  kmoe_kernels kernels;           /* kernel family (AUTO: by token count)      */
} kmoe_desc;

/* W8 expert weights relaid out once, at load time, for the gfx950 kernels
 * (the counterpart of the load-time quantize_qwen3_params step,
 * kappa/qwen3/weights.py:143-188). All four buffers are caller-owned device
 * memory of the sizes kmoe_prepack_bytes() reports:
 *   w13 [E][I/16][2][D/16][16][16] int8  gate (0) and up (1), 16 columns x 16 k per cell
 *   s13 [E][I/16][2][16]           f32   their scales as given (a scalar is repeated)
 *   w2  [E][D/16][I/16][16][16]    int8  down
 *   s2  [E][D]                     f32   its scales
 * The caller also records the shapes the buffers hold and the kind of the source
 * scales; a forward call checks them against its desc and impl. */
typedef struct kmoe_packed_experts {
  void* w13;
  void* s13;
  void* w2;
  void* s2;
  int64_t num_experts;              /* E */
  int64_t hidden;                   /* D */
  int64_t intermediate;             /* I */
  kmoe_scale_kind source_scale_kind; /* TENSOR if all three source scales were scalars, else CHANNEL */
} kmoe_packed_experts;

typedef struct kmoe_packed_sizes {
  size_t w13_bytes, s13_bytes, w2_bytes, s2_bytes;
} kmoe_packed_sizes;

/* --- library information ------------------------------------------------ */
const char* kmoe_version(void);
int kmoe_abi_version(void);
const char* kmoe_status_string(kmoe_status status);
/* Message of the last failing call on this thread ("" if none). */
const char* kmoe_last_error(void);
/* KMOE_OK if a HIP device is usable, KMOE_ERR_NO_DEVICE otherwise. */
kmoe_status kmoe_device_check(void);

/* --- sizes ---------------------------------------------------------------- */
/* Bytes of device workspace kmoe_forward needs for this problem. */
kmoe_status kmoe_workspace_bytes(const kmoe_desc* desc, size_t* bytes);
/* Sizes of the packed expert buffers (requires D % 64 == 0, I % 64 == 0). */
kmoe_status kmoe_prepack_bytes(const kmoe_desc* desc, kmoe_packed_sizes* sizes);

/* --- whole block ---------------------------------------------------------- */
/* moe_swiglu_ffn (kappa/qwen3/ffn_moe.py:226-299): router, top-k with
 * renormalisation, dispatch, SwiGLU experts and the weighted combine, with the
 * rounding points of desc->impl (after the decode switch, :219-223).
 * `packed` may be NULL: int8 experts then run on the layout-native kernels.
 * topk_idx_out [T,K] int32 and topk_w_out [T,K] (x dtype) are optional.
 * GATHER_EINSUM with per-channel scales and more than one expert is
 * KMOE_ERR_INVALID_ARG: the reference's gather program cannot apply them.
 * The RAGGED program with bf16 activations and packed experts feeds its down
 * product h as two int8 planes with one power-of-two scale per row (15 bits
 * of the row's largest |h|) from 96 rows per expert on average (T*K >= 96 E),
 * and as bf16 hi and lo planes below (see kmoe_expert_ffn). */
kmoe_status kmoe_forward(const kmoe_desc* desc, const void* x, const kmoe_weight* router, const kmoe_weight* gate,
                         const kmoe_weight* up, const kmoe_weight* down, const kmoe_packed_experts* packed, void* out,
                         int32_t* topk_idx_out, void* topk_w_out, void* workspace, size_t workspace_bytes,
                         void* stream);

/* kmoe_forward without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). No counterpart in the reference. The workspace is a
 * device array of KMOE_NOALLOC_SCRATCH_BYTES inside the library, one per GPU,
 * held until the process ends; the call allocates and frees nothing. A desc
 * whose kmoe_workspace_bytes exceeds it returns KMOE_ERR_WORKSPACE_TOO_SMALL
 * (with bf16 activations and the ragged program, the 30B-A3B layer fits up to
 * 291 tokens and the 235B-A22B layer up to 136).
 * Every call on one GPU shares the array: calls that overlap on a GPU (other
 * streams, other threads) race and must be serialised by the caller. */
#define KMOE_NOALLOC_SCRATCH_BYTES (16u << 20)
kmoe_status kmoe_forward_noalloc(const kmoe_desc* desc, const void* x, const kmoe_weight* router,
                                 const kmoe_weight* gate, const kmoe_weight* up, const kmoe_weight* down,
                                 const kmoe_packed_experts* packed, void* out, int32_t* topk_idx_out, void* topk_w_out,
                                 void* stream);

/* The MoE half of a Qwen3 MoE layer with the steps on either side of the
 * block fused in (kappa/qwen3/block.py:71-82, 153-164, 196-207):
 *   h2  = rms_norm(h, norm_scale, epsilon)        (kappa/qwen3/norms.py:10-16)
 *   out = h + moe_swiglu_ffn(h2, ...)             (rounded to h.dtype)
 * h and out are [T,D] in the activation dtype (out must not alias h);
 * norm_scale [D] is F32 or BF16 (pre_ffn_norm). h2 lives in the workspace
 * (kmoe_workspace_bytes covers it); the residual add happens in the combine
 * kernel, so the layer's separate add and its [T,D] round trip disappear.
 * topk_idx_out / topk_w_out as for kmoe_forward. */
kmoe_status kmoe_forward_block(const kmoe_desc* desc, const void* h, const void* norm_scale, kmoe_dtype norm_dtype,
                               float epsilon, const kmoe_weight* router, const kmoe_weight* gate,
                               const kmoe_weight* up, const kmoe_weight* down, const kmoe_packed_experts* packed,
                               void* out, int32_t* topk_idx_out, void* topk_w_out, void* workspace,
                               size_t workspace_bytes, void* stream);

/* rms_norm (kappa/qwen3/norms.py:10-16) of x [T,D] into out [T,D] (activation
 * dtype): the squares summed in the router's canonical slice order,
 * r = 1 / sqrt(S / D + epsilon), out = round((x * r) * scale). The first step
 * of kmoe_forward_block, for per-stage parity. */
kmoe_status kmoe_rms_norm(const kmoe_desc* desc, const void* x, const void* scale, kmoe_dtype scale_dtype,
                          float epsilon, void* out, void* stream);

/* --- stages (per-stage parity; kmoe_forward chains exactly these) ------- */
/* _route (kappa/qwen3/ffn_moe.py:38-56): logits [T,E] f32 (optional, may be
 * NULL), topk_idx [T,K] int32, topk_w [T,K] f32 holding values already
 * rounded to x.dtype, block_hist [ceil(T/64), E] int32 (per 64-token chunk
 * expert counts consumed by kmoe_dispatch). `scratch` (optional, may be NULL)
 * of kmoe_route_scratch_bytes(desc) bytes lets a call without logits take the
 * two-phase form when x and the router are bf16, D is 512, 1024, 2048 or
 * 4096, E % 16 == 0 and E <= 256: every logit on the matrix cores, then the
 * canonical order only for the experts within a rigorous f32 error bound of the
 * K-th (the form kmoe_forward uses from 2048 tokens). Selections, weights and
 * block_hist are the same either way. */
kmoe_status kmoe_route(const kmoe_desc* desc, const void* x, const kmoe_weight* router, float* logits,
                       void* scratch, size_t scratch_bytes, int32_t* topk_idx, float* topk_w, int32_t* block_hist,
                       void* stream);
/* Bytes of scratch the two-phase form of kmoe_route needs (the router
 * transposed to bf16 and its column norms' partial sums). */
kmoe_status kmoe_route_scratch_bytes(const kmoe_desc* desc, size_t* bytes);

/* Stable sort of assignments by expert (kappa/qwen3/ffn_moe.py:189-200, 212):
 * group_sizes [E], offsets [E+1], active [E+1] (active[0..n) = experts with
 * at least one assignment in increasing order, active[E] = n),
 * sorted_token [T*K], sorted_expert [T*K], inv [T*K]. */
kmoe_status kmoe_dispatch(const kmoe_desc* desc, const int32_t* topk_idx, const int32_t* block_hist,
                          int32_t* group_sizes, int32_t* offsets, int32_t* active, int32_t* sorted_token,
                          int32_t* sorted_expert, int32_t* inv, void* stream);

/* SwiGLU experts over the sorted rows (kappa/qwen3/ffn_moe.py:99-102,
 * 149-152, 207-210): y_sorted [T*K, D] in x.dtype; h_sorted [T*K, I] in x.dtype,
 * except for the RAGGED chain with bf16 activations, whose f32 h is stored as
 * [T*K, 2I] bf16: per row hi = bf16(h) in [0, I) and lo = bf16(h - hi) in [I, 2I). */
kmoe_status kmoe_expert_ffn(const kmoe_desc* desc, const void* x, const int32_t* offsets, const int32_t* active,
                            const int32_t* sorted_token, const int32_t* sorted_expert, const kmoe_weight* gate,
                            const kmoe_weight* up, const kmoe_weight* down, const kmoe_packed_experts* packed,
                            void* h_sorted, void* y_sorted, void* stream);

/* The two halves of kmoe_expert_ffn, for per-kernel timing and parity:
 * gate/up products + SwiGLU -> h_sorted (the ragged_dot pair at
 * kappa/qwen3/ffn_moe.py:207-209), and the down product -> y_sorted
 * (kappa/qwen3/ffn_moe.py:210). Weights that a stage does not read may be NULL. */
kmoe_status kmoe_expert_gate_up(const kmoe_desc* desc, const void* x, const int32_t* offsets, const int32_t* active,
                                const int32_t* sorted_token, const int32_t* sorted_expert, const kmoe_weight* gate,
                                const kmoe_weight* up, const kmoe_packed_experts* packed, void* h_sorted,
                                void* stream);
kmoe_status kmoe_expert_down(const kmoe_desc* desc, const void* h_sorted, const int32_t* offsets,
                             const int32_t* active, const int32_t* sorted_expert, const kmoe_weight* down,
                             const kmoe_packed_experts* packed, void* y_sorted, void* stream);

/* Weighted combine (kappa/qwen3/ffn_moe.py:103, 155-157, 213-215), atomic-free,
 * with the terms p_j = round(topk_w[t,j] * y_sorted[inv[t*K+j]]) in j order:
 * GATHER_EINSUM out[t] = round(sum_j p_j) (f32 sum); RAGGED and FIXED_CAPACITY
 * out[t] = round(...round(round(p_0) + p_1)... + p_{K-1}). inv < 0 skips a term. */
kmoe_status kmoe_combine(const kmoe_desc* desc, const void* y_sorted, const int32_t* inv, const float* topk_w,
                         void* out, void* stream);

/* --- weights -------------------------------------------------------------- */
/* Relayout gate/up/down ([E,D,I], [E,I,D]; int8 + per-tensor or per-channel
 * scale) into `packed` for the gfx950 kernels. */
kmoe_status kmoe_prepack(const kmoe_desc* desc, const kmoe_weight* gate, const kmoe_weight* up,
                         const kmoe_weight* down, const kmoe_packed_experts* packed, void* stream);

/* to_compute_dtype (kappa/qwen3/quant.py:34-38) of a weight viewed as
 * [outer, channels] (channels = the last axis; a per-channel scale holds one
 * value per (outer / rows_per_scale_block, channel) - pass rows_per_scale_block =
 * the input-axis length of a stacked [E, Kd, N] tensor). */
kmoe_status kmoe_to_compute_dtype(const kmoe_weight* w, int64_t outer, int64_t channels,
                                  int64_t rows_per_scale_block, kmoe_dtype out_dtype, void* out, void* stream);

/* Symmetric int8 quantiser per output channel of a stacked [E, Kd, N] tensor
 * (kappa/qwen3/quant.py:41-48 with the max-abs taken per channel):
 * s[e,n] = max(max_k |w| / 127, FLT_MIN), q = clip(rint(w / s), -128, 127). */
kmoe_status kmoe_quantize_per_channel(int64_t experts, int64_t rows, int64_t channels, const void* w,
                                      kmoe_dtype w_dtype, int8_t* q, float* s, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KMOE_H_ */
