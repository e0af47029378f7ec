// Host-only side of the C ABI (see host.h): argument validation, workspace
// layout, program and kernel-family choice. No HIP call is made here; the
// entry points in api.hip run these checks, then the device check, then the
// kernels.
//
// Reference: the ValueErrors of moe_swiglu_ffn and _route
// (kappa/qwen3/ffn_moe.py:47-48, 239-240, 251-252, 299), the decode switch
// _effective_moe_impl (:219-223) and the gather program's scale rule
// (moe_take_dequant, kappa/qwen3/quant.py:71-74).
#include "host.h"

#include <stdarg.h>
#include <stdio.h>

namespace kmoe_host {

namespace {
thread_local char g_err[512] = "";

size_t align_up(size_t v) { return (v + 255) & ~(size_t)255; }
}  // namespace

kmoe_status fail(kmoe_status st, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return st;
}

const char* last_error() { return g_err; }

const char* status_string(kmoe_status s) {
  switch (s) {
    case KMOE_OK:
      return "ok";
    case KMOE_ERR_INVALID_ARG:
      return "invalid argument";
    case KMOE_ERR_UNSUPPORTED:
      return "unsupported";
    case KMOE_ERR_WORKSPACE_TOO_SMALL:
      return "workspace too small";
    case KMOE_ERR_NO_DEVICE:
      return "no HIP device";
    case KMOE_ERR_HIP:
      return "HIP error";
  }
  return "unknown status";
}

int route_split_groups(const kmoe_desc& d) {
  const int S = (int)((d.hidden + kmoe::kRouterSlice - 1) / kmoe::kRouterSlice);
  int P = 1;
  while (P < S) P <<= 1;
  return P >= 4 ? P / 4 : 1;
}

size_t route_split_part_floats(const kmoe_desc& d) {
  return (size_t)d.tokens * route_split_groups(d) * d.num_experts;
}

bool route_mfma_fits(const kmoe_desc& d, const kmoe_weight& router) {
  const int64_t D = d.hidden;
  return enum_value(d.act_dtype) == KMOE_DTYPE_BF16 && enum_value(router.dtype) == KMOE_DTYPE_BF16 &&
         (D == 512 || D == 1024 || D == 2048 || D == 4096) && d.num_experts % 16 == 0 && d.num_experts <= 256;
}

bool route_mfma_preferred(const kmoe_desc& d, const kmoe_weight& router) {
  // (layout() reserves its scratch from 2048 tokens)
  return route_mfma_fits(d, router) && d.tokens >= 2048;
}

size_t route_mfma_scratch_offsets(const kmoe_desc& d, int part) {
  const size_t ED = (size_t)d.num_experts * (size_t)d.hidden;
  const size_t o1 = align_up(2 * ED);
  const size_t o2 = o1 + 4 * (((size_t)d.hidden + 255) / 256) * (size_t)d.num_experts;
  return part == 1 ? o1 : (part == 2 ? o2 : 0);
}

size_t route_mfma_scratch_bytes(const kmoe_desc& d) { return route_mfma_scratch_offsets(d, 2); }

bool is_float(kmoe_dtype t) {
  const int v = enum_value(t);
  return v == KMOE_DTYPE_F32 || v == KMOE_DTYPE_BF16;
}

kmoe_status check_desc(const kmoe_desc* d) {
  if (!d) return fail(KMOE_ERR_INVALID_ARG, "desc is NULL");
  if (d->tokens < 0) return fail(KMOE_ERR_INVALID_ARG, "tokens must be >= 0 (got %lld)", (long long)d->tokens);
  if (d->hidden < 1 || d->num_experts < 1 || d->intermediate < 1)
    return fail(KMOE_ERR_INVALID_ARG, "hidden, num_experts and intermediate must be >= 1");
  if (d->top_k < 1 || d->top_k > d->num_experts)
    return fail(KMOE_ERR_INVALID_ARG, "top_k must be in [1, num_experts] (got %lld, num_experts %lld)",
                (long long)d->top_k, (long long)d->num_experts);
  if (!is_float(d->act_dtype)) return fail(KMOE_ERR_INVALID_ARG, "act_dtype must be F32 or BF16");
  if (d->num_experts > kmoe::kMaxExperts)
    return fail(KMOE_ERR_UNSUPPORTED, "num_experts %lld exceeds %d", (long long)d->num_experts, kmoe::kMaxExperts);
  if (d->top_k > kmoe::kMaxTopK)
    return fail(KMOE_ERR_UNSUPPORTED, "top_k %lld exceeds %d", (long long)d->top_k, kmoe::kMaxTopK);
  if (d->hidden > (int64_t)kmoe::kRouterSlice * kmoe::kMaxRouterSlices)
    return fail(KMOE_ERR_UNSUPPORTED, "hidden %lld exceeds %d", (long long)d->hidden,
                kmoe::kRouterSlice * kmoe::kMaxRouterSlices);
  // every buffer size below stays far inside size_t and every kernel index
  // inside int32 (T * K) or 2^40 elements (T * D, T * K * max(D, 2I))
  if (d->intermediate > ((int64_t)1 << 24))
    return fail(KMOE_ERR_UNSUPPORTED, "intermediate %lld too large", (long long)d->intermediate);
  if (d->tokens > (int64_t)0x7fffffff / d->top_k || d->tokens > ((int64_t)1 << 40) / d->hidden)
    return fail(KMOE_ERR_UNSUPPORTED, "tokens %lld too large", (long long)d->tokens);
  const int64_t row = d->hidden > 2 * d->intermediate ? d->hidden : 2 * d->intermediate;
  if (d->tokens * d->top_k > ((int64_t)1 << 40) / row)
    return fail(KMOE_ERR_UNSUPPORTED, "tokens %lld too large", (long long)d->tokens);
  const int impl = enum_value(d->impl), kernels = enum_value(d->kernels);
  if (impl != KMOE_IMPL_GATHER_EINSUM && impl != KMOE_IMPL_RAGGED && impl != KMOE_IMPL_FIXED_CAPACITY)
    return fail(KMOE_ERR_INVALID_ARG, "unknown impl %d", impl);
  if (impl == KMOE_IMPL_FIXED_CAPACITY && d->expert_capacity < 1)
    return fail(KMOE_ERR_INVALID_ARG, "fixed_capacity needs expert_capacity >= 1 (got %lld)",
                (long long)d->expert_capacity);
  if (impl != KMOE_IMPL_FIXED_CAPACITY && d->expert_capacity != 0)
    return fail(KMOE_ERR_INVALID_ARG, "expert_capacity must be 0 unless impl is fixed_capacity (got %lld)",
                (long long)d->expert_capacity);
  if (kernels != KMOE_KERNELS_AUTO && kernels != KMOE_KERNELS_DECODE && kernels != KMOE_KERNELS_GROUPED)
    return fail(KMOE_ERR_INVALID_ARG, "unknown kernels %d", kernels);
  if (kernels == KMOE_KERNELS_DECODE && d->tokens > kmoe::kRowsPathMaxTokens)
    return fail(KMOE_ERR_UNSUPPORTED, "the decode kernels take at most %d tokens (got %lld)", kmoe::kRowsPathMaxTokens,
                (long long)d->tokens);
  return KMOE_OK;
}

kmoe_impl effective_impl(const kmoe_desc& d) {
  if (d.impl == KMOE_IMPL_RAGGED && d.tokens <= d.decode_token_threshold) return KMOE_IMPL_GATHER_EINSUM;
  return d.impl;
}

int chain_of(const kmoe_desc& d) {
  return effective_impl(d) == KMOE_IMPL_RAGGED ? kmoe::kChainF32 : kmoe::kChainAct;
}

bool scatter_of(const kmoe_desc& d) { return effective_impl(d) != KMOE_IMPL_GATHER_EINSUM; }

// The gather program multiplies the gathered [T, K, D, I] values by the scale as
// stored (kappa/qwen3/quant.py:71-74): a per-tensor scale, or [E, 1, N] with E = 1.
kmoe_status check_gather_scales(const kmoe_desc& d, kmoe_scale_kind kind, const char* name) {
  if (effective_impl(d) == KMOE_IMPL_GATHER_EINSUM && kind == KMOE_SCALE_CHANNEL && d.num_experts > 1)
    return fail(KMOE_ERR_INVALID_ARG,
                "%s: gather_einsum takes one scale per tensor; per-channel scales of %lld experts run with the "
                "ragged or fixed_capacity impl",
                name, (long long)d.num_experts);
  return KMOE_OK;
}

kmoe_status check_weight(const kmoe_weight* w, const char* name) {
  if (!w) return fail(KMOE_ERR_INVALID_ARG, "%s weight is NULL", name);
  if (!w->values) return fail(KMOE_ERR_INVALID_ARG, "%s values pointer is NULL", name);
  if (is_float(w->dtype)) {
    if (enum_value(w->scale_kind) != KMOE_SCALE_NONE)
      return fail(KMOE_ERR_INVALID_ARG, "%s: a float weight takes no scale (scale_kind must be NONE)", name);
    return KMOE_OK;
  }
  if (enum_value(w->dtype) != KMOE_DTYPE_I8) return fail(KMOE_ERR_INVALID_ARG, "%s: unsupported weight dtype", name);
  const int kind = enum_value(w->scale_kind);
  if (kind != KMOE_SCALE_TENSOR && kind != KMOE_SCALE_CHANNEL)
    return fail(KMOE_ERR_INVALID_ARG, "%s: int8 values need a TENSOR or CHANNEL scale", name);
  if (!w->scale) return fail(KMOE_ERR_INVALID_ARG, "%s scale pointer is NULL", name);
  if (!is_float(w->scale_dtype)) return fail(KMOE_ERR_INVALID_ARG, "%s scale dtype must be F32 or BF16", name);
  return KMOE_OK;
}

Workspace layout(const kmoe_desc& d, bool block) {
  const size_t T = (size_t)d.tokens, E = (size_t)d.num_experts, K = (size_t)d.top_k, D = (size_t)d.hidden,
               I = (size_t)d.intermediate;
  const size_t M = T * K;
  const size_t nblk = (T + kmoe::kDispatchBlock - 1) / kmoe::kDispatchBlock;
  const size_t act = dtype_size(d.act_dtype);
  Workspace w;
  size_t o = 0;
  auto take = [&](size_t bytes) {
    size_t at = o;
    o = align_up(o + bytes);
    return at;
  };
  w.topk_idx = take(4 * M);
  w.topk_w = take(4 * M);
  w.hist = take(4 * nblk * E);
  w.group_sizes = take(4 * E);
  w.offsets = take(4 * (E + 1));
  w.active = take(4 * (E + 1));
  w.sorted_token = take(4 * M);
  w.sorted_expert = take(4 * M);
  w.inv = take(4 * M);
  // the f32 chain keeps h as two bf16 planes per row for bf16 activations
  w.h_sorted = take((chain_of(d) == kmoe::kChainF32 && d.act_dtype == KMOE_DTYPE_BF16 ? 4 : act) * M * I);
  w.y_sorted = take(act * M * D);
  // the split router's group partials, or above its range the two-phase
  // router's scratch (a bf16 router; the others need none)
  w.route_part = take(T <= (size_t)kSplitRouterMaxTokens ? 4 * route_split_part_floats(d)
                                                         : (T >= 2048 ? route_mfma_scratch_bytes(d) : 0));
  w.h_scale = take(down_planes_fits(d) ? 4 * M : 0);
  w.normed = take(block ? act * T * D : 0);  // rms_norm(h) for kmoe_forward_block
  w.total = o;
  return w;
}

bool packed_ok(const kmoe_desc& d, const kmoe_packed_experts* p) {
  return p && p->w13 && p->s13 && p->w2 && p->s2 && d.act_dtype == KMOE_DTYPE_BF16 && d.hidden % 64 == 0 &&
         d.intermediate % 64 == 0 && p->num_experts == d.num_experts && p->hidden == d.hidden &&
         p->intermediate == d.intermediate;
}

// The GEMV-style kernels up to 64 tokens (the decode batches), the grouped
// GEMMs above (or whenever asked for). The GEMVs' row-group form covers 65 to
// 128 tokens when the decode kernels are asked for; left to choose, the
// grouped GEMMs (64-row tiles, every tile resident at once) are faster there:
// T = 80 / 100 / 128 140.5 -> 136.9, 145.9 -> 136.9, 152.9 -> 137.5 us per
// layer; at T = 40 they would lose (112.4 -> 125.6 us).
int family_of(const kmoe_desc& d) {
  if (d.kernels == KMOE_KERNELS_GROUPED) return kFamilyGemm;
  if (d.tokens <= 16 * kmoe::kDecodeMaxRowBlocks) return kFamilyDecode;
  if (d.kernels == KMOE_KERNELS_DECODE && d.tokens <= kmoe::kRowsPathMaxTokens) return kFamilyRows;
  return kFamilyGemm;
}

bool down_planes_fits(const kmoe_desc& d) {
  const int64_t M = d.tokens * d.top_k;
  return enum_value(d.act_dtype) == KMOE_DTYPE_BF16 && chain_of(d) == kmoe::kChainF32 &&
         family_of(d) == kFamilyGemm && M >= 96 * d.num_experts && d.hidden % 256 == 0 &&
         d.intermediate % 128 == 0 && d.intermediate <= 64 * kmoe::kPlanesMaxChunks;
}

// Weights a layout-native expert stage reads.
kmoe_status check_stage_weights(const kmoe_desc& d, const kmoe_packed_experts* packed, int stages,
                                const kmoe_weight* gate, const kmoe_weight* up, const kmoe_weight* down) {
  if (packed_ok(d, packed)) return KMOE_OK;
  if (stages & kStageGateUp) {
    KMOE_TRY(check_weight(gate, "gate"));
    KMOE_TRY(check_weight(up, "up"));
    KMOE_TRY(check_gather_scales(d, gate->scale_kind, "gate"));
    KMOE_TRY(check_gather_scales(d, up->scale_kind, "up"));
  }
  if (stages & kStageDown) {
    KMOE_TRY(check_weight(down, "down"));
    KMOE_TRY(check_gather_scales(d, down->scale_kind, "down"));
  }
  return KMOE_OK;
}

kmoe_status check_packed_arg(const kmoe_desc& d, const kmoe_packed_experts* packed) {
  if (!packed) return KMOE_OK;
  if (!packed->w13 || !packed->s13 || !packed->w2 || !packed->s2)
    return fail(KMOE_ERR_INVALID_ARG, "packed experts: every buffer must be non-NULL");
  if (d.act_dtype != KMOE_DTYPE_BF16)
    return fail(KMOE_ERR_UNSUPPORTED, "packed int8 experts run with bf16 activations only");
  if (d.hidden % 64 || d.intermediate % 64)
    return fail(KMOE_ERR_UNSUPPORTED, "packed experts need hidden and intermediate divisible by 64");
  if (packed->num_experts != d.num_experts || packed->hidden != d.hidden || packed->intermediate != d.intermediate)
    return fail(KMOE_ERR_INVALID_ARG,
                "packed experts hold E=%lld, D=%lld, I=%lld; the call has E=%lld, D=%lld, I=%lld",
                (long long)packed->num_experts, (long long)packed->hidden, (long long)packed->intermediate,
                (long long)d.num_experts, (long long)d.hidden, (long long)d.intermediate);
  const int kind = enum_value(packed->source_scale_kind);
  if (kind != KMOE_SCALE_TENSOR && kind != KMOE_SCALE_CHANNEL)
    return fail(KMOE_ERR_INVALID_ARG, "packed experts: source_scale_kind must be TENSOR or CHANNEL");
  KMOE_TRY(check_gather_scales(d, packed->source_scale_kind, "packed experts"));
  return KMOE_OK;
}

kmoe_status check_norm_args(const void* scale, kmoe_dtype scale_dtype, float epsilon) {
  if (!scale) return fail(KMOE_ERR_INVALID_ARG, "norm scale pointer is NULL");
  if (!is_float(scale_dtype)) return fail(KMOE_ERR_INVALID_ARG, "norm scale dtype must be F32 or BF16");
  if (!(epsilon >= 0.0f) || epsilon > 1.0f)
    return fail(KMOE_ERR_INVALID_ARG, "epsilon must be in [0, 1] (got %g)", (double)epsilon);
  return KMOE_OK;
}

namespace {

kmoe_status check_forward_args(const kmoe_desc* desc, const kmoe_weight* router, const kmoe_weight* gate,
                               const kmoe_weight* up, const kmoe_weight* down, const kmoe_packed_experts* packed) {
  KMOE_TRY(check_desc(desc));
  KMOE_TRY(check_weight(router, "router"));
  KMOE_TRY(check_packed_arg(*desc, packed));
  if (!packed) {
    KMOE_TRY(check_weight(gate, "gate"));
    KMOE_TRY(check_weight(up, "up"));
    KMOE_TRY(check_weight(down, "down"));
    KMOE_TRY(check_gather_scales(*desc, gate->scale_kind, "gate"));
    KMOE_TRY(check_gather_scales(*desc, up->scale_kind, "up"));
    KMOE_TRY(check_gather_scales(*desc, down->scale_kind, "down"));
  }
  return KMOE_OK;
}

}  // namespace

kmoe_status validate_forward(const kmoe_desc* desc, const void* x, const kmoe_weight* router,
                             const kmoe_weight* gate, const kmoe_weight* up, const kmoe_weight* down,
                             const kmoe_packed_experts* packed, const void* out, const void* workspace,
                             size_t workspace_bytes, Workspace* w) {
  KMOE_TRY(check_forward_args(desc, router, gate, up, down, packed));
  if (desc->tokens > 0 && (!x || !out)) return fail(KMOE_ERR_INVALID_ARG, "kmoe_forward: x and out must be non-NULL");
  *w = layout(*desc, false);
  if (desc->tokens > 0 && (!workspace || workspace_bytes < w->total))
    return fail(KMOE_ERR_WORKSPACE_TOO_SMALL, "workspace of %zu bytes is smaller than the %zu required",
                workspace_bytes, w->total);
  return KMOE_OK;
}

kmoe_status validate_forward_noalloc(const kmoe_desc* desc, const void* x, const kmoe_weight* router,
                                     const kmoe_weight* gate, const kmoe_weight* up, const kmoe_weight* down,
                                     const kmoe_packed_experts* packed, const void* out, size_t scratch_bytes,
                                     Workspace* w) {
  KMOE_TRY(check_forward_args(desc, router, gate, up, down, packed));
  if (desc->tokens > 0 && (!x || !out))
    return fail(KMOE_ERR_INVALID_ARG, "kmoe_forward_noalloc: x and out must be non-NULL");
  *w = layout(*desc, false);
  if (w->total > scratch_bytes)
    return fail(KMOE_ERR_WORKSPACE_TOO_SMALL,
                "kmoe_forward_noalloc: the call needs %zu bytes of workspace, beyond its %zu-byte scratch; use "
                "kmoe_forward with a workspace",
                w->total, scratch_bytes);
  return KMOE_OK;
}

kmoe_status validate_forward_block(const kmoe_desc* desc, const void* h, const void* norm_scale,
                                   kmoe_dtype norm_dtype, float epsilon, const kmoe_weight* router,
                                   const kmoe_weight* gate, const kmoe_weight* up, const kmoe_weight* down,
                                   const kmoe_packed_experts* packed, const void* out, const void* workspace,
                                   size_t workspace_bytes, Workspace* w) {
  KMOE_TRY(check_forward_args(desc, router, gate, up, down, packed));
  KMOE_TRY(check_norm_args(norm_scale, norm_dtype, epsilon));
  if (desc->tokens > 0 && (!h || !out))
    return fail(KMOE_ERR_INVALID_ARG, "kmoe_forward_block: h and out must be non-NULL");
  if (desc->tokens > 0 && out == h) return fail(KMOE_ERR_INVALID_ARG, "kmoe_forward_block: out must not alias h");
  *w = layout(*desc, true);
  if (desc->tokens > 0 && (!workspace || workspace_bytes < w->total))
    return fail(KMOE_ERR_WORKSPACE_TOO_SMALL, "workspace of %zu bytes is smaller than the %zu required",
                workspace_bytes, w->total);
  return KMOE_OK;
}

kmoe_status validate_workspace_bytes(const kmoe_desc* desc, size_t* bytes) {
  KMOE_TRY(check_desc(desc));
  if (!bytes) return fail(KMOE_ERR_INVALID_ARG, "bytes is NULL");
  *bytes = layout(*desc, true).total;
  return KMOE_OK;
}

kmoe_status validate_prepack_bytes(const kmoe_desc* desc, kmoe_packed_sizes* sizes) {
  KMOE_TRY(check_desc(desc));
  if (!sizes) return fail(KMOE_ERR_INVALID_ARG, "sizes is NULL");
  if (desc->hidden % 64 || desc->intermediate % 64)
    return fail(KMOE_ERR_UNSUPPORTED, "packed experts need hidden and intermediate divisible by 64");
  const size_t E = (size_t)desc->num_experts, D = (size_t)desc->hidden, I = (size_t)desc->intermediate;
  sizes->w13_bytes = E * 2 * D * I;
  sizes->s13_bytes = 4 * E * 2 * I;
  sizes->w2_bytes = E * I * D;
  sizes->s2_bytes = 4 * E * D;
  return KMOE_OK;
}

kmoe_status validate_route(const kmoe_desc* desc, const void* x, const kmoe_weight* router, const void* scratch,
                           size_t scratch_bytes, const int32_t* topk_idx, const float* topk_w,
                           const int32_t* block_hist) {
  KMOE_TRY(check_desc(desc));
  KMOE_TRY(check_weight(router, "router"));
  if (!x || !topk_idx || !topk_w || !block_hist) return fail(KMOE_ERR_INVALID_ARG, "kmoe_route: NULL buffer");
  if (scratch && scratch_bytes < route_mfma_scratch_bytes(*desc))
    return fail(KMOE_ERR_WORKSPACE_TOO_SMALL, "kmoe_route: scratch of %zu bytes is smaller than the %zu required",
                scratch_bytes, route_mfma_scratch_bytes(*desc));
  return KMOE_OK;
}

kmoe_status validate_route_scratch_bytes(const kmoe_desc* desc, size_t* bytes) {
  KMOE_TRY(check_desc(desc));
  if (!bytes) return fail(KMOE_ERR_INVALID_ARG, "bytes is NULL");
  *bytes = route_mfma_scratch_bytes(*desc);
  return KMOE_OK;
}

kmoe_status validate_dispatch(const kmoe_desc* desc, const int32_t* topk_idx, const int32_t* block_hist,
                              const int32_t* group_sizes, const int32_t* offsets, const int32_t* active,
                              const int32_t* sorted_token, const int32_t* sorted_expert, const int32_t* inv) {
  KMOE_TRY(check_desc(desc));
  if (!topk_idx || !block_hist || !group_sizes || !offsets || !active || !sorted_token || !sorted_expert || !inv)
    return fail(KMOE_ERR_INVALID_ARG, "kmoe_dispatch: NULL buffer");
  return KMOE_OK;
}

kmoe_status validate_expert(const kmoe_desc* desc, int stages, const void* src, const int32_t* offsets,
                            const int32_t* active, const int32_t* sorted_token, const int32_t* sorted_expert,
                            const kmoe_weight* gate, const kmoe_weight* up, const kmoe_weight* down,
                            const kmoe_packed_experts* packed, const void* h_sorted, const void* y_sorted) {
  KMOE_TRY(check_desc(desc));
  KMOE_TRY(check_packed_arg(*desc, packed));
  KMOE_TRY(check_stage_weights(*desc, packed, stages, gate, up, down));
  const char* what = stages == kStageGateUp ? "kmoe_expert_gate_up"
                                            : (stages == kStageDown ? "kmoe_expert_down" : "kmoe_expert_ffn");
  if (!src || !offsets || !active || !sorted_expert || !h_sorted)
    return fail(KMOE_ERR_INVALID_ARG, "%s: NULL buffer", what);
  if ((stages & kStageGateUp) && !sorted_token) return fail(KMOE_ERR_INVALID_ARG, "%s: NULL buffer", what);
  if ((stages & kStageDown) && !y_sorted) return fail(KMOE_ERR_INVALID_ARG, "%s: NULL buffer", what);
  return KMOE_OK;
}

kmoe_status validate_combine(const kmoe_desc* desc, const void* y_sorted, const int32_t* inv, const float* topk_w,
                             const void* out) {
  KMOE_TRY(check_desc(desc));
  if (!y_sorted || !inv || !topk_w || !out) return fail(KMOE_ERR_INVALID_ARG, "kmoe_combine: NULL buffer");
  return KMOE_OK;
}

kmoe_status validate_rms_norm(const kmoe_desc* desc, const void* x, const void* scale, kmoe_dtype scale_dtype,
                              float epsilon, const void* out) {
  KMOE_TRY(check_desc(desc));
  KMOE_TRY(check_norm_args(scale, scale_dtype, epsilon));
  if (desc->tokens > 0 && (!x || !out)) return fail(KMOE_ERR_INVALID_ARG, "kmoe_rms_norm: x and out must be non-NULL");
  return KMOE_OK;
}

kmoe_status validate_prepack(const kmoe_desc* desc, const kmoe_weight* gate, const kmoe_weight* up,
                             const kmoe_weight* down, const kmoe_packed_experts* packed) {
  KMOE_TRY(check_desc(desc));
  KMOE_TRY(check_weight(gate, "gate"));
  KMOE_TRY(check_weight(up, "up"));
  KMOE_TRY(check_weight(down, "down"));
  if (enum_value(gate->dtype) != KMOE_DTYPE_I8 || enum_value(up->dtype) != KMOE_DTYPE_I8 ||
      enum_value(down->dtype) != KMOE_DTYPE_I8)
    return fail(KMOE_ERR_UNSUPPORTED, "kmoe_prepack packs int8 (Q8) experts only");
  if (!packed || !packed->w13 || !packed->s13 || !packed->w2 || !packed->s2)
    return fail(KMOE_ERR_INVALID_ARG, "kmoe_prepack: packed buffers must be non-NULL");
  if (packed->num_experts != desc->num_experts || packed->hidden != desc->hidden ||
      packed->intermediate != desc->intermediate)
    return fail(KMOE_ERR_INVALID_ARG, "kmoe_prepack: the packed shapes must be the desc's E, D and I");
  if (desc->hidden % 64 || desc->intermediate % 64)
    return fail(KMOE_ERR_UNSUPPORTED, "packed experts need hidden and intermediate divisible by 64");
  // the forward calls trust the recorded kind (the gather program refuses
  // per-channel scales), so it must be the kind of the scales packed here
  const kmoe_scale_kind kind =
      gate->scale_kind == KMOE_SCALE_TENSOR && up->scale_kind == KMOE_SCALE_TENSOR &&
              down->scale_kind == KMOE_SCALE_TENSOR
          ? KMOE_SCALE_TENSOR
          : KMOE_SCALE_CHANNEL;
  if (enum_value(packed->source_scale_kind) != kind)
    return fail(KMOE_ERR_INVALID_ARG, "kmoe_prepack: source_scale_kind must be %s for these weights",
                kind == KMOE_SCALE_TENSOR ? "TENSOR" : "CHANNEL");
  return KMOE_OK;
}

kmoe_status validate_to_compute_dtype(const kmoe_weight* w, int64_t outer, int64_t channels,
                                      int64_t rows_per_scale_block, kmoe_dtype out_dtype, const void* out) {
  KMOE_TRY(check_weight(w, "weight"));
  if (outer < 0 || channels < 1 || rows_per_scale_block < 1)
    return fail(KMOE_ERR_INVALID_ARG, "kmoe_to_compute_dtype: bad shape");
  if (outer > ((int64_t)1 << 40) / channels) return fail(KMOE_ERR_UNSUPPORTED, "kmoe_to_compute_dtype: too large");
  if (!is_float(out_dtype)) return fail(KMOE_ERR_INVALID_ARG, "out_dtype must be F32 or BF16");
  if (!out) return fail(KMOE_ERR_INVALID_ARG, "out is NULL");
  return KMOE_OK;
}

kmoe_status validate_quantize(int64_t experts, int64_t rows, int64_t channels, const void* w, kmoe_dtype w_dtype,
                              const int8_t* q, const float* s) {
  if (experts < 1 || rows < 1 || channels < 1) return fail(KMOE_ERR_INVALID_ARG, "quantize: bad shape");
  if (!is_float(w_dtype)) return fail(KMOE_ERR_INVALID_ARG, "quantize: w_dtype must be F32 or BF16");
  if (!w || !q || !s) return fail(KMOE_ERR_INVALID_ARG, "quantize: NULL buffer");
  if (experts > 65535) return fail(KMOE_ERR_UNSUPPORTED, "quantize: too many experts");
  if (rows > ((int64_t)1 << 40) / channels / experts) return fail(KMOE_ERR_UNSUPPORTED, "quantize: too large");
  return KMOE_OK;
}

}  // namespace kmoe_host
