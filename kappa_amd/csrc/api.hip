// C ABI entry points (include/kmoe.h): argument validation on the host,
// workspace layout and the stage sequence of moe_swiglu_ffn
// (kappa/qwen3/ffn_moe.py:226-299).
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "common.h"
#include "launch.h"

namespace {

thread_local char g_err[512] = "";

kmoe_status fail(kmoe_status st, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return st;
}

kmoe_status hip_fail(hipError_t e, const char* what) {
  return fail(KMOE_ERR_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

kmoe_status device_status() {
  static std::once_flag once;
  static int count = -1;
  std::call_once(once, [] {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
    count = n;
  });
  if (count <= 0) return fail(KMOE_ERR_NO_DEVICE, "no HIP device is visible");
  return KMOE_OK;
}

bool is_float(kmoe_dtype t) { return t == KMOE_DTYPE_F32 || t == KMOE_DTYPE_BF16; }

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
  if ((d->hidden + kmoe::kRouterSlice - 1) / kmoe::kRouterSlice > kmoe::kMaxRouterSlices)
    return fail(KMOE_ERR_UNSUPPORTED, "hidden %lld exceeds %d", (long long)d->hidden,
                kmoe::kRouterSlice * kmoe::kMaxRouterSlices);
  if (d->tokens * d->top_k > (int64_t)0x7fffffff || d->tokens * d->hidden > ((int64_t)1 << 40))
    return fail(KMOE_ERR_UNSUPPORTED, "tokens %lld too large", (long long)d->tokens);
  if (d->impl != KMOE_IMPL_GATHER_EINSUM && d->impl != KMOE_IMPL_RAGGED && d->impl != KMOE_IMPL_FIXED_CAPACITY)
    return fail(KMOE_ERR_INVALID_ARG, "unknown impl %d", (int)d->impl);
  if (d->impl == KMOE_IMPL_FIXED_CAPACITY && d->expert_capacity < 1)
    return fail(KMOE_ERR_INVALID_ARG, "fixed_capacity needs expert_capacity >= 1 (got %lld)",
                (long long)d->expert_capacity);
  if (d->impl != KMOE_IMPL_FIXED_CAPACITY && d->expert_capacity != 0)
    return fail(KMOE_ERR_INVALID_ARG, "expert_capacity must be 0 unless impl is fixed_capacity (got %lld)",
                (long long)d->expert_capacity);
  if (d->kernels != KMOE_KERNELS_AUTO && d->kernels != KMOE_KERNELS_DECODE && d->kernels != KMOE_KERNELS_GROUPED)
    return fail(KMOE_ERR_INVALID_ARG, "unknown kernels %d", (int)d->kernels);
  if (d->kernels == KMOE_KERNELS_DECODE && d->tokens > kmoe::kRowsPathMaxTokens)
    return fail(KMOE_ERR_UNSUPPORTED, "the decode kernels take at most %d tokens (got %lld)", kmoe::kRowsPathMaxTokens,
                (long long)d->tokens);
  return KMOE_OK;
}

// _effective_moe_impl (kappa/qwen3/ffn_moe.py:219-223)
kmoe_impl effective_impl(const kmoe_desc& d) {
  if (d.impl == KMOE_IMPL_RAGGED && d.tokens <= d.decode_token_threshold) return KMOE_IMPL_GATHER_EINSUM;
  return d.impl;
}

// the expert products' rounding chain and the combine of the program that runs
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

kmoe_status check_weight(const kmoe_weight* w, const char* name, bool allow_int8 = true) {
  if (!w) return fail(KMOE_ERR_INVALID_ARG, "%s weight is NULL", name);
  if (!w->values) return fail(KMOE_ERR_INVALID_ARG, "%s values pointer is NULL", name);
  if (is_float(w->dtype)) {
    if (w->scale_kind != KMOE_SCALE_NONE)
      return fail(KMOE_ERR_INVALID_ARG, "%s: a float weight takes no scale (scale_kind must be NONE)", name);
    return KMOE_OK;
  }
  if (w->dtype != KMOE_DTYPE_I8 || !allow_int8) return fail(KMOE_ERR_INVALID_ARG, "%s: unsupported weight dtype", name);
  if (w->scale_kind != KMOE_SCALE_TENSOR && w->scale_kind != KMOE_SCALE_CHANNEL)
    return fail(KMOE_ERR_INVALID_ARG, "%s: int8 values need a TENSOR or CHANNEL scale", name);
  if (!w->scale) return fail(KMOE_ERR_INVALID_ARG, "%s scale pointer is NULL", name);
  if (!is_float(w->scale_dtype)) return fail(KMOE_ERR_INVALID_ARG, "%s scale dtype must be F32 or BF16", name);
  return KMOE_OK;
}

#define KMOE_TRY(expr)                 \
  do {                                 \
    kmoe_status _s = (expr);           \
    if (_s != KMOE_OK) return _s;      \
  } while (0)

#define KMOE_HIP(expr, what)                          \
  do {                                                \
    hipError_t _e = (expr);                           \
    if (_e != hipSuccess) return hip_fail(_e, what);  \
  } while (0)

size_t align_up(size_t v) { return (v + 255) & ~(size_t)255; }

struct Workspace {
  size_t topk_idx, topk_w, hist, group_sizes, offsets, active, sorted_token, sorted_expert, inv, h_sorted,
      y_sorted, route_part, normed, total;
};

Workspace layout(const kmoe_desc& d) {
  const size_t T = (size_t)d.tokens, E = (size_t)d.num_experts, K = (size_t)d.top_k, D = (size_t)d.hidden,
               I = (size_t)d.intermediate;
  const size_t M = T * K;
  const size_t nblk = (T + kmoe::kDispatchBlock - 1) / kmoe::kDispatchBlock;
  const size_t act = kmoe_host::dtype_size(d.act_dtype);
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
  w.route_part = take(T <= (size_t)kmoe_host::kSplitRouterMaxTokens ? 4 * kmoe_host::route_split_part_floats(d) : 0);
  w.normed = take(act * T * D);  // rms_norm(h) for kmoe_forward_block
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
  if (d.kernels == KMOE_KERNELS_GROUPED) return kmoe_host::kFamilyGemm;
  if (d.tokens <= 16 * kmoe::kDecodeMaxRowBlocks) return kmoe_host::kFamilyDecode;
  if (d.kernels == KMOE_KERNELS_DECODE && d.tokens <= kmoe::kRowsPathMaxTokens) return kmoe_host::kFamilyRows;
  return kmoe_host::kFamilyGemm;
}

kmoe_status expert_stage(const kmoe_desc& d, int stages, const void* x, const int32_t* offsets, const int32_t* active,
                         const int32_t* sorted_token, const int32_t* sorted_expert, const kmoe_weight* gate,
                         const kmoe_weight* up, const kmoe_weight* down, const kmoe_packed_experts* packed,
                         void* h_sorted, void* y_sorted, hipStream_t st) {
  hipError_t e;
  if (packed_ok(d, packed)) {
    e = kmoe_host::launch_expert_packed(d, chain_of(d), family_of(d), stages, x, offsets, active, sorted_token,
                                        *packed, h_sorted, y_sorted, st);
  } else {
    e = kmoe_host::launch_expert_generic(d, chain_of(d), stages, x, sorted_token, sorted_expert, gate, up, down,
                                         h_sorted, y_sorted, st);
  }
  if (e != hipSuccess) return hip_fail(e, "expert kernels");
  return KMOE_OK;
}

// Weights a layout-native expert stage reads.
kmoe_status check_stage_weights(const kmoe_desc& d, const kmoe_packed_experts* packed, int stages,
                                const kmoe_weight* gate, const kmoe_weight* up, const kmoe_weight* down) {
  if (packed_ok(d, packed)) return KMOE_OK;
  if (stages & kmoe_host::kStageGateUp) {
    KMOE_TRY(check_weight(gate, "gate"));
    KMOE_TRY(check_weight(up, "up"));
    KMOE_TRY(check_gather_scales(d, gate->scale_kind, "gate"));
    KMOE_TRY(check_gather_scales(d, up->scale_kind, "up"));
  }
  if (stages & kmoe_host::kStageDown) {
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
  if (packed->source_scale_kind != KMOE_SCALE_TENSOR && packed->source_scale_kind != KMOE_SCALE_CHANNEL)
    return fail(KMOE_ERR_INVALID_ARG, "packed experts: source_scale_kind must be TENSOR or CHANNEL");
  KMOE_TRY(check_gather_scales(d, packed->source_scale_kind, "packed experts"));
  return KMOE_OK;
}

}  // namespace

extern "C" {

const char* kmoe_version(void) { return "kmoe 0.2.0 (gfx950)"; }

int kmoe_abi_version(void) { return KMOE_ABI_VERSION; }

const char* kmoe_status_string(kmoe_status s) {
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

const char* kmoe_last_error(void) { return g_err; }

kmoe_status kmoe_device_check(void) { return device_status(); }

kmoe_status kmoe_workspace_bytes(const kmoe_desc* desc, size_t* bytes) {
  KMOE_TRY(check_desc(desc));
  if (!bytes) return fail(KMOE_ERR_INVALID_ARG, "bytes is NULL");
  *bytes = layout(*desc).total;
  return KMOE_OK;
}

kmoe_status kmoe_prepack_bytes(const kmoe_desc* desc, kmoe_packed_sizes* sizes) {
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

kmoe_status kmoe_route(const kmoe_desc* desc, const void* x, const kmoe_weight* router, float* logits,
                       float* logits_scratch, int32_t* topk_idx, float* topk_w, int32_t* block_hist, void* stream) {
  (void)logits_scratch;
  KMOE_TRY(check_desc(desc));
  KMOE_TRY(check_weight(router, "router"));
  if (!x || !topk_idx || !topk_w || !block_hist) return fail(KMOE_ERR_INVALID_ARG, "kmoe_route: NULL buffer");
  KMOE_TRY(device_status());
  if (desc->tokens == 0) return KMOE_OK;
  hipError_t e = kmoe_host::launch_route(*desc, x, *router, logits, topk_idx, topk_w, block_hist,
                                         (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "route kernels");
  return KMOE_OK;
}

kmoe_status kmoe_dispatch(const kmoe_desc* desc, const int32_t* topk_idx, const int32_t* block_hist,
                          int32_t* group_sizes, int32_t* offsets, int32_t* active, int32_t* sorted_token,
                          int32_t* sorted_expert, int32_t* inv, void* stream) {
  KMOE_TRY(check_desc(desc));
  if (!topk_idx || !block_hist || !group_sizes || !offsets || !active || !sorted_token || !sorted_expert || !inv)
    return fail(KMOE_ERR_INVALID_ARG, "kmoe_dispatch: NULL buffer");
  KMOE_TRY(device_status());
  if (desc->tokens == 0) return fail(KMOE_ERR_UNSUPPORTED, "kmoe_dispatch: tokens == 0");
  hipError_t e = kmoe_host::launch_dispatch(*desc, topk_idx, block_hist, group_sizes, offsets, active, sorted_token,
                                            sorted_expert, inv, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "dispatch kernel");
  return KMOE_OK;
}

kmoe_status kmoe_expert_ffn(const kmoe_desc* desc, const void* x, const int32_t* offsets, const int32_t* active,
                            const int32_t* sorted_token, const int32_t* sorted_expert, const kmoe_weight* gate,
                            const kmoe_weight* up, const kmoe_weight* down, const kmoe_packed_experts* packed,
                            void* h_sorted, void* y_sorted, void* stream) {
  const int both = kmoe_host::kStageGateUp | kmoe_host::kStageDown;
  KMOE_TRY(check_desc(desc));
  KMOE_TRY(check_packed_arg(*desc, packed));
  KMOE_TRY(check_stage_weights(*desc, packed, both, gate, up, down));
  if (!x || !offsets || !active || !sorted_token || !sorted_expert || !h_sorted || !y_sorted)
    return fail(KMOE_ERR_INVALID_ARG, "kmoe_expert_ffn: NULL buffer");
  KMOE_TRY(device_status());
  if (desc->tokens == 0) return KMOE_OK;
  return expert_stage(*desc, both, x, offsets, active, sorted_token, sorted_expert, gate, up, down, packed, h_sorted,
                      y_sorted, (hipStream_t)stream);
}

kmoe_status kmoe_expert_gate_up(const kmoe_desc* desc, const void* x, const int32_t* offsets, const int32_t* active,
                                const int32_t* sorted_token, const int32_t* sorted_expert, const kmoe_weight* gate,
                                const kmoe_weight* up, const kmoe_packed_experts* packed, void* h_sorted,
                                void* stream) {
  KMOE_TRY(check_desc(desc));
  KMOE_TRY(check_packed_arg(*desc, packed));
  KMOE_TRY(check_stage_weights(*desc, packed, kmoe_host::kStageGateUp, gate, up, nullptr));
  if (!x || !offsets || !active || !sorted_token || !sorted_expert || !h_sorted)
    return fail(KMOE_ERR_INVALID_ARG, "kmoe_expert_gate_up: NULL buffer");
  KMOE_TRY(device_status());
  if (desc->tokens == 0) return KMOE_OK;
  return expert_stage(*desc, kmoe_host::kStageGateUp, x, offsets, active, sorted_token, sorted_expert, gate, up,
                      nullptr, packed, h_sorted, nullptr, (hipStream_t)stream);
}

kmoe_status kmoe_expert_down(const kmoe_desc* desc, const void* h_sorted, const int32_t* offsets,
                             const int32_t* active, const int32_t* sorted_expert, const kmoe_weight* down,
                             const kmoe_packed_experts* packed, void* y_sorted, void* stream) {
  KMOE_TRY(check_desc(desc));
  KMOE_TRY(check_packed_arg(*desc, packed));
  KMOE_TRY(check_stage_weights(*desc, packed, kmoe_host::kStageDown, nullptr, nullptr, down));
  if (!h_sorted || !offsets || !active || !sorted_expert || !y_sorted)
    return fail(KMOE_ERR_INVALID_ARG, "kmoe_expert_down: NULL buffer");
  KMOE_TRY(device_status());
  if (desc->tokens == 0) return KMOE_OK;
  return expert_stage(*desc, kmoe_host::kStageDown, nullptr, offsets, active, nullptr, sorted_expert, nullptr,
                      nullptr, down, packed, const_cast<void*>(h_sorted), y_sorted, (hipStream_t)stream);
}

kmoe_status kmoe_combine(const kmoe_desc* desc, const void* y_sorted, const int32_t* inv, const float* topk_w,
                         void* out, void* stream) {
  KMOE_TRY(check_desc(desc));
  if (!y_sorted || !inv || !topk_w || !out) return fail(KMOE_ERR_INVALID_ARG, "kmoe_combine: NULL buffer");
  KMOE_TRY(device_status());
  if (desc->tokens == 0) return KMOE_OK;
  hipError_t e = kmoe_host::launch_combine(*desc, scatter_of(*desc), y_sorted, inv, topk_w, out, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "combine kernel");
  return KMOE_OK;
}

}  // extern "C"

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

kmoe_status forward_general(const kmoe_desc* desc, const void* x, const void* xin, const void* res,
                            const kmoe_host::SliceNorm* norm, const kmoe_weight* router, const kmoe_weight* gate,
                            const kmoe_weight* up, const kmoe_weight* down, const kmoe_packed_experts* packed,
                            void* out, char* base, const Workspace& w, int chain, bool scatter,
                            const kmoe_host::DispatchOut& dout, hipStream_t st);

// The stage sequence of moe_swiglu_ffn on x. With a norm, x is the residual
// stream h: the block runs on h2 = rms_norm(h) (norm->h2, computed by the
// split router at T <= 240, else by the norm kernel) and the combine adds the
// block's rounded output to h.
kmoe_status forward_stages(const kmoe_desc* desc, const void* x, const kmoe_host::SliceNorm* norm,
                           const kmoe_weight* router, const kmoe_weight* gate, const kmoe_weight* up,
                           const kmoe_weight* down, const kmoe_packed_experts* packed, void* out,
                           int32_t* topk_idx_out, void* topk_w_out, char* base, const Workspace& w, hipStream_t st) {
  const void* res = norm ? x : nullptr;
  const void* xin = norm ? norm->h2 : x;  // the block's input, after the norm
  int32_t* tidx = reinterpret_cast<int32_t*>(base + w.topk_idx);
  float* tw = reinterpret_cast<float*>(base + w.topk_w);
  int32_t* inv = reinterpret_cast<int32_t*>(base + w.inv);
  void* hs = base + w.h_sorted;
  const int chain = chain_of(*desc);
  const bool scatter = scatter_of(*desc);
  const kmoe_host::DispatchOut dout{reinterpret_cast<int32_t*>(base + w.group_sizes),
                                    reinterpret_cast<int32_t*>(base + w.offsets),
                                    reinterpret_cast<int32_t*>(base + w.active),
                                    reinterpret_cast<int32_t*>(base + w.sorted_token),
                                    reinterpret_cast<int32_t*>(base + w.sorted_expert), inv};
  if (packed_ok(*desc, packed) && family_of(*desc) == kmoe_host::kFamilyDecode &&
      kmoe_host::down_combine_fits(*desc, chain) && kmoe_host::gateup_routed_fits(*desc)) {
    // up to four tokens: the router's slices, then the gate/up kernel that
    // finishes the tokens and sorts their assignments itself, then the down
    // projection with the combine
    float* part = reinterpret_cast<float*>(base + w.route_part);
    KMOE_HIP(kmoe_host::launch_route_slices(*desc, x, *router, part, st, norm), "route kernel");
    KMOE_HIP(kmoe_host::launch_gateup_routed(*desc, chain, part, xin, *packed, hs, tidx, tw, dout, st),
             "gate/up kernel");
    KMOE_HIP(kmoe_host::launch_down_combine(*desc, chain, scatter, hs, tidx, inv, tw, *packed, out, st, res),
             "down+combine kernel");
  } else {
    KMOE_TRY(forward_general(desc, x, xin, res, norm, router, gate, up, down, packed, out, base, w, chain, scatter,
                             dout, st));
  }
  if (topk_idx_out)
    KMOE_HIP(hipMemcpyAsync(topk_idx_out, tidx, sizeof(int32_t) * desc->tokens * desc->top_k,
                            hipMemcpyDeviceToDevice, st),
             "copy topk_idx");
  if (topk_w_out) KMOE_HIP(kmoe_host::launch_topk_w_cast(*desc, tw, topk_w_out, st), "topk_w cast");
  return KMOE_OK;
}

// The other sizes: router (with the dispatch sort at T <= 16), dispatch,
// expert stages and combine.
kmoe_status forward_general(const kmoe_desc* desc, const void* x, const void* xin, const void* res,
                            const kmoe_host::SliceNorm* norm, const kmoe_weight* router, const kmoe_weight* gate,
                            const kmoe_weight* up, const kmoe_weight* down, const kmoe_packed_experts* packed,
                            void* out, char* base, const Workspace& w, int chain, bool scatter,
                            const kmoe_host::DispatchOut& dout, hipStream_t st) {
  int32_t* tidx = reinterpret_cast<int32_t*>(base + w.topk_idx);
  float* tw = reinterpret_cast<float*>(base + w.topk_w);
  int32_t* hist = reinterpret_cast<int32_t*>(base + w.hist);
  int32_t* gs = dout.group_sizes;
  int32_t* off = dout.offsets;
  int32_t* act = dout.active;
  int32_t* stok = dout.sorted_token;
  int32_t* sexp = dout.sorted_expert;
  int32_t* inv = dout.inv;
  void* hs = base + w.h_sorted;
  void* ys = base + w.y_sorted;
  if (desc->tokens <= kmoe_host::kSplitRouterMaxTokens) {
    // the split router (normalising its input rows when there is a norm, and
    // running the dispatch sort itself at T <= 16); one 64-token chunk counts
    // itself in the dispatch, two need the chunk histograms first
    float* part = reinterpret_cast<float*>(base + w.route_part);
    KMOE_HIP(kmoe_host::launch_route_split(*desc, x, *router, part, nullptr, tidx, tw, st, norm, &dout),
             "route kernels");
    if (desc->tokens > kmoe::kDispatchBlock) {
      KMOE_HIP(kmoe_host::launch_dispatch_count(*desc, tidx, hist, st), "dispatch count kernel");
      KMOE_HIP(kmoe_host::launch_dispatch(*desc, tidx, hist, gs, off, act, stok, sexp, inv, st), "dispatch kernel");
    } else if (!kmoe_host::split_router_dispatches(*desc)) {
      KMOE_HIP(kmoe_host::launch_dispatch(*desc, tidx, nullptr, gs, off, act, stok, sexp, inv, st),
               "dispatch kernel");
    }
  } else {
    if (norm)
      KMOE_HIP(kmoe_host::launch_rms_norm(*desc, x, norm->scale, norm->scale_bf16 ? KMOE_DTYPE_BF16 : KMOE_DTYPE_F32,
                                          norm->eps, norm->h2, st),
               "rms_norm kernel");
    KMOE_HIP(kmoe_host::launch_route(*desc, xin, *router, nullptr, tidx, tw, hist, st), "route kernels");
    KMOE_HIP(kmoe_host::launch_dispatch(*desc, tidx, hist, gs, off, act, stok, sexp, inv, st), "dispatch kernel");
  }
  if (packed_ok(*desc, packed) && family_of(*desc) == kmoe_host::kFamilyDecode &&
      kmoe_host::down_combine_fits(*desc, chain)) {
    // at most 32 assignments: the down projection and the combine in one kernel
    KMOE_TRY(expert_stage(*desc, kmoe_host::kStageGateUp, xin, off, act, stok, sexp, gate, up, down, packed, hs, ys,
                          st));
    KMOE_HIP(kmoe_host::launch_down_combine(*desc, chain, scatter, hs, tidx, inv, tw, *packed, out, st, res),
             "down+combine kernel");
  } else {
    KMOE_TRY(expert_stage(*desc, kmoe_host::kStageGateUp | kmoe_host::kStageDown, xin, off, act, stok, sexp, gate,
                          up, down, packed, hs, ys, st));
    KMOE_HIP(kmoe_host::launch_combine(*desc, scatter, ys, inv, tw, out, st, res), "combine kernel");
  }
  return KMOE_OK;
}

kmoe_status check_norm_args(const void* scale, kmoe_dtype scale_dtype, float epsilon) {
  if (!scale) return fail(KMOE_ERR_INVALID_ARG, "norm scale pointer is NULL");
  if (!is_float(scale_dtype)) return fail(KMOE_ERR_INVALID_ARG, "norm scale dtype must be F32 or BF16");
  if (!(epsilon >= 0.0f) || epsilon > 1.0f)
    return fail(KMOE_ERR_INVALID_ARG, "epsilon must be in [0, 1] (got %g)", (double)epsilon);
  return KMOE_OK;
}

}  // namespace

extern "C" {

kmoe_status kmoe_forward(const kmoe_desc* desc, const void* x, const kmoe_weight* router, const kmoe_weight* gate,
                         const kmoe_weight* up, const kmoe_weight* down, const kmoe_packed_experts* packed, void* out,
                         int32_t* topk_idx_out, void* topk_w_out, void* workspace, size_t workspace_bytes,
                         void* stream) {
  KMOE_TRY(check_forward_args(desc, router, gate, up, down, packed));
  if (desc->tokens > 0 && (!x || !out)) return fail(KMOE_ERR_INVALID_ARG, "kmoe_forward: x and out must be non-NULL");
  const Workspace w = layout(*desc);
  if (desc->tokens > 0 && (!workspace || workspace_bytes < w.total))
    return fail(KMOE_ERR_WORKSPACE_TOO_SMALL, "workspace of %zu bytes is smaller than the %zu required",
                workspace_bytes, w.total);
  KMOE_TRY(device_status());
  if (desc->tokens == 0) return KMOE_OK;
  return forward_stages(desc, x, nullptr, router, gate, up, down, packed, out, topk_idx_out, topk_w_out,
                        reinterpret_cast<char*>(workspace), w, (hipStream_t)stream);
}

}  // extern "C"

// The workspace of kmoe_forward_noalloc: a file-scope device array, one copy on
// every GPU the library runs on, held until the process ends. In host code the
// name is only a handle for hipGetSymbolAddress; kernels get the per-device
// address it returns.
static __device__ __align__(256) uint8_t scratch[KMOE_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The address of `scratch` on the current device, looked up once per device.
kmoe_status scratch_on_current_device(char** out) {
  int dev = -1;
  KMOE_HIP(hipGetDevice(&dev), "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices)
    return fail(KMOE_ERR_UNSUPPORTED, "device %d is beyond the %d devices kmoe_forward_noalloc serves", dev,
                kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    KMOE_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    g_scratch_ptr[dev] = p;
  }
  *out = reinterpret_cast<char*>(g_scratch_ptr[dev]);
  return KMOE_OK;
}

}  // namespace

extern "C" {

kmoe_status kmoe_forward_noalloc(const kmoe_desc* desc, const void* x, const kmoe_weight* router,
                                 const kmoe_weight* gate, const kmoe_weight* up, const kmoe_weight* down,
                                 const kmoe_packed_experts* packed, void* out, int32_t* topk_idx_out, void* topk_w_out,
                                 void* stream) {
  KMOE_TRY(check_forward_args(desc, router, gate, up, down, packed));
  if (desc->tokens > 0 && (!x || !out))
    return fail(KMOE_ERR_INVALID_ARG, "kmoe_forward_noalloc: x and out must be non-NULL");
  const Workspace w = layout(*desc);
  if (w.total > (size_t)KMOE_NOALLOC_SCRATCH_BYTES)
    return fail(KMOE_ERR_WORKSPACE_TOO_SMALL,
                "kmoe_forward_noalloc: the call needs %zu bytes of workspace, beyond its %zu-byte scratch; use "
                "kmoe_forward with a workspace",
                w.total, (size_t)KMOE_NOALLOC_SCRATCH_BYTES);
  KMOE_TRY(device_status());
  if (desc->tokens == 0) return KMOE_OK;
  char* base = nullptr;
  KMOE_TRY(scratch_on_current_device(&base));
  // every workspace buffer is written before it is read within a call, so the
  // previous call's contents need no clearing
  return forward_stages(desc, x, nullptr, router, gate, up, down, packed, out, topk_idx_out, topk_w_out, base, w,
                        (hipStream_t)stream);
}

kmoe_status kmoe_rms_norm(const kmoe_desc* desc, const void* x, const void* scale, kmoe_dtype scale_dtype,
                          float epsilon, void* out, void* stream) {
  KMOE_TRY(check_desc(desc));
  KMOE_TRY(check_norm_args(scale, scale_dtype, epsilon));
  if (desc->tokens > 0 && (!x || !out)) return fail(KMOE_ERR_INVALID_ARG, "kmoe_rms_norm: x and out must be non-NULL");
  KMOE_TRY(device_status());
  if (desc->tokens == 0) return KMOE_OK;
  KMOE_HIP(kmoe_host::launch_rms_norm(*desc, x, scale, scale_dtype, epsilon, out, (hipStream_t)stream),
           "rms_norm kernel");
  return KMOE_OK;
}

kmoe_status kmoe_forward_block(const kmoe_desc* desc, const void* h, const void* norm_scale, kmoe_dtype norm_dtype,
                               float epsilon, const kmoe_weight* router, const kmoe_weight* gate,
                               const kmoe_weight* up, const kmoe_weight* down, const kmoe_packed_experts* packed,
                               void* out, int32_t* topk_idx_out, void* topk_w_out, void* workspace,
                               size_t workspace_bytes, void* stream) {
  KMOE_TRY(check_forward_args(desc, router, gate, up, down, packed));
  KMOE_TRY(check_norm_args(norm_scale, norm_dtype, epsilon));
  if (desc->tokens > 0 && (!h || !out))
    return fail(KMOE_ERR_INVALID_ARG, "kmoe_forward_block: h and out must be non-NULL");
  if (desc->tokens > 0 && out == h) return fail(KMOE_ERR_INVALID_ARG, "kmoe_forward_block: out must not alias h");
  const Workspace w = layout(*desc);
  if (desc->tokens > 0 && (!workspace || workspace_bytes < w.total))
    return fail(KMOE_ERR_WORKSPACE_TOO_SMALL, "workspace of %zu bytes is smaller than the %zu required",
                workspace_bytes, w.total);
  KMOE_TRY(device_status());
  if (desc->tokens == 0) return KMOE_OK;
  char* base = reinterpret_cast<char*>(workspace);
  const kmoe_host::SliceNorm nm{norm_scale, norm_dtype == KMOE_DTYPE_BF16 ? 1 : 0, epsilon, base + w.normed};
  return forward_stages(desc, h, &nm, router, gate, up, down, packed, out, topk_idx_out, topk_w_out, base, w,
                        (hipStream_t)stream);
}

kmoe_status kmoe_prepack(const kmoe_desc* desc, const kmoe_weight* gate, const kmoe_weight* up,
                         const kmoe_weight* down, const kmoe_packed_experts* packed, void* stream) {
  KMOE_TRY(check_desc(desc));
  KMOE_TRY(check_weight(gate, "gate"));
  KMOE_TRY(check_weight(up, "up"));
  KMOE_TRY(check_weight(down, "down"));
  if (gate->dtype != KMOE_DTYPE_I8 || up->dtype != KMOE_DTYPE_I8 || down->dtype != KMOE_DTYPE_I8)
    return fail(KMOE_ERR_UNSUPPORTED, "kmoe_prepack packs int8 (Q8) experts only");
  if (!packed || !packed->w13 || !packed->s13 || !packed->w2 || !packed->s2)
    return fail(KMOE_ERR_INVALID_ARG, "kmoe_prepack: packed buffers must be non-NULL");
  if (packed->num_experts != desc->num_experts || packed->hidden != desc->hidden ||
      packed->intermediate != desc->intermediate)
    return fail(KMOE_ERR_INVALID_ARG, "kmoe_prepack: the packed shapes must be the desc's E, D and I");
  if (desc->hidden % 64 || desc->intermediate % 64)
    return fail(KMOE_ERR_UNSUPPORTED, "packed experts need hidden and intermediate divisible by 64");
  KMOE_TRY(device_status());
  KMOE_HIP(kmoe_host::launch_prepack(*desc, *gate, *up, *down, *packed, (hipStream_t)stream), "prepack kernels");
  return KMOE_OK;
}

kmoe_status kmoe_to_compute_dtype(const kmoe_weight* w, int64_t outer, int64_t channels,
                                  int64_t rows_per_scale_block, kmoe_dtype out_dtype, void* out, void* stream) {
  KMOE_TRY(check_weight(w, "weight"));
  if (outer < 0 || channels < 1 || rows_per_scale_block < 1)
    return fail(KMOE_ERR_INVALID_ARG, "kmoe_to_compute_dtype: bad shape");
  if (!is_float(out_dtype)) return fail(KMOE_ERR_INVALID_ARG, "out_dtype must be F32 or BF16");
  if (!out) return fail(KMOE_ERR_INVALID_ARG, "out is NULL");
  KMOE_TRY(device_status());
  if (outer == 0) return KMOE_OK;
  KMOE_HIP(kmoe_host::launch_to_compute_dtype(*w, outer, channels, rows_per_scale_block, out_dtype, out,
                                              (hipStream_t)stream),
           "to_compute_dtype kernel");
  return KMOE_OK;
}

kmoe_status kmoe_quantize_per_channel(int64_t experts, int64_t rows, int64_t channels, const void* w,
                                      kmoe_dtype w_dtype, int8_t* q, float* s, void* stream) {
  if (experts < 1 || rows < 1 || channels < 1) return fail(KMOE_ERR_INVALID_ARG, "quantize: bad shape");
  if (!is_float(w_dtype)) return fail(KMOE_ERR_INVALID_ARG, "quantize: w_dtype must be F32 or BF16");
  if (!w || !q || !s) return fail(KMOE_ERR_INVALID_ARG, "quantize: NULL buffer");
  if (experts > 65535) return fail(KMOE_ERR_UNSUPPORTED, "quantize: too many experts");
  KMOE_TRY(device_status());
  KMOE_HIP(kmoe_host::launch_quantize_per_channel(experts, rows, channels, w, w_dtype, q, s, (hipStream_t)stream),
           "quantize kernel");
  return KMOE_OK;
}

}  // extern "C"
