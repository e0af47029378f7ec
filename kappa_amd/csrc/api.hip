// C ABI entry points (include/kmoe.h): each runs its argument check (host.cpp,
// no HIP call), the device check, then the stage sequence of moe_swiglu_ffn
// (kappa/qwen3/ffn_moe.py:226-299).
#include <mutex>

#include "common.h"
#include "launch.h"

using namespace kmoe_host;

namespace {

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

#define KMOE_HIP(expr, what)                          \
  do {                                                \
    hipError_t _e = (expr);                           \
    if (_e != hipSuccess) return hip_fail(_e, what);  \
  } while (0)

kmoe_status expert_stage(const kmoe_desc& d, int stages, const void* x, const int32_t* offsets, const int32_t* active,
                         const int32_t* sorted_token, const int32_t* sorted_expert, const kmoe_weight* gate,
                         const kmoe_weight* up, const kmoe_weight* down, const kmoe_packed_experts* packed,
                         void* h_sorted, void* y_sorted, hipStream_t st, float* h_scale = nullptr) {
  hipError_t e;
  if (packed_ok(d, packed)) {
    e = launch_expert_packed(d, chain_of(d), family_of(d), stages, x, offsets, active, sorted_token, *packed,
                             h_sorted, y_sorted, st, h_scale);
  } else {
    e = launch_expert_generic(d, chain_of(d), stages, x, sorted_token, sorted_expert, gate, up, down, h_sorted,
                              y_sorted, st);
  }
  if (e != hipSuccess) return hip_fail(e, "expert kernels");
  return KMOE_OK;
}

}  // namespace

extern "C" {

const char* kmoe_version(void) { return "kmoe 0.2.0 (gfx950)"; }

int kmoe_abi_version(void) { return KMOE_ABI_VERSION; }

const char* kmoe_status_string(kmoe_status s) { return status_string(s); }

const char* kmoe_last_error(void) { return last_error(); }

kmoe_status kmoe_device_check(void) { return device_status(); }

kmoe_status kmoe_workspace_bytes(const kmoe_desc* desc, size_t* bytes) { return validate_workspace_bytes(desc, bytes); }

kmoe_status kmoe_route_scratch_bytes(const kmoe_desc* desc, size_t* bytes) {
  return validate_route_scratch_bytes(desc, bytes);
}

kmoe_status kmoe_prepack_bytes(const kmoe_desc* desc, kmoe_packed_sizes* sizes) {
  return validate_prepack_bytes(desc, sizes);
}

kmoe_status kmoe_route(const kmoe_desc* desc, const void* x, const kmoe_weight* router, float* logits,
                       void* scratch, size_t scratch_bytes, int32_t* topk_idx, float* topk_w, int32_t* block_hist,
                       void* stream) {
  KMOE_TRY(validate_route(desc, x, router, scratch, scratch_bytes, topk_idx, topk_w, block_hist));
  KMOE_TRY(device_status());
  if (desc->tokens == 0) return KMOE_OK;
  hipError_t e =
      !logits && scratch && route_mfma_fits(*desc, *router)
          ? launch_route_mfma(*desc, x, *router, scratch, topk_idx, topk_w, block_hist, (hipStream_t)stream)
          : launch_route(*desc, x, *router, logits, topk_idx, topk_w, block_hist, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "route kernels");
  return KMOE_OK;
}

kmoe_status kmoe_dispatch(const kmoe_desc* desc, const int32_t* topk_idx, const int32_t* block_hist,
                          int32_t* group_sizes, int32_t* offsets, int32_t* active, int32_t* sorted_token,
                          int32_t* sorted_expert, int32_t* inv, void* stream) {
  KMOE_TRY(validate_dispatch(desc, topk_idx, block_hist, group_sizes, offsets, active, sorted_token, sorted_expert,
                             inv));
  KMOE_TRY(device_status());
  if (desc->tokens == 0) return fail(KMOE_ERR_UNSUPPORTED, "kmoe_dispatch: tokens == 0");
  hipError_t e = launch_dispatch(*desc, topk_idx, block_hist, group_sizes, offsets, active, sorted_token,
                                 sorted_expert, inv, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "dispatch kernel");
  return KMOE_OK;
}

kmoe_status kmoe_expert_ffn(const kmoe_desc* desc, const void* x, const int32_t* offsets, const int32_t* active,
                            const int32_t* sorted_token, const int32_t* sorted_expert, const kmoe_weight* gate,
                            const kmoe_weight* up, const kmoe_weight* down, const kmoe_packed_experts* packed,
                            void* h_sorted, void* y_sorted, void* stream) {
  const int both = kStageGateUp | kStageDown;
  KMOE_TRY(validate_expert(desc, both, x, offsets, active, sorted_token, sorted_expert, gate, up, down, packed,
                           h_sorted, y_sorted));
  KMOE_TRY(device_status());
  if (desc->tokens == 0) return KMOE_OK;
  return expert_stage(*desc, both, x, offsets, active, sorted_token, sorted_expert, gate, up, down, packed, h_sorted,
                      y_sorted, (hipStream_t)stream);
}

kmoe_status kmoe_expert_gate_up(const kmoe_desc* desc, const void* x, const int32_t* offsets, const int32_t* active,
                                const int32_t* sorted_token, const int32_t* sorted_expert, const kmoe_weight* gate,
                                const kmoe_weight* up, const kmoe_packed_experts* packed, void* h_sorted,
                                void* stream) {
  KMOE_TRY(validate_expert(desc, kStageGateUp, x, offsets, active, sorted_token, sorted_expert, gate, up, nullptr,
                           packed, h_sorted, nullptr));
  KMOE_TRY(device_status());
  if (desc->tokens == 0) return KMOE_OK;
  return expert_stage(*desc, kStageGateUp, x, offsets, active, sorted_token, sorted_expert, gate, up, nullptr, packed,
                      h_sorted, nullptr, (hipStream_t)stream);
}

kmoe_status kmoe_expert_down(const kmoe_desc* desc, const void* h_sorted, const int32_t* offsets,
                             const int32_t* active, const int32_t* sorted_expert, const kmoe_weight* down,
                             const kmoe_packed_experts* packed, void* y_sorted, void* stream) {
  KMOE_TRY(validate_expert(desc, kStageDown, h_sorted, offsets, active, nullptr, sorted_expert, nullptr, nullptr,
                           down, packed, h_sorted, y_sorted));
  KMOE_TRY(device_status());
  if (desc->tokens == 0) return KMOE_OK;
  return expert_stage(*desc, kStageDown, nullptr, offsets, active, nullptr, sorted_expert, nullptr, nullptr, down,
                      packed, const_cast<void*>(h_sorted), y_sorted, (hipStream_t)stream);
}

kmoe_status kmoe_combine(const kmoe_desc* desc, const void* y_sorted, const int32_t* inv, const float* topk_w,
                         void* out, void* stream) {
  KMOE_TRY(validate_combine(desc, y_sorted, inv, topk_w, out));
  KMOE_TRY(device_status());
  if (desc->tokens == 0) return KMOE_OK;
  hipError_t e = launch_combine(*desc, scatter_of(*desc), y_sorted, inv, topk_w, out, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "combine kernel");
  return KMOE_OK;
}

}  // extern "C"

namespace {

kmoe_status forward_general(const kmoe_desc* desc, const void* x, const void* xin, const void* res,
                            const SliceNorm* norm, const kmoe_weight* router, const kmoe_weight* gate,
                            const kmoe_weight* up, const kmoe_weight* down, const kmoe_packed_experts* packed,
                            void* out, char* base, const Workspace& w, int chain, bool scatter,
                            const DispatchOut& dout, hipStream_t st);

// The stage sequence of moe_swiglu_ffn on x. With a norm, x is the residual
// stream h: the block runs on h2 = rms_norm(h) (norm->h2, computed by the
// split router at T <= 240, else by the norm kernel) and the combine adds the
// block's rounded output to h.
kmoe_status forward_stages(const kmoe_desc* desc, const void* x, const SliceNorm* norm,
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
  const DispatchOut dout{reinterpret_cast<int32_t*>(base + w.group_sizes),
                                    reinterpret_cast<int32_t*>(base + w.offsets),
                                    reinterpret_cast<int32_t*>(base + w.active),
                                    reinterpret_cast<int32_t*>(base + w.sorted_token),
                                    reinterpret_cast<int32_t*>(base + w.sorted_expert), inv};
  if (packed_ok(*desc, packed) && family_of(*desc) == kFamilyDecode &&
      down_combine_fits(*desc, chain) && gateup_routed_fits(*desc)) {
    // up to four tokens: the router's slices, then the gate/up kernel that
    // finishes the tokens and sorts their assignments itself, then the down
    // projection with the combine
    float* part = reinterpret_cast<float*>(base + w.route_part);
    KMOE_HIP(launch_route_slices(*desc, x, *router, part, st, norm), "route kernel");
    KMOE_HIP(launch_gateup_routed(*desc, chain, part, xin, *packed, hs, tidx, tw, dout, st),
             "gate/up kernel");
    KMOE_HIP(launch_down_combine(*desc, chain, scatter, hs, tidx, inv, tw, *packed, out, st, res),
             "down+combine kernel");
  } else {
    KMOE_TRY(forward_general(desc, x, xin, res, norm, router, gate, up, down, packed, out, base, w, chain, scatter,
                             dout, st));
  }
  if (topk_idx_out)
    KMOE_HIP(hipMemcpyAsync(topk_idx_out, tidx, sizeof(int32_t) * desc->tokens * desc->top_k,
                            hipMemcpyDeviceToDevice, st),
             "copy topk_idx");
  if (topk_w_out) KMOE_HIP(launch_topk_w_cast(*desc, tw, topk_w_out, st), "topk_w cast");
  return KMOE_OK;
}

// The other sizes: router (with the dispatch sort at T <= 16), dispatch,
// expert stages and combine.
kmoe_status forward_general(const kmoe_desc* desc, const void* x, const void* xin, const void* res,
                            const SliceNorm* norm, const kmoe_weight* router, const kmoe_weight* gate,
                            const kmoe_weight* up, const kmoe_weight* down, const kmoe_packed_experts* packed,
                            void* out, char* base, const Workspace& w, int chain, bool scatter,
                            const DispatchOut& dout, hipStream_t st) {
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
  if (desc->tokens <= kSplitRouterMaxTokens) {
    // the split router (normalising its input rows when there is a norm, and
    // running the dispatch sort itself at T <= 16); one 64-token chunk counts
    // itself in the dispatch, two need the chunk histograms first
    float* part = reinterpret_cast<float*>(base + w.route_part);
    KMOE_HIP(launch_route_split(*desc, x, *router, part, nullptr, tidx, tw, st, norm, &dout),
             "route kernels");
    if (desc->tokens > kmoe::kDispatchBlock) {
      KMOE_HIP(launch_dispatch_count(*desc, tidx, hist, st), "dispatch count kernel");
      KMOE_HIP(launch_dispatch(*desc, tidx, hist, gs, off, act, stok, sexp, inv, st), "dispatch kernel");
    } else if (!split_router_dispatches(*desc)) {
      KMOE_HIP(launch_dispatch(*desc, tidx, nullptr, gs, off, act, stok, sexp, inv, st),
               "dispatch kernel");
    }
  } else {
    if (norm)
      KMOE_HIP(launch_rms_norm(*desc, x, norm->scale, norm->scale_bf16 ? KMOE_DTYPE_BF16 : KMOE_DTYPE_F32,
                                          norm->eps, norm->h2, st),
               "rms_norm kernel");
    if (route_mfma_preferred(*desc, *router))
      KMOE_HIP(launch_route_mfma(*desc, xin, *router, base + w.route_part, tidx, tw, hist, st), "route kernels");
    else
      KMOE_HIP(launch_route(*desc, xin, *router, nullptr, tidx, tw, hist, st), "route kernels");
    KMOE_HIP(launch_dispatch(*desc, tidx, hist, gs, off, act, stok, sexp, inv, st), "dispatch kernel");
  }
  if (packed_ok(*desc, packed) && family_of(*desc) == kFamilyDecode &&
      down_combine_fits(*desc, chain)) {
    // at most 32 assignments: the down projection and the combine in one kernel
    KMOE_TRY(expert_stage(*desc, kStageGateUp, xin, off, act, stok, sexp, gate, up, down, packed, hs, ys,
                          st));
    KMOE_HIP(launch_down_combine(*desc, chain, scatter, hs, tidx, inv, tw, *packed, out, st, res),
             "down+combine kernel");
  } else {
    // with down_planes_fits the workspace's h rows become int8 planes, their
    // scales in w.h_scale
    float* hscale = down_planes_fits(*desc) ? reinterpret_cast<float*>(base + w.h_scale) : nullptr;
    KMOE_TRY(expert_stage(*desc, kStageGateUp | kStageDown, xin, off, act, stok, sexp, gate,
                          up, down, packed, hs, ys, st, hscale));
    KMOE_HIP(launch_combine(*desc, scatter, ys, inv, tw, out, st, res), "combine kernel");
  }
  return KMOE_OK;
}

}  // namespace

extern "C" {

kmoe_status kmoe_forward(const kmoe_desc* desc, const void* x, const kmoe_weight* router, const kmoe_weight* gate,
                         const kmoe_weight* up, const kmoe_weight* down, const kmoe_packed_experts* packed, void* out,
                         int32_t* topk_idx_out, void* topk_w_out, void* workspace, size_t workspace_bytes,
                         void* stream) {
  Workspace w;
  KMOE_TRY(validate_forward(desc, x, router, gate, up, down, packed, out, workspace, workspace_bytes, &w));
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
  Workspace w;
  KMOE_TRY(validate_forward_noalloc(desc, x, router, gate, up, down, packed, out, (size_t)KMOE_NOALLOC_SCRATCH_BYTES,
                                    &w));
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
  KMOE_TRY(validate_rms_norm(desc, x, scale, scale_dtype, epsilon, out));
  KMOE_TRY(device_status());
  if (desc->tokens == 0) return KMOE_OK;
  KMOE_HIP(launch_rms_norm(*desc, x, scale, scale_dtype, epsilon, out, (hipStream_t)stream),
           "rms_norm kernel");
  return KMOE_OK;
}

kmoe_status kmoe_forward_block(const kmoe_desc* desc, const void* h, const void* norm_scale, kmoe_dtype norm_dtype,
                               float epsilon, const kmoe_weight* router, const kmoe_weight* gate,
                               const kmoe_weight* up, const kmoe_weight* down, const kmoe_packed_experts* packed,
                               void* out, int32_t* topk_idx_out, void* topk_w_out, void* workspace,
                               size_t workspace_bytes, void* stream) {
  Workspace w;
  KMOE_TRY(validate_forward_block(desc, h, norm_scale, norm_dtype, epsilon, router, gate, up, down, packed, out,
                                  workspace, workspace_bytes, &w));
  KMOE_TRY(device_status());
  if (desc->tokens == 0) return KMOE_OK;
  char* base = reinterpret_cast<char*>(workspace);
  const SliceNorm nm{norm_scale, norm_dtype == KMOE_DTYPE_BF16 ? 1 : 0, epsilon, base + w.normed};
  return forward_stages(desc, h, &nm, router, gate, up, down, packed, out, topk_idx_out, topk_w_out, base, w,
                        (hipStream_t)stream);
}

kmoe_status kmoe_prepack(const kmoe_desc* desc, const kmoe_weight* gate, const kmoe_weight* up,
                         const kmoe_weight* down, const kmoe_packed_experts* packed, void* stream) {
  KMOE_TRY(validate_prepack(desc, gate, up, down, packed));
  KMOE_TRY(device_status());
  KMOE_HIP(launch_prepack(*desc, *gate, *up, *down, *packed, (hipStream_t)stream), "prepack kernels");
  return KMOE_OK;
}

kmoe_status kmoe_to_compute_dtype(const kmoe_weight* w, int64_t outer, int64_t channels,
                                  int64_t rows_per_scale_block, kmoe_dtype out_dtype, void* out, void* stream) {
  KMOE_TRY(validate_to_compute_dtype(w, outer, channels, rows_per_scale_block, out_dtype, out));
  KMOE_TRY(device_status());
  if (outer == 0) return KMOE_OK;
  KMOE_HIP(launch_to_compute_dtype(*w, outer, channels, rows_per_scale_block, out_dtype, out,
                                              (hipStream_t)stream),
           "to_compute_dtype kernel");
  return KMOE_OK;
}

kmoe_status kmoe_quantize_per_channel(int64_t experts, int64_t rows, int64_t channels, const void* w,
                                      kmoe_dtype w_dtype, int8_t* q, float* s, void* stream) {
  KMOE_TRY(validate_quantize(experts, rows, channels, w, w_dtype, q, s));
  KMOE_TRY(device_status());
  KMOE_HIP(launch_quantize_per_channel(experts, rows, channels, w, w_dtype, q, s, (hipStream_t)stream),
           "quantize kernel");
  return KMOE_OK;
}

}  // extern "C"
