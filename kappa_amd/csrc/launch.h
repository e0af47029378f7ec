// Host-side launch wrappers shared between the kernel files and the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include "host.h"
#include "kmoe.h"

namespace kmoe_host {

// route.hip
hipError_t launch_route(const kmoe_desc& d, const void* x, const kmoe_weight& router, float* logits, int32_t* topk_idx,
                        float* topk_w, int32_t* hist, hipStream_t st);
// per-64-token-chunk expert histograms of the selections (for launch_dispatch)
hipError_t launch_dispatch_count(const kmoe_desc& d, const int32_t* topk_idx, int32_t* hist, hipStream_t st);
// Split router (many blocks per token; same logits and selections as
// launch_route): part holds route_split_part_floats(d) floats of workspace.
// With a SliceNorm, x is the residual stream h: the router reduces and
// normalises the rows itself (rms_norm, kappa/qwen3/norms.py:10-16), routes
// the normalised rows and writes them to h2 for the expert kernels.
struct SliceNorm {
  const void* scale;  // [D] RMSNorm scale; NULL: x is routed as given
  int scale_bf16;
  float eps;
  void* h2;  // [T][D] normalised rows (activation dtype)
};
// The dispatch sort's outputs (as launch_dispatch). Given to the split router,
// it runs the sort itself when the finish is a single block of one wave per
// token (T <= 16; split_router_dispatches(d)), and the caller skips
// launch_dispatch.
struct DispatchOut {
  int32_t* group_sizes;
  int32_t* offsets;
  int32_t* active;
  int32_t* sorted_token;
  int32_t* sorted_expert;
  int32_t* inv;
};
hipError_t launch_route_split(const kmoe_desc& d, const void* x, const kmoe_weight& router, float* part, float* logits,
                              int32_t* topk_idx, float* topk_w, hipStream_t st, const SliceNorm* norm = nullptr,
                              const DispatchOut* dispatch = nullptr);
// The split router's first kernel alone (group partials into part; with a
// SliceNorm it also writes the normalised rows), for a caller that finishes
// the tokens itself (launch_gateup_routed); route_split_groups(d) partials per
// token and expert.
hipError_t launch_route_slices(const kmoe_desc& d, const void* x, const kmoe_weight& router, float* part,
                               hipStream_t st, const SliceNorm* norm = nullptr);
// The two-phase router (route_mfma_fits): topk_idx, topk_w and the per-64-token
// expert histograms hist (launch_dispatch's input) from x; scratch holds
// route_mfma_scratch_bytes(d) bytes. Same selections and weights as
// launch_route (no logits).
hipError_t launch_route_mfma(const kmoe_desc& d, const void* x, const kmoe_weight& router, void* scratch,
                             int32_t* topk_idx, float* topk_w, int32_t* hist, hipStream_t st);
hipError_t launch_dispatch(const kmoe_desc& d, const int32_t* topk_idx, const int32_t* hist, int32_t* group_sizes,
                           int32_t* offsets, int32_t* active, int32_t* sorted_token, int32_t* sorted_expert,
                           int32_t* inv, hipStream_t st);

// expert.hip
// chain: kmoe::kChainAct or kmoe::kChainF32 (common.h); with kChainF32 and bf16
// activations h_sorted holds [T*K][2I] bf16 (the hi and lo planes of h).
// Packed int8 experts on MFMA. With h_scale (M floats, the whole-block call
// only) and down_planes_fits, the down stage first turns h_sorted's rows into
// int8 planes in place (the caller's h_sorted is then no longer hi/lo planes).
hipError_t launch_expert_packed(const kmoe_desc& d, int chain, int family, int stages, const void* x,
                                const int32_t* offsets, const int32_t* active, const int32_t* sorted_token,
                                const kmoe_packed_experts& p, void* h_sorted, void* y_sorted, hipStream_t st,
                                float* h_scale = nullptr);
// Layout-native experts (any weight kind), one sequential fmaf chain per output.
hipError_t launch_expert_generic(const kmoe_desc& d, int chain, int stages, const void* x, const int32_t* sorted_token,
                                 const int32_t* sorted_expert, const kmoe_weight* gate, const kmoe_weight* up,
                                 const kmoe_weight* down, void* h_sorted, void* y_sorted, hipStream_t st);
// out = the terms round(w * y_sorted[inv]) summed in f32 and rounded once
// (scatter = false) or added into a rounded running sum (scatter = true)
// [+ residual res, rounded again], res may be NULL
hipError_t launch_combine(const kmoe_desc& d, bool scatter, const void* y_sorted, const int32_t* inv,
                          const float* topk_w, void* out, hipStream_t st, const void* res = nullptr);
// Packed decode with T * K <= 32 and K <= 8 (down_combine_fits): the down
// projection and the combine (with residual res, may be NULL) in one kernel;
// out is bit-identical to the packed decode down kernel followed by
// launch_combine.
bool down_combine_fits(const kmoe_desc& d, int chain);
hipError_t launch_down_combine(const kmoe_desc& d, int chain, bool scatter, const void* h_sorted,
                               const int32_t* topk_idx, const int32_t* inv, const float* topk_w,
                               const kmoe_packed_experts& p, void* out, hipStream_t st, const void* res);
hipError_t launch_topk_w_cast(const kmoe_desc& d, const float* topk_w, void* out, hipStream_t st);
// Packed decode with T <= 4 (gateup_routed_fits): the gate/up kernel finishes
// the tokens from the split router's partials (launch_route_slices) and runs
// the dispatch sort itself, writing topk_idx, topk_w and the dispatch arrays
// as launch_route_split + launch_dispatch would; h_sorted is bit-identical.
bool gateup_routed_fits(const kmoe_desc& d);
hipError_t launch_gateup_routed(const kmoe_desc& d, int chain, const float* part, const void* x,
                                const kmoe_packed_experts& p, void* h_sorted, int32_t* topk_idx, float* topk_w,
                                const DispatchOut& dout, hipStream_t st);

// block.hip
size_t rms_norm_lds_bytes(int64_t D);
hipError_t launch_rms_norm(const kmoe_desc& d, const void* h, const void* scale, kmoe_dtype scale_dtype, float eps,
                           void* out, hipStream_t st);

// weights.hip
hipError_t launch_prepack(const kmoe_desc& d, const kmoe_weight& gate, const kmoe_weight& up, const kmoe_weight& down,
                          const kmoe_packed_experts& p, hipStream_t st);
hipError_t launch_to_compute_dtype(const kmoe_weight& w, int64_t outer, int64_t channels, int64_t rows_per_block,
                                   kmoe_dtype out_dtype, void* out, hipStream_t st);
hipError_t launch_quantize_per_channel(int64_t E, int64_t Kd, int64_t N, const void* w, kmoe_dtype w_dtype, int8_t* q,
                                       float* s, hipStream_t st);

}  // namespace kmoe_host
