// Host-only side of the C ABI: the constants the kernels and the host share,
// argument validation, the workspace layout and the choice of rounding program
// and kernel family. Plain C++ (no HIP headers), so it also builds with g++
// under the address and undefined-behaviour sanitizers for the CPU tests.
//
// Reference: the ValueErrors of moe_swiglu_ffn and _route
// (kappa/qwen3/ffn_moe.py:47-48, 239-240, 251-252, 299) and the decode switch
// _effective_moe_impl (:219-223).
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "kmoe.h"

namespace kmoe {

// Slice length of the canonical router summation order: each slice of 64
// consecutive hidden indices is a sequential fmaf chain from +0.0f, and the
// slice partials are combined by a pairwise tree.
constexpr int kRouterSlice = 64;
// Tokens per dispatch block (per-block expert histograms).
constexpr int kDispatchBlock = 64;
// Largest expert count / top-k the routing kernels hold in registers and LDS.
constexpr int kMaxExperts = 1024;
constexpr int kMaxTopK = 64;
constexpr int kMaxRouterSlices = 64;  // D <= 4096
// Decode kernels keep up to this many 16-row blocks of one expert in registers.
constexpr int kDecodeMaxRowBlocks = 4;  // T <= 64 tokens
constexpr int kRowsPathMaxTokens = 128;  // above the decode sizes, the row-group kernels up to this T
constexpr int kDownCombineMaxRows = 8;          // assignments per block of the fused decode down + combine
constexpr int kDownCombineMaxAssignments = 32;  // T * K it takes

// Rounding chain of the expert products (which array program runs):
//   kChainAct: _moe_gather_einsum / _moe_fixed_capacity (kappa/qwen3/ffn_moe.py:99-102,
//     146-152): weights bf16(q * bf16(s)), g, u, every step of silu(g) * u and y
//     rounded to the activation dtype;
//   kChainF32: _moe_ragged (:202-213): weights q * s in f32 (the scale applied to the
//     f32 sum, a per-output-channel factor), g, u, h and the down sum in f32, only y
//     rounded. With bf16 activations h is stored as two bf16 planes per row, hi =
//     bf16(h) and lo = bf16(h - hi) ([M][2I]), which the MFMA down products take as
//     two operands (hi + lo carries h to ~2^-17 relative).
constexpr int kChainAct = 0;
constexpr int kChainF32 = 1;
// The whole-block call's large prefill chunks (down_planes_fits) feed the down
// product h as two int8 digit planes of a 15-bit fixed-point value with one
// power-of-two scale per row (k_h_planes), on the integer MFMA; rows up to
// this many 64-wide chunks (I <= 2048).
constexpr int kPlanesMaxChunks = 32;

}  // namespace kmoe

namespace kmoe_host {

// The whole-block call routes up to this many tokens with the split router
// (at T=256 the split router took 13 us against 21 us for k_route, whose
// blocks then hold one token each; from 512 tokens on they are even; 240 keeps
// every call up to 291 tokens inside the no-allocation scratch).
constexpr int kSplitRouterMaxTokens = 240;
// The split router runs the dispatch sort itself when its finish is a single
// block of one wave per token.
inline bool split_router_dispatches(const kmoe_desc& d) { return d.tokens <= 16; }

// Stage selection bits for the expert launchers.
constexpr int kStageGateUp = 1;  // x -> h_sorted (gate/up products + SwiGLU)
constexpr int kStageDown = 2;    // h_sorted -> y_sorted (down product)
// Kernel families of the packed experts: the GEMV-style decode kernels (T <= 64),
// their row-group form (T <= 128, the 30B and 235B shapes; others fall back to
// the GEMMs), the grouped GEMMs.
constexpr int kFamilyDecode = 0;
constexpr int kFamilyRows = 1;
constexpr int kFamilyGemm = 2;

// Rows an expert keeps: the fixed_capacity slot limit, or no limit.
inline int capacity_of(const kmoe_desc& d) {
  return d.expert_capacity > 0 && d.expert_capacity < 0x7fffffff ? (int)d.expert_capacity : 0x7fffffff;
}

inline size_t dtype_size(kmoe_dtype t) {
  switch (t) {
    case KMOE_DTYPE_F32:
      return 4;
    case KMOE_DTYPE_BF16:
      return 2;
    case KMOE_DTYPE_I8:
      return 1;
  }
  return 0;
}

// The integer a caller stored in an enum field or argument. A C caller (ctypes,
// cgo) may pass any int, and loading an out-of-range value as the enum type is
// undefined in C++, so the checks read the object representation instead.
template <typename En>
inline int enum_value(const En& e) {
  static_assert(sizeof(En) == sizeof(int), "the ABI enums are int-sized");
  int v;
  __builtin_memcpy(&v, &e, sizeof v);
  return v;
}

// Split router: group partials per token and expert, and their floats.
int route_split_groups(const kmoe_desc& d);
size_t route_split_part_floats(const kmoe_desc& d);
// Two-phase router (MFMA logits, canonical recompute of the candidates): the
// shapes it takes (bf16 activations and router, D one of 512, 1024, 2048,
// 4096, E % 16 == 0, E <= 256) and its scratch: the router transposed
// to bf16 [E][8][D/64][8] (offset 0) and the partial sums of squares of its
// columns [D/256][E] f32 (offset part 1); part 2 is the total.
bool route_mfma_fits(const kmoe_desc& d, const kmoe_weight& router);
// Whether kmoe_forward routes with it: it costs about one block's latency per
// round of blocks (16 tokens per block up to D = 2048, 8 at D = 4096) where the
// all-VALU k_route grows with T. Alone, with the router in cache, k_route wins
// up to ~2300 tokens at D = 2048 and ~4000 at D = 4096; inside the layer, where
// the expert GEMMs have evicted the router, whole layers with the one-phase and
// the two-phase router (two interleaved rounds) ran 30B-A3B T = 2048 / 2560 /
// 3072 / 4096 310 / 386 / 436 / 519 against 311 / 376 / 435 / 505 us, 235B-A22B
// T = 2048 / 3072 / 4096 874 / 1350 / 1696 against 873 / 1338 / 1668 us: even at
// 2048 tokens, ahead above, for both widths.
bool route_mfma_preferred(const kmoe_desc& d, const kmoe_weight& router);
size_t route_mfma_scratch_offsets(const kmoe_desc& d, int part);
size_t route_mfma_scratch_bytes(const kmoe_desc& d);

// --- status and message ------------------------------------------------------
// Records the message of a failing status for kmoe_last_error (per thread).
kmoe_status fail(kmoe_status st, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
const char* last_error();
const char* status_string(kmoe_status s);

#define KMOE_TRY(expr)            \
  do {                            \
    kmoe_status _s = (expr);      \
    if (_s != KMOE_OK) return _s; \
  } while (0)

// --- program, family, layout -------------------------------------------------
bool is_float(kmoe_dtype t);
kmoe_impl effective_impl(const kmoe_desc& d);  // _effective_moe_impl (:219-223)
int chain_of(const kmoe_desc& d);              // the expert products' rounding chain
bool scatter_of(const kmoe_desc& d);           // the combine: bf16 running add (true) or f32 sum
int family_of(const kmoe_desc& d);
bool packed_ok(const kmoe_desc& d, const kmoe_packed_experts* p);

// Byte offsets of the workspace buffers; block: also the normalised rows h2
// that only kmoe_forward_block writes.
struct Workspace {
  size_t topk_idx, topk_w, hist, group_sizes, offsets, active, sorted_token, sorted_expert, inv, h_sorted,
      y_sorted, route_part, h_scale, normed, total;
};
// Whether the whole-block call's f32-chain down product takes h as int8 planes
// (k_h_planes + the integer k_gemm): bf16 activations, the ragged program, at
// least 96 rows per expert on average (where the grouped GEMMs run 64-row
// planes tiles against 160-row bf16 ones; below, at T = 256 to 1280, the
// planes measured even with the bf16 hi/lo tiles), D % 256 == 0,
// I % 128 == 0, I <= 2048. The workspace then holds one scale per row
// (Workspace::h_scale).
bool down_planes_fits(const kmoe_desc& d);
Workspace layout(const kmoe_desc& d, bool block);

// --- argument checks ---------------------------------------------------------
kmoe_status check_desc(const kmoe_desc* d);
kmoe_status check_weight(const kmoe_weight* w, const char* name);
kmoe_status check_gather_scales(const kmoe_desc& d, kmoe_scale_kind kind, const char* name);
kmoe_status check_packed_arg(const kmoe_desc& d, const kmoe_packed_experts* packed);
kmoe_status check_stage_weights(const kmoe_desc& d, const kmoe_packed_experts* packed, int stages,
                                const kmoe_weight* gate, const kmoe_weight* up, const kmoe_weight* down);
kmoe_status check_norm_args(const void* scale, kmoe_dtype scale_dtype, float epsilon);

// The complete argument check of each entry point, in the order the entry point
// runs it, before its device check (no HIP call). *w receives the layout.
kmoe_status validate_forward(const kmoe_desc* desc, const void* x, const kmoe_weight* router,
                             const kmoe_weight* gate, const kmoe_weight* up, const kmoe_weight* down,
                             const kmoe_packed_experts* packed, const void* out, const void* workspace,
                             size_t workspace_bytes, Workspace* w);
kmoe_status validate_forward_noalloc(const kmoe_desc* desc, const void* x, const kmoe_weight* router,
                                     const kmoe_weight* gate, const kmoe_weight* up, const kmoe_weight* down,
                                     const kmoe_packed_experts* packed, const void* out, size_t scratch_bytes,
                                     Workspace* w);
kmoe_status validate_forward_block(const kmoe_desc* desc, const void* h, const void* norm_scale,
                                   kmoe_dtype norm_dtype, float epsilon, const kmoe_weight* router,
                                   const kmoe_weight* gate, const kmoe_weight* up, const kmoe_weight* down,
                                   const kmoe_packed_experts* packed, const void* out, const void* workspace,
                                   size_t workspace_bytes, Workspace* w);
kmoe_status validate_workspace_bytes(const kmoe_desc* desc, size_t* bytes);
kmoe_status validate_prepack_bytes(const kmoe_desc* desc, kmoe_packed_sizes* sizes);
kmoe_status validate_route(const kmoe_desc* desc, const void* x, const kmoe_weight* router, const void* scratch,
                           size_t scratch_bytes, const int32_t* topk_idx, const float* topk_w,
                           const int32_t* block_hist);
kmoe_status validate_route_scratch_bytes(const kmoe_desc* desc, size_t* bytes);
kmoe_status validate_dispatch(const kmoe_desc* desc, const int32_t* topk_idx, const int32_t* block_hist,
                              const int32_t* group_sizes, const int32_t* offsets, const int32_t* active,
                              const int32_t* sorted_token, const int32_t* sorted_expert, const int32_t* inv);
// stages: kStageGateUp and/or kStageDown; src is x (gate/up) or h_sorted (down alone)
kmoe_status validate_expert(const kmoe_desc* desc, int stages, const void* src, const int32_t* offsets,
                            const int32_t* active, const int32_t* sorted_token, const int32_t* sorted_expert,
                            const kmoe_weight* gate, const kmoe_weight* up, const kmoe_weight* down,
                            const kmoe_packed_experts* packed, const void* h_sorted, const void* y_sorted);
kmoe_status validate_combine(const kmoe_desc* desc, const void* y_sorted, const int32_t* inv, const float* topk_w,
                             const void* out);
kmoe_status validate_rms_norm(const kmoe_desc* desc, const void* x, const void* scale, kmoe_dtype scale_dtype,
                              float epsilon, const void* out);
kmoe_status validate_prepack(const kmoe_desc* desc, const kmoe_weight* gate, const kmoe_weight* up,
                             const kmoe_weight* down, const kmoe_packed_experts* packed);
kmoe_status validate_to_compute_dtype(const kmoe_weight* w, int64_t outer, int64_t channels,
                                      int64_t rows_per_scale_block, kmoe_dtype out_dtype, const void* out);
kmoe_status validate_quantize(int64_t experts, int64_t rows, int64_t channels, const void* w, kmoe_dtype w_dtype,
                              const int8_t* q, const float* s);

}  // namespace kmoe_host
