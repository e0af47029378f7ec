// The host-only layer of the C ABI (kappa_amd/csrc/host.cpp: argument
// validation, workspace layout, program choice) driven on the CPU. The pytest
// tests/test_host_sanitized.py builds this file with host.cpp under
// -fsanitize=address,undefined (no recovery) and runs it: every case of
// tests/test_abi.py's validation tests, the documented no-allocation limits,
// overflow edges of the size checks, and the layout invariants over a sweep of
// shapes. Prints "host checks: ok" and exits 0 when every check holds.
#include <math.h>
#include <stdio.h>
#include <string.h>

#include "host.h"

using namespace kmoe_host;

static int g_fail = 0;
static int g_checks = 0;

#define CHECK(cond)                                                        \
  do {                                                                     \
    ++g_checks;                                                            \
    if (!(cond)) {                                                         \
      ++g_fail;                                                            \
      fprintf(stderr, "%s:%d: check failed: %s\n", __FILE__, __LINE__, #cond); \
    }                                                                      \
  } while (0)

// status and a fragment of the message
static void expect(kmoe_status got, kmoe_status want, const char* frag, int line) {
  ++g_checks;
  if (got != want || (frag && !strstr(last_error(), frag))) {
    ++g_fail;
    fprintf(stderr, "line %d: status %d (want %d), message \"%s\" (want \"%s\")\n", line, (int)got, (int)want,
            last_error(), frag ? frag : "");
  }
}
#define EXPECT(call, want, frag) expect((call), (want), (frag), __LINE__)

static const void* const P = reinterpret_cast<const void*>(0x1000);  // placeholder device pointer

static kmoe_desc desc(int64_t T = 4, int64_t D = 128, int64_t E = 8, int64_t K = 2, int64_t I = 64,
                      kmoe_dtype act = KMOE_DTYPE_BF16, int64_t thr = 0, int64_t cap = 0,
                      kmoe_impl impl = KMOE_IMPL_RAGGED, kmoe_kernels kernels = KMOE_KERNELS_AUTO) {
  kmoe_desc d;
  d.tokens = T;
  d.hidden = D;
  d.num_experts = E;
  d.top_k = K;
  d.intermediate = I;
  d.act_dtype = act;
  d.impl = impl;
  d.decode_token_threshold = thr;
  d.expert_capacity = cap;
  d.kernels = kernels;
  return d;
}

static kmoe_weight weight(const void* values = P, kmoe_dtype dt = KMOE_DTYPE_I8, const void* scale = P,
                          kmoe_dtype sdt = KMOE_DTYPE_F32, kmoe_scale_kind kind = KMOE_SCALE_CHANNEL) {
  kmoe_weight w;
  w.values = values;
  w.dtype = dt;
  w.scale = scale;
  w.scale_dtype = sdt;
  w.scale_kind = kind;
  return w;
}

static kmoe_packed_experts packed(int64_t E = 8, int64_t D = 128, int64_t I = 64,
                                  kmoe_scale_kind kind = KMOE_SCALE_CHANNEL, void* s2 = (void*)P) {
  kmoe_packed_experts p;
  p.w13 = p.s13 = p.w2 = (void*)P;
  p.s2 = s2;
  p.num_experts = E;
  p.hidden = D;
  p.intermediate = I;
  p.source_scale_kind = kind;
  return p;
}

static const kmoe_weight F = weight(P, KMOE_DTYPE_BF16, nullptr, KMOE_DTYPE_F32, KMOE_SCALE_NONE);
static const kmoe_weight W = weight();

static kmoe_status fwd(const kmoe_desc& d, const void* x, const kmoe_weight& router, const kmoe_weight& g,
                       const kmoe_packed_experts* p, const void* ws, size_t ws_bytes) {
  Workspace w;
  return validate_forward(&d, x, &router, &g, &g, &g, p, P, ws, ws_bytes, &w);
}

static void desc_cases() {
  size_t n = 0;
  struct {
    kmoe_desc d;
    const char* frag;
  } bad[] = {
      {desc(-1), "tokens"},
      {desc(4, 0), "hidden"},
      {desc(4, 128, 8, 0), "top_k"},
      {desc(4, 128, 8, 9), "top_k"},
      {desc(4, 128, 8, 2, 64, KMOE_DTYPE_I8), "act_dtype"},
      {desc(4, 128, 8, 2, 64, KMOE_DTYPE_BF16, 0, -1), "expert_capacity"},
      {desc(4, 128, 8, 2, 64, KMOE_DTYPE_BF16, 0, 0, (kmoe_impl)7), "unknown impl"},
      {desc(4, 128, 8, 2, 64, KMOE_DTYPE_BF16, 0, 0, KMOE_IMPL_FIXED_CAPACITY), "expert_capacity >= 1"},
      {desc(4, 128, 8, 2, 64, KMOE_DTYPE_BF16, 0, 4, KMOE_IMPL_GATHER_EINSUM), "unless impl is fixed_capacity"},
      {desc(4, 128, 8, 2, 64, KMOE_DTYPE_BF16, 0, 0, KMOE_IMPL_RAGGED, (kmoe_kernels)5), "unknown kernels"},
  };
  for (auto& c : bad) EXPECT(validate_workspace_bytes(&c.d, &n), KMOE_ERR_INVALID_ARG, c.frag);
  EXPECT(validate_workspace_bytes(nullptr, &n), KMOE_ERR_INVALID_ARG, "desc is NULL");
  kmoe_desc ok = desc();
  EXPECT(validate_workspace_bytes(&ok, nullptr), KMOE_ERR_INVALID_ARG, "bytes is NULL");
  kmoe_desc e2048 = desc(4, 128, 2048, 2);
  EXPECT(validate_workspace_bytes(&e2048, &n), KMOE_ERR_UNSUPPORTED, nullptr);
  kmoe_desc d8192 = desc(4, 8192);
  EXPECT(validate_workspace_bytes(&d8192, &n), KMOE_ERR_UNSUPPORTED, nullptr);
  kmoe_desc k65 = desc(4, 128, 128, 65);
  EXPECT(validate_workspace_bytes(&k65, &n), KMOE_ERR_UNSUPPORTED, "top_k");
  kmoe_packed_sizes sz;
  kmoe_desc d96 = desc(4, 96);
  EXPECT(validate_prepack_bytes(&d96, &sz), KMOE_ERR_UNSUPPORTED, nullptr);
  kmoe_desc dec129 = desc(129, 128, 8, 2, 64, KMOE_DTYPE_BF16, 0, 0, KMOE_IMPL_RAGGED, KMOE_KERNELS_DECODE);
  EXPECT(validate_workspace_bytes(&dec129, &n), KMOE_ERR_UNSUPPORTED, "at most 128 tokens");
  // sizes whose products would overflow 64-bit arithmetic are refused, not wrapped
  const int64_t huge[] = {INT64_MAX, INT64_MAX / 2, (int64_t)1 << 40, (int64_t)1 << 32, (int64_t)1 << 31};
  for (int64_t T : huge) {
    kmoe_desc d = desc(T, 4096, 1024, 64, 1 << 20);
    EXPECT(validate_workspace_bytes(&d, &n), KMOE_ERR_UNSUPPORTED, "too large");
  }
  kmoe_desc bigI = desc(4, 128, 8, 2, INT64_MAX);
  EXPECT(validate_workspace_bytes(&bigI, &n), KMOE_ERR_UNSUPPORTED, "intermediate");
  kmoe_desc bigD = desc(4, INT64_MAX);
  EXPECT(validate_workspace_bytes(&bigD, &n), KMOE_ERR_UNSUPPORTED, "hidden");
  kmoe_desc bigE = desc(4, 128, INT64_MAX, 2);
  EXPECT(validate_workspace_bytes(&bigE, &n), KMOE_ERR_UNSUPPORTED, "num_experts");
  // the 30B-A3B and 235B-A22B shapes
  kmoe_desc l30 = desc(4096, 2048, 128, 8, 768);
  EXPECT(validate_workspace_bytes(&l30, &n), KMOE_OK, nullptr);
  const size_t M = 4096 * 8;
  CHECK(n >= 2 * M * (2 * 768 + 2048) + 4 * 3 * M);
  EXPECT(validate_prepack_bytes(&l30, &sz), KMOE_OK, nullptr);
  CHECK(sz.w13_bytes == (size_t)2 * 128 * 2048 * 768 && sz.w2_bytes == (size_t)128 * 2048 * 768);
  CHECK(sz.s13_bytes == (size_t)4 * 2 * 128 * 768 && sz.s2_bytes == (size_t)4 * 128 * 2048);
}

static void forward_cases() {
  const kmoe_desc d = desc();
  EXPECT(fwd(d, P, weight(nullptr), W, nullptr, P, (size_t)1 << 40), KMOE_ERR_INVALID_ARG, "router values");
  EXPECT(fwd(d, P, weight(P, KMOE_DTYPE_I8, P, KMOE_DTYPE_F32, KMOE_SCALE_NONE), W, nullptr, P, (size_t)1 << 40),
         KMOE_ERR_INVALID_ARG, "TENSOR or CHANNEL");
  EXPECT(fwd(d, P, weight(P, KMOE_DTYPE_I8, nullptr), W, nullptr, P, (size_t)1 << 40), KMOE_ERR_INVALID_ARG,
         "scale pointer");
  EXPECT(fwd(d, P, weight(P, KMOE_DTYPE_BF16), W, nullptr, P, (size_t)1 << 40), KMOE_ERR_INVALID_ARG,
         "takes no scale");
  EXPECT(fwd(d, P, weight(P, KMOE_DTYPE_I8, P, KMOE_DTYPE_I8), W, nullptr, P, (size_t)1 << 40), KMOE_ERR_INVALID_ARG,
         "scale dtype");
  EXPECT(fwd(d, nullptr, F, W, nullptr, P, (size_t)1 << 40), KMOE_ERR_INVALID_ARG, "x and out");
  EXPECT(fwd(d, P, F, W, nullptr, nullptr, (size_t)1 << 40), KMOE_ERR_WORKSPACE_TOO_SMALL, "workspace");
  EXPECT(fwd(d, P, F, W, nullptr, P, 16), KMOE_ERR_WORKSPACE_TOO_SMALL, "workspace");
  EXPECT(fwd(d, P, F, W, nullptr, P, (size_t)1 << 40), KMOE_OK, nullptr);
  // zero tokens validate without buffers
  EXPECT(fwd(desc(0, 128, 8, 2, 64, KMOE_DTYPE_BF16, -1), nullptr, F, W, nullptr, nullptr, 0), KMOE_OK, nullptr);

  // the gather program takes one scale per tensor (kappa/qwen3/quant.py:71-74)
  const kmoe_weight ch = weight(), pt = weight(P, KMOE_DTYPE_I8, P, KMOE_DTYPE_F32, KMOE_SCALE_TENSOR);
  const kmoe_desc gather = desc(4, 128, 8, 2, 64, KMOE_DTYPE_BF16, 0, 0, KMOE_IMPL_GATHER_EINSUM);
  EXPECT(fwd(gather, P, F, ch, nullptr, P, (size_t)1 << 40), KMOE_ERR_INVALID_ARG, "one scale per tensor");
  EXPECT(fwd(desc(4, 128, 8, 2, 64, KMOE_DTYPE_BF16, 64), P, F, ch, nullptr, P, (size_t)1 << 40),
         KMOE_ERR_INVALID_ARG, "one scale per tensor");
  EXPECT(fwd(desc(4, 128, 1, 1, 64, KMOE_DTYPE_BF16, 0, 0, KMOE_IMPL_GATHER_EINSUM), P, F, ch, nullptr, P,
             (size_t)1 << 40),
         KMOE_OK, nullptr);
  EXPECT(fwd(gather, P, F, pt, nullptr, P, (size_t)1 << 40), KMOE_OK, nullptr);
  EXPECT(fwd(desc(4, 128, 8, 2, 64, KMOE_DTYPE_BF16, 0, 3, KMOE_IMPL_FIXED_CAPACITY), P, F, ch, nullptr, P,
             (size_t)1 << 40),
         KMOE_OK, nullptr);
  EXPECT(fwd(d, P, F, ch, nullptr, P, (size_t)1 << 40), KMOE_OK, nullptr);
  kmoe_packed_experts pc = packed(), ptk = packed(8, 128, 64, KMOE_SCALE_TENSOR);
  EXPECT(fwd(gather, P, F, ch, &pc, P, (size_t)1 << 40), KMOE_ERR_INVALID_ARG, "one scale per tensor");
  EXPECT(fwd(gather, P, F, ch, &ptk, P, (size_t)1 << 40), KMOE_OK, nullptr);

  // packed-argument rules
  kmoe_packed_experts nos2 = packed(8, 128, 64, KMOE_SCALE_CHANNEL, nullptr);
  EXPECT(fwd(d, P, F, W, &nos2, P, (size_t)1 << 40), KMOE_ERR_INVALID_ARG, "non-NULL");
  EXPECT(fwd(desc(4, 128, 8, 2, 64, KMOE_DTYPE_F32), P, F, W, &pc, P, (size_t)1 << 40), KMOE_ERR_UNSUPPORTED,
         "bf16 activations");
  kmoe_packed_experts p96 = packed(8, 96);
  EXPECT(fwd(desc(4, 96), P, F, W, &p96, P, (size_t)1 << 40), KMOE_ERR_UNSUPPORTED, "divisible by 64");
  kmoe_packed_experts mism[] = {packed(16), packed(8, 256), packed(8, 128, 128)};
  for (auto& p : mism) EXPECT(fwd(d, P, F, W, &p, P, (size_t)1 << 40), KMOE_ERR_INVALID_ARG, "packed experts hold");
  kmoe_packed_experts pnone = packed(8, 128, 64, KMOE_SCALE_NONE);
  EXPECT(fwd(d, P, F, W, &pnone, P, (size_t)1 << 40), KMOE_ERR_INVALID_ARG, "source_scale_kind");
}

static void stage_cases() {
  const kmoe_desc d = desc();
  EXPECT(validate_route(&d, P, &F, nullptr, 0, nullptr, nullptr, nullptr), KMOE_ERR_INVALID_ARG, "kmoe_route");
  const int32_t* I = reinterpret_cast<const int32_t*>(P);
  const float* Fp = reinterpret_cast<const float*>(P);
  EXPECT(validate_route(&d, P, &F, nullptr, 0, I, Fp, I), KMOE_OK, nullptr);
  size_t rs = 0;
  EXPECT(validate_route_scratch_bytes(&d, &rs), KMOE_OK, nullptr);
  CHECK(rs >= (size_t)2 * 8 * 128 + 4 * 8);  // the bf16 transposed router and the norm partials
  EXPECT(validate_route(&d, P, &F, P, rs - 1, I, Fp, I), KMOE_ERR_WORKSPACE_TOO_SMALL, "scratch");
  EXPECT(validate_route(&d, P, &F, P, rs, I, Fp, I), KMOE_OK, nullptr);
  // the two-phase form's shapes: bf16 activations and router, 512 <= D <= 4096, D % 64, E % 16
  const kmoe_weight RB = weight(P, KMOE_DTYPE_BF16, nullptr, KMOE_DTYPE_F32, KMOE_SCALE_NONE);
  const kmoe_desc l30 = desc(4096, 2048, 128, 8, 768);
  CHECK(route_mfma_fits(l30, RB) && !route_mfma_fits(l30, W) && !route_mfma_fits(desc(4096, 256, 128, 8), RB));
  CHECK(!route_mfma_fits(desc(4096, 2048, 120, 8), RB) && !route_mfma_fits(desc(4096, 2048, 128, 8, 768, KMOE_DTYPE_F32), RB));
  CHECK(route_mfma_preferred(l30, RB) && !route_mfma_preferred(desc(1024, 2048, 128, 8), RB));
  CHECK(route_mfma_preferred(desc(2048, 4096, 128, 8, 1536), RB) && route_mfma_preferred(desc(4096, 4096, 128, 8, 1536), RB));
  CHECK(!route_mfma_preferred(desc(2047, 4096, 128, 8, 1536), RB) && !route_mfma_preferred(desc(4096, 4096, 128, 8, 1536, KMOE_DTYPE_F32), RB));
  // the int8-plane down product: the ragged program on bf16 activations from 96 rows per expert
  CHECK(down_planes_fits(desc(1536, 2048, 128, 8, 768)) && !down_planes_fits(desc(1535, 2048, 128, 8, 768)));
  CHECK(!down_planes_fits(desc(4096, 2048, 128, 8, 768, KMOE_DTYPE_F32)) &&
        !down_planes_fits(desc(4096, 2048, 128, 8, 768, KMOE_DTYPE_BF16, 0, 0, KMOE_IMPL_GATHER_EINSUM)));
  CHECK(!down_planes_fits(desc(4096, 2048, 128, 8, 768, KMOE_DTYPE_BF16, 4096)) &&  // threshold: gather program
        !down_planes_fits(desc(4096, 2048, 128, 8, 4096)) && down_planes_fits(desc(2048, 4096, 128, 8, 1536)));
  {
    const Workspace wp = layout(desc(2048, 2048, 128, 8, 768), false), wn = layout(desc(1024, 2048, 128, 8, 768), false);
    CHECK(wp.normed - wp.h_scale == (size_t)4 * 2048 * 8 && wn.normed == wn.h_scale);
  }
  EXPECT(validate_dispatch(&d, I, I, I, I, I, I, I, nullptr), KMOE_ERR_INVALID_ARG, "kmoe_dispatch");
  EXPECT(validate_dispatch(&d, I, I, I, I, I, I, I, I), KMOE_OK, nullptr);
  EXPECT(validate_combine(&d, P, nullptr, Fp, P), KMOE_ERR_INVALID_ARG, "kmoe_combine");
  EXPECT(validate_combine(&d, P, I, Fp, P), KMOE_OK, nullptr);
  const int both = kStageGateUp | kStageDown;
  EXPECT(validate_expert(&d, both, P, I, I, I, I, nullptr, nullptr, nullptr, nullptr, P, P), KMOE_ERR_INVALID_ARG,
         "gate weight is NULL");
  EXPECT(validate_expert(&d, both, P, I, I, nullptr, I, &W, &W, &W, nullptr, P, P), KMOE_ERR_INVALID_ARG,
         "kmoe_expert_ffn: NULL buffer");
  EXPECT(validate_expert(&d, both, P, I, I, I, I, &W, &W, &W, nullptr, P, P), KMOE_OK, nullptr);
  EXPECT(validate_expert(&d, kStageGateUp, P, I, I, I, I, &W, &W, nullptr, nullptr, P, nullptr), KMOE_OK, nullptr);
  EXPECT(validate_expert(&d, kStageDown, P, I, I, nullptr, I, nullptr, nullptr, &W, nullptr, P, nullptr),
         KMOE_ERR_INVALID_ARG, "kmoe_expert_down: NULL buffer");
  EXPECT(validate_expert(&d, kStageDown, P, I, I, nullptr, I, nullptr, nullptr, &W, nullptr, P, P), KMOE_OK,
         nullptr);
  // packed experts stand in for the layout-native weights
  kmoe_packed_experts pc = packed();
  EXPECT(validate_expert(&d, both, P, I, I, I, I, nullptr, nullptr, nullptr, &pc, P, P), KMOE_OK, nullptr);

  // prepack: int8 only, shapes, and the recorded kind of the source scales
  const kmoe_weight pt = weight(P, KMOE_DTYPE_I8, P, KMOE_DTYPE_F32, KMOE_SCALE_TENSOR);
  kmoe_packed_experts p4 = packed(4), ptk = packed(8, 128, 64, KMOE_SCALE_TENSOR);
  EXPECT(validate_prepack(&d, &F, &W, &W, &pc), KMOE_ERR_UNSUPPORTED, "int8");
  EXPECT(validate_prepack(&d, &W, &W, &W, &p4), KMOE_ERR_INVALID_ARG, "packed shapes");
  EXPECT(validate_prepack(&d, &W, &W, &W, nullptr), KMOE_ERR_INVALID_ARG, "non-NULL");
  EXPECT(validate_prepack(&d, &W, &W, &W, &ptk), KMOE_ERR_INVALID_ARG, "must be CHANNEL");
  EXPECT(validate_prepack(&d, &pt, &pt, &W, &ptk), KMOE_ERR_INVALID_ARG, "must be CHANNEL");
  EXPECT(validate_prepack(&d, &pt, &pt, &pt, &pc), KMOE_ERR_INVALID_ARG, "must be TENSOR");
  EXPECT(validate_prepack(&d, &pt, &pt, &pt, &ptk), KMOE_OK, nullptr);
  EXPECT(validate_prepack(&d, &W, &pt, &W, &pc), KMOE_OK, nullptr);

  EXPECT(validate_to_compute_dtype(&W, 4, 0, 1, KMOE_DTYPE_BF16, P), KMOE_ERR_INVALID_ARG, "bad shape");
  EXPECT(validate_to_compute_dtype(&W, INT64_MAX, 4, 1, KMOE_DTYPE_BF16, P), KMOE_ERR_UNSUPPORTED, "too large");
  EXPECT(validate_to_compute_dtype(&W, 4, 4, 1, KMOE_DTYPE_I8, P), KMOE_ERR_INVALID_ARG, "out_dtype");
  EXPECT(validate_to_compute_dtype(&W, 4, 4, 1, KMOE_DTYPE_BF16, nullptr), KMOE_ERR_INVALID_ARG, "out is NULL");
  EXPECT(validate_to_compute_dtype(&W, 4, 4, 1, KMOE_DTYPE_BF16, P), KMOE_OK, nullptr);
  const int8_t* q = reinterpret_cast<const int8_t*>(P);
  EXPECT(validate_quantize(1, 4, 4, P, KMOE_DTYPE_I8, q, Fp), KMOE_ERR_INVALID_ARG, "w_dtype");
  EXPECT(validate_quantize(0, 4, 4, P, KMOE_DTYPE_F32, q, Fp), KMOE_ERR_INVALID_ARG, "bad shape");
  EXPECT(validate_quantize(1, 4, 4, nullptr, KMOE_DTYPE_F32, q, Fp), KMOE_ERR_INVALID_ARG, "NULL buffer");
  EXPECT(validate_quantize(70000, 4, 4, P, KMOE_DTYPE_F32, q, Fp), KMOE_ERR_UNSUPPORTED, "too many experts");
  EXPECT(validate_quantize(128, INT64_MAX, 4096, P, KMOE_DTYPE_F32, q, Fp), KMOE_ERR_UNSUPPORTED, "too large");
  EXPECT(validate_quantize(128, 2048, 768, P, KMOE_DTYPE_F32, q, Fp), KMOE_OK, nullptr);
}

static void block_cases() {
  const kmoe_desc d = desc();
  Workspace w;
  struct {
    const void* h;
    const void* scale;
    kmoe_dtype sdt;
    float eps;
    const kmoe_weight* router;
    const void* out;
    const void* ws;
    kmoe_status want;
    const char* frag;
  } cases[] = {
      {P, nullptr, KMOE_DTYPE_BF16, 1e-6f, &F, (const void*)0x2000, P, KMOE_ERR_INVALID_ARG, "norm scale pointer"},
      {P, P, KMOE_DTYPE_I8, 1e-6f, &F, (const void*)0x2000, P, KMOE_ERR_INVALID_ARG, "norm scale dtype"},
      {P, P, KMOE_DTYPE_BF16, -1.0f, &F, (const void*)0x2000, P, KMOE_ERR_INVALID_ARG, "epsilon"},
      {P, P, KMOE_DTYPE_BF16, NAN, &F, (const void*)0x2000, P, KMOE_ERR_INVALID_ARG, "epsilon"},
      {nullptr, P, KMOE_DTYPE_BF16, 1e-6f, &F, (const void*)0x2000, P, KMOE_ERR_INVALID_ARG, "h and out"},
      {P, P, KMOE_DTYPE_BF16, 1e-6f, &F, P, P, KMOE_ERR_INVALID_ARG, "alias"},
      {P, P, KMOE_DTYPE_BF16, 1e-6f, &F, (const void*)0x2000, nullptr, KMOE_ERR_WORKSPACE_TOO_SMALL, "workspace"},
      {P, P, KMOE_DTYPE_BF16, 1e-6f, &W, (const void*)0x2000, P, KMOE_OK, nullptr},
  };
  const kmoe_weight badr = weight(nullptr);
  for (auto& c : cases)
    EXPECT(validate_forward_block(&d, c.h, c.scale, c.sdt, c.eps, c.router, &W, &W, &W, nullptr, c.out, c.ws,
                                  (size_t)1 << 40, &w),
           c.want, c.frag);
  EXPECT(validate_forward_block(&d, P, P, KMOE_DTYPE_BF16, 1e-6f, &badr, &W, &W, &W, nullptr, (const void*)0x2000, P,
                                (size_t)1 << 40, &w),
         KMOE_ERR_INVALID_ARG, "router values");
  EXPECT(validate_rms_norm(&d, P, nullptr, KMOE_DTYPE_BF16, 1e-6f, P), KMOE_ERR_INVALID_ARG, nullptr);
  EXPECT(validate_rms_norm(&d, P, P, KMOE_DTYPE_I8, 1e-6f, P), KMOE_ERR_INVALID_ARG, nullptr);
  EXPECT(validate_rms_norm(&d, nullptr, P, KMOE_DTYPE_BF16, 1e-6f, P), KMOE_ERR_INVALID_ARG, nullptr);
  EXPECT(validate_rms_norm(&d, P, P, KMOE_DTYPE_BF16, 1e-6f, P), KMOE_OK, nullptr);
}

// The no-allocation entry point: the documented token limits of its 16 MiB
// scratch with bf16 activations on the ragged program (include/kmoe.h).
static void noalloc_cases() {
  Workspace w;
  const size_t scratch = KMOE_NOALLOC_SCRATCH_BYTES;
  struct {
    int64_t D, I, limit;
  } shapes[] = {{2048, 768, 291}, {4096, 1536, 136}};
  for (auto& s : shapes) {
    kmoe_desc at = desc(s.limit, s.D, 128, 8, s.I), over = desc(s.limit + 1, s.D, 128, 8, s.I);
    EXPECT(validate_forward_noalloc(&at, P, &F, &W, &W, &W, nullptr, P, scratch, &w), KMOE_OK, nullptr);
    CHECK(w.total <= scratch);
    EXPECT(validate_forward_noalloc(&over, P, &F, &W, &W, &W, nullptr, P, scratch, &w), KMOE_ERR_WORKSPACE_TOO_SMALL,
           "scratch");
    EXPECT(validate_forward_noalloc(&at, nullptr, &F, &W, &W, &W, nullptr, P, scratch, &w), KMOE_ERR_INVALID_ARG,
           "x and out");
  }
  kmoe_desc big = desc(4096, 2048, 128, 8, 768);
  EXPECT(validate_forward_noalloc(&big, P, &F, &W, &W, &W, nullptr, P, scratch, &w), KMOE_ERR_WORKSPACE_TOO_SMALL,
         "scratch");
}

// Layout invariants over a sweep of shapes and programs: buffers in order,
// 256-byte aligned, each at least its size apart, the block layout the forward
// layout plus the normalised rows; the program and family choices consistent.
static void layout_sweep() {
  const int64_t Ts[] = {0, 1, 2, 4, 8, 15, 16, 17, 63, 64, 65, 127, 128, 129, 240, 241, 291, 1000, 4096, 65537};
  const int64_t Ds[] = {64, 100, 256, 2048, 4096};
  const int64_t Es[] = {1, 8, 128, 1024};
  const int64_t Is[] = {64, 96, 768, 1536};
  const kmoe_impl impls[] = {KMOE_IMPL_GATHER_EINSUM, KMOE_IMPL_RAGGED, KMOE_IMPL_FIXED_CAPACITY};
  const kmoe_dtype acts[] = {KMOE_DTYPE_BF16, KMOE_DTYPE_F32};
  for (int64_t T : Ts)
    for (int64_t D : Ds)
      for (int64_t E : Es)
        for (int64_t I : Is)
          for (kmoe_impl impl : impls)
            for (kmoe_dtype act : acts) {
              const int64_t K = E < 8 ? E : 8;
              const kmoe_desc d = desc(T, D, E, K, I, act, 64, impl == KMOE_IMPL_FIXED_CAPACITY ? 5 : 0, impl);
              size_t n = 0;
              if (validate_workspace_bytes(&d, &n) != KMOE_OK) {
                ++g_fail;
                fprintf(stderr, "desc T=%lld D=%lld E=%lld I=%lld refused: %s\n", (long long)T, (long long)D,
                        (long long)E, (long long)I, last_error());
                continue;
              }
              const Workspace f = layout(d, false), b = layout(d, true);
              CHECK(n == b.total);
              const size_t M = (size_t)T * K, a = act == KMOE_DTYPE_BF16 ? 2 : 4;
              const size_t hb = chain_of(d) == kmoe::kChainF32 && act == KMOE_DTYPE_BF16 ? 4 : a;
              const size_t nblk = ((size_t)T + 63) / 64;
              const size_t off[] = {f.topk_idx, f.topk_w,  f.hist,     f.group_sizes, f.offsets, f.active, f.sorted_token,
                                    f.sorted_expert, f.inv, f.h_sorted, f.y_sorted,   f.route_part, f.normed, f.total};
              const size_t need[] = {4 * M, 4 * M, 4 * nblk * E, 4 * (size_t)E, 4 * (size_t)(E + 1),
                                     4 * (size_t)(E + 1), 4 * M, 4 * M, 4 * M, hb * M * I, a * M * D,
                                     T <= kSplitRouterMaxTokens ? 4 * route_split_part_floats(d)
                                                                : (T >= 2048 ? route_mfma_scratch_bytes(d) : 0),
                                     0};
              bool ok = f.topk_idx == 0;
              for (int i = 0; i < 13; ++i) ok = ok && off[i] % 256 == 0 && off[i + 1] >= off[i] + need[i];
              CHECK(ok);
              CHECK(b.normed == f.normed && b.total >= f.total + a * (size_t)T * D);
              CHECK((effective_impl(d) == KMOE_IMPL_GATHER_EINSUM) ==
                    (impl == KMOE_IMPL_GATHER_EINSUM || (impl == KMOE_IMPL_RAGGED && T <= 64)));
              CHECK(scatter_of(d) == (effective_impl(d) != KMOE_IMPL_GATHER_EINSUM));
              CHECK(family_of(d) == (T <= 64 ? kFamilyDecode : kFamilyGemm));
            }
}

int main() {
  desc_cases();
  forward_cases();
  stage_cases();
  block_cases();
  noalloc_cases();
  layout_sweep();
  CHECK(strcmp(status_string((kmoe_status)99), "unknown status") == 0);
  for (int s = 0; s < 6; ++s) CHECK(status_string((kmoe_status)s)[0] != '\0');
  if (g_fail) {
    fprintf(stderr, "host checks: %d of %d failed\n", g_fail, g_checks);
    return 1;
  }
  printf("host checks: ok (%d checks)\n", g_checks);
  return 0;
}
