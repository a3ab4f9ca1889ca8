// capi.hip -- error reporting and the composed MoE-HLM layer entry point.
//
// ygg_moe_forward replaces HLMBlock._moe_forward (holograph/models/hlm_block.py:
// 154-183) end to end: router logits (or given logits), softmax / top-k /
// counting sort, dispatch, the two grouped CliffordLinear products with the
// grade-wise activation fused, and the weighted combine -- all enqueued on
// the caller's stream, all buffers caller-owned (one workspace, sized by
// ygg_moe_workspace_bytes), no host synchronisation.

#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "ygg_common.h"
#include "route_select.h"

namespace ygg {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return -1;
  }
  return 0;
}

static size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

}  // namespace ygg

using namespace ygg;

YGG_API const char* ygg_last_error(void) { return g_err; }

YGG_API int ygg_version(void) { return 1; }

// declared in the other translation units
extern "C" size_t ygg_route_workspace_bytes(int N, int E, int k);
extern "C" int ygg_route(const float*, int, int, int, int32_t*, float*, int32_t*, int32_t*, int32_t*, int32_t*, void*,
                         size_t, hipStream_t);
extern "C" int ygg_router_energy_logits(const void*, int, int, int, const float*, const float*, int, float*, float*,
                                        hipStream_t);
extern "C" int ygg_route_energy(const void*, int, int, int, const float*, const float*, int, int, int32_t*, float*,
                                int32_t*, int32_t*, int32_t*, int32_t*, float*, void*, size_t, hipStream_t);
extern "C" int ygg_dispatch(const void*, int, int, int, int, const int32_t*, void*, int, hipStream_t);
extern "C" int ygg_clifford_layer_norm(const void*, int, int, int, const float*, const float*, double, void*, int,
                                       hipStream_t);
extern "C" int ygg_combine(const void*, int, int, int, int, int, const int32_t*, const float*, const int32_t*,
                           const void*, void*, int, hipStream_t);
extern "C" int ygg_grouped_clifford_linear(const void*, int, const void*, int, const float*, const float*,
                                           const int32_t*, int, int, int, int, void*, int, int, hipStream_t);
extern "C" int ygg_pauli_grouped_linear(const void*, int, int, const int32_t*, int, const void*, const float*,
                                        const int32_t*, int, int, int, int, void*, int, int, hipStream_t);
extern "C" int ygg_pauli_rows_from_blade(const void*, int, int, void*, hipStream_t);
extern "C" int ygg_pauli_rows_from_blade_f32(const float*, int, int, float*, hipStream_t);
extern "C" int ygg_pauli_grouped_linear_f32(const float*, const int32_t*, int, const float*, const float*,
                                            const int32_t*, int, int, int, int, float*, int, hipStream_t);

// y_sorted region: bf16/fp32 rows, or for the decode-shape int8 path the fp32
// partial planes of the K-split down product
static size_t ys_bytes(size_t P, int E, int d, int F, int dtype, int w_format) {
  const size_t es = (dtype == kF32) ? 4 : 2;
  if (w_format == kWPauliI8) return (size_t)decode_pauli_planes(F) * P * d * 8 * 4;
  if (decode_shape((int)P, E, w_format)) {
    const int planes = decode_splits(F) > decode_layer_planes(F) ? decode_splits(F) : decode_layer_planes(F);
    return (size_t)planes * P * d * 8 * 4;
  }
  if (w_format == kWPauliF32) return (size_t)pauli_f32_splits((int)P, E, F, d) * P * d * 8 * 4;
  return P * d * 8 * es;
}

YGG_API size_t ygg_moe_workspace_bytes(int N, int d, int F, int E, int k, int dtype, int w_format) {
  const size_t P = (size_t)N * k;
  const size_t es = (dtype == kF32) ? 4 : 2;
  size_t b = 0;
  b += align256((size_t)N * E * 4);       // logits
  b += align256(P * 4) * 2;               // perm, slot_pos
  b += align256(ygg_route_workspace_bytes(N, E, k));
  b += align256(P * d * 8 * es);          // x_sorted (Pauli half-rows of x for format 3)
  b += align256(P * F * 8 * es);          // h
  b += align256(ys_bytes(P, E, d, F, dtype, w_format));  // y_sorted
  if (w_format == kWPauliF32) b += align256(P * 4);       // row_slot: each row's slot, for the partial planes
  return b;
}

// Sizes the layer's kernels cannot address, refused before the first launch: more
// than 2^31 - 1 token-expert rows, and the bf16 Pauli products' 32-bit limits (the
// up product gathers x's Pauli rows, N of them, into P rows of h; the down product
// reads h in place into P blade rows).
static int layer_size_check(const char* who, int N, int d, int F, int E, int k, int w_format) {
  YGG_CHECK_ARG((long long)N * k <= 0x7fffffffLL, "%s: N k = %lld token-expert rows exceed 2^31 - 1", who,
                (long long)N * k);
  if (w_format == kWPauli && N > 0) {
    const int P = N * k;
    const char* why = ygg::pauli_size_limit(/*Pauli rows*/ 1, N, /*gathered*/ true, P, E, d, F, /*Pauli rows*/ 0, kBF16);
    if (!why) why = ygg::pauli_size_limit(1, P, false, P, E, F, d, /*blade*/ 1, kBF16);
    if (why) {
      set_error("%s: %s (N=%d d=%d F=%d E=%d k=%d)", who, why, N, d, F, E, k);
      return -1;
    }
  }
  return 0;
}

static int moe_forward_impl(const void* x, int dtype, int N, int d, int F, int E, int k, int act,
                            const float* logits, const float* router_w, const float* router_b, const void* w_up,
                            const float* s_up, const float* b_up, const void* w_down, const float* s_down,
                            const float* b_down, int w_format, const void* residual, void* out, int32_t* topk_idx,
                            float* topk_w, int32_t* counts, int32_t* offsets, void* workspace,
                            size_t workspace_bytes, hipStream_t stream,
                            float* h_pre_out) {
  // every path checks the sizes here, also those that route inside a product
  YGG_CHECK_ARG(N >= 0 && d >= 1 && F >= 1, "ygg_moe_forward: bad sizes N=%d d=%d F=%d", N, d, F);
  YGG_CHECK_ARG(E >= 1 && E <= kMaxExperts, "ygg_moe_forward: E=%d out of range [1, %d]", E, kMaxExperts);
  YGG_CHECK_ARG(k >= 1 && k <= kMaxTopK && k <= E, "ygg_moe_forward: k=%d out of range [1, min(%d, E=%d)]", k,
                kMaxTopK, E);
  YGG_CHECK_ARG(act >= kActNone && act <= kActSigmoid, "ygg_moe_forward: activation %d", act);
  YGG_CHECK_ARG(N == 0 || (x && out && w_up && w_down && topk_idx && topk_w && counts && offsets && workspace),
                "ygg_moe_forward: null pointer");
  YGG_CHECK_ARG((w_format != kWI8 && w_format != kWPauliI8) || N == 0 || (s_up && s_down),
                "ygg_moe_forward: int8 weights need their scales");
  YGG_CHECK_ARG(dtype == kF32 || dtype == kBF16, "ygg_moe_forward: dtype %d unsupported", dtype);
  YGG_CHECK_ARG(dtype == kF32 ? (w_format == kWF32 || w_format == kWPauliF32)
                             : (w_format == kWBF16 || w_format == kWI8 || w_format == kWPauli ||
                                w_format == kWPauliI8),
                "ygg_moe_forward: weight format %d does not match dtype %d", w_format, dtype);
  YGG_CHECK_ARG(w_format != kWPauliI8 || N == 0 || decode_pauli_fusable(N, E, k, d, F),
                "ygg_moe_forward: int8 Pauli weights (format 5) serve decode batches of at most 128 tokens with "
                "d <= 128 (N=%d d=%d); use format 2 or 3 for larger calls",
                N, d);
  YGG_CHECK_ARG(w_format != kWPauli || (d % 2 == 0 && F % 2 == 0),
                "ygg_moe_forward: the Pauli weight format needs even d and F (d=%d F=%d)", d, F);
  if (layer_size_check("ygg_moe_forward", N, d, F, E, k, w_format)) return -1;
  YGG_CHECK_ARG(workspace_bytes >= ygg_moe_workspace_bytes(N, d, F, E, k, dtype, w_format),
                "ygg_moe_forward: workspace of %zu bytes, need %zu", workspace_bytes,
                ygg_moe_workspace_bytes(N, d, F, E, k, dtype, w_format));
  YGG_CHECK_ARG(N == 0 || logits || (router_w && router_b), "ygg_moe_forward: need logits or router parameters");
  if (N == 0)  // no tokens: every expert's count and offset is zero, as ygg_route writes them
    return (counts && offsets) ? ygg_route(nullptr, 0, E, k, nullptr, nullptr, counts, offsets, nullptr, nullptr,
                                           nullptr, 0, stream)
                               : 0;
  const size_t P = (size_t)N * k;
  const size_t es = (dtype == kF32) ? 4 : 2;
  char* p = static_cast<char*>(workspace);
  float* lg = reinterpret_cast<float*>(p);
  p += align256((size_t)N * E * 4);
  int32_t* perm = reinterpret_cast<int32_t*>(p);
  p += align256(P * 4);
  int32_t* slot_pos = reinterpret_cast<int32_t*>(p);
  p += align256(P * 4);
  void* rws = p;
  const size_t rws_bytes = align256(ygg_route_workspace_bytes(N, E, k));
  p += rws_bytes;
  void* xs = p;
  p += align256(P * d * 8 * es);
  void* h = p;
  p += align256(P * F * 8 * es);
  void* ys = p;

  if (w_format == kWPauliI8) {
    // int8 Pauli weights: routing, both products and the activation in one launch
    // (the grade-energy logits first when the caller gives none), then the combine
    // of its partial planes
    if (!logits) {
      if (ygg_router_energy_logits(x, dtype, N, d, router_w, router_b, E, lg, nullptr, stream)) return -1;
      logits = lg;
    }
    if (decode_pauli_layer(static_cast<const uint16_t*>(x), logits, N, E, k, d, F, act,
                           static_cast<const int8_t*>(w_up), s_up, b_up, static_cast<const int8_t*>(w_down), s_down,
                           b_down, topk_idx, topk_w, counts, offsets, perm, slot_pos, static_cast<float*>(ys),
                           stream))
      return -1;
    return combine_planes(static_cast<const float*>(ys), decode_pauli_planes(F), (int)P, N, k, d, topk_idx, topk_w,
                          slot_pos, residual, out, dtype, stream, /*slot rows*/ true);
  }
  // decode layers given logits route inside their up product (no routing launch)
  const bool decode = decode_shape((int)P, E, w_format);
  const bool fused_layer = decode && logits && dtype == kBF16 && decode_layer_fusable(N, E, k, d, F);
  const bool fused_route = decode && logits && !fused_layer && decode_route_fusable(N, E, k, d);
  if (fused_layer) {
    // decode layers given logits: routing, both products and the activation in one
    // launch, then the combine of its partial planes
    if (decode_layer(static_cast<const uint16_t*>(x), logits, N, E, k, d, F, act, static_cast<const int8_t*>(w_up),
                     s_up, b_up, static_cast<const int8_t*>(w_down), s_down, b_down, topk_idx, topk_w, counts,
                     offsets, perm, slot_pos, static_cast<float*>(ys), stream))
      return -1;
    return combine_planes(static_cast<const float*>(ys), decode_layer_planes(F), (int)P, N, k, d, topk_idx, topk_w,
                          slot_pos, residual, out, dtype, stream);
  }
  // fp32 Pauli weights, logits given, a batch of at most 256 tokens of at most 64
  // multivectors: the up product routes the batch itself and reads x's blade rows, so
  // no routing launch runs
  const bool f32_routed_up = w_format == kWPauliF32 && logits && pauli_f32_route_fusable(N, E, k, d);
  // the Pauli formats' conversion of x to Pauli rows (into the x_sorted region: N <= P
  // rows) runs as extra workgroups of the routing's first launch
  ygg::RowConvert cv;
  if ((w_format == kWPauli || w_format == kWPauliF32) && !f32_routed_up) {
    cv.x = x;
    cv.out = xs;
    cv.n = (long long)N * d;
    cv.d = d;
    cv.kind = w_format == kWPauli ? ygg::kConvBf16Pauli : ygg::kConvF32Pauli;
  }
  // fp32 Pauli: the routing also writes each row's slot, and the down product its
  // partial planes at slot rows t k + s (the combine's plane loads then need no
  // routing array)
  int32_t* row_slot = nullptr;
  if (w_format == kWPauliF32) {
    row_slot = reinterpret_cast<int32_t*>(static_cast<char*>(ys) + align256(ys_bytes(P, E, d, F, dtype, w_format)));
    cv.row_slot = row_slot;
  }
  if (fused_route || f32_routed_up) {
    // routed below
  } else if (!logits) {  // CliffordRouter energy signature, fused into the routing kernel for small N
    if (ygg::route_energy_convert(x, dtype, N, d, router_w, router_b, E, k, topk_idx, topk_w, counts, offsets, perm,
                                  slot_pos, lg, rws, rws_bytes, cv, stream))
      return -1;
  } else if (ygg::route_convert(logits, N, E, k, topk_idx, topk_w, counts, offsets, perm, slot_pos, rws, rws_bytes,
                                cv, stream)) {
    return -1;
  }
  if (w_format == kWPauliF32) {
    // fp32 Pauli: x's Pauli rows (converted with the routing) are gathered through perm
    // by the up product, or the routed up product reads x's blade rows itself; the
    // down product runs in K splits whose partial planes the combine adds in split order
    const int splits = pauli_f32_splits((int)P, E, F, d);
    if (f32_routed_up) {
      if (pauli_f32_up_routed(static_cast<const float*>(x), logits, N, E, k, topk_idx, topk_w, counts, offsets, perm,
                              slot_pos, row_slot, static_cast<const float*>(w_up), b_up, d, F, act,
                              static_cast<float*>(h), h_pre_out, stream))
        return -1;
    } else if (pauli_f32_linear_save_pre(static_cast<const float*>(xs), perm, (int)P,
                                         static_cast<const float*>(w_up), b_up, offsets, E, d, F, act,
                                         static_cast<float*>(h), h_pre_out, stream)) {
      return -1;
    }
    if (pauli_f32_linear_partial(static_cast<const float*>(h), (int)P, static_cast<const float*>(w_down), b_down,
                                 offsets, E, F, d, splits, static_cast<float*>(ys), stream, row_slot))
      return -1;
    return combine_planes(static_cast<const float*>(ys), splits, (int)P, N, k, d, topk_idx, topk_w, slot_pos,
                          residual, out, dtype, stream, /*slot rows*/ true);
  }
  if (w_format == kWPauli) {
    // x's Pauli half-rows (converted with the routing); up: gather those rows through
    // perm inside the product -> h in Pauli half-rows; down: h -> y_sorted in blade
    // order.  No expert-grouped copy of x is made.
    if (ygg_pauli_grouped_linear(xs, /*Pauli rows*/ 1, N, perm, (int)P, w_up, b_up, offsets, E, d, F, act, h,
                                 /*Pauli rows*/ 0, kBF16, stream))
      return -1;
    if (ygg_pauli_grouped_linear(h, /*Pauli rows*/ 1, (int)P, nullptr, (int)P, w_down, b_down, offsets, E, F, d, kActNone, ys,
                                 /*blade*/ 1, kBF16, stream))
      return -1;
    return ygg_combine(ys, kBF16, /*y_mask=*/0, N, k, d, topk_idx, topk_w, slot_pos, residual, out, dtype, stream);
  }
  if (decode) {
    // decode: weight-streaming products; the up product reads x through perm (no
    // dispatch copy) -- or routes itself --, the down product runs in K splits whose
    // fp32 partial planes the combine adds in split order
    if (fused_route) {
      if (decode_linear_gather_routed(static_cast<const uint16_t*>(x), logits, N, E, k, topk_idx, topk_w, counts,
                                      offsets, perm, slot_pos, static_cast<const int8_t*>(w_up), s_up, b_up, d, F,
                                      act, static_cast<uint16_t*>(h), stream))
        return -1;
    } else if (decode_linear_gather(static_cast<const uint16_t*>(x), perm, (int)P, static_cast<const int8_t*>(w_up),
                                    s_up, b_up, offsets, E, d, F, act, static_cast<uint16_t*>(h), stream)) {
      return -1;
    }
    if (decode_linear_partial(static_cast<const uint16_t*>(h), (int)P, static_cast<const int8_t*>(w_down), s_down,
                              b_down, offsets, E, F, d, static_cast<float*>(ys), stream))
      return -1;
    return combine_planes(static_cast<const float*>(ys), decode_splits(F), (int)P, N, k, d, topk_idx, topk_w,
                          slot_pos, residual, out, dtype, stream);
  }
  if (ygg_dispatch(x, dtype, N, k, d, slot_pos, xs, /*to_mask_order=*/1, stream)) return -1;
  if (ygg_grouped_clifford_linear(xs, (int)P, w_up, w_format, s_up, b_up, offsets, E, d, F, act, h, dtype,
                                  /*blade=*/0, stream))
    return -1;
  if (ygg_grouped_clifford_linear(h, (int)P, w_down, w_format, s_down, b_down, offsets, E, F, d, kActNone, ys, dtype,
                                  /*blade=*/1, stream))
    return -1;
  return ygg_combine(ys, dtype, /*y_mask=*/0, N, k, d, topk_idx, topk_w, slot_pos, residual, out, dtype, stream);
}

YGG_API int ygg_moe_forward(const void* x, int dtype, int N, int d, int F, int E, int k, int act,
                            const float* logits, const float* router_w, const float* router_b, const void* w_up,
                            const float* s_up, const float* b_up, const void* w_down, const float* s_down,
                            const float* b_down, int w_format, const void* residual, void* out, int32_t* topk_idx,
                            float* topk_w, int32_t* counts, int32_t* offsets, void* workspace,
                            size_t workspace_bytes, hipStream_t stream) {
  return moe_forward_impl(x, dtype, N, d, F, E, k, act, logits, router_w, router_b, w_up, s_up, b_up, w_down, s_down,
                          b_down, w_format, residual, out, topk_idx, topk_w, counts, offsets, workspace,
                          workspace_bytes, stream, nullptr);
}

// ---- the layer without allocation ------------------------------------------------
// For callers that cannot allocate device memory (code under graph capture, tight
// serving loops): ygg_moe_forward with its workspace taken from a file-scope device
// array instead of a caller-sized buffer.  Every GPU the library runs on holds its
// own copy of the array, from the first call on that GPU until the process ends.
// Its host-side name is only a stand-in: the device address of each GPU's copy
// comes from hipGetSymbolAddress, once per device, and only that address reaches
// kernels.  No region of it needs to start at zero (the layer writes every byte
// it later reads), so calls clear nothing; they share the array, so two calls
// that overlap on one GPU race.
constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;  // YGG_NOALLOC_SCRATCH_BYTES in ygg_moe.h
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the device `stream` runs on (looked up once per
// device, with that device current).
int device_scratch(hipStream_t stream, void** out) {
  int cur = -1;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) {
    set_error("ygg_moe_forward_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    return -1;
  }
  hipDevice_t sdev = cur;
  if (stream != nullptr && (e = hipStreamGetDevice(stream, &sdev)) != hipSuccess) {
    set_error("ygg_moe_forward_noalloc: hipStreamGetDevice: %s", hipGetErrorString(e));
    return -1;
  }
  if (sdev != cur) {
    set_error("ygg_moe_forward_noalloc: the stream belongs to device %d, the current device is %d", (int)sdev, cur);
    return -1;
  }
  if (cur < 0 || cur >= kMaxDevices) {
    set_error("ygg_moe_forward_noalloc: device %d beyond the %d the library tracks", cur, kMaxDevices);
    return -1;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[cur] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error("ygg_moe_forward_noalloc: hipGetSymbolAddress on device %d: %s", cur, hipGetErrorString(e));
      return -1;
    }
    g_scratch_ptr[cur] = p;
  }
  *out = g_scratch_ptr[cur];
  return 0;
}
}  // namespace

YGG_API int ygg_moe_forward_noalloc(const void* x, int dtype, int N, int d, int F, int E, int k, int act,
                                    const float* logits, const float* router_w, const float* router_b,
                                    const void* w_up, const float* s_up, const float* b_up, const void* w_down,
                                    const float* s_down, const float* b_down, int w_format, const void* residual,
                                    void* out, int32_t* topk_idx, float* topk_w, int32_t* counts, int32_t* offsets,
                                    hipStream_t stream) {
  YGG_CHECK_ARG(N >= 0 && d >= 1 && F >= 1 && k >= 1, "ygg_moe_forward_noalloc: bad sizes N=%d d=%d F=%d k=%d", N, d,
                F, k);
  const size_t need = ygg_moe_workspace_bytes(N, d, F, E, k, dtype, w_format);
  YGG_CHECK_ARG(need <= kNoAllocScratchBytes,
                "ygg_moe_forward_noalloc: this layer call needs %zu bytes of scratch, more than the %zu the library "
                "holds per device; use ygg_moe_forward with a workspace",
                need, kNoAllocScratchBytes);
  void* ws = nullptr;
  if (N > 0 && device_scratch(stream, &ws)) return -1;
  return moe_forward_impl(x, dtype, N, d, F, E, k, act, logits, router_w, router_b, w_up, s_up, b_up, w_down, s_down,
                          b_down, w_format, residual, out, topk_idx, topk_w, counts, offsets, ws,
                          kNoAllocScratchBytes, stream, nullptr);
}

// The forward of a training step (fp32 Pauli weights): ygg_moe_forward, and the
// up product's rows before the activation, kept for ygg_moe_backward.
YGG_API int ygg_moe_forward_train(const float* x, int N, int d, int F, int E, int k, int act, const float* logits,
                                  const float* router_w, const float* router_b, const float* w_up, const float* b_up,
                                  const float* w_down, const float* b_down, const float* residual, float* out,
                                  int32_t* topk_idx, float* topk_w, int32_t* counts, int32_t* offsets, float* h_pre,
                                  void* workspace, size_t workspace_bytes, hipStream_t stream) {
  YGG_CHECK_ARG(N == 0 || h_pre, "ygg_moe_forward_train: null h_pre");
  return moe_forward_impl(x, kF32, N, d, F, E, k, act, logits, router_w, router_b, w_up, nullptr, b_up, w_down,
                          nullptr, b_down, kWPauliF32, residual, out, topk_idx, topk_w, counts, offsets, workspace,
                          workspace_bytes, stream, h_pre);
}

YGG_API size_t ygg_moe_block_ffn_workspace_bytes(int N, int d, int F, int E, int k, int dtype, int w_format) {
  const size_t es = (dtype == kF32) ? 4 : 2;
  return align256((size_t)N * d * 8 * es) + ygg_moe_workspace_bytes(N, d, F, E, k, dtype, w_format);
}

YGG_API int ygg_moe_block_ffn(const void* x, int dtype, int N, int d, int F, int E, int k, int act,
                              const float* norm_gamma, const float* norm_beta, double norm_eps, const float* logits,
                              const float* router_w, const float* router_b, const void* w_up, const float* s_up,
                              const float* b_up, const void* w_down, const float* s_down, const float* b_down,
                              int w_format, void* out, int32_t* topk_idx, float* topk_w, int32_t* counts,
                              int32_t* offsets, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  YGG_CHECK_ARG(dtype == kF32 || dtype == kBF16, "ygg_moe_block_ffn: dtype %d unsupported", dtype);
  const size_t need = ygg_moe_block_ffn_workspace_bytes(N, d, F, E, k, dtype, w_format);
  YGG_CHECK_ARG(workspace_bytes >= need, "ygg_moe_block_ffn: workspace of %zu bytes, need %zu", workspace_bytes, need);
  YGG_CHECK_ARG(N == 0 || out != x, "ygg_moe_block_ffn: out must not alias x");
  if (N > 0 && layer_size_check("ygg_moe_block_ffn", N, d, F, E, k, w_format)) return -1;
  // x_norm = ffn_norm(x) at the front of the workspace; the MoE layer gets the
  // rest, and adds x back in its combine
  const size_t xn_bytes = align256((size_t)N * d * 8 * ((dtype == kF32) ? 4 : 2));
  void* xn = workspace;
  if (ygg_clifford_layer_norm(x, dtype, N, d, norm_gamma, norm_beta, norm_eps, xn, dtype, stream)) return -1;
  return ygg_moe_forward(xn, dtype, N, d, F, E, k, act, logits, router_w, router_b, w_up, s_up, b_up, w_down, s_down,
                         b_down, w_format, /*residual=*/x, out, topk_idx, topk_w, counts, offsets,
                         static_cast<char*>(workspace) + xn_bytes, workspace_bytes - xn_bytes, stream);
}

// ---- backward of the layer (fp32, fp32 Pauli weights) -----------------------------
// The routing is recomputed exactly as the forward computed it (same kernels,
// same inputs), so perm, slot_pos and offsets match the forward's; so are the
// activations the backward needs (h before and after the activation, y).
// The regions of its workspace, in order (each 256-byte aligned).
constexpr int kWgradMfmaRowsPerExpert = 256;  // mean rows per expert from which the MFMA weight gradient runs

static int bw_regions(int N, int d, int F, int E, int k, size_t* r) {
  const size_t P = (size_t)N * k;
  int n = 0;
  r[n++] = (size_t)N * k * 4;  // topk_idx
  r[n++] = (size_t)N * k * 4;  // topk_w
  r[n++] = (size_t)E * 4;      // counts
  r[n++] = (size_t)(E + 1) * 4;  // offsets
  r[n++] = P * 4;              // perm
  r[n++] = P * 4;              // slot_pos
  r[n++] = (size_t)N * E * 4;  // logits scratch
  r[n++] = ygg_route_workspace_bytes(N, E, k);
  r[n++] = (size_t)N * d * 32;  // x in Pauli rows
  for (int q = 0; q < 4; ++q) r[n++] = P * F * 32;  // h_pre, h, Pauli rows of h / dh_pre, dh / dh_pre
  for (int q = 0; q < 3; ++q) r[n++] = P * d * 32;  // y / dx rows, dy, Pauli rows of dy
  // weight-gradient partial sums, reused by both products: the up product's
  // (d_in = d, d_out = F) and the down product's (d_in = F, d_out = d, whose
  // bias planes are d-wide), so the larger of the two
  const size_t wg_up = weight_grad_pauli_workspace_bytes((int)P, E, d, F);
  const size_t wg_down = weight_grad_pauli_workspace_bytes((int)P, E, F, d);
  r[n++] = wg_up > wg_down ? wg_up : wg_down;
  return n;
}

YGG_API size_t ygg_moe_backward_workspace_bytes(int N, int d, int F, int E, int k) {
  size_t r[24], b = 0;
  const int n = bw_regions(N, d, F, E, k, r);
  for (int q = 0; q < n; ++q) b += align256(r[q]);
  return b;
}

YGG_API int ygg_moe_backward(const float* x, int N, int d, int F, int E, int k, int act, const float* logits,
                             const float* router_w, const float* router_b, const float* w_up, const float* w_up_adj,
                             const float* b_up, const float* w_down, const float* w_down_adj, const float* b_down,
                             int residual, const float* dout, const float* h_pre_saved, float* dx, float* dw_up,
                             float* db_up, float* dw_down, float* db_down, float* dtopk_w, void* workspace,
                             size_t workspace_bytes, hipStream_t stream) {
  YGG_CHECK_ARG(N >= 0 && d >= 1 && F >= 1 && E >= 1 && k >= 1 && k <= E, "ygg_moe_backward: bad sizes");
  YGG_CHECK_ARG(act >= kActNone && act <= kActSigmoid, "ygg_moe_backward: activation %d", act);
  YGG_CHECK_ARG(workspace_bytes >= ygg_moe_backward_workspace_bytes(N, d, F, E, k),
                "ygg_moe_backward: workspace of %zu bytes, need %zu", workspace_bytes,
                ygg_moe_backward_workspace_bytes(N, d, F, E, k));
  YGG_CHECK_ARG(N == 0 || logits || (router_w && router_b), "ygg_moe_backward: need logits or router parameters");
  YGG_CHECK_ARG(w_up && w_up_adj && w_down && w_down_adj && dw_up && dw_down, "ygg_moe_backward: null weights");
  if (N == 0) {  // no tokens: the weight and bias gradients are zero
    const size_t nw = (size_t)E * F * d * 8;
    if (fill_zero_f32(dw_up, nw, stream) || fill_zero_f32(dw_down, nw, stream)) return -1;
    if (db_up && fill_zero_f32(db_up, (size_t)E * F * 8, stream)) return -1;
    if (db_down && fill_zero_f32(db_down, (size_t)E * d * 8, stream)) return -1;
    return 0;
  }
  YGG_CHECK_ARG(x && dout && dx, "ygg_moe_backward: null x, dout or dx");
  const size_t P = (size_t)N * k;
  size_t sz[24];
  bw_regions(N, d, F, E, k, sz);
  char* base = static_cast<char*>(workspace);
  int next = 0;
  auto take = [&]() {
    void* r = base;
    base += align256(sz[next++]);
    return r;
  };
  int32_t* idx = static_cast<int32_t*>(take());
  float* tw = static_cast<float*>(take());
  int32_t* counts = static_cast<int32_t*>(take());
  int32_t* offsets = static_cast<int32_t*>(take());
  int32_t* perm = static_cast<int32_t*>(take());
  int32_t* slot_pos = static_cast<int32_t*>(take());
  float* lg = static_cast<float*>(take());
  const size_t rws_bytes = align256(sz[next]);
  void* rws = take();
  float* xp = static_cast<float*>(take());
  float* h_pre = static_cast<float*>(take());
  float* h = static_cast<float*>(take());
  float* fp = static_cast<float*>(take());  // Pauli rows of h, then of dh_pre
  float* dh = static_cast<float*>(take());  // dh, then dh_pre in place
  float* y = static_cast<float*>(take());   // y, then dx rows
  float* dy = static_cast<float*>(take());
  float* dp = static_cast<float*>(take());  // Pauli rows of dy
  void* wg = take();                        // weight-gradient partial sums

  // forward recompute: h_pre (unless the forward kept it), h (Pauli rows), y (blade, for dtopk_w)
  const float* hp_in = h_pre_saved;
  // the MFMA weight gradient pays off with enough rows per expert; below that the
  // vector-ALU kernel, which spreads a tile's pairs over more waves, is faster
  const bool wg_mfma = P >= (size_t)kWgradMfmaRowsPerExpert * E;
  // x's Pauli rows, when needed, are converted by extra workgroups of the routing launch
  ygg::RowConvert cv;
  if (!hp_in || wg_mfma) {
    cv.x = x;
    cv.out = xp;
    cv.n = (long long)N * d;
    cv.d = d;
    cv.kind = ygg::kConvF32Pauli;
  }
  if (logits) {
    if (ygg::route_convert(logits, N, E, k, idx, tw, counts, offsets, perm, slot_pos, rws, rws_bytes, cv, stream))
      return -1;
  } else if (ygg::route_energy_convert(x, kF32, N, d, router_w, router_b, E, k, idx, tw, counts, offsets, perm,
                                       slot_pos, lg, rws, rws_bytes, cv, stream)) {
    return -1;
  }
  if (!hp_in) {
    if (ygg_pauli_grouped_linear_f32(xp, perm, (int)P, w_up, b_up, offsets, E, d, F, kActNone, h_pre, 1, stream))
      return -1;
    hp_in = h_pre;
  }
  // h as Pauli rows for the down product (and in blade order for the vector-ALU weight gradient)
  if (activation_forward(hp_in, P * F, act, wg_mfma ? nullptr : h, fp, stream)) return -1;
  if (dtopk_w &&
      ygg_pauli_grouped_linear_f32(fp, nullptr, (int)P, w_down, b_down, offsets, E, F, d, kActNone, y, 1, stream))
    return -1;
  // combine backward -> dy; down backward -> dh, dW_down, db_down
  if (combine_backward(dout, dtopk_w ? y : nullptr, N, k, d, tw, slot_pos, wg_mfma ? nullptr : dy, dp, dtopk_w,
                       stream))
    return -1;
  if (ygg_pauli_grouped_linear_f32(dp, nullptr, (int)P, w_down_adj, nullptr, offsets, E, d, F, kActNone, dh, 1, stream))
    return -1;
  if (wg_mfma ? weight_grad_pauli(dp, fp, nullptr, offsets, (int)P, E, F, d, dw_down, db_down, wg, stream)
              : grouped_weight_grad(dy, h, nullptr, offsets, E, F, d, dw_down, db_down, stream))
    return -1;
  // activation backward -> Pauli rows of dh before the activation; up backward -> dx rows, dW_up, db_up
  if (activation_backward(hp_in, dh, P * F, act, wg_mfma ? nullptr : dh, fp, stream)) return -1;
  if (ygg_pauli_grouped_linear_f32(fp, nullptr, (int)P, w_up_adj, nullptr, offsets, E, F, d, kActNone, y, 1, stream))
    return -1;
  if (wg_mfma ? weight_grad_pauli(fp, xp, perm, offsets, (int)P, E, d, F, dw_up, db_up, wg, stream)
              : grouped_weight_grad(dh, x, perm, offsets, E, d, F, dw_up, db_up, stream))
    return -1;
  // dispatch backward: each token's rows summed, plus dout when the forward added x
  return dispatch_backward(y, N, k, d, slot_pos, residual ? dout : nullptr, dx, stream);
}
