// ygg_common.h -- shared definitions for the MI355X (gfx950) MoE-HLM kernels.
//
// Multivector layouts used on the device
// --------------------------------------
// * "blade order" -- the reference's flat layout 1,e1,e2,e3,e12,e13,e23,e123
//   (rune/types/multivector.py:7).  Every tensor that crosses the C ABI
//   (layer input x, layer output, user-visible weights) is in blade order.
// * "mask order" -- component c is the blade whose generator bitmask is c
//   (bit0 = e1, bit1 = e2, bit2 = e3): 1,e1,e2,e12,e3,e13,e23,e123.  In this
//   order the geometric product of basis blades is  e_p e_q = s(p,q) e_{p^q},
//   so the 8x8 block L(w) of a weight multivector is a signed XOR-permutation.
//   Internal activations between the two expert products are kept in mask
//   order, and the prepared weights are stored in mask order.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#ifndef YGG_API
#define YGG_API extern "C" __attribute__((visibility("default")))
#endif

namespace ygg {

// blade index (blade order) -> generator bitmask; the map is an involution
// except for the e3 / e12 swap: mask order position of blade b is kBladeMask[b].
__host__ __device__ constexpr int blade_to_mask(int b) {
  return b == 0 ? 0 : b == 1 ? 1 : b == 2 ? 2 : b == 3 ? 4 : b == 4 ? 3 : b == 5 ? 5 : b == 6 ? 6 : 7;
}
__host__ __device__ constexpr int mask_to_blade(int m) {
  return m == 0 ? 0 : m == 1 ? 1 : m == 2 ? 2 : m == 3 ? 4 : m == 4 ? 3 : m == 5 ? 5 : m == 6 ? 6 : 7;
}

// Sign of e_A e_B for generator bitmasks A, B in Cl(3,0): (-1)^(number of
// pairs x in A, y in B with x > y) -- each such pair is one transposition
// needed to bring the concatenated word into sorted order; e_i e_i = +1.
__host__ __device__ constexpr int mask_product_sign(int a, int b) {
  int swaps = 0;
  for (int x = 0; x < 3; ++x)
    if (a & (1 << x))
      for (int y = 0; y < x; ++y)
        if (b & (1 << y)) ++swaps;
  return (swaps & 1) ? -1 : 1;
}

// --- weight sign folding ---------------------------------------------------
// Prepared weights store  W'_p = kWFold[p] * W_p  (mask order) and every
// output blade r of a product is produced as  kOutFold[r] * y_r.  With this
// choice the remaining sign of every entry of the expanded block,
//   kOutFold[r] * kWFold[p] * s(p, p^r)   (A operand at mask position p),
// is -1 on exactly one aligned pair {2t, 2t+1} of p for each r and +1
// elsewhere, so one 32-bit XOR per output blade applies all signs to a
// packed bf16 operand.  (Found by exhaustive search over the 2^16 sign
// foldings of weights and inputs; checked by static_assert below.)
__host__ __device__ constexpr int kWFold(int p) { return (p == 2 || p == 4) ? -1 : 1; }
__host__ __device__ constexpr int kOutFold(int r) { return (r == 0 || r == 4) ? -1 : 1; }

// Residual sign of entry (r, p) after folding.
__host__ __device__ constexpr int folded_sign(int r, int p) {
  return kOutFold(r) * kWFold(p) * mask_product_sign(p, p ^ r);
}
// The aligned pair index t (p in {2t, 2t+1}) that carries the -1 for row r.
__host__ __device__ constexpr int neg_pair(int r) {
  return folded_sign(r, 0) < 0 ? 0 : folded_sign(r, 2) < 0 ? 1 : folded_sign(r, 4) < 0 ? 2 : 3;
}

constexpr bool check_folding() {
  for (int r = 0; r < 8; ++r) {
    int t = neg_pair(r);
    for (int p = 0; p < 8; ++p) {
      int want = (p / 2 == t) ? -1 : 1;
      if (folded_sign(r, p) != want) return false;
    }
  }
  return true;
}
static_assert(check_folding(), "sign folding must leave one negative aligned pair per output blade");

// --- bf16 helpers (bit-level; round to nearest even) --------------------------
__host__ __device__ inline uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7f800000u) == 0x7f800000u) return (uint16_t)((u >> 16) | ((u & 0xffffu) ? 0x40u : 0u));  // inf / nan
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__host__ __device__ inline float bf16_bits_to_f32(uint16_t h) {
  return __builtin_bit_cast(float, (uint32_t)h << 16);
}
__device__ inline uint32_t pack_bf16x2(float lo, float hi) {
  return (uint32_t)f32_to_bf16_bits(lo) | ((uint32_t)f32_to_bf16_bits(hi) << 16);
}

// --- raw buffer loads ----------------------------------------------------
// Descriptor word 3 for gfx9-family raw buffers (32-bit data format).  A raw
// buffer load whose offset lies past the descriptor's range reads zero, so
// tails and out-of-range lanes need no branch and no select on loaded data.
constexpr int kBufferFlags = 0x00020000;
constexpr uint32_t kBufferOff = 0x80000000u;  // an offset that reads zero

// --- error reporting ------------------------------------------------------
void set_error(const char* fmt, ...);
int check_launch(const char* what);

enum DType : int { kF32 = 0, kBF16 = 1, kI8 = 2 };
enum Act : int { kActNone = 0, kActGelu = 1, kActRelu = 2, kActSigmoid = 3 };
// prepared weight formats (ygg_prepare_weights)
enum WFormat : int { kWF32 = 0, kWBF16 = 1, kWI8 = 2, kWPauli = 3, kWPauliF32 = 4, kWPauliI8 = 5 };

// bf16 Pauli weight layout (pauli_gemm.hip)
int pauli_prepare_weights(const float* W, int E, int d_out, int d_in, void* out, hipStream_t stream);
// bf16 Pauli products: the kernel a call takes, and whether its sizes fit that
// kernel's 32-bit buffer offsets (nullptr) or why not; x_layout / y_layout as
// ygg_pauli_grouped_linear's (0: blade rows gathered / Pauli rows out; 1: Pauli rows
// in / blade rows out)
bool pauli_uses_dma(int x_layout, int d_in);
const char* pauli_size_limit(int x_layout, int x_rows, bool gathered, int P_max, int E, int d_in, int d_out,
                             int y_layout, int y_dtype);

// Blade rows -> Pauli rows carried by the workgroups of another launch (the routing
// kernels append them to their own): n multivectors of x, rows of d, bf16 -> bf16
// Pauli half-rows (ygg_pauli_rows_from_blade) or fp32 -> fp32 Pauli rows
// (ygg_pauli_rows_from_blade_f32), with the same results as those calls.
enum RowConvertKind : int { kConvNone = 0, kConvBf16Pauli = 1, kConvF32Pauli = 2 };
struct RowConvert {
  const void* x = nullptr;
  void* out = nullptr;
  long long n = 0;  // multivectors (rows x d)
  int d = 0;
  int kind = kConvNone;
  // when set, the routing also writes each expert-grouped row's slot:
  // row_slot[slot_pos[f]] = f (the K-split products then write slot rows)
  int32_t* row_slot = nullptr;
};
// The rows [r0, r1) of a conversion (the rows of d multivectors of x), as a
// conversion of its own: x and out advanced to row r0 (x: 8 values per
// multivector of bf16 or fp32; out: bf16 Pauli half-row pairs or fp32 Pauli rows,
// 8 values per multivector either way), the same results as the whole one.
inline RowConvert row_convert_part(const RowConvert& cv, long long r0, long long r1) {
  RowConvert p = cv;
  if (cv.kind == kConvNone || cv.d <= 0) return p;
  const size_t es = cv.kind == kConvBf16Pauli ? 2 : 4;
  p.x = static_cast<const char*>(cv.x) + (size_t)r0 * cv.d * 8 * es;
  p.out = static_cast<char*>(cv.out) + (size_t)r0 * cv.d * 8 * es;
  p.n = (r1 - r0) * cv.d;
  return p;
}
// ygg_route that also runs `cv` in the same launches
int route_convert(const float* logits, int N, int E, int k, int32_t* topk_idx, float* topk_w, int32_t* counts,
                  int32_t* offsets, int32_t* perm, int32_t* slot_pos, void* workspace, size_t workspace_bytes,
                  const RowConvert& cv, hipStream_t stream);
// ygg_route_energy likewise
int route_energy_convert(const void* x, int x_dtype, int N, int d, const float* router_w, const float* router_b, int E,
                         int k, int32_t* topk_idx, float* topk_w, int32_t* counts, int32_t* offsets, int32_t* perm,
                         int32_t* slot_pos, float* logits_scratch, void* workspace, size_t workspace_bytes,
                         const RowConvert& cv, hipStream_t stream);

// fp32 Pauli products (pauli_f32.hip): weight preparation (format 4), the
// number of K splits the layer uses for a down product, and that K-split
// product writing fp32 partial planes (splits, P_max, d_out, 8), blade order,
// bias in split 0, no activation.
int pauli_f32_prepare_weights(const float* W, int E, int d_out, int d_in, void* out, hipStream_t stream);
int pauli_f32_splits(int P_max, int E, int d_in, int d_out);
// The fp32 Pauli product writing Pauli rows (activation applied) and, when
// y_pre is not NULL, the blade-order rows before the activation.
int pauli_f32_linear_save_pre(const float* x, const int32_t* gather, int P_max, const float* w, const float* bias,
                              const int32_t* offsets, int E, int d_in, int d_out, int act, float* y_pauli,
                              float* y_pre, hipStream_t stream);
int pauli_f32_linear_partial(const float* x, int P_max, const float* w, const float* bias, const int32_t* offsets,
                             int E, int d_in, int d_out, int splits, float* y_planes, hipStream_t stream,
                             const int32_t* row_map = nullptr);  // row_map: the planes' row of each product row
// The up product with the routing of the batch inside it (no routing launch): from
// the logits and the blade rows of x, the routing arrays of ygg_route (and row_slot,
// when not NULL) and the Pauli rows of h, as pauli_f32_linear_save_pre writes them.
// For batches of at most 256 tokens, 32 experts and 64 input multivectors.
bool pauli_f32_route_fusable(int N, int E, int k, int d_in);
int pauli_f32_up_routed(const float* x, const float* logits, int N, int E, int k, int32_t* topk_idx, float* topk_w,
                        int32_t* counts, int32_t* offsets, int32_t* perm, int32_t* slot_pos, int32_t* row_slot,
                        const float* w, const float* bias, int d_in, int d_out, int act, float* y_pauli,
                        float* y_pre, hipStream_t stream);

// decode-shape int8 products (clifford_gemm.hip): whether (P_max rows, E
// experts, format) takes the weight-streaming kernel, its number of K splits
// for a given d_in, the up product reading blade-order rows of x through the
// routing permutation (mask-order bf16 output, activation fused), and the
// K-split product writing fp32 partial planes (splits, P_max, d_out, 8) in
// blade order, bias in split 0, no activation.
bool decode_shape(int P_max, int E, int format);
int decode_splits(int d_in);
int decode_linear_gather(const uint16_t* x, const int32_t* perm, int P_max, const int8_t* Wq, const float* scales,
                         const float* bias, const int32_t* offsets, int E, int d_in, int d_out, int act, uint16_t* h,
                         hipStream_t stream);
// The up product with the routing inside it (decode layers given logits):
// whether (N, E, k, d_in) qualifies, and the launch, which also writes the
// routing arrays (as ygg_route) for the down product and the combine.
bool decode_route_fusable(int N, int E, int k, int d_in);
int decode_linear_gather_routed(const uint16_t* x, const float* logits, int N, int E, int k, int32_t* topk_idx,
                                float* topk_w, int32_t* counts, int32_t* offsets, int32_t* perm, int32_t* slot_pos,
                                const int8_t* Wq, const float* scales, const float* bias, int d_in, int d_out, int act,
                                uint16_t* h, hipStream_t stream);
int decode_linear_partial(const uint16_t* x, int P_max, const int8_t* Wq, const float* scales, const float* bias,
                          const int32_t* offsets, int E, int d_in, int d_out, float* y_planes, hipStream_t stream);

// The decode-shape layer with int8 weights in one launch (decode.hip): routing
// of every token inside each workgroup, the up product with bias and
// activation, and the down product cut along its contraction into
// decode_layer_planes(F) fp32 partial planes (planes, P_max = N k, d, 8),
// blade order, the down bias in plane 0; the routing arrays as ygg_route.
bool decode_layer_fusable(int N, int E, int k, int d, int F);
int decode_layer_planes(int F);
int decode_layer(const uint16_t* x, const float* logits, int N, int E, int k, int d, int F, int act,
                 const int8_t* w_up, const float* s_up, const float* b_up, const int8_t* w_dn, const float* s_dn,
                 const float* b_dn, int32_t* topk_idx, float* topk_w, int32_t* counts, int32_t* offsets,
                 int32_t* perm, int32_t* slot_pos, float* planes, hipStream_t stream);

// The decode-shape layer on int8 Pauli weights (format 5, decode_pauli.hip):
// the prepared size and preparation (codes plus one fp32 scale per expert and
// output channel), whether (N, E, k, d, F) fits the one-launch layer, its number
// of partial planes, and the launch, with the outputs of decode_layer.
size_t decode_pauli_weight_bytes(int E, int d_out, int d_in);
int decode_pauli_prepare_weights(const float* W, int E, int d_out, int d_in, void* out, float* scales,
                                 hipStream_t stream);
bool decode_pauli_fusable(int N, int E, int k, int d, int F);
int decode_pauli_planes(int F);
int decode_pauli_layer(const uint16_t* x, const float* logits, int N, int E, int k, int d, int F, int act,
                       const int8_t* w_up, const float* s_up, const float* b_up, const int8_t* w_dn,
                       const float* s_dn, const float* b_dn, int32_t* topk_idx, float* topk_w, int32_t* counts,
                       int32_t* offsets, int32_t* perm, int32_t* slot_pos, float* planes, hipStream_t stream);

// combine of fp32 blade-order partial planes (dispatch.hip): the planes of a
// row are added in plane order, then weighted and combined as ygg_combine does.
// slot_rows: the planes hold slot (t, s) at row t k + s, not at slot_pos[t k + s]
int combine_planes(const float* y_planes, int planes, int P_max, int N, int k, int d, const int32_t* topk_idx,
                   const float* topk_w, const int32_t* slot_pos, const void* residual, void* out, int out_dtype,
                   hipStream_t stream, bool slot_rows = false);

// backward pieces (backward.hip), all fp32 blade order: the grouped weight
// gradient dW[e, j, i] = sum_rows dy[r, j] ~a[src(r), i] (src through gather
// when not NULL) and db (when not NULL); the activations' backward; the
// combine's (dy[slot] = w dout_t, dtopk_w = <dout_t, y[slot]> when y_sorted
// is not NULL) and the dispatch's (dx_t = residual_grad_t + sum_s dxs[slot]).
int grouped_weight_grad(const float* dy, const float* a, const int32_t* gather, const int32_t* offsets, int E,
                        int d_in, int d_out, float* dW, float* db, hipStream_t stream);
// The same weight and bias gradients on the fp32 MFMA units from fp32 Pauli rows
// (pauli_f32.hip's layout) of dy (P_max rows) and a; per-chunk partial sums go to
// `workspace` (weight_grad_pauli_workspace_bytes) and are added in chunk order.
size_t weight_grad_pauli_workspace_bytes(int P_max, int E, int d_in, int d_out);
int weight_grad_pauli(const float* dy_pauli, const float* a_pauli, const int32_t* gather, const int32_t* offsets,
                      int P_max, int E, int d_in, int d_out, float* dW, float* db, void* workspace,
                      hipStream_t stream);
// (out may alias g; out and out_pauli -- fp32 Pauli rows -- are each optional)
int activation_backward(const float* h, const float* g, size_t n_mv, int act, float* out, float* out_pauli,
                        hipStream_t stream);
int activation_forward(const float* h, size_t n_mv, int act, float* out, float* out_pauli, hipStream_t stream);
int fill_zero_f32(float* p, size_t n, hipStream_t stream);  // n floats at p set to zero
int combine_backward(const float* dout, const float* y_sorted, int N, int k, int d, const float* topk_w,
                     const int32_t* slot_pos, float* dy_sorted, float* dy_pauli, float* dtopk_w, hipStream_t stream);
int dispatch_backward(const float* dxs, int N, int k, int d, const int32_t* slot_pos, const float* residual_grad,
                      float* dx, hipStream_t stream);

inline int dtype_size(int dt) { return dt == kF32 ? 4 : dt == kBF16 ? 2 : dt == kI8 ? 1 : 0; }

}  // namespace ygg

#define YGG_CHECK_ARG(cond, ...)        \
  do {                                  \
    if (!(cond)) {                      \
      ::ygg::set_error(__VA_ARGS__);    \
      return -1;                        \
    }                                   \
  } while (0)
