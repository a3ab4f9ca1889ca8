// decode_common.h -- pieces shared by the decode-shape layer kernels
// (decode.hip: int8 L(w)-block weights; decode_pauli.hip: int8 Pauli weights):
// the routing outputs, wave reductions by DPP and the per-row power-of-two
// scaling of activations.
#pragma once

#include "ygg_common.h"

namespace ygg {

// Where a decode layer kernel writes the routing of its batch (as ygg_route does).
struct DcRoute {
  const float* logits;
  int N, E, k;
  int32_t* topk_idx;
  float* topk_w;
  int32_t* counts;
  int32_t* offsets;
  int32_t* perm;
  int32_t* slot_pos;
};

// Reductions over the 64 lanes without LDS round trips: DPP within each row of 16
// lanes (quad permutes, then row rotations by 4 and 8), then the four row results
// read into scalar registers.  The result is wave-uniform.
template <int CTRL>
__device__ inline float dc_dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ inline int dc_dpp(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
// maximum over each row of 16 lanes (every lane of the row holds it)
__device__ inline float dc_row_max(float v) {
  v = fmaxf(v, dc_dpp<0xB1>(v));   // quad_perm [1, 0, 3, 2]
  v = fmaxf(v, dc_dpp<0x4E>(v));   // quad_perm [2, 3, 0, 1]
  v = fmaxf(v, dc_dpp<0x124>(v));  // row_ror 4
  v = fmaxf(v, dc_dpp<0x128>(v));  // row_ror 8
  return v;
}
__device__ inline float dc_wave_max(float v) {
  v = dc_row_max(v);
  const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return fmaxf(fmaxf(a, b), fmaxf(c, d));
}
__device__ inline int dc_wave_sum(int v) {
  v += dc_dpp<0xB1>(v);
  v += dc_dpp<0x4E>(v);
  v += dc_dpp<0x124>(v);
  v += dc_dpp<0x128>(v);
  return (__builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16)) +
         (__builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48));
}

// exponent shift that brings a row's largest magnitude m into [2^13, 2^14).  The
// shift stops at 126 (2^126 and 2^-126 are normal floats), so a row whose largest
// magnitude is below 2^-112 is scaled to below 2^14 and its tiniest entries round to
// zero codes: its error stays below 2^-127 in absolute terms.  Zero and non-finite
// maxima give 0 (a non-finite row's inverse scale is NaN, dc_inv_scale).
__device__ inline int dc_shift(float m) {
  if (!(m > 0.f) || !(m < INFINITY)) return 0;
  int ex;
  frexpf(m, &ex);  // m = f 2^ex, f in [0.5, 1)
  return min(14 - ex, 126);
}
// |v| for a row maximum, with NaN counted as infinite: a row holding NaN or Inf has a
// non-finite maximum (fmaxf would drop a NaN operand)
__device__ inline float dc_mag(float v) {
  const float a = fabsf(v);
  return a == a ? a : INFINITY;
}
// the factor that undoes the shift sh of a row with maximum m: NaN for a non-finite
// row, so that its outputs are NaN as the reference's arithmetic makes them (integer
// codes cannot carry a NaN)
__device__ inline float dc_inv_scale(float m, int sh) { return m < INFINITY ? ldexpf(1.0f, -sh) : __builtin_nanf(""); }

}  // namespace ygg
