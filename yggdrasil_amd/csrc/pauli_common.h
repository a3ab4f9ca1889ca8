// pauli_common.h -- Pauli (2x2 complex) coordinates of Cl(3,0) multivectors
// and the grade-wise activations in blade coordinates, shared by the bf16 and
// fp32 Pauli expert-product kernels.
//
// A multivector  s + v1 e1 + v2 e2 + v3 e3 + b12 e12 + b13 e13 + b23 e23 + t e123
// (blade order 1,e1,e2,e3,e12,e13,e23,e123) maps to the matrix
//   M00 = (s + v3) + i (t + b12)     M01 = (v1 - b13) + i (b23 - v2)
//   M10 = (v1 + b13) + i (b23 + v2)  M11 = (s - v3) + i (t - b12)
// (e1 -> sx, e2 -> sy, e3 -> sz), and the geometric product to the matrix
// product.
#pragma once

#include "ygg_common.h"

namespace ygg {

typedef __bf16 pbf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 pbf16x2_t __attribute__((ext_vector_type(2)));
typedef float pf32x2_t __attribute__((ext_vector_type(2)));
typedef float pf32x16_t __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------------------
// activations in blade coordinates (hardware exp2 / rcp / sqrt)
// ---------------------------------------------------------------------------
// sigma(z) = 1 / (1 + e^-z).  tanh-GELU:  0.5 v (1 + tanh(u)) = v sigma(2u),
// u = sqrt(2/pi) (v + 0.044715 v^3); the magnitude gate (c / |c|) gelu(|c|)
// is  c sigma(2 u(|c|)); tanh(t) = 2 sigma(2t) - 1.
__device__ inline float fsigmoid(float z) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * z));
}
// gelu(v) / v = sigma(k2 (v + 0.044715 v^3)) with k2 = 2 sqrt(2/pi), i.e.
// 1 / (1 + 2^(v (a + b v^2))): a = -log2(e) k2, b = 0.044715 a folded into one
// multiply-add (three VALU operations before the exponential instead of five).
__device__ inline float gelu_gate(float v) {
  constexpr float a = -1.4426950408889634f * 2.0f * 0.7978845608028654f;
  constexpr float b = a * 0.044715f;
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(v * __builtin_fmaf(b, v * v, a)));
}
// tanh(t) = 2 sigma(2 t) - 1, with -2 log2(e) folded
__device__ inline float ftanh(float t) {
  return __builtin_fmaf(2.0f, __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-2.8853900817779268f * t)), -1.0f);
}

// y: blade order 1,e1,e2,e3,e12,e13,e23,e123
template <int ACT>
__device__ inline void activate_blade(float* y) {
  if constexpr (ACT == kActNone) {
    return;
  } else {
    // grade norms, sqrt(1e-12 + sum of squares) as three multiply-adds
    const float m1 =
        __builtin_amdgcn_sqrtf(__builtin_fmaf(y[3], y[3], __builtin_fmaf(y[2], y[2], __builtin_fmaf(y[1], y[1], 1e-12f))));
    const float m2 =
        __builtin_amdgcn_sqrtf(__builtin_fmaf(y[6], y[6], __builtin_fmaf(y[5], y[5], __builtin_fmaf(y[4], y[4], 1e-12f))));
    float f0, f1, f2;
    if constexpr (ACT == kActGelu) {
      f0 = gelu_gate(y[0]);
      f1 = gelu_gate(m1);
      f2 = gelu_gate(m2);
      y[7] = ftanh(y[7]);
    } else if constexpr (ACT == kActSigmoid) {
      y[0] = fsigmoid(y[0]);
      f0 = 1.0f;
      f1 = fsigmoid(m1) * __builtin_amdgcn_rcpf(m1);
      f2 = fsigmoid(m2) * __builtin_amdgcn_rcpf(m2);
      y[7] = ftanh(y[7]);
    } else {  // relu with zero thresholds: grade 0 clamps, the rest pass through
      f0 = y[0] > 0.f ? 1.0f : 0.0f;
      f1 = 1.0f;
      f2 = 1.0f;
    }
    y[0] *= f0;
    y[1] *= f1;
    y[2] *= f1;
    y[3] *= f1;
    y[4] *= f2;
    y[5] *= f2;
    y[6] *= f2;
  }
}

// blade -> Pauli columns: col0 = (M00, M10), col1 = (M01, M11), (re, im) each
__device__ inline void blade_to_pauli(const float* x, float* c0, float* c1) {
  c0[0] = x[0] + x[3];  // M00 re = s + v3
  c0[1] = x[7] + x[4];  // M00 im = t + b12
  c0[2] = x[1] + x[5];  // M10 re = v1 + b13
  c0[3] = x[6] + x[2];  // M10 im = b23 + v2
  c1[0] = x[1] - x[5];  // M01 re = v1 - b13
  c1[1] = x[6] - x[2];  // M01 im = b23 - v2
  c1[2] = x[0] - x[3];  // M11 re = s - v3
  c1[3] = x[7] - x[4];  // M11 im = t - b12
}

// Pauli (already halved by the weights) -> blade.  y00 = (re, im) of Y[0][0], ...
__device__ inline void pauli_to_blade(float y00r, float y00i, float y01r, float y01i, float y10r, float y10i,
                                      float y11r, float y11i, float* x) {
  x[0] = y00r + y11r;  // s
  x[3] = y00r - y11r;  // v3
  x[7] = y00i + y11i;  // t
  x[4] = y00i - y11i;  // b12
  x[1] = y10r + y01r;  // v1
  x[5] = y10r - y01r;  // b13
  x[6] = y10i + y01i;  // b23
  x[2] = y10i - y01i;  // v2
}

// blade -> one fp32 Pauli row multivector ([b][re, im][c], 8 floats; the layout of
// pauli_f32.hip) at dst
__device__ inline void store_pauli_f32(float* dst, const float* x) {
  float c0[4], c1[4];
  blade_to_pauli(x, c0, c1);  // c0 = (M00, M10), c1 = (M01, M11)
  float4* q = reinterpret_cast<float4*>(dst);
  q[0] = make_float4(c0[0], c0[2], c0[1], c0[3]);
  q[1] = make_float4(c1[0], c1[2], c1[1], c1[3]);
}

// two floats -> packed bf16 pair (v_cvt_pk_bf16_f32, round to nearest even)
__device__ inline uint32_t pack2_bf16(float lo, float hi) {
  const pf32x2_t f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, pbf16x2_t));
}
__device__ inline float bf_lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ inline float bf_hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

// Multivector n = m d + i of blade-order bf16 rows (rows, d, 8) -> its two Pauli
// half-rows (bf16, rounded to nearest even): (M00, M10) at half-row 2 m, (M01, M11)
// at 2 m + 1, (re, im) each.
__device__ inline void pauli_rows_bf16_one(const uint16_t* __restrict__ x, int d, size_t n,
                                           uint16_t* __restrict__ out) {
  const size_t m = n / d;
  const int i = (int)(n - m * d);
  const uint4 q = *reinterpret_cast<const uint4*>(x + n * 8);
  const float v[8] = {bf_lo(q.x), bf_hi(q.x), bf_lo(q.y), bf_hi(q.y), bf_lo(q.z), bf_hi(q.z), bf_lo(q.w), bf_hi(q.w)};
  float c0[4], c1[4];
  blade_to_pauli(v, c0, c1);
  *reinterpret_cast<uint2*>(out + ((2 * m) * d + i) * 4) = make_uint2(pack2_bf16(c0[0], c0[1]), pack2_bf16(c0[2], c0[3]));
  *reinterpret_cast<uint2*>(out + ((2 * m + 1) * d + i) * 4) =
      make_uint2(pack2_bf16(c1[0], c1[1]), pack2_bf16(c1[2], c1[3]));
}

// Multivector n of blade-order fp32 rows -> its fp32 Pauli row record: eight floats
// [b][k][c] (column b, re / im k, row c) at out + 8 n.
__device__ inline void pauli_rows_f32_one(const float* __restrict__ x, size_t n, float* __restrict__ out) {
  const float4 p0 = reinterpret_cast<const float4*>(x + n * 8)[0];
  const float4 p1 = reinterpret_cast<const float4*>(x + n * 8)[1];
  const float v[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
  float c0[4], c1[4];
  blade_to_pauli(v, c0, c1);
  float4* q = reinterpret_cast<float4*>(out + n * 8);
  q[0] = make_float4(c0[0], c0[2], c0[1], c0[3]);
  q[1] = make_float4(c1[0], c1[2], c1[1], c1[3]);
}

// Workgroup b's share of a RowConvert riding on another launch: THREADS x U
// multivectors, U per thread at a stride of THREADS (coalesced).  Every load of the
// thread is issued before the first conversion (an index past the end repeats the
// last multivector and is not stored), so a thread waits for memory once.
template <int THREADS, int U>
__device__ inline void convert_rows_block(const RowConvert& cv, int b) {
  const long long base = (long long)b * THREADS * U + threadIdx.x;
  if (base >= cv.n) return;
  size_t n[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const long long v = base + (long long)u * THREADS;
    n[u] = (size_t)(v < cv.n ? v : cv.n - 1);
  }
  if (cv.kind == kConvBf16Pauli) {
    const uint16_t* x = static_cast<const uint16_t*>(cv.x);
    uint16_t* out = static_cast<uint16_t*>(cv.out);
    uint4 q[U];
#pragma unroll
    for (int u = 0; u < U; ++u) q[u] = *reinterpret_cast<const uint4*>(x + n[u] * 8);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (base + (long long)u * THREADS >= cv.n) break;
      const size_t m = n[u] / cv.d;
      const int i = (int)(n[u] - m * cv.d);
      const float v[8] = {bf_lo(q[u].x), bf_hi(q[u].x), bf_lo(q[u].y), bf_hi(q[u].y),
                          bf_lo(q[u].z), bf_hi(q[u].z), bf_lo(q[u].w), bf_hi(q[u].w)};
      float c0[4], c1[4];
      blade_to_pauli(v, c0, c1);
      *reinterpret_cast<uint2*>(out + ((2 * m) * cv.d + i) * 4) =
          make_uint2(pack2_bf16(c0[0], c0[1]), pack2_bf16(c0[2], c0[3]));
      *reinterpret_cast<uint2*>(out + ((2 * m + 1) * cv.d + i) * 4) =
          make_uint2(pack2_bf16(c1[0], c1[1]), pack2_bf16(c1[2], c1[3]));
    }
  } else {
    const float* x = static_cast<const float*>(cv.x);
    float* out = static_cast<float*>(cv.out);
    float4 p0[U], p1[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      p0[u] = reinterpret_cast<const float4*>(x + n[u] * 8)[0];
      p1[u] = reinterpret_cast<const float4*>(x + n[u] * 8)[1];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (base + (long long)u * THREADS >= cv.n) break;
      const float v[8] = {p0[u].x, p0[u].y, p0[u].z, p0[u].w, p1[u].x, p1[u].y, p1[u].z, p1[u].w};
      float c0[4], c1[4];
      blade_to_pauli(v, c0, c1);
      float4* q = reinterpret_cast<float4*>(out + n[u] * 8);
      q[0] = make_float4(c0[0], c0[2], c0[1], c0[3]);
      q[1] = make_float4(c1[0], c1[2], c1[1], c1[3]);
    }
  }
}
template <int THREADS, int U>
inline int convert_rows_blocks(const RowConvert& cv) {
  return cv.kind == kConvNone ? 0 : (int)((cv.n + (long long)THREADS * U - 1) / ((long long)THREADS * U));
}

// (re, im) -> (im, -re) on each bf16 pair of a dword, in one packed 16-bit add:
// op_sel swaps the halves of w, and adding 0x8000 to the new high half flips its
// sign bit (no carry reaches the other half).  The compiler builds it from two
// instructions (a shift and an add), and this runs twice per MFMA.
__device__ inline uint32_t rot_conj(uint32_t w) {
  uint32_t r;
  asm("v_pk_add_u16 %0, %1, %2 op_sel:[1,0] op_sel_hi:[0,1]" : "=v"(r) : "v"(w), "s"(0x80000000u));
  return r;
}

}  // namespace ygg
