// norm.hip -- CliffordLayerNorm, the pre-norm in front of the MoE layer
// (holograph/layers/normalization.py:44-67), and the FFN half of
// HLMBlock.forward, x + moe(ffn_norm(x)) (holograph/models/hlm_block.py:144-151).
//
// The norm is HBM-bound: one read and one write of each token row (R bytes
// each) plus the (d, 8) gamma and beta, which stay in L2.  One wave owns one
// token: lane l holds multivectors l, l+64, ...; the per-multivector squared
// norms go to LDS, groups of 8 lanes sum the runs of NumPy's pairwise order,
// every lane combines the run sums into the mean, and the second pass writes
// gamma x_hat + beta.
//
// Bit-level parity with the reference's fp32 NumPy expression:
//  * |x_i|^2 = sum over the 8 components of the rounded squares, in NumPy's
//    pairwise order for 8 values: ((s0+s1)+(s2+s3)) + ((s4+s5)+(s6+s7));
//  * the mean over d is NumPy's pairwise sum (eight strided accumulators per
//    run of at most 128 values, a tree, then the remainder; longer runs split
//    at n/2 rounded down to a multiple of 8) divided by d;
//  * rms = sqrt(mean + fp32(2 eps)); x_hat = x / rms (IEEE divide and sqrt);
//  * the geometric product gamma x_hat adds, for each output blade, the eight
//    rounded products (s gamma_a) x_hat_b in the order of gamma's blade a,
//    starting from zero (rune/ops/batched.py:72-82), then beta.
// No multiply-add contraction anywhere (pragma in every arithmetic function).

#include <hip/hip_runtime.h>

#include "ygg_common.h"

namespace ygg {
namespace {

constexpr int kNormWaves = 4;       // tokens per 256-thread workgroup, one wave each
constexpr int kNormMaxD = 4096;     // the pairwise plan below covers this length
constexpr int kPwBlock = 128;       // NumPy's pairwise block
constexpr int kMaxLeaves = 40;      // runs of at most 128 values in the plan for d <= 4096 (33 at most)

// ---- NumPy's pairwise sum, spread over the lanes of a wave ------------------------
// The recursion (split n > 128 at n/2 rounded down to a multiple of 8) depends
// on d only, so the host lists its leaves -- runs of at most 128 values -- in
// order.  Eight lanes sum one leaf: lane j holds accumulator j (elements j,
// j+8, ... below the last full row of 8, added in order), three xor shuffles
// form ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)), and the remaining n % 8 values are
// added in order.  The leaf sums are then combined along the recursion.
struct PwPlan {
  int n_leaves;
  uint16_t start[kMaxLeaves];
  uint16_t len[kMaxLeaves];
};

constexpr int kPwDepth = 6;  // recursion levels pw_combine unrolls; d <= 4096 needs 6

// Appends the leaves of a run of n values at s; false if the plan would need
// more than kMaxLeaves leaves or kPwDepth levels.
bool pw_plan_add(PwPlan& p, int s, int n, int depth = 0) {
  if (n <= kPwBlock) {
    if (p.n_leaves >= kMaxLeaves) return false;
    p.start[p.n_leaves] = (uint16_t)s;
    p.len[p.n_leaves] = (uint16_t)n;
    ++p.n_leaves;
    return true;
  }
  if (depth >= kPwDepth) return false;
  int n2 = n / 2;
  n2 -= n2 % 8;
  return pw_plan_add(p, s, n2, depth + 1) && pw_plan_add(p, s + n2, n - n2, depth + 1);
}

// Sum of one leaf of n values at a (LDS) by the 8 lanes j = 0..7 of a group;
// every lane of the group returns the sum.
__device__ inline float pw_leaf_lanes(const float* a, int n, int j) {
#pragma clang fp contract(off)
  if (n < 8) {  // only d < 8: one leaf, summed in order from zero
    float s = 0.f;
    for (int i = 0; i < n; ++i) s = s + a[i];
    return s;
  }
  const int rows = n >> 3;  // 1..16
  float t[kPwBlock / 8];
#pragma unroll
  for (int q = 0; q < kPwBlock / 8; ++q) t[q] = (q < rows) ? a[8 * q + j] : 0.f;
  float r = t[0];
#pragma unroll
  for (int q = 1; q < kPwBlock / 8; ++q)
    if (q < rows) r = r + t[q];
  r = r + __shfl_xor(r, 1);
  r = r + __shfl_xor(r, 2);
  r = r + __shfl_xor(r, 4);
  for (int i = 8 * rows; i < n; ++i) r = r + a[i];
  return r;
}

// The leaf sums (in order) combined along the recursion over n.
template <int DEPTH>
__device__ float pw_combine(const float* leaf, int n, int& next) {
#pragma clang fp contract(off)
  if constexpr (DEPTH == 0) {
    return leaf[next++];
  } else {
    if (n <= kPwBlock) return leaf[next++];
    int n2 = n >> 1;
    n2 -= n2 & 7;
    const float l = pw_combine<DEPTH - 1>(leaf, n2, next);
    const float r = pw_combine<DEPTH - 1>(leaf, n - n2, next);
    return l + r;
  }
}

// ---- one multivector in and out ------------------------------------------------
// Raw storage of one input multivector: the loads are issued early and the
// values unpacked only when used, so bf16 rows hold 4 registers, not 8.
template <typename IT>
struct Mv;
template <>
struct Mv<float> {
  float4 a, b;
};
template <>
struct Mv<uint16_t> {
  uint4 a;
};

__device__ inline Mv<float> load_raw(const float* row, int i) {
  const float4* p = reinterpret_cast<const float4*>(row + (size_t)i * 8);
  return Mv<float>{p[0], p[1]};
}
__device__ inline Mv<uint16_t> load_raw(const uint16_t* row, int i) {
  return Mv<uint16_t>{*reinterpret_cast<const uint4*>(row + (size_t)i * 8)};
}
__device__ inline void unpack(const Mv<float>& m, float v[8]) {
  v[0] = m.a.x; v[1] = m.a.y; v[2] = m.a.z; v[3] = m.a.w;
  v[4] = m.b.x; v[5] = m.b.y; v[6] = m.b.z; v[7] = m.b.w;
}
__device__ inline void unpack(const Mv<uint16_t>& m, float v[8]) {
  const uint32_t w[4] = {m.a.x, m.a.y, m.a.z, m.a.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    v[2 * q] = __builtin_bit_cast(float, w[q] << 16);
    v[2 * q + 1] = __builtin_bit_cast(float, w[q] & 0xffff0000u);
  }
}
__device__ inline void store_mv(float* row, int i, const float v[8]) {
  float4* p = reinterpret_cast<float4*>(row + (size_t)i * 8);
  p[0] = make_float4(v[0], v[1], v[2], v[3]);
  p[1] = make_float4(v[4], v[5], v[6], v[7]);
}
__device__ inline void store_mv(uint16_t* row, int i, const float v[8]) {
  *reinterpret_cast<uint4*>(row + (size_t)i * 8) =
      make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
}

__device__ inline float squared_norm(const float v[8]) {
#pragma clang fp contract(off)
  float s[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) s[c] = v[c] * v[c];
  return ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
}

// y = gamma x_hat + beta for one multivector, x_hat = v / rms.
__device__ inline void scale_shift(float v[8], float rms, const Mv<float>& g, const Mv<float>& bt) {
#pragma clang fp contract(off)
  float xh[8], ga[8], be[8];
  unpack(g, ga);
  unpack(bt, be);
#pragma unroll
  for (int c = 0; c < 8; ++c) xh[c] = v[c] / rms;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int mc = blade_to_mask(c);
    float s = 0.f;
#pragma unroll
    for (int a = 0; a < 8; ++a) {
      const int ma = blade_to_mask(a);
      const int b = mask_to_blade(ma ^ mc);
      const float ga_s = mask_product_sign(ma, ma ^ mc) > 0 ? ga[a] : -ga[a];
      s = s + ga_s * xh[b];
    }
    v[c] = s + be[c];
  }
}

// One wave normalises one token.  Every load of the wave -- the first 64 CACHE
// multivectors of the row and of gamma and beta -- is issued before any
// arithmetic.  Multivectors past 64 CACHE (d > 256) are read again from L2 in
// the second pass.
template <typename IT, typename OT, int CACHE>
__global__ __launch_bounds__(256) void layer_norm_kernel(const IT* __restrict__ x, int N, int d,
                                                         const float* __restrict__ gamma,
                                                         const float* __restrict__ beta, float two_eps,
                                                         const PwPlan plan, OT* __restrict__ y) {
#pragma clang fp contract(off)
  extern __shared__ float lds[];  // per wave: d squared norms, then kMaxLeaves leaf sums
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x * kNormWaves + wave;
  const bool live = t < N;
  const IT* xr = x + (size_t)(live ? t : 0) * d * 8;
  float* ns = lds + wave * (d + kMaxLeaves);
  float* ls = ns + d;

  Mv<IT> raw[CACHE];
  Mv<float> g[CACHE], bt[CACHE];
#pragma unroll
  for (int q = 0; q < CACHE; ++q)
    if (live && lane + 64 * q < d) raw[q] = load_raw(xr, lane + 64 * q);
#pragma unroll
  for (int q = 0; q < CACHE; ++q)
    if (lane + 64 * q < d) {
      g[q] = load_raw(gamma, lane + 64 * q);
      bt[q] = load_raw(beta, lane + 64 * q);
    }

  // pass 1: |x_i|^2 of every multivector into LDS
  if (live) {
#pragma unroll
    for (int q = 0; q < CACHE; ++q)
      if (lane + 64 * q < d) {
        float v[8];
        unpack(raw[q], v);
        ns[lane + 64 * q] = squared_norm(v);
      }
    for (int i = lane + 64 * CACHE; i < d; i += 64) {
      float v[8];
      unpack(load_raw(xr, i), v);
      ns[i] = squared_norm(v);
    }
  }
  __syncthreads();
  // the pairwise sum: 8 leaves at a time, one per group of 8 lanes
  const int grp = lane >> 3, j = lane & 7;
  if (live) {
    for (int L = grp; L < plan.n_leaves; L += 8) {
      const float r = pw_leaf_lanes(ns + plan.start[L], plan.len[L], j);
      if (j == 0) ls[L] = r;
    }
  }
  __syncthreads();
  if (!live) return;
  int next = 0;
  const float mean = pw_combine<kPwDepth>(ls, d, next) / (float)d;
  const float rms = sqrtf(mean + two_eps);

  // pass 2: gamma x_hat + beta
  OT* yr = y + (size_t)t * d * 8;
#pragma unroll
  for (int q = 0; q < CACHE; ++q) {
    const int i = lane + 64 * q;
    if (i < d) {
      float v[8];
      unpack(raw[q], v);
      scale_shift(v, rms, g[q], bt[q]);
      store_mv(yr, i, v);
    }
  }
  for (int i = lane + 64 * CACHE; i < d; i += 64) {
    float v[8];
    unpack(load_raw(xr, i), v);
    scale_shift(v, rms, load_raw(gamma, i), load_raw(beta, i));
    store_mv(yr, i, v);
  }
}

template <typename IT, typename OT>
int launch_norm(const void* x, int N, int d, const float* gamma, const float* beta, float two_eps, void* y,
                hipStream_t stream) {
  PwPlan plan{};
  YGG_CHECK_ARG(pw_plan_add(plan, 0, d), "ygg_clifford_layer_norm: no pairwise plan for d=%d", d);
  const int blocks = (N + kNormWaves - 1) / kNormWaves;
  const size_t lds = (size_t)kNormWaves * (d + kMaxLeaves) * sizeof(float);
  if (d <= 128)
    hipLaunchKernelGGL((layer_norm_kernel<IT, OT, 2>), dim3(blocks), dim3(64 * kNormWaves), lds, stream,
                       static_cast<const IT*>(x), N, d, gamma, beta, two_eps, plan, static_cast<OT*>(y));
  else
    hipLaunchKernelGGL((layer_norm_kernel<IT, OT, 4>), dim3(blocks), dim3(64 * kNormWaves), lds, stream,
                       static_cast<const IT*>(x), N, d, gamma, beta, two_eps, plan, static_cast<OT*>(y));
  return check_launch("ygg_clifford_layer_norm");
}

}  // namespace
}  // namespace ygg

using namespace ygg;

YGG_API int ygg_clifford_layer_norm(const void* x, int x_dtype, int N, int d, const float* gamma, const float* beta,
                                    double eps, void* y, int y_dtype, hipStream_t stream) {
  YGG_CHECK_ARG(x_dtype == kF32 || x_dtype == kBF16, "ygg_clifford_layer_norm: x dtype %d unsupported", x_dtype);
  YGG_CHECK_ARG(y_dtype == kF32 || y_dtype == kBF16, "ygg_clifford_layer_norm: y dtype %d unsupported", y_dtype);
  YGG_CHECK_ARG(N >= 0 && d >= 1 && d <= kNormMaxD, "ygg_clifford_layer_norm: bad sizes N=%d d=%d (d <= %d)", N, d,
                kNormMaxD);
  YGG_CHECK_ARG(eps >= 0.0, "ygg_clifford_layer_norm: eps must be non-negative");
  if (N == 0) return 0;
  YGG_CHECK_ARG(x && gamma && beta && y, "ygg_clifford_layer_norm: null pointer argument");
  YGG_CHECK_ARG(x != y, "ygg_clifford_layer_norm: y must not alias x");
  const float two_eps = (float)(2.0 * eps);  // the reference adds the Python float 2*eps to an fp32 array
  if (x_dtype == kF32)
    return y_dtype == kF32 ? launch_norm<float, float>(x, N, d, gamma, beta, two_eps, y, stream)
                           : launch_norm<float, uint16_t>(x, N, d, gamma, beta, two_eps, y, stream);
  return y_dtype == kF32 ? launch_norm<uint16_t, float>(x, N, d, gamma, beta, two_eps, y, stream)
                         : launch_norm<uint16_t, uint16_t>(x, N, d, gamma, beta, two_eps, y, stream);
}
