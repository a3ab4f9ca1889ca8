// norm.hip -- CliffordLayerNorm, the pre-norm in front of the MoE layer
// (holograph/layers/normalization.py:44-67), and the FFN half of
// HLMBlock.forward, x + moe(ffn_norm(x)) (holograph/models/hlm_block.py:144-151).
//
// The norm is HBM-bound: one read and one write of each token row (R bytes
// each) plus the (d, 8) gamma and beta, which stay in L2.  One wave owns one
// token: lane l holds multivectors l, l+64, ...; the per-multivector squared
// norms go to LDS, every lane of the wave then forms the same mean in NumPy's
// pairwise order, and the second pass writes gamma x_hat + beta.
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
constexpr int kNormMaxD = 4096;     // the pairwise recursion below covers this length
constexpr int kNormCache = 4;       // multivectors per lane kept in registers between the passes
constexpr int kPwBlock = 128;       // NumPy's pairwise block

// ---- NumPy pairwise sum over LDS (all lanes read the same addresses) ----------
__device__ inline float pw_leaf(const float* a, int n) {
#pragma clang fp contract(off)
  if (n < 8) {
    float s = 0.f;
    for (int i = 0; i < n; ++i) s = s + a[i];
    return s;
  }
  float r[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = a[j];
  const int n8 = n - (n & 7);
  for (int i = 8; i < n8; i += 8) {
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = r[j] + a[i + j];
  }
  float s = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
  for (int i = n8; i < n; ++i) s = s + a[i];
  return s;
}

// Each split leaves pieces of at most n/2 + 8 values, so 6 levels take 4096
// values down to runs of at most 128.
template <int DEPTH>
__device__ float pw_sum(const float* a, int n) {
#pragma clang fp contract(off)
  if constexpr (DEPTH == 0) {
    return pw_leaf(a, n);
  } else {
    if (n <= kPwBlock) return pw_leaf(a, n);
    int n2 = n >> 1;
    n2 -= n2 & 7;
    return pw_sum<DEPTH - 1>(a, n2) + pw_sum<DEPTH - 1>(a + n2, n - n2);
  }
}

constexpr int kPwDepth = 6;

constexpr bool pw_depth_covers(int n, int depth) {
  if (n <= kPwBlock) return true;
  if (depth == 0) return false;
  int n2 = n / 2;
  n2 -= n2 % 8;
  return pw_depth_covers(n2, depth - 1) && pw_depth_covers(n - n2, depth - 1);
}
constexpr bool pw_depth_covers_all(int n_max, int depth) {
  for (int n = 1; n <= n_max; ++n)
    if (!pw_depth_covers(n, depth)) return false;
  return true;
}
static_assert(pw_depth_covers_all(kNormMaxD, kPwDepth), "pairwise recursion depth must cover every d <= kNormMaxD");

// ---- one multivector in and out ------------------------------------------------
__device__ inline void load_mv(const float* row, int i, float v[8]) {
  const float4* p = reinterpret_cast<const float4*>(row + (size_t)i * 8);
  const float4 a = p[0], b = p[1];
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
__device__ inline void load_mv(const uint16_t* row, int i, float v[8]) {
  const uint4 u = *reinterpret_cast<const uint4*>(row + (size_t)i * 8);
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
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
__device__ inline void scale_shift(float v[8], float rms, const float* __restrict__ g, const float* __restrict__ bt) {
#pragma clang fp contract(off)
  float xh[8], ga[8], be[8];
  const float4 g0 = reinterpret_cast<const float4*>(g)[0], g1 = reinterpret_cast<const float4*>(g)[1];
  const float4 b0 = reinterpret_cast<const float4*>(bt)[0], b1 = reinterpret_cast<const float4*>(bt)[1];
  ga[0] = g0.x; ga[1] = g0.y; ga[2] = g0.z; ga[3] = g0.w; ga[4] = g1.x; ga[5] = g1.y; ga[6] = g1.z; ga[7] = g1.w;
  be[0] = b0.x; be[1] = b0.y; be[2] = b0.z; be[3] = b0.w; be[4] = b1.x; be[5] = b1.y; be[6] = b1.z; be[7] = b1.w;
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

template <typename IT, typename OT>
__global__ __launch_bounds__(256) void layer_norm_kernel(const IT* __restrict__ x, int N, int d,
                                                         const float* __restrict__ gamma,
                                                         const float* __restrict__ beta, float two_eps,
                                                         OT* __restrict__ y) {
#pragma clang fp contract(off)
  extern __shared__ float norm_sq[];  // (kNormWaves, d)
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x * kNormWaves + wave;
  const bool live = t < N;
  const IT* xr = x + (size_t)(live ? t : 0) * d * 8;
  float* ns = norm_sq + wave * d;

  float v[kNormCache][8];
#pragma unroll
  for (int q = 0; q < kNormCache; ++q) {
    const int i = lane + 64 * q;
    if (live && i < d) {
      load_mv(xr, i, v[q]);
      ns[i] = squared_norm(v[q]);
    }
  }
  if (live) {
    for (int i = lane + 64 * kNormCache; i < d; i += 64) {
      float w[8];
      load_mv(xr, i, w);
      ns[i] = squared_norm(w);
    }
  }
  __syncthreads();
  if (!live) return;
  const float mean = pw_sum<kPwDepth>(ns, d) / (float)d;
  const float rms = sqrtf(mean + two_eps);

  OT* yr = y + (size_t)t * d * 8;
#pragma unroll
  for (int q = 0; q < kNormCache; ++q) {
    const int i = lane + 64 * q;
    if (i < d) {
      scale_shift(v[q], rms, gamma + (size_t)i * 8, beta + (size_t)i * 8);
      store_mv(yr, i, v[q]);
    }
  }
  for (int i = lane + 64 * kNormCache; i < d; i += 64) {
    float w[8];
    load_mv(xr, i, w);
    scale_shift(w, rms, gamma + (size_t)i * 8, beta + (size_t)i * 8);
    store_mv(yr, i, w);
  }
}

template <typename IT, typename OT>
int launch_norm(const void* x, int N, int d, const float* gamma, const float* beta, float two_eps, void* y,
                hipStream_t stream) {
  const int blocks = (N + kNormWaves - 1) / kNormWaves;
  const size_t lds = (size_t)kNormWaves * d * sizeof(float);
  hipLaunchKernelGGL((layer_norm_kernel<IT, OT>), dim3(blocks), dim3(64 * kNormWaves), lds, stream,
                     static_cast<const IT*>(x), N, d, gamma, beta, two_eps, static_cast<OT*>(y));
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
