// quantize.hip -- grade-aware quantization of multivector weights
// (bifrost/quantization/grade_quantize.py:86-118,153-238): every grade of a
// tensor gets its own bit width, scale and (asymmetric) zero point; codes are
// clip(round(x / scale) + zp, qmin, qmax) and values (q - zp) * scale.
//
// The reference computes in float64 on the whole tensor; so do these kernels
// (MI355X runs fp64 at full vector rate, and this is a one-off weight pass):
//   symmetric   scale = max(max|x|, 1e-12) / qmax,          zp = 0
//   asymmetric  scale = max(max x - min x, 1e-12) / (qmax - qmin),
//               zp = clip(round(qmin - min x / scale), qmin, qmax)
// with round() half to even.  The grade extrema are exact (fp32 inputs), so
// codes and values match the reference bit for bit.

#include <hip/hip_runtime.h>

#include <algorithm>

#include "ygg_common.h"

namespace ygg {
namespace {

struct GradeBits {
  int b[4];
};

__device__ inline int grade_of(int c) { return c == 0 ? 0 : c < 4 ? 1 : c < 7 ? 2 : 3; }

// Grade extrema by integer atomics on order-preserving keys (max and min are exact,
// so the result does not depend on the order of the atomics).  The 12 keys of a
// tensor -- max, min and max |x| of each grade -- live in its own output slots
// until the scales are computed: scales (8 words) hold max and min, zero_points
// (4 words) max |x|.
__device__ inline int order_key(float f) {
  const int u = __builtin_bit_cast(int, f);
  return u >= 0 ? u : u ^ 0x7fffffff;
}
__device__ inline float key_value(int k) { return __builtin_bit_cast(float, k >= 0 ? k : k ^ 0x7fffffff); }

__global__ void grade_init_kernel(int T, int* __restrict__ S, int* __restrict__ Z) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= T) return;
  for (int g = 0; g < 4; ++g) {
    S[t * 8 + g] = order_key(-INFINITY);
    S[t * 8 + 4 + g] = order_key(INFINITY);
    Z[t * 4 + g] = order_key(0.f);
  }
}

// grid (T, blocks per tensor): each thread reads whole multivectors (two 16-byte
// loads), the workgroup reduces its 12 extrema, one lane per extremum applies them.
__global__ __launch_bounds__(256) void grade_extrema_kernel(const float* __restrict__ W, size_t n_mv,
                                                            int* __restrict__ S, int* __restrict__ Z) {
  __shared__ float red[12][256];
  const int t = blockIdx.x;
  const float* base = W + (size_t)t * n_mv * 8;
  float mx[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY}, mn[4] = {INFINITY, INFINITY, INFINITY, INFINITY},
        am[4] = {0.f, 0.f, 0.f, 0.f};
  for (size_t m = (size_t)blockIdx.y * 256 + threadIdx.x; m < n_mv; m += (size_t)gridDim.y * 256) {
    const float4* p = reinterpret_cast<const float4*>(base + m * 8);
    const float4 u = p[0], v = p[1];
    const float x[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int g = grade_of(c);
      mx[g] = fmaxf(mx[g], x[c]);
      mn[g] = fminf(mn[g], x[c]);
      am[g] = fmaxf(am[g], fabsf(x[c]));
    }
  }
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    red[g][threadIdx.x] = mx[g];
    red[4 + g][threadIdx.x] = mn[g];
    red[8 + g][threadIdx.x] = am[g];
  }
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s)
#pragma unroll
      for (int q = 0; q < 12; ++q) {
        const float o = red[q][threadIdx.x + s];
        red[q][threadIdx.x] = (q >= 4 && q < 8) ? fminf(red[q][threadIdx.x], o) : fmaxf(red[q][threadIdx.x], o);
      }
    __syncthreads();
  }
  if (threadIdx.x < 12) {
    const int q = threadIdx.x, key = order_key(red[q][0]);
    if (q < 4) atomicMax(&S[t * 8 + q], key);
    else if (q < 8) atomicMin(&S[t * 8 + q], key);
    else atomicMax(&Z[t * 4 + q - 8], key);
  }
}

// One thread per tensor (it reads all 12 keys before overwriting them):
//   symmetric   scale = max(max|x|, 1e-12) / qmax,          zp = 0
//   asymmetric  scale = max(max x - min x, 1e-12) / (qmax - qmin),
//               zp = clip(round(qmin - min x / scale), qmin, qmax)
__global__ void grade_params_kernel(int T, size_t n_mv, GradeBits bits, int symmetric, double* __restrict__ scales,
                                    int32_t* __restrict__ zero_points) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= T) return;
  const int* S = reinterpret_cast<const int*>(scales);
  float mx[4], mn[4], am[4];
  for (int g = 0; g < 4; ++g) {
    mx[g] = key_value(S[t * 8 + g]);
    mn[g] = key_value(S[t * 8 + 4 + g]);
    am[g] = key_value(zero_points[t * 4 + g]);
  }
  for (int g = 0; g < 4; ++g) {
    const int b = bits.b[g];
    const double qmin = -(double)(1 << (b - 1)), qmax = (double)((1 << (b - 1)) - 1);
    double scale, zp = 0.0;
    if (symmetric) {
      const double a = n_mv ? (double)am[g] : 1.0;
      scale = fmax(a, 1e-12) / qmax;
    } else {
      const double dmin = n_mv ? (double)mn[g] : 0.0, dmax = n_mv ? (double)mx[g] : 1.0;
      scale = fmax(dmax - dmin, 1e-12) / (qmax - qmin);
      zp = fmin(fmax(rint(qmin - dmin / scale), qmin), qmax);
    }
    scales[t * 4 + g] = scale;
    zero_points[t * 4 + g] = (int32_t)zp;
  }
}

// One thread per component.
__global__ __launch_bounds__(256) void grade_quantize_kernel(const float* __restrict__ W, size_t n_mv, int T,
                                                             GradeBits bits, const double* __restrict__ scales,
                                                             const int32_t* __restrict__ zero_points,
                                                             int16_t* __restrict__ codes,
                                                             float* __restrict__ dequant) {
  const size_t n = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (n >= (size_t)T * n_mv * 8) return;
  const int tensor = (int)(n / (n_mv * 8)), c = (int)(n & 7), g = grade_of(c);
  const int b = bits.b[g];
  const double qmin = -(double)(1 << (b - 1)), qmax = (double)((1 << (b - 1)) - 1);
  const double s = scales[tensor * 4 + g], zp = (double)zero_points[tensor * 4 + g];
  const double q = fmin(fmax(rint((double)W[n] / s) + zp, qmin), qmax);
  if (codes) codes[n] = (int16_t)q;
  if (dequant) dequant[n] = (float)((q - zp) * s);
}

}  // namespace
}  // namespace ygg

using namespace ygg;

YGG_API int ygg_grade_quantize(const float* W, int T, size_t mv_per_tensor, const int32_t* grade_bits, int symmetric,
                               int16_t* codes, double* scales, int32_t* zero_points, float* dequant,
                               hipStream_t stream) {
  YGG_CHECK_ARG(T >= 0, "ygg_grade_quantize: T=%d", T);
  YGG_CHECK_ARG(grade_bits, "ygg_grade_quantize: null grade_bits");
  GradeBits bits;
  for (int g = 0; g < 4; ++g) {
    YGG_CHECK_ARG(grade_bits[g] >= 2 && grade_bits[g] <= 16, "ygg_grade_quantize: grade %d bit width %d not in [2, 16]",
                  g, grade_bits[g]);
    bits.b[g] = grade_bits[g];
  }
  if (T == 0) return 0;
  YGG_CHECK_ARG(W && scales && zero_points, "ygg_grade_quantize: null pointer argument");
  int* S = reinterpret_cast<int*>(scales);
  const unsigned tb = (unsigned)((T + 255) / 256);
  hipLaunchKernelGGL(grade_init_kernel, dim3(tb), dim3(256), 0, stream, T, S, zero_points);
  if (mv_per_tensor > 0) {
    // about four multivectors per thread, and at most 65535 blocks per tensor
    const size_t per = std::min<size_t>((mv_per_tensor + 1023) / 1024, 65535);
    hipLaunchKernelGGL(grade_extrema_kernel, dim3(T, (unsigned)per), dim3(256), 0, stream, W, mv_per_tensor, S,
                       zero_points);
  }
  hipLaunchKernelGGL(grade_params_kernel, dim3(tb), dim3(256), 0, stream, T, mv_per_tensor, bits, symmetric, scales,
                     zero_points);
  if (check_launch("ygg_grade_quantize")) return -1;
  const size_t total = (size_t)T * mv_per_tensor * 8;
  if (total == 0 || (!codes && !dequant)) return 0;
  hipLaunchKernelGGL(grade_quantize_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, W,
                     mv_per_tensor, T, bits, scales, zero_points, codes, dequant);
  return check_launch("ygg_grade_quantize");
}
