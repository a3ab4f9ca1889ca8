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

#include "ygg_common.h"

namespace ygg {
namespace {

struct GradeBits {
  int b[4];
};

__host__ __device__ constexpr int grade_lo(int g) { return g == 0 ? 0 : g == 1 ? 1 : g == 2 ? 4 : 7; }
__host__ __device__ constexpr int grade_width(int g) { return (g == 1 || g == 2) ? 3 : 1; }
__device__ inline int grade_of(int c) { return c == 0 ? 0 : c < 4 ? 1 : c < 7 ? 2 : 3; }

// One workgroup per (tensor, grade): extrema over that grade's components,
// then the grade's scale and zero point.
__global__ __launch_bounds__(256) void grade_params_kernel(const float* __restrict__ W, size_t n_mv, GradeBits bits,
                                                           int symmetric, double* __restrict__ scales,
                                                           int32_t* __restrict__ zero_points) {
  __shared__ float smax[256], smin[256];
  const int tensor = blockIdx.x >> 2, g = blockIdx.x & 3;
  const int lo = grade_lo(g), w = grade_width(g);
  const float* base = W + (size_t)tensor * n_mv * 8;
  float mx = -INFINITY, mn = INFINITY, amax = 0.f;
  const size_t n = n_mv * (size_t)w;
  for (size_t u = threadIdx.x; u < n; u += 256) {
    const float v = base[(u / w) * 8 + lo + (u % w)];
    mx = fmaxf(mx, v);
    mn = fminf(mn, v);
    amax = fmaxf(amax, fabsf(v));
  }
  smax[threadIdx.x] = symmetric ? amax : mx;
  smin[threadIdx.x] = mn;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s) {
      smax[threadIdx.x] = fmaxf(smax[threadIdx.x], smax[threadIdx.x + s]);
      smin[threadIdx.x] = fminf(smin[threadIdx.x], smin[threadIdx.x + s]);
    }
    __syncthreads();
  }
  if (threadIdx.x != 0) return;
  const int b = bits.b[g];
  const double qmin = -(double)(1 << (b - 1)), qmax = (double)((1 << (b - 1)) - 1);
  double scale, zp = 0.0;
  if (symmetric) {
    const double am = n ? (double)smax[0] : 1.0;
    scale = fmax(am, 1e-12) / qmax;
  } else {
    const double dmin = n ? (double)smin[0] : 0.0, dmax = n ? (double)smax[0] : 1.0;
    scale = fmax(dmax - dmin, 1e-12) / (qmax - qmin);
    zp = fmin(fmax(rint(qmin - dmin / scale), qmin), qmax);
  }
  scales[tensor * 4 + g] = scale;
  zero_points[tensor * 4 + g] = (int32_t)zp;
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
  hipLaunchKernelGGL(grade_params_kernel, dim3(4 * T), dim3(256), 0, stream, W, mv_per_tensor, bits, symmetric,
                     scales, zero_points);
  if (check_launch("ygg_grade_quantize")) return -1;
  const size_t total = (size_t)T * mv_per_tensor * 8;
  if (total == 0 || (!codes && !dequant)) return 0;
  hipLaunchKernelGGL(grade_quantize_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, W,
                     mv_per_tensor, T, bits, scales, zero_points, codes, dequant);
  return check_launch("ygg_grade_quantize");
}
