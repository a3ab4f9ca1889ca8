// clifford_gemm.hip -- grouped CliffordLinear expert products on gfx950.
//
// Replaces, for every expert e of the MoE-HLM layer, CliffordLinear.forward
// (holograph/layers/clifford_linear.py:101-123) on that expert's rows,
//     y[m, j] = sum_i  W[j, i] * x[m, i]  (+ b[j])      (* = geometric product)
// which the reference computes with rune.ops.batched.geom_matmul
// (rune/ops/batched.py:320-344), followed by the grade-wise activation
// (holograph/layers/activations.py:15-128) for the up projection.
//
// As a dense contraction:  Y[m, (j,r)] = sum_{(i,q)} X[m, (i,q)] L(W[j,i])[r, q],
// K = 8 d_in, N = 8 d_out, 128 d_in d_out FLOPs per row -- L(w) has no zeros.
//
// MFMA mapping (bf16 / int8 weights, v_mfma_f32_32x32x16_bf16)
// ------------------------------------------------------------
// * K is walked two input multivectors at a time: lane l of a wave holds
//   the 8 components (mask order) of multivector i0 + l/32 of row l%32 --
//   exactly one A fragment.  No activation expansion is needed.
// * One accumulator per output blade r: the B fragment for blade r holds,
//   in lane (j = l%32, i = i0 + l/32), row r of L(W[j,i]):  in mask order
//   L[r, q] = s(q^r, q) W[q^r], i.e. W permuted by XOR with r plus signs.
//   The prepared weights store each multivector twice (plain and with every
//   aligned pair swapped) with signs folded in (ygg_common.h), so B for
//   blade r is a static choice of 32-bit registers plus one XOR.
// * All 8 components of output multivector (m, j) land in the same lane, so
//   bias, grade-wise activation, int8 scale and the output layout are fused
//   into the epilogue with no shuffles.
//
// Row tiles never straddle experts: tile t of the launch maps to (expert,
// first row) by walking the device-side offsets, so the grid is sized from
// host-known bounds (ceil(P/BM) + E tiles) with no host synchronisation.

#include "route_select.h"
#include "ygg_common.h"

namespace ygg {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------------------
// activations (mask order: grade = popcount of the component index)
// ---------------------------------------------------------------------------
__device__ inline float gelu_f(float v) {
  const float k0 = 0.7978845608028654f;  // sqrt(2/pi)
  return 0.5f * v * (1.0f + tanhf(k0 * (v + 0.044715f * v * v * v)));
}
__device__ inline float sigmoid_f(float v) {
  return v >= 0.f ? 1.0f / (1.0f + expf(-v)) : expf(v) / (1.0f + expf(v));
}

template <int ACT>
__device__ inline void activate_mask_order(float* y) {
  if constexpr (ACT == kActNone) {
    return;
  } else {
    // grade 0 (scalar): component 0
    if constexpr (ACT == kActGelu) y[0] = gelu_f(y[0]);
    if constexpr (ACT == kActRelu) y[0] = fmaxf(y[0], 0.f);
    if constexpr (ACT == kActSigmoid) y[0] = sigmoid_f(y[0]);
    // grades 1 {1,2,4} and 2 {3,5,6}: direction times activated magnitude
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const int c0 = g == 0 ? 1 : 3, c1 = g == 0 ? 2 : 5, c2 = g == 0 ? 4 : 6;
      const float mag = sqrtf(y[c0] * y[c0] + y[c1] * y[c1] + y[c2] * y[c2] + 1e-12f);
      float gm;
      if constexpr (ACT == kActGelu) gm = gelu_f(mag);
      if constexpr (ACT == kActRelu) gm = fmaxf(mag, 0.f);
      if constexpr (ACT == kActSigmoid) gm = sigmoid_f(mag);
      const float f = gm / mag;
      y[c0] *= f;
      y[c1] *= f;
      y[c2] *= f;
    }
    // grade 3: tanh for gelu and sigmoid; relu keeps sign(t) * max(|t|, 0) = t
    if constexpr (ACT != kActRelu) y[7] = tanhf(y[7]);
  }
}

// ---------------------------------------------------------------------------
// row-tile -> expert mapping
// ---------------------------------------------------------------------------
__device__ inline bool find_tile(const int32_t* __restrict__ offsets, int E, int BM, int tile, int& e, int& row0,
                                 int& row_end) {
  int acc = 0;
  int beg = offsets[0];
  for (int x = 0; x < E; ++x) {
    const int end = offsets[x + 1];
    const int nt = (end - beg + BM - 1) / BM;
    if (tile < acc + nt) {
      e = x;
      row0 = beg + (tile - acc) * BM;
      row_end = end;
      return true;
    }
    acc += nt;
    beg = end;
  }
  return false;
}

// ---------------------------------------------------------------------------
// weight preparation
// ---------------------------------------------------------------------------
// Quantisation scale per (expert, output channel): max(absmax, 1e-12) / 127,
// computed in float64 and rounded to fp32.
__global__ __launch_bounds__(256) void quant_scale_kernel(const float* __restrict__ W, int d_in,
                                                          float* __restrict__ scales) {
  __shared__ float red[256];
  const size_t base = (size_t)blockIdx.x * d_in * 8;
  float m = 0.f;
  for (int i = threadIdx.x; i < d_in * 8; i += 256) m = fmaxf(m, fabsf(W[base + i]));
  red[threadIdx.x] = m;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + s]);
    __syncthreads();
  }
  if (threadIdx.x == 0) scales[blockIdx.x] = (float)(fmax((double)red[0], 1e-12) / 127.0);
}

__device__ inline int quantize_one(float w, float s) {
  double q = rint((double)w / (double)s);
  q = fmin(fmax(q, -127.0), 127.0);
  return (int)q;
}

// One thread per prepared multivector slot (padding included).
__global__ __launch_bounds__(256) void prep_weights_kernel(const float* __restrict__ W, int E, int d_out, int d_in,
                                                           int fmt, const float* __restrict__ scales,
                                                           void* __restrict__ out) {
  const int JB = (d_out + 31) / 32, IP = (d_in + 1) / 2;
  const size_t total = (fmt == kWF32) ? (size_t)E * d_out * d_in : (size_t)E * JB * IP * 64;
  const size_t n = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (n >= total) return;
  int e, j, i;
  if (fmt == kWF32) {
    i = (int)(n % d_in);
    j = (int)((n / d_in) % d_out);
    e = (int)(n / ((size_t)d_in * d_out));
  } else {
    const int ih = (int)(n & 1), jj = (int)((n >> 1) & 31);
    size_t rest = n >> 6;
    const int ip = (int)(rest % IP);
    rest /= IP;
    const int jb = (int)(rest % JB);
    e = (int)(rest / JB);
    j = jb * 32 + jj;
    i = ip * 2 + ih;
  }
  float v[8];  // mask order, folded
  const bool valid = (j < d_out) && (i < d_in);
#pragma unroll
  for (int p = 0; p < 8; ++p)
    v[p] = valid ? (float)kWFold(p) * W[(((size_t)e * d_out + j) * d_in + i) * 8 + mask_to_blade(p)] : 0.f;
  if (fmt == kWF32) {
    float* o = static_cast<float*>(out) + n * 8;
#pragma unroll
    for (int p = 0; p < 8; ++p) o[p] = v[p];
  } else if (fmt == kWBF16) {
    uint16_t* o = static_cast<uint16_t*>(out) + n * 16;
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      o[p] = f32_to_bf16_bits(v[p]);
      o[8 + p] = f32_to_bf16_bits(v[p ^ 1]);
    }
  } else {
    int8_t* o = static_cast<int8_t*>(out) + n * 8;
    const float s = valid ? scales[(size_t)e * d_out + j] : 1.f;
#pragma unroll
    for (int p = 0; p < 8; ++p) o[p] = (int8_t)(valid ? quantize_one(v[p], s) : 0);
  }
}

__global__ __launch_bounds__(256) void prep_bias_kernel(const float* __restrict__ b, size_t n_mv,
                                                        float* __restrict__ out) {
  const size_t n = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (n >= n_mv) return;
#pragma unroll
  for (int p = 0; p < 8; ++p) out[n * 8 + p] = b[n * 8 + mask_to_blade(p)];
}

// ---------------------------------------------------------------------------
// bf16 / int8-weight MFMA kernel
// ---------------------------------------------------------------------------
template <int R>
__device__ inline bf16x8_t blade_operand(const uint32_t (&raw)[4], const uint32_t (&sw)[4]) {
  constexpr int tneg = neg_pair(R) ^ (R >> 1);  // negative pair in k (input component) order
  uint32_t d[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    d[t] = (R & 1) ? sw[t ^ (R >> 1)] : raw[t ^ (R >> 1)];
    if (t == tneg) d[t] ^= 0x80008000u;
  }
  return __builtin_bit_cast(bf16x8_t, d);
}

__device__ inline uint32_t i8pair_to_bf16x2(int lo, int hi) {
  // |q| <= 127 has at most 7 significant bits: the top 16 bits of the fp32
  // value are the exact bf16 value.
  const uint32_t a = __builtin_bit_cast(uint32_t, (float)lo);
  const uint32_t b = __builtin_bit_cast(uint32_t, (float)hi);
  return (a >> 16) | (b & 0xffff0000u);
}

template <int OUT_DT>
__device__ inline void store_out8(void* Y, size_t mv, const float* y, bool blade_order) {
  float o[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) o[c] = y[c];
  if (blade_order) {
    o[3] = y[4];
    o[4] = y[3];
  }
  if constexpr (OUT_DT == kF32) {
    float4* p = reinterpret_cast<float4*>(static_cast<float*>(Y) + mv * 8);
    p[0] = make_float4(o[0], o[1], o[2], o[3]);
    p[1] = make_float4(o[4], o[5], o[6], o[7]);
  } else {
    uint4 q;
    q.x = pack_bf16x2(o[0], o[1]);
    q.y = pack_bf16x2(o[2], o[3]);
    q.z = pack_bf16x2(o[4], o[5]);
    q.w = pack_bf16x2(o[6], o[7]);
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(Y) + mv * 8) = q;
  }
}

constexpr int kMfmaBM = 64;  // rows per workgroup (2 waves x 32)
constexpr int kMfmaBN = 64;  // output multivectors per workgroup (2 waves x 32)

template <int ACT, bool OUT_BLADE, bool WI8, int OUT_DT>
__global__ __launch_bounds__(256, 2) void grouped_cl_mfma(const uint16_t* __restrict__ A, const void* __restrict__ Wp,
                                                          const float* __restrict__ wscale,
                                                          const float* __restrict__ bias,
                                                          const int32_t* __restrict__ offsets, int E, int d_in,
                                                          int d_out, void* __restrict__ Y) {
  int e, row0, row_end;
  if (!find_tile(offsets, E, kMfmaBM, blockIdx.x, e, row0, row_end)) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int JB = (d_out + 31) >> 5, IP = (d_in + 1) >> 1;
  const int jb = blockIdx.y * 2 + wn;
  if (jb >= JB) return;
  const int ih = lane >> 5, l32 = lane & 31;
  const int arow = row0 + wm * 32 + l32;
  const bool arow_ok = arow < row_end;
  const uint16_t* aptr = A + ((size_t)(arow_ok ? arow : row0) * d_in + ih) * 8;
  const size_t wslot0 = (((size_t)e * JB + jb) * IP) * 64 + l32 * 2 + ih;

  f32x16_t acc[8];
#pragma unroll
  for (int r = 0; r < 8; ++r)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[r][v] = 0.f;

  for (int ip = 0; ip < IP; ++ip) {
    const int i = 2 * ip + ih;
    uint4 a = make_uint4(0, 0, 0, 0);
    if (arow_ok && i < d_in) a = *reinterpret_cast<const uint4*>(aptr + (size_t)ip * 16);
    uint32_t raw[4], sw[4];
    if constexpr (!WI8) {
      const uint4* wp = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(Wp) + (wslot0 + (size_t)ip * 64) * 16);
      const uint4 w0 = wp[0], w1 = wp[1];
      raw[0] = w0.x; raw[1] = w0.y; raw[2] = w0.z; raw[3] = w0.w;
      sw[0] = w1.x; sw[1] = w1.y; sw[2] = w1.z; sw[3] = w1.w;
    } else {
      const uint2 q = *reinterpret_cast<const uint2*>(static_cast<const int8_t*>(Wp) + (wslot0 + (size_t)ip * 64) * 8);
      int c[8];
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        c[p] = (int)(int8_t)((q.x >> (8 * p)) & 0xff);
        c[4 + p] = (int)(int8_t)((q.y >> (8 * p)) & 0xff);
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        raw[t] = i8pair_to_bf16x2(c[2 * t], c[2 * t + 1]);
        sw[t] = (raw[t] >> 16) | (raw[t] << 16);
      }
    }
    const bf16x8_t av = __builtin_bit_cast(bf16x8_t, a);
    acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, blade_operand<0>(raw, sw), acc[0], 0, 0, 0);
    acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, blade_operand<1>(raw, sw), acc[1], 0, 0, 0);
    acc[2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, blade_operand<2>(raw, sw), acc[2], 0, 0, 0);
    acc[3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, blade_operand<3>(raw, sw), acc[3], 0, 0, 0);
    acc[4] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, blade_operand<4>(raw, sw), acc[4], 0, 0, 0);
    acc[5] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, blade_operand<5>(raw, sw), acc[5], 0, 0, 0);
    acc[6] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, blade_operand<6>(raw, sw), acc[6], 0, 0, 0);
    acc[7] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, blade_operand<7>(raw, sw), acc[7], 0, 0, 0);
  }

  const int j = jb * 32 + l32;
  if (j >= d_out) return;
  const float sc = WI8 ? wscale[(size_t)e * d_out + j] : 1.f;
  float bv[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) bv[r] = bias ? bias[((size_t)e * d_out + j) * 8 + r] : 0.f;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int row = row0 + wm * 32 + 8 * (v >> 2) + 4 * ih + (v & 3);
    if (row >= row_end) continue;
    float y[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) y[r] = (float)kOutFold(r) * acc[r][v] * sc + bv[r];
    activate_mask_order<ACT>(y);
    store_out8<OUT_DT>(Y, (size_t)row * d_out + j, y, OUT_BLADE);
  }
}

// ---------------------------------------------------------------------------
// decode-shape kernel: int8 weights, a few rows per expert
// ---------------------------------------------------------------------------
// Weight bytes, not FLOPs, bound this shape, so the work is cut for memory
// parallelism: one 256-thread workgroup per (expert, 32 output multivectors,
// K split).  Each wave takes 32 input multivectors of a 128-input chunk for
// both 16-column blocks, and every lane issues its eight 16-byte weight loads
// (input multivectors i and i + 1 of two output columns) as soon as the
// expert's row range is known: one launch keeps the whole weight stream in
// flight (2 workgroups per CU).  int8 is widened to bf16 in registers
// (exact) and v_mfma_f32_16x16x32_bf16 runs over 16-row blocks of the
// expert's rows.
//
// Here the 8x8 block L(w) is applied by permuting the A fragment instead of
// the weights: with q the weight component (mask order) at a K position,
//   y_r = kOutFold(r) * sum_q  sigma_r(q) x[q ^ r] * W'[q],
// W' the folded prepared weights (ygg_common.h), and sigma_r(q) = -1 on
// exactly one aligned pair of q (decode_neg_pair).  So one raw weight
// fragment serves all eight output blades, and the eight signed permutations
// of an A fragment (a register selection plus one XOR each) are shared by
// the two column blocks.
//
// The waves' partial sums are added in LDS in fixed wave order.  The A
// operand is either expert-grouped rows in mask order or (GATHER) the layer
// input in blade order read through the routing permutation, the e3 / e12
// exchange done in registers: no dispatch copy.  A split wider than one
// chunk walks its chunks in order.  With several K splits each split writes
// an fp32 partial plane (scale applied, bias in split 0) and the consumer
// adds the planes in split order -- deterministic either way.
constexpr int kDecWaves = 4;
constexpr int kDecCB = 2;                 // 16-column blocks per workgroup
constexpr int kDecJ = 16 * kDecCB;        // output multivectors per workgroup
constexpr int kDecRows = 16;              // rows per MFMA block
constexpr int kDecSteps = 4;              // steps of 8 input multivectors per wave and chunk
constexpr int kDecChunk = kDecWaves * kDecSteps * 8;  // 128 input multivectors
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// residual sign of the permuted-A form: the aligned pair of K positions q
// that is negated for output blade r
__host__ __device__ constexpr int decode_neg_pair(int r) {
  for (int t = 0; t < 4; ++t)
    if (kOutFold(r) * kWFold(2 * t) * mask_product_sign(2 * t, (2 * t) ^ r) < 0) return t;
  return -1;
}
constexpr bool check_decode_folding() {
  for (int r = 0; r < 8; ++r) {
    const int t = decode_neg_pair(r);
    if (t < 0) return false;
    for (int q = 0; q < 8; ++q) {
      const int sgn = kOutFold(r) * kWFold(q) * mask_product_sign(q, q ^ r);
      if (sgn != ((q / 2 == t) ? -1 : 1)) return false;
    }
  }
  return true;
}
static_assert(check_decode_folding(), "permuted-A form must leave one negative aligned pair per output blade");

// A_r[q] = sigma_r(q) a[q ^ r] from the packed fragment (raw) and its
// pair-swapped copy (sw)
template <int R>
__device__ inline bf16x8_t permuted_a(const uint32_t (&raw)[4], const uint32_t (&sw)[4]) {
  constexpr int tneg = decode_neg_pair(R);
  uint32_t d[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    d[t] = (R & 1) ? sw[t ^ (R >> 1)] : raw[t ^ (R >> 1)];
    if (t == tneg) d[t] ^= 0x80008000u;
  }
  return __builtin_bit_cast(bf16x8_t, d);
}

// bf16 components (c0 c1 | c2 c3 | c4 c5 | c6 c7) in blade order -> mask order
// (c0 c1 | c2 c4 | c3 c5 | c6 c7)
__device__ inline uint4 bf16x8_blade_to_mask(uint4 q) {
  return make_uint4(q.x, (q.y & 0xffffu) | (q.z << 16), (q.y >> 16) | (q.z & 0xffff0000u), q.w);
}

// eight int8 weight components -> eight bf16 (exact)
__device__ inline bf16x8_t i8x8_to_bf16(uint32_t lo, uint32_t hi) {
  uint32_t d[4];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const uint32_t w = t == 0 ? lo : hi;
    d[2 * t] = i8pair_to_bf16x2((int)(int8_t)(w & 0xff), (int)(int8_t)((w >> 8) & 0xff));
    d[2 * t + 1] = i8pair_to_bf16x2((int)(int8_t)((w >> 16) & 0xff), (int)(int8_t)(w >> 24));
  }
  return __builtin_bit_cast(bf16x8_t, d);
}

// one K step: A fragment a (mask order) against the weight fragments of both column blocks
__device__ inline void decode_step(f32x4_t (&acc)[kDecCB][8], const uint4 a, const bf16x8_t (&b)[kDecCB]) {
  const uint32_t raw[4] = {a.x, a.y, a.z, a.w};
  uint32_t sw[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) sw[t] = (raw[t] >> 16) | (raw[t] << 16);
#define YGG_STEP(R)                                                                      \
  {                                                                                      \
    const bf16x8_t ar = permuted_a<R>(raw, sw);                                          \
    _Pragma("unroll") for (int cb = 0; cb < kDecCB; ++cb) acc[cb][R] =                   \
        __builtin_amdgcn_mfma_f32_16x16x32_bf16(ar, b[cb], acc[cb][R], 0, 0, 0);         \
  }
  YGG_STEP(0) YGG_STEP(1) YGG_STEP(2) YGG_STEP(3) YGG_STEP(4) YGG_STEP(5) YGG_STEP(6) YGG_STEP(7)
#undef YGG_STEP
}

// Routing inside the up product (decode layers given logits, N <= kFuseMaxTokens):
// every workgroup selects the experts of all N tokens itself (the same
// select_from_logits as the routing kernels), so the layer needs no routing
// launch.  Its logits loads go out before the weight stream, which therefore
// stays in flight while it selects.  The workgroups of column block 0 also
// write the routing arrays of their expert's slots (every slot belongs to one
// expert), which the down product and the combine read.
struct DecodeRoute {
  const float* logits;
  int N, E, k;
  int32_t* topk_idx;
  float* topk_w;
  int32_t* counts;
  int32_t* offsets;
  int32_t* perm;
  int32_t* slot_pos;
};
constexpr int kFuseMaxTokens = 128;                    // 4 passes of 32 tokens
constexpr int kFuseMaxSlots = kFuseMaxTokens * kMaxTopK;
constexpr int kFusePasses = kFuseMaxTokens / (64 * kDecWaves / kSelLanes);

template <int ACT, bool GATHER, bool OUT_BLADE, int OUT_DT, bool PARTIAL, bool MULTI, int RQ = 0>
__global__ __launch_bounds__(64 * kDecWaves) void grouped_cl_decode_i8(
    const uint16_t* __restrict__ A, const int32_t* __restrict__ gather, const int8_t* __restrict__ Wq,
    const float* __restrict__ wscale, const float* __restrict__ bias, const int32_t* __restrict__ offsets, int d_in,
    int d_out, int k_split, int P_max, void* __restrict__ Y, DecodeRoute rt = DecodeRoute{}) {
  static_assert(RQ == 0 || (GATHER && !MULTI && !PARTIAL), "routing is fused into the one-chunk up product only");
  __shared__ float part[kDecWaves][kDecRows][kDecJ][9];  // +1 float of padding per multivector
  __shared__ int32_t rows_tok[RQ > 0 ? kFuseMaxTokens : 1];  // fused routing: this expert's tokens in order
  const int e = blockIdx.x, split = blockIdx.z;
  int row_beg = 0, row_end = 0;
  if constexpr (RQ == 0) {
    row_beg = offsets[e];
    row_end = offsets[e + 1];
    if (row_beg >= row_end) return;
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int jl = lane & 15, g = lane >> 4;  // output column (B) / row (A) within a block; K group
  const int col0 = blockIdx.y * kDecJ;
  const int JB = (d_out + 31) >> 5, IP = (d_in + 1) >> 1;
  const int k_lo = split * k_split, k_hi = min(d_in, k_lo + k_split);
  const int nchunks = (k_hi - k_lo + kDecChunk - 1) / kDecChunk;
  // Raw buffer loads (zero past the range): the weights of this expert's 32-column
  // block (col0 is a multiple of 32; columns past d_out hold zero padding), and x.
  const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int8_t*>(Wq) + (((size_t)e * JB + (col0 >> 5)) * IP) * 512, (short)0, (uint32_t)IP * 512,
      kBufferFlags);
  const __amdgpu_buffer_rsrc_t a_rsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(A), (short)0, 0x7fffffff, kBufferFlags);

  // weights of one chunk: step s holds input multivectors i, i + 1 (i even) of both
  // columns (16 bytes at pair i / 2, slot 2 (16 cb + jl)); steps past k_hi read zero
  uint4 wq[kDecSteps][kDecCB];
  auto load_w = [&](int kc) {
#pragma unroll
    for (int s = 0; s < kDecSteps; ++s) {
      const int i = kc + wave * (kDecSteps * 8) + 8 * s + 2 * g;
#pragma unroll
      for (int cb = 0; cb < kDecCB; ++cb) {
        const uint32_t off = i < k_hi ? (uint32_t)(i >> 1) * 512 + (uint32_t)(16 * cb + jl) * 16 : kBufferOff;
        wq[s][cb] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, off, 0, 0));
      }
    }
  };

  // epilogue operands, independent of the rows: thread tid owns outputs
  // (r0 + rl, col0 + jj) for o = tid + 256 h, rl = o / kDecJ, jj = o % kDecJ
  constexpr int kOut = kDecRows * kDecJ / (64 * kDecWaves);
  float sc[kOut], bv[kOut][8];
  // (raw buffer loads with no branch: a column past d_out, or no bias, reads zero,
  // so every path issues the same loads and the waits stay exact)
  const bool with_bias = bias != nullptr && (!PARTIAL || split == 0);
  const __amdgpu_buffer_rsrc_t s_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(wscale) + (size_t)e * d_out, (short)0, (uint32_t)d_out * 4, kBufferFlags);
  const __amdgpu_buffer_rsrc_t b_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      with_bias ? const_cast<float*>(bias) + (size_t)e * d_out * 8 : nullptr, (short)0,
      with_bias ? (uint32_t)d_out * 32 : 0u, kBufferFlags);
  auto load_epilogue = [&]() {
#pragma unroll
    for (int h = 0; h < kOut; ++h) {
      const uint32_t jo = (uint32_t)(col0 + (tid + 64 * kDecWaves * h) % kDecJ);  // past d_out: reads zero
      sc[h] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(s_rsrc, jo * 4, 0, 0));
      const float4 b0 = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(b_rsrc, jo * 32, 0, 0));
      const float4 b1 = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(b_rsrc, jo * 32 + 16, 0, 0));
      bv[h][0] = b0.x; bv[h][1] = b0.y; bv[h][2] = b0.z; bv[h][3] = b0.w;
      bv[h][4] = b1.x; bv[h][5] = b1.y; bv[h][6] = b1.z; bv[h][7] = b1.w;
    }
  };

  // one chunk of a row block: every A load goes out before the first MFMA
  auto chunk = [&](f32x4_t (&acc)[kDecCB][8], int kc, uint32_t arow_off) {
    uint4 af[kDecSteps][2];
#pragma unroll
    for (int s = 0; s < kDecSteps; ++s) {
      const int i = kc + wave * (kDecSteps * 8) + 8 * s + 2 * g;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t off = i + h < k_hi ? arow_off + (uint32_t)(i + h) * 16 : kBufferOff;
        af[s][h] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, off, 0, 0));
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < kDecSteps; ++s) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint4 a = GATHER ? bf16x8_blade_to_mask(af[s][h]) : af[s][h];
        bf16x8_t b[kDecCB];
#pragma unroll
        for (int cb = 0; cb < kDecCB; ++cb)
          b[cb] = h == 0 ? i8x8_to_bf16(wq[s][cb].x, wq[s][cb].y) : i8x8_to_bf16(wq[s][cb].z, wq[s][cb].w);
        decode_step(acc, a, b);
      }
    }
  };

  // the waves' partial sums of a row block -> LDS -> scaled, biased, stored
  auto finish = [&](f32x4_t (&acc)[kDecCB][8], int r0) {
    // lane holds columns 16 cb + jl, rows 4 g + v, all 8 output blades
#pragma unroll
    for (int cb = 0; cb < kDecCB; ++cb)
#pragma unroll
      for (int v = 0; v < 4; ++v)
#pragma unroll
        for (int r = 0; r < 8; ++r) part[wave][4 * g + v][16 * cb + jl][r] = acc[cb][r][v];
    __syncthreads();
#pragma unroll
    for (int h = 0; h < kOut; ++h) {
      const int o = tid + 64 * kDecWaves * h;
      const int rl = o / kDecJ, jj = o % kDecJ;
      const int row = r0 + rl, jo = col0 + jj;
      if (row < row_end && jo < d_out) {
        float y[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          float sum = 0.f;
#pragma unroll
          for (int w = 0; w < kDecWaves; ++w) sum += part[w][rl][jj][r];
          y[r] = (float)kOutFold(r) * sum * sc[h] + bv[h][r];
        }
        if constexpr (PARTIAL) {
          store_out8<kF32>(Y, ((size_t)split * P_max + row) * d_out + jo, y, /*blade_order=*/true);
        } else {
          activate_mask_order<ACT>(y);
          store_out8<OUT_DT>(Y, (size_t)row * d_out + jo, y, OUT_BLADE);
        }
      }
    }
    __syncthreads();
  };
  auto zero = [](f32x4_t (&acc)[kDecCB][8]) {
#pragma unroll
    for (int cb = 0; cb < kDecCB; ++cb)
#pragma unroll
      for (int r = 0; r < 8; ++r) acc[cb][r] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  };
  // lane row of the block at r0 (rows past the expert's range repeat its last
  // row and are not stored); its byte offset into x is src * d_in * 16
  auto row_src = [&](int r0) {
    int src = min(r0 + jl, row_end - 1);
    if constexpr (RQ > 0) src = rows_tok[src - row_beg];
    else if constexpr (GATHER) src = gather[src];
    return src;
  };

  if constexpr (RQ > 0) {
    // ---- fused routing: logits, then the weight stream, then the selection
    const int N = rt.N, E = rt.E, k = rt.k;
    const int j = tid & (kSelLanes - 1);
    float lg[kFusePasses][RQ];
#pragma unroll
    for (int ps = 0; ps < kFusePasses; ++ps) {
      const int t = ps * (64 * kDecWaves / kSelLanes) + (tid >> 3);
#pragma unroll
      for (int q = 0; q < RQ; ++q) {
        const int x = j + kSelLanes * q;
        lg[ps][q] = (t < N && x < E) ? rt.logits[(size_t)t * E + x] : -INFINITY;
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    load_w(k_lo);
    load_epilogue();
    __builtin_amdgcn_sched_barrier(0);
    // LDS scratch on top of part (free until the first finish())
    int32_t* s_sel = reinterpret_cast<int32_t*>(&part[0][0][0][0]);
    float* s_w = reinterpret_cast<float*>(s_sel + kFuseMaxTokens * kMaxTopK);
    int32_t* s_cnt = reinterpret_cast<int32_t*>(s_w + kFuseMaxTokens * kMaxTopK);
    int32_t* s_off = s_cnt + kMaxExperts;
    int32_t* s_wv = s_off + kMaxExperts + 1;
    if (tid < kMaxExperts) s_cnt[tid] = 0;
#pragma unroll
    for (int ps = 0; ps < kFusePasses; ++ps) {
      if (ps * (64 * kDecWaves / kSelLanes) < N) {
        const int t = ps * (64 * kDecWaves / kSelLanes) + (tid >> 3);
        int se;
        float sw;
        select_from_logits<RQ>(lg[ps], E, k, t < N, j, lane, se, sw);
        if (se >= 0) {
          s_sel[t * k + j] = se;
          s_w[t * k + j] = sw;
        }
      }
    }
    __syncthreads();
    for (int f = tid; f < N * k; f += 64 * kDecWaves) atomicAdd(&s_cnt[s_sel[f]], 1);
    // this expert's tokens in ascending order: a ballot per wave, then wave bases
    bool mine = false;
    if (tid < N)
      for (int s = 0; s < k; ++s) mine |= s_sel[tid * k + s] == e;
    const uint64_t bal = __ballot(mine);
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    if (lane == 0) s_wv[wave] = __popcll(bal);
    __syncthreads();
    if (wave == 0) {  // exclusive scan of the counts over experts
      const int c = lane < E ? s_cnt[lane] : 0;
      int incl = c;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int v = __shfl_up(incl, o);
        if (lane >= o) incl += v;
      }
      if (lane < E) s_off[lane] = incl - c;
      if (lane == E - 1) s_off[E] = incl;
    }
    if (mine) {
      int base = 0;
      for (int w = 0; w < wave; ++w) base += s_wv[w];
      rows_tok[base + __popcll(bal & lt_mask)] = tid;
    }
    __syncthreads();
    row_beg = s_off[e];
    row_end = s_off[e + 1];
    if (blockIdx.y == 0) {  // the routing arrays of this expert's slots, for the later launches
      for (int r = tid; r < row_end - row_beg; r += 64 * kDecWaves) {
        const int t = rows_tok[r];
        int s = 0;
        while (s_sel[t * k + s] != e) ++s;
        rt.topk_idx[t * k + s] = e;
        rt.topk_w[t * k + s] = s_w[t * k + s];
        rt.slot_pos[t * k + s] = row_beg + r;
        rt.perm[row_beg + r] = t;
      }
      if (tid == 0) {
        rt.counts[e] = row_end - row_beg;
        rt.offsets[e] = row_beg;
        if (e == E - 1) rt.offsets[E] = row_end;
      }
    }
    __syncthreads();  // part is overwritten from here on
    if (row_beg >= row_end) return;
    {
      f32x4_t acc[kDecCB][8];
      zero(acc);
      chunk(acc, k_lo, (uint32_t)row_src(row_beg) * d_in * 16);
      finish(acc, row_beg);
    }
    for (int r0 = row_beg + kDecRows; r0 < row_end; r0 += kDecRows) {
      f32x4_t acc[kDecCB][8];
      zero(acc);
      chunk(acc, k_lo, (uint32_t)row_src(r0) * d_in * 16);
      finish(acc, r0);
    }
  } else if constexpr (!MULTI) {
    // one chunk (the decode case): the weights stay in registers for every row
    // block, and the first block's row index is loaded ahead of them (vmcnt
    // retires in order, so its wait does not wait for the weight stream)
    const int first = row_src(row_beg);
    __builtin_amdgcn_sched_barrier(0);
    load_w(k_lo);
    load_epilogue();
    __builtin_amdgcn_sched_barrier(0);
    {
      f32x4_t acc[kDecCB][8];
      zero(acc);
      chunk(acc, k_lo, (uint32_t)first * d_in * 16);
      finish(acc, row_beg);
    }
    for (int r0 = row_beg + kDecRows; r0 < row_end; r0 += kDecRows) {
      f32x4_t acc[kDecCB][8];
      zero(acc);
      chunk(acc, k_lo, (uint32_t)row_src(r0) * d_in * 16);
      finish(acc, r0);
    }
  } else {
    load_epilogue();
    for (int r0 = row_beg; r0 < row_end; r0 += kDecRows) {
      const uint32_t off = (uint32_t)row_src(r0) * d_in * 16;
      f32x4_t acc[kDecCB][8];
      zero(acc);
      for (int c = 0; c < nchunks; ++c) {
        load_w(k_lo + c * kDecChunk);
        chunk(acc, k_lo + c * kDecChunk, off);
      }
      finish(acc, r0);
    }
  }
}

// ---------------------------------------------------------------------------
// fp32 kernel (VALU fused multiply-adds; LDS-staged tiles)
// ---------------------------------------------------------------------------
constexpr int kF32BM = 32, kF32BN = 32, kF32KI = 8;

template <int ACT, bool OUT_BLADE>
__global__ __launch_bounds__(256) void grouped_cl_f32(const float* __restrict__ A, const float* __restrict__ Wm,
                                                      const float* __restrict__ bias,
                                                      const int32_t* __restrict__ offsets, int E, int d_in,
                                                      int d_out, float* __restrict__ Y) {
  __shared__ float As[kF32BM][kF32KI * 8 + 4];
  __shared__ float Ws[kF32BN][kF32KI * 8 + 4];
  int e, row0, row_end;
  if (!find_tile(offsets, E, kF32BM, blockIdx.x, e, row0, row_end)) return;
  const int col0 = blockIdx.y * kF32BN;
  const int tid = threadIdx.x;
  const int tj = tid & 31, tm = tid >> 5;  // rows tm*4 .. tm*4+3
  float acc[4][8];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int r = 0; r < 8; ++r) acc[a][r] = 0.f;

  const int lr = tid >> 3, lm = tid & 7;  // loader: row/col lr, multivector lm of the K slice
  for (int i0 = 0; i0 < d_in; i0 += kF32KI) {
    {
      const int row = row0 + lr, i = i0 + lm;
      float4 p0 = make_float4(0, 0, 0, 0), p1 = p0;
      if (row < row_end && i < d_in) {
        const float4* s = reinterpret_cast<const float4*>(A + ((size_t)row * d_in + i) * 8);
        p0 = s[0];
        p1 = s[1];
      }
      float* d = &As[lr][lm * 8];
      d[0] = p0.x; d[1] = p0.y; d[2] = p0.z; d[3] = p0.w; d[4] = p1.x; d[5] = p1.y; d[6] = p1.z; d[7] = p1.w;
      const int j = col0 + lr;
      float4 q0 = make_float4(0, 0, 0, 0), q1 = q0;
      if (j < d_out && i < d_in) {
        const float4* s = reinterpret_cast<const float4*>(Wm + (((size_t)e * d_out + j) * d_in + i) * 8);
        q0 = s[0];
        q1 = s[1];
      }
      float* w = &Ws[lr][lm * 8];
      w[0] = q0.x; w[1] = q0.y; w[2] = q0.z; w[3] = q0.w; w[4] = q1.x; w[5] = q1.y; w[6] = q1.z; w[7] = q1.w;
    }
    __syncthreads();
#pragma unroll 2
    for (int mv = 0; mv < kF32KI; ++mv) {
      float w[8];
#pragma unroll
      for (int p = 0; p < 8; ++p) w[p] = Ws[tj][mv * 8 + p];
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        float x[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) x[q] = As[tm * 4 + a][mv * 8 + q];
#pragma unroll
        for (int r = 0; r < 8; ++r)
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            const float s = (float)folded_sign(r, q ^ r);
            acc[a][r] = fmaf(s * w[q ^ r], x[q], acc[a][r]);
          }
      }
    }
    __syncthreads();
  }
  const int j = col0 + tj;
  if (j >= d_out) return;
  float bv[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) bv[r] = bias ? bias[((size_t)e * d_out + j) * 8 + r] : 0.f;
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const int row = row0 + tm * 4 + a;
    if (row >= row_end) continue;
    float y[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) y[r] = (float)kOutFold(r) * acc[a][r] + bv[r];
    activate_mask_order<ACT>(y);
    store_out8<kF32>(Y, (size_t)row * d_out + j, y, OUT_BLADE);
  }
}

}  // namespace ygg

using namespace ygg;

YGG_API size_t ygg_prepared_weight_bytes(int E, int d_out, int d_in, int format) {
  const size_t JB = (size_t)(d_out + 31) / 32, IP = (size_t)(d_in + 1) / 2;
  switch (format) {
    case kWF32: return (size_t)E * d_out * d_in * 8 * 4;
    case kWBF16: return (size_t)E * JB * IP * 64 * 16 * 2;
    case kWI8: return (size_t)E * JB * IP * 64 * 8;
    case kWPauli: return (d_in % 2) ? 0 : (size_t)E * d_out * d_in * 8 * 2;
    case kWPauliF32: return (size_t)E * d_out * d_in * 16 * 4;
    case kWPauliI8: return decode_pauli_weight_bytes(E, d_out, d_in);
    default: return 0;
  }
}

YGG_API int ygg_prepare_weights(const float* W, int E, int d_out, int d_in, int format, void* out, float* scales,
                                hipStream_t stream) {
  YGG_CHECK_ARG(format >= kWF32 && format <= kWPauliI8, "ygg_prepare_weights: format %d", format);
  YGG_CHECK_ARG(E >= 1 && d_out >= 1 && d_in >= 1, "ygg_prepare_weights: bad sizes E=%d d_out=%d d_in=%d", E, d_out,
                d_in);
  YGG_CHECK_ARG(W && out, "ygg_prepare_weights: null pointer");
  if (format == kWPauli) return pauli_prepare_weights(W, E, d_out, d_in, out, stream);
  if (format == kWPauliF32) return pauli_f32_prepare_weights(W, E, d_out, d_in, out, stream);
  if (format == kWPauliI8) return decode_pauli_prepare_weights(W, E, d_out, d_in, out, scales, stream);
  YGG_CHECK_ARG(format != kWI8 || scales, "ygg_prepare_weights: int8 format needs a scales buffer [E, d_out]");
  if (format == kWI8) {
    quant_scale_kernel<<<E * d_out, 256, 0, stream>>>(W, d_in, scales);
    if (check_launch("quant_scale")) return -1;
  }
  const size_t JB = (size_t)(d_out + 31) / 32, IP = (size_t)(d_in + 1) / 2;
  const size_t total = (format == kWF32) ? (size_t)E * d_out * d_in : (size_t)E * JB * IP * 64;
  prep_weights_kernel<<<(unsigned)((total + 255) / 256), 256, 0, stream>>>(W, E, d_out, d_in, format, scales, out);
  return check_launch("prep_weights");
}

YGG_API int ygg_prepare_bias(const float* b, int E, int d_out, float* out, hipStream_t stream) {
  YGG_CHECK_ARG(b && out && E >= 1 && d_out >= 1, "ygg_prepare_bias: bad arguments");
  const size_t n = (size_t)E * d_out;
  prep_bias_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(b, n, out);
  return check_launch("prep_bias");
}

template <int ACT>
static void launch_mfma(dim3 grid, hipStream_t st, bool out_blade, bool wi8, int out_dt, const uint16_t* A,
                        const void* Wp, const float* sc, const float* bias, const int32_t* off, int E, int d_in,
                        int d_out, void* Y) {
#define YGG_L(OB, WI, OD) grouped_cl_mfma<ACT, OB, WI, OD><<<grid, 256, 0, st>>>(A, Wp, sc, bias, off, E, d_in, d_out, Y)
  if (out_dt == kBF16) {
    if (out_blade) { if (wi8) YGG_L(true, true, kBF16); else YGG_L(true, false, kBF16); }
    else { if (wi8) YGG_L(false, true, kBF16); else YGG_L(false, false, kBF16); }
  } else {
    if (out_blade) { if (wi8) YGG_L(true, true, kF32); else YGG_L(true, false, kF32); }
    else { if (wi8) YGG_L(false, true, kF32); else YGG_L(false, false, kF32); }
  }
#undef YGG_L
}

template <int ACT, bool MULTI>
static void launch_decode_m(dim3 grid, hipStream_t st, bool out_blade, int out_dt, const uint16_t* A,
                            const int32_t* gather, const int8_t* W, const float* sc, const float* bias,
                            const int32_t* off, int d_in, int d_out, int k_split, int P_max, void* Y) {
#define YGG_D(G, OB, OD)                                                                                  \
  grouped_cl_decode_i8<ACT, G, OB, OD, false, MULTI><<<grid, 64 * kDecWaves, 0, st>>>(A, gather, W, sc, bias, \
                                                                                     off, d_in, d_out,     \
                                                                                     k_split, P_max, Y)
  if (gather) YGG_D(true, false, kBF16);  // the layer's up product: blade-order input, mask-order bf16 h
  else if (out_dt == kBF16) { if (out_blade) YGG_D(false, true, kBF16); else YGG_D(false, false, kBF16); }
  else { if (out_blade) YGG_D(false, true, kF32); else YGG_D(false, false, kF32); }
#undef YGG_D
}

// the decode kernel addresses x with 32-bit byte offsets
static bool decode_offsets_fit(int rows, int d_in) { return (long long)rows * d_in * 16 < 0x7fffffffLL; }

// one 128-input chunk per workgroup (the decode case) or a walk over several
template <int ACT>
static void launch_decode(dim3 grid, hipStream_t st, bool out_blade, int out_dt, const uint16_t* A,
                          const int32_t* gather, const int8_t* W, const float* sc, const float* bias,
                          const int32_t* off, int d_in, int d_out, int k_split, int P_max, void* Y) {
  if (k_split <= kDecChunk)
    launch_decode_m<ACT, false>(grid, st, out_blade, out_dt, A, gather, W, sc, bias, off, d_in, d_out, k_split, P_max, Y);
  else
    launch_decode_m<ACT, true>(grid, st, out_blade, out_dt, A, gather, W, sc, bias, off, d_in, d_out, k_split, P_max, Y);
}

static int decode_dispatch(int act, dim3 grid, hipStream_t st, bool out_blade, int out_dt, const uint16_t* A,
                           const int32_t* gather, const int8_t* W, const float* sc, const float* bias,
                           const int32_t* off, int d_in, int d_out, int k_split, int P_max, void* Y) {
  switch (act) {
    case kActNone: launch_decode<kActNone>(grid, st, out_blade, out_dt, A, gather, W, sc, bias, off, d_in, d_out, k_split, P_max, Y); break;
    case kActGelu: launch_decode<kActGelu>(grid, st, out_blade, out_dt, A, gather, W, sc, bias, off, d_in, d_out, k_split, P_max, Y); break;
    case kActRelu: launch_decode<kActRelu>(grid, st, out_blade, out_dt, A, gather, W, sc, bias, off, d_in, d_out, k_split, P_max, Y); break;
    default: launch_decode<kActSigmoid>(grid, st, out_blade, out_dt, A, gather, W, sc, bias, off, d_in, d_out, k_split, P_max, Y); break;
  }
  return check_launch("grouped_cl_decode_i8");
}

template <int ACT>
static void launch_f32(dim3 grid, hipStream_t st, bool out_blade, const float* A, const float* W, const float* bias,
                       const int32_t* off, int E, int d_in, int d_out, float* Y) {
  if (out_blade) grouped_cl_f32<ACT, true><<<grid, 256, 0, st>>>(A, W, bias, off, E, d_in, d_out, Y);
  else grouped_cl_f32<ACT, false><<<grid, 256, 0, st>>>(A, W, bias, off, E, d_in, d_out, Y);
}

// x: [P, d_in, 8] in mask order (dtype f32 for format F32, bf16 otherwise).
// y: [P, d_out, 8] (f32 for format F32; y_dtype for the others), mask order
//    or blade order.  P_max bounds the rows (offsets[E] <= P_max).
YGG_API int ygg_grouped_clifford_linear(const void* x, int P_max, const void* Wp, int format, const float* scales,
                                        const float* bias, const int32_t* offsets, int E, int d_in, int d_out,
                                        int act, void* y, int y_dtype, int y_blade_order, hipStream_t stream) {
  YGG_CHECK_ARG(format == kWF32 || format == kWBF16 || format == kWI8, "grouped_clifford_linear: format %d", format);
  YGG_CHECK_ARG(act >= kActNone && act <= kActSigmoid, "grouped_clifford_linear: activation %d", act);
  YGG_CHECK_ARG(E >= 1 && d_in >= 1 && d_out >= 1 && P_max >= 0, "grouped_clifford_linear: bad sizes");
  YGG_CHECK_ARG(format != kWI8 || scales, "grouped_clifford_linear: int8 weights need scales");
  YGG_CHECK_ARG(format == kWF32 ? y_dtype == kF32 : (y_dtype == kF32 || y_dtype == kBF16),
                "grouped_clifford_linear: output dtype %d invalid for format %d", y_dtype, format);
  if (P_max == 0) return 0;
  YGG_CHECK_ARG(x && Wp && offsets && y, "grouped_clifford_linear: null pointer");
  const bool ob = y_blade_order != 0;
  if (format == kWF32) {
    dim3 grid((P_max + kF32BM - 1) / kF32BM + E, (d_out + kF32BN - 1) / kF32BN);
    const float* A = static_cast<const float*>(x);
    const float* W = static_cast<const float*>(Wp);
    float* Y = static_cast<float*>(y);
    switch (act) {
      case kActNone: launch_f32<kActNone>(grid, stream, ob, A, W, bias, offsets, E, d_in, d_out, Y); break;
      case kActGelu: launch_f32<kActGelu>(grid, stream, ob, A, W, bias, offsets, E, d_in, d_out, Y); break;
      case kActRelu: launch_f32<kActRelu>(grid, stream, ob, A, W, bias, offsets, E, d_in, d_out, Y); break;
      default: launch_f32<kActSigmoid>(grid, stream, ob, A, W, bias, offsets, E, d_in, d_out, Y); break;
    }
    return check_launch("grouped_cl_f32");
  }
  const uint16_t* A = static_cast<const uint16_t*>(x);
  const bool wi8 = format == kWI8;
  // decode shape (at most 16 rows per expert on average): weight-streaming kernel, one K split
  if (decode_shape(P_max, E, format) && decode_offsets_fit(P_max, d_in)) {
    const int k_split = decode_splits(d_in) * kDecChunk;
    return decode_dispatch(act, dim3(E, (d_out + kDecJ - 1) / kDecJ, 1), stream, ob, y_dtype, A, nullptr,
                           static_cast<const int8_t*>(Wp), scales, bias, offsets, d_in, d_out, k_split, P_max, y);
  }
  dim3 grid((P_max + kMfmaBM - 1) / kMfmaBM + E, (d_out + kMfmaBN - 1) / kMfmaBN);
  switch (act) {
    case kActNone: launch_mfma<kActNone>(grid, stream, ob, wi8, y_dtype, A, Wp, scales, bias, offsets, E, d_in, d_out, y); break;
    case kActGelu: launch_mfma<kActGelu>(grid, stream, ob, wi8, y_dtype, A, Wp, scales, bias, offsets, E, d_in, d_out, y); break;
    case kActRelu: launch_mfma<kActRelu>(grid, stream, ob, wi8, y_dtype, A, Wp, scales, bias, offsets, E, d_in, d_out, y); break;
    default: launch_mfma<kActSigmoid>(grid, stream, ob, wi8, y_dtype, A, Wp, scales, bias, offsets, E, d_in, d_out, y); break;
  }
  return check_launch("grouped_cl_mfma");
}

// Decode-shape int8 products inside ygg_moe_forward.  decode_linear_gather:
// the up product on the layer input (blade order, rows gathered through the
// routing permutation), one K split, output mask-order bf16.
// decode_linear_partial: the contraction cut into decode_splits() splits of
// one chunk; y_planes (splits, P_max, d_out, 8) fp32 blade order, to be summed
// in split order (no activation).
int ygg::decode_splits(int d_in) { return (d_in + kDecChunk - 1) / kDecChunk; }
bool ygg::decode_shape(int P_max, int E, int format) { return format == kWI8 && P_max <= kDecRows * E; }

int ygg::decode_linear_gather(const uint16_t* x, const int32_t* perm, int P_max, const int8_t* Wq,
                              const float* scales, const float* bias, const int32_t* offsets, int E, int d_in,
                              int d_out, int act, uint16_t* h, hipStream_t stream) {
  if (P_max == 0) return 0;
  YGG_CHECK_ARG(decode_offsets_fit(P_max, d_in), "decode up product: %d rows x %d inputs too large", P_max, d_in);
  return decode_dispatch(act, dim3(E, (d_out + kDecJ - 1) / kDecJ, 1), stream, false, kBF16, x, perm, Wq, scales,
                         bias, offsets, d_in, d_out, decode_splits(d_in) * kDecChunk, P_max, h);
}

bool ygg::decode_route_fusable(int N, int E, int k, int d_in) {
  return N >= 1 && N <= kFuseMaxTokens && N * k <= kFuseMaxSlots && E >= 1 && E <= kMaxExperts && k >= 1 &&
         k <= kMaxTopK && k <= E && d_in <= kDecChunk;
}

template <int ACT>
static void launch_routed(dim3 grid, hipStream_t st, int Q, const uint16_t* x, const int8_t* W, const float* sc,
                          const float* bias, int d_in, int d_out, int P_max, uint16_t* h, const DecodeRoute& rt) {
  if (Q <= 4)
    grouped_cl_decode_i8<ACT, true, false, kBF16, false, false, 4><<<grid, 64 * kDecWaves, 0, st>>>(
        x, nullptr, W, sc, bias, nullptr, d_in, d_out, kDecChunk, P_max, h, rt);
  else
    grouped_cl_decode_i8<ACT, true, false, kBF16, false, false, 8><<<grid, 64 * kDecWaves, 0, st>>>(
        x, nullptr, W, sc, bias, nullptr, d_in, d_out, kDecChunk, P_max, h, rt);
}

int ygg::decode_linear_gather_routed(const uint16_t* x, const float* logits, int N, int E, int k, int32_t* topk_idx,
                                     float* topk_w, int32_t* counts, int32_t* offsets, int32_t* perm,
                                     int32_t* slot_pos, const int8_t* Wq, const float* scales, const float* bias,
                                     int d_in, int d_out, int act, uint16_t* h, hipStream_t stream) {
  YGG_CHECK_ARG(decode_route_fusable(N, E, k, d_in), "decode routed up product: N=%d E=%d k=%d d_in=%d", N, E, k,
                d_in);
  const int P_max = N * k;
  YGG_CHECK_ARG(decode_offsets_fit(P_max, d_in), "decode up product: %d rows x %d inputs too large", P_max, d_in);
  const DecodeRoute rt{logits, N, E, k, topk_idx, topk_w, counts, offsets, perm, slot_pos};
  const dim3 grid(E, (d_out + kDecJ - 1) / kDecJ, 1);
  const int Q = (E + kSelLanes - 1) / kSelLanes;
  switch (act) {
    case kActNone: launch_routed<kActNone>(grid, stream, Q, x, Wq, scales, bias, d_in, d_out, P_max, h, rt); break;
    case kActGelu: launch_routed<kActGelu>(grid, stream, Q, x, Wq, scales, bias, d_in, d_out, P_max, h, rt); break;
    case kActRelu: launch_routed<kActRelu>(grid, stream, Q, x, Wq, scales, bias, d_in, d_out, P_max, h, rt); break;
    default: launch_routed<kActSigmoid>(grid, stream, Q, x, Wq, scales, bias, d_in, d_out, P_max, h, rt); break;
  }
  return check_launch("grouped_cl_decode_i8 (routed)");
}

int ygg::decode_linear_partial(const uint16_t* x, int P_max, const int8_t* Wq, const float* scales, const float* bias,
                               const int32_t* offsets, int E, int d_in, int d_out, float* y_planes,
                               hipStream_t stream) {
  if (P_max == 0) return 0;
  YGG_CHECK_ARG(decode_offsets_fit(P_max, d_in), "decode down product: %d rows x %d inputs too large", P_max, d_in);
  dim3 grid(E, (d_out + kDecJ - 1) / kDecJ, decode_splits(d_in));
  grouped_cl_decode_i8<kActNone, false, true, kF32, true, false><<<grid, 64 * kDecWaves, 0, stream>>>(
      x, nullptr, Wq, scales, bias, offsets, d_in, d_out, kDecChunk, P_max, y_planes);
  return check_launch("grouped_cl_decode_i8 (K split)");
}


