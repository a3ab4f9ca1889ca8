// backward.hip -- the expert-FFN backward pass of the MoE layer, fp32.
//
// The reference's CliffordLinear.backward (holograph/layers/clifford_linear.py:125-163)
// is two geometric matmuls with reversed operands: for y_j = sum_i W_ji x_i + b_j,
//   dx_i = sum_j ~W_ji dy_j        (the forward product with the adjoint weights
//                                   Wadj_ij = ~W_ji: the forward kernels run it)
//   dW_ji = sum_rows dy_j ~x_i     (a reduction over the rows of one expert)
//   db_j = sum_rows dy_j
// With the Pauli map (the algebra isomorphism Cl(3,0) -> 2x2 complex matrices
// of pauli_common.h), reversion is the conjugate transpose, so dW_ji is the
// complex matrix sum  sum_r M(dy_rj) M(x_ri)^H: 32 real multiply-adds per row
// and (j, i) pair instead of the 64 of the blade form.
//
// The activations' backward (holograph/layers/activations.py:135-287), the
// combine's (the routing weight times the output gradient, and <dout, y> for
// the routing weights) and the dispatch's (a sum of a token's rows) are
// elementwise kernels here.  The reference has no MoE backward
// (hlm_block.py:202-206); ygg_moe_backward composes these pieces for the layer.

#include <hip/hip_runtime.h>

#include <algorithm>

#include "pauli_common.h"
#include "ygg_common.h"

namespace ygg {
namespace {

__host__ __device__ constexpr float rev_sign(int c) { return c >= 4 ? -1.f : 1.f; }  // grades 2, 3 flip

// Wadj[e, i, j] = ~W[e, j, i]; one thread per output multivector.
__global__ __launch_bounds__(256) void adjoint_kernel(const float* __restrict__ W, int E, int d_out, int d_in,
                                                      float* __restrict__ Wadj) {
  const size_t n = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (n >= (size_t)E * d_out * d_in) return;
  const int j = (int)(n % d_out);
  const int i = (int)((n / d_out) % d_in);
  const int e = (int)(n / ((size_t)d_out * d_in));
  const float* src = W + (((size_t)e * d_out + j) * d_in + i) * 8;
#pragma unroll
  for (int c = 0; c < 8; ++c) Wadj[n * 8 + c] = rev_sign(c) * src[c];
}

// ---- activation backward -----------------------------------------------------
__device__ inline float gelu_f(float v) { return 0.5f * v * (1.0f + tanhf(0.7978845608028654f * (v + 0.044715f * v * v * v))); }
__device__ inline float gelu_d(float v) {
  const float c = 0.7978845608028654f;
  const float t = tanhf(c * (v + 0.044715f * v * v * v));
  return 0.5f * (1.0f + t) + 0.5f * v * (1.0f - t * t) * (c * (1.0f + 3.0f * 0.044715f * v * v));
}
__device__ inline float sigm_f(float v) { return v >= 0.f ? 1.0f / (1.0f + expf(-v)) : expf(v) / (1.0f + expf(v)); }
__device__ inline float sigm_d(float v) {
  const float s = sigm_f(v);
  return s * (1.0f - s);
}

// _magnitude_gate_backward (activations.py:150-178) on the 3 components at c
template <int ACT>
__device__ inline void gate_backward(const float* c, const float* g, float* out) {
  const float mag = sqrtf(c[0] * c[0] + c[1] * c[1] + c[2] * c[2] + 1e-12f);
  const float dir[3] = {c[0] / mag, c[1] / mag, c[2] / mag};
  const float dot = dir[0] * g[0] + dir[1] * g[1] + dir[2] * g[2];
  float gated, deriv;
  if constexpr (ACT == kActGelu) {
    gated = gelu_f(mag);
    deriv = gelu_d(mag);
  } else {
    gated = sigm_f(mag);
    deriv = sigm_d(mag);
  }
  const float a = gated / mag, b = (deriv - gated / mag) * dot;
#pragma unroll
  for (int q = 0; q < 3; ++q) out[q] = a * g[q] + b * dir[q];
}

// out may alias g (each thread reads its multivector before writing it)
template <int ACT>
__global__ __launch_bounds__(256) void act_backward_kernel(const float* __restrict__ h, const float* g, size_t n_mv,
                                                           float* out, float* __restrict__ out_pauli) {
  const size_t n = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (n >= n_mv) return;
  float x[8], gr[8], o[8];
  const float4* hp = reinterpret_cast<const float4*>(h + n * 8);
  const float4* gp = reinterpret_cast<const float4*>(g + n * 8);
  const float4 h0 = hp[0], h1 = hp[1], g0 = gp[0], g1 = gp[1];
  x[0] = h0.x; x[1] = h0.y; x[2] = h0.z; x[3] = h0.w; x[4] = h1.x; x[5] = h1.y; x[6] = h1.z; x[7] = h1.w;
  gr[0] = g0.x; gr[1] = g0.y; gr[2] = g0.z; gr[3] = g0.w; gr[4] = g1.x; gr[5] = g1.y; gr[6] = g1.z; gr[7] = g1.w;
  if constexpr (ACT == kActNone) {
#pragma unroll
    for (int c = 0; c < 8; ++c) o[c] = gr[c];
  } else if constexpr (ACT == kActRelu) {
    // zero thresholds: grade 0 passes where positive, grades 1 and 2 (|c| >= 1e-6
    // > 0) pass through, grade 3 where non-zero
    o[0] = x[0] > 0.f ? gr[0] : 0.f;
#pragma unroll
    for (int c = 1; c < 7; ++c) o[c] = gr[c];
    o[7] = x[7] != 0.f ? gr[7] : 0.f;
  } else {
    o[0] = gr[0] * (ACT == kActGelu ? gelu_d(x[0]) : sigm_d(x[0]));
    gate_backward<ACT>(x + 1, gr + 1, o + 1);
    gate_backward<ACT>(x + 4, gr + 4, o + 4);
    const float t = tanhf(x[7]);
    o[7] = gr[7] * (1.0f - t * t);
  }
  if (out != nullptr) {  // may be g itself
    float4* op = reinterpret_cast<float4*>(out + n * 8);
    op[0] = make_float4(o[0], o[1], o[2], o[3]);
    op[1] = make_float4(o[4], o[5], o[6], o[7]);
  }
  if (out_pauli != nullptr) store_pauli_f32(out_pauli + n * 8, o);
}

// The forward activation of blade-order rows (the same activate_blade the fused
// epilogues apply), for the backward's recompute of h from h before the activation.
template <int ACT>
__global__ __launch_bounds__(256) void act_forward_kernel(const float* __restrict__ h, size_t n_mv,
                                                          float* __restrict__ out, float* __restrict__ out_pauli) {
  const size_t n = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (n >= n_mv) return;
  const float4* hp = reinterpret_cast<const float4*>(h + n * 8);
  const float4 h0 = hp[0], h1 = hp[1];
  float y[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
  activate_blade<ACT>(y);
  if (out != nullptr) {
    float4* op = reinterpret_cast<float4*>(out + n * 8);
    op[0] = make_float4(y[0], y[1], y[2], y[3]);
    op[1] = make_float4(y[4], y[5], y[6], y[7]);
  }
  if (out_pauli != nullptr) store_pauli_f32(out_pauli + n * 8, y);
}

// ---- combine backward: dy[slot] = w dout_t; dw[t, s] = <dout_t, y[slot]> ----------
// One wave per token, a multivector per lane; dy goes out in blade order and/or as
// fp32 Pauli rows (whichever is not NULL).
__global__ __launch_bounds__(256) void combine_backward_kernel(const float* __restrict__ dout,
                                                               const float* __restrict__ y_sorted, int N, int k,
                                                               int d, const float* __restrict__ topk_w,
                                                               const int32_t* __restrict__ slot_pos,
                                                               float* __restrict__ dy_sorted,
                                                               float* __restrict__ dy_pauli,
                                                               float* __restrict__ dtopk_w) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= N) return;
  const float* go = dout + (size_t)t * d * 8;
  for (int s = 0; s < k; ++s) {
    const size_t row = (size_t)slot_pos[(size_t)t * k + s];
    const float w = topk_w[(size_t)t * k + s];
    float acc = 0.f;
    for (int i = lane; i < d; i += 64) {
      const float4* gp = reinterpret_cast<const float4*>(go + (size_t)i * 8);
      const float4 g0 = gp[0], g1 = gp[1];
      const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
      float o[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) o[c] = w * gv[c];
      const size_t mv = row * d + i;
      if (dy_sorted) {
        float4* q = reinterpret_cast<float4*>(dy_sorted + mv * 8);
        q[0] = make_float4(o[0], o[1], o[2], o[3]);
        q[1] = make_float4(o[4], o[5], o[6], o[7]);
      }
      if (dy_pauli) store_pauli_f32(dy_pauli + mv * 8, o);
      if (y_sorted) {
        const float4* yp = reinterpret_cast<const float4*>(y_sorted + mv * 8);
        const float4 y0 = yp[0], y1 = yp[1];
        acc += gv[0] * y0.x + gv[1] * y0.y + gv[2] * y0.z + gv[3] * y0.w + gv[4] * y1.x + gv[5] * y1.y +
               gv[6] * y1.z + gv[7] * y1.w;
      }
    }
    if (dtopk_w) {
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
      if (lane == 0) dtopk_w[(size_t)t * k + s] = acc;
    }
  }
}

// ---- dispatch backward: dx_t = (dout_t) + sum_s dxs[slot_pos[t, s]] ---------------
__global__ __launch_bounds__(256) void dispatch_backward_kernel(const float* __restrict__ dxs, int N, int k, int d,
                                                                const int32_t* __restrict__ slot_pos,
                                                                const float* __restrict__ residual_grad,
                                                                float* __restrict__ dx) {
  const size_t n = (size_t)blockIdx.x * 256 + threadIdx.x;  // (token, component)
  if (n >= (size_t)N * d * 8) return;
  const size_t t = n / ((size_t)d * 8), u = n % ((size_t)d * 8);
  float acc = residual_grad ? residual_grad[n] : 0.f;
  for (int s = 0; s < k; ++s) acc += dxs[(size_t)slot_pos[t * k + s] * d * 8 + u];
  dx[n] = acc;
}

// ---- weight gradient: dW[e, j, i] = sum_r dy[r, j] ~a[src(r), i] --------------------
// Workgroup: a 32 (j) x 32 (i) tile of one expert; thread (tj, ti) accumulates
// the 2 x 2 pairs (tj + 16 p, ti + 16 q) as 2x2 complex matrices.  The expert's
// rows are staged 8 at a time in LDS in Pauli coordinates.
constexpr int kWgRows = 8;
constexpr int kWgT = 32;

__global__ __launch_bounds__(256) void weight_grad_kernel(const float* __restrict__ dy, const float* __restrict__ a,
                                                          const int32_t* __restrict__ gather,
                                                          const int32_t* __restrict__ offsets, int d_in, int d_out,
                                                          float* __restrict__ dW, float* __restrict__ db) {
  __shared__ float4 sdy[kWgRows][kWgT][2];  // M(dy) as (M00, M10), (M01, M11): re, im each
  __shared__ float4 sa[kWgRows][kWgT][2];
  const int e = blockIdx.z;
  const int j0 = blockIdx.x * kWgT, i0 = blockIdx.y * kWgT;
  const int tid = threadIdx.x, tj = tid & 15, ti = tid >> 4;
  const int row_beg = offsets[e], row_end = offsets[e + 1];
  // C[p][q] = sum M(dy_j) M(a_i)^H, entries (re, im) of C00, C01, C10, C11
  float acc[2][2][8];
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int c = 0; c < 8; ++c) acc[p][q][c] = 0.f;

  // staging: thread tid loads multivector (row tid / 32, column tid % 32) of each operand;
  // the workgroups of i-tile 0 also sum the staged dy rows for db (blade order)
  const int sr = tid >> 5, sc = tid & 31;
  const bool bias_tile = db != nullptr && blockIdx.y == 0;
  float bsum[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int r0 = row_beg; r0 < row_end; r0 += kWgRows) {
    {
      const int r = r0 + sr;
      float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, z[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      if (r < row_end && j0 + sc < d_out) {
        const float4* p = reinterpret_cast<const float4*>(dy + ((size_t)r * d_out + j0 + sc) * 8);
        const float4 u = p[0], v = p[1];
        x[0] = u.x; x[1] = u.y; x[2] = u.z; x[3] = u.w; x[4] = v.x; x[5] = v.y; x[6] = v.z; x[7] = v.w;
      }
      if (r < row_end && i0 + sc < d_in) {
        const size_t src = gather ? (size_t)gather[r] : (size_t)r;
        const float4* p = reinterpret_cast<const float4*>(a + (src * d_in + i0 + sc) * 8);
        const float4 u = p[0], v = p[1];
        z[0] = u.x; z[1] = u.y; z[2] = u.z; z[3] = u.w; z[4] = v.x; z[5] = v.y; z[6] = v.z; z[7] = v.w;
      }
      if (bias_tile)
#pragma unroll
        for (int c = 0; c < 8; ++c) bsum[c] += x[c];
      float c0[4], c1[4];
      blade_to_pauli(x, c0, c1);
      sdy[sr][sc][0] = make_float4(c0[0], c0[1], c0[2], c0[3]);
      sdy[sr][sc][1] = make_float4(c1[0], c1[1], c1[2], c1[3]);
      blade_to_pauli(z, c0, c1);
      sa[sr][sc][0] = make_float4(c0[0], c0[1], c0[2], c0[3]);
      sa[sr][sc][1] = make_float4(c1[0], c1[1], c1[2], c1[3]);
    }
    __syncthreads();
    const int nr = min(kWgRows, row_end - r0);
    for (int rr = 0; rr < nr; ++rr) {
      float4 D[2][2], A[2][2];
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        D[p][0] = sdy[rr][tj + 16 * p][0];
        D[p][1] = sdy[rr][tj + 16 * p][1];
        A[p][0] = sa[rr][ti + 16 * p][0];
        A[p][1] = sa[rr][ti + 16 * p][1];
      }
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          // column c of M: D[p][c] = (M0c re, M0c im, M1c re, M1c im)
          // C[a][b] += sum_c D[a][c] conj(A[b][c])
#pragma unroll
          for (int cc = 0; cc < 2; ++cc) {
            const float4 dd = D[p][cc], aa = A[q][cc];
            // rows a = 0, 1 of D column cc: (dd.x, dd.y), (dd.z, dd.w); rows b of A: (aa.x, aa.y), (aa.z, aa.w)
            // C00 += D0c conj(A0c), C01 += D0c conj(A1c), C10 += D1c conj(A0c), C11 += D1c conj(A1c)
            acc[p][q][0] += dd.x * aa.x + dd.y * aa.y;
            acc[p][q][1] += dd.y * aa.x - dd.x * aa.y;
            acc[p][q][2] += dd.x * aa.z + dd.y * aa.w;
            acc[p][q][3] += dd.y * aa.z - dd.x * aa.w;
            acc[p][q][4] += dd.z * aa.x + dd.w * aa.y;
            acc[p][q][5] += dd.w * aa.x - dd.z * aa.y;
            acc[p][q][6] += dd.z * aa.z + dd.w * aa.w;
            acc[p][q][7] += dd.w * aa.z - dd.z * aa.w;
          }
        }
    }
    __syncthreads();
  }
  if (bias_tile) {  // the 8 staging rows' partial sums, added in row order
    float* red = reinterpret_cast<float*>(&sdy[0][0][0]);  // free after the last chunk's barrier
#pragma unroll
    for (int c = 0; c < 8; ++c) red[(sr * kWgT + sc) * 8 + c] = bsum[c];
    __syncthreads();
    if (sr == 0 && j0 + sc < d_out) {
      float o[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        float v = 0.f;
        for (int q = 0; q < kWgRows; ++q) v += red[(q * kWgT + sc) * 8 + c];
        o[c] = v;
      }
      float4* dst = reinterpret_cast<float4*>(db + ((size_t)e * d_out + j0 + sc) * 8);
      dst[0] = make_float4(o[0], o[1], o[2], o[3]);
      dst[1] = make_float4(o[4], o[5], o[6], o[7]);
    }
  }
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int j = j0 + tj + 16 * p, i = i0 + ti + 16 * q;
      if (j >= d_out || i >= d_in) continue;
      const float* C = acc[p][q];
      float o[8];
      pauli_to_blade(C[0], C[1], C[2], C[3], C[4], C[5], C[6], C[7], o);
      float4* dst = reinterpret_cast<float4*>(dW + (((size_t)e * d_out + j) * d_in + i) * 8);
      dst[0] = make_float4(0.5f * o[0], 0.5f * o[1], 0.5f * o[2], 0.5f * o[3]);
      dst[1] = make_float4(0.5f * o[4], 0.5f * o[5], 0.5f * o[6], 0.5f * o[7]);
    }
}

// ---------------------------------------------------------------------------
// The same weight gradient on the fp32 MFMA units, from Pauli rows (the fp32
// Pauli-row layout of pauli_f32.hip: [b][re, im][c] per multivector).
//
// C_ji[a][c] = sum_{r, b} D_rj[a][b] conj(A_ri[c][b]) with D = M(dy), A = M(x).
// v_mfma_f32_32x32x2_f32 contracts K = 2 lanes, taken as (re, im) of one
// (row, b) term: with the D entry's (re, im) as the A operand and the x entry's
// (re, im) as the B operand the sum is Re(D conj(A)); with (-im, re) as the B
// operand it is Im(D conj(A)).  A wave owns 32 j x 32 i, eight 32 x 32
// accumulators ((a, c) x (re, im)), 16 MFMAs per row.
//
// The rows of one expert are cut into chunks of kWgmChunk rows; every
// (chunk, 64 x 64 tile) is one workgroup, which writes its Pauli sums to a
// partial plane of its chunk.  The reduction adds an expert's chunks in chunk
// order, so the result does not depend on scheduling.  The workgroups of the
// first i tile also sum the D rows of their chunk for the bias gradient.
constexpr int kWgmChunk = 384;  // rows per chunk (measured best of 128-2048 at the C3 shape)
constexpr int kWgmTile = 64;     // j and i per workgroup (2 x 2 waves of 32)
constexpr int kWgmU = 2;         // rows per register-buffered block

__device__ inline bool wgm_find_chunk(const int32_t* __restrict__ offsets, int E, int chunk, int& e, int& r0,
                                      int& r1) {
  int acc = 0, beg = offsets[0];
  for (int x = 0; x < E; ++x) {
    const int end = offsets[x + 1];
    const int n = (end - beg + kWgmChunk - 1) / kWgmChunk;
    if (chunk < acc + n) {
      e = x;
      r0 = beg + (chunk - acc) * kWgmChunk;
      r1 = min(end, r0 + kWgmChunk);
      return true;
    }
    acc += n;
    beg = end;
  }
  return false;
}

// grid (chunks bound, ceil(d_out / 64), ceil(d_in / 64)), 256 threads.
// part: (chunks, d_out, d_in, 8) Pauli sums [a][c][re, im]; dbpart: (chunks, d_out, 8)
// Pauli-row sums [b][re, im][a] of D, or NULL.
__global__ __launch_bounds__(256) void weight_grad_mfma_kernel(const float* __restrict__ Dp,
                                                               const float* __restrict__ Ap,
                                                               const int32_t* __restrict__ gather,
                                                               const int32_t* __restrict__ offsets, int E, int d_in,
                                                               int d_out, float* __restrict__ part,
                                                               float* __restrict__ dbpart) {
  int e, r0, r1;
  if (!wgm_find_chunk(offsets, E, blockIdx.x, e, r0, r1)) return;
  (void)e;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  r0 = __builtin_amdgcn_readfirstlane(r0);
  r1 = __builtin_amdgcn_readfirstlane(r1);
  const int l32 = lane & 31, kk = lane >> 5;
  const int j0 = blockIdx.y * kWgmTile + (wave & 1) * 32, i0 = blockIdx.z * kWgmTile + (wave >> 1) * 32;
  const int jc = min(j0 + l32, d_out - 1), ic = min(i0 + l32, d_in - 1);  // clamped loads, not stored
  const float* dcol = Dp + (size_t)jc * 8 + kk * 2;  // + row * d_out * 8; b = 0 at +0, b = 1 at +4
  const float* acol = Ap + (size_t)ic * 8;           // + src * d_in * 8
  const bool bias_wave = dbpart != nullptr && blockIdx.z == 0 && (wave >> 1) == 0;

  pf32x16_t acc[2][2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[a][c][q][v] = 0.f;
  float bs[4] = {0.f, 0.f, 0.f, 0.f};

  struct RowOps {
    float2 d0, d1;  // component kk of D[0][b], D[1][b] for b = 0, 1
    float4 x0, x1;  // A[c][b], b = 0, 1: (re c0, re c1, im c0, im c1)
  };
  auto load_row = [&](int r, RowOps& o) {
    const size_t src = gather ? (size_t)gather[r] : (size_t)r;
    const float* dr = dcol + (size_t)r * d_out * 8;
    o.d0 = *reinterpret_cast<const float2*>(dr);
    o.d1 = *reinterpret_cast<const float2*>(dr + 4);
    const float4* ar = reinterpret_cast<const float4*>(acol + src * d_in * 8);
    o.x0 = ar[0];
    o.x1 = ar[1];
  };
  auto mma_row = [&](const RowOps& o) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const float2 dv = b ? o.d1 : o.d0;
      const float4 xv = b ? o.x1 : o.x0;
      const float dd[2] = {dv.x, dv.y};
      const float re[2] = {xv.x, xv.y}, im[2] = {xv.z, xv.w};
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const float bre = kk ? im[c] : re[c];   // (re, im)[kk]
        const float bim = kk ? re[c] : -im[c];  // (-im, re)[kk]
#pragma unroll
        for (int a = 0; a < 2; ++a) {
          acc[a][c][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(dd[a], bre, acc[a][c][0], 0, 0, 0);
          acc[a][c][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(dd[a], bim, acc[a][c][1], 0, 0, 0);
        }
      }
    }
    if (bias_wave) {
      bs[0] += o.d0.x;
      bs[1] += o.d0.y;
      bs[2] += o.d1.x;
      bs[3] += o.d1.y;
    }
  };
  // rows in blocks of kWgmU, double buffered in registers
  const int nblk = (r1 - r0) / kWgmU;
  RowOps b0[kWgmU], b1[kWgmU];
  if (nblk > 0) {
#pragma unroll
    for (int u = 0; u < kWgmU; ++u) load_row(r0 + u, b0[u]);
  }
  for (int b = 0; b < nblk; b += 2) {
    if (b + 1 < nblk) {
#pragma unroll
      for (int u = 0; u < kWgmU; ++u) load_row(r0 + (b + 1) * kWgmU + u, b1[u]);
    }
#pragma unroll
    for (int u = 0; u < kWgmU; ++u) mma_row(b0[u]);
    if (b + 1 < nblk) {
      if (b + 2 < nblk) {
#pragma unroll
        for (int u = 0; u < kWgmU; ++u) load_row(r0 + (b + 2) * kWgmU + u, b0[u]);
      }
#pragma unroll
      for (int u = 0; u < kWgmU; ++u) mma_row(b1[u]);
    }
  }
  for (int r = r0 + nblk * kWgmU; r < r1; ++r) {
    RowOps o;
    load_row(r, o);
    mma_row(o);
  }

  // lane holds column i0 + l32, rows j0 + 8 (v / 4) + 4 kk + v % 4
  const int i = i0 + l32;
  float* pc = part + (size_t)blockIdx.x * d_out * d_in * 8;
  if (i < d_in) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int j = j0 + 8 * (v >> 2) + 4 * kk + (v & 3);
      if (j >= d_out) continue;
      float4* q = reinterpret_cast<float4*>(pc + ((size_t)j * d_in + i) * 8);
      q[0] = make_float4(acc[0][0][0][v], acc[0][0][1][v], acc[0][1][0][v], acc[0][1][1][v]);
      q[1] = make_float4(acc[1][0][0][v], acc[1][0][1][v], acc[1][1][0][v], acc[1][1][1][v]);
    }
  }
  if (bias_wave && j0 + l32 < d_out) {
    float* q = dbpart + ((size_t)blockIdx.x * d_out + j0 + l32) * 8 + kk * 2;  // [b][k][a]
    *reinterpret_cast<float2*>(q) = make_float2(bs[0], bs[1]);
    *reinterpret_cast<float2*>(q + 4) = make_float2(bs[2], bs[3]);
  }
}

// dW[e, j, i] = (1/2) blade(sum over the expert's chunks, in order, of the Pauli sums);
// db[e, j] likewise from the D-row sums.  One thread per (e, j, i) multivector.
__global__ __launch_bounds__(256) void weight_grad_reduce_kernel(const float* __restrict__ part,
                                                                 const float* __restrict__ dbpart,
                                                                 const int32_t* __restrict__ offsets, int E, int d_in,
                                                                 int d_out, float* __restrict__ dW,
                                                                 float* __restrict__ db) {
  const size_t n = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (n >= (size_t)E * d_out * d_in) return;
  const size_t ji = n % ((size_t)d_out * d_in);
  const int e = (int)(n / ((size_t)d_out * d_in));
  int cb = 0, beg = offsets[0];
  for (int x = 0; x < e; ++x) {
    const int end = offsets[x + 1];
    cb += (end - beg + kWgmChunk - 1) / kWgmChunk;
    beg = end;
  }
  const int ce = cb + (offsets[e + 1] - beg + kWgmChunk - 1) / kWgmChunk;
  float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int c = cb; c < ce; ++c) {
    const float4* q = reinterpret_cast<const float4*>(part + ((size_t)c * d_out * d_in + ji) * 8);
    const float4 u = q[0], w = q[1];
    s[0] += u.x; s[1] += u.y; s[2] += u.z; s[3] += u.w;
    s[4] += w.x; s[5] += w.y; s[6] += w.z; s[7] += w.w;
  }
  float o[8];
  pauli_to_blade(s[0], s[1], s[2], s[3], s[4], s[5], s[6], s[7], o);
  float4* dst = reinterpret_cast<float4*>(dW + n * 8);
  dst[0] = make_float4(0.5f * o[0], 0.5f * o[1], 0.5f * o[2], 0.5f * o[3]);
  dst[1] = make_float4(0.5f * o[4], 0.5f * o[5], 0.5f * o[6], 0.5f * o[7]);
  if (db != nullptr && ji % d_in == 0) {
    const int j = (int)(ji / d_in);
    float t[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};  // [b][k][a]
    for (int c = cb; c < ce; ++c) {
      const float4* q = reinterpret_cast<const float4*>(dbpart + ((size_t)c * d_out + j) * 8);
      const float4 u = q[0], w = q[1];
      t[0] += u.x; t[1] += u.y; t[2] += u.z; t[3] += u.w;
      t[4] += w.x; t[5] += w.y; t[6] += w.z; t[7] += w.w;
    }
    // entry (a, b): re at b * 4 + a, im at b * 4 + 2 + a
    pauli_to_blade(t[0], t[2], t[4], t[6], t[1], t[3], t[5], t[7], o);
    float4* q = reinterpret_cast<float4*>(db + ((size_t)e * d_out + j) * 8);
    q[0] = make_float4(0.5f * o[0], 0.5f * o[1], 0.5f * o[2], 0.5f * o[3]);
    q[1] = make_float4(0.5f * o[4], 0.5f * o[5], 0.5f * o[6], 0.5f * o[7]);
  }
}

}  // namespace

int grouped_weight_grad(const float* dy, const float* a, const int32_t* gather, const int32_t* offsets, int E,
                        int d_in, int d_out, float* dW, float* db, hipStream_t stream) {
  if (E == 0) return 0;
  hipLaunchKernelGGL(weight_grad_kernel, dim3((d_out + kWgT - 1) / kWgT, (d_in + kWgT - 1) / kWgT, E), dim3(256), 0,
                     stream, dy, a, gather, offsets, d_in, d_out, dW, db);
  return check_launch("weight gradient");
}

size_t weight_grad_pauli_workspace_bytes(int P_max, int E, int d_in, int d_out) {
  const size_t chunks = (size_t)(P_max + kWgmChunk - 1) / kWgmChunk + E;
  return chunks * ((size_t)d_out * d_in * 8 + (size_t)d_out * 8) * sizeof(float);
}

int weight_grad_pauli(const float* dy_pauli, const float* a_pauli, const int32_t* gather, const int32_t* offsets,
                      int P_max, int E, int d_in, int d_out, float* dW, float* db, void* workspace,
                      hipStream_t stream) {
  if (E == 0) return 0;
  const size_t chunks = (size_t)(P_max + kWgmChunk - 1) / kWgmChunk + E;
  float* part = static_cast<float*>(workspace);
  float* dbpart = db ? part + chunks * d_out * d_in * 8 : nullptr;
  if (P_max > 0) {
    hipLaunchKernelGGL(weight_grad_mfma_kernel,
                       dim3((unsigned)chunks, (d_out + kWgmTile - 1) / kWgmTile, (d_in + kWgmTile - 1) / kWgmTile),
                       dim3(256), 0, stream, dy_pauli, a_pauli, gather, offsets, E, d_in, d_out, part, dbpart);
    if (check_launch("weight gradient (MFMA)")) return -1;
  }
  const size_t n = (size_t)E * d_out * d_in;
  hipLaunchKernelGGL(weight_grad_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, part, dbpart,
                     offsets, E, d_in, d_out, dW, db);
  return check_launch("weight gradient (reduction)");
}

int activation_backward(const float* h, const float* g, size_t n_mv, int act, float* out, float* out_pauli,
                        hipStream_t stream) {
  if (n_mv == 0) return 0;
  const dim3 grid((unsigned)((n_mv + 255) / 256));
#define YGG_AB(A) hipLaunchKernelGGL(act_backward_kernel<A>, grid, dim3(256), 0, stream, h, g, n_mv, out, out_pauli)
  switch (act) {
    case kActNone: YGG_AB(kActNone); break;
    case kActGelu: YGG_AB(kActGelu); break;
    case kActRelu: YGG_AB(kActRelu); break;
    default: YGG_AB(kActSigmoid); break;
  }
#undef YGG_AB
  return check_launch("activation backward");
}

int activation_forward(const float* h, size_t n_mv, int act, float* out, float* out_pauli, hipStream_t stream) {
  if (n_mv == 0) return 0;
  const dim3 grid((unsigned)((n_mv + 255) / 256));
#define YGG_AF(A) hipLaunchKernelGGL(act_forward_kernel<A>, grid, dim3(256), 0, stream, h, n_mv, out, out_pauli)
  switch (act) {
    case kActNone: YGG_AF(kActNone); break;
    case kActGelu: YGG_AF(kActGelu); break;
    case kActRelu: YGG_AF(kActRelu); break;
    default: YGG_AF(kActSigmoid); break;
  }
#undef YGG_AF
  return check_launch("activation forward");
}

// a kernel rather than hipMemsetAsync, so a captured graph replays it like the other launches
__global__ __launch_bounds__(256) void fill_zero_kernel(float* __restrict__ p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) p[i] = 0.f;
}

int fill_zero_f32(float* p, size_t n, hipStream_t stream) {
  if (n == 0) return 0;
  const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(fill_zero_kernel, dim3(blocks), dim3(256), 0, stream, p, n);
  return check_launch("zero fill");
}

int combine_backward(const float* dout, const float* y_sorted, int N, int k, int d, const float* topk_w,
                     const int32_t* slot_pos, float* dy_sorted, float* dy_pauli, float* dtopk_w, hipStream_t stream) {
  if (N == 0) return 0;
  hipLaunchKernelGGL(combine_backward_kernel, dim3((N + 3) / 4), dim3(256), 0, stream, dout, y_sorted, N, k, d, topk_w,
                     slot_pos, dy_sorted, dy_pauli, dtopk_w);
  return check_launch("combine backward");
}

int dispatch_backward(const float* dxs, int N, int k, int d, const int32_t* slot_pos, const float* residual_grad,
                      float* dx, hipStream_t stream) {
  const size_t n = (size_t)N * d * 8;
  if (n == 0) return 0;
  hipLaunchKernelGGL(dispatch_backward_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, dxs, N, k, d,
                     slot_pos, residual_grad, dx);
  return check_launch("dispatch backward");
}

}  // namespace ygg

using namespace ygg;

YGG_API int ygg_adjoint_weights_f32(const float* W, int E, int d_out, int d_in, float* W_adj, hipStream_t stream) {
  YGG_CHECK_ARG(E >= 0 && d_out >= 0 && d_in >= 0, "ygg_adjoint_weights_f32: bad sizes");
  const size_t n = (size_t)E * d_out * d_in;
  if (n == 0) return 0;
  YGG_CHECK_ARG(W && W_adj && W != W_adj, "ygg_adjoint_weights_f32: null or aliased pointers");
  hipLaunchKernelGGL(adjoint_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, W, E, d_out, d_in,
                     W_adj);
  return check_launch("ygg_adjoint_weights_f32");
}

YGG_API int ygg_grouped_weight_grad_f32(const float* dy, const float* a, const int32_t* gather,
                                        const int32_t* offsets, int E, int d_in, int d_out, float* dW, float* db,
                                        hipStream_t stream) {
  YGG_CHECK_ARG(E >= 0 && E <= 65535 && d_in >= 1 && d_out >= 1,
                "ygg_grouped_weight_grad_f32: bad sizes E=%d d_in=%d d_out=%d", E, d_in, d_out);
  YGG_CHECK_ARG(E == 0 || (dy && a && offsets && dW), "ygg_grouped_weight_grad_f32: null pointer argument");
  return grouped_weight_grad(dy, a, gather, offsets, E, d_in, d_out, dW, db, stream);
}

YGG_API size_t ygg_grouped_weight_grad_pauli_f32_workspace_bytes(int P_max, int E, int d_in, int d_out) {
  if (P_max < 0 || E < 0 || d_in < 1 || d_out < 1) return 0;
  return weight_grad_pauli_workspace_bytes(P_max, E, d_in, d_out);
}

YGG_API int ygg_grouped_weight_grad_pauli_f32(const float* dy_pauli, const float* a_pauli, const int32_t* gather,
                                              const int32_t* offsets, int P_max, int E, int d_in, int d_out,
                                              float* dW, float* db, void* workspace, size_t workspace_bytes,
                                              hipStream_t stream) {
  YGG_CHECK_ARG(P_max >= 0 && E >= 0 && E <= 65535 && d_in >= 1 && d_out >= 1,
                "ygg_grouped_weight_grad_pauli_f32: bad sizes P_max=%d E=%d d_in=%d d_out=%d", P_max, E, d_in, d_out);
  YGG_CHECK_ARG(E == 0 || (offsets && dW && workspace), "ygg_grouped_weight_grad_pauli_f32: null pointer argument");
  YGG_CHECK_ARG(P_max == 0 || (dy_pauli && a_pauli), "ygg_grouped_weight_grad_pauli_f32: null rows");
  YGG_CHECK_ARG(workspace_bytes >= weight_grad_pauli_workspace_bytes(P_max, E, d_in, d_out),
                "ygg_grouped_weight_grad_pauli_f32: workspace of %zu bytes, need %zu", workspace_bytes,
                weight_grad_pauli_workspace_bytes(P_max, E, d_in, d_out));
  return weight_grad_pauli(dy_pauli, a_pauli, gather, offsets, P_max, E, d_in, d_out, dW, db, workspace, stream);
}

YGG_API int ygg_activation_backward(const float* h, const float* grad_out, size_t n_mv, int act, float* grad_in,
                                    hipStream_t stream) {
  YGG_CHECK_ARG(act >= kActNone && act <= kActSigmoid, "ygg_activation_backward: activation %d", act);
  YGG_CHECK_ARG(n_mv == 0 || (h && grad_out && grad_in), "ygg_activation_backward: null pointer argument");
  return activation_backward(h, grad_out, n_mv, act, grad_in, nullptr, stream);
}
