// decode_pauli.hip -- the decode-shape MoE-HLM layer on int8 Pauli weights
// (weight format 5) in one launch: routing, the up product with its bias and
// grade-wise activation, and the down product, per (expert, 64-wide chunk of
// the hidden width); and the preparation of those weights.
//
// Replaces, for decode batches (a few tokens per expert), CliffordRouter's
// selection (holograph/layers/clifford_router.py:18-21,93-104), the per-expert
// gather (holograph/models/hlm_block.py:165-178) and CliffordFFN.forward
// (hlm_block.py:55-61: CliffordLinear.forward, clifford_linear.py:101-123, then
// the activation, activations.py:15-128, then CliffordLinear.forward) of every
// expert.  The weighted combine (hlm_block.py:180-181) adds the chunks' partial
// planes afterwards (combine_planes, dispatch.hip).
//
// The weights.  A multivector is a 2x2 complex matrix M (pauli_common.h), and
// the geometric product the matrix product, so y_j = sum_i W_ji x_i reads
//   Y[a][b] = sum_i sum_c W_ji[a][c] X_i[c][b].
// Format 5 holds the eight real entries of every W_ji -- U = Re W, V = Im W --
// as int8 codes with one fp32 scale per (expert, output channel j):
//   s_j = max(max_{i, entries} |W_ji|, 1e-12) / 127,  q = clip(rint(W / s_j), +-127)
// (float64 arithmetic).  Eight bytes per multivector pair, as for blade codes.
//
// The products, split complex.  With X = Xr + i Xi and W = U + i V,
//   Re Y = U Xr - V Xi,   Im Y = U Xi + V Xr,
// so two real products share one A operand: rows (token t, column b, part p)
// hold X[c][b].p over K = (input i, row c) of X, and the B operands are U and V
// as stored, K = (i, c), columns (channel j, row a).  Four rows per token fill a
// 16-row MFMA block with four tokens -- a decode expert's usual share -- and an
// expert product costs 32 multiply-adds per multivector pair.  The products run
// on v_mfma_i32_16x16x64_i8: the codes are B fragments with no conversion, and
// each activation row is held as 16-bit fixed point, V = rint(x 2^sh) with a
// power of two per token bringing its largest entry into [2^13, 2^14), split
// into two int8 planes V = 256 hi + lo; the two planes' exact integer products
// are joined in the epilogue.  The activation rows thus carry 15 significant
// bits relative to their largest entry (bf16 has 8).
//
// The schedule (one workgroup of eight waves per (expert e, hidden chunk c)):
// loads are issued in the order the products need them, since a CU serves its
// vector loads in issue order -- the logits and epilogue operands, the up
// weights (each wave: one 16-column block, 8 channels x 2 rows a, over all
// inputs), then, after the workgroup has routed the batch, the expert's input
// rows, then the down weights (each wave: two 16-column blocks over the chunk's
// 64 hidden channels).  The up passes (4 tokens each) run while the down
// weights stream in; the chunk's hidden rows never leave the CU; the down
// product is cut along its contraction, one fp32 partial plane per chunk.
//
// Every reduction has a fixed order (integer MFMA sums are exact; the partial
// planes are added by the consumer in chunk order), so results do not depend
// on scheduling.

#include "decode_common.h"
#include "pauli_common.h"
#include "route_select.h"

namespace ygg {

typedef int dp_i32x4_t __attribute__((ext_vector_type(4)));

constexpr int kDpWaves = 8;
constexpr int kDpThreads = 64 * kDpWaves;
constexpr int kDpChunk = 64;                    // hidden channels per workgroup
constexpr int kDpMaxD = 128;                    // d: the up product's inputs, the down product's outputs
constexpr int kDpKsUp = kDpMaxD / 32;           // up K steps of 32 inputs (64 int8 K values)
constexpr int kDpKsDn = kDpChunk / 32;          // down K steps per chunk
constexpr int kDpBatch = 16;                    // an expert's tokens are taken 16 at a time
constexpr int kDpRb = kDpBatch / 4;             // row blocks (4 tokens each) per batch
constexpr int kDpMaxTokens = 128;               // routing inside the kernel, 64 tokens per selection pass
constexpr int kDpSelPasses = kDpMaxTokens / (kDpThreads / kSelLanes);
// dynamic LDS on top of the static arrays, so that one workgroup fills a CU's LDS
// share and the 8 x 32 workgroups of a decode layer land on distinct CUs
constexpr size_t kDpLdsPad = 24 * 1024;

// Format 5 layout: per expert, [JB = ceil(d_out / 8)][KS = ceil(d_in / 32)][U, V]
// [g 4][n 16][16 bytes]: n = 2 jj + a (channel j = 8 jb + jj, matrix row a), inputs
// i = 32 ks + 8 g + m, byte 2 m + c holds the code of W_ji[a][c] (U or V).  A
// wave's B fragment for one (column block, K step, U/V) is one contiguous KiB,
// lane g 16 + n taking bytes 16 (g 16 + n) .. + 15.
constexpr size_t kDpBlockBytes = 2048;  // one (jb, ks): 8 channels x 32 inputs x 8 bytes

__host__ __device__ inline size_t dp_expert_bytes(int d_out, int d_in) {
  return (size_t)((d_out + 7) / 8) * ((d_in + 31) / 32) * kDpBlockBytes;
}

// The eight Pauli entries of a blade-order multivector, as float64 (exact sums of
// two floats): [U00, V00, U01, V01, U10, V10, U11, V11], entry (a, c) of U + iV.
__device__ inline void dp_pauli_f64(const float* w, double (&p)[8]) {
  const double s = w[0], v1 = w[1], v2 = w[2], v3 = w[3], b12 = w[4], b13 = w[5], b23 = w[6], t = w[7];
  p[0] = s + v3;    // U00
  p[1] = t + b12;   // V00
  p[2] = v1 - b13;  // U01
  p[3] = b23 - v2;  // V01
  p[4] = v1 + b13;  // U10
  p[5] = b23 + v2;  // V10
  p[6] = s - v3;    // U11
  p[7] = t - b12;   // V11
}

// scale of (expert, channel) blockIdx.x: max(|entries|, 1e-12) / 127 in float64, rounded to fp32
__global__ __launch_bounds__(256) void dp_scale_kernel(const float* __restrict__ W, int d_in,
                                                       float* __restrict__ scales) {
  __shared__ double red[256];
  const float* base = W + (size_t)blockIdx.x * d_in * 8;
  double m = 0.0;
  for (int i = threadIdx.x; i < d_in; i += 256) {
    float w[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) w[q] = base[(size_t)i * 8 + q];
    double p[8];
    dp_pauli_f64(w, p);
#pragma unroll
    for (int q = 0; q < 8; ++q) m = fmax(m, fabs(p[q]));
  }
  red[threadIdx.x] = m;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s) red[threadIdx.x] = fmax(red[threadIdx.x], red[threadIdx.x + s]);
    __syncthreads();
  }
  if (threadIdx.x == 0) scales[blockIdx.x] = (float)(fmax(red[0], 1e-12) / 127.0);
}

// one thread per 16-byte unit (expert, jb, ks, U/V, g, n) of the layout
__global__ __launch_bounds__(256) void dp_prep_kernel(const float* __restrict__ W, int E, int d_out, int d_in,
                                                      const float* __restrict__ scales, uint4* __restrict__ out) {
  const int JB = (d_out + 7) / 8, KS = (d_in + 31) / 32;
  const size_t total = (size_t)E * JB * KS * 128;
  const size_t u = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (u >= total) return;
  const int n = (int)(u & 15), g = (int)((u >> 4) & 3), uv = (int)((u >> 6) & 1);
  size_t rest = u >> 7;
  const int ks = (int)(rest % KS);
  rest /= KS;
  const int jb = (int)(rest % JB);
  const int e = (int)(rest / JB);
  const int j = jb * 8 + (n >> 1), a = n & 1;
  uint32_t word[4] = {0u, 0u, 0u, 0u};
  if (j < d_out) {
    const double s = (double)scales[(size_t)e * d_out + j];
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const int i = ks * 32 + g * 8 + m;
      if (i >= d_in) break;
      float w[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) w[q] = W[(((size_t)e * d_out + j) * d_in + i) * 8 + q];
      double p[8];
      dp_pauli_f64(w, p);
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const double v = p[4 * a + 2 * c + uv];  // entry (a, c), U or V
        const int q = (int)fmin(fmax(rint(v / s), -127.0), 127.0);
        const int byte = 2 * m + c;
        word[byte >> 2] |= (uint32_t)(q & 0xff) << (8 * (byte & 3));
      }
    }
  }
  out[u] = make_uint4(word[0], word[1], word[2], word[3]);
}

// 16-bit fixed point value -> (hi, lo) int8 planes with v = 256 hi + lo, |v| <= 2^14.
// x scale lies in [-2^14, 2^14] for every finite row; the clamp (fmaxf and fminf return
// the operand that is not NaN, so NaN lands on -2^14) keeps the conversion defined for a
// non-finite row, whose inverse scale makes its outputs NaN.
__device__ inline void dp_split(float x, float scale, int& hi, int& lo) {
  const float t = x * scale;
  const int v = (int)rintf(fminf(fmaxf(t, -16384.f), 16384.f));
  hi = (v + 128) >> 8;
  lo = v - (hi << 8);
}
__device__ inline uint32_t dp_pair16(int c0, int c1) { return (uint32_t)(c0 & 0xff) | ((uint32_t)(c1 & 0xff) << 8); }

// The products' epilogue shared by both: the lane's four accumulated rows of its
// token (column b, part p at row 2 b + p) for channel column (jj, a), U and V each
// as hi and lo planes -> the full 2x2 matrix of the output multivector (the partner
// lane n ^ 1 holds the other row a), returned in blade order times two.
__device__ inline void dp_join(const dp_i32x4_t& uh, const dp_i32x4_t& ul, const dp_i32x4_t& vh,
                               const dp_i32x4_t& vl, int a, float (&y)[8]) {
  float zu[4], zv[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    zu[v] = (float)(uh[v] * 256 + ul[v]);
    zv[v] = (float)(vh[v] * 256 + vl[v]);
  }
  // row a of the output: Y[a][0] = (re, im), Y[a][1] = (re, im)
  const float mine[4] = {zu[0] - zv[1], zu[1] + zv[0], zu[2] - zv[3], zu[3] + zv[2]};
  float other[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) other[q] = dc_dpp<0xB1>(mine[q]);  // lane n ^ 1: row a ^ 1
  float r0[4], r1[4];  // rows 0 and 1 (selects, not a pointer: the arrays stay in registers)
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    r0[q] = a ? other[q] : mine[q];
    r1[q] = a ? mine[q] : other[q];
  }
  pauli_to_blade(r0[0], r0[1], r0[2], r0[3], r1[0], r1[1], r1[2], r1[3], y);
}

template <int ACT, int RQ>
__global__ __launch_bounds__(kDpThreads) void decode_pauli_kernel(
    const uint16_t* __restrict__ x, DcRoute rt, const int8_t* __restrict__ w_up, const float* __restrict__ s_up,
    const float* __restrict__ b_up, const int8_t* __restrict__ w_dn, const float* __restrict__ s_dn,
    const float* __restrict__ b_dn, int d, int F, int P_max, float* __restrict__ planes) {
  // LDS: the A operands (fixed point hi and lo planes) of the up passes
  // [rb][ks][hi/lo][g][row] and of the down passes, per-token scales and the routing
  __shared__ uint4 a_up[kDpRb * kDpKsUp * 2 * 64];  // 32 KiB
  __shared__ uint4 a_dn[kDpRb * kDpKsDn * 2 * 64];  // 16 KiB
  __shared__ float s_xmax[kDpBatch][2], s_xinv[kDpBatch], s_hinv[kDpBatch];
  __shared__ float s_hmax[kDpRb][kDpWaves][4];
  __shared__ int32_t rows_tok[kDpMaxTokens];           // this expert's tokens, ascending
  __shared__ int32_t rows_slot[kDpMaxTokens];          // their slots t k + s: the partial planes' rows
  __shared__ int32_t s_cnt[kMaxExperts], s_wv[kDpSelPasses * kDpWaves];
  __shared__ int32_t s_sel[kDpMaxTokens * kMaxTopK];  // the selection: expert and weight of every slot
  __shared__ float s_w[kDpMaxTokens * kMaxTopK];
  uint16_t* const a_up16 = reinterpret_cast<uint16_t*>(a_up);
  uint16_t* const a_dn16 = reinterpret_cast<uint16_t*>(a_dn);

  const int e = blockIdx.x, c = blockIdx.y;
  // the wave index is uniform: readfirstlane keeps what is built from it in scalar registers
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, n = lane & 15, jj = n >> 1, a = n & 1;
  const int N = rt.N, E = rt.E, k = rt.k;
  const int j0 = c * kDpChunk;

  // ---- 1. loads, in the order the products need them.  Every load is a raw
  // buffer load with no branch (an offset past the range reads zero), so each
  // wave's loads retire in this order and the compiler's waits stay exact.
  // (a) the logits: lane j of an 8-lane group takes experts j + 8 q of token tid / 8
  const int sj = tid & (kSelLanes - 1);
  float lg[kDpSelPasses][RQ];
  {
    const __amdgpu_buffer_rsrc_t lr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(rt.logits), (short)0, (uint32_t)N * E * 4, kBufferFlags);
#pragma unroll
    for (int ps = 0; ps < kDpSelPasses; ++ps) {
      const int t = ps * (kDpThreads / kSelLanes) + (tid >> 3);
#pragma unroll
      for (int q = 0; q < RQ; ++q) {
        const int xe = sj + kSelLanes * q;
        const bool ok = t < N && xe < E;
        const float v = __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(lr, ok ? (uint32_t)(t * E + xe) * 4 : kBufferOff, 0, 0));
        lg[ps][q] = ok ? v : -INFINITY;
      }
    }
  }
  // (b) the epilogues' operands: up channel ju (scale, mask-order bias), down
  // outputs od[q] (scales; the bias in chunk 0 only)
  const int ju = j0 + 8 * wave + jj;
  const int od0 = 16 * wave + jj;  // down outputs od0 and od0 + 8
  float su, bu[8], sd[2], bdn[2][8];
  {
    const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(s_up) + (size_t)e * F, (short)0, (uint32_t)F * 4, kBufferFlags);
    const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(b_up) + (b_up ? (size_t)e * F * 8 : 0), (short)0, b_up ? (uint32_t)F * 32 : 0u,
        kBufferFlags);
    su = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sr, (uint32_t)ju * 4, 0, 0));
    const float4 b0 = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(br, (uint32_t)ju * 32, 0, 0));
    const float4 b1 =
        __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(br, (uint32_t)ju * 32 + 16, 0, 0));
    bu[0] = b0.x; bu[1] = b0.y; bu[2] = b0.z; bu[3] = b0.w; bu[4] = b1.x; bu[5] = b1.y; bu[6] = b1.z; bu[7] = b1.w;
    const bool wb = b_dn != nullptr && c == 0;  // the down bias goes into chunk 0's plane
    const __amdgpu_buffer_rsrc_t sr2 = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(s_dn) + (size_t)e * d, (short)0, (uint32_t)d * 4, kBufferFlags);
    const __amdgpu_buffer_rsrc_t br2 = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(b_dn) + (wb ? (size_t)e * d * 8 : 0), (short)0, wb ? (uint32_t)d * 32 : 0u, kBufferFlags);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint32_t o = (uint32_t)(od0 + 8 * q);
      sd[q] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sr2, o * 4, 0, 0));
      const float4 c0 = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(br2, o * 32, 0, 0));
      const float4 c1 = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(br2, o * 32 + 16, 0, 0));
      bdn[q][0] = c0.x; bdn[q][1] = c0.y; bdn[q][2] = c0.z; bdn[q][3] = c0.w;
      bdn[q][4] = c1.x; bdn[q][5] = c1.y; bdn[q][6] = c1.z; bdn[q][7] = c1.w;
    }
  }
  // every wave has issued its logits and epilogue operands before any wave issues weights:
  // the CU serves loads in issue order across its waves, so a wave's logits issued after
  // another wave's weights would wait for them
  __syncthreads();
  // (c) the up weights: wave w takes column block jb = j0 / 8 + w over every K step
  const int KSu = (d + 31) >> 5, KSd = (F + 31) >> 5;
  uint4 wu[kDpKsUp][2];
  {
    const int JBu = (F + 7) >> 3, jb = (j0 >> 3) + wave;
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(w_up) + (size_t)e * dp_expert_bytes(F, d), (short)0, (uint32_t)dp_expert_bytes(F, d),
        kBufferFlags);
#pragma unroll
    for (int ks = 0; ks < kDpKsUp; ++ks)
#pragma unroll
      for (int uv = 0; uv < 2; ++uv) {
        const uint32_t off = (jb < JBu && ks < KSu) ? ((uint32_t)((jb * KSu + ks) * 2 + uv) << 10) + lane * 16 : kBufferOff;
        wu[ks][uv] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, 0));
      }
  }

  // ---- 2. routing of the whole batch (every workgroup routes it).  Only this
  // expert's tokens, in ascending order, stand between the logits and the input
  // rows: they come from a ballot over each token's selected slots.  The
  // renormalised weights, every expert's count and this expert's first row follow
  // once the input rows and the down weights are in flight.
  if (tid < kMaxExperts) s_cnt[tid] = 0;
  int sel_e[kDpSelPasses];
  float sel_raw[kDpSelPasses];
  uint32_t tok_mask[kDpSelPasses];  // uniform: bit g -- token 64 ps + 8 wave + g chose e
#pragma unroll
  for (int ps = 0; ps < kDpSelPasses; ++ps) {
    sel_e[ps] = -1;
    sel_raw[ps] = 0.f;
    tok_mask[ps] = 0u;
    if (ps * (kDpThreads / kSelLanes) < N) {
      const int t = ps * (kDpThreads / kSelLanes) + (tid >> 3);
      select_topk_raw<RQ>(lg[ps], E, k, t < N, sj, lane, sel_e[ps], sel_raw[ps]);
      if (sel_e[ps] >= 0) s_sel[t * k + sj] = sel_e[ps];
      const uint64_t b = __ballot(sel_e[ps] == e);
      uint32_t m = 0u;
#pragma unroll
      for (int gq = 0; gq < kDpThreads / kSelLanes / kDpWaves; ++gq)
        m |= ((b >> (kSelLanes * gq)) & 0xffull) ? (1u << gq) : 0u;
      tok_mask[ps] = m;
      if (lane == 0) s_wv[ps * kDpWaves + wave] = __popc(m);
    }
  }
  __syncthreads();
  // this wave's tokens take the rows after those of the (pass, wave) pairs before it
  int n_e = 0, tok_base[kDpSelPasses];
#pragma unroll
  for (int ps = 0; ps < kDpSelPasses; ++ps) {
    tok_base[ps] = 0;
    if (ps * (kDpThreads / kSelLanes) < N)
      for (int w = 0; w < kDpWaves; ++w) {
        if (w == wave) tok_base[ps] = n_e;
        n_e += s_wv[ps * kDpWaves + w];
      }
  }
#pragma unroll
  for (int ps = 0; ps < kDpSelPasses; ++ps)
    if (lane < 8 && ((tok_mask[ps] >> lane) & 1u))
      rows_tok[tok_base[ps] + __popc(tok_mask[ps] & ((1u << lane) - 1u))] =
          ps * (kDpThreads / kSelLanes) + kSelLanes * wave + lane;
  // the rest of the routing: renormalised weights and every expert's count (for this
  // expert's first row and the routing arrays)
  auto finish_routing = [&]() {
#pragma unroll
    for (int ps = 0; ps < kDpSelPasses; ++ps) {
      if (ps * (kDpThreads / kSelLanes) < N) {
        const int t = ps * (kDpThreads / kSelLanes) + (tid >> 3);
        const float w = renorm_slot(sel_raw[ps], k, sj, lane);
        if (sel_e[ps] >= 0) {
          s_w[t * k + sj] = w;
          atomicAdd(&s_cnt[sel_e[ps]], 1);
        }
      }
    }
  };
  // the routing arrays of this expert's slots, for the combine and the caller: written
  // by chunk 0 once its loads are all in (its loop would otherwise wait for them early)
  auto write_routing = [&](int row_beg) {
    if (c != 0) return;
    for (int r = tid; r < n_e; r += kDpThreads) {
      const int t = rows_tok[r];
      int q = 0;
      while (s_sel[t * k + q] != e) ++q;
      rt.topk_idx[t * k + q] = e;
      rt.topk_w[t * k + q] = s_w[t * k + q];
      rt.slot_pos[t * k + q] = row_beg + r;
      rt.perm[row_beg + r] = t;
    }
    if (tid == 0) {
      rt.counts[e] = n_e;
      rt.offsets[e] = row_beg;
      if (e == E - 1) rt.offsets[E] = row_beg + n_e;
    }
  };
  if (n_e == 0) {  // uniform: no token chose this expert
    finish_routing();
    __syncthreads();
    write_routing(dc_wave_sum(lane < e ? s_cnt[lane] : 0));
    return;
  }
  __syncthreads();  // rows_tok is complete
  for (int r = tid; r < n_e; r += kDpThreads) {  // (read after the conversion's barrier)
    const int t = rows_tok[r];
    int q = 0;
    while (s_sel[t * k + q] != e) ++q;
    rows_slot[r] = t * k + q;
  }

  // ---- 3. the input rows of the first batch (load l: token 4 l + tid / 128, input
  // tid % 128), then the down weights: wave w takes output column blocks 2 w and
  // 2 w + 1 over the chunk's two K steps
  const int xi = tid & 127, xt = tid >> 7;
  const __amdgpu_buffer_rsrc_t x_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(x), (short)0, (uint32_t)N * d * 16, kBufferFlags);
  uint4 xr[kDpRb];
#pragma unroll
  for (int l = 0; l < kDpRb; ++l) {
    const int tk = 4 * l + xt;
    const uint32_t off = (tk < n_e && xi < d) ? (uint32_t)(rows_tok[tk] * d + xi) * 16 : kBufferOff;
    xr[l] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(x_rsrc, off, 0, 0));
  }
  // every wave's input rows ahead of any wave's down weights (loads are served in issue
  // order across the CU's waves; the conversion waits for all rows of the batch)
  __syncthreads();
  uint4 wd[2][kDpKsDn][2];
  {
    const int JBd = (d + 7) >> 3;
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(w_dn) + (size_t)e * dp_expert_bytes(d, F), (short)0, (uint32_t)dp_expert_bytes(d, F),
        kBufferFlags);
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int s = 0; s < kDpKsDn; ++s)
#pragma unroll
        for (int uv = 0; uv < 2; ++uv) {
          const int ob = 2 * wave + q, ks = c * kDpKsDn + s;
          const uint32_t off =
              (ob < JBd && ks < KSd) ? ((uint32_t)((ob * KSd + ks) * 2 + uv) << 10) + lane * 16 : kBufferOff;
          wd[q][s][uv] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, 0));
        }
  }

  // with the input rows and the down weights in flight: the rest of the routing; this
  // expert's rows start after those of the experts before it (E <= 64: one lane each)
  finish_routing();
  __syncthreads();
  const int row_beg = dc_wave_sum(lane < e ? s_cnt[lane] : 0);

  // bf16 rows (blade order) -> Pauli entries -> per-token fixed point, hi and lo
  // planes of the up A operand.  Thread (xt, xi) of load l writes the rows (token xt
  // of row block l, column b, part p) at K position (input xi, c = 0, 1): 16 bits
  // per plane and row.
  auto convert_x = [&](int nb) {
    float pv[kDpRb][8];
    // every load is converted (rows past the batch read zero): a load whose only use sat
    // behind a branch would be moved there by the compiler, behind the down weights
#pragma unroll
    for (int l = 0; l < kDpRb; ++l) {
      const uint32_t wv[4] = {xr[l].x, xr[l].y, xr[l].z, xr[l].w};
      float b[8];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        b[2 * u] = bf16_bits_to_f32((uint16_t)(wv[u] & 0xffffu));
        b[2 * u + 1] = bf16_bits_to_f32((uint16_t)(wv[u] >> 16));
      }
      blade_to_pauli(b, &pv[l][0], &pv[l][4]);  // column 0 (M00, M10), column 1 (M01, M11)
      float m = 0.f;
#pragma unroll
      for (int q = 0; q < 8; ++q) m = fmaxf(m, dc_mag(pv[l][q]));
      m = dc_wave_max(m);
      if (lane == 0) s_xmax[4 * l + xt][wave & 1] = m;
    }
    __syncthreads();
    const int ks = xi >> 5, gg = (xi >> 3) & 3, m8 = xi & 7;
#pragma unroll
    for (int l = 0; l < kDpRb; ++l) {
      if (4 * l >= nb) break;
      const int tk = 4 * l + xt;
      const float mt = fmaxf(s_xmax[tk][0], s_xmax[tk][1]);
      const int sh = dc_shift(mt);
      const float sc = ldexpf(1.0f, sh);
      if (xi == 0) s_xinv[tk] = dc_inv_scale(mt, sh);
#pragma unroll
      for (int v = 0; v < 4; ++v) {  // row (b, p) = (v / 2, v % 2): entries X[0][b].p, X[1][b].p
        const int b = v >> 1, p = v & 1;
        int h0, l0, h1, l1;
        dp_split(pv[l][4 * b + p], sc, h0, l0);
        dp_split(pv[l][4 * b + 2 + p], sc, h1, l1);
        const int unit = ((l * kDpKsUp + ks) * 2 * 4 + gg) * 16 + 4 * xt + v;
        a_up16[unit * 8 + m8] = (uint16_t)dp_pair16(h0, h1);
        a_up16[(unit + 64) * 8 + m8] = (uint16_t)dp_pair16(l0, l1);
      }
    }
  };
  convert_x(min(kDpBatch, n_e));

  for (int b0 = 0; b0 < n_e; b0 += kDpBatch) {
    if (b0 > 0) {  // a later batch: its rows load behind everything else
      __syncthreads();  // the previous batch's LDS readers are done
#pragma unroll
      for (int l = 0; l < kDpRb; ++l) {
        const int tk = b0 + 4 * l + xt;
        const uint32_t off = (tk < n_e && xi < d) ? (uint32_t)(rows_tok[tk] * d + xi) * 16 : kBufferOff;
        xr[l] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(x_rsrc, off, 0, 0));
      }
      convert_x(min(kDpBatch, n_e - b0));
    }
    const int nb = min(kDpBatch, n_e - b0), nrb = (nb + 3) >> 2;
    __syncthreads();  // the batch's up operand is complete

    // ---- 4. up passes of 4 tokens: 16 MFMAs per wave -> hidden rows of the chunk,
    // quantized per token into the down product's A operand
    for (int rb = 0; rb < nrb; ++rb) {  // uniform
      dp_i32x4_t uh = {0, 0, 0, 0}, ul = uh, vh = uh, vl = uh;
#pragma unroll
      for (int ks = 0; ks < kDpKsUp; ++ks) {
        const dp_i32x4_t Ah = __builtin_bit_cast(dp_i32x4_t, a_up[((rb * kDpKsUp + ks) * 2 + 0) * 64 + lane]);
        const dp_i32x4_t Al = __builtin_bit_cast(dp_i32x4_t, a_up[((rb * kDpKsUp + ks) * 2 + 1) * 64 + lane]);
        const dp_i32x4_t Bu = __builtin_bit_cast(dp_i32x4_t, wu[ks][0]);
        const dp_i32x4_t Bv = __builtin_bit_cast(dp_i32x4_t, wu[ks][1]);
        uh = __builtin_amdgcn_mfma_i32_16x16x64_i8(Ah, Bu, uh, 0, 0, 0);
        ul = __builtin_amdgcn_mfma_i32_16x16x64_i8(Al, Bu, ul, 0, 0, 0);
        vh = __builtin_amdgcn_mfma_i32_16x16x64_i8(Ah, Bv, vh, 0, 0, 0);
        vl = __builtin_amdgcn_mfma_i32_16x16x64_i8(Al, Bv, vl, 0, 0, 0);
      }
      // epilogue: lane group g is token 4 rb + g of the batch; (jj, a) its channel and row
      const int tk = 4 * rb + g;
      float hb[8];
      dp_join(uh, ul, vh, vl, a, hb);
      const float sc = 0.5f * su * s_xinv[tk];
#pragma unroll
      for (int r = 0; r < 8; ++r) hb[r] = hb[r] * sc + bu[blade_to_mask(r)];
      activate_blade<ACT>(hb);
      const bool ok = tk < nb && ju < F;
      float hc0[4], hc1[4];
      blade_to_pauli(hb, hc0, hc1);  // column 0 (H00, H10), column 1 (H01, H11)
      float m = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        hc0[q] = ok ? hc0[q] : 0.f;
        hc1[q] = ok ? hc1[q] : 0.f;
        m = fmaxf(m, fmaxf(fabsf(hc0[q]), fabsf(hc1[q])));
      }
      m = dc_row_max(m);  // over the token's 8 channels x 2 rows in this wave
      if (n == 0) s_hmax[rb][wave][g] = m;
      __syncthreads();
      float mx = 0.f;
#pragma unroll
      for (int w = 0; w < kDpWaves; ++w) mx = fmaxf(mx, s_hmax[rb][w][g]);
      const int sh = dc_shift(mx);
      const float hs = ldexpf(1.0f, sh);
      // a hidden row is non-finite through an infinite entry (its maximum) or through a
      // non-finite input row (NaN inverse scale: its hidden row is NaN)
      if (wave == 0 && n == 0) {
        const float xinv = s_xinv[tk];
        s_hinv[tk] = xinv == xinv ? dc_inv_scale(mx, sh) : xinv;
      }
      // lane (jj, a) writes the rows of column b = a: entries (H[0][a].p, H[1][a].p) at
      // K position hidden channel 8 wave + jj (K step wave / 4, lane group wave % 4)
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        int h0, l0, h1, l1;
        dp_split(a ? hc1[p] : hc0[p], hs, h0, l0);
        dp_split(a ? hc1[2 + p] : hc0[2 + p], hs, h1, l1);
        const int unit = ((rb * kDpKsDn + (wave >> 2)) * 2 * 4 + (wave & 3)) * 16 + 4 * g + 2 * a + p;
        a_dn16[unit * 8 + jj] = (uint16_t)dp_pair16(h0, h1);
        a_dn16[(unit + 64) * 8 + jj] = (uint16_t)dp_pair16(l0, l1);
      }
    }
    __syncthreads();  // the batch's down operand is complete

    // ---- 5. down passes of 4 tokens: 16 MFMAs per wave -> fp32 partial plane c
    for (int rb = 0; rb < nrb; ++rb) {
      dp_i32x4_t acc[2][4];
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[q][t] = dp_i32x4_t{0, 0, 0, 0};
#pragma unroll
      for (int s = 0; s < kDpKsDn; ++s) {
        const dp_i32x4_t Ah = __builtin_bit_cast(dp_i32x4_t, a_dn[((rb * kDpKsDn + s) * 2 + 0) * 64 + lane]);
        const dp_i32x4_t Al = __builtin_bit_cast(dp_i32x4_t, a_dn[((rb * kDpKsDn + s) * 2 + 1) * 64 + lane]);
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const dp_i32x4_t Bu = __builtin_bit_cast(dp_i32x4_t, wd[q][s][0]);
          const dp_i32x4_t Bv = __builtin_bit_cast(dp_i32x4_t, wd[q][s][1]);
          acc[q][0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(Ah, Bu, acc[q][0], 0, 0, 0);
          acc[q][1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(Al, Bu, acc[q][1], 0, 0, 0);
          acc[q][2] = __builtin_amdgcn_mfma_i32_16x16x64_i8(Ah, Bv, acc[q][2], 0, 0, 0);
          acc[q][3] = __builtin_amdgcn_mfma_i32_16x16x64_i8(Al, Bv, acc[q][3], 0, 0, 0);
        }
      }
      const int tk = 4 * rb + g;
      const float hsi = s_hinv[tk];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        float y[8];
        dp_join(acc[q][0], acc[q][1], acc[q][2], acc[q][3], a, y);
        const float sc = 0.5f * sd[q] * hsi;
        const int o = od0 + 8 * q;
        // lane a = 0 writes blades 0-3, a = 1 blades 4-7.  The halves are picked as whole
        // values: a lane-dependent index into y would turn y into a memory array (the
        // compiler then places it in LDS, indexed by the flat thread id)
        const float4 ylo = make_float4(y[0], y[1], y[2], y[3]), yhi = make_float4(y[4], y[5], y[6], y[7]);
        const float4 blo = make_float4(bdn[q][blade_to_mask(0)], bdn[q][blade_to_mask(1)], bdn[q][blade_to_mask(2)],
                                       bdn[q][blade_to_mask(3)]);
        const float4 bhi = make_float4(bdn[q][blade_to_mask(4)], bdn[q][blade_to_mask(5)], bdn[q][blade_to_mask(6)],
                                       bdn[q][blade_to_mask(7)]);
        const float4 ys = a ? yhi : ylo, bs = a ? bhi : blo;
        const float4 o4 = make_float4(ys.x * sc + bs.x, ys.y * sc + bs.y, ys.z * sc + bs.z, ys.w * sc + bs.w);
        if (tk < nb && o < d)
          *reinterpret_cast<float4*>(planes + (((size_t)c * P_max + rows_slot[b0 + tk]) * d + o) * 8 + 4 * a) = o4;
      }
    }
  }
  write_routing(row_beg);
}

}  // namespace ygg

using namespace ygg;

size_t ygg::decode_pauli_weight_bytes(int E, int d_out, int d_in) { return (size_t)E * dp_expert_bytes(d_out, d_in); }

int ygg::decode_pauli_prepare_weights(const float* W, int E, int d_out, int d_in, void* out, float* scales,
                                      hipStream_t stream) {
  YGG_CHECK_ARG(scales, "ygg_prepare_weights: the int8 Pauli format needs a scales buffer [E, d_out]");
  YGG_CHECK_ARG(decode_pauli_weight_bytes(1, d_out, d_in) < 0x7fffffffULL,
                "ygg_prepare_weights: one expert's int8 Pauli weights must stay below 2 GiB (d_out=%d d_in=%d)",
                d_out, d_in);
  dp_scale_kernel<<<E * d_out, 256, 0, stream>>>(W, d_in, scales);
  if (check_launch("dp_scale")) return -1;
  const size_t units = decode_pauli_weight_bytes(E, d_out, d_in) / 16;
  dp_prep_kernel<<<(unsigned)((units + 255) / 256), 256, 0, stream>>>(W, E, d_out, d_in, scales,
                                                                      static_cast<uint4*>(out));
  return check_launch("dp_prep");
}

bool ygg::decode_pauli_fusable(int N, int E, int k, int d, int F) {
  return N >= 1 && N <= kDpMaxTokens && E >= 1 && E <= kMaxExperts && k >= 1 && k <= kMaxTopK && k <= E && d >= 1 &&
         d <= kDpMaxD && F >= 1;
}

int ygg::decode_pauli_planes(int F) { return (F + kDpChunk - 1) / kDpChunk; }

template <int ACT, int RQ>
static void launch_dp(dim3 grid, hipStream_t st, const uint16_t* x, const DcRoute& rt, const int8_t* wu,
                      const float* su, const float* bu, const int8_t* wd, const float* sd, const float* bd, int d,
                      int F, int P_max, float* planes) {
  decode_pauli_kernel<ACT, RQ><<<grid, kDpThreads, kDpLdsPad, st>>>(x, rt, wu, su, bu, wd, sd, bd, d, F, P_max,
                                                                      planes);
}

int ygg::decode_pauli_layer(const uint16_t* x, const float* logits, int N, int E, int k, int d, int F, int act,
                            const int8_t* w_up, const float* s_up, const float* b_up, const int8_t* w_dn,
                            const float* s_dn, const float* b_dn, int32_t* topk_idx, float* topk_w, int32_t* counts,
                            int32_t* offsets, int32_t* perm, int32_t* slot_pos, float* planes, hipStream_t stream) {
  YGG_CHECK_ARG(decode_pauli_fusable(N, E, k, d, F),
                "int8 Pauli decode layer: N=%d E=%d k=%d d=%d F=%d outside its limits (N <= %d, d <= %d)", N, E, k,
                d, F, kDpMaxTokens, kDpMaxD);
  YGG_CHECK_ARG(act >= kActNone && act <= kActSigmoid, "int8 Pauli decode layer: activation %d", act);
  YGG_CHECK_ARG((size_t)N * d * 16 < 0x7fffffffULL, "int8 Pauli decode layer: x too large");
  const DcRoute rt{logits, N, E, k, topk_idx, topk_w, counts, offsets, perm, slot_pos};
  const dim3 grid(E, decode_pauli_planes(F));
  const int P_max = N * k;
#define YGG_DP(A)                                                                                          \
  ((E <= 32) ? launch_dp<A, 4>(grid, stream, x, rt, w_up, s_up, b_up, w_dn, s_dn, b_dn, d, F, P_max, planes) \
             : launch_dp<A, 8>(grid, stream, x, rt, w_up, s_up, b_up, w_dn, s_dn, b_dn, d, F, P_max, planes))
  switch (act) {
    case kActNone: YGG_DP(kActNone); break;
    case kActGelu: YGG_DP(kActGelu); break;
    case kActRelu: YGG_DP(kActRelu); break;
    default: YGG_DP(kActSigmoid); break;
  }
#undef YGG_DP
  return check_launch("decode_pauli_layer");
}
