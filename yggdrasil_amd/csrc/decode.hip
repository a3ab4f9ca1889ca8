// decode.hip -- the decode-shape MoE-HLM layer with int8 expert weights in one
// launch: routing, the up product with its bias and grade-wise activation, and
// the down product, per (expert, 64-wide chunk of the hidden width).
//
// Replaces, for decode batches (a few tokens per expert), CliffordRouter's
// selection (holograph/layers/clifford_router.py:18-21,93-104), the per-expert
// gather (holograph/models/hlm_block.py:165-178) and CliffordFFN.forward
// (hlm_block.py:55-61: CliffordLinear.forward, clifford_linear.py:101-123, then
// the activation, activations.py:15-128, then CliffordLinear.forward) of every
// expert.  The weighted combine (hlm_block.py:180-181) adds the chunks' partial
// planes afterwards (combine_planes, dispatch.hip).
//
// Weight bytes bound this shape (about four tokens per expert), so the design
// keeps the HBM stream full and puts everything else in its shadow:
//
// * One workgroup per (expert e, hidden chunk c of 64 multivectors), eight
//   waves, each holding one eighth of the chunk's weights in registers: the up
//   product's 64 output channels over every input, and the down product's every
//   output over the chunk's 64 inputs.  The chunk's hidden activations never
//   leave the CU: the down product is cut along its contraction, one fp32
//   partial plane per chunk, added by the combine.
// * A CU serves its vector loads in issue order, whichever wave issued them, so
//   the order of issue is the schedule: the logits and epilogue operands first,
//   then the up weights, then -- once the workgroup has routed the batch -- the
//   expert's input rows, then the down weights.  The input rows arrive with the
//   up weights, and the up products run while the down weights stream in.
// * The weights enter the MFMA as stored.  y = w x (weight on the left) is, in
//   mask order (e_p e_q = s(p, q) e_{p^q}),  y_r = sum_q s(q, q^r) x_{q^r} w_q,
//   so the activation is expanded instead of the weight: row (token, r) of the A
//   operand holds the signed permutation s(q, q^r) x_{q^r} of each input
//   multivector, K runs over (input, q), and B is the weight multivector.  Eight
//   output blades per token make eight MFMA rows: two tokens per 16-row block.
//   On packed fp16 pairs the expansion is a dword permutation, a half swap for
//   odd r and sign-bit flips.
// * int8 codes become exact fp16 B operands with one byte permute and one packed
//   fp16 subtract per two codes: with c = q ^ 0x80 = q + 128, the fp16 whose bits
//   are 0x64 c is 1024 + c = 1152 + q, and subtracting 1152 leaves q.
// * A operands are fp16: each token's input row (and its hidden row) is scaled
//   by a power of two that brings its largest magnitude into [2^13, 2^14), which
//   is undone in the epilogue.  bf16 inputs then convert exactly; hidden values
//   round to fp16 (11 significant bits).
//
// Every reduction has a fixed order (the two halves of the up contraction added
// in order, the partial planes added by the consumer in chunk order), so
// results do not depend on scheduling.

#include "decode_common.h"
#include "route_select.h"

namespace ygg {

typedef _Float16 dc_f16x8_t __attribute__((ext_vector_type(8)));
typedef float dc_f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kDcWaves = 8;
constexpr int kDcThreads = 64 * kDcWaves;
constexpr int kDcChunk = 64;                     // hidden multivectors per workgroup
constexpr int kDcMaxD = 128;                     // d: the up product's inputs, the down product's outputs
constexpr int kDcMaxTokens = 128;                // routing inside the kernel, 64 tokens per selection pass
constexpr int kDcSelPasses = kDcMaxTokens / (kDcThreads / kSelLanes);
constexpr int kDcBatch = 16;                     // an expert's tokens are taken 16 at a time
constexpr int kDcUpTok = 4;                      // tokens per up pass: 32 A rows = 2 blocks of 16
constexpr int kDcDnTok = 8;                      // tokens per down pass: 4 blocks
constexpr int kDcUpSteps = kDcMaxD / 4;          // K steps of 4 input multivectors (32 fp16)
constexpr int kDcDnSteps = kDcChunk / 4;
constexpr int kDcGrp = 20;                       // A staging slots per lane group of a K step
constexpr int kDcStep = 81;                      // slots per K step (4 groups of 16 rows, padded)
constexpr int kDcOpSlots = 2 * kDcUpSteps * kDcStep;  // the A staging area (= 4 * kDcDnSteps * kDcStep)
static_assert(kDcOpSlots == 4 * kDcDnSteps * kDcStep, "up and down passes share the A staging area");

typedef _Float16 dc_f16x2_t __attribute__((ext_vector_type(2)));

// sign of x_{q^r} in row r, column q of the expanded activation (prepared weights
// store kWFold(q) w_q, mask order)
__host__ __device__ constexpr int dc_sign(int r, int q) { return mask_product_sign(q, q ^ r) * kWFold(q); }

// The weight registers as seen at the point of conversion: the empty asm makes
// them look redefined there, so the compiler cannot hoist the conversion above
// it -- which, for the down weights, would wait for them (loads retire in order)
// before the first up pass could start.
__device__ inline uint4 dc_pin(uint4 q) {
  asm volatile("" : "+v"(q.x), "+v"(q.y), "+v"(q.z), "+v"(q.w));
  return q;
}

// int8 codes of one multivector (two dwords, components q = 0..7) -> B fragment
__device__ inline dc_f16x8_t dc_codes_to_f16(uint32_t lo, uint32_t hi) {
  const uint32_t kHi = 0x64646464u;
  lo ^= 0x80808080u;
  hi ^= 0x80808080u;
  const uint32_t u[4] = {__builtin_amdgcn_perm(kHi, lo, 0x04010400u),   // (1152 + q0, 1152 + q1)
                         __builtin_amdgcn_perm(kHi, lo, 0x04030402u), __builtin_amdgcn_perm(kHi, hi, 0x04010400u),
                         __builtin_amdgcn_perm(kHi, hi, 0x04030402u)};
  const dc_f16x2_t off = {(_Float16)1152.0f, (_Float16)1152.0f};
  uint32_t d[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) d[t] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(dc_f16x2_t, u[t]) - off);
  return __builtin_bit_cast(dc_f16x8_t, d);
}

__device__ inline uint32_t dc_pack_f16(float lo, float hi) {
  const _Float16 a = (_Float16)lo, b = (_Float16)hi;
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// The eight expanded rows (r = 0..7) of one multivector, packed fp16 in mask
// order (dword u = components 2u, 2u + 1), into the A staging area: row r, dword
// m holds components 2m ^ r and (2m + 1) ^ r -- dword m ^ (r >> 1), halves
// swapped for odd r -- with the signs s(q, q^r) kWFold(q) as sign-bit flips.
// dst points at row 0's 16-byte slot; rows are 16 B apart.
__device__ inline void dc_expand(const uint4 v, uint4* dst) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    uint32_t o[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const uint32_t src = w[m ^ (r >> 1)];
      const uint32_t sw = (r & 1) ? __builtin_amdgcn_alignbit(src, src, 16) : src;
      const uint32_t neg = (dc_sign(r, 2 * m) < 0 ? 0x8000u : 0u) | (dc_sign(r, 2 * m + 1) < 0 ? 0x80000000u : 0u);
      o[m] = sw ^ neg;
    }
    dst[r] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// activations in mask order (grade = popcount): as activate_mask_order in
// clifford_gemm.hip, with the hardware exp2 / rcp / sqrt
__device__ inline float dc_sigmoid(float z) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * z));
}
template <int ACT>
__device__ inline void dc_activate(float (&y)[8]) {
  if constexpr (ACT == kActNone) {
    return;
  } else {
    const float m1 = __builtin_amdgcn_sqrtf(y[1] * y[1] + y[2] * y[2] + y[4] * y[4] + 1e-12f);
    const float m2 = __builtin_amdgcn_sqrtf(y[3] * y[3] + y[5] * y[5] + y[6] * y[6] + 1e-12f);
    float f0, f1, f2;
    if constexpr (ACT == kActGelu) {  // gelu(v) = v sigmoid(2 sqrt(2/pi) (v + 0.044715 v^3))
      const float k2 = 2.0f * 0.7978845608028654f;
      f0 = dc_sigmoid(k2 * (y[0] + 0.044715f * y[0] * y[0] * y[0]));
      f1 = dc_sigmoid(k2 * (m1 + 0.044715f * m1 * m1 * m1));
      f2 = dc_sigmoid(k2 * (m2 + 0.044715f * m2 * m2 * m2));
      y[7] = 2.0f * dc_sigmoid(2.0f * y[7]) - 1.0f;
    } else if constexpr (ACT == kActSigmoid) {
      y[0] = dc_sigmoid(y[0]);
      f0 = 1.0f;
      f1 = dc_sigmoid(m1) * __builtin_amdgcn_rcpf(m1);
      f2 = dc_sigmoid(m2) * __builtin_amdgcn_rcpf(m2);
      y[7] = 2.0f * dc_sigmoid(2.0f * y[7]) - 1.0f;
    } else {  // relu with zero thresholds
      f0 = y[0] > 0.f ? 1.0f : 0.0f;
      f1 = 1.0f;
      f2 = 1.0f;
    }
    y[0] *= f0;
    y[1] *= f1;
    y[2] *= f1;
    y[4] *= f1;
    y[3] *= f2;
    y[5] *= f2;
    y[6] *= f2;
  }
}


// Slot (16 bytes) of the A staging area holding the A fragment of lane (g, row) at
// K step s of one 16-row block.  The strides make both access patterns free of
// bank conflicts within each 16-lane quarter of a wave: the MFMA loop's loads
// (fixed s and g, 16 consecutive rows) and the expansion's stores (fixed row, 16
// consecutive inputs: four steps x four lane groups, which land on slot
// residues s + 4 g mod 16, all distinct since kDcStep = 1 and kDcGrp = 4 mod 16).
__device__ inline int dc_slot(int s, int g, int row) { return s * kDcStep + g * kDcGrp + row; }

// Input multivector i (or hidden channel i) sits at K step 2 (i / 8) + i % 2, lane
// group (i % 8) / 2: K step pairs hold the inputs 8 p + 2 g and 8 p + 2 g + 1,
// one 16-byte slot of the int8 weight layout.
__device__ inline int dc_in_slot(int i, int row) { return dc_slot(2 * (i >> 3) + (i & 1), (i & 7) >> 1, row); }

// The down product of one pass: NRT row blocks over the chunk's 16 K steps.
template <int NRT>
__device__ inline void dc_down_mfma(const dc_f16x8_t (&bd)[kDcDnSteps], const uint4* a_op, int g, int n,
                                    dc_f32x4_t (&acc)[4]) {
#pragma unroll
  for (int st = 0; st < kDcDnSteps; ++st) {
#pragma unroll
    for (int rb = 0; rb < NRT; ++rb) {
      const dc_f16x8_t A = __builtin_bit_cast(dc_f16x8_t, a_op[rb * (kDcDnSteps * kDcStep) + dc_slot(st, g, n)]);
      acc[rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, bd[st], acc[rb], 0, 0, 0);
    }
  }
}

template <int ACT, int RQ>
__global__ __launch_bounds__(kDcThreads) void decode_layer_kernel(
    const uint16_t* __restrict__ x, DcRoute rt, const int8_t* __restrict__ w_up, const float* __restrict__ s_up,
    const float* __restrict__ b_up, const int8_t* __restrict__ w_dn, const float* __restrict__ s_dn,
    const float* __restrict__ b_dn, int d, int F, int P_max, float* __restrict__ planes) {
  // LDS: the expanded A operand (up passes: 2 row blocks x 32 steps; down passes:
  // 4 row blocks x 16 steps), the up product's two contraction halves, the hidden
  // rows of a batch, per-token scales and the routing
  __shared__ uint4 a_op[kDcOpSlots];                     // 81 KiB
  __shared__ float4 c_up[2][kDcUpTok][2][kDcChunk];      // [half][token][blades 0-3 / 4-7 (mask)][channel]
  __shared__ float4 h_st[kDcBatch][2][kDcChunk];         // hidden rows, fp32 mask order
  __shared__ float s_xmax[kDcBatch][2], s_xinv[kDcBatch], s_hmax[kDcBatch];
  __shared__ int32_t rows_tok[kDcMaxTokens];             // this expert's tokens, ascending
  __shared__ int32_t s_cnt[kMaxExperts], s_wv[kDcWaves];
  __shared__ int32_t s_sel[kDcMaxTokens * kMaxTopK];  // the selection: expert and weight of every slot
  __shared__ float s_w[kDcMaxTokens * kMaxTopK];

  const int e = blockIdx.x, c = blockIdx.y;
  // the wave index is uniform: readfirstlane keeps what is built from it in scalar registers
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, n = lane & 15;
  const int N = rt.N, E = rt.E, k = rt.k;
  const int j0 = c * kDcChunk;

  // ---- 1. loads, in the order the products need them.  Every load is a raw
  // buffer load with no branch (an offset past the range reads zero), so each
  // wave's loads retire in this order and the compiler's waits stay exact.
  // (a) the logits: lane j of an 8-lane group takes experts j + 8 q of token tid / 8
  const int sj = tid & (kSelLanes - 1);
  float lg[kDcSelPasses][RQ];
  {
    const __amdgpu_buffer_rsrc_t lr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(rt.logits), (short)0, (uint32_t)N * E * 4, kBufferFlags);
#pragma unroll
    for (int ps = 0; ps < kDcSelPasses; ++ps) {
      const int t = ps * (kDcThreads / kSelLanes) + (tid >> 3);
#pragma unroll
      for (int q = 0; q < RQ; ++q) {
        const int xe = sj + kSelLanes * q;
        const bool ok = t < N && xe < E;
        const float v =
            __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(lr, ok ? (uint32_t)(t * E + xe) * 4 : kBufferOff, 0, 0));
        lg[ps][q] = ok ? v : -INFINITY;
      }
    }
  }
  // (b) the epilogues' operands: up (channel j0 + lane, all 8 bias components),
  // down (output 16 wave + n, the 4 mask components 4 (g & 1) .. + 3 of this lane)
  const int ju = j0 + lane, od = 16 * wave + n;
  float su, bu[8], sd;
  float4 bd;
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
    sd = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sr2, (uint32_t)od * 4, 0, 0));
    bd = __builtin_bit_cast(float4,
                            __builtin_amdgcn_raw_buffer_load_b128(br2, (uint32_t)od * 32 + (uint32_t)(g & 1) * 16, 0, 0));
  }
  // (c) the up weights: wave w takes output channels j0 + 16 (w & 3) + n over the
  // inputs 64 (w >> 2) .. + 63 -- K-step pairs 8 (w >> 2) + q, lane group g
  const int ct = wave & 3, kh = wave >> 2;
  uint4 wu[kDcUpSteps / 4];
  {
    const int JBu = (F + 31) >> 5, IPu = (d + 1) >> 1;
    const int jbu = (j0 >> 5) + (ct >> 1), cbu = ct & 1;
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(w_up) + ((size_t)e * JBu + min(jbu, JBu - 1)) * IPu * 512, (short)0,
        (uint32_t)IPu * 512, kBufferFlags);
#pragma unroll
    for (int q = 0; q < kDcUpSteps / 4; ++q) {
      const uint32_t off =
          jbu < JBu ? (uint32_t)(4 * (8 * kh + q) + g) * 512 + (uint32_t)(16 * cbu + n) * 16 : kBufferOff;
      wu[q] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, 0));
    }
  }

  // ---- 2. routing of the whole batch (every workgroup routes it; chunk 0 writes
  // this expert's part of the routing arrays)
  if (tid < kMaxExperts) s_cnt[tid] = 0;
#pragma unroll
  for (int ps = 0; ps < kDcSelPasses; ++ps) {
    if (ps * (kDcThreads / kSelLanes) < N) {
      const int t = ps * (kDcThreads / kSelLanes) + (tid >> 3);
      int se;
      float swt;
      select_from_logits<RQ>(lg[ps], E, k, t < N, sj, lane, se, swt);
      if (se >= 0) {
        s_sel[t * k + sj] = se;
        s_w[t * k + sj] = swt;
      }
    }
  }
  __syncthreads();
  for (int f = tid; f < N * k; f += kDcThreads) atomicAdd(&s_cnt[s_sel[f]], 1);
  bool mine = false;
  if (tid < N)
    for (int q = 0; q < k; ++q) mine |= s_sel[tid * k + q] == e;
  const uint64_t bal = __ballot(mine);
  if (lane == 0) s_wv[wave] = __popcll(bal);
  __syncthreads();
  if (mine) {
    int base = 0;
    for (int w = 0; w < wave; ++w) base += s_wv[w];
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    rows_tok[base + __popcll(bal & lt)] = tid;
  }
  // this expert's rows start after those of the experts before it (E <= 64: one lane each)
  const int n_e = s_cnt[e], row_beg = dc_wave_sum(lane < e ? s_cnt[lane] : 0);
  __syncthreads();
  // the routing arrays of this expert's slots, for the combine and the caller: written
  // by chunk 0 once its loads are all in (its loop would otherwise wait for them early)
  auto write_routing = [&]() {
    if (c != 0) return;
    for (int r = tid; r < n_e; r += kDcThreads) {
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
    write_routing();
    return;
  }

  // ---- 3. the input rows of the first batch (load l: token 4 l + tid / 128, input
  // tid % 128), then the down weights: wave w takes outputs 16 w + n over the
  // chunk's inputs (K-step pairs q, lane group g)
  const int xi = tid & 127, xt = tid >> 7;
  const __amdgpu_buffer_rsrc_t x_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(x), (short)0, (uint32_t)N * d * 16, kBufferFlags);
  uint4 xr[kDcBatch / 4];
#pragma unroll
  for (int l = 0; l < kDcBatch / 4; ++l) {
    const int tk = 4 * l + xt;
    const uint32_t off = (tk < n_e && xi < d) ? (uint32_t)(rows_tok[tk] * d + xi) * 16 : kBufferOff;
    xr[l] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(x_rsrc, off, 0, 0));
  }
  uint4 wd[kDcDnSteps / 2];
  {
    const int JBd = (d + 31) >> 5, IPd = (F + 1) >> 1;
    const int jb = wave >> 1, cbd = wave & 1;
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(w_dn) + ((size_t)e * JBd + min(jb, JBd - 1)) * IPd * 512, (short)0,
        (uint32_t)IPd * 512, kBufferFlags);
#pragma unroll
    for (int q = 0; q < kDcDnSteps / 2; ++q) {
      const uint32_t off =
          jb < JBd ? (uint32_t)((j0 >> 1) + 4 * q + g) * 512 + (uint32_t)(16 * cbd + n) * 16 : kBufferOff;
      wd[q] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, 0));
    }
  }

  // bf16 rows (blade order) -> fp16 packed mask order, scaled per token (each
  // token's row spans two waves: the largest magnitude goes through LDS)
  uint4 xh[kDcBatch / 4] = {};
  auto convert_x = [&](int nb) {
#pragma unroll
    for (int l = 0; l < kDcBatch / 4; ++l) {
      if (4 * l >= nb) break;  // uniform: no token of the batch in this load
      const uint32_t wv[4] = {xr[l].x, xr[l].y, xr[l].z, xr[l].w};
      float m = 0.f;
#pragma unroll
      for (int u = 0; u < 4; ++u)
        m = fmaxf(m, fmaxf(fabsf(bf16_bits_to_f32((uint16_t)(wv[u] & 0xffffu))),
                           fabsf(bf16_bits_to_f32((uint16_t)(wv[u] >> 16)))));
      m = dc_wave_max(m);
      if (lane == 0) s_xmax[4 * l + xt][wave & 1] = m;
    }
    __syncthreads();
#pragma unroll
    for (int l = 0; l < kDcBatch / 4; ++l) {
      if (4 * l >= nb) break;
      const int tk = 4 * l + xt;
      const int sh = dc_shift(fmaxf(s_xmax[tk][0], s_xmax[tk][1]));
      const float sc = ldexpf(1.0f, sh);
      if (xi == 0) s_xinv[tk] = ldexpf(1.0f, -sh);
      const uint32_t wv[4] = {xr[l].x, xr[l].y, xr[l].z, xr[l].w};
      float b[8];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        b[2 * u] = bf16_bits_to_f32((uint16_t)(wv[u] & 0xffffu));
        b[2 * u + 1] = bf16_bits_to_f32((uint16_t)(wv[u] >> 16));
      }
      xh[l] = make_uint4(dc_pack_f16(b[mask_to_blade(0)] * sc, b[mask_to_blade(1)] * sc),
                         dc_pack_f16(b[mask_to_blade(2)] * sc, b[mask_to_blade(3)] * sc),
                         dc_pack_f16(b[mask_to_blade(4)] * sc, b[mask_to_blade(5)] * sc),
                         dc_pack_f16(b[mask_to_blade(6)] * sc, b[mask_to_blade(7)] * sc));
    }
  };
  convert_x(min(kDcBatch, n_e));

  for (int b0 = 0; b0 < n_e; b0 += kDcBatch) {
    if (b0 > 0) {  // a later batch: its rows load behind everything else
      __syncthreads();  // the previous batch's LDS readers are done
#pragma unroll
      for (int l = 0; l < kDcBatch / 4; ++l) {
        const int tk = b0 + 4 * l + xt;
        const uint32_t off = (tk < n_e && xi < d) ? (uint32_t)(rows_tok[tk] * d + xi) * 16 : kBufferOff;
        xr[l] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(x_rsrc, off, 0, 0));
      }
      convert_x(min(kDcBatch, n_e - b0));
    }
    const int nb = min(kDcBatch, n_e - b0);
    // the up weights as fp16 B fragments, converted once for all passes of the batch
    dc_f16x8_t bu16[kDcUpSteps / 2];
#pragma unroll
    for (int q = 0; q < kDcUpSteps / 4; ++q) {
      const uint4 wq = dc_pin(wu[q]);
      bu16[2 * q] = dc_codes_to_f16(wq.x, wq.y);
      bu16[2 * q + 1] = dc_codes_to_f16(wq.z, wq.w);
    }

    // ---- 4. up passes of 4 tokens -> hidden rows (fp32) of the batch in LDS
    for (int p = 0; p * kDcUpTok < nb; ++p) {  // uniform; one copy of the pass's code
      {
        const int nt = min(kDcUpTok, nb - p * kDcUpTok);
        // expanded operand: token xt of the pass (row block xt / 2, rows (xt % 2) 8 + r), input xi
        dc_expand(xh[0], &a_op[(xt >> 1) * (kDcUpSteps * kDcStep) + dc_in_slot(xi, (xt & 1) * 8)]);
#pragma unroll
        for (int l = 0; l + 1 < kDcBatch / 4; ++l) xh[l] = xh[l + 1];  // the next pass's rows move up
        __syncthreads();
        // both row blocks over all 16 K steps of this wave's half: past d (or past the
        // pass's tokens) the operand is zero, and straight-line code keeps the MFMA chain
        // free of branches (the full unroll keeps the weight registers statically indexed)
        dc_f32x4_t acc[2] = {dc_f32x4_t{0.f, 0.f, 0.f, 0.f}, dc_f32x4_t{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int st = 0; st < kDcUpSteps / 2; ++st) {
          const int gst = (kDcUpSteps / 2) * kh + st;
#pragma unroll
          for (int rb = 0; rb < 2; ++rb) {
            const dc_f16x8_t A = __builtin_bit_cast(dc_f16x8_t, a_op[rb * (kDcUpSteps * kDcStep) + dc_slot(gst, g, n)]);
            acc[rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, bu16[st], acc[rb], 0, 0, 0);
          }
        }
        // lane holds rows 4 g + v of each block: token 2 rb + g / 2, mask blades 4 (g % 2) + v
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
          c_up[kh][2 * rb + (g >> 1)][g & 1][16 * ct + n] = make_float4(acc[rb][0], acc[rb][1], acc[rb][2], acc[rb][3]);
        __syncthreads();
        if (wave < kDcUpTok) {  // epilogue: token `wave` of the pass, channel ju
          const int tk = p * kDcUpTok + wave;
          const float xs = s_xinv[tk];
          const float4 a0 = c_up[0][wave][0][lane], a1 = c_up[0][wave][1][lane];
          const float4 h0 = c_up[1][wave][0][lane], h1 = c_up[1][wave][1][lane];
          float hv[8] = {a0.x + h0.x, a0.y + h0.y, a0.z + h0.z, a0.w + h0.w,
                         a1.x + h1.x, a1.y + h1.y, a1.z + h1.z, a1.w + h1.w};
#pragma unroll
          for (int r = 0; r < 8; ++r) hv[r] = hv[r] * xs * su + bu[r];
          dc_activate<ACT>(hv);
          const bool ok = wave < nt && ju < F;
          float m = 0.f;
#pragma unroll
          for (int r = 0; r < 8; ++r) {
            hv[r] = ok ? hv[r] : 0.f;
            m = fmaxf(m, fabsf(hv[r]));
          }
          m = dc_wave_max(m);
          if (lane == 0) s_hmax[tk] = m;
          h_st[tk][0][lane] = make_float4(hv[0], hv[1], hv[2], hv[3]);
          h_st[tk][1][lane] = make_float4(hv[4], hv[5], hv[6], hv[7]);
        }
      }
    }
    __syncthreads();  // the batch's hidden rows are complete
    // the down weights as fp16 B fragments (the first use of the down weights: the
    // wait for them falls here, after the up passes)
    dc_f16x8_t bd16[kDcDnSteps];
#pragma unroll
    for (int q = 0; q < kDcDnSteps / 2; ++q) {
      const uint4 wq = dc_pin(wd[q]);
      bd16[2 * q] = dc_codes_to_f16(wq.x, wq.y);
      bd16[2 * q + 1] = dc_codes_to_f16(wq.z, wq.w);
    }

    // ---- 5. down passes of 8 tokens -> fp32 partial plane c
    for (int q0 = 0; q0 < nb; q0 += kDcDnTok) {
      const int nt = min(kDcDnTok, nb - q0), nrt = (nt + 1) >> 1;
      {  // expanded operand: token `wave` of the pass, hidden channel `lane`
        const int tk = q0 + wave;
        const bool ok = wave < nt;
        const float4 h0 = h_st[tk][0][lane], h1 = h_st[tk][1][lane];
        const float sc = ldexpf(1.0f, dc_shift(s_hmax[tk]));
        const uint4 hv = ok ? make_uint4(dc_pack_f16(h0.x * sc, h0.y * sc), dc_pack_f16(h0.z * sc, h0.w * sc),
                                         dc_pack_f16(h1.x * sc, h1.y * sc), dc_pack_f16(h1.z * sc, h1.w * sc))
                            : make_uint4(0u, 0u, 0u, 0u);
        dc_expand(hv, &a_op[(wave >> 1) * (kDcDnSteps * kDcStep) + dc_in_slot(lane, (wave & 1) * 8)]);
      }
      __syncthreads();
      dc_f32x4_t acc[4];
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) acc[rb] = dc_f32x4_t{0.f, 0.f, 0.f, 0.f};
      // uniform: a branch-free MFMA chain over 2 or 4 row blocks (the rows past the
      // pass's tokens are zero)
      if (nrt <= 2) dc_down_mfma<2>(bd16, a_op, g, n, acc);
      else dc_down_mfma<4>(bd16, a_op, g, n, acc);
      // epilogue: lane holds token 2 rb + g / 2, mask blades 4 (g % 2) + v of output od;
      // lanes g and g ^ 1 trade one value so that each holds four blade-order components
      // (blades 0-3 = mask 0, 1, 2, 4; blades 4-7 = mask 3, 5, 6, 7)
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        if (rb < nrt) {
          const int tk = q0 + 2 * rb + (g >> 1);
          const float hs = ldexpf(1.0f, -dc_shift(s_hmax[tk]));
          float y[4] = {acc[rb][0], acc[rb][1], acc[rb][2], acc[rb][3]};
          const float bb[4] = {bd.x, bd.y, bd.z, bd.w};
#pragma unroll
          for (int v = 0; v < 4; ++v) y[v] = y[v] * hs * sd + bb[v];
          const float recv = __shfl_xor((g & 1) ? y[0] : y[3], 16);
          const float4 o4 = (g & 1) ? make_float4(recv, y[1], y[2], y[3]) : make_float4(y[0], y[1], y[2], recv);
          if (tk - q0 < nt && od < d)
            *reinterpret_cast<float4*>(planes + (((size_t)c * P_max + row_beg + b0 + tk) * d + od) * 8 + (g & 1) * 4) = o4;
        }
      }
      __syncthreads();  // the staging area is free for the next pass
    }
  }
  write_routing();
}

}  // namespace ygg

using namespace ygg;

bool ygg::decode_layer_fusable(int N, int E, int k, int d, int F) {
  return N >= 1 && N <= kDcMaxTokens && E >= 1 && E <= kMaxExperts && k >= 1 && k <= kMaxTopK && k <= E && d >= 1 &&
         d <= kDcMaxD && F >= 1;
}

int ygg::decode_layer_planes(int F) { return (F + kDcChunk - 1) / kDcChunk; }

template <int ACT, int RQ>
static void launch_dc(dim3 grid, hipStream_t st, const uint16_t* x, const DcRoute& rt, const int8_t* wu,
                      const float* su, const float* bu, const int8_t* wd, const float* sd, const float* bd, int d,
                      int F, int P_max, float* planes) {
  decode_layer_kernel<ACT, RQ><<<grid, kDcThreads, 0, st>>>(x, rt, wu, su, bu, wd, sd, bd, d, F, P_max, planes);
}

int ygg::decode_layer(const uint16_t* x, const float* logits, int N, int E, int k, int d, int F, int act,
                      const int8_t* w_up, const float* s_up, const float* b_up, const int8_t* w_dn,
                      const float* s_dn, const float* b_dn, int32_t* topk_idx, float* topk_w, int32_t* counts,
                      int32_t* offsets, int32_t* perm, int32_t* slot_pos, float* planes, hipStream_t stream) {
  YGG_CHECK_ARG(decode_layer_fusable(N, E, k, d, F), "decode layer: N=%d E=%d k=%d d=%d F=%d outside its limits", N,
                E, k, d, F);
  YGG_CHECK_ARG(act >= kActNone && act <= kActSigmoid, "decode layer: activation %d", act);
  const DcRoute rt{logits, N, E, k, topk_idx, topk_w, counts, offsets, perm, slot_pos};
  const dim3 grid(E, decode_layer_planes(F));
  const int P_max = N * k;
#define YGG_DC(A)                                                                                          \
  ((E <= 32) ? launch_dc<A, 4>(grid, stream, x, rt, w_up, s_up, b_up, w_dn, s_dn, b_dn, d, F, P_max, planes) \
             : launch_dc<A, 8>(grid, stream, x, rt, w_up, s_up, b_up, w_dn, s_dn, b_dn, d, F, P_max, planes))
  switch (act) {
    case kActNone: YGG_DC(kActNone); break;
    case kActGelu: YGG_DC(kActGelu); break;
    case kActRelu: YGG_DC(kActRelu); break;
    default: YGG_DC(kActSigmoid); break;
  }
#undef YGG_DC
  return check_launch("decode_layer");
}
