// route_select.h -- the per-token routing selection (CliffordRouter's softmax,
// top-k and renormalisation, clifford_router.py:18-21,54-104), eight lanes per
// token (and one token per thread), shared by the routing kernels (route.hip) and
// the up products that route inside their own workgroups (clifford_gemm.hip,
// pauli_f32.hip).
#pragma once

#include "ygg_common.h"

namespace ygg {

// Exchange within the 8-lane token groups by DPP (a register move, no LDS round
// trip): step 0 pairs lanes i and i^1, step 1 lanes i and i^2 (quad permutes),
// step 2 lanes i and 7-i of each half row (row_half_mirror), which joins the two
// quads of a group as i^4 would.  After the three steps of a reduction every
// lane holds the same result; for sums that is the tree ((r0+r1)+(r2+r3)) +
// ((r4+r5)+(r6+r7)) exactly, as each addition only sees its operands swapped.
template <int STEP>
__device__ inline int grp_xchg(int v) {
  constexpr int ctrl = STEP == 0 ? 0xB1 : STEP == 1 ? 0x4E : 0x141;
  return __builtin_amdgcn_update_dpp(0, v, ctrl, 0xF, 0xF, false);
}
template <int STEP>
__device__ inline float grp_xchg(float v) {
  return __builtin_bit_cast(float, grp_xchg<STEP>(__builtin_bit_cast(int, v)));
}
template <int STEP>
__device__ inline uint64_t grp_xchg64(uint64_t v) {
  const uint32_t lo = (uint32_t)grp_xchg<STEP>((int)(uint32_t)v);
  const uint32_t hi = (uint32_t)grp_xchg<STEP>((int)(uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}

constexpr int kMaxExperts = 64;
constexpr int kMaxTopK = 8;
constexpr int kSelLanes = 8;                          // lanes per token

// The logits of one token straight from its activation row (the reference's
// CliffordRouter energy signature, clifford_router.py:54-90): per-grade sums of
// squares over the row (lane j takes multivectors j, j + 8, ...; the eight lanes
// of the token are combined by a DPP tree), normalised by their sum + 1e-12,
// then the (E, 4) map and bias.  Lane j returns the logits of experts j + 8 q.
template <int Q>
__device__ inline void energy_logits(const void* __restrict__ x, int x_dtype, int d, const float* __restrict__ rw,
                                     const float* __restrict__ rb, int E, int t, bool active, int j, float (&p)[Q]) {
  float gs[4] = {0.f, 0.f, 0.f, 0.f};
  if (active) {
    for (int i = j; i < d; i += kSelLanes) {
      float v[8];
      if (x_dtype == kF32) {
        const float4* q4 = reinterpret_cast<const float4*>(static_cast<const float*>(x) + ((size_t)t * d + i) * 8);
        const float4 a = q4[0], b = q4[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
      } else {
        const uint4 q = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + ((size_t)t * d + i) * 8);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          v[2 * c] = bf16_bits_to_f32((uint16_t)(w[c] & 0xffff));
          v[2 * c + 1] = bf16_bits_to_f32((uint16_t)(w[c] >> 16));
        }
      }
      gs[0] += v[0] * v[0];
      gs[1] += v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
      gs[2] += v[4] * v[4] + v[5] * v[5] + v[6] * v[6];
      gs[3] += v[7] * v[7];
    }
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    gs[c] += grp_xchg<0>(gs[c]);
    gs[c] += grp_xchg<1>(gs[c]);
    gs[c] += grp_xchg<2>(gs[c]);
  }
  const float tot = gs[0] + gs[1] + gs[2] + gs[3] + 1e-12f;
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const int e = j + kSelLanes * q;
    float l = -INFINITY;
    if (active && e < E) {
      l = 0.f;
#pragma unroll
      for (int c = 0; c < 4; ++c) l += (gs[c] / tot) * rw[e * 4 + c];
      l += rb[e];
    }
    p[q] = l;
  }
}

// The top-k of one token, eight lanes per token (lane j = tid % 8), from its
// logits p (lane j: experts j + 8 q, -inf past E or for an inactive token):
// probabilities and top-k; lane j returns slot j (expert, probability), or
// expert -1 for j >= k or an inactive token.  select_from_logits adds the
// renormalised weights.
template <int Q>  // Q >= ceil(E / 8) logits per lane (-inf past E)
__device__ inline void select_topk_raw(float (&p)[Q], int E, int k, bool active, int j, int lane, int& out_e,
                                       float& out_raw) {
  // ---- probabilities (the reference's fp32 softmax, clifford_router.py:18-21)
  float m = -INFINITY;
#pragma unroll
  for (int q = 0; q < Q; ++q) m = fmaxf(m, p[q]);
  m = fmaxf(m, grp_xchg<0>(m));
  m = fmaxf(m, grp_xchg<1>(m));
  m = fmaxf(m, grp_xchg<2>(m));
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const int e = j + kSelLanes * q;
    p[q] = (e < E) ? expf(__fsub_rn(p[q], m)) : 0.f;
  }
  // NumPy pairwise sum of the row: rows of fewer than 8 values are summed in
  // order; otherwise accumulator j sums the elements j, j+8, ... below
  // E8 = E - E % 8, the eight accumulators are combined as a tree and the
  // remaining E % 8 values are added in order.
  const int E8 = E - (E & 7);
  float sum;
  if (E < 8) {
    sum = 0.f;
    for (int e = 0; e < E; ++e) sum = __fadd_rn(sum, __shfl(p[0], (lane & ~7) + e));
  } else {
    float r = p[0];
#pragma unroll
    for (int q = 1; q < Q; ++q)
      if (j + kSelLanes * q < E8) r = __fadd_rn(r, p[q]);
    r = __fadd_rn(r, grp_xchg<0>(r));
    r = __fadd_rn(r, grp_xchg<1>(r));
    r = __fadd_rn(r, grp_xchg<2>(r));
    sum = r;
    // the remaining E % 8 values are element E / 8 of lanes 0 .. E % 8 - 1 (any Q >= ceil(E / 8))
    float prem = p[0];
#pragma unroll
    for (int q = 1; q < Q; ++q)
      if (q == (E >> 3)) prem = p[q];
    for (int e = E8; e < E; ++e) sum = __fadd_rn(sum, __shfl(prem, (lane & ~7) + (e & 7)));
  }
  const float denom = __fadd_rn(sum, 1e-12f);
#pragma unroll
  for (int q = 0; q < Q; ++q) p[q] = __fdiv_rn(p[q], denom);

  // ---- top-k: k rounds of (max probability, then min index) over the 8 lanes,
  // without branches.  Each candidate is one 64-bit key, (probability bits + 1)
  // << 32 | (63 - expert): probabilities are >= 0, so their bit patterns order
  // as the values do, and among equal probabilities the lower index has the
  // larger key.  A NaN probability keeps 0 in the upper half (below every real
  // probability, so the order is total and every slot gets a valid expert; its
  // weight is unspecified), padding experts and taken candidates are 0.
  uint64_t key[Q];
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const int e = j + kSelLanes * q;
    const uint64_t hi = (p[q] == p[q]) ? (uint64_t)(__builtin_bit_cast(uint32_t, p[q]) + 1u) << 32 : 0ull;
    key[q] = (e < E) ? (hi | (uint64_t)(63 - e)) : 0ull;
  }
  // a rolled loop: lane j keeps round j's winner (its slot), so no per-slot arrays
  int my_e = -1;  // lane j holds slot j
  float my_raw = 0.f;
#pragma unroll 1
  for (int s = 0; s < k; ++s) {
    uint64_t best = key[0];
#pragma unroll
    for (int q = 1; q < Q; ++q) best = key[q] > best ? key[q] : best;
    uint64_t o = grp_xchg64<0>(best);
    best = o > best ? o : best;
    o = grp_xchg64<1>(best);
    best = o > best ? o : best;
    o = grp_xchg64<2>(best);
    best = o > best ? o : best;
    // k <= E: at least one candidate remains, so the winner is a valid expert
    const uint32_t bhi = (uint32_t)(best >> 32);
    my_e = (s == j) ? 63 - (int)(best & 63ull) : my_e;
    my_raw = (s == j) ? (bhi ? __builtin_bit_cast(float, bhi - 1u) : -1.0f) : my_raw;
#pragma unroll
    for (int q = 0; q < Q; ++q) key[q] = key[q] == best ? 0ull : key[q];
  }
  out_e = active ? my_e : -1;
  out_raw = my_raw;
}

// The renormalised weight of slot j (lanes j < k of the token's 8 hold the slots'
// probabilities `raw`; every lane of the wave takes part): the sum runs from the
// least to the most probable slot (lane k-1 down to 0), then + 1e-12.
__device__ inline float renorm_slot(float raw, int k, int j, int lane) {
  float ssum = 0.f;
  for (int s = k - 1; s >= 0; --s) ssum = __fadd_rn(ssum, __shfl(raw, (lane & ~(kSelLanes - 1)) + s));
  ssum = __fadd_rn(ssum, 1e-12f);
  return (j < k) ? __fdiv_rn(raw, ssum) : 0.f;
}

// select_topk_raw, then the renormalised weights: lane j returns slot j (expert, weight).
template <int Q>
__device__ inline void select_from_logits(float (&p)[Q], int E, int k, bool active, int j, int lane, int& out_e,
                                          float& out_w) {
  float raw;
  select_topk_raw<Q>(p, E, k, active, j, lane, out_e, raw);
  out_w = renorm_slot(raw, k, j, lane);
}

// select_from_logits for one token in one thread (its E <= EMAX logits in p): the
// same operations in the same order -- the row maximum, the exponentials, the sum as
// the eight-lane tree forms it (E >= 8: accumulator j over elements j, j + 8, ...
// below E - E % 8, then ((a0 + a1) + (a2 + a3)) + ((a4 + a5) + (a6 + a7)), then the
// remaining E % 8 elements in order; fewer than 8 elements in order), the
// probabilities, k rounds of the (probability, lower index) maximum, and the
// renormalisation from the least probable slot -- so the experts and weights equal
// the eight-lane version's bit for bit.  Slot s < k -> out_e[s], out_w[s].
template <int EMAX>
__device__ inline void select_one_thread(float (&p)[EMAX], int E, int k, int (&out_e)[kMaxTopK],
                                         float (&out_w)[kMaxTopK]) {
  float m = -INFINITY;
#pragma unroll
  for (int e = 0; e < EMAX; ++e) m = e < E ? fmaxf(m, p[e]) : m;
#pragma unroll
  for (int e = 0; e < EMAX; ++e) p[e] = e < E ? expf(__fsub_rn(p[e], m)) : 0.f;
  float sum;
  if (E < 8) {
    sum = 0.f;
#pragma unroll
    for (int e = 0; e < EMAX && e < 8; ++e)
      if (e < E) sum = __fadd_rn(sum, p[e]);
  } else {
    const int E8 = E - (E & 7);
    float a[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float r = p[j];
#pragma unroll
      for (int e = j + 8; e < EMAX; e += 8)
        if (e < E8) r = __fadd_rn(r, p[e]);
      a[j] = r;
    }
    sum = __fadd_rn(__fadd_rn(__fadd_rn(a[0], a[1]), __fadd_rn(a[2], a[3])),
                    __fadd_rn(__fadd_rn(a[4], a[5]), __fadd_rn(a[6], a[7])));
#pragma unroll
    for (int e = 8; e < EMAX; ++e)
      if (e >= E8 && e < E) sum = __fadd_rn(sum, p[e]);
  }
  const float denom = __fadd_rn(sum, 1e-12f);
  uint64_t key[EMAX];  // as in select_topk_raw
#pragma unroll
  for (int e = 0; e < EMAX; ++e) {
    const float pr = __fdiv_rn(p[e], denom);
    const uint64_t hi = (pr == pr) ? (uint64_t)(__builtin_bit_cast(uint32_t, pr) + 1u) << 32 : 0ull;
    key[e] = (e < E) ? (hi | (uint64_t)(63 - e)) : 0ull;
  }
  float raw[kMaxTopK];
#pragma unroll
  for (int s = 0; s < kMaxTopK; ++s) {
    out_e[s] = -1;
    raw[s] = 0.f;
    if (s < k) {
      uint64_t best = key[0];
#pragma unroll
      for (int e = 1; e < EMAX; ++e) best = key[e] > best ? key[e] : best;
      const uint32_t bhi = (uint32_t)(best >> 32);
      out_e[s] = 63 - (int)(best & 63ull);
      raw[s] = bhi ? __builtin_bit_cast(float, bhi - 1u) : -1.0f;
#pragma unroll
      for (int e = 0; e < EMAX; ++e) key[e] = key[e] == best ? 0ull : key[e];
    }
  }
  float ssum = 0.f;
#pragma unroll
  for (int s = kMaxTopK - 1; s >= 0; --s)
    if (s < k) ssum = __fadd_rn(ssum, raw[s]);
  ssum = __fadd_rn(ssum, 1e-12f);
#pragma unroll
  for (int s = 0; s < kMaxTopK; ++s) out_w[s] = s < k ? __fdiv_rn(raw[s], ssum) : 0.f;
}

template <int Q>
__device__ inline void select_token(const float* __restrict__ logits, int E, int k, int t, bool active, int j,
                                    int lane, int& out_e, float& out_w) {
  float p[Q];
  const float* row = logits + (size_t)(active ? t : 0) * E;
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const int e = j + kSelLanes * q;
    p[q] = (active && e < E) ? row[e] : -INFINITY;
  }
  select_from_logits<Q>(p, E, k, active, j, lane, out_e, out_w);
}

}  // namespace ygg
