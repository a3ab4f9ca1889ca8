// dispatch.hip -- token dispatch (gather into expert-grouped rows) and the
// weighted combine, gfx950.
//
// Replaces hlm_block.py:178 (expert_input = flat_x[token_ids]) and
// hlm_block.py:180-181 (weighted = w * y; np.add.at(output, token_ids, ...)).
//
// Dispatch is token-driven: one wave reads a token's row once (coalesced
// 16-byte loads) and writes it to its k sorted positions, so x is read once
// (N*R bytes) and the sorted buffer written once (N*k*R bytes).  Optionally
// the two components e3/e12 are exchanged on the way, producing the "mask
// order" the expert products consume.
//
// Combine is gather-based and atomic-free: one wave per token reads its k
// rows and adds  w_s * y_s  in ascending expert order, each product rounded
// before its add (no fused multiply-add) -- the order and rounding of
// np.add.at called once per expert in ascending order.  Optionally a
// residual is added last (hlm_block.py:151, x + ffn_out).

#include "ygg_common.h"

namespace ygg {

// --- one multivector in registers ---------------------------------------
struct MV {
  float v[8];
};

template <int DT>
__device__ inline MV load_mv(const void* base, size_t mv_index) {
  MV m;
  if constexpr (DT == kF32) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(base) + mv_index * 8);
    const float4 a = p[0], b = p[1];
    m.v[0] = a.x; m.v[1] = a.y; m.v[2] = a.z; m.v[3] = a.w;
    m.v[4] = b.x; m.v[5] = b.y; m.v[6] = b.z; m.v[7] = b.w;
  } else {
    const uint4 q = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + mv_index * 8);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      m.v[2 * c] = bf16_bits_to_f32((uint16_t)(w[c] & 0xffff));
      m.v[2 * c + 1] = bf16_bits_to_f32((uint16_t)(w[c] >> 16));
    }
  }
  return m;
}

template <int DT>
__device__ inline void store_mv(void* base, size_t mv_index, const MV& m) {
  if constexpr (DT == kF32) {
    float4* p = reinterpret_cast<float4*>(static_cast<float*>(base) + mv_index * 8);
    p[0] = make_float4(m.v[0], m.v[1], m.v[2], m.v[3]);
    p[1] = make_float4(m.v[4], m.v[5], m.v[6], m.v[7]);
  } else {
    uint4 q;
    q.x = pack_bf16x2(m.v[0], m.v[1]);
    q.y = pack_bf16x2(m.v[2], m.v[3]);
    q.z = pack_bf16x2(m.v[4], m.v[5]);
    q.w = pack_bf16x2(m.v[6], m.v[7]);
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(base) + mv_index * 8) = q;
  }
}

// Raw 16/32-byte multivector copy (no conversion), optional e3<->e12 swap.
template <int DT>
struct RawMV {
  uint4 a, b;  // b unused for bf16
};

template <int DT, bool SWAP34>
__device__ inline RawMV<DT> load_raw(const void* base, size_t mv_index) {
  RawMV<DT> r;
  if constexpr (DT == kF32) {
    const uint4* p = reinterpret_cast<const uint4*>(static_cast<const float*>(base) + mv_index * 8);
    r.a = p[0];
    r.b = p[1];
    if constexpr (SWAP34) {  // components 3 (a.w) and 4 (b.x)
      const uint32_t t = r.a.w;
      r.a.w = r.b.x;
      r.b.x = t;
    }
  } else {
    r.a = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + mv_index * 8);
    if constexpr (SWAP34) {  // component 3 = hi half of dword 1, component 4 = lo half of dword 2
      const uint32_t d1 = r.a.y, d2 = r.a.z;
      r.a.y = (d1 & 0xffffu) | (d2 << 16);
      r.a.z = (d1 >> 16) | (d2 & 0xffff0000u);
    }
  }
  return r;
}

template <int DT>
__device__ inline void store_raw(void* base, size_t mv_index, const RawMV<DT>& r) {
  if constexpr (DT == kF32) {
    uint4* p = reinterpret_cast<uint4*>(static_cast<float*>(base) + mv_index * 8);
    p[0] = r.a;
    p[1] = r.b;
  } else {
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(base) + mv_index * 8) = r.a;
  }
}

constexpr int kTokPerBlock = 4;  // one wave per token
constexpr int kDispU = 4;        // multivectors per lane per dispatch round

template <int DT, bool TO_MASK>
__global__ __launch_bounds__(256) void dispatch_kernel(const void* __restrict__ x, int N, int k, int d,
                                                       const int32_t* __restrict__ slot_pos,
                                                       void* __restrict__ xs) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * kTokPerBlock + (threadIdx.x >> 6);
  if (t >= N) return;
  int dst[8];  // slots past k repeat the last one (unconditional loads: one round trip)
#pragma unroll
  for (int s = 0; s < 8; ++s) dst[s] = slot_pos[(size_t)t * k + min(s, k - 1)];
  // kDispU multivectors per lane are loaded before any is stored, so a wave
  // keeps that many 16/32-byte reads in flight instead of one
  for (int i0 = lane; i0 < d; i0 += 64 * kDispU) {
    RawMV<DT> r[kDispU];
#pragma unroll
    for (int u = 0; u < kDispU; ++u)
      if (i0 + 64 * u < d) r[u] = load_raw<DT, TO_MASK>(x, (size_t)t * d + i0 + 64 * u);
#pragma unroll
    for (int s = 0; s < 8; ++s)
      if (s < k) {
#pragma unroll
        for (int u = 0; u < kDispU; ++u)
          if (i0 + 64 * u < d) store_raw<DT>(xs, (size_t)dst[s] * d + i0 + 64 * u, r[u]);
      }
  }
}

// Compare-exchange of slots i < j by expert (slot j ends with the larger), as value
// selects: the slot arrays stay in registers and no lane branches.
template <int KM>
__device__ __forceinline__ void slot_cx(int (&ex)[KM], int (&row)[KM], float (&w)[KM], int i, int j) {
  const bool sw = ex[j] < ex[i];
  const int e0 = sw ? ex[j] : ex[i], e1 = sw ? ex[i] : ex[j];
  const int r0 = sw ? row[j] : row[i], r1 = sw ? row[i] : row[j];
  const float w0 = sw ? w[j] : w[i], w1 = sw ? w[i] : w[j];
  ex[i] = e0; ex[j] = e1;
  row[i] = r0; row[j] = r1;
  w[i] = w0; w[j] = w1;
}
// The slots in ascending expert order: sorting networks for 2, 4 and 8 slots (the
// experts of a token are distinct; unused slots carry the largest key and sort last)
template <int KM>
__device__ __forceinline__ void sort_slots(int (&ex)[KM], int (&row)[KM], float (&w)[KM]) {
  static_assert(KM == 2 || KM == 4 || KM == 8, "slot network");
  if constexpr (KM == 2) {
    slot_cx<KM>(ex, row, w, 0, 1);
  } else if constexpr (KM == 4) {
    constexpr int net[5][2] = {{0, 1}, {2, 3}, {0, 2}, {1, 3}, {1, 2}};
#pragma unroll
    for (int q = 0; q < 5; ++q) slot_cx<KM>(ex, row, w, net[q][0], net[q][1]);
  } else {  // Batcher's odd-even merge sort of 8
    constexpr int net[19][2] = {{0, 1}, {2, 3}, {4, 5}, {6, 7}, {0, 2}, {1, 3}, {4, 6}, {5, 7}, {1, 2}, {5, 6},
                                {0, 4}, {1, 5}, {2, 6}, {3, 7}, {2, 4}, {3, 5}, {1, 2}, {3, 4}, {5, 6}};
#pragma unroll
    for (int q = 0; q < 19; ++q) slot_cx<KM>(ex, row, w, net[q][0], net[q][1]);
  }
}

// KM: the slots a token can have, k <= KM (2, 4 or 8)
template <int YT, bool Y_MASK, int OT, bool RESID, int KM>
__global__ __launch_bounds__(256) void combine_kernel(const void* __restrict__ ys, int N, int k, int d,
                                                      const int32_t* __restrict__ topk_idx,
                                                      const float* __restrict__ topk_w,
                                                      const int32_t* __restrict__ slot_pos,
                                                      const void* __restrict__ resid, void* __restrict__ out) {
  // every product is rounded before its add, as in the reference: no contraction to fma
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * kTokPerBlock + (threadIdx.x >> 6);
  if (t >= N) return;
  int ex[KM], row[KM];
  float w[KM];
#pragma unroll
  for (int s = 0; s < KM; ++s) {  // unconditional loads (slots past k repeat the last one), then masked
    const size_t f = (size_t)t * k + min(s, k - 1);
    const int e = topk_idx[f], rw = slot_pos[f];
    const float ws = topk_w[f];
    const bool on = s < k;
    ex[s] = on ? e : 0x7fffffff;
    row[s] = on ? rw : 0;
    w[s] = on ? ws : 0.f;
  }
  sort_slots<KM>(ex, row, w);  // ascending expert order
  // bf16 rows, KM <= 4: the rows of the KM slots loaded raw and unconditionally (a slot
  // past k repeats the last row: a cache hit), all in flight before the first is used --
  // a load inside `if (s < k)` is waited for inside its branch, one round trip per slot.
  // Same products and adds, in the same order, as the loop below.
  if constexpr (YT == kBF16 && KM <= 4) {  // (fp32 rows: measured no faster, the loop below serves them)
    int rs[KM];
    const int last = row[0];
#pragma unroll
    for (int s = 0; s < KM; ++s) {
      int rl = last;  // row[k - 1] without indexing the register array
#pragma unroll
      for (int q = 1; q < KM; ++q)
        if (q == k - 1) rl = row[q];
      rs[s] = s < k ? row[s] : rl;
    }
    // two multivectors per lane per round (i and i + 64): every row load of both is in
    // flight before the first is used (past d the second repeats the first, not stored)
    for (int i0 = lane; i0 < d; i0 += 128) {
      const int i1 = i0 + 64 < d ? i0 + 64 : i0;
      RawMV<YT> y[2][KM];
#pragma unroll
      for (int s = 0; s < KM; ++s) {
        y[0][s] = load_raw<YT, false>(ys, (size_t)rs[s] * d + i0);
        y[1][s] = load_raw<YT, false>(ys, (size_t)rs[s] * d + i1);
      }
      MV r[2];
      if constexpr (RESID) {
        r[0] = load_mv<OT>(resid, (size_t)t * d + i0);
        r[1] = load_mv<OT>(resid, (size_t)t * d + i1);
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        MV acc;
#pragma unroll
        for (int c = 0; c < 8; ++c) acc.v[c] = 0.f;
#pragma unroll
        for (int s = 0; s < KM; ++s) {
          float v[8];
          const uint32_t u[4] = {y[h][s].a.x, y[h][s].a.y, y[h][s].a.z, y[h][s].a.w};
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            v[2 * c] = bf16_bits_to_f32((uint16_t)(u[c] & 0xffff));
            v[2 * c + 1] = bf16_bits_to_f32((uint16_t)(u[c] >> 16));
          }
#pragma unroll
          for (int c = 0; c < 8; ++c) acc.v[c] = s < k ? acc.v[c] + w[s] * v[c] : acc.v[c];
        }
        if constexpr (Y_MASK) {  // back to blade order
          const float t3 = acc.v[3];
          acc.v[3] = acc.v[4];
          acc.v[4] = t3;
        }
        if constexpr (RESID) {
#pragma unroll
          for (int c = 0; c < 8; ++c) acc.v[c] = r[h].v[c] + acc.v[c];
        }
        if (h == 0 || i1 != i0) store_mv<OT>(out, (size_t)t * d + (h ? i1 : i0), acc);
      }
    }
    return;
  }
  for (int i = lane; i < d; i += 64) {
    MV acc;
#pragma unroll
    for (int c = 0; c < 8; ++c) acc.v[c] = 0.f;
#pragma unroll
    for (int s = 0; s < KM; ++s) {
      if (s < k) {
        const MV y = load_mv<YT>(ys, (size_t)row[s] * d + i);
#pragma unroll
        for (int c = 0; c < 8; ++c) acc.v[c] = acc.v[c] + w[s] * y.v[c];
      }
    }
    if constexpr (Y_MASK) {  // back to blade order
      const float t3 = acc.v[3];
      acc.v[3] = acc.v[4];
      acc.v[4] = t3;
    }
    if constexpr (RESID) {
      const MV r = load_mv<OT>(resid, (size_t)t * d + i);
#pragma unroll
      for (int c = 0; c < 8; ++c) acc.v[c] = r.v[c] + acc.v[c];
    }
    store_mv<OT>(out, (size_t)t * d + i, acc);
  }
}

// Combine of K-split partial planes (fp32, blade order): one thread per
// (token, multivector), for the small token counts of decode.  The planes of
// a row are added in plane order, then  w_s * y_s  in ascending expert order
// as in combine_kernel.  The loads of two slots x four planes are issued
// together: a thread waits for memory twice (routing, then rows).
constexpr int kPlaneBatch = 4;

// SLOT_ROWS: the planes hold slot (t, s) at row t k + s (the int8 Pauli decode layer
// writes them so) instead of at slot_pos[t k + s]
template <int OT, bool RESID, bool SLOT_ROWS>
__global__ __launch_bounds__(256) void combine_planes_kernel(const float* __restrict__ ys, int N, int k, int d,
                                                             const int32_t* __restrict__ topk_idx,
                                                             const float* __restrict__ topk_w,
                                                             const int32_t* __restrict__ slot_pos,
                                                             const void* __restrict__ resid, void* __restrict__ out,
                                                             int planes, size_t plane_stride) {
#pragma clang fp contract(off)
  const size_t n = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (n >= (size_t)N * d) return;
  const int t = (int)(n / d), i = (int)(n % d);
  int ex[8], row[8];
  float w[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {  // unconditional loads (slots past k repeat the last one), then masked
    const size_t f = (size_t)t * k + min(s, k - 1);
    const int e = topk_idx[f], rw = SLOT_ROWS ? (int)f : slot_pos[f];
    const float ws = topk_w[f];
    const bool on = s < k;
    ex[s] = on ? e : 0x7fffffff;
    row[s] = on ? rw : 0;
    w[s] = on ? ws : 0.f;
  }
  MV r;
  if constexpr (RESID) r = load_mv<OT>(resid, n);
#pragma unroll
  for (int a = 1; a < 8; ++a)
#pragma unroll
    for (int b = a; b > 0; --b)
      if (ex[b] < ex[b - 1]) {
        int te = ex[b]; ex[b] = ex[b - 1]; ex[b - 1] = te;
        int tr = row[b]; row[b] = row[b - 1]; row[b - 1] = tr;
        float tw = w[b]; w[b] = w[b - 1]; w[b - 1] = tw;
      }
  MV acc;
#pragma unroll
  for (int c = 0; c < 8; ++c) acc.v[c] = 0.f;
  for (int s0 = 0; s0 < k; s0 += 2) {
    MV y[2];
    for (int p0 = 0; p0 < planes; p0 += kPlaneBatch) {
      MV v[2][kPlaneBatch];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int su = min(s0 + u, k - 1);
        int rs = row[0];  // row[su] without indexing the register array
#pragma unroll
        for (int q = 1; q < 8; ++q)
          if (q == su) rs = row[q];
#pragma unroll
        for (int b = 0; b < kPlaneBatch; ++b) {  // in-range loads only; the unused ones are not added
          const int p = min(p0 + b, planes - 1);
          v[u][b] = load_mv<kF32>(ys, p * plane_stride + (size_t)rs * d + i);
        }
      }
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int b = 0; b < kPlaneBatch; ++b) {
          if (p0 + b >= planes) continue;
          if (p0 + b == 0) {
            y[u] = v[u][b];
          } else {
#pragma unroll
            for (int c = 0; c < 8; ++c) y[u].v[c] = y[u].v[c] + v[u][b].v[c];
          }
        }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      if (s0 + u >= k) continue;
      float ws = w[0];
#pragma unroll
      for (int s = 1; s < 8; ++s)
        if (s == s0 + u) ws = w[s];
#pragma unroll
      for (int c = 0; c < 8; ++c) acc.v[c] = acc.v[c] + ws * y[u].v[c];
    }
  }
  if constexpr (RESID) {
#pragma unroll
    for (int c = 0; c < 8; ++c) acc.v[c] = r.v[c] + acc.v[c];
  }
  store_mv<OT>(out, n, acc);
}

// The same combine with PL planes known at compile time: one thread per half
// multivector (four blade components, one 16-byte piece), so twice the threads,
// and the loads of two slots x all planes issued together -- one wait for the
// routing, one for the rows.  Same additions in the same order as above, so the
// result is identical.
template <int OT, bool RESID, int PL, bool SLOT_ROWS>
__global__ __launch_bounds__(256) void combine_planes_half_kernel(const float* __restrict__ ys, int N, int k, int d,
                                                                  const int32_t* __restrict__ topk_idx,
                                                                  const float* __restrict__ topk_w,
                                                                  const int32_t* __restrict__ slot_pos,
                                                                  const void* __restrict__ resid,
                                                                  void* __restrict__ out, size_t plane_stride) {
#pragma clang fp contract(off)
  const size_t n = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (n >= (size_t)N * d * 2) return;
  const size_t mv = n >> 1;
  const int half = (int)(n & 1);
  const int t = (int)(mv / d), i = (int)(mv % d);
  float r[4] = {0.f, 0.f, 0.f, 0.f};
  if constexpr (RESID) {
    if constexpr (OT == kF32) {
      const float4 q = reinterpret_cast<const float4*>(resid)[n];
      r[0] = q.x; r[1] = q.y; r[2] = q.z; r[3] = q.w;
    } else {
      const uint2 q = reinterpret_cast<const uint2*>(resid)[n];
      r[0] = bf16_bits_to_f32((uint16_t)(q.x & 0xffffu)); r[1] = bf16_bits_to_f32((uint16_t)(q.x >> 16));
      r[2] = bf16_bits_to_f32((uint16_t)(q.y & 0xffffu)); r[3] = bf16_bits_to_f32((uint16_t)(q.y >> 16));
    }
  }
  auto store = [&](const float (&acc)[4]) __attribute__((always_inline)) {
    if constexpr (OT == kF32) {
      reinterpret_cast<float4*>(out)[n] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    } else {
      reinterpret_cast<uint2*>(out)[n] = make_uint2(pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3]));
    }
  };
  if constexpr (SLOT_ROWS) {
    if (k == 2) {  // uniform.  The rows do not depend on the routing arrays, so every load goes
      // out at once; and with two slots the ascending-expert order needs no sort:
      // (0 + a) + b == (0 + b) + a exactly
      const size_t f0 = (size_t)t * 2;
      float4 v[2][PL];
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int p = 0; p < PL; ++p)
          v[u][p] = reinterpret_cast<const float4*>(ys + p * plane_stride + ((f0 + u) * d + i) * 8)[half];
      const float w2[2] = {topk_w[f0], topk_w[f0 + 1]};
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        float y[4] = {v[u][0].x, v[u][0].y, v[u][0].z, v[u][0].w};
#pragma unroll
        for (int p = 1; p < PL; ++p) {
          y[0] = y[0] + v[u][p].x; y[1] = y[1] + v[u][p].y; y[2] = y[2] + v[u][p].z; y[3] = y[3] + v[u][p].w;
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[c] = acc[c] + w2[u] * y[c];
      }
      if constexpr (RESID) {
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[c] = r[c] + acc[c];
      }
      store(acc);
      return;
    }
  }
  int ex[8], row[8];
  float w[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {  // unconditional loads (slots past k repeat the last one), then masked
    const size_t f = (size_t)t * k + min(s, k - 1);
    const int e = topk_idx[f], rw = SLOT_ROWS ? (int)f : slot_pos[f];
    const float ws = topk_w[f];
    const bool on = s < k;
    ex[s] = on ? e : 0x7fffffff;
    row[s] = on ? rw : 0;
    w[s] = on ? ws : 0.f;
  }
#pragma unroll
  for (int a = 1; a < 8; ++a)
#pragma unroll
    for (int b = a; b > 0; --b)
      if (ex[b] < ex[b - 1]) {
        int te = ex[b]; ex[b] = ex[b - 1]; ex[b - 1] = te;
        int tr = row[b]; row[b] = row[b - 1]; row[b - 1] = tr;
        float tw = w[b]; w[b] = w[b - 1]; w[b - 1] = tw;
      }
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < k; s0 += 2) {
    float4 v[2][PL];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int su = min(s0 + u, k - 1);
      int rs = row[0];  // row[su] without indexing the register array
#pragma unroll
      for (int q = 1; q < 8; ++q)
        if (q == su) rs = row[q];
#pragma unroll
      for (int p = 0; p < PL; ++p)
        v[u][p] = reinterpret_cast<const float4*>(ys + p * plane_stride + ((size_t)rs * d + i) * 8)[half];
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      if (s0 + u >= k) continue;
      float y[4] = {v[u][0].x, v[u][0].y, v[u][0].z, v[u][0].w};
#pragma unroll
      for (int p = 1; p < PL; ++p) {
        y[0] = y[0] + v[u][p].x; y[1] = y[1] + v[u][p].y; y[2] = y[2] + v[u][p].z; y[3] = y[3] + v[u][p].w;
      }
      float ws = w[0];
#pragma unroll
      for (int s = 1; s < 8; ++s)
        if (s == s0 + u) ws = w[s];
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[c] = acc[c] + ws * y[c];
    }
  }
  if constexpr (RESID) {
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = r[c] + acc[c];
  }
  store(acc);
}

}  // namespace ygg

using namespace ygg;

YGG_API int ygg_dispatch(const void* x, int dtype, int N, int k, int d, const int32_t* slot_pos, void* x_sorted,
                         int to_mask_order, hipStream_t stream) {
  YGG_CHECK_ARG(dtype == kF32 || dtype == kBF16, "ygg_dispatch: dtype %d unsupported", dtype);
  YGG_CHECK_ARG(N >= 0 && k >= 1 && k <= 8 && d >= 1, "ygg_dispatch: bad sizes N=%d k=%d d=%d", N, k, d);
  if (N == 0) return 0;
  YGG_CHECK_ARG(x && slot_pos && x_sorted, "ygg_dispatch: null pointer");
  const int grid = (N + kTokPerBlock - 1) / kTokPerBlock;
  if (dtype == kF32) {
    if (to_mask_order) dispatch_kernel<kF32, true><<<grid, 256, 0, stream>>>(x, N, k, d, slot_pos, x_sorted);
    else dispatch_kernel<kF32, false><<<grid, 256, 0, stream>>>(x, N, k, d, slot_pos, x_sorted);
  } else {
    if (to_mask_order) dispatch_kernel<kBF16, true><<<grid, 256, 0, stream>>>(x, N, k, d, slot_pos, x_sorted);
    else dispatch_kernel<kBF16, false><<<grid, 256, 0, stream>>>(x, N, k, d, slot_pos, x_sorted);
  }
  return check_launch("dispatch");
}

template <int YT, int OT>
static void launch_combine(int grid, hipStream_t st, const void* ys, int N, int k, int d, const int32_t* idx,
                           const float* w, const int32_t* sp, const void* resid, void* out, bool y_mask) {
#define YGG_C1(YM, RS, KM) combine_kernel<YT, YM, OT, RS, KM><<<grid, 256, 0, st>>>(ys, N, k, d, idx, w, sp, resid, out)
#define YGG_C(YM, RS)                           \
  if (k <= 2) YGG_C1(YM, RS, 2);               \
  else if (k <= 4) YGG_C1(YM, RS, 4);          \
  else YGG_C1(YM, RS, 8)
  if (y_mask) {
    if (resid) { YGG_C(true, true); }
    else { YGG_C(true, false); }
  } else {
    if (resid) { YGG_C(false, true); }
    else { YGG_C(false, false); }
  }
#undef YGG_C
#undef YGG_C1
}

template <bool SR>
static int combine_planes_t(const float* y_planes, int planes, int P_max, int N, int k, int d,
                            const int32_t* topk_idx, const float* topk_w, const int32_t* slot_pos, const void* residual,
                            void* out, int out_dtype, hipStream_t stream) {
  if (N == 0) return 0;
  const size_t stride = (size_t)P_max * d;
  if ((planes >= 2 && planes <= 4) || planes == 8) {  // the half-multivector kernel
    const unsigned hgrid = (unsigned)(((size_t)N * d * 2 + 255) / 256);
#define YGG_CH(OT, RS, PL)                                                                                          \
  combine_planes_half_kernel<OT, RS, PL, SR><<<hgrid, 256, 0, stream>>>(y_planes, N, k, d, topk_idx, topk_w,        \
                                                                         slot_pos, \
                                                                     residual, out, stride * 8)
#define YGG_CH2(PL)                                                                        \
  if (out_dtype == kF32) { if (residual) YGG_CH(kF32, true, PL); else YGG_CH(kF32, false, PL); } \
  else { if (residual) YGG_CH(kBF16, true, PL); else YGG_CH(kBF16, false, PL); }
    if (planes == 8) { YGG_CH2(8) } else if (planes == 4) { YGG_CH2(4) } else if (planes == 3) { YGG_CH2(3) } else { YGG_CH2(2) }
#undef YGG_CH2
#undef YGG_CH
    return check_launch("combine (partial planes)");
  }
  const unsigned grid = (unsigned)(((size_t)N * d + 255) / 256);
#define YGG_CP(OT, RS)                                                                                            \
  combine_planes_kernel<OT, RS, SR><<<grid, 256, 0, stream>>>(y_planes, N, k, d, topk_idx, topk_w, slot_pos,        \
                                                              residual, \
                                                          out, planes, stride)
  if (out_dtype == kF32) { if (residual) YGG_CP(kF32, true); else YGG_CP(kF32, false); }
  else { if (residual) YGG_CP(kBF16, true); else YGG_CP(kBF16, false); }
#undef YGG_CP
  return check_launch("combine (partial planes)");
}

int ygg::combine_planes(const float* y_planes, int planes, int P_max, int N, int k, int d, const int32_t* topk_idx,
                        const float* topk_w, const int32_t* slot_pos, const void* residual, void* out, int out_dtype,
                        hipStream_t stream, bool slot_rows) {
  return slot_rows ? combine_planes_t<true>(y_planes, planes, P_max, N, k, d, topk_idx, topk_w, slot_pos, residual, out,
                                            out_dtype, stream)
                   : combine_planes_t<false>(y_planes, planes, P_max, N, k, d, topk_idx, topk_w, slot_pos, residual,
                                             out, out_dtype, stream);
}

YGG_API int ygg_combine(const void* y_sorted, int y_dtype, int y_mask_order, int N, int k, int d,
                        const int32_t* topk_idx, const float* topk_w, const int32_t* slot_pos, const void* residual,
                        void* out, int out_dtype, hipStream_t stream) {
  YGG_CHECK_ARG((y_dtype == kF32 || y_dtype == kBF16) && (out_dtype == kF32 || out_dtype == kBF16),
                "ygg_combine: dtypes %d/%d unsupported", y_dtype, out_dtype);
  YGG_CHECK_ARG(N >= 0 && k >= 1 && k <= 8 && d >= 1, "ygg_combine: bad sizes N=%d k=%d d=%d", N, k, d);
  if (N == 0) return 0;
  YGG_CHECK_ARG(y_sorted && topk_idx && topk_w && slot_pos && out, "ygg_combine: null pointer");
  const int grid = (N + kTokPerBlock - 1) / kTokPerBlock;
  const bool ym = y_mask_order != 0;
  if (y_dtype == kF32 && out_dtype == kF32)
    launch_combine<kF32, kF32>(grid, stream, y_sorted, N, k, d, topk_idx, topk_w, slot_pos, residual, out, ym);
  else if (y_dtype == kBF16 && out_dtype == kBF16)
    launch_combine<kBF16, kBF16>(grid, stream, y_sorted, N, k, d, topk_idx, topk_w, slot_pos, residual, out, ym);
  else if (y_dtype == kBF16 && out_dtype == kF32)
    launch_combine<kBF16, kF32>(grid, stream, y_sorted, N, k, d, topk_idx, topk_w, slot_pos, residual, out, ym);
  else
    launch_combine<kF32, kBF16>(grid, stream, y_sorted, N, k, d, topk_idx, topk_w, slot_pos, residual, out, ym);
  return check_launch("combine");
}
