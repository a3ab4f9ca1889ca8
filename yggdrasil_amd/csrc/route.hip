// route.hip -- CliffordRouter gating and the expert counting sort on gfx950.
//
// Replaces, for the MoE-HLM layer:
//   * clifford_router.py:54-90   grade energy -> normalised -> (E,4) map + bias
//                                 (ygg_router_energy_logits)
//   * clifford_router.py:18-21,93-104  softmax, top-k, renormalise
//   * hlm_block.py:165-177        flat slots grouped by expert (counts, perm)
//                                 (ygg_route)
//
// Design.  Routing is a few MB of traffic, so the kernels aim at few launches
// and no atomics (the permutation must be bit-exact and deterministic):
//   K1 route_topk_rank   one thread per token: max, exp, pairwise sum (the
//                        summation tree NumPy uses for a row of E floats),
//                        k selections with lowest-index ties, renormalise;
//                        then, per 256-token block, every slot's rank among
//                        the block's slots of the same expert from 64-lane
//                        ballots, and the block histogram.
//   K2 route_scan        one block: per expert, exclusive scan of the block
//                        histograms over blocks; counts and offsets.
//   K3 route_place       one thread per token: sorted position of every slot
//                        = offsets[e] + block_base[b][e] + rank; writes perm
//                        and slot_pos.
// The expert-grouped order within an expert is ascending token order, which
// is the reference's dispatch order (hlm_block.py:172-178).

#include "ygg_common.h"

namespace ygg {

constexpr int kRouteBlock = 256;
constexpr int kMaxExperts = 64;
constexpr int kMaxTopK = 8;

// Pairwise summation of n floats as NumPy does for one reduced row
// (blocks of 8 accumulators, combined as ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)),
// remainder added sequentially; fewer than 8 values: sequential from 0).
__device__ inline float numpy_row_sum(const float* v, int n) {
  if (n < 8) {
    float s = 0.f;
    for (int i = 0; i < n; ++i) s = __fadd_rn(s, v[i]);
    return s;
  }
  float r[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = v[j];
  int i = 8;
  for (; i + 8 <= n; i += 8) {
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = __fadd_rn(r[j], v[i + j]);
  }
  float s = __fadd_rn(__fadd_rn(__fadd_rn(r[0], r[1]), __fadd_rn(r[2], r[3])),
                      __fadd_rn(__fadd_rn(r[4], r[5]), __fadd_rn(r[6], r[7])));
  for (; i < n; ++i) s = __fadd_rn(s, v[i]);
  return s;
}

template <int MAXE>
__global__ __launch_bounds__(kRouteBlock) void route_topk_rank(const float* __restrict__ logits, int N, int E, int k,
                                                               int32_t* __restrict__ topk_idx,
                                                               float* __restrict__ topk_w,
                                                               int32_t* __restrict__ slot_rank,
                                                               int32_t* __restrict__ block_hist) {
  __shared__ int32_t wave_cnt[kRouteBlock / 64][MAXE];
  const int tid = threadIdx.x;
  const int t = blockIdx.x * kRouteBlock + tid;
  const bool active = t < N;
  const int lane = tid & 63, wave = tid >> 6;

  int sel[kMaxTopK];
#pragma unroll
  for (int s = 0; s < kMaxTopK; ++s) sel[s] = -1;

  if (active) {
    float p[MAXE];
    const float* row = logits + (size_t)t * E;
    float m = -INFINITY;
#pragma unroll
    for (int e = 0; e < MAXE; ++e)
      if (e < E) {
        p[e] = row[e];
        m = fmaxf(m, p[e]);
      }
#pragma unroll
    for (int e = 0; e < MAXE; ++e)
      if (e < E) p[e] = expf(__fsub_rn(p[e], m));
    const float denom = __fadd_rn(numpy_row_sum(p, E), 1e-12f);
#pragma unroll
    for (int e = 0; e < MAXE; ++e)
      if (e < E) p[e] = __fdiv_rn(p[e], denom);

    // k selections: highest probability, lowest index among equals
    uint64_t taken = 0;
    float wsel[kMaxTopK];
#pragma unroll
    for (int s = 0; s < kMaxTopK; ++s) {
      if (s < k) {
        int best = -1;
        float bv = 0.f;
#pragma unroll
        for (int e = 0; e < MAXE; ++e) {
          if (e < E && !((taken >> e) & 1ull) && (best < 0 || p[e] > bv)) {
            best = e;
            bv = p[e];
          }
        }
        taken |= 1ull << best;
        sel[s] = best;
        wsel[s] = bv;
      }
    }
    // renormalise; the sum runs from the least to the most probable slot
    float ssum = 0.f;
#pragma unroll
    for (int s = kMaxTopK - 1; s >= 0; --s)
      if (s < k) ssum = __fadd_rn(ssum, wsel[s]);
    ssum = __fadd_rn(ssum, 1e-12f);
#pragma unroll
    for (int s = 0; s < kMaxTopK; ++s)
      if (s < k) {
        topk_idx[(size_t)t * k + s] = sel[s];
        topk_w[(size_t)t * k + s] = __fdiv_rn(wsel[s], ssum);
      }
  }

  // per-expert rank of every slot among this block's slots (token order)
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int rank[kMaxTopK];
#pragma unroll
  for (int s = 0; s < kMaxTopK; ++s) rank[s] = 0;
  for (int e = 0; e < E; ++e) {
    bool has = false;
#pragma unroll
    for (int s = 0; s < kMaxTopK; ++s) has |= (sel[s] == e);
    const uint64_t bal = __ballot(has);
    const int r = __popcll(bal & lt_mask);
#pragma unroll
    for (int s = 0; s < kMaxTopK; ++s)
      if (sel[s] == e) rank[s] = r;
    if (lane == 0) wave_cnt[wave][e] = __popcll(bal);
  }
  __syncthreads();
  if (active) {
#pragma unroll
    for (int s = 0; s < kMaxTopK; ++s) {
      if (s < k) {
        const int e = sel[s];
        int base = 0;
        for (int w = 0; w < wave; ++w) base += wave_cnt[w][e];
        slot_rank[(size_t)t * k + s] = base + rank[s];
      }
    }
  }
  if (tid < E) {
    int c = 0;
#pragma unroll
    for (int w = 0; w < kRouteBlock / 64; ++w) c += wave_cnt[w][tid];
    block_hist[(size_t)blockIdx.x * E + tid] = c;
  }
}

// One block.  Thread e walks the blocks in order (coalesced across e).
__global__ __launch_bounds__(64) void route_scan(const int32_t* __restrict__ block_hist, int nblocks, int E,
                                                 int32_t* __restrict__ block_base, int32_t* __restrict__ counts,
                                                 int32_t* __restrict__ offsets) {
  __shared__ int32_t tot[kMaxExperts];
  const int e = threadIdx.x;
  int run = 0;
  if (e < E) {
    for (int b = 0; b < nblocks; ++b) {
      block_base[(size_t)b * E + e] = run;
      run += block_hist[(size_t)b * E + e];
    }
    counts[e] = run;
  }
  tot[e] = (e < E) ? run : 0;
  __syncthreads();
  if (e == 0) {
    int acc = 0;
    for (int i = 0; i < E; ++i) {
      offsets[i] = acc;
      acc += tot[i];
    }
    offsets[E] = acc;
  }
}

__global__ __launch_bounds__(kRouteBlock) void route_place(const int32_t* __restrict__ topk_idx,
                                                           const int32_t* __restrict__ slot_rank,
                                                           const int32_t* __restrict__ block_base,
                                                           const int32_t* __restrict__ offsets, int N, int E, int k,
                                                           int32_t* __restrict__ perm,
                                                           int32_t* __restrict__ slot_pos) {
  const int t = blockIdx.x * kRouteBlock + threadIdx.x;
  if (t >= N) return;
  for (int s = 0; s < k; ++s) {
    const size_t f = (size_t)t * k + s;
    const int e = topk_idx[f];
    const int pos = offsets[e] + block_base[(size_t)blockIdx.x * E + e] + slot_rank[f];
    perm[pos] = t;
    slot_pos[f] = pos;
  }
}

// Grade energy of one token -> normalised -> logits.  One wave per token;
// lanes stride over the d multivectors, a 64-lane tree reduces the 4 sums.
__global__ __launch_bounds__(256) void router_energy_logits_kernel(const void* __restrict__ x, int x_dtype, int N,
                                                                   int d, const float* __restrict__ rw,
                                                                   const float* __restrict__ rb, int E,
                                                                   float* __restrict__ logits,
                                                                   float* __restrict__ energy_out) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= N) return;
  float g[4] = {0.f, 0.f, 0.f, 0.f};
  for (int i = lane; i < d; i += 64) {
    float v[8];
    if (x_dtype == kF32) {
      const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(x) + ((size_t)t * d + i) * 8);
      const float4 a = p[0], b = p[1];
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
    g[0] += v[0] * v[0];
    g[1] += v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
    g[2] += v[4] * v[4] + v[5] * v[5] + v[6] * v[6];
    g[3] += v[7] * v[7];
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1)
#pragma unroll
    for (int c = 0; c < 4; ++c) g[c] += __shfl_xor(g[c], off);
  const float tot = g[0] + g[1] + g[2] + g[3] + 1e-12f;
  if (energy_out != nullptr && lane < 4) energy_out[(size_t)t * 4 + lane] = g[lane];
  for (int e = lane; e < E; e += 64) {
    float l = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) l += (g[c] / tot) * rw[e * 4 + c];
    logits[(size_t)t * E + e] = l + rb[e];
  }
}

}  // namespace ygg

using namespace ygg;

YGG_API size_t ygg_route_workspace_bytes(int N, int E, int k) {
  const size_t nb = (size_t)(N + kRouteBlock - 1) / kRouteBlock;
  const size_t bytes = (size_t)N * k * 4 + 2 * nb * E * 4;
  return (bytes + 255) & ~(size_t)255;
}

YGG_API int ygg_route(const float* logits, int N, int E, int k, int32_t* topk_idx, float* topk_w, int32_t* counts,
                      int32_t* offsets, int32_t* perm, int32_t* slot_pos, void* workspace, size_t workspace_bytes,
                      hipStream_t stream) {
  YGG_CHECK_ARG(N >= 0, "ygg_route: N=%d must be >= 0", N);
  YGG_CHECK_ARG(E >= 1 && E <= kMaxExperts, "ygg_route: E=%d out of range [1, %d]", E, kMaxExperts);
  YGG_CHECK_ARG(k >= 1 && k <= kMaxTopK && k <= E, "ygg_route: k=%d out of range [1, min(%d, E=%d)]", k, kMaxTopK, E);
  YGG_CHECK_ARG(workspace_bytes >= ygg_route_workspace_bytes(N, E, k),
                "ygg_route: workspace of %zu bytes, need %zu", workspace_bytes, ygg_route_workspace_bytes(N, E, k));
  YGG_CHECK_ARG(N == 0 || (logits && topk_idx && topk_w && perm && slot_pos && workspace),
                "ygg_route: null pointer argument");
  YGG_CHECK_ARG(counts && offsets, "ygg_route: null counts/offsets");
  const int nb = (N + kRouteBlock - 1) / kRouteBlock;
  int32_t* slot_rank = static_cast<int32_t*>(workspace);
  int32_t* block_hist = slot_rank + (size_t)N * k;
  int32_t* block_base = block_hist + (size_t)nb * E;
  if (nb > 0) {
    if (E <= 16)
      route_topk_rank<16><<<nb, kRouteBlock, 0, stream>>>(logits, N, E, k, topk_idx, topk_w, slot_rank, block_hist);
    else if (E <= 32)
      route_topk_rank<32><<<nb, kRouteBlock, 0, stream>>>(logits, N, E, k, topk_idx, topk_w, slot_rank, block_hist);
    else
      route_topk_rank<64><<<nb, kRouteBlock, 0, stream>>>(logits, N, E, k, topk_idx, topk_w, slot_rank, block_hist);
    if (check_launch("route_topk_rank")) return -1;
  }
  route_scan<<<1, 64, 0, stream>>>(block_hist, nb, E, block_base, counts, offsets);
  if (check_launch("route_scan")) return -1;
  if (nb > 0) {
    route_place<<<nb, kRouteBlock, 0, stream>>>(topk_idx, slot_rank, block_base, offsets, N, E, k, perm, slot_pos);
    if (check_launch("route_place")) return -1;
  }
  return 0;
}

YGG_API int ygg_router_energy_logits(const void* x, int x_dtype, int N, int d, const float* router_w,
                                     const float* router_b, int E, float* logits, float* energy,
                                     hipStream_t stream) {
  YGG_CHECK_ARG(x_dtype == kF32 || x_dtype == kBF16, "ygg_router_energy_logits: x dtype %d unsupported", x_dtype);
  YGG_CHECK_ARG(N >= 0 && d >= 1 && E >= 1, "ygg_router_energy_logits: bad sizes N=%d d=%d E=%d", N, d, E);
  YGG_CHECK_ARG(N == 0 || (x && router_w && router_b && logits), "ygg_router_energy_logits: null pointer");
  if (N == 0) return 0;
  router_energy_logits_kernel<<<(N + 3) / 4, 256, 0, stream>>>(x, x_dtype, N, d, router_w, router_b, E, logits,
                                                                energy);
  return check_launch("router_energy_logits");
}
