// route.hip -- CliffordRouter gating and the expert counting sort on gfx950.
//
// Replaces, for the MoE-HLM layer:
//   * clifford_router.py:54-90   grade energy -> normalised -> (E,4) map + bias
//                                 (ygg_router_energy_logits)
//   * clifford_router.py:18-21,93-104  softmax, top-k, renormalise
//   * hlm_block.py:165-177        flat slots grouped by expert (counts, perm)
//                                 (ygg_route)
//
// Design.  Routing moves a few MB, so it is latency bound: the aim is short
// dependency chains and enough waves, with no atomics (the permutation must
// be deterministic and bit-exact):
//   K1 route_select  eight lanes per token, 32 tokens per 256-thread block.
//                    Lane j holds the logits j, j+8, j+16, ...: a shuffle tree
//                    gives the row max, and lane j's running sum of its own
//                    elements followed by the xor-shuffle tree (1, 2, 4) is
//                    exactly NumPy's pairwise summation of a row (eight
//                    accumulators, ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)), then
//                    the remainder in order).  Top-k is k rounds of a shuffle
//                    argmax (higher probability, then lower index).  Lane j of
//                    a token then holds slot j, so a 64-lane ballot per expert
//                    ranks every slot among the block's slots of that expert
//                    in token order; the rank goes to slot_pos and the block
//                    histogram to the workspace.
//   K2 route_scan_place  one thread per slot, 256 per workgroup: the workgroup
//                    sums the block histograms it needs (every expert's total,
//                    an exclusive scan of those gives the offsets, and the base
//                    of each K1 block its slots come from), then slot_pos +=
//                    offsets[e] + block base; perm[slot_pos] = token.  Workgroup
//                    0 writes counts and offsets.
// Within an expert the rows are in ascending token order, the reference's
// dispatch order (hlm_block.py:172-178).

#include "pauli_common.h"
#include "route_select.h"
#include "ygg_common.h"

namespace ygg {

// Rank of each lane's slot among the wave's slots of the same expert (lower lanes
// first, i.e. token order), and the wave's count of every expert e in cnt[e stride]
// (E <= 64).  One ballot per expert the wave holds, not per expert of the layer.
__device__ inline int rank_in_wave(int my_e, int E, int lane, int32_t* __restrict__ cnt, int stride = 1) {
  if (lane < E) cnt[lane * stride] = 0;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int rank = 0;
  uint64_t todo = __ballot(my_e >= 0);
  while (todo) {
    const int e = __builtin_amdgcn_readlane(my_e, (int)__builtin_ctzll(todo));
    const uint64_t bal = __ballot(my_e == e);
    if (my_e == e) rank = __popcll(bal & lt_mask);
    if (lane == 0) cnt[e * stride] = __popcll(bal);
    todo &= ~bal;
  }
  return rank;
}

// Block histograms, expert-major: row e holds expert e's count in every selection
// block, rows padded to a multiple of 4 blocks so they are read in 16-byte pieces.
__host__ __device__ inline int hist_stride(int nb) { return (nb + 3) & ~3; }

constexpr int kSelBlock = 256;                        // threads per K1 block
constexpr int kSelTokens = kSelBlock / kSelLanes;     // tokens per K1 block
constexpr int kSelConvPerThread = 4;                  // multivectors per thread of a conversion workgroup
constexpr int kConvFirstShare = 6;                    // eighths of the conversion's rows in the first launch

template <int Q>  // Q = ceil(E / 8) logits per lane
__global__ __launch_bounds__(kSelBlock) void route_select(const float* __restrict__ logits, int N, int E, int k,
                                                          int32_t* __restrict__ topk_idx,
                                                          float* __restrict__ topk_w,
                                                          int32_t* __restrict__ slot_rank,
                                                          int32_t* __restrict__ block_hist, int n_sel,
                                                          RowConvert cv) {
  __shared__ int32_t wave_cnt[kSelBlock / 64][kMaxExperts];
  if ((int)blockIdx.x >= n_sel) {  // a conversion workgroup
    convert_rows_block<kSelBlock, kSelConvPerThread>(cv, (int)blockIdx.x - n_sel);
    return;
  }
  const int tid = threadIdx.x;
  const int j = tid & (kSelLanes - 1);
  const int t = blockIdx.x * kSelTokens + tid / kSelLanes;
  const bool active = t < N;
  const int lane = tid & 63, wave = tid >> 6;
  int my_e;
  float my_w;
  select_token<Q>(logits, E, k, t, active, j, lane, my_e, my_w);
  if (my_e >= 0) {
    topk_idx[(size_t)t * k + j] = my_e;
    topk_w[(size_t)t * k + j] = my_w;
  }

  // ---- rank of every slot among the block's slots of its expert (token order)
  const int rank = rank_in_wave(my_e, E, lane, wave_cnt[wave]);
  __syncthreads();
  if (my_e >= 0) {
    int base = 0;
    for (int w = 0; w < wave; ++w) base += wave_cnt[w][my_e];
    slot_rank[(size_t)t * k + j] = base + rank;
  }
  if (tid < E) {
    int c = 0;
#pragma unroll
    for (int w = 0; w < kSelBlock / 64; ++w) c += wave_cnt[w][tid];
    block_hist[(size_t)tid * hist_stride(n_sel) + blockIdx.x] = c;  // expert-major: [E][blocks]
  }
}

// The scan and the placement in one launch: every placing workgroup (256 slots)
// sums the block histograms itself -- each expert's total, and its base in each of
// the few K1 blocks its slots come from -- so no workgroup waits on another.
// Workgroup 0 also writes counts and offsets.  The histograms are read, not
// rewritten.
constexpr int kPlaceSlots = 256;
constexpr int kPlaceMaxSel = kPlaceSlots / kSelTokens + 2;  // K1 blocks one placing workgroup can touch

__global__ __launch_bounds__(kPlaceSlots) void route_scan_place(const int32_t* __restrict__ topk_idx,
                                                                const int32_t* __restrict__ block_hist, int N, int nb,
                                                                int E, int k, int32_t* __restrict__ perm,
                                                                int32_t* __restrict__ slot_pos,
                                                                int32_t* __restrict__ counts,
                                                                int32_t* __restrict__ offsets,
                                                                int32_t* __restrict__ row_slot, int n_place,
                                                                RowConvert cv) {
  __shared__ int32_t s_tot[kMaxExperts];
  __shared__ int32_t s_off[kMaxExperts];
  __shared__ int32_t s_base[kMaxExperts][kPlaceMaxSel];
  if ((int)blockIdx.x >= n_place) {  // a conversion workgroup (the second part of the rows)
    convert_rows_block<kPlaceSlots, kSelConvPerThread>(cv, (int)blockIdx.x - n_place);
    return;
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const long long slots = (long long)N * k;
  const long long f0 = (long long)blockIdx.x * kPlaceSlots;
  const long long f1 = f0 + kPlaceSlots < slots ? f0 + kPlaceSlots : slots;
  // this thread's slot: its loads first, they do not depend on the scan
  const long long f = f0 + tid;
  const bool has_slot = f < f1;
  const int my_e = has_slot ? topk_idx[f] : 0;
  const int my_rank = has_slot ? slot_pos[f] : 0;
  // the K1 blocks [sb0, sb1) holding this workgroup's tokens (at most kPlaceMaxSel)
  const int sb0 = f0 < slots ? (int)(f0 / k) / kSelTokens : 0;
  const int sb1 = f0 < slots ? (int)((f1 - 1) / k) / kSelTokens + 1 : 0;
  // Thread (e, part) sums part `part` of expert e's block counts: `parts` threads per
  // expert (a power of two, so a group is aligned within a wave), every expert at
  // once; each thread reads its share in 16-byte pieces, every piece in flight before
  // the first is added (the rows are padded with whole pieces).
  int parts = 1;
  while (parts < 64 && parts * 2 * E <= kPlaceSlots) parts *= 2;
  const int e_me = tid / parts, part = tid % parts;
  const int hs = hist_stride(nb);
  int pre = 0, all = 0;  // sums of the blocks before sb0, and of every block
  if (e_me < E) {
    const int4* h4 = reinterpret_cast<const int4*>(block_hist + (size_t)e_me * hs);
    const int n4 = hs >> 2;
    const int per = (n4 + parts - 1) / parts;
    const int q0 = part * per, q1 = min(n4, q0 + per);
    constexpr int kU = 8;
    for (int qb = q0; qb < q1; qb += kU) {
      int4 v[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) v[u] = qb + u < q1 ? h4[qb + u] : make_int4(0, 0, 0, 0);
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int b0 = 4 * (qb + u);  // padding blocks hold whatever: only blocks below nb count
        const int c[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int cv_ = b0 + i < nb ? c[i] : 0;
          all += cv_;
          pre += b0 + i < sb0 ? cv_ : 0;
        }
      }
    }
  }
  for (int o = parts / 2; o > 0; o >>= 1) {
    pre += __shfl_xor(pre, o);
    all += __shfl_xor(all, o);
  }
  if (e_me < E && part == 0) {
    const int32_t* h = block_hist + (size_t)e_me * hs;
    s_tot[e_me] = all;
    int run = pre;
#pragma unroll
    for (int q = 0; q < kPlaceMaxSel; ++q) {
      if (sb0 + q < sb1) {
        s_base[e_me][q] = run;
        run += h[sb0 + q];
      }
    }
  }
  __syncthreads();
  if (wave == 0) {  // exclusive scan of the expert totals
    const int c = lane < E ? s_tot[lane] : 0;
    int incl = c;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(incl, o);
      if (lane >= o) incl += v;
    }
    if (lane < E) s_off[lane] = incl - c;
    if (blockIdx.x == 0) {
      if (lane < E) {
        counts[lane] = c;
        offsets[lane] = incl - c;
      }
      if (lane == E - 1) offsets[E] = incl;
    }
  }
  __syncthreads();
  if (has_slot) {
    const int t = (int)(f / k);
    const int pos = s_off[my_e] + s_base[my_e][t / kSelTokens - sb0] + my_rank;
    slot_pos[f] = pos;
    perm[pos] = t;
    if (row_slot != nullptr) row_slot[pos] = (int32_t)f;
  }
}

// Small token counts (decode): the three steps above in one workgroup of
// 1024 threads, with the group histograms in LDS.  Wave w selects the
// 8-token groups w, w + 16, ...; each group's slots are ranked per expert by
// ballot in token order, the per-expert exclusive scan over groups (a wave
// per expert, shuffle scan) and the scan over experts follow, and every lane
// then places its slots --
// the same counts, offsets, permutation and slot positions as the
// multi-block path, from one launch.
constexpr int kSmallThreads = 1024;
constexpr int kSmallWaves = kSmallThreads / 64;
constexpr int kSmallIters = 8;                                     // groups per wave at most
constexpr int kSmallGroups = kSmallWaves * kSmallIters;            // 8-token groups
constexpr int kSmallMaxN = kSmallGroups * (64 / kSelLanes);        // 1024 tokens

template <int Q, bool FROM_X>
__global__ __launch_bounds__(kSmallThreads) void route_small(const float* __restrict__ logits, const void* __restrict__ x,
                                                             int x_dtype, int d, const float* __restrict__ rw,
                                                             const float* __restrict__ rb, int N, int E, int k,
                                                             int32_t* __restrict__ topk_idx,
                                                             float* __restrict__ topk_w,
                                                             int32_t* __restrict__ counts,
                                                             int32_t* __restrict__ offsets,
                                                             int32_t* __restrict__ perm,
                                                             int32_t* __restrict__ slot_pos, RowConvert cv) {
  __shared__ int32_t cnt[kMaxExperts][kSmallGroups];  // slots per (expert, group), then their base
  __shared__ int32_t tot[kMaxExperts];
  __shared__ int32_t eoff[kMaxExperts];
  if (blockIdx.x > 0) {  // a conversion workgroup
    convert_rows_block<kSmallThreads, 1>(cv, (int)blockIdx.x - 1);
    return;
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = tid & (kSelLanes - 1);
  const int ngroups = (N + 7) / 8;
  // a real loop (not unrolled): this kernel runs once per layer call, cold, and
  // its instruction fetch, not its arithmetic, sets its latency
#pragma unroll 1
  for (int grp = wave; grp < ngroups; grp += kSmallWaves) {
    const int t = grp * 8 + lane / kSelLanes;
    int e;
    float w;
    if constexpr (FROM_X) {
      float p[Q];
      energy_logits<Q>(x, x_dtype, d, rw, rb, E, t, t < N, j, p);
      select_from_logits<Q>(p, E, k, t < N, j, lane, e, w);
    } else {
      select_token<Q>(logits, E, k, t, t < N, j, lane, e, w);
    }
    const int rank = rank_in_wave(e, E, lane, &cnt[0][grp], kSmallGroups);
    if (e >= 0) {  // rank within the group for now; the placement below turns it into the row
      topk_idx[(size_t)t * k + j] = e;
      topk_w[(size_t)t * k + j] = w;
      slot_pos[(size_t)t * k + j] = rank;
    }
  }
  __syncthreads();
  // per expert (one wave each): exclusive scan of its group counts in group
  // order; lane l holds groups 2l and 2l + 1
  for (int x = wave; x < E; x += kSmallWaves) {
    const int g0 = 2 * lane, g1 = g0 + 1;
    const int c0 = g0 < ngroups ? cnt[x][g0] : 0;
    const int c1 = g1 < ngroups ? cnt[x][g1] : 0;
    int incl = c0 + c1;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(incl, o);
      if (lane >= o) incl += v;
    }
    const int excl = incl - c0 - c1;
    if (g0 < ngroups) cnt[x][g0] = excl;
    if (g1 < ngroups) cnt[x][g1] = excl + c0;
    if (lane == 63) tot[x] = incl;
  }
  __syncthreads();
  if (wave == 0) {  // exclusive scan over experts
    const int c = lane < E ? tot[lane] : 0;
    int incl = c;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(incl, o);
      if (lane >= o) incl += v;
    }
    if (lane < E) {
      eoff[lane] = incl - c;
      counts[lane] = c;
      offsets[lane] = incl - c;
    }
    if (lane == E - 1) offsets[E] = incl;
  }
  __syncthreads();
  // each thread revisits exactly the slots it selected above (same group order)
#pragma unroll 1
  for (int grp = wave; grp < ngroups; grp += kSmallWaves) {
    const int t = grp * 8 + lane / kSelLanes;
    if (t < N && j < k) {
      const size_t f = (size_t)t * k + j;
      const int e = topk_idx[f];
      const int pos = eoff[e] + cnt[e][grp] + slot_pos[f];
      slot_pos[f] = pos;
      perm[pos] = t;
      if (cv.row_slot != nullptr) cv.row_slot[pos] = (int32_t)f;
    }
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

namespace {
template <bool FROM_X>
int launch_route_small(const float* logits, const void* x, int x_dtype, int d, const float* rw, const float* rb, int N,
                       int E, int k, int32_t* topk_idx, float* topk_w, int32_t* counts, int32_t* offsets,
                       int32_t* perm, int32_t* slot_pos, const RowConvert& cv, hipStream_t stream) {
  const unsigned grid = 1u + (unsigned)convert_rows_blocks<kSmallThreads, 1>(cv);
  switch ((E + 7) / 8) {
#define YGG_SMALL(Q)                                                                                              \
  case Q:                                                                                                         \
    route_small<Q, FROM_X><<<grid, kSmallThreads, 0, stream>>>(logits, x, x_dtype, d, rw, rb, N, E, k, topk_idx,  \
                                                               topk_w, counts, offsets, perm, slot_pos, cv);      \
    break;
    YGG_SMALL(1) YGG_SMALL(2) YGG_SMALL(3) YGG_SMALL(4) YGG_SMALL(5) YGG_SMALL(6) YGG_SMALL(7) YGG_SMALL(8)
#undef YGG_SMALL
  }
  return check_launch("route_small");
}
}  // namespace

YGG_API size_t ygg_route_workspace_bytes(int N, int E, int k) {
  (void)k;
  const int nb = (N + kSelTokens - 1) / kSelTokens;
  return ((size_t)hist_stride(nb) * E * 4 + 255) & ~(size_t)255;
}

YGG_API int ygg_route(const float* logits, int N, int E, int k, int32_t* topk_idx, float* topk_w, int32_t* counts,
                      int32_t* offsets, int32_t* perm, int32_t* slot_pos, void* workspace, size_t workspace_bytes,
                      hipStream_t stream) {
  return ygg::route_convert(logits, N, E, k, topk_idx, topk_w, counts, offsets, perm, slot_pos, workspace,
                            workspace_bytes, RowConvert{}, stream);
}

YGG_API int ygg_route_pauli_rows(const float* logits, int N, int E, int k, const void* x, int x_dtype, int d,
                                 int32_t* topk_idx, float* topk_w, int32_t* counts, int32_t* offsets, int32_t* perm,
                                 int32_t* slot_pos, void* x_pauli, void* workspace, size_t workspace_bytes,
                                 hipStream_t stream) {
  YGG_CHECK_ARG(x_dtype == kF32 || x_dtype == kBF16, "ygg_route_pauli_rows: x dtype %d unsupported", x_dtype);
  YGG_CHECK_ARG(d >= 1 && (x_dtype == kF32 || d % 2 == 0), "ygg_route_pauli_rows: d=%d (even for bf16 rows)", d);
  YGG_CHECK_ARG(N == 0 || (x && x_pauli), "ygg_route_pauli_rows: null x or x_pauli");
  ygg::RowConvert cv;
  if (N > 0) {
    cv.x = x;
    cv.out = x_pauli;
    cv.n = (long long)N * d;
    cv.d = d;
    cv.kind = x_dtype == kBF16 ? ygg::kConvBf16Pauli : ygg::kConvF32Pauli;
  }
  return ygg::route_convert(logits, N, E, k, topk_idx, topk_w, counts, offsets, perm, slot_pos, workspace,
                            workspace_bytes, cv, stream);
}

// The conversion's workgroups follow the routing's own in both of its launches: they
// do not depend on it, and the short routing kernels leave most of the chip idle.
// The rows are split between the launches in proportion to what each launch's
// routing part is worth in conversion time, so the two end together.
int ygg::route_convert(const float* logits, int N, int E, int k, int32_t* topk_idx, float* topk_w, int32_t* counts,
                       int32_t* offsets, int32_t* perm, int32_t* slot_pos, void* workspace, size_t workspace_bytes,
                       const RowConvert& cv, hipStream_t stream) {
  YGG_CHECK_ARG(N >= 0, "ygg_route: N=%d must be >= 0", N);
  YGG_CHECK_ARG(E >= 1 && E <= kMaxExperts, "ygg_route: E=%d out of range [1, %d]", E, kMaxExperts);
  YGG_CHECK_ARG(k >= 1 && k <= kMaxTopK && k <= E, "ygg_route: k=%d out of range [1, min(%d, E=%d)]", k, kMaxTopK, E);
  YGG_CHECK_ARG(workspace_bytes >= ygg_route_workspace_bytes(N, E, k),
                "ygg_route: workspace of %zu bytes, need %zu", workspace_bytes, ygg_route_workspace_bytes(N, E, k));
  YGG_CHECK_ARG(N == 0 || (logits && topk_idx && topk_w && perm && slot_pos && workspace),
                "ygg_route: null pointer argument");
  YGG_CHECK_ARG(counts && offsets, "ygg_route: null counts/offsets");
  if (N > 0 && N <= kSmallMaxN)
    return launch_route_small<false>(logits, nullptr, 0, 0, nullptr, nullptr, N, E, k, topk_idx, topk_w, counts,
                                     offsets, perm, slot_pos, cv, stream);
  const int nb = (N + kSelTokens - 1) / kSelTokens;
  int32_t* block_hist = static_cast<int32_t*>(workspace);
  // the first launch converts rows [0, r_split), the second the rest
  const long long conv_rows = cv.kind == kConvNone || cv.d <= 0 ? 0 : cv.n / cv.d;
  const long long r_split = conv_rows * kConvFirstShare / 8;
  const RowConvert cv1 = row_convert_part(cv, 0, r_split), cv2 = row_convert_part(cv, r_split, conv_rows);
  const int conv_blocks = convert_rows_blocks<kSelBlock, kSelConvPerThread>(cv1);
  if (nb + conv_blocks > 0) {
    // slot ranks go to slot_pos; route_scan_place turns them into rows
    switch ((E + 7) / 8) {
#define YGG_SEL(Q)                                                                                          \
  case Q:                                                                                                   \
    route_select<Q><<<nb + conv_blocks, kSelBlock, 0, stream>>>(logits, N, E, k, topk_idx, topk_w, slot_pos, \
                                                                block_hist, nb, cv1);                       \
    break;
      YGG_SEL(1) YGG_SEL(2) YGG_SEL(3) YGG_SEL(4) YGG_SEL(5) YGG_SEL(6) YGG_SEL(7) YGG_SEL(8)
#undef YGG_SEL
    }
    if (check_launch("route_select")) return -1;
  }
  const size_t slots = (size_t)N * k;
  const unsigned place_blocks = slots ? (unsigned)((slots + kPlaceSlots - 1) / kPlaceSlots) : 1u;  // N = 0: counts 0
  const unsigned conv2_blocks = (unsigned)convert_rows_blocks<kPlaceSlots, kSelConvPerThread>(cv2);
  route_scan_place<<<place_blocks + conv2_blocks, kPlaceSlots, 0, stream>>>(
      topk_idx, block_hist, N, nb, E, k, perm, slot_pos, counts, offsets, cv.row_slot, (int)place_blocks, cv2);
  return check_launch("route_scan_place");
}

// The CliffordLinear(d -> E) head's scalar part (the router of the TinyHLMMoE-style
// layer, hlm.py:109,141-145): logits[t, e] = <sum_i W[e, i] x[t, i]>_0, in the fp32
// order of CliffordLinear.forward's geom_matmul (clifford_linear.py:101-123 over
// rune/ops/batched.py:72-82): for each i in turn, the eight diagonal terms
// (s_c W_c) x_c of the product's scalar part are added to zero in component order
// (s = -1 on grades 2 and 3), and that product is added to the running sum.  No
// multiply-add contraction, so the logits are the reference's bit for bit.
//
// One wave per token.  The per-i products are independent: lane i computes them
// for 64 input multivectors at a time (x and W rows read as contiguous 2 KiB runs
// across the wave) into LDS, then lane e adds its expert's 64 products in i order
// to its running sum.  Experts beyond 64 take further passes.  One wave per
// workgroup: a C1-sized batch (256 tokens) spreads over 256 CUs rather than 64
// (C1 step 41.4-42.0 -> 41.1-41.3 us).
constexpr int kHeadWaves = 1;

template <typename XT>
__global__ __launch_bounds__(64 * kHeadWaves) void router_head_logits_kernel(const XT* __restrict__ x, int N, int d,
                                                                            const float* __restrict__ head_w, int E,
                                                                            float* __restrict__ logits) {
#pragma clang fp contract(off)
  // kHeadWaves x min(E, 64) x 64 floats; product (e, i) sits at column i ^ e of row e, so the
  // lanes adding along a row hit distinct banks
  extern __shared__ float head_buf[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int EB = E < 64 ? E : 64;
  float* pb = head_buf + (size_t)wave * EB * 64;
  const int t = blockIdx.x * kHeadWaves + wave;
  const bool active = t < N;  // every wave takes part in the barriers below
  const XT* xr = x + (size_t)(active ? t : 0) * d * 8;
  for (int e0 = 0; e0 < E; e0 += 64) {
    const int ne = (E - e0) < 64 ? (E - e0) : 64;
    float acc = 0.f;
    for (int i0 = 0; i0 < d; i0 += 64) {
      const int i = i0 + lane, ni = (d - i0) < 64 ? (d - i0) : 64;
      if (active && i < d) {
        float xv[8];
        if constexpr (sizeof(XT) == 4) {
          const float4 a = reinterpret_cast<const float4*>(xr + (size_t)i * 8)[0];
          const float4 b = reinterpret_cast<const float4*>(xr + (size_t)i * 8)[1];
          xv[0] = a.x; xv[1] = a.y; xv[2] = a.z; xv[3] = a.w; xv[4] = b.x; xv[5] = b.y; xv[6] = b.z; xv[7] = b.w;
        } else {
          const uint4 q = *reinterpret_cast<const uint4*>(xr + (size_t)i * 8);
          const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            xv[2 * c] = __builtin_bit_cast(float, w[c] << 16);
            xv[2 * c + 1] = __builtin_bit_cast(float, w[c] & 0xffff0000u);
          }
        }
#pragma unroll 4
        for (int el = 0; el < ne; ++el) {
          const float4* wr = reinterpret_cast<const float4*>(head_w + ((size_t)(e0 + el) * d + i) * 8);
          const float4 a = wr[0], b = wr[1];
          const float wv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
          float p = 0.f;
#pragma unroll
          for (int c = 0; c < 8; ++c) p = p + (c < 4 ? wv[c] : -wv[c]) * xv[c];
          pb[el * 64 + (lane ^ el)] = p;
        }
      }
      __syncthreads();
      if (active && lane < ne)
        for (int il = 0; il < ni; ++il) acc = acc + pb[lane * 64 + (il ^ lane)];
      __syncthreads();
    }
    if (active && lane < ne) logits[(size_t)t * E + e0 + lane] = acc;
  }
}

YGG_API int ygg_router_head_logits(const void* x, int x_dtype, int N, int d, const float* head_w, int E,
                                   float* logits, hipStream_t stream) {
  YGG_CHECK_ARG(x_dtype == kF32 || x_dtype == kBF16, "ygg_router_head_logits: x dtype %d unsupported", x_dtype);
  YGG_CHECK_ARG(N >= 0 && d >= 1 && E >= 1, "ygg_router_head_logits: bad sizes N=%d d=%d E=%d", N, d, E);
  YGG_CHECK_ARG(N == 0 || (x && head_w && logits), "ygg_router_head_logits: null pointer");
  if (N == 0) return 0;
  const unsigned blocks = (unsigned)((N + kHeadWaves - 1) / kHeadWaves);
  const size_t lds = (size_t)kHeadWaves * (E < 64 ? E : 64) * 64 * sizeof(float);
  if (x_dtype == kF32)
    router_head_logits_kernel<float><<<blocks, 64 * kHeadWaves, lds, stream>>>(static_cast<const float*>(x), N, d,
                                                                               head_w, E, logits);
  else
    router_head_logits_kernel<uint16_t><<<blocks, 64 * kHeadWaves, lds, stream>>>(static_cast<const uint16_t*>(x), N,
                                                                                  d, head_w, E, logits);
  return check_launch("router_head_logits");
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

// CliffordRouter.forward end to end (clifford_router.py:54-104) plus the expert
// counting sort (hlm_block.py:165-177): grade energies of x, the (E, 4) map and
// bias, softmax, top-k, renormalisation, counts, offsets, perm and slot rows.
// Up to 1024 tokens it is one launch (the logits never leave the chip); beyond,
// the logits go through `logits_scratch` (N x E fp32) and ygg_route.
YGG_API int ygg_route_energy(const void* x, int x_dtype, int N, int d, const float* router_w, const float* router_b,
                             int E, int k, int32_t* topk_idx, float* topk_w, int32_t* counts, int32_t* offsets,
                             int32_t* perm, int32_t* slot_pos, float* logits_scratch, void* workspace,
                             size_t workspace_bytes, hipStream_t stream) {
  return ygg::route_energy_convert(x, x_dtype, N, d, router_w, router_b, E, k, topk_idx, topk_w, counts, offsets, perm,
                                   slot_pos, logits_scratch, workspace, workspace_bytes, RowConvert{}, stream);
}

int ygg::route_energy_convert(const void* x, int x_dtype, int N, int d, const float* router_w, const float* router_b,
                              int E, int k, int32_t* topk_idx, float* topk_w, int32_t* counts, int32_t* offsets,
                              int32_t* perm, int32_t* slot_pos, float* logits_scratch, void* workspace,
                              size_t workspace_bytes, const RowConvert& cv, hipStream_t stream) {
  YGG_CHECK_ARG(x_dtype == kF32 || x_dtype == kBF16, "ygg_route_energy: x dtype %d unsupported", x_dtype);
  YGG_CHECK_ARG(N >= 0 && d >= 1, "ygg_route_energy: bad sizes N=%d d=%d", N, d);
  YGG_CHECK_ARG(E >= 1 && E <= kMaxExperts, "ygg_route_energy: E=%d out of range [1, %d]", E, kMaxExperts);
  YGG_CHECK_ARG(k >= 1 && k <= kMaxTopK && k <= E, "ygg_route_energy: k=%d out of range [1, min(%d, E=%d)]", k,
                kMaxTopK, E);
  YGG_CHECK_ARG(counts && offsets, "ygg_route_energy: null counts/offsets");
  if (N > 0 && N <= kSmallMaxN) {
    YGG_CHECK_ARG(x && router_w && router_b && topk_idx && topk_w && perm && slot_pos,
                  "ygg_route_energy: null pointer argument");
    return launch_route_small<true>(nullptr, x, x_dtype, d, router_w, router_b, N, E, k, topk_idx, topk_w, counts,
                                    offsets, perm, slot_pos, cv, stream);
  }
  YGG_CHECK_ARG(N == 0 || logits_scratch, "ygg_route_energy: %d tokens need logits_scratch (N x E fp32)", N);
  if (N > 0 && ygg_router_energy_logits(x, x_dtype, N, d, router_w, router_b, E, logits_scratch, nullptr, stream))
    return -1;
  return ygg::route_convert(logits_scratch, N, E, k, topk_idx, topk_w, counts, offsets, perm, slot_pos, workspace,
                            workspace_bytes, cv, stream);
}
