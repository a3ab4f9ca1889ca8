// pauli_f32.hip -- fp32 grouped CliffordLinear expert products as complex
// GEMMs on the fp32 MFMA units of gfx950 (v_mfma_f32_32x32x2_f32).
//
// Replaces, for the fp32 layer, CliffordLinear.forward
// (holograph/layers/clifford_linear.py:101-123) of every expert and the
// grade-wise activation (holograph/layers/activations.py:15-128).  The algebra
// is the one of pauli_gemm.hip (Cl(3,0) = 2x2 complex matrices, 32 real
// multiply-adds per multivector pair); here every operand stays fp32.
//
// Layouts
// -------
// * Pauli rows (fp32): the four complex entries of every multivector, grouped
//   by matrix column b and real / imaginary part k:
//   X[((m * d + i) * 2 + b) * 2 + k) * 2 + c] = (re if k = 0, im if k = 1) of X_i[c][b]
//   for token row m; 8 floats per multivector, as in blade order.  The wave's 64
//   MFMA rows (16 tokens x (b, k)) read 32 contiguous bytes per token and input.
// * Prepared weights (format 4): per (e, i, k, j) eight floats [c][a][q]:
//   k = 0: (u, v), k = 1: (-v, u), where u + iv = W_ji[a, c] / 2, at
//   ((e * d_in + i) * 2 + k) * d_out + j.  With v_mfma_f32_32x32x2_f32 (K = 2:
//   lane l holds k = l / 32) the real part takes q = 0 and the imaginary part
//   q = 1, so both B operands come from memory as they are, and the 32 columns
//   of a wave are 1 KiB runs per (i, k).
//
// Work decomposition
// ------------------
// A workgroup of 4 waves owns a tile of 16 tokens (32 GEMM rows) of one expert
// x 32 output multivectors -- 32 tokens, two row blocks per wave, for long
// contractions -- and the waves split the contraction and add their 32x32
// accumulators (a = 0, 1 x re, im) in LDS in a fixed order.  The column tiles
// of a row tile run back to back on one XCD, so the row tile's activations come
// from HBM once.  blockIdx.z optionally splits the contraction further across
// workgroups into fp32 partial planes (no activation), which the consumer adds
// in split order.  Deterministic throughout.  (Wider tiles -- 32 tokens x 64
// columns, each wave a quadrant over the whole contraction, no cross-wave sum --
// were measured 40-80 % slower at the C3 shape.)

#include <algorithm>

#include "pauli_common.h"
#include "route_select.h"

namespace ygg {

typedef float f32x16v_t __attribute__((ext_vector_type(16)));

constexpr int kF32Waves = 4;
constexpr int kF32Tok = 16;  // tokens per tile (32 GEMM rows)
constexpr int kF32Cols = 32;  // output multivectors per tile
constexpr int kF32U = 4;      // input multivectors per register-buffered block of the K loop
constexpr long long kF32TwoBlockMinGroups = 2048;  // 32-token tiles from this many workgroups (8 per CU)

// output layouts: Pauli rows (for the next product), blade rows (row, d_out), fp32
// partial planes, and blade columns (d_out, rows) -- the transposed product geom_matmul
// returns
enum PauliF32Out : int { kF32OutPauliRows = 0, kF32OutBlade = 1, kF32OutPartial = 2, kF32OutBladeT = 3 };

template <int TOK>  // tokens per tile
__device__ inline bool f32_find_tile(const int32_t* __restrict__ offsets, int E, int tile, int& e, int& row0,
                                     int& row_end) {
  int acc = 0;
  int beg = offsets[0];
  for (int x = 0; x < E; ++x) {
    const int end = offsets[x + 1];
    const int nt = (end - beg + TOK - 1) / TOK;
    if (tile < acc + nt) {
      e = x;
      row0 = beg + (tile - acc) * TOK;
      row_end = end;
      return true;
    }
    acc += nt;
    beg = end;
  }
  return false;
}

// The contraction over inputs [i0, i1) of one wave's WR blocks of 32 GEMM rows x 32
// columns: operands of input i are x (re, im) of the lane's GEMM row in block r
// (arow[r] + 8 i) and the eight weight floats of its column (wrow + i w_step), which
// every row block shares.  Blocks of U inputs are double buffered in registers, so
// one block's loads are in flight while the previous block's MFMAs run.  i0, i1
// must be wave-uniform.
template <int WR>
__device__ inline void f32_kloop(f32x16v_t (&acc)[WR][2][2], const float* const (&arow)[WR],
                                 const float* __restrict__ wrow, size_t w_step, int i0, int i1) {
  constexpr int U = WR == 1 ? kF32U : kF32U / 2;
  struct Ops {
    float2 xa[WR];
    float4 w0, w1;
  };
  auto load_op = [&](int i, Ops& o) {
#pragma unroll
    for (int r = 0; r < WR; ++r) o.xa[r] = *reinterpret_cast<const float2*>(arow[r] + (size_t)i * 8);
    o.w0 = *reinterpret_cast<const float4*>(wrow + i * w_step);      // c = 0
    o.w1 = *reinterpret_cast<const float4*>(wrow + i * w_step + 4);  // c = 1
  };
  auto mma = [&](const Ops& o) {
#pragma unroll
    for (int r = 0; r < WR; ++r) {
      f32x16v_t(&a)[2][2] = acc[r];
      a[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(o.xa[r].x, o.w0.x, a[0][0], 0, 0, 0);
      a[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(o.xa[r].x, o.w0.y, a[0][1], 0, 0, 0);
      a[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(o.xa[r].x, o.w0.z, a[1][0], 0, 0, 0);
      a[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(o.xa[r].x, o.w0.w, a[1][1], 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < WR; ++r) {
      f32x16v_t(&a)[2][2] = acc[r];
      a[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(o.xa[r].y, o.w1.x, a[0][0], 0, 0, 0);
      a[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(o.xa[r].y, o.w1.y, a[0][1], 0, 0, 0);
      a[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(o.xa[r].y, o.w1.z, a[1][0], 0, 0, 0);
      a[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(o.xa[r].y, o.w1.w, a[1][1], 0, 0, 0);
    }
  };
#pragma unroll
  for (int r = 0; r < WR; ++r)
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[r][a][q][v] = 0.f;
  const int nblk = max(i1 - i0, 0) / U;
  Ops b0[U], b1[U];
  if (nblk > 0) {
#pragma unroll
    for (int u = 0; u < U; ++u) load_op(i0 + u, b0[u]);
  }
  for (int b = 0; b < nblk; b += 2) {  // buffer 0 holds block b, buffer 1 block b + 1
    if (b + 1 < nblk) {
#pragma unroll
      for (int u = 0; u < U; ++u) load_op(i0 + (b + 1) * U + u, b1[u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) mma(b0[u]);
    if (b + 1 < nblk) {
      if (b + 2 < nblk) {
#pragma unroll
        for (int u = 0; u < U; ++u) load_op(i0 + (b + 2) * U + u, b0[u]);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) mma(b1[u]);
    }
  }
  for (int i = i0 + nblk * U; i < i1; ++i) {
    Ops o;
    load_op(i, o);
    mma(o);
  }
}

// One output multivector (token row, column j) from its Pauli sums Y[a][b] = (re, im):
// blade map, bias (split 0 only for partial planes), the pre-activation rows when
// Ypre is set, activation, and the store in the OUT layout.
template <int ACT, int OUT>
__device__ inline void f32_store_mv(float y00r, float y00i, float y01r, float y01i, float y10r, float y10i, float y11r,
                                    float y11i, const float* __restrict__ bias, int e, int row, int j, int d_out,
                                    int split, int P_max, float* __restrict__ Y, float* __restrict__ Ypre,
                                    const int32_t* __restrict__ row_map) {
  float y[8];
  pauli_to_blade(y00r, y00i, y01r, y01i, y10r, y10i, y11r, y11i, y);
  if (bias != nullptr && (OUT != kF32OutPartial || split == 0)) {
#pragma unroll
    for (int c = 0; c < 8; ++c) y[c] += bias[((size_t)e * d_out + j) * 8 + blade_to_mask(c)];
  }
  if constexpr (OUT == kF32OutPauliRows) {
    if (Ypre != nullptr) {  // the pre-activation rows, blade order (kept for the backward)
      float4* q = reinterpret_cast<float4*>(Ypre + ((size_t)row * d_out + j) * 8);
      q[0] = make_float4(y[0], y[1], y[2], y[3]);
      q[1] = make_float4(y[4], y[5], y[6], y[7]);
    }
    activate_blade<ACT>(y);
    float c0[4], c1[4];
    blade_to_pauli(y, c0, c1);  // c0 = (M00, M10), c1 = (M01, M11)
    float4* q = reinterpret_cast<float4*>(Y + ((size_t)row * d_out + j) * 8);  // [b][k][c]
    q[0] = make_float4(c0[0], c0[2], c0[1], c0[3]);
    q[1] = make_float4(c1[0], c1[2], c1[1], c1[3]);
  } else {
    size_t mv = OUT == kF32OutBladeT ? (size_t)j * P_max + row : (size_t)row * d_out + j;
    if constexpr (OUT == kF32OutPartial)  // partial planes: at row_map[row] when given (slot rows)
      mv = (size_t)split * P_max * d_out + (size_t)(row_map != nullptr ? row_map[row] : row) * d_out + j;
    else activate_blade<ACT>(y);
    float4* p = reinterpret_cast<float4*>(Y + mv * 8);
    p[0] = make_float4(y[0], y[1], y[2], y[3]);
    p[1] = make_float4(y[4], y[5], y[6], y[7]);
  }
}

// The routing of a small batch inside the up product (RQ > 0): every workgroup
// selects the top-k of every token from the logits (the selection of ygg_route,
// route_select.h), counts each expert's slots, finds its own row tile among the
// experts' rows and this expert's tokens in ascending order, and writes the routing
// arrays of its tile's rows (the first column tile) -- the same counts, offsets,
// permutation and slot positions as ygg_route.  Workgroup 0 writes counts and
// offsets.  The tile's rows of x are then read as blade rows and staged in LDS as
// Pauli rows (no converted copy of x in memory).
constexpr int kF32FuseTokens = 64 * kF32Waves;           // one token per thread
constexpr int kF32FuseSlots = kF32FuseTokens * kMaxTopK;
constexpr int kF32FuseQ = 4;                             // up to 8 RQ logits per token: E <= 32
constexpr int kF32FuseMaxD = 64;                         // d_in of a routed product: the staged tile fits part
struct F32Route {
  const float* logits = nullptr;
  int N = 0, k = 0;
  int32_t* topk_idx = nullptr;
  float* topk_w = nullptr;
  int32_t* counts = nullptr;
  int32_t* offsets = nullptr;
  int32_t* perm = nullptr;
  int32_t* slot_pos = nullptr;
  int32_t* row_slot = nullptr;  // when set: row_slot[row] = the row's slot t k + s
};

template <int ACT, int OUT, int WR, int RQ = 0>  // WR row blocks of 16 tokens per wave; RQ > 0: routed
__global__ __launch_bounds__(64 * kF32Waves) __attribute__((amdgpu_waves_per_eu(2))) void pauli_f32_kernel(
    const float* __restrict__ X, const int32_t* __restrict__ gather, const float* __restrict__ Wp,
    const float* __restrict__ bias, const int32_t* __restrict__ offsets, int E, int d_in, int d_out, int P_max,
    float* __restrict__ Y, float* __restrict__ Ypre, const int32_t* __restrict__ row_map, int n_xcd,
    F32Route route = F32Route{}) {
  constexpr int TOK = kF32Tok * WR;  // tokens per tile
  // the waves' partial sums: one round for WR = 1; for WR = 2 waves 2, 3 hand theirs
  // to waves 0, 1 first, so the buffer holds two waves' tiles
  constexpr int PW = WR == 1 ? kF32Waves : 2;
  __shared__ float4 part[PW][2 * TOK][kF32Cols + 1];  // (a0 re, a0 im, a1 re, a1 im)
  int e = 0, row0 = 0, row_end = 0;
  // The column tiles of one row tile run on one XCD, one after the other in
  // dispatch order, so its rows are read once into that XCD's L2: workgroup b runs
  // on XCD b mod n_xcd and takes column tile (b / n_xcd) mod n_ct of row tile
  // (b / (n_xcd n_ct)) n_xcd + b mod n_xcd.
  const int n_ct = (d_out + kF32Cols - 1) / kF32Cols;
  const int xcd = blockIdx.x % n_xcd, q = blockIdx.x / n_xcd;
  const int ct = q % n_ct, rt = (q / n_ct) * n_xcd + xcd;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: the K loop runs on scalars
  const int l32 = lane & 31, k = lane >> 5;
  // routed: LDS scratch on top of part (free until the partial sums), and the
  // expert's first row (this expert's tokens are rows_tok[row - row_beg])
  int row_beg = 0;
  int32_t* const s_sel = reinterpret_cast<int32_t*>(&part[0][0][0]);
  float* const s_w = reinterpret_cast<float*>(s_sel + kF32FuseSlots);
  int32_t* const s_off = reinterpret_cast<int32_t*>(s_w + kF32FuseSlots);  // kMaxExperts + 1
  int32_t* const s_cnt = s_off + kMaxExperts + 1;                             // kMaxExperts
  int32_t* const s_wv = s_cnt + kMaxExperts;                                  // kF32Waves
  int32_t* const rows_tok = s_wv + kF32Waves;                                 // kF32FuseTokens
  static_assert((2 * kF32FuseSlots + 2 * kMaxExperts + 1 + kF32Waves + kF32FuseTokens) * 4 <= (int)sizeof(part),
                "routing scratch exceeds the partial-sum buffer");
  static_assert(RQ == 0 || TOK * (kF32FuseMaxD + 1) * 32 <= (int)sizeof(part), "staged tile exceeds part");
  if constexpr (RQ > 0) {
    const int N = route.N, kk = route.k;
    // one token per thread: its logits, then its selection (select_one_thread)
    constexpr int EMAX = kSelLanes * RQ;
    float lg[EMAX];
    if ((E & 3) == 0 && (reinterpret_cast<uintptr_t>(route.logits) & 15) == 0) {  // the row in 16-byte pieces
#pragma unroll
      for (int x = 0; x < EMAX; x += 4) {
        const float4 v = (tid < N && x < E) ? *reinterpret_cast<const float4*>(route.logits + (size_t)tid * E + x)
                                            : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
        lg[x] = v.x;
        lg[x + 1] = v.y;
        lg[x + 2] = v.z;
        lg[x + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int x = 0; x < EMAX; ++x) lg[x] = (tid < N && x < E) ? route.logits[(size_t)tid * E + x] : -INFINITY;
    }
    if (tid < kMaxExperts) s_cnt[tid] = 0;
    __syncthreads();  // the counters are zero before any thread counts (the logits are in flight)
    if (tid < N) {
      int se[kMaxTopK];
      float sw[kMaxTopK];
      select_one_thread<EMAX>(lg, E, kk, se, sw);
#pragma unroll
      for (int s = 0; s < kMaxTopK; ++s)
        if (s < kk) {
          s_sel[tid * kk + s] = se[s];
          s_w[tid * kk + s] = sw[s];
          atomicAdd(&s_cnt[se[s]], 1);
        }
    }
    __syncthreads();
    if (wave == 0) {  // exclusive scan of the counts over experts (E <= 64: one lane each)
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
    __syncthreads();
    if (blockIdx.x == 0 && blockIdx.z == 0 && tid <= E) {
      if (tid < E) route.counts[tid] = s_off[tid + 1] - s_off[tid];
      route.offsets[tid] = s_off[tid];
    }
    // this workgroup's row tile (as f32_find_tile, over the offsets just made)
    bool found = false;
    {
      int acc_t = 0;
      for (int x = 0; x < E && !found; ++x) {
        const int beg = s_off[x], end = s_off[x + 1];
        const int nt = (end - beg + TOK - 1) / TOK;
        if (rt < acc_t + nt) {
          e = x;
          row_beg = beg;
          row0 = beg + (rt - acc_t) * TOK;
          row_end = end;
          found = true;
        }
        acc_t += nt;
      }
    }
    if (!found) return;  // uniform
    // this expert's tokens in ascending order: a ballot per wave, then wave bases
    bool mine = false;
    if (tid < N)
      for (int s = 0; s < kk; ++s) mine |= s_sel[tid * kk + s] == e;
    const uint64_t bal = __ballot(mine);
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    if (lane == 0) s_wv[wave] = __popcll(bal);
    __syncthreads();
    if (mine) {
      int base = 0;
      for (int w = 0; w < wave; ++w) base += s_wv[w];
      rows_tok[base + __popcll(bal & lt_mask)] = tid;
    }
    __syncthreads();
    if (ct == 0 && blockIdx.z == 0) {  // the routing arrays of this tile's rows
      for (int r = row0 + tid; r < min(row0 + TOK, row_end); r += 64 * kF32Waves) {
        const int t = rows_tok[r - row_beg];
        int s = 0;
        while (s_sel[t * kk + s] != e) ++s;
        const int f = t * kk + s;
        route.topk_idx[f] = e;
        route.topk_w[f] = s_w[f];
        route.slot_pos[f] = r;
        route.perm[r] = t;
        if (route.row_slot != nullptr) route.row_slot[r] = f;
      }
    }
  } else {
    if (!f32_find_tile<TOK>(offsets, E, rt, e, row0, row_end)) return;
  }
  const int col0 = ct * kF32Cols;
  const int split = blockIdx.z, splits = gridDim.z;

  // A operand: GEMM row (t, b) = l32 of row block r, real (k = 0) or imaginary (k = 1)
  // part.  Routed: the tile's rows of x, blade to Pauli rows (the conversion's adds),
  // staged in LDS over part -- every thread issues the loads of its share at once --
  // with rows padded by one multivector, so that a wave's 16 rows spread over the banks.
  const float* arow[WR];
  if constexpr (RQ > 0) {
    float* const xs = reinterpret_cast<float*>(&part[0][0][0]);
    const int rs = (d_in + 1) * 8;  // floats per staged row
    const int nq = TOK * d_in;      // multivectors of the tile
    constexpr int kStage = 2 * kF32Tok * kF32FuseMaxD / (64 * kF32Waves);
    float4 v[kStage][2];
#pragma unroll
    for (int u = 0; u < kStage; ++u) {
      const int q = tid + u * 64 * kF32Waves;
      if (q < nq) {
        const int r = q / d_in, i = q - r * d_in;
        const int m = min(row0 + r, row_end - 1);  // rows past the expert's range: computed, not stored
        const float4* src = reinterpret_cast<const float4*>(X + ((size_t)rows_tok[m - row_beg] * d_in + i) * 8);
        v[u][0] = src[0];
        v[u][1] = src[1];
      }
    }
    __syncthreads();  // the routing scratch is read: the staged rows may overwrite it
#pragma unroll
    for (int u = 0; u < kStage; ++u) {
      const int q = tid + u * 64 * kF32Waves;
      if (q < nq) {
        const int r = q / d_in, i = q - r * d_in;
        const float b[8] = {v[u][0].x, v[u][0].y, v[u][0].z, v[u][0].w, v[u][1].x, v[u][1].y, v[u][1].z, v[u][1].w};
        store_pauli_f32(xs + r * rs + i * 8, b);
      }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < WR; ++r) arow[r] = xs + (r * kF32Tok + (l32 >> 1)) * rs + ((l32 & 1) * 2 + k) * 2;
  } else {
#pragma unroll
    for (int r = 0; r < WR; ++r) {
      int m = row0 + r * kF32Tok + (l32 >> 1);
      m = m < row_end ? m : row_end - 1;  // rows past the expert's range are computed, not stored
      const int src = gather ? gather[m] : m;
      arow[r] = X + (size_t)src * d_in * 8 + ((l32 & 1) * 2 + k) * 2;
    }
  }
  // B operand: output column j (clamped: columns past d_out are not stored)
  const int jc = min(col0 + l32, d_out - 1);
  const float* wrow = Wp + (((size_t)e * d_in * 2 + k) * d_out + jc) * 8;
  // contraction range of this (split, wave)
  const int per_split = (d_in + splits - 1) / splits;
  const int is0 = split * per_split, is1 = min(d_in, is0 + per_split);
  const int per_wave = (max(is1 - is0, 0) + kF32Waves - 1) / kF32Waves;
  const int i0 = is0 + wave * per_wave, i1 = min(is1, i0 + per_wave);

  f32x16v_t acc[WR][2][2];
  f32_kloop<WR>(acc, arow, wrow, (size_t)2 * d_out * 8, i0, i1);
  if constexpr (RQ > 0) __syncthreads();  // every wave has read the staged rows before part is written
  // lane holds column l32, GEMM rows 8 (v / 4) + 4 k + v % 4 of each row block
  if constexpr (WR == 2) {
    if (wave >= 2) {
#pragma unroll
      for (int r = 0; r < WR; ++r)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          part[wave - 2][r * 32 + 8 * (v >> 2) + 4 * k + (v & 3)][l32] =
              make_float4(acc[r][0][0][v], acc[r][0][1][v], acc[r][1][0][v], acc[r][1][1][v]);
    }
    __syncthreads();
    if (wave < 2) {
#pragma unroll
      for (int r = 0; r < WR; ++r)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float4 o = part[wave][r * 32 + 8 * (v >> 2) + 4 * k + (v & 3)][l32];
          acc[r][0][0][v] += o.x;
          acc[r][0][1][v] += o.y;
          acc[r][1][0][v] += o.z;
          acc[r][1][1][v] += o.w;
        }
    }
    __syncthreads();
  }
  if (WR == 1 || wave < 2) {
#pragma unroll
    for (int r = 0; r < WR; ++r)
#pragma unroll
      for (int v = 0; v < 16; ++v)
        part[wave][r * 32 + 8 * (v >> 2) + 4 * k + (v & 3)][l32] =
            make_float4(acc[r][0][0][v], acc[r][0][1][v], acc[r][1][0][v], acc[r][1][1][v]);
  }
  __syncthreads();

#pragma unroll
  for (int h = 0; h < (TOK * kF32Cols) / (64 * kF32Waves); ++h) {
    const int o = tid + h * 64 * kF32Waves;
    const int t = o / kF32Cols, jj = o % kF32Cols;
    const int row = row0 + t, j = col0 + jj;
    if (row >= row_end || j >= d_out) continue;
    float4 s0 = part[0][2 * t][jj], s1 = part[0][2 * t + 1][jj];  // b = 0, 1
#pragma unroll
    for (int w = 1; w < PW; ++w) {
      const float4 p0 = part[w][2 * t][jj], p1 = part[w][2 * t + 1][jj];
      s0.x += p0.x; s0.y += p0.y; s0.z += p0.z; s0.w += p0.w;
      s1.x += p1.x; s1.y += p1.y; s1.z += p1.z; s1.w += p1.w;
    }
    // Y[a][b]: a = 0 -> (x, y), a = 1 -> (z, w); b from the row
    f32_store_mv<ACT, OUT>(s0.x, s0.y, s1.x, s1.y, s0.z, s0.w, s1.z, s1.w, bias, e, row, j, d_out, split, P_max, Y,
                           Ypre, row_map);
  }
}

// (E, d_out, d_in, 8) fp32 blade -> format 4; one thread per (e, j, i)
__global__ __launch_bounds__(256) void pauli_f32_prep_kernel(const float* __restrict__ W, int E, int d_out, int d_in,
                                                             float* __restrict__ out) {
  const size_t n = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (n >= (size_t)E * d_out * d_in) return;
  const int i = (int)(n % d_in);
  const size_t ej = n / d_in;
  float x[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) x[c] = 0.5f * W[n * 8 + c];
  float c0[4], c1[4];
  blade_to_pauli(x, c0, c1);
  // W[a][c]: (a, c) = (0, 0) M00, (0, 1) M01, (1, 0) M10, (1, 1) M11 as (u, v)
  const float u[2][2] = {{c0[0], c1[0]}, {c0[2], c1[2]}};  // [a][c]
  const float v[2][2] = {{c0[1], c1[1]}, {c0[3], c1[3]}};
  const size_t e = ej / d_out, j = ej % d_out;
  float* r0 = out + (((e * d_in + i) * 2 + 0) * d_out + j) * 8;  // k = 0: (u, v)
  float* r1 = out + (((e * d_in + i) * 2 + 1) * d_out + j) * 8;  // k = 1: (-v, u)
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      r0[(c * 2 + a) * 2 + 0] = u[a][c];
      r0[(c * 2 + a) * 2 + 1] = v[a][c];
      r1[(c * 2 + a) * 2 + 0] = -v[a][c];
      r1[(c * 2 + a) * 2 + 1] = u[a][c];
    }
}

// blade fp32 rows (rows, d, 8) -> Pauli rows; one thread per multivector
__global__ __launch_bounds__(256) void blade_to_pauli_f32_rows_kernel(const float* __restrict__ x, int rows, int d,
                                                                      float* __restrict__ out) {
  const size_t n = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (n >= (size_t)rows * d) return;
  pauli_rows_f32_one(x, n, out);
}

// b (K, N, 8) fp32 blade -> Pauli rows of its transpose (N, K): row n holds b[:, n].
// Tiles of 32 columns n x 8 rows k pass through LDS, so both the reads (32
// consecutive n of one k) and the writes (8 consecutive k of one n) are contiguous.
// Thread 0 of workgroup 0 also writes the one-expert offsets {0, N}.
__global__ __launch_bounds__(256) void pauli_f32_rows_t_kernel(const float* __restrict__ b, int K, int N,
                                                               float* __restrict__ out, int32_t* __restrict__ offsets) {
  __shared__ float4 tile[8][32][2];
  const int n0 = blockIdx.x * 32, k0 = blockIdx.y * 8, t = threadIdx.x;
  if (blockIdx.x == 0 && blockIdx.y == 0 && t == 0) {
    offsets[0] = 0;
    offsets[1] = N;
  }
  {
    const int kk = t >> 5, nn = t & 31, k = k0 + kk, n = n0 + nn;
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (k < K && n < N) {
      const float4 p0 = reinterpret_cast<const float4*>(b + ((size_t)k * N + n) * 8)[0];
      const float4 p1 = reinterpret_cast<const float4*>(b + ((size_t)k * N + n) * 8)[1];
      v[0] = p0.x; v[1] = p0.y; v[2] = p0.z; v[3] = p0.w; v[4] = p1.x; v[5] = p1.y; v[6] = p1.z; v[7] = p1.w;
    }
    float c0[4], c1[4];
    blade_to_pauli(v, c0, c1);
    tile[kk][nn][0] = make_float4(c0[0], c0[2], c0[1], c0[3]);  // [b][k][c], as blade_to_pauli_f32_rows_kernel
    tile[kk][nn][1] = make_float4(c1[0], c1[2], c1[1], c1[3]);
  }
  __syncthreads();
  {
    const int nn = t >> 3, kk = t & 7, k = k0 + kk, n = n0 + nn;
    if (k < K && n < N) {
      float4* q = reinterpret_cast<float4*>(out + ((size_t)n * K + k) * 8);
      q[0] = tile[kk][nn][0];
      q[1] = tile[kk][nn][1];
    }
  }
}

}  // namespace ygg

using namespace ygg;

namespace {
int f32_cus() {  // CUs of the current device
  static thread_local int cached_dev = -1, cached = 64;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  if (dev != cached_dev) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 64;
    cached = cus;
    cached_dev = dev;
  }
  return cached;
}
int f32_xcds() { return (f32_cus() % 8 == 0) ? 8 : 1; }  // XCDs workgroups are dealt to round robin (8 on MI355X)

// x: (row tile, column tile) pairs, row tiles rounded up to a multiple of the XCD
// count; z: contraction splits
dim3 f32_grid(int P_max, int E, int d_out, int splits, int n_xcd, int tok) {
  long long rts = ((long long)P_max + tok - 1) / tok + E;
  rts = (rts + n_xcd - 1) / n_xcd * n_xcd;
  return dim3((unsigned)(rts * ((d_out + kF32Cols - 1) / kF32Cols)), 1, splits);
}

// 16- or 32-token tiles (32: two row blocks per wave, sharing the weight loads).
// Small grids: 16 while every workgroup gets a CU of its own, 32 when that keeps
// every workgroup on a CU of its own and 16 would put two on some (C1 step 65 ->
// 53 us).  Large grids: 32 for long contractions (d_in >= 2 d_out, where a tile's
// weight stream dominates: at the C3 shape the d_in = 512 products 1.94 -> 1.59 ms,
// while the d_in = 128 ones go 1.39 -> 1.66 ms), 16 otherwise.
template <int OUT>
int launch_f32_act(int act, int splits, hipStream_t st, const float* X, const int32_t* gather, const float* W,
                   const float* bias, const int32_t* offsets, int E, int d_in, int d_out, int P_max, float* Y,
                   float* Ypre = nullptr, const int32_t* row_map = nullptr, const F32Route* route = nullptr) {
  const int n_xcd = f32_xcds();
  const dim3 g1 = f32_grid(P_max, E, d_out, splits, n_xcd, kF32Tok);
  const dim3 g2 = f32_grid(P_max, E, d_out, splits, n_xcd, 2 * kF32Tok);
  const long long n1 = (long long)g1.x * g1.z, n2 = (long long)g2.x * g2.z, cus = f32_cus();
  bool two;
  if (n1 <= cus) two = false;        // one workgroup per CU already: the shorter chains win
  else if (n2 <= cus) two = true;    // 32-token tiles fit in one workgroup per CU, 16-token ones would double up
  else two = d_in >= 2 * d_out && n2 >= kF32TwoBlockMinGroups;
  const dim3 grid = two ? g2 : g1;
#define YGG_F(A)                                                                                              \
  if (route != nullptr) {                                                                                     \
    if constexpr (OUT == kF32OutPauliRows) {                                                                  \
      if (two && E <= kSelLanes)                                                                              \
        pauli_f32_kernel<A, OUT, 2, 1><<<grid, 64 * kF32Waves, 0, st>>>(                                      \
            X, nullptr, W, bias, nullptr, E, d_in, d_out, P_max, Y, Ypre, row_map, n_xcd, *route);            \
      else if (two)                                                                                           \
        pauli_f32_kernel<A, OUT, 2, kF32FuseQ><<<grid, 64 * kF32Waves, 0, st>>>(                              \
            X, nullptr, W, bias, nullptr, E, d_in, d_out, P_max, Y, Ypre, row_map, n_xcd, *route);            \
      else if (E <= kSelLanes)                                                                                \
        pauli_f32_kernel<A, OUT, 1, 1><<<grid, 64 * kF32Waves, 0, st>>>(                                      \
            X, nullptr, W, bias, nullptr, E, d_in, d_out, P_max, Y, Ypre, row_map, n_xcd, *route);            \
      else                                                                                                    \
        pauli_f32_kernel<A, OUT, 1, kF32FuseQ><<<grid, 64 * kF32Waves, 0, st>>>(                              \
            X, nullptr, W, bias, nullptr, E, d_in, d_out, P_max, Y, Ypre, row_map, n_xcd, *route);            \
    }                                                                                                         \
  } else if (two)                                                                                             \
    pauli_f32_kernel<A, OUT, 2><<<grid, 64 * kF32Waves, 0, st>>>(X, gather, W, bias, offsets, E, d_in, d_out, \
                                                                 P_max, Y, Ypre, row_map, n_xcd);             \
  else                                                                                                        \
    pauli_f32_kernel<A, OUT, 1><<<grid, 64 * kF32Waves, 0, st>>>(X, gather, W, bias, offsets, E, d_in, d_out, \
                                                                 P_max, Y, Ypre, row_map, n_xcd)
  switch (act) {
    case kActNone: YGG_F(kActNone); break;
    case kActGelu: YGG_F(kActGelu); break;
    case kActRelu: YGG_F(kActRelu); break;
    default: YGG_F(kActSigmoid); break;
  }
#undef YGG_F
  return check_launch("pauli_f32");
}
}  // namespace

int ygg::pauli_f32_prepare_weights(const float* W, int E, int d_out, int d_in, void* out, hipStream_t stream) {
  const size_t total = (size_t)E * d_out * d_in;
  pauli_f32_prep_kernel<<<(unsigned)((total + 255) / 256), 256, 0, stream>>>(W, E, d_out, d_in,
                                                                             static_cast<float*>(out));
  return check_launch("pauli_f32_prep");
}

// Contraction splits of the partial-plane product: as many as keep every workgroup of
// 16-token tiles on a CU of its own (the launch rounds row tiles up to the XCD count)
int ygg::pauli_f32_splits(int P_max, int E, int d_in, int d_out) {
  const int n_xcd = f32_xcds();
  long long rts = ((long long)P_max + kF32Tok - 1) / kF32Tok + E;
  rts = (rts + n_xcd - 1) / n_xcd * n_xcd;
  const long long tiles = rts * ((d_out + kF32Cols - 1) / kF32Cols);
  long long s = f32_cus() / tiles;
  s = std::min<long long>(s, std::max(1, d_in / 16));
  return (int)std::max<long long>(s, 1);
}

int ygg::pauli_f32_linear_partial(const float* x, int P_max, const float* w, const float* bias,
                                  const int32_t* offsets, int E, int d_in, int d_out, int splits, float* y_planes,
                                  hipStream_t stream, const int32_t* row_map) {
  if (P_max == 0) return 0;
  return launch_f32_act<kF32OutPartial>(kActNone, splits, stream, x, nullptr, w, bias, offsets, E, d_in, d_out, P_max,
                                        y_planes, nullptr, row_map);
}

bool ygg::pauli_f32_route_fusable(int N, int E, int k, int d_in) {
  return N >= 1 && N <= kF32FuseTokens && E >= 1 && E <= kSelLanes * kF32FuseQ && k >= 1 && k <= kMaxTopK &&
         k <= E && d_in >= 1 && d_in <= kF32FuseMaxD;
}

int ygg::pauli_f32_up_routed(const float* x, const float* logits, int N, int E, int k, int32_t* topk_idx,
                             float* topk_w, int32_t* counts, int32_t* offsets, int32_t* perm, int32_t* slot_pos,
                             int32_t* row_slot, const float* w, const float* bias, int d_in, int d_out, int act,
                             float* y_pauli, float* y_pre, hipStream_t stream) {
  YGG_CHECK_ARG(pauli_f32_route_fusable(N, E, k, d_in), "routed fp32 up product: N=%d E=%d k=%d d_in=%d", N, E, k,
                d_in);
  F32Route r;
  r.logits = logits;
  r.N = N;
  r.k = k;
  r.topk_idx = topk_idx;
  r.topk_w = topk_w;
  r.counts = counts;
  r.offsets = offsets;
  r.perm = perm;
  r.slot_pos = slot_pos;
  r.row_slot = row_slot;
  return launch_f32_act<kF32OutPauliRows>(act, 1, stream, x, nullptr, w, bias, nullptr, E, d_in, d_out, N * k, y_pauli,
                                          y_pre, nullptr, &r);
}

int ygg::pauli_f32_linear_save_pre(const float* x, const int32_t* gather, int P_max, const float* w,
                                   const float* bias, const int32_t* offsets, int E, int d_in, int d_out, int act,
                                   float* y_pauli, float* y_pre, hipStream_t stream) {
  if (P_max == 0) return 0;
  return launch_f32_act<kF32OutPauliRows>(act, 1, stream, x, gather, w, bias, offsets, E, d_in, d_out, P_max, y_pauli,
                                          y_pre);
}

YGG_API int ygg_pauli_rows_from_blade_f32(const float* x, int rows, int d, float* out, hipStream_t stream) {
  YGG_CHECK_ARG(rows >= 0 && d >= 1, "ygg_pauli_rows_from_blade_f32: rows=%d d=%d", rows, d);
  if (rows == 0) return 0;
  YGG_CHECK_ARG(x && out, "ygg_pauli_rows_from_blade_f32: null pointer");
  const size_t n = (size_t)rows * d;
  blade_to_pauli_f32_rows_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(x, rows, d, out);
  return check_launch("blade_to_pauli_f32_rows");
}

YGG_API int ygg_pauli_grouped_linear_f32(const float* x, const int32_t* gather, int P_max, const float* w,
                                         const float* bias, const int32_t* offsets, int E, int d_in, int d_out,
                                         int act, float* y, int y_layout, hipStream_t stream) {
  YGG_CHECK_ARG(y_layout == kF32OutPauliRows || y_layout == kF32OutBlade,
                "ygg_pauli_grouped_linear_f32: y layout %d", y_layout);
  YGG_CHECK_ARG(act >= kActNone && act <= kActSigmoid, "ygg_pauli_grouped_linear_f32: activation %d", act);
  YGG_CHECK_ARG(E >= 1 && E <= 64 && P_max >= 0 && d_in >= 1 && d_out >= 1,
                "ygg_pauli_grouped_linear_f32: bad sizes E=%d P=%d d_in=%d d_out=%d", E, P_max, d_in, d_out);
  if (P_max == 0) return 0;
  YGG_CHECK_ARG(x && w && offsets && y, "ygg_pauli_grouped_linear_f32: null pointer");
  if (y_layout == kF32OutPauliRows)
    return launch_f32_act<kF32OutPauliRows>(act, 1, stream, x, gather, w, bias, offsets, E, d_in, d_out, P_max, y);
  return launch_f32_act<kF32OutBlade>(act, 1, stream, x, gather, w, bias, offsets, E, d_in, d_out, P_max, y);
}

// ---------------------------------------------------------------------------
// geom_matmul: out[m, n] = sum_k a[m, k] b[k, n] as one fp32 Pauli product --
// a is the weight (d_out = M, d_in = K) of a single expert, the columns of b are
// the rows, and the output is written transposed, straight into (M, N, 8).
// ---------------------------------------------------------------------------

namespace {
__global__ __launch_bounds__(256) void gm_zero_kernel(float* __restrict__ out, size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) out[i] = 0.f;
}

constexpr size_t kGmAlign = 256;
size_t gm_align(size_t n) { return (n + kGmAlign - 1) / kGmAlign * kGmAlign; }
size_t gm_w_bytes(int M, int K) { return gm_align((size_t)M * K * 2 * 8 * sizeof(float)); }
size_t gm_x_bytes(int K, int N) { return gm_align((size_t)N * K * 8 * sizeof(float)); }
}  // namespace

YGG_API size_t ygg_geom_matmul_f32_workspace_bytes(int M, int K, int N) {
  if (M <= 0 || K <= 0 || N <= 0) return 0;
  return gm_w_bytes(M, K) + gm_x_bytes(K, N) + kGmAlign;
}

YGG_API int ygg_geom_matmul_f32_ws(const float* a, const float* b, float* out, int M, int K, int N, void* workspace,
                                   size_t workspace_bytes, hipStream_t stream) {
  YGG_CHECK_ARG(M >= 0 && K >= 0 && N >= 0, "ygg_geom_matmul_f32: bad sizes M=%d K=%d N=%d", M, K, N);
  if (M == 0 || N == 0) return 0;
  YGG_CHECK_ARG(out, "ygg_geom_matmul_f32: null output");
  if (K == 0) {  // an empty sum (a fill kernel, no memset node, so that the call can be captured)
    const size_t n = (size_t)M * N * 8;
    gm_zero_kernel<<<(unsigned)std::min<size_t>((n + 255) / 256, 65535), 256, 0, stream>>>(out, n);
    return check_launch("geom_matmul (K = 0)");
  }
  YGG_CHECK_ARG(a && b, "ygg_geom_matmul_f32: null input");
  YGG_CHECK_ARG((size_t)N * K * 8 < ((size_t)1 << 31) && (size_t)M * K * 16 < ((size_t)1 << 31),
                "ygg_geom_matmul_f32: operands of 2^31 floats or more (M=%d K=%d N=%d)", M, K, N);
  const size_t need = ygg_geom_matmul_f32_workspace_bytes(M, K, N);
  YGG_CHECK_ARG(workspace != nullptr && workspace_bytes >= need,
                "ygg_geom_matmul_f32: workspace of %zu bytes, %zu needed", workspace_bytes, need);
  char* ws = static_cast<char*>(workspace);
  float* wp = reinterpret_cast<float*>(ws);
  float* xp = reinterpret_cast<float*>(ws + gm_w_bytes(M, K));
  int32_t* off = reinterpret_cast<int32_t*>(ws + gm_w_bytes(M, K) + gm_x_bytes(K, N));
  if (pauli_f32_prepare_weights(a, 1, M, K, wp, stream)) return -1;
  const dim3 tgrid((unsigned)((N + 31) / 32), (unsigned)((K + 7) / 8));
  pauli_f32_rows_t_kernel<<<tgrid, 256, 0, stream>>>(b, K, N, xp, off);
  if (check_launch("pauli_f32_rows_t")) return -1;
  return launch_f32_act<kF32OutBladeT>(kActNone, 1, stream, xp, nullptr, wp, nullptr, off, 1, K, M, N, out);
}

YGG_API int ygg_geom_matmul_f32(const float* a, const float* b, float* out, int M, int K, int N, hipStream_t stream) {
  YGG_CHECK_ARG(M >= 0 && K >= 0 && N >= 0, "ygg_geom_matmul_f32: bad sizes M=%d K=%d N=%d", M, K, N);
  const size_t need = ygg_geom_matmul_f32_workspace_bytes(M, K, N);
  if (need == 0) return ygg_geom_matmul_f32_ws(a, b, out, M, K, N, nullptr, 0, stream);
  void* ws = nullptr;  // stream-ordered, returned to the pool after the product
  const hipError_t me = hipMallocAsync(&ws, need, stream);
  YGG_CHECK_ARG(me == hipSuccess, "ygg_geom_matmul_f32: workspace of %zu bytes: %s", need, hipGetErrorString(me));
  const int rc = ygg_geom_matmul_f32_ws(a, b, out, M, K, N, ws, need, stream);
  const hipError_t fe = hipFreeAsync(ws, stream);
  if (rc) return rc;
  YGG_CHECK_ARG(fe == hipSuccess, "ygg_geom_matmul_f32: freeing the workspace: %s", hipGetErrorString(fe));
  return 0;
}
