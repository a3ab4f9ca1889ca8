// pauli_gemm.hip -- grouped CliffordLinear expert products as complex GEMMs
// on the bf16 MFMA units of gfx950.
//
// Replaces, for every expert e of the MoE-HLM layer, CliffordLinear.forward
// (holograph/layers/clifford_linear.py:101-123), i.e. geom_matmul
// (rune/ops/batched.py:320-344) on that expert's rows, and the grade-wise
// activation (holograph/layers/activations.py:15-128) after the up projection.
//
// Algebra
// -------
// Cl(3,0) is isomorphic to the 2x2 complex matrices (Pauli representation):
//   e1 -> sx, e2 -> sy, e3 -> sz, e12 -> i sz, e13 -> -i sy, e23 -> i sx, e123 -> i I.
// A multivector  s + v1 e1 + v2 e2 + v3 e3 + b12 e12 + b13 e13 + b23 e23 + t e123
// maps to
//   M00 = (s + v3) + i (t + b12)     M01 = (v1 - b13) + i (b23 - v2)
//   M10 = (v1 + b13) + i (b23 + v2)  M11 = (s - v3) + i (t - b12)
// and the geometric product maps to the matrix product.  A CliffordLinear
//   y[m, j] = sum_i W[j, i] x[m, i]
// is therefore the complex contraction  Y_mj[a, b] = sum_{i, c} W_ji[a, c] X_mi[c, b]:
// rows (m, b), contraction (i, c), columns (j, a) -- 32 real multiply-adds per
// (input, output) multivector pair instead of the 64 of the 8x8 block L(w).
//
// Layouts
// -------
// * Pauli half-rows ("PH"): a row of d multivectors is stored as two halves,
//   b = 0 then b = 1; half b holds, for every multivector i, column b of its
//   matrix as 4 reals (c0 re, c0 im, c1 re, c1 im).  Row (m, b) of the GEMM is
//   then one contiguous run of 4 d values.
// * Prepared weights ("PW", bf16): per (expert, j, input pair p = i/2), 32
//   bytes: [a = 0 | a = 1] x [i = 2p | 2p + 1] x [c0 | c1] x (u, -v), where
//   u + iv = W_ji[a, c] / 2.  The 1/2 makes the inverse map a plain sum.
//   (u, -v) is the B operand of the real part; the imaginary part uses the
//   A operand rotated within each complex pair, (re, im) -> (im, -re).
//
// Work decomposition
// ------------------
// v_mfma_f32_32x32x16_bf16: one K step is 4 input multivectors.  A wave owns
// WR x 16 tokens (WR row blocks of 32 GEMM rows) and WC x 32 output
// multivectors, with four accumulators per block pair (a = 0, 1) x (re, im),
// so all 8 reals of an output multivector land in one lane: the inverse map,
// bias, grade-wise activation and the output layout are fused into the
// epilogue with no shuffles.
//
// The launch is persistent: two workgroups per CU walk a flat stream of
// (tile, K chunk) steps.  Tiles are (row tile of one expert) x (column tile);
// row tiles never straddle experts (device-side offsets, no host sync).  The
// tile list is cut into one contiguous range per XCD (workgroup b runs on XCD
// b mod 8), so the workgroups sharing an L2 work on neighbouring row tiles of
// the same expert.  Each step stages KC input multivectors of the activation
// and weight tiles in LDS (double buffered, one barrier per step); the raw
// buffer loads of step f + 1 are issued before step f computes, so the next
// tile's first loads are in flight during the current tile's epilogue.
// Activation rows are gathered through the expert-grouped row index, which
// fuses the dispatch copy into the up projection.

#include <type_traits>

#include "pauli_common.h"

namespace ygg {

enum PauliIn : int { kInBladeGather = 0, kInPauliRows = 1 };
enum PauliOut : int { kOutPauliRows = 0, kOutBlade = 1 };

constexpr int kPauliMaxExperts = 64;

template <int WR_, int WC_, int BWT_, int BWJ_, int KC_>
struct PauliTile {
  static constexpr int WR = WR_, WC = WC_, BWT = BWT_, BWJ = BWJ_, KC = KC_;
  static constexpr int NT = 64 * BWT * BWJ;       // threads
  static constexpr int T = BWT * WR * 16;         // tokens per tile
  static constexpr int BN = BWJ * WC * 32;        // output multivectors per tile
  static constexpr int A_STRIDE = KC * 8 + 16;    // bytes per LDS row (m, b): KC mv x 4 bf16, +16 pad
  static constexpr int W_STRIDE = KC * 16 + 16;   // bytes per LDS column j: KC/2 pairs x 32 B, +16 pad
  static constexpr int A_BYTES = 2 * T * A_STRIDE;
  static constexpr int W_BYTES = BN * W_STRIDE;
  static constexpr int STAGE = A_BYTES + W_BYTES;
  // 16-byte global pieces per stage
  static constexpr int A_ITEMS_GATHER = T * KC;   // one blade multivector each
  static constexpr int A_ITEMS_ROWS = T * KC;     // 2T rows x KC/2 pairs
  static constexpr int W_ITEMS = BN * KC;         // BN columns x KC/2 pairs x (a = 0, 1)
  static constexpr int A_PER = A_ITEMS_ROWS / NT, W_PER = W_ITEMS / NT;
  static_assert(KC % 4 == 0, "KC must be a multiple of the MFMA K step (4 multivectors)");
  static_assert(A_ITEMS_ROWS % NT == 0 && W_ITEMS % NT == 0, "staging split");
};

struct PauliTileInfo {
  int e, row0, row_end, col0;
  int half;  // -1: the whole tile; 0 / 1: only row block `half` of every wave
  // a compact tile (the last row tile of an expert, at most 32 rows): computed as a
  // half tile (block 0 of every wave), its rows staged at the token slots that block
  // covers, 0-15 and 32-47, so wave row group wt holds rows 16 wt .. 16 wt + 15
  bool compact = false;
};

// Epilogue of one tile for one wave: the inverse Pauli map, bias, grade-wise
// activation and the output layout, all in the lane that holds the 8 reals of
// an output multivector.  acc[rb][cb][a][re/im] is wave row block rb (of WR,
// each 16 tokens x b = 0, 1), column block cb (of WC, 32 output multivectors);
// bv[cb] is the bias of this lane's column in blade order, added here unless
// BIAS_IN_ACC (the accumulators started from it).  The output is written by
// buffer stores: y_rsrc starts at output row `row_base` and ends at the output's
// true end, the row-dependent part of each offset is a scalar, the lane's part a
// fixed per-lane offset.
template <int ACT, int OUT, int OUT_DT, int WR, int WC, int BWT, bool BIAS_IN_ACC>
__device__ __forceinline__ void pauli_tile_epilogue(const pf32x16_t (&acc)[WR][WC][2][2], const float (&bvs)[WC][8],
                                                    const PauliTileInfo& ti, int wave, int g, int l32, int d_out,
                                                    __amdgpu_buffer_rsrc_t y_rsrc, int row_base) {
  typedef unsigned int pu32x2_t __attribute__((ext_vector_type(2)));
  typedef unsigned int pu32x4_t __attribute__((ext_vector_type(4)));
  const int wt = wave % BWT, wj = wave / BWT;
  // bytes per output row (Pauli half-row pair, bf16 blade or fp32 blade row)
  constexpr int MV_BYTES = (OUT == kOutPauliRows || OUT_DT == kBF16) ? 16 : 32;
#pragma unroll
  for (int cb = 0; cb < WC; ++cb) {
    const int j = ti.col0 + (wj * WC + cb) * 32 + l32;
    if (j >= d_out) continue;
    const float* bv = bvs[cb];
    // lane part of the offset: token 2 g of the group of four, column j
    const uint32_t v_off = OUT == kOutPauliRows ? (uint32_t)((4 * g) * d_out + j) * 8
                                                : (uint32_t)((2 * g) * d_out + j) * MV_BYTES;
#pragma unroll
    for (int rb = 0; rb < WR; ++rb) {
      if (ti.half >= 0 && rb > 0) break;  // a half tile: the first accumulators hold block `half`
      const int rbr = ti.half >= 0 ? ti.half : rb;
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int rs = ti.row0 + (ti.compact ? wt * 16 : (wt * WR + rbr) * 16) + 4 * q + h;  // row of lanes with g = 0
          if (rs + 2 * g >= ti.row_end) continue;
          const uint32_t s_off = (uint32_t)(rs - row_base) * d_out * MV_BYTES;
          const int v0 = 4 * q + 2 * h;  // b = 0 at v0, b = 1 at v0 + 1
          float y[8];
          pauli_to_blade(acc[rb][cb][0][0][v0], acc[rb][cb][0][1][v0], acc[rb][cb][0][0][v0 + 1],
                         acc[rb][cb][0][1][v0 + 1], acc[rb][cb][1][0][v0], acc[rb][cb][1][1][v0],
                         acc[rb][cb][1][0][v0 + 1], acc[rb][cb][1][1][v0 + 1], y);
          if constexpr (!BIAS_IN_ACC) {
#pragma unroll
            for (int c = 0; c < 8; ++c) y[c] += bv[c];
          }
          activate_blade<ACT>(y);
          if constexpr (OUT == kOutPauliRows) {
            float c0[4], c1[4];
            blade_to_pauli(y, c0, c1);
            const pu32x2_t h0 = {pack2_bf16(c0[0], c0[1]), pack2_bf16(c0[2], c0[3])};
            const pu32x2_t h1 = {pack2_bf16(c1[0], c1[1]), pack2_bf16(c1[2], c1[3])};
            __builtin_amdgcn_raw_buffer_store_b64(h0, y_rsrc, v_off, s_off, 0);
            __builtin_amdgcn_raw_buffer_store_b64(h1, y_rsrc, v_off + (uint32_t)d_out * 8, s_off, 0);
          } else if constexpr (OUT_DT == kBF16) {
            const pu32x4_t o = {pack2_bf16(y[0], y[1]), pack2_bf16(y[2], y[3]), pack2_bf16(y[4], y[5]),
                                pack2_bf16(y[6], y[7])};
            __builtin_amdgcn_raw_buffer_store_b128(o, y_rsrc, v_off, s_off, 0);
          } else {
            const pu32x4_t lo = {__builtin_bit_cast(unsigned, y[0]), __builtin_bit_cast(unsigned, y[1]),
                                 __builtin_bit_cast(unsigned, y[2]), __builtin_bit_cast(unsigned, y[3])};
            const pu32x4_t hi = {__builtin_bit_cast(unsigned, y[4]), __builtin_bit_cast(unsigned, y[5]),
                                 __builtin_bit_cast(unsigned, y[6]), __builtin_bit_cast(unsigned, y[7])};
            __builtin_amdgcn_raw_buffer_store_b128(lo, y_rsrc, v_off, s_off, 0);
            __builtin_amdgcn_raw_buffer_store_b128(hi, y_rsrc, v_off + 16, s_off, 0);
          }
        }
    }
  }
}

// The accumulators of a tile started from the bias: entry (a, b) of the halved
// Pauli matrix of the lane's column bias, re and im (the weights hold W / 2, so
// the products are half the Pauli matrices and pauli_to_blade needs no scale).
template <int WR, int WC>
__device__ __forceinline__ void pauli_acc_from_bias(pf32x16_t (&acc)[WR][WC][2][2], const float (&bvs)[WC][8]) {
#pragma unroll
  for (int cb = 0; cb < WC; ++cb) {
    float c0[4], c1[4];
    blade_to_pauli(bvs[cb], c0, c1);  // c0 = (M00, M10), c1 = (M01, M11)
    // [a][re/im][b]
    const float e[2][2][2] = {{{0.5f * c0[0], 0.5f * c1[0]}, {0.5f * c0[1], 0.5f * c1[1]}},
                              {{0.5f * c0[2], 0.5f * c1[2]}, {0.5f * c0[3], 0.5f * c1[3]}}};
#pragma unroll
    for (int rb = 0; rb < WR; ++rb)
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int ri = 0; ri < 2; ++ri)
#pragma unroll
          for (int v = 0; v < 16; ++v) acc[rb][cb][a][ri][v] = e[a][ri][v & 1];
  }
}

template <int ACT, int IN, int OUT, int OUT_DT, class TL>
__global__ __launch_bounds__(TL::NT) __attribute__((amdgpu_waves_per_eu(2))) void pauli_gemm_kernel(
    const uint16_t* __restrict__ X, const int32_t* __restrict__ gather, const uint16_t* __restrict__ Wp,
    const float* __restrict__ bias, const int32_t* __restrict__ offsets, int E, int d_in, int d_out,
    void* __restrict__ Y, int n_xcd, uint32_t x_bytes, uint32_t y_bytes) {
  constexpr int NT = TL::NT, T = TL::T, BN = TL::BN, KC = TL::KC, WR = TL::WR, WC = TL::WC, BWT = TL::BWT;
  constexpr int A_PER = TL::A_PER, W_PER = TL::W_PER;
  __shared__ __attribute__((aligned(16))) unsigned char smem[2 * TL::STAGE];
  __shared__ int s_off[kPauliMaxExperts + 1];   // expert row offsets
  __shared__ int s_tbeg[kPauliMaxExperts + 1];  // first row tile of each expert

  const int tid = threadIdx.x;
  for (int i = tid; i <= E; i += NT) s_off[i] = offsets[i];
  __syncthreads();
  if (tid == 0) {
    int acc = 0;
    for (int x = 0; x < E; ++x) {
      s_tbeg[x] = acc;
      acc += (s_off[x + 1] - s_off[x] + T - 1) / T;
    }
    s_tbeg[E] = acc;
  }
  __syncthreads();

  const int CT = (d_out + BN - 1) / BN;
  const int n_tiles = s_tbeg[E] * CT;
  const int nk = (d_in + KC - 1) / KC;
  // this workgroup's tiles: XCD x gets the contiguous range [lo, hi), its
  // workgroups take every per_xcd-th tile of it
  const int per_xcd = gridDim.x / n_xcd;
  const int xcd = blockIdx.x % n_xcd, slot = blockIdx.x / n_xcd;
  const int lo = (int)((long long)n_tiles * xcd / n_xcd), hi = (int)((long long)n_tiles * (xcd + 1) / n_xcd);
  // Whole rounds of per_xcd tiles first.  A remainder of at most per_xcd / 2 tiles
  // would leave most workgroups idle while a few run one more tile, so each of those
  // tiles is cut in two halves -- a half computes one of each wave's two row blocks --
  // and the halves go to twice as many workgroups.
  const int R = hi - lo, rounds = R / per_xcd, rem = R - rounds * per_xcd;
  const bool split = WR == 2 && rem > 0 && 2 * rem <= per_xcd;
  const int n_full = split ? rounds : (R > slot ? (R - slot + per_xcd - 1) / per_xcd : 0);
  const int n_mine = n_full + ((split && slot < 2 * rem) ? 1 : 0);
  const int total = n_mine * nk;

  auto decode = [&](int n) __attribute__((always_inline)) {  // n-th tile of this workgroup
    const bool half = n >= n_full;
    const int L = half ? lo + rounds * per_xcd + (slot >> 1) : lo + slot + n * per_xcd;
    const int rt = L / CT, ct = L - rt * CT;
    int a = 0, b = E - 1;  // last expert with s_tbeg <= rt (experts with no tiles are skipped)
    while (a < b) {
      const int m = (a + b + 1) >> 1;
      if (s_tbeg[m] <= rt) a = m;
      else b = m - 1;
    }
    PauliTileInfo t;
    t.e = a;
    t.row0 = s_off[a] + (rt - s_tbeg[a]) * T;
    t.row_end = s_off[a + 1];
    t.col0 = ct * BN;
    t.half = half ? (slot & 1) : -1;
    return t;
  };

  const int lane = tid & 63, wave = tid >> 6;
  const int wt = wave % BWT, wj = wave / BWT;
  const int g = lane >> 5, l32 = lane & 31;
  const int IP = d_in >> 1;  // input pairs (d_in even)

  // ---- staging: global -> registers -> LDS --------------------------------
  // Staging loads are raw buffer loads: an offset past the end of the
  // descriptor's range reads zero, so the K tail and out-of-range columns
  // need no branches.  Row offsets are 32-bit: the host admits only operands
  // below 2 GiB, and x's range is its true size, so a row index past x's rows
  // reads zero rather than another row.
  const __amdgpu_buffer_rsrc_t x_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(X), (short)0,
                                                                          x_bytes, kBufferFlags);
  constexpr uint32_t kOff = 0x80000000u;  // reads zero
  PauliTileInfo ld = {0, 0, 1, 0, -1};  // tile of the chunk being loaded
  __amdgpu_buffer_rsrc_t w_rsrc = x_rsrc;
  uint32_t a_row[A_PER];  // byte offset of each staged A item's row, fixed for a tile
  auto load_chunk = [&](int f, uint4 (&ra)[A_PER], uint4 (&rw)[W_PER]) {
    const int kc = f % nk;
    if (kc == 0) {
      ld = decode(f / nk);
      w_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(Wp) + (size_t)ld.e * d_out * IP * 16, (short)0,
                                                 (uint32_t)d_out * IP * 32, kBufferFlags);
#pragma unroll
      for (int u = 0; u < A_PER; ++u) {
        const int item = tid + u * NT;
        const int tl = (IN == kInBladeGather) ? item / KC : (item / (KC / 2)) >> 1;
        int r = ld.row0 + tl;
        r = r < ld.row_end ? r : ld.row_end - 1;
        const int src = gather ? gather[r] : r;
        if constexpr (IN == kInBladeGather)
          a_row[u] = (uint32_t)src * d_in * 16;
        else
          a_row[u] = (uint32_t)(2 * src + ((item / (KC / 2)) & 1)) * d_in * 8;
      }
    }
    const int i0 = kc * KC;
#pragma unroll
    for (int u = 0; u < W_PER; ++u) {
      const int item = tid + u * NT;
      const int jl = item / KC, q = item % KC;  // q: pair (q / 2), a (q % 2)
      const int j = ld.col0 + jl;               // j >= d_out lies past the expert's range: zero
      const int p = (i0 >> 1) + (q >> 1);
      const uint32_t off = (p < IP) ? ((uint32_t)(j * IP + p) * 2 + (q & 1)) * 16 : kOff;
      rw[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, off, 0, 0));
    }
#pragma unroll
    for (int u = 0; u < A_PER; ++u) {
      const int item = tid + u * NT;
      uint32_t off;
      if constexpr (IN == kInBladeGather) {
        const int i = i0 + item % KC;
        off = (i < d_in) ? a_row[u] + (uint32_t)i * 16 : kOff;
      } else {
        const int p = (i0 >> 1) + item % (KC / 2);  // 16-byte piece = one input pair
        off = (p < IP) ? a_row[u] + (uint32_t)p * 16 : kOff;
      }
      ra[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(x_rsrc, off, 0, 0));
    }
  };
  auto store_chunk = [&](int buf, const uint4 (&ra)[A_PER], const uint4 (&rw)[W_PER]) {
    unsigned char* As = smem + buf * TL::STAGE;
    unsigned char* Ws = As + TL::A_BYTES;
#pragma unroll
    for (int u = 0; u < A_PER; ++u) {
      const int item = tid + u * NT;
      if constexpr (IN == kInBladeGather) {
        const int tl = item / KC, il = item % KC;
        const uint4 q = ra[u];
        const float x[8] = {bf_lo(q.x), bf_hi(q.x), bf_lo(q.y), bf_hi(q.y),
                            bf_lo(q.z), bf_hi(q.z), bf_lo(q.w), bf_hi(q.w)};
        float c0[4], c1[4];
        blade_to_pauli(x, c0, c1);
        *reinterpret_cast<uint2*>(As + (2 * tl) * TL::A_STRIDE + il * 8) =
            make_uint2(pack2_bf16(c0[0], c0[1]), pack2_bf16(c0[2], c0[3]));
        *reinterpret_cast<uint2*>(As + (2 * tl + 1) * TL::A_STRIDE + il * 8) =
            make_uint2(pack2_bf16(c1[0], c1[1]), pack2_bf16(c1[2], c1[3]));
      } else {
        const int rl = item / (KC / 2), q = item % (KC / 2);
        *reinterpret_cast<uint4*>(As + rl * TL::A_STRIDE + q * 16) = ra[u];
      }
    }
#pragma unroll
    for (int u = 0; u < W_PER; ++u) {
      const int item = tid + u * NT;
      const int jl = item / KC, q = item % KC;
      *reinterpret_cast<uint4*>(Ws + jl * TL::W_STRIDE + q * 16) = rw[u];
    }
  };

  pf32x16_t acc[WR][WC][2][2];
  auto zero_acc = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int a = 0; a < WR; ++a)
#pragma unroll
      for (int b = 0; b < WC; ++b)
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int d = 0; d < 2; ++d)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[a][b][c][d][v] = 0.f;
  };

  // NR row blocks per wave from row block rb0 on (NR = WR for a whole tile; a half
  // tile computes NR = 1 block, rb0 = its half, into the first accumulators)
  auto compute_chunk = [&](int buf, auto nr_tag, int rb0) __attribute__((always_inline)) {
    constexpr int NR = decltype(nr_tag)::value;
    const unsigned char* As = smem + buf * TL::STAGE;
    const unsigned char* Ws = As + TL::A_BYTES;
#pragma unroll
    for (int s = 0; s < KC / 4; ++s) {
      uint4 av[WR], wv[WC][2];
#pragma unroll
      for (int rb = 0; rb < NR; ++rb) {
        const int row = (wt * WR + rb0 + rb) * 32 + l32;
        av[rb] = *reinterpret_cast<const uint4*>(As + row * TL::A_STRIDE + (4 * s + 2 * g) * 8);
      }
#pragma unroll
      for (int cb = 0; cb < WC; ++cb) {
        const int col = (wj * WC + cb) * 32 + l32;
#pragma unroll
        for (int a = 0; a < 2; ++a)
          wv[cb][a] = *reinterpret_cast<const uint4*>(Ws + col * TL::W_STRIDE + (2 * s + g) * 32 + a * 16);
      }
#pragma unroll
      for (int rb = 0; rb < NR; ++rb) {
        const uint4 ap = make_uint4(rot_conj(av[rb].x), rot_conj(av[rb].y), rot_conj(av[rb].z), rot_conj(av[rb].w));
        const pbf16x8_t A0 = __builtin_bit_cast(pbf16x8_t, av[rb]);
        const pbf16x8_t A1 = __builtin_bit_cast(pbf16x8_t, ap);
#pragma unroll
        for (int cb = 0; cb < WC; ++cb)
#pragma unroll
          for (int a = 0; a < 2; ++a) {
            const pbf16x8_t B = __builtin_bit_cast(pbf16x8_t, wv[cb][a]);
            acc[rb][cb][a][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A0, B, acc[rb][cb][a][0], 0, 0, 0);
            acc[rb][cb][a][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A1, B, acc[rb][cb][a][1], 0, 0, 0);
          }
      }
    }
  };

  // Bias of the tile being computed, loaded when its first chunk is computed
  // (raw buffer loads: a null bias is an empty range and reads zero).
  const __amdgpu_buffer_rsrc_t b_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(bias), (short)0, bias ? (uint32_t)E * d_out * 32 : 0u, kBufferFlags);
  float bvs[WC][8];
  auto load_bias = [&](const PauliTileInfo& ti) __attribute__((always_inline)) {
#pragma unroll
    for (int cb = 0; cb < WC; ++cb) {
      const int j = ti.col0 + (wj * WC + cb) * 32 + l32;
      const uint32_t off = (j < d_out) ? (uint32_t)(ti.e * d_out + j) * 32 : kOff;
      const uint4 lo = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(b_rsrc, off, 0, 0));
      const uint4 hi = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(b_rsrc, off + 16, 0, 0));
      const uint32_t m[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};  // mask order
#pragma unroll
      for (int c = 0; c < 8; ++c) bvs[cb][c] = __builtin_bit_cast(float, m[blade_to_mask(c)]);
    }
  };

  const __amdgpu_buffer_rsrc_t y_rsrc = __builtin_amdgcn_make_buffer_rsrc(Y, (short)0, y_bytes, kBufferFlags);
  auto epilogue = [&](const PauliTileInfo& ti) __attribute__((always_inline)) {
    pauli_tile_epilogue<ACT, OUT, OUT_DT, WR, WC, BWT, false>(acc, bvs, ti, wave, g, l32, d_out, y_rsrc, 0);
  };

  // ---- the stream of (tile, chunk) steps ------------------------------------
  // step f loads chunk f + 1 into registers, computes chunk f from LDS buffer
  // f % 2, stores chunk f + 1 into the other buffer, then one barrier.  (Keeping
  // two chunks in flight, in two register sets, measured no faster.)
  uint4 ra[A_PER], rw[W_PER];
  zero_acc();
  if (total > 0) {
    load_chunk(0, ra, rw);
    store_chunk(0, ra, rw);
  }
  __syncthreads();
  PauliTileInfo cur = {0, 0, 1, 0, -1};  // tile being computed
  auto step = [&](int f, auto nr_tag) __attribute__((always_inline)) {
    const int buf = f & 1;
    if (f % nk == 0) {
      cur = decode(f / nk);
      load_bias(cur);
    }
    if (f + 1 < total) load_chunk(f + 1, ra, rw);
    compute_chunk(buf, nr_tag, cur.half < 0 ? 0 : cur.half);
    if (f % nk == nk - 1) {
      epilogue(cur);
      zero_acc();
    }
    if (f + 1 < total) store_chunk(buf ^ 1, ra, rw);
    __syncthreads();
  };
  // the whole tiles, then the half tile (if any) in a loop of its own, so that the
  // second row block's accumulators are dead there
  int f = 0;
  for (; f < n_full * nk; ++f) step(f, std::integral_constant<int, WR>{});
  for (; f < total; ++f) step(f, std::integral_constant<int, 1>{});
}

// ---------------------------------------------------------------------------
// Pauli half-row input: operands staged by direct-to-LDS buffer loads
// ---------------------------------------------------------------------------
// Every staged piece is a 16-byte raw buffer load that writes LDS itself
// (lane l of an instruction lands at the wave's LDS base + 16 l), so no
// registers hold operands between their load and their use, and several
// chunks are in flight.  A step computes K = 8 input multivectors (KC):
//   W: a chunk per step, 64 columns x 128 B (4 pairs x (a = 0, 1) x 16 B), in
//      NW = 3 slots, issued two steps ahead; slot s of column j holds piece
//      s ^ swz_w(j);
//   A: a chunk per two steps, 128 half-rows (m, b) x 128 B (8 input pairs), in
//      NA = 3 slots, issued four steps ahead; slot s of half-row r holds pair
//      s ^ swz_a(r).
// Both are whole 128-byte lines per half-row or column (the memory system's
// request unit), and the XOR swizzles keep the MFMA operand reads (16 B per
// lane over 32 consecutive half-rows or columns) free of bank conflicts; the
// lanes of a load pick their global pieces so that the fixed LDS order comes
// out swizzled.  The tile's gather indices and bias arrive the same way, in
// two slots by tile parity, so no register load queues behind the staged
// chunks: before each step one explicit vmcnt wait lets exactly the loads of
// the previous step stay outstanding (loads complete in issue order, and the
// newest chunk a step needs is the W chunk issued two steps before), and one
// barrier publishes the chunks and frees the slots computed before.  A tile's
// gather indices are loaded with the previous tile's first A chunk, which
// needs at least two A chunks per tile (d_in > 16; smaller products use the
// register-staged kernel).  The step loop carries its tile and chunk
// counters: a wave issues at most one instruction every four cycles, so the
// per-step bookkeeping is a few scalar operations.
struct PauliDmaTile {
  static constexpr int NT = 256, T = 64, BN = 64, KC = 8, WR = 2, WC = 1, BWT = 2;
  static constexpr int NA = 3, NW = 3;
  static constexpr int A_SLOT = 2 * T * 128;                // 16 KiB: 16 input multivectors
  static constexpr int W_SLOT = BN * 128;                   // 8 KiB: 8 input multivectors
  static constexpr int W_OFF = NA * A_SLOT;
  static constexpr int G_OFF = W_OFF + NW * W_SLOT;         // 2 x 64 row indices (tile parity)
  static constexpr int B_OFF = G_OFF + 2 * T * 4;           // 2 x 64 columns x 32 B of bias
  static constexpr int LDS = B_OFF + 2 * BN * 32;           // 78336 B: two workgroups per CU
  static constexpr int A_AHEAD = 2, W_AHEAD = 2;            // chunks issued ahead of use
};

__device__ __forceinline__ int swz8(int r) { return (r ^ (r >> 3)) & 7; }

typedef __attribute__((address_space(3))) void lds_void_t;
// One direct-to-LDS load of BYTES (4 or 16) bytes per lane at byte offset `off`
// of buffer `r`; lane l lands at lds + BYTES l (`lds` is the same in every
// lane).  Written as assembly: the compiler would otherwise wait for every
// outstanding direct load before any LDS read (it cannot tell the slots
// apart), which serialises the pipeline; here the explicit waits below are
// the only ones, and the compiler issues no vector-memory loads of its own in
// the steps (its waits for earlier loads only grow stricter with these in
// the queue).
template <int BYTES>
__device__ __forceinline__ void dma_to_lds(__amdgpu_buffer_rsrc_t r, unsigned char* lds, uint32_t off) {
  static_assert(BYTES == 4 || BYTES == 16, "direct load size");
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void_t*)lds);  // wave-uniform
  if constexpr (BYTES == 4)
    asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dword %0, %2, 0 offen lds" ::"v"(off), "s"(m0), "s"(r) : "m0");
  else
    asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %0, %2, 0 offen lds" ::"v"(off), "s"(m0), "s"(r) : "m0");
}
// the same 16-byte load with a wave-uniform byte offset `soff` added in a scalar
// register: a chunk's advance along K costs no vector instruction
__device__ __forceinline__ void dma_to_lds_s(__amdgpu_buffer_rsrc_t r, unsigned char* lds, uint32_t off,
                                             uint32_t soff) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void_t*)lds);
  const uint32_t so = __builtin_amdgcn_readfirstlane(soff);
  asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %0, %2, %3 offen lds" ::"v"(off), "s"(m0), "s"(r), "s"(so)
               : "m0");
}
// wait until at most N vector memory operations of this wave are outstanding
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 16, "vmcnt field");
  __builtin_amdgcn_s_waitcnt(0x3f70 | N);  // expcnt and lgkmcnt at their maxima: no wait on those
}
// workgroup barrier without the fences of __syncthreads: the waits that make
// the staged LDS contents ready are the explicit ones above
__device__ __forceinline__ void lds_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Sizes: x_bytes and y_bytes are the operands' whole sizes (64-bit).  Gathered rows
// (token ids through `gather`) index the whole of x, which the host keeps below
// 2 GiB; rows taken in place, and the output, are addressed from buffer resources
// whose 64-bit base is the tile's first row, so only one tile's span needs 32-bit
// offsets and the number of rows is not limited by them.
template <int ACT, int OUT, int OUT_DT>
__global__ __launch_bounds__(PauliDmaTile::NT) __attribute__((amdgpu_waves_per_eu(2))) void pauli_gemm_dma_kernel(
    const uint16_t* __restrict__ X, const int32_t* __restrict__ gather, const uint16_t* __restrict__ Wp,
    const float* __restrict__ bias, const int32_t* __restrict__ offsets, int E, int d_in, int d_out,
    void* __restrict__ Y, int n_xcd, uint64_t x_bytes, uint64_t y_bytes) {
  using C = PauliDmaTile;
  constexpr int NT = C::NT, T = C::T, BN = C::BN, KC = C::KC, WR = C::WR, WC = C::WC, BWT = C::BWT;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[C::LDS];
  __shared__ int s_off[kPauliMaxExperts + 1];   // expert row offsets
  __shared__ int s_tbeg[kPauliMaxExperts + 1];  // first whole row tile of each expert
  __shared__ int s_cbeg[kPauliMaxExperts + 1];  // first compact row tile of each expert

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  for (int i = tid; i <= E; i += NT) s_off[i] = offsets[i];
  __syncthreads();
  // Two lists of row tiles: every expert's row tiles but a short last one ("whole"
  // tiles), and the experts' last row tiles of at most T / 2 rows ("compact" tiles,
  // computed with half the MFMAs).  s_tbeg / s_cbeg: each expert's first whole /
  // compact row tile.
  if (tid == 0) {
    int acc = 0, accc = 0;
    for (int x = 0; x < E; ++x) {
      const int cnt = s_off[x + 1] - s_off[x];
      const int nrt = (cnt + T - 1) / T;
      const int comp = (cnt > 0 && cnt - (nrt - 1) * T <= T / 2) ? 1 : 0;
      s_tbeg[x] = acc;
      s_cbeg[x] = accc;
      acc += nrt - comp;
      accc += comp;
    }
    s_tbeg[E] = acc;
    s_cbeg[E] = accc;
  }
  __syncthreads();
  // lane x keeps expert x's first whole and compact row tile and its row range: a
  // tile's expert is the number of experts whose first tile of the list is at or
  // before it, minus one (experts without tiles in a list share their successor's
  // first tile there and are never chosen)
  const int v_tbeg = lane < E ? s_tbeg[lane] : 0x7fffffff;
  const int v_cbeg = lane < E ? s_cbeg[lane] : 0x7fffffff;
  const int v_off = s_off[lane < E ? lane : E], v_end = s_off[lane < E ? lane + 1 : E];
  // (LDS values are per lane to the compiler; these are the same in every lane)
  const int n_rows = __builtin_amdgcn_readfirstlane(s_off[E]);

  // The tile stream: as in the register-staged kernel, one contiguous range of whole
  // tiles per XCD, whole rounds first; then items of half the work, dealt round robin
  // over the XCD's workgroups: the XCD's range of compact tiles, then (when the whole
  // tiles leave at most half a round) the remaining whole tiles cut into half tiles.
  // When the whole tiles end in a partial round, the items go first to the workgroups
  // that run one whole tile fewer.
  const int CT = (d_out + BN - 1) / BN;
  const int n_tiles = __builtin_amdgcn_readfirstlane(s_tbeg[E]) * CT;
  const int n_ctiles = __builtin_amdgcn_readfirstlane(s_cbeg[E]) * CT;
  const int nka = (d_in + 2 * KC - 1) / (2 * KC);  // A chunks per tile
  const int nk = 2 * nka;                          // steps (W chunks) per tile
  const int per_xcd = gridDim.x / n_xcd;
  const int xcd = blockIdx.x % n_xcd, slot = blockIdx.x / n_xcd;
  const int lo = (int)((long long)n_tiles * xcd / n_xcd), hi = (int)((long long)n_tiles * (xcd + 1) / n_xcd);
  const int clo = (int)((long long)n_ctiles * xcd / n_xcd), chi = (int)((long long)n_ctiles * (xcd + 1) / n_xcd);
  const int R = hi - lo, rounds = R / per_xcd, rem = R - rounds * per_xcd;
  const bool split = rem > 0 && 2 * rem <= per_xcd;
  const int n_full = split ? rounds : (R > slot ? (R - slot + per_xcd - 1) / per_xcd : 0);
  const int n_comp = chi - clo;                                // compact items of this XCD
  const int n_items = n_comp + (split ? 2 * rem : 0);          // half-work items of this XCD
  // the items are dealt from the first workgroup that runs one whole tile fewer (slot
  // rem) on, wrapping round: ranks ir
  const int ir = split ? slot : (slot - rem + per_xcd) % per_xcd;
  const int n_mine = n_full + (n_items > ir ? (n_items - ir + per_xcd - 1) / per_xcd : 0);
  const int total = n_mine * nk, total_a = n_mine * nka;
  if (total == 0) return;

  auto decode = [&](int n) __attribute__((always_inline)) {
    PauliTileInfo t;
    const int item = n >= n_full ? ir + (n - n_full) * per_xcd : -1;
    if (item >= 0 && item < n_comp) {  // a compact tile: an expert's short last row tile
      const int C = clo + item;
      const int rt = C / CT, ct = C - rt * CT;
      const int e = __popcll(__ballot(v_cbeg <= rt)) - 1;
      const int beg = __builtin_amdgcn_readlane(v_off, e);
      t.e = e;
      t.row_end = __builtin_amdgcn_readlane(v_end, e);
      t.row0 = beg + ((t.row_end - beg - 1) / T) * T;
      t.col0 = ct * BN;
      t.compact = true;
      t.half = 0;
      return t;
    }
    // a whole tile, or half of one
    const int L = item >= 0 ? lo + rounds * per_xcd + ((item - n_comp) >> 1) : lo + slot + n * per_xcd;
    const int rt = L / CT, ct = L - rt * CT;
    const int e = __popcll(__ballot(v_tbeg <= rt)) - 1;
    t.e = e;
    t.row0 = __builtin_amdgcn_readlane(v_off, e) + (rt - __builtin_amdgcn_readlane(v_tbeg, e)) * T;
    t.row_end = __builtin_amdgcn_readlane(v_end, e);
    t.col0 = ct * BN;
    t.compact = false;
    t.half = item >= 0 ? ((item - n_comp) & 1) : -1;
    return t;
  };

  const int wt = wave % BWT, wj = wave / BWT;
  const int g = lane >> 5, l32 = lane & 31;
  const int IP = d_in >> 1;  // input pairs (d_in even)
  constexpr uint32_t kOff = 0x80000000u;  // past every range: reads zero

  // a buffer resource over `bytes` bytes from `base`, offset `off` bytes into it
  // (64-bit), its range clamped to what lies past `off` and below 2 GiB
  auto rsrc_from = [](const void* base, uint64_t bytes, uint64_t off) __attribute__((always_inline)) {
    const uint64_t left = bytes > off ? bytes - off : 0;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(static_cast<const char*>(base)) + off, (short)0,
                                             (uint32_t)(left < 0x7fffffffull ? left : 0x7fffffffull), kBufferFlags);
  };
  // gathered rows index the whole of x (below 2 GiB); in place, the resource is
  // re-based at each tile's first row when its first A chunk is issued
  __amdgpu_buffer_rsrc_t x_rsrc = rsrc_from(X, gather ? x_bytes : 0, 0);
  const uint64_t x_row_bytes = (uint64_t)d_in * 16;  // a row: two Pauli half-rows of d_in x 8 bytes
  const __amdgpu_buffer_rsrc_t g_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int32_t*>(gather), (short)0, gather ? (uint32_t)n_rows * 4 : 0u, kBufferFlags);
  const __amdgpu_buffer_rsrc_t b_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(bias), (short)0, bias ? (uint32_t)E * d_out * 32 : 0u, kBufferFlags);
  __amdgpu_buffer_rsrc_t w_rsrc = x_rsrc;

  // this lane's pieces: A loads 4 w .. 4 w + 3 (half-rows 8 q .. 8 q + 7, one
  // 128-byte line each), W loads 2 w and 2 w + 1 (columns 8 q .. 8 q + 7)
  int a_lim[4], w_lim[2];  // a piece is inside the K range while its chunk's first pair is below these
  uint32_t a_pc[4], w_pc[2];  // the piece's byte offset inside its row or column chunk
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int r = 8 * (4 * wave + u) + (lane >> 3);
    const int c = (lane & 7) ^ swz8(r);  // input pair of the chunk
    a_lim[u] = IP - c;
    a_pc[u] = c * 16;
  }
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int c = (lane & 7) ^ swz8(8 * (2 * wave + u) + (lane >> 3));  // piece (pair, a) of the chunk
    w_lim[u] = IP - (c >> 1);
    w_pc[u] = c * 16;
  }
  uint32_t a_cur[4], w_cur[2];  // offsets of those pieces in the tile's first chunk (the chunk's own
                                // advance along K is a scalar offset)

  // next A chunk: chunk iak of tile iam, slot ias; next W chunk: chunk iwk of
  // tile iwm, slot iws (value selects throughout: a branch that increments one
  // of two counters becomes an address select that keeps them in scratch)
  int ia = 0, iam = 0, iak = 0, ias = 0;
  int iw = 0, iwm = 0, iwk = 0, iws = 0;
  // issue the next A chunk (4 loads per wave); at a tile's first A chunk also the
  // next tile's gather indices (wave 3, before the chunk)
  auto issue_a = [&]() __attribute__((always_inline)) {
    if (iak == 0) {
      const PauliTileInfo t = decode(iam);
      const int* gs = reinterpret_cast<const int*>(smem + C::G_OFF + (iam & 1) * T * 4);
      if (gather == nullptr) x_rsrc = rsrc_from(X, x_bytes, (uint64_t)t.row0 * x_row_bytes);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int r = 8 * (4 * wave + u) + (lane >> 3);  // half-row (token slot r / 2, b = r % 2)
        // the tile's row at this token slot: the slot itself, or for a compact tile
        // rows 0-15 at slots 0-15 and rows 16-31 at slots 32-47 (the other slots
        // repeat them and are not computed)
        const int ts = r >> 1;
        const int tr = t.compact ? (ts & 15) | ((ts >> 5) << 4) : ts;
        // the gathered token, or the row relative to the tile's first
        const int src = gather ? gs[tr] : min(tr, t.row_end - 1 - t.row0);
        a_cur[u] = (uint32_t)(2 * src + (r & 1)) * d_in * 8 + a_pc[u];
      }
      if (gather != nullptr && wave == 3 && iam + 1 < n_mine) {
        const PauliTileInfo tn = decode(iam + 1);
        dma_to_lds<4>(g_rsrc, smem + C::G_OFF + ((iam + 1) & 1) * T * 4,
                      (uint32_t)min(tn.row0 + lane, tn.row_end - 1) * 4);
      }
    }
    const int p0 = iak * KC;  // first input pair of the chunk (16 multivectors)
    unsigned char* st = smem + ias * C::A_SLOT + 4 * wave * 1024;
    const uint32_t so = (uint32_t)p0 * 16;
    if (p0 + KC <= IP) {  // uniform: the whole chunk lies inside the K range
#pragma unroll
      for (int u = 0; u < 4; ++u) dma_to_lds_s(x_rsrc, st + u * 1024, a_cur[u], so);
    } else {  // the K tail: pieces past it read zero
#pragma unroll
      for (int u = 0; u < 4; ++u) dma_to_lds_s(x_rsrc, st + u * 1024, p0 < a_lim[u] ? a_cur[u] : kOff, so);
    }
    ++ia;
    ias = ias == C::NA - 1 ? 0 : ias + 1;
    const bool last = iak == nka - 1;
    iam += last ? 1 : 0;
    iak = last ? 0 : iak + 1;
  };
  // issue the next W chunk (2 loads per wave); at a tile's first W chunk also
  // the tile's bias (waves 0 and 1, before the chunk)
  auto issue_w = [&]() __attribute__((always_inline)) {
    if (iwk == 0) {
      const PauliTileInfo t = decode(iwm);
      w_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(Wp) + (size_t)t.e * d_out * IP * 16, (short)0,
                                                 (uint32_t)d_out * IP * 32, kBufferFlags);
      if (wave < 2) {  // bias: 64 columns x 32 B, two loads of 32 columns
        const int j = t.col0 + 32 * wave + (lane >> 1);
        dma_to_lds<16>(b_rsrc, smem + C::B_OFF + (iwm & 1) * BN * 32 + wave * 1024,
                       j < d_out ? (uint32_t)(t.e * d_out + j) * 32 + (lane & 1) * 16 : kOff);
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int j = t.col0 + 8 * (2 * wave + u) + (lane >> 3);  // past d_out: past the expert's range, reads zero
        w_cur[u] = (uint32_t)j * IP * 32 + w_pc[u];
      }
    }
    const int p0 = iwk * (KC / 2);  // first input pair of the chunk (8 multivectors)
    unsigned char* st = smem + C::W_OFF + iws * C::W_SLOT + 2 * wave * 1024;
    const uint32_t so = (uint32_t)p0 * 32;
    if (p0 + KC / 2 <= IP) {  // uniform: the whole chunk lies inside the K range
#pragma unroll
      for (int u = 0; u < 2; ++u) dma_to_lds_s(w_rsrc, st + u * 1024, w_cur[u], so);
    } else {
#pragma unroll
      for (int u = 0; u < 2; ++u) dma_to_lds_s(w_rsrc, st + u * 1024, p0 < w_lim[u] ? w_cur[u] : kOff, so);
    }
    ++iw;
    iws = iws == C::NW - 1 ? 0 : iws + 1;
    const bool last = iwk == nk - 1;
    iwm += last ? 1 : 0;
    iwk = last ? 0 : iwk + 1;
  };

  // MFMA operand reads: half-row (wt WR + rb) 32 + l32 at pair 4 (step parity)
  // + 2 s + g of the A chunk, and column (wj WC + cb) 32 + l32 at piece
  // 2 (2 s + g) + a of the W chunk, through the swizzles.  The odd step's pair
  // differs in bit 2, i.e. bit 6 of the byte offset: offset ^ 64.  (Selecting
  // between two offset arrays instead would turn into an address select that
  // keeps the arrays in scratch memory.)
  uint32_t a_rd[2][2], w_rd[WC][2][2];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const int row = (wt * WR + rb) * 32 + l32;
      a_rd[s][rb] = (uint32_t)row * 128 + ((2 * s + g) ^ swz8(row)) * 16;
    }
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int cb = 0; cb < WC; ++cb) {
      const int col = (wj * WC + cb) * 32 + l32;
#pragma unroll
      for (int a = 0; a < 2; ++a) w_rd[cb][s][a] = col * 128 + (((2 * (2 * s + g) + a) ^ swz8(col)) * 16);
    }

  pf32x16_t acc[WR][WC][2][2];
  // a step's operands: A chunk half `par` in slot as, W chunk in slot ws; NR row
  // blocks from rb0 (a half tile computes one block, rb0, with its offsets by
  // arithmetic: no dynamic register index)
  uint4 av[2][WR], wv[2][WC][2];
  auto read_operands = [&](int as, int ws, int par, auto nr_tag, int rb0) __attribute__((always_inline)) {
    constexpr int NR = decltype(nr_tag)::value;
    const unsigned char* As = smem + as * C::A_SLOT;
    const unsigned char* Ws = smem + C::W_OFF + ws * C::W_SLOT;
#pragma unroll
    for (int s = 0; s < KC / 4; ++s) {
      if constexpr (NR == WR) {
#pragma unroll
        for (int rb = 0; rb < NR; ++rb) av[s][rb] = *reinterpret_cast<const uint4*>(As + (a_rd[s][rb] ^ (par << 6)));
      } else {
        const int row = (wt * WR + rb0) * 32 + l32;
        av[s][0] = *reinterpret_cast<const uint4*>(As + row * 128 + ((4 * par + 2 * s + g) ^ swz8(row)) * 16);
      }
#pragma unroll
      for (int cb = 0; cb < WC; ++cb)
#pragma unroll
        for (int a = 0; a < 2; ++a) wv[s][cb][a] = *reinterpret_cast<const uint4*>(Ws + w_rd[cb][s][a]);
    }
  };
  auto mfmas = [&](auto nr_tag) __attribute__((always_inline)) {
    constexpr int NR = decltype(nr_tag)::value;
    // raised issue priority while this wave feeds the MFMA pipe: the co-resident
    // workgroup's wave on the SIMD then fills the gaps with its epilogue or loads
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int s = 0; s < KC / 4; ++s)
#pragma unroll
      for (int rb = 0; rb < NR; ++rb) {
        const uint4 x = av[s][rb];
        const uint4 ap = make_uint4(rot_conj(x.x), rot_conj(x.y), rot_conj(x.z), rot_conj(x.w));
        const pbf16x8_t A0 = __builtin_bit_cast(pbf16x8_t, x);
        const pbf16x8_t A1 = __builtin_bit_cast(pbf16x8_t, ap);
#pragma unroll
        for (int cb = 0; cb < WC; ++cb)
#pragma unroll
          for (int a = 0; a < 2; ++a) {
            const pbf16x8_t B = __builtin_bit_cast(pbf16x8_t, wv[s][cb][a]);
            acc[rb][cb][a][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A0, B, acc[rb][cb][a][0], 0, 0, 0);
            acc[rb][cb][a][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A1, B, acc[rb][cb][a][1], 0, 0, 0);
          }
      }
    __builtin_amdgcn_s_setprio(0);
  };

  // a tile's accumulators start from its bias (slot m % 2, complete by the tile's first step)
  float bvs[WC][8];
  auto acc_from_bias = [&](int m) __attribute__((always_inline)) {
    const unsigned char* bs = smem + C::B_OFF + (m & 1) * BN * 32;
#pragma unroll
    for (int cb = 0; cb < WC; ++cb) {
      const int jl = (wj * WC + cb) * 32 + l32;
      const uint4 lo4 = *reinterpret_cast<const uint4*>(bs + jl * 32);
      const uint4 hi4 = *reinterpret_cast<const uint4*>(bs + jl * 32 + 16);
      const uint32_t mk[8] = {lo4.x, lo4.y, lo4.z, lo4.w, hi4.x, hi4.y, hi4.z, hi4.w};  // mask order
#pragma unroll
      for (int c = 0; c < 8; ++c) bvs[cb][c] = __builtin_bit_cast(float, mk[blade_to_mask(c)]);
    }
    pauli_acc_from_bias<WR, WC>(acc, bvs);
  };
  // the output from the tile's first row on (64-bit base)
  constexpr uint64_t Y_MV_BYTES = (OUT == kOutPauliRows || OUT_DT == kBF16) ? 16 : 32;
  auto epilogue = [&](const PauliTileInfo& ti) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t y_rsrc = rsrc_from(Y, y_bytes, (uint64_t)ti.row0 * d_out * Y_MV_BYTES);
    pauli_tile_epilogue<ACT, OUT, OUT_DT, WR, WC, BWT, true>(acc, bvs, ti, wave, g, l32, d_out, y_rsrc, ti.row0);
  };

  // prologue: the first tile's gather indices; then what steps -4 .. -1 would
  // issue: A chunks 0 and 1, W chunk 0, and W chunk 1 last
  if (gather != nullptr && wave == 3) {
    const PauliTileInfo t = decode(0);
    dma_to_lds<4>(g_rsrc, smem + C::G_OFF, (uint32_t)min(t.row0 + lane, t.row_end - 1) * 4);
  }
  wait_vmcnt<0>();
  lds_barrier();
  issue_a();
  issue_a();  // every tile has at least two A chunks
  issue_w();
  issue_w();

  // Steps come in pairs (a tile has an even number): the even step issues the
  // A chunk two pairs ahead and the W chunk two steps ahead, the odd step the
  // W chunk.  The newest chunk a step reads is the W chunk issued two steps
  // before, so the loads of the previous step may stay outstanding: 2 after
  // an odd step, 6 after an even one (a tile's bias or gather indices, issued
  // before those, only make the wait stricter); near the end, none.
  PauliTileInfo cur = {0, 0, 1, 0, -1};
  int fm = 0, fkc = 0;   // tile and K chunk of the step computed
  int fas = 0, fws = 0;  // its A and W slots
  auto step = [&](int f, auto nr_tag) __attribute__((always_inline)) {
    constexpr int NR = decltype(nr_tag)::value;
    const bool odd = (f & 1) != 0;
    if (f + 3 < total) {
      if (odd) wait_vmcnt<6>();
      else wait_vmcnt<2>();
    } else {
      wait_vmcnt<0>();
    }
    lds_barrier();
    if (fkc == 0) {
      cur = decode(fm);
      acc_from_bias(fm);
    }
    read_operands(fas, fws, odd ? 1 : 0, nr_tag, cur.half < 0 ? 0 : cur.half);
    if (!odd && ia < total_a) issue_a();
    if (iw < total) issue_w();
    mfmas(nr_tag);
    const bool last = fkc == nk - 1;
    if (last) epilogue(cur);
    fm += last ? 1 : 0;
    fkc = last ? 0 : fkc + 1;
    fas = odd ? (fas == C::NA - 1 ? 0 : fas + 1) : fas;
    fws = fws == C::NW - 1 ? 0 : fws + 1;
  };
  int f = 0;
  for (; f < n_full * nk; f += 2) {
    step(f, std::integral_constant<int, WR>{});
    step(f + 1, std::integral_constant<int, WR>{});
  }
  for (; f < total; f += 2) {
    step(f, std::integral_constant<int, 1>{});
    step(f + 1, std::integral_constant<int, 1>{});
  }
  wait_vmcnt<0>();
}

// ---------------------------------------------------------------------------
// weight preparation: (E, d_out, d_in, 8) fp32 blade -> PW bf16
// ---------------------------------------------------------------------------
// One thread per (e, j, i): writes the 2 x 8-byte halves (a = 0, 1) of its
// multivector in the 32-byte record of its input pair.
__global__ __launch_bounds__(256) void pauli_prep_weights_kernel(const float* __restrict__ W, int E, int d_out,
                                                                 int d_in, uint16_t* __restrict__ out) {
  const size_t n = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t total = (size_t)E * d_out * d_in;
  if (n >= total) return;
  const int i = (int)(n % d_in);
  const size_t ej = n / d_in;  // e * d_out + j
  const float* w = W + n * 8;
  float x[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) x[c] = 0.5f * w[c];
  // Pauli entries W[a][c] = u + iv
  float c0[4], c1[4];
  blade_to_pauli(x, c0, c1);  // c0 = (M00, M10), c1 = (M01, M11)
  // a = 0: c = 0 -> M00, c = 1 -> M01;  a = 1: c = 0 -> M10, c = 1 -> M11; store (u, -v)
  const uint2 a0 = make_uint2(pack2_bf16(c0[0], -c0[1]), pack2_bf16(c1[0], -c1[1]));
  const uint2 a1 = make_uint2(pack2_bf16(c0[2], -c0[3]), pack2_bf16(c1[2], -c1[3]));
  const int IP = d_in >> 1;
  uint16_t* rec = out + ((ej * IP + (i >> 1)) * 2) * 8;  // 32-byte record of pair i/2
  *reinterpret_cast<uint2*>(rec + (i & 1) * 4) = a0;       // a = 0 half, slot of i within the pair
  *reinterpret_cast<uint2*>(rec + 8 + (i & 1) * 4) = a1;   // a = 1 half
}

// blade rows (bf16) -> Pauli half-rows (bf16); one thread per multivector
__global__ __launch_bounds__(256) void blade_to_pauli_rows_kernel(const uint16_t* __restrict__ x, int rows, int d,
                                                                  uint16_t* __restrict__ out) {
  const size_t n = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (n >= (size_t)rows * d) return;
  pauli_rows_bf16_one(x, d, n, out);
}

// Which kernel runs a product: the direct-to-LDS kernel for Pauli half-row input
// with at least two A chunks per tile, else the register-staged one.
bool pauli_uses_dma(int x_layout, int d_in) { return x_layout == kInPauliRows && d_in > 2 * PauliDmaTile::KC; }

// The 32-bit buffer offsets of the products: nullptr if the call fits, else why not.
// Both kernels address one expert's weights (a column tile may reach 64 columns
// past d_out) and the biases as whole buffers.  The direct-to-LDS kernel addresses
// gathered x rows over the whole of x, and rows in place and the output from each
// tile's first row (64-bit bases: any number of rows); the register-staged kernel
// addresses x and the output as whole buffers.  (x rows, blade or Pauli half-row
// pairs, are 16 d_in bytes either way.)
const char* pauli_size_limit(int x_layout, int x_rows, bool gathered, int P_max, int E, int d_in, int d_out,
                             int y_layout, int y_dtype) {
  const uint64_t lim = (uint64_t)1 << 31;
  const uint64_t y_mv = (y_layout == kOutPauliRows || y_dtype == kBF16) ? 16 : 32;
  if ((uint64_t)(d_out + 64) * d_in * 16 >= lim) return "one expert's weights reach 2 GiB";
  if ((uint64_t)E * d_out * 32 >= lim) return "the biases reach 2 GiB";
  if (pauli_uses_dma(x_layout, d_in)) {
    if (gathered && (uint64_t)x_rows * d_in * 16 >= lim) return "gathered x rows span 2 GiB or more";
    if ((uint64_t)PauliDmaTile::T * d_out * y_mv >= lim || (uint64_t)PauliDmaTile::T * d_in * 16 >= lim)
      return "one tile's rows span 2 GiB";
  } else if ((uint64_t)x_rows * d_in * 16 >= lim || (uint64_t)P_max * d_out * y_mv >= lim) {
    return "operands of 2 GiB or more need Pauli half-row input with d_in > 16";
  }
  return nullptr;
}

}  // namespace ygg

using namespace ygg;

namespace {
// Tile configuration: 256 threads (2 x 2 waves), 64 tokens x 64 output
// multivectors, 70 KiB of LDS, so two independent workgroups share a CU and
// one's epilogue and barriers overlap the other's MFMAs.  (Measured on C3:
// 199 + 167 us for the up + down products, against 204 + 185 us for one
// 512-thread 64 x 128 workgroup per CU.)
using Tile = PauliTile</*WR*/ 2, /*WC*/ 1, /*BWT*/ 2, /*BWJ*/ 2, /*KC*/ 16>;
constexpr int kWgPerCu = 2;

// persistent grid: as many workgroups as fit on the chip at once
struct DeviceShape {
  int cus = 0, xcds = 1;
};
DeviceShape device_shape() {
  static thread_local int cached_dev = -1;
  static thread_local DeviceShape cached;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  if (dev != cached_dev) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 64;
    cached.cus = cus;
    // MI355X (gfx950): 256 CUs in 8 XCDs; workgroups are dealt to the XCDs round robin
    cached.xcds = (cus % 8 == 0) ? 8 : 1;
    cached_dev = dev;
  }
  return cached;
}

template <int ACT, int IN, int OUT, int ODT>
int launch_pauli(hipStream_t st, const uint16_t* X, uint64_t x_bytes, const int32_t* gather, const uint16_t* Wp,
                 const float* bias, const int32_t* offsets, int E, int P_max, int d_in, int d_out, void* Y) {
  const DeviceShape ds = device_shape();
  // the output's size (rows past P_max, from offsets beyond it, are not written)
  const uint64_t y_bytes = (uint64_t)P_max * d_out * ((OUT == kOutPauliRows || ODT == kBF16) ? 16 : 32);
  // never more workgroups than tiles can exist
  const long long max_tiles =
      ((long long)(P_max + Tile::T - 1) / Tile::T + E) * ((d_out + Tile::BN - 1) / Tile::BN);
  int grid = ds.cus * kWgPerCu;
  int xcds = ds.xcds;
  if (max_tiles < grid) {
    grid = (int)max_tiles;
    xcds = 1;
  }
  if (pauli_uses_dma(IN, d_in))
    pauli_gemm_dma_kernel<ACT, OUT, ODT>
        <<<grid, PauliDmaTile::NT, 0, st>>>(X, gather, Wp, bias, offsets, E, d_in, d_out, Y, xcds, x_bytes, y_bytes);
  else  // the register-staged kernel: whole operands below 2 GiB (checked by the caller)
    pauli_gemm_kernel<ACT, IN, OUT, ODT, Tile><<<grid, Tile::NT, 0, st>>>(
        X, gather, Wp, bias, offsets, E, d_in, d_out, Y, xcds, (uint32_t)x_bytes, (uint32_t)y_bytes);
  return check_launch("pauli_gemm");
}

template <int ACT>
int launch_pauli_act(hipStream_t st, int in_layout, int out_layout, int y_dtype, const uint16_t* X, uint64_t x_bytes,
                     const int32_t* gather, const uint16_t* Wp, const float* bias, const int32_t* offsets, int E,
                     int P_max, int d_in, int d_out, void* Y) {
#define YGG_PL(IN, OUT, ODT) \
  launch_pauli<ACT, IN, OUT, ODT>(st, X, x_bytes, gather, Wp, bias, offsets, E, P_max, d_in, d_out, Y)
  if (in_layout == kInBladeGather) {
    if (out_layout == kOutPauliRows) return YGG_PL(kInBladeGather, kOutPauliRows, kBF16);
    if (y_dtype == kBF16) return YGG_PL(kInBladeGather, kOutBlade, kBF16);
    return YGG_PL(kInBladeGather, kOutBlade, kF32);
  }
  if (out_layout == kOutPauliRows) return YGG_PL(kInPauliRows, kOutPauliRows, kBF16);
  if (y_dtype == kBF16) return YGG_PL(kInPauliRows, kOutBlade, kBF16);
  return YGG_PL(kInPauliRows, kOutBlade, kF32);
#undef YGG_PL
}
}  // namespace

// Pauli weight preparation, called by ygg_prepare_weights (format 3).
int ygg::pauli_prepare_weights(const float* W, int E, int d_out, int d_in, void* out, hipStream_t stream) {
  YGG_CHECK_ARG(d_in >= 2 && (d_in % 2) == 0, "ygg_prepare_weights: the bf16 Pauli format needs an even d_in (got %d)",
                d_in);
  const size_t total = (size_t)E * d_out * d_in;
  pauli_prep_weights_kernel<<<(unsigned)((total + 255) / 256), 256, 0, stream>>>(W, E, d_out, d_in,
                                                                                  static_cast<uint16_t*>(out));
  return check_launch("pauli_prep_weights");
}

YGG_API int ygg_pauli_rows_from_blade(const void* x, int rows, int d, void* out, hipStream_t stream) {
  YGG_CHECK_ARG(rows >= 0 && d >= 2 && (d % 2) == 0, "ygg_pauli_rows_from_blade: rows=%d d=%d (d must be even)",
                rows, d);
  if (rows == 0) return 0;
  YGG_CHECK_ARG(x && out, "ygg_pauli_rows_from_blade: null pointer");
  const size_t n = (size_t)rows * d;
  blade_to_pauli_rows_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(static_cast<const uint16_t*>(x), rows,
                                                                               d, static_cast<uint16_t*>(out));
  return check_launch("blade_to_pauli_rows");
}

YGG_API int ygg_pauli_grouped_linear(const void* x, int x_layout, int x_rows, const int32_t* gather, int P_max,
                                     const void* w,
                                     const float* bias, const int32_t* offsets, int E, int d_in, int d_out, int act,
                                     void* y, int y_layout, int y_dtype, hipStream_t stream) {
  YGG_CHECK_ARG(x_layout == kInBladeGather || x_layout == kInPauliRows, "ygg_pauli_grouped_linear: x layout %d",
                x_layout);
  YGG_CHECK_ARG(y_layout == kOutPauliRows || y_layout == kOutBlade, "ygg_pauli_grouped_linear: y layout %d", y_layout);
  YGG_CHECK_ARG(y_layout == kOutPauliRows ? y_dtype == kBF16 : (y_dtype == kBF16 || y_dtype == kF32),
                "ygg_pauli_grouped_linear: y dtype %d invalid for layout %d", y_dtype, y_layout);
  YGG_CHECK_ARG(act >= kActNone && act <= kActSigmoid, "ygg_pauli_grouped_linear: activation %d", act);
  YGG_CHECK_ARG(E >= 1 && E <= kPauliMaxExperts && P_max >= 0 && d_in >= 2 && (d_in % 2) == 0 && d_out >= 1 &&
                    (y_layout != kOutPauliRows || (d_out % 2) == 0),
                "ygg_pauli_grouped_linear: bad sizes E=%d P=%d d_in=%d d_out=%d (E <= %d; d_in, and d_out of Pauli "
                "rows, must be even)",
                E, P_max, d_in, d_out, kPauliMaxExperts);
  YGG_CHECK_ARG(x_rows >= 0 && (gather != nullptr || x_rows >= P_max),
                "ygg_pauli_grouped_linear: x has %d rows, the product reads %d without a gather", x_rows, P_max);
  if (const char* why = ygg::pauli_size_limit(x_layout, x_rows, gather != nullptr, P_max, E, d_in, d_out, y_layout,
                                              y_dtype)) {
    ygg::set_error("ygg_pauli_grouped_linear: %s (x rows=%d d_in=%d d_out=%d output rows=%d)", why, x_rows, d_in,
                   d_out, P_max);
    return -1;
  }
  if (P_max == 0) return 0;
  YGG_CHECK_ARG(x && w && offsets && y, "ygg_pauli_grouped_linear: null pointer");
  const uint64_t x_bytes = (uint64_t)x_rows * d_in * 16;
  const uint16_t* X = static_cast<const uint16_t*>(x);
  const uint16_t* Wp = static_cast<const uint16_t*>(w);
  switch (act) {
    case kActNone:
      return launch_pauli_act<kActNone>(stream, x_layout, y_layout, y_dtype, X, x_bytes, gather, Wp, bias, offsets, E, P_max,
                                        d_in, d_out, y);
    case kActGelu:
      return launch_pauli_act<kActGelu>(stream, x_layout, y_layout, y_dtype, X, x_bytes, gather, Wp, bias, offsets, E, P_max,
                                        d_in, d_out, y);
    case kActRelu:
      return launch_pauli_act<kActRelu>(stream, x_layout, y_layout, y_dtype, X, x_bytes, gather, Wp, bias, offsets, E, P_max,
                                        d_in, d_out, y);
    default:
      return launch_pauli_act<kActSigmoid>(stream, x_layout, y_layout, y_dtype, X, x_bytes, gather, Wp, bias, offsets, E,
                                           P_max, d_in, d_out, y);
  }
}
