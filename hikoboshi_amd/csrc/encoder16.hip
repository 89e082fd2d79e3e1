// Featurisation and encoder on the fp16 MFMA, for the 16-bit design modes.
//
// The layers are those of encoder.hip and features.hip (edge embedding
// inverse_fold_scalar.cpp:236-279; encoder layers
// proteinmpnn_encoder_scalar.cpp:169-333). Every product runs on the
// 16x16x32 fp16 MFMA with both operands split, v = hi + lo / 2048 (hi =
// fp16(v), lo = fp16((v - hi) * 2048)): hi.hi + (hi.lo + lo.hi) / 2048 in fp32
// carries about 22 significant bits, so the encoder is fp32-accurate (not
// the reference's rounding sequence, which encoder.hip reproduces). Features,
// biases, GELU (gelu_poly in the edge kernels, gelu_fast in the node kernel),
// LayerNorm (two-pass), residuals and the neighbour sum are fp32, and h_V, h_E
// are stored in fp32. The kNN graph comes from the exact fp32 kernel.
//
// Edge products (the bulk of the work) run as workgroup tiles of 48 or 64 edge
// rows and four waves: the tile's operand sits in LDS already split into fp16
// hi / lo halves, every wave reads all of its rows and produces 32 of the 128
// output columns, so each weight fragment streamed from L2 feeds 3 or 4 row
// blocks (the edge embedding builds its features into such a tile in two
// parts). The node kernel keeps 16 rows per wave with the fp32 operand split
// as it is read (wave_gemm).
//
// W1 [h_i | e_ij | h_j] x (and W11) is W1a h_i + W1b e_ij + W1c h_j: node16
// forms the W1a and W1c products of every residue once per layer into four
// planes [L][128] (W11 h_i and W11 h_j for this layer's edge update, W1 h_i
// and W1 h_j for the next layer's messages; zero for layer 0, where h = 0),
// and the edge kernels run the K = 128 product over e_ij, starting from
// P[i] + P[j] (no h_j block for an empty slot).
//
// Kernels:
//   edge_embed16   64 edge slots per workgroup (4 waves): 416 features ->
//                  W_edge -> LN -> W_e -> h_E.
//   per layer:
//   edge_msg16     one residue per workgroup (48 slots, 4 waves): W1 e_ij +
//                  P, GELU, W2, GELU -> the sum over the residue's slots
//                  weighted by mask_i mask_j / 30, and the sum of the weights.
//   node16         16 residues per workgroup (4 waves): upd = W3 sum + (sum of
//                  weights) b3, LN1(h + upd), the FFN on the MFMA (a quarter
//                  of it per wave), LN2, mask; then the four W1 / W11 blocks
//                  of the new h.
//   edge_update16  64 edge slots per workgroup (4 waves): W11 e_ij + P, GELU,
//                  W12, GELU, W13, residual, LN3 -> h_E (valid slots).
#include "device_math.hpp"
#include "edge_chunk.hpp"
#include "mfma_tile.hpp"
#include "pmpnn_internal.hpp"

namespace hkbs {
namespace {


constexpr int kLdF = kFF + 4;      // floats per row of the FFN hidden layer
constexpr int kLdH = kH + 4;       // floats per row of a 128-wide activation
static_assert(kKmax == 48, "edge_msg16 covers a residue's slots with 3 waves of 16 rows");
static_assert(kEdgeIn % 32 == 0, "MFMA k-steps");


// out[row][n0 + col] = GELU(acc + bias) (fp32) for the wave's 16 rows.
template <int NT>
__device__ inline void store_gelu(const floatx4 (&acc)[NT], const float* __restrict__ bias, int n0, float* out,
                                  int ldo, const float* tbl) {
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int col = n0 + 16 * nt + r;
    const float bv = bias[col];
#pragma unroll
    for (int i = 0; i < 4; ++i) out[(4 * g + i) * ldo + col] = gelu_fast(acc[nt][i] + bv, tbl);
  }
}

// The tile's h_E rows (slot = slot_of(row); negative: a zero row) into the
// split slab (K = 128). Thread t fills float4 column t % 32 of rows t / 32,
// t / 32 + 8, ...; all of its row loads are issued before the first store.
template <int RB, typename SlotOf>
__device__ inline void tile_rows(_Float16* S, const float* __restrict__ h_e, SlotOf slot_of) {
  constexpr int R = 16 * RB, N = R * 32 / kTileThreads;
  const int col = 4 * (threadIdx.x & 31), row0 = threadIdx.x >> 5;
  float4 v[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const long long slot = slot_of(row0 + 8 * i);
    v[i] = slot >= 0 ? *reinterpret_cast<const float4*>(h_e + (size_t)slot * kH + col) : make_float4(0.F, 0.F, 0.F, 0.F);
  }
#pragma unroll
  for (int i = 0; i < N; ++i) put_split4(S, R, kLdS1, row0 + 8 * i, col, v[i]);
}

// Starting value of the first product of an edge row of residue i with
// neighbour j: P[pi][i][c] + P[pj][j][c] + b[c] for columns c0 .. c0 + 3 (P:
// planes of [L][128] floats holding the W1 h_i and h_j blocks of
// [h_i | e_ij | h_j], formed per residue by node16); an empty slot (j outside
// [0, L)) has no h_j term.
__device__ inline floatx4 edge_base(const float* __restrict__ P, size_t i, int j, int L, int pi, int pj,
                                    const float* __restrict__ b, int c0) {
  float4 a = *reinterpret_cast<const float4*>(P + ((size_t)pi * L + i) * kH + c0);
  if (j >= 0 && j < L) {
    const float4 q = *reinterpret_cast<const float4*>(P + ((size_t)pj * L + j) * kH + c0);
    a = make_float4(a.x + q.x, a.y + q.y, a.z + q.z, a.w + q.w);
  }
  const float4 bv = *reinterpret_cast<const float4*>(b + c0);
  return floatx4{a.x + bv.x, a.y + bv.y, a.z + bv.z, a.w + bv.w};
}

// GELU(acc + bias) of the wave's columns into the split slab (K = 128 operand
// of the next product); no bias when bias is null.
template <int RB>
__device__ inline void tile_store_gelu(const floatx4 (&acc)[RB][2], const float* __restrict__ bias, _Float16* S,
                                       const float* gtab) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int c0 = 32 * wave + 16 * nt + 4 * g;
    const float4 bv = bias ? *reinterpret_cast<const float4*>(bias + c0) : make_float4(0.F, 0.F, 0.F, 0.F);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const float4 v = make_float4(gelu_poly(acc[rb][nt][0] + bv.x, gtab), gelu_poly(acc[rb][nt][1] + bv.y, gtab),
                                   gelu_poly(acc[rb][nt][2] + bv.z, gtab), gelu_poly(acc[rb][nt][3] + bv.w, gtab));
      put_split4(S, 16 * RB, kLdS1, 16 * rb + r, c0, v);
    }
  }
}

// Two-pass LayerNorm (fp32, eps 1e-5) of each tile row, in place: a row's 128
// columns are spread over the four waves, which exchange per-row partial
// sums through stat[4][16 RB]. Ends with a barrier.
template <int RB>
__device__ inline void tile_layer_norm(floatx4 (&acc)[RB][2], const float* __restrict__ gam,
                                       const float* __restrict__ bet, float (*stat)[16 * RB]) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  float mean[RB], inv[RB];
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      float v = 0.0F;
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float d = pass == 0 ? acc[rb][nt][i] : acc[rb][nt][i] - mean[rb];
          v += pass == 0 ? d : d * d;
        }
      v += __shfl_xor(v, 16, 64);
      v += __shfl_xor(v, 32, 64);
      if (g == 0) stat[wave][16 * rb + r] = v;
    }
    __syncthreads();
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int row = 16 * rb + r;
      const float t = ((stat[0][row] + stat[1][row]) + stat[2][row]) + stat[3][row];
      if (pass == 0) mean[rb] = t * (1.0F / 128.0F);
      else inv[rb] = 1.0F / sqrtf(t * (1.0F / 128.0F) + 1.0e-5F);
    }
    __syncthreads();
  }
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int c0 = 32 * wave + 16 * nt + 4 * g;
    const float4 gm = *reinterpret_cast<const float4*>(gam + c0);
    const float4 bt = *reinterpret_cast<const float4*>(bet + c0);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      acc[rb][nt][0] = (acc[rb][nt][0] - mean[rb]) * inv[rb] * gm.x + bt.x;
      acc[rb][nt][1] = (acc[rb][nt][1] - mean[rb]) * inv[rb] * gm.y + bt.y;
      acc[rb][nt][2] = (acc[rb][nt][2] - mean[rb]) * inv[rb] * gm.z + bt.z;
      acc[rb][nt][3] = (acc[rb][nt][3] - mean[rb]) * inv[rb] * gm.w + bt.w;
    }
  }
}

// Two-pass LayerNorm (fp32, eps 1e-5) of the 4 rows a lane holds in acc[8]
// (all 128 columns of the row live in the 16 lanes of its group).
__device__ inline void ln_acc(floatx4 (&acc)[8], const float* __restrict__ gam, const float* __restrict__ bet) {
  const int r = threadIdx.x & 15;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float s = 0.0F;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) s += acc[nt][i];
    const float mean = sum16(s) * (1.0F / 128.0F);
    float q = 0.0F;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      const float d = acc[nt][i] - mean;
      q += d * d;
    }
    const float inv = 1.0F / sqrtf(sum16(q) * (1.0F / 128.0F) + 1.0e-5F);
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      const int col = 16 * nt + r;
      acc[nt][i] = (acc[nt][i] - mean) * inv * gam[col] + bet[col];
    }
  }
}

// 64 consecutive edge slots per workgroup: one tile of 4 row blocks. The 416
// features are built in four parts (feature chunks 0 .. 7, 8 .. 13, 14 .. 19
// and 20 .. 25, 16 features each), so that the split slab holds 128 inputs at
// a time and three workgroups fit a CU.
constexpr int kEmbedChunks0 = 8;  // chunks of the first part; the other three take 6 each
constexpr int kLdE = 16 * kEmbedChunks0 + 8;  // halves per slab row
__global__ __launch_bounds__(kTileThreads, 3) void edge_embed16_kernel(ModelDev m, const float* __restrict__ coords,
                                                                       const uint8_t* __restrict__ src,
                                                                       const int32_t* __restrict__ resid,
                                                                       const int32_t* __restrict__ chain,
                                                                       const int32_t* __restrict__ idx, int L, int K,
                                                                       float* __restrict__ h_e) {
  constexpr int RB = 4, R = 16 * RB;
  static_assert(kEdgeIn == 26 * 16 && kLdE >= kLdS1, "feature chunks");
  __shared__ __attribute__((aligned(16))) _Float16 S[2 * R * kLdE];
  __shared__ float stat[4][R];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const int n0 = 32 * wave;
  const long long S_ = (long long)L * K;
  const long long base = (long long)blockIdx.x * R;
  // Per tile row, staged once: the atoms of residue res (q) and of its
  // neighbour j (n), their presence bits (q: bits 0-4, n: bits 8-12; bit 16:
  // j is a residue) and the positional class. Waves 0, 1 and 2 load the three
  // parts for the row of their lane.
  // 17 floats per row: lane = row reads one column of 64 rows, so an odd stride keeps them in distinct banks
  __shared__ float xq[R][17], xn[R][17];
  __shared__ int info[R][2];
  __shared__ float tbl[17];
  if (threadIdx.x < 17) tbl[threadIdx.x] = kExpNegTable[threadIdx.x];
  {
    const int row = lane;
    const long long slot = base + row;
    const bool in = slot < S_;
    const int j = in ? idx[slot] : -1;
    const int res = in ? static_cast<int>(slot / K) : 0;
    const bool nb = j >= 0 && j < L;
    if (wave == 0) {
#pragma unroll
      for (int e = 0; e < 15; ++e) xq[row][e] = coords[(size_t)res * 15 + e];
    } else if (wave == 1) {
#pragma unroll
      for (int e = 0; e < 15; ++e) xn[row][e] = nb ? coords[(size_t)j * 15 + e] : 0.0F;
    } else if (wave == 2) {
      int bits = nb ? 1 << 16 : 0;
#pragma unroll
      for (int a = 0; a < 5; ++a) {
        bits |= (src[(size_t)res * 5 + a] != 0) << a;
        if (nb) bits |= (src[(size_t)j * 5 + a] != 0) << (8 + a);
      }
      info[row][0] = bits;
      info[row][1] = nb ? positional_class(resid, chain, res, j) : 0;
    }
  }
  __syncthreads();
  floatx4 acc[RB][2];
  // features of chunks [c0, c0 + nc) of the tile's rows into the split slab: wave w takes chunks c0 + w,
  // c0 + w + 4, ... (wave-uniform), its lanes the 64 rows
  auto build = [&](int c0, int nc) {
    const int row = lane;
    const int bits = info[row][0];
    for (int c = c0 + wave; c < c0 + nc; c += 4) {
      float out[16];
      if (!(bits >> 16)) {
#pragma unroll
        for (int f = 0; f < 16; ++f) out[f] = 0.0F;
      } else if (c == 0) {
        positional_chunk(m, info[row][1], out);
      } else {
        const int qa = kPairQ[c - 1], na = kPairN[c - 1];
        if (((bits >> qa) & (bits >> (8 + na)) & 1) == 0) {
#pragma unroll
          for (int f = 0; f < 16; ++f) out[f] = 0.0F;
        } else {
          rbf_chunk_fma(&xq[row][3 * qa], &xn[row][3 * na], out, tbl);
        }
      }
      // hi and lo halves 8 at a time (16-byte stores: 16 lanes, 16 rows 4 banks apart, fill all banks once)
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        f16x8 h, l;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float f = out[8 * q + e];
          const _Float16 hi = static_cast<_Float16>(__builtin_amdgcn_fmed3f(f, -65504.0F, 65504.0F));
          h[e] = hi;
          l[e] = static_cast<_Float16>((f - static_cast<float>(hi)) * 2048.0F);
        }
        *reinterpret_cast<f16x8*>(S + row * kLdE + 16 * (c - c0) + 8 * q) = h;
        *reinterpret_cast<f16x8*>(S + (R + row) * kLdE + 16 * (c - c0) + 8 * q) = l;
      }
    }
    __syncthreads();
  };
  constexpr int kC1 = 6;
  static_assert(kEmbedChunks0 + 3 * kC1 == 26, "feature parts");
  build(0, kEmbedChunks0);
  tile_gemm<RB, 16 * kEmbedChunks0>(S, kLdE, m.enc16.Wedge, n0, (size_t)kEdgeIn * kH, acc);
#pragma unroll
  for (int part = 0; part < 3; ++part) {
    const int c0 = kEmbedChunks0 + kC1 * part;
    __syncthreads();  // every wave is done with the previous part
    build(c0, kC1);
    tile_gemm<RB, 16 * kC1>(S, kLdE, m.enc16.Wedge + (size_t)(2 * c0) * kH * 8, n0, (size_t)kEdgeIn * kH, acc, true);
  }
  tile_layer_norm<RB>(acc, m.ne_g, m.ne_b, stat);
#pragma unroll
  for (int nt = 0; nt < 2; ++nt)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
      put_split4(S, R, kLdS1, 16 * rb + r, n0 + 16 * nt + 4 * g,
                 make_float4(acc[rb][nt][0], acc[rb][nt][1], acc[rb][nt][2], acc[rb][nt][3]));
  __syncthreads();
  tile_gemm<RB, kH>(S, kLdS1, m.enc16.We, n0, (size_t)kH * kH, acc);
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const long long slot = base + 16 * rb + r;
    if (slot >= S_) continue;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int c0 = n0 + 16 * nt + 4 * g;
      const float4 bv = *reinterpret_cast<const float4*>(m.We_b + c0);
      *reinterpret_cast<float4*>(h_e + (size_t)slot * kH + c0) =
          make_float4(acc[rb][nt][0] + bv.x, acc[rb][nt][1] + bv.y, acc[rb][nt][2] + bv.z, acc[rb][nt][3] + bv.w);
    }
  }
}

// One residue per workgroup: its 48 slots as one tile of 3 row blocks. The
// message of slot k is m_k = W3 g_k + b3 with g_k = GELU(W2 GELU(W1 x_k + b1) +
// b2), and upd_i = sum_k alpha_k m_k = W3 (sum_k alpha_k g_k) + (sum_k alpha_k)
// b3, so this kernel stops at s_i = sum_k alpha_k g_k and a_i = sum_k alpha_k
// (gsum[i][0 .. 127] and gsum[128 L + i]); node16 applies W3 to 16 residues
// at a time.
__global__ __launch_bounds__(kTileThreads, 4) void edge_msg16_kernel(EncLayerDev w, Enc16LayerDev w16,
                                                                  const float* __restrict__ h_e,
                                                                  const int32_t* __restrict__ idx,
                                                                  const float* __restrict__ mask,
                                                                  const float* __restrict__ prefix, int L, int K,
                                                                  float* __restrict__ gsum) {
  constexpr int RB = 3;
  __shared__ __attribute__((aligned(16))) _Float16 S[2 * 16 * RB * kLdS1];
  __shared__ __attribute__((aligned(16))) float gtab[kGeluPolyLds];
  const int res = blockIdx.x;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const int n0 = 32 * wave;
  load_gelu_poly(gtab, threadIdx.x, kTileThreads);
  tile_rows<RB>(S, h_e, [&](int row) -> long long { return row < K ? (long long)res * K + row : -1; });
  // weight of slot 16 rb + r in the neighbour sum: mask_i mask_j / 30 for a valid slot
  float alpha[RB];
  floatx4 acc[RB][2];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int k = 16 * rb + r;
    const int j = k < K ? idx[(size_t)res * K + k] : -1;
    alpha[rb] = (j >= 0 && j < L) ? mask[res] * mask[j] * (1.0F / 30.0F) : 0.0F;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) acc[rb][nt] = edge_base(prefix, res, j, L, 2, 3, w.b1, n0 + 16 * nt + 4 * g);
  }
  __syncthreads();
  // rows 128 .. 255 of W1 (packed k-blocks 16 .. 31) over e_ij, added to the h_i, h_j blocks and b1
  tile_gemm<RB, kH, 3>(S, kLdS1, w16.W1 + (size_t)16 * kH * 8, n0, (size_t)3 * kH * kH, acc, true);
  __syncthreads();  // every wave is done with e_ij
  tile_store_gelu<RB>(acc, nullptr, S, gtab);
  __syncthreads();
  tile_gemm<RB, kH, 3>(S, kLdS1, w16.W2, n0, (size_t)kH * kH, acc);
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int c0 = n0 + 16 * nt + 4 * g;
    const float4 bv = *reinterpret_cast<const float4*>(w.b2 + c0);
    float sv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float b = i == 0 ? bv.x : i == 1 ? bv.y : i == 2 ? bv.z : bv.w;
      float v = 0.0F;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) v += alpha[rb] * gelu_poly(acc[rb][nt][i] + b, gtab);
      sv[i] = sum16(v);
    }
    if (r == 0) *reinterpret_cast<float4*>(gsum + (size_t)res * kH + c0) = make_float4(sv[0], sv[1], sv[2], sv[3]);
  }
  if (wave == 0) {
    float a = 0.0F;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) a += alpha[rb];
    a = sum16(a);
    if (lane == 0) gsum[(size_t)L * kH + res] = a;
  }
}

// 16 residues per workgroup of four waves; lane (r, g) of a wave holds rows
// 4 g + i, columns 16 nt + r of a 128-wide block (the MFMA output layout).
// Wave w first forms columns [32 w, 32 w + 32) of the neighbour update
// upd = W3 s + a b3 from edge_msg16's sums; wave 0 forms h1 = LN1(h + upd)
// for all 16 rows; wave w computes the FFN hidden columns [128 w, 128 w + 128)
// and the W_out partial sum over those inputs; wave 0 adds the four partials
// in order, the residual, LN2 and the mask.
__global__ __launch_bounds__(256) void node16_kernel(EncLayerDev w, Enc16LayerDev w16, const float* __restrict__ gsum,
                                                     const float* __restrict__ mask, int L, float* __restrict__ h_v,
                                                     const uint16_t* __restrict__ W1_next, float* __restrict__ prefix) {
  __shared__ __attribute__((aligned(16))) float A[16 * kLdH];
  __shared__ __attribute__((aligned(16))) float F[16 * kLdF];
  __shared__ __attribute__((aligned(16))) float Pt[4][16 * kLdH];
  __shared__ float tbl[17];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const int r0 = blockIdx.x * 16;
  if (threadIdx.x < 17) tbl[threadIdx.x] = kExpNegTable[threadIdx.x];
  // the 16 rows of s into A (float4 column t % 32 of rows t / 32 and t / 32 + 8)
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int row = (threadIdx.x >> 5) + 8 * q, c = 4 * (threadIdx.x & 31);
    const int res = r0 + row;
    *reinterpret_cast<float4*>(A + row * kLdH + c) =
        res < L ? *reinterpret_cast<const float4*>(gsum + (size_t)res * kH + c) : make_float4(0.F, 0.F, 0.F, 0.F);
  }
  __syncthreads();
  {
    floatx4 u[2];
    wave_gemm<2>(A, kLdH, w16.W3, kH, 32 * wave, kH, u);
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int col = 32 * wave + 16 * nt + r;
      const float bv = w.b3[col];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int res = r0 + 4 * g + i;
        const float a = res < L ? gsum[(size_t)L * kH + res] : 0.0F;
        Pt[0][(4 * g + i) * kLdH + col] = u[nt][i] + a * bv;
      }
    }
  }
  __syncthreads();
  floatx4 x[8];
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int res = r0 + 4 * g + i;
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) {
        const int col = 16 * nt + r;
        x[nt][i] = res < L ? h_v[(size_t)res * kH + col] + Pt[0][(4 * g + i) * kLdH + col] : 0.0F;
      }
    }
  ln_acc(x, w.n1g, w.n1b);
#pragma unroll
    for (int nt = 0; nt < 8; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) A[(4 * g + i) * kLdH + 16 * nt + r] = x[nt][i];
  }
  __syncthreads();
  floatx4 acc[8];
  wave_gemm<8>(A, kLdH, w16.Win, kFF, kH * wave, kH, acc);
  store_gelu<8>(acc, w.bin, kH * wave, F, kLdF, tbl);
  __syncthreads();
  // inputs [128 w, 128 w + 128) of W_out: its packed rows 16 w .. 16 w + 15
  wave_gemm<8>(F + kH * wave, kLdF, w16.Wout + (size_t)wave * 16 * kH * 8, kH, 0, kH, acc, (size_t)kFF * kH);
#pragma unroll
  for (int nt = 0; nt < 8; ++nt)
#pragma unroll
    for (int i = 0; i < 4; ++i) Pt[wave][(4 * g + i) * kLdH + 16 * nt + r] = acc[nt][i];
  __syncthreads();
  if (wave == 0) {
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) {
    const int col = 16 * nt + r;
    const float bv = w.bout[col];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int at = (4 * g + i) * kLdH + col;
      x[nt][i] = x[nt][i] + ((((Pt[0][at] + Pt[1][at]) + Pt[2][at]) + Pt[3][at]) + bv);
    }
  }
  ln_acc(x, w.n2g, w.n2b);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int res = r0 + 4 * g + i;
    const float mk = res < L ? mask[res] : 0.0F;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      const float hv = x[nt][i] * mk;
      A[(4 * g + i) * kLdH + 16 * nt + r] = hv;
      if (res < L) h_v[(size_t)res * kH + 16 * nt + r] = hv;
    }
  }
  }
  __syncthreads();
  // products of the new h into the planes [W11 h_i | W11 h_j | next W1 h_i | next W1 h_j] of prefix
  // ([4][L][128]): wave w takes plane w (packed k-blocks 0 .. 15 for the h_i rows, 32 .. 47 for the h_j rows of the K = 384 matrices;
  // lo 384 x 128 halves after hi)
  if (wave >= 2 && !W1_next) return;
  floatx4 pacc[8];
  wave_gemm<8>(A, kLdH, (wave < 2 ? w16.W11 : W1_next) + (size_t)(wave & 1) * 32 * kH * 8, kH, 0, kH, pacc,
               (size_t)3 * kH * kH);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int res = r0 + 4 * g + i;
    if (res >= L) continue;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) prefix[((size_t)wave * L + res) * kH + 16 * nt + r] = pacc[nt][i];
  }
}

// 64 consecutive edge slots per workgroup: one tile of 4 row blocks.
__global__ __launch_bounds__(kTileThreads, 3) void edge_update16_kernel(EncLayerDev w, Enc16LayerDev w16,
                                                                     float* __restrict__ h_e,
                                                                     const int32_t* __restrict__ idx,
                                                                     const float* __restrict__ prefix, int L, int K) {
  constexpr int RB = 4;
  __shared__ __attribute__((aligned(16))) _Float16 S[2 * 16 * RB * kLdS1];
  __shared__ float stat[4][16 * RB];
  __shared__ __attribute__((aligned(16))) float gtab[kGeluPolyLds];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const int n0 = 32 * wave;
  load_gelu_poly(gtab, threadIdx.x, kTileThreads);
  const long long S_ = (long long)L * K;
  const long long base = (long long)blockIdx.x * 16 * RB;
  tile_rows<RB>(S, h_e, [&](int row) -> long long { return base + row < S_ ? base + row : -1; });
  floatx4 acc[RB][2];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const long long slot = base + 16 * rb + r;
    const size_t res = slot < S_ ? (size_t)(slot / K) : 0;
    const int j = slot < S_ ? idx[slot] : -1;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) acc[rb][nt] = edge_base(prefix, res, j, L, 0, 1, w.b11, n0 + 16 * nt + 4 * g);
  }
  __syncthreads();
  // rows 128 .. 255 of W11 (packed k-blocks 16 .. 31) over e_ij, added to the h_i, h_j blocks and b11
  tile_gemm<RB, kH, 3>(S, kLdS1, w16.W11 + (size_t)16 * kH * 8, n0, (size_t)3 * kH * kH, acc, true);
  __syncthreads();
  tile_store_gelu<RB>(acc, nullptr, S, gtab);
  __syncthreads();
  tile_gemm<RB, kH, 3>(S, kLdS1, w16.W12, n0, (size_t)kH * kH, acc);
  __syncthreads();
  tile_store_gelu<RB>(acc, w.b12, S, gtab);
  // x = (e + b13) + W13 g: the residual rows start the last product's accumulators
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int c0 = n0 + 16 * nt + 4 * g;
    const float4 bv = *reinterpret_cast<const float4*>(w.b13 + c0);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const long long slot = base + 16 * rb + r;
      const float4 e = slot < S_ ? *reinterpret_cast<const float4*>(h_e + (size_t)slot * kH + c0)
                                 : make_float4(0.F, 0.F, 0.F, 0.F);
      acc[rb][nt] = floatx4{e.x + bv.x, e.y + bv.y, e.z + bv.z, e.w + bv.w};
    }
  }
  __syncthreads();
  tile_gemm<RB, kH, 3>(S, kLdS1, w16.W13, n0, (size_t)kH * kH, acc, true);
  // LN3 over each row's 128 columns (four waves)
  tile_layer_norm<RB>(acc, w.n3g, w.n3b, stat);
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const long long slot = base + 16 * rb + r;
    if (slot >= S_) continue;
    const int j = idx[slot];
    if (j < 0 || j >= L) continue;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int c0 = n0 + 16 * nt + 4 * g;
      *reinterpret_cast<float4*>(h_e + (size_t)slot * kH + c0) =
          make_float4(acc[rb][nt][0], acc[rb][nt][1], acc[rb][nt][2], acc[rb][nt][3]);
    }
  }
}

}  // namespace

hipError_t launch_encoder16(const ModelDev& m, const float* coords, const uint8_t* atom_src, const int32_t* resid,
                            const int32_t* chain, const int32_t* idx, const float* mask, int L, int K, float* h_v,
                            float* h_e, const EncoderScratch& ws, hipStream_t stream) {
  if (L <= 0) return hipSuccess;
  if (K < 1 || K > kKmax) return hipErrorInvalidValue;
  const size_t S = (size_t)L * K;
  const unsigned tiles64 = (unsigned)((S + 63) / 64);
  hipError_t e = launch_zero(h_v, (size_t)L * kH, stream);
  if (e != hipSuccess) return e;
  edge_embed16_kernel<<<tiles64, kTileThreads, 0, stream>>>(m, coords, atom_src, resid, chain, idx, L, K, h_e);
  e = launch_zero(ws.prefix, (size_t)L * kPrefix, stream);  // layer 0: h = 0, so its W1 blocks are 0
  if (e != hipSuccess) return e;
  // [L][128] weighted GELU sums and [L] weight sums of edge_msg16 (the [S][128] + L message buffer is
  // otherwise unused here)
  float* gsum = ws.msg;
  for (int l = 0; l < kLayers; ++l) {
    const Enc16LayerDev& w16 = m.enc16.layer[l];
    const uint16_t* W1_next = l + 1 < kLayers ? m.enc16.layer[l + 1].W1 : nullptr;
    edge_msg16_kernel<<<(unsigned)L, kTileThreads, 0, stream>>>(m.enc[l], w16, h_e, idx, mask, ws.prefix, L, K,
                                                                 gsum);
    node16_kernel<<<(unsigned)((L + 15) / 16), 256, 0, stream>>>(m.enc[l], w16, gsum, mask, L, h_v, W1_next,
                                                                ws.prefix);
    edge_update16_kernel<<<tiles64, kTileThreads, 0, stream>>>(m.enc[l], w16, h_e, idx, ws.prefix, L, K);
  }
  return hipGetLastError();
}

}  // namespace hkbs
