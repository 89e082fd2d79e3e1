// Teacher-forced ProteinMPNN decoder (scoring).
//
// Reference: run_teacher_forced_decoder (cpp/modules/mpnn/inverse_fold_scalar.cpp:575-663)
// with proteinmpnn_decoder_layer_scalar over all L rows
// (cpp/modules/mpnn/decoder_layer_scalar.cpp:26-151) and a plain log_softmax
// (cpp/primitives/compute/log_softmax_scalar.cpp:8-37). With the causal masks
// of the decoding order, row t of layer l sees for neighbour j
//   bw (j before t): [h_E_tj, W_s[tok_j], h^l_j],  fw: [h_E_tj, 0, h^0_j],
// both scaled by the row mask. As in the autoregressive kernel the W1 product
// is split into A_t = W1a h^l_t + b1, E1 = W1b h_E (here computed in the edge
// kernel, every edge is used once per layer), R^l_j = W1d h^l_j +
// W1c W_s[tok_j] and Q^l_j = W1d h^0_j; and sum_k (W3 g_k + b3) = W3 sum_k g_k + K b3.
// Per layer:
//   tf_edge_kernel  tiles of whole residues (<= 48 edge rows): W1b and W2 on the
//                   fp16 MFMA with split operands (hi + lo / 2048 for weights and
//                   rows, about 22 significant bits), GELU, neighbour sum (all K
//                   slots, no attention mask).
//   tf_node_kernel  tiles of 16 residues: W3, LN1, FFN, LN2, row-mask gate,
//                   then the next layer's [A | R] terms (the products on the
//                   same split-operand fp16 MFMA), or for the last layer
//                   logits and log_softmax in the reference's order.
// Rows may belong to different proteins of a ragged batch: every neighbour
// index is global, so the kernels never look at protein boundaries.
#include "device_math.hpp"
#include "mfma_tile.hpp"
#include "pmpnn_internal.hpp"

namespace hkbs {
namespace {

constexpr int kRows = 48;
constexpr int kLd = kH + 4;
constexpr int kLdF = kFF + 4;

// NB[r] = [A^0_r = W1a_0 h^0_r + b1_0 | R^0_r = W1d_0 h^0_r + T_0[tok_r]]
__global__ void tf_init_kernel(ModelDev m, const float* __restrict__ Q, const int32_t* __restrict__ tokens, int L,
                               float* __restrict__ NB) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)L * kH) return;
  const size_t r = i / kH;
  const int c = static_cast<int>(i % kH);
  NB[r * 256 + c] = Q[((size_t)3 * L + r) * kH + c] + m.dec[0].b1[c];
  NB[r * 256 + kH + c] = Q[r * kH + c] + m.dec[0].T[tokens[r] * kH + c];
}

// One tile of kRows edge rows per workgroup: the K slots of kRows / K
// consecutive residues (one residue when K = 48), their h_E rows split into
// fp16 halves in LDS (hi [kRows][kLdS1] then lo, the layout of tile_gemm).
constexpr int kRB = kRows / 16;
static_assert(kRows % 16 == 0 && kRows >= kKmax, "a tile holds whole residues");

__global__ __launch_bounds__(256, 4) void tf_edge_kernel(DecLayerDev w, const float* __restrict__ h_e,
                                                      const int32_t* __restrict__ idx, const int32_t* __restrict__ pos,
                                                      const float* __restrict__ mask, const float* __restrict__ NB,
                                                      const float* __restrict__ Ql, int L, int K,
                                                      float* __restrict__ msg_sum) {
  // The split h_E slab; once the W2 product has read it, the same bytes hold
  // the fp32 message rows [kRows][kLd] for the neighbour sums (K < 48).
  __shared__ __attribute__((aligned(16))) _Float16 S[2 * kRows * kLdS1];
  float* A = reinterpret_cast<float*>(S);
  static_assert(kRows * kLd * sizeof(float) <= sizeof(S), "fp32 rows alias the slab");
  __shared__ __attribute__((aligned(16))) float gtab[kGeluPolyLds];
  const int nres = kRows / K;
  const int r0 = blockIdx.x * nres;
  const int nr = min(nres, L - r0);
  const int n_rows = nr * K;
  const size_t slot0 = (size_t)r0 * K;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const int n0 = 32 * wave;
  load_gelu_poly(gtab, threadIdx.x, blockDim.x);
  {
    // the tile's h_E rows, split: thread t loads float4 column t % 32 of rows t / 32 + 8 i, all loads
    // issued before the first store
    constexpr int N = kRows * (kH / 4) / 256;
    const int col = 4 * (threadIdx.x & 31), row0 = threadIdx.x >> 5;
    float4 v[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int row = row0 + 8 * i;
      v[i] = row < n_rows ? *reinterpret_cast<const float4*>(h_e + (slot0 + row) * kH + col)
                          : make_float4(0.F, 0.F, 0.F, 0.F);
    }
#pragma unroll
    for (int i = 0; i < N; ++i) put_split4(S, kRows, kLdS1, row0 + 8 * i, col, v[i]);
  }
  // Row 16 rb + r: its residue t and whether the slot adds a context (j a residue, t not masked). Then
  // x = A_t + (bw ? R_j : Q_j) + E1 with E1 = W1b h_E for a slot that adds one, else x = A_t: the
  // accumulators start at A_t + (R_j or Q_j) and the W1b product adds E1.
  int row_t[kRB];
  bool adds[kRB];
  floatx4 acc[kRB][2];
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) {
    const int row = 16 * rb + r;
    const bool valid = row < n_rows;
    const int t = r0 + (valid ? row / K : 0);
    const int j = valid ? idx[slot0 + row] : -1;
    adds[rb] = valid && j >= 0 && j < L && mask[t] != 0.0F;
    const bool bw = adds[rb] && pos[j] < pos[t];
    row_t[rb] = valid ? t : -1;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int c0 = n0 + 16 * nt + 4 * g;
      const float4 x = valid ? *reinterpret_cast<const float4*>(NB + (size_t)t * 256 + c0) : make_float4(0.F, 0.F, 0.F, 0.F);
      const float4 e = !adds[rb] ? make_float4(0.F, 0.F, 0.F, 0.F)
                                 : *reinterpret_cast<const float4*>(bw ? NB + (size_t)j * 256 + kH + c0
                                                                       : Ql + (size_t)j * kH + c0);
      acc[rb][nt] = floatx4{x.x + e.x, x.y + e.y, x.z + e.z, x.w + e.w};
    }
  }
  __syncthreads();
  tile_gemm<kRB, kH, 3>(S, kLdS1, w.W1b_s, n0, (size_t)kH * kH, acc, true);
  __syncthreads();  // every wave is done with the h_E rows
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int c0 = n0 + 16 * nt + 4 * g;
      floatx4 x = acc[rb][nt];
      if (!adds[rb]) {  // A_t alone (zero for a row past the tile's residues)
        const float4 a = row_t[rb] >= 0 ? *reinterpret_cast<const float4*>(NB + (size_t)row_t[rb] * 256 + c0)
                                        : make_float4(0.F, 0.F, 0.F, 0.F);
        x = floatx4{a.x, a.y, a.z, a.w};
      }
      const float4 o = row_t[rb] >= 0 ? make_float4(gelu_poly(x[0], gtab), gelu_poly(x[1], gtab),
                                                    gelu_poly(x[2], gtab), gelu_poly(x[3], gtab))
                                      : make_float4(0.F, 0.F, 0.F, 0.F);
      put_split4(S, kRows, kLdS1, 16 * rb + r, c0, o);
    }
  }
  __syncthreads();
  tile_gemm<kRB, kH, 3>(S, kLdS1, reinterpret_cast<const uint16_t*>(w.W2h), n0, (size_t)kH * kH, acc);
  // g = GELU(W2 x + b2) per valid row; msg_sum[t] = the sum over the residue's K slots
  if (nres == 1) {
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
        for (int rb = 0; rb < kRB; ++rb) v += row_t[rb] >= 0 ? gelu_poly(acc[rb][nt][i] + b, gtab) : 0.0F;
        sv[i] = sum16(v);
      }
      if (r == 0) *reinterpret_cast<float4*>(msg_sum + (size_t)r0 * kH + c0) = make_float4(sv[0], sv[1], sv[2], sv[3]);
    }
    return;
  }
  __syncthreads();  // the slab is consumed; A reuses its bytes
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int c0 = n0 + 16 * nt + 4 * g;
    const float4 bv = *reinterpret_cast<const float4*>(w.b2 + c0);
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb) {
      const floatx4 y = acc[rb][nt];
      *reinterpret_cast<float4*>(A + (16 * rb + r) * kLd + c0) =
          row_t[rb] >= 0 ? make_float4(gelu_poly(y[0] + bv.x, gtab), gelu_poly(y[1] + bv.y, gtab),
                                       gelu_poly(y[2] + bv.z, gtab), gelu_poly(y[3] + bv.w, gtab))
                         : make_float4(0.F, 0.F, 0.F, 0.F);
    }
  }
  __syncthreads();
  for (int task = threadIdx.x; task < nr * kH; task += blockDim.x) {
    const int lr = task / kH, c = task % kH;
    float s = 0.0F;
    for (int k = 0; k < K; ++k) s += A[(lr * K + k) * kLd + c];
    msg_sum[(size_t)(r0 + lr) * kH + c] = s;
  }
}

__global__ __launch_bounds__(256, 3) void tf_node_kernel(ModelDev m, int layer, const float* __restrict__ msg_sum,
                                                      const float* __restrict__ mask, const int32_t* __restrict__ tokens,
                                                      int L, int K, float* __restrict__ h, float* __restrict__ NB,
                                                      float* __restrict__ log_probs) {
  __shared__ __attribute__((aligned(16))) float A[16 * kLd];
  __shared__ __attribute__((aligned(16))) float X[16 * kLd];
  __shared__ __attribute__((aligned(16))) float F[16 * kLdF];
  __shared__ float tbl[17];
  if (threadIdx.x < 17) tbl[threadIdx.x] = kExpNegTable[threadIdx.x];
  const DecLayerDev& w = m.dec[layer];
  const int r0 = blockIdx.x * 16;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;

  for (int task = threadIdx.x; task < 16 * (kH / 4); task += blockDim.x) {
    const int row = task / (kH / 4), c4 = task % (kH / 4);
    float4 v = make_float4(0.F, 0.F, 0.F, 0.F);
    if (r0 + row < L) v = *reinterpret_cast<const float4*>(msg_sum + (size_t)(r0 + row) * kH + 4 * c4);
    *reinterpret_cast<float4*>(A + row * kLd + 4 * c4) = v;
  }
  __syncthreads();
  {
    floatx4 acc[2];
    wave_gemm<2>(A, kLd, w.W3_s, kH, wave * 32, kH, acc);
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 4 * (lane >> 4) + i;
        const int col = wave * 32 + nb * 16 + (lane & 15);
        float v = 0.0F;
        if (r0 + row < L)
          v = h[(size_t)(r0 + row) * kH + col] + (acc[nb][i] + static_cast<float>(K) * w.b3[col]) * (1.0F / 30.0F);
        X[row * kLd + col] = v;
      }
  }
  __syncthreads();
  for (int row = wave; row < 16; row += 4) ln_row_wave(X + row * kLd, w.n1g, w.n1b, A + row * kLd);  // h1
  __syncthreads();
  {
    floatx4 acc[8];
    wave_gemm<8>(A, kLd, w.Win_s, kFF, wave * 128, kH, acc);
#pragma unroll
    for (int nb = 0; nb < 8; ++nb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 4 * (lane >> 4) + i;
        const int col = wave * 128 + nb * 16 + (lane & 15);
        F[row * kLdF + col] = gelu(acc[nb][i] + w.bin[col], tbl);
      }
  }
  __syncthreads();
  {
    floatx4 acc[2];
    wave_gemm<2>(F, kLdF, w.Wout_s, kH, wave * 32, kFF, acc);
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 4 * (lane >> 4) + i;
        const int col = wave * 32 + nb * 16 + (lane & 15);
        X[row * kLd + col] = A[row * kLd + col] + (acc[nb][i] + w.bout[col]);
      }
  }
  __syncthreads();
  for (int row = wave; row < 16; row += 4) {
    float* out = A + row * kLd;
    ln_row_wave(X + row * kLd, w.n2g, w.n2b, out);
    const float mk = (r0 + row < L) ? mask[r0 + row] : 0.0F;
    if (mk != 1.0F) {  // decoder_layer_scalar.cpp:123-140
      out[lane] *= mk;
      out[lane + 64] *= mk;
    }
    if (r0 + row < L) {
      h[(size_t)(r0 + row) * kH + lane] = out[lane];
      h[(size_t)(r0 + row) * kH + lane + 64] = out[lane + 64];
    }
  }
  __syncthreads();
  if (layer + 1 < kLayers) {
    const DecLayerDev& wn = m.dec[layer + 1];
    floatx4 acc[4];
    wave_gemm<4>(A, kLd, w.Wnext_s, 2 * kH, wave * 64, kH, acc);
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 4 * (lane >> 4) + i;
        const int col = wave * 64 + nb * 16 + (lane & 15);  // [0,128): A, [128,256): R
        if (r0 + row >= L) continue;
        const size_t r = r0 + row;
        NB[r * 256 + col] = col < kH ? acc[nb][i] + wn.b1[col]
                                     : acc[nb][i] + wn.T[tokens[r] * kH + (col - kH)];
      }
    return;
  }
  // logits = W_out h + b, then log_softmax, both in the reference's order.
  __shared__ float lg[16 * 32];
  for (int task = threadIdx.x; task < 16 * kV; task += blockDim.x) {
    const int row = task / kV, v = task % kV;
    float acc = 0.0F;
    for (int p = 0; p < kH; ++p) acc += A[row * kLd + p] * m.Wlog_t[p * 32 + v];
    lg[row * 32 + v] = acc + m.blog[v];
  }
  __syncthreads();
  if (threadIdx.x < 16 && r0 + threadIdx.x < L) {
    const float* z = lg + threadIdx.x * 32;
    float row_max = -__builtin_inff();
    for (int d = 0; d < kV; ++d)
      if (z[d] > row_max) row_max = z[d];
    float row_sum = 0.0F;
    for (int d = 0; d < kV; ++d) row_sum += expf(z[d] - row_max);
    const float lrs = logf(row_sum);
    float* out = log_probs + (size_t)(r0 + threadIdx.x) * kV;
    for (int d = 0; d < kV; ++d) out[d] = (z[d] - row_max) - lrs;
  }
}

}  // namespace

hipError_t launch_teacher_forced(const ModelDev& m, const TfArgs& a, hipStream_t stream) {
  const int L = a.L, K = a.K;
  if (L <= 0) return hipSuccess;
  tf_init_kernel<<<(unsigned)(((size_t)L * kH + 255) / 256), 256, 0, stream>>>(m, a.Q, a.tokens, L, a.NB);
  const int nres = kRows / K;
  const unsigned edge_tiles = (unsigned)((L + nres - 1) / nres);
  const unsigned node_tiles = (unsigned)((L + 15) / 16);
  for (int l = 0; l < kLayers; ++l) {
    tf_edge_kernel<<<edge_tiles, 256, 0, stream>>>(m.dec[l], a.h_e, a.idx, a.pos, a.mask, a.NB,
                                                   a.Q + (size_t)l * L * kH, L, K, a.msg_sum);
    tf_node_kernel<<<node_tiles, 256, 0, stream>>>(m, l, a.msg_sum, a.mask, a.tokens, L, K, a.h, a.NB, a.log_probs);
  }
  return hipGetLastError();
}

}  // namespace hkbs
