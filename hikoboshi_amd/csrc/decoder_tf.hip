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
//   tf_edge_kernel  tiles of whole residues (<= 96 edge rows): W1b and W2 on the
//                   fp16 MFMA with split operands (hi + lo / 2048 for weights and
//                   rows, about 22 significant bits), GELU, neighbour sum (all K
//                   slots, no attention mask).
//   tf_node_kernel  tiles of 16 residues: W3, LN1, FFN, LN2, row-mask gate,
//                   then the next layer's [A | R] terms, or for the last layer
//                   logits and log_softmax in the reference's order.
// Rows may belong to different proteins of a ragged batch: every neighbour
// index is global, so the kernels never look at protein boundaries.
#include "device_math.hpp"
#include "mfma_tile.hpp"
#include "pmpnn_internal.hpp"

namespace hkbs {
namespace {

constexpr int kRows = 96;
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

// Edge rows of a tile as split fp16 operands: two half-tiles of 48 rows, each
// hi [48][kLdS1] then lo [48][kLdS1] (the layout of tile_gemm).
constexpr int kHalfRows = kRows / 2;
constexpr int kHalfRB = kHalfRows / 16;
constexpr int kHalfSlab = 2 * kHalfRows * kLdS1;  // halves

__global__ __launch_bounds__(256, 2) void tf_edge_kernel(DecLayerDev w, const float* __restrict__ h_e,
                                                      const int32_t* __restrict__ idx, const int32_t* __restrict__ pos,
                                                      const float* __restrict__ mask, const float* __restrict__ NB,
                                                      const float* __restrict__ Ql, int L, int K,
                                                      float* __restrict__ msg_sum) {
  // The two half-tile slabs; once the W2 product has read them, the same bytes
  // hold the fp32 message rows [kRows][kLd] for the neighbour sums.
  __shared__ __attribute__((aligned(16))) _Float16 S[2 * kHalfSlab];
  float* A = reinterpret_cast<float*>(S);
  static_assert(kRows * kLd * sizeof(float) <= sizeof(S), "fp32 rows alias the slabs");
  __shared__ __attribute__((aligned(16))) float gtab[kGeluPolyLds];
  // per edge row, formed once: its residue t, and its neighbour j with the
  // backward flag (pos[j] < pos[t]) in bit 31, or -1 when the slot adds nothing
  __shared__ int row_t[kRows], row_j[kRows];
  const int nres = kRows / K;
  const int r0 = blockIdx.x * nres;
  const int nr = min(nres, L - r0);
  const int n_rows = nr * K;
  const size_t slot0 = (size_t)r0 * K;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  load_gelu_poly(gtab, threadIdx.x, blockDim.x);
  if (threadIdx.x < n_rows) {
    const int row = threadIdx.x;
    const int t = r0 + row / K;
    const int j = idx[slot0 + row];
    row_t[row] = t;
    row_j[row] = (j >= 0 && j < L && mask[t] != 0.0F) ? (j | (pos[j] < pos[t] ? (int)0x80000000u : 0)) : -1;
  }
  {
    // the tile's h_E rows, split: thread (wave w, lane c) loads float4 column c % 32 of rows
    // 2 w + c / 32 + 8 i, all loads issued before the first store
    constexpr int N = kRows * (kH / 4) / 256;
    float4 v[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int row = 2 * wave + (lane >> 5) + 8 * i;
      v[i] = row < n_rows ? *reinterpret_cast<const float4*>(h_e + (slot0 + row) * kH + 4 * (lane & 31))
                          : make_float4(0.F, 0.F, 0.F, 0.F);
    }
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int row = 2 * wave + (lane >> 5) + 8 * i;
      put_split4(S + (row / kHalfRows) * kHalfSlab, kHalfRows, kLdS1, row % kHalfRows, 4 * (lane & 31), v[i]);
    }
  }
  __syncthreads();
  // Per half-tile: x = A_t + (E1 + (bw ? R_j : Q_j)) for a slot that adds something, else A_t, with
  // E1 = W1b h_E; GELU(x) replaces the half's h_E rows. The A and R|Q rows load before the E1 product.
#pragma unroll 1
  for (int hf = 0; hf < 2; ++hf) {
    _Float16* Sh = S + hf * kHalfSlab;
    float4 base[kHalfRB][2], nbr[kHalfRB][2];
#pragma unroll
    for (int mb = 0; mb < kHalfRB; ++mb) {
      const int row = hf * kHalfRows + mb * 16 + r;
      const int t = row < n_rows ? row_t[row] : 0;
      const int jb = row < n_rows ? row_j[row] : -1;
      const int j = jb & 0x7FFFFFFF;
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const int c0 = wave * 32 + nb * 16 + 4 * g;
        base[mb][nb] = row < n_rows ? *reinterpret_cast<const float4*>(NB + (size_t)t * 256 + c0)
                                    : make_float4(0.F, 0.F, 0.F, 0.F);
        nbr[mb][nb] = jb == -1 ? make_float4(0.F, 0.F, 0.F, 0.F)
                               : *reinterpret_cast<const float4*>(jb < 0 ? NB + (size_t)j * 256 + kH + c0
                                                                         : Ql + (size_t)j * kH + c0);
      }
    }
    floatx4 acc[kHalfRB][2];
    tile_gemm<kHalfRB, kH>(Sh, kLdS1, w.W1b_s, wave * 32, (size_t)kH * kH, acc);
    __syncthreads();  // every wave is done with this half's h_E rows
#pragma unroll
    for (int mb = 0; mb < kHalfRB; ++mb) {
      const int row = hf * kHalfRows + mb * 16 + r;
      const bool adds = row < n_rows && row_j[row] != -1;
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const int c0 = wave * 32 + nb * 16 + 4 * g;
        float4 o = make_float4(0.F, 0.F, 0.F, 0.F);
        if (row < n_rows) {
          const float4 x = base[mb][nb], e = nbr[mb][nb];
          const floatx4 y = acc[mb][nb];
          o = adds ? make_float4(gelu_poly(x.x + (y[0] + e.x), gtab), gelu_poly(x.y + (y[1] + e.y), gtab),
                                 gelu_poly(x.z + (y[2] + e.z), gtab), gelu_poly(x.w + (y[3] + e.w), gtab))
                   : make_float4(gelu_poly(x.x, gtab), gelu_poly(x.y, gtab), gelu_poly(x.z, gtab),
                                 gelu_poly(x.w, gtab));
        }
        put_split4(Sh, kHalfRows, kLdS1, mb * 16 + r, c0, o);
      }
    }
  }
  __syncthreads();
  floatx4 acc2[2][kHalfRB][2];
#pragma unroll
  for (int hf = 0; hf < 2; ++hf)
    tile_gemm<kHalfRB, kH>(S + hf * kHalfSlab, kLdS1, reinterpret_cast<const uint16_t*>(w.W2h), wave * 32,
                           (size_t)kH * kH, acc2[hf]);
  __syncthreads();  // the slabs are consumed; A reuses their bytes
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int c0 = wave * 32 + nb * 16 + 4 * g;
    const float4 bv = *reinterpret_cast<const float4*>(w.b2 + c0);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int mb = 0; mb < kHalfRB; ++mb) {
        const int row = hf * kHalfRows + mb * 16 + r;
        const floatx4 y = acc2[hf][mb][nb];
        *reinterpret_cast<float4*>(A + row * kLd + c0) =
            row < n_rows ? make_float4(gelu_poly(y[0] + bv.x, gtab), gelu_poly(y[1] + bv.y, gtab),
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

__global__ __launch_bounds__(256) void tf_node_kernel(ModelDev m, int layer, const float* __restrict__ msg_sum,
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
    floatx4 acc[1][2];
    zero_acc(acc);
    mfma_tile<1, 2>(A, kLd, w.W3_p, kH, wave * 32, kH, acc);
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 4 * (lane >> 4) + i;
        const int col = wave * 32 + nb * 16 + (lane & 15);
        float v = 0.0F;
        if (r0 + row < L)
          v = h[(size_t)(r0 + row) * kH + col] + (acc[0][nb][i] + static_cast<float>(K) * w.b3[col]) * (1.0F / 30.0F);
        X[row * kLd + col] = v;
      }
  }
  __syncthreads();
  for (int row = wave; row < 16; row += 4) ln_row_wave(X + row * kLd, w.n1g, w.n1b, A + row * kLd);  // h1
  __syncthreads();
  {
    floatx4 acc[1][8];
    zero_acc(acc);
    mfma_tile<1, 8>(A, kLd, w.Win_p, kFF, wave * 128, kH, acc);
#pragma unroll
    for (int nb = 0; nb < 8; ++nb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 4 * (lane >> 4) + i;
        const int col = wave * 128 + nb * 16 + (lane & 15);
        F[row * kLdF + col] = gelu(acc[0][nb][i] + w.bin[col], tbl);
      }
  }
  __syncthreads();
  {
    floatx4 acc[1][2];
    zero_acc(acc);
    mfma_tile<1, 2>(F, kLdF, w.Wout_p, kH, wave * 32, kFF, acc);
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 4 * (lane >> 4) + i;
        const int col = wave * 32 + nb * 16 + (lane & 15);
        X[row * kLd + col] = A[row * kLd + col] + (acc[0][nb][i] + w.bout[col]);
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
    floatx4 acc[1][4];
    zero_acc(acc);
    mfma_tile<1, 4>(A, kLd, w.Wnext_p, 2 * kH, wave * 64, kH, acc);
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 4 * (lane >> 4) + i;
        const int col = wave * 64 + nb * 16 + (lane & 15);  // [0,128): A, [128,256): R
        if (r0 + row >= L) continue;
        const size_t r = r0 + row;
        NB[r * 256 + col] = col < kH ? acc[0][nb][i] + wn.b1[col]
                                     : acc[0][nb][i] + wn.T[tokens[r] * kH + (col - kH)];
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
