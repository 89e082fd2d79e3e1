// ProteinMPNN encoder: 3 message-passing layers on the kNN graph, in the
// reference's rounding order.
//
// Reference: cpp/modules/mpnn/proteinmpnn_encoder_scalar.cpp:169-333. Per layer
//   m_ij  = W3 g(W2 g(W1 [h_i, e_ij, h_j] + b1) + b2) + b3        (g = GELU)
//   h_i  <- LN1(h_i + sum_j (1/30) mask_attend_ij m_ij)            (valid j, in slot order)
//   h_i  <- LN2(h_i + W_out g(W_in h_i + b_in) + b_out) * mask_i
//   e_ij <- LN3(e_ij + W13 g(W12 g(W11 [h_i, e_ij, h_j] + b11) + b12) + b13)  (valid j)
//
// The encoder runs once per backbone and its outputs feed every sequence,
// and its rounding dominates the log-prob deviation at design temperatures,
// so every product here reproduces the reference bit for bit: sequential
// k-order sums without FMA (seq_gemm), Welford LayerNorm, the same
// elementwise order. The only reuse is exact: the first 128 terms of the
// W1 / W11 sums ([h_i] part) are the same prefix for all K edges of residue
// i, so the node kernel computes that prefix once per residue and the edge
// kernels continue the sum with the e_ij and h_j terms.
//
// Kernels per layer:
//   edge_msg_kernel    tile of whole residues (<= 96 edge rows): W1 (e, h_j
//                      terms), W2, W3, then the masked neighbour sum.
//   node_kernel        tile of 32 residues: LN1, FFN, LN2, mask, and the W11
//                      and next-layer W1 prefixes.
//   edge_update_kernel tile of whole residues: W11, W12, W13, residual, LN3.
#include "device_math.hpp"
#include "pmpnn_internal.hpp"

namespace hkbs {
namespace {

constexpr int kRows = 96;    // edge rows per tile
constexpr int kLdE = 98;     // k-major leading dimension of edge tiles
constexpr int kEdgeRM = 6;   // rows per thread (16 row groups)
constexpr int kEdgeCN = 8;   // cols per thread (16 col groups)
constexpr int kKC = 32;      // weight rows staged per chunk
constexpr int kNodeRows = 32;
constexpr int kLdN = 36;

// Loads rows of a [*, 128] row-major matrix into a k-major LDS tile
// A[k * lda + row] (row < n_rows, gathered through rowptr), zero elsewhere.
template <typename RowFn>
__device__ inline void load_kmajor(float* A, int lda, int n_tile_rows, RowFn rowptr) {
  for (int i = threadIdx.x; i < n_tile_rows * 32; i += blockDim.x) {
    const int row = i % n_tile_rows;
    const int kb = i / n_tile_rows;
    const float* src = rowptr(row);
    float4 v = make_float4(0.F, 0.F, 0.F, 0.F);
    if (src) v = *reinterpret_cast<const float4*>(src + 4 * kb);
    A[(4 * kb + 0) * lda + row] = v.x;
    A[(4 * kb + 1) * lda + row] = v.y;
    A[(4 * kb + 2) * lda + row] = v.z;
    A[(4 * kb + 3) * lda + row] = v.w;
  }
}

// Message pass: msg_sum[i] = sum over valid slots (in order) of (1/30) mask_attend m_ij.
__global__ __launch_bounds__(256) void edge_msg_kernel(EncLayerDev w, const float* __restrict__ h_e,
                                                       const float* __restrict__ h_v, const int32_t* __restrict__ idx,
                                                       const float* __restrict__ mask,
                                                       const float* __restrict__ prefix, int L, int K,
                                                       float* __restrict__ msg_sum) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) float A[kH * kLdE];
  __shared__ __attribute__((aligned(16))) float Wbuf[kKC * kH];
  const int nres = kRows / K;
  const int r0 = blockIdx.x * nres;
  const int nr = min(nres, L - r0);
  const int n_rows = nr * K;
  const size_t slot0 = (size_t)r0 * K;
  const int rg = threadIdx.x / 16, cg = threadIdx.x % 16;
  const int row0 = rg * kEdgeRM, col0 = cg * kEdgeCN;

  float acc[kEdgeRM][kEdgeCN];
#pragma unroll
  for (int i = 0; i < kEdgeRM; ++i) {
    const int row = row0 + i;
    const float* pre = row < n_rows ? prefix + (size_t)(r0 + row / K) * 256 + 128 : nullptr;
#pragma unroll
    for (int j = 0; j < kEdgeCN; ++j) acc[i][j] = pre ? pre[col0 + j] : 0.0F;
  }
  load_kmajor(A, kLdE, kRows, [&](int row) -> const float* {
    return row < n_rows ? h_e + (slot0 + row) * kH : nullptr;
  });
  seq_gemm<kEdgeRM, kEdgeCN, kH, kKC>(acc, A, kLdE, row0, w.W1_t + 128 * kH, kH, kH, Wbuf, col0);
  __syncthreads();
  load_kmajor(A, kLdE, kRows, [&](int row) -> const float* {
    if (row >= n_rows) return nullptr;
    const int j = idx[slot0 + row];
    return (j >= 0 && j < L) ? h_v + (size_t)j * kH : nullptr;
  });
  seq_gemm<kEdgeRM, kEdgeCN, kH, kKC>(acc, A, kLdE, row0, w.W1_t + 256 * kH, kH, kH, Wbuf, col0);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kEdgeRM; ++i)
#pragma unroll
    for (int j = 0; j < kEdgeCN; ++j) {
      A[(col0 + j) * kLdE + row0 + i] = (row0 + i < n_rows) ? gelu(acc[i][j] + w.b1[col0 + j]) : 0.0F;
      acc[i][j] = 0.0F;
    }
  seq_gemm<kEdgeRM, kEdgeCN, kH, kKC>(acc, A, kLdE, row0, w.W2_t, kH, kH, Wbuf, col0);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kEdgeRM; ++i)
#pragma unroll
    for (int j = 0; j < kEdgeCN; ++j) {
      A[(col0 + j) * kLdE + row0 + i] = (row0 + i < n_rows) ? gelu(acc[i][j] + w.b2[col0 + j]) : 0.0F;
      acc[i][j] = 0.0F;
    }
  seq_gemm<kEdgeRM, kEdgeCN, kH, kKC>(acc, A, kLdE, row0, w.W3_t, kH, kH, Wbuf, col0);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kEdgeRM; ++i)
#pragma unroll
    for (int j = 0; j < kEdgeCN; ++j) A[(col0 + j) * kLdE + row0 + i] = acc[i][j] + w.b3[col0 + j];
  __syncthreads();
  const float scale = 1.0F / 30.0F;
  for (int task = threadIdx.x; task < nr * kH; task += blockDim.x) {
    const int lr = task / kH, c = task % kH;
    const int r = r0 + lr;
    float upd = 0.0F;
    for (int k = 0; k < K; ++k) {
      const int j = idx[slot0 + lr * K + k];
      if (!(j >= 0 && j < L)) continue;
      float alpha = scale;
      alpha *= mask[r] * mask[j];
      if (alpha == 0.0F) continue;
      upd = alpha * A[c * kLdE + lr * K + k] + upd;
    }
    msg_sum[(size_t)r * kH + c] = upd;
  }
}

// Node update for 32 residues: LN1(h + upd), FFN, LN2, mask; then the W11 prefix
// of this layer's edge update and (when Wnext_t is given) the next layer's W1 prefix.
__global__ __launch_bounds__(256) void node_kernel(EncLayerDev w, const float* __restrict__ Wnext_t,
                                                   const float* __restrict__ msg_sum, const float* __restrict__ mask,
                                                   int L, float* __restrict__ h_v, float* __restrict__ prefix) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) float A[kH * kLdN];
  __shared__ __attribute__((aligned(16))) float X[kH * kLdN];
  __shared__ __attribute__((aligned(16))) float F[kFF * kLdN];
  __shared__ __attribute__((aligned(16))) float Wbuf[16 * kFF];
  const int r0 = blockIdx.x * kNodeRows;
  const int nr = min(kNodeRows, L - r0);
  const int rg = threadIdx.x / 32, cg = threadIdx.x % 32;
  const int row0 = rg * 4;

  // X = h + upd (axpy order: 1 * residual + input)
  for (int i = threadIdx.x; i < kNodeRows * kH; i += blockDim.x) {
    const int row = i % kNodeRows, d = i / kNodeRows;
    float v = 0.0F;
    if (row < nr) v = h_v[(size_t)(r0 + row) * kH + d] + msg_sum[(size_t)(r0 + row) * kH + d];
    X[d * kLdN + row] = v;
  }
  __syncthreads();
  if (threadIdx.x < kNodeRows) welford_ln_col(X + threadIdx.x, A + threadIdx.x, kLdN, w.n1g, w.n1b);  // A = h1
  {
    float acc[4][16];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[i][j] = 0.0F;
    seq_gemm<4, 16, kFF, 16>(acc, A, kLdN, row0, w.Win_t, kFF, kH, Wbuf, cg * 16);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 16; ++j) F[(cg * 16 + j) * kLdN + row0 + i] = gelu(acc[i][j] + w.bin[cg * 16 + j]);
  }
  {
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = 0.0F;
    seq_gemm<4, 4, kH, 16>(acc, F, kLdN, row0, w.Wout_t, kH, kFF, Wbuf, cg * 4);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = cg * 4 + j;
        X[d * kLdN + row0 + i] = A[d * kLdN + row0 + i] + (acc[i][j] + w.bout[d]);
      }
  }
  __syncthreads();
  if (threadIdx.x < kNodeRows) {
    const int row = threadIdx.x;
    welford_ln_col(X + row, A + row, kLdN, w.n2g, w.n2b);
    const float mk = row < nr ? mask[r0 + row] : 0.0F;
    for (int d = 0; d < kH; ++d) A[d * kLdN + row] *= mk;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < nr * kH; i += blockDim.x) {
    const int row = i / kH, d = i % kH;
    h_v[(size_t)(r0 + row) * kH + d] = A[d * kLdN + row];
  }
  // prefixes: [0,128) of W11 and of the next layer's W1 over h'
  for (int part = 0; part < 2; ++part) {
    const float* Wt = part == 0 ? w.W11_t : Wnext_t;
    if (!Wt) break;
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = 0.0F;
    seq_gemm<4, 4, kH, 16>(acc, A, kLdN, row0, Wt, kH, kH, Wbuf, cg * 4);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (row0 + i < nr)
#pragma unroll
        for (int j = 0; j < 4; ++j) prefix[(size_t)(r0 + row0 + i) * 256 + part * 128 + cg * 4 + j] = acc[i][j];
  }
}

__global__ __launch_bounds__(256) void edge_update_kernel(EncLayerDev w, float* __restrict__ h_e,
                                                          const float* __restrict__ h_v,
                                                          const int32_t* __restrict__ idx,
                                                          const float* __restrict__ prefix, int L, int K) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) float A[kH * kLdE];
  __shared__ __attribute__((aligned(16))) float Wbuf[kKC * kH];
  const int nres = kRows / K;
  const int r0 = blockIdx.x * nres;
  const int nr = min(nres, L - r0);
  const int n_rows = nr * K;
  const size_t slot0 = (size_t)r0 * K;
  const int rg = threadIdx.x / 16, cg = threadIdx.x % 16;
  const int row0 = rg * kEdgeRM, col0 = cg * kEdgeCN;

  float acc[kEdgeRM][kEdgeCN];
#pragma unroll
  for (int i = 0; i < kEdgeRM; ++i) {
    const int row = row0 + i;
    const float* pre = row < n_rows ? prefix + (size_t)(r0 + row / K) * 256 : nullptr;
#pragma unroll
    for (int j = 0; j < kEdgeCN; ++j) acc[i][j] = pre ? pre[col0 + j] : 0.0F;
  }
  load_kmajor(A, kLdE, kRows, [&](int row) -> const float* {
    return row < n_rows ? h_e + (slot0 + row) * kH : nullptr;
  });
  seq_gemm<kEdgeRM, kEdgeCN, kH, kKC>(acc, A, kLdE, row0, w.W11_t + 128 * kH, kH, kH, Wbuf, col0);
  __syncthreads();
  load_kmajor(A, kLdE, kRows, [&](int row) -> const float* {
    if (row >= n_rows) return nullptr;
    const int j = idx[slot0 + row];
    return (j >= 0 && j < L) ? h_v + (size_t)j * kH : nullptr;
  });
  seq_gemm<kEdgeRM, kEdgeCN, kH, kKC>(acc, A, kLdE, row0, w.W11_t + 256 * kH, kH, kH, Wbuf, col0);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kEdgeRM; ++i)
#pragma unroll
    for (int j = 0; j < kEdgeCN; ++j) {
      A[(col0 + j) * kLdE + row0 + i] = (row0 + i < n_rows) ? gelu(acc[i][j] + w.b11[col0 + j]) : 0.0F;
      acc[i][j] = 0.0F;
    }
  seq_gemm<kEdgeRM, kEdgeCN, kH, kKC>(acc, A, kLdE, row0, w.W12_t, kH, kH, Wbuf, col0);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kEdgeRM; ++i)
#pragma unroll
    for (int j = 0; j < kEdgeCN; ++j) {
      A[(col0 + j) * kLdE + row0 + i] = (row0 + i < n_rows) ? gelu(acc[i][j] + w.b12[col0 + j]) : 0.0F;
      acc[i][j] = 0.0F;
    }
  seq_gemm<kEdgeRM, kEdgeCN, kH, kKC>(acc, A, kLdE, row0, w.W13_t, kH, kH, Wbuf, col0);
  __syncthreads();
  // x = 1 * e + m  (axpy order), then LN3 per valid row
#pragma unroll
  for (int i = 0; i < kEdgeRM; ++i)
#pragma unroll
    for (int j = 0; j < kEdgeCN; ++j) {
      const int row = row0 + i, c = col0 + j;
      A[c * kLdE + row] = (row < n_rows) ? h_e[(slot0 + row) * kH + c] + (acc[i][j] + w.b13[c]) : 0.0F;
    }
  __syncthreads();
  if (threadIdx.x < n_rows) {
    const int j = idx[slot0 + threadIdx.x];
    if (j >= 0 && j < L) welford_ln_col(A + threadIdx.x, A + threadIdx.x, kLdE, w.n3g, w.n3b);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < n_rows * kH; i += blockDim.x) {
    const int row = i / kH, c = i % kH;
    const int j = idx[slot0 + row];
    if (j >= 0 && j < L) h_e[(slot0 + row) * kH + c] = A[c * kLdE + row];
  }
}

__global__ void zero_kernel(float* __restrict__ p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0.0F;
}

}  // namespace

hipError_t launch_zero(float* p, size_t n, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  const size_t blocks = (n + 255) / 256;
  zero_kernel<<<(unsigned)(blocks < 4096 ? blocks : 4096), 256, 0, stream>>>(p, n);
  return hipGetLastError();
}

hipError_t launch_encoder(const ModelDev& m, const int32_t* idx, const float* mask, int L, int K, float* h_v,
                          float* h_e, const EncoderScratch& ws, hipStream_t stream) {
  if (L <= 0) return hipSuccess;
  hipError_t e = launch_zero(h_v, (size_t)L * kH, stream);
  if (e != hipSuccess) return e;
  e = launch_zero(ws.prefix, (size_t)L * 256, stream);
  if (e != hipSuccess) return e;
  const int nres = kRows / K;
  const unsigned edge_tiles = (unsigned)((L + nres - 1) / nres);
  const unsigned node_tiles = (unsigned)((L + kNodeRows - 1) / kNodeRows);
  for (int l = 0; l < kLayers; ++l) {
    edge_msg_kernel<<<edge_tiles, 256, 0, stream>>>(m.enc[l], h_e, h_v, idx, mask, ws.prefix, L, K, ws.msg_sum);
    node_kernel<<<node_tiles, 256, 0, stream>>>(m.enc[l], l + 1 < kLayers ? m.enc[l + 1].W1_t : nullptr, ws.msg_sum,
                                                mask, L, h_v, ws.prefix);
    edge_update_kernel<<<edge_tiles, 256, 0, stream>>>(m.enc[l], h_e, h_v, idx, ws.prefix, L, K);
  }
  return hipGetLastError();
}

}  // namespace hkbs
