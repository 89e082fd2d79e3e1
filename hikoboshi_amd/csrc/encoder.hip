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
//   edge_msg_kernel    tile of 32 edge rows: W1 (e, h_j terms), W2, W3 -> m_ij.
//   node_kernel        tile of 4 residues: the masked neighbour sum of m_ij in
//                      slot order, LN1, FFN, LN2, mask, and the W11 and
//                      next-layer W1 prefixes.
//   edge_update_kernel tile of 32 edge rows: W11, W12, W13, residual, LN3.
// Small tiles keep several workgroups on every CU; the weights stream through
// LDS in double-buffered chunks.
#include <cstdlib>

#include "device_math.hpp"
#include "pmpnn_internal.hpp"

namespace hkbs {
namespace {

constexpr int kRows = 32;    // edge rows per tile (any rows of the [L * K] edge list)
constexpr int kLdE = 36;     // k-major leading dimension of edge tiles
constexpr int kEdgeRM = 4;   // rows per thread (8 row groups)
constexpr int kEdgeCN = 4;   // cols per thread (32 col groups)
constexpr int kKC = 32;      // weight rows staged per chunk

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

// Edge messages m_ij = W3 GELU(W2 GELU(W1 [h_i, e_ij, h_j] + b1) + b2) + b3 for
// a tile of kRows consecutive edge rows; the neighbour sum is taken in order
// by node_kernel.
__global__ __launch_bounds__(256) void edge_msg_kernel(EncLayerDev w, const float* __restrict__ h_e,
                                                       const float* __restrict__ h_v, const int32_t* __restrict__ idx,
                                                       const float* __restrict__ prefix, int L, int K,
                                                       float* __restrict__ msg) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) float A[kH * kLdE];
  __shared__ __attribute__((aligned(16))) float Wbuf[2 * kKC * kH];
  __shared__ float tbl[17];
  if (threadIdx.x < 17) tbl[threadIdx.x] = kExpNegTable[threadIdx.x];
  const size_t S = (size_t)L * K;
  const size_t slot0 = (size_t)blockIdx.x * kRows;
  const int n_rows = (int)min((size_t)kRows, S - slot0);
  const int rg = threadIdx.x / 32, cg = threadIdx.x % 32;
  const int row0 = rg * kEdgeRM, col0 = cg * kEdgeCN;

  float acc[kEdgeRM][kEdgeCN];
#pragma unroll
  for (int i = 0; i < kEdgeRM; ++i) {
    const int row = row0 + i;
    const float* pre = row < n_rows ? prefix + ((slot0 + row) / K) * 256 + 128 : nullptr;
#pragma unroll
    for (int j = 0; j < kEdgeCN; ++j) acc[i][j] = pre ? pre[col0 + j] : 0.0F;
  }
  load_kmajor(A, kLdE, kRows, [&](int row) -> const float* {
    return row < n_rows ? h_e + (slot0 + row) * kH : nullptr;
  });
  seq_gemm<kEdgeRM, kEdgeCN, kH, kKC>(acc, A, kLdE, row0, w.W1_t + 128 * kH, kH, kH, Wbuf, col0);
  load_kmajor(A, kLdE, kRows, [&](int row) -> const float* {
    if (row >= n_rows) return nullptr;
    const int j = idx[slot0 + row];
    return (j >= 0 && j < L) ? h_v + (size_t)j * kH : nullptr;
  });
  seq_gemm<kEdgeRM, kEdgeCN, kH, kKC>(acc, A, kLdE, row0, w.W1_t + 256 * kH, kH, kH, Wbuf, col0);
#pragma unroll
  for (int i = 0; i < kEdgeRM; ++i)
#pragma unroll
    for (int j = 0; j < kEdgeCN; ++j) {
      A[(col0 + j) * kLdE + row0 + i] = (row0 + i < n_rows) ? gelu(acc[i][j] + w.b1[col0 + j], tbl) : 0.0F;
      acc[i][j] = 0.0F;
    }
  seq_gemm<kEdgeRM, kEdgeCN, kH, kKC>(acc, A, kLdE, row0, w.W2_t, kH, kH, Wbuf, col0);
#pragma unroll
  for (int i = 0; i < kEdgeRM; ++i)
#pragma unroll
    for (int j = 0; j < kEdgeCN; ++j) {
      A[(col0 + j) * kLdE + row0 + i] = (row0 + i < n_rows) ? gelu(acc[i][j] + w.b2[col0 + j], tbl) : 0.0F;
      acc[i][j] = 0.0F;
    }
  seq_gemm<kEdgeRM, kEdgeCN, kH, kKC>(acc, A, kLdE, row0, w.W3_t, kH, kH, Wbuf, col0);
#pragma unroll
  for (int i = 0; i < kEdgeRM; ++i)
    if (row0 + i < n_rows)
#pragma unroll
      for (int j = 0; j < kEdgeCN; ++j) msg[(slot0 + row0 + i) * kH + col0 + j] = acc[i][j] + w.b3[col0 + j];
}

// acc[j][r] += A[k][row0 + r] * Wt[k][c0 + j * CS] for k = k0 .. k0 + KB - 1 in
// order (A k-major with leading dimension lda, one rounding per product and
// per sum); w holds the KB weight rows of the thread's columns.
template <int KB, int CPT, int RPT>
__device__ inline void use_rows(const float (&w)[KB][CPT], const float* A, int lda, int row0, int k0,
                                float (&acc)[CPT][RPT]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int kk = 0; kk < KB; ++kk) {
    float a[RPT];
#pragma unroll
    for (int r = 0; r < RPT; ++r) a[r] = A[(k0 + kk) * lda + row0 + r];
#pragma unroll
    for (int j = 0; j < CPT; ++j)
#pragma unroll
      for (int r = 0; r < RPT; ++r) acc[j][r] = acc[j][r] + a[r] * w[kk][j];
  }
}

template <int KB, int N, int CPT, int CS>
__device__ inline void load_rows(float (&w)[KB][CPT], const float* __restrict__ Wt, int k0, int c0) {
#pragma unroll
  for (int kk = 0; kk < KB; ++kk)
#pragma unroll
    for (int j = 0; j < CPT; ++j) w[kk][j] = Wt[(size_t)(k0 + kk) * N + c0 + j * CS];
}

// Sequential-k product of a few rows with the thread's columns c0 + j * CS of
// Wt [K][N] (t-layout). Weights stream from global memory KB k-rows at a time
// with the next KB in flight while the current ones are used.
template <int K, int N, int CPT, int CS, int RPT, int KB>
__device__ inline void col_gemm(const float* __restrict__ Wt, const float* A, int lda, int row0, int c0,
                                float (&acc)[CPT][RPT]) {
  static_assert(K % (2 * KB) == 0, "k chunking");
  float wa[KB][CPT], wb[KB][CPT];
  load_rows<KB, N, CPT, CS>(wa, Wt, 0, c0);
  for (int k0 = 0; k0 < K; k0 += 2 * KB) {
    load_rows<KB, N, CPT, CS>(wb, Wt, k0 + KB, c0);
    use_rows<KB, CPT, RPT>(wa, A, lda, row0, k0, acc);
    if (k0 + 2 * KB < K) load_rows<KB, N, CPT, CS>(wa, Wt, k0 + 2 * KB, c0);
    use_rows<KB, CPT, RPT>(wb, A, lda, row0, k0 + KB, acc);
  }
}

// Node update for NR residues: LN1(h + upd), FFN, LN2, mask; then the W11
// prefix of this layer's edge update and (when Wnext_t is given) the next
// layer's W1 prefix. Every thread owns whole output columns, so each dot
// product runs over k in order. Each weight element read from L2 serves NR
// rows: few rows keep the grid wide when L is small, more rows cut the weight
// traffic when L is large.
template <int NR>
__global__ __launch_bounds__(256) void node_kernel(EncLayerDev w, const float* __restrict__ Wnext_t,
                                                   const float* __restrict__ msg, const int32_t* __restrict__ idx,
                                                   const float* __restrict__ mask, int L, int K,
                                                   float* __restrict__ h_v, float* __restrict__ prefix) {
#pragma clang fp contract(off)
  static_assert(NR % 2 == 0 && NR <= 16, "thread mapping");
  constexpr int NH = NR / 2;  // rows per thread in the column-per-thread phases
  constexpr int KB = NR <= 4 ? 32 : 64 / NR;  // weight rows in flight per half-step
  __shared__ __attribute__((aligned(16))) float X[kH * NR];   // k-major [d][row]
  __shared__ __attribute__((aligned(16))) float H1[kH * NR];
  __shared__ __attribute__((aligned(16))) float F[kFF * NR];
  __shared__ __attribute__((aligned(16))) float H2[kH * NR];
  __shared__ float tbl[17];
  if (threadIdx.x < 17) tbl[threadIdx.x] = kExpNegTable[threadIdx.x];
  const int r0 = blockIdx.x * NR;
  const int nr = min(NR, L - r0);
  const int t = threadIdx.x;

  // upd = sum over valid slots, in order, of (1/30) mask_i mask_j m_ij; then
  // X = h + upd (axpy order: 1 * residual + input). The weight of each
  // (row, slot) is computed once into LDS (0 for an invalid slot); thread t
  // owns column t % 128 of rows NH (t / 128) + q, q < NH, issues all of a
  // row's message loads at once and sums them in slot order.
  __shared__ float alpha_s[NR * kKmax];
  for (int i = t; i < NR * kKmax; i += blockDim.x) {
    const int row = i / kKmax, k = i % kKmax;
    float alpha = 0.0F;
    if (row < nr && k < K) {
      const int r = r0 + row;
      const int j = idx[(size_t)r * K + k];
      if (j >= 0 && j < L) {
        alpha = 1.0F / 30.0F;
        alpha *= mask[r] * mask[j];
      }
    }
    alpha_s[i] = alpha;
  }
  __syncthreads();
  {
    const int d = t % kH, rb = NH * (t / kH);
    for (int q = 0; q < NH; ++q) {
      const int row = rb + q;
      float v = 0.0F;
      if (row < nr) {
        const int r = r0 + row;
        float mv[kKmax];
#pragma unroll
        for (int k = 0; k < kKmax; ++k) mv[k] = k < K ? msg[((size_t)r * K + k) * kH + d] : 0.0F;
        float upd = 0.0F;
#pragma unroll
        for (int k = 0; k < kKmax; ++k) {
          const float alpha = alpha_s[row * kKmax + k];
          if (alpha == 0.0F) continue;  // also every invalid slot
          upd = alpha * mv[k] + upd;
        }
        v = h_v[(size_t)r * kH + d] + upd;
      }
      X[d * NR + row] = v;
    }
  }
  __syncthreads();
  // LayerNorms: Welford statistics of each row by one thread (the reference's
  // sequential recurrence), then every element normalised in parallel.
  __shared__ float ln_mean[NR], ln_inv[NR];
  if (t < NR) welford_stats_col(X + t, NR, ln_mean + t, ln_inv + t);
  __syncthreads();
  for (int i = t; i < NR * kH; i += blockDim.x) {
    const int row = i % NR, d = i / NR;
    H1[i] = (X[i] - ln_mean[row]) * ln_inv[row] * w.n1g[d] + w.n1b[d];
  }
  __syncthreads();
  {
    // W_in: columns t and t + 256 of all rows, then GELU
    float acc[2][NR] = {};
    col_gemm<kH, kFF, 2, 256, NR, KB>(w.Win_t, H1, NR, 0, t, acc);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < NR; ++r) F[(t + 256 * j) * NR + r] = gelu(acc[j][r] + w.bin[t + 256 * j], tbl);
  }
  __syncthreads();
  {
    // W_out: column t % 128 of rows NH (t / 128) + r, r < NH; X = h1 + (W_out f + b)
    const int c = t % kH, rr = NH * (t / kH);
    float acc[1][NH] = {};
    col_gemm<kFF, kH, 1, 0, NH, KB>(w.Wout_t, F, NR, rr, c, acc);
#pragma unroll
    for (int r = 0; r < NH; ++r) X[c * NR + rr + r] = H1[c * NR + rr + r] + (acc[0][r] + w.bout[c]);
  }
  __syncthreads();
  if (t < NR) welford_stats_col(X + t, NR, ln_mean + t, ln_inv + t);
  __syncthreads();
  for (int i = t; i < NR * kH; i += blockDim.x) {
    const int row = i % NR, d = i / NR;
    float v = (X[i] - ln_mean[row]) * ln_inv[row] * w.n2g[d] + w.n2b[d];
    v *= row < nr ? mask[r0 + row] : 0.0F;
    H2[i] = v;
  }
  __syncthreads();
  for (int i = t; i < nr * kH; i += blockDim.x) {
    const int row = i / kH, d = i % kH;
    h_v[(size_t)(r0 + row) * kH + d] = H2[d * NR + row];
  }
  // prefixes: [0,128) of W11 (threads 0..127) and of the next layer's W1 (128..255) over h'
  {
    const int part = t / kH, c = t % kH;
    const float* Wt = part == 0 ? w.W11_t : Wnext_t;
    if (Wt) {
      float acc[1][NR] = {};
      col_gemm<kH, kH, 1, 0, NR, KB>(Wt, H2, NR, 0, c, acc);
#pragma unroll
      for (int r = 0; r < NR; ++r)
        if (r < nr) prefix[(size_t)(r0 + r) * 256 + part * 128 + c] = acc[0][r];
    }
  }
}

__global__ __launch_bounds__(256) void edge_update_kernel(EncLayerDev w, float* __restrict__ h_e,
                                                          const float* __restrict__ h_v,
                                                          const int32_t* __restrict__ idx,
                                                          const float* __restrict__ prefix, int L, int K) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) float A[kH * kLdE];
  __shared__ __attribute__((aligned(16))) float Wbuf[2 * kKC * kH];
  __shared__ float tbl[17];
  if (threadIdx.x < 17) tbl[threadIdx.x] = kExpNegTable[threadIdx.x];
  const size_t S = (size_t)L * K;
  const size_t slot0 = (size_t)blockIdx.x * kRows;
  const int n_rows = (int)min((size_t)kRows, S - slot0);
  const int rg = threadIdx.x / 32, cg = threadIdx.x % 32;
  const int row0 = rg * kEdgeRM, col0 = cg * kEdgeCN;

  float acc[kEdgeRM][kEdgeCN];
#pragma unroll
  for (int i = 0; i < kEdgeRM; ++i) {
    const int row = row0 + i;
    const float* pre = row < n_rows ? prefix + ((slot0 + row) / K) * 256 : nullptr;
#pragma unroll
    for (int j = 0; j < kEdgeCN; ++j) acc[i][j] = pre ? pre[col0 + j] : 0.0F;
  }
  load_kmajor(A, kLdE, kRows, [&](int row) -> const float* {
    return row < n_rows ? h_e + (slot0 + row) * kH : nullptr;
  });
  seq_gemm<kEdgeRM, kEdgeCN, kH, kKC>(acc, A, kLdE, row0, w.W11_t + 128 * kH, kH, kH, Wbuf, col0);
  load_kmajor(A, kLdE, kRows, [&](int row) -> const float* {
    if (row >= n_rows) return nullptr;
    const int j = idx[slot0 + row];
    return (j >= 0 && j < L) ? h_v + (size_t)j * kH : nullptr;
  });
  seq_gemm<kEdgeRM, kEdgeCN, kH, kKC>(acc, A, kLdE, row0, w.W11_t + 256 * kH, kH, kH, Wbuf, col0);
#pragma unroll
  for (int i = 0; i < kEdgeRM; ++i)
#pragma unroll
    for (int j = 0; j < kEdgeCN; ++j) {
      A[(col0 + j) * kLdE + row0 + i] = (row0 + i < n_rows) ? gelu(acc[i][j] + w.b11[col0 + j], tbl) : 0.0F;
      acc[i][j] = 0.0F;
    }
  seq_gemm<kEdgeRM, kEdgeCN, kH, kKC>(acc, A, kLdE, row0, w.W12_t, kH, kH, Wbuf, col0);
#pragma unroll
  for (int i = 0; i < kEdgeRM; ++i)
#pragma unroll
    for (int j = 0; j < kEdgeCN; ++j) {
      A[(col0 + j) * kLdE + row0 + i] = (row0 + i < n_rows) ? gelu(acc[i][j] + w.b12[col0 + j], tbl) : 0.0F;
      acc[i][j] = 0.0F;
    }
  seq_gemm<kEdgeRM, kEdgeCN, kH, kKC>(acc, A, kLdE, row0, w.W13_t, kH, kH, Wbuf, col0);
  // x = 1 * e + m  (axpy order), then LN3 per valid row
#pragma unroll
  for (int i = 0; i < kEdgeRM; ++i)
#pragma unroll
    for (int j = 0; j < kEdgeCN; ++j) {
      const int row = row0 + i, c = col0 + j;
      A[c * kLdE + row] = (row < n_rows) ? h_e[(slot0 + row) * kH + c] + (acc[i][j] + w.b13[c]) : 0.0F;
    }
  __shared__ float ln_stat[2 * kRows];
  __shared__ int row_ok[kRows];
  if (threadIdx.x < kRows) {
    const int j = (int)threadIdx.x < n_rows ? idx[slot0 + threadIdx.x] : -1;
    row_ok[threadIdx.x] = j >= 0 && j < L;
  }
  ln_cols_block(A, A, kLdE, n_rows, w.n3g, w.n3b, ln_stat, [&](int r) { return row_ok[r] != 0; });
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

// Residues per node_kernel workgroup for a chain of L residues (2, 4, 8 or
// 16; HKBS_ENCODER_NODE_ROWS overrides). The arithmetic of every row is the
// same for all four, so the choice changes only the speed.
static int encoder_node_rows(int L) {
  if (const char* env = std::getenv("HKBS_ENCODER_NODE_ROWS")) {
    const int n = std::atoi(env);
    if (n == 2 || n == 4 || n == 8 || n == 16) return n;
  }
  return L >= 1500 ? 8 : 4;  // measured: 4 is fastest up to L = 1000, 8 from L = 2000
}

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
  const unsigned edge_tiles = (unsigned)(((size_t)L * K + kRows - 1) / kRows);
  const int node_rows = encoder_node_rows(L);
  const unsigned node_tiles = (unsigned)((L + node_rows - 1) / node_rows);
  for (int l = 0; l < kLayers; ++l) {
    edge_msg_kernel<<<edge_tiles, 256, 0, stream>>>(m.enc[l], h_e, h_v, idx, ws.prefix, L, K, ws.msg);
    const float* Wnext = l + 1 < kLayers ? m.enc[l + 1].W1_t : nullptr;
    if (node_rows == 16)
      node_kernel<16><<<node_tiles, 256, 0, stream>>>(m.enc[l], Wnext, ws.msg, idx, mask, L, K, h_v, ws.prefix);
    else if (node_rows == 8)
      node_kernel<8><<<node_tiles, 256, 0, stream>>>(m.enc[l], Wnext, ws.msg, idx, mask, L, K, h_v, ws.prefix);
    else if (node_rows == 4)
      node_kernel<4><<<node_tiles, 256, 0, stream>>>(m.enc[l], Wnext, ws.msg, idx, mask, L, K, h_v, ws.prefix);
    else
      node_kernel<2><<<node_tiles, 256, 0, stream>>>(m.enc[l], Wnext, ws.msg, idx, mask, L, K, h_v, ws.prefix);
    edge_update_kernel<<<edge_tiles, 256, 0, stream>>>(m.enc[l], h_e, h_v, idx, ws.prefix, L, K);
  }
  return hipGetLastError();
}

}  // namespace hkbs
