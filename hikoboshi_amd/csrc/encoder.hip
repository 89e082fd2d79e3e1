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
// k-order sums of rounded products (seq_gemm_mfma), Welford LayerNorm, the same
// elementwise order. The only reuse is exact: the first 128 terms of the
// W1 / W11 sums ([h_i] part) are the same prefix for all K edges of residue
// i, so the node kernel computes that prefix once per residue and the edge
// kernels continue the sum with the e_ij and h_j terms.
//
// Kernels per layer:
//   edge_msg_kernel    tile of 32 edge rows: W1 (e, h_j terms), W2, W3 -> m_ij.
//   node_kernel        tile of 2 to 16 residues: the masked neighbour sum of
//                      m_ij in slot order, LN1, FFN, LN2, mask, and the W11
//                      and next-layer W1 prefixes, its weights streamed
//                      through a ring of register stages and LDS.
//   edge_update_kernel tile of 32 edge rows: W11, W12, W13, residual, LN3.
// Small tiles keep several workgroups on every CU; the weights stream through
// LDS in double-buffered chunks.
#include <cstdlib>
#include <utility>

#include "device_math.hpp"
#include "pmpnn_internal.hpp"

namespace hkbs {
namespace {

constexpr int kRows = 32;    // edge rows per tile (any rows of the [L * K] edge list)
constexpr int kLdE = 36;     // k-major leading dimension of edge tiles
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
// by node_kernel. The products run on the matrix cores (seq_gemm_mfma): wave w
// owns rows [16 (w % 2), + 16) and columns [64 (w / 2), + 64) of the tile.
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
  const int wave = threadIdx.x >> 6;
  const int rb = 16 * (wave & 1), cb = 64 * (wave >> 1);

  float acc[16];
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int row = mfma_row(rb, v);
    acc[v] = row < n_rows ? prefix[((slot0 + row) / K) * 256 + 128 + mfma_col(cb, v)] : 0.0F;
  }
  load_kmajor(A, kLdE, kRows, [&](int row) -> const float* {
    return row < n_rows ? h_e + (slot0 + row) * kH : nullptr;
  });
  seq_gemm_mfma<kH, kKC>(acc, A, kLdE, rb, w.W1_t + 128 * kH, kH, kH, Wbuf, cb);
  load_kmajor(A, kLdE, kRows, [&](int row) -> const float* {
    if (row >= n_rows) return nullptr;
    const int j = idx[slot0 + row];
    return (j >= 0 && j < L) ? h_v + (size_t)j * kH : nullptr;
  });
  seq_gemm_mfma<kH, kKC>(acc, A, kLdE, rb, w.W1_t + 256 * kH, kH, kH, Wbuf, cb);
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int row = mfma_row(rb, v), c = mfma_col(cb, v);
    A[c * kLdE + row] = row < n_rows ? gelu(acc[v] + w.b1[c], tbl) : 0.0F;
    acc[v] = 0.0F;
  }
  seq_gemm_mfma<kH, kKC>(acc, A, kLdE, rb, w.W2_t, kH, kH, Wbuf, cb);
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int row = mfma_row(rb, v), c = mfma_col(cb, v);
    A[c * kLdE + row] = row < n_rows ? gelu(acc[v] + w.b2[c], tbl) : 0.0F;
    acc[v] = 0.0F;
  }
  seq_gemm_mfma<kH, kKC>(acc, A, kLdE, rb, w.W3_t, kH, kH, Wbuf, cb);
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int row = mfma_row(rb, v), c = mfma_col(cb, v);
    if (row < n_rows) msg[(slot0 + row) * kH + c] = acc[v] + w.b3[c];
  }
}

// The weights of the node update stream through the workgroup as 40 chunks
// of 4096 floats (16 KB), in the order they are used:
//   chunks  0..15  W_in rows 8 c .. 8 c + 7, all 512 columns;
//   chunks 16..31  W_out rows 32 (c - 16) .. + 31, all 128 columns;
//   chunks 32..39  rows 16 (c - 32) .. + 15 of the h_i block (first 128
//                  rows) of W11, then the same rows of the next layer's W1.
// Each chunk is contiguous in memory (two 8 KB halves for chunks 32..39) and
// lands in LDS in the same order, so thread t loads 16-byte vectors t and
// t + 512 from a workgroup-uniform base. Chunk c is loaded kNodeDepth chunks
// before it is used, so 128 KB are in flight while earlier chunks are
// multiplied: the node update is a few short dependency chains per thread,
// and without deep prefetch it waits on every weight row. Two waves per SIMD
// hide the LDS latency of one another's chains.
constexpr int kNodeThreads = 512;
constexpr int kNodeChunks = 40;
constexpr int kNodeDepth = 8;
constexpr int kNodePT = 4096 / 4 / kNodeThreads;  // 16-byte vectors per thread per chunk

__device__ __forceinline__ void node_chunk_load(floatx4 (&dst)[kNodePT], const EncLayerDev& w,
                                                const float* __restrict__ Wn, int c) {
  static_assert(kNodePT == 2, "chunk mapping");
  const int t = threadIdx.x;
  if (c < 32) {
    const floatx4* base = reinterpret_cast<const floatx4*>(c < 16 ? w.Win_t + (size_t)4096 * c
                                                                  : w.Wout_t + (size_t)4096 * (c - 16));
    dst[0] = base[t];
    dst[1] = base[t + kNodeThreads];
  } else {
    dst[0] = reinterpret_cast<const floatx4*>(w.W11_t + (size_t)2048 * (c - 32))[t];
    dst[1] = reinterpret_cast<const floatx4*>(Wn + (size_t)2048 * (c - 32))[t];
  }
}

// One step of the chunk ring (S = ring slot = c % kNodeDepth, compile-time so
// that the ring stays in registers): chunk c to LDS half c & 1, barrier,
// refill the slot with chunk c + kNodeDepth, then use(chunk in LDS, c). The
// LDS half that chunk c overwrites was last read while using chunk c - 2,
// which every thread finished before the barrier of chunk c - 1.
template <int S, typename Use>
__device__ __forceinline__ void node_step(floatx4 (&ring)[kNodeDepth][kNodePT], float* Wl, const EncLayerDev& w,
                                          const float* __restrict__ Wn, int c, Use& use) {
  float* buf = Wl + (S & 1) * 4096;
#pragma unroll
  for (int p = 0; p < kNodePT; ++p) reinterpret_cast<floatx4*>(buf)[threadIdx.x + kNodeThreads * p] = ring[S][p];
  __syncthreads();
  if (c + kNodeDepth < kNodeChunks) node_chunk_load(ring[S], w, Wn, c + kNodeDepth);
  use(static_cast<const float*>(buf), c);
}

template <typename Use, int... S>
__device__ __forceinline__ void node_steps(floatx4 (&ring)[kNodeDepth][kNodePT], float* Wl, const EncLayerDev& w,
                                           const float* __restrict__ Wn, int cb, Use& use,
                                           std::integer_sequence<int, S...>) {
  (node_step<S>(ring, Wl, w, Wn, cb + S, use), ...);
}

// Uses chunks [c_begin, c_end) (multiples of kNodeDepth) in order.
template <typename Use>
__device__ __forceinline__ void node_run(floatx4 (&ring)[kNodeDepth][kNodePT], float* Wl, const EncLayerDev& w,
                                         const float* __restrict__ Wn, int c_begin, int c_end, Use&& use) {
  for (int cb = c_begin; cb < c_end; cb += kNodeDepth)
    node_steps(ring, Wl, w, Wn, cb, use, std::make_integer_sequence<int, kNodeDepth>{});
}

template <int... S>
__device__ __forceinline__ void node_fill(floatx4 (&ring)[kNodeDepth][kNodePT], const EncLayerDev& w,
                                          const float* __restrict__ Wn, std::integer_sequence<int, S...>) {
  (node_chunk_load(ring[S], w, Wn, S), ...);
}

// Node update for NR residues: LN1(h + upd), FFN, LN2, mask; then the W11
// prefix of this layer's edge update and (when Wnext_t is given) the next
// layer's W1 prefix. Every thread owns whole output columns, so each dot
// product runs over k in order with one rounding per product and per sum.
// Each weight element read serves NR rows: few rows keep the grid wide when
// L is small, more rows cut the weight traffic when L is large.
template <int NR>
__global__ __launch_bounds__(kNodeThreads) void node_kernel(EncLayerDev w, const float* __restrict__ Wnext_t,
                                                            const float* __restrict__ msg,
                                                            const int32_t* __restrict__ idx,
                                                            const float* __restrict__ mask, int L, int K,
                                                            float* __restrict__ h_v, float* __restrict__ prefix) {
#pragma clang fp contract(off)
  static_assert(NR % 2 == 0 && NR <= 16, "thread mapping");
  static_assert(kNodeThreads == kFF && kNodeThreads == 4 * kH, "one W_in column and bias per thread; four row groups");
  static_assert(kNodeChunks % kNodeDepth == 0 && 16 % kNodeDepth == 0, "phases start on a ring boundary");
  constexpr int RQ = NR >= 4 ? NR / 4 : 1;  // rows per thread in the message sum and W_out (4 row groups)
  constexpr int RP = NR / 2;                // rows per thread in the prefix products (2 row groups)
  __shared__ __attribute__((aligned(16))) float X[kH * NR];   // k-major [d][row]
  __shared__ __attribute__((aligned(16))) float H1[kH * NR];
  __shared__ __attribute__((aligned(16))) float F[kFF * NR];
  __shared__ __attribute__((aligned(16))) float H2[kH * NR];
  __shared__ __attribute__((aligned(16))) float Wl[2 * 4096];
  // bias and LayerNorm vectors: bin [512], bout, n1g, n1b, n2g, n2b [128 each]
  __shared__ float par[kFF + 5 * kH];
  __shared__ float alpha_s[NR * kKmax];
  __shared__ float mask_s[NR];
  __shared__ float tbl[17];
  const int r0 = blockIdx.x * NR;
  const int nr = min(NR, L - r0);
  const int t = threadIdx.x;
  const float* Wn = Wnext_t ? Wnext_t : w.W11_t;  // loaded either way; its prefix is stored only if given

  floatx4 ring[kNodeDepth][kNodePT];
  node_fill(ring, w, Wn, std::make_integer_sequence<int, kNodeDepth>{});

  if (t < 17) tbl[t] = kExpNegTable[t];
  par[t] = w.bin[t];
  if (t < kH) {
    par[kFF + t] = w.bout[t];
    par[kFF + kH + t] = w.n1g[t];
    par[kFF + 2 * kH + t] = w.n1b[t];
    par[kFF + 3 * kH + t] = w.n2g[t];
    par[kFF + 4 * kH + t] = w.n2b[t];
  }
  if (t < NR) mask_s[t] = t < nr ? mask[r0 + t] : 0.0F;
  // upd = sum over valid slots, in order, of (1/30) mask_i mask_j m_ij; then
  // X = h + upd (axpy order: 1 * residual + input). The weight of each
  // (row, slot) is computed once into LDS (0 for an invalid slot); thread t
  // owns column t % 128 of rows RQ (t / 128) + q, q < RQ, issues all of a
  // row's message loads at once and sums them in slot order.
  for (int i = t; i < NR * kKmax; i += kNodeThreads) {
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
    const int d = t % kH, rb = RQ * (t / kH);
    for (int q = 0; q < RQ; ++q) {
      const int row = rb + q;
      if (row >= NR) break;
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
  for (int i = t; i < NR * kH; i += kNodeThreads) {
    const int row = i % NR, d = i / NR;
    H1[i] = (X[i] - ln_mean[row]) * ln_inv[row] * par[kFF + kH + d] + par[kFF + 2 * kH + d];
  }
  // (the barrier of the first chunk orders these writes before their use)
  {
    // W_in: column t of all rows, then GELU into F
    float acc[NR] = {};
    node_run(ring, Wl, w, Wn, 0, 16, [&](const float* Wc, int c) {
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const int k = 8 * c + kk;
        const float wv = Wc[kk * kFF + t];
#pragma unroll
        for (int r = 0; r < NR; ++r) acc[r] = acc[r] + H1[k * NR + r] * wv;
      }
    });
#pragma unroll
    for (int r = 0; r < NR; ++r) F[t * NR + r] = gelu(acc[r] + par[t], tbl);
  }
  {
    // W_out: column t % 128 of rows RQ (t / 128) + r, r < RQ; X = h1 + (W_out f + b).
    // Row groups past NR (NR = 2) have no rows: those waves only stream.
    const int c = t % kH, rr = RQ * (t / kH);
    const bool active = rr < NR;
    float acc[RQ] = {};
    node_run(ring, Wl, w, Wn, 16, 32, [&](const float* Wc, int ch) {
      if (!active) return;
#pragma unroll 8
      for (int kk = 0; kk < 32; ++kk) {
        const int k = 32 * (ch - 16) + kk;
        const float wv = Wc[kk * kH + c];
#pragma unroll
        for (int r = 0; r < RQ; ++r) acc[r] = acc[r] + F[k * NR + rr + r] * wv;
      }
    });
    if (active) {
#pragma unroll
      for (int r = 0; r < RQ; ++r) X[c * NR + rr + r] = H1[c * NR + rr + r] + (acc[r] + par[kFF + c]);
    }
  }
  __syncthreads();
  if (t < NR) welford_stats_col(X + t, NR, ln_mean + t, ln_inv + t);
  __syncthreads();
  for (int i = t; i < NR * kH; i += kNodeThreads) {
    const int row = i % NR, d = i / NR;
    float v = (X[i] - ln_mean[row]) * ln_inv[row] * par[kFF + 3 * kH + d] + par[kFF + 4 * kH + d];
    v *= mask_s[row];
    H2[i] = v;
  }
  __syncthreads();
  for (int i = t; i < nr * kH; i += kNodeThreads) {
    const int row = i / kH, d = i % kH;
    h_v[(size_t)(r0 + row) * kH + d] = H2[d * NR + row];
  }
  // prefixes over h': column q = t % 256 of [W11 h-block | next layer's W1 h-block]
  // (q < 128: W11), rows RP (t / 256) + r, r < RP
  {
    const int q = t % 256, part = q / kH, c = q % kH, rr = RP * (t / 256);
    float acc[RP] = {};
    node_run(ring, Wl, w, Wn, 32, kNodeChunks, [&](const float* Wc, int ch) {
#pragma unroll
      for (int kk = 0; kk < 16; ++kk) {
        const int k = 16 * (ch - 32) + kk;
        const float wv = Wc[part * 2048 + kk * kH + c];
#pragma unroll
        for (int r = 0; r < RP; ++r) acc[r] = acc[r] + H2[k * NR + rr + r] * wv;
      }
    });
    // the sums are complete here: without this the compiler sinks each row's
    // products into its conditional store below and holds every operand
#pragma unroll
    for (int r = 0; r < RP; ++r) asm volatile("" : "+v"(acc[r]));
    if (part == 0 || Wnext_t) {
#pragma unroll
      for (int r = 0; r < RP; ++r)
        if (rr + r < nr) prefix[(size_t)(r0 + rr + r) * 256 + part * 128 + c] = acc[r];
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
  const int wave = threadIdx.x >> 6;
  const int rb = 16 * (wave & 1), cb = 64 * (wave >> 1);  // this wave's block (seq_gemm_mfma)

  float acc[16];
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int row = mfma_row(rb, v);
    acc[v] = row < n_rows ? prefix[((slot0 + row) / K) * 256 + mfma_col(cb, v)] : 0.0F;
  }
  load_kmajor(A, kLdE, kRows, [&](int row) -> const float* {
    return row < n_rows ? h_e + (slot0 + row) * kH : nullptr;
  });
  seq_gemm_mfma<kH, kKC>(acc, A, kLdE, rb, w.W11_t + 128 * kH, kH, kH, Wbuf, cb);
  load_kmajor(A, kLdE, kRows, [&](int row) -> const float* {
    if (row >= n_rows) return nullptr;
    const int j = idx[slot0 + row];
    return (j >= 0 && j < L) ? h_v + (size_t)j * kH : nullptr;
  });
  seq_gemm_mfma<kH, kKC>(acc, A, kLdE, rb, w.W11_t + 256 * kH, kH, kH, Wbuf, cb);
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int row = mfma_row(rb, v), c = mfma_col(cb, v);
    A[c * kLdE + row] = row < n_rows ? gelu(acc[v] + w.b11[c], tbl) : 0.0F;
    acc[v] = 0.0F;
  }
  seq_gemm_mfma<kH, kKC>(acc, A, kLdE, rb, w.W12_t, kH, kH, Wbuf, cb);
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int row = mfma_row(rb, v), c = mfma_col(cb, v);
    A[c * kLdE + row] = row < n_rows ? gelu(acc[v] + w.b12[c], tbl) : 0.0F;
    acc[v] = 0.0F;
  }
  seq_gemm_mfma<kH, kKC>(acc, A, kLdE, rb, w.W13_t, kH, kH, Wbuf, cb);
  // x = 1 * e + m  (axpy order), then LN3 per valid row
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int row = mfma_row(rb, v), c = mfma_col(cb, v);
    A[c * kLdE + row] = (row < n_rows) ? h_e[(slot0 + row) * kH + c] + (acc[v] + w.b13[c]) : 0.0F;
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
  // measured on single chains: 2 rows are fastest at L = 300, 4 at L = 1000,
  // 8 from L = 2000 (16 is within noise of 8 at L = 4000)
  if (L < 700) return 2;
  return L < 1500 ? 4 : 8;
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
      node_kernel<16><<<node_tiles, kNodeThreads, 0, stream>>>(m.enc[l], Wnext, ws.msg, idx, mask, L, K, h_v, ws.prefix);
    else if (node_rows == 8)
      node_kernel<8><<<node_tiles, kNodeThreads, 0, stream>>>(m.enc[l], Wnext, ws.msg, idx, mask, L, K, h_v, ws.prefix);
    else if (node_rows == 4)
      node_kernel<4><<<node_tiles, kNodeThreads, 0, stream>>>(m.enc[l], Wnext, ws.msg, idx, mask, L, K, h_v, ws.prefix);
    else
      node_kernel<2><<<node_tiles, kNodeThreads, 0, stream>>>(m.enc[l], Wnext, ws.msg, idx, mask, L, K, h_v, ws.prefix);
    edge_update_kernel<<<edge_tiles, 256, 0, stream>>>(m.enc[l], h_e, h_v, idx, ws.prefix, L, K);
  }
  return hipGetLastError();
}

}  // namespace hkbs
