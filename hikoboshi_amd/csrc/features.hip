// Edge featurisation and edge embedding.
//
// Features per edge slot (residue r, neighbour j = idx[r,k]):
//   [0,16)    positional one-hot linear: W_pos[d, class] + b_pos[d],
//             class = 65 across chains, else clamp(res_r - res_j, +-32) + 32
//             (cpp/modules/mpnn/edge_rbf_features_scalar.cpp:45-76);
//   [16,416)  for each of the 25 atom pairs (query atom of r, neighbour atom
//             of j; cpp/primitives/compute/atom_pair_distance_scalar.cpp:21-72)
//             16 Gaussian RBFs of D = sqrt(sum (n - q)^2 + 1e-6) with centres
//             2 + f * 20/15 and 2 sigma^2 from sigma = 20 / (16 / 0.70710678)
//             (rbf_scalar.cpp:10-35, edge_rbf_features_scalar.cpp:135-137);
//             zero when either atom is missing; the whole row is zero for an
//             invalid neighbour. Float operations follow the reference order
//             with contraction disabled, so features are bit-identical to
//             the CPU path.
// Edge embedding (inverse_fold_scalar.cpp:236-279):
//   h_E = W_e . LayerNorm(W_edge . f) + b_e  (W_edge has no bias),
// fused in one kernel: a 32-slot tile of features is built in LDS (k-major),
// multiplied by W_edge, normalised and multiplied by W_e without leaving the
// CU, all in the reference's rounding order (h_E is bit-identical).
#include "device_math.hpp"
#include "edge_chunk.hpp"
#include "pmpnn_internal.hpp"

namespace hkbs {
namespace {

__global__ __launch_bounds__(256) void edge_features_kernel(ModelDev m, const float* __restrict__ coords,
                                                            const uint8_t* __restrict__ src,
                                                            const int32_t* __restrict__ resid,
                                                            const int32_t* __restrict__ chain,
                                                            const int32_t* __restrict__ idx, int L, int K,
                                                            float* __restrict__ features) {
  const size_t task = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t S = (size_t)L * K;
  if (task >= S * 26) return;
  const size_t slot = task / 26;
  const int c = static_cast<int>(task % 26);
  const int r = static_cast<int>(slot / K);
  float out[16];
  edge_chunk(m, coords, src, resid, chain, L, r, idx[slot], c, out);
  float* dst = features + slot * kEdgeIn + c * 16;
#pragma unroll
  for (int f = 0; f < 16; ++f) dst[f] = out[f];
}

constexpr int kTile = 32;  // edge slots per workgroup
constexpr int kLdT = 36;   // k-major leading dimension

// h_E = W_e . LN(W_edge . f) + b_e in the reference's rounding order
// (sequential sums without FMA, Welford LayerNorm). The 416 features of the
// tile are built in groups of kGroupChunks 16-feature chunks (one chunk of one
// slot per thread) and each group is consumed by the next k-range of the
// W_edge product, so one 128-row LDS tile serves features, the W_edge output
// and the LayerNorm output, and three workgroups fit on a CU.
constexpr int kGroupChunks = 8;
__global__ __launch_bounds__(256) void edge_embed_kernel(ModelDev m, const float* __restrict__ coords,
                                                         const uint8_t* __restrict__ src,
                                                         const int32_t* __restrict__ resid,
                                                         const int32_t* __restrict__ chain,
                                                         const int32_t* __restrict__ idx, int L, int K,
                                                         float* __restrict__ h_e) {
#pragma clang fp contract(off)
  static_assert(kGroupChunks * 16 <= kH && kGroupChunks * kTile == 256, "tile sizes");
  __shared__ __attribute__((aligned(16))) float A[kH * kLdT];
  __shared__ __attribute__((aligned(16))) float Wbuf[2 * 32 * kH];
  __shared__ float tbl[17];
  if (threadIdx.x < 17) tbl[threadIdx.x] = kExpNegTable[threadIdx.x];
  __syncthreads();
  const size_t S = (size_t)L * K;
  const size_t slot0 = (size_t)blockIdx.x * kTile;
  const int wave = threadIdx.x >> 6;
  const int rb = 16 * (wave & 1), cb = 64 * (wave >> 1);  // this wave's block (seq_gemm_mfma)
  const int frow = threadIdx.x % kTile, fchunk = threadIdx.x / kTile;
  const size_t fslot = slot0 + frow;
  const int fr = fslot < S ? static_cast<int>(fslot / K) : 0;
  const int fj = fslot < S ? idx[fslot] : -1;

  float acc[16];
#pragma unroll
  for (int v = 0; v < 16; ++v) acc[v] = 0.0F;
  for (int c0 = 0; c0 < 26; c0 += kGroupChunks) {
    const int nc = min(kGroupChunks, 26 - c0);
    // A is free here: seq_gemm_mfma ends with a barrier
    if (fchunk < nc) {
      float out[16];
      edge_chunk(m, coords, src, resid, chain, L, fr, fj, c0 + fchunk, out, tbl);  // zeros when fj is not a residue
#pragma unroll
      for (int f = 0; f < 16; ++f) A[(fchunk * 16 + f) * kLdT + frow] = out[f];
    }
    seq_gemm_mfma<kH, 32>(acc, A, kLdT, rb, m.edge_t + (size_t)c0 * 16 * kH, kH, nc * 16, Wbuf, cb);
  }
  float* X = A;
#pragma unroll
  for (int v = 0; v < 16; ++v) X[mfma_col(cb, v) * kLdT + mfma_row(rb, v)] = acc[v];
  __shared__ float ln_stat[2 * kTile];
  ln_cols_block(X, A, kLdT, kTile, m.ne_g, m.ne_b, ln_stat, [](int) { return true; });
#pragma unroll
  for (int v = 0; v < 16; ++v) acc[v] = 0.0F;
  seq_gemm_mfma<kH, 32>(acc, A, kLdT, rb, m.We_t, kH, kH, Wbuf, cb);
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const size_t slot = slot0 + mfma_row(rb, v);
    const int c = mfma_col(cb, v);
    if (slot < S) h_e[slot * kH + c] = acc[v] + m.We_b[c];
  }
}

}  // namespace

hipError_t launch_edge_features(const ModelDev& m, const float* coords, const uint8_t* atom_src,
                                const int32_t* resid, const int32_t* chain, const int32_t* idx, int L, int K,
                                float* features, hipStream_t stream) {
  const size_t tasks = (size_t)L * K * 26;
  if (tasks == 0) return hipSuccess;
  edge_features_kernel<<<(unsigned)((tasks + 255) / 256), 256, 0, stream>>>(m, coords, atom_src, resid, chain,
                                                                           idx, L, K, features);
  return hipGetLastError();
}

hipError_t launch_edge_embed(const ModelDev& m, const float* coords, const uint8_t* atom_src,
                             const int32_t* resid, const int32_t* chain, const int32_t* idx, int L, int K,
                             float* h_e, hipStream_t stream) {
  const size_t S = (size_t)L * K;
  if (S == 0) return hipSuccess;
  edge_embed_kernel<<<(unsigned)((S + kTile - 1) / kTile), 256, 0, stream>>>(m, coords, atom_src, resid, chain,
                                                                            idx, L, K, h_e);
  return hipGetLastError();
}

}  // namespace hkbs
