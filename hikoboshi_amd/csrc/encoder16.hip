// Featurisation and encoder on the fp16 MFMA, for the 16-bit design modes.
//
// The layers are those of encoder.hip and features.hip (edge embedding
// inverse_fold_scalar.cpp:236-279; encoder layers
// proteinmpnn_encoder_scalar.cpp:169-333). Every product runs on the
// 16x16x32 fp16 MFMA with both operands split, v = hi + lo / 2048 (hi =
// fp16(v), lo = fp16((v - hi) * 2048)): hi.hi + (hi.lo + lo.hi) / 2048 in fp32
// carries about 22 significant bits, so the encoder is fp32-accurate (not
// the reference's rounding sequence, which encoder.hip reproduces). Features,
// biases, GELU (gelu_fast), LayerNorm (two-pass), residuals and the neighbour
// sum are fp32, and h_V, h_E are stored in fp32. The kNN graph comes from the
// exact fp32 kernel.
//
// A wave owns 16 rows of every product: its A operand is a 16-row fp32 slab
// of LDS, split into hi / lo fragments as it is read, and it produces all 128
// output columns as 8 MFMA tiles while the split weights stream from L2.
//
// The h_i block of W1 [h_i | e_ij | h_j] (and of W11) is the same for all K
// slots of residue i, so node16 computes it once per residue into a prefix
// buffer [L][256] (W11 part for this layer's edge update, W1 part for the
// next layer's messages; zero for layer 0, where h = 0) and the edge kernels
// run K = 256 over [e_ij | h_j], starting from the prefix.
//
// Kernels:
//   edge_embed16   32 edge slots per workgroup (2 waves): 416 features ->
//                  W_edge -> LN -> W_e -> h_E.
//   per layer:
//   edge_msg16     one residue per workgroup (3 waves = 48 slots):
//                  prefix + W1 [e_ij | h_j], GELU, W2, GELU, W3 -> the masked
//                  sum over the residue's slots / 30 -> upd[i].
//   node16         16 residues per workgroup (4 waves, a quarter of the FFN
//                  each): LN1(h + upd), the FFN on the MFMA, LN2, mask; then
//                  the W11 and next-layer W1 prefixes of the new h.
//   edge_update16  32 edge slots per workgroup (2 waves): prefix + W11
//                  [e_ij | h_j], GELU, W12, GELU, W13, residual, LN3 -> h_E
//                  (valid slots).
#include "device_math.hpp"
#include "edge_chunk.hpp"
#include "pmpnn_internal.hpp"

namespace hkbs {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kLdA = 2 * kH + 4;   // floats per slab row of [e_ij | h_j] (16-byte pad)
constexpr int kLdX = kEdgeIn + 4;  // floats per slab row of edge features
constexpr int kLdF = kFF + 4;      // floats per row of the FFN hidden layer
constexpr int kLdH = kH + 4;       // floats per row of a 128-wide activation
static_assert(kKmax == 48, "edge_msg16 covers a residue's slots with 3 waves of 16 rows");
static_assert(kEdgeIn % 32 == 0, "MFMA k-steps");

__device__ inline floatx4 mfma_f16(f16x8 a, f16x8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// acc[nt] = A[16 rows][K] . W[K][n0 + 16 nt + (0..15)] for nt < NT. A is the
// wave's fp32 slab (lda floats per row); Wp the split weights, hi as
// [K / 8][N][8] halves and lo at Wp + K * N (or Wp + lo_off when Wp starts
// inside a larger matrix). With lane = 16 g + r, acc[nt][i]
// is row 4 g + i, column n0 + 16 nt + r. The next k-step's weight fragments
// load while the current ones are used.
template <int NT>
__device__ inline void wave_gemm(const float* A, int lda, const uint16_t* __restrict__ Wp, int N, int n0, int K,
                                 floatx4 (&acc)[NT], size_t lo_off = 0) {
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const uint16_t* wh = Wp + ((size_t)g * N + n0 + r) * 8;
  const uint16_t* wl = wh + (lo_off ? lo_off : (size_t)K * N);
  const size_t kstep = (size_t)4 * N * 8;  // halves per 32 inputs
  floatx4 cor[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    acc[nt] = floatx4{0.F, 0.F, 0.F, 0.F};
    cor[nt] = acc[nt];
  }
  const int nkb = K / 32;
  f16x8 bh[NT], bl[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    bh[nt] = *reinterpret_cast<const f16x8*>(wh + (size_t)nt * 16 * 8);
    bl[nt] = *reinterpret_cast<const f16x8*>(wl + (size_t)nt * 16 * 8);
  }
  for (int kb = 0; kb < nkb; ++kb) {
    const int kn = kb + 1 < nkb ? kb + 1 : kb;
    f16x8 nh[NT], nl[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      nh[nt] = *reinterpret_cast<const f16x8*>(wh + (size_t)kn * kstep + (size_t)nt * 16 * 8);
      nl[nt] = *reinterpret_cast<const f16x8*>(wl + (size_t)kn * kstep + (size_t)nt * 16 * 8);
    }
    const float4* ap = reinterpret_cast<const float4*>(A + r * lda + 32 * kb + 8 * g);
    const float4 a0 = ap[0], a1 = ap[1];
    const float av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    f16x8 ah, al;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = __builtin_amdgcn_fmed3f(av[e], -65504.0F, 65504.0F);
      ah[e] = static_cast<_Float16>(v);
      al[e] = static_cast<_Float16>((av[e] - static_cast<float>(ah[e])) * 2048.0F);
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      acc[nt] = mfma_f16(ah, bh[nt], acc[nt]);
      cor[nt] = mfma_f16(ah, bl[nt], cor[nt]);
      cor[nt] = mfma_f16(al, bh[nt], cor[nt]);
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      bh[nt] = nh[nt];
      bl[nt] = nl[nt];
    }
  }
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[nt][i] += cor[nt][i] * (1.0F / 2048.0F);
}

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

// Sum over the 16 lanes that hold one row (lanes 16 g .. 16 g + 15).
__device__ inline float sum16(float v) {
  v += __shfl_xor(v, 1, 64);
  v += __shfl_xor(v, 2, 64);
  v += __shfl_xor(v, 4, 64);
  v += __shfl_xor(v, 8, 64);
  return v;
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

// The wave's 16 slab rows [h_e[slot] | h_v[j]] with slot = slot_of(row)
// (negative: a zero row) and j = idx[slot] (outside [0, L): a zero h_j
// block).
template <typename SlotOf>
__device__ inline void build_rows(float* A, const float* __restrict__ h_v, const float* __restrict__ h_e,
                                  const int32_t* __restrict__ idx, int L, int K, SlotOf slot_of) {
  const int lane = threadIdx.x & 63;
  for (int t = lane; t < 16 * 64; t += 64) {
    const int row = t / 64, c4 = t % 64, part = c4 / 32, col = 4 * (c4 % 32);
    const long long slot = slot_of(row);
    float4 v = make_float4(0.F, 0.F, 0.F, 0.F);
    if (slot >= 0) {
      if (part == 0) {
        v = *reinterpret_cast<const float4*>(h_e + (size_t)slot * kH + col);
      } else {
        const int j = idx[slot];
        if (j >= 0 && j < L) v = *reinterpret_cast<const float4*>(h_v + (size_t)j * kH + col);
      }
    }
    *reinterpret_cast<float4*>(A + row * kLdA + part * kH + col) = v;
  }
}

__global__ __launch_bounds__(128) void edge_embed16_kernel(ModelDev m, const float* __restrict__ coords,
                                                           const uint8_t* __restrict__ src,
                                                           const int32_t* __restrict__ resid,
                                                           const int32_t* __restrict__ chain,
                                                           const int32_t* __restrict__ idx, int L, int K,
                                                           float* __restrict__ h_e) {
  __shared__ __attribute__((aligned(16))) float slab[2][16 * kLdX];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const size_t S = (size_t)L * K;
  const size_t base = (size_t)blockIdx.x * 32 + 16 * wave;
  float* A = slab[wave];
  for (int t = lane; t < 16 * 26; t += 64) {
    const int row = t & 15, c = t >> 4;
    const size_t slot = base + row;
    const int j = slot < S ? idx[slot] : -1;
    const int res = slot < S ? static_cast<int>(slot / K) : 0;
    float out[16];
    edge_chunk(m, coords, src, resid, chain, L, res, j, c, out);  // zeros when j is not a residue
#pragma unroll
    for (int f = 0; f < 16; ++f) A[row * kLdX + 16 * c + f] = out[f];
  }
  __syncthreads();
  floatx4 acc[8];
  wave_gemm<8>(A, kLdX, m.enc16.Wedge, kH, 0, kEdgeIn, acc);
  ln_acc(acc, m.ne_g, m.ne_b);
  __syncthreads();
#pragma unroll
  for (int nt = 0; nt < 8; ++nt)
#pragma unroll
    for (int i = 0; i < 4; ++i) A[(4 * g + i) * kLdH + 16 * nt + r] = acc[nt][i];
  __syncthreads();
  wave_gemm<8>(A, kLdH, m.enc16.We, kH, 0, kH, acc);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const size_t slot = base + 4 * g + i;
    if (slot >= S) continue;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      const int col = 16 * nt + r;
      h_e[slot * kH + col] = acc[nt][i] + m.We_b[col];
    }
  }
}

// One residue per workgroup: wave w holds its slots 16 w .. 16 w + 15.
__global__ __launch_bounds__(192) void edge_msg16_kernel(EncLayerDev w, Enc16LayerDev w16,
                                                         const float* __restrict__ h_e, const float* __restrict__ h_v,
                                                         const int32_t* __restrict__ idx,
                                                         const float* __restrict__ mask,
                                                         const float* __restrict__ prefix, int L, int K,
                                                         float* __restrict__ upd) {
  __shared__ __attribute__((aligned(16))) float slab[3][16 * kLdA];
  __shared__ float tbl[17];
  __shared__ float part[3][kH];
  const int res = blockIdx.x;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  if (threadIdx.x < 17) tbl[threadIdx.x] = kExpNegTable[threadIdx.x];
  float* A = slab[wave];
  build_rows(A, h_v, h_e, idx, L, K, [&](int row) -> long long {
    const int k = 16 * wave + row;
    return k < K ? (long long)res * K + k : -1;
  });
  __syncthreads();
  floatx4 acc[8];
  // rows 128 .. 383 of W1 (packed k-blocks 16 ..) over [e_ij | h_j], plus the h_i prefix
  wave_gemm<8>(A, kLdA, w16.W1 + (size_t)16 * kH * 8, kH, 0, 2 * kH, acc, (size_t)3 * kH * kH);
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) {
    const float pv = prefix[(size_t)res * 256 + kH + 16 * nt + r];
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[nt][i] += pv;
  }
  __syncthreads();
  store_gelu<8>(acc, w.b1, 0, A, kLdH, tbl);
  __syncthreads();
  wave_gemm<8>(A, kLdH, w16.W2, kH, 0, kH, acc);
  __syncthreads();
  store_gelu<8>(acc, w.b2, 0, A, kLdH, tbl);
  __syncthreads();
  wave_gemm<8>(A, kLdH, w16.W3, kH, 0, kH, acc);
  // upd = sum over valid slots of (mask_i mask_j / 30) (W3 g + b3)
  float alpha[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int k = 16 * wave + 4 * g + i;
    alpha[i] = 0.0F;
    if (k < K) {
      const int j = idx[(size_t)res * K + k];
      if (j >= 0 && j < L) alpha[i] = mask[res] * mask[j] * (1.0F / 30.0F);
    }
  }
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) {
    const int col = 16 * nt + r;
    const float bv = w.b3[col];
    float s = 0.0F;
#pragma unroll
    for (int i = 0; i < 4; ++i) s += alpha[i] * (acc[nt][i] + bv);
    s += __shfl_xor(s, 16, 64);
    s += __shfl_xor(s, 32, 64);
    if (g == 0) part[wave][col] = s;
  }
  __syncthreads();
  if (threadIdx.x < kH)
    upd[(size_t)res * kH + threadIdx.x] = (part[0][threadIdx.x] + part[1][threadIdx.x]) + part[2][threadIdx.x];
}

// 16 residues per workgroup of four waves; lane (r, g) of a wave holds rows
// 4 g + i, columns 16 nt + r of a 128-wide block (the MFMA output layout).
// Wave 0 forms h1 = LN1(h + upd) for all 16 rows; wave w computes the FFN
// hidden columns [128 w, 128 w + 128) and the W_out partial sum over those
// inputs; wave 0 adds the four partials in order, the residual, LN2 and the
// mask.
__global__ __launch_bounds__(256) void node16_kernel(EncLayerDev w, Enc16LayerDev w16, const float* __restrict__ upd,
                                                     const float* __restrict__ mask, int L, float* __restrict__ h_v,
                                                     const uint16_t* __restrict__ W1_next, float* __restrict__ prefix) {
  __shared__ __attribute__((aligned(16))) float A[16 * kLdH];
  __shared__ __attribute__((aligned(16))) float F[16 * kLdF];
  __shared__ __attribute__((aligned(16))) float Pt[4][16 * kLdH];
  __shared__ float tbl[17];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const int r0 = blockIdx.x * 16;
  if (threadIdx.x < 17) tbl[threadIdx.x] = kExpNegTable[threadIdx.x];
  floatx4 x[8];
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int res = r0 + 4 * g + i;
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) {
        const size_t at = (size_t)res * kH + 16 * nt + r;
        x[nt][i] = res < L ? h_v[at] + upd[at] : 0.0F;
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
  // prefixes of the new h: wave 0 the h_i rows of this layer's W11, wave 1
  // those of the next layer's W1 (packed k-blocks 0 .. 15 of the K = 384
  // matrices; lo 384 x 128 halves after hi)
  if (wave >= 2 || (wave == 1 && !W1_next)) return;
  floatx4 pacc[8];
  wave_gemm<8>(A, kLdH, wave == 0 ? w16.W11 : W1_next, kH, 0, kH, pacc, (size_t)3 * kH * kH);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int res = r0 + 4 * g + i;
    if (res >= L) continue;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) prefix[(size_t)res * 256 + kH * wave + 16 * nt + r] = pacc[nt][i];
  }
}

__global__ __launch_bounds__(128) void edge_update16_kernel(EncLayerDev w, Enc16LayerDev w16, float* __restrict__ h_e,
                                                            const float* __restrict__ h_v,
                                                            const int32_t* __restrict__ idx,
                                                            const float* __restrict__ prefix, int L, int K) {
  __shared__ __attribute__((aligned(16))) float slab[2][16 * kLdA];
  __shared__ float tbl[17];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  if (threadIdx.x < 17) tbl[threadIdx.x] = kExpNegTable[threadIdx.x];
  const long long S = (long long)L * K;
  const long long base = (long long)blockIdx.x * 32 + 16 * wave;
  float* A = slab[wave];
  build_rows(A, h_v, h_e, idx, L, K, [&](int row) -> long long { return base + row < S ? base + row : -1; });
  __syncthreads();
  floatx4 acc[8];
  wave_gemm<8>(A, kLdA, w16.W11 + (size_t)16 * kH * 8, kH, 0, 2 * kH, acc, (size_t)3 * kH * kH);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const long long slot = base + 4 * g + i;
    const size_t res = slot < S ? (size_t)(slot / K) : 0;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) acc[nt][i] += prefix[res * 256 + 16 * nt + r];
  }
  __syncthreads();
  store_gelu<8>(acc, w.b11, 0, A, kLdH, tbl);
  __syncthreads();
  wave_gemm<8>(A, kLdH, w16.W12, kH, 0, kH, acc);
  __syncthreads();
  store_gelu<8>(acc, w.b12, 0, A, kLdH, tbl);
  __syncthreads();
  wave_gemm<8>(A, kLdH, w16.W13, kH, 0, kH, acc);
  // x = e + (W13 g + b13), LN3, written for slots with a valid neighbour
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const long long slot = base + 4 * g + i;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      const int col = 16 * nt + r;
      const float e = slot < S ? h_e[(size_t)slot * kH + col] : 0.0F;
      acc[nt][i] = e + (acc[nt][i] + w.b13[col]);
    }
  }
  ln_acc(acc, w.n3g, w.n3b);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const long long slot = base + 4 * g + i;
    if (slot >= S) continue;
    const int j = idx[slot];
    if (j < 0 || j >= L) continue;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) h_e[(size_t)slot * kH + 16 * nt + r] = acc[nt][i];
  }
}

}  // namespace

hipError_t launch_encoder16(const ModelDev& m, const float* coords, const uint8_t* atom_src, const int32_t* resid,
                            const int32_t* chain, const int32_t* idx, const float* mask, int L, int K, float* h_v,
                            float* h_e, const EncoderScratch& ws, hipStream_t stream) {
  if (L <= 0) return hipSuccess;
  if (K < 1 || K > kKmax) return hipErrorInvalidValue;
  const size_t S = (size_t)L * K;
  const unsigned tiles = (unsigned)((S + 31) / 32);
  hipError_t e = launch_zero(h_v, (size_t)L * kH, stream);
  if (e != hipSuccess) return e;
  edge_embed16_kernel<<<tiles, 128, 0, stream>>>(m, coords, atom_src, resid, chain, idx, L, K, h_e);
  e = launch_zero(ws.prefix, (size_t)L * 256, stream);  // layer 0: h = 0, so its W1 prefix is 0
  if (e != hipSuccess) return e;
  float* upd = ws.msg;  // [L][128] neighbour sums (the [S][128] message buffer is otherwise unused here)
  for (int l = 0; l < kLayers; ++l) {
    const Enc16LayerDev& w16 = m.enc16.layer[l];
    const uint16_t* W1_next = l + 1 < kLayers ? m.enc16.layer[l + 1].W1 : nullptr;
    edge_msg16_kernel<<<(unsigned)L, 192, 0, stream>>>(m.enc[l], w16, h_e, h_v, idx, mask, ws.prefix, L, K, upd);
    node16_kernel<<<(unsigned)((L + 15) / 16), 256, 0, stream>>>(m.enc[l], w16, upd, mask, L, h_v, W1_next,
                                                                ws.prefix);
    edge_update16_kernel<<<tiles, 128, 0, stream>>>(m.enc[l], w16, h_e, h_v, idx, ws.prefix, L, K);
  }
  return hipGetLastError();
}

}  // namespace hkbs
