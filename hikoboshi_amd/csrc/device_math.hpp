// Device numerics shared by the kernels.
//
// fast_exp_neg and gelu restate the reference's approximations with the same
// operation order (cpp/include/hikoboshi/primitives/detail/fast_exp_neg.hpp:12-55,
// cpp/include/hikoboshi/primitives/compute/gelu.hpp:22-51) so that features
// and activations agree with the CPU path to float rounding.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "gelu_poly_table.hpp"

namespace hkbs {

typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __constant__ static const float kExpNegTable[17] = {
    1.0F,
    0.36787944117144232F,
    0.13533528323661270F,
    0.04978706836786394F,
    0.01831563888873418F,
    0.00673794699908547F,
    0.00247875217666636F,
    0.00091188196555452F,
    0.00033546262790251F,
    0.00012340980408668F,
    0.00004539992976248F,
    0.00001670170079024F,
    0.00000614421235333F,
    0.00000226032940698F,
    0.00000083152871910F,
    0.00000030590232050F,
    0.00000011253517471F,
};

// Table + degree-6 Taylor approximation of exp(x) on [-16, 0]; tbl holds the
// 17 values of kExpNegTable (an LDS copy in kernels that call it often: a
// per-lane index into __constant__ memory becomes a vector memory gather).
__device__ inline float fast_exp_neg(float x, const float* tbl = kExpNegTable) {
#pragma clang fp contract(off)
  if (x != x) return x;
  float neg_x = -x;
  if (neg_x > 16.0F) return 0.0F;
  if (neg_x < 0.0F) neg_x = 0.0F;
  int n = static_cast<int>(neg_x + 0.5F);
  if (n > 16) n = 16;
  const float r = -(neg_x - static_cast<float>(n));
  const float e =
      1.0F +
      r * (1.0F +
           r * (0.5F +
                r * (1.0F / 6.0F +
                     r * (1.0F / 24.0F + r * (1.0F / 120.0F + r * (1.0F / 720.0F))))));
  return tbl[n] * e;
}

// 1 / y for y in [1, 2.32] (the range of 1 + p v below), correctly rounded:
// the hardware reciprocal is within an ulp and one FMA Newton step rounds it
// to 1 / y (equal to IEEE division at every float of the range).
__device__ inline float recip_unit_range(float y) {
  const float r0 = __builtin_amdgcn_rcpf(y);
  const float e = __builtin_fmaf(-y, r0, 1.0F);
  return __builtin_fmaf(e, r0, r0);
}

// GELU with the Abramowitz-Stegun 7.1.26 erf used by the reference
// (gelu.hpp:22-51, fast_exp_neg.hpp:12-55): sign and magnitude of
// v = x / sqrt(2), erf = 1 - poly(t) exp(-v^2) with t = 1 / (1 + p v), exp by
// table and degree-6 Taylor, erf = sign for v > 4, GELU = 0.5 x (1 + erf),
// every operation rounded as in the reference. Evaluated without branches:
// for v <= 4 the exp argument v^2 lies in [0, 16], where fast_exp_neg's range
// checks do nothing; for v > 4 the value is selected away. The result equals
// the reference expression bit for bit for every float x (a GPU test compares
// all 2^32 inputs with the branching form).
__device__ inline float gelu(float x, const float* tbl = kExpNegTable) {  // tbl: as for fast_exp_neg
#pragma clang fp contract(off)
  const float vs = x * 0.7071067811865475F;
  const float v = fabsf(vs);
  const float t = recip_unit_range(1.0F + 0.3275911F * v);
  const float poly =
      (((((1.061405429F * t + -1.453152027F) * t) + 1.421413741F) * t + -0.284496736F) * t + 0.254829592F) * t;
  const float q = fminf(v * v, 16.0F);
  const int n = static_cast<int>(q + 0.5F);
  const float r = -(q - static_cast<float>(n));
  const float e =
      1.0F + r * (1.0F + r * (0.5F + r * (1.0F / 6.0F + r * (1.0F / 24.0F + r * (1.0F / 120.0F + r * (1.0F / 720.0F))))));
  const float mag = 1.0F - poly * (tbl[n] * e);
  const float erfv = __builtin_copysignf(v > 4.0F ? 1.0F : mag, vs);
  return 0.5F * x * (1.0F + erfv);
}

// The same GELU formula for code held to a tolerance rather than to bit
// identity (the 16-bit encoder's node kernel; the decode loop and the 16-bit
// edge kernels use gelu_poly below): the exp table is read from LDS (tbl = 17
// floats, kExpNegTable), 1/(1 + p v) is the hardware reciprocal (1 ulp) and
// contraction is allowed. No v > 4 case is needed: there q is clamped to 16
// and poly(t) exp(-16) < 2^-25, so mag rounds to exactly 1. The sign is copied
// from x (for x = -0 the result is -0 either way).
__device__ inline float gelu_fast(float x, const float* tbl) {
  const float v = fabsf(x) * 0.7071067811865475F;
  const float t = __builtin_amdgcn_rcpf(1.0F + 0.3275911F * v);
  const float poly =
      (((((1.061405429F * t + -1.453152027F) * t) + 1.421413741F) * t + -0.284496736F) * t + 0.254829592F) * t;
  const float q = fminf(v * v, 16.0F);
  const int n = static_cast<int>(q + 0.5F);
  const float r = static_cast<float>(n) - q;
  const float e =
      1.0F +
      r * (1.0F +
           r * (0.5F +
                r * (1.0F / 6.0F + r * (1.0F / 24.0F + r * (1.0F / 120.0F + r * (1.0F / 720.0F))))));
  const float ex = tbl[n];
  const float mag = 1.0F - poly * (ex * e);
  return 0.5F * x * (1.0F + __builtin_copysignf(mag, x));
}

// The decode loop's GELU with the A&S term P(v) (erf = 1 - P) taken from a
// per-segment polynomial instead of the reciprocal, the Horner in t and the
// exp Taylor polynomial (gelu_poly_gen.py fits the table to the reference
// expression, within 7.4e-8 absolute; the segments keep the reference's exp
// table breakpoints, and row 17, v >= sqrt(15.5), is zero since the
// reference's 1 - P rounds to 1 there). tab = the table in LDS as load_gelu_poly
// lays it out (16-byte aligned). The tail keeps the reference's rounding of
// mag = 1 - P and 0.5 x (1 + copysign(mag, x)). About 20 VALU slots against
// the 31 of gelu_fast. Over all 2^32 inputs it is closer to the reference
// expression than gelu_fast (5.1 against 7.5 units of ulp(result) + |x| 2^-25)
// and equal to it on infinities and NaN.
// LDS row stride of the table (floats): a lane reads the row of its own value,
// and 12 floats (48 bytes) put the rows of up to 8-16 distinct segments on
// distinct banks, where 8 floats let rows 4 or 8 apart share them.
constexpr int kGeluPolyStride = 12;
constexpr int kGeluPolyLds = kGeluPolyRows * kGeluPolyStride;  // floats of the LDS copy
// Copies the table into LDS rows of kGeluPolyStride floats (tab: kGeluPolyLds floats,
// 16-byte aligned); thread tid of n.
__device__ inline void load_gelu_poly(float* tab, int tid, int n) {
  for (int i = tid; i < kGeluPolyRows * 8; i += n) tab[(i / 8) * kGeluPolyStride + i % 8] = kGeluPoly[i];
}
__device__ inline float gelu_poly(float x, const float* tab) {
  // v > 4 takes row 17 (zero) as the reference's v > 4 case does; clamping v
  // rather than q keeps u finite for x = +-inf and NaN
  const float v = fminf(fabsf(x) * 0.7071067811865475F, 4.0F);
  const float q = v * v;
  const int row = static_cast<int>(q + 0.5F) + (v >= kGeluPolySplit ? 1 : 0);
  const float4 c0 = *reinterpret_cast<const float4*>(tab + kGeluPolyStride * row);
  const float4 c1 = *reinterpret_cast<const float4*>(tab + kGeluPolyStride * row + 4);
  const float u = v - c0.x;
  float p = c1.w * u + c1.z;
  p = p * u + c1.y;
  p = p * u + c1.x;
  p = p * u + c0.w;
  p = p * u + c0.z;
  p = p * u + c0.y;
  const float mag = 1.0F - p;
  return 0.5F * x * (1.0F + __builtin_copysignf(mag, x));
}

__device__ inline floatx4 mfma16(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// One wave computes an (16 MB) x (16 NB) tile of A . W^T with fp32 MFMA.
//   A : LDS, row-major with leading dimension lda (floats, multiple of 4).
//   Wp: kpack16 weights of a layer with N output columns.
//   n0: first output column of the wave's tile.
// acc[mb][nb][i] holds D[row = 16 mb + 4 (lane / 16) + i][col = n0 + 16 nb + lane % 16].
template <int MB, int NB>
__device__ inline void mfma_tile(const float* __restrict__ A, int lda,
                                 const float* __restrict__ Wp, int N, int n0, int kdim,
                                 floatx4 (&acc)[MB][NB]) {
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  for (int kb = 0; kb < kdim / 16; ++kb) {
    float4 a[MB];
    float4 b[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
      b[nb] = *reinterpret_cast<const float4*>(Wp + ((size_t)kb * N + n0 + nb * 16 + r) * 16 + 4 * g);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
      a[mb] = *reinterpret_cast<const float4*>(A + (mb * 16 + r) * lda + kb * 16 + 4 * g);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        acc[mb][nb] = mfma16(a[mb].x, b[nb].x, acc[mb][nb]);
        acc[mb][nb] = mfma16(a[mb].y, b[nb].y, acc[mb][nb]);
        acc[mb][nb] = mfma16(a[mb].z, b[nb].z, acc[mb][nb]);
        acc[mb][nb] = mfma16(a[mb].w, b[nb].w, acc[mb][nb]);
      }
  }
}

template <int MB, int NB>
__device__ inline void zero_acc(floatx4 (&acc)[MB][NB]) {
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = floatx4{0.F, 0.F, 0.F, 0.F};
}

// Writes an accumulator tile to LDS C (leading dimension ldc) at column n0.
template <int MB, int NB>
__device__ inline void store_acc(const floatx4 (&acc)[MB][NB], float* C, int ldc, int n0) {
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int i = 0; i < 4; ++i) C[(mb * 16 + 4 * g + i) * ldc + n0 + nb * 16 + r] = acc[mb][nb][i];
}

// ---------------------------------------------------------------------------
// Reference-order arithmetic.
//
// The reference's default linear layer accumulates every output element as
// one sequential float sum over k starting from 0.0f, each product rounded
// before the add (no FMA), then adds the bias
// (cpp/primitives/linalg/gemm_scalar_fast.cpp:107-176,249-314;
// cpp/include/hikoboshi/modules/mpnn/detail/mpnn_inner_inline.hpp:319-339).
// seq_gemm_mfma reproduces that rounding bit for bit with the products on the
// matrix cores: for each k, v_mfma_f32_16x16x1_4b_f32 forms the outer product
// of a column of A (16 rows) and a row of W (64 columns) with a zero addend,
// i.e. every product rounded once to fp32 as the VALU multiply rounds it, and
// the VALU adds it to the accumulators in k order, so each output is one
// sequential float sum of rounded products (one VALU add per product instead
// of a multiply and an add). The matrix cores flush products below 2^-126 to
// zero where the VALU keeps IEEE subnormals: such a term could change a sum
// only if all of the sum's terms were below about 2^-100. In the encoder every
// product has a weight of at least 3.7e-8 in magnitude or zero (the v_48_020
// package's smallest) and an input that is zero or at least about 1e-9 (GELU
// outputs, LayerNorm outputs, RBF features of at least exp(-16)), so no
// product is subnormal.
//   A   : LDS, k-major: A[k * lda + row].
//   W   : global, transposed weights W[k * ldw + col] (col < NC); kd (the rows
//         used) a multiple of 4.
//   Wbuf: LDS staging, 2 x KC x NC floats: chunk c + 1 of the weights is
//         loaded into registers while chunk c is used, then stored to the
//         other half.
// Every wave owns a 16 x 64 block of outputs at rows [rb, rb + 16), columns
// [cb, cb + 64); accumulator v of lane l is output row mfma_row(rb, v),
// column mfma_col(cb, v) (the instruction's lane layout on gfx950: block
// v / 4, row 4 (l / 16) + v % 4, column l % 16 of that block). The k loop runs
// in groups of four: a group's four products are issued before the next
// group's LDS operands are read, and both are in flight while the group's 64
// adds run. Every thread of the 256-thread block must call it (it contains
// barriers); it starts and ends with a barrier, so LDS writes made before the
// call are visible and A may be overwritten after it.
typedef float floatx16 __attribute__((ext_vector_type(16)));
__device__ inline int mfma_row(int rb, int v) { return rb + 4 * ((threadIdx.x & 63) >> 4) + (v & 3); }
__device__ inline int mfma_col(int cb, int v) { return cb + 16 * (v >> 2) + (threadIdx.x & 15); }

template <int NC, int KC>
__device__ inline void seq_gemm_mfma(float (&acc)[16], const float* A, int lda, int rb,
                                     const float* __restrict__ W, int ldw, int kd, float* Wbuf, int cb) {
#pragma clang fp contract(off)
  constexpr int kBlock = 256;
  constexpr int V = KC * (NC / 4);  // float4 per chunk
  constexpr int PT = (V + kBlock - 1) / kBlock;
  static_assert(NC % 64 == 0 && KC % 4 == 0, "64-column wave blocks, k groups of four");
  __builtin_assume(kd % 4 == 0 && kd > 0);
  const int lane = threadIdx.x & 63;
  float4 stage[PT];
  const int nchunks = (kd + KC - 1) / KC;
#pragma unroll
  for (int p = 0; p < PT; ++p) {
    const int i = threadIdx.x + p * kBlock;
    const int kk = i / (NC / 4), c4 = i % (NC / 4);
    stage[p] = make_float4(0.F, 0.F, 0.F, 0.F);
    if (i < V && kk < kd) stage[p] = *reinterpret_cast<const float4*>(W + (size_t)kk * ldw + 4 * c4);
  }
  __syncthreads();
#pragma unroll
  for (int p = 0; p < PT; ++p) {
    const int i = threadIdx.x + p * kBlock;
    if (i < V) *reinterpret_cast<float4*>(Wbuf + i * 4) = stage[p];
  }
  __syncthreads();
  const floatx16 zero = {};
  for (int c = 0; c < nchunks; ++c) {
    const int k0 = c * KC;
    const bool more = c + 1 < nchunks;
    if (more) {
#pragma unroll
      for (int p = 0; p < PT; ++p) {
        const int i = threadIdx.x + p * kBlock;
        const int kk = i / (NC / 4), c4 = i % (NC / 4);
        stage[p] = make_float4(0.F, 0.F, 0.F, 0.F);
        if (i < V && k0 + KC + kk < kd)
          stage[p] = *reinterpret_cast<const float4*>(W + (size_t)(k0 + KC + kk) * ldw + 4 * c4);
      }
    }
    const float* Wc = Wbuf + (c & 1) * (KC * NC);
    const int kn = (kd - k0) < KC ? (kd - k0) : KC;
    const float* ap = A + (size_t)k0 * lda + rb + (lane & 15);
    const float* wp = Wc + cb + lane;
    // kd is a multiple of 4 (every caller's), so every group of four k is whole
    float a[4], b[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      a[j] = ap[(size_t)j * lda];
      b[j] = wp[j * NC];
    }
#pragma unroll 1
    for (int kk = 0; kk < kn; kk += 4) {
      floatx16 p[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) p[j] = __builtin_amdgcn_mfma_f32_16x16x1f32(a[j], b[j], zero, 0, 0, 0);
      if (kk + 4 < kn) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          a[j] = ap[(size_t)(kk + 4 + j) * lda];
          b[j] = wp[(kk + 4 + j) * NC];
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[v] = acc[v] + p[j][v];
    }
    if (more) {
      float* Wn = Wbuf + ((c + 1) & 1) * (KC * NC);
#pragma unroll
      for (int p = 0; p < PT; ++p) {
        const int i = threadIdx.x + p * kBlock;
        if (i < V) *reinterpret_cast<float4*>(Wn + i * 4) = stage[p];
      }
    }
    __syncthreads();
  }
}

// Welford mean and 1 / sqrt(var + eps) of 128 values x[d * ld] (a k-major
// LDS column) in the reference's order
// (cpp/primitives/compute/layer_norm_scalar.cpp:8-40, eps 1e-5).
__device__ inline void welford_stats_col(const float* x, int ld, float* mean_out, float* inv_out) {
#pragma clang fp contract(off)
  float mean = 0.0F, m2 = 0.0F;
  for (int d = 0; d < 128; ++d) {
    const float v = x[d * ld];
    const float count = static_cast<float>(d + 1);
    const float delta = v - mean;
    mean += delta / count;
    const float delta2 = v - mean;
    m2 += delta * delta2;
  }
  const float var = m2 / 128.0F;
  *mean_out = mean;
  *inv_out = 1.0F / sqrtf(var + 1.0e-5F);
}

// LayerNorm of the rows r < rows of a column-major LDS tile (x[d * ld + r],
// d < 128) into out (may alias x), for rows with valid(r): thread r computes
// row r's Welford statistics (the reference's recurrence) into stat [2 *
// rows], then the whole block normalises the elements in parallel with the
// reference's per-element expression. Starts and ends with a barrier.
template <typename Valid>
__device__ inline void ln_cols_block(const float* x, float* out, int ld, int rows, const float* __restrict__ g,
                                     const float* __restrict__ b, float* stat, Valid valid) {
#pragma clang fp contract(off)
  __syncthreads();
  if ((int)threadIdx.x < rows && valid((int)threadIdx.x))
    welford_stats_col(x + threadIdx.x, ld, stat + threadIdx.x, stat + rows + threadIdx.x);
  __syncthreads();
  for (int i = threadIdx.x; i < rows * 128; i += blockDim.x) {
    const int r = i % rows, d = i / rows;
    if (!valid(r)) continue;
    out[d * ld + r] = (x[d * ld + r] - stat[r]) * stat[rows + r] * g[d] + b[d];
  }
  __syncthreads();
}

// Two-pass LayerNorm statistics of a 128-float row held as 2 floats per lane
// of one wave (lane holds elements lane and lane + 64). eps = 1e-5
// (cpp/include/hikoboshi/universal/detail/mpnn_d64_weights.hpp:27).
// Lane permutations within a row of 16 lanes on the DPP path (no LDS trip):
// 0xB1 = quad_perm [1,0,3,2], 0x4E = quad_perm [2,3,0,1], 0x141 =
// row_half_mirror, 0x140 = row_mirror.
template <int CTRL>
__device__ inline float dpp_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

__device__ inline float lane_f32(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Sum over the 64 lanes of a wave as a pairwise tree (lanes 2i and 2i + 1,
// then quads, 8s, rows of 16, then the four row sums as (r0 + r1) + (r2 +
// r3)); every lane gets the same bits.
__device__ inline float wave_sum(float v) {
  v += dpp_f32<0xB1>(v);
  v += dpp_f32<0x4E>(v);
  v += dpp_f32<0x141>(v);  // after the quads, mirroring within 8 lanes pairs quad 0 with quad 1
  v += dpp_f32<0x140>(v);  // and mirroring within 16 lanes pairs the two halves
  return (lane_f32(v, 0) + lane_f32(v, 16)) + (lane_f32(v, 32) + lane_f32(v, 48));
}

// Maximum over the 64 lanes of a wave (order does not matter for max).
__device__ inline float wave_max(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  v = fmaxf(v, dpp_f32<0x141>(v));
  v = fmaxf(v, dpp_f32<0x140>(v));
  return fmaxf(fmaxf(lane_f32(v, 0), lane_f32(v, 16)), fmaxf(lane_f32(v, 32), lane_f32(v, 48)));
}

// LayerNorm of a row held in registers (lane: elements lane and lane + 64).
__device__ inline void ln_regs_wave(float x0, float x1, const float* g, const float* b, float* out) {
  const int lane = threadIdx.x & 63;
  const float mean = wave_sum(x0 + x1) * (1.0F / 128.0F);
  const float d0 = x0 - mean, d1 = x1 - mean;
  const float var = wave_sum(d0 * d0 + d1 * d1) * (1.0F / 128.0F);
  const float inv = 1.0F / sqrtf(var + 1.0e-5F);
  out[lane] = d0 * inv * g[lane] + b[lane];
  out[lane + 64] = d1 * inv * g[lane + 64] + b[lane + 64];
}

__device__ inline void ln_row_wave(const float* in, const float* g, const float* b, float* out) {
  const int lane = threadIdx.x & 63;
  ln_regs_wave(in[lane], in[lane + 64], g, b, out);
}

}  // namespace hkbs
