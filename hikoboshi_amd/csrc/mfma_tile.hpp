// Split-operand fp16 MFMA tiles shared by the 16-bit encoder (encoder16.hip)
// and the decoder's layer-0 table (decoder.hip).
//
// A product carries fp32 accuracy on the fp16 MFMA by splitting both operands,
// v = hi + lo / 2048 with hi = fp16(v), lo = fp16((v - hi) 2048): the sum
// hi.hi + (hi.lo + lo.hi) / 2048, accumulated in fp32 by three 16x16x32 MFMAs,
// carries about 22 significant bits.
#pragma once

#include "device_math.hpp"
#include "pmpnn_internal.hpp"

namespace hkbs {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

__device__ inline floatx4 mfma_f16(f16x8 a, f16x8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Sum over the 16 lanes 16 g .. 16 g + 15 of a wave (a row of a wave_gemm
// output, or a column block of a tile_gemm output summed over its rows).
__device__ inline float sum16(float v) {
  v += __shfl_xor(v, 1, 64);
  v += __shfl_xor(v, 2, 64);
  v += __shfl_xor(v, 4, 64);
  v += __shfl_xor(v, 8, 64);
  return v;
}

// --------------------------------------------------------------- row blocks ----
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

// ------------------------------------------------------------ edge tiles ----
// A tile holds 16 RB edge rows. Its operands live in LDS split into fp16
// halves, hi [rows][ld] then lo [rows][ld] (v = hi + lo / 2048); a row stride
// of K + 8 halves steps 4 banks per row, so the 16-byte fragment reads of 8
// consecutive rows cover all banks once. Wave w produces output columns
// [32 w, 32 w + 32) as two 16-column MFMA tiles per row block, computed
// transposed (weights as the MFMA's A operand, rows as its B operand): lane
// (r, g) then holds row 16 rb + r, columns 32 w + 16 nt + 4 g + (0..3).
constexpr int kTileThreads = 256;
constexpr int kLdS1 = kH + 8;      // halves per row of a K = 128 operand

// Four consecutive floats into the split slab at (row, col).
__device__ inline void put_split4(_Float16* S, int rows, int ld, int row, int col, float4 v) {
  const float f[4] = {v.x, v.y, v.z, v.w};
  f16x4 h, l;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const _Float16 hi = static_cast<_Float16>(__builtin_amdgcn_fmed3f(f[e], -65504.0F, 65504.0F));
    h[e] = hi;
    l[e] = static_cast<_Float16>((f[e] - static_cast<float>(hi)) * 2048.0F);
  }
  *reinterpret_cast<f16x4*>(S + row * ld + col) = h;
  *reinterpret_cast<f16x4*>(S + (rows + row) * ld + col) = l;
}

// acc[rb][nt][i] = sum_k A[16 rb + r][k] W[n0 + 16 nt + 4 g + i][k] over K
// inputs (added to acc when accumulate), A the split slab (rows = 16 RB,
// stride ld), W (128 outputs) split as hi [K / 8][128][8] halves with lo at
// Wp + lo_off. Weight fragments stream through a ring of PF k-steps, so each
// load is issued PF - 1 k-steps before its use.
template <int RB, int K, int PF = 4>
__device__ inline void tile_gemm(const _Float16* S, int ld, const uint16_t* __restrict__ Wp, int n0, size_t lo_off,
                                 floatx4 (&acc)[RB][2], bool accumulate = false) {
  constexpr int NKB = K / 32;
  constexpr size_t kstep = (size_t)4 * kH * 8;  // halves per 32 inputs
  static_assert(K % 32 == 0 && PF >= 2, "k-steps");
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const _Float16* Sh = S + r * ld + 8 * g;
  const _Float16* Sl = Sh + 16 * RB * ld;
  const uint16_t* wh = Wp + ((size_t)g * kH + n0 + r) * 8;
  const uint16_t* wl = wh + lo_off;
  floatx4 cor[RB][2];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      cor[rb][nt] = floatx4{0.F, 0.F, 0.F, 0.F};
      if (!accumulate) acc[rb][nt] = cor[rb][nt];
    }
  f16x8 bh[PF][2], bl[PF][2];
#pragma unroll
  for (int kb = 0; kb < PF - 1 && kb < NKB; ++kb)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      bh[kb][nt] = *reinterpret_cast<const f16x8*>(wh + kb * kstep + (size_t)nt * 16 * 8);
      bl[kb][nt] = *reinterpret_cast<const f16x8*>(wl + kb * kstep + (size_t)nt * 16 * 8);
    }
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) {
    const int kn = kb + PF - 1;
    if (kn < NKB) {
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        bh[kn % PF][nt] = *reinterpret_cast<const f16x8*>(wh + kn * kstep + (size_t)nt * 16 * 8);
        bl[kn % PF][nt] = *reinterpret_cast<const f16x8*>(wl + kn * kstep + (size_t)nt * 16 * 8);
      }
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const f16x8 ah = *reinterpret_cast<const f16x8*>(Sh + 16 * rb * ld + 32 * kb);
      const f16x8 al = *reinterpret_cast<const f16x8*>(Sl + 16 * rb * ld + 32 * kb);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        acc[rb][nt] = mfma_f16(bh[kb % PF][nt], ah, acc[rb][nt]);
        cor[rb][nt] = mfma_f16(bh[kb % PF][nt], al, cor[rb][nt]);
        cor[rb][nt] = mfma_f16(bl[kb % PF][nt], ah, cor[rb][nt]);
      }
    }
  }
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[rb][nt][i] += cor[rb][nt][i] * (1.0F / 2048.0F);
}

}  // namespace hkbs
