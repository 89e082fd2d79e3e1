// Edge features of one 16-feature chunk of an edge slot, shared by the
// fp32 and the 16-bit edge embeddings (features.hip, encoder16.hip). The
// float operations of rbf_chunk follow the reference order with contraction
// disabled; rbf_chunk_fma is the 16-bit encoder's shorter form.
#pragma once

#include "device_math.hpp"
#include "pmpnn_internal.hpp"

namespace hkbs {

__device__ __constant__ static const int8_t kPairQ[25] = {1, 0, 2, 3, 4, 1, 1, 1, 1, 0, 0, 0, 4,
                                                          4, 3, 0, 2, 3, 4, 2, 3, 4, 2, 3, 2};
__device__ __constant__ static const int8_t kPairN[25] = {1, 0, 2, 3, 4, 0, 2, 3, 4, 2, 3, 4, 2,
                                                          3, 2, 1, 1, 1, 1, 0, 0, 0, 4, 4, 3};

// The 16 positional features of class cls (chain break: kPosClasses - 1).
__device__ inline void positional_chunk(const ModelDev& m, int cls, float* out) {
#pragma clang fp contract(off)
#pragma unroll
  for (int d = 0; d < 16; ++d) out[d] = m.pos_w[d * kPosClasses + cls] + m.pos_b[d];
}

// Positional class of edge (r, j): kPosClasses - 1 across chains, else the
// residue-index offset clamped to [-32, 32], shifted by 32.
__device__ inline int positional_class(const int32_t* __restrict__ resid, const int32_t* __restrict__ chain, int r,
                                       int j) {
  const int ci = chain ? chain[r] : 0;
  const int cj = chain ? chain[j] : 0;
  if (ci != cj) return kPosClasses - 1;
  int off = (resid ? resid[r] : r) - (resid ? resid[j] : j);
  off = off < -32 ? -32 : (off > 32 ? 32 : off);
  return off + 32;
}

// The 16 RBF features of the distance between atoms at qx and nx (3 floats
// each), in the reference's operation order; tbl is the exp table
// (kExpNegTable or a copy of it in LDS).
__device__ inline void rbf_chunk(const float* qx, const float* nx, float* out, const float* tbl) {
#pragma clang fp contract(off)
  float sq = 0.0F;
#pragma unroll
  for (int ax = 0; ax < 3; ++ax) {
    const float delta = nx[ax] - qx[ax];
    sq += delta * delta;
  }
  sq = sq + 1.0e-6F;
  const float dist = sqrtf(sq);
  const float center_step = (22.0F - 2.0F) / static_cast<float>(kRbf - 1);
  const float sigma = (22.0F - 2.0F) / (static_cast<float>(kRbf) / 0.7071067811865475F);
  const float two_sigma_sq = 2.0F * sigma * sigma;
#pragma unroll
  for (int f = 0; f < 16; ++f) {
    const float center = 2.0F + static_cast<float>(f) * center_step;
    const float delta = dist - center;
    out[f] = fast_exp_neg(-(delta * delta) / two_sigma_sq, tbl);
  }
}

// The 16 RBF features of rbf_chunk in fewer operations, for the 16-bit
// encoder (fp32-accurate, not the reference's rounding sequence): the same
// distance, centres, width and exp form (table value times the degree-6
// Taylor series of exp(r), |r| <= 1/2), with fused multiply-adds, a multiplication by
// 1 / (2 sigma^2) in place of the division, and no checks for inputs that
// cannot occur (the argument is never NaN or positive). A feature differs
// from rbf_chunk's by a few float ulps, or, where t lies within rounding of a
// half-integer and the two take neighbouring table entries, by up to the
// difference of the Taylor remainders at r = +1/2 and -1/2 (3.4e-6 of the
// value).
__device__ inline void rbf_chunk_fma(const float* qx, const float* nx, float* out, const float* tbl) {
#pragma clang fp contract(off)
  float sq = 0.0F;  // the distance as rbf_chunk rounds it: the far features are sensitive to its last bits
#pragma unroll
  for (int ax = 0; ax < 3; ++ax) {
    const float delta = nx[ax] - qx[ax];
    sq += delta * delta;
  }
  const float dist = sqrtf(sq + 1.0e-6F);
  const float center_step = (22.0F - 2.0F) / static_cast<float>(kRbf - 1);
  const float sigma = (22.0F - 2.0F) / (static_cast<float>(kRbf) / 0.7071067811865475F);
  const float inv_two_sigma_sq = 1.0F / (2.0F * sigma * sigma);
#pragma unroll
  for (int f = 0; f < 16; ++f) {
    const float center = 2.0F + static_cast<float>(f) * center_step;
    const float delta = dist - center;
    const float t = delta * delta * inv_two_sigma_sq;  // exp(-t), t >= 0
    const int n = static_cast<int>(fminf(t, 16.0F) + 0.5F);  // nearest integer, at most 16
    const float r = static_cast<float>(n) - t;
    float e = __builtin_fmaf(r, 1.0F / 720.0F, 1.0F / 120.0F);
    e = __builtin_fmaf(r, e, 1.0F / 24.0F);
    e = __builtin_fmaf(r, e, 1.0F / 6.0F);
    e = __builtin_fmaf(r, e, 0.5F);
    e = __builtin_fmaf(r, e, 1.0F);
    e = __builtin_fmaf(r, e, 1.0F);
    out[f] = t > 16.0F ? 0.0F : tbl[n] * e;
  }
}

// Writes the 16 features of chunk c (0 = positional, 1..25 = atom pair c-1)
// of edge slot (r, j) to out[0..16); tbl as for rbf_chunk.
__device__ inline void edge_chunk(const ModelDev& m, const float* __restrict__ coords,
                                  const uint8_t* __restrict__ src, const int32_t* __restrict__ resid,
                                  const int32_t* __restrict__ chain, int L, int r, int j, int c,
                                  float* out, const float* tbl = kExpNegTable) {
  if (j < 0 || j >= L) {
#pragma unroll
    for (int f = 0; f < 16; ++f) out[f] = 0.0F;
    return;
  }
  if (c == 0) {
    positional_chunk(m, positional_class(resid, chain, r, j), out);
    return;
  }
  const int p = c - 1;
  const int qa = kPairQ[p], na = kPairN[p];
  if (src[(size_t)r * 5 + qa] == 0 || src[(size_t)j * 5 + na] == 0) {
#pragma unroll
    for (int f = 0; f < 16; ++f) out[f] = 0.0F;
    return;
  }
  rbf_chunk(coords + ((size_t)r * 5 + qa) * 3, coords + ((size_t)j * 5 + na) * 3, out, tbl);
}

}  // namespace hkbs
