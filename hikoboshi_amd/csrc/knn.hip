// CA k-nearest-neighbour graph (bit-exact with the reference).
//
// Reference semantics (cpp/primitives/compute/knn_scalar.cpp:46-168, called
// with include_self and the residue validity mask by
// cpp/modules/mpnn/inverse_fold_scalar.cpp:181-234):
//   d(q,t) = ((dx*dx + dy*dy) + dz*dz) + 1e-6, dx = q - t, no FMA;
//   row_max = max(1e-6, max over valid t of d) (skipped for invalid q);
//   invalid q or t -> d = row_max;
//   strict-< insertion into a K-slot list initialised to +inf, so the list
//   is the K smallest finite d in (d, t) lexicographic order; slots never
//   filled keep index -1 and distance row_max.
// Because every finite d is a positive float, the key (bits(d) << 32) | t
// orders candidates exactly like that insertion. One wave owns one query
// row: it streams the candidates 64 at a time, bitonic-sorts each chunk in
// registers and merges it into a running sorted top-64.
#include "device_math.hpp"
#include "pmpnn_internal.hpp"

namespace hkbs {
namespace {

__device__ inline uint64_t shfl_xor_u64(uint64_t v, int mask) {
  const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), mask, 64);
  const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), mask, 64);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

__device__ inline uint64_t shfl_u64(uint64_t v, int src) {
  const uint32_t lo = __shfl(static_cast<uint32_t>(v), src, 64);
  const uint32_t hi = __shfl(static_cast<uint32_t>(v >> 32), src, 64);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// Sorts one key per lane across the wave; ascending when asc.
__device__ inline uint64_t bitonic_sort64(uint64_t key, bool asc) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int k = 2; k <= 64; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      const uint64_t p = shfl_xor_u64(key, j);
      const bool up = ((lane & k) == 0) == asc;
      const bool lower = (lane & j) == 0;
      key = (lower == up) ? (key < p ? key : p) : (key < p ? p : key);
    }
  }
  return key;
}

// Bitonic sequence -> ascending.
__device__ inline uint64_t bitonic_clean64(uint64_t key) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 32; j > 0; j >>= 1) {
    const uint64_t p = shfl_xor_u64(key, j);
    const bool lower = (lane & j) == 0;
    key = lower ? (key < p ? key : p) : (key < p ? p : key);
  }
  return key;
}

__device__ inline float knn_d2(float4 a, float4 b) {
#pragma clang fp contract(off)
  const float dx = a.x - b.x;
  const float dy = a.y - b.y;
  const float dz = a.z - b.z;
  return dx * dx + dy * dy + dz * dz + 1.0e-6F;
}

// Residue mask (N, CA, C, O present; inverse_fold_scalar.cpp:82-88,181-193)
// and compact CA coordinates (zero when CA is missing, :195-209); w = validity.
__global__ void prep_ca_kernel(const float* __restrict__ coords, const uint8_t* __restrict__ src, int L,
                               float4* __restrict__ ca, float* __restrict__ mask) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= L) return;
  const uint8_t* s = src + (size_t)r * 5;
  const bool valid = s[0] != 0 && s[1] != 0 && s[2] != 0 && s[3] != 0;
  const bool ca_present = s[1] != 0;
  const float* c = coords + ((size_t)r * 5 + 1) * 3;
  ca[r] = ca_present ? make_float4(c[0], c[1], c[2], valid ? 1.F : 0.F)
                     : make_float4(0.F, 0.F, 0.F, valid ? 1.F : 0.F);
  mask[r] = valid ? 1.0F : 0.0F;
}

// Rows of a ragged batch (seg != null) only see the residues of their own
// protein, [offsets[seg[q]], offsets[seg[q] + 1]); indices stay global.
__global__ __launch_bounds__(256) void knn_kernel(const float4* __restrict__ ca, int L, int K,
                                                  const int32_t* __restrict__ seg, const int64_t* __restrict__ offsets,
                                                  int32_t* __restrict__ idx, float* __restrict__ d2) {
  const int lane = threadIdx.x & 63;
  const int q = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (q >= L) return;  // whole wave exits together; no block barriers below
  int lo = 0, hi = L;
  if (seg) {
    lo = static_cast<int>(offsets[seg[q]]);
    hi = static_cast<int>(offsets[seg[q] + 1]);
  }
  const float4 qc = ca[q];
  const bool qvalid = qc.w != 0.F;

  float row_max = 1.0e-6F;
  if (qvalid) {
    for (int t = lo + lane; t < hi; t += 64) {
      const float4 tc = ca[t];
      if (tc.w == 0.F) continue;
      const float c = knn_d2(qc, tc);
      if (c > row_max) row_max = c;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const float o = __shfl_xor(row_max, off, 64);
      row_max = (o > row_max) ? o : row_max;
    }
  }

  const uint64_t kNone = ~0ull;
  uint64_t best = kNone;  // lane i: i-th smallest key so far
  for (int base = lo; base < hi; base += 64) {
    const int t = base + lane;
    uint64_t key = kNone;
    if (t < hi) {
      const float4 tc = ca[t];
      const float d = (qvalid && tc.w != 0.F) ? knn_d2(qc, tc) : row_max;
      if (d < __builtin_inff()) key = (static_cast<uint64_t>(__float_as_uint(d)) << 32) | static_cast<uint32_t>(t);
    }
    const uint64_t thresh = shfl_u64(best, K - 1);
    if (!__any(key < thresh)) continue;
    key = bitonic_sort64(key, false);
    best = bitonic_clean64(best < key ? best : key);
  }
  if (lane < K) {
    const size_t o = (size_t)q * K + lane;
    if (best == kNone) {
      idx[o] = -1;
      d2[o] = row_max;
    } else {
      idx[o] = static_cast<int32_t>(best & 0xffffffffu);
      d2[o] = __uint_as_float(static_cast<uint32_t>(best >> 32));
    }
  }
}

}  // namespace

hipError_t launch_knn(const float* coords, const uint8_t* atom_src, int L, int K, int32_t* idx, float* d2,
                      float* mask, float4* ca_scratch, hipStream_t stream, const int32_t* seg,
                      const int64_t* offsets) {
  if (L <= 0) return hipSuccess;
  prep_ca_kernel<<<(L + 255) / 256, 256, 0, stream>>>(coords, atom_src, L, ca_scratch, mask);
  knn_kernel<<<(L + 3) / 4, 256, 0, stream>>>(ca_scratch, L, K, seg, offsets, idx, d2);
  return hipGetLastError();
}

}  // namespace hkbs
