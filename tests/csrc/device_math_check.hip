// Exhaustive GPU check of the device GELUs in hikoboshi_amd/csrc/device_math.hpp
// against their straightforward forms, over all 2^32 float bit patterns.
//
//   gelu      (encoder, bit-exact path) vs gelu_branching: the reference's
//             expression as written in cpp/include/hikoboshi/primitives/compute/gelu.hpp:22-51
//             with fast_exp_neg (cpp/include/hikoboshi/primitives/detail/fast_exp_neg.hpp:12-55),
//             IEEE division and every range check taken as a branch;
//   gelu_fast (earlier decode loop) vs gelu_fast_select: the same formula with
//             the hardware reciprocal, the v > 4 case as a select and the sign
//             by comparison (the form gelu_fast replaced).
// Those results must agree bit for bit (any NaN equals any NaN). The decode
// loop's gelu_poly (the A&S term from per-segment polynomials) is measured
// against gelu: on non-finite inputs it must agree bit for bit; on finite
// inputs the largest |gelu_poly - gelu| in units of
//   ulp(gelu(x)) + |x| 2^-25  (one ulp of the result plus half an x-scaled step
//                              of the float grid under 1 that mag = 1 - P is
//                              rounded to)
// is reported, with the same figure for gelu_fast for comparison. A further
// kernel checks seq_gemm_mfma (the encoder's reference-order sums with the
// products on the matrix cores) against the same sums formed on the VALU, bit
// for bit. Test infrastructure only: built into tests/libdevice_math_check.so
// and called by tests/test_gpu_device_math.py.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../hikoboshi_amd/csrc/device_math.hpp"
#include "../../hikoboshi_amd/csrc/edge_chunk.hpp"

namespace {

using hkbs::kExpNegTable;

__device__ float fast_exp_neg_branching(float x) {
#pragma clang fp contract(off)
  if (x != x) return x;
  float neg_x = -x;
  if (neg_x > 16.0F) return 0.0F;
  if (neg_x < 0.0F) neg_x = 0.0F;
  int n = static_cast<int>(neg_x + 0.5F);
  if (n > 16) n = 16;
  const float r = -(neg_x - static_cast<float>(n));
  const float e =
      1.0F + r * (1.0F + r * (0.5F + r * (1.0F / 6.0F + r * (1.0F / 24.0F + r * (1.0F / 120.0F + r * (1.0F / 720.0F))))));
  return kExpNegTable[n] * e;
}

__device__ float gelu_branching(float x) {
#pragma clang fp contract(off)
  float v = x * 0.7071067811865475F;
  float sign = 1.0F;
  if (v < 0.0F) {
    sign = -1.0F;
    v = -v;
  }
  float erfv;
  if (v > 4.0F) {
    erfv = sign;
  } else {
    const float t = 1.0F / (1.0F + 0.3275911F * v);
    const float poly =
        (((((1.061405429F * t + -1.453152027F) * t) + 1.421413741F) * t + -0.284496736F) * t + 0.254829592F) * t;
    erfv = sign * (1.0F - poly * fast_exp_neg_branching(-(v * v)));
  }
  return 0.5F * x * (1.0F + erfv);
}

__device__ float gelu_fast_select(float x, const float* tbl) {
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
  float erfv = v > 4.0F ? 1.0F : mag;
  erfv = x < 0.0F ? -erfv : erfv;
  return 0.5F * x * (1.0F + erfv);
}

__device__ inline bool same_bits(float a, float b) {
  return (a != a && b != b) || __float_as_uint(a) == __float_as_uint(b);
}

// |a - b| in units of ulp(b) + |x| 2^-25 (b finite).
__device__ inline float dev_units(float a, float b, float x) {
  const float ab = fabsf(b);
  const float ulp = __uint_as_float(__float_as_uint(ab) + 1u) - ab;
  const float unit = fmaxf(ulp, 1.4e-45F) + fabsf(x) * 2.98023224e-08F;
  return fabsf(a - b) / unit;
}

// counts[0], first[0]: gelu; counts[1], first[1]: gelu_fast; counts[2],
// first[2]: gelu_poly on non-finite inputs (first = smallest mismatching bit
// pattern, 0xFFFFFFFF if none). worst[0], worst[1]: largest deviation units
// (float bits) of gelu_poly and gelu_fast against gelu on finite inputs;
// worst[2]: the input of worst[0].
__global__ void check_kernel(unsigned long long* counts, unsigned int* first, unsigned int* worst) {
  __shared__ float tbl[17];
  __shared__ __attribute__((aligned(16))) float gtab[hkbs::kGeluPolyLds];
  if (threadIdx.x < 17) tbl[threadIdx.x] = kExpNegTable[threadIdx.x];
  hkbs::load_gelu_poly(gtab, threadIdx.x, blockDim.x);
  __syncthreads();
  float w_poly = 0.0F, w_fast = 0.0F;
  unsigned int w_at = 0xFFFFFFFFu;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t bits = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; bits < (1ull << 32); bits += stride) {
    const float x = __uint_as_float(static_cast<unsigned int>(bits));
    if (!same_bits(hkbs::gelu(x), gelu_branching(x))) {
      atomicAdd(&counts[0], 1ull);
      atomicMin(&first[0], static_cast<unsigned int>(bits));
    }
    const float fast = hkbs::gelu_fast(x, tbl);
    if (!same_bits(fast, gelu_fast_select(x, tbl))) {
      atomicAdd(&counts[1], 1ull);
      atomicMin(&first[1], static_cast<unsigned int>(bits));
    }
    const float ref = hkbs::gelu(x);
    const float poly = hkbs::gelu_poly(x, gtab);
    if (!isfinite(x)) {
      if (!same_bits(poly, ref)) {
        atomicAdd(&counts[2], 1ull);
        atomicMin(&first[2], static_cast<unsigned int>(bits));
      }
    } else if (isfinite(ref)) {
      const float d = dev_units(poly, ref, x);
      if (!(d <= w_poly)) {  // also catches a NaN result
        w_poly = d != d ? 3.0e38F : d;
        w_at = static_cast<unsigned int>(bits);
      }
      const float df = dev_units(fast, ref, x);
      w_fast = fmaxf(w_fast, df != df ? 3.0e38F : df);
    }
  }
  const unsigned int prev = atomicMax(&worst[0], __float_as_uint(w_poly));
  if (__float_as_uint(w_poly) > prev) atomicExch(&worst[2], w_at);
  atomicMax(&worst[1], __float_as_uint(w_fast));
}

}  // namespace

// Runs the check on the current device; writes 3 counts, 3 first mismatches
// and worst[3] (see check_kernel). Returns the HIP status of the run.
extern "C" int hkbs_check_device_gelu(unsigned long long* counts_out, unsigned int* first_out,
                                      unsigned int* worst_out) {
  unsigned long long* counts = nullptr;
  unsigned int* first = nullptr;
  unsigned int* worst = nullptr;
  hipError_t e = hipMalloc(&counts, 3 * sizeof(unsigned long long));
  if (e == hipSuccess) e = hipMalloc(&first, 3 * sizeof(unsigned int));
  if (e == hipSuccess) e = hipMalloc(&worst, 3 * sizeof(unsigned int));
  if (e == hipSuccess) e = hipMemset(counts, 0, 3 * sizeof(unsigned long long));
  if (e == hipSuccess) e = hipMemset(first, 0xFF, 3 * sizeof(unsigned int));
  if (e == hipSuccess) e = hipMemset(worst, 0, 3 * sizeof(unsigned int));
  if (e == hipSuccess) {
    check_kernel<<<8192, 256>>>(counts, first, worst);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e == hipSuccess) e = hipMemcpy(counts_out, counts, 3 * sizeof(unsigned long long), hipMemcpyDeviceToHost);
  if (e == hipSuccess) e = hipMemcpy(first_out, first, 3 * sizeof(unsigned int), hipMemcpyDeviceToHost);
  if (e == hipSuccess) e = hipMemcpy(worst_out, worst, 3 * sizeof(unsigned int), hipMemcpyDeviceToHost);
  if (counts) (void)hipFree(counts);
  if (first) (void)hipFree(first);
  if (worst) (void)hipFree(worst);
  return static_cast<int>(e);
}

namespace {

// rbf_chunk_fma (16-bit encoder) against rbf_chunk (the reference's operation
// order) for n atom-pair offsets: offset i has length 30 i / n Angstrom along
// a direction that turns with i. out[0] = the largest |fma - ref| / ref over
// features with ref >= 1e-30 (float bits), out[1] = the largest |fma - ref|
// (float bits), out[2] = the number of features where exactly one of the two
// is zero (the exp(-16) cut-off).
__global__ void rbf_kernel(unsigned int n, unsigned int* out) {
  __shared__ float tbl[17];
  if (threadIdx.x < 17) tbl[threadIdx.x] = kExpNegTable[threadIdx.x];
  __syncthreads();
  float w_rel = 0.0F, w_abs = 0.0F;
  unsigned int cut = 0;
  for (unsigned int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    const float len = 30.0F * static_cast<float>(i) / static_cast<float>(n);
    const float a = 0.6180339F * static_cast<float>(i % 4096), b = 0.4142135F * static_cast<float>(i % 2048);
    const float q[3] = {1.25F, -3.5F, 7.0F};
    const float nx[3] = {q[0] + len * cosf(a) * sinf(b), q[1] + len * sinf(a) * sinf(b), q[2] + len * cosf(b)};
    float ref[16], fma[16];
    hkbs::rbf_chunk(q, nx, ref, tbl);
    hkbs::rbf_chunk_fma(q, nx, fma, tbl);
#pragma unroll
    for (int f = 0; f < 16; ++f) {
      const float d = fabsf(fma[f] - ref[f]);
      w_abs = fmaxf(w_abs, d != d ? 3.0e38F : d);
      if ((ref[f] == 0.0F) != (fma[f] == 0.0F)) ++cut;
      else if (ref[f] >= 1.0e-30F) w_rel = fmaxf(w_rel, d / ref[f]);
    }
  }
  atomicMax(&out[0], __float_as_uint(w_rel));
  atomicMax(&out[1], __float_as_uint(w_abs));
  atomicAdd(&out[2], cut);
}

// seq_gemm_mfma against the reference's sequential sums on the VALU (a product
// rounded, then added, k in order, starting from the initial accumulator): one
// 32 x 128 output tile with kd = 128 per workgroup, random operands from a
// counter hash. Operand magnitudes span 2^-40 .. 2^12 (A) and 2^-30 .. 2^2 (W)
// with random signs and about 1/16 exact zeros, so every product is a normal
// float or zero, as in the encoder; the initial accumulators are random too.
// out[0] counts outputs whose bits differ, out[1..3] = the first one's block,
// row * 128 + col and (MFMA bits) for the report.
__device__ inline uint32_t mix32(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return static_cast<uint32_t>(x ^ (x >> 31));
}
__device__ inline float rand_operand(uint64_t key, int lo_exp, int span) {
  const uint32_t r = mix32(key);
  if ((r & 15u) == 0u) return 0.0F;
  const uint32_t e = static_cast<uint32_t>(127 + lo_exp + (int)((r >> 4) % (uint32_t)span));
  return __uint_as_float(((r >> 31) << 31) | (e << 23) | (mix32(key ^ 0x5555ull) & 0x7FFFFFu));
}
constexpr int kGemmLd = 36;
__global__ __launch_bounds__(256) void seq_gemm_check_kernel(float* __restrict__ W, unsigned int* out) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) float A[128 * kGemmLd];
  __shared__ __attribute__((aligned(16))) float Wbuf[2 * 32 * 128];
  const uint64_t base = static_cast<uint64_t>(blockIdx.x) << 32;
  float* Wb = W + static_cast<size_t>(blockIdx.x) * 128 * 128;
  for (int i = threadIdx.x; i < 128 * 32; i += 256) A[(i / 32) * kGemmLd + i % 32] = rand_operand(base + i, -40, 52);
  for (int i = threadIdx.x; i < 128 * 128; i += 256) Wb[i] = rand_operand(base + 0x10000 + i, -30, 32);
  __threadfence();
  __syncthreads();
  const int wave = threadIdx.x >> 6;
  const int rb = 16 * (wave & 1), cb = 64 * (wave >> 1);
  float acc[16], ref[16];
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    acc[v] = rand_operand(base + 0x20000 + hkbs::mfma_row(rb, v) * 128 + hkbs::mfma_col(cb, v), -10, 14);
    ref[v] = acc[v];
  }
  hkbs::seq_gemm_mfma<128, 32>(acc, A, kGemmLd, rb, Wb, 128, 128, Wbuf, cb);
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int row = hkbs::mfma_row(rb, v), col = hkbs::mfma_col(cb, v);
    for (int k = 0; k < 128; ++k) ref[v] = ref[v] + A[k * kGemmLd + row] * Wb[k * 128 + col];
    if (__float_as_uint(ref[v]) != __float_as_uint(acc[v])) {
      if (atomicAdd(&out[0], 1u) == 0u) {
        out[1] = blockIdx.x;
        out[2] = static_cast<unsigned int>(row * 128 + col);
        out[3] = __float_as_uint(acc[v]);
      }
    }
  }
}

}  // namespace

// Runs seq_gemm_check_kernel on `blocks` tiles on the current device; out[4] as there.
extern "C" int hkbs_check_device_seq_gemm(unsigned int blocks, unsigned int* out_host) {
  unsigned int* out = nullptr;
  float* W = nullptr;
  hipError_t e = hipMalloc(&out, 4 * sizeof(unsigned int));
  if (e == hipSuccess) e = hipMalloc(&W, static_cast<size_t>(blocks) * 128 * 128 * sizeof(float));
  if (e == hipSuccess) e = hipMemset(out, 0, 4 * sizeof(unsigned int));
  if (e == hipSuccess) {
    seq_gemm_check_kernel<<<blocks, 256>>>(W, out);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e == hipSuccess) e = hipMemcpy(out_host, out, 4 * sizeof(unsigned int), hipMemcpyDeviceToHost);
  if (W) (void)hipFree(W);
  if (out) (void)hipFree(out);
  return static_cast<int>(e);
}

// Runs rbf_kernel over n offsets on the current device; out[3] as there.
extern "C" int hkbs_check_device_rbf(unsigned int n, unsigned int* out_host) {
  unsigned int* out = nullptr;
  hipError_t e = hipMalloc(&out, 3 * sizeof(unsigned int));
  if (e == hipSuccess) e = hipMemset(out, 0, 3 * sizeof(unsigned int));
  if (e == hipSuccess) {
    rbf_kernel<<<1024, 256>>>(n, out);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e == hipSuccess) e = hipMemcpy(out_host, out, 3 * sizeof(unsigned int), hipMemcpyDeviceToHost);
  if (out) (void)hipFree(out);
  return static_cast<int>(e);
}
