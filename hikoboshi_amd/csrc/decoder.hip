// ProteinMPNN autoregressive decoder (3 layers) + temperature sampler.
//
// Reference: run_autoregressive_decoder (cpp/modules/mpnn/inverse_fold_scalar.cpp:752-888)
// with proteinmpnn_decoder_layer_scalar (cpp/modules/mpnn/decoder_layer_scalar.cpp:26-151)
// and proteinmpnn_sample_scalar (cpp/modules/mpnn/sampler_scalar.cpp:27-131).
// For the residue t decoded at a step, layer l, neighbour slot k (j = idx[t,k]):
//   ctx_k = bw [h_E_tk, W_s[tok_j], h^l_j] + fw [h_E_tk, 0, h^0_j]
//   (bw = j decoded before t, fw otherwise; both 0 for an invalid slot),
//   m_k   = W3 g(W2 g(W1 [h^l_t, ctx_k] + b1) + b2) + b3,
//   h'    = LN1(h^l_t + sum_k m_k / 30),  h^{l+1}_t = LN2(h' + FFN(h')).
// With W1 = [W1a | W1b | W1c | W1d] over [h_t | h_E | h_S | h_V] the first
// product splits into terms that do not depend on the step:
//   W1 [h_t, ctx_k] + b1 = A_t + E1_tk + (bw ? R^l_j : Q^l_j)    (valid slot)
//   A_t    = W1a h^l_t + b1                         (precomputed for l = 0, one fused
//                                                    GEMV with the next W1d for l > 0)
//   E1_tk  = W1b h_E_tk                             (precomputed, all sequences)
//   Q^l_j  = W1d h^0_j                              (precomputed, all sequences)
//   R^l_j  = W1d h^l_j + W1c W_s[tok_j]             (written when j is decoded)
// and sum_k (W3 g_k + b3) = W3 sum_k g_k + K b3. The per-step K-row work is
// then one 128x128 product (W2) on fp32 MFMA; the rest are GEMVs.
//
// One workgroup decodes one sequence for all L steps (persistent); the
// sequences of a batch are independent once the encoder outputs exist.
// Consecutive independent residues are decoded together (see decode_kernel).
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "device_math.hpp"
#include "pmpnn_internal.hpp"

namespace hkbs {
namespace {

constexpr int kLd = kH + 4;  // 132
constexpr int kLdH = kH + 8;  // 136 halves: 16-byte rows that step 4 banks
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
// Per-layer vectors kept in LDS for the whole kernel: [b1 b2 b3 bin bout n1g n1b n2g n2b]
constexpr int kPrmB1 = 0, kPrmB2 = 128, kPrmB3 = 256, kPrmBin = 384, kPrmBout = 896, kPrmN1g = 1024,
              kPrmN1b = 1152, kPrmN2g = 1280, kPrmN2b = 1408, kPrmLayer = 1536;
constexpr int kPrmLog = kLayers * kPrmLayer;  // logits bias (32)
constexpr int kPrmSize = kPrmLog + 32;
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 512;

constexpr int kGroup = 4;  // members of the fp32 products' accumulators (Gemv)

// Y[i][o] = sum_p X[i][p] Wt[p][o] for i < m rows (m <= kGroup), OUT outputs
// and IN inputs on all threads. Thread (q, grp) owns float4 column q and
// inputs [grp PER, (grp + 1) PER), taken in NP parts of PP inputs so that a
// part's weight loads can be issued while the previous part (or the previous
// step's reduction) is still running. fma() accumulates one part in input
// order, store() leaves per-group partial sums in LDS (part >= 8192 floats),
// and after a barrier sum() adds the groups of one output in a fixed order.
// decode arithmetic (DecodeArgs.precision): fp32, bf16, fp16, split bf16 (two bf16 terms per operand)
constexpr int kPrecFp32 = 0, kPrecBf16 = 1, kPrecFp16 = 2, kPrecBf16x3 = 3;

template <int IN, int OUT, int NP = 1, int WT = kPrecFp32>
struct Gemv {
  static constexpr int Q4 = OUT / 4;            // float4 columns
  static constexpr int GROUPS = kThreads / Q4;  // input groups
  static constexpr int PER = IN / GROUPS;       // inputs per group
  static constexpr int PP = PER / NP;           // inputs per part
  static_assert(PP * NP == PER, "parts");
  // fp32 weights: one float4 per input; bf16 / fp16 weights: four 16-bit values (8 bytes) per input
  using W4 = typename std::conditional<WT == kPrecFp32, float4, uint2>::type;
  struct Part {
    W4 w[PP];
  };

  // spread = 0: every lane loads the first slice (a placeholder load that costs no L2 traffic)
  static __device__ inline void load(Part& P, const void* __restrict__ Wt, int k, size_t spread = 1) {
    const int q = threadIdx.x % Q4, grp = threadIdx.x / Q4;
    const size_t at = ((size_t)(grp * PER + k * PP) * OUT + 4 * q) * spread;
    if constexpr (WT != kPrecFp32) {
      const uint16_t* p = static_cast<const uint16_t*>(Wt) + at;
#pragma unroll
      for (int i = 0; i < PP; ++i) P.w[i] = *reinterpret_cast<const uint2*>(p + (size_t)i * OUT * spread);
    } else {
      const float* p = static_cast<const float*>(Wt) + at;
#pragma unroll
      for (int i = 0; i < PP; ++i) P.w[i] = *reinterpret_cast<const float4*>(p + (size_t)i * OUT * spread);
    }
  }
  static __device__ inline float half_lo(uint32_t v) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(v & 0xFFFFu)));
  }
  static __device__ inline float4 widen(const W4& w) {
    if constexpr (WT == kPrecBf16) {
      return make_float4(__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xFFFF0000u), __uint_as_float(w.y << 16),
                         __uint_as_float(w.y & 0xFFFF0000u));
    } else if constexpr (WT == kPrecFp16) {
      return make_float4(half_lo(w.x), half_lo(w.x >> 16), half_lo(w.y), half_lo(w.y >> 16));
    } else {
      return w;
    }
  }
  static __device__ inline void fma(const Part& P, int k, const float* X, int m, float4 (&acc)[kGroup]) {
    const int grp = threadIdx.x / Q4;
#pragma unroll
    for (int i = 0; i < kGroup; ++i) {
      if (i >= m) break;
      const float* x = X + i * IN + grp * PER + k * PP;
#pragma unroll
      for (int p = 0; p < PP; ++p) {
        const float xv = x[p];
        const float4 wv = widen(P.w[p]);
        acc[i].x += xv * wv.x;
        acc[i].y += xv * wv.y;
        acc[i].z += xv * wv.z;
        acc[i].w += xv * wv.w;
      }
    }
  }
  static __device__ inline void store(const float4 (&acc)[kGroup], int m, float* part) {
    const int q = threadIdx.x % Q4, grp = threadIdx.x / Q4;
#pragma unroll
    for (int i = 0; i < kGroup; ++i) {
      if (i >= m) break;
      *reinterpret_cast<float4*>(part + (i * GROUPS + grp) * OUT + 4 * q) = acc[i];
    }
  }
  static __device__ inline float sum(const float* part, int i, int o) {
    float s = 0.0F;
#pragma unroll
    for (int g = 0; g < GROUPS; ++g) s += part[(i * GROUPS + g) * OUT + o];
    return s;
  }
};

// Products of the 16-bit decode modes on the MFMA: y[m][n] = sum_k x[m][k] W[k][n]
// for the members m < ml (rows of the 16-row A operand; the other rows are zero),
// so that the arithmetic does not grow with the members a workgroup holds. W is
// stored as B fragments [IN / 8][OUT][8] (bf16 or fp16, pack_k8_t). The
// activations come from a split 16-bit copy in LDS (put_split16: x = hi + lo
// with bf16 parts, x = hi + lo / 2048 with fp16 parts), so that, as with the
// fp32 activations of the VALU products, only the weights are rounded to 16
// bits; the products accumulate in fp32. Wave w owns output columns [16 CPW w,
// 16 CPW (w + 1)) over the whole input range (no partial sums), which part p
// of NP splits into k-ranges loaded separately.
// PREC = kPrecBf16x3 (split bf16): the weights too are two bf16 terms (W and its
// remainder Wl, pack_k8_t kHalfBf16Lo), and each k-block takes three MFMAs,
// x_hi W + (x_hi Wl + x_lo W); the dropped x_lo Wl is below 2^-16 of the product.
template <int IN, int OUT, int NP, int PREC>
struct MGemv {
  static constexpr bool X3 = PREC == kPrecBf16x3;
  static constexpr bool BF = PREC == kPrecBf16 || X3;     // bf16 operands
  static constexpr int KB = IN / 32 / NP;                 // k-blocks of 32 inputs per part
  static constexpr int CPW = OUT / 16 / (kThreads / 64);  // 16-column blocks per wave
  static constexpr int GR = decode_group(PREC, 1);        // member rows of the split copies
  static_assert(PREC != kPrecFp32 && KB * 32 * NP == IN && CPW * 16 * (kThreads / 64) == OUT, "MFMA product shape");
  using Op = typename std::conditional<BF, bf16x8, half8>::type;
  struct Part {
    Op b[CPW][KB];
    Op bl[X3 ? CPW : 1][X3 ? KB : 1];  // split bf16: the weights' remainders
  };
  struct Acc {
    floatx4 a[CPW], c[CPW];  // c: the fp16 lo products (scaled by 2048), or the split bf16 remainder products
  };
  // spread = 0: every lane loads the first fragment (a placeholder load that costs no L2 traffic).
  // Wl (the remainders) is read only in the split bf16 mode.
  static __device__ inline void load(Part& P, const uint16_t* __restrict__ W, const uint16_t* __restrict__ Wl, int part,
                                     size_t spread = 1) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int cb = 0; cb < CPW; ++cb)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const size_t at = ((size_t)(4 * (part * KB + kb) + (lane >> 4)) * OUT + (wave * CPW + cb) * 16 + (lane & 15)) * 8;
        P.b[cb][kb] = *reinterpret_cast<const Op*>(W + at * spread);
        if constexpr (X3) P.bl[cb][kb] = *reinterpret_cast<const Op*>(Wl + at * spread);
      }
  }
  static __device__ inline void zero(Acc& A) {
#pragma unroll
    for (int cb = 0; cb < CPW; ++cb) {
      A.a[cb] = floatx4{0.F, 0.F, 0.F, 0.F};
      A.c[cb] = A.a[cb];
    }
  }
  // xs: the split copy, hi plane [GR][IN] then lo plane
  static __device__ inline void run(const Part& P, int part, const uint16_t* xs, int ml, Acc& A) {
    const int lane = threadIdx.x & 63, row = lane & 15;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      Op ah{}, al{};
      if (row < ml) {
        const int at = row * IN + 32 * (part * KB + kb) + 8 * (lane >> 4);
        ah = *reinterpret_cast<const Op*>(xs + at);
        al = *reinterpret_cast<const Op*>(xs + GR * IN + at);
      }
#pragma unroll
      for (int cb = 0; cb < CPW; ++cb) {
        if constexpr (X3) {
          A.a[cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, P.b[cb][kb], A.a[cb], 0, 0, 0);
          A.c[cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, P.bl[cb][kb], A.c[cb], 0, 0, 0);
          A.c[cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, P.b[cb][kb], A.c[cb], 0, 0, 0);
        } else if constexpr (BF) {
          A.a[cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, P.b[cb][kb], A.a[cb], 0, 0, 0);
          A.a[cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, P.b[cb][kb], A.a[cb], 0, 0, 0);
        } else {
          A.a[cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, P.b[cb][kb], A.a[cb], 0, 0, 0);
          A.c[cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, P.b[cb][kb], A.c[cb], 0, 0, 0);
        }
      }
    }
  }
  // y[m][n] into ys [GR][OUT]: lane j holds column j % 16 of rows (members) 4 (j / 16) + 0..3
  static __device__ inline void store(const Acc& A, int ml, float* ys) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r0 = 4 * (lane >> 4);
    if (r0 >= ml) return;
#pragma unroll
    for (int cb = 0; cb < CPW; ++cb) {
      const int col = (wave * CPW + cb) * 16 + (lane & 15);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (r0 + e >= ml) break;
        ys[(r0 + e) * OUT + col] =
            X3 ? A.a[cb][e] + A.c[cb][e] : BF ? A.a[cb][e] : A.a[cb][e] + A.c[cb][e] * (1.0F / 2048.0F);
      }
    }
  }
};

// Split 16-bit copy of one activation for MGemv: plane 0 = hi, plane 1 (lo_at
// elements later) = lo; bf16 and split bf16: x = hi + lo, fp16: x = hi + lo / 2048
// (|x| clamped to the fp16 range).
template <int PREC>
__device__ inline void put_split16(uint16_t* hi, int lo_at, float v) {
  if constexpr (PREC == kPrecBf16 || PREC == kPrecBf16x3) {
    const __bf16 h = static_cast<__bf16>(v);
    hi[0] = __builtin_bit_cast(uint16_t, h);
    hi[lo_at] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(v - static_cast<float>(h)));
  } else {
    const float c = __builtin_amdgcn_fmed3f(v, -65504.0F, 65504.0F);
    const _Float16 h = static_cast<_Float16>(c);
    hi[0] = __builtin_bit_cast(uint16_t, h);
    hi[lo_at] = __builtin_bit_cast(uint16_t, static_cast<_Float16>((c - static_cast<float>(h)) * 2048.0F));
  }
}

__device__ inline void zero4(float4 (&acc)[kGroup]) {
#pragma unroll
  for (int i = 0; i < kGroup; ++i) acc[i] = make_float4(0.F, 0.F, 0.F, 0.F);
}

// One sampler draw on a row of logits by one wave (reference operation order,
// sampler_scalar.cpp:49-92); state is the splitmix64 state before this draw.
// Lane v < kV computes token v's scaled logit, exponential and log-prob
// (returned in *lp); the sum of exponentials and the double-precision CDF
// walk run over the tokens in order, identically in every lane. Returns the
// drawn token, the same in every lane.
__device__ inline int sample_wave(float logit, float T, bool greedy, uint64_t state, float* lp) {
  const int lane = threadIdx.x & 63;
  const bool tok_lane = lane < kV;
  const float z = tok_lane ? logit / T : -__builtin_inff();
  const float row_max = wave_max(z);
  const float e = tok_lane ? expf(z - row_max) : 0.0F;
  float row_sum = 0.0F;
#pragma unroll
  for (int v = 0; v < kV; ++v) row_sum += lane_f32(e, v);
  const float log_sum = logf(row_sum);
  const float inv_sum = 1.0F / row_sum;
  *lp = (z - row_max) - log_sum;
  if (greedy) {
    // first token holding the maximum (strict > scan)
    const unsigned long long hits = __ballot(tok_lane && z == row_max);
    return __ffsll(static_cast<long long>(hits)) - 1;
  }
  uint64_t zz = state + 0x9E3779B97F4A7C15ull;
  zz = (zz ^ (zz >> 30)) * 0xBF58476D1CE4E5B9ull;
  zz = (zz ^ (zz >> 27)) * 0x94D049BB133111EBull;
  zz ^= zz >> 31;
  const double u = static_cast<double>(zz >> 11) * (1.0 / 9007199254740992.0);
  const float p = e * inv_sum;
  double cum = 0.0;
  int tok = kV - 1;
#pragma unroll
  for (int v = 0; v < kV; ++v) {
    cum += static_cast<double>(lane_f32(p, v));
    if (u < cum && tok == kV - 1 && v < kV - 1) tok = v;
  }
  return tok;
}

// Device-scope accesses of the state team members exchange (R rows, chosen
// log-probs): the stores write through to the device coherence point and the
// loads are served from it, never from a CU's L1 or an XCD's L2 copy that
// could predate another workgroup's store. Relaxed atomics at agent scope.
__device__ inline void store_dev(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ inline float load_dev(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void store_dev(int32_t* p, int32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline int32_t load_dev(const int32_t* p) {
  return __hip_atomic_load(const_cast<int32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Four consecutive floats (16-byte aligned) as two 8-byte device-scope loads.
__device__ inline float4 load4_dev(const float* p) {
  uint64_t* q = reinterpret_cast<uint64_t*>(const_cast<float*>(p));
  const uint64_t a = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t b = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_float4(__uint_as_float((uint32_t)a), __uint_as_float((uint32_t)(a >> 32)), __uint_as_float((uint32_t)b),
                     __uint_as_float((uint32_t)(b >> 32)));
}

// Four fp16 values (8 bytes) widened to fp32.
__device__ inline float4 widen_h4(uint64_t v) {
  const auto h = [](uint64_t x, int i) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(x >> (16 * i))));
  };
  return make_float4(h(v, 0), h(v, 1), h(v, 2), h(v, 3));
}
__device__ inline uint64_t load8_dev(const _Float16* p) {
  return __hip_atomic_load(reinterpret_cast<uint64_t*>(const_cast<_Float16*>(p)), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}
// Two fp32 values as fp16 (clamped to its range) packed into one 32-bit word, the lower address first.
__device__ inline int32_t pack_h2(float a, float b) {
  const uint32_t lo = __builtin_bit_cast(uint16_t, static_cast<_Float16>(__builtin_amdgcn_fmed3f(a, -65504.0F, 65504.0F)));
  const uint32_t hi = __builtin_bit_cast(uint16_t, static_cast<_Float16>(__builtin_amdgcn_fmed3f(b, -65504.0F, 65504.0F)));
  return static_cast<int32_t>(lo | (hi << 16));
}

constexpr uint32_t kSpinLimit = 1u << 20;  // default polls (~1 s) before a team gives up

// Split-phase barrier over the P workgroups of a team. team_arrive: every
// wave first waits for its own memory operations (so its device-scope stores
// of exchanged state have completed at the device coherence point) and the
// workgroup meets at a barrier; thread 0 then counts the workgroup in with a
// device-scope atomic. Work that reads no exchanged state may run between
// arrive and wait. team_wait: thread 0 polls the count with device-scope
// loads until all P have arrived `target / P` times, and the workgroup meets
// again. Exchanged state is read only after that, and only with device-scope
// loads (load_dev, load4_dev), so a member sees every store the others made
// before they arrived, wherever the members run on the device. team_wait
// returns false (and raises the fault word) if the wait does not end; the
// caller then stops so that every wave exits.
// With fences != 0 the barrier also carries the ordering of the HIP memory
// model: an agent-scope release fence before the count's add and an
// agent-scope acquire fence once the poll loop has seen the count (once per
// barrier, not per poll), so that the stores made before a member's arrival
// happen before the loads made after another member's wait. The relaxed form
// (fences == 0) gives the same bits in every test and is the default: on
// gfx950 those two fences write back and invalidate the XCD's L2
// (buffer_wbl2 / buffer_inv), which costs about 3 us per barrier.
// A team's members are dealt onto one XCD (round-robin dispatch) only for the
// barrier's latency; neither form depends on it for its results.
__device__ inline void team_arrive(uint32_t* counter, int fences) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    if (fences) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}
__device__ inline bool team_wait(uint32_t* counter, uint32_t target, uint32_t spin_limit, uint32_t* fault, int* bad,
                                 int fences) {
  if (threadIdx.x == 0) {
    uint32_t n = 0;
    while (__hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
      __builtin_amdgcn_s_sleep(1);
      if (++n >= spin_limit) {
        *bad = 1;
        __hip_atomic_store(fault, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
    if (fences) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  __syncthreads();
  return *bad == 0;
}

// Token of a residue whose step another workgroup of the team (or this one)
// decodes: tokens start the decode at -1 and a step's token is stored only
// after the R rows of that step have completed at the device coherence point,
// so once a device-scope load returns the token, device-scope loads of the
// step's R rows return the rows. Polls at most spin_limit times; a wait that
// runs out raises the fault word and *bad and returns 0 (the caller then
// stops). With fences != 0 an agent-scope acquire fence follows the poll
// (the writer puts a release fence before the token store).
__device__ inline int await_token(const int32_t* tok, uint32_t spin_limit, uint32_t* fault, int* bad, int fences) {
  int v = load_dev(tok);
  uint32_t n = 0;
  while (v < 0) {
    if (++n >= spin_limit) {
      *bad = 1;
      __hip_atomic_store(fault, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return 0;
    }
    __builtin_amdgcn_s_sleep(1);
    v = load_dev(tok);
  }
  if (fences) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  return v;
}
// Added to the team counter by a workgroup that stopped early (a wait ran out):
// the final count then tells rank 0 that the sequence was not decoded.
constexpr uint32_t kTeamAbort = 1u << 24;

// Decodes one sequence per team of P workgroups (P = a.team, 1..8) in the
// passes of the dependency schedule (ready_schedule_kernel): a pass holds up to
// a.max_members (<= G * P) steps whose earlier kNN neighbours were all
// decoded in earlier passes, so each step sees the inputs of sequential
// decoding (bw = the neighbour's position is before the step's own). Member i
// of a pass runs on team rank i % P; a rank with several members shares each
// weight load and workgroup barrier between them. A step's token comes from
// draw a.draw[u] of the sequence's counter stream, i.e. draws are consumed in
// order of u whatever pass decodes the step. The state a later pass reads (R
// rows, tokens) is written with device-scope stores; a step's token is stored
// after its R rows have completed, and a pass starts by waiting for the tokens
// of its steps' earlier neighbours (await_token), so the ranks of a team meet
// only after pass 0 and before the score. Pass 0 (inactive residues: fallback
// token, zero log-probs, no draw) runs first, on rank 0.
// With P > 1 the grid is 8 * ceil(B / 8) * P workgroups and rank r of
// sequence b runs as workgroup 8 (P (b / 8) + r) + b % 8, so that a team
// shares one XCD when workgroups are dealt round-robin over the 8 XCDs; the
// whole grid fits the device at once.
// PREC = kPrecFp32: fp32 weights; W2 product on the fp16 MFMA with hi/lo
// operands (fp32-level accuracy), the layer products (Gemv) on the VALU in
// fp32. kPrecBf16 / kPrecFp16: 16-bit weights for every product; message rows
// rounded to 16 bits for one 16x16x32 MFMA per k-block; the layer products
// (MGemv) on the MFMA with the fp32 activations split into two 16-bit parts,
// accumulated in fp32. kPrecBf16x3 (split bf16): every product on the bf16 MFMA
// with both operands as two bf16 terms (hi + lo) and three MFMAs per k-block
// (hi.hi + hi.lo + lo.hi): the message rows into W2 and the weights of W2 and
// of the layer products (MGemv); the message rows' inputs (E1, Q, R) stay
// fp32, and so do the logit weights (hi + lo, exact in fp32). In every mode
// activations, LayerNorm, the logits (one wave per member, weights in LDS) and
// the sampler are fp32.
template <int PREC, int G>
__global__ __launch_bounds__(kThreads) void decode_kernel(ModelDev m, DecodeArgs a) {
  constexpr bool BF = PREC == kPrecBf16, HF = PREC == kPrecFp16, X3 = PREC == kPrecBf16x3;
  constexpr bool H16 = BF || HF;        // message rows' inputs (E1, Q, R) in fp16
  constexpr bool M16 = BF || HF || X3;  // layer products on the MFMA (MGemv)
  using G3 = Gemv<kH, kH, 1, PREC>;
  using GIn = Gemv<kH, kFF, 2, PREC>;
  using GOut = Gemv<kFF, kH, 2, PREC>;
  using GDa = Gemv<kH, 2 * kH, 1, PREC>;
  // G: steps this workgroup can hold in a pass (decode_group(PREC, team size))
  static_assert(G == decode_group(PREC, 1) || G == decode_group(PREC, 2), "group size of this mode");
  // 16-bit modes: staging of the MFMA products (below). fp32: the products'
  // partial sums [member][group][output] (2048 floats per member); with more
  // members than kGroup they share G16's space: the message rows and the partial
  // sums are never live together (barriers separate a layer's last W2 product
  // from its W3 partial sums, and the fused next-layer sums from the next
  // layer's message rows).
  constexpr bool kPartInG16 = !M16 && G > kGroup;
  // message rows of two members as fp16 pairs: [member][hi, lo][row][kLdH]
  // (larger when it also holds the partial sums of more members)
  constexpr int kG16 = kPartInG16 && 2 * 2048 * G > 2 * 2 * kKmax * kLdH ? 2 * 2048 * G : 2 * 2 * kKmax * kLdH;
  __shared__ __attribute__((aligned(16))) _Float16 G16[kG16];
  constexpr int kPart = M16 ? G * kFF + (6 * G * kH + 2 * G * kFF) / 2 : kPartInG16 ? 1 : 2048 * G;
  __shared__ __attribute__((aligned(16))) float part16[kPart];
  float* const part = kPartInG16 ? reinterpret_cast<float*>(G16) : part16;
  static_assert(M16 || (G3::GROUPS * kH == 2048 && GIn::GROUPS * kFF == 2048 && GOut::GROUPS * kH == 2048 &&
                        GDa::GROUPS * 2 * kH == 2048 && (!kPartInG16 || 2048 * G * sizeof(float) <= sizeof(G16))),
                "fp32 partial sums fit");
  __shared__ __attribute__((aligned(16))) float ff[G * kFF];  // also [m][256] scratch
  __shared__ __attribute__((aligned(16))) float h[G * kH];
  __shared__ __attribute__((aligned(16))) float hA[G * kH];
  __shared__ __attribute__((aligned(16))) float x[G * kH];
  __shared__ __attribute__((aligned(16))) float h1[G * kH];
  __shared__ __attribute__((aligned(16))) float Pd[G * 2 * kH];  // W1d h^l of layers 1, 2
  // logits weights (32 outputs, 21 used) as fp32, [k / 4][v][k % 4]: lane v reads four k of its column at once
  __shared__ __attribute__((aligned(16))) float wlg[kH * 32];
  __shared__ __attribute__((aligned(16))) float prm[kPrmSize];
  __shared__ __attribute__((aligned(16))) float gtab[kGeluPolyLds];  // GELU polynomials
  // neighbour words of the step records: -1 for an empty slot, else j | 2^30 if j is decoded before the step
  __shared__ __attribute__((aligned(16))) int nbw[G * kKmax];
  __shared__ int cls[G * kKmax];  // layer-0 table row of each slot (with a.l0tab)
  __shared__ __attribute__((aligned(16))) float q0s[G * kH];  // Q^0 rows of the members (R^0 base)
  // per member: residue, sampler draw index, design weight chain_mask * mask as float bits (0: keep the
  // true token), true token or the fallback token
  __shared__ int4 meta[G];
  // per member: mask of the slots decoded before the step (lo, hi words), first layer-0 table row
  __shared__ int4 meta2[G];
  __shared__ int tok_s[G];
  __shared__ int bad;

  // 16-bit modes: the MFMA products' outputs and the split 16-bit copies of
  // their inputs (put_split16), in `part`, which only the fp32 products use
  float* ys = part;  // [G][up to kFF]
  uint16_t* const s16 = reinterpret_cast<uint16_t*>(part + G * kFF);
  uint16_t* const xs16 = s16;                    // message sums, [hi, lo][G][kH]
  uint16_t* const h1s16 = s16 + 2 * G * kH;  // h1
  uint16_t* const hs16 = s16 + 4 * G * kH;   // h
  uint16_t* const ffs16 = s16 + 6 * G * kH;  // ff, [hi, lo][G][kFF]
  static_assert(!M16 || G * kFF + (6 * G * kH + 2 * G * kFF) / 2 <= kPart, "16-bit staging fits part");
  const int P = a.team;
  int b = blockIdx.x, rank = 0;
  if (P > 1) {
    const int xcd = blockIdx.x % 8, slot = blockIdx.x / 8;
    rank = slot % P;
    b = (slot / P) * 8 + xcd;
  }
  if (b >= a.B) return;  // padding team: all of its ranks leave together
  const int L = a.L, K = a.K;
  const size_t S = (size_t)L * K;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int32_t* order = a.shared_order ? a.orders : a.orders + (size_t)b * L;
  const size_t qo = a.shared_order ? 0 : (size_t)b;
  const int32_t* nbj = a.nbj + qo * L * K;
  const int32_t* nbp = a.nbp + qo * L * K;
  const int32_t* sched = a.sched + qo * L;
  const int32_t* pstart = a.pstart + qo * (L + 2);
  const int32_t* draw = a.draw + qo * L;
  // An order that is not a permutation of 0..L-1 is not decoded (the reference
  // rejects it, decode_order_scalar.cpp:67-79; the host entry points check
  // orders before any GPU work, the device entry points cannot): the sequence
  // keeps a NaN score and its tokens and log-probs are not written. Every rank
  // of a team reads the same flag, so the team leaves together.
  if (sched_meta(a.sched_tmp, L, a.shared_order ? 1 : a.B)[qo * 4 + 3] == 0) {
    if (a.scores && rank == 0 && threadIdx.x == 0) a.scores[b] = __builtin_nanf("");
    return;
  }
  const int npass = a.npass[qo];
  float* R = a.R + (size_t)b * kLayers * L * kH;
  _Float16* Rh = H16 ? a.Rh + (size_t)b * kLayers * L * kH : nullptr;  // bf16 / fp16 modes: R in fp16
  int32_t* tokens = a.tokens + (size_t)b * L;
  float* lp_out = a.log_probs ? a.log_probs + (size_t)b * L * kV : nullptr;
  float* chosen = a.chosen_lp + (size_t)b * L;
  uint32_t* counter = a.sync + b;
  const uint64_t seed = a.seeds[b];
  const float T = (a.temperature > 0.0F && isfinite(a.temperature)) ? a.temperature : 1.0F;
  const bool greedy = a.greedy || a.temperature <= 0.0F;
  load_gelu_poly(gtab, threadIdx.x, kThreads);
  if (threadIdx.x == 0) bad = 0;
  for (int l = 0; l < kLayers; ++l) {
    const DecLayerDev& w = m.dec[l];
    float* p = prm + l * kPrmLayer;
    for (int i = threadIdx.x; i < kH; i += kThreads) {
      p[kPrmB1 + i] = w.b1[i];
      p[kPrmB2 + i] = w.b2[i];
      p[kPrmB3 + i] = w.b3[i];
      p[kPrmBout + i] = w.bout[i];
      p[kPrmN1g + i] = w.n1g[i];
      p[kPrmN1b + i] = w.n1b[i];
      p[kPrmN2g + i] = w.n2g[i];
      p[kPrmN2b + i] = w.n2b[i];
    }
    for (int i = threadIdx.x; i < kFF; i += kThreads) p[kPrmBin + i] = w.bin[i];
  }
  if (threadIdx.x < 32) prm[kPrmLog + threadIdx.x] = m.blog[threadIdx.x];
  for (int e = threadIdx.x; e < kH * 32; e += kThreads) {
    const int k = e / 32, v = e % 32;
    float wv;
    if constexpr (BF) {
      wv = __uint_as_float(static_cast<uint32_t>(m.Wlog_h[e]) << 16);
    } else if constexpr (X3) {  // hi + lo, exact in fp32
      const float w0 = m.Wlog_t[e];
      const float hi = static_cast<float>(static_cast<__bf16>(w0));
      wv = hi + static_cast<float>(static_cast<__bf16>(w0 - hi));
    } else if constexpr (HF) {
      wv = static_cast<float>(__builtin_bit_cast(_Float16, m.Wlog_f[e]));
    } else {
      wv = m.Wlog_t[e];
    }
    wlg[((k >> 2) * 32 + v) * 4 + (k & 3)] = wv;
  }
  // Every token starts at -1 (not decoded yet); later passes wait for the
  // tokens of their steps' earlier neighbours (await_token) instead of for
  // the whole team.
  if (rank == 0)
    for (int i = threadIdx.x; i < L; i += kThreads) store_dev(tokens + i, -1);
  __syncthreads();

  // Pass 0: inactive residues (inverse_fold_scalar.cpp:804-813): fallback
  // token, zero log-probs, no draw; R rows Q + T[tok] (layer 0) and T[tok].
  {
    const int s0 = pstart[0], n0 = pstart[1] - pstart[0];
    if (n0 > 0) {
      if (rank == 0) {
        for (int i = threadIdx.x; i < n0; i += kThreads) {
          const int t = order[sched[s0 + i]];
          const int tok = (a.true_tokens && a.true_tokens[t] >= 0 && a.true_tokens[t] < kV) ? a.true_tokens[t] : kV - 1;
          store_dev(tokens + t, tok);
          store_dev(chosen + t, 0.0F);
        }
        if (lp_out)
          for (int task = threadIdx.x; task < n0 * kV; task += kThreads)
            lp_out[(size_t)order[sched[s0 + task / kV]] * kV + task % kV] = 0.0F;
        if constexpr (H16) {  // fp16 rows, two columns per device-scope store
          for (int task = threadIdx.x; task < n0 * kLayers * (kH / 2); task += kThreads) {
            const int i = task / (kLayers * kH / 2), l = (task / (kH / 2)) % kLayers, c = 2 * (task % (kH / 2));
            const int t = order[sched[s0 + i]];
            const int tok = (a.true_tokens && a.true_tokens[t] >= 0 && a.true_tokens[t] < kV) ? a.true_tokens[t] : kV - 1;
            const float* q = a.Q + (size_t)t * kH + c;
            const float* tv = m.dec[l].T + tok * kH + c;
            const float v0 = ((l == 0) ? q[0] : 0.0F) + tv[0], v1 = ((l == 0) ? q[1] : 0.0F) + tv[1];
            store_dev(reinterpret_cast<int32_t*>(Rh + ((size_t)l * L + t) * kH + c), pack_h2(v0, v1));
          }
        } else {
          for (int task = threadIdx.x; task < n0 * kLayers * kH; task += kThreads) {
            const int i = task / (kLayers * kH), l = (task / kH) % kLayers, c = task % kH;
            const int t = order[sched[s0 + i]];
            const int tok = (a.true_tokens && a.true_tokens[t] >= 0 && a.true_tokens[t] < kV) ? a.true_tokens[t] : kV - 1;
            const float base = (l == 0) ? a.Q[(size_t)t * kH + c] : 0.0F;
            store_dev(R + ((size_t)l * L + t) * kH + c, base + m.dec[l].T[tok * kH + c]);
          }
        }
      }
    }
  }
  if (P > 1) team_arrive(counter, a.fences);  // the -1 tokens and pass 0 are in place before any wait
  // Inputs of a pass that no other workgroup writes come from its step
  // records: one 16-byte slice per thread, loaded during the previous pass's
  // logits and written to LDS once that pass is done with its copies.
  const float4* rec = a.rec + qo * (size_t)L * kRecFloat4;
  auto members = [&](int ps, int& s0) -> int {  // members of this rank in pass ps: rank + P i
    s0 = pstart[ps];
    const int mg = pstart[ps + 1] - s0;
    return mg > rank ? (mg - rank + P - 1) / P : 0;
  };
  // Slice e = threadIdx.x + kThreads q of the members' records is thread
  // threadIdx.x's slice of round q (kRecRounds rounds cover G members).
  constexpr int kRecRounds = (G * kRecFloat4 + kThreads - 1) / kThreads;
  auto rec_load = [&](int s0, int mlp, int q) -> float4 {
    const int e = threadIdx.x + kThreads * q, i = e / kRecFloat4;
    if (mlp > G || i >= mlp) return make_float4(0.F, 0.F, 0.F, 0.F);
    return rec[(size_t)(s0 + rank + P * i) * kRecFloat4 + e % kRecFloat4];
  };
  auto rec_store = [&](int mlp, const float4& v, int q) {
    // The destination is recomputed here on purpose: a copy hoisted out of the
    // pass loop would be spilled, and reloading it put memory latency in the
    // pass hand-over.
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int e = tid + kThreads * q;
    const int i = e / kRecFloat4, w = e % kRecFloat4;
    if (mlp > G || i >= mlp || (w > kKmax / 4 + 1 && w < 16)) return;
    float4* dst;
    if (w < kKmax / 4) {
      dst = reinterpret_cast<float4*>(nbw + i * kKmax) + w;
    } else if (w == kKmax / 4) {
      dst = reinterpret_cast<float4*>(meta + i);
    } else if (w == kKmax / 4 + 1) {
      dst = reinterpret_cast<float4*>(meta2 + i);
    } else {
      const int blk = (w - 16) / (kH / 4), c = 4 * ((w - 16) % (kH / 4));
      dst = reinterpret_cast<float4*>((blk == 0 ? h : (blk == 1 ? hA : q0s)) + i * kH + c);
    }
    *dst = v;
  };
  static_assert(kKmax % 4 == 0 && kRecFloat4 == 16 + 3 * kH / 4 && kRecRounds <= 2, "record layout");
  int ml = 0;
  if (npass >= 1) {
    int s0 = 0;
    ml = members(1, s0);
#pragma unroll
    for (int q = 0; q < kRecRounds; ++q) rec_store(ml, rec_load(s0, ml, q), q);
  }
  if (P > 1 && !team_wait(counter, P, a.spin_limit, a.fault, &bad, a.fences)) goto finish;  // pass 0
  __builtin_amdgcn_s_waitcnt(0);  // one workgroup per sequence: its own pass-0 stores are complete
  __syncthreads();
  for (int pass = 1; pass <= npass; ++pass) {
    if (ml > G) {  // a schedule built for a larger team: refuse rather than overrun LDS
      if (threadIdx.x == 0) __hip_atomic_store(a.fault, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      bad = 1;
      break;
    }
    int s0n = 0, mln = 0;  // the next pass
    if (pass < npass) mln = members(pass + 1, s0n);
    float4 rv[kRecRounds];
#pragma unroll
    for (int q = 0; q < kRecRounds; ++q) rv[q] = make_float4(0.F, 0.F, 0.F, 0.F);
    bool staged = false;
    if (ml > 0) {
      // Wait for the tokens of the members' earlier neighbours (their steps ran
      // in earlier passes, on any workgroup of the team; their R rows are then
      // complete), and with the layer-0 table pick each slot's table row from
      // the neighbour's token.
      constexpr bool kTab = PREC == kPrecFp32 || X3;
      int tid = threadIdx.x;
      asm volatile("" : "+v"(tid));  // keeps these addresses out of loop-invariant (spilled) registers
      static_assert(G * kKmax <= kThreads, "one slot per thread");
      if (tid < ml * kKmax && tid % kKmax < K) {
        const int i = tid / kKmax, k = tid % kKmax;
        const int wd = nbw[tid];
        const bool bw = wd >= 0 && (wd & 0x40000000) != 0;
        const int tok = bw ? await_token(tokens + (wd & 0x3FFFFFFF), a.spin_limit, a.fault, &bad, a.fences) : kV;
        if (kTab && a.l0tab) {
          const int4 m2 = meta2[i];
          if (a.l0base) {  // compact: kV rows for each earlier backward slot, one for any other
            const uint64_t before = ((uint64_t)(uint32_t)m2.x | ((uint64_t)(uint32_t)m2.y << 32)) & ((1ull << k) - 1);
            cls[tid] = m2.z + k + (kV - 1) * __popcll(before) + (bw ? tok : 0);
          } else {
            cls[tid] = m2.z + k * kL0Classes + tok;
          }
        }
      }
      __syncthreads();
      if (bad) break;
      if (kTab && a.l0tab) {
        // x[i] = sum over slots of table rows, in the order of the MFMA path
        // below: lane group g (rows 16 mb + 4 g + e, mb outer) sums its rows,
        // then the four groups add as (g0 + g1) + (g2 + g3).
        // The twelve row-index reads, then the twelve row loads, are issued before
        // the first use of each. Rows >= K (short chains) load row K - 1 and are
        // masked to +0 (an AND rather than a select, which the compiler would
        // turn into a branch around each load). Indices fit 32 bits (the table
        // is at most 4 GiB).
        // Members in rounds of four (128 threads each).
        static_assert(kThreads == 512, "table sum mapping");
        const int gq = (tid >> 5) & 3, q = tid & 31;
#pragma unroll 1
        for (int i = tid >> 7; i < ml; i += 4) {
          const float* tb = a.l0tab + 4u * q;
          int cl[12];  // table rows
#pragma unroll
          for (int n = 0; n < 12; ++n) cl[n] = cls[i * kKmax + min((n / 4) * 16 + 4 * gq + (n % 4), K - 1)];
          float4 v[12];
#pragma unroll
          for (int n = 0; n < 12; ++n) v[n] = *reinterpret_cast<const float4*>(tb + (uint32_t)cl[n] * (uint32_t)kH);
#pragma unroll
          for (int n = 0; n < 12; ++n) {
            const uint32_t keep = (n / 4) * 16 + 4 * gq + (n % 4) < K ? ~0u : 0u;
            v[n] = make_float4(__uint_as_float(__float_as_uint(v[n].x) & keep), __uint_as_float(__float_as_uint(v[n].y) & keep),
                               __uint_as_float(__float_as_uint(v[n].z) & keep), __uint_as_float(__float_as_uint(v[n].w) & keep));
          }
          float4 sum = make_float4(0.F, 0.F, 0.F, 0.F);
#pragma unroll
          for (int n = 0; n < 12; ++n) {
            sum.x += v[n].x;
            sum.y += v[n].y;
            sum.z += v[n].z;
            sum.w += v[n].w;
          }
          *reinterpret_cast<float4*>(ff + (i * 4 + gq) * kH + 4 * q) = sum;
          if constexpr (G <= 4) break;  // one round
        }
        __syncthreads();
        for (int task = threadIdx.x; task < ml * kH; task += kThreads) {
          const int im = task / kH, c = task % kH;
          const float* f = ff + im * 4 * kH + c;
          x[task] = (f[0] + f[kH]) + (f[2 * kH] + f[3 * kH]);
          if constexpr (X3) put_split16<PREC>(xs16 + task, G * kH, x[task]);  // W3's input on the MFMA
        }
        __syncthreads();
      }

      // Message-row gathers of members i0, i0 + 1 in layer ll (E1_tk and the R or Q
      // row of each slot's neighbour). Every row is known when the pass starts (R
      // rows of earlier passes), so the first pair of layer l + 1 is gathered
      // during layer l's LayerNorm and fused product, and its latency is hidden.
      constexpr bool kPipe = H16;
      constexpr int kS = 2 * kKmax / 16;
      static_assert(kKmax == 48 && kThreads == 512, "row mapping");
      const int c = 4 * (threadIdx.x & 31);
      const int r0 = threadIdx.x >> 5;
      // 16-bit modes: fp16 inputs, held raw (four per 8 bytes) until all loads are issued
      using Raw = typename std::conditional<H16, uint64_t, float4>::type;
      Raw e[kS], z[kS];
      auto gather = [&](int ll, int i0) {
          // The slots' neighbour words and the two residues are read from LDS
          // first, so that the row loads below issue back to back (read one
          // slot at a time, every load waited for its own LDS reads).
          int wd[kS];
          const int t0 = meta[min(i0, G - 1)].x, t1 = meta[min(i0 + 1, G - 1)].x;
#pragma unroll
          for (int s = 0; s < kS; ++s) {
            const int i = i0 + s / 3, k = 16 * (s % 3) + r0;  // k < kKmax
            wd[s] = nbw[min(i, G - 1) * kKmax + k] | ((i < ml && k < K) ? 0 : -1);
          }
#pragma unroll
          for (int s = 0; s < kS; ++s) {
            const int k = 16 * (s % 3) + r0;
            const size_t tk = (size_t)(s < 3 ? t0 : t1) * K + k;
            e[s] = Raw{};
            z[s] = e[s];
            if (wd[s] >= 0) {
              const int j = wd[s] & 0x3FFFFFFF;
              const bool bw = (wd[s] & 0x40000000) != 0;
              // z: the R row (written by the team) or the Q row, both read with a
              // device-scope load; one load per slot (two exec-masked loads into
              // one register set were issued one after the other)
              if constexpr (H16) {
                e[s] = *reinterpret_cast<const uint64_t*>(a.E1h + ((size_t)ll * S + tk) * kH + c);
                z[s] = load8_dev((bw ? Rh : a.Qh) + ((size_t)ll * L + j) * kH + c);
              } else {
                e[s] = *reinterpret_cast<const float4*>(a.E1 + ((size_t)ll * S + tk) * kH + c);
                z[s] = load4_dev((bw ? R : a.Q) + ((size_t)ll * L + j) * kH + c);
              }
            }
          }
      };
      // The first pair of layer l + 1 is gathered during layer l (kPrefetch); in
      // the fp32 kernel its registers would be spilled, so there it is gathered
      // where it is used.
      constexpr bool kPrefetch = H16;
      if (kPrefetch) gather(0, 0);
      for (int l = 0; l < kLayers; ++l) {
        const DecLayerDev& w = m.dec[l];
        // Layer 0 of the fp32 and split bf16 decodes reads its message rows from the table.
        const bool from_tab = (PREC == kPrecFp32 || X3) && l == 0 && a.l0tab != nullptr;
        const float* pl = prm + l * kPrmLayer;
        if (!from_tab) {  // else x holds the layer-0 message sums (table, above)
          // Message rows g1 = GELU(A + E1_tk + (bw ? R : Q)_j), two members at a time;
          // rows >= K are zero. Thread owns columns c..c+3 of rows r0 + 16 s
          // (member i0 + s / 3, slot 16 (s % 3) + r0); all gathers of a pair are
          // issued before the first use, and the next pair's once this pair's rows
          // are in G16, so that their latency overlaps this pair's product. In the
          // 16-bit modes the rows of all four members fit in G16 (one 16-bit copy
          // each); otherwise G16 holds one pair (hi and lo rows) at a time.
          // With kPrefetch the first pair's gathers are in flight already (issued
          // before the loop for layer 0, during the previous layer otherwise).
          if (!kPrefetch) gather(l, 0);
          // W2 fragments of this wave's 16 columns stay in registers for all members.
          const int r = lane & 15, g = lane >> 4;
          const int col = wave * 16 + r;
          // B fragments of the 16x16x32 MFMA: column col, k = 32 kb + 8 g + 0..7
          half8 bh[kH / 32], bl[kH / 32];
          bf16x8 bb[kH / 32], bbl[kH / 32];
#pragma unroll
          for (int kb = 0; kb < kH / 32; ++kb) {
            const size_t at = ((size_t)(4 * kb + g) * kH + col) * 4;  // float slots of 8 halves
            if constexpr (BF || X3) {
              bb[kb] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const float4*>(w.W2_b + 2 * at));
              if constexpr (X3) bbl[kb] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const float4*>(w.W2_bl + 2 * at));
            } else {
              bh[kb] = __builtin_bit_cast(half8, *reinterpret_cast<const float4*>(w.W2h + at));
              if constexpr (!HF) bl[kb] = __builtin_bit_cast(half8, *reinterpret_cast<const float4*>(w.W2l + at));
            }
          }
          const float b2 = pl[kPrmB2 + col];
          for (int i0 = 0; i0 < ml; i0 += 2) {
            {
#pragma unroll
              for (int s = 0; s < kS; ++s) {
                const int i = i0 + s / 3, k = 16 * (s % 3) + r0;
                if (i < ml) {
                  float4 ev, zv;
                  if constexpr (H16) {
                    ev = widen_h4(e[s]);
                    zv = widen_h4(z[s]);
                  } else {
                    ev = e[s];
                    zv = z[s];
                  }
                  float4 xv = *reinterpret_cast<const float4*>(hA + i * kH + c);
                  xv.x += ev.x + zv.x;
                  xv.y += ev.y + zv.y;
                  xv.z += ev.z + zv.z;
                  xv.w += ev.w + zv.w;
                  float4 v = make_float4(gelu_poly(xv.x, gtab), gelu_poly(xv.y, gtab), gelu_poly(xv.z, gtab),
                                         gelu_poly(xv.w, gtab));
                  if (k >= K) v = make_float4(0.F, 0.F, 0.F, 0.F);
                  _Float16* gh = G16 + ((kPipe ? i : (s / 3) * 2) * kKmax + k) * kLdH + c;  // 16-bit: slot = member
                  const float vv[4] = {v.x, v.y, v.z, v.w};
                  if constexpr (BF) {
                    bf16x4 bv;
#pragma unroll
                    for (int e = 0; e < 4; ++e) bv[e] = static_cast<__bf16>(vv[e]);
                    *reinterpret_cast<bf16x4*>(gh) = bv;
                  } else if constexpr (HF) {
                    half4 hv;
#pragma unroll
                    for (int e = 0; e < 4; ++e) hv[e] = static_cast<_Float16>(__builtin_amdgcn_fmed3f(vv[e], -65504.0F, 65504.0F));
                    *reinterpret_cast<half4*>(gh) = hv;
                  } else if constexpr (X3) {
                    // split for the bf16 MFMA: v = hi + lo, lo = bf16(v - hi), to about 2^-16 relative
                    bf16x4 hv, lv;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                      hv[e] = static_cast<__bf16>(vv[e]);
                      lv[e] = static_cast<__bf16>(vv[e] - static_cast<float>(hv[e]));
                    }
                    *reinterpret_cast<bf16x4*>(gh) = hv;
                    *reinterpret_cast<bf16x4*>(gh + kKmax * kLdH) = lv;
                  } else {
                    // split for the fp16 MFMA: v = hi + lo / 2048 to about 2^-22 relative
                    _Float16* gl = gh + kKmax * kLdH;
                    half4 hv, lv;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                      const float cl = __builtin_amdgcn_fmed3f(vv[e], -65504.0F, 65504.0F);
                      hv[e] = static_cast<_Float16>(cl);
                      lv[e] = static_cast<_Float16>((vv[e] - static_cast<float>(hv[e])) * 2048.0F);
                    }
                    *reinterpret_cast<half4*>(gh) = hv;
                    *reinterpret_cast<half4*>(gl) = lv;
                  }
                }
              }
            }
            __syncthreads();
            if (i0 + 2 < ml) gather(l, i0 + 2);
            for (int i = i0; i < ml && i < i0 + 2; ++i) {
              const _Float16* Gh = kPipe ? G16 + i * kKmax * kLdH : G16 + (i - i0) * 2 * kKmax * kLdH;
              const _Float16* Gl = Gh + kKmax * kLdH;
              // W2 product: hi.hi + (hi.lo + lo.hi) / 2048 on the fp16 MFMA, or bf16 x bf16
              floatx4 acc[3], cor[3];
#pragma unroll
              for (int mb = 0; mb < 3; ++mb) {
                acc[mb] = floatx4{0.F, 0.F, 0.F, 0.F};
                cor[mb] = acc[mb];
              }
              // A operands of k-block kb for the three row blocks, double buffered:
              // the next block's LDS reads are issued before this block's products.
              using AOp = typename std::conditional<BF || X3, bf16x8, half8>::type;
              AOp ah[2][3], al[2][3];
              auto aload = [&](int kb, int buf) {
#pragma unroll
                for (int mb = 0; mb < 3; ++mb) {
                  const int at = (mb * 16 + r) * kLdH + 32 * kb + 8 * g;
                  ah[buf][mb] = *reinterpret_cast<const AOp*>(Gh + at);
                  if constexpr (PREC == kPrecFp32 || X3) al[buf][mb] = *reinterpret_cast<const AOp*>(Gl + at);
                }
              };
              aload(0, 0);
#pragma unroll
              for (int kb = 0; kb < kH / 32; ++kb) {
                if (kb + 1 < kH / 32) aload(kb + 1, (kb + 1) & 1);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int mb = 0; mb < 3; ++mb) {
                  const AOp& a0 = ah[kb & 1][mb];
                  if constexpr (BF) {
                    acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, bb[kb], acc[mb], 0, 0, 0);
                  } else if constexpr (X3) {
                    acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, bb[kb], acc[mb], 0, 0, 0);
                    cor[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, bbl[kb], cor[mb], 0, 0, 0);
                    cor[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[kb & 1][mb], bb[kb], cor[mb], 0, 0, 0);
                  } else if constexpr (HF) {
                    acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, bh[kb], acc[mb], 0, 0, 0);
                  } else {
                    acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, bh[kb], acc[mb], 0, 0, 0);
                    cor[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, bl[kb], cor[mb], 0, 0, 0);
                    cor[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[kb & 1][mb], bh[kb], cor[mb], 0, 0, 0);
                  }
                }
              }
              if constexpr (PREC == kPrecFp32) {
#pragma unroll
                for (int mb = 0; mb < 3; ++mb)
#pragma unroll
                  for (int e = 0; e < 4; ++e) acc[mb][e] += cor[mb][e] * (1.0F / 2048.0F);
              } else if constexpr (X3) {
#pragma unroll
                for (int mb = 0; mb < 3; ++mb)
#pragma unroll
                  for (int e = 0; e < 4; ++e) acc[mb][e] += cor[mb][e];
              }
              // x[i][col] = sum over the member's K rows of GELU(acc + b2)
              float sum = 0.0F;
#pragma unroll
              for (int mb = 0; mb < 3; ++mb)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                  const int row = mb * 16 + 4 * g + e;
                  const float gv = gelu_poly(acc[mb][e] + b2, gtab);
                  sum += row < K ? gv : 0.0F;
                }
              sum += __shfl_xor(sum, 16, 64);
              sum += __shfl_xor(sum, 32, 64);
              if (lane < 16) {
                x[i * kH + col] = sum;
                if constexpr (M16) put_split16<PREC>(xs16 + i * kH + col, G * kH, sum);
              }
            }
            if constexpr (!kPipe) __syncthreads();
          }
          if constexpr (kPipe) __syncthreads();
        }
        if constexpr (M16) {
          // 16-bit modes: the four products on the MFMA (MGemv), inputs from the
          // split copies, outputs in ys. Weights in bf16 (bf16 and split bf16,
          // with the remainders of the latter) or fp16. The split bf16 mode holds
          // twice the fragments per k-block, so its products take more, smaller
          // parts, each loaded while the part before it runs.
          constexpr int kNpIn = X3 ? 4 : 1, kNpOut = X3 ? 8 : 2, kNpDa = X3 ? 2 : 1;
          using M3 = MGemv<kH, kH, 1, PREC>;
          using MIn = MGemv<kH, kFF, kNpIn, PREC>;
          using MOut = MGemv<kFF, kH, kNpOut, PREC>;
          using MDa = MGemv<kH, 2 * kH, kNpDa, PREC>;
          const auto wsel = [](const uint16_t* h16, const uint16_t* f16) { return HF ? f16 : h16; };
          // upd = (W3 s + K b3) / 30 ; h1 = LN1(h + upd): wave i owns member i
          {
            typename M3::Part g3;
            M3::load(g3, wsel(w.W3_h, w.W3_f), w.W3_hl, 0);
            typename M3::Acc a3;
            M3::zero(a3);
            M3::run(g3, 0, xs16, ml, a3);
            M3::store(a3, ml, ys);
          }
          typename MIn::Part pin[2];  // first part of W_in in flight during LN1
          MIn::load(pin[0], wsel(w.Win_h, w.Win_f), w.Win_hl, 0);
          __syncthreads();
          if (wave < ml) {
            float v[2];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
              const int c = lane + 64 * hh;
              v[hh] = h[wave * kH + c] + (ys[wave * kH + c] + static_cast<float>(K) * pl[kPrmB3 + c]) * (1.0F / 30.0F);
            }
            ln_regs_wave(v[0], v[1], pl + kPrmN1g, pl + kPrmN1b, h1 + wave * kH);
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
              const int c = lane + 64 * hh;
              put_split16<PREC>(h1s16 + wave * kH + c, G * kH, h1[wave * kH + c]);
            }
          }
          __syncthreads();
          // f = GELU(W_in h1 + b)
          typename MOut::Part po[2];  // first part of W_out in flight during W_in and the GELU
          MOut::load(po[0], wsel(w.Wout_h, w.Wout_f), w.Wout_hl, 0);
          {
            typename MIn::Acc ai;
            MIn::zero(ai);
#pragma unroll
            for (int pp = 0; pp < kNpIn; ++pp) {
              if (pp + 1 < kNpIn) MIn::load(pin[(pp + 1) & 1], wsel(w.Win_h, w.Win_f), w.Win_hl, pp + 1);
              MIn::run(pin[pp & 1], pp, h1s16, ml, ai);
            }
            MIn::store(ai, ml, ys);
          }
          __syncthreads();
          for (int task = threadIdx.x; task < ml * kFF; task += kThreads) {
            const int o = task % kFF;
            const float f = gelu_poly(ys[task] + pl[kPrmBin + o], gtab);
            ff[task] = f;
            put_split16<PREC>(ffs16 + task, G * kFF, f);
          }
          __syncthreads();
          // h^{l+1} = LN2(h1 + (W_out f + b)); each next part in flight during the current part's products
          {
            typename MOut::Acc ao;
            MOut::zero(ao);
#pragma unroll
            for (int pp = 0; pp < kNpOut; ++pp) {
              if (pp + 1 < kNpOut) MOut::load(po[(pp + 1) & 1], wsel(w.Wout_h, w.Wout_f), w.Wout_hl, pp + 1);
              MOut::run(po[pp & 1], pp, ffs16, ml, ao);
            }
            MOut::store(ao, ml, ys);
          }
          // the next layer's fused weights during LN2 (a placeholder load in the last layer)
          typename MDa::Part pda[2];
          const bool nxt = l + 1 < kLayers;
          const DecLayerDev& nx = m.dec[nxt ? l + 1 : l];
          MDa::load(pda[0], wsel(nx.W1da_h, nx.W1da_f), nx.W1da_hl, 0, nxt ? 1 : 0);
          if (kPrefetch && l + 1 < kLayers) gather(l + 1, 0);  // the next layer's first pair
          __syncthreads();
          if (wave < ml) {
            float v[2];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
              const int c = lane + 64 * hh;
              v[hh] = h1[wave * kH + c] + (ys[wave * kH + c] + pl[kPrmBout + c]);
            }
            ln_regs_wave(v[0], v[1], pl + kPrmN2g, pl + kPrmN2b, h + wave * kH);
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
              const int c = lane + 64 * hh;
              put_split16<PREC>(hs16 + wave * kH + c, G * kH, h[wave * kH + c]);
            }
          }
          __syncthreads();
          if (l + 1 < kLayers) {
            // fused [W1d | W1a] of the next layer (see the fp32 branch)
            {
              typename MDa::Acc ad;
              MDa::zero(ad);
#pragma unroll
              for (int pp = 0; pp < kNpDa; ++pp) {
                if (pp + 1 < kNpDa) MDa::load(pda[(pp + 1) & 1], wsel(nx.W1da_h, nx.W1da_f), nx.W1da_hl, pp + 1);
                MDa::run(pda[pp & 1], pp, hs16, ml, ad);
              }
              MDa::store(ad, ml, ys);
            }
            __syncthreads();
            for (int task = threadIdx.x; task < ml * kH; task += kThreads) {
              const int i = task / kH, c = task % kH;
              Pd[(i * 2 + l) * kH + c] = ys[i * 2 * kH + c];
              hA[task] = ys[i * 2 * kH + kH + c] + pl[kPrmLayer + kPrmB1 + c];
            }
            __syncthreads();
          }
        } else {
          // upd = (W3 s + K b3) / 30 ; h1 = LN1(h + upd): wave i owns member i
          // (W3 loads here: issued during the message rows they competed with the gathers and cost spills)
          typename G3::Part g3;
          G3::load(g3, (BF ? static_cast<const void*>(w.W3_h) : HF ? static_cast<const void*>(w.W3_f) : w.W3_t), 0);
          // The products accumulate kGroup members at a time: chunk i0 holds members
          // i0 .. i0 + n - 1 (each member's sums are the same whatever the chunk; one
          // chunk when G <= kGroup).
          float4 acc[kGroup];
          const int chunk_end = G <= kGroup ? 1 : ml;
          for (int i0 = 0; i0 < chunk_end; i0 += kGroup) {
            const int n = G <= kGroup ? ml : min(kGroup, ml - i0);
            zero4(acc);
            G3::fma(g3, 0, x + i0 * kH, n, acc);
            G3::store(acc, n, part + i0 * G3::GROUPS * kH);
          }
          typename GIn::Part in0;  // first half of W_in in flight during the reduction and LN1
          GIn::load(in0, (BF ? static_cast<const void*>(w.Win_h) : HF ? static_cast<const void*>(w.Win_f) : w.Win_t), 0);
          __syncthreads();
          if (wave < ml) {
            float v[2];
  #pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
              const int c = lane + 64 * hh;
              v[hh] = h[wave * kH + c] + (G3::sum(part, wave, c) + static_cast<float>(K) * pl[kPrmB3 + c]) * (1.0F / 30.0F);
            }
            ln_regs_wave(v[0], v[1], pl + kPrmN1g, pl + kPrmN1b, h1 + wave * kH);
          }
          __syncthreads();
          // f = GELU(W_in h1 + b)
          {
            // second half in flight during the first half's FMAs
            typename GIn::Part in1;
            GIn::load(in1, (BF ? static_cast<const void*>(w.Win_h) : HF ? static_cast<const void*>(w.Win_f) : w.Win_t), 1);
            for (int i0 = 0; i0 < chunk_end; i0 += kGroup) {
              const int n = G <= kGroup ? ml : min(kGroup, ml - i0);
              zero4(acc);
              GIn::fma(in0, 0, h1 + i0 * kH, n, acc);
              GIn::fma(in1, 1, h1 + i0 * kH, n, acc);
              GIn::store(acc, n, part + i0 * GIn::GROUPS * kFF);
            }
          }
          typename GOut::Part out0;  // first half of W_out in flight during the reduction and GELU
          GOut::load(out0, (BF ? static_cast<const void*>(w.Wout_h) : HF ? static_cast<const void*>(w.Wout_f) : w.Wout_t), 0);
          __syncthreads();
          for (int task = threadIdx.x; task < ml * kFF; task += kThreads) {
            const int i = task / kFF, o = task % kFF;
            ff[task] = gelu_poly(GIn::sum(part, i, o) + pl[kPrmBin + o], gtab);
          }
          __syncthreads();
          // h^{l+1} = LN2(h1 + (W_out f + b)) (the mask gate is 1 for an active residue)
          {
            typename GOut::Part out1;  // second half in flight during the first half's FMAs
            GOut::load(out1, (BF ? static_cast<const void*>(w.Wout_h) : HF ? static_cast<const void*>(w.Wout_f) : w.Wout_t), 1);
            for (int i0 = 0; i0 < chunk_end; i0 += kGroup) {
              const int n = G <= kGroup ? ml : min(kGroup, ml - i0);
              zero4(acc);
              GOut::fma(out0, 0, ff + i0 * kFF, n, acc);
              GOut::fma(out1, 1, ff + i0 * kFF, n, acc);
              GOut::store(acc, n, part + i0 * GOut::GROUPS * kH);
            }
          }
          // The next layer's fused weights load during LN2. The last layer issues
          // the same loads with every lane on one 16-byte slice (unused; an L1 hit):
          // an unconditional load keeps the register budget, and a full-size one
          // would hold the logits behind its 128 KB of L2 traffic.
          typename GDa::Part da;
          {
            const bool nxt = l + 1 < kLayers;
            const DecLayerDev& nx = m.dec[nxt ? l + 1 : l];
            GDa::load(da, (BF ? static_cast<const void*>(nx.W1da_h) : HF ? static_cast<const void*>(nx.W1da_f) : nx.W1da_t), 0,
                      nxt ? 1 : 0);
          }
          if (kPrefetch && l + 1 < kLayers) gather(l + 1, 0);  // the next layer's first pair
          __syncthreads();
          if (wave < ml) {
            float v[2];
  #pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
              const int c = lane + 64 * hh;
              v[hh] = h1[wave * kH + c] + (GOut::sum(part, wave, c) + pl[kPrmBout + c]);
            }
            ln_regs_wave(v[0], v[1], pl + kPrmN2g, pl + kPrmN2b, h + wave * kH);
          }
          __syncthreads();
          if (l + 1 < kLayers) {
            // fused [W1d | W1a] of the next layer: W1d h is kept for R (completed with
            // T[tok] after sampling), W1a h + b1 is the next A.
            for (int i0 = 0; i0 < chunk_end; i0 += kGroup) {
              const int n = G <= kGroup ? ml : min(kGroup, ml - i0);
              zero4(acc);
              GDa::fma(da, 0, h + i0 * kH, n, acc);
              GDa::store(acc, n, part + i0 * GDa::GROUPS * 2 * kH);
            }
            __syncthreads();
            for (int task = threadIdx.x; task < ml * kH; task += kThreads) {
              const int i = task / kH, c = task % kH;
              Pd[(i * 2 + l) * kH + c] = GDa::sum(part, i, c);
              hA[task] = GDa::sum(part, i, kH + c) + pl[kPrmLayer + kPrmB1 + c];
            }
            __syncthreads();
          }
        }
      }
#pragma unroll
      for (int q = 0; q < kRecRounds; ++q) rv[q] = rec_load(s0n, mln, q);  // in flight during logits and sampling
      staged = true;
      // Wave i computes member i's logits = W_out h + b and draws its token:
      // lane v + 32 kh sums inputs [64 kh, 64 kh + 64) of output v (weights
      // from LDS), and the two halves add across the wave.
      if (wave < ml) {
        const int i = wave;
        const int v = lane & 31, kh = lane >> 5;
        const float4* wr = reinterpret_cast<const float4*>(wlg) + kh * 16 * 32 + v;
        const float4* hr = reinterpret_cast<const float4*>(h + i * kH) + kh * 16;
        float4 s4 = make_float4(0.F, 0.F, 0.F, 0.F);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          // eight reads of each operand in flight before their FMAs (the
          // scheduler otherwise waits for every read)
          float4 wv[8], hv[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            wv[u] = wr[(8 * kb + u) * 32];
            hv[u] = hr[8 * kb + u];
          }
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            s4.x += hv[u].x * wv[u].x;
            s4.y += hv[u].y * wv[u].y;
            s4.z += hv[u].z * wv[u].z;
            s4.w += hv[u].w * wv[u].w;
          }
        }
        float lsum = (s4.x + s4.y) + (s4.z + s4.w);
        lsum += __shfl_xor(lsum, 32, 64);
        const float logit = lsum + prm[kPrmLog + v];
        const int4 mt = meta[i];  // residue, draw index, design weight bits, true token
        const int t = mt.x;
        float lpv;
        const uint64_t state = seed + (uint64_t)mt.y * 0x9E3779B97F4A7C15ull;
        const int s_tok = sample_wave(logit, T, greedy, state, &lpv);
        const int tok = __int_as_float(mt.z) == 0.0F ? mt.w : s_tok;
        if (lp_out && lane < kV) lp_out[(size_t)t * kV + lane] = lpv;
        if (lane == tok) store_dev(chosen + t, lpv);
        if (lane == 0) tok_s[i] = tok;
      }
      __syncthreads();
      if constexpr (H16) {  // fp16 rows, two columns per device-scope store
        for (int task = threadIdx.x; task < ml * kLayers * (kH / 2); task += kThreads) {
          const int i = task / (kLayers * kH / 2), l = (task / (kH / 2)) % kLayers, c = 2 * (task % (kH / 2));
          const int t = meta[i].x;
          const float* base = (l == 0) ? q0s + i * kH + c : Pd + (i * 2 + l - 1) * kH + c;
          const float* tv = m.dec[l].T + tok_s[i] * kH + c;
          store_dev(reinterpret_cast<int32_t*>(Rh + ((size_t)l * L + t) * kH + c), pack_h2(base[0] + tv[0], base[1] + tv[1]));
        }
      } else {
        for (int task = threadIdx.x; task < ml * kLayers * kH; task += kThreads) {
          const int i = task / (kLayers * kH), l = (task / kH) % kLayers, c = task % kH;
          const int t = meta[i].x;
          const float base = (l == 0) ? q0s[i * kH + c] : Pd[(i * 2 + l - 1) * kH + c];
          store_dev(R + ((size_t)l * L + t) * kH + c, base + m.dec[l].T[tok_s[i] * kH + c]);
        }
      }
      // The tokens last: every wave's R-row stores have completed at the device
      // coherence point before a member's token is stored (await_token).
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (threadIdx.x < ml) {
        if (a.fences) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        store_dev(tokens + meta[threadIdx.x].x, tok_s[threadIdx.x]);
      }
    }
    if (!staged)
#pragma unroll
      for (int q = 0; q < kRecRounds; ++q) rv[q] = rec_load(s0n, mln, q);
    __syncthreads();  // this pass's LDS state is consumed
#pragma unroll
    for (int q = 0; q < kRecRounds; ++q) rec_store(mln, rv[q], q);
    ml = mln;
    __syncthreads();
  }
  // The chosen log-probs of every member are in place before rank 0 sums them;
  // a workgroup that stopped early marks the count so that rank 0 leaves a NaN score.
  if (P > 1) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
      if (a.fences) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
      __hip_atomic_fetch_add(counter, bad ? 1u + kTeamAbort : 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (rank == 0 && !bad) {
      if (!team_wait(counter, 2 * P, a.spin_limit, a.fault, &bad, a.fences)) goto finish;
      if (threadIdx.x == 0 && __hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= kTeamAbort) bad = 1;
      __syncthreads();
    }
  }
finish:
  // Mean NLL over designed residues in residue order (inverse_fold_scalar.cpp:471-493).
  if (a.scores && rank == 0 && threadIdx.x == 0) {
    if (bad) {
      a.scores[b] = __builtin_nanf("");
      return;
    }
    double loss = 0.0, msum = 0.0;
    for (int r = 0; r < L; ++r) {
      const float act = (a.chain_mask ? a.chain_mask[r] : 1.0F) * a.mask[r];
      if (act == 0.0F) continue;
      loss -= static_cast<double>(load_dev(chosen + r));
      msum += static_cast<double>(act);
    }
    a.scores[b] = msum > 0.0 ? static_cast<float>(loss / msum) : 0.0F;
  }
}

// Layer-0 message table (launch_layer0_table): workgroup (t, y) writes the
// rows of slots [kTabSlots y, kTabSlots y + kTabSlots) of residue t, all
// classes, 48 rows at a time. Each row repeats the decode loop's fp32 steps
// for a slot whose neighbour is in that class (decode_kernel, PREC = fp32):
// the pre-activation hA + (E1 + z) with z = Q^0_j + T_0[c] for a neighbour
// decoded with token c (the R^0_j row its writer stores), z = Q^0_j
// otherwise and e = z = 0 for an empty slot; GELU and the hi/lo split into
// the same LDS layout; the same MFMA operands and order; GELU(acc + b2).
constexpr int kTabSlots = 12;  // 4 workgroups per residue: 73 us against 79 us with 24 slots at L = 300
// Rows of slot k of residue t in the compact table: the kV token states when its
// neighbour is decoded before t in the shared order, else its one state.
__device__ inline int l0_slot_rows(const int32_t* __restrict__ idx, const int32_t* __restrict__ pos, int L, int K,
                                   int t, int k) {
  const int j = idx[(size_t)t * K + k];
  return (j >= 0 && j < L && pos[j] < pos[t]) ? kV : 1;
}

// Compact-table row offsets (launch_l0_rows): one workgroup; every residue's
// row count goes to LDS (residues strided over the threads), then thread i
// scans a contiguous run of residues and a block scan gives each run's start.
constexpr int kL0RowsThreads = 1024;
constexpr int kL0RowsMaxL = 8192;  // the table is used while it takes <= 4 GiB: L <= 7,943
__global__ __launch_bounds__(kL0RowsThreads) void l0_rows_kernel(const int32_t* __restrict__ idx,
                                                                 const int32_t* __restrict__ pos, int L, int K,
                                                                 int32_t* __restrict__ base) {
  __shared__ int cnt[kL0RowsMaxL];
  __shared__ int run[kL0RowsThreads];
  for (int t = threadIdx.x; t < L; t += kL0RowsThreads) {
    int n = 0;
    for (int k = 0; k < K; ++k) n += l0_slot_rows(idx, pos, L, K, t, k);
    cnt[t] = n;
  }
  __syncthreads();
  const int per = (L + kL0RowsThreads - 1) / kL0RowsThreads;
  const int t0 = min(L, (int)threadIdx.x * per), t1 = min(L, t0 + per);
  int sum = 0;
  for (int t = t0; t < t1; ++t) sum += cnt[t];
  run[threadIdx.x] = sum;
  __syncthreads();
  for (int d = 1; d < kL0RowsThreads; d <<= 1) {  // inclusive scan
    const int v = threadIdx.x >= (unsigned)d ? run[threadIdx.x - d] : 0;
    __syncthreads();
    run[threadIdx.x] += v;
    __syncthreads();
  }
  int at = run[threadIdx.x] - sum;
  for (int t = t0; t < t1; ++t) {
    base[t] = at;
    at += cnt[t];
  }
  if (threadIdx.x == kL0RowsThreads - 1) base[L] = run[threadIdx.x];
}

__global__ __launch_bounds__(kThreads, 4) void layer0_table_kernel(ModelDev m, const float* __restrict__ E1,
                                                                  const float* __restrict__ Q,
                                                                  const int32_t* __restrict__ idx,
                                                                  const int32_t* __restrict__ pos,
                                                                  const int32_t* __restrict__ base, int L, int K,
                                                                  float* __restrict__ tab) {
  __shared__ __attribute__((aligned(16))) _Float16 G16[2 * kKmax * kLdH];  // hi rows, then lo rows
  __shared__ __attribute__((aligned(16))) float es[kTabSlots * kH];          // E1_tk
  __shared__ __attribute__((aligned(16))) float qs[kTabSlots * kH];          // Q^0_j
  __shared__ __attribute__((aligned(16))) float ts[kV * kH];                 // T_0
  __shared__ __attribute__((aligned(16))) float hA[kH];
  __shared__ __attribute__((aligned(16))) float gtab[kGeluPolyLds];
  __shared__ int js[kTabSlots];
  __shared__ int srows[kKmax + 1];  // rows of each slot of t, then (thread 0) their running start
  __shared__ int16_t rslot[kTabSlots * kL0Classes], rcls[kTabSlots * kL0Classes];  // row -> (slot, state)
  const int t = blockIdx.x;
  const int k0 = blockIdx.y * kTabSlots;
  const int nk = min(kTabSlots, K - k0);
  if (t >= L || nk <= 0) return;
  const DecLayerDev& w = m.dec[0];
  load_gelu_poly(gtab, threadIdx.x, kThreads);
  for (int i = threadIdx.x; i < kH; i += kThreads) hA[i] = Q[((size_t)3 * L + t) * kH + i] + w.b1[i];
  if (threadIdx.x < nk) {
    const int jj = idx[(size_t)t * K + k0 + threadIdx.x];
    js[threadIdx.x] = (jj >= 0 && jj < L) ? jj : -1;
  }
  if (threadIdx.x < K) srows[threadIdx.x] = base ? l0_slot_rows(idx, pos, L, K, t, threadIdx.x) : kL0Classes;
  for (int i = threadIdx.x; i < kV * kH; i += kThreads) ts[i] = w.T[i];
  __syncthreads();
  if (threadIdx.x == 0) {  // exclusive running start of every slot (srows[K] = the residue's row count)
    int at = 0;
    for (int k = 0; k < K; ++k) {
      const int n = srows[k];
      srows[k] = at;
      at += n;
    }
    srows[K] = at;
  }
  __syncthreads();
  // this block's rows: slot k0 + s owns rows [srows[k0 + s], srows[k0 + s + 1]) of the residue
  if (threadIdx.x < nk) {
    const int s = threadIdx.x, r0 = srows[k0 + s] - srows[k0], n = srows[k0 + s + 1] - srows[k0 + s];
    for (int r = 0; r < n; ++r) {
      rslot[r0 + r] = static_cast<int16_t>(s);
      rcls[r0 + r] = static_cast<int16_t>(n == 1 ? kV : r);  // one row: not decoded before t, or empty
    }
  }
  for (int task = threadIdx.x; task < nk * (kH / 4); task += kThreads) {
    const int s = task / (kH / 4), c = 4 * (task % (kH / 4));
    const int j = js[s];
    float4 e = make_float4(0.F, 0.F, 0.F, 0.F), z = e;
    if (j >= 0) {
      e = *reinterpret_cast<const float4*>(E1 + ((size_t)t * K + k0 + s) * kH + c);
      z = *reinterpret_cast<const float4*>(Q + (size_t)j * kH + c);
    }
    *reinterpret_cast<float4*>(es + s * kH + c) = e;
    *reinterpret_cast<float4*>(qs + s * kH + c) = z;
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r = lane & 15, g = lane >> 4;
  const int col = wave * 16 + r;
  half8 bh[kH / 32], bl[kH / 32];
#pragma unroll
  for (int kb = 0; kb < kH / 32; ++kb) {
    const size_t at = ((size_t)(4 * kb + g) * kH + col) * 4;
    bh[kb] = __builtin_bit_cast(half8, *reinterpret_cast<const float4*>(w.W2h + at));
    bl[kb] = __builtin_bit_cast(half8, *reinterpret_cast<const float4*>(w.W2l + at));
  }
  const float b2 = w.b2[col];
  const int rows = srows[k0 + nk] - srows[k0];
  float* out = tab + ((size_t)(base ? base[t] : t * K * kL0Classes) + srows[k0]) * kH;
  __syncthreads();
  for (int r0 = 0; r0 < rows; r0 += kKmax) {
    for (int task = threadIdx.x; task < kKmax * (kH / 4); task += kThreads) {
      const int row = task / (kH / 4), c = 4 * (task % (kH / 4));
      float vv[4] = {0.F, 0.F, 0.F, 0.F};
      if (r0 + row < rows) {
        const int s = rslot[r0 + row], cl = rcls[r0 + row];
        const float4 e = *reinterpret_cast<const float4*>(es + s * kH + c);
        float4 z = *reinterpret_cast<const float4*>(qs + s * kH + c);
        if (js[s] >= 0 && cl < kV) {
          const float4 tv = *reinterpret_cast<const float4*>(ts + cl * kH + c);
          z.x = z.x + tv.x;
          z.y = z.y + tv.y;
          z.z = z.z + tv.z;
          z.w = z.w + tv.w;
        }
        float4 xv = *reinterpret_cast<const float4*>(hA + c);
        xv.x += e.x + z.x;
        xv.y += e.y + z.y;
        xv.z += e.z + z.z;
        xv.w += e.w + z.w;
        vv[0] = gelu_poly(xv.x, gtab);
        vv[1] = gelu_poly(xv.y, gtab);
        vv[2] = gelu_poly(xv.z, gtab);
        vv[3] = gelu_poly(xv.w, gtab);
      }
      half4 hv, lv;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float cl = __builtin_amdgcn_fmed3f(vv[e], -65504.0F, 65504.0F);
        hv[e] = static_cast<_Float16>(cl);
        lv[e] = static_cast<_Float16>((vv[e] - static_cast<float>(hv[e])) * 2048.0F);
      }
      *reinterpret_cast<half4*>(G16 + row * kLdH + c) = hv;
      *reinterpret_cast<half4*>(G16 + (kKmax + row) * kLdH + c) = lv;
    }
    __syncthreads();
    floatx4 acc[3], cor[3];
#pragma unroll
    for (int mb = 0; mb < 3; ++mb) {
      acc[mb] = floatx4{0.F, 0.F, 0.F, 0.F};
      cor[mb] = acc[mb];
    }
#pragma unroll
    for (int kb = 0; kb < kH / 32; ++kb) {
#pragma unroll
      for (int mb = 0; mb < 3; ++mb) {
        const int at = (mb * 16 + r) * kLdH + 32 * kb + 8 * g;
        const half8 ah = *reinterpret_cast<const half8*>(G16 + at);
        const half8 al = *reinterpret_cast<const half8*>(G16 + kKmax * kLdH + at);
        acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh[kb], acc[mb], 0, 0, 0);
        cor[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl[kb], cor[mb], 0, 0, 0);
        cor[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh[kb], cor[mb], 0, 0, 0);
      }
    }
#pragma unroll
    for (int mb = 0; mb < 3; ++mb)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = r0 + mb * 16 + 4 * g + e;
        const float v = acc[mb][e] + cor[mb][e] * (1.0F / 2048.0F);
        if (row < rows) out[(size_t)row * kH + col] = gelu_poly(v + b2, gtab);
      }
    __syncthreads();
  }
}

// Step records (launch_step_records): block (s, q) writes record s of order q.
__global__ __launch_bounds__(128) void step_records_kernel(ModelDev m, DecodeArgs a, float4* __restrict__ rec) {
  const int s = blockIdx.x, q = blockIdx.y, w = threadIdx.x;
  if (w >= kRecFloat4) return;
  const int L = a.L, K = a.K;
  const int32_t* order = a.shared_order ? a.orders : a.orders + (size_t)q * L;
  const int u = a.sched[(size_t)q * L + s];
  const int t = (u >= 0 && u < L) ? order[u] : -1;
  float4 v = make_float4(0.F, 0.F, 0.F, 0.F);
  if (t >= 0 && t < L) {
    if (w < kKmax / 4) {
      int wd[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int k = 4 * w + e;
        wd[e] = -1;
        if (k < K) {
          const size_t at = ((size_t)q * L + u) * K + k;
          const int j = a.nbj[at];
          if (j >= 0) wd[e] = j | (a.nbp[at] < u ? 0x40000000 : 0);
        }
      }
      v = make_float4(__int_as_float(wd[0]), __int_as_float(wd[1]), __int_as_float(wd[2]), __int_as_float(wd[3]));
    } else if (w == kKmax / 4) {
      const int tt = (a.true_tokens && a.true_tokens[t] >= 0 && a.true_tokens[t] < kV) ? a.true_tokens[t] : kV - 1;
      v = make_float4(__int_as_float(t), __int_as_float(a.draw[(size_t)q * L + u]),
                      (a.chain_mask ? a.chain_mask[t] : 1.0F) * a.mask[t], __int_as_float(tt));
    } else if (w == kKmax / 4 + 1) {  // slots decoded before the step (bit k), first layer-0 table row
      uint32_t lo = 0, hi = 0;
      for (int k = 0; k < K; ++k) {
        const size_t at = ((size_t)q * L + u) * K + k;
        if (a.nbj[at] >= 0 && a.nbp[at] < u) {
          if (k < 32)
            lo |= 1u << k;
          else
            hi |= 1u << (k - 32);
        }
      }
      const int row0 = a.l0base ? a.l0base[t] : t * K * kL0Classes;
      v = make_float4(__uint_as_float(lo), __uint_as_float(hi), __int_as_float(row0), 0.F);
    } else if (w >= 16) {
      const int blk = (w - 16) / (kH / 4), c = 4 * ((w - 16) % (kH / 4));
      if (blk == 0) {
        v = *reinterpret_cast<const float4*>(a.h_v + (size_t)t * kH + c);
      } else if (blk == 1) {  // W1a_0 h^0_t + b1_0 (Q block 3)
        const float4 qv = *reinterpret_cast<const float4*>(a.Q + ((size_t)3 * L + t) * kH + c);
        const float* b1 = m.dec[0].b1 + c;
        v = make_float4(qv.x + b1[0], qv.y + b1[1], qv.z + b1[2], qv.w + b1[3]);
      } else {
        v = *reinterpret_cast<const float4*>(a.Q + (size_t)t * kH + c);
      }
    }
  }
  rec[((size_t)q * L + s) * kRecFloat4 + w] = v;
}

// out[c][row][:] = A[row] . Wp(cols 128c..128c+127) for a [M,128] input;
// out_h (if not null) receives blocks c < nh in fp16 (clamped to its range),
// out (if not null) every block in fp32.
constexpr int kGemmRows = 64;
__global__ __launch_bounds__(256) void rows_gemm_kernel(const float* __restrict__ Ain, size_t M,
                                                        const float* __restrict__ Wp, int N,
                                                        float* __restrict__ out, _Float16* __restrict__ out_h,
                                                        int nh) {
  __shared__ __attribute__((aligned(16))) float A[kGemmRows * kLd];
  const size_t row0 = (size_t)blockIdx.x * kGemmRows;
  const int cblk = blockIdx.y;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  for (int task = threadIdx.x; task < kGemmRows * (kH / 4); task += 256) {
    const int row = task / (kH / 4);
    const int c4 = task % (kH / 4);
    float4 v = make_float4(0.F, 0.F, 0.F, 0.F);
    if (row0 + row < M) v = *reinterpret_cast<const float4*>(Ain + (row0 + row) * kH + 4 * c4);
    *reinterpret_cast<float4*>(A + row * kLd + 4 * c4) = v;
  }
  __syncthreads();
  floatx4 acc[4][2];
  zero_acc(acc);
  mfma_tile<4, 2>(A, kLd, Wp, N, cblk * kH + wave * 32, kH, acc);
  float* o = out ? out + (size_t)cblk * M * kH : nullptr;
  _Float16* oh = (out_h && cblk < nh) ? out_h + (size_t)cblk * M * kH : nullptr;
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const size_t row = row0 + mb * 16 + 4 * (lane >> 4) + i;
        const int col = wave * 32 + nb * 16 + (lane & 15);
        if (row >= M) continue;
        if (o) o[row * kH + col] = acc[mb][nb][i];
        if (oh) oh[row * kH + col] = static_cast<_Float16>(__builtin_amdgcn_fmed3f(acc[mb][nb][i], -65504.0F, 65504.0F));
      }
}

__global__ void positions_kernel(const int32_t* __restrict__ orders, int L, int n_orders,
                                 int32_t* __restrict__ pos) {
  const int b = blockIdx.y;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < L; i += gridDim.x * blockDim.x) pos[(size_t)b * L + i] = L;
  __syncthreads();
}

__global__ void scatter_positions_kernel(const int32_t* __restrict__ orders, int L, int32_t* __restrict__ pos) {
  const int b = blockIdx.y;
  const int s = blockIdx.x * blockDim.x + threadIdx.x;
  if (s >= L) return;
  const int r = orders[(size_t)b * L + s];
  if (r >= 0 && r < L) pos[(size_t)b * L + r] = s;
}

// Neighbour lists in decoding order: for step s of order q, slot k holds
// j = idx[order[s], k] and its position pos[j] (-1 and L for an empty slot).
__global__ void neighbour_schedule_kernel(const int32_t* __restrict__ orders, const int32_t* __restrict__ pos,
                                          const int32_t* __restrict__ idx, int L, int K, int32_t* __restrict__ nbj,
                                          int32_t* __restrict__ nbp) {
  const int q = blockIdx.y;
  const size_t n = (size_t)L * K;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const int s = (int)(i / K), k = (int)(i % K);
    const int t = orders[(size_t)q * L + s];
    int j = -1, p = L;
    if (t >= 0 && t < L) {
      const int jj = idx[(size_t)t * K + k];
      if (jj >= 0 && jj < L) {
        j = jj;
        p = pos[(size_t)q * L + jj];
      }
    }
    nbj[(size_t)q * n + i] = j;
    nbp[(size_t)q * n + i] = p;
  }
}

// Dependency schedule of each decoding order q. Step u (residue order[u])
// reads the state of every kNN neighbour decoded before it, so it may run in
// any pass after those steps' passes; each step then sees exactly the inputs
// of sequential decoding, whatever pass it runs in. Pass p takes up to
// max_members of the steps whose earlier active neighbours are all placed in
// passes < p: the smallest u, or, for a team of workgroups, a count balanced
// for the team and the steps on the longest chains first (see
// ready_schedule_kernel). Inactive residues
// (mask 0) read nothing and form pass 0, which runs before all others; entries
// outside 0..L-1 are dropped. If the order is not a permutation (a residue
// repeated), every active step gets a pass of its own, in order, as with
// HKBS_DECODE_SCHEDULE=sequential, and the decode kernel refuses the order.
// Outputs per order: sched [L] (steps grouped by pass, increasing u within a
// pass), pstart [L + 2] (pass p holds sched[pstart[p] .. pstart[p + 1])),
// npass (passes after pass 0), draw [L] (index of the step's sampler draw
// among the active steps: the sampler stream is consumed in order of u) and
// the order's four sched_meta words (word 3 = permutation flag: the decode
// kernel does not decode an order that is not a permutation).
// Four kernels: pending-dependency and dependent counts over all (step, slot)
// pairs; per order the permutation check, draw indices, pass 0 and the
// dependents' offsets; the dependents lists; per order the step heights (for
// balanced passes) and the pass loop, with the pending counts as bytes in LDS.
constexpr int kSchedThreads = 512;
constexpr int kSchedMaxL = 60000;  // pending counts as L bytes of LDS
constexpr int kSchedPrioMaxL = 8192;  // balanced passes up to this length (heights, counts, frontier: 2 L bytes of LDS each)
constexpr int kSchedCand = 1024;      // ready steps a balanced pass chooses from

// Active step u of order q: valid residue with mask != 0.
__device__ inline bool sched_active(const int32_t* order, const float* mask, int L, int u) {
  const int t = order[u];
  return t >= 0 && t < L && mask[t] != 0.0F;
}

// indeg[q][u]: earlier active neighbours of active step u; dcnt[q][p]: later
// active steps that have step p as an earlier neighbour. Both zero on entry.
__global__ void dep_count_kernel(const int32_t* __restrict__ orders, const float* __restrict__ mask,
                                 const int32_t* __restrict__ nbp, int L, int K, int32_t* __restrict__ indeg,
                                 int32_t* __restrict__ dcnt) {
  const int q = blockIdx.y;
  const int32_t* order = orders + (size_t)q * L;
  const int32_t* np = nbp + (size_t)q * L * K;
  const size_t n = (size_t)L * K;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const int u = (int)(i / K);
    const int p = np[i];
    if (p >= u || p < 0 || !sched_active(order, mask, L, u) || !sched_active(order, mask, L, p)) continue;
    atomicAdd(indeg + (size_t)q * L + u, 1);
    atomicAdd(dcnt + (size_t)q * (L + 1) + p, 1);
  }
}

// Block-wide exclusive prefix sum of v over kSchedThreads threads; *total
// receives the sum. Uses 8 words of LDS at tmp; ends with a barrier.
__device__ inline int block_scan(int v, int* tmp, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int inc = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(inc, d, 64);
    if (lane >= d) inc += o;
  }
  if (lane == 63) tmp[wave] = inc;
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kSchedThreads / 64; ++w) {
    const int x = tmp[w];
    before += w < wave ? x : 0;
    all += x;
  }
  *total = all;
  __syncthreads();
  return before + inc - v;
}

// Per order (one block): permutation flag, draw indices, pass 0 (inactive
// steps in order), exclusive offsets of the dependents lists (dcnt -> off, in
// place, off[L] = total) and meta = {permutation, active steps, inactive steps}.
__global__ __launch_bounds__(kSchedThreads) void sched_prep_kernel(const int32_t* __restrict__ orders,
                                                                   const int32_t* __restrict__ pos,
                                                                   const float* __restrict__ mask, int L,
                                                                   int sequential, int32_t* __restrict__ off,
                                                                   int32_t* __restrict__ draw,
                                                                   int32_t* __restrict__ sched,
                                                                   int32_t* __restrict__ pstart,
                                                                   int32_t* __restrict__ meta) {
  __shared__ int tmp[kSchedThreads / 64];
  __shared__ int bad;
  const int q = blockIdx.x;
  const int32_t* order = orders + (size_t)q * L;
  const int32_t* pq = pos + (size_t)q * L;
  int32_t* oq = off + (size_t)q * (L + 1);
  int32_t* dq = draw + (size_t)q * L;
  int32_t* sq = sched + (size_t)q * L;
  if (threadIdx.x == 0) bad = 0;
  __syncthreads();
  for (int u = threadIdx.x; u < L; u += kSchedThreads) {
    const int t = order[u];
    if (t < 0 || t >= L || pq[t] != u) bad = 1;
  }
  __syncthreads();
  const int not_perm = bad;
  int act = 0, inact = 0, deps = 0;
  for (int u0 = 0; u0 < L; u0 += kSchedThreads) {
    const int u = u0 + threadIdx.x;
    const bool valid = u < L && order[u] >= 0 && order[u] < L;
    const bool a = valid && mask[order[u]] != 0.0F;
    const bool z = valid && !a;
    int tot;
    const int ra = block_scan(a ? 1 : 0, tmp, &tot);
    if (u < L) dq[u] = a ? act + ra : -1;
    act += tot;
    const int rz = block_scan(z ? 1 : 0, tmp, &tot);
    if (z) sq[inact + rz] = u;
    inact += tot;
    const int c = u < L ? oq[u] : 0;
    const int rc = block_scan(c, tmp, &tot);
    if (u < L) oq[u] = deps + rc;
    deps += tot;
  }
  if (threadIdx.x == 0) {
    oq[L] = deps;
    int32_t* ps = pstart + (size_t)q * (L + 2);
    ps[0] = 0;
    ps[1] = inact;
    meta[(size_t)q * 4 + 0] = !(not_perm || sequential);
    meta[(size_t)q * 4 + 1] = act;
    meta[(size_t)q * 4 + 2] = inact;
    meta[(size_t)q * 4 + 3] = !not_perm;
  }
}

// dlist[q][off[p] ..]: the later active steps that wait for step p (any order
// inside a list). cur is zero on entry.
__global__ void dep_fill_kernel(const int32_t* __restrict__ orders, const float* __restrict__ mask,
                                const int32_t* __restrict__ nbp, int L, int K, const int32_t* __restrict__ off,
                                int32_t* __restrict__ cur, int32_t* __restrict__ dlist) {
  const int q = blockIdx.y;
  const int32_t* order = orders + (size_t)q * L;
  const int32_t* np = nbp + (size_t)q * L * K;
  const size_t n = (size_t)L * K;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const int u = (int)(i / K);
    const int p = np[i];
    if (p >= u || p < 0 || !sched_active(order, mask, L, u) || !sched_active(order, mask, L, p)) continue;
    const int slot = atomicAdd(cur + (size_t)q * L + p, 1);
    dlist[(size_t)q * L * K + off[(size_t)q * (L + 1) + p] + slot] = u;
  }
}

// Pending count of step u: byte u of the packed LDS words; 0xFF = placed,
// inactive or dropped.
__device__ inline int sched_pending(const uint32_t* w, int u) { return (w[u >> 2] >> (8 * (u & 3))) & 0xFF; }

// Ready steps (pending count 0) among the 8 steps 8 i .. 8 i + 7 as a bit mask
// (bit b: step 8 i + b); words words .. of the count array read as all placed.
__device__ inline uint32_t sched_ready8(const uint32_t* w, int words, int i) {
  const uint32_t a = 2 * i < words ? w[2 * i] : 0xFFFFFFFFu;
  const uint32_t b = 2 * i + 1 < words ? w[2 * i + 1] : 0xFFFFFFFFu;
  uint32_t m = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    m |= (((a >> (8 * k)) & 0xFFu) == 0u ? 1u : 0u) << k;
    m |= (((b >> (8 * k)) & 0xFFu) == 0u ? 1u : 0u) << (4 + k);
  }
  return m;
}

// Height of every active step of one order: 1 + the largest height among the
// later steps that wait for it, 1 when none does (the longest chain of
// dependent steps it starts). Computed in rounds over a frontier list: round r
// gives height r to the steps in its frontier (all of whose dependents have
// heights), then takes them off their own earlier neighbours' counts of
// dependents still without one; a neighbour whose count reaches zero joins the
// next frontier. The first frontier is every active step no step waits for.
// ht[u] = 0xFFFF for an inactive step; outw holds the counts as 16-bit halves;
// list (nact 16-bit entries, L <= kSchedPrioMaxL) receives the frontiers one
// after another. Returns the
// number of rounds, the longest chain. The work is proportional to the
// dependency pairs, not to L per round.
__device__ int sched_heights(const int32_t* order, const float* mask, const int32_t* np, const int32_t* oq,
                             int L, int K, uint16_t* ht, uint32_t* outw, uint16_t* list, int* tmp, int* tail) {
  uint16_t* outc = reinterpret_cast<uint16_t*>(outw);
  for (int u = threadIdx.x; u < L; u += kSchedThreads) {
    const bool a = sched_active(order, mask, L, u);
    ht[u] = a ? 0 : 0xFFFF;
    outc[u] = (uint16_t)(a ? oq[u + 1] - oq[u] : 0);  // < L <= kSchedPrioMaxL
  }
  __syncthreads();
  int n = 0;
  for (int c0 = 0; c0 < L; c0 += kSchedThreads) {
    const int u = c0 + threadIdx.x;
    const bool sink = u < L && ht[u] == 0 && outc[u] == 0;
    int tot;
    const int r = block_scan(sink ? 1 : 0, tmp, &tot);
    if (sink) list[n + r] = (uint16_t)u;
    n += tot;
  }
  if (threadIdx.x == 0) *tail = n;
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int start = 0, end = n, rounds = 0;
  while (start < end) {
    ++rounds;
    for (int i = start + threadIdx.x; i < end; i += kSchedThreads) ht[list[i]] = (uint16_t)rounds;
    // wave w takes the frontier's steps w, w + 8, ...; lane k their slot k (K <= 64)
    for (int i = start + wave; i < end; i += kSchedThreads / 64) {
      const int v = list[i];
      if (lane < K) {
        const int p = np[(size_t)v * K + lane];
        if (p >= 0 && p < v && ht[p] != 0xFFFF) {
          const uint32_t old = atomicSub(outw + (p >> 1), 1u << (16 * (p & 1)));
          if (((old >> (16 * (p & 1))) & 0xFFFFu) == 1u) list[atomicAdd(tail, 1)] = (uint16_t)p;
        }
      }
    }
    __syncthreads();
    start = end;
    end = *tail;
    __syncthreads();  // every thread has read the tail before the next round appends to it
  }
  return rounds;
}

// Per order (one block): the pass loop. Pass p takes ready steps (pending
// count 0), at most max_members, then clears their dependents' counts.
//   - granule <= 1 (or L > kSchedPrioMaxL): the first ready steps in order of
//     u, scanning from the first unplaced one.
//   - granule G > 1 (a team of G workgroups shares each pass, so a pass costs
//     about as much as its share for the busiest workgroup, ceil(m / G)): a
//     step is forced when its height reaches the passes left in the longest
//     chain (deferring it would lengthen the schedule). The pass takes
//     k = max(G floor(n / G), G ceil(f / G), min(n, G)) of its n ready steps
//     (f forced; at most max_members): the k highest, ties to smaller u. It
//     never defers a forced step unless max_members does.
__global__ __launch_bounds__(kSchedThreads) void ready_schedule_kernel(
    const int32_t* __restrict__ orders, const float* __restrict__ mask, const int32_t* __restrict__ nbp, int L,
    int K, int max_members, int granule, const int32_t* __restrict__ indeg, const int32_t* __restrict__ off,
    const int32_t* __restrict__ dlist, const int32_t* __restrict__ draw, const int32_t* __restrict__ meta,
    int32_t* __restrict__ sched, int32_t* __restrict__ pstart, int32_t* __restrict__ npass) {
  // ceil(L / 4) words of pending counts, then (balanced passes) 16-bit heights
  // and dependents' counts, and the 16-bit frontier list of sched_heights,
  // ceil(L / 2) words each
  extern __shared__ __attribute__((aligned(16))) uint32_t pend[];
  __shared__ int tmp[kSchedThreads / 64];
  __shared__ int chosen[256];
  __shared__ int cand[kSchedCand];
  __shared__ int low_s, found_s, tail_s, thr_s, above_s;
  const int q = blockIdx.x;
  const int32_t* order = orders + (size_t)q * L;
  const int32_t* ig = indeg + (size_t)q * L;
  const int32_t* oq = off + (size_t)q * (L + 1);
  const int32_t* dl = dlist + (size_t)q * L * K;
  int32_t* sq = sched + (size_t)q * L;
  int32_t* ps = pstart + (size_t)q * (L + 2);
  const int perm = meta[(size_t)q * 4 + 0], nact = meta[(size_t)q * 4 + 1], n0 = meta[(size_t)q * 4 + 2];
  const int32_t* dq = draw + (size_t)q * L;
  if (!perm) {
    // One pass per active step, in order of u.
    for (int u = threadIdx.x; u < L; u += kSchedThreads) {
      const int d = dq[u];
      if (d >= 0) {
        sq[n0 + d] = u;
        ps[1 + d + 1] = n0 + d + 1;
      }
    }
    if (threadIdx.x == 0) {
      ps[1] = n0;
      npass[q] = nact;
    }
    return;
  }
  const int words = (L + 3) / 4;
  const bool balance = granule > 1 && L <= kSchedPrioMaxL;
  uint16_t* ht = reinterpret_cast<uint16_t*>(pend + words);
  int height = 0;
  if (balance)
    height = sched_heights(order, mask, nbp + (size_t)q * L * K, oq, L, K, ht, pend + words + (L + 1) / 2,
                           reinterpret_cast<uint16_t*>(pend + words + 2 * ((L + 1) / 2)), tmp, &tail_s);
  for (int w = threadIdx.x; w < words; w += kSchedThreads) {
    uint32_t v = 0;
    for (int b = 0; b < 4; ++b) {
      const int u = 4 * w + b;
      const uint32_t c = (u < L && sched_active(order, mask, L, u)) ? (uint32_t)min(ig[u], 254) : 0xFFu;
      v |= c << (8 * b);
    }
    pend[w] = v;
  }
  if (threadIdx.x == 0) low_s = 0;
  __syncthreads();
  int placed = 0, pass = 0, out = n0;
  const int cap = min(max_members, 256);
  while (placed < nact) {
    ++pass;
    int found = 0;
    // Ready steps are found 8 per thread (two words of pending counts), from
    // the first unplaced step on, in order of u.
    if (!balance) {
      for (int c8 = low_s / 8; found < cap && 8 * c8 < L; c8 += kSchedThreads) {
        const int i = c8 + threadIdx.x;
        const uint32_t rdy = sched_ready8(pend, words, i);
        int tot;
        int rank = found + block_scan(__popc(rdy), tmp, &tot);
        for (uint32_t m = rdy; m; m &= m - 1, ++rank)
          if (rank < cap) chosen[rank] = 8 * i + __ffs(m) - 1;
        found = min(cap, found + tot);
      }
    } else {
      // candidates: the first kSchedCand ready steps, in order of u
      const int remaining = height - pass + 1;
      int n = 0, myf = 0, tot;
      for (int c8 = low_s / 8; n < kSchedCand && 8 * c8 < L; c8 += kSchedThreads) {
        const int i = c8 + threadIdx.x;
        const uint32_t rdy = sched_ready8(pend, words, i);
        int rank = n + block_scan(__popc(rdy), tmp, &tot);
        for (uint32_t m = rdy; m; m &= m - 1, ++rank) {
          const int u = 8 * i + __ffs(m) - 1;
          if (rank < kSchedCand) {
            cand[rank] = u;
            myf += (int)ht[u] >= remaining;
          }
        }
        n = min(kSchedCand, n + tot);
      }
      const int G = granule;
      __syncthreads();  // cand complete
      if (n <= 64) {
        // one wave: lane i holds candidate i; its rank orders by height, then u
        if (threadIdx.x < 64) {
          const int lane = threadIdx.x;
          const bool in = lane < n;
          const int u = in ? cand[lane] : 0;
          const int h = in ? (int)ht[u] : -1;
          const int f = __popcll(__ballot(in && h >= remaining));
          const int k = min(max(max(G * (n / G), G * ((f + G - 1) / G)), min(n, G)), min(n, cap));
          bool sel = in;
          if (k < n) {
            int rank = 0;
            for (int j = 0; j < n; ++j) {
              const int hj = __shfl(h, j, 64);
              rank += (hj > h) || (hj == h && j < lane);
            }
            sel = in && rank < k;
          }
          const unsigned long long m = __ballot(sel);
          if (sel) chosen[__popcll(m & ((1ULL << lane) - 1))] = u;
          if (lane == 0) found_s = __popcll(m);
        }
        __syncthreads();
        found = found_s;
      } else {
        block_scan(myf, tmp, &tot);
        const int f = tot;
        int k = max(max(G * (n / G), G * ((f + G - 1) / G)), min(n, G));
        k = min(k, min(n, cap));
        if (k < n) {
          // Threshold height thr: the largest with at least k candidates at or above it, from a
          // histogram of the candidates' heights (in the dependents' counts of sched_heights, free
          // now); thread t holds heights [1 + t C, 1 + (t + 1) C) and finds the crossing in its range.
          uint32_t* histw = pend + words + (L + 1) / 2;
          const uint16_t* hist = reinterpret_cast<const uint16_t*>(histw);  // hist[h - 1]
          for (int i = threadIdx.x; i < (height + 1) / 2; i += kSchedThreads) histw[i] = 0;
          __syncthreads();
          for (int i = threadIdx.x; i < n; i += kSchedThreads) {
            const int h = (int)ht[cand[i]] - 1;
            atomicAdd(histw + (h >> 1), 1u << (16 * (h & 1)));
          }
          __syncthreads();
          const int C = (height + kSchedThreads - 1) / kSchedThreads;
          const int a0 = threadIdx.x * C, a1 = min(a0 + C, height);
          int local = 0;
          for (int i = a0; i < a1; ++i) local += hist[i];
          const int before = block_scan(local, tmp, &tot);
          int above = n - before - local;  // candidates with a histogram index >= a1
          for (int i = a1 - 1; i >= a0; --i) {
            const int higher = above;
            above += hist[i];
            if (above >= k && higher < k) {
              thr_s = i + 1;
              above_s = higher;
            }
          }
          __syncthreads();
          const int thr = thr_s, need = k - above_s;  // candidates at height thr to take, the smallest u first
          // thread t: candidates 2 t and 2 t + 1, so that the scans keep the order of u
          static_assert(kSchedCand <= 2 * kSchedThreads, "two candidates per thread");
          const int i0 = 2 * threadIdx.x;
          const int h0 = i0 < n ? (int)ht[cand[i0]] : 0, h1 = i0 + 1 < n ? (int)ht[cand[i0 + 1]] : 0;
          const int e0 = i0 < n && h0 == thr, e1 = i0 + 1 < n && h1 == thr;
          const int er = block_scan(e0 + e1, tmp, &tot);
          const int s0 = i0 < n && (h0 > thr || (e0 && er < need));
          const int s1 = i0 + 1 < n && (h1 > thr || (e1 && er + e0 < need));
          const int r = block_scan(s0 + s1, tmp, &tot);
          if (s0) chosen[r] = cand[i0];
          if (s1) chosen[r + s0] = cand[i0 + 1];
          found = tot;
        } else {
          for (int i = threadIdx.x; i < k; i += kSchedThreads) chosen[i] = cand[i];
          found = k;
        }
      }
    }
    // The first unplaced step is always ready (its earlier neighbours are all
    // placed); taking it when nothing was found guarantees progress.
    if (found == 0) {
      if (threadIdx.x == 0) chosen[0] = low_s;
      found = 1;
    }
    __syncthreads();
    // chosen[0 .. found) is increasing in u: the pass's members in order.
    for (int i = threadIdx.x; i < found; i += kSchedThreads) {
      const int u = chosen[i];
      sq[out + i] = u;
      atomicOr(pend + (u >> 2), 0xFFu << (8 * (u & 3)));
    }
    if (threadIdx.x == 0) ps[pass] = out;
    // Dependents: wave w takes members w, w + 8, ...; lane j their j-th dependent.
    {
      const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
      for (int i = wave; i < found; i += kSchedThreads / 64) {
        const int u = chosen[i];
        const int b = oq[u], e = oq[u + 1];
        for (int j = b + lane; j < e; j += 64) {
          const int v = dl[j];
          atomicSub(pend + (v >> 2), 1u << (8 * (v & 3)));
        }
      }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      int lo = low_s;
      while (lo < L && sched_pending(pend, lo) == 0xFF) ++lo;
      low_s = lo;
    }
    out += found;
    placed += found;
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    ps[pass + 1] = out;
    npass[q] = pass;
  }
}

}  // namespace

hipError_t launch_positions(const int32_t* orders, int L, int n_orders, int shared, int32_t* pos, hipStream_t stream) {
  (void)shared;
  if (L <= 0 || n_orders <= 0) return hipSuccess;
  const dim3 grid((unsigned)((L + 255) / 256), (unsigned)n_orders);
  positions_kernel<<<grid, 256, 0, stream>>>(orders, L, n_orders, pos);
  scatter_positions_kernel<<<grid, 256, 0, stream>>>(orders, L, pos);
  return hipGetLastError();
}

hipError_t launch_decoder_precompute(const ModelDev& m, const float* h_v, const float* h_e, int L, int K,
                                     float* E1, float* Q, hipStream_t stream, _Float16* E1h, _Float16* Qh) {
  const size_t S = (size_t)L * K;
  if (S == 0) return hipSuccess;
  rows_gemm_kernel<<<dim3((unsigned)((S + kGemmRows - 1) / kGemmRows), kLayers), 256, 0, stream>>>(
      h_e, S, m.W1b_dec_p, kLayers * kH, E1h ? nullptr : E1, E1h, kLayers);
  rows_gemm_kernel<<<dim3((unsigned)((L + kGemmRows - 1) / kGemmRows), kLayers + 1), 256, 0, stream>>>(
      h_v, (size_t)L, m.W1d_dec_p, (kLayers + 1) * kH, Q, Qh, kLayers);
  return hipGetLastError();
}

hipError_t launch_q_precompute(const ModelDev& m, const float* h_v, int L, float* Q, hipStream_t stream) {
  if (L <= 0) return hipSuccess;
  rows_gemm_kernel<<<dim3((unsigned)((L + kGemmRows - 1) / kGemmRows), kLayers + 1), 256, 0, stream>>>(
      h_v, (size_t)L, m.W1d_dec_p, (kLayers + 1) * kH, Q, nullptr, 0);
  return hipGetLastError();
}

hipError_t launch_step_records(const ModelDev& m, const DecodeArgs& a, float4* rec, hipStream_t stream) {
  if (a.L <= 0 || a.B <= 0) return hipSuccess;
  if (a.K > kKmax) return hipErrorInvalidValue;
  const int nq = a.shared_order ? 1 : a.B;
  step_records_kernel<<<dim3((unsigned)a.L, (unsigned)nq), 128, 0, stream>>>(m, a, rec);
  return hipGetLastError();
}

hipError_t launch_layer0_table(const ModelDev& m, const float* E1, const float* Q, const int32_t* idx,
                               const int32_t* pos, const int32_t* base, int L, int K, float* tab, hipStream_t stream) {
  if (L <= 0 || K <= 0) return hipSuccess;
  if (K > kKmax || (base && !pos)) return hipErrorInvalidValue;
  layer0_table_kernel<<<dim3((unsigned)L, (unsigned)((K + kTabSlots - 1) / kTabSlots)), kThreads, 0, stream>>>(
      m, E1, Q, idx, pos, base, L, K, tab);
  return hipGetLastError();
}

hipError_t launch_l0_rows(const int32_t* idx, const int32_t* pos, int L, int K, int32_t* base, hipStream_t stream) {
  if (L <= 0 || K <= 0) return hipSuccess;
  if (K > kKmax || L > kL0RowsMaxL) return hipErrorInvalidValue;
  l0_rows_kernel<<<1, kL0RowsThreads, 0, stream>>>(idx, pos, L, K, base);
  return hipGetLastError();
}

hipError_t launch_decode_schedule(const DecodeArgs& a, hipStream_t stream) {
  if (a.L <= 0 || a.B <= 0) return hipSuccess;
  const int nq = a.shared_order ? 1 : a.B;
  const size_t n = (size_t)a.L * a.K;
  neighbour_schedule_kernel<<<dim3((unsigned)std::min<size_t>((n + 255) / 256, 4096), nq), 256, 0, stream>>>(
      a.orders, a.pos, a.idx, a.L, a.K, a.nbj, a.nbp);
  const char* mode = std::getenv("HKBS_DECODE_SCHEDULE");
  const int sequential = (mode && std::strcmp(mode, "sequential") == 0) || a.L > kSchedMaxL;
  if (a.max_members < 1) return hipErrorInvalidValue;
  const size_t L = (size_t)a.L;
  int32_t* indeg = a.sched_tmp;            // [nq][L]
  int32_t* off = indeg + nq * L;           // [nq][L + 1]: counts, then offsets
  int32_t* cur = off + nq * (L + 1);       // [nq][L]
  int32_t* meta = cur + nq * L;            // [nq][4] (= sched_meta(a.sched_tmp, L, nq))
  int32_t* dlist = meta + nq * 4;          // [nq][L K]
  hipError_t err = launch_zero(reinterpret_cast<float*>(indeg), nq * (3 * L + 1), stream);
  if (err != hipSuccess) return err;
  const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 2048);
  dep_count_kernel<<<dim3(blocks, nq), 256, 0, stream>>>(a.orders, a.mask, a.nbp, a.L, a.K, indeg, off);
  sched_prep_kernel<<<nq, kSchedThreads, 0, stream>>>(a.orders, a.pos, a.mask, a.L, sequential, off, a.draw, a.sched,
                                                     a.pstart, meta);
  dep_fill_kernel<<<dim3(blocks, nq), 256, 0, stream>>>(a.orders, a.mask, a.nbp, a.L, a.K, off, cur, dlist);
  const bool balance = a.pass_granule > 1 && a.L <= kSchedPrioMaxL;
  const size_t lds_words = (L + 3) / 4 + (balance ? 3 * ((L + 1) / 2) : 0);
  ready_schedule_kernel<<<nq, kSchedThreads, sizeof(uint32_t) * lds_words, stream>>>(
      a.orders, a.mask, a.nbp, a.L, a.K, a.max_members, a.pass_granule, indeg, off, dlist, a.draw, meta, a.sched,
      a.pstart, a.npass);
  return hipGetLastError();
}

namespace {

// Workgroups per sequence: up to min(8, max_team, HKBS_DECODE_TEAM) while the
// grid (8 * ceil(B / 8) * P workgroups, one per CU) fits the device at once.
template <int PREC>
int team_size_as(int B, int max_team) {
  int dev = 0, cus = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_kernel<PREC, decode_group(PREC, 2)>, kThreads, 0) !=
          hipSuccess)
    return 1;
  const long resident = (long)cus * per_cu;
  const long teams_per_xcd = (B + 7) / 8;
  int P = std::max(1, std::min(8, max_team));
  if (const char* env = std::getenv("HKBS_DECODE_TEAM")) P = std::max(1, std::min(P, std::atoi(env)));
  while (P > 1 && 8 * teams_per_xcd * P > resident) --P;
  return P;
}

template <int PREC>
hipError_t launch_decode_as(const ModelDev& m, const DecodeArgs& args, hipStream_t stream, int max_team) {
  if (args.L <= 0 || args.B <= 0) return hipSuccess;
  DecodeArgs a = args;
  ModelDev mm = m;
  const long teams_per_xcd = (a.B + 7) / 8;
  int P = team_size_as<PREC>(a.B, max_team);
  if (!a.sync || !a.fault) P = 1;
  if (a.max_members < 1 || a.max_members > decode_group(PREC, P) * P)
    return hipErrorInvalidValue;  // the schedule assumed a larger team
  a.spin_limit = kSpinLimit;
  if (const char* env = std::getenv("HKBS_DECODE_SPIN_LIMIT")) a.spin_limit = (uint32_t)std::max(1, std::atoi(env));
  {
    const char* env = std::getenv("HKBS_DECODE_FENCES");
    a.fences = env && std::strcmp(env, "1") == 0;
  }
  if (P > 1) {
    a.team = P;
    const dim3 grid((unsigned)(8 * teams_per_xcd * P));
    // team_size_as sized the grid so that all of it is resident at once
    // (at most the occupancy limit per CU over all CUs), so on a device
    // running nothing else every team is resident. Every team barrier wait is
    // bounded: a member that is not resident ends the wait with the fault
    // word raised instead of hanging.
    decode_kernel<PREC, decode_group(PREC, 2)><<<grid, kThreads, 0, stream>>>(mm, a);
    return hipGetLastError();
  }
  a.team = 1;
  decode_kernel<PREC, decode_group(PREC, 1)><<<a.B, kThreads, 0, stream>>>(mm, a);
  return hipGetLastError();
}

}  // namespace

int decode_team_size(int precision, int B, int max_team) {
  switch (precision) {
    case kPrecBf16x3:
      return team_size_as<kPrecBf16x3>(B, max_team);
    case kPrecBf16:
      return team_size_as<kPrecBf16>(B, max_team);
    case kPrecFp16:
      return team_size_as<kPrecFp16>(B, max_team);
    default:
      return team_size_as<kPrecFp32>(B, max_team);
  }
}

hipError_t launch_decode(const ModelDev& m, const DecodeArgs& args, hipStream_t stream, int max_team) {
  switch (args.precision) {
    case kPrecBf16x3:
      return launch_decode_as<kPrecBf16x3>(m, args, stream, max_team);
    case kPrecBf16:
      return launch_decode_as<kPrecBf16>(m, args, stream, max_team);
    case kPrecFp16:
      return launch_decode_as<kPrecFp16>(m, args, stream, max_team);
    default:
      return launch_decode_as<kPrecFp32>(m, args, stream, max_team);
  }
}

}  // namespace hkbs
