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
#include "device_math.hpp"
#include "pmpnn_internal.hpp"

namespace hkbs {
namespace {

constexpr int kLd = kH + 4;  // 132
constexpr int kThreads = 512;

// y[o] = sum_p x[p] Wt[p][o] (+ bias) for OUT outputs and IN inputs on all
// threads of the block: each thread loads its PER float4 weights up front
// (all in flight), partial sums meet in LDS. part >= 2048 floats.
template <int IN, int OUT>
__device__ inline void gemv(const float* __restrict__ Wt, const float* x, const float* __restrict__ bias,
                            float* part, float* y) {
  constexpr int Q4 = OUT / 4;            // float4 columns
  constexpr int GROUPS = kThreads / Q4;  // input groups
  constexpr int PER = IN / GROUPS;       // inputs per group
  static_assert(GROUPS * OUT <= 2048, "partial buffer");
  const int q = threadIdx.x % Q4;
  const int grp = threadIdx.x / Q4;
  const float* w = Wt + (size_t)(grp * PER) * OUT + 4 * q;
  float4 wv[PER];
#pragma unroll
  for (int p = 0; p < PER; ++p) wv[p] = *reinterpret_cast<const float4*>(w + (size_t)p * OUT);
  float4 acc = make_float4(0.F, 0.F, 0.F, 0.F);
#pragma unroll
  for (int p = 0; p < PER; ++p) {
    const float xv = x[grp * PER + p];
    acc.x += xv * wv[p].x;
    acc.y += xv * wv[p].y;
    acc.z += xv * wv[p].z;
    acc.w += xv * wv[p].w;
  }
  *reinterpret_cast<float4*>(part + grp * OUT + 4 * q) = acc;
  __syncthreads();
  for (int o = threadIdx.x; o < OUT; o += kThreads) {
    float s = 0.0F;
#pragma unroll
    for (int g = 0; g < GROUPS; ++g) s += part[g * OUT + o];
    y[o] = bias ? s + bias[o] : s;
  }
  __syncthreads();
}

// LayerNorm of a 128-vector in LDS by wave 0; result visible after the barrier.
__device__ inline void ln_vec(const float* x, const float* g, const float* b, float* out) {
  if (threadIdx.x < 64) ln_row_wave(x, g, b, out);
  __syncthreads();
}

__global__ __launch_bounds__(kThreads) void decode_kernel(ModelDev m, DecodeArgs a) {
  __shared__ __attribute__((aligned(16))) float G[kKmax * kLd];
  __shared__ __attribute__((aligned(16))) float part[2048];
  __shared__ __attribute__((aligned(16))) float h[kH];
  __shared__ __attribute__((aligned(16))) float hA[2 * kH];  // [A | scratch]
  __shared__ __attribute__((aligned(16))) float x[kH];
  __shared__ __attribute__((aligned(16))) float h1[kH];
  __shared__ __attribute__((aligned(16))) float ff[kFF];
  __shared__ __attribute__((aligned(16))) float P[2][2 * kH];  // [W1d h | W1a h] of layers 1, 2
  __shared__ float logits[32];
  __shared__ float tbl[17];
  __shared__ int nbr[kKmax];
  __shared__ int bwf[kKmax];
  __shared__ int tok_s;

  const int b = blockIdx.x;
  const int L = a.L, K = a.K;
  const size_t S = (size_t)L * K;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int32_t* order = a.shared_order ? a.orders : a.orders + (size_t)b * L;
  const int32_t* pos = a.shared_order ? a.pos : a.pos + (size_t)b * L;
  float* R = a.R + (size_t)b * kLayers * L * kH;
  int32_t* tokens = a.tokens + (size_t)b * L;
  float* lp_out = a.log_probs ? a.log_probs + (size_t)b * L * kV : nullptr;
  float* chosen = a.chosen_lp + (size_t)b * L;
  uint64_t rng = a.seeds[b];
  const float T = (a.temperature > 0.0F && isfinite(a.temperature)) ? a.temperature : 1.0F;
  const bool greedy = a.greedy || a.temperature <= 0.0F;
  if (threadIdx.x < 17) tbl[threadIdx.x] = kExpNegTable[threadIdx.x];
  __syncthreads();

  for (int step = 0; step < L; ++step) {
    const int t = order[step];
    if (t < 0 || t >= L) continue;  // malformed device order: skip the entry
    const bool active = a.mask[t] != 0.0F;
    if (!active) {
      // inverse_fold_scalar.cpp:804-813: fallback token, zero log-probs, no draw.
      const int tok = (a.true_tokens && a.true_tokens[t] >= 0 && a.true_tokens[t] < kV) ? a.true_tokens[t] : kV - 1;
      if (threadIdx.x == 0) {
        tokens[t] = tok;
        chosen[t] = 0.0F;
      }
      if (lp_out && threadIdx.x < kV) lp_out[(size_t)t * kV + threadIdx.x] = 0.0F;
      for (int i = threadIdx.x; i < kLayers * kH; i += kThreads) {
        const int l = i / kH, c = i % kH;
        const float base = (l == 0) ? a.Q[(size_t)t * kH + c] : 0.0F;
        R[((size_t)l * L + t) * kH + c] = base + m.dec[l].T[tok * kH + c];
      }
      __syncthreads();
      continue;
    }
    if (threadIdx.x < K) {
      const int j = a.idx[(size_t)t * K + threadIdx.x];
      const bool valid = j >= 0 && j < L;
      nbr[threadIdx.x] = valid ? j : -1;
      bwf[threadIdx.x] = valid && pos[j] < step;
    }
    if (threadIdx.x < kH) {
      h[threadIdx.x] = a.h_v[(size_t)t * kH + threadIdx.x];
      // layer-0 W1a h^0_t comes from the precompute (Q block 3)
      hA[threadIdx.x] = a.Q[((size_t)3 * L + t) * kH + threadIdx.x] + m.dec[0].b1[threadIdx.x];
    }
    __syncthreads();

    for (int l = 0; l < kLayers; ++l) {
      const DecLayerDev& w = m.dec[l];
      // Message rows g1_k = GELU(A + E1_tk + (bw ? R : Q)_j); rows >= K are zero.
      const float* E1 = a.E1 + ((size_t)l * S + (size_t)t * K) * kH;
      const float* Ql = a.Q + (size_t)l * L * kH;
      const float* Rl = R + (size_t)l * L * kH;
      for (int task = threadIdx.x; task < kKmax * (kH / 4); task += kThreads) {
        const int k = task / (kH / 4);
        const int c = 4 * (task % (kH / 4));
        float4 xv = *reinterpret_cast<const float4*>(hA + c);
        const int j = k < K ? nbr[k] : -1;
        if (j >= 0) {
          const float4 e = *reinterpret_cast<const float4*>(E1 + (size_t)k * kH + c);
          const float4 z = *reinterpret_cast<const float4*>((bwf[k] ? Rl : Ql) + (size_t)j * kH + c);
          xv.x += e.x + z.x;
          xv.y += e.y + z.y;
          xv.z += e.z + z.z;
          xv.w += e.w + z.w;
        }
        float4 v = make_float4(gelu_fast(xv.x, tbl), gelu_fast(xv.y, tbl), gelu_fast(xv.z, tbl), gelu_fast(xv.w, tbl));
        if (k >= K) v = make_float4(0.F, 0.F, 0.F, 0.F);
        *reinterpret_cast<float4*>(G + k * kLd + c) = v;
      }
      __syncthreads();
      {
        floatx4 acc[3][1];
        zero_acc(acc);
        mfma_tile<3, 1>(G, kLd, w.W2_p, kH, wave * 16, kH, acc);
        // x[col] = sum over valid rows of GELU(acc + b2)
        const int col = wave * 16 + (lane & 15);
        const float b2 = w.b2[col];
        float s = 0.0F;
#pragma unroll
        for (int mb = 0; mb < 3; ++mb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int row = mb * 16 + 4 * (lane >> 4) + i;
            const float g = gelu_fast(acc[mb][0][i] + b2, tbl);
            s += row < K ? g : 0.0F;
          }
        s += __shfl_xor(s, 16, 64);
        s += __shfl_xor(s, 32, 64);
        if (lane < 16) x[col] = s;
      }
      __syncthreads();
      // upd = (W3 s + K b3) / 30 ; h1 = LN1(h + upd)
      gemv<kH, kH>(w.W3_t, x, nullptr, part, hA + kH);
      if (threadIdx.x < kH) {
        const int c = threadIdx.x;
        x[c] = h[c] + (hA[kH + c] + static_cast<float>(K) * w.b3[c]) * (1.0F / 30.0F);
      }
      __syncthreads();
      ln_vec(x, w.n1g, w.n1b, h1);
      gemv<kH, kFF>(w.Win_t, h1, w.bin, part, ff);
      ff[threadIdx.x] = gelu_fast(ff[threadIdx.x], tbl);
      __syncthreads();
      gemv<kFF, kH>(w.Wout_t, ff, w.bout, part, hA + kH);
      if (threadIdx.x < kH) x[threadIdx.x] = h1[threadIdx.x] + hA[kH + threadIdx.x];
      __syncthreads();
      ln_vec(x, w.n2g, w.n2b, h);  // h = h^{l+1}_t (active residue: mask gate is 1)
      if (l + 1 < kLayers) {
        // fused [W1d | W1a] of the next layer: P (for R) and A (next message rows)
        gemv<kH, 2 * kH>(m.dec[l + 1].W1da_t, h, nullptr, part, P[l]);
        if (threadIdx.x < kH) hA[threadIdx.x] = P[l][kH + threadIdx.x] + m.dec[l + 1].b1[threadIdx.x];
        __syncthreads();
      }
    }
    // logits = W_out h + b (padded to 32 outputs)
    gemv<kH, 32>(m.Wlog_t, h, m.blog, part, logits);
    if (threadIdx.x == 0) {
      // sampler_scalar.cpp:49-92 in the reference's operation order.
      float z[kV], p[kV];
      float row_max = -__builtin_inff();
      for (int i = 0; i < kV; ++i) {
        z[i] = logits[i] / T;
        row_max = (row_max < z[i]) ? z[i] : row_max;
      }
      float row_sum = 0.0F;
      for (int i = 0; i < kV; ++i) {
        const float e = expf(z[i] - row_max);
        p[i] = e;
        row_sum += e;
      }
      const float log_sum = logf(row_sum);
      const float inv_sum = 1.0F / row_sum;
      int s_tok;
      if (greedy) {
        s_tok = 0;
        float bv = z[0];
        for (int i = 1; i < kV; ++i)
          if (z[i] > bv) {
            s_tok = i;
            bv = z[i];
          }
      } else {
        rng += 0x9E3779B97F4A7C15ull;
        uint64_t zz = rng;
        zz = (zz ^ (zz >> 30)) * 0xBF58476D1CE4E5B9ull;
        zz = (zz ^ (zz >> 27)) * 0x94D049BB133111EBull;
        zz ^= zz >> 31;
        const double u = static_cast<double>(zz >> 11) * (1.0 / 9007199254740992.0);
        double cum = 0.0;
        s_tok = kV - 1;
        for (int i = 0; i < kV; ++i) {
          cum += static_cast<double>(p[i] * inv_sum);
          if (u < cum) {
            s_tok = i;
            break;
          }
        }
      }
      const float design = (a.chain_mask ? a.chain_mask[t] : 1.0F) * a.mask[t];
      int tok = s_tok;
      if (design == 0.0F)
        tok = (a.true_tokens && a.true_tokens[t] >= 0 && a.true_tokens[t] < kV) ? a.true_tokens[t] : kV - 1;
      tokens[t] = tok;
      tok_s = tok;
      for (int i = 0; i < kV; ++i) {
        const float lpv = (z[i] - row_max) - log_sum;
        if (lp_out) lp_out[(size_t)t * kV + i] = lpv;
        if (i == tok) chosen[t] = lpv;
      }
    }
    __syncthreads();
    const int tok = tok_s;
    for (int i = threadIdx.x; i < kLayers * kH; i += kThreads) {
      const int l = i / kH, c = i % kH;
      const float base = (l == 0) ? a.Q[(size_t)t * kH + c] : P[l - 1][c];
      R[((size_t)l * L + t) * kH + c] = base + m.dec[l].T[tok * kH + c];
    }
    __syncthreads();
  }
  // Mean NLL over designed residues in residue order (inverse_fold_scalar.cpp:471-493).
  if (a.scores && threadIdx.x == 0) {
    double loss = 0.0, msum = 0.0;
    for (int r = 0; r < L; ++r) {
      const float act = (a.chain_mask ? a.chain_mask[r] : 1.0F) * a.mask[r];
      if (act == 0.0F) continue;
      loss -= static_cast<double>(chosen[r]);
      msum += static_cast<double>(act);
    }
    a.scores[b] = msum > 0.0 ? static_cast<float>(loss / msum) : 0.0F;
  }
}

// out[c][row][:] = A[row] . Wp(cols 128c..128c+127) for a [M,128] input.
constexpr int kGemmRows = 64;
__global__ __launch_bounds__(256) void rows_gemm_kernel(const float* __restrict__ Ain, size_t M,
                                                        const float* __restrict__ Wp, int N,
                                                        float* __restrict__ out) {
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
  float* o = out + (size_t)cblk * M * kH;
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const size_t row = row0 + mb * 16 + 4 * (lane >> 4) + i;
        const int col = wave * 32 + nb * 16 + (lane & 15);
        if (row < M) o[row * kH + col] = acc[mb][nb][i];
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
                                     float* E1, float* Q, hipStream_t stream) {
  const size_t S = (size_t)L * K;
  if (S == 0) return hipSuccess;
  rows_gemm_kernel<<<dim3((unsigned)((S + kGemmRows - 1) / kGemmRows), kLayers), 256, 0, stream>>>(
      h_e, S, m.W1b_dec_p, kLayers * kH, E1);
  rows_gemm_kernel<<<dim3((unsigned)((L + kGemmRows - 1) / kGemmRows), kLayers + 1), 256, 0, stream>>>(
      h_v, (size_t)L, m.W1d_dec_p, (kLayers + 1) * kH, Q);
  return hipGetLastError();
}

hipError_t launch_q_precompute(const ModelDev& m, const float* h_v, int L, float* Q, hipStream_t stream) {
  if (L <= 0) return hipSuccess;
  rows_gemm_kernel<<<dim3((unsigned)((L + kGemmRows - 1) / kGemmRows), kLayers + 1), 256, 0, stream>>>(
      h_v, (size_t)L, m.W1d_dec_p, (kLayers + 1) * kH, Q);
  return hipGetLastError();
}

hipError_t launch_decode(const ModelDev& m, const DecodeArgs& a, hipStream_t stream) {
  if (a.L <= 0 || a.B <= 0) return hipSuccess;
  decode_kernel<<<a.B, kThreads, 0, stream>>>(m, a);
  return hipGetLastError();
}

}  // namespace hkbs
