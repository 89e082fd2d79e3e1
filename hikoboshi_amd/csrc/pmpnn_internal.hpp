// Internal declarations shared by the HIP kernels and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace hkbs {

constexpr int kH = 128;        // hidden width
constexpr int kV = 21;         // vocabulary
constexpr int kKmax = 48;      // neighbours
constexpr int kRbf = 16;       // RBF centres
constexpr int kPairs = 25;     // atom pairs
constexpr int kPos = 16;       // positional features
constexpr int kPosClasses = 66;
constexpr int kEdgeIn = 416;   // 16 + 25 * 16
constexpr int kFF = 512;       // FFN hidden
constexpr int kLayers = 3;
constexpr int kTensors = 118;

// Packed-weight layouts used on the device.
//  * "kpack16" for MFMA B operands: W [N][K] (row-major, out x in) stored as
//    Wp[K/16][N][16] with Wp[kb][n][j] = W[n][16 kb + j]. One float4 load per
//    lane per four MFMA k-steps, 1 KiB contiguous per 16 columns.
//  * "t" (transposed) for GEMVs: Wt[K][N] = W[n][k].
struct EncLayerDev {
  const float* W1_t;    // [384][128]  input order [h_i | e_ij | h_j]
  const float* W2_t;    // [128][128]
  const float* W3_t;    // [128][128]
  const float* W11_t;   // [384][128]
  const float* W12_t;   // [128][128]
  const float* W13_t;   // [128][128]
  const float* Win_t;   // [128][512]
  const float* Wout_t;  // [512][128]
  const float *b1, *b2, *b3, *b11, *b12, *b13, *bin, *bout;
  const float *n1g, *n1b, *n2g, *n2b, *n3g, *n3b;
};

// Encoder weights for the fp16 MFMA with split operands: W [N][K] (out x in)
// as hi = fp16(W) and lo = fp16((W - hi) * 2048), each stored as [K / 8][N][8]
// halves (lo follows hi, K * N halves later), so lane (r, g) of a wave reads
// the 8 consecutive k of column n = n0 + r with one 16-byte load.
struct Enc16LayerDev {
  const uint16_t *W1, *W2, *W3;     // K = 384 ([h_i | e_ij | h_j]), 128, 128; N = 128
  const uint16_t *W11, *W12, *W13;  // the same for the edge update
  const uint16_t *Win, *Wout;       // 128 -> 512, 512 -> 128
};
struct Enc16Dev {
  const uint16_t* Wedge;  // 416 -> 128
  const uint16_t* We;     // 128 -> 128
  Enc16LayerDev layer[kLayers];
};

struct DecLayerDev {
  const float* W1a_t;  // [128][128]
  const float* W2_p;   // kpack16 128 -> 128
  const float* W2h;    // [16][128][8] fp16: W2 = W2h + W2l / 2048 (decode loop)
  const float* W2l;
  const uint16_t* W1b_s;  // W1b [16][128][8] fp16 hi, then lo (lo follows 128 * 128 halves later): teacher forcing
  // bf16 copies for the bf16 decode (round to nearest even), all as MFMA B
  // fragments [inputs / 8][outputs][8] (W2 like W2h; W3, Win, Wout, W1da from
  // their t-layouts)
  const uint16_t *W2_b, *W3_h, *Win_h, *Wout_h, *W1da_h;
  // the bf16 remainders lo = bf16(w - hi) of the same, for the split bf16 decode
  // (w = hi + lo to about 16 significant bits)
  const uint16_t *W2_bl, *W3_hl, *Win_hl, *Wout_hl, *W1da_hl;
  const uint16_t *W3_f, *Win_f, *Wout_f, *W1da_f;  // fp16 copies (W2 in fp16 is W2h)
  const float* W3_t;   // [128][128]
  const float* Win_t;  // [128][512]
  const float* Wout_t; // [512][128]
  const float* W1da_t; // [128][256]: columns [W1d | W1a] (layers 1, 2)
  // teacher forcing, split fp16 [K / 8][N][8] hi then lo (lo K * N halves later), for wave_gemm
  const uint16_t* W3_s;    // 128 -> 128
  const uint16_t* Win_s;   // 128 -> 512
  const uint16_t* Wout_s;  // 512 -> 128
  const uint16_t* Wnext_s; // 128 -> 256: outputs [W1a; W1d] of the next layer (layers 0, 1)
  const float* T;      // [21][128]: W1c . W_s[v]
  const float *b1, *b2, *b3, *bin, *bout;
  const float *n1g, *n1b, *n2g, *n2b;
};

struct ModelDev {
  const float* pos_w;  // [16][66]
  const float* pos_b;  // [16]
  const float* edge_t; // [416][128]
  const float *ne_g, *ne_b;
  const float* We_t;   // [128][128]
  const float* We_b;
  const float* Ws;     // [21][128]
  EncLayerDev enc[kLayers];
  DecLayerDev dec[kLayers];
  const float* W1b_dec_p;  // kpack16 128 -> 384: rows = [W1b_0; W1b_1; W1b_2] (decoder)
  const float* W1d_dec_p;  // kpack16 128 -> 512: rows = [W1d_0; W1d_1; W1d_2; W1a_0]
  const float* Wlog_t;     // [128][32] (21 used)
  const float* blog;       // [32] (21 used)
  const uint16_t* Wlog_h;  // bf16 copy of Wlog_t
  const uint16_t* Wlog_f;  // fp16 copy of Wlog_t
  Enc16Dev enc16;          // split-fp16 encoder weights (16-bit design modes)
};

// Launchers (each enqueues on `stream`; shapes are validated by the caller).
// seg/offsets (optional): ragged batch, row q belongs to protein seg[q] whose
// residues are [offsets[seg[q]], offsets[seg[q] + 1]).
hipError_t launch_knn(const float* coords, const uint8_t* atom_src, int L, int K, int32_t* idx,
                      float* d2, float* mask, float4* ca_scratch, hipStream_t stream,
                      const int32_t* seg = nullptr, const int64_t* offsets = nullptr);
// pos[b][orders[b][s]] = s for each of n_orders orders of length L.
hipError_t launch_positions(const int32_t* orders, int L, int n_orders, int shared, int32_t* pos,
                            hipStream_t stream);
hipError_t launch_edge_features(const ModelDev& m, const float* coords, const uint8_t* atom_src,
                                const int32_t* resid, const int32_t* chain, const int32_t* idx,
                                int L, int K, float* features, hipStream_t stream);
hipError_t launch_edge_embed(const ModelDev& m, const float* coords, const uint8_t* atom_src,
                             const int32_t* resid, const int32_t* chain, const int32_t* idx, int L,
                             int K, float* h_e, hipStream_t stream);
// Floats per residue of EncoderScratch::prefix.
constexpr int kPrefix = 4 * kH;
struct EncoderScratch {
  float* prefix;   // L x kPrefix floats, per-residue products of h (fp32 encoder: [L][256], the [W11 | next W1]
                   // h_i blocks; 16-bit encoder: planes [4][L][128], W11 h_i, W11 h_j, next W1 h_i, next W1 h_j)
  float* msg;      // [L * K][128] edge messages of the current layer, plus L floats
};
// Fills n floats with zero (a kernel, so it can sit inside a captured graph).
hipError_t launch_zero(float* p, size_t n, hipStream_t stream);
// Host: out = coords + the reference's Gaussian backbone noise (host_noise.cpp).
void backbone_noise_host(const float* coords, const uint8_t* atom_sources, int32_t L, float sigma, uint64_t seed,
                         float* out);
hipError_t launch_encoder(const ModelDev& m, const int32_t* idx, const float* mask, int L, int K,
                          float* h_v, float* h_e, const EncoderScratch& ws, hipStream_t stream);
// Featurisation and encoder on the fp16 MFMA with split operands (fp32-level
// accuracy; the 16-bit design modes); kNN (idx, mask) comes from launch_knn.
// ws.prefix receives the per-residue h_i products ([L][256]) and ws.msg the
// neighbour sums ([L][128]).
hipError_t launch_encoder16(const ModelDev& m, const float* coords, const uint8_t* atom_src,
                            const int32_t* resid, const int32_t* chain, const int32_t* idx, const float* mask,
                            int L, int K, float* h_v, float* h_e, const EncoderScratch& ws, hipStream_t stream);
// E1 = W1b h_E [3][L*K][128] and Q [4][L][128]. With E1h (the 16-bit decode
// modes) E1 is written only in fp16 to E1h (E1 may be null) and Qh receives an
// fp16 copy of Q blocks 0..2; values are clamped to the fp16 range.
hipError_t launch_decoder_precompute(const ModelDev& m, const float* h_v, const float* h_e, int L,
                                     int K, float* E1, float* Q, hipStream_t stream, _Float16* E1h = nullptr,
                                     _Float16* Qh = nullptr);
struct DecodeArgs {
  const int32_t* idx;     // [L][K]
  const float* mask;      // [L]
  const float* h_v;       // [L][128] encoder output
  const float* E1;        // [3][S][128]
  const float* Q;         // [4][L][128]: W1d_l h^0 (l = 0..2), W1a_0 h^0
  const int32_t* orders;  // [B][L] or [L]
  int shared_order;
  const int32_t* pos;     // [B][L] or [L]: position of residue r in the order
  int32_t* nbj;           // [B][L][K] or [L][K] workspace: neighbours of the residue at each step
  int32_t* nbp;           // same shape: their positions in the order (L for an empty slot)
  // Pass schedule per order (nq = 1 for a shared order, else B), built by
  // launch_decode_schedule: pass p decodes the steps sched[pstart[p] ..
  // pstart[p + 1]); pass 0 holds the inactive steps; passes 1..npass follow.
  int32_t* sched;         // [nq][L]
  int32_t* pstart;        // [nq][L + 2]
  int32_t* npass;         // [nq]
  int32_t* draw;          // [nq][L]: sampler draw index of each active step, -1 otherwise
  int32_t* sched_tmp;     // scratch of the schedule kernels: sched_scratch_words(L, K, nq) words
  const float* chain_mask;   // [L] or null
  const int32_t* true_tokens; // [L] or null
  const uint64_t* seeds;  // [B]
  float temperature;
  int greedy;
  int L, K, B;
  float* R;               // [B][3][L][128] workspace
  int32_t* tokens;        // [B][L]
  float* log_probs;       // [B][L][21] or null
  float* scores;          // [B] or null
  float* chosen_lp;       // [B][L] workspace: log-prob of the written token
  uint32_t* sync;         // [B] team barrier counters, zero at launch
  uint32_t* fault;        // [1] set when a team barrier times out, zero at launch
  int team;               // workgroups per sequence (set by launch_decode)
  uint32_t spin_limit;    // polls before a team barrier gives up (set by launch_decode)
  int fences;             // team barrier with release/acquire fences (set by launch_decode, HKBS_DECODE_FENCES=1)
  int precision;          // 0 fp32, 1 bf16, 2 fp16, 3 split bf16 (see decode_kernel)
  int max_members;        // most steps one pass decodes (<= decode_group(precision, team) * team)
  int pass_granule;       // team size the schedule balances passes for (<= 1: none)
  const float* l0tab;     // layer-0 message rows (fp32 decode; launch_layer0_table), or null
  const int32_t* l0base;  // [L + 1] first table row of each residue (compact table of one shared order), or null
  const float4* rec;      // [nq][L][kRecFloat4] per-step inputs in schedule order (launch_step_records)
  // 16-bit decode modes: the message rows' inputs in fp16 (E1 and R unused then)
  const _Float16* E1h;    // [3][L*K][128]
  const _Float16* Qh;     // [3][L][128]: Q blocks 0..2
  _Float16* Rh;           // [B][3][L][128]
};
// Steps one workgroup decodes in a pass, for DecodeArgs.precision and the team
// size (workgroups per sequence): 8 in fp32 (0), where with one workgroup per
// sequence, or with long chains, this capacity rather than the depth of the step
// graph bounds the passes (one wave per member; the partial sums of 8 members
// fill the message rows' LDS); 6 in the split bf16 mode (3), whose layer
// products run on the MFMA with the members as rows of a 16-row operand, so that
// more members cost no more product time; 4 otherwise. Team size 1 gives the
// largest value of a mode.
constexpr int decode_group(int precision, int team) {
  return precision == 0 ? 8 : precision == 3 ? 6 : 4;
}
// int32 words of DecodeArgs.sched_tmp for nq orders of length L with K neighbours.
inline size_t sched_scratch_words(size_t L, size_t K, size_t nq) { return nq * (3 * L + 1 + 4 + L * K); }
// Four words per order inside sched_tmp, written by the schedule: {decoded in dependency
// passes, active steps, inactive steps, the order is a permutation of 0..L-1}.
__host__ __device__ inline int32_t* sched_meta(int32_t* sched_tmp, size_t L, size_t nq) {
  return sched_tmp + nq * (3 * L + 1);
}
// Per-step neighbour lists (a.nbj, a.nbp) and the pass schedule (a.sched,
// a.pstart, a.npass, a.draw) from the orders, positions, mask and kNN graph;
// launch_decode reads them.
hipError_t launch_decode_schedule(const DecodeArgs& a, hipStream_t stream);
// Per-step inputs of the decode in schedule order (after launch_decode_schedule
// and the decoder precompute): record s of order q describes step
// u = sched[q][s] (residue t = order[u]) as 112 float4: words 0..47 the
// neighbour slots (j | 2^30 if j is decoded before the step, -1 for an empty
// slot), word 48 t, 49 the draw index, 50 the design weight chain_mask[t]
// mask[t] (float bits), 51 the true token or the fallback token, 52 and 53 the
// mask of slots decoded before the step (bit k), 54 the residue's first row in
// the layer-0 table, 55..63 zero, then the rows h^0_t, W1a_0 h^0_t + b1_0 and
// W1d_0 h^0_t (128 floats each).
// The decode stages a pass's members with one 16-byte load per thread.
constexpr int kRecFloat4 = 112;
hipError_t launch_step_records(const ModelDev& m, const DecodeArgs& a, float4* rec, hipStream_t stream);
// Workgroups per sequence the decode will use for B sequences (1..min(8, max_team)).
int decode_team_size(int precision, int B, int max_team);
// Decodes with up to min(8, max_team) workgroups per sequence when the whole
// grid fits the device at once, else one per sequence; a.max_members must not
// exceed decode_group(a.precision, team) x that team size (the schedule has to be built for it).
// A team launch that could not run its members together raises *a.fault (and
// leaves NaN scores); rebuild the schedule with max_members = decode_group(a.precision, 1) and
// run it again with max_team = 1.
hipError_t launch_decode(const ModelDev& m, const DecodeArgs& a, hipStream_t stream, int max_team = 8);
// Q[l] = W1d_l h^0 (l < 3), Q[3] = W1a_0 h^0, without the E1 edge products.
hipError_t launch_q_precompute(const ModelDev& m, const float* h_v, int L, float* Q, hipStream_t stream);
// Layer-0 message table of the fp32 decode. Slot k of residue t sees its
// neighbour j = idx[t][k] in one of kL0Classes states: decoded before t with
// token c (c < kV), or not yet decoded / an empty slot (c = kV). A row holds
// GELU(W2 GELU(A_t + E1_tk + z) + b2) for that state's z, computed with the
// decode loop's own operations, so the decode sums K rows instead of computing
// them. Full table (base null): row (t K + k) kL0Classes + c, every state of
// every slot. Compact table of one shared order (base from launch_l0_rows): a
// slot whose neighbour is decoded before t has the kV token rows, any other
// slot only its one state; residue t's rows start at base[t], its slots in
// order. E1, Q as written by launch_decoder_precompute; pos = the order's
// positions (launch_positions).
constexpr int kL0Classes = kV + 1;
inline size_t l0_table_floats(size_t L, size_t K) { return L * K * kL0Classes * kH; }
hipError_t launch_layer0_table(const ModelDev& m, const float* E1, const float* Q, const int32_t* idx,
                               const int32_t* pos, const int32_t* base, int L, int K, float* tab, hipStream_t stream);
// Row offsets of the compact layer-0 table of one shared order: base[t] = the
// first row of residue t, base[L] = the row count (at most L K kV).
hipError_t launch_l0_rows(const int32_t* idx, const int32_t* pos, int L, int K, int32_t* base, hipStream_t stream);
struct TfArgs {
  const int32_t* idx;     // [L][K] global neighbour indices
  const int32_t* pos;     // [L] position of each residue in its protein's decoding order
  const float* mask;      // [L]
  const int32_t* tokens;  // [L]
  const float* h_e;       // [L*K][128] encoder edge states
  const float* Q;         // [4][L][128]
  float* h;               // [L][128] in: encoder h_V, out: decoder state (overwritten)
  float* NB;              // [L][256] workspace: [A | R] terms of the current layer
  float* msg_sum;         // [L][128] workspace
  float* log_probs;       // [L][21] output
  int L, K;
};
hipError_t launch_teacher_forced(const ModelDev& m, const TfArgs& a, hipStream_t stream);

}  // namespace hkbs
