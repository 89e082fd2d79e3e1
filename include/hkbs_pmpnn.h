/*
 * hkbs_pmpnn.h - C ABI of the MI355X-native ProteinMPNN v_48_020 design path.
 *
 * The library replaces, for one GPU, the reference's scalar module seam
 *   hikoboshi::modules::mpnn::proteinmpnn_inverse_fold_scalar
 *     (cpp/include/hikoboshi/modules/mpnn/inverse_fold.hpp:113-115)
 *   hikoboshi::modules::mpnn::proteinmpnn_teacher_forced_forward_scalar
 *     (cpp/include/hikoboshi/modules/mpnn/inverse_fold.hpp:140-142)
 * and the per-sample loop of
 *   hikoboshi::algorithms::inverse_fold_proteinmpnn_v48_020
 *     (cpp/algorithms/inverse_fold.cpp:292-337)
 * by one batched call that encodes the backbone once and decodes all
 * sequences together. Everything crosses the boundary as plain pointers and
 * sizes; no C++ or framework types.
 *
 * Conventions (mirroring the reference):
 *  - Status codes are the reference's StatusCode values
 *    (cpp/include/hikoboshi/universal/status.hpp:12-19). HIP failures map to
 *    HKBS_UNAVAILABLE (no device) or HKBS_INTERNAL_ERROR. hkbs_last_error()
 *    returns a static detail string for the calling thread's last failure.
 *  - Arrays are row-major. coords is [L,5,3] float in the atom order
 *    N, CA, C, O, CB; atom_sources is [L,5] uint8 with the reference's
 *    AtomSource codes (0 Missing, 1 Observed, 2 Inferred, 3 Virtual;
 *    cpp/include/hikoboshi/universal/structure.hpp:21-38).
 *  - Optional inputs may be NULL: residue_indices (default 0..L-1),
 *    chain_labels (default one chain), chain_mask (default ones),
 *    true_tokens (default: fallback token 20 for residues not designed).
 *  - Calls on one context are made from one host thread at a time (a context
 *    owns one HIP stream and its workspace). Their GPU work is ordered by the
 *    library: a call's work starts after that of the previous device design
 *    call on the context has ended, on whatever stream it ran (the new call's
 *    stream waits on the device, the host does not block), except on a stream
 *    that is being captured into a HIP graph. Distinct contexts are
 *    independent.
 */
#ifndef HKBS_PMPNN_H
#define HKBS_PMPNN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int32_t hkbs_status;
enum {
  HKBS_OK = 0,
  HKBS_INVALID_ARGUMENT = 1,
  HKBS_FAILED_PRECONDITION = 2,
  HKBS_UNAVAILABLE = 3,
  HKBS_UNIMPLEMENTED = 4,
  HKBS_INTERNAL_ERROR = 5
};

/* Decode-order modes for hkbs_pmpnn_design. */
enum {
  /* Per sequence b: the reference's random order seeded by order_seeds[b]
   * (cpp/modules/mpnn/decode_order_scalar.cpp:89-115). */
  HKBS_ORDER_RANDOM = 0,
  /* orders holds one permutation per sequence, [B,L]
   * (use_input_decoding_order, decode_order_scalar.cpp:68-87). */
  HKBS_ORDER_INPUT_PER_SEQUENCE = 1,
  /* orders holds one permutation [L] shared by every sequence. */
  HKBS_ORDER_INPUT_SHARED = 2,
  /* N-to-C order 0..L-1 (cpp/algorithms/inverse_fold.cpp:273-276). */
  HKBS_ORDER_N_TO_C = 3
};

/* Arithmetic of the design path (hkbs_pmpnn_set_precision). The kNN graph and
 * the decoding order are exact in every mode. */
enum {
  HKBS_PRECISION_FP32 = 0, /* default: featurisation and encoder in the reference's fp32 rounding,
                              log-probs within 1e-4 of the reference */
  HKBS_PRECISION_BF16 = 1, /* decoder in bf16: bf16 weights of every decoder product, bf16
                              message rows into the W2 MFMA, the other products on the MFMA with
                              their fp32 inputs split into two bf16 halves; fp32 accumulation,
                              GELU, LayerNorm and softmax. Featurisation and encoder run on the
                              fp16 MFMA with each operand split into two fp16 halves (fp32-level
                              accuracy, not the reference's rounding sequence) */
  HKBS_PRECISION_FP16 = 2, /* the same with an fp16 decoder (three more significant bits than
                              bf16) */
  HKBS_PRECISION_BF16X3 = 3 /* decoder in split bf16: every decoder product on the bf16 MFMA with
                              its weights and its inputs each carried as two bf16 terms
                              (x = hi + lo, hi = bf16(x), lo = bf16(x - hi): about 16
                              significant bits) and three MFMA products per product
                              (hi.hi + hi.lo + lo.hi); fp32 accumulation, GELU, LayerNorm and
                              softmax; the message rows' inputs (E1, Q, R) in fp32, and layer
                              0's message rows from the fp32 path's per-backbone table while
                              it fits 4 GiB. Featurisation and encoder as in
                              HKBS_PRECISION_BF16. Log-probs
                              within 2e-2 of the fp32 path at T = 0.1 (plain bf16 is not) */
};

typedef struct hkbs_pmpnn hkbs_pmpnn;

/* Static detail text of the calling thread's last non-OK status. */
const char* hkbs_last_error(void);

/* Library version string. */
const char* hkbs_version(void);

/* Number of visible HIP devices (0 when none; never fails). */
int32_t hkbs_device_count(void);

/* Creates a context on HIP device `device` from the v_48_020 weight package
 * bytes (safetensors, 118 F32 tensors). Replaces the embedded weight view
 * binding of cpp/weights/embedded_proteinmpnn_v48_eps020.cpp:136-286.
 * Returns HKBS_INVALID_ARGUMENT for a malformed package and
 * HKBS_UNAVAILABLE when the device cannot be used. */
hkbs_status hkbs_pmpnn_create(const uint8_t* safetensors, size_t nbytes, int32_t device,
                              hkbs_pmpnn** out);

void hkbs_pmpnn_destroy(hkbs_pmpnn* ctx);

/* Batched autoregressive design: B sequences on one backbone of L residues.
 * Sequence b follows proteinmpnn_inverse_fold_scalar with
 * options.seed = sampler_seeds[b] and, for HKBS_ORDER_RANDOM,
 * options.decode_order_seed = order_seeds[b]; greedy != 0 or
 * temperature <= 0 selects argmax (cpp/modules/mpnn/sampler_scalar.cpp:106-131).
 * Outputs (host memory): tokens [B,L]; log_probs [B,L,21] temperature-scaled
 * (or NULL); orders_out [B,L] (or NULL); scores [B] mean NLL (or NULL).
 * Synchronous. */
hkbs_status hkbs_pmpnn_design(hkbs_pmpnn* ctx, const float* coords, const uint8_t* atom_sources,
                              const int32_t* residue_indices, const int32_t* chain_labels,
                              const float* chain_mask, const int32_t* true_tokens, int32_t L,
                              int32_t B, int32_t order_mode, const int32_t* orders,
                              const uint64_t* order_seeds, const uint64_t* sampler_seeds,
                              float temperature, int32_t greedy, int32_t* tokens,
                              float* log_probs, int32_t* orders_out, float* scores);

/* Device-resident variant: every pointer argument is device memory, orders
 * is [B,L] or [L] (shared != 0), and the call is enqueued on `stream`
 * (a hipStream_t; NULL = the context's stream) without synchronising.
 * residue_indices / chain_labels / chain_mask / true_tokens may be NULL.
 * When B leaves CUs free, each sequence is decoded by a team of up to eight
 * workgroups that must run at the same time; on a device busy with other
 * work a team can fail to assemble, and then that sequence's score is NaN
 * (the synchronous hkbs_pmpnn_design detects this and decodes again with one
 * workgroup per sequence). HKBS_DECODE_TEAM=1 in the environment disables
 * teams. An order that is not a permutation of 0..L-1 is not decoded: that
 * sequence's score is NaN and its tokens and log-probs are not written (the
 * reference rejects such an order, cpp/modules/mpnn/decode_order_scalar.cpp:67-79;
 * hkbs_pmpnn_design returns HKBS_INVALID_ARGUMENT for it). On a stream that is
 * not being captured the call's work waits, on the device, for the end of the
 * previous calls on the context, and the next call waits for its own end. */
hkbs_status hkbs_pmpnn_design_device(hkbs_pmpnn* ctx, const float* coords,
                                     const uint8_t* atom_sources, const int32_t* residue_indices,
                                     const int32_t* chain_labels, const float* chain_mask,
                                     const int32_t* true_tokens, int32_t L, int32_t B,
                                     const int32_t* orders, int32_t shared_order,
                                     const uint64_t* sampler_seeds, float temperature,
                                     int32_t greedy, int32_t* tokens, float* log_probs,
                                     float* scores, void* stream);

/* Allocation-free variant of hkbs_pmpnn_design_device, with the same arguments,
 * outputs and bits. No counterpart in the reference (its scalar path allocates
 * std::vector workspaces per call); it is for callers that cannot allocate
 * device memory: code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc. Its scratch (encoder states, decoder precompute,
 * per-sequence decoder state, decode schedule and step records, team barrier
 * counters, and the fp32 layer-0 message table when it fits beside the rest)
 * lives in one static device array of 128 MiB per GPU, which each GPU the
 * library runs on holds until the process ends; the call makes no hipMalloc or
 * hipFree. A request whose scratch exceeds 128 MiB returns
 * HKBS_INVALID_ARGUMENT (at L = 300: up to 205 sequences with a shared order,
 * 81 with one order per sequence; L = 4,000 does not fit). Results equal
 * hkbs_pmpnn_design_device's with or without the table. Every call on one
 * GPU shares that GPU's array and leaves its contents behind (what must start
 * at zero is cleared by a kernel in the call): calls that overlap on one GPU,
 * from any context or stream, race and must be serialised by the caller. On a
 * stream that is being captured into a HIP graph the call records its kernels
 * (no memset nodes) and neither waits for nor marks the end of other calls on
 * the context; the caller then orders the graph after earlier calls. */
hkbs_status hkbs_pmpnn_design_device_noalloc(hkbs_pmpnn* ctx, const float* coords,
                                             const uint8_t* atom_sources,
                                             const int32_t* residue_indices,
                                             const int32_t* chain_labels, const float* chain_mask,
                                             const int32_t* true_tokens, int32_t L, int32_t B,
                                             const int32_t* orders, int32_t shared_order,
                                             const uint64_t* sampler_seeds, float temperature,
                                             int32_t greedy, int32_t* tokens, float* log_probs,
                                             float* scores, void* stream);

/* Teacher-forced scoring of one protein (proteinmpnn_teacher_forced_forward_scalar,
 * cpp/modules/mpnn/inverse_fold_scalar.cpp:905-952): plain log_softmax
 * log-probs [L,21] and mean NLL. order may be NULL (N-to-C). Host memory.
 * Scoring runs in fp32 accuracy in every precision mode; its encoder is the
 * split-operand MFMA one (fp32-accurate, not the reference's rounding
 * sequence), since untempered log-probs leave room within 1e-4. */
hkbs_status hkbs_pmpnn_score(hkbs_pmpnn* ctx, const float* coords, const uint8_t* atom_sources,
                             const int32_t* residue_indices, const int32_t* chain_labels,
                             const float* chain_mask, const int32_t* tokens,
                             const int32_t* order, int32_t L, float* log_probs, float* score);

/* Teacher-forced scoring of a ragged batch of n single-chain proteins
 * (configuration "4,096 backbones, L in [50, 500]"): protein i holds residues
 * [offsets[i], offsets[i+1]) of coords [sum L,5,3], atom_sources [sum L,5] and
 * tokens [sum L]; orders (or NULL = N-to-C) holds each protein's permutation
 * of 0..L_i-1 at the same offsets. Outputs log_probs [sum L,21] and scores [n].
 * Proteins are processed in chunks that share K = min(48, L). Host memory;
 * synchronous. Chunks go up and results come back through two staging slots
 * of pinned host memory that the context keeps (each a chunk's inputs and
 * log-probs, about 14 MB for chunks of K = 48) while the neighbouring chunks
 * compute. */
hkbs_status hkbs_pmpnn_score_batch(hkbs_pmpnn* ctx, int32_t n, const int64_t* offsets, const float* coords,
                                   const uint8_t* atom_sources, const int32_t* tokens,
                                   const int32_t* orders, float* log_probs, float* scores);

/* Host helper: the reference's decoding order (decode_order_scalar.cpp:61-116)
 * for one sequence; chain_mask may be NULL. Bit-exact on the same libm. */
hkbs_status hkbs_pmpnn_decode_order(const float* chain_mask, const uint8_t* atom_sources,
                                    int32_t L, uint64_t seed, int32_t* order);

/* Host helper: out[L,5,3] = coords + the reference's backbone noise for one
 * sample (cpp/algorithms/inverse_fold.cpp:191-207, applied per sample with
 * that sample's seed by the per-sample loop at :292-310): mt19937_64 seeded
 * with seed ^ 0x4D504E4E76343875, std::normal_distribution<float>(0, sigma),
 * x/y/z of every present atom in order. out may equal coords. */
hkbs_status hkbs_pmpnn_backbone_noise(const float* coords, const uint8_t* atom_sources, int32_t L,
                                      float sigma, uint64_t seed, float* out);

/* Selects the arithmetic of later design and encode calls on this context
 * (teacher-forced scoring is the same in every mode; no counterpart in the
 * reference, which has only its fp32 scalar path). */
hkbs_status hkbs_pmpnn_set_precision(hkbs_pmpnn* ctx, int32_t precision);

/* Phase timing (instrumentation; no counterpart in the reference, which has
 * no design-path profiler). With timing enabled, each design call records
 * HIP events on the stream its kernels run on around three phases;
 * hkbs_pmpnn_last_timing waits for the last call and returns the elapsed
 * milliseconds of [featurise + encode, decoder precompute and decode
 * schedule, decode loop (the decode kernel alone)]. */
hkbs_status hkbs_pmpnn_set_timing(hkbs_pmpnn* ctx, int32_t enable);
hkbs_status hkbs_pmpnn_last_timing(hkbs_pmpnn* ctx, float* ms /* [3] */);

/* Unit-parity entry points (host memory in/out). */

/* CA kNN graph: idx [L,K] and squared distances d2 [L,K], K = min(48, L)
 * (knn_scalar, cpp/primitives/compute/knn_scalar.cpp:72-168). */
hkbs_status hkbs_pmpnn_knn(hkbs_pmpnn* ctx, const float* coords, const uint8_t* atom_sources,
                           int32_t L, int32_t* idx, float* d2);

/* Featurise + encode (inverse_fold_scalar.cpp:300-352): residue mask [L],
 * neighbour idx [L,K], node states h_V [L,128], edge states h_E [L,K,128], in
 * the context's precision (the design path's encoder). Any output may be NULL. */
hkbs_status hkbs_pmpnn_encode(hkbs_pmpnn* ctx, const float* coords, const uint8_t* atom_sources,
                              const int32_t* residue_indices, const int32_t* chain_labels,
                              int32_t L, float* mask, int32_t* idx, float* h_v, float* h_e);

/* Edge features [L,K,416] = [positional 16 | 25 atom pairs x 16 RBF]
 * (edge_rbf_features_scalar, cpp/modules/mpnn/edge_rbf_features_scalar.cpp:117-152). */
hkbs_status hkbs_pmpnn_edge_features(hkbs_pmpnn* ctx, const float* coords,
                                     const uint8_t* atom_sources, const int32_t* residue_indices,
                                     const int32_t* chain_labels, int32_t L, float* features);

#ifdef __cplusplus
}
#endif

#endif /* HKBS_PMPNN_H */
