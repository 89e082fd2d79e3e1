/*
 * CPU oracle for the ProteinMPNN v_48_020 design path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference's
 * scalar C++ path, used as the checker for the HIP library. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it. The
 * product path (hikoboshi_amd/) never calls it.
 *
 * Each function names the reference file:line it follows. Floating-point
 * operations are written in the reference's order and the file is built with
 * -ffp-contract=off, so on x86-64 every stage is bit-identical to the
 * reference compiled the same way (checked against oracle/_ref in tests).
 *
 * Pinning (see tests/test_oracle.py):
 *   - pmo_knn:               reference known-answer cases + brute-force sort
 *                            + bit-exact vs oracle/_ref.
 *   - pmo_fast_exp_neg/gelu: vs libm exp/erf bounds (5e-5) + closed points.
 *   - pmo_edge_features..pmo_teacher_forced: the 5 committed PyTorch goldens
 *                            (1e-4) + bit-exact vs oracle/_ref.
 *   - pmo_decode_order:      permutation/monotone invariants + bit-exact vs
 *                            oracle/_ref.
 *   - pmo_decode (sampler):  bit-exact vs oracle/_ref design outputs,
 *                            invariants (sum p = 1, greedy = argmax).
 */
#ifndef HKBS_PMPNN_ORACLE_H
#define HKBS_PMPNN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  PMO_H = 128,
  PMO_V = 21,
  PMO_KMAX = 48,
  PMO_RBF = 16,
  PMO_PAIRS = 25,
  PMO_POS = 16,
  PMO_POS_CLASSES = 66,
  PMO_EDGE_IN = 416,
  PMO_FF = 512,
  PMO_LAYERS = 3,
  PMO_TENSORS = 118
};

typedef struct pmo_model pmo_model;

/* tensors: 118 row-major float arrays in the canonical order documented in
 * hikoboshi_amd/weights.py (CANONICAL_TENSORS). */
pmo_model* pmo_model_create(const float* const* tensors);
void pmo_model_destroy(pmo_model* model);

float pmo_fast_exp_neg(float x);
float pmo_gelu(float x);

void pmo_knn(const float* ca, const uint8_t* valid, int32_t L, int32_t K,
             int32_t* idx, float* d2);

int pmo_edge_features(const pmo_model* m, const float* coords,
                      const uint8_t* atom_src, const int32_t* resid,
                      const int32_t* chain, int32_t L, int32_t* idx,
                      float* features);

int pmo_encode(const pmo_model* m, const float* coords, const uint8_t* atom_src,
               const int32_t* resid, const int32_t* chain, int32_t L,
               float* mask, int32_t* idx, float* h_v, float* h_e);

int pmo_decode_order(const float* chain_mask, const float* residue_mask,
                     int32_t L, uint64_t seed, const int32_t* input_order,
                     int use_input_order, int32_t* order);

int pmo_decode(const pmo_model* m, const float* mask, const int32_t* idx,
               const float* h_v, const float* h_e, int32_t L,
               const float* chain_mask, const int32_t* true_tokens,
               const int32_t* order, uint64_t seed, float temperature,
               int greedy, const int32_t* forced_tokens, int32_t* tokens,
               float* log_probs, float* score, int32_t* sampled,
               double* cdf_gap);

int pmo_teacher_forced_decode(const pmo_model* m, const float* mask,
                              const int32_t* idx, const float* h_v,
                              const float* h_e, int32_t L,
                              const float* chain_mask, const int32_t* tokens,
                              const int32_t* order, float* log_probs,
                              float* score);

int pmo_inverse_fold(const pmo_model* m, const float* coords,
                     const uint8_t* atom_src, int32_t L, const int32_t* resid,
                     const int32_t* chain, const float* chain_mask,
                     const int32_t* input_order, const int32_t* true_tokens,
                     uint64_t seed, uint64_t order_seed, float temperature,
                     int greedy, int use_input_order, int32_t* tokens,
                     float* log_probs, int32_t* order_out, float* score);

int pmo_teacher_forced(const pmo_model* m, const float* coords,
                       const uint8_t* atom_src, int32_t L,
                       const int32_t* resid, const int32_t* chain,
                       const float* chain_mask, const int32_t* tokens,
                       const int32_t* input_order, float* log_probs,
                       float* score);

int pmo_algorithm_inverse_fold(const pmo_model* m, const float* coords,
                               const uint8_t* atom_src, int32_t L,
                               int32_t num_seqs, uint64_t seed,
                               float temperature, int n_to_c,
                               int32_t* tokens, float* log_probs,
                               float* scores);

#ifdef __cplusplus
}
#endif

#endif
