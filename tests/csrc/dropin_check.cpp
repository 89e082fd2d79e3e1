// Test shim: the C++ drop-in (hikoboshi_amd/dropin/inverse_fold_hip.cpp), built
// against the reference's own headers, called from Python through plain C
// entry points. Flattens the reference's InverseFoldResult into arrays.
#include <cstring>

#include <hikoboshi/universal/detail/proteinmpnn_v48_020_weights.hpp>

#include "inverse_fold_hip.hpp"

namespace hip = hikoboshi::dispatch::hip;
namespace a = hikoboshi::algorithms;
namespace u = hikoboshi::universal;

extern "C" {

int dropin_available(void) { return hip::inverse_fold_available() ? 1 : 0; }

// Opens an engine from the weight package bytes; returns a StatusCode value.
int dropin_open(const unsigned char* package, size_t nbytes, int device, void** engine, const char** detail) {
  auto* e = new hip::ProteinMpnnHip();
  const u::Status st = e->open(package, nbytes, device);
  *detail = st.detail;
  if (!st.ok()) {
    delete e;
    *engine = nullptr;
    return static_cast<int>(st.code);
  }
  *engine = e;
  return 0;
}

void dropin_close(void* engine) { delete static_cast<hip::ProteinMpnnHip*>(engine); }

// One InverseFoldRequest on a structure given as arrays (residue_codes may be
// null); with_weights = 0 leaves request.weights null. Outputs: sequences
// [n * L] letters, scores, recovery values and validity, seeds, decode order
// (0 random, 1 N-to-C) per sequence, and log-probs [n, L, 21] when keep != 0
// (*lp_count receives the number of values written).
int dropin_inverse_fold(void* engine, const float* coords, const unsigned char* atom_sources, const char* residue_codes,
                        size_t L, size_t num_seqs, unsigned long long seed, float temperature, int n_to_c,
                        float backbone_noise, int keep, int with_weights, char* sequences, double* scores,
                        double* recovery, int* recovery_valid, unsigned long long* seeds, int* orders, float* log_probs,
                        size_t* lp_count, const char** detail) {
  static const u::detail::ProteinMpnnV48020Weights view{};
  a::InverseFoldRequest req{};
  req.structure.residue_count = L;
  req.structure.coordinates = {coords, L * u::kCanonicalAtomCount * u::kCoordinateAxisCount};
  req.structure.atom_sources = {reinterpret_cast<const u::AtomSource*>(atom_sources), L * u::kCanonicalAtomCount};
  if (residue_codes) req.structure.residue_codes = {residue_codes, L};
  req.weights = with_weights ? &view : nullptr;
  req.options.sampling_temp = temperature;
  req.options.num_seqs = num_seqs;
  req.options.seed = seed;
  req.options.decode_order = n_to_c ? a::InverseFoldDecodeOrder::NToC : a::InverseFoldDecodeOrder::Random;
  req.options.backbone_noise = backbone_noise;
  req.options.keep_log_probs = keep != 0;
  const auto res = hip::inverse_fold_proteinmpnn_v48_020_hip(*static_cast<hip::ProteinMpnnHip*>(engine), req);
  *detail = res.status.detail;
  *lp_count = 0;
  if (!res.ok()) return static_cast<int>(res.status.code);
  for (size_t i = 0; i < res.value.sequences.size(); ++i) {
    const a::InverseFoldSequence& s = res.value.sequences[i];
    std::memcpy(sequences + i * L, s.sequence.data(), L);
    scores[i] = s.score;
    recovery[i] = s.recovery_vs_native.value;
    recovery_valid[i] = s.recovery_vs_native.valid ? 1 : 0;
    seeds[i] = s.seed;
    orders[i] = s.decode_order == a::InverseFoldDecodeOrder::NToC ? 1 : 0;
  }
  const std::vector<float>& v = res.value.logprobs.values;
  if (!v.empty()) std::memcpy(log_probs, v.data(), v.size() * sizeof(float));
  *lp_count = v.size();
  return 0;
}

}  // extern "C"
