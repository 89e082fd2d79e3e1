// See inverse_fold_hip.hpp. Reference behaviour mirrored here:
// cpp/algorithms/inverse_fold.cpp:221-356 (validation and its messages, seed + i
// per sample, N-to-C order, greedy at T <= 0, log-prob concatenation, per-sample
// backbone noise) and :160-184 (recovery against the native residue codes).
#include "inverse_fold_hip.hpp"

#include <cmath>
#include <string_view>
#include <utility>
#include <vector>

namespace hikoboshi::dispatch::hip {
namespace {

namespace u = hikoboshi::universal;
namespace a = hikoboshi::algorithms;

constexpr std::size_t kAtoms = u::kCanonicalAtomCount;
constexpr std::size_t kAxes = u::kCoordinateAxisCount;
constexpr std::size_t kVocab = 21;
constexpr std::string_view kAlphabet = "ACDEFGHIKLMNPQRSTVWYX";
constexpr std::string_view kStandard = "ACDEFGHIKLMNPQRSTVWY";

u::Status from_hkbs(hkbs_status st) {
  if (st == HKBS_OK) return u::ok_status();
  return u::make_status(static_cast<u::StatusCode>(st), hkbs_last_error());
}

char upper(char c) { return (c >= 'a' && c <= 'z') ? static_cast<char>(c - 'a' + 'A') : c; }

// Fraction of the native standard residues whose designed letter matches.
u::MetricValue recovery(const std::string& designed, u::Span<const char> native, std::size_t n) {
  if (native.data == nullptr || native.size < n) return {0.0, false, u::MetricInvalidReason::MissingStructureMetadata};
  std::size_t compared = 0, same = 0;
  for (std::size_t i = 0; i < n && i < designed.size(); ++i) {
    const char c = upper(native.data[i]);
    if (kStandard.find(c) == std::string_view::npos) continue;
    ++compared;
    same += upper(designed[i]) == c ? 1U : 0U;
  }
  if (compared == 0) return {0.0, false, u::MetricInvalidReason::MissingStructureMetadata};
  return {static_cast<double>(same) / static_cast<double>(compared), true, u::MetricInvalidReason::None};
}

}  // namespace

bool inverse_fold_available() noexcept { return hkbs_device_count() > 0; }

ProteinMpnnHip::~ProteinMpnnHip() { hkbs_pmpnn_destroy(ctx_); }

u::Status ProteinMpnnHip::open(const std::uint8_t* package, std::size_t nbytes, int device) {
  hkbs_pmpnn_destroy(ctx_);
  ctx_ = nullptr;
  return from_hkbs(hkbs_pmpnn_create(package, nbytes, device, &ctx_));
}

u::Result<a::InverseFoldResult> inverse_fold_proteinmpnn_v48_020_hip(const ProteinMpnnHip& engine,
                                                                    const a::InverseFoldRequest& request) {
  a::InverseFoldResult result{};
  const u::StructureView& s = request.structure;
  const std::size_t L = s.residue_count;
  const a::InverseFoldOptions& o = request.options;
  if (request.weights == nullptr)
    return {u::failed_precondition_status("ProteinMPNN inverse-folding weights are not available"), result};
  if (L == 0) return {u::invalid_argument_status("inverse-fold structure must contain at least one residue"), result};
  if (s.coordinates.data == nullptr || s.coordinates.size < L * kAtoms * kAxes || s.atom_sources.data == nullptr ||
      s.atom_sources.size < L * kAtoms)
    return {u::invalid_argument_status("inverse-fold structure must provide canonical backbone atoms"), result};
  if (o.num_seqs == 0) return {u::invalid_argument_status("inverse-fold num_seqs must be greater than zero"), result};
  if (!std::isfinite(o.sampling_temp) || o.sampling_temp < 0.0F)
    return {u::invalid_argument_status("inverse-fold sampling_temp must be finite and >= 0"), result};
  if (!std::isfinite(o.backbone_noise) || o.backbone_noise < 0.0F)
    return {u::invalid_argument_status("inverse-fold backbone_noise must be finite and >= 0"), result};
  if (engine.context() == nullptr)
    return {u::failed_precondition_status("HIP inverse-fold context is not open"), result};

  const a::InverseFoldDecodeOrder order =
      o.decode_order == a::InverseFoldDecodeOrder::NToC ? a::InverseFoldDecodeOrder::NToC : a::InverseFoldDecodeOrder::Random;
  const int32_t mode = order == a::InverseFoldDecodeOrder::NToC ? HKBS_ORDER_N_TO_C : HKBS_ORDER_RANDOM;
  const std::size_t B = o.num_seqs;
  const float* coords = s.coordinates.data;
  const auto* src = reinterpret_cast<const std::uint8_t*>(s.atom_sources.data);
  std::vector<std::uint64_t> seeds(B);
  for (std::size_t i = 0; i < B; ++i) seeds[i] = o.seed + static_cast<std::uint64_t>(i);
  std::vector<std::int32_t> tokens(B * L);
  std::vector<float> log_probs(B * L * kVocab);
  std::vector<float> scores(B);
  const int greedy = o.sampling_temp <= 0.0F ? 1 : 0;
  if (o.backbone_noise > 0.0F) {
    std::vector<float> noisy(L * kAtoms * kAxes);
    for (std::size_t i = 0; i < B; ++i) {
      hkbs_status st = hkbs_pmpnn_backbone_noise(coords, src, static_cast<int32_t>(L), o.backbone_noise, seeds[i],
                                                 noisy.data());
      if (st == HKBS_OK)
        st = hkbs_pmpnn_design(engine.context(), noisy.data(), src, nullptr, nullptr, nullptr, nullptr,
                               static_cast<int32_t>(L), 1, mode, nullptr, &seeds[i], &seeds[i], o.sampling_temp, greedy,
                               tokens.data() + i * L, log_probs.data() + i * L * kVocab, nullptr, &scores[i]);
      if (st != HKBS_OK) return {from_hkbs(st), result};
    }
  } else {
    const hkbs_status st = hkbs_pmpnn_design(engine.context(), coords, src, nullptr, nullptr, nullptr, nullptr,
                                             static_cast<int32_t>(L), static_cast<int32_t>(B), mode, nullptr,
                                             seeds.data(), seeds.data(), o.sampling_temp, greedy, tokens.data(),
                                             log_probs.data(), nullptr, scores.data());
    if (st != HKBS_OK) return {from_hkbs(st), result};
  }
  result.sequences.reserve(B);
  for (std::size_t i = 0; i < B; ++i) {
    a::InverseFoldSequence entry{};
    entry.sequence.resize(L);
    for (std::size_t r = 0; r < L; ++r) {
      const std::int32_t t = tokens[i * L + r];
      entry.sequence[r] = (t >= 0 && t < static_cast<std::int32_t>(kVocab)) ? kAlphabet[static_cast<std::size_t>(t)] : 'X';
    }
    entry.score = static_cast<double>(scores[i]);
    entry.recovery_vs_native = recovery(entry.sequence, s.residue_codes, L);
    entry.seed = seeds[i];
    entry.decode_order = order;
    result.sequences.push_back(std::move(entry));
  }
  if (o.keep_log_probs) {
    result.logprobs.num_seqs = B;
    result.logprobs.residue_count = L;
    result.logprobs.vocab_size = kVocab;
    result.logprobs.values = std::move(log_probs);
  }
  return {u::ok_status(), std::move(result)};
}

}  // namespace hikoboshi::dispatch::hip
