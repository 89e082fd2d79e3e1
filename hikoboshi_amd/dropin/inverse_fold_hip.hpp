// MI355X drop-in for the reference's algorithm-level inverse fold, written
// against the reference's own public headers (hikoboshi/algorithms/
// inverse_fold.hpp, hikoboshi/universal/*.hpp) and the C ABI of this library
// (include/hkbs_pmpnn.h). It is the file a maintainer adds under the
// reference's reserved cpp/dispatch/hip/ directory; the Engine's backend gate
// (cpp/api/engine.cpp:139-146) then routes Backend::Hip requests here
// instead of to inverse_fold_proteinmpnn_v48_020 (cpp/algorithms/
// inverse_fold.cpp:221-356).
#ifndef HKBS_DROPIN_INVERSE_FOLD_HIP_HPP
#define HKBS_DROPIN_INVERSE_FOLD_HIP_HPP

#include <cstddef>
#include <cstdint>

#include <hikoboshi/algorithms/inverse_fold.hpp>
#include <hikoboshi/universal/status.hpp>

#include "hkbs_pmpnn.h"

namespace hikoboshi::dispatch::hip {

// True when the HIP library sees a device: what the Engine's backend gate and
// the capability report (cpp/api/version.cpp:40,
// cpp/dispatch/registry/capability.cpp:105) need to admit Backend::Hip.
[[nodiscard]] bool inverse_fold_available() noexcept;

// One HIP context per engine, created from the weight package bytes the
// engine already holds (the embedded v_48_020 safetensors blob).
class ProteinMpnnHip {
 public:
  ProteinMpnnHip() = default;
  ProteinMpnnHip(const ProteinMpnnHip&) = delete;
  ProteinMpnnHip& operator=(const ProteinMpnnHip&) = delete;
  ~ProteinMpnnHip();

  [[nodiscard]] universal::Status open(const std::uint8_t* package, std::size_t nbytes, int device);
  [[nodiscard]] hkbs_pmpnn* context() const noexcept { return ctx_; }

 private:
  hkbs_pmpnn* ctx_ = nullptr;
};

// Same request, result, validation, status codes and messages as
// inverse_fold_proteinmpnn_v48_020: sample i uses seed + i for its decoding
// order and its sampler stream. Without backbone noise the num_seqs samples
// are one batched design call (one encode, all sequences decoded together);
// with noise each sample is encoded from its own noised coordinates, as the
// reference's per-sample loop does.
[[nodiscard]] universal::Result<algorithms::InverseFoldResult> inverse_fold_proteinmpnn_v48_020_hip(
    const ProteinMpnnHip& engine, const algorithms::InverseFoldRequest& request);

}  // namespace hikoboshi::dispatch::hip

#endif  // HKBS_DROPIN_INVERSE_FOLD_HIP_HPP
