// C entry points around the reference's own ProteinMPNN v_48_020 functions.
//
// TEST INFRASTRUCTURE ONLY. oracle/ref.mk compiles this file together with
// the reference's unmodified sources (read in place under the reference
// checkout) into oracle/_ref/libhkbs_ref.so. Tests use it to pin the C
// oracle bit-for-bit; bench.py times ref_algorithm_inverse_fold as the CPU
// baseline ("kind": "reference"). Nothing in the product links it.
//
// The weight view is filled from 118 caller-owned float arrays in the
// canonical order of hikoboshi_amd/weights.py, mirroring how the reference
// binds its embedded blob (cpp/weights/embedded_proteinmpnn_v48_eps020.cpp:
// 136-286) without needing the generated blob translation unit.

#include <hikoboshi/algorithms/inverse_fold.hpp>
#include <hikoboshi/api/results.hpp>
#include <hikoboshi/io/atom_inference.hpp>
#include <hikoboshi/io/design_fasta_writer.hpp>
#include <hikoboshi/io/residue_table.hpp>
#include <hikoboshi/io/structure_loader.hpp>
#include <hikoboshi/modules/detail/mpnn_workspace.hpp>
#include <hikoboshi/modules/mpnn/inverse_fold.hpp>
#include <hikoboshi/modules/mpnn/proteinmpnn_decoder.hpp>
#include <hikoboshi/primitives/compute/knn.hpp>
#include <hikoboshi/universal/detail/proteinmpnn_v48_020_weights.hpp>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

namespace {

namespace hd = hikoboshi::modules::detail;
namespace hm = hikoboshi::modules::mpnn;
namespace hu = hikoboshi::universal;
namespace pmp = hikoboshi::universal::detail;

constexpr std::size_t kH = pmp::kProteinMpnnV48020Hidden;

pmp::ProteinMpnnV48020Weights g_weights{};

hu::Span<const float> sp(const float* p, std::size_t n) { return {p, n}; }

void bind_linear(pmp::ProteinMpnnV48020LinearWeights& l, const float* w, const float* b,
                 std::size_t out, std::size_t in) {
  l.weight = sp(w, out * in);
  l.bias = sp(b, out);
}

void bind_norm(pmp::ProteinMpnnV48020NormWeights& n, const float* g, const float* b) {
  n.weight = sp(g, kH);
  n.bias = sp(b, kH);
}

template <typename T>
hu::Span<T> span_of(std::vector<T>& v) {
  return {v.empty() ? nullptr : v.data(), v.size()};
}

// Workspace sizing follows cpp/algorithms/inverse_fold.cpp:39-124.
struct EncoderStorage {
  EncoderStorage(std::size_t L, std::size_t K)
      : plan{L, kH, K, pmp::kProteinMpnnV48020RbfCount, pmp::kProteinMpnnV48020NumEncoderLayers},
        ca(hd::mpnn64_ca_coordinate_count(plan)),
        features(std::max(hd::mpnn64_residue_feature_count(plan),
                          hd::mpnn64_neighbor_slot_count(plan) * 3U * kH)),
        idx(hd::mpnn64_neighbor_slot_count(plan)),
        d2(hd::mpnn64_neighbor_slot_count(plan)),
        rbf(hd::mpnn64_neighbor_rbf_count(plan)),
        residue(hd::mpnn64_residue_hidden_count(plan)),
        gathered(hd::mpnn64_neighbor_hidden_count(plan)),
        edge(hd::mpnn64_neighbor_hidden_count(plan)),
        message(hd::mpnn64_neighbor_hidden_count(plan)),
        projected(hd::mpnn64_neighbor_hidden_count(plan)),
        scratch(hd::mpnn64_residue_hidden_count(plan)),
        ffn(hd::mpnn64_ffn_hidden_count(plan)) {}
  hd::Mpnn64Workspace view() {
    return {plan, span_of(ca), span_of(features), span_of(idx), span_of(d2), span_of(rbf),
            span_of(residue), span_of(gathered), span_of(edge), span_of(message),
            span_of(projected), span_of(scratch), span_of(ffn)};
  }
  hd::Mpnn64MemoryPlan plan;
  std::vector<float> ca, features;
  std::vector<std::int32_t> idx;
  std::vector<float> d2, rbf, residue, gathered, edge, message, projected, scratch, ffn;
};

struct DecoderStorage {
  DecoderStorage(std::size_t L, std::size_t K)
      : plan{std::max<std::size_t>(L, 1U), kH, K, pmp::kProteinMpnnV48020DecoderNumInDimension,
             pmp::kProteinMpnnV48020FfnHidden},
        input(hm::proteinmpnn_decoder_message_input_count(plan)),
        message(hm::proteinmpnn_decoder_neighbor_hidden_count(plan)),
        projected(hm::proteinmpnn_decoder_neighbor_hidden_count(plan)),
        scratch(hm::proteinmpnn_decoder_residue_hidden_count(plan)),
        ffn(hm::proteinmpnn_decoder_ffn_hidden_count(plan)) {}
  hm::ProteinMpnnDecoderWorkspace view() {
    return {plan, span_of(input), span_of(message), span_of(projected), span_of(scratch),
            span_of(ffn)};
  }
  hm::ProteinMpnnDecoderMemoryPlan plan;
  std::vector<float> input, message, projected, scratch, ffn;
};

int code(hu::Status s) { return static_cast<int>(s.code); }

}  // namespace

extern "C" {

void ref_set_weights(const float* const* t) {
  auto& w = g_weights;
  w.features.embeddings.linear.weight = sp(t[0], 16 * 66);
  w.features.embeddings.linear.bias = sp(t[1], 16);
  w.features.edge_embedding.weight = sp(t[2], kH * 416);
  bind_norm(w.features.norm_edges, t[3], t[4]);
  bind_linear(w.W_e, t[5], t[6], kH, kH);
  w.W_s.weight = sp(t[7], 21 * kH);
  for (int l = 0; l < 3; ++l) {
    const float* const* e = t + 8 + 22 * l;
    auto& L = w.encoder_layers[l];
    bind_linear(L.W1, e[0], e[1], kH, 3 * kH);
    bind_linear(L.W2, e[2], e[3], kH, kH);
    bind_linear(L.W3, e[4], e[5], kH, kH);
    bind_linear(L.W11, e[6], e[7], kH, 3 * kH);
    bind_linear(L.W12, e[8], e[9], kH, kH);
    bind_linear(L.W13, e[10], e[11], kH, kH);
    bind_norm(L.norm1, e[12], e[13]);
    bind_norm(L.norm2, e[14], e[15]);
    bind_norm(L.norm3, e[16], e[17]);
    bind_linear(L.dense.W_in, e[18], e[19], 4 * kH, kH);
    bind_linear(L.dense.W_out, e[20], e[21], kH, 4 * kH);
  }
  for (int l = 0; l < 3; ++l) {
    const float* const* d = t + 74 + 14 * l;
    auto& L = w.decoder_layers[l];
    bind_linear(L.W1, d[0], d[1], kH, 4 * kH);
    bind_linear(L.W2, d[2], d[3], kH, kH);
    bind_linear(L.W3, d[4], d[5], kH, kH);
    bind_norm(L.norm1, d[6], d[7]);
    bind_norm(L.norm2, d[8], d[9]);
    bind_linear(L.dense.W_in, d[10], d[11], 4 * kH, kH);
    bind_linear(L.dense.W_out, d[12], d[13], kH, 4 * kH);
  }
  bind_linear(w.W_out, t[116], t[117], 21, kH);
}

void ref_knn(const float* ca, const std::uint8_t* valid, std::int32_t L, std::int32_t K,
             std::int32_t* idx, float* d2) {
  hikoboshi::primitives::compute::KnnScalarRequest r{};
  r.query_coordinates = ca;
  r.target_coordinates = ca;
  r.query_validity_mask = valid;
  r.target_validity_mask = valid;
  r.query_count = static_cast<std::size_t>(L);
  r.target_count = static_cast<std::size_t>(L);
  r.k = static_cast<std::size_t>(K);
  r.include_self = true;
  r.treat_zero_coords_as_invalid = false;
  hikoboshi::primitives::compute::KnnScalarOutput o{idx, d2};
  hikoboshi::primitives::compute::knn_scalar(r, o);
}

int ref_inverse_fold(const float* coords, const std::uint8_t* atom_src, std::int32_t L,
                     const std::int32_t* resid, const std::int32_t* chain,
                     const float* chain_mask, const std::int32_t* input_order,
                     const std::int32_t* true_tokens, std::uint64_t seed,
                     std::uint64_t order_seed, float temperature, int greedy,
                     int use_input_order, std::int32_t* tokens, float* log_probs,
                     std::int32_t* order_out, float* score) {
  const std::size_t n = static_cast<std::size_t>(L);
  const std::size_t K = hm::proteinmpnn_v48_020_effective_neighbor_count(n);
  EncoderStorage es(n, K);
  DecoderStorage ds(n, K);
  hd::Mpnn64Workspace ew = es.view();
  hm::ProteinMpnnDecoderWorkspace dw = ds.view();
  std::vector<char> seq(n + 1U, '\0');
  hm::ProteinMpnnInverseFoldRequest req{};
  req.coordinates = coords;
  req.atom_sources = reinterpret_cast<const hu::AtomSource*>(atom_src);
  req.weights = &g_weights;
  req.encoder_workspace = &ew;
  req.decoder_workspace = &dw;
  req.residue_count = n;
  req.residue_indices = resid;
  req.chain_labels = chain;
  req.chain_mask = chain_mask;
  req.input_decoding_order = input_order;
  req.true_token_ids = true_tokens;
  req.options.seed = seed;
  req.options.decode_order_seed = order_seed;
  req.options.temperature = temperature;
  req.options.greedy = greedy != 0;
  req.options.use_input_decoding_order = use_input_order != 0;
  hm::ProteinMpnnInverseFoldOutput out{};
  out.token_ids = tokens;
  out.sequence = seq.data();
  out.log_probs = log_probs;
  out.decoding_order = order_out;
  out.sequence_score = score;
  out.residue_count = n;
  out.vocab_size = 21;
  return code(hm::proteinmpnn_inverse_fold_scalar(req, out));
}

int ref_teacher_forced(const float* coords, const std::uint8_t* atom_src, std::int32_t L,
                       const std::int32_t* resid, const std::int32_t* chain,
                       const float* chain_mask, const std::int32_t* tokens,
                       const std::int32_t* input_order, float* log_probs, float* score) {
  const std::size_t n = static_cast<std::size_t>(L);
  const std::size_t K = hm::proteinmpnn_v48_020_effective_neighbor_count(n);
  EncoderStorage es(n, K);
  DecoderStorage ds(n, K);
  hd::Mpnn64Workspace ew = es.view();
  hm::ProteinMpnnDecoderWorkspace dw = ds.view();
  std::vector<std::int32_t> iota(n);
  for (std::size_t i = 0; i < n; ++i) iota[i] = static_cast<std::int32_t>(i);
  std::vector<std::int32_t> order(n, -1);
  hm::ProteinMpnnTeacherForcedRequest req{};
  req.coordinates = coords;
  req.atom_sources = reinterpret_cast<const hu::AtomSource*>(atom_src);
  req.token_ids = tokens;
  req.weights = &g_weights;
  req.encoder_workspace = &ew;
  req.decoder_workspace = &dw;
  req.residue_count = n;
  req.residue_indices = resid;
  req.chain_labels = chain;
  req.chain_mask = chain_mask;
  req.input_decoding_order = input_order != nullptr ? input_order : iota.data();
  req.options.use_input_decoding_order = true;
  hm::ProteinMpnnTeacherForcedOutput out{};
  out.log_probs = log_probs;
  out.decoding_order = order.data();
  out.sequence_score = score;
  out.residue_count = n;
  out.vocab_size = 21;
  return code(hm::proteinmpnn_teacher_forced_forward_scalar(req, out));
}

// cpp/algorithms/inverse_fold.cpp:221-356 called as the API does, for the
// CPU baseline. tokens [N,L] and log_probs [N,L,21] are written from the
// result's sequences / log-prob block.
int ref_algorithm_inverse_fold(const float* coords, const std::uint8_t* atom_src,
                               std::int32_t L, std::int32_t num_seqs, std::uint64_t seed,
                               float temperature, int n_to_c, std::int32_t* tokens,
                               float* log_probs, float* scores) {
  const std::size_t n = static_cast<std::size_t>(L);
  std::vector<char> codes(n, 'X');
  hikoboshi::algorithms::InverseFoldRequest req{};
  req.structure.residue_count = n;
  req.structure.coordinates = sp(coords, n * 15U);
  req.structure.atom_sources = {reinterpret_cast<const hu::AtomSource*>(atom_src), n * 5U};
  req.structure.residue_codes = {codes.data(), n};
  req.structure.residues = {nullptr, 0};
  req.weights = &g_weights;
  req.options.sampling_temp = temperature;
  req.options.num_seqs = static_cast<std::size_t>(num_seqs);
  req.options.seed = seed;
  req.options.decode_order = n_to_c ? hikoboshi::algorithms::InverseFoldDecodeOrder::NToC
                                    : hikoboshi::algorithms::InverseFoldDecodeOrder::Random;
  req.options.keep_log_probs = true;
  const auto result = hikoboshi::algorithms::inverse_fold_proteinmpnn_v48_020(req);
  if (!result.status.ok()) return code(result.status);
  static const char kAlphabet[] = "ACDEFGHIKLMNPQRSTVWYX";
  for (std::size_t i = 0; i < result.value.sequences.size(); ++i) {
    const auto& s = result.value.sequences[i];
    scores[i] = static_cast<float>(s.score);
    for (std::size_t r = 0; r < n; ++r) {
      const char* hit = std::strchr(kAlphabet, s.sequence[r]);
      tokens[i * n + r] = hit ? static_cast<std::int32_t>(hit - kAlphabet) : 20;
    }
  }
  std::memcpy(log_probs, result.value.logprobs.values.data(),
              result.value.logprobs.values.size() * sizeof(float));
  return 0;
}

// The algorithm-level loop with backbone noise and native residue codes (for
// recovery_vs_native): recovery[i] = value, recovery_valid[i] = 0/1.
int ref_algorithm_inverse_fold_ex(const float* coords, const std::uint8_t* atom_src, const char* residue_codes,
                                  std::int32_t L, std::int32_t num_seqs, std::uint64_t seed, float temperature,
                                  int n_to_c, float backbone_noise, std::int32_t* tokens, float* log_probs,
                                  double* scores, double* recovery, std::int32_t* recovery_valid) {
  const std::size_t n = static_cast<std::size_t>(L);
  hikoboshi::algorithms::InverseFoldRequest req{};
  req.structure.residue_count = n;
  req.structure.coordinates = sp(coords, n * 15U);
  req.structure.atom_sources = {reinterpret_cast<const hu::AtomSource*>(atom_src), n * 5U};
  req.structure.residue_codes = {residue_codes, residue_codes ? n : 0};
  req.structure.residues = {nullptr, 0};
  req.weights = &g_weights;
  req.options.sampling_temp = temperature;
  req.options.num_seqs = static_cast<std::size_t>(num_seqs);
  req.options.seed = seed;
  req.options.decode_order = n_to_c ? hikoboshi::algorithms::InverseFoldDecodeOrder::NToC
                                    : hikoboshi::algorithms::InverseFoldDecodeOrder::Random;
  req.options.backbone_noise = backbone_noise;
  req.options.keep_log_probs = true;
  const auto result = hikoboshi::algorithms::inverse_fold_proteinmpnn_v48_020(req);
  if (!result.status.ok()) return code(result.status);
  static const char kAlphabet[] = "ACDEFGHIKLMNPQRSTVWYX";
  for (std::size_t i = 0; i < result.value.sequences.size(); ++i) {
    const auto& s = result.value.sequences[i];
    scores[i] = s.score;
    recovery[i] = s.recovery_vs_native.value;
    recovery_valid[i] = s.recovery_vs_native.valid ? 1 : 0;
    for (std::size_t r = 0; r < n; ++r) {
      const char* hit = std::strchr(kAlphabet, s.sequence[r]);
      tokens[i * n + r] = hit ? static_cast<std::int32_t>(hit - kAlphabet) : 20;
    }
  }
  std::memcpy(log_probs, result.value.logprobs.values.data(),
              result.value.logprobs.values.size() * sizeof(float));
  return 0;
}

// The reference's FASTA and NPZ writers on a result assembled from plain
// arrays: sequences [n][L] letters, scores [n], seeds [n]. An empty path
// skips that writer.
int ref_write_design_outputs(const char* fasta_path, const char* npz_path, std::int32_t num_seqs, std::int32_t L,
                             const char* sequences, const double* scores, const std::uint64_t* seeds, int n_to_c,
                             float temperature, const float* log_probs) {
  hikoboshi::api::InverseFoldResult res{};
  for (std::int32_t i = 0; i < num_seqs; ++i) {
    hikoboshi::api::InverseFoldSequenceResult s{};
    s.sequence.assign(sequences + static_cast<std::size_t>(i) * L, static_cast<std::size_t>(L));
    s.score = scores[i];
    s.seed = seeds[i];
    s.decode_order = n_to_c ? hikoboshi::api::InverseFoldDecodeOrder::NToC : hikoboshi::api::InverseFoldDecodeOrder::Random;
    res.sequences.push_back(std::move(s));
  }
  res.logprobs.num_seqs = static_cast<std::size_t>(num_seqs);
  res.logprobs.residue_count = static_cast<std::size_t>(L);
  res.logprobs.vocab_size = 21;
  if (log_probs) res.logprobs.values.assign(log_probs, log_probs + static_cast<std::size_t>(num_seqs) * L * 21);
  if (fasta_path && fasta_path[0]) {
    hikoboshi::io::DesignFastaWriterOptions opt{};
    opt.sampling_temp = temperature;
    const hu::Status st = hikoboshi::io::write_design_fasta(fasta_path, res, opt);
    if (!st.ok()) return code(st);
  }
  if (npz_path && npz_path[0]) {
    const hu::Status st = hikoboshi::io::write_inverse_fold_logprobs_npz(npz_path, res);
    if (!st.ok()) return code(st);
  }
  return 0;
}

// ------------------------------------------------------------------------
// The reference's structure loader (cpp/io/structure_loader.cpp) behind an
// opaque handle. source: 0 = file at path, 1 = PDB text, 2 = mmCIF text.
// Options follow StructureLoadOptions; returns the StatusCode value and sets
// *detail to the status detail.
int ref_structure_load(int source, const char* path, const char* content, std::size_t nbytes, const char* label,
                       int has_model_index, int model_index, const char* model_id, const char* chain_id,
                       int has_chain_index, std::uint64_t chain_index, int infer, int include_modified,
                       void** out, const char** detail) {
  namespace io = hikoboshi::io;
  io::StructureLoadOptions opt{};
  if (has_model_index) opt.model_index = model_index;
  if (model_id) opt.model_id = model_id;
  if (chain_id) opt.chain_id = chain_id;
  if (has_chain_index) opt.chain_index = static_cast<std::size_t>(chain_index);
  opt.infer_missing_atoms = infer != 0;
  opt.include_modified_residues = include_modified != 0;
  const std::string_view text(content ? content : "", content ? nbytes : 0);
  const std::string_view origin(label ? label : "");
  hu::Result<io::LoadedStructure> r = source == 0   ? io::load_structure_from_file(path, opt)
                                      : source == 1 ? io::load_pdb_from_string(text, origin, opt)
                                                    : io::load_mmcif_from_string(text, origin, opt);
  *detail = r.status.detail ? r.status.detail : "";
  *out = nullptr;
  if (!r.status.ok()) return code(r.status);
  *out = new io::LoadedStructure(std::move(r.value));
  return 0;
}

void ref_structure_free(void* h) { delete static_cast<hikoboshi::io::LoadedStructure*>(h); }

std::size_t ref_structure_count(void* h) { return static_cast<hikoboshi::io::LoadedStructure*>(h)->residue_count(); }

// coords [L,5,3], sources [L,5], codes [L], numbers [L], icodes [L],
// records [L] (source_record_index), breaks [n_breaks] (returns n_breaks).
std::size_t ref_structure_arrays(void* h, float* coords, std::uint8_t* sources, char* codes, std::int32_t* numbers,
                                 char* icodes, std::int64_t* records, std::uint64_t* breaks) {
  const hu::StructureView v = static_cast<hikoboshi::io::LoadedStructure*>(h)->view();
  std::memcpy(coords, v.coordinates.data, v.coordinates.size * sizeof(float));
  for (std::size_t i = 0; i < v.atom_sources.size; ++i) sources[i] = static_cast<std::uint8_t>(v.atom_sources.data[i]);
  for (std::size_t i = 0; i < v.residue_count; ++i) {
    codes[i] = v.residue_codes.data[i];
    numbers[i] = v.residues.data[i].residue_number;
    icodes[i] = v.residues.data[i].insertion_code;
    records[i] = v.residues.data[i].source_record_index;
  }
  if (breaks)
    for (std::size_t i = 0; i < v.chain_breaks.size; ++i) breaks[i] = v.chain_breaks.data[i].after_residue_index;
  return v.chain_breaks.size;
}

// 0 input id, 1 source filename, 2 selected model id, 3 selected chain id,
// 4 altloc note, 5 + i: original residue name of residue i.
const char* ref_structure_text(void* h, std::size_t field) {
  static thread_local std::string buf;
  const auto* s = static_cast<hikoboshi::io::LoadedStructure*>(h);
  switch (field) {
    case 0: buf = std::string(s->input_id()); break;
    case 1: buf = std::string(s->source_filename()); break;
    case 2: buf = std::string(s->selected_model_id()); break;
    case 3: buf = std::string(s->selected_chain_id()); break;
    case 4: buf = std::string(s->altloc_note()); break;
    default: buf = std::string(s->view().residues.data[field - 5].original_residue_name);
  }
  return buf.c_str();
}

int ref_structure_model_index(void* h) { return static_cast<hikoboshi::io::LoadedStructure*>(h)->selected_model_index(); }

int ref_detect_structure_format(const char* path, const char* content, std::size_t nbytes) {
  return static_cast<int>(hikoboshi::io::detect_structure_format(path ? path : "", std::string_view(content ? content : "", content ? nbytes : 0)));
}

void ref_residue_template(float* out) {
  const auto& t = hikoboshi::io::canonical_residue_template();
  std::memcpy(out, t.coords.data(), t.coords.size() * sizeof(float));
}

void ref_virtual_cb(const float* n, const float* ca, const float* c, float* out) {
  hikoboshi::io::glycine_virtual_cb(n, ca, c, out);
}

}  // extern "C"
