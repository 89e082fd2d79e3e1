// Structure input of the design path (include/hkbs_structure.h): PDB and
// mmCIF text -> one model, one polymer chain -> canonical N, CA, C, O, CB
// backbone with AtomSource codes, residue codes and numbering metadata.
//
// Stages and the reference code each one follows:
//   parse_pdb      fixed-column ATOM/HETATM/MODEL/ENDMDL   cpp/io/pdb_parser.cpp:88-196
//   parse_mmcif    _atom_site loops, quoted tokens,         cpp/io/mmcif_parser.cpp:118-398
//                  rows wrapped over several lines
//   select_chain   model by index or id (default 1), chain  cpp/io/structure_normalize.cpp:86-180
//                  by id, index, "A" or first polymer chain
//   collect        residues in file order, altloc per atom  cpp/io/structure_normalize.cpp:182-272
//                  (blank > A > first seen), chain breaks
//   infer          glycine virtual CB; rigid fit of the      cpp/io/atom_inference.cpp:38-111,
//                  residue template for other missing atoms  cpp/io/atom_inference_kabsch.cpp
//                  (>= 3 non-collinear anchors, RMSD <= 0.5)
// Number parsing uses std::from_chars as the reference does, and the
// inference arithmetic keeps the reference's operation order (this file is
// compiled without floating-point contraction), so coordinates match the
// reference loader bit for bit.
#include "../../include/hkbs_structure.h"
#include "host_status.hpp"

#include <algorithm>
#include <cctype>
#include <charconv>
#include <cmath>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <optional>
#include <sstream>
#include <string>
#include <string_view>
#include <tuple>
#include <utility>
#include <vector>

struct hkbs_structure {
  std::vector<float> coords;        // [L,5,3]
  std::vector<uint8_t> sources;     // [L,5]
  std::string codes;                // L one-letter codes
  std::vector<std::string> names;   // original residue names
  std::vector<int32_t> numbers;
  std::vector<char> icodes;
  std::vector<int64_t> first_records;
  std::vector<uint64_t> breaks;
  std::vector<int32_t> labels;      // chain of each residue (index into chains)
  std::vector<std::string> chains;  // selected chains in output order
  std::string input_id, model_id, chain_id, altloc_note;
  int32_t model_index = 0;
};

namespace {

using hkbs::report_error;
using std::string_view;

enum : uint8_t { kMissing = 0, kObserved = 1, kInferred = 2, kVirtual = 3 };
constexpr int kAtoms = 5;  // N, CA, C, O, CB

// ----------------------------------------------------------------- text ----
bool pdb_blank(char c) { return c == ' ' || c == '\t'; }

// PDB fields: spaces and tabs on both ends, plus a carriage return at the end.
string_view strip_pdb(string_view s) {
  size_t b = 0, e = s.size();
  while (b < e && pdb_blank(s[b])) ++b;
  while (e > b && (pdb_blank(s[e - 1]) || s[e - 1] == '\r')) --e;
  return s.substr(b, e - b);
}

// mmCIF text: any C-locale whitespace on both ends.
string_view strip_cif(string_view s) {
  size_t b = 0, e = s.size();
  while (b < e && std::isspace(static_cast<unsigned char>(s[b]))) ++b;
  while (e > b && std::isspace(static_cast<unsigned char>(s[e - 1]))) --e;
  return s.substr(b, e - b);
}

bool has_prefix(string_view s, string_view p) { return s.size() >= p.size() && s.substr(0, p.size()) == p; }

// Field of a fixed-column record; empty past the end of the line.
string_view column(string_view line, size_t at, size_t width) {
  return at >= line.size() ? string_view{} : line.substr(at, std::min(width, line.size() - at));
}

// Every '\n'-separated segment, including the (possibly empty) one after the
// last newline.
std::vector<string_view> split_lines(string_view text) {
  std::vector<string_view> lines;
  size_t at = 0;
  for (;;) {
    const size_t nl = text.find('\n', at);
    if (nl == string_view::npos) {
      lines.push_back(text.substr(at));
      return lines;
    }
    lines.push_back(text.substr(at, nl - at));
    at = nl + 1;
  }
}

// Integer field: an optional leading '+', then the whole field must be a
// base-10 integer that fits 64 bits; the value is narrowed to 32 bits.
bool to_int(string_view s, int32_t& out) {
  if (!s.empty() && s.front() == '+') s.remove_prefix(1);
  if (s.empty()) return false;
  int64_t v = 0;
  const auto r = std::from_chars(s.data(), s.data() + s.size(), v);
  if (r.ec != std::errc{} || r.ptr != s.data() + s.size()) return false;
  out = static_cast<int32_t>(v);
  return true;
}

// Real field: optional '+', whole field parsed as a double, finite, rounded
// to float.
bool to_float(string_view s, float& out) {
  if (!s.empty() && s.front() == '+') s.remove_prefix(1);
  if (s.empty()) return false;
  double v = 0.0;
  const auto r = std::from_chars(s.data(), s.data() + s.size(), v);
  if (r.ec != std::errc{} || r.ptr != s.data() + s.size() || !std::isfinite(v)) return false;
  out = static_cast<float>(v);
  return true;
}

// ------------------------------------------------------------- records ----
struct AtomRecord {
  int64_t record = 0;  // position among the file's atom records
  std::string atom, residue, chain, model_id;
  int32_t residue_number = 0;
  int32_t model = 1;
  char altloc = ' ';
  char icode = ' ';
  bool het = false;
  float xyz[3] = {0.0F, 0.0F, 0.0F};
};

struct Status {
  hkbs_status code = HKBS_OK;
  const char* detail = "";
  bool ok() const { return code == HKBS_OK; }
};
Status invalid(const char* detail) { return {HKBS_INVALID_ARGUMENT, detail}; }

// cpp/io/pdb_parser.cpp:88-196. Records outside MODEL/ENDMDL belong to model 1.
Status parse_pdb(string_view text, std::vector<AtomRecord>& out) {
  int32_t model = 1;
  bool in_model = false;
  for (const string_view line : split_lines(text)) {
    if (has_prefix(line, "MODEL ")) {
      if (!to_int(strip_pdb(column(line, 10, 4)), model))
        return invalid("PDB MODEL record missing or unparseable serial");
      in_model = true;
      continue;
    }
    if (has_prefix(line, "ENDMDL")) {
      in_model = false;
      continue;
    }
    const bool het = has_prefix(line, "HETATM");
    if (!het && !has_prefix(line, "ATOM  ")) continue;
    if (line.size() < 54) return invalid("PDB ATOM/HETATM record shorter than the 54-column coordinate block");
    AtomRecord r;
    r.record = static_cast<int64_t>(out.size());
    r.het = het;
    r.model = in_model ? model : 1;
    r.model_id = std::to_string(r.model);
    int32_t serial = 0;
    if (!to_int(strip_pdb(column(line, 6, 5)), serial))
      return invalid("PDB ATOM/HETATM record has invalid serial column");
    r.atom = std::string(strip_pdb(column(line, 12, 4)));
    r.altloc = line[16];
    r.residue = std::string(strip_pdb(column(line, 17, 3)));
    r.chain = std::string(strip_pdb(column(line, 21, 1)));
    if (!to_int(strip_pdb(column(line, 22, 4)), r.residue_number))
      return invalid("PDB ATOM/HETATM record has invalid residue number");
    r.icode = line[26];
    for (int a = 0; a < 3; ++a)
      if (!to_float(strip_pdb(column(line, 30 + 8 * a, 8)), r.xyz[a]))
        return invalid("PDB ATOM/HETATM record has invalid coordinate field; refusing to silently zero-fill");
    out.push_back(std::move(r));
  }
  return {};
}

// Whitespace-separated tokens; a token opened by ' or " runs to the next
// occurrence of the same quote character (cpp/io/mmcif_parser.cpp:77-112).
void cif_tokens(string_view line, std::vector<std::string>& out) {
  size_t i = 0;
  const size_t n = line.size();
  const auto space = [&](size_t k) { return std::isspace(static_cast<unsigned char>(line[k])) != 0; };
  while (true) {
    while (i < n && space(i)) ++i;
    if (i >= n) return;
    const char q = line[i];
    if (q == '\'' || q == '"') {
      const size_t from = ++i;
      while (i < n && line[i] != q) ++i;
      out.emplace_back(line.substr(from, i - from));
      if (i < n) ++i;
    } else {
      const size_t from = i;
      while (i < n && !space(i)) ++i;
      out.emplace_back(line.substr(from, i - from));
    }
  }
}

// _atom_site columns the loader reads; a preferred column and its fallback.
struct CifColumns {
  static constexpr size_t kNone = static_cast<size_t>(-1);
  size_t group = kNone, serial = kNone, atom = kNone, alt = kNone, residue = kNone, chain = kNone,
         number = kNone, icode = kNone, model = kNone, xyz[3] = {kNone, kNone, kNone};

  static size_t pick(const std::map<std::string, size_t, std::less<>>& idx, const char* a, const char* b) {
    auto it = idx.find(a);
    if (it != idx.end()) return it->second;
    if (b == nullptr) return kNone;
    it = idx.find(b);
    return it == idx.end() ? kNone : it->second;
  }
  explicit CifColumns(const std::vector<std::string>& names) {
    std::map<std::string, size_t, std::less<>> idx;
    for (size_t i = 0; i < names.size(); ++i) idx[names[i]] = i;  // a repeated name keeps its last column
    group = pick(idx, "group_PDB", nullptr);
    serial = pick(idx, "id", nullptr);
    atom = pick(idx, "label_atom_id", "auth_atom_id");
    alt = pick(idx, "label_alt_id", nullptr);
    residue = pick(idx, "auth_comp_id", "label_comp_id");
    chain = pick(idx, "auth_asym_id", "label_asym_id");
    number = pick(idx, "auth_seq_id", "label_seq_id");
    icode = pick(idx, "pdbx_PDB_ins_code", nullptr);
    model = pick(idx, "pdbx_PDB_model_num", nullptr);
    xyz[0] = pick(idx, "Cartn_x", nullptr);
    xyz[1] = pick(idx, "Cartn_y", nullptr);
    xyz[2] = pick(idx, "Cartn_z", nullptr);
  }
};

bool cif_unknown(const std::string& t) { return t == "." || t == "?"; }

Status cif_record(const std::vector<std::string>& tok, const CifColumns& c, int64_t index, AtomRecord& r) {
  constexpr size_t kNone = CifColumns::kNone;
  r.record = index;
  r.het = tok[c.group == kNone ? 0 : c.group] == "HETATM";
  r.atom = tok[c.atom];
  // An empty quoted altloc or insertion token reads as its terminating NUL.
  if (c.alt != kNone) r.altloc = cif_unknown(tok[c.alt]) ? ' ' : tok[c.alt].c_str()[0];
  if (c.residue != kNone) r.residue = tok[c.residue];
  if (c.chain != kNone) r.chain = cif_unknown(tok[c.chain]) ? std::string() : tok[c.chain];
  if (c.number != kNone && !to_int(strip_cif(tok[c.number]), r.residue_number))
    return invalid("mmCIF _atom_site row has unparseable residue number");
  if (c.icode != kNone) r.icode = (cif_unknown(tok[c.icode]) || tok[c.icode].empty()) ? ' ' : tok[c.icode][0];
  for (int a = 0; a < 3; ++a) {
    const string_view s = strip_cif(tok[c.xyz[a]]);
    if (s == "?" || s == "." || !to_float(s, r.xyz[a]))
      return invalid("mmCIF _atom_site row has unparseable coordinate; refusing to silently zero-fill");
  }
  int32_t model = 1;
  if (c.model != kNone && to_int(strip_cif(tok[c.model]), model)) {
    r.model = model;
    r.model_id = tok[c.model];
  } else {
    r.model = 1;
    r.model_id = "1";
  }
  return {};
}

// cpp/io/mmcif_parser.cpp:118-398, over a line array. Where the reference's
// header scan would spin forever (a loop_ followed only by blank or
// _atom_site. lines up to the end of the text) this loader treats the loop
// as having no rows.
Status parse_mmcif(string_view text, std::vector<AtomRecord>& out) {
  const std::vector<string_view> lines = split_lines(text);
  const size_t n = lines.size();
  bool found = false;
  size_t i = 0;
  while (i < n) {
    if (!has_prefix(strip_cif(lines[i]), "loop_")) {
      ++i;
      continue;
    }
    // Column headers of this loop; any other category abandons it.
    std::vector<std::string> names;
    bool atom_site = false;
    size_t j = i + 1;
    for (; j < n; ++j) {
      const string_view h = strip_cif(lines[j]);
      if (has_prefix(h, "_atom_site.")) {
        atom_site = true;
        names.emplace_back(h.substr(11));
      } else if (has_prefix(h, "_")) {
        names.clear();
        break;
      } else if (!h.empty()) {
        break;  // first data row
      }
    }
    if (!atom_site || names.empty()) {
      ++i;
      continue;
    }
    found = true;
    const CifColumns cols(names);
    if (cols.atom == CifColumns::kNone)
      return invalid("mmCIF _atom_site loop missing required atom-name column");
    if (cols.xyz[0] == CifColumns::kNone || cols.xyz[1] == CifColumns::kNone || cols.xyz[2] == CifColumns::kNone)
      return invalid("mmCIF _atom_site loop missing required Cartesian coordinate columns");
    std::vector<std::string> tok;
    while (j < n) {
      const string_view row = strip_cif(lines[j]);
      if (row.empty()) {
        ++j;
        continue;
      }
      if (has_prefix(row, "loop_") || has_prefix(row, "data_") || has_prefix(row, "_") || has_prefix(row, "#"))
        break;  // the outer scan resumes on this line
      tok.clear();
      cif_tokens(row, tok);
      while (tok.size() < names.size() && j + 1 < n) cif_tokens(strip_cif(lines[++j]), tok);  // wrapped row
      if (tok.size() < names.size()) return invalid("mmCIF _atom_site row column count mismatch");
      AtomRecord r;
      const Status st = cif_record(tok, cols, static_cast<int64_t>(out.size()), r);
      if (!st.ok()) return st;
      out.push_back(std::move(r));
      ++j;
    }
    i = j;
  }
  if (!found) return invalid("mmCIF input does not contain an _atom_site loop");
  return {};
}

// ------------------------------------------------------- residue table ----
// One-letter codes of the 20 standard residues and of the modified residues
// accepted from HETATM records (cpp/io/residue_table.cpp:29-53).
struct ResidueName {
  const char* name;
  char code;
  bool modified;
};
constexpr ResidueName kResidueNames[] = {
    {"ALA", 'A', false}, {"ARG", 'R', false}, {"ASN", 'N', false}, {"ASP", 'D', false}, {"CYS", 'C', false},
    {"GLN", 'Q', false}, {"GLU", 'E', false}, {"GLY", 'G', false}, {"HIS", 'H', false}, {"ILE", 'I', false},
    {"LEU", 'L', false}, {"LYS", 'K', false}, {"MET", 'M', false}, {"PHE", 'F', false}, {"PRO", 'P', false},
    {"SER", 'S', false}, {"THR", 'T', false}, {"TRP", 'W', false}, {"TYR", 'Y', false}, {"VAL", 'V', false},
    {"MSE", 'M', true},  {"SEC", 'C', true},  {"PYL", 'K', true},  {"SEP", 'S', true},  {"TPO", 'T', true},
    {"PTR", 'Y', true},  {"HYP", 'P', true},
};

// Name lookup ignoring case and surrounding spaces/tabs; nullptr if unknown.
const ResidueName* find_residue(string_view name) {
  size_t b = 0, e = name.size();
  while (b < e && pdb_blank(name[b])) ++b;
  while (e > b && pdb_blank(name[e - 1])) --e;
  name = name.substr(b, e - b);
  if (name.size() != 3) return nullptr;
  const auto up = [](char c) { return (c >= 'a' && c <= 'z') ? static_cast<char>(c - 'a' + 'A') : c; };
  for (const ResidueName& r : kResidueNames)
    if (up(name[0]) == r.name[0] && up(name[1]) == r.name[1] && up(name[2]) == r.name[2]) return &r;
  return nullptr;
}

char residue_code(string_view name) {
  const ResidueName* r = find_residue(name);
  return r ? r->code : 'X';
}

int canonical_slot(const std::string& atom) {
  static const char* const kNames[kAtoms] = {"N", "CA", "C", "O", "CB"};
  for (int a = 0; a < kAtoms; ++a)
    if (atom == kNames[a]) return a;
  return -1;
}

// A backbone atom of a polymer residue: ATOM records with a canonical atom
// name, and HETATM records only for whitelisted modified residues.
bool polymer_atom(const AtomRecord& r, bool include_modified) {
  if (canonical_slot(r.atom) < 0) return false;
  if (!r.het) return true;
  const ResidueName* id = find_residue(r.residue);
  return include_modified && id != nullptr && id->modified;
}

// ---------------------------------------------------------- selection ----
struct Options {
  std::optional<int32_t> model_index;
  std::string model_id, chain_id;
  std::optional<uint64_t> chain_index;
  std::optional<std::vector<std::string>> chain_list;  // several chains, in this order
  bool all_chains = false;
  bool infer = true, include_modified = true;
};

Status read_options(const hkbs_structure_options* o, Options& r) {
  if (o == nullptr) return {};
  if (o->has_model_index) r.model_index = o->model_index;
  if (o->model_id) r.model_id = o->model_id;
  if (o->chain_id) r.chain_id = o->chain_id;
  if (o->has_chain_index) r.chain_index = o->chain_index;
  r.infer = o->infer_missing_atoms != 0;
  r.include_modified = o->include_modified_residues != 0;
  r.all_chains = o->all_chains != 0;
  if (o->n_chain_ids > 0) {
    if (o->chain_ids == nullptr) return invalid("chain_ids must be non-null when n_chain_ids > 0");
    std::vector<std::string> ids;
    for (size_t i = 0; i < o->n_chain_ids; ++i) {
      if (o->chain_ids[i] == nullptr) return invalid("chain_ids entries must be non-null");
      if (std::find(ids.begin(), ids.end(), o->chain_ids[i]) != ids.end()) return invalid("chain ids must be distinct");
      ids.emplace_back(o->chain_ids[i]);
    }
    r.chain_list = std::move(ids);
  }
  // chain_id over chain_index is the reference's own precedence; the chain
  // lists exclude both.
  const int selections =
      (!r.chain_id.empty() || r.chain_index.has_value()) + r.chain_list.has_value() + r.all_chains;
  if (selections > 1) return invalid("choose one chain selection: chain_id, chain_index, chain_ids or all_chains");
  return {};
}

struct Residue {
  char code = 'X';
  std::string name;
  int32_t number = 0;
  char icode = ' ';
  int64_t first_record = -1;
  float xyz[kAtoms][3] = {};
  uint8_t src[kAtoms] = {};
  bool blank_seen[kAtoms] = {};
  char chosen[kAtoms] = {' ', ' ', ' ', ' ', ' '};
};

bool blank_altloc(char c) { return c == ' ' || c == '\0'; }

// Altloc policy per atom: the first blank altloc is final; otherwise blank
// beats 'A'/'a', which beats any other letter; ties keep the earlier record.
bool altloc_wins(char proposed, char current, bool current_is_final) {
  if (current_is_final) return false;
  if (blank_altloc(proposed)) return true;
  const auto rank = [](char c) { return blank_altloc(c) ? 0 : (c == 'A' || c == 'a') ? 1 : 2; };
  return rank(proposed) < rank(current);
}

// cpp/io/structure_normalize.cpp:86-352.
Status normalize(const std::vector<AtomRecord>& recs, const Options& opt, hkbs_structure& s,
                 std::vector<Residue>& residues) {
  int32_t model = 1;
  if (opt.model_index) {
    model = *opt.model_index;
  } else if (!opt.model_id.empty()) {
    const auto it = std::find_if(recs.begin(), recs.end(), [&](const AtomRecord& r) { return r.model_id == opt.model_id; });
    if (it == recs.end()) return invalid("requested model id not present in input");
    model = it->model;
  }
  const auto first = std::find_if(recs.begin(), recs.end(), [&](const AtomRecord& r) { return r.model == model; });
  if (first == recs.end()) return invalid("selected model index not present in input");
  s.model_index = model;
  s.model_id = first->model_id;

  // Polymer chains of the model in order of appearance.
  std::vector<std::string> chains;
  for (const AtomRecord& r : recs)
    if (r.model == model && polymer_atom(r, opt.include_modified) &&
        std::find(chains.begin(), chains.end(), r.chain) == chains.end())
      chains.push_back(r.chain);
  const auto present = [&](const std::string& c) { return std::find(chains.begin(), chains.end(), c) != chains.end(); };
  if (opt.chain_list) {
    for (const std::string& c : *opt.chain_list)
      if (!present(c)) return invalid("requested chain id not present in selected model");
    s.chains = *opt.chain_list;
  } else if (opt.all_chains) {
    if (chains.empty()) return invalid("selected model has no polymer chains");
    s.chains = chains;
  } else if (!opt.chain_id.empty()) {
    if (!present(opt.chain_id)) return invalid("requested chain id not present in selected model");
    s.chains = {opt.chain_id};
  } else if (opt.chain_index) {
    if (*opt.chain_index >= chains.size()) return invalid("requested chain index out of range");
    s.chains = {chains[*opt.chain_index]};
  } else if (present("A")) {
    s.chains = {"A"};
  } else if (!chains.empty()) {
    s.chains = {chains.front()};
  } else {
    return invalid("selected model has no polymer chains");
  }
  // The chain text field: the chain id, or the selected ids joined by commas.
  for (size_t c = 0; c < s.chains.size(); ++c) s.chain_id += (c ? "," : "") + s.chains[c];

  // Residues keyed by (chain, number, insertion code) in order of first
  // appearance; records arrive in file order, so creation order is file
  // order. Several chains are then grouped in the selected chain order.
  std::map<std::tuple<size_t, int32_t, char>, size_t> slot_of;
  std::vector<size_t> chain_of;
  bool altloc_used = false;
  for (const AtomRecord& r : recs) {
    if (r.model != model || !polymer_atom(r, opt.include_modified)) continue;
    const auto ch = std::find(s.chains.begin(), s.chains.end(), r.chain);
    if (ch == s.chains.end()) continue;
    const auto key = std::make_tuple(static_cast<size_t>(ch - s.chains.begin()), r.residue_number, r.icode);
    auto it = slot_of.find(key);
    if (it == slot_of.end()) {
      chain_of.push_back(std::get<0>(key));
      Residue res;
      res.code = residue_code(r.residue);
      res.name = r.residue;
      res.number = r.residue_number;
      res.icode = r.icode;
      res.first_record = r.record;
      residues.push_back(std::move(res));
      it = slot_of.emplace(key, residues.size() - 1).first;
    }
    Residue& res = residues[it->second];
    const int a = canonical_slot(r.atom);
    if (res.src[a] == kObserved) {
      if (!altloc_wins(r.altloc, res.chosen[a], res.blank_seen[a])) continue;
      altloc_used = true;
    }
    std::memcpy(res.xyz[a], r.xyz, sizeof(r.xyz));
    res.src[a] = kObserved;
    if (blank_altloc(r.altloc)) res.blank_seen[a] = true;
    res.chosen[a] = r.altloc;
  }
  if (residues.empty()) return invalid("selected chain has no accepted amino-acid residues");
  if (s.chains.size() > 1) {
    std::vector<size_t> perm(residues.size());
    for (size_t i = 0; i < perm.size(); ++i) perm[i] = i;
    std::stable_sort(perm.begin(), perm.end(), [&](size_t a, size_t b) { return chain_of[a] < chain_of[b]; });
    std::vector<Residue> grouped;
    std::vector<size_t> grouped_chain;
    for (size_t i : perm) {
      grouped.push_back(std::move(residues[i]));
      grouped_chain.push_back(chain_of[i]);
    }
    residues.swap(grouped);
    chain_of.swap(grouped_chain);
  }
  for (size_t c : chain_of) s.labels.push_back(static_cast<int32_t>(c));

  // A chain break follows residue i-1 when the numbering skips ahead, or when
  // an inserted residue (non-blank code) is followed by the plain number;
  // residues of different chains are never compared.
  for (size_t i = 1; i < residues.size(); ++i) {
    if (chain_of[i] != chain_of[i - 1]) continue;
    const Residue& p = residues[i - 1];
    const Residue& c = residues[i];
    const bool skip = static_cast<int64_t>(c.number) > static_cast<int64_t>(p.number) + 1;
    const bool back_to_plain = c.number == p.number && c.icode != p.icode && p.icode != ' ' && c.icode == ' ';
    if (skip || back_to_plain) s.breaks.push_back(i - 1);
  }
  if (altloc_used) s.altloc_note = "altloc selection applied";

  const size_t L = residues.size();
  s.coords.assign(L * kAtoms * 3, 0.0F);
  s.sources.assign(L * kAtoms, kMissing);
  s.codes.resize(L);
  for (size_t i = 0; i < L; ++i) {
    const Residue& r = residues[i];
    for (int a = 0; a < kAtoms; ++a) {
      s.sources[i * kAtoms + a] = r.src[a];
      if (r.src[a] == kObserved) std::memcpy(&s.coords[(i * kAtoms + a) * 3], r.xyz[a], 3 * sizeof(float));
    }
    s.codes[i] = r.code;
    s.names.push_back(r.name);
    s.numbers.push_back(r.number);
    s.icodes.push_back(r.icode);
    s.first_records.push_back(r.first_record);
  }
  return {};
}

// ---------------------------------------------------------- inference ----
// ProteinMPNN's virtual CB: CA + a*(b x c) + b'*b + c'*c with b = CA - N,
// c = C - CA (cpp/io/virtual_cb.cpp:19-38), evaluated left to right in fp32.
void virtual_cb(const float* n, const float* ca, const float* c, float* out) {
  constexpr float kA = -0.58273431F, kB = 0.56802827F, kC = -0.54067466F;
  const float b[3] = {ca[0] - n[0], ca[1] - n[1], ca[2] - n[2]};
  const float v[3] = {c[0] - ca[0], c[1] - ca[1], c[2] - ca[2]};
  const float x[3] = {b[1] * v[2] - b[2] * v[1], b[2] * v[0] - b[0] * v[2], b[0] * v[1] - b[1] * v[0]};
  for (int k = 0; k < 3; ++k) out[k] = ca[k] + kA * x[k] + kB * b[k] + kC * v[k];
}

// Ideal N, CA, C, O, CB of one residue in a local frame: CA at the origin, N
// on -x, C in the xy plane from the Engh-Huber N-CA-C angle, O from the
// CA-C-O angle, CB from the virtual-CB rule (cpp/io/residue_table.cpp:82-155).
struct ResidueTemplate {
  float xyz[kAtoms][3];
  ResidueTemplate() {
    constexpr float kNCA = 1.458F, kCAC = 1.525F, kCO = 1.231F;
    constexpr float kAngleNCAC = 1.9416F, kAngleCACO = 2.1031F;
    const float ca[3] = {0.0F, 0.0F, 0.0F};
    const float n[3] = {-kNCA, 0.0F, 0.0F};
    const float c[3] = {kCAC * std::cos(kAngleNCAC - 1.5707963267948966F),
                        kCAC * std::sin(kAngleNCAC - 1.5707963267948966F), 0.0F};
    const float d[3] = {c[0] - ca[0], c[1] - ca[1], c[2] - ca[2]};
    const float len = std::sqrt(d[0] * d[0] + d[1] * d[1] + d[2] * d[2]);
    const float u[3] = {d[0] / len, d[1] / len, d[2] / len};
    const float w[3] = {-u[1], u[0], 0.0F};
    const float co = std::cos(3.14159265358979F - kAngleCACO);
    const float si = std::sin(3.14159265358979F - kAngleCACO);
    float o[3];
    for (int k = 0; k < 3; ++k) o[k] = c[k] + kCO * (co * u[k] + si * w[k]);
    float cb[3];
    virtual_cb(n, ca, c, cb);
    const float* atoms[kAtoms] = {n, ca, c, o, cb};
    for (int a = 0; a < kAtoms; ++a) std::memcpy(xyz[a], atoms[a], sizeof(xyz[a]));
  }
};

const ResidueTemplate& residue_template() {
  static const ResidueTemplate t;
  return t;
}

using Mat3 = double[3][3];

void mat_mul(const Mat3 a, const Mat3 b, Mat3 out) {
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j) {
      double s = 0.0;
      for (int k = 0; k < 3; ++k) s += a[i][k] * b[k][j];
      out[i][j] = s;
    }
}

void transpose(const Mat3 m, Mat3 out) {
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j) out[i][j] = m[j][i];
}

double determinant(const Mat3 m) {
  return m[0][0] * (m[1][1] * m[2][2] - m[1][2] * m[2][1]) - m[0][1] * (m[1][0] * m[2][2] - m[1][2] * m[2][0]) +
         m[0][2] * (m[1][0] * m[2][1] - m[1][1] * m[2][0]);
}

// Cyclic Jacobi eigen-decomposition of a symmetric 3x3 matrix (in place):
// eigenvalues on the diagonal, eigenvectors in the columns of vec.
void symmetric_eigen(Mat3 a, Mat3 vec) {
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j) vec[i][j] = i == j ? 1.0 : 0.0;
  constexpr int kPairs[3][2] = {{0, 1}, {0, 2}, {1, 2}};
  for (int sweep = 0; sweep < 64; ++sweep) {
    double off = 0.0;
    for (const auto& pq : kPairs) off += std::fabs(a[pq[0]][pq[1]]);
    if (off < 1e-12) return;
    for (const auto& pq : kPairs) {
      const int p = pq[0], q = pq[1], r = 3 - p - q;
      const double app = a[p][p], aqq = a[q][q], apq = a[p][q];
      if (std::fabs(apq) < 1e-15) continue;
      // Rotation angle: t = tan(phi) is the smaller root of t^2 + 2 t theta - 1.
      const double theta = (aqq - app) / (2.0 * apq);
      const double root = std::sqrt(1.0 + theta * theta);
      const double t = theta >= 0.0 ? 1.0 / (theta + root) : 1.0 / (theta - root);
      const double cs = 1.0 / std::sqrt(1.0 + t * t);
      const double sn = t * cs;
      a[p][p] = app - t * apq;
      a[q][q] = aqq + t * apq;
      a[p][q] = a[q][p] = 0.0;
      const double arp = a[r][p], arq = a[r][q];
      a[r][p] = a[p][r] = cs * arp - sn * arq;
      a[r][q] = a[q][r] = sn * arp + cs * arq;
      for (int k = 0; k < 3; ++k) {
        const double vp = vec[k][p], vq = vec[k][q];
        vec[k][p] = cs * vp - sn * vq;
        vec[k][q] = sn * vp + cs * vq;
      }
    }
  }
}

// Least-squares rigid motion (rot, shift) taking points p onto points q
// (Kabsch): H = sum (p - p0)(q - q0)^T, right singular vectors of H from the
// eigenvectors of H^T H, left ones as H v / sigma (the third as a cross
// product), and a reflection guard on det(V U^T). False when fewer than three
// points or when they are collinear (second singular value ~ 0).
bool rigid_fit(const double (*p)[3], const double (*q)[3], int n, Mat3 rot, double shift[3], double& rmsd) {
  if (n < 3) return false;
  double cp[3] = {0.0, 0.0, 0.0}, cq[3] = {0.0, 0.0, 0.0};
  for (int i = 0; i < n; ++i)
    for (int k = 0; k < 3; ++k) {
      cp[k] += p[i][k];
      cq[k] += q[i][k];
    }
  for (int k = 0; k < 3; ++k) {
    cp[k] /= n;
    cq[k] /= n;
  }
  Mat3 h = {};
  for (int i = 0; i < n; ++i) {
    const double dp[3] = {p[i][0] - cp[0], p[i][1] - cp[1], p[i][2] - cp[2]};
    const double dq[3] = {q[i][0] - cq[0], q[i][1] - cq[1], q[i][2] - cq[2]};
    for (int a = 0; a < 3; ++a)
      for (int b = 0; b < 3; ++b) h[a][b] += dp[a] * dq[b];
  }
  Mat3 ht, hth, evec;
  transpose(h, ht);
  mat_mul(ht, h, hth);
  symmetric_eigen(hth, evec);
  const double eval[3] = {hth[0][0], hth[1][1], hth[2][2]};
  // Descending order by pairwise exchange over (0,1), (0,2), (1,2).
  int ord[3] = {0, 1, 2};
  constexpr int kPairs[3][2] = {{0, 1}, {0, 2}, {1, 2}};
  for (const auto& ij : kPairs)
    if (eval[ord[ij[1]]] > eval[ord[ij[0]]]) std::swap(ord[ij[0]], ord[ij[1]]);
  Mat3 v;
  double lam[3];
  for (int c = 0; c < 3; ++c) {
    lam[c] = eval[ord[c]];
    for (int r = 0; r < 3; ++r) v[r][c] = evec[r][ord[c]];
  }
  if (lam[0] <= 1e-12 || lam[1] <= 1e-12) return false;
  Mat3 u = {};
  for (int c = 0; c < 2; ++c) {
    const double sigma = std::sqrt(std::max(0.0, lam[c]));
    for (int r = 0; r < 3; ++r) {
      double s = 0.0;
      for (int k = 0; k < 3; ++k) s += h[r][k] * v[k][c];
      u[r][c] = sigma > 1e-12 ? s / sigma : 0.0;
    }
  }
  u[0][2] = u[1][0] * u[2][1] - u[2][0] * u[1][1];
  u[1][2] = u[2][0] * u[0][1] - u[0][0] * u[2][1];
  u[2][2] = u[0][0] * u[1][1] - u[1][0] * u[0][1];
  Mat3 ut, vut;
  transpose(u, ut);
  mat_mul(v, ut, vut);
  const double sign = determinant(vut) >= 0.0 ? 1.0 : -1.0;
  for (int r = 0; r < 3; ++r) v[r][2] = sign * v[r][2];
  mat_mul(v, ut, rot);
  for (int k = 0; k < 3; ++k) shift[k] = cq[k] - (rot[k][0] * cp[0] + rot[k][1] * cp[1] + rot[k][2] * cp[2]);
  double err = 0.0;
  for (int i = 0; i < n; ++i) {
    double m[3];
    for (int k = 0; k < 3; ++k) m[k] = rot[k][0] * p[i][0] + rot[k][1] * p[i][1] + rot[k][2] * p[i][2] + shift[k];
    for (int k = 0; k < 3; ++k) err += (m[k] - q[i][k]) * (m[k] - q[i][k]);
  }
  rmsd = std::sqrt(err / static_cast<double>(n));
  return true;
}

// Fills the Missing atoms of one residue from the template fitted onto its
// observed atoms, if at least three are observed, they are not collinear and
// the fit's RMSD is at most 0.5 A; filled atoms become Inferred.
void infer_from_template(float* xyz, uint8_t* src) {
  constexpr float kRmsdGuard = 0.5F;
  const ResidueTemplate& t = residue_template();
  double from[kAtoms][3], to[kAtoms][3];
  int anchors = 0, missing[kAtoms], n_missing = 0;
  for (int a = 0; a < kAtoms; ++a) {
    if (src[a] == kObserved) {
      for (int k = 0; k < 3; ++k) {
        from[anchors][k] = t.xyz[a][k];
        to[anchors][k] = xyz[a * 3 + k];
      }
      ++anchors;
    } else if (src[a] == kMissing) {
      missing[n_missing++] = a;
    }
  }
  if (n_missing == 0 || anchors < 3) return;
  Mat3 rot;
  double shift[3], rmsd = 0.0;
  if (!rigid_fit(from, to, anchors, rot, shift, rmsd) || rmsd > static_cast<double>(kRmsdGuard)) return;
  for (int m = 0; m < n_missing; ++m) {
    const int a = missing[m];
    const double tp[3] = {t.xyz[a][0], t.xyz[a][1], t.xyz[a][2]};
    for (int k = 0; k < 3; ++k)
      xyz[a * 3 + k] = static_cast<float>(rot[k][0] * tp[0] + rot[k][1] * tp[1] + rot[k][2] * tp[2] + shift[k]);
    src[a] = kInferred;
  }
}

// cpp/io/atom_inference.cpp:38-111. Glycine only ever gains a virtual CB,
// computed from whatever N, CA, C hold and marked Virtual only when all three
// were observed (else it stays Missing, with the computed coordinates).
void infer_missing(hkbs_structure& s) {
  for (size_t i = 0; i < s.codes.size(); ++i) {
    float* xyz = &s.coords[i * kAtoms * 3];
    uint8_t* src = &s.sources[i * kAtoms];
    if (s.codes[i] == 'G') {
      if (src[4] == kMissing) {
        virtual_cb(xyz + 0, xyz + 3, xyz + 6, xyz + 12);
        src[4] = (src[0] == kObserved && src[1] == kObserved && src[2] == kObserved) ? kVirtual : kMissing;
      }
      continue;
    }
    infer_from_template(xyz, src);
  }
}

// ------------------------------------------------------------ loading ----
bool ends_with_nocase(string_view s, string_view suffix) {
  if (s.size() < suffix.size()) return false;
  const auto low = [](char c) { return (c >= 'A' && c <= 'Z') ? static_cast<char>(c - 'A' + 'a') : c; };
  for (size_t i = 0; i < suffix.size(); ++i)
    if (low(s[s.size() - suffix.size() + i]) != low(suffix[i])) return false;
  return true;
}

int32_t detect_format(string_view path, string_view text) {
  if (ends_with_nocase(path, ".cif") || ends_with_nocase(path, ".mmcif")) return HKBS_FORMAT_MMCIF;
  if (ends_with_nocase(path, ".pdb") || ends_with_nocase(path, ".ent")) return HKBS_FORMAT_PDB;
  if (has_prefix(text, "data_") || text.find("_atom_site.") != string_view::npos) return HKBS_FORMAT_MMCIF;
  for (const string_view line : split_lines(text)) {
    const string_view tag = line.substr(0, std::min<size_t>(6, line.size()));
    if (tag == "ATOM  " || tag == "HETATM" || tag == "MODEL ") return HKBS_FORMAT_PDB;
  }
  return HKBS_FORMAT_UNKNOWN;
}

hkbs_status load(string_view text, int32_t format, string_view label, const hkbs_structure_options* options,
                 hkbs_structure** out) {
  if (out == nullptr) return report_error(HKBS_INVALID_ARGUMENT, "structure output handle must be non-null");
  *out = nullptr;
  if (format == HKBS_FORMAT_UNKNOWN) format = detect_format(label, text);
  if (format != HKBS_FORMAT_PDB && format != HKBS_FORMAT_MMCIF)
    return report_error(HKBS_INVALID_ARGUMENT,
                        "unrecognized structure file format; extension and content cues did not match PDB or mmCIF");
  std::vector<AtomRecord> recs;
  const Status parsed = format == HKBS_FORMAT_PDB ? parse_pdb(text, recs) : parse_mmcif(text, recs);
  if (!parsed.ok()) return report_error(parsed.code, parsed.detail);
  if (recs.empty())
    return report_error(HKBS_INVALID_ARGUMENT, format == HKBS_FORMAT_PDB ? "no ATOM or HETATM records present in PDB input"
                                                                         : "no _atom_site rows present in mmCIF input");
  auto s = std::make_unique<hkbs_structure>();
  s->input_id = std::string(label);
  Options opt;
  const Status read = read_options(options, opt);
  if (!read.ok()) return report_error(read.code, read.detail);
  std::vector<Residue> residues;
  const Status st = normalize(recs, opt, *s, residues);
  if (!st.ok()) return report_error(st.code, st.detail);
  if (opt.infer) infer_missing(*s);
  *out = s.release();
  return HKBS_OK;
}

const char* const kEmpty = "";

}  // namespace

extern "C" {

void hkbs_structure_default_options(hkbs_structure_options* o) {
  if (o == nullptr) return;
  *o = hkbs_structure_options{};
  o->infer_missing_atoms = 1;
  o->include_modified_residues = 1;
}

int32_t hkbs_structure_detect_format(const char* path, const char* content, size_t nbytes) {
  return detect_format(path ? string_view(path) : string_view(),
                       content ? string_view(content, nbytes) : string_view());
}

hkbs_status hkbs_structure_load_file(const char* path, const hkbs_structure_options* options, hkbs_structure** out) {
  if (out != nullptr) *out = nullptr;
  if (path == nullptr) return report_error(HKBS_INVALID_ARGUMENT, "structure path must be non-null");
  std::ifstream in(path, std::ios::binary);
  if (!in) return report_error(HKBS_UNAVAILABLE, "structure file not readable");
  std::ostringstream buf;
  buf << in.rdbuf();
  const std::string text = buf.str();
  const string_view p(path);
  const size_t slash = p.find_last_of("/\\");
  const string_view name = slash == string_view::npos ? p : p.substr(slash + 1);
  // The file's format comes from its full path; the label is the file name.
  const int32_t format = detect_format(p, text);
  if (format == HKBS_FORMAT_UNKNOWN)
    return report_error(HKBS_INVALID_ARGUMENT,
                        "unrecognized structure file format; extension and content cues did not match PDB or mmCIF");
  return load(text, format, name, options, out);
}

hkbs_status hkbs_structure_load_buffer(const char* content, size_t nbytes, int32_t format, const char* origin_label,
                                       const hkbs_structure_options* options, hkbs_structure** out) {
  if (content == nullptr && nbytes != 0) {
    if (out != nullptr) *out = nullptr;
    return report_error(HKBS_INVALID_ARGUMENT, "structure content must be non-null");
  }
  return load(content ? string_view(content, nbytes) : string_view(), format,
              origin_label ? string_view(origin_label) : string_view(), options, out);
}

void hkbs_structure_free(hkbs_structure* s) { delete s; }

size_t hkbs_structure_residue_count(const hkbs_structure* s) { return s ? s->codes.size() : 0; }
const float* hkbs_structure_coords(const hkbs_structure* s) { return s ? s->coords.data() : nullptr; }
const uint8_t* hkbs_structure_atom_sources(const hkbs_structure* s) { return s ? s->sources.data() : nullptr; }
const char* hkbs_structure_residue_codes(const hkbs_structure* s) { return s ? s->codes.c_str() : kEmpty; }
int32_t hkbs_structure_model_index(const hkbs_structure* s) { return s ? s->model_index : 0; }

const char* hkbs_structure_text(const hkbs_structure* s, int32_t field) {
  if (s == nullptr) return kEmpty;
  switch (field) {
    case HKBS_TEXT_INPUT_ID:
    case HKBS_TEXT_SOURCE_FILENAME: return s->input_id.c_str();
    case HKBS_TEXT_MODEL_ID: return s->model_id.c_str();
    case HKBS_TEXT_CHAIN_ID: return s->chain_id.c_str();
    case HKBS_TEXT_ALTLOC_NOTE: return s->altloc_note.c_str();
    default: return kEmpty;
  }
}

const char* hkbs_structure_residue_name(const hkbs_structure* s, size_t i) {
  return (s && i < s->names.size()) ? s->names[i].c_str() : kEmpty;
}

hkbs_status hkbs_structure_residue_numbering(const hkbs_structure* s, int32_t* numbers, char* icodes,
                                             int64_t* records) {
  if (s == nullptr) return report_error(HKBS_INVALID_ARGUMENT, "structure handle must be non-null");
  const size_t L = s->codes.size();
  if (numbers) std::copy(s->numbers.begin(), s->numbers.end(), numbers);
  if (icodes) std::copy(s->icodes.begin(), s->icodes.end(), icodes);
  if (records) std::copy(s->first_records.begin(), s->first_records.begin() + L, records);
  return HKBS_OK;
}

size_t hkbs_structure_chain_count(const hkbs_structure* s) { return s ? s->chains.size() : 0; }

const char* hkbs_structure_chain_name(const hkbs_structure* s, size_t chain) {
  return (s && chain < s->chains.size()) ? s->chains[chain].c_str() : kEmpty;
}

hkbs_status hkbs_structure_chain_labels(const hkbs_structure* s, int32_t* labels) {
  if (s == nullptr || labels == nullptr) return report_error(HKBS_INVALID_ARGUMENT, "structure handle and labels must be non-null");
  std::copy(s->labels.begin(), s->labels.end(), labels);
  return HKBS_OK;
}

size_t hkbs_structure_chain_break_count(const hkbs_structure* s) { return s ? s->breaks.size() : 0; }
const uint64_t* hkbs_structure_chain_breaks(const hkbs_structure* s) { return s ? s->breaks.data() : nullptr; }

}  // extern "C"
