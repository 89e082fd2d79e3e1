/*
 * hkbs_structure.h - structure input of the design path: PDB and mmCIF
 * loading into the canonical backbone layout consumed by hkbs_pmpnn_design.
 *
 * Replaces the reference's host-side loader
 *   hikoboshi::io::load_structure_from_file   (cpp/io/structure_loader.cpp:167-194)
 *   hikoboshi::io::load_pdb_from_string       (cpp/io/structure_loader.cpp:196-235)
 *   hikoboshi::io::load_mmcif_from_string     (cpp/io/structure_loader.cpp:237-276)
 *   hikoboshi::io::detect_structure_format    (cpp/io/structure_loader.cpp:149-165)
 * with its options struct StructureLoadOptions
 *   (cpp/include/hikoboshi/io/structure_loader.hpp:30-38)
 * and the accessors of LoadedStructure / StructureView
 *   (cpp/include/hikoboshi/io/structure_loader.hpp:86-130).
 *
 * Output layout: coords [L,5,3] float (N, CA, C, O, CB), atom_sources [L,5]
 * uint8 AtomSource codes (0 Missing, 1 Observed, 2 Inferred, 3 Virtual),
 * residue_codes L one-letter codes ('X' for unknown names). Status codes and
 * hkbs_last_error() are shared with hkbs_pmpnn.h; detail strings are the
 * reference's messages. Host code only: no call here touches a GPU.
 */
#ifndef HKBS_STRUCTURE_H
#define HKBS_STRUCTURE_H

#include <stddef.h>
#include <stdint.h>

#include "hkbs_pmpnn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* StructureFormat (cpp/include/hikoboshi/io/structure_loader.hpp). */
enum { HKBS_FORMAT_UNKNOWN = 0, HKBS_FORMAT_PDB = 1, HKBS_FORMAT_MMCIF = 2 };

/* Text fields of a loaded structure (hkbs_structure_text). */
enum {
  HKBS_TEXT_INPUT_ID = 0,        /* file name without directories */
  HKBS_TEXT_SOURCE_FILENAME = 1, /* same as the input id for file loads */
  HKBS_TEXT_MODEL_ID = 2,        /* id string of the selected model */
  HKBS_TEXT_CHAIN_ID = 3,        /* selected chain ("" for a blank chain column); several
                                    selected chains are joined by commas */
  HKBS_TEXT_ALTLOC_NOTE = 4      /* "altloc selection applied" or "" */
};

/* StructureLoadOptions. Unset selections fall back to model 1 and chain "A"
 * (else the first polymer chain of the model); model_index wins over
 * model_id and chain_id over chain_index. chain_ids and all_chains exclude
 * every other chain selection.
 *
 * chain_ids / all_chains extend the reference's options (which select one
 * chain) so that a multichain design reaches hkbs_pmpnn_design: residues are
 * grouped by chain in the requested order (all_chains: order of first
 * appearance in the model) and hkbs_structure_chain_labels gives each
 * residue's chain. */
typedef struct hkbs_structure_options {
  int32_t has_model_index;
  int32_t model_index;
  const char* model_id; /* NULL or "" = unset */
  const char* chain_id; /* NULL or "" = unset */
  int32_t has_chain_index;
  uint64_t chain_index;
  int32_t infer_missing_atoms;       /* default 1 */
  int32_t include_modified_residues; /* default 1 */
  const char* const* chain_ids;      /* n_chain_ids distinct chain ids ("" = blank chain) */
  size_t n_chain_ids;
  int32_t all_chains;                /* every polymer chain of the selected model */
} hkbs_structure_options;

typedef struct hkbs_structure hkbs_structure;

/* Fills the defaults above. */
void hkbs_structure_default_options(hkbs_structure_options* options);

/* Format from the path's extension (.cif/.mmcif, .pdb/.ent, any case), else
 * from content cues (leading "data_" or an "_atom_site." tag; a line starting
 * "ATOM  ", "HETATM" or "MODEL "). */
int32_t hkbs_structure_detect_format(const char* path, const char* content, size_t nbytes);

/* Reads and loads a file (format from hkbs_structure_detect_format).
 * HKBS_UNAVAILABLE "structure file not readable" if it cannot be opened.
 * options may be NULL (defaults). On success *out owns the result. */
hkbs_status hkbs_structure_load_file(const char* path, const hkbs_structure_options* options,
                                     hkbs_structure** out);

/* Loads text held in memory. format HKBS_FORMAT_PDB / _MMCIF selects the
 * parser; HKBS_FORMAT_UNKNOWN detects it from origin_label and content.
 * origin_label (may be NULL) becomes the input id and source filename. */
hkbs_status hkbs_structure_load_buffer(const char* content, size_t nbytes, int32_t format,
                                       const char* origin_label, const hkbs_structure_options* options,
                                       hkbs_structure** out);

void hkbs_structure_free(hkbs_structure* structure);

/* Accessors; pointers stay valid until hkbs_structure_free. */
size_t hkbs_structure_residue_count(const hkbs_structure* structure);
const float* hkbs_structure_coords(const hkbs_structure* structure);         /* [L,5,3] */
const uint8_t* hkbs_structure_atom_sources(const hkbs_structure* structure); /* [L,5] */
const char* hkbs_structure_residue_codes(const hkbs_structure* structure);   /* L chars + NUL */
int32_t hkbs_structure_model_index(const hkbs_structure* structure);
const char* hkbs_structure_text(const hkbs_structure* structure, int32_t field);
/* Original residue name of residue i as written in the file ("" if i >= L). */
const char* hkbs_structure_residue_name(const hkbs_structure* structure, size_t residue);
/* Per-residue numbering; each output (length L) may be NULL. */
hkbs_status hkbs_structure_residue_numbering(const hkbs_structure* structure, int32_t* residue_numbers,
                                             char* insertion_codes, int64_t* source_record_indices);
/* Selected chains in output order, and each residue's index into them (L values). */
size_t hkbs_structure_chain_count(const hkbs_structure* structure);
const char* hkbs_structure_chain_name(const hkbs_structure* structure, size_t chain);
hkbs_status hkbs_structure_chain_labels(const hkbs_structure* structure, int32_t* labels);
/* Chain breaks: indices of the residues after which the numbering jumps
 * within a chain. */
size_t hkbs_structure_chain_break_count(const hkbs_structure* structure);
const uint64_t* hkbs_structure_chain_breaks(const hkbs_structure* structure);

#ifdef __cplusplus
}
#endif

#endif /* HKBS_STRUCTURE_H */
