"""Minimal fixed-column PDB reader for design inputs.

Reads ATOM/HETATM records of one model and one chain into the canonical
``[L, 5, 3]`` N, CA, C, O, CB layout with ``AtomSource`` codes (Observed for
atoms in the file, Missing otherwise). A residue lacking CB but carrying
N, CA and C receives the ProteinMPNN virtual CB, marked Virtual, as the
reference's loader does for glycine (``cpp/io/atom_inference.cpp:46-84``).
The reference's Kabsch-template inference for other missing atoms
(``atom_inference.cpp:86-96``) is not reproduced: such atoms stay Missing,
which the design path treats as absent residues.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np

from .backbone import ALPHABET, MISSING, OBSERVED, VIRTUAL, Backbone, virtual_cb

THREE_TO_ONE = {
    "ALA": "A", "CYS": "C", "ASP": "D", "GLU": "E", "PHE": "F", "GLY": "G", "HIS": "H", "ILE": "I",
    "LYS": "K", "LEU": "L", "MET": "M", "ASN": "N", "PRO": "P", "GLN": "Q", "ARG": "R", "SER": "S",
    "THR": "T", "VAL": "V", "TRP": "W", "TYR": "Y", "MSE": "M",
}
ATOMS = {"N": 0, "CA": 1, "C": 2, "O": 3, "CB": 4}


def read_pdb(path: str | Path, chain: str | None = None) -> tuple[Backbone, str]:
    """Return (backbone, native one-letter sequence)."""
    residues: list[dict] = []
    keys: dict[tuple, int] = {}
    chosen_chain = chain
    for line in Path(path).read_text().splitlines():
        if line.startswith("ENDMDL"):
            break
        if not (line.startswith("ATOM") or line.startswith("HETATM")):
            continue
        name = line[12:16].strip()
        altloc = line[16]
        resn = line[17:20].strip()
        ch = line[21]
        resseq = int(line[22:26])
        icode = line[26]
        if chosen_chain is None:
            chosen_chain = ch
        if ch != chosen_chain or altloc not in (" ", "A") or resn not in THREE_TO_ONE:
            continue
        key = (resseq, icode)
        if key not in keys:
            keys[key] = len(residues)
            residues.append({"resn": resn, "atoms": {}})
        if name in ATOMS and name not in residues[keys[key]]["atoms"]:
            xyz = (float(line[30:38]), float(line[38:46]), float(line[46:54]))
            residues[keys[key]]["atoms"][name] = xyz
    L = len(residues)
    coords = np.zeros((L, 5, 3), dtype=np.float32)
    src = np.full((L, 5), MISSING, dtype=np.uint8)
    seq = []
    for i, r in enumerate(residues):
        seq.append(THREE_TO_ONE[r["resn"]])
        for name, a in ATOMS.items():
            if name in r["atoms"]:
                coords[i, a] = r["atoms"][name]
                src[i, a] = OBSERVED
        if src[i, 4] == MISSING and all(src[i, a] != MISSING for a in (0, 1, 2)):
            coords[i, 4] = virtual_cb(coords[i, 0], coords[i, 1], coords[i, 2])
            src[i, 4] = VIRTUAL
    return Backbone(coords, src, name=Path(path).stem), "".join(seq)


def sequence_to_tokens(seq: str) -> np.ndarray:
    return np.array([ALPHABET.index(c) if c in ALPHABET[:20] else 20 for c in seq], dtype=np.int32)
