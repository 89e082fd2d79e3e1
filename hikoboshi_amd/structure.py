"""Structure input of the design path: PDB / mmCIF files -> canonical backbone.

Python face of include/hkbs_structure.h, mirroring the reference's loader
(``hikoboshi::io``, cpp/include/hikoboshi/io/structure_loader.hpp:20-170):
``StructureLoadOptions``, ``load_structure_from_file``, ``load_pdb_from_string``,
``load_mmcif_from_string`` and ``detect_structure_format``, returning a
``LoadedStructure`` with the fields of the reference's ``StructureView``
(cpp/include/hikoboshi/universal/structure.hpp). Failures raise the structured
errors of ``hikoboshi_amd.exceptions`` with the reference's messages.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

from . import _lib
from .backbone import Backbone
from .exceptions import InvalidArgumentError, from_status

FORMATS = {_lib.FORMAT_UNKNOWN: "unknown", _lib.FORMAT_PDB: "pdb", _lib.FORMAT_MMCIF: "mmcif"}


@dataclass(frozen=True)
class StructureLoadOptions:
    """cpp/include/hikoboshi/io/structure_loader.hpp:30-38."""

    model_index: int | None = None
    model_id: str = ""
    chain_id: str = ""
    chain_index: int | None = None
    infer_missing_atoms: bool = True
    include_modified_residues: bool = True
    #: several chains, designed together in this order (an extension of the reference's options)
    chain_ids: tuple[str, ...] | None = None
    #: every polymer chain of the model in order of first appearance (extension)
    all_chains: bool = False

    def _c(self) -> tuple[_lib.StructureOptions, object]:
        """The C struct, and the buffer its chain_ids point into (keep it alive for the call)."""
        o = _lib.StructureOptions()
        _lib.load().hkbs_structure_default_options(C.byref(o))
        if self.model_index is not None:
            o.has_model_index, o.model_index = 1, int(self.model_index)
        o.model_id = (self.model_id or "").encode()
        o.chain_id = (self.chain_id or "").encode()
        if self.chain_index is not None:
            o.has_chain_index, o.chain_index = 1, int(self.chain_index)
        o.infer_missing_atoms = int(bool(self.infer_missing_atoms))
        o.include_modified_residues = int(bool(self.include_modified_residues))
        keep = None
        if self.chain_ids is not None:
            ids = [str(c).encode() for c in self.chain_ids]
            if not ids:
                raise InvalidArgumentError("chain_ids must name at least one chain")
            keep = (C.c_char_p * len(ids))(*ids)
            o.chain_ids = C.cast(keep, C.POINTER(C.c_char_p))
            o.n_chain_ids = len(ids)
        o.all_chains = int(bool(self.all_chains))
        return o, keep


@dataclass(frozen=True)
class ResidueMetadata:
    """Per-residue fields of ResidueMetadataView (cpp/io/structure_normalize.cpp:338-354)."""

    residue_code: str
    original_residue_name: str
    chain_id: str
    model_id: str
    model_index: int
    residue_number: int
    insertion_code: str
    source_id: str
    source_residue_index: int
    source_filename: str
    source_record_index: int


@dataclass(frozen=True)
class LoadedStructure:
    coords: np.ndarray  # [L,5,3] float32, N CA C O CB
    atom_sources: np.ndarray  # [L,5] uint8 AtomSource codes
    residue_codes: str
    residues: tuple[ResidueMetadata, ...]
    chain_breaks: tuple[int, ...]
    input_id: str
    source_filename: str
    selected_model_id: str
    selected_model_index: int
    selected_chain_id: str  # several selected chains: their ids joined by commas
    altloc_note: str
    numbering: dict = field(repr=False, compare=False, default_factory=dict)
    #: selected chains in output order, and each residue's index into them
    chain_ids: tuple[str, ...] = ()
    chain_labels: np.ndarray | None = field(default=None, repr=False, compare=False)

    @property
    def residue_count(self) -> int:
        return len(self.residue_codes)

    def backbone(self) -> Backbone:
        """The design input. Several chains carry ProteinMPNN's multichain encoding: chain labels, and residue
        indices that count positions with a jump of 100 between chains (only same-chain offsets enter the
        positional features)."""
        labels = resid = None
        if len(self.chain_ids) > 1:
            labels = np.ascontiguousarray(self.chain_labels, np.int32)
            resid = (np.arange(self.residue_count, dtype=np.int32) + 100 * labels).astype(np.int32)
        return Backbone(self.coords, self.atom_sources, residue_indices=resid, chain_labels=labels,
                        name=Path(self.input_id).stem or "structure",
                        meta={"residue_codes": self.residue_codes, "chain_id": self.selected_chain_id,
                              "model_id": self.selected_model_id})


def _status(code: int) -> None:
    if code != _lib.OK:
        detail = _lib.load().hkbs_last_error()
        raise from_status(code, detail.decode() if detail else "")


def _take(handle: C.c_void_p) -> LoadedStructure:
    lib = _lib.load()
    try:
        L = int(lib.hkbs_structure_residue_count(handle))
        coords = np.ctypeslib.as_array(lib.hkbs_structure_coords(handle), shape=(L * 15,)).copy() if L else \
            np.zeros(0, np.float32)
        src = np.ctypeslib.as_array(lib.hkbs_structure_atom_sources(handle), shape=(L * 5,)).copy() if L else \
            np.zeros(0, np.uint8)
        codes = lib.hkbs_structure_residue_codes(handle).decode()
        numbers = np.zeros(L, np.int32)
        icodes = np.zeros(L, np.uint8)
        records = np.zeros(L, np.int64)
        _status(lib.hkbs_structure_residue_numbering(handle, _lib.ptr(numbers), _lib.ptr(icodes), _lib.ptr(records)))
        nb = int(lib.hkbs_structure_chain_break_count(handle))
        breaks = tuple(int(b) for b in np.ctypeslib.as_array(lib.hkbs_structure_chain_breaks(handle), shape=(nb,))) \
            if nb else ()
        text = {f: lib.hkbs_structure_text(handle, f).decode("utf-8", "replace") for f in range(5)}
        model_index = int(lib.hkbs_structure_model_index(handle))
        names = [lib.hkbs_structure_residue_name(handle, i).decode("utf-8", "replace") for i in range(L)]
        chains = tuple(lib.hkbs_structure_chain_name(handle, c).decode("utf-8", "replace")
                       for c in range(int(lib.hkbs_structure_chain_count(handle))))
        labels = np.zeros(L, np.int32)
        if L:
            _status(lib.hkbs_structure_chain_labels(handle, _lib.ptr(labels)))
    finally:
        lib.hkbs_structure_free(handle)
    chain, model_id, fname = text[_lib.TEXT_CHAIN_ID], text[_lib.TEXT_MODEL_ID], text[_lib.TEXT_SOURCE_FILENAME]
    residues = tuple(
        ResidueMetadata(codes[i], names[i], chains[labels[i]], model_id, model_index, int(numbers[i]), chr(icodes[i]),
                        f"{chains[labels[i]]}_{int(numbers[i])}", i, fname, int(records[i]))
        for i in range(L))
    return LoadedStructure(coords.reshape(L, 5, 3), src.reshape(L, 5), codes, residues, breaks,
                           text[_lib.TEXT_INPUT_ID], fname, model_id, model_index, chain, text[_lib.TEXT_ALTLOC_NOTE],
                           {"residue_numbers": numbers, "insertion_codes": icodes, "source_record_indices": records},
                           chains, labels)


def detect_structure_format(path: str | os.PathLike = "", content: str | bytes = b"") -> str:
    """'pdb', 'mmcif' or 'unknown' (cpp/io/structure_loader.cpp:149-165)."""
    data = content.encode() if isinstance(content, str) else bytes(content)
    return FORMATS[int(_lib.load().hkbs_structure_detect_format(os.fsencode(path), data, len(data)))]


def load_structure_from_file(path: str | os.PathLike,
                             options: StructureLoadOptions | None = None) -> LoadedStructure:
    """cpp/io/structure_loader.cpp:167-194: read, detect format, parse, select, infer."""
    h = C.c_void_p()
    opts, keep = (options or StructureLoadOptions())._c()
    _status(_lib.load().hkbs_structure_load_file(os.fsencode(path), C.byref(opts), C.byref(h)))
    del keep
    return _take(h)


def _load_text(content: str | bytes, fmt: int, origin_label: str,
               options: StructureLoadOptions | None) -> LoadedStructure:
    data = content.encode() if isinstance(content, str) else bytes(content)
    h = C.c_void_p()
    opts, keep = (options or StructureLoadOptions())._c()
    _status(_lib.load().hkbs_structure_load_buffer(data, len(data), fmt, origin_label.encode(), C.byref(opts),
                                                   C.byref(h)))
    del keep
    return _take(h)


def load_pdb_from_string(content: str | bytes, origin_label: str = "",
                         options: StructureLoadOptions | None = None) -> LoadedStructure:
    """cpp/io/structure_loader.cpp:196-235."""
    return _load_text(content, _lib.FORMAT_PDB, origin_label, options)


def load_mmcif_from_string(content: str | bytes, origin_label: str = "",
                           options: StructureLoadOptions | None = None) -> LoadedStructure:
    """cpp/io/structure_loader.cpp:237-276."""
    return _load_text(content, _lib.FORMAT_MMCIF, origin_label, options)


def read_backbone(path: str | os.PathLike, options: StructureLoadOptions | None = None) -> tuple[Backbone, str]:
    """(backbone, residue codes) of a structure file."""
    loaded = load_structure_from_file(path, options)
    return loaded.backbone(), loaded.residue_codes


__all__ = ["StructureLoadOptions", "read_backbone", "LoadedStructure", "ResidueMetadata", "detect_structure_format",
           "load_structure_from_file", "load_pdb_from_string", "load_mmcif_from_string"]
