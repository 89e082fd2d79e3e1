"""Python mirror of the reference's ``hikoboshi.inverse_fold`` (python/hikoboshi/inverse_fold.py)
on the MI355X design path.

Semantics follow the reference's algorithm layer (cpp/algorithms/inverse_fold.cpp:221-356):
sample i uses seed + i for both its random decoding order and its sampler
stream, ``sampling_temp <= 0`` means greedy, ``decode_order="n_to_c"`` uses the
identity order for every sample, backbone noise (if > 0) perturbs the
coordinates of each sample with that sample's seed before it is encoded, and
``recovery_vs_native`` is the fraction of standard native residues the design
reproduces. Without noise the backbone is encoded once and all samples are
decoded in one batched call (value-identical to the per-sample loop).
"""
from __future__ import annotations

import os
import warnings
from dataclasses import dataclass, field
from typing import Any

import numpy as np

from . import _lib, design_io, structure, weights
from .backbone import ALPHABET, Backbone
from .exceptions import FailedPreconditionError, HikoboshiError, InternalError, InvalidArgumentError, from_status

#: package id and aliases accepted for design (cpp/weights/provider.cpp:36-41), case-insensitive
PACKAGE_ID = "proteinmpnn-v48-eps020"
PACKAGE_ALIASES = (PACKAGE_ID, "v_48_020", "Hikoboshi-ProteinMPNN-v48-020", "proteinmpnn-v48-020", "proteinmpnn")
#: the reference's other compiled packages, which resolve but are not design models
OTHER_PACKAGES = ("hikoboshi-mpnn-d64", "mpnn64", "mpnn-64", "Hikoboshi-MPNN-64", "hikoboshi-esm2-8m", "esm2-8m",
                  "esm2_8m", "Hikoboshi-ESM2-8M")
UNKNOWN_PACKAGE = ("unknown Hikoboshi package id; available compiled package IDs/aliases: "
                   "hikoboshi-mpnn-d64, mpnn64, mpnn-64, Hikoboshi-MPNN-64, hikoboshi-esm2-8m, esm2-8m, esm2_8m, "
                   "Hikoboshi-ESM2-8M, proteinmpnn-v48-eps020, v_48_020, Hikoboshi-ProteinMPNN-v48-020, "
                   "proteinmpnn-v48-020, proteinmpnn")
STANDARD_AA = set("ACDEFGHIKLMNPQRSTVWY")


@dataclass(frozen=True)
class InverseFoldSequenceResult:
    sequence: str
    score: float
    recovery_vs_native: float | None
    seed: int
    decode_order: str


@dataclass(frozen=True)
class InverseFoldLogProbsArtifact:
    path: str
    shape: tuple[int, int, int]
    written: bool


@dataclass(frozen=True)
class InverseFoldResult:
    sequences: tuple[InverseFoldSequenceResult, ...]
    logprobs: InverseFoldLogProbsArtifact
    #: [num_seqs, L, 21] temperature-scaled log-probs (not part of the reference's Python result)
    log_prob_values: np.ndarray | None = field(default=None, compare=False, repr=False)


def resolve_package(package: str | None) -> str:
    """Package alias resolution and the design-model check (cpp/api/inverse_fold.cpp:95-128)."""
    if package is None or package == "":
        return PACKAGE_ID
    low = str(package).lower()
    if any(low == a.lower() for a in PACKAGE_ALIASES):
        return PACKAGE_ID
    if any(low == a.lower() for a in OTHER_PACKAGES):
        raise InvalidArgumentError("inverse_fold requires proteinmpnn-v48-eps020; it does not use the aligner "
                                   "hikoboshi-mpnn-d64 package")
    raise InvalidArgumentError(UNKNOWN_PACKAGE)


def parse_decode_order(text: str | None) -> str:
    if text is None or text == "" or text == "random":
        return "random"
    if text in ("n_to_c", "n-to-c"):
        return "n_to_c"
    raise InvalidArgumentError("inverse_fold decode_order must be 'random' or 'n_to_c'")


def recovery_vs_native(sequence: str, native: str | None) -> float | None:
    """cpp/algorithms/inverse_fold.cpp:160-184 (None when no standard native residue is known)."""
    if not native or len(native) < len(sequence):
        return None
    compared = matches = 0
    for designed, nat in zip(sequence, native):
        nat = nat.upper()
        if nat not in STANDARD_AA:
            continue
        compared += 1
        matches += designed.upper() == nat
    return matches / compared if compared else None


_CONTEXT: _lib.Context | None = None


def _context() -> _lib.Context:
    global _CONTEXT
    if _CONTEXT is None:
        _CONTEXT = _lib.Context(weights.read_package_bytes(), device=0)
    return _CONTEXT


def _check_selection(chain_id, chain_index, pdb_model_id, pdb_model_index) -> None:
    if chain_id is not None and chain_index is not None:
        raise InvalidArgumentError("choose either chain_id or chain_index, not both")
    if pdb_model_id is not None and pdb_model_index is not None:
        raise InvalidArgumentError("choose either pdb_model_id or pdb_model_index, not both")
    for name, value in (("chain_id", chain_id), ("pdb_model_id", pdb_model_id)):
        if value is not None and not isinstance(value, str):
            raise TypeError(f"{name} must be a string or None")


def structure_options(chain_id: str | None = None, chain_index: int | None = None, pdb_model_id: str | None = None,
                      pdb_model_index: int | None = None, chain_ids: Any = None,
                      all_chains: bool = False) -> structure.StructureLoadOptions:
    """Selection keywords -> loader options, with the checks of python/hikoboshi/_chain_resolve.py:79-100 and
    cpp/include/hikoboshi/bindings/engine_helpers.hpp:302-332 (empty strings leave a selection unset)."""
    _check_selection(chain_id, chain_index, pdb_model_id, pdb_model_index)
    for name, value in (("chain_index", chain_index), ("pdb_model_index", pdb_model_index)):
        if value is not None and not isinstance(value, int):
            raise InvalidArgumentError(f"{name} must be an int")
    if chain_index is not None and chain_index < 0:
        raise InternalError("can't convert negative int to unsigned")
    if pdb_model_index is not None and not -2**63 <= pdb_model_index < 2**63:
        raise InternalError("Python int too large to convert to C long")
    model_index = None
    if pdb_model_index is not None:  # narrowed to a C int like the reference binding
        model_index = (int(pdb_model_index) + 2**31) % 2**32 - 2**31
    if chain_ids is not None or all_chains:
        if chain_id is not None or chain_index is not None or (chain_ids is not None and all_chains):
            raise InvalidArgumentError("choose one chain selection: chain_id, chain_index, chain_ids or all_chains")
        if chain_ids is not None:
            if isinstance(chain_ids, str) or not all(isinstance(c, str) for c in chain_ids):
                raise InvalidArgumentError("chain_ids must be a sequence of chain id strings")
            chain_ids = tuple(chain_ids)
    return structure.StructureLoadOptions(model_index=model_index, model_id=pdb_model_id or "",
                                          chain_id=chain_id or "",
                                          chain_index=None if chain_index is None else int(chain_index) % 2**64,
                                          chain_ids=chain_ids, all_chains=bool(all_chains))


def load_structure(structure_arg: Any, options: structure.StructureLoadOptions | None = None,
                   **selection: Any) -> tuple[Backbone, str | None]:
    """A PDB / mmCIF path (loaded by the library's structure loader with the given selection), a Backbone,
    or a mapping with coords [L,5,3], atom_sources [L,5] and optional residue_codes."""
    if isinstance(structure_arg, Backbone):
        return structure_arg, structure_arg.meta.get("residue_codes")
    if isinstance(structure_arg, dict):
        bb = Backbone(np.asarray(structure_arg["coords"], np.float32),
                      np.asarray(structure_arg["atom_sources"], np.uint8))
        return bb, structure_arg.get("residue_codes")
    if isinstance(structure_arg, (str, os.PathLike)):
        loaded = structure.load_structure_from_file(structure_arg, options or structure_options(**selection))
        return loaded.backbone(), loaded.residue_codes
    raise InvalidArgumentError("structure must be a path, a Backbone or a coordinate mapping")


def design(bb: Backbone, native: str | None, *, num_seqs: int = 1, sampling_temp: float = 0.1, seed: int = 0,
           decode_order: str = "random", backbone_noise: float = 0.0, keep_log_probs: bool = True) -> InverseFoldResult:
    """The algorithm-level design loop on a loaded backbone (validation order of inverse_fold.cpp:232-261)."""
    L = bb.L
    T = float(np.float32(sampling_temp))
    noise = float(np.float32(backbone_noise))
    if L == 0:
        raise InvalidArgumentError("inverse-fold structure must contain at least one residue")
    if num_seqs <= 0:
        raise InvalidArgumentError("inverse-fold num_seqs must be greater than zero")
    if not np.isfinite(T) or T < 0.0:
        raise InvalidArgumentError("inverse-fold sampling_temp must be finite and >= 0")
    if not np.isfinite(noise) or noise < 0.0:
        raise InvalidArgumentError("inverse-fold backbone_noise must be finite and >= 0")
    order = parse_decode_order(decode_order)
    seeds = (np.uint64(seed) + np.arange(num_seqs, dtype=np.uint64)).astype(np.uint64)
    mode = _lib.ORDER_N_TO_C if order == "n_to_c" else _lib.ORDER_RANDOM
    ctx = _context()
    try:
        if noise > 0.0:
            outs = []
            for s in seeds:
                coords = _lib.backbone_noise(bb.coords, bb.atom_sources, noise, int(s))
                outs.append(ctx.design(coords, bb.atom_sources, 1, np.array([s], np.uint64), order_mode=mode,
                                       order_seeds=np.array([s], np.uint64), temperature=T, greedy=T <= 0.0,
                                       residue_indices=bb.residue_indices, chain_labels=bb.chain_labels))
            res = {k: np.concatenate([o[k] for o in outs]) for k in ("tokens", "log_probs", "scores")}
        else:
            res = ctx.design(bb.coords, bb.atom_sources, int(num_seqs), seeds, order_mode=mode, order_seeds=seeds,
                             temperature=T, greedy=T <= 0.0, residue_indices=bb.residue_indices,
                             chain_labels=bb.chain_labels)
    except _lib.HkbsError as exc:
        raise from_status(exc.code, exc.detail) from exc
    seqs = []
    for i in range(num_seqs):
        s = "".join(ALPHABET[t] if 0 <= t < 21 else "X" for t in res["tokens"][i])
        seqs.append(InverseFoldSequenceResult(sequence=s, score=float(np.float32(res["scores"][i])),
                                              recovery_vs_native=recovery_vs_native(s, native), seed=int(seeds[i]),
                                              decode_order=order))
    values = res["log_probs"] if keep_log_probs else None
    return InverseFoldResult(tuple(seqs), InverseFoldLogProbsArtifact("", (0, 0, 0), False), values)


def _deprecated_model_kwargs(kwargs: dict, pdb_model_id: str | None,
                             pdb_model_index: int | None) -> tuple[str | None, int | None]:
    """model_id / model_index spellings (python/hikoboshi/_chain_resolve.py:30-61)."""
    context = "inverse_fold.from_structure"
    if "model_id" in kwargs:
        if pdb_model_id is not None:
            raise InvalidArgumentError(f"choose either pdb_model_id or deprecated model_id for {context}, not both")
        pdb_model_id = kwargs.pop("model_id")
        warnings.warn("model_id is deprecated; use pdb_model_id", DeprecationWarning, stacklevel=3)
    if "model_index" in kwargs:
        if pdb_model_index is not None:
            raise InvalidArgumentError(f"choose either pdb_model_index or deprecated model_index for {context}, "
                                       "not both")
        pdb_model_index = kwargs.pop("model_index")
        warnings.warn("model_index is deprecated; use pdb_model_index", DeprecationWarning, stacklevel=3)
    return pdb_model_id, pdb_model_index


class InverseFoldNamespace:
    def __call__(self, structure: Any, **kwargs: Any) -> InverseFoldResult:
        return self.from_structure(structure, **kwargs)

    def from_structure(self, structure: Any, *, num_seqs: int = 1, sampling_temp: float = 0.1, seed: int = 0,
                       decode_order: str = "random", package: str | None = None, backbone_noise: float = 0.0,
                       out_logprobs: str | None = None, chain_id: str | None = None, chain_index: int | None = None,
                       pdb_model_id: str | None = None, pdb_model_index: int | None = None,
                       chain_ids: Any = None, all_chains: bool = False, **kwargs: Any) -> InverseFoldResult:
        """python/hikoboshi/inverse_fold.py:20-65 and the argument order of
        cpp/bindings/inverse_fold_bindings.cpp:182-274 (decode order, structure selection and loading, then
        the package). ``chain_ids`` (a sequence) or ``all_chains=True`` extend the reference's one-chain
        selection: the chains are designed together, with ProteinMPNN's chain labels and residue offsets."""
        pdb_model_id, pdb_model_index = _deprecated_model_kwargs(kwargs, pdb_model_id, pdb_model_index)
        if kwargs:
            raise InvalidArgumentError(f"unknown inverse_fold.from_structure keyword(s): {', '.join(sorted(kwargs))}")
        _check_selection(chain_id, chain_index, pdb_model_id, pdb_model_index)
        order = parse_decode_order(decode_order)
        bb, native = load_structure(structure, structure_options(chain_id, chain_index, pdb_model_id,
                                                                 pdb_model_index, chain_ids, all_chains))
        resolve_package(package)
        result = design(bb, native, num_seqs=int(num_seqs), sampling_temp=float(sampling_temp), seed=int(seed),
                        decode_order=order, backbone_noise=float(backbone_noise))
        artifact = InverseFoldLogProbsArtifact("", (0, 0, 0), False)
        if out_logprobs:
            design_io.write_inverse_fold_logprobs_npz(out_logprobs, result.log_prob_values)
            artifact = InverseFoldLogProbsArtifact(str(out_logprobs), tuple(result.log_prob_values.shape), True)
        return InverseFoldResult(result.sequences, artifact, result.log_prob_values)

    def from_pdb(self, structure: Any, **kwargs: Any) -> InverseFoldResult:
        return self.from_structure(structure, **kwargs)

    def from_cif(self, structure: Any, **kwargs: Any) -> InverseFoldResult:
        return self.from_structure(structure, **kwargs)


inverse_fold = InverseFoldNamespace()

__all__ = ["InverseFoldNamespace", "inverse_fold", "InverseFoldResult", "InverseFoldSequenceResult",
           "InverseFoldLogProbsArtifact", "design", "resolve_package", "parse_decode_order", "recovery_vs_native", "load_structure",
           "structure_options",
           "HikoboshiError", "FailedPreconditionError"]
