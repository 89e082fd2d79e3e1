"""Design outputs in the reference's byte formats (cpp/io/design_fasta_writer.cpp:62-217).

FASTA: one record per sequence,
    >design_{i+1} score={score} seed={seed} T={T} decode_order={random|n_to_c}
with score and T printed like a C++ stream at precision 7 (``%.7g`` of the
value as a double) and the sequence wrapped at 80 columns.
NPZ: an uncompressed ZIP (version 2.0, zero timestamps) holding one member,
``log_probs.npy``: NPY 1.0, ``<f4``, shape (N, L, 21), header padded with
spaces to a 16-byte boundary.
"""
from __future__ import annotations

import struct
import zlib
from pathlib import Path

import numpy as np

from .exceptions import InvalidArgumentError, UnavailableError

NPY_NAME = b"log_probs.npy"


def _g7(value: float) -> str:
    return "%.7g" % float(value)


def design_fasta_text(sequences, sampling_temp: float) -> str:
    """sequences: iterable of objects with .sequence, .score, .seed, .decode_order."""
    t = _g7(np.float32(sampling_temp))
    out = []
    for i, s in enumerate(sequences):
        out.append(f">design_{i + 1} score={_g7(s.score)} seed={int(s.seed)} T={t} decode_order={s.decode_order}\n")
        seq = s.sequence
        for off in range(0, len(seq), 80):
            out.append(seq[off:off + 80] + "\n")
    return "".join(out)


def write_design_fasta(path, sequences, sampling_temp: float = 0.1) -> None:
    if not path:
        raise InvalidArgumentError("design FASTA output path is required")
    try:
        Path(path).write_bytes(design_fasta_text(sequences, sampling_temp).encode())
    except OSError as exc:
        raise UnavailableError("design FASTA output is not writable") from exc


def npy_bytes(values: np.ndarray) -> bytes:
    v = np.ascontiguousarray(values, dtype="<f4")
    header = "{'descr': '<f4', 'fortran_order': False, 'shape': (%d, %d, %d), }" % v.shape
    pad = (16 - ((10 + len(header) + 1) % 16)) % 16
    header = header + " " * pad + "\n"
    return b"\x93NUMPY\x01\x00" + struct.pack("<H", len(header)) + header.encode("latin1") + v.tobytes()


def npz_bytes(values: np.ndarray) -> bytes:
    payload = npy_bytes(values)
    if len(payload) > 0xFFFFFFFF:
        raise InvalidArgumentError("inverse-fold log-prob artifact is too large for ZIP32")
    crc = zlib.crc32(payload) & 0xFFFFFFFF
    size = len(payload)
    local = struct.pack("<IHHHHHIIIHH", 0x04034B50, 20, 0, 0, 0, 0, crc, size, size, len(NPY_NAME), 0)
    body = local + NPY_NAME + payload
    if len(body) > 0xFFFFFFFF:
        raise InvalidArgumentError("inverse-fold log-prob artifact is too large for ZIP32")
    cd_offset = len(body)
    central = struct.pack("<IHHHHHHIIIHHHHHII", 0x02014B50, 20, 20, 0, 0, 0, 0, crc, size, size, len(NPY_NAME),
                          0, 0, 0, 0, 0, 0) + NPY_NAME
    eocd = struct.pack("<IHHHHIIH", 0x06054B50, 0, 0, 1, 1, len(central), cd_offset, 0)
    return body + central + eocd


def write_inverse_fold_logprobs_npz(path, values: np.ndarray) -> None:
    if not path:
        raise InvalidArgumentError("inverse-fold log-prob output path is required")
    v = np.asarray(values)
    if v.ndim != 3 or v.size == 0:
        raise InvalidArgumentError("inverse-fold log-prob artifact shape is invalid")
    data = npz_bytes(v)
    try:
        Path(path).write_bytes(data)
    except OSError as exc:
        raise UnavailableError("inverse-fold log-prob artifact is not writable") from exc
