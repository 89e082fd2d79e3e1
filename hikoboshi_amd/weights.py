"""ProteinMPNN v_48_020 weight package: safetensors parsing and tensor order.

The package is the reference's embedded artefact
(``weights/Hikoboshi-ProteinMPNN-v48-020.safetensors``, 118 F32 tensors,
sha256 ``342b52ae...``; schema in the reference at
``cpp/include/hikoboshi/universal/detail/proteinmpnn_v48_020_schema.hpp:127-156``).
The HIP library parses the same bytes itself (``hkbs_pmpnn_create``); this
module gives Python callers the file bytes, an independent parse for the CPU
oracle, and the canonical tensor order shared by both.
"""
from __future__ import annotations

import hashlib
import json
import struct
from pathlib import Path

import numpy as np

PACKAGE_ID = "proteinmpnn-v48-eps020"
PACKAGE_ALIASES = ("proteinmpnn-v48-eps020", "proteinmpnn-v48-020", "proteinmpnn")
WEIGHTS_SHA256 = "342b52ae248f2b70b2059313bab5ae7a358cbabac940072f71f5907eeaa21536"
DEFAULT_WEIGHTS = Path(__file__).resolve().parent.parent / "weights" / "Hikoboshi-ProteinMPNN-v48-020.safetensors"


def _enc_names(layer: int) -> list[str]:
    p = f"encoder_layers.{layer}."
    out = []
    for lin in ("W1", "W2", "W3", "W11", "W12", "W13"):
        out += [p + lin + ".weight", p + lin + ".bias"]
    for n in ("norm1", "norm2", "norm3"):
        out += [p + n + ".weight", p + n + ".bias"]
    out += [p + "dense.W_in.weight", p + "dense.W_in.bias", p + "dense.W_out.weight", p + "dense.W_out.bias"]
    return out


def _dec_names(layer: int) -> list[str]:
    p = f"decoder_layers.{layer}."
    out = []
    for lin in ("W1", "W2", "W3"):
        out += [p + lin + ".weight", p + lin + ".bias"]
    for n in ("norm1", "norm2"):
        out += [p + n + ".weight", p + n + ".bias"]
    out += [p + "dense.W_in.weight", p + "dense.W_in.bias", p + "dense.W_out.weight", p + "dense.W_out.bias"]
    return out


#: Canonical order of the 118 tensors (index = position). The C oracle, the
#: reference driver and the HIP library's loader all use this order.
CANONICAL_TENSORS: tuple[str, ...] = tuple(
    [
        "features.embeddings.linear.weight",
        "features.embeddings.linear.bias",
        "features.edge_embedding.weight",
        "features.norm_edges.weight",
        "features.norm_edges.bias",
        "W_e.weight",
        "W_e.bias",
        "W_s.weight",
    ]
    + _enc_names(0)
    + _enc_names(1)
    + _enc_names(2)
    + _dec_names(0)
    + _dec_names(1)
    + _dec_names(2)
    + ["W_out.weight", "W_out.bias"]
)
assert len(CANONICAL_TENSORS) == 118

EXPECTED_SHAPES: dict[str, tuple[int, ...]] = {
    "features.embeddings.linear.weight": (16, 66),
    "features.embeddings.linear.bias": (16,),
    "features.edge_embedding.weight": (128, 416),
    "features.norm_edges.weight": (128,),
    "features.norm_edges.bias": (128,),
    "W_e.weight": (128, 128),
    "W_e.bias": (128,),
    "W_s.weight": (21, 128),
    "W_out.weight": (21, 128),
    "W_out.bias": (21,),
}
for _l in range(3):
    for _n in _enc_names(_l):
        if _n.endswith("W1.weight") or _n.endswith("W11.weight"):
            EXPECTED_SHAPES[_n] = (128, 384)
        elif _n.endswith("W_in.weight"):
            EXPECTED_SHAPES[_n] = (512, 128)
        elif _n.endswith("W_in.bias"):
            EXPECTED_SHAPES[_n] = (512,)
        elif _n.endswith("W_out.weight"):
            EXPECTED_SHAPES[_n] = (128, 512)
        elif _n.endswith(".weight") and ".W" in _n:
            EXPECTED_SHAPES[_n] = (128, 128)
        else:
            EXPECTED_SHAPES[_n] = (128,)
    for _n in _dec_names(_l):
        if _n.endswith("W1.weight"):
            EXPECTED_SHAPES[_n] = (128, 512)
        elif _n.endswith("W_in.weight"):
            EXPECTED_SHAPES[_n] = (512, 128)
        elif _n.endswith("W_in.bias"):
            EXPECTED_SHAPES[_n] = (512,)
        elif _n.endswith("W_out.weight"):
            EXPECTED_SHAPES[_n] = (128, 512)
        elif _n.endswith(".weight") and ".W" in _n:
            EXPECTED_SHAPES[_n] = (128, 128)
        else:
            EXPECTED_SHAPES[_n] = (128,)


class WeightsError(ValueError):
    """Raised for a malformed or mismatching weight package."""


def resolve_package(package: str | None) -> str:
    """Mirror of the reference's package alias resolution (cpp/weights/provider.cpp:516)."""
    if package is None or package in PACKAGE_ALIASES:
        return PACKAGE_ID
    raise WeightsError(f"unsupported design package: {package!r} (expected {PACKAGE_ID})")


def read_package_bytes(path: str | Path | None = None, verify: bool = True) -> bytes:
    data = Path(path or DEFAULT_WEIGHTS).read_bytes()
    if verify and hashlib.sha256(data).hexdigest() != WEIGHTS_SHA256:
        raise WeightsError("ProteinMPNN v_48_020 weights sha256 mismatch")
    return data


def parse_safetensors(data: bytes) -> dict[str, np.ndarray]:
    """Parse a safetensors byte string (8-byte LE header length, JSON header, payload)."""
    if len(data) < 8:
        raise WeightsError("safetensors blob too short")
    (n,) = struct.unpack("<Q", data[:8])
    if 8 + n > len(data):
        raise WeightsError("safetensors header length exceeds blob")
    header = json.loads(data[8 : 8 + n].decode("utf-8"))
    base = 8 + n
    out: dict[str, np.ndarray] = {}
    for name, meta in header.items():
        if name == "__metadata__":
            continue
        if meta.get("dtype") != "F32":
            raise WeightsError(f"{name}: only F32 tensors are supported")
        start, end = meta["data_offsets"]
        shape = tuple(int(s) for s in meta["shape"])
        count = int(np.prod(shape)) if shape else 1
        if end - start != 4 * count or base + end > len(data):
            raise WeightsError(f"{name}: bad data offsets")
        out[name] = np.frombuffer(data, dtype="<f4", count=count, offset=base + start).reshape(shape)
    return out


def load_tensors(path: str | Path | None = None) -> list[np.ndarray]:
    """Return the 118 tensors, C-contiguous float32, in canonical order."""
    tensors = parse_safetensors(read_package_bytes(path))
    ordered = []
    for name in CANONICAL_TENSORS:
        if name not in tensors:
            raise WeightsError(f"missing tensor {name}")
        t = np.ascontiguousarray(tensors[name], dtype=np.float32)
        if t.shape != EXPECTED_SHAPES[name]:
            raise WeightsError(f"{name}: shape {t.shape} != {EXPECTED_SHAPES[name]}")
        ordered.append(t)
    return ordered


def synthetic_tensors(seed: int = 0, scale: float = 0.05) -> list[np.ndarray]:
    """Random weights of the v_48_020 architecture (for shape/edge-case tests)."""
    rng = np.random.default_rng(seed)
    out = []
    for name in CANONICAL_TENSORS:
        shape = EXPECTED_SHAPES[name]
        if "norm" in name and name.endswith(".weight"):
            t = 1.0 + 0.1 * rng.standard_normal(shape)
        else:
            t = scale * rng.standard_normal(shape)
        out.append(np.ascontiguousarray(t, dtype=np.float32))
    return out


def tensors_to_safetensors(tensors: list[np.ndarray]) -> bytes:
    """Serialise canonical-order tensors back to safetensors bytes."""
    header = {}
    payload = bytearray()
    for name, t in zip(CANONICAL_TENSORS, tensors):
        b = np.ascontiguousarray(t, dtype="<f4").tobytes()
        header[name] = {"dtype": "F32", "shape": list(t.shape), "data_offsets": [len(payload), len(payload) + len(b)]}
        payload += b
    h = json.dumps(header).encode("utf-8")
    pad = (8 - len(h) % 8) % 8
    h += b" " * pad
    return struct.pack("<Q", len(h)) + h + bytes(payload)
