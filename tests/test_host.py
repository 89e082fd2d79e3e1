"""Host-side logic and the C ABI surface (no GPU compute)."""
import ctypes as C
import re

import numpy as np
import pytest

from hikoboshi_amd import _lib, backbone, structure, weights

from .conftest import FIXTURES, ROOT, golden_cases


def test_weights_package(tensors):
    assert len(tensors) == 118
    for name, t in zip(weights.CANONICAL_TENSORS, tensors):
        assert t.shape == weights.EXPECTED_SHAPES[name]
        assert t.dtype == np.float32 and np.isfinite(t).all()
    assert weights.resolve_package(None) == "proteinmpnn-v48-eps020"
    assert weights.resolve_package("proteinmpnn") == "proteinmpnn-v48-eps020"
    with pytest.raises(weights.WeightsError):
        weights.resolve_package("mpnn-d64")


def test_safetensors_roundtrip(tensors):
    blob = weights.tensors_to_safetensors(tensors)
    back = weights.parse_safetensors(blob)
    for name, t in zip(weights.CANONICAL_TENSORS, tensors):
        np.testing.assert_array_equal(back[name], t)


def _dihedral(p0, p1, p2, p3):
    b0, b1, b2 = p0 - p1, p2 - p1, p3 - p2
    b1 = b1 / np.linalg.norm(b1)
    v = b0 - np.dot(b0, b1) * b1
    w = b2 - np.dot(b2, b1) * b1
    return np.degrees(np.arctan2(np.dot(np.cross(b1, v), w), np.dot(v, w)))


def test_backbone_geometry():
    bb = backbone.single_chain(120, 7)
    x = bb.coords.astype(np.float64)
    n, ca, c, o, cb = (x[:, i] for i in range(5))
    np.testing.assert_allclose(np.linalg.norm(ca - n, axis=1), 1.458, atol=2e-4)
    np.testing.assert_allclose(np.linalg.norm(c - ca, axis=1), 1.525, atol=2e-4)
    np.testing.assert_allclose(np.linalg.norm(n[1:] - c[:-1], axis=1), 1.329, atol=2e-4)
    np.testing.assert_allclose(np.linalg.norm(o - c, axis=1), 1.231, atol=2e-4)
    # virtual CB sits ~1.52 A from CA for ideal geometry
    assert np.abs(np.linalg.norm(cb - ca, axis=1) - 1.52).max() < 0.03
    # omega = 180, O anti to N(i+1)
    for i in range(0, 119, 13):
        assert abs(abs(_dihedral(ca[i], c[i], n[i + 1], ca[i + 1])) - 180.0) < 1e-2
        assert abs(abs(_dihedral(n[i + 1], ca[i], c[i], o[i])) - 180.0) < 1e-2
    # helix and strand segments: phi near -57 / -120 within 4 sigma
    phis = [_dihedral(c[i - 1], n[i], ca[i], c[i]) for i in range(1, 120)]
    assert all(min(abs(p + 57), abs(p + 120)) < 40 for p in phis)
    assert (bb.atom_sources[:, :4] == backbone.OBSERVED).all() and (bb.atom_sources[:, 4] == backbone.VIRTUAL).all()


def test_complex_layout():
    cx = backbone.tetrahedral_complex(256, 7)
    assert cx.L == 1024
    cents = np.stack([cx.coords[cx.chain_labels == c, 1].mean(0) for c in range(4)])
    d = np.linalg.norm(cents[:, None] - cents[None], axis=-1)
    np.testing.assert_allclose(d[np.triu_indices(4, 1)], 25.0, atol=1e-3)
    assert (cx.residue_indices == np.arange(1024) + 100 * cx.chain_labels).all()


def test_ragged_batch():
    coords, src, tokens, offsets = backbone.ragged_batch(16, 3)
    lens = np.diff(offsets)
    assert (lens >= 50).all() and (lens <= 500).all()
    assert coords.shape[0] == offsets[-1] and (tokens < 20).all()


@pytest.mark.parametrize("case", golden_cases(), ids=lambda c: c["fixture_id"])
def test_pdb_reader(case):
    bb, seq = structure.read_backbone(FIXTURES / case["pdb"])
    assert seq == case["native_sequence"] and bb.L == case["residue_count"]
    assert (bb.atom_sources != 0).all()


def _declared_functions():
    text = "".join(h.read_text() for h in sorted((ROOT / "include").glob("*.h")))
    return sorted(set(re.findall(r"\b(hkbs_\w+)\s*\(", text)))


def test_library_exports_header():
    lib = _lib.load()
    names = _declared_functions()
    assert set(names) == set(_lib.EXPORTS)
    for name in names:
        assert hasattr(lib, name), name
    assert "gfx950" in _lib.version()
    assert _lib.device_count() >= 0


def test_create_rejects_bad_package():
    lib = _lib.load()
    h = C.c_void_p()
    junk = np.zeros(64, np.uint8)
    assert lib.hkbs_pmpnn_create(junk.ctypes.data_as(C.c_void_p), 64, 0, C.byref(h)) == _lib.INVALID_ARGUMENT
    assert "safetensors" in lib.hkbs_last_error().decode()
    assert lib.hkbs_pmpnn_create(None, 0, 0, C.byref(h)) == _lib.INVALID_ARGUMENT
    blob = np.frombuffer(weights.read_package_bytes(), np.uint8)
    assert lib.hkbs_pmpnn_create(blob.ctypes.data_as(C.c_void_p), blob.size // 2, 0, C.byref(h)) == _lib.INVALID_ARGUMENT
    assert lib.hkbs_pmpnn_design(None, None, None, None, None, None, None, 1, 1, 0, None, None, None,
                                 C.c_float(0.1), 0, None, None, None, None) == _lib.INVALID_ARGUMENT


def test_host_decode_order_bit_exact(oracle):
    bb = backbone.single_chain(150, 4)
    src = bb.atom_sources.copy()
    src[[10, 20], 3] = 0
    mask = np.where((src[:, :4] != 0).all(1), 1.0, 0.0).astype(np.float32)
    cm = np.ones(150, np.float32)
    cm[40:60] = 0.0
    for seed in (0, 7, 123456789, 2**64 - 1):
        np.testing.assert_array_equal(_lib.decode_order(src, seed, cm),
                                      oracle.decode_order(150, seed, chain_mask=cm, residue_mask=mask))
