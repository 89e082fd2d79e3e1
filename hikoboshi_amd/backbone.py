"""Synthetic protein backbones for the design workloads.

Backbones are built by NeRF (natural extension reference frame) from ideal
geometry, in float64, then stored as float32 ``[L, 5, 3]`` arrays in the
reference's canonical atom order N, CA, C, O, CB
(``cpp/include/hikoboshi/universal/structure.hpp:21-27``) with ``AtomSource``
codes Observed (1) for N/CA/C/O and Virtual (3) for CB
(``structure.hpp:33-38``), which is what the reference's structure loader
hands the design path.

Geometry: bond lengths N-CA 1.458, CA-C 1.525, C-N 1.329, C=O 1.231 A;
angles N-CA-C 111.2, CA-C-N 116.2, C-N-CA 121.7, CA-C-O 120.5 degrees;
omega 180; O in the peptide plane anti to N(i+1). phi/psi are drawn per
segment of 8-15 residues (uniform integer length), alternating helix
(-57, -47) and strand (-120, 130), each residue jittered by N(0, 10 degrees).
CB is the ProteinMPNN virtual CB computed in float32 in the reference's
operation order (``cpp/io/virtual_cb.cpp:16-39``).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

N_CA, CA_C, C_N, C_O = 1.458, 1.525, 1.329, 1.231
ANG_N_CA_C, ANG_CA_C_N, ANG_C_N_CA, ANG_CA_C_O = 111.2, 116.2, 121.7, 120.5
HELIX, STRAND = (-57.0, -47.0), (-120.0, 130.0)

OBSERVED, VIRTUAL, MISSING = 1, 3, 0
ALPHABET = "ACDEFGHIKLMNPQRSTVWYX"

#: UniProtKB/Swiss-Prot amino-acid composition (percent), alphabet order A..Y.
SWISSPROT_FREQ = {
    "A": 8.25, "C": 1.37, "D": 5.45, "E": 6.75, "F": 3.86, "G": 7.07, "H": 2.27,
    "I": 5.96, "K": 5.84, "L": 9.66, "M": 2.42, "N": 4.06, "P": 4.70, "Q": 3.93,
    "R": 5.53, "S": 6.56, "T": 5.34, "V": 6.87, "W": 1.08, "Y": 2.92,
}


@dataclass
class Backbone:
    coords: np.ndarray  # float32 [L, 5, 3]
    atom_sources: np.ndarray  # uint8 [L, 5]
    residue_indices: np.ndarray | None = None  # int32 [L]
    chain_labels: np.ndarray | None = None  # int32 [L]
    name: str = "synthetic"
    meta: dict = field(default_factory=dict)

    @property
    def L(self) -> int:
        return int(self.coords.shape[0])


def _norm3(v):
    """Euclidean norm over the last axis of [..., 3], summed x, y, z in order."""
    return np.sqrt((v[..., 0] * v[..., 0] + v[..., 1] * v[..., 1]) + v[..., 2] * v[..., 2])


def _cross3(a, b):
    return np.stack([a[..., 1] * b[..., 2] - a[..., 2] * b[..., 1],
                     a[..., 2] * b[..., 0] - a[..., 0] * b[..., 2],
                     a[..., 0] * b[..., 1] - a[..., 1] * b[..., 0]], axis=-1)


def _place(a, b, c, length, angle_deg, torsion_deg):
    """NeRF: position D with |CD| = length, angle BCD, torsion ABCD, for [n, 3] batches of points
    (torsion_deg a scalar or [n])."""
    ang = np.deg2rad(angle_deg)
    tor = np.deg2rad(torsion_deg)
    bc = c - b
    bc = bc / _norm3(bc)[:, None]
    n = _cross3(b - a, bc)
    n = n / _norm3(n)[:, None]
    m = _cross3(n, bc)
    d0 = -length * np.cos(ang)
    d1 = length * np.sin(ang) * np.cos(tor)
    d2 = length * np.sin(ang) * np.sin(tor)
    d1 = np.broadcast_to(d1, (a.shape[0],))[:, None]
    d2 = np.broadcast_to(d2, (a.shape[0],))[:, None]
    return c + ((bc * d0 + m * d1) + n * d2)


def virtual_cb(n: np.ndarray, ca: np.ndarray, c: np.ndarray) -> np.ndarray:
    """float32 virtual CB, same operation order as cpp/io/virtual_cb.cpp:23-39."""
    f = np.float32
    n, ca, c = n.astype(f), ca.astype(f), c.astype(f)
    b = ca - n
    cv = c - ca
    a = np.stack(
        [b[..., 1] * cv[..., 2] - b[..., 2] * cv[..., 1],
         b[..., 2] * cv[..., 0] - b[..., 0] * cv[..., 2],
         b[..., 0] * cv[..., 1] - b[..., 1] * cv[..., 0]],
        axis=-1,
    )
    return ((ca + f(-0.58273431) * a) + f(0.56802827) * b) + f(-0.54067466) * cv


def _phi_psi(L: int, rng: np.random.Generator) -> tuple[np.ndarray, np.ndarray]:
    """Per segment: its length, then (phi, psi) jitter pairs residue by residue."""
    phi = np.empty(L)
    psi = np.empty(L)
    pos, helix = 0, True
    while pos < L:
        seg = int(rng.integers(8, 16))
        base = HELIX if helix else STRAND
        end = min(L, pos + seg)
        z = rng.normal(0.0, 10.0, size=2 * (end - pos)).reshape(-1, 2)
        phi[pos:end] = base[0] + z[:, 0]
        psi[pos:end] = base[1] + z[:, 1]
        pos, helix = end, not helix
    return phi, psi


def _nerf(phi: np.ndarray, psi: np.ndarray) -> np.ndarray:
    """float64 [n, Lmax, 4, 3] N, CA, C, O of n chains built together residue by residue from
    [n, Lmax] torsions (a shorter chain ignores what lies beyond its own length)."""
    n, L = phi.shape
    xyz = np.zeros((n, L, 4, 3))
    t = np.deg2rad(180.0 - ANG_N_CA_C)
    xyz[:, 0, 1] = (N_CA, 0.0, 0.0)
    xyz[:, 0, 2] = xyz[:, 0, 1] + CA_C * np.array([np.cos(t), np.sin(t), 0.0])
    for i in range(L):
        N, CA, C = xyz[:, i, 0], xyz[:, i, 1], xyz[:, i, 2]
        n_next = _place(N, CA, C, C_N, ANG_CA_C_N, psi[:, i])
        xyz[:, i, 3] = _place(n_next, CA, C, C_O, ANG_CA_C_O, 180.0)
        if i + 1 < L:
            ca_next = _place(CA, C, n_next, N_CA, ANG_C_N_CA, 180.0)
            xyz[:, i + 1, 0] = n_next
            xyz[:, i + 1, 1] = ca_next
            xyz[:, i + 1, 2] = _place(C, n_next, ca_next, CA_C, ANG_N_CA_C, phi[:, i + 1])
    return xyz


def _chain_backbone(L: int, rng: np.random.Generator) -> np.ndarray:
    """float64 [L, 4, 3] N, CA, C, O."""
    phi, psi = _phi_psi(L, rng)
    return _nerf(phi[None], psi[None])[0]


def _assemble(bb4: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    L = bb4.shape[0]
    coords = np.zeros((L, 5, 3), dtype=np.float32)
    coords[:, :4] = bb4.astype(np.float32)
    coords[:, 4] = virtual_cb(coords[:, 0], coords[:, 1], coords[:, 2])
    src = np.full((L, 5), OBSERVED, dtype=np.uint8)
    src[:, 4] = VIRTUAL
    return coords, src


def single_chain(L: int, seed: int) -> Backbone:
    rng = np.random.default_rng(seed)
    bb = _chain_backbone(L, rng)
    bb -= bb[:, 1].mean(axis=0)
    coords, src = _assemble(bb)
    return Backbone(coords, src, name=f"nerf_L{L}_s{seed}", meta={"L": L, "seed": seed})


def tetrahedral_complex(chain_len: int, seed: int, n_chains: int = 4, edge: float = 25.0,
                        index_offset: int = 100) -> Backbone:
    """n_chains (<= 4) chains, centroids on a regular tetrahedron of the given edge."""
    rng = np.random.default_rng(seed)
    a = edge / (2.0 * np.sqrt(2.0))
    verts = np.array([[a, a, a], [a, -a, -a], [-a, a, -a], [-a, -a, a]])
    parts = []
    for c in range(n_chains):
        bb = _chain_backbone(chain_len, rng)
        bb -= bb[:, 1].mean(axis=0)
        parts.append(bb + verts[c])
    bb = np.concatenate(parts, axis=0)
    coords, src = _assemble(bb)
    L = bb.shape[0]
    chain = np.repeat(np.arange(n_chains, dtype=np.int32), chain_len)
    resid = (np.arange(L, dtype=np.int32) + index_offset * chain).astype(np.int32)
    return Backbone(coords, src, residue_indices=resid, chain_labels=chain,
                    name=f"tetra{n_chains}x{chain_len}_s{seed}",
                    meta={"chains": n_chains, "chain_len": chain_len, "seed": seed})


def native_tokens(L: int, rng: np.random.Generator) -> np.ndarray:
    aas = sorted(SWISSPROT_FREQ)
    p = np.array([SWISSPROT_FREQ[a] for a in aas])
    p /= p.sum()
    ids = np.array([ALPHABET.index(a) for a in aas], dtype=np.int32)
    return ids[rng.choice(len(aas), size=L, p=p)]


def ragged_batch(n: int, seed: int, lmin: int = 50, lmax: int = 500):
    """n backbones with L ~ U[lmin, lmax] and i.i.d. native tokens, packed ragged.

    Returns (coords [sum L,5,3], atom_sources [sum L,5], tokens [sum L], offsets int64 [n+1]).
    The random draws run protein by protein (lengths first, then per protein its torsions and
    tokens); the geometry of all proteins is built together.
    """
    rng = np.random.default_rng(seed)
    lens = rng.integers(lmin, lmax + 1, size=n)
    offsets = np.zeros(n + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(lens)
    Lmax = int(lens.max()) if n else 0
    phi = np.zeros((n, Lmax))
    psi = np.zeros((n, Lmax))
    tokens = np.empty(offsets[-1], dtype=np.int32)
    for i, L in enumerate(lens):
        phi[i, :L], psi[i, :L] = _phi_psi(int(L), rng)
        tokens[offsets[i]:offsets[i + 1]] = native_tokens(int(L), rng)
    coords = np.empty((offsets[-1], 5, 3), dtype=np.float32)
    src = np.empty((offsets[-1], 5), dtype=np.uint8)
    for b0 in range(0, n, 1024):  # bounded memory: [1024, Lmax, 4, 3] float64 per block
        xyz = _nerf(phi[b0:b0 + 1024], psi[b0:b0 + 1024])
        for i in range(b0, min(n, b0 + 1024)):
            bb = xyz[i - b0, :lens[i]].copy()
            bb -= bb[:, 1].mean(axis=0)
            sl = slice(offsets[i], offsets[i + 1])
            coords[sl], src[sl] = _assemble(bb)
    return coords, src, tokens, offsets


#: Design workloads (sizes as the benchmark configurations state them).
WORKLOADS = {
    "design_L120_B8": dict(L=120, B=8, temperature=0.1, seed=7, order="random_per_seq"),
    "design_L300_B64": dict(L=300, B=64, temperature=0.1, seed=7, order="shared_random"),
    "complex_4x256_B256": dict(L=1024, B=256, temperature=0.2, seed=7, order="shared_random"),
    "design_L4000_B32_bf16x3": dict(L=4000, B=32, temperature=0.1, seed=7, order="shared_random",
                                    precision="bf16x3"),
    "design_L4000_B32_bf16": dict(L=4000, B=32, temperature=0.1, seed=7, order="shared_random", precision="bf16"),
}


def sequence_to_tokens(seq: str) -> np.ndarray:
    """One-letter codes -> ProteinMPNN token ids (anything outside the 20 standard letters -> 20, X)."""
    return np.array([ALPHABET.index(c) if c in ALPHABET[:20] else 20 for c in seq], dtype=np.int32)
