"""Entry-point glue on the CPU: output formats, backbone noise, recovery, package
and CLI handling, each pinned against the reference build where it has one."""
import io
import subprocess
import sys
import zipfile
from types import SimpleNamespace

import numpy as np
import pytest

from hikoboshi_amd import _lib, backbone, design_io
from hikoboshi_amd import inverse_fold as ifold
from hikoboshi_amd.exceptions import InvalidArgumentError

from .conftest import ROOT


def _records(rng, n, L):
    alphabet = "ACDEFGHIKLMNPQRSTVWYX"
    seqs = ["".join(rng.choice(list(alphabet), L)) for _ in range(n)]
    scores = [float(np.float32(v)) for v in rng.standard_normal(n) * 3]
    seeds = [int(v) for v in rng.integers(0, 2**63, n, dtype=np.int64)]
    return seqs, scores, seeds


FASTA_CASES = [
    (3, 80, 0.1, False), (2, 81, 0.0, True), (1, 1, 1.0, False), (4, 160, 0.123456789, False),
    (2, 300, 1e-5, True), (1, 0, 0.1, False), (2, 7, 2.5e6, False),
]


@pytest.mark.parametrize("n,L,T,n_to_c", FASTA_CASES)
def test_design_fasta_bytes_match_reference(reference, tmp_path, n, L, T, n_to_c):
    rng = np.random.default_rng(n * 1000 + L)
    seqs, scores, seeds = _records(rng, n, L)
    if L == 7:  # special values the stream formatting must render alike
        scores = [float("nan"), float("inf")][:n]
        seeds[-1] = 2**64 - 1
    ref = tmp_path / "ref.fasta"
    reference.write_design_outputs(str(ref), "", seqs, scores, seeds, n_to_c, T)
    order = "n_to_c" if n_to_c else "random"
    recs = [SimpleNamespace(sequence=s, score=sc, seed=sd, decode_order=order) for s, sc, sd in zip(seqs, scores, seeds)]
    ours = tmp_path / "ours.fasta"
    design_io.write_design_fasta(str(ours), recs, T)
    assert ours.read_bytes() == ref.read_bytes()


@pytest.mark.parametrize("n,L", [(1, 1), (3, 17), (2, 300), (5, 64)])
def test_logprobs_npz_bytes_match_reference(reference, tmp_path, n, L):
    rng = np.random.default_rng(L)
    values = (rng.standard_normal((n, L, 21)) * 4 - 3).astype(np.float32)
    seqs, scores, seeds = _records(rng, n, L)
    ref = tmp_path / "ref.npz"
    reference.write_design_outputs("", str(ref), seqs, scores, seeds, False, 0.1, values)
    ours = tmp_path / "ours.npz"
    design_io.write_inverse_fold_logprobs_npz(str(ours), values)
    assert ours.read_bytes() == ref.read_bytes()
    # and it is a valid archive numpy reads back
    with np.load(io.BytesIO(ours.read_bytes())) as z:
        np.testing.assert_array_equal(z["log_probs"], values)
    assert zipfile.ZipFile(ours).testzip() is None


def test_writer_errors(tmp_path):
    with pytest.raises(InvalidArgumentError, match="design FASTA output path is required"):
        design_io.write_design_fasta("", [], 0.1)
    with pytest.raises(InvalidArgumentError, match="shape is invalid"):
        design_io.write_inverse_fold_logprobs_npz(str(tmp_path / "x.npz"), np.zeros((0, 3, 21), np.float32))


@pytest.mark.parametrize("sigma,n_to_c", [(0.2, False), (1.0, True)])
def test_backbone_noise_matches_reference(reference, oracle, sigma, n_to_c):
    """The host noise helper reproduces the reference's per-sample noise: the
    reference's own per-sample loop with noise equals the oracle's module call
    (bit-exact with the reference's module) on our noised coordinates."""
    bb = backbone.single_chain(40, 3)
    src = bb.atom_sources.copy()
    src[5, 4] = 0  # a missing atom draws no noise
    bb = backbone.Backbone(bb.coords, src)
    seed, n = 11, 2
    ref = reference.algorithm_inverse_fold_ex(bb, n, seed, 0.1, n_to_c=n_to_c, backbone_noise=sigma)
    for i in range(n):
        noisy = backbone.Backbone(_lib.backbone_noise(bb.coords, bb.atom_sources, sigma, seed + i), bb.atom_sources)
        assert not np.array_equal(noisy.coords, bb.coords)
        np.testing.assert_array_equal(noisy.coords[5, 4], bb.coords[5, 4])
        kw = dict(input_order=np.arange(40, dtype=np.int32), use_input_order=True) if n_to_c else {}
        o = oracle.inverse_fold(noisy, seed=seed + i, order_seed=seed + i, temperature=0.1, **kw)
        np.testing.assert_array_equal(o["tokens"], ref["tokens"][i])
        np.testing.assert_array_equal(o["log_probs"], ref["log_probs"][i])
        assert np.float32(o["score"]) == np.float32(ref["scores"][i])


def test_backbone_noise_zero_sigma_and_errors():
    bb = backbone.single_chain(12, 1)
    out = _lib.backbone_noise(bb.coords, bb.atom_sources, 0.0, 7)
    np.testing.assert_array_equal(out, bb.coords)
    with pytest.raises(_lib.HkbsError):
        _lib.backbone_noise(bb.coords, bb.atom_sources, -1.0, 7)


def test_recovery_matches_reference(reference):
    bb = backbone.single_chain(30, 8)
    native = "ACDEFGHIKLMNPQRSTVWYXXacdefgBZ"  # lower case compares upper; X/B/Z are not standard
    ref = reference.algorithm_inverse_fold_ex(bb, 3, 2, 0.5, residue_codes=native)
    for i in range(3):
        seq = "".join(backbone.ALPHABET[t] for t in ref["tokens"][i])
        assert ifold.recovery_vs_native(seq, native) == pytest.approx(ref["recovery"][i], abs=0)
    none = reference.algorithm_inverse_fold_ex(bb, 1, 2, 0.5, residue_codes="X" * 30)
    assert none["recovery"] == [None] and ifold.recovery_vs_native("A" * 30, "X" * 30) is None


def test_package_and_order_resolution():
    for name in (None, "", "proteinmpnn", "PROTEINMPNN-V48-EPS020", "v_48_020", "Hikoboshi-ProteinMPNN-v48-020"):
        assert ifold.resolve_package(name) == "proteinmpnn-v48-eps020"
    with pytest.raises(InvalidArgumentError, match="does not use the aligner"):
        ifold.resolve_package("mpnn64")
    with pytest.raises(InvalidArgumentError, match="unknown Hikoboshi package id"):
        ifold.resolve_package("nope")
    assert ifold.parse_decode_order("n-to-c") == "n_to_c" and ifold.parse_decode_order(None) == "random"
    with pytest.raises(InvalidArgumentError, match="must be 'random' or 'n_to_c'"):
        ifold.parse_decode_order("c_to_n")


CLI_ERRORS = [
    (["design"], 2, "hikoboshi: invalid_argument: design requires --pdb"),
    (["design", "--pdb", "a.pdb"], 2, "hikoboshi: invalid_argument: design requires --out"),
    (["design", "--pdb"], 2, "hikoboshi: invalid_argument: option requires a value"),
    (["design", "--pdb=a", "--out=b", "--num-seqs", "0"], 2, "num-seqs must be a positive integer"),
    (["design", "--pdb=a", "--out=b", "--seed", "x1"], 2, "seed must be a non-negative integer"),
    (["design", "--pdb=a", "--out=b", "--sampling-temp", "0.1x"], 2, "sampling-temp must be a finite number"),
    (["design", "--pdb=a", "--out=b", "--decode-order", "c"], 2, "decode-order must be random or n_to_c"),
    (["design", "--pdb=a", "--out=b", "--gpu"], 2, "historical or reserved flag"),
    (["design", "--pdb=a", "--out=b", "--weights=w"], 2, "external package paths are not supported"),
    (["design", "--pdb=a", "--out=b", "--package", "esm2-8m"], 2, "does not use the aligner"),
    (["design", "--pdb=a", "--out=b", "--frobnicate"], 2, "unknown design option"),
    (["design", "stray", "--out=b"], 2, "design requires explicit --pdb and --out options"),
    (["design", "--pdb=/nonexistent.pdb", "--out=b"], 3, "hikoboshi: unavailable: structure file not readable"),
]


@pytest.mark.parametrize("argv,code,message", CLI_ERRORS, ids=[" ".join(c[0][1:]) or "empty" for c in CLI_ERRORS])
def test_cli_errors(argv, code, message):
    r = subprocess.run([sys.executable, "-m", "hikoboshi_amd", *argv], cwd=ROOT, capture_output=True, text=True,
                       timeout=60)
    assert r.returncode == code, r.stderr
    assert message in r.stderr


def test_cli_help():
    r = subprocess.run([sys.executable, "-m", "hikoboshi_amd", "design", "--help"], cwd=ROOT, capture_output=True,
                       text=True, timeout=60)
    assert r.returncode == 0 and r.stdout.startswith("usage: hikoboshi design --pdb INPUT.pdb --out OUT.fasta")
