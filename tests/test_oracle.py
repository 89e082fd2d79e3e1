"""Pins the CPU oracle (oracle/pmpnn_oracle.c) before it is trusted as a checker.

Each oracle function is checked against something that does not restate its
own formula: the reference's committed PyTorch goldens, the reference's own
sources compiled by oracle/ref.mk (bit-exact), known-answer cases from the
reference's unit tests, closed forms and brute force.
"""
import math

import numpy as np
import pytest

from hikoboshi_amd import backbone, structure
from hikoboshi_amd.backbone import ALPHABET

from .conftest import FIXTURES, golden_cases


# ---------------------------------------------------------------- numerics --

def test_fast_exp_neg_matches_exp(oracle):
    # tests/parity/fast_exp_neg_parity_test.cpp:12-15: [-20, 1], 5e-5, x > 0 clamps to 1.
    xs = np.linspace(-20.0, 1.0, 10000, dtype=np.float32)
    worst = 0.0
    for x in xs:
        got = oracle.fast_exp_neg(float(x))
        want = 1.0 if x > 0 else math.exp(float(x))
        worst = max(worst, abs(got - want))
    assert worst <= 5e-5
    assert math.isnan(oracle.fast_exp_neg(float("nan")))
    assert oracle.fast_exp_neg(-16.5) == 0.0
    assert oracle.fast_exp_neg(0.0) == 1.0


def test_gelu_matches_erf_gelu(oracle):
    # A&S 7.1.26 (|erf error| <= 1.5e-7) with the table exp: GELU within 2e-5 |x| of the exact form.
    for x in np.linspace(-8, 8, 4001):
        want = 0.5 * x * (1.0 + math.erf(x / math.sqrt(2.0)))
        got = oracle.gelu(float(x))
        assert abs(got - want) <= 2e-5 * max(1.0, abs(x)), x
    assert oracle.gelu(0.0) == 0.0
    assert oracle.gelu(10.0) == pytest.approx(10.0)
    assert oracle.gelu(-10.0) == 0.0


# --------------------------------------------------------------------- kNN --

def brute_knn(ca, valid, K):
    """(d, index) lexicographic top-K with the reference's d and masking rules."""
    L = ca.shape[0]
    f = np.float32
    idx = np.full((L, K), -1, np.int32)
    d2 = np.zeros((L, K), np.float32)
    for q in range(L):
        d = np.empty(L, np.float32)
        for t in range(L):
            dx, dy, dz = (f(ca[q, a]) - f(ca[t, a]) for a in range(3))
            d[t] = f(f(f(f(dx * dx) + f(dy * dy)) + f(dz * dz)) + f(1e-6))
        row_max = f(1e-6)
        if valid[q]:
            for t in range(L):
                if valid[t] and d[t] > row_max:
                    row_max = d[t]
        dd = np.where(valid[q] & valid, d, row_max).astype(np.float32)
        cand = [(dd[t], t) for t in range(L) if np.isfinite(dd[t])]
        cand.sort()
        for s, (dv, t) in enumerate(cand[:K]):
            idx[q, s] = t
            d2[q, s] = dv
        for s in range(len(cand), K):
            d2[q, s] = row_max
    return idx, d2


def test_knn_tie_by_index_known_answer(oracle):
    # tests/cpp/primitive_compute_goldens.cpp:26-58: equidistant candidates keep the
    # earliest indices. Here the query is appended as index 5 (same-buffer kNN).
    ca = np.array([[1, 0, 0], [0, 1, 0], [-1, 0, 0], [0, -1, 0], [0, 0, 1], [0, 0, 0]], np.float32)
    idx, d2 = oracle.knn(ca, np.ones(6, np.uint8), 4)
    assert list(idx[5]) == [5, 0, 1, 2]
    assert d2[5, 0] == np.float32(1e-6)
    np.testing.assert_allclose(d2[5, 1:], 1.0, atol=1e-5)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_knn_brute_force(oracle, seed):
    rng = np.random.default_rng(seed)
    L = 70
    ca = rng.integers(-4, 5, size=(L, 3)).astype(np.float32)  # integer grid -> many exact ties
    valid = (rng.random(L) > 0.15).astype(np.uint8)
    K = 48
    idx, d2 = oracle.knn(ca, valid, K)
    bidx, bd2 = brute_knn(ca, valid.astype(bool), K)
    np.testing.assert_array_equal(idx, bidx)
    np.testing.assert_array_equal(d2, bd2)


def test_knn_bit_exact_vs_reference(oracle, reference):
    bb = backbone.single_chain(300, 11)
    ca = bb.coords[:, 1]
    valid = np.ones(300, np.uint8)
    valid[[3, 77]] = 0
    a = oracle.knn(ca, valid, 48)
    b = reference.knn(ca, valid, 48)
    np.testing.assert_array_equal(a[0], b[0])
    np.testing.assert_array_equal(a[1], b[1])


# ------------------------------------------------------------- whole model --

@pytest.mark.parametrize("case", golden_cases(), ids=lambda c: c["fixture_id"])
def test_teacher_forced_matches_pytorch_goldens(oracle, case):
    # tests/parity/proteinmpnn_v48_020/recovery_parity.py:78-176: log-probs within 1e-4,
    # teacher argmax sequence exact.
    bb, seq = structure.read_backbone(FIXTURES / case["pdb"])
    assert seq == case["native_sequence"]
    lp, score = oracle.teacher_forced(bb, backbone.sequence_to_tokens(seq))
    gold = np.asarray(case["teacher_log_probs"], np.float32).reshape(case["teacher_log_probs_shape"])
    assert np.abs(lp - gold).max() <= 1e-4
    argmax = "".join(ALPHABET[i] for i in lp.argmax(1))
    assert argmax == case["teacher_argmax_sequence"]
    assert score == pytest.approx(case["teacher_score"], abs=1e-4)


@pytest.mark.parametrize("case", golden_cases(), ids=lambda c: c["fixture_id"])
def test_teacher_forced_bit_exact_vs_reference(oracle, reference, case):
    bb, seq = structure.read_backbone(FIXTURES / case["pdb"])
    tok = backbone.sequence_to_tokens(seq)
    a = oracle.teacher_forced(bb, tok)
    b = reference.teacher_forced(bb, tok)
    np.testing.assert_array_equal(a[0], b[0])
    assert a[1] == b[1]


def _variants():
    bb = backbone.single_chain(40, 3)
    out = [("single", bb, {})]
    cm = np.ones(40, np.float32)
    cm[:10] = 0
    tt = np.arange(40, dtype=np.int32) % 20
    out.append(("chain_mask", bb, dict(chain_mask=cm, true_tokens=tt)))
    src = bb.atom_sources.copy()
    src[5, 3] = 0  # residue 5 loses O -> inactive
    src[9, 4] = 0  # residue 9 loses CB -> active, CB pairs zeroed
    out.append(("missing_atoms", backbone.Backbone(bb.coords, src), dict(true_tokens=tt)))
    cx = backbone.tetrahedral_complex(12, 5, n_chains=3)
    out.append(("multichain", cx, {}))
    out.append(("short_L7", backbone.single_chain(7, 9), {}))
    return out


@pytest.mark.parametrize("name,bb,kw", _variants(), ids=lambda v: v if isinstance(v, str) else "")
@pytest.mark.parametrize("mode", ["random", "n_to_c", "greedy"])
def test_design_bit_exact_vs_reference(oracle, reference, name, bb, kw, mode):
    use_input = mode == "n_to_c"
    temp = 0.0 if mode == "greedy" else 0.2
    args = dict(seed=123, order_seed=123, temperature=temp, greedy=mode == "greedy",
                use_input_order=use_input, input_order=None, **kw)
    a = oracle.inverse_fold(bb, **args)
    b = reference.inverse_fold(bb, **args)
    for k in ("tokens", "log_probs", "order"):
        np.testing.assert_array_equal(a[k], b[k], err_msg=k)
    assert a["score"] == b["score"]


def _k_below_l_cases():
    """Backbones longer than 48 residues, where K = 48 < L (cpp/modules/mpnn/inverse_fold_scalar.cpp:892-896):
    every kNN row is a strict subset of the chain, so a K/L mix-up changes the graph."""
    bb = backbone.single_chain(300, 6)
    src = bb.atom_sources.copy()
    src[[11, 150], 3] = 0  # inactive residues
    src[70, 4] = 0  # missing CB
    return [("L120", backbone.single_chain(120, 4)), ("L300_masked", backbone.Backbone(bb.coords, src)),
            ("complex4x64", backbone.tetrahedral_complex(64, 2))]


@pytest.mark.parametrize("name,bb", _k_below_l_cases(), ids=lambda v: v if isinstance(v, str) else "")
@pytest.mark.parametrize("mode", ["random", "n_to_c"])
def test_design_bit_exact_vs_reference_k_below_l(oracle, reference, name, bb, mode):
    kw = dict(seed=41, order_seed=41, temperature=0.1, use_input_order=mode == "n_to_c")
    if name == "L300_masked":
        cm = np.ones(bb.L, np.float32)
        cm[200:230] = 0
        kw.update(chain_mask=cm, true_tokens=(np.arange(bb.L) * 7 % 20).astype(np.int32))
    a = oracle.inverse_fold(bb, **kw)
    b = reference.inverse_fold(bb, **kw)
    assert oracle.encode(bb)[1].shape == (bb.L, 48) and bb.L > 48
    for k in ("tokens", "log_probs", "order"):
        np.testing.assert_array_equal(a[k], b[k], err_msg=k)
    assert a["score"] == b["score"]


@pytest.mark.parametrize("name,bb", _k_below_l_cases(), ids=lambda v: v if isinstance(v, str) else "")
def test_teacher_forced_bit_exact_vs_reference_k_below_l(oracle, reference, name, bb):
    """Teacher forcing with a random input order and a chain mask, K = 48 < L."""
    rng = np.random.default_rng(5)
    tok = rng.integers(0, 21, bb.L).astype(np.int32)
    order = rng.permutation(bb.L).astype(np.int32)
    cm = np.ones(bb.L, np.float32)
    cm[bb.L // 3:bb.L // 2] = 0
    a = oracle.teacher_forced(bb, tok, input_order=order, chain_mask=cm)
    b = reference.teacher_forced(bb, tok, input_order=order, chain_mask=cm)
    np.testing.assert_array_equal(a[0], b[0])
    assert a[1] == b[1]


def test_algorithm_loop_bit_exact_vs_reference(oracle, reference):
    bb = backbone.single_chain(30, 7)
    a = oracle.algorithm_inverse_fold(bb, 3, 7, 0.1)
    b = reference.algorithm_inverse_fold(bb, 3, 7, 0.1)
    np.testing.assert_array_equal(a["tokens"], b["tokens"])
    np.testing.assert_array_equal(a["log_probs"], b["log_probs"])
    np.testing.assert_array_equal(a["scores"], b["scores"])


# ------------------------------------------------- decode order + sampler --

def test_decode_order_invariants(oracle):
    L = 200
    order = oracle.decode_order(L, seed=99)
    assert sorted(order.tolist()) == list(range(L))
    cm = np.ones(L, np.float32)
    cm[50:60] = 0
    order2 = oracle.decode_order(L, seed=99, chain_mask=cm)
    # fixed positions (score x 1e-4) come first
    assert set(order2[:10].tolist()) == set(range(50, 60))
    with pytest.raises(ValueError):
        oracle.decode_order(3, 0, input_order=np.array([0, 0, 1]), use_input=True)


def test_decode_order_matches_reference_orders(oracle, reference):
    bb = backbone.single_chain(64, 1)
    for seed in (0, 1, 2**63 + 5):
        r = reference.inverse_fold(bb, seed=seed, order_seed=seed, temperature=0.1)
        mask = np.ones(64, np.float32)
        np.testing.assert_array_equal(oracle.decode_order(64, seed, residue_mask=mask), r["order"])


def test_sampler_invariants(oracle):
    bb = backbone.single_chain(30, 2)
    enc = oracle.encode(bb)
    order = np.arange(30, dtype=np.int32)
    out = oracle.decode(enc, order, seed=5, temperature=0.3)
    lp = out["log_probs"].astype(np.float64)
    np.testing.assert_allclose(np.exp(lp).sum(1), 1.0, atol=1e-5)
    assert (lp <= 1e-7).all()
    g = oracle.decode(enc, order, seed=5, temperature=0.0, greedy=True)
    np.testing.assert_array_equal(g["tokens"], g["log_probs"].argmax(1))
    # forced replay of its own tokens reproduces the run
    rep = oracle.decode(enc, order, seed=5, temperature=0.3, forced_tokens=out["tokens"])
    np.testing.assert_array_equal(rep["log_probs"], out["log_probs"])
    np.testing.assert_array_equal(rep["sampled"], out["tokens"])
