"""The float64 arbiter decoder (tests/exact_decoder.py), pinned before it is trusted.

- It equals the plain numpy float64 decoder of tests/bf16_error_model.py (the
  reference's [h_t, ctx] concatenation, one product per layer input) to float64
  reassociation, on a backbone with inactive residues, K < 48 and a random
  order: the restructured W1 product is an identity, not an approximation.
- At T = 1 it is within the fp32 tolerance of the oracle (the reference's
  fp32 arithmetic) on the same encoder output, tokens and order.
"""
import numpy as np

from hikoboshi_amd import backbone

from . import bf16_error_model as bm
from . import exact_decoder


def _case(L, seed):
    bb = backbone.single_chain(L, seed)
    src = bb.atom_sources.copy()
    src[[1, L // 2], 1] = 0  # inactive residues
    bb = backbone.Backbone(bb.coords, src)
    rng = np.random.default_rng(seed)
    return bb, rng.integers(0, 21, L).astype(np.int32), rng.permutation(L).astype(np.int32)


def test_arbiter_equals_the_numpy_model(oracle):
    for L in (30, 90):
        bb, tok, order = _case(L, 4)
        mask, idx, hv, he = oracle.encode(bb)
        K = idx.shape[1]
        ref = bm.log_softmax(bm.Model().decode(he.reshape(L * K, 128).astype(np.float64), hv.astype(np.float64), idx,
                                               mask.astype(np.float64), tok, order), 0.1)
        got = exact_decoder.log_probs((mask, idx, hv, he), tok, order, 0.1)
        assert np.abs(got - ref).max() <= 1e-9


def test_arbiter_matches_the_oracle_at_T1(oracle):
    bb, tok, order = _case(120, 8)
    enc = oracle.encode(bb)
    olp, _ = oracle.teacher_forced_decode(enc, tok, order)
    got = exact_decoder.log_probs(enc, tok, order, 1.0)
    active = enc[0] != 0
    assert np.abs(got[active] - olp[active]).max() <= 1e-4
