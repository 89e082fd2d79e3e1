"""GPU parity at the benchmark configurations' own shapes, through the C ABI.

- 4 x 256 tetrahedral complex, 256 sequences, T = 0.2, one shared random order,
  chain labels and residue offsets of +100 per chain (the module-level call of
  cpp/modules/mpnn/inverse_fold_scalar.cpp:954-1000 with an input decoding
  order; cross-chain edges take the chain-break class of
  cpp/modules/mpnn/edge_rbf_features_scalar.cpp:55-70).
- one 4,000-residue chain, T = 0.1: fp32 against the oracle (1e-4), and the
  split bf16 mode against the fp32 path at the contract's 2e-2 (plain bf16
  misses it: a strict xfail).
- teacher-forced scoring of the full 4,096-protein ragged batch
  (cpp/modules/mpnn/inverse_fold_scalar.cpp:575-663, 905-952), across the
  edge-bounded chunks of hkbs_pmpnn_score_batch.

Each oracle backbone is encoded once per test; forced replay re-runs the GPU's
token trajectory through the oracle (see test_gpu_parity.replay).
"""
import numpy as np
import pytest

from hikoboshi_amd import _lib, backbone

from .test_gpu_parity import LP_TOL, _fp32_on_trajectory, replay_many

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _logsumexp_rows(lp):
    x = lp.astype(np.float64)
    m = x.max(-1, keepdims=True)
    return (m + np.log(np.exp(x - m).sum(-1, keepdims=True)))[..., 0]


def _design_properties(res, L, B):
    """Invariants every design row must satisfy: tokens in the vocabulary, each log-prob row a
    normalised distribution, finite scores equal to the mean NLL of the written tokens."""
    tok, lp, sc = res["tokens"], res["log_probs"], res["scores"]
    assert tok.shape == (B, L) and lp.shape == (B, L, 21)
    assert ((tok >= 0) & (tok < 21)).all()
    assert np.isfinite(lp).all() and np.isfinite(sc).all()
    assert (lp <= 1e-6).all()
    assert np.abs(_logsumexp_rows(lp)).max() <= 2e-5
    nll = -np.take_along_axis(lp, tok[..., None], axis=-1)[..., 0].astype(np.float64).mean(1)
    np.testing.assert_allclose(sc, nll, atol=2e-5, rtol=1e-6)


def test_design_complex_4x256_b256(gpu_ctx, oracle):
    cx = backbone.tetrahedral_complex(256, 7)
    L, B, T = cx.L, 256, 0.2
    order = _lib.decode_order(cx.atom_sources, 7)
    np.testing.assert_array_equal(order, oracle.decode_order(L, 7, residue_mask=np.ones(L, np.float32)))
    seeds = (7 + np.arange(B)).astype(np.uint64)
    _say(f"design complex 4x256 L={L} B={B} T={T}")
    res = gpu_ctx.design(cx.coords, cx.atom_sources, B, seeds, order_mode=_lib.ORDER_INPUT_SHARED, orders=order,
                         temperature=T, residue_indices=cx.residue_indices, chain_labels=cx.chain_labels)
    assert (res["orders"] == order).all()
    _design_properties(res, L, B)
    _say("  oracle encode")
    enc = oracle.encode(cx)
    idx = enc[1]
    assert idx.shape == (L, 48)
    assert (cx.chain_labels[idx] != cx.chain_labels[:, None]).any(), "no cross-chain kNN edges"
    # every sequence; positions above the bar are arbitrated by the float64 decoder
    assert replay_many(oracle, enc, order, seeds, T, res, list(range(B)), arbitrate=True, bb=cx) <= LP_TOL


@pytest.fixture(scope="module")
def long_chain():
    bb = backbone.single_chain(4000, 21)
    return bb, _lib.decode_order(bb.atom_sources, 21)


def test_design_long_chain_fp32(gpu_ctx, oracle, long_chain):
    """The long-chain configuration's shape in fp32 (L = 4,000, 32 sequences, T = 0.1): forced replay of
    four sequences, the first and the last among them."""
    bb, order = long_chain
    L, B, T = bb.L, 32, 0.1
    seeds = (5 + np.arange(B)).astype(np.uint64)
    _say(f"design fp32 L={L} B={B} T={T}")
    res = gpu_ctx.design(bb.coords, bb.atom_sources, B, seeds, order_mode=_lib.ORDER_INPUT_SHARED, orders=order,
                         temperature=T)
    _design_properties(res, L, B)
    _say("  oracle encode L=4000")
    enc = oracle.encode(bb)
    assert replay_many(oracle, enc, order, seeds, T, res, [0, 1, 16, B - 1], arbitrate=True, bb=bb) <= LP_TOL


BF16_TOL = 2e-2  # bf16 per-position log-probs against the fp32 path of the same inputs


def _bf16_deviation(gpu_ctx, bb, order, B, T, precision=_lib.PRECISION_BF16):
    seeds = (5 + np.arange(B)).astype(np.uint64)
    gpu_ctx.set_precision(precision)
    try:
        res = gpu_ctx.design(bb.coords, bb.atom_sources, B, seeds, order_mode=_lib.ORDER_INPUT_SHARED,
                             orders=order, temperature=T)
    finally:
        gpu_ctx.set_precision(_lib.PRECISION_FP32)
    _design_properties(res, bb.L, B)
    worst = 0.0
    for b in range(B):
        ref = _fp32_on_trajectory(gpu_ctx, bb, res["tokens"][b], order, T)
        worst = max(worst, float(np.abs(res["log_probs"][b] - ref).max()))
    return worst


@pytest.mark.xfail(strict=True, reason="bf16 operands carry 8 significant bits: rounding any single product's "
                                       "weights or inputs to bf16 moves T = 0.1 log-probs by 0.05-0.23 "
                                       "(tests/bf16_error_model.py); the GPU's bf16 decode measured 0.2-0.4")
def test_design_long_chain_bf16_contract(gpu_ctx, long_chain):
    """The contract as written: L = 4,000, 32 sequences, T = 0.1, bf16 log-probs within 2e-2 of the fp32
    path on the same trajectory (the fp32 teacher-forced log-probs of the bf16 run's tokens and order)."""
    bb, order = long_chain
    _say("design bf16 L=4000 B=32 T=0.1 (contract)")
    worst = _bf16_deviation(gpu_ctx, bb, order, 32, 0.1)
    _say(f"  bf16 vs fp32 max|dlogp|={worst:.3g} at T=0.1")
    assert worst <= BF16_TOL


def test_design_long_chain_split_bf16_contract(gpu_ctx, long_chain):
    """The contract in the split bf16 mode (HKBS_PRECISION_BF16X3: every decoder product on the bf16
    MFMA with both operands as two bf16 terms, fp32 accumulation and softmax): L = 4,000, 32
    sequences, T = 0.1, log-probs within 2e-2 of the fp32 path on the same trajectory."""
    bb, order = long_chain
    _say("design split bf16 L=4000 B=32 T=0.1 (contract)")
    worst = _bf16_deviation(gpu_ctx, bb, order, 32, 0.1, _lib.PRECISION_BF16X3)
    _say(f"  split bf16 vs fp32 max|dlogp|={worst:.3g} at T=0.1")
    assert worst <= BF16_TOL


def _chunk_ids(offsets, max_edges=4 << 20):
    """The chunking rule of hkbs_pmpnn_score_batch: consecutive proteins with the same K = min(48, L),
    at most max_edges edge slots per chunk (a single protein always forms a chunk)."""
    n = len(offsets) - 1
    lens = np.diff(offsets)
    ks = np.minimum(48, lens)
    ids = np.empty(n, np.int64)
    c, i = 0, 0
    while i < n:
        j = i + 1
        while j < n and ks[j] == ks[i] and (offsets[j + 1] - offsets[i]) * ks[i] <= max_edges:
            j += 1
        ids[i:j] = c
        c += 1
        i = j
    return ids


def _check_scores(lp, scores, tok, off):
    assert np.isfinite(lp).all() and np.isfinite(scores).all()
    assert np.abs(_logsumexp_rows(lp)).max() <= 2e-5
    picked = lp[np.arange(len(tok)), tok].astype(np.float64)
    nll = -np.add.reduceat(picked, off[:-1]) / np.diff(off)
    np.testing.assert_allclose(scores, nll, atol=2e-5, rtol=1e-6)


def test_score_batch_full_4096(gpu_ctx, oracle):
    coords, src, tok, off = backbone.ragged_batch(4096, 7)
    _say(f"score ragged batch of 4096 proteins, {int(off[-1])} residues")
    lp, scores = gpu_ctx.score_batch(coords, src, tok, off)
    _check_scores(lp, scores, tok, off)
    chunk = _chunk_ids(off)
    assert chunk.max() >= 2, "the batch should span several chunks"
    lens = np.diff(off)
    first_of = [int(np.argmax(chunk == c)) for c in range(int(chunk.max()) + 1)]
    pick = {int(np.argmax(lens)), 0, 4095, first_of[1] - 1, first_of[1], first_of[2], first_of[-1], 2049}
    worst = 0.0
    for i in sorted(pick):
        sl = slice(off[i], off[i + 1])
        olp, oscore = oracle.teacher_forced(backbone.Backbone(coords[sl], src[sl]), tok[sl])
        d = float(np.abs(lp[sl] - olp).max())
        _say(f"  protein {i} (chunk {chunk[i]}, L={lens[i]}): max|dlogp|={d:.3g}")
        assert scores[i] == pytest.approx(oscore, abs=2e-5)
        worst = max(worst, d)
    assert worst <= LP_TOL


def test_score_batch_chunking_is_exact(gpu_ctx, monkeypatch):
    """Proteins scored in several small chunks give the bits of one chunk (including a K < 48 protein
    between two K = 48 runs, which starts a chunk of its own)."""
    coords, src, tok, off = backbone.ragged_batch(6, 13, lmin=50, lmax=200)
    small = backbone.single_chain(30, 4)
    cut = int(off[3])
    coords = np.concatenate([coords[:cut], small.coords, coords[cut:]])
    src = np.concatenate([src[:cut], small.atom_sources, src[cut:]])
    tok = np.concatenate([tok[:cut], np.arange(30, dtype=np.int32) % 20, tok[cut:]])
    lens = np.insert(np.diff(off), 3, 30)
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    one_lp, one_sc = gpu_ctx.score_batch(coords, src, tok, off)
    limit = 2 * 48 * 120
    monkeypatch.setenv("HKBS_SCORE_CHUNK_EDGES", str(limit))
    assert _chunk_ids(off, limit).max() >= 3
    _say(f"score ragged batch {lens.tolist()} in chunks of <= {limit} edges")
    lp, sc = gpu_ctx.score_batch(coords, src, tok, off)
    np.testing.assert_array_equal(lp, one_lp)
    np.testing.assert_array_equal(sc, one_sc)
