"""The C++ drop-in at the reference's algorithm layer (hikoboshi_amd/dropin/),
compiled against the reference's own headers by oracle/dropin.mk, against the
reference's per-sample loop inverse_fold_proteinmpnn_v48_020
(cpp/algorithms/inverse_fold.cpp:221-356, built by oracle/ref.mk) on the same
InverseFoldRequest: sequences identical except near-tie positions (forced
replay through the oracle), log-probs within 1e-4, scores, seeds, decode order
and recovery against the native sequence; the validation statuses and
messages of the reference.
"""
import ctypes as C

import numpy as np
import pytest

from hikoboshi_amd import _lib, backbone, structure, weights

from .conftest import FIXTURES, ROOT, golden_cases
from .test_gpu_parity import CDF_TOL, LP_TOL

pytestmark = pytest.mark.gpu

DROPIN_SO = ROOT / "oracle" / "_ref" / "libhkbs_dropin.so"


def _say(msg):
    print(msg, flush=True)


class DropIn:
    def __init__(self, path):
        lib = C.CDLL(str(path))
        lib.dropin_open.argtypes = [C.c_void_p, C.c_size_t, C.c_int, C.POINTER(C.c_void_p), C.POINTER(C.c_char_p)]
        lib.dropin_close.argtypes = [C.c_void_p]
        lib.dropin_inverse_fold.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_char_p, C.c_size_t, C.c_size_t,
                                            C.c_ulonglong, C.c_float, C.c_int, C.c_float, C.c_int, C.c_int,
                                            C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                            C.c_void_p, C.POINTER(C.c_size_t), C.POINTER(C.c_char_p)]
        self.lib = lib
        pkg = np.frombuffer(weights.read_package_bytes(), np.uint8)
        self.h, detail = C.c_void_p(), C.c_char_p()
        st = lib.dropin_open(pkg.ctypes.data, pkg.size, 0, C.byref(self.h), C.byref(detail))
        assert st == 0, detail.value

    def close(self):
        self.lib.dropin_close(self.h)

    def inverse_fold(self, bb, codes, num_seqs, seed, temperature, n_to_c=False, noise=0.0, keep=True,
                     with_weights=True):
        L = bb.L
        c = np.ascontiguousarray(bb.coords, np.float32)
        s = np.ascontiguousarray(bb.atom_sources, np.uint8)
        n = max(num_seqs, 1)
        seqs = C.create_string_buffer(n * L)
        scores, rec = np.zeros(n), np.zeros(n)
        rec_ok, orders = np.zeros(n, np.int32), np.zeros(n, np.int32)
        seeds = np.zeros(n, np.uint64)
        lp = np.zeros((n, L, 21), np.float32)
        count, detail = C.c_size_t(), C.c_char_p()
        st = self.lib.dropin_inverse_fold(self.h, c.ctypes.data, s.ctypes.data, codes.encode() if codes else None, L,
                                          num_seqs, seed, temperature, int(n_to_c), noise, int(keep),
                                          int(with_weights), seqs, scores.ctypes.data, rec.ctypes.data,
                                          rec_ok.ctypes.data, seeds.ctypes.data, orders.ctypes.data, lp.ctypes.data,
                                          C.byref(count), C.byref(detail))
        if st != 0:
            return st, detail.value.decode()
        letters = seqs.raw[:num_seqs * L].decode()
        return dict(sequences=[letters[i * L:(i + 1) * L] for i in range(num_seqs)], scores=scores[:num_seqs],
                    recovery=[float(r) if ok else None for r, ok in zip(rec[:num_seqs], rec_ok[:num_seqs])],
                    seeds=seeds[:num_seqs], orders=orders[:num_seqs], log_probs=lp[:num_seqs],
                    lp_count=count.value)


@pytest.fixture(scope="module")
def dropin():
    if not DROPIN_SO.exists():
        pytest.skip("oracle/_ref/libhkbs_dropin.so not built (needs the reference headers)")
    d = DropIn(DROPIN_SO)
    yield d
    d.close()


CASES = [("random_T0.1", dict(num_seqs=3, seed=5, temperature=0.1)),
         ("n_to_c_greedy", dict(num_seqs=2, seed=9, temperature=0.0, n_to_c=True)),
         ("noise_T0.2", dict(num_seqs=2, seed=13, temperature=0.2, noise=0.3))]


@pytest.mark.parametrize("name,kw", CASES, ids=[c[0] for c in CASES])
def test_dropin_matches_reference_algorithm(dropin, reference, oracle, name, kw):
    case = golden_cases()[1]
    bb, native = structure.read_backbone(FIXTURES / case["pdb"])
    _say(f"drop-in {name} on {case['fixture_id']} L={bb.L}")
    got = dropin.inverse_fold(bb, native, **kw)
    ref = reference.algorithm_inverse_fold_ex(bb, kw["num_seqs"], kw["seed"], kw["temperature"],
                                              n_to_c=kw.get("n_to_c", False), backbone_noise=kw.get("noise", 0.0),
                                              residue_codes=native)
    B = kw["num_seqs"]
    np.testing.assert_array_equal(got["seeds"], kw["seed"] + np.arange(B, dtype=np.uint64))
    assert (got["orders"] == int(kw.get("n_to_c", False))).all()
    assert got["lp_count"] == B * bb.L * 21
    worst = 0.0
    for i in range(B):
        seed = kw["seed"] + i
        tokens = np.array([backbone.ALPHABET.index(ch) for ch in got["sequences"][i]], np.int32)
        ref_tokens = ref["tokens"][i]
        # forced replay of the drop-in's sequence through the oracle on the sample's own backbone
        sb = bb if not kw.get("noise") else backbone.Backbone(
            _lib.backbone_noise(bb.coords, bb.atom_sources, kw["noise"], seed), bb.atom_sources)
        order = np.arange(bb.L, dtype=np.int32) if kw.get("n_to_c") else _lib.decode_order(bb.atom_sources, seed)
        rep = oracle.decode(oracle.encode(sb), order, seed, kw["temperature"], greedy=kw["temperature"] <= 0.0,
                            forced_tokens=tokens)
        flips = np.nonzero(rep["sampled"] != tokens)[0]
        assert all(rep["cdf_gap"][r] < CDF_TOL for r in flips), f"sample {i}: token differs with a clear margin"
        d = float(np.abs(rep["log_probs"] - got["log_probs"][i]).max())
        worst = max(worst, d)
        if np.array_equal(tokens, ref_tokens):
            worst = max(worst, float(np.abs(ref["log_probs"][i] - got["log_probs"][i]).max()))
            assert got["scores"][i] == pytest.approx(ref["scores"][i], abs=5e-5)
            assert got["recovery"][i] == ref["recovery"][i]
        else:
            assert len(flips) > 0, f"sample {i}: sequence differs from the reference without a near tie"
    _say(f"  max|dlogp|={worst:.3g}")
    assert worst <= LP_TOL


def test_dropin_validation_matches_reference(dropin):
    """Statuses and messages of cpp/algorithms/inverse_fold.cpp:232-261."""
    bb = backbone.single_chain(20, 1)
    assert dropin.inverse_fold(bb, None, 0, 1, 0.1) == (_lib.INVALID_ARGUMENT,
                                                       "inverse-fold num_seqs must be greater than zero")
    assert dropin.inverse_fold(bb, None, 1, 1, float("nan")) == (_lib.INVALID_ARGUMENT,
                                                                "inverse-fold sampling_temp must be finite and >= 0")
    assert dropin.inverse_fold(bb, None, 1, 1, 0.1, noise=-1.0) == (
        _lib.INVALID_ARGUMENT, "inverse-fold backbone_noise must be finite and >= 0")
    assert dropin.inverse_fold(bb, None, 1, 1, 0.1, with_weights=False) == (
        _lib.FAILED_PRECONDITION, "ProteinMPNN inverse-folding weights are not available")
    res = dropin.inverse_fold(bb, None, 1, 1, 0.1, keep=False)
    assert res["lp_count"] == 0 and res["recovery"] == [None]
