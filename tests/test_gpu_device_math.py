"""Exhaustive GPU check of the device GELUs (tests/csrc/device_math_check.hip).

The encoder's gelu is evaluated without branches and with a reciprocal plus
one Newton step in place of IEEE division; gelu_fast drops the v > 4 select
and copies the sign. Both must equal their straightforward forms (the
reference expression of cpp/include/hikoboshi/primitives/compute/gelu.hpp:22-51
with fast_exp_neg.hpp:12-55, and the select form) bit for bit for every one of
the 2^32 float inputs; the encoder tests then pin the straightforward form
against the oracle. The decode loop's gelu_poly takes the A&S term from
per-segment polynomials: on every finite input it must stay within
POLY_UNITS units of ulp(gelu(x)) + |x| 2^-25 of gelu (the bit-exact reference
form), and agree bit for bit on infinities and NaNs. The encoder's sums with the products
on the matrix cores (seq_gemm_mfma) must equal the same sums on the VALU bit
for bit.
"""
import ctypes as C
import struct
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

LIB = Path(__file__).resolve().parent / "libdevice_math_check.so"
POLY_UNITS = 6.0  # measured 5.08 (gelu_fast, the form it replaced: 7.55)


def test_device_gelu_all_inputs():
    if not LIB.exists():
        pytest.fail(f"{LIB} is not built (run __graft_entry__.build())")
    lib = C.CDLL(str(LIB))
    lib.hkbs_check_device_gelu.restype = C.c_int
    counts = (C.c_ulonglong * 3)()
    first = (C.c_uint * 3)()
    worst = (C.c_uint * 3)()
    print("device gelu: 2^32 inputs", flush=True)
    assert lib.hkbs_check_device_gelu(counts, first, worst) == 0
    as_float = lambda u: struct.unpack("<f", struct.pack("<I", u))[0]
    w_poly, w_fast, at = as_float(worst[0]), as_float(worst[1]), as_float(worst[2])
    print(f"gelu_poly: largest deviation {w_poly:.3f} units (near x = {at!r}); gelu_fast: {w_fast:.3f} units",
          flush=True)
    assert counts[0] == 0, f"gelu differs from the reference form on {counts[0]} inputs (first {first[0]:#010x})"
    assert counts[1] == 0, f"gelu_fast differs from the select form on {counts[1]} inputs (first {first[1]:#010x})"
    assert counts[2] == 0, f"gelu_poly differs on {counts[2]} non-finite inputs (first {first[2]:#010x})"
    assert w_poly <= POLY_UNITS, f"gelu_poly deviates by {w_poly} units at x = {at!r}"


def test_device_rbf_fused_form():
    """rbf_chunk_fma (the 16-bit encoder's RBF features) against rbf_chunk (the reference's operation order,
    bit-exact with the oracle through the fp32 encoder tests) over 2^22 atom-pair offsets of 0 .. 30 A. The two
    may take neighbouring exp-table entries where t = d^2 / (2 sigma^2) lies within rounding of a half-integer;
    there the degree-6 Taylor series are cut at r = +1/2 and -1/2, whose remainders are -1.0e-6 and +2.4e-6 of
    exp(r), so the bound is 5e-6 of the feature; where one of them falls under the exp(-16) cut-off the other
    is at most 1.2e-7."""
    if not LIB.exists():
        pytest.fail(f"{LIB} is not built (run __graft_entry__.build())")
    lib = C.CDLL(str(LIB))
    lib.hkbs_check_device_rbf.restype = C.c_int
    out = (C.c_uint * 3)()
    print("device rbf: 2^22 offsets", flush=True)
    assert lib.hkbs_check_device_rbf(1 << 22, out) == 0
    as_float = lambda u: struct.unpack("<f", struct.pack("<I", u))[0]
    rel, dabs = as_float(out[0]), as_float(out[1])
    print(f"rbf_chunk_fma: largest relative deviation {rel:.3g}, absolute {dabs:.3g}, cut-off disagreements {out[2]}",
          flush=True)
    assert rel <= 5e-6
    assert dabs <= 5e-6


def test_device_matrix_core_products_are_sequential_sums():
    """seq_gemm_mfma (the encoder's reference-order sums, products from v_mfma_f32_16x16x1_4b_f32 with a zero
    addend) against the same sums on the VALU (product rounded, added in k order) over 4096 tiles of 32 x 128
    outputs with 128 terms each: operands of random sign with exponents over 52 and 32 binades, about 1/16
    zeros, every product a normal float or zero. Bit-exact: a failure names the first differing output."""
    if not LIB.exists():
        pytest.fail(f"{LIB} is not built (run __graft_entry__.build())")
    lib = C.CDLL(str(LIB))
    lib.hkbs_check_device_seq_gemm.restype = C.c_int
    out = (C.c_uint * 4)()
    print("device seq_gemm_mfma: 4096 tiles of 32 x 128 x 128", flush=True)
    assert lib.hkbs_check_device_seq_gemm(4096, out) == 0
    assert out[0] == 0, f"{out[0]} sums differ (first: tile {out[1]}, row {out[2] // 128}, col {out[2] % 128})"
