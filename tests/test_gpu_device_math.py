"""Exhaustive GPU check of the device GELUs (tests/csrc/device_math_check.hip).

The encoder's gelu is evaluated without branches and with a reciprocal plus
one Newton step in place of IEEE division; the decode loop's gelu_fast drops
the v > 4 select and copies the sign. Both must equal their straightforward
forms (the reference expression of cpp/include/hikoboshi/primitives/compute/gelu.hpp:22-51
with fast_exp_neg.hpp:12-55, and the select form) bit for bit for every one of
the 2^32 float inputs; the encoder tests then pin the straightforward form
against the oracle.
"""
import ctypes as C
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

LIB = Path(__file__).resolve().parent / "libdevice_math_check.so"


def test_device_gelu_all_inputs():
    if not LIB.exists():
        pytest.fail(f"{LIB} is not built (run __graft_entry__.build())")
    lib = C.CDLL(str(LIB))
    lib.hkbs_check_device_gelu.restype = C.c_int
    counts = (C.c_ulonglong * 2)()
    first = (C.c_uint * 2)()
    print("device gelu: 2^32 inputs", flush=True)
    assert lib.hkbs_check_device_gelu(counts, first) == 0
    assert counts[0] == 0, f"gelu differs from the reference form on {counts[0]} inputs (first {first[0]:#010x})"
    assert counts[1] == 0, f"gelu_fast differs from the select form on {counts[1]} inputs (first {first[1]:#010x})"
