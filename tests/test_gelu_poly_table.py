"""The decode loop's GELU table (hikoboshi_amd/csrc/gelu_poly_table.hpp) against its generator.

gelu_poly_gen.py fits one degree-6 polynomial per exp-table segment to the A&S erfc term of the reference
GELU (cpp/include/hikoboshi/primitives/compute/gelu.hpp:22-65, fast_exp_neg.hpp:9-57). Here: the committed
header holds exactly what the generator produces; the fp32 evaluation stays within 1e-7 of the
exact-arithmetic reference expression; the segments tile [0, sqrt(15.5)) at the reference's breakpoints; and
at v = 0 and at the middle of every segment the table reproduces an independent evaluation of the reference
expression (erfc from the A&S coefficients and libm exp, within the reference's own 1.6e-6 relative error of
the Taylor exp).
"""
import importlib.util
import math
import re
from pathlib import Path

import numpy as np

CSRC = Path(__file__).resolve().parents[1] / "hikoboshi_amd" / "csrc"


def _gen():
    spec = importlib.util.spec_from_file_location("gelu_poly_gen", CSRC / "gelu_poly_gen.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _header_rows():
    text = (CSRC / "gelu_poly_table.hpp").read_text()
    body = text[text.index("kGeluPoly[kGeluPolyRows * 8] = {"):]
    body = body[body.index("{") + 1:body.index("};")]
    vals = [float(v.rstrip("F")) for v in re.findall(r"[-+0-9.eE]+F", body)]
    split = float(re.search(r"kGeluPolySplit = ([-+0-9.eE]+)F", text).group(1))
    return np.float32(vals).reshape(-1, 8), split


def test_header_matches_generator():
    g = _gen()
    rows, split, worst = g.build()
    hdr, hsplit = _header_rows()
    assert hdr.shape == (18, 8)
    np.testing.assert_array_equal(hdr, np.stack(rows))
    assert np.float32(hsplit) == np.float32(split)
    assert worst < 1e-7
    assert not hdr[-1].any()  # v >= sqrt(15.5): P taken as 0


def test_segments_follow_reference_breakpoints():
    g = _gen()
    segs, split = g.segments()
    assert segs[0][0] == 0.0 and segs[0][1] == segs[1][0] == split
    for (lo, hi, n), (lo2, _, _) in zip(segs[1:], segs[2:]):
        assert hi == lo2
    for lo, hi, n in segs[2:]:
        assert math.isclose(lo * lo, n - 0.5, rel_tol=1e-12) and math.isclose(hi * hi, n + 0.5, rel_tol=1e-12)


def test_table_against_independent_erfc_term():
    """P(v) = poly(t) exp(-v^2) with libm exp; the reference's Taylor exp differs by < 1.6e-6 relative."""
    g = _gen()
    hdr, split = _header_rows()
    a = [0.254829592, -0.284496736, 1.421413741, -1.453152027, 1.061405429]
    segs, _ = g.segments()
    for i, (lo, hi, n) in enumerate(segs):
        for v in (lo, 0.5 * (lo + hi)):
            t = 1.0 / (1.0 + 0.3275911 * v)
            ref = t * (a[0] + t * (a[1] + t * (a[2] + t * (a[3] + t * a[4])))) * math.exp(-v * v)
            got = g.eval32(hdr[i], v)
            assert abs(got - ref) <= 1.6e-6 * ref + 1e-7, (i, v, got, ref)
    # P(0) = sum of the A&S coefficients = 1 - 1e-9
    assert abs(g.eval32(hdr[0], 0.0) - sum(a)) < 1e-7
