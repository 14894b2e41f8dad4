"""CPU pin of the 2/pi table in mini-infer_amd/csrc/rope_sincos.h that the
RoPE kernels' Payne-Hanek reduction reads for angles above 2^24.

The table must equal what gen_two_over_pi.py writes, and the generator's
2/pi must match the constant's published hexadecimal expansion
(2/pi = 0x0.A2F9836E4E441529FC2757D1F534DDC0DB6295993C439041FE51...), so a
wrong digit in either the script or the header fails here.
"""
import re
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "mini-infer_amd" / "csrc"
sys.path.insert(0, str(CSRC))

import gen_two_over_pi as gen  # noqa: E402

PUBLISHED = "A2F9836E4E441529FC2757D1F534DDC0DB6295993C439041FE51"


def test_generator_matches_published_digits():
    bits = 4 * len(PUBLISHED)
    assert gen.two_over_pi_fixed(bits) == int(PUBLISHED, 16)


def test_header_table_is_the_generated_one():
    text = (CSRC / "rope_sincos.h").read_text()
    body = text[text.index("kTwoOverPiMod4[104][3] = {"):]
    body = body[:body.index("};")]
    rows = re.findall(r"\{(\S+), (\S+), (\S+)\},", body)
    assert len(rows) == 104
    for (a, b, c), (ga, gb, gc) in zip(rows, gen.table()):
        assert (float.fromhex(a), float.fromhex(b), float.fromhex(c)) == (ga, gb, gc)


def test_table_rows_are_2e_times_two_over_pi_mod_4():
    """Row e, read back as an exact rational, is 2^e * 2/pi mod 4 to 2^-157."""
    from fractions import Fraction
    ref = Fraction(gen.two_over_pi_fixed(400), 1 << 400)
    for e, row in enumerate(gen.table(), start=1):
        y = sum(Fraction(v) for v in row)
        want = (ref * (1 << e)) % 4
        assert abs(y - want) < Fraction(1, 1 << 156), e
        assert all(v >= 0 for v in row) and row[1] < 2.0 ** -51 and row[2] < 2.0 ** -104
