# SPDX-License-Identifier: MIT
"""Writes tests/golden/kat.json: known-answer values of the number formats.

Derived from the OCP 8-bit floating point (OFP8) and microscaling (MX)
format definitions, not from any code in this repository or the reference:
  e4m3fn  sign | 4-bit exponent (bias 7) | 3-bit mantissa; exponent 0 is
          subnormal (m/8 * 2^-6); S.1111.111 is NaN; no infinities.
  e2m1    sign | 2-bit exponent (bias 1) | 1-bit mantissa; exponent 0 is
          subnormal (m * 0.5).
  e8m0    2^(e - 127); byte 255 is NaN.

    python tests/golden/make_kat.py
"""

import json
from fractions import Fraction
from pathlib import Path


def e4m3(code: int):
    s, e, m = code >> 7, (code >> 3) & 15, code & 7
    if e == 15 and m == 7:
        return "nan"
    mag = Fraction(m, 8) * Fraction(1, 64) if e == 0 else (1 + Fraction(m, 8)) * Fraction(2) ** (e - 7)
    return float(-mag if s else mag)


def e2m1(code: int):
    s, e, m = code >> 3, (code >> 1) & 3, code & 1
    mag = Fraction(m, 2) if e == 0 else (1 + Fraction(m, 2)) * Fraction(2) ** (e - 1)
    return float(-mag if s else mag)


def main():
    kat = {
        "e4m3fn": [e4m3(c) for c in range(256)],
        "e2m1": [e2m1(c) for c in range(16)],
        "e8m0": {str(b): float(Fraction(2) ** (b - 127)) for b in (1, 100, 119, 120, 121, 122, 123, 127, 128, 200, 254)},
    }
    out = Path(__file__).with_name("kat.json")
    out.write_text(json.dumps(kat, indent=1) + "\n")
    print(out)


if __name__ == "__main__":
    main()
