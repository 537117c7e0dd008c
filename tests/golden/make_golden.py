"""Writes tests/golden/e4m3_vectors.json from the OCP FP8 specification alone.

The OCP 8-bit floating point spec (E4M3 "FN" variant) fixes: sign bit, 4
exponent bits with bias 7, 3 mantissa bits, subnormals at exponent field 0
(value m * 2^-9), no infinities, S.1111.111 = NaN, max finite 448. The
reference quantizer rounds to nearest even and saturates out-of-range finite
values to +-448 (reference src/kernels/quantization.cu:248-250).

This script encodes with exact rational arithmetic (fractions.Fraction), with
no code shared with the C oracle, so the committed vectors pin the oracle's
bit-level encoder independently. Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import math
import random
import struct
from fractions import Fraction
from pathlib import Path

OUT = Path(__file__).resolve().parent / "e4m3_vectors.json"


def e4m3_value(code: int) -> Fraction | None:
    """Exact value of an E4M3 code, None for NaN."""
    e = (code >> 3) & 0xF
    m = code & 0x7
    if e == 0xF and m == 0x7:
        return None
    if e == 0:
        mag = Fraction(m, 1 << 9)
    else:
        mag = Fraction(8 + m, 8) * (Fraction(2) ** (e - 7))
    return -mag if code & 0x80 else mag


POS = [(c, e4m3_value(c)) for c in range(0x7F)]  # codes 0..126, ascending values


def encode_exact(x: float) -> int:
    if math.isnan(x):
        return 0x7F
    sign = 0x80 if math.copysign(1.0, x) < 0 else 0
    if math.isinf(x):
        return sign | 0x7E
    a = abs(Fraction(x))
    if a >= 448:
        return sign | 0x7E
    best = None
    for c, val in POS:
        d = abs(a - val)
        if best is None or d < best[0] or (d == best[0] and c % 2 == 0):
            best = (d, c)
    return sign | best[1]


def f32(bits: int) -> float:
    return struct.unpack("<f", struct.pack("<I", bits & 0xFFFFFFFF))[0]


def bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def main() -> None:
    inputs: set[int] = set()
    vals = [v for _, v in POS]
    for i, v in enumerate(vals):
        b = bits(float(v))
        inputs.update({b, b + 1, b - 1 if b else 0})
        if i + 1 < len(vals):
            mid = (v + vals[i + 1]) / 2
            mb = bits(float(mid))  # exact: midpoints are representable in fp32
            inputs.update({mb - 1, mb, mb + 1})
    for special in (448.0, 448.5, 463.99, 464.0, 479.0, 480.0, 1e30, float("inf"),
                    2.0 ** -10, 2.0 ** -10 * 1.0000001, 2.0 ** -11, 1e-40, 1e-45, 0.0):
        inputs.add(bits(special))
    inputs.add(0x7FC00000)  # qNaN
    inputs.add(0x7F800001)  # sNaN pattern
    rng = random.Random(0x5EED)
    for _ in range(3000):
        inputs.add(rng.getrandbits(32))
    for _ in range(3000):  # concentrate on the E4M3 dynamic range
        inputs.add(bits(rng.uniform(-500.0, 500.0)))
        inputs.add(bits(rng.uniform(-0.02, 0.02)))
    neg = {b | 0x80000000 for b in inputs}
    inputs |= neg
    ordered = sorted(inputs)
    codes = [encode_exact(f32(b)) for b in ordered]
    table = []
    for c in range(256):
        v = e4m3_value(c)
        table.append(None if v is None else float(v))
    OUT.write_text(json.dumps({
        "doc": "OCP E4M3FN encode (RNE, satfinite, NaN->0x7F) from exact rationals",
        "decode_table": table,
        "inputs_f32_bits": ordered,
        "codes": codes,
    }, indent=None, separators=(",", ":")) + "\n")
    print(f"wrote {len(ordered)} vectors to {OUT}")


if __name__ == "__main__":
    main()
