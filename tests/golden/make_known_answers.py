"""Writes known_answers.json: small input/output vectors for the CPU oracle,
computed here by exact integer / rational arithmetic that shares no code with
the oracle, plus the published Max (1960) 8-level Gaussian quantizer table.

    python tests/golden/make_known_answers.py

Contents
  max1960        Max, "Quantizing for minimum distortion", IRE Trans. Inf.
                 Theory IT-6 (1960), Table I, N = 8: output levels y_i and
                 interval ends x_i of the minimum-MSE quantizer of N(0,1)
                 (positive half; the quantizer is odd-symmetric).
  fwht           integer vectors and their unnormalized Sylvester-Hadamard
                 transform H_n x, from the recursive definition of H_n.
  rtn_int8       fp32 rows, the fp32 scale absmax/127 and the int8 codes
                 round-half-even(x / scale) clamped to +-127, every division
                 rounded to fp32 exactly (round-to-nearest-even on the
                 rational quotient).
  pack3          3-bit codes and the bit-plane words (word 3g+b holds bit b of
                 codes 32g..32g+31, element 32g+i at bit i), assembled bit by
                 bit.
  flat_rows      flat slots -> storage rows (block*Hkv + h)*bs + slot%bs.
  block_bytes    per-block-per-layer HBM bytes for the byte layouts of the
                 reference cache (int8: K, V, two fp32 scales; lloydmax3:
                 int8 K, fp32 K scale, 3-bit V words, fp32 norms).
"""

from __future__ import annotations

import json
import random
import struct
from fractions import Fraction
from pathlib import Path

OUT = Path(__file__).resolve().parent / "known_answers.json"


def f32_round(q: Fraction) -> float:
    """Round a rational to the nearest fp32 (ties to even); finite normal or
    subnormal results only."""
    if q == 0:
        return 0.0
    sign = -1 if q < 0 else 1
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, -126)  # subnormal range keeps the exponent at -126
    scale = Fraction(2) ** (e - 23)
    m = a / scale  # in [2^23, 2^24) for normals
    n = m.numerator // m.denominator
    r = m - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1):
        n += 1
    val = Fraction(n) * scale
    out = float(val)
    assert struct.unpack("f", struct.pack("f", out))[0] == out
    return sign * out


def round_half_even(x: float) -> int:
    return round(x)  # Python rounds floats half to even, exactly


def sylvester(n: int):
    h = [[1]]
    while len(h) < n:
        h = [row + row for row in h] + [row + [-v for v in row] for row in h]
    return h


def fwht_cases(rng):
    cases = []
    for n in (2, 4, 8, 16, 32):
        h = sylvester(n)
        for _ in range(2):
            x = [rng.randint(-50, 50) for _ in range(n)]
            y = [sum(h[i][j] * x[j] for j in range(n)) for i in range(n)]
            cases.append({"x": x, "y": y})
    return cases


def rtn_cases(rng):
    rows = [
        [127.0, -63.5, 0.5, 1.5, -2.5, 0.0, 3.0, -127.0],  # scale 1: ties go to even
        [0.0] * 8,  # zero row: scale 0, codes 0
        [1.0, -0.25, 0.125, 0.0, 0.5, -1.0, 0.75, 0.375],
        [-3.0e-3, 1.0e-3, 2.5e-3, -7.5e-4, 0.0, 6.0e-4, -1.0e-5, 2.9e-3],
        [65504.0, -65504.0, 1.0, -1.0, 32752.0, 0.0, 258.0, -515.75],
    ]
    for _ in range(6):
        rows.append([float(struct.unpack("f", struct.pack("f", rng.gauss(0.0, 2.0)))[0]) for _ in range(8)])
    cases = []
    for row in rows:
        xs = [struct.unpack("f", struct.pack("f", v))[0] for v in row]
        amax = max(abs(v) for v in xs)
        scale = f32_round(Fraction(amax) / 127)
        if scale == 0.0:
            codes = [0] * len(xs)
        else:
            codes = []
            for v in xs:
                qf = f32_round(Fraction(v) / Fraction(scale))
                codes.append(max(-127, min(127, round_half_even(qf))))
        cases.append({"x": xs, "scale": scale, "codes": codes})
    return cases


def pack3_cases(rng):
    cases = []
    for d in (32, 128):
        for kind in ("random", "ramp", "single"):
            if kind == "random":
                codes = [rng.randint(0, 7) for _ in range(d)]
            elif kind == "ramp":
                codes = [i % 8 for i in range(d)]
            else:
                codes = [0] * d
                codes[d - 1] = 5
            words = []
            for g in range(d // 32):
                for b in range(3):
                    w = 0
                    for i in range(32):
                        if (codes[32 * g + i] >> b) & 1:
                            w |= 1 << i
                    words.append(w - (1 << 32) if w >= 1 << 31 else w)  # as int32
            cases.append({"codes": codes, "words": words})
    return cases


def flat_rows_cases():
    cases = []
    for hkv, bs in ((8, 256), (2, 16), (3, 4)):
        slots = [0, 1, bs - 1, bs, 5 * bs + 3, 17 * bs + bs - 1]
        rows = []
        for s in slots:
            blk, off = s // bs, s % bs
            rows.append([(blk * hkv + h) * bs + off for h in range(hkv)])
        cases.append({"num_kv_heads": hkv, "block_size": bs, "slots": slots, "rows": rows})
    return cases


def block_bytes_cases():
    out = []
    for hkv, bs, d in ((8, 16, 128), (2, 8, 32), (8, 256, 128), (4, 16, 256)):
        n = hkv * bs
        out.append({"num_kv_heads": hkv, "block_size": bs, "head_dim": d, "v_quant": "int8",
                    "bytes": n * d + n * d + n * 4 + n * 4})
        if d % 128 == 0:
            out.append({"num_kv_heads": hkv, "block_size": bs, "head_dim": d, "v_quant": "lloydmax3",
                        "bytes": n * d + n * 4 + n * (d // 32) * 3 * 4 + n * (d // 128) * 4})
    return out


def main() -> None:
    rng = random.Random(20260101)
    data = {
        "max1960": {"levels": [0.2451, 0.7560, 1.3440, 2.1520], "thresholds": [0.0, 0.5006, 1.0500, 1.7480]},
        "fwht": fwht_cases(rng),
        "rtn_int8": rtn_cases(rng),
        "pack3": pack3_cases(rng),
        "flat_rows": flat_rows_cases(),
        "block_bytes": block_bytes_cases(),
    }
    OUT.write_text(json.dumps(data, indent=1) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
