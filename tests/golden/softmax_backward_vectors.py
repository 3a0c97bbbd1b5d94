"""Writes the softmax / log-softmax backward known answers into reference_known_answers.json.

The cases and the expected-value rule are those of the reference's
testing/backend-conformance/.../CpuSoftmaxBackwardConformanceTest.java (FLOAT32 rows of its
tests; nothing from the reference is imported or run):
  * :32-48 finite operands, y = [-.5, -1, 0, -2, -.25, -.75] as two rows of 3, with two seeds g;
    expected (check, :172-183): the row sum is formed exactly (BigDecimal) and rounded once to
    binary32, of typed(g * y) for softmax and of g for log-softmax; then
    softmax: y * (g - sum), log-softmax: g - (float)exp(y) * sum, every operation in binary32;
  * :54-98 non-finite operands with the row sums the test states (softmax NaN, +inf;
    log-softmax 6, NaN) and the same per-element rule; NaN payloads are unspecified.
Expected values are stored as binary32 bit patterns (None = any NaN).
Run from the repo root: python tests/golden/softmax_backward_vectors.py
"""
import json
import math
from fractions import Fraction
from pathlib import Path

import numpy as np

SRC = "testing/backend-conformance/.../CpuSoftmaxBackwardConformanceTest.java"
F = np.float32


def bits(v):
    v = F(v)
    return None if math.isnan(v) else int(np.array([v], np.float32).view(np.uint32)[0])


def expected(y, g, log, sums=None):
    out = []
    for row in range(2):
        idx = range(3 * row, 3 * row + 3)
        if sums is None:
            exact = sum(Fraction(float(g[i])) if log else Fraction(float(F(g[i]) * F(y[i])))
                        for i in idx)
            s = F(float(exact))  # one rounding of the exact sum (finite operands only)
        else:
            s = F(sums[row])
        for i in idx:
            with np.errstate(all="ignore"):
                if log:
                    out.append(bits(F(g[i]) - F(F(math.exp(float(y[i]))) * s)))
                else:
                    out.append(bits(F(y[i]) * F(F(g[i]) - s)))
    return out


def main():
    inf, nan = math.inf, math.nan
    cases = []
    y = [-.5, -1, 0, -2, -.25, -.75]
    for log in (False, True):
        for g, name in (([1, -2, 3, 4, -5, 6], "finite, first seed"),
                        ([-7, 8, -9, 10, 11, -12], "finite, second seed")):
            cases.append({"source": SRC + ":32-48,172-183", "case": name, "log": log,
                          "y": y, "g": g, "expected_bits": expected(y, g, log)})
    yn = [nan, 0, 1, inf, -inf, -0.0]
    gn = [1, 2, 3, inf, -inf, 0]
    for log, sums in ((False, [nan, inf]), (True, [6, nan])):
        cases.append({"source": SRC + ":54-98", "case": "non-finite operands", "log": log,
                      "y": [_enc(v) for v in yn], "g": [_enc(v) for v in gn],
                      "row_sums": [_enc(v) for v in sums],
                      "expected_bits": expected(yn, gn, log, sums)})
    path = Path(__file__).parent / "reference_known_answers.json"
    d = json.loads(path.read_text())
    d["softmax_backward"] = cases
    path.write_text(json.dumps(d, indent=1) + "\n")


def _enc(v):
    if isinstance(v, float) and math.isnan(v):
        return "nan"
    if v == math.inf:
        return "inf"
    if v == -math.inf:
        return "-inf"
    if v == 0 and math.copysign(1, v) < 0:
        return "-0"
    return v


if __name__ == "__main__":
    main()
