"""Writes tests/golden/vectors.json: small inputs with expected outputs from
exact arithmetic (values chosen so every result is representable) or from
float64 closed forms rounded to the element type.  Independent of the oracle.
Run: python tests/golden/make_golden.py
"""
import json
import math
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent / "vectors.json"


def case(name, kind, dtype, a, expected, tolerance_ulp=0, **extra):
    a = np.asarray(a, dtype=np.float64)
    entry = {"name": name, "kind": kind, "dtype": dtype, "a": a.reshape(-1).tolist(),
             "shape_a": list(a.shape), "expected": np.asarray(expected).reshape(-1).tolist(),
             "tolerance_ulp": tolerance_ulp}
    entry.update(extra)
    return entry


def main():
    cases = []
    a = np.array([[1.5, -2.25, 3.0, 0.5], [-4.0, 8.0, 0.125, -1.0], [2.0, -0.5, 6.5, 16.0]])
    b = np.array([2.0, -0.5, 4.0, 0.25])
    ops = {"add": a + b, "subtract": a - b, "multiply": a * b, "divide": a / b}
    for op, value in ops.items():
        for dtype in ("float32", "float64"):
            cases.append(case(f"{op} row broadcast {dtype}", "binary", dtype, a, value, op=op,
                              b=b.tolist(), shape_b=[4]))
    col = np.array([[3.0], [-1.0], [0.5]])
    cases.append(case("multiply column broadcast", "binary", "float32", a, a * col, op="multiply",
                      b=col.reshape(-1).tolist(), shape_b=[3, 1]))
    cases.append(case("less", "binary", "float32", a, (a < b).astype(float), op="less",
                      b=b.tolist(), shape_b=[4]))
    x = np.array([0.0, 1.0, 2.0, -1.0, -3.0, 5.0, 10.0, -10.0])
    cases.append(case("exp", "unary", "float32", x, np.exp(x).astype(np.float32), 1, op="exp"))
    y = np.array([1.0, 2.0, 0.5, 10.0, 1e-3, 7.25])
    cases.append(case("log", "unary", "float32", y, np.log(y).astype(np.float32), 1, op="log"))
    cases.append(case("tanh", "unary", "float32", x, np.tanh(x).astype(np.float32), 2, op="tanh"))
    gelu = [0.5 * v * math.erfc(-v / math.sqrt(2)) for v in x]
    cases.append(case("gelu", "unary", "float32", x, np.array(gelu).astype(np.float32), 1,
                      op="gelu"))
    m = np.arange(24, dtype=np.float64).reshape(2, 3, 4) - 7.0
    cases.append(case("sum axis 1", "axis_sum", "float32", m, m.sum(axis=1), axes=[1]))
    cases.append(case("sum axes 0,2", "axis_sum", "float32", m, m.sum(axis=(0, 2)), axes=[0, 2]))
    s = np.array([[1.0, 2.0, 3.0], [0.0, 0.0, 0.0], [-1.0, 5.0, 2.5]])
    e = np.exp(s - s.max(axis=1, keepdims=True))
    cases.append(case("softmax rows", "softmax", "float32", s,
                      (e / e.sum(axis=1, keepdims=True)).astype(np.float32), 2, axis=1))
    OUT.write_text(json.dumps({"cases": cases}, indent=1) + "\n")
    print(f"wrote {len(cases)} cases to {OUT}")


if __name__ == "__main__":
    main()
