"""Writes tests/golden/vectors.npz: small seeded inputs and their outputs
computed with plain Python float64 loops (math module only; no numpy or
torch arithmetic), independently of the oracle's code. Regenerate with
`python tests/golden/make_golden.py`."""

import math
import random
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent / "vectors.npz"


def gauss_matrix(r, rows, cols, scale=1.0):
    return [[r.gauss(0.0, 1.0) * scale for _ in range(cols)] for _ in range(rows)]


def f32(m):
    return [[float(np.float32(v)) for v in row] for row in m]


def main():
    r = random.Random(1234)
    out = {}
    x = f32(gauss_matrix(r, 5, 37))
    w = [float(np.float32(1 + 0.1 * r.gauss(0, 1))) for _ in range(37)]
    out["rms_x"], out["rms_w"] = x, w
    out["rms_sum_y"] = [[v / math.sqrt(sum(t * t for t in row)) for v in row] for row in x]
    out["rms_w_y"] = [[v / math.sqrt(sum(t * t for t in row) / 37 + 1e-6) * w[j] for j, v in enumerate(row)]
                      for row in x]
    ln = []
    for row in x:
        mu = sum(row) / len(row)
        var = sum((t - mu) ** 2 for t in row) / len(row)
        ln.append([(t - mu) / math.sqrt(var + 1e-6) for t in row])
    out["ln_y"] = ln
    sm = []
    for row in x:
        e = [math.exp(t) for t in row]
        s = sum(e)
        sm.append([t / s for t in e])
    out["softmax_y"] = sm
    cs = []
    for row in x:
        acc, o = 0.0, []
        for t in row:
            acc += t
            o.append(acc)
        cs.append(o)
    out["cumsum_y"] = cs
    a = f32(gauss_matrix(r, 6, 11))
    b = f32(gauss_matrix(r, 11, 4))
    out["mm_a"], out["mm_b"] = a, b
    out["mm_y"] = [[sum(a[i][k] * b[k][j] for k in range(11)) for j in range(4)] for i in range(6)]
    s, d = 7, 4
    q, k, v = (f32(gauss_matrix(r, s, d)) for _ in range(3))
    out["at_q"], out["at_k"], out["at_v"] = q, k, v
    att = []
    for i in range(s):
        sc = [sum(q[i][t] * k[j][t] for t in range(d)) / math.sqrt(d) for j in range(i + 1)]
        mx = max(sc)
        p = [math.exp(t - mx) for t in sc]
        den = sum(p)
        att.append([sum(p[j] * v[j][t] for j in range(i + 1)) / den for t in range(d)])
    out["at_causal_y"] = att
    # token-major rotate-half RoPE, one token sequence of 3, one head, d = 8
    xr = f32(gauss_matrix(r, 3, 8))
    out["rope_x"] = xr
    ry = []
    for p_, row in enumerate(xr):
        o = [0.0] * 8
        for i in range(4):
            ang = p_ * 500000.0 ** (-2 * i / 8)
            c, sn = math.cos(ang), math.sin(ang)
            o[i] = row[i] * c - row[i + 4] * sn
            o[i + 4] = row[i + 4] * c + row[i] * sn
        ry.append(o)
    out["rope_y"] = ry
    np.savez(OUT, **{key: np.asarray(val, dtype=np.float64) for key, val in out.items()})
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
