"""Writes tests/golden/go_semantics.json: inputs and the oracle's outputs for
the reference routines whose rounding only a Go build can confirm —
LayerNormRow (linalg/vec_simd.go:285-327, vec_scalar.go:66-81), ExpShift
(vec_simd.go:220-264, its tail exp32 fastmath.go:36-52), QuantizeRowU8
(vec_simd.go:64-91, vec_scalar.go:23-31) and GeluMul (vec_simd.go:125-160,
gelu_amd64.s) — for every Go simd lane width V (0: a build without
GOEXPERIMENT=simd; 4, 8, 16). A maintainer with Go runs the reference on
the same inputs (a Go test that reads this file) and compares bit for bit.

The oracle restates the Go source with scalar code unfused (GOAMD64 v1/v2).
The QuantizeRowU8 rows end in crafted values where f32(x*inv) is exactly a
half-integer but the exact product is not: RNE of the rounded product and
RNE of the exact product (what a fused x*inv + magic gives) differ there,
so a build that fuses the tail fails those entries; `fused_differs` lists
them. Floats are stored as their IEEE bit patterns.

Run from the repository root: python tests/golden/make_go_vectors.py
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as orc  # noqa: E402

OUT = os.path.join(HERE, "go_semantics.json")
LANES = (0, 4, 8, 16)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).tolist()


def u8_ties(rng, inv, count):
    """float32 x > 0 with f32(x*inv) == k + 0.5 exactly but x*inv != k + 0.5
    (exact in float64), on the side where RNE of the exact product is not
    the even neighbour: the unfused and fused roundings of the tail differ."""
    out = []
    while len(out) < count:
        k = int(rng.integers(0, 254))
        x0 = int(np.array([(k + 0.5) / float(inv)], np.float32).view(np.uint32)[0])
        for d in (0, 1, -1, 2, -2, 3, -3, 4, -4):
            x = np.array([x0 + d], np.uint32).view(np.float32)[0]
            p = np.float32(x * np.float32(inv))
            exact = float(x) * float(inv)  # exact: a float32 product fits a float64
            if float(p) == k + 0.5 and exact != k + 0.5 and round(exact) != int(np.rint(p)):
                out.append(x)
                break
    return np.array(out, np.float32)


def main():
    rng = np.random.default_rng(20261202)
    doc = {
        "about": __doc__.strip().splitlines()[0],
        "layernorm": [], "expshift": [], "quantize_u8": [], "gelumul": [],
    }
    for V in LANES:
        for n, scale in ((768, 1.0), (384, 30.0), (37, 1e-3), (13, 1e3)):
            x = (rng.standard_normal(n) * scale).astype(np.float32)
            g = rng.uniform(0.9, 1.1, n).astype(np.float32)
            o = orc.layernorm_rows(x[None, :], g, eps=1e-5, lanes=V)[0]
            doc["layernorm"].append({"lanes": V, "eps": 1e-5, "x": bits(x), "gamma": bits(g), "o": bits(o)})
        for n in (1, 3, 7, 8, 9, 15, 16, 17, 33, 129, 257):
            x = (rng.standard_normal(n) * 3.0).astype(np.float32)
            if n >= 9:
                x[n // 2] = np.float32(-200.0)  # below -87.3 after the shift: 0
            m = np.float32(x.max())
            e, s = orc.exp_shift(x, m, lanes=V)
            doc["expshift"].append({"lanes": V, "m": bits([m])[0], "x": bits(x), "e": bits(e),
                                    "sum": bits([s])[0]})
        for n in (5, 16, 23, 40, 131):
            e = rng.uniform(0.0, 1.0, n).astype(np.float32)
            t = u8_ties(rng, 255.0, 6)
            x = np.concatenate([e, t]).astype(np.float32)
            q, s = orc.quantize_row_u8(x, 255.0, lanes=V)
            fused = [int(i) for i in range(len(x))
                     if round(float(x[i]) * 255.0) != int(q[i])]
            doc["quantize_u8"].append({"lanes": V, "inv": bits([np.float32(255.0)])[0], "x": bits(x),
                                       "q": q.astype(int).tolist(), "sum": s, "fused_differs": fused})
        for n in (1152, 37, 23, 16, 5):
            a = (rng.standard_normal(n) * 2.5).astype(np.float32)
            a[0] = np.float32(7.0)   # past the erf clamp
            a[-1] = np.float32(-6.0)
            b = rng.standard_normal(n).astype(np.float32)
            o = orc.gelu_mul(a[None, :], b[None, :], lanes=V)[0]
            doc["gelumul"].append({"lanes": V, "a": bits(a), "b": bits(b), "o": bits(o)})
    with open(OUT, "w") as f:
        json.dump(doc, f, separators=(",", ":"))
        f.write("\n")
    print(f"wrote {OUT}: {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
