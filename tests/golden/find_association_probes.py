"""Finds probe elements that separate the fp64 associations of loom's fp32-row
norms, for tests/test_oracle_kat.py.  Writes tests/golden/association_probes.json.

    python tests/golden/find_association_probes.py

Two sites produce fp32 rows from fp64 arithmetic whose association a
restatement could get wrong:
  * bitNetRMSNormTensorRowWeighted (poly/bitnet_cpu.go:893-913):
    T(float64(v) * scale * w) = fp32((v*scale)*w), not fp32(v*(scale*w));
  * RMSNormForwardPolymorphic (poly/norm.go:102-138):
    T((float64(x) / rms) * g), a division, not fp32((x*(1/rms))*g).
The two forms differ by about one fp64 ulp, which changes the fp32 result
only when the exact value lies within that ulp of an fp32 rounding midpoint
(about 2^-30 of random elements).  A row of BASE normal values (the oracle's
seeded generator) fixes scale / rms; probe elements of magnitude below 2^-22
appended after it leave the sequential sum of squares unchanged (their
squares are under half an ulp of the sum), so the search can scan every fp32
value of one binade for each candidate weight and keep the (x, w) pairs whose
two forms round to different fp32 values.  The file holds inputs only; the
test recomputes the expected values from the reference's formula.
"""
from __future__ import annotations

import json
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

BASE_N = 6900
BASE_SEED = 611
EPS = 1e-5
N_PROBES = 12
N_TOTAL = BASE_N + N_PROBES


def base_row():
    from oracle import oracle as orc
    return orc.normal_f32(BASE_N, BASE_SEED)


def seq_sum_sq(v64):
    return float(np.add.accumulate(v64 * v64)[-1])


def binade_x():
    # every fp32 value in [2^-24, 2^-23): squares < 2^-46, far below half an
    # ulp of a sum near 7000 (about 4.5e-13)
    lo = np.float32(2.0 ** -24).view(np.uint32)
    bits = np.arange(int(lo), int(lo) + (1 << 23), dtype=np.uint32)
    return bits.view(np.float32).astype(np.float64)


def search(form_ref, form_alt, ws, xs, want):
    found = []
    for w in ws:
        r = form_ref(xs, w)
        a = form_alt(xs, w)
        idx = np.nonzero(r.astype(np.float32).view(np.uint32) != a.astype(np.float32).view(np.uint32))[0]
        for i in idx[:2]:
            found.append((float(np.float32(xs[i])), float(np.float32(w))))
        if len(found) >= want:
            break
    return found[:want]


def main() -> None:
    row = base_row().astype(np.float64)
    ss = seq_sum_sq(row)
    scale = 1.0 / math.sqrt(ss / N_TOTAL + EPS)
    rms = math.sqrt(ss / N_TOTAL + EPS)
    xs = binade_x()
    rng = np.random.default_rng(5)
    ws = rng.uniform(0.5, 1.5, 4000).astype(np.float32).astype(np.float64)

    inner = search(lambda x, w: (x * scale) * w, lambda x, w: x * (scale * w), ws, xs, N_PROBES)
    rmsn = search(lambda x, w: (x / rms) * w, lambda x, w: (x * (1.0 / rms)) * w, ws, xs, N_PROBES)
    if len(inner) < N_PROBES or len(rmsn) < N_PROBES:
        raise SystemExit(f"too few probes: {len(inner)}, {len(rmsn)}")
    out = {
        "base_n": BASE_N, "base_seed": BASE_SEED, "eps": EPS,
        "inner_norm_f32": [{"x": x, "w": w} for x, w in inner],
        "rmsnorm": [{"x": x, "g": w} for x, w in rmsn],
    }
    path = os.path.join(HERE, "association_probes.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print("wrote", path)


if __name__ == "__main__":
    main()
